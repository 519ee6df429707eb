// Inter-chunk state scans (forward h and reverse dh) for chunked GLA.
//
// Forward (reference: tops/ops/common/chunk_h.py:18-119, ref chunk.py:206-292):
//   h[n] = h_n ;  h_{n+1} = diag(e^{gamma_n}) h_n + (k * e^{gamma_n - g~})^T v
// Reverse (reference: tops/ops/common/chunk_h.py:399-591):
//   dh[n] = dh ;  dh <- diag(e^{gamma_n}) dh + (scale * q * e^{g~})^T do
// g~ is the chunk-local cumsum of the raw gates (computed here unless given), gamma_n its
// value at the chunk's last row.
//
// One 256-thread block owns a 64(k) x 64(v) tile of the K x V state of one (sequence,
// head) and walks that sequence's chunks in order (reverse order for dh):
//  * the raw a (k or q), g and b (v or do) tiles of chunk n+1 are fetched with 16-byte loads
//    into registers while chunk n computes, then written to LDS;
//  * thread = two adjacent columns x C/8 rows: column cumsum, gating and the transposes
//    (a^T gated, b^T) are written as whole runs of rows;
//  * the state stays in MFMA accumulators: wave w holds v rows [16w, 16w+16) x all 64 k
//    columns as four 16x16 tiles (out[v][k] = sum_c b^T[v][c] a^T[k][c]), so a lane's four
//    values are four consecutive v of one k and go to the [.., K, V] layout as one vector.
#include "common.hpp"
#include "kernels.hpp"

namespace tops {

template <typename T, int C, bool REV, bool VEC>
__global__ __launch_bounds__(256) void state_scan_kernel(ScanArgs p) {
  constexpr int CP = C < 32 ? 32 : C;     // contraction length (zero padded)
  constexpr int PC = pitch_of<T>(CP);     // transposed operands [64][CP]
  constexpr int PR = pitch_of<T>(64);     // raw tiles [C][64]
  constexpr int EPP = 16 / (int)sizeof(T);
  constexpr int PPR = 64 / EPP;           // 16-byte pieces per raw row
  constexpr int NP = C * PPR;
  constexpr int PPT = (NP + 255) / 256;
  constexpr int NSEG = 8;                 // 32 column pairs x 8 row segments
  constexpr int RPS = C / NSEG;
  __shared__ __attribute__((aligned(16))) T sAr[C * PR];
  __shared__ __attribute__((aligned(16))) T sGr[C * PR];
  __shared__ __attribute__((aligned(16))) T sBr[C * PR];
  __shared__ __attribute__((aligned(16))) T sXT[64 * PC];  // gated a^T  [k][c]
  __shared__ __attribute__((aligned(16))) T sBT[64 * PC];  // b^T        [v][c]
  __shared__ float sGam[64];
  __shared__ float sTot[NSEG * 64];

  const T* __restrict__ a = (const T*)p.a;
  const T* __restrict__ b = (const T*)p.b;
  const T* __restrict__ g = (const T*)p.g;
  T* __restrict__ s_all = (T*)p.s_all;
  const int H = p.H, K = p.K, V = p.V;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int KT = (K + 63) >> 6, VT = (V + 63) >> 6;
  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int vt = L % VT;
  const int kt = (L / VT) % KT;
  const int bh = L / (VT * KT);
  const int seq = bh / H, hh = bh % H;
  const int kbase = kt * 64, vbase = vt * 64;

  int bos, eos, c0, nc;
  seq_range(p.si, seq, bos, eos, c0, nc);

  for (int i = tid; i < 64 * PC; i += 256) {
    sXT[i] = zero_elem<T>();
    sBT[i] = zero_elem<T>();
  }

  // accumulator element -> (k, v)
  const int kcol = kbase + (lane & 15);                 // + 16*n
  const int vrow = vbase + w * 16 + 4 * (lane >> 4);    // + r
  f32x4 acc[4];
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    acc[n] = zero4();
    const int kk = kcol + 16 * n;
    if (p.s_init && kk < K) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (vrow + r < V) acc[n][r] = p.s_init[(((long)seq * H + hh) * K + kk) * V + vrow + r];
    }
  }

  uint4 pa[PPT], pg[PPT], pb[PPT];
  auto issue = [&](int step) {
    const int ci = REV ? (nc - 1 - step) : step;
    const int t0 = bos + ci * C;
    const int len = min(C, eos - t0);
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      const int pc = tid + 256 * j;
      pa[j] = pg[j] = pb[j] = make_uint4(0, 0, 0, 0);
      if (pc < NP) {
        const int row = pc / PPR, col0 = (pc % PPR) * EPP;
        if (row < len) {
          const long rk = ((long)(t0 + row) * H + hh) * K + kbase;
          const long rv = ((long)(t0 + row) * H + hh) * V + vbase;
          pa[j] = gload16<T, VEC>(a + rk, col0, K - kbase - col0);
          pg[j] = gload16<T, VEC>(g + rk, col0, K - kbase - col0);
          pb[j] = gload16<T, VEC>(b + rv, col0, V - vbase - col0);
        }
      }
    }
  };
  auto commit = [&]() {
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      const int pc = tid + 256 * j;
      if (pc < NP) {
        const int row = pc / PPR, col0 = (pc % PPR) * EPP;
        *reinterpret_cast<uint4*>(sAr + row * PR + col0) = pa[j];
        *reinterpret_cast<uint4*>(sGr + row * PR + col0) = pg[j];
        *reinterpret_cast<uint4*>(sBr + row * PR + col0) = pb[j];
      }
    }
  };
  if (nc > 0) {
    issue(0);
    commit();
    if (nc > 1) issue(1);
  }
  __syncthreads();

  const int cp = tid & 31, seg = tid >> 5;   // columns 2cp, 2cp+1 ; rows [seg*RPS, +RPS)
  const int c_0 = 2 * cp, c_1 = 2 * cp + 1;
  const bool gcum = p.g_is_cumsum != 0;

  for (int step = 0; step < nc; ++step) {
    const int ci = REV ? (nc - 1 - step) : step;
    const int t0 = bos + ci * C;
    const int len = min(C, eos - t0);

    // ---- column cumsum (or given cumsum) ----
    float g0[RPS], g1[RPS];
    float run0 = 0.f, run1 = 0.f;
#pragma unroll
    for (int rr = 0; rr < RPS; ++rr) {
      float x0, x1;
      Pair<T>::ld(sGr + (seg * RPS + rr) * PR + c_0, x0, x1);
      if (gcum) {
        g0[rr] = x0;
        g1[rr] = x1;
      } else {
        run0 += x0;
        run1 += x1;
        g0[rr] = run0;
        g1[rr] = run1;
      }
    }
    if (gcum) {
      // gamma = given value at the last valid row
      const int lr = len - 1;
      if (lr >= seg * RPS && lr < seg * RPS + RPS) {
#pragma unroll
        for (int rr = 0; rr < RPS; ++rr)
          if (seg * RPS + rr == lr) {
            sTot[c_0] = g0[rr];
            sTot[c_1] = g1[rr];
          }
      }
    } else {
      sTot[seg * 64 + c_0] = run0;
      sTot[seg * 64 + c_1] = run1;
    }
    __syncthreads();
    float off0 = 0.f, off1 = 0.f, gam0 = 0.f, gam1 = 0.f;
    if (gcum) {
      gam0 = sTot[c_0];
      gam1 = sTot[c_1];
    } else {
#pragma unroll
      for (int s = 0; s < NSEG; ++s) {
        const float x0 = sTot[s * 64 + c_0], x1 = sTot[s * 64 + c_1];
        off0 += (s < seg) ? x0 : 0.f;
        off1 += (s < seg) ? x1 : 0.f;
        gam0 += x0;
        gam1 += x1;
      }
    }

    // ---- gated a^T and b^T, written as row runs ----
    float xa0[RPS], xa1[RPS], xb0[RPS], xb1[RPS];
#pragma unroll
    for (int rr = 0; rr < RPS; ++rr) {
      const int row = seg * RPS + rr;
      float a0, a1, b0, b1;
      Pair<T>::ld(sAr + row * PR + c_0, a0, a1);
      Pair<T>::ld(sBr + row * PR + c_0, b0, b1);
      float e0, e1;
      if (REV) {
        e0 = p.scale * gexp<T>(g0[rr] + off0);
        e1 = p.scale * gexp<T>(g1[rr] + off1);
      } else {
        e0 = gexp<T>(gam0 - (g0[rr] + off0));
        e1 = gexp<T>(gam1 - (g1[rr] + off1));
      }
      if (gcum && row >= len) e0 = e1 = 0.f;
      xa0[rr] = a0 * e0;
      xa1[rr] = a1 * e1;
      xb0[rr] = b0;
      xb1[rr] = b1;
    }
    store_run<T, RPS>(sXT + c_0 * PC + seg * RPS, xa0);
    store_run<T, RPS>(sXT + c_1 * PC + seg * RPS, xa1);
    store_run<T, RPS>(sBT + c_0 * PC + seg * RPS, xb0);
    store_run<T, RPS>(sBT + c_1 * PC + seg * RPS, xb1);
    if (seg == 0) {
      sGam[c_0] = gexp<T>(gam0);
      sGam[c_1] = gexp<T>(gam1);
    }
    __syncthreads();

    // ---- state entering this chunk (forward) / leaving it (reverse) ----
    if (s_all) {
      const long cbase = ((long)(c0 + ci) * H + hh) * K;
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const int kk = kcol + 16 * n;
        if (kk >= K) continue;
        T* dst = s_all + (cbase + kk) * V + vrow;
        if (VEC && vrow + 3 < V) {
          if constexpr (sizeof(T) == 2) {
            *reinterpret_cast<uint2*>(dst) =
                make_uint2(pack2_bf16(acc[n][0], acc[n][1]), pack2_bf16(acc[n][2], acc[n][3]));
          } else {
            *reinterpret_cast<float4*>(dst) =
                make_float4(acc[n][0], acc[n][1], acc[n][2], acc[n][3]);
          }
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (vrow + r < V) dst[r] = from_f32<T>(acc[n][r]);
        }
      }
    }
    // raw tiles are free now: stage the next chunk, fetch the one after
    if (step + 1 < nc) {
      commit();
      if (step + 2 < nc) issue(step + 2);
    }
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      acc[n] *= sGam[n * 16 + (lane & 15)];
      mma_tile<T>(acc[n], sBT + (w * 16) * PC, PC, sXT + (n * 16) * PC, PC, CP, lane);
    }
    __syncthreads();
  }

  if (p.s_final) {
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      const int kk = kcol + 16 * n;
      if (kk >= K) continue;
      float* dst = p.s_final + (((long)seq * H + hh) * K + kk) * V + vrow;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (vrow + r < V) dst[r] = acc[n][r];
    }
  }
}

template <typename T, int C, bool REV>
static hipError_t launch_scan(const ScanArgs& p, hipStream_t st) {
  const int KT = (p.K + 63) / 64, VT = (p.V + 63) / 64;
  const long blocks = (long)p.si.N * p.H * KT * VT;
  if (blocks == 0) return hipSuccess;
  if (p.vec)
    hipLaunchKernelGGL((state_scan_kernel<T, C, REV, true>), dim3((unsigned)blocks), dim3(256),
                       0, st, p);
  else
    hipLaunchKernelGGL((state_scan_kernel<T, C, REV, false>), dim3((unsigned)blocks),
                       dim3(256), 0, st, p);
  return hipGetLastError();
}

template <typename T, bool REV>
static hipError_t dispatch_c(const ScanArgs& p, hipStream_t st) {
  switch (p.si.C) {
    case 16: return launch_scan<T, 16, REV>(p, st);
    case 32: return launch_scan<T, 32, REV>(p, st);
    case 64: return launch_scan<T, 64, REV>(p, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t run_state_scan(const ScanArgs& p, bool reverse, int dtype, hipStream_t st) {
  if (dtype == DT_BF16)
    return reverse ? dispatch_c<bf16, true>(p, st) : dispatch_c<bf16, false>(p, st);
  if (dtype == DT_F32)
    return reverse ? dispatch_c<float, true>(p, st) : dispatch_c<float, false>(p, st);
  return hipErrorInvalidValue;
}

}  // namespace tops
