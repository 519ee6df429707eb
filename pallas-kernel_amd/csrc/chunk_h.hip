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
// head) and walks that sequence's chunks in order (reverse order for dh). The state stays
// in MFMA accumulators: wave w holds v rows [16w, 16w+16) x all 64 k columns as four
// 16x16 tiles, orientation out[v][k] = sum_c X[v][c] Y[k][c] with X = b^T and Y = gated a^T,
// so a lane's four accumulator values are four consecutive v of one k: they are stored to
// the [.., K, V] state layout as one vector.
#include "common.hpp"
#include "kernels.hpp"

namespace tops {

template <typename T, int C, bool REV>
__global__ __launch_bounds__(256) void state_scan_kernel(
    const T* __restrict__ a,         // forward: k ; reverse: q        [tokens, H, K]
    const T* __restrict__ b,         // forward: v ; reverse: do       [tokens, H, V]
    const T* __restrict__ g,         // raw gates (or cumsum)          [tokens, H, K]
    int g_is_cumsum,
    const float* __restrict__ s_init,  // forward: h0 ; reverse: dht  [N, H, K, V] or null
    T* __restrict__ s_all,             // per-chunk states [NC, H, K, V] or null
    float* __restrict__ s_final,       // forward: ht ; reverse: dh0  [N, H, K, V] or null
    float scale, int H, int K, int V, SeqInfo si) {
  constexpr int CP = C < 32 ? 32 : C;  // contraction length (zero padded)
  constexpr int PC = pitch_of<T>(CP);
  constexpr int RPS = C / 4;
  __shared__ __attribute__((aligned(16))) T sXT[64 * PC];  // gated a^T  [k][c]
  __shared__ __attribute__((aligned(16))) T sBT[64 * PC];  // b^T        [v][c]
  __shared__ float sGam[64];
  __shared__ float sTot[4 * 64];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int KT = (K + 63) >> 6, VT = (V + 63) >> 6;
  const int total = gridDim.x;
  const int L = xcd_remap(blockIdx.x, total);
  const int vt = L % VT;
  const int kt = (L / VT) % KT;
  const int bh = L / (VT * KT);
  const int seq = bh / H, hh = bh % H;

  int bos, eos, c0, nc;
  seq_range(si, seq, bos, eos, c0, nc);

  // zero the contraction padding [C, CP) once; chunk writes only touch [0, C)
  if (CP > C) {
    for (int i = tid; i < 64 * (CP - C); i += 256) {
      const int r = i / (CP - C), cc = C + i % (CP - C);
      sXT[r * PC + cc] = zero_elem<T>();
      sBT[r * PC + cc] = zero_elem<T>();
    }
  }

  // accumulator element -> (k, v)
  const int kcol = kt * 64 + (lane & 15);  // + 16*n
  const int vrow = vt * 64 + w * 16 + 4 * (lane >> 4);  // + r
  f32x4 acc[4];
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    acc[n] = zero4();
    if (s_init) {
      const int kk = kcol + 16 * n;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int vv = vrow + r;
        if (kk < K && vv < V)
          acc[n][r] = s_init[(((long)seq * H + hh) * K + kk) * V + vv];
      }
    }
  }

  // prologue mapping: column `col` of the tile, rows [seg*RPS, +RPS)
  const int col = tid & 63, seg = tid >> 6;
  const int gk_col = kt * 64 + col, gv_col = vt * 64 + col;
  const bool kvalid = gk_col < K, vvalid = gv_col < V;
  const long rsK = (long)H * K, rsV = (long)H * V;

  for (int step = 0; step < nc; ++step) {
    const int ci = REV ? (nc - 1 - step) : step;
    const int t0 = bos + ci * C;
    const int len = min(C, eos - t0);
    const long baseK = ((long)t0 * H + hh) * K;
    const long baseV = ((long)t0 * H + hh) * V;

    float gt[RPS];
    float gamma, first;
    tile_cumsum<C>(g + baseK + gk_col, rsK, len, kvalid, g_is_cumsum != 0, sTot, gt, gamma,
                   first);
    (void)first;
#pragma unroll
    for (int r = 0; r < RPS; ++r) {
      const int row = seg * RPS + r;
      float x = 0.f, y = 0.f;
      if (row < len) {
        if (kvalid) x = to_f32(a[baseK + (long)row * rsK + gk_col]);
        if (vvalid) y = to_f32(b[baseV + (long)row * rsV + gv_col]);
      }
      const float f = REV ? scale * gexp<T>(gt[r]) : gexp<T>(gamma - gt[r]);
      sXT[col * PC + row] = from_f32<T>(x * f);
      sBT[col * PC + row] = from_f32<T>(y);
    }
    if (seg == 0) sGam[col] = gexp<T>(gamma);
    __syncthreads();

    // store the state entering this chunk (forward) / leaving it (reverse)
    if (s_all) {
      const long cbase = ((long)(c0 + ci) * H + hh) * K;
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const int kk = kcol + 16 * n;
        if (kk >= K) continue;
        T* dst = s_all + (cbase + kk) * V + vrow;
        if (vrow + 3 < V && (V & 3) == 0) {
          if (sizeof(T) == 2) {
            uint2 pk;
            pk.x = (uint32_t)from_f32<bf16>(acc[n][0]).u |
                   ((uint32_t)from_f32<bf16>(acc[n][1]).u << 16);
            pk.y = (uint32_t)from_f32<bf16>(acc[n][2]).u |
                   ((uint32_t)from_f32<bf16>(acc[n][3]).u << 16);
            *reinterpret_cast<uint2*>(dst) = pk;
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

#pragma unroll
    for (int n = 0; n < 4; ++n) {
      const float d = sGam[n * 16 + (lane & 15)];
      acc[n] *= d;
      mma_tile<T>(acc[n], sBT + (w * 16) * PC, PC, sXT + (n * 16) * PC, PC, CP, lane);
    }
    __syncthreads();
  }

  if (s_final) {
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      const int kk = kcol + 16 * n;
      if (kk >= K) continue;
      float* dst = s_final + (((long)seq * H + hh) * K + kk) * V + vrow;
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
  hipLaunchKernelGGL((state_scan_kernel<T, C, REV>), dim3((unsigned)blocks), dim3(256), 0, st,
                     (const T*)p.a, (const T*)p.b, (const T*)p.g, p.g_is_cumsum, p.s_init,
                     (T*)p.s_all, p.s_final, p.scale, p.H, p.K, p.V, p.si);
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
