// Inter-chunk state scans (forward h and reverse dh) for chunked GLA.
//
// Forward (reference: tops/ops/common/chunk_h.py:18-119, ref chunk.py:206-292):
//   h[n] = h_n ;  h_{n+1} = diag(e^{gamma_n}) h_n + (k * e^{gamma_n - g~})^T v
// Reverse (reference: tops/ops/common/chunk_h.py:399-591):
//   dh[n] = dh ;  dh <- diag(e^{gamma_n}) dh + (scale * q * e^{g~})^T do
// g~ is the chunk-local cumsum of the raw gates (computed here unless given), gamma_n its
// value at the chunk's last valid row.
//
// One 256-thread block owns a 64(k) x VW(v) tile of the K x V state of one (sequence, head)
// and walks that sequence's chunks in order (reverse order for dh). Per chunk there is ONE
// block barrier:
//  * raw a (k or q), g and b (v or do) tiles are fetched with 16-byte loads two chunks ahead
//    (two register sets) and staged in a ring of LDS stages exactly as loaded (row-major);
//  * the chunk-local cumsum is wave-local: lane = 8 row segments x 8 column pairs of the
//    wave's 16 columns; segment offsets and gamma come from lane shuffles;
//  * the gate factor is applied to a in place; the MFMA reads both operands of
//    out[v][k] += sum_c b[c][v] a~[c][k] with transposed fragments, so nothing is transposed
//    in LDS;
//  * the state stays in MFMA accumulators: a lane's four values of a 16x16 tile are four
//    consecutive v of one k and go to the [.., K, V] layout as one vector.
// Stage reuse: a/b stages are written one chunk ahead and read by the MFMA of their chunk,
// so three stages separate every write from the last read by a barrier; g is only read by
// the cumsum before the barrier and needs two.
#include "common.hpp"
#include "kernels.hpp"

namespace tops {

template <typename T, int C, int VW>
struct ScanLayout {
  static constexpr int CP = C < 32 ? 32 : C;   // contraction length (zero padded rows)
  static constexpr int PA = pitch_of<T>(64), PB = pitch_of<T>(VW);
  static constexpr int ES = (int)sizeof(T);
  static constexpr int A = (CP * PA * ES + 15) / 16 * 16;
  static constexpr int B = (CP * PB * ES + 15) / 16 * 16;
  static constexpr int G = (C * PA * ES + 15) / 16 * 16;
  static constexpr int a0 = 0, b0 = 3 * A, g0 = 3 * A + 3 * B;
  static constexpr int gam = g0 + 2 * G;       // 3 x 64 floats
  static constexpr int bytes = gam + 3 * 64 * 4;
};

template <typename T, int C, int VW>
struct ScanRegs {
  static constexpr int EPP = 16 / (int)sizeof(T);
  static constexpr int PPA = (C * (64 / EPP) + 255) / 256;
  static constexpr int PPB = (C * (VW / EPP) + 255) / 256;
  uint4 a[PPA], g[PPA], b[PPB];
};

template <typename T, int C, int VW, bool REV, bool VEC, bool FULL>
__global__ __launch_bounds__(256) void state_scan_kernel(ScanArgs p) {
  using Lay = ScanLayout<T, C, VW>;
  using Regs = ScanRegs<T, C, VW>;
  constexpr int CP = Lay::CP, PA = Lay::PA, PB = Lay::PB;
  constexpr int EPP = Regs::EPP, PPA = Regs::PPA, PPB = Regs::PPB;
  constexpr int RPA = 64 / EPP, RPB = VW / EPP;   // 16-byte pieces per row
  constexpr int RPS = C / 8;                      // rows per lane segment
  constexpr int NVT = VW / 16;                    // 16-row v tiles; tiles per wave
  extern __shared__ __attribute__((aligned(16))) unsigned char dyn[];
  float* sGam = reinterpret_cast<float*>(dyn + Lay::gam);

  const T* __restrict__ a = (const T*)p.a;
  const T* __restrict__ b = (const T*)p.b;
  const T* __restrict__ g = (const T*)p.g;
  T* __restrict__ s_all = (T*)p.s_all;
  const int H = p.H, K = p.K, V = p.V;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int KT = (K + 63) >> 6, VT = (V + VW - 1) / VW;
  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int vt = L % VT;
  const int kt = (L / VT) % KT;
  const int bh = L / (VT * KT);
  const int seq = bh / H, hh = bh % H;
  const int kbase = kt * 64, vbase = vt * VW;

  int bos, eos, c0, nc;
  seq_range(p.si, seq, bos, eos, c0, nc);

  if (CP > C) {   // zero contraction rows [C, CP) of every a / b stage
    for (int s = 0; s < 3; ++s) {
      T* sa = reinterpret_cast<T*>(dyn + Lay::a0 + s * Lay::A);
      T* sb = reinterpret_cast<T*>(dyn + Lay::b0 + s * Lay::B);
      for (int i = tid; i < (CP - C) * PA; i += 256) sa[C * PA + i] = zero_elem<T>();
      for (int i = tid; i < (CP - C) * PB; i += 256) sb[C * PB + i] = zero_elem<T>();
    }
  }

  // accumulator tiles of this wave: v tile (w % NVT), k tiles (w / NVT) * NVT + n
  const int vtile = w % NVT, ktile0 = (w / NVT) * NVT;
  const int kcol = kbase + ktile0 * 16 + (lane & 15);        // + 16 n
  const int vrow = vbase + vtile * 16 + 4 * (lane >> 4);     // + r
  f32x4 acc[NVT];
#pragma unroll
  for (int n = 0; n < NVT; ++n) {
    acc[n] = zero4();
    const int kk = kcol + 16 * n;
    if (p.s_init && kk < K) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (vrow + r < V) {
          // routed through a VGPR: a load straight into the accumulator registers makes the
          // compiler drain every outstanding load at the top of the chunk loop
          const float x = p.s_init[(((long)seq * H + hh) * K + kk) * V + vrow + r];
          float y;
          asm volatile("v_mov_b32 %0, %1" : "=v"(y) : "v"(x));
          acc[n][r] = y;
        }
    }
  }

  // Fetch of chunk `step` into registers. Aligned path: every lane issues the same
  // unconditional loads (addresses clamped into the chunk and the row; steps past the end
  // re-read the last chunk), so the loads of the two register sets stay in flight across a
  // whole chunk; invalid pieces are zeroed when staged.
  auto issue = [&](int step, Regs& R) {
    const int sc = VEC ? min(step, nc - 1) : step;
    const int ci = REV ? (nc - 1 - sc) : sc;
    const int t0 = bos + ci * C;
    const int len = min(C, eos - t0);
#pragma unroll
    for (int j = 0; j < PPA; ++j) {
      if constexpr (VEC) {
        const int pc = min(tid + 256 * j, C * RPA - 1);
        const int row = min(pc / RPA, len - 1);
        const int col0 = FULL ? (pc % RPA) * EPP : min((pc % RPA) * EPP, K - kbase - EPP);
        const long o = ((long)(t0 + row) * H + hh) * K + kbase + col0;
        R.a[j] = *reinterpret_cast<const uint4*>(a + o);
        R.g[j] = *reinterpret_cast<const uint4*>(g + o);
      } else {
        const int pc = tid + 256 * j;
        const int row = pc / RPA, col0 = (pc % RPA) * EPP;
        R.a[j] = R.g[j] = make_uint4(0, 0, 0, 0);
        if (pc < C * RPA && row < len) {
          const long rk = ((long)(t0 + row) * H + hh) * K + kbase;
          R.a[j] = gload16<T, false>(a + rk, col0, K - kbase - col0);
          R.g[j] = gload16<T, false>(g + rk, col0, K - kbase - col0);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < PPB; ++j) {
      if constexpr (VEC) {
        const int pc = min(tid + 256 * j, C * RPB - 1);
        const int row = min(pc / RPB, len - 1);
        const int col0 = FULL ? (pc % RPB) * EPP : min((pc % RPB) * EPP, V - vbase - EPP);
        R.b[j] = *reinterpret_cast<const uint4*>(b + ((long)(t0 + row) * H + hh) * V + vbase +
                                                 col0);
      } else {
        const int pc = tid + 256 * j;
        const int row = pc / RPB, col0 = (pc % RPB) * EPP;
        R.b[j] = make_uint4(0, 0, 0, 0);
        if (pc < C * RPB && row < len)
          R.b[j] = gload16<T, false>(b + ((long)(t0 + row) * H + hh) * V + vbase, col0,
                                     V - vbase - col0);
      }
    }
  };
  // Stage chunk `step` (fetched by issue) into its LDS stages.
  auto commit = [&](const Regs& R, int step) {
    const int sc = min(step, nc - 1);
    const int ci = REV ? (nc - 1 - sc) : sc;
    const int len = min(C, eos - (bos + ci * C));
    T* sa = reinterpret_cast<T*>(dyn + Lay::a0 + (step % 3) * Lay::A);
    T* sb = reinterpret_cast<T*>(dyn + Lay::b0 + (step % 3) * Lay::B);
    T* sg = reinterpret_cast<T*>(dyn + Lay::g0 + (step & 1) * Lay::G);
#pragma unroll
    for (int j = 0; j < PPA; ++j) {
      const int pc = tid + 256 * j;
      if (pc < C * RPA) {
        const int row = pc / RPA, col0 = (pc % RPA) * EPP;
        const uint32_t m = (!VEC || (row < len && (FULL || kbase + col0 < K))) ? ~0u : 0u;
        const int o = row * PA + col0;
        *reinterpret_cast<uint4*>(sa + o) = mask16(R.a[j], m);
        *reinterpret_cast<uint4*>(sg + o) = mask16(R.g[j], m);
      }
    }
#pragma unroll
    for (int j = 0; j < PPB; ++j) {
      const int pc = tid + 256 * j;
      if (pc < C * RPB) {
        const int row = pc / RPB, col0 = (pc % RPB) * EPP;
        const uint32_t m = (!VEC || (row < len && (FULL || vbase + col0 < V))) ? ~0u : 0u;
        *reinterpret_cast<uint4*>(sb + row * PB + col0) = mask16(R.b[j], m);
      }
    }
  };

  const int cpl = lane & 7, seg = lane >> 3;
  const int c_0 = 16 * w + 2 * cpl, c_1 = c_0 + 1;
  const bool gcum = p.g_is_cumsum != 0;

  // one chunk: gating of chunk `step` (stage step%3), staging of chunk step+1 from Rn,
  // fetch of chunk step+3 into Rn, barrier, state store and update
  auto body = [&](int step, Regs& Rn) {
    const int ci = REV ? (nc - 1 - step) : step;
    const int t0 = bos + ci * C;
    const int len = min(C, eos - t0);
    T* sa = reinterpret_cast<T*>(dyn + Lay::a0 + (step % 3) * Lay::A);
    const T* sb = reinterpret_cast<const T*>(dyn + Lay::b0 + (step % 3) * Lay::B);
    const T* sg = reinterpret_cast<const T*>(dyn + Lay::g0 + (step & 1) * Lay::G);
    float* gam_s = sGam + (step % 3) * 64;

    float g0[RPS], g1[RPS];
    float run0 = 0.f, run1 = 0.f;
#pragma unroll
    for (int rr = 0; rr < RPS; ++rr) {
      float x0, x1;
      Pair<T>::ld(sg + (seg * RPS + rr) * PA + c_0, x0, x1);
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
    float gam0, gam1, off0 = 0.f, off1 = 0.f;
    if (gcum) {   // gamma = given value at the last valid row
      const int lr = len - 1;
      float v0 = 0.f, v1 = 0.f;
#pragma unroll
      for (int rr = 0; rr < RPS; ++rr)
        if (seg * RPS + rr == lr) {
          v0 = g0[rr];
          v1 = g1[rr];
        }
      const int src = (lr / RPS) * 8 + cpl;
      gam0 = __shfl(v0, src);
      gam1 = __shfl(v1, src);
    } else {      // inclusive scan of the 8 segment totals across lanes 8 apart
      float x0 = run0, x1 = run1;
#pragma unroll
      for (int d = 8; d < 64; d <<= 1) {
        const float y0 = __shfl_up(x0, d), y1 = __shfl_up(x1, d);
        if (lane >= d) {
          x0 += y0;
          x1 += y1;
        }
      }
      off0 = x0 - run0;
      off1 = x1 - run1;
      gam0 = __shfl(x0, 56 + cpl);
      gam1 = __shfl(x1, 56 + cpl);
    }
#pragma unroll
    for (int rr = 0; rr < RPS; ++rr) {
      const int row = seg * RPS + rr;
      float e0, e1;
      if (REV) {
        e0 = p.scale * gexp<T>(g0[rr] + off0);
        e1 = p.scale * gexp<T>(g1[rr] + off1);
      } else {
        e0 = gexp<T>(gam0 - (g0[rr] + off0));
        e1 = gexp<T>(gam1 - (g1[rr] + off1));
      }
      if (gcum && row >= len) e0 = e1 = 0.f;
      float x0, x1;
      Pair<T>::ld(sa + row * PA + c_0, x0, x1);
      Pair<T>::st(sa + row * PA + c_0, x0 * e0, x1 * e1);
    }
    if (seg == 0) {
      gam_s[c_0] = gexp<T>(gam0);
      gam_s[c_1] = gexp<T>(gam1);
    }
    if (VEC || step + 1 < nc) {
      commit(Rn, step + 1);
      if (VEC || step + 3 < nc) issue(step + 3, Rn);
    }
    __syncthreads();

    // state entering this chunk (forward) / leaving it (reverse)
    if (s_all) {
      const long cbase = ((long)(c0 + ci) * H + hh) * K;
#pragma unroll
      for (int n = 0; n < NVT; ++n) {
        const int kk = kcol + 16 * n;
        if (!FULL && kk >= K) continue;
        T* dst = s_all + (cbase + kk) * V + vrow;
        if (FULL || (VEC && vrow + 3 < V)) {
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
#pragma unroll
    for (int n = 0; n < NVT; ++n) acc[n] *= gam_s[(ktile0 + n) * 16 + (lane & 15)];
#pragma unroll
    for (int kk = 0; kk < CP; kk += 32) {
      const Frag<T> x = ld_frag_t(sb + kk * PB + vtile * 16, PB, lane);
#pragma unroll
      for (int n = 0; n < NVT; ++n)
        mma(acc[n], x, ld_frag_t(sa + kk * PA + (ktile0 + n) * 16, PA, lane));
    }
  };

  Regs R0, R1;
  if (nc > 0) {
    issue(0, R0);
    commit(R0, 0);
    if (VEC || nc > 1) issue(1, R1);
    __builtin_amdgcn_sched_barrier(0);   // keep chunk 1's loads ahead of chunk 2's
    if (VEC || nc > 2) issue(2, R0);
  }
  __syncthreads();
  for (int step = 0; step < nc; step += 2) {
    body(step, R1);
    if (step + 1 < nc) body(step + 1, R0);
  }

  if (p.s_final) {
#pragma unroll
    for (int n = 0; n < NVT; ++n) {
      const int kk = kcol + 16 * n;
      if (kk >= K) continue;
      float* dst = p.s_final + (((long)seq * H + hh) * K + kk) * V + vrow;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (vrow + r < V) dst[r] = acc[n][r];
    }
  }
}

template <typename T, int C, int VW, bool REV, bool VEC, bool FULL>
static hipError_t launch_scan1(const ScanArgs& p, hipStream_t st, long blocks) {
  using Lay = ScanLayout<T, C, VW>;
  const void* fn = (const void*)state_scan_kernel<T, C, VW, REV, VEC, FULL>;
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, Lay::bytes);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((state_scan_kernel<T, C, VW, REV, VEC, FULL>), dim3((unsigned)blocks),
                     dim3(256), Lay::bytes, st, p);
  return hipGetLastError();
}

template <typename T, int C, int VW, bool REV>
static hipError_t launch_scan(const ScanArgs& p, hipStream_t st, long blocks) {
  if (!p.vec) return launch_scan1<T, C, VW, REV, false, false>(p, st, blocks);
  if (p.K % 64 == 0 && p.V % VW == 0)
    return launch_scan1<T, C, VW, REV, true, true>(p, st, blocks);
  return launch_scan1<T, C, VW, REV, true, false>(p, st, blocks);
}

// V tiles of 64 when that already gives two blocks per CU (256 CUs), else 32.
template <typename T, int C, bool REV>
static hipError_t pick_vw(const ScanArgs& p, hipStream_t st) {
  const long nbh = (long)p.si.N * p.H * ((p.K + 63) / 64);
  if (nbh == 0) return hipSuccess;
  const long b64 = nbh * ((p.V + 63) / 64);
  if (b64 >= 512) return launch_scan<T, C, 64, REV>(p, st, b64);
  return launch_scan<T, C, 32, REV>(p, st, nbh * ((p.V + 31) / 32));
}

template <typename T, bool REV>
static hipError_t dispatch_c(const ScanArgs& p, hipStream_t st) {
  switch (p.si.C) {
    case 16: return pick_vw<T, 16, REV>(p, st);
    case 32: return pick_vw<T, 32, REV>(p, st);
    case 64: return pick_vw<T, 64, REV>(p, st);
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
