// Fused chunked-GLA forward: inter-chunk state scan and per-chunk output in one pass.
//
// Reference semantics: chunk_gla_fwd, tops/ops/gla/chunk.py:1083-1179 (state scan
// chunk_h.py:18-119, intra matrix chunk.py:350-383, output chunk.py:1259-1312). Per chunk n
// (g~ = chunk-local cumsum of g, gamma = its last row, r = (g~_first + gamma) / 2 per column):
//   qg = q e^{g~-r},  kg = k e^{r-g~},  kd = k e^{gamma-g~},  A = scale tril(qg kg^T)
//   o  = A v + qg (scale e^{r} h_n)
//   h_{n+1} = e^{gamma} h_n + kd^T v
//
// One 256-thread block per (sequence, head, VW-wide slab of V) walks the sequence's chunks
// in order. The K x VW state stays in MFMA accumulators (orientation out[v][k], so a lane's
// four values are four consecutive v of one k). Every chunk's q, k, g (all K columns) and v
// (the slab) are fetched with 16-byte loads one chunk ahead into registers and written to
// LDS while the current chunk computes. The slabs of one (sequence, head) recompute the
// same A (the price of parallelism) and are placed on one XCD so their q/k/g reads share L2.
//
// Per chunk: column scan of g (thread = column) -> gating (qg, kg row-major; kd, v
// transposed) -> [h' = scale e^r h into LDS, h_n to HBM, A on MFMA] -> [o^T = v^T A^T +
// h'^T qg^T on MFMA, stored 4 values per lane; state update kd^T v on MFMA].
#include "common.hpp"
#include "kernels.hpp"

namespace tops {

__host__ __device__ constexpr int a16(int b) { return (b + 15) / 16 * 16; }

template <typename T, int C, int KP, int VW>
struct FFLayout {
  static constexpr int CP = C < 32 ? 32 : C;
  static constexpr int PK = pitch_of<T>(KP), PV = pitch_of<T>(VW), PC = pitch_of<T>(CP);
  static constexpr int ES = (int)sizeof(T);
  static constexpr int qr = 0;
  static constexpr int kr = qr + a16(C * PK * ES);
  static constexpr int gr = kr + a16(C * PK * ES);
  static constexpr int vr = gr + a16(C * PK * ES);
  static constexpr int q = vr + a16(C * PV * ES);
  static constexpr int k = q + a16(C * PK * ES);
  static constexpr int kdT = k + a16(C * PK * ES);
  static constexpr int vT = kdT + a16(KP * PC * ES);
  static constexpr int ht = vT + a16(VW * PC * ES);
  static constexpr int a = ht + a16(VW * PK * ES);
  static constexpr int tot = a + a16(C * PC * ES);
  static constexpr int rs = tot + 256 * 4;
  static constexpr int gam = rs + KP * 4;
  static constexpr int first = gam + KP * 4;
  static constexpr int bytes = first + KP * 4;
};

// 16 bytes of a row starting at column col0 (zero-filled past `nvalid` columns).
template <typename T>
__device__ __forceinline__ uint4 load_piece(const T* __restrict__ row, int col0, int nvalid,
                                            bool vec) {
  constexpr int EPP = 16 / (int)sizeof(T);
  uint4 r = make_uint4(0, 0, 0, 0);
  if (nvalid >= EPP && vec) return *reinterpret_cast<const uint4*>(row + col0);
  if (nvalid > 0) {
    T tmp[EPP];
#pragma unroll
    for (int e = 0; e < EPP; ++e) tmp[e] = e < nvalid ? row[col0 + e] : zero_elem<T>();
    __builtin_memcpy(&r, tmp, 16);
  }
  return r;
}

template <typename T, int C, int KP, int VW>
__global__ __launch_bounds__(256) void chunk_fwd_fused_kernel(FusedFwdArgs p) {
  using Lay = FFLayout<T, C, KP, VW>;
  constexpr int CP = Lay::CP, PK = Lay::PK, PV = Lay::PV, PC = Lay::PC;
  constexpr int EPP = 16 / (int)sizeof(T);
  constexpr int NSEG = 256 / KP;         // column-scan row segments
  constexpr int RPS = C / NSEG;          // rows per thread in the column scan
  constexpr int QPR = KP / EPP;          // 16-byte pieces per [KP] row
  constexpr int QPIECES = C * QPR;
  constexpr int QPT = (QPIECES + 255) / 256;
  constexpr int VPR = VW / EPP;
  constexpr int VPIECES = C * VPR;
  constexpr int VPT = (VPIECES + 255) / 256;
  constexpr int VSEG = 256 / VW;         // v^T transpose row segments
  constexpr int VRPS = C / VSEG;
  constexpr int NTC = C / 16, NTV = VW / 16, NTK = KP / 16;
  constexpr int NST = NTV * NTK;         // state tiles (v tile, k tile)
  constexpr int SPW = NST / 4;
  constexpr int NOT = NTV * NTC;         // o^T tiles (v tile, row tile)
  constexpr int OPW = (NOT + 3) / 4;
  constexpr int NAL = NTC * (NTC + 1) / 2;  // lower-triangular A tiles
  constexpr int APW = (NAL + 3) / 4;
  static_assert(NST % 4 == 0, "state tiles must split over 4 waves");
  static_assert(RPS >= 1 && VRPS >= 1, "chunk too small for the thread mapping");
  static_assert(Lay::bytes <= 163840, "LDS budget of one workgroup exceeded");

  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  T* sQr = reinterpret_cast<T*>(smem + Lay::qr);
  T* sKr = reinterpret_cast<T*>(smem + Lay::kr);
  T* sGr = reinterpret_cast<T*>(smem + Lay::gr);
  T* sVr = reinterpret_cast<T*>(smem + Lay::vr);
  T* sQ = reinterpret_cast<T*>(smem + Lay::q);
  T* sK = reinterpret_cast<T*>(smem + Lay::k);
  T* sKdT = reinterpret_cast<T*>(smem + Lay::kdT);
  T* sVT = reinterpret_cast<T*>(smem + Lay::vT);
  T* sHt = reinterpret_cast<T*>(smem + Lay::ht);
  T* sA = reinterpret_cast<T*>(smem + Lay::a);
  float* sTot = reinterpret_cast<float*>(smem + Lay::tot);
  float* sRs = reinterpret_cast<float*>(smem + Lay::rs);
  float* sGam = reinterpret_cast<float*>(smem + Lay::gam);
  float* sFirst = reinterpret_cast<float*>(smem + Lay::first);

  const T* __restrict__ q = (const T*)p.q;
  const T* __restrict__ k = (const T*)p.k;
  const T* __restrict__ v = (const T*)p.v;
  const T* __restrict__ g = (const T*)p.g;
  T* __restrict__ o = (T*)p.o;
  T* __restrict__ hout = (T*)p.h_out;

  const int H = p.H, K = p.K, V = p.V;
  const int NV = (V + VW - 1) / VW;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int vt = L % NV;
  const int bh = L / NV;
  const int seq = bh / H, hh = bh % H;
  const int v0 = vt * VW;
  const bool vecK = p.vec_k != 0, vecV = p.vec_v != 0;

  int bos, eos, c0, nc;
  seq_range(p.si, seq, bos, eos, c0, nc);

  // zero buffers whose padding / masked part is never written
  for (int i = tid; i < C * PC; i += 256) sA[i] = zero_elem<T>();
  for (int i = tid; i < VW * PC; i += 256) sVT[i] = zero_elem<T>();
  for (int i = tid; i < KP * PC; i += 256) sKdT[i] = zero_elem<T>();

  // ---- state: tiles s = w*SPW + j, (mv = s / NTK, nk = s % NTK); out[v][k] ----
  f32x4 acc[SPW];
  const long sbase = ((long)seq * H + hh) * K;
#pragma unroll
  for (int j = 0; j < SPW; ++j) {
    const int s = w * SPW + j;
    const int mv = s / NTK, nk = s % NTK;
    const int kk = nk * 16 + (lane & 15);
    const int vv = v0 + mv * 16 + 4 * (lane >> 4);
    acc[j] = zero4();
    if (p.h0 && kk < K) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (vv + r < V) acc[j][r] = p.h0[(sbase + kk) * V + vv + r];
    }
  }

  // ---- prefetch machinery ----
  uint4 pq[QPT], pk[QPT], pg[QPT], pv[VPT];
  auto issue = [&](int ci) {
    const int t0 = bos + ci * C;
    const int len = min(C, eos - t0);
#pragma unroll
    for (int j = 0; j < QPT; ++j) {
      const int pc = tid + 256 * j;
      pq[j] = pk[j] = pg[j] = make_uint4(0, 0, 0, 0);
      if (pc < QPIECES) {
        const int row = pc / QPR, col0 = (pc % QPR) * EPP;
        if (row < len) {
          const long rb = ((long)(t0 + row) * H + hh) * K;
          pq[j] = load_piece<T>(q + rb, col0, K - col0, vecK);
          pk[j] = load_piece<T>(k + rb, col0, K - col0, vecK);
          pg[j] = load_piece<T>(g + rb, col0, K - col0, vecK);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int pc = tid + 256 * j;
      pv[j] = make_uint4(0, 0, 0, 0);
      if (pc < VPIECES) {
        const int row = pc / VPR, col0 = (pc % VPR) * EPP;
        if (row < len)
          pv[j] = load_piece<T>(v + ((long)(t0 + row) * H + hh) * V, v0 + col0,
                                V - (v0 + col0), vecV);
      }
    }
  };
  auto commit = [&]() {
#pragma unroll
    for (int j = 0; j < QPT; ++j) {
      const int pc = tid + 256 * j;
      if (pc < QPIECES) {
        const int row = pc / QPR, col0 = (pc % QPR) * EPP;
        *reinterpret_cast<uint4*>(sQr + row * PK + col0) = pq[j];
        *reinterpret_cast<uint4*>(sKr + row * PK + col0) = pk[j];
        *reinterpret_cast<uint4*>(sGr + row * PK + col0) = pg[j];
      }
    }
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int pc = tid + 256 * j;
      if (pc < VPIECES) {
        const int row = pc / VPR, col0 = (pc % VPR) * EPP;
        *reinterpret_cast<uint4*>(sVr + row * PV + col0) = pv[j];
      }
    }
  };

  if (nc > 0) {
    issue(0);
    commit();
    if (nc > 1) issue(1);
  }
  __syncthreads();

  const int col = tid % KP, seg = tid / KP;        // column-scan mapping
  const int vcol = tid % VW, vseg = tid / VW;      // v^T mapping

  for (int ci = 0; ci < nc; ++ci) {
    const int t0 = bos + ci * C;
    const int len = min(C, eos - t0);
    const long cidx = (long)(c0 + ci);

    // ---- (1) column scan of g, gating, transposes ----
    float gt[RPS];
    float run = 0.f;
#pragma unroll
    for (int rr = 0; rr < RPS; ++rr) {
      run += to_f32(sGr[(seg * RPS + rr) * PK + col]);
      gt[rr] = run;
    }
    sTot[seg * KP + col] = run;
    if (seg == 0) sFirst[col] = gt[0];
    __syncthreads();
    float off = 0.f, gamma = 0.f;
#pragma unroll
    for (int s = 0; s < NSEG; ++s) {
      const float x = sTot[s * KP + col];
      off += (s < seg) ? x : 0.f;
      gamma += x;
    }
    const float r = 0.5f * (sFirst[col] + gamma);
    const float fkd = gexp<T>(gamma - r);
#pragma unroll
    for (int rr = 0; rr < RPS; ++rr) {
      const int row = seg * RPS + rr;
      const float d = gt[rr] + off - r;
      const float qv = to_f32(sQr[row * PK + col]);
      const float kv = to_f32(sKr[row * PK + col]);
      const float e = gexp<T>(d), ei = gexp<T>(-d);
      sQ[row * PK + col] = from_f32<T>(qv * e);
      sK[row * PK + col] = from_f32<T>(kv * ei);
      sKdT[col * PC + row] = from_f32<T>(kv * ei * fkd);
    }
    if (seg == 0) {
      sRs[col] = p.scale * gexp<T>(r);
      sGam[col] = gexp<T>(gamma);
    }
#pragma unroll
    for (int rr = 0; rr < VRPS; ++rr) {
      const int row = vseg * VRPS + rr;
      sVT[vcol * PC + row] = sVr[row * PV + vcol];
    }
    __syncthreads();

    // ---- (2) h' = scale e^r h into LDS, h_n to HBM, A = scale tril(qg kg^T) ----
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
      const int s = w * SPW + j;
      const int mv = s / NTK, nk = s % NTK;
      const int kk = nk * 16 + (lane & 15);
      const int vl = mv * 16 + 4 * (lane >> 4);
      const float f = sRs[kk];
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) sHt[(vl + rr) * PK + kk] = from_f32<T>(acc[j][rr] * f);
      if (hout && kk < K) {
        const int vv = v0 + vl;
        T* dst = hout + ((cidx * H + hh) * K + kk) * V + vv;
        if (vecV && vv + 3 < V) {
          if (sizeof(T) == 2) {
            uint2 pk2;
            pk2.x = (uint32_t)from_f32<bf16>(acc[j][0]).u |
                    ((uint32_t)from_f32<bf16>(acc[j][1]).u << 16);
            pk2.y = (uint32_t)from_f32<bf16>(acc[j][2]).u |
                    ((uint32_t)from_f32<bf16>(acc[j][3]).u << 16);
            *reinterpret_cast<uint2*>(dst) = pk2;
          } else {
            *reinterpret_cast<float4*>(dst) =
                make_float4(acc[j][0], acc[j][1], acc[j][2], acc[j][3]);
          }
        } else {
#pragma unroll
          for (int rr = 0; rr < 4; ++rr)
            if (vv + rr < V) dst[rr] = from_f32<T>(acc[j][rr]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < APW; ++j) {
      const int a = w + 4 * j;
      if (a < NAL) {
        int mi = 0;
        while ((mi + 1) * (mi + 2) / 2 <= a) ++mi;
        const int ni = a - mi * (mi + 1) / 2;
        f32x4 t = zero4();
        mma_tile<T>(t, sQ + mi * 16 * PK, PK, sK + ni * 16 * PK, PK, KP, lane);
        const int jj = ni * 16 + (lane & 15);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int ii = mi * 16 + 4 * (lane >> 4) + rr;
          sA[ii * PC + jj] = from_f32<T>(jj <= ii ? t[rr] * p.scale : 0.f);
        }
      }
    }
    // next chunk's raw tiles (raw buffers are free since the sync above)
    if (ci + 1 < nc) {
      commit();
      if (ci + 2 < nc) issue(ci + 2);
    }
    __syncthreads();

    // ---- (3) o^T = v^T A^T + h'^T qg^T ; state update ----
#pragma unroll
    for (int j = 0; j < OPW; ++j) {
      const int t = w + 4 * j;
      if (t < NOT) {
        const int mv = t / NTC, ni = t % NTC;
        f32x4 ot = zero4();
        mma_tile<T>(ot, sVT + mv * 16 * PC, PC, sA + ni * 16 * PC, PC, CP, lane);
        mma_tile<T>(ot, sHt + mv * 16 * PK, PK, sQ + ni * 16 * PK, PK, KP, lane);
        const int ii = ni * 16 + (lane & 15);
        const int vv = v0 + mv * 16 + 4 * (lane >> 4);
        if (ii < len) {
          T* dst = o + ((long)(t0 + ii) * H + hh) * V + vv;
          if (vecV && vv + 3 < V) {
            if (sizeof(T) == 2) {
              uint2 pk2;
              pk2.x = (uint32_t)from_f32<bf16>(ot[0]).u |
                      ((uint32_t)from_f32<bf16>(ot[1]).u << 16);
              pk2.y = (uint32_t)from_f32<bf16>(ot[2]).u |
                      ((uint32_t)from_f32<bf16>(ot[3]).u << 16);
              *reinterpret_cast<uint2*>(dst) = pk2;
            } else {
              *reinterpret_cast<float4*>(dst) = make_float4(ot[0], ot[1], ot[2], ot[3]);
            }
          } else {
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
              if (vv + rr < V) dst[rr] = from_f32<T>(ot[rr]);
          }
        }
      }
    }
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
      const int s = w * SPW + j;
      const int mv = s / NTK, nk = s % NTK;
      acc[j] *= sGam[nk * 16 + (lane & 15)];
      mma_tile<T>(acc[j], sVT + mv * 16 * PC, PC, sKdT + nk * 16 * PC, PC, CP, lane);
    }
    __syncthreads();
  }

  if (p.ht) {
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
      const int s = w * SPW + j;
      const int mv = s / NTK, nk = s % NTK;
      const int kk = nk * 16 + (lane & 15);
      const int vv = v0 + mv * 16 + 4 * (lane >> 4);
      if (kk < K) {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          if (vv + rr < V) p.ht[(sbase + kk) * V + vv + rr] = acc[j][rr];
      }
    }
  }
}

template <typename T, int C, int KP, int VW>
static hipError_t launch_ff(const FusedFwdArgs& p, hipStream_t st) {
  using Lay = FFLayout<T, C, KP, VW>;
  const int NV = (p.V + VW - 1) / VW;
  const long blocks = (long)p.si.N * p.H * NV;
  if (blocks == 0) return hipSuccess;
  hipError_t e = hipFuncSetAttribute((const void*)chunk_fwd_fused_kernel<T, C, KP, VW>,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, Lay::bytes);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((chunk_fwd_fused_kernel<T, C, KP, VW>), dim3((unsigned)blocks), dim3(256),
                     Lay::bytes, st, p);
  return hipGetLastError();
}

template <typename T, int C, int KP>
static hipError_t pick_vw(const FusedFwdArgs& p, hipStream_t st) {
  // wider slabs recompute A fewer times; narrow ones give >= 256 blocks on 256 CUs
  const long wide = (long)p.si.N * p.H * ((p.V + 63) / 64);
  if (wide >= 256 || p.V <= 32) return p.V <= 32 ? launch_ff<T, C, KP, 32>(p, st)
                                                 : launch_ff<T, C, KP, 64>(p, st);
  return launch_ff<T, C, KP, 32>(p, st);
}

template <typename T, int C>
static hipError_t pick_kp(const FusedFwdArgs& p, hipStream_t st) {
  if (p.K <= 64) return pick_vw<T, C, 64>(p, st);
  return pick_vw<T, C, 128>(p, st);
}

bool fused_fwd_supported(int dtype, int C, int K) {
  if (K > 128) return false;
  if (dtype == DT_BF16) return C == 16 || C == 32 || C == 64;
  if (dtype == DT_F32) return C == 16 || C == 32;
  return false;
}

hipError_t run_chunk_fwd_fused(const FusedFwdArgs& p, int dtype, hipStream_t st) {
  if (!fused_fwd_supported(dtype, p.si.C, p.K)) return hipErrorInvalidValue;
  if (dtype == DT_BF16) {
    switch (p.si.C) {
      case 16: return pick_kp<bf16, 16>(p, st);
      case 32: return pick_kp<bf16, 32>(p, st);
      default: return pick_kp<bf16, 64>(p, st);
    }
  }
  if (p.si.C == 16) return pick_kp<float, 16>(p, st);
  return pick_kp<float, 32>(p, st);
}

}  // namespace tops
