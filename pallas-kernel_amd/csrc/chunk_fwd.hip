// Per-chunk intra matrix and output for chunked GLA.
//
// Reference: intra matrix tops/ops/gla/chunk.py:300-383 (A = scale (q e^{g~})(k e^{-g~})^T,
// unmasked), output combine chunk.py:441-496 / 1259-1312
// (o = scale (q e^{g~}) h_n + tril(A) v).
//
// One 256-thread block per (chunk, head). The exponent is factored around a per-column
// reference r = (g~_first + g~_last) / 2, so both factors stay within e^{+-|gamma|/2}:
//   qg = q e^{g~ - r},  kg = k e^{r - g~},  A = scale qg kg^T,
//   o  = tril(A) v + qg (scale e^{r} h)      (e^{r} folded into the rows of h).
// The reference kernels use r = 0 (e^{g~} and e^{-g~}), which overflows once a chunk's gate
// sum passes 88; this form holds to 2 x 88.
//
// K is processed in 64-column tiles (A accumulates over them; qg of every tile stays in
// LDS for the inter term), V in 64-column output tiles.
#include "common.hpp"
#include "kernels.hpp"

namespace tops {

template <typename T>
__host__ __device__ constexpr int fwd_o_dyn_bytes(int C, int KP) {
  return ((C * pitch_of<T>(KP) * (int)sizeof(T) + 15) / 16) * 16 + KP * 4;
}

template <typename T, int C>
__global__ __launch_bounds__(256) void chunk_fwd_o_kernel(FwdOArgs p) {
  constexpr int CP = C < 32 ? 32 : C;
  constexpr int RPS = C / 4;
  constexpr int P64 = pitch_of<T>(64), PCP = pitch_of<T>(CP);
  constexpr int NTM = C / 16;           // 16-row tiles of a chunk
  constexpr int NT_A = NTM * NTM;       // 16x16 tiles of A
  constexpr int NA = (NT_A + 3) / 4;    // A tiles per wave
  constexpr int NT_O = NTM * 4;         // 16x16 tiles of a C x 64 output tile
  constexpr int NO = NT_O / 4;          // output tiles per wave
  __shared__ __attribute__((aligned(16))) T sK[C * P64];
  __shared__ __attribute__((aligned(16))) T sA[C * PCP];
  __shared__ __attribute__((aligned(16))) T sVt[64 * PCP];
  __shared__ __attribute__((aligned(16))) T sHt[64 * P64];
  __shared__ float sTot[256];
  extern __shared__ __attribute__((aligned(16))) unsigned char dyn[];

  const int H = p.H, K = p.K, V = p.V;
  const int KT = (K + 63) >> 6, VT = (V + 63) >> 6, KP = KT * 64;
  const int PQ = pitch_of<T>(KP);
  T* sQ = reinterpret_cast<T*>(dyn);
  float* sR = reinterpret_cast<float*>(dyn + ((C * PQ * (int)sizeof(T) + 15) / 16) * 16);

  const T* __restrict__ q = (const T*)p.q;
  const T* __restrict__ k = (const T*)p.k;
  const T* __restrict__ v = (const T*)p.v;
  const T* __restrict__ g = (const T*)p.g;
  const T* __restrict__ hs = (const T*)p.h;
  T* __restrict__ o = (T*)p.o;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int c = L / H, hh = L % H;
  int seq, t0, len;
  chunk_range(p.si, c, seq, t0, len);
  (void)seq;
  const long rsK = (long)H * K, rsV = (long)H * V;
  const long baseK = ((long)t0 * H + hh) * K, baseV = ((long)t0 * H + hh) * V;
  const int col = tid & 63, seg = tid >> 6;

  if (CP > C) {
    for (int i = tid; i < C * (CP - C); i += 256) sA[(i / (CP - C)) * PCP + C + i % (CP - C)] =
        zero_elem<T>();
    for (int i = tid; i < 64 * (CP - C); i += 256)
      sVt[(i / (CP - C)) * PCP + C + i % (CP - C)] = zero_elem<T>();
  }

  const bool compute_A = (p.A_in == nullptr) && (p.A_out != nullptr || o != nullptr);
  f32x4 accA[NA];
#pragma unroll
  for (int j = 0; j < NA; ++j) accA[j] = zero4();

  // ---- phase 1: gates, qg (all K tiles kept), kg (per tile), A accumulation ----
  for (int kt = 0; kt < KT; ++kt) {
    const int gcol = kt * 64 + col;
    const bool kv = gcol < K;
    float gt[RPS];
    float gamma, first;
    tile_cumsum<C>(g + baseK + gcol, rsK, len, kv, p.g_is_cumsum != 0, sTot, gt, gamma,
                   first);
    const float r = 0.5f * (first + gamma);
    if (seg == 0) sR[gcol] = p.scale * gexp<T>(r);
#pragma unroll
    for (int rr = 0; rr < RPS; ++rr) {
      const int row = seg * RPS + rr;
      float qv = 0.f, kvv = 0.f;
      if (row < len && kv) {
        qv = to_f32(q[baseK + (long)row * rsK + gcol]);
        if (compute_A) kvv = to_f32(k[baseK + (long)row * rsK + gcol]);
      }
      const float d = gt[rr] - r;
      sQ[row * PQ + gcol] = from_f32<T>(qv * gexp<T>(d));
      if (compute_A) sK[row * P64 + col] = from_f32<T>(kvv * gexp<T>(-d));
    }
    __syncthreads();
    if (compute_A) {
#pragma unroll
      for (int j = 0; j < NA; ++j) {
        const int t = w + 4 * j;
        if (t < NT_A) {
          const int mi = t / NTM, ni = t % NTM;
          mma_tile<T>(accA[j], sQ + mi * 16 * PQ + kt * 64, PQ, sK + ni * 16 * P64, P64, 64,
                      lane);
        }
      }
    }
    __syncthreads();
  }

  // ---- A epilogue: optional fp32 output, masked copy for A.v ----
  if (compute_A) {
#pragma unroll
    for (int j = 0; j < NA; ++j) {
      const int t = w + 4 * j;
      if (t < NT_A) {
        const int mi = t / NTM, ni = t % NTM;
        const int jj = ni * 16 + (lane & 15);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int ii = mi * 16 + 4 * (lane >> 4) + r;
          const float a = accA[j][r] * p.scale;
          if (p.A_out) p.A_out[(((long)c * C + ii) * H + hh) * C + jj] = a;
          sA[ii * PCP + jj] = from_f32<T>(jj <= ii ? a : 0.f);
        }
      }
    }
  } else if (p.A_in) {
    for (int i = tid; i < C * C; i += 256) {
      const int ii = i / C, jj = i % C;
      const float a = p.A_in[(((long)c * C + ii) * H + hh) * C + jj];
      sA[ii * PCP + jj] = from_f32<T>(jj <= ii ? a : 0.f);
    }
  }
  if (o == nullptr) return;
  __syncthreads();

  // ---- phase 2: per 64-wide V tile, o = tril(A) v + qg (scale e^r h) ----
  for (int vt = 0; vt < VT; ++vt) {
    const int vcol = vt * 64 + col;
    const bool vv = vcol < V;
#pragma unroll
    for (int rr = 0; rr < RPS; ++rr) {
      const int row = seg * RPS + rr;
      float x = 0.f;
      if (row < len && vv) x = to_f32(v[baseV + (long)row * rsV + vcol]);
      sVt[col * PCP + row] = from_f32<T>(x);
    }
    f32x4 acc[NO];
#pragma unroll
    for (int j = 0; j < NO; ++j) acc[j] = zero4();
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NO; ++j) {
      const int t = w + 4 * j;
      const int mi = t >> 2, ni = t & 3;
      mma_tile<T>(acc[j], sA + mi * 16 * PCP, PCP, sVt + ni * 16 * PCP, PCP, CP, lane);
    }
    if (hs) {
      const long hbase = ((long)c * H + hh) * K;
      for (int kt = 0; kt < KT; ++kt) {
        __syncthreads();  // previous sHt readers are done
        // sHt[v][k] = scale e^{r_k} h[k][v]; thread: column v = col, 16 rows k
#pragma unroll 4
        for (int i = 0; i < 16; ++i) {
          const int kk = seg * 16 + i;
          const int gk = kt * 64 + kk;
          float x = 0.f;
          if (gk < K && vv) x = to_f32(hs[(hbase + gk) * V + vcol]) * sR[gk];
          sHt[col * P64 + kk] = from_f32<T>(x);
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < NO; ++j) {
          const int t = w + 4 * j;
          const int mi = t >> 2, ni = t & 3;
          mma_tile<T>(acc[j], sQ + mi * 16 * PQ + kt * 64, PQ, sHt + ni * 16 * P64, P64, 64,
                      lane);
        }
      }
    }
    // store
#pragma unroll
    for (int j = 0; j < NO; ++j) {
      const int t = w + 4 * j;
      const int mi = t >> 2, ni = t & 3;
      const int oc = vt * 64 + ni * 16 + (lane & 15);
      if (oc < V) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int ii = mi * 16 + 4 * (lane >> 4) + r;
          if (ii < len) o[baseV + (long)ii * rsV + oc] = from_f32<T>(acc[j][r]);
        }
      }
    }
    __syncthreads();
  }
}

template <typename T, int C>
static hipError_t launch_fwd_o(const FwdOArgs& p, hipStream_t st) {
  const long blocks = (long)p.si.NC * p.H;
  if (blocks == 0) return hipSuccess;
  const int KP = ((p.K + 63) / 64) * 64;
  const int dyn = fwd_o_dyn_bytes<T>(C, KP);
  hipError_t e = hipFuncSetAttribute((const void*)chunk_fwd_o_kernel<T, C>,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, dyn);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((chunk_fwd_o_kernel<T, C>), dim3((unsigned)blocks), dim3(256), dyn, st, p);
  return hipGetLastError();
}

template <typename T>
static hipError_t dispatch_fwd_o(const FwdOArgs& p, hipStream_t st) {
  switch (p.si.C) {
    case 16: return launch_fwd_o<T, 16>(p, st);
    case 32: return launch_fwd_o<T, 32>(p, st);
    case 64: return launch_fwd_o<T, 64>(p, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t run_chunk_fwd_o(const FwdOArgs& p, int dtype, hipStream_t st) {
  if (dtype == DT_BF16) return dispatch_fwd_o<bf16>(p, st);
  if (dtype == DT_F32) return dispatch_fwd_o<float>(p, st);
  return hipErrorInvalidValue;
}

}  // namespace tops
