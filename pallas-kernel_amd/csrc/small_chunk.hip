// Chunked GLA sub-functions at chunk sizes 4 and 8 (below the 16-row MFMA tile): the per-chunk
// states of the forward and reverse scans, the unmasked intra matrix and the output combine.
// They serve the reference's sub-function API at those chunk sizes (the reference's jnp
// refs take any chunk size; its test tables drive 4 and 8); the training path runs 64-row
// chunks. Plain fp32 vector code, one thread per output element.
//
// Reference semantics:
//  * forward states, tops/ops/gla/chunk.py:206-292 (chunk_fwd_h_ref): h[n] = state entering
//    chunk n; h_{n+1} = e^{gamma} h_n + sum_j (k_j e^{gamma - g~_j})^T v_j, gamma = g~ of the
//    chunk's last row;
//  * reverse states, tops/ops/common/chunk_h.py:399-492 (chunk_bwd_dh_ref): dh[n] = gradient
//    w.r.t. the state leaving chunk n; dh <- e^{gamma} dh + sum_i (scale q_i e^{g~_i})^T do_i;
//  * intra matrix, tops/ops/gla/chunk.py:300-342: A_ij = scale sum_k q_ik k_jk e^{g~_ik -
//    g~_jk} for every (i, j) of the chunk (unmasked);
//  * output, tops/ops/gla/chunk.py:441-496: o_i = scale (q_i e^{g~_i}) h_n + sum_{j<=i} A_ij v_j.
// g~ is the chunk-local cumsum of the gates (given, or formed here from raw gates). Rows past
// a sequence's end (partial last chunk) take no part; their A entries are zero.
#include "common.hpp"
#include "kernels.hpp"

namespace tops {

namespace {

template <typename T>
__device__ __forceinline__ float ldf(const T* p, long i) {
  return to_f32(p[i]);
}

// Chunk-local cumsum of column kk over rows [0, len) of the chunk starting at token t0
// (row stride rs elements): gt[j] for j < len.
template <typename T, int C>
__device__ __forceinline__ void col_cumsum(const T* g, long t0, long rs, long col, int len,
                                           bool is_cumsum, float (&gt)[C]) {
  float run = 0.f;
#pragma unroll
  for (int j = 0; j < C; ++j) {
    const float x = j < len ? ldf(g, (t0 + j) * rs + col) : 0.f;
    run = is_cumsum ? x : run + x;
    gt[j] = j < len ? run : 0.f;
  }
}

}  // namespace

// Grid: (sequence, head) x ceil(K V / 256) blocks of 256 threads; thread -> state element
// (kk, vv) with vv fastest. Walks the sequence's chunks in flow order (REV: last to first).
template <typename T, int C, bool REV>
__global__ __launch_bounds__(256) void small_state_kernel(ScanArgs p) {
  const int H = p.H, K = p.K, V = p.V;
  const long KV = (long)K * V;
  const long per = (KV + 255) / 256;
  const long L = blockIdx.x;
  const int sh = (int)(L / per);
  const int seq = sh / H, hh = sh % H;
  const long e = (L % per) * 256 + threadIdx.x;
  if (e >= KV) return;
  const int kk = (int)(e / V), vv = (int)(e % V);
  int bos, eos, c0, nc;
  seq_range(p.si, seq, bos, eos, c0, nc);
  const T* __restrict__ a = (const T*)p.a;
  const T* __restrict__ b = (const T*)p.b;
  const T* __restrict__ g = (const T*)p.g;
  T* __restrict__ s_all = (T*)p.s_all;
  const long rsK = (long)H * K, rsV = (long)H * V;
  const long sidx = ((long)seq * H + hh) * KV + e;
  float s = p.s_init ? p.s_init[sidx] : 0.f;
  for (int n = 0; n < nc; ++n) {
    const int c = REV ? nc - 1 - n : n;
    const long t0 = bos + (long)c * C;
    const int len = (int)min((long)C, (long)eos - t0);
    if (s_all) s_all[((long)(c0 + c) * H + hh) * KV + e] = from_f32<T>(s);
    float gt[C];
    col_cumsum<T, C>(g, t0, rsK, (long)hh * K + kk, len, p.g_is_cumsum != 0, gt);
    const float gam = gt[len - 1];
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < C; ++j) {
      if (j < len) {
        const float x = ldf(a, (t0 + j) * rsK + (long)hh * K + kk);
        const float y = ldf(b, (t0 + j) * rsV + (long)hh * V + vv);
        const float f = REV ? p.scale * expf(gt[j]) : expf(gam - gt[j]);
        acc += x * f * y;
      }
    }
    s = s * expf(gam) + acc;
  }
  if (p.s_final) p.s_final[sidx] = s;
}

// One 256-thread block per (chunk, head). LDS: the chunk's gate cumsum [C][K] and q e^{g~}
// [C][K] (float32), A [C][C].
template <typename T, int C>
__global__ __launch_bounds__(256) void small_out_kernel(FwdOArgs p) {
  extern __shared__ float sm[];
  const int H = p.H, K = p.K, V = p.V;
  float* sG = sm;                   // [C][K]
  float* sQe = sm + C * K;          // [C][K] q e^{g~}
  __shared__ float sA[C * C];
  const int c = blockIdx.x / H, hh = blockIdx.x % H;
  int seq, t0i, len;
  chunk_range(p.si, c, seq, t0i, len);
  const long t0 = t0i;
  const T* __restrict__ q = (const T*)p.q;
  const T* __restrict__ k = (const T*)p.k;
  const T* __restrict__ v = (const T*)p.v;
  const T* __restrict__ g = (const T*)p.g;
  const long rsK = (long)H * K, rsV = (long)H * V;
  for (int kk = threadIdx.x; kk < K; kk += 256) {
    float gt[C];
    col_cumsum<T, C>(g, t0, rsK, (long)hh * K + kk, len, p.g_is_cumsum != 0, gt);
#pragma unroll
    for (int j = 0; j < C; ++j) {
      sG[j * K + kk] = gt[j];
      sQe[j * K + kk] = j < len ? ldf(q, (t0 + j) * rsK + (long)hh * K + kk) * expf(gt[j])
                                : 0.f;
    }
  }
  __syncthreads();
  const int tid = threadIdx.x;
  if (tid < C * C) {
    const int i = tid / C, j = tid % C;
    float a = 0.f;
    if (p.A_in) {
      a = p.A_in[(((long)c * C + i) * H + hh) * C + j];
    } else if (i < len && j < len) {
      for (int kk = 0; kk < K; ++kk)
        a += ldf(q, (t0 + i) * rsK + (long)hh * K + kk) *
             ldf(k, (t0 + j) * rsK + (long)hh * K + kk) *
             expf(sG[i * K + kk] - sG[j * K + kk]);
      a *= p.scale;
    }
    if (p.A_out) p.A_out[(((long)c * C + i) * H + hh) * C + j] = a;
    sA[tid] = a;
  }
  if (!p.o) return;   // uniform
  __syncthreads();
  const T* __restrict__ hs = (const T*)p.h;
  T* __restrict__ o = (T*)p.o;
  const long KV = (long)K * V;
  for (int idx = tid; idx < len * V; idx += 256) {
    const int i = idx / V, vv = idx % V;
    float x = 0.f;
    if (hs) {
      const T* hc = hs + ((long)c * H + hh) * KV + vv;
      for (int kk = 0; kk < K; ++kk) x += sQe[i * K + kk] * ldf(hc, (long)kk * V);
      x *= p.scale;
    }
    for (int j = 0; j <= i; ++j) x += sA[i * C + j] * ldf(v, (t0 + j) * rsV + (long)hh * V + vv);
    o[(t0 + i) * rsV + (long)hh * V + vv] = from_f32<T>(x);
  }
}

template <typename T, int C>
static hipError_t launch_small_state(const ScanArgs& p, bool reverse, hipStream_t st) {
  const long per = ((long)p.K * p.V + 255) / 256;
  const long blocks = (long)p.si.N * p.H * per;
  if (blocks == 0) return hipSuccess;
  if (reverse)
    hipLaunchKernelGGL((small_state_kernel<T, C, true>), dim3((unsigned)blocks), dim3(256), 0,
                       st, p);
  else
    hipLaunchKernelGGL((small_state_kernel<T, C, false>), dim3((unsigned)blocks), dim3(256), 0,
                       st, p);
  return hipGetLastError();
}

template <typename T, int C>
static hipError_t launch_small_out(const FwdOArgs& p, hipStream_t st) {
  const long blocks = (long)p.si.NC * p.H;
  if (blocks == 0) return hipSuccess;
  const size_t lds = (size_t)2 * C * p.K * sizeof(float);
  hipError_t e = hipFuncSetAttribute((const void*)small_out_kernel<T, C>,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((small_out_kernel<T, C>), dim3((unsigned)blocks), dim3(256), lds, st, p);
  return hipGetLastError();
}

int small_chunk_max_k() { return 2048; }   // 2 C K floats of LDS at C = 8: 128 KiB

hipError_t run_small_state_scan(const ScanArgs& p, bool reverse, int dtype, hipStream_t st) {
  const int C = p.si.C;
  if (dtype == DT_BF16)
    return C == 4 ? launch_small_state<bf16, 4>(p, reverse, st)
                  : launch_small_state<bf16, 8>(p, reverse, st);
  return C == 4 ? launch_small_state<float, 4>(p, reverse, st)
                : launch_small_state<float, 8>(p, reverse, st);
}

hipError_t run_small_chunk_fwd_o(const FwdOArgs& p, int dtype, hipStream_t st) {
  const int C = p.si.C;
  if (dtype == DT_BF16)
    return C == 4 ? launch_small_out<bf16, 4>(p, st) : launch_small_out<bf16, 8>(p, st);
  return C == 4 ? launch_small_out<float, 4>(p, st) : launch_small_out<float, 8>(p, st);
}

}  // namespace tops
