// Gate-range check of the chunked paths that do not track it inside their own kernels (the
// per-chunk float32 kernels, and the bf16 wide-head and V > 128 backward).
//
// The chunk kernels factor e^{g~_i - g~_j} around a per-column reference
// r = (g~_first + g~_last) / 2 (g~ the chunk-local inclusive cumsum of the raw log-gates,
// tops/ops/gla/chunk.py:20-52 and the factoring of chunk.py:370-371), so each factor stays
// within e^{+-max|g~ - r|}. A (chunk, head) whose largest |g~ - r| over its columns passes
// kGateLimit2 (base 2, the full-head kernels' limit) is flagged; the recurrent scans then
// recompute every flagged (sequence, head) pair exactly, for any decay.
//
// One 256-thread block per (chunk, head); a thread walks one column's rows (whole columns
// of 256 threads for wider heads), keeping the running sum, its extremes and the first row;
// max|g~ - r| = max(max g~ - r, r - min g~). Flags: int32 [NC, H], every entry written (no
// clearing). HBM-bound: reads the gates once (tokens x H x K elements).
#include "common.hpp"
#include "kernels.hpp"

namespace tops {

template <typename T>
__global__ __launch_bounds__(256) void gate_range_kernel(GateCheckArgs p) {
  const long L = blockIdx.x;
  const int H = p.H, K = p.K;
  const int c = (int)(L / H), hh = (int)(L % H);
  int seq, t0, len;
  chunk_range(p.si, c, seq, t0, len);
  (void)seq;
  const long rs = (long)H * K;
  const T* __restrict__ g = (const T*)p.g + (long)t0 * rs + (long)hh * K;
  int bad = 0;
  for (int col = (int)threadIdx.x; col < K; col += 256) {
    float s = 0.f, first = 0.f, mx = -3.0e38f, mn = 3.0e38f;
    int i = 0;
    for (; i + 8 <= len; i += 8) {   // 8 loads in flight per thread
      float x[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) x[u] = to_f32(g[(long)(i + u) * rs + col]);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        s += x[u];
        if (i + u == 0) first = s;
        mx = fmaxf(mx, s);
        mn = fminf(mn, s);
      }
    }
    for (; i < len; ++i) {
      s += to_f32(g[(long)i * rs + col]);
      if (i == 0) first = s;
      mx = fmaxf(mx, s);
      mn = fminf(mn, s);
    }
    const float r = 0.5f * (first + s);
    const float d = fmaxf(mx - r, r - mn) * 1.4426950408889634f;   // base 2
    bad |= d > kGateLimit2 ? 1 : 0;
  }
  bad = __syncthreads_or(bad);
  if (threadIdx.x == 0) p.flags[L] = bad ? 1 : 0;
}

hipError_t run_gate_range(const GateCheckArgs& p, int dtype, hipStream_t st) {
  const long blocks = (long)p.si.NC * p.H;
  if (blocks == 0) return hipSuccess;
  if (blocks > 2147483647L) return hipErrorInvalidValue;
  if (dtype == DT_BF16)
    hipLaunchKernelGGL((gate_range_kernel<bf16>), dim3((unsigned)blocks), dim3(256), 0, st, p);
  else if (dtype == DT_F32)
    hipLaunchKernelGGL((gate_range_kernel<float>), dim3((unsigned)blocks), dim3(256), 0, st, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace tops
