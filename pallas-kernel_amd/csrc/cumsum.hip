// Chunk-local cumulative sum of gates.
// Reference: chunk_cumsum_kernel / chunk_local_cumsum_vector, tops/ops/gla/chunk.py:55-198.
// Chunks start at each sequence's first token; the last chunk of a sequence may be partial.
// One thread per (chunk, head, column); rows walked in order (or reverse) in fp32.
#include "common.hpp"
#include "kernels.hpp"

namespace tops {

template <typename TI, typename TO>
__global__ __launch_bounds__(256) void cumsum_kernel(CumsumArgs p) {
  const int H = p.H, S = p.S;
  const int c = blockIdx.x / H, hh = blockIdx.x % H;
  const int s = blockIdx.y * 256 + threadIdx.x;
  if (s >= S) return;
  int seq, t0, len;
  chunk_range(p.si, c, seq, t0, len);
  (void)seq;
  const TI* __restrict__ g = (const TI*)p.g;
  TO* __restrict__ out = (TO*)p.out;
  auto addr = [&](int tau) -> long {
    if (p.head_first) {
      const long b = tau / p.T_total, t = tau % p.T_total;
      return ((b * H + hh) * p.T_total + t) * S + s;
    }
    return ((long)tau * H + hh) * S + s;
  };
  const float sc = p.has_scale ? p.scale : 1.f;
  float acc = 0.f;
  if (p.reverse) {
    for (int r = len - 1; r >= 0; --r) {
      const long a = addr(t0 + r);
      acc += to_f32(g[a]);
      out[a] = from_f32<TO>(acc * sc);
    }
  } else {
    for (int r = 0; r < len; ++r) {
      const long a = addr(t0 + r);
      acc += to_f32(g[a]);
      out[a] = from_f32<TO>(acc * sc);
    }
  }
}

template <typename TI, typename TO>
static hipError_t launch_cumsum(const CumsumArgs& p, hipStream_t st) {
  const long nb = (long)p.si.NC * p.H;
  if (nb == 0 || p.S == 0) return hipSuccess;
  hipLaunchKernelGGL((cumsum_kernel<TI, TO>), dim3((unsigned)nb, (p.S + 255) / 256), dim3(256),
                     0, st, p);
  return hipGetLastError();
}

hipError_t run_cumsum(const CumsumArgs& p, int in_dtype, int out_dtype, hipStream_t st) {
  if (in_dtype == DT_F32 && out_dtype == DT_F32) return launch_cumsum<float, float>(p, st);
  if (in_dtype == DT_BF16 && out_dtype == DT_F32) return launch_cumsum<bf16, float>(p, st);
  if (in_dtype == DT_BF16 && out_dtype == DT_BF16) return launch_cumsum<bf16, bf16>(p, st);
  if (in_dtype == DT_F32 && out_dtype == DT_BF16) return launch_cumsum<float, bf16>(p, st);
  return hipErrorInvalidValue;
}

}  // namespace tops
