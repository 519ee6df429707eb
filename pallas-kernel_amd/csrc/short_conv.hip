// Causal depthwise 1D convolution with optional bias and SiLU, per sequence:
//   z[t, d] = sum_{j < W} w[d, j] x[t - W + 1 + j, d] (+ b[d]),  y = silu(z) or z,
// where rows before the sequence's first token read as zero.
// Reference: ShortConvolution._causal_conv1d, tops/modules/convolution.py:46-78 (the
// prefill / training path; the single-token decode step :76-118 is host glue).
// Block = (sequence, 32-token tile, 64-channel slab), 256 threads: a thread owns one token
// and 8 consecutive channels (16-byte rows of bf16, two of fp32). The backward recomputes
// z over the W tokens a dx row reads (W <= 8), and reduces dw / db over the block's 32
// tokens into a per-block partial row of a caller workspace; a second pass sums the
// partials (deterministic).
#include "common.hpp"
#include "kernels.hpp"

namespace tops {

namespace {

constexpr int SC_NT = 256;
constexpr int SC_TOK = 32;   // tokens per block
constexpr int SC_CH = 64;    // channels per block

template <typename T>
__device__ __forceinline__ void ld8(const T* p, float (&x)[8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = to_f32(p[e]);
}
template <>
__device__ __forceinline__ void ld8<bf16>(const bf16* p, float (&x)[8]) {
  const uint4 u = *reinterpret_cast<const uint4*>(p);
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = __uint_as_float(w[i] << 16);
    x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}
template <typename T>
__device__ __forceinline__ void st8(T* p, const float (&x)[8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) p[e] = from_f32<T>(x[e]);
}
template <>
__device__ __forceinline__ void st8<bf16>(bf16* p, const float (&x)[8]) {
  *reinterpret_cast<uint4*>(p) = make_uint4(pack2_bf16(x[0], x[1]), pack2_bf16(x[2], x[3]),
                                            pack2_bf16(x[4], x[5]), pack2_bf16(x[6], x[7]));
}

// 1 / (1 + e^{-x}) with the hardware reciprocal (v_rcp_f32, 1 ulp) instead of an IEEE
// division's scale / fix-up sequence; saturates to 0 / 1.
__device__ __forceinline__ float sig(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }

struct ScPos {
  int bos, eos, t, c0;
  bool valid;
};

// token and channel group of this thread
__device__ __forceinline__ ScPos sc_pos(const ShortConvArgs& p) {
  const int NSL = (p.D + SC_CH - 1) / SC_CH;
  const int slab = blockIdx.x % NSL, rest = blockIdx.x / NSL;
  int seq, tile;
  if (p.si.cu) {
    seq = blockIdx.y;
    tile = rest;
  } else {
    const int tiles = (p.si.T + SC_TOK - 1) / SC_TOK;
    seq = rest / tiles;
    tile = rest % tiles;
  }
  ScPos r;
  seq_bounds(p.si, seq, r.bos, r.eos);
  r.t = r.bos + tile * SC_TOK + threadIdx.x / 8;
  r.c0 = slab * SC_CH + (threadIdx.x % 8) * 8;
  r.valid = r.t < r.eos && r.c0 < p.D;
  return r;
}

template <typename T>
__device__ __forceinline__ void conv_at(const ShortConvArgs& p, const T* x, int t, int bos, int c0,
                                        float (&z)[8]) {
  const int W = p.W;
#pragma unroll
  for (int e = 0; e < 8; ++e) z[e] = p.bias ? p.bias[c0 + e] : 0.f;
  for (int j = 0; j < W; ++j) {
    const int ts = t - W + 1 + j;
    if (ts < bos) continue;
    float xv[8];
    ld8<T>(x + (long)ts * p.D + c0, xv);
#pragma unroll
    for (int e = 0; e < 8; ++e) z[e] = fmaf(p.w[(c0 + e) * W + j], xv[e], z[e]);
  }
}

}  // namespace

template <typename T>
__global__ __launch_bounds__(SC_NT) void short_conv_fwd_kernel(ShortConvArgs p) {
  const ScPos ps = sc_pos(p);
  if (!ps.valid) return;
  const T* x = (const T*)p.x;
  float z[8];
  conv_at<T>(p, x, ps.t, ps.bos, ps.c0, z);
  if (p.silu)
#pragma unroll
    for (int e = 0; e < 8; ++e) z[e] *= sig(z[e]);
  st8<T>((T*)p.y + (long)ps.t * p.D + ps.c0, z);
}

// dz = dy * act'(z); dx[t] = sum_j w[j] dz[t + W - 1 - j]; dw[d, j] += dz[t] x[t - W + 1 + j];
// db[d] += dz[t]. Partial dw / db of the block: part[block][(W + 1) * D] ([d][j], then b).
template <typename T>
__global__ __launch_bounds__(SC_NT) void short_conv_bwd_kernel(ShortConvArgs p) {
  __shared__ float sRed[SC_TOK][SC_CH * 9];   // per-token contributions (W <= 8, + bias)
  const ScPos ps = sc_pos(p);
  const T* x = (const T*)p.x;
  const T* dy = (const T*)p.dy;
  const int W = p.W, D = p.D;
  auto dz_at = [&](int t, float (&d)[8]) {
    float z[8], g[8];
    conv_at<T>(p, x, t, ps.bos, ps.c0, z);
    ld8<T>(dy + (long)t * D + ps.c0, g);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (p.silu) {
        const float s = sig(z[e]);
        g[e] *= s * (1.f + z[e] * (1.f - s));
      }
      d[e] = g[e];
    }
  };
  const int row = threadIdx.x / 8, cl = (threadIdx.x % 8) * 8;
  float own[8] = {};
  if (ps.valid) {
    float dx[8] = {};
    for (int j = 0; j < W; ++j) {
      const int tt = ps.t + W - 1 - j;
      if (tt >= ps.eos) continue;
      float d[8];
      dz_at(tt, d);
      if (tt == ps.t)
#pragma unroll
        for (int e = 0; e < 8; ++e) own[e] = d[e];
#pragma unroll
      for (int e = 0; e < 8; ++e) dx[e] = fmaf(p.w[(ps.c0 + e) * W + j], d[e], dx[e]);
    }
    st8<T>((T*)p.dx + (long)ps.t * D + ps.c0, dx);
  }
  if (!p.part) return;   // uniform: no weight gradient wanted
  // this token's dw / db terms, then the column sums over the block's tokens
  for (int j = 0; j <= W; ++j) {
    float xv[8] = {};
    const int ts = ps.t - W + 1 + j;
    if (j < W && ps.valid && ts >= ps.bos) ld8<T>(x + (long)ts * D + ps.c0, xv);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      sRed[row][(cl + e) * 9 + j] = ps.valid ? own[e] * (j < W ? xv[e] : 1.f) : 0.f;
  }
  __syncthreads();
  const int slab_c0 = ps.c0 - cl;
  for (int i = threadIdx.x; i < SC_CH * (W + 1); i += SC_NT) {
    const int c = i / (W + 1), j = i % (W + 1);
    float s = 0.f;
    for (int r = 0; r < SC_TOK; ++r) s += sRed[r][c * 9 + j];
    if (slab_c0 + c < D) {
      const long blk = (long)blockIdx.y * gridDim.x + blockIdx.x;   // unique per block
      const long tile = blk / ((D + SC_CH - 1) / SC_CH);
      float* out = p.part + tile * (long)(W + 1) * D;
      if (j < W)
        out[(long)(slab_c0 + c) * W + j] = s;
      else
        out[(long)W * D + slab_c0 + c] = s;
    }
  }
}

namespace {

dim3 sc_grid(const ShortConvArgs& p, long& tiles) {
  const int NSL = (p.D + SC_CH - 1) / SC_CH;
  if (p.si.cu) {
    // varlen: blockIdx.y = sequence, x = (tile, slab) over the longest sequence
    tiles = (long)((p.max_len + SC_TOK - 1) / SC_TOK);
    return dim3((unsigned)(tiles * NSL), (unsigned)p.si.N);
  }
  tiles = (long)p.si.N * ((p.si.T + SC_TOK - 1) / SC_TOK);
  return dim3((unsigned)(tiles * NSL), 1);
}

}  // namespace

// Partial rows of the backward: one per (sequence, token tile); varlen sequences each
// get the tiles of the longest one.
long short_conv_part_rows(long nseq, long len) { return nseq * ((len + SC_TOK - 1) / SC_TOK); }

hipError_t run_short_conv(const ShortConvArgs& p, bool backward, int dtype, hipStream_t st) {
  long tiles;
  const dim3 grid = sc_grid(p, tiles);
  if (grid.x == 0 || grid.y == 0) return hipSuccess;
  if (!backward) {
    if (dtype == DT_BF16)
      hipLaunchKernelGGL((short_conv_fwd_kernel<bf16>), grid, dim3(SC_NT), 0, st, p);
    else
      hipLaunchKernelGGL((short_conv_fwd_kernel<float>), grid, dim3(SC_NT), 0, st, p);
    return hipGetLastError();
  }
  if (dtype == DT_BF16)
    hipLaunchKernelGGL((short_conv_bwd_kernel<bf16>), grid, dim3(SC_NT), 0, st, p);
  else
    hipLaunchKernelGGL((short_conv_bwd_kernel<float>), grid, dim3(SC_NT), 0, st, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !p.part) return e;
  return run_rows_sum(p.part, (int)(tiles * grid.y), (p.W + 1) * p.D, p.dwb, st);
}

}  // namespace tops
