// The GLA layer's element-wise stages around the attention core:
//   * RMSNorm with an optional SiLU output gate, per row of D features:
//       y = x rsqrt(mean(x^2) + eps) [* w] [* silu(g)]
//     Reference: FusedRMSNormGated.__call__, tops/modules/fused_norm_gate.py:28-37, and
//     RMSNorm.__call__, tops/modules/layernorm.py:28-35 (no gate).
//   * the gate activation of the key-wise decay, y = max(log_sigmoid(x) / n, clamp_min),
//     tops/layers/gla.py:286-288.
// One wave per row (D up to 8192 features, 8 per lane and pass, 16-byte accesses), fp32
// arithmetic, output in the input dtype. In the backward, rows of up to 1024 features (the
// layer's per-head norm: D = V) are read once into registers -- the row reduction and the
// outputs use the same values -- and the next row's loads are issued before the current row
// is finished (224 -> 173 us at the C5 layer's 131072 x 512). The backward of the norm reduces dw over rows in
// two steps: each block sums its rows into its own partial row of a caller workspace, a
// second kernel sums the partials (deterministic, no atomics).
#include "common.hpp"
#include "kernels.hpp"

namespace tops {

namespace {

constexpr int NG_NT = 256;            // 4 waves, one row each at a time
constexpr int NG_ROWS = 16;           // forward: rows per block (4 per wave)
constexpr int NG_BWD_BLOCKS = 2048;   // backward grid (blocks stride over the rows)
constexpr int NG_REG = 2;             // register-resident rows: up to NG_REG x 512 features

template <typename T>
struct Vec8;
template <>
struct Vec8<bf16> {
  static __device__ __forceinline__ void load(const bf16* p, float (&x)[8]) {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = __uint_as_float(w[i] << 16);
      x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  static __device__ __forceinline__ void store(bf16* p, const float (&x)[8]) {
    *reinterpret_cast<uint4*>(p) = make_uint4(pack2_bf16(x[0], x[1]), pack2_bf16(x[2], x[3]),
                                              pack2_bf16(x[4], x[5]), pack2_bf16(x[6], x[7]));
  }
};
template <>
struct Vec8<float> {
  static __device__ __forceinline__ void load(const float* p, float (&x)[8]) {
    const float4 a = reinterpret_cast<const float4*>(p)[0];
    const float4 b = reinterpret_cast<const float4*>(p)[1];
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
  }
  static __device__ __forceinline__ void store(float* p, const float (&x)[8]) {
    reinterpret_cast<float4*>(p)[0] = make_float4(x[0], x[1], x[2], x[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(x[4], x[5], x[6], x[7]);
  }
};

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

// 1 / (1 + e^{-x}) with the hardware reciprocal (v_rcp_f32, 1 ulp): an IEEE division is a
// ten-instruction scale / fix-up sequence, a large share of these VALU-bound kernels' work.
// Saturates to 0 / 1 (e^{-x} overflowing to inf gives rcp(inf) = 0).
__device__ __forceinline__ float sigmoidf(float x) {
  return __builtin_amdgcn_rcpf(1.f + __expf(-x));
}

}  // namespace

// y = x * rstd * w * silu(g); rstd per row is kept for the backward (may be NULL).
template <typename T>
__global__ __launch_bounds__(NG_NT) void norm_gate_fwd_kernel(NormGateArgs p) {
  const T* __restrict__ x = (const T*)p.x;
  const T* __restrict__ g = (const T*)p.g;
  T* __restrict__ y = (T*)p.y;
  const int D = p.D, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const long r0 = (long)blockIdx.x * NG_ROWS;
  for (int rr = w; rr < NG_ROWS; rr += NG_NT / 64) {
    const long row = r0 + rr;
    if (row >= p.rows) break;
    const T* xr = x + row * D;
    float ss = 0.f;
    for (int c = lane * 8; c < D; c += 512) {
      float v[8];
      Vec8<T>::load(xr + c, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += v[e] * v[e];
    }
    const float rstd = rsqrtf(wave_sum(ss) / (float)D + p.eps);
    if (p.rstd && lane == 0) p.rstd[row] = rstd;
    for (int c = lane * 8; c < D; c += 512) {
      float v[8];
      Vec8<T>::load(xr + c, v);
      float wv[8];
      if (p.w) {
        Vec8<float>::load(p.w + c, wv);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) wv[e] = 1.f;
      }
      float gv[8];
      if (g) Vec8<T>::load(g + row * D + c, gv);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[e] = v[e] * rstd * wv[e];
        if (g) v[e] *= gv[e] * sigmoidf(gv[e]);
      }
      Vec8<T>::store(y + row * D + c, v);
    }
  }
}

// Rows held in registers (D <= R x 512: one wave a row, lane l holding features 8 l + 512 j,
// j < R), the next row's loads in flight; the lane's dw partials stay in registers and meet
// in LDS once. R = 1 for rows of up to 512 features (half the registers of R = 2).
template <typename T, int R>
__device__ __forceinline__ void norm_gate_bwd_rows(const NormGateArgs& p, float (*sDw)[1024]) {
  const T* __restrict__ x = (const T*)p.x;
  const T* __restrict__ g = (const T*)p.g;
  const T* __restrict__ dy = (const T*)p.dy;
  T* __restrict__ dx = (T*)p.dx;
  T* __restrict__ dg = (T*)p.dg;
  const int D = p.D, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const bool want_dw = p.w && p.dw_part;
  float wv[R][8], dwa[R][8];
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const int c = lane * 8 + 512 * j;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      wv[j][e] = 1.f;
      dwa[j][e] = 0.f;
    }
    if (p.w && c < D) Vec8<float>::load(p.w + c, wv[j]);
  }
  const long stride = (long)gridDim.x * (NG_NT / 64);
  float v[R][8], d[R][8], gv[R][8], rstd = 0.f;
  auto load_row = [&](long row, float (&xa)[R][8], float (&da)[R][8], float (&ga)[R][8],
                      float& rs) {
    rs = p.rstd[row];
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const int c = lane * 8 + 512 * j;
      if (c < D) {
        Vec8<T>::load(x + row * D + c, xa[j]);
        Vec8<T>::load(dy + row * D + c, da[j]);
        if (g) Vec8<T>::load(g + row * D + c, ga[j]);
      }
    }
  };
  long row = (long)blockIdx.x * (NG_NT / 64) + w;
  if (row < p.rows) load_row(row, v, d, gv, rstd);
  for (; row < p.rows; row += stride) {
    float nv[R][8], nd[R][8], ng[R][8], nrs = 0.f;
    if (row + stride < p.rows) load_row(row + stride, nv, nd, ng, nrs);
    float dot = 0.f, sgv[R][8];   // sigmoid(g), formed once per element
#pragma unroll
    for (int j = 0; j < R; ++j) {
      if (lane * 8 + 512 * j < D) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float dn = d[j][e] * wv[j][e];
          sgv[j][e] = g ? sigmoidf(gv[j][e]) : 1.f;
          if (g) dn *= gv[j][e] * sgv[j][e];
          dot += dn * v[j][e] * rstd;
        }
      }
    }
    const float mdot = wave_sum(dot) / (float)D;
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const int c = lane * 8 + 512 * j;
      if (c < D) {
        float ox[8], og[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float n = v[j][e] * rstd;
          float s = 1.f;
          if (g) {
            const float sg = sgv[j][e];
            s = gv[j][e] * sg;
            og[e] = d[j][e] * n * wv[j][e] * sg * (1.f + gv[j][e] * (1.f - sg));
          }
          ox[e] = rstd * (d[j][e] * s * wv[j][e] - n * mdot);
          dwa[j][e] += d[j][e] * s * n;
        }
        Vec8<T>::store(dx + row * D + c, ox);
        if (g) Vec8<T>::store(dg + row * D + c, og);
      }
    }
#pragma unroll
    for (int j = 0; j < R; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[j][e] = nv[j][e];
        d[j][e] = nd[j][e];
        gv[j][e] = ng[j][e];
      }
    rstd = nrs;
  }
  if (want_dw) {
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const int c = lane * 8 + 512 * j;
      if (c < D)
#pragma unroll
        for (int e = 0; e < 8; ++e) sDw[w][c + e] = dwa[j][e];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < D; i += NG_NT) {
      float t = 0.f;
#pragma unroll
      for (int ww = 0; ww < NG_NT / 64; ++ww) t += sDw[ww][i];
      p.dw_part[(long)blockIdx.x * D + i] = t;
    }
  }
}

// n = x rstd, a = n w, s = silu(g), y = a s:
//   dg = dy a silu'(g), silu'(g) = sig(g) (1 + g (1 - sig(g)))
//   dn = dy s w, dx = rstd (dn - n mean(dn n)), dw_part[block] = sum_rows dy s n
// R > 0: rows of at most R x 512 features in registers; R = 0: 1024-feature slabs.
template <typename T, int R>
__global__ __launch_bounds__(NG_NT) void norm_gate_bwd_kernel(NormGateArgs p) {
  __shared__ float sDw[NG_NT / 64][1024];   // per-wave dw partials of a 1024-feature slab
  const T* __restrict__ x = (const T*)p.x;
  const T* __restrict__ g = (const T*)p.g;
  const T* __restrict__ dy = (const T*)p.dy;
  T* __restrict__ dx = (T*)p.dx;
  T* __restrict__ dg = (T*)p.dg;
  const int D = p.D, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const bool want_dw = p.w && p.dw_part;
  static_assert(NG_REG * 512 <= 1024 && R <= NG_REG, "one dw slab");
  if constexpr (R > 0) {
    norm_gate_bwd_rows<T, R>(p, sDw);
    return;
  }
  for (int c0 = 0; c0 < D; c0 += 1024) {   // dw slabs: the row loop runs once per slab
    const int cend = want_dw ? min(D, c0 + 1024) : D;   // without dw: one pass, whole rows
    if (want_dw) {
      for (int i = threadIdx.x; i < (NG_NT / 64) * 1024; i += NG_NT) (&sDw[0][0])[i] = 0.f;
      __syncthreads();
    }
    for (long row = (long)blockIdx.x * (NG_NT / 64) + w; row < p.rows;
         row += (long)gridDim.x * (NG_NT / 64)) {   // a wave per row, rows interleaved
      const float rstd = p.rstd[row];
      const T* xr = x + row * D;
      // mean(dn n) over the whole row (every slab needs it)
      float dot = 0.f;
      for (int c = lane * 8; c < D; c += 512) {
        float v[8], d[8], wv[8], gv[8];
        Vec8<T>::load(xr + c, v);
        Vec8<T>::load(dy + row * D + c, d);
        if (p.w) Vec8<float>::load(p.w + c, wv);
        if (g) Vec8<T>::load(g + row * D + c, gv);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float dn = d[e] * (p.w ? wv[e] : 1.f);
          if (g) dn *= gv[e] * sigmoidf(gv[e]);
          dot += dn * v[e] * rstd;
        }
      }
      const float mdot = wave_sum(dot) / (float)D;
      for (int c = c0 + lane * 8; c < cend; c += 512) {
        float v[8], d[8], wv[8], gv[8], ox[8], og[8];
        Vec8<T>::load(xr + c, v);
        Vec8<T>::load(dy + row * D + c, d);
        if (p.w) Vec8<float>::load(p.w + c, wv);
        if (g) Vec8<T>::load(g + row * D + c, gv);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float n = v[e] * rstd, ww = p.w ? wv[e] : 1.f;
          float s = 1.f;
          if (g) {
            const float sg = sigmoidf(gv[e]);
            s = gv[e] * sg;
            og[e] = d[e] * n * ww * sg * (1.f + gv[e] * (1.f - sg));
          }
          const float dn = d[e] * s * ww;
          ox[e] = rstd * (dn - n * mdot);
          if (want_dw) sDw[w][c - c0 + e] += d[e] * s * n;
        }
        Vec8<T>::store(dx + row * D + c, ox);
        if (g) Vec8<T>::store(dg + row * D + c, og);
      }
    }
    if (want_dw) {
      __syncthreads();
      for (int i = threadIdx.x; i < min(1024, D - c0); i += NG_NT) {
        float t = 0.f;
#pragma unroll
        for (int ww = 0; ww < NG_NT / 64; ++ww) t += sDw[ww][i];
        p.dw_part[(long)blockIdx.x * D + c0 + i] = t;
      }
      __syncthreads();
    }
    if (!want_dw) break;   // without dw the first pass already wrote every slab
  }
}

// dw[c] = sum over the partial rows: block = 64 columns, its 4 waves split the rows.
// (rows b of part are `stride` floats apart; columns c < D are summed)
__global__ __launch_bounds__(256) void dw_reduce_kernel(const float* __restrict__ part, int nblk,
                                                        int D, long stride,
                                                        float* __restrict__ dw) {
  __shared__ float s[4][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + lane;
  float t = 0.f;
  if (c < D)
    for (int b = w; b < nblk; b += 4) t += part[(long)b * stride + c];
  s[w][lane] = t;
  __syncthreads();
  if (w == 0 && c < D) dw[c] = (s[0][lane] + s[1][lane]) + (s[2][lane] + s[3][lane]);
}

// y = max(log_sigmoid(x) / n, clamp) ; dx = dy sig(-x) / n where y is not clamped.
template <typename T>
__global__ __launch_bounds__(256) void gate_fwd_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                       long count, float inv_n, int has_clamp,
                                                       float clamp) {
  const long i0 = ((long)blockIdx.x * 256 + threadIdx.x) * 8;
  if (i0 >= count) return;
  float v[8];
  if (i0 + 8 <= count) {
    Vec8<T>::load(x + i0, v);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = i0 + e < count ? to_f32(x[i0 + e]) : 0.f;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    // log_sigmoid(x) = min(x, 0) - log(1 + exp(-|x|)) (hardware exp / log: the second term
    // is below 1 ulp of the first wherever 1 + exp(-|x|) rounds to 1)
    float r = (fminf(v[e], 0.f) - __logf(1.f + __expf(-fabsf(v[e])))) * inv_n;
    if (has_clamp) r = fmaxf(r, clamp);
    v[e] = r;
  }
  if (i0 + 8 <= count) {
    Vec8<T>::store(y + i0, v);
  } else {
    for (int e = 0; e < 8 && i0 + e < count; ++e) y[i0 + e] = from_f32<T>(v[e]);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void gate_bwd_kernel(const T* __restrict__ x,
                                                       const T* __restrict__ dy,
                                                       T* __restrict__ dx, long count,
                                                       float inv_n, int has_clamp, float clamp) {
  const long i0 = ((long)blockIdx.x * 256 + threadIdx.x) * 8;
  if (i0 >= count) return;
  float v[8], d[8];
  if (i0 + 8 <= count) {
    Vec8<T>::load(x + i0, v);
    Vec8<T>::load(dy + i0, d);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[e] = i0 + e < count ? to_f32(x[i0 + e]) : 0.f;
      d[e] = i0 + e < count ? to_f32(dy[i0 + e]) : 0.f;
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float gr = sigmoidf(-v[e]) * inv_n;
    if (has_clamp) {
      const float r = (fminf(v[e], 0.f) - __logf(1.f + __expf(-fabsf(v[e])))) * inv_n;
      if (r < clamp) gr = 0.f;   // clamped: no gradient (jnp.clip passes none below a_min)
    }
    v[e] = d[e] * gr;
  }
  if (i0 + 8 <= count) {
    Vec8<T>::store(dx + i0, v);
  } else {
    for (int e = 0; e < 8 && i0 + e < count; ++e) dx[i0 + e] = from_f32<T>(v[e]);
  }
}

static long norm_gate_blocks(long rows) { return (rows + NG_ROWS - 1) / NG_ROWS; }
long norm_gate_bwd_blocks(long rows) {
  const long b = norm_gate_blocks(rows);
  return b < NG_BWD_BLOCKS ? b : NG_BWD_BLOCKS;
}

hipError_t run_norm_gate_fwd(const NormGateArgs& p, int dtype, hipStream_t st) {
  const long blocks = norm_gate_blocks(p.rows);
  if (blocks == 0) return hipSuccess;
  if (dtype == DT_BF16)
    hipLaunchKernelGGL((norm_gate_fwd_kernel<bf16>), dim3((unsigned)blocks), dim3(NG_NT), 0, st,
                       p);
  else
    hipLaunchKernelGGL((norm_gate_fwd_kernel<float>), dim3((unsigned)blocks), dim3(NG_NT), 0,
                       st, p);
  return hipGetLastError();
}

hipError_t run_norm_gate_bwd(const NormGateArgs& p, float* dw, int dtype, hipStream_t st) {
  const long blocks = norm_gate_bwd_blocks(p.rows);
  if (blocks == 0) return hipSuccess;
  const int r = p.D <= 512 ? 1 : p.D <= NG_REG * 512 ? NG_REG : 0;
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(NG_NT), 0, st, p);
  };
  if (dtype == DT_BF16)
    r == 1 ? go(norm_gate_bwd_kernel<bf16, 1>)
           : r == NG_REG ? go(norm_gate_bwd_kernel<bf16, NG_REG>) : go(norm_gate_bwd_kernel<bf16, 0>);
  else
    r == 1 ? go(norm_gate_bwd_kernel<float, 1>)
           : r == NG_REG ? go(norm_gate_bwd_kernel<float, NG_REG>) : go(norm_gate_bwd_kernel<float, 0>);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !dw || !p.w || !p.dw_part) return e;
  return run_rows_sum(p.dw_part, (int)blocks, p.D, dw, st);
}

// Many partial rows: each of G groups of rows is summed by its own blocks into a second-level
// row (written over the group's first row), then the G rows are summed.
__global__ __launch_bounds__(256) void rows_sum_stage_kernel(float* __restrict__ part, int nblk,
                                                             int M, int per) {
  __shared__ float s[4][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + lane, grp = blockIdx.y;
  const int b0 = grp * per, b1 = min(nblk, b0 + per);
  float t = 0.f;
  if (c < M)
    for (int b = b0 + w; b < b1; b += 4) t += part[(long)b * M + c];
  s[w][lane] = t;
  __syncthreads();
  if (w == 0 && c < M) part[(long)b0 * M + c] = (s[0][lane] + s[1][lane]) + (s[2][lane] + s[3][lane]);
}

hipError_t run_rows_sum(const float* part, int nblk, int M, float* out, hipStream_t st) {
  if (M <= 0) return hipSuccess;
  const unsigned cb = (unsigned)((M + 63) / 64);
  if (nblk > 64) {
    const int per = 64, groups = (nblk + per - 1) / per;
    float* p = const_cast<float*>(part);
    hipLaunchKernelGGL(rows_sum_stage_kernel, dim3(cb, (unsigned)groups), dim3(256), 0, st, p,
                       nblk, M, per);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // the group sums sit in rows 0, per, 2 per, ...: a row stride of per * M
    hipLaunchKernelGGL(dw_reduce_kernel, dim3(cb), dim3(256), 0, st, part, groups, M,
                       (long)per * M, out);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(dw_reduce_kernel, dim3(cb), dim3(256), 0, st, part, nblk, M, (long)M, out);
  return hipGetLastError();
}

// Row-wise concatenation of up to kConcatMax [rows, w_i] sources into dst [rows, sum w_i]
// (widths multiples of 8 elements, 16-byte aligned buffers): one 16-byte piece a thread, the
// pieces of a destination row in order, so both the source reads and the destination writes
// are contiguous runs (torch.cat into a row slice of a wider tensor ran at ~2.8 TB/s here).
struct ConcatArgs {
  const void* src[kConcatMax];
  long w8[kConcatMax + 1];   // prefix sums of the widths in 16-byte pieces
  int nsrc;
  long rows;
};
__global__ __launch_bounds__(256) void concat_cols_kernel(ConcatArgs a, uint4* __restrict__ dst) {
  const long pw = a.w8[a.nsrc];   // pieces of a destination row
  const long total = a.rows * pw;
  for (long p = (long)blockIdx.x * 256 + threadIdx.x; p < total; p += (long)gridDim.x * 256) {
    const long row = p / pw, c = p - row * pw;
    int j = 0;
#pragma unroll
    for (int t = 1; t < kConcatMax; ++t) j += (t < a.nsrc && c >= a.w8[t]) ? 1 : 0;
    const long w = a.w8[j + 1] - a.w8[j];
    dst[p] = reinterpret_cast<const uint4*>(a.src[j])[row * w + (c - a.w8[j])];
  }
}

hipError_t run_concat_cols(const void* const* src, const long* widths, int nsrc, long rows,
                           void* dst, int esize, hipStream_t st) {
  ConcatArgs a = {};
  a.nsrc = nsrc;
  a.rows = rows;
  a.w8[0] = 0;
  for (int j = 0; j < nsrc; ++j) {
    a.src[j] = src[j];
    a.w8[j + 1] = a.w8[j] + widths[j] * esize / 16;
  }
  const long total = rows * a.w8[nsrc];
  if (total == 0) return hipSuccess;
  const long blocks = std::min<long>((total + 255) / 256, 256L * 32);
  hipLaunchKernelGGL(concat_cols_kernel, dim3((unsigned)blocks), dim3(256), 0, st, a,
                     (uint4*)dst);
  return hipGetLastError();
}

hipError_t run_gate(const void* x, const void* dy, void* out, long count, float inv_n,
                    int has_clamp, float clamp, int dtype, hipStream_t st) {
  const long blocks = (count + 2047) / 2048;
  if (blocks == 0) return hipSuccess;
  if (dy == nullptr) {
    if (dtype == DT_BF16)
      hipLaunchKernelGGL((gate_fwd_kernel<bf16>), dim3((unsigned)blocks), dim3(256), 0, st,
                         (const bf16*)x, (bf16*)out, count, inv_n, has_clamp, clamp);
    else
      hipLaunchKernelGGL((gate_fwd_kernel<float>), dim3((unsigned)blocks), dim3(256), 0, st,
                         (const float*)x, (float*)out, count, inv_n, has_clamp, clamp);
  } else {
    if (dtype == DT_BF16)
      hipLaunchKernelGGL((gate_bwd_kernel<bf16>), dim3((unsigned)blocks), dim3(256), 0, st,
                         (const bf16*)x, (const bf16*)dy, (bf16*)out, count, inv_n, has_clamp,
                         clamp);
    else
      hipLaunchKernelGGL((gate_bwd_kernel<float>), dim3((unsigned)blocks), dim3(256), 0, st,
                         (const float*)x, (const float*)dy, (float*)out, count, inv_n,
                         has_clamp, clamp);
  }
  return hipGetLastError();
}

}  // namespace tops
