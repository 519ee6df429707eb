// The backward's four per-chunk parts as separate kernels, over given intermediates
// (the reference exports them as jnp functions):
//   dA      = scale tril(do v^T)                                   chunk.py:504-539
//   dv      = tril(A)^T do + (k e^{gn - g~}) dh                      chunk.py:547-595
//   dq, dk  = e^{g~} (dA (k e^{-g~})),  e^{-g~} (dA^T (q e^{g~}))     chunk.py:603-648
//   dq, dk, dg (inter-chunk terms added to given dq / dk, gate gradient)  chunk.py:656-743
// The fused backward computes the same quantities in one pass without materialising A or
// dA; these kernels serve callers that hold the intermediates. Float32 in and out, chunk
// size C in {16, 32, 64}, tokens grouped as B * T / C chunks (T a multiple of C, as the
// reference's reshapes require). One block (256 threads) per (chunk, head[, 64-column
// slab]); contractions loop over 64-wide slabs staged in LDS (row pitch 65: conflict-free
// column reads), each thread owning C * 64 / 256 outputs (rows e / 64, column e % 64).
#include "common.hpp"
#include "kernels.hpp"

namespace tops {

namespace {

constexpr int PS = 64;       // slab width
constexpr int PP = PS + 1;   // LDS row pitch
constexpr int PNT = 256;

// rows [0, C) x columns [c0, c0 + 64) of a [tokens, H, D] fp32 tensor into s[C][PP]
// (zero outside D); optional per-element transform f(row, col, x).
template <int C, typename F>
__device__ __forceinline__ void stage(float* s, const float* src, long t0, int H, int hh, int D,
                                      int c0, F f) {
  for (int e = threadIdx.x; e < C * PS; e += PNT) {
    const int r = e / PS, c = e % PS;
    float x = 0.f;
    if (c0 + c < D) x = f(r, c0 + c, src[((t0 + r) * H + hh) * (long)D + c0 + c]);
    s[r * PP + c] = x;
  }
}

}  // namespace

// dA[i][j] = scale * sum_v do[i, v] v[j, v] for j <= i, else 0.
template <int C>
__global__ __launch_bounds__(PNT) void part_dA_kernel(PartArgs p) {
  __shared__ float sDo[C * PP], sV[C * PP];
  const int H = p.H, V = p.V;
  const int ch = blockIdx.x / H, hh = blockIdx.x % H;
  const long t0 = (long)ch * C;
  constexpr int EPT = (C * C + PNT - 1) / PNT;
  float acc[EPT] = {};
  for (int v0 = 0; v0 < V; v0 += PS) {
    __syncthreads();
    stage<C>(sDo, p.dout, t0, H, hh, V, v0, [](int, int, float x) { return x; });
    stage<C>(sV, p.v, t0, H, hh, V, v0, [](int, int, float x) { return x; });
    __syncthreads();
#pragma unroll
    for (int m = 0; m < EPT; ++m) {
      const int e = threadIdx.x + m * PNT;
      if (e < C * C) {
        const int i = e / C, j = e % C;
        float s = 0.f;
#pragma unroll 8
        for (int v = 0; v < PS; ++v) s += sDo[i * PP + v] * sV[j * PP + v];
        acc[m] += s;
      }
    }
  }
#pragma unroll
  for (int m = 0; m < EPT; ++m) {
    const int e = threadIdx.x + m * PNT;
    if (e < C * C) {
      const int i = e / C, j = e % C;
      p.out0[((t0 + i) * H + hh) * (long)C + j] = j <= i ? p.scale * acc[m] : 0.f;
    }
  }
}

// dv[j][v] = sum_{i >= j} A[i][j] do[i][v] + sum_k k[j][k] e^{gn[k] - g~[j][k]} dh[k][v],
// over one 64-wide slab of V.
template <int C>
__global__ __launch_bounds__(PNT) void part_dv_kernel(PartArgs p) {
  __shared__ float sA[C * (C + 1)], sDo[C * PP], sKd[C * PP], sDh[PS * PP], sGn[PS];
  const int H = p.H, K = p.K, V = p.V;
  const int NVS = (V + PS - 1) / PS;
  const int vs = blockIdx.x % NVS, hh = (blockIdx.x / NVS) % H, ch = blockIdx.x / (NVS * H);
  const long t0 = (long)ch * C;
  const int v0 = vs * PS;
  constexpr int EPT = C * PS / PNT;
  float acc[EPT] = {};
  for (int e = threadIdx.x; e < C * C; e += PNT) {
    const int i = e / C, j = e % C;
    sA[i * (C + 1) + j] = i >= j ? p.A[((t0 + i) * H + hh) * (long)C + j] : 0.f;
  }
  stage<C>(sDo, p.dout, t0, H, hh, V, v0, [](int, int, float x) { return x; });
  __syncthreads();
#pragma unroll
  for (int m = 0; m < EPT; ++m) {
    const int e = threadIdx.x + m * PNT, j = e / PS, vv = e % PS;
    float s = 0.f;
#pragma unroll 8
    for (int i = 0; i < C; ++i) s += sA[i * (C + 1) + j] * sDo[i * PP + vv];
    acc[m] = s;
  }
  const float* gc = p.g;
  for (int k0 = 0; k0 < K; k0 += PS) {
    __syncthreads();
    if (threadIdx.x < PS) {
      const int kk = k0 + threadIdx.x;
      sGn[threadIdx.x] = kk < K ? gc[((t0 + C - 1) * H + hh) * (long)K + kk] : 0.f;
    }
    __syncthreads();
    stage<C>(sKd, p.k, t0, H, hh, K, k0, [&](int r, int kk, float x) {
      return x * expf(sGn[kk - k0] - gc[((t0 + r) * H + hh) * (long)K + kk]);
    });
    for (int e = threadIdx.x; e < PS * PS; e += PNT) {
      const int kr = e / PS, vv = e % PS;
      float x = 0.f;
      if (k0 + kr < K && v0 + vv < V)
        x = p.dh[(((long)ch * H + hh) * K + k0 + kr) * V + v0 + vv];
      sDh[kr * PP + vv] = x;
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < EPT; ++m) {
      const int e = threadIdx.x + m * PNT, j = e / PS, vv = e % PS;
      float s = 0.f;
#pragma unroll 8
      for (int kr = 0; kr < PS; ++kr) s += sKd[j * PP + kr] * sDh[kr * PP + vv];
      acc[m] += s;
    }
  }
#pragma unroll
  for (int m = 0; m < EPT; ++m) {
    const int e = threadIdx.x + m * PNT, j = e / PS, vv = e % PS;
    if (v0 + vv < V) p.out0[((t0 + j) * H + hh) * (long)V + v0 + vv] = acc[m];
  }
}

// dq[i][k] = e^{g~[i][k]} sum_j dA[i][j] k[j][k] e^{-g~[j][k]},
// dk[j][k] = e^{-g~[j][k]} sum_i dA[i][j] q[i][k] e^{g~[i][k]}, over one 64-wide K slab.
// The exponentials are taken about the column's chunk midpoint r = (g~_0 + g~_{C-1}) / 2
// (same products, no overflow for strongly decaying gates).
template <int C>
__global__ __launch_bounds__(PNT) void part_dqk_intra_kernel(PartArgs p) {
  __shared__ float sDA[C * (C + 1)], sQ[C * PP], sKn[C * PP], sR[PS];
  const int H = p.H, K = p.K;
  const int NKS = (K + PS - 1) / PS;
  const int ks = blockIdx.x % NKS, hh = (blockIdx.x / NKS) % H, ch = blockIdx.x / (NKS * H);
  const long t0 = (long)ch * C;
  const int k0 = ks * PS;
  const float* gc = p.g;
  auto gat = [&](int r, int kk) { return gc[((t0 + r) * H + hh) * (long)K + kk]; };
  if (threadIdx.x < PS) {
    const int kk = min(k0 + (int)threadIdx.x, K - 1);
    sR[threadIdx.x] = 0.5f * (gat(0, kk) + gat(C - 1, kk));
  }
  for (int e = threadIdx.x; e < C * C; e += PNT) {
    const int i = e / C, j = e % C;
    sDA[i * (C + 1) + j] = p.dA[((t0 + i) * H + hh) * (long)C + j];
  }
  __syncthreads();
  stage<C>(sQ, p.q, t0, H, hh, K, k0,
           [&](int r, int kk, float x) { return x * expf(gat(r, kk) - sR[kk - k0]); });
  stage<C>(sKn, p.k, t0, H, hh, K, k0,
           [&](int r, int kk, float x) { return x * expf(sR[kk - k0] - gat(r, kk)); });
  __syncthreads();
  constexpr int EPT = C * PS / PNT;
#pragma unroll
  for (int m = 0; m < EPT; ++m) {
    const int e = threadIdx.x + m * PNT, r = e / PS, c = e % PS, kk = k0 + c;
    float sq = 0.f, sk = 0.f;
#pragma unroll 8
    for (int j = 0; j < C; ++j) {
      sq += sDA[r * (C + 1) + j] * sKn[j * PP + c];
      sk += sDA[j * (C + 1) + r] * sQ[j * PP + c];
    }
    if (kk < K) {
      const float g = gat(r, kk), rr = sR[c];
      const long o = ((t0 + r) * H + hh) * (long)K + kk;
      p.out0[o] = expf(g - rr) * sq;
      p.out1[o] = expf(rr - g) * sk;
    }
  }
}

// dq' = dq + scale e^{g~} (do h^T), dk' = dk + e^{gn - g~} (v dh^T),
// dg = revcumsum_chunk(q dq' - k dk') + e^{gn} sum_v h dh + sum_c dk_inter k,
// over one 64-wide K slab (h, dh rows of the slab, contracted over V slabs).
template <int C>
__global__ __launch_bounds__(PNT) void part_dqkg_kernel(PartArgs p) {
  __shared__ float sDo[C * PP], sV[C * PP], sH[PS * PP], sDh[PS * PP], sW[C * PP];
  const int H = p.H, K = p.K, V = p.V;
  const int NKS = (K + PS - 1) / PS;
  const int ks = blockIdx.x % NKS, hh = (blockIdx.x / NKS) % H, ch = blockIdx.x / (NKS * H);
  const long t0 = (long)ch * C;
  const int k0 = ks * PS;
  constexpr int EPT = C * PS / PNT;
  float aq[EPT] = {}, ak[EPT] = {};
  float hdh = 0.f;  // threads < 64: sum_v h dh of row k0 + tid
  const long sb = ((long)ch * H + hh) * K;
  for (int v0 = 0; v0 < V; v0 += PS) {
    __syncthreads();
    stage<C>(sDo, p.dout, t0, H, hh, V, v0, [](int, int, float x) { return x; });
    stage<C>(sV, p.v, t0, H, hh, V, v0, [](int, int, float x) { return x; });
    for (int e = threadIdx.x; e < PS * PS; e += PNT) {
      const int kr = e / PS, vv = e % PS;
      float x = 0.f, y = 0.f;
      if (k0 + kr < K && v0 + vv < V) {
        x = p.h[(sb + k0 + kr) * V + v0 + vv];
        y = p.dh[(sb + k0 + kr) * V + v0 + vv];
      }
      sH[kr * PP + vv] = x;
      sDh[kr * PP + vv] = y;
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < EPT; ++m) {
      const int e = threadIdx.x + m * PNT, c = e / PS, kr = e % PS;
      float sq = 0.f, sk = 0.f;
#pragma unroll 8
      for (int vv = 0; vv < PS; ++vv) {
        sq += sDo[c * PP + vv] * sH[kr * PP + vv];
        sk += sV[c * PP + vv] * sDh[kr * PP + vv];
      }
      aq[m] += sq;
      ak[m] += sk;
    }
    if (threadIdx.x < PS)
      for (int vv = 0; vv < PS; ++vv)
        hdh += sH[threadIdx.x * PP + vv] * sDh[threadIdx.x * PP + vv];
  }
  const float* gc = p.g;
  auto at = [&](int r, int kk) { return ((t0 + r) * H + hh) * (long)K + kk; };
  // dq', dk', the dg terms and sum_c dk_inter k
  __syncthreads();
#pragma unroll
  for (int m = 0; m < EPT; ++m) {
    const int e = threadIdx.x + m * PNT, c = e / PS, kr = e % PS, kk = k0 + kr;
    float w = 0.f, x = 0.f;
    if (kk < K) {
      const float g = gc[at(c, kk)], gn = gc[at(C - 1, kk)];
      const float dqi = p.scale * expf(g) * aq[m], dki = expf(gn - g) * ak[m];
      const float qv = p.q[at(c, kk)], kv = p.k[at(c, kk)];
      const float dqt = p.dq[at(c, kk)] + dqi, dkt = p.dk[at(c, kk)] + dki;
      p.out0[at(c, kk)] = dqt;
      p.out1[at(c, kk)] = dkt;
      w = qv * dqt - kv * dkt;
      x = dki * kv;
    }
    sW[c * PP + kr] = w;
    sDo[c * PP + kr] = x;  // reuse: dk_inter * k
  }
  __syncthreads();
  if (threadIdx.x < PS) {
    const int kr = threadIdx.x, kk = k0 + kr;
    if (kk < K) {
      float inter = expf(gc[at(C - 1, kk)]) * hdh;
      for (int c = 0; c < C; ++c) inter += sDo[c * PP + kr];
      float run = 0.f;
      for (int c = C - 1; c >= 0; --c) {
        run += sW[c * PP + kr];
        p.out2[at(c, kk)] = run + inter;
      }
    }
  }
}

namespace {

template <int C>
hipError_t launch_part(int which, const PartArgs& p, hipStream_t st) {
  const long NC = p.NC, H = p.H;
  const long nks = (p.K + PS - 1) / PS, nvs = (p.V + PS - 1) / PS;
  switch (which) {
    case PART_DA:
      hipLaunchKernelGGL((part_dA_kernel<C>), dim3((unsigned)(NC * H)), dim3(PNT), 0, st, p);
      break;
    case PART_DV:
      hipLaunchKernelGGL((part_dv_kernel<C>), dim3((unsigned)(NC * H * nvs)), dim3(PNT), 0, st,
                         p);
      break;
    case PART_DQK_INTRA:
      hipLaunchKernelGGL((part_dqk_intra_kernel<C>), dim3((unsigned)(NC * H * nks)), dim3(PNT),
                         0, st, p);
      break;
    case PART_DQKG:
      hipLaunchKernelGGL((part_dqkg_kernel<C>), dim3((unsigned)(NC * H * nks)), dim3(PNT), 0,
                         st, p);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t run_bwd_part(int which, const PartArgs& p, int C, hipStream_t st) {
  if ((long)p.NC * p.H == 0) return hipSuccess;
  if (C == 16) return launch_part<16>(which, p, st);
  if (C == 32) return launch_part<32>(which, p, st);
  if (C == 64) return launch_part<64>(which, p, st);
  return hipErrorInvalidValue;
}

}  // namespace tops
