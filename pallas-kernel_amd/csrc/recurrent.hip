// Fused recurrent GLA forward: per-token state update, no MFMA.
// Reference: _fused_recurrent_gla_fwd_kernel, tops/ops/gla/fused_recurrent.py:139-227
// (launcher :235-371, jnp ref :17-132):
//   h <- h * e^{gk_t}[:, None] * e^{gv_t}[None, :] + k_t v_t^T ;  o_t = (scale q_t) . h
// processed forward or in reverse within each sequence.
//
// One 256-thread block per (sequence, head, 64-wide V tile). Lane l owns value column
// vt*64 + l; wave w owns key rows [w*KPT, (w+1)*KPT), so a thread carries KPT fp32 state
// values in registers. q (pre-scaled), k, e^{gk}, v, e^{gv} of TB consecutive tokens are
// staged in LDS (the q/k/gk reads are wave-uniform broadcasts); each wave writes its partial
// o_t to LDS and the four partials are summed once per staged block.
#include "common.hpp"
#include "kernels.hpp"

namespace tops {

constexpr int REC_TB = 16;

template <typename T, typename TO, int KPT>
__global__ __launch_bounds__(256) void recurrent_fwd_kernel(RecArgs p) {
  constexpr int KP = 4 * KPT;
  constexpr int TB = REC_TB;
  __shared__ __attribute__((aligned(16))) float sQ[TB * KP];
  __shared__ __attribute__((aligned(16))) float sK[TB * KP];
  __shared__ __attribute__((aligned(16))) float sG[TB * KP];
  __shared__ float sV[TB * 64];
  __shared__ float sGV[TB * 64];
  __shared__ float sO[4 * TB * 64];

  const T* __restrict__ q = (const T*)p.q;
  const T* __restrict__ k = (const T*)p.k;
  const T* __restrict__ v = (const T*)p.v;
  const T* __restrict__ gk = (const T*)p.gk;
  const T* __restrict__ gv = (const T*)p.gv;
  TO* __restrict__ o = (TO*)p.o;

  const int H = p.H, K = p.K, V = p.V;
  const int VT = (V + 63) >> 6;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int vt = L % VT;
  const int bh = L / VT;
  const int seq = bh / H, hh = bh % H;
  int bos, eos;
  seq_bounds(p.si, seq, bos, eos);  // varlen here carries no chunk offsets
  const int Tq = eos - bos;
  const int vcol = vt * 64 + lane;
  const bool vvalid = vcol < V;
  const int k0 = w * KPT;

  const long sbase = (((long)seq * H + hh) * K + k0) * V + vcol;  // state element (k0, vcol)
  const int kn = min(KPT, K - k0);                                  // valid rows of this wave
  float hr[KPT];
#pragma unroll
  for (int j = 0; j < KPT; ++j) hr[j] = 0.f;
  if (p.h0 && vvalid) {
    const float* src = p.h0 + sbase;
#pragma unroll
    for (int j = 0; j < KPT; ++j)
      if (j < kn) hr[j] = src[(long)j * V];
  }
  const bool has_gk = gk != nullptr, has_gv = gv != nullptr;

  for (int b0 = 0; b0 < Tq; b0 += TB) {
    const int nb = min(TB, Tq - b0);
    // stage TB tokens
#pragma unroll 1
    for (int i = tid; i < TB * KP; i += 256) {
      const int s = i / KP, kk = i % KP;
      float xq = 0.f, xk = 0.f, xg = 1.f;
      if (s < nb && kk < K) {
        const int tau = p.reverse ? (eos - 1 - (b0 + s)) : (bos + b0 + s);
        const long a = ((long)tau * H + hh) * K + kk;
        xq = to_f32(q[a]) * p.scale;
        xk = to_f32(k[a]);
        if (has_gk) xg = gexp<T>(to_f32(gk[a]));
      }
      sQ[i] = xq;
      sK[i] = xk;
      sG[i] = xg;
    }
#pragma unroll 1
    for (int i = tid; i < TB * 64; i += 256) {
      const int s = i >> 6, vv = vt * 64 + (i & 63);
      float xv = 0.f, xg = 1.f;
      if (s < nb && vv < V) {
        const int tau = p.reverse ? (eos - 1 - (b0 + s)) : (bos + b0 + s);
        const long a = ((long)tau * H + hh) * V + vv;
        xv = to_f32(v[a]);
        if (has_gv) xg = gexp<T>(to_f32(gv[a]));
      }
      sV[i] = xv;
      sGV[i] = xg;
    }
    __syncthreads();
#pragma unroll 1
    for (int s = 0; s < nb; ++s) {
      const float vv = sV[s * 64 + lane];
      const float gvv = sGV[s * 64 + lane];
      const float4* q4 = reinterpret_cast<const float4*>(sQ + s * KP + k0);
      const float4* k4 = reinterpret_cast<const float4*>(sK + s * KP + k0);
      const float4* g4 = reinterpret_cast<const float4*>(sG + s * KP + k0);
      float o0 = 0.f, o1 = 0.f, o2 = 0.f, o3 = 0.f;
#pragma unroll
      for (int j4 = 0; j4 < KPT / 4; ++j4) {
        const float4 qq = q4[j4], kk = k4[j4];
        float4 gg = g4[j4];
        if (has_gv) {
          gg.x *= gvv;
          gg.y *= gvv;
          gg.z *= gvv;
          gg.w *= gvv;
        }
        hr[4 * j4 + 0] = fmaf(hr[4 * j4 + 0], gg.x, kk.x * vv);
        hr[4 * j4 + 1] = fmaf(hr[4 * j4 + 1], gg.y, kk.y * vv);
        hr[4 * j4 + 2] = fmaf(hr[4 * j4 + 2], gg.z, kk.z * vv);
        hr[4 * j4 + 3] = fmaf(hr[4 * j4 + 3], gg.w, kk.w * vv);
        o0 = fmaf(qq.x, hr[4 * j4 + 0], o0);
        o1 = fmaf(qq.y, hr[4 * j4 + 1], o1);
        o2 = fmaf(qq.z, hr[4 * j4 + 2], o2);
        o3 = fmaf(qq.w, hr[4 * j4 + 3], o3);
      }
      sO[(w * TB + s) * 64 + lane] = (o0 + o1) + (o2 + o3);
    }
    __syncthreads();
#pragma unroll 1
    for (int i = tid; i < nb * 64; i += 256) {
      const int s = i >> 6, vl = i & 63;
      const int vv = vt * 64 + vl;
      if (vv < V) {
        const float val = sO[(0 * TB + s) * 64 + vl] + sO[(1 * TB + s) * 64 + vl] +
                          sO[(2 * TB + s) * 64 + vl] + sO[(3 * TB + s) * 64 + vl];
        const int tau = p.reverse ? (eos - 1 - (b0 + s)) : (bos + b0 + s);
        o[((long)tau * H + hh) * V + vv] = from_f32<TO>(val);
      }
    }
  }
  if (p.ht && vvalid) {
    float* dst = p.ht + sbase;
#pragma unroll
    for (int j = 0; j < KPT; ++j)
      if (j < kn) dst[(long)j * V] = hr[j];
  }
}

template <typename T, typename TO, int KPT>
static hipError_t launch_rec(const RecArgs& p, hipStream_t st) {
  const int VT = (p.V + 63) / 64;
  const long blocks = (long)p.si.N * p.H * VT;
  if (blocks == 0) return hipSuccess;
  hipLaunchKernelGGL((recurrent_fwd_kernel<T, TO, KPT>), dim3((unsigned)blocks), dim3(256), 0,
                     st, p);
  return hipGetLastError();
}

template <typename T, typename TO>
static hipError_t dispatch_rec(const RecArgs& p, hipStream_t st) {
  const int need = (p.K + 3) / 4;
  if (need <= 4) return launch_rec<T, TO, 4>(p, st);
  if (need <= 8) return launch_rec<T, TO, 8>(p, st);
  if (need <= 16) return launch_rec<T, TO, 16>(p, st);
  if (need <= 32) return launch_rec<T, TO, 32>(p, st);
  if (need <= 64) return launch_rec<T, TO, 64>(p, st);
  return hipErrorInvalidValue;
}

hipError_t run_recurrent_fwd(const RecArgs& p, int dtype, int o_dtype, hipStream_t st) {
  if (dtype == DT_BF16 && o_dtype == DT_F32) return dispatch_rec<bf16, float>(p, st);
  if (dtype == DT_BF16 && o_dtype == DT_BF16) return dispatch_rec<bf16, bf16>(p, st);
  if (dtype == DT_F32 && o_dtype == DT_F32) return dispatch_rec<float, float>(p, st);
  return hipErrorInvalidValue;
}

}  // namespace tops
