// Per-chunk gradients of chunked GLA.
//
// Reference: fused Pallas kernel tops/ops/gla/chunk.py:1423-1479 and the jnp sub-functions
// chunk.py:504-743 (dA, dv, dq/dk intra, dq/dk inter + dg). With g~ the chunk-local cumsum,
// gamma its last row, h = state entering the chunk, dh = gradient w.r.t. the state leaving
// it, and the per-column exponent reference r = (g~_first + gamma) / 2:
//   dA  = scale tril(do v^T)
//   dq  = e^{g~-r} [ dA (k e^{r-g~}) + (scale e^{r}) do h^T ]
//   dk  = e^{r-g~} [ dA^T (q e^{g~-r}) + e^{gamma-r} v dh^T ]
//   dv  = tril(A)^T do + (k e^{gamma-g~}) dh,     A = scale (q e^{g~-r})(k e^{r-g~})^T
//   dg  = revcumsum_chunk(q dq - k dk) + e^{gamma} sum_v h dh + sum_j k dk_inter
//
// chunk_bwd_dqkg_kernel: one 256-thread block per (chunk, head, 64-wide K tile); every
//   quantity above except dv is local to a K tile (contractions run over V and the chunk).
// chunk_bwd_dv_kernel:   one block per (chunk, head, 64-wide V tile); accumulates the
//   K contraction of A^T and of kd.dh over K tiles.
#include "common.hpp"
#include "kernels.hpp"

namespace tops {

// dynamic LDS layout of chunk_bwd_dqkg_kernel (bytes); `exch` aliases the T buffers
template <typename T>
struct DqkgLayout {
  int qgT, kgT, do_, v, h, dh, dA, dAT, tbytes, exch_bytes, total;
  __host__ __device__ DqkgLayout(int C) {
    const int CP = C < 32 ? 32 : C;
    const int a64 = ((64 * pitch_of<T>(CP) * (int)sizeof(T)) + 15) / 16 * 16;  // [64][CP]
    const int c64 = ((C * pitch_of<T>(64) * (int)sizeof(T)) + 15) / 16 * 16;   // [C][64]
    const int s64 = ((64 * pitch_of<T>(64) * (int)sizeof(T)) + 15) / 16 * 16;  // [64][64]
    const int ccp = ((C * pitch_of<T>(CP) * (int)sizeof(T)) + 15) / 16 * 16;   // [C][CP]
    qgT = 0;
    kgT = qgT + a64;
    do_ = kgT + a64;
    v = do_ + c64;
    h = v + c64;
    dh = h + s64;
    dA = dh + s64;
    dAT = dA + ccp;
    tbytes = dAT + ccp;
    exch_bytes = 3 * C * 68 * 4;
    total = tbytes > exch_bytes ? tbytes : exch_bytes;
  }
};

template <typename T, int C>
__global__ __launch_bounds__(256) void chunk_bwd_dqkg_kernel(BwdArgs p) {
  constexpr int CP = C < 32 ? 32 : C;
  constexpr int RPS = C / 4;
  constexpr int P64 = pitch_of<T>(64), PCP = pitch_of<T>(CP);
  constexpr int NTM = C / 16, NT_A = NTM * NTM, NA = (NT_A + 3) / 4;
  constexpr int NO = NTM;  // C x 64 tile = 4*NTM 16x16 tiles over 4 waves
  constexpr int PX = 68;   // fp32 exchange pitch
  extern __shared__ __attribute__((aligned(16))) unsigned char dyn[];
  __shared__ float sTot[256], sAux[256];
  __shared__ float sR[64], sEg[64], sHd[64];
  const DqkgLayout<T> lay(C);
  T* sQgT = reinterpret_cast<T*>(dyn + lay.qgT);
  T* sKgT = reinterpret_cast<T*>(dyn + lay.kgT);
  T* sDo = reinterpret_cast<T*>(dyn + lay.do_);
  T* sV = reinterpret_cast<T*>(dyn + lay.v);
  T* sH = reinterpret_cast<T*>(dyn + lay.h);
  T* sDh = reinterpret_cast<T*>(dyn + lay.dh);
  T* sdA = reinterpret_cast<T*>(dyn + lay.dA);
  T* sdAT = reinterpret_cast<T*>(dyn + lay.dAT);
  float* XQ = reinterpret_cast<float*>(dyn);
  float* XK = XQ + C * PX;
  float* XM = XK + C * PX;

  const T* __restrict__ q = (const T*)p.q;
  const T* __restrict__ k = (const T*)p.k;
  const T* __restrict__ v = (const T*)p.v;
  const T* __restrict__ g = (const T*)p.g;
  const T* __restrict__ dout = (const T*)p.dout;
  const T* __restrict__ hs = (const T*)p.h;
  const T* __restrict__ dhs = (const T*)p.dh;

  const int H = p.H, K = p.K, V = p.V;
  const int KT = (K + 63) >> 6, VT = (V + 63) >> 6;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int kt = L % KT;
  const int c = (L / KT) / H, hh = (L / KT) % H;
  int seq, t0, len;
  chunk_range(p.si, c, seq, t0, len);
  (void)seq;
  const long rsK = (long)H * K, rsV = (long)H * V;
  const long baseK = ((long)t0 * H + hh) * K, baseV = ((long)t0 * H + hh) * V;
  const int col = tid & 63, seg = tid >> 6;
  const int gcol = kt * 64 + col;
  const bool kvalid = gcol < K;

  if (CP > C) {
    for (int i = tid; i < 64 * (CP - C); i += 256) {
      const int rr = i / (CP - C), cc = C + i % (CP - C);
      sQgT[rr * PCP + cc] = zero_elem<T>();
      sKgT[rr * PCP + cc] = zero_elem<T>();
    }
    for (int i = tid; i < C * (CP - C); i += 256) {
      const int rr = i / (CP - C), cc = C + i % (CP - C);
      sdA[rr * PCP + cc] = zero_elem<T>();
      sdAT[rr * PCP + cc] = zero_elem<T>();
    }
  }

  // ---- prologue: gates of this K tile ----
  float gt[RPS], qreg[RPS], kreg[RPS];
  float gamma, first;
  tile_cumsum<C>(g + baseK + gcol, rsK, len, kvalid, false, sTot, gt, gamma, first);
  const float r = 0.5f * (first + gamma);
#pragma unroll
  for (int rr = 0; rr < RPS; ++rr) {
    const int row = seg * RPS + rr;
    float qv = 0.f, kv = 0.f;
    if (row < len && kvalid) {
      qv = to_f32(q[baseK + (long)row * rsK + gcol]);
      kv = to_f32(k[baseK + (long)row * rsK + gcol]);
    }
    qreg[rr] = qv;
    kreg[rr] = kv;
    const float d = gt[rr] - r;
    sQgT[col * PCP + row] = from_f32<T>(qv * gexp<T>(d));
    sKgT[col * PCP + row] = from_f32<T>(kv * gexp<T>(-d));
  }
  if (seg == 0) {
    sR[col] = p.scale * gexp<T>(r);
    sEg[col] = gexp<T>(gamma - r);
  }

  f32x4 dA[NA], dAT[NA], Mqx[NO], M2[NO];
#pragma unroll
  for (int j = 0; j < NA; ++j) dA[j] = dAT[j] = zero4();
#pragma unroll
  for (int j = 0; j < NO; ++j) Mqx[j] = M2[j] = zero4();
  float hdp = 0.f;
  const long hbase = ((long)c * H + hh) * K;

  for (int vt = 0; vt < VT; ++vt) {
    const int vcol = vt * 64 + col;
    const bool vvalid = vcol < V;
#pragma unroll
    for (int rr = 0; rr < RPS; ++rr) {
      const int row = seg * RPS + rr;
      float x = 0.f, y = 0.f;
      if (row < len && vvalid) {
        x = to_f32(dout[baseV + (long)row * rsV + vcol]);
        y = to_f32(v[baseV + (long)row * rsV + vcol]);
      }
      sDo[row * P64 + col] = from_f32<T>(x);
      sV[row * P64 + col] = from_f32<T>(y);
    }
#pragma unroll 4
    for (int i = 0; i < 16; ++i) {
      const int kk = seg * 16 + i;
      const int gk = kt * 64 + kk;
      T a = zero_elem<T>(), b = zero_elem<T>();
      if (gk < K && vvalid) {
        a = hs[(hbase + gk) * V + vcol];
        b = dhs[(hbase + gk) * V + vcol];
      }
      sH[kk * P64 + col] = a;
      sDh[kk * P64 + col] = b;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NA; ++j) {
      const int t = w + 4 * j;
      if (t < NT_A) {
        const int mi = t / NTM, ni = t % NTM;
        mma_tile<T>(dA[j], sDo + mi * 16 * P64, P64, sV + ni * 16 * P64, P64, 64, lane);
        mma_tile<T>(dAT[j], sV + mi * 16 * P64, P64, sDo + ni * 16 * P64, P64, 64, lane);
      }
    }
#pragma unroll
    for (int j = 0; j < NO; ++j) {
      const int t = w + 4 * j;
      const int mi = t >> 2, ni = t & 3;
      mma_tile<T>(Mqx[j], sDo + mi * 16 * P64, P64, sH + ni * 16 * P64, P64, 64, lane);
      mma_tile<T>(M2[j], sV + mi * 16 * P64, P64, sDh + ni * 16 * P64, P64, 64, lane);
    }
    {
      const int kk = tid >> 2, v0 = (tid & 3) * 16;
#pragma unroll
      for (int i = 0; i < 16; ++i)
        hdp += to_f32(sH[kk * P64 + v0 + i]) * to_f32(sDh[kk * P64 + v0 + i]);
    }
    __syncthreads();
  }
  hdp += __shfl_xor(hdp, 1);
  hdp += __shfl_xor(hdp, 2);
  if ((tid & 3) == 0) sHd[tid >> 2] = hdp;

  // ---- masked dA / dA^T to LDS ----
#pragma unroll
  for (int j = 0; j < NA; ++j) {
    const int t = w + 4 * j;
    if (t < NT_A) {
      const int mi = t / NTM, ni = t % NTM;
      const int cc = ni * 16 + (lane & 15);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int ro = mi * 16 + 4 * (lane >> 4) + rr;
        // dA[i=ro][j=cc] kept for j <= i ; dA^T[j=ro][i=cc] kept for i >= j
        sdA[ro * PCP + cc] = from_f32<T>(cc <= ro ? dA[j][rr] * p.scale : 0.f);
        sdAT[ro * PCP + cc] = from_f32<T>(cc >= ro ? dAT[j][rr] * p.scale : 0.f);
      }
    }
  }
  __syncthreads();

  f32x4 Mqi[NO], Mk1[NO];
#pragma unroll
  for (int j = 0; j < NO; ++j) {
    const int t = w + 4 * j;
    const int mi = t >> 2, ni = t & 3;
    Mqi[j] = zero4();
    Mk1[j] = zero4();
    mma_tile<T>(Mqi[j], sdA + mi * 16 * PCP, PCP, sKgT + ni * 16 * PCP, PCP, CP, lane);
    mma_tile<T>(Mk1[j], sdAT + mi * 16 * PCP, PCP, sQgT + ni * 16 * PCP, PCP, CP, lane);
  }
  __syncthreads();  // T buffers are dead; the exchange area aliases them

#pragma unroll
  for (int j = 0; j < NO; ++j) {
    const int t = w + 4 * j;
    const int mi = t >> 2, ni = t & 3;
    const int kk = ni * 16 + (lane & 15);
    const float fr = sR[kk], fe = sEg[kk];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int ro = mi * 16 + 4 * (lane >> 4) + rr;
      XQ[ro * PX + kk] = Mqi[j][rr] + fr * Mqx[j][rr];
      XK[ro * PX + kk] = Mk1[j][rr] + fe * M2[j][rr];
      XM[ro * PX + kk] = fe * M2[j][rr];
    }
  }
  __syncthreads();

  // ---- column epilogue: dq, dk, dg ----
  T* __restrict__ dq = (T*)p.dq;
  T* __restrict__ dk = (T*)p.dk;
  T* __restrict__ dg = (T*)p.dg;
  float dgr[RPS];
  float run = 0.f, dki = 0.f;
#pragma unroll
  for (int rr = RPS - 1; rr >= 0; --rr) {
    const int row = seg * RPS + rr;
    const float ep = gexp<T>(gt[rr] - r), en = gexp<T>(r - gt[rr]);
    const float vq = ep * XQ[row * PX + col];
    const float vk = en * XK[row * PX + col];
    const float vm = en * XM[row * PX + col];
    dki += kreg[rr] * vm;
    run += qreg[rr] * vq - kreg[rr] * vk;
    dgr[rr] = run;
    if (row < len && kvalid) {
      dq[baseK + (long)row * rsK + gcol] = from_f32<T>(vq);
      dk[baseK + (long)row * rsK + gcol] = from_f32<T>(vk);
    }
  }
  sTot[seg * 64 + col] = run;
  sAux[seg * 64 + col] = dki;
  __syncthreads();
  float off = 0.f, dks = 0.f;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    off += (s > seg) ? sTot[s * 64 + col] : 0.f;
    dks += sAux[s * 64 + col];
  }
  const float dgk = gexp<T>(gamma) * sHd[col] + dks;
#pragma unroll
  for (int rr = 0; rr < RPS; ++rr) {
    const int row = seg * RPS + rr;
    if (row < len && kvalid) dg[baseK + (long)row * rsK + gcol] = from_f32<T>(dgr[rr] + off + dgk);
  }
}

template <typename T, int C>
__global__ __launch_bounds__(256) void chunk_bwd_dv_kernel(BwdArgs p) {
  constexpr int CP = C < 32 ? 32 : C;
  constexpr int RPS = C / 4;
  constexpr int P64 = pitch_of<T>(64), PCP = pitch_of<T>(CP);
  constexpr int NTM = C / 16, NT_A = NTM * NTM, NA = (NT_A + 3) / 4;
  constexpr int NO = NTM;
  __shared__ __attribute__((aligned(16))) T sKg[C * P64];
  __shared__ __attribute__((aligned(16))) T sQg[C * P64];
  __shared__ __attribute__((aligned(16))) T sKd[C * P64];
  __shared__ __attribute__((aligned(16))) T sDhT[64 * P64];
  __shared__ __attribute__((aligned(16))) T sAT[C * PCP];
  __shared__ __attribute__((aligned(16))) T sDoT[64 * PCP];
  __shared__ float sTot[256];

  const T* __restrict__ q = (const T*)p.q;
  const T* __restrict__ k = (const T*)p.k;
  const T* __restrict__ g = (const T*)p.g;
  const T* __restrict__ dout = (const T*)p.dout;
  const T* __restrict__ dhs = (const T*)p.dh;
  T* __restrict__ dv = (T*)p.dv;

  const int H = p.H, K = p.K, V = p.V;
  const int KT = (K + 63) >> 6, VT = (V + 63) >> 6;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int vt = L % VT;
  const int c = (L / VT) / H, hh = (L / VT) % H;
  int seq, t0, len;
  chunk_range(p.si, c, seq, t0, len);
  (void)seq;
  const long rsK = (long)H * K, rsV = (long)H * V;
  const long baseK = ((long)t0 * H + hh) * K, baseV = ((long)t0 * H + hh) * V;
  const int col = tid & 63, seg = tid >> 6;
  const int vcol = vt * 64 + col;
  const bool vvalid = vcol < V;

  if (CP > C) {
    for (int i = tid; i < C * (CP - C); i += 256)
      sAT[(i / (CP - C)) * PCP + C + i % (CP - C)] = zero_elem<T>();
    for (int i = tid; i < 64 * (CP - C); i += 256)
      sDoT[(i / (CP - C)) * PCP + C + i % (CP - C)] = zero_elem<T>();
  }

  f32x4 AT[NA], Mdv[NO];
#pragma unroll
  for (int j = 0; j < NA; ++j) AT[j] = zero4();
#pragma unroll
  for (int j = 0; j < NO; ++j) Mdv[j] = zero4();
  const long hbase = ((long)c * H + hh) * K;

  for (int kt = 0; kt < KT; ++kt) {
    const int gcol = kt * 64 + col;
    const bool kvalid = gcol < K;
    float gt[RPS];
    float gamma, first;
    tile_cumsum<C>(g + baseK + gcol, rsK, len, kvalid, false, sTot, gt, gamma, first);
    const float r = 0.5f * (first + gamma);
#pragma unroll
    for (int rr = 0; rr < RPS; ++rr) {
      const int row = seg * RPS + rr;
      float qv = 0.f, kv = 0.f;
      if (row < len && kvalid) {
        qv = to_f32(q[baseK + (long)row * rsK + gcol]);
        kv = to_f32(k[baseK + (long)row * rsK + gcol]);
      }
      const float d = gt[rr] - r;
      sQg[row * P64 + col] = from_f32<T>(qv * gexp<T>(d));
      sKg[row * P64 + col] = from_f32<T>(kv * gexp<T>(-d));
      sKd[row * P64 + col] = from_f32<T>(kv * gexp<T>(gamma - gt[rr]));
    }
#pragma unroll 4
    for (int i = 0; i < 16; ++i) {
      const int kk = seg * 16 + i;
      const int gk = kt * 64 + kk;
      T x = zero_elem<T>();
      if (gk < K && vvalid) x = dhs[(hbase + gk) * V + vcol];
      sDhT[col * P64 + kk] = x;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NA; ++j) {
      const int t = w + 4 * j;
      if (t < NT_A) {
        const int mi = t / NTM, ni = t % NTM;
        mma_tile<T>(AT[j], sKg + mi * 16 * P64, P64, sQg + ni * 16 * P64, P64, 64, lane);
      }
    }
#pragma unroll
    for (int j = 0; j < NO; ++j) {
      const int t = w + 4 * j;
      const int mi = t >> 2, ni = t & 3;
      mma_tile<T>(Mdv[j], sKd + mi * 16 * P64, P64, sDhT + ni * 16 * P64, P64, 64, lane);
    }
    __syncthreads();
  }

#pragma unroll
  for (int j = 0; j < NA; ++j) {
    const int t = w + 4 * j;
    if (t < NT_A) {
      const int mi = t / NTM, ni = t % NTM;
      const int cc = ni * 16 + (lane & 15);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int ro = mi * 16 + 4 * (lane >> 4) + rr;  // j ; cc = i
        sAT[ro * PCP + cc] = from_f32<T>(cc >= ro ? AT[j][rr] * p.scale : 0.f);
      }
    }
  }
#pragma unroll
  for (int rr = 0; rr < RPS; ++rr) {
    const int row = seg * RPS + rr;
    float x = 0.f;
    if (row < len && vvalid) x = to_f32(dout[baseV + (long)row * rsV + vcol]);
    sDoT[col * PCP + row] = from_f32<T>(x);
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < NO; ++j) {
    const int t = w + 4 * j;
    const int mi = t >> 2, ni = t & 3;
    mma_tile<T>(Mdv[j], sAT + mi * 16 * PCP, PCP, sDoT + ni * 16 * PCP, PCP, CP, lane);
    const int oc = vt * 64 + ni * 16 + (lane & 15);
    if (oc < V) {
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int ro = mi * 16 + 4 * (lane >> 4) + rr;
        if (ro < len) dv[baseV + (long)ro * rsV + oc] = from_f32<T>(Mdv[j][rr]);
      }
    }
  }
}

template <typename T, int C>
static hipError_t launch_bwd(const BwdArgs& p, hipStream_t st, int which) {
  const int KT = (p.K + 63) / 64, VT = (p.V + 63) / 64;
  const long nch = (long)p.si.NC * p.H;
  if (nch == 0) return hipSuccess;
  if (which & 1) {
    const DqkgLayout<T> lay(C);
    hipError_t e = hipFuncSetAttribute((const void*)chunk_bwd_dqkg_kernel<T, C>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, lay.total);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((chunk_bwd_dqkg_kernel<T, C>), dim3((unsigned)(nch * KT)), dim3(256),
                       lay.total, st, p);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (which & 2) {
    hipLaunchKernelGGL((chunk_bwd_dv_kernel<T, C>), dim3((unsigned)(nch * VT)), dim3(256), 0,
                       st, p);
    return hipGetLastError();
  }
  return hipSuccess;
}

template <typename T>
static hipError_t dispatch_bwd(const BwdArgs& p, hipStream_t st, int which) {
  switch (p.si.C) {
    case 16: return launch_bwd<T, 16>(p, st, which);
    case 32: return launch_bwd<T, 32>(p, st, which);
    case 64: return launch_bwd<T, 64>(p, st, which);
    default: return hipErrorInvalidValue;
  }
}

hipError_t run_chunk_bwd(const BwdArgs& p, int dtype, hipStream_t st, int which) {
  if (dtype == DT_BF16) return dispatch_bwd<bf16>(p, st, which);
  if (dtype == DT_F32) return dispatch_bwd<float>(p, st, which);
  return hipErrorInvalidValue;
}

}  // namespace tops
