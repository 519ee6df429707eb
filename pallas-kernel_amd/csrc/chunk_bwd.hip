// Per-chunk gradients of chunked GLA.
//
// Reference: fused Pallas kernel tops/ops/gla/chunk.py:1423-1479 and the jnp sub-functions
// chunk.py:504-743 (dA, dv, dq/dk intra, dq/dk inter + dg). With g~ the chunk-local cumsum,
// gamma its last row, h = state entering the chunk, dh = gradient w.r.t. the state leaving
// it, and the per-column exponent reference r = (g~_first + gamma) / 2:
//   dA  = scale tril(do v^T)
//   dq  = e^{g~-r} [ dA (k e^{r-g~}) + (scale e^{r}) do h^T ]
//   dk  = e^{r-g~} [ dA^T (q e^{g~-r}) + e^{gamma-r} v dh^T ]
//   dv  = tril(A)^T do + (k e^{r-g~}) (e^{gamma-r} dh),   A = scale (q e^{g~-r})(k e^{r-g~})^T
//   dg  = revcumsum_chunk(q dq - k dk) + e^{gamma} sum_v h dh + sum_j k dk_inter
//
// chunk_bwd_dqkg_kernel: one 256-thread block per (chunk, head, 64-wide K tile); everything
//   above except dv is local to a K tile (its contractions run over V and over the chunk).
// chunk_bwd_dv_kernel:   one block per (chunk, head, 64-wide V tile), accumulating the
//   K contractions of A and of k_d.dh over K tiles; it produces dv^T tiles so that each lane
//   holds four consecutive values of a row (bf16 with 64-row chunks: staged in LDS and
//   stored as whole 16-byte row pieces; otherwise stored directly). With the per-chunk
//   gating workspace (PRE: wide bf16 heads, chunk 64) it reads kg, e^{gamma-r} and A from
//   there instead: the gating and A would otherwise be recomputed by every V tile's block of
//   a (chunk, head).
// Tiles are staged in LDS row-major exactly as loaded (16-byte global loads); operands that
// are needed transposed (kg^T, qg^T, dA^T, dh^T, do^T, A^T) are read with transposed MFMA
// fragments. Element-wise work maps a thread to two adjacent columns x C/8 rows.
#include "common.hpp"
#include "kernels.hpp"

namespace tops {

// ---------------------------------------------------------------------------
// shared pieces
// ---------------------------------------------------------------------------

// 16-byte loads of an [R x 64] tile into registers: rows of stride `rs` elements, tile
// columns col0..col0+63 of rows whose valid width is `width`; rows >= len and columns past
// the width read as zero. Piece pc = tid + 256 j covers row pc / (64/EPP).
template <typename T, int R, bool VEC, int PPT>
__device__ __forceinline__ void tile_load(uint4 (&r)[PPT], const T* __restrict__ base, long rs,
                                          int len, int col0, int width, int tid) {
  constexpr int EPP = 16 / (int)sizeof(T);
  constexpr int PPR = 64 / EPP;
#pragma unroll
  for (int j = 0; j < PPT; ++j) {
    const int pc = tid + 256 * j;
    const int row = pc / PPR, c = (pc % PPR) * EPP;
    r[j] = make_uint4(0, 0, 0, 0);
    if (pc < R * PPR && row < len)
      r[j] = gload16<T, VEC>(base + row * rs + col0, c, width - col0 - c);
  }
}

template <typename T, int R, int PPT>
__device__ __forceinline__ void tile_store(T* s, int pitch, const uint4 (&r)[PPT], int tid) {
  constexpr int EPP = 16 / (int)sizeof(T);
  constexpr int PPR = 64 / EPP;
#pragma unroll
  for (int j = 0; j < PPT; ++j) {
    const int pc = tid + 256 * j;
    if (pc < R * PPR) *reinterpret_cast<uint4*>(s + (pc / PPR) * pitch + (pc % PPR) * EPP) = r[j];
  }
}

template <typename T, int R>
constexpr int pieces_per_thread() {
  return (R * (64 / (16 / (int)sizeof(T))) + 255) / 256;
}

// Column-pair chunk-local cumsum of a raw gate tile in LDS (thread: columns c0, c0+1, rows
// seg*RPS .. +RPS). On return d0/d1 hold g~ - r, gam0/1 = gamma, r0/1 = r for the two
// columns. sTot: 8*64 floats, sFirst: 64 floats. Contains one __syncthreads().
template <typename T, int C>
__device__ __forceinline__ void pair_cumsum(const T* sG, int pitch, int c0, int seg,
                                            float* sTot, float* sFirst, float (&d0)[C / 8],
                                            float (&d1)[C / 8], float& gam0, float& gam1,
                                            float& r0, float& r1) {
  constexpr int NSEG = 8, RPS = C / NSEG;
  float run0 = 0.f, run1 = 0.f;
#pragma unroll
  for (int rr = 0; rr < RPS; ++rr) {
    float x0, x1;
    Pair<T>::ld(sG + (seg * RPS + rr) * pitch + c0, x0, x1);
    run0 += x0;
    run1 += x1;
    d0[rr] = run0;
    d1[rr] = run1;
  }
  sTot[seg * 64 + c0] = run0;
  sTot[seg * 64 + c0 + 1] = run1;
  if (seg == 0) {
    sFirst[c0] = d0[0];
    sFirst[c0 + 1] = d1[0];
  }
  __syncthreads();
  float off0 = 0.f, off1 = 0.f;
  gam0 = gam1 = 0.f;
#pragma unroll
  for (int s = 0; s < NSEG; ++s) {
    const float x0 = sTot[s * 64 + c0], x1 = sTot[s * 64 + c0 + 1];
    off0 += (s < seg) ? x0 : 0.f;
    off1 += (s < seg) ? x1 : 0.f;
    gam0 += x0;
    gam1 += x1;
  }
  r0 = 0.5f * (sFirst[c0] + gam0);
  r1 = 0.5f * (sFirst[c0 + 1] + gam1);
#pragma unroll
  for (int rr = 0; rr < RPS; ++rr) {
    d0[rr] += off0 - r0;
    d1[rr] += off1 - r1;
  }
}

// ---------------------------------------------------------------------------
// dq, dk, dg
// ---------------------------------------------------------------------------

template <typename T, int C>
struct DqkgLayout {
  static constexpr int CP = C < 32 ? 32 : C;   // contraction over the chunk: multiple of 32
  static constexpr int P64 = pitch_of<T>(64), PCP = pitch_of<T>(CP);
  static constexpr int ES = (int)sizeof(T);
  static constexpr int TILE = ((CP * P64 * ES) + 15) / 16 * 16;   // [CP][64]
  static constexpr int SQ = ((64 * P64 * ES) + 15) / 16 * 16;     // [64][64]
  static constexpr int DA = ((CP * PCP * ES) + 15) / 16 * 16;     // [CP][CP]
  // region A: raw q, k, g (prologue) then do, v | h, dh | qg, kg | dA
  static constexpr int qr = 0, kr = TILE, gr = 2 * TILE;
  static constexpr int do_ = 0, v = TILE;
  static constexpr int h = 3 * TILE, dh = 3 * TILE + SQ;
  static constexpr int qg = 3 * TILE + 2 * SQ, kg = qg + TILE;
  static constexpr int dA = kg + TILE;
  static constexpr int tbytes = dA + DA;
  static constexpr int PX = 68;                      // fp32 exchange pitch
  static constexpr int exch = 3 * C * PX * 4;        // aliases everything above
  static constexpr int bytes = tbytes > exch ? tbytes : exch;
};

template <typename T, int C, bool VEC>
__global__ __launch_bounds__(256) void chunk_bwd_dqkg_kernel(BwdArgs p) {
  using Lay = DqkgLayout<T, C>;
  constexpr int CP = Lay::CP, P64 = Lay::P64, PCP = Lay::PCP, PX = Lay::PX;
  constexpr int PPT = pieces_per_thread<T, C>(), HPT = pieces_per_thread<T, 64>();
  constexpr int NSEG = 8, RPS = C / NSEG;
  constexpr int NTM = C / 16, NT_A = NTM * NTM, NA = (NT_A + 3) / 4;
  constexpr int NO = NTM;   // [C x 64] output = 4*NTM 16x16 tiles over 4 waves
  extern __shared__ __attribute__((aligned(16))) unsigned char dyn[];
  __shared__ float sTot[NSEG * 64], sAux[NSEG * 64];
  __shared__ float sR[64], sEg[64], sGm[64], sHd[64];
  T* sQr = reinterpret_cast<T*>(dyn + Lay::qr);
  T* sKr = reinterpret_cast<T*>(dyn + Lay::kr);
  T* sGr = reinterpret_cast<T*>(dyn + Lay::gr);
  T* sDo = reinterpret_cast<T*>(dyn + Lay::do_);
  T* sV = reinterpret_cast<T*>(dyn + Lay::v);
  T* sH = reinterpret_cast<T*>(dyn + Lay::h);
  T* sDh = reinterpret_cast<T*>(dyn + Lay::dh);
  T* sQg = reinterpret_cast<T*>(dyn + Lay::qg);
  T* sKg = reinterpret_cast<T*>(dyn + Lay::kg);
  T* sdA = reinterpret_cast<T*>(dyn + Lay::dA);
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
  const int kb = kt * 64, klen = min(64, K - kb);
  const T* __restrict__ hrow = hs + (((long)c * H + hh) * K + kb) * V;    // h[c][kb][0]
  const T* __restrict__ dhrow = dhs + (((long)c * H + hh) * K + kb) * V;  // dh[c][kb][0]

  // global -> registers: q, k, g of this K tile and V tile 0 of do, v, h, dh
  uint4 rq[PPT], rk[PPT], rg[PPT], rdo[PPT], rv[PPT], rh[HPT], rdh[HPT];
  tile_load<T, C, VEC>(rq, q + baseK, rsK, len, kb, K, tid);
  tile_load<T, C, VEC>(rk, k + baseK, rsK, len, kb, K, tid);
  tile_load<T, C, VEC>(rg, g + baseK, rsK, len, kb, K, tid);
  tile_load<T, C, VEC>(rdo, dout + baseV, rsV, len, 0, V, tid);
  tile_load<T, C, VEC>(rv, v + baseV, rsV, len, 0, V, tid);
  tile_load<T, 64, VEC>(rh, hrow, V, klen, 0, V, tid);
  tile_load<T, 64, VEC>(rdh, dhrow, V, klen, 0, V, tid);
  if (CP > C) {   // rows [C, CP) of the chunk-contraction operands stay zero
    for (int i = tid; i < (CP - C) * P64; i += 256) {
      sQg[C * P64 + i] = zero_elem<T>();
      sKg[C * P64 + i] = zero_elem<T>();
    }
    for (int i = tid; i < CP * PCP; i += 256)
      if (i >= C * PCP || i % PCP >= C) sdA[i] = zero_elem<T>();
  }
  tile_store<T, C>(sQr, P64, rq, tid);
  tile_store<T, C>(sKr, P64, rk, tid);
  tile_store<T, C>(sGr, P64, rg, tid);
  tile_store<T, 64>(sH, P64, rh, tid);
  tile_store<T, 64>(sDh, P64, rdh, tid);
  __syncthreads();

  // ---- cumsum and gating ----
  const int cp = tid & 31, seg = tid >> 5;
  const int c_0 = 2 * cp, c_1 = c_0 + 1;
  float q0[RPS], q1[RPS], k0[RPS], k1[RPS], d0[RPS], d1[RPS];
  float gam0, gam1, r0, r1;
  pair_cumsum<T, C>(sGr, P64, c_0, seg, sTot, sAux, d0, d1, gam0, gam1, r0, r1);
#pragma unroll
  for (int rr = 0; rr < RPS; ++rr) {
    const int row = seg * RPS + rr;
    Pair<T>::ld(sQr + row * P64 + c_0, q0[rr], q1[rr]);
    Pair<T>::ld(sKr + row * P64 + c_0, k0[rr], k1[rr]);
    const float e0 = gexp<T>(d0[rr]), e1 = gexp<T>(d1[rr]);
    Pair<T>::st(sQg + row * P64 + c_0, q0[rr] * e0, q1[rr] * e1);
    Pair<T>::st(sKg + row * P64 + c_0, gdiv<T>(k0[rr], d0[rr], e0),
                gdiv<T>(k1[rr], d1[rr], e1));
  }
  if (seg == 0) {
    sR[c_0] = p.scale * gexp<T>(r0);
    sR[c_1] = p.scale * gexp<T>(r1);
    sEg[c_0] = gexp<T>(gam0 - r0);
    sEg[c_1] = gexp<T>(gam1 - r1);
    sGm[c_0] = gexp<T>(gam0);
    sGm[c_1] = gexp<T>(gam1);
  }
  __syncthreads();   // raw q, k, g are dead: region A takes do, v
  tile_store<T, C>(sDo, P64, rdo, tid);
  tile_store<T, C>(sV, P64, rv, tid);
  __syncthreads();

  f32x4 dA[NA], Mqx[NO], M2[NO];
#pragma unroll
  for (int j = 0; j < NA; ++j) dA[j] = zero4();
#pragma unroll
  for (int j = 0; j < NO; ++j) Mqx[j] = M2[j] = zero4();
  float hdp = 0.f;
  // V tiles: the next tile's loads are issued before this tile's products (its registers
  // are free once the tile is in LDS), so they arrive under the MFMA work
  for (int vt = 0; vt < VT; ++vt) {
    if (vt > 0) {
      __syncthreads();   // readers of the previous V tile are done
      tile_store<T, C>(sDo, P64, rdo, tid);
      tile_store<T, C>(sV, P64, rv, tid);
      tile_store<T, 64>(sH, P64, rh, tid);
      tile_store<T, 64>(sDh, P64, rdh, tid);
      __syncthreads();
    }
    if (vt + 1 < VT) {
      const int vb = (vt + 1) * 64;
      tile_load<T, C, VEC>(rdo, dout + baseV, rsV, len, vb, V, tid);
      tile_load<T, C, VEC>(rv, v + baseV, rsV, len, vb, V, tid);
      tile_load<T, 64, VEC>(rh, hrow, V, klen, vb, V, tid);
      tile_load<T, 64, VEC>(rdh, dhrow, V, klen, vb, V, tid);
    }
#pragma unroll
    for (int j = 0; j < NA; ++j) {   // dA[i][j] += do[i] . v[j]   (lower tiles)
      const int t = w + 4 * j;
      if (t < NT_A) {
        const int mi = t / NTM, ni = t % NTM;
        if (ni <= mi)
          mma_tile<T>(dA[j], sDo + mi * 16 * P64, P64, sV + ni * 16 * P64, P64, 64, lane);
      }
    }
#pragma unroll
    for (int j = 0; j < NO; ++j) {   // do h^T and v dh^T, [C x 64 k]
      const int t = w + 4 * j;
      const int mi = t >> 2, ni = t & 3;
      mma_tile<T>(Mqx[j], sDo + mi * 16 * P64, P64, sH + ni * 16 * P64, P64, 64, lane);
      mma_tile<T>(M2[j], sV + mi * 16 * P64, P64, sDh + ni * 16 * P64, P64, 64, lane);
    }
    {   // sum_v h dh for row k = tid/4
      const int kk = tid >> 2, vv = (tid & 3) * 16;
#pragma unroll
      for (int i = 0; i < 16; i += 2) {
        float a0, a1, b0, b1;
        Pair<T>::ld(sH + kk * P64 + vv + i, a0, a1);
        Pair<T>::ld(sDh + kk * P64 + vv + i, b0, b1);
        hdp += a0 * b0 + a1 * b1;
      }
    }
  }
  hdp += __shfl_xor(hdp, 1);
  hdp += __shfl_xor(hdp, 2);
  if ((tid & 3) == 0) sHd[tid >> 2] = hdp;

  // ---- dA (masked, scaled) to LDS, then the chunk contractions ----
#pragma unroll
  for (int j = 0; j < NA; ++j) {
    const int t = w + 4 * j;
    if (t < NT_A) {
      const int mi = t / NTM, ni = t % NTM;
      const int cc = ni * 16 + (lane & 15);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int ro = mi * 16 + 4 * (lane >> 4) + rr;
        sdA[ro * PCP + cc] = from_f32<T>(cc <= ro ? dA[j][rr] * p.scale : 0.f);
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
    // dq_intra[i][k] = sum_j dA[i][j] kg[j][k]      (kg read transposed)
    mma_tile2<T, false, true>(Mqi[j], sdA + mi * 16 * PCP, PCP, sKg + ni * 16, P64, CP, lane);
    // dk_intra[j][k] = sum_i dA[i][j] qg[i][k]      (dA and qg read transposed)
    mma_tile2<T, true, true>(Mk1[j], sdA + mi * 16, PCP, sQg + ni * 16, P64, CP, lane);
  }
  __syncthreads();   // every staged tile is dead; the fp32 exchange aliases them

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

  // ---- epilogue: dq, dk, dg ----
  T* __restrict__ dq = (T*)p.dq;
  T* __restrict__ dk = (T*)p.dk;
  T* __restrict__ dg = (T*)p.dg;
  float dgr0[RPS], dgr1[RPS];
  float s0 = 0.f, s1 = 0.f, dki0 = 0.f, dki1 = 0.f;
  const int gc0 = kb + c_0;
  const bool ok0 = gc0 < K, ok1 = gc0 + 1 < K;
#pragma unroll
  for (int rr = RPS - 1; rr >= 0; --rr) {
    const int row = seg * RPS + rr;
    const float ep0 = gexp<T>(d0[rr]), ep1 = gexp<T>(d1[rr]);
    const float2 xq = *reinterpret_cast<const float2*>(XQ + row * PX + c_0);
    const float2 xk = *reinterpret_cast<const float2*>(XK + row * PX + c_0);
    const float2 xm = *reinterpret_cast<const float2*>(XM + row * PX + c_0);
    const float vq0 = ep0 * xq.x, vq1 = ep1 * xq.y;
    const float vk0 = gdiv<T>(xk.x, d0[rr], ep0), vk1 = gdiv<T>(xk.y, d1[rr], ep1);
    dki0 += k0[rr] * gdiv<T>(xm.x, d0[rr], ep0);
    dki1 += k1[rr] * gdiv<T>(xm.y, d1[rr], ep1);
    s0 += q0[rr] * vq0 - k0[rr] * vk0;
    s1 += q1[rr] * vq1 - k1[rr] * vk1;
    dgr0[rr] = s0;
    dgr1[rr] = s1;
    if (row < len) {
      const long a = baseK + (long)row * rsK + gc0;
      if (VEC && ok1) {
        Pair<T>::st(dq + a, vq0, vq1);
        Pair<T>::st(dk + a, vk0, vk1);
      } else {
        if (ok0) {
          dq[a] = from_f32<T>(vq0);
          dk[a] = from_f32<T>(vk0);
        }
        if (ok1) {
          dq[a + 1] = from_f32<T>(vq1);
          dk[a + 1] = from_f32<T>(vk1);
        }
      }
    }
  }
  sTot[seg * 64 + c_0] = s0;
  sTot[seg * 64 + c_1] = s1;
  sAux[seg * 64 + c_0] = dki0;
  sAux[seg * 64 + c_1] = dki1;
  __syncthreads();
  float o0 = 0.f, o1 = 0.f, dks0 = 0.f, dks1 = 0.f;
#pragma unroll
  for (int s = 0; s < NSEG; ++s) {
    o0 += (s > seg) ? sTot[s * 64 + c_0] : 0.f;
    o1 += (s > seg) ? sTot[s * 64 + c_1] : 0.f;
    dks0 += sAux[s * 64 + c_0];
    dks1 += sAux[s * 64 + c_1];
  }
  const float dgk0 = sGm[c_0] * sHd[c_0] + dks0, dgk1 = sGm[c_1] * sHd[c_1] + dks1;
#pragma unroll
  for (int rr = 0; rr < RPS; ++rr) {
    const int row = seg * RPS + rr;
    if (row < len) {
      const long a = baseK + (long)row * rsK + gc0;
      const float x0 = dgr0[rr] + o0 + dgk0, x1 = dgr1[rr] + o1 + dgk1;
      if (VEC && ok1) {
        Pair<T>::st(dg + a, x0, x1);
      } else {
        if (ok0) dg[a] = from_f32<T>(x0);
        if (ok1) dg[a + 1] = from_f32<T>(x1);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// dv
// ---------------------------------------------------------------------------

template <typename T, int C, bool PRE = false>
struct DvLayout {
  static constexpr int CP = C < 32 ? 32 : C;
  static constexpr int P64 = pitch_of<T>(64), PCP = pitch_of<T>(CP);
  static constexpr int ES = (int)sizeof(T);
  static constexpr int TILE = ((CP * P64 * ES) + 15) / 16 * 16;
  static constexpr int SQ = ((64 * P64 * ES) + 15) / 16 * 16;
  static constexpr int AT = ((CP * PCP * ES) + 15) / 16 * 16;
  // region R: raw q, k, g (per K tile), later A and do | qg, kg | dh' = e^{gamma-r} dh.
  // PRE (no raw tiles, no qg): kg | dh' in the loop, A | do after it, over the same bytes.
  static constexpr int qr = 0, kr = TILE, gr = 2 * TILE;
  static constexpr int a = 0, do_ = AT;
  static constexpr int R = PRE ? 0 : (3 * TILE > AT + TILE) ? 3 * TILE : AT + TILE;
  static constexpr int qg = R, kg = PRE ? 0 : R + TILE, dh = PRE ? TILE : R + 2 * TILE;
  static constexpr int loop_end = dh + SQ, after_end = do_ + TILE;
  static constexpr int base = loop_end > after_end ? loop_end : after_end;
  // bf16 64-row chunks: dv staged as rows (pitch P64) for whole-line stores
  static constexpr bool STG = ES == 2 && C == 64;
  static constexpr int stg = base;
  static constexpr int bytes = base + (STG ? SQ : 0);
};

template <typename T, int C, bool VEC, bool PRE = false>
__global__ __launch_bounds__(256) void chunk_bwd_dv_kernel(BwdArgs p) {
  static_assert(!PRE || C == 64, "the gating workspace holds chunks of 64");
  using Lay = DvLayout<T, C, PRE>;
  constexpr int CP = Lay::CP, P64 = Lay::P64, PCP = Lay::PCP;
  constexpr int EPP = 16 / (int)sizeof(T);
  constexpr int PPT = pieces_per_thread<T, C>(), HPT = pieces_per_thread<T, 64>();
  constexpr int NSEG = 8, RPS = C / NSEG;
  constexpr int NTM = C / 16, NT_A = NTM * NTM, NA = (NT_A + 3) / 4;
  constexpr int NO = NTM;
  extern __shared__ __attribute__((aligned(16))) unsigned char dyn[];
  __shared__ float sTot[NSEG * 64], sFirst[64], sEg[64];
  T* sQr = reinterpret_cast<T*>(dyn + Lay::qr);
  T* sKr = reinterpret_cast<T*>(dyn + Lay::kr);
  T* sGr = reinterpret_cast<T*>(dyn + Lay::gr);
  T* sA = reinterpret_cast<T*>(dyn + Lay::a);
  T* sDo = reinterpret_cast<T*>(dyn + Lay::do_);
  T* sQg = reinterpret_cast<T*>(dyn + Lay::qg);
  T* sKg = reinterpret_cast<T*>(dyn + Lay::kg);
  T* sDh = reinterpret_cast<T*>(dyn + Lay::dh);
  // dv rows staged for whole-line stores (bf16, 64-row chunks, 16-byte aligned rows)
  constexpr bool STG = Lay::STG && VEC;
  T* sStg = reinterpret_cast<T*>(dyn + Lay::stg);

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
  const int vb = vt * 64;
  const int cp = tid & 31, seg = tid >> 5;
  const int c_0 = 2 * cp, c_1 = c_0 + 1;
  // PRE: this (chunk, head)'s gating entry: kg [64][K], A [64][64], factors [3][K]
  const unsigned char* ent =
      PRE ? (const unsigned char*)p.gate_ws + ((long)c * H + hh) * gate_ws_entry(K) : nullptr;
  const T* gkg = reinterpret_cast<const T*>(ent) + 64 * K;
  const T* gA = reinterpret_cast<const T*>(ent) + 2 * 64 * K;
  const float* gpost = reinterpret_cast<const float*>(ent + 2L * 64 * K * 2 + 64 * 64 * 2) + 2 * K;

  // A[i][j] (lower tiles only) and dv^T[v][j], both accumulated over K tiles
  f32x4 Aacc[NA], Dacc[NO];
#pragma unroll
  for (int j = 0; j < NA; ++j) Aacc[j] = zero4();
#pragma unroll
  for (int j = 0; j < NO; ++j) Dacc[j] = zero4();

  uint4 rq[PPT], rk[PPT], rg[PPT], rdh[HPT];
  float reg = 0.f;   // PRE: the 2^{gamma-r} factor of column tid of the K tile
  // K tiles: the next tile's loads are issued once this tile's registers are in LDS, so they
  // arrive under the MFMA work
  auto load_kt = [&](int kt) {
    const int kb = kt * 64;
    if constexpr (PRE) {
      tile_load<T, C, VEC>(rk, gkg, K, C, kb, K, tid);   // rows past the chunk are zeros
      if (tid < 64) reg = kb + tid < K ? gpost[kb + tid] : 0.f;
    } else {
      tile_load<T, C, VEC>(rq, q + baseK, rsK, len, kb, K, tid);
      tile_load<T, C, VEC>(rk, k + baseK, rsK, len, kb, K, tid);
      tile_load<T, C, VEC>(rg, g + baseK, rsK, len, kb, K, tid);
    }
    tile_load<T, 64, VEC>(rdh, dhs + (((long)c * H + hh) * K + kb) * V, V, min(64, K - kb), vb,
                          V, tid);
  };
  if (KT > 0) load_kt(0);
  for (int kt = 0; kt < KT; ++kt) {
    if (kt > 0) __syncthreads();   // readers of the previous K tile are done
    if constexpr (PRE) {
      tile_store<T, C>(sKg, P64, rk, tid);
      if (tid < 64) sEg[tid] = reg;
    } else {
      tile_store<T, C>(sQr, P64, rq, tid);
      tile_store<T, C>(sKr, P64, rk, tid);
      tile_store<T, C>(sGr, P64, rg, tid);
      __syncthreads();
      float d0[RPS], d1[RPS], gam0, gam1, r0, r1;
      pair_cumsum<T, C>(sGr, P64, c_0, seg, sTot, sFirst, d0, d1, gam0, gam1, r0, r1);
#pragma unroll
      for (int rr = 0; rr < RPS; ++rr) {
        const int row = seg * RPS + rr;
        float qa, qb, ka, kb2;
        Pair<T>::ld(sQr + row * P64 + c_0, qa, qb);
        Pair<T>::ld(sKr + row * P64 + c_0, ka, kb2);
        const float e0 = gexp<T>(d0[rr]), e1 = gexp<T>(d1[rr]);
        Pair<T>::st(sQg + row * P64 + c_0, qa * e0, qb * e1);
        Pair<T>::st(sKg + row * P64 + c_0, gdiv<T>(ka, d0[rr], e0),
                    gdiv<T>(kb2, d1[rr], e1));
      }
      if (seg == 0) {
        sEg[c_0] = gexp<T>(gam0 - r0);
        sEg[c_1] = gexp<T>(gam1 - r1);
      }
    }
    __syncthreads();
    // dh' = dh scaled per K row by e^{gamma - r}, so that k_d . dh = kg . dh'
#pragma unroll
    for (int j = 0; j < HPT; ++j) {
      const int pc = tid + 256 * j;
      if (pc < 64 * (64 / EPP)) {
        const int row = pc / (64 / EPP), c8 = (pc % (64 / EPP)) * EPP;
        T vals[EPP];
        __builtin_memcpy(vals, &rdh[j], 16);
        const float f = sEg[row];
        float x[EPP];
#pragma unroll
        for (int e = 0; e < EPP; ++e) x[e] = to_f32(vals[e]) * f;
        store_run<T, EPP>(sDh + row * P64 + c8, x);
      }
    }
    __syncthreads();
    if (kt + 1 < KT) load_kt(kt + 1);
#pragma unroll
    for (int j = 0; j < NA; ++j) {   // A[i][j] += qg[i] . kg[j]
      const int t = w + 4 * j;
      if (!PRE && t < NT_A) {
        const int mi = t / NTM, ni = t % NTM;
        if (ni <= mi)
          mma_tile<T>(Aacc[j], sQg + mi * 16 * P64, P64, sKg + ni * 16 * P64, P64, 64, lane);
      }
    }
#pragma unroll
    for (int j = 0; j < NO; ++j) {   // dv^T[v][j] += sum_k dh'[k][v] kg[j][k]
      const int t = w + 4 * j;
      const int mv = t & 3, nj = t >> 2;
      mma_tile2<T, true, false>(Dacc[j], sDh + mv * 16, P64, sKg + nj * 16 * P64, P64, 64,
                                lane);
    }
  }
  __syncthreads();   // raw and gated tiles are dead: region R takes A and do

  {
    uint4 rdo[PPT];
    tile_load<T, C, VEC>(rdo, dout + baseV, rsV, len, vb, V, tid);
    if constexpr (PRE) {   // A as made by the gating kernel (masked and scaled)
      uint4 ra[PPT];
      tile_load<T, C, VEC>(ra, gA, 64, C, 0, 64, tid);
      tile_store<T, C>(sA, PCP, ra, tid);
    } else {
      for (int i = tid; i < CP * PCP; i += 256) sA[i] = zero_elem<T>();
      if (CP > C)
        for (int i = tid; i < (CP - C) * P64; i += 256) sDo[C * P64 + i] = zero_elem<T>();
      __syncthreads();   // zero fill before the tile writes below
    }
    tile_store<T, C>(sDo, P64, rdo, tid);
  }
#pragma unroll
  for (int j = 0; j < NA; ++j) {
    const int t = w + 4 * j;
    if (!PRE && t < NT_A) {
      const int mi = t / NTM, ni = t % NTM;
      if (ni <= mi) {
        const int cc = ni * 16 + (lane & 15);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int ro = mi * 16 + 4 * (lane >> 4) + rr;
          sA[ro * PCP + cc] = from_f32<T>(cc <= ro ? Aacc[j][rr] * p.scale : 0.f);
        }
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < NO; ++j) {   // dv^T[v][j] += sum_i do[i][v] A[i][j]
    const int t = w + 4 * j;
    const int mv = t & 3, nj = t >> 2;
    mma_tile2<T, true, true>(Dacc[j], sDo + mv * 16, P64, sA + nj * 16, PCP, CP, lane);
    const int jj = nj * 16 + (lane & 15);
    const int vv = vb + mv * 16 + 4 * (lane >> 4);
    if constexpr (STG) {
      *reinterpret_cast<uint2*>(sStg + jj * P64 + mv * 16 + 4 * (lane >> 4)) =
          make_uint2(pack2_bf16(Dacc[j][0], Dacc[j][1]), pack2_bf16(Dacc[j][2], Dacc[j][3]));
    } else if (jj < len) {
      T* dst = dv + baseV + (long)jj * rsV + vv;
      if (VEC && vv + 3 < V) {
        if constexpr (sizeof(T) == 2) {
          *reinterpret_cast<uint2*>(dst) =
              make_uint2(pack2_bf16(Dacc[j][0], Dacc[j][1]), pack2_bf16(Dacc[j][2], Dacc[j][3]));
        } else {
          *reinterpret_cast<float4*>(dst) =
              make_float4(Dacc[j][0], Dacc[j][1], Dacc[j][2], Dacc[j][3]);
        }
      } else {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          if (vv + rr < V) dst[rr] = from_f32<T>(Dacc[j][rr]);
      }
    }
  }
  if constexpr (STG) {
    __syncthreads();   // the tile's rows in LDS
    const bool nt = V % 64 == 0;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int pc = tid + 256 * e, r = pc >> 3, c8 = 8 * (pc & 7);
      if (r < len && vb + c8 < V)
        st16_sel(dv + baseV, ((uint32_t)r * (uint32_t)rsV + (uint32_t)(vb + c8)) * 2u,
                 *reinterpret_cast<const uint4*>(sStg + r * P64 + c8), nt);
    }
  }
}

template <typename T, int C, bool VEC>
static hipError_t launch_bwd(const BwdArgs& p, hipStream_t st, int which) {
  const int KT = (p.K + 63) / 64, VT = (p.V + 63) / 64;
  const long nch = (long)p.si.NC * p.H;
  if (nch == 0) return hipSuccess;
  if (which & 1) {
    using Lay = DqkgLayout<T, C>;
    hipError_t e = hipFuncSetAttribute((const void*)chunk_bwd_dqkg_kernel<T, C, VEC>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, Lay::bytes);
    if (e != hipSuccess) return e;
    ktimer_mark(KT_BWD_DQKG, false, st);
    hipLaunchKernelGGL((chunk_bwd_dqkg_kernel<T, C, VEC>), dim3((unsigned)(nch * KT)),
                       dim3(256), Lay::bytes, st, p);
    ktimer_mark(KT_BWD_DQKG, true, st);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (which & 2) {
    using Lay = DvLayout<T, C>;
    if constexpr (C == 64 && sizeof(T) == 2) {
      if (p.gate_ws) {
        using LP = DvLayout<T, C, true>;
        hipError_t e = hipFuncSetAttribute((const void*)chunk_bwd_dv_kernel<T, C, VEC, true>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           LP::bytes);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL((chunk_bwd_dv_kernel<T, C, VEC, true>), dim3((unsigned)(nch * VT)),
                           dim3(256), LP::bytes, st, p);
        return hipGetLastError();
      }
    }
    hipError_t e = hipFuncSetAttribute((const void*)chunk_bwd_dv_kernel<T, C, VEC>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, Lay::bytes);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((chunk_bwd_dv_kernel<T, C, VEC>), dim3((unsigned)(nch * VT)), dim3(256),
                       Lay::bytes, st, p);
    return hipGetLastError();
  }
  return hipSuccess;
}

template <typename T, int C>
static hipError_t launch_vec(const BwdArgs& p, hipStream_t st, int which) {
  return p.vec ? launch_bwd<T, C, true>(p, st, which) : launch_bwd<T, C, false>(p, st, which);
}

template <typename T>
static hipError_t dispatch_bwd(const BwdArgs& p, hipStream_t st, int which) {
  switch (p.si.C) {
    case 16: return launch_vec<T, 16>(p, st, which);
    case 32: return launch_vec<T, 32>(p, st, which);
    case 64: return launch_vec<T, 64>(p, st, which);
    default: return hipErrorInvalidValue;
  }
}

hipError_t run_chunk_bwd(const BwdArgs& p, int dtype, hipStream_t st, int which) {
  if (dtype == DT_BF16) return dispatch_bwd<bf16>(p, st, which);
  if (dtype == DT_F32) return dispatch_bwd<float>(p, st, which);
  return hipErrorInvalidValue;
}

}  // namespace tops
