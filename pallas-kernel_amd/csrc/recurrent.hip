// Fused recurrent GLA, forward and backward, on one element-wise scan kernel (fp32 VALU,
// no MFMA: the state update is a rank-1 outer product per token).
// Reference: tops/ops/gla/fused_recurrent.py — forward _fused_recurrent_gla_fwd_kernel
// :139-227 (launcher :235-371, jnp ref :17-132); backward _fused_recurrent_gla_bwd_kernel
// :495-624 (launcher :626-795), gate gradients _compute_gate_grads :798-876, entry :879-956.
//
// The scan, over an [R x C] fp32 state per (sequence, head), processed forward or backward
// in time:
//   S <- S (.) (e^{ga[r]} e^{gb[c]}) + (sa a[r]) b[c],   out[c] = so sum_r o[r] S[r][c]
//   forward : S = h    [K x V], a = k, b = v, o = q (so = scale); out = o, final state ht
//   bwd 1 dq: S = h^T  [V x K], a = v, b = k, o = do (so = scale), forward's direction
//   bwd 2 dk: S = dh^T [V x K], a = do (sa = scale), b = q, o = v, opposite direction
//   bwd 3 dv: S = dh   [K x V], a = q (sa = scale), b = do, o = k, opposite direction
// Each output reduces over the state's rows, which never leave the block, so no output
// needs a reduction across blocks. In the backward scans the gate of a step is applied when
// the next step is processed (dh_{t-1} = G_t (.) dh_t); scan 3 applies the last one before
// storing dh0. The gate gradients follow from the reference's identity (:798-876)
//   dgk_t = sum_{s at or after t in scan order} (q_s dq_s - k_s dk_s) + sum_v dht (.) h_T
//   dgv_t = sum_{s ...} (o_s do_s - v_s dv_s)                          + sum_k dht (.) h_T
// and scans 2 and 3 visit the steps in exactly that order, so they accumulate the sums as
// they emit dk and dv (the epilogue below); h_T is the final state of scan 1.
//
// Block = (sequence, head, tile of CB columns), 512 threads (8 waves). A thread holds an
// RPT x 4 sub-tile of the state: lane l = rgl * NCG + cg owns columns cg*4 .. cg*4+3 and
// row group rgl of its wave (RGW = 64 / NCG row groups per wave). Per step a thread reads
// its rows' a, gate, o and its columns' b, gate from LDS (staged TB steps at a time, the
// next stage's global loads in flight while the current one computes), updates 4 * RPT
// state values and folds its 4 partial outputs across the wave's row groups with
// v_permlane32_swap / v_permlane16_swap (and a DPP row rotate for 32-column tiles): the
// lane ends with one column's sum, and the 8 waves' sums meet in LDS.
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

namespace tops {

namespace {

constexpr int RNT = 512;  // threads per block
constexpr int RNW = RNT / 64;

template <int NCG, int RPT>
struct RecCfg {
  static constexpr int CB = NCG * 4;                 // columns per block
  static constexpr int RGW = 64 / NCG;               // row groups per wave
  static constexpr int NRG = RNW * RGW;              // row groups per block
  static constexpr int RP = NRG * RPT;               // rows covered
  static constexpr int TB = 16;                      // steps per stage
};

__device__ __forceinline__ long st_off(int r, int c, int R, int C, bool trans) {
  return trans ? (long)c * R + r : (long)r * C + c;
}

__device__ __forceinline__ float ror8(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xf, 0xf,
                                                    false));
}

// Sum of x[0..3] (columns cg*4 + j of this lane) over the wave's row groups. Lane l ends
// with the sum for column (l & (NCG - 1)) * 4 + (l >> 4); for NCG = 8, lanes with bit 3
// set hold a duplicate.
template <int NCG>
__device__ __forceinline__ float wave_colsum(float (&x)[4]) {
  if (NCG == 8) {
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j] += ror8(x[j]);
  }
  const auto p0 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x[0]),
                                                   __float_as_uint(x[2]), false, false);
  const auto p1 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x[1]),
                                                   __float_as_uint(x[3]), false, false);
  const float u0 = __uint_as_float(p0[0]) + __uint_as_float(p0[1]);
  const float u1 = __uint_as_float(p1[0]) + __uint_as_float(p1[1]);
  const auto p2 = __builtin_amdgcn_permlane16_swap(__float_as_uint(u0), __float_as_uint(u1),
                                                   false, false);
  return __uint_as_float(p2[0]) + __uint_as_float(p2[1]);
}

template <int NCG>
__device__ __forceinline__ int lane_col(int l) { return (l & (NCG - 1)) * 4 + (l >> 4); }
template <int NCG>
__device__ __forceinline__ bool lane_writes(int l) { return NCG == 16 || (l & 8) == 0; }

// N consecutive elements (N * sizeof(T) bytes aligned) to fp32, in one load.
template <typename T, int N>
__device__ __forceinline__ void ld_vec(const T* p, float (&x)[N]);
template <>
__device__ __forceinline__ void ld_vec<float, 1>(const float* p, float (&x)[1]) { x[0] = *p; }
template <>
__device__ __forceinline__ void ld_vec<float, 2>(const float* p, float (&x)[2]) {
  const float2 v = *reinterpret_cast<const float2*>(p);
  x[0] = v.x; x[1] = v.y;
}
template <>
__device__ __forceinline__ void ld_vec<float, 4>(const float* p, float (&x)[4]) {
  const float4 v = *reinterpret_cast<const float4*>(p);
  x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
}
template <>
__device__ __forceinline__ void ld_vec<float, 8>(const float* p, float (&x)[8]) {
  const float4 v = *reinterpret_cast<const float4*>(p);
  const float4 u = *reinterpret_cast<const float4*>(p + 4);
  x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w; x[4] = u.x; x[5] = u.y; x[6] = u.z; x[7] = u.w;
}
__device__ __forceinline__ void bf2(uint32_t u, float& lo, float& hi) {
  lo = __uint_as_float(u << 16);
  hi = __uint_as_float(u & 0xffff0000u);
}
template <>
__device__ __forceinline__ void ld_vec<bf16, 1>(const bf16* p, float (&x)[1]) {
  x[0] = to_f32(*p);
}
template <>
__device__ __forceinline__ void ld_vec<bf16, 2>(const bf16* p, float (&x)[2]) {
  bf2(*reinterpret_cast<const uint32_t*>(p), x[0], x[1]);
}
template <>
__device__ __forceinline__ void ld_vec<bf16, 4>(const bf16* p, float (&x)[4]) {
  const uint2 u = *reinterpret_cast<const uint2*>(p);
  bf2(u.x, x[0], x[1]);
  bf2(u.y, x[2], x[3]);
}
template <>
__device__ __forceinline__ void ld_vec<bf16, 8>(const bf16* p, float (&x)[8]) {
  const uint4 u = *reinterpret_cast<const uint4*>(p);
  bf2(u.x, x[0], x[1]);
  bf2(u.y, x[2], x[3]);
  bf2(u.z, x[4], x[5]);
  bf2(u.w, x[6], x[7]);
}

// N consecutive floats to LDS (N * 4 bytes aligned).
template <int N>
__device__ __forceinline__ void st_vec(float* p, const float (&x)[N]) {
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int i = 0; i < N; i += 4)
      *reinterpret_cast<float4*>(p + i) = make_float4(x[i], x[i + 1], x[i + 2], x[i + 3]);
  } else if constexpr (N == 2) {
    *reinterpret_cast<float2*>(p) = make_float2(x[0], x[1]);
  } else {
    p[0] = x[0];
  }
}

template <typename TO>
__device__ __forceinline__ void put(void* p, long i, float x) {
  static_cast<TO*>(p)[i] = from_f32<TO>(x);
}

}  // namespace

// Whether (sequence seq, head hh) is flagged: the pair's flags (one per segment or chunk and
// V tile) read by the lanes of every wave at once, so that an unflagged block leaves after a
// few loads. Uniform over the block.
__device__ __forceinline__ bool pair_flagged(const GateFlags& f, int seq, int hh, int H) {
  long s0 = (long)seq * f.ns;
  int n = f.ns * f.vt;
  if (f.co) {   // per-chunk flags of varlen sequences
    s0 = f.co[seq];
    n = (f.co[seq + 1] - f.co[seq]) * f.vt;
  }
  int x = 0;
  for (int i = (int)(threadIdx.x & 63); i < n; i += 64)
    x |= f.p[((s0 + i / f.vt) * H + hh) * f.vt + i % f.vt];
  return __ballot(x != 0) != 0ull;
}

// One unit L = (sequence, head) x NCT + column tile of a scan, run by the whole block. The
// LDS arrays are function-scope statics: units that one block runs in turn share them, with
// a barrier between.
// Elements as stored, for loads whose conversion waits until the data is needed: ld_bits
// one element (bf16 in the low half of the word), ld_raw N aligned elements in one load
// (raw_words: bf16 two a word, element 2i in the low half of word i; N == 1: the low half),
// and their fp32 values (bits_f32, cvt_raw).
__device__ __forceinline__ uint32_t ld_bits(const float* p) {
  return *reinterpret_cast<const uint32_t*>(p);
}
__device__ __forceinline__ uint32_t ld_bits(const bf16* p) {
  return *reinterpret_cast<const uint16_t*>(p);
}
template <typename T>
__device__ __forceinline__ float bits_f32(uint32_t x) {
  return sizeof(T) == 4 ? __uint_as_float(x) : __uint_as_float(x << 16);
}
template <typename T, int N>
constexpr int raw_words() { return sizeof(T) == 4 ? N : (N + 1) / 2; }
template <typename T, int N>
__device__ __forceinline__ void ld_raw(const T* p, uint32_t (&x)[raw_words<T, N>()]) {
  constexpr int W = raw_words<T, N>();
  if constexpr (sizeof(T) == 2 && N == 1) {
    x[0] = *reinterpret_cast<const uint16_t*>(p);
  } else if constexpr (W == 1) {
    x[0] = *reinterpret_cast<const uint32_t*>(p);
  } else if constexpr (W == 2) {
    const uint2 u = *reinterpret_cast<const uint2*>(p);
    x[0] = u.x; x[1] = u.y;
  } else {
    static_assert(W % 4 == 0, "words");
#pragma unroll
    for (int i = 0; i < W; i += 4) {
      const uint4 u = reinterpret_cast<const uint4*>(p)[i / 4];
      x[i] = u.x; x[i + 1] = u.y; x[i + 2] = u.z; x[i + 3] = u.w;
    }
  }
}
template <typename T, int N>
__device__ __forceinline__ void cvt_raw(const uint32_t (&x)[raw_words<T, N>()], float (&y)[N]) {
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int i = 0; i < N; ++i) y[i] = __uint_as_float(x[i]);
  } else if constexpr (N == 1) {
    y[0] = __uint_as_float(x[0] << 16);
  } else {
#pragma unroll
    for (int i = 0; i < N / 2; ++i) bf2(x[i], y[2 * i], y[2 * i + 1]);
  }
}

template <typename T, typename TO, int NCG, int RPT>
__device__ __forceinline__ void rec_scan_unit(const RecScanArgs& p, const int L) {
  using Cf = RecCfg<NCG, RPT>;
  constexpr int CB = Cf::CB, RP = Cf::RP, TB = Cf::TB, RGW = Cf::RGW;
  static_assert(RPT == 2 || RPT % 4 == 0, "rows are read as float2 / float4");
  __shared__ __attribute__((aligned(16))) float sA[TB * RP];   // sa * a
  __shared__ __attribute__((aligned(16))) float sGR[TB * RP];  // e^{ga} of the gate step
  __shared__ __attribute__((aligned(16))) float sOR[TB * RP];  // so * o
  __shared__ __attribute__((aligned(16))) float sB[TB * CB];
  __shared__ __attribute__((aligned(16))) float sGC[TB * CB];
  __shared__ float sXD[TB * CB];  // epilogue: gx * gxf
  __shared__ float sY[TB * CB];   // epilogue: gy
  __shared__ float sO[RNW * TB * CB];

  const T* __restrict__ a = (const T*)p.a;
  const T* __restrict__ ga = (const T*)p.ga;
  const T* __restrict__ orow = (const T*)p.o;
  const T* __restrict__ b = (const T*)p.b;
  const T* __restrict__ gb = (const T*)p.gb;
  const T* __restrict__ gx = (const T*)p.gx;
  const T* __restrict__ gy = (const T*)p.gy;

  const int H = p.H, R = p.R, C = p.C;
  const int NCT = (C + CB - 1) / CB;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ct = L % NCT;
  const int sh = L / NCT;
  const int seq = sh / H, hh = sh % H;
  int bos, eos;
  seq_bounds(p.si, seq, bos, eos);
  const int n = eos - bos;
  const int cg = lane % NCG;
  const int rg = w * RGW + lane / NCG;
  const int r0 = rg * RPT;
  const int cbase = ct * CB;
  const int c0 = cbase + cg * 4;
  const bool trans = p.s_trans != 0;
  const long sbase = ((long)seq * H + hh) * R * C;
  const bool has_ga = ga != nullptr, has_gb = gb != nullptr;
  const bool grad = p.dg != nullptr;
  const long rsR = (long)H * R, rsC = (long)H * C;
  auto tok = [&](int i) { return p.dir ? eos - 1 - i : bos + i; };

  // State element (r0 + j, c0 + i), clamped into range: unconditional loads, out-of-range
  // values dropped by a select (no per-element branches).
  auto st_at = [&](int j, int i) {
    return sbase + st_off(min(r0 + j, R - 1), min(c0 + i, C - 1), R, C, trans);
  };
  auto ok = [&](int j, int i) { return r0 + j < R && c0 + i < C; };
  float S[RPT][4];
#pragma unroll
  for (int j = 0; j < RPT; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) S[j][i] = 0.f;
  // states stored [R][C] with whole 16-byte column groups (C % 4 == 0, 16-byte aligned
  // arrays): a thread's 4 columns of a row are one float4 (uniform)
  const bool vst = !trans && (C & 3) == 0 &&
                   (((uintptr_t)p.s0 | (uintptr_t)p.sN | (uintptr_t)p.hfin) & 15) == 0;
  auto st_row = [&](int j) {   // the thread's row j, columns c0.. (clamped into the state)
    return sbase + (long)min(r0 + j, R - 1) * C + min(c0, C - 4);
  };
  if (p.s0) {
    if (vst) {
#pragma unroll
      for (int j = 0; j < RPT; ++j) {
        const float4 x = *reinterpret_cast<const float4*>(p.s0 + st_row(j));
        S[j][0] = ok(j, 0) ? x.x : 0.f;
        S[j][1] = ok(j, 1) ? x.y : 0.f;
        S[j][2] = ok(j, 2) ? x.z : 0.f;
        S[j][3] = ok(j, 3) ? x.w : 0.f;
      }
    } else {
#pragma unroll
      for (int j = 0; j < RPT; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float x = p.s0[st_at(j, i)];
          S[j][i] = ok(j, i) ? x : 0.f;
        }
    }
  }

  // Epilogue constant: sum_r s0 (.) hfin over the rows of each column.
  __shared__ float sCorr[CB];
  if (grad && tid < CB) sCorr[tid] = 0.f;
  if (grad && p.s0 && p.hfin) {
    float x[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < RPT; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] += S[j][i] * p.hfin[st_at(j, i)];  // S = 0 outside
    const float cs = wave_colsum<NCG>(x);
    if (lane_writes<NCG>(lane)) sO[w * CB + lane_col<NCG>(lane)] = cs;
    __syncthreads();
    if (tid < CB) {
      float corr = 0.f;
      for (int ww = 0; ww < RNW; ++ww) corr += sO[ww * CB + tid];
      sCorr[tid] = corr;
    }
  }
  float run[CB * 16 / RNT] = {};  // epilogue carries of this thread's columns

  // Staging: wave w loads steps w and w + 8 of a stage, so each load has a wave-uniform
  // token; lane l loads rows l*RL .. l*RL+RL-1 (one vector load per array when the rows are
  // whole and aligned) and column cbase + l of the column side. issue() only issues the
  // loads, into registers as stored; commit() converts, masks and stores them to LDS a stage
  // later (converted or masked at issue, every stage would wait there for its own loads).
  constexpr int RL = RP / 64;     // rows per lane
  constexpr int SPW = TB / RNW;   // steps per wave per stage
  static_assert(RL * 64 == RP && SPW * RNW == TB, "staging map");
  const int row0 = lane * RL;
  const bool vrow = row0 + RL <= R && R % RL == 0 &&
                    (((uintptr_t)a | (uintptr_t)orow | (uintptr_t)ga) % (RL * sizeof(T))) == 0;
  // a row piece as stored (bf16 two a word): vrow, RL elements in one load; else element by
  // element, rows clamped into the state (that path packs the halves, so it waits there)
  constexpr int RW = sizeof(T) == 4 ? RL : (RL + 1) / 2;   // words of a row piece
  auto ld_rows = [&](const T* src, long off, uint32_t (&x)[RW]) {
    if (vrow) {
      ld_raw<T, RL>(src + off + row0, x);
    } else if constexpr (sizeof(T) == 4) {
#pragma unroll
      for (int i = 0; i < RL; ++i) x[i] = ld_bits(src + off + min(row0 + i, R - 1));
    } else {
#pragma unroll
      for (int i = 0; i < RW; ++i) {
        const uint32_t lo = ld_bits(src + off + min(row0 + 2 * i, R - 1));
        const uint32_t hi = 2 * i + 1 < RL ? ld_bits(src + off + min(row0 + 2 * i + 1, R - 1)) : 0u;
        x[i] = lo | (hi << 16);
      }
    }
  };
  auto cvt_rows = [&](const uint32_t (&x)[RW], float (&y)[RL]) {
    cvt_raw<T, RL>(x, y);
    if (!vrow) {
#pragma unroll
      for (int i = 0; i < RL; ++i) y[i] = row0 + i < R ? y[i] : 0.f;
    }
  };
  uint32_t ua[SPW][RW], uo[SPW][RW], ug[SPW][RW];   // row side, as stored
  uint32_t ub[SPW], ugc[SPW];                      // column side, as stored
  float pxd[SPW], py[SPW];   // gate-gradient inputs (backward scans): converted at issue
  auto issue = [&](int b0) {
#pragma unroll
    for (int k = 0; k < SPW; ++k) {
      const int s = w + k * RNW;   // wave-uniform
      const int gi = b0 + s - p.shift;
      const int t = tok(min(b0 + s, n - 1)), tg = tok(max(min(gi, n - 1), 0));
      const long ro = (long)t * rsR + (long)hh * R, rgo = (long)tg * rsR + (long)hh * R;
      ld_rows(a, ro, ua[k]);
      ld_rows(orow, ro, uo[k]);
      if (has_ga) ld_rows(ga, rgo, ug[k]);
      const int c = cbase + lane;
      const long co = (long)t * rsC + (long)hh * C + min(c, C - 1);
      ub[k] = ld_bits(b + co);
      if (has_gb) ugc[k] = ld_bits(gb + (long)tg * rsC + (long)hh * C + min(c, C - 1));
      if (grad) {
        float xf = p.gxf_f32 ? static_cast<const float*>(p.gxf)[co]
                             : to_f32(static_cast<const TO*>(p.gxf)[co]);
        if (p.gxf_lo) xf += to_f32(static_cast<const TO*>(p.gxf_lo)[co]);
        pxd[k] = to_f32(gx[co]) * xf;
        py[k] = to_f32(gy[co]);
      }
    }
  };
  auto commit = [&](int b0) {
    const int nb = min(TB, n - b0);
#pragma unroll
    for (int k = 0; k < SPW; ++k) {
      const int s = w + k * RNW;
      const bool in = s < nb;
      const bool gin = in && b0 + s - p.shift >= 0;
      float xa[RL], xo[RL], xg[RL];
      cvt_rows(ua[k], xa);
      cvt_rows(uo[k], xo);
      if (has_ga) cvt_rows(ug[k], xg);
#pragma unroll
      for (int i = 0; i < RL; ++i) {
        xa[i] = in ? p.sa * xa[i] : 0.f;
        xo[i] = in ? p.so * xo[i] : 0.f;
        xg[i] = (has_ga && gin) ? gexp<T>(xg[i]) : 1.f;   // absent gate: factor 1
      }
      st_vec<RL>(sA + s * RP + row0, xa);
      st_vec<RL>(sOR + s * RP + row0, xo);
      st_vec<RL>(sGR + s * RP + row0, xg);
      if (lane < CB) {
        const bool cin = in && cbase + lane < C;
        sB[s * CB + lane] = cin ? bits_f32<T>(ub[k]) : 0.f;
        sGC[s * CB + lane] = (has_gb && cin && gin) ? gexp<T>(bits_f32<T>(ugc[k])) : 1.f;
        if (grad) {
          sXD[s * CB + lane] = cin ? pxd[k] : 0.f;
          sY[s * CB + lane] = cin ? py[k] : 0.f;
        }
      }
    }
  };

  if (n > 0) issue(0);
  for (int b0 = 0; b0 < n; b0 += TB) {
    const int nb = min(TB, n - b0);
    __syncthreads();  // the previous stage's reads of the staged arrays and sO are done
    commit(b0);
    __syncthreads();
    if (b0 + TB < n) issue(b0 + TB);
    // The column gate's presence is uniform: one copy of the step loop for each case.
    // One step's LDS operands.
    struct StepIn {
      float a[RPT], g[RPT], o[RPT], b[4], gc[4];
    };
    auto load_step = [&](auto gac, auto gbc, int s, StepIn& in) {
      constexpr bool GA = decltype(gac)::value, GB = decltype(gbc)::value;
      const float4 bq = *reinterpret_cast<const float4*>(sB + s * CB + cg * 4);
      in.b[0] = bq.x; in.b[1] = bq.y; in.b[2] = bq.z; in.b[3] = bq.w;
      if (GB) {
        const float4 gq = *reinterpret_cast<const float4*>(sGC + s * CB + cg * 4);
        in.gc[0] = gq.x; in.gc[1] = gq.y; in.gc[2] = gq.z; in.gc[3] = gq.w;
      }
      const float* ra = sA + s * RP + r0;
      const float* rgp = sGR + s * RP + r0;
      const float* ro = sOR + s * RP + r0;
      if (RPT == 2) {
        const float2 a2 = *reinterpret_cast<const float2*>(ra);
        const float2 g2 = GA ? *reinterpret_cast<const float2*>(rgp) : make_float2(1.f, 1.f);
        const float2 o2 = *reinterpret_cast<const float2*>(ro);
        in.a[0] = a2.x; in.a[1] = a2.y; in.g[0] = g2.x; in.g[1] = g2.y;
        in.o[0] = o2.x; in.o[1] = o2.y;
      } else {
#pragma unroll
        for (int j0 = 0; j0 < RPT; j0 += 4) {
          const float4 a4 = *reinterpret_cast<const float4*>(ra + j0);
          const float4 g4 = GA ? *reinterpret_cast<const float4*>(rgp + j0)
                               : make_float4(1.f, 1.f, 1.f, 1.f);
          const float4 o4 = *reinterpret_cast<const float4*>(ro + j0);
          in.a[j0] = a4.x; in.a[j0 + 1] = a4.y; in.a[j0 + 2] = a4.z; in.a[j0 + 3] = a4.w;
          in.g[j0] = g4.x; in.g[j0 + 1] = g4.y; in.g[j0 + 2] = g4.z; in.g[j0 + 3] = g4.w;
          in.o[j0] = o4.x; in.o[j0 + 1] = o4.y; in.o[j0 + 2] = o4.z; in.o[j0 + 3] = o4.w;
        }
      }
    };
    auto step = [&](auto gac, auto gbc, int s, const StepIn& in) {
      constexpr bool GA = decltype(gac)::value, GB = decltype(gbc)::value;
      float x[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < RPT; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // in place (scale, then accumulate): no copies of the state registers
          if (GA && GB)
            S[j][i] *= in.g[j] * in.gc[i];
          else if (GA)
            S[j][i] *= in.g[j];
          else if (GB)
            S[j][i] *= in.gc[i];
          S[j][i] = fmaf(in.a[j], in.b[i], S[j][i]);
          x[i] = fmaf(in.o[j], S[j][i], x[i]);
        }
      const float cs = wave_colsum<NCG>(x);
      if (lane_writes<NCG>(lane)) sO[(w * TB + s) * CB + lane_col<NCG>(lane)] = cs;
    };
    // Which gates exist is uniform: one copy of the step loop for each case. With 8 state
    // rows a thread (256 VGPRs), a step's LDS operands are read while the step before it
    // computes (two register sets, two steps a trip; the read past the stage's last step is
    // of a staged row that is not used); the 4-wave variants have no registers for that.
    auto steps = [&](auto gac, auto gbc) {
      if constexpr (RPT < 8) {
#pragma unroll 1
        for (int s = 0; s < nb; ++s) {
          StepIn in;
          load_step(gac, gbc, s, in);
          step(gac, gbc, s, in);
        }
        return;
      }
      StepIn x0, x1;
      load_step(gac, gbc, 0, x0);
#pragma unroll 1
      for (int s = 0; s < nb; s += 2) {
        load_step(gac, gbc, min(s + 1, TB - 1), x1);
        __builtin_amdgcn_sched_barrier(0);   // the reads issue before the step's products
        step(gac, gbc, s, x0);
        if (s + 1 >= nb) break;
        load_step(gac, gbc, min(s + 2, TB - 1), x0);
        __builtin_amdgcn_sched_barrier(0);
        step(gac, gbc, s + 1, x1);
      }
    };
    using yes = std::integral_constant<bool, true>;
    using no = std::integral_constant<bool, false>;
    if (has_ga && has_gb)
      steps(yes(), yes());
    else if (has_ga)
      steps(yes(), no());
    else if (has_gb)
      steps(no(), yes());
    else
      steps(no(), no());
    __syncthreads();
    // Outputs: sum of the 8 waves' column sums, stored coalesced (columns fastest).
#pragma unroll 1
    for (int i = tid; i < TB * CB; i += RNT) {
      const int s = i / CB, c = i % CB;
      if (s < nb && cbase + c < C) {
        float val = 0.f;
#pragma unroll
        for (int ww = 0; ww < RNW; ++ww) val += sO[(ww * TB + s) * CB + c];
        const long oi = (long)tok(b0 + s) * rsC + (long)hh * C + cbase + c;
        put<TO>(p.out, oi, val);
        if constexpr (!std::is_same<TO, float>::value)
          if (p.out_lo) put<TO>(p.out_lo, oi, val - to_f32(from_f32<TO>(val)));
        if (grad) sXD[i] -= sY[i] * val;   // this step's term of the gate gradient
      } else if (grad) {
        sXD[i] = 0.f;
      }
    }
    if (grad) {
      // Running sum in scan order (the gate gradient's suffix, or prefix, sum): 16 lanes
      // per column scan the stage's 16 steps; the carry moves on to the next stage.
      __syncthreads();
      static_assert(TB == 16, "one 16-lane row per column and stage");
#pragma unroll
      for (int e = 0; e < CB * 16 / RNT; ++e) {
        const int c = (tid >> 4) + e * (RNT / 16), s = tid & 15;
        float d = sXD[s * CB + c];
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) {
          const float y = __shfl_up(d, o, 16);
          if (s >= o) d += y;
        }
        sXD[s * CB + c] = run[e] + d + sCorr[c];
        run[e] += __shfl(d, 15, 16);
      }
      __syncthreads();
#pragma unroll 1
      for (int i = tid; i < nb * CB; i += RNT) {
        const int s = i / CB, c = i % CB;
        if (cbase + c < C)
          put<TO>(p.dg, (long)tok(b0 + s) * rsC + (long)hh * C + cbase + c, sXD[i]);
      }
    }
  }

  if (p.sN) {
    if (p.final_gate && n > 0) {
      const int t = tok(n - 1);
      float gcol[4], grow[RPT];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        gcol[i] = has_gb ? gexp<T>(to_f32(gb[(long)t * rsC + (long)hh * C + min(c0 + i, C - 1)]))
                         : 1.f;
#pragma unroll
      for (int j = 0; j < RPT; ++j)
        grow[j] = has_ga ? gexp<T>(to_f32(ga[(long)t * rsR + (long)hh * R + min(r0 + j, R - 1)]))
                         : 1.f;
#pragma unroll
      for (int j = 0; j < RPT; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) S[j][i] *= grow[j] * gcol[i];
    }
    if (vst) {
#pragma unroll
      for (int j = 0; j < RPT; ++j)
        if (ok(j, 0))   // C % 4 == 0: the thread's 4 columns are all in or all out
          *reinterpret_cast<float4*>(p.sN + st_row(j)) =
              make_float4(S[j][0], S[j][1], S[j][2], S[j][3]);
    } else {
#pragma unroll
      for (int j = 0; j < RPT; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (ok(j, i)) p.sN[st_at(j, i)] = S[j][i];
    }
  }
}

// 64-column tiles of up to 4 state rows per thread: held to 128 VGPRs (4 waves per SIMD), so
// that two blocks share a CU
// (the decode shapes, hundreds of short scans, are bound by how many run at once).
template <typename T, typename TO, int NCG, int RPT>
__global__ __launch_bounds__(RNT, (RPT <= 4 && NCG == 16) ? 4 : 1) void rec_scan_kernel(RecScanArgs p) {
  const int L = xcd_remap(blockIdx.x, gridDim.x);
  if (p.flags.p) {   // fallback launch: only the (sequence, head) pairs a block flagged
    const int NCT = (p.C + NCG * 4 - 1) / (NCG * 4);
    if (!pair_flagged(p.flags, L / NCT / p.H, (L / NCT) % p.H, p.H)) return;
  }
  rec_scan_unit<T, TO, NCG, RPT>(p, L);
}

// Every column tile of one (sequence, head) pair of a scan, in turn.
template <typename T, typename TO, int NCG, int RPT>
__device__ __forceinline__ void rec_scan_pair(const RecScanArgs& p, int pair) {
  const int NCT = (p.C + NCG * 4 - 1) / (NCG * 4);
#pragma unroll 1
  for (int ct = 0; ct < NCT; ++ct) {
    rec_scan_unit<T, TO, NCG, RPT>(p, pair * NCT + ct);
    __syncthreads();   // LDS reuse; the next scan's reads of this one's global writes
  }
}

// The backward's gate-range fallback in one launch: block = (sequence, head) pair; a
// flagged pair runs the three scans of run_recurrent_bwd in order, each over all of its
// column tiles (the second reads the first's dq and final state, written by this block);
// an unflagged one leaves after reading its flags. Three launches with a block per column
// tile cost about 4 us each even when nothing is flagged.
template <typename T, typename TO, int NCG, int RPT>
__global__ __launch_bounds__(RNT) void rec_bwd_fallback_kernel(RecScanArgs s1, RecScanArgs s2,
                                                               RecScanArgs s3) {
  const int pair = xcd_remap(blockIdx.x, gridDim.x);
  if (!pair_flagged(s1.flags, pair / s1.H, pair % s1.H, s1.H)) return;
  // each scan named directly (an array of pointers to the arguments would copy them to
  // scratch memory, whose set-up slows this launch and the next even when nothing is flagged)
  rec_scan_pair<T, TO, NCG, RPT>(s1, pair);
  rec_scan_pair<T, TO, NCG, RPT>(s2, pair);
  rec_scan_pair<T, TO, NCG, RPT>(s3, pair);
}

// ---------------------------------------------------------------------------
// Short forward scans (decode shapes: sequences of a few tokens, many sequences and heads):
// one 256-thread block per (sequence, head, 64-column tile). A thread holds RPT rows x 4
// columns of the state in registers (16 row groups: the four 16-lane rows of a wave, then the
// four waves); each step's a, o and row-gate values and its b and column-gate values are read
// straight from global memory, the next step's while the current one computes; a step's four
// column sums are folded over the wave's row groups (permlane swaps) and parked in LDS, and
// the four waves' sums of up to 16 steps are added and stored once per 16 steps. 16 KB of LDS
// and no staging: several blocks share a CU, where the staged scan (74 KB, 512 threads) fits
// two -- for hundreds of short scans, how many run at once is what sets the time.
// ---------------------------------------------------------------------------
// N consecutive elements of T kept as stored: 32-bit words (bf16: element 2i in the low half
// of word i, 2i + 1 in the high half; float: one element a word).
template <typename T, int N>
struct Raw {
  static constexpr int W = N * (int)sizeof(T) / 4;
  static_assert(W * 4 == N * (int)sizeof(T) && (W == 1 || W == 2 || W % 4 == 0), "words");
  uint32_t w[W];
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int i = 0; i < W; ++i) w[i] = 0u;
  }
  // N elements at p (aligned to N elements)
  __device__ __forceinline__ void ld(const T* p) {
    if constexpr (W == 1) {
      w[0] = *reinterpret_cast<const uint32_t*>(p);
    } else if constexpr (W == 2) {
      const uint2 u = *reinterpret_cast<const uint2*>(p);
      w[0] = u.x; w[1] = u.y;
    } else {
#pragma unroll
      for (int i = 0; i < W; i += 4) {
        const uint4 u = reinterpret_cast<const uint4*>(p)[i / 4];
        w[i] = u.x; w[i + 1] = u.y; w[i + 2] = u.z; w[i + 3] = u.w;
      }
    }
  }
  // elements base[i0 + e] for i0 + e < n, zero past n (addresses clamped to n - 1)
  __device__ __forceinline__ void ld_masked(const T* base, int i0, int n) {
    if constexpr (sizeof(T) == 4) {
#pragma unroll
      for (int e = 0; e < N; ++e) {
        const uint32_t x = reinterpret_cast<const uint32_t*>(base)[min(i0 + e, n - 1)];
        w[e] = i0 + e < n ? x : 0u;
      }
    } else {
#pragma unroll
      for (int i = 0; i < W; ++i) {
        const uint32_t lo = reinterpret_cast<const uint16_t*>(base)[min(i0 + 2 * i, n - 1)];
        const uint32_t hi = reinterpret_cast<const uint16_t*>(base)[min(i0 + 2 * i + 1, n - 1)];
        w[i] = (i0 + 2 * i < n ? lo : 0u) | ((i0 + 2 * i + 1 < n ? hi : 0u) << 16);
      }
    }
  }
  __device__ __forceinline__ void unpack(float (&x)[N]) const {
    if constexpr (sizeof(T) == 4) {
#pragma unroll
      for (int e = 0; e < N; ++e) x[e] = __uint_as_float(w[e]);
    } else {
#pragma unroll
      for (int i = 0; i < W; ++i) bf2(w[i], x[2 * i], x[2 * i + 1]);
    }
  }
};

constexpr int SNT = 256, SNW = SNT / 64, STB = 16;

template <typename T, typename TO, int RPT>
__global__ __launch_bounds__(SNT, 4) void rec_short_kernel(RecScanArgs p) {
  __shared__ float sO[SNW * STB * 64];
  const int H = p.H, R = p.R, C = p.C;
  const int NCT = (C + 63) >> 6;
  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int ct = L % NCT, sh = L / NCT;
  const int seq = sh / H, hh = sh % H;
  int bos, eos;
  seq_bounds(p.si, seq, bos, eos);
  const int n = eos - bos;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r0 = (w * 4 + (lane >> 4)) * RPT, c0 = ct * 64 + (lane & 15) * 4;
  const T* __restrict__ a = (const T*)p.a;
  const T* __restrict__ orow = (const T*)p.o;
  const T* __restrict__ ga = (const T*)p.ga;
  const T* __restrict__ b = (const T*)p.b;
  const T* __restrict__ gb = (const T*)p.gb;
  const bool has_ga = ga != nullptr, has_gb = gb != nullptr;
  const long rsR = (long)H * R, rsC = (long)H * C;
  const long sbase = ((long)seq * H + hh) * R * C;
  auto tok = [&](int i) { return p.dir ? eos - 1 - i : bos + i; };
  // whole vectors: the thread's RPT rows (R % RPT == 0, arrays aligned to RPT elements) and
  // its 4 columns (C % 4 == 0, aligned to 4 elements); uniform
  const bool vr = R % RPT == 0 &&
                  (((uintptr_t)a | (uintptr_t)orow | (uintptr_t)ga) % (RPT * sizeof(T))) == 0;
  const bool vc = C % 4 == 0 && (((uintptr_t)b | (uintptr_t)gb) % (4 * sizeof(T))) == 0;
  const bool vst = C % 4 == 0 && (((uintptr_t)p.s0 | (uintptr_t)p.sN) & 15) == 0;

  // a step's inputs in their stored form (bf16 pairs per 32-bit word), unpacked when used:
  // two steps' worth stay in flight in half the registers of floats
  struct In {
    Raw<T, RPT> a, o, g;
    Raw<T, 4> b, gc;
  };
  // rows / columns past the state read as 0 (a gate of 0: factor e^0)
  auto load = [&](int s, In& x) {
    const int t = tok(s);
    const long ro = (long)t * rsR + (long)hh * R, co = (long)t * rsC + (long)hh * C;
    if (vr && r0 < R) {
      x.a.ld(a + ro + r0);
      x.o.ld(orow + ro + r0);
      if (has_ga) x.g.ld(ga + ro + r0); else x.g.zero();
    } else {
      x.a.ld_masked(a + ro, r0, R);
      x.o.ld_masked(orow + ro, r0, R);
      if (has_ga) x.g.ld_masked(ga + ro, r0, R); else x.g.zero();
    }
    if (vc && c0 < C) {
      x.b.ld(b + co + c0);
      if (has_gb) x.gc.ld(gb + co + c0); else x.gc.zero();
    } else {
      x.b.ld_masked(b + co, c0, C);
      if (has_gb) x.gc.ld_masked(gb + co, c0, C); else x.gc.zero();
    }
  };

  float S[RPT][4];
#pragma unroll
  for (int j = 0; j < RPT; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) S[j][i] = 0.f;
  if (p.s0) {
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      if (r0 + j >= R) continue;
      const long rb = sbase + (long)(r0 + j) * C;
      if (vst && c0 < C) {
        const float4 x = *reinterpret_cast<const float4*>(p.s0 + rb + c0);
        S[j][0] = x.x; S[j][1] = x.y; S[j][2] = x.z; S[j][3] = x.w;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) S[j][i] = c0 + i < C ? p.s0[rb + c0 + i] : 0.f;
      }
    }
  }

  In cur, nxt;
  if (n > 0) load(0, cur);
#pragma unroll 1
  for (int s0 = 0; s0 < n; s0 += STB) {
    const int ns = min(STB, n - s0);
#pragma unroll 1
    for (int k = 0; k < ns; ++k) {
      const int s = s0 + k;
      if (s + 1 < n) load(s + 1, nxt);
      float va[RPT], vo[RPT], eg[RPT], vb[4], ec[4], x[4] = {0.f, 0.f, 0.f, 0.f};
      cur.a.unpack(va);
      cur.o.unpack(vo);
      cur.g.unpack(eg);
      cur.b.unpack(vb);
      cur.gc.unpack(ec);
#pragma unroll
      for (int j = 0; j < RPT; ++j) eg[j] = gexp<T>(eg[j]);
#pragma unroll
      for (int i = 0; i < 4; ++i) ec[i] = gexp<T>(ec[i]);
#pragma unroll
      for (int j = 0; j < RPT; ++j) {
        const float sa = p.sa * va[j];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          S[j][i] = fmaf(sa, vb[i], S[j][i] * (eg[j] * ec[i]));
          x[i] = fmaf(vo[j], S[j][i], x[i]);
        }
      }
      const float cs = wave_colsum<16>(x);
      sO[(w * STB + k) * 64 + lane_col<16>(lane)] = cs;
      cur = nxt;
    }
    __syncthreads();   // the stage's column sums of every wave
    for (int i = tid; i < ns * 64; i += SNT) {
      const int k = i >> 6, c = i & 63;
      if (ct * 64 + c < C) {
        float v = 0.f;
#pragma unroll
        for (int ww = 0; ww < SNW; ++ww) v += sO[(ww * STB + k) * 64 + c];
        put<TO>(p.out, (long)tok(s0 + k) * rsC + (long)hh * C + ct * 64 + c, p.so * v);
      }
    }
    __syncthreads();   // read before the next stage writes
  }

  if (p.sN) {
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      if (r0 + j >= R) continue;
      const long rb = sbase + (long)(r0 + j) * C;
      if (vst && c0 < C) {
        // streamed past the L2 (whole 256-byte row pieces): the final state is not read again
        // in this launch, and dirty lines left in the L2 would be written back at its end
        typedef float f32x4_t __attribute__((ext_vector_type(4)));
        const f32x4_t x = {S[j][0], S[j][1], S[j][2], S[j][3]};
        __builtin_nontemporal_store(x, reinterpret_cast<f32x4_t*>(p.sN + rb + c0));
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (c0 + i < C) p.sN[rb + c0 + i] = S[j][i];
      }
    }
  }
}

namespace {

template <typename T, typename TO, int NCG, int RPT>
hipError_t launch_scan(const RecScanArgs& p, hipStream_t st) {
  constexpr int CB = NCG * 4;
  const long blocks = (long)p.si.N * p.H * ((p.C + CB - 1) / CB);
  if (blocks == 0) return hipSuccess;
  hipLaunchKernelGGL((rec_scan_kernel<T, TO, NCG, RPT>), dim3((unsigned)blocks), dim3(RNT), 0,
                     st, p);
  return hipGetLastError();
}

// 64-column tiles (4 row groups per wave) when they give enough blocks to fill the chip;
// 32-column tiles (8 row groups per wave, twice the blocks) otherwise and for more than 256
// rows (at most 8 rows x 4 columns of state per thread).
template <typename T, typename TO>
hipError_t dispatch_scan(const RecScanArgs& p, hipStream_t st) {
  const long blocks64 = (long)p.si.N * p.H * ((p.C + 63) / 64);
  if (blocks64 >= 256 && p.C > 32 && p.R <= 256) {
    if (p.R <= 64) return launch_scan<T, TO, 16, 2>(p, st);
    if (p.R <= 128) return launch_scan<T, TO, 16, 4>(p, st);
    return launch_scan<T, TO, 16, 8>(p, st);
  }
  if (p.R <= 128) return launch_scan<T, TO, 8, 2>(p, st);
  if (p.R <= 256) return launch_scan<T, TO, 8, 4>(p, st);
  if (p.R <= 512) return launch_scan<T, TO, 8, 8>(p, st);
  return hipErrorInvalidValue;
}

template <typename T, typename TO, int RPT>
hipError_t launch_short(const RecScanArgs& p, hipStream_t st) {
  const long blocks = (long)p.si.N * p.H * ((p.C + 63) / 64);
  if (blocks == 0) return hipSuccess;
  hipLaunchKernelGGL((rec_short_kernel<T, TO, RPT>), dim3((unsigned)blocks), dim3(SNT), 0, st,
                     p);
  return hipGetLastError();
}

template <typename T, typename TO>
hipError_t dispatch_short(const RecScanArgs& p, hipStream_t st) {
  if (p.R <= 32) return launch_short<T, TO, 2>(p, st);
  if (p.R <= 64) return launch_short<T, TO, 4>(p, st);
  return launch_short<T, TO, 8>(p, st);
}

// Plain forward scans (no gate-gradient epilogue, transposed state, shifted gates or flags)
// of fixed-length sequences of at most kShortT tokens over at most 128 state rows: the short
// scan kernel. Its steps wait on their own loads (one step ahead), the staged scan's on 16
// steps loaded at once: measured at B64 H16 K=V=128, 27 + 3.5 us per token against 36 + 1.9,
// so the short kernel only for a few tokens (decode).
constexpr int kShortT = 4;
bool short_scan(const RecScanArgs& p) {
  return p.dg == nullptr && !p.s_trans && !p.shift && !p.final_gate && p.flags.p == nullptr &&
         p.si.cu == nullptr && p.si.T <= kShortT && p.R <= 128 &&
         (long)p.si.N * p.H * ((p.C + 63) / 64) >= 256;
}

hipError_t run_scan(const RecScanArgs& p, int dtype, int o_dtype, hipStream_t st) {
  if (short_scan(p)) {
    if (dtype == DT_BF16 && o_dtype == DT_F32) return dispatch_short<bf16, float>(p, st);
    if (dtype == DT_BF16 && o_dtype == DT_BF16) return dispatch_short<bf16, bf16>(p, st);
    if (dtype == DT_F32 && o_dtype == DT_F32) return dispatch_short<float, float>(p, st);
    return hipErrorInvalidValue;
  }
  if (dtype == DT_BF16 && o_dtype == DT_F32) return dispatch_scan<bf16, float>(p, st);
  if (dtype == DT_BF16 && o_dtype == DT_BF16) return dispatch_scan<bf16, bf16>(p, st);
  if (dtype == DT_F32 && o_dtype == DT_F32) return dispatch_scan<float, float>(p, st);
  return hipErrorInvalidValue;
}

template <typename T, typename TO, int RPT>
hipError_t launch_bwd_fallback(const RecScanArgs& s1, const RecScanArgs& s2,
                               const RecScanArgs& s3, hipStream_t st) {
  const long blocks = (long)s1.si.N * s1.H;
  if (blocks == 0) return hipSuccess;
  hipLaunchKernelGGL((rec_bwd_fallback_kernel<T, TO, 8, RPT>), dim3((unsigned)blocks), dim3(RNT),
                     0, st, s1, s2, s3);
  return hipGetLastError();
}

// 32-column tiles (the scans' layout for up to 512 rows) for the rows of every scan
template <typename T, typename TO>
hipError_t dispatch_bwd_fallback(const RecScanArgs& s1, const RecScanArgs& s2,
                                 const RecScanArgs& s3, hipStream_t st) {
  const int R = s1.R > s3.R ? s1.R : s3.R;
  if (R <= 128) return launch_bwd_fallback<T, TO, 2>(s1, s2, s3, st);
  if (R <= 256) return launch_bwd_fallback<T, TO, 4>(s1, s2, s3, st);
  if (R <= 512) return launch_bwd_fallback<T, TO, 8>(s1, s2, s3, st);
  return hipErrorInvalidValue;
}

hipError_t run_bwd_fallback(const RecScanArgs& s1, const RecScanArgs& s2, const RecScanArgs& s3,
                            int dtype, int o_dtype, hipStream_t st) {
  if (dtype == DT_BF16 && o_dtype == DT_F32) return dispatch_bwd_fallback<bf16, float>(s1, s2, s3, st);
  if (dtype == DT_BF16 && o_dtype == DT_BF16) return dispatch_bwd_fallback<bf16, bf16>(s1, s2, s3, st);
  if (dtype == DT_F32 && o_dtype == DT_F32) return dispatch_bwd_fallback<float, float>(s1, s2, s3, st);
  return hipErrorInvalidValue;
}

}  // namespace

bool recurrent_supported(int K, int V) { return K <= 512 && V <= 512; }

hipError_t run_recurrent_fwd(const RecArgs& p, int dtype, int o_dtype, hipStream_t st) {
  RecScanArgs s{};
  s.H = p.H;
  s.si = p.si;
  s.a = p.k;
  s.ga = p.gk;
  s.o = p.q;
  s.b = p.v;
  s.gb = p.gv;
  s.s0 = p.h0;
  s.sN = p.ht;
  s.out = p.o;
  s.sa = 1.f;
  s.so = p.scale;
  s.R = p.K;
  s.C = p.V;
  s.dir = p.reverse ? 1 : 0;
  s.flags = p.flags;
  ktimer_mark(KT_REC_FWD, false, st);
  const hipError_t e = run_scan(s, dtype, o_dtype, st);
  ktimer_mark(KT_REC_FWD, true, st);
  return e;
}

hipError_t run_recurrent_bwd(const RecBwdArgs& p, int dtype, int o_dtype, hipStream_t st) {
  if (dtype != DT_BF16 && dtype != DT_F32) return hipErrorInvalidValue;
  const bool need_ht = p.dht != nullptr && (p.gk != nullptr || p.gv != nullptr);
  auto run = [&](const RecScanArgs& a) { return run_scan(a, dtype, o_dtype, st); };

  // 1. dq (and h_T) : S = h^T, rows V, columns K, the forward's direction
  RecScanArgs s{};
  s.H = p.H;
  s.si = p.si;
  s.a = p.v;
  s.ga = p.gv;
  s.o = p.dout;
  s.b = p.k;
  s.gb = p.gk;
  s.s0 = p.h0;
  s.sN = need_ht ? p.ht_ws : nullptr;
  s.s_trans = 1;
  s.out = p.dq;
  s.sa = 1.f;
  s.so = p.scale;
  s.R = p.V;
  s.C = p.K;
  s.dir = p.reverse ? 1 : 0;
  s.flags = p.flags;

  // 2. dk (+ dgk) : S = dh^T, rows V, columns K, opposite direction
  RecScanArgs s2 = s;
  s2.a = p.dout;
  s2.o = p.v;
  s2.b = p.q;
  s2.s0 = p.dht;
  s2.sN = nullptr;
  s2.out = p.dk;
  s2.sa = p.scale;
  s2.so = 1.f;
  s2.dir = p.reverse ? 0 : 1;
  s2.shift = 1;
  if (p.gk) {
    s2.gx = p.q;
    s2.gxf = p.dq;
    s2.gy = p.k;
    s2.hfin = need_ht ? p.ht_ws : nullptr;
    s2.dg = p.dgk;
    if (o_dtype != DT_F32) {
      // bf16 dq: its rounding residual goes into dgk (same layout), where the dk scan reads
      // a token's residual before it writes that token's gate gradient, so the q dq terms of
      // the reverse cumsum keep their float32 accuracy over long sequences
      s.out_lo = p.dgk;
      s2.gxf_lo = p.dgk;
    }
  }

  // 3. dv (+ dgv, dh0) : S = dh, rows K, columns V, opposite direction
  RecScanArgs s3{};
  s3.H = p.H;
  s3.si = p.si;
  s3.a = p.q;
  s3.ga = p.gk;
  s3.o = p.k;
  s3.b = p.dout;
  s3.gb = p.gv;
  s3.s0 = p.dht;
  s3.sN = p.dh0;
  s3.final_gate = 1;
  s3.out = p.dv;
  s3.sa = p.scale;
  s3.so = 1.f;
  s3.R = p.K;
  s3.C = p.V;
  s3.dir = p.reverse ? 0 : 1;
  s3.shift = 1;
  s3.flags = p.flags;
  if (p.gv) {
    s3.gx = p.dout;
    s3.gxf = p.o;   // the forward output, float
    s3.gxf_f32 = 1;
    s3.gy = p.v;
    s3.hfin = need_ht ? p.ht_ws : nullptr;
    s3.dg = p.dgv;
  }
  // the chunked backward's gate-range fallback: one launch for the three scans
  if (p.flags.p) return run_bwd_fallback(s, s2, s3, dtype, o_dtype, st);
  hipError_t e = run(s);
  if (e == hipSuccess) e = run(s2);
  if (e == hipSuccess) e = run(s3);
  return e;
}

}  // namespace tops
