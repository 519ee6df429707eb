// Full-head chunked-GLA kernels (bf16, chunk 64, K and V up to 128): one 512-thread block
// (8 waves, two per SIMD) owns the whole K x V state of one (sequence, head) -- or of one
// segment of a sequence -- and walks its chunks in order.
//
// Reference semantics: state scan tops/ops/common/chunk_h.py:18-119 (forward h) and
// :399-591 (reverse dh); fused forward chunk_gla_fwd, tops/ops/gla/chunk.py:1083-1179.
//
// Layout of the per-chunk work (C = 64 rows):
//  * every thread owns one 8-column group and RPT consecutive rows of the q / k / g tiles
//    (and of the v / do tile); its 16-byte global loads land in registers in exactly that
//    shape, so the chunk-local cumsum of g runs in registers: a local cumsum over the
//    thread's rows, a lane-shuffle prefix over the row segments of a wave, and one LDS
//    exchange of the eight wave totals. Gates are carried in base 2 (g * log2 e), so every
//    gate factor is one hardware exp2;
//  * loads are unconditional (rows and columns clamped into the tensor); invalid pieces are
//    zeroed as raw 16-byte words when consumed;
//  * gated tiles are written to LDS row-major with 16-byte stores; MFMA operands that are
//    needed transposed (v^T, k_d^T, h'^T) are read with transposed fragments;
//  * the K x V state lives in MFMA accumulators, out[v][k]: a lane's four values are four
//    consecutive v of one k (one 8-byte store into the [.., K, V] state layout). Wave w
//    holds v tiles of half (w & 1) and k tiles of quarter (w >> 1).
//
// Sequence segments: with NS > 1 the chunks of a sequence are split into NS segments of SL
// chunks. Pass 1 (head_scan_kernel, pass 1) computes every segment's local final state
// (from a zero state; the first segment in flow order starts from the given initial state)
// and the segment's total log2 decay; then every segment's block (head_scan_kernel pass 3,
// head_fwd_kernel, head_bwd_kernel) folds the local states of the segments before it in
// flow order into its entry state (load_entry_state) and walks its chunks, all segments in
// parallel. State composition over a segment is exact: h_out = 2^{Gamma} h_in + L with
// Gamma the summed (base-2) gates of the segment.
#include "common.hpp"
#include "kernels.hpp"

namespace tops {

namespace {

constexpr int HC = 64;    // chunk size of the full-head kernels
constexpr int HNT = 512;  // threads per block
constexpr int HNW = HNT / 64;
constexpr float kLog2e = 1.4426950408889634f;

template <int KP, int NT = HNT, int CR = HC>
struct HMap {
  static constexpr int NCG = KP / 8;     // 8-column groups
  static constexpr int NRS = NT / NCG;   // row segments
  static constexpr int RPT = CR / NRS;   // rows per thread (CR rows per tile)
  static_assert(RPT >= 1 && NRS * RPT == CR, "thread mapping");
};

// State / output tile split over the 8 waves: v tiles by halves, k tiles by quarters.
template <int KP, int VP>
struct HTiles {
  static constexpr int NTV = VP / 16 / 2;   // v tiles per wave
  static constexpr int NTK = KP / 16 / 4;   // k tiles per wave
};
// The same split for NW waves: v tiles by halves (w & 1), k tiles over the NW / 2 pairs.
template <int KP, int VP, int NW>
struct HTilesN {
  static constexpr int NTV = VP / 16 / 2;
  static constexpr int NTK = KP / 16 / (NW / 2);
  static_assert(NTK >= 1, "tile split");
};

// LDS tiles of bf16, W columns (W a multiple of 16). Element (r, c) sits at
//   r (W + 16) + 8 (r & ~7) + (c ^ (r & 8)):
// rows padded by 16 elements, 64 more elements after every 8 rows, and the two 8-column
// halves of every 16-column group swapped in the rows with bit 3 set. The LDS has 64 banks of
// 4 bytes; ds_read_b128 serves each half-wave in two groups of 16 lanes (the quads with even,
// then odd, parity of lane bits 2-4) and ds_read_b64_tr_b16 32 lanes at a time. In this layout
// the 16-byte row fragments and the transposed fragments of every 16 x 32 / 32 x 16 MFMA
// operand hit each bank once per group (4 and 2 LDS cycles per instruction); a plain
// 16-element row pad conflicts 2-way on both (8 and 4 cycles, SQ_LDS_IDX_ACTIVE per
// instruction on MI355X). The swizzle only touches lane-dependent address bits: for a tile
// origin (r0, c0) with r0 and c0 multiples of 16, off(r0 + r, c0 + c) = at(r0, c0) + off(r, c),
// so a fragment address is a per-lane part plus a constant.
template <int W>
struct LT {
  static_assert(W % 16 == 0, "tile width");
  static constexpr int P = W + 16;
  // bytes of a tile of `rows` rows (rows % 8 == 0)
  __host__ __device__ static constexpr int bytes(int rows) { return rows * (P + 8) * 2; }
  // element offset of the tile origin (r0, c0), r0 % 16 == 0, c0 % 16 == 0
  __host__ __device__ static constexpr int at(int r0, int c0) { return r0 * (P + 8) + c0; }
  __device__ static __forceinline__ int off(int r, int c) {
    return r * P + 8 * (r & ~7) + (c ^ (r & 8));
  }
  // per-lane parts: row fragment (row lane & 15, columns 8 (lane >> 4) + 0..7)
  __device__ static __forceinline__ int row_frag(int lane) {
    return off(lane & 15, 8 * (lane >> 4));
  }
  // transposed fragment, first read (row 8 (lane >> 4) + ((lane & 15) >> 2), columns
  // 4 (lane & 3) + 0..3); the second read is 4 rows further (4 P: same 8-row group)
  __device__ static __forceinline__ int tr_frag(int lane) {
    return off(8 * (lane >> 4) + ((lane & 15) >> 2), 4 * (lane & 3));
  }
  // one transposed read of a 16 x 16 tile (rows 4 (lane >> 4) + ((lane & 15) >> 2)): lane l
  // receives rows 4 (l >> 4) + 0..3 of column l & 15, the MFMA accumulator layout
  __device__ static __forceinline__ int tr_rows4(int lane) {
    return off(4 * (lane >> 4) + ((lane & 15) >> 2), 4 * (lane & 3));
  }
  // accumulator position (row lane & 15, columns 4 (lane >> 4) + 0..3)
  __device__ static __forceinline__ int acc_pos(int lane) {
    return off(lane & 15, 4 * (lane >> 4));
  }
};

// Fragments of LT tiles; o = element offset (tile origin + per-lane part).
__device__ __forceinline__ Frag<bf16> ldr(const bf16* t, int o) {
  Frag<bf16> f;
  f.d = *reinterpret_cast<const uint4*>(t + o);
  return f;
}
template <int W>
__device__ __forceinline__ Frag<bf16> ldt(const bf16* t, int o) {
  const bf16* p1 = t + o;
  const s4_t a = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s4_t*)(p1));
  const s4_t b = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s4_t*)(p1 + 4 * LT<W>::P));
  const uint2 ua = __builtin_bit_cast(uint2, a), ub = __builtin_bit_cast(uint2, b);
  Frag<bf16> f;
  f.d = make_uint4(ua.x, ua.y, ub.x, ub.y);
  return f;
}
// acc += X Y^T over klen columns: X rows xr0.. of a WX-wide tile, Y rows yr0.. of a WY-wide
// tile (row fragments of both)
template <int WX, int WY>
__device__ __forceinline__ void mma_rr(f32x4& acc, const bf16* X, int xr0, const bf16* Y,
                                       int yr0, int klen, int lane) {
  const int ox = LT<WX>::at(xr0, 0) + LT<WX>::row_frag(lane);
  const int oy = LT<WY>::at(yr0, 0) + LT<WY>::row_frag(lane);
  for (int kk = 0; kk < klen; kk += 32) mma(acc, ldr(X, ox + kk), ldr(Y, oy + kk));
}
// The same over K = KL columns (a compile-time depth), every fragment read before the
// products
template <int WX, int WY, int KL>
__device__ __forceinline__ void mma_rr_b(f32x4& acc, const bf16* X, int xr0, const bf16* Y,
                                         int yr0, int lane) {
  const int ox = LT<WX>::at(xr0, 0) + LT<WX>::row_frag(lane);
  const int oy = LT<WY>::at(yr0, 0) + LT<WY>::row_frag(lane);
  Frag<bf16> x[KL / 32], y[KL / 32];
#pragma unroll
  for (int kk = 0; kk < KL / 32; ++kk) {
    x[kk] = ldr(X, ox + kk * 32);
    y[kk] = ldr(Y, oy + kk * 32);
  }
#pragma unroll
  for (int kk = 0; kk < KL / 32; ++kk) mma(acc, x[kk], y[kk]);
}
// acc += X^T Y^T-rows: X stored [k][m] (columns xc0.. of a WX-wide tile, transposed
// fragments), Y rows yr0.. of a WY-wide tile stored [n][k] (row fragments), over klen k
template <int WX, int WY>
__device__ __forceinline__ void mma_tr(f32x4& acc, const bf16* X, int xc0, const bf16* Y,
                                       int yr0, int klen, int lane) {
  const int ox = LT<WX>::at(0, xc0) + LT<WX>::tr_frag(lane);
  const int oy = LT<WY>::at(yr0, 0) + LT<WY>::row_frag(lane);
  for (int kk = 0; kk < klen; kk += 32)
    mma(acc, ldt<WX>(X, ox + LT<WX>::at(kk, 0)), ldr(Y, oy + kk));
}

__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// A loop-invariant per-lane offset kept out of loop-invariant code motion: hoisted out of a
// chunk loop, such offsets become long-lived registers (64-bit per-lane pointers for global
// accesses) that the fused backward cannot hold, and spill; recomputed in the loop they cost
// an integer op or two.
__device__ __forceinline__ uint32_t opaque(uint32_t x) {
  asm volatile("" : "+v"(x));
  return x;
}

// s_waitcnt vmcnt(0) (expcnt, lgkmcnt left at their maxima) as a real instruction, which the
// compiler's wait-count tracking takes into account. Placed before a chunk loop it clears the
// loads issued ahead of the loop: the counter is in order and counts stores as well, so a
// wait the compiler sizes for the loop's entry, where only those loads are outstanding,
// would otherwise also wait, on every later pass, for the stores of the pass before.
__device__ __forceinline__ void vm_wait_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// acc + sum of the products of 8 bf16 pairs (v_dot2c_f32_bf16: fp32 accumulation)
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float dot8_bf16(uint4 a, uint4 b, float acc) {
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a.x),
                                        __builtin_bit_cast(bf16x2_t, b.x), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a.y),
                                        __builtin_bit_cast(bf16x2_t, b.y), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a.z),
                                        __builtin_bit_cast(bf16x2_t, b.z), acc, false);
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a.w),
                                         __builtin_bit_cast(bf16x2_t, b.w), acc, false);
}

__device__ __forceinline__ void unpack8(const uint4& u, float (&x)[8]) {
  x[0] = bf16_lo(u.x); x[1] = bf16_hi(u.x);
  x[2] = bf16_lo(u.y); x[3] = bf16_hi(u.y);
  x[4] = bf16_lo(u.z); x[5] = bf16_hi(u.z);
  x[6] = bf16_lo(u.w); x[7] = bf16_hi(u.w);
}
__device__ __forceinline__ uint4 pack8(const float (&x)[8]) {
  return make_uint4(pack2_bf16(x[0], x[1]), pack2_bf16(x[2], x[3]), pack2_bf16(x[4], x[5]),
                    pack2_bf16(x[6], x[7]));
}
__device__ __forceinline__ void st_f8(float* p, const float (&x)[8]) {
  reinterpret_cast<float4*>(p)[0] = make_float4(x[0], x[1], x[2], x[3]);
  reinterpret_cast<float4*>(p)[1] = make_float4(x[4], x[5], x[6], x[7]);
}
__device__ __forceinline__ void ld_f8(const float* p, float (&x)[8]) {
  const float4 a = reinterpret_cast<const float4*>(p)[0];
  const float4 b = reinterpret_cast<const float4*>(p)[1];
  x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
  x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}

// A wave's 16 x 64 bf16 block written to HBM as whole rows: staged tile by tile
// (stage_tile: a 16 x 16 tile whose lane holds 4 consecutive columns, 4 (lane >> 4) + 0..3,
// of row lane & 15) in the wave's own 16 x 72 LDS area `stg` (no other wave touches it; a
// wave's LDS accesses complete in order), then read back 16 bytes a lane, 8 lanes a
// 128-byte row (rows_out), and stored at dst + row * ld + column (elements): nontemporally
// when `nt` (whole lines: ld, the columns and dst 64-element aligned). Rows >= nrows and
// columns >= ncols (a multiple of 8) are not stored.
constexpr int kStgPitch = 72;                       // 144-byte rows: 16-byte aligned
constexpr int kStgBytes = 16 * kStgPitch * 2;       // per wave
__device__ __forceinline__ void stage_tile(bf16* stg, int i, const uint2& x, int lane) {
  *reinterpret_cast<uint2*>(stg + (lane & 15) * kStgPitch + i * 16 + 4 * (lane >> 4)) = x;
}
__device__ __forceinline__ void rows_out(const bf16* stg, bf16* dst, uint32_t ld, int nrows,
                                         int ncols, bool nt, int lane) {
  __builtin_amdgcn_wave_barrier();
  const int c = 8 * (lane & 7);
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    const int r = (lane >> 3) + 8 * hf;
    const uint4 y = *reinterpret_cast<const uint4*>(stg + r * kStgPitch + c);
    const uint32_t off = ((uint32_t)r * ld + (uint32_t)c) * 2u;
    if (r < nrows && c < ncols) st16_sel(dst, off, y, nt);
  }
  __builtin_amdgcn_wave_barrier();
}

// RPT rows x 16 bytes starting at (row0, col0) of a row-major bf16 tile at `base` with
// row stride rs elements. Unconditional: rows are clamped to len-1 and the column to w-8
// (w % 8 == 0, w >= 8); the caller masks what it consumes.
template <int RPT>
__device__ __forceinline__ void hload(uint4 (&r)[RPT], const bf16* __restrict__ base, uint32_t rs,
                                      int row0, int len, int col0, int w) {
  const uint32_t c = (uint32_t)min(col0, w - 8);
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    const uint32_t row = (uint32_t)min(row0 + j, len - 1);
    r[j] = ld16(base, (row * rs + c) * 2u);
  }
}

// Zeroes, in place, a thread's N rows (16-byte column groups) at or past `len` and every row
// when its column group lies past the tile's width. Callers skip it (a uniform branch) for
// full tiles: it only matters for a sequence's partial last chunk and for narrow heads.
template <int N>
__device__ __forceinline__ void mask_rows(uint4 (&r)[N], int row0, int len, bool col_ok) {
#pragma unroll
  for (int j = 0; j < N; ++j) r[j] = mask16(r[j], (col_ok && row0 + j < len) ? ~0u : 0u);
}

// Chunk range of the block's segment.
struct Seg {
  int seq, s, bos, eos, c0, cb, ce;
};
__device__ __forceinline__ Seg seg_of(const SeqInfo& si, int seq, int s, int NS, int SL) {
  Seg r;
  int nc;
  seq_range(si, seq, r.bos, r.eos, r.c0, nc);
  r.seq = seq;
  r.s = s;
  r.cb = NS > 1 ? min(nc, s * SL) : 0;
  r.ce = NS > 1 ? min(nc, r.cb + SL) : nc;
  return r;
}

// Scans over the four 16-lane rows of a wave, lane l of every row holding the same column
// (8-column groups of a 128-wide tile): v_permlane16_swap gives each lane its pair partner
// (rows 0 / 1, 2 / 3), v_permlane32_swap the other half's pair sum; no LDS, no lane indices.
// Returned: x_0 + .. + x_r (rows4_prefix) or x_r + .. + x_3 (rows4_suffix) for row r.
__device__ __forceinline__ float rows4_prefix(float x, int lane) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  const float pair = __uint_as_float(p[0]) + __uint_as_float(p[1]);   // x_{2i} + x_{2i+1}
  float y = (lane & 16) ? pair : x;
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(pair), __float_as_uint(pair),
                                                  false, false);
  if (lane & 32) y += __uint_as_float(q[0]);   // rows 2, 3: + the pair sum of rows 0, 1
  return y;
}
__device__ __forceinline__ float rows4_suffix(float x, int lane, float* total = nullptr) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  const float pair = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  float y = (lane & 16) ? x : pair;
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(pair), __float_as_uint(pair),
                                                  false, false);
  if (!(lane & 32)) y += __uint_as_float(q[1]);   // rows 0, 1: + the pair sum of rows 2, 3
  if (total) *total = __uint_as_float(q[0]) + __uint_as_float(q[1]);   // x_0 + .. + x_3
  return y;
}

// Base-2 chunk-local cumsum of a [CR x KP] gate tile (CR = HC rows unless stated) held as
// RPT rows x 8 columns per thread: gt holds the raw gates (already masked) on entry and
// g~ log2 e on return; gam = its last row, first = its row 0. sTot [NT/64][KP],
// sFirst [KP]. One barrier.
template <int KP, int NT, int CR = HC>
using GateRows = float[HMap<KP, NT, CR>::RPT][8];

template <int KP, int NT = HNT, int CR = HC>
__device__ __forceinline__ void head_cumsum_f(GateRows<KP, NT, CR>& gt, float (&gam)[8],
                                              float (&first)[8], float* sTot, float* sFirst,
                                              int cg, int rs, int lane, int w) {
  using M = HMap<KP, NT, CR>;
#pragma unroll
  for (int j = 0; j < M::RPT; ++j) {
#pragma unroll
    for (int e = 0; e < 8; ++e) gt[j][e] = gt[j][e] * kLog2e + (j ? gt[j - 1][e] : 0.f);
  }
  float x[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = gt[M::RPT - 1][e];
  if constexpr (M::NCG == 16) {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = rows4_prefix(x[e], lane);
  } else {
#pragma unroll
    for (int d = M::NCG; d < 64; d <<= 1) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float y = __shfl_up(x[e], d);
        if (lane >= d) x[e] += y;
      }
    }
  }
  if (lane >= 64 - M::NCG) st_f8(sTot + w * KP + cg * 8, x);   // wave total
  if (rs == 0) st_f8(sFirst + cg * 8, gt[0]);
  __syncthreads();
  // earlier waves' totals (w is wave-uniform: plain loops, no per-lane selects); the lane's
  // column offset taken through opaque() so that it is formed here, not held (and spilled)
  // across the callers' chunk loops
  float off[8], t[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) off[e] = 0.f;
  const int c8 = (int)opaque((uint32_t)(cg * 8));
  for (int ww = 0; ww < w; ++ww) {
    ld_f8(sTot + ww * KP + c8, t);
#pragma unroll
    for (int e = 0; e < 8; ++e) off[e] += t[e];
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) gam[e] = off[e];
  for (int ww = w; ww < NT / 64; ++ww) {
    ld_f8(sTot + ww * KP + c8, t);
#pragma unroll
    for (int e = 0; e < 8; ++e) gam[e] += t[e];
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) off[e] += x[e] - gt[M::RPT - 1][e];   // + earlier segments
  ld_f8(sFirst + cg * 8, first);
#pragma unroll
  for (int j = 0; j < M::RPT; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) gt[j][e] += off[e];
}

// The same from the raw bf16 tile (16 bytes = 8 columns per row).
template <int KP, int NT = HNT, int CR = HC>
__device__ __forceinline__ void head_cumsum(const uint4 (&graw)[HMap<KP, NT, CR>::RPT],
                                            float (&gt)[HMap<KP, NT, CR>::RPT][8],
                                            float (&gam)[8], float (&first)[8], float* sTot,
                                            float* sFirst, int cg, int rs, int lane, int w) {
#pragma unroll
  for (int j = 0; j < HMap<KP, NT, CR>::RPT; ++j) unpack8(graw[j], gt[j]);
  head_cumsum_f<KP, NT, CR>(gt, gam, first, sTot, sFirst, cg, rs, lane, w);
}

// One-sided cumsum of the state scans, which gate a row with one side of the cumsum only:
// the reverse scan with the inclusive prefix g~_j, the forward one with the exclusive suffix
// gam - g~_j (the sum of the rows after j). gt holds the raw gates on entry and that exponent
// (base 2) on return; gam = the tile's total, valid in the row segment rs == total_rs<REV>
// only (the last one for the prefix, the first one for the suffix). Every wave reads only
// the wave totals on its side. sTot [NT/64][KP]; one barrier.
template <int KP, int NT, bool REV>
__host__ __device__ constexpr int total_rs() {
  return REV ? HMap<KP, NT, HC>::NRS - 1 : 0;
}
template <int KP, int NT, int CR, bool REV>
__device__ __forceinline__ void scan_cumsum_f(GateRows<KP, NT, CR>& gt, float (&gam)[8],
                                              float* sTot, int cg, int lane, int w) {
  using M = HMap<KP, NT, CR>;
  constexpr int NW = NT / 64;
#pragma unroll
  for (int j = 0; j < M::RPT; ++j) {   // the thread's own rows: inclusive prefix
#pragma unroll
    for (int e = 0; e < 8; ++e) gt[j][e] = gt[j][e] * kLog2e + (j ? gt[j - 1][e] : 0.f);
  }
  // over the wave's row segments: inclusive prefix (REV) / suffix of the thread sums
  float x[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = gt[M::RPT - 1][e];
  if constexpr (M::NCG == 16) {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = REV ? rows4_prefix(x[e], lane) : rows4_suffix(x[e], lane);
  } else {
#pragma unroll
    for (int d = M::NCG; d < 64; d <<= 1) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if constexpr (REV) {
          const float y = __shfl_up(x[e], d);
          if (lane >= d) x[e] += y;
        } else {
          const float y = __shfl_down(x[e], d);
          if (lane + d < 64) x[e] += y;
        }
      }
    }
  }
  // wave total: held by the last row segment (prefix) / the first one (suffix)
  if (REV ? lane >= 64 - M::NCG : lane < M::NCG) st_f8(sTot + w * KP + cg * 8, x);
  __syncthreads();
  float off[8], t[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) off[e] = 0.f;
  // the earlier (REV) / later waves' totals; w is wave-uniform: plain loops
  for (int ww = REV ? 0 : w + 1; ww < (REV ? w : NW); ++ww) {
    ld_f8(sTot + ww * KP + cg * 8, t);
#pragma unroll
    for (int e = 0; e < 8; ++e) off[e] += t[e];
  }
  float own[8];   // the thread's own row sum
#pragma unroll
  for (int e = 0; e < 8; ++e) own[e] = gt[M::RPT - 1][e];
#pragma unroll
  for (int j = 0; j < M::RPT; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e)
      gt[j][e] = REV ? gt[j][e] + (x[e] - own[e]) + off[e] : (x[e] - gt[j][e]) + off[e];
#pragma unroll
  for (int e = 0; e < 8; ++e) gam[e] = REV ? gt[M::RPT - 1][e] : x[e] + off[e];
}

// Scalar gates (simple GLA, g_gamma): one float per row and head, the same for every key
// column: gate(t, h) = gs[t * gs_ts + h] (gs_ts = 0: a per-head constant). Loads of rows
// past the chunk are clamped to its last row; the caller masks them.
template <int RPT>
__device__ __forceinline__ void sg_load(float (&x)[RPT], const float* gs, long gs_ts, int t0,
                                        int row0, int len, int h) {
#pragma unroll
  for (int j = 0; j < RPT; ++j) x[j] = gs[(long)(t0 + min(row0 + j, len - 1)) * gs_ts + h];
}

// Scalar gates in the fused kernels: lane l of every wave holds row l of the chunk, and the
// wave's inclusive scan gives G_l, the base-2 chunk-local cumsum at row l (rows past the
// chunk add 0). Every wave computes it for itself: no LDS, no barrier.
__device__ __forceinline__ float sg_row_cumsum(float graw, int lane, int len) {
  float x = lane < len ? graw * kLog2e : 0.f;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const float y = __shfl_up(x, d);
    if (lane >= d) x += y;
  }
  return x;
}

// A float routed through a VGPR. An accumulator initialised straight from a global load is
// loaded into the accumulator registers, which makes the compiler drain every outstanding
// load at the top of the chunk loop.
__device__ __forceinline__ float via_vgpr(float x) {
  float y;
  asm volatile("v_mov_b32 %0, %1" : "=v"(y) : "v"(x));
  return y;
}

// State slices: rows k < K, columns v < V of a [K][ld] row-major state (ld = V for a whole
// state; a V tile passes its base column's address and the full row stride).
template <int NTV, int NTK>
__device__ __forceinline__ void load_state(f32x4 (&acc)[NTV][NTK], const float* init, int K,
                                           int V, int vt0, int kt0, int lane, int ld = -1) {
  if (ld < 0) ld = V;
#pragma unroll
  for (int i = 0; i < NTV; ++i)
#pragma unroll
    for (int j = 0; j < NTK; ++j) {
      acc[i][j] = zero4();
      const int kk = (kt0 + j) * 16 + (lane & 15), vv = (vt0 + i) * 16 + 4 * (lane >> 4);
      if (init && kk < K && vv < V) {
        const float4 x = *reinterpret_cast<const float4*>(
            reinterpret_cast<const char*>(init) + (uint32_t)(kk * ld + vv) * 4u);
        acc[i][j][0] = via_vgpr(x.x);
        acc[i][j][1] = via_vgpr(x.y);
        acc[i][j][2] = via_vgpr(x.z);
        acc[i][j][3] = via_vgpr(x.w);
      }
    }
}

// Entry state of segment s of a segmented scan, folded from the pass-1 local states L_u and
// segment decays Gamma_u (base 2) in the workspace, in the order the scan runs: forward
// L_0, then H <- 2^{Gamma_u} H + L_u for u = 1 .. s-1; reverse L_{NS-1}, then u = NS-2 ..
// s+1. Slot u of (sequence, head) is st + ((seq NS + u) H + h) K ld (+ cv: a V tile's
// first column), its decays gm + ((seq NS + u) H + h) K.
template <int NTV, int NTK, bool REV>
__device__ __forceinline__ void load_entry_state(f32x4 (&acc)[NTV][NTK], const float* st,
                                                 const float* gm, int seq, int s, int NS,
                                                 int H, int hh, int K, int Vw, int cv, int ld,
                                                 int vt0, int kt0, int lane) {
  const long KV = (long)K * ld;
  auto slot = [&](int u) { return st + ((long)(seq * NS + u) * H + hh) * KV + cv; };
  const int u0 = REV ? NS - 1 : 0;
  load_state<NTV, NTK>(acc, slot(u0), K, Vw, vt0, kt0, lane, ld);
  for (int u = REV ? u0 - 1 : 1; REV ? u > s : u < s; u += REV ? -1 : 1) {
    f32x4 x[NTV][NTK];
    load_state<NTV, NTK>(x, slot(u), K, Vw, vt0, kt0, lane, ld);
#pragma unroll
    for (int j = 0; j < NTK; ++j) {
      const int kk = (kt0 + j) * 16 + (lane & 15);
      const float g = kk < K ? exp2_hw(gm[((long)(seq * NS + u) * H + hh) * K + kk]) : 0.f;
#pragma unroll
      for (int i = 0; i < NTV; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[i][j][e] = g * acc[i][j][e] + x[i][j][e];
    }
  }
}

template <int NTV, int NTK>
__device__ __forceinline__ void store_state_f32(const f32x4 (&acc)[NTV][NTK], float* dst,
                                                int K, int V, int vt0, int kt0, int lane,
                                                int ld = -1) {
  if (ld < 0) ld = V;
#pragma unroll
  for (int i = 0; i < NTV; ++i)
#pragma unroll
    for (int j = 0; j < NTK; ++j) {
      const int kk = (kt0 + j) * 16 + (lane & 15), vv = (vt0 + i) * 16 + 4 * (lane >> 4);
      if (kk < K && vv < V)
        *reinterpret_cast<float4*>(reinterpret_cast<char*>(dst) + (uint32_t)(kk * ld + vv) * 4u) =
            make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
    }
}

template <int NTV, int NTK>
__device__ __forceinline__ void store_state_bf16(const f32x4 (&acc)[NTV][NTK], bf16* dst,
                                                 int K, int V, int vt0, int kt0, int lane,
                                                 int ld = -1) {
  if (ld < 0) ld = V;
#pragma unroll
  for (int i = 0; i < NTV; ++i)
#pragma unroll
    for (int j = 0; j < NTK; ++j) {
      const int kk = (kt0 + j) * 16 + (lane & 15), vv = (vt0 + i) * 16 + 4 * (lane >> 4);
      if (kk < K && vv < V)
        st8(dst, (uint32_t)(kk * ld + vv) * 2u,
            make_uint2(pack2_bf16(acc[i][j][0], acc[i][j][1]),
                       pack2_bf16(acc[i][j][2], acc[i][j][3])));
    }
}

// acc = acc * decay[k] + X^T Y over the chunk's CR rows: X = b [c][v] (sB, a WB-wide LT
// tile), Y = a [c][k] (sA, WA wide), both read with transposed fragments.
// With `post`, the result is then scaled by post[k] (the update then reads
// acc = post (.) (acc * decay + X^T Y)).
template <int NTV, int NTK, int WB, int WA, int CR = HC>
__device__ __forceinline__ void state_update(f32x4 (&acc)[NTV][NTK], const bf16* sB,
                                             const bf16* sA, const float* decay,
                                             int vt0, int kt0, int lane,
                                             const float* post = nullptr) {
#pragma unroll
  for (int j = 0; j < NTK; ++j) {
    const float d = decay[(kt0 + j) * 16 + (lane & 15)];
#pragma unroll
    for (int i = 0; i < NTV; ++i) acc[i][j] *= d;
  }
  const int ob = LT<WB>::tr_frag(lane), oa = LT<WA>::tr_frag(lane);
#pragma unroll
  for (int kk = 0; kk < CR; kk += 32) {
    Frag<bf16> x[NTV], y[NTK];
#pragma unroll
    for (int i = 0; i < NTV; ++i) x[i] = ldt<WB>(sB, LT<WB>::at(kk, (vt0 + i) * 16) + ob);
#pragma unroll
    for (int j = 0; j < NTK; ++j) y[j] = ldt<WA>(sA, LT<WA>::at(kk, (kt0 + j) * 16) + oa);
#pragma unroll
    for (int i = 0; i < NTV; ++i)
#pragma unroll
      for (int j = 0; j < NTK; ++j) mma(acc[i][j], x[i], y[j]);
  }
  if (post) {
#pragma unroll
    for (int j = 0; j < NTK; ++j) {
      const float d = post[(kt0 + j) * 16 + (lane & 15)];
#pragma unroll
      for (int i = 0; i < NTV; ++i) acc[i][j] *= d;
    }
  }
}

// V tile width of the full-head kernels for a K-wide head: the state slice K x VP stays in
// the block's MFMA accumulators (8 tiles of 16 x 16 per wave for every supported shape).
__host__ __device__ constexpr int head_vp(int KP, int V) {
  return KP > 128 ? 64 : (V <= 64 ? 64 : 128);
}

}  // namespace

// ---------------------------------------------------------------------------
// State scan: forward h (a = k, b = v) or reverse dh (a = q, b = do)
// ---------------------------------------------------------------------------
// LDS of head_scan_kernel: the gated a tile and the b tile of CR rows, the wave totals of
// the cumsum, the step's decays.
template <int KP, int VP, int NT, int CR, bool STG = false>
struct HSLayout {
  static constexpr int a = 0;
  static constexpr int b = a + LT<KP>::bytes(CR);
  static constexpr int tot = b + LT<VP>::bytes(CR);
  static constexpr int gam = tot + (NT / 64) * KP * 4;
  static constexpr int post = gam + KP * 4;   // PRE: the per-column factor after the update
  static constexpr int stg = post + KP * 4;   // STG: the step's state, bf16 [k][v]
  static constexpr int bytes = stg + (STG ? LT<VP>::bytes(KP) : 0);
};

// CR = HC: one step per chunk (every pass). CR = 2 HC (pass 1 only, which needs the
// segment's final state and total decay but no per-chunk state): one step per pair of
// chunks, a 128-row tile with its own cumsum; the recurrence is the same row by row, so the
// final state is unchanged, and every factor stays <= 1.
// PRE (wide heads with the per-chunk gating workspace): the gated rows come from there --
// qs = scale q 2^{g~} for the reverse scan (s <- 2^gamma s + qs^T b), kg for the forward
// one -- with the chunk decays, so a step has no cumsum and no per-element exp2. kg's column
// factor f = 2^{gamma-r} goes on the state instead of the rows: s <- f (.) (s 2^r + kg^T b).
// One thread per column group loads the factors (all 16 row groups loading the same 64
// bytes doubled the bytes a step moves through the CU's vector memory path).
template <int KP, int VP, bool REV, int NT, bool SG, int CR = HC, bool PRE = false>
__global__ __launch_bounds__(NT) void head_scan_kernel(HeadScanArgs p) {
  static_assert(!PRE || (!SG && CR == HC && HMap<KP, NT, CR>::RPT >= 4), "gated-tile scan");
  using MA = HMap<KP, NT, CR>;
  using MB = HMap<VP, NT, CR>;
  using TL = HTilesN<KP, VP, NT / 64>;
  using Lay = HSLayout<KP, VP, NT, CR, PRE>;
  static_assert(CR == HC || CR == 2 * HC, "chunk rows");
  constexpr int RPT = MA::RPT, VRPT = MB::RPT;
  constexpr int NTV = TL::NTV, NTK = TL::NTK;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  bf16* sA = reinterpret_cast<bf16*>(smem + Lay::a);
  bf16* sB = reinterpret_cast<bf16*>(smem + Lay::b);
  float* sTot = reinterpret_cast<float*>(smem + Lay::tot);
  float* sGam = reinterpret_cast<float*>(smem + Lay::gam);
  float* sPost = reinterpret_cast<float*>(smem + Lay::post);
  bf16* sStg = reinterpret_cast<bf16*>(smem + Lay::stg);   // PRE

  const bf16* __restrict__ a = (const bf16*)p.a;
  const bf16* __restrict__ b = (const bf16*)p.b;
  const bf16* __restrict__ g = (const bf16*)p.g;
  bf16* __restrict__ s_all = (bf16*)p.s_all;
  const int H = p.H, K = p.K, V = p.V;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave index, scalar
  const int L0 = xcd_remap(blockIdx.x, gridDim.x);
  const int VT = (V + VP - 1) / VP;            // V tiles (blocks of one segment and head)
  const int vt = L0 % VT, L = L0 / VT;
  const int cv = vt * VP, Vw = min(VP, V - cv);   // this tile's first column and width
  const int hh = L % H;
  const int nsl = p.ns_launch;
  const int s = p.s_begin + (L / H) % nsl;
  const Seg sg = seg_of(p.si, (L / H) / nsl, s, p.NS, p.SL);
  const int nsteps = CR == HC ? sg.ce - sg.cb : (sg.ce - sg.cb + 1) / 2;
  const bool first_seg = REV ? (s == p.NS - 1) : (s == 0);
  const bool last_seg = REV ? (s == 0) : (s == p.NS - 1);
  const long rsK = (long)H * K, rsV = (long)H * V;
  const long KV = (long)K * V;

  const int cg = tid % MA::NCG, rs = tid / MA::NCG;    // a / g mapping
  const int vg = tid % MB::NCG, vrs = tid / MB::NCG;   // b mapping
  const bool colA = cg * 8 < K, colB = vg * 8 < Vw;
  // the row segment that holds the tile's total decay (every one with the gating workspace)
  constexpr int TRS = PRE ? 0 : total_rs<KP, NT, REV>();

  const int vt0 = (w & 1) * NTV, kt0 = (w >> 1) * NTK;
  f32x4 acc[NTV][NTK];
  {
    if (!first_seg && p.pass == 3)
      load_entry_state<NTV, NTK, REV>(acc, p.seg_state, p.seg_gam, sg.seq, s, p.NS, H, hh, K,
                                      Vw, cv, V, vt0, kt0, lane);
    else
      load_state<NTV, NTK>(acc,
                           first_seg && p.s_init
                               ? p.s_init + ((long)sg.seq * H + hh) * KV + cv
                               : nullptr,
                           K, Vw, vt0, kt0, lane, V);
  }

  struct Regs {
    uint4 a[RPT], g[RPT], b[VRPT];
    float gs[RPT];
    uint4 gx[2];   // PRE: the chunk gate sums gamma of the thread's 8 columns
  };
  // rows [t0, t0 + len) of step `step`; ci = its first chunk. Pairs of chunks (CR = 2 HC)
  // are taken in flow order, so an odd count leaves the segment's last chunk in flow order
  // on its own; len never crosses the segment's end.
  auto span = [&](int step, int& t0, int& len, int& ci) {
    if constexpr (CR == HC) {
      ci = REV ? (sg.ce - 1 - step) : (sg.cb + step);
      t0 = sg.bos + ci * HC;
      len = min(HC, sg.eos - t0);
    } else {
      const int lo = REV ? max(sg.cb, sg.ce - 2 * step - 2) : sg.cb + 2 * step;
      const int hi = REV ? sg.ce - 2 * step : min(sg.ce, lo + 2);
      ci = lo;
      t0 = sg.bos + lo * HC;
      len = min(sg.eos, sg.bos + hi * HC) - t0;
    }
  };
  auto issue = [&](int step, Regs& R) {
    int t0, len, ci;
    span(min(step, nsteps - 1), t0, len, ci);
    const long oa = (long)t0 * rsK + (long)hh * K;
    if constexpr (PRE) {
      // gated rows (zeros past the chunk); row group 0 only: gx = the 8 columns' chunk gate
      // sums gamma, forward also g[0..1] = their factors f = 2^{gamma-r}, g[2..3] = 2^r
      const unsigned char* ent =
          (const unsigned char*)p.gate_ws + ((long)(sg.c0 + ci) * H + hh) * gate_ws_entry(K);
      hload<RPT>(R.a, (const bf16*)ent + (REV ? 0 : HC * K), (uint32_t)K, rs * RPT, HC, cg * 8,
                 K);
      if (rs == 0) {
        const float* fac = (const float*)(ent + 2L * HC * K * 2 + HC * HC * 2);
        const uint32_t co = (uint32_t)min(cg * 8, K - 8) * 4u;
        if constexpr (!REV) {
          R.g[0] = ld16(fac + 2 * K, co);
          R.g[1] = ld16(fac + 2 * K, co + 16u);
          R.g[2] = ld16(fac + K, co);
          R.g[3] = ld16(fac + K, co + 16u);
        }
        R.gx[0] = ld16(fac + 3 * K, co);
        R.gx[1] = ld16(fac + 3 * K, co + 16u);
      }
    } else {
      hload<RPT>(R.a, a + oa, (uint32_t)rsK, rs * RPT, len, cg * 8, K);
    }
    if constexpr (PRE) {
    } else if constexpr (SG)
      sg_load<RPT>(R.gs, p.gs, p.gs_ts, t0, rs * RPT, len, hh);
    else
      hload<RPT>(R.g, g + oa, (uint32_t)rsK, rs * RPT, len, cg * 8, K);
    hload<VRPT>(R.b, b + (long)t0 * rsV + (long)hh * V + cv, (uint32_t)rsV, vrs * VRPT, len,
                vg * 8, Vw);
  };
  // Pass 1 issues a step's loads in three parts at three points of the steps before it: the
  // gates two steps ahead (after the gating), the a rows one step ahead (after the cumsum),
  // the b rows one step ahead (after the update). Issued at once, a step's 12 loads per
  // thread stall the issuing waves until the loads before them have drained, and nothing is
  // issued while the waves compute; spread out they keep the CU's memory path busy under
  // the cumsum, the gating and the update (pass 1 73 -> 55-62 us, and 24 fewer VGPRs).
  constexpr bool SPLIT = CR == 2 * HC && !PRE;
  auto issue_g = [&](int step, Regs& R) {
    int t0, len, ci;
    span(min(step, nsteps - 1), t0, len, ci);
    if constexpr (SG)
      sg_load<RPT>(R.gs, p.gs, p.gs_ts, t0, rs * RPT, len, hh);
    else
      hload<RPT>(R.g, g + (long)t0 * rsK + (long)hh * K, (uint32_t)rsK, rs * RPT, len, cg * 8,
                 K);
  };
  auto issue_a = [&](int step, Regs& R) {
    int t0, len, ci;
    span(min(step, nsteps - 1), t0, len, ci);
    hload<RPT>(R.a, a + (long)t0 * rsK + (long)hh * K, (uint32_t)rsK, rs * RPT, len, cg * 8, K);
  };
  auto issue_b = [&](int step, Regs& R) {
    int t0, len, ci;
    span(min(step, nsteps - 1), t0, len, ci);
    hload<VRPT>(R.b, b + (long)t0 * rsV + (long)hh * V + cv, (uint32_t)rsV, vrs * VRPT, len,
                vg * 8, Vw);
  };

  float gsum[8];   // pass 1: total base-2 decay of the segment
#pragma unroll
  for (int e = 0; e < 8; ++e) gsum[e] = 0.f;

  // PRE with per-chunk states: the staged state of chunk stg_ci (sStg) to s_all as whole
  // 128-byte rows, 16 bytes a thread (nontemporal when the rows are whole lines)
  int stg_ci = -1;
  auto copy_staged = [&](int c) {
    bf16* dst = s_all + ((long)(sg.c0 + c) * H + hh) * KV + cv;
    constexpr int PR = VP / 8;
#pragma unroll
    for (int j = 0; j < KP * PR / NT; ++j) {
      const int pc = tid + NT * j, r = pc / PR, c8 = (pc % PR) * 8;
      const uint4 x = *reinterpret_cast<const uint4*>(sStg + LT<VP>::off(r, c8));
      if (r < K && c8 < Vw) st16_sel(dst, ((uint32_t)r * (uint32_t)V + c8) * 2u, x, V % 64 == 0);
    }
  };

  // R: this step's registers; Rn: the next step's (SPLIT: its a and b rows issued here)
  auto body = [&](int step, Regs& R, Regs& Rn) {
    int t0, len, ci;
    span(step, t0, len, ci);
    // zero the rows past the step and the columns past the tile (a sequence's partial last
    // step, narrow heads); full steps skip it
    if (!(len == CR && K == KP && Vw == VP)) {
      if constexpr (!PRE) {
        mask_rows<RPT>(R.a, rs * RPT, len, colA);
        if constexpr (!SG) mask_rows<RPT>(R.g, rs * RPT, len, colA);
      }
      mask_rows<VRPT>(R.b, vrs * VRPT, len, colB);
    }
    float gt[RPT][8], gam[8];
    if constexpr (PRE) {
      __syncthreads();   // the previous step's reads of the tiles are done
      if (s_all && stg_ci >= 0) copy_staged(stg_ci);
#pragma unroll
      for (int j = 0; j < RPT; ++j) {
        const int row = rs * RPT + j;
        *reinterpret_cast<uint4*>(sA + LT<KP>::off(row, cg * 8)) =
            mask16(R.a[j], colA ? ~0u : 0u);
      }
      if (rs == 0) {
        float d[8];
        *reinterpret_cast<uint4*>(gam) = R.gx[0];
        *reinterpret_cast<uint4*>(gam + 4) = R.gx[1];
        if constexpr (REV) {
#pragma unroll
          for (int e = 0; e < 8; ++e) d[e] = exp2_hw(gam[e]);
        } else {
          float f[8];
          *reinterpret_cast<uint4*>(f) = R.g[0];
          *reinterpret_cast<uint4*>(f + 4) = R.g[1];
          *reinterpret_cast<uint4*>(d) = R.g[2];
          *reinterpret_cast<uint4*>(d + 4) = R.g[3];
          st_f8(sPost + cg * 8, f);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) gsum[e] += gam[e];
        st_f8(sGam + cg * 8, d);
      }
    } else if constexpr (SG) {
#pragma unroll
      for (int j = 0; j < RPT; ++j) {
        const float x = (colA && rs * RPT + j < len) ? R.gs[j] : 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) gt[j][e] = x;
      }
      scan_cumsum_f<KP, NT, CR, REV>(gt, gam, sTot, cg, lane, w);
    } else {
#pragma unroll
      for (int j = 0; j < RPT; ++j) unpack8(R.g[j], gt[j]);
      scan_cumsum_f<KP, NT, CR, REV>(gt, gam, sTot, cg, lane, w);
    }
    if constexpr (SPLIT) issue_a(step + 1, Rn);
    if constexpr (!PRE) {
#pragma unroll
      for (int j = 0; j < RPT; ++j) {
        const int row = rs * RPT + j;
        float x[8];
        unpack8(R.a[j], x);
#pragma unroll
        for (int e = 0; e < 8; ++e)
          x[e] *= REV ? p.scale * exp2_hw(gt[j][e]) : exp2_hw(gt[j][e]);
        *reinterpret_cast<uint4*>(sA + LT<KP>::off(row, cg * 8)) = pack8(x);
      }
    }
#pragma unroll
    for (int j = 0; j < VRPT; ++j) {
      const int row = vrs * VRPT + j;
      *reinterpret_cast<uint4*>(sB + LT<VP>::off(row, vg * 8)) = R.b[j];
    }
    if (!PRE && rs == TRS) {
      float eg[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        eg[e] = exp2_hw(gam[e]);
        gsum[e] += gam[e];
      }
      st_f8(sGam + cg * 8, eg);
    }
    if constexpr (SPLIT)
      issue_g(step + 2, R);
    else
      issue(step + 2, R);
    __syncthreads();
    if constexpr (CR == HC) {
      // state entering the chunk (forward) / leaving it (reverse). PRE: staged in LDS and
      // stored as whole rows after the next step's first barrier (the accumulators' 8-byte
      // pieces, 32 bytes of a 128-byte row per store, took the dh pass at C5 70 -> 235 us)
      if constexpr (PRE) {
        if (s_all) {
          const int oa = LT<VP>::acc_pos(lane);
#pragma unroll
          for (int j = 0; j < NTK; ++j)
#pragma unroll
            for (int i = 0; i < NTV; ++i)
              *reinterpret_cast<uint2*>(sStg + LT<VP>::at((kt0 + j) * 16, (vt0 + i) * 16) +
                                        oa) =
                  make_uint2(pack2_bf16(acc[i][j][0], acc[i][j][1]),
                             pack2_bf16(acc[i][j][2], acc[i][j][3]));
          stg_ci = ci;
        }
      } else if (s_all) {
        store_state_bf16<NTV, NTK>(acc, s_all + ((long)(sg.c0 + ci) * H + hh) * KV + cv, K,
                                   Vw, vt0, kt0, lane, V);
      }
    }
    state_update<NTV, NTK, VP, KP, CR>(acc, sB, sA, sGam, vt0, kt0, lane,
                                       PRE && !REV ? sPost : nullptr);
    if constexpr (SPLIT) issue_b(step + 1, Rn);
  };

  if (nsteps > 0) {
    // Both register sets are consumed in every trip of the loop (the odd step after it):
    // the loop is entered, and taken again, with the same outstanding loads -- the older
    // set first -- so the waits for a step's loads leave the next step's in flight.
    Regs R0, R1;
    issue(0, R0);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (SPLIT)
      issue_g(1, R1);
    else
      issue(1, R1);
    int step = 0;
    for (; step + 1 < nsteps; step += 2) {
      body(step, R0, R1);
      body(step + 1, R1, R0);
    }
    if (step < nsteps) body(step, R0, R1);
    if constexpr (PRE) {
      if (s_all && stg_ci >= 0) {
        __syncthreads();
        copy_staged(stg_ci);
      }
    }
  }

  if (p.pass == 1) {
    store_state_f32<NTV, NTK>(acc, p.seg_state + ((long)(sg.seq * p.NS + s) * H + hh) * KV + cv,
                              K, Vw, vt0, kt0, lane, V);
    if (vt == 0 && rs == TRS && colA)   // the decays are the same for every V tile
      st_f8(p.seg_gam + ((long)(sg.seq * p.NS + s) * H + hh) * K + cg * 8, gsum);
  } else if (last_seg && p.s_final) {
    store_state_f32<NTV, NTK>(acc, p.s_final + ((long)sg.seq * H + hh) * KV + cv, K, Vw, vt0,
                              kt0, lane, V);
  }
}

// ---------------------------------------------------------------------------
// Per-chunk gating of wide heads (K = 256, several V tiles per head). Every V tile's block of
// the fused forward needs the same gated tiles, intra matrix and column factors of a chunk;
// this kernel makes them once per (chunk, head) into a caller workspace, and the forward's
// PRE build reads them instead of gating for itself. Workspace entry of chunk c, head h at
// (c * H + h) * GW bytes: qs bf16 [64][K] (q scale 2^{g~}: the inter term's rows, i.e. qg
// times its column factor scale 2^r), kg bf16 [64][K], A bf16 [64][64] (scaled, causal),
// factors f32 [4][K]: scale 2^r, 2^r, 2^{gamma - r}, gamma (base 2).
// ---------------------------------------------------------------------------

template <int KP>
struct GPLayout {
  static constexpr int qg = 0;
  static constexpr int kg = qg + LT<KP>::bytes(HC);
  static constexpr int tot = kg + LT<KP>::bytes(HC);
  static constexpr int first = tot + HNW * KP * 4;
  static constexpr int bytes = first + KP * 4;
};

template <int KP>
__global__ __launch_bounds__(HNT) void head_gate_kernel(HeadFwdArgs p) {
  using M = HMap<KP>;
  using Lay = GPLayout<KP>;
  constexpr int RPT = M::RPT;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  bf16* sQg = reinterpret_cast<bf16*>(smem + Lay::qg);
  bf16* sKg = reinterpret_cast<bf16*>(smem + Lay::kg);
  float* sTot = reinterpret_cast<float*>(smem + Lay::tot);
  float* sFirst = reinterpret_cast<float*>(smem + Lay::first);
  const int H = p.H, K = p.K;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hh = blockIdx.x % H, ci = blockIdx.x / H, seq = blockIdx.y;
  int bos, eos, c0, nc;
  seq_range(p.si, seq, bos, eos, c0, nc);
  if (ci >= nc) return;   // uniform
  const int t0 = bos + ci * HC, len = min(HC, eos - t0);
  const long rsK = (long)H * K;
  const int cg = tid % M::NCG, rs = tid / M::NCG;
  const bool colA = cg * 8 < K;
  const long oa = (long)t0 * rsK + (long)hh * K;
  uint4 Rq[RPT], Rk[RPT], Rg[RPT];
  hload<RPT>(Rq, (const bf16*)p.q + oa, (uint32_t)rsK, rs * RPT, len, cg * 8, K);
  hload<RPT>(Rk, (const bf16*)p.k + oa, (uint32_t)rsK, rs * RPT, len, cg * 8, K);
  hload<RPT>(Rg, (const bf16*)p.g + oa, (uint32_t)rsK, rs * RPT, len, cg * 8, K);
  uint4 gm[RPT];
#pragma unroll
  for (int j = 0; j < RPT; ++j) gm[j] = mask16(Rg[j], (colA && rs * RPT + j < len) ? ~0u : 0u);
  float gt[RPT][8], gam[8], first[8];
  head_cumsum<KP>(gm, gt, gam, first, sTot, sFirst, cg, rs, lane, w);
  unsigned char* ent = (unsigned char*)p.gate_ws + ((long)(c0 + ci) * H + hh) * gate_ws_entry(K);
  bf16* gq = (bf16*)ent;
  bf16* gk = gq + HC * K;
  bf16* gA = gk + HC * K;
  float* gf = (float*)(gA + HC * HC);
  float r[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = 0.5f * (first[e] + gam[e]);
  if (p.flags) {   // uniform: the chunk's gate-range flag, per chunk [NC, H], always written
    float dmax = 0.f;   // rows past the chunk hold gam, columns past K zeros: both in range
#pragma unroll
    for (int j = 0; j < RPT; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) dmax = fmaxf(dmax, fabsf(gt[j][e] - r[e]));
    const int bad = __syncthreads_or(dmax > kGateLimit2 ? 1 : 0);
    if (tid == 0) p.flags[(long)(c0 + ci) * H + hh] = bad ? 1 : 0;
  }
  float fs[8];   // scale 2^r: qs = qg fs
#pragma unroll
  for (int e = 0; e < 8; ++e) fs[e] = p.scale * exp2_hw(r[e]);
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    const int row = rs * RPT + j;
    const uint32_t m = (colA && row < len) ? ~0u : 0u;
    float xq[8], xk[8], xs[8];
    unpack8(mask16(Rq[j], m), xq);
    unpack8(mask16(Rk[j], m), xk);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float d = gt[j][e] - r[e];
      xq[e] *= exp2_hw(d);
      xk[e] *= exp2_hw(-d);
      xs[e] = xq[e] * fs[e];
    }
    const uint4 pq = pack8(xq), pk = pack8(xk);
    *reinterpret_cast<uint4*>(sQg + LT<KP>::off(row, cg * 8)) = pq;
    *reinterpret_cast<uint4*>(sKg + LT<KP>::off(row, cg * 8)) = pk;
    if (colA) {
      *reinterpret_cast<uint4*>(gq + row * K + cg * 8) = pack8(xs);
      *reinterpret_cast<uint4*>(gk + row * K + cg * 8) = pk;
    }
  }
  if (rs == 0 && colA) {
    float f0[8], f1[8], f2[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      f1[e] = exp2_hw(r[e]);
      f0[e] = p.scale * f1[e];
      f2[e] = exp2_hw(gam[e] - r[e]);
    }
    st_f8(gf + cg * 8, f0);
    st_f8(gf + K + cg * 8, f1);
    st_f8(gf + 2 * K + cg * 8, f2);
    st_f8(gf + 3 * K + cg * 8, gam);
  }
  __syncthreads();
  // the 16 tiles of A (the upper ones as zeros), two per wave
  for (int t = w; t < 16; t += HNW) {
    const int mi = t >> 2, ni = t & 3;
    f32x4 at = zero4();
    if (ni <= mi) mma_rr<KP, KP>(at, sQg, mi * 16, sKg, ni * 16, KP, lane);
    const int jj = ni * 16 + (lane & 15);
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int ii = mi * 16 + 4 * (lane >> 4) + rr;
      gA[ii * HC + jj] = from_f32<bf16>(jj <= ii ? at[rr] * p.scale : 0.f);
    }
  }
}

// ---------------------------------------------------------------------------
// Per-chunk dq, dk, dg of heads wider than 64 on the per-chunk backward (bf16, chunk 64, K in
// (64, 256], any V): one 256-thread block per (chunk, head, 128-column key slice), streaming
// V in 64-column tiles. With G the base-2 chunk-local cumsum of the gates, R = (G_first +
// Gamma) / 2 per column, Gamma its last row, h the state entering the chunk and dh the
// gradient of the state leaving it:
//   qg = q 2^{G-R}, kg = k 2^{R-G}, dA = scale tril(do v^T)
//   Xq = dA kg + scale 2^R (do h^T),  Xm = 2^{Gamma-R} (v dh^T),  Xk = dA^T qg + Xm
//   dq = 2^{G-R} Xq,  dk = 2^{R-G} Xk
//   dg = revcumsum_rows(qg Xq - kg Xk) + 2^Gamma sum_v h dh + sum_rows kg Xm
// Every product is formed transposed ([k x i] tiles): an accumulator lane then holds four
// consecutive key columns of one chunk row, i.e. 8-byte row pieces of dq, dk, dg, qg and kg.
// Wave w owns key tiles KTW w .. KTW w + KTW - 1 of the slice over all 64 rows, so the chunk
// cumsum of the gates and dg's reverse cumsum over the rows run inside the wave (DPP row
// shifts over the 16 lanes of a row group, a running total over the four row tiles): no
// block-wide exchange. do, v, h and dh tiles are staged in LDS with whole-line loads, one V
// tile ahead; dA is formed once per slice; dq, dk and dg are written over the wave's own q, k
// and g pieces in LDS and stored as whole row pieces of the slice (8-byte pieces straight to
// HBM are partial-line stores). Two blocks share a CU (61.5 KB of LDS, two waves per SIMD),
// so one block's gating and epilogue run under the other's V loop; the two slices of a
// K = 256 head are adjacent blocks (one XCD), whose do / v reads meet in its L2. Replaces a
// grid of (chunk, head, 64-column key tile) blocks, each of which read all of do and v and
// formed dA again.
// ---------------------------------------------------------------------------
constexpr int DKB = 128;   // key columns per block
constexpr int DNW = 4;     // waves per block
// LDS of the V loop (do, v: 64 x 64; h, dh: the slice's KB key rows x 64), then, over the
// same bytes, of the epilogue (q -> qg, k -> kg, g: 64 x KB; dA 64 x 64)
template <int KB>
struct HDLayout {
  static constexpr int TB = LT<64>::bytes(HC);
  static constexpr int HB = LT<64>::bytes(KB);
  static constexpr int GB = LT<KB>::bytes(HC);
  static constexpr int dout = 0, v = TB, h = 2 * TB, dh = 2 * TB + HB;
  static constexpr int loop_end = 2 * TB + 2 * HB;
  static constexpr int qg = 0, kg = GB, g = 2 * GB, da = 3 * GB;
  static constexpr int after_end = 3 * GB + TB;
  static constexpr int bytes = loop_end > after_end ? loop_end : after_end;
};

// x + the value `SH` lanes below (row_shr) or above (row_shl) within each 16-lane row, zero
// past the row's end (bound_ctrl)
template <int CTRL>
__device__ __forceinline__ float dpp_add(float x) {
  return x + __uint_as_float(
                 __builtin_amdgcn_update_dpp(0u, __float_as_uint(x), CTRL, 0xF, 0xF, true));
}
// inclusive prefix / suffix over the 16 lanes of each row
__device__ __forceinline__ float row16_prefix(float x) {
  x = dpp_add<0x111>(x);
  x = dpp_add<0x112>(x);
  x = dpp_add<0x114>(x);
  return dpp_add<0x118>(x);
}
__device__ __forceinline__ float row16_suffix(float x) {
  x = dpp_add<0x101>(x);
  x = dpp_add<0x102>(x);
  x = dpp_add<0x104>(x);
  return dpp_add<0x108>(x);
}

// 4 bf16 (8 bytes) <-> floats
__device__ __forceinline__ void unpack4(const uint2& u, float (&x)[4]) {
  x[0] = bf16_lo(u.x); x[1] = bf16_hi(u.x);
  x[2] = bf16_lo(u.y); x[3] = bf16_hi(u.y);
}
__device__ __forceinline__ uint2 pack4(const float (&x)[4]) {
  return make_uint2(pack2_bf16(x[0], x[1]), pack2_bf16(x[2], x[3]));
}

// Base-2 chunk cumsum of one key tile in the transposed accumulator layout: x[mi][r] holds the
// raw gate of row 16 mi + (lane & 15), column 4 (lane >> 4) + r (rows past the chunk zero);
// on return G (base 2, inclusive over the rows), R = (G_first + Gamma) / 2 and Gamma.
__device__ __forceinline__ void acc_cumsum(float (&x)[4][4], float (&R)[4], float (&Gm)[4],
                                           int lane) {
  float run[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float pre = row16_prefix(x[mi][r] * kLog2e);
      const float tot = __shfl(pre, lane | 15);   // the row group's total
      x[mi][r] = run[r] + pre;
      run[r] += tot;
    }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float first = __shfl(x[0][r], lane & 0x30);   // row 0
    Gm[r] = run[r];
    R[r] = 0.5f * (first + run[r]);
  }
}

template <int KB, int NW>
__global__ __launch_bounds__(NW * 64, 2) void head_dqkg_kernel(BwdArgs p) {
  using Lay = HDLayout<KB>;
  constexpr int NT = NW * 64;
  constexpr int KTW = KB / 16 / NW;   // key tiles per wave
  static_assert(KTW >= 1 && KTW * 16 * NW == KB, "key tiles over the waves");
  // 16-byte pieces per thread: a 64 x 64 tile, a KB x 64 slice of h / dh, a 64 x KB slice of
  // q / k / g (8 or KB / 8 pieces a row)
  constexpr int P64 = 64 * 8 / NT, PH = KB * 8 / NT, PK = 64 * (KB / 8) / NT;
  static_assert(P64 * NT == 512 && PH * NT == KB * 8 && PK * NT == 8 * KB, "staging map");
  constexpr int NDA = 16 / NW;        // dA tiles (lower and upper) per wave
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  bf16* sDo = reinterpret_cast<bf16*>(smem + Lay::dout);
  bf16* sV = reinterpret_cast<bf16*>(smem + Lay::v);
  bf16* sH = reinterpret_cast<bf16*>(smem + Lay::h);
  bf16* sDh = reinterpret_cast<bf16*>(smem + Lay::dh);
  bf16* sQg = reinterpret_cast<bf16*>(smem + Lay::qg);
  bf16* sKg = reinterpret_cast<bf16*>(smem + Lay::kg);
  bf16* sG = reinterpret_cast<bf16*>(smem + Lay::g);
  bf16* sdA = reinterpret_cast<bf16*>(smem + Lay::da);

  const int H = p.H, K = p.K, V = p.V;
  const int KS = (K + KB - 1) / KB;   // key slices per head
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int kb = (L % KS) * KB;       // the slice's first key column
  const int c = (L / KS) / H, hh = (L / KS) % H;
  int seq, t0, len;
  chunk_range(p.si, c, seq, t0, len);
  (void)seq;
  const uint32_t rsK = (uint32_t)(H * K), rsV = (uint32_t)(H * V);
  const long oK = (long)t0 * rsK + (long)hh * K, oV = (long)t0 * rsV + (long)hh * V;
  const bf16* __restrict__ q = (const bf16*)p.q + oK;
  const bf16* __restrict__ k = (const bf16*)p.k + oK;
  const bf16* __restrict__ g = (const bf16*)p.g + oK;
  const bf16* __restrict__ v = (const bf16*)p.v + oV;
  const bf16* __restrict__ dout = (const bf16*)p.dout + oV;
  const long KV = (long)K * V;
  const bf16* __restrict__ hc = (const bf16*)p.h + ((long)c * H + hh) * KV;
  const bf16* __restrict__ dhc = (const bf16*)p.dh + ((long)c * H + hh) * KV;
  const float scale = p.scale;
  const int VT = (V + 63) >> 6;
  const int kt0 = w * KTW;   // this wave's first key tile in the slice
  const int ri = lane & 15;

  // ---- staging: whole 128-byte row pieces (8 lanes a row), rows / columns past the chunk
  // or the head as zeros ----
  // V tile vt of do, v (rows: chunk rows) and of h, dh (rows: the slice's key rows)
  auto ld_dv = [&](int vt, uint4 (&rd)[P64], uint4 (&rv)[P64]) {
#pragma unroll
    for (int e = 0; e < P64; ++e) {
      const int pc = tid + NT * e, row = pc >> 3, col = vt * 64 + 8 * (pc & 7);
      const uint32_t off = ((uint32_t)min(row, len - 1) * rsV + (uint32_t)min(col, V - 8)) * 2u;
      rd[e] = ld16(dout, off);
      rv[e] = ld16(v, off);
      if (row >= len || col >= V) rd[e] = rv[e] = make_uint4(0, 0, 0, 0);
    }
  };
  auto ld_h = [&](int vt, uint4 (&rh)[PH], uint4 (&rdh)[PH]) {
#pragma unroll
    for (int e = 0; e < PH; ++e) {
      const int pc = tid + NT * e, row = kb + (pc >> 3), col = vt * 64 + 8 * (pc & 7);
      const uint32_t off = ((uint32_t)min(row, K - 1) * (uint32_t)V +
                            (uint32_t)min(col, V - 8)) * 2u;
      rh[e] = ld16(hc, off);
      rdh[e] = ld16(dhc, off);
      if (row >= K || col >= V) rh[e] = rdh[e] = make_uint4(0, 0, 0, 0);
    }
  };
  auto ld_v = [&](int vt, uint4 (&rd)[P64], uint4 (&rv)[P64], uint4 (&rh)[PH],
                  uint4 (&rdh)[PH]) {
    ld_dv(vt, rd, rv);
    ld_h(vt, rh, rdh);
  };
  auto st_v = [&](const uint4 (&rd)[P64], const uint4 (&rv)[P64], const uint4 (&rh)[PH],
                  const uint4 (&rdh)[PH]) {
#pragma unroll
    for (int e = 0; e < P64; ++e) {
      const int pc = tid + NT * e;
      const int o = LT<64>::off(pc >> 3, 8 * (pc & 7));
      *reinterpret_cast<uint4*>(sDo + o) = rd[e];
      *reinterpret_cast<uint4*>(sV + o) = rv[e];
    }
#pragma unroll
    for (int e = 0; e < PH; ++e) {
      const int pc = tid + NT * e;
      const int o = LT<64>::off(pc >> 3, 8 * (pc & 7));
      *reinterpret_cast<uint4*>(sH + o) = rh[e];
      *reinterpret_cast<uint4*>(sDh + o) = rdh[e];
    }
  };
  // the chunk's q, k, g over the slice's key columns
  auto ld_k = [&](uint4 (&rq)[PK], uint4 (&rk)[PK], uint4 (&rg)[PK]) {
#pragma unroll
    for (int e = 0; e < PK; ++e) {
      const int pc = tid + NT * e, row = pc / (KB / 8), col = kb + 8 * (pc % (KB / 8));
      const uint32_t off = ((uint32_t)min(row, len - 1) * rsK + (uint32_t)min(col, K - 8)) * 2u;
      rq[e] = ld16(q, off);
      rk[e] = ld16(k, off);
      rg[e] = ld16(g, off);
      if (row >= len || col >= K) rq[e] = rk[e] = rg[e] = make_uint4(0, 0, 0, 0);
    }
  };
  auto st_k = [&](const uint4 (&rq)[PK], const uint4 (&rk)[PK], const uint4 (&rg)[PK]) {
#pragma unroll
    for (int e = 0; e < PK; ++e) {
      const int pc = tid + NT * e;
      const int o = LT<KB>::off(pc / (KB / 8), 8 * (pc % (KB / 8)));
      *reinterpret_cast<uint4*>(sQg + o) = rq[e];
      *reinterpret_cast<uint4*>(sKg + o) = rk[e];
      *reinterpret_cast<uint4*>(sG + o) = rg[e];
    }
  };

  // dA tiles (as [j x i] products): wave w takes tiles w + NW e, e < 16 / NW; tiles 0..9 are
  // the lower ones (j tile <= i tile; tile u: mi with mi (mi + 1) / 2 <= u, nj = u - mi (mi +
  // 1) / 2), 10..15 the upper ones, written as zeros (rows 0, 0, 0, 1, 1, 2, columns 1, 2, 3,
  // 2, 3, 3). Arithmetic, not a table: the values are uniform.
  int dmi[NDA], dnj[NDA];
#pragma unroll
  for (int e = 0; e < NDA; ++e) {
    const int u = w + NW * e;
    if (u < 10) {
      dmi[e] = (u >= 1) + (u >= 3) + (u >= 6);
      dnj[e] = u - dmi[e] * (dmi[e] + 1) / 2;
    } else {
      const int x = u - 10;
      dmi[e] = (x >= 3) + (x >= 5);
      dnj[e] = dmi[e] == 0 ? x + 1 : dmi[e] == 1 ? x - 1 : 3;
    }
  }

  // ---- V loop: do h^T, v dh^T (all key tiles of the wave), dA, sum_v h dh ----
  f32x4 Mq[KTW][4], M2[KTW][4], dA[NDA];
#pragma unroll
  for (int t = 0; t < KTW; ++t)
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) Mq[t][mi] = M2[t][mi] = zero4();
#pragma unroll
  for (int e = 0; e < NDA; ++e) dA[e] = zero4();
  float hd[KTW];
#pragma unroll
  for (int t = 0; t < KTW; ++t) hd[t] = 0.f;
  const int rf = LT<64>::row_frag(lane);

  uint4 rd[P64], rv[P64], rh[PH], rdh[PH];
  ld_v(0, rd, rv, rh, rdh);
#pragma unroll 1
  for (int vt = 0; vt < VT; ++vt) {
    st_v(rd, rv, rh, rdh);
    __syncthreads();   // this V tile in LDS
    // the next V tile's loads in two parts, h / dh here and do / v between the products:
    // all twelve at once stall the issuing waves behind each other
    if (vt + 1 < VT) ld_h(vt + 1, rh, rdh);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < KTW; ++t) {
      if (t == KTW / 2) {
        if (vt + 1 < VT) ld_dv(vt + 1, rd, rv);
        __builtin_amdgcn_sched_barrier(0);
      }
      Frag<bf16> fh[2], fdh[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int o = LT<64>::at((kt0 + t) * 16, 32 * s) + rf;
        fh[s] = ldr(sH, o);
        fdh[s] = ldr(sDh, o);
        hd[t] = dot8_bf16(fh[s].d, fdh[s].d, hd[t]);
      }
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const int o = LT<64>::at(16 * mi, 32 * s) + rf;
          mma(Mq[t][mi], fh[s], ldr(sDo, o));
          mma(M2[t][mi], fdh[s], ldr(sV, o));
        }
    }
#pragma unroll
    for (int e = 0; e < NDA; ++e) {
      if (w + NW * e < 10) {   // uniform
#pragma unroll
        for (int s = 0; s < 2; ++s)
          mma(dA[e], ldr(sV, LT<64>::at(16 * dnj[e], 32 * s) + rf),
              ldr(sDo, LT<64>::at(16 * dmi[e], 32 * s) + rf));
      }
    }
    __syncthreads();   // this tile's readers are done
  }

  // ---- q, k, g of the slice into LDS (over the V loop's tiles), dA, the gating ----
  {
    uint4 rq[PK], rk[PK], rg[PK];
    ld_k(rq, rk, rg);
    st_k(rq, rk, rg);
  }
  const int o0 = LT<64>::acc_pos(lane);
#pragma unroll
  for (int e = 0; e < NDA; ++e) {
    float x[4] = {0.f, 0.f, 0.f, 0.f};
    if (w + NW * e < 10) {
      const int i = 16 * dmi[e] + ri;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = 16 * dnj[e] + 4 * (lane >> 4) + r;
        x[r] = j <= i ? dA[e][r] * scale : 0.f;
      }
    }
    *reinterpret_cast<uint2*>(sdA + LT<64>::at(16 * dmi[e], 16 * dnj[e]) + o0) = pack4(x);
  }
  __syncthreads();   // q, k, g, dA in LDS
  // the lane's piece of a [k x i] tile of the slice: row 16 mi + (lane & 15), key columns
  // kc + 4 (lane >> 4) .. + 3 (the accumulator position of a transposed product)
  auto piece = [&](const bf16* t_, int mi, int kc, float (&x)[4]) {
    unpack4(*reinterpret_cast<const uint2*>(t_ + LT<KB>::at(16 * mi, kc) + LT<KB>::acc_pos(lane)),
            x);
  };
  // gating of the wave's own key tiles, in place (q -> qg, k -> kg): the wave reads and writes
  // only its own columns, each lane only its own pieces
  float G[KTW][4][4], R[KTW][4], Gm[KTW][4];
#pragma unroll
  for (int t = 0; t < KTW; ++t) {
    const int kc = (kt0 + t) * 16;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) piece(sG, mi, kc, G[t][mi]);
    acc_cumsum(G[t], R[t], Gm[t], lane);
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
      float xq[4], xk[4];
      piece(sQg, mi, kc, xq);
      piece(sKg, mi, kc, xk);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float d = G[t][mi][r] - R[t][r];
        xq[r] *= exp2_hw(d);
        xk[r] *= exp2_hw(-d);
      }
      const int o = LT<KB>::at(16 * mi, kc) + LT<KB>::acc_pos(lane);
      *reinterpret_cast<uint2*>(sQg + o) = pack4(xq);
      *reinterpret_cast<uint2*>(sKg + o) = pack4(xk);
    }
  }

  // ---- per key tile: the chunk products, then dq, dk, dg ----
  bf16* __restrict__ dq = (bf16*)p.dq + oK;
  bf16* __restrict__ dk = (bf16*)p.dk + oK;
  bf16* __restrict__ dg = (bf16*)p.dg + oK;
  const int tf = LT<KB>::tr_frag(lane), tf64 = LT<64>::tr_frag(lane);
#pragma unroll
  for (int t = 0; t < KTW; ++t) {
    const int kc = (kt0 + t) * 16;
    f32x4 Mqi[4], Mk1[4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
      Mqi[mi] = Mk1[mi] = zero4();
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        // Xq: sum_j kg[j][k] dA[i][j]; Xk: sum_i qg[i][k] dA[i][j] (row tile mi as j)
        mma(Mqi[mi], ldt<KB>(sKg, LT<KB>::at(32 * s, kc) + tf),
            ldr(sdA, LT<64>::at(16 * mi, 32 * s) + rf));
        mma(Mk1[mi], ldt<KB>(sQg, LT<KB>::at(32 * s, kc) + tf),
            ldt<64>(sdA, LT<64>::at(32 * s, 16 * mi) + tf64));
      }
    }
    // sum_v h dh: lane (lane & 15) of every row group holds row kc + (lane & 15) after the
    // sum over the four column groups; taken for rows kc + 4 (lane >> 4) + r
    float hs = hd[t];
    hs += __shfl_xor(hs, 16);
    hs += __shfl_xor(hs, 32);
    float fr[4], fe[4], hdp[4], y[4][4], dkc[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      hdp[r] = __shfl(hs, 4 * (lane >> 4) + r);
      fr[r] = scale * exp2_hw(R[t][r]);
      fe[r] = exp2_hw(Gm[t][r] - R[t][r]);
      dkc[r] = 0.f;
    }
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
      float qv[4], kv[4], vq[4], vk[4];
      piece(sQg, mi, kc, qv);
      piece(sKg, mi, kc, kv);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float xq = Mqi[mi][r] + fr[r] * Mq[t][mi][r];
        const float xm = fe[r] * M2[t][mi][r];
        const float xk = Mk1[mi][r] + xm;
        const float d = G[t][mi][r] - R[t][r];
        vq[r] = exp2_hw(d) * xq;
        vk[r] = exp2_hw(-d) * xk;
        y[mi][r] = qv[r] * xq - kv[r] * xk;
        dkc[r] += kv[r] * xm;
      }
      // dq, dk over the tile's qg, kg pieces (this lane's own, read above)
      const int o = LT<KB>::at(16 * mi, kc) + LT<KB>::acc_pos(lane);
      *reinterpret_cast<uint2*>(sQg + o) = pack4(vq);
      *reinterpret_cast<uint2*>(sKg + o) = pack4(vk);
    }
    // dg = suffix over the rows of y + 2^Gamma sum_v h dh + sum_rows kg Xm
    float add[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float tot = __shfl(row16_prefix(dkc[r]), lane | 15);
      add[r] = exp2_hw(Gm[t][r]) * hdp[r] + tot;
    }
    float run[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int mi = 3; mi >= 0; --mi) {
      float x[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float suf = row16_suffix(y[mi][r]);
        x[r] = suf + run[r] + add[r];
        run[r] += __shfl(suf, lane & 0x30);   // the row group's total (its row 0)
      }
      // dg over the tile's g pieces (read into G before the tiles)
      *reinterpret_cast<uint2*>(sG + LT<KB>::at(16 * mi, kc) + LT<KB>::acc_pos(lane)) =
          pack4(x);
    }
  }
  __syncthreads();   // dq, dk, dg of every key tile in LDS
  // whole row pieces of the slice (partial-line stores of the pieces above are slow)
  const bool ntk = K % 64 == 0;
#pragma unroll
  for (int e = 0; e < PK; ++e) {
    const int pc = tid + NT * e, row = pc / (KB / 8), c8 = 8 * (pc % (KB / 8));
    const int o = LT<KB>::off(row, c8);
    if (row < len && kb + c8 < K) {
      const uint32_t off = ((uint32_t)row * rsK + (uint32_t)(kb + c8)) * 2u;
      st16_sel(dq, off, *reinterpret_cast<const uint4*>(sQg + o), ntk);
      st16_sel(dk, off, *reinterpret_cast<const uint4*>(sKg + o), ntk);
      st16_sel(dg, off, *reinterpret_cast<const uint4*>(sG + o), ntk);
    }
  }
}

// ---------------------------------------------------------------------------
// Fused forward: per chunk (base-2 gates, r = (g~_first + gamma) / 2 per column)
//   qg = q 2^{g~-r}, kg = k 2^{r-g~}, kd = kg 2^{gamma-r}, A = scale tril(qg kg^T),
//   o = A v + qg (scale 2^r h), h <- 2^{gamma} h + kd^T v.
// ---------------------------------------------------------------------------
// KD: kd is staged in LDS (K <= 128). Wider heads (K = 256) do not have the room; their
// update runs on kg with the column factors split around the product:
// h <- 2^{gamma-r} (.) (2^r h + kg^T v)  (= 2^gamma h + kd^T v).
// PRE (wide heads streaming the per-chunk gating workspace): the qg tile holds qs = qg
// (scale 2^r), so h' = h and o = A v + qs h.
// SG (scalar gates): v2 = v 2^{gamma - G_j} for the state update and G (one float per row).
template <int KP, int VP, bool SG = false>
struct HFLayout {
  static constexpr bool KD = KP <= 128;
  static constexpr int qg = 0;
  static constexpr int kg = qg + LT<KP>::bytes(HC);
  static constexpr int kd = kg + LT<KP>::bytes(HC);
  static constexpr int v = kd + (KD ? LT<KP>::bytes(HC) : 0);
  static constexpr int hk = v + LT<VP>::bytes(HC);      // h' [k][v]
  static constexpr int a = hk + LT<VP>::bytes(KP);      // A  [i][j]
  static constexpr int tot = a + LT<HC>::bytes(HC);   // cumsum wave totals (!SG)
  // PRE (no cumsum): the chunk's output tile staged over the totals and the first rows
  static constexpr int ost = tot;
  static constexpr int first = tot + (SG ? 0 : HNW * KP * 4);
  static constexpr int gam = first + KP * 4;
  static constexpr int rsc = gam + KP * 4;
  static constexpr int pre = rsc + KP * 4;        // 2^r          (!KD)
  static constexpr int post = pre + KP * 4;       // 2^{gamma-r}  (!KD)
  static constexpr int v2 = post + KP * 4;        // SG only
  static constexpr int grow = v2 + (SG ? LT<VP>::bytes(HC) : 0);
  static constexpr int bytes = grow + (SG ? HC * 4 : 0);
};

// HO: p.h_out may be set (the PRE build is instantiated without the h residual's code for
// inference calls, which store none).
template <int KP, int VP, bool SG, bool PRE = false, bool HO = true>
__global__ __launch_bounds__(HNT) void head_fwd_kernel(HeadFwdArgs p) {
  using M = HMap<KP>;
  using MV = HMap<VP>;
  using TL = HTiles<KP, VP>;
  using Lay = HFLayout<KP, VP, SG>;
  constexpr int RPT = M::RPT, VRPT = MV::RPT;
  constexpr int NTV = TL::NTV, NTK = TL::NTK;
  // chunks of inputs in flight: two register sets, one for the wide head (K = 256), whose
  // rows take twice the registers (and whose loop body is only inlined once)
  constexpr int PF = KP > 128 ? 1 : 2;
  static_assert(!PRE || (!SG && !Lay::KD), "PRE: wide heads with per-element gates");
  static_assert(Lay::bytes <= 163840, "LDS budget exceeded");
  // o and h out as whole rows (stage_tile, rows_out), staged in the kg tile: it is read by A only
  // (the state update takes kd), so it is free from the barrier before the products to the
  // next chunk's gating, which comes after the cumsum's barrier. Scalar gates stage in the kd
  // tile, which they do not use.
  constexpr bool ROWS = !PRE && Lay::KD && NTV == 4 && HNW * kStgBytes <= LT<KP>::bytes(HC);
  // PRE: o staged in LDS (64 rows, pitch kStgPitch) and stored as whole rows after the next
  // chunk's first barrier; the wave pairs of a row tile each hold half its row
  static_assert(!PRE || HC * kStgPitch * 2 <= Lay::gam - Lay::ost, "PRE output staging");
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  bf16* sQg = reinterpret_cast<bf16*>(smem + Lay::qg);
  bf16* sKg = reinterpret_cast<bf16*>(smem + Lay::kg);
  bf16* sKd = reinterpret_cast<bf16*>(smem + Lay::kd);
  bf16* sV = reinterpret_cast<bf16*>(smem + Lay::v);
  bf16* sHk = reinterpret_cast<bf16*>(smem + Lay::hk);
  bf16* sA = reinterpret_cast<bf16*>(smem + Lay::a);
  float* sTot = reinterpret_cast<float*>(smem + Lay::tot);
  float* sFirst = reinterpret_cast<float*>(smem + Lay::first);
  float* sGam = reinterpret_cast<float*>(smem + Lay::gam);
  float* sRs = reinterpret_cast<float*>(smem + Lay::rsc);
  float* sPre = reinterpret_cast<float*>(smem + Lay::pre);
  float* sPost = reinterpret_cast<float*>(smem + Lay::post);
  bf16* sV2 = reinterpret_cast<bf16*>(smem + Lay::v2);
  float* sG = reinterpret_cast<float*>(smem + Lay::grow);
  bf16* sOst = reinterpret_cast<bf16*>(smem + Lay::ost);

  const bf16* __restrict__ q = (const bf16*)p.q;
  const bf16* __restrict__ k = (const bf16*)p.k;
  const bf16* __restrict__ v = (const bf16*)p.v;
  const bf16* __restrict__ g = (const bf16*)p.g;
  bf16* __restrict__ o = (bf16*)p.o;
  bf16* __restrict__ hout = HO ? (bf16*)p.h_out : nullptr;
  const int H = p.H, K = p.K, V = p.V;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave index, scalar
  const int L0 = xcd_remap(blockIdx.x, gridDim.x);
  const int VT = (V + VP - 1) / VP;            // V tiles (blocks of one segment and head)
  const int vt = L0 % VT, L = L0 / VT;
  const int cv = vt * VP, Vw = min(VP, V - cv);   // this tile's first column and width
  const int hh = L % H;
  const int s = (L / H) % p.NS;
  const Seg sg = seg_of(p.si, (L / H) / p.NS, s, p.NS, p.SL);
  const int nsteps = sg.ce - sg.cb;
  const long rsK = (long)H * K, rsV = (long)H * V;
  const long KV = (long)K * V;

  const int cg = tid % M::NCG, rs = tid / M::NCG;
  const int vg = tid % MV::NCG, vrs = tid / MV::NCG;
  const bool colA = cg * 8 < K, colB = vg * 8 < Vw;

  // zero A once (its upper triangle is never written); PRE: the column factors past K too
  for (int i = tid; i < LT<HC>::bytes(HC) / 16; i += HNT)
    reinterpret_cast<uint4*>(sA)[i] = make_uint4(0, 0, 0, 0);
  if constexpr (PRE) {
    for (int i = tid; i < KP; i += HNT) sRs[i] = sPre[i] = sPost[i] = 0.f;
  }

  const int vt0 = (w & 1) * NTV, kt0 = (w >> 1) * NTK;
  bf16* sStg = (SG ? sKd : sKg) + w * (kStgBytes / 2);   // ROWS: this wave's staging area
  const bool ntv = V % 64 == 0;              // ROWS: the row pieces are whole lines
  float dmax = 0.f;   // largest |g~ - r| of the factors (base 2): the gate-range check
  f32x4 acc[NTV][NTK];
  {
    if (s > 0)
      load_entry_state<NTV, NTK, false>(acc, p.seg_state, p.seg_gam, sg.seq, s, p.NS, H, hh, K,
                                        Vw, cv, V, vt0, kt0, lane);
    else
      load_state<NTV, NTK>(acc, p.h0 ? p.h0 + ((long)sg.seq * H + hh) * KV + cv : nullptr, K,
                           Vw, vt0, kt0, lane, V);
  }

  struct Regs {
    uint4 q[RPT], k[RPT], g[RPT], v[VRPT];
    float gs;   // SG: the gate of row `lane`
    uint4 a, f;  // PRE: 16 bytes of A, 16 bytes of the factors
  };
  auto issue = [&](int step, Regs& R) {
    const int st = min(step, nsteps - 1);
    const int t0 = sg.bos + (sg.cb + st) * HC;
    const int len = min(HC, sg.eos - t0);
    const long oa = (long)t0 * rsK + (long)hh * K;
    if constexpr (PRE) {
      const unsigned char* ent = (const unsigned char*)p.gate_ws +
                                 ((long)(sg.c0 + sg.cb + st) * H + hh) * gate_ws_entry(K);
      const bf16* gq = (const bf16*)ent;
      hload<RPT>(R.q, gq, (uint32_t)K, rs * RPT, HC, cg * 8, K);
      hload<RPT>(R.k, gq + HC * K, (uint32_t)K, rs * RPT, HC, cg * 8, K);
      R.a = ld16(gq + 2 * HC * K, (uint32_t)tid * 16u);   // 64 x 64 bf16 = 512 x 16 bytes
      R.f = ld16(gq + 2 * HC * K + HC * HC, (uint32_t)min(tid, 3 * K / 4 - 1) * 16u);
      hload<VRPT>(R.v, v + (long)t0 * rsV + (long)hh * V + cv, (uint32_t)rsV, vrs * VRPT, len,
                  vg * 8, Vw);
    } else {
      hload<RPT>(R.q, q + oa, (uint32_t)rsK, rs * RPT, len, cg * 8, K);
      hload<RPT>(R.k, k + oa, (uint32_t)rsK, rs * RPT, len, cg * 8, K);
      if constexpr (SG)
        R.gs = p.gs[(long)(t0 + min(lane, len - 1)) * p.gs_ts + hh];
      else
        hload<RPT>(R.g, g + oa, (uint32_t)rsK, rs * RPT, len, cg * 8, K);
      hload<VRPT>(R.v, v + (long)t0 * rsV + (long)hh * V + cv, (uint32_t)rsV, vrs * VRPT, len,
                  vg * 8, Vw);
    }
  };

  // Per-element gates: a chunk's loads go out in three parts, as in the scans' pass 1: q and
  // k one chunk ahead (after the cumsum), the gates two chunks ahead (after the gating), v
  // one chunk ahead (after the barrier before the output products). All at once they stall
  // the issuing waves until the loads before them drain, with nothing issued under the
  // products (head_fwd 217 -> 195 us, 6 fewer VGPRs; v after the gating's barrier instead:
  // 3 us slower, q and k after the gating: 7 us slower).
  constexpr bool SPLIT = !PRE && !SG && PF == 2;
  auto span1 = [&](int step, int& t0, int& len) {
    const int st = min(step, nsteps - 1);
    t0 = sg.bos + (sg.cb + st) * HC;
    len = min(HC, sg.eos - t0);
  };
  auto issue_qk = [&](int step, Regs& R) {
    int t0, len;
    span1(step, t0, len);
    const long oa = (long)t0 * rsK + (long)hh * K;
    hload<RPT>(R.q, q + oa, (uint32_t)rsK, rs * RPT, len, cg * 8, K);
    hload<RPT>(R.k, k + oa, (uint32_t)rsK, rs * RPT, len, cg * 8, K);
  };
  auto issue_g = [&](int step, Regs& R) {
    int t0, len;
    span1(step, t0, len);
    hload<RPT>(R.g, g + (long)t0 * rsK + (long)hh * K, (uint32_t)rsK, rs * RPT, len, cg * 8, K);
  };
  auto issue_v = [&](int step, Regs& R) {
    int t0, len;
    span1(step, t0, len);
    hload<VRPT>(R.v, v + (long)t0 * rsV + (long)hh * V + cv, (uint32_t)rsV, vrs * VRPT, len,
                vg * 8, Vw);
  };
  // PRE: the next chunk's gating-workspace loads in two parts (qg, A and the factors once
  // this chunk's tiles are in LDS, kg and v after the barrier before the output products):
  // all eleven at once queue behind each other and stall the issuing waves (the later four
  // waves of a block ~2000 cycles each chunk)
  auto pre_entry = [&](int step) {
    const int st = min(step, nsteps - 1);
    return (const bf16*)((const unsigned char*)p.gate_ws +
                         ((long)(sg.c0 + sg.cb + st) * H + hh) * gate_ws_entry(K));
  };
  auto issue_pq = [&](int step, Regs& R) {
    const bf16* gq = pre_entry(step);
    hload<RPT>(R.q, gq, (uint32_t)K, rs * RPT, HC, cg * 8, K);
    R.a = ld16(gq + 2 * HC * K, (uint32_t)tid * 16u);
    R.f = ld16(gq + 2 * HC * K + HC * HC, (uint32_t)min(tid, 3 * K / 4 - 1) * 16u);
  };
  auto issue_pk = [&](int step, Regs& R) {
    hload<RPT>(R.k, pre_entry(step) + HC * K, (uint32_t)K, rs * RPT, HC, cg * 8, K);
    issue_v(step, R);
  };
  // PRE: the staged output tile of chunk `step` to HBM, one 16-byte row piece a thread
  auto o_out = [&](int step) {
    static_assert(!PRE || HC * VP / 8 == HNT, "one piece a thread");
    const int t0s = sg.bos + (sg.cb + step) * HC, lens = min(HC, sg.eos - t0s);
    // lanes past the chunk or the tile store the last row / piece again (the same bytes to the
    // same address), so that no per-lane branch surrounds the stores (with it and the h
    // residual's: 282 against 271 us for the kernel at C5). Vw and K are multiples of 8 here.
    const int r = min(tid / (VP / 8), lens - 1), c8 = min(8 * (tid % (VP / 8)), Vw - 8);
    const uint4 x = *reinterpret_cast<const uint4*>(sOst + r * kStgPitch + c8);
    st16_sel(o + (long)t0s * rsV + (long)hh * V + cv, ((uint32_t)r * (uint32_t)rsV + c8) * 2u, x,
             ntv);
  };
  // R: this chunk's registers; Rn: the next chunk's (SPLIT: its q, k and v issued here)
  auto body = [&](int step, Regs& R, Regs& Rn) {
    // lane taken through opaque() every chunk: the per-lane LDS offsets are recomputed in
    // the loop instead of held in registers across it
    const int ln = (int)opaque((uint32_t)lane);
    const int ci = sg.cb + step;
    const int t0 = sg.bos + ci * HC;
    const int len = min(HC, sg.eos - t0);
    // h_n to HBM first: the vector memory path is idle here (the next chunk's loads are
    // issued at the end of the gating, and stores queued behind them wait for them). PRE
    // copies it from h' in LDS as whole rows instead, after the output products
    if (hout && !PRE) {
      bf16* hb = hout + ((long)(sg.c0 + ci) * H + hh) * KV + cv;
      if constexpr (ROWS) {
#pragma unroll
        for (int j = 0; j < NTK; ++j) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            stage_tile(sStg, i,
                       make_uint2(pack2_bf16(acc[i][j][0], acc[i][j][1]),
                                  pack2_bf16(acc[i][j][2], acc[i][j][3])), ln);
          rows_out(sStg, hb + (long)((kt0 + j) * 16) * V + vt0 * 16, (uint32_t)V,
                   K - (kt0 + j) * 16, Vw - vt0 * 16, ntv, ln);
        }
      } else {
        store_state_bf16<NTV, NTK>(acc, hb, K, Vw, vt0, kt0, lane, V);
      }
    }

    // ---- (1) cumsum, gating ----
    float Gl = 0.f, gam_s = 0.f;   // SG: G of row `lane`, the chunk's total (base 2)
    if constexpr (PRE) {   // gated tiles, A and factors as made by head_gate_kernel
      __syncthreads();   // the previous chunk's reads of the tiles are done
#pragma unroll
      for (int j = 0; j < RPT; ++j) {   // (rows past the chunk are zeros in the workspace)
        const int row = rs * RPT + j;
        *reinterpret_cast<uint4*>(sQg + LT<KP>::off(row, cg * 8)) = mask16(R.q[j], colA ? ~0u : 0u);
        *reinterpret_cast<uint4*>(sKg + LT<KP>::off(row, cg * 8)) = mask16(R.k[j], colA ? ~0u : 0u);
      }
#pragma unroll
      for (int j = 0; j < VRPT; ++j) {
        const int row = vrs * VRPT + j;
        *reinterpret_cast<uint4*>(sV + LT<VP>::off(row, vg * 8)) =
            mask16(R.v[j], (colB && row < len) ? ~0u : 0u);
      }
      *reinterpret_cast<uint4*>(sA + LT<HC>::off(tid >> 3, (tid & 7) * 8)) = R.a;
      if (tid < 3 * K / 4) {   // factors: scale 2^r, 2^r, 2^{gamma-r} (K floats each)
        const int i4 = tid * 4, which = i4 / K, col = i4 % K;
        const int off = which == 0 ? Lay::rsc : which == 1 ? Lay::pre : Lay::post;
        *reinterpret_cast<uint4*>(smem + off + col * 4) = R.f;
      }
      // the previous chunk's output (after this chunk's tile stores: their wait for the
      // loads would otherwise also wait for these stores)
      if (step > 0) o_out(step - 1);
    } else if constexpr (SG) {
      // scalar gates: A's decay 2^{G_i - G_j} is applied after q k^T, the inter term's 2^{G_i}
      // after q h', and the update runs on v 2^{gamma - G_j}; every factor is <= 1 for
      // decaying gates, whatever their size
      __syncthreads();   // the previous chunk's reads of the tiles are done
      Gl = sg_row_cumsum(R.gs, lane, len);
      gam_s = __shfl(Gl, len - 1);
#pragma unroll
      for (int j = 0; j < RPT; ++j) {
        const int row = rs * RPT + j;
        const uint32_t m = (colA && row < len) ? ~0u : 0u;
        *reinterpret_cast<uint4*>(sQg + LT<KP>::off(row, cg * 8)) = mask16(R.q[j], m);
        *reinterpret_cast<uint4*>(sKg + LT<KP>::off(row, cg * 8)) = mask16(R.k[j], m);
      }
#pragma unroll
      for (int j = 0; j < VRPT; ++j) {
        const int row = vrs * VRPT + j;
        const uint4 vm = mask16(R.v[j], (colB && row < len) ? ~0u : 0u);
        *reinterpret_cast<uint4*>(sV + LT<VP>::off(row, vg * 8)) = vm;
        const float f = exp2_hw(gam_s - __shfl(Gl, row));
        float x[8];
        unpack8(vm, x);
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] *= f;
        *reinterpret_cast<uint4*>(sV2 + LT<VP>::off(row, vg * 8)) = pack8(x);
      }
      if (w == 0) sG[lane] = Gl;
      if (rs == 0) {
        float eg[8], er[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          eg[e] = exp2_hw(gam_s);
          er[e] = p.scale;
        }
        st_f8(sGam + cg * 8, eg);
        st_f8(sRs + cg * 8, er);
      }
    } else {
      // zero the rows past the chunk and the columns past the tile (a sequence's partial last
      // chunk, narrow heads); full chunks skip it
      if (!(len == HC && K == KP && Vw == VP)) {
        mask_rows<RPT>(R.g, rs * RPT, len, colA);
        mask_rows<RPT>(R.q, rs * RPT, len, colA);
        mask_rows<RPT>(R.k, rs * RPT, len, colA);
        mask_rows<VRPT>(R.v, vrs * VRPT, len, colB);
      }
      float gt[RPT][8], gam[8], first[8];
      head_cumsum<KP>(R.g, gt, gam, first, sTot, sFirst, cg, rs, lane, w);
      if constexpr (SPLIT) issue_qk(step + 1, Rn);
      float r[8], fkd[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        r[e] = 0.5f * (first[e] + gam[e]);
        fkd[e] = exp2_hw(gam[e] - r[e]);
      }
#pragma unroll
      for (int j = 0; j < RPT; ++j) {
        const int row = rs * RPT + j;
        float xq[8], xk[8], xd[8];
        unpack8(R.q[j], xq);
        unpack8(R.k[j], xk);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = gt[j][e] - r[e];
          dmax = fmaxf(dmax, fabsf(d));
          xq[e] *= exp2_hw(d);
          xk[e] *= exp2_hw(-d);
          xd[e] = xk[e] * fkd[e];
        }
        *reinterpret_cast<uint4*>(sQg + LT<KP>::off(row, cg * 8)) = pack8(xq);
        *reinterpret_cast<uint4*>(sKg + LT<KP>::off(row, cg * 8)) = pack8(xk);
        if (Lay::KD) *reinterpret_cast<uint4*>(sKd + LT<KP>::off(row, cg * 8)) = pack8(xd);
      }
#pragma unroll
      for (int j = 0; j < VRPT; ++j) {
        const int row = vrs * VRPT + j;
        *reinterpret_cast<uint4*>(sV + LT<VP>::off(row, vg * 8)) = R.v[j];
      }
      if (rs == 0) {
        float eg[8], er[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          eg[e] = exp2_hw(gam[e]);
          er[e] = p.scale * exp2_hw(r[e]);
        }
        st_f8(sGam + cg * 8, eg);
        st_f8(sRs + cg * 8, er);
        if (!Lay::KD) {
          float ep[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) ep[e] = exp2_hw(r[e]);
          st_f8(sPre + cg * 8, ep);
          st_f8(sPost + cg * 8, fkd);
        }
      }
    }
    if constexpr (SPLIT)
      issue_g(step + 2, R);
    else if constexpr (PRE && PF == 1)
      issue_pq(step + 1, R);
    else
      issue(step + PF, R);
    __syncthreads();

    // ---- (2) A (lower tiles), h' = scale 2^r h into LDS ----
    for (int t = w; t < (PRE ? 0 : 10); t += HNW) {
      const int mi = t < 1 ? 0 : t < 3 ? 1 : t < 6 ? 2 : 3;
      const int ni = t - mi * (mi + 1) / 2;
      f32x4 at = zero4();
      mma_rr_b<KP, KP, KP>(at, sQg, mi * 16, sKg, ni * 16, ln);
      const int jj = ni * 16 + (lane & 15);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int ii = mi * 16 + 4 * (lane >> 4) + rr;
        float a = at[rr] * p.scale;
        if constexpr (SG) a *= exp2_hw(jj <= ii ? sG[ii] - sG[jj] : 0.f);
        sA[LT<HC>::off(ii, jj)] = from_f32<bf16>(jj <= ii ? a : 0.f);
      }
    }
    // (PRE: h' = h, the workspace's qs carrying the column factor scale 2^r)
    const int oacc = LT<VP>::acc_pos(ln);
#pragma unroll
    for (int j = 0; j < NTK; ++j) {
      const int kk = (kt0 + j) * 16 + (lane & 15);
      const float f = PRE ? 1.f : sRs[kk];
#pragma unroll
      for (int i = 0; i < NTV; ++i) {
        *reinterpret_cast<uint2*>(sHk + LT<VP>::at((kt0 + j) * 16, (vt0 + i) * 16) + oacc) =
            make_uint2(pack2_bf16(acc[i][j][0] * f, acc[i][j][1] * f),
                       pack2_bf16(acc[i][j][2] * f, acc[i][j][3] * f));
      }
    }
    __syncthreads();
    if constexpr (SPLIT) issue_v(step + 1, Rn);
    if constexpr (PRE && PF == 1) {
      issue_pk(step + 1, R);
      // kept ahead of the output products: scheduled among them, the loads stall the later
      // waves' MFMA issue and arrive later
      __builtin_amdgcn_sched_barrier(0);
    }

    // ---- (3) o^T = v^T A^T + h'^T qg^T (wave: v tiles of half w&1, row tile w>>1) ----
    {
      const int it = w >> 1;
      // per-element gates: the row fragments of A and qg of row tile it, shared by the wave's
      // v tiles, read once (scalar gates read them per tile: hoisted they measured slower)
      Frag<bf16> fa[SG ? 1 : HC / 32], fq[SG ? 1 : KP / 32];
      if constexpr (!SG) {
#pragma unroll
        for (int kk = 0; kk < HC / 32; ++kk)
          fa[kk] = ldr(sA, LT<HC>::at(it * 16, kk * 32) + LT<HC>::row_frag(ln));
#pragma unroll
        for (int kk = 0; kk < KP / 32; ++kk)
          fq[kk] = ldr(sQg, LT<KP>::at(it * 16, kk * 32) + LT<KP>::row_frag(ln));
      }
      f32x4 ot[NTV];
      if constexpr (SG) {
#pragma unroll
        for (int i = 0; i < NTV; ++i) {   // inter term first, scaled by 2^{G_i} (column i of o^T)
          const int vt = vt0 + i;
          ot[i] = zero4();
          mma_tr<VP, KP>(ot[i], sHk, vt * 16, sQg, it * 16, KP, ln);
          ot[i] *= exp2_hw(sG[it * 16 + (lane & 15)]);
          mma_tr<VP, HC>(ot[i], sV, vt * 16, sA, it * 16, HC, ln);
        }
      } else {
        // v^T A^T + h'^T qg^T for the wave's NTV v tiles at once: per k step the NTV
        // transposed fragments are read together, then the NTV products (independent
        // accumulators) issue back to back
#pragma unroll
        for (int i = 0; i < NTV; ++i) ot[i] = zero4();
#pragma unroll
        for (int kk = 0; kk < HC / 32; ++kk) {
          Frag<bf16> x[NTV];
#pragma unroll
          for (int i = 0; i < NTV; ++i)
            x[i] = ldt<VP>(sV, LT<VP>::at(kk * 32, (vt0 + i) * 16) + LT<VP>::tr_frag(ln));
#pragma unroll
          for (int i = 0; i < NTV; ++i) mma(ot[i], x[i], fa[kk]);
        }
#pragma unroll
        for (int kk = 0; kk < KP / 32; ++kk) {
          Frag<bf16> x[NTV];
#pragma unroll
          for (int i = 0; i < NTV; ++i)
            x[i] = ldt<VP>(sHk, LT<VP>::at(kk * 32, (vt0 + i) * 16) + LT<VP>::tr_frag(ln));
#pragma unroll
          for (int i = 0; i < NTV; ++i) mma(ot[i], x[i], fq[kk]);
        }
      }
#pragma unroll
      for (int i = 0; i < NTV; ++i) {
        const int vt = vt0 + i;
        const uint2 ox =
            make_uint2(pack2_bf16(ot[i][0], ot[i][1]), pack2_bf16(ot[i][2], ot[i][3]));
        if constexpr (ROWS) {
          stage_tile(sStg, i, ox, ln);
        } else if constexpr (PRE) {
          *reinterpret_cast<uint2*>(sOst + (it * 16 + (lane & 15)) * kStgPitch + vt * 16 +
                                    4 * (lane >> 4)) = ox;
        } else {
          const int row = it * 16 + (lane & 15);
          const int vv = vt * 16 + 4 * (lane >> 4);
          if (row < len && vv < Vw)
            st8(o + (long)t0 * rsV + (long)hh * V + cv,
                ((uint32_t)row * (uint32_t)rsV + vv) * 2u, ox);
        }
      }
      if constexpr (ROWS)
        rows_out(sStg, o + (long)(t0 + it * 16) * rsV + (long)hh * V + cv + vt0 * 16,
                 (uint32_t)rsV, len - it * 16, Vw - vt0 * 16, ntv, ln);
    }
    if constexpr (PRE) {
      // the h residual (the state entering the chunk, bf16) as whole rows of h' in LDS: the
      // accumulators' 8-byte pieces (32 bytes of a row a store) cost ~40 % of the chunk at C5.
      // Plain stores: nontemporal ones measured 7 % slower for this kernel at C5 (303 against
      // 282 us), though the o rows and the scans' states gain from them. Lanes past the head or
      // the tile store the last row / piece again, as in o_out: no branch around the stores.
      if constexpr (HO) {
        bf16* hb = hout + ((long)(sg.c0 + ci) * H + hh) * KV + cv;
        constexpr int PR = VP / 8;   // 16-byte pieces of a row
#pragma unroll
        for (int j = 0; j < KP * PR / HNT; ++j) {
          const int pc = tid + HNT * j, r = min(pc / PR, K - 1), c8 = min((pc % PR) * 8, Vw - 8);
          const uint4 x = *reinterpret_cast<const uint4*>(sHk + LT<VP>::off(r, c8));
          st16(hb, ((uint32_t)r * (uint32_t)V + c8) * 2u, x);
        }
      }
    }
    if constexpr (SG)
      state_update<NTV, NTK, VP, KP>(acc, sV2, sKg, sGam, vt0, kt0, ln);
    else if (Lay::KD)
      state_update<NTV, NTK, VP, KP>(acc, sV, sKd, sGam, vt0, kt0, ln);
    else
      state_update<NTV, NTK, VP, KP>(acc, sV, sKg, sPre, vt0, kt0, ln, sPost);
  };

  if (nsteps > 0 && PF == 2) {
    // both register sets every trip (the odd chunk after the loop): entered and taken again
    // with the same outstanding loads, so a chunk's waits leave the next chunk's in flight
    Regs R0, R1;
    issue(0, R0);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (SPLIT)
      issue_g(1, R1);
    else
      issue(1, R1);
    int step = 0;
    for (; step + 1 < nsteps; step += 2) {
      body(step, R0, R1);
      body(step + 1, R1, R0);
    }
    if (step < nsteps) body(step, R0, R1);
  } else if (nsteps > 0) {
    Regs R0;
    issue(0, R0);
    // the first chunk's loads waited for here (as in the backward): the loop's wait for a
    // chunk's loads, sized for this entry, would otherwise also wait on every later trip for
    // the previous chunk's h residual stores
    if constexpr (PRE) vm_wait_all();
    for (int step = 0; step < nsteps; ++step) body(step, R0, R0);
    if constexpr (PRE) {
      __syncthreads();   // the last chunk's output tile in LDS
      o_out(nsteps - 1);
    }
  }

  if (s == p.NS - 1 && p.ht)
    store_state_f32<NTV, NTK>(acc, p.ht + ((long)sg.seq * H + hh) * KV + cv, K, Vw, vt0, kt0,
                              lane, V);
  if (p.flags) {   // uniform; every block writes its flag, so nothing needs clearing
    const int bad = __syncthreads_or(dmax > kGateLimit2 ? 1 : 0);
    if (tid == 0) p.flags[L0] = bad ? 1 : 0;
  }
}


// ---------------------------------------------------------------------------
// Fused backward: one block per (sequence, segment, head) walks the segment's chunks in
// reverse with the state gradient dh (state leaving the chunk) in MFMA accumulators.
// Reference: chunk_gla_bwd_with_pl, tops/ops/gla/chunk.py:1019-1064 (dh scan
// chunk_h.py:495-591, fused gradients chunk.py:1423-1479). Per chunk, base-2 gates,
// r = (g~_first + gamma) / 2 per column, fr = scale 2^r, fe = 2^{gamma-r}:
//   qg = q 2^{g~-r}, kg = k 2^{r-g~}, dh' = fe (.) dh (rows k; kd = k 2^{gamma-g~} = kg fe)
//   A = scale tril(qg kg^T), dA = scale tril(do v^T)
//   dv = A^T do + kg dh'
//   dq = 2^{g~-r} [dA kg + fr do h^T]
//   dk = 2^{r-g~} [dA^T qg + v dh'^T]
//   dg = revcumsum_rows(q dq - k dk) + 2^r sum_v h dh' + sum_rows kg (.) (v dh'^T)
//   dh <- 2^gamma dh + (scale q 2^{g~})^T do
// (2^r sum_v h dh' = 2^gamma sum_v h dh; the last term is sum_rows k dk_inter, summed from
// the dk pre-factor while it is still in registers.)
// h (state entering the chunk) comes from the forward's per-chunk states; its MFMA
// fragments are read straight from HBM (16 bytes per lane).
// Waves: dq/dk own KTW k tiles x RT row tiles, dv^T VTW v tiles x JT row tiles, dh as in
// the scans. The next chunk's gates (needed first, by the cumsum) are fetched during the
// epilogue; its q, k, v and do when it starts (the cumsum runs under those loads) and h --
// needed last, in the second phase -- once dh' is in LDS, so that the vector memory path
// takes a chunk's loads in two smaller bursts (all waves issuing 14 loads at once kept them
// stalled for about 10 % of the chunk). There are no registers to hold more of the next
// chunk in flight: prefetching q and k (or v and do) as well spilled and measured slower.
// ---------------------------------------------------------------------------
// SG (scalar gates): q2 = scale q 2^{G_i} for the dh update and G (one float per row).
template <int KP, int VP, int NW, bool SG = false>
struct HBLayout {
  static constexpr int PX = KP + 4;                // fp32 exchange pitch
  // element (r, c) of an exchange array: the float4 halves of each 8-column group swapped in
  // rows with bit 1 set. A wave's row reads (8 columns a lane, two rows two apart) then hit
  // every bank once per group of 16 lanes (2-way conflicts unswizzled); the accumulator-layout
  // writes (rows r, r + 4, r + 8, r + 12) stay conflict-free.
  __device__ static int xo(int r, int c) { return r * PX + (c ^ (4 * ((r >> 1) & 1))); }
  // small fp32 arrays first: the exchange aliases the tiles only
  // row groups of the dq / dk tiles (waves sharing a k tile)
  static constexpr int NKT = KP / 16, KTW = NKT > NW ? NKT / NW : 1, NRG = NW / (NKT / KTW);
  static constexpr int tot = 0;                    // [NW][KP] cumsum wave totals (!SG)
  static constexpr int suf = tot + (SG ? 0 : NW * KP * 4);   // [NRG][KP] dg row-group totals
  static constexpr int first = suf + NRG * KP * 4;
  static constexpr int fr = first + KP * 4;        // scale 2^r
  static constexpr int fe = fr + KP * 4;           // 2^{gamma-r}
  static constexpr int dkc = fe + KP * 4;          // [NRG][KP] sum_rows kg (v dh'^T)
  static constexpr int qg = dkc + NRG * KP * 4;
  static constexpr int kg = qg + LT<KP>::bytes(HC);
  static constexpr int v = kg + LT<KP>::bytes(HC);
  static constexpr int dout = v + LT<VP>::bytes(HC);
  static constexpr int dh = dout + LT<VP>::bytes(HC);   // dh' [k][v] bf16
  static constexpr int a = dh + LT<VP>::bytes(KP);
  static constexpr int da = a + LT<HC>::bytes(HC);
  static constexpr int q2 = da + LT<HC>::bytes(HC);     // SG only
  static constexpr int grow = q2 + (SG ? LT<KP>::bytes(HC) : 0);
  static constexpr int end_tiles = grow + (SG ? HC * 4 : 0);
  // exchange [HC][PX] x 3 (dq, dk pre-factors, dg) from v on (qg, kg stay intact for the
  // epilogue); it may reach A / dA, which are therefore rewritten in full (zero upper tiles)
  // every chunk
  static constexpr int xq = v;
  static constexpr int xk = xq + HC * PX * 4;
  static constexpr int xg = xk + HC * PX * 4;
  static constexpr int end_x = xg + HC * PX * 4;
  static constexpr int bytes = end_tiles > end_x ? end_tiles : end_x;
};

// The 8 floats of columns c..c+7 (c a multiple of 8) of row r of an exchange array (HBLayout::xo).
template <class Lay>
__device__ __forceinline__ void ld_x8(const float* x, int r, int c, float (&v)[8]) {
  const float4 a = *reinterpret_cast<const float4*>(x + Lay::xo(r, c));
  const float4 b = *reinterpret_cast<const float4*>(x + Lay::xo(r, c + 4));
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

template <int KP, int VP, int NT, bool SG>
__global__ __launch_bounds__(NT) void head_bwd_kernel(HeadBwdArgs p) {
  constexpr int NW = NT / 64;
  using M = HMap<KP, NT>;
  using MV = HMap<VP, NT>;
  using Lay = HBLayout<KP, VP, NW, SG>;
  constexpr int RPT = M::RPT, VRPT = MV::RPT;
  constexpr int NKT = KP / 16, NVT = VP / 16;
  // dh tiles per wave: v by halves (w & 1), k split over the NW / 2 wave pairs
  constexpr int NTV = VP / 32, NTK = NKT / (NW / 2);
  // dq / dk: KTW k tiles x RT row tiles per wave; dv^T: VTW v tiles x JT row tiles
  constexpr int KTW = NKT > NW ? NKT / NW : 1, NKG = NKT / KTW, RT = 4 * NKG / NW;
  constexpr int VTW = NVT > NW ? NVT / NW : 1, NVG = NVT / VTW, JT = 4 * NVG / NW;
  static_assert(NTK >= 1 && RT >= 1 && JT >= 1, "tile split");
  static_assert(Lay::NRG == NW / NKG, "row groups of the dq / dk tiles");
  constexpr int NHF = VP / 32;                      // h fragments per lane
  static_assert(Lay::bytes <= 163840, "LDS budget exceeded");
  // dv out as whole rows (stage_tile, rows_out): a wave takes row tile w >> 1 and the v tiles
  // of half w & 1, staged in the v tile, which nothing reads after the A / dA products.
  // Plain, its 32-byte pieces leave dirty L2 lines whose writeback delays the next launch
  // (the next forward's pass 1: 11 us).
  constexpr bool ROWS = VP == 128 && NW == 8 && NW * kStgBytes <= LT<VP>::bytes(HC);
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  float* sTot = reinterpret_cast<float*>(smem + Lay::tot);
  float* sSuf = reinterpret_cast<float*>(smem + Lay::suf);
  float* sFirst = reinterpret_cast<float*>(smem + Lay::first);
  float* sFr = reinterpret_cast<float*>(smem + Lay::fr);
  float* sFe = reinterpret_cast<float*>(smem + Lay::fe);
  float* sDkc = reinterpret_cast<float*>(smem + Lay::dkc);
  bf16* sQg = reinterpret_cast<bf16*>(smem + Lay::qg);
  bf16* sKg = reinterpret_cast<bf16*>(smem + Lay::kg);
  bf16* sV = reinterpret_cast<bf16*>(smem + Lay::v);
  bf16* sDo = reinterpret_cast<bf16*>(smem + Lay::dout);
  bf16* sDh = reinterpret_cast<bf16*>(smem + Lay::dh);
  bf16* sA = reinterpret_cast<bf16*>(smem + Lay::a);
  bf16* sdA = reinterpret_cast<bf16*>(smem + Lay::da);
  float* XQ = reinterpret_cast<float*>(smem + Lay::xq);
  float* XK = reinterpret_cast<float*>(smem + Lay::xk);
  float* XG = reinterpret_cast<float*>(smem + Lay::xg);
  bf16* sQ2 = reinterpret_cast<bf16*>(smem + Lay::q2);
  float* sG = reinterpret_cast<float*>(smem + Lay::grow);

  const bf16* __restrict__ q = (const bf16*)p.q;
  const bf16* __restrict__ k = (const bf16*)p.k;
  const bf16* __restrict__ v = (const bf16*)p.v;
  const bf16* __restrict__ g = (const bf16*)p.g;
  const bf16* __restrict__ dout = (const bf16*)p.dout;
  const bf16* __restrict__ hs = (const bf16*)p.h;
  bf16* __restrict__ dq = (bf16*)p.dq;
  bf16* __restrict__ dk = (bf16*)p.dk;
  bf16* __restrict__ dv = (bf16*)p.dv;
  bf16* __restrict__ dg = (bf16*)p.dg;
  const int H = p.H, K = p.K, V = p.V;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave index, scalar
  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int hh = L % H;
  const int s = (L / H) % p.NS;
  const Seg sg = seg_of(p.si, (L / H) / p.NS, s, p.NS, p.SL);
  const int nsteps = sg.ce - sg.cb;
  const long rsK = (long)H * K, rsV = (long)H * V;
  const long KV = (long)K * V;
  const float inv_scale = 1.f / p.scale;   // uniform

  const int cg = tid % M::NCG, rs = tid / M::NCG;
  const int vg = tid % MV::NCG, vrs = tid / MV::NCG;
  const bool colA = cg * 8 < K, colB = vg * 8 < V;
  const int kq0 = (w % NKG) * KTW, rt0 = (w / NKG) * RT;   // dq / dk tiles
  const int vd0 = (w % NVG) * VTW, jt0 = (w / NVG) * JT;   // dv^T tiles

  const int vt0 = (w & 1) * NTV, kt0 = (w >> 1) * NTK;
  const bool full_kv = K == KP && V == VP;   // no column of the tiles lies past the head
  // dq, dk, dg (16 lanes a row) and dv (staged as whole rows, ROWS) stored nontemporally
  // where their row pieces are whole 128-byte lines
  const bool ntk = K % 64 == 0, ntv = V % 64 == 0;
  int gbad = 0;          // uniform: a chunk had a factor beyond the gate-range limit
  f32x4 acc[NTV][NTK];   // dh[v][k]
  {
    if (s < p.NS - 1)
      load_entry_state<NTV, NTK, true>(acc, p.seg_state, p.seg_gam, sg.seq, s, p.NS, H, hh, K, V,
                                       0, V, vt0, kt0, lane);
    else
      load_state<NTV, NTK>(acc, p.dht ? p.dht + ((long)sg.seq * H + hh) * KV : nullptr, K, V,
                           vt0, kt0, lane);
  }

  uint4 Rq[RPT], Rk[RPT], Rg[RPT], Rv[VRPT], Rd[VRPT], Rh[KTW][NHF];
  float Rs = 0.f;   // SG: the gate of row `lane`
  auto chunk_of = [&](int step, int& t0, int& len, int& ci) {
    ci = sg.ce - 1 - min(step, nsteps - 1);
    t0 = sg.bos + ci * HC;
    len = min(HC, sg.eos - t0);
  };
  auto issue_qk = [&](int step) {
    int t0, len, ci;
    chunk_of(step, t0, len, ci);
    const long oa = (long)t0 * rsK + (long)hh * K;
    hload<RPT>(Rq, q + oa, (uint32_t)rsK, rs * RPT, len, cg * 8, K);
    hload<RPT>(Rk, k + oa, (uint32_t)rsK, rs * RPT, len, cg * 8, K);
  };
  auto issue_g = [&](int step) {
    int t0, len, ci;
    chunk_of(step, t0, len, ci);
    const long oa = (long)t0 * rsK + (long)hh * K;
    if constexpr (SG)
      Rs = p.gs[(long)(t0 + min(lane, len - 1)) * p.gs_ts + hh];
    else
      hload<RPT>(Rg, g + oa, (uint32_t)rsK, rs * RPT, len, cg * 8, K);
  };
  auto issue_vd = [&](int step) {
    int t0, len, ci;
    chunk_of(step, t0, len, ci);
    const long ov = (long)t0 * rsV + (long)hh * V;
    hload<VRPT>(Rv, v + ov, (uint32_t)rsV, vrs * VRPT, len, vg * 8, V);
    hload<VRPT>(Rd, dout + ov, (uint32_t)rsV, vrs * VRPT, len, vg * 8, V);
  };
  auto issue_h = [&](int step) {
    int t0, len, ci;
    chunk_of(step, t0, len, ci);
    const bf16* hc = hs + ((long)(sg.c0 + ci) * H + hh) * KV;
#pragma unroll
    for (int t = 0; t < KTW; ++t) {
      const uint32_t hrow = (uint32_t)min((kq0 + t) * 16 + (lane & 15), K - 1) * (uint32_t)V;
#pragma unroll
      for (int f = 0; f < NHF; ++f)
        Rh[t][f] = ld16(hc, (hrow + (uint32_t)min(f * 32 + 8 * (lane >> 4), V - 8)) * 2u);
    }
  };


  if (nsteps > 0) issue_g(0);
  // the first gates waited for here: otherwise the loop's wait for the gates (in the
  // cumsum), sized for this entry, counts back over the previous chunk's stores and
  // holds every chunk until those have completed
  vm_wait_all();
  for (int step = 0; step < nsteps; ++step) {
    int t0, len, ci;
    chunk_of(step, t0, len, ci);
    issue_qk(step);
    issue_vd(step);
    // lane / thread indices for the per-lane offsets of the dv, dq, dk, dg stores and of the
    // transposed kg / qg reads: taken through opaque() every chunk so that those offsets are
    // recomputed in the loop (hoisted, they are long-lived registers the kernel cannot hold)
    const int ln = (int)opaque((uint32_t)lane), tl = (int)opaque((uint32_t)tid);

    // ---- (1) cumsum, gating; dh' = fe (.) dh to LDS ----
    float dd[RPT][8];   // g~ - r (base 2)
    float gam_s = 0.f;  // SG: the chunk's total gate (base 2)
    if constexpr (SG) {
      // scalar gates: raw q, k; the pairwise decays go on A and dA, the row factors on the
      // inter terms and on q for the dh update (all <= 1 for decaying gates)
      __syncthreads();   // the previous chunk's epilogue reads are done
      const float Gl = sg_row_cumsum(Rs, lane, len);
      gam_s = __shfl(Gl, len - 1);
      if (step + 1 < nsteps) issue_g(step + 1);   // the next chunk's gates, as below
#pragma unroll
      for (int j = 0; j < NTK; ++j) {
#pragma unroll
        for (int i = 0; i < NTV; ++i) {
          *reinterpret_cast<uint2*>(sDh + LT<VP>::at((kt0 + j) * 16, (vt0 + i) * 16) +
                                    LT<VP>::acc_pos(lane)) =
              make_uint2(pack2_bf16(acc[i][j][0], acc[i][j][1]),
                         pack2_bf16(acc[i][j][2], acc[i][j][3]));
        }
      }
      issue_h(step);
#pragma unroll
      for (int j = 0; j < RPT; ++j) {
        const int row = rs * RPT + j;
        const uint32_t m = (colA && row < len) ? ~0u : 0u;
        const uint4 qm = mask16(Rq[j], m);
        *reinterpret_cast<uint4*>(sQg + LT<KP>::off(row, cg * 8)) = qm;
        *reinterpret_cast<uint4*>(sKg + LT<KP>::off(row, cg * 8)) = mask16(Rk[j], m);
        const float f = p.scale * exp2_hw(__shfl(Gl, row));
        float x[8];
        unpack8(qm, x);
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] *= f;
        *reinterpret_cast<uint4*>(sQ2 + LT<KP>::off(row, cg * 8)) = pack8(x);
      }
#pragma unroll
      for (int j = 0; j < VRPT; ++j) {
        const int row = vrs * VRPT + j;
        const uint32_t m = (colB && row < len) ? ~0u : 0u;
        *reinterpret_cast<uint4*>(sV + LT<VP>::off(row, vg * 8)) = mask16(Rv[j], m);
        *reinterpret_cast<uint4*>(sDo + LT<VP>::off(row, vg * 8)) = mask16(Rd[j], m);
      }
      if (w == 0) sG[lane] = Gl;
      if (rs == 0) {   // fr = scale 2^gamma (the 2^gamma sum_v h dh term), fe = 2^gamma
        float b8[8], c8[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          c8[e] = exp2_hw(gam_s);
          b8[e] = p.scale * c8[e];
        }
        st_f8(sFr + cg * 8, b8);
        st_f8(sFe + cg * 8, c8);
      }
    } else {
      // zero the rows past the chunk and the columns past the tile (a sequence's partial last
      // chunk, narrow heads); full chunks skip it
      if (!(len == HC && full_kv)) {
        mask_rows<RPT>(Rg, rs * RPT, len, colA);
        mask_rows<RPT>(Rq, rs * RPT, len, colA);
        mask_rows<RPT>(Rk, rs * RPT, len, colA);
        mask_rows<VRPT>(Rv, vrs * VRPT, len, colB);
        mask_rows<VRPT>(Rd, vrs * VRPT, len, colB);
      }
      uint4 qm[RPT], km[RPT];
#pragma unroll
      for (int j = 0; j < RPT; ++j) {
        unpack8(Rg[j], dd[j]);
        qm[j] = Rq[j];
        km[j] = Rk[j];
      }
      float gam[8], first[8];
      head_cumsum_f<KP, NT>(dd, gam, first, sTot, sFirst, cg, rs, lane, w);
      // the next chunk's gates: their registers are free once the cumsum has them, and a
      // whole chunk ahead they have arrived by the next cumsum (issued in the epilogue they
      // had not: head_bwd 364 -> 351 us)
      if (step + 1 < nsteps) issue_g(step + 1);
      // gamma of this lane's dh rows from the wave totals (same order of sums as gam)
#pragma unroll
      for (int j = 0; j < NTK; ++j) {
        const int kk = (kt0 + j) * 16 + (lane & 15);
        float gk = 0.f;
#pragma unroll
        for (int ww = 0; ww < NW; ++ww) gk += sTot[ww * KP + kk];
        const float fe = exp2_hw(0.5f * (gk - sFirst[kk]));
#pragma unroll
        for (int i = 0; i < NTV; ++i) {
          *reinterpret_cast<uint2*>(sDh + LT<VP>::at((kt0 + j) * 16, (vt0 + i) * 16) +
                                    LT<VP>::acc_pos(lane)) =
              make_uint2(pack2_bf16(acc[i][j][0] * fe, acc[i][j][1] * fe),
                         pack2_bf16(acc[i][j][2] * fe, acc[i][j][3] * fe));
        }
      }
      issue_h(step);
      float r[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) r[e] = 0.5f * (first[e] + gam[e]);
      float dmax = 0.f;
#pragma unroll
      for (int j = 0; j < RPT; ++j) {
        const int row = rs * RPT + j;
        float xq[8], xk[8];
        unpack8(qm[j], xq);
        unpack8(km[j], xk);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          dd[j][e] -= r[e];
          dmax = fmaxf(dmax, fabsf(dd[j][e]));
          xq[e] *= exp2_hw(dd[j][e]);
          xk[e] *= exp2_hw(-dd[j][e]);
        }
        *reinterpret_cast<uint4*>(sQg + LT<KP>::off(row, cg * 8)) = pack8(xq);
        *reinterpret_cast<uint4*>(sKg + LT<KP>::off(row, cg * 8)) = pack8(xk);
      }
      gbad |= __ballot(dmax > kGateLimit2) != 0ull ? 1 : 0;
#pragma unroll
      for (int j = 0; j < VRPT; ++j) {
        const int row = vrs * VRPT + j;
        *reinterpret_cast<uint4*>(sV + LT<VP>::off(row, vg * 8)) = Rv[j];
        *reinterpret_cast<uint4*>(sDo + LT<VP>::off(row, vg * 8)) = Rd[j];
      }
      if (rs == 0) {
        float b8[8], c8[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          b8[e] = p.scale * exp2_hw(r[e]);
          c8[e] = exp2_hw(0.5f * (gam[e] - first[e]));
        }
        st_f8(sFr + cg * 8, b8);
        st_f8(sFe + cg * 8, c8);
      }
    }
    __syncthreads();

    // ---- (2) A, dA (all 16 tiles each: the upper ones as zeros); products that need no
    //      A / dA ----
    for (int t = w; t < 32; t += NW) {
      const int mi = (t >> 2) & 3, ni = t & 3;
      f32x4 at = zero4();
      if (ni <= mi) {
        if (t < 16)
          mma_rr_b<KP, KP, KP>(at, sQg, mi * 16, sKg, ni * 16, lane);
        else
          mma_rr_b<VP, VP, VP>(at, sDo, mi * 16, sV, ni * 16, lane);
      }
      bf16* dst = t < 16 ? sA : sdA;
      const int jj = ni * 16 + (lane & 15);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int ii = mi * 16 + 4 * (lane >> 4) + rr;
        float a = at[rr] * p.scale;
        if constexpr (SG) a *= exp2_hw(jj <= ii ? sG[ii] - sG[jj] : 0.f);   // A, dA decayed
        dst[LT<HC>::off(ii, jj)] = from_f32<bf16>(jj <= ii ? a : 0.f);
      }
    }
    // dq pre: fr do h^T (h fragments from HBM); dk pre: v dh'^T
    f32x4 aq[KTW][RT], ak[KTW][RT];
    float hdp[KTW], dkc[KTW];
#pragma unroll
    for (int t = 0; t < KTW; ++t) {
      const int hk = (kq0 + t) * 16 + (lane & 15);
      hdp[t] = 0.f;
#pragma unroll
      for (int i = 0; i < RT; ++i) aq[t][i] = ak[t][i] = zero4();
#pragma unroll
      for (int f = 0; f < NHF; ++f) {
        Frag<bf16> yh;
        yh.d = full_kv ? Rh[t][f]
                       : mask16(Rh[t][f], (hk < K && f * 32 + 8 * (lane >> 4) < V) ? ~0u : 0u);
        const Frag<bf16> ydh =
            ldr(sDh, LT<VP>::at((kq0 + t) * 16, f * 32) + LT<VP>::row_frag(lane));
        hdp[t] = dot8_bf16(yh.d, ydh.d, hdp[t]);
        // the RT row fragments of do and of v read together, then the 2 RT products
        Frag<bf16> xd[RT], xv[RT];
#pragma unroll
        for (int i = 0; i < RT; ++i) {
          const int o = LT<VP>::at((rt0 + i) * 16, f * 32) + LT<VP>::row_frag(lane);
          xd[i] = ldr(sDo, o);
          xv[i] = ldr(sV, o);
        }
#pragma unroll
        for (int i = 0; i < RT; ++i) {
          mma(aq[t][i], xd[i], yh);
          mma(ak[t][i], xv[i], ydh);
        }
      }
      hdp[t] += __shfl_xor(hdp[t], 16);
      hdp[t] += __shfl_xor(hdp[t], 32);
      if constexpr (SG) {   // row factors: scale 2^{G_i} on do h^T, 2^{gamma - G_j} on v dh^T
#pragma unroll
        for (int i = 0; i < RT; ++i)
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
            const float gr = sG[(rt0 + i) * 16 + 4 * (lane >> 4) + rr];
            aq[t][i][rr] *= p.scale * exp2_hw(gr);
            ak[t][i][rr] *= exp2_hw(gam_s - gr);
          }
      } else {
        const float fr = sFr[hk];
#pragma unroll
        for (int i = 0; i < RT; ++i) aq[t][i] *= fr;
      }
      // sum over this wave's rows of kg (.) ak: kg read in the accumulator layout (rows
      // 4 (lane >> 4) + 0..3 of column lane & 15 of each 16 x 16 tile) by transposed reads
      dkc[t] = 0.f;
#pragma unroll
      for (int i = 0; i < RT; ++i) {
        const bf16* pk = sKg + LT<KP>::at((rt0 + i) * 16, (kq0 + t) * 16) + LT<KP>::tr_rows4(ln);
        const s4_t kv = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s4_t*)(pk));
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          dkc[t] += __uint_as_float((uint32_t)(uint16_t)kv[rr] << 16) * ak[t][i][rr];
      }
      dkc[t] += __shfl_xor(dkc[t], 16);
      dkc[t] += __shfl_xor(dkc[t], 32);
    }

    __syncthreads();

    // ---- (3) products with A / dA; dv out; dh update ----
    // (operand fragments shared by a wave's tiles are read once)
#pragma unroll
    for (int t = 0; t < KTW; ++t) {
      const int kq = kq0 + t;
      Frag<bf16> fk[HC / 32], fq[HC / 32];   // kg^T, qg^T of this k tile
#pragma unroll
      for (int kk = 0; kk < HC / 32; ++kk) {
        const int o = LT<KP>::at(kk * 32, kq * 16) + LT<KP>::tr_frag(lane);
        fk[kk] = ldt<KP>(sKg, o);
        fq[kk] = ldt<KP>(sQg, o);
      }
#pragma unroll
      for (int i = 0; i < RT; ++i) {
        const int ro = (rt0 + i) * 16;
        // dq += dA kg; dk += dA^T qg
#pragma unroll
        for (int kk = 0; kk < HC / 32; ++kk) {
          mma(aq[t][i], ldr(sdA, LT<HC>::at(ro, kk * 32) + LT<HC>::row_frag(lane)), fk[kk]);
          mma(ak[t][i], ldt<HC>(sdA, LT<HC>::at(kk * 32, ro) + LT<HC>::tr_frag(lane)), fq[kk]);
        }
      }
    }
    if constexpr (ROWS) {
      // dv^T of row tile w >> 1 and the four v tiles of half w & 1 (independent
      // accumulators, each k step's transposed fragments read together), staged in the v
      // tile and stored as whole rows
      const int jt = w >> 1;
      Frag<bf16> fk[KP / 32], fa[HC / 32];   // kg rows, A^T rows of row tile jt
#pragma unroll
      for (int kk = 0; kk < KP / 32; ++kk)
        fk[kk] = ldr(sKg, LT<KP>::at(jt * 16, kk * 32) + LT<KP>::row_frag(lane));
#pragma unroll
      for (int kk = 0; kk < HC / 32; ++kk)
        fa[kk] = ldt<HC>(sA, LT<HC>::at(kk * 32, jt * 16) + LT<HC>::tr_frag(lane));
      f32x4 avt[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) avt[u] = zero4();
#pragma unroll
      for (int kk = 0; kk < KP / 32; ++kk) {
        Frag<bf16> x[4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
          x[u] = ldt<VP>(sDh, LT<VP>::at(kk * 32, ((w & 1) * 4 + u) * 16) + LT<VP>::tr_frag(lane));
#pragma unroll
        for (int u = 0; u < 4; ++u) mma(avt[u], x[u], fk[kk]);
      }
      if constexpr (SG) {
        const float f = exp2_hw(gam_s - sG[jt * 16 + (lane & 15)]);
#pragma unroll
        for (int u = 0; u < 4; ++u) avt[u] *= f;
      }
#pragma unroll
      for (int kk = 0; kk < HC / 32; ++kk) {
        Frag<bf16> x[4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
          x[u] = ldt<VP>(sDo, LT<VP>::at(kk * 32, ((w & 1) * 4 + u) * 16) + LT<VP>::tr_frag(lane));
#pragma unroll
        for (int u = 0; u < 4; ++u) mma(avt[u], x[u], fa[kk]);
      }
      bf16* sStg = sV + w * (kStgBytes / 2);
#pragma unroll
      for (int u = 0; u < 4; ++u)
        stage_tile(sStg, u,
                   make_uint2(pack2_bf16(avt[u][0], avt[u][1]), pack2_bf16(avt[u][2], avt[u][3])),
                   ln);
      rows_out(sStg, dv + (long)(t0 + jt * 16) * rsV + (long)hh * V + (w & 1) * 64,
               (uint32_t)rsV, len - jt * 16, V - (w & 1) * 64, ntv, ln);
    }
#pragma unroll
    for (int u = 0; u < (ROWS ? 0 : VTW); ++u) {
      const int vd = vd0 + u;
      Frag<bf16> fh[KP / 32], fd[HC / 32];   // dh'^T, do^T of this v tile
#pragma unroll
      for (int kk = 0; kk < KP / 32; ++kk)
        fh[kk] = ldt<VP>(sDh, LT<VP>::at(kk * 32, vd * 16) + LT<VP>::tr_frag(lane));
#pragma unroll
      for (int kk = 0; kk < HC / 32; ++kk)
        fd[kk] = ldt<VP>(sDo, LT<VP>::at(kk * 32, vd * 16) + LT<VP>::tr_frag(lane));
#pragma unroll
      for (int i = 0; i < JT; ++i) {
        const int jt = jt0 + i;
        // dv^T = dh'^T kg^T + do^T A (scalar gates: (dh^T k^T) 2^{gamma - G_j} + do^T A)
        f32x4 avt = zero4();
        Frag<bf16> xk[KP / 32], xa[HC / 32];   // kg rows, A^T rows of row tile jt
#pragma unroll
        for (int kk = 0; kk < KP / 32; ++kk)
          xk[kk] = ldr(sKg, LT<KP>::at(jt * 16, kk * 32) + LT<KP>::row_frag(lane));
#pragma unroll
        for (int kk = 0; kk < HC / 32; ++kk)
          xa[kk] = ldt<HC>(sA, LT<HC>::at(kk * 32, jt * 16) + LT<HC>::tr_frag(lane));
#pragma unroll
        for (int kk = 0; kk < KP / 32; ++kk) mma(avt, fh[kk], xk[kk]);
        if constexpr (SG) avt *= exp2_hw(gam_s - sG[jt * 16 + (lane & 15)]);
#pragma unroll
        for (int kk = 0; kk < HC / 32; ++kk) mma(avt, fd[kk], xa[kk]);
        const int jj = jt * 16 + (lane & 15);
        const int vv = vd * 16 + 4 * (lane >> 4);
        if (jj < len && vv < V) {
          const int jl = jt * 16 + (ln & 15), vl = vd * 16 + 4 * (ln >> 4);
          st8(dv + (long)t0 * rsV + (long)hh * V, ((uint32_t)jl * (uint32_t)rsV + vl) * 2u,
              make_uint2(pack2_bf16(avt[0], avt[1]), pack2_bf16(avt[2], avt[3])));
        }
      }
    }
    // dh <- 2^gamma dh + (scale q 2^{g~})^T do = fr * (dh fe / scale + qg^T do)
    // (scalar gates: 2^gamma dh + q2^T do, q2 = scale q 2^{G})
#pragma unroll
    for (int j = 0; j < NTK; ++j) {
      const float d = SG ? sFe[(kt0 + j) * 16 + (lane & 15)]
                         : sFe[(kt0 + j) * 16 + (lane & 15)] * inv_scale;
#pragma unroll
      for (int i = 0; i < NTV; ++i) acc[i][j] *= d;
    }
    const bf16* sQd = SG ? sQ2 : sQg;
#pragma unroll
    for (int kk = 0; kk < HC; kk += 32) {
      Frag<bf16> x[NTV], y[NTK];
#pragma unroll
      for (int i = 0; i < NTV; ++i)
        x[i] = ldt<VP>(sDo, LT<VP>::at(kk, (vt0 + i) * 16) + LT<VP>::tr_frag(lane));
#pragma unroll
      for (int j = 0; j < NTK; ++j)
        y[j] = ldt<KP>(sQd, LT<KP>::at(kk, (kt0 + j) * 16) + LT<KP>::tr_frag(lane));
#pragma unroll
      for (int i = 0; i < NTV; ++i)
#pragma unroll
        for (int j = 0; j < NTK; ++j) mma(acc[i][j], x[i], y[j]);
    }
    if constexpr (!SG) {
#pragma unroll
      for (int j = 0; j < NTK; ++j) {
        const float f = sFr[(kt0 + j) * 16 + (lane & 15)];
#pragma unroll
        for (int i = 0; i < NTV; ++i) acc[i][j] *= f;
      }
    }
    __syncthreads();   // every tile read is done: the exchange aliases them

    // ---- (4) exchange dq / dk pre-factors; dg in the accumulator layout ----
    // dg = revcumsum_rows(qg (.) xq - kg (.) xk) + 2^r sum_v h dh' + sum_rows kg (.) dk_inter,
    // xq / xk the pre-factors (q dq - k dk with the gate factors cancelled). A wave holds RT
    // row tiles of its k tile: the rows of its row group (all 64 when NRG = 1), so the reverse
    // cumsum runs in registers: in-lane over a tile's 4 rows, rows4_suffix over the lane
    // groups, a running total over the tiles; later row groups (NRG > 1) and their dk sums
    // are added in the epilogue.
#pragma unroll
    for (int t = 0; t < KTW; ++t) {
      const int hk = (kq0 + t) * 16 + (lane & 15);
#pragma unroll
      for (int i = 0; i < RT; ++i) {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int ro = (rt0 + i) * 16 + 4 * (lane >> 4) + rr;
          XQ[Lay::xo(ro, hk)] = aq[t][i][rr];
          XK[Lay::xo(ro, hk)] = ak[t][i][rr];
        }
      }
      if (p.dg) {   // uniform: absent for scalar gates without a gate gradient
        const float hd = hdp[t] * (sFr[hk] * inv_scale);   // 2^r sum_v h dh'
        float carry = Lay::NRG == 1 ? hd + dkc[t] : hd;
#pragma unroll
        for (int i = RT - 1; i >= 0; --i) {
          const int r0 = (rt0 + i) * 16 + 4 * (lane >> 4);
          const int off = LT<KP>::at((rt0 + i) * 16, (kq0 + t) * 16) + LT<KP>::tr_rows4(ln);
          const s4_t qv = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) s4_t*)(sQg + off));
          const s4_t kv = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) s4_t*)(sKg + off));
          float x[4];
#pragma unroll
          for (int rr = 0; rr < 4; ++rr)
            x[rr] = __uint_as_float((uint32_t)(uint16_t)qv[rr] << 16) * aq[t][i][rr] -
                    __uint_as_float((uint32_t)(uint16_t)kv[rr] << 16) * ak[t][i][rr];
          x[2] += x[3];
          x[1] += x[2];
          x[0] += x[1];
          float tot;
          const float later = rows4_suffix(x[0], lane, &tot) - x[0] + carry;
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) XG[Lay::xo(r0 + rr, hk)] = x[rr] + later;
          carry += tot;
        }
        if (Lay::NRG > 1 && lane < 16) {
          sSuf[(w / NKG) * KP + hk] = carry - hd;   // the row group's total
          sDkc[(w / NKG) * KP + hk] = dkc[t];
        }
      }
    }
    __syncthreads();

    // ---- (5) epilogue: dq, dk, dg rows ----
    // (the next chunk's first barrier, in its gating, comes before anything overwrites the
    // exchange)
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      const int row = rs * RPT + j;
      const int xr = (tl / M::NCG) * RPT + j, xc = (tl % M::NCG) * 8;   // row, cg * 8
      float xq[8], xk[8];
      ld_x8<Lay>(XQ, xr, xc, xq);
      ld_x8<Lay>(XK, xr, xc, xk);
      if constexpr (!SG) {   // scalar gates: the factors are in already
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          xq[e] *= exp2_hw(dd[j][e]);
          xk[e] *= exp2_hw(-dd[j][e]);
        }
      }
      const bool st_ok = row < len && colA;
      const long b0 = (long)t0 * rsK + (long)hh * K;
      const uint32_t a =
          ((uint32_t)((tl / M::NCG) * RPT + j) * (uint32_t)rsK + (tl % M::NCG) * 8) * 2u;
      if (st_ok) {
        st16_sel(dq + b0, a, pack8(xq), ntk);
        st16_sel(dk + b0, a, pack8(xk), ntk);
      }
      if (p.dg) {
        float xg[8];
        ld_x8<Lay>(XG, xr, xc, xg);
        if constexpr (Lay::NRG > 1) {   // later row groups' totals; every group's dk sum
          const int rg = row / (RT * 16);
          float t8[8];
#pragma unroll
          for (int gi = 0; gi < Lay::NRG; ++gi) {
            ld_f8(sDkc + gi * KP + cg * 8, t8);
#pragma unroll
            for (int e = 0; e < 8; ++e) xg[e] += t8[e];
            if (gi > rg) {
              ld_f8(sSuf + gi * KP + cg * 8, t8);
#pragma unroll
              for (int e = 0; e < 8; ++e) xg[e] += t8[e];
            }
          }
        }
        if (st_ok) st16_sel(dg + b0, a, pack8(xg), ntk);
      }
    }
  }

  if (s == 0 && p.dh0)
    store_state_f32<NTV, NTK>(acc, p.dh0 + ((long)sg.seq * H + hh) * KV, K, V, vt0, kt0, lane);
  if (p.flags) {   // uniform; every block writes its flag, so nothing needs clearing
    const int bad = __syncthreads_or(gbad);
    if (tid == 0) p.flags[L] = bad ? 1 : 0;
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
bool head_supported(int dtype, int C, int K, int V, bool g_is_cumsum) {
  return dtype == DT_BF16 && C == HC && K >= 8 && V >= 8 && K <= 256 && K % 8 == 0 &&
         V % 8 == 0 && !g_is_cumsum;
}

bool head_bwd_supported(int K, int V) { return K <= 128 && V <= 128; }

static int head_kp(int K) { return K <= 64 ? 64 : K <= 128 ? 128 : 256; }

int head_vtiles(int K, int V) {
  const int vp = head_vp(head_kp(K), V);
  return (V + vp - 1) / vp;
}

void head_seg_plan(int N, int H, int T, int C, bool varlen, int& NS, int& SL, int VT) {
  NS = 1;
  SL = 0;
  if (varlen || N <= 0 || H <= 0) return;
  const int nt = (T + C - 1) / C;
  const long nh = (long)N * H * (VT > 0 ? VT : 1);
  // one block per CU (MI355X: 256 CUs): the full-head kernels hold one block per CU (LDS),
  // so a second round of blocks would run as a tail
  const long want = 256 / nh;
  long ns = want < nt / 8 ? want : nt / 8;                     // segments of >= 8 chunks
  if (ns <= 1) return;
  SL = (int)((nt + ns - 1) / ns);
  NS = (nt + SL - 1) / SL;
  if (NS <= 1) {
    NS = 1;
    SL = 0;
  }
}

// Per-chunk gating workspace of the wide forward: K = 256 heads split into three or more V
// tiles (each tile's block would otherwise gate the same chunk again); fixed-length only.
long head_gate_ws_bytes(int N, int T, int H, int K, int V) {
  if (head_kp(K) != 256 || head_vtiles(K, V) < 3 || N <= 0 || T <= 0) return 0;
  const long nt = (T + HC - 1) / HC;
  return (long)N * nt * H * gate_ws_entry(K);
}

long head_seg_ws_bytes(int N, int NS, int H, int K, int V) {
  if (NS <= 1) return 0;
  const long st = (long)N * NS * H * K * V * 4;
  const long gm = (long)N * NS * H * K * 4;
  return st + (gm + 255) / 256 * 256;
}

template <int KP, int VP, bool REV, bool SG, int CR, bool PRE = false>
static hipError_t launch_head_scan_cr(const HeadScanArgs& p, hipStream_t st, long blocks) {
  constexpr int NT = HNT;
  using Lay = HSLayout<KP, VP, NT, CR, PRE>;
  static_assert(Lay::bytes <= 163840, "LDS budget exceeded");
  const void* fn = (const void*)head_scan_kernel<KP, VP, REV, NT, SG, CR, PRE>;
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                     Lay::bytes);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((head_scan_kernel<KP, VP, REV, NT, SG, CR, PRE>), dim3((unsigned)blocks),
                     dim3(NT), Lay::bytes, st, p);
  return hipGetLastError();
}

// Pass 1 of heads up to 128 wide steps over pairs of chunks (half the serial steps and
// barriers); the passes that store per-chunk states, and K = 256, step chunk by chunk.
template <int KP, int VP, bool REV>
static hipError_t launch_head_scan(const HeadScanArgs& p, hipStream_t st, long blocks) {
  if constexpr (KP <= 128) {
    if (p.pass == 1)
      return p.g ? launch_head_scan_cr<KP, VP, REV, false, 2 * HC>(p, st, blocks)
                 : launch_head_scan_cr<KP, VP, REV, true, 2 * HC>(p, st, blocks);
  } else {
    if (p.g && p.gate_ws) return launch_head_scan_cr<KP, VP, REV, false, HC, true>(p, st, blocks);
  }
  return p.g ? launch_head_scan_cr<KP, VP, REV, false, HC>(p, st, blocks)
             : launch_head_scan_cr<KP, VP, REV, true, HC>(p, st, blocks);
}

template <bool REV>
static hipError_t head_scan_kp(const HeadScanArgs& p, hipStream_t st, long blocks) {
  blocks *= head_vtiles(p.K, p.V);
  const int kp = head_kp(p.K);
  if (kp == 256) return launch_head_scan<256, 64, REV>(p, st, blocks);
  const bool v64 = head_vp(kp, p.V) == 64;
  if (kp == 64) return v64 ? launch_head_scan<64, 64, REV>(p, st, blocks)
                           : launch_head_scan<64, 128, REV>(p, st, blocks);
  return v64 ? launch_head_scan<128, 64, REV>(p, st, blocks)
             : launch_head_scan<128, 128, REV>(p, st, blocks);
}

static hipError_t head_scan_launch(HeadScanArgs p, bool reverse, hipStream_t st, int pass,
                                   int s_begin, int ns_launch) {
  p.pass = pass;
  p.s_begin = s_begin;
  p.ns_launch = ns_launch;
  if (pass == 1) {   // local states only
    p.s_all = nullptr;
    p.s_final = nullptr;
  }
  const long blocks = (long)p.si.N * ns_launch * p.H;
  if (blocks == 0) return hipSuccess;
  return reverse ? head_scan_kp<true>(p, st, blocks) : head_scan_kp<false>(p, st, blocks);
}

// Segment pass 1 (no-op when NS == 1): the local states; every segment's block folds its
// own entry state from them (load_entry_state).
static hipError_t head_prepare_segments(const HeadScanArgs& p, bool reverse, hipStream_t st) {
  if (p.NS <= 1) return hipSuccess;
  // pass 1 skips the last segment in flow order (its local state is never needed)
  return head_scan_launch(p, reverse, st, 1, reverse ? 1 : 0, p.NS - 1);
}

hipError_t run_head_scan(const HeadScanArgs& p0, bool reverse, hipStream_t st) {
  HeadScanArgs p = p0;
  hipError_t e = head_prepare_segments(p, reverse, st);
  if (e != hipSuccess) return e;
  return head_scan_launch(p, reverse, st, 3, 0, p.NS);
}

template <int KP, int VP, bool SG>
static hipError_t launch_head_fwd_sg(const HeadFwdArgs& p, hipStream_t st, long blocks) {
  using Lay = HFLayout<KP, VP, SG>;
  hipError_t e = hipFuncSetAttribute((const void*)head_fwd_kernel<KP, VP, SG>,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, Lay::bytes);
  if (e != hipSuccess) return e;
  ktimer_mark(KT_HEAD_FWD, false, st);
  hipLaunchKernelGGL((head_fwd_kernel<KP, VP, SG>), dim3((unsigned)blocks), dim3(HNT),
                     Lay::bytes, st, p);
  ktimer_mark(KT_HEAD_FWD, true, st);
  return hipGetLastError();
}

hipError_t run_head_gate(const HeadFwdArgs& p, hipStream_t st) {
  if (head_kp(p.K) != 256 || p.si.cu || !p.g || !p.gate_ws) return hipErrorInvalidValue;
  const int nt = (p.si.T + HC - 1) / HC;
  if ((long)nt * p.H * p.si.N == 0) return hipSuccess;
  using GL = GPLayout<256>;
  hipError_t e = hipFuncSetAttribute((const void*)head_gate_kernel<256>,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, GL::bytes);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((head_gate_kernel<256>), dim3((unsigned)(nt * p.H), (unsigned)p.si.N),
                     dim3(HNT), GL::bytes, st, p);
  return hipGetLastError();
}

static hipError_t launch_head_dqkg(const BwdArgs& p, hipStream_t st) {
  const long blocks = (long)p.si.NC * p.H * ((p.K + DKB - 1) / DKB);
  if (blocks == 0) return hipSuccess;
  if (blocks > 2147483647L) return hipErrorInvalidValue;
  using Lay = HDLayout<DKB>;
  static_assert(2 * Lay::bytes <= 163840, "two blocks per CU");
  hipError_t e = hipFuncSetAttribute((const void*)head_dqkg_kernel<DKB, DNW>,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, Lay::bytes);
  if (e != hipSuccess) return e;
  ktimer_mark(KT_BWD_DQKG, false, st);
  hipLaunchKernelGGL((head_dqkg_kernel<DKB, DNW>), dim3((unsigned)blocks), dim3(DNW * 64),
                     Lay::bytes, st, p);
  ktimer_mark(KT_BWD_DQKG, true, st);
  return hipGetLastError();
}

bool head_dqkg_supported(int K, int V) { return K > 64 && K <= 256 && V >= 8; }

hipError_t run_head_dqkg(const BwdArgs& p, hipStream_t st) {
  if (!head_dqkg_supported(p.K, p.V) || p.K % 8 || p.V % 8 || p.si.C != HC)
    return hipErrorInvalidValue;
  return launch_head_dqkg(p, st);
}

template <int KP, int VP>
static hipError_t launch_head_fwd(const HeadFwdArgs& p, hipStream_t st) {
  const long blocks = (long)p.si.N * p.NS * p.H * ((p.V + VP - 1) / VP);
  if (blocks == 0) return hipSuccess;
  if constexpr (KP == 256) {
    if (p.g && p.gate_ws) {   // the V tiles' blocks stream the per-chunk gating
      using Lay = HFLayout<KP, VP, false>;
      const void* fn = p.h_out ? (const void*)head_fwd_kernel<KP, VP, false, true, true>
                               : (const void*)head_fwd_kernel<KP, VP, false, true, false>;
      hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                         Lay::bytes);
      if (e != hipSuccess) return e;
      HeadFwdArgs q = p;
      q.flags = nullptr;   // the gating kernel wrote the per-chunk flags
      ktimer_mark(KT_HEAD_FWD, false, st);
      if (p.h_out)
        hipLaunchKernelGGL((head_fwd_kernel<KP, VP, false, true, true>), dim3((unsigned)blocks),
                           dim3(HNT), Lay::bytes, st, q);
      else
        hipLaunchKernelGGL((head_fwd_kernel<KP, VP, false, true, false>),
                           dim3((unsigned)blocks), dim3(HNT), Lay::bytes, st, q);
      ktimer_mark(KT_HEAD_FWD, true, st);
      return hipGetLastError();
    }
  }
  return p.g ? launch_head_fwd_sg<KP, VP, false>(p, st, blocks)
             : launch_head_fwd_sg<KP, VP, true>(p, st, blocks);
}

hipError_t run_head_fwd(const HeadFwdArgs& p, hipStream_t st) {
  // wide heads with a gating workspace: gate every chunk once, first; the segment pass and
  // the forward's V tiles stream it
  const bool gated = head_kp(p.K) == 256 && p.g && p.gate_ws;
  if (gated) {
    hipError_t e = run_head_gate(p, st);
    if (e != hipSuccess) return e;
  }
  if (p.NS > 1) {
    HeadScanArgs s = {};
    s.gate_ws = gated ? p.gate_ws : nullptr;
    s.a = p.k;
    s.b = p.v;
    s.g = p.g;
    s.gs = p.gs;
    s.gs_ts = p.gs_ts;
    s.s_init = p.h0;
    s.s_all = nullptr;
    s.s_final = nullptr;
    s.seg_state = p.seg_state;
    s.seg_gam = p.seg_gam;
    s.NS = p.NS;
    s.SL = p.SL;
    s.scale = 1.f;
    s.H = p.H;
    s.K = p.K;
    s.V = p.V;
    s.si = p.si;
    hipError_t e = head_prepare_segments(s, false, st);
    if (e != hipSuccess) return e;
  }
  const int kp = head_kp(p.K);
  if (kp == 256) return launch_head_fwd<256, 64>(p, st);
  const bool v64 = head_vp(kp, p.V) == 64;
  if (kp == 64) return v64 ? launch_head_fwd<64, 64>(p, st) : launch_head_fwd<64, 128>(p, st);
  return v64 ? launch_head_fwd<128, 64>(p, st) : launch_head_fwd<128, 128>(p, st);
}

template <int KP, int VP, bool SG>
static hipError_t launch_head_bwd_sg(const HeadBwdArgs& p, hipStream_t st, long blocks) {
  constexpr int NT = HNT;
  using Lay = HBLayout<KP, VP, NT / 64, SG>;
  hipError_t e = hipFuncSetAttribute((const void*)head_bwd_kernel<KP, VP, NT, SG>,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, Lay::bytes);
  if (e != hipSuccess) return e;
  ktimer_mark(KT_HEAD_BWD, false, st);
  hipLaunchKernelGGL((head_bwd_kernel<KP, VP, NT, SG>), dim3((unsigned)blocks), dim3(NT),
                     Lay::bytes, st, p);
  ktimer_mark(KT_HEAD_BWD, true, st);
  return hipGetLastError();
}

template <int KP, int VP>
static hipError_t launch_head_bwd(const HeadBwdArgs& p, hipStream_t st) {
  const long blocks = (long)p.si.N * p.NS * p.H;
  if (blocks == 0) return hipSuccess;
  return p.g ? launch_head_bwd_sg<KP, VP, false>(p, st, blocks)
             : launch_head_bwd_sg<KP, VP, true>(p, st, blocks);
}

hipError_t run_head_bwd(const HeadBwdArgs& p, hipStream_t st) {
  if (p.NS > 1) {
    HeadScanArgs s = {};
    s.a = p.q;
    s.b = p.dout;
    s.g = p.g;
    s.gs = p.gs;
    s.gs_ts = p.gs_ts;
    s.s_init = p.dht;
    s.seg_state = p.seg_state;
    s.seg_gam = p.seg_gam;
    s.NS = p.NS;
    s.SL = p.SL;
    s.scale = p.scale;
    s.H = p.H;
    s.K = p.K;
    s.V = p.V;
    s.si = p.si;
    hipError_t e = head_prepare_segments(s, true, st);
    if (e != hipSuccess) return e;
  }
  const bool k64 = p.K <= 64, v64 = p.V <= 64;
  if (k64 && v64) return launch_head_bwd<64, 64>(p, st);
  if (k64) return launch_head_bwd<64, 128>(p, st);
  if (v64) return launch_head_bwd<128, 64>(p, st);
  return launch_head_bwd<128, 128>(p, st);
}

}  // namespace tops
