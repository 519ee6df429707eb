// Device-side building blocks shared by every GLA kernel (gfx950 / CDNA4 only).
//
// * Element types: `float` and `bf16` (bit-exact storage of bfloat16). Inputs of one call
//   share one element type; the MFMA operand type equals it (bf16 -> 16x16x32 bf16 MFMA,
//   float -> 8 x 16x16x4 f32 MFMA), accumulation is always fp32.
// * MFMA operand fragments: lane l supplies row (l & 15) and the 8 contraction indices
//   8*(l >> 4) .. +7 of a 16 x 32 slab. Both operands are read from LDS "contraction-major"
//   (contraction index contiguous), so an output tile is `X[m][k] . Y[n][k]^T`.
// * Accumulator layout (16x16 f32x4): acc[r] holds row 4*(l >> 4) + r, column l & 15.
// * Sequence layout: tokens are flattened to one index tau over [B*T) (fixed length) or
//   [T_total) (varlen, B == 1); element (tau, head, d) lives at (tau*H + head)*D + d.
//   Chunks never cross a sequence boundary; the last chunk of a sequence may be partial.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tops {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct bf16 {
  uint16_t u;
};

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16 x) { return __uint_as_float((uint32_t)x.u << 16); }

template <typename T>
__device__ __forceinline__ T from_f32(float f);
template <>
__device__ __forceinline__ float from_f32<float>(float f) {
  return f;
}
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float f) {
  // gfx950 v_cvt_pk_bf16_f32: round to nearest even, NaN stays NaN
  bf16 r;
  r.u = __builtin_bit_cast(uint16_t, (__bf16)f);
  return r;
}

// Global accesses are a uniform base pointer (scalar registers) plus a 32-bit per-lane
// byte offset, which the compiler emits as the scalar-base form of the global loads and
// stores: one VGPR per address instead of a 64-bit pair.
__device__ __forceinline__ uint4 ld16(const void* base, uint32_t off) {
  return *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(base) + off);
}
__device__ __forceinline__ void st16(void* base, uint32_t off, const uint4& x) {
  *reinterpret_cast<uint4*>(reinterpret_cast<char*>(base) + off) = x;
}
__device__ __forceinline__ void st8(void* base, uint32_t off, const uint2& x) {
  *reinterpret_cast<uint2*>(reinterpret_cast<char*>(base) + off) = x;
}

// 16 bytes, nontemporal. The kernels' outputs are written once and not read again in the
// launch: streamed past the L2 they leave no dirty lines for the writeback at the end of
// the launch, which otherwise holds up the next launch (on MI355X 15-20 us after the fused
// kernels). Only for whole 128-byte row pieces: partial lines written this way are slow.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void st16_nt(void* base, uint32_t off, const uint4& x) {
  const u32x4_t v = {x.x, x.y, x.z, x.w};
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(reinterpret_cast<char*>(base) + off));
}
// st16_nt when `nt`, else st16. The empty asm statements keep the two stores from being
// merged into one (which would drop the nontemporal hint).
__device__ __forceinline__ void st16_sel(void* base, uint32_t off, const uint4& x, bool nt) {
  if (nt) {
    st16_nt(base, off, x);
  } else {
    asm volatile("");
    st16(base, off, x);
    asm volatile("");
  }
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Two floats -> two bf16 in one 32-bit word (element a in the low half), one instruction.
__device__ __forceinline__ uint32_t pack2_bf16(float a, float b) {
  bf16x2_t v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

template <typename T>
__device__ __forceinline__ T zero_elem() {
  return from_f32<T>(0.f);
}

// exp for gate factors: correctly rounded-ish ocml expf on the fp32 path (parity bar 1e-4
// absolute), the hardware exp2 path on the bf16 path (operands are rounded to bf16 anyway).
template <typename T>
__device__ __forceinline__ float gexp(float x);
template <>
__device__ __forceinline__ float gexp<float>(float x) {
  return expf(x);
}
template <>
__device__ __forceinline__ float gexp<bf16>(float x) {
  return __expf(x);
}

// x / e given e = gexp<T>(d): float inputs divide (the float32 path keeps the IEEE
// division); bf16 inputs multiply by e^{-d} instead (a hardware exp in place of the
// division's scale / fix-up sequence)
template <typename T>
__device__ __forceinline__ float gdiv(float x, float d, float e);
template <>
__device__ __forceinline__ float gdiv<float>(float x, float, float e) {
  return x / e;
}
template <>
__device__ __forceinline__ float gdiv<bf16>(float x, float d, float) {
  return x * __expf(-d);
}

// Workgroups are dispatched round-robin over the 8 XCDs (each with its own L2). Remap the
// hardware block id so that consecutive logical blocks land on the same XCD.
__device__ __forceinline__ int xcd_remap(int L, int total) {
  if ((total & 7) != 0) return L;
  return (L & 7) * (total >> 3) + (L >> 3);
}

// ---------------------------------------------------------------------------
// MFMA fragments
// ---------------------------------------------------------------------------
template <typename T>
struct Frag;
template <>
struct Frag<bf16> {
  uint4 d;
};
template <>
struct Frag<float> {
  float4 a, b;
};

__device__ __forceinline__ Frag<bf16> ld_frag(const bf16* p) {
  Frag<bf16> f;
  f.d = *reinterpret_cast<const uint4*>(p);
  return f;
}
__device__ __forceinline__ Frag<float> ld_frag(const float* p) {
  Frag<float> f;
  f.a = *reinterpret_cast<const float4*>(p);
  f.b = *reinterpret_cast<const float4*>(p + 4);
  return f;
}

__device__ __forceinline__ void mma(f32x4& acc, const Frag<bf16>& a, const Frag<bf16>& b) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a.d),
                                                 __builtin_bit_cast(bf16x8_t, b.d), acc, 0,
                                                 0, 0);
}
__device__ __forceinline__ void mma(f32x4& acc, const Frag<float>& a, const Frag<float>& b) {
  // Contraction index 8*(l>>4)+e is fed to MFMA #e as its k = l>>4 (a consistent
  // permutation of the 32 indices for both operands).
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.a.x, b.a.x, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.a.y, b.a.y, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.a.z, b.a.z, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.a.w, b.a.w, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.b.x, b.b.x, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.b.y, b.b.y, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.b.z, b.b.z, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.b.w, b.b.w, acc, 0, 0, 0);
}

// acc += X[0:16][0:klen] . Y[0:16][0:klen]^T, both in LDS, contraction-major, klen % 32 == 0.
template <typename T>
__device__ __forceinline__ void mma_tile(f32x4& acc, const T* X, int px, const T* Y, int py,
                                         int klen, int lane) {
  const T* xr = X + (lane & 15) * px + (lane >> 4) * 8;
  const T* yr = Y + (lane & 15) * py + (lane >> 4) * 8;
  for (int kk = 0; kk < klen; kk += 32) mma(acc, ld_frag(xr + kk), ld_frag(yr + kk));
}

// ---------------------------------------------------------------------------
// Transposed fragments: X[m][k] read from a ROW-MAJOR [k][m] LDS tile (pitch P elements),
// `M` pointing at element [k0][m0]. gfx950 ds_read_b64_tr_b16: within each 16-lane group,
// lane 4r+q supplies the address of row r, columns 4q..4q+3 of a 4 x 16 block and lane i
// receives column i of that block (rows 0..3). Two such reads give lane l the 8 values
// M[8*(l>>4) + 0..7][l & 15], i.e. the same fragment ld_frag returns from [m][k].
// P*sizeof(T) must be a multiple of 8 and m0 a multiple of 4.
// ---------------------------------------------------------------------------
typedef short s4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ Frag<bf16> ld_frag_t(const bf16* M, int P, int lane) {
  const int g = lane >> 4, j = lane & 15;
  const bf16* p1 = M + (8 * g + (j >> 2)) * P + 4 * (j & 3);
  const s4_t a = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s4_t*)(p1));
  const s4_t b = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s4_t*)(p1 + 4 * P));
  const uint2 ua = __builtin_bit_cast(uint2, a), ub = __builtin_bit_cast(uint2, b);
  Frag<bf16> f;
  f.d = make_uint4(ua.x, ua.y, ub.x, ub.y);
  return f;
}
__device__ __forceinline__ Frag<float> ld_frag_t(const float* M, int P, int lane) {
  const float* p = M + (8 * (lane >> 4)) * P + (lane & 15);
  Frag<float> f;
  f.a = make_float4(p[0], p[P], p[2 * P], p[3 * P]);
  f.b = make_float4(p[4 * P], p[5 * P], p[6 * P], p[7 * P]);
  return f;
}

// acc += X . Y^T over klen (multiple of 32). XT / YT: the operand is stored row-major as
// [k][m] (resp. [k][n]) and is read with transposed fragments; the pointer then addresses
// element [0][m0] and the pitch is the [k] row pitch.
template <typename T, bool XT, bool YT>
__device__ __forceinline__ void mma_tile2(f32x4& acc, const T* X, int px, const T* Y, int py,
                                          int klen, int lane) {
  for (int kk = 0; kk < klen; kk += 32) {
    const Frag<T> a = XT ? ld_frag_t(X + kk * px, px, lane)
                         : ld_frag(X + (lane & 15) * px + (lane >> 4) * 8 + kk);
    const Frag<T> b = YT ? ld_frag_t(Y + kk * py, py, lane)
                         : ld_frag(Y + (lane & 15) * py + (lane >> 4) * 8 + kk);
    mma(acc, a, b);
  }
}

__device__ __forceinline__ f32x4 zero4() {
  f32x4 z = {0.f, 0.f, 0.f, 0.f};
  return z;
}

// LDS row pitch (elements) for a contraction-major buffer of width w: +16 bytes of padding
// breaks the 16-way bank conflict of 16 lanes reading 16 consecutive rows.
template <typename T>
__host__ __device__ constexpr int pitch_of(int w) {
  return w + (int)(16 / sizeof(T));
}

// ---------------------------------------------------------------------------
// Element pairs (two adjacent columns) and short vector runs in LDS
// ---------------------------------------------------------------------------
template <typename T>
struct Pair;
template <>
struct Pair<bf16> {
  static __device__ __forceinline__ void ld(const bf16* p, float& a, float& b) {
    const uint32_t w = *reinterpret_cast<const uint32_t*>(p);
    a = bf16_lo(w);
    b = bf16_hi(w);
  }
  static __device__ __forceinline__ void st(bf16* p, float a, float b) {
    *reinterpret_cast<uint32_t*>(p) = pack2_bf16(a, b);
  }
};
template <>
struct Pair<float> {
  static __device__ __forceinline__ void ld(const float* p, float& a, float& b) {
    const float2 w = *reinterpret_cast<const float2*>(p);
    a = w.x;
    b = w.y;
  }
  static __device__ __forceinline__ void st(float* p, float a, float b) {
    *reinterpret_cast<float2*>(p) = make_float2(a, b);
  }
};

// Store N consecutive values (N in {2, 4, 8}, dst aligned to N elements) as wide writes.
template <typename T, int N>
__device__ __forceinline__ void store_run(T* dst, const float (&x)[N]) {
  if constexpr (sizeof(T) == 2) {
    uint32_t w[N / 2];
#pragma unroll
    for (int i = 0; i < N / 2; ++i) w[i] = pack2_bf16(x[2 * i], x[2 * i + 1]);
    if constexpr (N == 8) {
      *reinterpret_cast<uint4*>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
    } else if constexpr (N == 4) {
      *reinterpret_cast<uint2*>(dst) = make_uint2(w[0], w[1]);
    } else {
      *reinterpret_cast<uint32_t*>(dst) = w[0];
    }
  } else {
    if constexpr (N == 8) {
      reinterpret_cast<float4*>(dst)[0] = make_float4(x[0], x[1], x[2], x[3]);
      reinterpret_cast<float4*>(dst)[1] = make_float4(x[4], x[5], x[6], x[7]);
    } else if constexpr (N == 4) {
      *reinterpret_cast<float4*>(dst) = make_float4(x[0], x[1], x[2], x[3]);
    } else {
      *reinterpret_cast<float2*>(dst) = make_float2(x[0], x[1]);
    }
  }
}

// x & m per 32-bit word (m = all ones or zero): a branch-free "valid ? x : 0".
__device__ __forceinline__ uint4 mask16(uint4 x, uint32_t m) {
  return make_uint4(x.x & m, x.y & m, x.z & m, x.w & m);
}

// 16 bytes of a global row starting at column col0, zero-filled past `nvalid` columns.
// VEC: the row start and col0 are 16-byte aligned (only the tail check remains).
template <typename T, bool VEC>
__device__ __forceinline__ uint4 gload16(const T* __restrict__ row, int col0, int nvalid) {
  constexpr int EPP = 16 / (int)sizeof(T);
  uint4 r = make_uint4(0, 0, 0, 0);
  if (VEC) {
    if (nvalid >= EPP) r = *reinterpret_cast<const uint4*>(row + col0);
    return r;
  }
  if (nvalid > 0) {
    T tmp[EPP];
#pragma unroll
    for (int e = 0; e < EPP; ++e) tmp[e] = e < nvalid ? row[col0 + e] : zero_elem<T>();
    __builtin_memcpy(&r, tmp, 16);
  }
  return r;
}

// ---------------------------------------------------------------------------
// Sequence / chunk layout
// ---------------------------------------------------------------------------
struct SeqInfo {
  int N;                // sequences
  int T;                // tokens per sequence (fixed-length mode)
  int C;                // chunk size
  int NC;               // total chunks
  const int* cu;        // [N+1] token offsets (varlen) or nullptr
  const int* chunk_cu;  // [N+1] chunk offsets (varlen) or nullptr
};

__device__ __forceinline__ void seq_range(const SeqInfo& s, int i, int& bos, int& eos,
                                          int& c0, int& nc) {
  if (s.cu) {
    bos = s.cu[i];
    eos = s.cu[i + 1];
    c0 = s.chunk_cu[i];
    nc = s.chunk_cu[i + 1] - c0;
  } else {
    const int nt = (s.T + s.C - 1) / s.C;
    bos = i * s.T;
    eos = bos + s.T;
    c0 = i * nt;
    nc = nt;
  }
}

// Token range of sequence i only (reads no chunk offsets; valid with chunk_cu == nullptr).
__device__ __forceinline__ void seq_bounds(const SeqInfo& s, int i, int& bos, int& eos) {
  if (s.cu) {
    bos = s.cu[i];
    eos = s.cu[i + 1];
  } else {
    bos = i * s.T;
    eos = bos + s.T;
  }
}

// Global chunk index -> (sequence, first token, valid rows).
__device__ __forceinline__ void chunk_range(const SeqInfo& s, int c, int& seq, int& t0,
                                            int& len) {
  if (s.cu) {
    int lo = 0, hi = s.N - 1;  // largest i with chunk_cu[i] <= c (skips empty sequences)
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s.chunk_cu[mid] <= c) lo = mid; else hi = mid - 1;
    }
    seq = lo;
    t0 = s.cu[lo] + (c - s.chunk_cu[lo]) * s.C;
    len = min(s.C, s.cu[lo + 1] - t0);
  } else {
    const int nt = (s.T + s.C - 1) / s.C;
    seq = c / nt;
    const int n = c - seq * nt;
    t0 = seq * s.T + n * s.C;
    len = min(s.C, s.T - n * s.C);
  }
}

// ---------------------------------------------------------------------------
// Chunk-local cumsum of one 64-column gate tile, cooperative over a 256-thread block.
// Thread t owns column (t & 63) and rows [(t >> 6) * RPS, +RPS), RPS = C / 4.
// On return gt[] holds the inclusive cumsum of its rows, `gamma` the value at row C-1
// (rows >= len read as 0, so this equals the last valid row), `first` the value at row 0.
// If G_IS_CUMSUM the input already holds the cumsum and is only loaded.
// sTot needs 4*64 floats; contains a __syncthreads().
// ---------------------------------------------------------------------------
template <int C, typename TIN>
__device__ __forceinline__ void tile_cumsum(const TIN* __restrict__ g, long row_stride,
                                            int len, int col_valid, bool g_is_cumsum,
                                            float* sTot, float (&gt)[C / 4], float& gamma,
                                            float& first) {
  constexpr int RPS = C / 4;
  const int tid = threadIdx.x;
  const int col = tid & 63, seg = tid >> 6;
  const int r0 = seg * RPS;
  float run = 0.f;
#pragma unroll
  for (int r = 0; r < RPS; ++r) {
    const int row = r0 + r;
    float x = 0.f;
    if (row < len && col_valid) x = to_f32(g[(long)row * row_stride]);
    if (g_is_cumsum) {
      gt[r] = x;
    } else {
      run += x;
      gt[r] = run;
    }
  }
  if (g_is_cumsum) {
    // gamma = value at the last valid row; first = row 0
    sTot[seg * 64 + col] = 0.f;
    __syncthreads();
    if (len > 0) {
      const int lr = len - 1;
      if (lr >= r0 && lr < r0 + RPS) {
#pragma unroll
        for (int r = 0; r < RPS; ++r)
          if (r0 + r == lr) sTot[col] = gt[r];  // seg-local write into slot 0 of the column
      }
    }
    // slot 64+col: row 0
    if (seg == 0) sTot[64 + col] = gt[0];
    __syncthreads();
    gamma = sTot[col];
    first = sTot[64 + col];
    // rows beyond len keep their loaded 0; callers only use them multiplied by zero inputs,
    // but keep them equal to gamma so exp() stays bounded.
#pragma unroll
    for (int r = 0; r < RPS; ++r)
      if (r0 + r >= len) gt[r] = gamma;
    __syncthreads();
    return;
  }
  sTot[seg * 64 + col] = run;
  __syncthreads();
  float off = 0.f, tot = 0.f;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const float v = sTot[s * 64 + col];
    off += (s < seg) ? v : 0.f;
    tot += v;
  }
#pragma unroll
  for (int r = 0; r < RPS; ++r) gt[r] += off;
  gamma = tot;
  first = sTot[col];  // segment 0's total is not row 0; fixed below
  __syncthreads();
  if (seg == 0) sTot[col] = gt[0];
  __syncthreads();
  first = sTot[col];
  __syncthreads();
}

}  // namespace tops
