// Internal (C++) launch interface between the C-ABI layer (capi.hip) and the kernels.
#pragma once

#include <hip/hip_runtime.h>

#include "common.hpp"

namespace tops {

enum DType { DT_F32 = 0, DT_BF16 = 1 };

// Inter-chunk state scan (chunk_h.hip).
struct ScanArgs {
  const void* a;        // forward: k ; reverse: q
  const void* b;        // forward: v ; reverse: do
  const void* g;        // gates (raw, or chunk-local cumsum when g_is_cumsum)
  int g_is_cumsum;
  const float* s_init;  // forward: h0 ; reverse: dht (nullable)
  void* s_all;          // per-chunk states [NC, H, K, V] in the input dtype (nullable)
  float* s_final;       // forward: ht ; reverse: dh0 (nullable)
  float scale;          // reverse only
  int H, K, V;
  int vec;              // 16-byte loads/stores allowed (K, V multiples of 16 B, aligned)
  SeqInfo si;
};
hipError_t run_state_scan(const ScanArgs& p, bool reverse, int dtype, hipStream_t st);

// Per-chunk intra matrix and output (chunk_fwd.hip).
struct FwdOArgs {
  const void *q, *k, *v, *g;
  int g_is_cumsum;
  const void* h;        // [NC, H, K, V] state at chunk start (nullable: no inter term)
  const float* A_in;    // [NC*C, H, C] given intra matrix (nullable: computed)
  float* A_out;         // [NC*C, H, C] unmasked intra matrix (nullable)
  void* o;              // [tokens, H, V] (nullable)
  float scale;
  int H, K, V;
  SeqInfo si;
};
hipError_t run_chunk_fwd_o(const FwdOArgs& p, int dtype, hipStream_t st);

// The same two steps at chunk sizes 4 and 8 (small_chunk.hip): the per-chunk states (forward
// or reverse; no segment workspace) and the intra matrix / output combine.
hipError_t run_small_state_scan(const ScanArgs& p, bool reverse, int dtype, hipStream_t st);
hipError_t run_small_chunk_fwd_o(const FwdOArgs& p, int dtype, hipStream_t st);
int small_chunk_max_k();

// Fused forward: state scan + output in one sequential pass (chunk_fwd_fused.hip).
struct FusedFwdArgs {
  const void *q, *k, *v, *g;
  const float* h0;      // [N, H, K, V] or null
  void* o;              // [tokens, H, V]
  void* h_out;          // [NC, H, K, V] states entering each chunk (nullable)
  float* ht;            // [N, H, K, V] or null
  float scale;
  int H, K, V;
  int vec_k, vec_v;     // 16-byte loads/stores allowed for K- / V-rows
  SeqInfo si;
};
// True when the fused forward handles (dtype, C, K); otherwise use run_state_scan+run_chunk_fwd_o.
bool fused_fwd_supported(int dtype, int C, int K);
hipError_t run_chunk_fwd_fused(const FusedFwdArgs& p, int dtype, hipStream_t st);

// Per-chunk gradients (chunk_bwd.hip).
struct BwdArgs {
  const void *q, *k, *v, *g, *dout;
  const void* h;        // [NC, H, K, V] forward states (chunk start)
  const void* dh;       // [NC, H, K, V] state gradients (chunk end)
  void *dq, *dk, *dv, *dg;
  // per-chunk gating workspace (head_gate_kernel: bf16, chunk 64, fixed-length; nullable):
  // the dv kernel then streams gated k, A and the column factors instead of recomputing
  // them in every V tile's block
  const void* gate_ws;
  float scale;
  int H, K, V;
  int vec;              // every base pointer 16-byte aligned and K, V multiples of 16 bytes
  SeqInfo si;
};
// Bytes of one (chunk, head) entry of the per-chunk gating workspace (chunk 64): qs = scale
// q 2^{g~} and kg = k 2^{r-g~}, [64][K] bf16 each, A [64][64] bf16 (masked, scaled), the
// column factors scale 2^r, 2^r,
// 2^{gamma-r} and the chunk's summed gates gamma (base 2) [4][K] f32.
__host__ __device__ constexpr long gate_ws_entry(int K) {
  return 2L * 64 * K * 2 + 64L * 64 * 2 + 4L * K * 4;
}
// which: bit 0 = dq/dk/dg kernel, bit 1 = dv kernel
hipError_t run_chunk_bwd(const BwdArgs& p, int dtype, hipStream_t st, int which = 3);

// Chunk-local cumsum (cumsum.hip).
struct CumsumArgs {
  const void* g;
  void* out;
  int H, S;
  int reverse, has_scale, head_first;
  float scale;
  long T_total;         // tokens per batch row (head_first stride)
  SeqInfo si;
};
hipError_t run_cumsum(const CumsumArgs& p, int in_dtype, int out_dtype, hipStream_t st);

// Fused recurrent forward (recurrent.hip).
// Gate-range flags: 1 when a chunk has a gate range beyond what the per-element factoring
// holds (|g~ - r| > kGateLimit2 in base 2), written unconditionally (no clearing). Two
// layouts, both ((seq * ns + s) * H + h) * vt + t:
// * per block of the full-head kernels: s = segment, t = V tile;
// * per chunk (gate_range_kernel, head_gate_kernel; vt = 1): s = the sequence's chunk, i.e.
//   [NC, H]; with varlen sequences `co` (chunk offsets [N + 1]) gives each sequence's chunk
//   range instead of ns chunks from seq * ns.
// The recurrent fallback (exact for any decay) then recomputes the flagged (sequence, head)
// pairs.
struct GateFlags {
  int* p;         // nullable: no check, no fallback
  int ns, vt;     // segments (or chunks) and V tiles per (sequence, head)
  const int* co;  // nullable: per-chunk flags of varlen sequences (ns unused)
};
constexpr float kGateLimit2 = 100.f;

// Per-chunk gate-range check (gate_range.hip): flags[c * H + h] for every chunk c and head h.
struct GateCheckArgs {
  const void* g;   // raw log-gates [tokens, H, K]
  int* flags;      // [NC, H]
  int H, K;
  SeqInfo si;
};
hipError_t run_gate_range(const GateCheckArgs& p, int dtype, hipStream_t st);

struct RecArgs {
  const void *q, *k, *v, *gk, *gv;  // gk / gv nullable
  const float* h0;                  // nullable
  void* o;                          // [tokens, H, V] in o_dtype
  float* ht;                        // nullable
  float scale;
  int H, K, V;
  int reverse;
  SeqInfo si;                       // C unused
  GateFlags flags;                  // nullable: only the flagged (sequence, head) pairs run
};
hipError_t run_recurrent_fwd(const RecArgs& p, int dtype, int o_dtype, hipStream_t st);

// Fused recurrent forward / backward (recurrent.hip). One element-wise state scan:
//   S <- S (.) (e^{ga[r]} e^{gb[c]}) + (sa a[r]) b[c],  out[c] = so sum_r o[r] S[r][c]
struct RecScanArgs {
  const void *a, *ga, *o;  // row side [tokens, H, R]; ga nullable (raw log gate)
  const void *b, *gb;      // column side [tokens, H, C]; gb nullable
  const float* s0;         // initial state [N, H, ...] f32, nullable
  float* sN;               // final state, nullable
  int s_trans;             // states stored [C][R] (1) or [R][C] (0)
  int final_gate;          // apply the last step's gate before storing sN
  void* out;               // [tokens, H, C], out dtype (f32 in the backward)
  float sa, so;
  int R, C, H;
  int dir;    // 0: bos -> eos, 1: eos - 1 -> bos
  int shift;  // the gate of a step is applied at the next processed step
  // gate-gradient epilogue (dg nullable): dg = running sum of gx gxf - gy out
  // (+ sum_r s0 (.) hfin when hfin is given)
  const void* gx;
  const void* gxf;   // out dtype, or float when gxf_f32
  int gxf_f32;
  // bf16 outputs read back by a later scan's epilogue: `out_lo` (nullable, out dtype, out's
  // layout) receives out's rounding residual (out - bf16(out)), and a `gxf_lo` given with
  // gxf adds it back, so the epilogue sees out to about 16 significant bits
  void* out_lo;
  const void* gxf_lo;
  const void* gy;
  const float* hfin;
  void* dg;          // out dtype
  SeqInfo si;  // C unused
  GateFlags flags;   // nullable: only the flagged (sequence, head) pairs run
};
struct RecBwdArgs {
  const void *q, *k, *v, *gk, *gv, *dout;  // gk / gv nullable
  const float* o;                          // forward output f32 (needed with gv)
  const float *h0, *dht;                   // nullable
  void *dq, *dk, *dv, *dgk, *dgv;         // out dtype; dgk / dgv nullable
  float* dh0;                              // nullable
  float* ht_ws;                            // [N, H, K, V] f32, needed with dht and a gate
  float scale;
  int H, K, V;
  int reverse;
  SeqInfo si;
  GateFlags flags;                         // nullable: only the flagged pairs run
};
// The backward's per-chunk parts over given intermediates (chunk_bwd_parts.hip), float32.
enum { PART_DA = 0, PART_DV = 1, PART_DQK_INTRA = 2, PART_DQKG = 3 };
struct PartArgs {
  const float *q, *k, *v, *g, *A, *dA, *dout, *h, *dh, *dq, *dk;  // as each part needs
  float *out0, *out1, *out2;
  float scale;
  int H, K, V;
  long NC;  // chunks (B * T / C)
};
hipError_t run_bwd_part(int which, const PartArgs& p, int C, hipStream_t st);

// RMSNorm with optional SiLU gate and weight, and the log-sigmoid gate (norm_gate.hip).
struct NormGateArgs {
  const void *x, *g;     // [rows, D] input dtype; g nullable
  const float* w;        // [D] nullable
  void* y;               // forward output
  float* rstd;           // [rows] (forward: nullable; backward: input)
  const void* dy;        // backward
  void *dx, *dg;         // backward outputs (dg when g is given)
  float* dw_part;        // [norm_gate_bwd_blocks(rows), D] workspace for dw (nullable)
  long rows;
  int D;
  float eps;
};
long norm_gate_bwd_blocks(long rows);
hipError_t run_norm_gate_fwd(const NormGateArgs& p, int dtype, hipStream_t st);
hipError_t run_norm_gate_bwd(const NormGateArgs& p, float* dw, int dtype, hipStream_t st);
hipError_t run_gate(const void* x, const void* dy, void* out, long count, float inv_n,
                    int has_clamp, float clamp, int dtype, hipStream_t st);

// out[c] = sum_b part[b][c] for c < M (deterministic column sums of per-block partials).
hipError_t run_rows_sum(const float* part, int nblk, int M, float* out, hipStream_t st);
// dst [rows, sum w_i] = [src_0 | src_1 | ...] row by row (norm_gate.hip); widths in elements
// of esize bytes, each a multiple of 16 bytes, at most kConcatMax sources.
constexpr int kConcatMax = 8;
hipError_t run_concat_cols(const void* const* src, const long* widths, int nsrc, long rows,
                           void* dst, int esize, hipStream_t st);

// Causal depthwise convolution with optional bias and SiLU (short_conv.hip).
struct ShortConvArgs {
  const void *x, *dy;   // [tokens, D] input dtype
  void *y, *dx;
  const float* w;       // [D][W]
  const float* bias;    // [D] nullable
  float* part;          // backward: [short_conv_part_rows, (W + 1) * D] (nullable: no dw/db)
  float* dwb;           // backward: dw [D][W] then db [D]
  int D, W, silu;
  int max_len;          // longest sequence (varlen grid)
  SeqInfo si;           // C unused
};
long short_conv_part_rows(long nseq, long len);   // len: T, or the longest sequence
hipError_t run_short_conv(const ShortConvArgs& p, bool backward, int dtype, hipStream_t st);

bool recurrent_supported(int K, int V);  // state rows K (forward) and V, K (backward)
hipError_t run_recurrent_bwd(const RecBwdArgs& p, int dtype, int o_dtype, hipStream_t st);

// Full-head kernels (chunk_head.hip): bf16, chunk 64, raw gates, K and V multiples of 8
// (16-byte aligned rows); scans and forward for K <= 256 and any V (V tiles of 64 or 128
// columns), the fused backward for K, V <= 128. Optional sequence segments (fixed-length
// sequences): seg_state [N, NS, H, K, V] f32 and seg_gam [N, NS, H, K] f32 workspaces.
bool head_supported(int dtype, int C, int K, int V, bool g_is_cumsum);   // scans, forward
bool head_bwd_supported(int K, int V);                                     // + backward
int head_vtiles(int K, int V);   // V tiles (blocks per segment and head)
void head_seg_plan(int N, int H, int T, int C, bool varlen, int& NS, int& SL, int VT);
long head_seg_ws_bytes(int N, int NS, int H, int K, int V);
long head_gate_ws_bytes(int N, int T, int H, int K, int V);   // 0 unless it pays

// Full-head kernels. Gates: g ([T, H, K] bf16, raw) or, with g == nullptr, the scalar
// gates of simple GLA: gate(t, h) = gs[t * gs_ts + h] for every key column (float; gs_ts = H
// for per-token gates, 0 for a per-head constant).
struct HeadScanArgs {
  const void *a, *b, *g;  // forward: k, v ; reverse: q, do
  const float* gs;
  long gs_ts;
  const float* s_init;    // forward: h0 ; reverse: dht (nullable)
  void* s_all;            // per-chunk states [NC, H, K, V] bf16 (nullable)
  float* s_final;         // forward: ht ; reverse: dh0 (nullable)
  float* seg_state;       // NS > 1 only
  float* seg_gam;
  int NS, SL;
  int pass, s_begin, ns_launch;   // set by the launcher
  // per-chunk gating workspace of wide heads (nullable): the scans then stream qs (reverse)
  // or kg (forward) and the column factors instead of gating in every V tile's block
  const void* gate_ws;
  float scale;            // reverse only
  int H, K, V;
  SeqInfo si;
};
hipError_t run_head_scan(const HeadScanArgs& p, bool reverse, hipStream_t st);

struct HeadFwdArgs {
  const void *q, *k, *v, *g;
  const float* gs;
  long gs_ts;
  const float* h0;        // nullable
  void* o;
  void* h_out;            // [NC, H, K, V] bf16 (nullable)
  void* gate_ws;          // per-chunk gating workspace of wide heads (nullable; fixed length)
  float* ht;              // nullable
  float* seg_state;       // NS > 1 only
  float* seg_gam;
  int NS, SL;
  float scale;
  int H, K, V;
  SeqInfo si;
  // nullable: gate-range flags. head_fwd_kernel: per block (GateFlags, vt = V tiles); with
  // a gating workspace (K = 256) the gating kernel's per-chunk flags [NC, H] instead
  int* flags;
};
hipError_t run_head_fwd(const HeadFwdArgs& p, hipStream_t st);
// Per-chunk gating of wide heads (K = 256) into p.gate_ws (q, k, g, scale, H, K, si read;
// per-chunk gate-range flags [NC, H] into p.flags when given).
hipError_t run_head_gate(const HeadFwdArgs& p, hipStream_t st);

struct HeadBwdArgs {
  const void *q, *k, *v, *g, *dout;
  const float* gs;
  long gs_ts;
  const void* h;          // [NC, H, K, V] bf16 forward states (chunk start)
  const float* dht;       // nullable
  void *dq, *dk, *dv, *dg;  // dg nullable with scalar gates
  float* dh0;             // nullable
  float* seg_state;       // NS > 1 only
  float* seg_gam;
  int NS, SL;
  float scale;
  int H, K, V;
  SeqInfo si;
  int* flags;             // nullable: per-block gate-range flags (GateFlags layout, vt = 1)
};
hipError_t run_head_bwd(const HeadBwdArgs& p, hipStream_t st);

// Per-chunk dq, dk, dg of the per-chunk backward for bf16 heads of K in (64, 256] (any V,
// multiples of 8), chunk 64: one block per (chunk, head), V streamed in 64-column tiles
// (chunk_head.hip). p.gate_ws, p.dv and p.vec are not used.
bool head_dqkg_supported(int K, int V);
hipError_t run_head_dqkg(const BwdArgs& p, hipStream_t st);

// Optional HIP-event timing of the fused full-head kernels (a measurement hook): when
// enabled, an event is recorded on the launch stream right before and after the kernel.
enum { KT_HEAD_FWD = 0, KT_HEAD_BWD = 1, KT_REC_FWD = 2, KT_BWD_DQKG = 3, KT_COUNT = 4 };
void ktimer_mark(int which, bool stop, hipStream_t st);

}  // namespace tops
