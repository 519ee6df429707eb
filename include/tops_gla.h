/*
 * tops_gla.h -- C ABI of the MI355X (gfx950) Gated Linear Attention kernels.
 *
 * This is the drop-in boundary for the reference's GLA hot path (package `tops`,
 * primatrix/pallas-kernel). The reference has no native boundary: its Python functions
 * lower to `pl.pallas_call` custom calls. Each entry point below replaces one of those
 * launch sites (cited per function) and is what an XLA typed-FFI handler or a ctypes
 * binding calls.
 *
 * Conventions (all entry points):
 *  - Tensors are device pointers (HBM), row-major, in the reference layout: q/k/g
 *    [B, T, H, K], v/o/do [B, T, H, V], states [N, H, K, V]. No pointer is retained.
 *  - `dtype` is the element type of q, k, v, g, o and of the q/k/v/g/do gradients:
 *    TOPS_GLA_F32 or TOPS_GLA_BF16. Initial/final states and their gradients are float32.
 *  - Sequences: fixed-length when `cu_seqlens == NULL` (B sequences of T tokens, N == B);
 *    otherwise B must be 1, `cu_seqlens` is a device int32 array [N + 1] of token offsets
 *    and `chunk_offsets` a device int32 array [N + 1] with the prefix sums of
 *    ceil(len_i / chunk_size); `NC` is the total number of chunks (chunk_offsets[N]).
 *    Every sequence holds at least one token (cu_seqlens strictly increasing, ending at most
 *    at T): the library cannot read device offsets on the host, so this is the caller's
 *    precondition (the Python layer checks it before the call).
 *    For fixed-length calls NC must equal B * ceil(T / chunk_size).
 *  - Per-chunk state buffers ([NC, H, K, V], element type `dtype`) are caller-provided
 *    workspaces; the library allocates nothing.
 *  - Sizes: B * T and NC * H below 2^31; a tensor may hold more than 2^31 elements (the
 *    kernels form global offsets from 64-bit bases).
 *  - Work is enqueued on `stream` (a hipStream_t); nothing synchronizes the device.
 *  - Return value: TOPS_GLA_OK, or an error code with a message from
 *    tops_gla_last_error() (thread-local). Invalid arguments never launch a kernel.
 *  - chunk_size: 16, 32 or 64 for the MFMA kernels; also 4 and 8 for tops_gla_chunk_fwd_h,
 *    tops_gla_chunk_bwd_dh and tops_gla_chunk_fwd_o (float32 vector kernels, K <= 2048,
 *    seg_ws unused); any power of two for the cumsum.
 */
#ifndef TOPS_GLA_H_
#define TOPS_GLA_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum tops_gla_status {
  TOPS_GLA_OK = 0,
  TOPS_GLA_EINVAL = 1,      /* bad shape / pointer / flag */
  TOPS_GLA_EUNSUPPORTED = 2, /* valid for the reference, not supported by these kernels */
  TOPS_GLA_EHIP = 3          /* HIP launch error */
};

enum tops_gla_dtype { TOPS_GLA_F32 = 0, TOPS_GLA_BF16 = 1 };

/* Message describing the last error on the calling thread ("" if none). */
const char* tops_gla_last_error(void);

/* Library version string. */
const char* tops_gla_version(void);

/*
 * Chunk-local (optionally reverse, scaled) prefix sum of gates over the last-but-one axis
 * groups of `chunk_size` tokens, restarting at every sequence start.
 * Replaces: chunk_cumsum_kernel launch, tops/ops/gla/chunk.py:176-189
 *           (chunk_local_cumsum_vector, chunk.py:110-198).
 * g/out: [B, T, H, S] (or [B, H, T, S] when head_first), element types in_dtype/out_dtype.
 */
int tops_gla_chunk_local_cumsum(const void* g, void* out, int64_t B, int64_t T, int64_t H,
                                int64_t S, int chunk_size, int reverse, int has_scale,
                                float scale, int head_first, const int32_t* cu_seqlens,
                                const int32_t* chunk_offsets, int64_t N, int64_t NC,
                                int in_dtype, int out_dtype, void* stream);

/*
 * Inter-chunk state scan: h[c] = state entering chunk c ([NC, H, K, V], dtype), and the
 * final state ht [N, H, K, V] (float32). g holds raw log-gates (the chunk-local cumsum is
 * taken in-kernel) or, with g_is_cumsum, the cumsum itself. h0/h/ht may be NULL; seg_ws
 * as for tops_gla_chunk_fwd.
 * Replaces: chunk_fwd_h_kernel launch, tops/ops/common/chunk_h.py:252-271
 *           (body :18-119; jnp ref tops/ops/gla/chunk.py:206-292).
 */
int tops_gla_chunk_fwd_h(const void* k, const void* v, const void* g, int g_is_cumsum,
                         const float* h0, void* h, float* ht, void* seg_ws,
                         int64_t seg_ws_bytes, int64_t B, int64_t T, int64_t H, int64_t K,
                         int64_t V, int chunk_size, const int32_t* cu_seqlens,
                         const int32_t* chunk_offsets, int64_t N, int64_t NC, int dtype,
                         void* stream);

/*
 * Reverse state-gradient scan: dh[c] = dL/d(state leaving chunk c) ([NC, H, K, V], dtype),
 * dh0 [N, H, K, V] float32 (may be NULL). dht may be NULL (zero); seg_ws as for
 * tops_gla_chunk_fwd.
 * Replaces: chunk_bwd_dh_kernel launch, tops/ops/common/chunk_h.py:681-695
 *           (body :495-591; jnp ref chunk_bwd_dh_ref :399-492).
 */
int tops_gla_chunk_bwd_dh(const void* q, const void* g, int g_is_cumsum, const void* dout,
                          const float* dht, void* dh, float* dh0, void* seg_ws,
                          int64_t seg_ws_bytes, float scale, int64_t B, int64_t T, int64_t H,
                          int64_t K, int64_t V, int chunk_size, const int32_t* cu_seqlens,
                          const int32_t* chunk_offsets, int64_t N, int64_t NC, int dtype,
                          void* stream);

/*
 * Per-chunk intra matrix and output. A_out (float32, [NC * chunk_size, H, chunk_size],
 * unmasked, scaled) and o ([B, T, H, V], dtype) are optional; with A_in the given matrix
 * is used (causally masked) instead of recomputing it; h ([NC, H, K, V], dtype) may be NULL
 * (no inter-chunk term).
 * Replaces: chunk_gla_fwd_intra_gk launch, tops/ops/gla/chunk.py:416-427, and
 *           chunk_gla_fwd_o_gk_pl launch, chunk.py:1360-1376 (bodies :350-383, :1259-1312).
 */
int tops_gla_chunk_fwd_o(const void* q, const void* k, const void* v, const void* g,
                         int g_is_cumsum, const void* h, const float* A_in, float* A_out,
                         void* o, float scale, int64_t B, int64_t T, int64_t H, int64_t K,
                         int64_t V, int chunk_size, const int32_t* cu_seqlens,
                         const int32_t* chunk_offsets, int64_t N, int64_t NC, int dtype,
                         void* stream);

/*
 * Bytes of the optional workspace (`seg_ws`) of tops_gla_chunk_fwd (backward = 0) or
 * tops_gla_chunk_bwd (backward = 1) for this problem (0: the call does not use one); N =
 * sequences (B, or the number of cu_seqlens sequences with varlen = 1). Parts, each
 * 256-byte aligned, in this order:
 *  - sequence segments (full-head kernels, fixed length): the inter-chunk scans run as
 *    parallel segments (local states, then all segments at once, each folding its entry
 *    state from them) instead of one chunk after another;
 *  - gate-range flags (K <= 512): the chunk kernels factor e^{g~_i - g~_j} per element as
 *    e^{g~_i - r} e^{r - g~_j} about each column's chunk midpoint r, which holds while
 *    |g~ - r| <= 100 log(2) (a chunk's gate range up to about 138 in natural log units).
 *    Every chunk is checked (by the full-head kernels as they gate it, by the wide heads'
 *    gating kernel, or by a check kernel on the other paths), and the recurrent scans
 *    (exact for any decay) then recompute the flagged sequences and heads: o and ht in the
 *    forward; dq, dk, dv, dg and dh0 in the backward (K and V <= 512). Without this part a
 *    gate range beyond the limit gives non-finite or inaccurate values;
 *  - wide heads (K = 256, three or more 64-column V tiles, fixed length): the per-chunk
 *    gating that the scans, the forward and the dv kernel then stream;
 *  - backward only: the fallback's final states (f32 [N, H, K, V], K and V <= 512; without
 *    it a call with dht is not checked).
 * A shorter workspace drops the later parts. The per-chunk states h_ws that the forward
 * stores for flagged pairs are not meaningful (the backward recomputes those pairs).
 * No counterpart in the reference (its scans are sequential grid axes, chunk_h.py:252-271).
 */
int64_t tops_gla_chunk_ws_bytes(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V,
                                int chunk_size, int64_t N, int varlen, int dtype,
                                int backward);

/*
 * 1 when the full-head kernels run this shape (16-byte aligned buffers assumed): the
 * forward and the scans (backward = 0), or also the fused backward (backward = 1). On those
 * paths tops_gla_chunk_fwd's h_ws may be NULL (no states kept) and tops_gla_chunk_bwd's
 * dh_ws is not used (may be NULL). No counterpart in the reference (workspace sizing).
 */
int tops_gla_full_head(int64_t K, int64_t V, int chunk_size, int dtype, int backward);

/*
 * chunk_gla forward: inter-chunk states into h_ws ([NC, H, K, V], dtype: the residual the
 * backward reuses) and the per-chunk output. h_ws may be NULL on the full-head path (then
 * no states are stored); the other paths need it. h0/ht may be NULL. seg_ws (256-byte
 * aligned, seg_ws_bytes >= tops_gla_chunk_ws_bytes) may be NULL.
 * Replaces the device part of chunk_gla_fwd, tops/ops/gla/chunk.py:1145-1166.
 */
int tops_gla_chunk_fwd(const void* q, const void* k, const void* v, const void* g,
                       const float* h0, void* o, float* ht, void* h_ws, void* seg_ws,
                       int64_t seg_ws_bytes, float scale, int64_t B, int64_t T, int64_t H,
                       int64_t K, int64_t V, int chunk_size, const int32_t* cu_seqlens,
                       const int32_t* chunk_offsets, int64_t N, int64_t NC, int dtype,
                       void* stream);

/*
 * tops_gla_chunk_fwd without a caller workspace. No counterpart in the reference: for callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Arguments and results are those of tops_gla_chunk_fwd
 * without seg_ws / seg_ws_bytes; the caller still passes every input and output (and h_ws
 * where tops_gla_chunk_fwd requires it). The first two parts of the tops_gla_chunk_ws_bytes
 * workspace (sequence segments, gate-range flags) live in a file-scope device array of
 * 24 MiB per GPU (held by each GPU the library runs on until the process ends), whose
 * address is taken once per device on the first call with that device current; a shape
 * that needs more returns TOPS_GLA_EINVAL (the segment part never exceeds 17.04 MB; the
 * flags take 4 bytes per chunk and head, or per sequence, head, segment and V tile where
 * that is more). The wide heads' per-chunk
 * gating workspace is not used. Nothing here calls hipMalloc or hipFree.
 * Every call on one GPU shares that array: calls that overlap on one GPU (other streams,
 * other threads) race and must be serialized by the caller. Each call writes every part of
 * the array it later reads, so nothing needs clearing between calls.
 */
int tops_gla_chunk_fwd_noalloc(const void* q, const void* k, const void* v, const void* g,
                               const float* h0, void* o, float* ht, void* h_ws, float scale,
                               int64_t B, int64_t T, int64_t H, int64_t K, int64_t V,
                               int chunk_size, const int32_t* cu_seqlens,
                               const int32_t* chunk_offsets, int64_t N, int64_t NC, int dtype,
                               void* stream);

/*
 * chunk_gla backward: (dq, dk, dv, dg, dh0). `h` are the forward states ([NC, H, K, V]); if
 * NULL they are recomputed into h_ws (then required). dh_ws ([NC, H, K, V], dtype) is
 * required off the fused full-head backward (tops_gla_full_head(..., 1)), which does not use
 * it. h0, dht and dh0 may be NULL; seg_ws as for tops_gla_chunk_fwd.
 * Replaces the device part of chunk_gla_bwd_with_pl, tops/ops/gla/chunk.py:1019-1064
 * (chunk_bwd_dh_kernel + chunk_gla_bwd_fused_pl, :1482-1550).
 */
int tops_gla_chunk_bwd(const void* q, const void* k, const void* v, const void* g,
                       const float* h0, const void* h, const void* dout, const float* dht,
                       void* dq, void* dk, void* dv, void* dg, float* dh0, void* h_ws,
                       void* dh_ws, void* seg_ws, int64_t seg_ws_bytes, float scale,
                       int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int chunk_size,
                       const int32_t* cu_seqlens, const int32_t* chunk_offsets, int64_t N,
                       int64_t NC, int dtype, void* stream);

/*
 * Scalar-gate (simple GLA) forward on the full-head kernels: the gate of token t (global row
 * of the [B * T] token axis) and head h is gs[t * gs_ts + h] for every key column (float32;
 * gs_ts = H for per-token gates [B * T, H], 0 for a per-head constant [H] such as g_gamma),
 * raw per-step log-decays (the kernels take their chunk-local cumsum). Otherwise as
 * tops_gla_chunk_fwd; only shapes with tops_gla_full_head(K, V, 64, dtype, 0) == 1 are taken
 * (TOPS_GLA_EUNSUPPORTED otherwise).
 * Replaces the device part of chunk_simple_gla_fwd, tops/ops/simple_gla/chunk.py:471-519
 * (chunk_fwd_h_kernel with g / g_gamma, tops/ops/common/chunk_h.py:82-91, and
 * chunk_fwd_o, tops/ops/common/chunk_o.py:165-240), and chunk_gla's g_gamma path,
 * tops/ops/gla/chunk.py:1134-1143.
 */
int tops_gla_simple_chunk_fwd(const void* q, const void* k, const void* v, const float* gs,
                              int64_t gs_ts, const float* h0, void* o, float* ht, void* h_ws,
                              void* seg_ws, int64_t seg_ws_bytes, float scale, int64_t B,
                              int64_t T, int64_t H, int64_t K, int64_t V, int chunk_size,
                              const int32_t* cu_seqlens, const int32_t* chunk_offsets, int64_t N,
                              int64_t NC, int dtype, void* stream);

/*
 * Scalar-gate backward: (dq, dk, dv[, dg][, dh0]) with gates as tops_gla_simple_chunk_fwd.
 * dg ([B, T, H, K], dtype: the gradient of the per-column gates, whose sum over the key
 * columns is the scalar gate's gradient) may be NULL. h / h_ws as tops_gla_chunk_bwd. Only
 * shapes with tops_gla_full_head(K, V, 64, dtype, 1) == 1 (TOPS_GLA_EUNSUPPORTED otherwise).
 * Replaces the device part of chunk_simple_gla_bwd, tops/ops/simple_gla/chunk.py:538-615
 * (chunk_bwd_dh_kernel with g_gamma, chunk_h.py:552-563, and chunk_simple_gla_bwd_o_pl,
 * tops/ops/common/chunk_o.py:19-163).
 */
int tops_gla_simple_chunk_bwd(const void* q, const void* k, const void* v, const float* gs,
                              int64_t gs_ts, const float* h0, const void* h, const void* dout,
                              const float* dht, void* dq, void* dk, void* dv, void* dg,
                              float* dh0, void* h_ws, void* seg_ws, int64_t seg_ws_bytes,
                              float scale, int64_t B, int64_t T, int64_t H, int64_t K, int64_t V,
                              int chunk_size, const int32_t* cu_seqlens,
                              const int32_t* chunk_offsets, int64_t N, int64_t NC, int dtype,
                              void* stream);

/*
 * Per-chunk dq, dk, dg of the backward (intra-chunk dA computed in-kernel) from the forward
 * states h and the state gradients dh (both [NC, H, K, V], dtype, as produced by
 * tops_gla_chunk_fwd_h / tops_gla_chunk_bwd_dh on raw gates g).
 * Replaces: the dq/dk/dg part of chunk_gla_bwd_fused_kernel, tops/ops/gla/chunk.py:1423-1479
 *           (launch :1482-1550), i.e. the composition of chunk_gla_bwd_dA_ref,
 *           chunk_gla_bwd_dqk_intra_ref and chunk_gla_bwd_dqkg_ref (:504-539, :603-743) in one
 *           pass; tops_gla_bwd_part_* below replace those three one by one.
 */
int tops_gla_chunk_bwd_dqkg(const void* q, const void* k, const void* v, const void* g,
                            const void* h, const void* dout, const void* dh, void* dq, void* dk,
                            void* dg, float scale, int64_t B, int64_t T, int64_t H, int64_t K,
                            int64_t V, int chunk_size, const int32_t* cu_seqlens,
                            const int32_t* chunk_offsets, int64_t N, int64_t NC, int dtype,
                            void* stream);

/*
 * Per-chunk dv = tril(A)^T do + (k e^{gamma - g~}) dh (A recomputed in-kernel).
 * Replaces: the dv part of chunk_gla_bwd_fused_kernel, tops/ops/gla/chunk.py:1423-1479
 *           (chunk_gla_bwd_dv_ref :547-595 on an in-kernel A; tops_gla_bwd_part_dv takes A).
 */
int tops_gla_chunk_bwd_dv(const void* q, const void* k, const void* g, const void* dout,
                          const void* dh, void* dv, float scale, int64_t B, int64_t T,
                          int64_t H, int64_t K, int64_t V, int chunk_size,
                          const int32_t* cu_seqlens, const int32_t* chunk_offsets, int64_t N,
                          int64_t NC, int dtype, void* stream);

/*
 * The backward's four per-chunk parts over given intermediates, for callers that hold them
 * (the fused entry points above recompute A and dA in-kernel instead). All tensors float32,
 * [B, T, H, *] with T a multiple of chunk_size (16, 32 or 64); A and dA [B, T, H, C];
 * h / dh [B * T / C, H, K, V]; g_cumsum is the chunk-local cumsum of the gates.
 * Replace the reference's jnp functions:
 *   tops_gla_bwd_part_dA         chunk_gla_bwd_dA_ref          tops/ops/gla/chunk.py:504-539
 *   tops_gla_bwd_part_dv         chunk_gla_bwd_dv_ref          tops/ops/gla/chunk.py:547-595
 *   tops_gla_bwd_part_dqk_intra  chunk_gla_bwd_dqk_intra_ref   tops/ops/gla/chunk.py:603-648
 *   tops_gla_bwd_part_dqkg       chunk_gla_bwd_dqkg_ref        tops/ops/gla/chunk.py:656-743
 */
int tops_gla_bwd_part_dA(const float* v, const float* dout, float* dA, float scale, int64_t B,
                         int64_t T, int64_t H, int64_t V, int chunk_size, void* stream);
int tops_gla_bwd_part_dv(const float* k, const float* g_cumsum, const float* A,
                         const float* dout, const float* dh, float* dv, int64_t B, int64_t T,
                         int64_t H, int64_t K, int64_t V, int chunk_size, void* stream);
int tops_gla_bwd_part_dqk_intra(const float* q, const float* k, const float* g_cumsum,
                                const float* dA, float* dq, float* dk, int64_t B, int64_t T,
                                int64_t H, int64_t K, int chunk_size, void* stream);
int tops_gla_bwd_part_dqkg(const float* q, const float* k, const float* v, const float* h,
                           const float* g_cumsum, const float* dout, const float* dh,
                           const float* dq, const float* dk, float* dq_out, float* dk_out,
                           float* dg, float scale, int64_t B, int64_t T, int64_t H, int64_t K,
                           int64_t V, int chunk_size, void* stream);

/*
 * Fused recurrent forward. gk [B, T, H, K] / gv [B, T, H, V] gates may be NULL; o is
 * written in o_dtype (the reference returns float32); h0/ht float32, may be NULL. K <= 512.
 * Replaces: _fused_recurrent_gla_fwd pallas_call, tops/ops/gla/fused_recurrent.py:344-362
 *           (body :139-227).
 */
int tops_gla_fused_recurrent_fwd(const void* q, const void* k, const void* v, const void* gk,
                                 const void* gv, const float* h0, void* o, float* ht,
                                 float scale, int reverse, int64_t B, int64_t T, int64_t H,
                                 int64_t K, int64_t V, const int32_t* cu_seqlens, int64_t N,
                                 int dtype, int o_dtype, void* stream);

/*
 * Fused recurrent backward: dq, dk, dv [B, T, H, K|V] float32 (the reference's output
 * dtype), dgk / dgv float32 for the gates that are given (NULL otherwise), dh0 [N, H, K, V]
 * float32 (NULL: not computed). o is the forward output in float32, required with gv.
 * h0 / dht float32, may be NULL. ht_ws: caller workspace of N*H*K*V floats that receives the
 * recomputed final state; required when dht and a gate are given, else may be NULL.
 * K and V up to 512.
 * Replaces: _fused_recurrent_gla_bwd pallas_call + _compute_gate_grads,
 *           tops/ops/gla/fused_recurrent.py:776-795 and :798-876 (body :495-624, entry
 *           :879-956).
 */
int tops_gla_fused_recurrent_bwd(const void* q, const void* k, const void* v, const void* gk,
                                 const void* gv, const float* o, const void* dout,
                                 const float* dht, const float* h0, float* dq, float* dk,
                                 float* dv, float* dgk, float* dgv, float* dh0, float* ht_ws,
                                 float scale, int reverse, int64_t B, int64_t T, int64_t H,
                                 int64_t K, int64_t V, const int32_t* cu_seqlens, int64_t N,
                                 int dtype, void* stream);

/*
 * The GLA layer's stages around the attention core (rows = tokens x heads, D features per
 * row, D % 8 == 0, 16-byte aligned buffers; x, g, y, dy, dx, dg in `dtype`, w / dw float32):
 * RMSNorm with optional weight w and SiLU gate g:  y = x rsqrt(mean(x^2) + eps) [w] [silu(g)].
 * The forward keeps rstd [rows] (float32, may be NULL) for the backward. The backward writes
 * dx, dg (when g is given) and dw (when w is given; it needs dw_ws of
 * tops_gla_rmsnorm_ws_bytes(rows, D) bytes).
 * Replaces: FusedRMSNormGated.__call__, tops/modules/fused_norm_gate.py:28-37, and
 *           RMSNorm.__call__, tops/modules/layernorm.py:28-35 (g = NULL).
 */
int tops_gla_rmsnorm_gated_fwd(const void* x, const void* g, const float* w, void* y,
                               float* rstd, int64_t rows, int64_t D, float eps, int dtype,
                               void* stream);
int tops_gla_rmsnorm_gated_bwd(const void* x, const void* g, const float* w, const float* rstd,
                               const void* dy, void* dx, void* dg, float* dw, void* dw_ws,
                               int64_t dw_ws_bytes, int64_t rows, int64_t D, int dtype,
                               void* stream);
int64_t tops_gla_rmsnorm_ws_bytes(int64_t rows, int64_t D);

/*
 * Key-wise decay gate: y = max(log_sigmoid(x) / normalizer, clamp_min) (clamp when
 * has_clamp), element-wise over count elements; the backward writes
 * dx = dy sigmoid(-x) / normalizer where y was not clamped.
 * Replaces: tops/layers/gla.py:286-288 (jax.nn.log_sigmoid(gk) / gate_logit_normalizer,
 *           jnp.clip(gk, a_min=clamp_min)).
 */
int tops_gla_gate_logsigmoid_fwd(const void* x, void* y, int64_t count, float normalizer,
                                 int has_clamp, float clamp_min, int dtype, void* stream);
int tops_gla_gate_logsigmoid_bwd(const void* x, const void* dy, void* dx, int64_t count,
                                 float normalizer, int has_clamp, float clamp_min, int dtype,
                                 void* stream);

/*
 * Row-wise concatenation: dst [rows, sum w_j] = [src_0 | ... | src_{nsrc-1}], each source
 * [rows, w_j] row-major (1 <= nsrc <= 8; every w_j a positive multiple of 16 bytes; 16-byte
 * aligned buffers).
 * No counterpart in the reference: the layer's backward joins the output gradients of its
 * wide projections so that one GEMM pair forms their input and weight gradients
 * (tops/layers/gla.py:259-262, 333: separate dense layers there).
 */
int tops_gla_concat_cols(const void* const* srcs, const int64_t* widths, int nsrc,
                         int64_t rows, void* dst, int dtype, void* stream);

/*
 * Causal depthwise convolution of a [B, T, D] sequence (varlen: B = 1 and cu_seqlens [N+1];
 * max_len = the longest sequence), kernel width W <= 8, weight w [D][W] float32, optional
 * bias [D] float32, optional SiLU; rows before a sequence's first token read as zero.
 * D % 8 == 0, 16-byte aligned buffers. The backward writes dx and, when dw_db is given,
 * dw [D][W] then db [D] (float32) using ws of tops_gla_short_conv_ws_bytes bytes.
 * Replaces: ShortConvolution._causal_conv1d, tops/modules/convolution.py:46-78.
 */
int tops_gla_short_conv_fwd(const void* x, const float* w, const float* bias, void* y,
                            int64_t B, int64_t T, int64_t D, int W, int silu,
                            const int32_t* cu_seqlens, int64_t N, int64_t max_len, int dtype,
                            void* stream);
int tops_gla_short_conv_bwd(const void* x, const float* w, const float* bias, const void* dy,
                            void* dx, float* dw_db, void* ws, int64_t ws_bytes, int64_t B,
                            int64_t T, int64_t D, int W, int silu, const int32_t* cu_seqlens,
                            int64_t N, int64_t max_len, int dtype, void* stream);
int64_t tops_gla_short_conv_ws_bytes(int64_t B, int64_t T, int64_t D, int W, int64_t N,
                                     int64_t max_len, int varlen);

/*
 * Measurement hook (no counterpart in the reference): with timing enabled, HIP events are
 * recorded on the launch stream around every launch of the fused full-head forward
 * (which = 0) and backward (which = 1) kernels (tops_gla_chunk_fwd / _bwd and the
 * scalar-gate entry points), of the recurrent forward scan (which = 2,
 * tops_gla_fused_recurrent_fwd) and of the per-chunk dq / dk / dg kernel (which = 3, the
 * backward of shapes off the fused full-head backward, e.g. K = 256). tops_gla_kernel_ms waits for the last such launch and
 * returns the average duration in ms of the launches recorded since timing was enabled (the
 * last 256 of them; -1 if there is none).
 * A profiling aid with process-wide state: the first enable creates the host-side event
 * objects (no device memory); while timing is on, the marks of concurrent callers are
 * serialized by a lock and their launches share one count, so timings are meaningful for a
 * single caller. While timing is off (the default) the launch paths only read a flag and
 * every other entry point keeps its reentrancy.
 */
int tops_gla_kernel_timing(int enable);
float tops_gla_kernel_ms(int which);

#ifdef __cplusplus
}
#endif

#endif /* TOPS_GLA_H_ */
