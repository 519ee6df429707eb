// extern "C" entry points declared in include/tops_gla.h: argument validation, sequence
// layout, and kernel dispatch. No entry point allocates device memory or synchronizes (the
// measurement hook at the end, a profiling aid, creates host-side HIP events once and its
// reading call waits for its last event).
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <initializer_list>
#include <mutex>

#include "../../include/tops_gla.h"
#include "common.hpp"
#include "kernels.hpp"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = '\0';
  return TOPS_GLA_OK;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return ok();
  return fail(TOPS_GLA_EHIP, "%s: %s", what, hipGetErrorString(e));
}

bool dtype_ok(int d) { return d == TOPS_GLA_F32 || d == TOPS_GLA_BF16; }

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// 16-byte vector access is valid when K and V rows are whole 16-byte pieces and every
// base pointer is 16-byte aligned (NULL counts as aligned).
int vec_ok(int dtype, int64_t K, int64_t V, std::initializer_list<const void*> ptrs) {
  const int epp = dtype == TOPS_GLA_BF16 ? 8 : 4;
  if (K % epp != 0 || V % epp != 0) return 0;
  for (const void* p : ptrs)
    if (!aligned16(p)) return 0;
  return 1;
}

constexpr int64_t kMaxInt = 2147483647;

// Validates the sequence description and fills a SeqInfo.
int make_seq(int64_t B, int64_t T, int64_t H, int chunk, const int32_t* cu,
             const int32_t* chunk_off, int64_t N, int64_t NC, bool need_chunk_off,
             tops::SeqInfo* si) {
  if (B < 0 || T < 0 || H <= 0) return fail(TOPS_GLA_EINVAL, "bad B/T/H (%lld, %lld, %lld)",
                                            (long long)B, (long long)T, (long long)H);
  if (chunk <= 0) return fail(TOPS_GLA_EINVAL, "chunk_size must be positive");
  if (B * T > kMaxInt) return fail(TOPS_GLA_EUNSUPPORTED, "B*T exceeds 2^31 tokens");
  si->C = chunk;
  if (cu == nullptr) {
    const int64_t nt = (T + chunk - 1) / chunk;
    if (NC != B * nt)
      return fail(TOPS_GLA_EINVAL, "NC (%lld) != B * ceil(T / chunk_size) (%lld)",
                  (long long)NC, (long long)(B * nt));
    si->N = (int)B;
    si->T = (int)T;
    si->NC = (int)NC;
    si->cu = nullptr;
    si->chunk_cu = nullptr;
  } else {
    if (B != 1) return fail(TOPS_GLA_EINVAL, "cu_seqlens requires B == 1 (got %lld)",
                            (long long)B);
    if (N <= 0) return fail(TOPS_GLA_EINVAL, "cu_seqlens needs N >= 1 sequences");
    if (need_chunk_off && chunk_off == nullptr)
      return fail(TOPS_GLA_EINVAL, "chunk_offsets is required with cu_seqlens");
    if (NC < 0 || NC > kMaxInt) return fail(TOPS_GLA_EINVAL, "bad NC");
    si->N = (int)N;
    si->T = (int)T;
    si->NC = (int)NC;
    si->cu = cu;
    si->chunk_cu = chunk_off;
  }
  if ((int64_t)si->NC * H > kMaxInt) return fail(TOPS_GLA_EUNSUPPORTED, "NC*H too large");
  return TOPS_GLA_OK;
}

bool small_chunk(int chunk) { return chunk == 4 || chunk == 8; }

// Chunk sizes 4 and 8 (the sub-functions' small-chunk kernels): no layout limits beyond K
// (the output kernel holds 2 x chunk x K floats of the chunk in LDS).
int check_small_common(int64_t K, int64_t V, int dtype) {
  if (!dtype_ok(dtype)) return fail(TOPS_GLA_EINVAL, "dtype must be F32 (0) or BF16 (1)");
  if (K <= 0 || V <= 0) return fail(TOPS_GLA_EINVAL, "K and V must be positive");
  if (K > tops::small_chunk_max_k())
    return fail(TOPS_GLA_EUNSUPPORTED, "K=%lld exceeds %d at chunk sizes 4 and 8",
                (long long)K, tops::small_chunk_max_k());
  return TOPS_GLA_OK;
}

int check_mfma_common(int64_t K, int64_t V, int chunk, int dtype) {
  if (!dtype_ok(dtype)) return fail(TOPS_GLA_EINVAL, "dtype must be F32 (0) or BF16 (1)");
  if (K <= 0 || V <= 0) return fail(TOPS_GLA_EINVAL, "K and V must be positive");
  if (chunk != 16 && chunk != 32 && chunk != 64)
    return fail(TOPS_GLA_EUNSUPPORTED, "chunk_size %d: the MFMA kernels take 16, 32 or 64",
                chunk);
  // LDS of the per-chunk output kernel grows with K (all K tiles of q e^{g} stay resident)
  const int64_t esz = dtype == TOPS_GLA_BF16 ? 2 : 4;
  const int64_t CP = chunk < 32 ? 32 : chunk;
  const int64_t pad = 16 / esz;
  const int64_t KP = (K + 63) / 64 * 64;
  const int64_t lds = chunk * (KP + pad) * esz + KP * 4 + chunk * (64 + pad) * esz +
                      chunk * (CP + pad) * esz + 64 * (CP + pad) * esz +
                      64 * (64 + pad) * esz + 1024 + 64;
  if (lds > 160 * 1024)
    return fail(TOPS_GLA_EUNSUPPORTED,
                "K=%lld with chunk_size %d needs %lld B of LDS (> 160 KiB); use a smaller "
                "chunk_size or bf16",
                (long long)K, chunk, (long long)lds);
  return TOPS_GLA_OK;
}

// The full-head kernels: bf16, chunk 64, K and V <= 128 (multiples of 8), raw gates, every
// pointer 16-byte aligned (NULL counts as aligned).
bool use_head(int dtype, int chunk, int64_t K, int64_t V, bool g_is_cumsum,
              std::initializer_list<const void*> ptrs) {
  if (!tops::head_supported(dtype, chunk, (int)K, (int)V, g_is_cumsum)) return false;
  for (const void* p : ptrs)
    if (!aligned16(p)) return false;
  return true;
}

// Workspace of tops_gla_chunk_fwd / _bwd, each part 256-byte aligned:
//   [segment states, decays (full-head, NS > 1)] [gate-range flags, int32]
//   [wide heads' per-chunk gating (full-head, fixed length)]
//   [backward only: fallback final states f32 [N, H, K, V]]
// The flags part holds the full-head kernels' per-block flags or the per-chunk flags [NC, H]
// of the other paths (its size is the larger of the two, NC bounded by N ceil(T / C), or
// ceil(T / C) + N for varlen). Flags exist when the recurrent fallback runs the shape (K <=
// 512; the backward's also V <= 512). A workspace that ends early leaves the later parts
// out: no flags (no gate-range fallback), no gating workspace (every V tile's block gates its
// chunks), no backward fallback when dht is given.
long align256(long x) { return (x + 255) / 256 * 256; }

struct WsLayout {
  int NS = 1, SL = 0, VT = 1;
  long seg = 0, flags = 0, gate = 0, ht = 0;   // bytes of each part
  long off_flags = 0, off_gate = 0, off_ht = 0, total = 0;
};

WsLayout ws_layout(int N, int T, int H, int K, int V, int C, bool varlen, bool head,
                   bool backward) {
  WsLayout w;
  long nflag = (varlen ? (long)(T + C - 1) / C + N : (long)N * ((T + C - 1) / C)) * H;
  if (head) {
    w.VT = tops::head_vtiles(K, V);
    tops::head_seg_plan(N, H, T, C, varlen, w.NS, w.SL, w.VT);
    w.seg = align256(tops::head_seg_ws_bytes(N, w.NS, H, K, V));
    w.gate = varlen ? 0 : align256(tops::head_gate_ws_bytes(N, T, H, K, V));
    const long nblk = (long)N * w.NS * H * w.VT;
    if (nblk > nflag) nflag = nblk;
  }
  w.flags = K <= 512 ? align256(nflag * 4) : 0;
  w.ht = backward && tops::recurrent_supported(K, V) ? align256((long)N * H * K * V * 4) : 0;
  w.off_flags = w.seg;
  w.off_gate = w.off_flags + w.flags;
  w.off_ht = w.off_gate + w.gate;
  w.total = w.off_ht + w.ht;
  return w;
}

// The workspace pointers of one call from the caller's workspace (NULL parts are absent; NS
// = 1 without the segment part). `head`: the full-head kernels run the call.
struct WsParts {
  int NS = 1, SL = 0, VT = 1;
  float *st = nullptr, *gm = nullptr;
  void* gate = nullptr;
  int* flags = nullptr;
  float* ht = nullptr;
};

WsParts ws_parts(const tops::SeqInfo& si, int64_t H, int64_t K, int64_t V, void* ws,
                 int64_t ws_bytes, bool head, bool backward) {
  const WsLayout w = ws_layout(si.N, si.T, (int)H, (int)K, (int)V, si.C, si.cu != nullptr,
                               head, backward);
  WsParts p;
  p.VT = w.VT;
  const bool usable = ws != nullptr && ((uintptr_t)ws & 255u) == 0;
  if (!usable) return p;
  char* b = (char*)ws;
  if (w.NS > 1 && ws_bytes >= w.seg) {
    p.NS = w.NS;
    p.SL = w.SL;
    p.st = (float*)b;
    p.gm = (float*)(b + (long)si.N * w.NS * H * K * V * 4);
  }
  if (w.flags > 0 && ws_bytes >= w.off_gate) p.flags = (int*)(b + w.off_flags);
  if (w.gate > 0 && ws_bytes >= w.off_ht) p.gate = b + w.off_gate;
  if (w.ht > 0 && ws_bytes >= w.total) p.ht = (float*)(b + w.off_ht);
  return p;
}

// Per-chunk flags [NC, H] in the recurrent fallback's layout.
tops::GateFlags chunk_flags(int* f, const tops::SeqInfo& si) {
  tops::GateFlags g = {};
  g.p = f;
  g.vt = 1;
  if (si.cu) {
    g.ns = 0;
    g.co = si.chunk_cu;
  } else {
    g.ns = (si.T + si.C - 1) / si.C;
  }
  return g;
}

}  // namespace

namespace tops {

// Measurement hook state (process-wide, a profiling aid): a ring of KT_RING event pairs per
// kernel, one pair per launch while timing is on. The flag is read without the lock (off: the
// launch paths do nothing more); while it is on, marks, enabling and reading are serialized.
constexpr int KT_RING = 256;
static std::atomic<bool> g_kt_on{false};
static std::mutex g_kt_mu;
static bool g_kt_made = false;
static long g_kt_n[KT_COUNT] = {};            // launches recorded since timing was enabled
static hipEvent_t g_kt_ev[KT_COUNT][KT_RING][2];

void ktimer_mark(int which, bool stop, hipStream_t st) {
  if (!g_kt_on.load(std::memory_order_relaxed)) return;
  std::lock_guard<std::mutex> lk(g_kt_mu);
  if (!g_kt_on.load(std::memory_order_relaxed)) return;
  const long n = g_kt_n[which];
  if (hipEventRecord(g_kt_ev[which][n % KT_RING][stop ? 1 : 0], st) == hipSuccess && stop)
    g_kt_n[which] = n + 1;
}

}  // namespace tops

extern "C" {

int tops_gla_kernel_timing(int enable) {
  std::lock_guard<std::mutex> lk(tops::g_kt_mu);
  if (enable && !tops::g_kt_made) {   // host-side event objects, created once
    for (int i = 0; i < tops::KT_COUNT; ++i)
      for (int r = 0; r < tops::KT_RING; ++r)
        for (int j = 0; j < 2; ++j)
          if (hipEventCreate(&tops::g_kt_ev[i][r][j]) != hipSuccess)
            return fail(TOPS_GLA_EHIP, "hipEventCreate failed");
    tops::g_kt_made = true;
  }
  if (enable)
    for (int i = 0; i < tops::KT_COUNT; ++i) tops::g_kt_n[i] = 0;
  tops::g_kt_on.store(enable != 0);
  return ok();
}

float tops_gla_kernel_ms(int which) {
  std::lock_guard<std::mutex> lk(tops::g_kt_mu);
  if (which < 0 || which >= tops::KT_COUNT || tops::g_kt_n[which] == 0) return -1.f;
  const long n = tops::g_kt_n[which];
  const long m = n < tops::KT_RING ? n : tops::KT_RING;
  if (hipEventSynchronize(tops::g_kt_ev[which][(n - 1) % tops::KT_RING][1]) != hipSuccess)
    return -1.f;
  double sum = 0.0;
  for (long i = n - m; i < n; ++i) {
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, tops::g_kt_ev[which][i % tops::KT_RING][0],
                            tops::g_kt_ev[which][i % tops::KT_RING][1]) != hipSuccess)
      return -1.f;
    sum += ms;
  }
  return (float)(sum / m);
}


const char* tops_gla_last_error(void) { return g_err; }

const char* tops_gla_version(void) { return "tops-gla-mi355x 0.1.0 (gfx950)"; }

int tops_gla_full_head(int64_t K, int64_t V, int chunk_size, int dtype, int backward) {
  if (K <= 0 || V <= 0 || K > 4096 || V > (1 << 20)) return 0;
  if (!tops::head_supported(dtype, chunk_size, (int)K, (int)V, false)) return 0;
  return backward ? (int)tops::head_bwd_supported((int)K, (int)V) : 1;
}

int64_t tops_gla_chunk_ws_bytes(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V,
                                int chunk_size, int64_t N, int varlen, int dtype,
                                int backward) {
  if (B <= 0 || T <= 0 || H <= 0 || K <= 0 || V <= 0 || K > 512 || V > (1 << 20)) return 0;
  if (N <= 0 || N > kMaxInt || (!varlen && N != B) || B * T > kMaxInt) return 0;
  if (!dtype_ok(dtype) || chunk_size <= 0 || chunk_size > 64) return 0;
  const bool head = tops::head_supported(dtype, chunk_size, (int)K, (int)V, false);
  return ws_layout((int)N, (int)T, (int)H, (int)K, (int)V, chunk_size, varlen != 0, head,
                   backward != 0).total;
}

int tops_gla_chunk_local_cumsum(const void* g, void* out, int64_t B, int64_t T, int64_t H,
                                int64_t S, int chunk_size, int reverse, int has_scale,
                                float scale, int head_first, const int32_t* cu_seqlens,
                                const int32_t* chunk_offsets, int64_t N, int64_t NC,
                                int in_dtype, int out_dtype, void* stream) {
  if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) return fail(TOPS_GLA_EINVAL, "bad dtype");
  if (chunk_size <= 0 || (chunk_size & (chunk_size - 1)) != 0)
    return fail(TOPS_GLA_EINVAL, "chunk_size must be a power of 2 (got %d)", chunk_size);
  if (S < 0) return fail(TOPS_GLA_EINVAL, "bad S");
  if ((g == nullptr || out == nullptr) && B * T * H * S > 0)
    return fail(TOPS_GLA_EINVAL, "g and out must not be NULL");
  tops::SeqInfo si;
  int rc = make_seq(B, T, H, chunk_size, cu_seqlens, chunk_offsets, N, NC, true, &si);
  if (rc) return rc;
  if (NC * H > 2147483647LL || (S + 255) / 256 > 65535)
    return fail(TOPS_GLA_EUNSUPPORTED, "grid too large");
  tops::CumsumArgs p = {};
  p.g = g;
  p.out = out;
  p.H = (int)H;
  p.S = (int)S;
  p.reverse = reverse != 0;
  p.has_scale = has_scale != 0;
  p.head_first = head_first != 0;
  p.scale = scale;
  p.T_total = T;
  p.si = si;
  return hip_status(tops::run_cumsum(p, in_dtype, out_dtype, (hipStream_t)stream),
                    "chunk_local_cumsum");
}

int tops_gla_chunk_fwd_h(const void* k, const void* v, const void* g, int g_is_cumsum,
                         const float* h0, void* h, float* ht, void* seg_ws,
                         int64_t seg_ws_bytes, int64_t B, int64_t T, int64_t H, int64_t K,
                         int64_t V, int chunk_size, const int32_t* cu_seqlens,
                         const int32_t* chunk_offsets, int64_t N, int64_t NC, int dtype,
                         void* stream) {
  const bool small = small_chunk(chunk_size);
  int rc = small ? check_small_common(K, V, dtype) : check_mfma_common(K, V, chunk_size, dtype);
  if (rc) return rc;
  tops::SeqInfo si;
  rc = make_seq(B, T, H, chunk_size, cu_seqlens, chunk_offsets, N, NC, true, &si);
  if (rc) return rc;
  if ((k == nullptr || v == nullptr || g == nullptr) && B * T > 0)
    return fail(TOPS_GLA_EINVAL, "k, v and g must not be NULL");
  if (small) {
    tops::ScanArgs p = {};
    p.a = k;
    p.b = v;
    p.g = g;
    p.g_is_cumsum = g_is_cumsum != 0;
    p.s_init = h0;
    p.s_all = h;
    p.s_final = ht;
    p.scale = 1.f;
    p.H = (int)H;
    p.K = (int)K;
    p.V = (int)V;
    p.si = si;
    return hip_status(tops::run_small_state_scan(p, false, dtype, (hipStream_t)stream),
                      "chunk_fwd_h");
  }
  if (use_head(dtype, chunk_size, K, V, g_is_cumsum != 0, {k, v, g, h0, h, ht})) {
    tops::HeadScanArgs s = {};
    s.a = k;
    s.b = v;
    s.g = g;
    s.s_init = h0;
    s.s_all = h;
    s.s_final = ht;
    {
      const WsParts w = ws_parts(si, H, K, V, seg_ws, seg_ws_bytes, true, false);
      s.NS = w.NS;
      s.SL = w.SL;
      s.seg_state = w.st;
      s.seg_gam = w.gm;
    }
    s.scale = 1.f;
    s.H = (int)H;
    s.K = (int)K;
    s.V = (int)V;
    s.si = si;
    return hip_status(tops::run_head_scan(s, false, (hipStream_t)stream), "chunk_fwd_h");
  }
  tops::ScanArgs p = {};
  p.a = k;
  p.b = v;
  p.g = g;
  p.g_is_cumsum = g_is_cumsum != 0;
  p.s_init = h0;
  p.s_all = h;
  p.s_final = ht;
  p.scale = 1.f;
  p.H = (int)H;
  p.K = (int)K;
  p.V = (int)V;
  p.vec = vec_ok(dtype, K, V, {k, v, g, h});
  p.si = si;
  return hip_status(tops::run_state_scan(p, false, dtype, (hipStream_t)stream), "chunk_fwd_h");
}

int tops_gla_chunk_bwd_dh(const void* q, const void* g, int g_is_cumsum, const void* dout,
                          const float* dht, void* dh, float* dh0, void* seg_ws,
                          int64_t seg_ws_bytes, float scale, int64_t B, int64_t T, int64_t H,
                          int64_t K, int64_t V, int chunk_size, const int32_t* cu_seqlens,
                          const int32_t* chunk_offsets, int64_t N, int64_t NC, int dtype,
                          void* stream) {
  const bool small = small_chunk(chunk_size);
  int rc = small ? check_small_common(K, V, dtype) : check_mfma_common(K, V, chunk_size, dtype);
  if (rc) return rc;
  tops::SeqInfo si;
  rc = make_seq(B, T, H, chunk_size, cu_seqlens, chunk_offsets, N, NC, true, &si);
  if (rc) return rc;
  if ((q == nullptr || dout == nullptr || g == nullptr) && B * T > 0)
    return fail(TOPS_GLA_EINVAL, "q, g and do must not be NULL");
  if (small) {
    tops::ScanArgs p = {};
    p.a = q;
    p.b = dout;
    p.g = g;
    p.g_is_cumsum = g_is_cumsum != 0;
    p.s_init = dht;
    p.s_all = dh;
    p.s_final = dh0;
    p.scale = scale;
    p.H = (int)H;
    p.K = (int)K;
    p.V = (int)V;
    p.si = si;
    return hip_status(tops::run_small_state_scan(p, true, dtype, (hipStream_t)stream),
                      "chunk_bwd_dh");
  }
  if (use_head(dtype, chunk_size, K, V, g_is_cumsum != 0, {q, dout, g, dht, dh, dh0})) {
    tops::HeadScanArgs s = {};
    s.a = q;
    s.b = dout;
    s.g = g;
    s.s_init = dht;
    s.s_all = dh;
    s.s_final = dh0;
    {
      const WsParts w = ws_parts(si, H, K, V, seg_ws, seg_ws_bytes, true, false);
      s.NS = w.NS;
      s.SL = w.SL;
      s.seg_state = w.st;
      s.seg_gam = w.gm;
    }
    s.scale = scale;
    s.H = (int)H;
    s.K = (int)K;
    s.V = (int)V;
    s.si = si;
    return hip_status(tops::run_head_scan(s, true, (hipStream_t)stream), "chunk_bwd_dh");
  }
  tops::ScanArgs p = {};
  p.a = q;
  p.b = dout;
  p.g = g;
  p.g_is_cumsum = g_is_cumsum != 0;
  p.s_init = dht;
  p.s_all = dh;
  p.s_final = dh0;
  p.scale = scale;
  p.H = (int)H;
  p.K = (int)K;
  p.V = (int)V;
  p.vec = vec_ok(dtype, K, V, {q, dout, g, dh});
  p.si = si;
  return hip_status(tops::run_state_scan(p, true, dtype, (hipStream_t)stream), "chunk_bwd_dh");
}

int tops_gla_chunk_fwd_o(const void* q, const void* k, const void* v, const void* g,
                         int g_is_cumsum, const void* h, const float* A_in, float* A_out,
                         void* o, float scale, int64_t B, int64_t T, int64_t H, int64_t K,
                         int64_t V, int chunk_size, const int32_t* cu_seqlens,
                         const int32_t* chunk_offsets, int64_t N, int64_t NC, int dtype,
                         void* stream) {
  const bool small = small_chunk(chunk_size);
  int rc = small ? check_small_common(K, V, dtype) : check_mfma_common(K, V, chunk_size, dtype);
  if (rc) return rc;
  tops::SeqInfo si;
  rc = make_seq(B, T, H, chunk_size, cu_seqlens, chunk_offsets, N, NC, true, &si);
  if (rc) return rc;
  if (B * T > 0 && (q == nullptr || g == nullptr))
    return fail(TOPS_GLA_EINVAL, "q and g must not be NULL");
  if (B * T > 0 && A_in == nullptr && k == nullptr)
    return fail(TOPS_GLA_EINVAL, "k is required unless A_in is given");
  if (B * T > 0 && o != nullptr && v == nullptr)
    return fail(TOPS_GLA_EINVAL, "v is required for o");
  if (o == nullptr && A_out == nullptr) return ok();
  tops::FwdOArgs p = {};
  p.q = q;
  p.k = k;
  p.v = v;
  p.g = g;
  p.g_is_cumsum = g_is_cumsum != 0;
  p.h = h;
  p.A_in = A_in;
  p.A_out = A_in ? nullptr : A_out;
  p.o = o;
  p.scale = scale;
  p.H = (int)H;
  p.K = (int)K;
  p.V = (int)V;
  p.si = si;
  if (small)
    return hip_status(tops::run_small_chunk_fwd_o(p, dtype, (hipStream_t)stream), "chunk_fwd_o");
  return hip_status(tops::run_chunk_fwd_o(p, dtype, (hipStream_t)stream), "chunk_fwd_o");
}

namespace {

// tops_gla_chunk_fwd off the full-head path: the fused float32 forward, or the state scan
// and the per-chunk output kernel.
int chunk_fwd_other(const void* q, const void* k, const void* v, const void* g, const float* h0,
                    void* o, float* ht, void* h_ws, float scale, int64_t H, int64_t K,
                    int64_t V, int chunk_size, const tops::SeqInfo& si, int dtype,
                    hipStream_t st) {
  int rc;
  if (tops::fused_fwd_supported(dtype, chunk_size, (int)K)) {
    tops::FusedFwdArgs f = {};
    f.q = q;
    f.k = k;
    f.v = v;
    f.g = g;
    f.h0 = h0;
    f.o = o;
    f.h_out = h_ws;
    f.ht = ht;
    f.scale = scale;
    f.H = (int)H;
    f.K = (int)K;
    f.V = (int)V;
    const int epp = dtype == TOPS_GLA_BF16 ? 8 : 4;
    f.vec_k = (K % epp == 0) && aligned16(q) && aligned16(k) && aligned16(g);
    f.vec_v = (V % epp == 0) && aligned16(v) && aligned16(o) && aligned16(h_ws);
    f.si = si;
    return hip_status(tops::run_chunk_fwd_fused(f, dtype, st), "chunk_fwd (fused)");
  }
  tops::ScanArgs s = {};
  s.a = k;
  s.b = v;
  s.g = g;
  s.g_is_cumsum = 0;
  s.s_init = h0;
  s.s_all = h_ws;
  s.s_final = ht;
  s.scale = 1.f;
  s.H = (int)H;
  s.K = (int)K;
  s.V = (int)V;
  s.vec = vec_ok(dtype, K, V, {k, v, g, h_ws});
  s.si = si;
  rc = hip_status(tops::run_state_scan(s, false, dtype, st), "chunk_fwd (state scan)");
  if (rc) return rc;
  tops::FwdOArgs p = {};
  p.q = q;
  p.k = k;
  p.v = v;
  p.g = g;
  p.g_is_cumsum = 0;
  p.h = h_ws;
  p.A_in = nullptr;
  p.A_out = nullptr;
  p.o = o;
  p.scale = scale;
  p.H = (int)H;
  p.K = (int)K;
  p.V = (int)V;
  p.si = si;
  return hip_status(tops::run_chunk_fwd_o(p, dtype, st), "chunk_fwd (output)");
}

// Per-chunk gate-range flags [NC, H] of the raw gates g (into `flags`).
int gate_check(const void* g, int* flags, int64_t H, int64_t K, const tops::SeqInfo& si,
               int dtype, hipStream_t st) {
  tops::GateCheckArgs c = {};
  c.g = g;
  c.flags = flags;
  c.H = (int)H;
  c.K = (int)K;
  c.si = si;
  return hip_status(tops::run_gate_range(c, dtype, st), "gate-range check");
}

// The forward's fallback off the full-head path: check every chunk, then the recurrent
// forward over the flagged pairs.
int gate_fallback_fwd(const void* q, const void* k, const void* v, const void* g,
                      const float* h0, void* o, float* ht, float scale, int64_t H, int64_t K,
                      int64_t V, const tops::SeqInfo& si, int* flags, int dtype,
                      hipStream_t st) {
  int rc = gate_check(g, flags, H, K, si, dtype, st);
  if (rc) return rc;
  tops::RecArgs r = {};
  r.q = q;
  r.k = k;
  r.v = v;
  r.gk = g;
  r.h0 = h0;
  r.o = o;
  r.ht = ht;
  r.scale = scale;
  r.H = (int)H;
  r.K = (int)K;
  r.V = (int)V;
  r.si = si;
  r.flags = chunk_flags(flags, si);
  return hip_status(tops::run_recurrent_fwd(r, dtype, dtype, st),
                    "chunk_fwd (gate-range fallback)");
}

}  // namespace

int tops_gla_chunk_fwd(const void* q, const void* k, const void* v, const void* g,
                       const float* h0, void* o, float* ht, void* h_ws, void* seg_ws,
                       int64_t seg_ws_bytes, float scale, int64_t B, int64_t T, int64_t H,
                       int64_t K, int64_t V, int chunk_size, const int32_t* cu_seqlens,
                       const int32_t* chunk_offsets, int64_t N, int64_t NC, int dtype,
                       void* stream) {
  int rc = check_mfma_common(K, V, chunk_size, dtype);
  if (rc) return rc;
  tops::SeqInfo si;
  rc = make_seq(B, T, H, chunk_size, cu_seqlens, chunk_offsets, N, NC, true, &si);
  if (rc) return rc;
  if (B * T > 0 && (q == nullptr || k == nullptr || v == nullptr || g == nullptr ||
                    o == nullptr))
    return fail(TOPS_GLA_EINVAL, "q, k, v, g and o must not be NULL");
  hipStream_t st = (hipStream_t)stream;
  const bool head = use_head(dtype, chunk_size, K, V, false, {q, k, v, g, h0, o, ht, h_ws});
  if (!head && h_ws == nullptr && B * T > 0)
    return fail(TOPS_GLA_EINVAL, "h_ws must not be NULL off the full-head path");
  if (head) {
    tops::HeadFwdArgs f = {};
    f.q = q;
    f.k = k;
    f.v = v;
    f.g = g;
    f.h0 = h0;
    f.o = o;
    f.h_out = h_ws;
    f.ht = ht;
    const WsParts w = ws_parts(si, H, K, V, seg_ws, seg_ws_bytes, true, false);
    f.NS = w.NS;
    f.SL = w.SL;
    f.seg_state = w.st;
    f.seg_gam = w.gm;
    f.gate_ws = w.gate;
    // gate-range flags: per block where the forward gates its own chunks, per chunk from the
    // gating kernel where wide heads stream the gating workspace
    f.flags = w.flags;
    f.scale = scale;
    f.H = (int)H;
    f.K = (int)K;
    f.V = (int)V;
    f.si = si;
    rc = hip_status(tops::run_head_fwd(f, st), "chunk_fwd (full-head)");
    if (rc || f.flags == nullptr) return rc;
    const bool per_chunk = K > 128 && w.gate != nullptr;
    // sequences and heads with a chunk beyond the factoring's range: the recurrent forward
    // (exact for any decay) rewrites their o and final state; the other blocks return at once
    tops::RecArgs r = {};
    r.q = q;
    r.k = k;
    r.v = v;
    r.gk = g;
    r.h0 = h0;
    r.o = o;
    r.ht = ht;
    r.scale = scale;
    r.H = (int)H;
    r.K = (int)K;
    r.V = (int)V;
    r.si = si;
    r.flags = per_chunk ? chunk_flags(f.flags, si) : tops::GateFlags{f.flags, w.NS, w.VT};
    return hip_status(tops::run_recurrent_fwd(r, dtype, dtype, st),
                      "chunk_fwd (gate-range fallback)");
  }
  rc = chunk_fwd_other(q, k, v, g, h0, o, ht, h_ws, scale, H, K, V, chunk_size, si, dtype, st);
  if (rc) return rc;
  // the gate-range check of the per-chunk kernels, and the recurrent forward for the flagged
  // (sequence, head) pairs (o and the final state rewritten)
  const WsParts w = ws_parts(si, H, K, V, seg_ws, seg_ws_bytes, false, false);
  if (w.flags == nullptr || B * T == 0) return rc;
  return gate_fallback_fwd(q, k, v, g, h0, o, ht, scale, H, K, V, si, w.flags, dtype, st);
}


// ---------------------------------------------------------------------------
// tops_gla_chunk_fwd without a caller workspace: the segment workspace lives in one
// file-scope device array per GPU (`scratch`), shared by every call on that GPU.
// ---------------------------------------------------------------------------
namespace {

// The full-head segment plan keeps sequences x heads x V tiles x segments <= 256, so the
// segment part of the workspace is at most 256 x 128 x 128 x 4 B of states plus 256 x 256 x
// 4 B of decays (17.04 MB); 24 MiB holds it with room to spare.
constexpr long kScratchBytes = 24l << 20;
__device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current GPU's copy of `scratch`: hipGetSymbolAddress once per
// device, with that device current (the array's host-side name is not a device address).
int scratch_on(hipStream_t st, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e, "hipGetDevice");
  if (st != nullptr) {
    hipDevice_t sd = -1;
    e = hipStreamGetDevice(st, &sd);
    if (e != hipSuccess) return hip_status(e, "hipStreamGetDevice");
    if (sd != dev)
      return fail(TOPS_GLA_EINVAL, "the stream belongs to device %d, the current device is %d",
                  (int)sd, dev);
  }
  if (dev < 0 || dev >= kMaxDevices)
    return fail(TOPS_GLA_EUNSUPPORTED, "device %d: at most %d devices", dev, kMaxDevices);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_status(e, "hipGetSymbolAddress(scratch)");
    if (p == nullptr) return fail(TOPS_GLA_EHIP, "hipGetSymbolAddress(scratch) gave NULL");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return TOPS_GLA_OK;
}

}  // namespace

int tops_gla_chunk_fwd_noalloc(const void* q, const void* k, const void* v, const void* g,
                               const float* h0, void* o, float* ht, void* h_ws, float scale,
                               int64_t B, int64_t T, int64_t H, int64_t K, int64_t V,
                               int chunk_size, const int32_t* cu_seqlens,
                               const int32_t* chunk_offsets, int64_t N, int64_t NC, int dtype,
                               void* stream) {
  int rc = check_mfma_common(K, V, chunk_size, dtype);
  if (rc) return rc;
  // the arguments are checked before the scratch's address is taken
  tops::SeqInfo si;
  rc = make_seq(B, T, H, chunk_size, cu_seqlens, chunk_offsets, N, NC, true, &si);
  if (rc) return rc;
  if (B * T > 0 && (q == nullptr || k == nullptr || v == nullptr || g == nullptr ||
                    o == nullptr))
    return fail(TOPS_GLA_EINVAL, "q, k, v, g and o must not be NULL");
  if (B <= 0 || T <= 0 || H <= 0)   // nothing to segment: no scratch needed
    return tops_gla_chunk_fwd(q, k, v, g, h0, o, ht, h_ws, nullptr, 0, scale, B, T, H, K, V,
                              chunk_size, cu_seqlens, chunk_offsets, N, NC, dtype, stream);
  // the segment part (full-head shapes) and the gate-range flags
  const bool head = tops::head_supported(dtype, chunk_size, (int)K, (int)V, false);
  const long need = K <= 512 ? ws_layout(si.N, si.T, (int)H, (int)K, (int)V, chunk_size,
                                         si.cu != nullptr, head, false).off_gate
                             : 0;
  if (need > kScratchBytes)
    return fail(TOPS_GLA_EINVAL,
                "the workspace (segment part, gate-range flags) needs %ld bytes, the static "
                "scratch holds %ld; call "
                "tops_gla_chunk_fwd with a workspace",
                need, kScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    rc = scratch_on((hipStream_t)stream, &ws);
    if (rc) return rc;
  }
  // exactly the segment part: the wide heads' per-chunk gating workspace is not used (every
  // V tile then gates its chunk itself)
  return tops_gla_chunk_fwd(q, k, v, g, h0, o, ht, h_ws, ws, need, scale, B, T, H, K, V,
                            chunk_size, cu_seqlens, chunk_offsets, N, NC, dtype, stream);
}

int tops_gla_chunk_bwd(const void* q, const void* k, const void* v, const void* g,
                       const float* h0, const void* h, const void* dout, const float* dht,
                       void* dq, void* dk, void* dv, void* dg, float* dh0, void* h_ws,
                       void* dh_ws, void* seg_ws, int64_t seg_ws_bytes, float scale,
                       int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int chunk_size,
                       const int32_t* cu_seqlens, const int32_t* chunk_offsets, int64_t N,
                       int64_t NC, int dtype, void* stream) {
  int rc = check_mfma_common(K, V, chunk_size, dtype);
  if (rc) return rc;
  tops::SeqInfo si;
  rc = make_seq(B, T, H, chunk_size, cu_seqlens, chunk_offsets, N, NC, true, &si);
  if (rc) return rc;
  if (B * T > 0 && (q == nullptr || k == nullptr || v == nullptr || g == nullptr ||
                    dout == nullptr || dq == nullptr || dk == nullptr || dv == nullptr ||
                    dg == nullptr))
    return fail(TOPS_GLA_EINVAL, "q, k, v, g, do, dq, dk, dv and dg must not be NULL");
  if (h == nullptr && h_ws == nullptr && B * T > 0)
    return fail(TOPS_GLA_EINVAL, "h_ws is required when h is NULL");
  hipStream_t st = (hipStream_t)stream;
  // full-head scans for the state recompute; the fused backward for K, V <= 128
  // the fused backward writes dq, dk, dv and dg with 16- and 8-byte vector stores
  const bool head = use_head(dtype, chunk_size, K, V, false, {q, k, v, g, h0, h, dout, dht,
                                                              dq, dk, dv, dg, dh0, h_ws, dh_ws});
  const bool head_bwd = head && tops::head_bwd_supported((int)K, (int)V);
  if (!head_bwd && dh_ws == nullptr && B * T > 0)
    return fail(TOPS_GLA_EINVAL, "dh_ws must not be NULL off the fused full-head backward");
  int NS = 1, SL = 0;
  float *seg_st = nullptr, *seg_gm = nullptr;
  void* gate = nullptr;   // per-chunk gating of wide heads (when the workspace holds it)
  const WsParts wp = ws_parts(si, H, K, V, seg_ws, seg_ws_bytes, head, true);
  if (head) {
    NS = wp.NS;
    SL = wp.SL;
    seg_st = wp.st;
    seg_gm = wp.gm;
    gate = wp.gate;
  }
  if (head_bwd) gate = nullptr;
  // the recurrent fallback's needs: K, V <= 512 and, with dht, its final-state part
  const bool rec_ok = tops::recurrent_supported((int)K, (int)V) && B * T > 0 &&
                      (dht == nullptr || wp.ht != nullptr);
  // per-chunk gate-range flags of the paths below the fused backward: from the gating
  // kernel (wide heads with the gating workspace) or the check kernel
  int* cflags = (!head_bwd && rec_ok) ? wp.flags : nullptr;
  if (gate) {   // gated q, k, A and the column factors once per (chunk, head): the scans and
                // the dv kernel stream them
    tops::HeadFwdArgs a = {};
    a.q = q;
    a.k = k;
    a.g = g;
    a.gate_ws = gate;
    a.flags = cflags;
    a.scale = scale;
    a.H = (int)H;
    a.K = (int)K;
    a.V = (int)V;
    a.si = si;
    rc = hip_status(tops::run_head_gate(a, st), "chunk_bwd (gating)");
    if (rc) return rc;
  } else if (cflags) {
    rc = gate_check(g, cflags, H, K, si, dtype, st);
    if (rc) return rc;
  }
  auto head_scan = [&](bool rev, const void* a, const void* b, const float* s_init, void* s_all,
                       float* s_final, float sc) {
    tops::HeadScanArgs s = {};
    s.a = a;
    s.b = b;
    s.g = g;
    s.s_init = s_init;
    s.s_all = s_all;
    s.s_final = s_final;
    s.seg_state = seg_st;
    s.seg_gam = seg_gm;
    s.gate_ws = gate;
    s.NS = NS;
    s.SL = SL;
    s.scale = sc;
    s.H = (int)H;
    s.K = (int)K;
    s.V = (int)V;
    s.si = si;
    return tops::run_head_scan(s, rev, st);
  };
  if (h == nullptr && head) {
    rc = hip_status(head_scan(false, k, v, h0, h_ws, nullptr, 1.f),
                    "chunk_bwd (state recompute)");
    if (rc) return rc;
    h = h_ws;
  }
  if (h == nullptr) {
    tops::ScanArgs s = {};
    s.a = k;
    s.b = v;
    s.g = g;
    s.g_is_cumsum = 0;
    s.s_init = h0;
    s.s_all = h_ws;
    s.s_final = nullptr;
    s.scale = 1.f;
    s.H = (int)H;
    s.K = (int)K;
    s.V = (int)V;
    s.vec = vec_ok(dtype, K, V, {k, v, g, h_ws});
    s.si = si;
    rc = hip_status(tops::run_state_scan(s, false, dtype, st), "chunk_bwd (state recompute)");
    if (rc) return rc;
    h = h_ws;
  }
  if (head_bwd) {
    // fused: reverse dh scan and per-chunk gradients in one pass (dh_ws is not needed)
    tops::HeadBwdArgs b = {};
    b.q = q;
    b.k = k;
    b.v = v;
    b.g = g;
    b.dout = dout;
    b.h = h;
    b.dht = dht;
    b.dq = dq;
    b.dk = dk;
    b.dv = dv;
    b.dg = dg;
    b.dh0 = dh0;
    b.seg_state = seg_st;
    b.seg_gam = seg_gm;
    b.NS = NS;
    b.SL = SL;
    b.scale = scale;
    b.H = (int)H;
    b.K = (int)K;
    b.V = (int)V;
    b.si = si;
    // gate-range check (and fallback) when the workspace holds the flags and, with dht, the
    // fallback's final-state part
    b.flags = (dht == nullptr || wp.ht != nullptr) ? wp.flags : nullptr;
    rc = hip_status(tops::run_head_bwd(b, st), "chunk_bwd (full-head)");
    if (rc || b.flags == nullptr) return rc;
    // sequences and heads with a chunk beyond the factoring's range: the recurrent backward
    // (exact for any decay) rewrites their dq, dk, dv, dg and dh0
    tops::RecBwdArgs r = {};
    r.q = q;
    r.k = k;
    r.v = v;
    r.gk = g;
    r.dout = dout;
    r.h0 = h0;
    r.dht = dht;
    r.dq = dq;
    r.dk = dk;
    r.dv = dv;
    r.dgk = dg;
    r.dh0 = dh0;
    r.ht_ws = wp.ht;
    r.scale = scale;
    r.H = (int)H;
    r.K = (int)K;
    r.V = (int)V;
    r.si = si;
    r.flags = {b.flags, NS, 1};
    return hip_status(tops::run_recurrent_bwd(r, dtype, dtype, st),
                      "chunk_bwd (gate-range fallback)");
  } else if (head) {
    // wide heads: the full-head reverse scan stores dh for the per-chunk gradient kernels
    rc = hip_status(head_scan(true, q, dout, dht, dh_ws, dh0, scale), "chunk_bwd (dh scan)");
    if (rc) return rc;
  } else {
    tops::ScanArgs d = {};
    d.a = q;
    d.b = dout;
    d.g = g;
    d.g_is_cumsum = 0;
    d.s_init = dht;
    d.s_all = dh_ws;
    d.s_final = dh0;
    d.scale = scale;
    d.H = (int)H;
    d.K = (int)K;
    d.V = (int)V;
    d.vec = vec_ok(dtype, K, V, {q, dout, g, dh_ws});
    d.si = si;
    rc = hip_status(tops::run_state_scan(d, true, dtype, st), "chunk_bwd (dh scan)");
    if (rc) return rc;
  }
  tops::BwdArgs p = {};
  p.q = q;
  p.k = k;
  p.v = v;
  p.g = g;
  p.dout = dout;
  p.h = h;
  p.dh = dh_ws;
  p.dq = dq;
  p.dk = dk;
  p.dv = dv;
  p.dg = dg;
  p.gate_ws = gate;
  p.scale = scale;
  p.H = (int)H;
  p.K = (int)K;
  p.V = (int)V;
  p.vec = vec_ok(dtype, K, V, {q, k, v, g, dout, h, dh_ws, dq, dk, dv, dg});
  p.si = si;
  if (head && tops::head_dqkg_supported((int)K, (int)V)) {
    // dq, dk, dg one block per (chunk, head) over every V tile; dv by the per-chunk kernel
    rc = hip_status(tops::run_head_dqkg(p, st), "chunk_bwd (dq, dk, dg)");
    if (!rc) rc = hip_status(tops::run_chunk_bwd(p, dtype, st, 2), "chunk_bwd (dv)");
  } else {
    rc = hip_status(tops::run_chunk_bwd(p, dtype, st), "chunk_bwd (gradients)");
  }
  if (rc || cflags == nullptr) return rc;
  // sequences and heads with a chunk beyond the factoring's range: the recurrent backward
  // (exact for any decay) rewrites their dq, dk, dv, dg and dh0
  tops::RecBwdArgs r = {};
  r.q = q;
  r.k = k;
  r.v = v;
  r.gk = g;
  r.dout = dout;
  r.h0 = h0;
  r.dht = dht;
  r.dq = dq;
  r.dk = dk;
  r.dv = dv;
  r.dgk = dg;
  r.dh0 = dh0;
  r.ht_ws = wp.ht;
  r.scale = scale;
  r.H = (int)H;
  r.K = (int)K;
  r.V = (int)V;
  r.si = si;
  r.flags = chunk_flags(cflags, si);
  return hip_status(tops::run_recurrent_bwd(r, dtype, dtype, st),
                    "chunk_bwd (gate-range fallback)");
}

// ---------------------------------------------------------------------------
// Scalar gates (simple GLA): the full-head kernels with gate(t, h) = gs[t * gs_ts + h]
// ---------------------------------------------------------------------------
namespace {

int check_scalar_gate(const float* gs, int64_t gs_ts, int64_t H) {
  if (gs == nullptr) return fail(TOPS_GLA_EINVAL, "gs must not be NULL");
  if (gs_ts != 0 && gs_ts != H) return fail(TOPS_GLA_EINVAL, "gs_ts must be 0 or H");
  return 0;
}

}  // namespace

int tops_gla_simple_chunk_fwd(const void* q, const void* k, const void* v, const float* gs,
                              int64_t gs_ts, const float* h0, void* o, float* ht, void* h_ws,
                              void* seg_ws, int64_t seg_ws_bytes, float scale, int64_t B,
                              int64_t T, int64_t H, int64_t K, int64_t V, int chunk_size,
                              const int32_t* cu_seqlens, const int32_t* chunk_offsets, int64_t N,
                              int64_t NC, int dtype, void* stream) {
  int rc = check_mfma_common(K, V, chunk_size, dtype);
  if (rc) return rc;
  tops::SeqInfo si;
  rc = make_seq(B, T, H, chunk_size, cu_seqlens, chunk_offsets, N, NC, true, &si);
  if (rc) return rc;
  if (B * T == 0) return 0;
  if (q == nullptr || k == nullptr || v == nullptr || o == nullptr)
    return fail(TOPS_GLA_EINVAL, "q, k, v and o must not be NULL");
  if ((rc = check_scalar_gate(gs, gs_ts, H))) return rc;
  if (!use_head(dtype, chunk_size, K, V, false, {q, k, v, h0, o, ht, h_ws}))
    return fail(TOPS_GLA_EUNSUPPORTED,
                "scalar gates run on the full-head kernels (tops_gla_full_head(..., 0) == 1)");
  tops::HeadFwdArgs f = {};
  f.q = q;
  f.k = k;
  f.v = v;
  f.g = nullptr;
  f.gs = gs;
  f.gs_ts = (long)gs_ts;
  f.h0 = h0;
  f.o = o;
  f.h_out = h_ws;
  f.ht = ht;
  {
    const WsParts w = ws_parts(si, H, K, V, seg_ws, seg_ws_bytes, true, false);
    f.NS = w.NS;
    f.SL = w.SL;
    f.seg_state = w.st;
    f.seg_gam = w.gm;
  }
  f.scale = scale;
  f.H = (int)H;
  f.K = (int)K;
  f.V = (int)V;
  f.si = si;
  return hip_status(tops::run_head_fwd(f, (hipStream_t)stream), "simple_chunk_fwd");
}

int tops_gla_simple_chunk_bwd(const void* q, const void* k, const void* v, const float* gs,
                              int64_t gs_ts, const float* h0, const void* h, const void* dout,
                              const float* dht, void* dq, void* dk, void* dv, void* dg,
                              float* dh0, void* h_ws, void* seg_ws, int64_t seg_ws_bytes,
                              float scale, int64_t B, int64_t T, int64_t H, int64_t K, int64_t V,
                              int chunk_size, const int32_t* cu_seqlens,
                              const int32_t* chunk_offsets, int64_t N, int64_t NC, int dtype,
                              void* stream) {
  int rc = check_mfma_common(K, V, chunk_size, dtype);
  if (rc) return rc;
  tops::SeqInfo si;
  rc = make_seq(B, T, H, chunk_size, cu_seqlens, chunk_offsets, N, NC, true, &si);
  if (rc) return rc;
  if (B * T == 0) return 0;
  if (q == nullptr || k == nullptr || v == nullptr || dout == nullptr || dq == nullptr ||
      dk == nullptr || dv == nullptr)
    return fail(TOPS_GLA_EINVAL, "q, k, v, do, dq, dk and dv must not be NULL");
  if ((rc = check_scalar_gate(gs, gs_ts, H))) return rc;
  if (h == nullptr && h_ws == nullptr)
    return fail(TOPS_GLA_EINVAL, "h_ws is required when h is NULL");
  if (!use_head(dtype, chunk_size, K, V, false,
                {q, k, v, h0, h, dout, dht, dq, dk, dv, dg, dh0, h_ws}) ||
      !tops::head_bwd_supported((int)K, (int)V))
    return fail(TOPS_GLA_EUNSUPPORTED,
                "scalar gates run on the full-head kernels (tops_gla_full_head(..., 1) == 1)");
  hipStream_t st = (hipStream_t)stream;
  int NS = 1, SL = 0;
  float *seg_st = nullptr, *seg_gm = nullptr;
  {
    const WsParts w = ws_parts(si, H, K, V, seg_ws, seg_ws_bytes, true, false);
    NS = w.NS;
    SL = w.SL;
    seg_st = w.st;
    seg_gm = w.gm;
  }
  if (h == nullptr) {
    tops::HeadScanArgs s = {};
    s.a = k;
    s.b = v;
    s.g = nullptr;
    s.gs = gs;
    s.gs_ts = (long)gs_ts;
    s.s_init = h0;
    s.s_all = h_ws;
    s.seg_state = seg_st;
    s.seg_gam = seg_gm;
    s.NS = NS;
    s.SL = SL;
    s.scale = 1.f;
    s.H = (int)H;
    s.K = (int)K;
    s.V = (int)V;
    s.si = si;
    rc = hip_status(tops::run_head_scan(s, false, st), "simple_chunk_bwd (state recompute)");
    if (rc) return rc;
    h = h_ws;
  }
  tops::HeadBwdArgs b = {};
  b.q = q;
  b.k = k;
  b.v = v;
  b.g = nullptr;
  b.gs = gs;
  b.gs_ts = (long)gs_ts;
  b.dout = dout;
  b.h = h;
  b.dht = dht;
  b.dq = dq;
  b.dk = dk;
  b.dv = dv;
  b.dg = dg;
  b.dh0 = dh0;
  b.seg_state = seg_st;
  b.seg_gam = seg_gm;
  b.NS = NS;
  b.SL = SL;
  b.scale = scale;
  b.H = (int)H;
  b.K = (int)K;
  b.V = (int)V;
  b.si = si;
  return hip_status(tops::run_head_bwd(b, st), "simple_chunk_bwd");
}

int tops_gla_chunk_bwd_dqkg(const void* q, const void* k, const void* v, const void* g,
                            const void* h, const void* dout, const void* dh, void* dq, void* dk,
                            void* dg, float scale, int64_t B, int64_t T, int64_t H, int64_t K,
                            int64_t V, int chunk_size, const int32_t* cu_seqlens,
                            const int32_t* chunk_offsets, int64_t N, int64_t NC, int dtype,
                            void* stream) {
  int rc = check_mfma_common(K, V, chunk_size, dtype);
  if (rc) return rc;
  tops::SeqInfo si;
  rc = make_seq(B, T, H, chunk_size, cu_seqlens, chunk_offsets, N, NC, true, &si);
  if (rc) return rc;
  if (B * T > 0 && (q == nullptr || k == nullptr || v == nullptr || g == nullptr ||
                    h == nullptr || dout == nullptr || dh == nullptr || dq == nullptr ||
                    dk == nullptr || dg == nullptr))
    return fail(TOPS_GLA_EINVAL, "no argument of chunk_bwd_dqkg may be NULL");
  tops::BwdArgs p = {};
  p.q = q;
  p.k = k;
  p.v = v;
  p.g = g;
  p.dout = dout;
  p.h = h;
  p.dh = dh;
  p.dq = dq;
  p.dk = dk;
  p.dv = nullptr;
  p.dg = dg;
  p.scale = scale;
  p.H = (int)H;
  p.K = (int)K;
  p.V = (int)V;
  p.vec = vec_ok(dtype, K, V, {q, k, v, g, h, dout, dh, dq, dk, dg});
  p.si = si;
  return hip_status(tops::run_chunk_bwd(p, dtype, (hipStream_t)stream, 1), "chunk_bwd_dqkg");
}

int tops_gla_chunk_bwd_dv(const void* q, const void* k, const void* g, const void* dout,
                          const void* dh, void* dv, float scale, int64_t B, int64_t T,
                          int64_t H, int64_t K, int64_t V, int chunk_size,
                          const int32_t* cu_seqlens, const int32_t* chunk_offsets, int64_t N,
                          int64_t NC, int dtype, void* stream) {
  int rc = check_mfma_common(K, V, chunk_size, dtype);
  if (rc) return rc;
  tops::SeqInfo si;
  rc = make_seq(B, T, H, chunk_size, cu_seqlens, chunk_offsets, N, NC, true, &si);
  if (rc) return rc;
  if (B * T > 0 && (q == nullptr || k == nullptr || g == nullptr || dout == nullptr ||
                    dh == nullptr || dv == nullptr))
    return fail(TOPS_GLA_EINVAL, "no argument of chunk_bwd_dv may be NULL");
  tops::BwdArgs p = {};
  p.q = q;
  p.k = k;
  p.v = nullptr;
  p.g = g;
  p.dout = dout;
  p.h = nullptr;
  p.dh = dh;
  p.dq = p.dk = p.dg = nullptr;
  p.dv = dv;
  p.scale = scale;
  p.H = (int)H;
  p.K = (int)K;
  p.V = (int)V;
  p.vec = vec_ok(dtype, K, V, {q, k, g, dout, dh, dv});
  p.si = si;
  return hip_status(tops::run_chunk_bwd(p, dtype, (hipStream_t)stream, 2), "chunk_bwd_dv");
}

int tops_gla_fused_recurrent_fwd(const void* q, const void* k, const void* v, const void* gk,
                                 const void* gv, const float* h0, void* o, float* ht,
                                 float scale, int reverse, int64_t B, int64_t T, int64_t H,
                                 int64_t K, int64_t V, const int32_t* cu_seqlens, int64_t N,
                                 int dtype, int o_dtype, void* stream) {
  if (!dtype_ok(dtype) || !dtype_ok(o_dtype)) return fail(TOPS_GLA_EINVAL, "bad dtype");
  if (dtype == TOPS_GLA_F32 && o_dtype != TOPS_GLA_F32)
    return fail(TOPS_GLA_EUNSUPPORTED, "float32 inputs need a float32 output");
  if (K <= 0 || V <= 0) return fail(TOPS_GLA_EINVAL, "K and V must be positive");
  if (K > 512)
    return fail(TOPS_GLA_EUNSUPPORTED, "fused_recurrent keeps K <= 512 in registers (K=%lld)",
                (long long)K);
  tops::SeqInfo si;
  const int64_t NC = cu_seqlens ? 0 : B * T;  // chunk count unused; 1-token "chunks"
  int rc = make_seq(B, T, H, 1, cu_seqlens, nullptr, N, NC, false, &si);
  if (rc) return rc;
  if (B * T > 0 && (q == nullptr || k == nullptr || v == nullptr || o == nullptr))
    return fail(TOPS_GLA_EINVAL, "q, k, v and o must not be NULL");
  if ((int64_t)si.N * H * ((V + 31) / 32) > kMaxInt)
    return fail(TOPS_GLA_EUNSUPPORTED, "grid too large");
  tops::RecArgs p = {};
  p.q = q;
  p.k = k;
  p.v = v;
  p.gk = gk;
  p.gv = gv;
  p.h0 = h0;
  p.o = o;
  p.ht = ht;
  p.scale = scale;
  p.H = (int)H;
  p.K = (int)K;
  p.V = (int)V;
  p.reverse = reverse != 0;
  p.si = si;
  return hip_status(tops::run_recurrent_fwd(p, dtype, o_dtype, (hipStream_t)stream),
                    "fused_recurrent_fwd");
}

namespace {

int part_shape(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int C,
               std::initializer_list<const void*> ptrs, tops::PartArgs* p) {
  if (B < 0 || T < 0 || H <= 0 || K <= 0 || V <= 0)
    return fail(TOPS_GLA_EINVAL, "bad shape (B=%lld T=%lld H=%lld K=%lld V=%lld)",
                (long long)B, (long long)T, (long long)H, (long long)K, (long long)V);
  if (C != 16 && C != 32 && C != 64)
    return fail(TOPS_GLA_EUNSUPPORTED, "chunk_size %d (these kernels take 16, 32, 64)", C);
  if (T % C != 0)
    return fail(TOPS_GLA_EINVAL, "T (%lld) must be a multiple of chunk_size (%d)", (long long)T,
                C);
  if (B * T * H * std::max(K, std::max(V, (int64_t)C)) > (int64_t)1 << 40)
    return fail(TOPS_GLA_EUNSUPPORTED, "problem too large");
  if (B * T > 0)
    for (const void* q : ptrs)
      if (q == nullptr) return fail(TOPS_GLA_EINVAL, "NULL buffer");
  *p = tops::PartArgs{};
  p->H = (int)H;
  p->K = (int)K;
  p->V = (int)V;
  p->NC = (long)(B * (T / C));
  if (p->NC * H * ((std::max(K, V) + 63) / 64) > kMaxInt)
    return fail(TOPS_GLA_EUNSUPPORTED, "grid too large");
  return TOPS_GLA_OK;
}

}  // namespace

int tops_gla_bwd_part_dA(const float* v, const float* dout, float* dA, float scale, int64_t B,
                         int64_t T, int64_t H, int64_t V, int chunk_size, void* stream) {
  tops::PartArgs p = {};
  int rc = part_shape(B, T, H, 1, V, chunk_size, {v, dout, dA}, &p);
  if (rc) return rc;
  p.v = v;
  p.dout = dout;
  p.out0 = dA;
  p.scale = scale;
  return hip_status(tops::run_bwd_part(tops::PART_DA, p, chunk_size, (hipStream_t)stream),
                    "bwd_part_dA");
}

int tops_gla_bwd_part_dv(const float* k, const float* g_cumsum, const float* A,
                         const float* dout, const float* dh, float* dv, int64_t B, int64_t T,
                         int64_t H, int64_t K, int64_t V, int chunk_size, void* stream) {
  tops::PartArgs p = {};
  int rc = part_shape(B, T, H, K, V, chunk_size, {k, g_cumsum, A, dout, dh, dv}, &p);
  if (rc) return rc;
  p.k = k;
  p.g = g_cumsum;
  p.A = A;
  p.dout = dout;
  p.dh = dh;
  p.out0 = dv;
  return hip_status(tops::run_bwd_part(tops::PART_DV, p, chunk_size, (hipStream_t)stream),
                    "bwd_part_dv");
}

int tops_gla_bwd_part_dqk_intra(const float* q, const float* k, const float* g_cumsum,
                                const float* dA, float* dq, float* dk, int64_t B, int64_t T,
                                int64_t H, int64_t K, int chunk_size, void* stream) {
  tops::PartArgs p = {};
  int rc = part_shape(B, T, H, K, 1, chunk_size, {q, k, g_cumsum, dA, dq, dk}, &p);
  if (rc) return rc;
  p.q = q;
  p.k = k;
  p.g = g_cumsum;
  p.dA = dA;
  p.out0 = dq;
  p.out1 = dk;
  return hip_status(
      tops::run_bwd_part(tops::PART_DQK_INTRA, p, chunk_size, (hipStream_t)stream),
      "bwd_part_dqk_intra");
}

int tops_gla_bwd_part_dqkg(const float* q, const float* k, const float* v, const float* h,
                           const float* g_cumsum, const float* dout, const float* dh,
                           const float* dq, const float* dk, float* dq_out, float* dk_out,
                           float* dg, float scale, int64_t B, int64_t T, int64_t H, int64_t K,
                           int64_t V, int chunk_size, void* stream) {
  tops::PartArgs p = {};
  int rc = part_shape(B, T, H, K, V, chunk_size,
                      {q, k, v, h, g_cumsum, dout, dh, dq, dk, dq_out, dk_out, dg}, &p);
  if (rc) return rc;
  p.q = q;
  p.k = k;
  p.v = v;
  p.h = h;
  p.g = g_cumsum;
  p.dout = dout;
  p.dh = dh;
  p.dq = dq;
  p.dk = dk;
  p.out0 = dq_out;
  p.out1 = dk_out;
  p.out2 = dg;
  p.scale = scale;
  return hip_status(tops::run_bwd_part(tops::PART_DQKG, p, chunk_size, (hipStream_t)stream),
                    "bwd_part_dqkg");
}

namespace {

int norm_check(int64_t rows, int64_t D, int dtype, std::initializer_list<const void*> need,
               std::initializer_list<const void*> aligned) {
  if (!dtype_ok(dtype)) return fail(TOPS_GLA_EINVAL, "bad dtype");
  if (rows < 0 || D <= 0 || D % 8 != 0 || D > 8192)
    return fail(TOPS_GLA_EINVAL, "rows >= 0 and D a positive multiple of 8 up to 8192 "
                "(rows=%lld, D=%lld)", (long long)rows, (long long)D);
  if (rows > 0)
    for (const void* q : need)
      if (q == nullptr) return fail(TOPS_GLA_EINVAL, "NULL buffer");
  for (const void* q : aligned)
    if (!aligned16(q)) return fail(TOPS_GLA_EUNSUPPORTED, "buffers must be 16-byte aligned");
  return TOPS_GLA_OK;
}

}  // namespace

int64_t tops_gla_rmsnorm_ws_bytes(int64_t rows, int64_t D) {
  if (rows <= 0 || D <= 0) return 0;
  return tops::norm_gate_bwd_blocks((long)rows) * D * 4;
}

int tops_gla_rmsnorm_gated_fwd(const void* x, const void* g, const float* w, void* y,
                               float* rstd, int64_t rows, int64_t D, float eps, int dtype,
                               void* stream) {
  int rc = norm_check(rows, D, dtype, {x, y}, {x, g, w, y});
  if (rc) return rc;
  tops::NormGateArgs p = {};
  p.x = x;
  p.g = g;
  p.w = w;
  p.y = y;
  p.rstd = rstd;
  p.rows = (long)rows;
  p.D = (int)D;
  p.eps = eps;
  return hip_status(tops::run_norm_gate_fwd(p, dtype, (hipStream_t)stream), "rmsnorm_gated_fwd");
}

int tops_gla_rmsnorm_gated_bwd(const void* x, const void* g, const float* w, const float* rstd,
                               const void* dy, void* dx, void* dg, float* dw, void* dw_ws,
                               int64_t dw_ws_bytes, int64_t rows, int64_t D, int dtype,
                               void* stream) {
  int rc = norm_check(rows, D, dtype, {x, rstd, dy, dx}, {x, g, w, dy, dx, dg});
  if (rc) return rc;
  if (g != nullptr && dg == nullptr && rows > 0)
    return fail(TOPS_GLA_EINVAL, "dg is required when g is given");
  if (w != nullptr && dw != nullptr && rows > 0 &&
      (dw_ws == nullptr || dw_ws_bytes < tops_gla_rmsnorm_ws_bytes(rows, D)))
    return fail(TOPS_GLA_EINVAL, "dw needs dw_ws of tops_gla_rmsnorm_ws_bytes bytes");
  tops::NormGateArgs p = {};
  p.x = x;
  p.g = g;
  p.w = w;
  p.rstd = const_cast<float*>(rstd);
  p.dy = dy;
  p.dx = dx;
  p.dg = dg;
  p.dw_part = dw ? (float*)dw_ws : nullptr;
  p.rows = (long)rows;
  p.D = (int)D;
  return hip_status(tops::run_norm_gate_bwd(p, dw, dtype, (hipStream_t)stream),
                    "rmsnorm_gated_bwd");
}

int tops_gla_gate_logsigmoid_fwd(const void* x, void* y, int64_t count, float normalizer,
                                 int has_clamp, float clamp_min, int dtype, void* stream) {
  if (!dtype_ok(dtype)) return fail(TOPS_GLA_EINVAL, "bad dtype");
  if (count < 0 || normalizer == 0.f) return fail(TOPS_GLA_EINVAL, "bad count or normalizer");
  if (count > 0 && (x == nullptr || y == nullptr)) return fail(TOPS_GLA_EINVAL, "NULL buffer");
  if (!aligned16(x) || !aligned16(y))
    return fail(TOPS_GLA_EUNSUPPORTED, "buffers must be 16-byte aligned");
  return hip_status(tops::run_gate(x, nullptr, y, (long)count, 1.f / normalizer, has_clamp,
                                   clamp_min, dtype, (hipStream_t)stream),
                    "gate_logsigmoid_fwd");
}

int tops_gla_concat_cols(const void* const* srcs, const int64_t* widths, int nsrc,
                         int64_t rows, void* dst, int dtype, void* stream) {
  if (!dtype_ok(dtype)) return fail(TOPS_GLA_EINVAL, "bad dtype");
  if (nsrc < 1 || nsrc > tops::kConcatMax || rows < 0 || srcs == nullptr || widths == nullptr)
    return fail(TOPS_GLA_EINVAL, "nsrc must be in [1, 8], rows >= 0, srcs and widths set");
  const int es = dtype == TOPS_GLA_BF16 ? 2 : 4;
  long w[tops::kConcatMax];
  for (int j = 0; j < nsrc; ++j) {
    if (widths[j] <= 0 || (widths[j] * es) % 16 != 0)
      return fail(TOPS_GLA_EUNSUPPORTED, "every width must be a positive multiple of 16 bytes");
    if (rows > 0 && (srcs[j] == nullptr || !aligned16(srcs[j])))
      return fail(TOPS_GLA_EINVAL, "sources must be non-NULL and 16-byte aligned");
    w[j] = (long)widths[j];
  }
  if (rows > 0 && (dst == nullptr || !aligned16(dst)))
    return fail(TOPS_GLA_EINVAL, "dst must be non-NULL and 16-byte aligned");
  return hip_status(tops::run_concat_cols(srcs, w, nsrc, (long)rows, dst, es,
                                          (hipStream_t)stream),
                    "concat_cols");
}

int tops_gla_gate_logsigmoid_bwd(const void* x, const void* dy, void* dx, int64_t count,
                                 float normalizer, int has_clamp, float clamp_min, int dtype,
                                 void* stream) {
  if (!dtype_ok(dtype)) return fail(TOPS_GLA_EINVAL, "bad dtype");
  if (count < 0 || normalizer == 0.f) return fail(TOPS_GLA_EINVAL, "bad count or normalizer");
  if (count > 0 && (x == nullptr || dy == nullptr || dx == nullptr))
    return fail(TOPS_GLA_EINVAL, "NULL buffer");
  if (!aligned16(x) || !aligned16(dy) || !aligned16(dx))
    return fail(TOPS_GLA_EUNSUPPORTED, "buffers must be 16-byte aligned");
  return hip_status(tops::run_gate(x, dy, dx, (long)count, 1.f / normalizer, has_clamp,
                                   clamp_min, dtype, (hipStream_t)stream),
                    "gate_logsigmoid_bwd");
}

namespace {

int conv_setup(int64_t B, int64_t T, int64_t D, int W, const int32_t* cu, int64_t N,
               int64_t max_len, int dtype, tops::ShortConvArgs* p) {
  if (!dtype_ok(dtype)) return fail(TOPS_GLA_EINVAL, "bad dtype");
  if (D <= 0 || D % 8 != 0 || D > (1 << 20))
    return fail(TOPS_GLA_EINVAL, "D must be a positive multiple of 8 (D=%lld)", (long long)D);
  if (W < 1 || W > 8) return fail(TOPS_GLA_EUNSUPPORTED, "kernel width W in 1..8 (W=%d)", W);
  tops::SeqInfo si;
  const int64_t NC = cu ? 0 : B * T;
  int rc = make_seq(B, T, 1, 1, cu, nullptr, N, NC, false, &si);
  if (rc) return rc;
  if (cu && (max_len < 0 || max_len > T)) return fail(TOPS_GLA_EINVAL, "bad max_len");
  *p = tops::ShortConvArgs{};
  p->D = (int)D;
  p->W = W;
  p->max_len = (int)(cu ? max_len : T);
  p->si = si;
  return TOPS_GLA_OK;
}

}  // namespace

int64_t tops_gla_short_conv_ws_bytes(int64_t B, int64_t T, int64_t D, int W, int64_t N,
                                     int64_t max_len, int varlen) {
  if (B <= 0 || T <= 0 || D <= 0 || W < 1 || W > 8) return 0;
  const long rows = varlen ? tops::short_conv_part_rows((long)N, (long)max_len)
                           : tops::short_conv_part_rows((long)B, (long)T);
  return (int64_t)rows * (W + 1) * D * 4;
}

int tops_gla_short_conv_fwd(const void* x, const float* w, const float* bias, void* y,
                            int64_t B, int64_t T, int64_t D, int W, int silu,
                            const int32_t* cu_seqlens, int64_t N, int64_t max_len, int dtype,
                            void* stream) {
  tops::ShortConvArgs p = {};
  int rc = conv_setup(B, T, D, W, cu_seqlens, N, max_len, dtype, &p);
  if (rc) return rc;
  if (B * T > 0 && (x == nullptr || w == nullptr || y == nullptr))
    return fail(TOPS_GLA_EINVAL, "x, w and y must not be NULL");
  if (!aligned16(x) || !aligned16(y))
    return fail(TOPS_GLA_EUNSUPPORTED, "buffers must be 16-byte aligned");
  p.x = x;
  p.y = y;
  p.w = w;
  p.bias = bias;
  p.silu = silu != 0;
  return hip_status(tops::run_short_conv(p, false, dtype, (hipStream_t)stream), "short_conv_fwd");
}

int tops_gla_short_conv_bwd(const void* x, const float* w, const float* bias, const void* dy,
                            void* dx, float* dw_db, void* ws, int64_t ws_bytes, int64_t B,
                            int64_t T, int64_t D, int W, int silu, const int32_t* cu_seqlens,
                            int64_t N, int64_t max_len, int dtype, void* stream) {
  tops::ShortConvArgs p = {};
  int rc = conv_setup(B, T, D, W, cu_seqlens, N, max_len, dtype, &p);
  if (rc) return rc;
  if (B * T > 0 && (x == nullptr || w == nullptr || dy == nullptr || dx == nullptr))
    return fail(TOPS_GLA_EINVAL, "x, w, dy and dx must not be NULL");
  if (!aligned16(x) || !aligned16(dy) || !aligned16(dx))
    return fail(TOPS_GLA_EUNSUPPORTED, "buffers must be 16-byte aligned");
  p.x = x;
  p.dy = dy;
  p.dx = dx;
  p.w = w;
  p.bias = bias;
  p.silu = silu != 0;
  if (dw_db) {
    const int64_t need = tops_gla_short_conv_ws_bytes(B, T, D, W, N, max_len,
                                                      cu_seqlens != nullptr);
    if (ws == nullptr || ws_bytes < need)
      return fail(TOPS_GLA_EINVAL, "dw_db needs ws of tops_gla_short_conv_ws_bytes bytes");
    p.part = (float*)ws;
    p.dwb = dw_db;
  }
  return hip_status(tops::run_short_conv(p, true, dtype, (hipStream_t)stream), "short_conv_bwd");
}

int tops_gla_fused_recurrent_bwd(const void* q, const void* k, const void* v, const void* gk,
                                 const void* gv, const float* o, const void* dout,
                                 const float* dht, const float* h0, float* dq, float* dk,
                                 float* dv, float* dgk, float* dgv, float* dh0, float* ht_ws,
                                 float scale, int reverse, int64_t B, int64_t T, int64_t H,
                                 int64_t K, int64_t V, const int32_t* cu_seqlens, int64_t N,
                                 int dtype, void* stream) {
  if (!dtype_ok(dtype)) return fail(TOPS_GLA_EINVAL, "bad dtype");
  if (K <= 0 || V <= 0) return fail(TOPS_GLA_EINVAL, "K and V must be positive");
  if (!tops::recurrent_supported((int)std::min<int64_t>(K, 1 << 20),
                                 (int)std::min<int64_t>(V, 1 << 20)))
    return fail(TOPS_GLA_EUNSUPPORTED,
                "fused_recurrent backward keeps K, V <= 512 in registers (K=%lld, V=%lld)",
                (long long)K, (long long)V);
  tops::SeqInfo si;
  const int64_t NC = cu_seqlens ? 0 : B * T;
  int rc = make_seq(B, T, H, 1, cu_seqlens, nullptr, N, NC, false, &si);
  if (rc) return rc;
  if (B * T > 0 && (q == nullptr || k == nullptr || v == nullptr || dout == nullptr ||
                    dq == nullptr || dk == nullptr || dv == nullptr))
    return fail(TOPS_GLA_EINVAL, "q, k, v, dout, dq, dk and dv must not be NULL");
  if ((gk == nullptr) != (dgk == nullptr))
    return fail(TOPS_GLA_EINVAL, "dgk must be given exactly when gk is");
  if ((gv == nullptr) != (dgv == nullptr))
    return fail(TOPS_GLA_EINVAL, "dgv must be given exactly when gv is");
  if (gv != nullptr && B * T > 0 && o == nullptr)
    return fail(TOPS_GLA_EINVAL, "o (forward output) is required when gv is used");
  if (dht != nullptr && (gk != nullptr || gv != nullptr) && ht_ws == nullptr)
    return fail(TOPS_GLA_EINVAL, "ht_ws is required when dht and a gate are given");
  if ((int64_t)si.N * H * ((std::max(K, V) + 31) / 32) > kMaxInt)
    return fail(TOPS_GLA_EUNSUPPORTED, "grid too large");
  tops::RecBwdArgs p = {};
  p.q = q;
  p.k = k;
  p.v = v;
  p.gk = gk;
  p.gv = gv;
  p.dout = dout;
  p.o = o;
  p.h0 = h0;
  p.dht = dht;
  p.dq = dq;
  p.dk = dk;
  p.dv = dv;
  p.dgk = dgk;
  p.dgv = dgv;
  p.dh0 = dh0;
  p.ht_ws = ht_ws;
  p.scale = scale;
  p.H = (int)H;
  p.K = (int)K;
  p.V = (int)V;
  p.reverse = reverse != 0;
  p.si = si;
  return hip_status(tops::run_recurrent_bwd(p, dtype, tops::DT_F32, (hipStream_t)stream),
                    "fused_recurrent_bwd");
}

}  // extern "C"
