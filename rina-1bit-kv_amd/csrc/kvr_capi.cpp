// Host side of the C ABI declared in include/kvr_capi.h: argument validation
// (entirely before any HIP call, so a rejected call never touches the device),
// workspace planning, and the launch sequence of each entry point.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <atomic>
#include <cstdio>
#include <string>

#include "../../include/kvr_capi.h"
#include "kvr_internal.h"

namespace {

constexpr int kAbiVersion = 4;
constexpr int kMaxTopK = 1024;
constexpr size_t kAlign = 256;

thread_local std::string g_last_error;

int vfail(int code, const char* fmt, va_list ap) {
  char buf[512];
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  g_last_error = buf;
  return code;
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  const int r = vfail(code, fmt, ap);
  va_end(ap);
  return r;
}

// Bounded-wait settings of every later decode launch (kvr_set_wait_limit).
std::atomic<int> g_spin_max{1 << 20};
std::atomic<int> g_wait_fail{0};

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return KVR_OK;
  return fail(KVR_ERR_HIP, "%s: HIP error %d (%s)", what, (int)e, hipGetErrorString(e));
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }
size_t elem_size(int dt) { return dt == KVR_FP32 ? 4 : 2; }
bool valid_dtype(int dt) { return dt == KVR_BF16 || dt == KVR_FP16 || dt == KVR_FP32; }
bool valid_transform(int tf) { return tf == KVR_HADAMARD || tf == KVR_DCT || tf == KVR_NONE; }
size_t round_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

int check_common(int d, int T) {
  if (d != 128) return fail(KVR_ERR_INVALID, "head_dim d=%d unsupported (must be 128)", d);
  if (T != 64 && T != 128) return fail(KVR_ERR_INVALID, "tile size T=%d unsupported (64 or 128)", T);
  return KVR_OK;
}

int check_heads(int64_t B, int Hq, int Hkv) {
  if (B < 0) return fail(KVR_ERR_INVALID, "batch B=%lld < 0", (long long)B);
  if (Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0)
    return fail(KVR_ERR_INVALID, "Hq=%d must be a positive multiple of Hkv=%d", Hq, Hkv);
  if (Hq / Hkv > 16)
    return fail(KVR_ERR_UNSUPPORTED, "GQA group size g=%d > 16 is not built", Hq / Hkv);
  return KVR_OK;
}

// Window: 16-byte loads along head_dim (8 16-bit or 4 fp32 elements); a ring of win_cap
// slots holds the win_len valid tokens from slot win_start on.
int check_window(const void* wk, const void* wv, int wdt, int64_t win_len, int64_t win_start, int64_t win_cap,
                 int64_t sb, int64_t sh, int64_t st) {
  if (win_len < 0) return fail(KVR_ERR_INVALID, "win_len=%lld < 0", (long long)win_len);
  if (win_cap < 0) return fail(KVR_ERR_INVALID, "win_cap=%lld < 0", (long long)win_cap);
  if (win_cap > 0 && win_len > win_cap)
    return fail(KVR_ERR_INVALID, "win_len=%lld exceeds the ring capacity %lld", (long long)win_len,
                (long long)win_cap);
  if (win_start < 0 || (win_cap > 0 ? win_start >= win_cap : win_start != 0))
    return fail(KVR_ERR_INVALID, "win_start=%lld outside the ring (capacity %lld; 0 without a ring)",
                (long long)win_start, (long long)win_cap);
  if (win_cap % 32 || win_start % 32)
    return fail(KVR_ERR_INVALID, "a ring's capacity and start must be multiples of 32 (%lld, %lld)",
                (long long)win_cap, (long long)win_start);
  if (win_len == 0 && win_cap == 0) return KVR_OK;
  if (!valid_dtype(wdt)) return fail(KVR_ERR_INVALID, "window dtype %d unknown", wdt);
  if (!wk || !wv) return fail(KVR_ERR_INVALID, "window pointers are NULL");
  if (!aligned(wk, 16) || !aligned(wv, 16))
    return fail(KVR_ERR_ALIGN, "window pointers must be 16-byte aligned");
  const int64_t vec = 16 / (int64_t)elem_size(wdt);
  if (sb < 0 || sh < 0 || st <= 0 || sb % vec || sh % vec || st % vec)
    return fail(KVR_ERR_ALIGN, "window strides (b=%lld h=%lld t=%lld) must be non-negative multiples of %lld elements",
                (long long)sb, (long long)sh, (long long)st, (long long)vec);
  return KVR_OK;
}

int check_store(const uint64_t* kb, const uint64_t* vb, const uint16_t* ks, const uint16_t* vs,
                int64_t tile_stride) {
  if (!kb || !vb || !ks || !vs) return fail(KVR_ERR_INVALID, "tile store pointers are NULL");
  if (!aligned(kb, 16) || !aligned(vb, 16))
    return fail(KVR_ERR_ALIGN, "bit arrays must be 16-byte aligned");
  if (!aligned(ks, 2) || !aligned(vs, 2)) return fail(KVR_ERR_ALIGN, "scale arrays must be 2-byte aligned");
  if (tile_stride <= 0) return fail(KVR_ERR_INVALID, "tile_stride=%lld must be > 0", (long long)tile_stride);
  return KVR_OK;
}

struct StepLayout {
  size_t ctr, scores, cand, idx, rec, total;
};

// Workspace: [counters | scores | candidate lists | idx | partial records].  The counter
// region (same size and place in every decode workspace) must be zero before the
// workspace's first call; every call leaves it zero.  The rest is scratch.
StepLayout step_layout(int64_t B, int Hq, int Hkv, int64_t win_len, int64_t n_tiles, int k, int T) {
  StepLayout L{};
  size_t off = 0;
  L.ctr = off;
  off += round_up(kvr::counter_bytes());
  L.scores = off;
  off += round_up((size_t)(B * Hkv) * (size_t)(n_tiles > 0 ? n_tiles : 0) * sizeof(float));
  L.cand = off;
  off += round_up(kvr::cand_bytes(B, Hkv, n_tiles, k, T));
  L.idx = off;
  off += round_up((size_t)(B * Hkv) * (size_t)(k > 0 ? k : 0) * sizeof(int32_t));
  L.rec = off;
  off += round_up(kvr::records_bytes(B, Hq, Hkv, win_len, k, T));
  L.total = off;
  return L;
}

}  // namespace

extern "C" {

int kvr_abi_version(void) { return kAbiVersion; }

const char* kvr_last_error(void) { return g_last_error.c_str(); }

int kvr_encode_tiles(const void* x, int x_dtype, int64_t n_b, int64_t n_h, int64_t n_tok,
                     int64_t stride_b, int64_t stride_h, int64_t stride_t, int d, int T,
                     int transform, uint64_t* bits, uint16_t* scales, int64_t out_tile_stride,
                     int64_t out_tile_offset, float* dbg_rotated, uint8_t* counts, kvr_stream_t stream) {
  if (int r = check_common(d, T)) return r;
  if (!valid_dtype(x_dtype)) return fail(KVR_ERR_INVALID, "input dtype %d unknown", x_dtype);
  if (!valid_transform(transform)) return fail(KVR_ERR_INVALID, "transform %d unknown", transform);
  if (transform == KVR_NONE && x_dtype != KVR_FP32)
    return fail(KVR_ERR_INVALID, "transform NONE takes already-rotated fp32 input");
  if (n_b < 0 || n_h < 0 || n_tok < 0) return fail(KVR_ERR_INVALID, "negative size");
  if (n_tok % T) return fail(KVR_ERR_INVALID, "n_tok=%lld is not a multiple of T=%d", (long long)n_tok, T);
  const int64_t n_tiles = n_tok / T;
  if (out_tile_offset < 0 || out_tile_stride < out_tile_offset + n_tiles)
    return fail(KVR_ERR_INVALID, "tile slots [%lld, %lld) exceed out_tile_stride=%lld",
                (long long)out_tile_offset, (long long)(out_tile_offset + n_tiles),
                (long long)out_tile_stride);
  if (n_b * n_h * n_tiles == 0) return KVR_OK;
  if (!x || !bits || !scales) return fail(KVR_ERR_INVALID, "x, bits and scales must be non-NULL");
  const int64_t vec = 16 / (int64_t)elem_size(x_dtype);
  if (!aligned(x, 16) || stride_b % vec || stride_h % vec || stride_t % vec)
    return fail(KVR_ERR_ALIGN, "x and its strides must be 16-byte aligned");
  if (stride_b < 0 || stride_h < 0 || stride_t <= 0) return fail(KVR_ERR_INVALID, "bad input strides");
  if (!aligned(bits, 8) || !aligned(scales, 2) || (dbg_rotated && !aligned(dbg_rotated, 16)) ||
      (counts && !aligned(counts, 8)))
    return fail(KVR_ERR_ALIGN, "output pointers misaligned");
  return hip_status(kvr::launch_encode(x_dtype, transform, T, x, n_b, n_h, n_tok, stride_b,
                                       stride_h, stride_t, bits, scales, out_tile_stride,
                                       out_tile_offset, dbg_rotated, counts, (hipStream_t)stream),
                    "kvr_encode_tiles");
}

int kvr_query_prep(const void* q, int q_dtype, int64_t B, int Hq, int Hkv, int d, int transform,
                   float* qbar_rot, float* q_rot, kvr_stream_t stream) {
  if (d != 128) return fail(KVR_ERR_INVALID, "head_dim d=%d unsupported (must be 128)", d);
  if (int r = check_heads(B, Hq, Hkv)) return r;
  if (!valid_dtype(q_dtype)) return fail(KVR_ERR_INVALID, "q dtype %d unknown", q_dtype);
  if (!valid_transform(transform)) return fail(KVR_ERR_INVALID, "transform %d unknown", transform);
  if (B == 0) return KVR_OK;
  if (!q || !qbar_rot) return fail(KVR_ERR_INVALID, "q and qbar_rot must be non-NULL");
  return hip_status(kvr::launch_query_prep(q_dtype, transform, q, B, Hq, Hkv, qbar_rot, q_rot,
                                           (hipStream_t)stream),
                    "kvr_query_prep");
}

int kvr_score_tiles(const float* qbar_rot, const uint64_t* kbits, int64_t BH, int64_t n_tiles,
                    int64_t tile_stride, int d, int T, const int32_t* excl_lo,
                    const int32_t* excl_hi, int method, float* scores, kvr_stream_t stream) {
  if (int r = check_common(d, T)) return r;
  if (method != 0 && method != 1) return fail(KVR_ERR_INVALID, "score method %d unknown", method);
  if (BH < 0 || n_tiles < 0) return fail(KVR_ERR_INVALID, "negative size");
  if (tile_stride < n_tiles) return fail(KVR_ERR_INVALID, "tile_stride < n_tiles");
  if (BH * n_tiles == 0) return KVR_OK;
  if (!qbar_rot || !kbits || !scores) return fail(KVR_ERR_INVALID, "NULL pointer");
  if (!aligned(qbar_rot, 16) || !aligned(kbits, 16))
    return fail(KVR_ERR_ALIGN, "qbar_rot and kbits must be 16-byte aligned");
  if ((excl_lo == nullptr) != (excl_hi == nullptr))
    return fail(KVR_ERR_INVALID, "excl_lo and excl_hi must both be given or both NULL");
  return hip_status(kvr::launch_score(T, method, qbar_rot, kbits, BH, n_tiles, tile_stride, excl_lo,
                                      excl_hi, scores, (hipStream_t)stream),
                    "kvr_score_tiles");
}

int kvr_topk_tiles(const float* scores, int64_t BH, int64_t n_tiles, int64_t score_stride, int k,
                   int32_t* idx, kvr_stream_t stream) {
  if (BH < 0) return fail(KVR_ERR_INVALID, "negative size");
  if (k < 1 || k > kMaxTopK || k > n_tiles)
    return fail(KVR_ERR_INVALID, "k=%d must be in [1, min(n_tiles=%lld, %d)]", k,
                (long long)n_tiles, kMaxTopK);
  if (score_stride < n_tiles) return fail(KVR_ERR_INVALID, "score_stride < n_tiles");
  if (BH == 0) return KVR_OK;
  if (!scores || !idx) return fail(KVR_ERR_INVALID, "NULL pointer");
  return hip_status(kvr::launch_topk(scores, BH, n_tiles, score_stride, k, idx, (hipStream_t)stream),
                    "kvr_topk_tiles");
}

size_t kvr_decode_attn_workspace(int64_t B, int Hq, int Hkv, int64_t win_len, int k, int T) {
  if (B < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv) return 0;
  return step_layout(B, Hq, Hkv, win_len, 0, k, T).total;
}

}  // extern "C"

namespace {

int attn_checks(const void* q, int q_dtype, int64_t B, int Hq, int Hkv, int d,
                       const void* win_k, const void* win_v, int win_dtype, int64_t win_len,
                       int64_t win_start, int64_t win_cap, int64_t sb, int64_t sh, int64_t st,
                       const uint64_t* kbits, const uint64_t* vbits, const uint16_t* kscale,
                       const uint16_t* vscale, int64_t tile_stride, int T, int transform, int k,
                       void* out, int out_dtype) {
  if (int r = check_common(d, T)) return r;
  if (int r = check_heads(B, Hq, Hkv)) return r;
  if (!valid_dtype(q_dtype)) return fail(KVR_ERR_INVALID, "q dtype %d unknown", q_dtype);
  if (!valid_transform(transform)) return fail(KVR_ERR_INVALID, "transform %d unknown", transform);
  if (out_dtype != KVR_BF16 && out_dtype != KVR_FP32)
    return fail(KVR_ERR_INVALID, "out dtype %d unsupported (bf16 or fp32)", out_dtype);
  if (k < 0 || k > kMaxTopK) return fail(KVR_ERR_INVALID, "k=%d out of [0, %d]", k, kMaxTopK);
  if (int r = check_window(win_k, win_v, win_dtype, win_len, win_start, win_cap, sb, sh, st)) return r;
  if (k > 0)
    if (int r = check_store(kbits, vbits, kscale, vscale, tile_stride)) return r;
  if (B > 0 && (!q || !out)) return fail(KVR_ERR_INVALID, "q and out must be non-NULL");
  if (B > 0 && !aligned(q, 16)) return fail(KVR_ERR_ALIGN, "q must be 16-byte aligned");
  if (B > 0 && !aligned(out, 8)) return fail(KVR_ERR_ALIGN, "out must be 8-byte aligned");
  return KVR_OK;
}

kvr::DecodeLaunch base_launch(const void* q, int q_dtype, int64_t B, int Hq, int Hkv,
                                     const void* win_k, const void* win_v, int win_dtype, int64_t win_len,
                                     int64_t win_start, int64_t win_cap, int64_t sb, int64_t sh, int64_t st,
                                     const uint64_t* kbits, const uint64_t* vbits, const uint16_t* kscale,
                                     const uint16_t* vscale, int64_t tile_stride, int T, int transform, int k,
                                     void* out, int out_dtype) {
  kvr::DecodeLaunch L{};
  L.qt = q_dtype;
  L.q = q;
  L.B = B;
  L.Hq = Hq;
  L.Hkv = Hkv;
  const bool win = win_len > 0 || win_cap > 0;
  L.wk = win ? win_k : nullptr;
  L.wv = win ? win_v : nullptr;
  L.wdt = win ? win_dtype : KVR_BF16;
  L.win_len = win_len;
  L.win_start = win_start;
  L.win_cap = win_cap;
  L.sb = sb;
  L.sh = sh;
  L.st = st;
  L.kb = kbits;
  L.vb = vbits;
  L.ks = kscale;
  L.vs = vscale;
  L.tile_stride = tile_stride;
  L.T = T;
  L.tf = transform;
  L.k = k;
  L.out = out;
  L.ot = out_dtype;
  L.spin_max = g_spin_max.load(std::memory_order_relaxed);
  L.wait_fail = g_wait_fail.load(std::memory_order_relaxed);
  return L;
}

}  // namespace

namespace kvr {

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  const int r = vfail(code, fmt, ap);
  va_end(ap);
  return r;
}

size_t decode_step_workspace_bytes(int64_t B, int Hq, int Hkv, int64_t win_len, int64_t n_tiles, int k, int T) {
  if (B < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || n_tiles < 0 || (T != 64 && T != 128)) return 0;
  if (n_tiles == 0) k = 0;
  return step_layout(B, Hq, Hkv, win_len, k > 0 ? n_tiles : 0, k, T).total;
}

int decode_step_impl(const void* q, int q_dtype, int64_t B, int Hq, int Hkv, int d,
                     const void* win_k, const void* win_v, int win_dtype, int64_t win_len,
                     int64_t win_start, int64_t win_cap, int64_t win_stride_b, int64_t win_stride_h,
                     int64_t win_stride_t, const uint64_t* kbits, const uint64_t* vbits,
                     const uint16_t* kscale, const uint16_t* vscale, const uint8_t* kcounts,
                     int64_t n_tiles, int64_t tile_stride, int T, int transform,
                     const int32_t* excl_lo, const int32_t* excl_hi, int k, const int32_t* live_state,
                     void* out, int out_dtype, int32_t* idx_out, void* workspace, size_t ws_bytes,
                     hipStream_t stream, bool launch) {
  if (n_tiles < 0) return fail(KVR_ERR_INVALID, "n_tiles < 0");
  if (n_tiles == 0) k = 0;
  if (k > n_tiles) return fail(KVR_ERR_INVALID, "k=%d > n_tiles=%lld", k, (long long)n_tiles);
  if (k > 0 && tile_stride < n_tiles) return fail(KVR_ERR_INVALID, "tile_stride < n_tiles");
  if (int r = attn_checks(q, q_dtype, B, Hq, Hkv, d, win_k, win_v, win_dtype, win_len, live_state ? 0 : win_start,
                          win_cap, win_stride_b, win_stride_h, win_stride_t, kbits, vbits, kscale, vscale,
                          tile_stride, T, transform, k, out, out_dtype))
    return r;
  if ((excl_lo == nullptr) != (excl_hi == nullptr))
    return fail(KVR_ERR_INVALID, "excl_lo and excl_hi must both be given or both NULL");
  if (kcounts && !aligned(kcounts, 8)) return fail(KVR_ERR_ALIGN, "kcounts must be 8-byte aligned");
  if (live_state) {
    if (!aligned(live_state, 16)) return fail(KVR_ERR_ALIGN, "live_state must be 16-byte aligned");
    if (win_cap <= 0) return fail(KVR_ERR_INVALID, "a live state needs a ring window (win_cap > 0)");
    if (!kvr::step_is_fused(B * Hkv, k, true))
      return fail(KVR_ERR_UNSUPPORTED,
                  "a live state needs the one-launch step (1 <= k <= 64, B*Hkv <= 4096, MFMA retrieval); k=%d", k);
  }
  if (B == 0) return KVR_OK;
  const int64_t nt = (k > 0) ? n_tiles : 0;
  const StepLayout W = step_layout(B, Hq, Hkv, win_len, nt, k, T);
  if (!launch) {
    if (ws_bytes < W.total)
      return fail(KVR_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu available", W.total, ws_bytes);
    return KVR_OK;
  }
  if (!workspace || ws_bytes < W.total)
    return fail(KVR_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", W.total,
                workspace ? ws_bytes : (size_t)0);
  if (!aligned(workspace, kAlign)) return fail(KVR_ERR_ALIGN, "workspace must be 256-byte aligned");
  char* ws = (char*)workspace;
  kvr::DecodeLaunch L = base_launch(q, q_dtype, B, Hq, Hkv, win_k, win_v, win_dtype, win_len, win_start, win_cap,
                                    win_stride_b, win_stride_h, win_stride_t, kbits, vbits, kscale, vscale,
                                    tile_stride, T, transform, k, out, out_dtype);
  L.kc = kcounts;
  L.n_tiles = n_tiles;
  L.excl_lo = excl_lo;
  L.excl_hi = excl_hi;
  L.live = live_state;
  L.do_select = true;
  L.scores = (float*)(ws + W.scores);
  L.cand = (uint64_t*)(ws + W.cand);
  L.idx = idx_out ? idx_out : (int32_t*)(ws + W.idx);
  L.rec = (float*)(ws + W.rec);
  L.ctr = (int32_t*)(ws + W.ctr);
  return hip_status(kvr::launch_decode(L, stream), "kvr_decode_step");
}

}  // namespace kvr

extern "C" {

int kvr_decode_attn(const void* q, int q_dtype, int64_t B, int Hq, int Hkv, int d,
                    const void* win_k, const void* win_v, int win_dtype, int64_t win_len,
                    int64_t win_start, int64_t win_cap, int64_t win_stride_b, int64_t win_stride_h,
                    int64_t win_stride_t, const uint64_t* kbits, const uint64_t* vbits,
                    const uint16_t* kscale, const uint16_t* vscale, int64_t tile_stride, int T, int transform,
                    const int32_t* idx, int k, void* out, int out_dtype, void* workspace,
                    size_t ws_bytes, kvr_stream_t stream) {
  if (int r = attn_checks(q, q_dtype, B, Hq, Hkv, d, win_k, win_v, win_dtype, win_len, win_start, win_cap,
                          win_stride_b, win_stride_h, win_stride_t, kbits, vbits, kscale, vscale,
                          tile_stride, T, transform, k, out, out_dtype))
    return r;
  if (k > 0 && !idx) return fail(KVR_ERR_INVALID, "idx must be non-NULL when k > 0");
  if (B == 0) return KVR_OK;
  const StepLayout W = step_layout(B, Hq, Hkv, win_len, 0, k, T);
  if (!workspace || ws_bytes < W.total)
    return fail(KVR_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", W.total,
                workspace ? ws_bytes : (size_t)0);
  if (!aligned(workspace, kAlign)) return fail(KVR_ERR_ALIGN, "workspace must be 256-byte aligned");
  char* ws = (char*)workspace;
  kvr::DecodeLaunch L = base_launch(q, q_dtype, B, Hq, Hkv, win_k, win_v, win_dtype, win_len, win_start, win_cap,
                                    win_stride_b, win_stride_h, win_stride_t, kbits, vbits, kscale, vscale,
                                    tile_stride, T, transform, k, out, out_dtype);
  L.idx = const_cast<int32_t*>(idx);
  L.rec = (float*)(ws + W.rec);
  return hip_status(kvr::launch_decode(L, (hipStream_t)stream), "kvr_decode_attn");
}

size_t kvr_decode_step_workspace(int64_t B, int Hq, int Hkv, int64_t win_len, int64_t n_tiles,
                                 int k, int T) {
  return kvr::decode_step_workspace_bytes(B, Hq, Hkv, win_len, n_tiles, k, T);
}

int kvr_decode_step(const void* q, int q_dtype, int64_t B, int Hq, int Hkv, int d,
                    const void* win_k, const void* win_v, int win_dtype, int64_t win_len,
                    int64_t win_start, int64_t win_cap, int64_t win_stride_b, int64_t win_stride_h,
                    int64_t win_stride_t, const uint64_t* kbits, const uint64_t* vbits,
                    const uint16_t* kscale, const uint16_t* vscale, const uint8_t* kcounts,
                    int64_t n_tiles, int64_t tile_stride, int T, int transform, const int32_t* excl_lo,
                    const int32_t* excl_hi, int k, const int32_t* live_state, void* out, int out_dtype,
                    int32_t* idx_out, void* workspace, size_t ws_bytes, kvr_stream_t stream) {
  return kvr::decode_step_impl(q, q_dtype, B, Hq, Hkv, d, win_k, win_v, win_dtype, win_len, win_start, win_cap,
                               win_stride_b, win_stride_h, win_stride_t, kbits, vbits, kscale, vscale, kcounts,
                               n_tiles, tile_stride, T, transform, excl_lo, excl_hi, k, live_state, out,
                               out_dtype, idx_out, workspace, ws_bytes, (hipStream_t)stream);
}

int kvr_cache_append(const void* k_new, const void* v_new, int new_dtype, int64_t B, int Hkv, int d,
                     void* win_k, void* win_v, int win_dtype, int64_t win_stride_b, int64_t win_stride_h,
                     int64_t win_stride_t, int64_t W, int T, int transform, uint64_t* kbits, uint64_t* vbits,
                     uint16_t* kscale, uint16_t* vscale, uint8_t* kcounts, int64_t tile_stride,
                     int32_t* state, kvr_stream_t stream) {
  if (int r = check_common(d, T)) return r;
  if (B < 0 || Hkv <= 0) return fail(KVR_ERR_INVALID, "B=%lld, Hkv=%d", (long long)B, Hkv);
  if (!valid_dtype(new_dtype)) return fail(KVR_ERR_INVALID, "new-token dtype %d unknown", new_dtype);
  if (transform != KVR_HADAMARD && transform != KVR_DCT)
    return fail(KVR_ERR_INVALID, "transform %d unsupported for the cache (Hadamard or DCT)", transform);
  if (W < T || W % T) return fail(KVR_ERR_INVALID, "window W=%lld must be a positive multiple of T=%d", (long long)W, T);
  if (W + T > (1ll << 30)) return fail(KVR_ERR_INVALID, "window W=%lld too large", (long long)W);
  if (int r = check_window(win_k, win_v, win_dtype, W + T, 0, W + T, win_stride_b, win_stride_h, win_stride_t))
    return r;
  if (int r = check_store(kbits, vbits, kscale, vscale, tile_stride)) return r;
  if (tile_stride > (1ll << 30)) return fail(KVR_ERR_INVALID, "tile_stride too large");
  if (kcounts && !aligned(kcounts, 8)) return fail(KVR_ERR_ALIGN, "kcounts must be 8-byte aligned");
  if (B == 0) return KVR_OK;
  if (!k_new || !v_new || !state) return fail(KVR_ERR_INVALID, "k_new, v_new and state must be non-NULL");
  if (!aligned(state, 16)) return fail(KVR_ERR_ALIGN, "state must be 16-byte aligned");
  kvr::AppendLaunch L{};
  L.k_new = k_new;
  L.v_new = v_new;
  L.ndt = new_dtype;
  L.B = B;
  L.Hkv = Hkv;
  L.wk = win_k;
  L.wv = win_v;
  L.wdt = win_dtype;
  L.sb = win_stride_b;
  L.sh = win_stride_h;
  L.st = win_stride_t;
  L.W = W;
  L.T = T;
  L.tf = transform;
  L.kb = kbits;
  L.vb = vbits;
  L.ks = kscale;
  L.vs = vscale;
  L.kc = kcounts;
  L.tile_stride = tile_stride;
  L.state = state;
  return hip_status(kvr::launch_append(L, (hipStream_t)stream), "kvr_cache_append");
}

int kvr_set_wait_limit(int polls, int force_give_up) {
  if (polls < 0) return fail(KVR_ERR_INVALID, "polls=%d < 0", polls);
  g_spin_max.store(polls == 0 ? (1 << 20) : polls, std::memory_order_relaxed);
  g_wait_fail.store(force_give_up ? 1 : 0, std::memory_order_relaxed);
  return KVR_OK;
}

int kvr_gather_tiles(const uint64_t* bits, const uint16_t* scales, int64_t BH, int64_t tile_stride,
                     int T, int transform, const int32_t* idx, int k, float* out,
                     int64_t out_stride_s, int64_t out_stride_t, kvr_stream_t stream) {
  if (int r = check_common(128, T)) return r;
  if (!valid_transform(transform)) return fail(KVR_ERR_INVALID, "transform %d unknown", transform);
  if (BH < 0 || k < 0) return fail(KVR_ERR_INVALID, "negative size");
  if (BH * k == 0) return KVR_OK;
  if (!bits || !scales || !idx || !out) return fail(KVR_ERR_INVALID, "NULL pointer");
  if (tile_stride <= 0) return fail(KVR_ERR_INVALID, "tile_stride must be > 0");
  if (out_stride_t < 128 || out_stride_s < 0) return fail(KVR_ERR_INVALID, "bad output strides");
  if (!aligned(bits, 8)) return fail(KVR_ERR_ALIGN, "bits must be 8-byte aligned");
  return hip_status(kvr::launch_gather(bits, scales, BH, tile_stride, T, transform, idx, k, out,
                                       out_stride_s, out_stride_t, (hipStream_t)stream),
                    "kvr_gather_tiles");
}

}  // extern "C"
