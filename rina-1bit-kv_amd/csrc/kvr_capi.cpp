// Host side of the C ABI declared in include/kvr_capi.h: argument validation
// (entirely before any HIP call, so a rejected call never touches the device),
// workspace planning, and the launch sequence of each entry point.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/kvr_capi.h"

namespace kvr {
hipError_t launch_encode(int dt, int tf, int T, const void* x, int64_t n_b, int64_t n_h,
                         int64_t n_tok, int64_t sb, int64_t sh, int64_t st, uint64_t* bits,
                         uint16_t* scales, int64_t ots, int64_t oto, float* dbg, uint8_t* counts,
                         hipStream_t s);
hipError_t launch_query_prep(int qt, int tf, const void* q, int64_t B, int Hq, int Hkv,
                             float* qbar_rot, float* q_rot, hipStream_t s);
hipError_t launch_score(int T, int method, const float* qbar_rot, const uint64_t* kbits, int64_t BH,
                        int64_t n_tiles, int64_t tile_stride, const int32_t* excl_lo,
                        const int32_t* excl_hi, float* scores, hipStream_t s);
hipError_t launch_topk(const float* scores, int64_t BH, int64_t n, int64_t stride, int k,
                       int32_t* idx, hipStream_t s);
hipError_t launch_decode(int qt, const void* q, int64_t B, int Hq, int Hkv, const void* wk,
                         const void* wv, int wdt, int64_t win_len, int64_t sb, int64_t sh, int64_t st,
                         const uint64_t* kb, const uint64_t* vb, const uint16_t* ks,
                         const uint16_t* vs, const uint8_t* kc, int64_t n_tiles, int64_t tile_stride,
                         int T, int tf, const int32_t* excl_lo, const int32_t* excl_hi, int k, bool do_select,
                         float* scores, uint64_t* cand, int32_t* idx, float* rec, int32_t* ctr,
                         void* out, int ot, hipStream_t s);
size_t records_bytes(int64_t B, int Hq, int Hkv, int64_t win_len, int k, int T);
size_t counter_bytes();
size_t cand_bytes(int64_t B, int Hkv, int64_t n_tiles, int k, int T);
hipError_t launch_gather(const uint64_t* bits, const uint16_t* scales, int64_t BH,
                         int64_t tile_stride, int T, int tf, const int32_t* idx, int k, float* out,
                         int64_t oss, int64_t ost, hipStream_t s);
}  // namespace kvr

namespace {

constexpr int kAbiVersion = 2;
constexpr int kMaxTopK = 1024;
constexpr size_t kAlign = 256;

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

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

// Window: 16-byte loads of 8 elements along head_dim.
int check_window(const void* wk, const void* wv, int wdt, int64_t win_len, int64_t sb, int64_t sh,
                 int64_t st) {
  if (win_len < 0) return fail(KVR_ERR_INVALID, "win_len=%lld < 0", (long long)win_len);
  if (win_len == 0) return KVR_OK;
  if (wdt != KVR_BF16 && wdt != KVR_FP16)
    return fail(KVR_ERR_INVALID, "window dtype %d unsupported (bf16 or fp16)", wdt);
  if (!wk || !wv) return fail(KVR_ERR_INVALID, "window pointers are NULL");
  if (!aligned(wk, 16) || !aligned(wv, 16))
    return fail(KVR_ERR_ALIGN, "window pointers must be 16-byte aligned");
  if (sb < 0 || sh < 0 || st <= 0 || sb % 8 || sh % 8 || st % 8)
    return fail(KVR_ERR_ALIGN, "window strides (b=%lld h=%lld t=%lld) must be non-negative multiples of 8 elements",
                (long long)sb, (long long)sh, (long long)st);
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

static int attn_checks(const void* q, int q_dtype, int64_t B, int Hq, int Hkv, int d,
                       const void* win_k, const void* win_v, int win_dtype, int64_t win_len,
                       int64_t sb, int64_t sh, int64_t st, const uint64_t* kbits,
                       const uint64_t* vbits, const uint16_t* kscale, const uint16_t* vscale,
                       int64_t tile_stride, int T, int transform, int k, void* out,
                       int out_dtype) {
  if (int r = check_common(d, T)) return r;
  if (int r = check_heads(B, Hq, Hkv)) return r;
  if (!valid_dtype(q_dtype)) return fail(KVR_ERR_INVALID, "q dtype %d unknown", q_dtype);
  if (!valid_transform(transform)) return fail(KVR_ERR_INVALID, "transform %d unknown", transform);
  if (out_dtype != KVR_BF16 && out_dtype != KVR_FP32)
    return fail(KVR_ERR_INVALID, "out dtype %d unsupported (bf16 or fp32)", out_dtype);
  if (k < 0 || k > kMaxTopK) return fail(KVR_ERR_INVALID, "k=%d out of [0, %d]", k, kMaxTopK);
  if (int r = check_window(win_k, win_v, win_dtype, win_len, sb, sh, st)) return r;
  if (k > 0)
    if (int r = check_store(kbits, vbits, kscale, vscale, tile_stride)) return r;
  if (B > 0 && (!q || !out)) return fail(KVR_ERR_INVALID, "q and out must be non-NULL");
  if (B > 0 && !aligned(q, 16)) return fail(KVR_ERR_ALIGN, "q must be 16-byte aligned");
  if (B > 0 && !aligned(out, 8)) return fail(KVR_ERR_ALIGN, "out must be 8-byte aligned");
  return KVR_OK;
}

int kvr_decode_attn(const void* q, int q_dtype, int64_t B, int Hq, int Hkv, int d,
                    const void* win_k, const void* win_v, int win_dtype, int64_t win_len,
                    int64_t win_stride_b, int64_t win_stride_h, int64_t win_stride_t,
                    const uint64_t* kbits, const uint64_t* vbits, const uint16_t* kscale,
                    const uint16_t* vscale, int64_t tile_stride, int T, int transform,
                    const int32_t* idx, int k, void* out, int out_dtype, void* workspace,
                    size_t ws_bytes, kvr_stream_t stream) {
  if (int r = attn_checks(q, q_dtype, B, Hq, Hkv, d, win_k, win_v, win_dtype, win_len,
                          win_stride_b, win_stride_h, win_stride_t, kbits, vbits, kscale, vscale,
                          tile_stride, T, transform, k, out, out_dtype))
    return r;
  if (k > 0 && !idx) return fail(KVR_ERR_INVALID, "idx must be non-NULL when k > 0");
  if (B == 0) return KVR_OK;
  const StepLayout L = step_layout(B, Hq, Hkv, win_len, 0, k, T);
  if (!workspace || ws_bytes < L.total)
    return fail(KVR_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", L.total,
                workspace ? ws_bytes : (size_t)0);
  if (!aligned(workspace, kAlign)) return fail(KVR_ERR_ALIGN, "workspace must be 256-byte aligned");
  char* ws = (char*)workspace;
  return hip_status(kvr::launch_decode(q_dtype, q, B, Hq, Hkv, win_k, win_v, win_dtype, win_len,
                                       win_stride_b, win_stride_h, win_stride_t, kbits, vbits,
                                       kscale, vscale, nullptr, 0, tile_stride, T, transform, nullptr, nullptr,
                                       k, false, nullptr, nullptr, const_cast<int32_t*>(idx),
                                       (float*)(ws + L.rec), nullptr, out, out_dtype,
                                       (hipStream_t)stream),
                    "kvr_decode_attn");
}

size_t kvr_decode_step_workspace(int64_t B, int Hq, int Hkv, int64_t win_len, int64_t n_tiles,
                                 int k, int T) {
  if (B < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || n_tiles < 0 || (T != 64 && T != 128)) return 0;
  if (n_tiles == 0) k = 0;
  return step_layout(B, Hq, Hkv, win_len, k > 0 ? n_tiles : 0, k, T).total;
}

int kvr_decode_step(const void* q, int q_dtype, int64_t B, int Hq, int Hkv, int d,
                    const void* win_k, const void* win_v, int win_dtype, int64_t win_len,
                    int64_t win_stride_b, int64_t win_stride_h, int64_t win_stride_t,
                    const uint64_t* kbits, const uint64_t* vbits, const uint16_t* kscale,
                    const uint16_t* vscale, const uint8_t* kcounts, int64_t n_tiles,
                    int64_t tile_stride, int T, int transform, const int32_t* excl_lo,
                    const int32_t* excl_hi, int k, void* out, int out_dtype, int32_t* idx_out,
                    void* workspace, size_t ws_bytes, kvr_stream_t stream) {
  if (n_tiles < 0) return fail(KVR_ERR_INVALID, "n_tiles < 0");
  if (n_tiles == 0) k = 0;
  if (k > n_tiles) return fail(KVR_ERR_INVALID, "k=%d > n_tiles=%lld", k, (long long)n_tiles);
  if (k > 0 && tile_stride < n_tiles) return fail(KVR_ERR_INVALID, "tile_stride < n_tiles");
  if (int r = attn_checks(q, q_dtype, B, Hq, Hkv, d, win_k, win_v, win_dtype, win_len,
                          win_stride_b, win_stride_h, win_stride_t, kbits, vbits, kscale, vscale,
                          tile_stride, T, transform, k, out, out_dtype))
    return r;
  if ((excl_lo == nullptr) != (excl_hi == nullptr))
    return fail(KVR_ERR_INVALID, "excl_lo and excl_hi must both be given or both NULL");
  if (kcounts && !aligned(kcounts, 8)) return fail(KVR_ERR_ALIGN, "kcounts must be 8-byte aligned");
  if (B == 0) return KVR_OK;
  const int64_t nt = (k > 0) ? n_tiles : 0;
  const StepLayout L = step_layout(B, Hq, Hkv, win_len, nt, k, T);
  if (!workspace || ws_bytes < L.total)
    return fail(KVR_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", L.total,
                workspace ? ws_bytes : (size_t)0);
  if (!aligned(workspace, kAlign)) return fail(KVR_ERR_ALIGN, "workspace must be 256-byte aligned");
  char* ws = (char*)workspace;
  int32_t* idx = idx_out ? idx_out : (int32_t*)(ws + L.idx);
  return hip_status(kvr::launch_decode(q_dtype, q, B, Hq, Hkv, win_k, win_v, win_dtype, win_len,
                                       win_stride_b, win_stride_h, win_stride_t, kbits, vbits,
                                       kscale, vscale, kcounts, n_tiles, tile_stride, T, transform,
                                       excl_lo, excl_hi, k, true, (float*)(ws + L.scores),
                                       (uint64_t*)(ws + L.cand), idx,
                                       (float*)(ws + L.rec), (int32_t*)(ws + L.ctr), out,
                                       out_dtype, (hipStream_t)stream),
                    "kvr_decode_step");
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
