// Host-side interface between the C ABI (kvr_capi.cpp, kvr_noalloc.hip) and the
// kernel launchers (kvr_encode.hip, kvr_decode.hip).  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace kvr {

// Everything one decode launch sequence needs (validated by the caller).
struct DecodeLaunch {
  int qt;                 // query dtype
  const void* q;
  int64_t B;
  int Hq, Hkv;
  const void* wk;         // window K, V
  const void* wv;
  int wdt;                // window dtype
  int64_t win_len;        // valid window tokens (the capacity when live is given)
  int64_t win_start;      // ring start slot (ignored when live is given)
  int64_t win_cap;        // ring capacity in slots (0: no ring)
  int64_t sb, sh, st;     // window strides (elements)
  const uint64_t* kb;
  const uint64_t* vb;
  const uint16_t* ks;
  const uint16_t* vs;
  const uint8_t* kc;      // K channel counts (nullable)
  int64_t n_tiles;        // stored tiles (the capacity when live is given)
  int64_t tile_stride;
  int T, tf;
  const int32_t* excl_lo;
  const int32_t* excl_hi;
  int k;
  const int32_t* live;    // per segment {win_len, win_start, n_tiles, -} (nullable)
  bool do_select;
  float* scores;
  uint64_t* cand;
  int32_t* idx;
  float* rec;
  int32_t* ctr;
  void* out;
  int ot;                 // out dtype
  int spin_max;           // polls of a bounded wait before it gives up
  int wait_fail;          // test hook: make the bounded waits give up
};

hipError_t launch_decode(const DecodeLaunch& L, hipStream_t s);
bool step_is_fused(int64_t BH, int k, bool have_ctr);
size_t records_bytes(int64_t B, int Hq, int Hkv, int64_t win_len, int k, int T);
size_t counter_bytes();
size_t cand_bytes(int64_t B, int Hkv, int64_t n_tiles, int k, int T);

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
hipError_t launch_gather(const uint64_t* bits, const uint16_t* scales, int64_t BH,
                         int64_t tile_stride, int T, int tf, const int32_t* idx, int k, float* out,
                         int64_t oss, int64_t ost, hipStream_t s);

// One token per segment into a ring window, encoding the oldest T tokens into the next
// tile slot when the ring is full (see kvr_cache_append in kvr_capi.h).
struct AppendLaunch {
  const void* k_new;
  const void* v_new;
  int ndt;                // dtype of k_new / v_new
  int64_t B;
  int Hkv;
  void* wk;
  void* wv;
  int wdt;
  int64_t sb, sh, st;
  int64_t W;              // window tokens kept after an eviction; the ring holds W + T slots
  int T, tf;
  uint64_t* kb;
  uint64_t* vb;
  uint16_t* ks;
  uint16_t* vs;
  uint8_t* kc;            // nullable
  int64_t tile_stride;
  int32_t* state;         // per segment {n, start, n_tiles, error}
};
hipError_t launch_append(const AppendLaunch& L, hipStream_t s);

// Decode-step entry point shared by kvr_decode_step and the allocation-free variant:
// validates, lays out the workspace and launches (launch == false: validation only, the
// workspace pointer unchecked and only ws_bytes compared with the need).
int decode_step_impl(const void* q, int q_dtype, int64_t B, int Hq, int Hkv, int d,
                     const void* win_k, const void* win_v, int win_dtype, int64_t win_len,
                     int64_t win_start, int64_t win_cap, int64_t win_stride_b, int64_t win_stride_h,
                     int64_t win_stride_t, const uint64_t* kbits, const uint64_t* vbits,
                     const uint16_t* kscale, const uint16_t* vscale, const uint8_t* kcounts,
                     int64_t n_tiles, int64_t tile_stride, int T, int transform,
                     const int32_t* excl_lo, const int32_t* excl_hi, int k, const int32_t* live_state,
                     void* out, int out_dtype, int32_t* idx_out, void* workspace, size_t ws_bytes,
                     hipStream_t stream, bool launch = true);
// Workspace bytes decode_step_impl needs (0 for invalid sizes).
size_t decode_step_workspace_bytes(int64_t B, int Hq, int Hkv, int64_t win_len, int64_t n_tiles, int k, int T);
// Sets the thread-local error message; returns code.
int set_error(int code, const char* fmt, ...);

}  // namespace kvr
