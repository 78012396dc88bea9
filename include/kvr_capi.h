/*
 * kvr_capi.h -- C ABI of the MI355X (gfx950) compressed-KV decode hot path.
 *
 * Every entry point takes plain device pointers, sizes and strides (no torch
 * types), validates its arguments on the host, launches asynchronously on
 * `stream` (NULL = the default stream) and returns KVR_OK (0) or a negative
 * kvr_status.  On error nothing is launched and kvr_last_error() holds a
 * thread-local message.  The library never synchronises; all buffers belong
 * to the caller.  head_dim d must be 128; tiles hold T in {64, 128} tokens.
 *
 * Store layout (per layer): a "segment" is one (sequence, KV head).
 *   bits   : uint64 [n_seg][tile_stride][128][T/64]; bit (t mod 64) of word
 *            t/64 is the sigma-delta bit of token t of that channel.
 *   scales : fp16 bit patterns [n_seg][tile_stride], one per tile, K and V
 *            in separate arrays.
 *   window : bf16, fp16 or fp32 [.. strides ..][slots][128], the exact recent
 *            tokens (a plain run of slots, or a ring).
 *
 * Reference interfaces replaced (paths relative to Misaka477/RINA-1bit-KV):
 *   see the comment above each function.
 */
#ifndef KVR_CAPI_H
#define KVR_CAPI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* kvr_stream_t; /* == hipStream_t */

enum kvr_status {
  KVR_OK = 0,
  KVR_ERR_INVALID = -1,     /* bad size, dtype, transform, pointer or stride */
  KVR_ERR_ALIGN = -2,       /* pointer not aligned as the kernel requires    */
  KVR_ERR_WORKSPACE = -3,   /* workspace missing or too small                */
  KVR_ERR_HIP = -4,         /* a HIP launch failed                           */
  KVR_ERR_UNSUPPORTED = -5  /* valid request outside what is built (g > 16, ...) */
};

enum kvr_dtype { KVR_BF16 = 0, KVR_FP16 = 1, KVR_FP32 = 2 };
enum kvr_transform { KVR_HADAMARD = 0, KVR_DCT = 1, KVR_NONE = 2 };

/* ABI version of this header (bumped on any signature change; 3 added the ring
 * window, the live state, kvr_cache_append and kvr_set_wait_limit; 4 the tile-store
 * format functions of kvr_store.h). */
int kvr_abi_version(void);

/* Thread-local description of the last error returned on this thread. */
const char* kvr_last_error(void);

/*
 * Encode n_tok tokens (a multiple of T) of n_b*n_h segments into 1-bit tiles:
 * rotation along head_dim (Hadamard-128, DCT-II-128, or NONE for input that is
 * already rotated fp32), per-tile fp16 scale, sigma-delta along tokens, packing.
 * Input element (b, h, t, j) is at x[b*stride_b + h*stride_h + t*stride_t + j]
 * (strides in elements, channel stride 1).  Segment b*n_h+h writes its tiles to
 * tile slots [out_tile_offset, out_tile_offset + n_tok/T) of a store whose
 * segment pitch is out_tile_stride tiles.  dbg_rotated (nullable) receives the
 * fp32 rotated input, [n_b*n_h][n_tok][128].  counts (nullable; same tile slots,
 * [segment][tile][128] uint8) receives each channel's number of set bits over the
 * tile's T tokens -- the tile's column sums are 2*count - T, all a tile score reads
 * (the per-tile chunk summary kvr_decode_step scores from when it is given).
 * Replaces: RetrievalIndex.batch_append / append / _pack_int4 / _pack_int2
 *           (modules/kvr_retrieval.py:187-207, 162-185, 69-91).
 */
int kvr_encode_tiles(const void* x, int x_dtype, int64_t n_b, int64_t n_h, int64_t n_tok,
                     int64_t stride_b, int64_t stride_h, int64_t stride_t, int d, int T,
                     int transform, uint64_t* bits, uint16_t* scales, int64_t out_tile_stride,
                     int64_t out_tile_offset, float* dbg_rotated, uint8_t* counts,
                     kvr_stream_t stream);

/*
 * Query preparation for B sequences: qbar_rot[b*Hkv+h] = R * mean over the g =
 * Hq/Hkv query heads of group h (fp32 sum in head order, then /g), and, when
 * q_rot is non-NULL, q_rot[b*Hq+i] = R * q[b, i].  q is [B][Hq][128].
 * Replaces: the GQA mean of compute_all_scores / compute_chunk_scores
 *           (modules/kvr_retrieval.py:270, 296).
 */
int kvr_query_prep(const void* q, int q_dtype, int64_t B, int Hq, int Hkv, int d, int transform,
                   float* qbar_rot, float* q_rot, kvr_stream_t stream);

/*
 * Cosine score of qbar_rot[s] (fp32 [BH][128]) against the column sums of each
 * of the first n_tiles tiles of segment s: c_j = 2*popcount - T.  Tiles
 * [excl_lo[s], excl_hi[s]) score -inf (both arrays nullable, tile units).
 * scores: fp32 [BH][n_tiles].  method 0 = popcount, 1 = bit-unpack (same
 * result, different instruction mix).
 * Replaces: compute_scores (modules/kvr_cuda.cu:53-77), run_score_kernel
 *           (modules/kvr_triton.py:82-91), compute_chunk_scores
 *           (modules/kvr_retrieval.py:291-315).
 */
int kvr_score_tiles(const float* qbar_rot, const uint64_t* kbits, int64_t BH, int64_t n_tiles,
                    int64_t tile_stride, int d, int T, const int32_t* excl_lo,
                    const int32_t* excl_hi, int method, float* scores, kvr_stream_t stream);

/*
 * Per-row top-k of scores ([BH] rows of n_tiles, row pitch score_stride):
 * idx[s][0..k) = tile indices by score descending, ties by index ascending
 * (NaN counts as -inf).  1 <= k <= min(n_tiles, 1024).
 * Replaces: torch.topk in RetrievalIndex.retrieve_topk
 *           (modules/kvr_retrieval.py:379, 392).
 */
int kvr_topk_tiles(const float* scores, int64_t BH, int64_t n_tiles, int64_t score_stride, int k,
                   int32_t* idx, kvr_stream_t stream);

/* Workspace bytes kvr_decode_attn needs for these sizes.  A decode workspace (either
 * entry point) must be zeroed before its first call and is then reused across calls;
 * it begins with a 1,048,832-byte counter region the calls keep from one call to the
 * next, the rest is scratch.  The int32 at byte offset 0 is the workspace's sticky
 * STATUS word: nonzero once a bounded wait inside a decode step gave up (that call's
 * affected outputs are NaN); every call since the workspace was zeroed is then
 * suspect, and the workspace must be zeroed again before further use.  Calls that
 * run concurrently need their own workspaces. */
size_t kvr_decode_attn_workspace(int64_t B, int Hq, int Hkv, int64_t win_len, int k, int T);

/*
 * Decode attention for one query token per sequence: one softmax over the
 * win_len window tokens and the k*T tokens of tiles idx[s][0..k), with logits
 * scaled by 1/sqrt(128).  Retrieved keys/values are s*(2b-1) in the rotated
 * domain; their output is rotated back.  q: [B][Hq][128] (bf16, fp16 or fp32);
 * window slot element (b, h, t, j) at win[b*win_stride_b + h*win_stride_h +
 * t*win_stride_t + j] (bf16, fp16 or fp32); the window's tokens are slots
 * [0, win_len), or, for a ring (win_cap > 0), slots (win_start + i) mod win_cap,
 * i < win_len.  out: [B][Hq][128] in out_dtype (bf16 or fp32).
 * 1 <= Hq/Hkv <= 16.  win_len == 0 or k == 0 disables that part.
 * Replaces: run_fused_attn (modules/kvr_triton.py:94-104), WindowBuffer.attention
 *           (modules/kvr_window.py:43-69) and the attention merge of the hook
 *           (modules/kvr_hook.py:274-282).
 */
int kvr_decode_attn(const void* q, int q_dtype, int64_t B, int Hq, int Hkv, int d,
                    const void* win_k, const void* win_v, int win_dtype, int64_t win_len,
                    int64_t win_start, int64_t win_cap, int64_t win_stride_b, int64_t win_stride_h,
                    int64_t win_stride_t, const uint64_t* kbits, const uint64_t* vbits,
                    const uint16_t* kscale, const uint16_t* vscale, int64_t tile_stride, int T,
                    int transform, const int32_t* idx, int k, void* out, int out_dtype,
                    void* workspace, size_t ws_bytes, kvr_stream_t stream);

/* Workspace bytes kvr_decode_step needs for these sizes (zeroed before first use, as
 * above; with a live state pass the capacities). */
size_t kvr_decode_step_workspace(int64_t B, int Hq, int Hkv, int64_t win_len, int64_t n_tiles,
                                 int k, int T);

/*
 * The whole decode hot path for one layer: query prep, tile scoring over the
 * first n_tiles tiles (with optional per-segment exclusion), top-k, and the
 * fused window + retrieved-tile attention (window as in kvr_decode_attn).
 * idx_out (nullable, [BH][k] int32) receives the selected tiles.  k == 0 or
 * n_tiles == 0 attends the window only.  kcounts (nullable): the K store's
 * per-tile channel counts written by kvr_encode_tiles (same tile slots); when
 * given, tiles are scored from them (128 bytes per tile instead of the tile's
 * bits; the same scores bit for bit).
 * live_state (nullable, int32 [B*Hkv][4] on the device, 16-byte aligned): each
 * segment's {window length, ring start, tile count, -} as kvr_cache_append keeps
 * them, read by the kernel, so one captured launch serves every decode step;
 * win_len and n_tiles are then the capacities the launch is sized for (a live
 * count above them is clamped), win_start is ignored and win_cap must be the
 * ring's.  A live state needs the one-launch step (1 <= k <= 64, B*Hkv <= 4096);
 * with fewer live tiles than k every stored tile is taken (idx -1 past them).
 * Replaces: RetrievalIndex.retrieve_topk + the hook's merge
 *           (modules/kvr_retrieval.py:317-412, modules/kvr_hook.py:253-282)
 *           and KVRGenerator.step's attention (modules/kvr_generator.py:100-119).
 */
int kvr_decode_step(const void* q, int q_dtype, int64_t B, int Hq, int Hkv, int d,
                    const void* win_k, const void* win_v, int win_dtype, int64_t win_len,
                    int64_t win_start, int64_t win_cap, int64_t win_stride_b, int64_t win_stride_h,
                    int64_t win_stride_t, const uint64_t* kbits, const uint64_t* vbits,
                    const uint16_t* kscale, const uint16_t* vscale, const uint8_t* kcounts,
                    int64_t n_tiles, int64_t tile_stride, int T, int transform,
                    const int32_t* excl_lo, const int32_t* excl_hi, int k,
                    const int32_t* live_state, void* out, int out_dtype, int32_t* idx_out,
                    void* workspace, size_t ws_bytes, kvr_stream_t stream);

/* Scratch the allocation-free decode step holds per GPU (bytes). */
#define KVR_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)

/*
 * kvr_decode_step without a workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Same arguments (minus workspace, ws_bytes), semantics and
 * results as kvr_decode_step; its scratch is a KVR_NOALLOC_SCRATCH_BYTES device array
 * of the library, one per GPU, held until the process ends, zeroed on the first call
 * on each device (which must not be under graph capture).  Sizes whose workspace
 * (kvr_decode_step_workspace) exceeds it are rejected with KVR_ERR_WORKSPACE.  The
 * function calls no hipMalloc / hipFree.  Calls that overlap on one GPU share that
 * scratch and race: the caller serialises them.
 * Replaces: nothing in the reference -- an addition for the callers that cannot
 *           allocate (see above).
 */
int kvr_decode_step_noalloc(const void* q, int q_dtype, int64_t B, int Hq, int Hkv, int d,
                            const void* win_k, const void* win_v, int win_dtype, int64_t win_len,
                            int64_t win_start, int64_t win_cap, int64_t win_stride_b,
                            int64_t win_stride_h, int64_t win_stride_t, const uint64_t* kbits,
                            const uint64_t* vbits, const uint16_t* kscale, const uint16_t* vscale,
                            const uint8_t* kcounts, int64_t n_tiles, int64_t tile_stride, int T,
                            int transform, const int32_t* excl_lo, const int32_t* excl_hi, int k,
                            const int32_t* live_state, void* out, int out_dtype, int32_t* idx_out,
                            kvr_stream_t stream);

/*
 * Append one token per segment to a per-layer cache: a ring window of W + T slots
 * (window layout as in kvr_decode_attn, any of bf16 / fp16 / fp32) plus the
 * K / V tile stores (and, nullable, the K channel counts).  k_new, v_new:
 * [B][Hkv][128] in new_dtype (post-RoPE K), converted to the window dtype (RNE).
 * state: int32 [B*Hkv][4] on the device, per segment {n, start, n_tiles, error}:
 * the window holds n tokens from ring slot start on (W <= n < W + T once the
 * store is non-empty) and the store n_tiles tiles.  When the new token fills the
 * ring (n + 1 == W + T) its oldest T tokens are encoded into tile slot n_tiles
 * (same bits as kvr_encode_tiles on them), start advances by T and n drops to W.
 * error (sticky): 1 = the state was invalid (nothing written), 2 = the store was
 * full (tile_stride tiles; the evicted tokens were dropped).  W must be a
 * positive multiple of T.  Everything happens on the device, so the call can be
 * captured in a graph.
 * Replaces: KVRHook._update_stores (modules/kvr_hook.py:136-148) with
 *           WindowBuffer.append (modules/kvr_window.py:19-25) and
 *           RetrievalIndex.append (modules/kvr_retrieval.py:162-185).
 */
int kvr_cache_append(const void* k_new, const void* v_new, int new_dtype, int64_t B, int Hkv, int d,
                     void* win_k, void* win_v, int win_dtype, int64_t win_stride_b,
                     int64_t win_stride_h, int64_t win_stride_t, int64_t W, int T, int transform,
                     uint64_t* kbits, uint64_t* vbits, uint16_t* kscale, uint16_t* vscale,
                     uint8_t* kcounts, int64_t tile_stride, int32_t* state, kvr_stream_t stream);

/*
 * Bounded waits of later decode launches (process-wide): polls before a wait
 * gives up (0 restores the default, 2^20), and a diagnostic switch that makes
 * every wait of the one-launch step expect a tag no candidate list carries, so
 * it gives up after `polls` polls -- for tests of the failure path (status word,
 * NaN outputs) in which every kernel still ends normally.
 * Replaces: nothing in the reference (its fallbacks are silent,
 *           modules/kvr_retrieval.py:13-24); a testing and diagnostic hook.
 */
int kvr_set_wait_limit(int polls, int force_give_up);

/*
 * Materialise the tokens of the selected tiles in the original (unrotated)
 * domain: out[s*out_stride_s + (i*T + t)*out_stride_t + j] = (R^T x)_j with
 * x = scale*(2b-1), fp32.  idx: [BH][k].
 * Replaces: the gather / V reconstruction of retrieve_topk
 *           (modules/kvr_retrieval.py:394-412).
 */
int kvr_gather_tiles(const uint64_t* bits, const uint16_t* scales, int64_t BH, int64_t tile_stride,
                     int T, int transform, const int32_t* idx, int k, float* out,
                     int64_t out_stride_s, int64_t out_stride_t, kvr_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* KVR_CAPI_H */
