// Subsystems 2-4 of the compressed-KV decode path on gfx950: query preparation,
// tile scoring, top-k tile selection, fused window + retrieved-tile attention,
// the log-sum-exp merge, and the materialising tile gather.
//
// The selecting decode step (kvr_decode_step with k <= 64) is ONE launch,
// step_kernel, whose blocks are its work items in block order (segment = sequence x
// KV head):
//   score items     : one per (segment, 128 tiles at T = 64 / 64 at T = 128); the
//                     block loads the tiles' channel counts (or bits), rotates the
//                     segment's GQA-mean query meanwhile, and stores its tiles sorted
//                     by (score desc, tile asc) as a self-validating candidate list.
//   retrieved items : merge the segment's candidate lists into the top k (reloading
//                     until every entry carries this call's tag), then attend 8 (T = 64)
//                     or 4 (T = 128) selected tiles on MFMA with +-1 operands.
//   window items    : up to 512 exact window tokens each (MFMA; K into registers, V
//                     rows straight into LDS by direct loads, software-pipelined).
// Retrieved and window items write partial softmax records and count them into their
// segment; the item that brings the count to the segment's total merges the segment
// (log-sum-exp, inverse rotation of the retrieved part) and writes the output.  Blocks
// therefore do wait for other blocks inside the launch (retrieved items for score
// items); why every such wait ends is stated above step_kernel.
// The other entry points (given indices, k > 64, the VALU retrieval variant) run the
// same roles as a launch chain without cross-block waits: select_score_kernel ->
// attend_kernel -> merge_kernel.
//
// Partial records: per segment s and part p, g*(2+128) floats: m2[g] (running max,
// log2 units), l[g], o[g][128]; the retrieved parts first, then the window parts.
// Window parts hold o in the original domain, retrieved parts in the rotated domain
// (rotated back once per head in the merge).
// The window may be a ring (win_cap > 0): logical token i of the win_len valid ones is
// in slot (win_start + i) mod win_cap.  With a live state (decode step only) the
// window length, ring start and tile count are read per segment from device memory,
// and the launch's grid covers the capacities the host passed.
//
// Reference behaviour followed (Misaka477/RINA-1bit-KV):
//   GQA mean query          modules/kvr_retrieval.py:270, 296
//   chunk-mean cosine score modules/kvr_retrieval.py:291-315 (+1e-8 on both norms)
//   NaN -> -inf, exclusion  modules/kvr_retrieval.py:287-288, 373-377, 391
//   per-KV-head top-k       modules/kvr_retrieval.py:379, 392
//   joint softmax, 1/sqrt(d) modules/kvr_hook.py:274-282; online form of
//                            modules/kvr_triton.py:56-79
#include <cstdlib>

#include "kvr_common.h"
#include "kvr_internal.h"

namespace kvr {

constexpr int NT = 256;           // threads per block (4 waves) for every decode role
// Build-time tuning (defaults are the measured best on MI355X): waves per SIMD the
// attend kernel is compiled for (sets its VGPR budget), the number of window items
// below which window spans stay at one chunk per wave, and the selected tiles per
// retrieved item.
#ifndef KVR_ATTEND_WAVES
#define KVR_ATTEND_WAVES 3
#endif
#ifndef KVR_WIN_MIN_ITEMS
#define KVR_WIN_MIN_ITEMS 256
#endif
#ifndef KVR_MERGE_PB
#define KVR_MERGE_PB 3  // parts per wave in the parts-split merge (g in 5..8, n_parts <= 4 KVR_MERGE_PB): one
                        // load batch of 8 heads x KVR_MERGE_PB parts stays clear of spills
#endif
#ifndef KVR_WIN_MAX_PARTS
#define KVR_WIN_MAX_PARTS 4  // window items per segment (at most, spans allowing) when tiles are retrieved
#endif
#ifndef KVR_CAND_MAX
#define KVR_CAND_MAX 64  // k up to which score items write sorted candidate lists (0: never)
#endif
#ifndef KVR_RET_FIRST
#define KVR_RET_FIRST 1  // 1: all retrieved items first in the attend grid, else per segment
#endif
#ifndef KVR_FUSED_STEP
#define KVR_FUSED_STEP 1  // 1: the selecting step runs as one launch (step_kernel)
#endif
#ifndef KVR_STEP_ORDER
// step_kernel block order after the score items: 0 all window items, then all retrieved
// items; 1 the reverse; 2 per segment its window items, then its retrieved items
#define KVR_STEP_ORDER 1
#endif
#ifndef KVR_SCORE_TPG
#define KVR_SCORE_TPG 8  // tiles per 16-lane group of a score item at T = 64: 4, 6 or 8
#endif
#ifndef KVR_SCORE_TPG128  // the same at T = 128 (two words per channel)
#define KVR_SCORE_TPG128 4
#endif
#ifndef KVR_CTR_STRIDE
#define KVR_CTR_STRIDE 32  // int32 words between per-segment counters (32: a 128-byte line each)
#endif
#ifndef KVR_RET_PARTS
#define KVR_RET_PARTS 2  // fp16 parts of the retrieved MFMA operands q' and sv*P
#endif
#ifndef KVR_RET_PRIO
#define KVR_RET_PRIO 2  // wave issue priority of retrieved items: 0 none, 1 whole role, 2 tile loop
#endif
#ifndef KVR_RET_TILES
#define KVR_RET_TILES 8  // selected tiles per retrieved item (a multiple of 4: one per wave per round)
#endif

// Segments (B * Hkv) up to which the selecting step runs as one launch; the counter
// region at the start of every decode workspace holds their counters.
constexpr int STEP_MAX_SEG = 4096;
constexpr int CTR_ERR_WORD = 0;  // counter-region word set when a bounded wait gives up (sticky)
constexpr int WIN_CHUNK = 32;     // window tokens per wave per step
constexpr int WIN_UNIT = 4 * WIN_CHUNK;  // window items span a multiple of this
constexpr int TOPK_MAX_K = 1024;
constexpr float SCALE_LOG2 = 0.08838834764831845f * LOG2E;  // log2(e) / sqrt(128)

struct DecodeArgs {
  const void* q;
  int q_dtype, Hq, Hkv, g, transform, out_dtype;
  const void* wk;     // window K, V (bf16 / fp16 / fp32 as the role's template says)
  const void* wv;
  int64_t win_len, sb, sh, st;
  int64_t win_start, win_cap;  // ring: token i of the window is in slot (win_start + i) mod win_cap (0: no ring)
  const int32_t* live;  // per segment {win_len, win_start, n_tiles, -} on the device (step only; nullable)
  int n_chunks_cap, n_wparts_cap;  // grid decomposition (the capacities when live is given)
  int spin_max;       // polls of a bounded wait before it gives up
  int wait_fail;      // test hook: waits expect a tag no list carries, so they give up
  const uint64_t* kbits;
  const uint64_t* vbits;
  const uint16_t* kscale;
  const uint16_t* vscale;
  const uint8_t* kcount;  // per-tile channel counts of the K store (nullable: score from the bits)
  int64_t n_tiles, tile_stride;
  const int32_t* excl_lo;
  const int32_t* excl_hi;
  int k;
  float* scores;      // [BH][n_tiles]
  uint64_t* cand;     // [BH][n_chunks][64] per-item candidates, sorted (k <= 64), or null
  int32_t* idx;       // [BH][k]
  float* rec;         // [BH][n_parts][g][2+D]
  int32_t* ctr;       // fused step: work-queue header + per-segment counters (see step_kernel), or null
  int64_t n_seg;      // B * Hkv
  int n_chunks, n_wparts, n_rparts;
  int64_t win_span;   // window tokens per window item
  int do_select;      // retrieved items select their tiles from scores (else read idx)
  int ret_method;     // retrieved tiles: 0 = MFMA on unpacked +-1 operands, 1 = VALU nibble tables
  void* out;          // [B][Hq][D]
};

// ------------------------------------------------------------------ small helpers

// Materialise a loaded value here: keeps the compiler from sinking a load into the
// branch that uses it (which would serialise loads meant to be in flight together).
__device__ __forceinline__ void pin(float& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void pin(uint32_t& x) { asm volatile("" : "+v"(x)); }

// Query loads without conversion: the raw bits are pinned once after all loads of a
// batch, then converted.  An element pair (even offset) is one 32-bit word for 16-bit
// dtypes, two for fp32.  QT is the query dtype when the kernel knows it (straight-line
// loads, so the compiler's wait before the first use counts exactly the loads issued
// after them), or Q_RUNTIME (a.q_dtype; each load sits in a dtype branch, and the
// compiler then waits for every outstanding load before the first use).
constexpr int Q_RUNTIME = -1;
template <int QT = Q_RUNTIME>
__device__ __forceinline__ void q_pair_raw(const DecodeArgs& a, int64_t off, uint32_t& r0, uint32_t& r1) {
  const int qt = (QT == Q_RUNTIME) ? a.q_dtype : QT;
  if (qt == KVR_FP32) {
    const uint2 u = *(const uint2*)((const float*)a.q + off);
    r0 = u.x;
    r1 = u.y;
  } else {
    r0 = *(const uint32_t*)((const uint16_t*)a.q + off);
    r1 = 0u;
  }
}
template <int QT = Q_RUNTIME>
__device__ __forceinline__ void q_pair_cvt(const DecodeArgs& a, uint32_t r0, uint32_t r1, float& v0, float& v1) {
  const int qt = (QT == Q_RUNTIME) ? a.q_dtype : QT;
  if (qt == KVR_FP32) {
    v0 = __uint_as_float(r0);
    v1 = __uint_as_float(r1);
  } else if (qt == KVR_BF16) {
    v0 = __uint_as_float(r0 << 16);
    v1 = __uint_as_float(r0 & 0xffff0000u);
  } else {
    v0 = f16_to_f32((uint16_t)(r0 & 0xffffu));
    v1 = f16_to_f32((uint16_t)(r0 >> 16));
  }
}

// 2^x by the hardware v_exp_f32 (exact at 0 and -inf -> 0; results below the fp32
// normal range flush to 0, immaterial inside a softmax).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// LDS in-order completion within one wave (no block barrier).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  __builtin_amdgcn_wave_barrier();
}

// Data handed from one block to another inside a launch (candidate lists, partial
// records) is stored and loaded at agent scope: the stores write through to the
// device-coherent level, so a block on another XCD reads it without an L2 write-back
// or invalidate (agent-scope fences, which do those, cost far more than the data).
__device__ __forceinline__ void rec_store(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float rec_load(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void cand_store(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t cand_load(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Candidate lists validate themselves: an entry is stored as two 8-byte halves, the low
// half carrying the low 32 bits of a 64-bit tag of (epoch, segment, list) in its high
// word and the high half the tag's high 32 bits, so a reader that finds the expected
// tag halves in both words has this call's entry of that list, whenever it reads -- no
// completion wait and counter on the writer's side, no poll before the read.  The tag
// is the injective packing epoch << 32 | segment | list << 20 | 1 << 31 (segment <
// 2^20, list < 2^11), so an entry of any other (epoch, segment, list) -- an earlier
// call, another workspace layout -- never validates, and zeroed memory never does
// either (bit 31 is set).  The high half, which a waiting reader polls, is the epoch:
// the previous call's list in the same slot fails the poll.  The epoch is per segment
// (fused step: the segment's epoch word + 1, advanced by the segment's merging item) or
// CAND_EPOCH_CHAIN when the lists are written by an earlier launch.
constexpr uint32_t CAND_EPOCH_CHAIN = 0xffffffffu;
constexpr uint32_t WAIT_FAIL_EPOCH = 0x5bd1e995u;  // xor-ed into the expected epoch by the wait_fail hook
__device__ __forceinline__ uint64_t cand_tag(uint32_t epoch, int64_t seg, int list) {
  return ((uint64_t)epoch << 32) | ((uint32_t)seg & 0xfffffu) | (((uint32_t)list & 0x7ffu) << 20) | (1u << 31);
}
__device__ __forceinline__ void cand_put(uint64_t* list, int e, uint64_t v, uint64_t tag) {
  cand_store(list + 2 * e, (tag << 32) | (v & 0xffffffffull));
  cand_store(list + 2 * e + 1, (tag & 0xffffffff00000000ull) | (v >> 32));
}
__device__ __forceinline__ uint64_t cand_get(const uint64_t* list, int e, uint64_t tag, bool& ok) {
  const uint64_t lo = cand_load(list + 2 * e), hi = cand_load(list + 2 * e + 1);
  ok = ok && (uint32_t)(lo >> 32) == (uint32_t)tag && (uint32_t)(hi >> 32) == (uint32_t)(tag >> 32);
  return (hi << 32) | (lo & 0xffffffffull);
}

__device__ __forceinline__ void rotate_pair(float& v0, float& v1, int lane, int tf, float* xs) {
  if (tf == KVR_HADAMARD) hadamard_pair(v0, v1, lane);
  else if (tf == KVR_DCT) dct_pair(v0, v1, lane, xs);
}

__device__ __forceinline__ void unrotate_pair(float& v0, float& v1, int lane, int tf, float* xs) {
  if (tf == KVR_HADAMARD) hadamard_pair(v0, v1, lane);  // orthonormal and symmetric
  else if (tf == KVR_DCT) idct_pair(v0, v1, lane, xs);
}

// Rotated GQA-mean query of one segment into qs[128] (one wave; lane = channels
// 2*lane, 2*lane+1).  fp32 sum in head order, one correctly rounded division.
// Two consecutive query elements (even offset) by one 4- or 8-byte load.
__device__ __forceinline__ void q_pair(const DecodeArgs& a, int64_t off, float& v0, float& v1) {
  if (a.q_dtype == KVR_FP32) {
    const float2 u = *(const float2*)((const float*)a.q + off);
    v0 = u.x;
    v1 = u.y;
  } else {
    const uint32_t r = *(const uint32_t*)((const uint16_t*)a.q + off);
    const uint16_t lo = (uint16_t)(r & 0xffffu), hi = (uint16_t)(r >> 16);
    v0 = (a.q_dtype == KVR_BF16) ? bf16_to_f32(lo) : f16_to_f32(lo);
    v1 = (a.q_dtype == KVR_BF16) ? bf16_to_f32(hi) : f16_to_f32(hi);
  }
}

// Rotated GQA-mean query of a segment into qs[128] (one wave; lane = channel pair).
// qbar_load issues the loads of all g heads (clamped, branch-free) so they are in flight
// together; qbar_finish sums them in head order, divides by g once, rotates, stores.
template <int QT>
__device__ __forceinline__ void qbar_load(const DecodeArgs& a, int64_t seg, int lane, uint32_t* r0, uint32_t* r1) {
  const int64_t b = seg / a.Hkv;
  const int h = (int)(seg - b * a.Hkv);
  const int64_t q0 = (b * a.Hq + (int64_t)h * a.g) * D + 2 * lane;
#pragma unroll
  for (int i = 0; i < 16; ++i) {  // heads past g are not read (qbar_finish skips them)
    r0[i] = r1[i] = 0u;
    if (i < a.g) q_pair_raw<QT>(a, q0 + (int64_t)i * D, r0[i], r1[i]);
  }
}

// The GQA-mean query's channels (2 lane, 2 lane + 1) from the raw loads of qbar_load.
template <int QT>
__device__ __forceinline__ void qbar_mean(const DecodeArgs& a, uint32_t* r0, uint32_t* r1, float& m0, float& m1) {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    pin(r0[i]);
    if (QT == Q_RUNTIME || QT == KVR_FP32) pin(r1[i]);  // r1 is a constant 0 for 16-bit dtypes
  }
  q_pair_cvt<QT>(a, r0[0], r1[0], m0, m1);
#pragma unroll
  for (int i = 1; i < 16; ++i) {
    if (i < a.g) {
      float v0, v1;
      q_pair_cvt<QT>(a, r0[i], r1[i], v0, v1);
      m0 = m0 + v0;
      m1 = m1 + v1;
    }
  }
  m0 = __fdiv_rn(m0, (float)a.g);
  m1 = __fdiv_rn(m1, (float)a.g);
}

// Outputs k in [32 w, 32 w + 32) of y = C x (DCT-II) for a vector x held by the calling
// wave w as channels (2 lane, 2 lane + 1), into y_out[k]: each of the block's four waves
// calls it with its own scratch xs (the table staged at xs + D), and y_out holds all 128
// outputs after a block barrier.  With C[k][127 - n] = (-1)^k C[k][n], output k sums 64
// terms C[k][n] t[n] (t = x[n] + x[127 - n] for even k, x[n] - x[127 - n] for odd k),
// split over a lane pair (n < 32 and n >= 32) and added once: a quarter of dct_pair's
// LDS reads per lane.  Tolerance path (fmaf).
__device__ __forceinline__ void dct_quarter(float v0, float v1, int lane, int w, float* xs, float* y_out) {
  const float* cs = xs + D;
  xs[2 * lane] = v0;
  xs[2 * lane + 1] = v1;
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_wave_barrier();
  const float xa = xs[lane], xb = xs[127 - lane];
  __builtin_amdgcn_wave_barrier();
  ((float2*)xs)[lane] = make_float2(xa + xb, xa - xb);  // (s[n], d[n]) at n = lane
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_wave_barrier();
  const int k = 32 * w + (lane >> 1), h = lane & 1;
  // table index of C[k][n]: (2n+1) k mod 512, stepping by 2k from n = 32 h; row 0 stays at 512
  int r = (k == 0) ? 512 : ((64 * h + 1) * k) & 511;
  const int dr = (k == 0) ? 0 : (2 * k) & 511, msk = (k == 0) ? 1023 : 511;
  const bool odd = k & 1;
  float acc = 0.f;
#pragma unroll 8
  for (int i = 0; i < 32; ++i) {
    const float2 sd = ((const float2*)xs)[32 * h + i];
    acc = fmaf(cs[r], odd ? sd.y : sd.x, acc);
    r = (r + dr) & msk;
  }
  acc = acc + xor_lane_f<1>(acc);
  if (h == 0) y_out[k] = acc;
}

template <int QT>
__device__ __forceinline__ void qbar_finish(const DecodeArgs& a, uint32_t* r0, uint32_t* r1, float* qs, float* xs,
                                            int lane, const DctRegs& dt) {
  float m0, m1;
  qbar_mean<QT>(a, r0, r1, m0, m1);
  if (a.transform == KVR_DCT) dct_table_store(dt, xs, lane);
  rotate_pair(m0, m1, lane, a.transform, xs);
  qs[2 * lane] = m0;
  qs[2 * lane + 1] = m1;
}

__device__ void qbar_wave(const DecodeArgs& a, int64_t seg, float* qs, float* xs, int lane) {
  uint32_t r0[16], r1[16];
  qbar_load<Q_RUNTIME>(a, seg, lane, r0, r1);
  DctRegs dt{};
  if (a.transform == KVR_DCT) dt = dct_table_load(lane);
  qbar_finish<Q_RUNTIME>(a, r0, r1, qs, xs, lane, dt);
}

// Selection candidate (score_key << 32) | (0xffffffff - tile): a larger value is a
// better candidate in the (score desc, tile asc) order; 0 pads below every real key.
__device__ __forceinline__ uint64_t pack_cand(uint32_t key, uint32_t tile) {
  return ((uint64_t)key << 32) | (uint64_t)(0xffffffffu - tile);
}
__device__ __forceinline__ uint32_t cand_tile(uint64_t v) { return 0xffffffffu - (uint32_t)v; }


// ------------------------------------------------------------------ scoring

template <int METHOD>
__device__ __forceinline__ int count_bits(uint64_t w) {
  if constexpr (METHOD == 0) {
    return __popcll(w);  // v_bcnt_u32_b32 x 2
  } else {               // SWAR bit-unpack: pairwise bit sums, same count
    uint64_t x = w - ((w >> 1) & 0x5555555555555555ull);
    x = (x & 0x3333333333333333ull) + ((x >> 2) & 0x3333333333333333ull);
    x = (x + (x >> 4)) & 0x0f0f0f0f0f0f0f0full;
    return (int)((x * 0x0101010101010101ull) >> 56);
  }
}

// 16-lane tree h = 8, 4, 2, 1 by DPP (every lane of the group ends with the same value).
__device__ __forceinline__ float tree16(float p) {
  p = p + xor_lane_f<8>(p);
  p = p + xor_lane_f<4>(p);
  p = p + xor_lane_f<2>(p);
  p = p + xor_lane_f<1>(p);
  return p;
}

// Score items: 16 lanes per tile, lane li owns channels 8li..8li+7; each 16-lane group
// scores TPG tiles (16 * TPG * T / 64 words in flight per lane), so an item covers
// 16*TPG tiles.  The words are loaded before the query is ready (one HBM
// round trip per item, overlapped with the query prologue).
constexpr int score_tpg(int T) { return T == 64 ? KVR_SCORE_TPG : KVR_SCORE_TPG128; }

template <int T>
struct ScoreWords {
  static constexpr int W = T / 64;
  static constexpr int TPG = score_tpg(T);
  uint64_t w[TPG][8 * W];
};

constexpr int score_tiles_per_item(int T) { return 16 * score_tpg(T); }
// Candidate slots of a score item (its tiles, padded to a multiple of 64).
constexpr int score_cand_slots(int T) { return score_tiles_per_item(T) <= 64 ? 64 : 128; }

template <int T>
__device__ __forceinline__ void score_load(const uint64_t* kbits, int64_t seg, int64_t tile_stride,
                                           int64_t t0, int64_t t1, ScoreWords<T>& sw) {
  constexpr int W = T / 64;
  constexpr int TPG = ScoreWords<T>::TPG;
  const int grp = threadIdx.x >> 4;
  const int li = threadIdx.x & 15;
  const uint64_t* segbits = kbits + seg * tile_stride * (int64_t)(D * W);
#pragma unroll
  for (int i = 0; i < TPG; ++i) {
    int64_t tile = t0 + grp + 16 * i;
    tile = tile < t1 ? tile : t0;  // t0 < t1 <= tile_stride: always a stored tile
    const ulonglong2* wp = (const ulonglong2*)(segbits + tile * (D * W) + 8 * li * W);
#pragma unroll
    for (int j = 0; j < 4 * W; ++j) {
      const ulonglong2 v = wp[j];
      sw.w[i][2 * j] = v.x;
      sw.w[i][2 * j + 1] = v.y;
    }
  }
}

// A score item's channel counts from the K store's per-tile count summary: lane li of
// 16-lane group grp reads the 8 bytes of channels 8 li .. 8 li + 7 of its tiles.
template <int T>
struct ScoreCounts {
  uint64_t c[score_tpg(T)];
};

template <int T>
__device__ __forceinline__ void counts_load(const uint8_t* kcount, int64_t seg, int64_t tile_stride,
                                            int64_t t0, int64_t t1, ScoreCounts<T>& sc) {
  const int grp = threadIdx.x >> 4;
  const int li = threadIdx.x & 15;
  const uint8_t* segc = kcount + seg * tile_stride * (int64_t)D;
#pragma unroll
  for (int i = 0; i < score_tpg(T); ++i) {
    int64_t tile = t0 + grp + 16 * i;
    tile = tile < t1 ? tile : t0;
    sc.c[i] = *(const uint64_t*)(segc + tile * D + 8 * li);
  }
}

// Per-lane sequential fp32 sum of fl(q*c) over its 8 channels, then the 16-lane tree.
// pcf(i, k): the number of set bits of channel 8 li + k of the lane's tile i (from the
// words or from the count summary: the same integers, so the same scores).
template <int T, typename PC>
__device__ __forceinline__ void score_compute_pc(const float* qs, PC pcf, int64_t seg,
                                                 int64_t n_tiles, int64_t t0, int64_t t1, int32_t lo,
                                                 int32_t hi, float* scores, uint64_t* lc) {
  constexpr int TPG = score_tpg(T);
  const int grp = threadIdx.x >> 4;
  const int li = threadIdx.x & 15;
  float q[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) q[k] = qs[8 * li + k];
  float qq = q[0] * q[0];
#pragma unroll
  for (int k = 1; k < 8; ++k) qq = qq + q[k] * q[k];
  qq = tree16(qq);
  const float qn = sqrt_rn(qq) + EPS;
  static_assert(TPG <= 16, "one lane of the group per tile");
  float dsel = 0.f;
  int csel = 0;
#pragma unroll
  for (int i = 0; i < TPG; ++i) {
    float dot = 0.f;
    int cc = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int pc = pcf(i, k);
      const int c = 2 * pc - T;
      cc += c * c;
      const float prod = q[k] * (float)c;
      dot = (k == 0) ? prod : dot + prod;
    }
    dot = tree16(dot);  // butterflies: every lane of the group holds the same totals
    cc += (int)xor_lane_u<8>((uint32_t)cc);
    cc += (int)xor_lane_u<4>((uint32_t)cc);
    cc += (int)xor_lane_u<2>((uint32_t)cc);
    cc += (int)xor_lane_u<1>((uint32_t)cc);
    if (li == i) {  // lane i of the group finishes tile i
      dsel = dot;
      csel = cc;
    }
  }
  // One correctly rounded square root and division per lane for the group's TPG tiles
  // (lane li: tile t0 + grp + 16 li), instead of one pass per tile on lane 0.
  const int64_t tile = t0 + grp + 16 * li;
  if (li < TPG) {
    uint64_t cand = 0;  // pads below every real candidate
    if (tile < t1) {
      const float cn = sqrt_rn((float)csel) + EPS;
      float sc = __fdiv_rn(dsel, qn * cn);
      if (sc != sc) sc = -__builtin_inff();
      if (tile >= lo && tile < hi) sc = -__builtin_inff();
      if (scores) scores[seg * n_tiles + tile] = sc;  // not kept by the one-launch step
      cand = pack_cand(score_key(sc), (uint32_t)tile);
    }
    if (lc) lc[grp + 16 * li] = cand;
  } else if (lc && li < score_cand_slots(T) / 16) {
    lc[grp + 16 * li] = 0;  // padding slots
  }
}

template <int T, int METHOD>
__device__ __forceinline__ void score_compute(const float* qs, const ScoreWords<T>& sw, int64_t seg,
                                              int64_t n_tiles, int64_t t0, int64_t t1, int32_t lo,
                                              int32_t hi, float* scores, uint64_t* lc = nullptr) {
  constexpr int W = T / 64;
  score_compute_pc<T>(qs, [&](int i, int k) {
    int pc = 0;
#pragma unroll
    for (int w = 0; w < W; ++w) pc += count_bits<METHOD>(sw.w[i][k * W + w]);
    return pc;
  }, seg, n_tiles, t0, t1, lo, hi, scores, lc);
}

template <int T>
__device__ __forceinline__ void score_compute_counts(const float* qs, const ScoreCounts<T>& sc, int64_t seg,
                                                     int64_t n_tiles, int64_t t0, int64_t t1, int32_t lo,
                                                     int32_t hi, float* scores, uint64_t* lc) {
  score_compute_pc<T>(qs, [&](int i, int k) { return (int)((sc.c[i] >> (8 * k)) & 0xffu); },
                      seg, n_tiles, t0, t1, lo, hi, scores, lc);
}

// ------------------------------------------------------------------ top-k (one wave)

struct TopkSmem {
  uint32_t hist[256];
  uint32_t selk[TOPK_MAX_K];
  int32_t seli[TOPK_MAX_K];
};

// One compare-exchange stage of a 64-lane bitonic sort of (key, idx) pairs into the
// order key descending, idx ascending: block size S, partner lane ^ J.
template <int S, int J>
__device__ __forceinline__ void bitonic_step(uint32_t& key, int32_t& idx, int lane) {
  const uint32_t ok = xor_lane_u<J>(key);
  const int32_t oi = (int32_t)xor_lane_u<J>((uint32_t)idx);
  const bool lower = (lane & J) == 0;
  const bool asc = (lane & S) == 0;
  const bool mine_first = (key > ok) || (key == ok && idx < oi);
  if (mine_first != (lower == asc)) {
    key = ok;
    idx = oi;
  }
}

// Writes the k winners (key, index) into sm.selk / sm.seli in index order of the
// two classes (keys > tau first, then the first kk keys == tau), then orders them by
// (key desc, index asc) into out[0..k): a bitonic sort across the wave for k <= 64
// (padding sorts last), else each lane ranks one candidate per round of 64 against
// every candidate broadcast by readlane.
__device__ __forceinline__ void topk_rank_out(int k, int32_t* out, TopkSmem& sm, int lane) {
  wave_lds_sync();
  if (k <= 64) {
    uint32_t key = (lane < k) ? sm.selk[lane] : 0u;
    int32_t idx = (lane < k) ? sm.seli[lane] : 0x7fffffff;
    bitonic_step<2, 1>(key, idx, lane);
    bitonic_step<4, 2>(key, idx, lane);
    bitonic_step<4, 1>(key, idx, lane);
    bitonic_step<8, 4>(key, idx, lane);
    bitonic_step<8, 2>(key, idx, lane);
    bitonic_step<8, 1>(key, idx, lane);
    bitonic_step<16, 8>(key, idx, lane);
    bitonic_step<16, 4>(key, idx, lane);
    bitonic_step<16, 2>(key, idx, lane);
    bitonic_step<16, 1>(key, idx, lane);
    bitonic_step<32, 16>(key, idx, lane);
    bitonic_step<32, 8>(key, idx, lane);
    bitonic_step<32, 4>(key, idx, lane);
    bitonic_step<32, 2>(key, idx, lane);
    bitonic_step<32, 1>(key, idx, lane);
    bitonic_step<64, 32>(key, idx, lane);
    bitonic_step<64, 16>(key, idx, lane);
    bitonic_step<64, 8>(key, idx, lane);
    bitonic_step<64, 4>(key, idx, lane);
    bitonic_step<64, 2>(key, idx, lane);
    bitonic_step<64, 1>(key, idx, lane);
    if (lane < k) out[lane] = idx;
    return;
  }
  for (int a0 = 0; a0 < k; a0 += 64) {
    const bool act = a0 + lane < k;
    const uint32_t ka = act ? sm.selk[a0 + lane] : 0u;
    const int32_t ia = act ? sm.seli[a0 + lane] : 0;
    int rank = 0;
    for (int b0 = 0; b0 < k; b0 += 64) {
      const bool bv = b0 + lane < k;
      const uint32_t kbv = bv ? sm.selk[b0 + lane] : 0u;
      const int32_t ibv = bv ? sm.seli[b0 + lane] : 0;
      const int nb = (k - b0 < 64) ? k - b0 : 64;
      for (int j = 0; j < nb; ++j) {
        const uint32_t kb = (uint32_t)__builtin_amdgcn_readlane((int)kbv, j);
        const int32_t ib = __builtin_amdgcn_readlane(ibv, j);
        rank += (kb > ka) || (kb == ka && ib < ia);
      }
    }
    if (act) out[rank] = ia;
  }
}

// ---- two-level selection for k <= 64: every score item sorts its (up to 64) tiles,
// the retrieved items merge the per-item lists.  A candidate is packed as
// (score_key << 32) | (0xffffffff - tile), so a larger value is a better candidate in
// exactly the (score desc, tile asc) order; 0 pads (below every real key).

template <int J>
__device__ __forceinline__ uint64_t xor_lane_u64(uint64_t v) {
  const uint32_t lo = xor_lane_u<J>((uint32_t)v), hi = xor_lane_u<J>((uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}

// Compare-exchange stage of a 64-lane bitonic network sorting descending: block size S
// (S = 128: the whole wave is one descending block), partner lane ^ J.
template <int S, int J>
__device__ __forceinline__ void bitonic64(uint64_t& v, int lane) {
  const uint64_t o = xor_lane_u64<J>(v);
  const bool lower = (lane & J) == 0;
  const bool desc = (S >= 128) || ((lane & S) == 0);
  const bool keep_max = (lower == desc);
  v = keep_max ? (v > o ? v : o) : (v > o ? o : v);
}

// Full descending sort of one value per lane.
__device__ __forceinline__ void sort64_desc(uint64_t& v, int lane) {
  bitonic64<2, 1>(v, lane);
  bitonic64<4, 2>(v, lane);
  bitonic64<4, 1>(v, lane);
  bitonic64<8, 4>(v, lane);
  bitonic64<8, 2>(v, lane);
  bitonic64<8, 1>(v, lane);
  bitonic64<16, 8>(v, lane);
  bitonic64<16, 4>(v, lane);
  bitonic64<16, 2>(v, lane);
  bitonic64<16, 1>(v, lane);
  bitonic64<32, 16>(v, lane);
  bitonic64<32, 8>(v, lane);
  bitonic64<32, 4>(v, lane);
  bitonic64<32, 2>(v, lane);
  bitonic64<32, 1>(v, lane);
  bitonic64<128, 32>(v, lane);
  bitonic64<128, 16>(v, lane);
  bitonic64<128, 8>(v, lane);
  bitonic64<128, 4>(v, lane);
  bitonic64<128, 2>(v, lane);
  bitonic64<128, 1>(v, lane);
}

// Top 64 of two descending lists: lane l holds a[l] and b[63 - l]; max(a[l], b[63-l])
// is bitonic and holds the 64 largest, which six stages sort descending.
__device__ __forceinline__ uint64_t merge_top64(uint64_t a, uint64_t b_rev, int lane) {
  uint64_t v = a > b_rev ? a : b_rev;
  bitonic64<128, 32>(v, lane);
  bitonic64<128, 16>(v, lane);
  bitonic64<128, 8>(v, lane);
  bitonic64<128, 4>(v, lane);
  bitonic64<128, 2>(v, lane);
  bitonic64<128, 1>(v, lane);
  return v;
}

// sel[0..k) from the n_lists descending candidate lists of a segment (k <= 64), 128
// words per list: a batch of lists is loaded (list 0 in lane order, the others
// reversed for the merge, clamped), reloaded until every entry carries its tag (the
// lists' writers may still be running), then merged in order.  Every wait is bounded:
// after spin_max polls it gives up, stores 1 into the sticky error word *err and
// reports the failure to its caller, which poisons its output (NaN) -- a give-up is
// never a silent wrong answer.

__device__ __forceinline__ void wait_gave_up(int32_t* err, int lane) {
  if (err && lane == 0) __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Waits until one word (the last) of every list c = first + step * i < n_lists carries
// its tag: one 8-byte load per list and poll, so a waiting wave adds little traffic
// while the lists' writers run.  Returns false when it gave up.
__device__ __forceinline__ bool probe_list_set(const uint64_t* lists, int first, int step, int n_lists,
                                               int lane, uint32_t epoch, int64_t seg, int32_t* err,
                                               int spin_max) {
  for (int r0 = first; r0 < n_lists; r0 += 64 * step) {
    const int c = r0 + step * lane;
    const uint32_t tag_hi = (uint32_t)(cand_tag(epoch, seg, c) >> 32);
    for (int n = 0;; ++n) {
      const bool ok = c >= n_lists || (uint32_t)(cand_load(lists + (int64_t)c * 128 + 127) >> 32) == tag_hi;
      if (__all(ok)) break;
      if (n >= spin_max) {
        wait_gave_up(err, lane);
        return false;
      }
      __builtin_amdgcn_s_sleep(2);
    }
  }
  return true;
}

// Top 64 (descending, lane order; 0 pads) of the lists c = first + step * i < n_lists of
// a segment (128 words per list), loaded in batches of 8 (the first list in lane order,
// the others reversed for the merge) and reloaded until every entry carries its tag
// (the lists' writers may still be running).  The full loads start once probe_list_set
// has seen every list's last word.  failed is set when a wait gave up.
__device__ __forceinline__ uint64_t merge_list_set(const uint64_t* lists, int first, int step, int n_lists,
                                                   int lane, uint32_t epoch, int64_t seg, int32_t* err,
                                                   int spin_max, bool& failed) {
  constexpr int BATCH = 8;
  if (epoch != CAND_EPOCH_CHAIN && !probe_list_set(lists, first, step, n_lists, lane, epoch, seg, err, spin_max))
    failed = true;
  uint64_t acc = 0;
  for (int c0 = first; c0 < n_lists; c0 += BATCH * step) {
    uint64_t b[BATCH];
    for (int n = 0;; ++n) {
      bool ok = true;
#pragma unroll
      for (int i = 0; i < BATCH; ++i) {
        const int c = (c0 + i * step < n_lists) ? c0 + i * step : c0;
        b[i] = cand_get(lists + (int64_t)c * 128, (c0 == first && i == 0) ? lane : 63 - lane,
                        cand_tag(epoch, seg, c), ok);
      }
      if (__all(ok)) break;
      if (failed || n >= spin_max) {  // after a failed probe: one load, no further waiting
        wait_gave_up(err, lane);
        failed = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    // one copy of the merge code, rolled over the batch (straight-line copies of it cost
    // instruction fetches on their first and only run); b[0] is always the next list
    auto shift = [&]() {
#pragma unroll
      for (int r = 0; r + 1 < BATCH; ++r) b[r] = b[r + 1];  // static register moves
    };
    int i = 0;
    if (c0 == first) {  // the first list starts the accumulator
      acc = b[0];
      shift();
      i = 1;
    }
    const int nb = (n_lists - c0 + step - 1) / step < BATCH ? (n_lists - c0 + step - 1) / step : BATCH;
#pragma unroll 1
    for (; i < nb; ++i) {
      acc = merge_top64(acc, b[0], lane);
      shift();
    }
  }
  return acc;
}

// sel[0..k) from the n_lists descending candidate lists of a segment (k <= 64), merged by
// one wave.  Returns true when a wait gave up.
__device__ __forceinline__ bool select_from_cands(const uint64_t* lists, int n_lists, int k, int32_t* sel,
                                                  int lane, uint32_t epoch, int64_t seg, int32_t* err,
                                                  int spin_max) {
  bool failed = false;
  const uint64_t acc = merge_list_set(lists, 0, 1, n_lists, lane, epoch, seg, err, spin_max, failed);
  if (lane < k) sel[lane] = (int32_t)cand_tile(acc);
  return failed;
}

// Register-resident select for n <= 64*KPL: bitwise (MSB-first) search of tau, the
// largest key with #{key >= tau} >= k, from per-lane counts summed across the wave;
// no LDS atomics.
template <int KPL>
__device__ __forceinline__ void topk_wave_regs(const float* row, int64_t n, int k, int32_t* out, TopkSmem& sm, int lane) {
  uint32_t key[KPL];
  float vals[KPL];
#pragma unroll
  for (int r = 0; r < KPL; ++r) {
    const int64_t i = (int64_t)r * 64 + lane;
    vals[r] = row[i < n ? i : n - 1];  // clamped: every lane loads, all loads in flight
  }
#pragma unroll
  for (int r = 0; r < KPL; ++r) pin(vals[r]);
#pragma unroll
  for (int r = 0; r < KPL; ++r) {
    const int64_t i = (int64_t)r * 64 + lane;
    key[r] = (i < n) ? score_key(vals[r]) : 0u;  // padding sorts below every score (even -inf)
  }
  // MSB-first search; the count of keys >= cand is summed per lane, then across the
  // wave by DPP.  A count of exactly k ends the search: the keys >= tau are then the
  // answer (the tie classes below handle it unchanged).
  uint32_t tau = 0;
#pragma unroll 1
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t cand = tau | (1u << bit);
    float c = 0.f;
#pragma unroll
    for (int r = 0; r < KPL; ++r) c += (key[r] >= cand) ? 1.f : 0.f;
    const int cnt = __builtin_amdgcn_readfirstlane((int)wave_sum(c));
    if (cnt >= k) {
      tau = cand;
      if (cnt == k) break;
    }
  }
  int n_gt = 0;
#pragma unroll
  for (int r = 0; r < KPL; ++r) n_gt += __popcll(__ballot(key[r] > tau));
  const int kk = k - n_gt;
  const uint64_t lt_mask = (1ull << lane) - 1ull;
  int cg = 0, ce = 0;
#pragma unroll
  for (int r = 0; r < KPL; ++r) {  // slot r covers indices 64r..64r+63 in lane order
    const bool gt = key[r] > tau, eq = key[r] == tau;
    const uint64_t bg = __ballot(gt), be = __ballot(eq);
    const int i = r * 64 + lane;
    if (gt) {
      const int p = cg + __popcll(bg & lt_mask);
      sm.selk[p] = key[r];
      sm.seli[p] = i;
    }
    if (eq) {
      const int q = ce + __popcll(be & lt_mask);
      if (q < kk) {
        sm.selk[n_gt + q] = key[r];
        sm.seli[n_gt + q] = i;
      }
    }
    cg += __popcll(bg);
    ce += __popcll(be);
  }
  topk_rank_out(k, out, sm, lane);
}

// Any n: 4 x 8-bit radix passes with an LDS histogram, keys re-read from row.
__device__ __forceinline__ void topk_wave_hist(const float* row, int64_t n, int k, int32_t* out, TopkSmem& sm, int lane) {
  uint32_t prefix = 0, pmask = 0, kk = (uint32_t)k;
#pragma unroll 1
  for (int shift = 24; shift >= 0; shift -= 8) {
#pragma unroll
    for (int r = 0; r < 4; ++r) sm.hist[lane + 64 * r] = 0;
    wave_lds_sync();
    for (int64_t i = lane; i < n; i += 64) {
      const uint32_t key = score_key(row[i]);
      if ((key & pmask) == prefix) atomicAdd(&sm.hist[(key >> shift) & 255u], 1u);
    }
    wave_lds_sync();
    uint32_t c[4], tot = 0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {  // lane owns bins 255-4*lane .. 252-4*lane
      c[r] = sm.hist[255 - 4 * lane - r];
      tot += c[r];
    }
    uint32_t incl = tot;
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
      const uint32_t o = (uint32_t)__shfl_up((int)incl, m, 64);
      if (lane >= m) incl += o;
    }
    const uint32_t excl = incl - tot;
    uint32_t digit = 0, nkk = 0;
    const bool mine = excl < kk && kk <= incl;
    if (mine) {
      uint32_t run = excl;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (run < kk && kk <= run + c[r] && nkk == 0) {
          digit = 255u - 4u * lane - r;
          nkk = kk - run;
        }
        run += c[r];
      }
    }
    const int src = (int)__builtin_ctzll(__ballot(mine));  // exactly one lane owns the k-th key
    digit = (uint32_t)__shfl((int)digit, src, 64);
    kk = (uint32_t)__shfl((int)nkk, src, 64);
    prefix |= digit << shift;
    pmask |= 255u << shift;
  }
  const uint32_t tau = prefix;
  const uint32_t n_gt = (uint32_t)k - kk;
  uint32_t cnt_gt = 0, cnt_eq = 0;
  const uint64_t lt_mask = (1ull << lane) - 1ull;
#pragma unroll 1
  for (int64_t c0 = 0; c0 < n; c0 += 64) {
    const int64_t i = c0 + lane;
    const uint32_t key = (i < n) ? score_key(row[i]) : 0u;
    const bool gt = (i < n) && key > tau;
    const bool eq = (i < n) && key == tau;
    const uint64_t bg = __ballot(gt), be = __ballot(eq);
    if (gt) {
      const uint32_t p = cnt_gt + (uint32_t)__popcll(bg & lt_mask);
      if (p < n_gt) {
        sm.selk[p] = key;
        sm.seli[p] = (int32_t)i;
      }
    }
    if (eq) {
      const uint32_t r = cnt_eq + (uint32_t)__popcll(be & lt_mask);
      if (r < kk) {
        sm.selk[n_gt + r] = key;
        sm.seli[n_gt + r] = (int32_t)i;
      }
    }
    cnt_gt += (uint32_t)__popcll(bg);
    cnt_eq += (uint32_t)__popcll(be);
    if (cnt_gt >= n_gt && cnt_eq >= kk) break;  // uniform across the wave
  }
  topk_rank_out(k, out, sm, lane);
}

// idx[0..k) = indices of the k largest scores of row[0..n), score descending then
// index ascending (NaN counts as -inf).
__device__ __forceinline__ void topk_wave(const float* row, int64_t n, int k, int32_t* out, TopkSmem& sm, int lane) {
  if (n <= 512) topk_wave_regs<8>(row, n, k, out, sm, lane);
  else if (n <= 1024) topk_wave_regs<16>(row, n, k, out, sm, lane);
  else if (n <= 2048) topk_wave_regs<32>(row, n, k, out, sm, lane);
  else topk_wave_hist(row, n, k, out, sm, lane);
}

// The k selected tiles of a segment into sel[0..k): from the score items' sorted
// candidate lists when they were written (k <= 64), else by the wave select over the
// segment's scores.  Returns true when a bounded wait gave up.  The lists of a segment
// sit at the capacity pitch n_chunks_cap (the same as n_chunks without a live state).
__device__ __forceinline__ bool select_tiles(const DecodeArgs& a, int64_t seg, int k, int32_t* sel,
                                             TopkSmem& tk, int lane, uint32_t epoch = CAND_EPOCH_CHAIN) {
  if (a.cand)
    return select_from_cands(a.cand + seg * a.n_chunks_cap * (int64_t)128, a.n_chunks, k, sel, lane, epoch,
                             seg, a.ctr ? a.ctr + CTR_ERR_WORD : nullptr, a.spin_max);
  topk_wave(a.scores + seg * a.n_tiles, a.n_tiles, k, sel, tk, lane);
  return false;
}

// ------------------------------------------------------------------ MFMA helpers

template <int WDT>
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (WDT == KVR_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Split an fp32 value into NS 16-bit parts of the MFMA input type whose sum
// reproduces it to ~8*NS mantissa bits (bf16: truncation, exact remainders;
// fp16: round to nearest).
template <int WDT, int NS>
__device__ __forceinline__ void split16(float x, uint32_t* part) {
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    if constexpr (WDT == KVR_BF16) {
      const uint32_t hb = __float_as_uint(x) & 0xffff0000u;
      part[i] = hb >> 16;
      x = x - __uint_as_float(hb);
    } else {
      const _Float16 hh = (_Float16)x;
      part[i] = (uint32_t)__builtin_bit_cast(uint16_t, hh);
      x = x - (float)hh;
    }
  }
}

__device__ __forceinline__ uint32_t pack2(uint32_t lo16, uint32_t hi16) { return lo16 | (hi16 << 16); }

// Combine the 4 waves' softmax partials of one block into a record [m[g] | l[g] |
// o[g][128]].  Each wave leaves (m, l) per head column and its unscaled o in its own
// region ow[w][d*16 + n]; after one barrier every thread scales and sums the 4 waves'
// values of its (head, dim) elements in wave order.
struct CombineSmem {
  float cm[4][16];
  float cl[4][16];
};
constexpr int OW_WAVE = 16 * D;  // floats of one wave's partial o

template <typename DimOf>
__device__ __forceinline__ void combine_record(const f32x4 (&oacc)[8], float m_run, float l_run, float* ow,
                                               CombineSmem& cs, int g, float* R, DimOf dim_of,
                                               bool poison = false) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int n = lane & 15;
  const int kg = lane >> 4;
  if (kg == 0) {
    cs.cm[w][n] = m_run;
    cs.cl[w][n] = l_run;
  }
  if (n < g) {
    float* o = ow + w * OW_WAVE;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) o[dim_of(i, r, kg) * 16 + n] = oacc[i][r];
  }
  __syncthreads();
  if (tid < g) {
    float mh = -__builtin_inff();
#pragma unroll
    for (int v = 0; v < 4; ++v) mh = fmaxf(mh, cs.cm[v][tid]);
    const float muh = (mh == -__builtin_inff()) ? 0.f : mh;
    float lt = 0.f;
#pragma unroll
    for (int v = 0; v < 4; ++v) lt += cs.cl[v][tid] * fast_exp2(cs.cm[v][tid] - muh);
    rec_store(R + tid, mh);
    rec_store(R + g + tid, lt);
  }
  for (int e = tid; e < g * D; e += NT) {
    const int hn = e >> 7, d = e & (D - 1);
    float mh = -__builtin_inff();
#pragma unroll
    for (int v = 0; v < 4; ++v) mh = fmaxf(mh, cs.cm[v][hn]);
    const float muh = (mh == -__builtin_inff()) ? 0.f : mh;
    float acc = 0.f;
#pragma unroll
    for (int v = 0; v < 4; ++v) acc += ow[v * OW_WAVE + d * 16 + hn] * fast_exp2(cs.cm[v][hn] - muh);
    rec_store(R + 2 * g + e, poison ? __builtin_nanf("") : acc);  // a poisoned record makes the output NaN
  }
}

// Record stats from the per-wave (m, l) already in cs (the VALU retrieved role, which
// accumulates o in LDS itself).
__device__ void write_record_stats(const CombineSmem& cs, float* R, int g, int tid) {
  if (tid < g) {
    float mh = -__builtin_inff();
#pragma unroll
    for (int w = 0; w < 4; ++w) mh = fmaxf(mh, cs.cm[w][tid]);
    const float muh = (mh == -__builtin_inff()) ? 0.f : mh;
    float lt = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) lt += cs.cl[w][tid] * fast_exp2(cs.cm[w][tid] - muh);
    rec_store(R + tid, mh);
    rec_store(R + g + tid, lt);
  }
}

// ------------------------------------------------------------------ window role (MFMA)

// Window rows of a chunk of up to 32 logical tokens from c0 (c0 a multiple of 16).  Without
// a ring (RING false) row r is token c0 + r, clamped to the last token past win_len (the
// row is masked; the buffer may end there).  With a ring, row r is slot p0 + r, p0 = c0 +
// the ring start wrapped at the capacity: starts and capacities are multiples of 32 (the
// host checks), so a chunk never straddles the wrap and its rows past win_len stay inside
// the ring (masked).  p0 is uniform across the wave.
__device__ __forceinline__ int64_t ring_chunk_slot(const DecodeArgs& a, int64_t c0) {
  const int64_t s = c0 + a.win_start;
  return s >= a.win_cap ? s - a.win_cap : s;
}
template <bool RING>
__device__ __forceinline__ int64_t window_row(const DecodeArgs& a, int64_t c0, int64_t p0, int r) {
  if constexpr (RING) return p0 + r;
  const int64_t t = c0 + r;
  return t < a.win_len ? t : a.win_len - 1;
}

// Partial record of a segment: retrieved part r at index r, window part p at n_rparts + p,
// n_rparts + n_wparts_cap records per segment (live window parts fewer than the capacity
// leave the last slots unused, so the live records are always indices [0, n_parts)).
__device__ __forceinline__ float* rec_ptr(const DecodeArgs& a, int64_t seg, int index) {
  return a.rec + (seg * (a.n_wparts_cap + a.n_rparts) + index) * (int64_t)(a.g * (2 + D));
}

__device__ __forceinline__ f32x4 mfma16_f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

struct WindowSmem {
  union {
    uint16_t vstage[4][WIN_CHUNK * D];  // per-wave V rows, written by direct LDS loads
    float ow[4 * OW_WAVE];              // per-wave partial o (each over its own V rows)
  };
  CombineSmem cs;
};
static_assert(sizeof(uint16_t) * WIN_CHUNK * D == sizeof(float) * OW_WAVE, "ow[w] must overlay vstage[w]");

// Wait for this wave's outstanding vector-memory loads (including direct LDS loads).
__device__ __forceinline__ void wait_vm() { __builtin_amdgcn_s_waitcnt(0x0f70); }  // vmcnt(0)

typedef void __attribute__((address_space(3))) * lds_ptr_t;

// S^T[16 tok x 16 heads] = K[16 x 32 dims] Q^T[32 x 16];  O^T[16 dims x 16 heads] +=
// V^T[16 dims x 32 tok] P^T[32 tok x 16 heads].  Lane (n = lane & 15, kg = lane >> 4):
// Q^T/P^T column n = head n; S^T rows 4kg..4kg+3 of a 16-token block are tokens
// 16 tb + 4kg + r, which is the k-slot (kg, e = 4 tb + r) of the PV product, so the
// probabilities feed the B operand in place.  Block i of O^T has row m <-> dim 8m+i.
// K comes straight into registers in A-operand order; V rows go from HBM to the wave's
// LDS rows by direct 16-byte LDS loads (lane l of load i: token 4i + l/16, dims
// 8 (l%16) ..), both issued before the query is read.
template <int WDT, int QS, int PS, bool RING>
__device__ void window_role(const DecodeArgs& a, int64_t seg, int part, WindowSmem& sm) {
  constexpr int QT = (QS == 1) ? WDT : Q_RUNTIME;  // QS == 1: the query has the window's dtype
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv_id = tid >> 6;
  const int n = lane & 15;
  const int kg = lane >> 4;
  const int g = a.g;
  const int64_t b = seg / a.Hkv;
  const int64_t h = seg - b * a.Hkv;

  const uint16_t* kbase = (const uint16_t*)a.wk + b * a.sb + h * a.sh;
  const uint16_t* vbase = (const uint16_t*)a.wv + b * a.sb + h * a.sh;
  const int64_t win_len = a.win_len, st = a.st;
  const int64_t t_begin = (int64_t)part * a.win_span;
  const int64_t t_end = (t_begin + a.win_span < win_len) ? t_begin + a.win_span : win_len;
  uint16_t* vs = sm.vstage[wv_id];

  u32x4 ka[2][4];
  auto issue_chunk = [&](int64_t c0) {
    const int64_t p0 = RING ? ring_chunk_slot(a, c0) : c0;
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
      const uint16_t* kr = kbase + window_row<RING>(a, c0, p0, 16 * tb + n) * st + 8 * kg;  // rows past the end: masked
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) ka[tb][ks] = *(const u32x4*)(kr + 32 * ks);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(vbase + window_row<RING>(a, c0, p0, 4 * i + kg) * st + 8 * n),
                                       (lds_ptr_t)(vs + i * 4 * D), 16, 0, 0);
  };
  int64_t c0 = t_begin + (int64_t)wv_id * WIN_CHUNK;
  if (c0 < t_end) issue_chunk(c0);

  u32x4 qb[QS][4];
  {
    const int64_t qoff = (b * a.Hq + h * g + (n < g ? n : 0)) * D;
    uint32_t qr[4][8];  // raw query words: 4 pairs (16-bit) or 8 floats per k-step
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int pr = 0; pr < 4; ++pr) q_pair_raw<QT>(a, qoff + 32 * ks + 8 * kg + 2 * pr, qr[ks][2 * pr], qr[ks][2 * pr + 1]);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) pin(qr[ks][e]);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      float x[8];
#pragma unroll
      for (int pr = 0; pr < 4; ++pr) q_pair_cvt<QT>(a, qr[ks][2 * pr], qr[ks][2 * pr + 1], x[2 * pr], x[2 * pr + 1]);
      uint32_t pe[QS][8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        uint32_t p[QS];
        split16<WDT, QS>(n < g ? x[e] : 0.f, p);
#pragma unroll
        for (int sp = 0; sp < QS; ++sp) pe[sp][e] = p[sp];
      }
#pragma unroll
      for (int sp = 0; sp < QS; ++sp)
        qb[sp][ks] = u32x4{pack2(pe[sp][0], pe[sp][1]), pack2(pe[sp][2], pe[sp][3]),
                           pack2(pe[sp][4], pe[sp][5]), pack2(pe[sp][6], pe[sp][7])};
    }
  }

  f32x4 oacc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) oacc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -__builtin_inff();
  float l_run = 0.f;

  // Chunk c: wait for its K (registers) and V rows (LDS), S = K Q^T, read the V rows
  // into registers, then issue chunk c+1's loads, which fly during softmax and PV.
  for (; c0 < t_end; c0 += 4 * WIN_CHUNK) {
    wait_vm();
    f32x4 s[2];
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
      s[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int sp = 0; sp < QS; ++sp) s[tb] = mfma16<WDT>(ka[tb][ks], qb[sp][ks], s[tb]);
    }
    u32x4 rv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int trow = 16 * (e >> 2) + 4 * kg + (e & 3);
      rv[e] = *(const u32x4*)(vs + trow * D + 8 * n);
    }
    if (c0 + 4 * WIN_CHUNK < t_end) {
      wave_lds_sync();  // this chunk's V rows are in registers before they are reloaded
      issue_chunk(c0 + 4 * WIN_CHUNK);
    }

    float l2[8];
    float cmax = -__builtin_inff();
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int64_t tok = c0 + 16 * (e >> 2) + 4 * kg + (e & 3);
      float v = s[e >> 2][e & 3] * SCALE_LOG2;
      v = (tok < t_end) ? v : -__builtin_inff();
      l2[e] = v;
      cmax = fmaxf(cmax, v);
    }
    cmax = fmaxf(cmax, xor16_f(cmax));
    cmax = fmaxf(cmax, xor32_f(cmax));
    const float m_new = fmaxf(m_run, cmax);
    const float m_use = (m_new == -__builtin_inff()) ? 0.f : m_new;
    const float alpha = fast_exp2(m_run - m_use);
    m_run = m_new;
    float p[8];
    float psum = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      p[e] = fast_exp2(l2[e] - m_use);
      psum += p[e];
    }
    l_run = l_run * alpha + psum;
#pragma unroll
    for (int i = 0; i < 8; ++i) oacc[i] = oacc[i] * alpha;
    u32x4 pb[PS];
    {
      uint32_t pe[PS][8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        uint32_t pp[PS];
        split16<WDT, PS>(p[e], pp);
#pragma unroll
        for (int sp = 0; sp < PS; ++sp) pe[sp][e] = pp[sp];
      }
#pragma unroll
      for (int sp = 0; sp < PS; ++sp)
        pb[sp] = u32x4{pack2(pe[sp][0], pe[sp][1]), pack2(pe[sp][2], pe[sp][3]),
                       pack2(pe[sp][4], pe[sp][5]), pack2(pe[sp][6], pe[sp][7])};
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t sel = (i & 1) ? 0x07060302u : 0x05040100u;
      u32x4 av;
#pragma unroll
      for (int j = 0; j < 4; ++j) av[j] = __builtin_amdgcn_perm(rv[2 * j + 1][i >> 1], rv[2 * j][i >> 1], sel);
#pragma unroll
      for (int sp = 0; sp < PS; ++sp) oacc[i] = mfma16<WDT>(av, pb[sp], oacc[i]);
    }
  }

  l_run += xor16_f(l_run);
  l_run += xor32_f(l_run);
  // oacc[i][r] of lane (n, kg) is dim 32 kg + 8 r + i
  combine_record(oacc, m_run, l_run, sm.ow, sm.cs, g, rec_ptr(a, seg, a.n_rparts + part),
                 [](int i, int r, int kgv) { return 32 * kgv + 8 * r + i; });
}

// fp32 window tokens on fp32 MFMA (v_mfma_f32_16x16x4_f32; fp32 products, fp32
// accumulation).  Wave w takes 16-token tiles c0 = t_begin + 16 w, + 64, ...  Lane
// (n = lane & 15, kg = lane >> 4):
//   S^T[16 tok x 16 heads] = K Q^T over 32 k-steps; k-step s, k-slot kg is channel
//     32 kg + s, so lane (n, kg) loads channels 32 kg .. 32 kg + 31 of token c0 + n
//     (A) and holds query head n's same channels (B).
//   The S^T accumulator of lane (n, kg) holds tokens 4 kg + r of head n; for the PV
//   product k-step r's k-slot kg is token 4 kg + r, so the probabilities are the B
//   operand in place, and lane (n, kg) loads V[token 4 kg + r][dims 8 n .. 8 n + 7]
//   as the A operands of the eight dim blocks j (D row m <-> dim 8 m + j).
// The record layout matches the 16-bit window role: oacc[j][r] of lane (n, kg) is dim
// 32 kg + 8 r + j.
template <int QT, bool RING>
__device__ void window_role_f32(const DecodeArgs& a, int64_t seg, int part, WindowSmem& sm) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv_id = tid >> 6;
  const int n = lane & 15;
  const int kg = lane >> 4;
  const int g = a.g;
  const int64_t b = seg / a.Hkv;
  const int64_t h = seg - b * a.Hkv;
  const float* kbase = (const float*)a.wk + b * a.sb + h * a.sh;
  const float* vbase = (const float*)a.wv + b * a.sb + h * a.sh;
  const int64_t win_len = a.win_len, st = a.st;
  const int64_t t_begin = (int64_t)part * a.win_span;
  const int64_t t_end = (t_begin + a.win_span < win_len) ? t_begin + a.win_span : win_len;

  float qv[32];  // head n (zeros past g), channels 32 kg .. 32 kg + 31
  {
    const int64_t qoff = (b * a.Hq + h * g + (n < g ? n : 0)) * D + 32 * kg;
    uint32_t r0[16], r1[16];
#pragma unroll
    for (int p = 0; p < 16; ++p) q_pair_raw<QT>(a, qoff + 2 * p, r0[p], r1[p]);
#pragma unroll
    for (int p = 0; p < 16; ++p) {
      pin(r0[p]);
      if (QT == Q_RUNTIME || QT == KVR_FP32) pin(r1[p]);
    }
#pragma unroll
    for (int p = 0; p < 16; ++p) {
      q_pair_cvt<QT>(a, r0[p], r1[p], qv[2 * p], qv[2 * p + 1]);
      if (n >= g) qv[2 * p] = qv[2 * p + 1] = 0.f;
    }
  }
  f32x4 oacc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) oacc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -__builtin_inff();
  float l_run = 0.f;

  for (int64_t c0 = t_begin + 16 * (int64_t)wv_id; c0 < t_end; c0 += 64) {
    const int64_t p0 = RING ? ring_chunk_slot(a, c0) : c0;
    float kv[32];
    {
      const float4* kr = (const float4*)(kbase + window_row<RING>(a, c0, p0, n) * st + 32 * kg);  // past the end: masked
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float4 f = kr[i];
        kv[4 * i] = f.x;
        kv[4 * i + 1] = f.y;
        kv[4 * i + 2] = f.z;
        kv[4 * i + 3] = f.w;
      }
    }
    float vv[4][8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float4* vr = (const float4*)(vbase + window_row<RING>(a, c0, p0, 4 * kg + r) * st + 8 * n);
      const float4 f0 = vr[0], f1 = vr[1];
      vv[r][0] = f0.x; vv[r][1] = f0.y; vv[r][2] = f0.z; vv[r][3] = f0.w;
      vv[r][4] = f1.x; vv[r][5] = f1.y; vv[r][6] = f1.z; vv[r][7] = f1.w;
    }
    f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 32; ++ks) s = mfma16_f32(kv[ks], qv[ks], s);
    float p[4];
    float cmax = -__builtin_inff();
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t tok = c0 + 4 * kg + r;
      const float v = (tok < t_end) ? s[r] * SCALE_LOG2 : -__builtin_inff();
      p[r] = v;
      cmax = fmaxf(cmax, v);
    }
    cmax = fmaxf(cmax, xor16_f(cmax));
    cmax = fmaxf(cmax, xor32_f(cmax));
    const float m_new = fmaxf(m_run, cmax);
    const float m_use = (m_new == -__builtin_inff()) ? 0.f : m_new;
    const float alpha = fast_exp2(m_run - m_use);
    m_run = m_new;
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      p[r] = fast_exp2(p[r] - m_use);
      psum += p[r];
    }
    l_run = l_run * alpha + psum;
#pragma unroll
    for (int j = 0; j < 8; ++j) oacc[j] = oacc[j] * alpha;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int j = 0; j < 8; ++j) oacc[j] = mfma16_f32(vv[r][j], p[r], oacc[j]);
  }

  l_run += xor16_f(l_run);
  l_run += xor32_f(l_run);
  combine_record(oacc, m_run, l_run, sm.ow, sm.cs, g, rec_ptr(a, seg, a.n_rparts + part),
                 [](int j, int r, int kgv) { return 32 * kgv + 8 * r + j; });
}

// The window role for the window's dtype and layout (a plain run of slots or a ring).
template <int WDT, int QS, bool RING>
__device__ __forceinline__ void window_item(const DecodeArgs& a, int64_t seg, int part, WindowSmem& sm) {
  if constexpr (WDT == KVR_FP32) window_role_f32<(QS == 1) ? KVR_FP32 : Q_RUNTIME, RING>(a, seg, part, sm);
  else window_role<WDT, QS, 3, RING>(a, seg, part, sm);
}
template <int WDT, int QS>
__device__ __forceinline__ void window_item_any(const DecodeArgs& a, int64_t seg, int part, WindowSmem& sm) {
  if (a.win_cap > 0) window_item<WDT, QS, true>(a, seg, part, sm);
  else window_item<WDT, QS, false>(a, seg, part, sm);
}

// Query heads h0, h0 + step, ... (up to QH_MAX of them, the slots a wave rotates) of a
// segment: channel pair 2 lane, 2 lane + 1; loads clamped to head 0 past g, all issued
// before any is used.
constexpr int QH_MAX = 6;  // ceil(16 / 3): heads per wave when 3 waves share 16 slots
template <int QT>
__device__ __forceinline__ void load_heads_raw(const DecodeArgs& a, int64_t b, int64_t h, int h0, int step,
                                               int lane, uint32_t* r0, uint32_t* r1) {
  const int64_t base = (b * a.Hq + h * a.g) * D + 2 * lane;
#pragma unroll
  for (int j = 0; j < QH_MAX; ++j) {
    const int hh = h0 + step * j;
    q_pair_raw<QT>(a, base + (int64_t)(hh < a.g ? hh : 0) * D, r0[j], r1[j]);
  }
}
template <int QT>
__device__ __forceinline__ void load_heads_cvt(const DecodeArgs& a, uint32_t* r0, uint32_t* r1, float* v0,
                                               float* v1) {
#pragma unroll
  for (int j = 0; j < QH_MAX; ++j) {
    pin(r0[j]);
    if (QT == Q_RUNTIME || QT == KVR_FP32) pin(r1[j]);
  }
#pragma unroll
  for (int j = 0; j < QH_MAX; ++j) q_pair_cvt<QT>(a, r0[j], r1[j], v0[j], v1[j]);
}
template <int QT>
__device__ __forceinline__ void load_heads(const DecodeArgs& a, int64_t b, int64_t h, int h0, int step,
                                           int lane, float* v0, float* v1) {
  uint32_t r0[QH_MAX], r1[QH_MAX];
  load_heads_raw<QT>(a, b, h, h0, step, lane, r0, r1);
  load_heads_cvt<QT>(a, r0, r1, v0, v1);
}

// ------------------------------------------------------------------ retrieved role (VALU)

// 64x64 bit-matrix transpose across the wave: lane l holds row l (bit c = element
// (l, c)); afterwards lane c holds column c (bit l = element (l, c)).  Six block-swap
// stages; lane exchanges by v_permlane32_swap / permlane16 / DPP (no LDS).
template <int S>
__device__ __forceinline__ uint32_t tstage(uint32_t x, int lane, uint32_t m) {
  const uint32_t p = xor_lane_u<S>(x);
  return (lane & S) ? ((x & ~m) | ((p >> S) & m)) : ((x & m) | ((p & m) << S));
}

// The low four stages of transpose64 on one 32-bit word of the 64 channel words held
// one per lane (bit t of lane c: token t of channel c): lane bits 0..3 are swapped with
// bit-index bits 0..3, so lane (c5 c4 t3 t2 t1 t0) holds, at bit (t4 c3 c2 c1 c0), the
// bit of channel (c5 c4 c3 c2 c1 c0) and token (t4 t3 t2 t1 t0) of the word.
__device__ __forceinline__ void transpose_rows16(uint32_t& x, int lane) {
  x = tstage<8>(x, lane, 0x00ff00ffu);
  x = tstage<4>(x, lane, 0x0f0f0f0fu);
  x = tstage<2>(x, lane, 0x33333333u);
  x = tstage<1>(x, lane, 0x55555555u);
}

__device__ __forceinline__ void transpose64(uint32_t& lo, uint32_t& hi, int lane) {
  {
    // stage 32: lower lanes take the partner's lo as hi, upper lanes its hi as lo
    const auto r = __builtin_amdgcn_permlane32_swap(lo, hi, false, false);
    lo = r[0];
    hi = r[1];
  }
  lo = tstage<16>(lo, lane, 0x0000ffffu);
  hi = tstage<16>(hi, lane, 0x0000ffffu);
  lo = tstage<8>(lo, lane, 0x00ff00ffu);
  hi = tstage<8>(hi, lane, 0x00ff00ffu);
  lo = tstage<4>(lo, lane, 0x0f0f0f0fu);
  hi = tstage<4>(hi, lane, 0x0f0f0f0fu);
  lo = tstage<2>(lo, lane, 0x33333333u);
  hi = tstage<2>(hi, lane, 0x33333333u);
  lo = tstage<1>(lo, lane, 0x55555555u);
  hi = tstage<1>(hi, lane, 0x55555555u);
}

template <int G4>
struct RetSmem {
  int32_t sel[TOPK_MAX_K];    // the segment's selected tiles (score desc, index asc)
  float lq[32 * 16 * G4];     // [channel nibble][pattern][head]: sums of q'
  float qs[G4 * D];           // rotated query heads of the segment
  float qsum[G4];
  float xs[4][DCT_SCRATCH];   // per-wave scratch of the DCT helpers
  CombineSmem cs;
  union {
    TopkSmem tk;                // selection (before the tile loop)
    struct {
      float lu[4][16 * 16 * G4];  // per wave [token nibble][pattern][head]: sums of p
      float ps[4][64 * G4];       // per wave [token][head]
    } t;                        // tile loop
    float ost[16 * D];          // combine (after the tile loop)
  } u;
};

template <int W>
struct TileWords {
  uint64_t k0[W], k1[W], v0[W], v1[W];
  uint32_t sk, sv;  // fp16 bits of the tile's scales (converted where used)
};

template <int T>
__device__ __forceinline__ void load_tile(const DecodeArgs& a, int64_t seg, int64_t tile, int lane,
                                          TileWords<T / 64>& tw) {
  constexpr int W = T / 64;
  tile = tile < 0 ? 0 : (tile >= a.tile_stride ? a.tile_stride - 1 : tile);  // stay inside the store
  const int64_t slot = seg * a.tile_stride + tile;
  const uint64_t* kp = a.kbits + slot * (int64_t)(D * W);
  const uint64_t* vp = a.vbits + slot * (int64_t)(D * W);
#pragma unroll
  for (int w = 0; w < W; ++w) {
    tw.k0[w] = kp[lane * W + w];
    tw.k1[w] = kp[(lane + 64) * W + w];
    tw.v0[w] = vp[lane * W + w];
    tw.v1[w] = vp[(lane + 64) * W + w];
  }
  tw.sk = a.kscale[slot];
  tw.sv = a.vscale[slot];
}

// All selected tiles of one segment in one block: wave w takes tiles w, w+4, ...
// (the next tile's words are loaded while the current one is processed).  Keys /
// values of a retrieved token are s*(2b-1) per rotated channel.  Logits:
// dot_h(t) = sum_j q'_hj b_tj from the nibble table of q' applied to the transposed
// token rows; PV: sum_t p_ht b_tj from a per-tile nibble table of p applied to the
// channel words.  The 4 waves' online-softmax partials are combined into one record.
template <int T, int G4, int QT>
__device__ __forceinline__ void retrieved_role(const DecodeArgs& a, int64_t seg, int rp, RetSmem<G4>& sm, float* R) {
  constexpr int W = T / 64;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv_id = tid >> 6;
  const int g = a.g;
  const int k = a.k;
  const int64_t b = seg / a.Hkv;
  const int64_t h = seg - b * a.Hkv;
  const int RS = a.n_rparts;

  // wave 0 selects the tiles (when asked) while the other waves rotate query heads;
  // given indices are copied to LDS so every index read is an LDS read
  const int qw0 = a.do_select ? 1 : 0;
  if (!a.do_select)
    for (int i = tid; i < k; i += NT) sm.sel[i] = a.idx[seg * k + i];
  if (a.do_select && wv_id == 0) {
    select_tiles(a, seg, k, sm.sel, sm.u.tk, lane);
    wave_lds_sync();
    if (rp == 0)
      for (int i = lane; i < k; i += 64) a.idx[seg * k + i] = sm.sel[i];
  }
  if (wv_id >= qw0) {
    DctRegs dt{};
    if (a.transform == KVR_DCT) dt = dct_table_load(lane);
    float v0[QH_MAX], v1[QH_MAX];
    load_heads<QT>(a, b, h, wv_id - qw0, 4 - qw0, lane, v0, v1);
    if (a.transform == KVR_DCT) dct_table_store(dt, sm.xs[wv_id], lane);
#pragma unroll
    for (int j = 0; j < QH_MAX; ++j) {
      const int hh = wv_id - qw0 + (4 - qw0) * j;
      if (hh < G4) {
        float x0 = 0.f, x1 = 0.f;
        if (hh < g) {
          x0 = v0[j];
          x1 = v1[j];
          rotate_pair(x0, x1, lane, a.transform, sm.xs[wv_id]);
        }
        sm.qs[hh * D + 2 * lane] = x0;
        sm.qs[hh * D + 2 * lane + 1] = x1;
        const float tot = wave_sum(x0 + x1);
        if (lane == 0) sm.qsum[hh] = tot;
      }
    }
  }
  __syncthreads();
  for (int ent = tid; ent < 32 * 16; ent += NT) {
    const int c4 = ent >> 4, e = ent & 15;
#pragma unroll
    for (int hh = 0; hh < G4; ++hh) {
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (e & (1 << i)) acc += sm.qs[hh * D + 4 * c4 + i];
      sm.lq[ent * G4 + hh] = acc;
    }
  }
  TileWords<W> cur, nxt;
  const int j0 = rp * 4 + wv_id;
  if (j0 < k) load_tile<T>(a, seg, sm.sel[j0], lane, cur);
  __syncthreads();

  float m_run[G4], l_lane[G4], o0[G4], o1[G4];
#pragma unroll
  for (int hh = 0; hh < G4; ++hh) {
    m_run[hh] = -__builtin_inff();
    l_lane[hh] = 0.f;
    o0[hh] = 0.f;
    o1[hh] = 0.f;
  }
  float* lu = sm.u.t.lu[wv_id];
  float* ps = sm.u.t.ps[wv_id];
#pragma unroll 1
  for (int j = j0; j < k; j += 4 * RS) {
    if (j + 4 * RS < k)
      load_tile<T>(a, seg, sm.sel[j + 4 * RS], lane, nxt);
    const float sk = f16_to_f32(cur.sk), sv = f16_to_f32(cur.sv);
#pragma unroll 1
    for (int w = 0; w < W; ++w) {
      uint32_t a_lo = (uint32_t)cur.k0[w], a_hi = (uint32_t)(cur.k0[w] >> 32);
      uint32_t b_lo = (uint32_t)cur.k1[w], b_hi = (uint32_t)(cur.k1[w] >> 32);
      transpose64(a_lo, a_hi, lane);  // token row, channels 0..63
      transpose64(b_lo, b_hi, lane);  // token row, channels 64..127
      float dot[G4];
#pragma unroll
      for (int hh = 0; hh < G4; ++hh) dot[hh] = 0.f;
#pragma unroll
      for (int c4 = 0; c4 < 32; ++c4) {
        const uint32_t word = (c4 < 8) ? a_lo : (c4 < 16) ? a_hi : (c4 < 24) ? b_lo : b_hi;
        const uint32_t e = (word >> (4 * (c4 & 7))) & 15u;
        const float* ent = sm.lq + (c4 * 16 + e) * G4;
#pragma unroll
        for (int hh = 0; hh < G4; hh += 4) {
          const float4 v = *(const float4*)(ent + hh);
          dot[hh] += v.x;
          dot[hh + 1] += v.y;
          dot[hh + 2] += v.z;
          dot[hh + 3] += v.w;
        }
      }
      float alpha[G4], psum[G4];
#pragma unroll
      for (int hh = 0; hh < G4; ++hh) {
        const float lg = sk * (2.f * dot[hh] - sm.qsum[hh]) * SCALE_LOG2;
        const float m_new = fmaxf(m_run[hh], wave_max(lg));
        alpha[hh] = fast_exp2(m_run[hh] - m_new);
        m_run[hh] = m_new;
        const float p = fast_exp2(lg - m_new);
        l_lane[hh] = l_lane[hh] * alpha[hh] + p;
        psum[hh] = wave_sum(p);
        ps[lane * G4 + hh] = p;
      }
      wave_lds_sync();
      for (int ent = lane; ent < 16 * 16; ent += 64) {
        const int tn = ent >> 4, e = ent & 15;
#pragma unroll
        for (int hh = 0; hh < G4; ++hh) {
          float acc = 0.f;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (e & (1 << i)) acc += ps[(4 * tn + i) * G4 + hh];
          lu[ent * G4 + hh] = acc;
        }
      }
      wave_lds_sync();
      float x0[G4], x1[G4];
#pragma unroll
      for (int hh = 0; hh < G4; ++hh) {
        x0[hh] = 0.f;
        x1[hh] = 0.f;
      }
      const uint32_t vv[4] = {(uint32_t)cur.v0[w], (uint32_t)(cur.v0[w] >> 32), (uint32_t)cur.v1[w],
                              (uint32_t)(cur.v1[w] >> 32)};
#pragma unroll
      for (int tn = 0; tn < 16; ++tn) {
        const uint32_t e0 = (vv[tn >> 3] >> (4 * (tn & 7))) & 15u;
        const uint32_t e1 = (vv[2 + (tn >> 3)] >> (4 * (tn & 7))) & 15u;
        const float* t0 = lu + (tn * 16 + e0) * G4;
        const float* t1 = lu + (tn * 16 + e1) * G4;
#pragma unroll
        for (int hh = 0; hh < G4; hh += 4) {
          const float4 p0 = *(const float4*)(t0 + hh);
          const float4 p1 = *(const float4*)(t1 + hh);
          x0[hh] += p0.x; x0[hh + 1] += p0.y; x0[hh + 2] += p0.z; x0[hh + 3] += p0.w;
          x1[hh] += p1.x; x1[hh + 1] += p1.y; x1[hh + 2] += p1.z; x1[hh + 3] += p1.w;
        }
      }
#pragma unroll
      for (int hh = 0; hh < G4; ++hh) {
        o0[hh] = o0[hh] * alpha[hh] + sv * (2.f * x0[hh] - psum[hh]);
        o1[hh] = o1[hh] * alpha[hh] + sv * (2.f * x1[hh] - psum[hh]);
      }
      wave_lds_sync();  // ps / lu are rewritten by the next sub-tile
    }
    cur = nxt;
  }

  // combine the 4 waves (head hh of wave w: m_run[hh], l = wave sum of l_lane)
#pragma unroll
  for (int hh = 0; hh < G4; ++hh) {
    const float lt = wave_sum(l_lane[hh]);
    if (lane == 0) {
      sm.cs.cm[wv_id][hh] = m_run[hh];
      sm.cs.cl[wv_id][hh] = lt;
    }
  }
  __syncthreads();  // every wave is past its last use of lu / ps
  for (int i = tid; i < 16 * D; i += NT) sm.u.ost[i] = 0.f;
  __syncthreads();
#pragma unroll 1
  for (int w = 0; w < 4; ++w) {
    if (wv_id == w) {
#pragma unroll
      for (int hh = 0; hh < G4; ++hh) {
        if (hh < g) {
          float mx = -__builtin_inff();
#pragma unroll
          for (int w2 = 0; w2 < 4; ++w2) mx = fmaxf(mx, sm.cs.cm[w2][hh]);
          const float fw = fast_exp2(m_run[hh] - ((mx == -__builtin_inff()) ? 0.f : mx));
          sm.u.ost[hh * D + lane] += o0[hh] * fw;
          sm.u.ost[hh * D + lane + 64] += o1[hh] * fw;
        }
      }
    }
    __syncthreads();
  }
  write_record_stats(sm.cs, R, g, tid);
  for (int i = tid; i < g * D; i += NT) rec_store(R + 2 * g + i, sm.u.ost[i]);
}

// ------------------------------------------------------------------ retrieved role (MFMA)

struct RetMfmaSmem {
  union {
    struct {
      int32_t sel[TOPK_MAX_K];
      u32x4 pm1[256];         // byte -> 8 fp16 values (+1 for a set bit, -1 otherwise)
      u32x4 qb[4][2][64];     // Q'^T operands per k-step and fp16 part, per lane
      float xs[4][DCT_SCRATCH];
      union {
        TopkSmem tk;          // wave 0's selection from scores (while the other waves fill qb)
        uint64_t part[4][64]; // each wave's top 64 of its share of the candidate lists
      } p;
      int32_t selw[4][64];    // each wave's copy of the selection from candidate lists
    };
    float ow[4 * OW_WAVE];    // per-wave partial o' (after the tile loop)
  } u;
  CombineSmem cs;
  int fail[4];                // per wave: its selection's bounded wait gave up
};

__device__ __forceinline__ f32x4 mfma16_f16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                0, 0, 0);
}

// Retrieved tiles of one segment on MFMA (fp16 inputs, fp32 accumulate).  Block rs of
// the segment's RS blocks: wave w takes tiles rs*4 + w, then + 4*RS, ...
//   S^T[16 tok x 16 heads] = Khat[16 tok x 32 ch] Q'^T[32 ch x 16 heads]: Khat = +-1
//     from a partial bit transpose of the channel words (transpose_rows16: lane
//     (m, kq) then holds tokens 16 tb + m of channels 16 kq + 8 s + e, s < 2, e < 8,
//     tb < 4, so every A operand is a byte of the lane's own words -- no lane
//     exchange), k-step ks taking channels 64 (ks / 2) + 16 kq + 8 (ks % 2) + e;
//     Q' in that channel order, split in 2 fp16 parts.
//   O'^T[16 ch x 16 heads] += Vhat^T[16 ch x 32 tok] (sv P)^T[32 tok x 16 heads]: the
//     S^T accumulator slots are the PV k-slots (as in the window part); Vhat^T = +-1
//     from two nibbles of the lane's channel word; sv*P split in 2 fp16 parts.
// One 64-token unit of a selected tile (word `half` of each channel; a T = 128 tile is
// two units): the wave double-buffers units, not whole tiles, so its registers do not
// grow with T.
struct MfmaUnit {
  uint64_t kw[2];  // K channel words of channels lane and lane + 64 (bit-transpose rows)
  uint64_t vw[8];  // V channel words of channels 16 cb + n
  uint32_t sk, sv;  // fp16 bits of the tile's scales, converted where used (a conversion
                    // next to the loads would wait for them: no fetch ahead)
};

template <int T>
__device__ __forceinline__ void fetch_mfma_unit(const DecodeArgs& a, int64_t seg, int64_t tile, int half,
                                                int lane, MfmaUnit& t) {
  constexpr int W = T / 64;
  const int n = lane & 15;
  tile = tile < 0 ? 0 : (tile >= a.tile_stride ? a.tile_stride - 1 : tile);  // stay inside the store
  const int64_t slot = seg * a.tile_stride + tile;
  const uint64_t* kp = a.kbits + slot * (int64_t)(D * W) + half;
  const uint64_t* vp = a.vbits + slot * (int64_t)(D * W) + half;
  t.kw[0] = kp[lane * W];
  t.kw[1] = kp[(lane + 64) * W];
#pragma unroll
  for (int cb = 0; cb < 8; ++cb) t.vw[cb] = vp[(16 * cb + n) * W];
  t.sk = a.kscale[slot];
  t.sv = a.vscale[slot];
}

// epoch_word (fused step): the segment's epoch word; the selection reads the lists of
// this call (tag epoch + 1), which the segment's score items may still be writing.
// Null: lists of an earlier launch.
template <int T, int QT>
__device__ void retrieved_role_mfma(const DecodeArgs& a, int64_t seg, int rs, RetMfmaSmem& sm, float* R,
                                    const int32_t* epoch_word = nullptr) {
  constexpr int RP = KVR_RET_PARTS;  // fp16 parts of q' and sv*P
  constexpr int W = T / 64;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv_id = tid >> 6;
  const int kg = lane >> 4;  // k-slot group
  const int g = a.g;
  const int kp = a.k;  // pitch of the idx rows
  // tiles selected: k, fewer only when a live tile count is below it (then every stored
  // tile is taken; none at all when the store is empty)
  const int k = (a.live && a.n_tiles < (int64_t)a.k) ? (int)a.n_tiles : a.k;
  const bool do_sel = a.do_select && k > 0;
  const int64_t b = seg / a.Hkv;
  const int64_t h = seg - b * a.Hkv;
  if (KVR_RET_PRIO == 1) __builtin_amdgcn_s_setprio(3);

  // Wave w takes the selected tiles j = rs*4 + w, then + 4*RS, ..., as a sequence of
  // 64-token units (tile j0 + (u / W) * jstep, word u % W); the first unit's words are
  // fetched as soon as its index is known, each next one while the current unit is
  // processed.
  const int jstep = 4 * a.n_rparts;
  const int j0 = rs * 4 + wv_id;
  const int n_units = (j0 < k) ? ((k - 1 - j0) / jstep + 1) * W : 0;
  MfmaUnit cur;
  if (!a.do_select) {
    if (j0 < k) fetch_mfma_unit<T>(a, seg, a.idx[seg * kp + j0], 0, lane, cur);
    // the tile loop reads every next index from LDS in both modes (one address space:
    // an index read through a pointer that is LDS or global would be a FLAT load)
    for (int i = tid; i < k; i += NT) sm.u.sel[i] = a.idx[seg * kp + i];
  }

  // Selection (when asked).  From more than 8 candidate lists: every wave first rotates
  // its query heads (the lists are usually still being written), then merges lists
  // w, w + 4, ... into a partial top 64; the four partials meet in LDS and every wave
  // merges them (the same result in each) into its own copy of the selection.  (Merging
  // first, polling from the item's start, and rotating while the first tile's words are
  // in flight measured 3.6 us slower with 16 lists at T = 128.)  From fewer lists (one
  // load batch) or the scores: wave 0 selects while waves 1..3 rotate the query heads.  A
  // selection whose bounded wait gave up poisons the item's record.
  const bool par = do_sel && a.cand && a.n_chunks > 8;  // more than one load batch
  const int qw0 = (do_sel && !par) ? 1 : 0;
  uint32_t ep = epoch_word ? (uint32_t)__hip_atomic_load(epoch_word, __ATOMIC_RELAXED,
                                                          __HIP_MEMORY_SCOPE_AGENT) + 1u
                           : CAND_EPOCH_CHAIN;  // the lists' tag epoch
  if (a.wait_fail && epoch_word) ep ^= WAIT_FAIL_EPOCH;  // test hook: no list carries this tag
  bool failed = false;
  const bool rot_wave = wv_id >= qw0;
  uint32_t r0[QH_MAX], r1[QH_MAX];  // the wave's query heads, loaded first
  DctRegs dt{};
  if (rot_wave) {
    load_heads_raw<QT>(a, b, h, wv_id - qw0, 4 - qw0, lane, r0, r1);
    if (a.transform == KVR_DCT) dt = dct_table_load(lane);  // in flight with the query loads
  }
  // Q'^T operands: the wave's heads rotated into the B-operand layout
  auto rotate_heads = [&]() {
    float v0[QH_MAX], v1[QH_MAX];
    load_heads_cvt<QT>(a, r0, r1, v0, v1);
    if (a.transform == KVR_DCT) dct_table_store(dt, sm.u.xs[wv_id], lane);
#pragma unroll
    for (int j = 0; j < QH_MAX; ++j) {
      const int hh = wv_id - qw0 + (4 - qw0) * j;
      if (hh < 16) {
        float x0 = 0.f, x1 = 0.f;
        if (hh < g) {
          x0 = v0[j];
          x1 = v1[j];
          rotate_pair(x0, x1, lane, a.transform, sm.u.xs[wv_id]);
        }
        // Q'^T operand (B) of head column hh: lane (hh, kg) of k-step ks holds
        // q'[hh][64 (ks / 2) + 16 kg + 8 (ks % 2) + e], e < 8, in 2 fp16 parts; this
        // lane's channels 2 lane, 2 lane + 1 are k-step 2 (lane / 32) + (lane / 4) % 2,
        // slot group (lane / 8) % 4, word lane % 4
        uint32_t p0[RP], p1[RP];
        split16<KVR_FP16, RP>(x0, p0);
        split16<KVR_FP16, RP>(x1, p1);
        uint32_t* q32 = (uint32_t*)&sm.u.qb[2 * (lane >> 5) + ((lane >> 2) & 1)][0][hh + 16 * ((lane >> 3) & 3)];
#pragma unroll
        for (int sp = 0; sp < RP; ++sp) q32[sp * 64 * 4 + (lane & 3)] = pack2(p0[sp], p1[sp]);
      }
    }
  };
  if (do_sel && !par && wv_id == 0) {
    failed = select_tiles(a, seg, k, sm.u.sel, sm.u.p.tk, lane, ep);
    wave_lds_sync();
    if (rs == 0)
      for (int i = lane; i < kp; i += 64) a.idx[seg * kp + i] = (i < k) ? sm.u.sel[i] : -1;
  }
  if (rot_wave) rotate_heads();
  if (par)
    sm.u.p.part[wv_id][lane] = merge_list_set(a.cand + seg * a.n_chunks_cap * (int64_t)128, wv_id, 4, a.n_chunks,
                                              lane, ep, seg, a.ctr ? a.ctr + CTR_ERR_WORD : nullptr, a.spin_max,
                                              failed);
  {  // +-1 patterns: entry x, element e = bit e of x
    const int x = tid;
    uint32_t w[4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const uint32_t lo = ((x >> (2 * jj)) & 1) ? 0x3c00u : 0xbc00u;      // fp16 +1 / -1
      const uint32_t hi = ((x >> (2 * jj + 1)) & 1) ? 0x3c00u : 0xbc00u;
      w[jj] = lo | (hi << 16);
    }
    sm.u.pm1[x] = u32x4{w[0], w[1], w[2], w[3]};
  }
  sm.fail[wv_id] = failed ? 1 : 0;  // each wave its own flag: no clearing before the barrier
  __syncthreads();
  const bool poison = (sm.fail[0] | sm.fail[1] | sm.fail[2] | sm.fail[3]) != 0;  // any wave's wait gave up
  const int32_t* sel = sm.u.sel;
  if (par) {
    uint64_t acc = sm.u.p.part[0][lane];
#pragma unroll 1
    for (int w = 1; w < 4; ++w) acc = merge_top64(acc, sm.u.p.part[w][63 - lane], lane);
    sm.u.selw[wv_id][lane] = (int32_t)cand_tile(acc);
    wave_lds_sync();
    if (wv_id == 0 && rs == 0 && lane < kp) a.idx[seg * kp + lane] = (lane < k) ? (int32_t)cand_tile(acc) : -1;
    sel = sm.u.selw[wv_id];
  }
  if (do_sel && j0 < k) fetch_mfma_unit<T>(a, seg, sel[j0], 0, lane, cur);

  f32x4 oacc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) oacc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -__builtin_inff(), l_run = 0.f;

  if (KVR_RET_PRIO == 2) __builtin_amdgcn_s_setprio(3);
  for (int u = 0; u < n_units; ++u) {
    MfmaUnit nxt;  // the wave's next unit, fetched while this one is processed
    if (u + 1 < n_units)
      fetch_mfma_unit<T>(a, seg, sel[j0 + ((u + 1) / W) * jstep], (u + 1) % W, lane, nxt);
    const float sk = f16_to_f32((uint16_t)cur.sk) * SCALE_LOG2, sv = f16_to_f32((uint16_t)cur.sv);
    {
      uint32_t row[4] = {(uint32_t)cur.kw[0], (uint32_t)(cur.kw[0] >> 32), (uint32_t)cur.kw[1],
                         (uint32_t)(cur.kw[1] >> 32)};
#pragma unroll
      for (int i = 0; i < 4; ++i) transpose_rows16(row[i], lane);  // row[2 c + w]: channels 64 c.., tokens 32 w..

      // ---- S^T = Khat Q'^T (log2 units after * sk)
      f32x4 sacc[4];
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        sacc[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const uint32_t d = row[2 * (ks >> 1) + (tb >> 1)] >> (8 * (2 * (tb & 1) + (ks & 1)));
          const u32x4 av = sm.u.pm1[d & 255u];
#pragma unroll
          for (int sp = 0; sp < RP; ++sp) sacc[tb] = mfma16_f16(av, sm.u.qb[ks][sp][lane], sacc[tb]);
        }
      }
      // ---- online softmax over the 64 tokens (head n lane-local)
      float lg[16];
      float cmax = -__builtin_inff();
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        lg[e] = sacc[e >> 2][e & 3] * sk;
        cmax = fmaxf(cmax, lg[e]);
      }
      cmax = fmaxf(cmax, xor16_f(cmax));
      cmax = fmaxf(cmax, xor32_f(cmax));
      const float m_new = fmaxf(m_run, cmax);
      const float alpha = fast_exp2(m_run - m_new);
      m_run = m_new;
      float psum = 0.f;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        lg[e] = fast_exp2(lg[e] - m_new);
        psum += lg[e];
      }
      l_run = l_run * alpha + psum;
#pragma unroll
      for (int i = 0; i < 8; ++i) oacc[i] = oacc[i] * alpha;

      // ---- O'^T += Vhat^T (sv P)^T, two k-steps of 32 tokens (dword ks2 of the words)
#pragma unroll
      for (int ks2 = 0; ks2 < 2; ++ks2) {
        u32x4 pb[RP];
        {
          uint32_t pe[RP][8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            uint32_t pp[RP];
            split16<KVR_FP16, RP>(lg[8 * ks2 + e] * sv, pp);
#pragma unroll
            for (int sp = 0; sp < RP; ++sp) pe[sp][e] = pp[sp];
          }
#pragma unroll
          for (int sp = 0; sp < RP; ++sp)
            pb[sp] = u32x4{pack2(pe[sp][0], pe[sp][1]), pack2(pe[sp][2], pe[sp][3]),
                           pack2(pe[sp][4], pe[sp][5]), pack2(pe[sp][6], pe[sp][7])};
        }
        const int sh0 = 4 * kg;
#pragma unroll
        for (int cb = 0; cb < 8; ++cb) {
          const uint32_t vd = (uint32_t)(cur.vw[cb] >> (32 * ks2));
          const uint32_t lo = (vd >> sh0) & 15u;
          const uint32_t hi = (vd >> (sh0 + 16)) & 15u;
          const u32x4 av = sm.u.pm1[lo | (hi << 4)];
#pragma unroll
          for (int sp = 0; sp < RP; ++sp) oacc[cb] = mfma16_f16(av, pb[sp], oacc[cb]);
        }
      }
    }
    cur = nxt;
  }

  if (KVR_RET_PRIO == 2) __builtin_amdgcn_s_setprio(0);
  // ---- combine the 4 waves into one record (o' in the rotated domain); ow overlays
  // all of the role's scratch, dead once every wave has left the tile loop
  __syncthreads();
  l_run += xor16_f(l_run);
  l_run += xor32_f(l_run);
  // oacc[cb][r] of lane (n, kg) is channel 16 cb + 4 kg + r
  combine_record(oacc, m_run, l_run, sm.u.ow, sm.cs, g, R,
                 [](int i, int r, int kgv) { return 16 * i + 4 * kgv + r; }, poison);
  if (KVR_RET_PRIO == 1) __builtin_amdgcn_s_setprio(0);
}

// ------------------------------------------------------------------ merge

__device__ __forceinline__ float2 rec_load2(const float* p) {  // 8-byte aligned
  return __builtin_bit_cast(float2, __hip_atomic_load((const uint64_t*)p, __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_AGENT));
}

// One wave per (sequence, query head i of segment seg): LSE-merge every partial record
// of the segment (window parts in the original domain, retrieved parts rotated; their
// sum is rotated back once), normalise, store.  Parts go in batches of MAXP, every load
// of a batch in flight together: lane p loads part p's max and sum, every lane the
// part's two output channels; the batch max and the sum of l * exp2(m - max) are wave
// reductions, the per-part weights are read from their lanes.  The order of every sum
// is fixed, so the result is deterministic.
template <int MAXP>
__device__ __forceinline__ void merge_parts(const DecodeArgs& a, const float* R0, int64_t rs, int i, int lane,
                                            float& M, float& L, float& w0, float& w1, float& r0, float& r1) {
  const int g = a.g;
  const int n_parts = a.n_wparts + a.n_rparts;
  for (int p0 = 0; p0 < n_parts; p0 += MAXP) {
    const bool mine = lane < MAXP && p0 + lane < n_parts;  // this lane's part of the batch
    const float* Rl = R0 + (mine ? p0 + lane : p0) * rs;
    const float pm = rec_load(Rl + i);
    const float pl = rec_load(Rl + g + i);
    float2 po[MAXP];
#pragma unroll
    for (int p = 0; p < MAXP; ++p) {
      const int pc = (p0 + p < n_parts) ? p0 + p : n_parts - 1;
      po[p] = rec_load2(R0 + pc * rs + 2 * g + i * D + 2 * lane);
    }
    const float Mn = fmaxf(M, wave_max(mine ? pm : -__builtin_inff()));
    const float mu = (Mn == -__builtin_inff()) ? 0.f : Mn;
    const float sc = fast_exp2(M - mu);
    const float f = mine ? fast_exp2(pm - mu) : 0.f;
    L = L * sc + wave_sum(pl * f);
    w0 *= sc;
    w1 *= sc;
    r0 *= sc;
    r1 *= sc;
    M = Mn;
#pragma unroll
    for (int p = 0; p < MAXP; ++p) {
      const float fp = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f), p));  // 0 past the end
      if (p0 + p < a.n_rparts) {
        r0 = fmaf(po[p].x, fp, r0);
        r1 = fmaf(po[p].y, fp, r1);
      } else {
        w0 = fmaf(po[p].x, fp, w0);
        w1 = fmaf(po[p].y, fp, w1);
      }
    }
  }
}

// Sums of head i over the segment's parts on one wave (channels 2 lane, 2 lane + 1):
// L, the window part w and the (rotated) retrieved part r, all scaled to one max.
__device__ __forceinline__ void merge_sums(const DecodeArgs& a, int64_t seg, int i, int lane, float& L, float& w0,
                                           float& w1, float& r0, float& r1) {
  const int n_parts = a.n_wparts + a.n_rparts;
  const int64_t rs = a.g * (2 + D);
  const float* R0 = rec_ptr(a, seg, 0);
  // batches of 8, 20 or 32 parts: few more loads than parts (the merge code runs once,
  // fetched from L2, so every unused unrolled load costs time: a segment of 20 parts -- 16
  // retrieved items of 4 tiles of 128 and 4 window items -- merged ~1 us faster than with a
  // batch of 32)
  float M = -__builtin_inff();
  L = w0 = w1 = r0 = r1 = 0.f;
  if (n_parts <= 8) merge_parts<8>(a, R0, rs, i, lane, M, L, w0, w1, r0, r1);
  else if (n_parts <= 20) merge_parts<20>(a, R0, rs, i, lane, M, L, w0, w1, r0, r1);
  else merge_parts<32>(a, R0, rs, i, lane, M, L, w0, w1, r0, r1);
}

__device__ void merge_head(const DecodeArgs& a, int64_t seg, int i, int lane, float* xs) {
  const int64_t bq = (seg / a.Hkv) * a.Hq + (seg % a.Hkv) * a.g + i;  // b * Hq + head
  const bool dct = a.transform == KVR_DCT && a.n_rparts > 0;
  DctRegs dt{};
  if (dct) dt = dct_table_load(lane);
  float L, w0, w1, r0, r1;
  merge_sums(a, seg, i, lane, L, w0, w1, r0, r1);
  if (dct) dct_table_store(dt, xs, lane);
  if (a.n_rparts > 0) unrotate_pair(r0, r1, lane, a.transform, xs);
  const float inv = (L > 0.f) ? 1.f / L : 0.f;
  const float y0 = (w0 + r0) * inv, y1 = (w1 + r1) * inv;
  const int64_t o = bq * D + 2 * lane;
  if (a.out_dtype == KVR_FP32) {
    ((float2*)a.out)[o >> 1] = make_float2(y0, y1);
  } else {
    ((uint32_t*)a.out)[o >> 1] = pack2(f32_to_bf16_rne(y0), f32_to_bf16_rne(y1));
  }
}

// ---- whole-segment merge on the block's four waves
//
// Phase A gathers every head's window sums W and retrieved sums R (each part scaled to
// the head's max over all parts) into LDS slots [kind][slot][head][channel]:
//   parts-split (4 < g <= 8, n_parts <= 4 KVR_MERGE_PB): wave w takes parts w, w + 4, ...
//     for every head at once -- one load batch -- and every wave holds every
//     part's max and sum (lane p: part p), so all four scale to the same per-head max;
//     the four waves' sums go to four slots, added in slot order where used;
//   per head (otherwise): wave w takes heads w, w + 4, ... (merge_sums), one slot.
// Phase B rotates R back and stores (W + R_unrotated) / L:
//   DCT on MFMA: x = C^T y with the rows of C even or odd about n -> 127 - n
//     (C[k][127 - n] = (-1)^k C[k][n]), so wave w forms for its 16 output channels
//     n = 16 w + m the even-row sum E and the odd-row sum O (K = 64 each) and writes
//     x[n] = E + O and x[127 - n] = E - O: 12 fp16 16x16x32 products per wave with both
//     operands split into two fp16 parts (hi * hi + hi * lo + lo * hi, ~22-bit products,
//     fp32 accumulation); R enters already divided by L (fp16 range), C enters times 8
//     (fewer fp16 subnormals among its low parts), the table in constant memory holds
//     C's parts in operand order;
//   Hadamard / none: wave w takes heads w, w + 4, ... (in-register Hadamard).
constexpr int MG_PITCH = D + 4;  // floats per head row (padded: conflict-free 16-byte columns)
constexpr int MG_FLOATS = 2 * 4 * 8 * MG_PITCH;  // 2 kinds x 4 slots x 8 heads (or 1 slot x 16 heads)
struct MergeSmem {
  float buf[MG_FLOATS];
  float inv[16];  // 1 / L per head
};
static_assert(2 * 1 * 16 * MG_PITCH <= MG_FLOATS, "one slot of 16 heads");
__device__ __forceinline__ float* mg_row(MergeSmem& ms, int kind, int slot, int nslots, int g, int head) {
  return ms.buf + ((kind * nslots + slot) * g + head) * MG_PITCH;
}

// fp16 parts of C (times 8) in MFMA A-operand order: [w][eo][ks][part][lane] x 8 halves,
// lane (m, kq) element e = C[2 (32 ks + 8 kq + e) + eo][16 w + m] * 8, rounded to nearest
// even at compile time (hi = fp16(x), lo = fp16(x - hi)).
constexpr uint32_t f16_bits_rne(double x) {
  uint32_t sign = 0;
  if (x < 0) {
    sign = 0x8000u;
    x = -x;
  }
  if (x == 0.0) return sign;
  int e = 0;
  double p = 1.0;  // 2^e, x in [p, 2p) (or the subnormal range at e = -14)
  while (x >= 2.0 * p) {
    p *= 2.0;
    ++e;
  }
  while (x < p && e > -14) {
    p *= 0.5;
    --e;
  }
  const double m = x / (p / 1024.0);  // exact: a power-of-two quantum
  uint32_t mi = (uint32_t)m;
  const double fr = m - (double)mi;
  if (fr > 0.5 || (fr == 0.5 && (mi & 1u))) ++mi;
  if (mi >= 1024u) {
    if (mi == 2048u) {
      mi = 1024u;
      ++e;
    }
    return sign | ((uint32_t)(e + 15) << 10) | (mi - 1024u);
  }
  return sign | mi;
}
constexpr double f16_value(uint32_t b) {
  const int ex = (int)((b >> 10) & 31u);
  double v = (ex == 0) ? (double)(b & 1023u) : (double)(1024u + (b & 1023u));
  for (int sh = (ex == 0) ? -24 : ex - 25; sh != 0; sh += (sh < 0) ? 1 : -1) v = (sh < 0) ? v * 0.5 : v * 2.0;
  return (b & 0x8000u) ? -v : v;
}
struct DctF16Table {
  uint32_t v[4 * 2 * 2 * 2 * 64 * 4];
};
constexpr DctF16Table make_dct_f16_table() {
  DctF16Table t{};
  double c[512] = {};
  for (int r = 0; r < 512; ++r) c[r] = cos_pi_r256(r);
  for (int w = 0; w < 4; ++w)
    for (int eo = 0; eo < 2; ++eo)
      for (int ks = 0; ks < 2; ++ks)
        for (int lane = 0; lane < 64; ++lane)
          for (int e = 0; e < 8; ++e) {
            const int n = 16 * w + (lane & 15);
            const int k = 2 * (32 * ks + 8 * (lane >> 4) + e) + eo;
            const double sc = (k == 0) ? 0.088388347648318440550 : 0.125;
            const double x = (double)(float)(sc * c[((2 * n + 1) * k) % 512]) * 8.0;  // the fp32 C entry
            const uint32_t hi = f16_bits_rne(x);
            const uint32_t lo = f16_bits_rne(x - f16_value(hi));
            const int at = ((((w * 2 + eo) * 2 + ks) * 2) * 64 + lane) * 4 + (e >> 1);
            t.v[at] |= hi << (16 * (e & 1));
            t.v[at + 64 * 4] |= lo << (16 * (e & 1));
          }
  return t;
}
constexpr DctF16Table kDctF16 = make_dct_f16_table();
static __constant__ DctF16Table g_dct16 = kDctF16;

// A operands of wave w: [eo * 4 + ks * 2 + part]
__device__ __forceinline__ void dct16_load(int w, int lane, u32x4 (&A)[8]) {
  const u32x4* t = (const u32x4*)g_dct16.v + w * 8 * 64 + lane;
#pragma unroll
  for (int i = 0; i < 8; ++i) A[i] = t[i * 64];
}

// Block barrier over LDS only: LDS accesses complete and stay on their side of it; global
// loads in flight stay in flight.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ void store_out4(const DecodeArgs& a, int64_t o, float y0, float y1, float y2, float y3) {
  if (a.out_dtype == KVR_FP32) {
    *(float4*)((float*)a.out + o) = make_float4(y0, y1, y2, y3);
  } else {
    *(uint2*)((uint16_t*)a.out + o) = make_uint2(pack2(f32_to_bf16_rne(y0), f32_to_bf16_rne(y1)),
                                                 pack2(f32_to_bf16_rne(y2), f32_to_bf16_rne(y3)));
  }
}

// Phase A, parts-split (see above): G >= g heads, n_parts <= 4 PB (one load batch).
template <int G, int PB>
__device__ void merge_gather_split(const DecodeArgs& a, int64_t seg, MergeSmem& ms, int lane, int w) {
  const int g = a.g;
  const int P = a.n_wparts + a.n_rparts;
  const int nr = a.n_rparts;
  const int64_t rs = (int64_t)g * (2 + D);
  const float* R0 = rec_ptr(a, seg, 0);
  const bool mine = lane < P;  // lane p holds part p's max and sum
  const float* Rl = R0 + (mine ? lane : P - 1) * rs;
  // (every address below is a per-part base plus a constant head offset: loads of heads
  // past g are skipped, not clamped -- a clamped head index would cost an address per load)
  float pm[G], pq[G];
#pragma unroll
  for (int i = 0; i < G; ++i) {
    pm[i] = -__builtin_inff();
    pq[i] = 0.f;
    if (i < g) {
      pm[i] = rec_load(Rl + i);
      pq[i] = rec_load(Rl + g + i);
    }
  }
  const int npw = (P > w) ? (P - w + 3) / 4 : 0;  // parts of wave w
  float2 o[G][PB];  // in flight while the weights are formed
#pragma unroll
  for (int j = 0; j < PB; ++j) {
    int p = w + 4 * j;
    p = p < P ? p : P - 1;
    const float* Rp = R0 + p * rs + 2 * g + 2 * lane;
#pragma unroll
    for (int i = 0; i < G; ++i) o[i][j] = (i < g) ? rec_load2(Rp + i * D) : make_float2(0.f, 0.f);
  }
  float f[G], L[G];
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const float mx = wave_max(mine ? pm[i] : -__builtin_inff());
    const float mu = (mx == -__builtin_inff()) ? 0.f : mx;
    f[i] = mine ? fast_exp2(pm[i] - mu) : 0.f;
    L[i] = wave_sum(mine ? pq[i] * f[i] : 0.f);
  }
  // per head: the wave's parts in order, then the sums to the wave's slot (one head's
  // sums live at a time; the head's loads are dead after it)
#pragma unroll
  for (int i = 0; i < G; ++i) {
    if (i < g) {
      float r0 = 0.f, r1 = 0.f, w0 = 0.f, w1 = 0.f;
#pragma unroll
      for (int j = 0; j < PB; ++j) {
        const int p = w + 4 * j;
        if (j < npw) {
          const float fp = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f[i]), p));
          const float fr = p < nr ? fp : 0.f, fw = p < nr ? 0.f : fp;
          r0 = fmaf(o[i][j].x, fr, r0);
          r1 = fmaf(o[i][j].y, fr, r1);
          w0 = fmaf(o[i][j].x, fw, w0);
          w1 = fmaf(o[i][j].y, fw, w1);
        }
      }
      ((float2*)mg_row(ms, 0, w, 4, g, i))[lane] = make_float2(w0, w1);
      ((float2*)mg_row(ms, 1, w, 4, g, i))[lane] = make_float2(r0, r1);
      if (w == 0 && lane == 0) ms.inv[i] = (L[i] > 0.f) ? 1.f / L[i] : 0.f;
    }
  }
}

// Phase B, DCT (see above).  nslots: slots of phase A; A: the wave's C operands.
__device__ void merge_unrotate_dct(const DecodeArgs& a, int64_t seg, MergeSmem& ms, int nslots, const u32x4 (&A)[8],
                                   int lane, int w) {
  const int g = a.g;
  const int hc = lane & 15;  // head column of B and D
  const int kq = lane >> 4;  // k group of B, row group of D
  const int hs = hc < g ? hc : g - 1;
  const float inv = hc < g ? ms.inv[hc] : 0.f;
  // B[kk][h] = R[2 (32 ks + kk) + eo][h] / L[h]: for ks, the lane's 16 channels 64 ks + 16 kq + i
  u32x4 Bv[8];  // [eo * 4 + ks * 2 + part]
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    float v[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float4 t = ((const float4*)(mg_row(ms, 1, 0, nslots, g, hs) + 64 * ks + 16 * kq))[q];
      for (int sl = 1; sl < nslots; ++sl) {
        const float4 u = ((const float4*)(mg_row(ms, 1, sl, nslots, g, hs) + 64 * ks + 16 * kq))[q];
        t.x += u.x;
        t.y += u.y;
        t.z += u.z;
        t.w += u.w;
      }
      v[4 * q] = t.x * inv;
      v[4 * q + 1] = t.y * inv;
      v[4 * q + 2] = t.z * inv;
      v[4 * q + 3] = t.w * inv;
    }
#pragma unroll
    for (int eo = 0; eo < 2; ++eo) {
      uint32_t hi[8], lo[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        uint32_t pp[2];
        split16<KVR_FP16, 2>(v[2 * e + eo], pp);
        hi[e] = pp[0];
        lo[e] = pp[1];
      }
      Bv[eo * 4 + ks * 2] = u32x4{pack2(hi[0], hi[1]), pack2(hi[2], hi[3]), pack2(hi[4], hi[5]), pack2(hi[6], hi[7])};
      Bv[eo * 4 + ks * 2 + 1] = u32x4{pack2(lo[0], lo[1]), pack2(lo[2], lo[3]), pack2(lo[4], lo[5]), pack2(lo[6], lo[7])};
    }
  }
  f32x4 acc[2];
#pragma unroll
  for (int eo = 0; eo < 2; ++eo) {
    acc[eo] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int b = eo * 4 + ks * 2;
      acc[eo] = mfma16_f16(A[b], Bv[b], acc[eo]);
      acc[eo] = mfma16_f16(A[b], Bv[b + 1], acc[eo]);
      acc[eo] = mfma16_f16(A[b + 1], Bv[b], acc[eo]);
    }
  }
  if (hc < g) {
    const int n0 = 16 * w + 4 * kq;  // rows n0 .. n0 + 3, mirrors 127 - n0 .. 124 - n0
    float4 wl = *(const float4*)(mg_row(ms, 0, 0, nslots, g, hc) + n0);
    float4 wh = *(const float4*)(mg_row(ms, 0, 0, nslots, g, hc) + 124 - n0);
    for (int sl = 1; sl < nslots; ++sl) {
      const float4 ul = *(const float4*)(mg_row(ms, 0, sl, nslots, g, hc) + n0);
      const float4 uh = *(const float4*)(mg_row(ms, 0, sl, nslots, g, hc) + 124 - n0);
      wl.x += ul.x; wl.y += ul.y; wl.z += ul.z; wl.w += ul.w;
      wh.x += uh.x; wh.y += uh.y; wh.z += uh.z; wh.w += uh.w;
    }
    const float el[4] = {wl.x, wl.y, wl.z, wl.w}, eh[4] = {wh.w, wh.z, wh.y, wh.x};  // eh[r]: channel 127 - n0 - r
    float yl[4], yh[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float E = acc[0][r] * 0.125f, O = acc[1][r] * 0.125f;
      yl[r] = fmaf(el[r], inv, E + O);
      yh[r] = fmaf(eh[r], inv, E - O);
    }
    const int64_t bq = (seg / a.Hkv) * a.Hq + (seg % a.Hkv) * g + hc;  // b * Hq + head
    store_out4(a, bq * D + n0, yl[0], yl[1], yl[2], yl[3]);
    store_out4(a, bq * D + 124 - n0, yh[3], yh[2], yh[1], yh[0]);
  }
}

// Phase B, Hadamard or none, after a parts-split phase A: wave w takes heads w, w + 4, ...
__device__ void merge_finish_split(const DecodeArgs& a, int64_t seg, MergeSmem& ms, int lane, int w) {
  const int g = a.g;
  for (int hh = w; hh < g; hh += 4) {
    float2 ws = ((const float2*)mg_row(ms, 0, 0, 4, g, hh))[lane];
    float2 rv = ((const float2*)mg_row(ms, 1, 0, 4, g, hh))[lane];
#pragma unroll
    for (int sl = 1; sl < 4; ++sl) {
      const float2 u = ((const float2*)mg_row(ms, 0, sl, 4, g, hh))[lane];
      const float2 t = ((const float2*)mg_row(ms, 1, sl, 4, g, hh))[lane];
      ws.x += u.x;
      ws.y += u.y;
      rv.x += t.x;
      rv.y += t.y;
    }
    if (a.n_rparts > 0 && a.transform == KVR_HADAMARD) hadamard_pair(rv.x, rv.y, lane);
    const float inv = ms.inv[hh];
    const float y0 = (ws.x + rv.x) * inv, y1 = (ws.y + rv.y) * inv;
    const int64_t o = ((seg / a.Hkv) * a.Hq + (seg % a.Hkv) * g + hh) * D + 2 * lane;
    if (a.out_dtype == KVR_FP32) {
      ((float2*)a.out)[o >> 1] = make_float2(y0, y1);
    } else {
      ((uint32_t*)a.out)[o >> 1] = pack2(f32_to_bf16_rne(y0), f32_to_bf16_rne(y1));
    }
  }
}

// The merge of one segment by the block of its last record (all four waves).
__device__ void merge_segment(const DecodeArgs& a, int64_t seg, MergeSmem& ms, float (*xs)[DCT_SCRATCH], int tid) {
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = a.g;
  const bool dct = a.transform == KVR_DCT && a.n_rparts > 0;
  const bool split = g > 4 && g <= 8 && a.n_wparts + a.n_rparts <= 4 * KVR_MERGE_PB;
  if (!dct && !split) {  // one head per wave (and round trip)
    for (int hh = w; hh < g; hh += 4) merge_head(a, seg, hh, lane, xs[w]);
    return;
  }
  int nslots = 4;
  if (split) {
    merge_gather_split<8, KVR_MERGE_PB>(a, seg, ms, lane, w);
  } else {
    nslots = 1;
    for (int hh = w; hh < g; hh += 4) {
      float L, w0, w1, r0, r1;
      merge_sums(a, seg, hh, lane, L, w0, w1, r0, r1);
      ((float2*)mg_row(ms, 0, 0, 1, g, hh))[lane] = make_float2(w0, w1);
      ((float2*)mg_row(ms, 1, 0, 1, g, hh))[lane] = make_float2(r0, r1);
      if (lane == 0) ms.inv[hh] = (L > 0.f) ? 1.f / L : 0.f;
    }
  }
  if (dct) {
    u32x4 A[8];
    dct16_load(w, lane, A);  // in flight across the barrier
    lds_barrier();
    merge_unrotate_dct(a, seg, ms, nslots, A, lane, w);
  } else {
    lds_barrier();
    merge_finish_split(a, seg, ms, lane, w);
  }
}

__global__ __launch_bounds__(64) void merge_kernel(DecodeArgs a) {
  __shared__ float xs[DCT_SCRATCH];
  const int64_t bq = blockIdx.x;  // b * Hq + head
  const int64_t b = bq / a.Hq;
  const int hq = (int)(bq - b * a.Hq);
  const int h = hq / a.g;
  merge_head(a, b * a.Hkv + h, hq - h * a.g, threadIdx.x, xs);
}

// ------------------------------------------------------------------ kernels

// Score item: the query mean is computed in-block (wave 0) while the tile words load;
// with a candidate array the item's tiles are also sorted (wave 0) into its list.
struct ScoreSmem {
  float qs[4][D];  // per wave
  float xs[4][DCT_SCRATCH];
  uint64_t lc[128];
};

template <int T, int QT>
__device__ void score_item(const DecodeArgs& a, int64_t seg, int64_t chunk, int helper_wave, ScoreSmem& sm,
                           uint32_t epoch = CAND_EPOCH_CHAIN) {
  constexpr int TPI = score_tiles_per_item(T);
  const int64_t t0 = chunk * TPI;
  const int64_t t1 = (t0 + TPI < a.n_tiles) ? t0 + TPI : a.n_tiles;
  // every load of the item is issued before any result is used
  // (a value select, not a pointer select: a load through a pointer that may be
  // global or constant is a FLAT load, and a pending FLAT load makes the compiler
  // wait for every outstanding load at the next use of any of them)
  const int32_t lo = a.excl_lo ? a.excl_lo[seg] : 0;
  const int32_t hi = a.excl_hi ? a.excl_hi[seg] : 0;
  // Every wave builds the query mean itself (straight-line loads from L2, issued first:
  // loads complete in issue order, so the prologue runs while the words stream in) and
  // scores its tiles as soon as its own words are in (Hadamard: with no block barrier
  // before the sort).  The sort runs on wave helper_wave (the item number mod 4), so the
  // items resident on a CU spread it over the four SIMDs.
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const bool helper = wv == helper_wave;
  uint32_t qv0[16], qv1[16];
  qbar_load<QT>(a, seg, lane, qv0, qv1);
  DctRegs dt{};
  if (a.transform == KVR_DCT) dt = dct_table_load(lane);  // before the words: no wait on them
  // The rotated mean query: a Hadamard rotation is a few lane exchanges, done by every wave
  // for itself; a DCT is shared out over the four waves (dct_quarter) and met at a barrier.
  auto query = [&]() -> const float* {
    if (a.transform == KVR_DCT) {
      float m0, m1;
      qbar_mean<QT>(a, qv0, qv1, m0, m1);
      dct_table_store(dt, sm.xs[wv], lane);
      dct_quarter(m0, m1, lane, wv, sm.xs[wv], sm.qs[0]);
      __syncthreads();
      return sm.qs[0];
    }
    qbar_finish<QT>(a, qv0, qv1, sm.qs[wv], sm.xs[wv], lane, dt);
    wave_lds_sync();
    return sm.qs[wv];
  };
  if (a.kcount) {  // the count summary: 8 bytes per lane and tile instead of 8 words
    ScoreCounts<T> sc;
    counts_load<T>(a.kcount, seg, a.tile_stride, t0, t1, sc);
    const float* qs = query();
    score_compute_counts<T>(qs, sc, seg, a.n_tiles, t0, t1, lo, hi, a.scores, a.cand ? sm.lc : nullptr);
  } else {
    ScoreWords<T> sw;
    score_load<T>(a.kbits, seg, a.tile_stride, t0, t1, sw);
    const float* qs = query();
    score_compute<T, 0>(qs, sw, seg, a.n_tiles, t0, t1, lo, hi, a.scores, a.cand ? sm.lc : nullptr);
  }
  if (a.cand) {
    __syncthreads();
    if (helper) {
      uint64_t v = sm.lc[lane];
      sort64_desc(v, lane);
      if constexpr (score_cand_slots(T) == 128) {  // the top 64 of 128: sort the halves, merge
        uint64_t u = sm.lc[64 + lane];
        sort64_desc(u, lane);
        const uint64_t ur = ((uint64_t)(uint32_t)__shfl((int)(uint32_t)(u >> 32), 63 - lane, 64) << 32) |
                            (uint64_t)(uint32_t)__shfl((int)(uint32_t)u, 63 - lane, 64);
        v = merge_top64(v, ur, lane);
      }
      cand_put(a.cand + (seg * a.n_chunks_cap + chunk) * 128, lane, v, cand_tag(epoch, seg, (int)chunk));
    }
  }
}

// Launch 1 (selecting): the score items, grid = segments x items.
template <int T, int QT>
__global__ __launch_bounds__(NT) void select_score_kernel(DecodeArgs a) {
  __shared__ ScoreSmem sm;
  const int64_t seg = blockIdx.x / a.n_chunks;
  score_item<T, QT>(a, seg, blockIdx.x - seg * a.n_chunks, (int)(blockIdx.x & 3), sm);
}

// Launch 2: per segment its n_rparts retrieved items (one selected tile per wave)
// followed by its n_wparts window items; the latency-bound retrieved items run
// between the streaming window items.
// The VALU retrieval method's LDS (RetSmem<G4>) allows 2 blocks per CU at G4 = 8 and 1 at
// G4 = 16; the launch bound asks for what fits.
constexpr int attend_min_blocks(int RM, int G4) {
  return RM == 1 ? (G4 >= 16 ? 1 : (G4 >= 8 ? 2 : KVR_ATTEND_WAVES)) : KVR_ATTEND_WAVES;
}
template <int T, int WDT, int QS, int RM, int G4>
__global__ __launch_bounds__(NT, attend_min_blocks(RM, G4)) void attend_kernel(DecodeArgs a) {
  __shared__ union {
    WindowSmem win;
    RetSmem<G4> ret;
    RetMfmaSmem retm;
  } sm;
  const int parts = a.n_rparts + a.n_wparts;
  int64_t seg;
  int p;
  if (KVR_RET_FIRST) {  // blocks [0, BH*n_rparts): retrieved items, then the window items
    const int64_t nr = (int64_t)(gridDim.x / parts) * a.n_rparts;
    if ((int64_t)blockIdx.x < nr) {
      seg = blockIdx.x / a.n_rparts;
      p = (int)(blockIdx.x - seg * a.n_rparts);
    } else {
      const int64_t it = blockIdx.x - nr;
      seg = it / a.n_wparts;
      p = a.n_rparts + (int)(it - seg * a.n_wparts);
    }
  } else {
    seg = blockIdx.x / parts;
    p = (int)(blockIdx.x - seg * parts);
  }
  if (p < a.n_rparts) {
    float* R = rec_ptr(a, seg, p);
    constexpr int QT = (QS == 1) ? WDT : Q_RUNTIME;  // QS == 1: the query has the window's dtype
    if constexpr (RM == 0) retrieved_role_mfma<T, QT>(a, seg, p, sm.retm, R);
    else retrieved_role<T, G4, QT>(a, seg, p, sm.ret, R);
  } else {
    window_item_any<WDT, QS>(a, seg, p - a.n_rparts, sm.win);
  }
}

// ------------------------------------------------------------------ fused step (one launch)

// The selecting decode step as one launch whose blocks are its work items, in block
// order: every score item (segment-major), then the retrieved items, then the window
// items (KVR_STEP_ORDER).  A retrieved item selects from its segment's candidate lists,
// reloading until every entry carries this call's tag (the lists validate themselves,
// see cand_tag): it waits only on score items, which precede it in block order, and
// blocks are dispatched in block order on each XCD, so whatever keeps a score item
// from being dispatched is itself a score item (which never waits) -- the waits end;
// they are bounded anyway.  Each window and retrieved item counts its record into its
// segment; the segment's last record merges the segment, clears its record counter and
// advances its epoch (every item of the segment is done with both).  Partial records
// are stored and loaded at agent scope, and a block waits for its record stores
// (vmcnt 0) before it counts them in.  Every counter is per segment (no device-wide
// hot spot).
//
// Counter region (int32) at offset 0 of every decode workspace, zero before the
// workspace's first call: a header of CTR_HDR words ([CTR_ERR_WORD]: set when a bounded
// wait gives up; sticky), then per segment s < STEP_MAX_SEG its epoch and its records
// done, each in a 128-byte line of its own (counters sharing a line serialise at the
// coherence point under the loads and increments of many blocks).
constexpr int CTR_HDR = 64;    // 256 bytes
constexpr int CTR_STRIDE = KVR_CTR_STRIDE;  // int32 words per counter

__device__ __forceinline__ int ctr_load(const int32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int ctr_add(int32_t* p, int v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ctr_store(int32_t* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct StepSmem {
  union {
    WindowSmem win;
    RetMfmaSmem retm;
    ScoreSmem sc;
    float xs[4][DCT_SCRATCH];  // merge, one head per wave
    MergeSmem mg;              // merge, DCT segments
  } u;
  int last;
};

// The work of one step_kernel block, given its item (chunk >= 0: score item; wp >= 0:
// window item; else retrieved item rp).
template <int T, int WDT, int QS, bool RING>
__device__ __forceinline__ void step_item(const DecodeArgs& a, StepSmem& sm, int64_t it, int64_t seg, int chunk,
                                          int wp, int rp) {
  constexpr int QT = (QS == 1) ? WDT : Q_RUNTIME;  // QS == 1: the query has the window's dtype
  const int tid = threadIdx.x;
  int32_t* epoch = a.ctr + CTR_HDR;                       // [seg * CTR_STRIDE] the segment's epoch
  int32_t* rdone = epoch + STEP_MAX_SEG * CTR_STRIDE;    // [seg * CTR_STRIDE] records done
  if (chunk >= 0) {
    if (chunk >= a.n_chunks) return;  // past the live tiles
    const uint32_t ep = (uint32_t)ctr_load(epoch + seg * CTR_STRIDE) + 1u;  // used when the list is stored
    score_item<T, QT>(a, seg, chunk, (int)(it & 3), sm.u.sc, ep);
    return;
  }
  if (wp >= a.n_wparts) return;  // past the live window
  const int parts = a.n_wparts + a.n_rparts;
  if (wp >= 0) {
    window_item<WDT, QS, RING>(a, seg, wp, sm.u.win);
  } else {
    retrieved_role_mfma<T, QT>(a, seg, rp, sm.u.retm, rec_ptr(a, seg, rp), epoch + seg * CTR_STRIDE);
  }
  wait_vm();  // record stored
  __syncthreads();
  if (tid == 0) sm.last = ctr_add(rdone + seg * CTR_STRIDE, 1) == parts - 1;
  __syncthreads();
  if (sm.last) {
    if (tid == 0) {  // every item of the segment is past its counters
      ctr_add(epoch + seg * CTR_STRIDE, 1);
      ctr_store(rdone + seg * CTR_STRIDE, 0);
    }
    merge_segment(a, seg, sm.u.mg, sm.u.xs, tid);
  }
}

// LIVE: the window is a ring and its length, ring start and tile count of the block's
// segment come from the live state (the grid covers the capacities); else the window is a
// plain run of slots and everything comes from the arguments.  DCT: the transform is the
// DCT; else Hadamard or none -- fixed at compile time, so a launch carries only its own
// rotation code (the kernel's instruction footprint is what its concurrently running roles
// share in the instruction cache).
template <int T, int WDT, int QS, bool DCT, bool LIVE>
__global__ __launch_bounds__(NT, KVR_ATTEND_WAVES) void step_kernel(DecodeArgs a_in) {
  __shared__ StepSmem sm;
  const int64_t S = a_in.n_seg;
  // block -> work item, over the capacities (= the live counts without a live state)
  const int64_t n_score = S * a_in.n_chunks_cap, n_win = S * a_in.n_wparts_cap, n_ret = S * a_in.n_rparts;
  const int64_t it = blockIdx.x;
  int64_t seg;
  int chunk = -1, wp = -1, rp = -1;  // score chunk, window part or retrieved part
  if (it < n_score) {
    seg = it / a_in.n_chunks_cap;
    chunk = (int)(it - seg * a_in.n_chunks_cap);
  } else {
    const int64_t j = it - n_score;
    const int parts_cap = a_in.n_wparts_cap + a_in.n_rparts;
    if (KVR_STEP_ORDER == 2) {
      seg = j / parts_cap;
      const int p = (int)(j - seg * parts_cap);
      if (p < a_in.n_wparts_cap) wp = p;
      else rp = p - a_in.n_wparts_cap;
    } else {
      const bool win = (KVR_STEP_ORDER == 1) ? (j >= n_ret) : (j < n_win);
      const int64_t jj = win ? ((KVR_STEP_ORDER == 1) ? j - n_ret : j) : ((KVR_STEP_ORDER == 1) ? j : j - n_win);
      const int per = win ? a_in.n_wparts_cap : a_in.n_rparts;
      seg = jj / per;
      if (win) wp = (int)(jj - seg * per);
      else rp = (int)(jj - seg * per);
    }
  }
  DecodeArgs a = a_in;
  a.transform = DCT ? KVR_DCT : (a_in.transform == KVR_NONE ? KVR_NONE : KVR_HADAMARD);
  if constexpr (LIVE) {
    // the segment's live counts, clamped to the capacities the grid and buffers were sized for
    const int32_t* ls = a.live + seg * 4;
    const int64_t wl = ls[0], ws = ls[1], nt = ls[2];
    a.win_len = wl < 0 ? 0 : (wl > a_in.win_len ? a_in.win_len : wl);
    a.win_start = (ws < 0 || ws >= a.win_cap) ? 0 : ws;
    a.n_tiles = nt < 0 ? 0 : (nt > a_in.n_tiles ? a_in.n_tiles : nt);
    a.n_chunks = (int)((a.n_tiles + score_tiles_per_item(T) - 1) / score_tiles_per_item(T));
    a.n_wparts = (int)((a.win_len + a.win_span - 1) / a.win_span);
    if (a.n_wparts == 0 && a.n_rparts == 0) a.n_wparts = 1;  // an empty window item still writes the output (zeros)
  }
  step_item<T, WDT, QS, LIVE>(a, sm, it, seg, chunk, wp, rp);
}

// Bytes of the counter region that starts every decode workspace.
size_t counter_bytes() { return (size_t)(CTR_HDR + 2 * STEP_MAX_SEG * CTR_STRIDE) * sizeof(int32_t); }

// Output of segments with neither window tokens nor retrieved tiles: zeros.
__global__ __launch_bounds__(NT) void zero_out_kernel(DecodeArgs a, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * NT + threadIdx.x;
  if (i >= n) return;
  if (a.out_dtype == KVR_FP32) ((float*)a.out)[i] = 0.f;
  else ((uint16_t*)a.out)[i] = 0;
}

// Standalone component kernels ------------------------------------------------

template <int QT, int TF>
__global__ __launch_bounds__(64) void query_prep_kernel(const void* __restrict__ q, int Hq, int Hkv,
                                                        float* __restrict__ qbar_rot,
                                                        float* __restrict__ q_rot) {
  __shared__ float xs[DCT_SCRATCH];
  const int lane = threadIdx.x;
  const int64_t seg = blockIdx.x;
  if (TF == KVR_DCT) dct_table_to_lds(xs, lane);
  const int64_t b = seg / Hkv;
  const int h = (int)(seg - b * Hkv);
  const int g = Hq / Hkv;
  const int64_t q0 = (b * Hq + (int64_t)h * g) * D;
  float m0 = load_as_f32<QT>(q, q0 + 2 * lane);
  float m1 = load_as_f32<QT>(q, q0 + 2 * lane + 1);
  for (int i = 1; i < g; ++i) {
    m0 = m0 + load_as_f32<QT>(q, q0 + (int64_t)i * D + 2 * lane);
    m1 = m1 + load_as_f32<QT>(q, q0 + (int64_t)i * D + 2 * lane + 1);
  }
  m0 = __fdiv_rn(m0, (float)g);
  m1 = __fdiv_rn(m1, (float)g);
  rotate_pair(m0, m1, lane, TF, xs);
  qbar_rot[seg * D + 2 * lane] = m0;
  qbar_rot[seg * D + 2 * lane + 1] = m1;
  if (q_rot) {
    for (int i = 0; i < g; ++i) {
      float v0 = load_as_f32<QT>(q, q0 + (int64_t)i * D + 2 * lane);
      float v1 = load_as_f32<QT>(q, q0 + (int64_t)i * D + 2 * lane + 1);
      rotate_pair(v0, v1, lane, TF, xs);
      q_rot[q0 + (int64_t)i * D + 2 * lane] = v0;
      q_rot[q0 + (int64_t)i * D + 2 * lane + 1] = v1;
    }
  }
}

template <int T, int METHOD>
__global__ __launch_bounds__(NT) void score_kernel(const float* __restrict__ qbar_rot,
                                                   const uint64_t* __restrict__ kbits, int64_t n_tiles,
                                                   int64_t tile_stride, int64_t n_chunks,
                                                   const int32_t* __restrict__ excl_lo,
                                                   const int32_t* __restrict__ excl_hi,
                                                   float* __restrict__ scores) {
  constexpr int TPI = score_tiles_per_item(T);
  __shared__ float qs[D];
  const int64_t seg = blockIdx.x / n_chunks;
  const int64_t chunk = blockIdx.x - seg * n_chunks;
  const int64_t t0 = chunk * TPI;
  const int64_t t1 = (t0 + TPI < n_tiles) ? t0 + TPI : n_tiles;
  ScoreWords<T> sw;
  score_load<T>(kbits, seg, tile_stride, t0, t1, sw);
  if (threadIdx.x < D) qs[threadIdx.x] = qbar_rot[seg * D + threadIdx.x];
  __syncthreads();
  score_compute<T, METHOD>(qs, sw, seg, n_tiles, t0, t1, excl_lo ? excl_lo[seg] : 0,
                           excl_hi ? excl_hi[seg] : 0, scores);
}

__global__ __launch_bounds__(64) void topk_kernel(const float* __restrict__ scores, int64_t n,
                                                  int64_t stride, int k, int32_t* __restrict__ idx) {
  __shared__ TopkSmem sm;
  const int64_t seg = blockIdx.x;
  topk_wave(scores + seg * stride, n, k, idx + seg * k, sm, threadIdx.x);
}

template <int T, int TF>
__global__ __launch_bounds__(64) void gather_tiles_kernel(const uint64_t* __restrict__ bits,
                                                          const uint16_t* __restrict__ scales,
                                                          int64_t tile_stride,
                                                          const int32_t* __restrict__ idx, int k,
                                                          float* __restrict__ out, int64_t oss,
                                                          int64_t ost) {
  constexpr int W = T / 64;
  const int lane = threadIdx.x;
  const int64_t blk = blockIdx.x;  // (seg * k + j) * W + w
  const int w = (int)(blk % W);
  const int64_t sj = blk / W;
  const int64_t seg = sj / k;
  const int j = (int)(sj - seg * k);
  int64_t tile = idx[seg * k + j];
  tile = tile < 0 ? 0 : (tile >= tile_stride ? tile_stride - 1 : tile);  // stay inside the store
  const int64_t slot = seg * tile_stride + tile;
  const float s = f16_to_f32(scales[slot]);
  const uint64_t* wp = bits + slot * (int64_t)(D * W);
  const uint64_t wa = wp[lane * W + w], wc = wp[(lane + 64) * W + w];
  uint32_t a_lo = (uint32_t)wa, a_hi = (uint32_t)(wa >> 32), c_lo = (uint32_t)wc, c_hi = (uint32_t)(wc >> 32);
  transpose64(a_lo, a_hi, lane);
  transpose64(c_lo, c_hi, lane);
  const uint32_t rows[4] = {a_lo, a_hi, c_lo, c_hi};
  float v[D];
#pragma unroll
  for (int ch = 0; ch < D; ++ch) v[ch] = ((rows[ch >> 5] >> (ch & 31)) & 1u) ? s : -s;
  float* dst = out + seg * oss + ((int64_t)j * T + 64 * w + lane) * ost;
  if constexpr (TF == KVR_HADAMARD) {
    fwht128_regs(v);
#pragma unroll
    for (int ch = 0; ch < D; ++ch) dst[ch] = v[ch] * C_HAD;
  } else if constexpr (TF == KVR_DCT) {
#pragma unroll 1
    for (int n2 = 0; n2 < D; ++n2) {
      float acc = 0.f;
#pragma unroll
      for (int kk = 0; kk < D; ++kk) acc = fmaf(g_dct[kk * D + n2], v[kk], acc);
      dst[n2] = acc;
    }
  } else {
#pragma unroll
    for (int ch = 0; ch < D; ++ch) dst[ch] = v[ch];
  }
}

// ------------------------------------------------------------------ host launchers

// Window tokens per window item: one 32-token chunk per wave (128) unless the
// segments x window are large enough to keep >= KVR_WIN_MIN_ITEMS window items with
// longer spans (fewer partial records for the merge); at most 16 chunks per wave.  With
// retrieved tiles (k > 0) a segment's window takes at most KVR_WIN_MAX_PARTS items where
// spans allow: the window items then finish well inside the retrieved items' latency
// chain, and the merge loads fewer records.
int64_t window_span(int64_t BH, int64_t win_len, int k) {
  int64_t s = (BH * win_len) / ((int64_t)WIN_UNIT * KVR_WIN_MIN_ITEMS);
  if (k > 0) {
    const int64_t sp = (win_len + (int64_t)WIN_UNIT * KVR_WIN_MAX_PARTS - 1) / ((int64_t)WIN_UNIT * KVR_WIN_MAX_PARTS);
    s = s > sp ? s : sp;
  }
  s = s < 1 ? 1 : (s > 16 ? 16 : s);
  return s * WIN_UNIT;
}
int n_window_parts(int64_t BH, int64_t win_len, int k) {
  const int64_t span = window_span(BH, win_len, k);
  return (win_len > 0) ? (int)((win_len + span - 1) / span) : 0;
}
constexpr int RET_TILES_PER_BLOCK = KVR_RET_TILES;  // selected tiles per retrieved item
// Selected tiles per retrieved item: KVR_RET_TILES at T = 64, proportionally fewer at
// T = 128 (two 64-token units per tile), so a wave walks about two units either way.
int n_retrieved_parts(int k, int T) {
  const int per = RET_TILES_PER_BLOCK * 64 / T >= 4 ? RET_TILES_PER_BLOCK * 64 / T : 4;
  return (k > 0) ? (k + per - 1) / per : 0;
}

// Partial records in the workspace: one per window item and per retrieved item.
size_t records_bytes(int64_t B, int Hq, int Hkv, int64_t win_len, int k, int T) {
  const int g = Hq / Hkv;
  const int64_t parts = n_window_parts(B * Hkv, win_len, k) + n_retrieved_parts(k, T);
  return (size_t)(B * Hkv * (parts > 0 ? parts : 1) * g * (2 + D)) * sizeof(float);
}

// Sorted per-item candidate lists for the two-level selection (selecting, k <= 64).
size_t cand_bytes(int64_t B, int Hkv, int64_t n_tiles, int k, int T) {
  if (k <= 0 || k > 64 || n_tiles <= 0) return 0;
  const int64_t tpi = score_tiles_per_item(T);
  return (size_t)(B * Hkv * ((n_tiles + tpi - 1) / tpi) * 128) * sizeof(uint64_t);  // 64 entries x 2 tagged halves
}

hipError_t launch_query_prep(int qt, int tf, const void* q, int64_t B, int Hq, int Hkv,
                             float* qbar_rot, float* q_rot, hipStream_t s) {
  const int64_t nblk = B * Hkv;
  if (nblk == 0) return hipSuccess;
#define KVR_QP(QTV, TFV)                                                                        \
  if (qt == QTV && tf == TFV) {                                                                 \
    hipLaunchKernelGGL((query_prep_kernel<QTV, TFV>), dim3((unsigned)nblk), dim3(64), 0, s, q, Hq, \
                       Hkv, qbar_rot, q_rot);                                                   \
    return hipGetLastError();                                                                   \
  }
  KVR_QP(KVR_BF16, KVR_HADAMARD)
  KVR_QP(KVR_FP16, KVR_HADAMARD)
  KVR_QP(KVR_FP32, KVR_HADAMARD)
  KVR_QP(KVR_BF16, KVR_DCT)
  KVR_QP(KVR_FP16, KVR_DCT)
  KVR_QP(KVR_FP32, KVR_DCT)
  KVR_QP(KVR_BF16, KVR_NONE)
  KVR_QP(KVR_FP16, KVR_NONE)
  KVR_QP(KVR_FP32, KVR_NONE)
#undef KVR_QP
  return hipErrorInvalidValue;
}

hipError_t launch_score(int T, int method, const float* qbar_rot, const uint64_t* kbits, int64_t BH,
                        int64_t n_tiles, int64_t tile_stride, const int32_t* excl_lo,
                        const int32_t* excl_hi, float* scores, hipStream_t s) {
  const int64_t tpi = score_tiles_per_item(T);
  const int64_t n_chunks = (n_tiles + tpi - 1) / tpi;
  const int64_t nblk = BH * n_chunks;
  if (nblk == 0) return hipSuccess;
#define KVR_SC(TV, MV)                                                                           \
  if (T == TV && method == MV) {                                                                 \
    hipLaunchKernelGGL((score_kernel<TV, MV>), dim3((unsigned)nblk), dim3(NT), 0, s, qbar_rot, kbits, \
                       n_tiles, tile_stride, n_chunks, excl_lo, excl_hi, scores);                \
    return hipGetLastError();                                                                    \
  }
  KVR_SC(64, 0)
  KVR_SC(64, 1)
  KVR_SC(128, 0)
  KVR_SC(128, 1)
#undef KVR_SC
  return hipErrorInvalidValue;
}

hipError_t launch_topk(const float* scores, int64_t BH, int64_t n, int64_t stride, int k, int32_t* idx,
                       hipStream_t s) {
  if (BH == 0) return hipSuccess;
  hipLaunchKernelGGL(topk_kernel, dim3((unsigned)BH), dim3(64), 0, s, scores, n, stride, k, idx);
  return hipGetLastError();
}

// Retrieved-tile arithmetic: MFMA on unpacked +-1 operands (default) or the VALU
// nibble-table path, the measured alternative; KVR_RETRIEVE_METHOD=valu selects the
// latter (same results within the attention tolerance).  A diagnostic switch, read at
// each launch (a getenv; the tests flip it inside one process).
static int retrieve_method() {
  const char* e = getenv("KVR_RETRIEVE_METHOD");
  return (e && (e[0] == 'v' || e[0] == 'V')) ? 1 : 0;
}

// Whether a decode step with these sizes runs as the one-launch step_kernel (the only
// path that takes a live state).
bool step_is_fused(int64_t BH, int k, bool have_ctr) {
  return KVR_FUSED_STEP && have_ctr && k > 0 && k <= KVR_CAND_MAX && k <= 64 && retrieve_method() == 0 &&
         BH <= STEP_MAX_SEG;
}

// Full decode.  Selecting with candidate lists: one launch (step_kernel).
// Otherwise: [score launch when selecting] -> attend launch (retrieved + window items)
// -> merge launch.  With a live state (fused step only) win_len and n_tiles are the
// capacities; the kernel reads the live values per segment.
hipError_t launch_decode(const DecodeLaunch& L, hipStream_t s) {
  DecodeArgs a{};
  const int64_t B = L.B;
  const int T = L.T;
  a.q = L.q;
  a.q_dtype = L.qt;
  a.Hq = L.Hq;
  a.Hkv = L.Hkv;
  a.g = L.Hq / L.Hkv;
  a.transform = L.tf;
  a.out_dtype = L.ot;
  a.wk = L.wk;
  a.wv = L.wv;
  a.win_len = L.win_len;
  a.win_start = L.win_start;
  a.win_cap = L.win_cap;
  a.live = L.live;
  a.sb = L.sb;
  a.sh = L.sh;
  a.st = L.st;
  a.kbits = L.kb;
  a.vbits = L.vb;
  a.kscale = L.ks;
  a.vscale = L.vs;
  a.kcount = L.kc;
  a.n_tiles = L.n_tiles;
  a.tile_stride = L.tile_stride;
  a.excl_lo = L.excl_lo;
  a.excl_hi = L.excl_hi;
  a.k = L.k;
  a.scores = L.scores;
  a.idx = L.idx;
  a.rec = L.rec;
  a.n_chunks = (int)((L.n_tiles + score_tiles_per_item(T) - 1) / score_tiles_per_item(T));
  a.n_wparts = n_window_parts(B * L.Hkv, L.win_len, L.k);
  a.win_span = window_span(B * L.Hkv, L.win_len, L.k);
  a.n_rparts = n_retrieved_parts(L.k, T);
  a.n_chunks_cap = a.n_chunks;
  a.n_wparts_cap = a.n_wparts;
  a.spin_max = L.spin_max;
  a.wait_fail = L.wait_fail;
  a.do_select = (L.do_select && L.k > 0) ? 1 : 0;
  a.cand = (a.do_select && L.k <= KVR_CAND_MAX && L.k <= 64) ? L.cand : nullptr;
  a.ret_method = retrieve_method();
  a.out = L.out;
  a.ctr = L.ctr;
  a.n_seg = B * L.Hkv;
  const int64_t BH = B * L.Hkv;
  if (BH == 0) return hipSuccess;
  const int wdt = L.wdt, qt = L.qt;
  if (a.n_wparts + a.n_rparts == 0) {
    const int64_t n = B * L.Hq * D;
    hipLaunchKernelGGL(zero_out_kernel, dim3((unsigned)((n + NT - 1) / NT)), dim3(NT), 0, s, a, n);
    return hipGetLastError();
  }
  // the one-launch step takes a ring window exactly when it takes a live state (a ring
  // without one runs the launch chain, whose window role handles both layouts)
  const bool fused = L.do_select && step_is_fused(BH, L.k, L.ctr != nullptr) && a.cand &&
                     ((L.live != nullptr) == (L.win_cap > 0));
  if (L.live && !fused) return hipErrorInvalidValue;  // the host rejects this before launching
  if (fused) {
    a.scores = nullptr;  // the one-launch step keeps no score array
    const int64_t tickets = BH * (a.n_chunks_cap + a.n_wparts_cap + a.n_rparts);  // blocks = work items
    const bool same = (qt == wdt);
#define KVR_ST_L(TV, WV, QSV, DV)                                                                     \
  if (a.live) hipLaunchKernelGGL((step_kernel<TV, WV, QSV, DV, true>), dim3((unsigned)tickets), dim3(NT), 0, s, a); \
  else hipLaunchKernelGGL((step_kernel<TV, WV, QSV, DV, false>), dim3((unsigned)tickets), dim3(NT), 0, s, a);
#define KVR_ST(TV, WV, QSV) \
  if (a.transform == KVR_DCT) { KVR_ST_L(TV, WV, QSV, true) } else { KVR_ST_L(TV, WV, QSV, false) }
#define KVR_ST_Q(TV, WV) \
  if (same) { KVR_ST(TV, WV, 1) } else { KVR_ST(TV, WV, 3) }
    if (T == 64 && wdt == KVR_FP16) { KVR_ST_Q(64, KVR_FP16) }
    else if (T == 64 && wdt == KVR_FP32) { KVR_ST_Q(64, KVR_FP32) }
    else if (T == 64) { KVR_ST_Q(64, KVR_BF16) }
    else if (wdt == KVR_FP16) { KVR_ST_Q(128, KVR_FP16) }
    else if (wdt == KVR_FP32) { KVR_ST_Q(128, KVR_FP32) }
    else { KVR_ST_Q(128, KVR_BF16) }
#undef KVR_ST_Q
#undef KVR_ST
#undef KVR_ST_L
    return hipGetLastError();
  }
  if (a.do_select) {
    const dim3 grid((unsigned)(BH * a.n_chunks));
#define KVR_SS(TV, QTV) \
  if (T == TV && qt == QTV) hipLaunchKernelGGL((select_score_kernel<TV, QTV>), grid, dim3(NT), 0, s, a);
    KVR_SS(64, KVR_BF16)
    KVR_SS(64, KVR_FP16)
    KVR_SS(64, KVR_FP32)
    KVR_SS(128, KVR_BF16)
    KVR_SS(128, KVR_FP16)
    KVR_SS(128, KVR_FP32)
#undef KVR_SS
    if (hipError_t e = hipGetLastError()) return e;
  }
  {
    const dim3 grid((unsigned)(BH * (a.n_wparts + a.n_rparts)));
    const bool same = (qt == wdt);  // the QS = 1 instances take the query in the window dtype
    const int gsel = (a.g <= 4) ? 4 : (a.g <= 8) ? 8 : 16;
#define KVR_ATT(TV, WV, QSV, RMV, G4V) \
  hipLaunchKernelGGL((attend_kernel<TV, WV, QSV, RMV, G4V>), grid, dim3(NT), 0, s, a)
#define KVR_ATT_G(TV, WV, QSV)                        \
  if (a.ret_method == 0) KVR_ATT(TV, WV, QSV, 0, 4);  \
  else if (gsel == 4) KVR_ATT(TV, WV, QSV, 1, 4);     \
  else if (gsel == 8) KVR_ATT(TV, WV, QSV, 1, 8);     \
  else KVR_ATT(TV, WV, QSV, 1, 16);
#define KVR_ATT_Q(TV, WV) \
  if (same) { KVR_ATT_G(TV, WV, 1) } else { KVR_ATT_G(TV, WV, 3) }
    // an fp32 window takes the MFMA retrieval variant only
#define KVR_ATT_F32(TV) \
  if (same) { KVR_ATT(TV, KVR_FP32, 1, 0, 4); } else { KVR_ATT(TV, KVR_FP32, 3, 0, 4); }
    if (T == 64 && wdt == KVR_FP16) { KVR_ATT_Q(64, KVR_FP16) }
    else if (T == 64 && wdt == KVR_FP32) { KVR_ATT_F32(64) }
    else if (T == 64) { KVR_ATT_Q(64, KVR_BF16) }
    else if (wdt == KVR_FP16) { KVR_ATT_Q(128, KVR_FP16) }
    else if (wdt == KVR_FP32) { KVR_ATT_F32(128) }
    else { KVR_ATT_Q(128, KVR_BF16) }
#undef KVR_ATT_F32
#undef KVR_ATT_Q
#undef KVR_ATT_G
#undef KVR_ATT
    if (hipError_t e = hipGetLastError()) return e;
  }
  hipLaunchKernelGGL(merge_kernel, dim3((unsigned)(B * L.Hq)), dim3(64), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_gather(const uint64_t* bits, const uint16_t* scales, int64_t BH, int64_t tile_stride,
                         int T, int tf, const int32_t* idx, int k, float* out, int64_t oss, int64_t ost,
                         hipStream_t s) {
  const int64_t nblk = BH * k * (T / 64);
  if (nblk == 0) return hipSuccess;
  dim3 grid((unsigned)nblk), block(64);
#define KVR_GA(TV, TFV)                                                                            \
  if (T == TV && tf == TFV) {                                                                      \
    hipLaunchKernelGGL((gather_tiles_kernel<TV, TFV>), grid, block, 0, s, bits, scales, tile_stride, \
                       idx, k, out, oss, ost);                                                     \
    return hipGetLastError();                                                                      \
  }
  KVR_GA(64, KVR_HADAMARD)
  KVR_GA(64, KVR_DCT)
  KVR_GA(64, KVR_NONE)
  KVR_GA(128, KVR_HADAMARD)
  KVR_GA(128, KVR_DCT)
  KVR_GA(128, KVR_NONE)
#undef KVR_GA
  return hipErrorInvalidValue;
}

}  // namespace kvr
