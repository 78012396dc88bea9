// Subsystem 1: fused tile encoder (rotation -> per-tile fp16 scale ->
// sigma-delta 1-bit along tokens -> packed channel words).
//
// One 64-lane workgroup per (segment, tile).  Phase A: lane = token, the
// token's 128 channels are loaded into registers and rotated (Hadamard as an
// in-register FWHT in the codec's fixed stage order; DCT-II as a matrix-vector
// product with the matrix in constant memory), then stored transposed into
// LDS as [channel][token].  Phase B: lane = channel pair (lane, lane+64); the
// per-channel |y| sums run sequentially over tokens and feed the fixed
// stride-halving tree, then each lane runs the sigma-delta recurrence for its
// two channels and writes their uint64 words (coalesced, 512 B per store).
//
// Two specialisations below take the common cases: T = 64 with a Hadamard (or no)
// rotation transposes in two 64-channel halves (half the LDS, twice the waves per CU),
// and a DCT of bf16 input rotates on MFMA -- in bulk as a two-stage pipeline of
// rotating and quantising waves over double-buffered LDS (encode_dct_pipe_kernel).
//
// Replaces the int4/int2 packing of RetrievalIndex.batch_append / append
// (modules/kvr_retrieval.py:162-207) with the 1-bit tile codec.
#include "kvr_common.h"
#include "kvr_internal.h"

namespace kvr {

// Loads the 128 channels of one token (16-bit or fp32 input) as fp32.
template <int DT>
__device__ __forceinline__ void load_token(const void* x, int64_t base, float* v) {
  if constexpr (DT == KVR_FP32) {
    const float4* src = (const float4*)((const float*)x + base);
#pragma unroll
    for (int i = 0; i < D / 4; ++i) {
      float4 f = src[i];
      v[4 * i] = f.x;
      v[4 * i + 1] = f.y;
      v[4 * i + 2] = f.z;
      v[4 * i + 3] = f.w;
    }
  } else {
    const uint4* src = (const uint4*)((const uint16_t*)x + base);
#pragma unroll
    for (int i = 0; i < D / 8; ++i) {
      uint4 r = src[i];
      uint32_t w4[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if constexpr (DT == KVR_BF16) {
          v[8 * i + 2 * k] = __uint_as_float(w4[k] << 16);
          v[8 * i + 2 * k + 1] = __uint_as_float(w4[k] & 0xffff0000u);
        } else {
          v[8 * i + 2 * k] = f16_to_f32(w4[k] & 0xffffu);
          v[8 * i + 2 * k + 1] = f16_to_f32(w4[k] >> 16);
        }
      }
    }
  }
}

// LDS hand-off inside the one wave that encodes a tile: a block barrier when the block
// is that wave, else the wave's own LDS completion (the fused append kernel).
template <bool WAVE_SYNC>
__device__ __forceinline__ void tile_sync() {
  if constexpr (WAVE_SYNC) {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
  } else {
    __syncthreads();
  }
}

// Scale and sigma-delta of channels (lane, lane + 64) from their rows y0 / y1 of
// T rotated values, then the tile's words, scale and channel counts.
template <int T>
__device__ __forceinline__ void quantise_pair(const float* y0, const float* y1, float s0, float s1,
                                              uint64_t* out, uint16_t* scale_out, uint8_t* counts_out,
                                              int lane) {
  constexpr int W = T / 64;
  float a = s0 + s1;  // tree step j += j + 64
  a = a + xor_lane_f<32>(a);  // stride-halving tree across lanes, DPP / permlane (no LDS)
  a = a + xor_lane_f<16>(a);
  a = a + xor_lane_f<8>(a);
  a = a + xor_lane_f<4>(a);
  a = a + xor_lane_f<2>(a);
  a = a + xor_lane_f<1>(a);
  float mean = a * (1.0f / (float)(T * D));
  mean = (mean < FP16_MAX) ? mean : FP16_MAX;
  const uint32_t s16 = f32_to_f16_rne(mean);
  const float s32 = f16_to_f32(s16);

  uint32_t w0[2 * W], w1[2 * W];
#pragma unroll
  for (int i = 0; i < 2 * W; ++i) {
    w0[i] = 0u;
    w1[i] = 0u;
  }
  float e0 = 0.f, e1 = 0.f;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    float u0 = y0[t] + e0;
    float u1 = y1[t] + e1;
    bool b0 = u0 >= 0.f;
    bool b1 = u1 >= 0.f;
    e0 = u0 - (b0 ? s32 : -s32);
    e1 = u1 - (b1 ? s32 : -s32);
    w0[t >> 5] |= (uint32_t)b0 << (t & 31);
    w1[t >> 5] |= (uint32_t)b1 << (t & 31);
  }
#pragma unroll
  for (int w = 0; w < W; ++w) {
    out[lane * W + w] = ((uint64_t)w0[2 * w + 1] << 32) | w0[2 * w];
    out[(lane + 64) * W + w] = ((uint64_t)w1[2 * w + 1] << 32) | w1[2 * w];
  }
  if (lane == 0) *scale_out = (uint16_t)s16;
  if (counts_out) {  // set bits of each channel over the tile's T tokens (at most 128)
    int p0 = 0, p1 = 0;
#pragma unroll
    for (int i = 0; i < 2 * W; ++i) {
      p0 += __builtin_popcount(w0[i]);
      p1 += __builtin_popcount(w1[i]);
    }
    counts_out[lane] = (uint8_t)p0;
    counts_out[lane + 64] = (uint8_t)p1;
  }
}

// One tile on one wave, full-tile LDS transpose (ys: D * (T + 1) floats).  Token t of the
// tile is at x[base0 + t * stride_t]; out: the tile's D * T / 64 words; dbg (nullable):
// the tile's [T][128] rotated rows.
template <int DT, int TF, int T, bool WAVE_SYNC>
__device__ __forceinline__ void encode_tile_full(const void* x, int64_t base0, int64_t stride_t, uint64_t* out,
                                                 uint16_t* scale_out, uint8_t* counts_out, float* dbg,
                                                 float* ys, int lane) {
  constexpr int LDW = T + 1;  // padded row: conflict-free column writes and row reads
  constexpr int W = T / 64;
  // ---------------- phase A: lane = token
#pragma unroll 1
  for (int p = 0; p < W; ++p) {
    const int t = p * 64 + lane;
    float v[D];
    load_token<DT>(x, base0 + (int64_t)t * stride_t, v);
    float* drow = dbg ? dbg + (int64_t)t * D : nullptr;
    if constexpr (TF == KVR_DCT) {
#pragma unroll 1
      for (int k = 0; k < D; ++k) {
        const float* c = g_dct + k * D;
        float acc = 0.f;
#pragma unroll
        for (int n = 0; n < D; ++n) acc = fmaf(c[n], v[n], acc);
        ys[k * LDW + t] = acc;
        if (drow) drow[k] = acc;
      }
    } else {
      if constexpr (TF == KVR_HADAMARD) {
        fwht128_regs(v);
#pragma unroll
        for (int j = 0; j < D; ++j) v[j] = v[j] * C_HAD;
      }
#pragma unroll
      for (int j = 0; j < D; ++j) ys[j * LDW + t] = v[j];
      if (drow) {
        float4* d4 = (float4*)drow;
#pragma unroll
        for (int i = 0; i < D / 4; ++i) d4[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
      }
    }
  }
  tile_sync<WAVE_SYNC>();

  // ---------------- phase B: lane = channels (lane, lane + 64)
  const float* y0 = ys + lane * LDW;
  const float* y1 = ys + (lane + 64) * LDW;
  float s0 = 0.f, s1 = 0.f;
#pragma unroll 8
  for (int t = 0; t < T; ++t) {
    s0 = s0 + fabsf(y0[t]);
    s1 = s1 + fabsf(y1[t]);
  }
  quantise_pair<T>(y0, y1, s0, s1, out, scale_out, counts_out, lane);
  tile_sync<WAVE_SYNC>();  // ys is rewritten by a next tile
}

template <int DT, int TF, int T>
__global__ __launch_bounds__(64) void encode_tiles_kernel(
    const void* __restrict__ x, int64_t n_h, int64_t n_tiles, int64_t n_tok, int64_t stride_b,
    int64_t stride_h, int64_t stride_t, uint64_t* __restrict__ bits, uint16_t* __restrict__ scales,
    int64_t out_tile_stride, int64_t out_tile_offset, float* __restrict__ dbg,
    uint8_t* __restrict__ counts) {
  constexpr int W = T / 64;
  __shared__ float ys[D * (T + 1)];
  const int lane = threadIdx.x;
  const int64_t blk = blockIdx.x;
  const int64_t seg = blk / n_tiles;
  const int64_t tile = blk - seg * n_tiles;
  const int64_t b = seg / n_h;
  const int64_t h = seg - b * n_h;
  const int64_t slot = seg * out_tile_stride + out_tile_offset + tile;
  encode_tile_full<DT, TF, T, false>(x, b * stride_b + h * stride_h + tile * T * stride_t, stride_t,
                                     bits + slot * (int64_t)(D * W), scales + slot,
                                     counts ? counts + slot * D : nullptr,
                                     dbg ? dbg + (seg * n_tok + tile * T) * D : nullptr, ys, lane);
}

// T = 64 with a Hadamard or no rotation: the same codec with half the LDS.  Phase A
// (lane = token) rotates the token in registers; its channels 0..63 go through the LDS
// transpose first, and lane c keeps channel c's 64 values in registers (with the first
// half of its |y| sum) while channels 64..127 take the same LDS rows.  The scale's sum
// order is the codec's (per channel sequential over tokens, then j += j + 64 and the
// lane tree), and so is the sigma-delta.  A 16.6 KB transpose lets about nine waves
// share a CU (the full-tile kernel's 33 KB allows four), so one wave's loads run
// while others rotate and quantise.
template <int DT, int TF, bool WAVE_SYNC>
__device__ __forceinline__ void encode_tile64(const void* x, int64_t base0, int64_t stride_t, uint64_t* out,
                                              uint16_t* scale_out, uint8_t* counts_out, float* dbg, float* ys,
                                              int lane) {
  static_assert(TF != KVR_DCT, "the DCT rotation uses the full-tile body");
  constexpr int T = 64;
  constexpr int H = D / 2;     // channels per transpose half
  constexpr int LDW = T + 1;  // padded row: conflict-free column writes and row reads

  // ---------------- phase A: lane = token
  float v[D];
  load_token<DT>(x, base0 + (int64_t)lane * stride_t, v);
  if constexpr (TF == KVR_HADAMARD) {
    fwht128_regs(v);
#pragma unroll
    for (int j = 0; j < D; ++j) v[j] = v[j] * C_HAD;
  }
  if (dbg) {
    float4* d4 = (float4*)(dbg + (int64_t)lane * D);
#pragma unroll
    for (int i = 0; i < D / 4; ++i) d4[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
  }

  // ---------------- channels 0..63: lane c keeps channel c in registers
#pragma unroll
  for (int j = 0; j < H; ++j) ys[j * LDW + lane] = v[j];
  tile_sync<WAVE_SYNC>();
  const float* yr = ys + lane * LDW;
  float y0[T];
  float s0 = 0.f;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    y0[t] = yr[t];
    s0 = s0 + fabsf(y0[t]);
  }
  tile_sync<WAVE_SYNC>();
  // ---------------- channels 64..127 through the same rows
#pragma unroll
  for (int j = 0; j < H; ++j) ys[j * LDW + lane] = v[H + j];
  tile_sync<WAVE_SYNC>();
  float s1 = 0.f;
#pragma unroll 8
  for (int t = 0; t < T; ++t) s1 = s1 + fabsf(yr[t]);
  quantise_pair<T>(y0, yr, s0, s1, out, scale_out, counts_out, lane);
  tile_sync<WAVE_SYNC>();  // ys is rewritten by a next tile
}

// T = 64 with a Hadamard or no rotation: the same codec with half the LDS.  Phase A
// (lane = token) rotates the token in registers; its channels 0..63 go through the LDS
// transpose first, and lane c keeps channel c's 64 values in registers (with the first
// half of its |y| sum) while channels 64..127 take the same LDS rows.  The scale's sum
// order is the codec's (per channel sequential over tokens, then j += j + 64 and the
// lane tree), and so is the sigma-delta.  A 16.6 KB transpose lets about nine waves
// share a CU (the full-tile kernel's 33 KB allows four), so one wave's loads run
// while others rotate and quantise.
template <int DT, int TF>
__global__ __launch_bounds__(64) void encode_tiles64_kernel(
    const void* __restrict__ x, int64_t n_h, int64_t n_tiles, int64_t n_tok, int64_t stride_b,
    int64_t stride_h, int64_t stride_t, uint64_t* __restrict__ bits, uint16_t* __restrict__ scales,
    int64_t out_tile_stride, int64_t out_tile_offset, float* __restrict__ dbg,
    uint8_t* __restrict__ counts) {
  constexpr int T = 64;
  __shared__ float ys[(D / 2) * (T + 1)];
  const int lane = threadIdx.x;
  const int64_t blk = blockIdx.x;
  const int64_t seg = blk / n_tiles;
  const int64_t tile = blk - seg * n_tiles;
  const int64_t b = seg / n_h;
  const int64_t h = seg - b * n_h;
  const int64_t slot = seg * out_tile_stride + out_tile_offset + tile;
  encode_tile64<DT, TF, false>(x, b * stride_b + h * stride_h + tile * T * stride_t, stride_t,
                               bits + slot * (int64_t)D, scales + slot, counts ? counts + slot * D : nullptr,
                               dbg ? dbg + (seg * n_tok + tile * T) * D : nullptr, ys, lane);
}

// DCT-II rotation of bf16 input on MFMA, then the same scale and sigma-delta.  Per tile,
// Y[token][out] = sum_in X[token][in] C[out][in] as v_mfma_f32_16x16x32_bf16 products:
// the input is exact in bf16, and C is split into three bf16 parts (c1 + c2 + c3 carries
// C's fp32 value to about 2^-27 relative), so every product is exact in fp32 and the
// rotation matches C x to fp32 accumulation error (the DCT rotation is held to a
// tolerance; the codec is exact given the rotation the kernel wrote).  Four waves per
// block: wave w owns output channels [32 w, 32 w + 32) and keeps their C operands in
// registers; blocks are persistent over tiles so the split is done once per block.
// Phase A writes Y to LDS as [channel][token]; phase B: threads 0..127 take channel
// tid (per-channel sequential |y| sum, the codec's j += j + 64 then lane tree, then
// the sigma-delta recurrence and the channel's words).
__device__ __forceinline__ f32x4 mfma_bf16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}


// B operands of wave wv: C^T[in 32 ks + 8 kg + e][out 32 wv + 16 mb + n] in three bf16 parts.
struct DctOperands {
  u32x4 cb[2][4][3];
};
__device__ __forceinline__ void dct_operands(DctOperands& o, int wv, int lane) {
  const int n = lane & 15;
  const int kg = lane >> 4;
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      uint32_t hp[3][8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float r = g_dct[(32 * wv + 16 * mb + n) * D + 32 * ks + 8 * kg + e];
#pragma unroll
        for (int p = 0; p < 3; ++p) {
          const uint32_t hb = f32_to_bf16_rne(r);
          hp[p][e] = hb;
          r = r - __uint_as_float(hb << 16);  // exact: r and its bf16 rounding are close
        }
      }
#pragma unroll
      for (int p = 0; p < 3; ++p)
        o.cb[mb][ks][p] = u32x4{hp[p][0] | (hp[p][1] << 16), hp[p][2] | (hp[p][3] << 16),
                                hp[p][4] | (hp[p][5] << 16), hp[p][6] | (hp[p][7] << 16)};
    }
}

struct DctTileSmem {
  float ssum[D];
  float sbc;
};

// One tile on the block's four waves (256 threads): token t of the tile at
// xs[t * stride_t] (bf16), out: the tile's words; dbg (nullable): its [T][128] rows.
template <int T>
__device__ __forceinline__ void encode_tile_dct_mfma(const uint16_t* xs, int64_t stride_t, const DctOperands& o,
                                                     uint64_t* out, uint16_t* scale_out, uint8_t* counts_out,
                                                     float* dbg, float* ys, DctTileSmem& sm) {
  constexpr int LDW = T + 1;  // padded row
  constexpr int W = T / 64;
  constexpr int NBC = 4;      // 16-token blocks per load batch
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int n = lane & 15;   // token row of A, output column of B and D
  const int kg = lane >> 4;  // k group (8 inputs) of A and B, row group of D

  // ---------------- phase A: Y = X C^T into ys[out][token]
#pragma unroll
  for (int nb0 = 0; nb0 < T / 16; nb0 += NBC) {
    u32x4 xa[NBC][4];  // A operands: token 16 nb + n, inputs 32 ks + 8 kg .. + 7
#pragma unroll
    for (int j = 0; j < NBC; ++j) {
      const uint16_t* xr = xs + (int64_t)(16 * (nb0 + j) + n) * stride_t + 8 * kg;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) xa[j][ks] = *(const u32x4*)(xr + 32 * ks);
    }
#pragma unroll
    for (int j = 0; j < NBC; ++j)
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
          for (int p = 0; p < 3; ++p) acc = mfma_bf16(xa[j][ks], o.cb[mb][ks][p], acc);
        // acc[r] = Y[token 16 nb + 4 kg + r][out 32 wv + 16 mb + n]
        const int ch = 32 * wv + 16 * mb + n;
        const int t0 = 16 * (nb0 + j) + 4 * kg;
#pragma unroll
        for (int r = 0; r < 4; ++r) ys[ch * LDW + t0 + r] = acc[r];
        if (dbg) {
#pragma unroll
          for (int r = 0; r < 4; ++r) dbg[(int64_t)(t0 + r) * D + ch] = acc[r];
        }
      }
  }
  __syncthreads();

  // ---------------- phase B: thread c < 128 takes channel c
  const float* yr = ys + tid * LDW;
  if (tid < D) {
    float sa = 0.f;
#pragma unroll 8
    for (int t = 0; t < T; ++t) sa = sa + fabsf(yr[t]);
    sm.ssum[tid] = sa;
  }
  __syncthreads();
  if (wv == 0) {
    float a = sm.ssum[lane] + sm.ssum[lane + 64];  // tree step j += j + 64
    a = a + xor_lane_f<32>(a);
    a = a + xor_lane_f<16>(a);
    a = a + xor_lane_f<8>(a);
    a = a + xor_lane_f<4>(a);
    a = a + xor_lane_f<2>(a);
    a = a + xor_lane_f<1>(a);
    float mean = a * (1.0f / (float)(T * D));
    mean = (mean < FP16_MAX) ? mean : FP16_MAX;
    if (lane == 0) sm.sbc = mean;
  }
  __syncthreads();
  if (tid < D) {
    const uint32_t s16 = f32_to_f16_rne(sm.sbc);
    const float s32 = f16_to_f32(s16);
    uint32_t wd[2 * W];
#pragma unroll
    for (int i = 0; i < 2 * W; ++i) wd[i] = 0u;
    float e = 0.f;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const float u = yr[t] + e;
      const bool bt = u >= 0.f;
      e = u - (bt ? s32 : -s32);
      wd[t >> 5] |= (uint32_t)bt << (t & 31);
    }
#pragma unroll
    for (int w = 0; w < W; ++w) out[tid * W + w] = ((uint64_t)wd[2 * w + 1] << 32) | wd[2 * w];
    if (tid == 0) *scale_out = (uint16_t)s16;
    if (counts_out) {  // set bits of the channel over the tile's T tokens (at most 128)
      int pc = 0;
#pragma unroll
      for (int i = 0; i < 2 * W; ++i) pc += __builtin_popcount(wd[i]);
      counts_out[tid] = (uint8_t)pc;
    }
  }
  __syncthreads();  // ys and sbc are rewritten by the next tile
}

// The bulk DCT encoder (bf16 input): one persistent 384-thread block per CU runs a
// two-stage pipeline over its tiles.  Step i: waves 0..3 rotate tile i on MFMA (wave w:
// output channels 32 w .. 32 w + 31, C operands in registers, as encode_tile_dct_mfma)
// into LDS buffer i % 2, while waves 4 and 5 quantise tile i - 1 from the other buffer
// (each forms all 128 channel |y| sums -- lane: channels lane and lane + 64, two chains --
// so both hold the tile scale without an exchange; then wave 4 + q runs the sigma-delta
// of channels 64 q + lane); one block barrier ends the step.  The rotating waves keep the
// next blocks of 16 tokens in flight while they multiply (a tile's last blocks prefetch
// the next tile's first).  Every operation and its order are those of
// encode_tile_dct_mfma: the same bits, scales and counts.  Measured per step on MI355X:
// the rotation's loads (four waves each load the whole tile) dominate (~5 us of MFMA
// phase against ~1.5 us with the loads taken out); the quantisers need ~4 us (the sums,
// then 128 dependent sigma-delta steps per channel).
constexpr int DCT_PIPE_THREADS = 384;

struct DctPipeTile {
  int64_t base;  // element offset of the tile's token 0 in x
  int64_t slot;  // tile slot in the store
  int64_t dbg;   // element offset of the tile's rotated rows in dbg
};

__device__ __forceinline__ DctPipeTile dct_pipe_tile(int64_t blk, int T, int64_t n_h, int64_t n_tiles, int64_t n_tok,
                                                     int64_t sb, int64_t sh, int64_t st, int64_t ots, int64_t oto) {
  const int64_t seg = blk / n_tiles;
  const int64_t tile = blk - seg * n_tiles;
  const int64_t b = seg / n_h;
  const int64_t h = seg - b * n_h;
  return DctPipeTile{b * sb + h * sh + tile * T * st, seg * ots + oto + tile, (seg * n_tok + tile * T) * D};
}

// A operands of 16 tokens of a tile: token 16 j + n, inputs 32 ks + 8 kg .. + 7.
__device__ __forceinline__ void dct_pipe_load(const uint16_t* xs, int64_t stride_t, int lane, u32x4 (&xa)[4]) {
  const uint16_t* xr = xs + (int64_t)(lane & 15) * stride_t + 8 * (lane >> 4);
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) xa[ks] = *(const u32x4*)(xr + 32 * ks);
}

template <int T, bool DBG>
__global__ __launch_bounds__(DCT_PIPE_THREADS, 1) void encode_dct_pipe_kernel(
    const uint16_t* __restrict__ x, int64_t n_h, int64_t n_tiles, int64_t n_tok, int64_t stride_b,
    int64_t stride_h, int64_t stride_t, uint64_t* __restrict__ bits, uint16_t* __restrict__ scales,
    int64_t out_tile_stride, int64_t out_tile_offset, float* __restrict__ dbg,
    uint8_t* __restrict__ counts, int64_t n_blk) {
  constexpr int LDW = T + 1;      // padded row
  constexpr int W = T / 64;
  constexpr int NBATCH = T / 64;  // 64-token load batches per tile
  __shared__ float ys[2][D * LDW];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t G = gridDim.x;
  const int64_t n_my = (blockIdx.x < n_blk) ? (n_blk - 1 - blockIdx.x) / G + 1 : 0;  // this block's tiles
  auto tile_of = [&](int64_t i) {
    return dct_pipe_tile(blockIdx.x + i * G, T, n_h, n_tiles, n_tok, stride_b, stride_h, stride_t,
                         out_tile_stride, out_tile_offset);
  };

  // The two roles run separate loops (each keeps only its own state in registers); both
  // execute n_my + 1 block barriers, one per step, so every s_barrier of the block is met by
  // all six waves (the hardware barrier counts waves, not code locations).
  if (wv < 4) {  // ---------------- rotating waves
    const int n = lane & 15;
    const int kg = lane >> 4;
    DctOperands o;
    dct_operands(o, wv, lane);
    // A operands of 4 blocks of 16 tokens: block j holds tokens 64 bi + 16 j + .. of batch bi;
    // once a block's products are issued its registers load the same block of the next
    // batch (this tile's next 64 tokens, or the next tile's first), so three blocks of
    // loads are in flight behind every block of products
    u32x4 xa[4][4];
    if (n_my > 0) {
      const int64_t b0 = tile_of(0).base;
#pragma unroll
      for (int j = 0; j < 4; ++j) dct_pipe_load(x + b0 + (int64_t)16 * j * stride_t, stride_t, lane, xa[j]);
    }
    for (int64_t i = 0; i < n_my; ++i) {
      const DctPipeTile tl = tile_of(i);
      const bool has_next = i + 1 < n_my;
      const int64_t next_base = has_next ? tile_of(i + 1).base : 0;
      float* Y = ys[i & 1];
#pragma unroll
      for (int bi = 0; bi < NBATCH; ++bi) {
        const bool more = bi + 1 < NBATCH || has_next;  // a next batch to load
        const int64_t nb = (bi + 1 < NBATCH) ? tl.base + (int64_t)64 * (bi + 1) * stride_t : next_base;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          // the two output blocks' accumulation chains interleaved (each product's
          // predecessor in its chain is two instructions back); per chain the order of
          // encode_tile_dct_mfma
          f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
          for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (int p = 0; p < 3; ++p)
#pragma unroll
              for (int mb = 0; mb < 2; ++mb) acc[mb] = mfma_bf16(xa[j][ks], o.cb[mb][ks][p], acc[mb]);
#pragma unroll
          for (int mb = 0; mb < 2; ++mb) {
            // acc[mb][r] = Y[token 64 bi + 16 j + 4 kg + r][out 32 wv + 16 mb + n]
            const int ch = 32 * wv + 16 * mb + n;
            const int t0 = 64 * bi + 16 * j + 4 * kg;
#pragma unroll
            for (int r = 0; r < 4; ++r) Y[ch * LDW + t0 + r] = acc[mb][r];
            if constexpr (DBG) {
#pragma unroll
              for (int r = 0; r < 4; ++r) dbg[tl.dbg + (int64_t)(t0 + r) * D + ch] = acc[mb][r];
            }
          }
          if (more) dct_pipe_load(x + nb + (int64_t)16 * j * stride_t, stride_t, lane, xa[j]);
          __builtin_amdgcn_sched_barrier(0);  // keeps each block's loads behind its products (one register set)
        }
      }
      __syncthreads();
    }
    __syncthreads();  // the quantisers' last step
  } else {  // ---------------- quantising waves (q = 0, 1)
    const int q = wv - 4;
    for (int64_t i = 0; i <= n_my; ++i) {
      if (i >= 1) {
        const DctPipeTile tl = tile_of(i - 1);
        const float* Y = ys[(i - 1) & 1];
        const float* y0 = Y + lane * LDW;
        const float* y1 = Y + (lane + 64) * LDW;
        float s0 = 0.f, s1 = 0.f;  // the sequential |y| sums of channels lane and lane + 64
#pragma unroll 16
        for (int t = 0; t < T; ++t) {
          s0 = s0 + fabsf(y0[t]);
          s1 = s1 + fabsf(y1[t]);
        }
        float a = s0 + s1;  // tree step j += j + 64, then the lane tree
        a = a + xor_lane_f<32>(a);
        a = a + xor_lane_f<16>(a);
        a = a + xor_lane_f<8>(a);
        a = a + xor_lane_f<4>(a);
        a = a + xor_lane_f<2>(a);
        a = a + xor_lane_f<1>(a);
        float mean = a * (1.0f / (float)(T * D));
        mean = (mean < FP16_MAX) ? mean : FP16_MAX;
        const uint32_t s16 = f32_to_f16_rne(mean);
        const float s32 = f16_to_f32(s16);
        const int c = 64 * q + lane;
        const float* yr = q ? y1 : y0;
        uint64_t* out = bits + tl.slot * (int64_t)(D * W) + c * W;
        float e = 0.f;
        int pc = 0;
#pragma unroll 1
        for (int w = 0; w < W; ++w) {  // one 64-token word at a time (bounded register use)
          uint32_t h[2] = {0u, 0u};
#pragma unroll
          for (int t = 0; t < 64; ++t) {
            const float u = yr[64 * w + t] + e;
            h[t >> 5] |= (uint32_t)(u >= 0.f) << (t & 31);
            // (u >= 0 ? s : -s) as copysign(s, u): u is never -0 (e never is: it starts at +0
            // and x - x rounds to +0), and for a NaN u both give e = u - (+-s), the NaN of u --
            // the same bits, with the bit test off the e chain
            e = u - __builtin_copysignf(s32, u);
          }
          out[w] = ((uint64_t)h[1] << 32) | h[0];
          pc += __builtin_popcount(h[0]) + __builtin_popcount(h[1]);
        }
        if (q == 0 && lane == 0) scales[tl.slot] = (uint16_t)s16;
        if (counts) counts[tl.slot * D + c] = (uint8_t)pc;  // set bits over the tile's T tokens (<= 128)
      }
      __syncthreads();
    }
  }
}

template <int DT, int TF>
static hipError_t launch_encode_t(int T, const void* x, int64_t n_b, int64_t n_h, int64_t n_tok,
                                  int64_t sb, int64_t sh, int64_t st, uint64_t* bits,
                                  uint16_t* scales, int64_t ots, int64_t oto, float* dbg,
                                  uint8_t* counts, hipStream_t s) {
  const int64_t n_tiles = n_tok / T;
  const int64_t nblk = n_b * n_h * n_tiles;
  if (nblk == 0) return hipSuccess;
  dim3 grid((unsigned)nblk), block(64);
  if (DT == KVR_BF16 && TF == KVR_DCT) {
    int dev = 0, n_cu = 0;  // one persistent block per CU (the pipeline's LDS fills the CU)
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu <= 0)
      n_cu = 256;
    const dim3 pgrid((unsigned)(nblk < n_cu ? nblk : n_cu));
#define KVR_DCT_PIPE(TV, DBGV)                                                                               \
  hipLaunchKernelGGL((encode_dct_pipe_kernel<TV, DBGV>), pgrid, dim3(DCT_PIPE_THREADS), 0, s, (const uint16_t*)x, \
                     n_h, n_tiles, n_tok, sb, sh, st, bits, scales, ots, oto, dbg, counts, nblk)
    if (T == 64 && dbg) KVR_DCT_PIPE(64, true);
    else if (T == 64) KVR_DCT_PIPE(64, false);
    else if (dbg) KVR_DCT_PIPE(128, true);
    else KVR_DCT_PIPE(128, false);
#undef KVR_DCT_PIPE
  } else if (T == 64 && TF != KVR_DCT)
    hipLaunchKernelGGL((encode_tiles64_kernel<DT, TF == KVR_DCT ? KVR_NONE : TF>), grid, block, 0, s, x,
                       n_h, n_tiles, n_tok, sb, sh, st, bits, scales, ots, oto, dbg, counts);
  else if (T == 64)
    hipLaunchKernelGGL((encode_tiles_kernel<DT, TF, 64>), grid, block, 0, s, x, n_h, n_tiles, n_tok,
                       sb, sh, st, bits, scales, ots, oto, dbg, counts);
  else
    hipLaunchKernelGGL((encode_tiles_kernel<DT, TF, 128>), grid, block, 0, s, x, n_h, n_tiles,
                       n_tok, sb, sh, st, bits, scales, ots, oto, dbg, counts);
  return hipGetLastError();
}

hipError_t launch_encode(int dt, int tf, int T, const void* x, int64_t n_b, int64_t n_h,
                         int64_t n_tok, int64_t sb, int64_t sh, int64_t st, uint64_t* bits,
                         uint16_t* scales, int64_t ots, int64_t oto, float* dbg, uint8_t* counts,
                         hipStream_t s) {
#define KVR_ENC(DTV, TFV)                                                                       \
  if (dt == DTV && tf == TFV)                                                                   \
    return launch_encode_t<DTV, TFV>(T, x, n_b, n_h, n_tok, sb, sh, st, bits, scales, ots, oto, \
                                     dbg, counts, s);
  KVR_ENC(KVR_BF16, KVR_HADAMARD)
  KVR_ENC(KVR_FP16, KVR_HADAMARD)
  KVR_ENC(KVR_FP32, KVR_HADAMARD)
  KVR_ENC(KVR_BF16, KVR_DCT)
  KVR_ENC(KVR_FP16, KVR_DCT)
  KVR_ENC(KVR_FP32, KVR_DCT)
  KVR_ENC(KVR_FP32, KVR_NONE)
#undef KVR_ENC
  return hipErrorInvalidValue;
}

// ---------------------------------------------------------------- ring append

// One token per segment into a ring window of W + T slots, and, when that fills the
// ring, the oldest T tokens (the T slots from the ring start: contiguous, the start is
// a multiple of T) into the next tile slot of the K and V stores -- with the same tile
// bodies, hence the same bits, as kvr_encode_tiles.  One 256-thread block per segment;
// the segment's state {n, start, n_tiles, error} is read at the start and written by
// thread 0 at the end, so no other block touches it.  The new token's slot is never in
// the evicted tile (W >= T).  Invalid states and a full store set the sticky error
// field and write nothing out of bounds.
template <int WDT, int TF, int T>
__global__ __launch_bounds__(256) void cache_append_kernel(AppendLaunch p) {
  constexpr bool DCT_MFMA = (WDT == KVR_BF16 && TF == KVR_DCT);
  constexpr bool E64 = (T == 64 && TF != KVR_DCT);
  constexpr int W = T / 64;
  constexpr int YS = E64 ? (D / 2) * (T + 1) : D * (T + 1);
  __shared__ float ys[YS];
  __shared__ DctTileSmem dsm;
  const int tid = threadIdx.x;
  const int64_t seg = blockIdx.x;
  const int64_t b = seg / p.Hkv;
  const int64_t h = seg - b * p.Hkv;
  int32_t* st = p.state + seg * 4;
  const int64_t n = st[0], start = st[1], nt = st[2];
  const int64_t cap = p.W + T;
  if (n < 0 || n >= cap || start < 0 || start >= cap || start % T != 0 || nt < 0) {
    if (tid == 0) st[3] = 1;  // invalid state: nothing written
    return;
  }
  int64_t slot = start + n;
  slot = slot >= cap ? slot - cap : slot;
  const int64_t wbase = b * p.sb + h * p.sh;
  {  // the new token: threads 0..127 K channel tid, 128..255 V channel tid - 128
    const int j = tid & (D - 1);
    const void* src = (tid < D) ? p.k_new : p.v_new;
    void* dst = (tid < D) ? p.wk : p.wv;
    const float x = load_as_f32(src, p.ndt, seg * D + j);
    const int64_t o = wbase + slot * p.st + j;
    if constexpr (WDT == KVR_FP32) ((float*)dst)[o] = x;
    else if constexpr (WDT == KVR_BF16) ((uint16_t*)dst)[o] = (uint16_t)f32_to_bf16_rne(x);
    else ((uint16_t*)dst)[o] = (uint16_t)f32_to_f16_rne(x);
  }
  const bool evict = (n + 1 == cap);
  const bool room = nt < p.tile_stride;
  if (evict && room) {
    const int64_t tslot = seg * p.tile_stride + nt;
    const int64_t src0 = wbase + start * p.st;
    uint8_t* kc = p.kc ? p.kc + tslot * D : nullptr;
    if constexpr (DCT_MFMA) {
      DctOperands o;
      dct_operands(o, tid >> 6, tid & 63);
      encode_tile_dct_mfma<T>((const uint16_t*)p.wk + src0, p.st, o, p.kb + tslot * (int64_t)(D * W), p.ks + tslot,
                              kc, nullptr, ys, dsm);
      encode_tile_dct_mfma<T>((const uint16_t*)p.wv + src0, p.st, o, p.vb + tslot * (int64_t)(D * W), p.vs + tslot,
                              nullptr, nullptr, ys, dsm);
    } else if (tid < 64) {  // wave 0: the K tile, then the V tile through the same LDS
      if constexpr (E64) {
        encode_tile64<WDT, TF, true>(p.wk, src0, p.st, p.kb + tslot * (int64_t)D, p.ks + tslot, kc, nullptr, ys, tid);
        encode_tile64<WDT, TF, true>(p.wv, src0, p.st, p.vb + tslot * (int64_t)D, p.vs + tslot, nullptr, nullptr, ys,
                                     tid);
      } else {
        encode_tile_full<WDT, TF, T, true>(p.wk, src0, p.st, p.kb + tslot * (int64_t)(D * W), p.ks + tslot, kc,
                                           nullptr, ys, tid);
        encode_tile_full<WDT, TF, T, true>(p.wv, src0, p.st, p.vb + tslot * (int64_t)(D * W), p.vs + tslot, nullptr,
                                           nullptr, ys, tid);
      }
    }
  }
  __syncthreads();  // every thread has read the state
  if (tid == 0) {
    if (evict) {
      st[0] = (int32_t)p.W;
      st[1] = (int32_t)(start + T >= cap ? start + T - cap : start + T);
      st[2] = (int32_t)(room ? nt + 1 : nt);
      if (!room) st[3] = 2;  // the store was full: the evicted tile is lost
    } else {
      st[0] = (int32_t)(n + 1);
    }
  }
}

hipError_t launch_append(const AppendLaunch& L, hipStream_t s) {
  const int64_t nseg = L.B * L.Hkv;
  if (nseg == 0) return hipSuccess;
  const dim3 grid((unsigned)nseg), block(256);
#define KVR_AP(WV, TFV, TV)                                                     \
  if (L.wdt == WV && L.tf == TFV && L.T == TV) {                                \
    hipLaunchKernelGGL((cache_append_kernel<WV, TFV, TV>), grid, block, 0, s, L); \
    return hipGetLastError();                                                   \
  }
#define KVR_AP_T(WV, TFV) KVR_AP(WV, TFV, 64) KVR_AP(WV, TFV, 128)
  KVR_AP_T(KVR_BF16, KVR_HADAMARD)
  KVR_AP_T(KVR_FP16, KVR_HADAMARD)
  KVR_AP_T(KVR_FP32, KVR_HADAMARD)
  KVR_AP_T(KVR_BF16, KVR_DCT)
  KVR_AP_T(KVR_FP16, KVR_DCT)
  KVR_AP_T(KVR_FP32, KVR_DCT)
#undef KVR_AP_T
#undef KVR_AP
  return hipErrorInvalidValue;
}

}  // namespace kvr
