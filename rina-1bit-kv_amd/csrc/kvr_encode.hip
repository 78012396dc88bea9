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
// and a DCT of bf16 input rotates on MFMA.
//
// Replaces the int4/int2 packing of RetrievalIndex.batch_append / append
// (modules/kvr_retrieval.py:162-207) with the 1-bit tile codec.
#include "kvr_common.h"

namespace kvr {

template <int DT, int TF, int T>
__global__ __launch_bounds__(64) void encode_tiles_kernel(
    const void* __restrict__ x, int64_t n_h, int64_t n_tiles, int64_t n_tok, int64_t stride_b,
    int64_t stride_h, int64_t stride_t, uint64_t* __restrict__ bits, uint16_t* __restrict__ scales,
    int64_t out_tile_stride, int64_t out_tile_offset, float* __restrict__ dbg,
    uint8_t* __restrict__ counts) {
  constexpr int LDW = T + 1;  // padded row: conflict-free column writes and row reads
  constexpr int W = T / 64;
  __shared__ float ys[D * LDW];

  const int lane = threadIdx.x;
  const int64_t blk = blockIdx.x;
  const int64_t seg = blk / n_tiles;
  const int64_t tile = blk - seg * n_tiles;
  const int64_t b = seg / n_h;
  const int64_t h = seg - b * n_h;

  // ---------------- phase A: lane = token
#pragma unroll 1
  for (int p = 0; p < W; ++p) {
    const int t = p * 64 + lane;
    const int64_t tok = tile * T + t;
    const int64_t base = b * stride_b + h * stride_h + tok * stride_t;
    float v[D];
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
    float* drow = dbg ? dbg + (seg * n_tok + tok) * D : nullptr;
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
  __syncthreads();

  // ---------------- phase B: lane = channels (lane, lane + 64)
  const float* y0 = ys + lane * LDW;
  const float* y1 = ys + (lane + 64) * LDW;
  float s0 = 0.f, s1 = 0.f;
#pragma unroll 8
  for (int t = 0; t < T; ++t) {
    s0 = s0 + fabsf(y0[t]);
    s1 = s1 + fabsf(y1[t]);
  }
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

  const int64_t slot = seg * out_tile_stride + out_tile_offset + tile;
  uint64_t* out = bits + slot * (int64_t)(D * W);
#pragma unroll
  for (int w = 0; w < W; ++w) {
    out[lane * W + w] = ((uint64_t)w0[2 * w + 1] << 32) | w0[2 * w];
    out[(lane + 64) * W + w] = ((uint64_t)w1[2 * w + 1] << 32) | w1[2 * w];
  }
  if (lane == 0) scales[slot] = (uint16_t)s16;
  if (counts) {  // set bits of each channel over the tile's T tokens (at most 128)
    int p0 = 0, p1 = 0;
#pragma unroll
    for (int i = 0; i < 2 * W; ++i) {
      p0 += __builtin_popcount(w0[i]);
      p1 += __builtin_popcount(w1[i]);
    }
    counts[slot * D + lane] = (uint8_t)p0;
    counts[slot * D + lane + 64] = (uint8_t)p1;
  }
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
  static_assert(TF != KVR_DCT, "the DCT rotation uses the full-tile kernel");
  constexpr int T = 64;
  constexpr int H = D / 2;     // channels per transpose half
  constexpr int LDW = T + 1;  // padded row: conflict-free column writes and row reads
  __shared__ float ys[H * LDW];

  const int lane = threadIdx.x;
  const int64_t blk = blockIdx.x;
  const int64_t seg = blk / n_tiles;
  const int64_t tile = blk - seg * n_tiles;
  const int64_t b = seg / n_h;
  const int64_t h = seg - b * n_h;

  // ---------------- phase A: lane = token
  const int64_t tok = tile * T + lane;
  const int64_t base = b * stride_b + h * stride_h + tok * stride_t;
  float v[D];
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
  if constexpr (TF == KVR_HADAMARD) {
    fwht128_regs(v);
#pragma unroll
    for (int j = 0; j < D; ++j) v[j] = v[j] * C_HAD;
  }
  if (dbg) {
    float4* d4 = (float4*)(dbg + (seg * n_tok + tok) * D);
#pragma unroll
    for (int i = 0; i < D / 4; ++i) d4[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
  }

  // ---------------- channels 0..63: lane c keeps channel c in registers
#pragma unroll
  for (int j = 0; j < H; ++j) ys[j * LDW + lane] = v[j];
  __syncthreads();
  const float* yr = ys + lane * LDW;
  float y0[T];
  float s0 = 0.f;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    y0[t] = yr[t];
    s0 = s0 + fabsf(y0[t]);
  }
  __syncthreads();
  // ---------------- channels 64..127 through the same rows
#pragma unroll
  for (int j = 0; j < H; ++j) ys[j * LDW + lane] = v[H + j];
  __syncthreads();
  float s1 = 0.f;
#pragma unroll 8
  for (int t = 0; t < T; ++t) s1 = s1 + fabsf(yr[t]);

  float a = s0 + s1;  // tree step j += j + 64
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

  uint32_t w0[2] = {0u, 0u}, w1[2] = {0u, 0u};
  float e0 = 0.f, e1 = 0.f;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    float u0 = y0[t] + e0;
    float u1 = yr[t] + e1;
    bool b0 = u0 >= 0.f;
    bool b1 = u1 >= 0.f;
    e0 = u0 - (b0 ? s32 : -s32);
    e1 = u1 - (b1 ? s32 : -s32);
    w0[t >> 5] |= (uint32_t)b0 << (t & 31);
    w1[t >> 5] |= (uint32_t)b1 << (t & 31);
  }

  const int64_t slot = seg * out_tile_stride + out_tile_offset + tile;
  uint64_t* out = bits + slot * (int64_t)D;
  out[lane] = ((uint64_t)w0[1] << 32) | w0[0];
  out[lane + 64] = ((uint64_t)w1[1] << 32) | w1[0];
  if (lane == 0) scales[slot] = (uint16_t)s16;
  if (counts) {  // set bits of each channel over the tile's 64 tokens
    counts[slot * D + lane] = (uint8_t)(__builtin_popcount(w0[0]) + __builtin_popcount(w0[1]));
    counts[slot * D + lane + 64] = (uint8_t)(__builtin_popcount(w1[0]) + __builtin_popcount(w1[1]));
  }
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

constexpr int DCT_ENC_BLOCKS = 512;  // persistent blocks (two per CU: 66 KB of LDS each at T = 128)

template <int T>
__global__ __launch_bounds__(256, 2) void encode_dct_mfma_kernel(
    const uint16_t* __restrict__ x, int64_t n_h, int64_t n_tiles, int64_t n_tok, int64_t stride_b,
    int64_t stride_h, int64_t stride_t, uint64_t* __restrict__ bits, uint16_t* __restrict__ scales,
    int64_t out_tile_stride, int64_t out_tile_offset, float* __restrict__ dbg,
    uint8_t* __restrict__ counts, int64_t n_blk) {
  constexpr int LDW = T + 1;  // padded row
  constexpr int W = T / 64;
  constexpr int NBC = 4;      // 16-token blocks per load batch
  __shared__ float ys[D * LDW];
  __shared__ float ssum[D];
  __shared__ float sbc;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int n = lane & 15;   // token row of A, output column of B and D
  const int kg = lane >> 4;  // k group (8 inputs) of A and B, row group of D

  // B operands: C^T[in 32 ks + 8 kg + e][out 32 wv + 16 mb + n] in three bf16 parts
  u32x4 cb[2][4][3];
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
        cb[mb][ks][p] = u32x4{hp[p][0] | (hp[p][1] << 16), hp[p][2] | (hp[p][3] << 16),
                              hp[p][4] | (hp[p][5] << 16), hp[p][6] | (hp[p][7] << 16)};
    }

  for (int64_t blk = blockIdx.x; blk < n_blk; blk += gridDim.x) {
    const int64_t seg = blk / n_tiles;
    const int64_t tile = blk - seg * n_tiles;
    const int64_t b = seg / n_h;
    const int64_t h = seg - b * n_h;
    const uint16_t* xs = x + b * stride_b + h * stride_h;

    // ---------------- phase A: Y = X C^T into ys[out][token]
#pragma unroll
    for (int nb0 = 0; nb0 < T / 16; nb0 += NBC) {
      u32x4 xa[NBC][4];  // A operands: token 16 nb + n, inputs 32 ks + 8 kg .. + 7
#pragma unroll
      for (int j = 0; j < NBC; ++j) {
        const uint16_t* xr = xs + (tile * T + 16 * (nb0 + j) + n) * stride_t + 8 * kg;
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
            for (int p = 0; p < 3; ++p) acc = mfma_bf16(xa[j][ks], cb[mb][ks][p], acc);
          // acc[r] = Y[token 16 nb + 4 kg + r][out 32 wv + 16 mb + n]
          const int ch = 32 * wv + 16 * mb + n;
          const int t0 = 16 * (nb0 + j) + 4 * kg;
#pragma unroll
          for (int r = 0; r < 4; ++r) ys[ch * LDW + t0 + r] = acc[r];
          if (dbg) {
#pragma unroll
            for (int r = 0; r < 4; ++r) dbg[(seg * n_tok + tile * T + t0 + r) * D + ch] = acc[r];
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
      ssum[tid] = sa;
    }
    __syncthreads();
    if (wv == 0) {
      float a = ssum[lane] + ssum[lane + 64];  // tree step j += j + 64
      a = a + xor_lane_f<32>(a);
      a = a + xor_lane_f<16>(a);
      a = a + xor_lane_f<8>(a);
      a = a + xor_lane_f<4>(a);
      a = a + xor_lane_f<2>(a);
      a = a + xor_lane_f<1>(a);
      float mean = a * (1.0f / (float)(T * D));
      mean = (mean < FP16_MAX) ? mean : FP16_MAX;
      if (lane == 0) sbc = mean;
    }
    __syncthreads();
    if (tid < D) {
      const uint32_t s16 = f32_to_f16_rne(sbc);
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
      const int64_t slot = seg * out_tile_stride + out_tile_offset + tile;
      uint64_t* out = bits + slot * (int64_t)(D * W);
#pragma unroll
      for (int w = 0; w < W; ++w) out[tid * W + w] = ((uint64_t)wd[2 * w + 1] << 32) | wd[2 * w];
      if (tid == 0) scales[slot] = (uint16_t)s16;
      if (counts) {  // set bits of the channel over the tile's T tokens (at most 128)
        int pc = 0;
#pragma unroll
        for (int i = 0; i < 2 * W; ++i) pc += __builtin_popcount(wd[i]);
        counts[slot * D + tid] = (uint8_t)pc;
      }
    }
    __syncthreads();  // ys and sbc are rewritten by the next tile
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
    const dim3 pgrid((unsigned)(nblk < DCT_ENC_BLOCKS ? nblk : DCT_ENC_BLOCKS));
    if (T == 64)
      hipLaunchKernelGGL(encode_dct_mfma_kernel<64>, pgrid, dim3(256), 0, s, (const uint16_t*)x, n_h, n_tiles,
                         n_tok, sb, sh, st, bits, scales, ots, oto, dbg, counts, nblk);
    else
      hipLaunchKernelGGL(encode_dct_mfma_kernel<128>, pgrid, dim3(256), 0, s, (const uint16_t*)x, n_h, n_tiles,
                         n_tok, sb, sh, st, bits, scales, ots, oto, dbg, counts, nblk);
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

}  // namespace kvr
