// Subsystem 4: fused window + retrieved-tile decode attention (split-K with a
// log-sum-exp merge), plus the materialising tile gather.
//
// Partial records: for each segment s = b*Hkv + h and part p, a record of
// g*(2+128) floats: m2[g] (running max in log2 units), l[g], o[g][128].
// Window parts hold o in the original domain, retrieved parts in the rotated
// domain; the merge rotates the retrieved sum back once per head.
//
// Window part (MFMA, gfx950 v_mfma_f32_16x16x32_{bf16,f16}):
//   S^T[16 tokens x 16 heads] = K[16 x 32 dims] * Q^T[32 dims x 16 heads]
//   O^T[16 dims x 16 heads]  += V^T[16 dims x 32 tokens] * P^T[32 tokens x 16 heads]
//   Heads are the N dimension (g <= 16, zero padded).  K comes straight from
//   HBM as the A operand (16 B per lane).  The S^T accumulators of a 32-token
//   chunk are exactly the P^T operand of the PV product (the token <-> k-slot
//   assignment of the PV contraction is chosen to match), so P never moves.
//   V is staged through LDS and repacked with v_perm.  fp32 Q / P are split
//   into 2-3 bf16 (or fp16) parts to keep fp32-level accuracy.
// Retrieved part (VALU bit-unpack):
//   keys/values of a token are s*(2b-1) per rotated channel.  A 64x64 bit
//   transpose across lanes turns channel words into token rows; logits use a
//   nibble lookup table of partial sums of q' (32 channel nibbles x 16
//   patterns x heads, in LDS); PV uses a per-tile nibble table of partial sums
//   of p over 4 tokens, applied to the channel words directly.
//
// Reference behaviour followed: one joint softmax over window and retrieved
// tokens, scale 1/sqrt(d), GQA by head groups (modules/kvr_hook.py:274-282,
// online-softmax form of modules/kvr_triton.py:56-79).
#include "kvr_common.h"

namespace kvr {

constexpr float SCALE_LOG2 = 0.08838834764831845f * LOG2E;  // log2(e) / sqrt(128)

__device__ __forceinline__ float safe_exp2(float x) { return exp2f(x); }

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

// Split an fp32 value into NS 16-bit parts of the window's MFMA type whose
// sum reproduces it to ~8*NS mantissa bits.  bf16: truncation (remainders are
// exact); fp16: round to nearest.
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

// ------------------------------------------------------------------ window attention

constexpr int WIN_THREADS = 256;
constexpr int WIN_CHUNK = 32;
constexpr int VROW = D + 8;  // bf16 elements per staged V row (16 B pad)

template <int QT, int WDT, int QS, int PS>
__global__ __launch_bounds__(WIN_THREADS) void window_attn_kernel(
    const void* __restrict__ q, int Hq, int Hkv, const uint16_t* __restrict__ wk,
    const uint16_t* __restrict__ wv, int64_t win_len, int64_t sb, int64_t sh, int64_t st,
    int64_t span, int n_wparts, int n_parts, float* __restrict__ rec) {
  __shared__ __attribute__((aligned(16))) uint16_t vstage[4][WIN_CHUNK * VROW];
  __shared__ float cm[4][16], cl[4][16];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv_id = tid >> 6;
  const int n = lane & 15;   // head column
  const int kg = lane >> 4;  // k-slot group
  const int g = Hq / Hkv;
  const int64_t seg = blockIdx.x / n_wparts;  // grid = segments x window parts
  const int part = (int)(blockIdx.x - seg * n_wparts);
  const int64_t b = seg / Hkv;
  const int64_t h = seg - b * Hkv;

  // ---- Q^T operand: lane (head n, kg) holds Q[n][32ks + 8kg + e], split in QS parts
  u32x4 qb[QS][4];
  {
    const int64_t qoff = (b * Hq + h * g + n) * D;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      uint32_t pe[QS][8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float x = (n < g) ? load_as_f32<QT>(q, qoff + 32 * ks + 8 * kg + e) : 0.f;
        uint32_t p[QS];
        split16<WDT, QS>(x, p);
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

  const uint16_t* kbase = wk + b * sb + h * sh;
  const uint16_t* vbase = wv + b * sb + h * sh;
  const int64_t t_begin = (int64_t)part * span;
  int64_t t_end = t_begin + span;
  if (t_end > win_len) t_end = win_len;
  uint16_t* vs = vstage[wv_id];

  for (int64_t c0 = t_begin + (int64_t)wv_id * WIN_CHUNK; c0 < t_end; c0 += 4 * WIN_CHUNK) {
    // ---- loads: K as the A operand, V rows for staging
    u32x4 ka[2][4];
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
      int64_t tok = c0 + 16 * tb + n;
      tok = tok < win_len ? tok : win_len - 1;
      const uint16_t* kr = kbase + tok * st + 8 * kg;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) ka[tb][ks] = *(const u32x4*)(kr + 32 * ks);
    }
    u32x4 vr[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      int64_t tok = c0 + 4 * i + kg;
      tok = tok < win_len ? tok : win_len - 1;
      vr[i] = *(const u32x4*)(vbase + tok * st + 8 * n);
    }

    // ---- S^T = K Q^T
    f32x4 s[2];
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
      s[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int sp = 0; sp < QS; ++sp) s[tb] = mfma16<WDT>(ka[tb][ks], qb[sp][ks], s[tb]);
    }

    // ---- stage V rows: row 4i+kg, columns 8n..8n+7
#pragma unroll
    for (int i = 0; i < 8; ++i) *(u32x4*)(vs + (4 * i + kg) * VROW + 8 * n) = vr[i];

    // ---- online softmax (head n is lane-local; tokens spread over e and kg)
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
    cmax = fmaxf(cmax, shfl_xor_f(cmax, 16));
    cmax = fmaxf(cmax, shfl_xor_f(cmax, 32));
    const float m_new = fmaxf(m_run, cmax);
    const float m_use = (m_new == -__builtin_inff()) ? 0.f : m_new;
    const float alpha = safe_exp2(m_run - m_use);
    m_run = m_new;
    float p[8];
    float psum = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      p[e] = safe_exp2(l2[e] - m_use);
      psum += p[e];
    }
    l_run = l_run * alpha + psum;
#pragma unroll
    for (int i = 0; i < 8; ++i) oacc[i] = oacc[i] * alpha;

    // ---- P^T operand (B): lane (head n, kg) slot e <-> token 16(e>>2) + 4kg + (e&3)
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

    // ---- V^T operand (A): lane (row m = n, kg); block i row m <-> dim 8m + i
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    u32x4 rv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int trow = 16 * (e >> 2) + 4 * kg + (e & 3);
      rv[e] = *(const u32x4*)(vs + trow * VROW + 8 * n);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t sel = (i & 1) ? 0x07060302u : 0x05040100u;
      u32x4 a;
#pragma unroll
      for (int j = 0; j < 4; ++j) a[j] = __builtin_amdgcn_perm(rv[2 * j + 1][i >> 1], rv[2 * j][i >> 1], sel);
#pragma unroll
      for (int sp = 0; sp < PS; ++sp) oacc[i] = mfma16<WDT>(a, pb[sp], oacc[i]);
    }
    __builtin_amdgcn_wave_barrier();
  }

  // ---- reduce l over kg lanes (same head, same m_run)
  l_run += shfl_xor_f(l_run, 16);
  l_run += shfl_xor_f(l_run, 32);

  // ---- combine the 4 waves: record m2, l, o for heads < g
  if (kg == 0) {
    cm[wv_id][n] = m_run;
    cl[wv_id][n] = l_run;
  }
  __syncthreads();  // every wave is past its last read of vstage
  float mx = -__builtin_inff();
#pragma unroll
  for (int w = 0; w < 4; ++w) mx = fmaxf(mx, cm[w][n]);
  const float fw = safe_exp2(m_run - ((mx == -__builtin_inff()) ? 0.f : mx));
  float* ost = (float*)&vstage[0][0];  // [16 heads][128 dims] fp32 = 8 KB
  for (int i = tid; i < 16 * D; i += WIN_THREADS) ost[i] = 0.f;
  __syncthreads();
#pragma unroll 1
  for (int w = 0; w < 4; ++w) {
    if (wv_id == w && n < g) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) ost[n * D + 32 * kg + 8 * r + i] += oacc[i][r] * fw;
    }
    __syncthreads();
  }
  float* R = rec + (seg * n_parts + part) * (int64_t)(g * (2 + D));
  if (tid < g) {
    float mh = -__builtin_inff();
#pragma unroll
    for (int w = 0; w < 4; ++w) mh = fmaxf(mh, cm[w][tid]);
    const float muh = (mh == -__builtin_inff()) ? 0.f : mh;
    float lt = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) lt += cl[w][tid] * safe_exp2(cm[w][tid] - muh);
    R[tid] = mh;
    R[g + tid] = lt;
  }
  for (int i = tid; i < g * D; i += WIN_THREADS) R[2 * g + i] = ost[i];
}

// ------------------------------------------------------------------ bit transpose

// 64x64 bit-matrix transpose across the wave: lane l holds row l (bit c = element
// (l, c)); afterwards lane c holds column c (bit l = element (l, c)).
__device__ __forceinline__ void transpose64(uint32_t& lo, uint32_t& hi, int lane) {
  {
    const bool up = lane & 32;
    const uint32_t recv = shfl_xor_u(up ? lo : hi, 32);
    if (up) lo = recv;
    else hi = recv;
  }
#define KVR_TSTAGE(S, M)                                                          \
  {                                                                               \
    const uint32_t plo = shfl_xor_u(lo, S), phi = shfl_xor_u(hi, S);              \
    if (lane & S) {                                                               \
      lo = (lo & ~(M)) | ((plo >> S) & (M));                                      \
      hi = (hi & ~(M)) | ((phi >> S) & (M));                                      \
    } else {                                                                      \
      lo = (lo & (M)) | ((plo & (M)) << S);                                       \
      hi = (hi & (M)) | ((phi & (M)) << S);                                       \
    }                                                                             \
  }
  KVR_TSTAGE(16, 0x0000ffffu)
  KVR_TSTAGE(8, 0x00ff00ffu)
  KVR_TSTAGE(4, 0x0f0f0f0fu)
  KVR_TSTAGE(2, 0x33333333u)
  KVR_TSTAGE(1, 0x55555555u)
#undef KVR_TSTAGE
}

// ------------------------------------------------------------------ retrieved-tile attention

constexpr int RET_TILES_PER_BLOCK = 4;

// G4 = head slots per LUT entry (g rounded up to 4, 8 or 16).
template <int T, int G4>
__global__ __launch_bounds__(64) void retrieved_attn_kernel(
    const float* __restrict__ q_rot, int Hq, int Hkv, const uint64_t* __restrict__ kbits,
    const uint64_t* __restrict__ vbits, const uint16_t* __restrict__ kscale,
    const uint16_t* __restrict__ vscale, int64_t tile_stride, const int32_t* __restrict__ idx,
    int k, int n_rparts, int part0, int n_parts, float* __restrict__ rec) {
  constexpr int W = T / 64;
  __shared__ __attribute__((aligned(16))) float lq[32 * 16 * G4];  // [c4][pattern][head]
  __shared__ __attribute__((aligned(16))) float lu[16 * 16 * G4];  // [token nibble][pattern][head]
  __shared__ __attribute__((aligned(16))) float ps[64 * G4];       // [token][head]
  __shared__ float qs[G4 * D];

  const int lane = threadIdx.x;
  const int g = Hq / Hkv;
  const int64_t seg = blockIdx.x / n_rparts;
  const int rp = (int)(blockIdx.x - seg * n_rparts);
  const int64_t b = seg / Hkv;
  const int64_t h = seg - b * Hkv;
  const float* qr = q_rot + (b * Hq + h * g) * D;

  for (int i = lane; i < G4 * D; i += 64) qs[i] = (i < g * D) ? qr[i] : 0.f;
  __syncthreads();
  // logit table: lq[c4][e][hh] = sum_{bit i of e} q'[hh][4 c4 + i]
  for (int ent = lane; ent < 32 * 16; ent += 64) {
    const int c4 = ent >> 4, e = ent & 15;
#pragma unroll
    for (int hh = 0; hh < G4; ++hh) {
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (e & (1 << i)) acc += qs[hh * D + 4 * c4 + i];
      lq[ent * G4 + hh] = acc;
    }
  }
  __syncthreads();
  float qsum[G4];
#pragma unroll
  for (int hh = 0; hh < G4; ++hh) {
    float a = 0.f;
    for (int c4 = 0; c4 < 32; ++c4) a += lq[(c4 * 16 + 15) * G4 + hh];
    qsum[hh] = a;
  }

  float m_run[G4], l_lane[G4], o0[G4], o1[G4];
#pragma unroll
  for (int hh = 0; hh < G4; ++hh) {
    m_run[hh] = -__builtin_inff();
    l_lane[hh] = 0.f;
    o0[hh] = 0.f;
    o1[hh] = 0.f;
  }

  const int j0 = rp * RET_TILES_PER_BLOCK;
  const int j1 = (j0 + RET_TILES_PER_BLOCK < k) ? j0 + RET_TILES_PER_BLOCK : k;
  const int64_t segt = seg * tile_stride;
  for (int j = j0; j < j1; ++j) {
    int64_t tile = idx[seg * k + j];
    tile = tile < 0 ? 0 : (tile >= tile_stride ? tile_stride - 1 : tile);  // never read outside the store
    const float sk = f16_to_f32(kscale[segt + tile]);
    const float sv = f16_to_f32(vscale[segt + tile]);
    const uint64_t* kw = kbits + (segt + tile) * (int64_t)(D * W);
    const uint64_t* vw = vbits + (segt + tile) * (int64_t)(D * W);
#pragma unroll 1
    for (int w = 0; w < W; ++w) {
      const uint64_t ka = kw[lane * W + w], kb = kw[(lane + 64) * W + w];
      const uint64_t va = vw[lane * W + w], vb = vw[(lane + 64) * W + w];
      uint32_t a_lo = (uint32_t)ka, a_hi = (uint32_t)(ka >> 32);
      uint32_t b_lo = (uint32_t)kb, b_hi = (uint32_t)(kb >> 32);
      transpose64(a_lo, a_hi, lane);  // token row, channels 0..63
      transpose64(b_lo, b_hi, lane);  // token row, channels 64..127
      float dot[G4];
#pragma unroll
      for (int hh = 0; hh < G4; ++hh) dot[hh] = 0.f;
#pragma unroll
      for (int c4 = 0; c4 < 32; ++c4) {
        const uint32_t word = (c4 < 8) ? a_lo : (c4 < 16) ? a_hi : (c4 < 24) ? b_lo : b_hi;
        const uint32_t e = (word >> (4 * (c4 & 7))) & 15u;
        const float* ent = lq + (c4 * 16 + e) * G4;
#pragma unroll
        for (int hh = 0; hh < G4; hh += 4) {
          const float4 v = *(const float4*)(ent + hh);
          dot[hh] += v.x;
          dot[hh + 1] += v.y;
          dot[hh + 2] += v.z;
          dot[hh + 3] += v.w;
        }
      }
      float alpha[G4];
#pragma unroll
      for (int hh = 0; hh < G4; ++hh) {
        const float lg = sk * (2.f * dot[hh] - qsum[hh]) * SCALE_LOG2;
        const float tmax = wave_max(lg);
        const float m_new = fmaxf(m_run[hh], tmax);
        alpha[hh] = safe_exp2(m_run[hh] - m_new);
        m_run[hh] = m_new;
        const float p = safe_exp2(lg - m_new);
        l_lane[hh] = l_lane[hh] * alpha[hh] + p;
        ps[lane * G4 + hh] = p;
      }
      __syncthreads();
      // value table: lu[tn][e][hh] = sum_{bit i of e} p[4 tn + i][hh]
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
      __syncthreads();
      float x0[G4], x1[G4], psum[G4];
#pragma unroll
      for (int hh = 0; hh < G4; ++hh) {
        x0[hh] = 0.f;
        x1[hh] = 0.f;
        psum[hh] = 0.f;
      }
      const uint32_t vlo[4] = {(uint32_t)va, (uint32_t)(va >> 32), (uint32_t)vb, (uint32_t)(vb >> 32)};
#pragma unroll
      for (int tn = 0; tn < 16; ++tn) {
        const uint32_t e0 = (vlo[tn >> 3] >> (4 * (tn & 7))) & 15u;
        const uint32_t e1 = (vlo[2 + (tn >> 3)] >> (4 * (tn & 7))) & 15u;
        const float* t0 = lu + (tn * 16 + e0) * G4;
        const float* t1 = lu + (tn * 16 + e1) * G4;
        const float* tf = lu + (tn * 16 + 15) * G4;
#pragma unroll
        for (int hh = 0; hh < G4; hh += 4) {
          const float4 a = *(const float4*)(t0 + hh);
          const float4 c = *(const float4*)(t1 + hh);
          const float4 f = *(const float4*)(tf + hh);
          x0[hh] += a.x; x0[hh + 1] += a.y; x0[hh + 2] += a.z; x0[hh + 3] += a.w;
          x1[hh] += c.x; x1[hh + 1] += c.y; x1[hh + 2] += c.z; x1[hh + 3] += c.w;
          psum[hh] += f.x; psum[hh + 1] += f.y; psum[hh + 2] += f.z; psum[hh + 3] += f.w;
        }
      }
#pragma unroll
      for (int hh = 0; hh < G4; ++hh) {
        o0[hh] = o0[hh] * alpha[hh] + sv * (2.f * x0[hh] - psum[hh]);
        o1[hh] = o1[hh] * alpha[hh] + sv * (2.f * x1[hh] - psum[hh]);
      }
      __syncthreads();  // ps / lu reused by the next sub-tile
    }
  }

  float* R = rec + (seg * n_parts + part0 + rp) * (int64_t)(g * (2 + D));
#pragma unroll
  for (int hh = 0; hh < G4; ++hh) {
    if (hh < g) {
      const float lt = wave_sum(l_lane[hh]);
      if (lane == 0) {
        R[hh] = m_run[hh];
        R[g + hh] = lt;
      }
      R[2 * g + hh * D + lane] = o0[hh];
      R[2 * g + hh * D + lane + 64] = o1[hh];
    }
  }
}

// ------------------------------------------------------------------ merge

template <int TF, int OT>
__global__ __launch_bounds__(64) void merge_kernel(const float* __restrict__ rec, int Hq, int Hkv,
                                                   int n_wparts, int n_parts, void* __restrict__ out) {
  __shared__ float xs[D];
  const int lane = threadIdx.x;
  const int g = Hq / Hkv;
  const int64_t bq = blockIdx.x;  // b * Hq + head
  const int64_t b = bq / Hq;
  const int hq = (int)(bq - b * Hq);
  const int h = hq / g, i = hq - h * g;
  const int64_t seg = b * Hkv + h;
  const int64_t rs = g * (2 + D);
  const float* R0 = rec + seg * n_parts * rs;

  float M = -__builtin_inff();
  for (int p = 0; p < n_parts; ++p) M = fmaxf(M, R0[p * rs + i]);
  const float mu = (M == -__builtin_inff()) ? 0.f : M;
  float L = 0.f, w0 = 0.f, w1 = 0.f, r0 = 0.f, r1 = 0.f;
  for (int p = 0; p < n_parts; ++p) {
    const float* R = R0 + p * rs;
    const float f = safe_exp2(R[i] - mu);
    L += R[g + i] * f;
    const float a = R[2 * g + i * D + 2 * lane] * f;
    const float c = R[2 * g + i * D + 2 * lane + 1] * f;
    if (p < n_wparts) {
      w0 += a;
      w1 += c;
    } else {
      r0 += a;
      r1 += c;
    }
  }
  if (n_parts > n_wparts) {
    if constexpr (TF == KVR_HADAMARD) hadamard_pair(r0, r1, lane);
    else if constexpr (TF == KVR_DCT) idct_pair(r0, r1, lane, xs);
  }
  const float inv = (L > 0.f) ? 1.f / L : 0.f;
  const float y0 = (w0 + r0) * inv, y1 = (w1 + r1) * inv;
  const int64_t o = bq * D + 2 * lane;
  if constexpr (OT == KVR_FP32) {
    ((float*)out)[o] = y0;
    ((float*)out)[o + 1] = y1;
  } else {
    ((uint32_t*)out)[o >> 1] = pack2(f32_to_bf16_rne(y0), f32_to_bf16_rne(y1));
  }
}

// ------------------------------------------------------------------ gather (materialise)

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
  tile = tile < 0 ? 0 : (tile >= tile_stride ? tile_stride - 1 : tile);  // never read outside the store
  const int64_t slot = seg * tile_stride + tile;
  const float s = f16_to_f32(scales[slot]);
  const uint64_t* wp = bits + slot * (int64_t)(D * W);
  const uint64_t a = wp[lane * W + w], c = wp[(lane + 64) * W + w];
  uint32_t a_lo = (uint32_t)a, a_hi = (uint32_t)(a >> 32), c_lo = (uint32_t)c, c_hi = (uint32_t)(c >> 32);
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

// ------------------------------------------------------------------ launchers

struct AttnPlan {
  int n_wparts;
  int n_rparts;
  int64_t span;
};

AttnPlan attn_plan(int64_t win_len, int k) {
  AttnPlan p;
  p.n_wparts = (win_len > 0) ? (int)((win_len + 255) / 256) : 0;
  p.span = 256;
  p.n_rparts = (k > 0) ? (k + RET_TILES_PER_BLOCK - 1) / RET_TILES_PER_BLOCK : 0;
  return p;
}

size_t attn_records_bytes(int64_t B, int Hq, int Hkv, int64_t win_len, int k) {
  const AttnPlan p = attn_plan(win_len, k);
  const int g = Hq / Hkv;
  const int64_t parts = p.n_wparts + p.n_rparts;
  return (size_t)(B * Hkv * (parts > 0 ? parts : 1) * g * (2 + D)) * sizeof(float);
}

template <int QT, int WDT>
static hipError_t launch_window_t(bool f32out, const void* q, int64_t B, int Hq, int Hkv,
                                  const void* wk, const void* wv, int64_t win_len, int64_t sb,
                                  int64_t sh, int64_t st, const AttnPlan& p, int n_parts,
                                  float* rec, hipStream_t s) {
  constexpr int QS = (QT == WDT) ? 1 : 3;
  dim3 grid((unsigned)(B * Hkv * p.n_wparts)), block(WIN_THREADS);
  if (f32out)
    hipLaunchKernelGGL((window_attn_kernel<QT, WDT, QS, 3>), grid, block, 0, s, q, Hq, Hkv,
                       (const uint16_t*)wk, (const uint16_t*)wv, win_len, sb, sh, st, p.span,
                       p.n_wparts, n_parts, rec);
  else
    hipLaunchKernelGGL((window_attn_kernel<QT, WDT, QS, 2>), grid, block, 0, s, q, Hq, Hkv,
                       (const uint16_t*)wk, (const uint16_t*)wv, win_len, sb, sh, st, p.span,
                       p.n_wparts, n_parts, rec);
  return hipGetLastError();
}

template <int T, int G4>
static hipError_t launch_ret_t(const float* q_rot, int64_t B, int Hq, int Hkv, const uint64_t* kb,
                               const uint64_t* vb, const uint16_t* ks, const uint16_t* vs,
                               int64_t tile_stride, const int32_t* idx, int k, const AttnPlan& p,
                               int n_parts, float* rec, hipStream_t s) {
  dim3 grid((unsigned)(B * Hkv * p.n_rparts)), block(64);
  hipLaunchKernelGGL((retrieved_attn_kernel<T, G4>), grid, block, 0, s, q_rot, Hq, Hkv, kb, vb, ks,
                     vs, tile_stride, idx, k, p.n_rparts, p.n_wparts, n_parts, rec);
  return hipGetLastError();
}

hipError_t launch_attention(int qt, const void* q, const float* q_rot, int64_t B, int Hq, int Hkv,
                            const void* wk, const void* wv, int wdt, int64_t win_len, int64_t sb,
                            int64_t sh, int64_t st, const uint64_t* kb, const uint64_t* vb,
                            const uint16_t* ks, const uint16_t* vs, int64_t tile_stride, int T,
                            int tf, const int32_t* idx, int k, void* out, int ot, float* rec,
                            hipStream_t s) {
  const AttnPlan p = attn_plan(win_len, k);
  const int n_parts = p.n_wparts + p.n_rparts;
  const int g = Hq / Hkv;
  hipError_t err = hipSuccess;
  if (p.n_wparts > 0) {
    const bool f32 = (ot == KVR_FP32);
#define KVR_WIN(QTV, WDTV) \
  if (qt == QTV && wdt == WDTV) err = launch_window_t<QTV, WDTV>(f32, q, B, Hq, Hkv, wk, wv, win_len, sb, sh, st, p, n_parts, rec, s); else
    KVR_WIN(KVR_BF16, KVR_BF16)
    KVR_WIN(KVR_FP16, KVR_BF16)
    KVR_WIN(KVR_FP32, KVR_BF16)
    KVR_WIN(KVR_BF16, KVR_FP16)
    KVR_WIN(KVR_FP16, KVR_FP16)
    KVR_WIN(KVR_FP32, KVR_FP16)
    err = hipErrorInvalidValue;
#undef KVR_WIN
    if (err != hipSuccess) return err;
  }
  if (p.n_rparts > 0) {
#define KVR_RET(TV, G4V) \
  if (T == TV && g <= G4V) err = launch_ret_t<TV, G4V>(q_rot, B, Hq, Hkv, kb, vb, ks, vs, tile_stride, idx, k, p, n_parts, rec, s); else
    KVR_RET(64, 4)
    KVR_RET(64, 8)
    KVR_RET(64, 16)
    KVR_RET(128, 4)
    KVR_RET(128, 8)
    KVR_RET(128, 16)
    err = hipErrorInvalidValue;
#undef KVR_RET
    if (err != hipSuccess) return err;
  }
  dim3 grid((unsigned)(B * Hq)), block(64);
#define KVR_MRG(TFV, OTV)                                                                       \
  if (tf == TFV && ot == OTV) {                                                                 \
    hipLaunchKernelGGL((merge_kernel<TFV, OTV>), grid, block, 0, s, rec, Hq, Hkv, p.n_wparts,     \
                       n_parts, out);                                                           \
    return hipGetLastError();                                                                   \
  }
  KVR_MRG(KVR_HADAMARD, KVR_FP32)
  KVR_MRG(KVR_HADAMARD, KVR_BF16)
  KVR_MRG(KVR_DCT, KVR_FP32)
  KVR_MRG(KVR_DCT, KVR_BF16)
  KVR_MRG(KVR_NONE, KVR_FP32)
  KVR_MRG(KVR_NONE, KVR_BF16)
#undef KVR_MRG
  return hipErrorInvalidValue;
}

hipError_t launch_gather(const uint64_t* bits, const uint16_t* scales, int64_t BH,
                         int64_t tile_stride, int T, int tf, const int32_t* idx, int k, float* out,
                         int64_t oss, int64_t ost, hipStream_t s) {
  const int64_t nblk = BH * k * (T / 64);
  if (nblk == 0) return hipSuccess;
  dim3 grid((unsigned)nblk), block(64);
#define KVR_GA(TV, TFV)                                                                          \
  if (T == TV && tf == TFV) {                                                                    \
    hipLaunchKernelGGL((gather_tiles_kernel<TV, TFV>), grid, block, 0, s, bits, scales,           \
                       tile_stride, idx, k, out, oss, ost);                                      \
    return hipGetLastError();                                                                    \
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
