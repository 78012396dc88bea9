// Subsystems 2 and 3: query preparation, tile scoring and top-k tile selection.
//
// Query prep  : GQA mean of the g query heads of each KV head (fp32 sum in head
//               order, one correctly rounded division by g; the reference's
//               q.view(Hkv, g, d).mean(1), modules/kvr_retrieval.py:270,296),
//               then the codec rotation.  One wave per (sequence, KV head);
//               lane = channels (2*lane, 2*lane+1); the Hadamard butterflies
//               run across lanes in the codec's stage order (bit-exact).
// Tile scoring: cosine of the rotated mean query with the tile's column sums
//               c_j = 2*popcount(word_j) - T (the chunk-mean cosine of
//               modules/kvr_retrieval.py:291-315 on +-1 codes; the per-tile
//               scale cancels).  16 lanes per tile, 8 channels per lane, so a
//               wave reads 4 whole tiles (4 KB at T=64) per step, coalesced.
//               The fp32 order (per-lane sequential over 8 channels, then the
//               16-lane tree h = 8,4,2,1) is fixed so the oracle reproduces it.
// Top-k       : per segment, radix select of the k-th largest orderable key
//               (4 passes x 8 bits, LDS histogram), ordered compaction of the
//               winners (ties: lowest tile index first), then a rank sort by
//               (score desc, index asc).
#include "kvr_common.h"

namespace kvr {

// ------------------------------------------------------------------ query prep

template <int QT, int TF>
__global__ __launch_bounds__(64) void query_prep_kernel(const void* __restrict__ q, int Hq, int Hkv,
                                                        float* __restrict__ qbar_rot,
                                                        float* __restrict__ q_rot) {
  __shared__ float xs[D];
  const int lane = threadIdx.x;
  const int64_t seg = blockIdx.x;  // b * Hkv + h
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
  if constexpr (TF == KVR_HADAMARD) hadamard_pair(m0, m1, lane);
  else if constexpr (TF == KVR_DCT) dct_pair(m0, m1, lane, xs);
  qbar_rot[seg * D + 2 * lane] = m0;
  qbar_rot[seg * D + 2 * lane + 1] = m1;

  if (q_rot) {
    for (int i = 0; i < g; ++i) {
      float v0 = load_as_f32<QT>(q, q0 + (int64_t)i * D + 2 * lane);
      float v1 = load_as_f32<QT>(q, q0 + (int64_t)i * D + 2 * lane + 1);
      if constexpr (TF == KVR_HADAMARD) hadamard_pair(v0, v1, lane);
      else if constexpr (TF == KVR_DCT) dct_pair(v0, v1, lane, xs);
      q_rot[q0 + (int64_t)i * D + 2 * lane] = v0;
      q_rot[q0 + (int64_t)i * D + 2 * lane + 1] = v1;
    }
  }
}

hipError_t launch_query_prep(int qt, int tf, const void* q, int64_t B, int Hq, int Hkv,
                             float* qbar_rot, float* q_rot, hipStream_t s) {
  const int64_t nblk = B * Hkv;
  if (nblk == 0) return hipSuccess;
#define KVR_QP(QTV, TFV)                                                                   \
  if (qt == QTV && tf == TFV) {                                                            \
    hipLaunchKernelGGL((query_prep_kernel<QTV, TFV>), dim3((unsigned)nblk), dim3(64), 0, s, q, \
                       Hq, Hkv, qbar_rot, q_rot);                                          \
    return hipGetLastError();                                                              \
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

// ------------------------------------------------------------------ tile scoring

// Number of set bits of a 64-bit word.  METHOD 0: hardware popcount
// (v_bcnt_u32_b32); METHOD 1: SWAR bit-unpack (pairwise bit sums), same count.
template <int METHOD>
__device__ __forceinline__ int count_bits(uint64_t w) {
  if constexpr (METHOD == 0) {
    return __popcll(w);
  } else {
    uint64_t x = w - ((w >> 1) & 0x5555555555555555ull);
    x = (x & 0x3333333333333333ull) + ((x >> 2) & 0x3333333333333333ull);
    x = (x + (x >> 4)) & 0x0f0f0f0f0f0f0f0full;
    return (int)((x * 0x0101010101010101ull) >> 56);
  }
}

// 16-lane tree h = 8, 4, 2, 1 (lanes of one 16-lane group; every lane ends
// with the same value since fp32 addition is commutative).
__device__ __forceinline__ float tree16(float p) {
  p = p + shfl_xor_f(p, 8);
  p = p + shfl_xor_f(p, 4);
  p = p + shfl_xor_f(p, 2);
  p = p + shfl_xor_f(p, 1);
  return p;
}

constexpr int SCORE_TILES_PER_BLOCK = 64;  // 16 groups x 4 tiles

template <int T, int METHOD>
__global__ __launch_bounds__(256) void score_tiles_kernel(
    const float* __restrict__ qbar_rot, const uint64_t* __restrict__ kbits, int64_t n_tiles,
    int64_t tile_stride, int64_t n_chunks, const int32_t* __restrict__ excl_lo,
    const int32_t* __restrict__ excl_hi, float* __restrict__ scores) {
  constexpr int W = T / 64;
  const int64_t seg = blockIdx.x / n_chunks;
  const int64_t chunk = blockIdx.x - seg * n_chunks;
  const int tid = threadIdx.x;
  const int grp = tid >> 4;  // 16 groups of 16 lanes
  const int li = tid & 15;   // channels 8*li .. 8*li+7

  float q[8];
  {
    const float4* qp = (const float4*)(qbar_rot + seg * D + 8 * li);
    float4 a = qp[0], c = qp[1];
    q[0] = a.x; q[1] = a.y; q[2] = a.z; q[3] = a.w;
    q[4] = c.x; q[5] = c.y; q[6] = c.z; q[7] = c.w;
  }
  float qq = q[0] * q[0];
#pragma unroll
  for (int k = 1; k < 8; ++k) qq = qq + q[k] * q[k];
  qq = tree16(qq);
  const float qn = sqrt_rn(qq) + EPS;

  const int32_t lo = excl_lo ? excl_lo[seg] : 0;
  const int32_t hi = excl_hi ? excl_hi[seg] : 0;
  const uint64_t* segbits = kbits + seg * tile_stride * (int64_t)(D * W);
  const int64_t t0 = chunk * SCORE_TILES_PER_BLOCK;
  const int64_t t1 = (t0 + SCORE_TILES_PER_BLOCK < n_tiles) ? t0 + SCORE_TILES_PER_BLOCK : n_tiles;

  for (int64_t tile = t0 + grp; tile < t1; tile += 16) {
    const uint64_t* wp = segbits + tile * (D * W) + 8 * li * W;
    uint64_t wd[8 * W];
#pragma unroll
    for (int i = 0; i < 4 * W; ++i) {
      ulonglong2 v = ((const ulonglong2*)wp)[i];
      wd[2 * i] = v.x;
      wd[2 * i + 1] = v.y;
    }
    float dot = 0.f;
    int cc = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      int pc = 0;
#pragma unroll
      for (int w = 0; w < W; ++w) pc += count_bits<METHOD>(wd[k * W + w]);
      const int c = 2 * pc - T;
      cc += c * c;
      const float prod = q[k] * (float)c;
      dot = (k == 0) ? prod : dot + prod;
    }
    dot = tree16(dot);
    cc += __shfl_xor(cc, 8, 64);
    cc += __shfl_xor(cc, 4, 64);
    cc += __shfl_xor(cc, 2, 64);
    cc += __shfl_xor(cc, 1, 64);
    if (li == 0) {
      const float cn = sqrt_rn((float)cc) + EPS;
      float sc = __fdiv_rn(dot, qn * cn);
      if (sc != sc) sc = -__builtin_inff();
      if (tile >= lo && tile < hi) sc = -__builtin_inff();
      scores[seg * n_tiles + tile] = sc;
    }
  }
}

hipError_t launch_score(int T, int method, const float* qbar_rot, const uint64_t* kbits, int64_t BH,
                        int64_t n_tiles, int64_t tile_stride, const int32_t* excl_lo,
                        const int32_t* excl_hi, float* scores, hipStream_t s) {
  const int64_t n_chunks = (n_tiles + SCORE_TILES_PER_BLOCK - 1) / SCORE_TILES_PER_BLOCK;
  const int64_t nblk = BH * n_chunks;
  if (nblk == 0) return hipSuccess;
  dim3 grid((unsigned)nblk), block(256);
#define KVR_SC(TV, MV)                                                                          \
  if (T == TV && method == MV) {                                                                \
    hipLaunchKernelGGL((score_tiles_kernel<TV, MV>), grid, block, 0, s, qbar_rot, kbits, n_tiles, \
                       tile_stride, n_chunks, excl_lo, excl_hi, scores);                        \
    return hipGetLastError();                                                                   \
  }
  KVR_SC(64, 0)
  KVR_SC(64, 1)
  KVR_SC(128, 0)
  KVR_SC(128, 1)
#undef KVR_SC
  return hipErrorInvalidValue;
}

// ------------------------------------------------------------------ top-k

constexpr int TOPK_THREADS = 256;
constexpr int TOPK_MAX_K = 1024;

__global__ __launch_bounds__(TOPK_THREADS) void topk_tiles_kernel(const float* __restrict__ scores,
                                                                  int64_t n, int64_t stride, int k,
                                                                  int32_t* __restrict__ idx) {
  __shared__ uint32_t hist[256];
  __shared__ uint32_t sel_key[TOPK_MAX_K];
  __shared__ int32_t sel_idx[TOPK_MAX_K];
  __shared__ uint32_t sh_digit, sh_kk, sh_ngt;
  __shared__ uint32_t wave_cnt[TOPK_THREADS / 64];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int64_t seg = blockIdx.x;
  const float* row = scores + seg * stride;

  // ---- radix select: tau = k-th largest key, kk = how many keys == tau to take
  uint32_t prefix = 0, pmask = 0, kk = (uint32_t)k;
#pragma unroll 1
  for (int shift = 24; shift >= 0; shift -= 8) {
    hist[tid] = 0;
    __syncthreads();
    for (int64_t i = tid; i < n; i += TOPK_THREADS) {
      const uint32_t key = score_key(row[i]);
      if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (wv == 0) {
      // lane handles bins 255-4*lane .. 252-4*lane (descending)
      uint32_t c[4], tot = 0;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        c[r] = hist[255 - 4 * lane - r];
        tot += c[r];
      }
      uint32_t incl = tot;
#pragma unroll
      for (int m = 1; m < 64; m <<= 1) {
        uint32_t o = (uint32_t)__shfl_up((int)incl, m, 64);
        if (lane >= m) incl += o;
      }
      uint32_t excl = incl - tot;
      if (excl < kk && kk <= incl) {
        uint32_t run = excl;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (run < kk && kk <= run + c[r]) {
            sh_digit = 255u - 4u * lane - r;
            sh_kk = kk - run;
          }
          run += c[r];
        }
      }
    }
    __syncthreads();
    prefix |= sh_digit << shift;
    pmask |= 255u << shift;
    kk = sh_kk;
    __syncthreads();
  }
  const uint32_t tau = prefix;

  // ---- ordered compaction: every key > tau, plus the first kk keys == tau
  if (tid == 0) sh_ngt = 0;
  __syncthreads();
  const uint32_t n_gt_total = (uint32_t)k - kk;
  uint32_t eq_base = 0;  // keys == tau seen in earlier chunks (uniform)
#pragma unroll 1
  for (int64_t c0 = 0; c0 < n; c0 += TOPK_THREADS) {
    const int64_t i = c0 + tid;
    uint32_t key = 0;
    bool gt = false, eq = false;
    if (i < n) {
      key = score_key(row[i]);
      gt = key > tau;
      eq = key == tau;
    }
    if (gt) {
      const uint32_t p = atomicAdd(&sh_ngt, 1u);
      if (p < n_gt_total) {  // exactly n_gt_total keys exceed tau; never write past them
        sel_key[p] = key;
        sel_idx[p] = (int32_t)i;
      }
    }
    const uint64_t bal = __ballot(eq);
    const uint32_t below = (uint32_t)__popcll(bal & ((1ull << lane) - 1ull));
    if (lane == 0) wave_cnt[wv] = (uint32_t)__popcll(bal);
    __syncthreads();
    uint32_t off = eq_base, chunk_tot = 0;
    for (int w = 0; w < TOPK_THREADS / 64; ++w) {
      if (w < wv) off += wave_cnt[w];
      chunk_tot += wave_cnt[w];
    }
    if (eq) {
      const uint32_t r = off + below;  // rank among keys == tau in index order
      if (r < kk) {
        sel_key[n_gt_total + r] = key;
        sel_idx[n_gt_total + r] = (int32_t)i;
      }
    }
    eq_base += chunk_tot;
    __syncthreads();
    if (eq_base >= kk && sh_ngt >= n_gt_total) break;  // uniform: all winners found
  }
  __syncthreads();

  // ---- rank sort of the k winners by (key desc, index asc)
  for (int a = tid; a < k; a += TOPK_THREADS) {
    const uint32_t ka = sel_key[a];
    const int32_t ia = sel_idx[a];
    int rank = 0;
    for (int bb = 0; bb < k; ++bb) {
      const uint32_t kb = sel_key[bb];
      const int32_t ib = sel_idx[bb];
      rank += (kb > ka) || (kb == ka && ib < ia);
    }
    idx[seg * k + rank] = ia;
  }
}

hipError_t launch_topk(const float* scores, int64_t BH, int64_t n, int64_t stride, int k,
                       int32_t* idx, hipStream_t s) {
  if (BH == 0) return hipSuccess;
  hipLaunchKernelGGL(topk_tiles_kernel, dim3((unsigned)BH), dim3(TOPK_THREADS), 0, s, scores, n,
                     stride, k, idx);
  return hipGetLastError();
}

}  // namespace kvr
