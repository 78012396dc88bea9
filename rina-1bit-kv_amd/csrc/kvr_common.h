// Shared device helpers for the gfx950 compressed-KV kernels.
//
// Everything here is compiled with -ffp-contract=off: each fp32 add/mul rounds
// once, in program order, so the CPU oracle can reproduce the codec and the
// tile scores bit for bit.  Explicit fmaf() is used only where a result is a
// tolerance (attention), never on a bit-exact path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/kvr_capi.h"

namespace kvr {

constexpr int D = 128;                // head_dim
constexpr float C_HAD = 0x1.6a09e6p-4f;  // fp32(2^-3.5) = 0x3db504f3
constexpr float EPS = 1e-8f;
constexpr float FP16_MAX = 65504.0f;
constexpr float LOG2E = 1.4426950408889634f;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------ conversions

__device__ __forceinline__ float bf16_to_f32(uint32_t raw16) { return __uint_as_float(raw16 << 16); }

__device__ __forceinline__ float f16_to_f32(uint32_t raw16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)raw16);
}

// Round-to-nearest-even fp32 -> bf16 bit pattern (NaN kept quiet).
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ uint32_t f32_to_f16_rne(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

// Load element i of a bf16 / fp16 / fp32 array as fp32 (exact).
template <int DT>
__device__ __forceinline__ float load_as_f32(const void* p, int64_t i) {
  if constexpr (DT == KVR_BF16) return bf16_to_f32(((const uint16_t*)p)[i]);
  else if constexpr (DT == KVR_FP16) return f16_to_f32(((const uint16_t*)p)[i]);
  else return ((const float*)p)[i];
}
__device__ __forceinline__ float load_as_f32(const void* p, int dt, int64_t i) {
  if (dt == KVR_BF16) return bf16_to_f32(((const uint16_t*)p)[i]);
  if (dt == KVR_FP16) return f16_to_f32(((const uint16_t*)p)[i]);
  return ((const float*)p)[i];
}

// Correctly rounded fp32 square root: the f64 root of an f32 is correctly
// rounded to 53 bits, and 53 >= 2*24+2, so rounding it to f32 is correct.
__device__ __forceinline__ float sqrt_rn(float x) { return (float)__builtin_sqrt((double)x); }

// ------------------------------------------------------------------ wave helpers

__device__ __forceinline__ float shfl_xor_f(float v, int m) { return __shfl_xor(v, m, 64); }
__device__ __forceinline__ uint32_t shfl_xor_u(uint32_t v, int m) {
  return (uint32_t)__shfl_xor((int)v, m, 64);
}

// Cross-lane moves without LDS: DPP inside 16-lane rows, v_permlane{16,32}_swap
// across rows (gfx950).  xor16 / xor32 return the value of lane ^ 16 / lane ^ 32.
#define KVR_DPP(v, ctrl) __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), ctrl, 0xf, 0xf, false))
__device__ __forceinline__ float xor16_f(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((__lane_id() & 16) ? r[0] : r[1]);
}
__device__ __forceinline__ float xor32_f(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((__lane_id() & 32) ? r[0] : r[1]);
}

// Row (16-lane) reductions: xor 1, xor 2 (quad_perm), then half-mirror and mirror,
// after which every lane of the row holds the row's result.
__device__ __forceinline__ float row_max(float v) {
  v = fmaxf(v, KVR_DPP(v, 0xb1));   // quad_perm [1,0,3,2]
  v = fmaxf(v, KVR_DPP(v, 0x4e));   // quad_perm [2,3,0,1]
  v = fmaxf(v, KVR_DPP(v, 0x141));  // row_half_mirror
  v = fmaxf(v, KVR_DPP(v, 0x140));  // row_mirror
  return v;
}
__device__ __forceinline__ float row_sum(float v) {
  v = v + KVR_DPP(v, 0xb1);
  v = v + KVR_DPP(v, 0x4e);
  v = v + KVR_DPP(v, 0x141);
  v = v + KVR_DPP(v, 0x140);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
  v = row_max(v);
  v = fmaxf(v, xor16_f(v));
  return fmaxf(v, xor32_f(v));
}

__device__ __forceinline__ float wave_sum(float v) {
  v = row_sum(v);
  v = v + xor16_f(v);
  return v + xor32_f(v);
}

// Value of lane ^ M for a compile-time M (no LDS): quad_perm for 1, 2; half-mirror
// then quad-reverse for 4; row_ror:8 for 8; permlane swaps for 16, 32.  All 64
// lanes must be active.
template <int M>
__device__ __forceinline__ float xor_lane_f(float v) {
  if constexpr (M == 1) return KVR_DPP(v, 0xb1);
  else if constexpr (M == 2) return KVR_DPP(v, 0x4e);
  else if constexpr (M == 4) return KVR_DPP(KVR_DPP(v, 0x141), 0x1b);
  else if constexpr (M == 8) return KVR_DPP(v, 0x128);
  else if constexpr (M == 16) return xor16_f(v);
  else return xor32_f(v);
}
template <int M>
__device__ __forceinline__ uint32_t xor_lane_u(uint32_t v) {
  return __float_as_uint(xor_lane_f<M>(__uint_as_float(v)));
}

// One FWHT butterfly stage across lanes for a value held one-per-lane: lanes with
// (lane & M) == 0 hold the lower element of each pair.  Lower: a + b; upper: a - b
// (a = lower value, b = upper value) -- the same single fp32 add/sub the oracle does.
template <int M>
__device__ __forceinline__ float fwht_xlane(float v, int lane) {
  const float p = xor_lane_f<M>(v);
  return (lane & M) ? (p - v) : (v + p);
}

// Full orthonormal Hadamard-128 (spec order h = 1..64, then * C_HAD) of a
// vector held as channels (2*lane, 2*lane+1) in (v0, v1).  Bit-exact.
__device__ __forceinline__ void hadamard_pair(float& v0, float& v1, int lane) {
  float a = v0 + v1, b = v0 - v1;  // h = 1
  v0 = fwht_xlane<1>(a, lane);     // h = 2m: partner lane = lane ^ m
  v1 = fwht_xlane<1>(b, lane);
  v0 = fwht_xlane<2>(v0, lane);
  v1 = fwht_xlane<2>(v1, lane);
  v0 = fwht_xlane<4>(v0, lane);
  v1 = fwht_xlane<4>(v1, lane);
  v0 = fwht_xlane<8>(v0, lane);
  v1 = fwht_xlane<8>(v1, lane);
  v0 = fwht_xlane<16>(v0, lane);
  v1 = fwht_xlane<16>(v1, lane);
  v0 = fwht_xlane<32>(v0, lane);
  v1 = fwht_xlane<32>(v1, lane);
  v0 = v0 * C_HAD;
  v1 = v1 * C_HAD;
}

// In-register unnormalised FWHT of 128 values (spec order), bit-exact.
__device__ __forceinline__ void fwht128_regs(float* x) {
#pragma unroll
  for (int h = 1; h < 128; h <<= 1) {
#pragma unroll
    for (int j = 0; j < 128; ++j) {
      if ((j & h) == 0) {
        float a = x[j], b = x[j + h];
        x[j] = a + b;
        x[j + h] = a - b;
      }
    }
  }
}

// Orthonormal DCT-II matrix C[k][n] = a_k cos(pi (2n+1) k / 256), fp32, row k =
// frequency.  Built at compile time: only the 512 angles pi*r/256 occur, each
// evaluated in double by a Taylor series on [0, pi/2] (error < 1e-16), then
// scaled by a_0 = sqrt(1/128) or a_k = 1/8 and rounded once to fp32.
struct DctTable {
  float v[D * D];
};

constexpr double cos_pi_r256(int r) {  // cos(pi * r / 256), r in [0, 512)
  double sign = 1.0;
  if (r > 256) r = 512 - r;
  if (r > 128) {
    r = 256 - r;
    sign = -1.0;
  }
  const double x = 3.14159265358979323846 * (double)r / 256.0;
  double term = 1.0, sum = 1.0;
  for (int i = 1; i < 20; ++i) {
    term *= -x * x / (double)((2 * i - 1) * (2 * i));
    sum += term;
  }
  return sign * sum;
}

constexpr DctTable make_dct_table() {
  DctTable t{};
  double c[512] = {};
  for (int r = 0; r < 512; ++r) c[r] = cos_pi_r256(r);
  for (int k = 0; k < D; ++k) {
    const double a = (k == 0) ? 0.088388347648318440550 : 0.125;
    for (int n = 0; n < D; ++n) t.v[k * D + n] = (float)(a * c[((2 * n + 1) * k) % 512]);
  }
  return t;
}

static __constant__ DctTable g_dct_tab = make_dct_table();
#define g_dct (g_dct_tab.v)

// The entries of C as a 2 KB table: [r] = cos(pi r / 256) / 8 for r < 512 (C[k][n] for
// k >= 1 is entry (2n+1) k mod 512, the same rounding as the matrix), [512] = C[0][n]
// = sqrt(1/128); padded to a multiple of 4 floats.
struct CosTable {
  float v[516];
};
constexpr CosTable make_cos_table() {
  CosTable t{};
  for (int r = 0; r < 512; ++r) t.v[r] = (float)(0.125 * cos_pi_r256(r));
  t.v[512] = (float)(0.088388347648318440550 * cos_pi_r256(0));
  return t;
}
static __constant__ CosTable g_cos_tab = make_cos_table();

// Floats of a wave's LDS scratch for dct_pair / idct_pair: the vector, then the table.
constexpr int DCT_SCRATCH = D + 516;

// The table is staged by each wave that uses it, at xs + D of its scratch: loaded into
// registers first (dct_table_load, issued early so that its latency overlaps other
// loads), then stored (dct_table_store) before the wave's first DCT.
struct DctRegs {
  float4 t0, t1, t2;
};
__device__ __forceinline__ DctRegs dct_table_load(int lane) {
  const float4* src = (const float4*)g_cos_tab.v;
  return DctRegs{src[lane], src[lane + 64], src[128]};
}
__device__ __forceinline__ void dct_table_store(const DctRegs& r, float* xs, int lane) {
  float4* cs = (float4*)(xs + D);
  cs[lane] = r.t0;
  cs[lane + 64] = r.t1;
  if (lane == 0) cs[128] = r.t2;
}
__device__ __forceinline__ void dct_table_to_lds(float* xs, int lane) { dct_table_store(dct_table_load(lane), xs, lane); }

// y = C x for a vector held as channels (2*lane, 2*lane+1), through the caller's
// wave-private LDS scratch xs[DCT_SCRATCH] (the table staged at xs + D).  C[k][127-n] = (-1)^k C[k][n], so with
// s[n] = x[n] + x[127-n] and d[n] = x[n] - x[127-n] (n < 64) an even row is
// sum_n C[k][n] s[n] and an odd row sum_n C[k][n] d[n]: 64 LDS table reads per output.
// Tolerance path (fmaf, a different summation order than the plain product).
__device__ __forceinline__ void dct_pair(float& v0, float& v1, int lane, float* xs) {
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
  // table index of C[k][n]: (2n+1) k mod 512, stepping by 2k; row 0 stays at 512
  int r0 = lane == 0 ? 512 : 2 * lane;
  const int d0 = lane == 0 ? 0 : 4 * lane, m0 = lane == 0 ? 1023 : 511;
  int r1 = 2 * lane + 1;
  const int d1 = 4 * lane + 2;
  float a0 = 0.f, a1 = 0.f;
#pragma unroll 8
  for (int n = 0; n < 64; ++n) {
    const float2 sd = ((const float2*)xs)[n];
    a0 = fmaf(cs[r0], sd.x, a0);
    a1 = fmaf(cs[r1], sd.y, a1);
    r0 = (r0 + d0) & m0;
    r1 = (r1 + d1) & 511;
  }
  __builtin_amdgcn_wave_barrier();
  v0 = a0;
  v1 = a1;
}

// x = C^T y for a vector held as channels (2*lane, 2*lane+1) (the table staged at
// xs + D): lane n < 64 sums the even rows E = sum C[2j][n] y[2j] and the odd rows
// O = sum C[2j+1][n] y[2j+1]; then x[n] = E + O and x[127-n] = E - O.
__device__ __forceinline__ void idct_pair(float& v0, float& v1, int lane, float* xs) {
  const float* cs = xs + D;
  xs[2 * lane] = v0;
  xs[2 * lane + 1] = v1;
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_wave_barrier();
  const int st = 2 * lane + 1;  // 2n + 1
  const float2 y01 = ((const float2*)xs)[0];
  float e = cs[512] * y01.x;               // row 0
  float o = cs[st] * y01.y;                // row 1
  int re = (2 * st) & 511, ro = (3 * st) & 511;
  const int dr = (2 * st) & 511;
#pragma unroll 7
  for (int j = 1; j < 64; ++j) {
    const float2 y = ((const float2*)xs)[j];  // (y[2j], y[2j+1])
    e = fmaf(cs[re], y.x, e);
    o = fmaf(cs[ro], y.y, o);
    re = (re + dr) & 511;
    ro = (ro + dr) & 511;
  }
  __builtin_amdgcn_wave_barrier();
  xs[lane] = e + o;
  xs[127 - lane] = e - o;
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_wave_barrier();
  v0 = xs[2 * lane];
  v1 = xs[2 * lane + 1];
  __builtin_amdgcn_wave_barrier();
}

// Orderable key of an fp32 score: larger float -> larger key; NaN -> -inf.
__device__ __forceinline__ uint32_t score_key(float f) {
  if (f != f) f = -__builtin_inff();
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

}  // namespace kvr
