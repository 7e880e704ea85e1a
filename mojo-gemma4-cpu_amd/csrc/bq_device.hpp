// bq_device.hpp -- device-side building blocks shared by the butterquant HIP
// kernels (gfx950 / CDNA4, wave64).
//
// Numerics follow the reference CPU path exactly where the reference fixes
// them (all files are compiled with -ffp-contract=off; fmaf appears only where
// the reference calls .fma):
//   * f32 -> bf16 is round-to-nearest-even by bit arithmetic
//     (butterquant/convert.mojo:14-17);
//   * FWHT stages run strides 1,2,4,... as (a+b, a-b), then one multiply by
//     f32(1/f64(sqrtf(B))) (butterquant/fwht.mojo:20-57);
//   * quantization is q = clamp(rne(x * (127/amax)), -128, 127)
//     (butterquant/kernels.mojo:68-78, simd_math/ops.mojo:26-31);
//   * GELU is the reference's tanh form with its fast exp polynomial
//     (simd_math/ops.mojo:73-156).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;
constexpr float kInv127 = 1.0f / 127.0f;

// ---------------------------------------------------------------------------
// GPU weight layout "tile16x64": the int8 codes of W[N,K] are stored as 1 KiB
// fragments of 16 rows x 64 K, fragment (n/16, k/64) at
// ((n/16)*(K/64) + k/64) * 1024; inside it lane L = ((k%64)/16)*16 + n%16 owns
// bytes [L*16, L*16+16) holding k%16 = 0..15.  One 16-byte load per lane
// fetches exactly the B operand of one v_mfma_i32_16x16x64_i8 for 16 output
// rows, and a wave's 64 loads cover 1 KiB of contiguous HBM.
// ---------------------------------------------------------------------------
__host__ __device__ inline size_t tile_offset(int n, int k, int K) {
  return ((size_t)(n >> 4) * (size_t)(K >> 6) + (size_t)(k >> 6)) * 1024u +
         (size_t)((((k & 63) >> 4) << 4) + (n & 15)) * 16u + (size_t)(k & 15);
}

// The reference's load-time VNNI layout (butterquant/vnni.mojo:146-163).
__host__ __device__ inline size_t vnni_offset(int n, int k, int K) {
  return (size_t)(n / 32) * 32u * (size_t)K + (size_t)(k / 64) * 2048u +
         (size_t)((n % 32) / 16) * 1024u + (size_t)((k % 64) / 4) * 64u +
         (size_t)(n % 16) * 4u + (size_t)(k % 4);
}

// ---------------------------------------------------------------------------
// scalar numerics
// ---------------------------------------------------------------------------
__device__ inline uint16_t f32_to_bf16(float v) {
  uint32_t bits = __float_as_uint(v);
  uint32_t rne = bits + ((bits >> 16) & 1u) + 0x7FFFu;
  return (uint16_t)(rne >> 16);
}

__device__ inline float bf16_to_f32(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}

__device__ inline int8_t quantize_i8(float v, float inv) {
  float r = __builtin_rintf(v * inv);  // v_rndne_f32: round half to even
  r = r < -128.0f ? -128.0f : r;
  r = r > 127.0f ? 127.0f : r;
  return (int8_t)(int)r;
}

// f32(1.0 / f64(sqrtf(B))) (butterquant/fwht.mojo:55); host computes it.
__host__ inline float fwht_scale_host(int block) {
  float s = __builtin_sqrtf((float)block);
  return (float)(1.0 / (double)s);
}

// simd_math/ops.mojo:73-96
__device__ inline float exp_f32_fast(float x) {
  const float LN2 = 0.6931471805599453f;
  const float INV_LN2 = 1.4426950408889634f;
  float xc = x > -87.0f ? x : -87.0f;
  float xn = xc * INV_LN2;
  int n = (int)__builtin_rintf(xn);
  float r = xc - (float)n * LN2;
  float p = 1.0f + r * (0.9999f + r * (0.4985f + r * (0.1681f)));
  int nc = n > -126 ? n : -126;
  float pow2n = __uint_as_float(((uint32_t)(nc + 127)) << 23);
  return p * pow2n;
}

// simd_math/ops.mojo:128-141
__device__ inline float tanh_f32(float x) {
  uint32_t sign_bits = __float_as_uint(x) & 0x80000000u;
  float ax = __uint_as_float(__float_as_uint(x) & 0x7FFFFFFFu);
  float e = exp_f32_fast(-2.0f * ax);
  float t = (1.0f - e) / (1.0f + e);
  return __uint_as_float(__float_as_uint(t) ^ sign_bits);
}

// simd_math/ops.mojo:145-156
__device__ inline float gelu_tanh_f32(float x) {
  const float sqrt_2_over_pi = 0.7978845608028654f;
  const float gelu_a = 0.044715f;
  float x3 = x * x * x;
  float inner = sqrt_2_over_pi * (x + gelu_a * x3);
  float t = tanh_f32(inner);
  return 0.5f * x * (1.0f + t);
}

// simd_math/exponential.mojo:178-194, the router softmax's exp: a bit-level
// 2^(x/ln2) with a quadratic mantissa correction.  The f32 -> i32 truncation
// is the one of the x86 build the reference runs on: NaN and values outside
// [-2^31, 2^31) give INT32_MIN (so x near -1e30 returns -0.0), where
// v_cvt_i32_f32 alone would saturate positive values and map NaN to 0.
__device__ inline float fast_exp_softmax_biased(float x) {
  const float A_MAGIC = 12102203.16156148f;
  const float BIAS_F = 1059208216.0f;
  const float INV_TWO23 = 1.0f / (float)(1 << 23);
  const float QC_A = 1.6501418352127075f;
  const float QC_B = -0.37554836273193359f;
  const float QC_C = 0.38696467876434326f;
  const float v = A_MAGIC * x + BIAS_F;
  const int32_t i = (v >= -2147483648.0f && v < 2147483648.0f) ? (int32_t)v : INT32_MIN;
  const uint32_t u = (uint32_t)i;
  const float k = __uint_as_float(u);
  const float f = (float)(u & 0x7FFFFFu) * INV_TWO23;
  return k * (QC_A + f * (QC_B + f * QC_C));
}

// simd_math/ops.mojo:35-69 exp_f32: input clamped to [-87, 88] through
// sign-bit masks, n = trunc(xn + 0.5 - sign(xn)), Cody-Waite reduction with
// two ln2 constants, degree-6 polynomial, times 2^n.
__device__ inline float exp_f32(float x) {
  const float LN2_HI = 0.693145751953125f, LN2_LO = 1.4286068203094172e-06f;
  const float INV_LN2 = 1.4426950408889634f, EXP_LO = -87.0f, EXP_HI = 88.0f;
  const float lo = (float)((__float_as_uint(x - EXP_LO) >> 31) & 1u);
  float xc = x * (1.0f - lo) + EXP_LO * lo;
  const float hi = (float)((__float_as_uint(EXP_HI - xc) >> 31) & 1u);
  xc = xc * (1.0f - hi) + EXP_HI * hi;
  const float xn = xc * INV_LN2;
  const float sign = (float)(__float_as_uint(xn) >> 31);
  const int n = (int)(xn + 0.5f - sign);
  const float nf = (float)n;
  const float r = (xc - nf * LN2_HI) - nf * LN2_LO;
  const float p = 1.0f + r * (0.9999999995f + r * (0.5000000004f + r * (0.1666666456f +
                  r * (0.04166685110f + r * (0.008333621758f + r * 0.001389404636f)))));
  return p * __uint_as_float(((uint32_t)(n + 127)) << 23);
}

// simd_math/ops.mojo:100-124 log_f32: exponent / mantissa split, mantissa
// folded into [sqrt2/2, sqrt2), odd series in z = (m-1)/(m+1).
__device__ inline float log_f32(float x) {
  const float LN2 = 0.6931471805599453f, SQRT2 = 1.4142135623730951f;
  const uint32_t bits = __float_as_uint(x);
  int e = (int)(bits >> 23) - 127;
  float m = __uint_as_float((bits & 0x007FFFFFu) | 0x3F800000u);
  const uint32_t big = __float_as_uint(SQRT2 - m) >> 31;
  m = m * (1.0f - 0.5f * (float)big);
  e = e + (int)big;
  const float z = (m - 1.0f) / (m + 1.0f);
  const float z2 = z * z;
  float t = (float)(1.0 / 11.0);
  t = (float)(1.0 / 9.0) + z2 * t;
  t = (float)(1.0 / 7.0) + z2 * t;
  t = (float)(1.0 / 5.0) + z2 * t;
  t = (float)(1.0 / 3.0) + z2 * t;
  t = 1.0f + z2 * t;
  return 2.0f * z * t + (float)e * LN2;
}

// simd_math/sampling_rng.mojo:10-43: SplitMix64 finalizer, counter
// (row << 32) ^ idx, u = (f32(h >> 40) + 1) / f32(2^24 + 1), Gumbel draw
// -log(-log(u)).
__device__ inline uint64_t mix64(uint64_t x) {
  uint64_t z = x + 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__device__ inline float gumbel_noise(uint64_t seed, int64_t row, int64_t idx) {
  const uint64_t counter = ((uint64_t)row << 32) ^ (uint64_t)idx;
  const uint64_t h = mix64(seed ^ mix64(counter));
  const float top24 = 16777216.0f;
  const float u = ((float)(int64_t)(h >> 40) + 1.0f) / (top24 + 1.0f);
  return -log_f32(-log_f32(u));
}

// ---------------------------------------------------------------------------
// wave helpers
// ---------------------------------------------------------------------------
__device__ inline int lane_id() { return (int)(threadIdx.x & (kWave - 1)); }

// (after the cross-lane partner helpers below)
template <int ST>
__device__ inline float xlane_partner(float v);

__device__ inline float wave_max(float v) {
  v = fmaxf(v, xlane_partner<32>(v));
  v = fmaxf(v, xlane_partner<16>(v));
  v = fmaxf(v, xlane_partner<8>(v));
  v = fmaxf(v, xlane_partner<4>(v));
  v = fmaxf(v, xlane_partner<2>(v));
  v = fmaxf(v, xlane_partner<1>(v));
  return v;
}

// max over aligned groups of `width` lanes (width a power of two <= 64), on
// the VALU lane moves of xlane_partner (defined below)
__device__ inline float group_max(float v, int width) {
  if (width > 32) v = fmaxf(v, xlane_partner<32>(v));
  if (width > 16) v = fmaxf(v, xlane_partner<16>(v));
  if (width > 8) v = fmaxf(v, xlane_partner<8>(v));
  if (width > 4) v = fmaxf(v, xlane_partner<4>(v));
  if (width > 2) v = fmaxf(v, xlane_partner<2>(v));
  if (width > 1) v = fmaxf(v, xlane_partner<1>(v));
  return v;
}

// The value that lane (lane ^ ST) of the wave holds, all on the VALU.  Strides
// 1 and 2 are one DPP quad permutation, stride 8 one DPP row rotation by 8
// (within a row of 16 lanes that is lane ^ 8), stride 4 two DPP row shifts
// (lane + 4 for lanes with bit 2 clear, lane - 4 otherwise) and a select.
// Strides 16 and 32 cross rows: v_permlane16_swap(v, v) leaves row r's
// partner row (r ^ 1) in the second result for even rows and in the first
// for odd rows; v_permlane32_swap(v, v) likewise for the two 32-lane halves.
template <int ST>
__device__ inline float xlane_partner(float v) {
  static_assert(ST >= 1 && ST <= 32 && (ST & (ST - 1)) == 0, "stride");
  const int x = __float_as_int(v);
  // (mov_dpp where every lane is written: no old value to keep, so no copy)
  if constexpr (ST == 1) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, true));  // [1,0,3,2]
  } else if constexpr (ST == 2) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, true));  // [2,3,0,1]
  } else if constexpr (ST == 4) {
    const int up = __builtin_amdgcn_update_dpp(x, x, 0x104, 0xF, 0xF, false);  // row_shl:4
    const int dn = __builtin_amdgcn_update_dpp(x, x, 0x114, 0xF, 0xF, false);  // row_shr:4
    return __int_as_float((threadIdx.x & 4) ? dn : up);
  } else if constexpr (ST == 8) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, true));  // row_ror:8
  } else if constexpr (ST == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap((unsigned)x, (unsigned)x, false, false);
    return __int_as_float((int)((threadIdx.x & 16) ? r[0] : r[1]));
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap((unsigned)x, (unsigned)x, false, false);
    return __int_as_float((int)((threadIdx.x & 32) ? r[0] : r[1]));
  }
}

// The value that lane (lane & 15) + 16 * R of the wave holds, for lanes 0..15
// (row 0; the other lanes get values of no use): row R's lane j brought to
// row 0 by the row swaps of xlane_partner<16> / <32>.
template <int R>
__device__ inline float row_to_row0(float v) {
  static_assert(R >= 0 && R < 4, "row");
  const unsigned x = (unsigned)__float_as_int(v);
  if constexpr (R == 0) {
    return v;
  } else if constexpr (R == 1) {
    return __int_as_float((int)__builtin_amdgcn_permlane16_swap(x, x, false, false)[1]);
  } else if constexpr (R == 2) {
    return __int_as_float((int)__builtin_amdgcn_permlane32_swap(x, x, false, false)[1]);
  } else {
    const unsigned hi = __builtin_amdgcn_permlane32_swap(x, x, false, false)[1];  // row 1: row 3
    return __int_as_float((int)__builtin_amdgcn_permlane16_swap(hi, hi, false, false)[1]);
  }
}

// lane i of row 0 receives lane i + H of the same row (DPP row_shl:H)
template <int H>
__device__ inline float row_shl(float v) {
  const int x = __float_as_int(v);
  return __int_as_float(__builtin_amdgcn_update_dpp(x, x, 0x100 + H, 0xF, 0xF, false));
}

// One element of a cross-lane FWHT stage of stride ST: the lane with bit ST
// clear holds a and gets a + b, its partner holds b and gets a - b.  Computed
// as fmaf(s, v, p) with s = +1 / -1 and p the partner's value: s*v is exact,
// so the one rounding gives exactly v + p (= a + b) or p - v (= a - b).
template <int ST>
__device__ inline float xlane_bfly(float v) {
  return fmaf((threadIdx.x & ST) ? -1.0f : 1.0f, v, xlane_partner<ST>(v));
}

template <int ST>
struct Stride { static constexpr int value = ST; };

// f(Stride<ST>{}) for the cross-lane strides ST = 1, 2, 4, ... below
// min(block, 64), in that order.
template <typename F>
__device__ inline void for_each_xlane_stride(int block, F&& f) {
  if (block > 1) f(Stride<1>{});
  if (block > 2) f(Stride<2>{});
  if (block > 4) f(Stride<4>{});
  if (block > 8) f(Stride<8>{});
  if (block > 16) f(Stride<16>{});
  if (block > 32) f(Stride<32>{});
}

// In-wave FWHT of one segment of S = R*64 values (R = max(1, B/64)), value
// index r*64 + lane.  For B < 64 the wave holds 64/B independent blocks (one
// value per lane, block = lane / B).  Every (a, b) pair of a stage is
// combined as a+b (lower index) and a-b (upper index), exactly as the
// reference's stage loop, so the result is bit-identical to it.
template <int R>
__device__ inline void fwht_wave(float (&v)[R], int block) {
  for_each_xlane_stride(block, [&](auto st) {
    constexpr int ST = decltype(st)::value;
#pragma unroll
    for (int r = 0; r < R; ++r) v[r] = xlane_bfly<ST>(v[r]);
  });
#pragma unroll
  for (int rs = 1; rs < R; rs <<= 1) {
    if (rs * kWave >= block) break;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (r & rs) continue;
      float a = v[r], b = v[r + rs];
      v[r] = a + b;
      v[r + rs] = a - b;
    }
  }
}

// Block-quant of one block of B = 8*LPB values held 8 per lane by LPB
// aligned lanes (lane i of the group owns values [8i, 8i+8)): bf16 values
// widened to f32 in v, [FWHT(B): strides 1, 2, 4 inside the lane, 8 ... B/2
// across lanes, ascending, then x fwht_scale], amax over the block, codes
// q = rne(v * 127/amax) packed little-endian into w (bytes 8i .. 8i+7 of the
// block).  Returns the amax (the block's activation scale).  The op order is
// that of prepare_block_activation (butterquant/runtime.mojo:62-80).
template <int LPB>
__device__ inline float block_quant_lanes(float (&v)[8], bool apply_fwht, float fwht_scale,
                                          uint32_t (&w)[2]) {
  if (apply_fwht) {
#pragma unroll
    for (int s = 1; s < 8; s <<= 1)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (j & s) continue;
        const float a = v[j], b = v[j + s];
        v[j] = a + b;
        v[j + s] = a - b;
      }
    for_each_xlane_stride(LPB, [&](auto st) {
      constexpr int ST = decltype(st)::value;
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = xlane_bfly<ST>(v[j]);
    });
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = v[j] * fwht_scale;
  }
  float m = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(v[j]));
  for_each_xlane_stride(LPB, [&](auto st) { m = fmaxf(m, xlane_partner<decltype(st)::value>(m)); });
  const float inv = m > 0.0f ? 127.0f / m : 0.0f;
  w[0] = w[1] = 0u;
#pragma unroll
  for (int j = 0; j < 8; ++j) w[j >> 2] |= (uint32_t)(uint8_t)quantize_i8(v[j], inv) << (8 * (j & 3));
  return m;
}

// 8 bf16 values (16 bytes) widened to f32
__device__ inline void bf16x8_to_f32(v4i raw, float (&v)[8]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[2 * j] = __uint_as_float((uint32_t)raw[j] << 16);
    v[2 * j + 1] = __uint_as_float((uint32_t)raw[j] & 0xFFFF0000u);
  }
}

// Workgroup barrier for LDS producer/consumer hand-offs: waits for this
// wave's LDS operations only.  (__syncthreads() also carries a release fence,
// which on gfx9 waits for every outstanding global load -- it would drain the
// global-load prefetch pipeline at each stage.)  Global loads land in private
// registers and are waited for by the compiler at their use.
__device__ inline void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// 16-byte global loads/stores
__device__ inline v4i ld16(const int8_t* p) { return *reinterpret_cast<const v4i*>(p); }
__device__ inline void st16(int8_t* p, v4i v) { *reinterpret_cast<v4i*>(p) = v; }

// Sum of squares of a bf16 row in the order of rms_reduce_row (rmsnorm.mojo:
// 16-17 -> dot_products.mojo:144-191): chain c = p*16 + j (p < pu) takes the
// bf16 pairs c + i*pu*16, odd element first; s_j = sum_p chain(p, j) in p
// order; then a 16-lane halving tree.  Wave-uniform result.
__device__ inline float wave_row_ssq(const uint32_t* __restrict__ pairs, int hidden, int pu) {
  const int lane = lane_id();
  const int chains = pu * 16;
  const int iters = hidden / (pu * 32);
  const int c0 = min(lane, chains - 1), c1 = min(lane + 64, chains - 1);
  float a0 = 0.0f, a1 = 0.0f;
#pragma unroll 4
  for (int i = 0; i < iters; ++i) {
    const uint32_t p0 = pairs[i * chains + c0], p1 = pairs[i * chains + c1];
    a0 = fmaf(__uint_as_float(p0 & 0xFFFF0000u), __uint_as_float(p0 & 0xFFFF0000u), a0);
    a0 = fmaf(__uint_as_float(p0 << 16), __uint_as_float(p0 << 16), a0);
    a1 = fmaf(__uint_as_float(p1 & 0xFFFF0000u), __uint_as_float(p1 & 0xFFFF0000u), a1);
    a1 = fmaf(__uint_as_float(p1 << 16), __uint_as_float(p1 << 16), a1);
  }
  float sum = 0.0f;
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const int c = p * 16 + (lane & 15);
    const float v0 = __shfl(a0, c & 63, kWave);
    const float v1 = __shfl(a1, c & 63, kWave);
    if (p < pu) sum = sum + (c < 64 ? v0 : v1);
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) sum = sum + __shfl_down(sum, 8 >> q, 16);
  return __shfl(sum, 0, kWave);
}

__device__ inline v4i mfma16x16x64(v4i a, v4i b, v4i c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// 32x32 output, 32 of K: A lane L = row L%32, K bytes 16*(L/32)..+16; B lane
// L = column L%32, the same K bytes; D lane L register j = row
// 8*(j/4) + 4*(L/32) + j%4, column L%32.  Twice the 16x16x64 product's work
// in twice its cycles: the int8 peak rate (the 16x16x64 form reaches ~3.9
// POPS with 16 independent chains per wave; this one ~4.8 with 4).
__device__ inline v16i mfma32x32x32(v4i a, v4i b, v16i c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

// Inclusive prefix sum over the 64 lanes of a wave by DPP adds: row_shr 1,
// 2, 4, 8 within each 16-lane row, then row_bcast15 / row_bcast31 carry the
// row totals up (lanes a DPP move does not reach add 0).
__device__ inline int wave_incl_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31
  return v;
}

// Map a global m-tile index (BM records per tile, tiles of consecutive
// experts concatenated) to (expert, first record, end record).  Every lane of
// the calling wave gets the same answer.  Up to 256 experts every lane's
// expert offsets are requested at once (one memory round trip, not one per
// 64 experts) and the tile counts are prefix-summed with DPP adds.
__device__ inline bool find_mtile(const int32_t* __restrict__ eo, int E, int BM, int mt,
                                  int max_routes, int& e, int& r0, int& r1) {
  const int lane = lane_id();
  if (E <= 0) return false;
  if (E <= 256) {
    int lo[4], hi[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int ex = min(lane + 64 * q, E - 1);  // lanes past E read a valid offset, count 0
      lo[q] = eo[ex];
      hi[q] = eo[ex + 1];
    }
    int carry = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (64 * q >= E) break;  // uniform
      const int tiles = lane + 64 * q < E ? (hi[q] - lo[q] + BM - 1) / BM : 0;
      const int inc = wave_incl_scan(tiles), excl = inc - tiles;
      const bool hit = tiles > 0 && mt >= carry + excl && mt < carry + inc;
      const unsigned long long m = __ballot(hit);
      if (m) {  // uniform
        const int l = __ffsll((long long)m) - 1;
        e = 64 * q + l;
        const int local = mt - carry - __builtin_amdgcn_readlane(excl, l);
        r0 = __builtin_amdgcn_readlane(lo[q], l) + local * BM;
        r1 = min(min(__builtin_amdgcn_readlane(hi[q], l), r0 + BM), max_routes);
        return r0 < r1;
      }
      carry += __builtin_amdgcn_readlane(inc, 63);
    }
    return false;
  }
  int carry = 0;
  for (int base = 0; base < E; base += 64) {
    const int ex = base + lane;
    int tiles = 0;
    if (ex < E) tiles = (eo[ex + 1] - eo[ex] + BM - 1) / BM;
    const int inc = wave_incl_scan(tiles), excl = inc - tiles;
    const bool hit = tiles > 0 && mt >= carry + excl && mt < carry + inc;
    const unsigned long long m = __ballot(hit);
    if (m) {
      const int l = __ffsll((long long)m) - 1;
      e = base + l;
      const int local = mt - carry - __builtin_amdgcn_readlane(excl, l);
      r0 = eo[e] + local * BM;
      r1 = min(min(eo[e + 1], r0 + BM), max_routes);
      return r0 < r1;
    }
    carry += __builtin_amdgcn_readlane(inc, 63);
  }
  return false;
}

// ---------------------------------------------------------------------------
// Norm-quant in the pair layout (hidden % 256 == 0, so the reference's sum of
// squares runs on pu = 8 port-unrolled accumulators, i.e. 128 chains).  Lane
// L holds the bf16 pair (128 q + 2 L, 128 q + 2 L + 1) of every 128-value
// segment q -- one coalesced 4-byte load per segment -- and with it exactly
// the pairs of chains L (segments 0, 2, 4, ...) and L + 64 (segments 1, 3,
// 5, ...), in chain order (rms_reduce_row, butterquant/runtime.mojo:11-37:
// chain c takes pairs c, c + 128, c + 256, ...; odd element first).  The
// FWHT of block B: stride 1 inside the pair, strides 2 .. 64 across lanes
// (lane ^ s/2), strides 128 and 256 across segments, ascending.  Shared by
// k_norm_quant_pair and the fused norm-quant + linear kernel.

// sum of squares of the row whose pairs xp holds (every segment < nseg), in
// the reference's order: the 128 chains, then s_j = sum over p of chain
// p*16 + j in p order, then the 16-lane halving tree; all 64 lanes active
template <int NSEG>
__device__ inline float nq_pair_sumsq(const uint32_t (&xp)[NSEG], int nseg) {
  float a0 = 0.0f, a1 = 0.0f;  // chains L (even segments) and L + 64 (odd)
#pragma unroll
  for (int q = 0; q < NSEG; q += 2) {
    if (q >= nseg) break;
    const float o0 = __uint_as_float(xp[q] & 0xFFFF0000u), e0 = __uint_as_float(xp[q] << 16);
    const float o1 = __uint_as_float(xp[q + 1] & 0xFFFF0000u), e1 = __uint_as_float(xp[q + 1] << 16);
    a0 = fmaf(o0, o0, a0);
    a0 = fmaf(e0, e0, a0);
    a1 = fmaf(o1, o1, a1);
    a1 = fmaf(e1, e1, a1);
  }
  // lanes 0..15 (row 0) take chains p*16 + j: rows 0..3 of a0, then of a1
  float sum = 0.0f;
  sum = sum + row_to_row0<0>(a0);
  sum = sum + row_to_row0<1>(a0);
  sum = sum + row_to_row0<2>(a0);
  sum = sum + row_to_row0<3>(a0);
  sum = sum + row_to_row0<0>(a1);
  sum = sum + row_to_row0<1>(a1);
  sum = sum + row_to_row0<2>(a1);
  sum = sum + row_to_row0<3>(a1);
  sum = sum + row_shl<8>(sum);
  sum = sum + row_shl<4>(sum);
  sum = sum + row_shl<2>(sum);
  sum = sum + row_shl<1>(sum);
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sum)));  // lane 0
}

// x * inv_rms * gamma of this wave's SPW segments q0 .. q0 + SPW - 1 (pairs
// x[i], gains g[i]; segments >= nseg give 0), the FWHT of block B, times
// fwht_scale, into v; returns the wave-local max |v|
template <int SPW>
__device__ inline float nq_pair_transform(const uint32_t (&x)[SPW], const uint32_t (&g)[SPW],
                                          float inv_rms, int q0, int nseg, int block,
                                          float fwht_scale, float (&v)[SPW][2]) {
#pragma unroll
  for (int i = 0; i < SPW; ++i) {
    if (q0 + i < nseg) {
      const float e = __uint_as_float(x[i] << 16), o = __uint_as_float(x[i] & 0xFFFF0000u);
      const float ge = __uint_as_float(g[i] << 16), go = __uint_as_float(g[i] & 0xFFFF0000u);
      v[i][0] = e * inv_rms * ge;
      v[i][1] = o * inv_rms * go;
    } else {
      v[i][0] = v[i][1] = 0.0f;
    }
  }
  // stride 1 inside the pair
#pragma unroll
  for (int i = 0; i < SPW; ++i) {
    const float x0 = v[i][0], x1 = v[i][1];
    v[i][0] = x0 + x1;
    v[i][1] = x0 - x1;
  }
  // strides 2 .. min(B/2, 64) across lanes: element bit k is lane bit k - 1
  auto lanes = [&](auto st) {
    constexpr int ST = decltype(st)::value;
    if (block > 2 * ST) {
#pragma unroll
      for (int i = 0; i < SPW; ++i)
#pragma unroll
        for (int r = 0; r < 2; ++r) v[i][r] = xlane_bfly<ST>(v[i][r]);
    }
  };
  lanes(Stride<1>{}); lanes(Stride<2>{}); lanes(Stride<4>{});
  lanes(Stride<8>{}); lanes(Stride<16>{}); lanes(Stride<32>{});
  // strides 128 and 256 across segments (SPW and q0 are multiples of B/128)
#pragma unroll
  for (int ss = 1; ss <= 2; ss <<= 1) {
    if (block <= 128 * ss) break;
#pragma unroll
    for (int i = 0; i < SPW; ++i) {
      if ((i & ss) || i + ss >= SPW) continue;
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const float x0 = v[i][r], x1 = v[i + ss][r];
        v[i][r] = x0 + x1;
        v[i + ss][r] = x0 - x1;
      }
    }
  }
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < SPW; ++i)
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      v[i][r] = v[i][r] * fwht_scale;
      m = fmaxf(m, fabsf(v[i][r]));
    }
  return m;
}

// ---------------------------------------------------------------------------
// Norm-quant transform with FWHT block 128 on 8 consecutive values per lane
// (lane L of a 512-value round holds values 8L .. 8L+7, so a 128-value block
// is one row of 16 lanes): x * inv_rms * gain, the FWHT's strides 1, 2, 4
// inside the lane and strides 8, 16, 32, 64 across lanes 1, 2, 4, 8 apart,
// times fwht_scale -- the reference's stages in its order.  Each cross-lane
// stage computes own + s * partner, s = -1 on the upper lane of a pair, so
// the upper lane holds b - a = -(a - b); before every such stage both lanes
// of a pair carry the same sign (the parity of the lane bits already
// crossed), so each stage is exactly a + b / a - b up to that sign
// (negation commutes with round-to-nearest), and the final sign,
// (-1)^parity(lane & 15), is folded into the scale multiply.  Returns the
// lane's max |v|.
__device__ inline float xlane_partner4_banks(float v) {
  // lane ^ 4 inside rows of 16: row_shl:4 written into banks 0 and 2 (lanes
  // 0-3, 8-11), row_shr:4 into banks 1 and 3
  const int x = __float_as_int(v);
  const int t = __builtin_amdgcn_update_dpp(x, x, 0x104, 0xF, 0x5, false);
  return __int_as_float(__builtin_amdgcn_update_dpp(t, x, 0x114, 0xF, 0xA, false));
}

__device__ inline float nq_v8_transform(v4i xv, v4i gv, float inv_rms, float fwht_scale,
                                        float (&v)[8]) {
  const int lane = lane_id();
  const float s1 = (lane & 1) ? -1.0f : 1.0f, s2 = (lane & 2) ? -1.0f : 1.0f;
  const float s4 = (lane & 4) ? -1.0f : 1.0f, s8 = (lane & 8) ? -1.0f : 1.0f;
  const float sc_lane = (__builtin_popcount(lane & 15) & 1) ? -fwht_scale : fwht_scale;
  float xf[8], gf[8];
  bf16x8_to_f32(xv, xf);
  bf16x8_to_f32(gv, gf);
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = xf[j] * inv_rms * gf[j];
#pragma unroll
  for (int st = 1; st < 8; st <<= 1)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (j & st) continue;
      const float a = v[j], b = v[j + st];
      v[j] = a + b;
      v[j + st] = a - b;
    }
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = fmaf(xlane_partner<1>(v[j]), s1, v[j]);
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = fmaf(xlane_partner<2>(v[j]), s2, v[j]);
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = fmaf(xlane_partner4_banks(v[j]), s4, v[j]);
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = fmaf(xlane_partner<8>(v[j]), s8, v[j]);
  float m = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    v[j] = v[j] * sc_lane;
    m = fmaxf(m, fabsf(v[j]));
  }
  return m;
}

// the 8 int8 codes of v, little-endian in two words
__device__ inline void nq_v8_codes(const float (&v)[8], float inv, uint32_t (&w)[2]) {
  w[0] = w[1] = 0u;
#pragma unroll
  for (int j = 0; j < 8; ++j)
    w[j >> 2] |= (uint32_t)(uint8_t)quantize_i8(v[j], inv) << (8 * (j & 3));
}

// the int8 code pair of v[i] (low byte: the even element)
__device__ inline uint16_t nq_pair_code(const float (&vi)[2], float inv) {
  return (uint16_t)((uint8_t)quantize_i8(vi[0], inv) | ((uint16_t)(uint8_t)quantize_i8(vi[1], inv) << 8));
}

// Norm-quant of token t with FWHT block 128 by one wave (hidden % 256 == 0,
// hidden <= 128 * NSEG, 16-byte aligned gain, 8-byte aligned codes): the
// transform on 8 consecutive values per lane (nq_v8_transform, round r of
// 512 values: lane L holds 512 r + 8 L .. + 7), the sum of squares from a
// second read of the row in the pair layout (nq_pair_sumsq: the reference's
// 128 chains in order), the codes of a lane one 8-byte store.
template <int NSEG>
__device__ __attribute__((always_inline)) inline void nq_v8_token(const uint16_t* __restrict__ src,
                                   const uint16_t* __restrict__ gamma, int8_t* __restrict__ xq,
                                   float* __restrict__ sa, int t, int hidden, float sqrt_n,
                                   float n_eps, float fwht_scale) {
  constexpr int NR = (NSEG + 3) / 4;  // rounds of 512 values
  const int lane = lane_id();
  const int nseg = hidden >> 7;
  const uint16_t* row = src + (size_t)t * hidden;
  // the pair layout for the sum of squares, then this lane's 8-value runs
  // (loads return in issue order: the sum of squares' first)
  const uint32_t* xr = reinterpret_cast<const uint32_t*>(row) + lane;
  uint32_t xp[NSEG];
#pragma unroll
  for (int q = 0; q < NSEG; ++q)
    if (q < nseg) xp[q] = xr[64 * q];
  v4i xv[NR], gv[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    // runs past the row are read, never stored
    const int e0 = min(512 * r + 8 * lane, hidden - 8);
    xv[r] = *reinterpret_cast<const v4i*>(row + e0);
    gv[r] = *reinterpret_cast<const v4i*>(gamma + e0);
  }
  const float total = nq_pair_sumsq<NSEG>(xp, nseg);
  const float inv_rms = sqrt_n / __builtin_sqrtf(total + n_eps);
  float v[NR][8];
  float m = 0.0f;
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const float mr = nq_v8_transform(xv[r], gv[r], inv_rms, fwht_scale, v[r]);
    if (512 * r + 8 * lane < hidden) m = fmaxf(m, mr);
  }
  const float amax = wave_max(m);
  const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
  int8_t* qrow = xq + (size_t)t * hidden;
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    if (512 * r + 8 * lane >= hidden) continue;
    uint32_t w[2];
    nq_v8_codes(v[r], inv, w);
    typedef uint32_t u2 __attribute__((ext_vector_type(2)));
    *reinterpret_cast<u2*>(qrow + 512 * r + 8 * lane) = u2{w[0], w[1]};
  }
  if (lane == 0) sa[t] = amax;
}

}  // namespace bq
