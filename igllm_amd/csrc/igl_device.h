// igl_device.h - device helpers shared by the gfx950 kernels.
//
// Written for CDNA4 (gfx950) only: 64-lane wavefronts, DPP row operations for
// in-wave reductions, packed half-precision registers fed to v_fma_mix_f32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace igl {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef uint32_t uint4_t __attribute__((ext_vector_type(4)));
typedef uint32_t uint2_t __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// A DPP move with out-of-row reads bound to zero.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_move(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xF, true));
}

// Sum of a value over the 64 lanes of a wavefront; the total lands in lane 63
// (other lanes hold partial sums).  Six DPP adds: pairs, quads, half rows and
// rows within each 16-lane row, then the two row broadcasts.
__device__ __forceinline__ float wave_sum_to_last(float v) {
  v += dpp_move<0xB1>(v);        // quad_perm [1,0,3,2]
  v += dpp_move<0x4E>(v);        // quad_perm [2,3,0,1]
  v += dpp_move<0x141>(v);       // row_half_mirror
  v += dpp_move<0x140>(v);       // row_mirror
  v += dpp_move<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
  v += dpp_move<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
  return v;
}

// The same six DPP steps on a double (two 32-bit moves a step).
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ double dpp_move_f64(double v) {
  const uint64_t bits = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)bits, CTRL, ROW_MASK, 0xF, true);
  const uint32_t hi =
      (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(bits >> 32), CTRL, ROW_MASK, 0xF, true);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ double wave_sum_f64_to_last(double v) {
  v += dpp_move_f64<0xB1>(v);
  v += dpp_move_f64<0x4E>(v);
  v += dpp_move_f64<0x141>(v);
  v += dpp_move_f64<0x140>(v);
  v += dpp_move_f64<0x142, 0xA>(v);
  v += dpp_move_f64<0x143, 0xC>(v);
  return v;
}

__device__ __forceinline__ double lane_read_f64(double v, int lane) {
  const uint64_t bits = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)bits, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(bits >> 32), lane);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Sum of one double per thread over a workgroup of up to 16 waves, the same
// total in every thread: DPP within each wave, then the wave sums in wave
// order.  `red` holds one double a wave; the trailing barrier lets the caller
// reuse it.
__device__ __forceinline__ double block_sum_f64(double v, double *red) {
  const int waves = (blockDim.x + 63) >> 6;
  v = wave_sum_f64_to_last(v);
  if ((threadIdx.x & 63) == 63) red[threadIdx.x >> 6] = v;
  __syncthreads();
  double total = red[0];
  for (int w = 1; w < waves; ++w) total += red[w];
  __syncthreads();
  return total;
}

// The reference's RMS step (kern_norm_rms, app_core.c:4667-4684):
// (float)pow(square_total / n + eps, -0.5), as 1 / sqrt in double.  The two
// doubles differ by at most an ulp, so the floats they round to are equal
// unless the double lies within an ulp of a float rounding boundary.
__device__ __forceinline__ float rms_shrink(double square_total, int n, float eps) {
  return (float)(1.0 / __builtin_sqrt(square_total / (double)n + (double)eps));
}

// Sum over each 16-lane row; every lane of the row holds the row total.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_move<0xB1>(v);
  v += dpp_move<0x4E>(v);
  v += dpp_move<0x141>(v);
  v += dpp_move<0x140>(v);
  return v;
}

__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_move<0xB1>(v));
  v = fmaxf(v, dpp_move<0x4E>(v));
  v = fmaxf(v, dpp_move<0x141>(v));
  v = fmaxf(v, dpp_move<0x140>(v));
  return v;
}

__device__ __forceinline__ float lane_read(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

__device__ __forceinline__ half2_t as_half2(uint32_t bits) { return __builtin_bit_cast(half2_t, bits); }

// Two int4 codes of one packed dword as the exact halves (16 + c): the code
// at bit offset `4*i` of the low half and its partner at `16 + 4*i` are moved
// to mantissa bits [6,10) of two binary16 values whose exponent field is 19
// (0x4C00 = 16.0), so each half reads 16 + c with no rounding.
//
// The mask and the exponent are one v_and_or_b32; gfx950's VOP3 encoding takes
// no literal and reads at most one SGPR, so the caller keeps the exponent in a
// VGPR (`exp16`, loaded once) and the mask comes in as an SGPR.
__device__ __forceinline__ uint32_t and_or_b32(uint32_t a, uint32_t mask, uint32_t bits) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(mask), "v"(bits));
  return r;
}

template <int I>
__device__ __forceinline__ half2_t nibble_pair16(uint32_t d, uint32_t exp16) {
  constexpr int kShift = 6 - 4 * I;
  uint32_t moved;
  if constexpr (kShift >= 0)
    moved = d << kShift;
  else
    moved = d >> (-kShift);
  return as_half2(and_or_b32(moved, 0x03C003C0u, exp16));
}

// e4m3 grid rounding of a value already divided by its scale: nearest, ties
// to even, saturating at +-448 (and NaN to +448); below 2^-6 steps of 2^-9; a
// negative that rounds to zero is +0 (cache_pack8/cache_code8,
// app_core.c:10980-11016).
__device__ __forceinline__ uint8_t e4m3_code(float value) {
  const float top = 448.0f, norm = 1.0f / 64.0f, step = 1.0f / 512.0f;
  uint8_t sign = 0;
  float mag = value;
  if (value < 0.0f) { sign = 0x80u; mag = -value; }
  if (!(mag < top)) return (uint8_t)(sign | 0x7Eu);
  if (mag < norm) {
    const float lv = __builtin_rintf(mag / step);
    if (lv == 0.0f) return 0x00u;
    if (lv >= 8.0f) return (uint8_t)(sign | 0x08u);  // rounded up to 2^-6
    return (uint8_t)(sign | (uint8_t)lv);
  }
  int power;
  (void)frexpf(mag, &power);  // mag in [2^(power-1), 2^power)
  const float unit = ldexpf(1.0f, power - 4);
  float r = __builtin_rintf(mag / unit) * unit;
  if (r > top) r = top;
  (void)frexpf(r, &power);
  const int mant = (int)(ldexpf(r, 4 - power) + 0.5f) - 8;
  return (uint8_t)(sign | (uint8_t)((power + 6) << 3) | (uint8_t)mant);
}

// int8 bytes: rint(value / scale) clamped to +-127, two's complement.
__device__ __forceinline__ uint8_t int8_code(float value, float scale) {
  float level = __builtin_rintf(value / scale);
  if (!(level > -127.0f)) level = -127.0f;
  if (level > 127.0f) level = 127.0f;
  return (uint8_t)(int8_t)level;
}

// The reference's series exponential (kern_exp_near, app_core.c:4739-4777):
// 2^k e^r, k the nearest integer to x / ln 2, r reduced in two pieces of ln 2,
// e^r by its Taylor series to the seventh term, arguments below -87 floored.
__device__ __forceinline__ float exp_near(float x) {
  if (x < -87.0f) x = -87.0f;
  const float stepped = x * 1.4426950408889634f + 0.5f;
  float whole = (float)(int)stepped;
  if (whole > stepped) whole -= 1.0f;
  float rest = x - whole * 0.693359375f;
  rest -= whole * -2.1219444005469057e-4f;
  float poly = 1.0f / 5040.0f;
  poly = poly * rest + 1.0f / 720.0f;
  poly = poly * rest + 1.0f / 120.0f;
  poly = poly * rest + 1.0f / 24.0f;
  poly = poly * rest + 1.0f / 6.0f;
  poly = poly * rest + 1.0f / 2.0f;
  poly = poly * rest + 1.0f;
  poly = poly * rest + 1.0f;
  return poly * __builtin_bit_cast(float, (uint32_t)((int)whole + 127) << 23);
}

// gelu_tanh(x) = x t / (t + 1), t = e^(2 sqrt(2/pi)(x + 0.044715 x^3)); zero
// at or below 2y = -30, t clamped at 2y = 30 (kern_gelu_tanh, 5105-5118).
__device__ __forceinline__ float gelu_near(float x) {
  const float cube = x * x * x;
  const float turn = 2.0f * 0.7978845608028654f * (x + 0.044715f * cube);
  if (!(turn > -30.0f)) return x * 0.0f;
  const float t = exp_near(turn > 30.0f ? 30.0f : turn);
  return x * (t / (t + 1.0f));
}

}  // namespace igl
