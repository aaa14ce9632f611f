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
  uint32_t moved = kShift >= 0 ? (d << kShift) : (d >> (-kShift));
  return as_half2(and_or_b32(moved, 0x03C003C0u, exp16));
}

}  // namespace igl
