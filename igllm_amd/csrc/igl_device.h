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

// Sum of one double per thread over a workgroup of WAVES waves, the same
// total in every thread: DPP within each wave, then the wave sums in wave
// order.  `red` holds one double a wave; the trailing barrier lets the caller
// reuse it.  The wave count is a constant, not blockDim: blockDim comes from
// the dispatch packet through a vector load, and the wait for it would also
// wait for every load the kernel issued before it (a GEMV's weights).
// block_sum_f64 without the trailing barrier, for an LDS slot read once.
template <int WAVES = 4>
__device__ __forceinline__ double block_sum_f64_once(double v, double *red) {
  v = wave_sum_f64_to_last(v);
  if ((threadIdx.x & 63) == 63) red[threadIdx.x >> 6] = v;
  __syncthreads();
  double total = red[0];
#pragma unroll
  for (int w = 1; w < WAVES; ++w) total += red[w];
  return total;
}

template <int WAVES = 4>
__device__ __forceinline__ double block_sum_f64(double v, double *red) {
  v = wave_sum_f64_to_last(v);
  if ((threadIdx.x & 63) == 63) red[threadIdx.x >> 6] = v;
  __syncthreads();
  double total = red[0];
#pragma unroll
  for (int w = 1; w < WAVES; ++w) total += red[w];
  __syncthreads();
  return total;
}

// The reference's RMS step (kern_norm_rms, app_core.c:4667-4684):
// (float)pow(square_total / n + eps, -0.5) in double.  Here 1/n and then
// y^-1/2 come from the hardware reciprocal and reciprocal-square-root
// estimates, each refined by two Newton-Raphson steps in double
// (r <- r + r (1 - n r) and r <- r + r (1/2 - y/2 r^2)), which leaves the
// double within a few ulps of pow's; the floats they round to are equal unless
// that double lies within a few ulps of a float rounding boundary (none of
// 16.7M random sums over n = 256, 512, 1536, 2048 differed from the correctly
// rounded 1 / sqrt form).  The dependent chain is a third of the divide /
// square root / divide sequence's (about 100 against 300 shader cycles).
__device__ __forceinline__ float rms_shrink(double square_total, int n, float eps) {
  const double dn = (double)n;
  double inv = __builtin_amdgcn_rcp(dn);
  inv = __builtin_fma(__builtin_fma(-dn, inv, 1.0), inv, inv);
  inv = __builtin_fma(__builtin_fma(-dn, inv, 1.0), inv, inv);
  const double y = __builtin_fma(square_total, inv, (double)eps);
  const double h = 0.5 * y;
  double r = __builtin_amdgcn_rsq(y);
  r = __builtin_fma(r, __builtin_fma(-h * r, r, 0.5), r);
  r = __builtin_fma(r, __builtin_fma(-h * r, r, 0.5), r);
  return (float)r;
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

// ---- activations as signed base-16 digits (the integer-dot GEMV form) -----
//
// A 32-element unit of x is scaled by 2^(P - E), E the frexp exponent of its
// largest |x| and P = 4 DIG - 2 (v_ldexp_f32: exact at any exponent), and
// rounded to the nearest integer q (ties to even), so |q| <= 2^P.  q + B,
// B = 0x888888 cut to DIG hex digits, is then a DIG-digit unsigned number
// whose digits d_j give q = sum_j (d_j - 8) 16^j, and d_j - 8 as a 4-bit
// two's complement value is d_j ^ 8.  A dword of codes c (eight of them, low
// nibble first) xor 0x88888888 is likewise the signed values c - 8, so
// v_dot8_i32_i4 of it against the dword that holds digit j of the same eight
// elements is sum (c - 8)(d_j - 8), exactly, and the DIG of them weighted by
// 16^j give sum (c - 8) q exactly.  The unit's product is that sum, rounded
// once to float, times 2^(E - P) (ldexp again): the only other rounding is
// q's, half a unit in the P-th bit below the unit's largest |x|.  x must be
// finite; a unit of zeros has E = 0 and q = 0.

template <int DIG>
struct DigitForm {
  static_assert(DIG == 5 || DIG == 6, "five or six digits");
  static constexpr int kP = 4 * DIG - 2;
  static constexpr uint32_t kBias = 0x888888u >> (4 * (6 - DIG));
  // bits(x 2^(P - E) + 1.5 * 2^23) = 0x4B400000 + q, as |q| <= 2^22
  static constexpr uint32_t kLess = 0x4B400000u - kBias;
};

// Digits 0 .. DIG-1 of eight elements that share `scale`: nibble e of d[j] is
// digit j of element e.  Three rounds of block swaps (halves between rows
// four apart, bytes two apart, nibbles one apart) transpose the 8 x 8 nibble
// matrix whose row e is element e's biased q.
template <int DIG>
__device__ __forceinline__ void digits_of_eight(const float (&x)[8], int up, uint32_t (&d)[DIG]) {
  uint32_t v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e)
    v[e] = __float_as_uint(__builtin_amdgcn_ldexpf(x[e], up) + 12582912.0f) - DigitForm<DIG>::kLess;
  uint32_t w[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    w[e] = __builtin_amdgcn_perm(v[e + 4], v[e], 0x05040100u);      // a.lo, b.lo
    w[e + 4] = __builtin_amdgcn_perm(v[e + 4], v[e], 0x07060302u);  // a.hi, b.hi
  }
  uint32_t z[8];
#pragma unroll
  for (int h = 0; h < 8; h += 4)
#pragma unroll
    for (int e = h; e < h + 2; ++e) {
      z[e] = __builtin_amdgcn_perm(w[e + 2], w[e], 0x06020400u);      // a0 b0 a2 b2
      z[e + 2] = __builtin_amdgcn_perm(w[e + 2], w[e], 0x07030501u);  // a1 b1 a3 b3
    }
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const uint32_t a = z[e], b = z[e + 1];
    if (e < DIG) d[e] = ((a & 0x0F0F0F0Fu) | ((b << 4) & 0xF0F0F0F0u)) ^ 0x88888888u;
    if (e + 1 < DIG) d[e + 1] = (((a >> 4) & 0x0F0F0F0Fu) | (b & 0xF0F0F0F0u)) ^ 0x88888888u;
  }
}

// sum_j t[j] 16^j as a float, with one rounding: each |t[j]| <= 32 * 64, so
// the two halves are exact in 24 bits.
template <int DIG>
__device__ __forceinline__ float digit_sum(const int (&t)[DIG]) {
  const int lo = t[0] + 16 * t[1] + 256 * t[2];
  int hi = t[3] + 16 * t[4];
  if constexpr (DIG == 6) hi += 256 * t[5];
  return __builtin_fmaf((float)hi, 4096.0f, (float)lo);
}

// ---- the other code widths on the same digit form -------------------------
//
// The staged q is the same 23-bit integer for every code width (P = 22); how
// its digits are laid out in LDS follows the codes it meets:
//   DIGITS_NIBBLE  4-bit codes: six hex digits, nibble e of a dword element e
//                  of its eight (the codes' own order);
//   DIGITS_PAIRS   2-bit codes: the same six hex digits, but the dwords of a
//                  unit hold elements 0,2,..,14 / 1,3,..,15 / 16,18,..,30 /
//                  17,19,..,31, the order in which `w & 0x33333333` and
//                  `(w >> 2) & 0x33333333` spread a dword of sixteen 2-bit
//                  codes into two dwords of nibbles;
//   DIGITS_BYTE    8-bit codes: three base-256 digits, q + 0x808080, byte e
//                  of a dword element e of its four, for v_dot4_i32_i8.
// Every form fills six 16-byte slots a unit, unit-major with a pitch of
// seven: uint4 dig[(m units + u) kDigitPitch + s] (digit_slot).  Nibble forms:
// slot s = digit j, dword k = the k-th eight elements.  Byte form: slot
// 2 j + h = digit j of elements 16 h .. 16 h + 15, four a dword.
// The pair form also stores qsum[m units + u] = sum_e q_e, which takes the
// code bias out of a dot against unsigned codes: sum (c - b) q = sum c q - b qsum.
enum { DIGITS_NIBBLE = 0, DIGITS_PAIRS = 1, DIGITS_BYTE = 2 };

// A unit's digits sit together, so a quad stores them, and a lane reads them,
// at constant offsets from one address; the seventh slot is padding that
// spreads the 16 units a b128 read or a b32 store touches at once over every
// bank (a unit 28 dwords on: 28 u mod 64 is a distinct multiple of 4 for u < 16).
constexpr int kDigitPitch = 7;

__host__ __device__ constexpr int digit_slot(int m, int u, int units) { return (m * units + u) * kDigitPitch; }

template <int BITS>
struct CodeForm {
  static_assert(BITS == 2 || BITS == 4 || BITS == 8, "2, 4 or 8-bit codes");
  static constexpr int kDigits = BITS == 2 ? DIGITS_PAIRS : BITS == 8 ? DIGITS_BYTE : DIGITS_NIBBLE;
  static constexpr int kUnitsPerSlot2 = 256 / (32 * BITS);  // twice the units a 16-byte slot holds
};

constexpr int kDigitP = 22;  // |q| <= 2^22 for every form
constexpr uint32_t kByteBias = 0x808080u;

// Digits 0..2 of four elements in byte form: byte e of d[j] is base-256
// digit j of element e, as a signed byte (d - 128).
__device__ __forceinline__ void bytes_of_four(uint32_t v0, uint32_t v1, uint32_t v2, uint32_t v3,
                                              uint32_t (&d)[3]) {
  const uint32_t t01 = __builtin_amdgcn_perm(v1, v0, 0x05010400u);   // v0.b0 v1.b0 v0.b1 v1.b1
  const uint32_t t23 = __builtin_amdgcn_perm(v3, v2, 0x05010400u);
  const uint32_t t01h = __builtin_amdgcn_perm(v1, v0, 0x07030602u);  // v0.b2 v1.b2 v0.b3 v1.b3
  const uint32_t t23h = __builtin_amdgcn_perm(v3, v2, 0x07030602u);
  d[0] = __builtin_amdgcn_perm(t23, t01, 0x05040100u) ^ 0x80808080u;
  d[1] = __builtin_amdgcn_perm(t23, t01, 0x07060302u) ^ 0x80808080u;
  d[2] = __builtin_amdgcn_perm(t23h, t01h, 0x05040100u) ^ 0x80808080u;
}

// sum_j t[j] 256^j: |t[j]| <= 16 * 128 * 128 per half unit, so t0 + 256 t1
// is an exact int, and the float is formed with two roundings.
__device__ __forceinline__ float byte_digit_sum(int t0, int t1, int t2) {
  return __builtin_fmaf((float)t2, 65536.0f, (float)(t0 + 256 * t1));
}

// sum_j t[j] 16^j - bias qsum as an exact int (|sum c q| <= 3 * 2^22 * 32 and
// |bias qsum| <= 2 * 2^27 for 2-bit codes), rounded once to float.
__device__ __forceinline__ float pair_digit_sum(const int (&t)[6], int bias_qsum) {
  uint32_t v = (uint32_t)t[5];
#pragma unroll
  for (int j = 4; j >= 0; --j) v = (v << 4) + (uint32_t)t[j];
  return (float)(int)(v - (uint32_t)bias_qsum);
}

// One eight-element group (lane m, group gg of K / 8) into LDS in form FORM.
// The four threads of a quad hold one unit's four groups and all four must
// run it (the pair form also trades elements between threads 0-1 and 2-3).
template <int FORM>
__device__ __forceinline__ void digit_group_store_form(const float (&xin)[8], int m, int gg, int units,
                                                       uint4_t *dig, int *down, int *qsum) {
  float peak = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) peak = fmaxf(peak, fabsf(xin[e]));
  peak = fmaxf(peak, dpp_move<0xB1>(peak));  // quad_perm [1,0,3,2]
  peak = fmaxf(peak, dpp_move<0x4E>(peak));  // quad_perm [2,3,0,1]
  const int E = __builtin_amdgcn_frexp_expf(peak);
  const int up = kDigitP - E;
  const int u = gg >> 2, dw = gg & 3;
  uint32_t *base = reinterpret_cast<uint32_t *>(dig);
  float x[8];
  if constexpr (FORM == DIGITS_PAIRS) {
    // Thread dw even holds elements 16h + 0..7 and wants the even ones of
    // 16h + 0..15; its partner (dw + 1) holds 16h + 8..15 and wants the odd.
    const bool odd = dw & 1;
    float recv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) recv[i] = dpp_move<0xB1>(odd ? xin[2 * i] : xin[2 * i + 1]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[i] = odd ? recv[i] : xin[2 * i];
      x[4 + i] = odd ? xin[2 * i + 1] : recv[i];
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = xin[e];
  }
  if constexpr (FORM == DIGITS_BYTE) {
    uint32_t v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
      v[e] = __float_as_uint(__builtin_amdgcn_ldexpf(x[e], up) + 12582912.0f) - (0x4B400000u - kByteBias);
    uint32_t lo[3], hi[3];
    bytes_of_four(v[0], v[1], v[2], v[3], lo);
    bytes_of_four(v[4], v[5], v[6], v[7], hi);
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      uint32_t *slot = base + (digit_slot(m, u, units) + 2 * j + (dw >> 1)) * 4 + 2 * (dw & 1);
      *reinterpret_cast<uint2_t *>(slot) = uint2_t{lo[j], hi[j]};
    }
  } else {
    uint32_t d[6];
    digits_of_eight<6>(x, up, d);
    uint32_t *slot = base + digit_slot(m, u, units) * 4 + dw;
#pragma unroll
    for (int j = 0; j < 6; ++j) slot[4 * j] = d[j];
    if constexpr (FORM == DIGITS_PAIRS) {
      int s = 0;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        s += (int)(__float_as_uint(__builtin_amdgcn_ldexpf(x[e], up) + 12582912.0f) - 0x4B400000u);
      s += __builtin_amdgcn_update_dpp(0, s, 0xB1, 0xF, 0xF, true);
      s += __builtin_amdgcn_update_dpp(0, s, 0x4E, 0xF, 0xF, true);
      if (dw == 0) qsum[m * units + u] = s;
    }
  }
  if (dw == 0) down[m * units + u] = E - kDigitP;
}

// Staging x in digit form, for a workgroup of 256 threads.  Eight-element
// group g of lane m (g < K / 8) is thread (m K / 8 + g) % 256's item
// (m K / 8 + g) / 256; a thread holds GPT items.  The LDS form: uint4
// dig[digit_slot(m, u, units) + j] holds digit j of unit u's four dwords of eight
// elements, and down[m units + u] = E - P.  K % 32 == 0, so the four
// groups of a unit sit in one quad of threads, and a quad is wholly inside
// or wholly past the end.
//
// The loads are a step of their own so that a kernel issues them before its
// weight loads: vmcnt retires loads in order, so activations requested after
// the weights could not be converted until every weight had arrived.
template <int GPT>
struct DigitLoads {
  float x[GPT][8];
};

// An item past the end stands for the same quarter of the last unit, so a
// quad past the end recomputes that unit exactly and its LDS writes repeat
// the owner's values: nothing on the way from the loads to the stores
// branches, and the compiler's wait counts (exact only in straight-line
// code) let the conversion start as soon as the activations arrive.
__device__ __forceinline__ int digit_item(int i, int groups) {
  const int g = (int)threadIdx.x + 256 * i;
  return g < groups ? g : groups - 4 + (g & 3);
}

// VEC: x 16-byte aligned and act_stride % 4 == 0.
template <int M, int GPT, bool VEC>
__device__ __forceinline__ void digit_loads(DigitLoads<GPT> &h, const float *act, int act_stride,
                                            int K) {
  const int per_lane = K >> 3;
#pragma unroll
  for (int i = 0; i < GPT; ++i) {
    const int g = digit_item(i, M * per_lane);
    const int m = M == 1 ? 0 : M == 2 ? (g >= per_lane ? 1 : 0) : g / per_lane;
    const float *src = act + (size_t)m * act_stride + 8 * (g - m * per_lane);
    if (VEC) {
      const float4_t p = *reinterpret_cast<const float4_t *>(src);
      const float4_t q = *reinterpret_cast<const float4_t *>(src + 4);
      h.x[i][0] = p.x; h.x[i][1] = p.y; h.x[i][2] = p.z; h.x[i][3] = p.w;
      h.x[i][4] = q.x; h.x[i][5] = q.y; h.x[i][6] = q.z; h.x[i][7] = q.w;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) h.x[i][e] = src[e];
    }
  }
}

// One eight-element group (lane m, group gg of K / 8) into LDS.  The four
// threads of a quad hold one unit's four groups and all four must run it.
template <int DIG>
__device__ __forceinline__ void digit_group_store(const float (&x)[8], int m, int gg, int units,
                                                  uint4_t *dig, int *down) {
  float peak = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) peak = fmaxf(peak, fabsf(x[e]));
  peak = fmaxf(peak, dpp_move<0xB1>(peak));  // quad_perm [1,0,3,2]
  peak = fmaxf(peak, dpp_move<0x4E>(peak));  // quad_perm [2,3,0,1]
  const int E = __builtin_amdgcn_frexp_expf(peak);
  uint32_t d[DIG];
  digits_of_eight<DIG>(x, DigitForm<DIG>::kP - E, d);
  const int u = gg >> 2, dw = gg & 3;
  uint32_t *base = reinterpret_cast<uint32_t *>(dig);
  uint32_t *slot = base + digit_slot(m, u, units) * 4 + dw;
#pragma unroll
  for (int j = 0; j < DIG; ++j) slot[4 * j] = d[j];
  if (dw == 0) down[m * units + u] = E - DigitForm<DIG>::kP;
}

// The held groups into LDS; ends with a barrier every thread reaches.
template <int M, int GPT, int DIG>
__device__ __forceinline__ void digit_store(const DigitLoads<GPT> &h, int K, uint4_t *dig,
                                            int *down) {
  const int units = K >> 5;
  const int per_lane = K >> 3;
#pragma unroll
  for (int i = 0; i < GPT; ++i) {
    const int g = digit_item(i, M * per_lane);
    const int m = M == 1 ? 0 : M == 2 ? (g >= per_lane ? 1 : 0) : g / per_lane;
    digit_group_store<DIG>(h.x[i], m, g - m * per_lane, units, dig, down);
  }
  __syncthreads();
}

// One lane of x already in LDS (`xs`, K floats, 16-byte aligned) into digit
// form; ends with a barrier every thread reaches.
template <int DIG>
__device__ __forceinline__ void digit_store_lds(const float *xs, int K, uint4_t *dig, int *down) {
  const int units = K >> 5;
  const int groups = K >> 3;
  for (int i = 0; i * 256 < groups; ++i) {
    const int g = digit_item(i, groups);
    const float4_t p = *reinterpret_cast<const float4_t *>(xs + 8 * g);
    const float4_t q = *reinterpret_cast<const float4_t *>(xs + 8 * g + 4);
    const float x[8] = {p.x, p.y, p.z, p.w, q.x, q.y, q.z, q.w};
    digit_group_store<DIG>(x, 0, g, units, dig, down);
  }
  __syncthreads();
}

// ---- activations as grid levels (a plane the export calibrated) -----------
//
// L = rint(x / step) clamped to [-128, 127], quant_step's level (the division
// correctly rounded, as quant_step's).  Nibble forms store two dwords a group
// of eight: `lo` holds L & 15 (unsigned), `hi` holds L >> 4 (a signed
// nibble), so L = 16 hi + lo and a dot against codes splits into one signed
// and one unsigned v_dot8; the byte form stores L itself, four a dword.  The
// element order is the digit form's (DIGITS_PAIRS for 2-bit codes).  LDS,
// unit-major at a pitch of three slots (level_slot; the pad puts the 16 units
// of one b128 read 12 dwords apart, a distinct 4-bank group each):
// uint4 lv[level_slot(m, u, units) + s], s = 0 / 1 the lo / hi dwords (bytes:
// elements 0..15 / 16..31); corr[m units + u] = the bias correction of the unit
// (4-bit: 8 sum lo; 2-bit: code_bias sum L; 8-bit: 0); nanu[m units + u] != 0
// where the unit holds a NaN (its level is no level; the lane's outputs are NaN).
// x / step rounded to nearest, for rounding to a level: with inv = 1 / step
// correctly rounded, q0 = x inv is within an ulp of the quotient, the residual
// x - q0 step is exact (one fma), and q0 + residual inv rounds to the
// correctly rounded quotient (Markstein's theorem on division by a correctly
// rounded reciprocal and an fma correction).  q0 is first clamped to
// [-256, 256] (one med3): below that the clamp changes nothing; past it the
// level clamps at -128 / 127 whatever the correction gives, and the clamp
// keeps an overflowed q0 (an infinity) out of the residual, where inf - inf
// would turn it into a NaN; a NaN x stays NaN through the residual.  A host
// check of 4e8 random and near-half-integer quotients found no level that
// differs from rint(x / step).  The theorem needs inv normal and the residual
// exact (no underflow): step in [2^-96, 2^96] gives both for every quotient
// under 256, and level_recip returns 0 outside it, where the caller divides
// instead.
__device__ __forceinline__ float quot_near(float x, float step, float inv) {
  const float q0 = __builtin_amdgcn_fmed3f(x * inv, -256.0f, 256.0f);
  const float r = __builtin_fmaf(-q0, step, x);
  return __builtin_fmaf(r, inv, q0);
}

__device__ __forceinline__ float level_recip(float step) {
  return step >= 0x1p-96f && step <= 0x1p96f ? 1.0f / step : 0.0f;
}

constexpr int kLevelPitch = 3;

__host__ __device__ constexpr int level_slot(int m, int u, int units) { return (m * units + u) * kLevelPitch; }

// NEAR: x / step by quot_near (inv = level_recip(step) != 0); else divided.
template <int FORM, bool NEAR>
__device__ __forceinline__ void level_group_store(const float (&xin)[8], float step, float inv, int code_bias, int m,
                                                  int gg, int units, uint4_t *lv, int *corr, int *nanu) {
  const int u = gg >> 2, dw = gg & 3;
  float x[8];
  if constexpr (FORM == DIGITS_PAIRS) {
    const bool odd = dw & 1;
    float recv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) recv[i] = dpp_move<0xB1>(odd ? xin[2 * i] : xin[2 * i + 1]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[i] = odd ? recv[i] : xin[2 * i];
      x[4 + i] = odd ? xin[2 * i + 1] : recv[i];
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = xin[e];
  }
  float qt[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) qt[e] = NEAR ? quot_near(x[e], step, inv) : x[e] / step;
  // A NaN quotient (a NaN x) marks the unit; its bytes below are then any
  // value, as the lane's outputs are NaN.
  const int bad = (__builtin_isunordered(qt[0], qt[1]) || __builtin_isunordered(qt[2], qt[3]) ||
                   __builtin_isunordered(qt[4], qt[5]) || __builtin_isunordered(qt[6], qt[7])) ? 1 : 0;
  // B = L + 128 as bytes: rint, the two clamps as one med3, then an exact
  // integer in [0, 255] into its byte (v_cvt_pk_u8_f32)
  auto biased = [&](int e) { return __builtin_amdgcn_fmed3f(__builtin_rintf(qt[e]), -128.0f, 127.0f) + 128.0f; };
  uint32_t *base = reinterpret_cast<uint32_t *>(lv);
  int c = 0;
  if constexpr (FORM == DIGITS_BYTE) {
    // elements 0..3 and 4..7, four a dword, as signed bytes L = B ^ 0x80
    uint32_t b0 = 0, b1 = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      b0 = __builtin_amdgcn_cvt_pk_u8_f32(biased(e), e, b0);
      b1 = __builtin_amdgcn_cvt_pk_u8_f32(biased(e + 4), e, b1);
    }
    *reinterpret_cast<uint2_t *>(base + (level_slot(m, u, units) + (dw >> 1)) * 4 + 2 * (dw & 1)) =
        uint2_t{b0 ^ 0x80808080u, b1 ^ 0x80808080u};
  } else {
    // even and odd elements' bytes: byte k of be / bo is element 2k / 2k + 1,
    // so their low nibbles interleave into L & 15 (nibble e = element e) and
    // their high nibbles into (L >> 4) + 8, a signed nibble once xor 8
    uint32_t be = 0, bo = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      be = __builtin_amdgcn_cvt_pk_u8_f32(biased(2 * k), k, be);
      bo = __builtin_amdgcn_cvt_pk_u8_f32(biased(2 * k + 1), k, bo);
    }
    const uint32_t lo = (be & 0x0F0F0F0Fu) | ((bo << 4) & 0xF0F0F0F0u);
    const uint32_t hi = (((be >> 4) & 0x0F0F0F0Fu) | (bo & 0xF0F0F0F0u)) ^ 0x88888888u;
    uint32_t *slot = base + level_slot(m, u, units) * 4 + dw;
    slot[0] = lo;
    slot[4] = hi;
    if constexpr (FORM == DIGITS_PAIRS) {
      // sum L = sum B - 8 * 128
      const int sum_b = (int)__builtin_amdgcn_udot4(be, 0x01010101u, __builtin_amdgcn_udot4(bo, 0x01010101u, 0u, false), false);
      c = (sum_b - 1024) * code_bias;
    } else {
      c = 8 * (int)__builtin_amdgcn_udot8(lo, 0x11111111u, 0u, false);  // 8 sum (L & 15)
    }
  }
  int bad_sum = bad;
  c += __builtin_amdgcn_update_dpp(0, c, 0xB1, 0xF, 0xF, true);
  c += __builtin_amdgcn_update_dpp(0, c, 0x4E, 0xF, 0xF, true);
  bad_sum += __builtin_amdgcn_update_dpp(0, bad_sum, 0xB1, 0xF, 0xF, true);
  bad_sum += __builtin_amdgcn_update_dpp(0, bad_sum, 0x4E, 0xF, 0xF, true);
  if (dw == 0) {
    corr[m * units + u] = c;
    nanu[m * units + u] = bad_sum;
  }
}

// Items of M lanes into LDS in form FORM; ends with a barrier every thread
// reaches.  Item i of a thread: digit_item.
template <int M, int GPT, int FORM>
__device__ __forceinline__ void digit_store_form(const DigitLoads<GPT> &h, int K, uint4_t *dig,
                                                 int *down, int *qsum) {
  const int units = K >> 5;
  const int per_lane = K >> 3;
#pragma unroll
  for (int i = 0; i < GPT; ++i) {
    const int g = digit_item(i, M * per_lane);
    const int m = M == 1 ? 0 : M == 2 ? (g >= per_lane ? 1 : 0) : g / per_lane;
    digit_group_store_form<FORM>(h.x[i], m, g - m * per_lane, units, dig, down, qsum);
  }
  __syncthreads();
}

// Items of M lanes into LDS as grid levels; ends with a barrier every thread
// reaches.
template <int M, int GPT, int FORM>
__device__ __forceinline__ void level_store_form(const DigitLoads<GPT> &h, int K, float step, int code_bias,
                                                 uint4_t *lv, int *corr, int *nanu) {
  const int units = K >> 5;
  const int per_lane = K >> 3;
  const float inv = level_recip(step);  // once a thread
  // one branch (uniform: one step for the launch), each arm straight-line
  if (inv != 0.0f) {
#pragma unroll
    for (int i = 0; i < GPT; ++i) {
      const int g = digit_item(i, M * per_lane);
      const int m = M == 1 ? 0 : g / per_lane;
      level_group_store<FORM, true>(h.x[i], step, inv, code_bias, m, g - m * per_lane, units, lv, corr, nanu);
    }
  } else {
#pragma unroll
    for (int i = 0; i < GPT; ++i) {
      const int g = digit_item(i, M * per_lane);
      const int m = M == 1 ? 0 : g / per_lane;
      level_group_store<FORM, false>(h.x[i], step, inv, code_bias, m, g - m * per_lane, units, lv, corr, nanu);
    }
  }
  __syncthreads();
}

// One lane of x already in LDS (`xs`, K floats, 16-byte aligned) into form
// FORM; ends with a barrier every thread reaches.
template <int FORM>
__device__ __forceinline__ void digit_store_lds_form(const float *xs, int K, uint4_t *dig, int *down,
                                                     int *qsum) {
  const int units = K >> 5;
  const int groups = K >> 3;
  for (int i = 0; i * 256 < groups; ++i) {
    const int g = digit_item(i, groups);
    const float4_t p = *reinterpret_cast<const float4_t *>(xs + 8 * g);
    const float4_t q = *reinterpret_cast<const float4_t *>(xs + 8 * g + 4);
    const float x[8] = {p.x, p.y, p.z, p.w, q.x, q.y, q.z, q.w};
    digit_group_store_form<FORM>(x, 0, g, units, dig, down, qsum);
  }
  __syncthreads();
}


// The tile (x, y) a workgroup of a 2-D grid computes, so that each of the
// eight XCDs (workgroups go to them round-robin by linear id, each with its
// own L2) owns one compact block of the tile grid: XCD k takes tile rows
// (k / 4) of two and tile columns (k % 4) of four.  Its workgroups then share
// the rows of one operand and the columns of the other in their L2 instead of
// each reading all of one.  Grids whose sides do not divide keep the plain map.
__device__ __forceinline__ void xcd_tile(int &tx, int &ty) {
  const int gx = gridDim.x, gy = gridDim.y;
  tx = blockIdx.x;
  ty = blockIdx.y;
  if (gx % 4 || gy % 2) return;
  const int id = blockIdx.x + blockIdx.y * gx;
  const int k = id & 7, q = id >> 3;
  const int sx = gx / 4, sy = gy / 2;
  tx = (k & 3) * sx + q % sx;
  ty = (k >> 2) * sy + q / sx;
}
}  // namespace igl
