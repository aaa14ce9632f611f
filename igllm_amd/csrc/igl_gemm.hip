// igl_gemm.hip - packed int4 projection for batched prefill (M >= 64 lanes),
// gfx950 MFMA, with the reference's float arithmetic.
//
// C[m][n] = sum_g gain[n][g] * sum_{k in g} x[m][k] * (c[n][k] - code_bias - zero[n][g])
// with the codes read straight from the checkpoint's rows (two a byte, low
// nibble first).  This is the reference's back_mat_mat (app_core.c:5247-5323)
// over kern_row_code / kern_row_code_many (3688-3706, 4075-4117) for a lane
// count it would chunk by sixteen: a group's dot product, then its gain, in
// fp32, group after group.
//
// Nothing on the way to the fp32 accumulators is rounded more coarsely than
// the reference rounds:
//   * the weight operand is c - bias - zero as an exact binary16 integer (one
//     v_and_or_b32 puts a nibble in the mantissa of 1024.0, and subtracting
//     1024 + bias + zero is exact); the gain is not folded into it;
//   * the activations of a row are scaled by a power of two 2^t that puts the
//     row's largest magnitude in [2^14, 2^15) and split into binary16 terms:
//     a bf16 activation is exactly one term; an fp32 activation is hi + lo,
//     24 bits but for the last rounding of lo (a relative 2^-22 at most);
//   * one v_mfma_f32_16x16x32_f16 covers exactly one 32-code group, so its
//     fp32 result is that group's dot product (every partial product exact),
//     and one fp32 FMA adds gain * dot to the accumulator, as kern_row_code
//     does;
//   * the row's 2^-t is applied, exactly, at the store.
// Planes with one gain a row accumulate all of K in the matrix cores and take
// the gain once at the store (kern_row_code's single group).
//
// Tiling.  A workgroup of WN x WM x KS waves owns a TN x TM tile of C
// (TN = 16 NB WN weight rows, TM = 16 MB WM lanes).  K advances through LDS
// stages written only by the LDS DMA (global_load_lds: no registers hold loads
// in flight); a stage holds KS consecutive 64-wide steps, and wave group ks of
// the workgroup takes the ks-th: the K split happens inside the workgroup, and
// the KS partial tiles are added in ks order through LDS at the end, so the
// result does not depend on the tiling's timing.  Small tile counts (few
// lanes, or few rows) take a deeper KS; on long rows (K >= 4096) they also
// split K across workgroups (grid z = slice), each slice's fp32 product going
// to the work area and one launch adding the slices in slice order.
#include "igl_device.h"
#include "igl_launch.h"

namespace igl {

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void global_void_t;

constexpr int kStepK = 64;  // k of one wave step: two 32-code groups

// Round-to-nearest-even fp32 -> bf16.
__device__ __forceinline__ uint16_t float_to_bf16(float v) { return __builtin_bit_cast(uint16_t, (__bf16)v); }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// ---- activations -----------------------------------------------------------
//
// One workgroup a row: the row's largest magnitude fixes t, then every eight
// consecutive k are written as binary16 operands in the order the weight
// decoding produces them, positions 0 4 1 5 2 6 3 7, with k = 1, 5, 3, 7
// (where the weight holds 16 (c - bias - zero)) divided by 16, in rows of Kp
// (K padded with zeros to a whole number of steps).  hi =
// binary16(x 2^t), lo = binary16(x 2^t - hi) (both of x 2^t / 16 at the
// divided positions); inv[m] = 2^-t.
// With level_step > 0 (a calibrated plane's prefill) each x is first its
// quant_step level rint(x / level_step) clamped to [-128, 127] (quant_step,
// app_core.c:1930-1940), an integer hi holds exactly.
constexpr int kActThreads = 256;

template <bool IN_BF16>
__device__ __forceinline__ void act_load8(const void *row, int k8, float (&x)[8]) {
  if (IN_BF16) {
    const uint4_t raw = *reinterpret_cast<const uint4_t *>(reinterpret_cast<const uint16_t *>(row) + k8);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = __builtin_bit_cast(float, raw[i] << 16);
      x[2 * i + 1] = __builtin_bit_cast(float, raw[i] & 0xFFFF0000u);
    }
  } else {
    const float4_t *src = reinterpret_cast<const float4_t *>(reinterpret_cast<const float *>(row) + k8);
    const float4_t a = src[0], b = src[1];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[i] = a[i];
      x[4 + i] = b[i];
    }
  }
}

__device__ __forceinline__ float level_of(float x, float step) {
  float level = __builtin_rintf(x / step);
  level = level < -128.0f ? -128.0f : level;
  return level > 127.0f ? 127.0f : level;
}

// A row's values stay in registers between its peak and its conversion: at
// most kActChunks chunks of eight a thread (rows up to 16384 wide in one
// pass); wider rows read their values again for the conversion.
constexpr int kActChunks = 8;

template <bool IN_BF16, bool LO>
__global__ __launch_bounds__(kActThreads) void act_scale_kernel(const void *act, int act_stride, int K,
                                                                  int Kp, _Float16 *hi, _Float16 *lo,
                                                                  float *inv, float level_step) {
  __shared__ float red[kActThreads / 64];
  const int m = blockIdx.x;
  const int tid = threadIdx.x;
  const void *row = IN_BF16 ? static_cast<const void *>(reinterpret_cast<const uint16_t *>(act) + (size_t)m * act_stride)
                            : static_cast<const void *>(reinterpret_cast<const float *>(act) + (size_t)m * act_stride);
  float held[kActChunks][8];
  float peak = 0.0f;
#pragma unroll
  for (int c = 0; c < kActChunks; ++c) {
    const int k8 = (tid + c * kActThreads) * 8;
    if (k8 < K) {
      act_load8<IN_BF16>(row, k8, held[c]);
      if (level_step > 0.0f) {
#pragma unroll
        for (int i = 0; i < 8; ++i) held[c][i] = level_of(held[c][i], level_step);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) peak = fmaxf(peak, fabsf(held[c][i]));
    }
  }
  for (int k8 = (tid + kActChunks * kActThreads) * 8; k8 < K; k8 += kActThreads * 8) {
    float x[8];
    act_load8<IN_BF16>(row, k8, x);
#pragma unroll
    for (int i = 0; i < 8; ++i) peak = fmaxf(peak, fabsf(level_step > 0.0f ? level_of(x[i], level_step) : x[i]));
  }
  peak = wave_max(peak);
  if ((tid & 63) == 0) red[tid >> 6] = peak;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < kActThreads / 64; ++w) peak = fmaxf(peak, red[w]);
  // peak in [2^(e-1), 2^e): t = 15 - e puts it in [2^14, 2^15)
  int t = 0;
  if (peak > 0.0f && peak <= 3.402823466e38f) {
    int e;
    (void)frexpf(peak, &e);
    t = 15 - e;
    t = t < -126 ? -126 : (t > 126 ? 126 : t);
  }
  const float scale = ldexpf(1.0f, t);
  if (tid == 0) inv[m] = ldexpf(1.0f, -t);
  _Float16 *hrow = hi + (size_t)m * Kp;
  _Float16 *lrow = LO ? lo + (size_t)m * Kp : nullptr;
  auto store = [&](int k8, const float (&x)[8]) {
    half8_t h, l;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      // operand slot 2 j + p holds k = j + 4 p, divided by 16 for odd j
      const int j = i >> 1, p = i & 1;
      const float v = x[j + 4 * p] * ((j & 1) ? scale * 0.0625f : scale);
      const _Float16 vh = (_Float16)v;
      h[i] = vh;
      if (LO) l[i] = (_Float16)(v - (float)vh);
    }
    *reinterpret_cast<half8_t *>(hrow + k8) = h;
    if (LO) *reinterpret_cast<half8_t *>(lrow + k8) = l;
  };
#pragma unroll
  for (int c = 0; c < kActChunks; ++c) {
    const int k8 = (tid + c * kActThreads) * 8;
    if (k8 < K) store(k8, held[c]);
  }
  for (int k8 = (tid + kActChunks * kActThreads) * 8; k8 < K; k8 += kActThreads * 8) {
    float x[8];
    act_load8<IN_BF16>(row, k8, x);
    if (level_step > 0.0f) {
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = level_of(x[i], level_step);
    }
    store(k8, x);
  }
  // the padding to a whole step: zeros, so the codes it meets add nothing
  for (int k8 = K + tid * 8; k8 < Kp; k8 += kActThreads * 8) {
    const half8_t z = {0, 0, 0, 0, 0, 0, 0, 0};
    *reinterpret_cast<half8_t *>(hrow + k8) = z;
    if (LO) *reinterpret_cast<half8_t *>(lrow + k8) = z;
  }
}

// ---- the product -----------------------------------------------------------

struct GemmCodesArgs {
  const _Float16 *a_hi;     // [M][K] act_scale_kernel's form
  const _Float16 *a_lo;     // [M][K], two-term activations only
  const float *row_inv;     // [M] 2^-t
  const uint8_t *codes;
  long long row_stride;
  const float *gains;       // [N][gain_stride]
  int gain_stride;
  int group_shift;          // gain of 32-code unit u: u >> group_shift
  const uint32_t *zero_pairs;  // [N][gain_stride] binary16 (1024 + b + z, 1024 + 16 (b + z))
  uint32_t bias_pair;       // the same pair without zero points
  void *out;                // [M][out_stride] bf16 or fp32
  int out_stride;
  int M, N, K;
  int Kp;                   // K padded to whole steps: the activation rows' length
  int slice_k;              // k a workgroup covers: Kp, or K / gridDim.z with K split across workgroups
  long long slice_stride;   // fp32 C only: floats between the partial products of K slices z and z + 1
  igl_gemm_close close;     // fp32 C only: C = grid(close.gains[n] step acc, leave)
};

// The row close of a calibrated plane's product on levels and unit gains:
// gain * step * part (one rounding each, as the reference's level path), then
// the leave grid (quant_step).
__device__ __forceinline__ float close_value(const igl_gemm_close &c, int n, float part) {
  float y = c.gains[n] * c.step * part;
  if (c.leave > 0.0f) {
    float level = __builtin_rintf(y / c.leave);
    level = level < -128.0f ? -128.0f : level;
    level = level > 127.0f ? 127.0f : level;
    y = level * c.leave;
  }
  return y;
}

constexpr int round_up(int v, int q) { return (v + q - 1) / q * q; }

// Waits until this wave's loads but the last N are in (vmcnt retires them in
// issue order) and its LDS reads have landed.
template <int N>
__device__ __forceinline__ void wait_loads() {
  static_assert(N >= 0 && N < 64, "vmcnt holds six bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70);
}

// The stage layout of one form, in bytes.  Every array is padded to a whole
// number of DMA instructions per wave (a lane past the data loads a valid
// address into the padding), so every wave issues the same loads.
template <int WN, int WM, int KS, int NB, int MB, int LIM, bool LO, bool ROWGAIN, bool ZERO>
struct CodesForm {
  static constexpr int W = WN * WM * KS;
  static constexpr int THREADS = 64 * W;
  static constexpr int TN = WN * NB * 16;
  static constexpr int TM = WM * MB * 16;
  static constexpr int A_PAD = round_up(KS * TM * 128, 1024 * W);
  static constexpr int C_PAD = round_up(KS * TN * 32, 1024 * W);
  static constexpr int G_PAD = ROWGAIN ? 0 : round_up(KS * 2 * TN * 4, 256 * W);
  static constexpr int Z_PAD = ZERO ? round_up(KS * 2 * TN * 4, 256 * W) : 0;
  static constexpr int L_OFF = A_PAD;
  static constexpr int C_OFF = A_PAD * (LO ? 2 : 1);
  static constexpr int G_OFF = C_OFF + C_PAD;
  static constexpr int Z_OFF = G_OFF + G_PAD;
  static constexpr int STAGE = Z_OFF + Z_PAD;
  // three stages where they fit the form's LDS budget (LIM KiB: 160 for one
  // workgroup a CU, 80 for two), else two
  static constexpr int STAGES = 3 * STAGE <= LIM * 1024 ? 3 : 2;
  static constexpr int RED = (KS - 1) * TN * TM * 4;
  static constexpr int LDS = STAGES * STAGE > RED ? STAGES * STAGE : RED;
  static constexpr int NA = A_PAD / (1024 * W);
  static constexpr int NC = C_PAD / (1024 * W);
  static constexpr int NG = G_PAD / (256 * W);
  static constexpr int NZ = Z_PAD / (256 * W);
  static constexpr int LOADS = NA * (LO ? 2 : 1) + NC + NG + NZ;
  static_assert(LDS <= LIM * 1024, "LDS");
  static_assert(LOADS * (STAGES - 2) < 64, "vmcnt");
};

template <int WN, int WM, int KS, int NB, int MB, int LIM, bool LO, bool ROWGAIN, bool ZERO, bool C_BF16>
__global__ __launch_bounds__(64 * WN * WM * KS) void gemm_codes_kernel(GemmCodesArgs g) {
  using F = CodesForm<WN, WM, KS, NB, MB, LIM, LO, ROWGAIN, ZERO>;
  constexpr int W = F::W, TN = F::TN, TM = F::TM, STAGES = F::STAGES;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave % WN, wm = (wave / WN) % WM, ks = wave / (WN * WM);
  int tile_x, tile_y;
  xcd_tile(tile_x, tile_y);
  const int n0 = tile_x * TN, m0 = tile_y * TM;
  const int steps = g.slice_k / (kStepK * KS);
  const int kbase = (int)blockIdx.z * g.slice_k;
  const int gq = lane >> 4;  // lane group: k 8 gq .. 8 gq + 7 of a 32-code group
  const int n = lane & 15;

  // DMA sources at step 0.  Activations: 16-byte chunk f of a stage is step
  // f / (8 TM), row (f / 8) % TM, physical chunk f % 8 holding logical chunk
  // (f % 8) ^ ((row >> 1) & 7) (the 16 rows a read spans land in 16 distinct
  // bank groups).  Codes: chunk f is step f / (2 TN), row (f / 2) % TN,
  // physical half f % 2 holding group (f % 2) ^ (bit 3 of the row) (rows r and
  // r + 8 read different banks).  Gains and zero pairs (4 bytes a lane): slot
  // f is group f / TN of the stage (step (f / TN) / 2), row f % TN.
  size_t a_off[F::NA];
#pragma unroll
  for (int u = 0; u < F::NA; ++u) {
    const int f = 64 * (wave + W * u) + lane;
    int kss = 0, row = 0, lc = 0;
    if (f < KS * TM * 8) {
      kss = f / (TM * 8);
      row = (f / 8) % TM;
      lc = (f & 7) ^ ((row >> 1) & 7);
    }
    a_off[u] = (size_t)min(m0 + row, g.M - 1) * g.Kp + kss * kStepK + 8 * lc;
  }
  const uint8_t *c_row[F::NC];
  int c_in[F::NC];
#pragma unroll
  for (int u = 0; u < F::NC; ++u) {
    const int f = 64 * (wave + W * u) + lane;
    int kss = 0, row = 0, lh = 0;
    if (f < KS * TN * 2) {
      kss = f / (TN * 2);
      row = (f / 2) % TN;
      lh = (f & 1) ^ ((row >> 3) & 1);
    }
    c_row[u] = g.codes + (size_t)min(n0 + row, g.N - 1) * (size_t)g.row_stride;
    c_in[u] = kss * (kStepK / 2) + 16 * lh;
  }
  const int row_bytes = g.K / 2;  // a group past K (padding) reads the row's first: its activations are 0
  const unsigned last_unit = (unsigned)(g.K / 32 - 1);
  const float *g_src[F::NG > 0 ? F::NG : 1];
  int g_unit[F::NG > 0 ? F::NG : 1];
#pragma unroll
  for (int u = 0; u < F::NG; ++u) {
    const int f = 64 * (wave + W * u) + lane;
    int kq = 0, row = 0;
    if (f < KS * 2 * TN) {
      kq = f / TN;
      row = f % TN;
    }
    g_src[u] = g.gains + (size_t)min(n0 + row, g.N - 1) * g.gain_stride;
    g_unit[u] = kq;
  }
  const uint32_t *z_src[F::NZ > 0 ? F::NZ : 1];
  int z_unit[F::NZ > 0 ? F::NZ : 1];
#pragma unroll
  for (int u = 0; u < F::NZ; ++u) {
    const int f = 64 * (wave + W * u) + lane;
    int kq = 0, row = 0;
    if (f < KS * 2 * TN) {
      kq = f / TN;
      row = f % TN;
    }
    z_src[u] = g.zero_pairs + (size_t)min(n0 + row, g.N - 1) * g.gain_stride;
    z_unit[u] = kq;
  }
  auto stage = [&](int s) { return lds + (s % STAGES) * F::STAGE; };
  auto issue = [&](int s) {
    uint8_t *st = stage(s);
    const size_t k0 = (size_t)kbase + (size_t)s * (kStepK * KS);
#pragma unroll
    for (int u = 0; u < F::NA; ++u)
      __builtin_amdgcn_global_load_lds((global_void_t *)(g.a_hi + a_off[u] + k0),
                                       (lds_void_t *)(st + 1024 * (wave + W * u)), 16, 0, 0);
    if (LO) {
#pragma unroll
      for (int u = 0; u < F::NA; ++u)
        __builtin_amdgcn_global_load_lds((global_void_t *)(g.a_lo + a_off[u] + k0),
                                         (lds_void_t *)(st + F::L_OFF + 1024 * (wave + W * u)), 16, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < F::NC; ++u) {
      const int b = c_in[u] + (int)(k0 / 2);
      __builtin_amdgcn_global_load_lds((global_void_t *)(c_row[u] + (b < row_bytes ? b : 0)),
                                       (lds_void_t *)(st + F::C_OFF + 1024 * (wave + W * u)), 16, 0, 0);
    }
    const unsigned unit0 = (unsigned)(k0 / 32);
#pragma unroll
    for (int u = 0; u < F::NG; ++u)
      __builtin_amdgcn_global_load_lds(
          (global_void_t *)(g_src[u] + (min(unit0 + (unsigned)g_unit[u], last_unit) >> g.group_shift)),
          (lds_void_t *)(st + F::G_OFF + 256 * (wave + W * u)), 4, 0, 0);
#pragma unroll
    for (int u = 0; u < F::NZ; ++u)
      __builtin_amdgcn_global_load_lds(
          (global_void_t *)(z_src[u] + (min(unit0 + (unsigned)z_unit[u], last_unit) >> g.group_shift)),
          (lds_void_t *)(st + F::Z_OFF + 256 * (wave + W * u)), 4, 0, 0);
  };

  float4_t acc[MB][NB];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[i][j] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const uint32_t exp10 = 0x64006400u;  // 1024.0 in both halves
  const half2_t pair_c = as_half2(g.bias_pair);
  // A dword of eight codes k .. k + 7 as the binary16 operand
  // (k, k+4, 16 k+1, 16 k+5, k+2, k+6, 16 k+3, 16 k+7) minus the bias pair.
  auto decode = [&](uint32_t d, half2_t pair) {
    const half2_t blo = half2_t{pair[0], pair[0]};
    const half2_t bhi = half2_t{pair[1], pair[1]};
    const uint32_t e = d >> 8;
    const half2_t p0 = as_half2(and_or_b32(d, 0x000F000Fu, exp10)) - blo;
    const half2_t p1 = as_half2(and_or_b32(d, 0x00F000F0u, exp10)) - bhi;
    const half2_t p2 = as_half2(and_or_b32(e, 0x000F000Fu, exp10)) - blo;
    const half2_t p3 = as_half2(and_or_b32(e, 0x00F000F0u, exp10)) - bhi;
    return __builtin_bit_cast(half8_t, uint4_t{__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1),
                                               __builtin_bit_cast(uint32_t, p2), __builtin_bit_cast(uint32_t, p3)});
  };

  // Software pipeline: STAGES - 1 steps in flight.  Iteration s waits for
  // step s (this wave's loads but those of the later steps already issued),
  // meets every wave at a bare barrier (step s - 1's stage is then free; a
  // fence would also wait for the later steps' loads), refills that stage
  // with step s + STAGES - 1 and runs step s.
  constexpr int AHEAD = STAGES - 1;
  for (int t = 0; t < AHEAD && t < steps; ++t) issue(t);
  for (int s = 0; s < steps; ++s) {
    if (AHEAD >= 2 && s + 1 < steps)
      wait_loads<F::LOADS * (AHEAD >= 2 ? 1 : 0)>();
    else
      wait_loads<0>();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (s + AHEAD < steps) issue(s + AHEAD);
    const uint8_t *st = stage(s);
    half8_t bf[NB][2];
    float gain[NB][2];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int row = wn * NB * 16 + 16 * j + n;
      const int sw = (row >> 3) & 1;
      const uint8_t *cr = st + F::C_OFF + (ks * TN + row) * 32 + 4 * gq;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const uint32_t d = *reinterpret_cast<const uint32_t *>(cr + 16 * (q ^ sw));
        const int slot = (ks * 2 + q) * TN + row;
        half2_t pair = pair_c;
        if (ZERO) pair = as_half2(*reinterpret_cast<const uint32_t *>(st + F::Z_OFF + 4 * slot));
        bf[j][q] = decode(d, pair);
        if (!ROWGAIN) gain[j][q] = *reinterpret_cast<const float *>(st + F::G_OFF + 4 * slot);
      }
    }
    // The step's MB x NB x 2 products as one chain of tasks (lane block i,
    // row block j, group q): task t's product is issued, then the gain FMAs of
    // task t - kLag, whose product has had kLag products' time to land, so the
    // matrix cores and the FMAs overlap instead of each FMA waiting on its
    // own product.  A lane block's activations are read from LDS one block
    // ahead.
    constexpr int T = MB * NB * 2;
    constexpr int kLag = ROWGAIN ? 0 : 3;
    half8_t ah[2][2], al[2][2];
    auto read_acts = [&](int i, half8_t (&h)[2], half8_t (&l)[2]) {
      const int arow = wm * MB * 16 + 16 * i + n;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int pc = (4 * q + gq) ^ ((arow >> 1) & 7);
        const int at = ((ks * TM + arow) * 64 + 8 * pc) * 2;
        h[q] = *reinterpret_cast<const half8_t *>(st + at);
        if (LO) l[q] = *reinterpret_cast<const half8_t *>(st + F::L_OFF + at);
      }
    };
    read_acts(0, ah[0], al[0]);
    float4_t part[kLag + 1];
#pragma unroll
    for (int t = 0; t < T + kLag; ++t) {
      if (t < T) {
        const int i = t / (NB * 2), j = (t / 2) % NB, q = t & 1;
        if (j == 0 && q == 0 && i + 1 < MB) read_acts(i + 1, ah[(i + 1) & 1], al[(i + 1) & 1]);
        const half8_t &a = ah[i & 1][q];
        if (ROWGAIN) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bf[j][q], acc[i][j], 0, 0, 0);
          if (LO) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i & 1][q], bf[j][q], acc[i][j], 0, 0, 0);
        } else {
          float4_t p = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bf[j][q], float4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
          if (LO) p = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i & 1][q], bf[j][q], p, 0, 0, 0);
          part[t % (kLag + 1)] = p;
        }
      }
      if (!ROWGAIN && t >= kLag) {
        const int u = t - kLag;
        const int i = u / (NB * 2), j = (u / 2) % NB, q = u & 1;
        const float4_t p = part[u % (kLag + 1)];
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][j][r] = __builtin_fmaf(gain[j][q], p[r], acc[i][j][r]);
      }
      // keep the chain's order (the scheduler would otherwise put each FMA
      // right behind its own product)
      if (!ROWGAIN) __builtin_amdgcn_sched_barrier(0);
    }
  }

  // The K split's partial tiles, added in ks order.
  if (KS > 1) {
    __syncthreads();
    float *red = reinterpret_cast<float *>(lds);
    const int tile = wm * WN + wn;
    if (ks > 0) {
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            red[((((ks - 1) * WM * WN + tile) * MB * NB + i * NB + j) * 4 + r) * 64 + lane] = acc[i][j][r];
    }
    __syncthreads();
    if (ks > 0) return;
#pragma unroll
    for (int z = 1; z < KS; ++z)
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            acc[i][j][r] += red[((((z - 1) * WM * WN + tile) * MB * NB + i * NB + j) * 4 + r) * 64 + lane];
  }

  // A 16 x 16 tile of D: lane l holds lanes (C rows) 4 (l / 16) .. + 3 of
  // weight row (C column) l % 16.
  float inv[MB][4];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) inv[i][r] = g.row_inv[min(m0 + wm * MB * 16 + 16 * i + 4 * gq + r, g.M - 1)];
  // Row by row: the wave's NB stores of one output row go out back to back,
  // so each row's NB x 16 contiguous outputs reach the L2 together (with the
  // row blocks outermost, a 256 x 256 tile's bf16 rows were written a quarter
  // line at a time, far apart: 2.5x the output bytes in WRITE_SIZE).
  float row_gain[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j)
    row_gain[j] = ROWGAIN ? g.gains[(size_t)min(n0 + wn * NB * 16 + 16 * j + n, g.N - 1) * g.gain_stride] : 1.0f;
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = m0 + wm * MB * 16 + 16 * i + 4 * gq + r;
      if (m >= g.M) continue;
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int nn = n0 + wn * NB * 16 + 16 * j + n;
        if (nn >= g.N) continue;
        float v = acc[i][j][r] * inv[i][r];
        if (ROWGAIN) v = row_gain[j] * v;
        if (C_BF16) {
          reinterpret_cast<uint16_t *>(g.out)[(size_t)m * g.out_stride + nn] = float_to_bf16(v);
        } else {
          if (g.close.gains) v = close_value(g.close, nn, v);
          reinterpret_cast<float *>(g.out)[(size_t)blockIdx.z * g.slice_stride + (size_t)m * g.out_stride + nn] = v;
        }
      }
    }
}

// ---- K slices ---------------------------------------------------------------
//
// With K split across workgroups each slice's product (already scaled by the
// row's 2^-t, an exact power of two) is an fp32 tile of its own; a thread
// takes V consecutive outputs of a row (V = 4, 16-byte loads, where N is a
// multiple of 4), adds the S slices in slice order (all S loads issued first)
// and converts once.  The order is fixed, so the result does not depend on
// timing.
constexpr int kFoldThreads = 256;

template <int S, int V>
__global__ __launch_bounds__(kFoldThreads) void gemm_slice_fold_kernel(const float *part, long long slice_stride,
                                                                       int M, int N, void *out, int out_bf16,
                                                                       int out_stride) {
  const size_t i = ((size_t)blockIdx.x * kFoldThreads + threadIdx.x) * V;
  if (i >= (size_t)M * (size_t)N) return;
  typedef float vec_t __attribute__((ext_vector_type(V)));
  vec_t v[S];
#pragma unroll
  for (int z = 0; z < S; ++z) v[z] = *reinterpret_cast<const vec_t *>(part + (size_t)z * slice_stride + i);
  vec_t sum = v[0];
#pragma unroll
  for (int z = 1; z < S; ++z) sum += v[z];
  const size_t m = i / (size_t)N, n = i % (size_t)N;
#pragma unroll
  for (int e = 0; e < V; ++e) {
    if (out_bf16)
      reinterpret_cast<uint16_t *>(out)[m * (size_t)out_stride + n + e] = float_to_bf16(sum[e]);
    else
      reinterpret_cast<float *>(out)[m * (size_t)out_stride + n + e] = sum[e];
  }
}

template <int S>
static void launch_fold(const float *part, long long slice_stride, int M, int N, void *out, int out_bf16,
                        int out_stride, hipStream_t stream) {
  const size_t count = (size_t)M * (size_t)N;
  if (N % 4 == 0)
    hipLaunchKernelGGL((gemm_slice_fold_kernel<S, 4>), dim3((unsigned)((count / 4 + kFoldThreads - 1) / kFoldThreads)),
                       dim3(kFoldThreads), 0, stream, part, slice_stride, M, N, out, out_bf16, out_stride);
  else
    hipLaunchKernelGGL((gemm_slice_fold_kernel<S, 1>), dim3((unsigned)((count + kFoldThreads - 1) / kFoldThreads)),
                       dim3(kFoldThreads), 0, stream, part, slice_stride, M, N, out, out_bf16, out_stride);
}

// ---- forms and their choice -----------------------------------------------

// (WN, WM, KS, NB, MB) of the forms, widest tile first; choose_form below
// says which a launch takes.
struct FormShape {
  int wn, wm, ks, nb, mb, lim;
};
constexpr FormShape kForms[] = {
    {4, 2, 1, 4, 8, 160},  // 256 x 256, eight waves
    {2, 2, 2, 4, 4, 160},  // 128 x 128, eight waves, K split in two
    {2, 1, 4, 2, 4, 160},  // 64 x 64, eight waves, K split in four
    {1, 1, 4, 2, 4, 160},  // 32 x 64, four waves, K split in four (three stages fit:
                           // 8192 x 2048 at 64 lanes 19.8 -> 15.5 us against eight)
    {1, 1, 8, 1, 4, 160},  // 16 x 64, eight waves, K split in eight (2048 x 8192 at 64
                           // lanes: 26.5 us, against 29.0 split in four)
    {2, 1, 2, 2, 4, 80},   // 64 x 64, four waves, K split in two, two workgroups a CU
};
constexpr int kPairForm = 5;   // 64 x 64 tiles, two workgroups a CU
constexpr int kSplitForm = 2;  // the form a K split across workgroups takes
// Two-term activations: the same forms with the K split capped where the
// stages would not fit.
constexpr FormShape kFormsLo[] = {
    {4, 2, 1, 4, 4, 160},
    {2, 2, 2, 4, 4, 160},
    {2, 1, 4, 2, 4, 160},
    {1, 1, 4, 2, 4, 160},
    {1, 1, 4, 1, 4, 160},
    {2, 1, 2, 2, 4, 80},
};

// A launch takes, of the forms whose K split divides K:
//   * the 256 x 256 or 128 x 128 form where its tiles fill the 256 CUs;
//   * else, where the 64 x 64 tiles exceed one round of 256 (one workgroup a
//     CU at 126 KB of stages), the same tiles in four-wave workgroups, two a
//     CU at 74-75 KB;
//   * else, of the 64 x 64, 32 x 64 and 16 x 64 forms, the one with the most
//     tiles one round holds.
// Against the widest form that filled the CUs (the choice before), replayed,
// us, bf16 / fp32 activations: 8192 x 2048 at 256 lanes 30.2 / 41.5 -> 27.2 /
// 35.1 (two a CU); 6144 x 1536 at 128 lanes 22.5 / 30.0 -> 15.0 / 18.7 (64 x 64,
// 192 tiles, not 32 x 64 at 384), at 256 lanes 25.3 / 31.9 -> 21.7 / 26.7;
// 12288 x 1536 at 64 lanes 22.4 / 29.8 -> 14.8 / 18.3.  The 128 x 128 form on
// fewer tiles than CUs lost to the two-a-CU form (6144 x 1536 at 256 lanes,
// 96 tiles: 28.5 against 21.7 us).
static int choose_form(int M, int N, int K, int two_terms) {
  const FormShape *forms = two_terms ? kFormsLo : kForms;
  auto divides = [&](int f) { return forms[f].ks > 1 ? K % (kStepK * forms[f].ks) == 0 : K % 32 == 0; };
  auto tiles = [&](int f) {
    const long tn = 16L * forms[f].nb * forms[f].wn, tm = 16L * forms[f].mb * forms[f].wm;
    return ((N + tn - 1) / tn) * ((M + tm - 1) / tm);
  };
  for (int f = 0; f < 2; ++f)
    if (divides(f) && tiles(f) >= 256) return f;
  if (divides(kPairForm) && tiles(kPairForm) > 256) return kPairForm;
  int best = -1;
  for (int f = 2; f < 5; ++f) {
    if (!divides(f)) continue;
    const bool one_round = tiles(f) <= 256;
    if (best < 0 || (one_round && tiles(f) > tiles(best)) || (!one_round && tiles(best) > 256 && tiles(f) < tiles(best)))
      best = f;
  }
  if (best >= 0) return best;
  // K a multiple of 128 but not of 256 takes the two-a-CU form; other K (a
  // multiple of 32) the 256 x 256 form, which pads K to whole steps
  return divides(kPairForm) ? kPairForm : 0;
}

struct GemmPlan {
  int form;
  int slices;  // K split across workgroups: 1, or 2 .. 16 slices folded by gemm_slice_fold_kernel
};

// Long rows (K >= 4096) where choose_form ends past the 128 x 128 form take the
// 64 x 64 form in eight-wave workgroups (at 1024 lanes of 2048 x 8192 the
// two-a-CU form was no faster: 79.0 against 77.0 us), with K split across
// workgroups into S = 1, 2, 4 or 8 slices: each workgroup then
// stages K / S of its lanes' activations instead of all of K, for S fp32
// partial tiles written and folded.  S is the most slices whose workgroups
// still run in one round on the 256 CUs (one a CU at this form's LDS): a
// second round, or more partials, cost more than the shorter K saves (1536 x
// 6144 at 128 lanes: 48 tiles, 19.4 us in four slices, 25.7 in eight; at 512
// lanes 36.7 unsplit, 43.8 in two).  Replayed, us, bf16 / fp32 activations,
// the walk's form against the split:
//   2048 x 8192:  64 lanes 25.0 / 39.9 -> 18.9 / 22.1 (S 8), 128 lanes 26.6 /
//                 43.0 -> 22.8 / 27.3 (S 4), 256 lanes 38.1 / 55.1 -> 30.9 /
//                 39.7 (S 2)
//   1536 x 6144:  64 lanes 20.7 / 32.7 -> 16.5 / 18.2, 256 lanes 36.5 / 62.5
//                 -> 26.9 / 33.2, 512 lanes 53.7 / 77.2 -> 36.7 / 47.4 (S 1)
//   1536 x 12288: 64 lanes 37.2 / 61.9 -> 21.3 / 25.6, 256 lanes 66.2 / 114.7
//                 -> 39.9 / 52.3
// Rows of 2048 (8192 x 2048) were slower split at every lane count tried
// (64-256): the partials cost more than the shorter staging saves.
static GemmPlan choose_plan(int M, int N, int K, int two_terms, bool close) {
  GemmPlan p{choose_form(M, N, K, two_terms), 1};
  if (close || K < 4096 || p.form < kSplitForm) return p;
  const FormShape &s = (two_terms ? kFormsLo : kForms)[kSplitForm];
  if (K % (kStepK * s.ks)) return p;
  const long tiles = (long)((N + 16 * s.nb * s.wn - 1) / (16 * s.nb * s.wn)) *
                     (long)((M + 16 * s.mb * s.wm - 1) / (16 * s.mb * s.wm));
  int slices = 1;
  while (slices < 8 && tiles * 2 * slices <= 256 && K % (2 * slices * kStepK * s.ks) == 0) slices *= 2;
  return GemmPlan{kSplitForm, slices};
}

template <int WN, int WM, int KS, int NB, int MB, int LIM, bool LO, bool ROWGAIN, bool ZERO, bool C_BF16>
static hipError_t launch_form(const GemmCodesArgs &a, hipStream_t stream) {
  using F = CodesForm<WN, WM, KS, NB, MB, LIM, LO, ROWGAIN, ZERO>;
  const void *fn =
      reinterpret_cast<const void *>(&gemm_codes_kernel<WN, WM, KS, NB, MB, LIM, LO, ROWGAIN, ZERO, C_BF16>);
  static bool granted = false;  // the dynamic LDS a kernel asks for is granted once
  if (!granted) {
    const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, F::LDS);
    if (e != hipSuccess) return e;
    granted = true;
  }
  const dim3 grid((a.N + F::TN - 1) / F::TN, (a.M + F::TM - 1) / F::TM, a.Kp / a.slice_k);
  hipLaunchKernelGGL((gemm_codes_kernel<WN, WM, KS, NB, MB, LIM, LO, ROWGAIN, ZERO, C_BF16>), grid, dim3(F::THREADS),
                     (size_t)F::LDS, stream, a);
  return hipGetLastError();
}

template <int F, bool LO, bool ROWGAIN, bool ZERO, bool C_BF16>
static hipError_t launch_shape(const GemmCodesArgs &a, hipStream_t stream) {
  constexpr FormShape s = LO ? kFormsLo[F] : kForms[F];
  return launch_form<s.wn, s.wm, s.ks, s.nb, s.mb, s.lim, LO, ROWGAIN, ZERO, C_BF16>(a, stream);
}

template <bool LO, bool ROWGAIN, bool ZERO, bool C_BF16>
static hipError_t launch_pick(int form, const GemmCodesArgs &a, hipStream_t stream) {
  switch (form) {
    case 0: return launch_shape<0, LO, ROWGAIN, ZERO, C_BF16>(a, stream);
    case 1: return launch_shape<1, LO, ROWGAIN, ZERO, C_BF16>(a, stream);
    case 2: return launch_shape<2, LO, ROWGAIN, ZERO, C_BF16>(a, stream);
    case 3: return launch_shape<3, LO, ROWGAIN, ZERO, C_BF16>(a, stream);
    case 4: return launch_shape<4, LO, ROWGAIN, ZERO, C_BF16>(a, stream);
    default: return launch_shape<5, LO, ROWGAIN, ZERO, C_BF16>(a, stream);
  }
}

template <bool LO, bool ROWGAIN, bool ZERO>
static hipError_t launch_out(int form, int out_bf16, const GemmCodesArgs &a, hipStream_t stream) {
  return out_bf16 ? launch_pick<LO, ROWGAIN, ZERO, true>(form, a, stream)
                  : launch_pick<LO, ROWGAIN, ZERO, false>(form, a, stream);
}

}  // namespace igl

using namespace igl;

static size_t half_bytes(int M, int K) { return ((size_t)M * (size_t)K * sizeof(_Float16) + 255) & ~(size_t)255; }

// K padded to the chosen form's whole steps (only the forms without a K split
// pad: by one 32-code group at most).
static int padded_k(int K) { return (K + kStepK - 1) / kStepK * kStepK; }

extern "C" int igl_gemm_fits(int M, int N, int K) { return M >= 1 && N >= 1 && K >= 32 && K % 32 == 0; }

static size_t inv_bytes(int M) { return ((size_t)M * sizeof(float) + 255) & ~(size_t)255; }

// The K slices' fp32 partial products, [slices][M][N].
static size_t slice_bytes(const GemmPlan &p, int M, int N) {
  return p.slices > 1 ? ((size_t)p.slices * (size_t)M * (size_t)N * sizeof(float) + 255) & ~(size_t)255 : 0;
}

extern "C" size_t igl_gemm_work_bytes(int M, int N, int K, int act_terms) {
  if (!igl_gemm_fits(M, N, K)) return 0;
  return half_bytes(M, padded_k(K)) * (act_terms == 2 ? 2 : 1) + inv_bytes(M) +
         slice_bytes(choose_plan(M, N, K, act_terms == 2, false), M, N);
}

extern "C" int igl_gemm_form(int M, int N, int K, int act_terms) {
  return igl_gemm_fits(M, N, K) ? choose_plan(M, N, K, act_terms == 2, false).form : -1;
}

extern "C" int igl_gemm_slices(int M, int N, int K, int act_terms) {
  return igl_gemm_fits(M, N, K) ? choose_plan(M, N, K, act_terms == 2, false).slices : 0;
}

extern "C" hipError_t igl_launch_gemm_q4(const void *act, int act_bf16, int act_stride, const uint8_t *codes,
                                         long long row_stride, const float *gains, int gain_stride,
                                         int group_shift, int code_bias, const uint32_t *zero_pairs, void *out,
                                         int out_bf16, int out_stride, int M, int N, int K, int act_terms,
                                         void *work, const igl_gemm_close *close, hipStream_t stream) {
  const igl_gemm_close no_close = {nullptr, 0.0f, 0.0f};
  const igl_gemm_close cl = close ? *close : no_close;
  const bool lo = act_terms == 2;
  if (!igl_gemm_fits(M, N, K) || !work || (act_terms != 1 && act_terms != 2) || (lo && act_bf16) ||
      (cl.gains && (out_bf16 || act_bf16)) || ((uintptr_t)act & 15) || (act_stride % (act_bf16 ? 8 : 4)) ||
      code_bias < 0 || code_bias > 15)
    return hipErrorInvalidValue;
  const int Kp = padded_k(K);
  _Float16 *hi = reinterpret_cast<_Float16 *>(work);
  _Float16 *lo_p = reinterpret_cast<_Float16 *>(reinterpret_cast<uint8_t *>(work) + half_bytes(M, Kp));
  float *inv = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(work) + half_bytes(M, Kp) * (lo ? 2 : 1));
  const float level_step = cl.gains ? cl.step : 0.0f;
  if (act_bf16)
    hipLaunchKernelGGL((act_scale_kernel<true, false>), dim3(M), dim3(kActThreads), 0, stream, act, act_stride, K,
                       Kp, hi, lo_p, inv, level_step);
  else if (lo)
    hipLaunchKernelGGL((act_scale_kernel<false, true>), dim3(M), dim3(kActThreads), 0, stream, act, act_stride, K,
                       Kp, hi, lo_p, inv, level_step);
  else
    hipLaunchKernelGGL((act_scale_kernel<false, false>), dim3(M), dim3(kActThreads), 0, stream, act, act_stride, K,
                       Kp, hi, lo_p, inv, level_step);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  GemmCodesArgs a;
  a.a_hi = hi;
  a.a_lo = lo ? lo_p : nullptr;
  a.row_inv = inv;
  a.codes = codes;
  a.row_stride = row_stride;
  a.gains = gains;
  a.gain_stride = gain_stride;
  a.group_shift = group_shift;
  a.zero_pairs = zero_pairs;
  {
    const _Float16 b_lo = (_Float16)(1024.0f + (float)code_bias);
    const _Float16 b_hi = (_Float16)(1024.0f + 16.0f * (float)code_bias);
    a.bias_pair = (uint32_t)__builtin_bit_cast(uint16_t, b_lo) | ((uint32_t)__builtin_bit_cast(uint16_t, b_hi) << 16);
  }
  a.out = out;
  a.out_stride = out_stride;
  a.M = M;
  a.N = N;
  a.K = K;
  a.Kp = Kp;
  a.slice_k = Kp;
  a.slice_stride = 0;
  a.close = cl;
  const GemmPlan plan = choose_plan(M, N, K, lo, cl.gains != nullptr);
  const int form = plan.form;
  int c_bf16 = out_bf16;
  float *part = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(work) + half_bytes(M, Kp) * (lo ? 2 : 1) +
                                          inv_bytes(M));
  if (plan.slices > 1) {
    // each slice's fp32 product into the work area; the fold writes C
    a.slice_k = K / plan.slices;
    a.slice_stride = (long long)M * (long long)N;
    a.out = part;
    a.out_stride = N;
    c_bf16 = 0;
  }
  const bool rowgain = group_shift >= 31;
  const bool zero = zero_pairs != nullptr;
  if (lo) {
    if (rowgain)
      e = zero ? launch_out<true, true, true>(form, c_bf16, a, stream)
               : launch_out<true, true, false>(form, c_bf16, a, stream);
    else
      e = zero ? launch_out<true, false, true>(form, c_bf16, a, stream)
               : launch_out<true, false, false>(form, c_bf16, a, stream);
  } else if (rowgain) {
    e = zero ? launch_out<false, true, true>(form, c_bf16, a, stream)
             : launch_out<false, true, false>(form, c_bf16, a, stream);
  } else {
    e = zero ? launch_out<false, false, true>(form, c_bf16, a, stream)
             : launch_out<false, false, false>(form, c_bf16, a, stream);
  }
  if (e != hipSuccess || plan.slices == 1) return e;
  switch (plan.slices) {
    case 2: launch_fold<2>(part, a.slice_stride, M, N, out, out_bf16, out_stride, stream); break;
    case 4: launch_fold<4>(part, a.slice_stride, M, N, out, out_bf16, out_stride, stream); break;
    case 8: launch_fold<8>(part, a.slice_stride, M, N, out, out_bf16, out_stride, stream); break;
    default: return hipErrorInvalidValue;  // choose_plan takes 1, 2, 4 or 8 slices
  }
  return hipGetLastError();
}
