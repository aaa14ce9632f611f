// igl_gemm.hip - packed int4 projection for batched prefill (M >= 64 lanes),
// gfx950 MFMA.
//
// C[m][n] = sum_k A[m][k] * w[n][k],  w[n][k] = (c[n][k] - code_bias) * gain[n][k / group]
// with the codes read straight from the checkpoint's rows (two a byte, low
// nibble first).  This is the reference's back_mat_mat (app_core.c:5247-5323)
// for a lane count it would chunk by sixteen; the arithmetic is the same
// product, evaluated as a dense contraction.
//
// Each workgroup owns a 128 x 128 tile of C and walks K in steps of 64 (two
// 32-wide groups):
//   * the int4 tile (128 rows x 32 bytes) is read with one 16-byte load a
//     thread, dequantized in registers to binary16 (c - code_bias) * gain and
//     written to LDS;
//   * the activation tile (128 x 64) is read as bf16 or fp32, converted to
//     binary16 and written to LDS;
//   * four waves (2 x 2) each run a 64 x 64 block as 4 x 4
//     v_mfma_f32_16x16x32_f16 tiles, fp32 accumulate.
// binary16 rather than bf16 on both sides: a dequantized weight keeps eleven
// significant bits instead of eight, and bf16 activations convert exactly to
// binary16 over its normal range (|a| < 65504; larger values saturate).
#include "igl_device.h"
#include "igl_launch.h"

namespace igl {

constexpr int kGemmBM = 128;
constexpr int kGemmBN = 128;
constexpr int kGemmBK = 64;
constexpr int kGemmPitch = kGemmBK + 8;  // halves per LDS row (pad breaks bank aliasing)
constexpr int kGemmThreads = 256;

struct GemmArgs {
  const void *act;        // [M][act_stride] of bf16 (raw uint16) or fp32
  int act_stride;
  const uint8_t *codes;
  long long row_stride;
  const float *gains;
  int gain_stride;
  int group_shift;        // gain of unit u: u >> group_shift (31: one gain a row)
  float code_bias;
  void *out;              // [M][out_stride] of bf16 or fp32
  int out_stride;
  int M, N, K;
};

__device__ __forceinline__ _Float16 sat_half(float v) {
  v = fminf(fmaxf(v, -65504.0f), 65504.0f);
  return (_Float16)v;
}

__device__ __forceinline__ float bf16_to_float(uint16_t raw) {
  return __builtin_bit_cast(float, (uint32_t)raw << 16);
}

// Round-to-nearest-even fp32 -> bf16 (NaN kept quiet): the conversion
// instruction, two values at a time where a pair is stored together.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint16_t float_to_bf16(float v) { return __builtin_bit_cast(uint16_t, (__bf16)v); }
__device__ __forceinline__ uint32_t bf16_pair(float lo, float hi) {
  bf16x2_t p;
  p[0] = (__bf16)lo;
  p[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, p);
}

template <bool A_BF16, bool C_BF16>
__global__ __launch_bounds__(kGemmThreads) void gemm_q4_kernel(GemmArgs g) {
  __shared__ _Float16 As[kGemmBM * kGemmPitch];
  __shared__ _Float16 Bs[kGemmBN * kGemmPitch];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1;  // wave row block (M)
  const int wn = wave & 1;   // wave column block (N)
  const int m0 = blockIdx.y * kGemmBM;
  const int n0 = blockIdx.x * kGemmBN;

  float4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // Work assignment for the tile loads.
  const int b_row = tid >> 1;        // 0..127: W row within the tile
  const int b_half = tid & 1;        // which 32-code group of the 64-wide step
  const int n_b = n0 + b_row;

  for (int k0 = 0; k0 < g.K; k0 += kGemmBK) {
    // ---- W tile: 16 bytes (one group of 32 codes) per thread.
    {
      const int kcol = k0 + b_half * 32;
      _Float16 *dst = Bs + b_row * kGemmPitch + b_half * 32;
      if (n_b < g.N && kcol < g.K) {
        const uint4_t w = __builtin_nontemporal_load(reinterpret_cast<const uint4_t *>(
            g.codes + (size_t)n_b * (size_t)g.row_stride + (size_t)(kcol >> 1)));
        const float s = g.gains[(size_t)n_b * g.gain_stride + ((unsigned)(kcol >> 5) >> g.group_shift)];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          half8_t h;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float c = (float)((w[j] >> (4 * i)) & 15u);
            h[i] = (_Float16)((c - g.code_bias) * s);
          }
          *reinterpret_cast<half8_t *>(dst + 8 * j) = h;
        }
      } else {
        const half8_t z = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 4; ++j) *reinterpret_cast<half8_t *>(dst + 8 * j) = z;
      }
    }
    // ---- A tile: 128 rows x 64 columns, 32 values per thread.
    {
      const int a_row = tid >> 1;
      const int a_col = (tid & 1) * 32;
      const int m = m0 + a_row;
      _Float16 *dst = As + a_row * kGemmPitch + a_col;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        half8_t h;
        const int kc = k0 + a_col + 8 * j;
        if (m < g.M && kc < g.K) {
          if (A_BF16) {
            const uint4_t raw = *reinterpret_cast<const uint4_t *>(
                reinterpret_cast<const uint16_t *>(g.act) + (size_t)m * g.act_stride + kc);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              h[2 * i] = sat_half(__builtin_bit_cast(float, raw[i] << 16));
              h[2 * i + 1] = sat_half(__builtin_bit_cast(float, raw[i] & 0xFFFF0000u));
            }
          } else {
            const float *src = reinterpret_cast<const float *>(g.act) + (size_t)m * g.act_stride + kc;
            const float4_t lo = *reinterpret_cast<const float4_t *>(src);
            const float4_t hi = *reinterpret_cast<const float4_t *>(src + 4);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              h[i] = sat_half(lo[i]);
              h[4 + i] = sat_half(hi[i]);
            }
          }
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) h[i] = (_Float16)0.0f;
        }
        *reinterpret_cast<half8_t *>(dst + 8 * j) = h;
      }
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kGemmBK; kk += 32) {
      const int koff = kk + 8 * (lane >> 4);
      half8_t af[4], bf[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        af[i] = *reinterpret_cast<const half8_t *>(As + (wm * 64 + i * 16 + (lane & 15)) * kGemmPitch + koff);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        bf[j] = *reinterpret_cast<const half8_t *>(Bs + (wn * 64 + j * 16 + (lane & 15)) * kGemmPitch + koff);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }

  // D layout of a 16x16 tile: lane l holds rows 4*(l/16) + r, column l % 16.
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + wn * 64 + j * 16 + (lane & 15);
      if (n >= g.N) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * 64 + i * 16 + 4 * (lane >> 4) + r;
        if (m >= g.M) continue;
        if (C_BF16)
          reinterpret_cast<uint16_t *>(g.out)[(size_t)m * g.out_stride + n] = float_to_bf16(acc[i][j][r]);
        else
          reinterpret_cast<float *>(g.out)[(size_t)m * g.out_stride + n] = acc[i][j][r];
      }
    }
}

// ---- the large-tile form ---------------------------------------------------
//
// For M and N of 256 and up, K a multiple of 64.  The activations are first
// converted once to a binary16 copy (act_half_kernel) in the operand order
// the weights are decoded in (below), so the tile loop only moves them.
//
// A workgroup owns a 256 x 256 tile of C; its eight waves (2 x 4) each hold a
// 128 x 64 block as 8 x 4 v_mfma_f32_16x16x32_f16 accumulators.  K advances
// 64 a step through LDS stages that only the LDS DMA writes (global_load_lds:
// no registers held for loads in flight):
//   * three stages of the step's 256 x 64 binary16 activations (two steps
//     ahead), 16-byte chunks of a row XOR-swizzled by bits 1..3 of the row
//     (no padding; the 16 rows of a read land in 16 distinct 16-byte slots
//     of the 64 banks.  Measured alone, these reads count the conflict
//     counter's floor of four cycles per 64-lane 16-byte read, as the row's
//     low three bits do; unswizzled, three times that);
//   * four stages (three steps ahead) of the 256 rows' 64 codes as they are
//     packed (32 bytes a row) and their two fp32 gains.
// A wave turns its 64 columns' codes into binary16 operands in registers as
// it consumes them: one v_and_or_b32 puts a nibble in the mantissa of 1024.0
// (ulp 1: 1024 + c) or, four bits up, of 1024.0 with ulp 16 (1024 + 16 c), so
// a dword of eight codes takes one shift; subtracting 1024 + bias (or
// 1024 + 16 bias) is exact, and one multiply by the gain rounded to binary16
// gives (c - bias) gain or 16 (c - bias) gain, rounded once.  The activation
// copy holds x / 16 where the weight holds 16 (c - bias) gain, and each eight
// consecutive k appear in the order 0 4 1 5 2 6 3 7 the pairs come in.
// A wave's step runs 64 products in eight blocks of eight, reading the next
// block's activations and decoding one of the next step's eight weight
// operands beside each block.  The weights are the products' first operand,
// so each accumulator holds C transposed: four consecutive columns of one row,
// stored as one vector.
//
// Measured on this tile (M = 2048, 8192 x 2048): the same loop with only its
// products (no decode, no activation reads, no DMA) takes ~70% of the whole
// kernel, and the final 32 MB of output drains in ~15 us with every CU
// finishing its one tile at once.
constexpr int kBigM = 256;
constexpr int kBigN = 256;
constexpr int kBigK = 64;
constexpr int kBigStages = 3;                 // activation stages (DMA two steps ahead)
constexpr int kBigCodeStages = 4;             // code stages (decoded a step early)
constexpr int kBigA = kBigM * kBigK;          // halves of a stage's activations
constexpr int kBigB = kBigN * kBigK / 2;      // bytes of a stage's codes
constexpr int kBigG = kBigN * kBigK / 32;     // floats of a stage's gains
constexpr int kBigCodeStage = kBigB + kBigG * 4;
constexpr int kBigLds = kBigStages * kBigA * 2 + kBigCodeStages * kBigCodeStage;

// a16 = binary16(a), saturating at +-65504, in the large-tile form's operand
// order: within each eight k, positions 0 4 1 5 2 6 3 7, and k = 1, 5, 3, 7
// divided by 16 (exact for every normal binary16).
// With level_step > 0 (a calibrated plane's prefill), each x is first its
// quant_step level rint(x / level_step) clamped to [-128, 127]: an integer the
// binary16 operand holds exactly (and so does a level / 16).
// Rows a thread of act_half_kernel converts (its loads all issued first).
constexpr int kHalfRows = 4;

template <bool A_BF16>
__global__ void act_half_kernel(const void *act, int act_stride, int M, int K, _Float16 *a16,
                                float level_step) {
  const int k8 = (blockIdx.x * blockDim.x + threadIdx.x) * 8;
  const int m0 = blockIdx.y * kHalfRows;
  if (k8 >= K) return;
  float x[kHalfRows][8];
#pragma unroll
  for (int r = 0; r < kHalfRows; ++r) {
    const int m = min(m0 + r, M - 1);  // rows past M reread the last one, not stored
    if (A_BF16) {
      // rows are 16-byte aligned (act_stride % 8 == 0): one load for 8 values
      const uint4_t raw = *reinterpret_cast<const uint4_t *>(
          reinterpret_cast<const uint16_t *>(act) + (size_t)m * act_stride + k8);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x[r][2 * i] = __builtin_bit_cast(float, raw[i] << 16);
        x[r][2 * i + 1] = __builtin_bit_cast(float, raw[i] & 0xFFFF0000u);
      }
    } else {
      const float4_t *src = reinterpret_cast<const float4_t *>(
          reinterpret_cast<const float *>(act) + (size_t)m * act_stride + k8);
      const float4_t lo = src[0], hi = src[1];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x[r][i] = lo[i];
        x[r][4 + i] = hi[i];
      }
    }
  }
  const _Float16 sixteenth = (_Float16)0.0625f;
#pragma unroll
  for (int r = 0; r < kHalfRows; ++r) {
    if (m0 + r >= M) break;
    if (level_step > 0.0f) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float level = __builtin_rintf(x[r][i] / level_step);
        level = level < -128.0f ? -128.0f : level;
        x[r][i] = level > 127.0f ? 127.0f : level;
      }
    }
    half8_t h;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool up = i & 1;  // k = 1, 3 and their partners 5, 7
      const _Float16 a = sat_half(x[r][i]), b = sat_half(x[r][i + 4]);
      h[2 * i] = up ? a * sixteenth : a;
      h[2 * i + 1] = up ? b * sixteenth : b;
    }
    *reinterpret_cast<half8_t *>(a16 + (size_t)(m0 + r) * K + k8) = h;
  }
}

struct GemmBigArgs {
  const _Float16 *a16;    // [M][K], act_half_kernel's form
  const uint8_t *codes;
  long long row_stride;
  const float *gains;
  int gain_stride;
  int group_shift;
  float code_bias;
  void *out;              // C, or with K slices fp32 partials [slice][M][N]
  int out_stride;
  int M, N, K;            // K: the whole plane's columns
  int k_steps;            // 64-wide steps of one K slice (blockIdx.z)
  size_t slice_floats;    // floats between slices' partials (0: no split)
  igl_gemm_close close;   // fp32 C only: C = grid(close.gains[n] step acc, leave)
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

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void global_void_t;

template <bool C_BF16>
__global__ __launch_bounds__(512) void gemm_q4_big_kernel(GemmBigArgs g) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds_b[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2;      // 2 wave rows of 128
  const int wn = wave & 3;       // 4 wave columns of 64
  int tile_x, tile_y;
  xcd_tile(tile_x, tile_y);
  const int m0 = tile_y * kBigM;
  const int n0 = tile_x * kBigN;
  const int steps = g.k_steps;
  const int k_first = blockIdx.z * g.k_steps * kBigK;

  // DMA sources (a lane's 16 bytes land at the wave's LDS address + 16 lane).
  // Activations: wave w's instruction i fills rows 8 (4 w + i) .. +7, lane l
  // row R0 + l / 8 at physical chunk l % 8, logical chunk (l % 8) ^ ((row >> 1) & 7).
  const _Float16 *a_src[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 8 * (4 * wave + i) + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    a_src[i] = g.a16 + (size_t)min(m0 + r, g.M - 1) * g.K + k_first + 8 * c;
  }
  // codes: wave w fills rows 32 w .. +31, lane l row 32 w + l / 2, physical
  // half l & 1, which holds logical half (l & 1) ^ (bit 3 of the row): rows
  // n and n + 8 then read their eight bytes from different banks.  Gains
  // (4 bytes a lane): the same rows, group l & 1.
  const int br = min(n0 + 32 * wave + (lane >> 1), g.N - 1);
  const uint8_t *b_src = g.codes + (size_t)br * (size_t)g.row_stride + k_first / 2 +
                         16 * ((lane & 1) ^ ((lane >> 4) & 1));
  const float *s_src = g.gains + (size_t)br * g.gain_stride;
  const int s_first = k_first / 32;
  const int s_grp = lane & 1;
  // Activation stages first, then the code stages.
  auto a_stage = [&](int step) { return lds_b + (step % kBigStages) * (kBigA * 2); };
  auto b_stage = [&](int step) { return lds_b + kBigStages * kBigA * 2 + (step % kBigCodeStages) * kBigCodeStage; };
  auto issue_a = [&](int step) {
    uint8_t *st = a_stage(step);
    const int k0 = step * kBigK;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_global_load_lds((global_void_t *)(a_src[i] + k0),
                                       (lds_void_t *)(st + (4 * wave + i) * 1024), 16, 0, 0);
  };
  auto issue_b = [&](int step) {
    uint8_t *st = b_stage(step);
    const int k0 = step * kBigK;
    __builtin_amdgcn_global_load_lds((global_void_t *)(b_src + k0 / 2), (lds_void_t *)(st + wave * 1024), 16, 0, 0);
    __builtin_amdgcn_global_load_lds(
        (global_void_t *)(s_src + (((unsigned)(s_first + k0 / 32 + s_grp)) >> g.group_shift)),
        (lds_void_t *)(st + kBigB + wave * 256), 4, 0, 0);
  };

  float4_t acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const uint32_t exp10 = 0x64006400u;  // 1024.0 in both halves
  const _Float16 lo_bias = (_Float16)(1024.0f + g.code_bias);
  const _Float16 hi_bias = (_Float16)(1024.0f + 16.0f * g.code_bias);
  const half2_t bias_lo = half2_t{lo_bias, lo_bias};
  const half2_t bias_hi = half2_t{hi_bias, hi_bias};
  const int gq = lane >> 4;     // lane group: k 16 gq .. 16 gq + 15 of a step
  const int n = lane & 15;

  // The codes of a step are read and decoded into binary16 operands a step
  // ahead, eight fragments a step: one v_and_or_b32 puts a nibble pair in the
  // mantissas of 1024.0 (ulp 1, or four bits up ulp 16); subtracting
  // 1024 + bias (or 1024 + 16 bias) is exact; one multiply by the gain rounds
  // once.  k-half q of lane group gq is k 16 gq + 8 q .. + 7: its activations
  // are logical chunk 2 gq + q of the row, its codes dword q of the eight bytes.
  auto read_codes = [&](const uint8_t *st, uint2_t (&braw)[4], half2_t (&bscale)[4]) {
    const float *gs = reinterpret_cast<const float *>(st + kBigB);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = wn * 64 + 16 * j + n;
      const int half = (gq >> 1) ^ ((n >> 3) & 1);
      braw[j] = *reinterpret_cast<const uint2_t *>(st + row * 32 + 16 * half + 8 * (gq & 1));
      const _Float16 sh = (_Float16)gs[row * 2 + (gq >> 1)];
      bscale[j] = half2_t{sh, sh};
    }
  };
  auto read_rows = [&](const uint8_t *st, int i, half8_t (&a)[2]) {
    const _Float16 *as = reinterpret_cast<const _Float16 *>(st);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int r = wm * 128 + 16 * i + n;
      const int p = (2 * gq + q) ^ ((r >> 1) & 7);
      a[q] = *reinterpret_cast<const half8_t *>(as + r * kBigK + 8 * p);
    }
  };
  auto decode = [&](uint32_t d, half2_t scale) {
    const uint32_t e = d >> 8;
    const half2_t p0 = (as_half2(and_or_b32(d, 0x000F000Fu, exp10)) - bias_lo) * scale;
    const half2_t p1 = (as_half2(and_or_b32(d, 0x00F000F0u, exp10)) - bias_hi) * scale;
    const half2_t p2 = (as_half2(and_or_b32(e, 0x000F000Fu, exp10)) - bias_lo) * scale;
    const half2_t p3 = (as_half2(and_or_b32(e, 0x00F000F0u, exp10)) - bias_hi) * scale;
    return __builtin_bit_cast(half8_t, uint4_t{__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1),
                                               __builtin_bit_cast(uint32_t, p2), __builtin_bit_cast(uint32_t, p3)});
  };
  // Waits until this wave's loads but the last `after` are in (vmcnt retires
  // them in order) and its LDS reads have landed (the stages they read are
  // refilled after the next barrier), then meets every wave at a bare barrier
  // (a fence would also wait for the loads still in flight for later steps).
  auto wait_meet = [&](int after) {
    if (after >= 12)
      __builtin_amdgcn_s_waitcnt(0x007C);  // vmcnt(12) lgkmcnt(0)
    else if (after >= 6)
      __builtin_amdgcn_s_waitcnt(0x0076);  // vmcnt(6) lgkmcnt(0)
    else if (after >= 4)
      __builtin_amdgcn_s_waitcnt(0x0074);  // vmcnt(4) lgkmcnt(0)
    else
      __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  // Software pipeline.  Iteration s issues the activations of step s + 2 and
  // the codes of step s + 3, and runs step s's 64 products in eight blocks of
  // eight; between the blocks it reads step s's next row tile of activations
  // (one block ahead) and decodes one of step s + 1's eight code fragments, so
  // the decoding runs beside the matrix cores instead of between steps.  A
  // wave's loads retire in issue order: before iteration s they are ...,
  // [A s, B s+1], [A s+1, B s+2] (4 + 2 each), so A s and B s+1 are in when
  // all but the last 4 [s+1 < steps] + 2 [s+2 < steps] are.
  issue_b(0);
  issue_a(0);
  if (steps > 1) issue_b(1);
  if (steps > 1) issue_a(1);
  if (steps > 2) issue_b(2);
  wait_meet((steps > 1 ? 10 : 0) + (steps > 2 ? 2 : 0) >= 12 ? 12 : 0);
  half8_t bf[2][4];
  {
    uint2_t braw[4];
    half2_t bscale[4];
    read_codes(b_stage(0), braw, bscale);
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int j = 0; j < 4; ++j) bf[q][j] = decode(braw[j][q], bscale[j]);
  }
  for (int s = 0; s < steps; ++s) {
    wait_meet(4 * (s + 1 < steps) + 2 * (s + 2 < steps));
    if (s + 2 < steps) issue_a(s + 2);
    if (s + 3 < steps) issue_b(s + 3);
    const bool more = s + 1 < steps;
    const uint8_t *ast = a_stage(s);
    half8_t bn[2][4];
    uint2_t braw[4];
    half2_t bscale[4];
    read_codes(b_stage(more ? s + 1 : s), braw, bscale);
    half8_t a_cur[2], a_next[2];
    read_rows(ast, 0, a_cur);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (i + 1 < 8) read_rows(ast, i + 1, a_next);
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf[q][j], a_cur[q], acc[i][j], 0, 0, 0);
      bn[i >> 2][i & 3] = decode(braw[i & 3][i >> 2], bscale[i & 3]);
      __builtin_amdgcn_sched_barrier(0);
      a_cur[0] = a_next[0];
      a_cur[1] = a_next[1];
    }
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int j = 0; j < 4; ++j) bf[q][j] = bn[q][j];
  }

  // The products take the codes as the first operand, so a 16x16 tile of D is
  // C transposed: lane l holds row l % 16 of its row tile and the four
  // consecutive columns 4 (l / 16) .. + 3, stored as one 8- or 16-byte vector.
  float *part = reinterpret_cast<float *>(g.out) + blockIdx.z * g.slice_floats;
  const bool vec_ok = g.slice_floats ? (g.N % 4 == 0)
                                     : (g.out_stride % 4 == 0 &&
                                        ((uintptr_t)g.out & (C_BF16 ? 7u : 15u)) == 0);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int m = m0 + wm * 128 + i * 16 + n;
    if (m >= g.M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int nb = n0 + wn * 64 + j * 16 + 4 * gq;
      float4_t v = acc[i][j];
      if (!g.slice_floats && !C_BF16 && g.close.gains) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (nb + r < g.N) v[r] = close_value(g.close, nb + r, v[r]);
      }
      if (vec_ok && nb + 3 < g.N) {
        if (g.slice_floats) {
          *reinterpret_cast<float4_t *>(part + (size_t)m * g.N + nb) = v;
        } else if (C_BF16) {
          const uint32_t lo = bf16_pair(v[0], v[1]);
          const uint32_t hi = bf16_pair(v[2], v[3]);
          *reinterpret_cast<uint2_t *>(reinterpret_cast<uint16_t *>(g.out) + (size_t)m * g.out_stride + nb) =
              uint2_t{lo, hi};
        } else {
          *reinterpret_cast<float4_t *>(reinterpret_cast<float *>(g.out) + (size_t)m * g.out_stride + nb) = v;
        }
        continue;
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int nn = nb + r;
        if (nn >= g.N) continue;
        if (g.slice_floats)
          part[(size_t)m * g.N + nn] = v[r];
        else if (C_BF16)
          reinterpret_cast<uint16_t *>(g.out)[(size_t)m * g.out_stride + nn] = float_to_bf16(v[r]);
        else
          reinterpret_cast<float *>(g.out)[(size_t)m * g.out_stride + nn] = v[r];
      }
    }
  }
}

// C = the K slices' partials added in slice order (four columns a thread).
template <bool C_BF16>
__global__ void gemm_slice_sum_kernel(const float *part, int slices, size_t slice_floats, int M,
                                      int N, void *out, int out_stride, igl_gemm_close close) {
  const int n = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
  const int m = blockIdx.y;
  if (n >= N) return;
  const float *src = part + (size_t)m * N + n;
  float4_t t = *reinterpret_cast<const float4_t *>(src);
  for (int z = 1; z < slices; ++z) t += *reinterpret_cast<const float4_t *>(src + z * slice_floats);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if (n + e >= N) break;
    if (C_BF16)
      reinterpret_cast<uint16_t *>(out)[(size_t)m * out_stride + n + e] = float_to_bf16(t[e]);
    else
      reinterpret_cast<float *>(out)[(size_t)m * out_stride + n + e] =
          close.gains ? close_value(close, n + e, t[e]) : t[e];
  }
}

// ---- the skinny form (64 <= M < 256 lanes) --------------------------------
//
// Few lanes leave the product bound by the weight stream, which must be read
// once: a workgroup of four waves owns 128 weight rows x 64 lanes and walks its
// K slice in steps of 64, with the large-tile form's operand order, decoding
// and DMA staging (three stages, issued two steps ahead; eight stages measured
// slower: a CU's outstanding reads, not their latency, bound the stream).  Wave w decodes rows
// 32 w .. 32 w + 31 and multiplies them by all 64 lanes (2 x 4 products of
// 16 x 16 a k-half), so no row is decoded twice.  K slices (blockIdx.z) keep
// at least 128 workgroups; their fp32 partials are added in slice order by
// gemm_slice_sum_kernel.
constexpr int kMidM = 64;
constexpr int kMidN = 128;
constexpr int kMidK = 64;
constexpr int kMidStages = 3;
constexpr int kMidAhead = kMidStages - 1;
constexpr int kMidA = kMidM * kMidK;                  // halves of a stage's activations
constexpr int kMidB = kMidN * kMidK / 2;              // bytes of a stage's codes
constexpr int kMidG = kMidN * kMidK / 32;             // floats of a stage's gains
constexpr int kMidStage = kMidA * 2 + kMidB + kMidG * 4;
constexpr int kMidLds = kMidStages * kMidStage;

template <bool C_BF16>
__global__ __launch_bounds__(256) void gemm_q4_mid_kernel(GemmBigArgs g) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds_m[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n0 = blockIdx.x * kMidN;
  const int m0 = blockIdx.y * kMidM;
  const int steps = g.k_steps;
  const int k_first = blockIdx.z * g.k_steps * kMidK;

  // DMA sources.  Activations: wave w's instruction i fills rows 8 (2 w + i)
  // .. +7, lane l row R0 + l / 8 at physical chunk l % 8, logical chunk
  // (l % 8) ^ ((row >> 1) & 7).  Codes: wave w fills rows 32 w .. +31, lane l row
  // 32 w + l / 2, physical half l & 1 holding logical half (l & 1) ^ (bit 3 of
  // the row).  Gains: the same rows, group l & 1.
  const _Float16 *a_src[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = 8 * (2 * wave + i) + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    a_src[i] = g.a16 + (size_t)min(m0 + r, g.M - 1) * g.K + k_first + 8 * c;
  }
  const int br = min(n0 + 32 * wave + (lane >> 1), g.N - 1);
  const uint8_t *b_src = g.codes + (size_t)br * (size_t)g.row_stride + k_first / 2 +
                         16 * ((lane & 1) ^ ((lane >> 4) & 1));
  const float *s_src = g.gains + (size_t)br * g.gain_stride;
  const int s_first = k_first / 32;
  const int s_grp = lane & 1;
  auto stage = [&](int step) { return lds_m + (step % kMidStages) * kMidStage; };
  auto issue = [&](int step) {
    uint8_t *st = stage(step);
    const int k0 = step * kMidK;
#pragma unroll
    for (int i = 0; i < 2; ++i)
      __builtin_amdgcn_global_load_lds((global_void_t *)(a_src[i] + k0),
                                       (lds_void_t *)(st + (2 * wave + i) * 1024), 16, 0, 0);
    __builtin_amdgcn_global_load_lds((global_void_t *)(b_src + k0 / 2),
                                     (lds_void_t *)(st + kMidA * 2 + wave * 1024), 16, 0, 0);
    __builtin_amdgcn_global_load_lds(
        (global_void_t *)(s_src + (((unsigned)(s_first + k0 / 32 + s_grp)) >> g.group_shift)),
        (lds_void_t *)(st + kMidA * 2 + kMidB + wave * 256), 4, 0, 0);
  };

  float4_t acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const uint32_t exp10 = 0x64006400u;  // 1024.0 in both halves
  const _Float16 lo_bias = (_Float16)(1024.0f + g.code_bias);
  const _Float16 hi_bias = (_Float16)(1024.0f + 16.0f * g.code_bias);
  const half2_t bias_lo = half2_t{lo_bias, lo_bias};
  const half2_t bias_hi = half2_t{hi_bias, hi_bias};
  const int gq = lane >> 4;
  const int n = lane & 15;
  auto decode = [&](uint32_t d, half2_t scale) {
    const uint32_t e = d >> 8;
    const half2_t p0 = (as_half2(and_or_b32(d, 0x000F000Fu, exp10)) - bias_lo) * scale;
    const half2_t p1 = (as_half2(and_or_b32(d, 0x00F000F0u, exp10)) - bias_hi) * scale;
    const half2_t p2 = (as_half2(and_or_b32(e, 0x000F000Fu, exp10)) - bias_lo) * scale;
    const half2_t p3 = (as_half2(and_or_b32(e, 0x00F000F0u, exp10)) - bias_hi) * scale;
    return __builtin_bit_cast(half8_t, uint4_t{__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1),
                                               __builtin_bit_cast(uint32_t, p2), __builtin_bit_cast(uint32_t, p3)});
  };

  // A wave's loads retire in issue order, four a step: before iteration s
  // steps s .. min(s + kMidAhead, steps) - 1 are in flight, so step s is in
  // when all but the last 4 min(kMidAhead - 1, steps - s - 1) are.
  for (int t = 0; t < kMidAhead && t < steps; ++t) issue(t);
  for (int s = 0; s < steps; ++s) {
    switch (min(kMidAhead - 1, steps - s - 1)) {  // vmcnt(4 n) lgkmcnt(0)
      case 0: __builtin_amdgcn_s_waitcnt(0x0070); break;
      case 1: __builtin_amdgcn_s_waitcnt(0x0074); break;
      case 2: __builtin_amdgcn_s_waitcnt(0x0078); break;
      case 3: __builtin_amdgcn_s_waitcnt(0x007C); break;
      case 4: __builtin_amdgcn_s_waitcnt(0x4070); break;
      case 5: __builtin_amdgcn_s_waitcnt(0x4074); break;
      default: __builtin_amdgcn_s_waitcnt(0x4078); break;
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();  // every wave's DMA of step s is in; step s - 1's stage is free
    asm volatile("" ::: "memory");
    if (s + kMidAhead < steps) issue(s + kMidAhead);
    const uint8_t *st = stage(s);
    const _Float16 *as = reinterpret_cast<const _Float16 *>(st);
    const uint8_t *cs = st + kMidA * 2;
    const float *gs = reinterpret_cast<const float *>(cs + kMidB);
    half8_t bf[2][2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int row = 32 * wave + 16 * j + n;
      const int half = (gq >> 1) ^ ((n >> 3) & 1);
      const uint2_t raw = *reinterpret_cast<const uint2_t *>(cs + row * 32 + 16 * half + 8 * (gq & 1));
      const _Float16 sh = (_Float16)gs[row * 2 + (gq >> 1)];
      const half2_t sc = half2_t{sh, sh};
      bf[0][j] = decode(raw[0], sc);
      bf[1][j] = decode(raw[1], sc);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      half8_t a[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int r = 16 * i + n;
        const int p = (2 * gq + q) ^ ((r >> 1) & 7);
        a[q] = *reinterpret_cast<const half8_t *>(as + r * kMidK + 8 * p);
      }
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf[q][j], a[q], acc[i][j], 0, 0, 0);
    }
  }

  // D is C transposed (as in the large-tile form): lane l holds lane row
  // l % 16 of its tile and four consecutive weight rows 4 (l / 16) .. + 3.
  float *part = reinterpret_cast<float *>(g.out) + blockIdx.z * g.slice_floats;
  const bool vec_ok = g.slice_floats ? (g.N % 4 == 0)
                                     : (g.out_stride % 4 == 0 &&
                                        ((uintptr_t)g.out & (C_BF16 ? 7u : 15u)) == 0);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + 16 * i + n;
    if (m >= g.M) continue;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int nb = n0 + 32 * wave + 16 * j + 4 * gq;
      float4_t v = acc[i][j];
      if (!g.slice_floats && !C_BF16 && g.close.gains) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (nb + r < g.N) v[r] = close_value(g.close, nb + r, v[r]);
      }
      if (vec_ok && nb + 3 < g.N) {
        if (g.slice_floats) {
          *reinterpret_cast<float4_t *>(part + (size_t)m * g.N + nb) = v;
        } else if (C_BF16) {
          *reinterpret_cast<uint2_t *>(reinterpret_cast<uint16_t *>(g.out) + (size_t)m * g.out_stride + nb) =
              uint2_t{bf16_pair(v[0], v[1]), bf16_pair(v[2], v[3])};
        } else {
          *reinterpret_cast<float4_t *>(reinterpret_cast<float *>(g.out) + (size_t)m * g.out_stride + nb) = v;
        }
        continue;
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int nn = nb + r;
        if (nn >= g.N) continue;
        if (g.slice_floats)
          part[(size_t)m * g.N + nn] = v[r];
        else if (C_BF16)
          reinterpret_cast<uint16_t *>(g.out)[(size_t)m * g.out_stride + nn] = float_to_bf16(v[r]);
        else
          reinterpret_cast<float *>(g.out)[(size_t)m * g.out_stride + nn] = v[r];
      }
    }
  }
}

}  // namespace igl

using namespace igl;

// K slices of a large-tile launch: while the tiles fill fewer than 256
// workgroups (one a CU) and every slice keeps four 64-wide steps, K is cut in
// two again; N % 4 == 0 for the slice sum's four-column reads.
static int gemm_slices(int M, int N, int K) {
  const int tiles = ((M + kBigM - 1) / kBigM) * ((N + kBigN - 1) / kBigN);
  int slices = 1;
  while (slices < 8 && tiles * slices < 256 && N % 4 == 0 && K % (2 * slices * kBigK) == 0 &&
         K / (2 * slices) >= 4 * kBigK)
    slices *= 2;
  return slices;
}

static size_t gemm_half_bytes(int M, int K) {
  return ((size_t)M * (size_t)K * sizeof(_Float16) + 255) & ~(size_t)255;
}

// Bytes of workspace igl_launch_gemm_q4 needs for an M x N x K product (the
// binary16 activations of the large-tile form, then any K slices' fp32
// partials), 0 when it takes the small form.
// K slices of a skinny-form launch: while the tiles fill fewer than 128
// workgroups (the weight stream needs about half the CUs).
static int gemm_mid_slices(int M, int N, int K) {
  const int tiles = ((M + kMidM - 1) / kMidM) * ((N + kMidN - 1) / kMidN);
  int slices = 1;
  while (slices < 8 && tiles * slices < 128 && N % 4 == 0 && K % (2 * slices * kMidK) == 0 &&
         K / (2 * slices) >= 4 * kMidK)
    slices *= 2;
  return slices;
}

static int gemm_is_mid(int M, int N, int K) {
  return M >= 64 && M < kBigM && N >= kMidN && K % kMidK == 0;
}

extern "C" size_t igl_gemm_work_bytes(int M, int N, int K) {
  if (gemm_is_mid(M, N, K)) {
    const int slices = gemm_mid_slices(M, N, K);
    return gemm_half_bytes(M, K) + (slices > 1 ? (size_t)slices * M * N * sizeof(float) : 0);
  }
  if (M < kBigM || N < kBigN || K % kBigK) return 0;
  const int slices = gemm_slices(M, N, K);
  return gemm_half_bytes(M, K) + (slices > 1 ? (size_t)slices * M * N * sizeof(float) : 0);
}

extern "C" hipError_t igl_launch_gemm_q4(const void *act, int act_bf16, int act_stride,
                                         const uint8_t *codes, long long row_stride,
                                         const float *gains, int gain_stride, int group_shift,
                                         int code_bias, void *out, int out_bf16, int out_stride,
                                         int M, int N, int K, void *work,
                                         const igl_gemm_close *close, hipStream_t stream) {
  const igl_gemm_close no_close = {nullptr, 0.0f, 0.0f};
  const igl_gemm_close cl = close ? *close : no_close;
  if (cl.gains && (out_bf16 || act_bf16 || !igl_gemm_work_bytes(M, N, K) || !work))
    return hipErrorInvalidValue;  // the close rides only on the large-tile form's fp32 C
  if (igl_gemm_work_bytes(M, N, K) && work) {
    _Float16 *a16 = reinterpret_cast<_Float16 *>(work);
    const bool mid = gemm_is_mid(M, N, K);
    const int slices = mid ? gemm_mid_slices(M, N, K) : gemm_slices(M, N, K);
    float *part = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(work) + gemm_half_bytes(M, K));
    dim3 cgrid((K / 8 + 255) / 256, (M + kHalfRows - 1) / kHalfRows);
    if (act_bf16)
      hipLaunchKernelGGL((act_half_kernel<true>), cgrid, dim3(256), 0, stream, act, act_stride, M, K, a16, 0.0f);
    else
      hipLaunchKernelGGL((act_half_kernel<false>), cgrid, dim3(256), 0, stream, act, act_stride, M, K, a16,
                         cl.gains ? cl.step : 0.0f);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    GemmBigArgs b;
    b.a16 = a16;
    b.codes = codes;
    b.row_stride = row_stride;
    b.gains = gains;
    b.gain_stride = gain_stride;
    b.group_shift = group_shift;
    b.code_bias = (float)code_bias;
    b.out = slices > 1 ? static_cast<void *>(part) : out;
    b.out_stride = out_stride;
    b.M = M;
    b.N = N;
    b.K = K;
    b.k_steps = K / kBigK / slices;
    b.slice_floats = slices > 1 ? (size_t)M * N : 0;
    b.close = cl;
    // The dynamic LDS each form asks for is granted once per kernel.
    static int granted[4];
    const int use_bf16 = out_bf16 && (!mid || slices == 1);
    const void *fn = mid ? (use_bf16 ? reinterpret_cast<const void *>(&gemm_q4_mid_kernel<true>)
                                     : reinterpret_cast<const void *>(&gemm_q4_mid_kernel<false>))
                         : (use_bf16 ? reinterpret_cast<const void *>(&gemm_q4_big_kernel<true>)
                                     : reinterpret_cast<const void *>(&gemm_q4_big_kernel<false>));
    const int lds = mid ? kMidLds : kBigLds;
    const int which = 2 * mid + use_bf16;
    if (!granted[which]) {
      e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
      if (e != hipSuccess) return e;
      granted[which] = 1;
    }
    if (mid) {
      const dim3 grid((N + kMidN - 1) / kMidN, (M + kMidM - 1) / kMidM, slices);
      if (use_bf16)
        hipLaunchKernelGGL((gemm_q4_mid_kernel<true>), grid, dim3(256), (size_t)lds, stream, b);
      else
        hipLaunchKernelGGL((gemm_q4_mid_kernel<false>), grid, dim3(256), (size_t)lds, stream, b);
    } else {
      const dim3 grid((N + kBigN - 1) / kBigN, (M + kBigM - 1) / kBigM, slices);
      if (use_bf16)
        hipLaunchKernelGGL((gemm_q4_big_kernel<true>), grid, dim3(512), (size_t)lds, stream, b);
      else
        hipLaunchKernelGGL((gemm_q4_big_kernel<false>), grid, dim3(512), (size_t)lds, stream, b);
    }
    e = hipGetLastError();
    if (e != hipSuccess || slices == 1) return e;
    dim3 sgrid((N / 4 + 255) / 256, M);
    if (out_bf16)
      hipLaunchKernelGGL((gemm_slice_sum_kernel<true>), sgrid, dim3(256), 0, stream, part, slices,
                         b.slice_floats, M, N, out, out_stride, cl);
    else
      hipLaunchKernelGGL((gemm_slice_sum_kernel<false>), sgrid, dim3(256), 0, stream, part, slices,
                         b.slice_floats, M, N, out, out_stride, cl);
    return hipGetLastError();
  }
  GemmArgs g;
  g.act = act;
  g.act_stride = act_stride;
  g.codes = codes;
  g.row_stride = row_stride;
  g.gains = gains;
  g.gain_stride = gain_stride;
  g.group_shift = group_shift;
  g.code_bias = (float)code_bias;
  g.out = out;
  g.out_stride = out_stride;
  g.M = M;
  g.N = N;
  g.K = K;
  dim3 grid((N + kGemmBN - 1) / kGemmBN, (M + kGemmBM - 1) / kGemmBM);
  if (act_bf16 && out_bf16)
    hipLaunchKernelGGL((gemm_q4_kernel<true, true>), grid, dim3(kGemmThreads), 0, stream, g);
  else if (act_bf16)
    hipLaunchKernelGGL((gemm_q4_kernel<true, false>), grid, dim3(kGemmThreads), 0, stream, g);
  else if (out_bf16)
    hipLaunchKernelGGL((gemm_q4_kernel<false, true>), grid, dim3(kGemmThreads), 0, stream, g);
  else
    hipLaunchKernelGGL((gemm_q4_kernel<false, false>), grid, dim3(kGemmThreads), 0, stream, g);
  return hipGetLastError();
}
