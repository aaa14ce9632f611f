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
  int group_shift;        // log2(group_size / 32)
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

// Round-to-nearest-even fp32 -> bf16 (NaN kept quiet).
__device__ __forceinline__ uint16_t float_to_bf16(float v) {
  uint32_t bits = __builtin_bit_cast(uint32_t, v);
  if ((bits & 0x7F800000u) == 0x7F800000u && (bits & 0x7FFFFFu)) return (uint16_t)((bits >> 16) | 0x40u);
  bits += 0x7FFFu + ((bits >> 16) & 1u);
  return (uint16_t)(bits >> 16);
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

}  // namespace igl

using namespace igl;

extern "C" hipError_t igl_launch_gemm_q4(const void *act, int act_bf16, int act_stride,
                                         const uint8_t *codes, long long row_stride,
                                         const float *gains, int gain_stride, int group_size,
                                         int code_bias, void *out, int out_bf16, int out_stride,
                                         int M, int N, int K, hipStream_t stream) {
  GemmArgs g;
  g.act = act;
  g.act_stride = act_stride;
  g.codes = codes;
  g.row_stride = row_stride;
  g.gains = gains;
  g.gain_stride = gain_stride;
  g.group_shift = __builtin_ctz((unsigned)(group_size / 32));
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
