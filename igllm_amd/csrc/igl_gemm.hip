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

// ---- the large-tile form ---------------------------------------------------
//
// For M and N of 256 and up.  The activations are first converted once to a
// binary16 copy (act_half_kernel), so the tile loop moves them into LDS
// unchanged instead of converting every element once per column tile.  Each
// workgroup owns a 256 x 256 tile of C; its four waves (2 x 2) each hold a
// 128 x 128 block as 8 x 8 v_mfma_f32_16x16x32_f16 accumulators, four times
// the products per byte of LDS read of a 64 x 64 block.  K advances one 32-code
// group a step through two LDS buffers: the next step's global loads are in
// flight while the current step's 64 products a wave run, then it is
// dequantized into the other buffer, one barrier a step.  The dequantized
// weight is (c - code_bias) * gain in packed binary16: exact code times the
// gain rounded to binary16, rounded once more (both within 2^-11).
constexpr int kBigM = 256;
constexpr int kBigN = 256;
constexpr int kBigK = 64;
constexpr int kBigPitch = kBigK + 8;          // halves per LDS row
constexpr int kBigTile = kBigM * kBigPitch;   // halves per LDS tile (A or B)

// a16[m][k] = binary16(a[m][k]), saturating at +-65504.
template <bool A_BF16>
__global__ void act_half_kernel(const void *act, int act_stride, int M, int K, _Float16 *a16) {
  const int k8 = (blockIdx.x * blockDim.x + threadIdx.x) * 8;
  const int m = blockIdx.y;
  if (k8 >= K || m >= M) return;
  half8_t h;
  if (A_BF16) {
    // rows are 16-byte aligned (act_stride % 8 == 0): one load for 8 values
    const uint4_t raw = *reinterpret_cast<const uint4_t *>(
        reinterpret_cast<const uint16_t *>(act) + (size_t)m * act_stride + k8);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      h[2 * i] = sat_half(__builtin_bit_cast(float, raw[i] << 16));
      h[2 * i + 1] = sat_half(__builtin_bit_cast(float, raw[i] & 0xFFFF0000u));
    }
  } else {
    const float4_t *src = reinterpret_cast<const float4_t *>(
        reinterpret_cast<const float *>(act) + (size_t)m * act_stride + k8);
    const float4_t lo = src[0], hi = src[1];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      h[i] = sat_half(lo[i]);
      h[4 + i] = sat_half(hi[i]);
    }
  }
  *reinterpret_cast<half8_t *>(a16 + (size_t)m * K + k8) = h;
}

struct GemmBigArgs {
  const _Float16 *a16;    // [M][K]
  const uint8_t *codes;
  long long row_stride;
  const float *gains;
  int gain_stride;
  int group_shift;
  float code_bias;
  void *out;
  int out_stride;
  int M, N, K;
};

template <bool C_BF16>
__global__ __launch_bounds__(512) void gemm_q4_big_kernel(GemmBigArgs g) {
  extern __shared__ __attribute__((aligned(16))) _Float16 lds_h[];  // A[2], B[2]
  constexpr int G = kBigK / 32;  // groups a step
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 2;      // 2 wave rows of 128
  const int wn = wave & 3;       // 4 wave columns of 64
  const int m0 = blockIdx.y * kBigM;
  const int n0 = blockIdx.x * kBigN;

  // Thread t stages half (t & 1) of row t / 2 of the A tile (32 halves) and
  // group (t & 1) of row t / 2 of the weight tile (16 bytes and its gain).
  const int row = tid >> 1;
  const int part = tid & 1;
  const int am = min(m0 + row, g.M - 1);
  const int bn = min(n0 + row, g.N - 1);
  const bool a_live = m0 + row < g.M;
  const bool b_live = n0 + row < g.N;
  const uint4_t *a_src = reinterpret_cast<const uint4_t *>(g.a16 + (size_t)am * g.K + 32 * part);
  const uint4_t *b_src =
      reinterpret_cast<const uint4_t *>(g.codes + (size_t)bn * (size_t)g.row_stride) + part;
  const float *gain_row = g.gains + (size_t)bn * g.gain_stride;
  uint4_t ra[4], rb;
  float rs;
  auto fetch = [&](int k) {
#pragma unroll
    for (int i = 0; i < 4; ++i) ra[i] = a_src[(k >> 3) + i];
    rb = __builtin_nontemporal_load(b_src + (k >> 5));
    rs = gain_row[(unsigned)((k >> 5) + part) >> g.group_shift];
  };
  const uint32_t exp16 = 0x4C004C00u;
  const _Float16 lift = (_Float16)(16.0f + g.code_bias);
  auto stage = [&](int buf) {
    _Float16 *as = lds_h + buf * kBigTile + row * kBigPitch + 32 * part;
    _Float16 *bs = lds_h + (2 + buf) * kBigTile + row * kBigPitch + 32 * part;
    const uint4_t zero = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4_t *>(as + 8 * i) = a_live ? ra[i] : zero;
    const half2_t shift = half2_t{lift, lift};
    const _Float16 sh = (_Float16)rs;
    const half2_t scale = b_live ? half2_t{sh, sh} : half2_t{(_Float16)0.0f, (_Float16)0.0f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // codes 8j .. 8j+7, pairs (i, i + 4) in the halves of nibble_pair16<i>
      const uint32_t d = rb[j];
      const half2_t p0 = (nibble_pair16<0>(d, exp16) - shift) * scale;
      const half2_t p1 = (nibble_pair16<1>(d, exp16) - shift) * scale;
      const half2_t p2 = (nibble_pair16<2>(d, exp16) - shift) * scale;
      const half2_t p3 = (nibble_pair16<3>(d, exp16) - shift) * scale;
      const half8_t h = {p0.x, p1.x, p2.x, p3.x, p0.y, p1.y, p2.y, p3.y};
      *reinterpret_cast<half8_t *>(bs + 8 * j) = h;
    }
  };

  float4_t acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};

  fetch(0);
  stage(0);
  __syncthreads();
  const int steps = g.K / kBigK;
  const int koff = 8 * (lane >> 4);
  for (int s = 0; s < steps; ++s) {
    const int cur = s & 1;
    if (s + 1 < steps) fetch((s + 1) * kBigK);
#pragma unroll
    for (int q = 0; q < G; ++q) {
      const _Float16 *as = lds_h + cur * kBigTile + (wm * 128 + (lane & 15)) * kBigPitch + 32 * q + koff;
      const _Float16 *bs = lds_h + (2 + cur) * kBigTile + (wn * 64 + (lane & 15)) * kBigPitch + 32 * q + koff;
      half8_t af[8], bf[4];
#pragma unroll
      for (int i = 0; i < 8; ++i) af[i] = *reinterpret_cast<const half8_t *>(as + i * 16 * kBigPitch);
#pragma unroll
      for (int j = 0; j < 4; ++j) bf[j] = *reinterpret_cast<const half8_t *>(bs + j * 16 * kBigPitch);
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (s + 1 < steps) stage(cur ^ 1);
    __syncthreads();
  }

  // D layout of a 16x16 tile: lane l holds rows 4*(l/16) + r, column l % 16.
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + wn * 64 + j * 16 + (lane & 15);
      if (n >= g.N) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * 128 + i * 16 + 4 * (lane >> 4) + r;
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

// Bytes of workspace igl_launch_gemm_q4 needs for an M x K product (the
// binary16 activations of the large-tile form), 0 when it takes the small one.
extern "C" size_t igl_gemm_work_bytes(int M, int N, int K) {
  if (M < kBigM || N < kBigN || K % kBigK) return 0;
  return (size_t)M * (size_t)K * sizeof(_Float16);
}

extern "C" hipError_t igl_launch_gemm_q4(const void *act, int act_bf16, int act_stride,
                                         const uint8_t *codes, long long row_stride,
                                         const float *gains, int gain_stride, int group_size,
                                         int code_bias, void *out, int out_bf16, int out_stride,
                                         int M, int N, int K, void *work, hipStream_t stream) {
  if (igl_gemm_work_bytes(M, N, K) && work) {
    _Float16 *a16 = reinterpret_cast<_Float16 *>(work);
    dim3 cgrid((K / 8 + 255) / 256, M);
    if (act_bf16)
      hipLaunchKernelGGL((act_half_kernel<true>), cgrid, dim3(256), 0, stream, act, act_stride, M, K, a16);
    else
      hipLaunchKernelGGL((act_half_kernel<false>), cgrid, dim3(256), 0, stream, act, act_stride, M, K, a16);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    GemmBigArgs b;
    b.a16 = a16;
    b.codes = codes;
    b.row_stride = row_stride;
    b.gains = gains;
    b.gain_stride = gain_stride;
    b.group_shift = __builtin_ctz((unsigned)(group_size / 32));
    b.code_bias = (float)code_bias;
    b.out = out;
    b.out_stride = out_stride;
    b.M = M;
    b.N = N;
    b.K = K;
    const size_t lds = 4 * (size_t)kBigTile * sizeof(_Float16);
    static int granted[2];
    const void *fn = out_bf16 ? reinterpret_cast<const void *>(&gemm_q4_big_kernel<true>)
                              : reinterpret_cast<const void *>(&gemm_q4_big_kernel<false>);
    if (!granted[out_bf16 ? 1 : 0]) {
      e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) return e;
      granted[out_bf16 ? 1 : 0] = 1;
    }
    dim3 grid((N + kBigN - 1) / kBigN, (M + kBigM - 1) / kBigM);
    if (out_bf16)
      hipLaunchKernelGGL((gemm_q4_big_kernel<true>), grid, dim3(512), lds, stream, b);
    else
      hipLaunchKernelGGL((gemm_q4_big_kernel<false>), grid, dim3(512), lds, stream, b);
    return hipGetLastError();
  }
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
