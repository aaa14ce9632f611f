// igl_gemv.hip - packed int4 projection for decode and small-lane verify
// (M = 1..8 lanes), gfx950.
//
// Computes, for every row n of a code plane and every lane m,
//     y[m][n] = sum_g gain[n][g] * (sum_{k in g} x[m][k] * c[n][k] - code_bias * X[m][g])
// which is the reference's float path (kern_row_code, app_core.c:3688-3706,
// and kern_row_code_many, 4075-4117) with X the per-group activation sum
// (kern_group_sum, 4288-4300).  Codes are 4-bit, two a byte, low nibble first,
// stored as value + 8 (plane_bind_gemma, app_core.c:7932), read straight out
// of the checkpoint's own row layout: nothing is repacked.
//
// Layout of the work:
//   * A "unit" is 32 consecutive codes of one row: 16 bytes, one 128-bit load.
//     Lane l of a wave takes units l, l+64, ... of each row it owns, so a
//     wave's load of one row is 1 KiB of contiguous bytes.
//   * Each wave owns R rows at once (R independent 128-bit loads in flight per
//     lane) and, where a row is long and rows are few, a share of the units of
//     those rows (`ksplit` waves of the workgroup split one row tile).
//   * The activations are staged once per workgroup into LDS, laid out so
//     that the 64 lanes of a read touch 64 consecutive 16-byte slots (no bank
//     conflicts), together with (16 + code_bias) * X per unit.
//   * A code is never converted to float on its own: two nibbles become two
//     exact binary16 values (16 + c) with one shift and one and-or, and
//     v_fma_mix_f32 multiplies each half into an fp32 accumulator.  The 16 is
//     removed with the staged per-unit term, so a unit's contribution is
//     gain * (sum (16 + c) x - (16 + code_bias) X).
//   * Row sums close with six DPP adds across the wave.
#include "igl_device.h"

namespace igl {

struct GemvArgs {
  const uint8_t *codes;
  long long row_stride;   // bytes between rows of codes
  const float *gains;     // [N][gain_stride]
  int gain_stride;        // groups per row
  int group_shift;        // log2(group_size / 32)
  const float *act;       // lanes of K floats, act_stride apart
  int act_stride;
  float *out;             // lanes of N floats, out_stride apart (grid K-split: partials)
  int out_stride;
  int N;
  int K;                  // columns of the whole plane
  int chunk_cols;         // columns per grid K-chunk (blockIdx.y)
  int ksplit;             // waves of a workgroup sharing one row tile: 1, 2 or 4
  float unit_bias;        // 16 + code_bias
  int act_vec;            // activations 16-byte aligned with act_stride % 4 == 0
};

constexpr int kGemvThreads = 256;

template <int M, int R>
__global__ __launch_bounds__(kGemvThreads) void gemv_q4_kernel(GemvArgs a) {
  extern __shared__ float4_t lds_f4[];
  const int chunk = blockIdx.y;
  const int col0 = chunk * a.chunk_cols;
  const int cols = min(a.chunk_cols, a.K - col0);
  const int units = cols >> 5;
  float4_t *xs = lds_f4;                                   // [M][8][units]
  float *cs = reinterpret_cast<float *>(xs + M * 8 * units);  // [M][units]
  float *red = cs + M * units;                             // [4][R][M]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int tiles_per_block = 4 / a.ksplit;
  const int tile = blockIdx.x * tiles_per_block + wave / a.ksplit;
  const int ks = wave % a.ksplit;
  const int row0 = tile * R;

  // Stage the chunk's activations: thread t moves float4 slot i = t + 256 j,
  // which is columns 4i .. 4i+3, unit i / 8, quarter i % 8.
  for (int i = tid; i < M * units * 8; i += kGemvThreads) {
    const int m = i / (units * 8);
    const int slot = i - m * units * 8;
    const float *src = a.act + (size_t)m * a.act_stride + col0 + slot * 4;
    float4_t v;
    if (a.act_vec) {
      v = *reinterpret_cast<const float4_t *>(src);
    } else {
      v.x = src[0]; v.y = src[1]; v.z = src[2]; v.w = src[3];
    }
    xs[(m * 8 + (slot & 7)) * units + (slot >> 3)] = v;
  }
  __syncthreads();
  // Per-unit activation sums, in column order, times (16 + code_bias).
  for (int i = tid; i < M * units; i += kGemvThreads) {
    const int m = i / units;
    const int u = i - m * units;
    float total = 0.0f;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      float4_t v = xs[(m * 8 + q) * units + u];
      total += v.x; total += v.y; total += v.z; total += v.w;
    }
    cs[i] = a.unit_bias * total;
  }
  __syncthreads();

  float acc[R][M];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;

  const int u_begin = (units * ks) / a.ksplit;
  const int u_end = (units * (ks + 1)) / a.ksplit;
  const uint8_t *row_base[R];
  const float *gain_base[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = min(row0 + r, a.N - 1);  // tail rows are computed, never stored
    row_base[r] = a.codes + (size_t)row * (size_t)a.row_stride + (size_t)(col0 >> 1);
    gain_base[r] = a.gains + (size_t)row * (size_t)a.gain_stride;
  }
  const int unit0 = col0 >> 5;

  const uint32_t exp16 = 0x4C004C00u;  // binary16 16.0 in both halves
  if (row0 < a.N) {
    for (int u = u_begin + lane; u < u_end; u += kWave) {
      uint4_t w[R];
      float s[R];
#pragma unroll
      for (int r = 0; r < R; ++r)
        w[r] = __builtin_nontemporal_load(reinterpret_cast<const uint4_t *>(row_base[r]) + u);
#pragma unroll
      for (int r = 0; r < R; ++r) s[r] = gain_base[r][(unsigned)(unit0 + u) >> a.group_shift];

      float part[R][M];
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) part[r][m] = 0.0f;

#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float4_t xa[M], xb[M];
#pragma unroll
        for (int m = 0; m < M; ++m) {
          xa[m] = xs[(m * 8 + 2 * j) * units + u];
          xb[m] = xs[(m * 8 + 2 * j + 1) * units + u];
        }
        half2_t p[R][4];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const uint32_t d = w[r][j];
          p[r][0] = nibble_pair16<0>(d, exp16);
          p[r][1] = nibble_pair16<1>(d, exp16);
          p[r][2] = nibble_pair16<2>(d, exp16);
          p[r][3] = nibble_pair16<3>(d, exp16);
        }
        // Codes 8j+i (low halves) against xa, 8j+4+i (high halves) against
        // xb; rows and lanes interleaved so R*M accumulator chains overlap.
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < M; ++m)
              part[r][m] = __builtin_fmaf((float)p[r][i].x, xa[m][i], part[r][m]);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < M; ++m)
              part[r][m] = __builtin_fmaf((float)p[r][i].y, xb[m][i], part[r][m]);
      }
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float c = cs[m * units + u];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r][m] = __builtin_fmaf(s[r], part[r][m] - c, acc[r][m]);
      }
    }
  }

#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = wave_sum_to_last(acc[r][m]);

  float *dst = a.out + (size_t)chunk * (size_t)M * (size_t)a.out_stride;
  if (a.ksplit == 1) {
    if (lane == 63) {
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (row0 + r < a.N)
#pragma unroll
          for (int m = 0; m < M; ++m) dst[(size_t)m * a.out_stride + row0 + r] = acc[r][m];
    }
    return;
  }
  if (lane == 63) {
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) red[(wave * R + r) * M + m] = acc[r][m];
  }
  __syncthreads();
  if (ks == 0 && lane < R * M) {
    const int r = lane / M;
    const int m = lane - r * M;
    float total = 0.0f;
    for (int k = 0; k < a.ksplit; ++k) total += red[((wave + k) * R + r) * M + m];
    if (row0 + r < a.N) dst[(size_t)m * a.out_stride + row0 + r] = total;
  }
}

// Sums the grid K-chunk partials in chunk order: out[m][n] = sum_c part[c][m][n].
__global__ void gemv_chunk_sum_kernel(const float *part, int chunks, int M, int N, float *out,
                                      int out_stride) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M * N) return;
  const int m = i / N;
  const int n = i - m * N;
  float total = 0.0f;
  for (int c = 0; c < chunks; ++c) total += part[((size_t)c * M + m) * N + n];
  out[(size_t)m * out_stride + n] = total;
}

// The one- and two-lane form, for planes whose units fit one per lane of the
// waves sharing a row tile (K <= 8192).  A lane's 32 activations per lane of
// the batch live in VGPRs for the rows the wave owns, so there is no LDS
// staging and no barrier before the arithmetic: the row loads, the gains and
// the activations are all requested first and the launch pays one memory
// round trip.  The arithmetic is gemv_q4_kernel's, term for term.
template <int M, int R>
__global__ __launch_bounds__(kGemvThreads) void gemv_q4_reg_kernel(GemvArgs a) {
  __shared__ float red[4][R][M];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int tiles_per_block = 4 / a.ksplit;
  const int tile = blockIdx.x * tiles_per_block + wave / a.ksplit;
  const int ks = wave % a.ksplit;
  const int row0 = tile * R;
  const int units = a.K >> 5;
  const int u = (units * ks) / a.ksplit + lane;
  const bool has = row0 < a.N && u < (units * (ks + 1)) / a.ksplit;

  uint4_t w[R];
  float s[R];
  float4_t x[M][8];
  if (has) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = min(row0 + r, a.N - 1);  // tail rows are computed, never stored
      w[r] = __builtin_nontemporal_load(
          reinterpret_cast<const uint4_t *>(a.codes + (size_t)row * (size_t)a.row_stride) + u);
      s[r] = a.gains[(size_t)row * (size_t)a.gain_stride + ((unsigned)u >> a.group_shift)];
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float *src = a.act + (size_t)m * a.act_stride + u * 32;
      if (a.act_vec) {
#pragma unroll
        for (int q = 0; q < 8; ++q) x[m][q] = *reinterpret_cast<const float4_t *>(src + 4 * q);
      } else {
#pragma unroll
        for (int q = 0; q < 8; ++q)
          x[m][q] = float4_t{src[4 * q], src[4 * q + 1], src[4 * q + 2], src[4 * q + 3]};
      }
    }
  }

  float acc[R][M];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;
  if (has) {
    const uint32_t exp16 = 0x4C004C00u;
    float part[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) part[r][m] = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      half2_t p[R][4];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint32_t d = w[r][j];
        p[r][0] = nibble_pair16<0>(d, exp16);
        p[r][1] = nibble_pair16<1>(d, exp16);
        p[r][2] = nibble_pair16<2>(d, exp16);
        p[r][3] = nibble_pair16<3>(d, exp16);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int m = 0; m < M; ++m)
            part[r][m] = __builtin_fmaf((float)p[r][i].x, x[m][2 * j][i], part[r][m]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int m = 0; m < M; ++m)
            part[r][m] = __builtin_fmaf((float)p[r][i].y, x[m][2 * j + 1][i], part[r][m]);
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float total = 0.0f;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        total += x[m][q].x; total += x[m][q].y; total += x[m][q].z; total += x[m][q].w;
      }
      const float c = a.unit_bias * total;
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r][m] = s[r] * (part[r][m] - c);
    }
  }

#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = wave_sum_to_last(acc[r][m]);

  if (a.ksplit == 1) {
    if (lane == 63) {
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (row0 + r < a.N)
#pragma unroll
          for (int m = 0; m < M; ++m) a.out[(size_t)m * a.out_stride + row0 + r] = acc[r][m];
    }
    return;
  }
  if (lane == 63) {
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) red[wave][r][m] = acc[r][m];
  }
  __syncthreads();
  if (ks == 0 && lane < R * M) {
    const int r = lane / M;
    const int m = lane - r * M;
    float total = 0.0f;
    for (int k = 0; k < a.ksplit; ++k) total += red[wave + k][r][m];
    if (row0 + r < a.N) a.out[(size_t)m * a.out_stride + row0 + r] = total;
  }
}

template <int M, int R>
static hipError_t gemv_reg_launch(const GemvArgs &a, hipStream_t stream) {
  const int tiles = (a.N + R - 1) / R;
  const int tiles_per_block = 4 / a.ksplit;
  dim3 grid((tiles + tiles_per_block - 1) / tiles_per_block);
  hipLaunchKernelGGL((gemv_q4_reg_kernel<M, R>), grid, dim3(kGemvThreads), 0, stream, a);
  return hipGetLastError();
}

template <int M, int R>
static size_t gemv_lds_bytes(int units) {
  return (size_t)M * units * (8 * sizeof(float4_t) + sizeof(float)) + sizeof(float) * 4 * R * M;
}

template <int M, int R>
static hipError_t gemv_launch(const GemvArgs &a, int chunks, hipStream_t stream) {
  const size_t lds = gemv_lds_bytes<M, R>(a.chunk_cols >> 5);
  static size_t lds_granted = 65536;  // launches above 64 KiB ask once
  if (lds > lds_granted) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemv_q4_kernel<M, R>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    lds_granted = lds;
  }
  const int tiles = (a.N + R - 1) / R;
  const int tiles_per_block = 4 / a.ksplit;
  dim3 grid((tiles + tiles_per_block - 1) / tiles_per_block, chunks);
  hipLaunchKernelGGL((gemv_q4_kernel<M, R>), grid, dim3(kGemvThreads), lds, stream, a);
  return hipGetLastError();
}

}  // namespace igl

using namespace igl;

extern "C" int igl_gemv_rows_per_tile(int lanes) { return lanes <= 4 ? 4 : 2; }

// Columns one grid K-chunk covers for `lanes` lanes of a K-column plane when a
// workgroup may hold `lds_limit` bytes of LDS: the staged activations take 132
// bytes per (lane, 32-column unit), the wave reductions 16 R M.
extern "C" int igl_gemv_chunk_cols(int lanes, int K, int lds_limit) {
  const int R = igl_gemv_rows_per_tile(lanes);
  const int units = K / 32;
  int max_units = (lds_limit - 16 * R * lanes) / (132 * lanes);
  if (max_units < 1) max_units = 1;
  const int chunks = (units + max_units - 1) / max_units;
  const int per = (units + chunks - 1) / chunks;
  return per * 32;
}

// Launches y = W x for 1..8 lanes.  `part` must hold chunks * lanes * N floats
// when the plane needs more than one K-chunk, and may be NULL otherwise;
// `lds_limit` is the device's LDS bytes per workgroup.
extern "C" hipError_t igl_launch_gemv_q4(const uint8_t *codes, long long row_stride,
                                         const float *gains, int gain_stride, int group_size,
                                         int code_bias, const float *act, int act_stride,
                                         int lanes, float *out, int out_stride, int N, int K,
                                         float *part, int lds_limit, hipStream_t stream) {
  GemvArgs a;
  a.codes = codes;
  a.row_stride = row_stride;
  a.gains = gains;
  a.gain_stride = gain_stride;
  a.group_shift = __builtin_ctz((unsigned)(group_size / 32));
  a.act = act;
  a.act_stride = act_stride;
  a.N = N;
  a.K = K;
  a.unit_bias = 16.0f + (float)code_bias;
  a.act_vec = ((((uintptr_t)act) & 15u) == 0 && (act_stride & 3) == 0) ? 1 : 0;
  // One and two lanes with at most 256 units a row: the register form, with
  // enough waves on a row tile that each lane holds one unit.
  if (lanes <= 2 && K / 32 <= 4 * kWave) {
    const int units = K / 32;
    const int R = 4;
    const int tiles = (N + R - 1) / R;
    int ksplit = 1;
    while (ksplit < 4 && (units > ksplit * kWave || (tiles * ksplit < 2048 && units / (ksplit * 2) >= 32)))
      ksplit *= 2;
    a.ksplit = ksplit;
    a.chunk_cols = K;
    a.out = out;
    a.out_stride = out_stride;
    return lanes == 1 ? gemv_reg_launch<1, 4>(a, stream) : gemv_reg_launch<2, 4>(a, stream);
  }
  a.chunk_cols = igl_gemv_chunk_cols(lanes, K, lds_limit);
  const int chunks = (K + a.chunk_cols - 1) / a.chunk_cols;
  const int R = igl_gemv_rows_per_tile(lanes);
  // Waves of a workgroup that split one row tile: enough waves to fill the
  // chip when rows are few, as long as every wave keeps a full 64 units.
  const int units = a.chunk_cols / 32;
  const int tiles = (N + R - 1) / R;
  int ksplit = 1;
  while (ksplit < 4 && tiles * ksplit * chunks < 2048 && units / (ksplit * 2) >= 64) ksplit *= 2;
  a.ksplit = ksplit;
  if (chunks > 1) {
    if (!part) return hipErrorInvalidValue;
    a.out = part;
    a.out_stride = N;
  } else {
    a.out = out;
    a.out_stride = out_stride;
  }
  hipError_t e;
  switch (lanes) {
    case 1: e = gemv_launch<1, 4>(a, chunks, stream); break;
    case 2: e = gemv_launch<2, 4>(a, chunks, stream); break;
    case 3: e = gemv_launch<3, 4>(a, chunks, stream); break;
    case 4: e = gemv_launch<4, 4>(a, chunks, stream); break;
    case 5: e = gemv_launch<5, 2>(a, chunks, stream); break;
    case 6: e = gemv_launch<6, 2>(a, chunks, stream); break;
    case 7: e = gemv_launch<7, 2>(a, chunks, stream); break;
    case 8: e = gemv_launch<8, 2>(a, chunks, stream); break;
    default: return hipErrorInvalidValue;
  }
  if (e != hipSuccess || chunks == 1) return e;
  const int total = lanes * N;
  hipLaunchKernelGGL(gemv_chunk_sum_kernel, dim3((total + 255) / 256), dim3(256), 0, stream, part,
                     chunks, lanes, N, out, out_stride);
  return hipGetLastError();
}
