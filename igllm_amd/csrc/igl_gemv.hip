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
#include "igl_launch.h"

namespace igl {

struct GemvArgs {
  const uint8_t *codes;
  long long row_stride;   // bytes between rows of codes
  const float *gains;     // [N][gain_stride]
  int gain_stride;        // groups per row
  int group_shift;        // gain of unit u: u >> group_shift (31: one gain a row)
  const float *act;       // lanes of K floats, act_stride apart
  int act_stride;
  float *out;             // lanes of N floats, out_stride apart (grid K-split: partials)
  int out_stride;
  int N;
  int K;                  // columns of the whole plane
  int chunk_cols;         // columns per grid K-chunk (blockIdx.y)
  int ksplit;             // waves of a workgroup sharing one row tile: 1, 2 or 4
  int ks_log;             // log2(ksplit)
  float unit_bias;        // 16 + code_bias
  int act_vec;            // activations 16-byte aligned with act_stride % 4 == 0
  int lane_rows;          // > 1 (one-lane dot form): grid row blockIdx.y is lane blockIdx.y
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
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (k < a.ksplit) total += red[((wave + k) * R + r) * M + m];
    if (row0 + r < a.N) dst[(size_t)m * a.out_stride + row0 + r] = total;
  }
}

// Sums the grid K-chunk partials in chunk order: out[m][n] = sum_c part[c][m][n].
// Eight chunks' loads go out together, then their adds in order (chunks past
// the count are skipped, not added as zeros): one memory round trip per eight
// chunks instead of one per chunk.
__global__ void gemv_chunk_sum_kernel(const float *part, int chunks, int M, int N, float *out,
                                      int out_stride) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M * N) return;
  const int m = i / N;
  const int n = i - m * N;
  const size_t step = (size_t)M * (size_t)N;  // part[c][m][n] = part[c * step + i]
  float total = 0.0f;
  for (int c0 = 0; c0 < chunks; c0 += 8) {
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = c0 + j < chunks ? part[(size_t)(c0 + j) * step + i] : 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (c0 + j < chunks) total += v[j];
  }
  out[(size_t)m * out_stride + n] = total;
}

// The one- and two-lane form, for planes whose units fit one per lane of the
// waves sharing a row tile (K <= 8192).  A lane's 32 activations per lane of
// the batch live in VGPRs for the rows the wave owns, so there is no LDS
// staging and no barrier before the arithmetic: the row loads, the gains and
// the activations are all requested first and the launch pays one memory
// round trip.  The arithmetic is gemv_q4_kernel's, term for term.
template <int M, int R, int UPL>
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
  const int u_end = (units * (ks + 1)) / a.ksplit;
  // A lane's units: u_first + 64 j for j < UPL, those before u_end.
  const int u_first = (units * ks) / a.ksplit + lane;

  uint4_t w[UPL][R];
  float s[UPL][R];
  float4_t x[UPL][M][8];
#pragma unroll
  for (int j = 0; j < UPL; ++j) {
    const int u = u_first + kWave * j;
    if (row0 < a.N && u < u_end) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int row = min(row0 + r, a.N - 1);  // tail rows are computed, never stored
        w[j][r] = __builtin_nontemporal_load(
            reinterpret_cast<const uint4_t *>(a.codes + (size_t)row * (size_t)a.row_stride) + u);
        s[j][r] = a.gains[(size_t)row * (size_t)a.gain_stride + ((unsigned)u >> a.group_shift)];
      }
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float *src = a.act + (size_t)m * a.act_stride + u * 32;
        if (a.act_vec) {
#pragma unroll
          for (int q = 0; q < 8; ++q) x[j][m][q] = *reinterpret_cast<const float4_t *>(src + 4 * q);
        } else {
#pragma unroll
          for (int q = 0; q < 8; ++q)
            x[j][m][q] = float4_t{src[4 * q], src[4 * q + 1], src[4 * q + 2], src[4 * q + 3]};
        }
      }
    }
  }

  float acc[R][M];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;
#pragma unroll
  for (int uj = 0; uj < UPL; ++uj) {
    if (!(row0 < a.N && u_first + kWave * uj < u_end)) continue;
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
        const uint32_t d = w[uj][r][j];
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
            part[r][m] = __builtin_fmaf((float)p[r][i].x, x[uj][m][2 * j][i], part[r][m]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int m = 0; m < M; ++m)
            part[r][m] = __builtin_fmaf((float)p[r][i].y, x[uj][m][2 * j + 1][i], part[r][m]);
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float total = 0.0f;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        total += x[uj][m][q].x; total += x[uj][m][q].y; total += x[uj][m][q].z; total += x[uj][m][q].w;
      }
      const float c = a.unit_bias * total;
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r][m] = __builtin_fmaf(s[uj][r], part[r][m] - c, acc[r][m]);
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
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (k < a.ksplit) total += red[wave + k][r][m];
    if (row0 + r < a.N) a.out[(size_t)m * a.out_stride + row0 + r] = total;
  }
}

// ---- the integer-dot form (one and two lanes) ------------------------------
//
// The register form's layout (a lane holds one unit of R rows; `ksplit` waves
// share a row tile), with the unit's product taken on the integer dot path:
// the workgroup stages x in digit form (stage_digits) while the row loads
// are in flight, and a lane then spends, per row and unit, four xors and
// 4 DIG v_dot8_i32_i4 on exact integer sums where the float form spends
// 32 conversions and 32 FMAs.  y = sum_units gain 2^(E - P) sum (c - 8) q.
constexpr int kDigits = 6;

__host__ __device__ constexpr size_t gemv_dot_lds_bytes(int M, int units) {
  return (size_t)M * units * (kDigitPitch * 16 + 4);
}

// LR (one lane only): lanes as workgroup rows, grid row blockIdx.y being lane
// blockIdx.y of the launch; a template constant, so the decode step's own
// one-lane launches carry no offset arithmetic (1-2% of their time).
template <int M, int R, int UPL, int GPT, bool LR = false>
__global__ __launch_bounds__(kGemvThreads) void gemv_q4_dot_kernel(GemvArgs a) {
  static_assert(!LR || M == 1, "lanes as rows run the one-lane form");
  extern __shared__ uint4_t lds_dig[];
  __shared__ float red[4][R][M];
  const size_t lane0 = LR ? blockIdx.y : 0;
  // wave-uniform indices in scalar registers; ksplit a power of two
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ks_log = __builtin_amdgcn_readfirstlane(a.ks_log);
  const int tile = blockIdx.x * (4 >> ks_log) + (wave >> ks_log);
  const int ks = wave & ((1 << ks_log) - 1);
  const int row0 = tile * R;
  const int units = a.K >> 5;
  const int u_end = (units * (ks + 1)) >> ks_log;
  const int u_first = ((units * ks) >> ks_log) + lane;
  uint4_t *dig = lds_dig;
  int *down = reinterpret_cast<int *>(dig + M * kDigitPitch * units);

  // Activations first, then the weights, all unconditionally: rows and
  // units past the end reload valid ones and get gain 0, so the arithmetic
  // needs no branch either (tail rows of a tile are computed, never stored).
  DigitLoads<GPT> held;
  digit_loads<M, GPT, true>(held, a.act + lane0 * (size_t)a.act_stride, a.act_stride, a.K);
  // Gains before codes, and each row's codes in row order: the row loop
  // below waits for one row at a time.
  uint4_t w[UPL][R];
  float s[UPL][R];
  bool live[UPL];
#pragma unroll
  for (int j = 0; j < UPL; ++j) {
    live[j] = row0 < a.N && u_first + kWave * j < u_end;
    const int u = min(u_first + kWave * j, units - 1);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = min(row0 + r, a.N - 1);
      s[j][r] = a.gains[(size_t)row * (size_t)a.gain_stride + ((unsigned)u >> a.group_shift)];
    }
  }
#pragma unroll
  for (int j = 0; j < UPL; ++j) {
    const int u = min(u_first + kWave * j, units - 1);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = min(row0 + r, a.N - 1);
      w[j][r] = __builtin_nontemporal_load(
          reinterpret_cast<const uint4_t *>(a.codes + (size_t)row * (size_t)a.row_stride) + u);
    }
  }
  digit_store<M, GPT, kDigits>(held, a.K, dig, down);

  float acc[R][M];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;
#pragma unroll
  for (int uj = 0; uj < UPL; ++uj) {
    const int u = min(u_first + kWave * uj, units - 1);
    if constexpr (M <= 2) {
      // every lane's digits held across the rows; a row waits for its own codes
      uint4_t dd[M][kDigits];
      int shift[M];
#pragma unroll
      for (int m = 0; m < M; ++m) {
#pragma unroll
        for (int j = 0; j < kDigits; ++j) dd[m][j] = dig[digit_slot(m, u, units) + j];
        shift[m] = down[m * units + u];
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint4_t c = w[uj][r] ^ 0x88888888u;
        const float gain = live[uj] ? s[uj][r] : 0.0f;
#pragma unroll
        for (int m = 0; m < M; ++m) {
          int t[kDigits];
#pragma unroll
          for (int j = 0; j < kDigits; ++j) t[j] = 0;
#pragma unroll
          for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int j = 0; j < kDigits; ++j)
              t[j] = __builtin_amdgcn_sdot8((int)c[q], (int)dd[m][j][q], t[j], false);
          acc[r][m] = __builtin_fmaf(gain, __builtin_amdgcn_ldexpf(digit_sum<kDigits>(t), shift[m]),
                                     acc[r][m]);
        }
      }
    } else {
      // one lane's digits at a time
      uint4_t c[R];
      float gain[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        c[r] = w[uj][r] ^ 0x88888888u;
        gain[r] = live[uj] ? s[uj][r] : 0.0f;
      }
#pragma unroll
      for (int m = 0; m < M; ++m) {
        uint4_t dd[kDigits];
#pragma unroll
        for (int j = 0; j < kDigits; ++j) dd[j] = dig[digit_slot(m, u, units) + j];
        const int shift = down[m * units + u];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          int t[kDigits];
#pragma unroll
          for (int j = 0; j < kDigits; ++j) t[j] = 0;
#pragma unroll
          for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int j = 0; j < kDigits; ++j)
              t[j] = __builtin_amdgcn_sdot8((int)c[r][q], (int)dd[j][q], t[j], false);
          acc[r][m] = __builtin_fmaf(gain[r], __builtin_amdgcn_ldexpf(digit_sum<kDigits>(t), shift),
                                     acc[r][m]);
        }
      }
    }
  }

#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = wave_sum_to_last(acc[r][m]);

  if (ks_log == 0) {
    if (lane == 63) {
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (row0 + r < a.N)
#pragma unroll
          for (int m = 0; m < M; ++m) a.out[(lane0 + (size_t)m) * a.out_stride + row0 + r] = acc[r][m];
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
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (k < (1 << ks_log)) total += red[wave + k][r][m];
    if (row0 + r < a.N) a.out[(lane0 + (size_t)m) * a.out_stride + row0 + r] = total;
  }
}

// ---- the integer-dot form for every code width (2, 4, 8 bits) --------------
//
// The shipped export's other planes: 2-bit (four codes a byte, low bits
// first, value + 2), 8-bit signed I8 (code_flip 128: the byte itself is the
// value) and one gain a row (group_shift 31).  The same arithmetic as
// gemv_q4_dot_kernel, over 16-byte slots of codes instead of units: a slot
// is two units of 2-bit codes, one of 4-bit codes, half of one of 8-bit codes.
// Per row and slot a lane spends
//   2-bit: 8 and/shift ops to spread 64 codes into nibbles, 48 v_dot8_i32_i4;
//   4-bit: 4 xors, 24 v_dot8_i32_i4;
//   8-bit: 4 xors, 12 v_dot4_i32_i8,
// on exact integer sums, then as before one float per unit (half unit at 8
// bits), times 2^(E - P) and the gain.  2-bit codes are dotted unsigned and
// their bias leaves through the staged activation sum (qsum); 4- and 8-bit
// codes are made signed by one xor with (code_flip ^ code_bias) replicated.
//
// Layout: a wave's 64 lanes are 2^subs_log sub-waves of 64 >> subs_log lanes,
// each over R rows of its own (short rows: a 2-bit row of 1536 codes is 24
// slots, so two sub-waves of 32 lanes keep 48 lanes busy instead of 24); a
// lane takes slots sl, sl + 64, ... of its rows; `ksplit` waves may share a
// row tile.  After the one staging of x, a workgroup walks `tile_iters` row
// tiles, gridDim.x tile groups apart, with the next tile's gains and codes
// requested before the current tile's arithmetic.  `blockIdx.y` takes a
// K-chunk of `chunk_cols` columns (a multiple of 128); chunks write partials
// [chunk][lanes][N] that gemv_chunk_sum_kernel adds.  `lanes` <= M: lanes past
// it reread the last lane and are not stored.
struct GemvCodeArgs {
  const uint8_t *codes;
  long long row_stride;
  const float *gains;
  int gain_stride;
  int group_shift;        // gain of unit u: u >> group_shift (31: one gain a row)
  const float *act;       // 16-byte aligned, act_stride % 4 == 0
  int act_stride;
  float *out;             // [lanes][out_stride], or partials [chunk][lanes][N]
  int out_stride;
  int lanes;
  int N, K;
  int chunk_cols;
  int ks_log;             // log2 of the waves that share a row tile
  int subs_log;           // log2 of the sub-waves (0 unless ks_log == 0 and UPL == 1)
  int tile_iters;         // row tiles a wave walks
  uint32_t code_xor;      // 4, 8-bit: makes a dword of codes signed values; 2-bit: undoes the flip
  int code_bias;          // 2-bit: taken off through qsum
};

__host__ __device__ constexpr size_t gemv_code_lds_bytes(int M, int units) {
  return (size_t)M * units * (kDigitPitch * 16 + 8);
}

// Sum over each sub-wave of 64 >> subs_log lanes; the total lands in the
// sub-wave's last lane.
__device__ __forceinline__ float sub_sum_to_last(float v, int subs_log) {
  v += dpp_move<0xB1>(v);
  v += dpp_move<0x4E>(v);
  v += dpp_move<0x141>(v);
  v += dpp_move<0x140>(v);
  if (subs_log >= 2) return v;
  v += dpp_move<0x142, 0xA>(v);
  if (subs_log == 1) return v;
  v += dpp_move<0x143, 0xC>(v);
  return v;
}

template <int BITS, int R, int UPL>
struct CodeTile {
  static constexpr int kSub = BITS == 2 ? 2 : 1;  // units a slot's gains cover
  uint4_t w[UPL][R];
  float s[UPL][R][kSub];
};

// TILED: the workgroup walks a.tile_iters tiles; otherwise exactly one.
template <int BITS, int M, int R, int UPL, int GPT, bool TILED>
__global__ __launch_bounds__(kGemvThreads) void gemv_code_dot_kernel(GemvCodeArgs a) {
  constexpr int FORM = CodeForm<BITS>::kDigits;
  constexpr int kSub = CodeTile<BITS, R, UPL>::kSub;
  extern __shared__ uint4_t lds_dig[];
  __shared__ float red[4][R][M];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ks_log = __builtin_amdgcn_readfirstlane(a.ks_log);
  const int subs_log = __builtin_amdgcn_readfirstlane(a.subs_log);
  const int ks = wave & ((1 << ks_log) - 1);
  const int sub = lane >> (6 - subs_log);
  const int sub_lane = lane & ((64 >> subs_log) - 1);
  const int rows_per_tile = R << subs_log;
  const int tile_step = gridDim.x * (4 >> ks_log);
  const int col0 = blockIdx.y * a.chunk_cols;
  const int cols = min(a.chunk_cols, a.K - col0);
  const int units = cols >> 5;
  const int slots = (cols * BITS + 127) >> 7;
  const int s_end = (slots * (ks + 1)) >> ks_log;
  const int s_first = ((slots * ks) >> ks_log) + sub_lane;
  const int unit0 = col0 >> 5;
  const uint8_t *code0 = a.codes + (size_t)(col0 / 8) * BITS;
  uint4_t *dig = lds_dig;
  int *down = reinterpret_cast<int *>(dig + M * kDigitPitch * units);
  int *qsum = down + M * units;

  // Every load unconditional (clamped rows, slots and units), gains before
  // codes; rows past N and slots past the part get gain 0.
  auto load_tile = [&](int tile, CodeTile<BITS, R, UPL> &t) {
    const int row0 = tile * rows_per_tile + sub * R;
#pragma unroll
    for (int j = 0; j < UPL; ++j) {
      const int sl = min(s_first + 64 * j, slots - 1);
      const bool in = s_first + 64 * j < s_end;
#pragma unroll
      for (int h = 0; h < kSub; ++h) {
        const int u_raw = BITS == 2 ? 2 * sl + h : BITS == 8 ? sl >> 1 : sl;
        const int u = min(u_raw, units - 1);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int row = min(row0 + r, a.N - 1);
          const float g = a.gains[(size_t)row * (size_t)a.gain_stride + ((unsigned)(unit0 + u) >> a.group_shift)];
          t.s[j][r][h] = in && u_raw < units && row0 + r < a.N ? g : 0.0f;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < UPL; ++j) {
      const int sl = min(s_first + 64 * j, slots - 1);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int row = min(row0 + r, a.N - 1);
        t.w[j][r] = __builtin_nontemporal_load(
            reinterpret_cast<const uint4_t *>(code0 + (size_t)row * (size_t)a.row_stride) + sl);
      }
    }
  };

  // Activations first, then the first tile's weights.
  DigitLoads<GPT> held;
  {
    const int last = a.lanes - 1;
    const int per_lane = cols >> 3;
#pragma unroll
    for (int i = 0; i < GPT; ++i) {
      const int g = digit_item(i, M * per_lane);
      const int m = M == 1 ? 0 : g / per_lane;
      const float *src = a.act + (size_t)min(m, last) * a.act_stride + col0 + 8 * (g - m * per_lane);
      const float4_t p = *reinterpret_cast<const float4_t *>(src);
      const float4_t q = *reinterpret_cast<const float4_t *>(src + 4);
      held.x[i][0] = p.x; held.x[i][1] = p.y; held.x[i][2] = p.z; held.x[i][3] = p.w;
      held.x[i][4] = q.x; held.x[i][5] = q.y; held.x[i][6] = q.z; held.x[i][7] = q.w;
    }
  }
  int tile = blockIdx.x * (4 >> ks_log) + (wave >> ks_log);
  CodeTile<BITS, R, UPL> cur;
  load_tile(tile, cur);
  digit_store_form<M, GPT, FORM>(held, cols, dig, down, qsum);

  const uint32_t cx = a.code_xor;
  const int tiles_total = (a.N + rows_per_tile - 1) / rows_per_tile;
  const int iters = TILED ? a.tile_iters : 1;
  for (int it = 0; it < iters; ++it) {
    CodeTile<BITS, R, UPL> nxt;
    if constexpr (TILED) load_tile(min(tile + tile_step, tiles_total - 1), nxt);

    float acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;
#pragma unroll
    for (int uj = 0; uj < UPL; ++uj) {
      const int sl = min(s_first + 64 * uj, slots - 1);
      if constexpr (BITS == 4) {
        const int u = sl;
#pragma unroll
        for (int m = 0; m < M; ++m) {
          uint4_t dd[6];
#pragma unroll
          for (int j = 0; j < 6; ++j) dd[j] = dig[digit_slot(m, u, units) + j];
          const int shift = down[m * units + u];
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const uint4_t c = cur.w[uj][r] ^ cx;
            int t[6];
#pragma unroll
            for (int j = 0; j < 6; ++j) t[j] = 0;
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
              for (int j = 0; j < 6; ++j) t[j] = __builtin_amdgcn_sdot8((int)c[q], (int)dd[j][q], t[j], false);
            acc[r][m] = __builtin_fmaf(cur.s[uj][r][0], __builtin_amdgcn_ldexpf(digit_sum<6>(t), shift), acc[r][m]);
          }
        }
      } else if constexpr (BITS == 2) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int u = min(2 * sl + h, units - 1);
#pragma unroll
          for (int m = 0; m < M; ++m) {
            uint4_t dd[6];
#pragma unroll
            for (int j = 0; j < 6; ++j) dd[j] = dig[digit_slot(m, u, units) + j];
            const int shift = down[m * units + u];
            const int bq = a.code_bias * qsum[m * units + u];
#pragma unroll
            for (int r = 0; r < R; ++r) {
              const uint32_t c0 = cur.w[uj][r][2 * h] ^ cx, c1 = cur.w[uj][r][2 * h + 1] ^ cx;
              const uint32_t n[4] = {c0 & 0x33333333u, (c0 >> 2) & 0x33333333u, c1 & 0x33333333u,
                                     (c1 >> 2) & 0x33333333u};
              int t[6];
#pragma unroll
              for (int j = 0; j < 6; ++j) t[j] = 0;
#pragma unroll
              for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int j = 0; j < 6; ++j) t[j] = __builtin_amdgcn_sdot8((int)n[q], (int)dd[j][q], t[j], false);
              acc[r][m] = __builtin_fmaf(cur.s[uj][r][h], __builtin_amdgcn_ldexpf(pair_digit_sum(t, bq), shift),
                                         acc[r][m]);
            }
          }
        }
      } else {
        const int u = sl >> 1, hf = sl & 1;
#pragma unroll
        for (int m = 0; m < M; ++m) {
          uint4_t dd[3];
#pragma unroll
          for (int j = 0; j < 3; ++j) dd[j] = dig[digit_slot(m, u, units) + 2 * j + hf];
          const int shift = down[m * units + u];
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const uint4_t c = cur.w[uj][r] ^ cx;
            int t[3] = {0, 0, 0};
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
              for (int j = 0; j < 3; ++j) t[j] = __builtin_amdgcn_sdot4((int)c[q], (int)dd[j][q], t[j], false);
            acc[r][m] = __builtin_fmaf(cur.s[uj][r][0],
                                       __builtin_amdgcn_ldexpf(byte_digit_sum(t[0], t[1], t[2]), shift), acc[r][m]);
          }
        }
      }
    }

#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) acc[r][m] = sub_sum_to_last(acc[r][m], subs_log);

    const int row0 = tile * rows_per_tile + sub * R;
    float *dst = a.out + (size_t)blockIdx.y * (size_t)a.lanes * (size_t)a.out_stride;
    if (ks_log == 0) {
      if (sub_lane == (64 >> subs_log) - 1) {
#pragma unroll
        for (int r = 0; r < R; ++r)
          if (row0 + r < a.N)
#pragma unroll
            for (int m = 0; m < M; ++m)
              if (m < a.lanes) dst[(size_t)m * a.out_stride + row0 + r] = acc[r][m];
      }
    } else {
      // one tile a wave group (tile_iters == 1, subs_log == 0)
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
#pragma unroll
        for (int k = 0; k < 4; ++k)
          if (k < (1 << ks_log)) total += red[wave + k][r][m];
        if (row0 + r < a.N && m < a.lanes) dst[(size_t)m * a.out_stride + row0 + r] = total;
      }
    }
    if constexpr (TILED) {
      tile += tile_step;
      cur = nxt;
    }
  }
}

// ---- calibrated planes: the product on the activation grid ------------------
//
// A plane whose export carries input_activation_scale (enter_gain = step > 0)
// is multiplied on quant_step's grid: each activation is its level L, an
// integer in [-128, 127] (level_group_store), so a row's sum
//     part = sum ((c ^ flip) - bias) L
// is an exact integer (the reference's level path, kern_row_code_level,
// app_core.c:3272-3296) and costs, per row and unit, a third of the digit
// form's dots: 4-bit codes 4 v_dot8_i32_i4 (c - 8 against L >> 4) and 4
// v_dot8_u32_u4 (c against L & 15); 2-bit codes the same on the spread
// nibbles; 8-bit codes 8 v_dot4_i32_i8 against L.  With one gain a row the
// row's integer parts add exactly across lanes and waves and the row closes
// as the reference closes it, gain * step * (float)part, one rounding each;
// with several groups each unit closes on its own group's gain.  The output
// then goes on the plane's leave grid (quant_step with leave_gain), fused.
// One K-chunk (M K <= 16384); layout as gemv_code_dot_kernel.
struct GemvLevelArgs {
  const uint8_t *codes;
  long long row_stride;
  const float *gains;
  int gain_stride;
  int group_shift;
  const float *act;
  int act_stride;
  float *out;
  int out_stride;
  int lanes;
  int N, K;
  int ks_log;
  int subs_log;
  uint32_t code_xor;      // 4-bit: undoes the flip; 8-bit: makes the bytes signed values; 2-bit: undoes the flip
  int code_bias;
  float step;             // enter_gain
  float leave;            // leave_gain (<= 0: none)
  int epi;                // IGL_LEVEL_EPI_*: the elementwise step that follows, fused
  const float *epi_in;    // its other operand, lane m at epi_in + m * epi_stride
  int epi_stride;
  // One lane (PRO): x is not read from `act` but formed by the residual
  // update of GemvGroupArgs; workgroup 0 writes s to `state_out` and, with
  // `x_out`, x itself there for the launches that read the same x next.
  const float *state_in;
  float *state_out;
  const float *lift;
  const float *lift_gain;
  float scale;
  int apply_scale;
  const float *norm_gain;
  float eps;
  int pro_vec;            // the K-vectors, state_out and x_out 16-byte aligned
  float *x_out;
  // FUSE (one lane, the same kind and enter step):
  //   kLevelPair: the up projection (`*2`) beside the gate one, the same
  //     rows; out = gelu(gate) * up;
  //   kLevelSegments: the rows of up to three planes one after the other,
  //     plane 2 from row first2, plane 3 from row first3 (N in all), each
  //     on its own leave grid into its own output
  const uint8_t *codes2;
  long long row_stride2;
  const float *gains2;
  int gain_stride2;
  float leave2;
  float *out2;
  const uint8_t *codes3;
  long long row_stride3;
  const float *gains3;
  int gain_stride3;
  float leave3;
  float *out3;
  int first2, first3;
};

enum { kLevelOne = 0, kLevelPair = 1, kLevelSegments = 2 };

__host__ __device__ constexpr size_t gemv_level_lds_bytes(int M, int units) {
  return (size_t)M * units * (kLevelPitch * 16 + 8);
}

__device__ __forceinline__ int sub_sum_to_last_int(int v, int subs_log) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, true);
  if (subs_log >= 2) return v;
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, true);
  if (subs_log == 1) return v;
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, true);
  return v;
}

// quant_step of one value (app_core.c:1930-1940); a step that is not positive
// leaves it.
__device__ __forceinline__ float grid_value(float v, float step) {
  if (!(step > 0.0f)) return v;
  float level = __builtin_rintf(v / step);
  if (level < -128.0f) level = -128.0f;
  if (level > 127.0f) level = 127.0f;
  return level * step;
}

// The prologue's loads of one thread: its eight-element groups of state_in,
// lift, lift_gain and norm_gain (an absent vector reads state_in in its place).
template <int PG>
struct PrologueLoads {
  float v[PG][4][8];
};

__device__ __forceinline__ void store_eight(float *dst, const float (&v)[8], int vec) {
  if (vec) {
    *reinterpret_cast<float4_t *>(dst) = float4_t{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<float4_t *>(dst + 4) = float4_t{v[4], v[5], v[6], v[7]};
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) dst[e] = v[e];
  }
}

// The residual update and norms of the level form's one-lane prologue, in two
// steps (loads ahead of the weights, then the arithmetic).  Thread t holds the
// eight-element groups of digit_item (t + 256 j, a group past the end standing
// for the same quarter of the last unit), so level_store_form stores x as it
// stores loaded activations; only groups in range count in the two sums.  The
// element operations are norm_add_kernel's.
template <int PG>
__device__ __forceinline__ void level_prologue_loads(const GemvLevelArgs &a, PrologueLoads<PG> &p) {
  const float *src[4] = {a.state_in, a.lift ? a.lift : a.state_in,
                         a.lift ? a.lift_gain : a.state_in,
                         a.norm_gain ? a.norm_gain : a.state_in};
  const int groups = a.K >> 3;
#pragma unroll
  for (int j = 0; j < PG; ++j) {
    const int g = digit_item(j, groups);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float *q = src[w] + 8 * g;
      if (a.pro_vec) {
        const float4_t lo = *reinterpret_cast<const float4_t *>(q);
        const float4_t hi = *reinterpret_cast<const float4_t *>(q + 4);
        p.v[j][w][0] = lo.x; p.v[j][w][1] = lo.y; p.v[j][w][2] = lo.z; p.v[j][w][3] = lo.w;
        p.v[j][w][4] = hi.x; p.v[j][w][5] = hi.y; p.v[j][w][6] = hi.z; p.v[j][w][7] = hi.w;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) p.v[j][w][e] = q[e];
      }
    }
  }
}

template <int PG>
__device__ __forceinline__ void level_prologue(const GemvLevelArgs &a, const PrologueLoads<PG> &p,
                                               DigitLoads<PG> &held, double *red) {
  const int n = a.K;
  const int groups = n >> 3;
  const bool lift = a.lift != nullptr;
  const bool normed = a.norm_gain != nullptr;
  double acc = 0.0;
#pragma unroll
  for (int j = 0; j < PG; ++j) {
    const bool in = (int)threadIdx.x + 256 * j < groups;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float l = in && lift ? p.v[j][1][e] : 0.0f;
      acc += (double)l * (double)l;
    }
  }
  // (a uniform branch: without lift or norm_gain its sum is skipped)
  const float shrink = lift ? rms_shrink(block_sum_f64_once(acc, red), n, a.eps) : 0.0f;
  float sv[PG][8];
  double acc2 = 0.0;
#pragma unroll
  for (int j = 0; j < PG; ++j) {
    const bool in = (int)threadIdx.x + 256 * j < groups;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float sum = p.v[j][0][e] + (lift ? p.v[j][1][e] : 0.0f) * shrink * (lift ? p.v[j][2][e] : 0.0f);
      if (a.apply_scale) sum *= a.scale;
      sv[j][e] = lift ? sum : p.v[j][0][e];
      const float c = in ? sv[j][e] : 0.0f;
      acc2 += (double)c * (double)c;
    }
  }
  const float shrink2 = normed ? rms_shrink(block_sum_f64_once(acc2, red + 4), n, a.eps) : 0.0f;
#pragma unroll
  for (int j = 0; j < PG; ++j) {
#pragma unroll
    for (int e = 0; e < 8; ++e) held.x[j][e] = normed ? sv[j][e] * shrink2 * p.v[j][3][e] : sv[j][e];
  }
  if (blockIdx.x == 0) {
#pragma unroll
    for (int j = 0; j < PG; ++j) {
      const int g = threadIdx.x + 256 * j;
      if (g >= groups) continue;
      if (lift) store_eight(a.state_out + 8 * g, sv[j], a.pro_vec);
      if (a.x_out) store_eight(a.x_out + 8 * g, held.x[j], a.pro_vec);
    }
  }
}

// PRO: one lane whose x is formed by the prologue above (M == 1).
template <int BITS, int M, int R, int UPL, int GPT, bool PRO = false, int FUSE = kLevelOne>
__global__ __launch_bounds__(kGemvThreads) void gemv_level_kernel(GemvLevelArgs a) {
  static_assert(!PRO || M == 1, "the prologue forms one lane");
  constexpr bool PAIR = FUSE == kLevelPair;
  constexpr bool SEG = FUSE == kLevelSegments;
  static_assert(!PAIR || (M == 1 && R % 2 == 0), "a pair: one lane, rows of both planes");
  static_assert(!SEG || M == 1, "segments: one lane");
  // rows of one plane a sub-wave: a pair's tile holds RP gate rows, then the
  // same RP rows of the up plane
  constexpr int RP = PAIR ? R / 2 : R;
  constexpr int FORM = CodeForm<BITS>::kDigits;
  constexpr int kSub = BITS == 2 ? 2 : 1;
  extern __shared__ uint4_t lds_lv[];
  __shared__ int ired[4][R][M];
  __shared__ float fred[4][R][M];
  __shared__ int bred[4][M];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ks_log = __builtin_amdgcn_readfirstlane(a.ks_log);
  const int subs_log = __builtin_amdgcn_readfirstlane(a.subs_log);
  const bool one_group = a.group_shift == 31;
  const int ks = wave & ((1 << ks_log) - 1);
  const int sub = lane >> (6 - subs_log);
  const int sub_lane = lane & ((64 >> subs_log) - 1);
  const int tile = blockIdx.x * (4 >> ks_log) + (wave >> ks_log);
  const int row0 = tile * (RP << subs_log) + sub * RP;
  const int units = a.K >> 5;
  const int slots = (a.K * BITS + 127) >> 7;
  const int s_end = (slots * (ks + 1)) >> ks_log;
  const int s_first = ((slots * ks) >> ks_log) + sub_lane;
  uint4_t *lv = lds_lv;
  int *corr = reinterpret_cast<int *>(lv + M * kLevelPitch * units);
  int *nanu = corr + M * units;

  DigitLoads<GPT> held;
  PrologueLoads<PRO ? GPT : 1> pl;
  __shared__ double pro_red[PRO ? 8 : 1];
  if (PRO) {
    level_prologue_loads<PRO ? GPT : 1>(a, pl);
  } else {
    const int last = a.lanes - 1;
    const int per_lane = a.K >> 3;
#pragma unroll
    for (int i = 0; i < GPT; ++i) {
      const int g = digit_item(i, M * per_lane);
      const int m = M == 1 ? 0 : g / per_lane;
      const float *src = a.act + (size_t)min(m, last) * a.act_stride + 8 * (g - m * per_lane);
      const float4_t p = *reinterpret_cast<const float4_t *>(src);
      const float4_t q = *reinterpret_cast<const float4_t *>(src + 4);
      held.x[i][0] = p.x; held.x[i][1] = p.y; held.x[i][2] = p.z; held.x[i][3] = p.w;
      held.x[i][4] = q.x; held.x[i][5] = q.y; held.x[i][6] = q.z; held.x[i][7] = q.w;
    }
  }
  // gains (one a row, or one a unit and row) before codes, all clamped
  uint4_t w[UPL][R];
  float s[UPL][R][kSub];
#pragma unroll
  for (int j = 0; j < UPL; ++j) {
    const int sl = min(s_first + 64 * j, slots - 1);
    const bool in = s_first + 64 * j < s_end;
#pragma unroll
    for (int h = 0; h < kSub; ++h) {
      const int u_raw = BITS == 2 ? 2 * sl + h : BITS == 8 ? sl >> 1 : sl;
      const int u = min(u_raw, units - 1);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const bool up = PAIR && r >= RP;
        int row = min(row0 + r % RP, a.N - 1);
        const float *gp = up ? a.gains2 : a.gains;
        int gs = up ? a.gain_stride2 : a.gain_stride;
        if constexpr (SEG) {
          const int sg = row >= a.first3 ? 2 : row >= a.first2 ? 1 : 0;
          row -= sg == 2 ? a.first3 : sg == 1 ? a.first2 : 0;
          gp = sg == 2 ? a.gains3 : sg == 1 ? a.gains2 : a.gains;
          gs = sg == 2 ? a.gain_stride3 : sg == 1 ? a.gain_stride2 : a.gain_stride;
        }
        const float g = gp[(size_t)row * (size_t)gs + ((unsigned)u >> a.group_shift)];
        s[j][r][h] = in && u_raw < units && row0 + r % RP < a.N ? g : 0.0f;
      }
    }
  }
#pragma unroll
  for (int j = 0; j < UPL; ++j) {
    const int sl = min(s_first + 64 * j, slots - 1);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const bool up = PAIR && r >= RP;
      int row = min(row0 + r % RP, a.N - 1);
      const uint8_t *cp = up ? a.codes2 : a.codes;
      long long rs = up ? a.row_stride2 : a.row_stride;
      if constexpr (SEG) {
        const int sg = row >= a.first3 ? 2 : row >= a.first2 ? 1 : 0;
        row -= sg == 2 ? a.first3 : sg == 1 ? a.first2 : 0;
        cp = sg == 2 ? a.codes3 : sg == 1 ? a.codes2 : a.codes;
        rs = sg == 2 ? a.row_stride3 : sg == 1 ? a.row_stride2 : a.row_stride;
      }
      w[j][r] = __builtin_nontemporal_load(reinterpret_cast<const uint4_t *>(cp + (size_t)row * (size_t)rs) + sl);
    }
  }
  if constexpr (PRO) level_prologue<GPT>(a, pl, held, pro_red);
  level_store_form<M, GPT, FORM>(held, a.K, a.step, a.code_bias, lv, corr, nanu);

  // one gain a row: exact integer parts (a slot past the part or the row adds
  // nothing: its gain is 0, so it is masked by that); several groups: floats
  int ip[R][M];
  float fp[R][M];
  int bad[M];
#pragma unroll
  for (int m = 0; m < M; ++m) bad[m] = 0;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) {
      ip[r][m] = 0;
      fp[r][m] = 0.0f;
    }
  const uint32_t cx = a.code_xor;
#pragma unroll
  for (int uj = 0; uj < UPL; ++uj) {
    const int sl = min(s_first + 64 * uj, slots - 1);
    const bool in = s_first + 64 * uj < s_end;
#pragma unroll
    for (int h = 0; h < kSub; ++h) {
      const int u_raw = BITS == 2 ? 2 * sl + h : BITS == 8 ? sl >> 1 : sl;
      const int u = min(u_raw, units - 1);
      const bool live = in && u_raw < units;
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const int cu = corr[m * units + u];
        bad[m] |= live && nanu[m * units + u] != 0;
        uint4_t lo, hi;
        if constexpr (BITS == 8) {
          lo = lv[level_slot(m, u, units) + (sl & 1)];
        } else {
          lo = lv[level_slot(m, u, units)];
          hi = lv[level_slot(m, u, units) + 1];
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
          int part;
          if constexpr (BITS == 8) {
            const uint4_t c = w[uj][r] ^ cx;
            part = 0;
#pragma unroll
            for (int q = 0; q < 4; ++q) part = __builtin_amdgcn_sdot4((int)c[q], (int)lo[q], part, false);
          } else {
            uint32_t n[4];
            if constexpr (BITS == 4) {
#pragma unroll
              for (int q = 0; q < 4; ++q) n[q] = w[uj][r][q] ^ cx;
            } else {
              const uint32_t c0 = w[uj][r][2 * h] ^ cx, c1 = w[uj][r][2 * h + 1] ^ cx;
              n[0] = c0 & 0x33333333u;
              n[1] = (c0 >> 2) & 0x33333333u;
              n[2] = c1 & 0x33333333u;
              n[3] = (c1 >> 2) & 0x33333333u;
            }
            int th = 0;
            uint32_t tl = 0;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              // 4-bit: c - 8 (signed) against the high nibbles; 2-bit: c itself
              const uint32_t sc = BITS == 4 ? n[q] ^ 0x88888888u : n[q];
              th = __builtin_amdgcn_sdot8((int)sc, (int)hi[q], th, false);
              tl = __builtin_amdgcn_udot8(n[q], lo[q], tl, false);
            }
            part = 16 * th + (int)tl - cu;
          }
          const float g = s[uj][r][h];
          if (one_group) {
            ip[r][m] += g != 0.0f ? part : 0;
          } else {
            fp[r][m] += g * a.step * (float)part;
          }
        }
      }
    }
  }

  // sums over the sub-wave, then over the waves that share the tile
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) {
      if (one_group)
        ip[r][m] = sub_sum_to_last_int(ip[r][m], subs_log);
      else
        fp[r][m] = sub_sum_to_last(fp[r][m], subs_log);
    }
#pragma unroll
  for (int m = 0; m < M; ++m) bad[m] = sub_sum_to_last_int(bad[m], subs_log);
  // One output (row r of the sub-wave's R, lane m): the row close as the
  // reference's, fl(fl(gain step) fl(part)), NaN for a lane that held one,
  // the leave grid, then the fused elementwise step.
  auto close = [&](int r, int m, int it, float ft, int b) {
    int row = row0 + r;
    if (row >= a.N || m >= a.lanes) return;
    const float *gp = a.gains;
    int gs = a.gain_stride;
    float leave = a.leave;
    float *out = a.out;
    if constexpr (SEG) {
      const int sg = row >= a.first3 ? 2 : row >= a.first2 ? 1 : 0;
      row -= sg == 2 ? a.first3 : sg == 1 ? a.first2 : 0;
      gp = sg == 2 ? a.gains3 : sg == 1 ? a.gains2 : a.gains;
      gs = sg == 2 ? a.gain_stride3 : sg == 1 ? a.gain_stride2 : a.gain_stride;
      leave = sg == 2 ? a.leave3 : sg == 1 ? a.leave2 : a.leave;
      out = sg == 2 ? a.out3 : sg == 1 ? a.out2 : a.out;
    }
    float y = one_group ? gp[(size_t)row * (size_t)gs] * a.step * (float)it : ft;
    if (b) y = __builtin_nanf("");
    y = grid_value(y, leave);
    // the reference's next step on this output (kern_gelu_gate): with the gate
    // projection's output, gelu(gate) * y; with the per-layer input, gelu(y) * it
    if (a.epi == IGL_LEVEL_EPI_GELU_RISE)
      y = gelu_near(a.epi_in[(size_t)m * a.epi_stride + row]) * y;
    else if (a.epi == IGL_LEVEL_EPI_GELU_MUL)
      y = gelu_near(y) * a.epi_in[(size_t)m * a.epi_stride + row];
    out[(size_t)m * a.out_stride + row] = y;
  };
  // A pair's output (row r of the sub-wave's RP, the one lane): both row
  // closes on their own leave grids, then kern_gelu_gate's gelu(gate) * up.
  auto close_pair = [&](int r, int itg, float ftg, int itu, float ftu, int b) {
    const int row = row0 + r;
    if (row >= a.N) return;
    float yg = one_group ? a.gains[(size_t)row * (size_t)a.gain_stride] * a.step * (float)itg : ftg;
    float yu = one_group ? a.gains2[(size_t)row * (size_t)a.gain_stride2] * a.step * (float)itu : ftu;
    if (b) {
      yg = __builtin_nanf("");
      yu = yg;
    }
    yg = grid_value(yg, a.leave);
    yu = grid_value(yu, a.leave2);
    a.out[row] = gelu_near(yg) * yu;
  };
  const bool owner = sub_lane == (64 >> subs_log) - 1;
  if (ks_log > 0) {
    // one tile a wave group (subs_log == 0): the waves' sums meet in LDS, and
    // lane r M + m of the first wave closes output (r, m), adding the waves'
    // parts in wave order
    if (owner) {
#pragma unroll
      for (int m = 0; m < M; ++m) {
        bred[wave][m] = bad[m];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          ired[wave][r][m] = ip[r][m];
          fred[wave][r][m] = fp[r][m];
        }
      }
    }
    __syncthreads();
    if constexpr (PAIR) {
      if (ks != 0 || lane >= RP) return;
      int itg = 0, itu = 0, b = 0;
      float ftg = 0.0f, ftu = 0.0f;
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (k < (1 << ks_log)) {
          itg += ired[wave + k][lane][0];
          ftg += fred[wave + k][lane][0];
          itu += ired[wave + k][lane + RP][0];
          ftu += fred[wave + k][lane + RP][0];
          b += bred[wave + k][0];
        }
      close_pair(lane, itg, ftg, itu, ftu, b);
      return;
    }
    if (ks != 0 || lane >= R * M) return;
    const int r = lane / M;
    const int m = lane - r * M;
    int it = 0, b = 0;
    float ft = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (k < (1 << ks_log)) {
        it += ired[wave + k][r][m];
        ft += fred[wave + k][r][m];
        b += bred[wave + k][m];
      }
    close(r, m, it, ft, b);
    return;
  }
  if (!owner) return;
  if constexpr (PAIR) {
#pragma unroll
    for (int r = 0; r < RP; ++r) close_pair(r, ip[r][0], fp[r][0], ip[r + RP][0], fp[r + RP][0], bad[0]);
    return;
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) close(r, m, ip[r][m], fp[r][m], bad[m]);
}

// ---- real planes: F32, F16 or BF16 rows -------------------------------------
//
// kern_mat_vec_band's PLANE_REAL arm (app_core.c:4239-4248): every row dotted
// with every lane in fp32.  The export keeps one such plane,
// per_layer_model_projection (8960 x 1536 bf16, 26.25 MiB a decode step).
// A wave owns R rows; a lane streams 16-byte slots of them (eight bf16/f16
// or four f32 values), converts each value exactly to fp32 (bf16: a shift;
// f16: the conversion) and multiplies it into per-lane fp32 accumulators
// against x, which the workgroup stages once in LDS.  `blockIdx.y` takes a
// K-chunk; chunks write partials [chunk][lanes][N] for gemv_chunk_sum_kernel.
struct GemvRealArgs {
  const uint8_t *rows;
  long long row_bytes;
  const float *act;       // 16-byte aligned, act_stride % 4 == 0
  int act_stride;
  int lanes;              // <= M
  float *out;
  int out_stride;
  int N, K;
  int chunk_cols;         // a multiple of 64
};

template <int TYPE>
struct RealSlot {
  static constexpr int kValues = TYPE == IGL_STORE_F32 ? 4 : 8;
  static constexpr int kBytes = TYPE == IGL_STORE_F32 ? 4 : 2;
};

template <int TYPE>
__device__ __forceinline__ void real_values(const uint4_t w, float (&v)[RealSlot<TYPE>::kValues]) {
  if constexpr (TYPE == IGL_STORE_F32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = __uint_as_float(w[i]);
  } else if constexpr (TYPE == IGL_STORE_BF16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const half2_t h = as_half2(w[i]);
      v[2 * i] = (float)h.x;
      v[2 * i + 1] = (float)h.y;
    }
  }
}

constexpr int kRealRows = 4;

template <int TYPE, int M>
__global__ __launch_bounds__(kGemvThreads) void gemv_real_kernel(GemvRealArgs a) {
  extern __shared__ float4_t real_xs[];  // [M][cols / 4]
  constexpr int R = kRealRows;
  constexpr int kPer = RealSlot<TYPE>::kValues;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col0 = blockIdx.y * a.chunk_cols;
  const int cols = min(a.chunk_cols, a.K - col0);
  const int quads = cols >> 2;
  const int slots = cols / kPer;
  const int row0 = (blockIdx.x * 4 + wave) * R;

  const uint8_t *base[R];
#pragma unroll
  for (int r = 0; r < R; ++r)
    base[r] = a.rows + (size_t)min(row0 + r, a.N - 1) * (size_t)a.row_bytes +
              (size_t)col0 * RealSlot<TYPE>::kBytes;
  // the first slot's rows go out before the staging loads
  uint4_t w[R];
  const int s0 = min(lane, slots - 1);
#pragma unroll
  for (int r = 0; r < R; ++r) w[r] = __builtin_nontemporal_load(reinterpret_cast<const uint4_t *>(base[r]) + s0);
  for (int i = tid; i < M * quads; i += kGemvThreads) {
    const int m = i / quads;
    const int q = i - m * quads;
    real_xs[i] = *reinterpret_cast<const float4_t *>(a.act + (size_t)min(m, a.lanes - 1) * a.act_stride +
                                                     col0 + 4 * q);
  }
  __syncthreads();

  float acc[R][M];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;
  for (int s = lane; s < slots; s += kWave) {
    uint4_t next[R];
    const int sn = min(s + kWave, slots - 1);
#pragma unroll
    for (int r = 0; r < R; ++r) next[r] = __builtin_nontemporal_load(reinterpret_cast<const uint4_t *>(base[r]) + sn);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float x[kPer];
      const float4_t xa = real_xs[m * quads + s * (kPer / 4)];
      x[0] = xa.x; x[1] = xa.y; x[2] = xa.z; x[3] = xa.w;
      if constexpr (kPer == 8) {
        const float4_t xb = real_xs[m * quads + s * 2 + 1];
        x[4] = xb.x; x[5] = xb.y; x[6] = xb.z; x[7] = xb.w;
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float v[kPer];
        real_values<TYPE>(w[r], v);
#pragma unroll
        for (int i = 0; i < kPer; ++i) acc[r][m] = __builtin_fmaf(v[i], x[i], acc[r][m]);
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) w[r] = next[r];
  }

#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = wave_sum_to_last(acc[r][m]);
  if (lane != 63) return;
  float *dst = a.out + (size_t)blockIdx.y * (size_t)a.lanes * (size_t)a.out_stride;
#pragma unroll
  for (int r = 0; r < R; ++r)
    if (row0 + r < a.N)
#pragma unroll
      for (int m = 0; m < M; ++m)
        if (m < a.lanes) dst[(size_t)m * a.out_stride + row0 + r] = acc[r][m];
}

// ---- a few activation rows against several planes in one launch (decode) ---
//
// The integer-dot form for one lane and four rows a wave, over up to three
// planes that read the same activations (the query, key and value
// projections; the gate and up projections), with the epilogue the decode
// step applies next:
//   GEMV_SEGMENTS  the planes' rows one after another, each stored as it is;
//   GEMV_GELU_PAIR planes 0 and 1 have the same rows: a wave takes rows n, n+1
//                  of both and stores gelu(plane 0) * plane 1 (kern_gelu_gate,
//                  app_core.c:5105-5190);
//   GEMV_GELU_MUL  one plane, stored as gelu(y[n]) * mul[n] (the per-layer
//                  input gate, session_layer 11718-11723).
// Each row's sum is formed as gemv_q4_dot_kernel forms it with one unit a
// lane; with the same K-split the results are those of separate launches
// followed by the elementwise kernel, bit for bit.  Two to eight lanes (a
// speculative block) run as that many rows of workgroups (blockIdx.y = lane,
// `lane_rows`): every lane's arithmetic is the one-lane step's, and each row
// reads the planes again, the repeats served by the L2 and the MALL (a
// two-lane block 1.75 -> 1.64 ms against a form that holds both lanes in
// each wave, whose sums cost twice the dot instructions a row).
enum { GEMV_SEGMENTS = 0, GEMV_GELU_PAIR = 1, GEMV_GELU_MUL = 2 };

struct GemvGroupArgs {
  const uint8_t *codes[3];
  long long row_stride[3];
  const float *gains[3];
  int gain_stride[3];
  int rows[3];            // rows of each plane
  float *out[3];          // GEMV_SEGMENTS: one output row per plane; otherwise out[0]
  int out_stride[3];      // floats between lanes of out[s]
  int segments;
  int tiles;              // four-row tiles over all planes
  int group_shift;
  const float *act;
  int act_stride;         // floats between lanes of act
  int act_vec;            // act 16-byte aligned and act_stride % 4 == 0
  int K;
  int ksplit;
  float unit_bias;
  const float *mul;       // GEMV_GELU_MUL
  int mul_stride;         // floats between lanes of mul
  int lane_rows;          // lanes, one a row of workgroups (blockIdx.y)
  // The residual update in front of the product (with `state_in` set): the
  // activations are not read from `act` but formed in every workgroup as
  //   s = (state_in + norm(lift) * lift_gain) * scale   (lift NULL: s = state_in)
  //   x = norm(s) * norm_gain                           (norm_gain NULL: x = s)
  // with the float operations of norm_add_kernel; workgroup 0 of each lane
  // writes s to `state_out`, which must not alias `state_in`.  Lanes of
  // state_in, state_out and lift lie `lane_stride` floats apart.
  int lane_stride;
  const float *state_in;
  float *state_out;
  const float *lift;
  const float *lift_gain;
  float scale;
  int apply_scale;
  const float *norm_gain;
  float eps;
  int pro_vec;            // every prologue vector (and state_out) 16-byte aligned
};

// The update above in the kernel's digit form (into `dig` / `down`, as
// digit_store stages x), in two steps so that a kernel can issue the loads
// ahead of its weight loads.  Thread t holds the eight-element groups
// g = t + 256 j (j < PG) of every K-vector, so a group's x is formed in
// registers and digitized there (the four groups of a unit sit in one quad):
// nothing passes through LDS but the two block sums and the digits.  Every
// load is issued: an absent vector reads state_in in its place, groups past
// K / 8 reread the last one, and the values are then masked.  The element
// operations are norm_add_kernel's; only the double sums of the two norms add
// in another order (a thread's eight elements, then the waves).
template <int PG>
__device__ __forceinline__ void prologue_loads(const GemvGroupArgs &a, PrologueLoads<PG> &p, int lane0) {
  const size_t off = (size_t)lane0 * (size_t)a.lane_stride;  // the workgroup row's lane
  const float *state = a.state_in + off;
  const float *src[4] = {state, a.lift ? a.lift + off : state, a.lift ? a.lift_gain : state,
                         a.norm_gain ? a.norm_gain : state};
  const int groups = a.K >> 3;
#pragma unroll
  for (int j = 0; j < PG; ++j) {
    const int g = min((int)threadIdx.x + 256 * j, groups - 1);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float *q = src[w] + 8 * g;
      if (a.pro_vec) {
        const float4_t lo = *reinterpret_cast<const float4_t *>(q);
        const float4_t hi = *reinterpret_cast<const float4_t *>(q + 4);
        p.v[j][w][0] = lo.x; p.v[j][w][1] = lo.y; p.v[j][w][2] = lo.z; p.v[j][w][3] = lo.w;
        p.v[j][w][4] = hi.x; p.v[j][w][5] = hi.y; p.v[j][w][6] = hi.z; p.v[j][w][7] = hi.w;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) p.v[j][w][e] = q[e];
      }
    }
  }
}

// The two block sums use their own LDS slots (`red`, 2 x 4 doubles), so
// neither needs a barrier after its reads; ends with the barrier after the
// digit stores.
template <int PG>
__device__ __forceinline__ void group_prologue(const GemvGroupArgs &a, const PrologueLoads<PG> &p,
                                               uint4_t *dig, int *down, double *red, int lane0) {
  const int n = a.K;
  const int groups = n >> 3;
  const int units = n >> 5;
  const bool lift = a.lift != nullptr;
  const bool normed = a.norm_gain != nullptr;
  float sv[PG][8], lv[PG][8], gv[PG][8], nv[PG][8];
#pragma unroll
  for (int j = 0; j < PG; ++j) {
    const bool in = (int)threadIdx.x + 256 * j < groups;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      sv[j][e] = in ? p.v[j][0][e] : 0.0f;
      lv[j][e] = in && lift ? p.v[j][1][e] : 0.0f;
      gv[j][e] = in && lift ? p.v[j][2][e] : 0.0f;
      nv[j][e] = in && normed ? p.v[j][3][e] : 0.0f;
    }
  }
  double acc = 0.0;
#pragma unroll
  for (int j = 0; j < PG; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc += (double)lv[j][e] * (double)lv[j][e];
  // (a uniform branch: without lift or norm_gain its sum is skipped)
  const float shrink = lift ? rms_shrink(block_sum_f64_once(acc, red), n, a.eps) : 0.0f;
#pragma unroll
  for (int j = 0; j < PG; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float sum = sv[j][e] + lv[j][e] * shrink * gv[j][e];
      if (a.apply_scale) sum *= a.scale;
      sv[j][e] = lift ? sum : sv[j][e];
    }
  if (lift && blockIdx.x == 0) {
#pragma unroll
    for (int j = 0; j < PG; ++j) {
      const int g = threadIdx.x + 256 * j;
      if (g < groups) {
        float *q = a.state_out + (size_t)lane0 * (size_t)a.lane_stride + 8 * g;
        if (a.pro_vec) {
          *reinterpret_cast<float4_t *>(q) = float4_t{sv[j][0], sv[j][1], sv[j][2], sv[j][3]};
          *reinterpret_cast<float4_t *>(q + 4) = float4_t{sv[j][4], sv[j][5], sv[j][6], sv[j][7]};
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) q[e] = sv[j][e];
        }
      }
    }
  }
  double acc2 = 0.0;
#pragma unroll
  for (int j = 0; j < PG; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc2 += (double)sv[j][e] * (double)sv[j][e];
  const float shrink2 = normed ? rms_shrink(block_sum_f64_once(acc2, red + 4), n, a.eps) : 0.0f;
#pragma unroll
  for (int j = 0; j < PG; ++j) {
    const int g = threadIdx.x + 256 * j;
    float x[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = normed ? sv[j][e] * shrink2 * nv[j][e] : sv[j][e];
    // a unit's four groups are one quad, all in or all out (K % 32 == 0)
    if (g < groups) digit_group_store<kDigits>(x, 0, g, units, dig, down);
  }
  __syncthreads();
}

// PRO: 0, or the eight-element groups a thread holds in the prologue
// (K <= 2048 PRO).
// GPT (PRO 0): the eight-element groups of x a thread stages, K <= 2048 GPT.
// TPW: the four-row tiles a wave walks (KS 1 only): one workgroup then serves
// 16 TPW rows, so TPW times fewer workgroups repeat the prologue and the
// staging of x; a wave requests every tile's gains and codes up front.
// Each row's sum is formed as gemv_q4_dot_kernel forms it.
template <int MODE, int PRO, int GPT, int KS, int TPW>
__global__ __launch_bounds__(kGemvThreads) void gemv_q4_group_kernel(GemvGroupArgs a) {
  static_assert(TPW == 1 || KS == 1, "several tiles a wave only without a K split");
  constexpr int R = 4;
  constexpr int kTilesPerBlock = 4 / KS;
  constexpr int kItems = GPT;
  __shared__ float red[4][R];
  __shared__ double pro_red[8];
  // the digit form of x, sized at launch (gemv_dot_lds_bytes(1, K / 32)):
  // the LDS a workgroup holds bounds how many share a CU
  extern __shared__ uint4_t lds_grp[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tile0 = (blockIdx.x * kTilesPerBlock + wave / KS) * TPW;
  const int ks = wave % KS;
  // the lane of this row of workgroups (the arguments stay as passed: a
  // written copy would live in scratch)
  const int lane0 = a.lane_rows > 1 ? (int)blockIdx.y : 0;
  const int units = a.K >> 5;
  const int u_raw = (units * ks) / KS + lane;
  const bool lane_has = u_raw < (units * (ks + 1)) / KS;
  const int u = min(u_raw, units - 1);
  uint4_t *dig = lds_grp;
  int *down = reinterpret_cast<int *>(lds_grp + kDigitPitch * units);

  // Row r of tile i: which plane, which row of it (tiles past the end reread
  // the last row; their sums are dropped).
  int plane[TPW][R], prow[TPW][R];
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const int tile_c = min(tile0 + i, a.tiles - 1);
    if (MODE == GEMV_GELU_PAIR) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        plane[i][r] = r >> 1;
        prow[i][r] = min(2 * tile_c + (r & 1), a.rows[0] - 1);
      }
    } else {
      int seg = 0, first = 0;
      const int row0 = tile_c * R;
      if (a.segments > 1 && row0 >= a.rows[0]) { seg = 1; first = a.rows[0]; }
      if (a.segments > 2 && row0 >= a.rows[0] + a.rows[1]) { seg = 2; first = a.rows[0] + a.rows[1]; }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        plane[i][r] = seg;
        prow[i][r] = min(row0 - first + r, a.rows[seg] - 1);
      }
    }
  }

  // The activation side first (the prologue's vectors, or x itself), then the
  // weights, gains before codes: vmcnt retires loads in order, so the block
  // forms x while the weights are in flight, and each row waits only for its
  // own codes.
  PrologueLoads<PRO ? PRO : 1> pl;
  DigitLoads<kItems> held;
  if (PRO)
    prologue_loads<PRO ? PRO : 1>(a, pl, lane0);
  else if (a.act_vec)
    digit_loads<1, kItems, true>(held, a.act + (size_t)lane0 * (size_t)a.act_stride, 0, a.K);
  else
    digit_loads<1, kItems, false>(held, a.act + (size_t)lane0 * (size_t)a.act_stride, 0, a.K);
  float s[TPW][R];
  uint4_t w[TPW][R];
  // GEMV_GELU_MUL: the multipliers of the tiles' rows, requested now rather
  // than after the sums (a round trip at the end of the chain)
  float mulv[TPW][R];
  if (MODE == GEMV_GELU_MUL) {
#pragma unroll
    for (int i = 0; i < TPW; ++i)
#pragma unroll
      for (int r = 0; r < R; ++r)
        mulv[i][r] = a.mul[(size_t)lane0 * (size_t)a.mul_stride + min((tile0 + i) * R + r, a.rows[0] - 1)];
  }
#pragma unroll
  for (int i = 0; i < TPW; ++i)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int p = plane[i][r];
      s[i][r] = a.gains[p][(size_t)prow[i][r] * (size_t)a.gain_stride[p] + ((unsigned)u >> a.group_shift)];
    }
#pragma unroll
  for (int i = 0; i < TPW; ++i)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int p = plane[i][r];
      w[i][r] = __builtin_nontemporal_load(
          reinterpret_cast<const uint4_t *>(a.codes[p] + (size_t)prow[i][r] * (size_t)a.row_stride[p]) + u);
    }
  if (PRO) {
    group_prologue<PRO ? PRO : 1>(a, pl, dig, down, pro_red, lane0);
  } else {
    digit_store<1, kItems, kDigits>(held, a.K, dig, down);
  }

  uint4_t dd[kDigits];
#pragma unroll
  for (int j = 0; j < kDigits; ++j) dd[j] = dig[digit_slot(0, u, units) + j];
  const int shift = down[u];
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const int tile = tile0 + i;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint4_t c = w[i][r] ^ 0x88888888u;
      int t[kDigits];
#pragma unroll
      for (int j = 0; j < kDigits; ++j) t[j] = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int j = 0; j < kDigits; ++j)
          t[j] = __builtin_amdgcn_sdot8((int)c[q], (int)dd[j][q], t[j], false);
      const float gain = lane_has && tile < a.tiles ? s[i][r] : 0.0f;
      acc[r] = wave_sum_to_last(gain * __builtin_amdgcn_ldexpf(digit_sum<kDigits>(t), shift));
    }

    if (KS > 1) {
      if (lane == 63) {
#pragma unroll
        for (int r = 0; r < R; ++r) red[wave][r] = acc[r];
      }
      __syncthreads();
      if (ks != 0 || lane != 63) return;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float total = 0.0f;
        for (int k = 0; k < KS; ++k) total += red[wave + k][r];
        acc[r] = total;
      }
    } else if (lane != 63) {
      continue;
    }
    if (tile >= a.tiles) continue;
    if (MODE == GEMV_GELU_PAIR) {
      const int n0 = 2 * tile;
      float *o = a.out[0] + (size_t)lane0 * (size_t)a.out_stride[0];
      if (n0 < a.rows[0]) o[n0] = gelu_near(acc[0]) * acc[2];
      if (n0 + 1 < a.rows[0]) o[n0 + 1] = gelu_near(acc[1]) * acc[3];
    } else {
      const int row0 = tile * R;
      const int first = plane[i][0] == 0 ? 0 : plane[i][0] == 1 ? a.rows[0] : a.rows[0] + a.rows[1];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int n = row0 - first + r;
        if (n >= a.rows[plane[i][0]]) break;
        if (MODE == GEMV_GELU_MUL)
          a.out[0][(size_t)lane0 * (size_t)a.out_stride[0] + n] = gelu_near(acc[r]) * mulv[i][r];
        else
          a.out[plane[i][0]][(size_t)lane0 * (size_t)a.out_stride[plane[i][0]] + n] = acc[r];
      }
    }
  }
}


// ---- the small-lane form on the matrix cores (1..16 lanes) ----------------
//
// One v_mfma_f32_16x16x32_f16 per (16 rows, unit):
//   * A (16 rows x 32 codes) is c - code_bias, exact in binary16.  A lane
//     loads one row's whole unit (16 bytes); four units sit across the four
//     16-lane groups of a wave and a 4 x 4 exchange of dwords between the
//     groups (two permlane32 and two permlane16 swaps) leaves in group q the
//     q-th eight codes of each unit, the layout the instruction reads.
//   * B (32 codes x 16 columns): up to 8 lanes (narrow), column m < 8 is
//     lane m's activations times 2^e rounded to binary16 (the high part),
//     column m + 8 the remainder rounded again (the low part), so hi + lo
//     carries x to 22 bits; 9 to 16 lanes (WIDE), column m is lane m in two
//     B tiles, the high parts and the low parts.  e is chosen per (unit,
//     lane) to put the unit's largest |x| in [2^14, 2^15): neither part
//     overflows, and the low part stays normal.
//   * narrow: D columns m and m + 8 hold 2^e sum (c - bias) x_hi and ... x_lo,
//     each a sum of exact products in fp32; 2^-e and the gain multiply them
//     into the fp32 accumulator, and row_shr:8 adds the pair at the end.
//     WIDE: the low tile's product accumulates onto the high tile's, so D
//     column m holds 2^e sum (c - bias) (x_hi + x_lo) for lane m; the weights
//     are read and converted once for all 16 lanes.
// A workgroup owns `tiles_per_block` 16-row tiles over a chunk of
// `chunk_units` units; its four waves split that as tiles x K-parts and build
// the chunk's B tiles and gains in LDS once while their code loads are in
// flight.  K-parts add in a fixed order through LDS; K-chunks (blockIdx.y)
// write partials that gemv_chunk_sum_kernel adds in chunk order.
struct GemvMfmaArgs {
  const uint8_t *codes;
  long long row_stride;
  const float *gains;
  int gain_stride;
  int group_shift;
  const float *act;
  int act_stride;
  int act_vec;
  float *out;             // [M][out_stride], or partials [chunk][M][N]
  int out_stride;
  int M, N, K;
  int tiles_per_block;    // 1, 2 or 4
  int chunk_units;        // units of K one workgroup covers
  float code_bias;
  int gain_vec;           // one gain a unit, rows 16-byte aligned: float4 gain loads
};

__device__ __forceinline__ void lane_group_exchange(uint32_t &d0, uint32_t &d1, uint32_t &d2,
                                                    uint32_t &d3) {
  // Group g's dword j goes to group j's register g.
  auto s02 = __builtin_amdgcn_permlane32_swap(d0, d2, false, false);
  auto s13 = __builtin_amdgcn_permlane32_swap(d1, d3, false, false);
  auto s01 = __builtin_amdgcn_permlane16_swap(s02[0], s13[0], false, false);
  auto s23 = __builtin_amdgcn_permlane16_swap(s02[1], s13[1], false, false);
  d0 = s01[0];
  d1 = s01[1];
  d2 = s23[0];
  d3 = s23[1];
}

// Eight codes of a dword as binary16 (c - bias), in the order 0,4,1,5,2,6,3,7.
__device__ __forceinline__ half8_t codes_less_bias(uint32_t d, uint32_t exp16, half2_t shift) {
  const half2_t p0 = nibble_pair16<0>(d, exp16) - shift;
  const half2_t p1 = nibble_pair16<1>(d, exp16) - shift;
  const half2_t p2 = nibble_pair16<2>(d, exp16) - shift;
  const half2_t p3 = nibble_pair16<3>(d, exp16) - shift;
  return half8_t{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

constexpr int kMfmaGains = 4;  // pad of the gain rows in LDS (keeps 16-byte reads aligned)

template <int NG, bool VEC, bool WIDE>
__global__ __launch_bounds__(256) void gemv_q4_mfma_kernel(GemvMfmaArgs a) {
  // lanes a B column holds, the tiles a k-chunk has, activation items a thread
  constexpr int kCols = WIDE ? 16 : 8;
  constexpr int kTerms = WIDE ? 2 : 1;
  constexpr int kIt = WIDE ? 16 : 8;
  extern __shared__ uint4_t lds_u4[];
  const int RTB = a.tiles_per_block;
  const int parts = 4 / RTB;
  const int CU = a.chunk_units;
  const int rows_b = RTB * 16;
  const int pitch = rows_b + kMfmaGains;
  uint4_t *bt = lds_u4;                                       // [CU][4 groups][terms][16 columns]
  float *gs = reinterpret_cast<float *>(bt + CU * 64 * kTerms);  // [CU][pitch]
  float *sc = gs + CU * pitch;                                // [CU][kCols]
  float *red = sc + CU * kCols;                               // [parts][RTB][16][kCols]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int t = wave % RTB;
  const int part = wave / RTB;
  const int r = lane & 15;
  const int q = lane >> 4;
  const int chunk = blockIdx.y;
  const int unit_c0 = chunk * CU;
  const int row_b0 = blockIdx.x * rows_b;
  const int u_w0 = part * (NG * 4);

  // Staging loads go out first and unconditionally (indices past the end are
  // clamped and their values dropped), then the code loads.  The activations
  // go first: they come from the cache, the gains and codes from memory, and
  // loads retire in order, so the B tiles are formed while the gains and
  // codes are still in flight (gains first: 3.3 us into the launch under a
  // full stream, against about 1 us for the activations).
  // Activations: item i = 4 M u + 4 m + g is x[m][32 u + 8 g .. + 7] (at most
  // kIt a thread: 64 units x 16 lanes x 4 groups).  B columns m >= M are never
  // written; they only reach outputs that are not stored.  u = i / (4 M) by a
  // multiply, exact for every i < 4096 and M <= 16 (the 2^21 reciprocal's
  // excess, i / 2^21 < 1 / 512, stays under 1 / (4 M)).
  const int per_u = 4 * a.M;
  const int items = CU * per_u;
  const uint32_t inv_u = ((1u << 21) + (uint32_t)per_u - 1u) / (uint32_t)per_u;
  float4_t xa[kIt], xb[kIt];
#pragma unroll
  for (int k = 0; k < kIt; ++k) {
    const int i = min(tid + 256 * k, items - 1);
    const int u = (int)(((uint32_t)i * inv_u) >> 21);
    const int m = (i - u * per_u) >> 2;
    const float *src =
        a.act + (size_t)m * (size_t)a.act_stride + (size_t)(unit_c0 + u) * 32 + 8 * (i & 3);
    if (VEC) {
      xa[k] = *reinterpret_cast<const float4_t *>(src);
      xb[k] = *reinterpret_cast<const float4_t *>(src + 4);
    } else {
      xa[k] = float4_t{src[0], src[1], src[2], src[3]};
      xb[k] = float4_t{src[4], src[5], src[6], src[7]};
    }
  }
  // Gains (VEC): each wave loads the slice it reads, its tile's 16 rows over
  // its part's 4 NG units, as float4 runs (lane i: row i % 16, run i / 16),
  // and transposes it into LDS itself after the barrier, so the barrier waits
  // only for the B tiles and the products start while gains and codes are
  // still arriving.
  constexpr int kRunsPerLane = (NG + 3) / 4;
  float4_t gv[kRunsPerLane];
  if (VEC) {
#pragma unroll
    for (int k = 0; k < kRunsPerLane; ++k) {
      const int i = lane + 64 * k;
      const int c4 = min(i >> 4, NG - 1);
      const int row = min(row_b0 + 16 * t + (i & 15), a.N - 1);
      gv[k] = *reinterpret_cast<const float4_t *>(a.gains + (size_t)row * (size_t)a.gain_stride +
                                                 unit_c0 + u_w0 + 4 * c4);
    }
  }

  // Codes: lane (r, q) takes unit u_w0 + 4 g + q of its row.
  uint4_t w[NG];
  {
    const int row = min(row_b0 + 16 * t + r, a.N - 1);  // tail rows are computed, never stored
    const uint4_t *src =
        reinterpret_cast<const uint4_t *>(a.codes + (size_t)row * (size_t)a.row_stride) + unit_c0 +
        u_w0 + q;
#pragma unroll
    for (int g = 0; g < NG; ++g) w[g] = __builtin_nontemporal_load(src + 4 * g);
  }

  // Nothing below may sink a staging load past the code loads (a load used
  // only under a branch is otherwise moved into it, and its wait then covers
  // every code load).
  asm volatile("" ::: "memory");

  // B tiles; the four items of a (unit, lane) sit in one quad and agree on e.
  // Past the items (a bound uniform over the workgroup) a thread's quads
  // recompute the last item and store nothing.
#pragma unroll
  for (int k = 0; k < kIt; ++k) {
    if (256 * k >= items) break;
    const int i_raw = tid + 256 * k;
    const bool own = i_raw < items;
    const int i = min(i_raw, items - 1);
    const int u = (int)(((uint32_t)i * inv_u) >> 21);
    const int rem = i - u * per_u;
    const int g = rem & 3;
    const int m = rem >> 2;
    const float v[8] = {xa[k].x, xa[k].y, xa[k].z, xa[k].w, xb[k].x, xb[k].y, xb[k].z, xb[k].w};
    float peak = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) peak = fmaxf(peak, fabsf(v[j]));
    peak = fmaxf(peak, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, peak), 0xB1, 0xF, 0xF, false)));
    peak = fmaxf(peak, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, peak), 0x4E, 0xF, 0xF, false)));
    int e = 0;
    if (peak > 0.0f && peak <= 3.4e38f) {
      int power;
      (void)frexpf(peak, &power);  // peak in [2^(power-1), 2^power)
      e = min(max(15 - power, -126), 126);
    }
    const float up = __builtin_bit_cast(float, (uint32_t)(e + 127) << 23);
    if (own && g == 0) sc[u * kCols + m] = __builtin_bit_cast(float, (uint32_t)(127 - e) << 23);
    half8_t hi, lo;
    constexpr int kOrder[8] = {0, 4, 1, 5, 2, 6, 3, 7};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float s = v[kOrder[j]] * up;
      const _Float16 h = (_Float16)s;
      hi[j] = h;
      lo[j] = (_Float16)(s - (float)h);
    }
    if (own) {
      if (WIDE) {
        bt[((u * 4 + g) * 2 + 0) * 16 + m] = __builtin_bit_cast(uint4_t, hi);
        bt[((u * 4 + g) * 2 + 1) * 16 + m] = __builtin_bit_cast(uint4_t, lo);
      } else {
        bt[(u * 4 + g) * 16 + m] = __builtin_bit_cast(uint4_t, hi);
        bt[(u * 4 + g) * 16 + m + 8] = __builtin_bit_cast(uint4_t, lo);
      }
    }
  }
  // Gains stored [unit][row]: here only without VEC (every thread over the
  // whole block, before the barrier).
  if (!VEC) {
    for (int i = tid; i < CU * rows_b; i += 256) {
      const int rr = i / CU;
      const int u = i - rr * CU;
      const int row = min(row_b0 + rr, a.N - 1);
      gs[u * pitch + rr] =
          a.gains[(size_t)row * (size_t)a.gain_stride + ((unsigned)(unit_c0 + u) >> a.group_shift)];
    }
  }

  __syncthreads();
  // VEC: the wave's own gain slice, written and then read by this wave only
  // (LDS operations of one wave complete in order).
  if (VEC) {
#pragma unroll
    for (int k = 0; k < kRunsPerLane; ++k) {
      const int i = lane + 64 * k;
      if ((i >> 4) < NG) {
        const int rr = 16 * t + (i & 15);
        const int u = u_w0 + 4 * (i >> 4);
        gs[(u + 0) * pitch + rr] = gv[k].x;
        gs[(u + 1) * pitch + rr] = gv[k].y;
        gs[(u + 2) * pitch + rr] = gv[k].z;
        gs[(u + 3) * pitch + rr] = gv[k].w;
      }
    }
  }

  const uint32_t exp16 = 0x4C004C00u;
  const _Float16 lift = (_Float16)(16.0f + a.code_bias);
  const half2_t shift = half2_t{lift, lift};
  // narrow: lanes r and r - 8 hold one lane's high and low columns, one scale
  const int m_col = WIDE ? r : (r & 7);
  float4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
  // A group is four units: its B tiles, gains and scales are read from LDS
  // one group ahead, its four products issue back to back, then the gains.
  // B tile of unit u for this lane (k-chunk q, column r): narrow one, WIDE
  // the high and the low parts.
  auto b_at = [&](int u, int term) { return WIDE ? bt[u * 128 + q * 32 + term * 16 + r] : bt[u * 64 + lane]; };
  const float *gbase = gs + 16 * t + 4 * q;
  uint4_t bq[2][4][kTerms];
  float4_t gq[2][4];
  float sq[2][4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int u = u_w0 + j;
#pragma unroll
    for (int e = 0; e < kTerms; ++e) bq[0][j][e] = b_at(u, e);
    gq[0][j] = *reinterpret_cast<const float4_t *>(gbase + u * pitch);
    sq[0][j] = sc[u * kCols + m_col];
  }
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    const int cur = g & 1;
    if (g + 1 < NG) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int u = u_w0 + 4 * (g + 1) + j;
#pragma unroll
        for (int e = 0; e < kTerms; ++e) bq[cur ^ 1][j][e] = b_at(u, e);
        gq[cur ^ 1][j] = *reinterpret_cast<const float4_t *>(gbase + u * pitch);
        sq[cur ^ 1][j] = sc[u * kCols + m_col];
      }
    }
    uint32_t d[4] = {w[g].x, w[g].y, w[g].z, w[g].w};
    lane_group_exchange(d[0], d[1], d[2], d[3]);
    float4_t D[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const half8_t c = codes_less_bias(d[j], exp16, shift);
      D[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(c, __builtin_bit_cast(half8_t, bq[cur][j][0]),
                                                    float4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
      if (WIDE)
        D[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(c, __builtin_bit_cast(half8_t, bq[cur][j][kTerms - 1]), D[j],
                                                      0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float s = sq[cur][j];
      acc.x = __builtin_fmaf(gq[cur][j].x * s, D[j].x, acc.x);
      acc.y = __builtin_fmaf(gq[cur][j].y * s, D[j].y, acc.y);
      acc.z = __builtin_fmaf(gq[cur][j].z * s, D[j].z, acc.z);
      acc.w = __builtin_fmaf(gq[cur][j].w * s, D[j].w, acc.w);
    }
  }
  // narrow: low columns into their high partners (lane r >= 8 holds lane
  // m = r - 8); WIDE: lane r holds lane m = r whole.
  if (!WIDE) {
    acc.x += dpp_move<0x118>(acc.x);
    acc.y += dpp_move<0x118>(acc.y);
    acc.z += dpp_move<0x118>(acc.z);
    acc.w += dpp_move<0x118>(acc.w);
  }
  const int m = WIDE ? r : r - 8;
  const bool owner = (WIDE || r >= 8) && m < a.M;
  float *dst;
  int dst_stride;
  if (gridDim.y > 1) {
    dst = a.out + (size_t)chunk * (size_t)a.M * (size_t)a.N;
    dst_stride = a.N;
  } else {
    dst = a.out;
    dst_stride = a.out_stride;
  }
  const int row0 = row_b0 + 16 * t + 4 * q;
  if (parts == 1) {
    if (owner) {
      float *o = dst + (size_t)m * (size_t)dst_stride;
      if (row0 + 0 < a.N) o[row0 + 0] = acc.x;
      if (row0 + 1 < a.N) o[row0 + 1] = acc.y;
      if (row0 + 2 < a.N) o[row0 + 2] = acc.z;
      if (row0 + 3 < a.N) o[row0 + 3] = acc.w;
    }
    return;
  }
  if (owner) {
    float *slot = red + ((part * RTB + t) * 16 + 4 * q) * kCols + m;
    slot[0] = acc.x;
    slot[kCols] = acc.y;
    slot[2 * kCols] = acc.z;
    slot[3 * kCols] = acc.w;
  }
  __syncthreads();
  if (part == 0 && owner) {
    float *o = dst + (size_t)m * (size_t)dst_stride;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float total = 0.0f;
      for (int k = 0; k < parts; ++k) total += red[((k * RTB + t) * 16 + 4 * q + i) * kCols + m];
      if (row0 + i < a.N) o[row0 + i] = total;
    }
  }
}

// Work split of the matrix-core form for `lanes` lanes of an N x K plane, or 0
// when the form does not apply (K not a multiple of 128, or more than 8 lanes).
struct GemvMfmaPlan {
  int tiles_per_block, chunk_units, chunks, groups_per_wave;
};

static int gemv_mfma_plan(int lanes, int N, int K, GemvMfmaPlan *plan) {
  if (lanes < 1 || lanes > 16 || K % 128 || N < 1) return 0;
  const int units = K / 32;
  const int groups = units / 4;
  const int tiles = (N + 15) / 16;
  if (units <= 64) {
    int rtb = 0;
    for (int c = 4; c >= 1; c /= 2)
      if ((tiles + c - 1) / c >= 256 && groups % (4 / c) == 0) { rtb = c; break; }
    if (!rtb)
      for (int c = 1; c <= 4; c *= 2)
        if (groups % (4 / c) == 0) { rtb = c; break; }
    plan->tiles_per_block = rtb;
    plan->chunk_units = units;
    plan->chunks = 1;
    plan->groups_per_wave = groups / (4 / rtb);
  } else {
    // The fewest chunks that give 256 workgroups, keeping two groups a wave.
    int kb = 0;
    for (int c = (units + 63) / 64; c <= groups; ++c) {
      if (groups % c || groups / c > 16) continue;
      kb = c;
      if ((tiles + 3) / 4 * c >= 256 || groups / c <= 2) break;
    }
    if (!kb) return 0;
    plan->tiles_per_block = 4;
    plan->chunk_units = units / kb;
    plan->chunks = kb;
    plan->groups_per_wave = groups / kb;
  }
  // past 8 lanes a wave holds twice the B tiles: more than 8 groups a wave
  // would spill, and such planes take launches of 8 lanes instead
  if (lanes > 8 && plan->groups_per_wave > 8) return 0;
  return plan->groups_per_wave >= 1 && plan->groups_per_wave <= 16;
}

// LDS of a launch: the B tiles (one or, past 8 lanes, two a k-chunk), the
// gains, the scales and the reduction across K-parts.
static size_t gemv_mfma_lds(const GemvMfmaPlan &p, int lanes) {
  const int rows_b = p.tiles_per_block * 16;
  const size_t cols = lanes > 8 ? 16 : 8;
  return (size_t)p.chunk_units * 1024 * (lanes > 8 ? 2 : 1) + (size_t)p.chunk_units * (rows_b + kMfmaGains) * 4 +
         (size_t)p.chunk_units * cols * 4 + (size_t)4 * 16 * cols * 4;
}

template <int NG, bool VEC, bool WIDE>
static hipError_t gemv_mfma_launch_form(const GemvMfmaArgs &a, const GemvMfmaPlan &p,
                                        hipStream_t stream) {
  const size_t lds = gemv_mfma_lds(p, a.M);
  static size_t lds_granted = 65536;  // launches above 64 KiB ask once
  if (lds > lds_granted) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemv_q4_mfma_kernel<NG, VEC, WIDE>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    lds_granted = lds;
  }
  const int tiles = (a.N + 15) / 16;
  dim3 grid((tiles + p.tiles_per_block - 1) / p.tiles_per_block, p.chunks);
  hipLaunchKernelGGL((gemv_q4_mfma_kernel<NG, VEC, WIDE>), grid, dim3(256), lds, stream, a);
  return hipGetLastError();
}

template <int NG>
static hipError_t gemv_mfma_launch(const GemvMfmaArgs &a, const GemvMfmaPlan &p, hipStream_t stream) {
  const bool vec = a.act_vec && a.gain_vec;
  if (a.M > 8) {
    if (NG > 8) return hipErrorInvalidValue;  // the plan refuses it
    constexpr int kNG = NG > 8 ? 8 : NG;
    return vec ? gemv_mfma_launch_form<kNG, true, true>(a, p, stream)
               : gemv_mfma_launch_form<kNG, false, true>(a, p, stream);
  }
  return vec ? gemv_mfma_launch_form<NG, true, false>(a, p, stream)
             : gemv_mfma_launch_form<NG, false, false>(a, p, stream);
}

static hipError_t gemv_mfma_dispatch(const GemvMfmaArgs &a, const GemvMfmaPlan &p, hipStream_t stream) {
  switch (p.groups_per_wave) {
    case 1: return gemv_mfma_launch<1>(a, p, stream);
    case 2: return gemv_mfma_launch<2>(a, p, stream);
    case 3: return gemv_mfma_launch<3>(a, p, stream);
    case 4: return gemv_mfma_launch<4>(a, p, stream);
    case 5: return gemv_mfma_launch<5>(a, p, stream);
    case 6: return gemv_mfma_launch<6>(a, p, stream);
    case 7: return gemv_mfma_launch<7>(a, p, stream);
    case 8: return gemv_mfma_launch<8>(a, p, stream);
    case 9: return gemv_mfma_launch<9>(a, p, stream);
    case 10: return gemv_mfma_launch<10>(a, p, stream);
    case 11: return gemv_mfma_launch<11>(a, p, stream);
    case 12: return gemv_mfma_launch<12>(a, p, stream);
    case 13: return gemv_mfma_launch<13>(a, p, stream);
    case 14: return gemv_mfma_launch<14>(a, p, stream);
    case 15: return gemv_mfma_launch<15>(a, p, stream);
    case 16: return gemv_mfma_launch<16>(a, p, stream);
    default: return hipErrorInvalidValue;
  }
}

// ---- planes with zero points -----------------------------------------------
//
// An asymmetric plane carries a zero point a row and group (plane_bind_part's
// weight_zero_point, unpacked by zero_read, app_core.c:7855-7866, 8053-8063).
// It is multiplied in kern_row_code's own form (app_core.c:3688-3706): for
// each group of a row,
//     y += gain * (dot - (code_bias + zero) * sum),
// dot = sum x_k (c_k ^ flip) over the group's codes and sum = sum x_k, in fp32.
// A wave takes one row; its lanes take the row's 32-code units in turn (a
// group of 32 2^s codes closes as its 2^s units, each on the group's gain and
// zero: the same terms, associated differently) and their partials meet in
// DPP sums.  A plain fp32 form: zero points are a storage format of the
// compressed-tensors export, not of the shipped Gemma one, and this kernel
// does not carry a headline workload.
struct GemvZeroArgs {
  const uint8_t *codes;
  long long row_stride;
  const float *gains;     // [N][gain_stride]
  const int8_t *zeros;    // [N][gain_stride]
  int gain_stride;
  int group_shift;
  int code_bias;
  uint32_t code_flip;
  const float *act;       // 16-byte aligned, act_stride % 4 == 0
  int act_stride;
  int lanes;              // <= M: lanes past it reread the last one and are not stored
  float *out;
  int out_stride;
  int N, K;
};

template <int BITS, int M>
__global__ __launch_bounds__(kGemvThreads) void gemv_zero_kernel(GemvZeroArgs a) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * (kGemvThreads / 64) + (threadIdx.x >> 6);
  if (row >= a.N) return;  // a whole wave
  const int units = a.K >> 5;
  const uint8_t *crow = a.codes + (size_t)row * (size_t)a.row_stride;
  float acc[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = 0.0f;
  for (int u = lane; u < units; u += 64) {
    uint32_t w[BITS];
#pragma unroll
    for (int i = 0; i < BITS; ++i) w[i] = reinterpret_cast<const uint32_t *>(crow + (size_t)u * BITS * 4)[i];
    const size_t slot = (size_t)row * (size_t)a.gain_stride + ((unsigned)u >> a.group_shift);
    const float gain = a.gains[slot];
    const float bias = (float)(a.code_bias + (int)a.zeros[slot]);
    float c[32];
#pragma unroll
    for (int k = 0; k < 32; ++k)
      c[k] = (float)(((w[(k * BITS) >> 5] >> ((k * BITS) & 31)) & ((1u << BITS) - 1u)) ^ a.code_flip);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float4_t *x = reinterpret_cast<const float4_t *>(a.act + (size_t)min(m, a.lanes - 1) * a.act_stride +
                                                             32 * (size_t)u);
      float dot = 0.0f, sum = 0.0f;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const float4_t v = x[q];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          dot = __builtin_fmaf(v[e], c[4 * q + e], dot);
          sum += v[e];
        }
      }
      acc[m] = __builtin_fmaf(gain, __builtin_fmaf(-bias, sum, dot), acc[m]);
    }
  }
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const float v = wave_sum_to_last(acc[m]);
    if (lane == 63 && m < a.lanes) a.out[(size_t)m * a.out_stride + row] = v;
  }
}

template <int BITS>
static hipError_t gemv_zero_launch_bits(const GemvZeroArgs &a, hipStream_t stream) {
  const dim3 grid((a.N + kGemvThreads / 64 - 1) / (kGemvThreads / 64));
  if (a.lanes <= 1)
    hipLaunchKernelGGL((gemv_zero_kernel<BITS, 1>), grid, dim3(kGemvThreads), 0, stream, a);
  else if (a.lanes <= 2)
    hipLaunchKernelGGL((gemv_zero_kernel<BITS, 2>), grid, dim3(kGemvThreads), 0, stream, a);
  else if (a.lanes <= 4)
    hipLaunchKernelGGL((gemv_zero_kernel<BITS, 4>), grid, dim3(kGemvThreads), 0, stream, a);
  else
    hipLaunchKernelGGL((gemv_zero_kernel<BITS, 8>), grid, dim3(kGemvThreads), 0, stream, a);
  return hipGetLastError();
}

template <int M, int R, int UPL, int GPT, bool LR>
static hipError_t gemv_dot_launch_rows(const GemvArgs &a, hipStream_t stream) {
  const int tiles = (a.N + R - 1) / R;
  const int tiles_per_block = 4 / a.ksplit;
  dim3 grid((tiles + tiles_per_block - 1) / tiles_per_block, LR ? a.lane_rows : 1);
  const size_t lds = gemv_dot_lds_bytes(M, a.K >> 5);
  static size_t lds_granted = 65536;  // launches above 64 KiB ask once
  if (lds > lds_granted) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemv_q4_dot_kernel<M, R, UPL, GPT, LR>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    lds_granted = lds;
  }
  hipLaunchKernelGGL((gemv_q4_dot_kernel<M, R, UPL, GPT, LR>), grid, dim3(kGemvThreads), lds, stream, a);
  return hipGetLastError();
}

template <int M, int R, int UPL, int GPT>
static hipError_t gemv_dot_launch_gpt(const GemvArgs &a, hipStream_t stream) {
  if constexpr (M == 1)
    if (a.lane_rows > 1) return gemv_dot_launch_rows<M, R, UPL, GPT, true>(a, stream);
  return gemv_dot_launch_rows<M, R, UPL, GPT, false>(a, stream);
}

// Items a thread stages: M K / 8 groups over 256 threads, at most 8 (12 for
// two lanes).
constexpr int kDotMaxItems = 8;

// The integer-dot form with 16-byte aligned activations and M K <= 16384 (a
// thread stages at most eight groups of eight), or two lanes up to K 12288
// (twelve); `a.ksplit` a power of two.
template <int M, int R, int UPL>
static hipError_t gemv_dot_launch(GemvArgs a, hipStream_t stream) {
  const int items = (M * (a.K >> 3) + kGemvThreads - 1) / kGemvThreads;
  if (!a.act_vec) return hipErrorInvalidValue;
  a.ks_log = a.ksplit == 1 ? 0 : a.ksplit == 2 ? 1 : a.ksplit == 4 ? 2 : -1;
  if (a.ks_log < 0) return hipErrorInvalidValue;
  // every unit of K has a lane: the row tile's waves times UPL units a lane
  if (a.ksplit * kWave * UPL < (a.K >> 5)) return hipErrorInvalidValue;
  if (items <= 1) return gemv_dot_launch_gpt<M, R, UPL, 1>(a, stream);
  if (items <= 2) return gemv_dot_launch_gpt<M, R, UPL, 2>(a, stream);
  if (items <= 4) return gemv_dot_launch_gpt<M, R, UPL, 4>(a, stream);
  if (items <= kDotMaxItems) return gemv_dot_launch_gpt<M, R, UPL, kDotMaxItems>(a, stream);
  if constexpr (M == 2)
    if (items <= 12) return gemv_dot_launch_gpt<M, R, UPL, 12>(a, stream);
  return hipErrorInvalidValue;
}

template <int M, int R, int UPL>
static hipError_t gemv_reg_launch(const GemvArgs &a, hipStream_t stream) {
  const int tiles = (a.N + R - 1) / R;
  const int tiles_per_block = 4 / a.ksplit;
  dim3 grid((tiles + tiles_per_block - 1) / tiles_per_block);
  hipLaunchKernelGGL((gemv_q4_reg_kernel<M, R, UPL>), grid, dim3(kGemvThreads), 0, stream, a);
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

// One to eight activation rows (lanes) against `segments` planes of the same
// width and group size (see gemv_q4_group_kernel for the modes; lane l of
// act, out[s], mul and the prologue's vectors lies l act_stride, l
// out_stride[s], l mul_stride, l lane_stride floats in).  Every plane but the
// last of a GEMV_SEGMENTS launch has a multiple of four rows; a
// GEMV_GELU_PAIR launch takes two planes of equal rows.  K / 32 must fit the
// waves of a row tile (K <= 8192).
extern "C" hipError_t igl_launch_gemv_group(int mode, int lanes, int segments, const uint8_t *const *codes,
                                            const long long *row_stride,
                                            const float *const *gains, const int *gain_stride,
                                            const int *rows, float *const *out, const int *out_stride,
                                            int group_shift, int code_bias, const float *act,
                                            int act_stride, int K, const float *mul, int mul_stride,
                                            const igl_gemv_prologue *pro, hipStream_t stream) {
  GemvGroupArgs a{};
  const int units = K / 32;
  if (lanes < 1 || lanes > 8 || segments < 1 || segments > 3 || K % 32 || units > 4 * kWave ||
      group_shift < 0)
    return hipErrorInvalidValue;
  // lanes past the first: their strides keep them apart
  if (lanes > 1 && (pro ? pro->lane_stride < K : act_stride < K)) return hipErrorInvalidValue;
  a.lane_rows = lanes;
  a.lane_stride = pro && lanes > 1 ? pro->lane_stride : 0;
  a.act_stride = lanes > 1 ? act_stride : 0;
  a.mul_stride = lanes > 1 ? mul_stride : 0;
  if (pro && (K > 4096 || !pro->state_in || (pro->lift && (!pro->state_out || !pro->lift_gain ||
                                                            pro->state_out == pro->state_in))))
    return hipErrorInvalidValue;
  a.state_in = pro ? pro->state_in : nullptr;
  a.state_out = pro ? pro->state_out : nullptr;
  a.lift = pro ? pro->lift : nullptr;
  a.lift_gain = pro ? pro->lift_gain : nullptr;
  a.scale = pro ? pro->scale : 1.0f;
  a.apply_scale = pro ? pro->apply_scale : 0;
  a.norm_gain = pro ? pro->norm_gain : nullptr;
  a.eps = pro ? pro->eps : 0.0f;
  a.pro_vec = 0;
  if ((mode == GEMV_GELU_PAIR && (segments != 2 || rows[0] != rows[1])) ||
      (mode == GEMV_GELU_MUL && (segments != 1 || !mul)))
    return hipErrorInvalidValue;
  int total = 0;
  for (int s = 0; s < 3; ++s) {
    const int live = s < segments;
    if (live && (rows[s] < 1 || (mode == GEMV_SEGMENTS && s + 1 < segments && rows[s] % 4)))
      return hipErrorInvalidValue;
    a.codes[s] = live ? codes[s] : nullptr;
    a.row_stride[s] = live ? row_stride[s] : 0;
    a.gains[s] = live ? gains[s] : nullptr;
    a.gain_stride[s] = live ? gain_stride[s] : 0;
    a.rows[s] = live ? rows[s] : 0;
    a.out[s] = live ? out[s] : nullptr;
    // lanes of one plane's output must not overlap (GEMV_GELU_PAIR writes out[0] only)
    if (live && lanes > 1 && (mode != GEMV_GELU_PAIR || s == 0) && out_stride[s] < rows[s])
      return hipErrorInvalidValue;
    a.out_stride[s] = live && lanes > 1 ? out_stride[s] : 0;
    total += a.rows[s];
  }
  a.segments = segments;
  a.tiles = mode == GEMV_GELU_PAIR ? (rows[0] + 1) / 2 : (total + 3) / 4;
  a.group_shift = group_shift;
  a.act = act;
  a.act_vec = ((((uintptr_t)act) & 15u) == 0 && (a.act_stride & 3) == 0) ? 1 : 0;
  a.K = K;
  a.unit_bias = 16.0f + (float)code_bias;
  a.mul = mul;
  if (mode == GEMV_GELU_MUL && lanes > 1 && mul_stride < rows[0]) return hipErrorInvalidValue;
  int ksplit = 1;
  while (ksplit < 4 && (units > ksplit * kWave || (a.tiles * ksplit < 2048 && units / (ksplit * 2) >= 32)))
    ksplit *= 2;
  // Few tiles (the per-layer-input gate's 64): four waves on each tile, a
  // workgroup a tile, so more workgroups share the launch's chains (lab, K
  // 1536 with the prologue: 4.70 -> 4.24 us; at 640 tiles it is slower).
  if (a.tiles * 4 <= 256 && units >= 16) ksplit = 4;
  a.ksplit = ksplit;
  // The prologue loads its K-vectors 16 bytes at a time where all are aligned.
  const bool vec16 = pro && ((((uintptr_t)pro->state_in) | (uintptr_t)(pro->lift ? pro->lift : pro->state_in) |
                              (uintptr_t)(pro->lift_gain ? pro->lift_gain : pro->state_in) |
                              (uintptr_t)(pro->norm_gain ? pro->norm_gain : pro->state_in) |
                              (uintptr_t)(pro->state_out ? pro->state_out : pro->state_in) |
                              (uintptr_t)a.lane_stride * sizeof(float)) & 15u) == 0;
  a.pro_vec = vec16 ? 1 : 0;
  // With the prologue, each workgroup repeats the residual update (four
  // K-vectors read, two block sums): past four workgroups a CU, two tiles a
  // wave halve that (measured: the 2 x 12288-row gate/up pair at K 1536, 11.5
  // -> 9.7 us; at 6144 rows, and without the prologue, one tile is faster).
  const int tpw = pro && ksplit == 1 && (a.tiles + 3) / 4 >= 1024 ? 2 : 1;
  const int tiles_per_block = 4 / ksplit * tpw;
  dim3 grid((a.tiles + tiles_per_block - 1) / tiles_per_block, lanes);
  const size_t lds = gemv_dot_lds_bytes(1, units);  // at most 29 KiB (K <= 8192)
  // eight-element groups of x a thread stages without a prologue
  const int gpt = K <= 2048 ? 1 : K <= 4096 ? 2 : 4;
#define IGL_GROUP_KS(M_, P_, G_)                                                                    \
  do {                                                                                              \
    if (ksplit == 1 && tpw == 2 && P_ != 0)                                                         \
      hipLaunchKernelGGL((gemv_q4_group_kernel<M_, P_, G_, 1, 2>), grid, dim3(kGemvThreads), lds, stream, a); \
    else if (ksplit == 1)                                                                           \
      hipLaunchKernelGGL((gemv_q4_group_kernel<M_, P_, G_, 1, 1>), grid, dim3(kGemvThreads), lds, stream, a); \
    else if (ksplit == 2)                                                                           \
      hipLaunchKernelGGL((gemv_q4_group_kernel<M_, P_, G_, 2, 1>), grid, dim3(kGemvThreads), lds, stream, a); \
    else                                                                                            \
      hipLaunchKernelGGL((gemv_q4_group_kernel<M_, P_, G_, 4, 1>), grid, dim3(kGemvThreads), lds, stream, a); \
  } while (0)
#define IGL_GROUP_LAUNCH(M_, P_)                                  \
  do {                                                            \
    if (P_ != 0 || gpt == 1) IGL_GROUP_KS(M_, P_, 1);             \
    else if (gpt == 2) IGL_GROUP_KS(M_, P_, 2);                   \
    else IGL_GROUP_KS(M_, P_, 4);                                 \
  } while (0)
  // groups of eight the prologue holds a thread: 1 up to K 2048, 2 up to 4096
  const int held = !pro ? 0 : K <= 2048 ? 1 : K <= 4096 ? 2 : -1;
  if (held < 0) return hipErrorInvalidValue;
  switch (mode * 3 + held) {
    case 0: IGL_GROUP_LAUNCH(GEMV_SEGMENTS, 0); break;
    case 1: IGL_GROUP_LAUNCH(GEMV_SEGMENTS, 1); break;
    case 2: IGL_GROUP_LAUNCH(GEMV_SEGMENTS, 2); break;
    case 3: IGL_GROUP_LAUNCH(GEMV_GELU_PAIR, 0); break;
    case 4: IGL_GROUP_LAUNCH(GEMV_GELU_PAIR, 1); break;
    case 5: IGL_GROUP_LAUNCH(GEMV_GELU_PAIR, 2); break;
    case 6: IGL_GROUP_LAUNCH(GEMV_GELU_MUL, 0); break;
    case 7: IGL_GROUP_LAUNCH(GEMV_GELU_MUL, 1); break;
    case 8: IGL_GROUP_LAUNCH(GEMV_GELU_MUL, 2); break;
    default: return hipErrorInvalidValue;
  }
#undef IGL_GROUP_LAUNCH
#undef IGL_GROUP_KS
  return hipGetLastError();
}

// ---- every code width: gemv_code_dot_kernel --------------------------------

namespace igl {

// Lanes a launch of the every-width form carries (template M).
static int code_launch_lanes(int lanes) { return lanes <= 2 ? lanes : 4; }

// Columns of one K-chunk: a multiple of 128 with M cols <= 16384 (eight
// staged groups a thread) and at most 512 slots a row.
static int code_chunk_cols(int bits, int M, int K) {
  int most = (16384 / M < 65536 / bits ? 16384 / M : 65536 / bits) / 128 * 128;
  const int chunks = (K + most - 1) / most;
  const int per = (K + chunks - 1) / chunks;
  return (per + 127) / 128 * 128;
}

// Workgroups a tiled launch keeps: eight a CU.
constexpr int kCodeTiledBlocks = 2048;

template <int BITS, int M, int UPL, int GPT>
static hipError_t gemv_code_launch4(const GemvCodeArgs &a, dim3 grid, size_t lds, hipStream_t stream) {
  // the tiled walk only for one lane and one slot a lane (tall decode planes)
  if constexpr (M == 1 && UPL == 1) {
    if (a.tile_iters > 1) {
      hipLaunchKernelGGL((gemv_code_dot_kernel<BITS, M, 4, UPL, GPT, true>), grid, dim3(kGemvThreads), lds,
                         stream, a);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((gemv_code_dot_kernel<BITS, M, 4, UPL, GPT, false>), grid, dim3(kGemvThreads), lds, stream,
                     a);
  return hipGetLastError();
}

template <int BITS, int M>
static hipError_t gemv_code_launch_m(const GemvCodeArgs &a, int upl, int gpt, dim3 grid, size_t lds,
                                     hipStream_t stream) {
  // more than 256 slots a row happen only for one lane of 4- or 8-bit codes and
  // two lanes of 8-bit codes (code_chunk_cols)
  constexpr bool kTwoSlots = (M == 1 && BITS >= 4) || (M == 2 && BITS == 8);
  if (upl == 1 || !kTwoSlots) {
    if (upl != 1) return hipErrorInvalidValue;
    switch (gpt) {
      case 1: return gemv_code_launch4<BITS, M, 1, 1>(a, grid, lds, stream);
      case 2: return gemv_code_launch4<BITS, M, 1, 2>(a, grid, lds, stream);
      case 4: return gemv_code_launch4<BITS, M, 1, 4>(a, grid, lds, stream);
      default: return gemv_code_launch4<BITS, M, 1, 8>(a, grid, lds, stream);
    }
  }
  if constexpr (kTwoSlots) {
    switch (gpt) {
      case 1: return gemv_code_launch4<BITS, M, 2, 1>(a, grid, lds, stream);
      case 2: return gemv_code_launch4<BITS, M, 2, 2>(a, grid, lds, stream);
      case 4: return gemv_code_launch4<BITS, M, 2, 4>(a, grid, lds, stream);
      default: return gemv_code_launch4<BITS, M, 2, 8>(a, grid, lds, stream);
    }
  }
  return hipErrorInvalidValue;
}

template <int BITS>
static hipError_t gemv_code_launch_bits(const GemvCodeArgs &a, int M, int upl, int gpt, dim3 grid,
                                        size_t lds, hipStream_t stream) {
  switch (M) {
    case 1: return gemv_code_launch_m<BITS, 1>(a, upl, gpt, grid, lds, stream);
    case 2: return gemv_code_launch_m<BITS, 2>(a, upl, gpt, grid, lds, stream);
    default: return gemv_code_launch_m<BITS, 4>(a, upl, gpt, grid, lds, stream);
  }
}

}  // namespace igl

extern "C" size_t igl_gemv_code_part_floats(int bit_count, int lanes, int N, int K) {
  size_t most = 0;
  for (int l = 1; l <= (lanes < 4 ? lanes : 4); ++l) {
    const int M = code_launch_lanes(l);
    const int cols = code_chunk_cols(bit_count, M, K);
    const size_t chunks = (size_t)((K + cols - 1) / cols);
    const size_t need = chunks > 1 ? chunks * (size_t)l * (size_t)N : 0;
    if (need > most) most = need;
  }
  return most;
}

// y = W x for any number of lanes over a 2, 4 or 8-bit code plane, four
// lanes a launch.  Activations 16-byte aligned with act_stride % 4 == 0;
// `part` holds igl_gemv_code_part_floats(bits, lanes, N, K) floats.
extern "C" hipError_t igl_launch_gemv_codes(const igl_code_view *v, const float *act, int act_stride,
                                            int lanes, float *out, int out_stride, int N, int K,
                                            float *part, hipStream_t stream) {
  const int bits = v->bit_count;
  if ((bits != 2 && bits != 4 && bits != 8) || K % 32 || (((uintptr_t)act) & 15u) ||
      (lanes > 1 && (act_stride & 3)))
    return hipErrorInvalidValue;
  GemvCodeArgs a;
  a.codes = v->codes;
  a.row_stride = v->row_stride;
  a.gains = v->gains;
  a.gain_stride = v->gain_stride;
  a.group_shift = v->group_shift;
  a.N = N;
  a.K = K;
  a.code_bias = v->code_bias;
  const uint32_t field = bits == 2 ? (uint32_t)(v->code_flip & 3)
                                   : (uint32_t)((v->code_flip ^ v->code_bias) & ((1 << bits) - 1));
  a.code_xor = field * (bits == 2 ? 0x55555555u : bits == 4 ? 0x11111111u : 0x01010101u);
  for (int done = 0; done < lanes; done += 4) {
    const int l = lanes - done < 4 ? lanes - done : 4;
    const int M = code_launch_lanes(l);
    const int cols = code_chunk_cols(bits, M, K);
    const int chunks = (K + cols - 1) / cols;
    const int slots = (cols * bits + 127) / 128;
    const int upl = slots > 4 * kWave ? 2 : 1;
    // short rows: sub-waves of 16 or 32 lanes, each over its own rows
    const int subs_log = upl == 1 && slots <= 16 ? 2 : upl == 1 && slots <= 32 ? 1 : 0;
    const int tiles = (N + (4 << subs_log) - 1) / (4 << subs_log);
    int ksplit = 1;
    while (subs_log == 0 && ksplit < 4 &&
           (slots > ksplit * kWave * upl || (tiles * ksplit * chunks < 2048 && slots / (ksplit * 2) >= 32 * upl)))
      ksplit *= 2;
    const int items = (M * (cols >> 3) + kGemvThreads - 1) / kGemvThreads;
    const int gpt = items <= 1 ? 1 : items <= 2 ? 2 : items <= 4 ? 4 : 8;
    a.act = act + (size_t)done * (size_t)act_stride;
    a.act_stride = act_stride;
    a.lanes = l;
    a.chunk_cols = cols;
    a.ks_log = ksplit == 1 ? 0 : ksplit == 2 ? 1 : 2;
    a.subs_log = subs_log;
    if (chunks > 1) {
      if (!part) return hipErrorInvalidValue;
      a.out = part;
      a.out_stride = N;
    } else {
      a.out = out + (size_t)done * (size_t)out_stride;
      a.out_stride = out_stride;
    }
    const int per_block = 4 / ksplit;
    const int blocks = (tiles + per_block - 1) / per_block;
    // a tall one-lane plane: fewer workgroups, each walking several row tiles
    // after one staging of x
    const bool tiled = M == 1 && upl == 1 && ksplit == 1 && chunks == 1 && blocks > kCodeTiledBlocks;
    a.tile_iters = tiled ? (blocks + kCodeTiledBlocks - 1) / kCodeTiledBlocks : 1;
    const dim3 grid(tiled ? kCodeTiledBlocks : blocks, chunks);
    const size_t lds = gemv_code_lds_bytes(M, cols / 32);
    hipError_t e = bits == 2   ? gemv_code_launch_bits<2>(a, M, upl, gpt, grid, lds, stream)
                   : bits == 4 ? gemv_code_launch_bits<4>(a, M, upl, gpt, grid, lds, stream)
                               : gemv_code_launch_bits<8>(a, M, upl, gpt, grid, lds, stream);
    if (e != hipSuccess) return e;
    if (chunks > 1) {
      const int total = l * N;
      hipLaunchKernelGGL(gemv_chunk_sum_kernel, dim3((total + 255) / 256), dim3(256), 0, stream, part,
                         chunks, l, N, out + (size_t)done * (size_t)out_stride, out_stride);
      if ((e = hipGetLastError()) != hipSuccess) return e;
    }
  }
  return hipSuccess;
}

// ---- calibrated planes: gemv_level_kernel ----------------------------------

namespace igl {

template <int BITS, int M, int UPL, int GPT>
static hipError_t gemv_level_launch4(const GemvLevelArgs &a, dim3 grid, size_t lds, hipStream_t stream,
                                     int rows) {
  // one lane: two-row tiles, twice the workgroups (the export-kinds decode
  // measured 2.52 against 2.68 ms a token with four); six on wide rows
  if constexpr (M == 1) {
    if (rows == 6) {
      hipLaunchKernelGGL((gemv_level_kernel<BITS, 1, 6, UPL, GPT>), grid, dim3(kGemvThreads), lds, stream, a);
      return hipGetLastError();
    }
    if (a.state_in) {
      hipLaunchKernelGGL((gemv_level_kernel<BITS, 1, 2, UPL, GPT, true>), grid, dim3(kGemvThreads), lds, stream, a);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((gemv_level_kernel<BITS, M, (M == 1 ? 2 : 4), UPL, GPT>), grid, dim3(kGemvThreads), lds, stream,
                     a);
  return hipGetLastError();
}

template <int BITS, int M>
static hipError_t gemv_level_launch_m(const GemvLevelArgs &a, int upl, int gpt, dim3 grid, size_t lds,
                                      hipStream_t stream, int rows) {
  // more than 256 slots a row: one lane of 4-bit codes, one or two of 8-bit codes
  constexpr bool kTwoSlots = (M == 1 && BITS >= 4) || (M == 2 && BITS == 8);
  if (upl == 1) {
    switch (gpt) {
      case 1: return gemv_level_launch4<BITS, M, 1, 1>(a, grid, lds, stream, rows);
      case 2: return gemv_level_launch4<BITS, M, 1, 2>(a, grid, lds, stream, rows);
      case 4: return gemv_level_launch4<BITS, M, 1, 4>(a, grid, lds, stream, rows);
      default: return gemv_level_launch4<BITS, M, 1, 8>(a, grid, lds, stream, rows);
    }
  }
  if constexpr (kTwoSlots) {
    switch (gpt) {
      case 1: return gemv_level_launch4<BITS, M, 2, 1>(a, grid, lds, stream, rows);
      case 2: return gemv_level_launch4<BITS, M, 2, 2>(a, grid, lds, stream, rows);
      case 4: return gemv_level_launch4<BITS, M, 2, 4>(a, grid, lds, stream, rows);
      default: return gemv_level_launch4<BITS, M, 2, 8>(a, grid, lds, stream, rows);
    }
  }
  return hipErrorInvalidValue;
}

template <int BITS>
static hipError_t gemv_level_launch_bits(const GemvLevelArgs &a, int M, int upl, int gpt, dim3 grid,
                                         size_t lds, hipStream_t stream, int rows) {
  switch (M) {
    case 1: return gemv_level_launch_m<BITS, 1>(a, upl, gpt, grid, lds, stream, rows);
    case 2: return gemv_level_launch_m<BITS, 2>(a, upl, gpt, grid, lds, stream, rows);
    default: return gemv_level_launch_m<BITS, 4>(a, upl, gpt, grid, lds, stream, rows);
  }
}

}  // namespace igl

static hipError_t igl_level_launch(GemvLevelArgs a, const igl_code_view *v, float step, float leave,
                                   const float *act, int act_stride, int lanes, float *out,
                                   int out_stride, int N, int K, int epi, const float *epi_in,
                                   int epi_stride, hipStream_t stream);

// Whether igl_launch_gemv_level takes this plane's shape.
extern "C" int igl_gemv_level_fits(int bit_count, int K) {
  return (bit_count == 2 || bit_count == 4 || bit_count == 8) && K >= 32 && K % 32 == 0 && K <= 16384 &&
         (K * bit_count + 127) / 128 <= 512;
}

// y = quant_step(W quant_step(x, step), leave) for any number of lanes of a
// 2, 4 or 8-bit code plane, on the activation grid (gemv_level_kernel).
// Activations 16-byte aligned with act_stride % 4 == 0; every condition is
// checked before anything is launched.
extern "C" hipError_t igl_launch_gemv_level(const igl_code_view *v, float step, float leave,
                                            const float *act, int act_stride, int lanes, float *out,
                                            int out_stride, int N, int K, hipStream_t stream) {
  return igl_launch_gemv_level_epi(v, step, leave, act, act_stride, lanes, out, out_stride, N, K,
                                   IGL_LEVEL_EPI_NONE, nullptr, 0, stream);
}

// The same, with the elementwise step that follows the product fused into its
// store (IGL_LEVEL_EPI_*; epi_in may be `out` itself: each output reads its
// own element first).
extern "C" hipError_t igl_launch_gemv_level_epi(const igl_code_view *v, float step, float leave,
                                                const float *act, int act_stride, int lanes, float *out,
                                                int out_stride, int N, int K, int epi, const float *epi_in,
                                                int epi_stride, hipStream_t stream) {
  GemvLevelArgs a;
  a.state_in = a.lift = a.lift_gain = a.norm_gain = nullptr;
  a.state_out = a.x_out = nullptr;
  a.scale = 1.0f;
  a.apply_scale = 0;
  a.eps = 0.0f;
  a.pro_vec = 0;
  return igl_level_launch(a, v, step, leave, act, act_stride, lanes, out, out_stride, N, K, epi, epi_in,
                          epi_stride, stream);
}

// One lane with the residual update of igl_launch_gemv_group as the
// prologue (`pro`: state_in, lift and its gain, scale, norm_gain, eps), x
// written to `x_out` as well where it is not NULL (the launches that read the
// same x next), K at most 2048.  y and the fused elementwise step as
// igl_launch_gemv_level_epi.
extern "C" hipError_t igl_launch_gemv_level_pro(const igl_code_view *v, float step, float leave,
                                                const igl_gemv_prologue *pro, float *x_out, float *out,
                                                int N, int K, int epi, const float *epi_in,
                                                hipStream_t stream) {
  if (!pro || !pro->state_in || K > 2048 || (pro->lift && (!pro->lift_gain || !pro->state_out)) ||
      pro->state_out == pro->state_in)
    return hipErrorInvalidValue;
  GemvLevelArgs a;
  a.state_in = pro->state_in;
  a.state_out = pro->state_out;
  a.lift = pro->lift;
  a.lift_gain = pro->lift_gain;
  a.scale = pro->scale;
  a.apply_scale = pro->apply_scale;
  a.norm_gain = pro->norm_gain;
  a.eps = pro->eps;
  a.x_out = x_out;
  a.pro_vec = ((((uintptr_t)a.state_in) | (uintptr_t)(a.lift ? a.lift : a.state_in) |
                (uintptr_t)(a.lift_gain ? a.lift_gain : a.state_in) |
                (uintptr_t)(a.norm_gain ? a.norm_gain : a.state_in) |
                (uintptr_t)(a.state_out ? a.state_out : a.state_in) |
                (uintptr_t)(x_out ? x_out : a.state_in)) & 15u) == 0;
  return igl_level_launch(a, v, step, leave, nullptr, K, 1, out, N, N, K, epi, epi_in, 0, stream);
}

// Rows a sub-wave of a pair launch (half of them the gate plane's): the
// export-kinds decode measured 1.54 ms a token with four, 1.57 with two and
// 1.59-1.60 with eight.
constexpr int kLevelPairRows = 4;

template <int BITS>
static hipError_t gemv_level_pair_launch(const GemvLevelArgs &a, dim3 grid, size_t lds, hipStream_t stream) {
  hipLaunchKernelGGL((gemv_level_kernel<BITS, 1, kLevelPairRows, 1, 1, true, kLevelPair>), grid, dim3(kGemvThreads),
                     lds, stream, a);
  return hipGetLastError();
}

template <int BITS>
static hipError_t gemv_level_segments_launch(const GemvLevelArgs &a, dim3 grid, size_t lds, hipStream_t stream) {
  hipLaunchKernelGGL((gemv_level_kernel<BITS, 1, 2, 1, 1, true, kLevelSegments>), grid, dim3(kGemvThreads), lds,
                     stream, a);
  return hipGetLastError();
}

// The residual update's prologue and its fields, shared by the fused level entries.
static void level_prologue_args(GemvLevelArgs &a, const igl_gemv_prologue *pro) {
  a.state_in = pro->state_in;
  a.state_out = pro->state_out;
  a.lift = pro->lift;
  a.lift_gain = pro->lift_gain;
  a.scale = pro->scale;
  a.apply_scale = pro->apply_scale;
  a.norm_gain = pro->norm_gain;
  a.eps = pro->eps;
  a.x_out = nullptr;
  a.pro_vec = ((((uintptr_t)a.state_in) | (uintptr_t)(a.lift ? a.lift : a.state_in) |
                (uintptr_t)(a.lift_gain ? a.lift_gain : a.state_in) |
                (uintptr_t)(a.norm_gain ? a.norm_gain : a.state_in) |
                (uintptr_t)(a.state_out ? a.state_out : a.state_in)) & 15u) == 0;
}

// Up to three calibrated planes of one lane that read the same input (a
// layer's q, k and v) in one launch, the residual update as the prologue:
// every plane the same kind and enter step, K <= 2048; plane s's rows into
// out[s] on its own leave grid.
extern "C" hipError_t igl_launch_gemv_level_segments(const igl_code_view *v, int segments, const int *rows,
                                                     float *const *out, const float *leave, float step,
                                                     const igl_gemv_prologue *pro, int K, hipStream_t stream) {
  if (!v || segments < 1 || segments > 3 || !rows || !out || !leave || !pro || !pro->state_in || K > 2048 ||
      !(step > 0.0f) || (pro->lift && (!pro->lift_gain || !pro->state_out)) || pro->state_out == pro->state_in)
    return hipErrorInvalidValue;
  const int bits = v[0].bit_count;
  if (!igl_gemv_level_fits(bits, K)) return hipErrorInvalidValue;
  int total = 0;
  for (int i = 0; i < segments; ++i) {
    if (rows[i] < 1 || !out[i] || v[i].bit_count != bits || v[i].code_bias != v[0].code_bias ||
        v[i].code_flip != v[0].code_flip || v[i].group_shift != v[0].group_shift)
      return hipErrorInvalidValue;
    total += rows[i];
  }
  GemvLevelArgs a{};
  level_prologue_args(a, pro);
  const int last = segments - 1;
  a.codes = v[0].codes;
  a.row_stride = v[0].row_stride;
  a.gains = v[0].gains;
  a.gain_stride = v[0].gain_stride;
  a.leave = leave[0];
  a.out = out[0];
  a.codes2 = v[min(1, last)].codes;
  a.row_stride2 = v[min(1, last)].row_stride;
  a.gains2 = v[min(1, last)].gains;
  a.gain_stride2 = v[min(1, last)].gain_stride;
  a.leave2 = leave[min(1, last)];
  a.out2 = out[min(1, last)];
  a.codes3 = v[last].codes;
  a.row_stride3 = v[last].row_stride;
  a.gains3 = v[last].gains;
  a.gain_stride3 = v[last].gain_stride;
  a.leave3 = leave[last];
  a.out3 = out[last];
  // planes past `segments` start past the last row
  a.first2 = segments > 1 ? rows[0] : total;
  a.first3 = segments > 2 ? rows[0] + rows[1] : total;
  a.group_shift = v[0].group_shift;
  a.act = nullptr;
  a.act_stride = K;
  a.out_stride = 0;
  a.lanes = 1;
  a.N = total;
  a.K = K;
  a.code_bias = v[0].code_bias;
  a.step = step;
  a.epi = IGL_LEVEL_EPI_NONE;
  const uint32_t field = bits == 8 ? (uint32_t)((v[0].code_flip ^ v[0].code_bias) & 255)
                                   : (uint32_t)(v[0].code_flip & ((1 << bits) - 1));
  a.code_xor = field * (bits == 2 ? 0x55555555u : bits == 4 ? 0x11111111u : 0x01010101u);
  const int slots = (K * bits + 127) / 128;
  if (slots > 4 * kWave) return hipErrorInvalidValue;
  const int subs_log = slots <= 16 ? 2 : slots <= 32 ? 1 : 0;
  const int tiles = (total + (2 << subs_log) - 1) / (2 << subs_log);
  int ksplit = 1;
  while (subs_log == 0 && ksplit < 4 &&
         (slots > ksplit * kWave || (tiles * ksplit < 2048 && slots / (ksplit * 2) >= 32)))
    ksplit *= 2;
  a.ks_log = ksplit == 1 ? 0 : ksplit == 2 ? 1 : 2;
  a.subs_log = subs_log;
  const int per_block = 4 / ksplit;
  const dim3 grid((tiles + per_block - 1) / per_block);
  const size_t lds = gemv_level_lds_bytes(1, K / 32);
  return bits == 2   ? gemv_level_segments_launch<2>(a, grid, lds, stream)
         : bits == 4 ? gemv_level_segments_launch<4>(a, grid, lds, stream)
                     : gemv_level_segments_launch<8>(a, grid, lds, stream);
}

// The gate and up projections of one lane in one launch (kern_gelu_gate's
// gelu(gate) * up into `out`), the residual update as the prologue: both
// planes the same kind, rows and enter step, K <= 2048.
extern "C" hipError_t igl_launch_gemv_level_pair(const igl_code_view *gate, const igl_code_view *up, float step,
                                                 float leave_gate, float leave_up, const igl_gemv_prologue *pro,
                                                 float *out, int N, int K, hipStream_t stream) {
  const int bits = gate ? gate->bit_count : 0;
  if (!gate || !up || !pro || !pro->state_in || !out || N < 1 || K > 2048 || !(step > 0.0f) ||
      !igl_gemv_level_fits(bits, K) || up->bit_count != bits || up->code_bias != gate->code_bias ||
      up->code_flip != gate->code_flip || up->group_shift != gate->group_shift ||
      (pro->lift && (!pro->lift_gain || !pro->state_out)) || pro->state_out == pro->state_in)
    return hipErrorInvalidValue;
  GemvLevelArgs a{};
  level_prologue_args(a, pro);
  a.codes = gate->codes;
  a.row_stride = gate->row_stride;
  a.gains = gate->gains;
  a.gain_stride = gate->gain_stride;
  a.codes2 = up->codes;
  a.row_stride2 = up->row_stride;
  a.gains2 = up->gains;
  a.gain_stride2 = up->gain_stride;
  a.group_shift = gate->group_shift;
  a.act = nullptr;
  a.act_stride = K;
  a.out = out;
  a.out_stride = N;
  a.lanes = 1;
  a.N = N;
  a.K = K;
  a.code_bias = gate->code_bias;
  a.step = step;
  a.leave = leave_gate;
  a.leave2 = leave_up;
  a.epi = IGL_LEVEL_EPI_NONE;
  a.epi_in = nullptr;
  a.epi_stride = 0;
  const uint32_t field = bits == 8 ? (uint32_t)((gate->code_flip ^ gate->code_bias) & 255)
                                   : (uint32_t)(gate->code_flip & ((1 << bits) - 1));
  a.code_xor = field * (bits == 2 ? 0x55555555u : bits == 4 ? 0x11111111u : 0x01010101u);
  const int slots = (K * bits + 127) / 128;
  if (slots > 4 * kWave) return hipErrorInvalidValue;
  const int subs_log = slots <= 16 ? 2 : slots <= 32 ? 1 : 0;
  const int rp = kLevelPairRows / 2;
  const int tiles = (N + (rp << subs_log) - 1) / (rp << subs_log);
  int ksplit = 1;
  while (subs_log == 0 && ksplit < 4 &&
         (slots > ksplit * kWave || (tiles * ksplit < 2048 && slots / (ksplit * 2) >= 32)))
    ksplit *= 2;
  a.ks_log = ksplit == 1 ? 0 : ksplit == 2 ? 1 : 2;
  a.subs_log = subs_log;
  const int per_block = 4 / ksplit;
  const dim3 grid((tiles + per_block - 1) / per_block);
  const size_t lds = gemv_level_lds_bytes(1, K / 32);
  return bits == 2   ? gemv_level_pair_launch<2>(a, grid, lds, stream)
         : bits == 4 ? gemv_level_pair_launch<4>(a, grid, lds, stream)
                     : gemv_level_pair_launch<8>(a, grid, lds, stream);
}

static hipError_t igl_level_launch(GemvLevelArgs a, const igl_code_view *v, float step, float leave,
                                   const float *act, int act_stride, int lanes, float *out,
                                   int out_stride, int N, int K, int epi, const float *epi_in,
                                   int epi_stride, hipStream_t stream) {
  const int bits = v->bit_count;
  // activations come from `act` (16-byte aligned) unless the prologue forms them
  if (!(step > 0.0f) || !igl_gemv_level_fits(bits, K) ||
      (!a.state_in && (!act || (((uintptr_t)act) & 15u))) || (lanes > 1 && (act_stride & 3)) ||
      lanes < 1 || N < 1 || epi < IGL_LEVEL_EPI_NONE || epi > IGL_LEVEL_EPI_GELU_MUL ||
      (epi != IGL_LEVEL_EPI_NONE && !epi_in))
    return hipErrorInvalidValue;
  a.epi = epi;
  a.epi_stride = epi_stride;
  a.codes = v->codes;
  a.row_stride = v->row_stride;
  a.gains = v->gains;
  a.gain_stride = v->gain_stride;
  a.group_shift = v->group_shift;
  a.N = N;
  a.K = K;
  a.code_bias = v->code_bias;
  a.step = step;
  a.leave = leave;
  const uint32_t field = bits == 8 ? (uint32_t)((v->code_flip ^ v->code_bias) & 255)
                                   : (uint32_t)(v->code_flip & ((1 << bits) - 1));
  a.code_xor = field * (bits == 2 ? 0x55555555u : bits == 4 ? 0x11111111u : 0x01010101u);
  // lanes a launch: M K <= 16384 (eight staged groups a thread), at most four
  const int most = 16384 / K >= 4 ? 4 : 16384 / K >= 2 ? 2 : 1;
  for (int done = 0; done < lanes; done += most) {
    const int l = lanes - done < most ? lanes - done : most;
    const int M = l <= 2 ? l : 4;
    const int slots = (K * bits + 127) / 128;
    int upl = slots > 4 * kWave ? 2 : 1;
    const int subs_log = upl == 1 && slots <= 16 ? 2 : upl == 1 && slots <= 32 ? 1 : 0;
    int rows_t = M == 1 ? 2 : 4;  // rows a sub-wave (the kernel's R)
    int tiles = (N + (rows_t << subs_log) - 1) / (rows_t << subs_log);
    int ksplit = 1;
    while (subs_log == 0 && ksplit < 4 &&
           (slots > ksplit * kWave * upl || (tiles * ksplit < 2048 && slots / (ksplit * 2) >= 32 * upl)))
      ksplit *= 2;
    // One lane on wide rows (four waves a tile, 192 slots and up): six-row
    // tiles where two give a CU several workgroups that each stage all of x
    // and six give every CU at most one (lab, 1536 rows: 2-bit K 12288 14.13
    // -> 10.34 us, 4-bit K 6144 8.08 -> 7.10 us; the same sums; at 128 slots,
    // 4-bit K 4096, the decode step measured it slower, 6.2 -> 7.6 us).
    if (M == 1 && subs_log == 0 && ksplit == 4 && slots >= 192 && !a.state_in && (N + 1) / 2 > 256 &&
        (N + 5) / 6 <= 256) {
      rows_t = 6;
      tiles = (N + 5) / 6;
    }
    // One lane on a small plane (under 4096 rows, at most 128 slots; two
    // slots a lane past 64, for the widths that have that form): one wave a
    // two-row tile, no K split -- the integer-dot form's rule for the same
    // shapes.
    if (M == 1 && subs_log == 0 && !a.state_in && N < 4096 &&
        (slots <= kWave || (bits >= 4 && slots <= 2 * kWave))) {
      upl = slots > kWave ? 2 : 1;
      ksplit = 1;
    }
    const int items = (M * (K >> 3) + kGemvThreads - 1) / kGemvThreads;
    const int gpt = items <= 1 ? 1 : items <= 2 ? 2 : items <= 4 ? 4 : 8;
    a.act = act ? act + (size_t)done * (size_t)act_stride : nullptr;
    a.act_stride = act_stride;
    a.lanes = l;
    a.out = out + (size_t)done * (size_t)out_stride;
    a.out_stride = out_stride;
    a.epi_in = epi_in ? epi_in + (size_t)done * (size_t)epi_stride : nullptr;
    a.ks_log = ksplit == 1 ? 0 : ksplit == 2 ? 1 : 2;
    a.subs_log = subs_log;
    const int per_block = 4 / ksplit;
    const dim3 grid((tiles + per_block - 1) / per_block);
    const size_t lds = gemv_level_lds_bytes(M, K / 32);
    hipError_t e = bits == 2   ? gemv_level_launch_bits<2>(a, M, upl, gpt, grid, lds, stream, rows_t)
                   : bits == 4 ? gemv_level_launch_bits<4>(a, M, upl, gpt, grid, lds, stream, rows_t)
                               : gemv_level_launch_bits<8>(a, M, upl, gpt, grid, lds, stream, rows_t);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// ---- real planes: gemv_real_kernel -----------------------------------------

namespace igl {

static int real_launch_lanes(int lanes) { return lanes <= 1 ? 1 : lanes <= 2 ? 2 : lanes <= 4 ? 4 : 8; }

// Columns of one K-chunk: a multiple of 64 with M cols floats <= 32 KiB.
static int real_chunk_cols(int M, int K) {
  const int most = 8192 / M;
  const int chunks = (K + most - 1) / most;
  const int per = (K + chunks - 1) / chunks;
  return (per + 63) / 64 * 64;
}

template <int TYPE>
static hipError_t gemv_real_launch_type(const GemvRealArgs &a, int M, dim3 grid, size_t lds,
                                        hipStream_t stream) {
  switch (M) {
    case 1: hipLaunchKernelGGL((gemv_real_kernel<TYPE, 1>), grid, dim3(kGemvThreads), lds, stream, a); break;
    case 2: hipLaunchKernelGGL((gemv_real_kernel<TYPE, 2>), grid, dim3(kGemvThreads), lds, stream, a); break;
    case 4: hipLaunchKernelGGL((gemv_real_kernel<TYPE, 4>), grid, dim3(kGemvThreads), lds, stream, a); break;
    default: hipLaunchKernelGGL((gemv_real_kernel<TYPE, 8>), grid, dim3(kGemvThreads), lds, stream, a); break;
  }
  return hipGetLastError();
}

}  // namespace igl

extern "C" size_t igl_gemv_real_part_floats(int lanes, int N, int K) {
  size_t most = 0;
  for (int l = 1; l <= (lanes < 8 ? lanes : 8); ++l) {
    const int cols = real_chunk_cols(real_launch_lanes(l), K);
    const size_t chunks = (size_t)((K + cols - 1) / cols);
    const size_t need = chunks > 1 ? chunks * (size_t)l * (size_t)N : 0;
    if (need > most) most = need;
  }
  return most;
}

// y = W x for any number of lanes over a real plane (F32, F16 or BF16 rows of
// K values, K % 8 == 0), eight lanes a launch.  Activations 16-byte aligned
// with act_stride % 4 == 0; `part` holds igl_gemv_real_part_floats floats.
extern "C" hipError_t igl_launch_gemv_real(const void *rows, int real_type, const float *act,
                                           int act_stride, int lanes, float *out, int out_stride,
                                           int N, int K, float *part, hipStream_t stream) {
  if ((real_type != IGL_STORE_F32 && real_type != IGL_STORE_F16 && real_type != IGL_STORE_BF16) ||
      K % 8 || N < 1 || (((uintptr_t)act) & 15u) || (((uintptr_t)rows) & 15u) ||
      (lanes > 1 && (act_stride & 3)))
    return hipErrorInvalidValue;
  GemvRealArgs a;
  a.rows = static_cast<const uint8_t *>(rows);
  a.row_bytes = (long long)K * (real_type == IGL_STORE_F32 ? 4 : 2);
  a.N = N;
  a.K = K;
  for (int done = 0; done < lanes; done += 8) {
    const int l = lanes - done < 8 ? lanes - done : 8;
    const int M = real_launch_lanes(l);
    const int cols = real_chunk_cols(M, K);
    const int chunks = (K + cols - 1) / cols;
    a.act = act + (size_t)done * (size_t)act_stride;
    a.act_stride = act_stride;
    a.lanes = l;
    a.chunk_cols = cols;
    if (chunks > 1) {
      if (!part) return hipErrorInvalidValue;
      a.out = part;
      a.out_stride = N;
    } else {
      a.out = out + (size_t)done * (size_t)out_stride;
      a.out_stride = out_stride;
    }
    const dim3 grid((N + 4 * kRealRows - 1) / (4 * kRealRows), chunks);
    const size_t lds = (size_t)M * (size_t)cols * sizeof(float);
    hipError_t e = real_type == IGL_STORE_F32    ? gemv_real_launch_type<IGL_STORE_F32>(a, M, grid, lds, stream)
                   : real_type == IGL_STORE_F16 ? gemv_real_launch_type<IGL_STORE_F16>(a, M, grid, lds, stream)
                                                : gemv_real_launch_type<IGL_STORE_BF16>(a, M, grid, lds, stream);
    if (e != hipSuccess) return e;
    if (chunks > 1) {
      const int total = l * N;
      hipLaunchKernelGGL(gemv_chunk_sum_kernel, dim3((total + 255) / 256), dim3(256), 0, stream, part,
                         chunks, l, N, out + (size_t)done * (size_t)out_stride, out_stride);
      if ((e = hipGetLastError()) != hipSuccess) return e;
    }
  }
  return hipSuccess;
}

// Floats of K-chunk partials a launch of `lanes` lanes over an N x K plane
// writes (0 when it needs none).
extern "C" size_t igl_gemv_part_floats(int lanes, int N, int K, int lds_limit) {
  GemvMfmaPlan plan;
  // past 8 lanes without the matrix-core form: launches of 8 lanes in turn
  if (lanes > 8 && !gemv_mfma_plan(lanes, N, K, &plan)) return igl_gemv_part_floats(8, N, K, lds_limit);
  if (lanes >= 3 && gemv_mfma_plan(lanes, N, K, &plan))
    return plan.chunks > 1 ? (size_t)plan.chunks * (size_t)lanes * (size_t)N : 0;
  if (lanes <= 2 && K / 32 <= 8 * kWave) return 0;
  const int cols = igl_gemv_chunk_cols(lanes, K, lds_limit);
  const size_t chunks = (size_t)((K + cols - 1) / cols);
  return chunks > 1 ? chunks * (size_t)lanes * (size_t)N : 0;
}

// Whether two to four lanes of an N x K plane run as one-lane grids side by
// side rather than in one multi-lane form.  Measured (replayed, us, lanes 2 /
// 3 / 4, one-lane grids against the form): 1536 x 2048 2.87 / 3.03 / 3.11
// against 3.11 / 4.44 / 4.93, 1536 x 6144 5.21 / 6.66 / 7.76 against 6.08 /
// 8.55 / 8.64, 4096 x 2048 3.86 / 4.50 / 5.14 against 4.69 / 6.38 / 7.09;
// but 8192 x 2048 5.47 / 7.17 / 8.52 against 5.17 / 6.23 / 7.09, and past
// about 40M lane-codes the repeated reads cost more than the form (1536 x
// 12288: 9.07 / 11.58 / 15.03 against 9.42 / 11.31 / 11.40; 2048 x 8192 four
// lanes 9.24 against 8.52).  The head's 262144 rows never split.
static bool gemv_lane_rows_pay(int lanes, int N, int K) {
  return lanes >= 2 && lanes <= 4 && N <= 4096 && (long long)lanes * N * K <= 40LL * 1024 * 1024;
}

// Launches y = W x for 1..16 lanes (past 16: chunks of 8).  `part` must hold chunks * lanes * N floats
// when the plane needs more than one K-chunk, and may be NULL otherwise;
// `lds_limit` is the device's LDS bytes per workgroup.
extern "C" hipError_t igl_launch_gemv_q4(const uint8_t *codes, long long row_stride,
                                         const float *gains, int gain_stride, int group_shift,
                                         int code_bias, const float *act, int act_stride,
                                         int lanes, float *out, int out_stride, int N, int K,
                                         float *part, int lds_limit, hipStream_t stream) {
  // 9 to 16 lanes: one matrix-core launch where the form applies, else
  // launches of 8 lanes in turn
  if (lanes > 8) {
    GemvMfmaPlan probe;
    if (lanes > 16 || !gemv_mfma_plan(lanes, N, K, &probe)) {
      for (int done = 0; done < lanes; done += 8) {
        const int n = lanes - done < 8 ? lanes - done : 8;
        const hipError_t e = igl_launch_gemv_q4(codes, row_stride, gains, gain_stride, group_shift, code_bias,
                                                act + (size_t)done * (size_t)act_stride, act_stride, n,
                                                out + (size_t)done * (size_t)out_stride, out_stride, N, K, part,
                                                lds_limit, stream);
        if (e != hipSuccess) return e;
      }
      return hipSuccess;
    }
  }
  GemvArgs a{};
  a.codes = codes;
  a.row_stride = row_stride;
  a.gains = gains;
  a.gain_stride = gain_stride;
  a.group_shift = group_shift;
  a.act = act;
  a.act_stride = act_stride;
  a.N = N;
  a.K = K;
  a.unit_bias = 16.0f + (float)code_bias;
  a.act_vec = ((((uintptr_t)act) & 15u) == 0 && (act_stride & 3) == 0) ? 1 : 0;
  // One to four lanes on the integer dot path (aligned activations, M K <=
  // 16384, or two lanes up to K 12288: the 1536 x 12288 down projection of
  // a two-lane speculative block, 11.4 -> 8.3 us against the float form,
  // and the matrix-core form's 10.9): eight-row tiles from 128 units up for one and two lanes, so the
  // staging of x is shared by more rows, and on tall planes (32768 rows and
  // up: at least 1024 workgroups of 32 rows), where every workgroup's staging
  // of x would otherwise be read as often as the weights (the 262144 x 1536
  // head: 52 -> 41 us); below that two-row tiles for one lane (twice the
  // workgroups, half the loads a lane in flight: measured ~2% faster at
  // 8192 x 2048 than four, and eight rows 25% slower); enough waves on a row
  // tile that each lane holds one unit (two past 256).
  //
  // Two to four lanes of a small plane run as that many one-lane grids side
  // by side (lane_rows, gemv_lane_rows_pay): the arithmetic of a lane is the
  // one-lane form's, the plane is read once a lane (the repeats from the L2
  // and the MALL), and each workgroup stages one lane of x.
  const int form = gemv_lane_rows_pay(lanes, N, K) ? 1 : lanes;  // lanes of the kernel's form
  if (a.act_vec && lanes <= 4 &&
      (form * K <= kDotMaxItems * kGemvThreads * 8 || (form == 2 && K <= 12288)) &&
      K / 32 <= 8 * kWave) {
    const int units = K / 32;
    a.lane_rows = form == 1 ? lanes : 1;
    int R = form <= 2 && (units >= 128 || N >= 32768) ? 8 : form == 1 ? 2 : 4;
    // One or two lanes on wide rows: six-row tiles where eight leave CUs
    // without a workgroup and six give every CU at most one (1536 x 12288:
    // 192 -> 256 workgroups, one lane 7.77 -> 6.94 us, two lanes 10.57 ->
    // 9.46 us; 1536 x 6144 4.36 -> 4.27 us and 6.74 -> 6.10 us; the same sums).
    if (form <= 2 && R == 8 && N < 32768 && (N + 7) / 8 < 256 && (N + 5) / 6 <= 256) R = 6;
    const int tiles = (N + R - 1) / R;
    int upl = units > 4 * kWave ? 2 : 1;
    int ksplit = 1;
    while (ksplit < 4 && (units > ksplit * kWave * upl ||
                          (tiles * ksplit < 2048 && units / (ksplit * 2) >= 32 * upl)))
      ksplit *= 2;
    // One or two lanes on a small plane (under 4096 rows, at most 128
    // units): two-row tiles, one wave a tile, two units a lane past 64 --
    // fewer workgroups than the split above gives, and faster (lab, one lane:
    // 1536 x 2048 2.95 -> 2.61 us, the same sums; 1536 x 4096 3.49 -> 2.97
    // us; two lanes: 1536 x 4096 5.22 -> 3.85 us, 1536 x 2048 3.43 -> 3.14,
    // 1536 x 256 3.10 -> 2.60).
    if (form <= 2 && N < 4096 && units <= 2 * kWave) {
      R = 2;
      upl = units > kWave ? 2 : 1;
      ksplit = 1;
    }
    a.ksplit = ksplit;
    a.chunk_cols = K;
    a.out = out;
    a.out_stride = out_stride;
    switch (form) {
      case 1:
        if (R == 2) return upl == 2 ? gemv_dot_launch<1, 2, 2>(a, stream) : gemv_dot_launch<1, 2, 1>(a, stream);
        if (R == 4) return gemv_dot_launch<1, 4, 1>(a, stream);
        if (R == 6) return upl == 2 ? gemv_dot_launch<1, 6, 2>(a, stream) : gemv_dot_launch<1, 6, 1>(a, stream);
        return upl == 2 ? gemv_dot_launch<1, 8, 2>(a, stream) : gemv_dot_launch<1, 8, 1>(a, stream);
      case 2:
        if (R == 6) return upl == 2 ? gemv_dot_launch<2, 6, 2>(a, stream) : gemv_dot_launch<2, 6, 1>(a, stream);
        if (R == 2) return upl == 2 ? gemv_dot_launch<2, 2, 2>(a, stream) : gemv_dot_launch<2, 2, 1>(a, stream);
        if (R == 4) return upl == 2 ? gemv_dot_launch<2, 4, 2>(a, stream) : gemv_dot_launch<2, 4, 1>(a, stream);
        return upl == 2 ? gemv_dot_launch<2, 8, 2>(a, stream) : gemv_dot_launch<2, 8, 1>(a, stream);
      case 3: return gemv_dot_launch<3, 4, 1>(a, stream);
      default: return gemv_dot_launch<4, 4, 1>(a, stream);
    }
  }
  // Three to eight lanes on the matrix cores where the plane's width allows.
  GemvMfmaPlan plan;
  if (lanes >= 3 && gemv_mfma_plan(lanes, N, K, &plan)) {
    GemvMfmaArgs b;
    b.codes = codes;
    b.row_stride = row_stride;
    b.gains = gains;
    b.gain_stride = gain_stride;
    b.group_shift = a.group_shift;
    b.act = act;
    b.act_stride = act_stride;
    b.act_vec = a.act_vec;
    b.M = lanes;
    b.N = N;
    b.K = K;
    b.tiles_per_block = plan.tiles_per_block;
    b.chunk_units = plan.chunk_units;
    b.code_bias = (float)code_bias;
    b.gain_vec = (a.group_shift == 0 && (((uintptr_t)gains) & 15u) == 0 && (gain_stride & 3) == 0) ? 1 : 0;
    if (plan.chunks > 1) {
      if (!part) return hipErrorInvalidValue;
      b.out = part;
      b.out_stride = N;
    } else {
      b.out = out;
      b.out_stride = out_stride;
    }
    hipError_t e = gemv_mfma_dispatch(b, plan, stream);
    if (e != hipSuccess || plan.chunks == 1) return e;
    const int total = lanes * N;
    hipLaunchKernelGGL(gemv_chunk_sum_kernel, dim3((total + 255) / 256), dim3(256), 0, stream, part,
                       plan.chunks, lanes, N, out, out_stride);
    return hipGetLastError();
  }
  // One and two lanes with unaligned activations and at most 512 units a
  // row: the float register form, the integer form's layout.
  if (lanes <= 2 && K / 32 <= 8 * kWave) {
    const int units = K / 32;
    const int R = 4;
    const int tiles = (N + R - 1) / R;
    const int upl = units > 4 * kWave ? 2 : 1;
    int ksplit = 1;
    while (ksplit < 4 && (units > ksplit * kWave * upl ||
                          (tiles * ksplit < 2048 && units / (ksplit * 2) >= 32 * upl)))
      ksplit *= 2;
    a.ksplit = ksplit;
    a.chunk_cols = K;
    a.out = out;
    a.out_stride = out_stride;
    if (upl == 2)
      return lanes == 1 ? gemv_reg_launch<1, 4, 2>(a, stream) : gemv_reg_launch<2, 4, 2>(a, stream);
    return lanes == 1 ? gemv_reg_launch<1, 4, 1>(a, stream) : gemv_reg_launch<2, 4, 1>(a, stream);
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

extern "C" hipError_t igl_launch_gemv_zero(const igl_code_view *v, const int8_t *zeros, const float *act,
                                           int act_stride, int lanes, float *out, int out_stride, int N, int K,
                                           hipStream_t stream) {
  const int bits = v->bit_count;
  if ((bits != 2 && bits != 4 && bits != 8) || K % 32 || !zeros || (((uintptr_t)act) & 15u) ||
      (lanes > 1 && (act_stride & 3)) || (v->row_stride & 7) || N < 1 || lanes < 1)
    return hipErrorInvalidValue;
  GemvZeroArgs a;
  a.codes = v->codes;
  a.row_stride = v->row_stride;
  a.gains = v->gains;
  a.zeros = zeros;
  a.gain_stride = v->gain_stride;
  a.group_shift = v->group_shift;
  a.code_bias = v->code_bias;
  a.code_flip = (uint32_t)v->code_flip;
  a.act_stride = act_stride;
  a.out_stride = out_stride;
  a.N = N;
  a.K = K;
  for (int done = 0; done < lanes; done += 8) {
    a.act = act + (size_t)done * (size_t)act_stride;
    a.out = out + (size_t)done * (size_t)out_stride;
    a.lanes = lanes - done < 8 ? lanes - done : 8;
    const hipError_t e = bits == 2   ? gemv_zero_launch_bits<2>(a, stream)
                         : bits == 4 ? gemv_zero_launch_bits<4>(a, stream)
                                     : gemv_zero_launch_bits<8>(a, stream);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}
