// igl_gemm_level.hip - prefill of a calibrated plane on the integer matrix
// cores, gfx950 v_mfma_i32_16x16x64_i8.
//
// A calibrated plane (enter_gain > 0, one gain a row) is the reference's level
// path (kern_row_code_level, app_core.c:3272-3296, with quant_step 1930-1940):
//     L[m][k] = clamp(rint(x[m][k] / step), -128, 127)
//     part    = sum_k L[m][k] * ((c[n][k] ^ flip) - code_bias)      (exact)
//     y[m][n] = gain[n] * step * part, then the leave grid
// Here the levels are int8 operands and the codes become int8 operands with a
// power-of-two factor, so every product and sum is an exact int32:
//   * 4-bit: (c ^ flip ^ 8) is c - 8 as a signed nibble; moved to the top of
//     its byte it reads as 16 (c - 8).  A dword of eight codes gives two
//     dwords of operands in three ops; the sum carries the factor 16.
//   * 2-bit: (c ^ flip ^ 2) at the top of a byte reads as 64 (c - 2).
//   * 8-bit: c ^ flip ^ 0x80 is (c ^ flip) - 128 as a signed byte.
// The factor leaves the int32 sum exactly (an arithmetic shift), and the row
// close is the reference's to the bit.  No level sums are needed.
//
// The operands' k order inside each sixteen follows the decoding: for 4-bit
// codes 0 2 4 6 1 3 5 7 8 10 12 14 9 11 13 15, for 2-bit 0 4 8 12 1 5 9 13 2
// 6 10 14 3 7 11 15; the levels are written in the same order
// (act_level_kernel), so a lane's sixteen levels and sixteen codes meet.
//
// Tile: 256 x 256 a workgroup, eight waves (2 x 4) of 128 x 64 as 8 x 4
// accumulators; K 128 a step (64 for 8-bit codes, whose stages are twice as
// large), three LDS stages of levels and codes filled only by global_load_lds
// two steps ahead.  16-byte chunks of a row are XOR-swizzled (lv_key) so that
// rows read together by the sixteen lanes of a row tile spread over the banks.
// K is cut into slices when the tiles leave CUs idle; slices write int32
// partials that level_close_kernel adds (exactly, in any order) and closes.
#include "igl_device.h"
#include "igl_launch.h"

namespace igl {

typedef int32_t int4v_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void global_void_t;

constexpr int kLvM = 256;
constexpr int kLvN = 256;
constexpr int kLvStages = 3;
constexpr int kLvThreads = 512;

template <int BITS>
struct LevelForm {
  static constexpr int K = BITS == 8 ? 64 : 128;        // k a step
  static constexpr int Q = K / 64;                      // products a (row, column) tile a step
  static constexpr int RA = K;                          // bytes of a level row in a stage
  static constexpr int RB = K * BITS / 8;               // bytes of a code row in a stage
  static constexpr int A_BYTES = kLvM * RA;
  static constexpr int B_BYTES = kLvN * RB;
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int LDS = kLvStages * STAGE;
  static constexpr int SHIFT = BITS == 4 ? 4 : BITS == 2 ? 6 : 0;
  static constexpr int A_LOADS = A_BYTES / (8 * 1024);  // 16-byte DMA instructions a wave, levels
  static constexpr int B_LOADS = B_BYTES / (8 * 1024);  // and codes
};

// The swizzle of a row of `RB` bytes: its 16-byte chunk c sits at c ^ key,
// the key changing every 256 bytes of rows.
template <int RB>
__device__ __forceinline__ int lv_key(int row) {
  constexpr int per_cycle = 256 / RB;  // rows whose chunks share one LDS cycle's 64 banks
  constexpr int chunks = RB / 16;
  return (row / per_cycle) & (chunks - 1);
}

struct LevelArgs {
  const int8_t *levels;   // [M][K], act_level_kernel's order
  const int32_t *nan_rows;  // [M]: 1 where the row held a NaN
  const uint8_t *codes;
  long long row_stride;
  uint32_t code_xor;      // replicated (flip ^ bias) of the code width
  const float *gains;     // [N], one a row
  float step, leave;
  float *out;             // [M][out_stride] fp32
  int out_stride;
  int32_t *part;          // with slices: [slice][M][N] int32 partials
  int M, N, K;
  int k_steps;            // steps of one slice (blockIdx.z)
};

// y / leave as rint needs it: quot_near (the correctly rounded quotient below
// 256, the rest clamps alike, NaN stays NaN) from leave_rcp =
// level_recip(leave); a leave outside that range (leave_rcp 0) divides.
__device__ __forceinline__ float div_leave(float y, float leave, float leave_rcp) {
  return leave_rcp != 0.0f ? quot_near(y, leave, leave_rcp) : y / leave;
}

// The leave grid (quant_step) on y = fl(gain * step) * part.
__device__ __forceinline__ float level_grid(float gain_step, int32_t part, float leave, float leave_rcp) {
  float y = gain_step * (float)part;
  if (leave > 0.0f) {
    float level = __builtin_rintf(div_leave(y, leave, leave_rcp));
    level = level < -128.0f ? -128.0f : level;
    level = level > 127.0f ? 127.0f : level;
    y = level * leave;
  }
  return y;
}

// Sixteen codes (one k-sixteen of a row) as sixteen int8 operands.
template <int BITS>
__device__ __forceinline__ int4v_t level_codes(const uint8_t *p, uint32_t code_xor) {
  if (BITS == 4) {
    const uint2_t raw = *reinterpret_cast<const uint2_t *>(p);
    const uint32_t a = raw[0] ^ code_xor, b = raw[1] ^ code_xor;
    return int4v_t{(int)((a << 4) & 0xF0F0F0F0u), (int)(a & 0xF0F0F0F0u), (int)((b << 4) & 0xF0F0F0F0u),
                   (int)(b & 0xF0F0F0F0u)};
  } else if (BITS == 2) {
    const uint32_t d = *reinterpret_cast<const uint32_t *>(p) ^ code_xor;
    return int4v_t{(int)((d << 6) & 0xC0C0C0C0u), (int)((d << 4) & 0xC0C0C0C0u), (int)((d << 2) & 0xC0C0C0C0u),
                   (int)(d & 0xC0C0C0C0u)};
  } else {
    const uint4_t raw = *reinterpret_cast<const uint4_t *>(p);
    return int4v_t{(int)(raw[0] ^ code_xor), (int)(raw[1] ^ code_xor), (int)(raw[2] ^ code_xor),
                   (int)(raw[3] ^ code_xor)};
  }
}

template <int BITS>
__global__ __launch_bounds__(kLvThreads) void gemm_level_kernel(LevelArgs g) {
  using F = LevelForm<BITS>;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds_l[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2;      // 2 wave rows of 128
  const int wn = wave & 3;       // 4 wave columns of 64
  int tile_x, tile_y;
  xcd_tile(tile_x, tile_y);
  const int m0 = tile_y * kLvM;
  const int n0 = tile_x * kLvN;
  const int steps = g.k_steps;
  const int k_first = blockIdx.z * g.k_steps * F::K;

  // DMA sources.  A wave instruction moves 64 lanes x 16 bytes: lane l fills
  // physical chunk l % C of row R0 + l / C (C chunks a row) with the row's
  // logical chunk (l % C) ^ key(row).
  constexpr int CA = F::RA / 16, CB = F::RB / 16;
  const int8_t *a_src[F::A_LOADS];
#pragma unroll
  for (int i = 0; i < F::A_LOADS; ++i) {
    const int r = (64 / CA) * (F::A_LOADS * wave + i) + lane / CA;
    const int c = (lane % CA) ^ lv_key<F::RA>(r);
    a_src[i] = g.levels + (size_t)min(m0 + r, g.M - 1) * g.K + k_first + 16 * c;
  }
  const uint8_t *b_src[F::B_LOADS];
#pragma unroll
  for (int i = 0; i < F::B_LOADS; ++i) {
    const int r = (64 / CB) * (F::B_LOADS * wave + i) + lane / CB;
    const int c = (lane % CB) ^ lv_key<F::RB>(r);
    b_src[i] = g.codes + (size_t)min(n0 + r, g.N - 1) * (size_t)g.row_stride + (size_t)k_first * BITS / 8 + 16 * c;
  }
  auto stage_of = [&](int step) { return lds_l + (step % kLvStages) * F::STAGE; };
  auto issue = [&](int step) {
    uint8_t *st = stage_of(step);
    const int k0 = step * F::K;
#pragma unroll
    for (int i = 0; i < F::A_LOADS; ++i)
      __builtin_amdgcn_global_load_lds((global_void_t *)(a_src[i] + k0),
                                       (lds_void_t *)(st + (F::A_LOADS * wave + i) * 1024), 16, 0, 0);
#pragma unroll
    for (int i = 0; i < F::B_LOADS; ++i)
      __builtin_amdgcn_global_load_lds((global_void_t *)(b_src[i] + (size_t)k0 * BITS / 8),
                                       (lds_void_t *)(st + F::A_BYTES + (F::B_LOADS * wave + i) * 1024), 16, 0,
                                       0);
  };
  // Waits until this wave's loads of all but the last step issued are in
  // (vmcnt retires them in order) and its LDS reads have landed, then meets
  // every wave at a bare barrier.
  constexpr int kPerStep = F::A_LOADS + F::B_LOADS;
  auto wait_meet = [&](bool one_pending) {
    if (one_pending)
      __builtin_amdgcn_s_waitcnt(0x0070 | kPerStep);  // vmcnt(kPerStep) lgkmcnt(0)
    else
      __builtin_amdgcn_s_waitcnt(0x0070);             // vmcnt(0) lgkmcnt(0)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  int4v_t acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = int4v_t{0, 0, 0, 0};
  const int gq = lane >> 4;  // lane group: the step's k-sixteen Q gq .. of product q is 4 q + gq
  const int n = lane & 15;

  auto read_rows = [&](const uint8_t *st, int i, int4v_t (&a)[F::Q]) {
#pragma unroll
    for (int q = 0; q < F::Q; ++q) {
      const int r = wm * 128 + 16 * i + n;
      const int c = (4 * q + gq) ^ lv_key<F::RA>(r);
      a[q] = *reinterpret_cast<const int4v_t *>(st + r * F::RA + 16 * c);
    }
  };
  auto read_codes = [&](const uint8_t *st, int4v_t (&b)[F::Q][4]) {
    const uint8_t *bs = st + F::A_BYTES;
#pragma unroll
    for (int q = 0; q < F::Q; ++q)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = wn * 64 + 16 * j + n;
        const int s = 4 * q + gq;                      // the k-sixteen's slot of BITS * 2 bytes
        const int byte = s * BITS * 2;                 // logical offset in the row
        const int c = (byte >> 4) ^ lv_key<F::RB>(r);  // its 16-byte chunk, swizzled
        b[q][j] = level_codes<BITS>(bs + r * F::RB + 16 * c + (byte & 15), g.code_xor);
      }
  };

  issue(0);
  if (steps > 1) issue(1);
  for (int s = 0; s < steps; ++s) {
    wait_meet(s + 1 < steps);
    if (s + 2 < steps) issue(s + 2);
    const uint8_t *st = stage_of(s);
    int4v_t bf[F::Q][4];
    read_codes(st, bf);
    int4v_t a_cur[F::Q], a_next[F::Q];
    read_rows(st, 0, a_cur);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (i + 1 < 8) read_rows(st, i + 1, a_next);
#pragma unroll
      for (int q = 0; q < F::Q; ++q)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf[q][j], a_cur[q], acc[i][j], 0, 0, 0);
#pragma unroll
      for (int q = 0; q < F::Q; ++q) a_cur[q] = a_next[q];
    }
  }

  // The codes are the products' first operand: lane l of a 16 x 16 tile holds
  // row l % 16 of its row tile and columns 4 (l / 16) .. + 3.
  const bool vec_ok = g.part ? (g.N % 4 == 0) : (g.out_stride % 4 == 0 && ((uintptr_t)g.out & 15u) == 0);
  int32_t *part = g.part ? g.part + (size_t)blockIdx.z * (size_t)g.M * (size_t)g.N : nullptr;
  // fl(gain * step) of the lane's sixteen columns, loaded before any store
  // (the outputs could alias the gains as far as the compiler knows)
  float gs[4][4];
  const float leave_rcp = g.leave > 0.0f ? level_recip(g.leave) : 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) gs[j][r] = g.gains[min(n0 + wn * 64 + j * 16 + 4 * gq + r, g.N - 1)] * g.step;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int m = m0 + wm * 128 + i * 16 + n;
    if (m >= g.M) continue;
    const bool nan_row = !part && g.nan_rows[m];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int nb = n0 + wn * 64 + j * 16 + 4 * gq;
      if (part) {
        if (vec_ok && nb + 3 < g.N) {
          *reinterpret_cast<int4v_t *>(part + (size_t)m * g.N + nb) = acc[i][j];
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (nb + r < g.N) part[(size_t)m * g.N + nb + r] = acc[i][j][r];
        }
        continue;
      }
      float4_t v;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        v[r] = nan_row ? __builtin_nanf("") : level_grid(gs[j][r], acc[i][j][r] >> F::SHIFT, g.leave, leave_rcp);
      if (vec_ok && nb + 3 < g.N) {
        // streamed past L2: the fp32 tile outgrows the L2s, whose half-filled
        // lines were otherwise written back twice (WRITE_SIZE 1.5x the output)
        __builtin_nontemporal_store(v, reinterpret_cast<float4_t *>(g.out + (size_t)m * g.out_stride + nb));
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (nb + r < g.N) g.out[(size_t)m * g.out_stride + nb + r] = v[r];
      }
    }
  }
}

// The K slices' int32 partials added (exact), the factor shifted out, the row
// closed.
__global__ void level_close_kernel(const int32_t *part, int slices, int M, int N, int shift,
                                   const int32_t *nan_rows, const float *gains, float step, float leave,
                                   float *out, int out_stride) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  const int m = blockIdx.y;
  if (n >= N) return;
  int32_t t = 0;
  for (int z = 0; z < slices; ++z) t += part[((size_t)z * M + m) * N + n];
  const float leave_rcp = leave > 0.0f ? level_recip(leave) : 0.0f;
  out[(size_t)m * out_stride + n] =
      nan_rows[m] ? __builtin_nanf("") : level_grid(gains[n] * step, t >> shift, leave, leave_rcp);
}

// One block a row: levels rint(x / step) clamped to [-128, 127] (quant_step,
// app_core.c:1930-1940, as integers), written in the operand order of the
// plane's code width, and whether the row held a NaN (its outputs are NaN).
template <int BITS>
__global__ void act_level_kernel(const float *act, int act_stride, int K, float step, int8_t *levels,
                                 int32_t *nan_rows) {
  __shared__ int any_nan;
  const int m = blockIdx.x;
  if (threadIdx.x == 0) any_nan = 0;
  __syncthreads();
  const float *row = act + (size_t)m * act_stride;
  int8_t *dst = levels + (size_t)m * K;
  int nan_here = 0;
  for (int g16 = threadIdx.x; g16 < K / 16; g16 += blockDim.x) {
    float x[16];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float4_t f = *reinterpret_cast<const float4_t *>(row + 16 * g16 + 4 * v);
#pragma unroll
      for (int e = 0; e < 4; ++e) x[4 * v + e] = f[e];
    }
    int lv[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      nan_here |= x[e] != x[e];
      float level = __builtin_rintf(x[e] / step);
      level = level < -128.0f ? -128.0f : level;
      level = level > 127.0f ? 127.0f : level;
      lv[e] = x[e] != x[e] ? 0 : (int)level;
    }
    uint32_t w[4];
#pragma unroll
    for (int p4 = 0; p4 < 4; ++p4) {
      uint32_t word = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int p = 4 * p4 + b;  // operand position -> logical k inside the sixteen
        const int k = BITS == 4 ? ((p & 8) | ((p & 3) << 1) | ((p >> 2) & 1))
                    : BITS == 2 ? (((p & 3) << 2) | (p >> 2))
                                : p;
        word |= (uint32_t)(lv[k] & 0xFF) << (8 * b);
      }
      w[p4] = word;
    }
    *reinterpret_cast<uint4_t *>(dst + 16 * g16) = uint4_t{w[0], w[1], w[2], w[3]};
  }
  if (nan_here) any_nan = 1;
  __syncthreads();
  if (threadIdx.x == 0) nan_rows[m] = any_nan;
}

static int level_step_k(int bits) { return bits == 8 ? 64 : 128; }

// K slices while the tiles fill under half the CUs: a slice's int32 partials
// are M x N words each way, and at M = 2048 they cost more than idle CUs do
// (6144 x 1536, 192 tiles: 47 us unsplit, 86 us in two slices; 2048 x 1536,
// 64 tiles: 44.6 us in two, 46.2 us unsplit).
static int level_slices(int M, int N, int K, int bits) {
  const int tiles = ((M + kLvM - 1) / kLvM) * ((N + kLvN - 1) / kLvN);
  const int steps = K / level_step_k(bits);
  int slices = 1;
  while (slices < 16 && tiles * slices < 128 && steps % (2 * slices) == 0 && steps / (2 * slices) >= 2)
    slices *= 2;
  return slices;
}

static size_t level_levels_bytes(int M, int K) { return ((size_t)M * (size_t)K + 255) & ~(size_t)255; }
static size_t level_flag_bytes(int M) { return ((size_t)M * 4 + 255) & ~(size_t)255; }

}  // namespace igl

using namespace igl;

extern "C" int igl_gemm_level_fits(int bits, int code_bias, int K) {
  if (bits != 2 && bits != 4 && bits != 8) return 0;
  if (code_bias != (1 << (bits - 1))) return 0;
  return K >= level_step_k(bits) && K % level_step_k(bits) == 0;
}

extern "C" size_t igl_gemm_level_work_bytes(int M, int N, int K, int bits) {
  const int slices = level_slices(M, N, K, bits);
  return level_levels_bytes(M, K) + level_flag_bytes(M) +
         (slices > 1 ? (size_t)slices * (size_t)M * (size_t)N * sizeof(int32_t) : 0);
}

template <int BITS>
static hipError_t gemm_level_launch(const LevelArgs &a, int slices, hipStream_t stream) {
  const size_t lds = (size_t)LevelForm<BITS>::LDS;
  static bool granted = false;
  if (!granted) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_level_kernel<BITS>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    granted = true;
  }
  dim3 grid((a.N + kLvN - 1) / kLvN, (a.M + kLvM - 1) / kLvM, slices);
  hipLaunchKernelGGL((gemm_level_kernel<BITS>), grid, dim3(kLvThreads), lds, stream, a);
  return hipGetLastError();
}

extern "C" hipError_t igl_launch_gemm_level(const float *act, int act_stride, const uint8_t *codes,
                                            long long row_stride, int bits, int code_flip, int code_bias,
                                            const igl_gemm_close *close, float *out, int out_stride, int M,
                                            int N, int K, void *work, hipStream_t stream) {
  if (!act || !codes || !close || !close->gains || !out || !work || M < 1 || N < 1 ||
      !igl_gemm_level_fits(bits, code_bias, K) || !(close->step > 0.0f) || row_stride % 16 ||
      ((uintptr_t)codes & 15u) || ((uintptr_t)act & 15u) || act_stride % 4 || (M > 1 && act_stride < K) ||
      (M > 1 && out_stride < N))
    return hipErrorInvalidValue;
  const int slices = level_slices(M, N, K, bits);
  int8_t *levels = reinterpret_cast<int8_t *>(work);
  int32_t *nan_rows = reinterpret_cast<int32_t *>(reinterpret_cast<uint8_t *>(work) + level_levels_bytes(M, K));
  int32_t *part = slices > 1 ? reinterpret_cast<int32_t *>(reinterpret_cast<uint8_t *>(nan_rows) +
                                                           level_flag_bytes(M))
                             : nullptr;
  const float step = close->step;
  const int threads = K / 16 < 256 ? ((K / 16 + 63) / 64) * 64 : 256;
  if (bits == 4)
    hipLaunchKernelGGL((act_level_kernel<4>), dim3(M), dim3(threads), 0, stream, act, act_stride, K, step, levels,
                       nan_rows);
  else if (bits == 2)
    hipLaunchKernelGGL((act_level_kernel<2>), dim3(M), dim3(threads), 0, stream, act, act_stride, K, step, levels,
                       nan_rows);
  else
    hipLaunchKernelGGL((act_level_kernel<8>), dim3(M), dim3(threads), 0, stream, act, act_stride, K, step, levels,
                       nan_rows);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  LevelArgs a;
  a.levels = levels;
  a.nan_rows = nan_rows;
  a.codes = codes;
  a.row_stride = row_stride;
  const uint32_t x = (uint32_t)(code_flip ^ code_bias);
  a.code_xor = bits == 4 ? (x & 15u) * 0x11111111u : bits == 2 ? (x & 3u) * 0x55555555u : (x & 255u) * 0x01010101u;
  a.gains = close->gains;
  a.step = step;
  a.leave = close->leave;
  a.out = out;
  a.out_stride = M == 1 ? N : out_stride;
  a.part = part;
  a.M = M;
  a.N = N;
  a.K = K;
  a.k_steps = K / level_step_k(bits) / slices;
  e = bits == 4 ? gemm_level_launch<4>(a, slices, stream)
      : bits == 2 ? gemm_level_launch<2>(a, slices, stream)
                  : gemm_level_launch<8>(a, slices, stream);
  if (e != hipSuccess || slices == 1) return e;
  const int shift = bits == 4 ? 4 : bits == 2 ? 6 : 0;
  hipLaunchKernelGGL(level_close_kernel, dim3((N + 255) / 256, M), dim3(256), 0, stream, part, slices, M, N, shift,
                     nan_rows, close->gains, step, close->leave, out, a.out_stride);
  return hipGetLastError();
}
