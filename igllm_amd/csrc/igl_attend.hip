// igl_attend.hip - decode attention over the byte-quantized key/value ring,
// gfx950.
//
// For one lane (one query position) and each key/value head shared by 8
// query heads, computes
//     o_h = sum_t softmax_t(score_scale * q_h . k_t) v_t
// over the visible positions t = place_start .. place_start + span - 1, whose
// rows sit in ring slot t % cache_span (session_attend_group with
// attend_score_band and attend_blend_band, app_core.c:11296-11453; ring and
// span rules 11500, 11516-11526).  A stored byte decodes to
//     e4m3:  cache_real8(byte) * scale   (cache_real8, app_core.c:11018-11030)
//     int8:  (int8_t)byte * scale
// The reference scores every row against `grid[byte] = real8 * scale`; here
// the scale multiplies the finished dot product, the same value up to fp32
// rounding.
//
// Why MFMA: with 8 query heads on one key/value head every key and value
// byte feeds 8 multiply-adds, 8 MAC per byte of HBM traffic, above the ~5
// fp32 MAC per byte the vector ALU can sustain at the HBM rate.  Both
// products therefore run on v_mfma_f32_16x16x32_f16:
//   scores  S[16 x 32 positions] = [q_hi; q_lo] (16 x d) . K^T (d x 32)
//   blend   O[16 x d]            = [p_hi; p_lo] (16 x 32) . V (32 x d)
// The 16 MFMA rows hold each head twice, as an exact two-term binary16 split
// (x = hi + lo, |lo| <= 2^-11 |x|), so the products keep ~22 significant
// bits and accumulate in fp32; the two rows are added at the end.  Bytes
// decode to binary16 exactly:
//   e4m3: move bit 7 to bit 8 and shift the byte up by 7, giving
//         real8(byte) / 256 for all 256 codes (0x7F/0xFF read +-480, as the
//         reference reads them);
//   int8: (byte ^ 0x80) in the mantissa of 1024.0, minus 1152.
//
// Work layout: a workgroup owns W waves of 32 positions, W = 1 for spans up
// to kAttendShortSpan (the most workgroups and the shortest chain each: at a
// 2048-position decode context one wave measured 3% faster a token than four,
// the merge launch costing little in the replayed step) and 4 beyond.  A wave
// loads its 32 key rows straight into MFMA operand order (each lane a
// contiguous d/4-byte run of a row), its 32 value rows into LDS (transposed on
// read), runs the scores, the softmax against its peak, and the blend; the
// waves' (max, total, output) are merged in LDS and written as the
// workgroup's partial.  A second kernel merges the partials in order
// (flash-decoding); a span of one chunk is written directly.
#include <mutex>

#include "igl_backend.h"
#include "igl_device.h"

namespace igl {

constexpr int kAttendTile = 32;                    // positions per wave
// Waves a workgroup (its chunk: 32 positions a wave), by the longest span a
// launch covers: one up to kAttendShortSpan positions (the most workgroups,
// the shortest chain each), four beyond (fewer partials to write and merge: at
// 16384 positions four measured 14.7 us against 20.4 us for one).
constexpr int kAttendShortSpan = 4096;
constexpr int kAttendGroup = 8;                    // query heads per key/value head

struct AttendArgs {
  const uint8_t *key_store;    // [cache_span][kv_width]
  const uint8_t *value_store;
  int kv_width;
  int cache_span;
  int place0;                  // position of lane 0; lane l is at place0 + l
  const int *place_dev;        // when set, lane 0's position is read here instead
  int window;                  // positions a lane sees (0: all from position 0)
  int chunks;                  // workgroup slots per lane in the partial buffers
  float *final_out;            // when one workgroup covers a lane: the blend, [lanes][q_stride]
  int q_stride;                // floats between lanes of query / blend
  const float *query;          // [lanes][head_count][HEAD]
  float key_scale;             // decoded-byte multiplier, score_scale folded in
  float value_scale;
  float *part_out;             // [chunks][head_count][HEAD]
  float *part_peak;            // [chunks][head_count]
  float *part_total;           // [chunks][head_count]
  int head_count;
};

// Two bytes held in bits [0,8) and [16,24) of `x`, as two exact binary16.
template <int FMT>
__device__ __forceinline__ uint32_t decode_pair(uint32_t x) {
  if (FMT == 0) {
    return (x + (x & 0x00800080u)) << 7;  // e4m3 -> real8 / 256
  } else {
    half2_t h = as_half2(x ^ 0x64806480u);  // 1152 + (int8)byte
    h = h + half2_t{(_Float16)-1152.0f, (_Float16)-1152.0f};
    return __builtin_bit_cast(uint32_t, h);
  }
}

// Eight bytes (two dwords, low byte first) as eight binary16 operand values.
template <int FMT>
__device__ __forceinline__ half8_t decode8(uint32_t lo, uint32_t hi) {
  uint32_t w[4];
  w[0] = decode_pair<FMT>(__builtin_amdgcn_perm(0u, lo, 0x0C010C00u));
  w[1] = decode_pair<FMT>(__builtin_amdgcn_perm(0u, lo, 0x0C030C02u));
  w[2] = decode_pair<FMT>(__builtin_amdgcn_perm(0u, hi, 0x0C010C00u));
  w[3] = decode_pair<FMT>(__builtin_amdgcn_perm(0u, hi, 0x0C030C02u));
  return __builtin_bit_cast(half8_t, w);
}

// v plus its partner 32 lanes away, the same value in both lanes: one
// v_permlane32_swap of two copies of v leaves the lower halves in one and the
// upper halves in the other.  Written out because the builtin given the same
// value twice is folded as if both results were its first; the s_nops are the
// waits the compiler itself places around this instruction.
__device__ __forceinline__ float xsum32(float v) {
  float lo = v, hi = v;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(lo), "+v"(hi));
  return lo + hi;
}

// One workgroup takes one chunk of kChunk positions of one lane; each wave
// owns 32 positions of it.  The query, key and value loads all go out first, so the
// launch pays one memory round trip; then the scores, the wave's softmax
// against its own peak, and the blend.  The waves merge in LDS.  A
// workgroup that covers the lane's whole span writes the blend; otherwise it
// writes a partial (blend, peak, total) for attend_merge_kernel.
//
// (Measured: the last workgroup to finish merging the partials itself, after
// an agent-scope release/acquire ticket, was slower than the merge launch at
// every span tried, 15 vs 13 us at a 512 window and 52 vs 29 us at 2300
// positions of 512 dims: one CU then reads every partial.)
template <int HEAD, int FMT, bool QVEC, int W>
__global__ __launch_bounds__(64 * W) void attend_mfma_kernel(AttendArgs a) {
  constexpr int kThreads = 64 * W;            // W waves
  constexpr int kChunk = kAttendTile * W;     // positions a workgroup
  constexpr int S = HEAD / 32;        // k-steps of the score product
  constexpr int QD = HEAD / 4;        // bytes of a key row one lane group reads
  constexpr int TILES = HEAD / 16;    // 16-wide dim tiles of the blend
  constexpr int QUADS = TILES / 4;    // four tiles share one LDS read
  constexpr int VPITCH = HEAD + 8;    // staged value row: (HEAD/4 + 2) dwords, conflict-free reads
  constexpr int kWaveV = kAttendTile * VPITCH;

  __shared__ __attribute__((aligned(16))) uint8_t vs[W * kWaveV];
  __shared__ float ps[W][kAttendGroup][kAttendTile];
  __shared__ float wm[W][kAttendGroup];
  __shared__ float wl[W][kAttendGroup];
  __shared__ float head_peak[kAttendGroup];
  __shared__ float head_norm[kAttendGroup];
  // the query block as binary16 operands: [part hi / lo][head][HEAD / 8]
  __shared__ half8_t qs[2][kAttendGroup][HEAD / 8];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 4;        // lane group
  const int n = lane & 15;        // MFMA row (A) / column (B, D)
  const int kv = blockIdx.y;
  const int head0 = kv * kAttendGroup;
  const int block = blockIdx.x;
  const int lane_id = blockIdx.z;
  // The lane's visible positions: the last `window` up to and including its
  // own (session_attend 11516-11526); `start` is the first, ring slot p % span.
  const int pos = (a.place_dev ? *a.place_dev : a.place0) + lane_id;
  const int span_count = a.window > 0 ? min(pos + 1, a.window) : pos + 1;
  const int place_start = pos - span_count + 1;
  const int blocks_seen = (span_count + kChunk - 1) / kChunk;
  if (block >= blocks_seen) return;  // past this lane's span
  const int pc = lane_id * a.chunks + block;
  const size_t kv_off = (size_t)kv * HEAD;
  const int t0 = block * kChunk + wave * kAttendTile;
  const bool live = t0 < span_count;

  // ---- loads.  The query block (8 heads x HEAD floats) is split among the
  // workgroup's threads, eight floats each, to be converted once; key rows n
  // and n + 16 of the wave's 32, bytes QD g .. QD g + QD - 1 (operand order);
  // value rows lane / 2, half lane & 1.  Rows past the span repeat the last.
  constexpr int kQTotal = kAttendGroup * HEAD / 8;                 // eight-float items
  constexpr int kQItems = (kQTotal + kThreads - 1) / kThreads;
  float qf[kQItems][8];
  {
    const float *qb = a.query + (size_t)lane_id * a.q_stride + (size_t)head0 * HEAD;
#pragma unroll
    for (int i = 0; i < kQItems; ++i) {
      const int item = tid + kThreads * i;
      const float *q = qb + 8 * (kQTotal % kThreads == 0 ? item : min(item, kQTotal - 1));
      if (QVEC) {
        const float4_t u = *reinterpret_cast<const float4_t *>(q);
        const float4_t v = *reinterpret_cast<const float4_t *>(q + 4);
        qf[i][0] = u.x; qf[i][1] = u.y; qf[i][2] = u.z; qf[i][3] = u.w;
        qf[i][4] = v.x; qf[i][5] = v.y; qf[i][6] = v.z; qf[i][7] = v.w;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) qf[i][e] = q[e];
      }
    }
  }
  uint4_t kr[2][QD / 16];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int t = min(t0 + n + 16 * j, span_count - 1);
    const int slot = (place_start + t) % a.cache_span;
    const uint4_t *row =
        reinterpret_cast<const uint4_t *>(a.key_store + (size_t)slot * a.kv_width + kv_off + QD * g);
#pragma unroll
    for (int q = 0; q < QD / 16; ++q) kr[j][q] = __builtin_nontemporal_load(row + q);
  }
  uint2_t vr[HEAD / 16];
  {
    const int t = min(t0 + (lane >> 1), span_count - 1);
    const int slot = (place_start + t) % a.cache_span;
    const uint2_t *src = reinterpret_cast<const uint2_t *>(
        a.value_store + (size_t)slot * a.kv_width + kv_off + (lane & 1) * (HEAD / 2));
#pragma unroll
    for (int q = 0; q < HEAD / 16; ++q) vr[q] = __builtin_nontemporal_load(src + q);
  }

  // query operands: x = hi + lo, each rounded to binary16 (|lo| <= 2^-11 |x|);
  // row n of the score product is head n & 7, its hi part (n < 8) or lo part
#pragma unroll
  for (int i = 0; i < kQItems; ++i) {
    half8_t hi8, lo8;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const _Float16 hi = (_Float16)qf[i][e];
      hi8[e] = hi;
      lo8[e] = (_Float16)(qf[i][e] - (float)hi);
    }
    const int item = tid + kThreads * i;  // head item / (HEAD / 8), chunk item % (HEAD / 8)
    if (kQTotal % kThreads == 0 || item < kQTotal) {
      qs[0][item / (HEAD / 8)][item % (HEAD / 8)] = hi8;
      qs[1][item / (HEAD / 8)][item % (HEAD / 8)] = lo8;
    }
  }
  __syncthreads();
  half8_t qa[S];
#pragma unroll
  for (int s = 0; s < S; ++s) qa[s] = qs[n >> 3][n & 7][QD * g / 8 + s];

  // ---- scores.  After the half-wave sum, lane groups 0/2 hold heads 0-3 and
  // 1/3 heads 4-7 (row r of the group is head 4 (g & 1) + r), for positions
  // n and n + 16 of the wave's 32.
  float sc[2][4];
  float m_w[4];
  {
    float4_t sacc[2] = {float4_t{0, 0, 0, 0}, float4_t{0, 0, 0, 0}};
    if (live) {
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int s = 0; s < S; ++s) {
          const uint4_t w = kr[j][s >> 1];
          const half8_t kb = (s & 1) ? decode8<FMT>(w[2], w[3]) : decode8<FMT>(w[0], w[1]);
          sacc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[s], kb, sacc[j], 0, 0, 0);
        }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float s0 = xsum32(sacc[0][r]);
      float s1 = xsum32(sacc[1][r]);
      s0 = (t0 + n < span_count) ? s0 * a.key_scale : -INFINITY;
      s1 = (t0 + n + 16 < span_count) ? s1 * a.key_scale : -INFINITY;
      sc[0][r] = s0;
      sc[1][r] = s1;
      m_w[r] = row16_max(fmaxf(s0, s1));
    }
  }

  // ---- probabilities against the wave's peak; the blend with A =
  // probabilities (row n: head n & 7, hi/lo), k = positions 8g .. 8g+7.
  float l_w[4];
  float4_t o[TILES];
#pragma unroll
  for (int t = 0; t < TILES; ++t) o[t] = float4_t{0, 0, 0, 0};
  uint8_t *vw = vs + wave * kWaveV;
  {
    float p[2][4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      p[0][r] = live ? __expf(sc[0][r] - m_w[r]) : 0.0f;
      p[1][r] = live ? __expf(sc[1][r] - m_w[r]) : 0.0f;
      l_w[r] = row16_sum(p[0][r] + p[1][r]);
    }
    if (g < 2) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        ps[wave][4 * g + r][n] = p[0][r];
        ps[wave][4 * g + r][n + 16] = p[1][r];
      }
    }
    if (live) {
      uint2_t *dst = reinterpret_cast<uint2_t *>(vw + (lane >> 1) * VPITCH + (lane & 1) * (HEAD / 2));
#pragma unroll
      for (int q = 0; q < HEAD / 16; ++q) dst[q] = vr[q];
    }
    // Only this wave's rows of `ps` and `vs` are read below: a wave barrier.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (live) {
      half8_t pa;
      {
        const float *src = &ps[wave][n & 7][8 * g];
        const bool lo_part = n >= 8;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float v = src[e];
          const _Float16 hi = (_Float16)v;
          pa[e] = lo_part ? (_Float16)(v - (float)hi) : hi;
        }
      }
#pragma unroll
      for (int qd = 0; qd < QUADS; ++qd) {
        uint32_t dw[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          dw[e] = *reinterpret_cast<const uint32_t *>(vw + (8 * g + e) * VPITCH + 64 * qd + 4 * n);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          uint32_t w[4];
          const uint32_t sel = 0x0C000C00u | ((uint32_t)(4 + t) << 16) | (uint32_t)t;
#pragma unroll
          for (int pr = 0; pr < 4; ++pr)
            w[pr] = decode_pair<FMT>(__builtin_amdgcn_perm(dw[2 * pr + 1], dw[2 * pr], sel));
          o[4 * qd + t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, __builtin_bit_cast(half8_t, w),
                                                                 o[4 * qd + t], 0, 0, 0);
        }
      }
    }
  }
  // hi + lo rows
#pragma unroll
  for (int t = 0; t < TILES; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) o[t][r] = xsum32(o[t][r]);
  if (g < 2 && n == 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      wm[wave][4 * g + r] = m_w[r];
      wl[wave][4 * g + r] = l_w[r];
    }
  }

  // ---- merge the W waves: scale each by e^(m_w - M) per head.
  __syncthreads();  // wm, wl written and every wave done with vs, reused as float[W][8][HEAD]
  auto peak_of = [&](int h) {
    float M = wm[0][h];
#pragma unroll
    for (int w = 1; w < W; ++w) M = fmaxf(M, wm[w][h]);
    return M;
  };
  if (tid < kAttendGroup) {
    const int h = tid;
    const float M = peak_of(h);
    float L = 0.0f;
#pragma unroll
    for (int w = 0; w < W; ++w)
      if (wm[w][h] != -INFINITY) L += wl[w][h] * __expf(wm[w][h] - M);
    head_peak[h] = M;
    head_norm[h] = L;
  }
  float *ob = reinterpret_cast<float *>(vs);
  {
    float scale[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int h = 4 * (g & 1) + r;
      const float M = peak_of(h);
      scale[r] = m_w[r] != -INFINITY ? __expf(m_w[r] - M) : 0.0f;
    }
    if (g < 2) {
#pragma unroll
      for (int qd = 0; qd < QUADS; ++qd)
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            ob[(wave * kAttendGroup + 4 * g + r) * HEAD + 64 * qd + 4 * n + t] = o[4 * qd + t][r] * scale[r];
    }
  }
  __syncthreads();
  if (a.final_out) {
    // The block saw every visible position: normalize and write the blend.
    float *out = a.final_out + (size_t)lane_id * a.q_stride + (size_t)head0 * HEAD;
    for (int i = tid; i < kAttendGroup * HEAD; i += kThreads) {
      const int h = i / HEAD;
      const int d = i - h * HEAD;
      const float L = head_norm[h];
      float v = ob[h * HEAD + d];
#pragma unroll
      for (int w = 1; w < W; ++w) v += ob[(w * kAttendGroup + h) * HEAD + d];
      out[(size_t)h * HEAD + d] = L > 0.0f ? v * a.value_scale * (1.0f / L) : 0.0f;
    }
    return;
  }
  for (int i = tid; i < kAttendGroup * HEAD; i += kThreads) {
    const int h = i / HEAD;
    const int d = i - h * HEAD;
    float v = ob[h * HEAD + d];
#pragma unroll
    for (int w = 1; w < W; ++w) v += ob[(w * kAttendGroup + h) * HEAD + d];
    a.part_out[((size_t)pc * a.head_count + head0 + h) * HEAD + d] = v * a.value_scale;
  }
  if (tid < kAttendGroup) {
    a.part_peak[(size_t)pc * a.head_count + head0 + tid] = head_peak[tid];
    a.part_total[(size_t)pc * a.head_count + head0 + tid] = head_norm[tid];
  }
}

// Merges chunk partials.  One workgroup per (head, lane, 64 dims): the
// chunk weights e^(peak_c - peak) once in LDS, then thread (d, slice) sums
// chunks c = slice (mod 4) of dim d, 32 loads in flight, and the four slices
// are added in a fixed order, so the result does not depend on timing.
__global__ __launch_bounds__(256) void attend_merge_kernel(const float *part_out_all,
                                                           const float *part_peak_all,
                                                           const float *part_total_all,
                                                           int chunk_slots, int chunk,
                                                           int place0, const int *place_dev,
                                                           int window, int head_count,
                                                           int head_size, float *blend_all,
                                                           int o_stride) {
  extern __shared__ float wgt[];  // [chunks]
  __shared__ float red[4];
  __shared__ float slice_sum[4][64];
  const int h = blockIdx.x;
  const int lane_id = blockIdx.y;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int pos = (place_dev ? *place_dev : place0) + lane_id;
  const int span = window > 0 ? min(pos + 1, window) : pos + 1;
  // the workgroups that saw part of this lane's span
  const int chunks = (span + chunk - 1) / chunk;
  const size_t base = (size_t)lane_id * chunk_slots;
  const float *part_out = part_out_all + base * head_count * head_size;
  const float *part_peak = part_peak_all + base * head_count;
  const float *part_total = part_total_all + base * head_count;
  float *blend_out = blend_all + (size_t)lane_id * o_stride;
  float peak = -INFINITY;
  for (int c = tid; c < chunks; c += 256) peak = fmaxf(peak, part_peak[(size_t)c * head_count + h]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) peak = fmaxf(peak, __shfl_xor(peak, o));
  if ((tid & 63) == 0) red[wave] = peak;
  __syncthreads();
  peak = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float total = 0.0f;
  for (int c = tid; c < chunks; c += 256) {
    const float m = part_peak[(size_t)c * head_count + h];
    const float wv = m == -INFINITY ? 0.0f : __expf(m - peak);
    wgt[c] = wv;
    total += wv * part_total[(size_t)c * head_count + h];
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) total += __shfl_xor(total, o);
  if ((tid & 63) == 0) red[wave] = total;
  __syncthreads();  // also: wgt complete
  total = ((red[0] + red[1]) + red[2]) + red[3];
  const float inv = total > 0.0f ? 1.0f / total : 0.0f;
  const int d = blockIdx.z * 64 + (tid & 63);
  const int slice = wave;
  const float *col = part_out + (size_t)h * head_size + d;
  const size_t step = (size_t)head_count * head_size;
  // 32 chunks of the slice at a time, every load issued before the sums
  // (past the end: the last chunk again, weight 0)
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int c0 = slice; c0 < chunks; c0 += 128) {
    float v[32];
#pragma unroll
    for (int u = 0; u < 32; ++u) v[u] = col[(size_t)min(c0 + 4 * u, chunks - 1) * step];
#pragma unroll
    for (int u = 0; u < 32; ++u) {
      const int c = c0 + 4 * u;
      acc[u & 7] += (c < chunks ? wgt[c] : 0.0f) * v[u];
    }
  }
  slice_sum[slice][tid & 63] =
      ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
  __syncthreads();
  if (slice == 0 && d < head_size)
    blend_out[(size_t)h * head_size + d] =
        (((slice_sum[0][tid] + slice_sum[1][tid]) + slice_sum[2][tid]) + slice_sum[3][tid]) * inv;
}

}  // namespace igl

using namespace igl;

static int attend_max_span(int place0, int window, int lanes) {
  const int last = place0 + lanes;  // span of the last lane when unwindowed
  return window > 0 ? (last < window ? last : window) : last;
}

static int attend_waves(int place0, int window, int lanes) {
  return attend_max_span(place0, window, lanes) <= kAttendShortSpan ? 1 : 4;
}

static int attend_blocks(int place0, int window, int lanes) {
  const int chunk = attend_waves(place0, window, lanes) * kAttendTile;
  return (attend_max_span(place0, window, lanes) + chunk - 1) / chunk;
}

template <int HEAD, int FMT, int W>
static void attend_launch(const AttendArgs &a, dim3 grid, bool qvec, hipStream_t stream) {
  if (qvec)
    hipLaunchKernelGGL((attend_mfma_kernel<HEAD, FMT, true, W>), grid, dim3(64 * W), 0, stream, a);
  else
    hipLaunchKernelGGL((attend_mfma_kernel<HEAD, FMT, false, W>), grid, dim3(64 * W), 0, stream, a);
}

// `lanes` query lanes at positions place0 .. place0 + lanes - 1, each seeing
// the last `window` positions up to its own (0: every position from 0).  Lane
// l's query and output are `q_stride` floats after lane l - 1's.  With
// `place_dev`, lane 0's position is read from device memory when the kernels
// run and `place0` is only its upper bound, which sizes the grid (a launch
// that a graph replays at every step).
extern "C" hipError_t igl_launch_attend(const uint8_t *key_store, const uint8_t *value_store,
                                        int fmt, float key_scale, float value_scale,
                                        int cache_span, int kv_width, int kv_count,
                                        int group_share, int head_size, const float *query,
                                        int q_stride, int place0, const int *place_dev,
                                        int window, int lanes, float score_scale,
                                        float *blend_out, float *work, hipStream_t stream) {
  AttendArgs a;
  const int waves = attend_waves(place0, window, lanes);
  const int chunks = attend_blocks(place0, window, lanes);  // workgroups a lane
  const int head_count = kv_count * group_share;
  if (group_share != kAttendGroup || lanes < 1) return hipErrorInvalidValue;
  a.key_store = key_store;
  a.value_store = value_store;
  a.kv_width = kv_width;
  a.cache_span = cache_span;
  a.place0 = place0;
  a.place_dev = place_dev;
  a.window = window;
  a.chunks = chunks;
  a.final_out = chunks == 1 ? blend_out : nullptr;
  a.q_stride = q_stride;
  a.query = query;
  // e4m3 decodes to real8 / 256; the 256 goes back in with the scale.
  const float unit = fmt == 0 ? 256.0f : 1.0f;
  a.key_scale = key_scale * unit * score_scale;
  a.value_scale = value_scale * unit;
  a.head_count = head_count;
  const size_t slots = (size_t)lanes * chunks;
  a.part_out = work;
  a.part_peak = work + slots * head_count * head_size;
  a.part_total = a.part_peak + slots * head_count;
  dim3 grid(chunks, kv_count, lanes);
  const bool qvec = (((uintptr_t)query) & 15u) == 0 && (q_stride & 3) == 0;
  if (head_size == 256 && fmt == 0)
    waves == 1 ? attend_launch<256, 0, 1>(a, grid, qvec, stream) : attend_launch<256, 0, 4>(a, grid, qvec, stream);
  else if (head_size == 256 && fmt == 1)
    waves == 1 ? attend_launch<256, 1, 1>(a, grid, qvec, stream) : attend_launch<256, 1, 4>(a, grid, qvec, stream);
  else if (head_size == 512 && fmt == 0)
    waves == 1 ? attend_launch<512, 0, 1>(a, grid, qvec, stream) : attend_launch<512, 0, 4>(a, grid, qvec, stream);
  else if (head_size == 512 && fmt == 1)
    waves == 1 ? attend_launch<512, 1, 1>(a, grid, qvec, stream) : attend_launch<512, 1, 4>(a, grid, qvec, stream);
  else
    return hipErrorInvalidValue;
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || chunks == 1) return e;
  hipLaunchKernelGGL(attend_merge_kernel, dim3(head_count, lanes, (head_size + 63) / 64), dim3(256),
                     chunks * sizeof(float), stream, a.part_out, a.part_peak, a.part_total, chunks,
                     waves * kAttendTile, place0, place_dev, window, head_count, head_size, blend_out,
                     q_stride);
  return hipGetLastError();
}

// Floats of workspace igl_launch_attend needs for the same arguments.
extern "C" size_t igl_attend_work_floats(int place0, int window, int lanes, int head_count,
                                         int head_size) {
  const size_t blocks = (size_t)attend_blocks(place0, window, lanes);
  return (size_t)lanes * blocks * (size_t)head_count * ((size_t)head_size + 2);
}

// Floats of workspace enough for every igl_launch_attend call of at most
// `lanes` lanes whose spans stay within `span_limit` positions.  The chunk
// count is not monotonic in the span: chunks are kAttendTile positions up to
// kAttendShortSpan and four times that beyond, so a span just under
// kAttendShortSpan has more chunks than one just over it.  The largest count
// of each regime is taken.
extern "C" size_t igl_attend_work_floats_limit(int span_limit, int lanes, int head_count,
                                               int head_size) {
  if (span_limit < 1 || lanes < 1) return 0;
  const int short_top = span_limit < kAttendShortSpan ? span_limit : kAttendShortSpan;
  const int b_short = attend_blocks(short_top - 1, 0, 1);
  const int b_long = attend_blocks(span_limit - 1, 0, 1);
  const size_t blocks = (size_t)(b_short > b_long ? b_short : b_long);
  return (size_t)lanes * blocks * (size_t)head_count * ((size_t)head_size + 2);
}

// ---- the workspace of the entry that allocates nothing ---------------------
//
// igl_attend_lanes_fixed_dev writes its chunk partials here instead of into
// the desk's grow-only workspace.  One copy of the array lives on each GPU the
// library runs on, until the process ends.  On the host, `scratch` names a
// stand-in, not device memory: host code passes the address that
// hipGetSymbolAddress gives for the current device, resolved once per device
// (igl_attend_fixed_resolve, called by igl_back_open with that device current).
static __device__ __align__(256) float scratch[IGL_ATTEND_FIXED_FLOATS];

namespace {
constexpr int kFixedDevices = 64;
std::mutex fixed_lock;
float *fixed_ptr[kFixedDevices];
}  // namespace

extern "C" hipError_t igl_attend_fixed_resolve(int device) {
  if (device < 0 || device >= kFixedDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> hold(fixed_lock);
  if (fixed_ptr[device]) return hipSuccess;
  void *ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return e;
  fixed_ptr[device] = static_cast<float *>(ptr);
  return hipSuccess;
}

extern "C" float *igl_attend_fixed_ptr(int device) {
  if (device < 0 || device >= kFixedDevices) return nullptr;
  std::lock_guard<std::mutex> hold(fixed_lock);
  return fixed_ptr[device];
}
