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
// Work layout (flash-decoding): a lane's span is cut into chunks of C
// positions (32 up to kAttendShortSpan, 64 beyond), one workgroup of four
// waves a chunk.  The two products split the chunk differently among the
// waves, so each wave's dependent chain is a quarter of the chunk's work:
// scores by positions (wave w: C/4 positions over every dim), the blend by
// dims (wave w: a quarter of the dims over every position).  A span of one
// chunk is written directly; otherwise each chunk writes a partial (blend,
// peak, total) and attend_fold_kernel folds them in one memory round trip.
//
// (Measured on the box, one launch pair inside a graph: a 512-position
// sliding window of 256-dim heads takes 9.5 us, of which 4.9 us is the chunk
// kernel and 1.55 us the bare cost of each dependent launch; the former form,
// one wave per 32 positions over every dim with a cross-wave merge, took 6.9
// us for the same chunks.  A last-workgroup fold in the same kernel, after an
// agent-scope release/acquire ticket, was slower at every chunk count tried:
// 10.5 us at 8 chunks, over 100 us at 256.)
#include <mutex>

#include "igl_backend.h"
#include "igl_device.h"

namespace igl {

// Positions a chunk, by the longest span a launch covers: 32 up to
// kAttendShortSpan (the most workgroups, the shortest chain each), 64 beyond
// (half the partials: at 16384 positions 11.4 us against 13.0 us for 32).
// Launches of kAttendWideLanes lanes and more take 64 whatever the span: a
// prefill pass has workgroups enough, and half the partials to fold (the
// 2047-lane fast prefill 46 700 -> 49 300 tok/s with it on windowed spans,
// 52 400 with it on every span; one lane keeps 32: its sliding window
// measured 6.8 against 7.3 us with 64).
constexpr int kAttendShortSpan = 8192;
constexpr int kAttendWideLanes = 64;
constexpr int kAttendGroup = 8;                    // query heads per key/value head
constexpr int kAttendPrepLanes = 4;                // lanes of one prepared launch

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
  // The heads of a decode step or a small block prepared here
  // (attend_split_kernel's PREP form): `query` holds the query heads before
  // their norm; q_gain their gain; turn, lane by lane, the (cos, sin) of the
  // lane's position times each rotation step, HEAD / 2 pairs.  With k_raw
  // set, the block's new positions place .. place + l (lane l's, and the
  // lanes' before it) get a workgroup of lane l's own after the chunks of the
  // positions before the block (attend_fresh_rows): it prepares their key and
  // value heads (norm and gain and turn; norm), writes lane l's bytes into
  // ring slot (place + l) % cache_span of k_ring / v_ring (the rings read
  // here), code = e4m3(value / scale), and writes the partial of those
  // positions; the chunk workgroups never read those slots.
  const float *q_gain;
  const float *turn;           // [lanes][HEAD / 2][2]
  int turn_stride;             // floats between lanes of turn
  const float *k_raw;          // [lanes][kv_raw_stride], as v_raw
  int kv_raw_stride;
  const float *v_raw;
  const float *k_gain;
  uint8_t *k_ring;
  uint8_t *v_ring;
  float k_code_scale;
  float v_code_scale;
  float eps;
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

// The block's new positions seen by lane l, pos0 .. pos0 + l, a workgroup of
// the lane's own (PREP with k_raw): the key and value heads of each new
// position prepared (norm, gain, turn; norm), lane l writing only its own
// position's bytes to the rings (lanes before it write theirs, from the same
// arithmetic on the same inputs); the lane's 8 query heads prepared as every
// chunk prepares them; and one partial over those l + 1 positions: score_h,j
// = key_scale q_h . key_j(bytes) in fp32, peak_h = max_j score_h,j, total_h =
// sum_j e^(score_h,j - peak_h), blend_h = sum_j e^(score_h,j - peak_h)
// value_j(bytes) value_scale (one position: peak = its score, total 1, blend
// its value).  Off the path of the chunk workgroups, which end before it.
template <int HEAD>
__device__ __forceinline__ void attend_fresh_rows(const AttendArgs &a, int pos0, int l, int pc) {
  constexpr int HALF = HEAD / 2;
  constexpr int W = 4;
  constexpr int F = kAttendPrepLanes;
  constexpr int kHeadItems = HEAD / 8;
  constexpr int kQItems = kAttendGroup * HEAD / 8 / 256;
  __shared__ double nr_red[F][2][W];
  __shared__ __attribute__((aligned(16))) uint8_t nr_bytes[F][2][HEAD];
  __shared__ float nr_score[kAttendGroup][F];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int rows = l + 1;  // uniform, at most F
  // every load first: the key/value pairs of the thread (threads below
  // HALF) of each new position, then its query items with their gains and
  // turns
  float kx[F][2], vx[F][2], kt[F][2], kg[2] = {0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < F; ++j) {
    kx[j][0] = kx[j][1] = vx[j][0] = vx[j][1] = kt[j][0] = kt[j][1] = 0.0f;
  }
  if (tid < HALF) {
    kg[0] = a.k_gain[tid];
    kg[1] = a.k_gain[tid + HALF];
#pragma unroll
    for (int j = 0; j < F; ++j) {
      if (j < rows) {
        const float *kr = a.k_raw + (size_t)j * a.kv_raw_stride;
        const float *vr = a.v_raw + (size_t)j * a.kv_raw_stride;
        const float *tr = a.turn + (size_t)j * a.turn_stride;
        kx[j][0] = kr[tid];
        kx[j][1] = kr[tid + HALF];
        vx[j][0] = vr[tid];
        vx[j][1] = vr[tid + HALF];
        kt[j][0] = tr[2 * tid];
        kt[j][1] = tr[2 * tid + 1];
      }
    }
  }
  float qf[kQItems][8];
  float4_t qgain[kQItems][2], qturn[kQItems][4];
  const float *own_turn = a.turn + (size_t)l * a.turn_stride;
#pragma unroll
  for (int i = 0; i < kQItems; ++i) {
    const int item = tid + 256 * i;
    const float4_t *q = reinterpret_cast<const float4_t *>(a.query + (size_t)l * a.q_stride + 8 * item);
    const float4_t u = q[0], v = q[1];
    qf[i][0] = u.x; qf[i][1] = u.y; qf[i][2] = u.z; qf[i][3] = u.w;
    qf[i][4] = v.x; qf[i][5] = v.y; qf[i][6] = v.z; qf[i][7] = v.w;
    const int d0 = 8 * (item % kHeadItems);
    const int j0 = d0 < HALF ? d0 : d0 - HALF;
    qgain[i][0] = *reinterpret_cast<const float4_t *>(a.q_gain + d0);
    qgain[i][1] = *reinterpret_cast<const float4_t *>(a.q_gain + d0 + 4);
#pragma unroll
    for (int w = 0; w < 4; ++w) qturn[i][w] = *reinterpret_cast<const float4_t *>(own_turn + 2 * j0 + 4 * w);
  }
  // keys: norm, gain, turn; values: norm (session_attend 11504-11510), every
  // new position's sums behind one barrier
  {
#pragma unroll
    for (int j = 0; j < F; ++j) {
      if (j < rows) {
        double ks = (double)kx[j][0] * (double)kx[j][0] + (double)kx[j][1] * (double)kx[j][1];
        double vs2 = (double)vx[j][0] * (double)vx[j][0] + (double)vx[j][1] * (double)vx[j][1];
        ks = wave_sum_f64_to_last(ks);
        vs2 = wave_sum_f64_to_last(vs2);
        if (lane == 63) {
          nr_red[j][0][wave] = ks;
          nr_red[j][1][wave] = vs2;
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < F; ++j) {
      if (j < rows) {
        double kt_sum = nr_red[j][0][0], vt_sum = nr_red[j][1][0];
#pragma unroll
        for (int w = 1; w < W; ++w) {
          kt_sum += nr_red[j][0][w];
          vt_sum += nr_red[j][1][w];
        }
        if (tid < HALF) {
          const float ksh = rms_shrink(kt_sum, HEAD, a.eps);
          const float vsh = rms_shrink(vt_sum, HEAD, a.eps);
          float lo = kx[j][0] * ksh, hi = kx[j][1] * ksh;
          lo = lo * kg[0];
          hi = hi * kg[1];
          const float k0 = lo * kt[j][0] - hi * kt[j][1];
          const float k1 = hi * kt[j][0] + lo * kt[j][1];
          const uint8_t b0 = e4m3_code(k0 / a.k_code_scale), b1 = e4m3_code(k1 / a.k_code_scale);
          const uint8_t c0b = e4m3_code(vx[j][0] * vsh / a.v_code_scale);
          const uint8_t c1b = e4m3_code(vx[j][1] * vsh / a.v_code_scale);
          if (j == l) {
            const size_t row = (size_t)((pos0 + l) % a.cache_span) * a.kv_width;
            a.k_ring[row + tid] = b0;
            a.k_ring[row + tid + HALF] = b1;
            a.v_ring[row + tid] = c0b;
            a.v_ring[row + tid + HALF] = c1b;
          }
          nr_bytes[j][0][tid] = b0;
          nr_bytes[j][0][tid + HALF] = b1;
          nr_bytes[j][1][tid] = c0b;
          nr_bytes[j][1][tid + HALF] = c1b;
        }
      }
    }
  }
  __syncthreads();
  // the query heads as the chunks prepare them, then each item's share of
  // its head's score against each new position's decoded key bytes
#pragma unroll
  for (int i = 0; i < kQItems; ++i) {
    const int item = tid + 256 * i;
    const int h = item / kHeadItems;
    const int d0 = 8 * (item % kHeadItems);
    double ss = 0.0;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += (double)qf[i][e] * (double)qf[i][e];
#pragma unroll
    for (int off = kHeadItems / 2; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    const float shrink = rms_shrink(ss, HEAD, a.eps);
    const float gg[8] = {qgain[i][0].x, qgain[i][0].y, qgain[i][0].z, qgain[i][0].w,
                         qgain[i][1].x, qgain[i][1].y, qgain[i][1].z, qgain[i][1].w};
    float own[8], other[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      own[e] = qf[i][e] * shrink;
      own[e] = own[e] * gg[e];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) other[e] = __shfl_xor(own[e], kHeadItems / 2);
    const bool low = d0 < HALF;
    float qv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float c = qturn[i][e >> 1][2 * (e & 1)];
      const float sn = qturn[i][e >> 1][2 * (e & 1) + 1];
      qv[e] = low ? own[e] * c - other[e] * sn : own[e] * c + other[e] * sn;
    }
#pragma unroll
    for (int j = 0; j < F; ++j) {
      if (j < rows) {
        const uint2_t kb = *reinterpret_cast<const uint2_t *>(&nr_bytes[j][0][d0]);
        const half8_t kd = decode8<0>(kb.x, kb.y);
        float part = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) part = __builtin_fmaf(qv[e], (float)kd[e], part);
#pragma unroll
        for (int off = kHeadItems / 2; off > 0; off >>= 1) part += __shfl_xor(part, off);
        if (item % kHeadItems == 0) nr_score[h][j] = part * a.key_scale;
      }
    }
  }
  __syncthreads();
  // the partial: each head blends the new value rows, weighted against its peak
  for (int i = tid; i < kAttendGroup * HEAD / 8; i += 256) {
    const int h = i / (HEAD / 8);
    const int d0 = 8 * (i % (HEAD / 8));
    float peak = nr_score[h][0];
    for (int j = 1; j < rows; ++j) peak = fmaxf(peak, nr_score[h][j]);
    float o[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    for (int j = 0; j < rows; ++j) {
      const float wgt = __expf(nr_score[h][j] - peak);
      const uint2_t vb = *reinterpret_cast<const uint2_t *>(&nr_bytes[j][1][d0]);
      const half8_t vd = decode8<0>(vb.x, vb.y);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] += wgt * ((float)vd[e] * a.value_scale);
    }
    float *dst = a.part_out + ((size_t)pc * a.head_count + h) * HEAD + d0;
    *reinterpret_cast<float4_t *>(dst) = float4_t{o[0], o[1], o[2], o[3]};
    *reinterpret_cast<float4_t *>(dst + 4) = float4_t{o[4], o[5], o[6], o[7]};
  }
  if (tid < kAttendGroup) {
    float peak = nr_score[tid][0];
    for (int j = 1; j < rows; ++j) peak = fmaxf(peak, nr_score[tid][j]);
    float total = 0.0f;
    for (int j = 0; j < rows; ++j) total += __expf(nr_score[tid][j] - peak);
    a.part_peak[(size_t)pc * a.head_count + tid] = peak;
    a.part_total[(size_t)pc * a.head_count + tid] = total;
  }
}

// The split form.  A workgroup of four waves takes a chunk of C positions
// (32 or 64) of one lane.  The two products are split differently among the
// waves, so that each wave's dependent chain is a quarter of the chunk's work:
//   scores: wave w takes positions w*C/4 .. (w+1)*C/4 - 1 over every dim (its
//           key rows straight into MFMA operand order, as above);
//   blend:  wave w takes dims w*HEAD/4 .. (w+1)*HEAD/4 - 1 over every position
//           of the chunk (its slice of each value row staged in its own LDS).
// Between the two, the probabilities (against each wave's own peak) and the
// waves' peaks and sums go through LDS: one barrier.  Each wave then owns its
// dims of the output outright, so nothing is merged across waves.
template <int HEAD, int FMT, int C, bool QVEC, bool PREP>
__global__ __launch_bounds__(256) void attend_split_kernel(AttendArgs a) {
  constexpr int W = 4;                // waves
  constexpr int PW = C / W;           // positions a wave scores: 8 or 16
  constexpr int DS = HEAD / W;        // dims a wave blends: 64 or 128
  constexpr int S = HEAD / 32;        // k-steps of the score product
  constexpr int QD = HEAD / 4;        // bytes of a key row one lane group reads
  constexpr int QUADS = DS / 64;      // 64-dim groups of a wave's blend
  constexpr int KS = C / 32;          // k-steps of the blend (32 positions each)
  constexpr int VP = DS + 8;          // staged value row pitch in bytes (8-byte aligned rows)
  constexpr int LPR = DS / 16;        // lanes that load one value row (16 bytes each)
  constexpr int RPI = 64 / LPR;       // value rows one load instruction covers
  constexpr int VL = C / RPI;         // value loads a lane issues
  static_assert(PW == 8 || PW == 16, "chunk of 32 or 64 positions");
  static_assert(!PREP || (FMT == 0 && QVEC), "prepared heads: e4m3 rings, aligned queries");
  constexpr int HALF = HEAD / 2;

  __shared__ half8_t qs[2][kAttendGroup][HEAD / 8];
  __shared__ float ps[kAttendGroup][C];
  __shared__ __attribute__((aligned(16))) float wm[W][kAttendGroup];
  __shared__ __attribute__((aligned(16))) float wl[W][kAttendGroup];
  __shared__ __attribute__((aligned(16))) uint8_t vs[W][C * VP];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 4;
  const int n = lane & 15;
  const int kv = blockIdx.y;
  const int head0 = kv * kAttendGroup;
  const int block = blockIdx.x;
  const int lane_id = blockIdx.z;
  const int pos0 = a.place_dev ? *a.place_dev : a.place0;
  const int pos = pos0 + lane_id;
  const int span_full = a.window > 0 ? min(pos + 1, a.window) : pos + 1;
  const int place_start = pos - span_full + 1;
  // PREP with k_raw: the block's new positions up to the lane's own are the
  // workgroup after the chunks, which cover the positions before the block
  // (lane_id + 1 <= kAttendPrepLanes is inside every window)
  const bool new_row = PREP && a.k_raw != nullptr;
  const int span_count = new_row ? span_full - (lane_id + 1) : span_full;
  const int blocks_seen = (span_count + C - 1) / C;
  const int pc = lane_id * a.chunks + block;
  if (new_row && block == blocks_seen) {
    if (PREP) attend_fresh_rows<HEAD>(a, pos0, lane_id, pc);
    return;
  }
  if (block >= blocks_seen) return;  // past this lane's span: the whole workgroup
  const size_t kv_off = (size_t)kv * HEAD;
  const int c0 = block * C;  // the chunk's first position (relative to place_start)
  // ring slot of relative position t: (place_start + t) % cache_span, from one
  // uniform remainder (0 <= t < span <= cache_span, so one wrap at most)
  const int ring0 = place_start % a.cache_span;
  auto ring_slot = [&](int t) {
    const int slot = ring0 + t;
    return slot >= a.cache_span ? slot - a.cache_span : slot;
  };

  // ---- loads, all issued before the first wait
  constexpr int kQTotal = kAttendGroup * HEAD / 8;
  constexpr int kQItems = kQTotal / 256;
  float qf[kQItems][8];
  {
    const float *qb = a.query + (size_t)lane_id * a.q_stride + (size_t)head0 * HEAD;
#pragma unroll
    for (int i = 0; i < kQItems; ++i) {
      const float *q = qb + 8 * (tid + 256 * i);
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
  // PREP: the gains and turns of the thread's query dims, requested with the
  // query itself (one round trip, not two): item i covers dims d0 .. d0 + 7 of
  // its head, whose turn pairs j0 .. j0 + 7 are 16 consecutive floats.
  constexpr int kHeadItems = HEAD / 8;
  float4_t qgain[PREP ? kQItems : 1][2];
  float4_t qturn[PREP ? kQItems : 1][4];
  if (PREP) {
#pragma unroll
    for (int i = 0; i < kQItems; ++i) {
      const int d0 = 8 * ((tid + 256 * i) % kHeadItems);
      const int j0 = d0 < HALF ? d0 : d0 - HALF;
      qgain[i][0] = *reinterpret_cast<const float4_t *>(a.q_gain + d0);
      qgain[i][1] = *reinterpret_cast<const float4_t *>(a.q_gain + d0 + 4);
#pragma unroll
      for (int v = 0; v < 4; ++v)
        qturn[i][v] = *reinterpret_cast<const float4_t *>(a.turn + (size_t)lane_id * a.turn_stride + 2 * j0 + 4 * v);
    }
  }
  // key row: position c0 + wave*PW + (n % PW), bytes QD*g .. QD*g + QD - 1
  const int tk = c0 + wave * PW + (n % PW);
  uint4_t kr[QD / 16];
  {
    const int t = min(tk, span_count - 1);
    const int slot = ring_slot(t);
    const uint4_t *row =
        reinterpret_cast<const uint4_t *>(a.key_store + (size_t)slot * a.kv_width + kv_off + QD * g);
#pragma unroll
    for (int q = 0; q < QD / 16; ++q) kr[q] = __builtin_nontemporal_load(row + q);
  }
  // value rows: row (lane / LPR) + RPI*i of the chunk, bytes of dims
  // wave*DS + 16*(lane % LPR) .. + 15
  uint4_t vr[VL];
#pragma unroll
  for (int i = 0; i < VL; ++i) {
    const int t = min(c0 + lane / LPR + RPI * i, span_count - 1);
    const int slot = ring_slot(t);
    vr[i] = __builtin_nontemporal_load(reinterpret_cast<const uint4_t *>(
        a.value_store + (size_t)slot * a.kv_width + kv_off + wave * DS + 16 * (lane % LPR)));
  }

  if (PREP) {
    // Each head's items are 32 (HEAD 256) or 64 (HEAD 512) consecutive
    // threads; the pair (j, j + HALF) of a dim sits HALF / 8 items apart.
#pragma unroll
    for (int i = 0; i < kQItems; ++i) {
      const int item = tid + 256 * i;
      const int d0 = 8 * (item % kHeadItems);
      double ss = 0.0;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += (double)qf[i][e] * (double)qf[i][e];
#pragma unroll
      for (int off = kHeadItems / 2; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
      const float shrink = rms_shrink(ss, HEAD, a.eps);
      float own[8], other[8];
      const float4_t g0 = qgain[i][0], g1 = qgain[i][1];
      const float gg[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        own[e] = qf[i][e] * shrink;
        own[e] = own[e] * gg[e];
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) other[e] = __shfl_xor(own[e], kHeadItems / 2);
      const bool low = d0 < HALF;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float c = qturn[i][e >> 1][2 * (e & 1)];
        const float sn = qturn[i][e >> 1][2 * (e & 1) + 1];
        qf[i][e] = low ? own[e] * c - other[e] * sn : own[e] * c + other[e] * sn;
      }
    }
  }

  // query operands, x = hi + lo in binary16
#pragma unroll
  for (int i = 0; i < kQItems; ++i) {
    half8_t hi8, lo8;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const _Float16 hi = (_Float16)qf[i][e];
      hi8[e] = hi;
      lo8[e] = (_Float16)(qf[i][e] - (float)hi);
    }
    const int item = tid + 256 * i;
    qs[0][item / (HEAD / 8)][item % (HEAD / 8)] = hi8;
    qs[1][item / (HEAD / 8)][item % (HEAD / 8)] = lo8;
  }
  __syncthreads();

  // ---- scores of the wave's PW positions for the 8 heads, all dims
  float sc[4];
  float m_w[4];
  {
    float4_t sacc = float4_t{0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const half8_t qa = qs[n >> 3][n & 7][QD * g / 8 + s];
      const uint4_t w = kr[s >> 1];
      const half8_t kb = (s & 1) ? decode8<FMT>(w[2], w[3]) : decode8<FMT>(w[0], w[1]);
      sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa, kb, sacc, 0, 0, 0);
    }
    const bool valid = n < PW && tk < span_count;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float v = xsum32(sacc[r]);
      sc[r] = valid ? v * a.key_scale : -INFINITY;
      m_w[r] = row16_max(sc[r]);
    }
  }
  // probabilities against the wave's peak, and the wave's sums
  {
    float l_w[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float p = m_w[r] != -INFINITY && sc[r] != -INFINITY ? __expf(sc[r] - m_w[r]) : 0.0f;
      l_w[r] = row16_sum(p);
      if (g < 2 && n < PW) ps[4 * g + r][wave * PW + n] = p;
    }
    if (g < 2 && n == 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        wm[wave][4 * g + r] = m_w[r];
        wl[wave][4 * g + r] = l_w[r];
      }
    }
  }
  // the wave's value slice into its own LDS rows
  {
    uint8_t *vw = vs[wave];
#pragma unroll
    for (int i = 0; i < VL; ++i) {
      uint2_t *dst = reinterpret_cast<uint2_t *>(vw + (lane / LPR + RPI * i) * VP + 16 * (lane % LPR));
      dst[0] = uint2_t{vr[i][0], vr[i][1]};
      dst[1] = uint2_t{vr[i][2], vr[i][3]};
    }
  }
  __syncthreads();

  // ---- blend of the wave's dims over the chunk's positions.  A = the
  // probabilities (row n: head n & 7, hi part for n < 8, lo part otherwise;
  // k = positions 8g .. 8g + 7 of the k-step), each scaled by e^(m_w - M),
  // M the chunk's peak of the head.
  const int hh = n & 7;
  float M = wm[0][hh];
#pragma unroll
  for (int w = 1; w < W; ++w) M = fmaxf(M, wm[w][hh]);
  float4_t o[4 * QUADS];
#pragma unroll
  for (int t = 0; t < 4 * QUADS; ++t) o[t] = float4_t{0, 0, 0, 0};
  const uint8_t *vw = vs[wave];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const int p0 = 32 * ks + 8 * g;  // the lane's first position of the k-step
    const float mw = wm[p0 / PW][hh];
    const float f = mw != -INFINITY ? __expf(mw - M) : 0.0f;
    half8_t pa;
    {
      const float *src = &ps[hh][p0];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float v = src[e] * f;
        const _Float16 hi = (_Float16)v;
        pa[e] = n >= 8 ? (_Float16)(v - (float)hi) : hi;
      }
    }
#pragma unroll
    for (int qd = 0; qd < QUADS; ++qd) {
      uint32_t dw[8];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        dw[e] = *reinterpret_cast<const uint32_t *>(vw + (p0 + e) * VP + 64 * qd + 4 * n);
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
  // hi + lo rows; lanes g < 2 hold head 4g + r, dims wave*DS + 64qd + 4n + t
#pragma unroll
  for (int t = 0; t < 4 * QUADS; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) o[t][r] = xsum32(o[t][r]);
  if (g >= 2) return;
  // the waves' peaks and sums of heads 4g .. 4g + 3, read at once
  float4_t pk[W], tl[W];
#pragma unroll
  for (int w = 0; w < W; ++w) {
    pk[w] = *reinterpret_cast<const float4_t *>(&wm[w][4 * g]);
    tl[w] = *reinterpret_cast<const float4_t *>(&wl[w][4 * g]);
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int h = 4 * g + r;
    float Mh = pk[0][r];
#pragma unroll
    for (int w = 1; w < W; ++w) Mh = fmaxf(Mh, pk[w][r]);
    float L = 0.0f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float e = pk[w][r] != -INFINITY ? __expf(pk[w][r] - Mh) : 0.0f;
      L += tl[w][r] * e;
    }
    float *dst;
    float mul;
    if (a.final_out) {
      dst = a.final_out + (size_t)lane_id * a.q_stride + (size_t)(head0 + h) * HEAD + wave * DS + 4 * n;
      mul = L > 0.0f ? a.value_scale * (1.0f / L) : 0.0f;
    } else {
      dst = a.part_out + ((size_t)pc * a.head_count + head0 + h) * HEAD + wave * DS + 4 * n;
      mul = a.value_scale;
      if (wave == 0 && n == 0) {
        a.part_peak[(size_t)pc * a.head_count + head0 + h] = Mh;
        a.part_total[(size_t)pc * a.head_count + head0 + h] = L;
      }
    }
#pragma unroll
    for (int qd = 0; qd < QUADS; ++qd)
      *reinterpret_cast<float4_t *>(dst + 64 * qd) =
          float4_t{o[4 * qd][r] * mul, o[4 * qd + 1][r] * mul, o[4 * qd + 2][r] * mul, o[4 * qd + 3][r] * mul};
  }
}

// Wide launches (a prefill pass of kAttendWideLanes lanes or more): one
// workgroup a lane and key/value head walks the lane's chunks of 64 positions
// in order, each chunk's scores and blend computed as attend_split_kernel
// computes them, and merges them into a running peak, total and blend in
// registers (the online form of attend_fold_kernel's fold), so no partial goes
// to memory and no fold launch follows.  The lanes give the launch its
// workgroups, and the workgroups a CU holds hide each other's loads: three
// at 512-dim heads (the registers capped for it, as many as their LDS
// allows), four at 256.  Requesting the next chunk's bytes ahead in registers
// instead held one a CU and was slower (2047 lanes, 2048 positions, 512-dim
// heads: 955 against 667 us at two a CU, 596 at three; a 512 window of
// 256-dim heads: 146 against 114, 109).
template <int HEAD, int FMT, bool QVEC>
__global__ __launch_bounds__(256, 3) void attend_rows_kernel(AttendArgs a) {
  constexpr int C = 64;               // positions a chunk
  constexpr int W = 4;                // waves
  constexpr int PW = C / W;           // positions a wave scores
  constexpr int DS = HEAD / W;        // dims a wave blends: 64 or 128
  constexpr int S = HEAD / 32;        // k-steps of the score product
  constexpr int QD = HEAD / 4;        // bytes of a key row one lane group reads
  constexpr int QUADS = DS / 64;      // 64-dim groups of a wave's blend
  constexpr int KS = C / 32;          // k-steps of the blend
  constexpr int VP = DS + 8;          // staged value row pitch in bytes
  constexpr int LPR = DS / 16;        // lanes that load one value row
  constexpr int RPI = 64 / LPR;       // value rows one load instruction covers
  constexpr int VL = C / RPI;         // value loads a lane issues

  __shared__ half8_t qs[2][kAttendGroup][HEAD / 8];
  __shared__ float ps[kAttendGroup][C];
  __shared__ __attribute__((aligned(16))) float wm[W][kAttendGroup];
  __shared__ __attribute__((aligned(16))) float wl[W][kAttendGroup];
  __shared__ __attribute__((aligned(16))) uint8_t vs[W][C * VP];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 4;
  const int n = lane & 15;
  const int kv = blockIdx.y;
  const int head0 = kv * kAttendGroup;
  // the last lanes, with the most chunks, first: the workgroups are handed
  // out in grid order, and the long ones would otherwise start last
  const int lane_id = (int)gridDim.z - 1 - (int)blockIdx.z;
  const int pos0 = a.place_dev ? *a.place_dev : a.place0;
  const int pos = pos0 + lane_id;
  const int span = a.window > 0 ? min(pos + 1, a.window) : pos + 1;
  const int place_start = pos - span + 1;
  const int blocks = (span + C - 1) / C;
  const size_t kv_off = (size_t)kv * HEAD;
  const int ring0 = place_start % a.cache_span;
  auto ring_slot = [&](int t) {
    const int slot = ring0 + t;
    return slot >= a.cache_span ? slot - a.cache_span : slot;
  };
  // key row of chunk b: position b C + wave PW + n, bytes QD g .. QD g + QD - 1;
  // value rows: lane / LPR + RPI i, dims wave DS + 16 (lane % LPR) .. + 15
  auto load_keys = [&](int b, uint4_t (&kr)[QD / 16]) {
    const int t = min(b * C + wave * PW + n, span - 1);
    const uint4_t *row =
        reinterpret_cast<const uint4_t *>(a.key_store + (size_t)ring_slot(t) * a.kv_width + kv_off + QD * g);
#pragma unroll
    for (int q = 0; q < QD / 16; ++q) kr[q] = __builtin_nontemporal_load(row + q);
  };
  auto load_values = [&](int b, uint4_t (&vr)[VL]) {
#pragma unroll
    for (int i = 0; i < VL; ++i) {
      const int t = min(b * C + lane / LPR + RPI * i, span - 1);
      vr[i] = __builtin_nontemporal_load(reinterpret_cast<const uint4_t *>(
          a.value_store + (size_t)ring_slot(t) * a.kv_width + kv_off + wave * DS + 16 * (lane % LPR)));
    }
  };

  // ---- the query, once: x = hi + lo in binary16
  constexpr int kQItems = kAttendGroup * HEAD / 8 / 256;
  {
    float qf[kQItems][8];
    const float *qb = a.query + (size_t)lane_id * a.q_stride + (size_t)head0 * HEAD;
#pragma unroll
    for (int i = 0; i < kQItems; ++i) {
      const float *q = qb + 8 * (tid + 256 * i);
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
#pragma unroll
    for (int i = 0; i < kQItems; ++i) {
      half8_t hi8, lo8;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const _Float16 hi = (_Float16)qf[i][e];
        hi8[e] = hi;
        lo8[e] = (_Float16)(qf[i][e] - (float)hi);
      }
      const int item = tid + 256 * i;
      qs[0][item / (HEAD / 8)][item % (HEAD / 8)] = hi8;
      qs[1][item / (HEAD / 8)][item % (HEAD / 8)] = lo8;
    }
  }

  // running peak, total and blend of heads 4g + r (lanes g < 2), dims
  // wave DS + 64 qd + 4 n + t
  float run_m[4], run_l[4];
  float4_t run_o[4 * QUADS];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    run_m[r] = -INFINITY;
    run_l[r] = 0.0f;
  }
#pragma unroll
  for (int t = 0; t < 4 * QUADS; ++t) run_o[t] = float4_t{0, 0, 0, 0};

  uint4_t kr[QD / 16], vr[VL];
  const int hh = n & 7;
  for (int b = 0; b < blocks; ++b) {
    __syncthreads();  // the query in LDS; the chunk before done with ps, wm, wl, vs
    const int c0 = b * C;
    // requested after the barrier: before it, 709 against 667 us (2047 lanes,
    // 2048 positions, 512-dim heads)
    load_keys(b, kr);
    load_values(b, vr);
    // scores of the wave's PW positions for the 8 heads, all dims
    float sc[4], m_w[4];
    {
      float4_t sacc = float4_t{0, 0, 0, 0};
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const half8_t qa = qs[n >> 3][n & 7][QD * g / 8 + s];
        const uint4_t w = kr[s >> 1];
        const half8_t kb = (s & 1) ? decode8<FMT>(w[2], w[3]) : decode8<FMT>(w[0], w[1]);
        sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa, kb, sacc, 0, 0, 0);
      }
      const bool valid = c0 + wave * PW + n < span;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float v = xsum32(sacc[r]);
        sc[r] = valid ? v * a.key_scale : -INFINITY;
        m_w[r] = row16_max(sc[r]);
      }
    }
    {
      float l_w[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = m_w[r] != -INFINITY && sc[r] != -INFINITY ? __expf(sc[r] - m_w[r]) : 0.0f;
        l_w[r] = row16_sum(p);
        if (g < 2) ps[4 * g + r][wave * PW + n] = p;
      }
      if (g < 2 && n == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          wm[wave][4 * g + r] = m_w[r];
          wl[wave][4 * g + r] = l_w[r];
        }
      }
    }
    {
      uint8_t *vw = vs[wave];
#pragma unroll
      for (int i = 0; i < VL; ++i) {
        uint2_t *dst = reinterpret_cast<uint2_t *>(vw + (lane / LPR + RPI * i) * VP + 16 * (lane % LPR));
        dst[0] = uint2_t{vr[i][0], vr[i][1]};
        dst[1] = uint2_t{vr[i][2], vr[i][3]};
      }
    }
    __syncthreads();
    // blend of the wave's dims over the chunk, against the chunk's peak M
    float M = wm[0][hh];
#pragma unroll
    for (int w = 1; w < W; ++w) M = fmaxf(M, wm[w][hh]);
    float4_t o[4 * QUADS];
#pragma unroll
    for (int t = 0; t < 4 * QUADS; ++t) o[t] = float4_t{0, 0, 0, 0};
    const uint8_t *vw = vs[wave];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int p0 = 32 * ks + 8 * g;
      const float mw = wm[p0 / PW][hh];
      const float f = mw != -INFINITY ? __expf(mw - M) : 0.0f;
      half8_t pa;
      {
        const float *src = &ps[hh][p0];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float v = src[e] * f;
          const _Float16 hi = (_Float16)v;
          pa[e] = n >= 8 ? (_Float16)(v - (float)hi) : hi;
        }
      }
#pragma unroll
      for (int qd = 0; qd < QUADS; ++qd) {
        uint32_t dw[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          dw[e] = *reinterpret_cast<const uint32_t *>(vw + (p0 + e) * VP + 64 * qd + 4 * n);
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
#pragma unroll
    for (int t = 0; t < 4 * QUADS; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) o[t][r] = xsum32(o[t][r]);
    // merge the chunk (peak Mh, total L, blend o) into the running state
    if (g < 2) {
      float4_t pk[W], tl[W];
#pragma unroll
      for (int w = 0; w < W; ++w) {
        pk[w] = *reinterpret_cast<const float4_t *>(&wm[w][4 * g]);
        tl[w] = *reinterpret_cast<const float4_t *>(&wl[w][4 * g]);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float Mh = pk[0][r];
#pragma unroll
        for (int w = 1; w < W; ++w) Mh = fmaxf(Mh, pk[w][r]);
        float L = 0.0f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
          const float e = pk[w][r] != -INFINITY ? __expf(pk[w][r] - Mh) : 0.0f;
          L += tl[w][r] * e;
        }
        const float Mn = fmaxf(run_m[r], Mh);
        const float keep = run_m[r] != -INFINITY ? __expf(run_m[r] - Mn) : 0.0f;
        const float take = Mh != -INFINITY ? __expf(Mh - Mn) : 0.0f;
        run_l[r] = run_l[r] * keep + L * take;
#pragma unroll
        for (int t = 0; t < 4 * QUADS; ++t) run_o[t][r] = run_o[t][r] * keep + o[t][r] * take;
        run_m[r] = Mn;
      }
    }
  }
  if (g >= 2) return;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int h = 4 * g + r;
    const float mul = run_l[r] > 0.0f ? a.value_scale * (1.0f / run_l[r]) : 0.0f;
    float *dst = a.final_out + (size_t)lane_id * a.q_stride + (size_t)(head0 + h) * HEAD + wave * DS + 4 * n;
#pragma unroll
    for (int qd = 0; qd < QUADS; ++qd)
      *reinterpret_cast<float4_t *>(dst + 64 * qd) = float4_t{run_o[4 * qd][r] * mul, run_o[4 * qd + 1][r] * mul,
                                                              run_o[4 * qd + 2][r] * mul, run_o[4 * qd + 3][r] * mul};
  }
}

// Folds chunk partials in one memory round trip.  A workgroup per (head, lane,
// DIMS dims) of 256 threads: thread (d, s) loads, for up to PER chunks
// c = s, s + 256/DIMS, ..., its dim's partial and the chunk's peak and total
// together; the slices' peaks meet in LDS (the head's peak M), each thread
// weights its chunks by e^(peak_c - M), and the slices' sums meet in LDS in a
// fixed order.  Spans of more chunks than one pass holds take further passes,
// each rescaled to the running peak.
template <int DIMS, int PER>
__global__ __launch_bounds__(256) void attend_fold_kernel(const float *part_out_all,
                                                          const float *part_peak_all,
                                                          const float *part_total_all,
                                                          int chunk_slots, int chunk, int place0,
                                                          const int *place_dev, int window,
                                                          int extra, int head_count, int head_size,
                                                          float *blend_all, int o_stride) {
  constexpr int SL = 256 / DIMS;
  __shared__ float red_m[SL];
  __shared__ float red_a[SL][DIMS];
  __shared__ float red_l[SL];
  const int h = blockIdx.x, lane_id = blockIdx.y, tid = threadIdx.x;
  const int d = tid % DIMS, sl = tid / DIMS;
  const int pos = (place_dev ? *place_dev : place0) + lane_id;
  const int span = window > 0 ? min(pos + 1, window) : pos + 1;
  // extra: the block's new positions up to the lane's own have a partial of
  // their own, after the chunks of the positions before the block
  const int fresh = extra ? lane_id + 1 : 0;
  const int chunks = (span - fresh + chunk - 1) / chunk + (extra ? 1 : 0);
  const size_t base = (size_t)lane_id * chunk_slots;
  const size_t step = (size_t)head_count * head_size;
  const float *pout = part_out_all + base * step + (size_t)h * head_size + blockIdx.z * DIMS + d;
  const float *ppk = part_peak_all + base * head_count + h;
  const float *ptt = part_total_all + base * head_count + h;
  float run_m = -INFINITY, acc = 0.0f, tot = 0.0f;
  for (int c0 = 0; c0 < chunks; c0 += SL * PER) {
    float v[PER], m[PER], l[PER];
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int c = min(c0 + sl + SL * u, chunks - 1);
      v[u] = pout[(size_t)c * step];
      m[u] = ppk[(size_t)c * head_count];
      l[u] = ptt[(size_t)c * head_count];
    }
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < PER; ++u)
      if (c0 + sl + SL * u < chunks) mx = fmaxf(mx, m[u]);
    __syncthreads();  // red_m of the previous pass read by every thread
    if (d == 0) red_m[sl] = mx;
    __syncthreads();
    float M = run_m;
#pragma unroll
    for (int i = 0; i < SL; ++i) M = fmaxf(M, red_m[i]);
    if (M != -INFINITY && run_m != -INFINITY && M != run_m) {
      const float f = __expf(run_m - M);
      acc *= f;
      tot *= f;
    }
    run_m = M;
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const bool in = c0 + sl + SL * u < chunks && m[u] != -INFINITY;
      const float w = in ? __expf(m[u] - M) : 0.0f;
      acc += w * v[u];
      tot += w * l[u];
    }
  }
  red_a[sl][d] = acc;
  if (d == 0) red_l[sl] = tot;
  __syncthreads();
  if (sl == 0) {
    float A = 0.0f, T = 0.0f;
#pragma unroll
    for (int i = 0; i < SL; ++i) {
      A += red_a[i][d];
      T += red_l[i];
    }
    blend_all[(size_t)lane_id * o_stride + (size_t)h * head_size + blockIdx.z * DIMS + d] =
        T > 0.0f ? A * (1.0f / T) : 0.0f;
  }
}

}  // namespace igl

using namespace igl;

static int attend_max_span(int place0, int window, int lanes) {
  const int last = place0 + lanes;  // span of the last lane when unwindowed
  return window > 0 ? (last < window ? last : window) : last;
}

static int attend_chunk(int place0, int window, int lanes) {
  if (lanes >= kAttendWideLanes) return 64;
  return attend_max_span(place0, window, lanes) <= kAttendShortSpan ? 32 : 64;
}

static int attend_blocks(int place0, int window, int lanes) {
  const int chunk = attend_chunk(place0, window, lanes);
  return (attend_max_span(place0, window, lanes) + chunk - 1) / chunk;
}

template <int HEAD, int FMT, int C>
static void attend_launch(const AttendArgs &a, dim3 grid, bool qvec, hipStream_t stream) {
  if (qvec)
    hipLaunchKernelGGL((attend_split_kernel<HEAD, FMT, C, true, false>), grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((attend_split_kernel<HEAD, FMT, C, false, false>), grid, dim3(256), 0, stream, a);
}

template <int HEAD, int FMT>
static void attend_launch_rows(const AttendArgs &a, dim3 grid, bool qvec, hipStream_t stream) {
  if (qvec)
    hipLaunchKernelGGL((attend_rows_kernel<HEAD, FMT, true>), grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((attend_rows_kernel<HEAD, FMT, false>), grid, dim3(256), 0, stream, a);
}

template <int HEAD, int FMT>
static void attend_launch_chunk(const AttendArgs &a, dim3 grid, int chunk, bool qvec, hipStream_t stream) {
  if (chunk == 32)
    attend_launch<HEAD, FMT, 32>(a, grid, qvec, stream);
  else
    attend_launch<HEAD, FMT, 64>(a, grid, qvec, stream);
}

static hipError_t attend_fold(const AttendArgs &a, int chunks, int chunk, int place0,
                              const int *place_dev, int window, int lanes, int head_size,
                              float *blend_out, hipStream_t stream, int extra = 0);

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
  const int chunk = attend_chunk(place0, window, lanes);
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
  a.q_gain = a.turn = a.k_raw = a.v_raw = a.k_gain = nullptr;
  a.k_ring = a.v_ring = nullptr;
  a.k_code_scale = a.v_code_scale = a.eps = 0.0f;
  dim3 grid(chunks, kv_count, lanes);
  const bool qvec = (((uintptr_t)query) & 15u) == 0 && (q_stride & 3) == 0;
  if (lanes >= kAttendWideLanes && chunks > 1) {
    // a prefill pass: one workgroup a lane walks its chunks, no partials
    a.final_out = blend_out;
    const dim3 rows(1, kv_count, lanes);
    if (head_size == 256 && fmt == 0)
      attend_launch_rows<256, 0>(a, rows, qvec, stream);
    else if (head_size == 256 && fmt == 1)
      attend_launch_rows<256, 1>(a, rows, qvec, stream);
    else if (head_size == 512 && fmt == 0)
      attend_launch_rows<512, 0>(a, rows, qvec, stream);
    else if (head_size == 512 && fmt == 1)
      attend_launch_rows<512, 1>(a, rows, qvec, stream);
    else
      return hipErrorInvalidValue;
    return hipGetLastError();
  }
  if (head_size == 256 && fmt == 0)
    attend_launch_chunk<256, 0>(a, grid, chunk, qvec, stream);
  else if (head_size == 256 && fmt == 1)
    attend_launch_chunk<256, 1>(a, grid, chunk, qvec, stream);
  else if (head_size == 512 && fmt == 0)
    attend_launch_chunk<512, 0>(a, grid, chunk, qvec, stream);
  else if (head_size == 512 && fmt == 1)
    attend_launch_chunk<512, 1>(a, grid, chunk, qvec, stream);
  else
    return hipErrorInvalidValue;
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || chunks == 1) return e;
  return attend_fold(a, chunks, chunk, place0, place_dev, window, lanes, head_size, blend_out,
                     stream);
}

// The fold of a launch's chunk partials into `blend_out`.
static hipError_t attend_fold(const AttendArgs &a, int chunks, int chunk, int place0,
                              const int *place_dev, int window, int lanes, int head_size,
                              float *blend_out, hipStream_t stream, int extra) {
  const int head_count = a.head_count;
  const int q_stride = a.q_stride;
  // One lane: 16 dims a fold workgroup (the most workgroups); many lanes
  // (a prime or a block): 64.  Chunks a thread loads: enough for one pass.
  const int dims = lanes <= kAttendPrepLanes ? 16 : 64;
  const int slices = 256 / dims;
  int per = 1;
  while (per < 32 && per * slices < chunks) per *= 2;
  const dim3 fgrid(head_count, lanes, head_size / dims);
#define IGL_FOLD(D, P)                                                                             \
  hipLaunchKernelGGL((attend_fold_kernel<D, P>), fgrid, dim3(256), 0, stream, a.part_out,         \
                     a.part_peak, a.part_total, chunks, chunk, place0, place_dev, window, extra,   \
                     head_count, head_size, blend_out, q_stride)
#define IGL_FOLD_PER(D)                                                                            \
  switch (per) {                                                                                   \
    case 1: IGL_FOLD(D, 1); break;                                                                 \
    case 2: IGL_FOLD(D, 2); break;                                                                 \
    case 4: IGL_FOLD(D, 4); break;                                                                 \
    case 8: IGL_FOLD(D, 8); break;                                                                 \
    case 16: IGL_FOLD(D, 16); break;                                                               \
    default: IGL_FOLD(D, 32); break;                                                               \
  }
  if (dims == 16) {
    IGL_FOLD_PER(16)
  } else {
    IGL_FOLD_PER(64)
  }
#undef IGL_FOLD_PER
#undef IGL_FOLD
  return hipGetLastError();
}

// The attention of a decode step or a small block with the heads prepared in
// the same launch (attend_split_kernel's PREP form): 1 to kAttendPrepLanes
// lanes, lane 0 at the position in *place_dev (place_bound its upper bound,
// which sizes the grid), e4m3 rings, one key/value head.  query: the query
// heads before their norm, 16-byte aligned, lanes q_stride floats apart (a
// multiple of 4; the blend out the same); turn: lane by lane, turn_stride
// floats apart (a multiple of 4), the (cos, sin) pairs of the lane's position
// times each step, head_size / 2 of them; k_raw, v_raw, k_gain: the key and
// value heads before their norms, lanes kv_stride floats apart, and the key
// gain, whose bytes go to ring slot position % cache_span (NULL for a layer
// that reads another layer's rings and writes none).
extern "C" hipError_t igl_launch_attend_prep(const uint8_t *key_store, const uint8_t *value_store,
                                             float key_scale, float value_scale, int cache_span,
                                             int head_size, int lanes, const float *query,
                                             int q_stride, const float *q_gain, const float *turn,
                                             int turn_stride, const float *k_raw,
                                             const float *v_raw, int kv_stride, const float *k_gain,
                                             uint8_t *k_ring, uint8_t *v_ring, float eps,
                                             int place_bound, const int *place_dev, int window,
                                             float score_scale, float *blend_out, float *work,
                                             hipStream_t stream) {
  AttendArgs a;
  if (lanes < 1 || lanes > kAttendPrepLanes) return hipErrorInvalidValue;
  const int chunk = attend_chunk(place_bound, window, lanes);
  // with k_raw, one slot more a lane: the partial of the block's new positions
  const int extra = k_raw ? 1 : 0;
  const int chunks = attend_blocks(place_bound, window, lanes) + extra;
  if ((((uintptr_t)query) & 15u) || (((uintptr_t)q_gain) & 15u) || (((uintptr_t)turn) & 15u) ||
      !place_dev || !turn)
    return hipErrorInvalidValue;
  if (lanes > 1 && (q_stride < kAttendGroup * head_size || (q_stride & 3) || turn_stride < head_size ||
                    (turn_stride & 3) || (k_raw && kv_stride < head_size)))
    return hipErrorInvalidValue;
  if (k_raw && (!v_raw || !k_gain || !k_ring || !v_ring)) return hipErrorInvalidValue;
  // the new positions of the block sit inside every lane's window and the
  // ring holds them beside every older position a lane reads
  if (window > 0 && lanes > window) return hipErrorInvalidValue;
  if (k_raw && cache_span < (window > 0 ? window : place_bound + 1) + lanes - 1 &&
      cache_span < place_bound + lanes)
    return hipErrorInvalidValue;
  a.key_store = key_store;
  a.value_store = value_store;
  a.kv_width = head_size;
  a.cache_span = cache_span;
  a.place0 = place_bound;
  a.place_dev = place_dev;
  a.window = window;
  a.chunks = chunks;
  a.final_out = chunks == 1 && !extra ? blend_out : nullptr;
  a.q_stride = lanes > 1 ? q_stride : kAttendGroup * head_size;
  a.query = query;
  a.key_scale = key_scale * 256.0f * score_scale;
  a.value_scale = value_scale * 256.0f;
  a.head_count = kAttendGroup;
  a.part_out = work;
  a.part_peak = work + (size_t)lanes * chunks * kAttendGroup * head_size;
  a.part_total = a.part_peak + (size_t)lanes * chunks * kAttendGroup;
  a.q_gain = q_gain;
  a.turn = turn;
  a.turn_stride = lanes > 1 ? turn_stride : 0;
  a.k_raw = k_raw;
  a.kv_raw_stride = lanes > 1 ? kv_stride : 0;
  a.v_raw = v_raw;
  a.k_gain = k_gain;
  a.k_ring = k_ring;
  a.v_ring = v_ring;
  a.k_code_scale = key_scale;
  a.v_code_scale = value_scale;
  a.eps = eps;
  const dim3 grid(chunks, 1, lanes);
  if (head_size == 256 && chunk == 32)
    hipLaunchKernelGGL((attend_split_kernel<256, 0, 32, true, true>), grid, dim3(256), 0, stream, a);
  else if (head_size == 256)
    hipLaunchKernelGGL((attend_split_kernel<256, 0, 64, true, true>), grid, dim3(256), 0, stream, a);
  else if (head_size == 512 && chunk == 32)
    hipLaunchKernelGGL((attend_split_kernel<512, 0, 32, true, true>), grid, dim3(256), 0, stream, a);
  else if (head_size == 512)
    hipLaunchKernelGGL((attend_split_kernel<512, 0, 64, true, true>), grid, dim3(256), 0, stream, a);
  else
    return hipErrorInvalidValue;
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.final_out) return e;
  return attend_fold(a, chunks, chunk, place_bound, place_dev, window, lanes, head_size, blend_out, stream,
                     extra);
}

// Floats of workspace igl_launch_attend_prep needs for the same arguments
// (with key/value rows to write: one partial slot a lane more than the chunks).
extern "C" size_t igl_attend_prep_work_floats(int place_bound, int window, int head_size, int lanes,
                                              int writes_row) {
  const size_t blocks = (size_t)attend_blocks(place_bound, window, lanes) + (writes_row ? 1 : 0);
  return (size_t)lanes * blocks * (size_t)kAttendGroup * ((size_t)head_size + 2);
}

// Floats of workspace igl_launch_attend needs for the same arguments.
extern "C" size_t igl_attend_work_floats(int place0, int window, int lanes, int head_count,
                                         int head_size) {
  const size_t blocks = (size_t)attend_blocks(place0, window, lanes);
  // a wide launch of more than one chunk merges its chunks in registers
  // (attend_rows_kernel): no partials
  if (lanes >= kAttendWideLanes && blocks > 1) return 0;
  return (size_t)lanes * blocks * (size_t)head_count * ((size_t)head_size + 2);
}

// Floats of workspace enough for every igl_launch_attend call of at most
// `lanes` lanes whose spans stay within `span_limit` positions.  The chunk
// count is not monotonic in the span: chunks are 32 positions up to
// kAttendShortSpan and 64 beyond, so a span just under kAttendShortSpan has
// more chunks than one just over it.  The largest count of each regime is
// taken.  Launches of kAttendWideLanes lanes and more keep no partials (one
// chunk: the blend written directly; more: merged in registers), so the most
// lanes that keep partials is kAttendWideLanes - 1.
extern "C" size_t igl_attend_work_floats_limit(int span_limit, int lanes, int head_count,
                                               int head_size) {
  if (span_limit < 1 || lanes < 1) return 0;
  const int short_top = span_limit < kAttendShortSpan ? span_limit : kAttendShortSpan;
  const int b_short = attend_blocks(short_top - 1, 0, 1);
  const int b_long = attend_blocks(span_limit - 1, 0, 1);
  const size_t blocks = (size_t)(b_short > b_long ? b_short : b_long);
  const size_t narrow = (size_t)(lanes < kAttendWideLanes ? lanes : kAttendWideLanes - 1);
  // a prepared launch of up to kAttendPrepLanes lanes (a decode step, a small
  // block) needs blocks + 1 slots a lane: its new positions' partial
  const size_t prep = (size_t)(lanes < kAttendPrepLanes ? lanes : kAttendPrepLanes) * (blocks + 1);
  const size_t slots = narrow * blocks > prep ? narrow * blocks : prep;
  return slots * (size_t)head_count * ((size_t)head_size + 2);
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
