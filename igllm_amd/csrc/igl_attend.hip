// igl_attend.hip - decode attention over the byte-quantized key/value ring,
// gfx950.
//
// For one lane (one query position) and one key/value head shared by GROUP
// query heads, computes
//     o_h = sum_t softmax_t(score_scale * q_h . k_t) v_t
// over the visible positions t = place_start .. place_start + span - 1, whose
// rows sit in ring slot t % cache_span (session_attend_group with
// attend_score_band and attend_blend_band, app_core.c:11296-11453; ring and
// span rules 11500, 11516-11526).  A stored byte decodes to
//     e4m3:  cache_real8(byte) * scale  (cache_real8, app_core.c:11018-11030)
//     int8:  (int8_t)byte * scale
// The reference computes every score against `grid[byte] = real8 * scale`;
// here the scale is applied to the finished dot product instead, which is the
// same value up to fp32 rounding.
//
// e4m3 bytes are decoded without a table: moving the byte's exponent and
// mantissa to bits [7,14) of a binary16 and its sign to bit 15 gives exactly
// real8(byte) / 256 for all 256 codes, including 0x7F/0xFF, which the
// reference reads as +-480 and which this mapping also reads as +-480 (no NaN
// code exists on either side).
//
// Split over the span (flash-decoding): a workgroup takes CHUNK positions,
// computes the chunk's scores, its running maximum, exponentials and their
// sum, and its unnormalized blend; a second kernel merges the chunks in chunk
// order.  v1 runs the dot products on the vector ALU.
#include "igl_device.h"

namespace igl {

constexpr int kAttendThreads = 256;
constexpr int kAttendChunk = 128;

struct AttendArgs {
  const uint8_t *key_store;    // [cache_span][kv_width]
  const uint8_t *value_store;
  int kv_width;
  int cache_span;
  int place_start;
  int span_count;
  const float *query;          // [head_count][HEAD]
  float key_scale;             // decoded-byte multiplier, score_scale folded in
  float value_scale;
  int fmt;                     // 0 = e4m3, 1 = int8
  float *part_out;             // [chunks][head_count][HEAD]
  float *part_peak;            // [chunks][head_count]
  float *part_total;           // [chunks][head_count]
  int head_count;
};

__device__ __forceinline__ float decode_byte(uint32_t b, int fmt) {
  if (fmt == 0) {
    const uint32_t h = ((b & 0x7Fu) << 7) | ((b & 0x80u) << 8);
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
  }
  return (float)(int8_t)(uint8_t)b;
}

template <int HEAD, int GROUP>
__global__ __launch_bounds__(kAttendThreads) void attend_chunk_kernel(AttendArgs a) {
  constexpr int kPosHalves = kAttendChunk / 64;  // position blocks of 64 in a chunk
  constexpr int kDimSplit = 4 / kPosHalves;      // waves sharing one position block
  constexpr int kDimsPerWave = HEAD / kDimSplit;
  constexpr int kBlendDims = HEAD / kAttendThreads;  // dims a thread blends (1 or 2)

  __shared__ float ps[4][GROUP][64];               // partial scores per wave
  __shared__ float pt[kAttendChunk][GROUP];        // probabilities, position-major

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int chunk = blockIdx.x;
  const int kv = blockIdx.y;
  const int head0 = kv * GROUP;
  const int t_base = chunk * kAttendChunk;
  const size_t kv_off = (size_t)kv * HEAD;

  // ---- scores: lane = position, waves split (position block, dim range).
  {
    const int pblk = wave / kDimSplit;
    const int dpart = wave % kDimSplit;
    const int t = t_base + pblk * 64 + lane;
    float sc[GROUP];
#pragma unroll
    for (int h = 0; h < GROUP; ++h) sc[h] = 0.0f;
    if (t < a.span_count) {
      const int slot = (a.place_start + t) % a.cache_span;
      const uint4_t *row = reinterpret_cast<const uint4_t *>(
          a.key_store + (size_t)slot * a.kv_width + kv_off + dpart * kDimsPerWave);
      const float *q = a.query + (size_t)head0 * HEAD + dpart * kDimsPerWave;
      for (int d16 = 0; d16 < kDimsPerWave / 16; ++d16) {
        const uint4_t w = __builtin_nontemporal_load(row + d16);
        float kf[16];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i) kf[4 * j + i] = decode_byte((w[j] >> (8 * i)) & 0xFFu, a.fmt);
#pragma unroll
        for (int h = 0; h < GROUP; ++h) {
          float s = sc[h];
#pragma unroll
          for (int i = 0; i < 16; ++i) s = __builtin_fmaf(kf[i], q[h * HEAD + d16 * 16 + i], s);
          sc[h] = s;
        }
      }
    }
#pragma unroll
    for (int h = 0; h < GROUP; ++h) ps[wave][h][lane] = sc[h];
  }
  __syncthreads();

  // ---- chunk softmax: wave w takes heads w, w+4; lane = position in a block.
  for (int h = wave; h < GROUP; h += 4) {
    float s[kPosHalves];
    float m = -INFINITY;
#pragma unroll
    for (int pb = 0; pb < kPosHalves; ++pb) {
      const int t = t_base + pb * 64 + lane;
      float v = 0.0f;
#pragma unroll
      for (int dp = 0; dp < kDimSplit; ++dp) v += ps[pb * kDimSplit + dp][h][lane];
      v = (t < a.span_count) ? v * a.key_scale : -INFINITY;
      s[pb] = v;
      m = fmaxf(m, v);
    }
    // wave max
    m = row16_max(m);
    m = fmaxf(fmaxf(lane_read(m, 0), lane_read(m, 16)), fmaxf(lane_read(m, 32), lane_read(m, 48)));
    float l = 0.0f;
#pragma unroll
    for (int pb = 0; pb < kPosHalves; ++pb) {
      const float p = s[pb] == -INFINITY ? 0.0f : __expf(s[pb] - m);
      pt[pb * 64 + lane][h] = p;
      l += p;
    }
    l = wave_sum_to_last(l);
    if (lane == 63) {
      a.part_peak[(size_t)chunk * a.head_count + head0 + h] = m;
      a.part_total[(size_t)chunk * a.head_count + head0 + h] = l;
    }
  }
  __syncthreads();

  // ---- blend: thread = dims [kBlendDims*tid, +kBlendDims), every position of
  // the chunk in order; a wave's row read is 64 (or 128) contiguous bytes.
  {
    float o[GROUP][kBlendDims];
#pragma unroll
    for (int h = 0; h < GROUP; ++h)
#pragma unroll
      for (int i = 0; i < kBlendDims; ++i) o[h][i] = 0.0f;
    const int d0 = tid * kBlendDims;
    const int t_end = min(kAttendChunk, a.span_count - t_base);
    for (int tl = 0; tl < t_end; ++tl) {
      const int slot = (a.place_start + t_base + tl) % a.cache_span;
      const uint8_t *row = a.value_store + (size_t)slot * a.kv_width + kv_off + d0;
      float vf[kBlendDims];
      if (kBlendDims == 1) {
        vf[0] = decode_byte(row[0], a.fmt);
      } else {
        const uint32_t w = *reinterpret_cast<const uint16_t *>(row);
#pragma unroll
        for (int i = 0; i < kBlendDims; ++i) vf[i] = decode_byte((w >> (8 * i)) & 0xFFu, a.fmt);
      }
#pragma unroll
      for (int h = 0; h < GROUP; ++h) {
        const float p = pt[tl][h];
#pragma unroll
        for (int i = 0; i < kBlendDims; ++i) o[h][i] = __builtin_fmaf(p, vf[i], o[h][i]);
      }
    }
#pragma unroll
    for (int h = 0; h < GROUP; ++h)
#pragma unroll
      for (int i = 0; i < kBlendDims; ++i)
        a.part_out[((size_t)chunk * a.head_count + head0 + h) * HEAD + d0 + i] = o[h][i] * a.value_scale;
  }
}

// Merges chunk partials in chunk order: one workgroup per head.
__global__ void attend_merge_kernel(const float *part_out, const float *part_peak,
                                    const float *part_total, int chunks, int head_count,
                                    int head_size, float *blend_out) {
  const int h = blockIdx.x;
  float peak = -INFINITY;
  for (int c = 0; c < chunks; ++c) peak = fmaxf(peak, part_peak[(size_t)c * head_count + h]);
  float total = 0.0f;
  for (int c = 0; c < chunks; ++c) {
    const float m = part_peak[(size_t)c * head_count + h];
    if (m != -INFINITY) total += part_total[(size_t)c * head_count + h] * __expf(m - peak);
  }
  const float inv = total > 0.0f ? 1.0f / total : 0.0f;
  for (int d = threadIdx.x; d < head_size; d += blockDim.x) {
    float acc = 0.0f;
    for (int c = 0; c < chunks; ++c) {
      const float m = part_peak[(size_t)c * head_count + h];
      if (m != -INFINITY)
        acc += part_out[((size_t)c * head_count + h) * head_size + d] * __expf(m - peak);
    }
    blend_out[(size_t)h * head_size + d] = acc * inv;
  }
}

}  // namespace igl

using namespace igl;

extern "C" int igl_attend_chunk_size(void) { return kAttendChunk; }

extern "C" hipError_t igl_launch_attend(const uint8_t *key_store, const uint8_t *value_store,
                                        int fmt, float key_scale, float value_scale,
                                        int cache_span, int kv_width, int kv_count,
                                        int group_share, int head_size, const float *query,
                                        int place_start, int span_count, float score_scale,
                                        float *blend_out, float *work, hipStream_t stream) {
  AttendArgs a;
  const int chunks = (span_count + kAttendChunk - 1) / kAttendChunk;
  const int head_count = kv_count * group_share;
  a.key_store = key_store;
  a.value_store = value_store;
  a.kv_width = kv_width;
  a.cache_span = cache_span;
  a.place_start = place_start;
  a.span_count = span_count;
  a.query = query;
  // e4m3 decodes to real8 / 256; the 256 goes back in with the scale.
  const float unit = fmt == 0 ? 256.0f : 1.0f;
  a.key_scale = key_scale * unit * score_scale;
  a.value_scale = value_scale * unit;
  a.fmt = fmt;
  a.head_count = head_count;
  a.part_out = work;
  a.part_peak = work + (size_t)chunks * head_count * head_size;
  a.part_total = a.part_peak + (size_t)chunks * head_count;
  dim3 grid(chunks, kv_count);
  if (head_size == 256 && group_share == 8)
    hipLaunchKernelGGL((attend_chunk_kernel<256, 8>), grid, dim3(kAttendThreads), 0, stream, a);
  else if (head_size == 512 && group_share == 8)
    hipLaunchKernelGGL((attend_chunk_kernel<512, 8>), grid, dim3(kAttendThreads), 0, stream, a);
  else
    return hipErrorInvalidValue;
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(attend_merge_kernel, dim3(head_count), dim3(256), 0, stream, a.part_out,
                     a.part_peak, a.part_total, chunks, head_count, head_size, blend_out);
  return hipGetLastError();
}

// Floats of workspace igl_launch_attend needs.
extern "C" size_t igl_attend_work_floats(int span_count, int head_count, int head_size) {
  const size_t chunks = (size_t)((span_count + kAttendChunk - 1) / kAttendChunk);
  return chunks * (size_t)head_count * ((size_t)head_size + 2);
}
