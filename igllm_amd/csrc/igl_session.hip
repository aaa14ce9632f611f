// igl_session.hip - the device side of a decode pass besides the projections
// and attention: embedding gathers, the per-layer-embedding mix, head norms
// with the rotary turn, residual updates, the cache writer for a batch of
// lanes, the logit cap and the greedy pick.  gfx950.
//
// Each restates a step of the reference's session graph (session_pass
// app_core.c:11843-11975, session_layer 11637-11743, session_attend
// 11455-11580) in the same order of float operations where the reference has
// one; reductions the reference does in double (norms) are done in double.
#include "igl_device.h"
#include "igl_launch.h"

namespace igl {

// Rows `ids[l]` of a 2, 4 or 8-bit code plane as floats times `factor`:
// (((code ^ flip) - code_bias) * gain) * factor (plane_row 1826-1856, then
// kern_scale).
__global__ void gather_rows_kernel(const uint8_t *codes, long long row_stride, const float *gains,
                                   int group_count, int group_shift, int code_bias, int code_flip,
                                   int bits, int cols, int rows, const int32_t *ids, float factor,
                                   float *out, int out_stride) {
  const int lane = blockIdx.y;
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= cols) return;
  int id = ids[lane];
  if (id < 0) id = 0;
  id %= rows;
  const int at = k * bits;
  const uint8_t b = codes[(size_t)id * row_stride + (at >> 3)];
  const int c = ((b >> (at & 7)) & ((1 << bits) - 1)) ^ code_flip;
  const float gain = gains[(size_t)id * group_count + ((unsigned)(k >> 5) >> group_shift)];
  const float v = (float)(c - code_bias) * gain;
  out[(size_t)lane * out_stride + k] = v * factor;
}

// The per-layer inputs of one lane (session_pass 11877-11902): the projected
// chunk scaled by 1/sqrt(hidden), RMS-normed with the shared gain, plus the
// token's per-layer embedding row scaled by sqrt(ple), times 1/sqrt(2).
// One workgroup per (chunk, lane); `seed` is already scaled by sqrt(ple).
__global__ __launch_bounds__(256) void ple_mix_kernel(float *room, int room_stride,
                                                      const float *seed, int seed_stride,
                                                      const float *gain, int ple, float eps,
                                                      float lift_scale, float blend) {
  __shared__ double red[256];
  const int chunk = blockIdx.x;
  const int lane = blockIdx.y;
  float *x = room + (size_t)lane * room_stride + (size_t)chunk * ple;
  const float *s = seed + (size_t)lane * seed_stride + (size_t)chunk * ple;
  double acc = 0.0;
  for (int i = threadIdx.x; i < ple; i += blockDim.x) {
    const float v = x[i] * lift_scale;
    acc += (double)v * (double)v;
  }
  const double total = block_sum_f64(acc, red);
  const float shrink = rms_shrink(total, ple, eps);
  for (int i = threadIdx.x; i < ple; i += blockDim.x) {
    const float v = x[i] * lift_scale;
    const float normed = v * shrink * gain[i];
    x[i] = (normed + s[i]) * blend;
  }
}

// Head norms and the rotary turn for a batch of lanes (session_attend
// 11487-11514).  One workgroup per (head, lane).  `gain` NULL normalizes
// without a gain (the value heads); `turn` 0 skips the rotation.  The angle of
// pair j at position p is p * step[j] in double, its cos and sin rounded to
// float (rope_wave 8147-8154); pairs past `turns` have step 0 (identity).
__global__ __launch_bounds__(256) void head_prep_kernel(float *v, int lane_stride, int head_size,
                                                        const float *gain, float eps,
                                                        const float *step, int turn,
                                                        int place_first) {
  __shared__ double red[256];
  const int head = blockIdx.x;
  const int lane = blockIdx.y;
  float *x = v + (size_t)lane * lane_stride + (size_t)head * head_size;
  double acc = 0.0;
  for (int i = threadIdx.x; i < head_size; i += blockDim.x) acc += (double)x[i] * (double)x[i];
  const double total = block_sum_f64(acc, red);
  const float shrink = rms_shrink(total, head_size, eps);
  const int half = head_size / 2;
  const double place = (double)(place_first + lane);
  for (int j = threadIdx.x; j < half; j += blockDim.x) {
    float lo = x[j] * shrink;
    float hi = x[j + half] * shrink;
    if (gain) {
      lo = lo * gain[j];
      hi = hi * gain[j + half];
    }
    if (turn) {
      const double angle = place * (double)step[j];
      const float c = (float)cos(angle);
      const float s = (float)sin(angle);
      x[j] = lo * c - hi * s;
      x[j + half] = hi * c + lo * s;
    } else {
      x[j] = lo;
      x[j + half] = hi;
    }
  }
}

// One head of head_prep_kernel's arithmetic, returned through `put(j, value)`
// for every dim j instead of written back.
template <typename Put>
__device__ __forceinline__ void head_turn(const float *x, int head_size, const float *gain,
                                          float eps, const float *step, int turn, double place,
                                          double *red, Put put) {
  double acc = 0.0;
  for (int i = threadIdx.x; i < head_size; i += blockDim.x) acc += (double)x[i] * (double)x[i];
  const double total = block_sum_f64(acc, red);
  const float shrink = rms_shrink(total, head_size, eps);
  const int half = head_size / 2;
  for (int j = threadIdx.x; j < half; j += blockDim.x) {
    float lo = x[j] * shrink;
    float hi = x[j + half] * shrink;
    if (gain) {
      lo = lo * gain[j];
      hi = hi * gain[j + half];
    }
    if (turn) {
      const double angle = place * (double)step[j];
      const float c = (float)cos(angle);
      const float s = (float)sin(angle);
      put(j, lo * c - hi * s);
      put(j + half, hi * c + lo * s);
    } else {
      put(j, lo);
      put(j + half, hi);
    }
  }
}

// The query, key and value heads of a batch of lanes in one launch
// (session_attend 11487-11514, then cache_lay 11205-11236 for the key and
// value rows).  Workgroup (b, lane): b < heads is query head b (norm, gain,
// turn, written back in place); b == heads the key head (norm, gain, turn,
// then its e4m3 bytes into ring slot (place + lane) % span); b == heads + 1
// the value head (norm without gain, no turn, into the value ring).  Lane 0's
// position is read from `place_dev`, so a captured launch serves every step.
// The arithmetic is head_prep_kernel's and cache_lay_rows_kernel's.
__global__ __launch_bounds__(256) void qkv_prep_kernel(
    float *q, int q_stride, const float *k, const float *v, int kv_stride, int heads,
    int head_size, const float *q_gain, const float *k_gain, float eps, const float *step,
    const int *place_dev, uint8_t *k_store, uint8_t *v_store, float k_scale, float v_scale,
    int span) {
  __shared__ double red[256];
  const int b = blockIdx.x;
  const int lane = blockIdx.y;
  const int place = *place_dev + lane;
  if (b < heads) {
    float *x = q + (size_t)lane * q_stride + (size_t)b * head_size;
    // Every read of x finishes (block_sum_f64's barriers) before a write.
    head_turn(x, head_size, q_gain, eps, step, 1, (double)place, red,
              [&](int j, float value) { x[j] = value; });
    return;
  }
  const bool key = b == heads;
  const float *x = (key ? k : v) + (size_t)lane * kv_stride;
  uint8_t *row = (key ? k_store : v_store) + (size_t)(place % span) * head_size;
  const float scale = key ? k_scale : v_scale;
  head_turn(x, head_size, key ? k_gain : nullptr, eps, step, key ? 1 : 0, (double)place, red,
            [&](int j, float value) { row[j] = e4m3_code(value / scale); });
}

// A residual update with the norms on either side of it (session_layer
// 11660-11737), one workgroup a lane: state <- state + norm(lift) *
// after_gain, times `scale` when `apply_scale` (the layer scalar); then, with
// `next_gain`, out <- norm(state) * next_gain, the next sub-block's input.
// The same float operations as norm_rms_kernel, add_rows_kernel and
// norm_rms_kernel in turn.
__global__ __launch_bounds__(256) void norm_add_kernel(float *state, int state_stride,
                                                       const float *lift, int lift_stride,
                                                       const float *after_gain,
                                                       int n, float eps, float scale,
                                                       int apply_scale, const float *next_gain,
                                                       float *out, int out_stride) {
  constexpr int kHeld = 16;  // values a thread holds: rows up to 4096
  __shared__ double red[16];
  const int lane = blockIdx.x;
  float *s = state + (size_t)lane * state_stride;
  const float *x = lift + (size_t)lane * lift_stride;
  // Every load is issued before the first use (one round trip, not one per value).
  float xv[kHeld], sv[kHeld], gv[kHeld];
#pragma unroll
  for (int k = 0; k < kHeld; ++k) {
    const int i = threadIdx.x + 256 * k;
    xv[k] = i < n ? x[i] : 0.0f;
    sv[k] = i < n ? s[i] : 0.0f;
    gv[k] = i < n ? after_gain[i] : 0.0f;
  }
  double acc = 0.0;
#pragma unroll
  for (int k = 0; k < kHeld; ++k) acc += (double)xv[k] * (double)xv[k];
  const float shrink = rms_shrink(block_sum_f64(acc, red), n, eps);
  double acc2 = 0.0;
#pragma unroll
  for (int k = 0; k < kHeld; ++k) {
    const int i = threadIdx.x + 256 * k;
    const float normed = xv[k] * shrink * gv[k];
    float sum = sv[k] + normed;
    if (apply_scale) sum *= scale;
    sv[k] = sum;
    if (i < n) {
      s[i] = sum;
      acc2 += (double)sum * (double)sum;
    }
  }
  if (!next_gain) return;
  const float shrink2 = rms_shrink(block_sum_f64(acc2, red), n, eps);
  float *y = out + (size_t)lane * out_stride;
#pragma unroll
  for (int k = 0; k < kHeld; ++k) {
    const int i = threadIdx.x + 256 * k;
    if (i < n) y[i] = sv[k] * shrink2 * next_gain[i];
  }
}

// into[l][i] += from[l][i] (kern_add), optionally then times `gain` (kern_scale).
__global__ void add_rows_kernel(float *into, int into_stride, const float *from, int from_stride,
                                int n, float gain, int apply_gain) {
  const int lane = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float v = into[(size_t)lane * into_stride + i] + from[(size_t)lane * from_stride + i];
  if (apply_gain) v *= gain;
  into[(size_t)lane * into_stride + i] = v;
}

__global__ void scale_rows_kernel(float *v, int stride, int n, float gain) {
  const int lane = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  v[(size_t)lane * stride + i] *= gain;
}

// The per-layer-input gate of a layer: gate[l][i] = gelu(gate[l][i]) * ple[l][i]
// (session_layer 11718-11723).
__global__ void gelu_mul_kernel(float *gate, int gate_stride, const float *ple, int ple_stride, int n) {
  const int lane = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float *g = gate + (size_t)lane * gate_stride + i;
  *g = gelu_near(*g) * ple[(size_t)lane * ple_stride + i];
}

// The feed-forward gate over a batch: gate = gelu(gate) * rise (kern_gelu_gate).
__global__ void gelu_gate_rows_kernel(float *gate, int gate_stride, const float *rise,
                                      int rise_stride, int n) {
  const int lane = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float *g = gate + (size_t)lane * gate_stride + i;
  *g = gelu_near(*g) * rise[(size_t)lane * rise_stride + i];
}

// Byte cache rows for a batch of lanes: lane l at position place_first + l
// goes to slot (place_first + l) % span (cache_lay 11205-11236).
__global__ void cache_lay_rows_kernel(const float *rows, int row_stride, int width, float scale,
                                      uint8_t *store, int span, int place_first) {
  const int lane = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= width) return;
  const size_t slot = (size_t)((place_first + lane) % span);
  store[slot * width + i] = e4m3_code(rows[(size_t)lane * row_stride + i] / scale);
}

// Greedy pick: the first index of the largest logit (session_pick_at
// 14672-14677), and the gap to the second largest value.  Stage one: per-block
// (best, index, second); stage two in one block.
struct Top2 {
  float best;
  int index;
  float second;
};

__device__ __forceinline__ Top2 top2_merge(Top2 a, Top2 b) {
  Top2 r;
  if (b.best > a.best || (b.best == a.best && b.index < a.index)) {
    r.best = b.best;
    r.index = b.index;
    r.second = fmaxf(a.best, b.second);
  } else {
    r.best = a.best;
    r.index = a.index;
    r.second = fmaxf(a.second, b.best);
  }
  return r;
}

// One lane of logits a grid row (blockIdx.y), `stride` floats apart.  With
// cap > 0 each logit is first capped, cap * (1 - 2 / (e^(2y) + 1)) with y =
// x / cap clamped to +-10 (kern_logit_cap_one, 5009-5014), and written back,
// so the row holds the capped logits the pick reads.
__global__ __launch_bounds__(256) void pick_stage_kernel(float *v, int n, size_t stride, float cap,
                                                         Top2 *part) {
  __shared__ Top2 red[256];
  v += (size_t)blockIdx.y * stride;
  part += (size_t)blockIdx.y * gridDim.x;
  Top2 t{-INFINITY, 0x7FFFFFFF, -INFINITY};
  const float back = cap > 0.0f ? 1.0f / cap : 0.0f;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    float x = v[i];
    if (cap > 0.0f) {
      float y = x * back;
      if (y > 10.0f) y = 10.0f;
      if (y < -10.0f) y = -10.0f;
      x = cap * (1.0f - 2.0f / (exp_near(y + y) + 1.0f));
      v[i] = x;
    }
    Top2 one{x, i, -INFINITY};
    t = top2_merge(t, one);
  }
  red[threadIdx.x] = t;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] = top2_merge(red[threadIdx.x], red[threadIdx.x + w]);
    __syncthreads();
  }
  if (threadIdx.x == 0) part[blockIdx.x] = red[0];
}

// Workgroup l closes lane l: pairs[2 l] = its pick, pairs[2 l + 1] = the
// margin's float bits.
__global__ __launch_bounds__(256) void pick_final_kernel(const Top2 *part, int parts, int32_t *pairs) {
  __shared__ Top2 red[256];
  part += (size_t)blockIdx.x * parts;
  int32_t *index_out = pairs + 2 * blockIdx.x;
  float *margin_out = reinterpret_cast<float *>(pairs + 2 * blockIdx.x + 1);
  Top2 t{-INFINITY, 0x7FFFFFFF, -INFINITY};
  for (int i = threadIdx.x; i < parts; i += blockDim.x) t = top2_merge(t, part[i]);
  red[threadIdx.x] = t;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] = top2_merge(red[threadIdx.x], red[threadIdx.x + w]);
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    *index_out = red[0].index;
    *margin_out = red[0].best - red[0].second;
  }
}

}  // namespace igl

using namespace igl;

static const int kPickBlocks = 256;

extern "C" hipError_t igl_launch_gather_rows(const igl_code_view *v, int cols, int rows,
                                             const int32_t *ids, int lanes, float factor, float *out,
                                             int out_stride, hipStream_t stream) {
  hipLaunchKernelGGL(gather_rows_kernel, dim3((cols + 255) / 256, lanes), dim3(256), 0, stream, v->codes,
                     v->row_stride, v->gains, v->gain_stride, v->group_shift, v->code_bias, v->code_flip,
                     v->bit_count, cols, rows, ids, factor, out, out_stride);
  return hipGetLastError();
}

extern "C" hipError_t igl_launch_ple_mix(float *room, int room_stride, const float *seed,
                                         int seed_stride, const float *gain, int ple, int chunks,
                                         int lanes, float eps, float lift_scale, float blend,
                                         hipStream_t stream) {
  hipLaunchKernelGGL(ple_mix_kernel, dim3(chunks, lanes), dim3(256), 0, stream, room, room_stride,
                     seed, seed_stride, gain, ple, eps, lift_scale, blend);
  return hipGetLastError();
}

extern "C" hipError_t igl_launch_head_prep(float *v, int lane_stride, int heads, int head_size,
                                           int lanes, const float *gain, float eps,
                                           const float *step, int turn, int place_first,
                                           hipStream_t stream) {
  hipLaunchKernelGGL(head_prep_kernel, dim3(heads, lanes), dim3(256), 0, stream, v, lane_stride,
                     head_size, gain, eps, step, turn, place_first);
  return hipGetLastError();
}

__global__ void put_int_kernel(int32_t *dst, int value) { *dst = value; }

// One int written on the stream (a batch's position, ahead of its kernels).
extern "C" hipError_t igl_launch_put_int(int32_t *dst, int value, hipStream_t stream) {
  hipLaunchKernelGGL(put_int_kernel, dim3(1), dim3(1), 0, stream, dst, value);
  return hipGetLastError();
}

// The rotation rows of a pass's positions, for each kind of layer: turn[j] =
// ((float)cos(p * step[j]), (float)sin(p * step[j])) in double, as head_turn
// forms them (the reference's cos_room / sin_room at that position), p =
// *place_dev + lane, one workgroup a lane.  Computed once a decode step (or a
// small block) for every layer's attention.
__global__ __launch_bounds__(256) void turn_row_kernel(const float *step0, int half0,
                                                       const float *step1, int half1,
                                                       const int *place_dev, float *turn0,
                                                       float *turn1) {
  const int lane = blockIdx.x;
  const double place = (double)(*place_dev + lane);
  for (int j = threadIdx.x; j < half0 + half1; j += blockDim.x) {
    const bool first = j < half0;
    const int i = first ? j : j - half0;
    const double angle = place * (double)(first ? step0 : step1)[i];
    float *t = first ? turn0 + (size_t)lane * 2 * half0 : turn1 + (size_t)lane * 2 * half1;
    t[2 * i] = (float)cos(angle);
    t[2 * i + 1] = (float)sin(angle);
  }
}

extern "C" hipError_t igl_launch_turn_row(const float *step0, int half0, const float *step1,
                                          int half1, const int *place_dev, int lanes, float *turn0,
                                          float *turn1, hipStream_t stream) {
  if (lanes < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(turn_row_kernel, dim3(lanes), dim3(256), 0, stream, step0, half0, step1, half1,
                     place_dev, turn0, turn1);
  return hipGetLastError();
}

extern "C" hipError_t igl_launch_qkv_prep(float *q, int q_stride, const float *k, const float *v,
                                          int kv_stride, int heads, int head_size, int lanes,
                                          const float *q_gain, const float *k_gain, float eps,
                                          const float *step, const int *place_dev,
                                          uint8_t *k_store, uint8_t *v_store, float k_scale,
                                          float v_scale, int span, hipStream_t stream) {
  const int blocks = heads + (k ? 2 : 0);
  hipLaunchKernelGGL(qkv_prep_kernel, dim3(blocks, lanes), dim3(256), 0, stream, q, q_stride, k, v,
                     kv_stride, heads, head_size, q_gain, k_gain, eps, step, place_dev, k_store,
                     v_store, k_scale, v_scale, span);
  return hipGetLastError();
}

extern "C" hipError_t igl_launch_norm_add(float *state, int state_stride, const float *lift,
                                          int lift_stride, const float *after_gain, int n,
                                          int lanes, float eps, float scale, int apply_scale,
                                          const float *next_gain, float *out, int out_stride,
                                          hipStream_t stream) {
  if (n > 4096) return hipErrorInvalidValue;
  hipLaunchKernelGGL(norm_add_kernel, dim3(lanes), dim3(256), 0, stream, state, state_stride, lift,
                     lift_stride, after_gain, n, eps, scale, apply_scale, next_gain, out,
                     out_stride);
  return hipGetLastError();
}

extern "C" hipError_t igl_launch_add_rows(float *into, int into_stride, const float *from,
                                          int from_stride, int n, int lanes, float gain,
                                          int apply_gain, hipStream_t stream) {
  hipLaunchKernelGGL(add_rows_kernel, dim3((n + 255) / 256, lanes), dim3(256), 0, stream, into,
                     into_stride, from, from_stride, n, gain, apply_gain);
  return hipGetLastError();
}

extern "C" hipError_t igl_launch_scale_rows(float *v, int stride, int n, int lanes, float gain,
                                            hipStream_t stream) {
  hipLaunchKernelGGL(scale_rows_kernel, dim3((n + 255) / 256, lanes), dim3(256), 0, stream, v,
                     stride, n, gain);
  return hipGetLastError();
}

extern "C" hipError_t igl_launch_gelu_mul(float *gate, int gate_stride, const float *ple,
                                          int ple_stride, int n, int lanes, hipStream_t stream) {
  hipLaunchKernelGGL(gelu_mul_kernel, dim3((n + 255) / 256, lanes), dim3(256), 0, stream, gate,
                     gate_stride, ple, ple_stride, n);
  return hipGetLastError();
}

extern "C" hipError_t igl_launch_gelu_gate_rows(float *gate, int gate_stride, const float *rise,
                                                int rise_stride, int n, int lanes,
                                                hipStream_t stream) {
  hipLaunchKernelGGL(gelu_gate_rows_kernel, dim3((n + 255) / 256, lanes), dim3(256), 0, stream,
                     gate, gate_stride, rise, rise_stride, n);
  return hipGetLastError();
}

extern "C" hipError_t igl_launch_cache_lay_rows(const float *rows, int row_stride, int width,
                                                float scale, uint8_t *store, int span,
                                                int place_first, int lanes, hipStream_t stream) {
  hipLaunchKernelGGL(cache_lay_rows_kernel, dim3((width + 255) / 256, lanes), dim3(256), 0, stream,
                     rows, row_stride, width, scale, store, span, place_first);
  return hipGetLastError();
}

// Workspace for `lanes` lanes of igl_launch_pick.
extern "C" size_t igl_pick_work_bytes(int lanes) { return sizeof(Top2) * kPickBlocks * (size_t)lanes; }

// The greedy pick of `lanes` rows of n logits, `stride` floats apart, into
// pairs[2 l] (index) and pairs[2 l + 1] (the top-1/top-2 gap's float bits).
extern "C" hipError_t igl_launch_pick(float *v, int n, size_t stride, int lanes, float cap, void *work,
                                      int32_t *pairs, hipStream_t stream) {
  hipLaunchKernelGGL(pick_stage_kernel, dim3(kPickBlocks, lanes), dim3(256), 0, stream, v, n,
                     stride, cap, reinterpret_cast<Top2 *>(work));
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(pick_final_kernel, dim3(lanes), dim3(256), 0, stream,
                     reinterpret_cast<const Top2 *>(work), kPickBlocks, pairs);
  return hipGetLastError();
}
