// igl_elem.hip - the backend table's elementwise entries and the cache
// writer, gfx950.
//
// These are the entries of back_desk that are not projections (norm_rms,
// soft_max, gelu_gate, rope_turn; app_core.c:5223-5245) plus the key/value
// ring writer that the reference keeps outside the table (cache_lay,
// app_core.c:11205-11236).  They read no weights; each is one small launch.
#include "igl_device.h"

namespace igl {

// RMS norm of one vector per workgroup: sum of squares in double (the
// reference accumulates in double, kern_norm_rms app_core.c:4667-4684), then
// x * (mean + eps)^-1/2 * gain.
__global__ __launch_bounds__(256) void norm_rms_kernel(const float *in, const float *gain, int n,
                                                       int stride, float eps, float *out) {
  __shared__ double part[16];
  const float *x = in + (size_t)blockIdx.x * stride;
  float *y = out + (size_t)blockIdx.x * stride;
  double acc = 0.0;
  for (int i = threadIdx.x; i < n; i += 256) acc += (double)x[i] * (double)x[i];
  const float shrink = rms_shrink(block_sum_f64(acc, part), n, eps);
  for (int i = threadIdx.x; i < n; i += 256) {
    const float v = x[i] * shrink;
    y[i] = gain ? v * gain[i] : v;
  }
}

// Softmax of one vector per workgroup: peak, e^(v - peak), total, scale.
__global__ void soft_max_kernel(float *v, int n, int stride) {
  __shared__ float part[256];
  float *x = v + (size_t)blockIdx.x * stride;
  float peak = -INFINITY;
  for (int i = threadIdx.x; i < n; i += blockDim.x) peak = fmaxf(peak, x[i]);
  part[threadIdx.x] = peak;
  __syncthreads();
  for (int w = blockDim.x / 2; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) part[threadIdx.x] = fmaxf(part[threadIdx.x], part[threadIdx.x + w]);
    __syncthreads();
  }
  peak = part[0];
  __syncthreads();
  float total = 0.0f;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const float e = __expf(x[i] - peak);
    x[i] = e;
    total += e;
  }
  part[threadIdx.x] = total;
  __syncthreads();
  for (int w = blockDim.x / 2; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) part[threadIdx.x] += part[threadIdx.x + w];
    __syncthreads();
  }
  const float shrink = part[0] > 0.0f ? 1.0f / part[0] : 0.0f;
  if (part[0] > 0.0f)
    for (int i = threadIdx.x; i < n; i += blockDim.x) x[i] *= shrink;
}

// gate <- gelu_tanh(gate) * rise, with gelu_tanh(x) = x t / (t + 1),
// t = e^(2 sqrt(2/pi) (x + 0.044715 x^3)), zero where 2y <= -30 and t
// clamped at 2y = 30 (kern_gelu_tanh, app_core.c:5105-5118).
__global__ void gelu_gate_kernel(float *gate, const float *rise, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  gate[i] = gelu_near(gate[i]) * rise[i];
}

// Rotate-half RoPE on `heads` heads of `head_size` (kern_rope_turn,
// app_core.c:5196-5207).
__global__ void rope_turn_kernel(float *v, int heads, int head_size, const float *cosv,
                                 const float *sinv) {
  const int half = head_size / 2;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= heads * half) return;
  const int h = i / half;
  const int j = i - h * half;
  float *x = v + (size_t)h * head_size;
  const float lo = x[j], hi = x[j + half];
  x[j] = lo * cosv[j] - hi * sinv[j];
  x[j + half] = hi * cosv[j] + lo * sinv[j];
}

// Writes `width` values of `row` into ring slot `slot` of a byte store.
__global__ void cache_lay_kernel(const float *row, int width, float scale, int fmt, uint8_t *store,
                                 size_t slot_first) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= width) return;
  store[slot_first + i] = fmt == 0 ? e4m3_code(row[i] / scale) : int8_code(row[i], scale);
}

// The static activation grid on `lanes` rows of n (quant_step,
// app_core.c:1930-1940): rint(x / step) with the division correctly rounded,
// clamped to [-128, 127] by the reference's two comparisons (a NaN passes
// through), times step.  A step that is not positive copies x unchanged.
// src may be dst.
__global__ void quant_step_kernel(const float *src, int src_stride, float *dst, int dst_stride,
                                  int n, float step) {
  const int lane = blockIdx.y;
  const float *in = src + (size_t)lane * src_stride;
  float *out = dst + (size_t)lane * dst_stride;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    const float x = in[i];
    if (!(step > 0.0f)) {
      out[i] = x;
      continue;
    }
    float level = __builtin_rintf(x / step);
    if (level < -128.0f) level = -128.0f;
    if (level > 127.0f) level = 127.0f;
    out[i] = level * step;
  }
}

// ---- the prefill of a calibrated plane on the activation grid -------------
//
// With one gain a row, y = gain * step * sum ((c ^ flip) - bias) L is taken as
// an MFMA product of integer-valued operands: the lanes as their levels L
// (quant_level_kernel), the codes as 4-bit planes with unit gains (widened by
// code_widen_kernel), so every product and partial sum is an integer below
// 2^24 that binary16 operands and fp32 accumulation carry exactly; then
// grid_close_kernel closes each row as the reference's level path does.

// L = rint(x / step) clamped to [-128, 127], as a float; also sum L per lane
// into `lsum` (which must start at zero: integers below 2^24, exact in fp32).
__global__ void quant_level_kernel(const float *src, int src_stride, float *dst, int dst_stride, int n,
                                   float step, float *lsum) {
  const int lane = blockIdx.y;
  const float *in = src + (size_t)lane * src_stride;
  float *out = dst + (size_t)lane * dst_stride;
  float total = 0.0f;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    float level = __builtin_rintf(in[i] / step);
    if (level < -128.0f) level = -128.0f;
    if (level > 127.0f) level = 127.0f;
    out[i] = level;
    total += level;
  }
  if (lsum) {
    total = wave_sum_to_last(total);
    if ((threadIdx.x & 63) == 63) atomicAdd(lsum + lane, total);
  }
}

// Codes of any width as 4-bit planes of value + 8, two a byte, low nibble
// first, rows of K / 2 bytes:
//   2-bit and 4-bit codes: one plane, (c ^ flip) - bias + 8;
//   8-bit codes (bias 128): two planes, hi = c' >> 4 and lo = c' & 15 with
//   c' = c ^ flip, so c' - 128 = 16 (hi - 8) + (lo - 8) + 8.
// One thread writes one byte (two codes) of each plane.
__global__ void code_widen_kernel(const uint8_t *codes, long long row_stride, int N, int K, int bits,
                                  int flip, int bias, uint8_t *hi_plane, uint8_t *lo_plane) {
  const int half = K >> 1;
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)N * half) return;
  const int n = (int)(i / half);
  const int k = 2 * (int)(i - (size_t)n * half);
  const uint8_t *row = codes + (size_t)n * row_stride;
  int c[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int at = (k + j) * bits;
    c[j] = ((row[at >> 3] >> (at & 7)) & ((1 << bits) - 1)) ^ flip;
  }
  if (bits == 8) {
    hi_plane[i] = (uint8_t)((c[0] >> 4) | ((c[1] >> 4) << 4));
    lo_plane[i] = (uint8_t)((c[0] & 15) | ((c[1] & 15) << 4));
  } else {
    hi_plane[i] = (uint8_t)((c[0] - bias + 8) | ((c[1] - bias + 8) << 4));
  }
}

// out = quant_step(gain[n] * step * part, leave): part = a, the widened
// plane's product, or for an 8-bit plane part = 16 a + b + 8 lsum[m], a and b
// the hi and lo planes' products.  In place on `a` allowed.
__global__ void grid_close_kernel(const float *a, const float *b, const float *lsum, int in_stride,
                                  const float *gains, float step, float leave, int N, float *out,
                                  int out_stride) {
  const int m = blockIdx.y;
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  float part = a[(size_t)m * in_stride + n];
  if (b) part = (16.0f * part + b[(size_t)m * in_stride + n]) + 8.0f * lsum[m];
  float y = gains[n] * step * part;
  if (leave > 0.0f) {
    float level = __builtin_rintf(y / leave);
    if (level < -128.0f) level = -128.0f;
    if (level > 127.0f) level = 127.0f;
    y = level * leave;
  }
  out[(size_t)m * out_stride + n] = y;
}

__global__ void fill_kernel(float *dst, size_t n, float value) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = value;
}

}  // namespace igl

using namespace igl;

extern "C" hipError_t igl_launch_quant_level(const float *src, int src_stride, float *dst, int dst_stride,
                                             int n, int lanes, float step, float *lsum, hipStream_t stream) {
  const int blocks = (n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024;
  if (lsum) hipLaunchKernelGGL(fill_kernel, dim3((lanes + 255) / 256), dim3(256), 0, stream, lsum, (size_t)lanes, 0.0f);
  hipLaunchKernelGGL(quant_level_kernel, dim3(blocks, lanes), dim3(256), 0, stream, src, src_stride, dst,
                     dst_stride, n, step, lsum);
  return hipGetLastError();
}

extern "C" hipError_t igl_launch_code_widen(const uint8_t *codes, long long row_stride, int N, int K, int bits,
                                            int flip, int bias, uint8_t *hi_plane, uint8_t *lo_plane,
                                            hipStream_t stream) {
  const size_t total = (size_t)N * (size_t)(K / 2);
  hipLaunchKernelGGL(code_widen_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, codes,
                     row_stride, N, K, bits, flip, bias, hi_plane, lo_plane);
  return hipGetLastError();
}

extern "C" hipError_t igl_launch_grid_close(const float *a, const float *b, const float *lsum, int in_stride,
                                            const float *gains, float step, float leave, int N, int lanes,
                                            float *out, int out_stride, hipStream_t stream) {
  hipLaunchKernelGGL(grid_close_kernel, dim3((N + 255) / 256, lanes), dim3(256), 0, stream, a, b, lsum, in_stride,
                     gains, step, leave, N, out, out_stride);
  return hipGetLastError();
}

// The read floor: every 16-byte word of `src` loaded once (two a thread, both
// in flight before either is used) and folded; the fold is stored only when it
// equals a constant, so the loads stay and nothing else costs.  The time of a
// kernel that must read `n16` words once, against which a GEMV that reads the
// same bytes is judged.
__global__ void read_floor_kernel(const uint4_t *src, size_t n16, uint32_t *sink) {
  const size_t i0 = (size_t)blockIdx.x * blockDim.x * 2 + threadIdx.x;
  const size_t i1 = i0 + blockDim.x;
  const uint4_t a = i0 < n16 ? __builtin_nontemporal_load(src + i0) : uint4_t{0, 0, 0, 0};
  const uint4_t b = i1 < n16 ? __builtin_nontemporal_load(src + i1) : uint4_t{0, 0, 0, 0};
  const uint32_t fold = a[0] ^ a[1] ^ a[2] ^ a[3] ^ b[0] ^ b[1] ^ b[2] ^ b[3];
  if (fold == 0x9E3779B9u && threadIdx.x == 0) sink[0] = fold;
}

extern "C" hipError_t igl_launch_read_floor(const void *src, size_t bytes, uint32_t *sink, hipStream_t stream) {
  const size_t n16 = bytes / 16;
  const size_t blocks = (n16 + 511) / 512;
  if (blocks == 0 || blocks > 0x7FFFFFFFu) return hipErrorInvalidValue;
  hipLaunchKernelGGL(read_floor_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                     reinterpret_cast<const uint4_t *>(src), n16, sink);
  return hipGetLastError();
}

extern "C" hipError_t igl_launch_fill(float *dst, size_t n, float value, hipStream_t stream) {
  hipLaunchKernelGGL(fill_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, dst, n, value);
  return hipGetLastError();
}

extern "C" hipError_t igl_launch_quant_step(const float *src, int src_stride, float *dst,
                                            int dst_stride, int n, int lanes, float step,
                                            hipStream_t stream) {
  const int blocks = (n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024;
  hipLaunchKernelGGL(quant_step_kernel, dim3(blocks, lanes), dim3(256), 0, stream, src, src_stride, dst,
                     dst_stride, n, step);
  return hipGetLastError();
}

extern "C" hipError_t igl_launch_norm_rms(const float *in, const float *gain, int n, int rows,
                                          int stride, float eps, float *out, hipStream_t stream) {
  hipLaunchKernelGGL(norm_rms_kernel, dim3(rows), dim3(256), 0, stream, in, gain, n, stride, eps, out);
  return hipGetLastError();
}

extern "C" hipError_t igl_launch_soft_max(float *v, int n, int rows, int stride, hipStream_t stream) {
  hipLaunchKernelGGL(soft_max_kernel, dim3(rows), dim3(256), 0, stream, v, n, stride);
  return hipGetLastError();
}

extern "C" hipError_t igl_launch_gelu_gate(float *gate, const float *rise, int n, hipStream_t stream) {
  hipLaunchKernelGGL(gelu_gate_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, gate, rise, n);
  return hipGetLastError();
}

extern "C" hipError_t igl_launch_rope_turn(float *v, int heads, int head_size, const float *cosv,
                                           const float *sinv, hipStream_t stream) {
  const int total = heads * (head_size / 2);
  hipLaunchKernelGGL(rope_turn_kernel, dim3((total + 255) / 256), dim3(256), 0, stream, v, heads,
                     head_size, cosv, sinv);
  return hipGetLastError();
}

extern "C" hipError_t igl_launch_cache_lay(const float *row, int width, float scale, int fmt,
                                           uint8_t *store, size_t slot_first, hipStream_t stream) {
  hipLaunchKernelGGL(cache_lay_kernel, dim3((width + 255) / 256), dim3(256), 0, stream, row, width,
                     scale, fmt, store, slot_first);
  return hipGetLastError();
}
