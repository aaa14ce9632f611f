/* audit_stub.c - a host-only stand-in for the HIP runtime, for auditing the
 * backend's host code on a machine without a GPU.  TEST INFRASTRUCTURE ONLY.
 *
 * The product's own host code is linked against it unchanged: the C files
 * (back_hip.c, igl_engine.c, ...) and the host side of every .hip file
 * (compiled with --cuda-host-only, so the launchers compute their grids,
 * partial sizes and argument structs exactly as they do on the GPU).  What
 * this file supplies instead of libamdhip64:
 *   - device memory: host allocations, each recorded (base, size); copies and
 *     fills are carried out, so values the host code reads back are real;
 *   - kernel launches: every launch's grid and block are checked against the
 *     hardware's limits, and the launch is counted; nothing runs;
 *   - graph capture and replay, streams and events: bookkeeping only;
 *   - for every launcher the engine and the desk call, a wrapper (linked in
 *     with ld's --wrap) that checks each buffer the kernel will touch, at the
 *     extent the kernel's arguments imply, lies inside one recorded
 *     allocation, before the real launcher runs.
 * Violations are counted and the first ones printed; audit_report() returns
 * their number.
 */
#define _POSIX_C_SOURCE 200809L
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "igl_backend.h"
#include "igl_launch.h"

/* ---- the allocation registry ------------------------------------------- */

typedef struct audit_block {
  uintptr_t base;
  size_t size;
  int host;  /* pinned host (hipHostMalloc) */
} audit_block;

static audit_block *blocks;
static int block_count, block_room;
static long violations, launches, checks;

static void note_violation(const char *fmt, ...) {
  va_list ap;
  ++violations;
  if (violations > 25) return;
  va_start(ap, fmt);
  fprintf(stderr, "AUDIT VIOLATION: ");
  vfprintf(stderr, fmt, ap);
  fputc('\n', stderr);
  va_end(ap);
}

static void add_block(void *p, size_t size, int host) {
  if (block_count == block_room) {
    block_room = block_room ? 2 * block_room : 256;
    blocks = (audit_block *)realloc(blocks, (size_t)block_room * sizeof(*blocks));
    if (!blocks) abort();
  }
  blocks[block_count].base = (uintptr_t)p;
  blocks[block_count].size = size;
  blocks[block_count].host = host;
  block_count++;
}

static int find_block(const void *p) {
  const uintptr_t a = (uintptr_t)p;
  for (int i = block_count - 1; i >= 0; --i)
    if (a >= blocks[i].base && a < blocks[i].base + blocks[i].size) return i;
  return -1;
}

static void drop_block(void *p) {
  for (int i = 0; i < block_count; ++i)
    if (blocks[i].base == (uintptr_t)p) {
      blocks[i] = blocks[--block_count];
      return;
    }
  note_violation("free of an address never allocated: %p", p);
}

/* [p, p + bytes) must lie inside one recorded allocation. */
static void check_range(const char *what, const char *arg, const void *p, size_t bytes) {
  int i;
  ++checks;
  if (!bytes) return;
  if (!p) {
    note_violation("%s: %s is NULL (%zu bytes needed)", what, arg, bytes);
    return;
  }
  i = find_block(p);
  if (i < 0) {
    note_violation("%s: %s = %p is in no allocation (%zu bytes needed)", what, arg, p, bytes);
    return;
  }
  if ((uintptr_t)p + bytes > blocks[i].base + blocks[i].size)
    note_violation("%s: %s overruns its allocation by %zu bytes (offset %zu + %zu > %zu)", what, arg,
                   (size_t)((uintptr_t)p + bytes - (blocks[i].base + blocks[i].size)),
                   (size_t)((uintptr_t)p - blocks[i].base), bytes, blocks[i].size);
}

/* rows of n elements, `stride` apart */
static size_t rows_bytes(int rows, size_t stride, size_t n, size_t elem) {
  if (rows < 1 || !n) return 0;
  return ((size_t)(rows - 1) * stride + n) * elem;
}

long audit_report(long *launch_count, long *check_count) {
  if (launch_count) *launch_count = launches;
  if (check_count) *check_count = checks;
  return violations;
}

/* ---- the runtime ----------------------------------------------------------- */

hipError_t hipMalloc(void **ptr, size_t size) {
  void *p = NULL;
  if (!ptr) return hipErrorInvalidValue;
  if (posix_memalign(&p, 256, size ? (size + 255) / 256 * 256 : 256)) return hipErrorOutOfMemory;
  /* zeroed up to a page (control words, counters); the rest is never read
   * before the host code writes it, and touching gigabytes costs minutes */
  memset(p, 0, size < 4096 ? size : 4096);
  add_block(p, size, 0);
  *ptr = p;
  return hipSuccess;
}

hipError_t hipFree(void *p) {
  if (!p) return hipSuccess;
  drop_block(p);
  free(p);
  return hipSuccess;
}

hipError_t hipHostMalloc(void **ptr, size_t size, unsigned int flags) {
  (void)flags;
  hipError_t e = hipMalloc(ptr, size);
  if (e == hipSuccess) blocks[block_count - 1].host = 1;
  return e;
}

hipError_t hipHostFree(void *p) { return hipFree(p); }

/* A copy's device side must be recorded; its host side is the caller's
 * memory, checked too where it is pinned (hipHostMalloc). */
static hipError_t copy_checked(const char *what, void *dst, const void *src, size_t bytes, hipMemcpyKind kind) {
  const int h2d = kind == hipMemcpyHostToDevice, d2h = kind == hipMemcpyDeviceToHost;
  if (!d2h || find_block(dst) >= 0) check_range(what, "dst", dst, bytes);
  if (!h2d || find_block(src) >= 0) check_range(what, "src", src, bytes);
  if (bytes) memmove(dst, src, bytes);
  return hipSuccess;
}

hipError_t hipMemcpy(void *dst, const void *src, size_t bytes, hipMemcpyKind kind) {
  return copy_checked("hipMemcpy", dst, src, bytes, kind);
}

hipError_t hipMemcpyAsync(void *dst, const void *src, size_t bytes, hipMemcpyKind kind, hipStream_t stream) {
  (void)stream;
  return copy_checked("hipMemcpyAsync", dst, src, bytes, kind);
}

hipError_t hipMemcpy2DAsync(void *dst, size_t dpitch, const void *src, size_t spitch, size_t width,
                            size_t height, hipMemcpyKind kind, hipStream_t stream) {
  (void)stream;
  if (!height || !width) return hipSuccess;
  if (kind == hipMemcpyHostToDevice || kind == hipMemcpyDeviceToDevice)
    check_range("hipMemcpy2DAsync", "dst", dst, (height - 1) * dpitch + width);
  if (kind == hipMemcpyDeviceToHost || kind == hipMemcpyDeviceToDevice)
    check_range("hipMemcpy2DAsync", "src", src, (height - 1) * spitch + width);
  for (size_t r = 0; r < height; ++r) memmove((char *)dst + r * dpitch, (const char *)src + r * spitch, width);
  return hipSuccess;
}

hipError_t hipMemsetAsync(void *dst, int value, size_t bytes, hipStream_t stream) {
  (void)stream;
  check_range("hipMemsetAsync", "dst", dst, bytes);
  if (bytes) memset(dst, value, bytes);
  return hipSuccess;
}

hipError_t hipSetDevice(int device) { return device == 0 ? hipSuccess : hipErrorInvalidDevice; }
hipError_t hipGetDeviceCount(int *count) {
  *count = 1;
  return hipSuccess;
}
hipError_t hipDeviceGetAttribute(int *value, hipDeviceAttribute_t attr, int device) {
  (void)device;
  switch (attr) {
    case hipDeviceAttributeMaxSharedMemoryPerBlock: *value = 160 * 1024; break;
    case hipDeviceAttributeMultiprocessorCount: *value = 256; break;
    case hipDeviceAttributeWarpSize: *value = 64; break;
    default: *value = 0; break;
  }
  return hipSuccess;
}

static hipError_t last_error;
hipError_t hipGetLastError(void) {
  hipError_t e = last_error;
  last_error = hipSuccess;
  return e;
}
const char *hipGetErrorString(hipError_t e) { return e == hipSuccess ? "hipSuccess" : "hip error (audit stub)"; }

hipError_t hipStreamCreateWithFlags(hipStream_t *stream, unsigned int flags) {
  (void)flags;
  *stream = (hipStream_t)malloc(64);
  return hipSuccess;
}
hipError_t hipStreamDestroy(hipStream_t stream) {
  free(stream);
  return hipSuccess;
}
hipError_t hipStreamSynchronize(hipStream_t stream) {
  (void)stream;
  return hipSuccess;
}

hipError_t hipEventCreate(hipEvent_t *event) {
  *event = (hipEvent_t)malloc(16);
  return hipSuccess;
}
hipError_t hipEventDestroy(hipEvent_t event) {
  free(event);
  return hipSuccess;
}
hipError_t hipEventRecord(hipEvent_t event, hipStream_t stream) {
  (void)event;
  (void)stream;
  return hipSuccess;
}
hipError_t hipEventSynchronize(hipEvent_t event) {
  (void)event;
  return hipSuccess;
}
hipError_t hipEventElapsedTime(float *ms, hipEvent_t start, hipEvent_t stop) {
  (void)start;
  (void)stop;
  *ms = 0.0f;
  return hipSuccess;
}

hipError_t hipStreamBeginCapture(hipStream_t stream, hipStreamCaptureMode mode) {
  (void)stream;
  (void)mode;
  return hipSuccess;
}
hipError_t hipStreamEndCapture(hipStream_t stream, hipGraph_t *graph) {
  (void)stream;
  *graph = (hipGraph_t)malloc(16);
  return hipSuccess;
}
hipError_t hipGraphInstantiate(hipGraphExec_t *exec, hipGraph_t graph, hipGraphNode_t *error_node, char *log,
                               size_t log_size) {
  (void)graph;
  (void)error_node;
  (void)log;
  (void)log_size;
  *exec = (hipGraphExec_t)malloc(16);
  return hipSuccess;
}
hipError_t hipGraphLaunch(hipGraphExec_t exec, hipStream_t stream) {
  (void)exec;
  (void)stream;
  return hipSuccess;
}
hipError_t hipGraphDestroy(hipGraph_t graph) {
  free(graph);
  return hipSuccess;
}
hipError_t hipGraphExecDestroy(hipGraphExec_t exec) {
  free(exec);
  return hipSuccess;
}

hipError_t hipFuncSetAttribute(const void *func, hipFuncAttribute attr, int value) {
  (void)func;
  if (attr == hipFuncAttributeMaxDynamicSharedMemorySize && (value < 0 || value > 160 * 1024))
    note_violation("hipFuncSetAttribute: %d bytes of dynamic LDS", value);
  return hipSuccess;
}

/* ---- code objects, variables and launches ------------------------------- */

typedef struct audit_var {
  const void *host;
  size_t size;
  void *dev;
} audit_var;
static audit_var vars[64];
static int var_count;

void **__hipRegisterFatBinary(const void *data) {
  (void)data;
  static void *handle;
  return &handle;
}
void __hipUnregisterFatBinary(void **modules) { (void)modules; }
void __hipRegisterFunction(void **modules, const void *host, char *dev_fn, const char *dev_name, unsigned int limit,
                           void *tid, void *bid, dim3 *block, dim3 *grid, int *wsize) {
  (void)modules; (void)host; (void)dev_fn; (void)dev_name; (void)limit;
  (void)tid; (void)bid; (void)block; (void)grid; (void)wsize;
}
void __hipRegisterVar(void **modules, void *var, char *host_name, char *dev_name, int ext, size_t size,
                      int constant, int global) {
  (void)modules; (void)host_name; (void)dev_name; (void)ext; (void)constant; (void)global;
  if (var_count < 64) {
    vars[var_count].host = var;
    vars[var_count].size = size;
    vars[var_count].dev = NULL;
    var_count++;
  }
}

/* A static __device__ array: its own recorded block, of the registered size. */
hipError_t hipGetSymbolAddress(void **dev, const void *symbol) {
  for (int i = 0; i < var_count; ++i)
    if (vars[i].host == symbol) {
      if (!vars[i].dev && hipMalloc(&vars[i].dev, vars[i].size) != hipSuccess) return hipErrorOutOfMemory;
      *dev = vars[i].dev;
      return hipSuccess;
    }
  return hipErrorInvalidSymbol;
}

static dim3 pushed_grid, pushed_block;
static size_t pushed_shared;
static hipStream_t pushed_stream;

hipError_t __hipPushCallConfiguration(dim3 grid, dim3 block, size_t shared, hipStream_t stream) {
  pushed_grid = grid;
  pushed_block = block;
  pushed_shared = shared;
  pushed_stream = stream;
  return hipSuccess;
}
hipError_t __hipPopCallConfiguration(dim3 *grid, dim3 *block, size_t *shared, hipStream_t *stream) {
  *grid = pushed_grid;
  *block = pushed_block;
  *shared = pushed_shared;
  *stream = pushed_stream;
  return hipSuccess;
}

/* gfx950 limits: grid x < 2^31, y and z <= 65535, a workgroup <= 1024
 * work-items (and each dimension likewise), dynamic LDS <= 160 KiB. */
hipError_t hipLaunchKernel(const void *fn, dim3 grid, dim3 block, void **args, size_t shared,
                           hipStream_t stream) {
  (void)fn;
  (void)args;
  (void)stream;
  ++launches;
  if (!grid.x || !grid.y || !grid.z || grid.x > 0x7FFFFFFFu || grid.y > 65535 || grid.z > 65535)
    note_violation("launch %ld: grid %u x %u x %u", launches, grid.x, grid.y, grid.z);
  if (!block.x || !block.y || !block.z || (size_t)block.x * block.y * block.z > 1024)
    note_violation("launch %ld: block %u x %u x %u", launches, block.x, block.y, block.z);
  if (shared > 160 * 1024) note_violation("launch %ld: %zu bytes of dynamic LDS", launches, shared);
  return hipSuccess;
}

/* ---- the launchers, checked ------------------------------------------------ */

#define W(name) __wrap_##name
#define R(name) __real_##name

static size_t code_row_bytes(int K, int bits) { return ((size_t)K * (size_t)bits + 7) / 8; }

/* A plane's codes and gains: N rows of row_stride bytes (the row's own
 * K * bits / 8 at least), N rows of gain_stride gains. */
static void check_plane(const char *what, const uint8_t *codes, long long row_stride, int K, int bits,
                        const float *gains, int gain_stride, int N) {
  check_range(what, "codes", codes, (size_t)(N - 1) * (size_t)row_stride + code_row_bytes(K, bits));
  if (gains) check_range(what, "gains", gains, (size_t)N * (size_t)gain_stride * sizeof(float));
}

static void check_view(const char *what, const igl_code_view *v, int K, int N) {
  check_plane(what, v->codes, v->row_stride, K, v->bit_count, v->gains, v->gain_stride, N);
}

/* lanes of state_in, state_out and lift lie lane_stride floats apart */
static void check_pro_lanes(const char *what, const igl_gemv_prologue *pro, int K, int lanes) {
  if (!pro) return;
  const size_t lane_bytes = ((size_t)(lanes - 1) * (size_t)pro->lane_stride + (size_t)K) * sizeof(float);
  check_range(what, "pro.state_in", pro->state_in, lane_bytes);
  if (pro->state_out) check_range(what, "pro.state_out", pro->state_out, lane_bytes);
  if (pro->lift) check_range(what, "pro.lift", pro->lift, lane_bytes);
  if (pro->lift_gain) check_range(what, "pro.lift_gain", pro->lift_gain, (size_t)K * sizeof(float));
  if (pro->norm_gain) check_range(what, "pro.norm_gain", pro->norm_gain, (size_t)K * sizeof(float));
}

static void check_pro(const char *what, const igl_gemv_prologue *pro, int K) { check_pro_lanes(what, pro, K, 1); }

hipError_t R(igl_launch_gemv_q4)(const uint8_t *, long long, const float *, int, int, int, const float *, int, int,
                                 float *, int, int, int, float *, int, hipStream_t);
hipError_t W(igl_launch_gemv_q4)(const uint8_t *codes, long long row_stride, const float *gains, int gain_stride,
                                 int group_shift, int code_bias, const float *act, int act_stride, int lanes,
                                 float *out, int out_stride, int N, int K, float *part, int lds_limit,
                                 hipStream_t stream) {
  const char *w = "igl_launch_gemv_q4";
  const size_t pf = igl_gemv_part_floats(lanes, N, K, lds_limit);
  check_plane(w, codes, row_stride, K, 4, gains, gain_stride, N);
  check_range(w, "act", act, rows_bytes(lanes, (size_t)act_stride, (size_t)K, 4));
  check_range(w, "out", out, rows_bytes(lanes, (size_t)out_stride, (size_t)N, 4));
  if (pf) check_range(w, "part", part, pf * sizeof(float));
  return R(igl_launch_gemv_q4)(codes, row_stride, gains, gain_stride, group_shift, code_bias, act, act_stride,
                               lanes, out, out_stride, N, K, part, lds_limit, stream);
}

hipError_t R(igl_launch_gemv_codes)(const igl_code_view *, const float *, int, int, float *, int, int, int, float *,
                                    hipStream_t);
hipError_t W(igl_launch_gemv_codes)(const igl_code_view *v, const float *act, int act_stride, int lanes, float *out,
                                    int out_stride, int N, int K, float *part, hipStream_t stream) {
  const char *w = "igl_launch_gemv_codes";
  const size_t pf = igl_gemv_code_part_floats(v->bit_count, lanes, N, K);
  check_view(w, v, K, N);
  check_range(w, "act", act, rows_bytes(lanes, (size_t)act_stride, (size_t)K, 4));
  check_range(w, "out", out, rows_bytes(lanes, (size_t)out_stride, (size_t)N, 4));
  if (pf) check_range(w, "part", part, pf * sizeof(float));
  return R(igl_launch_gemv_codes)(v, act, act_stride, lanes, out, out_stride, N, K, part, stream);
}

hipError_t R(igl_launch_gemv_zero)(const igl_code_view *, const int8_t *, const float *, int, int, float *, int, int,
                                   int, hipStream_t);
hipError_t W(igl_launch_gemv_zero)(const igl_code_view *v, const int8_t *zeros, const float *act, int act_stride,
                                   int lanes, float *out, int out_stride, int N, int K, hipStream_t stream) {
  const char *w = "igl_launch_gemv_zero";
  check_view(w, v, K, N);
  check_range(w, "zeros", zeros, (size_t)N * (size_t)v->gain_stride);
  check_range(w, "act", act, rows_bytes(lanes, (size_t)act_stride, (size_t)K, 4));
  check_range(w, "out", out, rows_bytes(lanes, (size_t)out_stride, (size_t)N, 4));
  return R(igl_launch_gemv_zero)(v, zeros, act, act_stride, lanes, out, out_stride, N, K, stream);
}

hipError_t R(igl_launch_gemv_real)(const void *, int, const float *, int, int, float *, int, int, int, float *,
                                   hipStream_t);
hipError_t W(igl_launch_gemv_real)(const void *rows, int real_type, const float *act, int act_stride, int lanes,
                                   float *out, int out_stride, int N, int K, float *part, hipStream_t stream) {
  const char *w = "igl_launch_gemv_real";
  const size_t pf = igl_gemv_real_part_floats(lanes, N, K);
  check_range(w, "rows", rows, (size_t)N * (size_t)K * (real_type == IGL_STORE_F32 ? 4u : 2u));
  check_range(w, "act", act, rows_bytes(lanes, (size_t)act_stride, (size_t)K, 4));
  check_range(w, "out", out, rows_bytes(lanes, (size_t)out_stride, (size_t)N, 4));
  if (pf) check_range(w, "part", part, pf * sizeof(float));
  return R(igl_launch_gemv_real)(rows, real_type, act, act_stride, lanes, out, out_stride, N, K, part, stream);
}

hipError_t R(igl_launch_gemv_level)(const igl_code_view *, float, float, const float *, int, int, float *, int, int,
                                    int, hipStream_t);
hipError_t W(igl_launch_gemv_level)(const igl_code_view *v, float step, float leave, const float *act, int act_stride,
                                    int lanes, float *out, int out_stride, int N, int K, hipStream_t stream) {
  const char *w = "igl_launch_gemv_level";
  check_view(w, v, K, N);
  check_range(w, "act", act, rows_bytes(lanes, (size_t)act_stride, (size_t)K, 4));
  check_range(w, "out", out, rows_bytes(lanes, (size_t)out_stride, (size_t)N, 4));
  return R(igl_launch_gemv_level)(v, step, leave, act, act_stride, lanes, out, out_stride, N, K, stream);
}

hipError_t R(igl_launch_gemv_level_epi)(const igl_code_view *, float, float, const float *, int, int, float *, int,
                                        int, int, int, const float *, int, hipStream_t);
hipError_t W(igl_launch_gemv_level_epi)(const igl_code_view *v, float step, float leave, const float *act,
                                        int act_stride, int lanes, float *out, int out_stride, int N, int K, int epi,
                                        const float *epi_in, int epi_stride, hipStream_t stream) {
  const char *w = "igl_launch_gemv_level_epi";
  check_view(w, v, K, N);
  check_range(w, "act", act, rows_bytes(lanes, (size_t)act_stride, (size_t)K, 4));
  check_range(w, "out", out, rows_bytes(lanes, (size_t)out_stride, (size_t)N, 4));
  if (epi) check_range(w, "epi_in", epi_in, rows_bytes(lanes, (size_t)epi_stride, (size_t)N, 4));
  return R(igl_launch_gemv_level_epi)(v, step, leave, act, act_stride, lanes, out, out_stride, N, K, epi, epi_in,
                                      epi_stride, stream);
}

hipError_t R(igl_launch_gemv_level_pro)(const igl_code_view *, float, float, const igl_gemv_prologue *, float *,
                                        float *, int, int, int, const float *, hipStream_t);
hipError_t W(igl_launch_gemv_level_pro)(const igl_code_view *v, float step, float leave, const igl_gemv_prologue *pro,
                                        float *x_out, float *out, int N, int K, int epi, const float *epi_in,
                                        hipStream_t stream) {
  const char *w = "igl_launch_gemv_level_pro";
  check_view(w, v, K, N);
  check_pro(w, pro, K);
  if (x_out) check_range(w, "x_out", x_out, (size_t)K * 4);
  check_range(w, "out", out, (size_t)N * 4);
  if (epi) check_range(w, "epi_in", epi_in, (size_t)N * 4);
  return R(igl_launch_gemv_level_pro)(v, step, leave, pro, x_out, out, N, K, epi, epi_in, stream);
}

hipError_t R(igl_launch_gemv_level_pair)(const igl_code_view *, const igl_code_view *, float, float, float,
                                         const igl_gemv_prologue *, float *, int, int, hipStream_t);
hipError_t W(igl_launch_gemv_level_pair)(const igl_code_view *gate, const igl_code_view *up, float step,
                                         float leave_gate, float leave_up, const igl_gemv_prologue *pro, float *out,
                                         int N, int K, hipStream_t stream) {
  const char *w = "igl_launch_gemv_level_pair";
  check_view(w, gate, K, N);
  check_view(w, up, K, N);
  check_pro(w, pro, K);
  check_range(w, "out", out, (size_t)N * 4);
  return R(igl_launch_gemv_level_pair)(gate, up, step, leave_gate, leave_up, pro, out, N, K, stream);
}

hipError_t R(igl_launch_gemv_level_segments)(const igl_code_view *, int, const int *, float *const *, const float *,
                                             float, const igl_gemv_prologue *, int, hipStream_t);
hipError_t W(igl_launch_gemv_level_segments)(const igl_code_view *v, int segments, const int *rows,
                                             float *const *out, const float *leave, float step,
                                             const igl_gemv_prologue *pro, int K, hipStream_t stream) {
  const char *w = "igl_launch_gemv_level_segments";
  for (int s = 0; s < segments; ++s) {
    check_view(w, &v[s], K, rows[s]);
    check_range(w, "out[s]", out[s], (size_t)rows[s] * 4);
  }
  check_pro(w, pro, K);
  return R(igl_launch_gemv_level_segments)(v, segments, rows, out, leave, step, pro, K, stream);
}

hipError_t R(igl_launch_gemv_group)(int, int, int, const uint8_t *const *, const long long *, const float *const *,
                                    const int *, const int *, float *const *, const int *, int, int, const float *,
                                    int, int, const float *, int, const igl_gemv_prologue *, hipStream_t);
hipError_t W(igl_launch_gemv_group)(int mode, int lanes, int segments, const uint8_t *const *codes,
                                    const long long *row_stride, const float *const *gains, const int *gain_stride,
                                    const int *rows, float *const *out, const int *out_stride, int group_shift,
                                    int code_bias, const float *act, int act_stride, int K, const float *mul,
                                    int mul_stride, const igl_gemv_prologue *pro, hipStream_t stream) {
  const char *w = "igl_launch_gemv_group";
  const size_t before = (size_t)(lanes - 1);
  for (int s = 0; s < segments; ++s) {
    check_plane(w, codes[s], row_stride[s], K, 4, gains[s], gain_stride[s], rows[s]);
    /* GELU_PAIR writes gelu(gate) * up once, into out[0] */
    if (mode != IGL_GEMV_GELU_PAIR || s == 0)
      check_range(w, "out[s]", out[s], (before * (size_t)out_stride[s] + (size_t)rows[s]) * 4);
  }
  if (pro) check_pro_lanes(w, pro, K, lanes);
  else check_range(w, "act", act, (before * (size_t)act_stride + (size_t)K) * 4);
  if (mode == IGL_GEMV_GELU_MUL) check_range(w, "mul", mul, (before * (size_t)mul_stride + (size_t)rows[0]) * 4);
  return R(igl_launch_gemv_group)(mode, lanes, segments, codes, row_stride, gains, gain_stride, rows, out, out_stride,
                                  group_shift, code_bias, act, act_stride, K, mul, mul_stride, pro, stream);
}

hipError_t R(igl_launch_gemm_q4)(const void *, int, int, const uint8_t *, long long, const float *, int, int, int,
                                 const uint32_t *, void *, int, int, int, int, int, int, void *,
                                 const igl_gemm_close *, hipStream_t);
hipError_t W(igl_launch_gemm_q4)(const void *act, int act_bf16, int act_stride, const uint8_t *codes,
                                 long long row_stride, const float *gains, int gain_stride, int group_shift,
                                 int code_bias, const uint32_t *zero_pairs, void *out, int out_bf16, int out_stride,
                                 int M, int N, int K, int act_terms, void *work, const igl_gemm_close *close,
                                 hipStream_t stream) {
  const char *w = "igl_launch_gemm_q4";
  check_plane(w, codes, row_stride, K, 4, gains, gain_stride, N);
  if (zero_pairs) check_range(w, "zero_pairs", zero_pairs, (size_t)N * (size_t)gain_stride * 4);
  check_range(w, "act", act, rows_bytes(M, (size_t)act_stride, (size_t)K, act_bf16 ? 2 : 4));
  check_range(w, "out", out, rows_bytes(M, (size_t)out_stride, (size_t)N, out_bf16 ? 2 : 4));
  check_range(w, "work", work, igl_gemm_work_bytes(M, N, K, act_terms));
  if (close && close->gains) check_range(w, "close.gains", close->gains, (size_t)N * 4);
  return R(igl_launch_gemm_q4)(act, act_bf16, act_stride, codes, row_stride, gains, gain_stride, group_shift,
                               code_bias, zero_pairs, out, out_bf16, out_stride, M, N, K, act_terms, work, close,
                               stream);
}

hipError_t R(igl_launch_gemm_level)(const float *, int, const uint8_t *, long long, int, int, int,
                                    const igl_gemm_close *, float *, int, int, int, int, void *, hipStream_t);
hipError_t W(igl_launch_gemm_level)(const float *act, int act_stride, const uint8_t *codes, long long row_stride,
                                    int bits, int code_flip, int code_bias, const igl_gemm_close *close, float *out,
                                    int out_stride, int M, int N, int K, void *work, hipStream_t stream) {
  const char *w = "igl_launch_gemm_level";
  check_plane(w, codes, row_stride, K, bits, NULL, 0, N);
  check_range(w, "act", act, rows_bytes(M, (size_t)act_stride, (size_t)K, 4));
  check_range(w, "out", out, rows_bytes(M, (size_t)out_stride, (size_t)N, 4));
  check_range(w, "work", work, igl_gemm_level_work_bytes(M, N, K, bits));
  if (close && close->gains) check_range(w, "close.gains", close->gains, (size_t)N * 4);
  return R(igl_launch_gemm_level)(act, act_stride, codes, row_stride, bits, code_flip, code_bias, close, out,
                                  out_stride, M, N, K, work, stream);
}

hipError_t R(igl_launch_attend)(const uint8_t *, const uint8_t *, int, float, float, int, int, int, int, int,
                                const float *, int, int, const int *, int, int, float, float *, float *, hipStream_t);
hipError_t W(igl_launch_attend)(const uint8_t *key_store, const uint8_t *value_store, int fmt, float key_scale,
                                float value_scale, int cache_span, int kv_width, int kv_count, int group_share,
                                int head_size, const float *query, int q_stride, int place0, const int *place_dev,
                                int window, int lanes, float score_scale, float *blend_out, float *work,
                                hipStream_t stream) {
  const char *w = "igl_launch_attend";
  const size_t heads = (size_t)kv_count * (size_t)group_share;
  check_range(w, "key_store", key_store, (size_t)cache_span * (size_t)kv_width);
  check_range(w, "value_store", value_store, (size_t)cache_span * (size_t)kv_width);
  check_range(w, "query", query, rows_bytes(lanes, (size_t)q_stride, heads * (size_t)head_size, 4));
  check_range(w, "blend_out", blend_out, rows_bytes(lanes, (size_t)q_stride, heads * (size_t)head_size, 4));
  if (place_dev) check_range(w, "place_dev", place_dev, 4);
  check_range(w, "work", work,
              igl_attend_work_floats(place0, window, lanes, (int)heads, head_size) * sizeof(float));
  return R(igl_launch_attend)(key_store, value_store, fmt, key_scale, value_scale, cache_span, kv_width, kv_count,
                              group_share, head_size, query, q_stride, place0, place_dev, window, lanes, score_scale,
                              blend_out, work, stream);
}

hipError_t R(igl_launch_attend_prep)(const uint8_t *, const uint8_t *, float, float, int, int, int, const float *, int,
                                     const float *, const float *, int, const float *, const float *, int,
                                     const float *, uint8_t *, uint8_t *, float, int, const int *, int, float, float *,
                                     float *, hipStream_t);
hipError_t W(igl_launch_attend_prep)(const uint8_t *key_store, const uint8_t *value_store, float key_scale,
                                     float value_scale, int cache_span, int head_size, int lanes, const float *query,
                                     int q_stride, const float *q_gain, const float *turn, int turn_stride,
                                     const float *k_raw, const float *v_raw, int kv_stride, const float *k_gain,
                                     uint8_t *k_ring, uint8_t *v_ring, float eps, int place_bound,
                                     const int *place_dev, int window, float score_scale, float *blend_out,
                                     float *work, hipStream_t stream) {
  const char *w = "igl_launch_attend_prep";
  const size_t qs = lanes > 1 ? (size_t)q_stride : 8 * (size_t)head_size;
  check_range(w, "key_store", key_store, (size_t)cache_span * (size_t)head_size);
  check_range(w, "value_store", value_store, (size_t)cache_span * (size_t)head_size);
  check_range(w, "query", query, rows_bytes(lanes, qs, 8 * (size_t)head_size, 4));
  check_range(w, "q_gain", q_gain, (size_t)head_size * 4);
  /* head_size / 2 (cos, sin) pairs a lane */
  check_range(w, "turn", turn, rows_bytes(lanes, (size_t)turn_stride, (size_t)head_size, 4));
  check_range(w, "place_dev", place_dev, 4);
  if (k_raw) {
    check_range(w, "k_raw", k_raw, rows_bytes(lanes, (size_t)kv_stride, (size_t)head_size, 4));
    check_range(w, "v_raw", v_raw, rows_bytes(lanes, (size_t)kv_stride, (size_t)head_size, 4));
    check_range(w, "k_gain", k_gain, (size_t)head_size * 4);
    check_range(w, "k_ring", k_ring, (size_t)cache_span * (size_t)head_size);
    check_range(w, "v_ring", v_ring, (size_t)cache_span * (size_t)head_size);
  }
  check_range(w, "blend_out", blend_out, rows_bytes(lanes, qs, 8 * (size_t)head_size, 4));
  check_range(w, "work", work, igl_attend_prep_work_floats(place_bound, window, head_size, lanes, k_raw != NULL) * 4);
  return R(igl_launch_attend_prep)(key_store, value_store, key_scale, value_scale, cache_span, head_size, lanes, query,
                                   q_stride, q_gain, turn, turn_stride, k_raw, v_raw, kv_stride, k_gain, k_ring,
                                   v_ring, eps, place_bound, place_dev, window, score_scale, blend_out, work, stream);
}

hipError_t R(igl_launch_gather_rows)(const igl_code_view *, int, int, const int32_t *, int, float, float *, int,
                                     hipStream_t);
hipError_t W(igl_launch_gather_rows)(const igl_code_view *v, int cols, int rows, const int32_t *ids, int lanes,
                                     float factor, float *out, int out_stride, hipStream_t stream) {
  const char *w = "igl_launch_gather_rows";
  check_view(w, v, cols, rows);
  /* the kernel clamps an id into 0 .. rows - 1 itself */
  check_range(w, "ids", ids, (size_t)lanes * 4);
  check_range(w, "out", out, rows_bytes(lanes, (size_t)out_stride, (size_t)cols, 4));
  return R(igl_launch_gather_rows)(v, cols, rows, ids, lanes, factor, out, out_stride, stream);
}

hipError_t R(igl_launch_ple_mix)(float *, int, const float *, int, const float *, int, int, int, float, float, float,
                                 hipStream_t);
hipError_t W(igl_launch_ple_mix)(float *room, int room_stride, const float *seed, int seed_stride, const float *gain,
                                 int ple, int chunks, int lanes, float eps, float lift_scale, float blend,
                                 hipStream_t stream) {
  const char *w = "igl_launch_ple_mix";
  check_range(w, "room", room, rows_bytes(lanes, (size_t)room_stride, (size_t)chunks * (size_t)ple, 4));
  check_range(w, "seed", seed, rows_bytes(lanes, (size_t)seed_stride, (size_t)chunks * (size_t)ple, 4));
  check_range(w, "gain", gain, (size_t)ple * 4);
  return R(igl_launch_ple_mix)(room, room_stride, seed, seed_stride, gain, ple, chunks, lanes, eps, lift_scale, blend,
                               stream);
}

hipError_t R(igl_launch_put_int)(int32_t *, int, hipStream_t);
hipError_t W(igl_launch_put_int)(int32_t *dst, int value, hipStream_t stream) {
  check_range("igl_launch_put_int", "dst", dst, 4);
  return R(igl_launch_put_int)(dst, value, stream);
}

hipError_t R(igl_launch_turn_row)(const float *, int, const float *, int, const int *, int, float *, float *,
                                  hipStream_t);
hipError_t W(igl_launch_turn_row)(const float *step0, int half0, const float *step1, int half1, const int *place_dev,
                                  int lanes, float *turn0, float *turn1, hipStream_t stream) {
  const char *w = "igl_launch_turn_row";
  if (step0) {
    check_range(w, "step0", step0, (size_t)half0 * 4);
    check_range(w, "turn0", turn0, (size_t)lanes * (size_t)half0 * 8);
  }
  if (step1) {
    check_range(w, "step1", step1, (size_t)half1 * 4);
    check_range(w, "turn1", turn1, (size_t)lanes * (size_t)half1 * 8);
  }
  check_range(w, "place_dev", place_dev, 4);
  return R(igl_launch_turn_row)(step0, half0, step1, half1, place_dev, lanes, turn0, turn1, stream);
}

hipError_t R(igl_launch_qkv_prep)(float *, int, const float *, const float *, int, int, int, int, const float *,
                                  const float *, float, const float *, const int *, uint8_t *, uint8_t *, float, float,
                                  int, hipStream_t);
hipError_t W(igl_launch_qkv_prep)(float *q, int q_stride, const float *k, const float *v, int kv_stride, int heads,
                                  int head_size, int lanes, const float *q_gain, const float *k_gain, float eps,
                                  const float *step, const int *place_dev, uint8_t *k_store, uint8_t *v_store,
                                  float k_scale, float v_scale, int span, hipStream_t stream) {
  const char *w = "igl_launch_qkv_prep";
  check_range(w, "q", q, rows_bytes(lanes, (size_t)q_stride, (size_t)heads * (size_t)head_size, 4));
  check_range(w, "q_gain", q_gain, (size_t)head_size * 4);
  check_range(w, "step", step, (size_t)(head_size / 2) * 4);
  check_range(w, "place_dev", place_dev, 4);
  if (k) {
    check_range(w, "k", k, rows_bytes(lanes, (size_t)kv_stride, (size_t)head_size, 4));
    check_range(w, "v", v, rows_bytes(lanes, (size_t)kv_stride, (size_t)head_size, 4));
    check_range(w, "k_gain", k_gain, (size_t)head_size * 4);
    check_range(w, "k_store", k_store, (size_t)span * (size_t)head_size);
    check_range(w, "v_store", v_store, (size_t)span * (size_t)head_size);
  }
  return R(igl_launch_qkv_prep)(q, q_stride, k, v, kv_stride, heads, head_size, lanes, q_gain, k_gain, eps, step,
                                place_dev, k_store, v_store, k_scale, v_scale, span, stream);
}

hipError_t R(igl_launch_norm_add)(float *, int, const float *, int, const float *, int, int, float, float, int,
                                  const float *, float *, int, hipStream_t);
hipError_t W(igl_launch_norm_add)(float *state, int state_stride, const float *lift, int lift_stride,
                                  const float *after_gain, int n, int lanes, float eps, float scale, int apply_scale,
                                  const float *next_gain, float *out, int out_stride, hipStream_t stream) {
  const char *w = "igl_launch_norm_add";
  check_range(w, "state", state, rows_bytes(lanes, (size_t)state_stride, (size_t)n, 4));
  check_range(w, "lift", lift, rows_bytes(lanes, (size_t)lift_stride, (size_t)n, 4));
  check_range(w, "after_gain", after_gain, (size_t)n * 4);
  if (next_gain) check_range(w, "next_gain", next_gain, (size_t)n * 4);
  if (out) check_range(w, "out", out, rows_bytes(lanes, (size_t)out_stride, (size_t)n, 4));
  return R(igl_launch_norm_add)(state, state_stride, lift, lift_stride, after_gain, n, lanes, eps, scale, apply_scale,
                                next_gain, out, out_stride, stream);
}

hipError_t R(igl_launch_add_rows)(float *, int, const float *, int, int, int, float, int, hipStream_t);
hipError_t W(igl_launch_add_rows)(float *into, int into_stride, const float *from, int from_stride, int n, int lanes,
                                  float gain, int apply_gain, hipStream_t stream) {
  check_range("igl_launch_add_rows", "into", into, rows_bytes(lanes, (size_t)into_stride, (size_t)n, 4));
  check_range("igl_launch_add_rows", "from", from, rows_bytes(lanes, (size_t)from_stride, (size_t)n, 4));
  return R(igl_launch_add_rows)(into, into_stride, from, from_stride, n, lanes, gain, apply_gain, stream);
}

hipError_t R(igl_launch_scale_rows)(float *, int, int, int, float, hipStream_t);
hipError_t W(igl_launch_scale_rows)(float *v, int stride, int n, int lanes, float gain, hipStream_t stream) {
  check_range("igl_launch_scale_rows", "v", v, rows_bytes(lanes, (size_t)stride, (size_t)n, 4));
  return R(igl_launch_scale_rows)(v, stride, n, lanes, gain, stream);
}

hipError_t R(igl_launch_gelu_mul)(float *, int, const float *, int, int, int, hipStream_t);
hipError_t W(igl_launch_gelu_mul)(float *gate, int gate_stride, const float *ple, int ple_stride, int n, int lanes,
                                  hipStream_t stream) {
  check_range("igl_launch_gelu_mul", "gate", gate, rows_bytes(lanes, (size_t)gate_stride, (size_t)n, 4));
  check_range("igl_launch_gelu_mul", "ple", ple, rows_bytes(lanes, (size_t)ple_stride, (size_t)n, 4));
  return R(igl_launch_gelu_mul)(gate, gate_stride, ple, ple_stride, n, lanes, stream);
}

hipError_t R(igl_launch_gelu_gate_rows)(float *, int, const float *, int, int, int, hipStream_t);
hipError_t W(igl_launch_gelu_gate_rows)(float *gate, int gate_stride, const float *rise, int rise_stride, int n,
                                        int lanes, hipStream_t stream) {
  check_range("igl_launch_gelu_gate_rows", "gate", gate, rows_bytes(lanes, (size_t)gate_stride, (size_t)n, 4));
  check_range("igl_launch_gelu_gate_rows", "rise", rise, rows_bytes(lanes, (size_t)rise_stride, (size_t)n, 4));
  return R(igl_launch_gelu_gate_rows)(gate, gate_stride, rise, rise_stride, n, lanes, stream);
}

hipError_t R(igl_launch_pick)(float *, int, size_t, int, float, void *, int32_t *, hipStream_t);
hipError_t W(igl_launch_pick)(float *v, int n, size_t stride, int lanes, float cap, void *work, int32_t *pairs,
                              hipStream_t stream) {
  check_range("igl_launch_pick", "v", v, rows_bytes(lanes, stride, (size_t)n, 4));
  check_range("igl_launch_pick", "work", work, igl_pick_work_bytes(lanes));
  check_range("igl_launch_pick", "pairs", pairs, (size_t)lanes * 8);
  return R(igl_launch_pick)(v, n, stride, lanes, cap, work, pairs, stream);
}

hipError_t R(igl_launch_norm_rms)(const float *, const float *, int, int, int, float, float *, hipStream_t);
hipError_t W(igl_launch_norm_rms)(const float *in, const float *gain, int n, int rows, int stride, float eps,
                                  float *out, hipStream_t stream) {
  check_range("igl_launch_norm_rms", "in", in, rows_bytes(rows, (size_t)stride, (size_t)n, 4));
  check_range("igl_launch_norm_rms", "out", out, rows_bytes(rows, (size_t)stride, (size_t)n, 4));
  if (gain) check_range("igl_launch_norm_rms", "gain", gain, (size_t)n * 4);
  return R(igl_launch_norm_rms)(in, gain, n, rows, stride, eps, out, stream);
}

hipError_t R(igl_launch_quant_step)(const float *, int, float *, int, int, int, float, hipStream_t);
hipError_t W(igl_launch_quant_step)(const float *src, int src_stride, float *dst, int dst_stride, int n, int lanes,
                                    float step, hipStream_t stream) {
  check_range("igl_launch_quant_step", "src", src, rows_bytes(lanes, (size_t)src_stride, (size_t)n, 4));
  check_range("igl_launch_quant_step", "dst", dst, rows_bytes(lanes, (size_t)dst_stride, (size_t)n, 4));
  return R(igl_launch_quant_step)(src, src_stride, dst, dst_stride, n, lanes, step, stream);
}

hipError_t R(igl_launch_fill)(float *, size_t, float, hipStream_t);
hipError_t W(igl_launch_fill)(float *dst, size_t n, float value, hipStream_t stream) {
  check_range("igl_launch_fill", "dst", dst, n * 4);
  return R(igl_launch_fill)(dst, n, value, stream);
}
