/* back_hip.c - the C11 shim that fills igllm's backend table with the gfx950
 * kernels.
 *
 * It owns what back_open owned on the CPU (app_core.c:5415-5443): the scratch
 * a product needs, allocated once, so nothing is allocated in the token loop.
 * Here that is device staging, a HIP stream (default priority), two timing
 * events and the sticky error the void entries report through.  Every entry
 * checks shapes, strides and alignment on the host before anything is
 * launched; an entry that cannot run records IGL_FAIL_SUPPORT or
 * IGL_FAIL_ARGUMENT and leaves its output unwritten.  There is no CPU path.
 */
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "igl_backend.h"
#include "igl_launch.h"

#define IGL_GEMV_LANES 8  /* lanes one GEMV launch carries */
#define IGL_GEMV_Q4_LANES 16 /* lanes one 4-bit GEMV launch carries (the matrix-core form) */
#define IGL_GEMM_FLOOR 64 /* lanes from which mat_mat takes the MFMA GEMM */

struct igl_device_plane {
  const void  *codes;
  const float *gains;
  int          owned; /* allocated by igl_plane_attach */
  /* zero points (bias_data), always owned: int8 [rows][groups] for the GEMV,
   * and for 4-bit unflipped planes the GEMM's binary16 pairs
   * (1024 + bias + zero, 1024 + 16 (bias + zero)) a word */
  int8_t      *zeros;
  uint32_t    *zero_pairs;
};

struct igl_desk_state {
  int         device;
  hipStream_t stream;
  hipEvent_t  mark[2];
  int         mark_turn;
  int         marks_made;
  int         error;
  int         lane_limit;
  int         col_limit;
  int         sum_limit;
  int         lds_limit;  /* LDS bytes a workgroup may hold on this device */
  /* The table entries share the staging below, and the reference calls one of
   * them (soft_max, from attend_blend_band app_core.c:11333-11346) from every
   * worker of its pool at once: the entries take this lock. */
  pthread_mutex_t table_lock;
  int             table_lock_live;
  /* device and pinned staging for the host-pointer table entries */
  float *act_dev;
  float *act_pin;
  float *out_dev;
  float *out_pin;
  size_t out_floats;
  /* GEMV K-chunk partials and attention split partials */
  float *part_dev;
  size_t part_floats;
  float *work_dev;
  size_t work_floats;
  float *quant_dev;   /* plane_lift: the activations on the plane's entry grid */
  size_t quant_floats;
  /* plane_lift's prefill on the grid: widened codes, unit gains, level sums,
   * the two planes' products of an 8-bit plane */
  float *wide_dev;
  size_t wide_floats;
  float *ones_dev;
  size_t ones_floats;
  float *lsum_dev;
  size_t lsum_floats;
  float *prod_dev;
  size_t prod_floats;
  /* staging for the elementwise host entries */
  float *elem_dev;
  size_t elem_floats;
  /* the GEMM's binary16 copy of its activations */
  float *gemm_dev;
  size_t gemm_floats;
  /* a recording in progress on the stream, and replays not yet freed (both
   * freeze the scratch above: a replay keeps the addresses it recorded) */
  int recording;
  int record_error;  /* the first failure while recording (error_take keeps it) */
  int replays_live;
  /* counts the workspace reallocations: a graph captured by a caller outside
   * the recording API is stale once it changes (igl_desk_generation) */
  unsigned generation;
};

struct igl_replay {
  hipGraphExec_t exec;
  igl_desk_state *owner;
};

static void desk_fail(igl_desk_state *st, int code) {
  if (st && st->error == IGL_OKAY) st->error = code;
  if (st && st->recording && st->record_error == IGL_OKAY) st->record_error = code;
}

/* Entries that touch host memory, synchronize or allocate cannot be recorded. */
static int refuse_recording(igl_desk_state *st) {
  if (!st->recording) return 0;
  desk_fail(st, IGL_FAIL_STATE);
  return 1;
}

static int hip_check(igl_desk_state *st, hipError_t e) {
  if (e == hipSuccess) return IGL_OKAY;
  desk_fail(st, e == hipErrorOutOfMemory ? IGL_FAIL_MEMORY : IGL_FAIL_DEVICE);
  return e == hipErrorOutOfMemory ? IGL_FAIL_MEMORY : IGL_FAIL_DEVICE;
}

const char *igl_code_text(int code) {
  switch (code) {
    case IGL_OKAY: return "okay";
    case IGL_FAIL_ARGUMENT: return "bad argument";
    case IGL_FAIL_MEMORY: return "out of memory";
    case IGL_FAIL_FILE: return "file error";
    case IGL_FAIL_FORMAT: return "bad format";
    case IGL_FAIL_MISSING: return "missing";
    case IGL_FAIL_SUPPORT: return "unsupported by the gfx950 backend";
    case IGL_FAIL_STATE: return "bad state";
    case IGL_FAIL_DEVICE: return "device error";
    default: return "unknown";
  }
}

void *igl_desk_stream(igl_desk *desk) {
  return desk && desk->state ? (void *)desk->state->stream : NULL;
}

int igl_desk_error_take(igl_desk *desk) {
  int code;
  if (!desk || !desk->state) return IGL_FAIL_STATE;
  code = desk->state->error;
  desk->state->error = IGL_OKAY;
  return code;
}

/* Grows a device buffer to at least `floats`; used only at load time or on
 * the first call that needs more room. */
static int grow_dev(igl_desk_state *st, float **buf, size_t *have, size_t floats) {
  void *fresh = NULL;
  if (*have >= floats) return IGL_OKAY;
  if (st->recording || st->replays_live) {
    desk_fail(st, IGL_FAIL_STATE);
    return IGL_FAIL_STATE;
  }
  if (hipMalloc(&fresh, floats * sizeof(float)) != hipSuccess) {
    desk_fail(st, IGL_FAIL_MEMORY);
    return IGL_FAIL_MEMORY;
  }
  if (*buf) (void)hipFree(*buf);
  *buf = (float *)fresh;
  *have = floats;
  st->generation += 1;
  return IGL_OKAY;
}

static int grow_out(igl_desk_state *st, size_t floats) {
  void *dev = NULL, *pin = NULL;
  if (st->out_floats >= floats) return IGL_OKAY;
  if (st->recording || st->replays_live) {
    desk_fail(st, IGL_FAIL_STATE);
    return IGL_FAIL_STATE;
  }
  if (hipMalloc(&dev, floats * sizeof(float)) != hipSuccess) goto fail;
  if (hipHostMalloc(&pin, floats * sizeof(float), hipHostMallocDefault) != hipSuccess) goto fail;
  if (st->out_dev) (void)hipFree(st->out_dev);
  if (st->out_pin) (void)hipHostFree(st->out_pin);
  st->out_dev = (float *)dev;
  st->out_pin = (float *)pin;
  st->out_floats = floats;
  st->generation += 1;
  return IGL_OKAY;
fail:
  if (dev) (void)hipFree(dev);
  desk_fail(st, IGL_FAIL_MEMORY);
  return IGL_FAIL_MEMORY;
}

/* ---- plane checks -------------------------------------------------------- */

static int is_pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }

/* Bytes of one value of a real plane the kernels read, 0 for other types. */
static int real_bytes_of(int real_type) {
  return real_type == IGL_STORE_F32 ? 4 : real_type == IGL_STORE_F16 || real_type == IGL_STORE_BF16 ? 2 : 0;
}

/* The planes the kernels take: real planes of F32, F16 or BF16 rows, K a
 * multiple of 8; code planes of 2, 4 or 8-bit codes with the offset of half
 * their range (code_bias = 2^(bits-1)) and any flip (the signed I8 planes flip
 * 128), F32 gains over groups of 32 times a power of two columns or one group
 * a row.  Everything else is refused, not emulated. */
static int plane_supported(const igl_plane *sheet) {
  if (sheet && sheet->form == IGL_PLANE_REAL)
    return real_bytes_of(sheet->real_type) && sheet->row_count >= 1 && sheet->col_count >= 8 &&
                   (sheet->col_count & 7) == 0
               ? IGL_OKAY
               : IGL_FAIL_SUPPORT;
  if (!sheet || sheet->form != IGL_PLANE_CODE) return IGL_FAIL_SUPPORT;
  if (sheet->bit_count != 2 && sheet->bit_count != 4 && sheet->bit_count != 8) return IGL_FAIL_SUPPORT;
  if (sheet->code_bias != 1 << (sheet->bit_count - 1) || sheet->code_flip < 0 ||
      sheet->code_flip >= 1 << sheet->bit_count)
    return IGL_FAIL_SUPPORT;
  if (sheet->gain_type != IGL_STORE_F32) return IGL_FAIL_SUPPORT;
  if (sheet->row_count < 1 || sheet->col_count < 32 || (sheet->col_count & 31)) return IGL_FAIL_SUPPORT;
  if (sheet->group_count == 1) {
    if (sheet->group_size < sheet->col_count) return IGL_FAIL_SUPPORT;
  } else {
    if (sheet->group_size < 32 || (sheet->group_size & 31) || !is_pow2(sheet->group_size / 32))
      return IGL_FAIL_SUPPORT;
    if (sheet->group_count * sheet->group_size < sheet->col_count ||
        (sheet->group_count - 1) * sheet->group_size >= sheet->col_count)
      return IGL_FAIL_SUPPORT;
  }
  if ((sheet->row_stride & 15u) ||
      sheet->row_stride < ((size_t)sheet->col_count * (size_t)sheet->bit_count + 7u) / 8u)
    return IGL_FAIL_SUPPORT;
  return IGL_OKAY;
}

/* The tuned 4-bit kernels take codes stored value + 8 with no flip; every
 * other code plane goes through the every-width form. */
static int plane_is_q4(const igl_plane *sheet) {
  return sheet->form == IGL_PLANE_CODE && sheet->bit_count == 4 && sheet->code_flip == 0;
}

/* Room the GEMV's K-chunk partials need for this plane, over every lane count
 * a launch can carry. */
static size_t plane_part_floats(const igl_desk_state *st, const igl_plane *sheet) {
  size_t most = 0;
  if (sheet->form == IGL_PLANE_REAL)
    return igl_gemv_real_part_floats(IGL_GEMV_LANES, sheet->row_count, sheet->col_count);
  if (!plane_is_q4(sheet))
    return igl_gemv_code_part_floats(sheet->bit_count, IGL_GEMV_LANES, sheet->row_count,
                                     sheet->col_count);
  for (int lanes = 1; lanes <= IGL_GEMV_Q4_LANES; ++lanes) {
    size_t need = igl_gemv_part_floats(lanes, sheet->row_count, sheet->col_count, st->lds_limit);
    if (need > most) most = need;
  }
  return most;
}

static int plane_reserve(igl_desk_state *st, const igl_plane *sheet) {
  size_t part = plane_part_floats(st, sheet);
  size_t out = (size_t)st->lane_limit * (size_t)sheet->row_count;
  if (part && grow_dev(st, &st->part_dev, &st->part_floats, part) != IGL_OKAY) return IGL_FAIL_MEMORY;
  return grow_out(st, out);
}

/* The plane's zero points on the device (none without bias_data): the int8
 * table as it stands, and for 4-bit unflipped planes whose bias + zero stays
 * in 0..63 the GEMM's binary16 subtrahends, 1024 + (bias + zero) and
 * 1024 + 16 (bias + zero), exact integers in [1024, 2048) (exponent field 25:
 * 0x6400 plus the integer). */
static int attach_zeros(const igl_plane *sheet, igl_device_plane *dp) {
  const size_t count = (size_t)sheet->row_count * (size_t)sheet->group_count;
  uint32_t *pairs = NULL;
  int pairs_ok = sheet->bit_count == 4 && sheet->code_flip == 0;
  if (sheet->form != IGL_PLANE_CODE || !sheet->bias_data) return IGL_OKAY;
  if (hipMalloc((void **)&dp->zeros, count) != hipSuccess) return IGL_FAIL_MEMORY;
  if (hipMemcpy(dp->zeros, sheet->bias_data, count, hipMemcpyHostToDevice) != hipSuccess)
    return IGL_FAIL_DEVICE;
  for (size_t i = 0; i < count && pairs_ok; ++i) {
    const int bz = sheet->code_bias + sheet->bias_data[i];
    if (bz < 0 || bz > 63) pairs_ok = 0;
  }
  if (!pairs_ok) return IGL_OKAY;
  pairs = (uint32_t *)malloc(count * sizeof(uint32_t));
  if (!pairs) return IGL_FAIL_MEMORY;
  for (size_t i = 0; i < count; ++i) {
    const uint32_t bz = (uint32_t)(sheet->code_bias + sheet->bias_data[i]);
    pairs[i] = (0x6400u + bz) | ((0x6400u + 16u * bz) << 16);
  }
  if (hipMalloc((void **)&dp->zero_pairs, count * sizeof(uint32_t)) != hipSuccess) {
    free(pairs);
    return IGL_FAIL_MEMORY;
  }
  if (hipMemcpy(dp->zero_pairs, pairs, count * sizeof(uint32_t), hipMemcpyHostToDevice) != hipSuccess) {
    free(pairs);
    return IGL_FAIL_DEVICE;
  }
  free(pairs);
  return IGL_OKAY;
}

static void free_zeros(igl_device_plane *dp) {
  if (dp->zeros) (void)hipFree(dp->zeros);
  if (dp->zero_pairs) (void)hipFree(dp->zero_pairs);
  dp->zeros = NULL;
  dp->zero_pairs = NULL;
}

int igl_plane_attach(igl_desk *desk, igl_plane *sheet) {
  igl_desk_state *st = desk ? desk->state : NULL;
  igl_device_plane *dp;
  size_t code_bytes, gain_bytes;
  void *codes = NULL, *gains = NULL;
  int code;
  if (!st) return IGL_FAIL_STATE;
  const void *code_src, *gain_src;
  if ((code = plane_supported(sheet)) != IGL_OKAY) return code;
  if (sheet->form == IGL_PLANE_REAL) {
    /* a real plane's rows travel as the codes, with no gains */
    code_src = sheet->real_data;
    gain_src = NULL;
    code_bytes = (size_t)sheet->row_count * (size_t)sheet->col_count * (size_t)real_bytes_of(sheet->real_type);
    gain_bytes = 0;
    if (!code_src) return IGL_FAIL_ARGUMENT;
  } else {
    code_src = sheet->code_data;
    gain_src = sheet->gain_data;
    code_bytes = (size_t)sheet->row_count * sheet->row_stride;
    gain_bytes = (size_t)sheet->row_count * (size_t)sheet->group_count * sizeof(float);
    if (!code_src || !gain_src) return IGL_FAIL_ARGUMENT;
  }
  dp = (igl_device_plane *)calloc(1, sizeof(*dp));
  if (!dp) return IGL_FAIL_MEMORY;
  if (hipMalloc(&codes, code_bytes) != hipSuccess ||
      (gain_bytes && hipMalloc(&gains, gain_bytes) != hipSuccess)) {
    if (codes) (void)hipFree(codes);
    free(dp);
    return IGL_FAIL_MEMORY;
  }
  if (hipMemcpy(codes, code_src, code_bytes, hipMemcpyHostToDevice) != hipSuccess ||
      (gain_bytes && hipMemcpy(gains, gain_src, gain_bytes, hipMemcpyHostToDevice) != hipSuccess)) {
    (void)hipFree(codes);
    (void)hipFree(gains);
    free(dp);
    return IGL_FAIL_DEVICE;
  }
  dp->codes = codes;
  dp->gains = (const float *)gains;
  dp->owned = 1;
  if ((code = attach_zeros(sheet, dp)) != IGL_OKAY || (code = plane_reserve(st, sheet)) != IGL_OKAY) {
    free_zeros(dp);
    (void)hipFree(codes);
    (void)hipFree(gains);
    free(dp);
    return code;
  }
  sheet->device = dp;
  return IGL_OKAY;
}

int igl_plane_bind_dev(igl_desk *desk, igl_plane *sheet, const void *code_dev, const float *gain_dev) {
  igl_desk_state *st = desk ? desk->state : NULL;
  igl_device_plane *dp;
  int code;
  if (!st) return IGL_FAIL_STATE;
  if ((code = plane_supported(sheet)) != IGL_OKAY) return code;
  if (!code_dev || ((uintptr_t)code_dev & 15u) ||
      (sheet->form == IGL_PLANE_CODE && (!gain_dev || ((uintptr_t)gain_dev & 3u))))
    return IGL_FAIL_ARGUMENT;
  dp = (igl_device_plane *)calloc(1, sizeof(*dp));
  if (!dp) return IGL_FAIL_MEMORY;
  dp->codes = code_dev;
  dp->gains = gain_dev;
  dp->owned = 0;
  if ((code = attach_zeros(sheet, dp)) != IGL_OKAY || (code = plane_reserve(st, sheet)) != IGL_OKAY) {
    free_zeros(dp);
    free(dp);
    return code;
  }
  sheet->device = dp;
  return IGL_OKAY;
}

void igl_plane_detach(igl_desk *desk, igl_plane *sheet) {
  igl_device_plane *dp;
  (void)desk;
  if (!sheet || !sheet->device) return;
  dp = sheet->device;
  if (dp->owned) {
    (void)hipFree((void *)dp->codes);
    (void)hipFree((void *)dp->gains);
  }
  free_zeros(dp);
  free(dp);
  sheet->device = NULL;
}

/* ---- device-resident projection ------------------------------------------ */

static int check_lanes(const igl_plane *sheet, const void *act, int act_stride, int lanes,
                       const void *out, int out_stride) {
  if (!act || !out || lanes < 1) return IGL_FAIL_ARGUMENT;
  if (lanes > 1 && (act_stride < sheet->col_count || out_stride < sheet->row_count))
    return IGL_FAIL_ARGUMENT;
  return IGL_OKAY;
}

int igl_gemv_dev(igl_desk *desk, const igl_plane *sheet, const float *act_dev, int act_stride,
                 int lane_count, float *out_dev, int out_stride) {
  igl_desk_state *st = desk ? desk->state : NULL;
  const igl_device_plane *dp;
  int code, done;
  if (!st) return IGL_FAIL_STATE;
  if ((code = plane_supported(sheet)) != IGL_OKAY || !sheet->device) {
    code = code != IGL_OKAY ? code : IGL_FAIL_STATE;
    desk_fail(st, code);
    return code;
  }
  if ((code = check_lanes(sheet, act_dev, act_stride, lane_count, out_dev, out_stride)) != IGL_OKAY) {
    desk_fail(st, code);
    return code;
  }
  if (plane_part_floats(st, sheet) > st->part_floats) {
    desk_fail(st, IGL_FAIL_STATE);
    return IGL_FAIL_STATE;
  }
  dp = sheet->device;
  if (dp->zeros) {
    igl_code_view view = igl_plane_view(sheet, dp->codes, dp->gains);
    if (((uintptr_t)act_dev & 15u) || (lane_count > 1 && (act_stride & 3))) {
      desk_fail(st, IGL_FAIL_ARGUMENT);
      return IGL_FAIL_ARGUMENT;
    }
    return hip_check(st, igl_launch_gemv_zero(&view, dp->zeros, act_dev, act_stride, lane_count, out_dev,
                                              out_stride, sheet->row_count, sheet->col_count, st->stream));
  }
  if (sheet->form == IGL_PLANE_REAL) {
    if (((uintptr_t)act_dev & 15u) || (lane_count > 1 && (act_stride & 3))) {
      desk_fail(st, IGL_FAIL_ARGUMENT);
      return IGL_FAIL_ARGUMENT;
    }
    return hip_check(st, igl_launch_gemv_real(dp->codes, sheet->real_type, act_dev, act_stride,
                                              lane_count, out_dev, out_stride, sheet->row_count,
                                              sheet->col_count, st->part_dev, st->stream));
  }
  if (!plane_is_q4(sheet)) {
    igl_code_view view = igl_plane_view(sheet, dp->codes, dp->gains);
    if (((uintptr_t)act_dev & 15u) || (lane_count > 1 && (act_stride & 3))) {
      desk_fail(st, IGL_FAIL_ARGUMENT);
      return IGL_FAIL_ARGUMENT;
    }
    return hip_check(st, igl_launch_gemv_codes(&view, act_dev, act_stride, lane_count, out_dev,
                                               out_stride, sheet->row_count, sheet->col_count,
                                               st->part_dev, st->stream));
  }
  for (done = 0; done < lane_count; done += IGL_GEMV_Q4_LANES) {
    int lanes = lane_count - done < IGL_GEMV_Q4_LANES ? lane_count - done : IGL_GEMV_Q4_LANES;
    hipError_t e = igl_launch_gemv_q4(
        (const uint8_t *)dp->codes, (long long)sheet->row_stride, dp->gains, sheet->group_count,
        igl_plane_group_shift(sheet), sheet->code_bias, act_dev + (size_t)done * (size_t)act_stride,
        act_stride, lanes, out_dev + (size_t)done * (size_t)out_stride, out_stride,
        sheet->row_count, sheet->col_count, st->part_dev, st->lds_limit, st->stream);
    if ((code = hip_check(st, e)) != IGL_OKAY) return code;
  }
  return IGL_OKAY;
}

static int gemm_run(igl_desk *desk, const igl_plane *sheet, const void *act_dev, int act_bf16,
                    int act_stride, int lane_count, void *out_dev, int out_bf16, int out_stride) {
  igl_desk_state *st = desk->state;
  const igl_device_plane *dp = sheet->device;
  const int align = act_bf16 ? 8 : 4;
  /* bf16 activations are one exact binary16 term; fp32 ones two (hi + lo) */
  const int terms = act_bf16 ? 1 : 2;
  int code;
  if ((code = check_lanes(sheet, act_dev, act_stride, lane_count, out_dev, out_stride)) != IGL_OKAY ||
      ((uintptr_t)act_dev & 15u) || (act_stride % align) ||
      (lane_count == 1 && act_stride % align)) {
    code = code != IGL_OKAY ? code : IGL_FAIL_ARGUMENT;
    desk_fail(st, code);
    return code;
  }
  {
    size_t bytes = igl_gemm_work_bytes(lane_count, sheet->row_count, sheet->col_count, terms);
    if (bytes && grow_dev(st, &st->gemm_dev, &st->gemm_floats, (bytes + 3) / 4) != IGL_OKAY)
      return IGL_FAIL_MEMORY;
  }
  return hip_check(st, igl_launch_gemm_q4(act_dev, act_bf16, act_stride, (const uint8_t *)dp->codes,
                                          (long long)sheet->row_stride, dp->gains,
                                          sheet->group_count, igl_plane_group_shift(sheet),
                                          sheet->code_bias, dp->zero_pairs,
                                          out_dev, out_bf16, out_stride, lane_count,
                                          sheet->row_count, sheet->col_count, terms, st->gemm_dev,
                                          NULL, st->stream));
}

int igl_gemm_lane_floor(void) { return IGL_GEMM_FLOOR; }

unsigned igl_desk_generation(igl_desk *desk) {
  const igl_desk_state *st = desk ? desk->state : NULL;
  return st ? st->generation : 0u;
}

int igl_mat_mat_dev(igl_desk *desk, const igl_plane *sheet, const float *act_dev, int act_stride,
                    int lane_count, float *out_dev, int out_stride) {
  igl_desk_state *st = desk ? desk->state : NULL;
  int code;
  if (!st) return IGL_FAIL_STATE;
  if (lane_count < IGL_GEMM_FLOOR || (sheet && !plane_is_q4(sheet)) ||
      (sheet && !igl_gemm_fits(lane_count, sheet->row_count, sheet->col_count)) ||
      (sheet && sheet->device && sheet->device->zeros && !sheet->device->zero_pairs))
    return igl_gemv_dev(desk, sheet, act_dev, act_stride, lane_count, out_dev, out_stride);
  if ((code = plane_supported(sheet)) != IGL_OKAY || !sheet->device) {
    code = code != IGL_OKAY ? code : IGL_FAIL_STATE;
    desk_fail(st, code);
    return code;
  }
  return gemm_run(desk, sheet, act_dev, 0, act_stride, lane_count, out_dev, 0, out_stride);
}

int igl_gemm_bf16_dev(igl_desk *desk, const igl_plane *sheet, const uint16_t *act_dev,
                      int act_stride, int lane_count, uint16_t *out_dev, int out_stride) {
  igl_desk_state *st = desk ? desk->state : NULL;
  int code;
  if (!st) return IGL_FAIL_STATE;
  if ((code = plane_supported(sheet)) != IGL_OKAY || !sheet->device) {
    code = code != IGL_OKAY ? code : IGL_FAIL_STATE;
    desk_fail(st, code);
    return code;
  }
  if (!plane_is_q4(sheet) || !igl_gemm_fits(lane_count, sheet->row_count, sheet->col_count) ||
      (sheet->device->zeros && !sheet->device->zero_pairs)) {
    desk_fail(st, IGL_FAIL_SUPPORT);
    return IGL_FAIL_SUPPORT;
  }
  return gemm_run(desk, sheet, act_dev, 1, act_stride, lane_count, out_dev, 1, out_stride);
}

/* ---- the static activation grid around a product --------------------------- */

int igl_quant_step_dev(igl_desk *desk, const float *src_dev, int src_stride, float *dst_dev,
                       int dst_stride, int n, int lanes, float step) {
  igl_desk_state *st = desk ? desk->state : NULL;
  if (!st) return IGL_FAIL_STATE;
  if (!src_dev || !dst_dev || n < 1 || lanes < 1 ||
      (lanes > 1 && (src_stride < n || dst_stride < n))) {
    desk_fail(st, IGL_FAIL_ARGUMENT);
    return IGL_FAIL_ARGUMENT;
  }
  return hip_check(st, igl_launch_quant_step(src_dev, src_stride, dst_dev, dst_stride, n, lanes,
                                             step, st->stream));
}

/* plane_lift_many (app_core.c:7814-7843) without the model-wide input rule:
 * with enter_gain > 0 the lanes are put on that grid (in desk scratch) before
 * the product, and with leave_gain > 0 the outputs after it.  The product is
 * igl_mat_mat_dev's.  The table's mat_mat does neither: its caller does. */
/* The prefill of a calibrated plane with one gain a row on the activation
 * grid, closed as the reference's level path closes a row
 * (kern_row_code_level, app_core.c:3272-3296): on the int8 matrix cores where
 * the plane's width fits (igl_launch_gemm_level: exact int32 sums); otherwise
 * the lanes as levels, the codes as 4-bit planes of unit gain, the binary16
 * MFMA GEMM on those integer-valued operands (exact: every partial sum an
 * integer below 2^24), then gain * step * part and the leave grid. */
static int lift_levels_gemm(igl_desk_state *st, const igl_plane *sheet, const float *act_dev,
                            int act_stride, int lanes, float *out_dev, int out_stride) {
  const int N = sheet->row_count, K = sheet->col_count, bits = sheet->bit_count;
  if (igl_gemm_level_fits(bits, sheet->code_bias, K) && sheet->row_stride % 16 == 0) {
    /* the integer matrix cores: int8 levels against the codes as int8 */
    const igl_gemm_close close = {sheet->device->gains, sheet->enter_gain, sheet->leave_gain};
    const size_t need = igl_gemm_level_work_bytes(lanes, N, K, bits);
    if (grow_dev(st, &st->gemm_dev, &st->gemm_floats, (need + 3) / 4) != IGL_OKAY) return IGL_FAIL_MEMORY;
    return hip_check(st, igl_launch_gemm_level(act_dev, act_stride, (const uint8_t *)sheet->device->codes,
                                               (long long)sheet->row_stride, bits, sheet->code_flip,
                                               sheet->code_bias, &close, out_dev, out_stride, lanes, N, K,
                                               st->gemm_dev, st->stream));
  }
  const int two = bits == 8;
  const int widen = !(bits == 4 && sheet->code_flip == 0);
  const size_t plane_bytes = (size_t)N * (size_t)(K / 2);
  const uint8_t *hi_plane = (const uint8_t *)sheet->device->codes;
  const uint8_t *lo_plane = NULL;
  long long row_stride = (long long)sheet->row_stride;
  size_t work = igl_gemm_work_bytes(lanes, N, K, 1);
  float *a_out = two ? NULL : out_dev;
  int a_stride = two ? N : out_stride;
  int code;
  if ((two && grow_dev(st, &st->quant_dev, &st->quant_floats, (size_t)lanes * (size_t)K) != IGL_OKAY) ||
      (widen && grow_dev(st, &st->wide_dev, &st->wide_floats, (two ? 2 : 1) * plane_bytes / 4) != IGL_OKAY) ||
      (two && grow_dev(st, &st->lsum_dev, &st->lsum_floats, (size_t)lanes) != IGL_OKAY) ||
      (two && grow_dev(st, &st->prod_dev, &st->prod_floats, 2 * (size_t)lanes * (size_t)N) != IGL_OKAY) ||
      (work && grow_dev(st, &st->gemm_dev, &st->gemm_floats, (work + 3) / 4) != IGL_OKAY))
    return IGL_FAIL_MEMORY;
  if (st->ones_floats < (size_t)N) {
    if (grow_dev(st, &st->ones_dev, &st->ones_floats, (size_t)N) != IGL_OKAY) return IGL_FAIL_MEMORY;
    if ((code = hip_check(st, igl_launch_fill(st->ones_dev, st->ones_floats, 1.0f, st->stream))) != IGL_OKAY)
      return code;
  }
  if (two) a_out = st->prod_dev;
  if (widen) {
    hi_plane = (const uint8_t *)st->wide_dev;
    lo_plane = two ? hi_plane + plane_bytes : NULL;
    row_stride = K / 2;
    if ((code = hip_check(st, igl_launch_code_widen((const uint8_t *)sheet->device->codes,
                                                    (long long)sheet->row_stride, N, K, bits,
                                                    sheet->code_flip, sheet->code_bias,
                                                    (uint8_t *)hi_plane, (uint8_t *)lo_plane,
                                                    st->stream))) != IGL_OKAY)
      return code;
  }
  if (!two) {
    /* the GEMM takes the levels and the row close in its own conversion and
     * store */
    const igl_gemm_close close = {sheet->device->gains, sheet->enter_gain, sheet->leave_gain};
    return hip_check(st, igl_launch_gemm_q4(act_dev, 0, act_stride, hi_plane, row_stride, st->ones_dev, 1, 31,
                                            8, NULL, out_dev, 0, out_stride, lanes, N, K, 1, st->gemm_dev,
                                            &close, st->stream));
  }
  if ((code = hip_check(st, igl_launch_quant_level(act_dev, act_stride, st->quant_dev, K, K, lanes,
                                                   sheet->enter_gain, two ? st->lsum_dev : NULL,
                                                   st->stream))) != IGL_OKAY)
    return code;
  if ((code = hip_check(st, igl_launch_gemm_q4(st->quant_dev, 0, K, hi_plane, row_stride, st->ones_dev, 1, 31,
                                               8, NULL, a_out, 0, a_stride, lanes, N, K, 1, st->gemm_dev,
                                               NULL, st->stream))) != IGL_OKAY)
    return code;
  if (two &&
      (code = hip_check(st, igl_launch_gemm_q4(st->quant_dev, 0, K, lo_plane, row_stride, st->ones_dev, 1, 31,
                                               8, NULL, st->prod_dev + (size_t)lanes * (size_t)N, 0, N, lanes,
                                               N, K, 1, st->gemm_dev, NULL, st->stream))) != IGL_OKAY)
    return code;
  return hip_check(st, igl_launch_grid_close(a_out, two ? st->prod_dev + (size_t)lanes * (size_t)N : NULL,
                                             two ? st->lsum_dev : NULL, a_stride,
                                             sheet->device->gains, sheet->enter_gain, sheet->leave_gain, N,
                                             lanes, out_dev, out_stride, st->stream));
}

int igl_plane_lift_dev(igl_desk *desk, const igl_plane *sheet, const float *act_dev,
                       int act_stride, int lane_count, float *out_dev, int out_stride) {
  igl_desk_state *st = desk ? desk->state : NULL;
  int code;
  if (!st) return IGL_FAIL_STATE;
  if (!sheet || !act_dev || !out_dev || lane_count < 1 ||
      (lane_count > 1 && (act_stride < sheet->col_count || out_stride < sheet->row_count))) {
    desk_fail(st, IGL_FAIL_ARGUMENT);
    return IGL_FAIL_ARGUMENT;
  }
  /* A calibrated code plane below the GEMM's lane floor: one launch on the
   * activation grid, entry and leave grids fused, the reference's level path
   * (exact integer sums) rather than the float path on quant_step values. */
  if (sheet->enter_gain > 0.0f && sheet->form == IGL_PLANE_CODE && lane_count < IGL_GEMM_FLOOR &&
      plane_supported(sheet) == IGL_OKAY && sheet->device && !sheet->device->zeros &&
      igl_gemv_level_fits(sheet->bit_count, sheet->col_count) && ((uintptr_t)act_dev & 15u) == 0 &&
      (lane_count == 1 || (act_stride & 3) == 0)) {
    igl_code_view view = igl_plane_view(sheet, sheet->device->codes, sheet->device->gains);
    return hip_check(st, igl_launch_gemv_level(&view, sheet->enter_gain, sheet->leave_gain, act_dev,
                                               act_stride, lane_count, out_dev, out_stride,
                                               sheet->row_count, sheet->col_count, st->stream));
  }
  if (sheet->enter_gain > 0.0f && sheet->form == IGL_PLANE_CODE && lane_count >= IGL_GEMM_FLOOR &&
      plane_supported(sheet) == IGL_OKAY && sheet->device && !sheet->device->zeros && sheet->group_count == 1 &&
      (igl_gemm_level_fits(sheet->bit_count, sheet->code_bias, sheet->col_count) ||
       igl_gemm_fits(lane_count, sheet->row_count, sheet->col_count)) &&
      ((uintptr_t)act_dev & 15u) == 0 && (act_stride & 3) == 0)
    return lift_levels_gemm(st, sheet, act_dev, act_stride, lane_count, out_dev, out_stride);
  if (sheet->enter_gain > 0.0f) {
    const int cols = sheet->col_count;
    if (grow_dev(st, &st->quant_dev, &st->quant_floats, (size_t)lane_count * (size_t)cols) != IGL_OKAY)
      return IGL_FAIL_MEMORY;
    if ((code = hip_check(st, igl_launch_quant_step(act_dev, act_stride, st->quant_dev, cols, cols,
                                                    lane_count, sheet->enter_gain, st->stream))) !=
        IGL_OKAY)
      return code;
    code = igl_mat_mat_dev(desk, sheet, st->quant_dev, cols, lane_count, out_dev, out_stride);
  } else {
    code = igl_mat_mat_dev(desk, sheet, act_dev, act_stride, lane_count, out_dev, out_stride);
  }
  if (code != IGL_OKAY || !(sheet->leave_gain > 0.0f)) return code;
  return hip_check(st, igl_launch_quant_step(out_dev, out_stride, out_dev, out_stride,
                                             sheet->row_count, lane_count, sheet->leave_gain,
                                             st->stream));
}

/* ---- attention and cache ------------------------------------------------- */

/* The checks both lane entries make before anything is launched. */
static int attend_check(igl_desk_state *st, const uint8_t *key_store, const uint8_t *value_store,
                        int format, int cache_span, int kv_count, int group_share, int head_size,
                        const float *query_dev, int lane_stride, int place_first, int window,
                        int lane_count, const float *blend_out_dev) {
  int widest = window > 0 && window < place_first + lane_count ? window : place_first + lane_count;
  if (!key_store || !value_store || !query_dev || !blend_out_dev || kv_count < 1 ||
      cache_span < 1 || lane_count < 1 || place_first < 0 || window < 0 || widest > cache_span ||
      (lane_count > 1 && lane_stride < kv_count * group_share * head_size) ||
      (format != IGL_CACHE_E4M3 && format != IGL_CACHE_INT8)) {
    desk_fail(st, IGL_FAIL_ARGUMENT);
    return IGL_FAIL_ARGUMENT;
  }
  if ((head_size != 256 && head_size != 512) || group_share != 8) {
    desk_fail(st, IGL_FAIL_SUPPORT);
    return IGL_FAIL_SUPPORT;
  }
  if (((uintptr_t)key_store & 15u) || ((uintptr_t)value_store & 15u)) {
    desk_fail(st, IGL_FAIL_ARGUMENT);
    return IGL_FAIL_ARGUMENT;
  }
  return IGL_OKAY;
}

int igl_attend_lanes_dev(igl_desk *desk, const uint8_t *key_store, const uint8_t *value_store,
                         int format, float key_scale, float value_scale, int cache_span,
                         int kv_count, int group_share, int head_size, const float *query_dev,
                         int lane_stride, int place_first, int window, int lane_count,
                         float score_scale, float *blend_out_dev) {
  igl_desk_state *st = desk ? desk->state : NULL;
  size_t need;
  int code;
  if (!st) return IGL_FAIL_STATE;
  if ((code = attend_check(st, key_store, value_store, format, cache_span, kv_count, group_share,
                           head_size, query_dev, lane_stride, place_first, window, lane_count,
                           blend_out_dev)) != IGL_OKAY)
    return code;
  need = igl_attend_work_floats(place_first, window, lane_count, kv_count * group_share, head_size);
  if (grow_dev(st, &st->work_dev, &st->work_floats, need) != IGL_OKAY) return IGL_FAIL_MEMORY;
  return hip_check(st, igl_launch_attend(key_store, value_store, format, key_scale, value_scale,
                                         cache_span, kv_count * head_size, kv_count, group_share,
                                         head_size, query_dev, lane_stride, place_first, NULL,
                                         window, lane_count, score_scale, blend_out_dev,
                                         st->work_dev, st->stream));
}

/* The same kernels with the partials in the fixed per-device array
 * (igl_attend.hip); nothing is allocated or freed. */
int igl_attend_lanes_fixed_dev(igl_desk *desk, const uint8_t *key_store,
                               const uint8_t *value_store, int format, float key_scale,
                               float value_scale, int cache_span, int kv_count, int group_share,
                               int head_size, const float *query_dev, int lane_stride,
                               int place_first, int window, int lane_count, float score_scale,
                               float *blend_out_dev) {
  igl_desk_state *st = desk ? desk->state : NULL;
  float *work;
  int code;
  if (!st) return IGL_FAIL_STATE;
  if ((code = attend_check(st, key_store, value_store, format, cache_span, kv_count, group_share,
                           head_size, query_dev, lane_stride, place_first, window, lane_count,
                           blend_out_dev)) != IGL_OKAY)
    return code;
  if (igl_attend_work_floats(place_first, window, lane_count, kv_count * group_share, head_size) >
      (size_t)IGL_ATTEND_FIXED_FLOATS) {
    desk_fail(st, IGL_FAIL_SUPPORT);
    return IGL_FAIL_SUPPORT;
  }
  if (!(work = igl_attend_fixed_ptr(st->device))) {
    desk_fail(st, IGL_FAIL_STATE);
    return IGL_FAIL_STATE;
  }
  return hip_check(st, igl_launch_attend(key_store, value_store, format, key_scale, value_scale,
                                         cache_span, kv_count * head_size, kv_count, group_share,
                                         head_size, query_dev, lane_stride, place_first, NULL,
                                         window, lane_count, score_scale, blend_out_dev, work,
                                         st->stream));
}

int igl_attend_dev(igl_desk *desk, const uint8_t *key_store, const uint8_t *value_store,
                   int format, float key_scale, float value_scale, int cache_span,
                   int kv_count, int group_share, int head_size, const float *query_dev,
                   int place_start, int span_count, float score_scale, float *blend_out_dev) {
  if (desk && desk->state && (span_count < 1 || place_start < 0)) {
    desk_fail(desk->state, IGL_FAIL_ARGUMENT);
    return IGL_FAIL_ARGUMENT;
  }
  /* One lane whose window is exactly its span: it sits at place_start + span - 1. */
  return igl_attend_lanes_dev(desk, key_store, value_store, format, key_scale, value_scale,
                              cache_span, kv_count, group_share, head_size, query_dev, 0,
                              place_start + span_count - 1, span_count, 1, score_scale,
                              blend_out_dev);
}

int igl_cache_lay_dev(igl_desk *desk, const float *row_dev, int width, float scale, int format,
                      uint8_t *store_dev, size_t slot_first) {
  igl_desk_state *st = desk ? desk->state : NULL;
  if (!st) return IGL_FAIL_STATE;
  if (!row_dev || !store_dev || width < 1 || !(scale > 0.0f) ||
      (format != IGL_CACHE_E4M3 && format != IGL_CACHE_INT8)) {
    desk_fail(st, IGL_FAIL_ARGUMENT);
    return IGL_FAIL_ARGUMENT;
  }
  return hip_check(st, igl_launch_cache_lay(row_dev, width, scale, format, store_dev, slot_first,
                                            st->stream));
}

int igl_norm_rms_dev(igl_desk *desk, const float *in_dev, const float *gain_dev, int n, int rows,
                     int stride, float eps, float *out_dev) {
  igl_desk_state *st = desk ? desk->state : NULL;
  if (!st) return IGL_FAIL_STATE;
  if (!in_dev || !out_dev || n < 1 || rows < 1 || (rows > 1 && stride < n)) {
    desk_fail(st, IGL_FAIL_ARGUMENT);
    return IGL_FAIL_ARGUMENT;
  }
  return hip_check(st, igl_launch_norm_rms(in_dev, gain_dev, n, rows, stride, eps, out_dev, st->stream));
}

int igl_soft_max_dev(igl_desk *desk, float *v_dev, int n, int rows, int stride) {
  igl_desk_state *st = desk ? desk->state : NULL;
  if (!st) return IGL_FAIL_STATE;
  if (!v_dev || n < 1 || rows < 1 || (rows > 1 && stride < n)) {
    desk_fail(st, IGL_FAIL_ARGUMENT);
    return IGL_FAIL_ARGUMENT;
  }
  return hip_check(st, igl_launch_soft_max(v_dev, n, rows, stride, st->stream));
}

int igl_read_floor_dev(igl_desk *desk, const void *src_dev, size_t bytes) {
  igl_desk_state *st = desk ? desk->state : NULL;
  if (!st) return IGL_FAIL_STATE;
  if (!src_dev || bytes < 16 || bytes % 16 || ((uintptr_t)src_dev & 15u) || !st->act_dev) {
    desk_fail(st, IGL_FAIL_ARGUMENT);
    return IGL_FAIL_ARGUMENT;
  }
  /* the sink: a word of the table's activation staging, scratch between calls */
  return hip_check(st, igl_launch_read_floor(src_dev, bytes, (uint32_t *)st->act_dev, st->stream));
}

int igl_gelu_gate_dev(igl_desk *desk, float *gate_dev, const float *rise_dev, int n) {
  igl_desk_state *st = desk ? desk->state : NULL;
  if (!st) return IGL_FAIL_STATE;
  if (!gate_dev || !rise_dev || n < 1) {
    desk_fail(st, IGL_FAIL_ARGUMENT);
    return IGL_FAIL_ARGUMENT;
  }
  return hip_check(st, igl_launch_gelu_gate(gate_dev, rise_dev, n, st->stream));
}

int igl_rope_turn_dev(igl_desk *desk, float *v_dev, int heads, int head_size, const float *cos_dev,
                      const float *sin_dev) {
  igl_desk_state *st = desk ? desk->state : NULL;
  if (!st) return IGL_FAIL_STATE;
  if (!v_dev || !cos_dev || !sin_dev || heads < 1 || head_size < 2 || (head_size & 1)) {
    desk_fail(st, IGL_FAIL_ARGUMENT);
    return IGL_FAIL_ARGUMENT;
  }
  return hip_check(st, igl_launch_rope_turn(v_dev, heads, head_size, cos_dev, sin_dev, st->stream));
}

/* ---- the table entries (host pointers, synchronous) ---------------------- */

static void table_mat_mat_body(igl_desk *desk, const igl_plane *sheet, const float *act_data,
                          int act_stride, int lane_count, float *out_data, int out_stride) {
  igl_desk_state *st = desk->state;
  int done = 0;
  if (refuse_recording(st)) return;
  if (!sheet || !sheet->device || !act_data || !out_data || lane_count < 1) {
    desk_fail(st, IGL_FAIL_ARGUMENT);
    return;
  }
  if (lane_count == 1) act_stride = sheet->col_count, out_stride = sheet->row_count;
  if (sheet->col_count > st->col_limit || (size_t)sheet->row_count * st->lane_limit > st->out_floats) {
    desk_fail(st, IGL_FAIL_STATE);
    return;
  }
  while (done < lane_count) {
    int lanes = lane_count - done < st->lane_limit ? lane_count - done : st->lane_limit;
    size_t K = (size_t)sheet->col_count, N = (size_t)sheet->row_count;
    if (hip_check(st, hipMemcpy2DAsync(st->act_dev, K * sizeof(float),
                                       act_data + (size_t)done * (size_t)act_stride,
                                       (size_t)act_stride * sizeof(float), K * sizeof(float),
                                       (size_t)lanes, hipMemcpyHostToDevice, st->stream)) != IGL_OKAY)
      return;
    if (igl_mat_mat_dev(desk, sheet, st->act_dev, (int)K, lanes, st->out_dev, (int)N) != IGL_OKAY)
      return;
    if (hip_check(st, hipMemcpy2DAsync(out_data + (size_t)done * (size_t)out_stride,
                                       (size_t)out_stride * sizeof(float), st->out_dev,
                                       N * sizeof(float), N * sizeof(float), (size_t)lanes,
                                       hipMemcpyDeviceToHost, st->stream)) != IGL_OKAY)
      return;
    if (hip_check(st, hipStreamSynchronize(st->stream)) != IGL_OKAY) return;
    done += lanes;
  }
}

/* The elementwise entries stage their vectors through the device. */
static float *elem_stage(igl_desk_state *st, size_t floats) {
  if (refuse_recording(st)) return NULL;
  if (grow_dev(st, &st->elem_dev, &st->elem_floats, floats) != IGL_OKAY) return NULL;
  return st->elem_dev;
}

static int elem_put(igl_desk_state *st, float *dst, const float *src, int n) {
  return hip_check(st, hipMemcpyAsync(dst, src, (size_t)n * sizeof(float), hipMemcpyHostToDevice,
                                      st->stream));
}

static void elem_get(igl_desk_state *st, float *dst, const float *src, int n) {
  if (hip_check(st, hipMemcpyAsync(dst, src, (size_t)n * sizeof(float), hipMemcpyDeviceToHost,
                                   st->stream)) == IGL_OKAY)
    (void)hip_check(st, hipStreamSynchronize(st->stream));
}

static void table_norm_rms_body(igl_desk *desk, const float *value_list, const float *gain_list,
                           int value_count, float eps_value, float *value_out) {
  igl_desk_state *st = desk->state;
  float *room = elem_stage(st, 3 * (size_t)value_count);
  if (!room || value_count < 1) {
    desk_fail(st, IGL_FAIL_ARGUMENT);
    return;
  }
  if (elem_put(st, room, value_list, value_count) != IGL_OKAY) return;
  if (gain_list && elem_put(st, room + value_count, gain_list, value_count) != IGL_OKAY) return;
  if (igl_norm_rms_dev(desk, room, gain_list ? room + value_count : NULL, value_count, 1,
                       value_count, eps_value, room + 2 * (size_t)value_count) != IGL_OKAY)
    return;
  elem_get(st, value_out, room + 2 * (size_t)value_count, value_count);
}

static void table_soft_max_body(igl_desk *desk, float *value_list, int value_count) {
  igl_desk_state *st = desk->state;
  float *room = elem_stage(st, (size_t)value_count);
  if (!room || value_count < 1) {
    desk_fail(st, IGL_FAIL_ARGUMENT);
    return;
  }
  if (elem_put(st, room, value_list, value_count) != IGL_OKAY) return;
  if (igl_soft_max_dev(desk, room, value_count, 1, value_count) != IGL_OKAY) return;
  elem_get(st, value_list, room, value_count);
}

static void table_gelu_gate_body(igl_desk *desk, float *gate_list, const float *rise_list,
                            int value_count) {
  igl_desk_state *st = desk->state;
  float *room = elem_stage(st, 2 * (size_t)value_count);
  if (!room || value_count < 1) {
    desk_fail(st, IGL_FAIL_ARGUMENT);
    return;
  }
  if (elem_put(st, room, gate_list, value_count) != IGL_OKAY) return;
  if (elem_put(st, room + value_count, rise_list, value_count) != IGL_OKAY) return;
  if (igl_gelu_gate_dev(desk, room, room + value_count, value_count) != IGL_OKAY) return;
  elem_get(st, gate_list, room, value_count);
}

static void table_rope_turn_body(igl_desk *desk, float *value_list, int head_size, const float *cos_list,
                            const float *sin_list) {
  igl_desk_state *st = desk->state;
  int half = head_size / 2;
  float *room = elem_stage(st, 2 * (size_t)head_size);
  if (!room || head_size < 2) {
    desk_fail(st, IGL_FAIL_ARGUMENT);
    return;
  }
  if (elem_put(st, room, value_list, head_size) != IGL_OKAY) return;
  if (elem_put(st, room + head_size, cos_list, half) != IGL_OKAY) return;
  if (elem_put(st, room + head_size + half, sin_list, half) != IGL_OKAY) return;
  if (igl_rope_turn_dev(desk, room, 1, head_size, room + head_size, room + head_size + half) != IGL_OKAY)
    return;
  elem_get(st, value_list, room, head_size);
}

/* The entries the table holds: each body under the desk's lock. */
static void table_mat_mat(igl_desk *desk, const igl_plane *sheet, const float *act_data,
                          int act_stride, int lane_count, float *out_data, int out_stride) {
  pthread_mutex_lock(&desk->state->table_lock);
  table_mat_mat_body(desk, sheet, act_data, act_stride, lane_count, out_data, out_stride);
  pthread_mutex_unlock(&desk->state->table_lock);
}

static void table_mat_vec(igl_desk *desk, const igl_plane *sheet, const float *act_data,
                          float *out_data) {
  table_mat_mat(desk, sheet, act_data, 0, 1, out_data, 0);
}

static void table_norm_rms(igl_desk *desk, const float *value_list, const float *gain_list,
                           int value_count, float eps_value, float *value_out) {
  pthread_mutex_lock(&desk->state->table_lock);
  table_norm_rms_body(desk, value_list, gain_list, value_count, eps_value, value_out);
  pthread_mutex_unlock(&desk->state->table_lock);
}

static void table_soft_max(igl_desk *desk, float *value_list, int value_count) {
  pthread_mutex_lock(&desk->state->table_lock);
  table_soft_max_body(desk, value_list, value_count);
  pthread_mutex_unlock(&desk->state->table_lock);
}

static void table_gelu_gate(igl_desk *desk, float *gate_list, const float *rise_list,
                            int value_count) {
  pthread_mutex_lock(&desk->state->table_lock);
  table_gelu_gate_body(desk, gate_list, rise_list, value_count);
  pthread_mutex_unlock(&desk->state->table_lock);
}

static void table_rope_turn(igl_desk *desk, float *value_list, int head_size, const float *cos_list,
                            const float *sin_list) {
  pthread_mutex_lock(&desk->state->table_lock);
  table_rope_turn_body(desk, value_list, head_size, cos_list, sin_list);
  pthread_mutex_unlock(&desk->state->table_lock);
}

/* ---- open / close --------------------------------------------------------- */

int igl_back_open(igl_desk *desk, int device_index, int sum_limit, int col_limit, int lane_limit) {
  igl_desk_state *st;
  int count = 0;
  if (!desk) return IGL_FAIL_ARGUMENT;
  memset(desk, 0, sizeof(*desk));
  if (hipGetDeviceCount(&count) != hipSuccess || count < 1) return IGL_FAIL_DEVICE;
  if (device_index < 0 || device_index >= count) return IGL_FAIL_ARGUMENT;
  if (hipSetDevice(device_index) != hipSuccess) return IGL_FAIL_DEVICE;
  /* the fixed attention workspace's address on this device, once */
  if (igl_attend_fixed_resolve(device_index) != hipSuccess) return IGL_FAIL_DEVICE;
  st = (igl_desk_state *)calloc(1, sizeof(*st));
  if (!st) return IGL_FAIL_MEMORY;
  st->device = device_index;
  if (pthread_mutex_init(&st->table_lock, NULL) != 0) {
    free(st);
    return IGL_FAIL_MEMORY;
  }
  st->table_lock_live = 1;
  st->lane_limit = lane_limit > 0 ? lane_limit : 16;
  st->col_limit = col_limit > 0 ? col_limit : 1;
  st->sum_limit = sum_limit > 0 ? sum_limit : 1;
  if (hipDeviceGetAttribute(&st->lds_limit, hipDeviceAttributeMaxSharedMemoryPerBlock,
                            device_index) != hipSuccess || st->lds_limit < 16384)
    st->lds_limit = 65536;
  if (hipStreamCreateWithFlags(&st->stream, hipStreamNonBlocking) != hipSuccess ||
      hipEventCreate(&st->mark[0]) != hipSuccess || hipEventCreate(&st->mark[1]) != hipSuccess ||
      hipMalloc((void **)&st->act_dev, (size_t)st->lane_limit * st->col_limit * sizeof(float)) != hipSuccess ||
      hipHostMalloc((void **)&st->act_pin, (size_t)st->lane_limit * st->col_limit * sizeof(float),
                    hipHostMallocDefault) != hipSuccess) {
    desk->state = st;
    igl_back_close(desk);
    return IGL_FAIL_DEVICE;
  }
  desk->state = st;
  desk->name_text = "hip/gfx950";
  desk->mat_vec = table_mat_vec;
  desk->mat_mat = table_mat_mat;
  desk->norm_rms = table_norm_rms;
  desk->soft_max = table_soft_max;
  desk->gelu_gate = table_gelu_gate;
  desk->rope_turn = table_rope_turn;
  return IGL_OKAY;
}

void igl_back_close(igl_desk *desk) {
  igl_desk_state *st;
  if (!desk || !desk->state) return;
  st = desk->state;
  if (st->stream) (void)hipStreamSynchronize(st->stream);
  if (st->act_dev) (void)hipFree(st->act_dev);
  if (st->act_pin) (void)hipHostFree(st->act_pin);
  if (st->out_dev) (void)hipFree(st->out_dev);
  if (st->out_pin) (void)hipHostFree(st->out_pin);
  if (st->part_dev) (void)hipFree(st->part_dev);
  if (st->work_dev) (void)hipFree(st->work_dev);
  if (st->quant_dev) (void)hipFree(st->quant_dev);
  if (st->wide_dev) (void)hipFree(st->wide_dev);
  if (st->ones_dev) (void)hipFree(st->ones_dev);
  if (st->lsum_dev) (void)hipFree(st->lsum_dev);
  if (st->prod_dev) (void)hipFree(st->prod_dev);
  if (st->elem_dev) (void)hipFree(st->elem_dev);
  if (st->gemm_dev) (void)hipFree(st->gemm_dev);
  if (st->mark[0]) (void)hipEventDestroy(st->mark[0]);
  if (st->mark[1]) (void)hipEventDestroy(st->mark[1]);
  if (st->stream) (void)hipStreamDestroy(st->stream);
  if (st->table_lock_live) pthread_mutex_destroy(&st->table_lock);
  free(st);
  memset(desk, 0, sizeof(*desk));
}

/* ---- plumbing ------------------------------------------------------------ */

void *igl_dev_alloc(igl_desk *desk, size_t bytes) {
  void *p = NULL;
  (void)desk;
  if (hipMalloc(&p, bytes ? bytes : 1) != hipSuccess) return NULL;
  return p;
}

void igl_dev_free(igl_desk *desk, void *ptr) {
  (void)desk;
  if (ptr) (void)hipFree(ptr);
}

int igl_copy_to_dev(igl_desk *desk, void *dst_dev, const void *src_host, size_t bytes) {
  igl_desk_state *st = desk ? desk->state : NULL;
  if (!st) return IGL_FAIL_STATE;
  if (refuse_recording(st)) return IGL_FAIL_STATE;
  if (hip_check(st, hipMemcpyAsync(dst_dev, src_host, bytes, hipMemcpyHostToDevice, st->stream)) != IGL_OKAY)
    return IGL_FAIL_DEVICE;
  return hip_check(st, hipStreamSynchronize(st->stream));
}

int igl_copy_to_host(igl_desk *desk, void *dst_host, const void *src_dev, size_t bytes) {
  igl_desk_state *st = desk ? desk->state : NULL;
  if (!st) return IGL_FAIL_STATE;
  if (refuse_recording(st)) return IGL_FAIL_STATE;
  if (hip_check(st, hipMemcpyAsync(dst_host, src_dev, bytes, hipMemcpyDeviceToHost, st->stream)) != IGL_OKAY)
    return IGL_FAIL_DEVICE;
  return hip_check(st, hipStreamSynchronize(st->stream));
}

int igl_fill_dev(igl_desk *desk, void *dst_dev, int byte_value, size_t bytes) {
  igl_desk_state *st = desk ? desk->state : NULL;
  if (!st) return IGL_FAIL_STATE;
  /* a memset node is not recorded: replays after the first have gone wrong */
  if (refuse_recording(st)) return IGL_FAIL_STATE;
  return hip_check(st, hipMemsetAsync(dst_dev, byte_value, bytes, st->stream));
}

int igl_sync(igl_desk *desk) {
  igl_desk_state *st = desk ? desk->state : NULL;
  if (!st) return IGL_FAIL_STATE;
  if (refuse_recording(st)) return IGL_FAIL_STATE;
  return hip_check(st, hipStreamSynchronize(st->stream));
}

int igl_mark(igl_desk *desk) {
  igl_desk_state *st = desk ? desk->state : NULL;
  if (!st) return IGL_FAIL_STATE;
  if (refuse_recording(st)) return IGL_FAIL_STATE;
  st->mark_turn ^= 1;
  st->marks_made += 1;
  return hip_check(st, hipEventRecord(st->mark[st->mark_turn], st->stream));
}

float igl_marks_ms(igl_desk *desk) {
  igl_desk_state *st = desk ? desk->state : NULL;
  float ms = -1.0f;
  if (!st || st->marks_made < 2 || refuse_recording(st)) return -1.0f;
  if (hip_check(st, hipEventSynchronize(st->mark[st->mark_turn])) != IGL_OKAY) return -1.0f;
  if (hip_check(st, hipEventElapsedTime(&ms, st->mark[st->mark_turn ^ 1], st->mark[st->mark_turn])) != IGL_OKAY)
    return -1.0f;
  return ms;
}

/* ---- recording and replay (HIP graphs) ----------------------------------- */

int igl_record_begin(igl_desk *desk) {
  igl_desk_state *st = desk ? desk->state : NULL;
  if (!st) return IGL_FAIL_STATE;
  if (st->recording) {
    desk_fail(st, IGL_FAIL_STATE);
    return IGL_FAIL_STATE;
  }
  if (hip_check(st, hipStreamBeginCapture(st->stream, hipStreamCaptureModeThreadLocal)) != IGL_OKAY)
    return IGL_FAIL_DEVICE;
  st->recording = 1;
  st->record_error = IGL_OKAY;
  return IGL_OKAY;
}

int igl_record_end(igl_desk *desk, igl_replay **replay_out) {
  igl_desk_state *st = desk ? desk->state : NULL;
  hipGraph_t graph = NULL;
  hipGraphExec_t exec = NULL;
  igl_replay *replay;
  hipError_t e;
  int code;
  if (replay_out) *replay_out = NULL;
  if (!st) return IGL_FAIL_STATE;
  if (!st->recording) {
    desk_fail(st, IGL_FAIL_STATE);
    return IGL_FAIL_STATE;
  }
  st->recording = 0;
  e = hipStreamEndCapture(st->stream, &graph);
  /* an entry refused or failed while recording: no replay, the code returned */
  code = st->record_error != IGL_OKAY ? st->record_error : st->error;
  st->record_error = IGL_OKAY;
  st->error = IGL_OKAY;
  if (code == IGL_OKAY && e != hipSuccess) code = IGL_FAIL_DEVICE;
  if (code == IGL_OKAY && !replay_out) code = IGL_FAIL_ARGUMENT;
  if (code == IGL_OKAY && hipGraphInstantiate(&exec, graph, NULL, NULL, 0) != hipSuccess)
    code = IGL_FAIL_DEVICE;
  if (graph) (void)hipGraphDestroy(graph);
  if (code != IGL_OKAY) {
    if (exec) (void)hipGraphExecDestroy(exec);
    return code;
  }
  replay = (igl_replay *)malloc(sizeof(*replay));
  if (!replay) {
    (void)hipGraphExecDestroy(exec);
    return IGL_FAIL_MEMORY;
  }
  replay->exec = exec;
  replay->owner = st;
  st->replays_live += 1;
  *replay_out = replay;
  return IGL_OKAY;
}

int igl_replay_run(igl_desk *desk, igl_replay *replay) {
  igl_desk_state *st = desk ? desk->state : NULL;
  if (!st) return IGL_FAIL_STATE;
  if (!replay || replay->owner != st) {
    desk_fail(st, IGL_FAIL_ARGUMENT);
    return IGL_FAIL_ARGUMENT;
  }
  if (refuse_recording(st)) return IGL_FAIL_STATE;
  return hip_check(st, hipGraphLaunch(replay->exec, st->stream));
}

void igl_replay_free(igl_desk *desk, igl_replay *replay) {
  (void)desk;
  if (!replay) return;
  /* the replay's own desk (open until its replays are freed) */
  (void)hipStreamSynchronize(replay->owner->stream);
  replay->owner->replays_live -= 1;
  (void)hipGraphExecDestroy(replay->exec);
  free(replay);
}
