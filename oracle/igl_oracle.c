/* igl_oracle.c - CPU restatement of igllm's plain-build float path.
 *
 * TEST INFRASTRUCTURE ONLY (see igl_oracle.h).  Compiled with
 * -std=c11 -ffp-contract=off so that every multiply and add rounds where the
 * reference's SSE2 tier rounds it: a plain build of app_core.c has no fused
 * multiply-add, and `-std=c11` keeps GCC from contracting.
 *
 * The summation orders below are those of the SSE2 tier, written as scalar C:
 * a "four-lane accumulator" is an array of four floats updated lane by lane,
 * and the horizontal sum is spelled out as the reference's shuffle sequence
 * computes it.
 */
#define _POSIX_C_SOURCE 200809L
#include "igl_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#define ORACLE_LANE_LIMIT  16   /* KERN_LANE_LIMIT, app_core.c:1980 */
#define ORACLE_SPREAD_LIMIT 256 /* KERN_SPREAD_LIMIT, app_core.c:1981 */

/* ------------------------------------------------------------------------ */
/* quant layer                                                              */
/* ------------------------------------------------------------------------ */

/* Element i of a dense little-endian stream of `bit_count`-bit fields: bits
 * [i*b, i*b+b) of the byte string read as one little-endian integer
 * (pack_read, app_core.c:1757-1769). */
uint32_t oracle_pack_read(const uint8_t *code_data, size_t element_index, int bit_count) {
  size_t first_bit = element_index * (size_t)bit_count;
  uint64_t gathered = 0;
  int have = 0;
  size_t byte_at = first_bit / 8u;
  int skip = (int)(first_bit % 8u);
  while (have < skip + bit_count) {
    gathered |= (uint64_t)code_data[byte_at++] << have;
    have += 8;
  }
  gathered >>= skip;
  if (bit_count >= 32) return (uint32_t)gathered;
  return (uint32_t)(gathered & ((1ull << bit_count) - 1ull));
}

/* One row as floats: ((code ^ flip) - code_bias - zero) * gain, group by group
 * (plane_row, app_core.c:1826-1856). */
void oracle_plane_row(const oracle_plane *sheet, int row_index, float *row_out) {
  const uint8_t *row_bytes = sheet->code_data + (size_t)row_index * sheet->row_stride;
  for (int g = 0; g < sheet->group_count; ++g) {
    size_t gain_at = (size_t)row_index * (size_t)sheet->group_count + (size_t)g;
    float gain = sheet->gain_data[gain_at];
    int zero = sheet->bias_data ? sheet->bias_data[gain_at] : 0;
    int lo = g * sheet->group_size;
    int hi = lo + sheet->group_size < sheet->col_count ? lo + sheet->group_size : sheet->col_count;
    for (int k = lo; k < hi; ++k) {
      int code = (int)(oracle_pack_read(row_bytes, (size_t)k, sheet->bit_count) ^
                       (uint32_t)sheet->code_flip);
      row_out[k] = (float)(code - sheet->code_bias - zero) * gain;
    }
  }
}

/* The static activation grid: rint(x/step) clamped to [-128, 127], times step
 * (quant_step, app_core.c:1930-1940).  A step of zero leaves x alone. */
float oracle_quant_step(float value, float step) {
  float level;
  if (!(step > 0.0f)) return value;
  level = rintf(value / step);
  if (level < -128.0f) level = -128.0f;
  if (level > 127.0f) level = 127.0f;
  return level * step;
}

/* ------------------------------------------------------------------------ */
/* projection                                                               */
/* ------------------------------------------------------------------------ */

/* The SSE2 horizontal sum of a four-lane accumulator (kern_wide_total /
 * kern_dot_total, app_core.c:1990-2003, 2157-2161): lanes 0+2 and 1+3 first. */
static float oracle_fold4(const float lane[4]) {
  float even = lane[0] + lane[2];
  float odd = lane[1] + lane[3];
  return even + odd;
}

/* Sequential walk of the bit stream, the reference's general fallback
 * (app_core.c:2762-2765). */
static float oracle_dot_walk(const uint8_t *code_row, int from_index, int slot, int span_count,
                             const float *act, int bit_count, int code_flip, float total) {
  for (; slot < span_count; ++slot)
    total += (float)(oracle_pack_read(code_row, (size_t)(from_index + slot), bit_count) ^
                     (uint32_t)code_flip) * act[slot];
  return total;
}

/* Activation times code over one group (kern_dot_code, app_core.c:2363-2766,
 * SSE2 tier).
 *
 * For 2, 4 and 8 bits on an aligned start the SSE2 tier walks blocks of
 * sixteen codes with two four-lane accumulators, codes 0-3 and 8-11 into the
 * first and 4-7 and 12-15 into the second (4-bit: 2412-2440; 8-bit: 2501-2524;
 * 2-bit: 2623-2640), folds them, and finishes the span one code at a time.
 * Three, five, six and seven bits on a start that is a multiple of eight
 * alternate two scalar sums over the same blocks (2735-2759).  Everything
 * else walks the stream. */
float oracle_dot_code(const uint8_t *code_row, int from_index, int span_count,
                      const float *act, int bit_count, int code_flip) {
  int slot = 0;
  int block_path = (bit_count == 4 && code_flip == 0 && (from_index & 1) == 0) ||
                   (bit_count == 2 && code_flip == 0 && (from_index & 3) == 0) ||
                   bit_count == 8;
  if (block_path) {
    float part_a[4] = {0.0f, 0.0f, 0.0f, 0.0f}, part_b[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float sum_lane[4];
    float code[16];
    for (; slot + 16 <= span_count; slot += 16) {
      for (int j = 0; j < 16; ++j)
        code[j] = (float)(oracle_pack_read(code_row, (size_t)(from_index + slot + j), bit_count) ^
                          (uint32_t)code_flip);
      for (int i = 0; i < 4; ++i) part_a[i] = part_a[i] + code[i] * act[slot + i];
      for (int i = 0; i < 4; ++i) part_b[i] = part_b[i] + code[4 + i] * act[slot + 4 + i];
      for (int i = 0; i < 4; ++i) part_a[i] = part_a[i] + code[8 + i] * act[slot + 8 + i];
      for (int i = 0; i < 4; ++i) part_b[i] = part_b[i] + code[12 + i] * act[slot + 12 + i];
    }
    for (int i = 0; i < 4; ++i) sum_lane[i] = part_a[i] + part_b[i];
    return oracle_dot_walk(code_row, from_index, slot, span_count, act, bit_count, code_flip,
                           oracle_fold4(sum_lane));
  }
  if ((bit_count == 3 || bit_count == 5 || bit_count == 6 || bit_count == 7) &&
      (from_index & 7) == 0) {
    float sum_a = 0.0f, sum_b = 0.0f;
    for (; slot + 16 <= span_count; slot += 16)
      for (int j = 0; j < 16; j += 2) {
        sum_a += (float)(oracle_pack_read(code_row, (size_t)(from_index + slot + j), bit_count) ^
                         (uint32_t)code_flip) * act[slot + j];
        sum_b += (float)(oracle_pack_read(code_row, (size_t)(from_index + slot + j + 1), bit_count) ^
                         (uint32_t)code_flip) * act[slot + j + 1];
      }
    return oracle_dot_walk(code_row, from_index, slot, span_count, act, bit_count, code_flip,
                           sum_a + sum_b);
  }
  return oracle_dot_walk(code_row, from_index, 0, span_count, act, bit_count, code_flip, 0.0f);
}

/* Per-group activation sums, in order (kern_group_sum, app_core.c:4288-4300). */
void oracle_group_sum(const oracle_plane *sheet, const float *act, float *sum_out) {
  for (int g = 0; g < sheet->group_count; ++g) {
    int lo = g * sheet->group_size;
    int span = sheet->col_count - lo < sheet->group_size ? sheet->col_count - lo : sheet->group_size;
    float total = 0.0f;
    for (int k = 0; k < span; ++k) total += act[lo + k];
    sum_out[g] = total;
  }
}

/* One lane, one row: sum over groups of gain * (dot - (bias + zero) * sum),
 * accumulated in group order (kern_row_code, app_core.c:3688-3706). */
float oracle_row_code(const oracle_plane *sheet, int row_index, const float *act,
                      const float *sum_data) {
  const uint8_t *row_bytes = sheet->code_data + (size_t)row_index * sheet->row_stride;
  size_t gain_base = (size_t)row_index * (size_t)sheet->group_count;
  float total = 0.0f;
  for (int g = 0; g < sheet->group_count; ++g) {
    int lo = g * sheet->group_size;
    int span = sheet->col_count - lo < sheet->group_size ? sheet->col_count - lo : sheet->group_size;
    float gain = sheet->gain_data[gain_base + (size_t)g];
    float bias = (float)(sheet->code_bias + (sheet->bias_data ? sheet->bias_data[gain_base + (size_t)g] : 0));
    float part = oracle_dot_code(row_bytes, lo, span, act + lo, sheet->bit_count, sheet->code_flip);
    total += gain * (part - bias * sum_data[g]);
  }
  return total;
}

/* kern_dot_real on fp32, SSE2 tier (app_core.c:2054-2066): blocks of eight
 * into two four-lane accumulators, then blocks of four into the first, fold,
 * then the rest one at a time. */
static float oracle_dot_real(const float *row, const float *act, int span_count) {
  float part_a[4] = {0.0f, 0.0f, 0.0f, 0.0f}, part_b[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  float sum_lane[4];
  float total;
  int slot = 0;
  for (; slot + 8 <= span_count; slot += 8) {
    for (int i = 0; i < 4; ++i) part_a[i] = part_a[i] + row[slot + i] * act[slot + i];
    for (int i = 0; i < 4; ++i) part_b[i] = part_b[i] + row[slot + 4 + i] * act[slot + 4 + i];
  }
  for (; slot + 4 <= span_count; slot += 4)
    for (int i = 0; i < 4; ++i) part_a[i] = part_a[i] + row[slot + i] * act[slot + i];
  for (int i = 0; i < 4; ++i) sum_lane[i] = part_a[i] + part_b[i];
  total = oracle_fold4(sum_lane);
  for (; slot < span_count; ++slot) total += row[slot] * act[slot];
  return total;
}

/* Several lanes, one row (kern_row_code_many, app_core.c:4075-4117, SSE2 tier):
 * each group's codes are spread to floats once (kern_code_spread, 3485) and
 * dotted against every lane (kern_dot_real_many, 3871).  On the SSE2 tier the
 * four-lane blocks of kern_dot_real_many carry exactly kern_dot_real's two
 * accumulators per lane, so every lane's part equals kern_dot_real on the
 * spread codes; the row's output is accumulated group by group in place. */
void oracle_row_code_many(const oracle_plane *sheet, int row_index, const float *act,
                          int act_stride, int lane_count, const float *sum_data, int sum_stride,
                          float *out, int out_stride) {
  const uint8_t *row_bytes = sheet->code_data + (size_t)row_index * sheet->row_stride;
  size_t gain_base = (size_t)row_index * (size_t)sheet->group_count;
  float part[ORACLE_LANE_LIMIT];
  float spread[ORACLE_SPREAD_LIMIT];
  for (int l = 0; l < lane_count; ++l) out[(size_t)l * (size_t)out_stride + (size_t)row_index] = 0.0f;
  for (int g = 0; g < sheet->group_count; ++g) {
    int lo = g * sheet->group_size;
    int span = sheet->col_count - lo < sheet->group_size ? sheet->col_count - lo : sheet->group_size;
    float gain = sheet->gain_data[gain_base + (size_t)g];
    float bias = (float)(sheet->code_bias + (sheet->bias_data ? sheet->bias_data[gain_base + (size_t)g] : 0));
    int done = 0;
    for (int l = 0; l < lane_count; ++l) part[l] = 0.0f;
    while (done < span) {
      int chunk = span - done < ORACLE_SPREAD_LIMIT ? span - done : ORACLE_SPREAD_LIMIT;
      for (int k = 0; k < chunk; ++k)
        spread[k] = (float)(oracle_pack_read(row_bytes, (size_t)(lo + done + k), sheet->bit_count) ^
                            (uint32_t)sheet->code_flip);
      for (int l = 0; l < lane_count; ++l)
        part[l] += oracle_dot_real(spread, act + (size_t)l * (size_t)act_stride + lo + done, chunk);
      done += chunk;
    }
    for (int l = 0; l < lane_count; ++l)
      out[(size_t)l * (size_t)out_stride + (size_t)row_index] +=
          gain * (part[l] - bias * sum_data[(size_t)l * (size_t)sum_stride + (size_t)g]);
  }
}

/* Even split of `total` rows into `slice_count` bands, the first `total %
 * slice_count` one row longer (slice_span, app_core.c:1036-1043). */
static void oracle_band(int total, int slice_index, int slice_count, int *from, int *upto) {
  int base = total / slice_count, extra = total % slice_count;
  *from = slice_index * base + (slice_index < extra ? slice_index : extra);
  *upto = *from + base + (slice_index < extra ? 1 : 0);
}

typedef struct oracle_job {
  const oracle_plane *sheet;
  const float *act;
  const float *sum;
  float *out;
  int act_stride, out_stride, lane_count;
  int slice_index, slice_count;
} oracle_job;

static void *oracle_band_run(void *state) {
  oracle_job *job = (oracle_job *)state;
  int from, upto;
  oracle_band(job->sheet->row_count, job->slice_index, job->slice_count, &from, &upto);
  for (int n = from; n < upto; ++n) {
    if (job->lane_count == 1)
      job->out[n] = oracle_row_code(job->sheet, n, job->act, job->sum);
    else
      oracle_row_code_many(job->sheet, n, job->act, job->act_stride, job->lane_count, job->sum,
                           job->sheet->group_count, job->out, job->out_stride);
  }
  return NULL;
}

/* back_mat_mat on a build without the integer grid (app_core.c:5247-5323):
 * lanes in chunks of sixteen, group sums for each lane, then rows banded over
 * the threads (the reference forks its pool only from 64 rows, 5318). */
int oracle_mat_mat(const oracle_plane *sheet, const float *act, int act_stride, int lane_count,
                   float *out, int out_stride, int thread_count) {
  float *sum_room = (float *)malloc(sizeof(float) * (size_t)sheet->group_count * ORACLE_LANE_LIMIT);
  pthread_t tid[256];
  oracle_job job[256];
  int done = 0;
  if (!sum_room) return -2;
  if (thread_count < 1) thread_count = 1;
  if (thread_count > 256) thread_count = 256;
  if (sheet->row_count < 64) thread_count = 1;
  while (done < lane_count) {
    int chunk = lane_count - done < ORACLE_LANE_LIMIT ? lane_count - done : ORACLE_LANE_LIMIT;
    const float *chunk_act = act + (size_t)done * (size_t)act_stride;
    float *chunk_out = out + (size_t)done * (size_t)out_stride;
    for (int l = 0; l < chunk; ++l)
      oracle_group_sum(sheet, chunk_act + (size_t)l * (size_t)act_stride,
                       sum_room + (size_t)l * (size_t)sheet->group_count);
    for (int t = 0; t < thread_count; ++t) {
      job[t].sheet = sheet;
      job[t].act = chunk_act;
      job[t].sum = sum_room;
      job[t].out = chunk_out;
      job[t].act_stride = act_stride;
      job[t].out_stride = out_stride;
      job[t].lane_count = chunk;
      job[t].slice_index = t;
      job[t].slice_count = thread_count;
    }
    for (int t = 1; t < thread_count; ++t) pthread_create(&tid[t], NULL, oracle_band_run, &job[t]);
    oracle_band_run(&job[0]);
    for (int t = 1; t < thread_count; ++t) pthread_join(tid[t], NULL);
    done += chunk;
  }
  free(sum_room);
  return 0;
}

/* The product of a plane the export calibrated (enter_gain = step > 0) on the
 * integer grid, the reference's level path (back_mat_mat 5283-5306 with
 * exact_flag; kern_level_stage 2924-2963, kern_row_code_level 3272-3296 and
 * kern_row_code_level_many 4204-4229): each activation is its quant_step
 * level L = rint(x / step) clamped to [-128, 127] (kern_level_of reads the
 * same level back off quant_step's output), and per group
 *     part = sum ((code ^ flip) L) - bias sum L        (exact, 64-bit)
 *     total += gain * step * (float)part               (in group order).
 * The reference takes this path only where kern_level_ready holds (2, 4 or 8
 * bits; one group, or groups a multiple of 64 columns) and every value of every
 * lane of the 16-lane chunk is on the grid; otherwise the chunk goes to the
 * float path on the quant_step values, and so does this function (a NaN is
 * what puts a value off the grid here).  Returns 0. */
static int oracle_level_ready(const oracle_plane *sheet) {
  int span;
  if (sheet->bit_count != 2 && sheet->bit_count != 4 && sheet->bit_count != 8) return 0;
  if (sheet->group_count > 1 && sheet->group_size % 64) return 0;
  span = sheet->group_count > 1 ? sheet->group_size : sheet->col_count;
  return (int64_t)span * (int64_t)((1 << sheet->bit_count) - 1) * 128 <= (int64_t)INT32_MAX;
}

int oracle_mat_mat_level(const oracle_plane *sheet, const float *act, int act_stride,
                         int lane_count, float step, float *out, int out_stride) {
  int K = sheet->col_count;
  int8_t *levels = (int8_t *)malloc((size_t)K * ORACLE_LANE_LIMIT);
  float *grid = (float *)malloc(sizeof(float) * (size_t)K * ORACLE_LANE_LIMIT);
  int64_t *lsum = (int64_t *)malloc(sizeof(int64_t) * (size_t)sheet->group_count * ORACLE_LANE_LIMIT);
  int done = 0, rc = 0;
  if (!levels || !grid || !lsum) {
    rc = -2;
    goto out;
  }
  while (done < lane_count) {
    int chunk = lane_count - done < ORACLE_LANE_LIMIT ? lane_count - done : ORACLE_LANE_LIMIT;
    int on_grid = oracle_level_ready(sheet);
    for (int l = 0; l < chunk; ++l)
      for (int k = 0; k < K; ++k) {
        float v = act[(size_t)(done + l) * (size_t)act_stride + (size_t)k];
        float level = rintf(v / step);
        if (level < -128.0f) level = -128.0f;
        if (level > 127.0f) level = 127.0f;
        grid[(size_t)l * (size_t)K + (size_t)k] = level * step;
        if (level != level) on_grid = 0;
        else levels[(size_t)l * (size_t)K + (size_t)k] = (int8_t)level;
      }
    if (!on_grid) {
      rc = oracle_mat_mat(sheet, grid, K, chunk, out + (size_t)done * (size_t)out_stride, out_stride, 1);
      if (rc) goto out;
      done += chunk;
      continue;
    }
    for (int l = 0; l < chunk; ++l)
      for (int g = 0; g < sheet->group_count; ++g) {
        int lo = g * sheet->group_size;
        int hi = lo + sheet->group_size < K ? lo + sheet->group_size : K;
        int64_t s = 0;
        for (int k = lo; k < hi; ++k) s += levels[(size_t)l * (size_t)K + (size_t)k];
        lsum[(size_t)l * (size_t)sheet->group_count + (size_t)g] = s;
      }
    for (int n = 0; n < sheet->row_count; ++n) {
      const uint8_t *row = sheet->code_data + (size_t)n * sheet->row_stride;
      for (int l = 0; l < chunk; ++l) {
        float total = 0.0f;
        for (int g = 0; g < sheet->group_count; ++g) {
          size_t at = (size_t)n * (size_t)sheet->group_count + (size_t)g;
          int lo = g * sheet->group_size;
          int hi = lo + sheet->group_size < K ? lo + sheet->group_size : K;
          int64_t bias = sheet->code_bias + (sheet->bias_data ? sheet->bias_data[at] : 0);
          int64_t part = 0;
          for (int k = lo; k < hi; ++k)
            part += (int64_t)(oracle_pack_read(row, (size_t)k, sheet->bit_count) ^ (uint32_t)sheet->code_flip) *
                    (int64_t)levels[(size_t)l * (size_t)K + (size_t)k];
          part -= bias * lsum[(size_t)l * (size_t)sheet->group_count + (size_t)g];
          total += sheet->gain_data[at] * step * (float)part;
        }
        out[(size_t)(done + l) * (size_t)out_stride + (size_t)n] = total;
      }
    }
    done += chunk;
  }
out:
  free(levels);
  free(grid);
  free(lsum);
  return rc;
}

/* A real plane's product (kern_mat_vec_band's PLANE_REAL arm,
 * app_core.c:4239-4248): every row against every lane with kern_dot_real.
 * fp32 and bf16 rows take its SSE2 blocks (2048-2066 and 2102-2112: a bf16
 * value widens exactly, so the bf16 arm is the fp32 arm on the widened row);
 * any other type the sequential walk (2137-2139), here binary16.
 * `real_type`: ORACLE_REAL_F32, ORACLE_REAL_F16 or ORACLE_REAL_BF16. */
static float oracle_real_read(const void *row, int real_type, int slot) {
  uint32_t bits;
  float value;
  if (real_type == ORACLE_REAL_F32) return ((const float *)row)[slot];
  if (real_type == ORACLE_REAL_BF16) {
    bits = (uint32_t)((const uint16_t *)row)[slot] << 16;
    memcpy(&value, &bits, 4);
    return value;
  }
  {
    uint16_t h = ((const uint16_t *)row)[slot];
    int e = (h >> 10) & 31, m = h & 1023;
    value = e == 0 ? ldexpf((float)m, -24) : e == 31 ? (m ? NAN : INFINITY) : ldexpf((float)(m + 1024), e - 25);
    return (h & 0x8000) ? -value : value;
  }
}

int oracle_mat_mat_real(const void *real_data, int real_type, int row_count, int col_count,
                        const float *act, int act_stride, int lane_count, float *out,
                        int out_stride) {
  size_t row_bytes = (size_t)col_count * (real_type == ORACLE_REAL_F32 ? 4u : 2u);
  float *wide = (float *)malloc(sizeof(float) * (size_t)col_count);
  if (!wide) return -2;
  for (int n = 0; n < row_count; ++n) {
    const void *row = (const uint8_t *)real_data + (size_t)n * row_bytes;
    for (int k = 0; k < col_count; ++k) wide[k] = oracle_real_read(row, real_type, k);
    for (int l = 0; l < lane_count; ++l) {
      const float *x = act + (size_t)l * (size_t)act_stride;
      float total = 0.0f;
      if (real_type == ORACLE_REAL_F16)
        for (int k = 0; k < col_count; ++k) total += wide[k] * x[k];
      else
        total = oracle_dot_real(wide, x, col_count);
      out[(size_t)l * (size_t)out_stride + (size_t)n] = total;
    }
  }
  free(wide);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* FP8 E4M3 cache codec (app_core.c:7488-7490, 10980-11036)                  */
/* ------------------------------------------------------------------------ */

#define ORACLE_FP8_TOP  448.0f
#define ORACLE_FP8_NORM (1.0f / 64.0f)
#define ORACLE_FP8_STEP (1.0f / 512.0f)

/* Nearest grid value, ties to even, saturating at +-448 (NaN saturates too):
 * below 2^-6 the grid is uniform in steps of 2^-9; above it a value in
 * [2^(e-1), 2^e) is a multiple of 2^(e-4) (cache_pack8, 10980-10991). */
float oracle_pack8(float value) {
  float sign = value < 0.0f ? -1.0f : 1.0f;
  float mag = value < 0.0f ? -value : value;
  int power;
  float unit;
  if (!(mag < ORACLE_FP8_TOP)) return sign * ORACLE_FP8_TOP;
  if (mag < ORACLE_FP8_NORM) return sign * rintf(mag / ORACLE_FP8_STEP) * ORACLE_FP8_STEP;
  (void)frexpf(mag, &power);
  unit = ldexpf(1.0f, power - 4);
  mag = rintf(mag / unit) * unit;
  return sign * (mag > ORACLE_FP8_TOP ? ORACLE_FP8_TOP : mag);
}

/* The byte of the rounded value: sign, four exponent bits biased by seven,
 * three mantissa bits; exponent field zero holds multiples of 2^-9
 * (cache_code8, 11006-11016). */
uint8_t oracle_code8(float value) {
  float mag = oracle_pack8(value);
  uint8_t sign = 0;
  int power, mant;
  if (mag < 0.0f) { sign = 0x80u; mag = -mag; }
  if (mag < ORACLE_FP8_NORM) return (uint8_t)(sign | (uint8_t)(int)(mag / ORACLE_FP8_STEP + 0.5f));
  (void)frexpf(mag, &power);
  mant = (int)(ldexpf(mag, 4 - power) + 0.5f) - 8;
  return (uint8_t)(sign | (uint8_t)((power + 6) << 3) | (uint8_t)mant);
}

/* Byte to value: (8 + m) * 2^(e - 10) for e > 0, m * 2^-9 for e = 0; 0x7F
 * decodes as 480 here, not NaN (cache_real8, 11018-11030). */
float oracle_real8(uint8_t code) {
  int e = (code >> 3) & 15, m = code & 7;
  float mag = e == 0 ? (float)m * ORACLE_FP8_STEP : ldexpf((float)(8 + m), e - 10);
  return (code & 0x80u) ? -mag : mag;
}

/* The table a byte row is read through, with the scale folded in
 * (cache_grid_fill, 11032-11036). */
void oracle_grid_fill8(float *grid, float scale) {
  for (int c = 0; c < 256; ++c) grid[c] = oracle_real8((uint8_t)c) * scale;
}

/* int8 variant (not in the reference, which stores e4m3): a byte is the
 * two's-complement level rint(x / scale) clamped to +-127. */
uint8_t oracle_code_i8(float value, float scale) {
  float level = rintf(value / scale);
  if (!(level > -127.0f)) level = -127.0f; /* also catches NaN */
  if (level > 127.0f) level = 127.0f;
  return (uint8_t)(int8_t)level;
}

void oracle_grid_fill_i8(float *grid, float scale) {
  for (int c = 0; c < 256; ++c) grid[c] = (float)(int8_t)(uint8_t)c * scale;
}

void oracle_encode8_many(const float *row, size_t count, float scale, uint8_t *out) {
  for (size_t i = 0; i < count; ++i) out[i] = oracle_code8(row[i] / scale);
}

void oracle_encode_i8_many(const float *row, size_t count, float scale, uint8_t *out) {
  for (size_t i = 0; i < count; ++i) out[i] = oracle_code_i8(row[i], scale);
}

/* ------------------------------------------------------------------------ */
/* softmax                                                                  */
/* ------------------------------------------------------------------------ */

/* e^x as 2^k * e^r with k the nearest integer to x/ln2 and r reduced in two
 * pieces of ln2, e^r by its Taylor series to the 7th term in Horner form, and
 * arguments below -87 floored (kern_exp_near, app_core.c:4739-4777). */
#define ORACLE_EXP_FLOOR (-87.0f)
#define ORACLE_LOG2E 1.4426950408889634f
#define ORACLE_LN2_HI 0.693359375f
#define ORACLE_LN2_LO (-2.1219444005469057e-4f)

float oracle_exp_near(float value) {
  float stepped, whole, rest, poly, scale;
  uint32_t bits;
  if (value < ORACLE_EXP_FLOOR) value = ORACLE_EXP_FLOOR;
  stepped = value * ORACLE_LOG2E + 0.5f;
  whole = (float)(int)stepped;
  if (whole > stepped) whole -= 1.0f;
  rest = value - whole * ORACLE_LN2_HI;
  rest -= whole * ORACLE_LN2_LO;
  poly = 1.0f / 5040.0f;
  poly = poly * rest + 1.0f / 720.0f;
  poly = poly * rest + 1.0f / 120.0f;
  poly = poly * rest + 1.0f / 24.0f;
  poly = poly * rest + 1.0f / 6.0f;
  poly = poly * rest + 1.0f / 2.0f;
  poly = poly * rest + 1.0f;
  poly = poly * rest + 1.0f;
  bits = (uint32_t)((int)whole + 127) << 23;
  memcpy(&scale, &bits, sizeof(scale));
  return poly * scale;
}

/* Three passes, SSE2 tier (kern_soft_max, app_core.c:4856-4993): the peak
 * over four-lane blocks then the tail; e^(v - peak) per element with the four
 * lane totals folded like the dot's, the tail added one at a time; then every
 * value times 1/total.  The SSE2 exponential is the scalar series with the
 * same roundings (no fused multiply-add on that tier). */
void oracle_soft_max(float *v, int n) {
  float peak = -FLT_MAX, total = 0.0f;
  int i = 0;
  if (n >= 4) {
    float lane_peak[4] = {v[0], v[1], v[2], v[3]};
    float lane_total[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float even, odd;
    for (i = 4; i + 4 <= n; i += 4)
      for (int j = 0; j < 4; ++j)
        lane_peak[j] = v[i + j] > lane_peak[j] ? v[i + j] : lane_peak[j];
    /* _mm_max_ps(a, b) returns b unless a > b; the fold mirrors that. */
    even = lane_peak[0] > lane_peak[2] ? lane_peak[0] : lane_peak[2];
    odd = lane_peak[1] > lane_peak[3] ? lane_peak[1] : lane_peak[3];
    peak = even > odd ? even : odd;
    for (; i < n; ++i)
      if (v[i] > peak) peak = v[i];
    for (i = 0; i + 4 <= n; i += 4)
      for (int j = 0; j < 4; ++j) {
        v[i + j] = oracle_exp_near(v[i + j] - peak);
        lane_total[j] = lane_total[j] + v[i + j];
      }
    total = oracle_fold4(lane_total);
  } else {
    for (; i < n; ++i)
      if (v[i] > peak) peak = v[i];
    i = 0;
  }
  for (; i < n; ++i) {
    v[i] = oracle_exp_near(v[i] - peak);
    total += v[i];
  }
  if (total > 0.0f) {
    float shrink = 1.0f / total;
    for (i = 0; i < n; ++i) v[i] *= shrink;
  }
}

/* ------------------------------------------------------------------------ */
/* decode attention                                                         */
/* ------------------------------------------------------------------------ */

/* Scores for every visible position and every head of the group, each a
 * kern_dot_real of the decoded key row against the head's query
 * (attend_score_band, 11296-11321); a softmax per head and the blend
 * o_h = sum_t p_h[t] v_t added in position order (attend_blend_band,
 * 11333-11365).  Ring slot of position p is p % cache_span (cache_block,
 * 11165-11181).  Blocking rows into 8 KB runs changes no arithmetic, so the
 * rows are decoded one at a time here. */
void oracle_attend(const uint8_t *key_store, const uint8_t *value_store, const float *key_grid,
                   const float *value_grid, int cache_span, int kv_width, int kv_index,
                   const float *query, int head_first, int group_share, int head_size,
                   int place_start, int span_count, float score_scale, float *blend_out,
                   float *score_room) {
  float row[1024];
  for (int t = 0; t < span_count; ++t) {
    size_t at = (size_t)((place_start + t) % cache_span) * (size_t)kv_width +
                (size_t)kv_index * (size_t)head_size;
    for (int d = 0; d < head_size; ++d) row[d] = key_grid[key_store[at + (size_t)d]];
    for (int h = 0; h < group_share; ++h) {
      float s = oracle_dot_real(row, query + (size_t)(head_first + h) * (size_t)head_size, head_size);
      if (score_scale != 1.0f) s *= score_scale;
      score_room[(size_t)h * (size_t)span_count + (size_t)t] = s;
    }
  }
  for (int h = 0; h < group_share; ++h) {
    float *blend = blend_out + (size_t)(head_first + h) * (size_t)head_size;
    oracle_soft_max(score_room + (size_t)h * (size_t)span_count, span_count);
    for (int d = 0; d < head_size; ++d) blend[d] = 0.0f;
  }
  for (int t = 0; t < span_count; ++t) {
    size_t at = (size_t)((place_start + t) % cache_span) * (size_t)kv_width +
                (size_t)kv_index * (size_t)head_size;
    for (int d = 0; d < head_size; ++d) row[d] = value_grid[value_store[at + (size_t)d]];
    for (int h = 0; h < group_share; ++h) {
      float *blend = blend_out + (size_t)(head_first + h) * (size_t)head_size;
      float w = score_room[(size_t)h * (size_t)span_count + (size_t)t];
      for (int d = 0; d < head_size; ++d) blend[d] += w * row[d];
    }
  }
}

/* ------------------------------------------------------------------------ */
/* the other table entries                                                  */
/* ------------------------------------------------------------------------ */

/* x * (mean of squares in double + eps)^-1/2 (* gain), the scale rounded to
 * float once (kern_norm_rms, app_core.c:4667-4684). */
void oracle_norm_rms(const float *value_list, const float *gain_list, int value_count,
                     float eps_value, float *value_out) {
  double squares = 0.0;
  float shrink;
  for (int i = 0; i < value_count; ++i) squares += (double)value_list[i] * (double)value_list[i];
  shrink = (float)pow(squares / (double)value_count + (double)eps_value, -0.5);
  for (int i = 0; i < value_count; ++i)
    value_out[i] = gain_list ? value_list[i] * shrink * gain_list[i] : value_list[i] * shrink;
}

/* gate * rise with gate = x t / (t + 1), t = e^(2 sqrt(2/pi)(x + 0.044715 x^3)),
 * zero when that exponent is at or below -30, and clamped at +30
 * (kern_gelu_tanh, app_core.c:5105-5118). */
void oracle_gelu_gate(float *gate_list, const float *rise_list, int value_count) {
  for (int i = 0; i < value_count; ++i) {
    float x = gate_list[i];
    float cube = x * x * x;
    float turn = 2.0f * 0.7978845608028654f * (x + 0.044715f * cube);
    float g;
    if (!(turn > -30.0f)) {
      g = x * 0.0f;
    } else {
      float t = oracle_exp_near(turn > 30.0f ? 30.0f : turn);
      g = x * (t / (t + 1.0f));
    }
    gate_list[i] = g * rise_list[i];
  }
}

/* Rotate-half: (a, b) -> (a cos - b sin, b cos + a sin) over the two halves
 * (kern_rope_turn, app_core.c:5196-5207). */
void oracle_rope_turn(float *value_list, int head_size, const float *cos_list,
                      const float *sin_list) {
  int half = head_size / 2;
  for (int i = 0; i < half; ++i) {
    float lo = value_list[i], hi = value_list[i + half];
    value_list[i] = lo * cos_list[i] - hi * sin_list[i];
    value_list[i + half] = hi * cos_list[i] + lo * sin_list[i];
  }
}

double oracle_clock(void) {
  struct timespec now;
  clock_gettime(CLOCK_MONOTONIC, &now);
  return (double)now.tv_sec + 1e-9 * (double)now.tv_nsec;
}
