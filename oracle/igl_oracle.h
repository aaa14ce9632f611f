/* igl_oracle.h - CPU restatement of igllm's fp32 projection and decode-attention
 * path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the HIP backend is
 * held against; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it.  Nothing in igllm_amd/ links or calls it, and the
 * product fails loudly when its own HIP library is missing instead of falling
 * back to this code.
 *
 * Each function restates one piece of the reference's *plain* (SSE2 tier)
 * float path, in the same summation order, so that it agrees with a plain
 * build of app_core.c to the bit (the harness in ref_harness.c checks that).
 * Citations are app_core.c line numbers.
 *
 * Parity pins (tests/test_oracle.py):
 *   pack_read / plane_row  - the reference's nibble KAT (app_test.c:593-594,
 *                            651-658) and an independent bit writer
 *   row_code / mat_mat     - closed form in double; bit-exact vs oracle/_ref
 *   mat_mat_level          - closed form in double; bit-exact vs the level
 *                            (AVX-512 VNNI) build of oracle/_ref
 *   mat_mat_real           - closed form in double; bit-exact vs oracle/_ref
 *   FP8 codec              - all 256 codes against the e4m3 definition and
 *                            torch.float8_e4m3fn; round trip; bit-exact vs _ref
 *   exp_near / soft_max    - libm exp and the softmax definition; vs _ref
 *   attend                 - brute-force double attention; bit-exact vs _ref
 */
#ifndef IGL_ORACLE_H
#define IGL_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The fields of the reference's `plane` (app_core.c:1775-1795) a code plane
 * uses.  Gains are always fp32 here, as on every plane of the export. */
typedef struct oracle_plane {
  int            row_count;   /* N, output features */
  int            col_count;   /* K, input features */
  const uint8_t *code_data;   /* rows of a dense little-endian bit stream */
  size_t         row_stride;  /* bytes between rows */
  const float   *gain_data;   /* [N * group_count] */
  const int8_t  *bias_data;   /* zero points [N * group_count], NULL when symmetric */
  int            bit_count;
  int            code_bias;   /* 2^(bits-1) */
  int            code_flip;   /* 128 for signed byte planes, else 0 */
  int            group_size;
  int            group_count;
} oracle_plane;

/* quant layer */
uint32_t oracle_pack_read(const uint8_t *code_data, size_t element_index, int bit_count);
void     oracle_plane_row(const oracle_plane *sheet, int row_index, float *row_out);
float    oracle_quant_step(float value, float step);

/* projection, float path */
void  oracle_group_sum(const oracle_plane *sheet, const float *act, float *sum_out);
float oracle_dot_code(const uint8_t *code_row, int from_index, int span_count,
                      const float *act, int bit_count, int code_flip);
float oracle_row_code(const oracle_plane *sheet, int row_index, const float *act,
                      const float *sum_data);
void  oracle_row_code_many(const oracle_plane *sheet, int row_index, const float *act,
                           int act_stride, int lane_count, const float *sum_data,
                           int sum_stride, float *out, int out_stride);
/* back_mat_mat on a plain build: chunks of 16 lanes, group sums, then rows
 * banded over `thread_count` threads (1 = serial). */
int   oracle_mat_mat(const oracle_plane *sheet, const float *act, int act_stride,
                     int lane_count, float *out, int out_stride, int thread_count);
/* back_mat_mat on a calibrated plane (enter_gain = step) on the level tier:
 * activations as their quant_step levels, exact integer sums per group. */
int   oracle_mat_mat_level(const oracle_plane *sheet, const float *act, int act_stride,
                           int lane_count, float step, float *out, int out_stride);
/* back_mat_mat on a real plane (kern_dot_real per row and lane). */
#define ORACLE_REAL_F32  1  /* STORE_F32, app_core.c:1414 */
#define ORACLE_REAL_F16  2
#define ORACLE_REAL_BF16 3
int   oracle_mat_mat_real(const void *real_data, int real_type, int row_count, int col_count,
                          const float *act, int act_stride, int lane_count, float *out,
                          int out_stride);

/* FP8 E4M3 cache codec and its decode table */
float   oracle_pack8(float value);
uint8_t oracle_code8(float value);
float   oracle_real8(uint8_t code);
void    oracle_grid_fill8(float *grid, float scale);
/* The int8 variant: code = clamp(rint(x / scale), -127, 127) as a byte,
 * decoded by the same 256-entry table idea. */
uint8_t oracle_code_i8(float value, float scale);
void    oracle_grid_fill_i8(float *grid, float scale);

/* cache_lay's store loop (app_core.c:11230-11233): bytes of row[i] / scale. */
void    oracle_encode8_many(const float *row, size_t count, float scale, uint8_t *out);
void    oracle_encode_i8_many(const float *row, size_t count, float scale, uint8_t *out);

/* softmax and its exponential */
float oracle_exp_near(float value);
void  oracle_soft_max(float *value_list, int value_count);

/* One lane's decode attention for the `group_share` heads that read KV head
 * `kv_index` (session_attend_group with attend_score_band and attend_blend_band,
 * run serially).  `score_scale` multiplies every score after the dot; the
 * reference graph uses 1.0.  `score_room` holds group_share * span_count floats.
 * Byte stores only (grids non-NULL). */
void oracle_attend(const uint8_t *key_store, const uint8_t *value_store,
                   const float *key_grid, const float *value_grid, int cache_span,
                   int kv_width, int kv_index, const float *query, int head_first,
                   int group_share, int head_size, int place_start, int span_count,
                   float score_scale, float *blend_out, float *score_room);

/* The other table entries (kern_norm_rms 4667-4684, kern_gelu_gate 5105-5190
 * scalar form, kern_rope_turn 5196-5207). */
void oracle_norm_rms(const float *value_list, const float *gain_list, int value_count,
                     float eps_value, float *value_out);
void oracle_gelu_gate(float *gate_list, const float *rise_list, int value_count);
void oracle_rope_turn(float *value_list, int head_size, const float *cos_list,
                      const float *sin_list);

/* Seconds of wall clock, for the CPU baseline timer. */
double oracle_clock(void);

#ifdef __cplusplus
}
#endif

#endif
