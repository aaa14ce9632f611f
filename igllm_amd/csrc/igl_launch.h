/* igl_launch.h - launchers the HIP kernel files export to the C11 shim.
 * Each returns the launch's hipError_t; none validates its arguments (the shim
 * does, before calling). */
#ifndef IGL_LAUNCH_H
#define IGL_LAUNCH_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#include "igl_backend.h"

#ifdef __cplusplus
extern "C" {
#endif

/* A code plane as the kernels read it: 32-column unit u of a row takes gain
 * u >> group_shift of that row (group_shift 31: one gain a row); a code's
 * value is (code ^ code_flip) - code_bias. */
typedef struct igl_code_view {
  const uint8_t *codes;
  long long row_stride;
  const float *gains;
  int gain_stride;
  int group_shift;
  int bit_count;
  int code_bias;
  int code_flip;
} igl_code_view;

/* The group_shift of a plane whose group size is 32 times a power of two, or
 * that has one group a row. */
static inline int igl_plane_group_shift(const igl_plane *sheet) {
  int shift = 0;
  if (sheet->group_count == 1) return 31;
  while ((32 << shift) < sheet->group_size) ++shift;
  return shift;
}

static inline igl_code_view igl_plane_view(const igl_plane *sheet, const void *codes,
                                           const float *gains) {
  igl_code_view v;
  v.codes = (const uint8_t *)codes;
  v.row_stride = (long long)sheet->row_stride;
  v.gains = gains;
  v.gain_stride = sheet->group_count;
  v.group_shift = igl_plane_group_shift(sheet);
  v.bit_count = sheet->bit_count;
  v.code_bias = sheet->code_bias;
  v.code_flip = sheet->code_flip;
  return v;
}

size_t igl_gemv_code_part_floats(int bit_count, int lanes, int N, int K);
/* A plane with zero points (`zeros` [N][gain_stride], int8): kern_row_code's
 * form, gain * (dot - (code_bias + zero) * sum) a group, any lane count. */
hipError_t igl_launch_gemv_zero(const igl_code_view *v, const int8_t *zeros, const float *act,
                                int act_stride, int lanes, float *out, int out_stride, int N, int K,
                                hipStream_t stream);
hipError_t igl_launch_gemv_codes(const igl_code_view *v, const float *act, int act_stride,
                                 int lanes, float *out, int out_stride, int N, int K,
                                 float *part, hipStream_t stream);

int igl_gemv_level_fits(int bit_count, int K);
hipError_t igl_launch_gemv_level(const igl_code_view *v, float step, float leave, const float *act,
                                 int act_stride, int lanes, float *out, int out_stride, int N, int K,
                                 hipStream_t stream);
/* The step after a product, fused into its store: none; out = gelu(epi_in) * y
 * (the up projection after the gate's, kern_gelu_gate); out = gelu(y) * epi_in
 * (the per-layer-input gate). */
enum { IGL_LEVEL_EPI_NONE = 0, IGL_LEVEL_EPI_GELU_RISE = 1, IGL_LEVEL_EPI_GELU_MUL = 2 };
hipError_t igl_launch_gemv_level_epi(const igl_code_view *v, float step, float leave, const float *act,
                                     int act_stride, int lanes, float *out, int out_stride, int N, int K,
                                     int epi, const float *epi_in, int epi_stride, hipStream_t stream);
size_t igl_gemv_real_part_floats(int lanes, int N, int K);
hipError_t igl_launch_gemv_real(const void *rows, int real_type, const float *act, int act_stride,
                                int lanes, float *out, int out_stride, int N, int K, float *part,
                                hipStream_t stream);

int igl_gemv_rows_per_tile(int lanes);
int igl_gemv_chunk_cols(int lanes, int K, int lds_limit);
size_t igl_gemv_part_floats(int lanes, int N, int K, int lds_limit);
/* modes of igl_launch_gemv_group */
#define IGL_GEMV_SEGMENTS 0
#define IGL_GEMV_GELU_PAIR 1
#define IGL_GEMV_GELU_MUL 2
/* The residual update a grouped launch can form in front of its product, in
 * place of reading `act`: s = (state_in + norm(lift) * lift_gain) * scale
 * (lift NULL: s = state_in), written to state_out by one workgroup; the
 * activations are norm(s) * norm_gain (norm_gain NULL: s).  K <= 4096.
 * Lanes of state_in, state_out and lift lie lane_stride floats apart (read
 * by igl_launch_gemv_group with several lanes only).  Callers outside C
 * mirror this layout field for field. */
typedef struct igl_gemv_prologue {
  const float *state_in;
  float *state_out;
  const float *lift;
  const float *lift_gain;
  float scale;
  int apply_scale;
  const float *norm_gain;
  float eps;
  int lane_stride;
} igl_gemv_prologue;
/* One lane of a calibrated plane (igl_launch_gemv_level_epi) with the residual
 * update of igl_launch_gemv_group as its prologue; x also to x_out (NULL:
 * not kept); K <= 2048. */
hipError_t igl_launch_gemv_level_pro(const igl_code_view *v, float step, float leave,
                                     const igl_gemv_prologue *pro, float *x_out, float *out, int N,
                                     int K, int epi, const float *epi_in, hipStream_t stream);
/* The gate and up planes of one lane in one launch, out = gelu(gate) * up
 * (each product on its own leave grid), the residual update as the prologue:
 * both planes the same kind (bits, bias, flip, gain layout), N rows and enter
 * step; K <= 2048. */
hipError_t igl_launch_gemv_level_pair(const igl_code_view *gate, const igl_code_view *up, float step,
                                      float leave_gate, float leave_up, const igl_gemv_prologue *pro,
                                      float *out, int N, int K, hipStream_t stream);
/* Up to three calibrated planes of one lane that read the same input (a
 * layer's q, k and v) in one launch, the residual update as the prologue:
 * every plane the same kind and enter step, K <= 2048; plane s's rows[s]
 * outputs into out[s], on its own leave grid leave[s]. */
hipError_t igl_launch_gemv_level_segments(const igl_code_view *v, int segments, const int *rows,
                                          float *const *out, const float *leave, float step,
                                          const igl_gemv_prologue *pro, int K, hipStream_t stream);
/* One to eight lanes against up to three 4-bit planes that read the same
 * activations, in one launch with the mode's epilogue; lane m of act, out[s]
 * and mul lies m act_stride, m out_stride[s], m mul_stride floats in. */
hipError_t igl_launch_gemv_group(int mode, int lanes, int segments, const uint8_t *const *codes,
                                 const long long *row_stride, const float *const *gains,
                                 const int *gain_stride, const int *rows, float *const *out,
                                 const int *out_stride, int group_shift, int code_bias,
                                 const float *act, int act_stride, int K, const float *mul,
                                 int mul_stride, const igl_gemv_prologue *pro, hipStream_t stream);
hipError_t igl_launch_gemv_q4(const uint8_t *codes, long long row_stride, const float *gains,
                              int gain_stride, int group_shift, int code_bias, const float *act,
                              int act_stride, int lanes, float *out, int out_stride, int N, int K,
                              float *part, int lds_limit, hipStream_t stream);

/* The row close of a calibrated plane's product taken on levels and unit gains:
 * C = quant_step(gains[n] * step * acc, leave) (fp32 C).  With `gains` set the
 * activations are also put on the grid of `step` (their levels) as they are
 * converted.  fp32 activations and output only. */
typedef struct igl_gemm_close {
  const float *gains;
  float step;
  float leave;
} igl_gemm_close;

/* The prefill GEMM on 4-bit codes (code_bias 0..15, no flip): shapes it takes
 * (K a multiple of 64), the workspace it needs, and the form it would pick
 * (for tests and the bench).  `act_terms`: 1 takes each activation as one
 * binary16 term after its row's power-of-two scale (exact for bf16
 * activations and for levels), 2 as hi + lo (fp32 activations to a relative
 * 2^-22).  `zero_pairs`: NULL, or per (row, group) the binary16 pair
 * (1024 + code_bias + zero, 1024 + 16 (code_bias + zero)) as one word
 * (igl_launch_zero_pairs). */
int igl_gemm_fits(int M, int N, int K);
size_t igl_gemm_work_bytes(int M, int N, int K, int act_terms);
int igl_gemm_form(int M, int N, int K, int act_terms);
int igl_gemm_slices(int M, int N, int K, int act_terms);
hipError_t igl_launch_gemm_q4(const void *act, int act_bf16, int act_stride, const uint8_t *codes,
                              long long row_stride, const float *gains, int gain_stride,
                              int group_shift, int code_bias, const uint32_t *zero_pairs, void *out,
                              int out_bf16, int out_stride, int M, int N, int K, int act_terms,
                              void *work, const igl_gemm_close *close, hipStream_t stream);

size_t igl_attend_work_floats(int place0, int window, int lanes, int head_count, int head_size);
/* The device address of the fixed attention workspace on `device`
 * (IGL_ATTEND_FIXED_FLOATS floats), resolved once per device with it current
 * (igl_back_open); NULL before. */
hipError_t igl_attend_fixed_resolve(int device);
float *igl_attend_fixed_ptr(int device);
/* Enough for every call of at most `lanes` lanes whose spans stay within
 * `span_limit` positions (the chunk count is not monotonic in the span). */
size_t igl_attend_work_floats_limit(int span_limit, int lanes, int head_count, int head_size);
hipError_t igl_launch_attend(const uint8_t *key_store, const uint8_t *value_store, int fmt,
                             float key_scale, float value_scale, int cache_span, int kv_width,
                             int kv_count, int group_share, int head_size, const float *query,
                             int q_stride, int place0, const int *place_dev, int window,
                             int lanes, float score_scale, float *blend_out, float *work,
                             hipStream_t stream);

/* The attention of a decode step or a small block (1 to 4 lanes) with the
 * query, key and value heads prepared in the same launch (norms, gains, turns,
 * the new ring rows): e4m3 rings, one key/value head; lane l's query, turn row
 * and raw key/value heads q_stride, turn_stride and kv_stride floats after
 * lane l - 1's; k_raw NULL for a layer that writes no row. */
hipError_t igl_launch_attend_prep(const uint8_t *key_store, const uint8_t *value_store,
                                  float key_scale, float value_scale, int cache_span,
                                  int head_size, int lanes, const float *query, int q_stride,
                                  const float *q_gain, const float *turn, int turn_stride,
                                  const float *k_raw, const float *v_raw, int kv_stride,
                                  const float *k_gain, uint8_t *k_ring, uint8_t *v_ring,
                                  float eps, int place_bound, const int *place_dev, int window,
                                  float score_scale, float *blend_out, float *work,
                                  hipStream_t stream);

size_t igl_attend_prep_work_floats(int place_bound, int window, int head_size, int lanes,
                                   int writes_row);

/* The desk's HIP stream, for the engine's own launches (back_hip.c). */
void *igl_desk_stream(igl_desk *desk);
/* Changes whenever the desk reallocates a workspace: a graph captured over
 * desk launches outside igl_record_begin / igl_record_end is stale once it
 * differs from the value at capture. */
unsigned igl_desk_generation(igl_desk *desk);

/* session kernels (igl_session.hip) */
hipError_t igl_launch_gather_rows(const igl_code_view *v, int cols, int rows, const int32_t *ids,
                                  int lanes, float factor, float *out, int out_stride,
                                  hipStream_t stream);
hipError_t igl_launch_ple_mix(float *room, int room_stride, const float *seed, int seed_stride,
                              const float *gain, int ple, int chunks, int lanes, float eps,
                              float lift_scale, float blend, hipStream_t stream);
hipError_t igl_launch_head_prep(float *v, int lane_stride, int heads, int head_size, int lanes,
                                const float *gain, float eps, const float *step, int turn,
                                int place_first, hipStream_t stream);
hipError_t igl_launch_put_int(int32_t *dst, int value, hipStream_t stream);
/* (cos, sin) of the positions *place_dev .. *place_dev + lanes - 1 times each
 * step of both kinds of layer, as float pairs [lanes][half][2]. */
hipError_t igl_launch_turn_row(const float *step0, int half0, const float *step1, int half1,
                               const int *place_dev, int lanes, float *turn0, float *turn1,
                               hipStream_t stream);
hipError_t igl_launch_qkv_prep(float *q, int q_stride, const float *k, const float *v,
                               int kv_stride, int heads, int head_size, int lanes,
                               const float *q_gain, const float *k_gain, float eps,
                               const float *step, const int *place_dev, uint8_t *k_store,
                               uint8_t *v_store, float k_scale, float v_scale, int span,
                               hipStream_t stream);
hipError_t igl_launch_norm_add(float *state, int state_stride, const float *lift, int lift_stride,
                               const float *after_gain, int n, int lanes, float eps, float scale,
                               int apply_scale, const float *next_gain, float *out,
                               int out_stride, hipStream_t stream);
hipError_t igl_launch_add_rows(float *into, int into_stride, const float *from, int from_stride,
                               int n, int lanes, float gain, int apply_gain, hipStream_t stream);
hipError_t igl_launch_scale_rows(float *v, int stride, int n, int lanes, float gain,
                                 hipStream_t stream);
hipError_t igl_launch_gelu_mul(float *gate, int gate_stride, const float *ple, int ple_stride,
                               int n, int lanes, hipStream_t stream);
hipError_t igl_launch_gelu_gate_rows(float *gate, int gate_stride, const float *rise,
                                     int rise_stride, int n, int lanes, hipStream_t stream);
hipError_t igl_launch_cache_lay_rows(const float *rows, int row_stride, int width, float scale,
                                     uint8_t *store, int span, int place_first, int lanes,
                                     hipStream_t stream);
size_t igl_pick_work_bytes(int lanes);
/* The greedy pick of `lanes` rows of n logits, `stride` floats apart; with
 * cap > 0 the rows are first capped in place (the final logit softcap). */
hipError_t igl_launch_pick(float *v, int n, size_t stride, int lanes, float cap, void *work,
                           int32_t *pairs, hipStream_t stream);

hipError_t igl_launch_quant_step(const float *src, int src_stride, float *dst, int dst_stride,
                                 int n, int lanes, float step, hipStream_t stream);
/* the prefill of a calibrated plane (igl_elem.hip) */
hipError_t igl_launch_quant_level(const float *src, int src_stride, float *dst, int dst_stride,
                                  int n, int lanes, float step, float *lsum, hipStream_t stream);
hipError_t igl_launch_code_widen(const uint8_t *codes, long long row_stride, int N, int K, int bits,
                                 int flip, int bias, uint8_t *hi_plane, uint8_t *lo_plane,
                                 hipStream_t stream);
hipError_t igl_launch_grid_close(const float *a, const float *b, const float *lsum, int in_stride,
                                 const float *gains, float step, float leave, int N, int lanes,
                                 float *out, int out_stride, hipStream_t stream);
hipError_t igl_launch_fill(float *dst, size_t n, float value, hipStream_t stream);
/* The prefill of a calibrated plane with one gain a row on the integer matrix
 * cores (igl_gemm_level.hip): levels of act on close->step, exact int32 sums
 * against the codes, then gain * step * part and the leave grid; a lane with a
 * NaN gives NaN outputs.  Fits: 2-, 4- or 8-bit codes with code_bias
 * 2^(bits-1), K a multiple of 128 (64 for 8-bit); row_stride a multiple of 16;
 * act 16-byte aligned with act_stride % 4 == 0.  `work` holds
 * igl_gemm_level_work_bytes(M, N, K, bits) bytes. */
int igl_gemm_level_fits(int bits, int code_bias, int K);
size_t igl_gemm_level_work_bytes(int M, int N, int K, int bits);
hipError_t igl_launch_gemm_level(const float *act, int act_stride, const uint8_t *codes, long long row_stride,
                                 int bits, int code_flip, int code_bias, const igl_gemm_close *close, float *out,
                                 int out_stride, int M, int N, int K, void *work, hipStream_t stream);
/* Reads `bytes` (a multiple of 16) of src once and keeps nothing (sink: one
 * word, written only on an improbable fold). */
hipError_t igl_launch_read_floor(const void *src, size_t bytes, uint32_t *sink, hipStream_t stream);
hipError_t igl_launch_norm_rms(const float *in, const float *gain, int n, int rows, int stride,
                               float eps, float *out, hipStream_t stream);
hipError_t igl_launch_soft_max(float *v, int n, int rows, int stride, hipStream_t stream);
hipError_t igl_launch_gelu_gate(float *gate, const float *rise, int n, hipStream_t stream);
hipError_t igl_launch_rope_turn(float *v, int heads, int head_size, const float *cosv,
                                const float *sinv, hipStream_t stream);
hipError_t igl_launch_cache_lay(const float *row, int width, float scale, int fmt, uint8_t *store,
                                size_t slot_first, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif
