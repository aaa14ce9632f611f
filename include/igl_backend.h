/* igl_backend.h - C ABI of the MI355X (gfx950) backend for igllm's quantized
 * projection path.
 *
 * The reference engine reaches every projection through `back_desk`, a table
 * of function pointers filled by `back_open` (app_core.c:5223-5245,
 * 5415-5443).  This header is that table's drop-in: the same six entries with
 * the same signatures and meanings, filled by `igl_back_open`, plus the pieces
 * the reference names as missing for an accelerator (GUIDE.md:567-577,
 * TODO.md:134-137): a device buffer handle beside each plane, device-resident
 * forms of the entries, a decode-attention entry and a cache writer, and a
 * sticky error, because the table's entries return void and must not fail
 * (app_core.c:5236-5244).
 *
 * Plain C11: pointers, sizes and enums only.  Two groups of entries:
 *   - the table entries take host pointers, exactly as the reference's do, and
 *     stage through the device (synchronous: the result is in `out` on return);
 *   - the `_dev` entries take device pointers, enqueue on the desk's stream
 *     and return at once; `igl_sync` waits.
 * Results of an entry that fails are left unwritten and the error is kept in
 * the desk until `igl_desk_error_take` reads it.
 */
#ifndef IGL_BACKEND_H
#define IGL_BACKEND_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Result codes: the reference's `app_code` values (app_core.c:40-49), plus one
 * for a failure the device itself reported. */
typedef enum igl_code {
  IGL_OKAY = 0,
  IGL_FAIL_ARGUMENT = -1,
  IGL_FAIL_MEMORY = -2,
  IGL_FAIL_FILE = -3,
  IGL_FAIL_FORMAT = -4,
  IGL_FAIL_MISSING = -5,
  IGL_FAIL_SUPPORT = -6,
  IGL_FAIL_STATE = -7,
  IGL_FAIL_DEVICE = -8
} igl_code;

/* `store_type` (app_core.c:1412-1424), same values. */
typedef enum igl_store_type {
  IGL_STORE_VOID = 0,
  IGL_STORE_F32,
  IGL_STORE_F16,
  IGL_STORE_BF16,
  IGL_STORE_F64,
  IGL_STORE_I8,
  IGL_STORE_U8,
  IGL_STORE_I16,
  IGL_STORE_I32,
  IGL_STORE_I64,
  IGL_STORE_BOOL
} igl_store_type;

/* `plane_form` (app_core.c:1772), same values. */
typedef enum igl_plane_form { IGL_PLANE_VOID = 0, IGL_PLANE_REAL, IGL_PLANE_CODE } igl_plane_form;

typedef struct igl_device_plane igl_device_plane;

/* A weight, field for field the reference's `plane` (app_core.c:1775-1795),
 * with the device handle `igl_plane_attach` sets beside it.  The code bytes
 * are the checkpoint's own rows (`row_stride` bytes apart, a dense
 * little-endian bit stream, low field first); nothing is repacked. */
typedef struct igl_plane {
  int            form;        /* igl_plane_form */
  int            row_count;   /* N, output features */
  int            col_count;   /* K, input features */
  const void    *real_data;
  int            real_type;   /* igl_store_type */
  const uint8_t *code_data;
  size_t         row_stride;
  const void    *gain_data;   /* [row_count * group_count] */
  int            gain_type;   /* igl_store_type; F32 is supported */
  const int8_t  *bias_data;   /* zero points, NULL when symmetric */
  int            bit_count;
  int            code_bias;
  int            code_flip;
  int            group_size;
  int            group_count;
  float          enter_gain;
  float          leave_gain;
  void          *own_block;
  igl_device_plane *device;   /* set by igl_plane_attach / igl_plane_bind_dev */
} igl_plane;

typedef struct igl_desk_state igl_desk_state;

/* The backend table: `back_desk`'s entries (app_core.c:5236-5244) with the
 * same argument meanings.  `state` replaces the reference's CPU scratch. */
typedef struct igl_desk {
  const char     *name_text;
  igl_desk_state *state;
  void (*mat_vec)(struct igl_desk *desk, const igl_plane *sheet, const float *act_data,
                  float *out_data);
  void (*mat_mat)(struct igl_desk *desk, const igl_plane *sheet, const float *act_data,
                  int act_stride, int lane_count, float *out_data, int out_stride);
  void (*norm_rms)(struct igl_desk *desk, const float *value_list, const float *gain_list,
                   int value_count, float eps_value, float *value_out);
  void (*soft_max)(struct igl_desk *desk, float *value_list, int value_count);
  void (*gelu_gate)(struct igl_desk *desk, float *gate_list, const float *rise_list,
                    int value_count);
  void (*rope_turn)(struct igl_desk *desk, float *value_list, int head_size,
                    const float *cos_list, const float *sin_list);
} igl_desk;

/* ---- opening and closing ------------------------------------------------ */

/* Replaces back_open (app_core.c:5415-5443).  `sum_limit` and `col_limit` are
 * the widest group count and column count the model binds, as the reference
 * passes them (app_core.c:12585); `lane_limit` sizes the host staging (0
 * selects the reference's 16, KERN_LANE_LIMIT app_core.c:1980).  Allocates
 * everything the token loop needs, on device `device_index`. */
int  igl_back_open(igl_desk *desk, int device_index, int sum_limit, int col_limit, int lane_limit);
/* Replaces back_close (app_core.c:5445-5453). */
void igl_back_close(igl_desk *desk);

/* The first failure since the last call, and clears it (IGL_OKAY if none). */
int  igl_desk_error_take(igl_desk *desk);
const char *igl_code_text(int code);

/* ---- weights ------------------------------------------------------------ */

/* Copies a plane's bytes (and gains) to the device unchanged and sets
 * `sheet->device`.  Supported code planes: 2, 4 or 8-bit codes with
 * code_bias 2^(bits-1) and any code_flip (the export's signed I8 planes flip
 * 128), F32 gains, optional int8 zero points (bias_data [rows][groups], as
 * plane_bind_part unpacks weight_zero_point, app_core.c:8053-8063; copied to
 * the device with the plane), group_size a power-of-two multiple of 32 or
 * one group a row, col_count a multiple of 32, row_stride a multiple of 16.
 * A row_stride of whole 32-bit words is the compressed-tensors weight_packed
 * layout (8015-8065): the same dense bit stream.
 * Supported real planes (plane_bind_part's `weight` of a float type,
 * app_core.c:7985-7998): F32, F16 or BF16 rows, col_count a multiple of 8.
 * Anything else is IGL_FAIL_SUPPORT. */
int  igl_plane_attach(igl_desk *desk, igl_plane *sheet);
/* The same for bytes and gains already on the device (no copy; the caller
 * keeps ownership).  A real plane passes its rows as `code_dev` and no gains. */
int  igl_plane_bind_dev(igl_desk *desk, igl_plane *sheet, const void *code_dev,
                        const float *gain_dev);
void igl_plane_detach(igl_desk *desk, igl_plane *sheet);

/* ---- device-resident entries (enqueue on the desk's stream) -------------- */

/* y = W x for `lane_count` lanes of fp32 activations: 1..8 lanes a launch
 * take the HBM-streaming GEMV (more lanes run in chunks of 8); from
 * `igl_gemm_lane_floor()` lanes on, the MFMA GEMM. */
int igl_mat_mat_dev(igl_desk *desk, const igl_plane *sheet, const float *act_dev, int act_stride,
                    int lane_count, float *out_dev, int out_stride);
/* Always the GEMV path (lanes in chunks of 8), whatever the lane count. */
int igl_gemv_dev(igl_desk *desk, const igl_plane *sheet, const float *act_dev, int act_stride,
                 int lane_count, float *out_dev, int out_stride);
/* Batched prefill: bf16 activations [lanes][act_stride] -> bf16 [lanes][out_stride],
 * fp32 accumulate, on the MFMA GEMM. */
int igl_gemm_bf16_dev(igl_desk *desk, const igl_plane *sheet, const uint16_t *act_dev,
                      int act_stride, int lane_count, uint16_t *out_dev, int out_stride);
int igl_gemm_lane_floor(void);

/* quant_step (app_core.c:1930-1940) on `lanes` rows of n floats: rint(x / step)
 * clamped to [-128, 127], times step; a step that is not positive copies.  src
 * may be dst. */
int igl_quant_step_dev(igl_desk *desk, const float *src_dev, int src_stride, float *dst_dev,
                       int dst_stride, int n, int lanes, float step);
/* plane_lift_many (app_core.c:7814-7843), the caller-side wrapper of the
 * table's mat_mat: the lanes on the plane's enter_gain grid before the
 * product (igl_mat_mat_dev's), the outputs on its leave_gain grid after;
 * either step is skipped when its gain is not positive.  The model-wide
 * input rule (quant_act) is not applied. */
int igl_plane_lift_dev(igl_desk *desk, const igl_plane *sheet, const float *act_dev,
                       int act_stride, int lane_count, float *out_dev, int out_stride);

/* Byte formats of the key/value ring. */
typedef enum igl_cache_format { IGL_CACHE_E4M3 = 0, IGL_CACHE_INT8 = 1 } igl_cache_format;

/* Decode attention for one lane: for every key/value head, the `group_share`
 * query heads that read it attend over positions place_start ..
 * place_start + span_count - 1, stored in ring slot p % cache_span, each row
 * kv_count * head_size bytes.  A byte decodes to real8(byte) * scale (e4m3, the
 * reference's cache_real8) or (int8)byte * scale.  Scores are multiplied by
 * `score_scale` (1.0 in the reference graph, whose q/k norms absorb it).
 * query/blend_out: [kv_count * group_share][head_size] fp32.
 * Supported: head_size 256 or 512, group_share 8. */
int igl_attend_dev(igl_desk *desk, const uint8_t *key_store, const uint8_t *value_store,
                   int format, float key_scale, float value_scale, int cache_span,
                   int kv_count, int group_share, int head_size, const float *query_dev,
                   int place_start, int span_count, float score_scale, float *blend_out_dev);
/* The same for `lane_count` lanes at positions place_first .. + lane_count - 1
 * (a prefill chunk or a speculative block), one launch: lane l sees the last
 * `window` positions up to and including its own (0: all from position 0),
 * its query and output `lane_stride` floats after lane l - 1's.  Every lane's
 * keys and values must already be in the ring, which must be deep enough
 * that no lane's visible rows were overwritten by a later lane's. */
int igl_attend_lanes_dev(igl_desk *desk, const uint8_t *key_store, const uint8_t *value_store,
                         int format, float key_scale, float value_scale, int cache_span,
                         int kv_count, int group_share, int head_size, const float *query_dev,
                         int lane_stride, int place_first, int window, int lane_count,
                         float score_scale, float *blend_out_dev);
/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): igl_attend_lanes_dev with the same arguments and results,
 * whose chunk partials live in a fixed array of IGL_ATTEND_FIXED_FLOATS floats
 * (8 MiB) that each GPU holds from the library's load until the process ends,
 * instead of in the desk's grow-only workspace.  It allocates and frees
 * nothing.  A call whose partials exceed the array (at most
 * lane_count * kv_count * group_share * (head_size + 2) * ceil(span / 32)
 * floats, span the longest lane's) is refused with IGL_FAIL_SUPPORT before
 * anything is launched.  Every call on one GPU shares that GPU's array and
 * nothing in it needs to start at zero (each partial is written before it is
 * read); calls that overlap on one GPU (two desks, or two streams) race. */
#define IGL_ATTEND_FIXED_FLOATS (1u << 21)
int igl_attend_lanes_fixed_dev(igl_desk *desk, const uint8_t *key_store,
                               const uint8_t *value_store, int format, float key_scale,
                               float value_scale, int cache_span, int kv_count, int group_share,
                               int head_size, const float *query_dev, int lane_stride,
                               int place_first, int window, int lane_count, float score_scale,
                               float *blend_out_dev);
/* cache_lay (app_core.c:11205-11236) for a byte store: row / scale to the ring
 * at byte offset slot_first. */
int igl_cache_lay_dev(igl_desk *desk, const float *row_dev, int width, float scale, int format,
                      uint8_t *store_dev, size_t slot_first);

int igl_norm_rms_dev(igl_desk *desk, const float *in_dev, const float *gain_dev, int n, int rows,
                     int stride, float eps, float *out_dev);
int igl_soft_max_dev(igl_desk *desk, float *v_dev, int n, int rows, int stride);
int igl_gelu_gate_dev(igl_desk *desk, float *gate_dev, const float *rise_dev, int n);
int igl_rope_turn_dev(igl_desk *desk, float *v_dev, int heads, int head_size, const float *cos_dev,
                      const float *sin_dev);

/* ---- device memory and timing (plumbing) --------------------------------- */

void *igl_dev_alloc(igl_desk *desk, size_t bytes);
void  igl_dev_free(igl_desk *desk, void *ptr);
int   igl_copy_to_dev(igl_desk *desk, void *dst_dev, const void *src_host, size_t bytes);
int   igl_copy_to_host(igl_desk *desk, void *dst_host, const void *src_dev, size_t bytes);
int   igl_fill_dev(igl_desk *desk, void *dst_dev, int byte_value, size_t bytes);
int   igl_sync(igl_desk *desk);
/* Events on the desk's stream around enqueued work: mark, then read the
 * milliseconds between the last two marks after they complete. */
int   igl_mark(igl_desk *desk);
float igl_marks_ms(igl_desk *desk);
/* No counterpart in the reference (a calibration for the benchmark): reads
 * `bytes` (a multiple of 16, 16-byte aligned) of src_dev once with 16-byte
 * loads, two a thread, and keeps nothing.  Its time is the floor of any kernel
 * that must read those bytes once, the yardstick of the GEMV's rate. */
int   igl_read_floor_dev(igl_desk *desk, const void *src_dev, size_t bytes);

/* ---- recording and replay (HIP graphs) ------------------------------------ */

/* No counterpart in the reference; for callers that replay a fixed sequence of
 * device entries (a decode step, a benchmark loop) without paying a host launch
 * for each.  igl_record_begin starts recording the desk's stream: the device
 * entries called until igl_record_end (the *_dev products and lifts,
 * attention, the elementwise *_dev entries) are recorded, not run, and
 * igl_record_end returns them as one replay; igl_replay_run enqueues it.
 * While recording, every entry that touches host memory, synchronizes,
 * allocates or fills (the table entries, copies, igl_sync, marks,
 * igl_fill_dev) is refused with IGL_FAIL_STATE, and igl_record_end then
 * returns that code and no replay.  A replay keeps the addresses it recorded:
 * the buffers and planes it names must outlive it, and while any replay of a
 * desk is alive the desk's scratch cannot grow (a call that would need more
 * room fails with IGL_FAIL_STATE), so call each entry once before recording.
 * Free every replay before igl_back_close. */
typedef struct igl_replay igl_replay;
int  igl_record_begin(igl_desk *desk);
int  igl_record_end(igl_desk *desk, igl_replay **replay_out);
int  igl_replay_run(igl_desk *desk, igl_replay *replay);
void igl_replay_free(igl_desk *desk, igl_replay *replay);

/* ---- synthetic inputs (seeded, shared by the CPU and GPU hosts) ----------- */

/* splitmix64-seeded xoshiro256**; normals by Box-Muller in double. */
typedef struct igl_rng { uint64_t s[4]; } igl_rng;
void     igl_rng_seed(igl_rng *rng, uint64_t seed);
uint64_t igl_rng_next(igl_rng *rng);
void     igl_rng_normal(igl_rng *rng, float *out, size_t count, float mean, float stddev);
/* N rows of K int4 codes uniform in -8..7, stored as value + 8, two a byte,
 * low nibble first, rows `row_stride` bytes apart (row_stride >= K/2). */
void     igl_rng_codes4(igl_rng *rng, uint8_t *codes, int N, int K, size_t row_stride);
/* |N(0, stddev)| gains. */
void     igl_rng_gains(igl_rng *rng, float *gains, size_t count, float stddev);

/* ---- synthetic Gemma 4 E2B-shaped checkpoint ------------------------------ */

/* The text stack's dimensions (model/config.json of the reference's export). */
typedef struct igl_gemma_shape {
  int   vocab, hidden, inner, layers, heads, kv_heads, head_dim, full_head_dim;
  int   window, ple_size, shared_layers, double_wide, full_every, max_positions;
  int   cache_scales;  /* write k/v_cache_scale so a byte cache is used */
  int   kinds;         /* 0: int4 group-32 planes everywhere; 1: the export's own kinds;
                          2: the layer projections in the compressed-tensors pack
                          (I32 weight_packed, weight_shape, weight_zero_point) */
  float norm_eps, logit_cap, rope_local, rope_global, partial_rotary;
} igl_gemma_shape;

/* config.json's dimensions: 35 layers, hidden 1536, FFN 6144 (12288 on the 20
 * key/value-sharing layers), 8 heads, 1 KV head, head 256 / 512, window 512,
 * vocab 262144. */
void igl_gemma_shape_e2b(igl_gemma_shape *shape);
int  igl_gemma_full_layer(const igl_gemma_shape *shape, int layer);
/* Writes config.json, tokenizer.json and model.safetensors (int4 group-32
 * planes in the export's U8 + F32-scale layout) into `folder`, seeded. */
int  igl_gemma_write(const char *folder, const igl_gemma_shape *shape, uint64_t seed);

/* zero_read (app_core.c:7855-7866) over a whole plane: `words` is a
 * weight_zero_point tensor, I32 [ceil(rows * bits / 32)][groups], each group's
 * zero points packed along the rows, low bits first, stored value +
 * 2^(bits-1); `out` receives them as int8 [rows][groups] (the plane's
 * bias_data, as plane_bind_part fills it, 8053-8063). */
void igl_zero_unpack(const uint32_t *words, int groups, int rows, int bits, int8_t *out);

/* ---- a device-resident decode session ------------------------------------- */

/* The reference's session graph (session_pass app_core.c:11843-11975) with
 * activations and the byte key/value cache in HBM: ids in, greedy picks out.
 * Loads config.json + model.safetensors from `folder` (4-bit planes, one KV
 * head per 8 query heads, byte cache scales).  `lane_limit` lanes run per pass
 * (the reference's is 16); `precise` keeps every projection on the fp32
 * activation GEMV, otherwise batches of 64+ lanes take the MFMA GEMM. */
typedef struct igl_engine igl_engine;
int  igl_engine_open(igl_engine **engine_out, igl_desk *desk, const char *folder,
                     int window_limit, int lane_limit, int precise);
void igl_engine_close(igl_engine *engine);
/* session_prime (app_core.c:14469): every id but the last. */
int  igl_engine_prime(igl_engine *engine, const int32_t *ids, int count);
/* session_step + the greedy pick (first maximum, 14672-14677); margin_out
 * receives the gap to the runner-up logit. */
int  igl_engine_step(igl_engine *engine, int32_t id, int32_t *pick_out, float *margin_out);
/* The last pass's logits of `lane` (below min(lane_limit, 64)). */
int  igl_engine_logits(igl_engine *engine, float *out, int lane);
int  igl_engine_fill(const igl_engine *engine);
int  igl_engine_vocab(const igl_engine *engine);
int  igl_engine_reset(igl_engine *engine);
/* Whether decode steps replay one captured HIP graph (on by default): the
 * first step runs as enqueued and is captured; later steps launch the capture,
 * whose kernels read the position and id from device memory. */
int  igl_engine_set_graph(igl_engine *engine, int on);
/* session_guess (app_core.c:12139-12203): one pass over ids[0 .. count) (the
 * next input, then a proposed continuation) with the greedy pick and top-1 /
 * top-2 gap of every lane; the block stays open until igl_engine_keep, and
 * step / prime / guess refuse meanwhile.  count <= min(lane_limit, 64): the
 * logit rows are held for that many lanes (the reference's blocks carry at
 * most 16). */
int  igl_engine_guess(igl_engine *engine, const int32_t *ids, int count, int32_t *picks_out,
                      float *margins_out);
/* session_guess_keep (12207-12223): keep the block's first `keep` lanes. */
int  igl_engine_keep(igl_engine *engine, int keep);

/* The prompt-lookup proposer (the reference's scout, app_core.c:12225-12361):
 * the committed ids in order, and what followed the latest earlier occurrence
 * of the last 3 (else 2) of them. */
typedef struct igl_scout igl_scout;
int  igl_scout_open(igl_scout **scout_out);
void igl_scout_close(igl_scout *scout);
int  igl_scout_note(igl_scout *scout, const int32_t *ids, int count);
int  igl_scout_draw(const igl_scout *scout, int32_t *out, int want);

#ifdef __cplusplus
}
#endif

#endif
