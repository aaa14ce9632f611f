/* dropin_harness.c - the reference engine itself, with its backend table
 * pointed at the gfx950 backend: the drop-in as a maintainer would make it.
 *
 * TEST INFRASTRUCTURE ONLY.  Built by oracle/Makefile from the reference's own
 * app_core.c where it lies (included below through -I) and linked against the
 * product library igllm_amd/libigl_hip.so, into oracle/_ref/ (git-ignored).
 * Here the reference is the caller and the product is the callee: the
 * reference loads the checkpoint (model_load, its safetensors mmap and plane
 * binding), opens its session, primes and steps exactly as its CLI does, and
 * every call it makes through `model->desk` (app_core.c:5223-5245) lands in
 * an igl_desk.  The reference's own attention, cache codec, embedding rows,
 * residual arithmetic and sampler stay on the host, untouched, as the table
 * boundary leaves them (app_core.c:11296-11365, 11205, 11870).
 *
 * What the shim does, beyond forwarding:
 *   - at load, every plane of the text stack is copied to the device once
 *     (igl_plane_attach) and recorded in a side table keyed by the reference's
 *     plane address (the planes live inside the model and never move);
 *   - a product on a plane the load-time walk did not attach is counted as a
 *     miss and fails the run, so the walk is shown to cover what the session
 *     multiplies;
 *   - the backend's sticky error is read after the prime and after each step
 *     (the table's entries return void, app_core.c:5236-5244).
 */
#include "app_core.c"

#include "igl_backend.h"

#if defined(APP_SIMD_AVX512VNNI)
#  error "the drop-in harness is built on the float tier"
#endif

typedef struct dropin_slot {
  const plane *key;
  igl_plane    gpu;
} dropin_slot;

/* One drop-in at a time per process (the harness's own state). */
static struct {
  igl_desk     gpu;
  dropin_slot *slot;
  int          slot_count, slot_room;
  long         calls[6];  /* mat_vec, mat_mat, norm_rms, soft_max, gelu_gate, rope_turn */
  long         misses;
} dropin;

static igl_plane *dropin_find(const plane *sheet) {
  for (int i = 0; i < dropin.slot_count; ++i)
    if (dropin.slot[i].key == sheet) return &dropin.slot[i].gpu;
  return NULL;
}

/* The reference's plane and igl_plane carry the same fields in the same
 * order; igl_plane adds the device handle. */
static int dropin_attach(const plane *sheet) {
  igl_plane *p;
  int code;
  if (sheet->form == PLANE_VOID || dropin_find(sheet)) return IGL_OKAY;
  if (dropin.slot_count == dropin.slot_room) {
    int room = dropin.slot_room ? 2 * dropin.slot_room : 64;
    dropin_slot *grown = (dropin_slot *)realloc(dropin.slot, (size_t)room * sizeof(*grown));
    if (!grown) return IGL_FAIL_MEMORY;
    dropin.slot = grown;
    dropin.slot_room = room;
  }
  p = &dropin.slot[dropin.slot_count].gpu;
  memset(p, 0, sizeof(*p));
  p->form = (int)sheet->form;
  p->row_count = sheet->row_count;
  p->col_count = sheet->col_count;
  p->real_data = sheet->real_data;
  p->real_type = (int)sheet->real_type;
  p->code_data = sheet->code_data;
  p->row_stride = sheet->row_stride;
  p->gain_data = sheet->gain_data;
  p->gain_type = (int)sheet->gain_type;
  p->bias_data = sheet->bias_data;
  p->bit_count = sheet->bit_count;
  p->code_bias = sheet->code_bias;
  p->code_flip = sheet->code_flip;
  p->group_size = sheet->group_size;
  p->group_count = sheet->group_count;
  p->enter_gain = sheet->enter_gain;
  p->leave_gain = sheet->leave_gain;
  if ((code = igl_plane_attach(&dropin.gpu, p)) != IGL_OKAY) return code;
  dropin.slot[dropin.slot_count].key = sheet;
  dropin.slot_count++;
  return IGL_OKAY;
}

/* ---- the six entries, forwarded --------------------------------------- */

static void fwd_mat_mat(back_desk *desk, const plane *sheet, const float *act_data, int act_stride,
                        int lane_count, float *out_data, int out_stride) {
  igl_plane *p = dropin_find(sheet);
  (void)desk;
  dropin.calls[1]++;
  if (!p) {
    dropin.misses++;
    return;
  }
  dropin.gpu.mat_mat(&dropin.gpu, p, act_data, act_stride, lane_count, out_data, out_stride);
}

static void fwd_mat_vec(back_desk *desk, const plane *sheet, const float *act_data,
                        float *out_data) {
  igl_plane *p = dropin_find(sheet);
  (void)desk;
  dropin.calls[0]++;
  if (!p) {
    dropin.misses++;
    return;
  }
  dropin.gpu.mat_vec(&dropin.gpu, p, act_data, out_data);
}

static void fwd_norm_rms(back_desk *desk, const float *value_list, const float *gain_list,
                         int value_count, float eps_value, float *value_out) {
  (void)desk;
  dropin.calls[2]++;
  dropin.gpu.norm_rms(&dropin.gpu, value_list, gain_list, value_count, eps_value, value_out);
}

/* Called from every pool worker at once (attend_blend_band): the counter is
 * only a tally, the backend entry serializes itself. */
static void fwd_soft_max(back_desk *desk, float *value_list, int value_count) {
  (void)desk;
  __atomic_fetch_add(&dropin.calls[3], 1, __ATOMIC_RELAXED);
  dropin.gpu.soft_max(&dropin.gpu, value_list, value_count);
}

static void fwd_gelu_gate(back_desk *desk, float *gate_list, const float *rise_list,
                          int value_count) {
  (void)desk;
  dropin.calls[4]++;
  dropin.gpu.gelu_gate(&dropin.gpu, gate_list, rise_list, value_count);
}

static void fwd_rope_turn(back_desk *desk, float *value_list, int head_size, const float *cos_list,
                          const float *sin_list) {
  (void)desk;
  dropin.calls[5]++;
  dropin.gpu.rope_turn(&dropin.gpu, value_list, head_size, cos_list, sin_list);
}

/* The text stack's planes (the walk model_load makes to size the desk,
 * app_core.c:12524-12548), attached once. */
static int dropin_attach_model(app_model *model) {
  int code;
  if ((code = dropin_attach(&model->embed_sheet)) != IGL_OKAY ||
      (code = dropin_attach(&model->head_sheet)) != IGL_OKAY ||
      (code = dropin_attach(&model->ple_lift_sheet)) != IGL_OKAY)
    return code;
  for (int li = 0; li < model->form.layer_count; ++li) {
    layer_wing *w = &model->wing_list[li];
    const plane *list[] = {&w->query_sheet, &w->key_sheet,      &w->value_sheet,
                           &w->exit_sheet,  &w->gate_sheet,     &w->rise_sheet,
                           &w->drop_sheet,  &w->ple_gate_sheet, &w->ple_lift_sheet};
    for (size_t i = 0; i < sizeof(list) / sizeof(list[0]); ++i)
      if ((code = dropin_attach(list[i])) != IGL_OKAY) return code;
  }
  return IGL_OKAY;
}

static void dropin_release(void) {
  for (int i = 0; i < dropin.slot_count; ++i) igl_plane_detach(&dropin.gpu, &dropin.slot[i].gpu);
  free(dropin.slot);
  dropin.slot = NULL;
  dropin.slot_count = dropin.slot_room = 0;
  igl_back_close(&dropin.gpu);
}

/* Loads the checkpoint with the reference's own model_load, opens the GPU
 * desk sized as back_open sizes the CPU one (app_core.c:12585; 16 lanes, the
 * session's batch, KERN_LANE_LIMIT), attaches the text stack, points the
 * model's table at the forwarders and opens the reference's session. */
static int dropin_open(const char *folder, int device, int thread_count, int cache_bits, int window_limit,
                       app_model **model_out, app_session **session_out) {
  app_setup setup = app_setup_plain();
  app_model *model = NULL;
  int code;
  memset(&dropin, 0, sizeof(dropin));
  *model_out = NULL;
  *session_out = NULL;
  setup.thread_count = thread_count;
  setup.cache_bits = cache_bits;
  setup.window_limit = window_limit;
  code = (int)model_load(folder, &setup, &model);
  if (code != APP_OKAY) return code;
  *model_out = model;
  code = igl_back_open(&dropin.gpu, device, model->desk.sum_limit, 65536, KERN_LANE_LIMIT);
  if (code == IGL_OKAY) code = dropin_attach_model(model);
  if (code != IGL_OKAY) return code;
  model->desk.name_text = dropin.gpu.name_text;
  model->desk.mat_vec = fwd_mat_vec;
  model->desk.mat_mat = fwd_mat_mat;
  model->desk.norm_rms = fwd_norm_rms;
  model->desk.soft_max = fwd_soft_max;
  model->desk.gelu_gate = fwd_gelu_gate;
  model->desk.rope_turn = fwd_rope_turn;
  return (int)session_open(model, session_out);
}

/* The backend's sticky error, then any product on a plane the load did not
 * attach. */
static int dropin_check(void) {
  int code = igl_desk_error_take(&dropin.gpu);
  if (code == IGL_OKAY && dropin.misses) code = IGL_FAIL_STATE;
  return code;
}

static void dropin_close(app_model *model, app_session *session, long *calls_out) {
  if (calls_out) {
    for (int i = 0; i < 6; ++i) calls_out[i] = dropin.calls[i];
    calls_out[6] = dropin.misses;
  }
  if (session) session_close(session);
  dropin_release();
  model_free(model);
}

/* The first maximum of a row (session_pick_at's greedy rule,
 * app_core.c:14672-14677) and its gap to the runner-up. */
static int32_t dropin_top(const float *logits, int vocab, float *gap_out) {
  int best = 0;
  float second = -FLT_MAX;
  for (int v = 1; v < vocab; ++v)
    if (logits[v] > logits[best]) best = v;
  for (int v = 0; v < vocab; ++v)
    if (v != best && logits[v] > second) second = logits[v];
  if (gap_out) *gap_out = logits[best] - second;
  return best;
}

/* The reference engine's greedy run (its prime, then `gen_count` steps with
 * the first-maximum pick) with the backend table on device `device`.
 * calls_out[0..5]: the entries' call counts; calls_out[6]: products on planes
 * the load did not attach.  Returns 0, the reference's app_code, or the
 * backend's igl_code. */
int dropin_engine_greedy(const char *folder, int device, int thread_count, int cache_bits,
                         int window_limit, const int32_t *prompt, int prompt_count, int gen_count,
                         int32_t *out_ids, float *margin_out, long *calls_out) {
  app_model *model = NULL;
  app_session *session = NULL;
  int32_t id;
  int code = dropin_open(folder, device, thread_count, cache_bits, window_limit, &model, &session);
  if (code == APP_OKAY) code = (int)session_prime(session, prompt, prompt_count);
  if (code == APP_OKAY) code = dropin_check();
  id = prompt[prompt_count - 1];
  for (int step = 0; code == APP_OKAY && step < gen_count; ++step) {
    const float *logits = session_step(session, id);
    if (!logits) {
      code = APP_FAIL_STATE;
      break;
    }
    if ((code = dropin_check()) != IGL_OKAY) break;
    id = dropin_top(logits, model_vocab_count(model), margin_out ? margin_out + step : NULL);
    out_ids[step] = id;
  }
  dropin_close(model, session, calls_out);
  return code;
}

/* The CLI's greedy --guess loop (main_answer_guess, app_main.c:520-598,
 * without the stop-id check) on the reference engine with the backend table
 * on the GPU: the reference's scout proposes up to span - 1 ids
 * (scout_draw), its session_guess runs the block (a batch of up to `span`
 * lanes through the table's mat_mat), the argmax rows keep the agreed prefix
 * plus the next id, session_guess_keep commits them; with nothing proposed,
 * an ordinary step.  stats_out: rounds, ids proposed, ids taken. */
int dropin_engine_guess(const char *folder, int device, int thread_count, int cache_bits, int window_limit,
                        const int32_t *prompt, int prompt_count, int gen_count, int span, int32_t *out_ids,
                        long *stats_out, long *calls_out) {
  app_model *model = NULL;
  app_session *session = NULL;
  app_scout *scout = NULL;
  int32_t block[16];
  int32_t id_value = prompt[prompt_count - 1];
  int made = 0, vocab = 0;
  long rounds = 0, drawn = 0, taken = 0;
  int code = dropin_open(folder, device, thread_count, cache_bits, window_limit, &model, &session);
  if (code == APP_OKAY) code = (int)scout_open(&scout);
  if (code == APP_OKAY) code = (int)session_prime(session, prompt, prompt_count);
  if (code == APP_OKAY) code = dropin_check();
  if (code == APP_OKAY) code = (int)scout_note(scout, prompt, prompt_count);
  if (code == APP_OKAY) {
    vocab = model_vocab_count(model);
    if (span > session_guess_limit(session)) span = session_guess_limit(session);
    if (span > 16) span = 16;
    if (span < 1) span = 1;
  }
  while (code == APP_OKAY && made < gen_count) {
    int want = span - 1, count, take = 0;
    const float *rows;
    int32_t after;
    if (want > gen_count - made - 1) want = gen_count - made - 1;
    if (want < 0) want = 0;
    block[0] = id_value;
    count = 1 + scout_draw(scout, block + 1, want);
    rounds += 1;
    if (count == 1) {
      const float *logits = session_step(session, id_value);
      if (!logits) {
        code = APP_FAIL_STATE;
        break;
      }
      if ((code = dropin_check()) != IGL_OKAY) break;
      id_value = dropin_top(logits, vocab, NULL);
      out_ids[made++] = id_value;
      code = (int)scout_note(scout, &id_value, 1);
      continue;
    }
    rows = session_guess(session, block, count);
    if (!rows) {
      code = APP_FAIL_STATE;
      break;
    }
    if ((code = dropin_check()) != IGL_OKAY) break;
    drawn += count - 1;
    while (take + 1 < count && dropin_top(rows + (size_t)take * (size_t)vocab, vocab, NULL) == block[take + 1])
      take += 1;
    after = dropin_top(rows + (size_t)take * (size_t)vocab, vocab, NULL);
    taken += take;
    for (int slot = 0; slot <= take && made < gen_count; ++slot) {
      id_value = slot < take ? block[slot + 1] : after;
      out_ids[made++] = id_value;
      if (scout_note(scout, &id_value, 1) != APP_OKAY) code = APP_FAIL_MEMORY;
    }
    if (code == APP_OKAY) code = (int)session_guess_keep(session, take + 1);
  }
  if (stats_out) {
    stats_out[0] = rounds;
    stats_out[1] = drawn;
    stats_out[2] = taken;
  }
  if (scout) scout_close(scout);
  dropin_close(model, session, calls_out);
  return code;
}
