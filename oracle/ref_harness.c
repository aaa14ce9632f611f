/* ref_harness.c - exports the reference engine's own projection, codec and
 * attention functions under a flat C ABI, for the parity tests and the CPU
 * baseline.
 *
 * TEST INFRASTRUCTURE ONLY.  It is built by oracle/Makefile straight from the
 * reference's single translation unit where it lies (app_core.c, included
 * below through -I), into oracle/_ref/, which git ignores.  No reference source
 * is copied into this repository; nothing in igllm_amd/ links this.
 *
 * Three builds are made: a plain one (SSE2 tier, the float path the oracle
 * restates to the bit), a tuned one (-mavx2 -mfma, the reference's fastest
 * float path on x86, used as the CPU baseline), and a level one
 * (REF_LEVEL_TIER: AVX-512 VNNI), whose products take the integer grid: the
 * calibrated-plane path oracle_mat_mat_level restates.  The float builds
 * refuse the VNNI tier, whose uncalibrated products round activations.
 */
#include "app_core.c"

#if defined(APP_SIMD_AVX512VNNI) && !defined(REF_LEVEL_TIER)
#  error "the float builds of the harness must not take the integer-grid tier"
#endif

/* Flat description of a code plane; the fields of `plane` (app_core.c:1775)
 * a code plane uses, gains fp32. */
typedef struct ref_plane_desc {
  int            row_count;
  int            col_count;
  const uint8_t *code_data;
  size_t         row_stride;
  const float   *gain_data;
  const int8_t  *bias_data;
  int            bit_count;
  int            code_bias;
  int            code_flip;
  int            group_size;
  int            group_count;
} ref_plane_desc;

static void ref_plane_fill(const ref_plane_desc *desc, plane *sheet) {
  memset(sheet, 0, sizeof(*sheet));
  sheet->form = PLANE_CODE;
  sheet->row_count = desc->row_count;
  sheet->col_count = desc->col_count;
  sheet->code_data = desc->code_data;
  sheet->row_stride = desc->row_stride;
  sheet->gain_data = desc->gain_data;
  sheet->gain_type = STORE_F32;
  sheet->bias_data = desc->bias_data;
  sheet->bit_count = desc->bit_count;
  sheet->code_bias = desc->code_bias;
  sheet->code_flip = desc->code_flip;
  sheet->group_size = desc->group_size;
  sheet->group_count = desc->group_count;
}

const char *ref_flavor(void) { return back_flavor(); }

uint32_t ref_pack_read(const uint8_t *code_data, size_t element_index, int bit_count) {
  return pack_read(code_data, element_index, bit_count);
}

/* zero_read (app_core.c:7855-7866): a row's zero point in a weight_zero_point
 * tensor packed along rows. */
int ref_zero_read(const uint32_t *word_list, int group_count, int group_index, int row_index,
                  int bit_count) {
  return zero_read(word_list, group_count, group_index, row_index, bit_count);
}

void ref_plane_row(const ref_plane_desc *desc, int row_index, float *row_out) {
  plane sheet;
  ref_plane_fill(desc, &sheet);
  plane_row(&sheet, row_index, row_out);
}

/* A desk and its pool, held open so the CPU baseline times products and not
 * thread creation. */
typedef struct ref_desk {
  back_desk  desk;
  pool_group pool;
} ref_desk;

void *ref_desk_open(int thread_count, int sum_limit, int col_limit) {
  ref_desk *box = (ref_desk *)calloc(1, sizeof(ref_desk));
  if (!box) return NULL;
  if (pool_open(&box->pool, thread_count) != APP_OKAY ||
      back_open(&box->desk, &box->pool, sum_limit, col_limit) != APP_OKAY) {
    free(box);
    return NULL;
  }
  return box;
}

void ref_desk_close(void *handle) {
  ref_desk *box = (ref_desk *)handle;
  if (!box) return;
  back_close(&box->desk);
  pool_close(&box->pool);
  free(box);
}

void ref_desk_mat_mat(void *handle, const ref_plane_desc *desc, const float *act, int act_stride,
                      int lane_count, float *out, int out_stride) {
  ref_desk *box = (ref_desk *)handle;
  plane sheet;
  ref_plane_fill(desc, &sheet);
  box->desk.mat_mat(&box->desk, &sheet, act, act_stride, lane_count, out, out_stride);
}

/* The desk entry on a calibrated plane (enter_gain = step): on the level
 * build (REF_LEVEL_TIER, AVX-512 VNNI) a chunk whose values all sit on the
 * step's grid takes the integer level path (back_mat_mat 5283-5306). */
void ref_desk_mat_mat_step(void *handle, const ref_plane_desc *desc, float step, const float *act,
                           int act_stride, int lane_count, float *out, int out_stride) {
  ref_desk *box = (ref_desk *)handle;
  plane sheet;
  ref_plane_fill(desc, &sheet);
  sheet.enter_gain = step;
  box->desk.mat_mat(&box->desk, &sheet, act, act_stride, lane_count, out, out_stride);
}

int ref_level_live(void *handle) { return ((ref_desk *)handle)->desk.level_live; }

/* The same desk entry on a real plane: `real_type` is the reference's
 * store_type (STORE_F32, STORE_F16, STORE_BF16). */
void ref_desk_mat_mat_real(void *handle, const void *real_data, int real_type, int row_count,
                           int col_count, const float *act, int act_stride, int lane_count,
                           float *out, int out_stride) {
  ref_desk *box = (ref_desk *)handle;
  plane sheet;
  memset(&sheet, 0, sizeof(sheet));
  sheet.form = PLANE_REAL;
  sheet.row_count = row_count;
  sheet.col_count = col_count;
  sheet.real_data = real_data;
  sheet.real_type = (store_type)real_type;
  box->desk.mat_mat(&box->desk, &sheet, act, act_stride, lane_count, out, out_stride);
}

float ref_cache_pack8(float value) { return cache_pack8(value); }
uint8_t ref_cache_code8(float value) { return cache_code8(value); }
float ref_cache_real8(uint8_t code) { return cache_real8(code); }
void ref_cache_grid_fill(float *grid, float scale) { cache_grid_fill(grid, scale); }
float ref_exp_near(float value) { return kern_exp_near(value); }
void ref_soft_max(float *value_list, int value_count) { kern_soft_max(value_list, value_count); }
float ref_quant_step(float value, float step) {
  quant_step(&value, 1, step);
  return value;
}

static int32_t ref_top(const float *logits, int vocab) {
  int32_t best = 0;
  for (int v = 1; v < vocab; ++v)
    if (logits[v] > logits[best]) best = v;
  return best;
}

/* The reference engine end to end: load the checkpoint in `folder`, prime the
 * prompt (all but its last id, app_core.c:14443-14471), then step and take the
 * greedy pick `gen_count` times, the way the CLI's answer loop does
 * (app_main.c:600-611) but without stopping at the close id.  The pick is the
 * first maximum (session_pick_at, app_core.c:14672-14677).  `margin_out`, when
 * given, receives each step's gap between the best and second-best logit.
 * Returns 0 or the app_code that stopped it. */
int ref_engine_greedy(const char *folder, int thread_count, int cache_bits, int window_limit,
                      const int32_t *prompt, int prompt_count, int gen_count, int32_t *out_ids,
                      float *margin_out) {
  app_setup setup = app_setup_plain();
  app_model *model = NULL;
  app_session *session = NULL;
  app_code code;
  int32_t id;
  setup.thread_count = thread_count;
  setup.cache_bits = cache_bits;
  setup.window_limit = window_limit;
  code = model_load(folder, &setup, &model);
  if (code != APP_OKAY) return (int)code;
  code = session_open(model, &session);
  if (code != APP_OKAY) {
    model_free(model);
    return (int)code;
  }
  code = session_prime(session, prompt, prompt_count);
  id = prompt[prompt_count - 1];
  for (int step = 0; code == APP_OKAY && step < gen_count; ++step) {
    const float *logits = session_step(session, id);
    int vocab = model_vocab_count(model);
    int best = 0;
    float second = -FLT_MAX;
    if (!logits) {
      code = APP_FAIL_STATE;
      break;
    }
    for (int v = 1; v < vocab; ++v)
      if (logits[v] > logits[best]) best = v;
    for (int v = 0; v < vocab; ++v)
      if (v != best && logits[v] > second) second = logits[v];
    out_ids[step] = best;
    if (margin_out) margin_out[step] = logits[best] - second;
    id = best;
  }
  session_close(session);
  model_free(model);
  return (int)code;
}

/* The greedy run of ref_engine_greedy, keeping the whole row of logits at
 * each of `probe_count` steps (ascending step indices in `probe_steps`) in
 * `rows_out` [probe_count][vocab].  Returns 0 or the app_code that stopped it. */
int ref_engine_probe(const char *folder, int thread_count, int cache_bits, int window_limit,
                     const int32_t *prompt, int prompt_count, int gen_count, const int32_t *probe_steps,
                     int probe_count, int32_t *out_ids, float *rows_out) {
  app_setup setup = app_setup_plain();
  app_model *model = NULL;
  app_session *session = NULL;
  app_code code;
  int32_t id;
  int next_probe = 0;
  setup.thread_count = thread_count;
  setup.cache_bits = cache_bits;
  setup.window_limit = window_limit;
  code = model_load(folder, &setup, &model);
  if (code != APP_OKAY) return (int)code;
  code = session_open(model, &session);
  if (code != APP_OKAY) {
    model_free(model);
    return (int)code;
  }
  code = session_prime(session, prompt, prompt_count);
  id = prompt[prompt_count - 1];
  for (int step = 0; code == APP_OKAY && step < gen_count; ++step) {
    const float *logits = session_step(session, id);
    const int vocab = model_vocab_count(model);
    if (!logits) {
      code = APP_FAIL_STATE;
      break;
    }
    if (next_probe < probe_count && probe_steps[next_probe] == step) {
      memcpy(rows_out + (size_t)next_probe * (size_t)vocab, logits, sizeof(float) * (size_t)vocab);
      ++next_probe;
    }
    out_ids[step] = ref_top(logits, vocab);
    id = out_ids[step];
  }
  session_close(session);
  model_free(model);
  return (int)code;
}

/* The reference engine's own timing of a bounded run: prime `prompt`, then
 * `gen_count` greedy steps; the wall seconds of each phase (the CPU baseline of
 * the end-to-end decode).  Returns 0 or the app_code that stopped it. */
int ref_engine_clock(const char *folder, int thread_count, int cache_bits, int window_limit,
                     const int32_t *prompt, int prompt_count, int gen_count, double *prime_s,
                     double *step_s) {
  app_setup setup = app_setup_plain();
  app_model *model = NULL;
  app_session *session = NULL;
  app_code code;
  struct timespec t0, t1, t2;
  int32_t id;
  setup.thread_count = thread_count;
  setup.cache_bits = cache_bits;
  setup.window_limit = window_limit;
  code = model_load(folder, &setup, &model);
  if (code != APP_OKAY) return (int)code;
  code = session_open(model, &session);
  if (code != APP_OKAY) {
    model_free(model);
    return (int)code;
  }
  clock_gettime(CLOCK_MONOTONIC, &t0);
  code = session_prime(session, prompt, prompt_count);
  clock_gettime(CLOCK_MONOTONIC, &t1);
  id = prompt[prompt_count - 1];
  for (int step = 0; code == APP_OKAY && step < gen_count; ++step) {
    const float *logits = session_step(session, id);
    int vocab = model_vocab_count(model), best = 0;
    if (!logits) {
      code = APP_FAIL_STATE;
      break;
    }
    for (int v = 1; v < vocab; ++v)
      if (logits[v] > logits[best]) best = v;
    id = best;
  }
  clock_gettime(CLOCK_MONOTONIC, &t2);
  *prime_s = (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
  *step_s = (double)(t2.tv_sec - t1.tv_sec) + 1e-9 * (double)(t2.tv_nsec - t1.tv_nsec);
  session_close(session);
  model_free(model);
  return (int)code;
}

/* The same, but the step inputs are `forced` (not the picks): each step's
 * pick and margin against a given token sequence, so a stream that a random
 * model would collapse onto one id still walks many inputs. */
int ref_engine_forced(const char *folder, int thread_count, int cache_bits, int window_limit,
                      const int32_t *prompt, int prompt_count, const int32_t *forced, int gen_count,
                      int32_t *out_ids, float *margin_out) {
  app_setup setup = app_setup_plain();
  app_model *model = NULL;
  app_session *session = NULL;
  app_code code;
  setup.thread_count = thread_count;
  setup.cache_bits = cache_bits;
  setup.window_limit = window_limit;
  code = model_load(folder, &setup, &model);
  if (code != APP_OKAY) return (int)code;
  code = session_open(model, &session);
  if (code != APP_OKAY) {
    model_free(model);
    return (int)code;
  }
  code = session_prime(session, prompt, prompt_count);
  for (int step = 0; code == APP_OKAY && step < gen_count; ++step) {
    const float *logits = session_step(session, step == 0 ? prompt[prompt_count - 1] : forced[step - 1]);
    int vocab = model_vocab_count(model);
    int best = 0;
    float second = -FLT_MAX;
    if (!logits) {
      code = APP_FAIL_STATE;
      break;
    }
    for (int v = 1; v < vocab; ++v)
      if (logits[v] > logits[best]) best = v;
    for (int v = 0; v < vocab; ++v)
      if (v != best && logits[v] > second) second = logits[v];
    out_ids[step] = best;
    margin_out[step] = logits[best] - second;
  }
  session_close(session);
  model_free(model);
  return (int)code;
}

/* The CLI's greedy --guess loop (main_answer_guess, app_main.c:520-598) on
 * the reference engine, without the stop-id check: the scout proposes up to
 * span - 1 ids (scout_draw), session_guess runs the block, the argmax rows
 * keep the agreed prefix plus the next id, session_guess_keep commits them;
 * with nothing proposed, an ordinary step.  stats_out: rounds, ids proposed,
 * ids taken. */
int ref_engine_guess(const char *folder, int thread_count, int cache_bits, int window_limit,
                     const int32_t *prompt, int prompt_count, int gen_count, int span,
                     int32_t *out_ids, long *stats_out) {
  app_setup setup = app_setup_plain();
  app_model *model = NULL;
  app_session *session = NULL;
  app_scout *scout = NULL;
  app_code code;
  int32_t block[16];
  int32_t id_value;
  int made = 0, vocab;
  long rounds = 0, drawn = 0, taken = 0;
  setup.thread_count = thread_count;
  setup.cache_bits = cache_bits;
  setup.window_limit = window_limit;
  code = model_load(folder, &setup, &model);
  if (code != APP_OKAY) return (int)code;
  code = session_open(model, &session);
  if (code == APP_OKAY) code = scout_open(&scout);
  if (code == APP_OKAY) code = session_prime(session, prompt, prompt_count);
  if (code == APP_OKAY) code = scout_note(scout, prompt, prompt_count);
  vocab = model_vocab_count(model);
  if (span > session_guess_limit(session)) span = session_guess_limit(session);
  if (span < 1) span = 1;
  id_value = prompt[prompt_count - 1];
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
      if (!logits) { code = APP_FAIL_STATE; break; }
      id_value = ref_top(logits, vocab);
      out_ids[made++] = id_value;
      code = scout_note(scout, &id_value, 1);
      continue;
    }
    rows = session_guess(session, block, count);
    if (!rows) { code = APP_FAIL_STATE; break; }
    drawn += count - 1;
    while (take + 1 < count && ref_top(rows + (size_t)take * vocab, vocab) == block[take + 1]) take += 1;
    after = ref_top(rows + (size_t)take * vocab, vocab);
    taken += take;
    for (int slot = 0; slot <= take && made < gen_count; ++slot) {
      id_value = slot < take ? block[slot + 1] : after;
      out_ids[made++] = id_value;
      if (scout_note(scout, &id_value, 1) != APP_OKAY) code = APP_FAIL_MEMORY;
    }
    if (code == APP_OKAY) code = session_guess_keep(session, take + 1);
  }
  if (stats_out) {
    stats_out[0] = rounds;
    stats_out[1] = drawn;
    stats_out[2] = taken;
  }
  if (scout) scout_close(scout);
  if (session) session_close(session);
  model_free(model);
  return (int)code;
}

/* Fixed speculative blocks after a prompt: block b is ids[first .. first +
 * counts[b]) (first the sum of the earlier counts), run by session_guess
 * (app_core.c:12139-12203) with every lane's pick (first maximum) and
 * top-1/top-2 gap recorded, then session_guess_keep (12205-12223) of keeps[b]
 * lanes.  Multi-lane blocks over inputs a random model's greedy stream never
 * takes. */
int ref_engine_blocks(const char *folder, int thread_count, int cache_bits, int window_limit,
                      const int32_t *prompt, int prompt_count, const int32_t *ids, const int *counts,
                      const int *keeps, int block_count, int32_t *picks_out, float *margins_out) {
  app_setup setup = app_setup_plain();
  app_model *model = NULL;
  app_session *session = NULL;
  app_code code;
  int first = 0, vocab;
  setup.thread_count = thread_count;
  setup.cache_bits = cache_bits;
  setup.window_limit = window_limit;
  code = model_load(folder, &setup, &model);
  if (code != APP_OKAY) return (int)code;
  code = session_open(model, &session);
  if (code == APP_OKAY) code = session_prime(session, prompt, prompt_count);
  vocab = model_vocab_count(model);
  for (int b = 0; code == APP_OKAY && b < block_count; ++b) {
    const float *rows = session_guess(session, ids + first, counts[b]);
    if (!rows) {
      code = APP_FAIL_STATE;
      break;
    }
    for (int l = 0; l < counts[b]; ++l) {
      const float *logits = rows + (size_t)l * (size_t)vocab;
      int best = ref_top(logits, vocab);
      float second = -FLT_MAX;
      for (int v = 0; v < vocab; ++v)
        if (v != best && logits[v] > second) second = logits[v];
      picks_out[first + l] = best;
      margins_out[first + l] = logits[best] - second;
    }
    code = session_guess_keep(session, keeps[b]);
    first += counts[b];
  }
  if (session) session_close(session);
  model_free(model);
  return (int)code;
}

/* One lane's grouped decode attention through the reference's own two jobs
 * (attend_score_band / attend_blend_band, app_core.c:11296-11365), forked over
 * the desk's pool exactly as session_attend_group forks them (11415-11453).
 * Only the session and model fields those jobs read are set. */
void ref_attend(void *handle, const uint8_t *key_store, const uint8_t *value_store,
                const float *key_grid, const float *value_grid, int cache_span, int kv_width,
                int kv_index, const float *query, int head_first, int group_share, int head_size,
                int place_start, int span_count, float *blend_out) {
  ref_desk *box = (ref_desk *)handle;
  app_model *model = (app_model *)calloc(1, sizeof(app_model));
  app_session *session = (app_session *)calloc(1, sizeof(app_session));
  int bands = pool_bands(&box->pool);
  attend_job job;
  if (!model || !session) {
    free(model);
    free(session);
    return;
  }
  model->desk = box->desk;
  session->model = model;
  session->score_stride = span_count;
  session->block_room = cache_block_rows(head_size) * head_size;
  session->score_room = (float *)calloc((size_t)group_share * (size_t)span_count, sizeof(float));
  session->cache_room = (float *)calloc((size_t)bands * (size_t)session->block_room, sizeof(float));
  memset(&job, 0, sizeof(job));
  job.session = session;
  job.key_store = key_store;
  job.value_store = value_store;
  job.key_grid = key_grid;
  job.value_grid = value_grid;
  job.query_lane = query;
  job.blend_lane = blend_out;
  job.cache_span = cache_span;
  job.place_start = place_start;
  job.span_count = span_count;
  job.block_rows = cache_block_rows(head_size);
  job.block_room = session->block_room;
  job.kv_index = kv_index;
  job.head_first = head_first;
  job.group_share = group_share;
  job.head_size = head_size;
  job.kv_width = kv_width;
  if (box->pool.worker_count > 0 && span_count >= ATTEND_BAND_SPAN) {
    pool_run(&box->pool, attend_score_band, &job);
    pool_run(&box->pool, attend_blend_band, &job);
  } else {
    attend_score_band(&job, 0, 1);
    attend_blend_band(&job, 0, 1);
  }
  free(session->score_room);
  free(session->cache_room);
  free(session);
  free(model);
}
