/* igl_engine.c - a device-resident decode session for the Gemma 4 text stack
 * on this backend.
 *
 * It restates the reference's session graph (session_pass app_core.c:11843-
 * 11975, session_layer 11637-11743, session_attend 11455-11580) with every
 * activation and the key/value cache held in HBM, so a decode step crosses
 * the host boundary twice: the token id in, the greedy pick out.  The weights
 * are the checkpoint's payload copied to the device unchanged; every plane is
 * a view into that copy (the reference's plane_bind_gemma layout, 7886-7955).
 *
 * What it reads: config.json (the text_config fields config_read reads,
 * 8325-8475) and model.safetensors (U8 code planes with F32 group scales, F32
 * norm gains and scalars).  What it supports is what the kernels take: 4-bit
 * planes, one key/value head per 8 query heads, heads of 256 or 512, a byte
 * key/value cache (every owning layer ships k/v_cache_scale).  Anything else is
 * refused at open with IGL_FAIL_SUPPORT.
 *
 * Differences of arrangement, none of arithmetic: a batch of lanes writes all
 * its keys and values before any of them attends (the reference interleaves
 * lane by lane, 11481-11483), so a sliding layer's ring is `window + lanes`
 * rows deep instead of `window`, which keeps every row a lane can see; the
 * attention and norms reduce in their own order.
 */
#define _POSIX_C_SOURCE 200809L
#include <ctype.h>
#include <fcntl.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <hip/hip_runtime_api.h>

#include "igl_backend.h"
#include "igl_launch.h"

#define ENG_LAYER_LIMIT 128
/* Lanes a speculative block may carry: the only pass that takes logits on
 * more than one lane (a prime takes none), so the 262144-wide logit rows are
 * sized by this and not by the prime's lane limit.  The reference's blocks
 * carry at most KERN_LANE_LIMIT = 16 (app_core.c:1980). */
#define ENG_GUESS_LIMIT 64
/* lanes a pass runs with the prepared attention (a decode step, a small
 * speculative block) */
#define ENG_SMALL_LANES 4
/* lanes a pass runs with the grouped projections, one row of workgroups a
 * lane (blocks of 5, 6 and 8 lanes: 3.12 / 3.16 / 3.31 -> 2.54 / 2.69 / 3.04
 * ms against separate projections and updates) */
#define ENG_GROUP_LANES 8
#define ENG_TENSOR_LIMIT 4096

typedef struct eng_tensor {
  char      name[160];
  int       dtype;     /* 0 U8, 1 F32, 2 I8, 3 BF16, 4 I32, -1 other */
  int       rank;
  long long shape[3];
  size_t    begin, end;
} eng_tensor;

/* Host side of a decode step, in pinned memory so a captured graph's copies
 * read and write it at every replay. */
typedef struct igl_step_io {
  int32_t place, id;   /* copied to ctl_dev[0..1] */
  int32_t pick;        /* copied back from pick_dev[0..1] */
  float margin;
} igl_step_io;

typedef struct eng_layer {
  int full, shared, source, keep, head_size, inner, cache_span;
  igl_plane q, k, v, o, gate, up, down, ple_gate, ple_proj;
  const float *q_norm, *k_norm, *enter_norm, *after_attn, *before_ff, *after_ff, *after_ple;
  float layer_gain, k_scale, v_scale;
  uint8_t *k_store, *v_store;
} eng_layer;

struct igl_engine {
  igl_desk   *desk;
  hipStream_t stream;
  int vocab, hidden, layers, heads, kv_heads, window, ple, share_count;
  float eps, cap;
  int window_limit, lane_limit, guess_limit, fill, precise;
  int turns[2], halves[2];
  float *steps_dev[2];
  float *turn_dev[2];  /* a small pass's rotation rows of each kind: [lane][half][cos, sin] */
  /* the checkpoint */
  void   *map;
  size_t  map_bytes;
  size_t  payload_at;
  eng_tensor *tensor;
  int     tensor_count;
  uint8_t *payload_dev;
  size_t   payload_bytes;
  igl_plane embed, ple_embed, ple_lift, head;
  const float *ple_norm, *final_norm;
  eng_layer layer[ENG_LAYER_LIMIT];
  /* device rooms, lane_limit lanes each */
  int32_t *ctl_dev;   /* [0] position of lane 0, [1 ..] the lanes' token ids */
  int32_t *ids_dev;   /* ctl_dev + 1 */
  float *state, *scrap, *lift, *q, *k, *v, *blend, *gate, *rise, *ple_seed, *ple_room, *logits;
  float *state_buf[2];  /* the residual row and its other half of a pair (fused updates) */
  int cur, pending;
  const float *pending_gain;
  float pending_scale;
  /* the first layer's input norm, left by run_pass to that layer's first
   * launch (a grouped launch's prologue forms it, others norm into scrap) */
  int enter_pending;
  float *attend_work;
  size_t attend_floats;
  int q_stride, kv_stride, inner_max, ple_stride;
  void *pick_work;
  int32_t *pick_dev;  /* per lane: the pick, its margin (as float bits) */
  int32_t *pairs_host; /* pinned: a block's picks and margins */
  int guess_from, guess_count; /* a block in flight (igl_engine_guess) */
  /* the decode step as one captured graph */
  igl_step_io *io;    /* pinned: what the step reads and writes on the host */
  int graph_on, graph_ready, graph_tried;
  hipGraphExec_t graph;
  /* a speculative block of `count` lanes as one captured graph per count
   * (blocks below the GEMM's lane floor, whose launches use only buffers
   * fixed at open and attach): ctl_host[0 .. count] is copied to ctl_dev */
  int32_t *ctl_host;  /* pinned: the block's position and ids */
  unsigned graph_gen; /* the desk's workspace generation the graphs were captured at */
  hipGraphExec_t guess_graph[ENG_GUESS_LIMIT + 1];
  unsigned char guess_ready[ENG_GUESS_LIMIT + 1], guess_tried[ENG_GUESS_LIMIT + 1];
};

/* ---- a little JSON, enough for config.json and a safetensors header ------ */

static const char *skip_ws(const char *p) {
  while (*p && isspace((unsigned char)*p)) ++p;
  return p;
}

/* End of the JSON value starting at p (string, number, literal, object or list). */
static const char *value_end(const char *p) {
  int depth = 0;
  p = skip_ws(p);
  if (*p == '"') {
    for (++p; *p && *p != '"'; ++p)
      if (*p == '\\' && p[1]) ++p;
    return *p ? p + 1 : p;
  }
  if (*p != '{' && *p != '[') {
    while (*p && *p != ',' && *p != '}' && *p != ']') ++p;
    return p;
  }
  for (; *p; ++p) {
    if (*p == '"') {
      for (++p; *p && *p != '"'; ++p)
        if (*p == '\\' && p[1]) ++p;
      if (!*p) return p;
    } else if (*p == '{' || *p == '[') {
      ++depth;
    } else if (*p == '}' || *p == ']') {
      if (--depth == 0) return p + 1;
    }
  }
  return p;
}

/* The value of member `key` directly inside the object [obj, obj_end). */
static const char *member(const char *obj, const char *obj_end, const char *key) {
  const char *p = skip_ws(obj);
  size_t klen = strlen(key);
  if (*p != '{') return NULL;
  ++p;
  while (p < obj_end) {
    const char *name;
    p = skip_ws(p);
    if (*p != '"') return NULL;
    name = p + 1;
    p = value_end(p);
    p = skip_ws(p);
    if (*p != ':') return NULL;
    p = skip_ws(p + 1);
    if ((size_t)(p - name) >= klen + 2 && strncmp(name, key, klen) == 0 && name[klen] == '"') return p;
    p = skip_ws(value_end(p));
    if (*p == ',') ++p;
    else return NULL;
  }
  return NULL;
}

static double member_number(const char *obj, const char *key, double spare) {
  const char *v = member(obj, value_end(obj), key);
  if (!v) return spare;
  if (*v == 't') return 1.0;
  if (*v == 'f') return 0.0;
  if (*v == '[') v = skip_ws(v + 1);
  return strtod(v, NULL);
}

static char *read_text(const char *path) {
  FILE *f = fopen(path, "rb");
  long n;
  char *text;
  if (!f) return NULL;
  fseek(f, 0, SEEK_END);
  n = ftell(f);
  fseek(f, 0, SEEK_SET);
  text = (char *)malloc((size_t)n + 1);
  if (text && fread(text, 1, (size_t)n, f) != (size_t)n) {
    free(text);
    text = NULL;
  }
  if (text) text[n] = '\0';
  fclose(f);
  return text;
}

/* ---- the checkpoint ------------------------------------------------------ */

static int parse_header(igl_engine *e, const char *h, size_t len) {
  const char *p = skip_ws(h), *end = h + len;
  if (*p != '{') return IGL_FAIL_FORMAT;
  ++p;
  e->tensor = (eng_tensor *)calloc(ENG_TENSOR_LIMIT, sizeof(eng_tensor));
  if (!e->tensor) return IGL_FAIL_MEMORY;
  while (p < end) {
    const char *name, *obj, *obj_end, *v;
    size_t nlen;
    p = skip_ws(p);
    if (*p == '}') break;
    if (*p != '"') return IGL_FAIL_FORMAT;
    name = p + 1;
    p = value_end(p);
    nlen = (size_t)(p - 1 - name);
    p = skip_ws(p);
    if (*p != ':') return IGL_FAIL_FORMAT;
    obj = skip_ws(p + 1);
    obj_end = value_end(obj);
    if (!(nlen == 12 && strncmp(name, "__metadata__", 12) == 0)) {
      eng_tensor *t;
      if (e->tensor_count >= ENG_TENSOR_LIMIT || nlen >= sizeof(t->name)) return IGL_FAIL_SUPPORT;
      t = &e->tensor[e->tensor_count++];
      memcpy(t->name, name, nlen);
      t->name[nlen] = '\0';
      v = member(obj, obj_end, "dtype");
      t->dtype = !v                                   ? -1
                 : strncmp(v, "\"U8\"", 4) == 0   ? 0
                 : strncmp(v, "\"F32\"", 5) == 0  ? 1
                 : strncmp(v, "\"I8\"", 4) == 0   ? 2
                 : strncmp(v, "\"BF16\"", 6) == 0 ? 3
                 : strncmp(v, "\"I32\"", 5) == 0  ? 4
                                                  : -1;
      v = member(obj, obj_end, "shape");
      if (!v || *v != '[') return IGL_FAIL_FORMAT;
      ++v;
      while (1) {
        v = skip_ws(v);
        if (*v == ']') break;
        if (t->rank >= 3) return IGL_FAIL_SUPPORT;
        t->shape[t->rank++] = strtoll(v, (char **)&v, 10);
        v = skip_ws(v);
        if (*v == ',') ++v;
      }
      v = member(obj, obj_end, "data_offsets");
      if (!v || *v != '[') return IGL_FAIL_FORMAT;
      t->begin = (size_t)strtoull(v + 1, (char **)&v, 10);
      v = skip_ws(v);
      if (*v == ',') ++v;
      t->end = (size_t)strtoull(v, NULL, 10);
    }
    p = skip_ws(obj_end);
    if (*p == ',') ++p;
  }
  return IGL_OKAY;
}

static const eng_tensor *find_tensor(const igl_engine *e, const char *name) {
  for (int i = 0; i < e->tensor_count; ++i)
    if (strcmp(e->tensor[i].name, name) == 0) return &e->tensor[i];
  return NULL;
}

static const char *k_prefix[] = {"model.language_model.", "language_model.model.", "model.", ""};

static const eng_tensor *find_stem(const igl_engine *e, const char *stem, const char *leaf) {
  char name[256];
  snprintf(name, sizeof(name), "%s.%s", stem, leaf);
  return find_tensor(e, name);
}

static float read_scalar(const igl_engine *e, const char *name, float spare) {
  const eng_tensor *t = find_tensor(e, name);
  float v;
  if (!t || t->dtype != 1 || t->end - t->begin != 4) return spare;
  memcpy(&v, (const uint8_t *)e->map + e->payload_at + t->begin, 4);
  return v;
}

/* A plane in the export's layout (plane_bind_gemma, 7886-7955, and
 * plane_bind_part's real arm, 7985-7998), bound in place on the device copy of
 * the payload:
 *   `weight` (or `embedding_quantized`) U8 [rows, cols * bits / 8], the width
 *   the one that makes the byte count come out for `col_hint` (8, 4, 2 bits),
 *   or I8 [rows, cols] (8 bits, code_flip 128), with an F32 scale [rows, G];
 *   `input_activation_scale` / `output_activation_scale`, where present, are
 *   the plane's enter and leave grids (7946-7953);
 *   a BF16 or F32 `weight` [rows, col_hint] with no scale is a real plane. */
static int bind_packed(igl_engine *e, const char *stem, const eng_tensor *w, igl_plane *out);

/* The tensor whose first dimension is a projection's row count: `weight`, or
 * the compressed-tensors pack's `weight_packed`. */
static const eng_tensor *plane_tensor(const igl_engine *e, const char *stem) {
  const eng_tensor *t = find_stem(e, stem, "weight");
  return t ? t : find_stem(e, stem, "weight_packed");
}

static int bind_plane(igl_engine *e, const char *stem, int col_hint, igl_plane *out) {
  static const int widths[] = {8, 4, 2};
  const eng_tensor *w = find_stem(e, stem, "embedding_quantized");
  const eng_tensor *s = w ? find_stem(e, stem, "embedding_scale") : NULL;
  char name[320];
  int bits = 0, groups;
  if (!w) {
    w = find_stem(e, stem, "weight");
    s = find_stem(e, stem, "weight_scale");
  }
  if (!w) {
    const eng_tensor *packed = find_stem(e, stem, "weight_packed");
    return packed ? bind_packed(e, stem, packed, out) : IGL_FAIL_MISSING;
  }
  memset(out, 0, sizeof(*out));
  if (!s && (w->dtype == 1 || w->dtype == 3)) {
    if (w->rank != 2 || w->shape[1] != col_hint) return IGL_FAIL_FORMAT;
    out->form = IGL_PLANE_REAL;
    out->row_count = (int)w->shape[0];
    out->col_count = col_hint;
    out->real_data = (const uint8_t *)e->map + e->payload_at + w->begin;
    out->real_type = w->dtype == 3 ? IGL_STORE_BF16 : IGL_STORE_F32;
    return igl_plane_bind_dev(e->desk, out, e->payload_dev + w->begin, NULL);
  }
  if (!s) return IGL_FAIL_MISSING;
  if ((w->dtype != 0 && w->dtype != 2) || s->dtype != 1 || w->rank != 2 || s->rank < 1 || s->rank > 2)
    return IGL_FAIL_SUPPORT;
  if (w->dtype == 2) {
    bits = w->shape[1] == col_hint ? 8 : 0;
  } else {
    for (size_t i = 0; i < sizeof(widths) / sizeof(widths[0]) && !bits; ++i)
      if (((long long)col_hint * widths[i] + 7) / 8 == w->shape[1]) bits = widths[i];
  }
  groups = s->rank == 2 ? (int)s->shape[1] : 1;
  if (!bits || groups < 1 || col_hint % groups) return IGL_FAIL_FORMAT;
  out->form = IGL_PLANE_CODE;
  out->row_count = (int)w->shape[0];
  out->col_count = col_hint;
  out->code_data = (const uint8_t *)e->map + e->payload_at + w->begin;
  out->row_stride = (size_t)w->shape[1];
  out->gain_data = (const uint8_t *)e->map + e->payload_at + s->begin;
  out->gain_type = IGL_STORE_F32;
  out->bit_count = bits;
  out->code_bias = 1 << (bits - 1);
  out->code_flip = w->dtype == 2 ? out->code_bias : 0;
  out->group_count = groups;
  out->group_size = col_hint / groups;
  snprintf(name, sizeof(name), "%s.input_activation_scale", stem);
  out->enter_gain = read_scalar(e, name, 0.0f);
  snprintf(name, sizeof(name), "%s.output_activation_scale", stem);
  out->leave_gain = read_scalar(e, name, 0.0f);
  return igl_plane_bind_dev(e->desk, out, e->payload_dev + w->begin,
                            (const float *)(e->payload_dev + s->begin));
}

void igl_zero_unpack(const uint32_t *words, int groups, int rows, int bits, int8_t *out) {
  const uint32_t mask = bits >= 32 ? 0xFFFFFFFFu : (1u << bits) - 1u;
  for (int n = 0; n < rows; ++n) {
    const size_t first = (size_t)n * (size_t)bits;  /* the row's first bit in its group's column */
    const size_t word = first >> 5;
    const int shift = (int)(first & 31u);
    for (int g = 0; g < groups; ++g) {
      uint64_t window = words[word * (size_t)groups + (size_t)g];
      if (shift + bits > 32) window |= (uint64_t)words[(word + 1) * (size_t)groups + (size_t)g] << 32;
      out[(size_t)n * (size_t)groups + (size_t)g] =
          (int8_t)((int)((window >> shift) & mask) - (1 << (bits - 1)));
    }
  }
}

/* A plane in the compressed-tensors pack (plane_bind_part's packed branch,
 * app_core.c:8015-8065), bound in place on the device copy of the payload:
 * `weight_packed` I32 [rows, words] holds each row as a dense little-endian
 * bit stream (the same stream a U8 row holds, in whole 32-bit words); the
 * input width is the last entry of `weight_shape`; the bit width is the one
 * that makes ceil(cols * bits / 32) come out to `words`; `weight_scale` F32
 * [rows, G] has group_size ceil(cols / G); codes are stored value + 2^(bits-1)
 * with no flip; an optional `weight_zero_point` I32 [ceil(rows * bits / 32), G]
 * packs each group's zero points along the rows (zero_read 7855-7866), here
 * unpacked once into the plane's bias_data (owned: own_block). */
static int bind_packed(igl_engine *e, const char *stem, const eng_tensor *w, igl_plane *out) {
  const eng_tensor *s = find_stem(e, stem, "weight_scale");
  const eng_tensor *shape = find_stem(e, stem, "weight_shape");
  const eng_tensor *zero = find_stem(e, stem, "weight_zero_point");
  char name[320];
  int bits = 0, cols, groups, words, rows;
  memset(out, 0, sizeof(*out));
  if (!s) return IGL_FAIL_MISSING;
  if (w->dtype != 4 || w->rank != 2 || s->dtype != 1 || s->rank < 1 || s->rank > 2) return IGL_FAIL_SUPPORT;
  if (!shape || shape->dtype != 4 || shape->rank != 1 || shape->shape[0] < 2) return IGL_FAIL_FORMAT;
  {
    int32_t last;
    memcpy(&last, (const uint8_t *)e->map + e->payload_at + shape->begin + 4 * (shape->shape[0] - 1), 4);
    cols = last;
  }
  rows = (int)w->shape[0];
  words = (int)w->shape[1];
  for (int b = 1; b <= 8 && !bits; ++b)
    if (((long long)cols * b + 31) / 32 == words) bits = b;
  groups = s->rank == 2 ? (int)s->shape[1] : 1;
  if (!bits || cols < 1 || groups < 1 || s->shape[0] != rows) return IGL_FAIL_FORMAT;
  out->form = IGL_PLANE_CODE;
  out->row_count = rows;
  out->col_count = cols;
  out->code_data = (const uint8_t *)e->map + e->payload_at + w->begin;
  out->row_stride = (size_t)words * 4u;
  out->gain_data = (const uint8_t *)e->map + e->payload_at + s->begin;
  out->gain_type = IGL_STORE_F32;
  out->bit_count = bits;
  out->code_bias = 1 << (bits - 1);
  out->code_flip = 0;
  out->group_count = groups;
  out->group_size = (cols + groups - 1) / groups;
  if (zero) {
    int8_t *table;
    if (zero->dtype != 4 || zero->rank != 2 || zero->shape[1] != groups ||
        zero->shape[0] != ((long long)rows * bits + 31) / 32)
      return IGL_FAIL_FORMAT;
    table = (int8_t *)malloc((size_t)rows * (size_t)groups);
    if (!table) return IGL_FAIL_MEMORY;
    igl_zero_unpack((const uint32_t *)((const uint8_t *)e->map + e->payload_at + zero->begin), groups, rows, bits,
                    table);
    out->bias_data = table;
    out->own_block = table;
  }
  snprintf(name, sizeof(name), "%s.input_activation_scale", stem);
  out->enter_gain = read_scalar(e, name, 0.0f);
  snprintf(name, sizeof(name), "%s.output_activation_scale", stem);
  out->leave_gain = read_scalar(e, name, 0.0f);
  return igl_plane_bind_dev(e->desk, out, e->payload_dev + w->begin, (const float *)(e->payload_dev + s->begin));
}

/* Detaches a plane and frees what the binder unpacked for it. */
static void drop_plane(igl_engine *e, igl_plane *p) {
  igl_plane_detach(e->desk, p);
  free(p->own_block);
  p->own_block = NULL;
  p->bias_data = NULL;
}

static const float *bind_vector(igl_engine *e, const char *stem, int n) {
  const eng_tensor *t = find_stem(e, stem, "weight");
  if (!t) t = find_tensor(e, stem);
  if (!t || t->dtype != 1 || (long long)(t->end - t->begin) != 4LL * n) return NULL;
  return (const float *)(e->payload_dev + t->begin);
}


/* rope_build (8121-8145): inverse frequencies 1/theta^(2i/d) in double, as
 * float; "proportional" rotates only partial * d / 2 pairs. */
static int rope_table(igl_engine *e, int kind, int head_size, double theta, double part, int proportional) {
  int half = head_size / 2, turns = half;
  float *steps = (float *)calloc((size_t)half, sizeof(float));
  if (!steps) return IGL_FAIL_MEMORY;
  if (proportional) {
    turns = (int)(part * head_size / 2.0);
    if (turns > half) turns = half;
    if (turns < 0) turns = 0;
  }
  for (int i = 0; i < turns; ++i) steps[i] = (float)(1.0 / pow(theta, (double)(2 * i) / (double)head_size));
  e->turns[kind] = turns;
  e->halves[kind] = half;
  if (hipMalloc((void **)&e->steps_dev[kind], (size_t)half * sizeof(float)) != hipSuccess ||
      hipMalloc((void **)&e->turn_dev[kind], (size_t)ENG_SMALL_LANES * half * 2 * sizeof(float)) != hipSuccess ||
      hipMemcpy(e->steps_dev[kind], steps, (size_t)half * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) {
    free(steps);
    return IGL_FAIL_DEVICE;
  }
  free(steps);
  return IGL_OKAY;
}

static int dev_alloc(void **p, size_t bytes) {
  return hipMalloc(p, bytes ? bytes : 16) == hipSuccess ? IGL_OKAY : IGL_FAIL_MEMORY;
}

/* ---- open / close ---------------------------------------------------------- */

int igl_engine_open(igl_engine **out, igl_desk *desk, const char *folder, int window_limit,
                    int lane_limit, int precise) {
  char path[1024], stem[256];
  char *config = NULL;
  const char *text, *rope, *kinds;
  igl_engine *e;
  int fd = -1, code = IGL_OKAY;
  struct stat st;
  uint64_t header_len = 0;
  const char *prefix = NULL;
  double theta[2], part[2];
  int proportional[2];
  if (!out || !desk || !desk->state || !folder) return IGL_FAIL_ARGUMENT;
  *out = NULL;
  e = (igl_engine *)calloc(1, sizeof(*e));
  if (!e) return IGL_FAIL_MEMORY;
  e->desk = desk;
  e->stream = (hipStream_t)igl_desk_stream(desk);
  e->lane_limit = lane_limit > 0 ? lane_limit : 16;
  e->guess_limit = e->lane_limit < ENG_GUESS_LIMIT ? e->lane_limit : ENG_GUESS_LIMIT;
  e->precise = precise;

  /* config.json */
  snprintf(path, sizeof(path), "%s/config.json", folder);
  config = read_text(path);
  if (!config) { code = IGL_FAIL_MISSING; goto fail; }
  text = member(config, config + strlen(config), "text_config");
  if (!text) text = skip_ws(config);
  e->vocab = (int)member_number(text, "vocab_size", 262144);
  e->hidden = (int)member_number(text, "hidden_size", 2304);
  e->layers = (int)member_number(text, "num_hidden_layers", 30);
  e->heads = (int)member_number(text, "num_attention_heads", 8);
  e->kv_heads = (int)member_number(text, "num_key_value_heads", 4);
  e->window = (int)member_number(text, "sliding_window", 512);
  e->ple = (int)member_number(text, "hidden_size_per_layer_input", 256);
  e->share_count = (int)member_number(text, "num_kv_shared_layers", 0);
  e->eps = (float)member_number(text, "rms_norm_eps", 1e-6);
  e->cap = (float)member_number(text, "final_logit_softcapping", 0.0);
  e->window_limit = (int)member_number(text, "max_position_embeddings", 131072);
  if (window_limit > 0 && window_limit < e->window_limit) e->window_limit = window_limit;
  /* norm_add holds a row of up to 4096 per workgroup */
  if (e->layers < 1 || e->layers > ENG_LAYER_LIMIT || e->kv_heads != 1 || e->heads != 8 ||
      e->hidden > 4096) {
    code = IGL_FAIL_SUPPORT;
    goto fail;
  }
  kinds = member(text, value_end(text), "layer_types");
  for (int i = 0; i < e->layers; ++i) {
    int full = ((i + 1) % 6) == 0;
    if (kinds && *kinds == '[') {
      const char *p = kinds + 1;
      for (int j = 0; j <= i && p; ++j) {
        p = skip_ws(p);
        if (*p != '"') { p = NULL; break; }
        if (j == i) full = strncmp(p, "\"sliding_attention\"", 19) != 0;
        p = skip_ws(value_end(p));
        if (*p == ',') ++p;
      }
    }
    e->layer[i].full = full;
  }
  e->layer[e->layers - 1].full = 1;
  rope = member(text, value_end(text), "rope_parameters");
  for (int kind = 0; kind < 2; ++kind) {
    const char *r = rope ? member(rope, value_end(rope), kind ? "full_attention" : "sliding_attention") : NULL;
    const char *type = r ? member(r, value_end(r), "rope_type") : NULL;
    theta[kind] = r ? member_number(r, "rope_theta", kind ? 1e6 : 1e4) : (kind ? 1e6 : 1e4);
    part[kind] = r ? member_number(r, "partial_rotary_factor", 1.0) : (kind ? 0.25 : 1.0);
    proportional[kind] = type ? strncmp(type, "\"proportional\"", 14) == 0 : kind == 1;
  }

  /* model.safetensors, mapped; the payload copied to the device as it lies */
  snprintf(path, sizeof(path), "%s/model.safetensors", folder);
  fd = open(path, O_RDONLY);
  if (fd < 0 || fstat(fd, &st) != 0 || st.st_size < 8) { code = IGL_FAIL_FILE; goto fail; }
  e->map_bytes = (size_t)st.st_size;
  e->map = mmap(NULL, e->map_bytes, PROT_READ, MAP_PRIVATE, fd, 0);
  if (e->map == MAP_FAILED) { e->map = NULL; code = IGL_FAIL_FILE; goto fail; }
  for (int b = 0; b < 8; ++b) header_len |= (uint64_t)((const uint8_t *)e->map)[b] << (8 * b);
  if (8 + header_len > e->map_bytes) { code = IGL_FAIL_FORMAT; goto fail; }
  {
    char *header = (char *)malloc(header_len + 1);
    if (!header) { code = IGL_FAIL_MEMORY; goto fail; }
    memcpy(header, (const uint8_t *)e->map + 8, header_len);
    header[header_len] = '\0';
    code = parse_header(e, header, header_len);
    free(header);
    if (code != IGL_OKAY) goto fail;
  }
  e->payload_at = 8 + header_len;
  e->payload_bytes = e->map_bytes - e->payload_at;
  if ((code = dev_alloc((void **)&e->payload_dev, e->payload_bytes)) != IGL_OKAY) goto fail;
  if (hipMemcpy(e->payload_dev, (const uint8_t *)e->map + e->payload_at, e->payload_bytes,
                hipMemcpyHostToDevice) != hipSuccess) { code = IGL_FAIL_DEVICE; goto fail; }

  for (size_t c = 0; c < sizeof(k_prefix) / sizeof(k_prefix[0]) && !prefix; ++c) {
    snprintf(stem, sizeof(stem), "%sembed_tokens", k_prefix[c]);
    if (find_stem(e, stem, "embedding_quantized") || find_stem(e, stem, "weight")) prefix = k_prefix[c];
  }
  if (!prefix) { code = IGL_FAIL_MISSING; goto fail; }
#define STEM(...) (snprintf(stem, sizeof(stem), __VA_ARGS__), stem)
  if ((code = bind_plane(e, STEM("%sembed_tokens", prefix), e->hidden, &e->embed)) != IGL_OKAY ||
      (code = bind_plane(e, STEM("%sembed_tokens_per_layer", prefix), e->layers * e->ple, &e->ple_embed)) != IGL_OKAY ||
      (code = bind_plane(e, STEM("%sper_layer_model_projection", prefix), e->hidden, &e->ple_lift)) != IGL_OKAY)
    goto fail;
  /* the embedding gathers decode rows without zero points (the exports keep
   * the embeddings symmetric or float) */
  if (e->embed.bias_data || e->ple_embed.bias_data) {
    code = IGL_FAIL_SUPPORT;
    goto fail;
  }
  if (bind_plane(e, "lm_head", e->hidden, &e->head) != IGL_OKAY &&
      bind_plane(e, STEM("%slm_head", prefix), e->hidden, &e->head) != IGL_OKAY)
    e->head = e->embed;
  e->vocab = e->head.row_count;
  e->ple_norm = bind_vector(e, STEM("%sper_layer_projection_norm", prefix), e->ple);
  e->final_norm = bind_vector(e, STEM("%snorm", prefix), e->hidden);
  if (!e->ple_norm || !e->final_norm) { code = IGL_FAIL_MISSING; goto fail; }

  {
    int first_share = e->layers - e->share_count;
    e->inner_max = 0;
    e->q_stride = 0;
    for (int i = 0; i < e->layers; ++i) {
      eng_layer *L = &e->layer[i];
      const eng_tensor *t;
      L->shared = e->share_count > 0 && i >= first_share;
      L->source = i;
      if (L->shared) {
        L->source = -1;
        for (int j = first_share - 1; j >= 0; --j)
          if (e->layer[j].full == L->full) { L->source = j; break; }
        if (L->source < 0) { code = IGL_FAIL_FORMAT; goto fail; }
      } else {
        int last = -1;
        for (int j = 0; j < first_share; ++j)
          if (e->layer[j].full == L->full) last = j;
        L->keep = e->share_count > 0 && last == i;
      }
      t = plane_tensor(e, STEM("%slayers.%d.self_attn.q_proj", prefix, i));
      if (!t) { code = IGL_FAIL_MISSING; goto fail; }
      L->head_size = (int)t->shape[0] / e->heads;
      if (L->head_size != 256 && L->head_size != 512) { code = IGL_FAIL_SUPPORT; goto fail; }
      t = plane_tensor(e, STEM("%slayers.%d.mlp.gate_proj", prefix, i));
      if (!t) { code = IGL_FAIL_MISSING; goto fail; }
      L->inner = (int)t->shape[0];
      if (L->inner > e->inner_max) e->inner_max = L->inner;
      if (e->heads * L->head_size > e->q_stride) e->q_stride = e->heads * L->head_size;
      if ((code = bind_plane(e, STEM("%slayers.%d.self_attn.q_proj", prefix, i), e->hidden, &L->q)) ||
          (code = bind_plane(e, STEM("%slayers.%d.self_attn.o_proj", prefix, i), e->heads * L->head_size, &L->o)) ||
          (code = bind_plane(e, STEM("%slayers.%d.mlp.gate_proj", prefix, i), e->hidden, &L->gate)) ||
          (code = bind_plane(e, STEM("%slayers.%d.mlp.up_proj", prefix, i), e->hidden, &L->up)) ||
          (code = bind_plane(e, STEM("%slayers.%d.mlp.down_proj", prefix, i), L->inner, &L->down)) ||
          (code = bind_plane(e, STEM("%slayers.%d.per_layer_input_gate", prefix, i), e->hidden, &L->ple_gate)) ||
          (code = bind_plane(e, STEM("%slayers.%d.per_layer_projection", prefix, i), e->ple, &L->ple_proj)))
        goto fail;
      L->q_norm = bind_vector(e, STEM("%slayers.%d.self_attn.q_norm", prefix, i), L->head_size);
      L->enter_norm = bind_vector(e, STEM("%slayers.%d.input_layernorm", prefix, i), e->hidden);
      L->after_attn = bind_vector(e, STEM("%slayers.%d.post_attention_layernorm", prefix, i), e->hidden);
      L->before_ff = bind_vector(e, STEM("%slayers.%d.pre_feedforward_layernorm", prefix, i), e->hidden);
      L->after_ff = bind_vector(e, STEM("%slayers.%d.post_feedforward_layernorm", prefix, i), e->hidden);
      L->after_ple = bind_vector(e, STEM("%slayers.%d.post_per_layer_input_norm", prefix, i), e->hidden);
      if (!L->q_norm || !L->enter_norm || !L->after_attn || !L->before_ff || !L->after_ff || !L->after_ple) {
        code = IGL_FAIL_MISSING;
        goto fail;
      }
      L->layer_gain = read_scalar(e, STEM("%slayers.%d.layer_scalar", prefix, i), 1.0f);
      if (!L->shared) {
        if ((code = bind_plane(e, STEM("%slayers.%d.self_attn.k_proj", prefix, i), e->hidden, &L->k)) ||
            (code = bind_plane(e, STEM("%slayers.%d.self_attn.v_proj", prefix, i), e->hidden, &L->v)))
          goto fail;
        if (L->k.row_count != L->head_size) { code = IGL_FAIL_SUPPORT; goto fail; }
        L->k_norm = bind_vector(e, STEM("%slayers.%d.self_attn.k_norm", prefix, i), L->head_size);
        if (!L->k_norm) { code = IGL_FAIL_MISSING; goto fail; }
        L->k_scale = read_scalar(e, STEM("%slayers.%d.self_attn.k_cache_scale", prefix, i), 0.0f);
        L->v_scale = read_scalar(e, STEM("%slayers.%d.self_attn.v_cache_scale", prefix, i), 0.0f);
        if (!(L->k_scale > 0.0f) || !(L->v_scale > 0.0f)) { code = IGL_FAIL_SUPPORT; goto fail; }
        /* full depth where sharers or the full rule need it; a sliding ring
         * otherwise, widened by a batch so a batch can write before it reads */
        L->cache_span = (L->full || L->keep) ? e->window_limit : e->window + e->lane_limit;
        if (L->cache_span > e->window_limit) L->cache_span = e->window_limit;
        if ((code = dev_alloc((void **)&L->k_store, (size_t)L->cache_span * L->head_size)) ||
            (code = dev_alloc((void **)&L->v_store, (size_t)L->cache_span * L->head_size)))
          goto fail;
      } else {
        const eng_layer *S = &e->layer[L->source];
        if (S->head_size != L->head_size) { code = IGL_FAIL_FORMAT; goto fail; }
      }
    }
  }
#undef STEM
  for (int kind = 0; kind < 2; ++kind) {
    int hs = 0;
    for (int i = 0; i < e->layers; ++i)
      if (e->layer[i].full == kind) hs = e->layer[i].head_size;
    if (hs && (code = rope_table(e, kind, hs, theta[kind], part[kind], proportional[kind])) != IGL_OKAY)
      goto fail;
  }

  /* rooms */
  {
    size_t lanes = (size_t)e->lane_limit;
    e->kv_stride = e->q_stride / e->heads;
    e->ple_stride = e->layers * e->ple;
    int widest = 0;
    for (int i = 0; i < e->layers; ++i)
      if (e->layer[i].head_size > widest) widest = e->layer[i].head_size;
    /* attention partials: every launch has at most lane_limit lanes, each
     * seeing at most window_limit positions */
    e->attend_floats = igl_attend_work_floats_limit(e->window_limit, e->lane_limit, e->heads, widest);
    if ((code = dev_alloc((void **)&e->ctl_dev, (lanes + 1) * sizeof(int32_t))) ||
        (code = dev_alloc((void **)&e->attend_work, e->attend_floats * sizeof(float))) ||
        (code = dev_alloc((void **)&e->state_buf[0], lanes * e->hidden * 4)) ||
        (code = dev_alloc((void **)&e->state_buf[1], lanes * e->hidden * 4)) ||
        (code = dev_alloc((void **)&e->scrap, lanes * e->hidden * 4)) ||
        (code = dev_alloc((void **)&e->lift, lanes * e->hidden * 4)) ||
        (code = dev_alloc((void **)&e->q, lanes * e->q_stride * 4)) ||
        (code = dev_alloc((void **)&e->blend, lanes * e->q_stride * 4)) ||
        (code = dev_alloc((void **)&e->k, lanes * e->kv_stride * 4)) ||
        (code = dev_alloc((void **)&e->v, lanes * e->kv_stride * 4)) ||
        (code = dev_alloc((void **)&e->gate, lanes * e->inner_max * 4)) ||
        (code = dev_alloc((void **)&e->rise, lanes * e->inner_max * 4)) ||
        (code = dev_alloc((void **)&e->ple_seed, lanes * e->ple_stride * 4)) ||
        (code = dev_alloc((void **)&e->ple_room, lanes * e->ple_stride * 4)) ||
        (code = dev_alloc((void **)&e->logits, (size_t)e->guess_limit * (size_t)e->vocab * 4)) ||
        (code = dev_alloc(&e->pick_work, igl_pick_work_bytes(e->guess_limit))) ||
        (code = dev_alloc((void **)&e->pick_dev, 2 * (size_t)e->guess_limit * sizeof(int32_t))))
      goto fail;
    e->ids_dev = e->ctl_dev + 1;
    e->state = e->state_buf[0];
    if (hipHostMalloc((void **)&e->io, sizeof(igl_step_io), hipHostMallocDefault) != hipSuccess ||
        hipHostMalloc((void **)&e->pairs_host, 2 * (size_t)e->guess_limit * sizeof(int32_t),
                      hipHostMallocDefault) != hipSuccess ||
        hipHostMalloc((void **)&e->ctl_host, (1 + (size_t)e->guess_limit) * sizeof(int32_t),
                      hipHostMallocDefault) != hipSuccess) {
      code = IGL_FAIL_MEMORY;
      goto fail;
    }
    e->graph_on = 1;
  }
  free(config);
  close(fd);
  *out = e;
  return IGL_OKAY;
fail:
  free(config);
  if (fd >= 0) close(fd);
  igl_engine_close(e);
  return code;
}

void igl_engine_close(igl_engine *e) {
  if (!e) return;
  (void)hipStreamSynchronize(e->stream);
  for (int i = 0; i < e->layers && i < ENG_LAYER_LIMIT; ++i) {
    eng_layer *L = &e->layer[i];
    igl_plane *pl[] = {&L->q, &L->k, &L->v, &L->o, &L->gate, &L->up, &L->down, &L->ple_gate, &L->ple_proj};
    for (size_t j = 0; j < sizeof(pl) / sizeof(pl[0]); ++j) drop_plane(e, pl[j]);
    if (L->k_store) (void)hipFree(L->k_store);
    if (L->v_store) (void)hipFree(L->v_store);
  }
  if (e->head.device == e->embed.device) {
    e->head.device = NULL;
    e->head.own_block = NULL;
  }
  drop_plane(e, &e->embed);
  drop_plane(e, &e->ple_embed);
  drop_plane(e, &e->ple_lift);
  drop_plane(e, &e->head);
  if (e->graph_ready) (void)hipGraphExecDestroy(e->graph);
  for (int c = 0; c <= ENG_GUESS_LIMIT; ++c)
    if (e->guess_ready[c]) (void)hipGraphExecDestroy(e->guess_graph[c]);
  {
    void *bufs[] = {e->payload_dev, e->ctl_dev, e->attend_work, e->state_buf[0],
                    e->state_buf[1], e->scrap, e->lift, e->q,
                    e->blend, e->k, e->v, e->gate, e->rise, e->ple_seed, e->ple_room, e->logits,
                    e->pick_work, e->pick_dev, e->steps_dev[0], e->steps_dev[1],
                    e->turn_dev[0], e->turn_dev[1]};
    for (size_t j = 0; j < sizeof(bufs) / sizeof(bufs[0]); ++j)
      if (bufs[j]) (void)hipFree(bufs[j]);
  }
  if (e->io) (void)hipHostFree(e->io);
  if (e->pairs_host) (void)hipHostFree(e->pairs_host);
  if (e->ctl_host) (void)hipHostFree(e->ctl_host);
  if (e->map) munmap(e->map, e->map_bytes);
  free(e->tensor);
  free(e);
}

/* ---- the pass ------------------------------------------------------------- */

#define RUN(x)                                            \
  do {                                                    \
    hipError_t run_e = (x);                               \
    if (run_e != hipSuccess) return IGL_FAIL_DEVICE;      \
  } while (0)
#define OKAY(x)                                           \
  do {                                                    \
    int okay_c = (x);                                     \
    if (okay_c != IGL_OKAY) return okay_c;                \
  } while (0)

/* Device addresses of a plane's codes and gains: the same offsets into the
 * device copy of the payload as into the mapped file. */
static const uint8_t *dev_codes(const igl_engine *e, const igl_plane *p) {
  return e->payload_dev + ((const uint8_t *)p->code_data - ((const uint8_t *)e->map + e->payload_at));
}

static const float *dev_gains(const igl_engine *e, const igl_plane *p) {
  return (const float *)(e->payload_dev +
                         ((const uint8_t *)p->gain_data - ((const uint8_t *)e->map + e->payload_at)));
}

static int project(igl_engine *e, const igl_plane *p, const float *act, int act_stride, int lanes,
                   float *out, int out_stride) {
  /* plane_lift_many (7814-7843): a calibrated plane's product on its grids */
  if (p->form == IGL_PLANE_CODE && (p->enter_gain > 0.0f || p->leave_gain > 0.0f))
    return igl_plane_lift_dev(e->desk, p, act, act_stride, lanes, out, out_stride);
  if (e->precise) return igl_gemv_dev(e->desk, p, act, act_stride, lanes, out, out_stride);
  return igl_mat_mat_dev(e->desk, p, act, act_stride, lanes, out, out_stride);
}

/* One lane through a calibrated plane on the level GEMV (the route
 * igl_plane_lift_dev takes for it) with the elementwise step that follows
 * fused into the store: the same kernel and the same arithmetic, one launch
 * fewer.  0 where that route does not take the plane. */
static int level_epi_fits(const igl_plane *p, const float *act, int lanes) {
  return lanes == 1 && p->form == IGL_PLANE_CODE && p->enter_gain > 0.0f && p->device && !p->bias_data &&
         igl_gemv_level_fits(p->bit_count, p->col_count) && ((uintptr_t)act & 15u) == 0;
}

static int project_level_epi(igl_engine *e, const igl_plane *p, const float *act, float *out, int epi,
                             const float *epi_in) {
  const igl_code_view view = igl_plane_view(p, dev_codes(e, p), dev_gains(e, p));
  RUN(igl_launch_gemv_level_epi(&view, p->enter_gain, p->leave_gain, act, p->col_count, 1, out, p->row_count,
                                p->row_count, p->col_count, epi, epi_in, 0, e->stream));
  return IGL_OKAY;
}

/* One lane through a calibrated plane whose x is formed by a residual update
 * in the launch's prologue (igl_launch_gemv_level_pro): x is also written to
 * x_out (NULL: not kept) for the planes that read it next. */
static int level_pro_fits(const igl_engine *e, const igl_plane *p) {
  return p->form == IGL_PLANE_CODE && p->enter_gain > 0.0f && p->device && !p->bias_data &&
         igl_gemv_level_fits(p->bit_count, p->col_count) && p->col_count == e->hidden &&
         p->col_count <= 2048;
}

static int project_level_pro(igl_engine *e, const igl_plane *p, const igl_gemv_prologue *pro, float *x_out,
                             float *out, int epi, const float *epi_in) {
  const igl_code_view view = igl_plane_view(p, dev_codes(e, p), dev_gains(e, p));
  RUN(igl_launch_gemv_level_pro(&view, p->enter_gain, p->leave_gain, pro, x_out, out, p->row_count,
                                p->col_count, epi, epi_in, e->stream));
  return IGL_OKAY;
}

/* Gate and up planes that one pair launch takes: both calibrated one-lane
 * prologue planes of the same kind, rows and enter step. */
static int level_pair_fits(const igl_engine *e, const igl_plane *g, const igl_plane *u, int rows) {
  return level_pro_fits(e, g) && level_pro_fits(e, u) && g->bit_count == u->bit_count &&
         g->code_bias == u->code_bias && g->code_flip == u->code_flip && g->group_count == u->group_count &&
         g->row_count == rows && u->row_count == rows && g->enter_gain == u->enter_gain;
}

static int project_level_pair(igl_engine *e, const igl_plane *g, const igl_plane *u,
                              const igl_gemv_prologue *pro, float *out) {
  const igl_code_view vg = igl_plane_view(g, dev_codes(e, g), dev_gains(e, g));
  const igl_code_view vu = igl_plane_view(u, dev_codes(e, u), dev_gains(e, u));
  RUN(igl_launch_gemv_level_pair(&vg, &vu, g->enter_gain, g->leave_gain, u->leave_gain, pro, out, g->row_count,
                                 g->col_count, e->stream));
  return IGL_OKAY;
}

/* Planes that one segments launch takes with p: calibrated one-lane prologue
 * planes of p's kind and enter step. */
static int level_same_kind(const igl_engine *e, const igl_plane *p, const igl_plane *u) {
  return level_pro_fits(e, u) && p->bit_count == u->bit_count && p->code_bias == u->code_bias &&
         p->code_flip == u->code_flip && p->group_count == u->group_count && p->enter_gain == u->enter_gain;
}

static int project_level_segments(igl_engine *e, const igl_plane *const *p, int count, float *const *out,
                                  const igl_gemv_prologue *pro) {
  igl_code_view v[3];
  int rows[3];
  float leave[3];
  for (int i = 0; i < count; ++i) {
    v[i] = igl_plane_view(p[i], dev_codes(e, p[i]), dev_gains(e, p[i]));
    rows[i] = p[i]->row_count;
    leave[i] = p[i]->leave_gain;
  }
  RUN(igl_launch_gemv_level_segments(v, count, rows, out, leave, p[0]->enter_gain, pro, p[0]->col_count,
                                     e->stream));
  return IGL_OKAY;
}

static int norm_rows(igl_engine *e, const float *in, const float *gain, int n, int lanes, int stride,
                     float *out) {
  return igl_norm_rms_dev(e->desk, in, gain, n, lanes, stride, e->eps, out);
}

/* One plane of a one-lane group launch. */
typedef struct eng_group {
  int count;
  const uint8_t *codes[3];
  long long row_stride[3];
  const float *gains[3];
  int gain_stride[3], rows[3];
  float *out[3];
  int out_stride[3];
} eng_group;

static void group_add(igl_engine *e, eng_group *g, const igl_plane *p, float *out, int out_stride) {
  g->codes[g->count] = dev_codes(e, p);
  g->row_stride[g->count] = (long long)p->row_stride;
  g->gains[g->count] = dev_gains(e, p);
  g->gain_stride[g->count] = p->group_count;
  g->rows[g->count] = p->row_count;
  g->out[g->count] = out;
  g->out_stride[g->count] = out_stride;
  g->count++;
}

/* Planes that can share one launch: 4-bit and uncalibrated, the same width
 * and groups, K within the register form, 4-row multiples between segments. */
static int group_fits(const eng_group *g, const igl_plane *const *p, int mode) {
  for (int i = 0; i < g->count; ++i) {
    if (p[i]->col_count != p[0]->col_count || p[i]->group_size != p[0]->group_size ||
        p[i]->group_count != p[0]->group_count || p[i]->code_bias != p[0]->code_bias ||
        p[i]->bit_count != 4 || p[i]->code_flip != 0 || p[i]->col_count > 8192 ||
        p[i]->enter_gain > 0.0f || p[i]->leave_gain > 0.0f || p[i]->bias_data)
      return 0;
    if (mode == IGL_GEMV_SEGMENTS && i + 1 < g->count && p[i]->row_count % 4) return 0;
  }
  return mode != IGL_GEMV_GELU_PAIR || p[0]->row_count == p[1]->row_count;
}

static int group_run(igl_engine *e, const eng_group *g, const igl_plane *first, int mode, int lanes,
                     const float *act, const float *mul, int mul_stride, const igl_gemv_prologue *pro) {
  RUN(igl_launch_gemv_group(mode, lanes, g->count, g->codes, g->row_stride, g->gains, g->gain_stride,
                            g->rows, g->out, g->out_stride, igl_plane_group_shift(first),
                            first->code_bias, act, e->hidden, first->col_count, mul, mul_stride, pro,
                            e->stream));
  return IGL_OKAY;
}

/* A residual update formed in the next grouped launch's prologue: state
 * moves to the other buffer of the pair. */
static igl_gemv_prologue state_update(igl_engine *e, const float *lift, const float *lift_gain,
                                      float scale, const float *norm_gain) {
  igl_gemv_prologue pro;
  pro.lane_stride = e->hidden;
  pro.state_in = e->state;
  pro.state_out = e->state_buf[e->cur ^ 1];
  pro.lift = lift;
  pro.lift_gain = lift_gain;
  pro.scale = scale;
  pro.apply_scale = scale != 1.0f;
  pro.norm_gain = norm_gain;
  pro.eps = e->eps;
  return pro;
}

static void state_flip(igl_engine *e) {
  e->cur ^= 1;
  e->state = e->state_buf[e->cur];
}

/* The previous layer's last update, if a fused step left it for this layer's
 * first launch and that launch cannot take it: applied in place, with the
 * next input norm into scrap (`next_norm` NULL: none). */
static int settle(igl_engine *e, int lanes, const float *next_norm) {
  if (!e->pending) return IGL_OKAY;
  e->pending = 0;
  RUN(igl_launch_norm_add(e->state, e->hidden, e->lift, e->hidden, e->pending_gain, e->hidden,
                          lanes, e->eps, e->pending_scale, e->pending_scale != 1.0f, next_norm,
                          e->scrap, e->hidden, e->stream));
  return IGL_OKAY;
}

/* One layer for `lanes` lanes at positions place .. place + lanes - 1 (the
 * position is read from ctl_dev[0] when the kernels run; `bound` is its
 * largest value, which sizes the attention grid) - session_layer
 * 11637-11743 with session_attend 11455-11580.
 *
 * A batch runs every residual update as its own launch, with scrap holding
 * the next sub-block's normed input.  One to eight lanes (a decode step, a
 * speculative block) fold each update into the prologue of the grouped
 * launch that consumes it - the post-attention update into the gate/up
 * launch, the post-feed-forward one into the per-layer-input gate, and this
 * layer's last (per-layer-input) update into the next layer's
 * query/key/value launch - so a layer is eight launches for one lane. */
static int run_layer(igl_engine *e, int li, int bound, int lanes) {
  eng_layer *L = &e->layer[li];
  const eng_layer *S = &e->layer[L->source];
  const int H = e->hidden, hs = L->head_size;
  const int kind = L->full ? 1 : 0;
  hipStream_t st = e->stream;
  eng_group gq = {0}, gf = {0}, gp = {0};
  const igl_plane *pq[3] = {&L->q, &L->k, &L->v};
  const igl_plane *pf[2] = {&L->gate, &L->up};
  const igl_plane *pp[1] = {&L->ple_gate};
  const float *slice = e->ple_room + (size_t)li * e->ple;
  int fused;

  group_add(e, &gq, &L->q, e->q, e->q_stride);
  if (!L->shared) {
    group_add(e, &gq, &L->k, e->k, e->kv_stride);
    group_add(e, &gq, &L->v, e->v, e->kv_stride);
  }
  group_add(e, &gf, &L->gate, e->gate, e->inner_max);
  group_add(e, &gf, &L->up, e->rise, e->inner_max);
  group_add(e, &gp, &L->ple_gate, e->gate, e->inner_max);
  /* the grouped launches take one to eight lanes up to hidden 4096 */
  fused = lanes <= ENG_GROUP_LANES && H <= 4096 &&
          group_fits(&gq, pq, IGL_GEMV_SEGMENTS) &&
          group_fits(&gf, pf, IGL_GEMV_GELU_PAIR) && group_fits(&gp, pp, IGL_GEMV_GELU_MUL) &&
          L->q.col_count == H && L->gate.col_count == H && L->ple_gate.col_count == H;

  /* query, key, value projections; then their norms and turns and the cache rows */
  if (fused && e->pending) {
    igl_gemv_prologue pro = state_update(e, e->lift, e->pending_gain, e->pending_scale, L->enter_norm);
    e->pending = 0;
    OKAY(group_run(e, &gq, &L->q, IGL_GEMV_SEGMENTS, lanes, NULL, NULL, 0, &pro));
    state_flip(e);
  } else if (lanes == 1 && e->pending && level_pro_fits(e, &L->q) && !L->shared &&
             level_same_kind(e, &L->q, &L->k) && level_same_kind(e, &L->q, &L->v)) {
    /* calibrated query, key and value planes in one launch, the update as its
     * prologue */
    const igl_plane *qkv[3] = {&L->q, &L->k, &L->v};
    float *outs[3] = {e->q, e->k, e->v};
    igl_gemv_prologue pro = state_update(e, e->lift, e->pending_gain, e->pending_scale, L->enter_norm);
    e->pending = 0;
    OKAY(project_level_segments(e, qkv, 3, outs, &pro));
    state_flip(e);
  } else if (lanes == 1 && e->pending && level_pro_fits(e, &L->q)) {
    /* a calibrated query plane takes the update in its prologue and leaves
     * the normed input in scrap for the key and value planes */
    igl_gemv_prologue pro = state_update(e, e->lift, e->pending_gain, e->pending_scale, L->enter_norm);
    e->pending = 0;
    OKAY(project_level_pro(e, &L->q, &pro, e->scrap, e->q, IGL_LEVEL_EPI_NONE, NULL));
    state_flip(e);
    if (!L->shared) {
      OKAY(project(e, &L->k, e->scrap, H, lanes, e->k, e->kv_stride));
      OKAY(project(e, &L->v, e->scrap, H, lanes, e->v, e->kv_stride));
    }
  } else if (fused && e->enter_pending) {
    /* the first layer: its input norm in the prologue, the state as it is */
    igl_gemv_prologue pro = state_update(e, NULL, NULL, 1.0f, L->enter_norm);
    e->enter_pending = 0;
    OKAY(group_run(e, &gq, &L->q, IGL_GEMV_SEGMENTS, lanes, NULL, NULL, 0, &pro));
  } else {
    OKAY(settle(e, lanes, L->enter_norm));
    if (e->enter_pending) {
      OKAY(norm_rows(e, e->state, L->enter_norm, H, lanes, H, e->scrap));
      e->enter_pending = 0;
    }
    if (fused) {
      OKAY(group_run(e, &gq, &L->q, IGL_GEMV_SEGMENTS, lanes, e->scrap, NULL, 0, NULL));
    } else {
      OKAY(project(e, &L->q, e->scrap, H, lanes, e->q, e->q_stride));
      if (!L->shared) {
        OKAY(project(e, &L->k, e->scrap, H, lanes, e->k, e->kv_stride));
        OKAY(project(e, &L->v, e->scrap, H, lanes, e->v, e->kv_stride));
      }
    }
  }
  if (lanes <= ENG_SMALL_LANES) {
    /* a decode step or a small block: the heads' norms and turns and the new
     * ring rows in the attention launch (the pass's rotation rows are
     * already on device) */
    RUN(igl_launch_attend_prep(S->k_store, S->v_store, S->k_scale, S->v_scale, S->cache_span, hs, lanes,
                               e->q, e->q_stride, L->q_norm, e->turn_dev[kind], 2 * e->halves[kind],
                               L->shared ? NULL : e->k, e->v, e->kv_stride, L->k_norm, L->k_store,
                               L->v_store, e->eps, bound, e->ctl_dev, L->full ? 0 : e->window, 1.0f,
                               e->blend, e->attend_work, st));
  } else {
    RUN(igl_launch_qkv_prep(e->q, e->q_stride, L->shared ? NULL : e->k, e->v, e->kv_stride, e->heads,
                            hs, lanes, L->q_norm, L->k_norm, e->eps, e->steps_dev[kind], e->ctl_dev,
                            L->k_store, L->v_store, L->k_scale, L->v_scale, L->cache_span, st));
    RUN(igl_launch_attend(S->k_store, S->v_store, IGL_CACHE_E4M3, S->k_scale, S->v_scale,
                          S->cache_span, hs, 1, e->heads, hs, e->q, e->q_stride, bound, e->ctl_dev,
                          L->full ? 0 : e->window, lanes, 1.0f, e->blend, e->attend_work, st));
  }
  OKAY(project(e, &L->o, e->blend, e->q_stride, lanes, e->lift, H));
  /* state += norm(o) * after_attn; gate = gelu(gate proj) * up proj of norm(state) * before_ff */
  if (fused) {
    igl_gemv_prologue pro = state_update(e, e->lift, L->after_attn, 1.0f, L->before_ff);
    OKAY(group_run(e, &gf, &L->gate, IGL_GEMV_GELU_PAIR, lanes, NULL, NULL, 0, &pro));
    state_flip(e);
  } else if (lanes == 1 && level_pair_fits(e, &L->gate, &L->up, L->inner)) {
    /* calibrated gate and up planes in one launch, the update as its prologue */
    igl_gemv_prologue pro = state_update(e, e->lift, L->after_attn, 1.0f, L->before_ff);
    OKAY(project_level_pair(e, &L->gate, &L->up, &pro, e->gate));
    state_flip(e);
  } else {
    if (lanes == 1 && level_pro_fits(e, &L->gate)) {
      /* a calibrated gate plane takes the update in its prologue */
      igl_gemv_prologue pro = state_update(e, e->lift, L->after_attn, 1.0f, L->before_ff);
      OKAY(project_level_pro(e, &L->gate, &pro, e->scrap, e->gate, IGL_LEVEL_EPI_NONE, NULL));
      state_flip(e);
    } else {
      RUN(igl_launch_norm_add(e->state, H, e->lift, H, L->after_attn, H, lanes, e->eps, 1.0f, 0,
                              L->before_ff, e->scrap, H, st));
      OKAY(project(e, &L->gate, e->scrap, H, lanes, e->gate, e->inner_max));
    }
    if (level_epi_fits(&L->up, e->scrap, lanes) && L->up.row_count == L->inner) {
      /* gate = gelu(gate) * up proj, in the up projection's store */
      OKAY(project_level_epi(e, &L->up, e->scrap, e->gate, IGL_LEVEL_EPI_GELU_RISE, e->gate));
    } else {
      OKAY(project(e, &L->up, e->scrap, H, lanes, e->rise, e->inner_max));
      RUN(igl_launch_gelu_gate_rows(e->gate, e->inner_max, e->rise, e->inner_max, L->inner, lanes, st));
    }
  }
  OKAY(project(e, &L->down, e->gate, e->inner_max, lanes, e->lift, H));
  /* state += norm(down) * after_ff; gate = gelu(per-layer gate proj of state) * slice */
  if (fused) {
    igl_gemv_prologue pro = state_update(e, e->lift, L->after_ff, 1.0f, NULL);
    OKAY(group_run(e, &gp, &L->ple_gate, IGL_GEMV_GELU_MUL, lanes, NULL, slice, e->ple_stride, &pro));
    state_flip(e);
  } else if (lanes == 1 && level_pro_fits(e, &L->ple_gate) && L->ple_gate.row_count == e->ple) {
    /* gate = gelu(per-layer gate proj of the updated state) * slice, the
     * update in the projection's prologue */
    igl_gemv_prologue pro = state_update(e, e->lift, L->after_ff, 1.0f, NULL);
    OKAY(project_level_pro(e, &L->ple_gate, &pro, NULL, e->gate, IGL_LEVEL_EPI_GELU_MUL, slice));
    state_flip(e);
  } else {
    RUN(igl_launch_norm_add(e->state, H, e->lift, H, L->after_ff, H, lanes, e->eps, 1.0f, 0, NULL,
                            NULL, 0, st));
    if (level_epi_fits(&L->ple_gate, e->state, lanes) && L->ple_gate.row_count == e->ple) {
      /* gate = gelu(per-layer gate proj) * slice, in the projection's store */
      OKAY(project_level_epi(e, &L->ple_gate, e->state, e->gate, IGL_LEVEL_EPI_GELU_MUL, slice));
    } else {
      OKAY(project(e, &L->ple_gate, e->state, H, lanes, e->gate, e->inner_max));
      RUN(igl_launch_gelu_mul(e->gate, e->inner_max, slice, e->ple_stride, e->ple, lanes, st));
    }
  }
  OKAY(project(e, &L->ple_proj, e->gate, e->inner_max, lanes, e->lift, H));
  /* state = (state + norm(ple) * after_ple) * layer_scalar: applied by the
   * next launch that reads state (settle, or a fused prologue) */
  e->pending = 1;
  e->pending_gain = L->after_ple;
  e->pending_scale = L->layer_gain;
  return IGL_OKAY;
}

/* session_pass (11843-11975) for `lanes` ids already in ids_dev, lane 0 at
 * the position in ctl_dev[0] (at most `bound`); with `logits`, the head runs
 * on the last lane (1) or every lane (2), its logits not yet capped: the pick
 * that follows every such pass caps them in place as it reads them. */
static int run_pass(igl_engine *e, int bound, int lanes, int logits) {
  hipStream_t st = e->stream;
  const int H = e->hidden;
  e->cur = 0;
  e->state = e->state_buf[0];
  e->pending = 0;
  /* embedding row times sqrt(hidden) */
  {
    const igl_plane *p = &e->embed;
    const igl_code_view view = igl_plane_view(p, dev_codes(e, p), dev_gains(e, p));
    RUN(igl_launch_gather_rows(&view, H, p->row_count, e->ids_dev, lanes, (float)sqrt((double)H),
                               e->state, H, st));
  }
  /* per-layer inputs */
  {
    const igl_plane *p = &e->ple_embed;
    const int chunk_all = e->layers * e->ple;
    OKAY(project(e, &e->ple_lift, e->state, H, lanes, e->ple_room, e->ple_stride));
    const igl_code_view view = igl_plane_view(p, dev_codes(e, p), dev_gains(e, p));
    RUN(igl_launch_gather_rows(&view, chunk_all, p->row_count, e->ids_dev, lanes,
                               (float)sqrt((double)e->ple), e->ple_seed, e->ple_stride, st));
    RUN(igl_launch_ple_mix(e->ple_room, e->ple_stride, e->ple_seed, e->ple_stride, e->ple_norm,
                           e->ple, e->layers, lanes, e->eps, (float)(1.0 / sqrt((double)H)),
                           (float)(1.0 / sqrt(2.0)), st));
  }
  e->enter_pending = 1;
  if (lanes <= ENG_SMALL_LANES)
    RUN(igl_launch_turn_row(e->steps_dev[0], e->steps_dev[0] ? e->halves[0] : 0, e->steps_dev[1],
                            e->steps_dev[1] ? e->halves[1] : 0, e->ctl_dev, lanes, e->turn_dev[0],
                            e->turn_dev[1], st));
  for (int li = 0; li < e->layers; ++li) OKAY(run_layer(e, li, bound, lanes));
  /* the last update with the final norm in one launch when the head reads
   * every lane */
  const int head_all = logits == 2 || (logits == 1 && lanes == 1);
  const int settled = e->pending;
  OKAY(settle(e, lanes, head_all ? e->final_norm : NULL));
  if (logits) {
    const int from = logits == 2 ? 0 : lanes - 1;
    const int span = lanes - from;
    if (!(head_all && settled))
      OKAY(norm_rows(e, e->state + (size_t)from * H, e->final_norm, H, span, H, e->scrap));
    OKAY(project(e, &e->head, e->scrap, H, span, e->logits, e->vocab));
  }
  return IGL_OKAY;
}

int igl_engine_prime(igl_engine *e, const int32_t *ids, int count) {
  if (!e || !ids || count < 1) return IGL_FAIL_ARGUMENT;
  if (e->guess_count || e->fill + count > e->window_limit) return IGL_FAIL_STATE;
  for (int l = 0; l < count; ++l)
    if (ids[l] < 0 || ids[l] >= e->embed.row_count) return IGL_FAIL_ARGUMENT;
  /* every id but the last, in chunks of the lane limit (session_prime_media 14443-14467) */
  for (int at = 0; at + 1 < count;) {
    int lanes = count - 1 - at < e->lane_limit ? count - 1 - at : e->lane_limit;
    RUN(igl_launch_put_int(e->ctl_dev, e->fill, e->stream));
    RUN(hipMemcpyAsync(e->ids_dev, ids + at, (size_t)lanes * sizeof(int32_t), hipMemcpyHostToDevice,
                       e->stream));
    OKAY(run_pass(e, e->fill, lanes, 0));
    e->fill += lanes;
    at += lanes;
  }
  return igl_desk_error_take(e->desk);
}

/* One decode step as the graph replays it: the position and id in from the
 * pinned io block, the pass at any position up to the last, the greedy pick,
 * the pick and its margin out to the io block. */
static int step_body(igl_engine *e) {
  RUN(hipMemcpyAsync(e->ctl_dev, &e->io->place, 2 * sizeof(int32_t), hipMemcpyHostToDevice,
                     e->stream));
  OKAY(run_pass(e, e->window_limit - 1, 1, 1));
  RUN(igl_launch_pick(e->logits, e->vocab, (size_t)e->vocab, 1, e->cap, e->pick_work, e->pick_dev,
                      e->stream));
  RUN(hipMemcpyAsync(&e->io->pick, e->pick_dev, 2 * sizeof(int32_t), hipMemcpyDeviceToHost,
                     e->stream));
  return IGL_OKAY;
}

/* Drops every captured graph if the desk has reallocated a workspace since
 * the captures (a larger batch through a path that grows one): the graphs
 * would launch on freed addresses.  They are captured again on next use. */
static void graphs_check(igl_engine *e) {
  const unsigned gen = igl_desk_generation(e->desk);
  if (gen == e->graph_gen) return;
  if (e->graph_ready) (void)hipGraphExecDestroy(e->graph);
  e->graph_ready = e->graph_tried = 0;
  for (int c = 0; c <= ENG_GUESS_LIMIT; ++c) {
    if (e->guess_ready[c]) (void)hipGraphExecDestroy(e->guess_graph[c]);
    e->guess_ready[c] = e->guess_tried[c] = 0;
  }
  e->graph_gen = gen;
}

static int capture_step(igl_engine *e) {
  hipGraph_t graph = NULL;
  int code;
  hipError_t end;
  if (hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal) != hipSuccess)
    return IGL_FAIL_DEVICE;
  code = step_body(e);
  end = hipStreamEndCapture(e->stream, &graph);
  if (code == IGL_OKAY && end != hipSuccess) code = IGL_FAIL_DEVICE;
  if (code == IGL_OKAY && hipGraphInstantiate(&e->graph, graph, NULL, NULL, 0) != hipSuccess)
    code = IGL_FAIL_DEVICE;
  if (graph) (void)hipGraphDestroy(graph);
  if (code == IGL_OKAY) e->graph_ready = 1;
  return code;
}

int igl_engine_step(igl_engine *e, int32_t id, int32_t *pick_out, float *margin_out) {
  if (!e) return IGL_FAIL_ARGUMENT;
  if (e->guess_count || e->fill + 1 > e->window_limit) return IGL_FAIL_STATE;
  if (id < 0 || id >= e->embed.row_count) return IGL_FAIL_ARGUMENT;
  e->io->place = e->fill;
  e->io->id = id;
  e->io->pick = -1;
  e->io->margin = 0.0f;
  graphs_check(e);
  /* the first step runs as it is enqueued (every kernel's first launch
   * happens outside a capture); later ones replay its capture */
  if (e->graph_on && !e->graph_ready && !e->graph_tried) {
    OKAY(step_body(e));
    RUN(hipStreamSynchronize(e->stream));
    OKAY(igl_desk_error_take(e->desk));
    graphs_check(e);  /* the run may have grown a workspace */
    e->graph_tried = 1;
    OKAY(capture_step(e));
  } else if (e->graph_on && e->graph_ready) {
    RUN(hipGraphLaunch(e->graph, e->stream));
  } else {
    OKAY(step_body(e));
  }
  RUN(hipStreamSynchronize(e->stream));
  e->fill += 1;
  if (pick_out) *pick_out = e->io->pick;
  if (margin_out) *margin_out = e->io->margin;
  return igl_desk_error_take(e->desk);
}

int igl_engine_set_graph(igl_engine *e, int on) {
  if (!e) return IGL_FAIL_ARGUMENT;
  e->graph_on = on ? 1 : 0;
  return IGL_OKAY;
}

/* ---- a speculative block (session_guess / session_guess_keep) ------------ */

/* session_guess (app_core.c:12139-12203): ids[0] is the next input and
 * ids[1 ..] the proposed continuation; one pass over all of them, with the
 * greedy pick (and its top-1/top-2 gap) of every lane's row of logits.  The
 * cache keeps the block's rows until igl_engine_keep.  Nothing needs saving
 * first: a sliding ring here is window + lane_limit rows deep, so the rows a
 * block overwrites are past every window a later position can reach, and a
 * full-depth ring only gains rows past the kept positions, which later
 * steps overwrite before any query reads them. */
/* One block of `count` lanes as a captured graph replays it: the position
 * and ids in from ctl_host, the pass with the attention grid sized for
 * `bound` (the position is read on the device), every lane's pick and margin
 * out to pairs_host. */
static int guess_body(igl_engine *e, int count, int bound) {
  RUN(hipMemcpyAsync(e->ctl_dev, e->ctl_host, (1 + (size_t)count) * sizeof(int32_t), hipMemcpyHostToDevice,
                     e->stream));
  OKAY(run_pass(e, bound, count, 2));
  RUN(igl_launch_pick(e->logits, e->vocab, (size_t)e->vocab, count, e->cap, e->pick_work, e->pick_dev,
                      e->stream));
  RUN(hipMemcpyAsync(e->pairs_host, e->pick_dev, 2 * (size_t)count * sizeof(int32_t),
                     hipMemcpyDeviceToHost, e->stream));
  return IGL_OKAY;
}

static int capture_guess(igl_engine *e, int count) {
  hipGraph_t graph = NULL;
  int code;
  hipError_t end;
  if (hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal) != hipSuccess)
    return IGL_FAIL_DEVICE;
  code = guess_body(e, count, e->window_limit - count);
  end = hipStreamEndCapture(e->stream, &graph);
  if (code == IGL_OKAY && end != hipSuccess) code = IGL_FAIL_DEVICE;
  if (code == IGL_OKAY && hipGraphInstantiate(&e->guess_graph[count], graph, NULL, NULL, 0) != hipSuccess)
    code = IGL_FAIL_DEVICE;
  if (graph) (void)hipGraphDestroy(graph);
  if (code == IGL_OKAY) e->guess_ready[count] = 1;
  return code;
}

/* session_guess (app_core.c:12139-12203): ids[0] is the next input and
 * ids[1 ..] the proposed continuation; one pass over all of them, with the
 * greedy pick (and its top-1/top-2 gap) of every lane's row of logits.  The
 * cache keeps the block's rows until igl_engine_keep.  Nothing needs saving
 * first: a sliding ring here is window + lane_limit rows deep, so the rows a
 * block overwrites are past every window a later position can reach, and a
 * full-depth ring only gains rows past the kept positions, which later
 * steps overwrite before any query reads them.
 *
 * With graphs on, a block of fewer lanes than the GEMM's floor replays one
 * graph captured for its lane count (the first block of each count runs as
 * enqueued, with the same grid, then is captured): every projection of such a
 * block is a GEMV, whose launches use only the workspace reserved at attach,
 * so no captured address can move.  Larger blocks run as enqueued. */
int igl_engine_guess(igl_engine *e, const int32_t *ids, int count, int32_t *picks_out,
                     float *margins_out) {
  if (!e || !ids || count < 1 || count > e->guess_limit) return IGL_FAIL_ARGUMENT;
  if (e->guess_count || e->fill + count > e->window_limit) return IGL_FAIL_STATE;
  for (int l = 0; l < count; ++l)
    if (ids[l] < 0 || ids[l] >= e->embed.row_count) return IGL_FAIL_ARGUMENT;
  e->ctl_host[0] = e->fill;
  memcpy(e->ctl_host + 1, ids, (size_t)count * sizeof(int32_t));
  graphs_check(e);
  if (e->graph_on && count < igl_gemm_lane_floor() && e->guess_ready[count]) {
    RUN(hipGraphLaunch(e->guess_graph[count], e->stream));
  } else if (e->graph_on && count < igl_gemm_lane_floor() && !e->guess_tried[count]) {
    OKAY(guess_body(e, count, e->window_limit - count));
    RUN(hipStreamSynchronize(e->stream));
    OKAY(igl_desk_error_take(e->desk));
    graphs_check(e);  /* the run may have grown a workspace */
    e->guess_tried[count] = 1;
    OKAY(capture_guess(e, count));
  } else {
    OKAY(guess_body(e, count, e->fill));
  }
  RUN(hipStreamSynchronize(e->stream));
  OKAY(igl_desk_error_take(e->desk));
  for (int l = 0; l < count; ++l) {
    if (picks_out) picks_out[l] = e->pairs_host[2 * l];
    if (margins_out) memcpy(&margins_out[l], &e->pairs_host[2 * l + 1], sizeof(float));
  }
  e->guess_from = e->fill;
  e->guess_count = count;
  return IGL_OKAY;
}

/* session_guess_keep (12207-12223): the first `keep` lanes of the block stay
 * in the session; 0 leaves it as it was before the block. */
int igl_engine_keep(igl_engine *e, int keep) {
  if (!e) return IGL_FAIL_ARGUMENT;
  if (!e->guess_count) return IGL_FAIL_STATE;
  if (keep < 0 || keep > e->guess_count) return IGL_FAIL_ARGUMENT;
  e->fill = e->guess_from + keep;
  e->guess_count = 0;
  return IGL_OKAY;
}

/* ---- the prompt-lookup proposer (the reference's scout, 12225-12361) ---- */

#define IGL_SCOUT_REACH 3
#define IGL_SCOUT_REACH_LEAST 2
#define IGL_SCOUT_GRAMS (IGL_SCOUT_REACH - IGL_SCOUT_REACH_LEAST + 1)

/* The committed stream, and for each reach an index from an n-gram of the
 * stream to the latest position it starts at among the positions a draw may
 * use: those with at least one committed id after the n-gram.  A draw is then
 * one lookup a reach instead of a scan of the stream.  Index slots hold start
 * positions (-1 empty); a slot's key is the n-gram the stream holds there. */
typedef struct scout_index {
  int32_t *slot;
  size_t   room;  /* a power of two */
  size_t   used;
} scout_index;

struct igl_scout {
  int32_t    *ids;
  size_t      count, room;
  scout_index gram[IGL_SCOUT_GRAMS];  /* [r]: reach IGL_SCOUT_REACH - r */
};

static uint32_t scout_hash(const int32_t *g, int reach) {
  uint32_t h = 0x811C9DC5u ^ (uint32_t)reach;
  for (int i = 0; i < reach; ++i) {
    h = (h ^ (uint32_t)g[i]) * 0x01000193u;
    h ^= h >> 15;
  }
  return h;
}

/* The slot that holds `g` (its start is the latest occurrence), or the empty
 * slot where it would go. */
static size_t scout_probe(const igl_scout *sc, const scout_index *ix, const int32_t *g, int reach) {
  size_t at = scout_hash(g, reach) & (ix->room - 1);
  for (;; at = (at + 1) & (ix->room - 1)) {
    const int32_t start = ix->slot[at];
    if (start < 0 || memcmp(sc->ids + start, g, sizeof(int32_t) * (size_t)reach) == 0) return at;
  }
}

static int scout_index_grow(igl_scout *sc, scout_index *ix, int reach) {
  const size_t room = ix->room ? 2 * ix->room : 256;
  scout_index fresh = {(int32_t *)malloc(sizeof(int32_t) * room), room, ix->used};
  if (!fresh.slot) return IGL_FAIL_MEMORY;
  memset(fresh.slot, 0xFF, sizeof(int32_t) * room);
  for (size_t i = 0; i < ix->room; ++i)
    if (ix->slot[i] >= 0) fresh.slot[scout_probe(sc, &fresh, sc->ids + ix->slot[i], reach)] = ix->slot[i];
  free(ix->slot);
  *ix = fresh;
  return IGL_OKAY;
}

int igl_scout_open(igl_scout **out) {
  if (!out) return IGL_FAIL_ARGUMENT;
  *out = (igl_scout *)calloc(1, sizeof(igl_scout));
  return *out ? IGL_OKAY : IGL_FAIL_MEMORY;
}

void igl_scout_close(igl_scout *scout) {
  if (!scout) return;
  for (int r = 0; r < IGL_SCOUT_GRAMS; ++r) free(scout->gram[r].slot);
  free(scout->ids);
  free(scout);
}

/* Appends ids the stream has committed to (scout_note, app_core.c:12311-12328).
 * Each id appended at position c makes the n-grams starting at c - reach
 * usable (they now have an id after them); each is recorded as its gram's
 * latest start. */
int igl_scout_note(igl_scout *scout, const int32_t *ids, int count) {
  if (!scout || (!ids && count > 0) || count < 0) return IGL_FAIL_ARGUMENT;
  if (scout->count + (size_t)count > (size_t)INT32_MAX) return IGL_FAIL_ARGUMENT;
  if (scout->count + (size_t)count > scout->room) {
    size_t room = scout->room + scout->room / 2 + 256;
    int32_t *fresh;
    if (room < scout->count + (size_t)count) room = scout->count + (size_t)count;
    fresh = (int32_t *)realloc(scout->ids, sizeof(int32_t) * room);
    if (!fresh) return IGL_FAIL_MEMORY;
    scout->ids = fresh;
    scout->room = room;
  }
  for (int i = 0; i < count; ++i) {
    const size_t c = scout->count;
    scout->ids[c] = ids[i];
    scout->count = c + 1;
    for (int r = 0; r < IGL_SCOUT_GRAMS; ++r) {
      const int reach = IGL_SCOUT_REACH - r;
      scout_index *ix = &scout->gram[r];
      size_t at;
      if (c < (size_t)reach) continue;
      if (2 * (ix->used + 1) > ix->room && scout_index_grow(scout, ix, reach) != IGL_OKAY)
        return IGL_FAIL_MEMORY;
      at = scout_probe(scout, ix, scout->ids + c - reach, reach);
      if (ix->slot[at] < 0) ix->used++;
      ix->slot[at] = (int32_t)(c - reach);
    }
  }
  return IGL_OKAY;
}

/* Up to `want` ids that followed the latest earlier occurrence of the
 * stream's last `reach` ids, the longest reach (3, then 2) that matches
 * anywhere; 0 when none does (scout_draw, 12341-12361). */
int igl_scout_draw(const igl_scout *scout, int32_t *out, int want) {
  if (!scout || !out || want < 1) return 0;
  for (int r = 0; r < IGL_SCOUT_GRAMS; ++r) {
    const int reach = IGL_SCOUT_REACH - r;
    const scout_index *ix = &scout->gram[r];
    const int32_t *tail;
    size_t at, from, take;
    if (scout->count < (size_t)reach + 1 || !ix->room) continue;
    tail = scout->ids + scout->count - reach;
    at = scout_probe(scout, ix, tail, reach);
    if (ix->slot[at] < 0) continue;
    from = (size_t)ix->slot[at] + (size_t)reach;
    take = scout->count - from;
    if (take > (size_t)want) take = (size_t)want;
    memcpy(out, scout->ids + from, sizeof(int32_t) * take);
    return (int)take;
  }
  return 0;
}

int igl_engine_logits(igl_engine *e, float *out, int lane) {
  if (!e || !out || lane < 0 || lane >= e->guess_limit) return IGL_FAIL_ARGUMENT;
  RUN(hipMemcpyAsync(out, e->logits + (size_t)lane * e->vocab, (size_t)e->vocab * sizeof(float),
                     hipMemcpyDeviceToHost, e->stream));
  RUN(hipStreamSynchronize(e->stream));
  return IGL_OKAY;
}

int igl_engine_fill(const igl_engine *e) { return e ? e->fill : 0; }
int igl_engine_vocab(const igl_engine *e) { return e ? e->vocab : 0; }

int igl_engine_reset(igl_engine *e) {
  if (!e) return IGL_FAIL_ARGUMENT;
  e->fill = 0;
  return IGL_OKAY;
}
