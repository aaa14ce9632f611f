/* igl_gemma.c - a seeded synthetic checkpoint in the Gemma 4 E2B text layout,
 * written the way the quantized export lays its tensors down, so the
 * reference engine (config_read, app_core.c:8325; model_bind, 8497-8733) and
 * this backend's engine both load it.
 *
 * Every projection and both embedding tables are int4 group-32 planes in the
 * export's byte layout (plane_bind_gemma, app_core.c:7886-7955): a U8 tensor
 * [rows, cols/2] of codes value + 8, two a byte, low nibble first, and an F32
 * scale [rows, cols/32].  Norm gains, the per-layer scalars and the key/value
 * cache ranges are F32.  Three files: config.json, tokenizer.json (a minimal
 * BPE vocabulary; the ids the engines run are drawn directly) and
 * model.safetensors, every payload 256-byte aligned so a device copy of the
 * payload can bind planes in place.
 *
 * Values: codes uniform over 0..15 (16 per xoshiro256** draw); scales
 * |N(0, 0.02)|; norm gains 1 + 0.1 N(0,1); layer scalars uniform in
 * [0.85, 1.15]; cache scales 6/448 (keys, values) so a unit-rms row fits the
 * e4m3 grid.  The draws run in tensor order from one seeded stream.
 */
#define _POSIX_C_SOURCE 200809L
#include <errno.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>

#include "igl_backend.h"

#define GEMMA_TENSOR_LIMIT 4096
#define GEMMA_ALIGN 256u

typedef struct gemma_tensor {
  char   name[160];
  int    dtype;       /* 0 = U8, 1 = F32, 2 = I8, 3 = BF16, 4 = I32 */
  int    rank;
  long long shape[2];
  size_t offset;      /* within the payload */
  size_t bytes;
  int    fill;        /* 0 codes, 1 scales, 2 norm gain, 3 layer scalar, 4 cache scale,
                         5 the constant `value`, 6 scales value * U(0.75, 1.25), 7 bf16 N(0, value),
                         8 scales value * U(0.99, 1.01), 9 2-bit codes of mean value 0,
                         10 zero points packed along rows (`value` bits, `rows` rows),
                         11 the I32 pair `rows`, `cols`,
                         12 codes centred on each group's zero point (`value` bits,
                            `rows` x `cols`) */
  float  value;
  long long rows, cols;
} gemma_tensor;

static const char *const k_dtype_name[] = {"U8", "F32", "I8", "BF16", "I32"};

typedef struct gemma_list {
  gemma_tensor item[GEMMA_TENSOR_LIMIT];
  int count;
  size_t payload;
} gemma_list;

void igl_gemma_shape_e2b(igl_gemma_shape *s) {
  memset(s, 0, sizeof(*s));
  s->vocab = 262144;
  s->hidden = 1536;
  s->inner = 6144;
  s->layers = 35;
  s->heads = 8;
  s->kv_heads = 1;
  s->head_dim = 256;
  s->full_head_dim = 512;
  s->window = 512;
  s->ple_size = 256;
  s->shared_layers = 20;
  s->double_wide = 1;
  s->full_every = 5;
  s->max_positions = 131072;
  s->norm_eps = 1e-6f;
  s->logit_cap = 30.0f;
  s->rope_local = 10000.0f;
  s->rope_global = 1000000.0f;
  s->partial_rotary = 0.25f;
  s->cache_scales = 1;
}

int igl_gemma_full_layer(const igl_gemma_shape *s, int layer) {
  return ((layer + 1) % s->full_every) == 0 || layer == s->layers - 1;
}

static int add_tensor(gemma_list *list, const char *name, int dtype, int rank, long long d0,
                      long long d1, int fill) {
  gemma_tensor *t;
  size_t elems = (size_t)d0 * (size_t)(rank > 1 ? d1 : 1);
  if (rank == 0) elems = 1;
  if (list->count >= GEMMA_TENSOR_LIMIT) return IGL_FAIL_SUPPORT;
  t = &list->item[list->count++];
  snprintf(t->name, sizeof(t->name), "%s", name);
  t->dtype = dtype;
  t->rank = rank;
  t->shape[0] = d0;
  t->shape[1] = d1;
  t->bytes = elems * (dtype == 1 || dtype == 4 ? 4u : dtype == 3 ? 2u : 1u);
  t->offset = list->payload;
  t->fill = fill;
  list->payload += (t->bytes + GEMMA_ALIGN - 1) / GEMMA_ALIGN * GEMMA_ALIGN;
  return IGL_OKAY;
}

/* A code plane: the export's `weight` + `weight_scale`, or the embedding
 * tables' `embedding_quantized` + `embedding_scale`. */
static int add_plane(gemma_list *list, const char *stem, long long rows, long long cols, int embed) {
  char name[200];
  int code;
  snprintf(name, sizeof(name), "%s.%s", stem, embed ? "embedding_quantized" : "weight");
  if ((code = add_tensor(list, name, 0, 2, rows, cols / 2, 0)) != IGL_OKAY) return code;
  snprintf(name, sizeof(name), "%s.%s", stem, embed ? "embedding_scale" : "weight_scale");
  return add_tensor(list, name, 1, 2, rows, cols / 32, 1);
}

/* A plane in the export's own kinds (plane_bind_gemma, app_core.c:7886-7955):
 * `bits`-wide codes (U8, or I8 for signed bytes), `groups` scale columns of
 * gain_std * U(0.75, 1.25) (one a row, as a per-channel export's absmax scales
 * sit close together), and where `enter` > 0 the calibrated activation steps
 * `input_activation_scale` / `output_activation_scale` (7946-7953). */
static int add_plane_kind(gemma_list *list, const char *stem, long long rows, long long cols, int embed,
                          int bits, int i8, long long groups, float gain_std, float enter, float leave) {
  char name[200];
  int code;
  snprintf(name, sizeof(name), "%s.%s", stem, embed ? "embedding_quantized" : "weight");
  if ((code = add_tensor(list, name, i8 ? 2 : 0, 2, rows, cols * bits / 8, bits == 2 ? 9 : 0)) != IGL_OKAY)
    return code;
  snprintf(name, sizeof(name), "%s.%s", stem, embed ? "embedding_scale" : "weight_scale");
  if ((code = add_tensor(list, name, 1, 2, rows, groups, 6)) != IGL_OKAY) return code;
  list->item[list->count - 1].value = gain_std;
  if (enter > 0.0f) {
    snprintf(name, sizeof(name), "%s.input_activation_scale", stem);
    if ((code = add_tensor(list, name, 1, 1, 1, 0, 5)) != IGL_OKAY) return code;
    list->item[list->count - 1].value = enter;
    snprintf(name, sizeof(name), "%s.output_activation_scale", stem);
    if ((code = add_tensor(list, name, 1, 1, 1, 0, 5)) != IGL_OKAY) return code;
    list->item[list->count - 1].value = leave;
  }
  return IGL_OKAY;
}

/* A plane in the compressed-tensors pack (plane_bind_part's packed branch,
 * app_core.c:8015-8065): `weight_packed` I32 [rows, cols * bits / 32] (the
 * same dense little-endian rows, codes value + 2^(bits-1)), `weight_scale` F32
 * [rows, cols / 32] (group 32), `weight_shape` I32 [rows, cols] and
 * `weight_zero_point` I32 [ceil(rows * bits / 32), cols / 32], each group's
 * zero points packed along the rows (zero_read, 7855-7866). */
static int add_plane_packed(gemma_list *list, const char *stem, long long rows, long long cols, int bits,
                            float gain_std) {
  char name[200];
  int code;
  snprintf(name, sizeof(name), "%s.weight_packed", stem);
  if ((code = add_tensor(list, name, 4, 2, rows, cols * bits / 32, 12)) != IGL_OKAY) return code;
  list->item[list->count - 1].value = (float)bits;
  list->item[list->count - 1].rows = rows;
  list->item[list->count - 1].cols = cols;
  snprintf(name, sizeof(name), "%s.weight_scale", stem);
  if ((code = add_tensor(list, name, 1, 2, rows, cols / 32, 6)) != IGL_OKAY) return code;
  list->item[list->count - 1].value = gain_std;
  snprintf(name, sizeof(name), "%s.weight_shape", stem);
  if ((code = add_tensor(list, name, 4, 1, 2, 0, 11)) != IGL_OKAY) return code;
  list->item[list->count - 1].rows = rows;
  list->item[list->count - 1].cols = cols;
  snprintf(name, sizeof(name), "%s.weight_zero_point", stem);
  if ((code = add_tensor(list, name, 4, 2, (rows * bits + 31) / 32, cols / 32, 10)) != IGL_OKAY) return code;
  list->item[list->count - 1].value = (float)bits;
  list->item[list->count - 1].rows = rows;
  return IGL_OKAY;
}

static int add_vector(gemma_list *list, const char *stem, long long n, int fill) {
  char name[200];
  snprintf(name, sizeof(name), "%s.weight", stem);
  return add_tensor(list, name, 1, 1, n, 0, fill);
}

#define P "model.language_model."

static int igl_gemma_layout(const igl_gemma_shape *s, gemma_list *list) {
  char stem[200];
  int first_share = s->layers - s->shared_layers;
  long long ple_all = (long long)s->layers * s->ple_size;
  memset(list, 0, sizeof(*list));
  if (s->hidden % 32 || s->inner % 32 || s->ple_size % 32 || s->head_dim % 32 || s->full_head_dim % 32)
    return IGL_FAIL_ARGUMENT;
  if (s->kinds == 1) {
    /* the export's kinds: 2-bit embedding (the head, tied), 4-bit per-layer
     * embedding with a scale column per layer, bf16 per_layer_model_projection */
    /* the tied head's rows: 2-bit values average -0.5, so scales that differ
     * from row to row would put a row-dependent bias into every logit; the
     * embedding's scales sit within 1% of each other */
    if (add_plane_kind(list, P "embed_tokens", s->vocab, s->hidden, 1, 2, 0, 1, 0.05f, 0.0f, 0.0f) ||
        add_plane_kind(list, P "embed_tokens_per_layer", s->vocab, ple_all, 1, 4, 0, s->layers, 0.02f, 0.0f,
                       0.0f) ||
        add_tensor(list, P "per_layer_model_projection.weight", 3, 2, ple_all, s->hidden, 7))
      return IGL_FAIL_SUPPORT;
    list->item[1].fill = 8;
    list->item[list->count - 1].value = 0.02f;
  } else if (add_plane(list, P "embed_tokens", s->vocab, s->hidden, 1) ||
             add_plane(list, P "embed_tokens_per_layer", s->vocab, ple_all, 1) ||
             add_plane(list, P "per_layer_model_projection", ple_all, s->hidden, 0)) {
    return IGL_FAIL_SUPPORT;
  }
  if (add_vector(list, P "per_layer_projection_norm", s->ple_size, 2) ||
      add_vector(list, P "norm", s->hidden, 2))
    return IGL_FAIL_SUPPORT;
  for (int i = 0; i < s->layers; ++i) {
    int full = igl_gemma_full_layer(s, i);
    int hd = full ? s->full_head_dim : s->head_dim;
    int shared = i >= first_share;
    long long inner = (long long)s->inner * (shared && s->double_wide ? 2 : 1);
    int code = 0;
    /* the export's kinds: 4-bit attention, MLPs of layers 0-14 4-bit and the
     * rest 2-bit, signed-byte per-layer planes; one scale a row, every
     * projection calibrated (module_quant_configs, model/config.json) */
    const int mlp_bits = i < 15 ? 4 : 2;
    const float mlp_std = mlp_bits == 4 ? 0.02f : 0.05f;
#define L(fmt) (snprintf(stem, sizeof(stem), P "layers.%d." fmt, i), stem)
    /* the compressed-tensors pack: 4-bit attention, MLPs of the first half
     * 4-bit and the rest 2-bit, 8-bit per-layer planes, every one with zero
     * points */
    const int pack_mlp = i < s->layers / 2 ? 4 : 2;
#define PLANE(name, rows, cols, bits, i8, std, enter, leave)                                                  \
  (s->kinds == 1   ? add_plane_kind(list, L(name), rows, cols, 0, bits, i8, 1, std, enter, leave)            \
   : s->kinds == 2 ? add_plane_packed(list, L(name), rows, cols,                                             \
                                      (bits) == 8 ? 8 : strstr(name, "mlp.") ? pack_mlp : 4,                 \
                                      (bits) == 8 ? 0.0012f : strstr(name, "mlp.") && pack_mlp == 2 ? 0.05f  \
                                                                                               : 0.02f)    \
                   : add_plane(list, L(name), rows, cols, 0))
    code |= PLANE("self_attn.q_proj", (long long)s->heads * hd, s->hidden, 4, 0, 0.02f, 0.04f, 0.04f);
    if (!shared) {
      code |= PLANE("self_attn.k_proj", (long long)s->kv_heads * hd, s->hidden, 4, 0, 0.02f, 0.04f, 0.04f);
      code |= PLANE("self_attn.v_proj", (long long)s->kv_heads * hd, s->hidden, 4, 0, 0.02f, 0.04f, 0.04f);
      code |= add_vector(list, L("self_attn.k_norm"), hd, 2);
      if (s->cache_scales) {
        code |= add_tensor(list, L("self_attn.k_cache_scale"), 1, 0, 1, 0, 4);
        code |= add_tensor(list, L("self_attn.v_cache_scale"), 1, 0, 1, 0, 4);
      }
    }
    code |= PLANE("self_attn.o_proj", s->hidden, (long long)s->heads * hd, 4, 0, 0.02f, 0.04f, 0.04f);
    code |= add_vector(list, L("self_attn.q_norm"), hd, 2);
    code |= add_vector(list, L("input_layernorm"), s->hidden, 2);
    code |= add_vector(list, L("post_attention_layernorm"), s->hidden, 2);
    code |= add_vector(list, L("pre_feedforward_layernorm"), s->hidden, 2);
    code |= add_vector(list, L("post_feedforward_layernorm"), s->hidden, 2);
    code |= PLANE("mlp.gate_proj", inner, s->hidden, mlp_bits, 0, mlp_std, 0.04f, mlp_bits == 4 ? 0.04f : 0.02f);
    code |= PLANE("mlp.up_proj", inner, s->hidden, mlp_bits, 0, mlp_std, 0.04f, mlp_bits == 4 ? 0.04f : 0.02f);
    code |= PLANE("mlp.down_proj", s->hidden, inner, mlp_bits, 0, mlp_std, mlp_bits == 4 ? 0.1f : 0.02f,
                  mlp_bits == 4 ? 0.1f : 0.02f);
    code |= PLANE("per_layer_input_gate", s->ple_size, s->hidden, 8, 1, 0.0012f, 0.1f, 0.05f);
    code |= PLANE("per_layer_projection", s->hidden, s->ple_size, 8, 1, 0.0012f, 0.05f, 0.05f);
#undef PLANE
    code |= add_vector(list, L("post_per_layer_input_norm"), s->hidden, 2);
    code |= add_tensor(list, L("layer_scalar"), 1, 0, 1, 0, 3);
#undef L
    if (code) return IGL_FAIL_SUPPORT;
  }
  if (s->kinds != 1 && add_plane(list, "lm_head", s->vocab, s->hidden, 0)) return IGL_FAIL_SUPPORT;
  return IGL_OKAY;
}

static int write_text(const char *folder, const char *leaf, const char *text) {
  char path[1024];
  FILE *f;
  snprintf(path, sizeof(path), "%s/%s", folder, leaf);
  f = fopen(path, "wb");
  if (!f) return IGL_FAIL_FILE;
  if (fwrite(text, 1, strlen(text), f) != strlen(text)) {
    fclose(f);
    return IGL_FAIL_FILE;
  }
  return fclose(f) == 0 ? IGL_OKAY : IGL_FAIL_FILE;
}

static const char gemma_tokenizer[] =
    "{\"normalizer\":{\"type\":\"Prepend\",\"prepend\":\"\\u2581\"},"
    "\"pre_tokenizer\":{\"type\":\"Metaspace\",\"replacement\":\"\\u2581\"},"
    "\"added_tokens\":["
    "{\"id\":0,\"content\":\"<pad>\",\"special\":true},"
    "{\"id\":1,\"content\":\"<eos>\",\"special\":true},"
    "{\"id\":2,\"content\":\"<bos>\",\"special\":true}],"
    "\"model\":{\"type\":\"BPE\",\"vocab\":{\"<pad>\":0,\"<eos>\":1,\"<bos>\":2,"
    "\"\\u2581\":3,\"a\":4,\"b\":5},\"merges\":[]}}";

static int write_config(const char *folder, const igl_gemma_shape *s) {
  char *text = (char *)malloc(64 * 1024);
  size_t at = 0, cap = 64 * 1024;
  int code;
  if (!text) return IGL_FAIL_MEMORY;
#define W(...) (at += (size_t)snprintf(text + at, cap - at, __VA_ARGS__))
  W("{\n  \"model_type\": \"gemma4\",\n");
  W("  \"quantization_config\": {\"quant_method\": \"gemma\", \"num_bits\": 4},\n");
  W("  \"text_config\": {\n");
  W("    \"vocab_size\": %d,\n    \"hidden_size\": %d,\n    \"intermediate_size\": %d,\n",
    s->vocab, s->hidden, s->inner);
  W("    \"num_hidden_layers\": %d,\n    \"num_attention_heads\": %d,\n    \"num_key_value_heads\": %d,\n",
    s->layers, s->heads, s->kv_heads);
  W("    \"head_dim\": %d,\n    \"global_head_dim\": %d,\n    \"sliding_window\": %d,\n",
    s->head_dim, s->full_head_dim, s->window);
  W("    \"vocab_size_per_layer_input\": %d,\n    \"hidden_size_per_layer_input\": %d,\n",
    s->vocab, s->ple_size);
  W("    \"num_kv_shared_layers\": %d,\n    \"use_double_wide_mlp\": %s,\n", s->shared_layers,
    s->double_wide ? "true" : "false");
  W("    \"rms_norm_eps\": %.9g,\n    \"final_logit_softcapping\": %.9g,\n", (double)s->norm_eps,
    (double)s->logit_cap);
  W("    \"max_position_embeddings\": %d,\n    \"bos_token_id\": 2,\n    \"eos_token_id\": 1,\n"
    "    \"pad_token_id\": 0,\n", s->max_positions);
  W("    \"rope_parameters\": {\n"
    "      \"full_attention\": {\"partial_rotary_factor\": %.9g, \"rope_theta\": %.9g, "
    "\"rope_type\": \"proportional\"},\n"
    "      \"sliding_attention\": {\"rope_theta\": %.9g, \"rope_type\": \"default\"}\n    },\n",
    (double)s->partial_rotary, (double)s->rope_global, (double)s->rope_local);
  W("    \"layer_types\": [");
  for (int i = 0; i < s->layers; ++i)
    W("%s\"%s\"", i ? ", " : "", igl_gemma_full_layer(s, i) ? "full_attention" : "sliding_attention");
  W("]\n  }\n}\n");
#undef W
  code = write_text(folder, "config.json", text);
  free(text);
  return code;
}

/* 2-bit codes whose values c - 2 average zero, as a trained plane's do (a
 * uniform draw would put a mean of -0.5 a code into every row and every
 * activation it touches): P(c) = 2/16, 3/16, 4/16, 7/16 for c = 0..3, one
 * nibble of a draw a code, four codes a byte, low bits first. */
static void fill_codes2(igl_rng *rng, uint8_t *dst, size_t count) {
  static const uint8_t k_code[16] = {0, 0, 1, 1, 1, 2, 2, 2, 2, 3, 3, 3, 3, 3, 3, 3};
  size_t i = 0;
  while (i < count) {
    uint64_t bits = igl_rng_next(rng);
    for (int b = 0; b < 4 && i < count; ++b, ++i) {
      uint8_t v = 0;
      for (int f = 0; f < 4; ++f) v |= (uint8_t)(k_code[(bits >> (16 * b + 4 * f)) & 15] << (2 * f));
      dst[i] = v;
    }
  }
}

/* The zero point of row r, group g of a packed plane: -1 throughout.  Zero
 * points that vary from row to row or group to group give each its own mean
 * weight (c - bias - zero averages -0.5 - zero on uniform codes) and make
 * this random model's stream chaotic under the byte cache: the reference's
 * own SSE2 and AVX2 builds then part within a few steps.  Varying zero points
 * are the projection tests' business. */
static int zero_of(long long r, long long g) {
  (void)r;
  (void)g;
  return -1;
}

/* Zero points of a packed plane, I32 [words][groups]: each word of group g
 * holds rows 32/bits w .. + 32/bits - 1, `bits` each, low bits first, stored
 * value + 2^(bits-1); rows past the plane hold 0. */
static void fill_zeros(uint32_t *dst, long long words, long long groups, long long rows, int bits) {
  const int per = 32 / bits;
  const int bias = 1 << (bits - 1);
  for (long long w = 0; w < words; ++w)
    for (long long g = 0; g < groups; ++g) {
      uint32_t word = 0;
      for (int r = 0; r < per; ++r) {
        const int z = w * per + r < rows ? zero_of(w * per + r, g) : 0;
        word |= (uint32_t)(z + bias) << (bits * r);
      }
      dst[w * groups + g] = word;
    }
}

/* Codes of a packed plane, rows of cols * bits / 8 bytes, low bits first:
 * c = 2^(bits-1) + zero + d, one field of a draw a code: 4 and 8 bits d
 * uniform over -2^(bits-1) .. 2^(bits-1) - 1 (the symmetric planes' values,
 * moved by the zero point; a code below 0 wraps to the top), 2 bits
 * d = -1, 0, 0, 1. */
static void fill_codes_centred(igl_rng *rng, uint8_t *dst, long long rows, long long cols, int bits) {
  const int field = bits == 2 ? 2 : bits == 4 ? 4 : 8;
  const int per_draw = 64 / field;
  const size_t row_bytes = (size_t)(cols * bits / 8);
  uint64_t draw = 0;
  int left = 0;
  memset(dst, 0, (size_t)rows * row_bytes);
  for (long long r = 0; r < rows; ++r)
    for (long long k = 0; k < cols; ++k) {
      int v, d;
      if (!left) {
        draw = igl_rng_next(rng);
        left = per_draw;
      }
      v = (int)(draw & ((1u << field) - 1u));
      draw >>= field;
      --left;
      if (bits == 2) d = v == 0 ? -1 : v == 3 ? 1 : 0;
      else if (bits == 4) d = v - 8;
      else d = v - 128;
      if ((1 << (bits - 1)) + zero_of(r, k / 32) + d < 0) d += 1 << bits;
      {
        const uint32_t c = (uint32_t)((1 << (bits - 1)) + zero_of(r, k / 32) + d);
        const size_t bit = (size_t)k * (size_t)bits;
        dst[(size_t)r * row_bytes + bit / 8] |= (uint8_t)(c << (bit % 8));
      }
    }
}

/* Fills `count` bytes of codes: 16 nibbles a draw, low nibble first. */
static void fill_codes(igl_rng *rng, uint8_t *dst, size_t count) {
  size_t i = 0;
  while (i < count) {
    uint64_t bits = igl_rng_next(rng);
    for (int b = 0; b < 8 && i < count; ++b, ++i) dst[i] = (uint8_t)(bits >> (8 * b));
  }
}

int igl_gemma_write(const char *folder, const igl_gemma_shape *shape, uint64_t seed) {
  gemma_list *list;
  igl_rng rng;
  char path[1024], *header = NULL;
  size_t header_cap = 1024 * 1024, at = 0, pad;
  FILE *f = NULL;
  uint8_t *buf = NULL;
  const size_t buf_cap = 64u << 20;
  int code = IGL_OKAY;
  if (!folder || !shape) return IGL_FAIL_ARGUMENT;
  if (mkdir(folder, 0755) != 0 && errno != EEXIST) return IGL_FAIL_FILE;
  list = (gemma_list *)malloc(sizeof(*list));
  header = (char *)malloc(header_cap);
  buf = (uint8_t *)malloc(buf_cap);
  if (!list || !header || !buf) {
    code = IGL_FAIL_MEMORY;
    goto done;
  }
  if ((code = igl_gemma_layout(shape, list)) != IGL_OKAY) goto done;
  if ((code = write_config(folder, shape)) != IGL_OKAY) goto done;
  if ((code = write_text(folder, "tokenizer.json", gemma_tokenizer)) != IGL_OKAY) goto done;

  at += (size_t)snprintf(header + at, header_cap - at, "{\"__metadata__\":{\"format\":\"pt\"}");
  for (int t = 0; t < list->count; ++t) {
    const gemma_tensor *x = &list->item[t];
    char shape_text[64];
    if (x->rank == 0) snprintf(shape_text, sizeof(shape_text), "[]");
    else if (x->rank == 1) snprintf(shape_text, sizeof(shape_text), "[%lld]", x->shape[0]);
    else snprintf(shape_text, sizeof(shape_text), "[%lld,%lld]", x->shape[0], x->shape[1]);
    at += (size_t)snprintf(header + at, header_cap - at,
                           ",\"%s\":{\"dtype\":\"%s\",\"shape\":%s,\"data_offsets\":[%zu,%zu]}",
                           x->name, k_dtype_name[x->dtype], shape_text, x->offset,
                           x->offset + x->bytes);
    if (at + 512 > header_cap) {
      code = IGL_FAIL_SUPPORT;
      goto done;
    }
  }
  header[at++] = '}';
  /* payload starts 256-aligned in the file: 8 + header (space padded) */
  pad = (GEMMA_ALIGN - (8 + at) % GEMMA_ALIGN) % GEMMA_ALIGN;
  memset(header + at, ' ', pad);
  at += pad;

  snprintf(path, sizeof(path), "%s/model.safetensors", folder);
  f = fopen(path, "wb");
  if (!f) {
    code = IGL_FAIL_FILE;
    goto done;
  }
  {
    uint64_t n = (uint64_t)at;
    uint8_t le[8];
    for (int b = 0; b < 8; ++b) le[b] = (uint8_t)(n >> (8 * b));
    if (fwrite(le, 1, 8, f) != 8 || fwrite(header, 1, at, f) != at) {
      code = IGL_FAIL_FILE;
      goto done;
    }
  }
  igl_rng_seed(&rng, seed);
  {
    size_t written = 0;
    for (int t = 0; t < list->count; ++t) {
      const gemma_tensor *x = &list->item[t];
      size_t left = x->bytes;
      /* alignment gap before this tensor */
      while (written < x->offset) {
        size_t gap = x->offset - written < buf_cap ? x->offset - written : buf_cap;
        memset(buf, 0, gap);
        if (fwrite(buf, 1, gap, f) != gap) { code = IGL_FAIL_FILE; goto done; }
        written += gap;
      }
      while (left > 0) {
        size_t take = left < buf_cap ? left : buf_cap;
        if (x->fill == 0) {
          fill_codes(&rng, buf, take);
        } else if (x->fill == 9) {
          fill_codes2(&rng, buf, take);
        } else if (x->fill == 10) {
          if (x->bytes > buf_cap) { code = IGL_FAIL_SUPPORT; goto done; }
          fill_zeros((uint32_t *)buf, x->shape[0], x->shape[1], x->rows, (int)x->value);
        } else if (x->fill == 12) {
          if (x->bytes > buf_cap) { code = IGL_FAIL_SUPPORT; goto done; }
          fill_codes_centred(&rng, buf, x->rows, x->cols, (int)x->value);
        } else if (x->fill == 11) {
          const int32_t pair[2] = {(int32_t)x->rows, (int32_t)x->cols};
          memcpy(buf, pair, sizeof(pair));
        } else {
          float *v = (float *)buf;
          size_t n = take / 4;
          if (x->fill == 1) {
            igl_rng_gains(&rng, v, n, 0.02f);
          } else if (x->fill == 2) {
            igl_rng_normal(&rng, v, n, 1.0f, 0.1f);
          } else if (x->fill == 3) {
            for (size_t i = 0; i < n; ++i)
              v[i] = 0.85f + 0.3f * (float)((igl_rng_next(&rng) >> 11) * 0x1.0p-53);
          } else if (x->fill == 4) {
            for (size_t i = 0; i < n; ++i) v[i] = 6.0f / 448.0f;
          } else if (x->fill == 5) {
            for (size_t i = 0; i < n; ++i) v[i] = x->value;
          } else if (x->fill == 6 || x->fill == 8) {
            const float spread = x->fill == 6 ? 0.5f : 0.02f;
            for (size_t i = 0; i < n; ++i)
              v[i] = x->value * (1.0f - 0.5f * spread +
                                 spread * (float)((igl_rng_next(&rng) >> 11) * 0x1.0p-53));
          } else {
            /* bf16: the top halves of N(0, value) floats, two a word */
            uint16_t *h = (uint16_t *)buf;
            size_t count = take / 2;
            float tmp[256];
            for (size_t i = 0; i < count; i += 256) {
              size_t m = count - i < 256 ? count - i : 256;
              igl_rng_normal(&rng, tmp, m, 0.0f, x->value);
              for (size_t j = 0; j < m; ++j) {
                uint32_t bits;
                memcpy(&bits, &tmp[j], 4);
                h[i + j] = (uint16_t)(bits >> 16);
              }
            }
          }
        }
        if (fwrite(buf, 1, take, f) != take) { code = IGL_FAIL_FILE; goto done; }
        left -= take;
        written += take;
      }
    }
  }
done:
  if (f && fclose(f) != 0 && code == IGL_OKAY) code = IGL_FAIL_FILE;
  free(buf);
  free(header);
  free(list);
  return code;
}
