/* audit_main.c - drives the decode engine's host code against the audit stub
 * (audit_stub.c): every launch it makes has its grid checked and every buffer
 * a launcher is handed checked against the allocation it lies in, at the
 * extent the launcher's arguments imply.  TEST INFRASTRUCTURE ONLY: nothing
 * runs on a GPU and no value is computed.
 *
 *   audit <case> <folder>
 *
 * case: e2b-decode  the synthetic E2B checkpoint, lane limit 16, the precise
 *                   GEMV path, a 2048-id prime, 12 eager steps then 4 with the
 *                   step graph (the trace workload of bench.py --kernel decode)
 *       e2b-fast    the same checkpoint, lane limit 2048, the GEMM path, a
 *                   2048-id prime in one pass, 4 steps
 *       small-guess the small shape, lane limit 16, a 600-id prime, guess
 *                   blocks of 1..16 lanes each kept in part, then steps
 *       packed      the small shape in the compressed-tensors pack (zero
 *                   points), precise and fast
 *       planted     the audit's own sensitivity: launches handed a buffer one
 *                   float short, a pointer past its allocation and a workspace
 *                   below the launcher's stated need; passes only if each is
 *                   reported (folder unused)
 * Prints one line "audit <case>: launches L, checks C, violations V" and exits
 * with V != 0 (planted: with V != 3). */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "igl_backend.h"
#include "igl_launch.h"

long audit_report(long *launch_count, long *check_count);

static uint32_t lcg_state = 12345u;
static int32_t next_id(int vocab) {
  lcg_state = lcg_state * 1664525u + 1013904223u;
  return 3 + (int32_t)((lcg_state >> 8) % (uint32_t)(vocab - 3));
}

/* Nothing runs, so a pick read back is whatever the buffers held (a graph
 * replay leaves the io block's -1): any out-of-range pick is replaced. */
static int32_t usable(int32_t pick, int vocab) { return pick >= 0 && pick < vocab ? pick : next_id(vocab); }

#define TRY(x, what)                                                      \
  do {                                                                    \
    int try_c = (x);                                                      \
    if (try_c != IGL_OKAY) {                                              \
      fprintf(stderr, "%s failed: %s (%d)\n", what, igl_code_text(try_c), try_c); \
      return 2;                                                           \
    }                                                                     \
  } while (0)

/* prime `prompt` ids, then `eager` steps without the graph and `graphed`
 * with it */
static int run_engine(igl_desk *desk, const char *folder, int window, int lanes, int precise, int prompt,
                      int eager, int graphed, int vocab) {
  igl_engine *e = NULL;
  int32_t *ids = (int32_t *)malloc((size_t)prompt * sizeof(int32_t));
  int32_t pick = 0;
  float margin = 0.0f;
  for (int i = 0; i < prompt; ++i) ids[i] = next_id(vocab);
  TRY(igl_engine_open(&e, desk, folder, window, lanes, precise), "igl_engine_open");
  TRY(igl_engine_set_graph(e, 0), "igl_engine_set_graph");
  TRY(igl_engine_prime(e, ids, prompt), "igl_engine_prime");
  pick = ids[prompt - 1];
  for (int s = 0; s < eager; ++s) {
    TRY(igl_engine_step(e, pick, &pick, &margin), "igl_engine_step");
    pick = usable(pick, vocab);
  }
  TRY(igl_engine_set_graph(e, 1), "igl_engine_set_graph");
  for (int s = 0; s < graphed; ++s) {
    TRY(igl_engine_step(e, pick, &pick, &margin), "igl_engine_step (graph)");
    pick = usable(pick, vocab);
  }
  igl_engine_close(e);
  free(ids);
  return 0;
}

/* guess blocks of every count up to the lane limit, each kept in part */
static int run_guess(igl_desk *desk, const char *folder, int window, int lanes, int precise, int prompt,
                     int vocab) {
  igl_engine *e = NULL;
  int32_t ids[64], picks[64];
  float margins[64];
  int32_t *head = (int32_t *)malloc((size_t)prompt * sizeof(int32_t));
  int32_t pick = 0;
  float margin = 0.0f;
  for (int i = 0; i < prompt; ++i) head[i] = next_id(vocab);
  TRY(igl_engine_open(&e, desk, folder, window, lanes, precise), "igl_engine_open");
  TRY(igl_engine_prime(e, head, prompt), "igl_engine_prime");
  pick = head[prompt - 1];
  for (int count = 1; count <= lanes && count <= 64; ++count) {
    ids[0] = pick;
    for (int i = 1; i < count; ++i) ids[i] = next_id(vocab);
    TRY(igl_engine_guess(e, ids, count, picks, margins), "igl_engine_guess");
    TRY(igl_engine_keep(e, 1 + count / 2), "igl_engine_keep");
    pick = usable(picks[count / 2], vocab);
  }
  for (int s = 0; s < 4; ++s) {
    TRY(igl_engine_step(e, pick, &pick, &margin), "igl_engine_step");
    pick = usable(pick, vocab);
  }
  igl_engine_close(e);
  free(head);
  return 0;
}

/* three planted mistakes, each of which the wrappers must report */
static int run_planted(void) {
  const int n = 1024, lanes = 4;
  float *gate = NULL, *ple = NULL, *logits = NULL;
  void *work = NULL;
  int32_t *pairs = NULL;
  if (hipMalloc((void **)&gate, (size_t)lanes * n * 4 - 4) != hipSuccess ||   /* one float short */
      hipMalloc((void **)&ple, (size_t)lanes * n * 4) != hipSuccess ||
      hipMalloc((void **)&logits, (size_t)n * 4) != hipSuccess ||
      hipMalloc(&work, igl_pick_work_bytes(2) - 16) != hipSuccess ||           /* below the need */
      hipMalloc((void **)&pairs, 4 * sizeof(int32_t)) != hipSuccess)
    return 2;
  (void)igl_launch_gelu_mul(gate, n, ple, n, n, lanes, NULL);
  (void)igl_launch_add_rows(ple + n, n, ple, n, n, lanes, 1.0f, 0, NULL);    /* past the end */
  (void)igl_launch_pick(logits, n / 2, (size_t)n / 2, 2, 0.0f, work, pairs, NULL);
  hipFree(gate);
  hipFree(ple);
  hipFree(logits);
  hipFree(work);
  hipFree(pairs);
  return 0;
}

int main(int argc, char **argv) {
  igl_desk desk;
  igl_gemma_shape shape;
  const char *which, *folder;
  long launches = 0, checks = 0, bad;
  int rc = 0;
  if (argc != 3) {
    fprintf(stderr, "usage: audit <e2b-decode|e2b-fast|small-guess|packed> <folder>\n");
    return 2;
  }
  which = argv[1];
  folder = argv[2];
  if (!strcmp(which, "planted")) {
    rc = run_planted();
    bad = audit_report(&launches, &checks);
    printf("audit %s: launches %ld, checks %ld, violations %ld\n", which, launches, checks, bad);
    return rc ? rc : bad == 3 ? 0 : 1;
  }
  memset(&desk, 0, sizeof(desk));
  igl_gemma_shape_e2b(&shape);
  if (!strcmp(which, "small-guess") || !strcmp(which, "packed")) {
    shape.vocab = 4096;
    shape.hidden = 512;
    shape.inner = 1024;
    shape.layers = 10;
    shape.shared_layers = 4;
    if (!strcmp(which, "packed")) shape.kinds = 2;
  }
  TRY(igl_gemma_write(folder, &shape, 1), "igl_gemma_write");
  /* the limits bench.py opens its desk with */
  TRY(igl_back_open(&desk, 0, 256, 8192, 16), "igl_back_open");
  if (!strcmp(which, "e2b-decode")) {
    rc = run_engine(&desk, folder, 2048 + 16 + 64, 16, 1, 2048, 12, 4, shape.vocab);
  } else if (!strcmp(which, "e2b-fast")) {
    rc = run_engine(&desk, folder, 2048 + 4 + 64, 2048, 0, 2048, 4, 0, shape.vocab);
  } else if (!strcmp(which, "small-guess")) {
    rc = run_guess(&desk, folder, 600 + 2048, 16, 1, 600, shape.vocab);
    if (!rc) rc = run_guess(&desk, folder, 600 + 2048, 64, 0, 600, shape.vocab);
  } else if (!strcmp(which, "packed")) {
    rc = run_engine(&desk, folder, 600 + 64 + 64, 16, 1, 600, 8, 4, shape.vocab);
    if (!rc) rc = run_engine(&desk, folder, 600 + 64 + 64, 600, 0, 600, 4, 0, shape.vocab);
  } else {
    fprintf(stderr, "unknown case %s\n", which);
    return 2;
  }
  igl_back_close(&desk);
  bad = audit_report(&launches, &checks);
  printf("audit %s: launches %ld, checks %ld, violations %ld\n", which, launches, checks, bad);
  if (rc) return rc;
  return bad ? 1 : 0;
}
