/*
 * decode_client.c -- a C client of libxdna_engine.so, the engine-side seam
 * of the reference's runtime (rust/npu-runtime/src/loader.rs:8-35: a loader
 * builds an Inference whose decode calls go through the backend; the C
 * smoke client rust/npu-capi/tests/c_smoke.rs compiles a C program against
 * the header and the shared library).
 *
 * Usage: decode_client [n_new]
 * Without a GPU it prints "devices=0" and exits 0 (host-safe, as c_smoke).
 * With one it builds a small Gemma-3-shaped decoder from the synthetic
 * weights (seed 7), then, for two streams at different positions:
 *   1. runs both streams through xe_decoder_step with per-stream positions:
 *      stream 0 starts alone (batch 1), stream 1 joins two steps later and
 *      from then on both step as batch 2 at different positions (prompt
 *      forced, then greedy);
 *   2. repeats the stream from a reset through the resident step
 *      (xe_resident_open / write / dispatch_start + xe_run_wait / read);
 * and prints both token streams, one line per stream and path:
 *   "step <b>: t0 t1 ...", "resident <b>: t0 t1 ...".
 * Every call's return value is checked; a failure prints xe_last_error()
 * and exits 1.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "xdna_engine.h"

#define CHECK(cond, what)                                             \
  do {                                                                \
    if (!(cond)) {                                                    \
      fprintf(stderr, "%s failed: %s\n", what, xe_last_error());      \
      exit(1);                                                        \
    }                                                                 \
  } while (0)

enum { B = 2, NP = 5, MAX_NEW = 64 };

static const int32_t prompt[B][NP] = {{11, 503, 77, 1024, 9}, {42, 42, 1999, 3, 640}};

/* Token stream b reads at position p: its prompt, then what it emitted
 * (emitted[k] is the greedy token after position NP - 1 + k). */
static int32_t token_at(int b, int p, int32_t out[B][MAX_NEW + NP]) {
  return p < NP ? prompt[b][p] : out[b][p - NP];
}

/* Per-stream positions: stream 0 starts alone (batch 1) and stream 1 joins
 * `lag` steps later; from then on both step together as batch 2, each at
 * its own position.  Runs until stream 1 has emitted n_new tokens. */
static void run_step_api(xe_decoder *dec, int n_new, int32_t out[B][MAX_NEW + NP]) {
  const int lag = 2;
  int32_t tok[B], pos[B], next[B];
  CHECK(xe_decoder_reset(dec) == 0, "xe_decoder_reset");
  const int last = lag + NP - 1 + n_new - 1;  /* round of stream 1's last emission */
  for (int r = 0; r <= last; r++) {
    const int nb = r < lag ? 1 : 2;
    for (int b = 0; b < nb; b++) {
      pos[b] = r - (b == 0 ? 0 : lag);
      tok[b] = token_at(b, pos[b], out);
    }
    CHECK(xe_decoder_step(dec, tok, pos, nb, NULL, next) == 0, "xe_decoder_step");
    for (int b = 0; b < nb; b++)
      if (pos[b] >= NP - 1) out[b][pos[b] - (NP - 1)] = next[b];
  }
}

/* The same streams through the resident step, both streams in lockstep
 * from position 0 (stream 1 then follows its own history). */
static void run_resident(xe_decoder *dec, int n_new, int32_t out[B][MAX_NEW + NP]) {
  xe_resident *res = xe_resident_open(dec, B);
  CHECK(res, "xe_resident_open");
  CHECK(xe_decoder_reset(dec) == 0, "xe_decoder_reset");
  int32_t tok[B], pos[B], next[B];
  for (int s = 0; s < NP - 1 + n_new; s++) {
    for (int b = 0; b < B; b++) {
      tok[b] = token_at(b, s, out);
      pos[b] = s;
    }
    CHECK(xe_resident_write(res, tok, pos) == 0, "xe_resident_write");
    xe_run *run = xe_resident_dispatch_start(res);
    CHECK(run, "xe_resident_dispatch_start");
    CHECK(xe_run_wait(run) == 0, "xe_run_wait");
    CHECK(xe_run_query(run) == 1, "xe_run_query");
    xe_run_free(run);
    CHECK(xe_resident_read(res, next, NULL) == 0, "xe_resident_read");
    if (s >= NP - 1)
      for (int b = 0; b < B; b++) out[b][s - (NP - 1)] = next[b];
  }
  xe_resident_close(res);
}

int main(int argc, char **argv) {
  const int n_new = argc > 1 ? atoi(argv[1]) : 12;
  CHECK(n_new > 0 && n_new <= MAX_NEW, "n_new in 1..64");
  CHECK(xe_abi_version() == XE_ABI_VERSION, "xe_abi_version");
  const int n = xe_device_count();
  printf("devices=%d\n", n);
  if (n <= 0) return 0;
  xe_device *dev = xe_device_open(0);
  CHECK(dev, "xe_device_open");
  char name[64];
  CHECK(xe_device_name(dev, name, sizeof name) > 0, "xe_device_name");
  printf("device=%s\n", name);
  xe_model_config cfg;
  memset(&cfg, 0, sizeof cfg);
  cfg.family = XE_GEMMA3;
  cfg.n_layers = 2;
  cfg.d_model = 256;
  cfg.n_heads = 4;
  cfg.n_kv_heads = 1;
  cfg.head_dim = 256;
  cfg.ffn = 1024;
  cfg.vocab = 2048;
  cfg.max_pos = 0;
  cfg.max_ctx = 128;
  cfg.wdtype = XE_I8;
  cfg.eps = 1e-6f;
  cfg.rope_theta = 1e6f;
  xe_decoder *dec = xe_decoder_create(dev, &cfg, B);
  CHECK(dec, "xe_decoder_create");
  CHECK(xe_decoder_init_synthetic(dec, 7) == 0, "xe_decoder_init_synthetic");
  static int32_t a[B][MAX_NEW + NP], r[B][MAX_NEW + NP];
  run_step_api(dec, n_new, a);
  run_resident(dec, n_new, r);
  for (int b = 0; b < B; b++) {
    printf("step %d:", b);
    for (int i = 0; i < n_new; i++) printf(" %d", a[b][i]);
    printf("\nresident %d:", b);
    for (int i = 0; i < n_new; i++) printf(" %d", r[b][i]);
    printf("\n");
  }
  xe_decoder_destroy(dec);
  xe_device_close(dev);
  return 0;
}
