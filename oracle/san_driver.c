/* san_driver.c -- TEST INFRASTRUCTURE ONLY: runs every function of the C
 * restatement (mx_oracle.c) on seeded random and edge-case inputs, built with
 * AddressSanitizer and UndefinedBehaviorSanitizer (see the Makefile's `san`
 * target), so that an out-of-bounds access, a leak or undefined behaviour in
 * the checker aborts the run.  It also asserts a few invariants that hold for
 * any input (sorted keys ascend, run lengths sum to N, repaired offsets are
 * monotone and in range, quantize/dequantize stay within one step).
 * Exit status 0 = clean.  tests/test_oracle_sanitize.py builds and runs it. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "mx_oracle.h"

static uint64_t g_rng = 0x9E3779B97F4A7C15ull;

static uint32_t rnd(void) {
  g_rng = g_rng * 6364136223846793005ull + 1442695040888963407ull;
  return (uint32_t)(g_rng >> 33);
}

static int64_t rnd_below(int64_t n) { return n > 0 ? (int64_t)(rnd() % (uint64_t)n) : 0; }

static float rnd_unit(void) { return (float)(rnd() & 0xffffff) / (float)0x1000000; }

#define CHECK(cond)                                                           \
  do {                                                                        \
    if (!(cond)) {                                                            \
      fprintf(stderr, "san_driver: check failed at line %d: %s\n", __LINE__, #cond); \
      exit(1);                                                                \
    }                                                                         \
  } while (0)

static void* xmalloc(size_t n) {
  void* p = malloc(n > 0 ? n : 1);
  CHECK(p != NULL);
  return p;
}

/* A batch: T tables of rows[t] rows, B bags each, lengths in [0, max_L],
 * about `empty_pct` percent empty bags. */
typedef struct {
  int32_t T;
  int64_t B, N;
  int64_t* rows;
  int32_t* D_off;
  int64_t* offsets;
  int64_t* indices;
} Batch;

static Batch make_batch(int32_t T, int64_t B, int max_L, int empty_pct, const int32_t* dims) {
  Batch b;
  b.T = T;
  b.B = B;
  b.rows = (int64_t*)xmalloc(sizeof(int64_t) * T);
  b.D_off = (int32_t*)xmalloc(sizeof(int32_t) * (T + 1));
  b.offsets = (int64_t*)xmalloc(sizeof(int64_t) * (T * B + 1));
  b.D_off[0] = 0;
  for (int32_t t = 0; t < T; ++t) {
    b.rows[t] = 1 + rnd_below(300);
    b.D_off[t + 1] = b.D_off[t] + dims[t];
  }
  b.offsets[0] = 0;
  for (int64_t i = 0; i < T * B; ++i) {
    const int64_t len = (int)rnd_below(100) < empty_pct ? 0 : rnd_below(max_L + 1);
    b.offsets[i + 1] = b.offsets[i] + len;
  }
  b.N = b.offsets[T * B];
  b.indices = (int64_t*)xmalloc(sizeof(int64_t) * b.N);
  for (int64_t i = 0; i < T * B; ++i) {
    const int32_t t = (int32_t)(i / B);
    for (int64_t l = b.offsets[i]; l < b.offsets[i + 1]; ++l) b.indices[l] = rnd_below(b.rows[t]);
  }
  return b;
}

static void free_batch(Batch* b) {
  free(b->rows);
  free(b->D_off);
  free(b->offsets);
  free(b->indices);
}

/* Every table of one width: the batch can be a sequence (nobag) lookup. */
static int32_t uniform_D(const Batch* b) {
  const int32_t D = b->T > 0 ? b->D_off[1] - b->D_off[0] : 0;
  for (int32_t t = 1; t < b->T; ++t)
    if (b->D_off[t + 1] - b->D_off[t] != D) return -1;
  return D;
}

static int bits_for(int64_t n) {
  int b = 1;
  while ((int64_t)1 << b < n) ++b;
  return b;
}

static void run_tbe(const Batch* b) {
  int64_t* w_off = (int64_t*)xmalloc(sizeof(int64_t) * b->T);
  int64_t* hsc = (int64_t*)xmalloc(sizeof(int64_t) * (b->T + 1));
  int64_t* m1_off = (int64_t*)xmalloc(sizeof(int64_t) * b->T);
  int64_t nw = 0, nm = 0;
  hsc[0] = 0;
  for (int32_t t = 0; t < b->T; ++t) {
    w_off[t] = nw;
    m1_off[t] = nm;
    nw += b->rows[t] * (b->D_off[t + 1] - b->D_off[t]);
    nm += b->rows[t];
    hsc[t + 1] = hsc[t] + b->rows[t];
  }
  const int64_t total_D = b->D_off[b->T];
  float* W = (float*)xmalloc(sizeof(float) * nw);
  float* m1 = (float*)xmalloc(sizeof(float) * nm);
  float* iw = (float*)xmalloc(sizeof(float) * b->N);
  float* out = (float*)xmalloc(sizeof(float) * b->B * total_D);
  float* grad = (float*)xmalloc(sizeof(float) * b->B * total_D);
  float* giw = (float*)xmalloc(sizeof(float) * b->N);
  int32_t* frg = (int32_t*)xmalloc(sizeof(int32_t) * b->T);
  for (int64_t i = 0; i < nw; ++i) W[i] = rnd_unit() * 0.02f - 0.01f;
  for (int64_t i = 0; i < nm; ++i) m1[i] = rnd_unit() * 1e-4f;
  for (int64_t i = 0; i < b->N; ++i) iw[i] = rnd_unit() * 2.0f - 1.0f;
  for (int64_t i = 0; i < b->B * total_D; ++i) grad[i] = rnd_unit() * 0.02f - 0.01f;
  for (int32_t t = 0; t < b->T; ++t) frg[t] = t % 2;
  for (int pooling = 0; pooling < 2; ++pooling) {
    orc_tbe_forward_f32(W, w_off, b->D_off, b->T, b->B, b->indices, b->offsets, pooling, NULL,
                        out, total_D);
    orc_tbe_forward_f32(W, w_off, b->D_off, b->T, b->B, b->indices, b->offsets, pooling, iw,
                        out, total_D);
    orc_grad_indice_weights(grad, total_D, W, w_off, b->D_off, b->T, b->B, b->indices,
                            b->offsets, pooling, frg, giw);
    orc_grad_indice_weights(grad, total_D, W, w_off, b->D_off, b->T, b->B, b->indices,
                            b->offsets, pooling, NULL, giw);
  }

  /* transpose: keys ascend, runs tile the batch, the cumsum is complete */
  const int32_t bits = bits_for(hsc[b->T]);
  const int32_t nb = 26;
  const int64_t n = b->N > 0 ? b->N : 1;
  int64_t* linear = (int64_t*)xmalloc(sizeof(int64_t) * n);
  int64_t* sorted = (int64_t*)xmalloc(sizeof(int64_t) * n);
  int32_t* infos = (int32_t*)xmalloc(sizeof(int32_t) * n);
  int64_t* run = (int64_t*)xmalloc(sizeof(int64_t) * n);
  int32_t* lens = (int32_t*)xmalloc(sizeof(int32_t) * n);
  int32_t* cum = (int32_t*)xmalloc(sizeof(int32_t) * (n + 1));
  int64_t num_runs = 0;
  if (b->N > 0) {
    CHECK(orc_transpose(hsc, b->T, b->B, nb, bits, b->indices, b->offsets, b->N, linear, sorted,
                        infos, run, lens, &num_runs, cum) == 0);
    int64_t total = 0;
    for (int64_t i = 1; i < b->N; ++i) CHECK(sorted[i - 1] <= sorted[i]);
    for (int64_t r = 0; r < num_runs; ++r) total += lens[r];
    CHECK(total == b->N);
    for (int64_t k = num_runs; k <= b->N; ++k) CHECK(cum[k] == b->N);
    for (int64_t k = num_runs; k < b->N; ++k) CHECK(lens[k] == 0);
  }
  for (int mode = 0; mode < 3; ++mode)
    for (int pooling = 0; pooling < 2; ++pooling) {
      CHECK(orc_backward_rowwise_adagrad(W, w_off, b->D_off, b->T, b->B, hsc, bits, b->indices,
                                         b->offsets, b->N, pooling, NULL, grad, total_D, m1,
                                         m1_off, 0.01f, 1e-8f, 0.01f, mode, nb) == 0);
      CHECK(orc_backward_rowwise_adagrad(W, w_off, b->D_off, b->T, b->B, hsc, bits, b->indices,
                                         b->offsets, b->N, pooling, iw, grad, total_D, m1,
                                         m1_off, 0.01f, 1e-8f, 0.0f, mode, nb) == 0);
    }
  for (int64_t i = 0; i < nw; ++i) CHECK(isfinite(W[i]));
  const int32_t Du = uniform_D(b);
  if (Du > 0) { /* the nobag backward: one gradient row per position */
    float* gn = (float*)xmalloc(sizeof(float) * n * Du);
    for (int64_t i = 0; i < b->N * Du; ++i) gn[i] = rnd_unit() * 0.02f - 0.01f;
    for (int mode = 0; mode < 3; ++mode)
      CHECK(orc_backward_rowwise_adagrad_nobag(W, w_off, Du, b->T, b->B, hsc, bits, b->indices,
                                               b->offsets, b->N, gn, m1, m1_off, 0.01f, 1e-8f,
                                               0.01f, mode, nb) == 0);
    for (int64_t i = 0; i < nw; ++i) CHECK(isfinite(W[i]));
    free(gn);
  }

  /* bounds check on a broken copy: repaired offsets are monotone in [0, N] */
  int64_t* idx2 = (int64_t*)xmalloc(sizeof(int64_t) * n);
  int64_t* off2 = (int64_t*)xmalloc(sizeof(int64_t) * (b->T * b->B + 1));
  for (int mode = 0; mode < 4; ++mode) {
    memcpy(idx2, b->indices, sizeof(int64_t) * b->N);
    memcpy(off2, b->offsets, sizeof(int64_t) * (b->T * b->B + 1));
    for (int64_t l = 0; l < b->N; ++l)
      if (rnd_below(20) == 0) idx2[l] = rnd_below(700) - 200;
    for (int k = 0; k < 3; ++k) off2[rnd_below(b->T * b->B + 1)] = rnd_below(3 * b->N + 3) - b->N;
    const int64_t bad = orc_bounds_check(b->rows, b->T, b->B, idx2, off2, b->N, mode);
    CHECK(bad >= 0);
    if (mode == 1 || mode == 2) {
      for (int64_t i = 0; i <= b->T * b->B; ++i) {
        CHECK(off2[i] >= 0 && off2[i] <= b->N);
        if (i > 0) CHECK(off2[i - 1] <= off2[i]);
      }
    }
  }
  free(idx2);
  free(off2);
  free(linear);
  free(sorted);
  free(infos);
  free(run);
  free(lens);
  free(cum);
  free(w_off);
  free(hsc);
  free(m1_off);
  free(W);
  free(m1);
  free(iw);
  free(out);
  free(grad);
  free(giw);
  free(frg);
}

static void run_nbit(const Batch* b, const int32_t* tys) {
  int64_t* w_off = (int64_t*)xmalloc(sizeof(int64_t) * b->T);
  uint8_t* tys8 = (uint8_t*)xmalloc(b->T);
  int64_t bytes = 0;
  for (int32_t t = 0; t < b->T; ++t) {
    const int32_t D = b->D_off[t + 1] - b->D_off[t];
    w_off[t] = bytes;
    tys8[t] = (uint8_t)tys[t];
    bytes += b->rows[t] * orc_nbit_row_bytes(tys[t], D, 16);
  }
  uint8_t* W = (uint8_t*)xmalloc(bytes);
  for (int64_t i = 0; i < bytes; ++i) W[i] = (uint8_t)rnd();
  /* finite fp16/fp32 values and qparams: rewrite each row's leading words */
  for (int32_t t = 0; t < b->T; ++t) {
    const int32_t D = b->D_off[t + 1] - b->D_off[t];
    const int64_t stride = orc_nbit_row_bytes(tys[t], D, 16);
    for (int64_t r = 0; r < b->rows[t]; ++r) {
      uint8_t* row = W + w_off[t] + r * stride;
      if (tys[t] == ORC_FP32) {
        for (int32_t d = 0; d < D; ++d) {
          const float f = rnd_unit() - 0.5f;
          memcpy(row + 4 * d, &f, 4);
        }
      } else if (tys[t] == ORC_FP16) {
        for (int32_t d = 0; d < D; ++d) {
          const uint16_t h = orc_float_to_half(rnd_unit() - 0.5f);
          memcpy(row + 2 * d, &h, 2);
        }
      } else if (tys[t] == ORC_FP8) {
        /* every byte is a finite hfp8 code */
      } else {
        const uint16_t s = orc_float_to_half(1e-3f + rnd_unit() * 9e-3f);
        const uint16_t bi = orc_float_to_half(rnd_unit() * 0.2f - 0.1f);
        memcpy(row, &s, 2);
        memcpy(row + 2, &bi, 2);
      }
    }
  }
  const int64_t total_D = b->D_off[b->T];
  float* iw = (float*)xmalloc(sizeof(float) * (b->N > 0 ? b->N : 1));
  for (int64_t i = 0; i < b->N; ++i) iw[i] = rnd_unit();
  void* out = xmalloc(sizeof(float) * b->B * total_D);
  for (int pooling = 0; pooling < 2; ++pooling)
    for (int f16 = 0; f16 < 3; ++f16) { /* fp32, fp16, bf16 output */
      CHECK(orc_nbit_forward(W, w_off, tys8, b->D_off, b->T, b->B, b->indices, b->offsets,
                             pooling, NULL, 16, f16, out, total_D, 4, 7) == 0);
      CHECK(orc_nbit_forward(W, w_off, tys8, b->D_off, b->T, b->B, b->indices, b->offsets,
                             pooling, iw, 16, f16, out, total_D, 5, 15) == 0);
    }
  const int32_t Du = uniform_D(b);
  if (Du > 0) { /* the nobag lookup: one output row per position */
    void* on = xmalloc(sizeof(float) * (b->N > 0 ? b->N : 1) * Du);
    for (int kind = 0; kind < 3; ++kind)
      CHECK(orc_nbit_forward_nobag(W, w_off, tys8, Du, b->T, b->B, b->indices, b->offsets, 16,
                                   kind, on, 4, 7) == 0);
    free(on);
  }
  free(W);
  free(w_off);
  free(tys8);
  free(iw);
  free(out);
}

static void run_codecs(int64_t rows, int64_t D) {
  float* x = (float*)xmalloc(sizeof(float) * rows * D);
  float* y = (float*)xmalloc(sizeof(float) * rows * D);
  for (int64_t i = 0; i < rows * D; ++i) x[i] = rnd_unit() * 4.0f - 2.0f;
  if (rows > 1)
    for (int64_t j = 0; j < D; ++j) x[j] = 0.5f; /* a constant row: zero range */
  uint8_t* q8 = (uint8_t*)xmalloc(rows * (D + 8));
  orc_quantize_8bit(x, rows, D, q8);
  orc_dequantize_8bit(q8, rows, D, y);
  for (int64_t i = 0; i < rows * D; ++i) CHECK(fabsf(x[i] - y[i]) <= 4.0f / 255.0f + 1e-6f);
  for (int bits = 2; bits <= 8; bits *= 2) {
    const int64_t nbytes = (D * bits + 7) / 8;
    uint8_t* qn = (uint8_t*)xmalloc(rows * (nbytes + 4));
    orc_quantize_nbit(x, rows, D, bits, qn);
    orc_dequantize_nbit(qn, rows, D, bits, y);
    for (int64_t i = 0; i < rows * D; ++i) CHECK(isfinite(y[i]));
    free(qn);
  }
  free(x);
  free(y);
  free(q8);
}

int main(void) {
  /* every fp16 bit pattern round-trips through float (NaNs stay NaNs) */
  for (uint32_t h = 0; h < 65536; ++h) {
    const float f = orc_half_to_float((uint16_t)h);
    if (isnan(f))
      CHECK(isnan(orc_half_to_float(orc_float_to_half(f))));
    else
      CHECK(orc_float_to_half(f) == (uint16_t)h);
  }
  const int32_t dims3[3] = {4, 32, 128};
  const int32_t dims5[5] = {8, 16, 24, 64, 256};
  const int32_t tys5[5] = {ORC_FP32, ORC_FP16, ORC_INT8, ORC_INT4, ORC_INT2};
  const int32_t tys5b[5] = {ORC_FP8, ORC_FP16, ORC_INT8, ORC_INT4, ORC_FP8};
  const int32_t dims3u[3] = {32, 32, 32};
  const int32_t dims5u[5] = {16, 16, 16, 16, 16};
  for (int rep = 0; rep < 24; ++rep) {
    Batch a = make_batch(3, 17 + 13 * rep, 9 + rep, 20, dims3);
    run_tbe(&a);
    free_batch(&a);
    Batch c = make_batch(5, 13 + 5 * rep, 7, 25, dims5);
    run_nbit(&c, rep % 2 ? tys5b : tys5);
    free_batch(&c);
    Batch u = make_batch(3, 11 + 7 * rep, 12, 20, dims3u); /* sequence lookups */
    run_tbe(&u);
    free_batch(&u);
    Batch v = make_batch(5, 9 + 3 * rep, 6, 25, dims5u);
    run_nbit(&v, rep % 2 ? tys5b : tys5);
    free_batch(&v);
  }
  /* hfp8: every code decodes to a value that encodes back to the code */
  for (int cfg = 0; cfg < 2; ++cfg) {
    const int ebits = cfg ? 5 : 4, ebias = cfg ? 15 : 7, m = 7 - ebits;
    const float max_pos = ldexpf(2.0f - ldexpf(1.0f, -m), (1 << ebits) - 1 - ebias);
    for (int v = 0; v < 256; ++v)
      CHECK(orc_float_to_hfp8(orc_hfp8_to_float((uint8_t)v, ebits, ebias), ebits, ebias,
                              max_pos) == (uint8_t)v);
  }
  /* edge cases: all bags empty (N = 0), one bag, no bags */
  Batch e = make_batch(3, 5, 9, 100, dims3);
  run_tbe(&e);
  run_nbit(&e, tys5);
  free_batch(&e);
  Batch one = make_batch(1, 1, 40, 0, dims3);
  run_tbe(&one);
  free_batch(&one);
  Batch none = make_batch(2, 0, 5, 0, dims3);
  run_tbe(&none);
  free_batch(&none);
  run_codecs(7, 33);
  run_codecs(1, 1);
  run_codecs(3, 128);
  printf("san_driver: ok\n");
  return 0;
}
