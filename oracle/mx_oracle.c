/*
 * mx_oracle.c -- TEST INFRASTRUCTURE ONLY.  A plain, single-threaded C
 * restatement of the operators the HIP kernels implement, used by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker.
 * Nothing in the product links, loads or calls this file.
 *
 * The reference snapshot (/root/reference) contains no FBGEMM code; each
 * function follows the in-container statement of the algorithm it cites:
 *   torch/include/fbgemm/FbgemmEmbedding.h (FBGEMM's CPU embedding kernels,
 *   the CPU path fbgemm_gpu's TBE ops wrap), and the recalled fbgemm_gpu
 *   semantics of transpose_embedding_input and rowwise Adagrad.
 * Floating point is compiled with -ffp-contract=off: every fmaf() below is
 * deliberate, every other product is rounded on its own.
 *
 * Pins (tests/test_oracle_*.py): FBGEMM's exported CPU kernels called through
 * oracle/fbgemm_cpu.cpp, torch.nn.functional.embedding_bag, torch autograd,
 * numpy brute force, and closed forms.
 */
#include "mx_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---- fp16 helpers (IEEE binary16, round to nearest even) ----------------- */

float orc_half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  const uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: normalise */
      int e = -1;
      uint32_t m = man;
      do {
        ++e;
        m <<= 1;
      } while ((m & 0x400u) == 0);
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((m & 0x3ffu) << 13);
    }
  } else if (exp == 0x1f) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* bfloat16 of f as FBGEMM's CPU embedding kernels write bf16 output: the
 * top half of f's bits after adding 0x8000, i.e. to nearest with ties away
 * from zero (matched bit for bit against their is_bf16_out output, where
 * every tie went away from zero and every other value to nearest); NaN stays
 * a quiet NaN. */
uint16_t orc_float_to_bf16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
  return (uint16_t)((x + 0x8000u) >> 16);
}

uint16_t orc_float_to_half(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u); /* NaN */
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to inf */
  if (ax < 0x38800000u) { /* result is subnormal or zero */
    if (ax < 0x33000000u) return sign; /* below half the smallest subnormal */
    const uint32_t e = ax >> 23;
    const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    /* value = m * 2^(e-150); in units of 2^-24 that is m >> (126 - e) */
    const int shift = 126 - (int)e; /* 14..24 */
    const uint32_t rem = m & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    uint32_t r = m >> shift;
    if (rem > half || (rem == half && (r & 1u))) ++r;
    return (uint16_t)(sign | r);
  }
  /* normal */
  uint32_t r = ((ax >> 13) - ((127 - 15) << 10));
  const uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
  return (uint16_t)(sign | r);
}

/* ---- TBE forward ------------------------------------------------------------
 * FbgemmEmbedding.h:26-39: out[i] = sum_j in[indices[j]] (times weights[j]);
 * if normalize_by_lengths and len > 0: out /= len.  Applied per table with
 * the TBE layout: bag (t, b) is offsets[t*B+b] .. offsets[t*B+b+1], the
 * result lands in out[b, D_off[t] : D_off[t+1]].  Weighted rows accumulate
 * with one fma each (what FBGEMM's vfmadd does); MEAN multiplies by the
 * float reciprocal of L. */
void orc_tbe_forward_f32(const float* W, const int64_t* w_off, const int32_t* D_off, int32_t T,
                         int64_t B, const int64_t* indices, const int64_t* offsets,
                         int32_t pooling, const float* iw, float* out, int64_t total_D) {
  for (int32_t t = 0; t < T; ++t) {
    const int32_t D0 = D_off[t], D = D_off[t + 1] - D_off[t];
    const float* Wt = W + w_off[t];
    for (int64_t b = 0; b < B; ++b) {
      const int64_t s = offsets[t * B + b], e = offsets[t * B + b + 1];
      float* o = out + b * total_D + D0;
      for (int32_t d = 0; d < D; ++d) o[d] = 0.0f;
      for (int64_t l = s; l < e; ++l) {
        const float* row = Wt + indices[l] * D;
        if (iw) {
          for (int32_t d = 0; d < D; ++d) o[d] = fmaf(iw[l], row[d], o[d]);
        } else {
          for (int32_t d = 0; d < D; ++d) o[d] = o[d] + row[d];
        }
      }
      if (pooling == ORC_POOL_MEAN && e > s) {
        const float inv = 1.0f / (float)(e - s);
        for (int32_t d = 0; d < D; ++d) o[d] = o[d] * inv;
      }
    }
  }
}

/* ---- hfp8 ---------------------------------------------------------------------
 * FBGEMM's 8-bit float of the nbit TBE (SparseType FP8; fbgemm::Float8ToFloat_ref
 * and FloatToFloat8_ref, torch/include/fbgemm/FbgemmConvert.h:181-200): a sign
 * bit, `ebits` exponent bits and m = 7 - ebits mantissa bits, exponent bias
 * `ebias`, subnormals where the exponent field is 0, no infinity or NaN codes:
 *   E > 0: (-1)^s * 2^(E - ebias) * (1 + M / 2^m)
 *   E = 0: (-1)^s * 2^(1 - ebias) * M / 2^m
 * Every code is exact in fp32.  Encoding clamps |x| to max_pos, then rounds
 * to the nearest code, ties to even (the grid of x's binade, or the
 * subnormal grid below 2^(1 - ebias)); NaN inputs are not defined. */
float orc_hfp8_to_float(uint8_t v, int32_t ebits, int32_t ebias) {
  const int m = 7 - ebits;
  const int E = (v & 0x7f) >> m, M = v & ((1 << m) - 1);
  const float a = E > 0 ? ldexpf(1.0f + ldexpf((float)M, -m), E - ebias)
                        : ldexpf((float)M, 1 - ebias - m);
  return (v & 0x80) ? -a : a;
}

uint8_t orc_float_to_hfp8(float x, int32_t ebits, int32_t ebias, float max_pos) {
  const int m = 7 - ebits;
  const uint8_t s = signbit(x) ? 0x80 : 0;
  float a = fabsf(x);
  if (a > max_pos) a = max_pos;
  if (a < ldexpf(1.0f, 1 - ebias)) /* subnormal grid, quantum 2^(1 - ebias - m) */
    return (uint8_t)(s | (uint8_t)rintf(ldexpf(a, ebias + m - 1)));
  int e;
  (void)frexpf(a, &e); /* a in [2^(e-1), 2^e) */
  const float k = rintf(ldexpf(a, m - (e - 1))); /* in [2^m, 2^(m+1)] */
  int E = e - 1 + ebias, M = (int)k - (1 << m);
  if (M == (1 << m)) { /* rounded up into the next binade */
    E += 1;
    M = 0;
  }
  return (uint8_t)(s | (uint8_t)((E << m) | M));
}

/* ---- nbit forward -------------------------------------------------------------
 * Row (t, i) starts at byte w_off[t] + i * stride_t, stride_t =
 * round_up(unpadded, row_align).  Quantized rows carry an fp16 scale and
 * fp16 bias first (scale_bias_last = false, FbgemmEmbedding.h:88-92,
 * 144-149); INT4/INT2 pack element 0 in the lowest bits.  Per element the
 * accumulator takes bias then scale*q in one fma, the order of FBGEMM's
 * rowwise kernels: acc = fma(scale, q, acc + bias). */
int64_t orc_nbit_row_bytes(int32_t ty, int32_t D, int32_t row_align) {
  int64_t u;
  switch (ty) {
    case ORC_FP32: u = 4ll * D; break;
    case ORC_FP16: u = 2ll * D; break;
    case ORC_INT8: u = D + 4ll; break;
    case ORC_INT4: u = D / 2 + 4ll; break;
    case ORC_INT2: u = D / 4 + 4ll; break;
    case ORC_FP8: u = D; break;
    default: return -1;
  }
  if (row_align > 1) u = (u + row_align - 1) / row_align * row_align;
  return u;
}

static float nbit_code(const uint8_t* codes, int32_t ty, int32_t d, int32_t ebits,
                       int32_t ebias) {
  switch (ty) {
    case ORC_FP8: return orc_hfp8_to_float(codes[d], ebits, ebias);
    case ORC_FP32: {
      float f;
      memcpy(&f, codes + 4 * d, 4);
      return f;
    }
    case ORC_FP16: {
      uint16_t h;
      memcpy(&h, codes + 2 * d, 2);
      return orc_half_to_float(h);
    }
    case ORC_INT8: return (float)codes[d];
    case ORC_INT4: return (float)((codes[d >> 1] >> ((d & 1) * 4)) & 0xf);
    default: return (float)((codes[d >> 2] >> ((d & 3) * 2)) & 0x3);
  }
}

int orc_nbit_forward(const uint8_t* W, const int64_t* w_off, const uint8_t* tys,
                     const int32_t* D_off, int32_t T, int64_t B, const int64_t* indices,
                     const int64_t* offsets, int32_t pooling, const float* iw, int32_t row_align,
                     int32_t out_kind, void* out, int64_t total_D, int32_t fp8_ebits,
                     int32_t fp8_ebias) {
  float* acc = NULL;
  for (int32_t t = 0; t < T; ++t) {
    const int32_t ty = tys[t];
    const int32_t D0 = D_off[t], D = D_off[t + 1] - D_off[t];
    const int64_t stride = orc_nbit_row_bytes(ty, D, row_align);
    if (stride < 0) {
      free(acc);
      return -1;
    }
    const int quant = ty == ORC_INT8 || ty == ORC_INT4 || ty == ORC_INT2;
    float* tmp = (float*)realloc(acc, sizeof(float) * (D > 0 ? D : 1));
    if (!tmp) {
      free(acc);
      return -2;
    }
    acc = tmp;
    for (int64_t b = 0; b < B; ++b) {
      const int64_t s = offsets[t * B + b], e = offsets[t * B + b + 1];
      for (int32_t d = 0; d < D; ++d) acc[d] = 0.0f;
      for (int64_t l = s; l < e; ++l) {
        const uint8_t* row = W + w_off[t] + indices[l] * stride;
        const float wgt = iw ? iw[l] : 1.0f;
        if (quant) {
          uint16_t hs, hb;
          memcpy(&hs, row, 2);
          memcpy(&hb, row + 2, 2);
          float scale = orc_half_to_float(hs), bias = orc_half_to_float(hb);
          if (iw) {
            scale = scale * wgt;
            bias = bias * wgt;
          }
          for (int32_t d = 0; d < D; ++d) acc[d] = fmaf(scale, nbit_code(row + 4, ty, d, 0, 0), acc[d] + bias);
        } else {
          for (int32_t d = 0; d < D; ++d) {
            const float v = nbit_code(row, ty, d, fp8_ebits, fp8_ebias);
            acc[d] = iw ? fmaf(wgt, v, acc[d]) : acc[d] + v;
          }
        }
      }
      if (pooling == ORC_POOL_MEAN && e > s) {
        const float inv = 1.0f / (float)(e - s);
        for (int32_t d = 0; d < D; ++d) acc[d] = acc[d] * inv;
      }
      if (out_kind == 1 || out_kind == 2) { /* fp16, bf16 */
        uint16_t* o = (uint16_t*)out + b * total_D + D0;
        for (int32_t d = 0; d < D; ++d)
          o[d] = out_kind == 1 ? orc_float_to_half(acc[d]) : orc_float_to_bf16(acc[d]);
      } else {
        float* o = (float*)out + b * total_D + D0;
        for (int32_t d = 0; d < D; ++d) o[d] = acc[d];
      }
    }
  }
  free(acc);
  return 0;
}

/* ---- transpose_embedding_input -----------------------------------------------
 * linear[l] = hash_size_cumsum[t] + indices[l]; info[l] = (t << nb) | b;
 * (linear, info) pairs sorted stably on the low `bits` bits of linear;
 * runs = maximal blocks of equal keys, with their lengths and the exclusive
 * cumsum of the lengths (recalled fbgemm_gpu transpose_embedding_input:
 * linearize_index_kernel, radix_sort_pairs, RunLengthEncode,
 * asynchronous_complete_cumsum).  Stable merge sort on (masked key, position). */
static const int64_t* g_sort_keys;
static uint64_t g_sort_mask;

static void merge_sort(int64_t* a, int64_t* tmp, int64_t n) {
  if (n < 2) return;
  const int64_t h = n / 2;
  merge_sort(a, tmp, h);
  merge_sort(a + h, tmp, n - h);
  int64_t i = 0, j = h, k = 0;
  while (i < h && j < n) {
    const uint64_t ki = (uint64_t)g_sort_keys[a[i]] & g_sort_mask;
    const uint64_t kj = (uint64_t)g_sort_keys[a[j]] & g_sort_mask;
    if (kj < ki)
      tmp[k++] = a[j++];
    else
      tmp[k++] = a[i++]; /* ties keep the earlier position: stable */
  }
  while (i < h) tmp[k++] = a[i++];
  while (j < n) tmp[k++] = a[j++];
  memcpy(a, tmp, sizeof(int64_t) * n);
}

/* pos (optional): pos[i] = position in `indices` of the i-th sorted entry. */
static int transpose_impl(const int64_t* hsc, int32_t T, int64_t B, int32_t nb, int32_t bits,
                          const int64_t* indices, const int64_t* offsets, int64_t N,
                          int64_t* linear, int64_t* sorted, int32_t* infos, int64_t* run,
                          int32_t* run_lengths, int64_t* num_runs, int32_t* cum, int64_t* pos) {
  uint32_t* info_raw = (uint32_t*)malloc(sizeof(uint32_t) * (N > 0 ? N : 1));
  int64_t* perm = (int64_t*)malloc(sizeof(int64_t) * (N > 0 ? N : 1));
  int64_t* tmp = (int64_t*)malloc(sizeof(int64_t) * (N > 0 ? N : 1));
  if (!info_raw || !perm || !tmp) {
    free(info_raw);
    free(perm);
    free(tmp);
    return -2;
  }
  for (int32_t t = 0; t < T; ++t)
    for (int64_t b = 0; b < B; ++b)
      for (int64_t l = offsets[t * B + b]; l < offsets[t * B + b + 1]; ++l) {
        linear[l] = hsc[t] + indices[l];
        info_raw[l] = (nb >= 32 ? 0u : ((uint32_t)t << nb)) | (uint32_t)b;
      }
  for (int64_t l = 0; l < N; ++l) perm[l] = l;
  g_sort_keys = linear;
  g_sort_mask = bits >= 64 ? ~0ull : ((1ull << bits) - 1ull);
  merge_sort(perm, tmp, N);
  int64_t r = -1;
  for (int64_t i = 0; i < N; ++i) {
    sorted[i] = linear[perm[i]];
    infos[i] = (int32_t)info_raw[perm[i]];
    if (pos) pos[i] = perm[i];
    if (i == 0 || sorted[i] != sorted[i - 1]) {
      ++r;
      run[r] = sorted[i];
      cum[r] = (int32_t)i;
    }
  }
  *num_runs = r + 1;
  /* Past the runs the arrays are the complete cumsum of the zero-padded
   * lengths: cum = N, run_lengths = 0 (cum has N+1 entries, run_lengths N). */
  for (int64_t k = r + 1; k <= N; ++k) cum[k] = (int32_t)N;
  for (int64_t k = 0; k < N; ++k) run_lengths[k] = k <= r ? cum[k + 1] - cum[k] : 0;
  free(info_raw);
  free(perm);
  free(tmp);
  return 0;
}

int orc_transpose(const int64_t* hsc, int32_t T, int64_t B, int32_t nb, int32_t bits,
                  const int64_t* indices, const int64_t* offsets, int64_t N, int64_t* linear,
                  int64_t* sorted, int32_t* infos, int64_t* run, int32_t* run_lengths,
                  int64_t* num_runs, int32_t* cum) {
  return transpose_impl(hsc, T, B, nb, bits, indices, offsets, N, linear, sorted, infos, run,
                        run_lengths, num_runs, cum, NULL);
}

/* ---- backward + exact rowwise Adagrad --------------------------------------
 * For each run (distinct (t, i)), in sorted order of its occurrences:
 *   g_d  = sum grad_output[b, D_off[t] + d]      (MEAN: each term * (1/L),
 *                                                 weighted: then * iw[l])
 *   L2 (mode 1):   s_d = g_d + wd * w_d,  else s_d = g_d
 *   h   += (sum_d s_d^2) / D
 *   m    = lr / (sqrtf(h) + eps)
 *   c    = 1 (mode 0), 1 - m*wd (mode 1), 1 - lr*wd (mode 2)
 *   w_d  = fmaf(-m, g_d, c * w_d)
 * (recalled rowwise_adagrad rule of fbgemm_gpu's optimizer templates). */
static void adagrad_row(float* w, float* h, const float* g, int32_t D, float lr, float eps,
                        float wd, int32_t wd_mode) {
  float ss = 0.0f;
  for (int32_t d = 0; d < D; ++d) {
    const float s = wd_mode == 1 ? fmaf(wd, w[d], g[d]) : g[d];
    ss = ss + s * s;
  }
  const float hn = *h + ss / (float)D;
  const float m = lr / (sqrtf(hn) + eps);
  float c = 1.0f;
  if (wd_mode == 1) c = 1.0f - m * wd;
  if (wd_mode == 2) c = 1.0f - lr * wd;
  for (int32_t d = 0; d < D; ++d) w[d] = fmaf(-m, g[d], c * w[d]);
  *h = hn;
}

int orc_backward_rowwise_adagrad(float* W, const int64_t* w_off, const int32_t* D_off,
                                 int32_t T, int64_t B, const int64_t* hsc, int32_t bits,
                                 const int64_t* indices, const int64_t* offsets, int64_t N,
                                 int32_t pooling, const float* iw, const float* grad,
                                 int64_t total_D, float* m1,
                                 const int64_t* m1_off, float lr, float eps, float wd,
                                 int32_t wd_mode, int32_t nb) {
  const int64_t n = N > 0 ? N : 1;
  int64_t* linear = (int64_t*)malloc(sizeof(int64_t) * n);
  int64_t* sorted = (int64_t*)malloc(sizeof(int64_t) * n);
  int32_t* infos = (int32_t*)malloc(sizeof(int32_t) * n);
  int64_t* run = (int64_t*)malloc(sizeof(int64_t) * n);
  int32_t* lens = (int32_t*)malloc(sizeof(int32_t) * n);
  int32_t* cum = (int32_t*)malloc(sizeof(int32_t) * (n + 1));
  int64_t* pos = (int64_t*)malloc(sizeof(int64_t) * n);
  float* g = (float*)malloc(sizeof(float) * 1024);
  int rc = 0;
  if (!linear || !sorted || !infos || !run || !lens || !cum || !pos || !g) {
    rc = -2;
    goto done;
  }
  int64_t nruns = 0;
  if (N > 0) {
    rc = transpose_impl(hsc, T, B, nb, bits, indices, offsets, N, linear, sorted, infos, run,
                        lens, &nruns, cum, pos);
    if (rc) goto done;
  }
  const uint32_t bmask = nb >= 32 ? 0xffffffffu : ((1u << nb) - 1u);
  for (int64_t r = 0; r < nruns; ++r) {
    /* The row: from the run's first occurrence (features that share a table
     * share its rows, hash offset and width).  Each occurrence's gradient
     * slice and bag length: from its own feature tj. */
    const uint32_t info0 = (uint32_t)infos[cum[r]];
    const int64_t t = nb >= 32 ? 0 : (int64_t)(info0 >> nb);
    const int32_t D = D_off[t + 1] - D_off[t];
    if (D > 1024) {
      rc = -1;
      goto done;
    }
    const int64_t idx = run[r] - hsc[t];
    for (int32_t d = 0; d < D; ++d) g[d] = 0.0f;
    for (int32_t j = cum[r]; j < cum[r + 1]; ++j) {
      const int64_t tj = nb >= 32 ? 0 : (int64_t)((uint32_t)infos[j] >> nb);
      if (D_off[tj + 1] - D_off[tj] != D) {
        rc = -1; /* one key, two widths: not one table */
        goto done;
      }
      const int64_t b = (int64_t)((uint32_t)infos[j] & bmask);
      const float* gr = grad + b * total_D + D_off[tj];
      const int64_t L = offsets[tj * B + b + 1] - offsets[tj * B + b];
      const float sc = pooling == ORC_POOL_MEAN ? 1.0f / (float)L : 1.0f; /* L >= 1 here */
      const float wl = iw ? iw[pos[j]] : 1.0f;
      for (int32_t d = 0; d < D; ++d) g[d] = g[d] + (gr[d] * sc) * wl;
    }
    adagrad_row(W + w_off[t] + idx * D, m1 + m1_off[t] + idx, g, D, lr, eps, wd, wd_mode);
  }
done:
  free(linear);
  free(sorted);
  free(infos);
  free(run);
  free(lens);
  free(cum);
  free(pos);
  free(g);
  return rc;
}

/* ---- gradient of the per-sample weights ------------------------------------
 * giw[l] = sum_d grad_output[b, D_off[t] + d] * W_t[indices[l], d], d ascending,
 * times 1/L under MEAN; 0 for tables with frg[t] == 0 (frg may be NULL).
 * Summation order differs from the GPU's (tree over lanes): compare at rtol. */
void orc_grad_indice_weights(const float* grad, int64_t total_D, const float* W,
                             const int64_t* w_off, const int32_t* D_off, int32_t T, int64_t B,
                             const int64_t* indices, const int64_t* offsets, int32_t pooling,
                             const int32_t* frg, float* giw) {
  for (int32_t t = 0; t < T; ++t) {
    const int32_t D0 = D_off[t], D = D_off[t + 1] - D_off[t];
    for (int64_t b = 0; b < B; ++b) {
      const int64_t s = offsets[t * B + b], e = offsets[t * B + b + 1];
      const float sc = pooling == ORC_POOL_MEAN && e > s ? 1.0f / (float)(e - s) : 1.0f;
      for (int64_t l = s; l < e; ++l) {
        if (frg && frg[t] == 0) {
          giw[l] = 0.0f;
          continue;
        }
        const float* row = W + w_off[t] + indices[l] * D;
        const float* gr = grad + b * total_D + D0;
        double acc = 0.0;
        for (int32_t d = 0; d < D; ++d) acc += (double)gr[d] * (double)row[d];
        giw[l] = pooling == ORC_POOL_MEAN ? (float)acc * sc : (float)acc;
      }
    }
  }
}

/* ---- bounds_check_indices -------------------------------------------------
 * fbgemm_gpu bounds_check_indices (recalled), modes FATAL 0 / WARNING 1 /
 * IGNORE 2 / NONE 3, with this build's stated repair contract: offsets
 * o'[i] = max_{j<=i} clamp(o[j], 0, N); indices of bag (t, b) -- positions
 * [o'[t*B+b], o'[t*B+b+1]) -- outside [0, rows[t]) set to 0; each repaired
 * entry counts one; FATAL counts without repairing. */
int64_t orc_bounds_check(const int64_t* rows, int32_t T, int64_t B, int64_t* indices,
                         int64_t* offsets, int64_t N, int32_t mode) {
  if (mode == 3) return 0;
  int64_t bad = 0;
  const int64_t nb = (int64_t)T * B;
  int64_t* rep = (int64_t*)malloc(sizeof(int64_t) * (nb + 1));
  if (!rep) return -1;
  int64_t run = 0;
  for (int64_t i = 0; i <= nb; ++i) {
    const int64_t c = offsets[i] < 0 ? 0 : (offsets[i] > N ? N : offsets[i]);
    run = c > run ? c : run;
    rep[i] = run;
  }
  for (int64_t bag = 0; bag < nb; ++bag) {
    const int64_t t = bag / B;
    for (int64_t l = rep[bag]; l < rep[bag + 1]; ++l) {
      if (indices[l] < 0 || indices[l] >= rows[t]) {
        ++bad;
        if (mode != 0) indices[l] = 0;
      }
    }
  }
  for (int64_t i = 0; i <= nb; ++i) {
    if (rep[i] != offsets[i]) {
      ++bad;
      if (mode != 0) offsets[i] = rep[i];
    }
  }
  free(rep);
  return bad;
}

/* ---- rowwise quantization codecs -------------------------------------------
 * FBGEMM's FloatOrHalfToFused8BitRowwiseQuantizedSBFloat and
 * FloatOrHalfToFusedNBitRowwiseQuantizedSBHalf (declared in
 * torch/include/fbgemm/QuantUtils.h), as fbgemm_gpu's
 * FloatToFused8BitRowwiseQuantized / FloatToFusedNBitRowwiseQuantizedSBHalf
 * use them:
 *   8-bit: scale = (max - min) / 255, q = rint((x - min) * (255 / (range +
 *          1e-8))), row = D codes + fp32 scale + fp32 bias(=min);
 *   N-bit: bias = half(min), scale = half((max - bias) / (2^b - 1)) (1 when
 *          the range is 0, or when the scale underflows / its inverse
 *          overflows), q = clamp(rint((x - bias) / scale'), 0, 2^b - 1) with
 *          scale' = 1/scale computed once, packed low bits first, row =
 *          ceil(D*b/8) bytes + fp16 scale + fp16 bias. */
void orc_quantize_8bit(const float* x, int64_t rows, int64_t D, uint8_t* out) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* v = x + r * D;
    uint8_t* o = out + r * (D + 8);
    float mn = INFINITY, mx = -INFINITY;
    for (int64_t j = 0; j < D; ++j) {
      mn = v[j] < mn ? v[j] : mn;
      mx = v[j] > mx ? v[j] : mx;
    }
    const float range = mx - mn;
    const float scale = range / 255.0f;
    const float inv = 255.0f / (range + 1e-8f);
    for (int64_t j = 0; j < D; ++j) o[j] = (uint8_t)rintf((v[j] - mn) * inv);
    memcpy(o + D, &scale, 4);
    memcpy(o + D + 4, &mn, 4);
  }
}

void orc_dequantize_8bit(const uint8_t* in, int64_t rows, int64_t D, float* out) {
  for (int64_t r = 0; r < rows; ++r) {
    const uint8_t* q = in + r * (D + 8);
    float scale, bias;
    memcpy(&scale, q + D, 4);
    memcpy(&bias, q + D + 4, 4);
    for (int64_t j = 0; j < D; ++j) out[r * D + j] = fmaf((float)q[j], scale, bias);
  }
}

void orc_quantize_nbit(const float* x, int64_t rows, int64_t D, int32_t bits, uint8_t* out) {
  const int per = 8 / bits;
  const int64_t nbytes = (D + per - 1) / per;
  const int qmax = (1 << bits) - 1;
  for (int64_t r = 0; r < rows; ++r) {
    const float* v = x + r * D;
    uint8_t* o = out + r * (nbytes + 4);
    float mn = INFINITY, mx = -INFINITY;
    for (int64_t j = 0; j < D; ++j) {
      mn = v[j] < mn ? v[j] : mn;
      mx = v[j] > mx ? v[j] : mx;
    }
    const float bias = orc_half_to_float(orc_float_to_half(mn));
    const float range = mx - bias;
    float scale = range == 0.0f ? 1.0f : range / (float)qmax;
    scale = orc_half_to_float(orc_float_to_half(scale));
    if (scale == 0.0f) scale = 1.0f;
    float inv = 1.0f / scale;
    if (isinf(inv)) {
      scale = 1.0f;
      inv = 1.0f;
    }
    memset(o, 0, nbytes);
    for (int64_t j = 0; j < D; ++j) {
      float q = rintf((v[j] - bias) * inv);
      q = q < 0.0f ? 0.0f : (q > (float)qmax ? (float)qmax : q);
      o[j / per] |= (uint8_t)((uint32_t)q << ((j % per) * bits));
    }
    const uint16_t hs = orc_float_to_half(scale), hb = orc_float_to_half(bias);
    memcpy(o + nbytes, &hs, 2);
    memcpy(o + nbytes + 2, &hb, 2);
  }
}

void orc_dequantize_nbit(const uint8_t* in, int64_t rows, int64_t D, int32_t bits, float* out) {
  const int per = 8 / bits;
  const int64_t nbytes = (D + per - 1) / per;
  for (int64_t r = 0; r < rows; ++r) {
    const uint8_t* q = in + r * (nbytes + 4);
    uint16_t hs, hb;
    memcpy(&hs, q + nbytes, 2);
    memcpy(&hb, q + nbytes + 2, 2);
    const float scale = orc_half_to_float(hs), bias = orc_half_to_float(hb);
    for (int64_t j = 0; j < D; ++j) {
      const uint32_t c = (q[j / per] >> ((j % per) * bits)) & ((1u << bits) - 1u);
      out[r * D + j] = fmaf((float)c, scale, bias);
    }
  }
}

/* ---- sequence lookups (PoolingMode NONE) -------------------------------------
 * Every table of width D; position l of bag (t, b) is its own occurrence
 * (recalled fbgemm_gpu nobag kernels). */

/* out[l, :] = the dequantized row of position l: fmaf(scale, q, bias) for
 * INT8/INT4/INT2, the stored value for FP32/FP16/FP8; then the output type
 * (out_kind 0 fp32, 1 fp16, 2 bf16).  Positions outside every bag stay as
 * the caller left them. */
int orc_nbit_forward_nobag(const uint8_t* W, const int64_t* w_off, const uint8_t* tys,
                           int32_t D, int32_t T, int64_t B, const int64_t* indices,
                           const int64_t* offsets, int32_t row_align, int32_t out_kind,
                           void* out, int32_t fp8_ebits, int32_t fp8_ebias) {
  for (int32_t t = 0; t < T; ++t) {
    const int32_t ty = tys[t];
    const int64_t stride = orc_nbit_row_bytes(ty, D, row_align);
    if (stride < 0) return -1;
    const int quant = ty == ORC_INT8 || ty == ORC_INT4 || ty == ORC_INT2;
    for (int64_t l = offsets[t * B]; l < offsets[(t + 1) * B]; ++l) {
      const uint8_t* row = W + w_off[t] + indices[l] * stride;
      float scale = 0.0f, bias = 0.0f;
      if (quant) {
        uint16_t hs, hb;
        memcpy(&hs, row, 2);
        memcpy(&hb, row + 2, 2);
        scale = orc_half_to_float(hs);
        bias = orc_half_to_float(hb);
      }
      for (int32_t d = 0; d < D; ++d) {
        const float v = quant ? fmaf(scale, nbit_code(row + 4, ty, d, 0, 0), bias)
                              : nbit_code(row, ty, d, fp8_ebits, fp8_ebias);
        if (out_kind == 1 || out_kind == 2)
          ((uint16_t*)out)[l * D + d] = out_kind == 1 ? orc_float_to_half(v) : orc_float_to_bf16(v);
        else
          ((float*)out)[l * D + d] = v;
      }
    }
  }
  return 0;
}

/* The nobag backward: keys hsc[t] + indices[l] stably sorted (ties in
 * position order); each run sums grad[l, :] of its positions in that order,
 * then the rowwise Adagrad step of orc_backward_rowwise_adagrad. */
int orc_backward_rowwise_adagrad_nobag(float* W, const int64_t* w_off, int32_t D, int32_t T,
                                       int64_t B, const int64_t* hsc, int32_t bits,
                                       const int64_t* indices, const int64_t* offsets, int64_t N,
                                       const float* grad, float* m1, const int64_t* m1_off,
                                       float lr, float eps, float wd, int32_t wd_mode,
                                       int32_t nb) {
  const int64_t n = N > 0 ? N : 1;
  int64_t* linear = (int64_t*)malloc(sizeof(int64_t) * n);
  int64_t* sorted = (int64_t*)malloc(sizeof(int64_t) * n);
  int32_t* infos = (int32_t*)malloc(sizeof(int32_t) * n);
  int64_t* run = (int64_t*)malloc(sizeof(int64_t) * n);
  int32_t* lens = (int32_t*)malloc(sizeof(int32_t) * n);
  int32_t* cum = (int32_t*)malloc(sizeof(int32_t) * (n + 1));
  int64_t* pos = (int64_t*)malloc(sizeof(int64_t) * n);
  float* g = (float*)malloc(sizeof(float) * (D > 0 ? D : 1));
  int rc = 0;
  if (!linear || !sorted || !infos || !run || !lens || !cum || !pos || !g) {
    rc = -2;
    goto done;
  }
  int64_t nruns = 0;
  if (N > 0) {
    rc = transpose_impl(hsc, T, B, nb, bits, indices, offsets, N, linear, sorted, infos, run,
                        lens, &nruns, cum, pos);
    if (rc) goto done;
  }
  for (int64_t r = 0; r < nruns; ++r) {
    const uint32_t info0 = (uint32_t)infos[cum[r]];
    const int64_t t = nb >= 32 ? 0 : (int64_t)(info0 >> nb);
    const int64_t idx = run[r] - hsc[t];
    for (int32_t d = 0; d < D; ++d) g[d] = 0.0f;
    for (int32_t j = cum[r]; j < cum[r + 1]; ++j) {
      const float* gr = grad + pos[j] * D;
      for (int32_t d = 0; d < D; ++d) g[d] = g[d] + gr[d];
    }
    adagrad_row(W + w_off[t] + idx * D, m1 + m1_off[t] + idx, g, D, lr, eps, wd, wd_mode);
  }
done:
  free(linear);
  free(sorted);
  free(infos);
  free(run);
  free(lens);
  free(cum);
  free(pos);
  free(g);
  return rc;
}
