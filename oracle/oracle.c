/*
 * oracle.c - scalar CPU restatement of the reference's non-GEMM layer kernels.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h): the checker for libllmk's HIP kernels, never part of
 * the product path.
 *
 * Pinning (what each function is checked against, besides the GPU it checks):
 *   or_h2f / or_f2h          exhaustive: all 65536 halves vs numpy; all 2^32 floats vs F16C
 *   or_embedding_lookup      numpy fancy indexing (bit-exact); Hugging Face nn.Embedding fixture
 *   or_residual_add          numpy float16 addition (bit-exact); the reference's own
 *                            known-answer test (xorshift32 seed 12345, n = 1,000,003)
 *   or_rmsnorm/add_rmsnorm   Hugging Face LlamaRMSNorm fixture (tolerance); closed form for
 *                            constant rows; float64 evaluation; residual output bit-exact
 *   or_compute_rope_inv_freq Hugging Face llama3 rope-init fixture (rel <= 1e-5); closed-form
 *                            special cases (i = 0 -> 1; long wavelengths -> f / factor)
 *   or_rope_apply            Hugging Face LlamaRotaryEmbedding + apply_rotary_pos_emb fixture;
 *                            pos = 0 is the identity; a quarter turn swaps the halves
 *   or_swiglu                torch silu * up fixture; g = 0 -> 0; large |g| limits
 *   or_kv_scatter(_batch)    numpy scatter by the closed-form row address; untouched rows keep
 *                            their 0x7F7F poison; exactly T (or n) rows change
 *   or_linear                float64 matmul of the same fp16 inputs (error within the fp32
 *                            summation bound); identity and one-hot weights select exact
 *                            columns; torch.nn.functional.linear on the CPU in float32
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------------------------ */
/* binary16 conversions, from the IEEE 754 binary16 / binary32 encodings                       */
/* ------------------------------------------------------------------------------------------ */

static inline uint32_t f_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float bits_f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

float or_h2f(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
  if (e == 0x1F) return bits_f(sign | 0x7F800000u | (m << 13)); /* inf / NaN */
  if (e == 0) {
    /* zero or subnormal: m * 2^-24, exact in binary32 */
    const float v = (float)m * 0x1p-24f;
    return bits_f(sign | f_bits(v));
  }
  return bits_f(sign | ((e + 112u) << 23) | (m << 13)); /* rebias 15 -> 127 */
}

uint16_t or_f2h(float f) {
  const uint32_t x = f_bits(f);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t ax = x & 0x7FFFFFFFu;
  if (ax > 0x7F800000u) /* NaN: quiet, keep the top payload bits */
    return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu));
  if (ax >= 0x477FF000u) /* >= 65520 rounds to infinity (65520 is the tie to even 2^16) */
    return (uint16_t)(sign | 0x7C00u);
  if (ax >= 0x38800000u) { /* normal half: |f| >= 2^-14 */
    const uint32_t v = ax - 0x38000000u; /* rebias exponent 127 -> 15 */
    uint32_t r = v >> 13;
    const uint32_t rem = v & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r; /* carry may bump the exponent */
    return (uint16_t)(sign | r);
  }
  if (ax <= 0x33000000u) return sign; /* <= 2^-25: rounds to zero (2^-25 ties to even 0) */
  { /* subnormal half: round |f| / 2^-24 to an integer */
    const uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
    const int e = (int)(ax >> 23) - 127; /* -25 .. -15 */
    const int shift = -e - 1;            /* 14 .. 24 */
    uint32_t r = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u), halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (r & 1u))) ++r;
    return (uint16_t)(sign | r);
  }
}

void or_h2f_array(const uint16_t* in, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = or_h2f(in[i]);
}
void or_f2h_array(const float* in, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = or_f2h(in[i]);
}

/* r16(x): round an fp32 value to fp16 and back. */
static inline float r16(float x) { return or_h2f(or_f2h(x)); }

/* ------------------------------------------------------------------------------------------ */
/* the ops                                                                                      */
/* ------------------------------------------------------------------------------------------ */

void or_embedding_lookup(const uint16_t* table, const int32_t* ids, uint16_t* out, int n_tokens,
                         int hidden) {
  for (int t = 0; t < n_tokens; ++t)
    memcpy(out + (size_t)t * hidden, table + (size_t)ids[t] * hidden, (size_t)hidden * 2);
}

void or_residual_add(const uint16_t* a, const uint16_t* b, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) {
    const float s = or_h2f(a[i]) + or_h2f(b[i]); /* fp32 add */
    out[i] = or_f2h(s);                          /* one rounding to fp16 */
  }
}

/* One row of RMSNorm on already-final fp16 values h[0..hidden). */
static void norm_row(const uint16_t* h, const uint16_t* w, uint16_t* out, int hidden, float eps) {
  float ss = 0.0f; /* fp32 accumulation, in index order */
  for (int j = 0; j < hidden; ++j) {
    const float f = or_h2f(h[j]);
    ss = ss + f * f;
  }
  const float inv = 1.0f / sqrtf(ss / (float)hidden + eps);
  for (int j = 0; j < hidden; ++j) {
    const float a = r16(or_h2f(h[j]) * inv); /* normalise, round to fp16 ... */
    out[j] = or_f2h(or_h2f(w[j]) * a);      /* ... then scale by the weight */
  }
}

void or_rmsnorm(const uint16_t* x, const uint16_t* w, uint16_t* out, int n_rows, int hidden,
                float eps) {
  for (int r = 0; r < n_rows; ++r)
    norm_row(x + (size_t)r * hidden, w, out + (size_t)r * hidden, hidden, eps);
}

static void add_rmsnorm_rows(uint16_t* residual, const uint16_t* x, const uint16_t* w,
                             uint16_t* out, int r0, int r1, int hidden, float eps) {
  for (int r = r0; r < r1; ++r) {
    uint16_t* res = residual + (size_t)r * hidden;
    or_residual_add(res, x + (size_t)r * hidden, res, (size_t)hidden);
    norm_row(res, w, out + (size_t)r * hidden, hidden, eps);
  }
}

void or_add_rmsnorm(uint16_t* residual, const uint16_t* x, const uint16_t* w, uint16_t* out,
                    int n_rows, int hidden, float eps) {
  add_rmsnorm_rows(residual, x, w, out, 0, n_rows, hidden, eps);
}

void or_compute_rope_inv_freq(int head_dim, double theta, double factor, double low_freq_factor,
                              double high_freq_factor, double original_max_pos, float* out) {
  /* fp32 throughout, one operation at a time, as the reference's host routine */
  const float two_pi = (float)(2.0 * 3.14159265358979323846);
  const float th = (float)theta, fac = (float)factor;
  const float lo = (float)low_freq_factor, hi = (float)high_freq_factor;
  const float orig = (float)original_max_pos;
  const float wl_low = (float)(original_max_pos / low_freq_factor);
  const float wl_high = (float)(original_max_pos / high_freq_factor);
  for (int i = 0; i < head_dim / 2; ++i) {
    const float expo = (float)(2 * i) / (float)head_dim;
    const float f = 1.0f / powf(th, expo);
    const float wl = two_pi / f;
    const float base = (wl > wl_low) ? f / fac : f;
    const float smooth = (orig / wl - lo) / (hi - lo);
    const float smoothed = (1.0f - smooth) * base / fac + smooth * base;
    const int medium = !(wl < wl_high) && !(wl > wl_low);
    out[i] = medium ? smoothed : base;
  }
}

/* cos and sin of an fp32 angle, from libm in double, rounded to fp32 and then to fp16. */
static void cos_sin_r16(float a, float* c, float* s) {
  *c = r16((float)cos((double)a));
  *s = r16((float)sin((double)a));
}

static void rope_head(uint16_t* v, const float* c, const float* s, int half) {
  for (int i = 0; i < half; ++i) {
    const float x1 = or_h2f(v[i]), x2 = or_h2f(v[i + half]);
    v[i] = or_f2h(r16(x1 * c[i]) - r16(x2 * s[i]));
    v[i + half] = or_f2h(r16(x2 * c[i]) + r16(x1 * s[i]));
  }
}

static void rope_tokens(uint16_t* q, uint16_t* k, const int32_t* positions,
                        const float* inv_freq, int t0, int t1, int n_heads, int n_kv_heads,
                        int head_dim) {
  const int half = head_dim / 2;
  float* c = (float*)malloc(sizeof(float) * (size_t)half * 2);
  float* s = c + half;
  for (int t = t0; t < t1; ++t) {
    const float p = (float)positions[t];
    for (int i = 0; i < half; ++i) cos_sin_r16(p * inv_freq[i], &c[i], &s[i]);
    for (int h = 0; h < n_heads; ++h) rope_head(q + ((size_t)t * n_heads + h) * head_dim, c, s, half);
    for (int h = 0; h < n_kv_heads; ++h)
      rope_head(k + ((size_t)t * n_kv_heads + h) * head_dim, c, s, half);
  }
  free(c);
}

void or_rope_apply(uint16_t* q, uint16_t* k, const int32_t* positions, const float* inv_freq,
                   int n_tokens, int n_heads, int n_kv_heads, int head_dim) {
  rope_tokens(q, k, positions, inv_freq, 0, n_tokens, n_heads, n_kv_heads, head_dim);
}

static void swiglu_range(const uint16_t* gate, const uint16_t* up, uint16_t* out, size_t i0,
                         size_t i1) {
  for (size_t i = i0; i < i1; ++i) {
    const float g = or_h2f(gate[i]), u = or_h2f(up[i]);
    const float e = (float)exp(-(double)g);
    const float d = 1.0f + e;
    const float s = r16(g / d); /* silu rounded to fp16 before the multiply */
    out[i] = or_f2h(s * u);
  }
}

void or_swiglu(const uint16_t* gate, const uint16_t* up, uint16_t* out, size_t n) {
  swiglu_range(gate, up, out, 0, n);
}

void or_kv_scatter(const uint16_t* src, uint16_t* pool, const int32_t* block_table,
                   int start_pos, int T, int page_size, int kvdim) {
  for (int t = 0; t < T; ++t) {
    const int pos = start_pos + t;
    const size_t row = (size_t)block_table[pos / page_size] * page_size + (size_t)(pos % page_size);
    memcpy(pool + row * kvdim, src + (size_t)t * kvdim, (size_t)kvdim * 2);
  }
}

void or_kv_scatter_batch(const uint16_t* src, uint16_t* pool, const int32_t* block_tables,
                         const int32_t* positions, int n, int max_pages, int page_size,
                         int kvdim) {
  for (int b = 0; b < n; ++b) {
    const int pos = positions[b];
    const int32_t* table = block_tables + (size_t)b * max_pages;
    const size_t row = (size_t)table[pos / page_size] * page_size + (size_t)(pos % page_size);
    memcpy(pool + row * kvdim, src + (size_t)b * kvdim, (size_t)kvdim * 2);
  }
}

void or_rope_kv_scatter_batch(uint16_t* q, const uint16_t* k, const uint16_t* v,
                              uint16_t* k_pool, uint16_t* v_pool, const int32_t* block_tables,
                              const int32_t* positions, const float* inv_freq, int n,
                              int max_pages, int page_size, int n_heads, int n_kv_heads,
                              int head_dim) {
  const int kvdim = n_kv_heads * head_dim;
  uint16_t* kr = (uint16_t*)malloc((size_t)n * kvdim * 2);
  memcpy(kr, k, (size_t)n * kvdim * 2);
  or_rope_apply(q, kr, positions, inv_freq, n, n_heads, n_kv_heads, head_dim);
  or_kv_scatter_batch(kr, k_pool, block_tables, positions, n, max_pages, page_size, kvdim);
  or_kv_scatter_batch(v, v_pool, block_tables, positions, n, max_pages, page_size, kvdim);
  free(kr);
}

void or_attention_decode_paged(const uint16_t* q, const uint16_t* k_pool, const uint16_t* v_pool,
                               const int32_t* block_tables, const int32_t* seq_lens,
                               uint16_t* out, int n_seq, int max_pages, int page_size,
                               int n_heads, int n_kv_heads, int head_dim) {
  const int group = n_heads / n_kv_heads;
  const float scale = 1.0f / sqrtf((float)head_dim);
  const size_t kvrow = (size_t)n_kv_heads * head_dim;
  int max_s = 1;
  for (int s = 0; s < n_seq; ++s) max_s = seq_lens[s] > max_s ? seq_lens[s] : max_s;
  float* sc = (float*)malloc(sizeof(float) * (size_t)max_s);
  for (int s = 0; s < n_seq; ++s) {
    const int S = seq_lens[s];
    const int32_t* table = block_tables + (size_t)s * max_pages;
    for (int h = 0; h < n_heads; ++h) {
      const int g = h / group;
      const uint16_t* qv = q + ((size_t)s * n_heads + h) * head_dim;
      uint16_t* o = out + ((size_t)s * n_heads + h) * head_dim;
      if (S <= 0) { /* every split empty: the merge divides 0 by 0 */
        for (int d = 0; d < head_dim; ++d) o[d] = 0x7E00u;
        continue;
      }
      for (int j = 0; j < S; ++j) {
        const size_t row = (size_t)table[j / page_size] * page_size + (size_t)(j % page_size);
        const uint16_t* kv = k_pool + row * kvrow + (size_t)g * head_dim;
        float dot = 0.0f;
        for (int d = 0; d < head_dim; ++d) dot = dot + or_h2f(qv[d]) * or_h2f(kv[d]);
        sc[j] = dot * scale;
      }
      float m = -INFINITY;
      for (int j = 0; j < S; ++j) m = sc[j] > m ? sc[j] : m;
      float sum = 0.0f;
      for (int j = 0; j < S; ++j) {
        sc[j] = (float)exp((double)(sc[j] - m));
        sum = sum + sc[j];
      }
      for (int j = 0; j < S; ++j) sc[j] = sc[j] / sum;
      for (int d = 0; d < head_dim; ++d) {
        float acc = 0.0f;
        for (int j = 0; j < S; ++j) {
          const size_t row = (size_t)table[j / page_size] * page_size + (size_t)(j % page_size);
          acc = acc + sc[j] * or_h2f(v_pool[row * kvrow + (size_t)g * head_dim + d]);
        }
        o[d] = or_f2h(acc);
      }
    }
  }
  free(sc);
}

void or_argmax_rows(const uint16_t* logits, int32_t* out, int n_rows, int n_cols) {
  for (int r = 0; r < n_rows; ++r) {
    const uint16_t* row = logits + (size_t)r * n_cols;
    int best = 0x7FFFFFFF; /* no element above -inf (all -inf or NaN): INT_MAX */
    float bv = -INFINITY;
    for (int c = 0; c < n_cols; ++c) {
      const float v = or_h2f(row[c]);
      if (v > bv) { /* strictly greater: ties keep the lowest index; NaN never wins */
        bv = v;
        best = c;
      }
    }
    out[r] = best;
  }
}

/* ------------------------------------------------------------------------------------------ */
/* projection                                                                                   */
/* ------------------------------------------------------------------------------------------ */

/* Output features [o0, o1) of y = x W^T for every row t: the fp32 sum of fp32 products in index
 * order, rounded once to fp16. */
static void linear_cols(const uint16_t* x, const uint16_t* w, uint16_t* y, int T, int in, int out,
                        size_t o0, size_t o1) {
  float* xf = (float*)malloc(sizeof(float) * (size_t)in * (size_t)T);
  float* wf = (float*)malloc(sizeof(float) * (size_t)in);
  or_h2f_array(x, xf, (size_t)in * (size_t)T);
  for (size_t o = o0; o < o1; ++o) {
    or_h2f_array(w + o * (size_t)in, wf, (size_t)in);
    for (int t = 0; t < T; ++t) {
      const float* xr = xf + (size_t)t * in;
      float acc = 0.0f;
      for (int k = 0; k < in; ++k) acc += xr[k] * wf[k];
      y[(size_t)t * out + o] = or_f2h(acc);
    }
  }
  free(xf);
  free(wf);
}

void or_linear(const uint16_t* x, const uint16_t* w, uint16_t* y, int T, int in_features,
               int out_features) {
  linear_cols(x, w, y, T, in_features, out_features, 0, (size_t)out_features);
}

/* ------------------------------------------------------------------------------------------ */
/* row-parallel variants (CPU baseline)                                                         */
/* ------------------------------------------------------------------------------------------ */

typedef struct {
  int kind;
  size_t r0, r1;
  uint16_t* o0;
  const uint16_t *i0, *i1, *i2;
  const int32_t* ids;
  const float* f;
  int a, b, c, d;
  float eps;
  uint16_t* o1;
} job_t;

static void* run_job(void* p) {
  job_t* j = (job_t*)p;
  switch (j->kind) {
    case 0:
      add_rmsnorm_rows(j->o0, j->i0, j->i1, j->o1, (int)j->r0, (int)j->r1, j->a, j->eps);
      break;
    case 1:
      swiglu_range(j->i0, j->i1, j->o0, j->r0, j->r1);
      break;
    case 2:
      rope_tokens(j->o0, j->o1, j->ids, j->f, (int)j->r0, (int)j->r1, j->a, j->b, j->c);
      break;
    case 3:
      or_embedding_lookup(j->i0, j->ids + j->r0, j->o0 + j->r0 * (size_t)j->a,
                          (int)(j->r1 - j->r0), j->a);
      break;
    case 4:
      linear_cols(j->i0, j->i1, j->o0, j->a, j->b, j->c, j->r0, j->r1);
      break;
    case 5:
      or_residual_add(j->i0 + j->r0, j->i1 + j->r0, j->o0 + j->r0, j->r1 - j->r0);
      break;
    case 6:
      or_rmsnorm(j->i0 + j->r0 * (size_t)j->a, j->i1, j->o0 + j->r0 * (size_t)j->a,
                 (int)(j->r1 - j->r0), j->a, j->eps);
      break;
    case 7: /* rows r0..r1 of the source are positions start_pos + r0 .. */
      or_kv_scatter(j->i0 + j->r0 * (size_t)j->c, j->o0, j->ids, j->a + (int)j->r0,
                    (int)(j->r1 - j->r0), j->b, j->c);
      break;
  }
  return NULL;
}

static void run_split(job_t proto, size_t n, int nthreads) {
  if (nthreads < 1) nthreads = 1;
  if ((size_t)nthreads > n) nthreads = n > 0 ? (int)n : 1;
  pthread_t th[256];
  job_t jobs[256];
  if (nthreads > 256) nthreads = 256;
  for (int i = 0; i < nthreads; ++i) {
    jobs[i] = proto;
    jobs[i].r0 = n * (size_t)i / (size_t)nthreads;
    jobs[i].r1 = n * (size_t)(i + 1) / (size_t)nthreads;
    pthread_create(&th[i], NULL, run_job, &jobs[i]);
  }
  for (int i = 0; i < nthreads; ++i) pthread_join(th[i], NULL);
}

void or_add_rmsnorm_mt(uint16_t* residual, const uint16_t* x, const uint16_t* w, uint16_t* out,
                       int n_rows, int hidden, float eps, int nthreads) {
  job_t j = {0};
  j.kind = 0;
  j.o0 = residual;
  j.i0 = x;
  j.i1 = w;
  j.o1 = out;
  j.a = hidden;
  j.eps = eps;
  run_split(j, (size_t)n_rows, nthreads);
}

void or_swiglu_mt(const uint16_t* gate, const uint16_t* up, uint16_t* out, size_t n,
                  int nthreads) {
  job_t j = {0};
  j.kind = 1;
  j.i0 = gate;
  j.i1 = up;
  j.o0 = out;
  run_split(j, n, nthreads);
}

void or_rope_apply_mt(uint16_t* q, uint16_t* k, const int32_t* positions, const float* inv_freq,
                      int n_tokens, int n_heads, int n_kv_heads, int head_dim, int nthreads) {
  job_t j = {0};
  j.kind = 2;
  j.o0 = q;
  j.o1 = k;
  j.ids = positions;
  j.f = inv_freq;
  j.a = n_heads;
  j.b = n_kv_heads;
  j.c = head_dim;
  run_split(j, (size_t)n_tokens, nthreads);
}

void or_embedding_lookup_mt(const uint16_t* table, const int32_t* ids, uint16_t* out,
                            int n_tokens, int hidden, int nthreads) {
  job_t j = {0};
  j.kind = 3;
  j.i0 = table;
  j.ids = ids;
  j.o0 = out;
  j.a = hidden;
  run_split(j, (size_t)n_tokens, nthreads);
}

void or_residual_add_mt(const uint16_t* a, const uint16_t* b, uint16_t* out, size_t n,
                        int nthreads) {
  job_t j = {0};
  j.kind = 5;
  j.i0 = a;
  j.i1 = b;
  j.o0 = out;
  run_split(j, n, nthreads);
}

void or_rmsnorm_mt(const uint16_t* x, const uint16_t* w, uint16_t* out, int n_rows, int hidden,
                   float eps, int nthreads) {
  job_t j = {0};
  j.kind = 6;
  j.i0 = x;
  j.i1 = w;
  j.o0 = out;
  j.a = hidden;
  j.eps = eps;
  run_split(j, (size_t)n_rows, nthreads);
}

void or_kv_scatter_mt(const uint16_t* src, uint16_t* pool, const int32_t* block_table,
                      int start_pos, int T, int page_size, int kvdim, int nthreads) {
  job_t j = {0};
  j.kind = 7;
  j.i0 = src;
  j.o0 = pool;
  j.ids = block_table;
  j.a = start_pos;
  j.b = page_size;
  j.c = kvdim;
  run_split(j, (size_t)T, nthreads);
}

/* ------------------------------------------------------------------------------------------ */
/* test helpers                                                                                 */
/* ------------------------------------------------------------------------------------------ */

void or_residual_add_kat_inputs(uint32_t seed, size_t n, uint16_t* a, uint16_t* b) {
  uint32_t s = seed;
  for (size_t i = 0; i < n; ++i) {
    float v[2];
    for (int k = 0; k < 2; ++k) {
      s ^= s << 13;
      s ^= s >> 17;
      s ^= s << 5;
      v[k] = (float)(s & 0xFFFFFFu) / 16777216.0f * 8.0f - 4.0f;
    }
    a[i] = or_f2h(v[0]);
    b[i] = or_f2h(v[1]);
  }
}

#if defined(__x86_64__)
#include <immintrin.h>

typedef struct {
  uint64_t lo, hi;
  long long bad;
} f16c_job;

__attribute__((target("f16c"))) static void* f16c_range(void* p) {
  f16c_job* j = (f16c_job*)p;
  long long bad = 0;
  for (uint64_t u = j->lo; u < j->hi; ++u) {
    const float f = bits_f((uint32_t)u);
    const uint16_t hw = (uint16_t)_cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT);
    const uint16_t mine = or_f2h(f);
    if (hw != mine) {
      const int hw_nan = (hw & 0x7C00u) == 0x7C00u && (hw & 0x3FFu);
      const int my_nan = (mine & 0x7C00u) == 0x7C00u && (mine & 0x3FFu);
      if (!(hw_nan && my_nan)) ++bad;
    }
  }
  j->bad = bad;
  return NULL;
}

long long or_f16c_mismatches(int nthreads) {
  __builtin_cpu_init();
  if (!__builtin_cpu_supports("f16c")) return -1;
  if (nthreads < 1) nthreads = 1;
  if (nthreads > 64) nthreads = 64;
  pthread_t th[64];
  f16c_job jobs[64];
  const uint64_t total = 1ull << 32;
  for (int i = 0; i < nthreads; ++i) {
    jobs[i].lo = total * (uint64_t)i / (uint64_t)nthreads;
    jobs[i].hi = total * (uint64_t)(i + 1) / (uint64_t)nthreads;
    jobs[i].bad = 0;
    pthread_create(&th[i], NULL, f16c_range, &jobs[i]);
  }
  long long bad = 0;
  for (int i = 0; i < nthreads; ++i) {
    pthread_join(th[i], NULL);
    bad += jobs[i].bad;
  }
  return bad;
}
#else
long long or_f16c_mismatches(int nthreads) {
  (void)nthreads;
  return -1;
}
#endif

void or_linear_mt(const uint16_t* x, const uint16_t* w, uint16_t* y, int T, int in_features,
                  int out_features, int nthreads) {
  job_t j = {0};
  j.kind = 4;
  j.i0 = x;
  j.i1 = w;
  j.o0 = y;
  j.a = T;
  j.b = in_features;
  j.c = out_features;
  run_split(j, (size_t)out_features, nthreads);
}
