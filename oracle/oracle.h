/*
 * oracle.h - scalar CPU restatement of the reference's non-GEMM layer kernels.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker the HIP kernels of libllmk are compared
 * against; it is never linked into, loaded by, or used as a fallback for the product. Only the
 * tests, the smoke check and the bench's CPU-baseline leg call it.
 *
 * Every function restates the arithmetic of the reference kernel it cites
 * (JayeshNikam36/cuda-llm-engine, file:line), in scalar C with fp32 arithmetic, IEEE binary16
 * storage and round-to-nearest-even conversions written out from the binary16 format. Built
 * with -ffp-contract=off so that no product and sum are fused. Transcendentals come from libm
 * in double precision, rounded to float (exp, sin, cos); the reference's device library is
 * not reproduced.
 */
#ifndef LLMK_ORACLE_H
#define LLMK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* binary16 <-> binary32 (round to nearest, ties to even; subnormals kept; NaN stays NaN). */
float or_h2f(uint16_t h);
uint16_t or_f2h(float f);
void or_h2f_array(const uint16_t* in, float* out, size_t n);
void or_f2h_array(const float* in, uint16_t* out, size_t n);

/* ref: kernels/embedding.cu:6-8 */
void or_embedding_lookup(const uint16_t* table, const int32_t* ids, uint16_t* out, int n_tokens,
                         int hidden);
/* ref: kernels/residual_add.cu:10-11; tests/test_residual_add.cu:19 */
void or_residual_add(const uint16_t* a, const uint16_t* b, uint16_t* out, size_t n);
/* ref: kernels/rmsnorm.cu:14-24, :37, :42-57 */
void or_rmsnorm(const uint16_t* x, const uint16_t* w, uint16_t* out, int n_rows, int hidden,
                float eps);
/* ref: kernels/residual_add.cu:10-11 then kernels/rmsnorm.cu (engine/batched.cu:64->66) */
void or_add_rmsnorm(uint16_t* residual, const uint16_t* x, const uint16_t* w, uint16_t* out,
                    int n_rows, int hidden, float eps);
/* ref: kernels/rope.cu:4-23 */
void or_compute_rope_inv_freq(int head_dim, double theta, double factor, double low_freq_factor,
                              double high_freq_factor, double original_max_pos, float* out);
/* ref: kernels/rope.cu:30-43 */
void or_rope_apply(uint16_t* q, uint16_t* k, const int32_t* positions, const float* inv_freq,
                   int n_tokens, int n_heads, int n_kv_heads, int head_dim);
/* ref: kernels/swiglu.cu:8-14 */
void or_swiglu(const uint16_t* gate, const uint16_t* up, uint16_t* out, size_t n);
/* ref: kernels/kv_scatter.cu:7-11 */
void or_kv_scatter(const uint16_t* src, uint16_t* pool, const int32_t* block_table,
                   int start_pos, int T, int page_size, int kvdim);
/* ref: kernels/kv_scatter.cu:17-23; tests/test_attention_decode_fast.cu:35-41 */
void or_kv_scatter_batch(const uint16_t* src, uint16_t* pool, const int32_t* block_tables,
                         const int32_t* positions, int n, int max_pages, int page_size,
                         int kvdim);
/* Composition rope_apply -> kv_scatter_batch(K) -> kv_scatter_batch(V) of
 * ref: engine/batched.cu:55-58; k is read only (rotated into a scratch copy). */
void or_rope_kv_scatter_batch(uint16_t* q, const uint16_t* k, const uint16_t* v,
                              uint16_t* k_pool, uint16_t* v_pool, const int32_t* block_tables,
                              const int32_t* positions, const float* inv_freq, int n,
                              int max_pages, int page_size, int n_heads, int n_kv_heads,
                              int head_dim);

/* Decode attention over a paged KV cache, one query token per sequence: the arithmetic of
 * ref: kernels/attention_decode_paged.cu:24-62, the kernel the split-KV kernel
 * (kernels/attention_decode_fast.cu) is checked against in tests/test_attention_decode_fast.cu:58-61,
 * applied to every sequence of the batch. For sequence s and query head h, kv head
 * g = h / (n_heads / n_kv_heads), positions j < seq_lens[s] at pool row
 * block_tables[s][j / page_size] * page_size + j % page_size: score_j = (sum_d q[d] * k_j[d]) *
 * (1 / sqrt(head_dim)) in fp32; p_j = exp(score_j - max) / sum_j exp(...); out[d] =
 * fp16(sum_j p_j * v_j[d]); every sum in fp32, in index order. A sequence with seq_lens <= 0
 * gets NaN, as the split-KV kernel's merge yields 0 / 0 there
 * (ref: kernels/attention_decode_fast.cu:42-48, 141-148). */
void or_attention_decode_paged(const uint16_t* q, const uint16_t* k_pool, const uint16_t* v_pool,
                               const int32_t* block_tables, const int32_t* seq_lens,
                               uint16_t* out, int n_seq, int max_pages, int page_size,
                               int n_heads, int n_kv_heads, int head_dim);

/* Row argmax of fp16 logits [n_rows, n_cols] (ref: kernels/argmax.cu:11-40): the index of the
 * largest value, the lowest index among equal ones (+0 equals -0); NaN never wins; a row with no
 * value above -inf gives INT_MAX (the reduction's initial index). */
void or_argmax_rows(const uint16_t* logits, int32_t* out, int n_rows, int n_cols);

/* Projection y[T, out] = x[T, in] W^T with W [out, in] row-major, fp16 in and out: each output
 * is the fp32 sum, in index order, of the fp32 products float(x) * float(w), rounded once to
 * fp16 -- a GEMM with fp16 data and fp32 accumulation, as ref: kernels/linear.cu:8-20 requests
 * of cuBLAS (CUBLAS_COMPUTE_32F). The summation order of a library GEMM is unspecified, so the
 * GPU agrees within tolerance, not bit for bit. or_linear_mt splits the output features over
 * nthreads threads (same results). */
void or_linear(const uint16_t* x, const uint16_t* w, uint16_t* y, int T, int in_features,
               int out_features);
void or_linear_mt(const uint16_t* x, const uint16_t* w, uint16_t* y, int T, int in_features,
                  int out_features, int nthreads);

/* Row-parallel variants for the CPU baseline: the same per-row code split over nthreads
 * threads by contiguous row ranges (results identical to the single-thread functions). */
void or_add_rmsnorm_mt(uint16_t* residual, const uint16_t* x, const uint16_t* w, uint16_t* out,
                       int n_rows, int hidden, float eps, int nthreads);
void or_swiglu_mt(const uint16_t* gate, const uint16_t* up, uint16_t* out, size_t n,
                  int nthreads);
void or_rope_apply_mt(uint16_t* q, uint16_t* k, const int32_t* positions, const float* inv_freq,
                      int n_tokens, int n_heads, int n_kv_heads, int head_dim, int nthreads);
void or_embedding_lookup_mt(const uint16_t* table, const int32_t* ids, uint16_t* out,
                            int n_tokens, int hidden, int nthreads);

/* Input generator of the reference's residual-add known-answer test
 * (ref: tests/test_residual_add.cu:6-10, 16-18): xorshift32 from `seed`, each draw mapped to
 * (state & 0xFFFFFF) / 2^24 * 8 - 4 in fp32; a[i] and b[i] are consecutive draws, rounded to
 * fp16. */
void or_residual_add_kat_inputs(uint32_t seed, size_t n, uint16_t* a, uint16_t* b);

/* Exhaustive check of or_f2h against the host's F16C conversion (vcvtps2ph, round to nearest
 * even) over all 2^32 fp32 bit patterns, split over nthreads threads. Returns the number of
 * mismatches, or -1 when the CPU has no F16C. NaN inputs are compared as "both NaN". */
long long or_f16c_mismatches(int nthreads);

#ifdef __cplusplus
}
#endif

#endif
