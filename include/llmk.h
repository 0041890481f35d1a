/*
 * llmk.h - C-ABI of libllmk, the MI355X (gfx950) implementation of the non-GEMM layer kernels
 * of a Llama-style fp16 decoder: embedding gather, residual add, RMSNorm, fused residual add +
 * RMSNorm, RoPE with Llama-3 frequency scaling, SwiGLU, and the paged KV scatter (plain and
 * fused with RoPE).
 *
 * Conventions shared by every entry point:
 *  - Tensors are device pointers owned by the caller; fp16 values travel as uint16_t bit
 *    patterns, indices as int32_t. Nothing is allocated and no state is kept between calls.
 *  - `stream` is a hipStream_t (NULL = the null stream). Work is enqueued, never waited for.
 *  - The return value is LLMK_OK (0), a hipError_t value from the launch, or one of the
 *    LLMK_ERR_* codes below for an argument that violates a precondition (then nothing is
 *    enqueued). llmk_error_string() names either kind.
 *  - A zero element/row/token count is a no-op that returns LLMK_OK.
 *  - Functions are re-entrant; different host threads may call them on different streams.
 *
 * Citations "ref: file:line" point into JayeshNikam36/cuda-llm-engine, whose free C++ launchers
 * these entry points replace one for one (names, argument order and meaning kept; __half* ->
 * uint16_t*, cudaStream_t -> void*, void -> status code). include/llmk.hpp restores the
 * reference's exact C++ signatures on top of this header.
 */
#ifndef LLMK_H
#define LLMK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define LLMK_API __attribute__((visibility("default")))
#else
#define LLMK_API
#endif

/* Status codes that are not hipError_t values. */
#define LLMK_OK 0
#define LLMK_ERR_INVALID_VALUE 10001 /* negative size, NULL pointer with a nonzero size */
#define LLMK_ERR_SHAPE 10002         /* size not a multiple the layout requires */
#define LLMK_ERR_ALIGNMENT 10003     /* a pointer that must be 16-byte aligned is not */
#define LLMK_ERR_UNSUPPORTED 10004   /* a shape outside what the kernels implement */
#define LLMK_ERR_BLAS 10005          /* hipBLASLt refused or failed a GEMM */
#define LLMK_ERR_IO 10006            /* a weight file is missing, short, or lacks a tensor */
#define LLMK_ERR_CAPACITY 10007      /* a request can never fit in the page pool or block table */
#define LLMK_ERR_SCRATCH 10008       /* more scratch than the allocation-free entry point holds */

/* Human-readable name of a status code (LLMK_ERR_* or hipError_t). Never NULL. */
LLMK_API const char* llmk_error_string(int status);

/* Library version, major * 10000 + minor * 100 + patch. */
LLMK_API int llmk_version(void);

/* out[t, :] = table[ids[t], :] for t < n_tokens; bit-exact copy of hidden fp16 values per row.
 * hidden % 8 == 0; table and out 16-byte aligned. ids are not range-checked (as in the
 * reference): every id must lie in [0, rows of table).
 * ref: kernels/embedding.cuh:6-7, kernels/embedding.cu:4-16 (embedding_lookup). */
LLMK_API int llmk_embedding_lookup(const uint16_t* table, const int32_t* ids, uint16_t* out,
                          int n_tokens, int hidden, void* stream);

/* out[i] = fp16_rne(float(a[i]) + float(b[i])) for i < n. out may be the same pointer as a or
 * b (in place); any alignment and any n are accepted.
 * ref: kernels/residual_add.cuh:5-6, kernels/residual_add.cu:5-18 (residual_add). */
LLMK_API int llmk_residual_add(const uint16_t* a, const uint16_t* b, uint16_t* out, size_t n,
                      void* stream);

/* Per row r < n_rows of width hidden: ss = sum of float(x)^2 in fp32; inv = 1 / sqrt(ss/hidden +
 * eps); out = fp16(float(w) * r16(float(x) * inv)) where r16 rounds to fp16 and back.
 * hidden % 8 == 0; x, w, out 16-byte aligned.
 * ref: kernels/rmsnorm.cuh:5-7, kernels/rmsnorm.cu:9-68 (rmsnorm). */
LLMK_API int llmk_rmsnorm(const uint16_t* x, const uint16_t* w, uint16_t* out, int n_rows, int hidden,
                 float eps, void* stream);

/* Fused residual add + RMSNorm: residual <- fp16(residual + x) in place (bit-exact, the same
 * value llmk_residual_add writes), then out = rmsnorm(residual) as llmk_rmsnorm.
 * Replaces the residual_add -> rmsnorm pairs at ref: engine/batched.cu:64->66 and :71->:51
 * (engine/layer.cu:76->79, :84->69). New entry point; no single reference function. */
LLMK_API int llmk_add_rmsnorm(uint16_t* residual, const uint16_t* x, const uint16_t* w, uint16_t* out,
                     int n_rows, int hidden, float eps, void* stream);

/* Host function: the head_dim/2 rotation speeds with Llama-3 frequency scaling, computed in
 * fp32 step by step, written to out[0 .. head_dim/2). head_dim even and > 0.
 * ref: kernels/rope.cuh:7-9, kernels/rope.cu:4-23 (compute_rope_inv_freq). */
LLMK_API int llmk_compute_rope_inv_freq(int head_dim, double theta, double factor,
                               double low_freq_factor, double high_freq_factor,
                               double original_max_pos, float* out);

/* In-place rotary embedding of q [n_tokens, n_heads, head_dim] and k [n_tokens, n_kv_heads,
 * head_dim]; element i is paired with i + head_dim/2. For angle a = float(pos[t]) * inv_freq[i]
 * (fp32 product): c = r16(cos a), s = r16(sin a); x1' = fp16(r16(x1*c) - r16(x2*s)),
 * x2' = fp16(r16(x2*c) + r16(x1*s)). inv_freq is a device pointer to head_dim/2 floats.
 * head_dim even; q and k 16-byte aligned when head_dim % 16 == 0 (the vector path).
 * ref: kernels/rope.cuh:11-15, kernels/rope.cu:24-49 (rope_apply). */
LLMK_API int llmk_rope_apply(uint16_t* q, uint16_t* k, const int32_t* positions, const float* inv_freq,
                    int n_tokens, int n_heads, int n_kv_heads, int head_dim, void* stream);

/* out[i] = fp16(r16(g / (1 + exp(-g))) * float(up[i])) with g = float(gate[i]), for i < n.
 * Any alignment and any n are accepted.
 * ref: kernels/swiglu.cuh:5-6, kernels/swiglu.cu:4-21 (swiglu). */
LLMK_API int llmk_swiglu(const uint16_t* gate, const uint16_t* up, uint16_t* out, size_t n,
                void* stream);

/* Prefill scatter: for t < T, pos = start_pos + t, row = block_table[pos / page_size] *
 * page_size + pos % page_size, pool[row*kvdim .. +kvdim) = src[t*kvdim .. +kvdim). Pool layout
 * [num_pages, page_size, n_kv_heads, head_dim]. kvdim % 8 == 0; src and pool 16-byte aligned.
 * Page numbers are not range-checked (as in the reference).
 * ref: kernels/kv_scatter.cuh:5-8, kernels/kv_scatter.cu:4-12,26-32 (kv_scatter). */
LLMK_API int llmk_kv_scatter(const uint16_t* src, uint16_t* pool, const int32_t* block_table,
                    int start_pos, int T, int page_size, int kvdim, void* stream);

/* Decode scatter: for b < n, row = block_tables[b*max_pages + pos[b]/page_size] * page_size +
 * pos[b] % page_size; pool[row*kvdim .. +kvdim) = src[b*kvdim .. +kvdim).
 * kvdim % 8 == 0; src and pool 16-byte aligned.
 * ref: kernels/kv_scatter.cuh:10-13, kernels/kv_scatter.cu:14-24,34-40 (kv_scatter_batch). */
LLMK_API int llmk_kv_scatter_batch(const uint16_t* src, uint16_t* pool, const int32_t* block_tables,
                          const int32_t* positions, int n, int max_pages, int page_size,
                          int kvdim, void* stream);

/* Fused decode RoPE + KV scatter, one new token per sequence b < n at position positions[b]:
 * q [n, n_heads, head_dim] is rotated in place (as llmk_rope_apply); k [n, n_kv_heads,
 * head_dim] is rotated (as llmk_rope_apply) and written to k_pool at the llmk_kv_scatter_batch
 * address; v [n, n_kv_heads, head_dim] is copied bit-exact to v_pool at the same address. k and
 * v are only read. head_dim % 16 == 0; q, k, v, k_pool, v_pool 16-byte aligned.
 * Replaces ref: engine/batched.cu:55-58 (rope_apply, then kv_scatter_batch for K and V). New
 * entry point; no single reference function. */
LLMK_API int llmk_rope_kv_scatter_batch(uint16_t* q, const uint16_t* k, const uint16_t* v,
                               uint16_t* k_pool, uint16_t* v_pool, const int32_t* block_tables,
                               const int32_t* positions, const float* inv_freq, int n,
                               int max_pages, int page_size, int n_heads, int n_kv_heads,
                               int head_dim, void* stream);

/* Default target block count of choose_num_splits (llmk.hpp) for MI355X. The reference's
 * default, 64, was fitted to a 20-SM laptop GPU (ref: kernels/attention_decode_fast.cuh:20-22).
 * Here num_splits only caps how many pieces a sequence may be cut into (libllmk balances the
 * pages of the whole batch over one block per CU), so the default asks for as many
 * as the rule allows: 32 for batches up to 256 sequences of 8 kv heads. */
#define LLMK_ATTN_TARGET_BLOCKS 65536

/* Floats of workspace llmk_attention_decode_fast needs for n_seq sequences, n_heads query
 * heads and up to num_splits splits per sequence: n_seq * n_heads * num_splits * (64 + 2), the
 * reference's figure. 0 for non-positive arguments; SIZE_MAX when the product exceeds the size_t
 * range (it saturates instead of wrapping; llmk_attention_decode_fast then refuses the call with
 * LLMK_ERR_INVALID_VALUE, the allocation-free variant with LLMK_ERR_SCRATCH).
 * ref: kernels/attention_decode_fast.cuh:6, kernels/attention_decode_fast.cu:151-153. */
LLMK_API size_t llmk_attention_decode_fast_workspace_floats(int n_seq, int n_heads,
                                                            int num_splits);

/* Batched decode attention over the paged KV cache, one new token per sequence:
 * out[s, h, :] = softmax_j(q[s, h, :] . K_j / sqrt(head_dim)) . V_j over the positions
 * j < seq_lens[s], K_j / V_j the pool rows block_tables[s * max_pages + j / page_size] *
 * page_size + j % page_size, kv head h / (n_heads / n_kv_heads). Layouts: q and out
 * [n_seq, n_heads, head_dim]; pools [num_pages, page_size, n_kv_heads, head_dim]; block_tables
 * [n_seq, max_pages]. Requires page_size 16, head_dim 64, n_heads == 4 * n_kv_heads (the
 * reference's preconditions: LLMK_ERR_SHAPE otherwise) and n_seq <= 65535 (the reference's grid
 * limit too; LLMK_ERR_UNSUPPORTED otherwise). Each sequence is cut into at most num_splits runs of
 * ceil(max_pages / num_splits) pages; with more than one run the partial results go through
 * `workspace` (llmk_attention_decode_fast_workspace_floats(n_seq, n_heads, num_splits) floats,
 * 16-byte aligned; may be NULL when num_splits == 1) and a second launch merges them. A
 * sequence with seq_lens <= 0 gets NaN (the reference's 0 / 0). Positions past max_pages *
 * page_size are not read. q, pools and out 16-byte aligned.
 * ref: kernels/attention_decode_fast.cuh:8-18, kernels/attention_decode_fast.cu:155-172. */
LLMK_API int llmk_attention_decode_fast(const uint16_t* q, const uint16_t* k_pool,
                                        const uint16_t* v_pool, const int32_t* block_tables,
                                        const int32_t* seq_lens, uint16_t* out,
                                        float* workspace, int n_seq, int max_pages,
                                        int page_size, int n_heads, int n_kv_heads,
                                        int head_dim, int num_splits, void* stream);

/* Scratch floats of llmk_attention_decode_fast_noalloc: the workspace of 256 sequences x 32
 * query heads x 32 splits (66 MiB per GPU, held from the library's load to the process's end). */
#define LLMK_ATTN_NOALLOC_MAX_FLOATS ((size_t)256 * 32 * 32 * 66)

/* llmk_attention_decode_fast without a workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference. The same kernels and results as
 * llmk_attention_decode_fast; the partial results go to a device array inside the library
 * instead, one per GPU. Returns LLMK_ERR_SCRATCH, before any launch, when
 * llmk_attention_decode_fast_workspace_floats(n_seq, n_heads, num_splits) exceeds
 * LLMK_ATTN_NOALLOC_MAX_FLOATS. Calls no allocating routine. All calls on one GPU share that
 * GPU's array: calls that may overlap on one GPU (unordered streams) race, and must be ordered
 * by the caller. The first call on a device also resolves the array's device address there
 * (hipGetSymbolAddress, not a stream operation). */
LLMK_API int llmk_attention_decode_fast_noalloc(const uint16_t* q, const uint16_t* k_pool,
                                                const uint16_t* v_pool,
                                                const int32_t* block_tables,
                                                const int32_t* seq_lens, uint16_t* out, int n_seq,
                                                int max_pages, int page_size, int n_heads,
                                                int n_kv_heads, int head_dim, int num_splits,
                                                void* stream);

/* Row argmax of fp16 logits [n_rows, vocab]: out[r] = the index of the largest value of row r,
 * the lowest index among equal values (+0 equals -0); NaN is never chosen; a row with no value
 * above -inf gives INT_MAX. Any vocab and alignment (16-byte vector path when vocab % 8 == 0,
 * the rows are 16-byte aligned and vocab >= 8192).
 * ref: kernels/argmax.cuh:5-7, kernels/argmax.cu:5-44. */
LLMK_API int llmk_argmax_rows(const uint16_t* logits, int32_t* out, int n_rows, int vocab,
                              void* stream);

/* Device-to-device copy of nbytes with 16-byte vector loads and stores, used to measure the
 * practical HBM ceiling and to calibrate rocprof traffic counters. src and dst 16-byte aligned,
 * nbytes % 16 == 0. ref: bench/bandwidth.cu:11-15 (copy_vec4, the reference's bandwidth probe). */
LLMK_API int llmk_copy_bytes(const void* src, void* dst, size_t nbytes, void* stream);

/* Bandwidth probe for one traffic mix, with the layer kernels' 16-byte non-temporal accesses:
 * LLMK_PROBE_READ reads a (dst receives nothing in practice, but must hold nbytes), _COPY a ->
 * dst, _READ2 a, b -> dst (2 reads : 1 write), _INPLACE dst -> dst (read and rewrite the same
 * addresses), _WRITE fills dst. blocks > 0: a grid-stride loop over that many 256-thread
 * blocks; blocks == 0: one pass, every thread `unroll` vectors. unroll is 1, 2, 4 or 8.
 * Buffers 16-byte aligned, nbytes % 16 == 0. INPLACE and WRITE change dst's contents.
 * ref: bench/bandwidth.cu:11-62 (a copy kernel swept over block and grid sizes). */
#define LLMK_PROBE_READ 0
#define LLMK_PROBE_COPY 1
#define LLMK_PROBE_READ2 2
#define LLMK_PROBE_INPLACE 3
#define LLMK_PROBE_WRITE 4
LLMK_API int llmk_bw_probe(int mode, const void* a, const void* b, void* dst, size_t nbytes,
                           int blocks, int unroll, void* stream);

/* Launches an empty kernel of `blocks` blocks of `threads` threads: the launch floor a
 * sequence of launches pays whatever the kernels do (the reference times its stages one by one
 * with events, bench/bench_breakdown.cu:18-26; this measures what is left when the work is
 * gone). */
LLMK_API int llmk_empty_launch(int blocks, int threads, void* stream);

/* One non-GEMM decode-step pass: the embedding gather into `residual`, then per layer l the
 * operations the reference's batched layer issues between its GEMMs and attention
 * (ref: engine/batched.cu:51-71, :112-115): add+RMSNorm of residual with x[l] (out normed[l]),
 * RoPE of q[l] / k[l] with the scatter of k[l] and v[l] into k_pool[l] / v_pool[l], and SwiGLU
 * of gate[l], up[l] into act[l]. The per-layer arrays are HOST arrays of n_layers device
 * pointers. Every launch goes to `stream` in that order, so the pass can be captured into a
 * HIP graph. */
typedef struct llmk_decode_pass {
  int n_seqs, n_layers, hidden, n_heads, n_kv_heads, head_dim, inter;
  int page_size, max_pages;
  float eps;
  const uint16_t* embed_table; /* [vocab, hidden] */
  const int32_t* token_ids;    /* [n_seqs] */
  uint16_t* residual;          /* [n_seqs, hidden]: embedding output, then the residual chain */
  const int32_t* block_tables; /* [n_seqs, max_pages] */
  const int32_t* positions;    /* [n_seqs] */
  const float* inv_freq;       /* [head_dim / 2] */
  const uint16_t* const* x;        /* per layer [n_seqs, hidden]: added into residual */
  const uint16_t* const* norm_w;   /* per layer [hidden] */
  uint16_t* const* normed;         /* per layer [n_seqs, hidden] */
  uint16_t* const* q;              /* per layer [n_seqs, n_heads, head_dim], rotated in place */
  const uint16_t* const* k;        /* per layer [n_seqs, n_kv_heads, head_dim] */
  const uint16_t* const* v;        /* per layer [n_seqs, n_kv_heads, head_dim] */
  uint16_t* const* k_pool;         /* per layer [num_pages, page_size, n_kv_heads, head_dim] */
  uint16_t* const* v_pool;         /* per layer, same layout */
  const uint16_t* const* gate;     /* per layer [n_seqs, inter] */
  const uint16_t* const* up;       /* per layer [n_seqs, inter] */
  uint16_t* const* act;            /* per layer [n_seqs, inter] */
  /* Optional, all NULL or all set: each layer's second add + RMSNorm, as the reference layer
   * adds the attention output and normalises for the MLP (engine/batched.cu:64-66); it runs
   * after the RoPE + K/V scatter and before the SwiGLU. */
  const uint16_t* const* x2;       /* per layer [n_seqs, hidden]: added into residual */
  const uint16_t* const* norm_w2;  /* per layer [hidden] */
  uint16_t* const* normed2;        /* per layer [n_seqs, hidden] */
} llmk_decode_pass;

LLMK_API int llmk_decode_nongemm_pass(const llmk_decode_pass* pass, void* stream);

/* The same pass and results with one launch per layer (n_layers launches instead of
 * 1 + 3 * n_layers): a layer's add + RMSNorm rows, RoPE + K/V scatter tokens and SwiGLU chunks
 * are blocks of one launch, and the embedding gather is fused into the first layer's residual
 * add (the residual buffer never holds the bare embedding rows). Valid because the pass's
 * per-layer inputs are independent of each other; in a decode step with GEMMs between these
 * ops they are not, and the engine launches them one by one. Requires head_dim 64, hidden a
 * power-of-two multiple of 512 up to 8192, (n_heads + 2 * n_kv_heads) * 8 <= 1024 and every
 * pointer 16-byte aligned (LLMK_ERR_UNSUPPORTED / LLMK_ERR_ALIGNMENT otherwise: use
 * llmk_decode_nongemm_pass). */
LLMK_API int llmk_decode_nongemm_pass_layers(const llmk_decode_pass* pass, void* stream);

/* The same pass and results in one launch per 16 layers (config 5's pass is one launch): one
 * wave per sequence carries its residual row through all of the launch's layers (each layer's
 * add + RMSNorm, or both of them, in order, the residual kept in registers and stored after
 * every layer), while the other blocks of the launch run every layer's RoPE + K/V scatter
 * tokens and SwiGLU chunks. Valid for the same reason and under the same requirements as
 * llmk_decode_nongemm_pass_layers, and hidden <= 4096 (LLMK_ERR_UNSUPPORTED above: use
 * llmk_decode_nongemm_pass_layers). New entry point; the reference runs these ops as separate
 * launches (engine/batched.cu:44-72,112-116). */
LLMK_API int llmk_decode_nongemm_pass_fused(const llmk_decode_pass* pass, void* stream);

/* ------------------------------------------------------------------------------------------
 * The decode step around the kernels above: projections (hipBLASLt), the fused layouts they
 * produce, and an engine that runs a whole Llama-3 forward pass over a batch of token rows.
 * ------------------------------------------------------------------------------------------ */

/* A GEMM handle: one hipBLASLt handle, a 32 MiB workspace allocated at creation, and a cache
 * of per-shape plans. Calls on one handle share its workspace, so they must be ordered (one
 * stream, or one handle per stream), as calls on one cuBLAS handle are. */
typedef struct llmk_blas llmk_blas;
LLMK_API int llmk_blas_create(llmk_blas** out);
/* Lifetime: a HIP graph that captured llmk_linear (or llmk_blas_tune) on this handle holds its
 * workspace address and hipBLASLt's kernels by reference. Destroy every such graph and graph
 * exec, and let the work already launched from them finish, before destroying the handle.
 * Destroying the handle first leaves those graphs pointing at freed memory and at kernels of
 * code objects the handle has released. */
LLMK_API void llmk_blas_destroy(llmk_blas* h);

/* y[T, out_features] = x[T, in_features] * W^T, W stored [out_features, in_features] row-major
 * (a PyTorch Linear without bias); fp16 in and out, fp32 accumulation. With T <= 8,
 * in_features % 512 == 0 and x, W 16-byte aligned it runs llmk_linear_rows; otherwise the first
 * call of a shape takes hipBLASLt's heuristic choice (make that call outside graph capture) and
 * later calls only enqueue. ref: kernels/linear.cuh:5-7, kernels/linear.cu:5-25 (linear;
 * cublasHandle_t -> llmk_blas*). */
LLMK_API int llmk_linear(llmk_blas* h, const uint16_t* x, const uint16_t* w, uint16_t* y, int T,
                         int in_features, int out_features, void* stream);

/* The row limit of llmk_linear_rows. */
#define LLMK_LINEAR_ROWS_MAX 8

/* llmk_linear for a few rows (T <= LLMK_LINEAR_ROWS_MAX): a kernel of this library that streams
 * W from HBM (a decode step with few sequences is a GEMV; its time is the weight read).
 * in_features % 512 == 0; x and W 16-byte aligned; no handle, no workspace, allocates nothing.
 * Sums run in another order than hipBLASLt's, so results agree to fp32 rounding. New entry
 * point; the reference's linear (kernels/linear.cu:5-25) covers every T with cuBLAS. */
LLMK_API int llmk_linear_rows(const uint16_t* x, const uint16_t* w, uint16_t* y, int T,
                              int in_features, int out_features, void* stream);

/* The few-rows projection with the decode step's neighbouring element-wise work done in the same
 * kernel (T <= LLMK_LINEAR_ROWS_MAX, in_features % 512 == 0, 16-byte aligned operands). With
 * norm_w non-null the x rows are first RMSNorm-ed with weight norm_w [in_features] and eps,
 * giving the bits llmk_rmsnorm gives (in_features / 512 a power of two up to 16); with norm_w
 * null x is used as is. Each epilogue rounds the projection to fp16 first and then
 * applies the reference's formula, so every result has the bits of llmk_linear_rows followed
 * by the separate launch. New entry points, for the engine's decode steps with few sequences;
 * they replace ref: engine/batched.cu:51-58 (rmsnorm, three projections, rope_apply, two
 * kv_scatter_batch), :62-64 (o projection, residual_add), :66-69 (rmsnorm, gate and up
 * projections, swiglu) and :70-71 (down projection, residual_add).
 *   _norm: y[T, out] = norm(x) W^T.
 *   _residual: residual[T, out] = fp16(residual + fp16(x W^T)) (llmk_residual_add).
 *   _swiglu: w_gate_up [2 inter, in] (gate rows, then up rows); act[T, inter] =
 *     llmk_swiglu(g, u) of g, u = fp16(norm(x) W^T) of the two halves.
 *   _qkv_rope_scatter: w_qkv [(n_heads + 2 n_kv_heads) 64, in] (q, k, v rows, head_dim 64);
 *     the projection's q, k and v rows go through llmk_qkv_rope_scatter with page size 16. */
LLMK_API int llmk_linear_rows_norm(const uint16_t* x, const uint16_t* norm_w, float eps,
                                   const uint16_t* w, uint16_t* y, int T, int in_features,
                                   int out_features, void* stream);
LLMK_API int llmk_linear_rows_residual(const uint16_t* x, const uint16_t* w, uint16_t* residual,
                                       int T, int in_features, int out_features, void* stream);
LLMK_API int llmk_linear_rows_swiglu(const uint16_t* x, const uint16_t* norm_w, float eps,
                                     const uint16_t* w_gate_up, uint16_t* act, int T,
                                     int in_features, int inter, void* stream);
LLMK_API int llmk_linear_rows_qkv_rope_scatter(const uint16_t* x, const uint16_t* norm_w,
                                               float eps, const uint16_t* w_qkv,
                                               uint16_t* q_out, uint16_t* k_pool,
                                               uint16_t* v_pool, const int32_t* block_tables,
                                               const int32_t* positions, const float* inv_freq,
                                               int T, int in_features, int n_heads,
                                               int n_kv_heads, int max_pages, void* stream);

/* Chooses the algorithm of one shape by timing hipBLASLt's heuristic candidates with cold
 * caches, on `stream` with these operands (y is overwritten; synchronous; not while the stream
 * is capturing). Later llmk_linear calls of the shape use it. New entry point. */
LLMK_API int llmk_blas_tune(llmk_blas* h, const uint16_t* x, const uint16_t* w, uint16_t* y,
                            int T, int in_features, int out_features, void* stream);

/* RoPE + KV scatter reading the rows of one fused QKV projection: row b of qkv (stride ld
 * elements) holds q [n_heads, head_dim] at column 0, k [n_kv_heads, head_dim] after it and v
 * after k. q is rotated into q_out [n, n_heads, head_dim] (contiguous); k is rotated and v copied
 * into the pools at the llmk_kv_scatter_batch address of positions[b], exactly as
 * llmk_rope_kv_scatter_batch does with separate q, k, v. head_dim % 16 == 0, ld % 8 == 0,
 * ld >= (n_heads + 2 n_kv_heads) head_dim; qkv, q_out and the pools 16-byte aligned.
 * Replaces ref: engine/batched.cu:52-58 (three projections' outputs, rope_apply, two
 * kv_scatter_batch). New entry point; no single reference function. */
LLMK_API int llmk_qkv_rope_scatter(const uint16_t* qkv, int ld, uint16_t* q_out,
                                   uint16_t* k_pool, uint16_t* v_pool,
                                   const int32_t* block_tables, const int32_t* positions,
                                   const float* inv_freq, int n, int max_pages, int page_size,
                                   int n_heads, int n_kv_heads, int head_dim, void* stream);

/* SwiGLU over the rows of one fused gate/up projection: row r of gate_up holds gate in columns
 * [0, inter) and up in [inter, 2 inter); out[r, j] = llmk_swiglu of (gate[r, j], up[r, j]), out
 * [n_rows, inter]. inter % 8 == 0, n_rows <= 65535, both pointers 16-byte aligned.
 * Replaces ref: engine/batched.cu:67-69 (two projections' outputs, swiglu). New entry point. */
LLMK_API int llmk_swiglu_rows(const uint16_t* gate_up, uint16_t* out, int n_rows, int inter,
                              void* stream);

/* Model shape and RoPE scaling of a Llama-3 decoder (ref: engine/layer.h:6-9 LayerConfig,
 * engine/model.h:7 n_layers / vocab, engine/model.cu:20 rope arguments). */
typedef struct llmk_model_config {
  int n_layers, hidden, n_heads, n_kv_heads, head_dim, inter, vocab;
  float eps;
  double rope_theta, rope_factor, rope_low_freq_factor, rope_high_freq_factor,
      rope_original_max_pos;
} llmk_model_config;

/* One layer's weights in the reference's layout: row-major [out, in] projections, [hidden]
 * norms (ref: engine/layer.h:11-13 LayerWeights). */
typedef struct llmk_layer_weights {
  const uint16_t *attn_norm, *wq, *wk, *wv, *wo, *mlp_norm, *w_gate, *w_up, *w_down;
} llmk_layer_weights;

/* The engine: weights (wq|wk|wv and w_gate|w_up stored concatenated), the paged K and V pools
 * of every layer ([num_pages, 16, n_kv_heads, head_dim], NaN-filled at creation), row inputs,
 * activations, the attention workspace and a GEMM handle -- all allocated by create. A row is
 * one new token of a sequence: (token id, position, block-table row of max_pages page numbers).
 * Decode is one row per sequence; a prompt is one row per prompt token, all with that
 * sequence's table. Requires head_dim 64 and n_heads == 4 n_kv_heads (the attention's
 * preconditions), hidden and inter multiples of 8; page size 16.
 * ref: engine/model.h:9-19 Model, engine/paged.h:6-13 PagedKVCache, engine/batched.h:13-20
 * BatchState; engine/model.cu:9-33, engine/paged.cu:15-28, engine/batched.cu:22-35. */
typedef struct llmk_engine llmk_engine;
LLMK_API int llmk_engine_create(const llmk_model_config* cfg, int max_rows, int max_pages,
                                int num_pages, llmk_engine** out);
/* Lifetime: the engine's own graphs (llmk_engine_forward_graph) are destroyed here, first. A
 * graph the caller captured around llmk_engine_forward (or around anything reading the
 * engine's buffers) references the engine's buffers, its GEMM handle's workspace and
 * hipBLASLt's kernels: destroy it, and let its launched work finish, before destroying the
 * engine. */
LLMK_API void llmk_engine_destroy(llmk_engine* e);

/* Copies the weights (host or device pointers; layers[n_layers]) into the engine. Synchronous. */
LLMK_API int llmk_engine_set_weights(llmk_engine* e, const uint16_t* embed,
                                     const uint16_t* final_norm,
                                     const llmk_layer_weights* layers);

/* Loads dir/weights.bin + dir/index.tsv (Hugging Face tensor names, fp16; the lm head is the
 * embedding matrix). LLMK_ERR_IO for a missing file or tensor, LLMK_ERR_SHAPE for a tensor
 * whose shape differs from the config. Synchronous.
 * ref: engine/model.cu:9-16, engine/layer.cu:12-27, engine/weights.h:9-18, engine/util.h:29-50. */
LLMK_API int llmk_engine_load_weights(llmk_engine* e, const char* dir);

/* Uploads the rows of the next forward pass from HOST arrays: tokens[n_rows],
 * positions[n_rows], block_tables[n_rows, max_pages], and the n_logit_rows row indices whose
 * logits are wanted. Checks every index on the host first (ids < vocab, positions <
 * max_pages * 16, the table entries of every page a row reads < num_pages, logit rows <
 * n_rows): LLMK_ERR_INVALID_VALUE and nothing uploaded otherwise. The copy is enqueued on
 * `stream`; use the same stream for the forward pass. Not capturable (it waits for the
 * previous upload to leave the staging buffer). ref: engine/batched.cu:87-105. */
LLMK_API int llmk_engine_set_rows(llmk_engine* e, int n_rows, const int32_t* tokens,
                                  const int32_t* positions, const int32_t* block_tables,
                                  int n_logit_rows, const int32_t* logit_rows, void* stream);

/* Enqueues the forward pass over the first n_rows uploaded rows: embedding, every layer (K and
 * V of each row written to the pools), final norm, logits [nl, vocab] and their argmax [nl]
 * (nl = n_rows if n_logit_rows < 0, else the uploaded logit rows; no argmax with the option
 * LLMK_ENGINE_HOST_ARGMAX set). n_rows may not exceed the
 * rows of the last llmk_engine_set_rows, nor n_logit_rows its logit rows
 * (LLMK_ERR_INVALID_VALUE before any launch): only those rows' indices were checked.
 * num_splits <= 0 picks the split count: 1 when every uploaded row's attention reads at most 4
 * pages (no merge launch), else LLMK_ATTN_TARGET_BLOCKS / (n_rows * n_kv_heads) at most
 * max_pages; always capped at 32, the workspace. On a stream that is being captured the first
 * rule is skipped, so that a captured pass keeps enough splits for the longer contexts it may
 * be replayed with. Allocates nothing; capturable into a HIP graph for a fixed n_rows.
 * ref: engine/batched.cu:107-120 (decode_step_gpu), :44-72 (layer_forward_batched), :150
 * (argmax_rows in model_decode_batch_greedy). */
LLMK_API int llmk_engine_forward(llmk_engine* e, int n_rows, int n_logit_rows, int num_splits,
                                 void* stream);

/* Device buffers of the engine, for reading results and for tests. */
#define LLMK_BUF_LOGITS 0      /* fp16 [max_rows, vocab]: the last forward's logit rows */
#define LLMK_BUF_NEXT_TOKENS 1 /* int32 [max_rows]: their argmax */
#define LLMK_BUF_RESIDUAL 2    /* fp16 [max_rows, hidden]: the residual stream after the pass */
#define LLMK_BUF_K_POOL 3      /* fp16 [num_pages, 16, n_kv_heads, head_dim] of `layer` */
#define LLMK_BUF_V_POOL 4      /* same, V */
#define LLMK_BUF_EMBED 5       /* fp16 [vocab, hidden]: the embedding (and lm head) matrix */
LLMK_API void* llmk_engine_buffer(llmk_engine* e, int which, int layer);

/* Refills every pool slot with 0x7F7F (fp16 NaN), as at creation. Not capturable. */
LLMK_API int llmk_engine_reset_pools(llmk_engine* e, void* stream);

/* Engine options (llmk_engine_set_option). LLMK_ENGINE_FUSE_FEW_ROWS (default 1): passes of at
 * most LLMK_LINEAR_ROWS_MAX rows run the fused few-rows projections (llmk_linear_rows_*), which
 * give the bits of the unfused pass in 6 launches per layer instead of 10; 0 runs the unfused
 * pass. Changing it drops the cached graphs. New entry point. */
#define LLMK_ENGINE_FUSE_FEW_ROWS 1
/* LLMK_ENGINE_HOST_ARGMAX (default 0): 1 leaves the greedy choice to the host. The forward pass
 * then ends with the logits (LLMK_BUF_NEXT_TOKENS is not written), and the scheduler callbacks
 * (llmk_engine_sched_model) copy them back and pick each row's token on the host, as the
 * reference's scheduler does without gpu_argmax. Setting it allocates the pinned host copy of
 * max_rows logit rows (a hipError_t status on failure); the graph cache of
 * llmk_engine_forward_graph keeps the passes of both settings apart. */
#define LLMK_ENGINE_HOST_ARGMAX 2
LLMK_API int llmk_engine_set_option(llmk_engine* e, int option, int value);

/* Tunes the GEMM plans of a forward pass over n_rows rows with n_logit_rows logit rows (< 0:
 * all rows) -- llmk_blas_tune on every projection shape. Overwrites the activation buffers (not
 * the pools); call it between passes, for the row counts that will repeat (decode batches).
 * Synchronous; not capturable. */
LLMK_API int llmk_engine_tune(llmk_engine* e, int n_rows, int n_logit_rows, void* stream);

/* llmk_engine_forward through a HIP graph cache keyed by (n_rows, n_logit_rows, the resolved
 * split count -- num_splits <= 0 resolved against the rows last uploaded, as above -- and the
 * LLMK_ENGINE_HOST_ARGMAX setting):
 * the first call of a key runs eagerly (choosing the GEMM plans), the second captures the pass
 * on `stream` and instantiates it, later calls launch the instance. Same results as
 * llmk_engine_forward. `stream` must not be the null stream (it cannot be captured) and must
 * not be capturing already; the rows are whatever llmk_engine_set_rows uploaded last. */
LLMK_API int llmk_engine_forward_graph(llmk_engine* e, int n_rows, int n_logit_rows,
                                       int num_splits, void* stream);

/* ------------------------------------------------------------------------------------------
 * Continuous batching: page allocator and request scheduler (host code).
 * ------------------------------------------------------------------------------------------ */

/* Hands out page numbers of the pools from a free list; page 0 first, then ascending, until
 * pages are released or the list is reordered (ref: engine/paging.h:7-23 PageAllocator).
 * alloc returns -1 when no page is free; release rejects a page that is out of range or
 * already free (LLMK_ERR_INVALID_VALUE; the reference does not check). set_free_list reorders
 * the currently free pages (a permutation of them), as the reference's tests shuffle the free
 * list (ref: tests/test_scheduler.cu:21-22). */
typedef struct llmk_page_allocator llmk_page_allocator;
LLMK_API int llmk_pages_create(int num_pages, llmk_page_allocator** out);
LLMK_API void llmk_pages_destroy(llmk_page_allocator* a);
LLMK_API int llmk_pages_total(const llmk_page_allocator* a);
LLMK_API int llmk_pages_num_free(const llmk_page_allocator* a);
LLMK_API int llmk_pages_alloc(llmk_page_allocator* a);
LLMK_API int llmk_pages_release(llmk_page_allocator* a, int page);
LLMK_API int llmk_pages_set_free_list(llmk_page_allocator* a, const int32_t* order, int n);

/* One request (ref: engine/scheduler.h:6-14 Request). The caller fills id, prompt,
 * prompt_len >= 1, max_new >= 1, arrival_step and an output buffer of max_new entries; the
 * scheduler fills n_output and the times (milliseconds from the start of the run, -1 if never
 * reached). */
typedef struct llmk_request {
  int id;
  const int32_t* prompt;
  int prompt_len;
  int max_new;
  int arrival_step;
  int32_t* output;
  int n_output;
  double t_arrive_ms, t_first_ms, t_done_ms;
} llmk_request;

/* One decode step's time split, milliseconds (ref: engine/batched.h:6-11 StepTimes):
 * prep_ms host-side batch preparation and uploads; gpu_ms GPU time from the step's first kernel
 * to its last (events); copy_ms the copy of the results back to the host (the chosen tokens, or
 * the logits in host-argmax mode); convert_ms the half -> float conversion of the logits on the
 * host, and argmax_ms the host argmax over them (host-argmax mode only; the reference's
 * scheduler times that argmax, engine/scheduler.cu:88-93). A decode callback adds its step's
 * times to the fields (they start at 0). */
typedef struct llmk_step_times {
  double prep_ms, gpu_ms, copy_ms, convert_ms, argmax_ms;
} llmk_step_times;

/* Totals of one run (ref: engine/scheduler.h:16-22 SchedulerStats): decode_ms is the
 * host-observed time of the decode steps, and prep_ms .. argmax_ms sum the steps'
 * llmk_step_times, as the reference's time split does. */
typedef struct llmk_sched_stats {
  int decode_steps, total_words, prefills, max_batch, iterations;
  double total_ms, mean_batch, prefill_ms, decode_ms;
  double prep_ms, gpu_ms, copy_ms, convert_ms, argmax_ms;
} llmk_sched_stats;

/* The model as the scheduler sees it. prefill: run prompt[0 .. len) at positions 0 .. len-1 of
 * the sequence whose block table is table[max_pages], write the greedy next token. decode: run
 * n rows (tokens[i] at positions[i] of the sequence with table row i of tables[n, max_pages]),
 * write the n greedy next tokens, and add the step's time split to *times (never NULL; a model
 * that does not measure leaves it alone). Both return LLMK_OK or an error code, which ends the
 * run. */
typedef struct llmk_sched_model {
  void* user;
  int (*prefill)(void* user, const int32_t* table, int max_pages, const int32_t* prompt, int len,
                 int32_t* next_token);
  int (*decode)(void* user, int n, const int32_t* tokens, const int32_t* positions,
                const int32_t* tables, int max_pages, int32_t* next_tokens,
                llmk_step_times* times);
} llmk_sched_model;

/* Runs every request to completion with continuous batching: arrivals by iteration, at most one
 * admission per iteration when max_running allows and the free pages minus the pages running
 * requests may still take cover the request's whole length, the admitted prompt prefilled at
 * once, then one batched decode step for all running requests; a request leaves with max_new
 * tokens and its pages go back to `pages` at once. Requests sorted by arrival_step.
 * LLMK_ERR_CAPACITY if a request can never fit (nothing running and still too few pages, or
 * more pages than max_pages); every page is returned before an error is reported.
 * ref: engine/scheduler.cu:15-106 (run_scheduler). */
LLMK_API int llmk_scheduler_run(llmk_request* reqs, int n_reqs, int max_running, int max_pages,
                                int page_size, llmk_page_allocator* pages,
                                const llmk_sched_model* model, llmk_sched_stats* stats);

/* Scheduler callbacks that run the engine on `stream` (not the null stream): prefill in chunks
 * of at most max_rows rows (eager), decode through llmk_engine_forward_graph, each step's time
 * split measured as the reference measures it (engine/batched.cu:90-150). The greedy tokens come
 * from the engine's GPU argmax (the reference's gpu_argmax mode, ref: engine/batched.cu:146-150),
 * or, with the engine option LLMK_ENGINE_HOST_ARGMAX set, from the logits copied to the host,
 * converted to float and searched there with the reference's rule (the first maximum wins;
 * ref: engine/scheduler.cu:9-13,88-93, engine/batched.cu:126-139), for prompts as well. The
 * engine's block tables must have the same max_pages. */
LLMK_API int llmk_engine_sched_model(llmk_engine* e, void* stream, llmk_sched_model* out);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* LLMK_H */
