// llmk.hpp - the reference engine's C++ operator API on top of libllmk's C-ABI.
//
// Each function below has the name, argument list and argument meaning of the reference
// launcher it replaces (ref: kernels/*.cuh of JayeshNikam36/cuda-llm-engine), with
// cudaStream_t -> hipStream_t (default: the null stream) and __half from <hip/hip_fp16.h>.
// Including this header in place of the reference's kernels/*.cuh lets engine code such as
// ref: engine/batched.cu:44-72 call the MI355X kernels unchanged.
//
// Error behaviour follows the reference: launchers return void; a launch error is left in
// HIP's last-error state for the caller's hipGetLastError() (ref: engine/batched.cu:118); a
// violated precondition (hidden % 8, kvdim % 8, 16-byte alignment) is a fatal host error,
// printed to stderr followed by exit(1), like the reference's CUDA_CHECK (ref: engine/util.h:8-10).
// A zero-sized call is a no-op.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <vector>

#include "llmk.h"

namespace llmk_shim {
inline void check(int status, const char* fn) {
  if (status >= LLMK_ERR_INVALID_VALUE && status <= LLMK_ERR_UNSUPPORTED) {
    std::fprintf(stderr, "%s: %s\n", fn, llmk_error_string(status));
    std::exit(1);
  }
}
inline uint16_t* h(__half* p) { return reinterpret_cast<uint16_t*>(p); }
inline const uint16_t* h(const __half* p) { return reinterpret_cast<const uint16_t*>(p); }
}  // namespace llmk_shim

// ref: kernels/embedding.cuh:6-7
inline void embedding_lookup(const __half* table, const int* ids, __half* out, int n_tokens,
                             int hidden, hipStream_t stream = 0) {
  llmk_shim::check(llmk_embedding_lookup(llmk_shim::h(table), ids, llmk_shim::h(out), n_tokens,
                                         hidden, stream),
                   "embedding_lookup");
}

// ref: kernels/rmsnorm.cuh:6-7
inline void rmsnorm(const __half* x, const __half* w, __half* out, int n_rows, int hidden,
                    float eps, hipStream_t stream = 0) {
  llmk_shim::check(llmk_rmsnorm(llmk_shim::h(x), llmk_shim::h(w), llmk_shim::h(out), n_rows,
                                hidden, eps, stream),
                   "rmsnorm");
}

// ref: kernels/residual_add.cuh:6
inline void residual_add(const __half* a, const __half* b, __half* out, size_t n,
                         hipStream_t stream = 0) {
  llmk_shim::check(
      llmk_residual_add(llmk_shim::h(a), llmk_shim::h(b), llmk_shim::h(out), n, stream),
      "residual_add");
}

// New fused entry point: residual_add(residual, x, residual) then rmsnorm(residual, w, out).
inline void add_rmsnorm(__half* residual, const __half* x, const __half* w, __half* out,
                        int n_rows, int hidden, float eps, hipStream_t stream = 0) {
  llmk_shim::check(llmk_add_rmsnorm(llmk_shim::h(residual), llmk_shim::h(x), llmk_shim::h(w),
                                    llmk_shim::h(out), n_rows, hidden, eps, stream),
                   "add_rmsnorm");
}

// ref: kernels/rope.cuh:7-9
inline std::vector<float> compute_rope_inv_freq(int head_dim, double theta, double factor,
                                                double low_freq_factor, double high_freq_factor,
                                                double original_max_pos) {
  std::vector<float> out(head_dim > 0 ? head_dim / 2 : 0);
  llmk_shim::check(llmk_compute_rope_inv_freq(head_dim, theta, factor, low_freq_factor,
                                              high_freq_factor, original_max_pos, out.data()),
                   "compute_rope_inv_freq");
  return out;
}

// ref: kernels/rope.cuh:13-15
inline void rope_apply(__half* q, __half* k, const int* positions, const float* inv_freq,
                       int n_tokens, int n_heads, int n_kv_heads, int head_dim,
                       hipStream_t stream = 0) {
  llmk_shim::check(llmk_rope_apply(llmk_shim::h(q), llmk_shim::h(k), positions, inv_freq,
                                   n_tokens, n_heads, n_kv_heads, head_dim, stream),
                   "rope_apply");
}

// ref: kernels/swiglu.cuh:6
inline void swiglu(const __half* gate, const __half* up, __half* out, size_t n,
                   hipStream_t stream = 0) {
  llmk_shim::check(
      llmk_swiglu(llmk_shim::h(gate), llmk_shim::h(up), llmk_shim::h(out), n, stream), "swiglu");
}

// ref: kernels/kv_scatter.cuh:7-8
inline void kv_scatter(const __half* src, __half* pool, const int* block_table, int start_pos,
                       int T, int page_size, int kvdim, hipStream_t stream = 0) {
  llmk_shim::check(llmk_kv_scatter(llmk_shim::h(src), llmk_shim::h(pool), block_table, start_pos,
                                   T, page_size, kvdim, stream),
                   "kv_scatter");
}

// ref: kernels/kv_scatter.cuh:12-13
inline void kv_scatter_batch(const __half* src, __half* pool, const int* block_tables,
                             const int* positions, int n, int max_pages, int page_size,
                             int kvdim, hipStream_t stream = 0) {
  llmk_shim::check(llmk_kv_scatter_batch(llmk_shim::h(src), llmk_shim::h(pool), block_tables,
                                         positions, n, max_pages, page_size, kvdim, stream),
                   "kv_scatter_batch");
}

// New fused decode entry point: rope_apply(q, k, ...) then kv_scatter_batch of k and v, with k
// left unrotated (decode attention reads K from the pool only).
inline void rope_kv_scatter_batch(__half* q, const __half* k, const __half* v, __half* k_pool,
                                  __half* v_pool, const int* block_tables, const int* positions,
                                  const float* inv_freq, int n, int max_pages, int page_size,
                                  int n_heads, int n_kv_heads, int head_dim,
                                  hipStream_t stream = 0) {
  llmk_shim::check(
      llmk_rope_kv_scatter_batch(llmk_shim::h(q), llmk_shim::h(k), llmk_shim::h(v),
                                 llmk_shim::h(k_pool), llmk_shim::h(v_pool), block_tables,
                                 positions, inv_freq, n, max_pages, page_size, n_heads,
                                 n_kv_heads, head_dim, stream),
      "rope_kv_scatter_batch");
}

// ref: kernels/attention_decode_fast.cuh:6
inline size_t attention_decode_fast_workspace_floats(int n_seq, int n_heads, int num_splits) {
  return llmk_attention_decode_fast_workspace_floats(n_seq, n_heads, num_splits);
}

// ref: kernels/attention_decode_fast.cuh:14-18. Preconditions as the reference's (page_size 16,
// head_dim 64, n_heads == 4 * n_kv_heads): a violation is a fatal host error.
inline void attention_decode_fast(const __half* q, const __half* k_pool, const __half* v_pool,
                                  const int* block_tables, const int* seq_lens, __half* out,
                                  float* workspace, int n_seq, int max_pages, int page_size,
                                  int n_heads, int n_kv_heads, int head_dim, int num_splits,
                                  hipStream_t stream = 0) {
  llmk_shim::check(
      llmk_attention_decode_fast(llmk_shim::h(q), llmk_shim::h(k_pool), llmk_shim::h(v_pool),
                                 block_tables, seq_lens, llmk_shim::h(out), workspace, n_seq,
                                 max_pages, page_size, n_heads, n_kv_heads, head_dim,
                                 num_splits, stream),
      "attention_decode_fast");
}

// The reference's split-count rule (ref: kernels/attention_decode_fast.cuh:22-29), with the
// default target rescaled for MI355X (LLMK_ATTN_TARGET_BLOCKS).
inline int choose_num_splits(int n_seq, int n_kv_heads, int max_seq_len,
                             int target_blocks = LLMK_ATTN_TARGET_BLOCKS) {
  int splits = target_blocks / (n_seq * n_kv_heads);
  const int max_splits = (max_seq_len + 15) / 16;  // never more splits than pages
  if (splits > max_splits) splits = max_splits;
  if (splits > 32) splits = 32;  // the engine's workspace holds 32 (ref: engine/batched.cu:29)
  if (splits < 1) splits = 1;
  return splits;
}

// ref: kernels/argmax.cuh:7
inline void argmax_rows(const __half* logits, int* out, int n_rows, int vocab,
                        hipStream_t stream = 0) {
  llmk_shim::check(llmk_argmax_rows(llmk_shim::h(logits), out, n_rows, vocab, stream),
                   "argmax_rows");
}
