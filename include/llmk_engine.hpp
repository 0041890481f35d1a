// llmk_engine.hpp - C++ face of libllmk's decode step and continuous batching, on top of the
// C-ABI (llmk.h), with the reference engine's names where a concept maps one to one.
//
//  - linear(): ref: kernels/linear.cuh:5-7, with the cuBLAS handle replaced by a libllmk GEMM
//    handle (llmk_blas*, hipBLASLt underneath).
//  - PageAllocator, Request, SchedulerStats, run_scheduler(): ref: engine/paging.h:7-23,
//    engine/scheduler.h:6-27. The reference's scheduler takes (Model&, PagedKVCache&,
//    BatchState&): here one llmk::Engine holds the weights, the pools and the batch buffers, so
//    run_scheduler takes the engine, the allocator and a stream.
//  - llmk::Engine: the token-row forward pass (engine.cpp), RAII over llmk_engine*.
//
// Error behaviour follows the reference: a failed call is a fatal host error, printed to
// stderr followed by exit(1) (ref: engine/util.h:8-10, engine/paging.h:17).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "llmk.h"

namespace llmk_shim_engine {
inline void check(int status, const char* fn) {
  if (status != LLMK_OK) {
    std::fprintf(stderr, "%s: %s\n", fn, llmk_error_string(status));
    std::exit(1);
  }
}
}  // namespace llmk_shim_engine

// ref: kernels/linear.cuh:7 -- y[T, out] = x[T, in] * W^T, W [out, in] row-major.
inline void linear(llmk_blas* handle, const __half* x, const __half* w, __half* y, int T,
                   int in_features, int out_features, hipStream_t stream = 0) {
  llmk_shim_engine::check(
      llmk_linear(handle, reinterpret_cast<const uint16_t*>(x),
                  reinterpret_cast<const uint16_t*>(w), reinterpret_cast<uint16_t*>(y), T,
                  in_features, out_features, stream),
      "linear");
}

namespace llmk {

// Llama-3.2-1B (ref: engine/layer.h:6-9, engine/model.h:7, engine/model.cu:20).
inline llmk_model_config llama32_1b_config() {
  llmk_model_config c;
  c.n_layers = 16;
  c.hidden = 2048;
  c.n_heads = 32;
  c.n_kv_heads = 8;
  c.head_dim = 64;
  c.inter = 8192;
  c.vocab = 128256;
  c.eps = 1e-5f;
  c.rope_theta = 500000.0;
  c.rope_factor = 32.0;
  c.rope_low_freq_factor = 1.0;
  c.rope_high_freq_factor = 4.0;
  c.rope_original_max_pos = 8192.0;
  return c;
}

class Engine {
 public:
  Engine(const llmk_model_config& cfg, int max_rows, int max_pages, int num_pages)
      : cfg_(cfg), max_rows_(max_rows), max_pages_(max_pages), num_pages_(num_pages) {
    llmk_shim_engine::check(llmk_engine_create(&cfg, max_rows, max_pages, num_pages, &e_),
                            "llmk_engine_create");
  }
  ~Engine() { llmk_engine_destroy(e_); }
  Engine(const Engine&) = delete;
  Engine& operator=(const Engine&) = delete;

  // ref: engine/model.cu:9-16 (load_model reads weights.bin + index.tsv)
  void load_weights(const std::string& dir) {
    llmk_shim_engine::check(llmk_engine_load_weights(e_, dir.c_str()), "llmk_engine_load_weights");
  }
  void set_weights(const __half* embed, const __half* final_norm,
                   const std::vector<llmk_layer_weights>& layers) {
    llmk_shim_engine::check(
        llmk_engine_set_weights(e_, reinterpret_cast<const uint16_t*>(embed),
                                reinterpret_cast<const uint16_t*>(final_norm), layers.data()),
        "llmk_engine_set_weights");
  }
  void set_rows(const std::vector<int32_t>& tokens, const std::vector<int32_t>& positions,
                const std::vector<int32_t>& tables, const std::vector<int32_t>& logit_rows = {},
                hipStream_t stream = 0) {
    llmk_shim_engine::check(
        llmk_engine_set_rows(e_, (int)tokens.size(), tokens.data(), positions.data(),
                             tables.data(), (int)logit_rows.size(),
                             logit_rows.empty() ? nullptr : logit_rows.data(), stream),
        "llmk_engine_set_rows");
  }
  void forward(int n_rows, int n_logit_rows = -1, int num_splits = 0, hipStream_t stream = 0) {
    llmk_shim_engine::check(llmk_engine_forward(e_, n_rows, n_logit_rows, num_splits, stream),
                            "llmk_engine_forward");
  }
  void tune(int n_rows, int n_logit_rows = -1, hipStream_t stream = 0) {
    llmk_shim_engine::check(llmk_engine_tune(e_, n_rows, n_logit_rows, stream),
                            "llmk_engine_tune");
  }
  const __half* logits() const {
    return static_cast<const __half*>(llmk_engine_buffer(e_, LLMK_BUF_LOGITS, 0));
  }
  const int32_t* next_tokens() const {
    return static_cast<const int32_t*>(llmk_engine_buffer(e_, LLMK_BUF_NEXT_TOKENS, 0));
  }
  llmk_engine* get() const { return e_; }
  const llmk_model_config& config() const { return cfg_; }
  int max_rows() const { return max_rows_; }
  int max_pages() const { return max_pages_; }
  int num_pages() const { return num_pages_; }

 private:
  llmk_model_config cfg_;
  int max_rows_, max_pages_, num_pages_;
  llmk_engine* e_ = nullptr;
};

// ref: engine/paging.h:7-23
class PageAllocator {
 public:
  explicit PageAllocator(int n) {
    llmk_shim_engine::check(llmk_pages_create(n, &a_), "PageAllocator");
  }
  ~PageAllocator() { llmk_pages_destroy(a_); }
  PageAllocator(const PageAllocator&) = delete;
  PageAllocator& operator=(const PageAllocator&) = delete;
  int num_free() const { return llmk_pages_num_free(a_); }
  bool can_alloc(int n) const { return num_free() >= n; }
  int total() const { return llmk_pages_total(a_); }
  int alloc() {
    const int p = llmk_pages_alloc(a_);
    if (p < 0) {
      std::fprintf(stderr, "PageAllocator: out of pages\n");
      std::exit(1);
    }
    return p;
  }
  void release(int p) { llmk_shim_engine::check(llmk_pages_release(a_, p), "PageAllocator"); }
  void set_free_list(const std::vector<int32_t>& order) {
    llmk_shim_engine::check(llmk_pages_set_free_list(a_, order.data(), (int)order.size()),
                            "PageAllocator");
  }
  llmk_page_allocator* get() const { return a_; }

 private:
  llmk_page_allocator* a_ = nullptr;
};

// ref: engine/scheduler.h:6-14
struct Request {
  int id = 0;
  std::vector<int> prompt;
  int max_new = 32;
  int arrival_step = 0;
  std::vector<int> output;
  double t_arrive_ms = -1, t_first_ms = -1, t_done_ms = -1;
};

// ref: engine/scheduler.h:16-22 (decode_ms: the host-observed time of the decode steps; the
// time split summed over the decode steps, as the reference's)
struct SchedulerStats {
  int decode_steps = 0;
  int total_words = 0;
  double total_ms = 0, mean_batch = 0;
  double prefill_ms = 0, decode_ms = 0;
  double prep_ms = 0, gpu_ms = 0, copy_ms = 0, convert_ms = 0, argmax_ms = 0;
};

// ref: engine/scheduler.h:24-27, engine/scheduler.cu:15-106. gpu_argmax (the reference's
// parameter, same default): the greedy tokens come from the engine's GPU argmax; otherwise the
// logits are copied back and searched on the host (LLMK_ENGINE_HOST_ARGMAX, left set as chosen
// here). `stream` should be a created stream: decode steps then replay HIP graphs.
inline SchedulerStats run_scheduler(Engine& e, PageAllocator& pages, std::vector<Request>& reqs,
                                    int max_running, hipStream_t stream,
                                    bool gpu_argmax = false) {
  llmk_shim_engine::check(llmk_engine_set_option(e.get(), LLMK_ENGINE_HOST_ARGMAX,
                                                 gpu_argmax ? 0 : 1),
                          "run_scheduler");
  std::vector<llmk_request> rq(reqs.size());
  for (size_t i = 0; i < reqs.size(); ++i) {
    reqs[i].output.assign(reqs[i].max_new > 0 ? reqs[i].max_new : 1, 0);
    rq[i].id = reqs[i].id;
    rq[i].prompt = reqs[i].prompt.data();
    rq[i].prompt_len = (int)reqs[i].prompt.size();
    rq[i].max_new = reqs[i].max_new;
    rq[i].arrival_step = reqs[i].arrival_step;
    rq[i].output = reqs[i].output.data();
  }
  llmk_sched_model model;
  llmk_shim_engine::check(llmk_engine_sched_model(e.get(), stream, &model), "run_scheduler");
  llmk_sched_stats st;
  llmk_shim_engine::check(llmk_scheduler_run(rq.data(), (int)rq.size(), max_running,
                                             e.max_pages(), 16, pages.get(), &model, &st),
                          "run_scheduler");
  for (size_t i = 0; i < reqs.size(); ++i) {
    reqs[i].output.resize(rq[i].n_output);
    reqs[i].t_arrive_ms = rq[i].t_arrive_ms;
    reqs[i].t_first_ms = rq[i].t_first_ms;
    reqs[i].t_done_ms = rq[i].t_done_ms;
  }
  SchedulerStats out;
  out.decode_steps = st.decode_steps;
  out.total_words = st.total_words;
  out.total_ms = st.total_ms;
  out.mean_batch = st.mean_batch;
  out.prefill_ms = st.prefill_ms;
  out.decode_ms = st.decode_ms;
  out.prep_ms = st.prep_ms;
  out.gpu_ms = st.gpu_ms;
  out.copy_ms = st.copy_ms;
  out.convert_ms = st.convert_ms;
  out.argmax_ms = st.argmax_ms;
  return out;
}

}  // namespace llmk
