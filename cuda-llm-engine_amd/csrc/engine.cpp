// The decode-step engine: a Llama-3 decoder's forward pass over a batch of token rows, each row
// one new token of some sequence at some position, with its K and V stored in the paged pools.
// ref: engine/batched.cu:44-72 (layer_forward_batched), :81-120 (decode_step_gpu),
// engine/model.cu:9-33 (load_model), engine/layer.cu:12-27 (load_layer_weights),
// engine/paged.cu:15-28 (alloc_paged_cache).
//
// A row is (token, position, block-table row). A decode step has one row per running sequence;
// a prompt of L tokens is L rows of one sequence at positions start..start+L-1, all with that
// sequence's table (each row's attention covers positions <= its own, and every row's K and V
// are in the pool before the attention runs). So one path serves batched decode, prefill and any
// mix of the two.
//
// Per layer, with the weights stored fused (wq|wk|wv as one [qdim + 2 kvdim, hidden] matrix,
// w_gate|w_up as one [2 inter, hidden] matrix; both plain concatenations of the reference's
// row-major matrices):
//   qkv    = normed @ wqkv^T                      (one GEMM for the three projections)
//   q, K, V: llmk_qkv_rope_scatter                (RoPE on q and k, K/V into the pools)
//   attn   = llmk_attention_decode_fast(q, pools)
//   proj   = attn @ wo^T
//   residual += proj; normed = rmsnorm(residual)  (llmk_add_rmsnorm)
//   gu     = normed @ wgu^T                       (one GEMM for gate and up)
//   act    = swiglu(gu)                           (llmk_swiglu_rows)
//   proj   = act @ wdown^T
//   residual += proj; normed = rmsnorm(residual) with the next layer's (or the final) norm
// Then the logits of the selected rows, lm head = the embedding matrix (tied weights, ref:
// engine/batched.cu:117), and their argmax.
//
// Every buffer is allocated at creation; llmk_engine_forward allocates nothing and only enqueues
// kernels on its stream, so it can be captured into a HIP graph (one graph per row count).
#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include <chrono>
#include <map>
#include <string>
#include <tuple>
#include <unordered_map>
#include <vector>

#include "llmk.h"

namespace {

constexpr int kPage = 16;       // page size of the pools (the attention's precondition)
constexpr int kMaxSplits = 32;  // attention workspace slots per row (ref: engine/batched.cu:29)

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

struct LayerPtrs {
  uint16_t *attn_norm, *wqkv, *wo, *mlp_norm, *wgu, *wdown;
};

}  // namespace

struct llmk_engine {
  llmk_model_config cfg;
  int max_rows = 0, max_pages = 0, num_pages = 0;
  int qdim = 0, kvdim = 0, qkvdim = 0;
  llmk_blas* blas = nullptr;

  // weights (one allocation)
  void* wbuf = nullptr;
  uint16_t *embed = nullptr, *final_norm = nullptr;
  std::vector<LayerPtrs> layers;

  // paged K and V pools, [num_pages, 16, n_kv_heads, head_dim] per layer (one allocation)
  void* pool_buf = nullptr;
  size_t pool_elems = 0;  // elements of one pool
  std::vector<uint16_t*> k_pool, v_pool;

  // row inputs (one allocation, uploaded by llmk_engine_set_rows from a pinned staging copy)
  void* in_buf = nullptr;
  void* staging = nullptr;
  size_t in_bytes = 0;
  hipEvent_t staged = nullptr;
  int32_t *tokens = nullptr, *positions = nullptr, *lens = nullptr, *logit_rows = nullptr,
          *tables = nullptr;

  // activations (one allocation)
  void* act_buf = nullptr;
  float* inv_freq = nullptr;
  uint16_t *x = nullptr, *normed = nullptr, *qkv = nullptr, *q = nullptr, *attn = nullptr,
           *proj = nullptr, *gu = nullptr, *act = nullptr, *fin = nullptr, *logits = nullptr;
  int32_t* next = nullptr;
  float* ws = nullptr;

  // Pages the longest attention of the rows last set reads (position / 16 + 1).
  int rows_span = 0;
  // Rows and logit rows uploaded by the last llmk_engine_set_rows: a pass may not ask for more,
  // since the device copies past them hold no checked indices.
  int rows_set = 0, logit_rows_set = 0;

  // HIP graphs of the forward pass, keyed by (n_rows, n_logit_rows, resolved num_splits,
  // host_argmax: whether the pass ends before the GPU argmax)
  struct Graph {
    bool seen = false;
    hipGraphExec_t exec = nullptr;
  };
  std::map<std::tuple<int, int, int, int>, Graph> graphs;
  hipStream_t sched_stream = nullptr;  // the stream the scheduler callbacks run on
  bool fuse_rows = true;  // passes of <= LLMK_LINEAR_ROWS_MAX rows use the fused projections
  // LLMK_ENGINE_HOST_ARGMAX: the pass ends with the logits; the scheduler callbacks copy them
  // to host_logits (pinned, max_rows rows), convert them into host_float and pick there.
  bool host_argmax = false;
  uint16_t* host_logits = nullptr;
  std::vector<float> host_float;
  hipEvent_t step_begin = nullptr, step_end = nullptr;  // a decode step's GPU time
};

namespace {

// Carves consecutive 256-byte-aligned pieces out of one allocation.
struct Carver {
  char* base;
  size_t off = 0;
  template <typename T>
  T* take(size_t count) {
    T* p = reinterpret_cast<T*>(base ? base + off : nullptr);
    off += align256(count * sizeof(T));
    return p;
  }
};

int valid_config(const llmk_model_config& c) {
  if (c.n_layers < 0 || c.hidden <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 ||
      c.head_dim <= 0 || c.inter <= 0 || c.vocab <= 0 || !(c.eps > 0.0f))
    return LLMK_ERR_INVALID_VALUE;
  // The attention's preconditions (head_dim 64, 4 query heads per kv head), 16-byte rows.
  if (c.head_dim != 64 || c.n_heads != 4 * c.n_kv_heads || c.hidden % 8 != 0 ||
      c.inter % 8 != 0)
    return LLMK_ERR_SHAPE;
  return LLMK_OK;
}

// Weight carving: the same order is used to size and to place.
void carve_weights(llmk_engine* e, Carver& c) {
  const llmk_model_config& m = e->cfg;
  const size_t H = m.hidden;
  e->embed = c.take<uint16_t>((size_t)m.vocab * H);
  e->final_norm = c.take<uint16_t>(H);
  e->layers.resize(m.n_layers);
  for (auto& l : e->layers) {
    l.attn_norm = c.take<uint16_t>(H);
    l.wqkv = c.take<uint16_t>((size_t)e->qkvdim * H);
    l.wo = c.take<uint16_t>(H * e->qdim);
    l.mlp_norm = c.take<uint16_t>(H);
    l.wgu = c.take<uint16_t>(2 * (size_t)m.inter * H);
    l.wdown = c.take<uint16_t>(H * m.inter);
  }
}

void carve_inputs(llmk_engine* e, Carver& c) {
  const size_t R = e->max_rows;
  e->tokens = c.take<int32_t>(R);
  e->positions = c.take<int32_t>(R);
  e->lens = c.take<int32_t>(R);
  e->logit_rows = c.take<int32_t>(R);
  e->tables = c.take<int32_t>(R * e->max_pages);
}

void carve_activations(llmk_engine* e, Carver& c) {
  const llmk_model_config& m = e->cfg;
  const size_t R = e->max_rows, H = m.hidden;
  e->inv_freq = c.take<float>(m.head_dim / 2);
  e->x = c.take<uint16_t>(R * H);
  e->normed = c.take<uint16_t>(R * H);
  e->qkv = c.take<uint16_t>(R * e->qkvdim);
  e->q = c.take<uint16_t>(R * e->qdim);
  e->attn = c.take<uint16_t>(R * e->qdim);
  e->proj = c.take<uint16_t>(R * H);
  e->gu = c.take<uint16_t>(R * 2 * m.inter);
  e->act = c.take<uint16_t>(R * m.inter);
  e->fin = c.take<uint16_t>(R * H);
  e->logits = c.take<uint16_t>(R * m.vocab);
  e->next = c.take<int32_t>(R);
  e->ws = c.take<float>(llmk_attention_decode_fast_workspace_floats(e->max_rows, m.n_heads,
                                                                    kMaxSplits));
}

void release(llmk_engine* e) {
  for (auto& kv : e->graphs)
    if (kv.second.exec) (void)hipGraphExecDestroy(kv.second.exec);
  if (e->blas) llmk_blas_destroy(e->blas);
  if (e->wbuf) (void)hipFree(e->wbuf);
  if (e->pool_buf) (void)hipFree(e->pool_buf);
  if (e->in_buf) (void)hipFree(e->in_buf);
  if (e->act_buf) (void)hipFree(e->act_buf);
  if (e->staging) (void)hipHostFree(e->staging);
  if (e->staged) (void)hipEventDestroy(e->staged);
  if (e->host_logits) (void)hipHostFree(e->host_logits);
  if (e->step_begin) (void)hipEventDestroy(e->step_begin);
  if (e->step_end) (void)hipEventDestroy(e->step_end);
  delete e;
}

}  // namespace

extern "C" int llmk_engine_create(const llmk_model_config* cfg, int max_rows, int max_pages,
                                  int num_pages, llmk_engine** out) {
  if (!cfg || !out) return LLMK_ERR_INVALID_VALUE;
  *out = nullptr;
  int st = valid_config(*cfg);
  if (st != LLMK_OK) return st;
  if (max_rows <= 0 || max_pages <= 0 || num_pages <= 0) return LLMK_ERR_INVALID_VALUE;
  if (max_rows > 65535) return LLMK_ERR_UNSUPPORTED;  // the attention's grid limit
  llmk_engine* e = new llmk_engine();
  e->cfg = *cfg;
  e->max_rows = max_rows;
  e->max_pages = max_pages;
  e->num_pages = num_pages;
  e->qdim = cfg->n_heads * cfg->head_dim;
  e->kvdim = cfg->n_kv_heads * cfg->head_dim;
  e->qkvdim = e->qdim + 2 * e->kvdim;

  Carver cw{nullptr}, ci{nullptr}, ca{nullptr};
  carve_weights(e, cw);
  carve_inputs(e, ci);
  carve_activations(e, ca);
  e->pool_elems = (size_t)num_pages * kPage * e->kvdim;
  e->in_bytes = ci.off;
  st = (int)hipMalloc(&e->wbuf, cw.off);
  if (st == LLMK_OK) st = (int)hipMalloc(&e->in_buf, ci.off);
  if (st == LLMK_OK) st = (int)hipMalloc(&e->act_buf, ca.off);
  if (st == LLMK_OK && cfg->n_layers > 0)
    st = (int)hipMalloc(&e->pool_buf, 2 * (size_t)cfg->n_layers * e->pool_elems * 2);
  if (st == LLMK_OK) st = (int)hipHostMalloc(&e->staging, ci.off, hipHostMallocDefault);
  if (st == LLMK_OK) memset(e->staging, 0, ci.off);  // every upload copies all of it
  if (st == LLMK_OK) st = (int)hipEventCreateWithFlags(&e->staged, hipEventDisableTiming);
  if (st == LLMK_OK) st = (int)hipEventCreate(&e->step_begin);
  if (st == LLMK_OK) st = (int)hipEventCreate(&e->step_end);
  if (st == LLMK_OK) st = llmk_blas_create(&e->blas);
  if (st != LLMK_OK) {
    release(e);
    return st;
  }
  Carver w2{static_cast<char*>(e->wbuf)}, i2{static_cast<char*>(e->in_buf)},
      a2{static_cast<char*>(e->act_buf)};
  carve_weights(e, w2);
  carve_inputs(e, i2);
  carve_activations(e, a2);
  for (int l = 0; l < cfg->n_layers; ++l) {
    uint16_t* base = static_cast<uint16_t*>(e->pool_buf) + 2 * (size_t)l * e->pool_elems;
    e->k_pool.push_back(base);
    e->v_pool.push_back(base + e->pool_elems);
  }
  // Unwritten pool slots hold 0x7F7F, an fp16 NaN, so a read of an unmapped slot poisons the
  // output (ref: engine/paged.cu:22).
  if (e->pool_buf)
    st = (int)hipMemset(e->pool_buf, 0x7F, 2 * (size_t)cfg->n_layers * e->pool_elems * 2);
  // Zeroed row inputs: a forward before any llmk_engine_set_rows reads valid rows.
  if (st == LLMK_OK) st = (int)hipMemset(e->in_buf, 0, ci.off);
  std::vector<float> inv(cfg->head_dim / 2);
  if (st == LLMK_OK)
    st = llmk_compute_rope_inv_freq(cfg->head_dim, cfg->rope_theta, cfg->rope_factor,
                                    cfg->rope_low_freq_factor, cfg->rope_high_freq_factor,
                                    cfg->rope_original_max_pos, inv.data());
  if (st == LLMK_OK)
    st = (int)hipMemcpy(e->inv_freq, inv.data(), inv.size() * sizeof(float),
                        hipMemcpyHostToDevice);
  if (st != LLMK_OK) {
    release(e);
    return st;
  }
  *out = e;
  return LLMK_OK;
}

extern "C" void llmk_engine_destroy(llmk_engine* e) {
  if (e) release(e);
}

extern "C" int llmk_engine_set_weights(llmk_engine* e, const uint16_t* embed,
                                       const uint16_t* final_norm,
                                       const llmk_layer_weights* layers) {
  if (!e || !embed || !final_norm || (e->cfg.n_layers > 0 && !layers))
    return LLMK_ERR_INVALID_VALUE;
  const llmk_model_config& m = e->cfg;
  const size_t H = m.hidden;
  auto cp = [](void* dst, const void* src, size_t elems) {
    return (int)hipMemcpy(dst, src, elems * 2, hipMemcpyDefault);
  };
  int st = cp(e->embed, embed, (size_t)m.vocab * H);
  if (st == LLMK_OK) st = cp(e->final_norm, final_norm, H);
  for (int l = 0; l < m.n_layers && st == LLMK_OK; ++l) {
    const llmk_layer_weights& w = layers[l];
    const LayerPtrs& d = e->layers[l];
    if (!w.attn_norm || !w.wq || !w.wk || !w.wv || !w.wo || !w.mlp_norm || !w.w_gate ||
        !w.w_up || !w.w_down)
      return LLMK_ERR_INVALID_VALUE;
    st = cp(d.attn_norm, w.attn_norm, H);
    if (st == LLMK_OK) st = cp(d.wqkv, w.wq, e->qdim * H);
    if (st == LLMK_OK) st = cp(d.wqkv + e->qdim * H, w.wk, e->kvdim * H);
    if (st == LLMK_OK) st = cp(d.wqkv + (e->qdim + e->kvdim) * H, w.wv, e->kvdim * H);
    if (st == LLMK_OK) st = cp(d.wo, w.wo, H * e->qdim);
    if (st == LLMK_OK) st = cp(d.mlp_norm, w.mlp_norm, H);
    if (st == LLMK_OK) st = cp(d.wgu, w.w_gate, (size_t)m.inter * H);
    if (st == LLMK_OK) st = cp(d.wgu + (size_t)m.inter * H, w.w_up, (size_t)m.inter * H);
    if (st == LLMK_OK) st = cp(d.wdown, w.w_down, H * m.inter);
  }
  return st;
}

// ---------------------------------------------------------------------------------------------
// Weight files: weights.bin holds the fp16 tensors back to back; index.tsv has one line per
// tensor, "name<TAB>offset<TAB>nbytes<TAB>d0,d1,..." (ref: scripts/export_for_cpp.py:14-24,
// scripts/make_index_tsv.py:5-7, read by engine/util.h:29-50). Tensors use the Hugging Face
// names (ref: engine/layer.cu:13-27, engine/model.cu:12-15).
// ---------------------------------------------------------------------------------------------
namespace {

struct TensorEntry {
  unsigned long long offset = 0, nbytes = 0;
  std::vector<long long> shape;
};

int parse_index(const std::string& path, std::unordered_map<std::string, TensorEntry>* out) {
  FILE* f = fopen(path.c_str(), "r");
  if (!f) return LLMK_ERR_IO;
  char line[2048];
  while (fgets(line, sizeof(line), f)) {
    char name[1024], shape[512];
    unsigned long long off = 0, nb = 0;
    if (sscanf(line, "%1023[^\t]\t%llu\t%llu\t%511s", name, &off, &nb, shape) != 4) continue;
    TensorEntry t;
    t.offset = off;
    t.nbytes = nb;
    for (char* p = shape; *p;) {
      char* end = nullptr;
      t.shape.push_back(strtoll(p, &end, 10));
      if (end == p) break;
      p = *end == ',' ? end + 1 : end;
    }
    (*out)[name] = t;
  }
  fclose(f);
  return LLMK_OK;
}

}  // namespace

extern "C" int llmk_engine_load_weights(llmk_engine* e, const char* dir) {
  if (!e || !dir) return LLMK_ERR_INVALID_VALUE;
  std::unordered_map<std::string, TensorEntry> index;
  int st = parse_index(std::string(dir) + "/index.tsv", &index);
  if (st != LLMK_OK) return st;
  const int fd = open((std::string(dir) + "/weights.bin").c_str(), O_RDONLY);
  if (fd < 0) return LLMK_ERR_IO;
  const size_t chunk = 64u << 20;
  void* host = nullptr;
  st = (int)hipHostMalloc(&host, chunk, hipHostMallocDefault);
  // Copies tensor `name` of shape {d0, d1} (d1 = 0 for a vector) to dst.
  auto load = [&](const std::string& name, long long d0, long long d1, uint16_t* dst) -> int {
    auto it = index.find(name);
    if (it == index.end()) return LLMK_ERR_IO;
    const TensorEntry& t = it->second;
    const bool shape_ok = d1 == 0 ? (t.shape.size() == 1 && t.shape[0] == d0)
                                  : (t.shape.size() == 2 && t.shape[0] == d0 && t.shape[1] == d1);
    const unsigned long long want = (unsigned long long)d0 * (d1 ? d1 : 1) * 2;
    if (!shape_ok || t.nbytes != want) return LLMK_ERR_SHAPE;
    for (unsigned long long done = 0; done < want;) {
      const size_t n = (size_t)(want - done < chunk ? want - done : chunk);
      const ssize_t got = pread(fd, host, n, (off_t)(t.offset + done));
      if (got != (ssize_t)n) return LLMK_ERR_IO;
      const int s = (int)hipMemcpy(reinterpret_cast<char*>(dst) + done, host, n,
                                   hipMemcpyHostToDevice);
      if (s != LLMK_OK) return s;
      done += n;
    }
    return LLMK_OK;
  };
  const llmk_model_config& m = e->cfg;
  const long long H = m.hidden;
  if (st == LLMK_OK) st = load("model.embed_tokens.weight", m.vocab, H, e->embed);
  if (st == LLMK_OK) st = load("model.norm.weight", H, 0, e->final_norm);
  for (int l = 0; l < m.n_layers && st == LLMK_OK; ++l) {
    const std::string p = "model.layers." + std::to_string(l) + ".";
    const LayerPtrs& d = e->layers[l];
    st = load(p + "input_layernorm.weight", H, 0, d.attn_norm);
    if (st == LLMK_OK) st = load(p + "self_attn.q_proj.weight", e->qdim, H, d.wqkv);
    if (st == LLMK_OK)
      st = load(p + "self_attn.k_proj.weight", e->kvdim, H, d.wqkv + (size_t)e->qdim * H);
    if (st == LLMK_OK)
      st = load(p + "self_attn.v_proj.weight", e->kvdim, H,
                d.wqkv + (size_t)(e->qdim + e->kvdim) * H);
    if (st == LLMK_OK) st = load(p + "self_attn.o_proj.weight", H, e->qdim, d.wo);
    if (st == LLMK_OK) st = load(p + "post_attention_layernorm.weight", H, 0, d.mlp_norm);
    if (st == LLMK_OK) st = load(p + "mlp.gate_proj.weight", m.inter, H, d.wgu);
    if (st == LLMK_OK)
      st = load(p + "mlp.up_proj.weight", m.inter, H, d.wgu + (size_t)m.inter * H);
    if (st == LLMK_OK) st = load(p + "mlp.down_proj.weight", H, m.inter, d.wdown);
  }
  if (host) (void)hipHostFree(host);
  close(fd);
  return st;
}

extern "C" int llmk_engine_set_rows(llmk_engine* e, int n_rows, const int32_t* tokens,
                                    const int32_t* positions, const int32_t* block_tables,
                                    int n_logit_rows, const int32_t* logit_rows, void* stream) {
  if (!e || n_rows < 0 || n_rows > e->max_rows) return LLMK_ERR_INVALID_VALUE;
  if (n_rows == 0) return LLMK_OK;
  if (!tokens || !positions || !block_tables) return LLMK_ERR_INVALID_VALUE;
  if (n_logit_rows > n_rows || (n_logit_rows > 0 && !logit_rows)) return LLMK_ERR_INVALID_VALUE;
  // Every index a kernel will follow is checked here, on the host, so that no kernel reads or
  // writes outside its buffers: token ids, positions within the table, the table entries of
  // every page a row's attention reads, and the logit rows.
  const int P = e->max_pages;
  for (int r = 0; r < n_rows; ++r) {
    if (tokens[r] < 0 || tokens[r] >= e->cfg.vocab) return LLMK_ERR_INVALID_VALUE;
    if (positions[r] < 0 || positions[r] >= P * kPage) return LLMK_ERR_INVALID_VALUE;
    for (int j = 0; j <= positions[r] / kPage; ++j) {
      const int32_t pg = block_tables[(size_t)r * P + j];
      if (pg < 0 || pg >= e->num_pages) return LLMK_ERR_INVALID_VALUE;
    }
  }
  for (int i = 0; i < n_logit_rows; ++i)
    if (logit_rows[i] < 0 || logit_rows[i] >= n_rows) return LLMK_ERR_INVALID_VALUE;
  // The previous upload must have left the staging buffer before it is rewritten.
  int st = (int)hipEventSynchronize(e->staged);
  if (st != LLMK_OK) return st;
  Carver c{static_cast<char*>(e->staging)};
  int32_t* h_tokens = c.take<int32_t>(e->max_rows);
  int32_t* h_pos = c.take<int32_t>(e->max_rows);
  int32_t* h_lens = c.take<int32_t>(e->max_rows);
  int32_t* h_logit = c.take<int32_t>(e->max_rows);
  int32_t* h_tables = c.take<int32_t>((size_t)e->max_rows * P);
  memcpy(h_tokens, tokens, n_rows * sizeof(int32_t));
  memcpy(h_pos, positions, n_rows * sizeof(int32_t));
  int span = 0;
  for (int r = 0; r < n_rows; ++r) {
    h_lens[r] = positions[r] + 1;
    span = positions[r] / kPage + 1 > span ? positions[r] / kPage + 1 : span;
  }
  e->rows_span = span;
  if (n_logit_rows > 0) memcpy(h_logit, logit_rows, n_logit_rows * sizeof(int32_t));
  memcpy(h_tables, block_tables, (size_t)n_rows * P * sizeof(int32_t));
  hipStream_t s = static_cast<hipStream_t>(stream);
  st = (int)hipMemcpyAsync(e->in_buf, e->staging, e->in_bytes, hipMemcpyHostToDevice, s);
  if (st == LLMK_OK) st = (int)hipEventRecord(e->staged, s);
  if (st == LLMK_OK) {
    e->rows_set = n_rows;
    e->logit_rows_set = n_logit_rows > 0 ? n_logit_rows : 0;
  }
  return st;
}

// A pass over n rows with n_logit_rows selected rows (< 0: all rows) reads only row inputs the
// last llmk_engine_set_rows uploaded and checked.
static bool rows_uploaded(const llmk_engine* e, int n_rows, int n_logit_rows) {
  return n_rows <= e->rows_set && n_logit_rows <= e->logit_rows_set;
}

// Attention splits of a pass over n rows. num_splits <= 0 asks for the engine's choice:
// - every row's attention spans at most kOneSplitPages pages (short contexts): one split. One
//   block per (row, kv group) then reads all of a row's pages and no merge launch follows; at
//   this size a launch costs more than the parallelism saves. The scheduler workload (contexts
//   of 6-47 tokens but one of 434, max_pages 28) ran 28 one-page splits plus a merge launch
//   (4.7 + 2.9 us per layer at one row); with this rule, same box: 1421 -> 1463-1469 words/s
//   one request at a time, 5934 -> 5984-6016 at up to 8.
// - otherwise the reference's rule (ref: kernels/attention_decode_fast.cuh:22-29) with MI355X's
//   target, taking the table's capacity as the longest sequence.
// The split count changes the fp32 summation order of a row's attention, not its value beyond
// rounding; a graph is cached per resolved count, so replays keep their launch shapes.
constexpr int kOneSplitPages = 4;

static int resolve_splits(const llmk_engine* e, int n, int num_splits, bool capturing = false) {
  if (num_splits <= 0) {
    // A pass captured by the caller is replayed for rows set later: the short-context rule,
    // which follows the rows set now, would bake one split into every replay.
    if (!capturing && e->rows_span <= kOneSplitPages) return 1;
    num_splits = LLMK_ATTN_TARGET_BLOCKS / (n * e->cfg.n_kv_heads);
    if (num_splits > e->max_pages) num_splits = e->max_pages;
    if (num_splits < 1) num_splits = 1;
  }
  return num_splits > kMaxSplits ? kMaxSplits : num_splits;
}

// Whether a pass over n rows takes the fused few-rows path: every projection is a
// llmk_linear_rows_* call with the norms, RoPE + scatter, SwiGLU and residual adds in its
// prologue or epilogue (5 + 1 launches per layer instead of 9 + 1).
// Logit rows from which the fused pass normalises the lm head's input in a launch of its own.
constexpr int kLmSeparateNormRows = 4;

static bool fused_rows_path(const llmk_engine* e, int n) {
  const llmk_model_config& m = e->cfg;
  if (!e->fuse_rows || n > LLMK_LINEAR_ROWS_MAX) return false;
  const int steps = m.hidden / 512;  // the norm prologue: one 512-wide step per wave
  return m.hidden % 512 == 0 && e->qdim % 512 == 0 && m.inter % 512 == 0 && m.head_dim == 64 &&
         (steps & (steps - 1)) == 0 && steps <= 16;
}

static int forward_fused_rows(llmk_engine* e, int n, int nl, bool all_rows, int num_splits,
                              void* s) {
  const llmk_model_config& m = e->cfg;
  const int H = m.hidden, L = m.n_layers;
#define LLMK_TRY(call)               \
  do {                               \
    const int st_ = (call);          \
    if (st_ != LLMK_OK) return st_;  \
  } while (0)
  LLMK_TRY(llmk_embedding_lookup(e->embed, e->tokens, e->x, n, H, s));
  for (int l = 0; l < L; ++l) {
    const LayerPtrs& w = e->layers[l];
    LLMK_TRY(llmk_linear_rows_qkv_rope_scatter(
        e->x, w.attn_norm, m.eps, w.wqkv, e->q, e->k_pool[l], e->v_pool[l], e->tables,
        e->positions, e->inv_freq, n, H, m.n_heads, m.n_kv_heads, e->max_pages, s));
    LLMK_TRY(llmk_attention_decode_fast(e->q, e->k_pool[l], e->v_pool[l], e->tables, e->lens,
                                        e->attn, e->ws, n, e->max_pages, kPage, m.n_heads,
                                        m.n_kv_heads, m.head_dim, num_splits, s));
    LLMK_TRY(llmk_linear_rows_residual(e->attn, w.wo, e->x, n, e->qdim, H, s));
    LLMK_TRY(llmk_linear_rows_swiglu(e->x, w.mlp_norm, m.eps, w.wgu, e->act, n, H, m.inter, s));
    LLMK_TRY(llmk_linear_rows_residual(e->act, w.wdown, e->x, n, m.inter, H, s));
  }
  const uint16_t* lm_in = e->x;
  if (!all_rows) {
    if (nl == 0) return LLMK_OK;
    LLMK_TRY(llmk_embedding_lookup(e->x, e->logit_rows, e->fin, nl, H, s));
    lm_in = e->fin;
  }
  if (nl >= kLmSeparateNormRows) {
    // Each of the lm head's vocab / 8 blocks would normalise all of its rows again; a separate
    // RMSNorm launch costs less from a few rows up (the same bits either way).
    LLMK_TRY(llmk_rmsnorm(lm_in, e->final_norm, e->normed, nl, H, m.eps, s));
    LLMK_TRY(llmk_linear_rows(e->normed, e->embed, e->logits, nl, H, m.vocab, s));
  } else {
    LLMK_TRY(llmk_linear_rows_norm(lm_in, e->final_norm, m.eps, e->embed, e->logits, nl, H,
                                   m.vocab, s));
  }
  if (!e->host_argmax) LLMK_TRY(llmk_argmax_rows(e->logits, e->next, nl, m.vocab, s));
#undef LLMK_TRY
  return LLMK_OK;
}

extern "C" int llmk_engine_set_option(llmk_engine* e, int option, int value) {
  if (!e) return LLMK_ERR_INVALID_VALUE;
  switch (option) {
    case LLMK_ENGINE_FUSE_FEW_ROWS:
      if (e->fuse_rows != (value != 0)) {
        // cached graphs hold the other path
        for (auto& kv : e->graphs)
          if (kv.second.exec) (void)hipGraphExecDestroy(kv.second.exec);
        e->graphs.clear();
      }
      e->fuse_rows = value != 0;
      return LLMK_OK;
    case LLMK_ENGINE_HOST_ARGMAX:
      if (value != 0 && !e->host_logits) {
        const size_t rows = (size_t)e->max_rows * e->cfg.vocab;
        const int st = (int)hipHostMalloc(reinterpret_cast<void**>(&e->host_logits),
                                          rows * sizeof(uint16_t), hipHostMallocDefault);
        if (st != LLMK_OK) {
          e->host_logits = nullptr;
          return st;
        }
        e->host_float.resize(rows);
      }
      e->host_argmax = value != 0;  // the graph cache keys the two kinds of pass apart
      return LLMK_OK;
    default:
      return LLMK_ERR_INVALID_VALUE;
  }
}

extern "C" int llmk_engine_forward(llmk_engine* e, int n_rows, int n_logit_rows, int num_splits,
                                   void* stream) {
  if (!e || n_rows < 0 || n_rows > e->max_rows || n_logit_rows > n_rows)
    return LLMK_ERR_INVALID_VALUE;
  if (n_rows == 0) return LLMK_OK;
  if (!rows_uploaded(e, n_rows, n_logit_rows)) return LLMK_ERR_INVALID_VALUE;
  const llmk_model_config& m = e->cfg;
  const int n = n_rows, H = m.hidden, L = m.n_layers;
  const bool all_rows = n_logit_rows < 0;
  const int nl = all_rows ? n : n_logit_rows;
  bool capturing = false;
  if (num_splits <= 0) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    const int st = (int)hipStreamIsCapturing(static_cast<hipStream_t>(stream), &cap);
    if (st != LLMK_OK) return st;
    capturing = cap != hipStreamCaptureStatusNone;
  }
  num_splits = resolve_splits(e, n, num_splits, capturing);
  void* s = stream;
  if (fused_rows_path(e, n)) return forward_fused_rows(e, n, nl, all_rows, num_splits, s);
#define LLMK_TRY(call)               \
  do {                               \
    const int st_ = (call);          \
    if (st_ != LLMK_OK) return st_;  \
  } while (0)
  LLMK_TRY(llmk_embedding_lookup(e->embed, e->tokens, e->x, n, H, s));
  if (L > 0) LLMK_TRY(llmk_rmsnorm(e->x, e->layers[0].attn_norm, e->normed, n, H, m.eps, s));
  for (int l = 0; l < L; ++l) {
    const LayerPtrs& w = e->layers[l];
    LLMK_TRY(llmk_linear(e->blas, e->normed, w.wqkv, e->qkv, n, H, e->qkvdim, s));
    LLMK_TRY(llmk_qkv_rope_scatter(e->qkv, e->qkvdim, e->q, e->k_pool[l], e->v_pool[l],
                                   e->tables, e->positions, e->inv_freq, n, e->max_pages, kPage,
                                   m.n_heads, m.n_kv_heads, m.head_dim, s));
    LLMK_TRY(llmk_attention_decode_fast(e->q, e->k_pool[l], e->v_pool[l], e->tables, e->lens,
                                        e->attn, e->ws, n, e->max_pages, kPage, m.n_heads,
                                        m.n_kv_heads, m.head_dim, num_splits, s));
    LLMK_TRY(llmk_linear(e->blas, e->attn, w.wo, e->proj, n, e->qdim, H, s));
    LLMK_TRY(llmk_add_rmsnorm(e->x, e->proj, w.mlp_norm, e->normed, n, H, m.eps, s));
    LLMK_TRY(llmk_linear(e->blas, e->normed, w.wgu, e->gu, n, H, 2 * m.inter, s));
    LLMK_TRY(llmk_swiglu_rows(e->gu, e->act, n, m.inter, s));
    LLMK_TRY(llmk_linear(e->blas, e->act, w.wdown, e->proj, n, m.inter, H, s));
    if (l + 1 < L)
      LLMK_TRY(llmk_add_rmsnorm(e->x, e->proj, e->layers[l + 1].attn_norm, e->normed, n, H,
                                m.eps, s));
  }
  const uint16_t* lm_in = e->normed;
  if (all_rows) {
    if (L > 0) LLMK_TRY(llmk_add_rmsnorm(e->x, e->proj, e->final_norm, e->normed, n, H, m.eps, s));
    else LLMK_TRY(llmk_rmsnorm(e->x, e->final_norm, e->normed, n, H, m.eps, s));
  } else if (nl > 0) {
    // Only the selected rows go through the final norm and the lm head: gather them (the
    // embedding gather with the residual as the table), then normalise.
    if (L > 0) LLMK_TRY(llmk_residual_add(e->x, e->proj, e->x, (size_t)n * H, s));
    LLMK_TRY(llmk_embedding_lookup(e->x, e->logit_rows, e->fin, nl, H, s));
    LLMK_TRY(llmk_rmsnorm(e->fin, e->final_norm, e->normed, nl, H, m.eps, s));
  } else {
    if (L > 0) LLMK_TRY(llmk_residual_add(e->x, e->proj, e->x, (size_t)n * H, s));
    return LLMK_OK;
  }
  LLMK_TRY(llmk_linear(e->blas, lm_in, e->embed, e->logits, nl, H, m.vocab, s));
  if (!e->host_argmax) LLMK_TRY(llmk_argmax_rows(e->logits, e->next, nl, m.vocab, s));
#undef LLMK_TRY
  return LLMK_OK;
}

extern "C" void* llmk_engine_buffer(llmk_engine* e, int which, int layer) {
  if (!e) return nullptr;
  switch (which) {
    case LLMK_BUF_LOGITS: return e->logits;
    case LLMK_BUF_NEXT_TOKENS: return e->next;
    case LLMK_BUF_RESIDUAL: return e->x;
    case LLMK_BUF_K_POOL: return layer >= 0 && layer < e->cfg.n_layers ? e->k_pool[layer] : nullptr;
    case LLMK_BUF_V_POOL: return layer >= 0 && layer < e->cfg.n_layers ? e->v_pool[layer] : nullptr;
    case LLMK_BUF_EMBED: return e->embed;
    default: return nullptr;
  }
}

extern "C" int llmk_engine_reset_pools(llmk_engine* e, void* stream) {
  if (!e) return LLMK_ERR_INVALID_VALUE;
  if (!e->pool_buf) return LLMK_OK;
  return (int)hipMemsetAsync(e->pool_buf, 0x7F, 2 * (size_t)e->cfg.n_layers * e->pool_elems * 2,
                             static_cast<hipStream_t>(stream));
}

extern "C" int llmk_engine_forward_graph(llmk_engine* e, int n_rows, int n_logit_rows,
                                         int num_splits, void* stream) {
  if (!e || !stream) return LLMK_ERR_INVALID_VALUE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  int st = (int)hipStreamIsCapturing(s, &cap);
  if (st != LLMK_OK) return st;
  if (cap != hipStreamCaptureStatusNone) return LLMK_ERR_INVALID_VALUE;
  if (n_rows < 0 || n_rows > e->max_rows || n_logit_rows > n_rows) return LLMK_ERR_INVALID_VALUE;
  if (n_rows == 0) return LLMK_OK;
  if (!rows_uploaded(e, n_rows, n_logit_rows)) return LLMK_ERR_INVALID_VALUE;
  num_splits = resolve_splits(e, n_rows, num_splits);  // the key holds the launch shapes
  llmk_engine::Graph& g = e->graphs[std::make_tuple(n_rows, n_logit_rows < 0 ? -1 : n_logit_rows,
                                                    num_splits, e->host_argmax ? 1 : 0)];
  if (g.exec) return (int)hipGraphLaunch(g.exec, s);
  if (!g.seen) {  // first use: eager, which also makes the GEMM plans of these shapes
    g.seen = true;
    return llmk_engine_forward(e, n_rows, n_logit_rows, num_splits, stream);
  }
  st = (int)hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
  if (st != LLMK_OK) return st;
  const int fwd = llmk_engine_forward(e, n_rows, n_logit_rows, num_splits, stream);
  hipGraph_t graph = nullptr;
  st = (int)hipStreamEndCapture(s, &graph);
  if (fwd != LLMK_OK || st != LLMK_OK) {
    if (graph) (void)hipGraphDestroy(graph);
    return fwd != LLMK_OK ? fwd : st;
  }
  st = (int)hipGraphInstantiate(&g.exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  if (st != LLMK_OK) {
    g.exec = nullptr;
    return st;
  }
  return (int)hipGraphLaunch(g.exec, s);
}

// ---------------------------------------------------------------------------------------------
// Scheduler callbacks (llmk_sched_model) backed by the engine.
// ---------------------------------------------------------------------------------------------
namespace {

using Clock = std::chrono::steady_clock;

double ms_since(Clock::time_point t) {
  return std::chrono::duration<double, std::milli>(Clock::now() - t).count();
}

int read_tokens(llmk_engine* e, int32_t* dst, int n) {
  int st = (int)hipMemcpyAsync(dst, e->next, (size_t)n * sizeof(int32_t), hipMemcpyDeviceToHost,
                               e->sched_stream);
  if (st == LLMK_OK) st = (int)hipStreamSynchronize(e->sched_stream);
  return st;
}

// The reference's host argmax (engine/scheduler.cu:9-13): the first index holding the row's
// maximum; comparisons with NaN are false, so a NaN never replaces the running best (and a NaN
// at index 0 is never replaced). The running best value is kept rather than re-read.
int host_argmax_row(const float* lg, int vocab) {
  int best = 0;
  float bv = lg[0];
  for (int v = 1; v < vocab; ++v)
    if (lg[v] > bv) {
      bv = lg[v];
      best = v;
    }
  return best;
}

// fp16 -> fp32, exact and branch-free: the magnitude bits moved into place read as a float
// 2^112 too small for normal numbers and as the float subnormal m * 2^-136 for fp16 subnormals
// (value m * 2^-24); the product with 2^112 is exact in both cases. Inf and NaN keep their
// mantissa under an all-ones exponent. (The reference converts with __half2float on the host,
// engine/batched.cu:135.)
inline float half_to_float(uint16_t h) {
  const uint32_t em = h & 0x7FFFu;
  float f = __builtin_bit_cast(float, em << 13) * 0x1.0p112f;
  if (em >= 0x7C00u) f = __builtin_bit_cast(float, (em << 13) | 0x7F800000u);
  return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, f) | ((uint32_t)(h & 0x8000u) << 16));
}

// Host-argmax mode: copies the n logit rows back (copy_ms), converts them to float
// (convert_ms) and picks each row's token (argmax_ms); ref: engine/batched.cu:126-139,
// engine/scheduler.cu:88-93.
int host_pick(llmk_engine* e, int n, int32_t* out, llmk_step_times* times) {
  const size_t count = (size_t)n * e->cfg.vocab;
  const auto t0 = Clock::now();
  int st = (int)hipMemcpyAsync(e->host_logits, e->logits, count * sizeof(uint16_t),
                               hipMemcpyDeviceToHost, e->sched_stream);
  if (st == LLMK_OK) st = (int)hipStreamSynchronize(e->sched_stream);
  if (st != LLMK_OK) return st;
  const auto t1 = Clock::now();
  for (size_t i = 0; i < count; ++i) e->host_float[i] = half_to_float(e->host_logits[i]);
  const auto t2 = Clock::now();
  for (int r = 0; r < n; ++r)
    out[r] = host_argmax_row(e->host_float.data() + (size_t)r * e->cfg.vocab, e->cfg.vocab);
  if (times) {
    times->copy_ms += std::chrono::duration<double, std::milli>(t1 - t0).count();
    times->convert_ms += std::chrono::duration<double, std::milli>(t2 - t1).count();
    times->argmax_ms += ms_since(t2);
  }
  return LLMK_OK;
}

// A prompt as rows at positions 0 .. len-1, in chunks of at most max_rows rows; only the last
// chunk's last row goes through the lm head (ref: engine/paged.cu:111-127, model_prefill_paged).
int sched_prefill(void* user, const int32_t* table, int max_pages, const int32_t* prompt, int len,
                  int32_t* next_token) {
  llmk_engine* e = static_cast<llmk_engine*>(user);
  if (!table || !prompt || !next_token || len <= 0 || max_pages != e->max_pages)
    return LLMK_ERR_INVALID_VALUE;
  std::vector<int32_t> pos, tab;
  for (int s0 = 0; s0 < len; s0 += e->max_rows) {
    const int n = len - s0 < e->max_rows ? len - s0 : e->max_rows;
    const bool last = s0 + n == len;
    pos.resize(n);
    tab.resize((size_t)n * max_pages);
    for (int r = 0; r < n; ++r) {
      pos[r] = s0 + r;
      memcpy(&tab[(size_t)r * max_pages], table, (size_t)max_pages * sizeof(int32_t));
    }
    const int32_t lr = n - 1;
    int st = llmk_engine_set_rows(e, n, prompt + s0, pos.data(), tab.data(), last ? 1 : 0,
                                  last ? &lr : nullptr, e->sched_stream);
    if (st == LLMK_OK) st = llmk_engine_forward(e, n, last ? 1 : 0, 0, e->sched_stream);
    if (st != LLMK_OK) return st;
  }
  return e->host_argmax ? host_pick(e, 1, next_token, nullptr) : read_tokens(e, next_token, 1);
}

// One decode step with the reference's time split (engine/batched.cu:90-150): prep = the rows'
// host preparation and upload, gpu = events around the pass, then the copy back and, in
// host-argmax mode, the conversion and the search.
int sched_decode(void* user, int n, const int32_t* tokens, const int32_t* positions,
                 const int32_t* tables, int max_pages, int32_t* next_tokens,
                 llmk_step_times* times) {
  llmk_engine* e = static_cast<llmk_engine*>(user);
  if (n <= 0 || n > e->max_rows || max_pages != e->max_pages || !next_tokens)
    return LLMK_ERR_INVALID_VALUE;
  const auto t0 = Clock::now();
  int st = llmk_engine_set_rows(e, n, tokens, positions, tables, 0, nullptr, e->sched_stream);
  if (st != LLMK_OK) return st;
  const double prep = ms_since(t0);
  st = (int)hipEventRecord(e->step_begin, e->sched_stream);
  if (st != LLMK_OK) return st;
  st = e->sched_stream ? llmk_engine_forward_graph(e, n, -1, 0, e->sched_stream)
                       : llmk_engine_forward(e, n, -1, 0, e->sched_stream);
  if (st != LLMK_OK) return st;
  st = (int)hipEventRecord(e->step_end, e->sched_stream);
  if (st == LLMK_OK) st = (int)hipEventSynchronize(e->step_end);
  float gpu = 0.0f;
  if (st == LLMK_OK) st = (int)hipEventElapsedTime(&gpu, e->step_begin, e->step_end);
  if (st != LLMK_OK) return st;
  if (times) {
    times->prep_ms += prep;
    times->gpu_ms += gpu;
  }
  if (e->host_argmax) return host_pick(e, n, next_tokens, times);
  const auto t2 = Clock::now();
  st = read_tokens(e, next_tokens, n);
  if (st == LLMK_OK && times) times->copy_ms += ms_since(t2);
  return st;
}

}  // namespace

extern "C" int llmk_engine_sched_model(llmk_engine* e, void* stream, llmk_sched_model* out) {
  if (!e || !out) return LLMK_ERR_INVALID_VALUE;
  e->sched_stream = static_cast<hipStream_t>(stream);
  out->user = e;
  out->prefill = sched_prefill;
  out->decode = sched_decode;
  return LLMK_OK;
}

extern "C" int llmk_engine_tune(llmk_engine* e, int n_rows, int n_logit_rows, void* stream) {
  if (!e || n_rows <= 0 || n_rows > e->max_rows || n_logit_rows > n_rows)
    return LLMK_ERR_INVALID_VALUE;
  const llmk_model_config& m = e->cfg;
  const int n = n_rows, H = m.hidden, nl = n_logit_rows < 0 ? n : n_logit_rows;
  if (m.n_layers > 0) {
    const LayerPtrs& w = e->layers[0];
    const struct {
      const uint16_t *x, *w;
      uint16_t* y;
      int in, out;
    } shapes[] = {{e->normed, w.wqkv, e->qkv, H, e->qkvdim},
                  {e->attn, w.wo, e->proj, e->qdim, H},
                  {e->normed, w.wgu, e->gu, H, 2 * m.inter},
                  {e->act, w.wdown, e->proj, m.inter, H}};
    for (const auto& g : shapes) {
      const int st = llmk_blas_tune(e->blas, g.x, g.w, g.y, n, g.in, g.out, stream);
      if (st != LLMK_OK) return st;
    }
  }
  if (nl > 0) return llmk_blas_tune(e->blas, e->normed, e->embed, e->logits, nl, H, m.vocab, stream);
  return LLMK_OK;
}
