// The non-GEMM decode pass with one launch per layer (llmk_decode_nongemm_pass_layers).
//
// llmk_decode_nongemm_pass runs each op of a layer as its own launch (49 launches for 16
// layers), the way a decode step with its GEMMs in between must. In the non-GEMM pass by itself
// (config 5) a layer's add + RMSNorm, RoPE + K/V scatter and SwiGLU read independent inputs;
// only the residual carries from one layer's norm to the next. So each layer here is ONE launch
// of one-wave blocks: blocks [0, n) take the add + RMSNorm rows, blocks [n, 2n) the RoPE + K/V
// scatter of one token each, the rest the SwiGLU chunks. The first layer's norm rows read their
// residual input straight from the embedding table (the gather fused into the add), so the
// pass is n_layers launches. With the layer's second add + RMSNorm (x2 set), a norm block runs
// both on its row, the residual kept in registers between them. Every block runs the same body
// as the stand-alone kernel (layer_ops.hpp), so the results are the same bits. Blocks are
// dispatched in index order: the latency-bound norm and RoPE blocks go first, the SwiGLU stream
// fills the rest.
//
// llmk_decode_nongemm_pass_fused goes one step further: one launch for up to kFusedLayers
// layers (config 5's 16 in one). Blocks [0, n) each run one row's residual chain through all of
// the launch's layers -- add + RMSNorm of layer 0, then of layer 1, ... -- with the residual in
// registers and the next layers' x rows and norm weights already in flight (their loads do not
// depend on the residual); then come the RoPE + K/V scatter tokens of every layer and the SwiGLU
// chunks of every layer. The chains are few (one wave per row) and dispatched first, so they run
// beside the streaming blocks instead of in front of them.
#include "layer_ops.hpp"

namespace llmk {
namespace {

struct LayerArgs {
  const f16 *x, *norm_w;
  f16* normed;
  const f16 *x2, *norm_w2;  // the second add + RMSNorm (NORM2)
  f16* normed2;
  f16* q;
  const f16 *k, *v;
  f16 *k_pool, *v_pool;
  const f16 *gate, *up;
  f16* act;
  f16* residual;
  const f16* embed;  // the embedding table (first layer only)
  const int* ids;
  const int *tables, *pos;
  const float* inv_freq;
  FastDiv qdiv, kdiv;
  size_t swiglu_nvec;
  int n, vpr, max_pages, page_size, nh, nkv;
  float hidden_f, eps;
};

constexpr int kWave = 64;

template <int VPL, bool EMBED, int TASKS, bool NORM2>
__global__ void __launch_bounds__(kWave) k_layer_pass(LayerArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int b = blockIdx.x;
  if (b < a.n) {
    const size_t base = (size_t)b * a.vpr * 8;
    const f16* r_in = EMBED ? a.embed + (size_t)a.ids[b] * a.vpr * 8 : a.residual + base;
    if (NORM2)
      rmsnorm_row2<VPL, true>(a.x + base, a.x2 + base, r_in, a.residual + base, a.norm_w,
                              a.norm_w2, a.normed + base, a.normed2 + base, a.vpr, a.hidden_f,
                              a.eps, threadIdx.x);
    else
      rmsnorm_row<VPL, true, true>(a.x + base, r_in, a.residual + base, a.norm_w,
                                   a.normed + base, a.vpr, a.hidden_f, a.eps, threadIdx.x);
  } else if (b < 2 * a.n) {
    rope_tile<4, TASKS, true, false>(b - a.n, kWave, smem, a.q, a.k, a.v, a.k_pool, a.v_pool,
                                     a.tables, a.pos, a.inv_freq, a.n, a.nh, a.nkv, 1,
                                     a.max_pages, a.page_size, a.qdiv, a.kdiv, nullptr, 0);
  } else {
    constexpr size_t chunk = (size_t)kSwigluThreads * kSwigluUnroll;
    static_assert(kSwigluThreads == kWave, "SwiGLU chunks are one-wave blocks");
    const size_t cb = (size_t)(b - 2 * a.n) * chunk;
    if (cb + chunk <= a.swiglu_nvec)
      swiglu_block<kSwigluUnroll>(a.gate, a.up, a.act, cb, a.swiglu_nvec, true);
    else
      swiglu_block<kSwigluUnroll>(a.gate, a.up, a.act, cb, a.swiglu_nvec, false);
  }
}

template <int VPL, bool EMBED, bool NORM2>
int launch_layer(const LayerArgs& a, int tasks, unsigned blocks, size_t lds, hipStream_t s) {
  const dim3 g(blocks), t(kWave);
  switch (tasks) {
    case 6: return launch(k_layer_pass<VPL, EMBED, 6, NORM2>, g, t, lds, s, a);
    case 8: return launch(k_layer_pass<VPL, EMBED, 8, NORM2>, g, t, lds, s, a);
    case 12: return launch(k_layer_pass<VPL, EMBED, 12, NORM2>, g, t, lds, s, a);
    default: return launch(k_layer_pass<VPL, EMBED, 16, NORM2>, g, t, lds, s, a);
  }
}

template <bool EMBED, bool NORM2>
int launch_layer_vpl(const LayerArgs& a, int tasks, unsigned blocks, size_t lds, hipStream_t s) {
  switch (a.vpr / 64) {
    case 1: return launch_layer<1, EMBED, NORM2>(a, tasks, blocks, lds, s);
    case 2: return launch_layer<2, EMBED, NORM2>(a, tasks, blocks, lds, s);
    case 4: return launch_layer<4, EMBED, NORM2>(a, tasks, blocks, lds, s);
    case 8: return launch_layer<8, EMBED, NORM2>(a, tasks, blocks, lds, s);
    default: return launch_layer<16, EMBED, NORM2>(a, tasks, blocks, lds, s);
  }
}

// ---------------------------------------------------------------------------------------------
// One launch for up to kFusedLayers layers.
// ---------------------------------------------------------------------------------------------
constexpr int kFusedLayers = 16;

// Vectors per lane of the one-launch pass's SwiGLU chunks (one-wave blocks). With one norm per
// layer, two halve the launch's blocks: same box, config 5, bits unchanged, 54.3 us with one,
// 53.0 with two, 55.5 with four. With both of the layer's norms (longer residual chains) two
// measured 69.5 us against 59.2 with one. (The stand-alone SwiGLU kernels keep one: there two
// measured slower.)
template <bool NORM2>
constexpr int fused_swiglu_unroll() { return NORM2 ? 1 : 2; }

struct FusedArgs {
  const f16* x[kFusedLayers];
  const f16* norm_w[kFusedLayers];
  f16* normed[kFusedLayers];
  const f16* x2[kFusedLayers];
  const f16* norm_w2[kFusedLayers];
  f16* normed2[kFusedLayers];
  f16* q[kFusedLayers];
  const f16* k[kFusedLayers];
  const f16* v[kFusedLayers];
  f16* k_pool[kFusedLayers];
  f16* v_pool[kFusedLayers];
  const f16* gate[kFusedLayers];
  const f16* up[kFusedLayers];
  f16* act[kFusedLayers];
  f16* residual;
  const f16* embed;  // non-null: the chains start from the embedding rows of ids
  const int* ids;
  const int *tables, *pos;
  const float* inv_freq;
  FastDiv qdiv, kdiv, ndiv, cdiv;  // cdiv: SwiGLU chunks per layer
  size_t swiglu_nvec;
  int n, layers, vpr, max_pages, page_size, nh, nkv;
  float hidden_f, eps;
};

// One row's residual chain through the launch's layers by one wave (ref: engine/batched.cu:
// 64-66, residual_add then rmsnorm, once or twice per layer). Per layer the same arithmetic as
// rmsnorm_row<VPL, true, true> (and rmsnorm_row2 with NORM2) on the residual kept in registers;
// the x rows (and x2) and weights of W layers ahead are loaded while the current layer computes.
// STORE_ALL: the residual row is stored after every layer, as the per-layer passes leave it,
// rather than only after the last (the value left in the buffer is the same).
template <int VPL, int W, bool NORM2, bool STORE_ALL>
__device__ __forceinline__ void norm_chain(const FusedArgs& a, int row, int lane) {
  const size_t base = (size_t)row * a.vpr * 8;
  const f16* r_in = a.embed ? a.embed + (size_t)a.ids[row] * a.vpr * 8 : a.residual + base;
  f16* r_out = a.residual + base;
  f16x8 h[VPL];
#pragma unroll
  for (int k = 0; k < VPL; ++k) h[k] = as_h8(ld16_stream(r_in + 8 * (lane + 64 * k)));
  u32x4 xb[W][VPL], wb[W][VPL], x2b[W][NORM2 ? VPL : 1], w2b[W][NORM2 ? VPL : 1];
  auto fetch = [&](int l, int j) {
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      const size_t v = 8 * (size_t)(lane + 64 * k);
      xb[j][k] = ld16_stream(a.x[l] + base + v);
      wb[j][k] = ld16(a.norm_w[l] + v);
      if constexpr (NORM2) {
        x2b[j][k] = ld16_stream(a.x2[l] + base + v);
        w2b[j][k] = ld16(a.norm_w2[l] + v);
      }
    }
  };
#pragma unroll
  for (int j = 0; j < W; ++j)
    if (j < a.layers) fetch(j, j);
#pragma unroll
  for (int l = 0; l < kFusedLayers; ++l) {
    if (l >= a.layers) break;
    const int j = l % W;
    const bool last = l + 1 == a.layers;
    f16x8 wv[VPL];
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      h[k] = h[k] + as_h8(xb[j][k]);
      wv[k] = as_h8(wb[j][k]);
    }
    if (!NORM2 && (STORE_ALL || last)) {
#pragma unroll
      for (int k = 0; k < VPL; ++k) st16_stream(r_out + 8 * (lane + 64 * k), as_u4(h[k]));
    }
    norm_store<VPL, true>(h, wv, a.normed[l] + base, a.vpr, a.hidden_f, a.eps, lane);
    if constexpr (NORM2) {
#pragma unroll
      for (int k = 0; k < VPL; ++k) {
        h[k] = h[k] + as_h8(x2b[j][k]);
        wv[k] = as_h8(w2b[j][k]);
      }
      if (STORE_ALL || last) {
#pragma unroll
        for (int k = 0; k < VPL; ++k) st16_stream(r_out + 8 * (lane + 64 * k), as_u4(h[k]));
      }
      norm_store<VPL, true>(h, wv, a.normed2[l] + base, a.vpr, a.hidden_f, a.eps, lane);
    }
    if (l + W < a.layers) fetch(l + W, j);
  }
}

// Prefetch depth: W layers of x (and x2) rows and weights in flight, about 8 vectors per lane
// per tensor pair at most.
template <int VPL, bool NORM2>
constexpr int fused_window() {
  constexpr int w = (NORM2 ? 4 : 8) / VPL;
  return w < 1 ? 1 : (w > 4 ? 4 : w);
}

template <int VPL, int TASKS, bool NORM2, bool STORE_ALL>
__global__ void __launch_bounds__(kWave) k_layers_fused(FusedArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int b = blockIdx.x;
  if (b < a.n) {
    norm_chain<VPL, fused_window<VPL, NORM2>(), NORM2, STORE_ALL>(a, b, threadIdx.x);
    return;
  }
  const int r = b - a.n;
  if (r < a.layers * a.n) {
    const int l = (int)fdiv((uint32_t)r, a.ndiv);
    rope_tile<4, TASKS, true, false>(r - l * a.n, kWave, smem, a.q[l], a.k[l], a.v[l],
                                     a.k_pool[l], a.v_pool[l], a.tables, a.pos, a.inv_freq, a.n,
                                     a.nh, a.nkv, 1, a.max_pages, a.page_size, a.qdiv, a.kdiv,
                                     nullptr, 0);
    return;
  }
  constexpr int U = fused_swiglu_unroll<NORM2>();
  constexpr size_t chunk = (size_t)kSwigluThreads * U;
  const int c = r - a.layers * a.n;
  const int l = (int)fdiv((uint32_t)c, a.cdiv);
  const size_t cb = (size_t)(c - l * (int)a.cdiv.d) * chunk;
  if (cb + chunk <= a.swiglu_nvec)
    swiglu_block<U>(a.gate[l], a.up[l], a.act[l], cb, a.swiglu_nvec, true);
  else
    swiglu_block<U>(a.gate[l], a.up[l], a.act[l], cb, a.swiglu_nvec, false);
}

template <bool STORE_ALL>
int launch_fused(const FusedArgs& a, int vpl, int tasks, bool norm2, unsigned blocks,
                 size_t lds, hipStream_t s) {
  const dim3 g(blocks), t(kWave);
#define LLMK_FUSED_TASKS(V, N2)                                                                 \
  switch (tasks) {                                                                              \
    case 6: return launch(k_layers_fused<V, 6, N2, STORE_ALL>, g, t, lds, s, a);               \
    case 8: return launch(k_layers_fused<V, 8, N2, STORE_ALL>, g, t, lds, s, a);               \
    case 12: return launch(k_layers_fused<V, 12, N2, STORE_ALL>, g, t, lds, s, a);             \
    default: return launch(k_layers_fused<V, 16, N2, STORE_ALL>, g, t, lds, s, a);             \
  }
#define LLMK_FUSED_VPL(V)          \
  case V:                          \
    if (norm2) {                   \
      LLMK_FUSED_TASKS(V, true)    \
    } else {                       \
      LLMK_FUSED_TASKS(V, false)   \
    }
  switch (vpl) {
    LLMK_FUSED_VPL(1)
    LLMK_FUSED_VPL(2)
    LLMK_FUSED_VPL(4)
    LLMK_FUSED_VPL(8)
    default:
      return LLMK_ERR_UNSUPPORTED;
  }
#undef LLMK_FUSED_VPL
#undef LLMK_FUSED_TASKS
}

}  // namespace
}  // namespace llmk

using namespace llmk;

// Checks shared by the one-launch passes: the shapes they implement and the operands. Returns
// LLMK_OK and fills *two_norms, *ptasks (the RoPE task count to instantiate) and *vpl, or the
// status to return; *empty is set when there is nothing beyond the embedding to run.
static int check_pass(const llmk_decode_pass* p, bool* two_norms, int* ptasks, int* vpl) {
  if (!p->x || !p->norm_w || !p->normed || !p->q || !p->k || !p->v || !p->k_pool ||
      !p->v_pool || !p->gate || !p->up || !p->act || !p->block_tables || !p->positions ||
      !p->inv_freq)
    return LLMK_ERR_INVALID_VALUE;
  *two_norms = p->x2 || p->norm_w2 || p->normed2;
  if (*two_norms && (!p->x2 || !p->norm_w2 || !p->normed2)) return LLMK_ERR_INVALID_VALUE;
  const int per_tok = (p->n_heads + 2 * p->n_kv_heads) * 8;  // 16-byte vectors per token
  const int tasks = (per_tok + kWave - 1) / kWave;
  *vpl = p->hidden / 512;
  if (p->head_dim != 64 || p->hidden % 512 != 0 || (*vpl & (*vpl - 1)) != 0 || *vpl > 16 ||
      p->inter % 8 != 0 || tasks > 16)
    return LLMK_ERR_UNSUPPORTED;
  *ptasks = tasks <= 6 ? 6 : tasks <= 8 ? 8 : tasks <= 12 ? 12 : 16;
  auto al = [](const void* q) { return aligned16(q); };
  if (!al(p->embed_table) || !al(p->residual)) return LLMK_ERR_ALIGNMENT;
  for (int l = 0; l < p->n_layers; ++l) {
    if (!p->x[l] || !p->norm_w[l] || !p->normed[l] || !p->q[l] || !p->k[l] || !p->v[l] ||
        !p->k_pool[l] || !p->v_pool[l] || !p->gate[l] || !p->up[l] || !p->act[l])
      return LLMK_ERR_INVALID_VALUE;
    if (!al(p->x[l]) || !al(p->norm_w[l]) || !al(p->normed[l]) || !al(p->q[l]) ||
        !al(p->k[l]) || !al(p->v[l]) || !al(p->k_pool[l]) || !al(p->v_pool[l]) ||
        !al(p->gate[l]) || !al(p->up[l]) || !al(p->act[l]))
      return LLMK_ERR_ALIGNMENT;
    if (*two_norms) {
      if (!p->x2[l] || !p->norm_w2[l] || !p->normed2[l]) return LLMK_ERR_INVALID_VALUE;
      if (!al(p->x2[l]) || !al(p->norm_w2[l]) || !al(p->normed2[l])) return LLMK_ERR_ALIGNMENT;
    }
  }
  return LLMK_OK;
}

// The arguments before the layer loop: sizes, returns LLMK_OK or the status to return.
static int check_pass_head(const llmk_decode_pass* p) {
  if (!p) return LLMK_ERR_INVALID_VALUE;
  if (p->n_seqs < 0 || p->n_layers < 0 || p->hidden <= 0 || p->inter <= 0 ||
      p->max_pages <= 0 || p->page_size <= 0 || p->n_heads < 0 || p->n_kv_heads <= 0)
    return LLMK_ERR_INVALID_VALUE;
  if (p->n_seqs == 0) return LLMK_OK;
  if (!p->embed_table || !p->token_ids || !p->residual) return LLMK_ERR_INVALID_VALUE;
  return LLMK_OK;
}

extern "C" int llmk_decode_nongemm_pass_layers(const llmk_decode_pass* p, void* stream) {
  int st = check_pass_head(p);
  if (st != LLMK_OK || p->n_seqs == 0) return st;
  if (p->n_layers == 0)  // the embedding alone
    return llmk_embedding_lookup(p->embed_table, p->token_ids, p->residual, p->n_seqs,
                                 p->hidden, stream);
  bool two_norms;
  int ptasks, vpl;
  st = check_pass(p, &two_norms, &ptasks, &vpl);
  if (st != LLMK_OK) return st;
  const int n = p->n_seqs;
  LayerArgs a;
  a.residual = reinterpret_cast<f16*>(p->residual);
  a.embed = reinterpret_cast<const f16*>(p->embed_table);
  a.ids = p->token_ids;
  a.tables = p->block_tables;
  a.pos = p->positions;
  a.inv_freq = p->inv_freq;
  a.qdiv = make_fastdiv((uint32_t)(p->n_heads > 0 ? p->n_heads * 8 : 1));
  a.kdiv = make_fastdiv((uint32_t)(p->n_kv_heads * 8));
  a.swiglu_nvec = (size_t)n * p->inter / 8;
  a.n = n;
  a.vpr = p->hidden / 8;
  a.max_pages = p->max_pages;
  a.page_size = p->page_size;
  a.nh = p->n_heads;
  a.nkv = p->n_kv_heads;
  a.hidden_f = (float)p->hidden;
  a.eps = p->eps;
  const size_t chunks = (a.swiglu_nvec + kSwigluThreads * kSwigluUnroll - 1) /
                        (kSwigluThreads * kSwigluUnroll);
  if (2 * (size_t)n + chunks > 0x7FFFFFFFu) return LLMK_ERR_UNSUPPORTED;
  const unsigned blocks = (unsigned)(2 * (size_t)n + chunks);
  const size_t lds = 8 + 64 * sizeof(f16);  // one token: its pool row, its (cos, sin) pairs
  hipStream_t s = static_cast<hipStream_t>(stream);
  for (int l = 0; l < p->n_layers; ++l) {
    a.x = reinterpret_cast<const f16*>(p->x[l]);
    a.norm_w = reinterpret_cast<const f16*>(p->norm_w[l]);
    a.normed = reinterpret_cast<f16*>(p->normed[l]);
    a.q = reinterpret_cast<f16*>(p->q[l]);
    a.k = reinterpret_cast<const f16*>(p->k[l]);
    a.v = reinterpret_cast<const f16*>(p->v[l]);
    a.k_pool = reinterpret_cast<f16*>(p->k_pool[l]);
    a.v_pool = reinterpret_cast<f16*>(p->v_pool[l]);
    a.gate = reinterpret_cast<const f16*>(p->gate[l]);
    a.up = reinterpret_cast<const f16*>(p->up[l]);
    a.act = reinterpret_cast<f16*>(p->act[l]);
    a.x2 = two_norms ? reinterpret_cast<const f16*>(p->x2[l]) : nullptr;
    a.norm_w2 = two_norms ? reinterpret_cast<const f16*>(p->norm_w2[l]) : nullptr;
    a.normed2 = two_norms ? reinterpret_cast<f16*>(p->normed2[l]) : nullptr;
    if (two_norms)
      st = l == 0 ? launch_layer_vpl<true, true>(a, ptasks, blocks, lds, s)
                  : launch_layer_vpl<false, true>(a, ptasks, blocks, lds, s);
    else
      st = l == 0 ? launch_layer_vpl<true, false>(a, ptasks, blocks, lds, s)
                  : launch_layer_vpl<false, false>(a, ptasks, blocks, lds, s);
    if (st != LLMK_OK) return st;
  }
  return LLMK_OK;
}

// The launches of the fused pass, STORE_ALL chosen by the caller (the entry point stores the
// residual after every layer).
template <bool STORE_ALL>
static int fused_pass(const llmk_decode_pass* p, void* stream) {
  int st = check_pass_head(p);
  if (st != LLMK_OK || p->n_seqs == 0) return st;
  if (p->n_layers == 0)
    return llmk_embedding_lookup(p->embed_table, p->token_ids, p->residual, p->n_seqs,
                                 p->hidden, stream);
  bool two_norms;
  int ptasks, vpl;
  st = check_pass(p, &two_norms, &ptasks, &vpl);
  if (st != LLMK_OK) return st;
  if (vpl > 8) return LLMK_ERR_UNSUPPORTED;  // hidden 8192: llmk_decode_nongemm_pass_layers
  const int n = p->n_seqs;
  FusedArgs a;
  a.residual = reinterpret_cast<f16*>(p->residual);
  a.ids = p->token_ids;
  a.tables = p->block_tables;
  a.pos = p->positions;
  a.inv_freq = p->inv_freq;
  a.qdiv = make_fastdiv((uint32_t)(p->n_heads > 0 ? p->n_heads * 8 : 1));
  a.kdiv = make_fastdiv((uint32_t)(p->n_kv_heads * 8));
  a.ndiv = make_fastdiv((uint32_t)n);
  a.swiglu_nvec = (size_t)n * p->inter / 8;
  a.n = n;
  a.vpr = p->hidden / 8;
  a.max_pages = p->max_pages;
  a.page_size = p->page_size;
  a.nh = p->n_heads;
  a.nkv = p->n_kv_heads;
  a.hidden_f = (float)p->hidden;
  a.eps = p->eps;
  const size_t chunk = (size_t)kSwigluThreads *
                       (two_norms ? fused_swiglu_unroll<true>() : fused_swiglu_unroll<false>());
  const size_t chunks = (a.swiglu_nvec + chunk - 1) / chunk;
  a.cdiv = make_fastdiv((uint32_t)chunks);
  if ((1 + (size_t)kFusedLayers) * n + kFusedLayers * chunks > 0x7FFFFFFFu)
    return LLMK_ERR_UNSUPPORTED;
  const size_t lds = 8 + 64 * sizeof(f16);  // one token: its pool row, its (cos, sin) pairs
  hipStream_t s = static_cast<hipStream_t>(stream);
  for (int l0 = 0; l0 < p->n_layers; l0 += kFusedLayers) {
    const int cnt = p->n_layers - l0 < kFusedLayers ? p->n_layers - l0 : kFusedLayers;
    a.layers = cnt;
    a.embed = l0 == 0 ? reinterpret_cast<const f16*>(p->embed_table) : nullptr;
    for (int j = 0; j < kFusedLayers; ++j) {
      const int l = l0 + (j < cnt ? j : 0);  // unused slots repeat a valid layer
      a.x[j] = reinterpret_cast<const f16*>(p->x[l]);
      a.norm_w[j] = reinterpret_cast<const f16*>(p->norm_w[l]);
      a.normed[j] = reinterpret_cast<f16*>(p->normed[l]);
      a.x2[j] = two_norms ? reinterpret_cast<const f16*>(p->x2[l]) : nullptr;
      a.norm_w2[j] = two_norms ? reinterpret_cast<const f16*>(p->norm_w2[l]) : nullptr;
      a.normed2[j] = two_norms ? reinterpret_cast<f16*>(p->normed2[l]) : nullptr;
      a.q[j] = reinterpret_cast<f16*>(p->q[l]);
      a.k[j] = reinterpret_cast<const f16*>(p->k[l]);
      a.v[j] = reinterpret_cast<const f16*>(p->v[l]);
      a.k_pool[j] = reinterpret_cast<f16*>(p->k_pool[l]);
      a.v_pool[j] = reinterpret_cast<f16*>(p->v_pool[l]);
      a.gate[j] = reinterpret_cast<const f16*>(p->gate[l]);
      a.up[j] = reinterpret_cast<const f16*>(p->up[l]);
      a.act[j] = reinterpret_cast<f16*>(p->act[l]);
    }
    const unsigned blocks = (unsigned)((1 + (size_t)cnt) * n + cnt * chunks);
    st = launch_fused<STORE_ALL>(a, vpl, ptasks, two_norms, blocks, lds, s);
    if (st != LLMK_OK) return st;
  }
  return LLMK_OK;
}

extern "C" int llmk_decode_nongemm_pass_fused(const llmk_decode_pass* p, void* stream) {
  return fused_pass<true>(p, stream);
}
