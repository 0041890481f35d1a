// Host-side parts of libllmk: status strings, the Llama-3 rotation-speed table, and the
// non-GEMM decode-step driver.
#include <hip/hip_runtime.h>
#include <math.h>

#include "llmk.h"

extern "C" const char* llmk_error_string(int status) {
  switch (status) {
    case LLMK_OK: return "success";
    case LLMK_ERR_INVALID_VALUE: return "llmk: invalid value (negative size or NULL pointer)";
    case LLMK_ERR_SHAPE: return "llmk: size is not a multiple the data layout requires";
    case LLMK_ERR_ALIGNMENT: return "llmk: pointer is not 16-byte aligned";
    case LLMK_ERR_UNSUPPORTED: return "llmk: shape outside what the kernels implement";
    case LLMK_ERR_BLAS: return "llmk: hipBLASLt could not run the GEMM";
    case LLMK_ERR_IO: return "llmk: weight file missing, short, or without a required tensor";
    case LLMK_ERR_CAPACITY: return "llmk: a request can never fit in the page pool or block table";
    case LLMK_ERR_SCRATCH:
      return "llmk: the call needs more scratch than the allocation-free entry point holds";
    default: return hipGetErrorString(static_cast<hipError_t>(status));
  }
}

extern "C" int llmk_version(void) { return 100; }  // 0.1.0

// Llama-3 frequency scaling of the RoPE rotation speeds, evaluated in fp32 one step at a time
// so that the table is the same bit for bit as the reference's host routine
// (ref: kernels/rope.cu:4-23, which follows Hugging Face's llama3 rope initialisation):
//   f      = 1 / powf(theta, 2i / head_dim)
//   lambda = (float)(2 pi) / f
//   base   = lambda > orig/low ? f / factor : f
//   smooth = (orig / lambda - low) / (high - low)
//   out    = orig/high <= lambda <= orig/low ? (1 - smooth) * base / factor + smooth * base
//                                            : base
extern "C" int llmk_compute_rope_inv_freq(int head_dim, double theta, double factor,
                                          double low_freq_factor, double high_freq_factor,
                                          double original_max_pos, float* out) {
  if (head_dim <= 0 || head_dim % 2 != 0 || !out) return LLMK_ERR_INVALID_VALUE;
  const float two_pi = (float)(2.0 * M_PI);
  const float th = (float)theta, fac = (float)factor;
  const float lo = (float)low_freq_factor, hi = (float)high_freq_factor;
  const float orig = (float)original_max_pos;
  const float wl_low = (float)(original_max_pos / low_freq_factor);    // long wavelength edge
  const float wl_high = (float)(original_max_pos / high_freq_factor);  // short wavelength edge
  for (int i = 0; i < head_dim / 2; ++i) {
    const float f = 1.0f / powf(th, (float)(2 * i) / (float)head_dim);
    const float wl = two_pi / f;
    const float base = wl > wl_low ? f / fac : f;
    const bool medium = !(wl < wl_high) && !(wl > wl_low);
    if (medium) {
      const float smooth = (orig / wl - lo) / (hi - lo);
      out[i] = (1.0f - smooth) * base / fac + smooth * base;
    } else {
      out[i] = base;
    }
  }
  return LLMK_OK;
}

// One non-GEMM decode pass, launched op by op on one stream (capturable into a HIP graph).
// Mirrors the per-layer order of ref: engine/batched.cu:112-115 with the layer body of
// engine/batched.cu:51-71 reduced to its non-GEMM operations: one add + RMSNorm per layer, or
// both of the layer's (x2 set), the second between the RoPE + K/V scatter and the SwiGLU.
extern "C" int llmk_decode_nongemm_pass(const llmk_decode_pass* p, void* stream) {
  if (!p) return LLMK_ERR_INVALID_VALUE;
  if (p->n_seqs < 0 || p->n_layers < 0 || p->hidden <= 0 || p->inter <= 0)
    return LLMK_ERR_INVALID_VALUE;
  if (p->n_seqs == 0) return LLMK_OK;
  if (p->n_layers > 0 && (!p->x || !p->norm_w || !p->normed || !p->q || !p->k || !p->v ||
                          !p->k_pool || !p->v_pool || !p->gate || !p->up || !p->act))
    return LLMK_ERR_INVALID_VALUE;
  const bool two_norms = p->x2 || p->norm_w2 || p->normed2;
  if (two_norms && p->n_layers > 0 && (!p->x2 || !p->norm_w2 || !p->normed2))
    return LLMK_ERR_INVALID_VALUE;
  const int n = p->n_seqs;
  int st = llmk_embedding_lookup(p->embed_table, p->token_ids, p->residual, n, p->hidden, stream);
  if (st != LLMK_OK) return st;
  for (int l = 0; l < p->n_layers; ++l) {
    st = llmk_add_rmsnorm(p->residual, p->x[l], p->norm_w[l], p->normed[l], n, p->hidden, p->eps,
                          stream);
    if (st != LLMK_OK) return st;
    st = llmk_rope_kv_scatter_batch(p->q[l], p->k[l], p->v[l], p->k_pool[l], p->v_pool[l],
                                    p->block_tables, p->positions, p->inv_freq, n, p->max_pages,
                                    p->page_size, p->n_heads, p->n_kv_heads, p->head_dim, stream);
    if (st != LLMK_OK) return st;
    if (two_norms) {
      st = llmk_add_rmsnorm(p->residual, p->x2[l], p->norm_w2[l], p->normed2[l], n, p->hidden,
                            p->eps, stream);
      if (st != LLMK_OK) return st;
    }
    st = llmk_swiglu(p->gate[l], p->up[l], p->act[l], (size_t)n * p->inter, stream);
    if (st != LLMK_OK) return st;
  }
  return LLMK_OK;
}
