// Rotary position embedding with the Llama-3 rotation speeds, and its fusion with the paged KV
// scatter of the decode step.
//
// Semantics (ref: kernels/rope.cu:27-44): for token t, pair i < head_dim/2 (element i with
// element i + head_dim/2), angle a = float(pos[t]) * inv_freq[i] as one fp32 product,
// c = r16(cos a), s = r16(sin a), x1' = fp16(r16(x1*c) - r16(x2*s)), x2' = fp16(r16(x2*c) +
// r16(x1*s)). Once c and s are fp16 values, every remaining step is an fp16 multiply or add of
// two fp16 values rounded to fp16, which the packed fp16 instructions compute bit for bit.
//
// Work split: a block owns `tpb` consecutive tokens. Their Q rows, K rows (and V rows in the
// fused variant) are contiguous runs of 16-byte vectors, walked so that each wave instruction
// covers 1 KiB of consecutive memory; the two halves of each pair group meet through a
// cross-lane move. The tpb * head_dim/2 (cos, sin) pairs are computed once each and shared
// through LDS as fp16 (the reference evaluates sincosf once per head, 40x as often). Q and K are
// read and written exactly once.
//
// Fused decode variant (replaces ref: engine/batched.cu:55-58): the K task writes its rotated
// vectors to the K pool row of its sequence instead of back to k, and V tasks copy the value
// row to the V pool at the same address (ref: kernels/kv_scatter.cu:17-23).
#include <math.h>

#include "layer_ops.hpp"

namespace llmk {

// HV = 16-byte vectors per half head row (head_dim = 16 * HV); TASKS = vectors per thread;
// NT = threads per block (256, or 512 for the standalone shapes below). One block per tile of
// tpb tokens; the tile body (layer_ops.hpp, rope_tile) describes the layout and the load order.
template <int HV, int TASKS, bool FUSED, bool STRIDED, int NT>
__global__ void __launch_bounds__(NT)
k_rope_vec(f16* q, const f16* k, const f16* __restrict__ v, f16* k_out, f16* v_pool,
           const int* __restrict__ tables, const int* __restrict__ pos,
           const float* __restrict__ inv_freq, int n_tokens, int nh, int nkv, int tpb,
           int max_pages, int page_size, FastDiv qdiv, FastDiv kdiv, const f16* q_src,
           int ld) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  rope_tile<HV, TASKS, FUSED, STRIDED>(blockIdx.x, NT, smem, q, k, v, k_out, v_pool, tables, pos,
                                       inv_freq, n_tokens, nh, nkv, tpb, max_pages, page_size,
                                       qdiv, kdiv, q_src, ld);
}

// Any head_dim (even) and any alignment: one pair per thread per step, same arithmetic.
__global__ void __launch_bounds__(256)
k_rope_scalar(f16* q, f16* k, const int* __restrict__ pos, const float* __restrict__ inv_freq,
              int n_tokens, int nh, int nkv, int hd, int tpb) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  f16* cs = reinterpret_cast<f16*>(smem);  // [tpb][cos half | sin half]
  const int half = hd / 2;
  const int t0 = blockIdx.x * tpb;
  const int ntok = min(tpb, n_tokens - t0);
  for (int e = threadIdx.x; e < ntok * half; e += blockDim.x) {
    const int tt = e / half, i = e % half;
    cos_sin_f16((float)pos[t0 + tt] * inv_freq[i], cs + tt * hd + i, cs + tt * hd + half + i);
  }
  __syncthreads();
  const int per_tok = (nh + nkv) * half;
  for (int e = threadIdx.x; e < ntok * per_tok; e += blockDim.x) {
    const int tt = e / per_tok, r = e % per_tok;
    const int head = r / half, i = r % half;
    const int t = t0 + tt;
    f16* row = head < nh ? q + ((size_t)t * nh + head) * hd
                         : k + ((size_t)t * nkv + (head - nh)) * hd;
    const f16 c = cs[tt * hd + i], s = cs[tt * hd + half + i];
    const f16 x1 = row[i], x2 = row[i + half];
    row[i] = x1 * c - x2 * s;
    row[i + half] = x2 * c + x1 * s;
  }
}

// Tokens per block: about 512 blocks for long runs, one token per block for short ones. At
// 8192 tokens of 32 + 8 heads, 16 tokens per 256-thread block (20 vectors per thread) measured
// 14.76-14.81 us against 15.03-15.11 with 8 (1024 blocks) and 17.1 with 32, same box.
static int tokens_per_block(int n_tokens) {
  int tpb = 1;
  while (tpb < 16 && n_tokens / (2 * tpb) >= 512) tpb *= 2;
  return tpb;
}

// Launch shape of the standalone kernel: threads per block (*nthr) and tokens per tile (*tpb),
// for tokens of per_tok vectors.
//  - At most 512 tiles (a tile of at least 1024 vectors): 512-thread blocks. Two 8-wave blocks
//    per CU then hold the whole grid in one resident round.
//  - From 16384 tokens' worth of 320-vector tokens (Q [T, 32, 64] + K [T, 8, 64]) up: tiles of
//    about 1280 vectors in 512-thread blocks, many rounds of them.
//  - Otherwise 256-thread blocks of tokens_per_block tokens.
// Same box, Q [T, 32, 64] + K [T, 8, 64], every shape bit-identical, best of two rounds (us,
// 256-thread blocks of tokens_per_block tokens -> this shape): T = 4096 7.77 -> 7.45,
// 8192 14.60 -> 14.13, 16384 30.86 -> 28.77, 32768 60.65 -> 54.01, 65536 121.66 -> 104.87;
// at 12288 (768 tiles of 16) 256-thread blocks stay best, 21.4 against 22.7 with 512 threads.
static void standalone_shape(int n_tokens, int per_tok, int* nthr, int* tpb) {
  constexpr long long kManyVectors = 16384LL * 320;
  *nthr = 256;
  *tpb = tokens_per_block(n_tokens);
  if ((long long)n_tokens * per_tok >= kManyVectors) {
    int t = 1;
    while (t < 16 && 2 * t * per_tok <= 1280) t *= 2;
    if (t * per_tok >= 1024) {
      *nthr = 512;
      *tpb = t;
    }
    return;
  }
  if (ceil_div((size_t)n_tokens, (size_t)*tpb) <= 512 && *tpb * per_tok >= 1024) *nthr = 512;
}

template <bool FUSED, bool STRIDED = false>
static int rope_vec_launch(f16* q, const f16* k, const f16* v, f16* k_out, f16* v_pool,
                           const int* tables, const int* pos, const float* inv_freq,
                           int n_tokens, int nh, int nkv, int hd, int max_pages, int page_size,
                           hipStream_t stream, const f16* q_src = nullptr, int ld = 0) {
  const int hv = hd / 16;
  const int per_tok = (nh + nkv + (FUSED ? nkv : 0)) * 2 * hv;  // vectors per token
  constexpr int kMaxTasks = 20;
  int nthr = 256, tpb = tokens_per_block(n_tokens);
  if (!FUSED) standalone_shape(n_tokens, per_tok, &nthr, &tpb);
  while (tpb > 1 && ceil_div((size_t)tpb * per_tok, nthr) > (unsigned)kMaxTasks) tpb /= 2;
  const unsigned tasks = ceil_div((size_t)tpb * per_tok, nthr);
  if (tasks > (unsigned)kMaxTasks) return LLMK_ERR_UNSUPPORTED;
  const FastDiv qdiv = make_fastdiv((uint32_t)(nh > 0 ? nh * 2 * hv : 1));
  const FastDiv kdiv = make_fastdiv((uint32_t)(nkv > 0 ? nkv * 2 * hv : 1));
  const dim3 grid(ceil_div((size_t)n_tokens, (size_t)tpb)), block(nthr);
  const size_t lds = (FUSED ? 8 * (size_t)tpb : 0) + (size_t)tpb * hd * sizeof(f16);
#define LLMK_ROPE_LAUNCH(H, TK, NT)                                                              \
  return launch(k_rope_vec<H, TK, FUSED, STRIDED, NT>, grid, block, lds, stream, q, k, v,      \
                k_out, v_pool, tables, pos, inv_freq, n_tokens, nh, nkv, tpb, max_pages,         \
                page_size, qdiv, kdiv, q_src, ld)
  // 256 threads: 2, 4, 8, 10, 12, 16 or 20 vectors per thread. 512 threads (standalone only):
  // the counts its shapes give exactly (3, 5, 10 for 320-vector tokens), else the next above.
#define LLMK_ROPE_CASE(H)                                \
  case H:                                                \
    if constexpr (!FUSED) {                              \
      if (nthr == 512) {                                 \
        if (tasks <= 2) LLMK_ROPE_LAUNCH(H, 2, 512);     \
        if (tasks <= 3) LLMK_ROPE_LAUNCH(H, 3, 512);     \
        if (tasks <= 5) LLMK_ROPE_LAUNCH(H, 5, 512);     \
        if (tasks <= 10) LLMK_ROPE_LAUNCH(H, 10, 512);   \
        if (tasks <= 16) LLMK_ROPE_LAUNCH(H, 16, 512);   \
        LLMK_ROPE_LAUNCH(H, 20, 512);                    \
      }                                                  \
    }                                                    \
    if (tasks <= 2) LLMK_ROPE_LAUNCH(H, 2, 256);         \
    if (tasks <= 4) LLMK_ROPE_LAUNCH(H, 4, 256);         \
    if (tasks <= 8) LLMK_ROPE_LAUNCH(H, 8, 256);         \
    if (tasks <= 10) LLMK_ROPE_LAUNCH(H, 10, 256);       \
    if (tasks <= 12) LLMK_ROPE_LAUNCH(H, 12, 256);       \
    if (tasks <= 16) LLMK_ROPE_LAUNCH(H, 16, 256);       \
    LLMK_ROPE_LAUNCH(H, 20, 256);
  switch (hv) {
    LLMK_ROPE_CASE(1)
    LLMK_ROPE_CASE(2)
    LLMK_ROPE_CASE(4)
    LLMK_ROPE_CASE(8)
    LLMK_ROPE_CASE(16)
    default:
      return LLMK_ERR_UNSUPPORTED;
  }
#undef LLMK_ROPE_CASE
#undef LLMK_ROPE_LAUNCH
}

}  // namespace llmk

using namespace llmk;

static bool vec_head_dim(int hd) {
  return hd % 16 == 0 && (hd / 16 == 1 || hd / 16 == 2 || hd / 16 == 4 || hd / 16 == 8 ||
                          hd / 16 == 16);
}

extern "C" int llmk_rope_apply(uint16_t* q, uint16_t* k, const int32_t* positions,
                               const float* inv_freq, int n_tokens, int n_heads, int n_kv_heads,
                               int head_dim, void* stream) {
  if (n_tokens < 0 || n_heads < 0 || n_kv_heads < 0 || head_dim <= 0)
    return LLMK_ERR_INVALID_VALUE;
  if (n_tokens == 0 || n_heads + n_kv_heads == 0) return LLMK_OK;
  if (!positions || !inv_freq || (n_heads > 0 && !q) || (n_kv_heads > 0 && !k))
    return LLMK_ERR_INVALID_VALUE;
  if (head_dim % 2 != 0) return LLMK_ERR_SHAPE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  f16* pq = reinterpret_cast<f16*>(q);
  f16* pk = reinterpret_cast<f16*>(k);
  if (vec_head_dim(head_dim) && aligned16(q) && aligned16(k)) {
    const int st = rope_vec_launch<false>(pq, pk, nullptr, pk, nullptr, nullptr, positions,
                                          inv_freq, n_tokens, n_heads, n_kv_heads, head_dim, 0,
                                          1, s);
    if (st != LLMK_ERR_UNSUPPORTED) return st;  // else: a token too wide for one block
  }
  if (head_dim > 4096) return LLMK_ERR_UNSUPPORTED;
  const int tpb = tokens_per_block(n_tokens);
  return launch(k_rope_scalar, dim3(ceil_div((size_t)n_tokens, (size_t)tpb)), dim3(256),
                (size_t)tpb * head_dim * sizeof(f16), s, pq, pk, positions, inv_freq, n_tokens,
                n_heads, n_kv_heads, head_dim, tpb);
}

extern "C" int llmk_rope_kv_scatter_batch(uint16_t* q, const uint16_t* k, const uint16_t* v,
                                          uint16_t* k_pool, uint16_t* v_pool,
                                          const int32_t* block_tables, const int32_t* positions,
                                          const float* inv_freq, int n, int max_pages,
                                          int page_size, int n_heads, int n_kv_heads,
                                          int head_dim, void* stream) {
  if (n < 0 || max_pages <= 0 || page_size <= 0 || n_heads < 0 || n_kv_heads <= 0 ||
      head_dim <= 0)
    return LLMK_ERR_INVALID_VALUE;
  if (n == 0) return LLMK_OK;
  if ((n_heads > 0 && !q) || !k || !v || !k_pool || !v_pool || !block_tables || !positions ||
      !inv_freq)
    return LLMK_ERR_INVALID_VALUE;
  if (!vec_head_dim(head_dim)) return LLMK_ERR_SHAPE;
  if ((n_heads > 0 && !aligned16(q)) || !aligned16(k) || !aligned16(v) || !aligned16(k_pool) ||
      !aligned16(v_pool))
    return LLMK_ERR_ALIGNMENT;
  return rope_vec_launch<true>(
      reinterpret_cast<f16*>(q), reinterpret_cast<const f16*>(k),
      reinterpret_cast<const f16*>(v), reinterpret_cast<f16*>(k_pool),
      reinterpret_cast<f16*>(v_pool), block_tables, positions, inv_freq, n, n_heads, n_kv_heads,
      head_dim, max_pages, page_size, static_cast<hipStream_t>(stream));
}

extern "C" int llmk_qkv_rope_scatter(const uint16_t* qkv, int ld, uint16_t* q_out,
                                     uint16_t* k_pool, uint16_t* v_pool,
                                     const int32_t* block_tables, const int32_t* positions,
                                     const float* inv_freq, int n, int max_pages, int page_size,
                                     int n_heads, int n_kv_heads, int head_dim, void* stream) {
  if (n < 0 || max_pages <= 0 || page_size <= 0 || n_heads <= 0 || n_kv_heads <= 0 ||
      head_dim <= 0)
    return LLMK_ERR_INVALID_VALUE;
  if (n == 0) return LLMK_OK;
  if (!qkv || !q_out || !k_pool || !v_pool || !block_tables || !positions || !inv_freq)
    return LLMK_ERR_INVALID_VALUE;
  if (!vec_head_dim(head_dim)) return LLMK_ERR_SHAPE;
  if ((long long)ld < (long long)(n_heads + 2 * n_kv_heads) * head_dim || ld % 8 != 0)
    return LLMK_ERR_SHAPE;
  if (!aligned16(qkv) || !aligned16(q_out) || !aligned16(k_pool) || !aligned16(v_pool))
    return LLMK_ERR_ALIGNMENT;
  const f16* src = reinterpret_cast<const f16*>(qkv);
  const f16* k = src + (size_t)n_heads * head_dim;
  const f16* v = k + (size_t)n_kv_heads * head_dim;
  return rope_vec_launch<true, true>(
      reinterpret_cast<f16*>(q_out), k, v, reinterpret_cast<f16*>(k_pool),
      reinterpret_cast<f16*>(v_pool), block_tables, positions, inv_freq, n, n_heads, n_kv_heads,
      head_dim, max_pages, page_size, static_cast<hipStream_t>(stream), src, ld);
}
