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

#include "common.hpp"
#include "pointwise.hpp"

namespace llmk {

// Unsigned division by a launch-constant divisor with a multiply-high (valid for n < 2^31).
struct FastDiv {
  uint32_t d, m, s;
};
static FastDiv make_fastdiv(uint32_t d) {
  uint32_t s = 0;
  while ((1ull << s) < d) ++s;
  const uint64_t m = ((1ull << 32) * ((1ull << s) - d)) / d + 1;
  return FastDiv{d, (uint32_t)m, s};
}
__device__ __forceinline__ uint32_t fdiv(uint32_t n, FastDiv f) {
  return (__umulhi(n, f.m) + n) >> f.s;
}

// The 16 bytes held by lane (lane ^ HV) of the same wave. HV < 16 stays inside a 16-lane DPP
// row: lanes with bit HV clear read lane + HV (row_shl), the others lane - HV (row_shr).
template <int HV>
__device__ __forceinline__ u32x4 partner_vec(u32x4 x, bool upper) {
  u32x4 p;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int v = (int)x[c];
    int r;
    if (HV == 1) {
      r = __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    } else if (HV == 2) {
      r = __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    } else if (HV == 4 || HV == 8) {
      const int hi = __builtin_amdgcn_mov_dpp(v, 0x100 + HV, 0xF, 0xF, false);  // row_shl:HV
      const int lo = __builtin_amdgcn_mov_dpp(v, 0x110 + HV, 0xF, 0xF, false);  // row_shr:HV
      r = upper ? lo : hi;
    } else {
      r = __shfl_xor(v, HV);
    }
    p[c] = (uint32_t)r;
  }
  return p;
}

// HV = 16-byte vectors per half head row (head_dim = 16 * HV); TASKS = vectors per thread.
//
// Layout: a block owns tpb consecutive tokens. Their Q rows form one contiguous run of
// tpb * nh * 2HV vectors, their K rows another of tpb * nkv * 2HV (and, fused, V a third).
// Thread tid takes vectors v = tid + m * blockDim of the concatenated runs, so every wave load
// and store instruction covers 1 KiB of consecutive memory. The two halves of a pair group sit
// in lanes l and l ^ HV (vector j and j + HV of the same head row); each lane fetches its
// partner's 16 bytes with a cross-lane move and writes its own half:
//   first half:  x1' = x1*c - x2*s        second half: x2' = x2*c + x1*s
// All loads are issued before the (cos, sin) phase so their latency overlaps it.
//
// STRIDED (fused variant only): Q, K and V are read from rows of stride `ld` elements -- the
// output of one fused QKV projection, q at column 0, k at nh * head_dim, v after k -- and the
// rotated Q goes to `q`, contiguous [n, nh, head_dim]. The stores are the same as without it.
template <int HV, int TASKS, bool FUSED, bool STRIDED>
__global__ void __launch_bounds__(256)
k_rope_vec(f16* q, const f16* k, const f16* __restrict__ v, f16* k_out, f16* v_pool,
           const int* __restrict__ tables, const int* __restrict__ pos,
           const float* __restrict__ inv_freq, int n_tokens, int nh, int nkv, int tpb,
           int max_pages, int page_size, FastDiv qdiv, FastDiv kdiv, const f16* q_src,
           int ld) {
  static_assert(FUSED || !STRIDED, "strided rows come from the fused QKV projection");
  constexpr int HD = 16 * HV, HALF = 8 * HV;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  long long* pool_row = reinterpret_cast<long long*>(smem);       // [tpb] (FUSED only)
  f16* cs = reinterpret_cast<f16*>(smem + (FUSED ? 8 * tpb : 0));  // [tpb][cos HALF | sin HALF]

  const int t0 = blockIdx.x * tpb;
  const int ntok = min(tpb, n_tokens - t0);
  const int qv = ntok * nh * 2 * HV, kv = ntok * nkv * 2 * HV;
  const int total = qv + (FUSED ? 2 : 1) * kv;
  const size_t kvdim = (size_t)nkv * HD;
  f16* qb = q + (size_t)t0 * nh * HD;
  const f16* kb = k + (size_t)t0 * kvdim;
  const f16* vb = FUSED ? v + (size_t)t0 * kvdim : nullptr;

  u32x4 x[TASKS];
  if constexpr (FUSED) {
    // Fused (decode-sized) launches: the (cos, sin) inputs of the thread's first (token, pair)
    // and the position of its token's pool row are loaded first; then the data loads, all
    // unconditional (a vector past the block's runs loads the last one again and is not
    // stored). Memory waits are in issue order, so the sincos and the page-table lookup
    // proceed while the data is in flight; with conditional data loads in front, each waited
    // for all of them.
    const int cs_n = ntok * HALF;
    const int e0 = (int)threadIdx.x < cs_n ? (int)threadIdx.x : 0;
    const int pos0 = pos[t0 + e0 / HALF];
    const float freq0 = inv_freq[e0 % HALF];
    const int tr = (int)threadIdx.x < ntok ? (int)threadIdx.x : 0;  // the pool row's token
    const int prow = pos[t0 + tr];
#pragma unroll
    for (int m = 0; m < TASKS; ++m) {
      const int e = min((int)threadIdx.x + m * (int)blockDim.x, total - 1);
      if (STRIDED) {
        // vector e of the concatenated runs -> (token, column) of its strided source row
        const bool isq = e < qv;
        const int r = isq ? e : (e < qv + kv ? e - qv : e - qv - kv);
        const FastDiv dv = isq ? qdiv : kdiv;
        const int tt = (int)fdiv((uint32_t)r, dv);
        const int col = r - tt * (int)dv.d;
        const f16* src = isq ? q_src : (e < qv + kv ? k : v);
        x[m] = ld16_stream(src + (size_t)(t0 + tt) * ld + 8 * col);
      } else {
        const f16* src =
            e < qv ? qb + 8 * e : (e < qv + kv ? kb + 8 * (e - qv) : vb + 8 * (e - qv - kv));
        x[m] = ld16_stream(src);
      }
    }
    const int page = tables[(size_t)(t0 + tr) * max_pages + prow / page_size];
    if ((int)threadIdx.x < cs_n) {
      const int tt = threadIdx.x / HALF, i = threadIdx.x % HALF;
      cos_sin_f16((float)pos0 * freq0, cs + tt * HD + i, cs + tt * HD + HALF + i);
    }
    for (int e = threadIdx.x + blockDim.x; e < cs_n; e += blockDim.x) {
      const int tt = e / HALF, i = e % HALF;
      cos_sin_f16((float)pos[t0 + tt] * inv_freq[i], cs + tt * HD + i, cs + tt * HD + HALF + i);
    }
    if ((int)threadIdx.x < ntok) pool_row[tr] = (long long)page * page_size + prow % page_size;
    for (int tt = threadIdx.x + blockDim.x; tt < ntok; tt += blockDim.x) {
      const int b = t0 + tt, p = pos[b];
      const int pg = tables[(size_t)b * max_pages + p / page_size];
      pool_row[tt] = (long long)pg * page_size + p % page_size;
    }
  } else {
    // Standalone launches (many tokens per block, many blocks): the data loads go first, the
    // positions after them. (Issuing the positions first, as above, measured 0.5 us slower at
    // 8192 tokens; at 256 tokens, fused, it is 0.25 us faster.)
#pragma unroll
    for (int m = 0; m < TASKS; ++m) {
      const int e = threadIdx.x + m * blockDim.x;
      if (e < qv) x[m] = ld16_stream(qb + 8 * e);
      else if (e < qv + kv) x[m] = ld16_stream(kb + 8 * (e - qv));
      else x[m] = u32x4{0, 0, 0, 0};
    }
    for (int e = threadIdx.x; e < ntok * HALF; e += blockDim.x) {
      const int tt = e / HALF, i = e % HALF;
      cos_sin_f16((float)pos[t0 + tt] * inv_freq[i], cs + tt * HD + i, cs + tt * HD + HALF + i);
    }
  }
  __syncthreads();

  const bool upper = (threadIdx.x & HV) != 0;  // this lane holds the second half of its group
#pragma unroll
  for (int m = 0; m < TASKS; ++m) {
    const int e = threadIdx.x + m * blockDim.x;
    // Every lane takes part in the exchange, in uniform control flow; pair groups never straddle
    // the Q / K / V boundaries (all multiples of 2HV), so a Q or K lane's partner is valid.
    const u32x4 p = partner_vec<HV>(x[m], upper);
    if (FUSED && e >= qv + kv) {  // value vector: copied unchanged into the V pool row
      if (e < total) {
        const int r = e - qv - kv;
        const int tt = (int)fdiv((uint32_t)r, kdiv);
        st16_stream(v_pool + pool_row[tt] * kvdim + 8 * (r - tt * (int)kdiv.d), x[m]);
      }
    } else if (e < qv + kv) {
      int tt;
      f16* dst;
      if (e < qv) {
        tt = (int)fdiv((uint32_t)e, qdiv);
        dst = qb + 8 * e;
      } else {
        const int r = e - qv;
        tt = (int)fdiv((uint32_t)r, kdiv);
        dst = FUSED ? k_out + pool_row[tt] * kvdim + 8 * (r - tt * (int)kdiv.d)
                    : k_out + (size_t)t0 * kvdim + 8 * r;
      }
      const int j = e & (HV - 1);
      const f16x8 c = *reinterpret_cast<const f16x8*>(cs + tt * HD + 8 * j);
      const f16x8 s = *reinterpret_cast<const f16x8*>(cs + tt * HD + HALF + 8 * j);
      const f16x8 own = as_h8(x[m]), oth = as_h8(p);
      const f16x8 y = upper ? own * c + oth * s : own * c - oth * s;
      st16_stream(dst, as_u4(y));
    }
  }
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

// Tokens per block: about 1024 blocks for long runs, one token per block for short ones.
static int tokens_per_block(int n_tokens) {
  int tpb = 1;
  while (tpb < 16 && n_tokens / (2 * tpb) >= 1024) tpb *= 2;
  return tpb;
}

template <bool FUSED, bool STRIDED = false>
static int rope_vec_launch(f16* q, const f16* k, const f16* v, f16* k_out, f16* v_pool,
                           const int* tables, const int* pos, const float* inv_freq,
                           int n_tokens, int nh, int nkv, int hd, int max_pages, int page_size,
                           hipStream_t stream, const f16* q_src = nullptr, int ld = 0) {
  const int hv = hd / 16;
  const int per_tok = (nh + nkv + (FUSED ? nkv : 0)) * 2 * hv;  // vectors per token
  constexpr int kThreads = 256, kMaxTasks = 16;
  int tpb = tokens_per_block(n_tokens);
  while (tpb > 1 && ceil_div((size_t)tpb * per_tok, kThreads) > (unsigned)kMaxTasks) tpb /= 2;
  const unsigned tasks = ceil_div((size_t)tpb * per_tok, kThreads);
  if (tasks > (unsigned)kMaxTasks) return LLMK_ERR_UNSUPPORTED;
  const FastDiv qdiv = make_fastdiv((uint32_t)(nh > 0 ? nh * 2 * hv : 1));
  const FastDiv kdiv = make_fastdiv((uint32_t)(nkv > 0 ? nkv * 2 * hv : 1));
  const dim3 grid(ceil_div((size_t)n_tokens, (size_t)tpb)), block(kThreads);
  const size_t lds = (FUSED ? 8 * (size_t)tpb : 0) + (size_t)tpb * hd * sizeof(f16);
#define LLMK_ROPE_LAUNCH(H, TK)                                                                  \
  return launch(k_rope_vec<H, TK, FUSED, STRIDED>, grid, block, lds, stream, q, k, v, k_out,   \
                v_pool, tables, pos, inv_freq, n_tokens, nh, nkv, tpb, max_pages, page_size,     \
                qdiv, kdiv, q_src, ld)
#define LLMK_ROPE_CASE(H)                \
  case H:                                \
    if (tasks <= 2) LLMK_ROPE_LAUNCH(H, 2);  \
    if (tasks <= 4) LLMK_ROPE_LAUNCH(H, 4);  \
    if (tasks <= 8) LLMK_ROPE_LAUNCH(H, 8);  \
    if (tasks <= 10) LLMK_ROPE_LAUNCH(H, 10); \
    if (tasks <= 12) LLMK_ROPE_LAUNCH(H, 12); \
    LLMK_ROPE_LAUNCH(H, 16);
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
