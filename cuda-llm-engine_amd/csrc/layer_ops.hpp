// Per-block bodies of the layer kernels -- one RMSNorm row, one RoPE tile of tokens (with the
// paged K/V scatter in the fused variant), one SwiGLU chunk -- shared by their stand-alone
// kernels (norm.hip, rope.hip, swiglu.hip) and by the one-launch-per-layer decode pass
// (layer_pass.hip), so that every path computes the same bits. Semantics and layouts are
// described where the stand-alone kernels are defined.
#pragma once

#include "common.hpp"
#include "pointwise.hpp"

namespace llmk {

// ---------------------------------------------------------------------------------------------
// RMSNorm of one row by one wave (ref: kernels/rmsnorm.cu:9-68). VPL = 16-byte vectors per lane
// per tensor. FUSED: the row is r_in + x, rounded to fp16 and stored to r_out first (the
// residual update; r_in and r_out are the same row except when r_in is an embedding row), and
// the norm is taken of it. FULL: vpr == 64 * VPL, every lane owns exactly VPL vectors.
// ---------------------------------------------------------------------------------------------
// The normalised row of the lane's vectors h (fp16, already rounded) times the weights wv,
// stored to out.
template <int VPL, bool FULL>
__device__ __forceinline__ void norm_store(const f16x8 (&h)[VPL], const f16x8 (&wv)[VPL],
                                           f16* out, int vpr, float hidden_f, float eps,
                                           int lane) {
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < VPL; ++k)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float f = (float)h[k][j];
      ss = ss + f * f;
    }
  ss = wave_sum(ss);
  const float inv = 1.0f / __builtin_sqrtf(ss / hidden_f + eps);
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int v = lane + 64 * k;
    if (FULL || v < vpr) {
      f16x8 a;
#pragma unroll
      for (int j = 0; j < 8; ++j) a[j] = (f16)((float)h[k][j] * inv);
      st16_stream(out + 8 * v, as_u4(wv[k] * a));
    }
  }
}

template <int VPL, bool FUSED, bool FULL>
__device__ __forceinline__ void rmsnorm_row(const f16* x, const f16* r_in, f16* r_out,
                                            const f16* __restrict__ w, f16* out, int vpr,
                                            float hidden_f, float eps, int lane) {
  auto owned = [&](int v) { return FULL || v < vpr; };
  f16x8 h[VPL], wv[VPL];
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int v = lane + 64 * k;
    if (owned(v)) {
      h[k] = as_h8(ld16_stream(x + 8 * v));
      if (FUSED) h[k] = as_h8(ld16_stream(r_in + 8 * v)) + h[k];
      wv[k] = as_h8(ld16(w + 8 * v));
    } else {
      h[k] = (f16x8)(f16)0;
      wv[k] = (f16x8)(f16)0;
    }
  }
  if (FUSED) {
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      const int v = lane + 64 * k;
      if (owned(v)) st16_stream(r_out + 8 * v, as_u4(h[k]));
    }
  }
  norm_store<VPL, FULL>(h, wv, out, vpr, hidden_f, eps, lane);
}

// Both of a layer's add + RMSNorm pairs on one row: h = r_in + x, out = norm(h) * w, then
// h = h + x2, r_out = h, out2 = norm(h) * w2. The same bits as two rmsnorm_row<VPL, true, FULL>
// calls with the residual stored and re-read in between; here it stays in registers.
template <int VPL, bool FULL>
__device__ __forceinline__ void rmsnorm_row2(const f16* x, const f16* x2, const f16* r_in,
                                             f16* r_out, const f16* __restrict__ w,
                                             const f16* __restrict__ w2, f16* out, f16* out2,
                                             int vpr, float hidden_f, float eps, int lane) {
  auto owned = [&](int v) { return FULL || v < vpr; };
  f16x8 h[VPL], wv[VPL], x2v[VPL], wv2[VPL];
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int v = lane + 64 * k;
    if (owned(v)) {
      h[k] = as_h8(ld16_stream(x + 8 * v));
      x2v[k] = as_h8(ld16_stream(x2 + 8 * v));
      h[k] = as_h8(ld16_stream(r_in + 8 * v)) + h[k];
      wv[k] = as_h8(ld16(w + 8 * v));
      wv2[k] = as_h8(ld16(w2 + 8 * v));
    } else {
      h[k] = x2v[k] = wv[k] = wv2[k] = (f16x8)(f16)0;
    }
  }
  norm_store<VPL, FULL>(h, wv, out, vpr, hidden_f, eps, lane);
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    h[k] = h[k] + x2v[k];
    const int v = lane + 64 * k;
    if (owned(v)) st16_stream(r_out + 8 * v, as_u4(h[k]));
  }
  norm_store<VPL, FULL>(h, wv2, out2, vpr, hidden_f, eps, lane);
}

// ---------------------------------------------------------------------------------------------
// RoPE (ref: kernels/rope.cu:27-44) and its fusion with the paged K/V scatter
// (ref: kernels/kv_scatter.cu:17-23).
// ---------------------------------------------------------------------------------------------
// Unsigned division by a launch-constant divisor with a multiply-high (valid for n < 2^31).
struct FastDiv {
  uint32_t d, m, s;
};
static inline FastDiv make_fastdiv(uint32_t d) {
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

// One tile of `tpb` consecutive tokens (tile number `tile`) by one block of `nthr` threads;
// `smem` is the block's dynamic LDS: the tile's (cos, sin) pairs, tpb * head_dim fp16, then
// (FUSED) the tokens' pool rows, 8 * tpb bytes. HV = 16-byte vectors per half head row
// (head_dim = 16 * HV); TASKS = vectors per thread.
//
// Layout: the tile's Q rows form one contiguous run of tpb * nh * 2HV vectors, its K rows
// another of tpb * nkv * 2HV (and, fused, V a third). Thread tid takes vectors v = tid + m * nthr
// of the concatenated runs, so every wave load and store instruction covers 1 KiB of consecutive
// memory. The two halves of a pair group sit in lanes l and l ^ HV (vector j and j + HV of the
// same head row); each lane fetches its partner's 16 bytes with a cross-lane move and writes its
// own half:
//   first half:  x1' = x1*c - x2*s        second half: x2' = x2*c + x1*s
// All loads are issued before the (cos, sin) phase so their latency overlaps it.
//
// STRIDED (fused variant only): Q, K and V are read from rows of stride `ld` elements -- the
// output of one fused QKV projection, q at column 0, k at nh * head_dim, v after k -- and the
// rotated Q goes to `q`, contiguous [n, nh, head_dim]. The stores are the same as without it.
template <int HV, int TASKS, bool FUSED, bool STRIDED>
__device__ __forceinline__ void rope_tile(
    int tile, int nthr, unsigned char* smem, f16* q, const f16* k, const f16* __restrict__ v,
    f16* k_out, f16* v_pool, const int* __restrict__ tables, const int* __restrict__ pos,
    const float* __restrict__ inv_freq, int n_tokens, int nh, int nkv, int tpb, int max_pages,
    int page_size, FastDiv qdiv, FastDiv kdiv, const f16* q_src, int ld) {
  static_assert(FUSED || !STRIDED, "strided rows come from the fused QKV projection");
  constexpr int HD = 16 * HV, HALF = 8 * HV;
  f16* cs = reinterpret_cast<f16*>(smem);  // [tpb][cos HALF | sin HALF], 16-byte rows
  long long* pool_row = reinterpret_cast<long long*>(smem + (size_t)tpb * HD * sizeof(f16));
  const int tid = threadIdx.x;

  const int t0 = tile * tpb;
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
    // unconditional (a vector past the tile's runs loads the last one again and is not
    // stored). Memory waits are in issue order, so the sincos and the page-table lookup
    // proceed while the data is in flight; with conditional data loads in front, each waited
    // for all of them.
    const int cs_n = ntok * HALF;
    const int e0 = tid < cs_n ? tid : 0;
    const int pos0 = pos[t0 + e0 / HALF];
    const float freq0 = inv_freq[e0 % HALF];
    const int tr = tid < ntok ? tid : 0;  // the pool row's token
    const int prow = pos[t0 + tr];
#pragma unroll
    for (int m = 0; m < TASKS; ++m) {
      const int e = min(tid + m * nthr, total - 1);
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
    if (tid < cs_n) {
      const int tt = tid / HALF, i = tid % HALF;
      cos_sin_f16((float)pos0 * freq0, cs + tt * HD + i, cs + tt * HD + HALF + i);
    }
    for (int e = tid + nthr; e < cs_n; e += nthr) {
      const int tt = e / HALF, i = e % HALF;
      cos_sin_f16((float)pos[t0 + tt] * inv_freq[i], cs + tt * HD + i, cs + tt * HD + HALF + i);
    }
    if (tid < ntok) pool_row[tr] = (long long)page * page_size + prow % page_size;
    for (int tt = tid + nthr; tt < ntok; tt += nthr) {
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
      const int e = tid + m * nthr;
      if (e < qv) x[m] = ld16_stream(qb + 8 * e);
      else if (e < qv + kv) x[m] = ld16_stream(kb + 8 * (e - qv));
      else x[m] = u32x4{0, 0, 0, 0};
    }
    for (int e = tid; e < ntok * HALF; e += nthr) {
      const int tt = e / HALF, i = e % HALF;
      cos_sin_f16((float)pos[t0 + tt] * inv_freq[i], cs + tt * HD + i, cs + tt * HD + HALF + i);
    }
  }
  __syncthreads();

  const bool upper = (tid & HV) != 0;  // this lane holds the second half of its group
#pragma unroll
  for (int m = 0; m < TASKS; ++m) {
    const int e = tid + m * nthr;
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

// ---------------------------------------------------------------------------------------------
// SwiGLU (ref: kernels/swiglu.cu:4-21): out = fp16(r16(silu(g)) * u).
// ---------------------------------------------------------------------------------------------
// silu of the NV * 8 fp16 values in g, rounded to fp16, into s. One fast pass over all of them
// records the unsettled ones in a bit mask; a per-lane loop then recomputes just those, so a
// wave runs the exact path as many times as its busiest lane needs it (usually once or never)
// rather than once for every element slot some lane needs it in.
template <int NV>
__device__ __forceinline__ void silu_vectors(const u32x4 (&g)[NV], u32x4 (&s)[NV]) {
  // One bit per element: 4 vectors of 8 at most. A wider shift of the 32-bit mask is undefined,
  // and the compiler then drops the code that follows (8 vectors per lane lost every
  // v_exp_f32 of the kernel, whose waves ran past its end).
  static_assert(NV >= 1 && NV <= 4, "the pending mask holds 32 elements");
  uint32_t pending = 0;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const f16x8 gh = as_h8(g[v]);
    f16x8 sh;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      bool unsettled;
      sh[j] = (f16)silu_fast((float)gh[j], &unsettled);
      pending |= (uint32_t)unsettled << (8 * v + j);
    }
    s[v] = as_u4(sh);
  }
  while (pending) {
    const int idx = __builtin_ctz(pending);
    pending &= pending - 1;
    const int word = idx >> 1, upper = idx & 1;  // 32-bit word (of 4 * NV) and half within it
    uint32_t gw = 0;
#pragma unroll
    for (int k = 0; k < 4 * NV; ++k) gw = word == k ? g[k >> 2][k & 3] : gw;
    const uint16_t gb = (uint16_t)(upper ? gw >> 16 : gw);
    const f16 r = (f16)silu_exact((float)__builtin_bit_cast(f16, gb));
    const uint32_t rb = __builtin_bit_cast(uint16_t, r);
#pragma unroll
    for (int k = 0; k < 4 * NV; ++k) {
      const uint32_t old = s[k >> 2][k & 3];
      const uint32_t upd = upper ? (old & 0xFFFFu) | (rb << 16) : (old & 0xFFFF0000u) | rb;
      s[k >> 2][k & 3] = word == k ? upd : old;
    }
  }
}

// A block owns kSwigluThreads * UNROLL consecutive vectors of each input. One wave per block and
// one vector of each input per lane: waves start, wait and finish on their own, so one wave's
// silu overlaps others' loads. Same box against 256-thread blocks of 2 vectors per lane: 64.8 ->
// 61.3 us at [8192, 8192], 4.58 -> 4.38 us at [256, 8192] (128- and 256-thread blocks of 1
// vector and 4 vectors per lane measured in between). The block size is a constant, not
// blockDim: the kernel arguments arrive preloaded in SGPRs, blockDim would cost a scalar fetch
// before the first address.
constexpr int kSwigluThreads = 64;
constexpr int kSwigluUnroll = 1;

// Vectors [b, b + kSwigluThreads * UNROLL) of gate, up and out; `whole`: all of them < nvec, so
// the straight-line path without per-vector tests issues every load back to back.
template <int UNROLL>
__device__ __forceinline__ void swiglu_block(const f16* __restrict__ gate, const f16* __restrict__ up,
                                             f16* __restrict__ out, size_t b, size_t nvec,
                                             bool whole) {
  u32x4 g[UNROLL], u[UNROLL], sv[UNROLL];
  const u32x4 ones = {0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u};
#pragma unroll
  for (int m = 0; m < UNROLL; ++m) {
    const size_t i = b + threadIdx.x + (size_t)m * kSwigluThreads;
    // Past the end: gate 1.0 (a value the fast path settles); nothing is stored there.
    g[m] = whole || i < nvec ? ld16_stream(gate + 8 * i) : ones;
    u[m] = whole || i < nvec ? ld16_stream(up + 8 * i) : ones;
  }
  silu_vectors<UNROLL>(g, sv);
#pragma unroll
  for (int m = 0; m < UNROLL; ++m) {
    const size_t i = b + threadIdx.x + (size_t)m * kSwigluThreads;
    if (whole || i < nvec) st16_stream(out + 8 * i, as_u4(as_h8(sv[m]) * as_h8(u[m])));
  }
}

}  // namespace llmk
