// Decode attention over the paged KV pool, split over the cached positions (split-KV): one query
// token per sequence against all of its cached K and V rows.
//
// Interface and workspace contract: ref kernels/attention_decode_fast.cuh:5-18 and
// kernels/attention_decode_fast.cu:151-172 (page_size 16, head_dim 64, 4 query heads per kv
// head; the caller's workspace of n_seq * n_heads * num_splits * 66 floats).
// Values: those of the plain paged kernel the reference checks it against
// (kernels/attention_decode_paged.cu:24-62): softmax over positions of q.k / sqrt(64), then the
// weighted sum of the V rows, all in fp32, the result rounded once to fp16. Sums run in a
// different order here, so results agree within the reference test's tolerance
// (tests/test_attention_decode_fast.cu:83-91), not bit for bit.
//
// Layout on gfx950. A pool row holds one position's K (or V) for all n_kv heads: n_kv * 128
// bytes, [kv head][64 dims]. The kv heads are taken in kv groups of KVW = 8, 4, 2 or 1 heads
// (one grid row of blocks per group). A wave reads 1 KiB per instruction, 16 bytes per lane:
// lane (octet o = lane / 8, d8 = lane % 8) holds dims 8*d8 .. 8*d8+7 of one kv head of one
// position. With KVW = 8 the octets are the group's 8 heads of one position; with KVW < 8 they
// cover 8 / KVW consecutive positions (KVW heads each). The 8 lanes of an octet hold one
// (position, kv head): their q.k partial dots meet in three DPP steps, and every lane then owns
// the scores of the 4 query heads that share its kv head.
//
// Each block (4 waves; 2 for the smallest batches in kv groups of 2) takes a run of pages of one
// sequence (sequence-split grid) or of the batch's pages laid end to end (page-balanced grid)
// for one kv group. Waves take chunks of kChunk row reads in turn and keep an online softmax
// per query head (running max m and sum l in log2 units, fp32 accumulators for their 8 dims),
// rescaling once per chunk. The block merges its waves through LDS. A sequence in one piece
// gets its output written directly; otherwise each piece leaves an unnormalised partial
// (A, m, l) in the workspace and a second kernel merges them.
#include <math.h>

#include <mutex>

#include "common.hpp"

namespace llmk {
namespace {

constexpr int kHeadDim = 64;
constexpr int kGroup = 4;  // query heads per kv head
constexpr int kPage = 16;  // positions per page
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kChunk = 4;  // row reads per wave between softmax rescales
// 1/sqrt(64) times log2(e): scores are kept in log2 units so that exp(x - m) is one v_exp_f32.
constexpr float kScoreScale = 0.125f * 1.44269504088896341f;

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// Partial dot product of 8 fp16 dims (4 packed pairs), fp32 accumulation.
__device__ __forceinline__ float dot8(u32x4 a, u32x4 b) {
  float s = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t ak = elem(a, k), bk = elem(b, k);
    s = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, ak), __builtin_bit_cast(h2, bk), s, false);
  }
  return s;
}

// Sum over the 8 lanes of each octet; every lane of the octet gets the total.
__device__ __forceinline__ float octet_sum(float x) {
  x = x + dpp_f32<0xB1>(x);   // quad_perm [1,0,3,2]
  x = x + dpp_f32<0x4E>(x);   // quad_perm [2,3,0,1]
  x = x + dpp_f32<0x141>(x);  // row_half_mirror: lane i <-> 7 - i within each 8 lanes
  return x;
}

// Pages of the sequence that hold cached positions, capped at the block table's width.
__device__ __forceinline__ int seq_pages(int S, int max_pages) {
  const int P = S > 0 ? (S + kPage - 1) / kPage : 0;
  return P < max_pages ? P : max_pages;
}

struct SoftmaxState {
  float m[kGroup], l[kGroup], acc[kGroup][8];
};

// Row reads per chunk: kChunk, fewer when a row read spans many positions, so that a chunk
// never crosses a page (chunks start at multiples of their size within page-aligned ranges).
template <int KVW>
constexpr int chunk_rows() {
  return kChunk * (8 / KVW) <= kPage ? kChunk : kPage / (8 / KVW);
}

// The row reads of one chunk, K and V.
template <int KVW>
struct Chunk {
  static constexpr int ROWS = chunk_rows<KVW>();
  u32x4 k[ROWS], v[ROWS];
};

// Where a block finds the pool page of the sequence's page i: its block-table row, read as each
// chunk needs it ...
struct TablePages {
  const int* __restrict__ row;
  __device__ __forceinline__ int operator()(int i) const { return row[i]; }
};

// ... or, for a run of at most kRunPages pages starting at page `first`, the run's entries read
// once when the block starts, together with the sequence length. They are wave-uniform, so they
// sit in scalar registers (four named members rather than an array, which the compiler would
// place in memory to index it), and the pick is a chain of scalar selects. A chunk's loads then
// wait for nothing but the length.
constexpr int kRunPages = 4;
struct RunPages {
  int first, p0, p1, p2, p3;
  // Entries of pages first .. first + 3, each index clamped to the row's width (the entries past
  // the sequence's last page are read but never used).
  __device__ __forceinline__ RunPages(const int* __restrict__ row, int first_page, int max_pages)
      : first(first_page) {
    const int last = max_pages - 1;
    p0 = entry(row, first_page < last ? first_page : last);
    p1 = entry(row, first_page + 1 < last ? first_page + 1 : last);
    p2 = entry(row, first_page + 2 < last ? first_page + 2 : last);
    p3 = entry(row, first_page + 3 < last ? first_page + 3 : last);
  }
  static __device__ __forceinline__ int entry(const int* __restrict__ row, int i) {
    return row[i];
  }
  // Waits for the entries and `len` together. The compiler would otherwise sink each entry's
  // load to its first use, behind the branch on the length, and the two round trips would
  // follow one another.
  __device__ __forceinline__ void settle(int& len) {
    asm volatile("" : "+s"(p0), "+s"(p1), "+s"(p2), "+s"(p3), "+s"(len));
  }
  __device__ __forceinline__ int operator()(int i) const {
    const int k = i - first;
    const int a = __builtin_amdgcn_readfirstlane(p0), b = __builtin_amdgcn_readfirstlane(p1);
    const int c = __builtin_amdgcn_readfirstlane(p2), d = __builtin_amdgcn_readfirstlane(p3);
    return k == 0 ? a : k == 1 ? b : k == 2 ? c : d;
  }
};

// Element offset of the first row of the chunk that starts at row `row0` of the block's position
// range [pos0, ...): its page from `pages` (wave-uniform, so the pool address of the chunk stays
// in scalar registers and each lane adds only its 32-bit offset).
template <int KVW, class Pages>
__device__ __forceinline__ size_t chunk_base(const Pages& pages, int pos0, int row0,
                                             size_t row_halves) {
  const int cpos = pos0 + row0 * (8 / KVW);  // first position of the chunk
  const int page = pages(cpos / kPage);
  return ((size_t)page * kPage + (size_t)(cpos % kPage)) * row_halves;
}

// Issues the loads of a chunk whose every position is cached (unconditional, so that the loads
// of the next chunk can be in flight while this one is folded). lane_off: the lane's element
// offset inside the first row; row_step: elements from one row read to the next.
template <int KVW, class Pages>
__device__ __forceinline__ void load_chunk(Chunk<KVW>& c, const f16* __restrict__ k_pool,
                                           const f16* __restrict__ v_pool, const Pages& pages,
                                           int pos0, int row0, size_t row_halves,
                                           uint32_t lane_off, uint32_t row_step) {
  const size_t base = chunk_base<KVW>(pages, pos0, row0, row_halves);
  const f16* kb = k_pool + base;
  const f16* vb = v_pool + base;
  // All K rows first: the scores wait only for them, and the softmax runs while V arrives
  // (memory waits are counted in issue order).
#pragma unroll
  for (int r = 0; r < Chunk<KVW>::ROWS; ++r)
    c.k[r] = ld16_stream(kb + lane_off + (uint32_t)r * row_step);
#pragma unroll
  for (int r = 0; r < Chunk<KVW>::ROWS; ++r)
    c.v[r] = ld16_stream(vb + lane_off + (uint32_t)r * row_step);
}

// Folds a loaded chunk into the online softmax. FULL: every position of the chunk is cached;
// otherwise ok[r] says whether the lane's position of row read r is.
template <int KVW, bool FULL>
__device__ __forceinline__ void fold_chunk(SoftmaxState& st, const u32x4 (&qv)[kGroup],
                                           const Chunk<KVW>& c,
                                           const bool (&ok)[Chunk<KVW>::ROWS]) {
  constexpr int ROWS = Chunk<KVW>::ROWS;
  // Raw scores q.k (uncached positions: -inf); the scale is applied inside the exponent.
  float s[ROWS][kGroup];
#pragma unroll
  for (int r = 0; r < ROWS; ++r)
#pragma unroll
    for (int i = 0; i < kGroup; ++i) {
      const float d = octet_sum(dot8(qv[i], c.k[r]));
      s[r][i] = FULL || ok[r] ? d : -INFINITY;
    }
  float corr[kGroup], p[ROWS][kGroup];
  bool grew = false;
#pragma unroll
  for (int i = 0; i < kGroup; ++i) {
    float mx = s[0][i];
#pragma unroll
    for (int r = 1; r < ROWS; ++r) mx = fmaxf(mx, s[r][i]);
    const float mn = fmaxf(st.m[i], mx * kScoreScale);
    const float base = mn == -INFINITY ? 0.0f : mn;  // nothing seen yet: keep everything at 0
    corr[i] = __builtin_amdgcn_exp2f(st.m[i] - base);
    grew = grew || mn != st.m[i];
    float psum = 0.0f;
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      p[r][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r][i], kScoreScale, -base));
      psum = psum + p[r][i];
    }
    st.l[i] = __builtin_fmaf(st.l[i], corr[i], psum);
    st.m[i] = mn;
  }
  // The running max rarely grows once a few chunks are in; when it did not grow anywhere in the
  // wave every correction factor is exactly 2^0 = 1 and the rescale is skipped.
  if (__builtin_amdgcn_ballot_w64(grew)) {
#pragma unroll
    for (int i = 0; i < kGroup; ++i)
#pragma unroll
      for (int d = 0; d < 8; ++d) st.acc[i][d] = st.acc[i][d] * corr[i];
  }
#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
    const f16x8 vh = as_h8(c.v[r]);
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const float v = (float)vh[d];
#pragma unroll
      for (int i = 0; i < kGroup; ++i) st.acc[i][d] = __builtin_fmaf(p[r][i], v, st.acc[i][d]);
    }
  }
}

// The one chunk of a wave that holds uncached positions: rows [row0, row0 + ROWS) of the block's
// range [pos0, pos1), only the cached positions loaded.
template <int KVW, class Pages>
__device__ __forceinline__ void attend_partial_chunk(SoftmaxState& st,
                                                     const u32x4 (&qv)[kGroup],
                                                     const f16* __restrict__ k_pool,
                                                     const f16* __restrict__ v_pool,
                                                     const Pages& pages, int pos0, int pos1,
                                                     int row0, size_t row_halves,
                                                     uint32_t lane_off, uint32_t row_step,
                                                     int slot) {
  constexpr int PPL = 8 / KVW;
  constexpr int ROWS = Chunk<KVW>::ROWS;
  const int cpos = pos0 + row0 * PPL;
  const size_t base = chunk_base<KVW>(pages, pos0, row0, row_halves);
  Chunk<KVW> c;
  bool ok[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
    const uint32_t off = lane_off + (uint32_t)r * row_step;
    ok[r] = cpos + r * PPL + slot < pos1;
    const u32x4 zero = {0u, 0u, 0u, 0u};
    c.k[r] = zero;
    c.v[r] = zero;
    if (ok[r]) {
      c.k[r] = ld16_stream(k_pool + base + off);
      c.v[r] = ld16_stream(v_pool + base + off);
    }
  }
  fold_chunk<KVW, false>(st, qv, c, ok);
}

// Per-block LDS: the softmax states of a block's W waves for the merge at the end of a segment.
template <int KVW, int W = kWaves>
struct MergeLds {
  static constexpr int NP = W * (8 / KVW);    // partial states per query head
  static constexpr int HEADS = KVW * kGroup;  // query heads a block serves (32 for KVW = 8)
  // After the merge thread t holds query head t / 8: the block needs a thread for every dim
  // octet of every head it serves.
  static_assert(HEADS * 8 <= 64 * W, "too few threads for the kv group");
  float acc[NP][HEADS][kHeadDim];
  float m[NP][HEADS], l[NP][HEADS];
};

// The kv head of the lane's octet: kvg * KVW + octet % KVW (kv group kvg holds KVW heads). A
// last group of 8 with fewer heads (n_kv_heads not a multiple of 8: rows of 3, 5, 6, 7, 12, ...
// heads) gives its spare octets the group's last head, so that they read inside the row and the
// query; their results are never stored (every store checks the query head against n_heads).
template <int KVW>
__device__ __forceinline__ int lane_kv_head(int kvg, int n_kv_heads) {
  const int kvh = kvg * KVW + ((threadIdx.x & 63) >> 3) % KVW;
  return KVW == 8 && kvh >= n_kv_heads ? n_kv_heads - 1 : kvh;
}

// The lane's 8 dims of the 4 query heads that share its kv head (lane_kv_head) for sequence
// `seq`.
template <int KVW>
__device__ __forceinline__ void load_query(u32x4 (&qv)[kGroup], const f16* __restrict__ q,
                                           int seq, int kvg, int n_heads) {
  const int lane = threadIdx.x & 63;
  const int kvh = lane_kv_head<KVW>(kvg, n_heads / kGroup);
#pragma unroll
  for (int i = 0; i < kGroup; ++i)
    qv[i] = ld16(q + ((size_t)seq * n_heads + kvh * kGroup + i) * kHeadDim + (lane & 7) * 8);
}

// The block's attention over positions [pos0, pos1) of one sequence (all cached, in the pool
// pages that `pages` names) for the query heads of kv group `kvg`, with the lane's query dims in
// qv (load_query), by a block of W waves. On return thread t with t / 8 < HEADS holds the
// block's combined unnormalised state of query head kvg * HEADS + t / 8, dims 8 * (t % 8) ..
// + 8: A (sum of p * v), M (max score, log2 units) and L (sum of p). Ends with a barrier, so
// the LDS can be reused at once.
// NJ > 0: the wave has at most NJ chunks whose every position is cached; their loads are all
// issued before the first fold (one round trip for a short segment). NJ = 0: any number, streamed
// two at a time.
template <int KVW, int NJ = 0, int W = kWaves, class Pages>
__device__ __forceinline__ void attend_segment(const u32x4 (&qv)[kGroup],
                                               const f16* __restrict__ k_pool,
                                               const f16* __restrict__ v_pool,
                                               const Pages& pages, int pos0, int pos1, int kvg,
                                               int n_kv_heads, MergeLds<KVW, W>& lds,
                                               float (&A)[8], float& M, float& L) {
  constexpr int PPL = 8 / KVW;
  constexpr int NP = MergeLds<KVW, W>::NP, HEADS = MergeLds<KVW, W>::HEADS;
  constexpr int ROWS = chunk_rows<KVW>();
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int octet = lane >> 3, d8 = lane & 7;
  const int slot = octet / KVW, kvl = octet % KVW;
  const size_t row_halves = (size_t)n_kv_heads * kHeadDim;
  // Lane's offset inside a row read: its position's row (for KVW < 8 a row read spans PPL
  // consecutive positions of a page, one per slot), its kv head (lane_kv_head), then 16 bytes
  // per lane of the octet. With KVW == n_kv_heads the row read is one contiguous run; with fewer
  // (a row cut into n_kv_heads / KVW kv groups) it is PPL pieces of KVW * 128 bytes.
  const uint32_t lane_off =
      (uint32_t)(slot * row_halves + lane_kv_head<KVW>(kvg, n_kv_heads) * kHeadDim + d8 * 8);
  const uint32_t row_step = (uint32_t)(PPL * row_halves);

  SoftmaxState st;
#pragma unroll
  for (int i = 0; i < kGroup; ++i) {
    st.m[i] = -INFINITY;
    st.l[i] = 0.0f;
#pragma unroll
    for (int d = 0; d < 8; ++d) st.acc[i][d] = 0.0f;
  }

  const int n_rows = (pos1 - pos0 + PPL - 1) / PPL;
  const int full_rows = (pos1 - pos0) / PPL;  // rows whose every position is cached
  // The wave's chunks whose every position is cached start at rows first + j * STEP, j < nj.
  // They are double-buffered: the loads of chunk j + 1 are issued before chunk j is folded. The
  // steady loop issues its loads unconditionally; a conditional load would make the compiler
  // wait for every outstanding load, the new ones included, before each fold.
  constexpr int STEP = W * ROWS;
  const int first = wave * ROWS;
  const int nj = first + ROWS <= full_rows ? (full_rows - first - ROWS) / STEP + 1 : 0;
  bool all[ROWS];  // unused by the FULL fold
#pragma unroll
  for (int i = 0; i < ROWS; ++i) all[i] = true;
  if constexpr (NJ > 0) {
    if (nj > 0) {
      // Slots past the wave's last chunk load that chunk again (in bounds, and unconditional, so
      // that each fold waits only for its own loads); they are not folded.
      Chunk<KVW> c[NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        load_chunk<KVW>(c[j], k_pool, v_pool, pages, pos0, first + (j < nj ? j : nj - 1) * STEP,
                        row_halves, lane_off, row_step);
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        if (j < nj) fold_chunk<KVW, true>(st, qv, c[j], all);
    }
  } else if (nj > 0) {
    Chunk<KVW> a, b;
    load_chunk<KVW>(a, k_pool, v_pool, pages, pos0, first, row_halves, lane_off,
                    row_step);
    int j = 1, r = first + STEP;
    for (; j + 1 < nj; j += 2, r += 2 * STEP) {
      load_chunk<KVW>(b, k_pool, v_pool, pages, pos0, r, row_halves, lane_off,
                      row_step);
      fold_chunk<KVW, true>(st, qv, a, all);
      load_chunk<KVW>(a, k_pool, v_pool, pages, pos0, r + STEP, row_halves,
                      lane_off, row_step);
      fold_chunk<KVW, true>(st, qv, b, all);
    }
    if (j < nj) {
      load_chunk<KVW>(b, k_pool, v_pool, pages, pos0, r, row_halves, lane_off,
                      row_step);
      fold_chunk<KVW, true>(st, qv, a, all);
      fold_chunk<KVW, true>(st, qv, b, all);
    } else {
      fold_chunk<KVW, true>(st, qv, a, all);
    }
  }
  const int row0 = first + nj * STEP;
  if (row0 < n_rows)  // at most one partly cached chunk per wave
    attend_partial_chunk<KVW>(st, qv, k_pool, v_pool, pages, pos0, pos1, row0, row_halves,
                              lane_off, row_step, slot);

  // Merge the NP partial states of every query head through LDS.
  const int pi = wave * PPL + slot;
#pragma unroll
  for (int i = 0; i < kGroup; ++i) {
    float* dst = &lds.acc[pi][kvl * kGroup + i][d8 * 8];
#pragma unroll
    for (int d = 0; d < 8; ++d) dst[d] = st.acc[i][d];
    if (d8 == 0) {
      lds.m[pi][kvl * kGroup + i] = st.m[i];
      lds.l[pi][kvl * kGroup + i] = st.l[i];
    }
  }
  __syncthreads();
  const int hl = tid >> 3, e8 = tid & 7;
  M = -INFINITY;
  L = 0.0f;
#pragma unroll
  for (int d = 0; d < 8; ++d) A[d] = 0.0f;
  if (hl < HEADS) {
#pragma unroll
    for (int k = 0; k < NP; ++k) M = fmaxf(M, lds.m[k][hl]);
#pragma unroll
    for (int k = 0; k < NP; ++k) {
      const float w = __builtin_amdgcn_exp2f(lds.m[k][hl] - M);  // a state that saw nothing: 0
      L = __builtin_fmaf(lds.l[k][hl], w, L);
      const float* src = &lds.acc[k][hl][e8 * 8];
#pragma unroll
      for (int d = 0; d < 8; ++d) A[d] = __builtin_fmaf(src[d], w, A[d]);
    }
  }
  __syncthreads();
}

__device__ __forceinline__ void store_out(f16* __restrict__ out, int seq, int h, int n_heads,
                                          const float (&A)[8], float L) {
  f16x8 o;
#pragma unroll
  for (int d = 0; d < 8; ++d) o[d] = (f16)(A[d] / L);
  st16(out + ((size_t)seq * n_heads + h) * kHeadDim + (threadIdx.x & 7) * 8, as_u4(o));
}

__device__ __forceinline__ void store_partial(float* __restrict__ part_o,
                                              float2* __restrict__ part_ml, size_t slot_idx,
                                              const float (&A)[8], float M, float L) {
  float* po = part_o + slot_idx * kHeadDim + (threadIdx.x & 7) * 8;
  st16(po, u32x4{__builtin_bit_cast(uint32_t, A[0]), __builtin_bit_cast(uint32_t, A[1]),
                 __builtin_bit_cast(uint32_t, A[2]), __builtin_bit_cast(uint32_t, A[3])});
  st16(po + 4, u32x4{__builtin_bit_cast(uint32_t, A[4]), __builtin_bit_cast(uint32_t, A[5]),
                     __builtin_bit_cast(uint32_t, A[6]), __builtin_bit_cast(uint32_t, A[7])});
  if ((threadIdx.x & 7) == 0) part_ml[slot_idx] = make_float2(M, L);
}

__device__ __forceinline__ void store_nan(f16* __restrict__ out, int seq, int h, int n_heads) {
  const u32x4 nan = {0x7E007E00u, 0x7E007E00u, 0x7E007E00u, 0x7E007E00u};
  st16(out + ((size_t)seq * n_heads + h) * kHeadDim + (threadIdx.x & 7) * 8, nan);
}

// Sequence-split grid (num_splits, kv groups, n_seq): block (split, g, s) takes pages
// [split * pages_per_split, +pages_per_split) of sequence s. Used with one or two splits, and for
// small batches cut into runs of at most kRunPages pages (NJ: as in attend_segment). RUN: the
// runs are that short, and the block reads its query, the sequence length and its run's
// block-table entries all at once, so that its first K/V loads follow one round trip.
// The arguments are ordered so that those the block needs before its first K/V loads fill the
// 16 kernel-argument dwords preloaded into scalar registers; the output pointers, needed last,
// are read from the argument buffer. W: waves per block.
template <int KVW, int NJ, bool RUN, int W>
__global__ void __launch_bounds__(64 * W)
k_attn_split(const int* __restrict__ block_tables, const int* __restrict__ seq_lens,
             int max_pages, int pages_per_split, int n_heads, int n_kv_heads, int num_splits,
             const f16* __restrict__ q, const f16* __restrict__ k_pool,
             const f16* __restrict__ v_pool, f16* __restrict__ out, float* __restrict__ part_o,
             float2* __restrict__ part_ml) {
  __shared__ MergeLds<KVW, W> lds;
  const int split = blockIdx.x, kvg = blockIdx.y, seq = blockIdx.z;
  const int* __restrict__ row = block_tables + (size_t)seq * max_pages;
  const int page0 = split * pages_per_split;
  // RUN: the run's page entries, read ahead of the length (unused, and dropped, otherwise).
  RunPages run(row, RUN ? page0 : 0, RUN ? max_pages : 1);
  int S = seq_lens[seq];
  if constexpr (RUN) run.settle(S);
  const int P = seq_pages(S, max_pages);
  const int h = kvg * MergeLds<KVW, W>::HEADS + (threadIdx.x >> 3);
  const bool writer = (int)(threadIdx.x >> 3) < MergeLds<KVW, W>::HEADS && h < n_heads;
  const int page1 = page0 + pages_per_split < P ? page0 + pages_per_split : P;
  const int pos1 = S < page1 * kPage ? S : page1 * kPage;
  float A[8], M, L;
  u32x4 qv[kGroup];
  if constexpr (RUN) {
    load_query<KVW>(qv, q, seq, kvg, n_heads);
    if (page0 >= P) {
      // No cached position: the quotient 0 / 0 of an all-empty merge, as the reference yields.
      if (split == 0 && writer) store_nan(out, seq, h, n_heads);
      return;
    }
    attend_segment<KVW, NJ, W>(qv, k_pool, v_pool, run, page0 * kPage, pos1, kvg, n_kv_heads,
                               lds, A, M, L);
  } else {
    if (page0 >= P) {
      if (split == 0 && writer) store_nan(out, seq, h, n_heads);
      return;
    }
    load_query<KVW>(qv, q, seq, kvg, n_heads);
    attend_segment<KVW, NJ, W>(qv, k_pool, v_pool, TablePages{row}, page0 * kPage, pos1, kvg,
                               n_kv_heads, lds, A, M, L);
  }
  if (!writer) return;
  if ((P + pages_per_split - 1) / pages_per_split == 1)
    store_out(out, seq, h, n_heads, A, L);
  else
    store_partial(part_o, part_ml, ((size_t)seq * num_splits + split) * n_heads + h, A, M, L);
}

// Sum and maximum of an int over the block (every thread gets both). red: 2 * kWaves ints.
__device__ __forceinline__ void block_sum_max(int v, int* red, int* sum, int* mx) {
  int m = v;
  for (int o = 32; o > 0; o >>= 1) {
    v += __shfl_xor(v, o);
    const int t = __shfl_xor(m, o);
    m = t > m ? t : m;
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    red[wave] = v;
    red[kWaves + wave] = m;
  }
  __syncthreads();
  int a = 0, b = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    a += red[w];
    b = red[kWaves + w] > b ? red[kWaves + w] : b;
  }
  *sum = a;
  *mx = b;
  __syncthreads();
}

// Inclusive prefix sum of an int over the block in thread order; *total gets the block's sum.
__device__ __forceinline__ int block_scan(int v, int* red, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(v, o);
    if (lane >= o) v += t;
  }
  if (lane == 63) red[wave] = v;
  __syncthreads();
  int before = 0, t = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    before += w < wave ? red[w] : 0;
    t += red[w];
  }
  *total = t;
  __syncthreads();
  return v + before;
}

// Sequences whose page counts a thread keeps in registers during the page-balanced prologue;
// longer batches read the lengths a second time.
constexpr int kPrologueTiles = 4;

// The cost of starting a sequence inside a block's run, in pages of KVW kv heads. Switching
// to a new sequence costs a block about 4 us (per-block timestamps, 256 sequences of lengths
// uniform in [1, 2048], 8 kv heads: the first fold of a segment 1.9 us after its start, the
// waves' LDS merge 1.7 us, the stores and the tail chunk 0.7 us), the time it takes to stream
// about 4 pages of 8 kv heads; narrower rows stream their pages faster, so a start weighs
// proportionally more pages. Cutting runs by pages alone left the blocks holding 4 segments
// 12 us behind those holding one; with starts counted, block end times no longer depend on the
// segment count (same box, 256 of U[1, 2048]: 95.2 -> 92.0 us, both kernels; 3 and 5 units
// measured within 0.3 us of 4).
template <int KVW>
constexpr int start_units() { return 32 / KVW; }

// Page-balanced grid (blocks, kv groups). The sequences are laid end to end in sequence order
// as units of work: a sequence with P > 0 pages takes kStartUnits<KVW> units for its start
// followed by one unit per page (U units in all). The units are cut into runs of
// q = max(ceil(U / blocks), q_min) and block b takes run b, whatever sequences it spans: the
// pages of a sequence whose units fall in the run, and none for a start unit. Every block gets
// the same amount of work, starts included, so one resident round of blocks ends together. Each
// (sequence, block) piece is a segment; a sequence whose page 0 sits at unit r_s has segments in
// blocks r_s / q .. (r_s + P_s - 1) / q, and its k-th segment leaves its partial in workspace
// slot k. q_min = ceil((P_max - 1) / (num_splits - 2)) over the batch's largest page count
// P_max keeps that count at most num_splits - 1, so slot num_splits - 1 of every sequence is
// free: the block holding a sequence's first segment records there how many segments it has. A
// sequence with a single segment gets its output written here; the merge kernel finishes the
// others and writes the NaN of empty sequences.
// Argument order as in k_attn_split: what the prologue needs first sits in the preloaded dwords.
template <int KVW>
__global__ void __launch_bounds__(kThreads)
k_attn_balanced(const int* __restrict__ seq_lens, const int* __restrict__ block_tables,
                int n_seq, int max_pages, int n_heads, int n_kv_heads, int num_splits,
                int n_blocks, const f16* __restrict__ q, const f16* __restrict__ k_pool,
                const f16* __restrict__ v_pool, f16* __restrict__ out,
                float* __restrict__ part_o, float2* __restrict__ part_ml) {
  __shared__ MergeLds<KVW> lds;
  __shared__ int red[2 * kWaves];
  __shared__ int found[3];
  const int b = blockIdx.x, kvg = blockIdx.y, tid = threadIdx.x;

  // Page counts: thread t holds sequences t, t + kThreads, ... (the first kPrologueTiles).
  constexpr int C = start_units<KVW>();
  const bool held = n_seq <= kPrologueTiles * kThreads;
  int lv[kPrologueTiles], pv[kPrologueTiles];  // lengths and page counts
  int mine = 0, pmax = 0;  // units of the thread's sequences, their largest page count
#pragma unroll
  for (int t = 0; t < kPrologueTiles; ++t) {
    const int s = t * kThreads + tid;
    lv[t] = s < n_seq ? seq_lens[s] : 0;
    pv[t] = seq_pages(lv[t], max_pages);
    mine += pv[t] > 0 ? C + pv[t] : 0;
    pmax = pv[t] > pmax ? pv[t] : pmax;
  }
  if (!held)
    for (int s = kPrologueTiles * kThreads + tid; s < n_seq; s += kThreads) {
      const int P = seq_pages(seq_lens[s], max_pages);
      mine += P > 0 ? C + P : 0;
      pmax = P > pmax ? P : pmax;
    }
  int U, P_max;
  block_sum_max(mine, red, &U, &P_max);
  const int per = (U + n_blocks - 1) / n_blocks;  // n_blocks == gridDim.x, passed in SGPRs
  const int q_min = P_max > 1 ? (P_max - 1 + num_splits - 3) / (num_splits - 2) : 1;
  const int qp = per > q_min ? per : q_min;
  const long long u0l = (long long)b * qp;
  if (u0l >= U) return;
  const int u0 = (int)u0l;
  const int u1 = u0 + qp < U ? u0 + qp : U;

  // The sequence holding unit u0, its first unit and its length.
  int running = 0;
  const int tiles = (n_seq + kThreads - 1) / kThreads;
  for (int t = 0; t < tiles && running <= u0; ++t) {
    const int s = t * kThreads + tid;
    int S = 0;
    if (held) {
#pragma unroll
      for (int u = 0; u < kPrologueTiles; ++u) S = u == t ? lv[u] : S;
    } else {
      S = s < n_seq ? seq_lens[s] : 0;
    }
    const int P = seq_pages(S, max_pages);
    const int E = P > 0 ? C + P : 0;
    int tile;
    const int incl = running + block_scan(E, red, &tile);
    if (E > 0 && incl - E <= u0 && u0 < incl) {
      found[0] = s;
      found[1] = incl - E;
      found[2] = S;
    }
    running += tile;
  }
  __syncthreads();
  int s = __builtin_amdgcn_readfirstlane(found[0]), us = __builtin_amdgcn_readfirstlane(found[1]);
  int S = __builtin_amdgcn_readfirstlane(found[2]);

  const int h = kvg * MergeLds<KVW>::HEADS + (tid >> 3);
  const bool writer = (tid >> 3) < MergeLds<KVW>::HEADS && h < n_heads;
  while (us < u1) {
    // The next sequence's length, read while this one is attended: a new segment then starts
    // with its query and table reads, one round trip sooner.
    const int S_next = s + 1 < n_seq ? seq_lens[s + 1] : 0;
    const int P = seq_pages(S, max_pages);
    if (P > 0) {
      const int r = us + C;  // the unit of the sequence's page 0
      const int a0 = u0 > r ? u0 : r, a1 = u1 < r + P ? u1 : r + P;
      if (a0 < a1) {  // the run holds some of its pages, not only its start
        const int lp0 = a0 - r, lp1 = a1 - r;
        const int pos1 = S < lp1 * kPage ? S : lp1 * kPage;
        float A[8], M, L;
        u32x4 qv[kGroup];
        load_query<KVW>(qv, q, s, kvg, n_heads);
        attend_segment<KVW>(qv, k_pool, v_pool,
                            TablePages{block_tables + (size_t)s * max_pages}, lp0 * kPage, pos1,
                            kvg, n_kv_heads, lds, A, M, L);
        const int first = r / qp, n_seg = (r + P - 1) / qp - first + 1, k = b - first;
        if (writer) {
          if (n_seg == 1)
            store_out(out, s, h, n_heads, A, L);
          else
            store_partial(part_o, part_ml, ((size_t)s * num_splits + k) * n_heads + h, A, M,
                          L);
        }
        if (k == 0 && tid == 0)
          part_ml[((size_t)s * num_splits + num_splits - 1) * n_heads] =
              make_float2(__builtin_bit_cast(float, n_seg), 0.0f);
      }
      us += C + P;
    }
    S = S_next;
    ++s;
  }
}

// Merge for a few pieces per sequence (the page-balanced grid, one or two splits). Grid
// (ceil(n_heads / 8), n_seq) of one-wave blocks: thread (head, 8 dims). Merges the pieces of
// every sequence that has more than one. (One-wave rather than 256-thread blocks, same box,
// bits unchanged: 32 x 2048 29.2 -> 28.7 us, 32 of U[1, 2048] 25.5 -> 25.1, 64 of U[1, 2048]
// 34.2 -> 33.9, 256 sequences unchanged.) pages_per_split > 0: the sequence-split grid's
// layout, splits = ceil(P / pages_per_split), empty sequences already written. 0: the
// page-balanced layout, the segment count read from the sequence's last slot. The partials are
// folded in four at a time, their loads issued together, with a running maximum.
__global__ void __launch_bounds__(64)
k_attn_merge(const float* __restrict__ part_o, const float2* __restrict__ part_ml,
             const int* __restrict__ seq_lens, f16* __restrict__ out, int max_pages, int n_heads,
             int num_splits, int pages_per_split) {
  constexpr int kBatch = 4;
  const int seq = blockIdx.y;
  const int h = blockIdx.x * 8 + (threadIdx.x >> 3), e8 = threadIdx.x & 7;
  if (h >= n_heads) return;
  const size_t base = (size_t)seq * num_splits * n_heads + h;  // slot of split 0
  // The first batch of slots is loaded together with the length and the segment count; slots
  // beyond the count hold stale data and are masked below (they lie inside the workspace).
  float2 ml[kBatch];
  u32x4 a0[kBatch], a1[kBatch];
  const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int j = 0; j < kBatch; ++j) {
    const size_t k = base + (size_t)j * n_heads;
    const bool in = j < num_splits;
    ml[j] = in ? part_ml[k] : make_float2(-INFINITY, 0.0f);
    a0[j] = in ? ld16(part_o + k * kHeadDim + e8 * 8) : zero;
    a1[j] = in ? ld16(part_o + k * kHeadDim + e8 * 8 + 4) : zero;
  }
  const int S = seq_lens[seq];
  const float2 meta =
      pages_per_split > 0 ? make_float2(0.0f, 0.0f)
                          : part_ml[((size_t)seq * num_splits + num_splits - 1) * n_heads];
  const int P = seq_pages(S, max_pages);
  int used;
  if (pages_per_split > 0) {
    used = (P + pages_per_split - 1) / pages_per_split;
  } else {
    if (P == 0) {
      store_nan(out, seq, h, n_heads);
      return;
    }
    used = __builtin_bit_cast(int, meta.x);
  }
  if (used <= 1) return;
  float M = -INFINITY, L = 0.0f, A[8];
#pragma unroll
  for (int d = 0; d < 8; ++d) A[d] = 0.0f;
  for (int s0 = 0; s0 < used; s0 += kBatch) {
    if (s0 > 0) {
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const size_t k = base + (size_t)(s0 + j) * n_heads;
        const bool in = s0 + j < used;
        ml[j] = in ? part_ml[k] : make_float2(-INFINITY, 0.0f);
        a0[j] = in ? ld16(part_o + k * kHeadDim + e8 * 8) : zero;
        a1[j] = in ? ld16(part_o + k * kHeadDim + e8 * 8 + 4) : zero;
      }
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j)
      if (s0 + j >= used) {  // stale slot (may hold NaN): weight 0 and zero data
        ml[j] = make_float2(-INFINITY, 0.0f);
        a0[j] = zero;
        a1[j] = zero;
      }
    float mx = M;
#pragma unroll
    for (int j = 0; j < kBatch; ++j) mx = fmaxf(mx, ml[j].x);
    const float corr = __builtin_amdgcn_exp2f(M - mx);  // first batch: M = -inf -> 0
    L = L * corr;
#pragma unroll
    for (int d = 0; d < 8; ++d) A[d] = A[d] * corr;
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const float w = __builtin_amdgcn_exp2f(ml[j].x - mx);  // masked slot: exp2(-inf) = 0
      L = __builtin_fmaf(ml[j].y, w, L);
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const uint32_t x0 = elem(a0[j], d), x1 = elem(a1[j], d);
        A[d] = __builtin_fmaf(__builtin_bit_cast(float, x0), w, A[d]);
        A[d + 4] = __builtin_fmaf(__builtin_bit_cast(float, x1), w, A[d + 4]);
      }
    }
    M = mx;
  }
  store_out(out, seq, h, n_heads, A, L);
}

// Merge for many pieces per sequence (the small-batch grid's short runs). Grid (n_heads, n_seq)
// of one-wave blocks: block (h, seq) merges the pieces of query head h of sequence seq, for
// every sequence that has more than one. (One wave per block rather than four per 256-thread
// block puts the few waves of a small batch on more CUs: same box, bits unchanged, 1 x 2048
// 8.23 -> 8.15 us, 2 x 2048 8.73 -> 8.57, 8 x 2048 12.27 -> 12.12, 16 and more sequences
// unchanged.)
// pages_per_split > 0: the sequence-split grid's layout, pieces = ceil(P / pages_per_split),
// empty sequences already written. 0: the page-balanced layout, the piece count read from the
// sequence's last slot. Lane (sg = lane / 16, dq = lane % 16) folds pieces sg, sg + 4, ... for
// dims 4 dq .. 4 dq + 3, 32 pieces per wave per round. The first round is loaded together with
// the length and the piece count, before the count is known (slots past the count lie inside
// the workspace and are masked afterwards), so up to 32 pieces cost one round trip. The four
// piece groups then meet in two exchanges across rows. The running maximum M is shared by the
// whole wave, so every lane's partial sums carry the same scale. (With ~4 pieces per sequence,
// as the page-balanced grid leaves at 256 sequences, this layout was 2 us slower per launch
// than k_attn_merge; with 10-30, as the short runs leave, 8 us faster.)
constexpr int kMergePer = 8;  // pieces per lane per round

__device__ __forceinline__ void store_nan4(f16* __restrict__ out, int seq, int h, int n_heads,
                                           int dq) {
  const uint32_t nan = 0x7E007E00u;
  *reinterpret_cast<uint2*>(out + ((size_t)seq * n_heads + h) * kHeadDim + 4 * dq) =
      make_uint2(nan, nan);
}

__global__ void __launch_bounds__(64)
k_attn_merge_many(const float* __restrict__ part_o, const float2* __restrict__ part_ml,
                  const int* __restrict__ seq_lens, f16* __restrict__ out, int max_pages,
                  int n_heads, int num_splits, int pages_per_split) {
  const int seq = blockIdx.y;
  const int h = blockIdx.x;
  const int lane = threadIdx.x, sg = lane >> 4, dq = lane & 15;
  const size_t base = (size_t)seq * num_splits * n_heads + h;  // slot of piece 0
  float2 ml[kMergePer];
  float4 a[kMergePer];
  // Loads the pieces s0 + sg + 4 j in [from, to) of the round starting at s0.
  auto load_round = [&](int s0, int from, int to) {
#pragma unroll
    for (int j = 0; j < kMergePer; ++j) {
      const int piece = s0 + sg + 4 * j;
      if (piece >= from && piece < to) {
        const size_t k = base + (size_t)piece * n_heads;
        ml[j] = part_ml[k];
        a[j] = *reinterpret_cast<const float4*>(part_o + k * kHeadDim + 4 * dq);
      }
    }
  };
#pragma unroll
  for (int j = 0; j < kMergePer; ++j) {
    ml[j] = make_float2(-INFINITY, 0.0f);  // no piece: weight exp2(-inf) = 0
    a[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
  const int spec_end = 4 * kMergePer < num_splits ? 4 * kMergePer : num_splits;
  load_round(0, 0, spec_end);
  const int S = seq_lens[seq];
  const float2 meta =
      pages_per_split > 0 ? make_float2(0.0f, 0.0f)
                          : part_ml[((size_t)seq * num_splits + num_splits - 1) * n_heads];
  const int P = seq_pages(S, max_pages);
  int used;
  if (pages_per_split > 0) {
    used = (P + pages_per_split - 1) / pages_per_split;
  } else {
    if (P == 0) {
      if (sg == 0) store_nan4(out, seq, h, n_heads, dq);
      return;
    }
    used = __builtin_bit_cast(int, meta.x);
  }
  if (used <= 1) return;
  float M = -INFINITY, L = 0.0f, A[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int s0 = 0; s0 < used; s0 += 4 * kMergePer) {
    if (s0 > 0) {
#pragma unroll
      for (int j = 0; j < kMergePer; ++j) {
        ml[j] = make_float2(-INFINITY, 0.0f);
        a[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
    }
    load_round(s0, s0 > 0 ? s0 : spec_end, used);
#pragma unroll
    for (int j = 0; j < kMergePer; ++j)
      if (s0 + sg + 4 * j >= used) {  // a slot past the count (may hold NaN): weight 0, no data
        ml[j] = make_float2(-INFINITY, 0.0f);
        a[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
    float mx = M;
#pragma unroll
    for (int j = 0; j < kMergePer; ++j) mx = fmaxf(mx, ml[j].x);
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float corr = __builtin_amdgcn_exp2f(M - mx);  // first round: M = -inf -> 0
    L = L * corr;
#pragma unroll
    for (int d = 0; d < 4; ++d) A[d] = A[d] * corr;
#pragma unroll
    for (int j = 0; j < kMergePer; ++j) {
      const float w = __builtin_amdgcn_exp2f(ml[j].x - mx);
      L = __builtin_fmaf(ml[j].y, w, L);
      A[0] = __builtin_fmaf(a[j].x, w, A[0]);
      A[1] = __builtin_fmaf(a[j].y, w, A[1]);
      A[2] = __builtin_fmaf(a[j].z, w, A[2]);
      A[3] = __builtin_fmaf(a[j].w, w, A[3]);
    }
    M = mx;
  }
  L = L + __shfl_xor(L, 16);
  L = L + __shfl_xor(L, 32);
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    A[d] = A[d] + __shfl_xor(A[d], 16);
    A[d] = A[d] + __shfl_xor(A[d], 32);
  }
  if (sg == 0) {
    f16 o[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) o[d] = (f16)(A[d] / L);
    uint2 v;
    v.x = (uint32_t)__builtin_bit_cast(uint16_t, o[0]) |
          ((uint32_t)__builtin_bit_cast(uint16_t, o[1]) << 16);
    v.y = (uint32_t)__builtin_bit_cast(uint16_t, o[2]) |
          ((uint32_t)__builtin_bit_cast(uint16_t, o[3]) << 16);
    *reinterpret_cast<uint2*>(out + ((size_t)seq * n_heads + h) * kHeadDim + 4 * dq) = v;
  }
}

// The page-balanced grid's block count: one 4-wave block per CU (cached per device). Two
// resident blocks per CU, twice the waves, measured slower: the runs are half as long, so
// sequences split into twice the pieces and each block switches segments twice as often
// (same box: 256 of U[1, 2048] 100.1 -> 98.9 us with one block per CU, 64 x 2048
// 50.3 -> 48.5, 256 x 2048 172.6 -> 168.4; one 8-wave block per CU 101.2 / 50.2 / 170.9).
int balanced_blocks() { return device_cus(); }

struct AttnArgs {
  const f16 *q, *k_pool, *v_pool;
  const int *tables, *lens;
  f16* out;
  float* part_o;
  float2* part_ml;
  int n_seq, max_pages, n_heads, n_kv_heads, num_splits;
};

// Batches of at most this many (sequence, kv group) pairs whose splits are at most
// kShortRunPages pages long take the sequence-split grid: there is no length scan, and a block's
// few chunks are in flight together. Larger batches, or longer runs, take the page-balanced
// grid, which follows the actual lengths. Measured at 8 sequences of lengths uniform in
// [1, 2048], both kernels together: 12.1 us with 4-page runs against 16.1 us page-balanced.
constexpr int kSplitGridPairs = 16;
constexpr int kShortRunPages = kRunPages;

// attend_segment's NJ for runs of pps pages: all of a wave's chunks in flight at once when it
// has at most two, else 0 (streamed two at a time: with all four in flight, 188 VGPRs, 16 x 2048
// measured 18.1 -> 19.1 us and 1 x 2048 10.4 -> 11.1 us).
template <int KVW, int W = kWaves>
int short_run_chunks(int pps) {
  constexpr int PPL = 8 / KVW, ROWS = chunk_rows<KVW>();
  const int rows = pps * kPage / PPL;
  const int per_wave = ((rows + ROWS - 1) / ROWS + W - 1) / W;
  return per_wave <= 1 ? 1 : per_wave <= 2 ? 2 : 0;
}

template <int KVW, int NJ, bool RUN, int W = kWaves>
int split_launch(const AttnArgs& a, int groups, int pps, hipStream_t s) {
  const dim3 grid((unsigned)a.num_splits, (unsigned)groups, (unsigned)a.n_seq);
  return launch(k_attn_split<KVW, NJ, RUN, W>, grid, dim3(64 * W), 0, s, a.tables, a.lens,
                a.max_pages, pps, a.n_heads, a.n_kv_heads, a.num_splits, a.q, a.k_pool, a.v_pool,
                a.out, a.part_o, a.part_ml);
}

// The short-run grid with W waves per block.
template <int KVW, int W>
int short_run_launch(const AttnArgs& a, int groups, int pps, hipStream_t s) {
  switch (short_run_chunks<KVW, W>(pps)) {
    case 1: return split_launch<KVW, 1, true, W>(a, groups, pps, s);
    case 2: return split_launch<KVW, 2, true, W>(a, groups, pps, s);
    default: return split_launch<KVW, 0, true, W>(a, groups, pps, s);
  }
}

// Batches of at most this many (sequence, kv group) pairs in kv groups of 2 heads (one or two
// sequences of 8 kv heads) run the short-run grid in 2-wave blocks: the block's chunks in half
// as many waves, and half as many wave states to merge through LDS. Same box, 8 kv heads, 2048
// positions, 32 splits: 1 sequence 8.14 -> 7.72 us, 2 sequences 8.50 -> 7.99. At 4 sequences
// (groups of 4) 2-wave blocks were no faster (9.54 -> 9.63), and slower from 8 on; 1-wave
// blocks lose (8.84 us at 1 sequence).
constexpr int kTwoWavePairs = 8;

template <int KVW>
int attn_launch(const AttnArgs& a, hipStream_t s) {
  const int groups = KVW == 8 ? (a.n_kv_heads + 7) / 8 : a.n_kv_heads / KVW;
  const int pps = (a.max_pages + a.num_splits - 1) / a.num_splits;  // pages per split
  const bool short_runs = a.part_o && a.num_splits >= 3 && pps <= kShortRunPages &&
                          (long long)a.n_seq * groups <= kSplitGridPairs;
  // The page-balanced kernel counts the batch's units in 32-bit ints: at most
  // n_seq * (start_units + max_pages) of them. Batches that could exceed that take the
  // sequence-split grid, which needs no count.
  const bool units_fit =
      (long long)a.n_seq * (start_units<KVW>() + (long long)a.max_pages) <= 0x7FFFFFFFLL;
  if (a.num_splits >= 3 && a.part_o && !short_runs && units_fit) {
    int blocks = balanced_blocks() / groups;
    if (blocks < 1) blocks = 1;
    int st = launch(k_attn_balanced<KVW>, dim3((unsigned)blocks, (unsigned)groups), dim3(kThreads),
                    0, s, a.lens, a.tables, a.n_seq, a.max_pages, a.n_heads, a.n_kv_heads,
                    a.num_splits, blocks, a.q, a.k_pool, a.v_pool, a.out, a.part_o, a.part_ml);
    if (st != 0) return st;
    const dim3 mgrid((unsigned)((a.n_heads + 7) / 8), (unsigned)a.n_seq);
    return launch(k_attn_merge, mgrid, dim3(64), 0, s, a.part_o, a.part_ml, a.lens, a.out,
                  a.max_pages, a.n_heads, a.num_splits, 0);
  }
  int st;
  if (short_runs) {
    if constexpr (KVW == 2) {
      st = (long long)a.n_seq * groups <= kTwoWavePairs
               ? short_run_launch<KVW, 2>(a, groups, pps, s)
               : short_run_launch<KVW, kWaves>(a, groups, pps, s);
    } else {
      st = short_run_launch<KVW, kWaves>(a, groups, pps, s);
    }
  } else {
    st = split_launch<KVW, 0, false>(a, groups, pps, s);
  }
  if (st != 0 || pps >= a.max_pages) return st;  // every sequence fits in one split
  if (short_runs) {
    const dim3 mgrid((unsigned)a.n_heads, (unsigned)a.n_seq);
    return launch(k_attn_merge_many, mgrid, dim3(64), 0, s, a.part_o, a.part_ml, a.lens, a.out,
                  a.max_pages, a.n_heads, a.num_splits, pps);
  }
  const dim3 mgrid((unsigned)((a.n_heads + 7) / 8), (unsigned)a.n_seq);
  return launch(k_attn_merge, mgrid, dim3(64), 0, s, a.part_o, a.part_ml, a.lens, a.out,
                a.max_pages, a.n_heads, a.num_splits, pps);
}

}  // namespace
}  // namespace llmk

using namespace llmk;

extern "C" size_t llmk_attention_decode_fast_workspace_floats(int n_seq, int n_heads,
                                                             int num_splits) {
  if (n_seq <= 0 || n_heads <= 0 || num_splits <= 0) return 0;
  // Below 2^100 for any int arguments; SIZE_MAX when it does not fit a size_t, so that no
  // product wraps to a size some buffer could hold.
  const unsigned __int128 f =
      (unsigned __int128)n_seq * (unsigned)n_heads * (unsigned)num_splits * (kHeadDim + 2);
  return f > (unsigned __int128)SIZE_MAX ? SIZE_MAX : (size_t)f;
}

// Argument checks shared by both entry points; -1 means "go ahead".
static int check_attention(const uint16_t* q, const uint16_t* k_pool, const uint16_t* v_pool,
                           const int32_t* block_tables, const int32_t* seq_lens,
                           const uint16_t* out, int n_seq, int max_pages, int page_size,
                           int n_heads, int n_kv_heads, int head_dim, int num_splits) {
  if (n_seq == 0) return LLMK_OK;
  // The reference's preconditions (kernels/attention_decode_fast.cu:160-163).
  if (page_size != kPage || head_dim != kHeadDim || n_kv_heads <= 0 ||
      n_heads != kGroup * n_kv_heads)
    return LLMK_ERR_SHAPE;
  if (n_seq < 0 || max_pages <= 0 || num_splits <= 0) return LLMK_ERR_INVALID_VALUE;
  if (n_seq > 65535 || (n_kv_heads + 7) / 8 > 65535) return LLMK_ERR_UNSUPPORTED;
  if (!q || !k_pool || !v_pool || !block_tables || !seq_lens || !out)
    return LLMK_ERR_INVALID_VALUE;
  if (!aligned16(q) || !aligned16(k_pool) || !aligned16(v_pool) || !aligned16(out))
    return LLMK_ERR_ALIGNMENT;
  return -1;
}

// Kv heads per kv group (one grid row of blocks each). Rows of 1, 2 or 4 kv heads put several
// positions in one row read. Any other count takes groups of 8 (the last one partly idle when
// the count is not a multiple of 8), except for very small batches. At most 8 (sequence, kv
// group) pairs cut their rows into narrower groups: 4 or 2 heads of 2 or 4 positions per row
// read. That gives more blocks, each with a shorter chain of dependent loads. Same box, 2048
// positions, 8 kv heads: 1 sequence 10.31 -> 8.25 us with groups of 2, 2 sequences 10.44 ->
// 8.71, 4 sequences 10.67 -> 9.67 with groups of 4. At 8 or more sequences, groups of 8 are as
// fast or faster; groups of 1 lose everywhere.
static int kv_group_width(int n_seq, int n_kv_heads) {
  if (n_kv_heads == 1 || n_kv_heads == 2 || n_kv_heads == 4) {
    int w = n_kv_heads;
    while (w > 2 && (long long)n_seq * (n_kv_heads / (w / 2)) <= 8) w /= 2;
    return w;
  }
  for (int w = 2; w <= 4; w *= 2)  // the narrowest width whose pairs fit
    if (n_kv_heads % w == 0 && (long long)n_seq * (n_kv_heads / w) <= 8) return w;
  return 8;
}

static int run_attention(const uint16_t* q, const uint16_t* k_pool, const uint16_t* v_pool,
                         const int32_t* block_tables, const int32_t* seq_lens, uint16_t* out,
                         float* workspace, int n_seq, int max_pages, int n_heads, int n_kv_heads,
                         int num_splits, void* stream) {
  AttnArgs a;
  a.q = reinterpret_cast<const f16*>(q);
  a.k_pool = reinterpret_cast<const f16*>(k_pool);
  a.v_pool = reinterpret_cast<const f16*>(v_pool);
  a.tables = block_tables;
  a.lens = seq_lens;
  a.out = reinterpret_cast<f16*>(out);
  a.part_o = workspace;
  a.part_ml = workspace ? reinterpret_cast<float2*>(
                              workspace + (size_t)n_seq * num_splits * n_heads * kHeadDim)
                        : nullptr;
  a.n_seq = n_seq;
  a.max_pages = max_pages;
  a.n_heads = n_heads;
  a.n_kv_heads = n_kv_heads;
  a.num_splits = num_splits;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (kv_group_width(n_seq, n_kv_heads)) {
    case 4: return attn_launch<4>(a, s);
    case 2: return attn_launch<2>(a, s);
    case 1: return attn_launch<1>(a, s);
    default: return attn_launch<8>(a, s);
  }
}

extern "C" int llmk_attention_decode_fast(const uint16_t* q, const uint16_t* k_pool,
                                          const uint16_t* v_pool, const int32_t* block_tables,
                                          const int32_t* seq_lens, uint16_t* out,
                                          float* workspace, int n_seq, int max_pages,
                                          int page_size, int n_heads, int n_kv_heads,
                                          int head_dim, int num_splits, void* stream) {
  const int st = check_attention(q, k_pool, v_pool, block_tables, seq_lens, out, n_seq,
                                 max_pages, page_size, n_heads, n_kv_heads, head_dim,
                                 num_splits);
  if (st != -1) return st;
  if (num_splits > 1 && !workspace) return LLMK_ERR_INVALID_VALUE;
  // A workspace no allocation can hold (the size saturates): its slot offsets would not fit a
  // size_t either.
  if (num_splits > 1 &&
      llmk_attention_decode_fast_workspace_floats(n_seq, n_heads, num_splits) == SIZE_MAX)
    return LLMK_ERR_INVALID_VALUE;
  if (workspace && !aligned16(workspace)) return LLMK_ERR_ALIGNMENT;
  return run_attention(q, k_pool, v_pool, block_tables, seq_lens, out, workspace, n_seq,
                       max_pages, n_heads, n_kv_heads, num_splits, stream);
}

// ---------------------------------------------------------------------------------------------
// Allocation-free variant: the per-piece partials go to `scratch`, a file-scope device array
// (each GPU the library runs on holds its own copy until the process ends), instead of a
// caller workspace. Its size is the workspace of 256 sequences x 32 query heads x 32 splits,
// 66 MiB. Host code never passes the array's name to a kernel or a copy: the name is a host
// stand-in, and its device address is resolved once per device (with that device current) by
// hipGetSymbolAddress and kept in scratch_dev[]. All calls on one GPU share its array, so
// calls that overlap on one GPU (different streams, no ordering between them) race. Nothing
// in it needs clearing: every call writes each partial it reads, and the piece count, first.
// ---------------------------------------------------------------------------------------------
constexpr size_t kScratchFloats = (size_t)256 * 32 * 32 * (kHeadDim + 2);
static_assert(kScratchFloats == LLMK_ATTN_NOALLOC_MAX_FLOATS, "llmk.h states the scratch size");
static __device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;
static float* scratch_dev[kMaxDevices];
static std::mutex scratch_mu;

// The current device's address of `scratch`, resolved on the first call on that device.
static int scratch_address(float** out) {
  int dev = 0;
  int st = (int)hipGetDevice(&dev);
  if (st != LLMK_OK) return st;
  if (dev < 0 || dev >= kMaxDevices) return LLMK_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (!scratch_dev[dev]) {
    void* p = nullptr;
    st = (int)hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (st != LLMK_OK) return st;
    if (!p) return LLMK_ERR_INVALID_VALUE;
    scratch_dev[dev] = static_cast<float*>(p);
  }
  *out = scratch_dev[dev];
  return LLMK_OK;
}

extern "C" int llmk_attention_decode_fast_noalloc(const uint16_t* q, const uint16_t* k_pool,
                                                  const uint16_t* v_pool,
                                                  const int32_t* block_tables,
                                                  const int32_t* seq_lens, uint16_t* out,
                                                  int n_seq, int max_pages, int page_size,
                                                  int n_heads, int n_kv_heads, int head_dim,
                                                  int num_splits, void* stream) {
  const int st = check_attention(q, k_pool, v_pool, block_tables, seq_lens, out, n_seq,
                                 max_pages, page_size, n_heads, n_kv_heads, head_dim,
                                 num_splits);
  if (st != -1) return st;
  // The size saturates rather than wraps (llmk_attention_decode_fast_workspace_floats), so a
  // call whose partials would not fit is refused here whatever its arguments' magnitudes.
  const size_t need = llmk_attention_decode_fast_workspace_floats(n_seq, n_heads, num_splits);
  if (need > kScratchFloats) return LLMK_ERR_SCRATCH;
  float* ws = nullptr;
  const int sa = scratch_address(&ws);
  if (sa != LLMK_OK) return sa;
  return run_attention(q, k_pool, v_pool, block_tables, seq_lens, out, ws, n_seq, max_pages,
                       n_heads, n_kv_heads, num_splits, stream);
}
