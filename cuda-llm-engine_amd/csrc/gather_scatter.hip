// Row gathers and scatters: the embedding lookup, the paged KV scatter (prefill and decode),
// and the device copy used as the bandwidth probe. All are bit-exact 16-byte copies; the only
// arithmetic is the row address.
//
// Mapping: one wave64 per row. The row index and the source/destination row addresses are
// wave-uniform, so they are computed once per wave in scalar registers (the index arrays are
// read with scalar loads); lane l copies vectors l, l+64, ... of the row, UNROLL of them
// loaded before any is stored.
//
// ref: kernels/embedding.cu:4-16 (embedding_lookup), kernels/kv_scatter.cu:4-40 (kv_scatter,
// kv_scatter_batch), bench/bandwidth.cu:11-15 (copy probe).
#include <type_traits>

#include "common.hpp"

namespace llmk {

// Copies one row of vpr 16-byte vectors with one wave: lane l moves vectors l, l+64, ...;
// UNROLL of them are loaded before any is stored. FULL: vpr is a multiple of 64 * UNROLL, so no
// lane needs a bounds test.
template <int UNROLL, bool FULL>
__device__ __forceinline__ void copy_row(const f16* __restrict__ src, f16* __restrict__ dst,
                                         int vpr, int lane) {
  for (int v0 = 0; v0 < vpr; v0 += 64 * UNROLL) {
    u32x4 r[UNROLL];
#pragma unroll
    for (int m = 0; m < UNROLL; ++m) {
      const int v = v0 + lane + 64 * m;
      if (FULL || v < vpr) r[m] = ld16_stream(src + 8 * v);
    }
#pragma unroll
    for (int m = 0; m < UNROLL; ++m) {
      const int v = v0 + lane + 64 * m;
      if (FULL || v < vpr) st16_stream(dst + 8 * v, r[m]);
    }
  }
}

// 0: vpr a multiple of 256, 1: a multiple of 64, 2: anything.
static int row_kind(int vpr) { return vpr % 256 == 0 ? 0 : (vpr % 64 == 0 ? 1 : 2); }

template <int KIND>
__device__ __forceinline__ void copy_row_kind(const f16* __restrict__ src, f16* __restrict__ dst,
                                              int vpr, int lane) {
  if (KIND == 0) copy_row<4, true>(src, dst, vpr, lane);
  else if (KIND == 1) copy_row<1, true>(src, dst, vpr, lane);
  else copy_row<4, false>(src, dst, vpr, lane);
}

// The wave's row; wpb (waves per block) comes as a kernel argument, not from blockDim: the
// arguments arrive preloaded in SGPRs, blockDim would cost a scalar fetch first.
__device__ __forceinline__ int wave_row(int wpb) {
  return __builtin_amdgcn_readfirstlane(blockIdx.x * wpb + (threadIdx.x >> 6));
}

template <int KIND>
__global__ void __launch_bounds__(256)
k_embedding(const f16* __restrict__ table, const int* __restrict__ ids, f16* __restrict__ out,
            int n_tokens, int vpr, int wpb) {
  const int row = wave_row(wpb);
  if (row >= n_tokens) return;
  const long long id = ids[row];
  copy_row_kind<KIND>(table + id * vpr * 8, out + (size_t)row * vpr * 8, vpr, threadIdx.x & 63);
}

// Rows whose width is a multiple of 256 vectors (hidden % 2048 == 0), R rows per wave: for each
// 256-vector slice, the R rows' loads (4 per lane per row) are all issued before any store, so
// a wave keeps 16 * 4 * R bytes per lane in flight. Groups of R consecutive tokens are dealt to
// the waves round-robin; the host sizes the grid at one 4-wave block per CU at most.
// The group's ids are wave-uniform and come through the scalar cache (one s_load_dwordx8 for a
// full group of 8) instead of one vector load and 8 readlanes. VPR > 0 fixes the row width at
// compile time (256 vectors = hidden 2048, 512 = hidden 4096): the row bases then stay in scalar
// registers and each load is base + lane offset, where a runtime width costs a 64-bit VGPR
// address per load (12.1 -> 11.7 us at 8192 tokens of 2048).
template <int R>
__device__ __forceinline__ void gather_group(const f16* __restrict__ table,
                                             const int* __restrict__ ids, f16* __restrict__ out,
                                             int row0, int n_rows, int vpr, int lane) {
  long long off[R];  // offsets, not pointers: loads index the restrict-qualified table
#pragma unroll
  for (int h = 0; h < R; ++h) {
    // A partial group (n_rows < R) reads its last id again for the rows it does not store.
    const int t = h < n_rows ? h : n_rows - 1;
    off[h] = (long long)__builtin_amdgcn_readfirstlane(ids[row0 + t]) * vpr * 8;
  }
  for (int v0 = 0; v0 < vpr; v0 += 256) {
    u32x4 r[4 * R];
#pragma unroll
    for (int h = 0; h < R; ++h)
#pragma unroll
      for (int m = 0; m < 4; ++m)
        r[4 * h + m] = ld16_stream(table + off[h] + 8 * (v0 + lane + 64 * m));
    // Keep the scheduler from sinking loads below stores to save registers: the point is to
    // have all 4 * R loads in flight at once.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int h = 0; h < R; ++h) {
      if (h < n_rows) {
        f16* dst = out + (size_t)(row0 + h) * vpr * 8;
#pragma unroll
        for (int m = 0; m < 4; ++m) st16_stream(dst + 8 * (v0 + lane + 64 * m), r[4 * h + m]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// ONE: the grid has a wave for every group (up to 8192 tokens), so no loop (0.1-0.15 us less
// than the loop's single pass at 8192 tokens).
template <int R, int VPR, bool ONE>
__global__ void __launch_bounds__(256)
k_embedding_rows(const f16* __restrict__ table, const int* __restrict__ ids,
                 f16* __restrict__ out, int n_tokens, int vpr_arg, int n_waves) {
  const int vpr = VPR > 0 ? VPR : vpr_arg;
  const int lane = threadIdx.x & 63;
  const int n_groups = (n_tokens + R - 1) / R;
  if (ONE) {
    const int g = wave_row(4);
    if (g >= n_groups) return;
    const int row0 = g * R;
    if (row0 + R <= n_tokens)
      gather_group<R>(table, ids, out, row0, R, vpr, lane);
    else
      gather_group<R>(table, ids, out, row0, n_tokens - row0, vpr, lane);
    return;
  }
  for (int g = wave_row(4); g < n_groups; g += n_waves) {
    const int row0 = g * R;
    if (row0 + R <= n_tokens)
      gather_group<R>(table, ids, out, row0, R, vpr, lane);  // constant row count: no guards
    else
      gather_group<R>(table, ids, out, row0, n_tokens - row0, vpr, lane);
  }
}

// BATCH: row b goes to position positions[b] of sequence b (table row b of `tables`).
// otherwise: row t goes to position start_pos + t of the one sequence whose table is `tables`.
template <bool BATCH, int KIND>
__global__ void __launch_bounds__(256)
k_kv_scatter(const f16* __restrict__ src, f16* __restrict__ pool, const int* __restrict__ tables,
             const int* __restrict__ positions, int start_pos, int n_rows, int max_pages,
             int page_size, int vpr, int wpb) {
  const int row = wave_row(wpb);
  if (row >= n_rows) return;
  const int p = BATCH ? positions[row] : start_pos + row;
  const int* table = BATCH ? tables + (size_t)row * max_pages : tables;
  const long long prow = (long long)table[p / page_size] * page_size + p % page_size;
  copy_row_kind<KIND>(src + (size_t)row * vpr * 8, pool + prow * vpr * 8, vpr, threadIdx.x & 63);
}

template <int UNROLL>
__global__ void __launch_bounds__(256)
k_copy(const u32x4* __restrict__ src, u32x4* __restrict__ dst, size_t nvec) {
  const size_t chunk = (size_t)blockDim.x * UNROLL;
  for (size_t b = (size_t)blockIdx.x * chunk; b < nvec; b += (size_t)gridDim.x * chunk) {
    u32x4 r[UNROLL];
#pragma unroll
    for (int m = 0; m < UNROLL; ++m) {
      const size_t i = b + threadIdx.x + (size_t)m * blockDim.x;
      if (i < nvec) r[m] = __builtin_nontemporal_load(src + i);
    }
#pragma unroll
    for (int m = 0; m < UNROLL; ++m) {
      const size_t i = b + threadIdx.x + (size_t)m * blockDim.x;
      if (i < nvec) __builtin_nontemporal_store(r[m], dst + i);
    }
  }
}

static dim3 rows_grid(int n_rows, int* wpb) {
  *wpb = n_rows >= 4096 ? 4 : 1;
  return dim3(ceil_div((size_t)n_rows, (size_t)*wpb));
}

}  // namespace llmk

using namespace llmk;

extern "C" int llmk_embedding_lookup(const uint16_t* table, const int32_t* ids, uint16_t* out,
                                     int n_tokens, int hidden, void* stream) {
  if (n_tokens < 0 || hidden <= 0) return LLMK_ERR_INVALID_VALUE;
  if (n_tokens == 0) return LLMK_OK;
  if (!table || !ids || !out) return LLMK_ERR_INVALID_VALUE;
  if (hidden % 8 != 0) return LLMK_ERR_SHAPE;
  if (!aligned16(table) || !aligned16(out)) return LLMK_ERR_ALIGNMENT;
  const int vpr = hidden / 8;
  if (vpr % 256 == 0 && n_tokens > 1024) {
    // 1024 waves (4 per CU, one block per CU), each moving R rows at a time: at 8192 tokens of
    // 2048 this measured 11.7 us against 13.9 us for one row per wave.
    const int R = n_tokens >= 8 * 1024 ? 8 : (n_tokens >= 4 * 1024 ? 4 : 2);
    const int groups = (n_tokens + R - 1) / R;
    const unsigned blocks = ceil_div((size_t)(groups < 1024 ? groups : 1024), 4);
    auto go = [&](auto kern) {
      return launch(kern, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                    reinterpret_cast<const f16*>(table), ids, reinterpret_cast<f16*>(out),
                    n_tokens, vpr, (int)(4 * blocks));
    };
    const bool one = groups <= (int)(4 * blocks);
    auto width = [&](auto r) {
      constexpr int RR = decltype(r)::value;
      if (vpr == 256)
        return one ? go(k_embedding_rows<RR, 256, true>) : go(k_embedding_rows<RR, 256, false>);
      if (vpr == 512)
        return one ? go(k_embedding_rows<RR, 512, true>) : go(k_embedding_rows<RR, 512, false>);
      return one ? go(k_embedding_rows<RR, 0, true>) : go(k_embedding_rows<RR, 0, false>);
    };
    if (R == 8) return width(std::integral_constant<int, 8>());
    if (R == 4) return width(std::integral_constant<int, 4>());
    return width(std::integral_constant<int, 2>());
  }
  int wpb;
  const dim3 grid = rows_grid(n_tokens, &wpb);
  auto go = [&](auto kern) {
    return launch(kern, grid, dim3(64 * wpb), 0, static_cast<hipStream_t>(stream),
                  reinterpret_cast<const f16*>(table), ids, reinterpret_cast<f16*>(out), n_tokens,
                  vpr, wpb);
  };
  switch (row_kind(vpr)) {
    case 0: return go(k_embedding<0>);
    case 1: return go(k_embedding<1>);
    default: return go(k_embedding<2>);
  }
}

template <bool BATCH>
static int scatter_launch(const uint16_t* src, uint16_t* pool, const int32_t* tables,
                          const int32_t* positions, int start_pos, int n_rows, int max_pages,
                          int page_size, int kvdim, void* stream) {
  int wpb;
  const dim3 grid = rows_grid(n_rows, &wpb);
  const int vpr = kvdim / 8;
  auto go = [&](auto kern) {
    return launch(kern, grid, dim3(64 * wpb), 0, static_cast<hipStream_t>(stream),
                  reinterpret_cast<const f16*>(src), reinterpret_cast<f16*>(pool), tables,
                  positions, start_pos, n_rows, max_pages, page_size, vpr, wpb);
  };
  switch (row_kind(vpr)) {
    case 0: return go(k_kv_scatter<BATCH, 0>);
    case 1: return go(k_kv_scatter<BATCH, 1>);
    default: return go(k_kv_scatter<BATCH, 2>);
  }
}

static int check_scatter(const void* src, const void* pool, const void* table, int n_rows,
                         int page_size, int kvdim) {
  if (n_rows < 0 || page_size <= 0 || kvdim <= 0) return LLMK_ERR_INVALID_VALUE;
  if (n_rows == 0) return LLMK_OK;
  if (!src || !pool || !table) return LLMK_ERR_INVALID_VALUE;
  if (kvdim % 8 != 0) return LLMK_ERR_SHAPE;
  if (!aligned16(src) || !aligned16(pool)) return LLMK_ERR_ALIGNMENT;
  return -1;
}

extern "C" int llmk_kv_scatter(const uint16_t* src, uint16_t* pool, const int32_t* block_table,
                               int start_pos, int T, int page_size, int kvdim, void* stream) {
  const int st = check_scatter(src, pool, block_table, T, page_size, kvdim);
  if (st != -1) return st;
  if (start_pos < 0) return LLMK_ERR_INVALID_VALUE;
  return scatter_launch<false>(src, pool, block_table, nullptr, start_pos, T, 0, page_size, kvdim,
                               stream);
}

extern "C" int llmk_kv_scatter_batch(const uint16_t* src, uint16_t* pool,
                                     const int32_t* block_tables, const int32_t* positions, int n,
                                     int max_pages, int page_size, int kvdim, void* stream) {
  const int st = check_scatter(src, pool, block_tables, n, page_size, kvdim);
  if (st != -1) return st;
  if (!positions || max_pages <= 0) return LLMK_ERR_INVALID_VALUE;
  return scatter_launch<true>(src, pool, block_tables, positions, 0, n, max_pages, page_size,
                              kvdim, stream);
}

extern "C" int llmk_copy_bytes(const void* src, void* dst, size_t nbytes, void* stream) {
  if (nbytes == 0) return LLMK_OK;
  if (!src || !dst) return LLMK_ERR_INVALID_VALUE;
  if (nbytes % 16 != 0) return LLMK_ERR_SHAPE;
  if (!aligned16(src) || !aligned16(dst)) return LLMK_ERR_ALIGNMENT;
  constexpr int UNROLL = 4;
  const size_t nvec = nbytes / 16;
  const size_t need = ceil_div(nvec, 256 * UNROLL);
  const unsigned blocks = need < 8192 ? (unsigned)need : 8192u;
  return launch(k_copy<UNROLL>, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                reinterpret_cast<const u32x4*>(src), reinterpret_cast<u32x4*>(dst), nvec);
}
