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
#include "common.hpp"

namespace llmk {

template <int UNROLL>
__device__ __forceinline__ void copy_row(const f16* __restrict__ src, f16* __restrict__ dst,
                                         int vpr, int lane) {
  for (int v0 = 0; v0 < vpr; v0 += 64 * UNROLL) {
    u32x4 r[UNROLL];
#pragma unroll
    for (int m = 0; m < UNROLL; ++m) {
      const int v = v0 + lane + 64 * m;
      if (v < vpr) r[m] = ld16_stream(src + 8 * v);
    }
#pragma unroll
    for (int m = 0; m < UNROLL; ++m) {
      const int v = v0 + lane + 64 * m;
      if (v < vpr) st16_stream(dst + 8 * v, r[m]);
    }
  }
}

__device__ __forceinline__ int wave_row() {
  return __builtin_amdgcn_readfirstlane(blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6));
}

__global__ void __launch_bounds__(256)
k_embedding(const f16* __restrict__ table, const int* __restrict__ ids, f16* __restrict__ out,
            int n_tokens, int vpr) {
  const int row = wave_row();
  if (row >= n_tokens) return;
  const long long id = ids[row];
  copy_row<4>(table + id * vpr * 8, out + (size_t)row * vpr * 8, vpr, threadIdx.x & 63);
}

// BATCH: row b goes to position positions[b] of sequence b (table row b of `tables`).
// otherwise: row t goes to position start_pos + t of the one sequence whose table is `tables`.
template <bool BATCH>
__global__ void __launch_bounds__(256)
k_kv_scatter(const f16* __restrict__ src, f16* __restrict__ pool, const int* __restrict__ tables,
             const int* __restrict__ positions, int start_pos, int n_rows, int max_pages,
             int page_size, int vpr) {
  const int row = wave_row();
  if (row >= n_rows) return;
  const int p = BATCH ? positions[row] : start_pos + row;
  const int* table = BATCH ? tables + (size_t)row * max_pages : tables;
  const long long prow = (long long)table[p / page_size] * page_size + p % page_size;
  copy_row<4>(src + (size_t)row * vpr * 8, pool + prow * vpr * 8, vpr, threadIdx.x & 63);
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
  int wpb;
  const dim3 grid = rows_grid(n_tokens, &wpb);
  return launch(k_embedding, grid, dim3(64 * wpb), 0, static_cast<hipStream_t>(stream),
                reinterpret_cast<const f16*>(table), ids, reinterpret_cast<f16*>(out), n_tokens,
                hidden / 8);
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
  int wpb;
  const dim3 grid = rows_grid(T, &wpb);
  return launch(k_kv_scatter<false>, grid, dim3(64 * wpb), 0, static_cast<hipStream_t>(stream),
                reinterpret_cast<const f16*>(src), reinterpret_cast<f16*>(pool), block_table,
                (const int*)nullptr, start_pos, T, 0, page_size, kvdim / 8);
}

extern "C" int llmk_kv_scatter_batch(const uint16_t* src, uint16_t* pool,
                                     const int32_t* block_tables, const int32_t* positions, int n,
                                     int max_pages, int page_size, int kvdim, void* stream) {
  const int st = check_scatter(src, pool, block_tables, n, page_size, kvdim);
  if (st != -1) return st;
  if (!positions || max_pages <= 0) return LLMK_ERR_INVALID_VALUE;
  int wpb;
  const dim3 grid = rows_grid(n, &wpb);
  return launch(k_kv_scatter<true>, grid, dim3(64 * wpb), 0, static_cast<hipStream_t>(stream),
                reinterpret_cast<const f16*>(src), reinterpret_cast<f16*>(pool), block_tables,
                positions, 0, n, max_pages, page_size, kvdim / 8);
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
