// Row argmax of fp16 logits: out[r] = index of the largest value of row r, the lowest index
// among equal values, NaN never chosen, INT_MAX for a row with no value above -inf.
// ref: kernels/argmax.cuh:5-7, kernels/argmax.cu:5-44 (the selection rule; that kernel's own
// initial state, best = -inf with index INT_MAX and a strictly-greater update, is what makes
// NaN and -inf lose and gives INT_MAX to a row of them).
//
// One block per row. At vocab 128256 a row is 256.5 KB: 1024 threads issue all of their 16-byte
// loads (16 per thread) before comparing, so the whole row is in flight at once, and one
// 1024-thread block per CU is 16 waves. Each thread scans its vectors in increasing index order
// with a strictly-greater update (lowest index on ties); the block then reduces (value, index)
// pairs with "greater value, or equal value and lower index", which is associative and
// commutative, so the reduction order does not matter.
#include <limits.h>
#include <math.h>

#include "common.hpp"

namespace llmk {
namespace {

constexpr int kArgmaxThreads = 1024;
constexpr int kArgmaxWaves = kArgmaxThreads / 64;
constexpr int kArgmaxUnroll = 16;  // vectors per thread per pass: 16 * 1024 * 8 >= 128256

__device__ __forceinline__ void better(float& v, int& i, float ov, int oi) {
  if (ov > v || (ov == v && oi < i)) {
    v = ov;
    i = oi;
  }
}

// Block-wide reduction of (value, index) over the block's nw waves; thread 0 gets the result.
__device__ __forceinline__ void block_best(float& v, int& i, int nw) {
  __shared__ float sv[kArgmaxWaves];
  __shared__ int si[kArgmaxWaves];
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(v, o);
    const int oi = __shfl_xor(i, o);
    better(v, i, ov, oi);
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) {
    sv[wave] = v;
    si[wave] = i;
  }
  __syncthreads();
  if (wave == 0) {
    v = lane < nw ? sv[lane] : -INFINITY;
    i = lane < nw ? si[lane] : INT_MAX;
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(v, o);
      const int oi = __shfl_xor(i, o);
      better(v, i, ov, oi);
    }
  }
}

// 16-byte path: rows 16-byte aligned (vocab % 8 == 0 and an aligned base).
__global__ void __launch_bounds__(kArgmaxThreads)
k_argmax_vec(const f16* __restrict__ logits, int* __restrict__ out, int vocab) {
  const f16* row = logits + (size_t)blockIdx.x * vocab;
  const int nvec = vocab / 8;
  float best = -INFINITY;
  int best_i = INT_MAX;
  for (int base = 0; base < nvec; base += kArgmaxUnroll * kArgmaxThreads) {
    // Vectors past the row's end load its last vector again and compare as -inf: the loads
    // stay unconditional, so the compares of vector u wait only for load u (with a masked load
    // the compiler waited for all 16 first; 14.1 -> 13.3 us at [256, 128256]).
    u32x4 x[kArgmaxUnroll];
#pragma unroll
    for (int u = 0; u < kArgmaxUnroll; ++u) {
      const int j = base + u * kArgmaxThreads + (int)threadIdx.x;
      x[u] = ld16_stream(row + (size_t)(j < nvec ? j : nvec - 1) * 8);
    }
#pragma unroll
    for (int u = 0; u < kArgmaxUnroll; ++u) {
      const int j = base + u * kArgmaxThreads + (int)threadIdx.x;
      const f16x8 h = as_h8(x[u]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float v = j < nvec ? (float)h[e] : -INFINITY;
        if (v > best) {  // increasing index within the thread: ties keep the earlier one
          best = v;
          best_i = j * 8 + e;
        }
      }
    }
  }
  block_best(best, best_i, kArgmaxWaves);
  if (threadIdx.x == 0) out[blockIdx.x] = best_i;
}

// Any vocab and alignment: 2-byte loads, strided by the block.
__global__ void __launch_bounds__(kArgmaxThreads)
k_argmax_scalar(const f16* __restrict__ logits, int* __restrict__ out, int vocab) {
  const f16* row = logits + (size_t)blockIdx.x * vocab;
  float best = -INFINITY;
  int best_i = INT_MAX;
  for (int i = threadIdx.x; i < vocab; i += blockDim.x) {
    const float v = (float)row[i];
    if (v > best) {
      best = v;
      best_i = i;
    }
  }
  block_best(best, best_i, (int)blockDim.x >> 6);
  if (threadIdx.x == 0) out[blockIdx.x] = best_i;
}

}  // namespace
}  // namespace llmk

using namespace llmk;

extern "C" int llmk_argmax_rows(const uint16_t* logits, int32_t* out, int n_rows, int vocab,
                                void* stream) {
  if (n_rows == 0) return LLMK_OK;
  if (n_rows < 0 || vocab <= 0 || !logits || !out) return LLMK_ERR_INVALID_VALUE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const f16* l = reinterpret_cast<const f16*>(logits);
  // Fewer threads for short rows, so a block is not mostly idle.
  const unsigned threads = vocab >= 8 * kArgmaxThreads ? kArgmaxThreads : 256;
  if (vocab % 8 == 0 && aligned16(logits) && threads == kArgmaxThreads)
    return launch(k_argmax_vec, dim3((unsigned)n_rows), dim3(threads), 0, s, l, out, vocab);
  return launch(k_argmax_scalar, dim3((unsigned)n_rows), dim3(threads), 0, s, l, out, vocab);
}
