// Row argmax of fp16 logits: out[r] = index of the largest value of row r, the lowest index
// among equal values, NaN never chosen, INT_MAX for a row with no value above -inf.
// ref: kernels/argmax.cuh:5-7, kernels/argmax.cu:5-44 (the selection rule; that kernel's own
// initial state, best = -inf with index INT_MAX and a strictly-greater update, is what makes
// NaN and -inf lose and gives INT_MAX to a row of them).
//
// One block per row. At vocab 128256 a row is 256.5 KB: 1024 threads (16 waves, one block per
// CU) read 16 vectors of 16 bytes each, two loads in flight per thread. Each thread scans its
// vectors in increasing index order with a strictly-greater update (lowest index on ties); the
// block then reduces (value, index) pairs with "greater value, or equal value and lower index",
// which is associative and commutative, so the reduction order does not matter.
#include <limits.h>
#include <math.h>

#include "common.hpp"

namespace llmk {
namespace {

constexpr int kArgmaxThreads = 1024;
constexpr int kArgmaxWaves = kArgmaxThreads / 64;
constexpr int kArgmaxUnroll = 16;  // vectors per thread per pass: 16 * 1024 * 8 >= 128256
// Loads in flight per thread (32 KB per CU). Measured at [256, 128256] with the compares below:
// 1 -> 11.9 us, 2 -> 11.7-11.8, 3 -> 12.0, 4 -> 12.0, 6 -> 12.2, 8 or all 16 -> 12.5. With the
// whole row in flight at once the memory system delivers it more slowly.
constexpr int kArgmaxDepth = 2;

// "Greater value, or equal value and lower index", without branches (a short-circuit || here
// becomes exec-mask branches around every step of the reduction).
__device__ __forceinline__ void better(float& v, int& i, float ov, int oi) {
  const bool take = (ov > v) | ((ov == v) & (oi < i));
  v = take ? ov : v;
  i = take ? oi : i;
}

// One step of the (value, index) reduction over a DPP lane permute; CTRL is a control whose
// source lane always exists (quad_perm, row_half_mirror, row_mirror).
template <int CTRL>
__device__ __forceinline__ void better_dpp(float& v, int& i) {
  const float ov = dpp_f32<CTRL>(v);
  const int oi = __builtin_amdgcn_update_dpp(0, i, CTRL, 0xF, 0xF, true);
  better(v, i, ov, oi);
}

// After this every lane of each 16-lane row holds the row's best pair.
__device__ __forceinline__ void row_best(float& v, int& i) {
  better_dpp<0xB1>(v, i);   // quad_perm [1,0,3,2]
  better_dpp<0x4E>(v, i);   // quad_perm [2,3,0,1]
  better_dpp<0x141>(v, i);  // row_half_mirror
  better_dpp<0x140>(v, i);  // row_mirror
}

// Block-wide reduction of (value, index) over the block's nw <= 16 full waves; thread 0 gets the
// result. DPP within rows, readlane across the four rows, then one LDS slot per wave and a final
// row reduction in wave 0. The ds_bpermute shuffles this replaces cost ~100 cycles per step on a
// dependent chain of 24 steps: 13.1 -> 11.6 us at [256, 128256] together with the f16 compares.
__device__ __forceinline__ void block_best(float& v, int& i, int nw) {
  __shared__ float sv[kArgmaxWaves];
  __shared__ int si[kArgmaxWaves];
  row_best(v, i);
  float v0 = readlane_f32(v, 0), v1 = readlane_f32(v, 16);
  float v2 = readlane_f32(v, 32), v3 = readlane_f32(v, 48);
  int i0 = __builtin_amdgcn_readlane(i, 0), i1 = __builtin_amdgcn_readlane(i, 16);
  int i2 = __builtin_amdgcn_readlane(i, 32), i3 = __builtin_amdgcn_readlane(i, 48);
  better(v0, i0, v1, i1);
  better(v2, i2, v3, i3);
  better(v0, i0, v2, i2);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) {
    sv[wave] = v0;
    si[wave] = i0;
  }
  __syncthreads();
  if (wave == 0) {
    v = lane < nw ? sv[lane] : -INFINITY;
    i = lane < nw ? si[lane] : INT_MAX;
    row_best(v, i);  // the nw entries sit in lanes 0-15, so row 0 ends with the answer
  }
}

// 16-byte path: rows 16-byte aligned (vocab % 8 == 0 and an aligned base). ONE: the row fits
// one pass (vocab <= 131072, Llama-3's 128256 included), and the pass loop is left out: 11.66
// against 11.74 us at [256, 128256], same box, same bits.
template <bool ONE>
__global__ void __launch_bounds__(kArgmaxThreads)
k_argmax_vec(const f16* __restrict__ logits, int* __restrict__ out, int vocab) {
  const f16* row = logits + (size_t)blockIdx.x * vocab;
  const int nvec = vocab / 8;
  f16 best = (f16)-INFINITY;  // fp16 compares order exactly as the fp32 values do
  int best_i = INT_MAX;
  for (int base = 0; ONE ? base == 0 : base < nvec; base += kArgmaxUnroll * kArgmaxThreads) {
    // Vectors past the row's end load its last vector again, unmasked: a copy repeats values
    // that the vector's own thread also sees, at a larger index, so under the lowest-index rule
    // it never wins. The loads stay unconditional (a masked load makes the compiler wait for
    // every earlier load at its first use), and no per-element mask is computed.
    u32x4 x[kArgmaxUnroll];
    auto load = [&](int u) {
      const int j = base + u * kArgmaxThreads + (int)threadIdx.x;
      x[u] = ld16_stream(row + (size_t)(j < nvec ? j : nvec - 1) * 8);
    };
#pragma unroll
    for (int u = 0; u < kArgmaxDepth; ++u) load(u);
#pragma unroll
    for (int u = 0; u < kArgmaxUnroll; ++u) {
      const int j = base + u * kArgmaxThreads + (int)threadIdx.x;
      const f16x8 h = as_h8(x[u]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (e == 4) {
          // The next load goes out mid-vector; the barrier keeps the scheduler from hoisting
          // the remaining loads, which puts the whole row in flight again.
          if (u + kArgmaxDepth < kArgmaxUnroll) load(u + kArgmaxDepth);
          __builtin_amdgcn_sched_barrier(0);
        }
        if (h[e] > best) {  // increasing index within the thread: ties keep the earlier one
          best = h[e];
          best_i = j * 8 + e;
        }
      }
    }
  }
  float best_f = (float)best;
  block_best(best_f, best_i, kArgmaxWaves);
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
  if (vocab % 8 == 0 && aligned16(logits) && threads == kArgmaxThreads) {
    if (vocab / 8 <= kArgmaxUnroll * kArgmaxThreads)
      return launch(k_argmax_vec<true>, dim3((unsigned)n_rows), dim3(threads), 0, s, l, out,
                    vocab);
    return launch(k_argmax_vec<false>, dim3((unsigned)n_rows), dim3(threads), 0, s, l, out,
                  vocab);
  }
  return launch(k_argmax_scalar, dim3((unsigned)n_rows), dim3(threads), 0, s, l, out, vocab);
}
