// The projections of a decode step with few rows: y[T, out] = x[T, in] * W^T, W stored [out, in]
// row-major (a PyTorch Linear without bias), fp16 in and out, fp32 accumulation, for T <= 8.
// ref: kernels/linear.cu:5-25 (cublasGemmEx with CUBLAS_COMPUTE_32F), the reference's only GEMM,
// which the engine calls for every projection whatever the batch size.
//
// With T <= 8 rows a projection does at most 16 flops per weight byte, far below MI355X's ~300
// flop/byte balance point, so it is a stream over W: the design goal is to keep HBM busy.
//   - A block owns kRows = 8 consecutive output rows. The in dimension is cut into steps of 512
//     (64 lanes x 8 halves), and the block's WV waves (4, 8 or 16: one step each where the
//     registers allow) take steps w, w + WV, ... For each step a wave issues one 16-byte load per
//     W row (64 lanes cover 1 KiB of the row, fully coalesced) and one per x row (x is small and
//     stays in the L2), then accumulates the 8 x T partial dot products of its lane in fp32 with
//     v_dot2_f32_f16.
//   - The 8 * TP partial sums of a lane are then reduced over the wave in a halving butterfly:
//     at each exchange a lane keeps half of its values and adds its partner's copy of them, so
//     the 64 lanes end up holding distinct (row, token) sums after 63 adds (mostly DPP) instead
//     of 8 * TP full reductions. The waves' sums meet in LDS.
// Summation order differs from cuBLAS/hipBLASLt (lane-strided partial sums, then the butterfly),
// so results agree with the fp32 dot product to fp32 rounding, not bit for bit.
#include "common.hpp"

namespace llmk {
namespace {

constexpr int kRows = 8;      // output rows per block
constexpr int kStep = 512;    // in elements per wave step: 64 lanes x 8 halves

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t elem(u32x4 v, int k) {
  const uint32_t e = v[k];
  return e;
}

// acc + the dot product of 8 fp16 pairs, fp32 accumulation.
__device__ __forceinline__ float dot8(u32x4 a, u32x4 b, float acc) {
#pragma unroll
  for (int k = 0; k < 4; ++k)
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, elem(a, k)),
                                 __builtin_bit_cast(h2, elem(b, k)), acc, false);
  return acc;
}

// The halving butterfly: N partial sums per lane (value index r * TP + t) are reduced over the 64
// lanes in six exchanges. An exchange pairs lanes that differ in lane bit M: while more than one
// value is left, a lane with that bit set keeps the upper half of its values, its partner the
// lower half, and each adds the half its partner kept; with one value left the pair simply adds.
// The exchanges run in the order M = 8, 4, 2, 1, 16, 32: the first four pair lanes of one 16-lane
// row through DPP (row_mirror pairs i with 15 - i, row_half_mirror i with 7 - i, quad_perm i with
// i ^ 2 and i ^ 1; each pair differs in bit M and agrees in the bits already used), which leaves
// at most 4 values for the two exchanges across rows (LDS permutes).
constexpr int kMask[6] = {8, 4, 2, 1, 16, 32};
constexpr int kDpp[4] = {0x140, 0x141, 0x4E, 0xB1};  // row_mirror, row_half_mirror, quad_perm x2

template <int S>
__device__ __forceinline__ float partner(float v) {
  if constexpr (S < 4) return dpp_f32<kDpp[S]>(v);
  else return __shfl_xor(v, kMask[S]);
}

template <int N, int S>
__device__ __forceinline__ void butterfly(float (&v)[64]) {
  if constexpr (S < 6) {
    if constexpr (N > 1) {
      const bool up = (threadIdx.x & kMask[S]) != 0;
#pragma unroll
      for (int i = 0; i < N / 2; ++i) {
        const float send = up ? v[i] : v[i + N / 2];
        const float keep = up ? v[i + N / 2] : v[i];
        v[i] = keep + partner<S>(send);
      }
      butterfly<N / 2, S + 1>(v);
    } else {
      v[0] = v[0] + partner<S>(v[0]);
      butterfly<1, S + 1>(v);
    }
  }
}

// After butterfly<N, 0>: the value index whose total lane `lane` holds (its bits, from the top,
// are the lane's bits kMask[0], kMask[1], ... of the halving exchanges), and whether the lane is
// the one of its group that stores it (lane bits of the full-add exchanges clear).
template <int N>
__device__ __forceinline__ int butterfly_index(int lane, bool* writer) {
  int idx = 0, n = N;
  bool w = true;
#pragma unroll
  for (int s = 0; s < 6; ++s) {
    const bool bit = (lane & kMask[s]) != 0;
    if (n > 1) {
      idx = 2 * idx + (bit ? 1 : 0);
      n /= 2;
    } else {
      w = w && !bit;
    }
  }
  *writer = w;
  return idx;
}

// TP: rows computed (a power of two >= T; rows t >= T reuse row T - 1 and are not stored).
// WV: waves per block, dividing the in dimension's steps between them.
template <int TP, int WV>
__global__ void __launch_bounds__(64 * WV)
k_gemv(const f16* __restrict__ x, const f16* __restrict__ w, f16* __restrict__ y, int T, int in,
       int out) {
  constexpr int N = kRows * TP;  // partial sums per lane: value index r * TP + t
  __shared__ float part[WV][N];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j0 = blockIdx.x * kRows;
  const int steps = in / kStep;

  float v[64];
#pragma unroll
  for (int i = 0; i < 64; ++i) v[i] = 0.0f;
  const f16* wr[kRows];
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const int j = j0 + r < out ? j0 + r : out - 1;  // rows past `out`: computed, not stored
    wr[r] = w + (size_t)j * in + lane * 8;
  }
  const f16* xr[TP];
#pragma unroll
  for (int t = 0; t < TP; ++t) xr[t] = x + (size_t)(t < T ? t : T - 1) * in + lane * 8;

  for (int s = wave; s < steps; s += WV) {
    const size_t k = (size_t)s * kStep;
    u32x4 wv[kRows], xv[TP];
#pragma unroll
    for (int r = 0; r < kRows; ++r) wv[r] = ld16_stream(wr[r] + k);
#pragma unroll
    for (int t = 0; t < TP; ++t) xv[t] = ld16(xr[t] + k);
    // Every load of the step is in flight before the first product (left alone, the scheduler
    // reuses one register for the W rows and waits for each load in turn).
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < kRows; ++r)
#pragma unroll
      for (int t = 0; t < TP; ++t) v[r * TP + t] = dot8(wv[r], xv[t], v[r * TP + t]);
  }

  butterfly<N, 0>(v);
  bool writer;
  const int idx = butterfly_index<N>(lane, &writer);
  if (writer) part[wave][idx] = v[0];
  __syncthreads();
  if (threadIdx.x < N) {
    const int r = threadIdx.x / TP, t = threadIdx.x % TP;
    float sum = 0.0f;
#pragma unroll
    for (int q = 0; q < WV; ++q) sum += part[q][threadIdx.x];
    if (j0 + r < out && t < T) y[(size_t)t * out + j0 + r] = (f16)sum;
  }
}

// Waves per block: enough that a wave takes one step of the in dimension, up to 16 (8 with 8
// rows, whose 130 registers a 1024-thread block cannot give every wave).
template <int TP>
int gemv_launch(const f16* x, const f16* w, f16* y, int T, int in, int out, hipStream_t s) {
  const dim3 grid(ceil_div((size_t)out, kRows));
  const int steps = in / kStep;
  if constexpr (TP < 8)
    if (steps > 8) return launch(k_gemv<TP, 16>, grid, dim3(64 * 16), 0, s, x, w, y, T, in, out);
  if (steps > 4) return launch(k_gemv<TP, 8>, grid, dim3(64 * 8), 0, s, x, w, y, T, in, out);
  return launch(k_gemv<TP, 4>, grid, dim3(64 * 4), 0, s, x, w, y, T, in, out);
}

}  // namespace
}  // namespace llmk

using namespace llmk;

extern "C" int llmk_linear_rows(const uint16_t* x, const uint16_t* w, uint16_t* y, int T,
                                int in_features, int out_features, void* stream) {
  if (T < 0 || in_features <= 0 || out_features <= 0) return LLMK_ERR_INVALID_VALUE;
  if (T == 0) return LLMK_OK;
  if (!x || !w || !y) return LLMK_ERR_INVALID_VALUE;
  if (T > LLMK_LINEAR_ROWS_MAX || in_features % kStep != 0) return LLMK_ERR_UNSUPPORTED;
  if (!aligned16(x) || !aligned16(w)) return LLMK_ERR_ALIGNMENT;
  if ((size_t)out_features > (size_t)0xFFFFFFFFu * kRows) return LLMK_ERR_UNSUPPORTED;
  const f16* xh = reinterpret_cast<const f16*>(x);
  const f16* wh = reinterpret_cast<const f16*>(w);
  f16* yh = reinterpret_cast<f16*>(y);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (T == 1) return gemv_launch<1>(xh, wh, yh, T, in_features, out_features, s);
  if (T == 2) return gemv_launch<2>(xh, wh, yh, T, in_features, out_features, s);
  if (T <= 4) return gemv_launch<4>(xh, wh, yh, T, in_features, out_features, s);
  return gemv_launch<8>(xh, wh, yh, T, in_features, out_features, s);
}
