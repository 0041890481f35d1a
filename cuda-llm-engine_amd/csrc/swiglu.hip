// SwiGLU: out[i] = fp16(r16(silu(g)) * u) with silu(g) = g / (1 + exp(-g)) in fp32.
// ref: kernels/swiglu.cu:4-21. silu is rounded to fp16 before the multiply (ref:
// kernels/swiglu.cu:12); the product of two fp16 values rounded to fp16 is one packed fp16
// multiply.
//
// At [8192, 8192] the kernel is as close to compute-bound as to memory-bound: the exact silu
// (library expf + IEEE divide) costs ~28 VALU instructions per element, about the time the
// 402 MB take at HBM speed. silu_r16 below settles ~99% of elements with ~14 instructions and
// recomputes the rest exactly, keeping the output bit-identical to the exact formula.
//
// Gate and up are streamed once, in 16-byte vectors, UNROLL vectors of each per thread so that
// 2 * UNROLL loads are in flight before the first use.
#include "common.hpp"
#include "pointwise.hpp"

namespace llmk {

// silu of the NV * 8 fp16 values in g, rounded to fp16, into s. One fast pass over all of them
// records the unsettled ones in a bit mask; a per-lane loop then recomputes just those, so a
// wave runs the exact path as many times as its busiest lane needs it (usually once or never)
// rather than once for every element slot some lane needs it in.
template <int NV>
__device__ __forceinline__ void silu_vectors(const u32x4 (&g)[NV], u32x4 (&s)[NV]) {
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

// Each block owns 256 * UNROLL consecutive vectors of each input; the grid covers the whole
// range in one pass. Blocks wholly inside the range take a straight-line path without
// per-vector tests, so all 2 * UNROLL loads issue back to back; only the last block tests.
// (A grid-stride loop around the same body measured 10% slower at [8192, 8192].)
// Threads per block of the vector kernels (a constant, not blockDim: the kernel arguments
// arrive preloaded in SGPRs, blockDim would cost a scalar fetch before the first address).
constexpr int kSwigluThreads = 256;

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

template <int UNROLL>
__global__ void __launch_bounds__(kSwigluThreads)
k_swiglu_vec(const f16* __restrict__ gate, const f16* __restrict__ up, f16* __restrict__ out,
             size_t nvec, size_t n) {
  const size_t chunk = (size_t)kSwigluThreads * UNROLL;
  const size_t b = (size_t)blockIdx.x * chunk;
  if (b + chunk <= nvec) swiglu_block<UNROLL>(gate, up, out, b, nvec, true);
  else if (b < nvec) swiglu_block<UNROLL>(gate, up, out, b, nvec, false);
  const size_t t = nvec * 8 + (size_t)blockIdx.x * kSwigluThreads + threadIdx.x;  // n % 8 tail
  if (t < n) out[t] = silu_r16(gate[t]) * up[t];
}

__global__ void __launch_bounds__(256)
k_swiglu_scalar(const f16* __restrict__ gate, const f16* __restrict__ up, f16* __restrict__ out,
                size_t n) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    out[i] = silu_r16(gate[i]) * up[i];
}

// Rows of the fused gate/up projection: row r of `gu` holds gate in columns [0, inter) and up
// in [inter, 2 * inter); out row r = swiglu(gate row, up row). Grid (column blocks, rows), the
// same per-block body as the flat kernel over each row's two runs.
template <int UNROLL>
__global__ void __launch_bounds__(kSwigluThreads)
k_swiglu_rows(const f16* __restrict__ gu, f16* __restrict__ out, int inter) {
  const size_t r = blockIdx.y;
  const f16* g = gu + r * 2 * (size_t)inter;
  const size_t nvec = (size_t)inter / 8;
  const size_t chunk = (size_t)kSwigluThreads * UNROLL;
  const size_t b = (size_t)blockIdx.x * chunk;
  if (b + chunk <= nvec) swiglu_block<UNROLL>(g, g + inter, out + r * inter, b, nvec, true);
  else if (b < nvec) swiglu_block<UNROLL>(g, g + inter, out + r * inter, b, nvec, false);
}

}  // namespace llmk

using namespace llmk;

extern "C" int llmk_swiglu_rows(const uint16_t* gate_up, uint16_t* out, int n_rows, int inter,
                                void* stream) {
  if (n_rows < 0 || inter <= 0) return LLMK_ERR_INVALID_VALUE;
  if (n_rows == 0) return LLMK_OK;
  if (!gate_up || !out) return LLMK_ERR_INVALID_VALUE;
  if (inter % 8 != 0) return LLMK_ERR_SHAPE;
  if (n_rows > 65535) return LLMK_ERR_UNSUPPORTED;
  if (!aligned16(gate_up) || !aligned16(out)) return LLMK_ERR_ALIGNMENT;
  constexpr int UNROLL = 2;
  const dim3 grid(ceil_div((size_t)inter / 8, kSwigluThreads * UNROLL), (unsigned)n_rows);
  return launch(k_swiglu_rows<UNROLL>, grid, dim3(kSwigluThreads), 0,
                static_cast<hipStream_t>(stream),
                reinterpret_cast<const f16*>(gate_up), reinterpret_cast<f16*>(out), inter);
}

extern "C" int llmk_swiglu(const uint16_t* gate, const uint16_t* up, uint16_t* out, size_t n,
                           void* stream) {
  if (n == 0) return LLMK_OK;
  if (!gate || !up || !out) return LLMK_ERR_INVALID_VALUE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const f16* g = reinterpret_cast<const f16*>(gate);
  const f16* u = reinterpret_cast<const f16*>(up);
  f16* o = reinterpret_cast<f16*>(out);
  if (aligned16(gate) && aligned16(up) && aligned16(out)) {
    // One pass over the range: each thread owns UNROLL vectors of each input.
    constexpr int UNROLL = 2;
    const size_t nvec = n / 8;
    const size_t need =
        ((nvec > 0 ? nvec : 1) + kSwigluThreads * UNROLL - 1) / (kSwigluThreads * UNROLL);
    if (need > 0x7FFFFFFFu) return LLMK_ERR_UNSUPPORTED;  // > 2^40 elements
    const unsigned blocks = (unsigned)need;
    return launch(k_swiglu_vec<UNROLL>, dim3(blocks), dim3(kSwigluThreads), 0, s, g, u, o, nvec,
                  n);
  }
  const unsigned blocks = ceil_div(n, 256) < 8192u ? ceil_div(n, 256) : 8192u;
  return launch(k_swiglu_scalar, dim3(blocks), dim3(256), 0, s, g, u, o, n);
}
