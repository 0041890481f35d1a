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
// Gate and up are streamed once, in 16-byte vectors, UNROLL vectors of each per thread, all
// loads issued before the first use.
#include "layer_ops.hpp"

namespace llmk {

// The grid covers the whole range in one pass, one block per chunk of kSwigluThreads * UNROLL
// vectors (layer_ops.hpp: swiglu_block, and the launch shape measured for it). Blocks wholly
// inside the range take a straight-line path without per-vector tests; only the last block
// tests. (A grid-stride loop around the same body measured 10% slower at [8192, 8192].)
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
  constexpr int UNROLL = kSwigluUnroll;
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
    constexpr int UNROLL = kSwigluUnroll;
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
