// SwiGLU: out[i] = fp16(r16(silu(g)) * u) with silu(g) = g / (1 + exp(-g)) in fp32.
// ref: kernels/swiglu.cu:4-21. silu is rounded to fp16 before the multiply (ref:
// kernels/swiglu.cu:12); the product of two fp16 values rounded to fp16 is one packed fp16
// multiply. exp is the full-accuracy device expf, the quotient a correctly rounded fp32 divide.
//
// Gate and up are streamed once, in 16-byte vectors, UNROLL vectors of each per thread per
// step so that 2 * UNROLL loads are in flight before the first use.
#include "common.hpp"

namespace llmk {

__device__ __forceinline__ f16 silu_r16(f16 gh) {
  const float g = (float)gh;
  return (f16)(g / (1.0f + expf(-g)));
}

template <int UNROLL>
__global__ void __launch_bounds__(256)
k_swiglu_vec(const f16* __restrict__ gate, const f16* __restrict__ up, f16* __restrict__ out,
             size_t nvec, size_t n) {
  const size_t chunk = (size_t)blockDim.x * UNROLL;
  for (size_t b = (size_t)blockIdx.x * chunk; b < nvec; b += (size_t)gridDim.x * chunk) {
    f16x8 g[UNROLL], u[UNROLL];
#pragma unroll
    for (int m = 0; m < UNROLL; ++m) {
      const size_t i = b + threadIdx.x + (size_t)m * blockDim.x;
      if (i < nvec) {
        g[m] = as_h8(ld16_stream(gate + 8 * i));
        u[m] = as_h8(ld16_stream(up + 8 * i));
      }
    }
#pragma unroll
    for (int m = 0; m < UNROLL; ++m) {
      const size_t i = b + threadIdx.x + (size_t)m * blockDim.x;
      if (i < nvec) {
        f16x8 s;
#pragma unroll
        for (int j = 0; j < 8; ++j) s[j] = silu_r16(g[m][j]);
        st16_stream(out + 8 * i, as_u4(s * u[m]));
      }
    }
  }
  const size_t t = nvec * 8 + (size_t)blockIdx.x * blockDim.x + threadIdx.x;  // n % 8 tail
  if (t < n) out[t] = silu_r16(gate[t]) * up[t];
}

__global__ void __launch_bounds__(256)
k_swiglu_scalar(const f16* __restrict__ gate, const f16* __restrict__ up, f16* __restrict__ out,
                size_t n) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    out[i] = silu_r16(gate[i]) * up[i];
}

}  // namespace llmk

using namespace llmk;

extern "C" int llmk_swiglu(const uint16_t* gate, const uint16_t* up, uint16_t* out, size_t n,
                           void* stream) {
  if (n == 0) return LLMK_OK;
  if (!gate || !up || !out) return LLMK_ERR_INVALID_VALUE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const f16* g = reinterpret_cast<const f16*>(gate);
  const f16* u = reinterpret_cast<const f16*>(up);
  f16* o = reinterpret_cast<f16*>(out);
  if (aligned16(gate) && aligned16(up) && aligned16(out)) {
    constexpr int UNROLL = 2;
    const size_t nvec = n / 8;
    const size_t need = ceil_div(nvec > 0 ? nvec : 1, 256 * UNROLL);
    const unsigned blocks = need < 8192 ? (unsigned)need : 8192u;
    return launch(k_swiglu_vec<UNROLL>, dim3(blocks), dim3(256), 0, s, g, u, o, nvec, n);
  }
  const unsigned blocks = ceil_div(n, 256) < 8192u ? ceil_div(n, 256) : 8192u;
  return launch(k_swiglu_scalar, dim3(blocks), dim3(256), 0, s, g, u, o, n);
}
