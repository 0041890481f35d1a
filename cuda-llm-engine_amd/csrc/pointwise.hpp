// Element-wise device functions shared by the kernels that apply them: the RoPE (cos, sin) pair
// and the rounded silu. Each is the one place its numerics are defined, so a fused kernel
// produces the same bits as the stand-alone one.
#pragma once
#include <math.h>

#include "common.hpp"

namespace llmk {

// silu(g) = g / (1 + exp(-g)) in fp32, rounded to fp16 -- the reference's value with exp taken
// in fp64 and rounded to fp32 (the closest fp32 to the true exponential). Used for the few
// inputs the fast path below cannot settle.
__device__ __forceinline__ float silu_exact(float g) {
  const float e = (float)exp(-(double)g);
  return g / (1.0f + e);
}

// Fast path: exp from v_exp_f32 (2^x) on -g*log2(e), the quotient from v_rcp_f32 and one
// Newton correction. For g > -12.4 its result is within about 14 fp32 ulps of the exact one
// (argument rounding of -g*log2(e) contributes at most 11); below that silu(g) is under the
// smallest fp16 normal. The fp16 rounding of the fast value is therefore the same as that of
// the exact value whenever the fast value is a finite fp16-normal number more than kWin fp32
// ulps away from an fp16 rounding midpoint (low 13 bits 0x1000). Every other input -- near a
// midpoint (about 0.8% of them), tiny, or NaN when exp overflows -- is flagged for exact
// recomputation. silu depends on the 16-bit input only, and the tests check all 65536 of them.
constexpr uint32_t kWin = 32;

__device__ __forceinline__ float silu_fast(float g, bool* unsettled) {
  const float e = __builtin_amdgcn_exp2f(g * -1.44269504088896341f);
  const float d = 1.0f + e;
  const float r = __builtin_amdgcn_rcpf(d);
  const float q0 = g * r;
  const float q = __builtin_fmaf(__builtin_fmaf(-d, q0, g), r, q0);
  const uint32_t b = __builtin_bit_cast(uint32_t, q);
  *unsettled = (b & 0x1FFFu) - (0x1000u - kWin) <= 2 * kWin ||  // near an fp16 midpoint
               (b & 0x7FFFFFFFu) < 0x38800000u ||              // below the fp16 normal range
               (b & 0x7F800000u) == 0x7F800000u;               // inf or NaN
  return q;
}

__device__ __forceinline__ f16 silu_r16(f16 gh) {
  bool unsettled;
  const float q = silu_fast((float)gh, &unsettled);
  return (f16)(unsettled ? silu_exact((float)gh) : q);
}

// cos and sin of the fp32 angle `a`, rounded to fp16. They are evaluated in fp64 (OCML sincos,
// full-range argument reduction) and rounded fp64 -> fp32 -> fp16, so the fp16 values are the
// roundings of the fp32 roundings of the exact results except in vanishingly rare ties. The
// angles reach 131071 rad; an fp32 sincos with a last-bit error can move c or s by one fp16 ulp,
// and x1*c - x2*s then cancels to a value with a large relative error. Callers evaluate each
// (token, pair) once and share it across heads, which keeps the fp64 cost small.
__device__ __forceinline__ void cos_sin_f16(float a, f16* c, f16* s) {
  double sd, cd;
  sincos((double)a, &sd, &cd);
  const float cf = (float)cd, sf = (float)sd;
  *c = (f16)cf;
  *s = (f16)sf;
}

}  // namespace llmk
