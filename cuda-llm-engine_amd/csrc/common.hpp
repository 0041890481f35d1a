// Device-side building blocks shared by every kernel in libllmk: fp16 vector types, 16-byte
// global accesses, wave64 reductions, and the launch helper that turns a kernel launch into a
// status code for the C-ABI.
//
// Arithmetic conventions (they are what make the results reproducible on the CPU):
//  * All code is built with -ffp-contract=off: no multiply-add contraction anywhere, so every
//    fp32 product and sum is rounded on its own, exactly as the scalar restatement does it.
//  * fp32 -> fp16 conversion is v_cvt_f16_f32 under the default round-to-nearest-even mode.
//  * An fp32 add, subtract or multiply of two fp16 values followed by rounding to fp16 gives
//    the same bits as the native fp16 operation (binary32 carries 24 >= 2*11 + 2 significand
//    bits, so the double rounding is innocuous). The kernels therefore use packed fp16 math
//    (v_pk_add_f16 / v_pk_mul_f16) for those steps. fp16 denormals are kept (the default f16
//    denormal mode on gfx950), so this holds for subnormal inputs and results as well.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "llmk.h"

namespace llmk {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------------------------
// 16-byte global memory access. `stream` variants set the non-temporal hint for data that is
// touched exactly once (it must not displace the rows other waves still need).
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }
__device__ __forceinline__ u32x4 ld16_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void st16_stream(void* p, u32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

__device__ __forceinline__ f16x8 as_h8(u32x4 v) { return __builtin_bit_cast(f16x8, v); }
__device__ __forceinline__ u32x4 as_u4(f16x8 v) { return __builtin_bit_cast(u32x4, v); }

// Element k of a 4 x 32-bit vector as a scalar. Copy an element out this way before any
// __builtin_bit_cast: this compiler (ROCm 7.2 clang) lowers a bit_cast applied directly to a
// vector-element expression (v[k]) as a read of element 0, whatever k is.
__device__ __forceinline__ uint32_t elem(u32x4 v, int k) {
  const uint32_t e = v[k];
  return e;
}

// ---------------------------------------------------------------------------------------------
// wave64 reduction. The first four steps run on DPP lane permutes (no LDS traffic); after them
// every lane of each 16-lane row holds that row's sum, and the four row sums are combined as
// (r0 + r1) + (r2 + r3) from lanes 0, 16, 32, 48. Every lane returns the same value. Must be
// called with all 64 lanes active.
// ---------------------------------------------------------------------------------------------
// DPP lane permute for controls whose source lane always exists (quad_perm, row_half_mirror,
// row_mirror). Written as update_dpp with a zero `old` so that the compiler folds it into the
// consuming VALU instruction (v_add_f32_dpp) instead of emitting a separate v_mov_b32_dpp.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float readlane_f32(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
__device__ __forceinline__ float wave_sum(float v) {
  v = v + dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
  v = v + dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
  v = v + dpp_f32<0x141>(v);  // row_half_mirror: quads 0+1 and 2+3 of each row
  v = v + dpp_f32<0x140>(v);  // row_mirror: both halves of each 16-lane row
  const float r0 = readlane_f32(v, 0), r1 = readlane_f32(v, 16);
  const float r2 = readlane_f32(v, 32), r3 = readlane_f32(v, 48);
  return (r0 + r1) + (r2 + r3);
}

// ---------------------------------------------------------------------------------------------
// Launch helper: hipLaunchKernel returns the launch status directly, and a failed launch also
// leaves it in HIP's last-error state, as a reference-style caller expects.
// ---------------------------------------------------------------------------------------------
template <typename... Params, typename... Args>
inline int launch(void (*kernel)(Params...), dim3 grid, dim3 block, size_t shmem,
                  hipStream_t stream, Args... args) {
  static_assert(sizeof...(Params) == sizeof...(Args), "argument count mismatch");
  // Convert every argument to the exact parameter type before taking its address.
  auto call = [&](Params... p) -> int {
    void* argv[] = {reinterpret_cast<void*>(&p)..., nullptr};
    return (int)hipLaunchKernel(reinterpret_cast<const void*>(kernel), grid, block, argv, shmem,
                                stream);
  };
  return call(static_cast<Params>(args)...);
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---------------------------------------------------------------------------------------------
// Block barrier for LDS traffic only. __syncthreads() is a workgroup fence over every address
// space, for which the compiler waits for all of the wave's outstanding global loads and stores
// (s_waitcnt vmcnt(0)) before s_barrier; this one waits for the wave's LDS accesses alone, so
// global loads issued before it stay in flight across it. For barriers that order LDS accesses
// only.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

inline unsigned ceil_div(size_t a, size_t b) { return (unsigned)((a + b - 1) / b); }

// The current device's CU count, read once per device (0 if it cannot be read). Launch shapes
// that size a grid to one resident round of blocks use it.
inline int device_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  const int known = __atomic_load_n(&cache[dev], __ATOMIC_RELAXED);
  if (known > 0) return known;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    return 0;
  __atomic_store_n(&cache[dev], cus, __ATOMIC_RELAXED);
  return cus;
}

}  // namespace llmk
