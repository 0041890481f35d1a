// Residual add, RMSNorm and the fused residual add + RMSNorm for gfx950.
//
// Semantics follow the reference launchers (ref: kernels/residual_add.cu:5-18,
// kernels/rmsnorm.cu:9-68); the fused kernel equals residual_add followed by rmsnorm on the
// updated residual (ref: engine/batched.cu:64->66).
//
// Layout and mapping: rows of `hidden` fp16 values, row-major and contiguous. One wave64 owns
// one row: lane l holds the 16-byte vectors l, l+64, l+128, ... of the row in registers (for
// hidden = 2048 that is 4 vectors per tensor per lane, each load instruction covering 1 KiB of
// consecutive memory). The row is read from HBM exactly once; the sum of squares is reduced
// across the wave with DPP permutes, so no LDS and no barrier is involved. Row data is streamed
// with the non-temporal hint (loads and stores): each byte is touched once, and keeping it out
// of the normal cache-allocation path measured 9% faster at [8192, 2048] than plain accesses. Rows wider than
// 64 * 8 * 16 = 8192 values take a block-per-row kernel that reads the row twice (the second
// time from L2).
#include "layer_ops.hpp"

namespace llmk {

// ----------------------------------------------------------------------------------------------
// residual_add: out = fp16(a + b). Packed fp16 add == fp32 add then RNE rounding (see common.hpp).
// ----------------------------------------------------------------------------------------------
// One 16-byte vector per lane in one-wave blocks, one pass over the data: waves start, wait and
// finish on their own, as in the SwiGLU kernel. Same box, in place at [8192, 2048]: 17.2 us with
// 256-thread blocks in a grid-stride loop, 17.0 with 128- or 512-thread blocks, 16.5 here.
__global__ void __launch_bounds__(64)
k_residual_add_vec(const f16* a, const f16* b, f16* out, size_t nvec, size_t n) {
  const size_t i = (size_t)blockIdx.x * 64 + threadIdx.x;
  if (i < nvec) {
    const f16x8 va = as_h8(ld16_stream(a + 8 * i));
    const f16x8 vb = as_h8(ld16_stream(b + 8 * i));
    st16_stream(out + 8 * i, as_u4(va + vb));
  }
  const size_t t = nvec * 8 + i;  // the n % 8 trailing values
  if (t < n) out[t] = a[t] + b[t];
}

// Any-alignment path: one fp16 value per thread per step.
__global__ void __launch_bounds__(256)
k_residual_add_scalar(const f16* a, const f16* b, f16* out, size_t n) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    out[i] = a[i] + b[i];
}

// ----------------------------------------------------------------------------------------------
// RMSNorm, one wave per row (the row body is layer_ops.hpp's rmsnorm_row). VPL = 16-byte
// vectors per lane per tensor. FUSED: resid <- fp16(resid + x) first, and the norm is taken of
// the updated resid. FULL: vpr == 64 * VPL, every lane owns exactly VPL vectors.
// ----------------------------------------------------------------------------------------------
template <int VPL, bool FUSED, bool FULL>
__global__ void __launch_bounds__(256)
k_rmsnorm_wave(const f16* x, f16* resid, const f16* __restrict__ w, f16* out, int n_rows,
               int vpr, float hidden_f, float eps, int wpb) {
  // wpb (waves per block) is an argument, not blockDim: the arguments arrive preloaded in
  // SGPRs, blockDim would cost a scalar fetch before the first address is known.
  const int row = blockIdx.x * wpb + (threadIdx.x >> 6);
  if (row >= n_rows) return;  // uniform per wave
  const size_t base = (size_t)row * vpr * 8;
  rmsnorm_row<VPL, FUSED, FULL>(x + base, FUSED ? resid + base : nullptr,
                                FUSED ? resid + base : nullptr, w, out + base, vpr, hidden_f,
                                eps, threadIdx.x & 63);
}

// RMSNorm of 2048-wide rows, R rows per wave (waves of 4 per block). Wave w of the grid's
// `stride` waves takes rows w, w + stride, ..., w + (R - 1) * stride; it issues every load of
// its R rows (R x 4 vectors per lane, twice that FUSED) before the first row's sum, so load
// instruction r of all waves covers one contiguous band of `stride` rows. Each row then goes
// through rmsnorm_row's arithmetic (the residual add, norm_store), so the bits are those of
// k_rmsnorm_wave. Rows past n_rows load the last row again and store nothing.
template <int R, bool FUSED>
__global__ void __launch_bounds__(256)
k_rmsnorm_rows(const f16* x, f16* resid, const f16* __restrict__ w, f16* out, int n_rows,
               int stride, float hidden_f, float eps) {
  constexpr int VPL = 4, VPR = 64 * VPL;
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  f16x8 wv[VPL];
#pragma unroll
  for (int k = 0; k < VPL; ++k) wv[k] = as_h8(ld16(w + 8 * (lane + 64 * k)));
  f16x8 h[R][VPL], xv[FUSED ? R : 1][VPL];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = min(wave + r * stride, n_rows - 1);
    const size_t base = (size_t)row * VPR * 8;
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      h[r][k] = as_h8(ld16_stream((FUSED ? resid : x) + base + 8 * (lane + 64 * k)));
      if (FUSED) xv[FUSED ? r : 0][k] = as_h8(ld16_stream(x + base + 8 * (lane + 64 * k)));
    }
  }
  // Keep the compiler from sinking loads below the first row's arithmetic and stores: the
  // point is to have all of them in flight at once.
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = wave + r * stride;
    if (row < n_rows) {
      const size_t base = (size_t)row * VPR * 8;
      if (FUSED) {
#pragma unroll
        for (int k = 0; k < VPL; ++k) {
          h[r][k] = h[r][k] + xv[FUSED ? r : 0][k];
          st16_stream(resid + base + 8 * (lane + 64 * k), as_u4(h[r][k]));
        }
      }
      norm_store<VPL, true>(h[r], wv, out + base, VPR, hidden_f, eps, lane);
    }
  }
}

// Rows per wave for k_rmsnorm_rows, or 0 for the one-row kernel: the grid must fit one resident
// round of 4 waves per CU, so rows <= R * 4 * CUs, and the batch must be large enough to fill
// it. Same box, 2048-wide rows, us (one row per wave -> R rows per wave):
//   RMSNorm, R = 8: 6144 rows 10.08 -> 9.60, 7168 11.34 -> 10.13, 8192 12.68 -> 10.82; 5120
//     8.38 -> 9.07 and R = 4 at 3072-4096 rows (5.34 -> 6.75, 6.45 -> 6.79) lose.
//   add + RMSNorm, R = 4: 3072 rows 9.62 -> 8.62, 4096 12.00 -> 10.94; R = 8: 5120 14.70 ->
//     13.84, 6144 17.38 -> 15.90, 7168 20.18 -> 18.55, 8192 22.76 -> 21.23.
//   Past one round (9216, 12288, 16384 rows) both lose or tie; so does R = 16 (VGPR spills).
// The gain is in dispatch: one wave per row is 2048 4-wave blocks at 8192 rows against 256 here.
static int rmsnorm_rows_per_wave(int n_rows, bool fused) {
  const long long slots = 4LL * device_cus();
  if (slots <= 0) return 0;
  if (fused) {
    if (n_rows > 2 * slots && n_rows <= 4 * slots) return 4;
    if (n_rows > 4 * slots && n_rows <= 8 * slots) return 8;
    return 0;
  }
  return n_rows > 5 * slots && n_rows <= 8 * slots ? 8 : 0;
}

// Wide rows: one 256-thread block per row, two passes over the row.
template <bool FUSED>
__global__ void __launch_bounds__(256)
k_rmsnorm_block(const f16* x, f16* resid, const f16* __restrict__ w, f16* out, int vpr,
                float hidden_f, float eps) {
  __shared__ float part[4];
  const size_t base = (size_t)blockIdx.x * vpr * 8;
  float ss = 0.f;
  for (int v = threadIdx.x; v < vpr; v += 256) {
    f16x8 h = as_h8(ld16(x + base + 8 * v));
    if (FUSED) {
      h = as_h8(ld16(resid + base + 8 * v)) + h;
      st16(resid + base + 8 * v, as_u4(h));
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float f = (float)h[j];
      ss = ss + f * f;
    }
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float total = (part[0] + part[1]) + (part[2] + part[3]);
  const float inv = 1.0f / __builtin_sqrtf(total / hidden_f + eps);
  // Each thread re-reads exactly the vectors it wrote above, so its own stores are visible.
  const f16* src = FUSED ? resid : x;
  for (int v = threadIdx.x; v < vpr; v += 256) {
    const f16x8 h = as_h8(ld16(src + base + 8 * v));
    const f16x8 wv = as_h8(ld16(w + 8 * v));
    f16x8 a;
#pragma unroll
    for (int j = 0; j < 8; ++j) a[j] = (f16)((float)h[j] * inv);
    st16(out + base + 8 * v, as_u4(wv * a));
  }
}

template <bool FUSED>
static int rmsnorm_launch(const f16* x, f16* resid, const f16* w, f16* out, int n_rows,
                          int hidden, float eps, hipStream_t stream) {
  const int vpr = hidden / 8;
  const float hf = (float)hidden;
  const int vpl = (vpr + 63) / 64;
  if (vpr == 256) {
    const int R = rmsnorm_rows_per_wave(n_rows, FUSED);
    if (R > 0) {
      const int blocks = (int)ceil_div(ceil_div((size_t)n_rows, (size_t)R), 4);
      auto go = [&](auto kern) {
        return launch(kern, dim3(blocks), dim3(256), 0, stream, x, resid, w, out, n_rows,
                      4 * blocks, hf, eps);
      };
      return R == 4 ? go(k_rmsnorm_rows<4, FUSED>) : go(k_rmsnorm_rows<8, FUSED>);
    }
  }
  // Few rows: one wave per block so the rows spread over as many CUs as possible.
  const int wpb = n_rows >= 4096 ? 4 : 1;
  const dim3 grid(ceil_div((size_t)n_rows, (size_t)wpb)), block(64 * wpb);
#define LLMK_NORM_CASE(V)                                                                     \
  return vpr == 64 * V ? launch(k_rmsnorm_wave<V, FUSED, true>, grid, block, 0, stream, x, resid, \
                                w, out, n_rows, vpr, hf, eps, wpb)                               \
                       : launch(k_rmsnorm_wave<V, FUSED, false>, grid, block, 0, stream, x,      \
                                resid, w, out, n_rows, vpr, hf, eps, wpb)
  if (vpl <= 1) LLMK_NORM_CASE(1);
  if (vpl <= 2) LLMK_NORM_CASE(2);
  if (vpl <= 4) LLMK_NORM_CASE(4);
  if (vpl <= 8) LLMK_NORM_CASE(8);
  if (vpl <= 16) LLMK_NORM_CASE(16);
#undef LLMK_NORM_CASE
  return launch(k_rmsnorm_block<FUSED>, dim3(n_rows), dim3(256), 0, stream, x, resid, w, out,
                vpr, hf, eps);
}

}  // namespace llmk

using namespace llmk;

extern "C" int llmk_residual_add(const uint16_t* a, const uint16_t* b, uint16_t* out, size_t n,
                                 void* stream) {
  if (n == 0) return LLMK_OK;
  if (!a || !b || !out) return LLMK_ERR_INVALID_VALUE;
  const f16* pa = reinterpret_cast<const f16*>(a);
  const f16* pb = reinterpret_cast<const f16*>(b);
  f16* po = reinterpret_cast<f16*>(out);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t nvec = n / 8;
  const size_t need = nvec > 0 ? nvec : 1;  // the tail of fewer than 8 values takes one block
  if (aligned16(a) && aligned16(b) && aligned16(out) && need / 64 < 0x7FFFFFFFu)
    return launch(k_residual_add_vec, dim3(ceil_div(need, 64)), dim3(64), 0, s, pa, pb, po,
                  nvec, n);
  const unsigned blocks = ceil_div(n, 256) < 8192u ? ceil_div(n, 256) : 8192u;
  return launch(k_residual_add_scalar, dim3(blocks), dim3(256), 0, s, pa, pb, po, n);
}

static int check_norm_args(const void* x, const void* w, const void* out, int n_rows,
                           int hidden) {
  if (n_rows < 0 || hidden <= 0) return LLMK_ERR_INVALID_VALUE;
  if (n_rows == 0) return LLMK_OK;
  if (!x || !w || !out) return LLMK_ERR_INVALID_VALUE;
  if (hidden % 8 != 0) return LLMK_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(w) || !aligned16(out)) return LLMK_ERR_ALIGNMENT;
  return -1;  // arguments fine, proceed
}

extern "C" int llmk_rmsnorm(const uint16_t* x, const uint16_t* w, uint16_t* out, int n_rows,
                            int hidden, float eps, void* stream) {
  const int st = check_norm_args(x, w, out, n_rows, hidden);
  if (st != -1) return st;
  return rmsnorm_launch<false>(reinterpret_cast<const f16*>(x), nullptr,
                               reinterpret_cast<const f16*>(w), reinterpret_cast<f16*>(out),
                               n_rows, hidden, eps, static_cast<hipStream_t>(stream));
}

extern "C" int llmk_add_rmsnorm(uint16_t* residual, const uint16_t* x, const uint16_t* w,
                                uint16_t* out, int n_rows, int hidden, float eps, void* stream) {
  int st = check_norm_args(x, w, out, n_rows, hidden);
  if (st != -1) return st;
  if (!residual) return LLMK_ERR_INVALID_VALUE;
  if (!aligned16(residual)) return LLMK_ERR_ALIGNMENT;
  return rmsnorm_launch<true>(reinterpret_cast<const f16*>(x), reinterpret_cast<f16*>(residual),
                              reinterpret_cast<const f16*>(w), reinterpret_cast<f16*>(out),
                              n_rows, hidden, eps, static_cast<hipStream_t>(stream));
}
