// The projections of a decode step with few rows: y[T, out] = x[T, in] * W^T, W stored [out, in]
// row-major (a PyTorch Linear without bias), fp16 in and out, fp32 accumulation, for T <= 8.
// ref: kernels/linear.cu:5-25 (cublasGemmEx with CUBLAS_COMPUTE_32F), the reference's only GEMM,
// which the engine calls for every projection whatever the batch size.
//
// With T <= 8 rows a projection does at most 16 flops per weight byte, far below MI355X's ~300
// flop/byte balance point, so it is a stream over W: the design goal is to keep HBM busy.
//   - A block owns kRows = 8 output rows. The in dimension is cut into steps of 512 (64 lanes x
//     8 halves), and the block's WV waves (1 to 16: one step each where the registers allow)
//     take steps w, w + WV, ... For each step a wave issues one 16-byte load per W row (64 lanes
//     cover 1 KiB of the row, fully coalesced) and one per x row (x is small and stays in the
//     L2), then accumulates the 8 x T partial dot products of its lane in fp32 with
//     v_dot2_f32_f16.
//   - Fused variants (the entry points at the end) normalise x on the fly and replace the store
//     with the residual add, SwiGLU, or RoPE + KV scatter of the decode step.
//   - The 8 * TP partial sums of a lane are then reduced over the wave in a halving butterfly:
//     at each exchange a lane keeps half of its values and adds its partner's copy of them, so
//     the 64 lanes end up holding distinct (row, token) sums after 63 adds (mostly DPP) instead
//     of 8 * TP full reductions. The value index is token-major (t * 8 + r), so the exchanges
//     that pair tokens come first and run row by row, right after the row's dot products: a
//     lane holds the TP sums of one row and 8 per-row shares, not 8 * TP sums (at T = 8: 91
//     VGPRs, 5 waves per SIMD, against 130 and 3). The waves' sums meet in LDS.
//   - A normalising launch stages each wave's raw x slice in LDS once; the norms are taken from
//     there instead of every wave re-reading whole rows.
// Summation order differs from cuBLAS/hipBLASLt (lane-strided partial sums, then the butterfly),
// so results agree with the fp32 dot product to fp32 rounding, not bit for bit.
#include "common.hpp"
#include "pointwise.hpp"

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

template <int N, int S, int M>
__device__ __forceinline__ void butterfly(float (&v)[M]) {
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

// The halving exchanges S, S + 1, ... of the butterfly on v[0 .. N) until one value is left
// (no full adds): v[0] then holds the lane's share.
template <int N, int S, int M>
__device__ __forceinline__ void halve(float (&v)[M]) {
  if constexpr (N > 1) {
    const bool up = (threadIdx.x & kMask[S]) != 0;
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      const float send = up ? v[i] : v[i + N / 2];
      const float keep = up ? v[i + N / 2] : v[i];
      v[i] = keep + partner<S>(send);
    }
    halve<N / 2, S + 1>(v);
  }
}

template <int N>
constexpr int log2c() { return N <= 1 ? 0 : 1 + log2c<N / 2>(); }

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

// What a launch computes besides the plain product. See the entry points at the end of the file.
enum Epi : int {
  kEpiStore = 0,     // y[t][j] = r16(sum)
  kEpiResidual = 1,  // y[t][j] = r16(y[t][j] + r16(sum)), in place (the residual add)
  kEpiSwiglu = 2,    // rows j (gate) and inter + j (up) -> y[t][j] = r16(r16(silu(g)) * u)
  kEpiRope = 3,      // rows of q, k, v heads: RoPE on q and k, k and v into the paged pools
};

struct RowsArgs {
  const f16* x;       // [T, in]; with norm_w, the rows are normalised first (RMSNorm)
  const f16* w;       // [out, in] row-major
  f16* y;             // see Epi
  int T, in, out;
  const f16* norm_w;  // [in] or null
  float eps;
  // kEpiRope: out = (n_heads + 2 n_kv_heads) * 64 rows: q heads, k heads, v heads
  f16* q_out;         // [T, n_heads, 64]
  f16* k_pool;        // [num_pages * 16, n_kv_heads * 64]
  f16* v_pool;
  const int* tables;  // [T, max_pages]
  const int* positions;
  const float* inv_freq;  // [32]
  int n_heads, n_kv_heads, max_pages;
};

// Output row r (0..7) of block b. The swiglu and rope blocks take pairs: rows r and r + 4 are a
// (gate, up) pair of the same column, or the two halves (i, i + 32) of a rotation pair.
template <int EPI>
__device__ __forceinline__ int row_of(int b, int r, const RowsArgs& a) {
  if constexpr (EPI == kEpiSwiglu) {
    const int j = 4 * b + (r & 3);
    return r < 4 ? j : a.out / 2 + j;
  } else if constexpr (EPI == kEpiRope) {
    const int h = b >> 3, i = 4 * (b & 7) + (r & 3);
    return h * 64 + (r < 4 ? i : 32 + i);
  } else {
    const int j = b * kRows + r;
    return j < a.out ? j : a.out - 1;  // rows past `out`: computed, not stored
  }
}

// TP: rows computed (a power of two >= T; rows t >= T reuse row T - 1 and are not stored).
// WV: waves per block, dividing the in dimension's steps between them.
// NORM: x is RMSNorm-ed on the fly; the launcher then gives every wave exactly one step
// (steps == WV). Each row's sum of squares is taken exactly as the RMSNorm kernel takes it
// (k_rmsnorm_wave: lane l sums elements 8 (l + 64 k) + j, k then j in order, then wave_sum), by
// wave t % WV, so the normalised values are the RMSNorm kernel's bits.
template <int TP, int WV, int EPI, bool NORM>
__global__ void __launch_bounds__(64 * WV) k_rows(RowsArgs a) {
  constexpr int N = kRows * TP;  // partial sums per lane: value index r * TP + t
  __shared__ float part[WV][N];
  __shared__ float inv_s[TP];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = blockIdx.x;
  const int in = a.in, T = a.T;
  const int steps = in / kStep;

  // Token-major value index t * 8 + r: the butterfly's first log2(TP) halvings pair tokens of
  // one row, so they run row by row right after its dot products, and only the row's TP sums
  // and the 8 per-row shares are live.
  constexpr int LT = log2c<TP>();
  float red[kRows];
#pragma unroll
  for (int r = 0; r < kRows; ++r) red[r] = 0.0f;
  auto rows_dot = [&](const u32x4 (&wv)[kRows], const u32x4 (&xv)[TP]) {
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      float acc[TP];
#pragma unroll
      for (int t = 0; t < TP; ++t) acc[t] = dot8(wv[r], xv[t], 0.0f);
      halve<TP, 0>(acc);
      red[r] = red[r] + acc[0];
    }
  };
  const f16* wr[kRows];
#pragma unroll
  for (int r = 0; r < kRows; ++r) wr[r] = a.w + (size_t)row_of<EPI>(b, r, a) * in + lane * 8;
  const f16* xr[TP];
#pragma unroll
  for (int t = 0; t < TP; ++t) xr[t] = a.x + (size_t)(t < T ? t : T - 1) * in + lane * 8;

  if constexpr (NORM) {
    // Every wave loads its step of all TP rows (x first: the norms wait only for those) and
    // leaves the raw slices in LDS; wave t % WV then sums the squares of row t from there, in
    // the RMSNorm kernel's order.
    __shared__ u32x4 xs[TP][WV][64];
    const size_t k0 = (size_t)wave * kStep;  // this wave's one step
    u32x4 wv[kRows], xv[TP];
#pragma unroll
    for (int t = 0; t < TP; ++t) xv[t] = ld16(xr[t] + k0);
    const u32x4 nw = ld16(a.norm_w + k0 + lane * 8);
#pragma unroll
    for (int r = 0; r < kRows; ++r) wv[r] = ld16_stream(wr[r] + k0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < TP; ++t) xs[t][wave][lane] = xv[t];
    __syncthreads();
    constexpr int NQ = (TP + WV - 1) / WV;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int t = wave + WV * q;
      if (t < TP) {
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < WV; ++k) {
          const f16x8 h = as_h8(xs[t][k][lane]);
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float f = (float)h[j];
            ss = ss + f * f;
          }
        }
        ss = wave_sum(ss);
        if (lane == 0) inv_s[t] = 1.0f / __builtin_sqrtf(ss / (float)in + a.eps);
      }
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < TP; ++t) {
      const f16x8 h = as_h8(xv[t]);
      const float inv = inv_s[t];
      f16x8 an;
#pragma unroll
      for (int j = 0; j < 8; ++j) an[j] = (f16)((float)h[j] * inv);
      xv[t] = as_u4(as_h8(nw) * an);
    }
    rows_dot(wv, xv);
  } else {
    for (int s = wave; s < steps; s += WV) {
      const size_t k = (size_t)s * kStep;
      u32x4 wv[kRows], xv[TP];
#pragma unroll
      for (int r = 0; r < kRows; ++r) wv[r] = ld16_stream(wr[r] + k);
#pragma unroll
      for (int t = 0; t < TP; ++t) xv[t] = ld16(xr[t] + k);
      // Every load of the step is in flight before the first product (left alone, the
      // scheduler reuses one register for the W rows and waits for each load in turn).
      __builtin_amdgcn_sched_barrier(0);
      rows_dot(wv, xv);
    }
  }

  butterfly<kRows, LT>(red);
  bool writer;
  const int tidx = butterfly_index<N>(lane, &writer);  // t * 8 + r
  const int idx = (tidx % kRows) * TP + tidx / kRows;  // the epilogue's r * TP + t
  const float* v = red;
  if (writer) part[wave][idx] = v[0];
  __syncthreads();
  auto total = [&](int i) {
    float sum = 0.0f;
#pragma unroll
    for (int q = 0; q < WV; ++q) sum += part[q][i];
    return sum;
  };
  const int tid = threadIdx.x;
  if constexpr (EPI == kEpiStore || EPI == kEpiResidual) {
    if (tid < N) {
      const int r = tid / TP, t = tid % TP, j = b * kRows + r;
      if (j < a.out && t < T) {
        const f16 p = (f16)total(tid);
        f16* dst = a.y + (size_t)t * a.out + j;
        *dst = EPI == kEpiStore ? p : (f16)((float)*dst + (float)p);
      }
    }
  } else if (tid < 4 * TP) {
    const int r = tid / TP, t = tid % TP;  // the pair (r, r + 4) of token t
    if (t < T) {
      const f16 lo = (f16)total(tid), hi = (f16)total(tid + 4 * TP);
      if constexpr (EPI == kEpiSwiglu) {
        const int inter = a.out / 2, j = 4 * b + r;
        a.y[(size_t)t * inter + j] = silu_r16(lo) * hi;
      } else {
        const int h = b >> 3, i = 4 * (b & 7) + r, nq = a.n_heads, nkv = a.n_kv_heads;
        const int pos = a.positions[t];
        f16 x1 = lo, x2 = hi;
        if (h < nq + nkv) {
          f16 c, sn;
          cos_sin_f16((float)pos * a.inv_freq[i], &c, &sn);
          x1 = lo * c - hi * sn;
          x2 = hi * c + lo * sn;
        }
        f16* dst;
        if (h < nq) {
          dst = a.q_out + ((size_t)t * nq + h) * 64;
        } else {
          const size_t prow = (size_t)a.tables[(size_t)t * a.max_pages + pos / 16] * 16 + pos % 16;
          const int hk = h < nq + nkv ? h - nq : h - nq - nkv;
          dst = (h < nq + nkv ? a.k_pool : a.v_pool) + prow * nkv * 64 + hk * 64;
        }
        dst[i] = x1;
        dst[i + 32] = x2;
      }
    }
  }
}

// Waves per block: one per step of the in dimension, up to 16. A normalising launch needs
// exactly one step per wave, so steps must be 1, 2, 4, 8 or 16; 0 otherwise.
template <int TP>
int rows_waves(int steps, bool norm) {
  const int cap = 16;
  if (norm) {
    const bool pow2 = (steps & (steps - 1)) == 0;
    return steps >= 1 && steps <= cap && pow2 ? steps : 0;
  }
  return steps <= 1 ? 1 : steps <= 2 ? 2 : steps <= 4 ? 4 : steps <= 8 ? 8 : cap;
}

template <int TP, int EPI, bool NORM>
int rows_launch_tp(const RowsArgs& a, unsigned blocks, hipStream_t s) {
  const int wv = rows_waves<TP>(a.in / kStep, NORM);
  switch (wv) {
    case 1: return launch(k_rows<TP, 1, EPI, NORM>, dim3(blocks), dim3(64), 0, s, a);
    case 2: return launch(k_rows<TP, 2, EPI, NORM>, dim3(blocks), dim3(128), 0, s, a);
    case 4: return launch(k_rows<TP, 4, EPI, NORM>, dim3(blocks), dim3(256), 0, s, a);
    case 8: return launch(k_rows<TP, 8, EPI, NORM>, dim3(blocks), dim3(512), 0, s, a);
    case 16:
      return launch(k_rows<TP, 16, EPI, NORM>, dim3(blocks), dim3(1024), 0, s, a);
    default: return LLMK_ERR_UNSUPPORTED;
  }
}

template <int EPI, bool NORM>
int rows_launch(const RowsArgs& a, unsigned blocks, hipStream_t s) {
  if (a.T == 1) return rows_launch_tp<1, EPI, NORM>(a, blocks, s);
  if (a.T == 2) return rows_launch_tp<2, EPI, NORM>(a, blocks, s);
  if (a.T <= 4) return rows_launch_tp<4, EPI, NORM>(a, blocks, s);
  return rows_launch_tp<8, EPI, NORM>(a, blocks, s);
}

template <int EPI>
int rows_dispatch(const RowsArgs& a, unsigned blocks, hipStream_t s) {
  return a.norm_w ? rows_launch<EPI, true>(a, blocks, s) : rows_launch<EPI, false>(a, blocks, s);
}

// Checks shared by the entry points; fills the common fields.
int rows_common(RowsArgs* a, const uint16_t* x, const uint16_t* norm_w, float eps,
                const uint16_t* w, uint16_t* y, int T, int in, int out) {
  if (T < 0 || in <= 0 || out <= 0) return LLMK_ERR_INVALID_VALUE;
  if (T > 0 && (!x || !w || !y)) return LLMK_ERR_INVALID_VALUE;
  if (T > LLMK_LINEAR_ROWS_MAX || in % kStep != 0) return LLMK_ERR_UNSUPPORTED;
  if ((size_t)out > (size_t)0xFFFFFFFFu * kRows) return LLMK_ERR_UNSUPPORTED;
  if (norm_w) {
    const int steps = in / kStep;
    const int wv = rows_waves<8>(steps, true);
    if (wv == 0) return LLMK_ERR_UNSUPPORTED;
    if (!aligned16(norm_w)) return LLMK_ERR_ALIGNMENT;
  }
  if (T > 0 && (!aligned16(x) || !aligned16(w))) return LLMK_ERR_ALIGNMENT;
  *a = RowsArgs{};
  a->x = reinterpret_cast<const f16*>(x);
  a->w = reinterpret_cast<const f16*>(w);
  a->y = reinterpret_cast<f16*>(y);
  a->T = T;
  a->in = in;
  a->out = out;
  a->norm_w = reinterpret_cast<const f16*>(norm_w);
  a->eps = eps;
  return LLMK_OK;
}

}  // namespace
}  // namespace llmk

using namespace llmk;

extern "C" int llmk_linear_rows(const uint16_t* x, const uint16_t* w, uint16_t* y, int T,
                                int in_features, int out_features, void* stream) {
  return llmk_linear_rows_norm(x, nullptr, 0.0f, w, y, T, in_features, out_features, stream);
}

extern "C" int llmk_linear_rows_norm(const uint16_t* x, const uint16_t* norm_w, float eps,
                                     const uint16_t* w, uint16_t* y, int T, int in_features,
                                     int out_features, void* stream) {
  RowsArgs a;
  const int st = rows_common(&a, x, norm_w, eps, w, y, T, in_features, out_features);
  if (st != LLMK_OK || T == 0) return st;
  return rows_dispatch<kEpiStore>(a, ceil_div((size_t)out_features, kRows),
                                  static_cast<hipStream_t>(stream));
}

extern "C" int llmk_linear_rows_residual(const uint16_t* x, const uint16_t* w,
                                         uint16_t* residual, int T, int in_features,
                                         int out_features, void* stream) {
  RowsArgs a;
  const int st = rows_common(&a, x, nullptr, 0.0f, w, residual, T, in_features, out_features);
  if (st != LLMK_OK || T == 0) return st;
  return rows_dispatch<kEpiResidual>(a, ceil_div((size_t)out_features, kRows),
                                     static_cast<hipStream_t>(stream));
}

extern "C" int llmk_linear_rows_swiglu(const uint16_t* x, const uint16_t* norm_w, float eps,
                                       const uint16_t* w_gate_up, uint16_t* act, int T,
                                       int in_features, int inter, void* stream) {
  if (inter <= 0 || inter % 4 != 0) return inter <= 0 ? LLMK_ERR_INVALID_VALUE
                                                      : LLMK_ERR_UNSUPPORTED;
  RowsArgs a;
  const int st = rows_common(&a, x, norm_w, eps, w_gate_up, act, T, in_features, 2 * inter);
  if (st != LLMK_OK || T == 0) return st;
  return rows_dispatch<kEpiSwiglu>(a, (unsigned)(inter / 4), static_cast<hipStream_t>(stream));
}

extern "C" int llmk_linear_rows_qkv_rope_scatter(
    const uint16_t* x, const uint16_t* norm_w, float eps, const uint16_t* w_qkv,
    uint16_t* q_out, uint16_t* k_pool, uint16_t* v_pool, const int32_t* block_tables,
    const int32_t* positions, const float* inv_freq, int T, int in_features, int n_heads,
    int n_kv_heads, int max_pages, void* stream) {
  if (n_heads <= 0 || n_kv_heads <= 0 || max_pages <= 0) return LLMK_ERR_INVALID_VALUE;
  if (T > 0 && (!q_out || !k_pool || !v_pool || !block_tables || !positions || !inv_freq))
    return LLMK_ERR_INVALID_VALUE;
  RowsArgs a;
  const int out = (n_heads + 2 * n_kv_heads) * 64;
  const int st = rows_common(&a, x, norm_w, eps, w_qkv, q_out, T, in_features, out);
  if (st != LLMK_OK || T == 0) return st;
  a.q_out = reinterpret_cast<f16*>(q_out);
  a.k_pool = reinterpret_cast<f16*>(k_pool);
  a.v_pool = reinterpret_cast<f16*>(v_pool);
  a.tables = block_tables;
  a.positions = positions;
  a.inv_freq = inv_freq;
  a.n_heads = n_heads;
  a.n_kv_heads = n_kv_heads;
  a.max_pages = max_pages;
  return rows_dispatch<kEpiRope>(a, (unsigned)(out / kRows), static_cast<hipStream_t>(stream));
}
