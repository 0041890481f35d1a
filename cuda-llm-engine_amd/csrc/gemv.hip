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
//   - Launches of 5 to 8 rows of matrices of at most kMfmaMaxOut x kMfmaMaxIn run the same
//     blocks on the matrix cores instead (k_rows_mfma, v_mfma_f32_4x4x4_16b_f16;
//     rows_launch_tp says why), and those with many output rows at in = 2048 (gate/up, the
//     lm head) run 16-wave blocks that stage x once per 64 rows through direct-to-LDS loads
//     (k_rows_mfma_wide).
//   - A residual epilogue reads the value it adds to at the start of the kernel, not after the
//     products (0.25-0.3 us per launch on the o and down shapes at every row count).
// Summation order differs from cuBLAS/hipBLASLt (lane-strided partial sums, then the butterfly),
// so results agree with the fp32 dot product to fp32 rounding, not bit for bit.
#include <type_traits>

#include "common.hpp"
#include "pointwise.hpp"

namespace llmk {
namespace {

constexpr int kRows = 8;      // output rows per block
constexpr int kStep = 512;    // in elements per wave step: 64 lanes x 8 halves

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

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

// Threads of the epilogue of one row group: one per (row, token) for a plain or residual store,
// one per pair of rows (gate and up, or the two halves of a rotation) and token otherwise.
template <int EPI, int TPP>
constexpr int epi_threads() {
  return EPI == kEpiStore || EPI == kEpiResidual ? kRows * TPP : 4 * TPP;
}

// kEpiResidual: the residual value epilogue thread `tid` of row group b adds to. Read at the start
// of the kernel, so that this read is not a memory round trip after the products.
template <int EPI, int TPP>
__device__ __forceinline__ f16 epi_residual(const RowsArgs& a, int b, int tid) {
  if constexpr (EPI == kEpiResidual) {
    if (tid < kRows * TPP) {
      const int r = tid / TPP, t = tid % TPP, j = b * kRows + r;
      if (j < a.out && t < a.T) return a.y[(size_t)t * a.out + j];
    }
  }
  return (f16)0.0f;
}

// The epilogue of row group b (see Epi), by threads tid < epi_threads: part[wave][r * TPP + t]
// holds each wave's sum for output row r of the group (0..7) and token t (TPP >= T tokens
// computed); the waves' sums are added here. res: epi_residual's value for this thread.
template <int EPI, int TPP, int WV>
__device__ __forceinline__ void rows_epilogue(const RowsArgs& a, int b,
                                              const float (&part)[WV][kRows * TPP], int tid,
                                              f16 res) {
  const int T = a.T;
  auto total = [&](int i) {
    float sum = 0.0f;
#pragma unroll
    for (int q = 0; q < WV; ++q) sum += part[q][i];
    return sum;
  };
  if constexpr (EPI == kEpiStore || EPI == kEpiResidual) {
    if (tid < kRows * TPP) {
      const int r = tid / TPP, t = tid % TPP, j = b * kRows + r;
      if (j < a.out && t < T) {
        const f16 p = (f16)total(tid);
        f16* dst = a.y + (size_t)t * a.out + j;
        *dst = EPI == kEpiStore ? p : (f16)((float)res + (float)p);
      }
    }
  } else if (tid < 4 * TPP) {
    const int r = tid / TPP, t = tid % TPP;  // the pair (r, r + 4) of token t
    if (t < T) {
      const f16 lo = (f16)total(tid), hi = (f16)total(tid + 4 * TPP);
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
  const f16 res = epi_residual<EPI, TP>(a, b, threadIdx.x);

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
    lds_barrier();  // the W loads stay in flight through the norms
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
    lds_barrier();
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
  rows_epilogue<EPI, TP, WV>(a, b, part, threadIdx.x, res);
}

// ---------------------------------------------------------------------------------------------
// The same products on the matrix cores: v_mfma_f32_4x4x4_16b_f16 computes 16 independent
// 4 x 4 x 4 products; block q of the instruction is lanes 4q .. 4q + 3, lane 4q + i holding row i
// of its A (4 k values, 64 bits), lane 4q + j column j of its B and D[0..3][j] (checked on
// gfx950 with one-hot and index-coded operands). Here A is 4 tokens of x and B 4 rows of W, and
// the 16 blocks take 16 different slices of k, so a wave's 16-byte load of W covers 4 rows x
// 256 contiguous bytes (lane 4q + j: row j, k = 8q .. 8q + 7 of a 128-wide chunk) and four such
// loads the rows' 1 KiB of a step, the bytes the dot-product kernel loads; each 16-byte load
// feeds two instructions (k = 8q .. 8q + 3 and 8q + 4 .. 8q + 7). The block slices are summed
// once, after the last step, by a four-exchange butterfly over lane bits 2-5.
// ---------------------------------------------------------------------------------------------
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x4 mfma4(u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(h4, a), __builtin_bit_cast(h4, b),
                                           c, 0, 0, 0);
}
__device__ __forceinline__ u32x2 lo2(u32x4 v) { return u32x2{v[0], v[1]}; }
__device__ __forceinline__ u32x2 hi2(u32x4 v) { return u32x2{v[2], v[3]}; }

// The value lane (lane ^ M) holds, M = 4, 8 (DPP inside a 16-lane row) or 16, 32 (swizzle).
template <int M>
__device__ __forceinline__ float xpartner(float v) {
  if constexpr (M == 4 || M == 8) {
    const int x = __builtin_bit_cast(int, v);
    const int up = __builtin_amdgcn_mov_dpp(x, 0x110 + M, 0xF, 0xF, false);  // row_shr:M
    const int dn = __builtin_amdgcn_mov_dpp(x, 0x100 + M, 0xF, 0xF, false);  // row_shl:M
    return __builtin_bit_cast(float, (threadIdx.x & M) ? up : dn);
  } else {
    return __shfl_xor(v, M);
  }
}

// The 16 bytes of x (token quad p: tokens 4p .. 4p + 3) and of two W row quads (rq: rows 4rq ..
// 4rq + 3) at one k slice of the lane: two instructions per row quad, k = 8q .. 8q + 3 and
// 8q + 4 .. 8q + 7.
template <int TQ>
__device__ __forceinline__ void mfma_chunk(f32x4 (&acc)[TQ][2], const u32x4 (&wv)[2],
                                           const u32x4 (&xv)[TQ]) {
#pragma unroll
  for (int p = 0; p < TQ; ++p)
#pragma unroll
    for (int rq = 0; rq < 2; ++rq) {
      acc[p][rq] = mfma4(lo2(xv[p]), lo2(wv[rq]), acc[p][rq]);
      acc[p][rq] = mfma4(hi2(xv[p]), hi2(wv[rq]), acc[p][rq]);
    }
}

// Sums the 16 instruction blocks' slices of a wave's accumulators and stores the wave's sum of
// each (row, token) of its row group into part[r * TPP + t]: value index (p * 2 + rq) * 4 + v
// (token 4p + v, row 4rq + q4), halved over lane bits 2, 3, 4, 5 (masks 4, 8, 16, 32).
template <int TQ>
__device__ __forceinline__ void mfma_store_part(const f32x4 (&acc)[TQ][2], float* part) {
  constexpr int TPP = 4 * TQ;
  constexpr int NV = 8 * TQ;  // values per lane
  const int lane = threadIdx.x & 63;
  float v[NV];
#pragma unroll
  for (int p = 0; p < TQ; ++p)
#pragma unroll
    for (int rq = 0; rq < 2; ++rq)
#pragma unroll
      for (int e = 0; e < 4; ++e) v[(p * 2 + rq) * 4 + e] = acc[p][rq][e];
  auto exchange = [&](auto mtag, int n) {
    constexpr int M = decltype(mtag)::value;
    const bool up = (threadIdx.x & M) != 0;
    if (n > 1) {
#pragma unroll
      for (int i = 0; i < NV / 2; ++i) {
        if (i < n / 2) {
          const float send = up ? v[i] : v[i + n / 2];
          const float keep = up ? v[i + n / 2] : v[i];
          v[i] = keep + xpartner<M>(send);
        }
      }
    } else {
      v[0] = v[0] + xpartner<M>(v[0]);
    }
  };
  exchange(std::integral_constant<int, 4>{}, NV);
  exchange(std::integral_constant<int, 8>{}, NV / 2);
  exchange(std::integral_constant<int, 16>{}, NV / 4);
  exchange(std::integral_constant<int, 32>{}, NV / 8);
  // The lane's value index: bits from the top = lane bits 2, 3, 4, 5 of the halving exchanges
  // (NV = 16: all four halve; NV = 8: three halve, and only the lane with bit 5 clear writes).
  int idx = 0;
  bool writer = true;
  {
    int n = NV;
#pragma unroll
    for (int sb = 2; sb < 6; ++sb) {
      const int bit = (lane >> sb) & 1;
      if (n > 1) {
        idx = 2 * idx + bit;
        n /= 2;
      } else {
        writer = writer && bit == 0;
      }
    }
  }
  const int pr = idx >> 2, e = idx & 3;  // (p * 2 + rq), v
  const int t = 4 * (pr >> 1) + e, r = 4 * (pr & 1) + (lane & 3);
  if (writer) part[r * TPP + t] = v[0];
}

template <int TP, int WV, int EPI, bool NORM>
__global__ void __launch_bounds__(64 * WV) k_rows_mfma(RowsArgs a) {
  constexpr int TQ = TP <= 4 ? 1 : 2;  // token quads
  constexpr int TPP = 4 * TQ;          // tokens computed (rows >= T repeat row T - 1, unstored)
  __shared__ float part[WV][kRows * TPP];
  __shared__ float inv_s[TP];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = blockIdx.x;
  const int in = a.in, T = a.T;
  const int steps = in / kStep;
  const int qb = lane >> 2, q4 = lane & 3;  // the lane's instruction block and its row in it
  const f16 res = epi_residual<EPI, TPP>(a, b, threadIdx.x);

  f32x4 acc[TQ][2];
#pragma unroll
  for (int p = 0; p < TQ; ++p)
#pragma unroll
    for (int rq = 0; rq < 2; ++rq) acc[p][rq] = f32x4{0.f, 0.f, 0.f, 0.f};
  const f16* wr[2];
#pragma unroll
  for (int rq = 0; rq < 2; ++rq)
    wr[rq] = a.w + (size_t)row_of<EPI>(b, 4 * rq + q4, a) * in + 8 * qb;
  int tok[TQ];
#pragma unroll
  for (int p = 0; p < TQ; ++p) tok[p] = 4 * p + q4 < T ? 4 * p + q4 : T - 1;

  if constexpr (NORM) {
    // As in k_rows: every wave stages its step of the TP rows in LDS (the lane-strided layout
    // of the RMSNorm kernel), wave t % WV takes row t's sum of squares in that kernel's order,
    // and each lane then normalises the 16 bytes its instructions need, read back from LDS.
    __shared__ u32x4 xs[TP][WV][64];
    const size_t k0 = (size_t)wave * kStep;  // this wave's one step
    // x first, then the norm weights, then W: the waits for the first two leave W in flight
    // (memory waits are in issue order), and the barriers below order LDS accesses only.
    u32x4 xl[TP], wv[4][2], nw[4];
#pragma unroll
    for (int t = 0; t < TP; ++t)
      xl[t] = ld16(a.x + (size_t)(t < T ? t : T - 1) * in + k0 + lane * 8);
#pragma unroll
    for (int c = 0; c < 4; ++c) nw[c] = ld16(a.norm_w + k0 + 128 * c + 8 * qb);
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int rq = 0; rq < 2; ++rq) wv[c][rq] = ld16_stream(wr[rq] + k0 + 128 * c);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < TP; ++t) xs[t][wave][lane] = xl[t];
    lds_barrier();
    constexpr int NQ = (TP + WV - 1) / WV;
#pragma unroll
    for (int qq = 0; qq < NQ; ++qq) {
      const int t = wave + WV * qq;
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
    lds_barrier();
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      u32x4 xv[TQ];
#pragma unroll
      for (int p = 0; p < TQ; ++p) {
        const f16x8 h = as_h8(xs[tok[p]][wave][16 * c + qb]);
        const float inv = inv_s[tok[p]];
        f16x8 an;
#pragma unroll
        for (int j = 0; j < 8; ++j) an[j] = (f16)((float)h[j] * inv);
        xv[p] = as_u4(as_h8(nw[c]) * an);
      }
      mfma_chunk<TQ>(acc, wv[c], xv);
    }
  } else {
    const f16* xr[TQ];
#pragma unroll
    for (int p = 0; p < TQ; ++p) xr[p] = a.x + (size_t)tok[p] * in + 8 * qb;
    for (int s = wave; s < steps; s += WV) {
      const size_t k = (size_t)s * kStep;
      u32x4 wv[4][2], xv[4][TQ];
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int rq = 0; rq < 2; ++rq) wv[c][rq] = ld16_stream(wr[rq] + k + 128 * c);
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int p = 0; p < TQ; ++p) xv[c][p] = ld16(xr[p] + k + 128 * c);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int c = 0; c < 4; ++c) mfma_chunk<TQ>(acc, wv[c], xv[c]);
    }
  }

  mfma_store_part<TQ>(acc, part[wave]);
  __syncthreads();
  rows_epilogue<EPI, TPP, WV>(a, b, part, threadIdx.x, res);
}

// ---------------------------------------------------------------------------------------------
// 5 to 8 rows, many output rows (gate/up, the lm head): blocks of 16 waves, WV steps of the in
// dimension x RG row-group pairs, so that x is staged (and normalised, NORM) once per 16 * RG
// output rows rather than once per 8.
//   - The block's x rows (and the norm weights) go from memory straight into LDS
//     (global_load_lds_dwordx4: no registers held while they are in flight).
//   - Each wave streams 16 W rows (two row groups) of its step into registers: 16 KiB in flight
//     per wave, 256 KiB per CU with one block per CU, the one-row kernel's figure.
//   - NORM: wave t takes row t's sum of squares in the RMSNorm kernel's order and writes the
//     row back normalised, once per block. The products, the waves' sums and the epilogues are
//     those of k_rows_mfma: every output has k_rows_mfma's bits.
// The compiler cannot tell which outstanding loads an LDS read after global_load_lds depends on
// and waits for all of them (s_waitcnt vmcnt(0)) at an LDS fence, which would hold the barriers
// until every W load had landed. So each wave waits for exactly its own DMA loads (issued before
// its W loads; loads complete in issue order) and for its own LDS writes, and then crosses a plain
// s_barrier (dma_barrier).
// ---------------------------------------------------------------------------------------------
template <int VM, int LGKM>
__device__ __forceinline__ void wait_vm_lgkm() {  // s_waitcnt vmcnt(VM) lgkmcnt(LGKM), gfx9 fields
  static_assert(VM >= 0 && VM < 64 && LGKM >= 0 && LGKM < 16, "waitcnt field range");
  __builtin_amdgcn_s_waitcnt((VM & 15) | ((VM >> 4) << 14) | (7 << 4) | (LGKM << 8));
}
__device__ __forceinline__ void dma_barrier() {
  asm volatile("" ::: "memory");  // no LDS access moves across the barrier
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
typedef __attribute__((address_space(3))) void lds_void;
// 16 bytes per lane from `g` into LDS at `wave_base` + 16 * lane (wave_base is the wave's).
__device__ __forceinline__ void dma16(const void* g, void* wave_base) {
  __builtin_amdgcn_global_load_lds(g, (lds_void*)wave_base, 16, 0, 0);
}

template <int WV, int RG, int EPI, bool NORM>
__global__ void __launch_bounds__(64 * WV * RG, 1) k_rows_mfma_wide(RowsArgs a) {
  constexpr int TP = 8, TQ = 2, TPP = 8, G = 2;  // G: row groups per wave
  constexpr int NW = WV * RG;                     // waves per block
  constexpr int NWL = 4 * G * 2;                  // W loads per wave
  static_assert(NW <= 16 && NW >= TP, "one wave per row's sum of squares");
  static_assert(EPI != kEpiResidual, "the residual epilogue keeps the narrow kernels");
  __shared__ float part[RG * G][WV][kRows * TPP];
  __shared__ u32x4 xs[TP][WV][64];
  __shared__ u32x4 nws[WV][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int step = wave % WV, rg = wave / WV;
  const int in = a.in, T = a.T;
  const int qb = lane >> 2, q4 = lane & 3;
  const int g0 = (blockIdx.x * RG + rg) * G;  // the wave's first row group

  f32x4 acc[G][TQ][2];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int p = 0; p < TQ; ++p)
#pragma unroll
      for (int rq = 0; rq < 2; ++rq) acc[g][p][rq] = f32x4{0.f, 0.f, 0.f, 0.f};
  int tok[TQ];
#pragma unroll
  for (int p = 0; p < TQ; ++p) tok[p] = 4 * p + q4 < T ? 4 * p + q4 : T - 1;

  // The (row, step) slices of x and the steps of the norm weights, spread over the waves.
  for (int i = wave; i < (NORM ? TP + 1 : TP) * WV; i += NW) {
    const int t = i / WV, k = i % WV;
    if (t < TP)
      dma16(a.x + (size_t)(t < T ? t : T - 1) * in + (size_t)k * kStep + lane * 8, &xs[t][k][0]);
    else
      dma16(a.norm_w + (size_t)k * kStep + lane * 8, &nws[k][0]);
  }
  __builtin_amdgcn_sched_barrier(0);
  const size_t k0 = (size_t)step * kStep;
  u32x4 wv[4][G][2];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int rq = 0; rq < 2; ++rq)
        wv[c][g][rq] = ld16_stream(a.w + (size_t)row_of<EPI>(g0 + g, 4 * rq + q4, a) * in +
                                   k0 + 128 * c + 8 * qb);
  __builtin_amdgcn_sched_barrier(0);
  wait_vm_lgkm<NWL, 15>();  // this wave's DMA loads have landed; its W loads stay in flight
  dma_barrier();
  if constexpr (NORM) {
    // Wave t takes row t: its sum of squares, then the row normalised in place from the slices
    // it already holds (no second pass over LDS, one barrier).
    if (wave < TP) {
      const int t = wave;
      u32x4 xr[WV];
      float ss = 0.0f;
#pragma unroll
      for (int k = 0; k < WV; ++k) {
        xr[k] = xs[t][k][lane];
        const f16x8 h = as_h8(xr[k]);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float f = (float)h[j];
          ss = ss + f * f;
        }
      }
      ss = wave_sum(ss);
      const float inv = 1.0f / __builtin_sqrtf(ss / (float)in + a.eps);
#pragma unroll
      for (int k = 0; k < WV; ++k) {
        const f16x8 h = as_h8(xr[k]);
        f16x8 an;
#pragma unroll
        for (int j = 0; j < 8; ++j) an[j] = (f16)((float)h[j] * inv);
        xs[t][k][lane] = as_u4(as_h8(nws[k][lane]) * an);
      }
    }
    wait_vm_lgkm<63, 0>();
    dma_barrier();
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    u32x4 xv[TQ];
#pragma unroll
    for (int p = 0; p < TQ; ++p) xv[p] = xs[tok[p]][step][16 * c + qb];
#pragma unroll
    for (int g = 0; g < G; ++g) mfma_chunk<TQ>(acc[g], wv[c][g], xv);
  }
#pragma unroll
  for (int g = 0; g < G; ++g) mfma_store_part<TQ>(acc[g], part[rg * G + g][step]);
  __syncthreads();
  // The RG * G row groups' epilogues, side by side.
  constexpr int E = epi_threads<EPI, TPP>();
  static_assert(RG * G * E <= 64 * NW, "threads for every epilogue");
  const int e = threadIdx.x / E, tid = threadIdx.x % E;
  if (e < RG * G)
    rows_epilogue<EPI, TPP, WV>(a, blockIdx.x * RG * G + e, part[e], tid, (f16)0.0f);
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

// Which kernel: for 5 to 8 rows of a matrix with at most kMfmaMaxIn input features, the
// matrix-core kernels (k_rows_mfma, k_rows_mfma_wide) up to kMfmaMaxOut output features and where
// the wide kernel applies; the dot-product kernel (k_rows) otherwise. The family is chosen by the
// row count and the matrix shape alone, and both matrix-core kernels sum every output in the
// same order, so a fused launch (RMSNorm + QKV + RoPE, RMSNorm + gate/up + SwiGLU, a projection
// + residual) and the unfused launches it replaces give the same bits. Same box, Llama-3.2-1B
// shapes, weights rotated past the caches, us (dot products -> k_rows_mfma) at 8 rows: RMSNorm +
// gate/up + SwiGLU 19.1 -> 17.0, RMSNorm + the QKV shape 7.34 -> 6.09, o + residual 6.32 ->
// 6.24, and the lm head (128256 outputs) 93.1 -> 117.3, which therefore takes the wide kernel or
// none; 4 rows of the lm head 77.3 -> 86.1, 1 to 4 rows of the other shapes within 2% either
// way. (Each of the matrix-core kernels' 16-byte loads covers 4 rows x 256 bytes rather than
// 1 KiB of one row.) Over in = 8192 (down + residual) the dot products win once the residual is
// read at the start: 10.3 -> 9.0-9.3 us at 8 rows, equal at 5.
constexpr int kMfmaMaxOut = 16384;
constexpr int kMfmaMaxIn = 4096;

// k_rows_mfma_wide: launches of 5 to 8 rows with in = 2048 (4 steps, 4 row-group pairs per
// block) and at least kWideMinGroups row groups, so that every CU gets a block (gate/up of
// Llama-3.2-1B: 2048 groups, 256 blocks), except the residual epilogue; above kMfmaMaxOut
// outputs too (the lm head), since there it beats the dot products as well. Its outputs are
// k_rows_mfma's bits. Same box, 8 rows, us: RMSNorm + gate/up + SwiGLU 16.7-17.1 -> 14.8-14.9
// (5 rows 16.2 -> 14.6), gate/up alone 17.1 -> 13.7, lm head (128256 x 2048) 93.7 -> 89.7,
// with the RMSNorm 126 -> 96 (5 rows: equal, 88.5).
constexpr int kWideWaves = 4, kWideRG = 4;
constexpr unsigned kWideMinGroups = 2048;

template <int EPI, bool NORM>
int rows_launch_wide(const RowsArgs& a, unsigned blocks, hipStream_t s) {
  if constexpr (EPI == kEpiResidual) {
    return LLMK_ERR_UNSUPPORTED;
  } else {
    return launch(k_rows_mfma_wide<kWideWaves, kWideRG, EPI, NORM>,
                  dim3(blocks / (2 * kWideRG)), dim3(64 * kWideWaves * kWideRG), 0, s, a);
  }
}

template <int TP, int EPI, bool NORM>
int rows_launch_tp(const RowsArgs& a, unsigned blocks, hipStream_t s) {
  const int wv = rows_waves<TP>(a.in / kStep, NORM);
  // exactly kWideWaves steps: the wide kernel gives every wave one step (without the norm,
  // rows_waves rounds 3 steps up to 4 waves)
  const bool wide = EPI != kEpiResidual && wv == kWideWaves && a.in == kWideWaves * kStep &&
                    blocks >= kWideMinGroups && blocks % (2 * kWideRG) == 0;
  const bool mfma = TP == 8 && a.in <= kMfmaMaxIn && (a.out <= kMfmaMaxOut || wide);
  if constexpr (TP == 8)
    if (mfma && wide) return rows_launch_wide<EPI, NORM>(a, blocks, s);
#define LLMK_ROWS_LAUNCH(W)                                                                     \
  if constexpr (TP == 8)                                                                        \
    if (mfma)                                                                                   \
      return launch(k_rows_mfma<TP, W, EPI, NORM>, dim3(blocks), dim3(64 * W), 0, s, a);      \
  return launch(k_rows<TP, W, EPI, NORM>, dim3(blocks), dim3(64 * W), 0, s, a)
  switch (wv) {
    case 1: LLMK_ROWS_LAUNCH(1);
    case 2: LLMK_ROWS_LAUNCH(2);
    case 4: LLMK_ROWS_LAUNCH(4);
    case 8: LLMK_ROWS_LAUNCH(8);
    case 16: LLMK_ROWS_LAUNCH(16);
    default: return LLMK_ERR_UNSUPPORTED;
  }
#undef LLMK_ROWS_LAUNCH
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
