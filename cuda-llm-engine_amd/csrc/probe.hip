// Measurement kernels: HBM bandwidth probes for each traffic mix the layer kernels have, and an
// empty kernel for the launch floor of a sequence of launches.
//
// The probes move 16-byte vectors with the same non-temporal accesses the layer kernels use, so
// their rate is the ceiling a kernel of that mix can reach on the box (ref: bench/bandwidth.cu:
// 11-62, which sweeps block and grid sizes of a copy kernel for the same purpose). Modes:
//   READ     a -> nothing        (read-only: argmax, attention)
//   COPY     a -> dst            (1 read : 1 write, separate buffers: gather, copy)
//   READ2    a, b -> dst         (2 reads : 1 write: SwiGLU)
//   INPLACE  dst -> dst          (1 read : 1 write, same addresses: RoPE, the residual update)
//   WRITE    nothing -> dst      (write-only)
// `blocks` > 0 runs a grid-stride loop over that many 256-thread blocks; 0 gives every thread
// exactly `unroll` vectors (one pass, as the layer kernels are launched). All of a thread's
// loads of one step are issued before its first store.
#include "common.hpp"

namespace llmk {

enum ProbeMode { kRead = 0, kCopy = 1, kRead2 = 2, kInplace = 3, kWrite = 4 };

template <int MODE, int UNROLL>
__global__ void __launch_bounds__(256)
k_bw_probe(const u32x4* __restrict__ a, const u32x4* __restrict__ b, u32x4* dst, size_t nvec,
           uint32_t key, int blocks) {
  const size_t chunk = (size_t)256 * UNROLL;
  const size_t stride = blocks > 0 ? (size_t)blocks * chunk : nvec + chunk;
  u32x4 acc = {0, 0, 0, 0};
  for (size_t base = (size_t)blockIdx.x * chunk; base < nvec; base += stride) {
    u32x4 r[UNROLL], s[UNROLL];
#pragma unroll
    for (int m = 0; m < UNROLL; ++m) {
      const size_t i = base + threadIdx.x + (size_t)m * 256;
      if (i < nvec) {
        if (MODE == kRead || MODE == kCopy || MODE == kRead2) r[m] = ld16_stream(a + i);
        if (MODE == kRead2) s[m] = ld16_stream(b + i);
        if (MODE == kInplace) r[m] = ld16_stream(dst + i);
      }
    }
#pragma unroll
    for (int m = 0; m < UNROLL; ++m) {
      const size_t i = base + threadIdx.x + (size_t)m * 256;
      if (i >= nvec) continue;
      if (MODE == kRead) acc ^= r[m];
      if (MODE == kCopy) st16_stream(dst + i, r[m]);
      if (MODE == kRead2) st16_stream(dst + i, r[m] ^ s[m]);
      if (MODE == kInplace) st16_stream(dst + i, r[m] ^ key);
      if (MODE == kWrite) st16_stream(dst + i, u32x4{key, key, key, (uint32_t)i});
    }
  }
  // READ: the loads must not be optimised away; the store happens only if the xor of everything
  // a thread read equals the key in all four words, and stays inside dst's nvec vectors.
  if (MODE == kRead && acc[0] == key && acc[1] == key && acc[2] == key && acc[3] == key)
    dst[((size_t)blockIdx.x * 256 + threadIdx.x) % nvec] = acc;
}

__global__ void k_empty() {}

template <int MODE>
static int probe_launch(const u32x4* a, const u32x4* b, u32x4* dst, size_t nvec, uint32_t key,
                        int blocks, int unroll, hipStream_t s) {
  auto go = [&](auto kern, int u) {
    const size_t need = ceil_div(nvec, (size_t)256 * u);
    const unsigned grid = blocks > 0 ? (unsigned)blocks : (unsigned)need;
    return launch(kern, dim3(grid), dim3(256), 0, s, a, b, dst, nvec, key, blocks);
  };
  switch (unroll) {
    case 1: return go(k_bw_probe<MODE, 1>, 1);
    case 2: return go(k_bw_probe<MODE, 2>, 2);
    case 4: return go(k_bw_probe<MODE, 4>, 4);
    case 8: return go(k_bw_probe<MODE, 8>, 8);
    default: return LLMK_ERR_INVALID_VALUE;
  }
}

}  // namespace llmk

using namespace llmk;

extern "C" int llmk_bw_probe(int mode, const void* a, const void* b, void* dst, size_t nbytes,
                             int blocks, int unroll, void* stream) {
  if (mode < kRead || mode > kWrite || blocks < 0) return LLMK_ERR_INVALID_VALUE;
  if (nbytes == 0) return LLMK_OK;
  const bool need_a = mode == kRead || mode == kCopy || mode == kRead2;
  if ((need_a && !a) || (mode == kRead2 && !b) || !dst) return LLMK_ERR_INVALID_VALUE;
  if (nbytes % 16 != 0) return LLMK_ERR_SHAPE;
  if ((need_a && !aligned16(a)) || (mode == kRead2 && !aligned16(b)) || !aligned16(dst))
    return LLMK_ERR_ALIGNMENT;
  const size_t nvec = nbytes / 16;
  if (blocks == 0 && ceil_div(nvec, 256) > 0x7FFFFFFFu) return LLMK_ERR_UNSUPPORTED;
  const u32x4* pa = static_cast<const u32x4*>(a);
  const u32x4* pb = static_cast<const u32x4*>(b);
  u32x4* pd = static_cast<u32x4*>(dst);
  hipStream_t s = static_cast<hipStream_t>(stream);
  // READ stores to dst (nbytes, like the source) only if a thread's xor of what it read equals
  // this key in all four words.
  const uint32_t key = 0x9E3779B9u;
  switch (mode) {
    case kRead: return probe_launch<kRead>(pa, pb, pd, nvec, key, blocks, unroll, s);
    case kCopy: return probe_launch<kCopy>(pa, pb, pd, nvec, key, blocks, unroll, s);
    case kRead2: return probe_launch<kRead2>(pa, pb, pd, nvec, key, blocks, unroll, s);
    case kInplace: return probe_launch<kInplace>(pa, pb, pd, nvec, key, blocks, unroll, s);
    default: return probe_launch<kWrite>(pa, pb, pd, nvec, key, blocks, unroll, s);
  }
}

extern "C" int llmk_empty_launch(int blocks, int threads, void* stream) {
  if (blocks <= 0 || threads <= 0 || threads > 1024) return LLMK_ERR_INVALID_VALUE;
  return launch(k_empty, dim3(blocks), dim3(threads), 0, static_cast<hipStream_t>(stream));
}
