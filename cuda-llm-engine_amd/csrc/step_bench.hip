// llmk_step_bench: times the engine's decode step from a C++ process, the way a C or C++ caller
// of the library runs it (the reference's engine is such a caller: engine/batched.cu:107-120).
// In a Python process that has imported torch, libllmk's hipBLASLt and HIP runtime are the
// copies torch loaded (its bundled builds, same sonames); here they are the system's, which is
// what a C/C++ application linking the library gets. The workload comes from a file bench.py
// writes, so both processes time the same rows:
//   "LLMKROWS" | llmk_model_config | int32 n_rows, max_pages, num_pages |
//   int32 tokens[n_rows] | int32 positions[n_rows] | int32 block_tables[n_rows * max_pages]
// Weights and pools are filled on the device with the distributions bench.py uses (projections
// and embedding N(0, 0.02), norm weights N(1, 0.1), K/V pools N(0, 1)); every layer gets the
// same values, copied into the engine's own storage per layer. The program tunes the GEMM
// plans (llmk_engine_tune), runs llmk_engine_forward_graph until its graph is instantiated,
// checks that the logits are finite, and times `steps` back-to-back graph launches with HIP
// events. It prints one JSON line.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "llmk.h"

namespace {

int fail(const char* what, int st) {
  std::fprintf(stderr, "llmk_step_bench: %s failed (%d)\n", what, st);
  return 1;
}

// x[i] = mean + std * N(0, 1), the normal from two hashed uniforms (Box-Muller).
__global__ void k_fill_normal(_Float16* x, size_t n, uint32_t seed, float mean, float stdev) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    uint32_t a = (uint32_t)i * 2654435761u ^ seed, b = (uint32_t)(i >> 32) * 40503u ^ (seed * 7919u + 1u);
    a ^= a >> 16; a *= 0x7FEB352Du; a ^= a >> 15; a *= 0x846CA68Bu; a ^= a >> 16;
    b ^= a + 0x9E3779B9u; b ^= b >> 16; b *= 0x7FEB352Du; b ^= b >> 15; b *= 0x846CA68Bu; b ^= b >> 16;
    const float u1 = ((float)(a >> 8) + 1.0f) * (1.0f / 16777217.0f);  // (0, 1]
    const float u2 = (float)(b >> 8) * (1.0f / 16777216.0f);           // [0, 1)
    const float z = sqrtf(-2.0f * logf(u1)) * cosf(6.2831853f * u2);
    x[i] = (_Float16)(mean + stdev * z);
  }
}

int fill(void* p, size_t n, uint32_t seed, float mean, float stdev, hipStream_t s) {
  hipLaunchKernelGGL(k_fill_normal, dim3(4096), dim3(256), 0, s, static_cast<_Float16*>(p), n,
                     seed, mean, stdev);
  return (int)hipGetLastError();
}

std::string mapped(const char* name) {  // the path of the loaded library whose name contains `name`
  FILE* f = std::fopen("/proc/self/maps", "r");
  if (!f) return "";
  char line[4096];
  std::string out;
  while (std::fgets(line, sizeof line, f)) {
    const char* p = std::strchr(line, '/');
    if (p && std::strstr(p, name)) {
      out = p;
      while (!out.empty() && (out.back() == '\n' || out.back() == ' ')) out.pop_back();
      break;
    }
  }
  std::fclose(f);
  return out;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 2) {
    std::fprintf(stderr, "usage: llmk_step_bench ROWS_FILE [steps] [warmup]\n");
    return 2;
  }
  const int steps = argc > 2 ? std::atoi(argv[2]) : 50;
  const int warmup = argc > 3 ? std::atoi(argv[3]) : 10;
  FILE* f = std::fopen(argv[1], "rb");
  if (!f) return fail("open rows file", 0);
  char magic[8];
  llmk_model_config cfg;
  int32_t hdr[3];
  if (std::fread(magic, 1, 8, f) != 8 || std::memcmp(magic, "LLMKROWS", 8) != 0 ||
      std::fread(&cfg, sizeof cfg, 1, f) != 1 || std::fread(hdr, sizeof hdr, 1, f) != 1)
    return fail("read rows header", 0);
  const int n = hdr[0], max_pages = hdr[1], num_pages = hdr[2];
  if (n <= 0 || max_pages <= 0 || num_pages <= 0) return fail("rows header values", 0);
  std::vector<int32_t> tokens(n), positions(n), tables((size_t)n * max_pages);
  if (std::fread(tokens.data(), 4, n, f) != (size_t)n ||
      std::fread(positions.data(), 4, n, f) != (size_t)n ||
      std::fread(tables.data(), 4, tables.size(), f) != tables.size())
    return fail("read rows", 0);
  std::fclose(f);

  int st = (int)hipSetDevice(0);
  if (st) return fail("hipSetDevice", st);
  hipStream_t s;
  if ((st = (int)hipStreamCreate(&s))) return fail("hipStreamCreate", st);
  llmk_engine* e = nullptr;
  if ((st = llmk_engine_create(&cfg, n, max_pages, num_pages, &e))) return fail("engine_create", st);

  // One layer's weights in the reference's layout, reused for every layer.
  const size_t H = cfg.hidden, Q = (size_t)cfg.n_heads * cfg.head_dim,
               KV = (size_t)cfg.n_kv_heads * cfg.head_dim, I = cfg.inter, V = cfg.vocab;
  const size_t counts[11] = {V * H, H, H, Q * H, KV * H, KV * H, H * Q, H, I * H, I * H, H * I};
  void* buf[11] = {};
  for (int i = 0; i < 11; ++i) {
    if ((st = (int)hipMalloc(&buf[i], counts[i] * 2))) return fail("hipMalloc", st);
    const bool norm = i == 1 || i == 2 || i == 7;  // final norm, attention norm, MLP norm
    if ((st = fill(buf[i], counts[i], 1000u + 17u * i, norm ? 1.0f : 0.0f, norm ? 0.1f : 0.02f, s)))
      return fail("fill weights", st);
  }
  if ((st = (int)hipStreamSynchronize(s))) return fail("fill weights", st);
  auto u16 = [&](int i) { return static_cast<const uint16_t*>(buf[i]); };
  std::vector<llmk_layer_weights> layers(cfg.n_layers);
  for (auto& l : layers)
    l = llmk_layer_weights{u16(2), u16(3), u16(4), u16(5), u16(6), u16(7), u16(8), u16(9), u16(10)};
  if ((st = llmk_engine_set_weights(e, u16(0), u16(1), layers.data()))) return fail("set_weights", st);
  for (int i = 0; i < 11; ++i) (void)hipFree(buf[i]);

  const size_t pool = (size_t)num_pages * 16 * KV;
  for (int l = 0; l < cfg.n_layers; ++l)
    for (int which : {LLMK_BUF_K_POOL, LLMK_BUF_V_POOL})
      if ((st = fill(llmk_engine_buffer(e, which, l), pool, 77u + 2u * l + (uint32_t)which, 0.0f,
                     1.0f, s)))
        return fail("fill pools", st);
  if ((st = (int)hipStreamSynchronize(s))) return fail("fill pools", st);

  if ((st = llmk_engine_tune(e, n, -1, s))) return fail("engine_tune", st);
  if ((st = llmk_engine_set_rows(e, n, tokens.data(), positions.data(), tables.data(), 0, nullptr,
                                 s)))
    return fail("engine_set_rows", st);
  for (int i = 0; i < warmup + 2; ++i)
    if ((st = llmk_engine_forward_graph(e, n, -1, 0, s))) return fail("engine_forward_graph", st);
  if ((st = (int)hipStreamSynchronize(s))) return fail("warm-up passes", st);

  std::vector<uint16_t> logits((size_t)n * V);
  if ((st = (int)hipMemcpy(logits.data(), llmk_engine_buffer(e, LLMK_BUF_LOGITS, 0),
                           logits.size() * 2, hipMemcpyDeviceToHost)))
    return fail("copy logits", st);
  for (uint16_t b : logits)
    if ((b & 0x7C00u) == 0x7C00u) return fail("finite logits", (int)b);

  hipEvent_t e0, e1;
  if ((st = (int)hipEventCreate(&e0)) || (st = (int)hipEventCreate(&e1))) return fail("events", st);
  (void)hipEventRecord(e0, s);
  for (int i = 0; i < steps; ++i)
    if ((st = llmk_engine_forward_graph(e, n, -1, 0, s))) return fail("engine_forward_graph", st);
  (void)hipEventRecord(e1, s);
  if ((st = (int)hipEventSynchronize(e1))) return fail("timed passes", st);
  float ms = 0.0f;
  (void)hipEventElapsedTime(&ms, e0, e1);
  std::printf("{\"us_mean\": %.3f, \"steps\": %d, \"warmup\": %d, \"rows\": %d, "
              "\"hipblaslt\": \"%s\", \"amdhip64\": \"%s\"}\n",
              1000.0 * ms / steps, steps, warmup, n, mapped("libhipblaslt").c_str(),
              mapped("libamdhip64").c_str());
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  llmk_engine_destroy(e);
  (void)hipStreamDestroy(s);
  return 0;
}
