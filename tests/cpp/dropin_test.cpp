// Drop-in test: engine-style C++ that includes llmk.hpp in place of the reference's kernels/*.cuh
// and calls the reference's launcher names with the reference's argument lists, on hipMalloc'd
// buffers and the null stream, exactly as ref: engine/batched.cu:44-72 does. Each case mirrors
// one of the reference's kernel unit tests (ref: tests/test_*.cu) and checks the result against
// the CPU oracle (oracle/oracle.h): bit-exact for copies and the residual add, the reference's
// tolerance |d| <= 1e-3 + 4e-3 |e| for norm, rotary and activation.
//
// Exit status = number of failed checks (0 = pass), like the reference's test mains.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <numeric>
#include <random>
#include <vector>

#include "llmk.hpp"
#include "llmk_engine.hpp"
#include "../../oracle/oracle.h"

#define HIP_CHECK(x)                                                                      \
  do {                                                                                    \
    hipError_t e_ = (x);                                                                  \
    if (e_ != hipSuccess) {                                                               \
      std::fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
      std::exit(100);                                                                     \
    }                                                                                     \
  } while (0)

static int failures = 0;

static void report(const char* name, bool ok, const char* detail = "") {
  std::printf("%-48s %s %s\n", name, ok ? "PASS" : "FAIL", detail);
  std::fflush(stdout);
  failures += !ok;
}

template <typename T>
static T* to_dev(const std::vector<T>& h, size_t extra = 0, int fill = 0) {
  T* d = nullptr;
  HIP_CHECK(hipMalloc(&d, (h.size() + extra) * sizeof(T)));
  if (extra) HIP_CHECK(hipMemset(d, fill, (h.size() + extra) * sizeof(T)));
  if (!h.empty()) HIP_CHECK(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
  return d;
}
template <typename T>
static std::vector<T> to_host(const T* d, size_t n) {
  std::vector<T> h(n);
  HIP_CHECK(hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost));
  return h;
}

static std::vector<uint16_t> normal_f16(size_t n, std::mt19937& rng, float mean, float stdv) {
  std::normal_distribution<float> N(mean, stdv);
  std::vector<uint16_t> v(n);
  for (auto& x : v) x = or_f2h(N(rng));
  return v;
}

// Tolerance rule of ref: tests/test_rmsnorm.cu:50.
static bool within_tol(const std::vector<uint16_t>& got, const std::vector<uint16_t>& exp,
                       char* detail, size_t dlen) {
  size_t bad = 0, exact = 0;
  double max_abs = 0;
  for (size_t i = 0; i < got.size(); ++i) {
    const double g = or_h2f(got[i]), e = or_h2f(exp[i]), d = std::fabs(g - e);
    exact += got[i] == exp[i];
    max_abs = std::max(max_abs, d);
    if (got[i] != exp[i] && !(d <= 1e-3 + 4e-3 * std::fabs(e))) ++bad;  // NaN poison: bits
  }
  std::snprintf(detail, dlen, "(max_abs %.2e, exact %.3f%%)", max_abs,
                100.0 * exact / std::max<size_t>(1, got.size()));
  return bad == 0;
}

int main() {
  std::mt19937 rng(1234);
  char detail[128];
  const float eps = 1e-5f;

  // residual_add: the reference's own known-answer test (ref: tests/test_residual_add.cu:12-58).
  {
    const size_t n = 1000003, pad = 256;
    std::vector<uint16_t> a(n), b(n), expected(n);
    or_residual_add_kat_inputs(12345u, n, a.data(), b.data());
    or_residual_add(a.data(), b.data(), expected.data(), n);
    __half* da = reinterpret_cast<__half*>(to_dev(a));
    __half* db = reinterpret_cast<__half*>(to_dev(b));
    uint16_t* dout_u = to_dev(std::vector<uint16_t>(), n + pad, 0xAB);
    __half* dout = reinterpret_cast<__half*>(dout_u);
    residual_add(da, db, dout, n);
    HIP_CHECK(hipGetLastError());
    HIP_CHECK(hipDeviceSynchronize());
    auto got = to_host(dout_u, n + pad);
    report("residual_add out-of-place exact", std::memcmp(got.data(), expected.data(), n * 2) == 0);
    bool canary = true;
    for (size_t i = n; i < n + pad; ++i) canary &= got[i] == 0xABAB;
    report("residual_add padding untouched", canary);
    residual_add(da, db, da, n);
    HIP_CHECK(hipDeviceSynchronize());
    auto got2 = to_host(reinterpret_cast<uint16_t*>(da), n);
    report("residual_add in place exact", std::memcmp(got2.data(), expected.data(), n * 2) == 0);
    (void)hipFree(da); (void)hipFree(db); (void)hipFree(dout_u);
  }

  // embedding_lookup (ref: tests/test_embedding.cu:21-45): bit-exact gather.
  {
    const int vocab = 4096, hidden = 2048, n = 333;
    auto table = normal_f16((size_t)vocab * hidden, rng, 0.f, 0.02f);
    std::vector<int32_t> ids(n);
    std::uniform_int_distribution<int> U(0, vocab - 1);
    for (auto& i : ids) i = U(rng);
    std::vector<uint16_t> expected((size_t)n * hidden);
    or_embedding_lookup(table.data(), ids.data(), expected.data(), n, hidden);
    uint16_t* dt = to_dev(table);
    int32_t* di = to_dev(ids);
    uint16_t* dout = to_dev(std::vector<uint16_t>(), (size_t)n * hidden, 0x7F);
    embedding_lookup(reinterpret_cast<__half*>(dt), di, reinterpret_cast<__half*>(dout), n, hidden);
    HIP_CHECK(hipDeviceSynchronize());
    auto got = to_host(dout, (size_t)n * hidden);
    report("embedding_lookup exact", got == expected);
    (void)hipFree(dt); (void)hipFree(di); (void)hipFree(dout);
  }

  // rmsnorm (ref: tests/test_rmsnorm.cu:24-57) and the fused add_rmsnorm.
  {
    const int rows = 16, hidden = 2048;
    auto x = normal_f16((size_t)rows * hidden, rng, 0.f, 1.f);
    auto r = normal_f16((size_t)rows * hidden, rng, 0.f, 1.f);
    auto w = normal_f16(hidden, rng, 1.f, 0.1f);
    std::vector<uint16_t> expected((size_t)rows * hidden);
    or_rmsnorm(x.data(), w.data(), expected.data(), rows, hidden, eps);
    uint16_t *dx = to_dev(x), *dw = to_dev(w), *dr = to_dev(r);
    uint16_t* dout = to_dev(std::vector<uint16_t>(), (size_t)rows * hidden, 0x7F);
    rmsnorm(reinterpret_cast<__half*>(dx), reinterpret_cast<__half*>(dw),
            reinterpret_cast<__half*>(dout), rows, hidden, eps);
    HIP_CHECK(hipDeviceSynchronize());
    bool ok = within_tol(to_host(dout, expected.size()), expected, detail, sizeof detail);
    report("rmsnorm within tolerance", ok, detail);

    std::vector<uint16_t> r_exp = r, o_exp((size_t)rows * hidden);
    or_add_rmsnorm(r_exp.data(), x.data(), w.data(), o_exp.data(), rows, hidden, eps);
    add_rmsnorm(reinterpret_cast<__half*>(dr), reinterpret_cast<__half*>(dx),
                reinterpret_cast<__half*>(dw), reinterpret_cast<__half*>(dout), rows, hidden, eps);
    HIP_CHECK(hipDeviceSynchronize());
    report("add_rmsnorm residual exact", to_host(dr, r_exp.size()) == r_exp);
    ok = within_tol(to_host(dout, o_exp.size()), o_exp, detail, sizeof detail);
    report("add_rmsnorm out within tolerance", ok, detail);
    (void)hipFree(dx); (void)hipFree(dw); (void)hipFree(dr); (void)hipFree(dout);
  }

  // compute_rope_inv_freq and rope_apply (ref: tests/test_rope.cu:22-80), positions 0..T-1.
  {
    const int NH = 32, NKV = 8, HD = 64, T = 402;
    auto inv = compute_rope_inv_freq(HD, 500000.0, 32.0, 1.0, 4.0, 8192.0);
    std::vector<float> inv_exp(HD / 2);
    or_compute_rope_inv_freq(HD, 500000.0, 32.0, 1.0, 4.0, 8192.0, inv_exp.data());
    report("compute_rope_inv_freq exact", inv == inv_exp);
    auto q = normal_f16((size_t)T * NH * HD, rng, 0.f, 1.f);
    auto k = normal_f16((size_t)T * NKV * HD, rng, 0.f, 1.f);
    std::vector<int32_t> pos(T);
    std::iota(pos.begin(), pos.end(), 0);
    uint16_t *dq = to_dev(q), *dk = to_dev(k);
    int32_t* dp = to_dev(pos);
    float* dinv = to_dev(inv);
    rope_apply(reinterpret_cast<__half*>(dq), reinterpret_cast<__half*>(dk), dp, dinv, T, NH, NKV,
               HD);
    HIP_CHECK(hipDeviceSynchronize());
    or_rope_apply(q.data(), k.data(), pos.data(), inv_exp.data(), T, NH, NKV, HD);
    bool okq = within_tol(to_host(dq, q.size()), q, detail, sizeof detail);
    report("rope_apply Q within tolerance", okq, detail);
    bool okk = within_tol(to_host(dk, k.size()), k, detail, sizeof detail);
    report("rope_apply K within tolerance", okk, detail);
    (void)hipFree(dq); (void)hipFree(dk); (void)hipFree(dp); (void)hipFree(dinv);
  }

  // swiglu (ref: tests/test_swiglu.cu:13-48), n not a multiple of the vector width.
  {
    const size_t n = 8192 * 13 + 5;
    auto g = normal_f16(n, rng, 0.f, 1.f), u = normal_f16(n, rng, 0.f, 1.f);
    std::vector<uint16_t> expected(n);
    or_swiglu(g.data(), u.data(), expected.data(), n);
    uint16_t *dg = to_dev(g), *du = to_dev(u), *dout = to_dev(std::vector<uint16_t>(), n, 0);
    swiglu(reinterpret_cast<__half*>(dg), reinterpret_cast<__half*>(du),
           reinterpret_cast<__half*>(dout), n);
    HIP_CHECK(hipDeviceSynchronize());
    bool ok = within_tol(to_host(dout, n), expected, detail, sizeof detail);
    report("swiglu within tolerance", ok, detail);
    (void)hipFree(dg); (void)hipFree(du); (void)hipFree(dout);
  }

  // kv_scatter (prefill) and kv_scatter_batch + rope_kv_scatter_batch (decode) into shuffled
  // pages of a NaN-filled pool (ref: engine/paged.cu:22, tests/test_paged_attention.cu:60-71).
  {
    const int P = 16, NKV = 8, HD = 64, NH = 32, kvdim = NKV * HD, POOL = 96, T = 100;
    const size_t pool_elems = (size_t)POOL * P * kvdim;
    std::vector<int32_t> perm(POOL);
    std::iota(perm.begin(), perm.end(), 0);
    std::shuffle(perm.begin(), perm.end(), rng);
    const int npages = (T + P - 1) / P;
    std::vector<int32_t> table(perm.begin(), perm.begin() + npages);
    auto src = normal_f16((size_t)T * kvdim, rng, 0.f, 1.f);
    std::vector<uint16_t> pool_exp(pool_elems, 0x7F7F);
    or_kv_scatter(src.data(), pool_exp.data(), table.data(), 0, T, P, kvdim);
    uint16_t* dsrc = to_dev(src);
    uint16_t* dpool = to_dev(std::vector<uint16_t>(), pool_elems, 0x7F);
    int32_t* dtab = to_dev(table);
    kv_scatter(reinterpret_cast<__half*>(dsrc), reinterpret_cast<__half*>(dpool), dtab, 0, T, P,
               kvdim);
    HIP_CHECK(hipDeviceSynchronize());
    report("kv_scatter exact (NaN pool elsewhere)", to_host(dpool, pool_elems) == pool_exp);

    // decode: 6 sequences, each with its own table row, one new token each
    const int n = 6, max_pages = 8;
    std::vector<int32_t> tables((size_t)n * max_pages, 0), positions(n);
    int next = npages;
    for (int b = 0; b < n; ++b) {
      const int len = 1 + (int)(rng() % (max_pages * P));
      positions[b] = len - 1;
      for (int i = 0; i < (len + P - 1) / P; ++i) tables[(size_t)b * max_pages + i] = perm[next++ % POOL];
    }
    auto kb = normal_f16((size_t)n * kvdim, rng, 0.f, 1.f);
    auto vb = normal_f16((size_t)n * kvdim, rng, 0.f, 1.f);
    auto qb = normal_f16((size_t)n * NH * HD, rng, 0.f, 1.f);
    std::vector<uint16_t> kp_exp(pool_elems, 0x7F7F), vp_exp(pool_elems, 0x7F7F);
    or_kv_scatter_batch(kb.data(), kp_exp.data(), tables.data(), positions.data(), n, max_pages,
                        P, kvdim);
    uint16_t* dkb = to_dev(kb);
    uint16_t* dkp = to_dev(std::vector<uint16_t>(), pool_elems, 0x7F);
    int32_t *dtabs = to_dev(tables), *dpos = to_dev(positions);
    kv_scatter_batch(reinterpret_cast<__half*>(dkb), reinterpret_cast<__half*>(dkp), dtabs, dpos,
                     n, max_pages, P, kvdim);
    HIP_CHECK(hipDeviceSynchronize());
    report("kv_scatter_batch exact (NaN pool elsewhere)", to_host(dkp, pool_elems) == kp_exp);

    std::vector<float> inv(HD / 2);
    or_compute_rope_inv_freq(HD, 500000.0, 32.0, 1.0, 4.0, 8192.0, inv.data());
    std::vector<uint16_t> q_exp = qb;
    std::fill(kp_exp.begin(), kp_exp.end(), 0x7F7F);
    or_rope_kv_scatter_batch(q_exp.data(), kb.data(), vb.data(), kp_exp.data(), vp_exp.data(),
                             tables.data(), positions.data(), inv.data(), n, max_pages, P, NH,
                             NKV, HD);
    uint16_t *dqb = to_dev(qb), *dvb = to_dev(vb);
    uint16_t* dvp = to_dev(std::vector<uint16_t>(), pool_elems, 0x7F);
    HIP_CHECK(hipMemset(dkp, 0x7F, pool_elems * 2));
    float* dinv = to_dev(inv);
    rope_kv_scatter_batch(reinterpret_cast<__half*>(dqb), reinterpret_cast<__half*>(dkb),
                          reinterpret_cast<__half*>(dvb), reinterpret_cast<__half*>(dkp),
                          reinterpret_cast<__half*>(dvp), dtabs, dpos, dinv, n, max_pages, P, NH,
                          NKV, HD);
    HIP_CHECK(hipDeviceSynchronize());
    report("rope_kv_scatter_batch V pool exact", to_host(dvp, pool_elems) == vp_exp);
    bool ok = within_tol(to_host(dkp, pool_elems), kp_exp, detail, sizeof detail);
    report("rope_kv_scatter_batch K pool within tolerance", ok, detail);
    ok = within_tol(to_host(dqb, qb.size()), q_exp, detail, sizeof detail);
    report("rope_kv_scatter_batch Q within tolerance", ok, detail);
    (void)hipFree(dsrc); (void)hipFree(dpool); (void)hipFree(dtab); (void)hipFree(dkb); (void)hipFree(dkp); (void)hipFree(dtabs);
    (void)hipFree(dpos); (void)hipFree(dqb); (void)hipFree(dvb); (void)hipFree(dvp); (void)hipFree(dinv);
  }

  // ---- attention_decode_fast (ref: tests/test_attention_decode_fast.cu:16-99): its lengths,
  // shuffled pages, NaN in every unused slot, the output memset to 0x7F, and one run per split
  // count with a workspace sized by attention_decode_fast_workspace_floats.
  {
    const int NH = 32, NKV = 8, HD = 64, P = 16, kvdim = NKV * HD;
    const std::vector<int> lens = {1, 15, 16, 17, 33, 100, 402, 2048};
    const int n_seq = (int)lens.size();
    int max_pages = 0, total_pages = 0;
    for (int S : lens) {
      const int np = (S + P - 1) / P;
      max_pages = std::max(max_pages, np);
      total_pages += np;
    }
    std::mt19937 rng(2024);
    std::uniform_real_distribution<float> U(-1.f, 1.f);
    std::vector<uint16_t> q((size_t)n_seq * NH * HD);
    for (auto& x : q) x = or_f2h(U(rng));
    std::vector<int> perm(total_pages);
    std::iota(perm.begin(), perm.end(), 0);
    std::shuffle(perm.begin(), perm.end(), rng);
    std::vector<int> tables((size_t)n_seq * max_pages, 0);
    std::vector<uint16_t> kp((size_t)total_pages * P * kvdim, 0x7F7F), vp(kp.size(), 0x7F7F);
    int next = 0;
    for (int s = 0; s < n_seq; s++) {
      const int np = (lens[s] + P - 1) / P;
      for (int i = 0; i < np; i++) tables[(size_t)s * max_pages + i] = perm[next++];
      for (int j = 0; j < lens[s]; j++) {
        const size_t dst = ((size_t)tables[(size_t)s * max_pages + j / P] * P + j % P) * kvdim;
        for (int d = 0; d < kvdim; d++) {
          kp[dst + d] = or_f2h(U(rng));
          vp[dst + d] = or_f2h(U(rng));
        }
      }
    }
    std::vector<uint16_t> expected(q.size());
    or_attention_decode_paged(q.data(), kp.data(), vp.data(), tables.data(), lens.data(),
                              expected.data(), n_seq, max_pages, P, NH, NKV, HD);
    uint16_t *dq = to_dev(q), *dk = to_dev(kp), *dv = to_dev(vp);
    uint16_t* dout = to_dev(std::vector<uint16_t>(), q.size());
    int *dtab = to_dev(tables), *dlens = to_dev(lens);
    for (int splits : {1, 2, 3, 8, 16, 32}) {
      float* dws = nullptr;
      HIP_CHECK(hipMalloc(&dws, attention_decode_fast_workspace_floats(n_seq, NH, splits) *
                                    sizeof(float)));
      HIP_CHECK(hipMemset(dout, 0x7F, q.size() * 2));
      attention_decode_fast(reinterpret_cast<__half*>(dq), reinterpret_cast<__half*>(dk),
                            reinterpret_cast<__half*>(dv), dtab, dlens,
                            reinterpret_cast<__half*>(dout), dws, n_seq, max_pages, P, NH, NKV,
                            HD, splits);
      HIP_CHECK(hipGetLastError());
      HIP_CHECK(hipDeviceSynchronize());
      const bool ok = within_tol(to_host(dout, q.size()), expected, detail, sizeof detail);
      char name[64];
      std::snprintf(name, sizeof name, "attention_decode_fast splits %d", splits);
      report(name, ok, detail);
      (void)hipFree(dws);
    }
    const int pick = choose_num_splits(256, NKV, 2048);
    report("choose_num_splits MI355X default", pick == 32);
    (void)hipFree(dq); (void)hipFree(dk); (void)hipFree(dv); (void)hipFree(dout);
    (void)hipFree(dtab); (void)hipFree(dlens);
  }

  // ---- argmax_rows (ref: tests/test_argmax.cu:9-46): 8 rows of 128256 -- four rows of exact
  // ties, a constant row (answer 0), the maximum at the last index, two equal maxima at 0 and
  // 77777 (answer 0), a random row.
  {
    const int V = 128256, R = 8;
    std::mt19937 rng(3);
    std::uniform_real_distribution<float> U(-5.f, 5.f);
    std::uniform_int_distribution<int> small(-8, 8);
    std::vector<uint16_t> h((size_t)R * V);
    for (int r = 0; r < R; r++)
      for (int i = 0; i < V; i++) {
        float v;
        if (r < 4) v = small(rng) * 0.5f;
        else if (r == 4) v = 1.0f;
        else v = U(rng);
        h[(size_t)r * V + i] = or_f2h(v);
      }
    h[(size_t)5 * V + (V - 1)] = or_f2h(100.f);
    h[(size_t)6 * V + 0] = or_f2h(100.f);
    h[(size_t)6 * V + 77777] = or_f2h(100.f);
    std::vector<int32_t> expected(R);
    or_argmax_rows(h.data(), expected.data(), R, V);
    uint16_t* d = to_dev(h);
    int* dout = to_dev(std::vector<int>(R, -1));
    argmax_rows(reinterpret_cast<__half*>(d), dout, R, V);
    HIP_CHECK(hipGetLastError());
    HIP_CHECK(hipDeviceSynchronize());
    const std::vector<int> got = to_host(dout, R);
    bool ok = true;
    for (int r = 0; r < R; r++) ok = ok && got[r] == expected[r];
    report("argmax_rows exact (reference rows)", ok);
    report("argmax_rows constant row -> 0, tie -> 0, last", got[4] == 0 && got[6] == 0 &&
                                                               got[5] == V - 1);
    (void)hipFree(d); (void)hipFree(dout);
  }

  // ---- linear (ref: tests/test_linear.cu:20-50): y = x W^T against the oracle's fp32
  // accumulation, the reference's rule |d| <= 3e-3 + 8e-3 |e|.
  {
    const int T = 7, in = 2048, out = 3072;
    std::mt19937 rng(5);
    auto x = normal_f16((size_t)T * in, rng, 0.f, 1.f);
    auto w = normal_f16((size_t)out * in, rng, 0.f, 0.02f);
    std::vector<uint16_t> expected((size_t)T * out);
    or_linear(x.data(), w.data(), expected.data(), T, in, out);
    llmk_blas* handle = nullptr;
    if (llmk_blas_create(&handle) != LLMK_OK) {
      report("linear handle", false);
    } else {
      uint16_t* dx = to_dev(x);
      uint16_t* dw = to_dev(w);
      uint16_t* dy = to_dev(std::vector<uint16_t>(), (size_t)T * out, 0x7F);
      linear(handle, reinterpret_cast<__half*>(dx), reinterpret_cast<__half*>(dw),
             reinterpret_cast<__half*>(dy), T, in, out);
      HIP_CHECK(hipDeviceSynchronize());
      auto got = to_host(dy, (size_t)T * out);
      size_t bad = 0;
      for (size_t i = 0; i < got.size(); ++i) {
        const double g = or_h2f(got[i]), e = or_h2f(expected[i]);
        bad += !(std::fabs(g - e) <= 3e-3 + 8e-3 * std::fabs(e));
      }
      std::snprintf(detail, sizeof(detail), "(%zu outside)", bad);
      report("linear within the reference's rule", bad == 0, detail);
      (void)hipFree(dx); (void)hipFree(dw); (void)hipFree(dy);
      llmk_blas_destroy(handle);
    }
  }

  // ---- run_scheduler over the engine (ref: tests/test_scheduler.cu:14-76): a small Llama-3
  // shape with seeded weights; the same requests one at a time and up to 3 at once give the
  // same outputs, batching takes fewer decode steps, and every page comes back.
  {
    llmk_model_config cfg = llmk::llama32_1b_config();
    cfg.n_layers = 2;
    cfg.hidden = 256;
    cfg.n_heads = 4;
    cfg.n_kv_heads = 1;
    cfg.inter = 512;
    cfg.vocab = 512;
    const int num_pages = 40, max_pages = 8;
    llmk::Engine eng(cfg, 16, max_pages, num_pages);
    std::mt19937 rng(9);
    const int H = cfg.hidden, I = cfg.inter, qd = cfg.n_heads * 64, kvd = cfg.n_kv_heads * 64;
    std::vector<std::vector<uint16_t>> keep;
    auto add = [&](size_t n, float mean, float sd) {
      keep.push_back(normal_f16(n, rng, mean, sd));
      return reinterpret_cast<const uint16_t*>(keep.back().data());
    };
    const uint16_t* embed = add((size_t)cfg.vocab * H, 0.f, 0.5f);
    const uint16_t* fnorm = add(H, 1.f, 0.1f);
    std::vector<llmk_layer_weights> layers(cfg.n_layers);
    for (auto& l : layers) {
      l.attn_norm = add(H, 1.f, 0.1f);
      l.wq = add((size_t)qd * H, 0.f, 0.05f);
      l.wk = add((size_t)kvd * H, 0.f, 0.05f);
      l.wv = add((size_t)kvd * H, 0.f, 0.05f);
      l.wo = add((size_t)H * qd, 0.f, 0.05f);
      l.mlp_norm = add(H, 1.f, 0.1f);
      l.w_gate = add((size_t)I * H, 0.f, 0.05f);
      l.w_up = add((size_t)I * H, 0.f, 0.05f);
      l.w_down = add((size_t)H * I, 0.f, 0.05f);
    }
    eng.set_weights(reinterpret_cast<const __half*>(embed), reinterpret_cast<const __half*>(fnorm),
                    layers);
    std::vector<llmk::Request> base(9);
    std::uniform_int_distribution<int> tok(0, cfg.vocab - 1), len(2, 40), nnew(1, 7);
    for (int i = 0; i < 9; ++i) {
      base[i].id = i;
      base[i].prompt.resize(len(rng));
      for (auto& t : base[i].prompt) t = tok(rng);
      base[i].max_new = nnew(rng);
      base[i].arrival_step = i;
    }
    hipStream_t stream;
    HIP_CHECK(hipStreamCreate(&stream));
    std::vector<llmk::Request> one = base, three = base, three_gpu = base;
    llmk::PageAllocator pages(num_pages);
    // the reference's default: the greedy choice on the host
    const llmk::SchedulerStats s1 = llmk::run_scheduler(eng, pages, one, 1, stream);
    const int free1 = pages.num_free();
    const llmk::SchedulerStats s3 = llmk::run_scheduler(eng, pages, three, 3, stream);
    const llmk::SchedulerStats g3 =
        llmk::run_scheduler(eng, pages, three_gpu, 3, stream, /*gpu_argmax=*/true);
    bool same = true, same_gpu = true;
    for (int i = 0; i < 9; ++i) {
      same = same && one[i].output == three[i].output &&
             (int)one[i].output.size() == base[i].max_new;
      same_gpu = same_gpu && three_gpu[i].output == three[i].output;
    }
    std::snprintf(detail, sizeof(detail), "(%d vs %d decode steps)", s1.decode_steps,
                  s3.decode_steps);
    report("run_scheduler: batched outputs = one at a time", same, detail);
    report("run_scheduler: GPU argmax = host argmax", same_gpu);
    report("run_scheduler: batching takes fewer steps", s3.decode_steps < s1.decode_steps);
    report("run_scheduler: every page returned", free1 == num_pages &&
                                                     pages.num_free() == num_pages);
    std::snprintf(detail, sizeof(detail),
                  "(host: prep %.2f gpu %.2f copy %.2f convert %.2f argmax %.2f ms; gpu mode: "
                  "convert %.2f argmax %.2f)",
                  s3.prep_ms, s3.gpu_ms, s3.copy_ms, s3.convert_ms, s3.argmax_ms, g3.convert_ms,
                  g3.argmax_ms);
    report("run_scheduler: time split filled in",
           s3.gpu_ms > 0 && s3.copy_ms > 0 && s3.convert_ms > 0 && s3.argmax_ms > 0 &&
               s3.prep_ms > 0 && g3.gpu_ms > 0 && g3.copy_ms > 0 && g3.convert_ms == 0 &&
               g3.argmax_ms == 0 && s3.gpu_ms <= s3.decode_ms && g3.gpu_ms <= g3.decode_ms,
           detail);
    HIP_CHECK(hipStreamDestroy(stream));
  }

  std::printf("%s: %d failure(s)\n", failures ? "FAILED" : "ALL PASSED", failures);
  return failures;
}
