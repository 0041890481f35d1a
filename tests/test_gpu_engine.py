"""GPU parity of the decode-step pieces and the engine against the CPU oracle.

- llmk_linear (hipBLASLt) vs the oracle's projection, with the reference's projection test rule
  |d| <= 3e-3 + 8e-3 |e| (ref: tests/test_linear.cu:47) at the engine's shapes.
- llmk_qkv_rope_scatter and llmk_swiglu_rows (the fused layouts) vs the oracle's separate
  operations on the same data: bit-exact, like the unfused kernels.
- The engine (llmk_engine_*) vs oracle.engine_forward on a small Llama-3 shape and on the
  Llama-3.2-1B shape: mixed prefill and decode rows, shuffled pages, teacher-forced steps.
  Library GEMMs sum in their own order, so the bar is the reference's for its engine against
  Hugging Face: relative L2 of every logit row below 5e-3 (ref:
  tests/test_generate_batched.cu:53), the same greedy token wherever the oracle's top two are
  clearly apart, and the same set of written pool slots with every other slot still 0x7F7F.
- The engine's forward pass captured in a HIP graph replays bit-identically to eager runs.
"""
import importlib

import numpy as np
import pytest
import torch

from _helpers import POISON, TINY, normal_f16, oracle_pools, tiny_weights

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def dev(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.float16)).to(DEV)


def dev_i32(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(DEV)


def host(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def linear_rule(got: np.ndarray, exp: np.ndarray):
    g = got.view(np.float16).astype(np.float64)
    e = exp.view(np.float16).astype(np.float64)
    bad = ~(np.abs(g - e) <= 3e-3 + 8e-3 * np.abs(e))
    return int(bad.sum()), float(np.mean(got == exp))


# ------------------------------------------------------------------------------------------
# projections
# ------------------------------------------------------------------------------------------
@pytest.fixture(scope="module")
def blas(llmk):
    return llmk.Blas()


@pytest.mark.parametrize("T,K,N", [(1, 2048, 3072), (8, 2048, 16384), (37, 8192, 2048),
                                   (256, 512, 1024), (402, 2048, 2048), (3, 256, 512)])
def test_linear_matches_oracle(llmk, orc, blas, T, K, N):
    rng = np.random.default_rng(0x5EED0200 + T)
    x = normal_f16(rng, (T, K))
    w = normal_f16(rng, (N, K), std=0.02)
    y = torch.full((T * N + 64,), float("nan"), dtype=torch.float16, device=DEV)
    print(f"linear T={T} K={K} N={N}", flush=True)
    llmk.linear(blas, dev(x), dev(w), y, T, K, N)
    torch.cuda.synchronize()
    got = host(y)
    assert np.all(got[T * N:] == 0x7E00), "write past the output"
    bad, exact = linear_rule(got[:T * N], orc.linear(x, w, T, K, N, threads=16).ravel())
    print(f"  bad {bad} exact {100 * exact:.2f}%")
    assert bad == 0 and exact > 0.9


@pytest.mark.parametrize("K,N", [(2048, 3072), (2048, 2048), (8192, 2048), (512, 1000),
                                 (2048, 16384), (2048, 20480), (2048, 16392), (1536, 16384),
                                 (1024, 13)])
@pytest.mark.parametrize("T", [1, 2, 3, 4, 5, 8])
def test_linear_rows_matches_oracle(llmk, orc, T, K, N):
    """The few-rows kernels (T <= 8): every row count of each padded width (1, 2, 4, 8), output
    widths that are not multiples of the kernel's 8 rows per block, in_features over several
    steps per wave (8192), and at 5 to 8 rows the matrix-core kernels (2048 x 20480: the wide
    one above 16384 outputs; 2048 x 16392: above 16384 outputs in groups the wide kernel does
    not tile, so the dot products; 1536 x 16384: three steps, which the wide kernel must not
    take)."""
    rng = np.random.default_rng(0x5EED0210 + 16 * T + K // 512)
    x = normal_f16(rng, (T, K))
    w = normal_f16(rng, (N, K), std=0.02)
    y = torch.full((T * N + 64,), float("nan"), dtype=torch.float16, device=DEV)
    print(f"linear_rows T={T} K={K} N={N}", flush=True)
    llmk.linear_rows(dev(x), dev(w), y, T, K, N)
    torch.cuda.synchronize()
    got = host(y)
    assert np.all(got[T * N:] == 0x7E00), "write past the output"
    bad, exact = linear_rule(got[:T * N], orc.linear(x, w, T, K, N, threads=16).ravel())
    print(f"  bad {bad} exact {100 * exact:.2f}%")
    assert bad == 0 and exact > 0.9


def test_linear_rows_preconditions(llmk, blas):
    x = torch.zeros(9 * 512 + 8, dtype=torch.float16, device=DEV)
    w = torch.zeros(16 * 512 + 8, dtype=torch.float16, device=DEV)
    y = torch.zeros(9 * 16, dtype=torch.float16, device=DEV)
    with pytest.raises(llmk.LlmkError, match="shape outside"):
        llmk.linear_rows(x, w, y, 9, 512, 16)                    # more than 8 rows
    with pytest.raises(llmk.LlmkError, match="shape outside"):
        llmk.linear_rows(x, w, y, 2, 256, 16)                    # in_features % 512 != 0
    with pytest.raises(llmk.LlmkError, match="aligned"):
        llmk.linear_rows(x[1:], w, y, 2, 512, 16)                # x not 16-byte aligned
    llmk.linear_rows(x, w, y, 0, 512, 16)                        # no rows: nothing to do
    # llmk_linear takes the hipBLASLt path where the few-rows kernel does not apply
    xs = normal_f16(np.random.default_rng(7), (2, 256))
    ws = normal_f16(np.random.default_rng(8), (16, 256), std=0.02)
    yy = torch.empty(32, dtype=torch.float16, device=DEV)
    llmk.linear(blas, dev(xs), dev(ws), yy, 2, 256, 16)
    torch.cuda.synchronize()
    ref = (xs.view(np.float16).astype(np.float32) @ ws.view(np.float16).astype(np.float32).T).ravel()
    assert np.allclose(host(yy).view(np.float16).astype(np.float32), ref, atol=2e-2, rtol=2e-2)


@pytest.mark.parametrize("T", [1, 3, 8])
def test_linear_rows_fused_give_the_bits_of_the_separate_launches(llmk, orc, T):
    """Each fused few-rows entry point against its unfused composition on the GPU (RMSNorm, the
    few-rows projection, then residual_add / swiglu_rows / qkv_rope_scatter): every output bit,
    pool slots included."""
    rng = np.random.default_rng(0x5EED0230 + T)
    H, eps = 2048, 1e-5
    x = dev(normal_f16(rng, (T, H)))
    nw = dev(normal_f16(rng, (H,), 1.0, 0.1))
    normed = torch.empty(T * H, dtype=torch.float16, device=DEV)
    llmk.rmsnorm(x, nw, normed, T, H, eps)

    # norm prologue, plain store
    N = 1000
    w = dev(normal_f16(rng, (N, H), std=0.02))
    y1 = torch.full((T * N,), float("nan"), dtype=torch.float16, device=DEV)
    y2 = y1.clone()
    llmk.linear_rows_norm(x, nw, eps, w, y1, T, H, N)
    llmk.linear_rows(normed, w, y2, T, H, N)
    y3 = y1.clone()
    llmk.linear_rows_norm(x, None, eps, w, y3, T, H, N)
    y4 = y1.clone()
    llmk.linear_rows(x, w, y4, T, H, N)
    torch.cuda.synchronize()
    assert np.array_equal(host(y1), host(y2)) and np.array_equal(host(y3), host(y4))

    # norm prologue over in = 8192: one block of 16 waves, the raw slices of all T rows staged
    # in LDS (135 KB at T = 8)
    K = 8192
    xk = dev(normal_f16(rng, (T, K)))
    nwk = dev(normal_f16(rng, (K,), 1.0, 0.1))
    normed_k = torch.empty(T * K, dtype=torch.float16, device=DEV)
    llmk.rmsnorm(xk, nwk, normed_k, T, K, eps)
    wk = dev(normal_f16(rng, (N, K), std=0.02))
    z1 = torch.full((T * N,), float("nan"), dtype=torch.float16, device=DEV)
    z2 = z1.clone()
    llmk.linear_rows_norm(xk, nwk, eps, wk, z1, T, K, N)
    llmk.linear_rows(normed_k, wk, z2, T, K, N)
    torch.cuda.synchronize()
    assert np.array_equal(host(z1), host(z2))

    # residual-add epilogue (in = 8192, 16 waves per block)
    a = dev(normal_f16(rng, (T, K)))
    wd = dev(normal_f16(rng, (H, K), std=0.02))
    r1 = dev(normal_f16(rng, (T, H)))
    r2 = r1.clone()
    llmk.linear_rows_residual(a, wd, r1, T, K, H)
    p = torch.empty(T * H, dtype=torch.float16, device=DEV)
    llmk.linear_rows(a, wd, p, T, K, H)
    llmk.residual_add(r2, p, r2, T * H)
    torch.cuda.synchronize()
    assert np.array_equal(host(r1), host(r2))

    # norm prologue + swiglu epilogue
    inter = 520
    wgu = dev(normal_f16(rng, (2 * inter, H), std=0.05))
    act1 = torch.full((T * inter,), float("nan"), dtype=torch.float16, device=DEV)
    llmk.linear_rows_swiglu(x, nw, eps, wgu, act1, T, H, inter)
    gu = torch.empty(T * 2 * inter, dtype=torch.float16, device=DEV)
    llmk.linear_rows(normed, wgu, gu, T, H, 2 * inter)
    act2 = act1.clone()
    llmk.swiglu_rows(gu, act2, T, inter)
    torch.cuda.synchronize()
    assert np.array_equal(host(act1), host(act2))

    # norm prologue + RoPE / KV scatter epilogue
    nh, nkv, hd, ps, max_pages = 32, 8, 64, 16, 6
    qkvdim, kvdim = (nh + 2 * nkv) * hd, nkv * hd
    num_pages = T * max_pages
    wqkv = dev(normal_f16(rng, (qkvdim, H), std=0.05))
    pos = dev_i32(rng.integers(0, max_pages * ps, T))
    tables = dev_i32(rng.permutation(num_pages).reshape(T, max_pages))
    inv = torch.from_numpy(orc.compute_rope_inv_freq(hd, 500000.0, 32.0, 1.0, 4.0,
                                                     8192.0)).to(DEV)
    pools = [dev(np.full(num_pages * ps * kvdim, POISON, np.uint16)) for _ in range(4)]
    q1 = torch.full((T * nh * hd,), float("nan"), dtype=torch.float16, device=DEV)
    q2 = q1.clone()
    llmk.linear_rows_qkv_rope_scatter(x, nw, eps, wqkv, q1, pools[0], pools[1], tables, pos, inv,
                                      T, H, nh, nkv, max_pages)
    qkv = torch.empty(T * qkvdim, dtype=torch.float16, device=DEV)
    llmk.linear_rows(normed, wqkv, qkv, T, H, qkvdim)
    llmk.qkv_rope_scatter(qkv, qkvdim, q2, pools[2], pools[3], tables, pos, inv, T, max_pages,
                          ps, nh, nkv, hd)
    torch.cuda.synchronize()
    assert np.array_equal(host(q1), host(q2))
    assert np.array_equal(host(pools[0]), host(pools[2]))
    assert np.array_equal(host(pools[1]), host(pools[3]))
    assert int((host(pools[0]) != POISON).sum()) == T * kvdim  # one row per token, no more


@pytest.mark.parametrize("T", [3, 5, 7, 8])
def test_linear_rows_wide_normalising_launches_give_the_bits_of_the_separate_launches(llmk, orc,
                                                                                       T):
    """Normalising few-rows launches with at least 2048 groups of 8 output rows (gate/up at
    in = 2048; at 5 to 8 rows the 16-wave blocks that stage x in LDS once per 64 rows) against
    RMSNorm + the plain few-rows projection + the separate epilogue: every output bit, for the
    plain store (16384 and 20480 outputs), the SwiGLU epilogue and the RoPE / K/V scatter
    epilogue (240 query heads, so that the QKV rows reach 2048 groups). T = 3 takes the
    dot-product kernel for both."""
    rng = np.random.default_rng(0x5EED0250 + T)
    H, eps, inter = 2048, 1e-5, 8192
    x = dev(normal_f16(rng, (T, H)))
    nw = dev(normal_f16(rng, (H,), 1.0, 0.1))
    normed = torch.empty(T * H, dtype=torch.float16, device=DEV)
    llmk.rmsnorm(x, nw, normed, T, H, eps)
    wgu = dev(normal_f16(rng, (2 * inter, H), std=0.02))
    print(f"wide few-rows T={T}: store", flush=True)
    y1 = torch.full((T * 2 * inter,), float("nan"), dtype=torch.float16, device=DEV)
    y2 = y1.clone()
    llmk.linear_rows_norm(x, nw, eps, wgu, y1, T, H, 2 * inter)
    llmk.linear_rows(normed, wgu, y2, T, H, 2 * inter)
    torch.cuda.synchronize()
    assert np.array_equal(host(y1), host(y2))
    bad, exact = linear_rule(host(y2), orc.linear(host(normed), host(wgu), T, H, 2 * inter,
                                                  threads=16).ravel())
    assert bad == 0 and exact > 0.9

    print(f"wide few-rows T={T}: store above 16384 outputs", flush=True)
    N = 20480
    w = dev(normal_f16(rng, (N, H), std=0.02))
    z1 = torch.full((T * N,), float("nan"), dtype=torch.float16, device=DEV)
    z2 = z1.clone()
    llmk.linear_rows_norm(x, nw, eps, w, z1, T, H, N)
    llmk.linear_rows(normed, w, z2, T, H, N)
    torch.cuda.synchronize()
    assert np.array_equal(host(z1), host(z2))

    print(f"wide few-rows T={T}: swiglu", flush=True)
    act1 = torch.full((T * inter,), float("nan"), dtype=torch.float16, device=DEV)
    act2 = act1.clone()
    llmk.linear_rows_swiglu(x, nw, eps, wgu, act1, T, H, inter)
    llmk.swiglu_rows(y2, act2, T, inter)
    torch.cuda.synchronize()
    assert np.array_equal(host(act1), host(act2))

    print(f"wide few-rows T={T}: qkv rope scatter", flush=True)
    nh, nkv, hd, ps, max_pages = 240, 8, 64, 16, 4
    qkvdim, kvdim = (nh + 2 * nkv) * hd, nkv * hd
    num_pages = T * max_pages
    wqkv = dev(normal_f16(rng, (qkvdim, H), std=0.05))
    pos = dev_i32(rng.integers(0, max_pages * ps, T))
    tables = dev_i32(rng.permutation(num_pages).reshape(T, max_pages))
    inv = torch.from_numpy(orc.compute_rope_inv_freq(hd, 500000.0, 32.0, 1.0, 4.0,
                                                     8192.0)).to(DEV)
    pools = [dev(np.full(num_pages * ps * kvdim, POISON, np.uint16)) for _ in range(4)]
    q1 = torch.full((T * nh * hd,), float("nan"), dtype=torch.float16, device=DEV)
    q2 = q1.clone()
    llmk.linear_rows_qkv_rope_scatter(x, nw, eps, wqkv, q1, pools[0], pools[1], tables, pos, inv,
                                      T, H, nh, nkv, max_pages)
    qkv = torch.empty(T * qkvdim, dtype=torch.float16, device=DEV)
    llmk.linear_rows(normed, wqkv, qkv, T, H, qkvdim)
    llmk.qkv_rope_scatter(qkv, qkvdim, q2, pools[2], pools[3], tables, pos, inv, T, max_pages,
                          ps, nh, nkv, hd)
    torch.cuda.synchronize()
    assert np.array_equal(host(q1), host(q2))
    assert np.array_equal(host(pools[0]), host(pools[2]))
    assert np.array_equal(host(pools[1]), host(pools[3]))
    assert int((host(pools[0]) != POISON).sum()) == T * kvdim


def test_linear_rows_fused_preconditions(llmk):
    z = torch.zeros(8 * 8192 + 64, dtype=torch.float16, device=DEV)
    w = torch.zeros(64 * 8192, dtype=torch.float16, device=DEV)
    with pytest.raises(llmk.LlmkError, match="shape outside"):
        llmk.linear_rows_norm(z, z, 1e-5, w, z, 2, 16384, 32)  # the norm of rows of 16384
    with pytest.raises(llmk.LlmkError, match="shape outside"):
        llmk.linear_rows_swiglu(z, None, 1e-5, w, z, 2, 512, 6)  # inter % 4 != 0
    with pytest.raises(llmk.LlmkError, match="aligned"):
        llmk.linear_rows_norm(z, z[1:], 1e-5, w, z, 2, 512, 64)  # norm weight misaligned
    llmk.linear_rows_norm(z, z, 1e-5, w, z, 8, 8192, 64)          # 8 rows of 8192: supported
    torch.cuda.synchronize()


def test_linear_after_tuning_matches_oracle(llmk, orc, blas):
    """llmk_blas_tune swaps a shape's algorithm for the fastest timed candidate; the result
    keeps the same bar."""
    T, K, N = 256, 2048, 3072
    rng = np.random.default_rng(0x5EED0205)
    x, w = normal_f16(rng, (T, K)), normal_f16(rng, (N, K), std=0.02)
    dx, dw = dev(x), dev(w)
    y = torch.empty(T * N, dtype=torch.float16, device=DEV)
    llmk.blas_tune(blas, dx, dw, y, T, K, N)
    y.fill_(float("nan"))
    llmk.linear(blas, dx, dw, y, T, K, N)
    torch.cuda.synchronize()
    bad, exact = linear_rule(host(y), orc.linear(x, w, T, K, N, threads=16).ravel())
    assert bad == 0 and exact > 0.9


def test_linear_rejects_bad_arguments(llmk, blas):
    x = torch.zeros(4, 64, dtype=torch.float16, device=DEV)
    with pytest.raises(llmk.LlmkError):
        llmk.linear(blas, x, x, x, 8, 64, 64)          # x holds fewer than T * in values
    st = llmk.lib().llmk_linear(blas.handle, x.data_ptr(), x.data_ptr(), x.data_ptr(), 4, 0, 4,
                                None)
    assert st == llmk.LLMK_ERR_INVALID_VALUE
    assert llmk.lib().llmk_linear(blas.handle, 0, 0, 0, 0, 64, 64, None) == llmk.LLMK_OK


# ------------------------------------------------------------------------------------------
# fused layouts
# ------------------------------------------------------------------------------------------
def test_qkv_rope_scatter_matches_the_separate_operations(llmk, orc):
    rng = np.random.default_rng(0x5EED0210)
    n, nh, nkv, hd, ps, max_pages = 37, 32, 8, 64, 16, 6
    qdim, kvdim = nh * hd, nkv * hd
    ld = qdim + 2 * kvdim + 8  # a padded row stride
    num_pages = n * max_pages
    qkv = normal_f16(rng, (n, ld))
    pos = rng.integers(0, max_pages * ps, n).astype(np.int32)
    tables = rng.permutation(num_pages).astype(np.int32).reshape(n, max_pages)  # distinct slots
    inv = orc.compute_rope_inv_freq(hd, 500000.0, 32.0, 1.0, 4.0, 8192.0)
    q = np.ascontiguousarray(qkv[:, :qdim])
    k = np.ascontiguousarray(qkv[:, qdim:qdim + kvdim])
    v = np.ascontiguousarray(qkv[:, qdim + kvdim:qdim + 2 * kvdim])
    kp = np.full(num_pages * ps * kvdim, POISON, np.uint16)
    vp = kp.copy()
    q_exp = q.copy()
    orc.rope_kv_scatter_batch(q_exp, k, v, kp, vp, tables, pos, inv, n, max_pages, ps, nh, nkv,
                              hd)
    d_kp, d_vp = dev(np.full_like(kp, POISON)), dev(np.full_like(vp, POISON))
    q_out = torch.full((n * qdim,), float("nan"), dtype=torch.float16, device=DEV)
    d_inv = torch.from_numpy(inv).to(DEV)
    llmk.qkv_rope_scatter(dev(qkv), ld, q_out, d_kp, d_vp, dev_i32(tables), dev_i32(pos), d_inv,
                          n, max_pages, ps, nh, nkv, hd)
    torch.cuda.synchronize()
    assert np.array_equal(host(q_out), q_exp.ravel())
    assert np.array_equal(host(d_kp), kp)
    assert np.array_equal(host(d_vp), vp)
    # and the same bits as the unfused GPU entry point on the split buffers
    q2, kp2, vp2 = dev(q), dev(np.full_like(kp, POISON)), dev(np.full_like(vp, POISON))
    llmk.rope_kv_scatter_batch(q2, dev(k), dev(v), kp2, vp2, dev_i32(tables), dev_i32(pos),
                               d_inv, n, max_pages, ps, nh, nkv, hd)
    torch.cuda.synchronize()
    assert np.array_equal(host(q2).ravel(), host(q_out))
    assert np.array_equal(host(kp2), kp) and np.array_equal(host(vp2), vp)


@pytest.mark.parametrize("n,inter", [(19, 8192), (5, 520), (1, 8)])
def test_swiglu_rows_matches_oracle(llmk, orc, n, inter):
    rng = np.random.default_rng(0x5EED0220 + inter)
    gu = normal_f16(rng, (n, 2 * inter))
    gu[0, :8] = np.array([0.0, -0.0, 20.0, -20.0, 88.0, -88.0, 6e-8, -6e-8],
                         np.float16).view(np.uint16)
    exp = orc.swiglu(np.ascontiguousarray(gu[:, :inter]), np.ascontiguousarray(gu[:, inter:]))
    out = torch.full((n * inter + 8,), float("nan"), dtype=torch.float16, device=DEV)
    llmk.swiglu_rows(dev(gu), out, n, inter)
    torch.cuda.synchronize()
    got = host(out)
    assert np.array_equal(got[:n * inter], exp.ravel())
    assert np.all(got[n * inter:] == 0x7E00), "write past the output"


# ------------------------------------------------------------------------------------------
# the engine
# ------------------------------------------------------------------------------------------
def make_engine(llmk, cfg: dict, w: dict, max_rows: int, max_pages: int, num_pages: int):
    weights = importlib.import_module("llmk.weights")
    e = llmk.Engine(llmk.ModelConfig(**cfg), max_rows, max_pages, num_pages)
    tensors = {k: torch.from_numpy(np.ascontiguousarray(v)).to(DEV) if isinstance(v, np.ndarray)
               else v for k, v in w.items()}
    e.set_weights(*weights.engine_layers(tensors, cfg))
    return e


class Session:
    """Sequences with shuffled pages; builds the rows of a step (prefill chunks and decode
    tokens) and runs them through both the engine and the oracle, teacher-forcing both with the
    oracle's greedy tokens."""

    def __init__(self, llmk, orc, cfg, w_engine, w_oracle, n_seqs, max_rows, max_pages,
                 num_pages, seed):
        self.cfg, self.orc = cfg, orc
        self.w = {k: np.asarray(v).view(np.uint16) for k, v in w_oracle.items()}
        self.rng = np.random.default_rng(seed)
        self.max_pages, self.num_pages = max_pages, num_pages
        perm = self.rng.permutation(num_pages).astype(np.int32)
        assert n_seqs * max_pages <= num_pages
        self.tables = perm[:n_seqs * max_pages].reshape(n_seqs, max_pages)
        self.len = np.zeros(n_seqs, np.int64)
        self.engine = make_engine(llmk, cfg, w_engine, max_rows, max_pages, num_pages)
        self.kp, self.vp = oracle_pools(num_pages, cfg)
        self.last = {}

    def step(self, parts):
        """parts: list of (seq, tokens or None); None = one decode row fed with the sequence's
        last greedy token. Returns (engine logits, oracle logits, oracle next) of the last row of
        every part."""
        tok, pos, tab, logit_rows = [], [], [], []
        for s, toks in parts:
            toks = [self.last[s]] if toks is None else list(toks)
            for t in toks:
                tok.append(t)
                pos.append(self.len[s])
                tab.append(self.tables[s])
                self.len[s] += 1
            logit_rows.append(len(tok) - 1)
        tok, pos, tab = np.array(tok, np.int32), np.array(pos, np.int32), np.array(tab, np.int32)
        e = self.engine
        e.set_rows(tok, pos, tab, logit_rows)
        e.forward(len(tok), len(logit_rows))
        torch.cuda.synchronize()
        got = e.logits(len(logit_rows)).numpy().view(np.uint16)
        got_next = e.next_tokens(len(logit_rows)).numpy()
        exp, exp_next, _ = self.orc.engine_forward(self.cfg, self.w, tok, pos, tab, self.kp,
                                                   self.vp, logit_rows, threads=16)
        for (s, _), t in zip(parts, exp_next):
            self.last[s] = int(t)
        return got, got_next, exp, exp_next

    def check_pools(self, llmk):
        written_e, written_o = [], []
        for l in range(self.cfg["n_layers"]):
            for which, pools in ((llmk.BUF_K_POOL, self.kp), (llmk.BUF_V_POOL, self.vp)):
                g = self.engine.pool(which, l).numpy().view(np.uint16).reshape(-1, 16, self.cfg[
                    "n_kv_heads"] * self.cfg["head_dim"])
                o = pools[l].reshape(g.shape)
                we, wo = (g != POISON).any(2), (o != POISON).any(2)
                assert np.array_equal(we, wo), "different pool slots written"
                assert np.all(g[~we] == POISON)
                a = g[we].view(np.float16).astype(np.float64)
                b = o[wo].view(np.float16).astype(np.float64)
                rel = np.linalg.norm(a - b) / np.linalg.norm(b)
                assert rel < 5e-3, (l, which, rel)
                written_e.append(int(we.sum()))
        return written_e


def check_logits(orc, got, got_next, exp, exp_next, what):
    g = got.view(np.float16).astype(np.float64)
    e = exp.view(np.float16).astype(np.float64)
    rel = np.linalg.norm(g - e, axis=1) / np.linalg.norm(e, axis=1)
    top2 = np.sort(e, axis=1)[:, -2:]
    clear = top2[:, 1] - top2[:, 0] > 0.05 * np.abs(top2[:, 1]).clip(1, None)
    print(f"{what}: rel L2 max {rel.max():.2e} exact {100 * np.mean(got == exp):.1f}% "
          f"clear {clear.sum()}/{len(clear)}", flush=True)
    assert rel.max() < 5e-3, rel
    assert np.array_equal(got_next[clear], exp_next[clear])
    # the engine's own argmax is exactly the argmax of its logits
    assert np.array_equal(got_next, orc.argmax_rows(got, got.shape[0], got.shape[1]))


@pytest.mark.parametrize("cfg", [TINY, dict(TINY, n_heads=12, n_kv_heads=3)],
                         ids=["1_kv_head", "3_kv_heads"])
def test_engine_matches_oracle_small_model(llmk, orc, cfg):
    """Prefill and decode rows through the engine against the oracle; with one kv head, and
    with three (a count the attention runs as a partly idle group of 8)."""
    w = tiny_weights(0x5EED0230, embed_std=0.5, cfg=cfg)
    rng = np.random.default_rng(0x5EED0231)
    s = Session(llmk, orc, cfg, w, w, n_seqs=3, max_rows=64, max_pages=8, num_pages=30,
                seed=0x5EED0232)
    V = cfg["vocab"]
    prompts = [rng.integers(0, V, L) for L in (20, 33, 7)]
    # step 1: two prompts in one batch (53 rows); step 2: the third prompt plus two decode rows;
    # then decode steps for all three
    plan = [[(0, prompts[0]), (1, prompts[1])], [(2, prompts[2]), (0, None), (1, None)]]
    plan += [[(0, None), (1, None), (2, None)] for _ in range(5)]
    for i, parts in enumerate(plan):
        check_logits(orc, *s.step(parts), f"step {i}")
    written = s.check_pools(llmk)
    assert written[0] == int(s.len.sum())  # one slot per row ever run


WIDE = dict(TINY, hidden=512, n_heads=8, n_kv_heads=2, inter=1024, vocab=1000)
WIDE6 = dict(WIDE, n_heads=24, n_kv_heads=6)


@pytest.mark.parametrize("n,cfg", [(1, WIDE), (3, WIDE), (8, WIDE), (3, WIDE6)],
                         ids=["1", "3", "8", "3_six_kv_heads"])
def test_engine_fused_few_rows_pass_gives_the_bits_of_the_unfused_pass(llmk, orc, n, cfg):
    """A decode step of n <= 8 rows runs the fused few-rows projections (norms, RoPE + scatter,
    SwiGLU and residual adds inside the projections). It must reproduce the unfused pass bit for
    bit: logits, greedy tokens, residual stream and every pool of every layer."""
    w = tiny_weights(0x5EED0250, embed_std=0.5, cfg=cfg)
    num_pages, max_pages = 64, 8
    e = make_engine(llmk, cfg, w, 16, max_pages, num_pages)
    rng = np.random.default_rng(0x5EED0251 + n)
    tables = rng.permutation(num_pages).astype(np.int32)[:n * max_pages].reshape(n, max_pages)
    pos = rng.integers(0, max_pages * 16, n).astype(np.int32)
    tok = rng.integers(0, cfg["vocab"], n).astype(np.int32)
    kvdim = cfg["n_kv_heads"] * cfg["head_dim"]
    fill = torch.randn(num_pages * 16 * kvdim, device=DEV).half()

    def run(fuse):
        e.set_option(llmk.ENGINE_FUSE_FEW_ROWS, fuse)
        for l in range(cfg["n_layers"]):
            for which in (llmk.BUF_K_POOL, llmk.BUF_V_POOL):
                e.write_pool(which, l, fill)
        e.set_rows(tok, pos, tables)
        e.forward(n)
        torch.cuda.synchronize()
        got = [e.logits(n), e.next_tokens(n), e.residual(n)]
        got += [e.pool(wh, l) for l in range(cfg["n_layers"])
                for wh in (llmk.BUF_K_POOL, llmk.BUF_V_POOL)]
        return [t.clone().view(torch.int16) if t.dtype == torch.float16 else t.clone()
                for t in got]

    fused, plain = run(1), run(0)
    assert not torch.isnan(fused[0].view(torch.float16)).any()
    for a, b in zip(fused, plain):
        assert torch.equal(a, b)


def test_engine_split_rule_short_contexts_take_one_split(llmk, orc):
    """num_splits = 0 lets the engine choose: one attention split (no merge launch) when every
    row's attention spans at most 4 pages, else the reference's rule, target blocks / (rows x kv
    heads) capped at the table's pages. The automatic pass must give the bits of that explicit
    split count, eagerly and through the graph cache (first use eager, then captured and
    replayed: the cache is keyed by the resolved count)."""
    w = tiny_weights(0x5EED0260, embed_std=0.5, cfg=WIDE)
    num_pages, max_pages, n = 96, 16, 3
    e = make_engine(llmk, WIDE, w, 16, max_pages, num_pages)
    rng = np.random.default_rng(0x5EED0261)
    tables = rng.permutation(num_pages).astype(np.int32)[:n * max_pages].reshape(n, max_pages)
    tok = rng.integers(0, WIDE["vocab"], n).astype(np.int32)
    kvdim = WIDE["n_kv_heads"] * WIDE["head_dim"]
    fill = torch.randn(num_pages * 16 * kvdim, device=DEV).half()
    long_rule = min(65536 // (n * WIDE["n_kv_heads"]), max_pages, 32)
    s = torch.cuda.Stream()
    for pos, splits in ((np.array([0, 37, 63], np.int32), 1),            # spans 1, 3, 4 pages
                        (np.array([5, 64, 255], np.int32), long_rule)):  # spans up to 16
        def run(**kw):
            for l in range(WIDE["n_layers"]):
                for which in (llmk.BUF_K_POOL, llmk.BUF_V_POOL):
                    e.write_pool(which, l, fill)
            e.set_rows(tok, pos, tables)
            if kw.pop("graph", False):
                with torch.cuda.stream(s):
                    e.forward_graph(n, stream=s, **kw)
            else:
                e.forward(n, **kw)
            torch.cuda.synchronize()
            return e.logits(n).view(torch.int16).clone()

        explicit = run(num_splits=splits)
        assert not torch.isnan(explicit.view(torch.float16)).any()
        assert torch.equal(run(), explicit), (pos, splits)
        for rep in range(3):  # eager, captured, replayed
            assert torch.equal(run(graph=True), explicit), (pos, splits, rep)


def test_engine_graph_replays_match_eager(llmk, orc):
    w = tiny_weights(0x5EED0240, embed_std=0.5)
    e = make_engine(llmk, TINY, w, 16, 4, 64)
    rng = np.random.default_rng(0x5EED0241)
    n = 12  # two prompts, of 5 and 7 tokens, in one batch of rows
    tok = rng.integers(0, TINY["vocab"], n).astype(np.int32)
    pos = np.array(list(range(5)) + list(range(7)), np.int32)
    pages = rng.permutation(64).astype(np.int32).reshape(16, 4)
    tab = np.array([pages[0]] * 5 + [pages[1]] * 7, np.int32)
    e.set_rows(tok, pos, tab)
    # A pass captured with num_splits = 0 takes the capacity rule (the rows' short contexts
    # would give one split): the eager reference uses that count explicitly.
    splits = min(65536 // (n * TINY["n_kv_heads"]), 4, 32)
    e.forward(n, num_splits=splits)   # eager: chooses the GEMM plans before capture
    torch.cuda.synchronize()
    ref_logits = e.logits(n).view(torch.int16).clone()
    ref_pool = e.pool(llmk.BUF_K_POOL, 1).view(torch.int16).clone()
    assert not torch.isnan(ref_logits.view(torch.float16)).any()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        e.forward(n, stream=s)        # warm on the capture stream too
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        e.forward(n)
    junk = torch.randn(1 << 20, device=DEV)
    for r in range(4):
        e.reset_pools()
        torch.cuda.synchronize()
        junk.mul_(1.0001)             # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(e.logits(n).view(torch.int16), ref_logits), f"replay {r}"
        assert torch.equal(e.pool(llmk.BUF_K_POOL, 1).view(torch.int16), ref_pool), f"replay {r}"


def test_engine_loads_the_reference_weight_format(llmk, tmp_path):
    weights = importlib.import_module("llmk.weights")
    w = tiny_weights(0x5EED0250, embed_std=0.5)
    weights.write_weights_dir(str(tmp_path), w)
    a = make_engine(llmk, TINY, w, 8, 2, 16)
    b = llmk.Engine(llmk.ModelConfig(**TINY), 8, 2, 16)
    b.load_weights(str(tmp_path))
    tok = np.arange(8, dtype=np.int32) * 7
    pos = np.arange(8, dtype=np.int32)
    tab = np.tile(np.array([[3, 5]], np.int32), (8, 1))
    for e in (a, b):
        e.set_rows(tok, pos, tab)
        e.forward(8)
    torch.cuda.synchronize()
    assert torch.equal(a.logits(8), b.logits(8))
    # a missing directory, and a config whose shapes the files do not have
    with pytest.raises(llmk.LlmkError) as ei:
        b.load_weights(str(tmp_path / "nowhere"))
    assert ei.value.status == llmk.LLMK_ERR_IO
    c = llmk.Engine(llmk.ModelConfig(**dict(TINY, vocab=TINY["vocab"] + 8)), 8, 2, 16)
    with pytest.raises(llmk.LlmkError) as ei:
        c.load_weights(str(tmp_path))
    assert ei.value.status == llmk.LLMK_ERR_SHAPE


def test_engine_rejects_rows_that_address_outside_its_buffers(llmk):
    e = make_engine(llmk, TINY, tiny_weights(0x5EED0260), 4, 2, 8)
    ok = dict(tokens=[1, 2], positions=[0, 17], block_tables=[[0, 1], [2, 3]])
    e.set_rows(**ok)
    bad = [dict(ok, tokens=[1, TINY["vocab"]]), dict(ok, tokens=[-1, 2]),
           dict(ok, positions=[0, 32]), dict(ok, positions=[-1, 0]),
           dict(ok, block_tables=[[0, 1], [2, 8]]), dict(ok, block_tables=[[-1, 1], [2, 3]])]
    for b in bad:
        with pytest.raises(llmk.LlmkError):
            e.set_rows(**b)
    with pytest.raises(llmk.LlmkError):
        e.set_rows(**ok, logit_rows=[2])
    with pytest.raises(llmk.LlmkError):
        e.forward(5)                                   # more rows than max_rows


def test_engine_rejects_a_pass_over_rows_not_uploaded(llmk):
    """A pass may not ask for more rows (or logit rows) than the last set_rows uploaded: the
    device copies past them were never checked. The call fails before any launch, so the
    outputs of the previous pass stay as they were."""
    e = make_engine(llmk, TINY, tiny_weights(0x5EED0270, embed_std=0.5), 4, 2, 8)
    s = torch.cuda.Stream()
    with pytest.raises(llmk.LlmkError) as ei:
        e.forward(1)                                   # nothing uploaded yet
    assert ei.value.status == llmk.LLMK_ERR_INVALID_VALUE
    e.set_rows([1, 2, 3], [0, 5, 17], [[0, 1], [2, 3], [4, 5]], logit_rows=[2])
    e.forward(3, 1)
    torch.cuda.synchronize()
    before = e.logits(1).view(torch.int16).clone()
    e.set_rows([4, 5], [0, 0], [[0, 1], [2, 3]])     # each row reads only its own position
    for n, nl in ((3, -1), (2, 1), (3, 1)):
        with pytest.raises(llmk.LlmkError) as ei:
            e.forward(n, nl)
        assert ei.value.status == llmk.LLMK_ERR_INVALID_VALUE
        with pytest.raises(llmk.LlmkError) as ei:
            e.forward_graph(n, nl, stream=s)
        assert ei.value.status == llmk.LLMK_ERR_INVALID_VALUE
    torch.cuda.synchronize()
    assert torch.equal(e.logits(1).view(torch.int16), before)
    e.forward(2)                                       # the rows that were uploaded
    torch.cuda.synchronize()
    assert not torch.isnan(e.logits(2).float()).any()


def test_engine_rejects_a_head_dim_other_than_64(llmk):
    """The attention kernels take head_dim 64 only: a model of another head size is refused when
    the engine is created."""
    with pytest.raises(llmk.LlmkError) as ei:
        llmk.Engine(llmk.ModelConfig(**dict(TINY, head_dim=128)), 4, 2, 8)
    assert ei.value.status == llmk.LLMK_ERR_SHAPE


def test_engine_matches_oracle_llama_3_2_1b_shape(llmk, orc):
    """The Llama-3.2-1B shape (16 layers, vocab 128256) with seeded random weights: two prompts
    and one decode step."""
    weights = importlib.import_module("llmk.weights")
    cfg = llmk.ModelConfig().as_dict()
    w_dev = weights.random_weights(cfg, 0x5EED0270, device=DEV, std=0.02, embed_std=0.5)
    w_host = {k: v.cpu().numpy() for k, v in w_dev.items()}
    s = Session(llmk, orc, cfg, w_dev, w_host, n_seqs=2, max_rows=16, max_pages=4,
                num_pages=12, seed=0x5EED0271)
    del w_dev
    rng = np.random.default_rng(0x5EED0272)
    check_logits(orc, *s.step([(0, rng.integers(0, cfg["vocab"], 5)),
                               (1, rng.integers(0, cfg["vocab"], 9))]), "1B prefill")
    check_logits(orc, *s.step([(0, None), (1, None)]), "1B decode")
    s.check_pools(llmk)
