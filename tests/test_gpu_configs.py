"""GPU parity at the benchmark configurations' full sizes (the oracle finishes each in seconds),
the 16-layer decode-step pass (config 5) checked layer by layer, HIP-graph replay of that pass,
and the engine-style C++ drop-in test."""
import os
import subprocess

import numpy as np
import pytest
import torch

from _helpers import EPS, POISON, ROPE, assert_tol

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
THREADS = min(16, os.cpu_count() or 1)


def host(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def host_i32(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy().astype(np.int32)


@pytest.fixture(scope="module")
def wl(llmk):
    import llmk.workloads as w
    return w


@pytest.fixture(scope="module")
def inv(llmk, orc):
    hd = 64
    inv_h = orc.compute_rope_inv_freq(hd, ROPE["theta"], ROPE["factor"], ROPE["low"],
                                      ROPE["high"], ROPE["orig"])
    inv_lib = np.array(llmk.compute_rope_inv_freq(hd, ROPE["theta"], ROPE["factor"], ROPE["low"],
                                                  ROPE["high"], ROPE["orig"]), np.float32)
    assert np.array_equal(inv_h.view(np.uint32), inv_lib.view(np.uint32))
    return inv_h, torch.from_numpy(inv_lib).to(DEV)


def test_config1_rmsnorm_16x2048(llmk, orc, wl):
    d = wl.add_rmsnorm_inputs(rows=16, seed=wl.SEED_BASE + 1)
    llmk.rmsnorm(d["x"], d["w"], d["out"], 16, 2048, EPS)
    exp = orc.rmsnorm(host(d["x"]), host(d["w"]), 16, 2048, EPS)
    assert_tol(orc.compare(host(d["out"]), exp), 0.99, "config 1")


def test_config2_add_rmsnorm_8192x2048(llmk, orc, wl):
    d = wl.add_rmsnorm_inputs()
    r, x, w = host(d["residual"]), host(d["x"]), host(d["w"])
    llmk.add_rmsnorm(d["residual"], d["x"], d["w"], d["out"], d["rows"], d["hidden"], EPS)
    o_exp = orc.add_rmsnorm(r, x, w, d["rows"], d["hidden"], EPS, threads=THREADS)
    assert np.array_equal(host(d["residual"]), r), "updated residual must be bit-exact"
    cmp = orc.compare(host(d["out"]), o_exp)
    print(f"config 2 out: {cmp}")
    assert_tol(cmp, 0.99, "config 2")


def test_config3_rope_8192_tokens(llmk, orc, wl, inv):
    d = wl.rope_inputs(inv_freq=inv[1])
    q, k, pos = host(d["q"]), host(d["k"]), host_i32(d["positions"])
    assert pos.min() >= 0 and pos.max() < wl.MAX_POS
    llmk.rope_apply(d["q"], d["k"], d["positions"], d["inv_freq"], d["T"], d["nh"], d["nkv"],
                    d["hd"])
    orc.rope_apply(q, k, pos, inv[0], d["T"], d["nh"], d["nkv"], d["hd"], threads=THREADS)
    cq, ck = orc.compare(host(d["q"]), q), orc.compare(host(d["k"]), k)
    print(f"config 3 Q: {cq}\nconfig 3 K: {ck}")
    assert_tol(cq, 0.995, "config 3 Q")
    assert_tol(ck, 0.995, "config 3 K")


def test_config3_rope_position_zero_is_the_identity(llmk, wl, inv):
    """A size-independent property at config 3's full size: with every position 0, cos = 1 and
    sin = 0, so x1' = fp16(r16(x1) - r16(x2 * 0)) = x1 for finite inputs and Q and K keep every
    bit. (The oracle comparison above covers the other positions.)"""
    d = wl.rope_inputs(inv_freq=inv[1])
    d["positions"].zero_()
    q0, k0 = d["q"].clone(), d["k"].clone()
    llmk.rope_apply(d["q"], d["k"], d["positions"], d["inv_freq"], d["T"], d["nh"], d["nkv"],
                    d["hd"])
    torch.cuda.synchronize()
    assert torch.equal(d["q"].view(torch.int16), q0.view(torch.int16))
    assert torch.equal(d["k"].view(torch.int16), k0.view(torch.int16))


def test_config4_swiglu_8192x8192(llmk, orc, wl):
    d = wl.swiglu_inputs()
    g, u = host(d["gate"]), host(d["up"])
    llmk.swiglu(d["gate"], d["up"], d["out"], d["n"])
    cmp = orc.compare(host(d["out"]), orc.swiglu(g, u, threads=THREADS))
    print(f"config 4 swiglu: {cmp}")
    assert_tol(cmp, 0.995, "config 4")


def test_config4_embedding_8192_of_128256(llmk, orc, wl):
    d = wl.embedding_inputs()
    llmk.embedding_lookup(d["table"], d["ids"], d["out"], d["n"], d["hidden"])
    ids = host_i32(d["ids"])
    table = host(d["table"]).reshape(-1, d["hidden"])
    assert np.array_equal(host(d["out"]), orc.embedding_lookup(table, ids, d["hidden"],
                                                               threads=THREADS))


def _check_decode_pass(orc, wl, p, inv_h, expected_residual_in):
    """Checks every layer of a finished pass against the oracle; returns the final residual."""
    n, hidden, kvdim = p.n, wl.HIDDEN, wl.N_KV * wl.HEAD_DIM
    rows = torch.from_numpy(p.pool_rows()).to(DEV)
    pos = (p.lens - 1).astype(np.int32)
    res = expected_residual_in.copy()
    for l, L in enumerate(p.per_layer):
        normed = orc.add_rmsnorm(res, host(L["x"]), host(L["norm_w"]), n, hidden, EPS)
        assert_tol(orc.compare(host(L["normed"]), normed), 0.99, f"layer {l} normed")
        q_e, k_e = host(L["q_in"]), host(L["k"])
        orc.rope_apply(q_e, k_e, pos, inv_h, n, wl.N_HEADS, wl.N_KV, wl.HEAD_DIM)
        assert_tol(orc.compare(host(L["q"]), q_e), 0.995, f"layer {l} q")
        kp = L["k_pool"].view(-1, kvdim)
        vp = L["v_pool"].view(-1, kvdim)
        assert_tol(orc.compare(host(kp.index_select(0, rows)), k_e.reshape(n, kvdim)), 0.995,
                   f"layer {l} K pool")
        assert np.array_equal(host(vp.index_select(0, rows)), host(L["v"]).reshape(n, kvdim))
        poison = torch.tensor(POISON, dtype=torch.int16, device=DEV)
        for pool in (kp, vp):
            changed = (pool.view(torch.int16) != poison).any(dim=1)
            assert int(changed.sum()) == n, f"layer {l}: rows outside the addressed slots changed"
        if "x2" in L:  # the layer's second add + RMSNorm, after the scatter
            normed2 = orc.add_rmsnorm(res, host(L["x2"]), host(L["norm_w2"]), n, hidden, EPS)
            assert_tol(orc.compare(host(L["normed2"]), normed2), 0.99, f"layer {l} normed2")
        act = orc.swiglu(host(L["gate"]), host(L["up"]), threads=THREADS)
        assert_tol(orc.compare(host(L["act"]), act), 0.995, f"layer {l} act")
    return res


def test_config5_decode_pass_16_layers_256_seqs(llmk, orc, wl, inv):
    p = wl.decode_pass_inputs(inv[1])
    for L in p.per_layer:
        L["q_in"] = L["q"].clone()
    dp = llmk.DecodeNonGemmPass(p.table, p.token_ids, p.residual, p.block_tables, p.positions,
                                p.inv_freq, p.per_layer, n_heads=wl.N_HEADS,
                                n_kv_heads=wl.N_KV, head_dim=wl.HEAD_DIM, inter=wl.INTER,
                                page_size=wl.PAGE, max_pages=p.max_pages, eps=EPS)
    dp.run()
    torch.cuda.synchronize()
    ids = host_i32(p.token_ids)
    emb = host(p.table.index_select(0, p.token_ids.long()))
    assert np.array_equal(emb, host(p.table).reshape(-1, wl.HIDDEN)[ids])
    final = _check_decode_pass(orc, wl, p, inv[0], emb)
    assert np.array_equal(host(p.residual), final), "residual chain must be bit-exact"


def test_decode_pass_with_both_norms_per_layer(llmk, orc, wl, inv):
    """The real layer's two add + RMSNorm pairs (the reference adds the attention output and
    normalises again before the MLP, engine/batched.cu:64-66): 4 layers x 256 sequences against
    the oracle layer by layer, the residual chain bit-exact; then the one-launch-per-layer pass
    on the same inputs gives every output's bits."""
    kw = dict(layers=4, seed=wl.SEED_BASE + 61, two_norms=True)
    p = wl.decode_pass_inputs(inv[1], **kw)
    for L in p.per_layer:
        L["q_in"] = L["q"].clone()
    dp = llmk.DecodeNonGemmPass(p.table, p.token_ids, p.residual, p.block_tables, p.positions,
                                p.inv_freq, p.per_layer, n_heads=wl.N_HEADS,
                                n_kv_heads=wl.N_KV, head_dim=wl.HEAD_DIM, inter=wl.INTER,
                                page_size=wl.PAGE, max_pages=p.max_pages, eps=EPS)
    dp.run()
    torch.cuda.synchronize()
    emb = host(p.table.index_select(0, p.token_ids.long()))
    final = _check_decode_pass(orc, wl, p, inv[0], emb)
    assert np.array_equal(host(p.residual), final), "residual chain must be bit-exact"
    (pa, da), (pb, db) = _pass_pair(llmk, wl, inv, **kw)
    _same_pass_bits(pa, da, pb, db)
    # The second pair goes in every layer or in none: a layer with only some of its tensors,
    # or layers that disagree, are refused before anything runs.
    partial = [dict(L) for L in p.per_layer]
    del partial[2]["normed2"]
    mixed = [dict(L) for L in p.per_layer]
    for key in ("x2", "norm_w2", "normed2"):
        del mixed[0][key]
    for layers in (partial, mixed):
        with pytest.raises(llmk.LlmkError):
            llmk.DecodeNonGemmPass(p.table, p.token_ids, p.residual, p.block_tables, p.positions,
                                   p.inv_freq, layers, n_heads=wl.N_HEADS, n_kv_heads=wl.N_KV,
                                   head_dim=wl.HEAD_DIM, inter=wl.INTER, page_size=wl.PAGE,
                                   max_pages=p.max_pages, eps=EPS)


def test_decode_pass_hip_graph_replays(llmk, orc, wl, inv):
    """The pass captured into a HIP graph (through torch.cuda.CUDAGraph) and replayed three
    times, with eager work and synchronisation between replays, gives the eager result each
    time."""
    p = wl.decode_pass_inputs(inv[1], n=64, layers=3, max_pages=32, seed=wl.SEED_BASE + 55)
    state0 = [(L["q"].clone(), L["k_pool"].clone(), L["v_pool"].clone()) for L in p.per_layer]
    dp = llmk.DecodeNonGemmPass(p.table, p.token_ids, p.residual, p.block_tables, p.positions,
                                p.inv_freq, p.per_layer, n_heads=wl.N_HEADS,
                                n_kv_heads=wl.N_KV, head_dim=wl.HEAD_DIM, inter=wl.INTER,
                                page_size=wl.PAGE, max_pages=p.max_pages, eps=EPS)

    def reset():
        for L, (q0, kp0, vp0) in zip(p.per_layer, state0):
            L["q"].copy_(q0)
            L["k_pool"].copy_(kp0)
            L["v_pool"].copy_(vp0)
            L["normed"].zero_()
            L["act"].zero_()
        p.residual.zero_()

    def snapshot():
        torch.cuda.synchronize()
        outs = [host(p.residual)]
        for L in p.per_layer:
            outs += [host(L[k]) for k in ("normed", "q", "k_pool", "v_pool", "act")]
        return outs

    dp.run()
    eager = snapshot()
    reset()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        dp.run()  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        dp.run()
    for i in range(3):
        reset()
        torch.cuda.synchronize()
        _ = torch.randn(1 << 20, device=DEV).sum().item()  # unrelated eager work in between
        graph.replay()
        got = snapshot()
        for j, (a, b) in enumerate(zip(got, eager)):
            assert np.array_equal(a, b), f"replay {i}, output {j} differs from the eager pass"


def _pass_pair(llmk, wl, inv, **kw):
    """Two identical input sets of the decode pass (same seed) and their pass objects."""
    out = []
    for _ in range(2):
        p = wl.decode_pass_inputs(inv[1], **kw)
        dp = llmk.DecodeNonGemmPass(p.table, p.token_ids, p.residual, p.block_tables,
                                    p.positions, p.inv_freq, p.per_layer,
                                    n_heads=kw.get("n_heads", wl.N_HEADS),
                                    n_kv_heads=kw.get("n_kv", wl.N_KV), head_dim=wl.HEAD_DIM,
                                    inter=kw.get("inter", wl.INTER), page_size=wl.PAGE,
                                    max_pages=p.max_pages, eps=EPS)
        out.append((p, dp))
    return out


def _same_pass_bits(pa, da, pb, db, method="run_layers"):
    """Runs the op-by-op pass on set a and, on set b (whose outputs start as NaN), the pass
    ``method`` names (one launch per layer, or the fused one), and compares every output bit for
    bit."""
    for L in pa.per_layer:
        L["act"].zero_()
        L["normed"].zero_()
    for L in pb.per_layer:
        L["act"].fill_(float("nan"))
        L["normed"].fill_(float("nan"))
        if "normed2" in L:
            L["normed2"].fill_(float("nan"))
    pb.residual.fill_(float("nan"))
    da.run()
    getattr(db, method)()
    torch.cuda.synchronize()
    assert torch.equal(pa.residual.view(torch.int16), pb.residual.view(torch.int16))
    for l, (A, B) in enumerate(zip(pa.per_layer, pb.per_layer)):
        for key in ("normed", "q", "act", "k_pool", "v_pool", "normed2"):
            if key in A:
                assert torch.equal(A[key].view(torch.int16), B[key].view(torch.int16)), (l, key)


@pytest.mark.parametrize("shape", [dict(n=64, layers=3, max_pages=32, seed=0x5EED0000 + 56),
                                   dict(n=37, layers=2, max_pages=8, seed=0x5EED0000 + 57),
                                   dict()])
def test_decode_pass_one_launch_per_layer_gives_the_bits_of_the_op_by_op_pass(llmk, wl, inv,
                                                                            shape):
    """llmk_decode_nongemm_pass_layers (each layer's norm rows, RoPE + scatter tokens and SwiGLU
    chunks in one launch, the embedding gather fused into the first residual add) against
    llmk_decode_nongemm_pass on identical inputs: the residual, and every layer's normed rows,
    rotated Q, SwiGLU output and whole K and V pools, bit for bit. Shapes: a small pass, a
    ragged one (37 sequences: a partial last SwiGLU chunk), and config 5 (256 x 16 layers)."""
    (pa, da), (pb, db) = _pass_pair(llmk, wl, inv, **shape)
    _same_pass_bits(pa, da, pb, db)


# (hidden, n_heads, n_kv, inter): every row width the launch takes (hidden / 512 = 1, 2, 4, 8,
# 16 vectors per lane) and every RoPE task count it compiles (16-byte vectors per token over 64
# lanes: 2, 3, 8, 10, 16 and 12 tasks, run as 6, 6, 8, 12, 16 and 12).
PASS_MODELS = [(512, 8, 2, 1376), (1024, 16, 4, 2816), (2048, 48, 8, 5632),
               (4096, 64, 8, 11008), (8192, 112, 8, 8192), (2048, 64, 16, 4096)]


@pytest.mark.parametrize("model,two_norms",
                         [(m, False) for m in PASS_MODELS] + [(PASS_MODELS[1], True),
                                                              (PASS_MODELS[4], True)],
                         ids=lambda v: ("h%d_q%d_kv%d" % v[:3]) if isinstance(v, tuple)
                         else ("two_norms" if v else "one_norm"))
def test_decode_pass_one_launch_per_layer_across_model_shapes(llmk, wl, inv, model, two_norms):
    """The one-launch-per-layer pass against the op-by-op pass (each of whose kernels is checked
    against the oracle on its own) at other model dimensions than config 5's: 29 sequences
    (a partial last SwiGLU chunk), 2 layers, bit for bit; with both of a layer's norms at two of
    the row widths."""
    hidden, nh, nkv, inter = model
    kw = dict(n=29, layers=2, max_pages=8, seed=0x5EED0000 + 58, hidden=hidden, n_heads=nh,
              n_kv=nkv, inter=inter, vocab=1000, two_norms=two_norms)
    (pa, da), (pb, db) = _pass_pair(llmk, wl, inv, **kw)
    _same_pass_bits(pa, da, pb, db)


def test_decode_pass_one_launch_per_layer_refuses_other_shapes(llmk, wl, inv):
    """Shapes outside the single launch's (a head_dim other than 64, a hidden size that is not
    512 times a power of two up to 8192) are refused with LLMK_ERR_UNSUPPORTED, and the
    op-by-op pass still takes them."""
    p = wl.decode_pass_inputs(inv[1], n=5, layers=1, max_pages=4, seed=0x5EED0000 + 59,
                              hidden=1536, vocab=100)
    dp = llmk.DecodeNonGemmPass(p.table, p.token_ids, p.residual, p.block_tables, p.positions,
                                p.inv_freq, p.per_layer, n_heads=wl.N_HEADS,
                                n_kv_heads=wl.N_KV, head_dim=wl.HEAD_DIM, inter=wl.INTER,
                                page_size=wl.PAGE, max_pages=p.max_pages, eps=EPS)
    with pytest.raises(llmk.LlmkError) as err:
        dp.run_layers()
    assert err.value.status == llmk.LLMK_ERR_UNSUPPORTED
    dp.run()
    torch.cuda.synchronize()
    assert torch.isfinite(p.residual).all()


@pytest.mark.parametrize("shape", [dict(n=64, layers=3, max_pages=32, seed=0x5EED0000 + 60),
                                   dict(n=37, layers=1, max_pages=8, seed=0x5EED0000 + 61),
                                   dict(n=29, layers=19, max_pages=8, seed=0x5EED0000 + 62),
                                   dict()],
                         ids=["64x3", "37x1", "29x19_two_launches", "config5"])
def test_decode_pass_fused_gives_the_bits_of_the_op_by_op_pass(llmk, wl, inv, shape):
    """llmk_decode_nongemm_pass_fused (one launch per 16 layers: each sequence's residual chain
    through every layer by one wave, beside every layer's RoPE + scatter tokens and SwiGLU
    chunks) against llmk_decode_nongemm_pass: residual, normed rows, rotated Q, SwiGLU output
    and whole K and V pools of every layer, bit for bit. Shapes: a small pass, one layer of 37
    sequences (partial last SwiGLU chunk), 19 layers (a launch of 16 and one of 3, the second
    starting from the residual the first left), and config 5 (256 x 16: one launch)."""
    (pa, da), (pb, db) = _pass_pair(llmk, wl, inv, **shape)
    _same_pass_bits(pa, da, pb, db, "run_fused")


@pytest.mark.parametrize("model,two_norms",
                         [(m, False) for m in PASS_MODELS if m[0] <= 4096]
                         + [(PASS_MODELS[0], True), (PASS_MODELS[1], True),
                            (PASS_MODELS[2], True), (PASS_MODELS[3], True)],
                         ids=lambda v: ("h%d_q%d_kv%d" % v[:3]) if isinstance(v, tuple)
                         else ("two_norms" if v else "one_norm"))
def test_decode_pass_fused_across_model_shapes(llmk, wl, inv, model, two_norms):
    """The fused pass against the op-by-op pass at every row width it takes (hidden 512-4096:
    1, 2, 4, 8 vectors per lane, each with its own prefetch depth) and every RoPE task count,
    with one and with both of a layer's norms: 29 sequences, 3 layers, bit for bit."""
    hidden, nh, nkv, inter = model
    kw = dict(n=29, layers=3, max_pages=8, seed=0x5EED0000 + 63, hidden=hidden, n_heads=nh,
              n_kv=nkv, inter=inter, vocab=1000, two_norms=two_norms)
    (pa, da), (pb, db) = _pass_pair(llmk, wl, inv, **kw)
    _same_pass_bits(pa, da, pb, db, "run_fused")


def test_decode_pass_fused_two_norms_config5(llmk, wl, inv):
    """The fused pass with both of the real layer's add + RMSNorm pairs, at config 5's shape
    (256 sequences, 16 layers, one launch), against the op-by-op pass, bit for bit."""
    (pa, da), (pb, db) = _pass_pair(llmk, wl, inv, two_norms=True)
    _same_pass_bits(pa, da, pb, db, "run_fused")


def test_decode_pass_fused_refuses_wide_rows(llmk, wl, inv):
    """Rows wider than 4096 (hidden 8192) are refused by the fused pass with
    LLMK_ERR_UNSUPPORTED; the one-launch-per-layer pass takes them."""
    hidden, nh, nkv, inter = PASS_MODELS[4]
    p = wl.decode_pass_inputs(inv[1], n=5, layers=1, max_pages=4, seed=0x5EED0000 + 64,
                              hidden=hidden, n_heads=nh, n_kv=nkv, inter=inter, vocab=100)
    dp = llmk.DecodeNonGemmPass(p.table, p.token_ids, p.residual, p.block_tables, p.positions,
                                p.inv_freq, p.per_layer, n_heads=nh, n_kv_heads=nkv,
                                head_dim=wl.HEAD_DIM, inter=inter, page_size=wl.PAGE,
                                max_pages=p.max_pages, eps=EPS)
    with pytest.raises(llmk.LlmkError) as err:
        dp.run_fused()
    assert err.value.status == llmk.LLMK_ERR_UNSUPPORTED
    dp.run_layers()
    torch.cuda.synchronize()
    assert torch.isfinite(p.residual).all()


def test_cpp_dropin_binary():
    """Engine-style C++ through llmk.hpp (the reference's launcher names and argument lists)."""
    exe = os.path.join(ROOT, "tests", "cpp", "llmk_dropin_test")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=100)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ALL PASSED" in r.stdout
