"""Pins the CPU oracle before it is trusted as the checker of the HIP kernels.

Each oracle function is checked against something other than its own formula: Hugging Face's
modules (tests/golden/hf_goldens.npz), the reference's own known-answer test, numpy, the host's
F16C converter, closed forms and invariants. The "mutant" tests show that the fixtures and the
criteria used here reject plausible mistakes (a dropped rounding step, a wrong pairing).
"""
import numpy as np
import pytest

from _helpers import (ATTN_LENS, EPS, POISON, ROPE, assert_tol, attention_case, attention_f64,
                      goldens, normal_f16, shuffled_page_tables, uniform_f16)


def f16(bits):
    return np.asarray(bits).view(np.float16)


# --------------------------------------------------------------------------------------------
# binary16 conversions
# --------------------------------------------------------------------------------------------
def test_h2f_all_halves_match_numpy(orc):
    allh = np.arange(65536, dtype=np.uint16)
    mine = orc.h2f(allh)
    ref = allh.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(mine), nan)
    assert np.array_equal(mine.view(np.uint32)[~nan], ref.view(np.uint32)[~nan])


def test_f2h_rounding_boundaries_match_numpy(orc):
    # every midpoint between adjacent positive halves, and the floats just around it
    h = np.arange(0, 0x7C00, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    hi[-1] = 65536.0
    mid = ((lo + hi) / 2).astype(np.float32)  # exact: midpoints have <= 12 significant bits
    cands = np.concatenate([mid, np.nextafter(mid, np.float32(np.inf)),
                            np.nextafter(mid, np.float32(0)), lo.astype(np.float32)])
    cands = np.concatenate([cands, -cands, np.array([np.inf, -np.inf, 65520.0, 65519.996,
                                                     1e-8, 2.98e-8, 2.9802322e-8, 3e-8],
                                                    dtype=np.float32)])
    with np.errstate(over="ignore"):
        ref = cands.astype(np.float16).view(np.uint16)
    assert np.array_equal(orc.f2h(cands), ref)


def test_f2h_random_bit_patterns_match_numpy(orc):
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2 ** 32, 2_000_000, dtype=np.uint64).astype(np.uint32)
    vals = bits.view(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    mine = orc.f2h(vals)
    nan = np.isnan(vals)
    assert np.array_equal(mine[~nan], ref[~nan])
    assert np.all(np.isnan(mine[nan].view(np.float16)))


def test_f2h_exhaustive_against_f16c(orc):
    bad = orc.f16c_mismatches(8)
    if bad < 0:
        pytest.skip("host CPU has no F16C")
    assert bad == 0


# --------------------------------------------------------------------------------------------
# residual add
# --------------------------------------------------------------------------------------------
def _xorshift_draws(seed, count):
    s, out = seed, []
    for _ in range(count):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        out.append(np.float32(s & 0xFFFFFF) / np.float32(16777216.0) * np.float32(8.0)
                   - np.float32(4.0))
    return np.array(out, dtype=np.float32)


def test_residual_add_reference_kat(orc):
    """The reference's own known-answer test (ref: tests/test_residual_add.cu:6-19): xorshift32
    seed 12345, values in [-4, 4), n = 1,000,003; expected = fp16(float(a) + float(b))."""
    n = 1_000_003
    a, b = orc.residual_add_kat_inputs(12345, n)
    draws = _xorshift_draws(12345, 2000)  # independent re-derivation of the first draws
    assert np.array_equal(a[:1000], draws[0::2].astype(np.float16).view(np.uint16))
    assert np.array_equal(b[:1000], draws[1::2].astype(np.float16).view(np.uint16))
    expected = (f16(a).astype(np.float32) + f16(b).astype(np.float32)).astype(np.float16)
    assert np.array_equal(orc.residual_add(a, b), expected.view(np.uint16))


def test_residual_add_matches_numpy_float16_add(orc):
    rng = np.random.default_rng(11)
    a = rng.integers(0, 65536, 1 << 20, dtype=np.uint32).astype(np.uint16)
    b = rng.integers(0, 65536, 1 << 20, dtype=np.uint32).astype(np.uint16)
    with np.errstate(all="ignore"):
        ref = (f16(a) + f16(b)).view(np.uint16)  # numpy: float32 add, one rounding
    mine = orc.residual_add(a, b)
    nan = np.isnan(f16(ref))
    assert np.array_equal(mine[~nan], ref[~nan])
    assert np.all(np.isnan(f16(mine[nan])))


# --------------------------------------------------------------------------------------------
# RMSNorm
# --------------------------------------------------------------------------------------------
def test_rmsnorm_matches_hf_llama_rmsnorm(orc):
    g = goldens()
    rows, hidden = g["rms_x"].shape
    got = orc.rmsnorm(g["rms_x"], g["rms_w"], rows, hidden, EPS)
    assert_tol(orc.compare(got, g["rms_out"]), 0.99, "oracle rmsnorm vs HF")


def test_rmsnorm_constant_rows_closed_form(orc):
    hidden = 2048
    vals = np.array([0.5, -3.0, 1e-3, 200.0, 6e-5], dtype=np.float16)
    x = np.repeat(vals[:, None], hidden, axis=1).view(np.uint16)
    w = np.ones(hidden, np.float16).view(np.uint16)
    got = f16(orc.rmsnorm(x, w, vals.size, hidden, EPS))
    c = vals.astype(np.float64)
    expect = (c / np.sqrt(c * c + EPS)).astype(np.float16)  # w = 1: out = r16(c / rms)
    assert np.all(got == expect[:, None])


def test_rmsnorm_float64_evaluation(orc):
    rng = np.random.default_rng(3)
    rows, hidden = 64, 2048
    x = normal_f16(rng, (rows, hidden))
    w = normal_f16(rng, hidden, 1.0, 0.1)
    xf, wf = f16(x).astype(np.float64), f16(w).astype(np.float64)
    inv = 1.0 / np.sqrt((xf * xf).mean(axis=1, keepdims=True) + EPS)
    ref = (wf * (xf * inv).astype(np.float16).astype(np.float64)).astype(np.float16)
    assert_tol(orc.compare(orc.rmsnorm(x, w, rows, hidden, EPS), ref.view(np.uint16)), 0.99,
               "oracle rmsnorm vs float64")


def test_add_rmsnorm_is_the_composition(orc):
    rng = np.random.default_rng(4)
    rows, hidden = 32, 2048
    r = normal_f16(rng, (rows, hidden))
    x = normal_f16(rng, (rows, hidden))
    w = normal_f16(rng, hidden, 1.0, 0.1)
    res = r.copy()
    out = orc.add_rmsnorm(res, x, w, rows, hidden, EPS)
    summed = (f16(r).astype(np.float32) + f16(x).astype(np.float32)).astype(np.float16)
    assert np.array_equal(res, summed.view(np.uint16))
    assert np.array_equal(out, orc.rmsnorm(res, w, rows, hidden, EPS))


def test_mutant_rmsnorm_without_fp16_rounding_is_caught(orc):
    """Dropping the round-to-fp16 before the weight (ref: kernels/rmsnorm.cu:54-56) stays inside
    the loose tolerance but falls below the exact-share floor against Hugging Face."""
    g = goldens()
    x = f16(g["rms_x"]).astype(np.float32)
    w = f16(g["rms_w"]).astype(np.float32)
    ss = np.zeros(x.shape[0], np.float32)
    for j in range(x.shape[1]):
        ss = ss + x[:, j] * x[:, j]
    inv = np.float32(1.0) / np.sqrt(ss / np.float32(x.shape[1]) + np.float32(EPS))
    mutant = (w * (x * inv[:, None])).astype(np.float16).view(np.uint16)
    cmp = orc.compare(mutant, g["rms_out"])
    assert cmp["exact"] < 0.99


# --------------------------------------------------------------------------------------------
# RoPE
# --------------------------------------------------------------------------------------------
def test_inv_freq_matches_hf_llama3_init(orc):
    g = goldens()
    mine = orc.compute_rope_inv_freq(64, **_rope_args())
    ref = g["inv_freq"].astype(np.float64)
    assert np.max(np.abs(mine - ref) / np.abs(ref)) <= 1e-5  # ref: tests/test_rope.cu:33


def _rope_args():
    return dict(theta=ROPE["theta"], factor=ROPE["factor"], low=ROPE["low"], high=ROPE["high"],
                orig=ROPE["orig"])


def test_inv_freq_closed_form_bands(orc):
    hd = 64
    mine = orc.compute_rope_inv_freq(hd, **_rope_args()).astype(np.float64)
    i = np.arange(hd // 2)
    f = 1.0 / ROPE["theta"] ** (2 * i / hd)
    wl = 2 * np.pi / f
    assert mine[0] == 1.0
    high = wl < ROPE["orig"] / ROPE["high"]
    low = wl > ROPE["orig"] / ROPE["low"]
    mid = ~high & ~low
    assert high.sum() > 0 and low.sum() > 0 and mid.sum() > 0
    np.testing.assert_allclose(mine[high], f[high], rtol=1e-5)
    np.testing.assert_allclose(mine[low], f[low] / ROPE["factor"], rtol=1e-5)
    s = (ROPE["orig"] / wl[mid] - ROPE["low"]) / (ROPE["high"] - ROPE["low"])
    np.testing.assert_allclose(mine[mid], (1 - s) * f[mid] / ROPE["factor"] + s * f[mid],
                               rtol=1e-5)


def test_rope_matches_hf_apply_rotary_pos_emb(orc):
    g = goldens()
    q, k = g["rope_q_in"].copy(), g["rope_k_in"].copy()
    T, nh, hd = q.shape
    inv = orc.compute_rope_inv_freq(hd, **_rope_args())
    orc.rope_apply(q, k, g["rope_pos"], inv, T, nh, k.shape[1], hd)
    assert_tol(orc.compare(q, g["rope_q_out"]), 0.99, "oracle rope Q vs HF")
    assert_tol(orc.compare(k, g["rope_k_out"]), 0.99, "oracle rope K vs HF")


def test_rope_position_zero_is_identity(orc):
    rng = np.random.default_rng(5)
    T, nh, nkv, hd = 4, 32, 8, 64
    q0, k0 = normal_f16(rng, (T, nh, hd)), normal_f16(rng, (T, nkv, hd))
    q, k = q0.copy(), k0.copy()
    inv = orc.compute_rope_inv_freq(hd, **_rope_args())
    orc.rope_apply(q, k, np.zeros(T, np.int32), inv, T, nh, nkv, hd)
    # c = 1, s = 0: x1' = r16(x1) - r16(x2 * 0) = x1 (signed zeros aside)
    assert np.array_equal(f16(q), f16(q0)) and np.array_equal(f16(k), f16(k0))


def test_rope_quarter_turn_swaps_halves(orc):
    rng = np.random.default_rng(6)
    hd = 64
    q0 = normal_f16(rng, (1, 1, hd))
    q, k = q0.copy(), np.zeros((1, 0, hd), np.uint16)
    inv = np.full(hd // 2, np.float32(np.pi / 2), np.float32)
    orc.rope_apply(q, k, np.ones(1, np.int32), inv, 1, 1, 0, hd)
    x = f16(q0).astype(np.float64).ravel()
    expect = np.concatenate([-x[hd // 2:], x[:hd // 2]]).astype(np.float16)
    assert_tol(orc.compare(q.ravel(), expect.view(np.uint16)), 0.0, "quarter turn")


def test_mutant_rope_adjacent_pairing_is_caught(orc):
    """Pairing element 2i with 2i+1 (the GPT-J layout) instead of i with i + hd/2 (ref:
    kernels/rope.cuh:11-12) must fail the Hugging Face fixture."""
    g = goldens()
    q = f16(g["rope_q_in"]).astype(np.float32)
    T, nh, hd = q.shape
    inv = orc.compute_rope_inv_freq(hd, **_rope_args())
    a = g["rope_pos"].astype(np.float32)[:, None] * inv[None, :]
    c = np.cos(a.astype(np.float64)).astype(np.float32).astype(np.float16).astype(np.float32)
    s = np.sin(a.astype(np.float64)).astype(np.float32).astype(np.float16).astype(np.float32)
    x1, x2 = q[..., 0::2], q[..., 1::2]
    out = np.empty_like(q)
    out[..., 0::2] = x1 * c[:, None, :] - x2 * s[:, None, :]
    out[..., 1::2] = x2 * c[:, None, :] + x1 * s[:, None, :]
    cmp = orc.compare(out.astype(np.float16).view(np.uint16), g["rope_q_out"])
    assert cmp["bad"] > 0


# --------------------------------------------------------------------------------------------
# SwiGLU
# --------------------------------------------------------------------------------------------
def test_swiglu_matches_torch_silu(orc):
    g = goldens()
    got = orc.swiglu(g["swiglu_gate"], g["swiglu_up"])
    assert_tol(orc.compare(got, g["swiglu_out"]), 0.99, "oracle swiglu vs HF")


def test_swiglu_special_values(orc):
    gate = np.array([0.0, -0.0, 30.0, 65504.0, -30.0, -65504.0], np.float16)
    up = np.full(gate.size, 1.5, np.float16)
    got = f16(orc.swiglu(gate.view(np.uint16), up.view(np.uint16))).astype(np.float64)
    assert got[0] == 0 and got[1] == 0
    assert got[2] == 45.0 and got[3] == np.float16(65504.0 * 1.5)  # silu(g) -> g for large g
    assert got[4] == np.float16(-30.0 / (1 + np.exp(30.0)) * 1.5) and got[5] == 0


def test_swiglu_float64_evaluation(orc):
    rng = np.random.default_rng(8)
    gate, up = normal_f16(rng, 1 << 16, 0, 3.0), normal_f16(rng, 1 << 16)
    gf = f16(gate).astype(np.float64)
    silu = (gf / (1.0 + np.exp(-gf))).astype(np.float16).astype(np.float64)
    ref = (silu * f16(up).astype(np.float64)).astype(np.float16)
    assert_tol(orc.compare(orc.swiglu(gate, up), ref.view(np.uint16)), 0.995, "swiglu f64")


def test_mutant_swiglu_without_silu_rounding_is_caught(orc):
    """Skipping the fp16 rounding of silu before the multiply (ref: kernels/swiglu.cu:12)."""
    g = goldens()
    gf = f16(g["swiglu_gate"]).astype(np.float64)
    uf = f16(g["swiglu_up"]).astype(np.float64)
    mutant = ((gf / (1 + np.exp(-gf))) * uf).astype(np.float16).view(np.uint16)
    assert orc.compare(mutant, g["swiglu_out"])["exact"] < 0.99


# --------------------------------------------------------------------------------------------
# embedding and the paged scatter
# --------------------------------------------------------------------------------------------
def test_embedding_matches_hf_and_numpy(orc):
    g = goldens()
    got = orc.embedding_lookup(g["emb_table"], g["emb_ids"], g["emb_table"].shape[1])
    assert np.array_equal(got, g["emb_out"])
    assert np.array_equal(got, g["emb_table"][g["emb_ids"]])


def _pool_rows(pool, kvdim):
    return pool.reshape(-1, kvdim)


def test_kv_scatter_prefill_addressing(orc):
    rng = np.random.default_rng(9)
    ps, kvdim, T, start = 16, 512, 77, 21
    table = rng.permutation(40).astype(np.int32)
    pool = np.full(40 * ps * kvdim, POISON, np.uint16)
    src = normal_f16(rng, (T, kvdim))
    orc.kv_scatter(src, pool, table, start, T, ps, kvdim)
    pos = start + np.arange(T)
    rows = table[pos // ps] * ps + pos % ps
    view = _pool_rows(pool, kvdim)
    assert np.array_equal(view[rows], src)
    touched = np.zeros(view.shape[0], bool)
    touched[rows] = True
    assert np.all(view[~touched] == POISON)
    assert int((view != POISON).any(axis=1).sum()) == T


def test_kv_scatter_batch_addressing(orc):
    rng = np.random.default_rng(10)
    n, ps, kvdim, max_pages = 64, 16, 512, 128
    lens = rng.integers(1, max_pages * ps + 1, n)
    tables, total = shuffled_page_tables(rng, lens, ps, max_pages)
    pool = np.full(total * ps * kvdim, POISON, np.uint16)
    src = normal_f16(rng, (n, kvdim))
    pos = (lens - 1).astype(np.int32)
    orc.kv_scatter_batch(src, pool, tables, pos, n, max_pages, ps, kvdim)
    rows = tables[np.arange(n), pos // ps] * ps + pos % ps
    view = _pool_rows(pool, kvdim)
    assert np.array_equal(view[rows], src)
    assert int((view != POISON).any(axis=1).sum()) == n


def test_rope_kv_scatter_batch_is_the_composition(orc):
    rng = np.random.default_rng(12)
    n, nh, nkv, hd, ps, max_pages = 16, 32, 8, 64, 16, 8
    kvdim = nkv * hd
    lens = rng.integers(1, max_pages * ps + 1, n)
    tables, total = shuffled_page_tables(rng, lens, ps, max_pages)
    pos = (lens - 1).astype(np.int32)
    q0, k, v = normal_f16(rng, (n, nh, hd)), normal_f16(rng, (n, nkv, hd)), normal_f16(rng, (n, nkv, hd))
    inv = orc.compute_rope_inv_freq(hd, **_rope_args())
    q = q0.copy()
    kp = np.full(total * ps * kvdim, POISON, np.uint16)
    vp = kp.copy()
    orc.rope_kv_scatter_batch(q, k, v, kp, vp, tables, pos, inv, n, max_pages, ps, nh, nkv, hd)
    q2, k2 = q0.copy(), k.copy()
    orc.rope_apply(q2, k2, pos, inv, n, nh, nkv, hd)
    rows = tables[np.arange(n), pos // ps] * ps + pos % ps
    assert np.array_equal(q, q2)
    assert np.array_equal(_pool_rows(kp, kvdim)[rows], k2.reshape(n, kvdim))
    assert np.array_equal(_pool_rows(vp, kvdim)[rows], v.reshape(n, kvdim))


# --------------------------------------------------------------------------------------------
# threaded variants used by the CPU baseline
# --------------------------------------------------------------------------------------------
def test_threaded_variants_equal_single_thread(orc):
    rng = np.random.default_rng(13)
    rows, hidden = 37, 2048
    r, x, w = normal_f16(rng, (rows, hidden)), normal_f16(rng, (rows, hidden)), normal_f16(rng, hidden, 1, .1)
    r1, r2 = r.copy(), r.copy()
    assert np.array_equal(orc.add_rmsnorm(r1, x, w, rows, hidden, EPS),
                          orc.add_rmsnorm(r2, x, w, rows, hidden, EPS, threads=5))
    assert np.array_equal(r1, r2)
    g, u = normal_f16(rng, 100_003), normal_f16(rng, 100_003)
    assert np.array_equal(orc.swiglu(g, u), orc.swiglu(g, u, threads=7))
    T, nh, nkv, hd = 29, 32, 8, 64
    q, k = normal_f16(rng, (T, nh, hd)), normal_f16(rng, (T, nkv, hd))
    pos = rng.integers(0, 131072, T).astype(np.int32)
    inv = orc.compute_rope_inv_freq(hd, **_rope_args())
    qa, ka, qb, kb = q.copy(), k.copy(), q.copy(), k.copy()
    orc.rope_apply(qa, ka, pos, inv, T, nh, nkv, hd)
    orc.rope_apply(qb, kb, pos, inv, T, nh, nkv, hd, threads=4)
    assert np.array_equal(qa, qb) and np.array_equal(ka, kb)
    table = normal_f16(rng, (100, 256))
    ids = rng.integers(0, 100, 53).astype(np.int32)
    assert np.array_equal(orc.embedding_lookup(table, ids, 256),
                          orc.embedding_lookup(table, ids, 256, threads=3))
    a, b = normal_f16(rng, 100_003), normal_f16(rng, 100_003)
    assert np.array_equal(orc.residual_add(a, b), orc.residual_add(a, b, threads=6))
    assert np.array_equal(orc.rmsnorm(x, w, rows, hidden, EPS),
                          orc.rmsnorm(x, w, rows, hidden, EPS, threads=5))
    # prefill scatter of 45 rows from position 7 over a shuffled 4-page table
    kvdim, ps = 512, 16
    src = normal_f16(rng, (45, kvdim))
    tab = rng.permutation(4).astype(np.int32)
    pa = np.full(4 * ps * kvdim, 0x7F7F, np.uint16)
    pb = pa.copy()
    orc.kv_scatter(src, pa, tab, 7, 45, ps, kvdim)
    orc.kv_scatter(src, pb, tab, 7, 45, ps, kvdim, threads=4)
    assert np.array_equal(pa, pb)
    assert (pa != 0x7F7F).sum() > 0


# --------------------------------------------------------------------------------------------
# decode attention over the paged pool
# --------------------------------------------------------------------------------------------
def _attend(orc, c):
    return orc.attention_decode_paged(c["q"], c["k_pool"], c["v_pool"], c["tables"], c["lens"],
                                      c["n_seq"], c["max_pages"], c["page_size"], c["n_heads"],
                                      c["n_kv_heads"], c["head_dim"])


def test_attention_matches_float64_definition(orc):
    """The reference test's lengths and U(-1, 1) data: within the reference's tolerance of a
    float64 evaluation from the definition, nearly always its fp16 rounding exactly."""
    c = attention_case(np.random.default_rng(20), ATTN_LENS)
    ref = attention_f64(c).astype(np.float16).view(np.uint16)
    assert_tol(orc.compare(_attend(orc, c), ref), 0.97, "oracle attention vs float64")


def test_attention_grouped_query_mapping_and_scale_are_pinned(orc):
    """Two plausible mistakes fail the float64 check: query head h reading kv head h % n_kv
    instead of h // (n_heads / n_kv), and a score scale of 1 / head_dim instead of
    1 / sqrt(head_dim)."""
    c = attention_case(np.random.default_rng(21), (5, 40, 300))
    got = _attend(orc, c)
    nh, nkv, hd, ps = 32, 8, 64, 16
    q = c["q"].view(np.float16).astype(np.float64).reshape(-1, nh, hd)
    kp = c["k_pool"].view(np.float16).astype(np.float64).reshape(-1, nkv, hd)
    vp = c["v_pool"].view(np.float16).astype(np.float64).reshape(-1, nkv, hd)

    def variant(kv_of, scale):
        out = np.empty_like(q)
        for b, S in enumerate(c["lens"]):
            j = np.arange(S)
            rows = c["tables"][b, j // ps] * ps + j % ps
            for h in range(nh):
                s = kp[rows, kv_of(h)] @ q[b, h] * scale
                p = np.exp(s - s.max())
                out[b, h] = (p / p.sum()) @ vp[rows, kv_of(h)]
        return out.astype(np.float16).view(np.uint16)

    assert orc.compare(got, variant(lambda h: h // 4, 0.125))["bad"] == 0
    assert orc.compare(got, variant(lambda h: h % nkv, 0.125))["bad"] > 0
    assert orc.compare(got, variant(lambda h: h // 4, 1.0 / 64))["bad"] > 0


def test_attention_single_position_returns_its_value_row(orc):
    """With one cached position the softmax weight is exactly 1: out = V row, bit for bit."""
    c = attention_case(np.random.default_rng(22), (1, 1, 1))
    got = _attend(orc, c).reshape(3, 32, 64)
    rows = c["tables"][:, 0] * 16
    v = c["v_pool"].reshape(-1, 8, 64)[rows]  # [3, nkv, hd]
    assert np.array_equal(got, np.repeat(v, 4, axis=1))


def test_attention_equal_keys_average_the_values(orc):
    """Identical K rows give uniform weights: out = mean of the V rows."""
    rng = np.random.default_rng(23)
    c = attention_case(rng, (37, 200))
    kp = c["k_pool"].reshape(-1, 512)
    kp[:] = uniform_f16(rng, 512)[None, :]
    ref = np.empty((2, 32, 64))
    vp = c["v_pool"].view(np.float16).astype(np.float64).reshape(-1, 8, 64)
    for b, S in enumerate(c["lens"]):
        j = np.arange(S)
        rows = c["tables"][b, j // 16] * 16 + j % 16
        ref[b] = np.repeat(vp[rows].mean(axis=0), 4, axis=0)
    assert_tol(orc.compare(_attend(orc, c), ref.astype(np.float16).view(np.uint16)), 0.9,
               "uniform weights")


def test_attention_page_placement_does_not_change_results(orc):
    """The same per-position data placed in shuffled pages or in pages 0, 1, 2, ... gives
    bit-identical outputs: only the position order enters the sums."""
    rng = np.random.default_rng(24)
    c = attention_case(rng, (50, 129, 16))
    got = _attend(orc, c)
    d = dict(c)
    kv = {}
    for name in ("k_pool", "v_pool"):
        pool = c[name].reshape(-1, 512)
        flat = np.full_like(pool, POISON)
        nxt = 0
        tables = np.zeros_like(c["tables"])
        for b, S in enumerate(c["lens"]):
            npg = (S + 15) // 16
            tables[b, :npg] = np.arange(nxt, nxt + npg)
            for i in range(npg):
                flat[(nxt + i) * 16:(nxt + i + 1) * 16] = pool[c["tables"][b, i] * 16:
                                                              (c["tables"][b, i] + 1) * 16]
            nxt += npg
        kv[name] = flat.reshape(-1)
    d.update(kv, tables=tables)
    assert np.array_equal(_attend(orc, d), got)


def test_attention_empty_sequence_is_nan(orc):
    c = attention_case(np.random.default_rng(25), (0, 3))
    got = _attend(orc, c).reshape(2, -1).view(np.float16)
    assert np.all(np.isnan(got[0])) and np.all(np.isfinite(got[1]))


# --------------------------------------------------------------------------------------------
# argmax over logits rows
# --------------------------------------------------------------------------------------------
def argmax_reference_rows(rng, V=128256):
    """The rows of ref: tests/test_argmax.cu:10-25: four rows of many exact ties, a constant
    row, the maximum at the last index, two equal maxima at 0 and 77777, a random row."""
    rows = np.empty((8, V), np.float32)
    rows[:4] = rng.integers(-8, 9, (4, V)) * 0.5
    rows[4] = 1.0
    rows[5:] = rng.uniform(-5, 5, (3, V))
    rows[5, V - 1] = 100.0
    rows[6, 0] = rows[6, 77777] = 100.0
    return rows.astype(np.float16).view(np.uint16)


def test_argmax_reference_rows_match_numpy(orc):
    rows = argmax_reference_rows(np.random.default_rng(3))
    got = orc.argmax_rows(rows, 8, rows.shape[1])
    assert np.array_equal(got, np.argmax(rows.view(np.float16), axis=1))  # first maximum
    assert got[4] == 0 and got[5] == rows.shape[1] - 1 and got[6] == 0


def test_argmax_nan_inf_and_signed_zero(orc):
    nan, inf = np.float16(np.nan), np.float16(np.inf)
    rows = np.array([[nan, 1, 3, nan, 3],        # NaN never wins: first 3
                     [nan, nan, nan, nan, nan],   # nothing above -inf: INT_MAX
                     [-inf, -inf, -inf, -inf, -inf],
                     [-0.0, 0.0, -0.0, -1, -2],   # +0 == -0: the first zero
                     [-inf, -inf, -60000, nan, -inf],
                     [inf, 1, inf, 2, nan]], np.float16)
    got = orc.argmax_rows(rows.view(np.uint16), rows.shape[0], rows.shape[1])
    assert list(got) == [2, 0x7FFFFFFF, 0x7FFFFFFF, 0, 2, 0]
    finite_rows = [0, 3, 4, 5]
    assert np.array_equal(got[finite_rows], np.nanargmax(rows[finite_rows], axis=1))


def test_mutant_argmax_last_index_on_ties_is_caught(orc):
    """Keeping the last of equal maxima (>= instead of >) fails the reference's tie rows."""
    rows = argmax_reference_rows(np.random.default_rng(3)).view(np.float16)
    last = rows.shape[1] - 1 - np.argmax(rows[:, ::-1], axis=1)
    assert not np.array_equal(orc.argmax_rows(rows.view(np.uint16), 8, rows.shape[1]), last)
