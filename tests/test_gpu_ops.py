"""GPU parity of every libllmk entry point against the CPU oracle, on seeded inputs, over the
shapes that select each kernel variant (full and partial lanes, wide-row block kernel, scalar
fallbacks for unaligned pointers and odd head sizes, tails not a multiple of the vector width,
few and many rows). Outputs are pre-filled with the fp16 NaN pattern 0x7F7F and followed by a
canary, as the reference's tests do (ref: tests/test_residual_add.cu:27,39-42,
engine/paged.cu:22), so a missing or stray write shows.

Bar: bit-exact for the gather, the scatters, the residual add and the residual output of the
fused norm; for norm, rotary and activation outputs the reference's rule
|d| <= 1e-3 + 4e-3 |e| for every element plus a floor on the bit-identical share."""
import numpy as np
import pytest
import torch

from _helpers import EPS, POISON, ROPE, assert_tol, normal_f16, shuffled_page_tables

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
CANARY = 0x5A5A


def dev(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.float16)).to(DEV)


def dev_i32(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(DEV)


def host(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def filled(n: int, value: int = POISON) -> torch.Tensor:
    return torch.full((n,), value if value < 32768 else value - 65536, dtype=torch.int16,
                      device=DEV).view(torch.float16)


def inv_freq_dev(orc, hd: int) -> tuple:
    inv = orc.compute_rope_inv_freq(hd, ROPE["theta"], ROPE["factor"], ROPE["low"], ROPE["high"],
                                    ROPE["orig"])
    return inv, torch.from_numpy(inv).to(DEV)


# --------------------------------------------------------------------------------------------
@pytest.mark.parametrize("hidden", [8, 64, 520, 2048, 4096, 8200])
@pytest.mark.parametrize("n", [1, 3, 4097])
def test_embedding_lookup(llmk, orc, hidden, n):
    rng = np.random.default_rng(hidden * 7 + n)
    vocab = 3000
    table = normal_f16(rng, (vocab, hidden), 0.0, 0.02)
    ids = rng.integers(0, vocab, n).astype(np.int32)
    ids[0] = vocab - 1
    if n > 2:
        ids[1], ids[2] = 0, ids[0]
    out = filled((n + 1) * hidden, CANARY)
    llmk.embedding_lookup(dev(table), dev_i32(ids), out, n, hidden)
    got = host(out).reshape(n + 1, hidden)
    assert np.array_equal(got[:n], orc.embedding_lookup(table, ids, hidden))
    assert np.all(got[n] == CANARY)


@pytest.mark.parametrize("hidden", [2048, 4096, 6144])
@pytest.mark.parametrize("n", [1500, 2047, 4096, 8192, 8193])
def test_embedding_lookup_grouped_rows(llmk, orc, hidden, n):
    """The many-token kernel (hidden a multiple of 2048, more than 1024 tokens): 2, 4 or 8 rows
    per wave, one group per wave (n <= 8192) or a loop over groups (8193), a partial last group
    (1500 with 2 per wave leaves waves without one; 2047 and 8193 end in a part group), and
    compile-time (2048, 4096) or runtime (6144) row widths."""
    rng = np.random.default_rng(hidden + n)
    vocab = 3000
    table = normal_f16(rng, (vocab, hidden), 0.0, 0.02)
    ids = rng.integers(0, vocab, n).astype(np.int32)
    ids[-1] = vocab - 1
    out = filled((n + 1) * hidden, CANARY)
    llmk.embedding_lookup(dev(table), dev_i32(ids), out, n, hidden)
    got = host(out).reshape(n + 1, hidden)
    assert np.array_equal(got[:n], orc.embedding_lookup(table, ids, hidden))
    assert np.all(got[n] == CANARY)


# --------------------------------------------------------------------------------------------
def test_residual_add_reference_kat(llmk, orc):
    """ref: tests/test_residual_add.cu:12-58 -- out of place with a canary, then in place."""
    n, pad = 1_000_003, 256
    a, b = orc.residual_add_kat_inputs(12345, n)
    expected = orc.residual_add(a, b)
    da, db = dev(a), dev(b)
    out = filled(n + pad, 0xABAB)
    llmk.residual_add(da, db, out, n)
    got = host(out)
    assert np.array_equal(got[:n], expected)
    assert np.all(got[n:] == 0xABAB)
    llmk.residual_add(da, db, da, n)  # out == a
    assert np.array_equal(host(da), expected)
    da2 = dev(a)
    llmk.residual_add(da2, db, db, n)  # out == b
    assert np.array_equal(host(db), expected)


@pytest.mark.parametrize("n", [1, 7, 8, 9, 4093, 1 << 20])
@pytest.mark.parametrize("offset", [0, 1, 3])
def test_residual_add_sizes_and_alignment(llmk, orc, n, offset):
    rng = np.random.default_rng(n + offset)
    a, b = normal_f16(rng, n, 0, 30.0), normal_f16(rng, n, 0, 30.0)
    # offset > 0 makes every pointer 2-byte aligned only: the any-alignment kernel runs
    ba, bb, bo = filled(n + offset), filled(n + offset), filled(n + offset + 8, CANARY)
    ba[offset:offset + n] = dev(a)
    bb[offset:offset + n] = dev(b)
    llmk.residual_add(ba[offset:], bb[offset:], bo[offset:], n)
    got = host(bo)
    assert np.array_equal(got[offset:offset + n], orc.residual_add(a, b))
    assert np.all(got[:offset] == CANARY) and np.all(got[offset + n:] == CANARY)


# --------------------------------------------------------------------------------------------
NORM_SHAPES = [(1, 8), (3, 64), (5, 512), (4, 520), (16, 2048), (7, 4096), (2, 8192),
               (3, 8200), (2, 16384), (4097, 256), (4100, 2048)]


@pytest.mark.parametrize("rows,hidden", NORM_SHAPES)
def test_rmsnorm(llmk, orc, rows, hidden):
    rng = np.random.default_rng(rows * 31 + hidden)
    x = normal_f16(rng, (rows, hidden))
    w = normal_f16(rng, hidden, 1.0, 0.1)
    out = filled((rows + 1) * hidden, CANARY)
    llmk.rmsnorm(dev(x), dev(w), out, rows, hidden, EPS)
    got = host(out).reshape(rows + 1, hidden)
    assert_tol(orc.compare(got[:rows], orc.rmsnorm(x, w, rows, hidden, EPS)), 0.99,
               f"rmsnorm {rows}x{hidden}")
    assert np.all(got[rows] == CANARY)


def test_rmsnorm_in_place_and_row_offset(llmk, orc):
    """out == x, and the reference's n_rows = 1 call on an offset row (ref: engine/model.cu:58-59)."""
    rng = np.random.default_rng(17)
    rows, hidden = 9, 2048
    x = normal_f16(rng, (rows, hidden))
    w = normal_f16(rng, hidden, 1.0, 0.1)
    dx = dev(x)
    llmk.rmsnorm(dx, dev(w), dx, rows, hidden, EPS)
    assert_tol(orc.compare(host(dx), orc.rmsnorm(x, w, rows, hidden, EPS)), 0.99, "in place")
    dx = dev(x)
    out = filled(hidden)
    llmk.rmsnorm(dx[rows - 1], dev(w), out, 1, hidden, EPS)
    assert_tol(orc.compare(host(out), orc.rmsnorm(x[rows - 1].copy(), w, 1, hidden, EPS)), 0.99,
               "last row")


@pytest.mark.parametrize("rows,hidden", NORM_SHAPES)
def test_add_rmsnorm(llmk, orc, rows, hidden):
    rng = np.random.default_rng(rows * 37 + hidden)
    r = normal_f16(rng, (rows, hidden))
    x = normal_f16(rng, (rows, hidden))
    w = normal_f16(rng, hidden, 1.0, 0.1)
    dr = dev(r)
    out = filled((rows + 1) * hidden, CANARY)
    llmk.add_rmsnorm(dr, dev(x), dev(w), out, rows, hidden, EPS)
    r_exp = r.copy()
    o_exp = orc.add_rmsnorm(r_exp, x, w, rows, hidden, EPS)
    assert np.array_equal(host(dr), r_exp), "residual must be bit-exact"
    got = host(out).reshape(rows + 1, hidden)
    assert_tol(orc.compare(got[:rows], o_exp), 0.99, f"add_rmsnorm {rows}x{hidden}")
    assert np.all(got[rows] == CANARY)


@pytest.mark.parametrize("rows", [3072, 4096, 5000, 6000, 8191, 8192])
def test_norms_of_many_rows_give_the_bits_of_one_row_per_wave(llmk, rows):
    """Batches of 2048-wide rows that fill one resident round run several rows per wave (4 at
    3072-4096 rows, 8 up to 8192, the fused kernel from 3072 rows and RMSNorm alone from 5120);
    slices of 1024 rows run one row per wave. Every bit of both outputs and of the updated
    residual must agree, including the partial last wave (5000, 6000, 8191 rows), and nothing
    past the last row may be written."""
    hidden = 2048
    rng = np.random.default_rng(rows)
    r, x = normal_f16(rng, (rows, hidden)), normal_f16(rng, (rows, hidden))
    w = normal_f16(rng, hidden, 1.0, 0.1)
    dx, dw = dev(x).reshape(-1), dev(w)
    whole = filled((rows + 1) * hidden, CANARY)
    llmk.rmsnorm(dx, dw, whole, rows, hidden, EPS)
    sliced = filled(rows * hidden)
    for r0 in range(0, rows, 1024):
        n = min(1024, rows - r0)
        llmk.rmsnorm(dx[r0 * hidden:], dw, sliced[r0 * hidden:], n, hidden, EPS)
    got = host(whole)
    assert np.array_equal(got[:rows * hidden], host(sliced)), f"rmsnorm {rows} rows"
    assert np.all(got[rows * hidden:] == CANARY)
    d1, d2 = dev(r).reshape(-1), dev(r).reshape(-1)
    o1, o2 = filled((rows + 1) * hidden, CANARY), filled(rows * hidden)
    llmk.add_rmsnorm(d1, dx, dw, o1, rows, hidden, EPS)
    for r0 in range(0, rows, 1024):
        n = min(1024, rows - r0)
        llmk.add_rmsnorm(d2[r0 * hidden:], dx[r0 * hidden:], dw, o2[r0 * hidden:], n, hidden,
                         EPS)
    assert np.array_equal(host(d1), host(d2)), f"residual {rows} rows"
    got = host(o1)
    assert np.array_equal(got[:rows * hidden], host(o2)), f"add_rmsnorm {rows} rows"
    assert np.all(got[rows * hidden:] == CANARY)
    # in place (out == x): each wave reads all of its rows before it writes any
    dx2 = dx.clone()
    llmk.rmsnorm(dx2, dw, dx2, rows, hidden, EPS)
    assert np.array_equal(host(dx2), host(whole)[:rows * hidden]), f"in place {rows} rows"


def test_add_rmsnorm_equals_residual_add_then_rmsnorm(llmk):
    """The fused kernel writes exactly what the two reference launches write on the GPU."""
    rng = np.random.default_rng(19)
    rows, hidden = 256, 2048
    r, x = normal_f16(rng, (rows, hidden)), normal_f16(rng, (rows, hidden))
    w = normal_f16(rng, hidden, 1.0, 0.1)
    d1, d2, dx, dw = dev(r), dev(r), dev(x), dev(w)
    o1, o2 = filled(rows * hidden), filled(rows * hidden)
    llmk.add_rmsnorm(d1, dx, dw, o1, rows, hidden, EPS)
    llmk.residual_add(d2, dx, d2, rows * hidden)
    llmk.rmsnorm(d2, dw, o2, rows, hidden, EPS)
    assert np.array_equal(host(d1), host(d2))
    assert np.array_equal(host(o1), host(o2))


# --------------------------------------------------------------------------------------------
ROPE_SHAPES = [  # (T, n_heads, n_kv_heads, head_dim)
    (1, 32, 8, 64), (5, 32, 8, 64), (1023, 32, 8, 64),
    (1500, 32, 8, 64),             # 256 threads, 2 tokens per block
    (3001, 32, 8, 64),             # 256 threads, 4 tokens per block, partial last block
    (4100, 32, 8, 64),             # 256 threads, 8 tokens per block, partial last block
    (2048, 32, 8, 64),             # 512 threads, 4 tokens (3 vectors per thread), 512 tiles
    (4096, 32, 8, 64),             # 512 threads, 8 tokens (5 vectors per thread), 512 tiles
    (8192, 6, 2, 64),              # 512 threads, 16 tokens of 64 vectors (2 per thread)
    (8192, 12, 4, 256),            # 512 threads, 16 tokens of 512 vectors (16 per thread)
    (8192, 32, 4, 128),            # 512 threads, 16 tokens of 576 vectors (18 per thread)
    (17, 16, 4, 128), (9, 8, 2, 256), (33, 4, 1, 32), (6, 3, 1, 16),
    (7, 32, 0, 64), (5, 0, 8, 64),
    (11, 4, 2, 40), (3, 2, 1, 6),  # head_dim not a multiple of 16: scalar path
    (16385, 32, 8, 64),            # 512 threads, 4 tokens per block (3 vectors per thread),
                                   # a last block of one token
    (33001, 4, 1, 64),             # 256 threads, 16 tokens per block, partial last block
    (7, 64, 8, 256),               # wide tokens: 512 threads, 5 vectors per thread
    (2, 128, 32, 256),             # one token exceeds a block: scalar path
]


@pytest.mark.parametrize("T,nh,nkv,hd", ROPE_SHAPES)
def test_rope_apply(llmk, orc, T, nh, nkv, hd):
    rng = np.random.default_rng(T * 1000 + nh * 10 + hd)
    q, k = normal_f16(rng, (T, nh, hd)), normal_f16(rng, (T, nkv, hd))
    pos = rng.integers(0, 131072, T).astype(np.int32)
    pos[0] = 131071
    if T > 2:
        pos[1], pos[2] = 0, 1
    inv, dinv = inv_freq_dev(orc, hd)
    dq = dev(q) if nh else filled(1)
    dk = dev(k) if nkv else filled(1)
    llmk.rope_apply(dq, dk, dev_i32(pos), dinv, T, nh, nkv, hd)
    orc.rope_apply(q, k, pos, inv, T, nh, nkv, hd)
    if nh:
        assert_tol(orc.compare(host(dq), q), 0.995, "rope Q")
    if nkv:
        assert_tol(orc.compare(host(dk), k), 0.995, "rope K")


def test_rope_apply_unaligned_falls_back(llmk, orc):
    rng = np.random.default_rng(23)
    T, nh, nkv, hd = 13, 8, 2, 64
    q, k = normal_f16(rng, (T, nh, hd)), normal_f16(rng, (T, nkv, hd))
    pos = rng.integers(0, 131072, T).astype(np.int32)
    inv, dinv = inv_freq_dev(orc, hd)
    bq = filled(q.size + 1)
    bq[1:] = dev(q).reshape(-1)
    dk = dev(k)
    llmk.rope_apply(bq[1:], dk, dev_i32(pos), dinv, T, nh, nkv, hd)
    orc.rope_apply(q, k, pos, inv, T, nh, nkv, hd)
    assert_tol(orc.compare(host(bq)[1:], q.ravel()), 0.995, "unaligned Q")
    assert_tol(orc.compare(host(dk), k), 0.995, "K")
    assert host(bq)[0] == POISON


# --------------------------------------------------------------------------------------------
@pytest.mark.parametrize("n", [1, 8, 13, 4096 * 3 + 5, 1 << 21])
@pytest.mark.parametrize("offset", [0, 1])
def test_swiglu(llmk, orc, n, offset):
    rng = np.random.default_rng(n * 3 + offset)
    g, u = normal_f16(rng, n, 0, 3.0), normal_f16(rng, n)
    bg, bu, bo = filled(n + offset), filled(n + offset), filled(n + offset + 8, CANARY)
    bg[offset:] = dev(g)
    bu[offset:] = dev(u)
    llmk.swiglu(bg[offset:], bu[offset:], bo[offset:], n)
    got = host(bo)
    assert_tol(orc.compare(got[offset:offset + n], orc.swiglu(g, u)), 0.995, "swiglu")
    assert np.all(got[offset + n:] == CANARY)


@pytest.mark.parametrize("up_value", [1.0, -1.5, 0.0999, 7.0, 65504.0])
def test_swiglu_all_fp16_gate_values_bit_exact(llmk, orc, up_value):
    """silu depends on the 16-bit gate only: every one of the 65536 fp16 gate values (NaNs,
    infinities, subnormals included) gives the oracle's bits, in the vector kernel and in the
    any-alignment kernel."""
    gate = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    up = np.full(65536, up_value, np.float16).view(np.uint16)
    with np.errstate(all="ignore"):
        exp = orc.swiglu(gate, up)
    for offset in (0, 1):
        bg, bu, bo = filled(65536 + offset), filled(65536 + offset), filled(65536 + offset)
        bg[offset:] = dev(gate)
        bu[offset:] = dev(up)
        llmk.swiglu(bg[offset:], bu[offset:], bo[offset:], 65536)
        got = host(bo)[offset:]
        nan = np.isnan(exp.view(np.float16))
        assert np.array_equal(np.isnan(got.view(np.float16)), nan)
        bad = np.flatnonzero((got != exp) & ~nan)
        assert bad.size == 0, f"offset {offset}: gate values {gate[bad[:8]]} differ"


def test_swiglu_special_values(llmk, orc):
    specials = np.array([0.0, -0.0, 6e-8, -6e-8, 1e-4, -1e-4, 8.0, -8.0, 16.0, -16.0, 20.0,
                         -20.0, 88.0, -88.0, 1000.0, -1000.0, 65504.0, -65504.0, 11.0, -11.0,
                         0.5, -0.5, 3.0, -3.0], np.float16).view(np.uint16)
    up = np.full(specials.size, 1.5, np.float16).view(np.uint16)
    out = filled(specials.size)
    llmk.swiglu(dev(specials), dev(up), out, specials.size)
    assert_tol(orc.compare(host(out), orc.swiglu(specials, up)), 0.9, "specials")


# --------------------------------------------------------------------------------------------
def _rows_changed(pool: np.ndarray, kvdim: int) -> int:
    return int((pool.reshape(-1, kvdim) != POISON).any(axis=1).sum())


@pytest.mark.parametrize("kvdim", [8, 128, 512, 1032])
@pytest.mark.parametrize("start,T", [(0, 100), (37, 1), (5, 4100)])
def test_kv_scatter(llmk, orc, kvdim, start, T):
    rng = np.random.default_rng(kvdim + T + start)
    ps = 16
    npages = (start + T + ps - 1) // ps + 3
    table = rng.permutation(npages).astype(np.int32)
    src = normal_f16(rng, (T, kvdim))
    pool = filled(npages * ps * kvdim)
    llmk.kv_scatter(dev(src), pool, dev_i32(table), start, T, ps, kvdim)
    exp = np.full(npages * ps * kvdim, POISON, np.uint16)
    orc.kv_scatter(src, exp, table, start, T, ps, kvdim)
    got = host(pool)
    assert np.array_equal(got, exp)
    assert _rows_changed(got, kvdim) == T


@pytest.mark.parametrize("n,max_pages,ps", [(256, 128, 16), (1, 4, 16), (4099, 8, 16),
                                            (64, 32, 64)])
def test_kv_scatter_batch(llmk, orc, n, max_pages, ps):
    rng = np.random.default_rng(n + max_pages)
    kvdim = 512
    lens = rng.integers(1, max_pages * ps + 1, n)
    tables, total = shuffled_page_tables(rng, lens, ps, max_pages)
    pos = (lens - 1).astype(np.int32)
    src = normal_f16(rng, (n, kvdim))
    pool = filled(total * ps * kvdim)
    llmk.kv_scatter_batch(dev(src), pool, dev_i32(tables), dev_i32(pos), n, max_pages, ps, kvdim)
    exp = np.full(total * ps * kvdim, POISON, np.uint16)
    orc.kv_scatter_batch(src, exp, tables, pos, n, max_pages, ps, kvdim)
    got = host(pool)
    assert np.array_equal(got, exp)
    assert _rows_changed(got, kvdim) == n


@pytest.mark.parametrize("n,nh,nkv,hd", [(256, 32, 8, 64), (1, 32, 8, 64), (3, 32, 8, 64),
                                         (2048, 32, 8, 64), (4100, 32, 8, 64),
                                         (64, 16, 4, 128), (33, 8, 8, 32), (5, 0, 2, 64)])
def test_rope_kv_scatter_batch(llmk, orc, n, nh, nkv, hd):
    rng = np.random.default_rng(n * 7 + hd + nh)
    ps, max_pages = 16, 128
    kvdim = nkv * hd
    lens = rng.integers(1, max_pages * ps + 1, n)
    tables, total = shuffled_page_tables(rng, lens, ps, max_pages)
    pos = (lens - 1).astype(np.int32)
    q, k, v = normal_f16(rng, (n, nh, hd)), normal_f16(rng, (n, nkv, hd)), normal_f16(rng, (n, nkv, hd))
    inv, dinv = inv_freq_dev(orc, hd)
    dq = dev(q) if nh else filled(1)
    dk, dv = dev(k), dev(v)
    kp, vp = filled(total * ps * kvdim), filled(total * ps * kvdim)
    llmk.rope_kv_scatter_batch(dq, dk, dv, kp, vp, dev_i32(tables), dev_i32(pos), dinv, n,
                               max_pages, ps, nh, nkv, hd)
    kp_e = np.full(total * ps * kvdim, POISON, np.uint16)
    vp_e = kp_e.copy()
    q_e = q.copy()
    orc.rope_kv_scatter_batch(q_e, k, v, kp_e, vp_e, tables, pos, inv, n, max_pages, ps, nh,
                              nkv, hd)
    got_v, got_k = host(vp), host(kp)
    assert np.array_equal(got_v, vp_e), "V pool must be bit-exact"
    assert _rows_changed(got_v, kvdim) == n and _rows_changed(got_k, kvdim) == n
    rows = tables[np.arange(n), pos // ps] * ps + pos % ps
    assert_tol(orc.compare(got_k.reshape(-1, kvdim)[rows], kp_e.reshape(-1, kvdim)[rows]), 0.995,
               "K pool")
    assert np.array_equal(host(dk), k), "k is read only"
    if nh:
        assert_tol(orc.compare(host(dq), q_e), 0.995, "Q")


def test_rope_kv_scatter_batch_rejects_a_token_wider_than_a_block(llmk, orc):
    n, nh, nkv, hd = 2, 128, 32, 256
    _, dinv = inv_freq_dev(orc, hd)
    q, k = filled(n * nh * hd), filled(n * nkv * hd)
    pool = filled(16 * nkv * hd)
    tab, pos = dev_i32(np.zeros((n, 1), np.int32)), dev_i32(np.zeros(n, np.int32))
    with pytest.raises(llmk.LlmkError, match="outside what the kernels implement"):
        llmk.rope_kv_scatter_batch(q, k, k, pool, pool, tab, pos, dinv, n, 1, 16, nh, nkv, hd)
    assert np.all(host(pool) == POISON)


def test_rope_kv_scatter_batch_equals_the_three_reference_launches(llmk, orc):
    """Fused decode op == rope_apply + kv_scatter_batch(K) + kv_scatter_batch(V) on the GPU
    (ref: engine/batched.cu:55-58), bit for bit."""
    rng = np.random.default_rng(29)
    n, nh, nkv, hd, ps, max_pages = 256, 32, 8, 64, 16, 128
    kvdim = nkv * hd
    lens = rng.integers(1, 2049, n)
    tables, total = shuffled_page_tables(rng, lens, ps, max_pages)
    pos = dev_i32((lens - 1).astype(np.int32))
    tab = dev_i32(tables)
    q, k, v = normal_f16(rng, (n, nh, hd)), normal_f16(rng, (n, nkv, hd)), normal_f16(rng, (n, nkv, hd))
    _, dinv = inv_freq_dev(orc, hd)
    q1, q2, k1, k2, dv = dev(q), dev(q), dev(k), dev(k), dev(v)
    pools = [filled(total * ps * kvdim) for _ in range(4)]
    llmk.rope_kv_scatter_batch(q1, k1, dv, pools[0], pools[1], tab, pos, dinv, n, max_pages, ps,
                               nh, nkv, hd)
    llmk.rope_apply(q2, k2, pos, dinv, n, nh, nkv, hd)
    llmk.kv_scatter_batch(k2, pools[2], tab, pos, n, max_pages, ps, kvdim)
    llmk.kv_scatter_batch(dv, pools[3], tab, pos, n, max_pages, ps, kvdim)
    assert np.array_equal(host(q1), host(q2))
    assert np.array_equal(host(pools[0]), host(pools[2]))
    assert np.array_equal(host(pools[1]), host(pools[3]))


# --------------------------------------------------------------------------------------------
def test_copy_bytes(llmk):
    src = torch.randint(-30000, 30000, (1 << 22,), dtype=torch.int16, device=DEV)
    dst = torch.zeros(src.numel() + 64, dtype=torch.int16, device=DEV)
    llmk.copy_bytes(src, dst, src.numel() * 2)
    assert torch.equal(dst[:src.numel()], src) and int(dst[src.numel():].abs().sum()) == 0


def test_launch_on_a_side_stream(llmk, orc):
    rng = np.random.default_rng(31)
    rows, hidden = 512, 2048
    r, x = normal_f16(rng, (rows, hidden)), normal_f16(rng, (rows, hidden))
    w = normal_f16(rng, hidden, 1.0, 0.1)
    s = torch.cuda.Stream()
    dr, dx, dw = dev(r), dev(x), dev(w)
    out = filled(rows * hidden)
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        llmk.add_rmsnorm(dr, dx, dw, out, rows, hidden, EPS)
    llmk.add_rmsnorm(dr, dx, dw, out, rows, hidden, EPS, stream=s)  # explicit stream argument
    torch.cuda.current_stream().wait_stream(s)
    r_e = r.copy()
    orc.add_rmsnorm(r_e, x, w, rows, hidden, EPS)
    o_e = orc.add_rmsnorm(r_e, x, w, rows, hidden, EPS)
    assert np.array_equal(host(dr), r_e)
    assert_tol(orc.compare(host(out), o_e), 0.99, "side stream")
