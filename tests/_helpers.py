"""Shared helpers for the tests: seeded synthetic fp16 inputs, the golden fixtures, and the
tolerance rule of the reference's kernel tests."""
from __future__ import annotations

import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden", "hf_goldens.npz")

# Llama-3 rope parameters of the reference (ref: engine/model.cu:20)
ROPE = dict(theta=500000.0, factor=32.0, low=1.0, high=4.0, orig=8192.0)
EPS = 1e-5
POISON = 0x7F7F  # fp16 NaN pattern the reference fills unused pool slots with (engine/paged.cu:22)


def goldens() -> dict:
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def normal_f16(rng: np.random.Generator, shape, mean=0.0, std=1.0) -> np.ndarray:
    """fp16 bit patterns of N(mean, std) draws (float32 draws rounded by numpy, RNE)."""
    v = rng.standard_normal(shape, dtype=np.float32)
    if std != 1.0:
        v *= np.float32(std)
    if mean != 0.0:
        v += np.float32(mean)
    return v.astype(np.float16).view(np.uint16)


def assert_tol(cmp: dict, min_exact: float = 0.99, what: str = "") -> None:
    """The reference's rule |d| <= 1e-3 + 4e-3 |e| for every element, plus a floor on the share
    of bit-identical elements, which catches systematic errors the loose rule would let pass."""
    assert cmp["bad"] == 0, f"{what}: {cmp['bad']} of {cmp['n']} elements outside tolerance {cmp}"
    assert cmp["exact"] >= min_exact, f"{what}: only {100 * cmp['exact']:.3f}% exact {cmp}"


def shuffled_page_tables(rng: np.random.Generator, lens: np.ndarray, page_size: int,
                         max_pages: int, extra_pages: int = 0):
    """Block tables [n, max_pages] (unused entries 0) assigning Σ ceil(len/ps) pages from a
    shuffled permutation of the pool, as ref: tests/test_attention_decode_fast.cu:25-41."""
    npages = (lens + page_size - 1) // page_size
    total = int(npages.sum()) + extra_pages
    perm = rng.permutation(total).astype(np.int32)
    tables = np.zeros((lens.size, max_pages), np.int32)
    nxt = 0
    for b, np_b in enumerate(npages):
        tables[b, :np_b] = perm[nxt:nxt + np_b]
        nxt += np_b
    return tables, total


def uniform_f16(rng: np.random.Generator, shape, lo=-1.0, hi=1.0) -> np.ndarray:
    """fp16 bit patterns of U(lo, hi) draws, as the reference's attention and argmax tests use."""
    return rng.uniform(lo, hi, shape).astype(np.float32).astype(np.float16).view(np.uint16)


# The shape the reference's split-KV attention is specified for (Llama-3.2-1B,
# ref: kernels/attention_decode_fast.cuh:13) and its test's sequence lengths, which include the
# page-boundary cases (ref: tests/test_attention_decode_fast.cu:17-18).
ATTN = dict(n_heads=32, n_kv_heads=8, head_dim=64, page_size=16)
ATTN_LENS = (1, 15, 16, 17, 33, 100, 402, 2048)


def attention_case(rng: np.random.Generator, lens, n_heads=32, n_kv_heads=8, head_dim=64,
                   page_size=16, max_pages=None, extra_pages=0):
    """Inputs laid out as ref: tests/test_attention_decode_fast.cu:22-41: q [n, nh, hd] and the
    cached K, V rows U(-1, 1); pages assigned from a shuffled permutation; every pool slot that
    no position uses holds the NaN pattern 0x7F7F. Returns a dict of numpy arrays and sizes."""
    lens = np.asarray(lens, np.int32)
    n = lens.size
    kvdim = n_kv_heads * head_dim
    npages = (np.maximum(lens, 0) + page_size - 1) // page_size
    if max_pages is None:
        max_pages = max(1, int(npages.max()))
    tables, total = shuffled_page_tables(rng, np.maximum(lens, 0), page_size, max_pages,
                                         extra_pages)
    total = max(total, 1)
    q = uniform_f16(rng, (n, n_heads, head_dim))
    kp = np.full((total * page_size, kvdim), POISON, np.uint16)
    vp = kp.copy()
    for b in range(n):
        if lens[b] <= 0:
            continue
        j = np.arange(lens[b])
        rows = tables[b, j // page_size] * page_size + j % page_size
        kp[rows] = uniform_f16(rng, (lens[b], kvdim))
        vp[rows] = uniform_f16(rng, (lens[b], kvdim))
    return dict(q=q, k_pool=kp.reshape(-1), v_pool=vp.reshape(-1), tables=tables, lens=lens,
                n_seq=n, max_pages=max_pages, total_pages=total, n_heads=n_heads,
                n_kv_heads=n_kv_heads, head_dim=head_dim, page_size=page_size)


def attention_f64(case: dict) -> np.ndarray:
    """Decode attention in float64 with numpy, written from the definition: softmax over the
    cached positions of q . k / sqrt(head_dim), then the weighted sum of the V rows; query head
    h reads kv head h // (n_heads / n_kv_heads). Returns float64 [n, nh, hd]."""
    nh, nkv, hd, ps = case["n_heads"], case["n_kv_heads"], case["head_dim"], case["page_size"]
    q = case["q"].view(np.float16).astype(np.float64).reshape(case["n_seq"], nh, hd)
    kp = case["k_pool"].view(np.float16).astype(np.float64).reshape(-1, nkv, hd)
    vp = case["v_pool"].view(np.float16).astype(np.float64).reshape(-1, nkv, hd)
    out = np.full((case["n_seq"], nh, hd), np.nan)
    for b, S in enumerate(case["lens"]):
        if S <= 0:
            continue
        j = np.arange(S)
        rows = case["tables"][b, j // ps] * ps + j % ps
        K, V = kp[rows], vp[rows]  # [S, nkv, hd]
        for h in range(nh):
            g = h // (nh // nkv)
            s = K[:, g, :] @ q[b, h] / np.sqrt(hd)
            p = np.exp(s - s.max())
            out[b, h] = (p / p.sum()) @ V[:, g, :]
    return out


# A small Llama-3 shape for whole-model checks: the engine's constraints (head_dim 64, 4 query
# heads per kv head, page size 16) at a size the scalar oracle runs in well under a second.
TINY = dict(n_layers=2, hidden=256, n_heads=4, n_kv_heads=1, head_dim=64, inter=512, vocab=512,
            eps=1e-5, rope_theta=500000.0, rope_factor=32.0, rope_low_freq_factor=1.0,
            rope_high_freq_factor=4.0, rope_original_max_pos=8192.0)


def tiny_weights(seed: int, embed_std: float = 0.02, cfg: dict = TINY) -> dict:
    """Seeded fp16 weights under the Hugging Face names: projections ~N(0, 0.05), the
    embedding ~N(0, embed_std), norm weights ~N(1, 0.1)."""
    rng = np.random.default_rng(seed)
    c = cfg
    H, I, V = c["hidden"], c["inter"], c["vocab"]
    qd, kvd = c["n_heads"] * c["head_dim"], c["n_kv_heads"] * c["head_dim"]

    def f16(shape, scale):
        return (scale * rng.standard_normal(shape, dtype=np.float32)).astype(np.float16)

    w = {"model.embed_tokens.weight": f16((V, H), embed_std),
         "model.norm.weight": (1 + 0.1 * rng.standard_normal(H)).astype(np.float16)}
    for l in range(c["n_layers"]):
        p = f"model.layers.{l}."
        w[p + "input_layernorm.weight"] = (1 + 0.1 * rng.standard_normal(H)).astype(np.float16)
        w[p + "post_attention_layernorm.weight"] = (1 + 0.1 * rng.standard_normal(H)).astype(
            np.float16)
        for name, shape in (("self_attn.q_proj", (qd, H)), ("self_attn.k_proj", (kvd, H)),
                            ("self_attn.v_proj", (kvd, H)), ("self_attn.o_proj", (H, qd)),
                            ("mlp.gate_proj", (I, H)), ("mlp.up_proj", (I, H)),
                            ("mlp.down_proj", (H, I))):
            w[p + name + ".weight"] = f16(shape, 0.05)
    return w


def oracle_pools(num_pages: int, cfg: dict = TINY):
    """Per-layer K and V pools for the oracle, every slot 0x7F7F (ref: engine/paged.cu:22)."""
    kvd = cfg["n_kv_heads"] * cfg["head_dim"]
    n = num_pages * 16 * kvd
    return ([np.full(n, POISON, np.uint16) for _ in range(cfg["n_layers"])],
            [np.full(n, POISON, np.uint16) for _ in range(cfg["n_layers"])])
