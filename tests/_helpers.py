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
