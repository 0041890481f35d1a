"""CPU checks of the decode-step oracle: the projection (or_linear) and the whole forward pass
over token rows (oracle.engine_forward), pinned against float64 arithmetic, closed forms and an
independent implementation of the same model (Hugging Face's LlamaForCausalLM in float32).

The reference pins its generation path the same way, against Hugging Face logits of the real
model (ref: tests/test_generate_batched.cu:44-53, relative L2 of the logits below 5e-3); the
real weights are not available offline, so seeded random weights of a small Llama-3 shape are
used.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import oracle  # noqa: E402

from _helpers import TINY, oracle_pools as _pools, tiny_weights as _tiny_weights  # noqa: E402

def _f16(rng, shape, scale=1.0):
    return (scale * rng.standard_normal(shape, dtype=np.float32)).astype(np.float16)


# ------------------------------------------------------------------------------------------
# or_linear
# ------------------------------------------------------------------------------------------
def test_linear_matches_float64_within_the_fp32_summation_bound():
    rng = np.random.default_rng(0x5EED0100)
    T, K, N = 7, 1000, 96
    x, w = _f16(rng, (T, K)), _f16(rng, (N, K), 0.05)
    y = oracle.linear(x, w, T, K, N).view(np.float16).astype(np.float64)
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    # fp32 sequential summation: |err| <= K * 2^-24 * sum|x w| (plus the final fp16 rounding,
    # half an fp16 ulp of the result).
    bound = K * 2.0 ** -24 * (np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T)
    half_ulp = np.abs(exact) * 2.0 ** -11 + 2.0 ** -25
    assert np.all(np.abs(y - exact) <= bound + half_ulp + 1e-12)
    # and the fp16 result is the correctly rounded float64 value almost everywhere
    assert np.mean(y == exact.astype(np.float16).astype(np.float64)) > 0.97


def test_linear_one_hot_and_identity_select_exact_values():
    rng = np.random.default_rng(0x5EED0101)
    T, K = 5, 64
    x = _f16(rng, (T, K))
    eye = np.eye(K, dtype=np.float16)
    assert np.array_equal(oracle.linear(x, eye, T, K, K), x.view(np.uint16))
    perm = rng.permutation(K)
    sel = np.eye(K, dtype=np.float16)[perm]          # row o picks column perm[o]
    assert np.array_equal(oracle.linear(x, sel, T, K, K), x[:, perm].view(np.uint16))
    # a dropped or transposed operand fails: W^T instead of W
    w = _f16(rng, (3, K))
    y = oracle.linear(x, w, T, K, 3)
    assert y.shape == (T, 3)
    assert not np.array_equal(y, oracle.linear(x, np.ascontiguousarray(w[::-1]), T, K, 3))


def test_linear_matches_torch_float32_linear():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(0x5EED0102)
    T, K, N = 9, 512, 40
    x, w = _f16(rng, (T, K)), _f16(rng, (N, K), 0.05)
    ref = torch.nn.functional.linear(torch.from_numpy(x).float(), torch.from_numpy(w).float())
    ref16 = ref.half().numpy()
    got = oracle.linear(x, w, T, K, N).view(np.float16)
    cmp = oracle.compare(got, ref16)
    assert cmp["bad"] == 0 and cmp["exact"] > 0.97, cmp


# ------------------------------------------------------------------------------------------
# engine_forward
# ------------------------------------------------------------------------------------------
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "hf_goldens.npz")


def _hf_case():
    """The whole-model Hugging Face case of tests/golden/hf_goldens.npz: the seeded weights
    (regenerated here and checked against the hash the fixture records), the prompt's token ids
    and LlamaForCausalLM's float32 logits over it."""
    import hashlib
    import json
    g = np.load(GOLDEN)
    meta = json.loads(bytes(g["meta_json"]).decode())["llama"]
    assert meta["config"] == TINY
    w = _tiny_weights(meta["weight_seed"], embed_std=meta["embed_std"])
    h = hashlib.sha256()
    for k in sorted(w):
        h.update(k.encode())
        h.update(np.ascontiguousarray(w[k]).view(np.uint16).tobytes())
    assert h.hexdigest() == meta["weights_sha256"], "tiny_weights no longer gives the fixture's"
    return w, g["llama_ids"].astype(np.int64), g["llama_logits"].astype(np.float64)


def _prompt_rows(ids, pages, max_pages, start=0):
    T = len(ids)
    tables = np.zeros((T, max_pages), np.int32)
    tables[:, :len(pages)] = pages
    return np.asarray(ids, np.int32), np.arange(start, start + T, dtype=np.int32), tables


def test_engine_forward_matches_hugging_face_llama():
    """The oracle's forward pass over a prompt (one row per token, all with the sequence's
    shuffled block table) against LlamaForCausalLM in float32 on the same weights (the committed
    fixture tests/golden/hf_goldens.npz, made by tests/golden/make_hf_goldens.py): logits of
    every position within a relative L2 of 5e-3 (the reference's bar for its fp16 engine
    against Hugging Face; measured 1.0e-3), and the same greedy token wherever Hugging Face's
    top two differ by more than 0.05."""
    w, ids, ref = _hf_case()
    rng = np.random.default_rng(0x5EED0112)
    T, max_pages, num_pages = len(ids), 8, 16
    pages = rng.permutation(num_pages)[:max_pages].astype(np.int32)
    tok, pos, tab = _prompt_rows(ids, pages, max_pages)
    kp, vp = _pools(num_pages)
    logits, nxt, _ = oracle.engine_forward(TINY, w, tok, pos, tab, kp, vp)
    got = logits.view(np.float16).astype(np.float64)
    rel = np.linalg.norm(got - ref, axis=1) / np.linalg.norm(ref, axis=1)
    assert rel.max() < 5e-3, rel.max()
    top2 = np.sort(ref, axis=1)[:, -2:]
    clear = top2[:, 1] - top2[:, 0] > 0.05
    assert clear.sum() >= T // 2
    assert np.array_equal(nxt[clear], ref.argmax(1)[clear])
    # a mutant that pairs RoPE elements (2i, 2i+1) or drops the norm weight would not pass; one
    # that forgets the rotation altogether is checked here: positions all 0 differ from HF
    bad, _, _ = oracle.engine_forward(TINY, w, tok, np.zeros_like(pos), tab, *_pools(num_pages))
    bad_rel = (np.linalg.norm(bad.view(np.float16).astype(np.float64) - ref, axis=1)
               / np.linalg.norm(ref, axis=1))
    assert bad_rel[1:].max() > 5e-2


def test_engine_forward_rows_split_into_chunks_give_the_same_result():
    """A prompt as one batch of rows, or as a prefix batch followed by the remaining rows one
    decode step at a time, writes the same pools and gives bit-identical logits: every op is
    row-wise, and a row's attention reads only positions <= its own."""
    w = _tiny_weights(0x5EED0112)
    rng = np.random.default_rng(0x5EED0113)
    T, max_pages, num_pages = 37, 4, 9
    ids = rng.integers(0, TINY["vocab"], T)
    pages = rng.permutation(num_pages)[:max_pages].astype(np.int32)
    tok, pos, tab = _prompt_rows(ids, pages, max_pages)
    kp1, vp1 = _pools(num_pages)
    full, full_next, _ = oracle.engine_forward(TINY, w, tok, pos, tab, kp1, vp1)
    kp2, vp2 = _pools(num_pages)
    split = 21
    part, _, _ = oracle.engine_forward(TINY, w, tok[:split], pos[:split], tab[:split], kp2, vp2)
    rows = [part]
    for t in range(split, T):
        lg, _, _ = oracle.engine_forward(TINY, w, tok[t:t + 1], pos[t:t + 1], tab[t:t + 1], kp2,
                                         vp2)
        rows.append(lg)
    assert np.array_equal(np.concatenate(rows), full)
    for a, b in zip(kp1 + vp1, kp2 + vp2):
        assert np.array_equal(a, b)
    # slots past the prompt keep the 0x7F7F poison; exactly T slots per pool were written
    kvd = TINY["n_kv_heads"] * TINY["head_dim"]
    written = (kp1[0].reshape(-1, kvd) != 0x7F7F).any(1).sum()
    assert written == T
    # logit rows: a subset gives the same rows
    sub, sub_next, _ = oracle.engine_forward(TINY, w, tok, pos, tab, *_pools(num_pages),
                                             logit_rows=[T - 1, 3])
    assert np.array_equal(sub, full[[T - 1, 3]])
    assert np.array_equal(sub_next, full_next[[T - 1, 3]])


def test_weights_dir_round_trip(tmp_path, llmk):
    import importlib
    weights = importlib.import_module("llmk.weights")
    w = _tiny_weights(0x5EED0114)
    weights.write_weights_dir(str(tmp_path), w)
    back = weights.read_weights_dir(str(tmp_path))
    assert set(back) == set(w)
    for k in w:
        assert back[k].shape == w[k].shape and np.array_equal(back[k].view(np.uint16),
                                                              w[k].view(np.uint16))
    # index.tsv lines: name, offset, nbytes, shape -- sorted names, back-to-back offsets
    lines = open(tmp_path / "index.tsv").read().splitlines()
    names = [ln.split("\t")[0] for ln in lines]
    assert names == sorted(w)
    off = 0
    for ln in lines:
        name, o, nb, shape = ln.split("\t")
        assert int(o) == off and int(nb) == w[name].nbytes
        assert tuple(int(d) for d in shape.split(",")) == w[name].shape
        off += int(nb)
    assert os.path.getsize(tmp_path / "weights.bin") == off
