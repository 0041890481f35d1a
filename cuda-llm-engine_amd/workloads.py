"""Seeded synthetic workloads of the benchmark configurations, built directly in device memory,
and the algorithmic byte count of each kernel (bytes that must cross HBM once: inputs read
once, outputs written once).

Shapes are Llama-3.2-1B's (ref: engine/layer.h:6-9, engine/model.cu:20): hidden 2048, 32 query
heads, 8 KV heads, head_dim 64, MLP width 8192, vocab 128256, 16 layers, KV pages of 16 tokens
in per-layer pools laid out [num_pages, page_size, n_kv_heads, head_dim] (ref:
engine/paged.h:6-9) and filled with the fp16 NaN pattern 0x7F7F (ref: engine/paged.cu:22).

Random data comes from torch's device generator (fp32 normal draws rounded to fp16); page
assignment from a seeded numpy permutation, as the reference's paged tests shuffle their free
list (ref: tests/test_generate_batched.cu:28-29).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

HIDDEN, N_HEADS, N_KV, HEAD_DIM, INTER, VOCAB, LAYERS = 2048, 32, 8, 64, 8192, 128256, 16
PAGE, EPS = 16, 1e-5
ROPE_ARGS = (500000.0, 32.0, 1.0, 4.0, 8192.0)  # theta, factor, low, high, original max pos
MAX_POS = 131072
POISON = 0x7F7F
SEED_BASE = 0x5EED0000


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def normal_f16(shape, g, device, mean=0.0, std=1.0) -> torch.Tensor:
    t = torch.randn(shape, generator=g, device=device, dtype=torch.float32)
    if std != 1.0:
        t.mul_(std)
    if mean != 0.0:
        t.add_(mean)
    return t.to(torch.float16)


def poisoned(numel: int, device) -> torch.Tensor:
    return torch.full((numel,), POISON, dtype=torch.int16, device=device).view(torch.float16)


# ---------------------------------------------------------------------------------------------
# algorithmic bytes per launch
# ---------------------------------------------------------------------------------------------
def bytes_add_rmsnorm(rows: int, hidden: int) -> int:
    return 4 * rows * hidden * 2 + hidden * 2  # read residual + x, write residual + out; w once


def bytes_rmsnorm(rows: int, hidden: int) -> int:
    return 2 * rows * hidden * 2 + hidden * 2


def bytes_residual_add(n: int) -> int:
    return 3 * n * 2  # a and b read, out written


def bytes_kv_scatter(T: int, kvdim: int, page_size: int = PAGE) -> int:
    # source rows read, pool rows written, one table entry per page touched
    return 2 * T * kvdim * 2 + (T + page_size - 1) // page_size * 4


def bytes_kv_scatter_batch(n: int, kvdim: int) -> int:
    return n * (2 * kvdim * 2 + 4 + 4)  # the row read and written; its position and table entry


def bytes_rope(T: int, nh: int, nkv: int, hd: int) -> int:
    return 2 * T * (nh + nkv) * hd * 2 + T * 4 + hd // 2 * 4  # q, k in place; positions; table


def bytes_swiglu(n: int) -> int:
    return 3 * n * 2


def bytes_embedding(n: int, hidden: int) -> int:
    return n * 4 + 2 * n * hidden * 2  # ids; the gathered rows read once and written once


def bytes_rope_kv_scatter(n: int, nh: int, nkv: int, hd: int) -> int:
    q = 2 * n * nh * hd * 2           # q rotated in place
    kv = 2 * 2 * n * nkv * hd * 2     # k and v read, their pool rows written
    return q + kv + n * 4 + n * 4 + hd // 2 * 4  # positions, the one table entry each
    # sequence's row address needs, the rotation table


def bytes_decode_pass(n: int, layers: int, two_norms: bool = False) -> int:
    per_layer = ((2 if two_norms else 1) * bytes_add_rmsnorm(n, HIDDEN)
                 + bytes_rope_kv_scatter(n, N_HEADS, N_KV, HEAD_DIM)
                 + bytes_swiglu(n * INTER))
    return bytes_embedding(n, HIDDEN) + layers * per_layer


def bytes_decode_pass_fused(n: int, layers: int, two_norms: bool = False) -> int:
    """What the fused pass (llmk_decode_nongemm_pass_fused) must move: config 5's bytes less
    the residual rows it keeps in registers -- the embedding rows are not written and re-read,
    and per layer the residual is stored once (after its last add) and never re-read."""
    row = n * HIDDEN * 2
    saved = row + layers * (3 if two_norms else 1) * row
    return bytes_decode_pass(n, layers, two_norms) - saved


def bytes_attention(lens: np.ndarray, nh: int = N_HEADS, nkv: int = N_KV,
                    hd: int = HEAD_DIM) -> int:
    """Cached K and V rows of every sequence read once, q read and out written once, plus the
    page-table entries and lengths read."""
    lens = np.maximum(np.asarray(lens, np.int64), 0)
    pages = (lens + PAGE - 1) // PAGE
    return (int(lens.sum()) * 2 * nkv * hd * 2 + 2 * lens.size * nh * hd * 2
            + int(pages.sum()) * 4 + lens.size * 4)


def bytes_argmax(n: int, vocab: int) -> int:
    return n * vocab * 2 + n * 4  # logits read once, one int32 per row written


def bytes_linear(T: int, in_f: int, out_f: int) -> int:
    return out_f * in_f * 2 + T * in_f * 2 + T * out_f * 2  # weights and x read once, y written


def bytes_decode_step(lens: np.ndarray, layers: int = LAYERS) -> int:
    """Sum of the algorithmic bytes of every kernel of one engine forward pass over one decode
    row per sequence (context lengths `lens`, the new token included): embedding, per layer the
    QKV projection, RoPE + K/V scatter from the QKV rows, attention, o projection, add+RMSNorm,
    gate/up projection, SwiGLU, down projection, add+RMSNorm; then the lm head and argmax.
    Activations count once as written and once as read, as they cross HBM between kernels."""
    n = int(np.asarray(lens).size)
    qdim, kvdim = N_HEADS * HEAD_DIM, N_KV * HEAD_DIM
    qkv = qdim + 2 * kvdim
    per_layer = (bytes_linear(n, HIDDEN, qkv)
                 + n * qkv * 2 + n * qdim * 2 + 2 * n * kvdim * 2 + 2 * n * 4 + HEAD_DIM // 2 * 4
                 + bytes_attention(lens)
                 + bytes_linear(n, qdim, HIDDEN)
                 + bytes_add_rmsnorm(n, HIDDEN)
                 + bytes_linear(n, HIDDEN, 2 * INTER)
                 + bytes_swiglu(n * INTER)
                 + bytes_linear(n, INTER, HIDDEN)
                 + bytes_add_rmsnorm(n, HIDDEN))
    return (bytes_embedding(n, HIDDEN) + bytes_rmsnorm(n, HIDDEN) + layers * per_layer
            + bytes_linear(n, HIDDEN, VOCAB) + bytes_argmax(n, VOCAB))


def decode_step_rows(lens: np.ndarray, max_pages: int = 128, seed: int = SEED_BASE + 8):
    """One decode row per sequence: a token id, position len - 1, and the sequence's block table
    over pages assigned from a shuffled permutation (unused entries 0). Returns (tokens,
    positions, tables [n, max_pages], number of pages used)."""
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, np.int64)
    npages = (lens + PAGE - 1) // PAGE
    total = int(npages.sum())
    perm = rng.permutation(total).astype(np.int32)
    tables = np.zeros((lens.size, max_pages), np.int32)
    at = 0
    for b, k in enumerate(npages):
        tables[b, :k] = perm[at:at + k]
        at += k
    tokens = rng.integers(0, VOCAB, lens.size).astype(np.int32)
    return tokens, (lens - 1).astype(np.int32), tables, total


# The reference's continuous-batching workload (ref: tests/test_scheduler.cu:15,35-40,
# docs/scheduler_results.md): its 8 prompts (token counts from tests/reference/reference.json),
# three times each, 32 new tokens per request, one request eligible every 2 scheduler
# iterations, 256 pages of 16 positions, at most 8 sequences at once.
SCHED_PROMPT_LENS = (6, 5, 5, 11, 12, 15, 12, 402)
SCHED_REQUESTS, SCHED_NEW, SCHED_SPACING, SCHED_PAGES, SCHED_MAX_RUNNING = 24, 32, 2, 256, 8


def scheduler_requests(seed: int = SEED_BASE + 11) -> list:
    """The reference scheduler workload with seeded synthetic prompt ids (the weights are random,
    so the prompts' text does not matter; their lengths set the prefill work)."""
    rng = np.random.default_rng(seed)
    prompts = [rng.integers(0, VOCAB, n).tolist() for n in SCHED_PROMPT_LENS]
    return [{"id": i, "prompt": prompts[i % len(prompts)], "max_new": SCHED_NEW,
             "arrival_step": i * SCHED_SPACING} for i in range(SCHED_REQUESTS)]


def attention_lens(n: int = 256, max_len: int = 2048, seed: int = SEED_BASE + 6) -> np.ndarray:
    """Sequence lengths uniform in [1, max_len] (the decode configuration's context lengths)."""
    return np.random.default_rng(seed).integers(1, max_len + 1, n)


# ---------------------------------------------------------------------------------------------
# workloads
# ---------------------------------------------------------------------------------------------
def add_rmsnorm_inputs(rows=8192, hidden=HIDDEN, seed=SEED_BASE + 2, device="cuda") -> dict:
    g = _gen(seed, device)
    return dict(residual=normal_f16((rows, hidden), g, device),
                x=normal_f16((rows, hidden), g, device),
                w=normal_f16((hidden,), g, device, 1.0, 0.1),
                out=torch.empty((rows, hidden), dtype=torch.float16, device=device),
                rows=rows, hidden=hidden, eps=EPS)


def rope_inputs(T=8192, nh=N_HEADS, nkv=N_KV, hd=HEAD_DIM, seed=SEED_BASE + 3,
                device="cuda", inv_freq=None) -> dict:
    g = _gen(seed, device)
    return dict(q=normal_f16((T, nh, hd), g, device), k=normal_f16((T, nkv, hd), g, device),
                positions=torch.randint(0, MAX_POS, (T,), generator=g, device=device,
                                        dtype=torch.int32),
                inv_freq=inv_freq, T=T, nh=nh, nkv=nkv, hd=hd)


def swiglu_inputs(rows=8192, inter=INTER, seed=SEED_BASE + 4, device="cuda") -> dict:
    g = _gen(seed, device)
    return dict(gate=normal_f16((rows, inter), g, device), up=normal_f16((rows, inter), g, device),
                out=torch.empty((rows, inter), dtype=torch.float16, device=device),
                n=rows * inter)


def embedding_table(vocab=VOCAB, hidden=HIDDEN, seed=SEED_BASE + 40, device="cuda"):
    return normal_f16((vocab, hidden), _gen(seed, device), device, 0.0, 0.02)


def embedding_inputs(n=8192, table=None, seed=SEED_BASE + 41, device="cuda") -> dict:
    if table is None:
        table = embedding_table(device=device)
    g = _gen(seed, device)
    return dict(table=table,
                ids=torch.randint(0, table.shape[0], (n,), generator=g, device=device,
                                  dtype=torch.int32),
                out=torch.empty((n, table.shape[1]), dtype=torch.float16, device=device),
                n=n, hidden=table.shape[1])


@dataclass
class DecodePassInputs:
    """Config 5: one non-GEMM decode step for n sequences over `layers` layers."""
    n: int
    layers: int
    max_pages: int
    total_pages: int
    lens: np.ndarray             # context lengths L_b (host)
    tables_host: np.ndarray      # [n, max_pages] int32
    table: torch.Tensor          # embedding table [vocab, hidden]
    token_ids: torch.Tensor      # [n]
    residual: torch.Tensor       # [n, hidden]
    block_tables: torch.Tensor   # [n, max_pages]
    positions: torch.Tensor      # [n] = L_b - 1
    inv_freq: torch.Tensor       # [hd/2]
    per_layer: list = field(default_factory=list)  # dicts for llmk.DecodeNonGemmPass

    def pool_rows(self) -> np.ndarray:
        """Pool row written for each sequence (host)."""
        pos = self.lens - 1
        return (self.tables_host[np.arange(self.n), pos // PAGE] * PAGE + pos % PAGE).astype(
            np.int64)


def decode_pass_inputs(inv_freq: torch.Tensor, n=256, layers=LAYERS, max_pages=128,
                       table=None, seed=SEED_BASE + 5, device="cuda", hidden=HIDDEN,
                       n_heads=N_HEADS, n_kv=N_KV, inter=INTER, vocab=VOCAB,
                       two_norms=False) -> DecodePassInputs:
    """Config 5's inputs (by default); the model dimensions can be changed for shape tests.
    two_norms: each layer also gets x2, norm_w2 and normed2 for its second add + RMSNorm (the
    real layer's two; config 5 lists one)."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(1, max_pages * PAGE + 1, n)
    npages = (lens + PAGE - 1) // PAGE
    total = int(npages.sum())
    perm = rng.permutation(total).astype(np.int32)
    tables = np.zeros((n, max_pages), np.int32)
    off = 0
    for b, p in enumerate(npages):
        tables[b, :p] = perm[off:off + p]
        off += p
    g = _gen(seed, device)
    if table is None:
        table = embedding_table(vocab, hidden, device=device)
    ids = torch.randint(0, table.shape[0], (n,), generator=g, device=device, dtype=torch.int32)
    kvdim = n_kv * HEAD_DIM
    per_layer = []
    for _ in range(layers):
        per_layer.append(dict(
            x=normal_f16((n, hidden), g, device),
            norm_w=normal_f16((hidden,), g, device, 1.0, 0.1),
            normed=torch.empty((n, hidden), dtype=torch.float16, device=device),
            q=normal_f16((n, n_heads, HEAD_DIM), g, device),
            k=normal_f16((n, n_kv, HEAD_DIM), g, device),
            v=normal_f16((n, n_kv, HEAD_DIM), g, device),
            k_pool=poisoned(total * PAGE * kvdim, device),
            v_pool=poisoned(total * PAGE * kvdim, device),
            gate=normal_f16((n, inter), g, device),
            up=normal_f16((n, inter), g, device),
            act=torch.empty((n, inter), dtype=torch.float16, device=device)))
        if two_norms:
            per_layer[-1].update(
                x2=normal_f16((n, hidden), g, device),
                norm_w2=normal_f16((hidden,), g, device, 1.0, 0.1),
                normed2=torch.empty((n, hidden), dtype=torch.float16, device=device))
    return DecodePassInputs(
        n=n, layers=layers, max_pages=max_pages, total_pages=total, lens=lens,
        tables_host=tables, table=table, token_ids=ids,
        residual=torch.empty((n, hidden), dtype=torch.float16, device=device),
        block_tables=torch.from_numpy(tables).to(device),
        positions=torch.from_numpy((lens - 1).astype(np.int32)).to(device),
        inv_freq=inv_freq, per_layer=per_layer)


def attention_inputs(lens: np.ndarray, max_pages: int = 128, num_splits: int = 32,
                     seed: int = SEED_BASE + 6, device="cuda") -> dict:
    """One decode-attention batch: q [n, 32, 64] and the cached K, V rows ~N(0, 1) in pages
    assigned from a shuffled permutation; the slots past each sequence's length in its last page
    hold the NaN pattern; a workspace for num_splits splits."""
    lens = np.asarray(lens, np.int64)
    n = lens.size
    rng = np.random.default_rng(seed + 1)
    npages = (lens + PAGE - 1) // PAGE
    total = int(npages.sum())
    perm = rng.permutation(total).astype(np.int32)
    tables = np.zeros((n, max_pages), np.int32)
    off = 0
    for b, p in enumerate(npages):
        tables[b, :p] = perm[off:off + p]
        off += p
    kvdim = N_KV * HEAD_DIM
    g = _gen(seed, device)
    k_pool = normal_f16((total * PAGE, kvdim), g, device)
    v_pool = normal_f16((total * PAGE, kvdim), g, device)
    tail = [tables[b, npages[b] - 1] * PAGE + j for b in range(n)
            for j in range(int(lens[b]) % PAGE or PAGE, PAGE)]
    if tail:
        idx = torch.tensor(tail, dtype=torch.int64, device=device)
        k_pool.view(torch.int16).index_fill_(0, idx, POISON)
        v_pool.view(torch.int16).index_fill_(0, idx, POISON)
    from . import attention_decode_fast_workspace_floats as ws_floats
    return dict(q=normal_f16((n, N_HEADS, HEAD_DIM), g, device), k_pool=k_pool.view(-1),
                v_pool=v_pool.view(-1), block_tables=torch.from_numpy(tables).to(device),
                seq_lens=torch.from_numpy(lens.astype(np.int32)).to(device),
                out=torch.empty((n, N_HEADS, HEAD_DIM), dtype=torch.float16, device=device),
                workspace=torch.empty(ws_floats(n, N_HEADS, num_splits), dtype=torch.float32,
                                      device=device),
                n=n, max_pages=max_pages, num_splits=num_splits, total_pages=total)
