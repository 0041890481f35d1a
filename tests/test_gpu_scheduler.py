"""The continuous-batching scheduler driving the engine on the GPU, as the reference's scheduler
test does (ref: tests/test_scheduler.cu:14-76): the same workload one request at a time and
several at once gives the same greedy outputs, they match the oracle (the reference's loop
restated, driving the oracle's forward pass), and every page returns to the allocator.

The model is the small Llama-3 shape with seeded random weights (the real checkpoint is not
available offline); the embedding scale makes its logits clearly peaked, so greedy choices do
not hinge on last-bit differences between GEMM algorithms of different batch sizes. The
engine's row limit is below the longest prompts, so prefills run in chunks; decode steps go
through the engine's HIP graph cache.
"""
import numpy as np
import pytest
import torch

from _helpers import TINY, oracle_pools, tiny_weights
from test_gpu_engine import make_engine

pytestmark = pytest.mark.gpu
P = 16


def workload(seed, n=12):
    rng = np.random.default_rng(seed)
    return [{"id": i, "prompt": rng.integers(0, TINY["vocab"], int(rng.integers(3, 60))).tolist(),
             "max_new": int(rng.integers(1, 9)), "arrival_step": i} for i in range(n)]


class OracleModel:
    def __init__(self, orc, w, num_pages):
        self.orc, self.w = orc, {k: np.asarray(v).view(np.uint16) for k, v in w.items()}
        self.kp, self.vp = oracle_pools(num_pages)

    def prefill(self, table, prompt):
        n = len(prompt)
        tabs = np.tile(np.asarray(table, np.int32), (n, 1))
        _, nxt, _ = self.orc.engine_forward(TINY, self.w, prompt, np.arange(n, dtype=np.int32),
                                            tabs, self.kp, self.vp, [n - 1], threads=16)
        return int(nxt[0])

    def decode(self, tokens, positions, tables):
        _, nxt, _ = self.orc.engine_forward(TINY, self.w, tokens, positions, tables, self.kp,
                                            self.vp, threads=16)
        return nxt.tolist()


def test_scheduler_with_the_engine(llmk, orc):
    w = tiny_weights(0x5EED0400, embed_std=0.5)
    num_pages, max_pages, max_rows = 48, 8, 16
    eng = make_engine(llmk, TINY, w, max_rows, max_pages, num_pages)
    stream = torch.cuda.Stream()
    model = eng.sched_model(stream)
    reqs = workload(0x5EED0401)
    order = np.random.default_rng(0x5EED0402).permutation(num_pages).astype(np.int32)
    results = {}
    for max_running in (1, 4):
        pages = llmk.PageAllocator(num_pages)
        pages.set_free_list(order)
        outs, stats, _ = llmk.run_scheduler(reqs, max_running, max_pages, P, pages, model)
        print(f"max_running {max_running}: {stats}", flush=True)
        assert pages.num_free() == num_pages
        assert stats["total_words"] == sum(r["max_new"] for r in reqs)
        results[max_running] = (outs, stats)
    assert results[1][0] == results[4][0]
    assert results[4][1]["decode_steps"] < results[1][1]["decode_steps"]
    om = OracleModel(orc, w, num_pages)
    o_outs, o_stats, o_free = orc.scheduler_run(reqs, 4, max_pages, P, list(order), om.prefill,
                                                om.decode)
    assert results[4][0] == o_outs
    assert results[4][1]["decode_steps"] == o_stats["decode_steps"]
    assert sorted(o_free) == list(range(num_pages))


def test_scheduler_host_argmax_mode(llmk):
    """The reference's default mode (run_scheduler without gpu_argmax): the logits come back to
    the host, are converted to float there and searched with its rule (first maximum wins;
    ref: engine/scheduler.cu:9-13,88-93). The same workload gives the same tokens as the GPU
    argmax, one at a time and batched, and the time split is filled in as the reference fills
    it: prep, GPU, copy, convert and argmax in host mode; convert and argmax stay 0 in GPU
    mode, and the GPU time of the steps never exceeds their host-observed time."""
    w = tiny_weights(0x5EED0410, embed_std=0.5)
    num_pages, max_pages, max_rows = 48, 8, 16
    eng = make_engine(llmk, TINY, w, max_rows, max_pages, num_pages)
    stream = torch.cuda.Stream()
    model = eng.sched_model(stream)
    reqs = workload(0x5EED0411)
    order = np.random.default_rng(0x5EED0412).permutation(num_pages).astype(np.int32)

    def run(max_running):
        pages = llmk.PageAllocator(num_pages)
        pages.set_free_list(order)
        outs, stats, _ = llmk.run_scheduler(reqs, max_running, max_pages, P, pages, model)
        assert pages.num_free() == num_pages
        return outs, stats

    gpu = {mr: run(mr) for mr in (1, 4)}
    eng.set_option(llmk.ENGINE_HOST_ARGMAX, 1)
    host = {mr: run(mr) for mr in (1, 4)}
    eng.set_option(llmk.ENGINE_HOST_ARGMAX, 0)
    again = run(4)
    for mr in (1, 4):
        assert host[mr][0] == gpu[mr][0], mr
        h, g = host[mr][1], gpu[mr][1]
        print(f"max_running {mr}: host {h}\n  gpu {g}", flush=True)
        assert h["decode_steps"] == g["decode_steps"]
        for key in ("prep_ms", "gpu_ms", "copy_ms", "convert_ms", "argmax_ms"):
            assert h[key] > 0, key
        for key in ("prep_ms", "gpu_ms", "copy_ms"):
            assert g[key] > 0, key
        assert g["convert_ms"] == 0 and g["argmax_ms"] == 0
        assert h["gpu_ms"] <= h["decode_ms"] and g["gpu_ms"] <= g["decode_ms"]
    assert again[0] == gpu[4][0]
