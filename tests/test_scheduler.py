"""CPU tests of the page allocator and the continuous-batching scheduler (host code in libllmk;
no GPU call is made).

The model is a fake with paged memory: prefill and decode write each row's token into its pool
slot (page = table[pos // 16], slot pos % 16), and the next token is a hash of every token the
row reads back through its table, positions 0 .. pos. A request's outputs are therefore fixed by
its prompt alone -- unless the scheduler hands one page to two live sequences, releases pages
early, or mis-addresses a table, in which case reads return another sequence's tokens and the
outputs change. The reference checks the same property with real logits (one-at-a-time and
batched runs both match Hugging Face, ref: tests/test_scheduler.cu:48-67) and its page-leak
check (ref: tests/test_scheduler.cu:72-74).

The C++ scheduler is also run against oracle.scheduler_run, a step-for-step restatement of
ref: engine/scheduler.cu:15-106: both must make the same model calls in the same order.
"""
import numpy as np
import pytest

import oracle

P, VOCAB = 16, 50021


def expected_outputs(prompt, max_new):
    hist, out = list(prompt), []
    for _ in range(max_new):
        t = token_hash(hist)
        out.append(t)
        hist.append(t)
    return out[:max_new]


def token_hash(tokens):
    h = 1469598103934665603
    for i, t in enumerate(tokens):
        h = ((h ^ (int(t) + 7 * i)) * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    return int(h % VOCAB)


class FakePagedModel:
    def __init__(self, num_pages, max_pages):
        self.slots = np.full((num_pages, P), -1, np.int64)
        self.max_pages = max_pages
        self.calls = []

    def _row(self, table, tok, pos):
        self.slots[table[pos // P], pos % P] = tok
        hist = [self.slots[table[p // P], p % P] for p in range(pos + 1)]
        assert min(hist) >= 0, "read of a slot never written"
        return token_hash(hist)

    def prefill(self, table, prompt):
        self.calls.append(("prefill", tuple(table), tuple(prompt)))
        t = None
        for pos, tok in enumerate(prompt):
            t = self._row(table, tok, pos)
        return t

    def decode(self, tokens, positions, tables):
        self.calls.append(("decode", tuple(tokens), tuple(positions),
                           tuple(map(tuple, tables))))
        # every row's table must be distinct in its used pages (no page shared in one batch)
        used = [set(tab[:pos // P + 1]) for tab, pos in zip(tables, positions)]
        for i in range(len(used)):
            for j in range(i):
                assert not (used[i] & used[j]), "two running sequences share a page"
        return [self._row(tab, tok, pos) for tok, pos, tab in zip(tokens, positions, tables)]


def workload(rng, n, spacing=2, max_new_range=(1, 12), prompt_range=(1, 60)):
    reqs = []
    for i in range(n):
        L = int(rng.integers(*prompt_range))
        reqs.append({"id": i, "prompt": rng.integers(0, VOCAB, L).tolist(),
                     "max_new": int(rng.integers(*max_new_range)), "arrival_step": i * spacing})
    return reqs


def run_cpp(llmk, reqs, max_running, num_pages, max_pages, order=None):
    pages = llmk.PageAllocator(num_pages)
    if order is not None:
        pages.set_free_list(order)
    fake = FakePagedModel(num_pages, max_pages)
    m = llmk.python_sched_model(fake.prefill, fake.decode)
    outs, stats, times = llmk.run_scheduler(reqs, max_running, max_pages, P, pages, m)
    return outs, stats, times, fake, pages


def run_oracle(reqs, max_running, num_pages, max_pages, order=None, **rule):
    fake = FakePagedModel(num_pages, max_pages)
    free = list(range(num_pages - 1, -1, -1)) if order is None else list(order)
    outs, stats, free_end = oracle.scheduler_run(reqs, max_running, max_pages, P, free,
                                                 fake.prefill, fake.decode, **rule)
    return outs, stats, fake, free_end


def test_page_allocator_hands_out_page_zero_first_and_checks_releases(llmk):
    a = llmk.PageAllocator(5)
    assert a.total == 5 and a.num_free() == 5
    assert [a.alloc() for _ in range(5)] == [0, 1, 2, 3, 4]
    assert a.alloc() == -1 and a.num_free() == 0
    a.release(3)
    a.release(1)
    assert a.alloc() == 1 and a.alloc() == 3          # last released, first handed out
    with pytest.raises(llmk.LlmkError):
        a.release(7)                                   # out of range
    a.release(2)
    with pytest.raises(llmk.LlmkError):
        a.release(2)                                   # already free
    a.set_free_list([2])
    with pytest.raises(llmk.LlmkError):
        a.set_free_list([0])                           # 0 is in use
    with pytest.raises(llmk.LlmkError):
        a.set_free_list([2, 2])
    assert llmk.lib().llmk_pages_create(0, None) == llmk.LLMK_ERR_INVALID_VALUE


@pytest.mark.parametrize("max_running", [1, 3, 8])
def test_outputs_are_each_requests_own_and_pages_all_return(llmk, max_running):
    rng = np.random.default_rng(0x5EED0300 + max_running)
    reqs = workload(rng, 24)
    num_pages, max_pages = 40, 8
    order = rng.permutation(num_pages).astype(np.int32)   # shuffled free list
    outs, stats, times, fake, pages = run_cpp(llmk, reqs, max_running, num_pages, max_pages,
                                             order)
    for r, o in zip(reqs, outs):
        assert o == expected_outputs(r["prompt"], r["max_new"]), r["id"]
    assert pages.num_free() == num_pages                  # no leak
    assert stats["total_words"] == sum(r["max_new"] for r in reqs)
    assert stats["max_batch"] <= max_running
    assert stats["prefills"] == len(reqs)
    for (ta, tf, td), r in zip(times, reqs):
        assert 0 <= ta <= tf <= td


@pytest.mark.parametrize("max_running,num_pages", [(1, 12), (4, 12), (8, 40), (8, 9)])
def test_schedule_matches_the_reference_loop(llmk, max_running, num_pages):
    """Same model calls, in the same order, as the restatement of the reference's loop -- also
    under page pressure (9 or 12 pages for prompts of up to 60 tokens plus 11 new ones), where
    admission waits until the free pages, less those the admitted requests are still owed,
    hold the next request's quota."""
    rng = np.random.default_rng(0x5EED0310 + max_running + num_pages)
    reqs = workload(rng, 20, spacing=1)
    max_pages = 8
    order = rng.permutation(num_pages).astype(np.int32)
    outs, stats, _, fake, pages = run_cpp(llmk, reqs, max_running, num_pages, max_pages, order)
    o_outs, o_stats, o_fake, o_free = run_oracle(reqs, max_running, num_pages, max_pages, order)
    assert fake.calls == o_fake.calls
    assert outs == o_outs
    for k in ("decode_steps", "iterations", "total_words"):
        assert stats[k] == o_stats[k], k
    assert stats["mean_batch"] == pytest.approx(o_stats["mean_batch"])
    assert pages.num_free() == num_pages and len(o_free) == num_pages


def test_a_strict_admission_rule_is_caught(llmk):
    """A restatement that admits only when the spare pages exceed the quota (> for >=) makes
    other model calls than the library under page pressure, so the comparison above would catch
    that mistake; the correct restatement matches on the same cases."""
    caught = 0
    for seed in range(6):
        rng = np.random.default_rng(0x5EED0330 + seed)
        reqs = workload(rng, 20, spacing=1)
        num_pages, max_pages = 9, 8
        order = rng.permutation(num_pages).astype(np.int32)
        _, stats, _, fake, _ = run_cpp(llmk, reqs, 4, num_pages, max_pages, order)
        _, o_stats, o_fake, _ = run_oracle(reqs, 4, num_pages, max_pages, order)
        assert fake.calls == o_fake.calls, seed
        _, m_stats, m_fake, _ = run_oracle(reqs, 4, num_pages, max_pages, order,
                                           fits=lambda spare, quota: spare > quota)
        caught += m_fake.calls != fake.calls
    assert caught >= 3, f"the strict rule changed the calls in only {caught} of 6 workloads"


def test_batching_raises_throughput_in_model_calls(llmk):
    """More requests at once means fewer decode steps for the same words, the reference's
    headline effect (ref: docs/scheduler_results.md: 744 steps one at a time, 107 with up to
    8)."""
    rng = np.random.default_rng(0x5EED0320)
    reqs = workload(rng, 24, max_new_range=(8, 9))
    one, s1, *_ = run_cpp(llmk, reqs, 1, 64, 8)
    many, s8, *_ = run_cpp(llmk, reqs, 8, 64, 8)
    assert one == many
    assert s8["decode_steps"] < s1["decode_steps"] / 2
    assert s8["mean_batch"] > 3 * s1["mean_batch"]


def test_a_request_that_can_never_fit_is_an_error_and_pages_come_back(llmk):
    reqs = [{"prompt": [1] * 20, "max_new": 4, "arrival_step": 0},
            {"prompt": [2] * 100, "max_new": 40, "arrival_step": 0}]   # 9 pages, pool of 6
    pages = llmk.PageAllocator(6)
    fake = FakePagedModel(6, 16)
    with pytest.raises(llmk.LlmkError) as ei:
        llmk.run_scheduler(reqs, 2, 16, P, pages, llmk.python_sched_model(fake.prefill,
                                                                         fake.decode))
    assert ei.value.status == llmk.LLMK_ERR_CAPACITY
    assert pages.num_free() == 6
    with pytest.raises(RuntimeError):
        oracle.scheduler_run(reqs, 2, 16, P, list(range(5, -1, -1)), fake.prefill, fake.decode)
    # a request longer than a block table
    with pytest.raises(llmk.LlmkError) as ei:
        llmk.run_scheduler([{"prompt": [1] * 40, "max_new": 1, "arrival_step": 0}], 1, 2, P,
                           llmk.PageAllocator(8), llmk.python_sched_model(fake.prefill,
                                                                          fake.decode))
    assert ei.value.status == llmk.LLMK_ERR_CAPACITY


def test_invalid_requests_are_rejected(llmk):
    fake = FakePagedModel(8, 4)
    m = llmk.python_sched_model(fake.prefill, fake.decode)
    bad = [[{"prompt": [], "max_new": 1, "arrival_step": 0}],
           [{"prompt": [1], "max_new": 0, "arrival_step": 0}],
           [{"prompt": [1], "max_new": 1, "arrival_step": 3},
            {"prompt": [1], "max_new": 1, "arrival_step": 1}]]      # not sorted by arrival
    for reqs in bad:
        with pytest.raises(llmk.LlmkError):
            llmk.run_scheduler(reqs, 1, 4, P, llmk.PageAllocator(8), m)
    assert fake.calls == []


def test_a_model_error_ends_the_run_and_returns_the_pages(llmk):
    pages = llmk.PageAllocator(16)
    calls = {"n": 0}

    def prefill(table, prompt):
        return 5

    def decode(tokens, positions, tables):
        calls["n"] += 1
        if calls["n"] == 3:
            raise ValueError("device lost")
        return [7] * len(tokens)

    reqs = [{"prompt": [1, 2, 3], "max_new": 10, "arrival_step": 0} for _ in range(3)]
    with pytest.raises(ValueError):
        llmk.run_scheduler(reqs, 3, 4, P, pages, llmk.python_sched_model(prefill, decode))
    assert pages.num_free() == 16


@pytest.mark.parametrize("max_running,steps", [(1, 744), (8, 107)])
def test_the_reference_workload_gives_its_published_schedule(llmk, max_running, steps):
    """The reference's scheduler benchmark (ref: tests/test_scheduler.cu:15,35-40): its 8 prompt
    lengths three times, 32 new tokens each, one request every 2 iterations, 256 pages. The
    reference publishes 744 decode steps one at a time and 107 with up to 8 at once, mean batch
    7.0 (docs/scheduler_results.md); the schedule depends only on the lengths and the rules, so
    this scheduler must reproduce both counts."""
    import importlib
    wl = importlib.import_module("llmk.workloads")
    reqs = wl.scheduler_requests()
    assert [len(r["prompt"]) for r in reqs[:8]] == [6, 5, 5, 11, 12, 15, 12, 402]
    max_pages = (max(len(r["prompt"]) for r in reqs) + wl.SCHED_NEW + P - 1) // P
    outs, stats, _, fake, pages = run_cpp(llmk, reqs, max_running, wl.SCHED_PAGES, max_pages)
    assert stats["decode_steps"] == steps
    assert stats["total_words"] == 24 * 32
    assert round(stats["mean_batch"], 1) == (1.0 if max_running == 1 else 7.0)
    assert pages.num_free() == wl.SCHED_PAGES
    assert outs == [expected_outputs(r["prompt"], r["max_new"]) for r in reqs]
    o_outs, o_stats, _, _ = run_oracle(reqs, max_running, wl.SCHED_PAGES, max_pages)
    assert o_stats["decode_steps"] == steps and o_outs == outs
