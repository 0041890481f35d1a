"""GPU parity of the split-KV paged decode attention (llmk_attention_decode_fast) against the
CPU oracle, following the reference's own test (ref: tests/test_attention_decode_fast.cu):
its sequence lengths (page-boundary cases 15/16/17, one position, 2048), its split counts
{1, 2, 3, 8, 16, 32}, pages assigned in shuffled order, every unused pool slot and the output
pre-filled with NaN patterns, and its pass rule |d| <= 1e-3 + 4e-3 |e| for every element.

The kernel sums in another order than the oracle (which follows the reference's plain paged
kernel), so the bar is the reference's tolerance, plus a floor on the bit-identical share: at
least 99% of the output elements equal the oracle's bit for bit (a drift of a systematic kind
on a few percent of the elements fails it)."""
import numpy as np
import pytest
import torch

from _helpers import ATTN_LENS, POISON, assert_tol, attention_case

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
EXACT_FLOOR = 0.99  # share of bit-identical output elements


def dev(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.float16)).to(DEV)


def dev_i32(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(DEV)


def host(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def oracle_out(orc, c):
    return orc.attention_decode_paged(c["q"], c["k_pool"], c["v_pool"], c["tables"], c["lens"],
                                      c["n_seq"], c["max_pages"], c["page_size"], c["n_heads"],
                                      c["n_kv_heads"], c["head_dim"]).reshape(-1)


class OnDevice:
    """One attention case resident on the GPU, runnable at any split count."""

    def __init__(self, c):
        self.c = c
        self.q, self.kp, self.vp = dev(c["q"]), dev(c["k_pool"]), dev(c["v_pool"])
        self.tables, self.lens = dev_i32(c["tables"]), dev_i32(c["lens"])
        self.n_out = c["n_seq"] * c["n_heads"] * c["head_dim"]

    def run(self, llmk, splits, workspace="alloc", stream=None, fill=0x7F7F):
        c = self.c
        out = torch.full((self.n_out + 8,), fill - 65536 if fill >= 32768 else fill,
                         dtype=torch.int16, device=DEV).view(torch.float16)
        if workspace == "alloc":
            ws = torch.full((llmk.attention_decode_fast_workspace_floats(
                c["n_seq"], c["n_heads"], splits),), float("nan"), device=DEV)
        else:
            ws = workspace
        llmk.attention_decode_fast(self.q, self.kp, self.vp, self.tables, self.lens, out, ws,
                                   c["n_seq"], c["max_pages"], c["page_size"], c["n_heads"],
                                   c["n_kv_heads"], c["head_dim"], splits, stream=stream)
        torch.cuda.synchronize()
        got = host(out)
        assert np.all(got[self.n_out:] == (fill & 0xFFFF)), "write past the output"
        return got[:self.n_out]


@pytest.fixture(scope="module")
def reference_case():
    return attention_case(np.random.default_rng(2024), ATTN_LENS)


@pytest.mark.parametrize("splits", [1, 2, 3, 8, 16, 32])
def test_reference_lengths_and_splits(llmk, orc, reference_case, splits):
    """ref: tests/test_attention_decode_fast.cu:66-99, every split count it runs."""
    d = OnDevice(reference_case)
    got = d.run(llmk, splits)
    cmp = orc.compare(got, oracle_out(orc, reference_case))
    print(f"splits {splits}: max_abs {cmp['max_abs']:.2e} exact {100 * cmp['exact']:.2f}%")
    assert_tol(cmp, EXACT_FLOOR, f"attention splits={splits}")


def test_results_do_not_depend_much_on_the_split_count(llmk, orc, reference_case):
    d = OnDevice(reference_case)
    one = d.run(llmk, 1)
    for splits in (2, 5, 32):
        assert_tol(orc.compare(d.run(llmk, splits), one), EXACT_FLOOR, f"splits {splits} vs 1")


@pytest.mark.parametrize("nkv", [1, 2, 3, 4, 5, 6, 7, 12, 16])
def test_other_kv_head_counts(llmk, orc, nkv):
    """The reference accepts any n_kv with 4 query heads each; rows of 1, 2 or 4 kv heads put
    several positions in one 1 KiB row read, 16 kv heads take two blocks per split, and a count
    that is not a multiple of 8 (3, 5, 6, 7, 12) leaves part of its last kv group idle."""
    c = attention_case(np.random.default_rng(nkv), (1, 7, 16, 33, 130, 500), n_heads=4 * nkv,
                       n_kv_heads=nkv)
    d = OnDevice(c)
    for splits in (1, 3):
        cmp = orc.compare(d.run(llmk, splits), oracle_out(orc, c))
        assert_tol(cmp, EXACT_FLOOR, f"n_kv {nkv} splits {splits}")


@pytest.mark.parametrize("splits", [32, 43, 64, 128])
def test_small_batch_in_short_runs(llmk, orc, reference_case, splits):
    """A small batch cut into runs of at most 4 pages takes the sequence-split grid: 4, 3, 2 and
    1 pages per split of a 128-page table (the last one folds 128 pieces of the 2048-position
    sequence, four rounds of the merge)."""
    d = OnDevice(reference_case)
    cmp = orc.compare(d.run(llmk, splits), oracle_out(orc, reference_case))
    assert_tol(cmp, EXACT_FLOOR, f"short runs, splits {splits}")


@pytest.mark.parametrize("nkv", [1, 2, 4, 6, 12, 16])
def test_short_runs_with_other_kv_head_counts(llmk, orc, nkv):
    """Short runs with rows of 1, 2 or 4 kv heads (several positions per row read), with 16
    kv heads (two kv groups) and with 6 and 12 (a partly idle last group): 32-page tables cut
    into runs of 1, 2 and 4 pages."""
    c = attention_case(np.random.default_rng(100 + nkv), (1, 7, 16, 33, 130, 500),
                       n_heads=4 * nkv, n_kv_heads=nkv)
    assert c["max_pages"] == 32
    d = OnDevice(c)
    ref = oracle_out(orc, c)
    for splits in (8, 16, 32):
        assert_tol(orc.compare(d.run(llmk, splits), ref), EXACT_FLOOR, f"n_kv {nkv} splits {splits}")


@pytest.mark.parametrize("lens,nkv", [((2048,), 8), ((2048, 17), 8), ((33, 2048, 1, 500), 8),
                                      ((2048,), 16), ((700, 1500), 16), ((2048,), 12),
                                      ((130, 2048), 12), ((2048,), 6), ((1, 2047), 4)])
def test_very_small_batches_take_narrower_kv_groups(llmk, orc, lens, nkv):
    """At most 8 (sequence, kv group) pairs cut each row into narrower kv groups (2 or 4 heads, a
    row read spanning 4 or 2 positions): 1-4 sequences with 4, 6, 8, 12 and 16 kv heads, at the
    split counts the short-run grid (32), the page-balanced grid (3) and a single split (1)
    take."""
    c = attention_case(np.random.default_rng(300 + nkv + len(lens)), lens, n_heads=4 * nkv,
                       n_kv_heads=nkv)
    d = OnDevice(c)
    ref = oracle_out(orc, c)
    for splits in (1, 3, 32):
        assert_tol(orc.compare(d.run(llmk, splits), ref), EXACT_FLOOR,
                   f"lens {lens} n_kv {nkv} splits {splits}")


@pytest.mark.parametrize("n_seq", [1024, 1025, 3000])
def test_many_sequences(llmk, orc, n_seq):
    """Batches around and past the 1024 sequences (4 tiles of 256 threads) whose page counts the
    page-balanced kernel keeps in registers; past it, each block re-reads the lengths tile by tile
    while it looks for its first sequence. Short contexts (1-48 positions), so blocks cross
    dozens of sequences each; one split (the sequence-split grid), 3 and 32 (page-balanced)."""
    rng = np.random.default_rng(7000 + n_seq)
    c = attention_case(rng, rng.integers(1, 49, n_seq))
    d = OnDevice(c)
    ref = oracle_out(orc, c)
    for splits in (1, 3, 32):
        assert_tol(orc.compare(d.run(llmk, splits), ref), EXACT_FLOOR,
                   f"{n_seq} sequences, splits {splits}")


def test_empty_sequences_give_nan_and_leave_the_rest_intact(llmk, orc):
    c = attention_case(np.random.default_rng(5), (0, 5, -3, 40))
    d = OnDevice(c)
    ref = oracle_out(orc, c).reshape(4, -1)
    for splits in (1, 4):
        got = d.run(llmk, splits, fill=0x1234).reshape(4, -1)
        for b in (0, 2):
            assert np.all(np.isnan(got[b].view(np.float16))), f"seq {b} splits {splits}"
        assert_tol(orc.compare(got[[1, 3]].reshape(-1), ref[[1, 3]].reshape(-1)), EXACT_FLOOR,
                   "non-empty rows")


@pytest.mark.parametrize("lens", [(0, 2048), (2048, -3), (0,), (1,), (1, 1), (1, 2048)])
def test_smallest_batches_empty_and_single_positions(llmk, orc, lens):
    """One or two sequences of 8 kv heads take 2-head kv groups, and at 3 or more splits of
    short runs 2-wave blocks: an empty sequence gives NaN, a single cached position returns its
    V row exactly, and the rest agrees with the oracle, at every split count."""
    n = len(lens)
    c = attention_case(np.random.default_rng(900 + 7 * n + sum(lens)), lens)
    d = OnDevice(c)
    ref = oracle_out(orc, c).reshape(n, -1)
    for splits in (1, 3, 32):
        got = d.run(llmk, splits, fill=0x1234).reshape(n, -1)
        for b, L in enumerate(lens):
            what = f"lens {lens} seq {b} splits {splits}"
            if L <= 0:
                assert np.all(np.isnan(got[b].view(np.float16))), what
            elif L == 1:
                assert np.array_equal(got[b], ref[b]), what
            else:
                assert_tol(orc.compare(got[b], ref[b]), EXACT_FLOOR, what)


def test_single_position_returns_the_value_row_exactly(llmk, orc):
    """Weight exactly 1: out = the V row, bit for bit, whatever the split count."""
    c = attention_case(np.random.default_rng(6), (1,) * 9)
    d = OnDevice(c)
    ref = oracle_out(orc, c)
    for splits in (1, 2, 7):
        assert np.array_equal(d.run(llmk, splits), ref)


def test_workspace_may_be_null_with_one_split(llmk, orc, reference_case):
    d = OnDevice(reference_case)
    got = d.run(llmk, 1, workspace=None)
    assert_tol(orc.compare(got, oracle_out(orc, reference_case)), EXACT_FLOOR, "no workspace")


def test_preconditions_are_reported(llmk, reference_case):
    d = OnDevice(reference_case)
    c = reference_case
    out = torch.empty(d.n_out, dtype=torch.float16, device=DEV)
    ws = torch.empty(llmk.attention_decode_fast_workspace_floats(c["n_seq"], 32, 4), device=DEV)
    base = dict(n_seq=c["n_seq"], max_pages=c["max_pages"], page_size=16, n_heads=32,
                n_kv_heads=8, head_dim=64, num_splits=4)

    def call(**kw):
        a = dict(base, **kw)
        llmk.attention_decode_fast(d.q, d.kp, d.vp, d.tables, d.lens, out, ws, a["n_seq"],
                                   a["max_pages"], a["page_size"], a["n_heads"], a["n_kv_heads"],
                                   a["head_dim"], a["num_splits"], check_indices=False)

    for kw, status in [(dict(page_size=32), llmk.LLMK_ERR_SHAPE),
                       (dict(n_heads=16), llmk.LLMK_ERR_SHAPE),
                       (dict(n_kv_heads=3, n_heads=16), llmk.LLMK_ERR_SHAPE),
                       (dict(num_splits=0), llmk.LLMK_ERR_INVALID_VALUE)]:
        with pytest.raises(llmk.LlmkError) as e:
            call(**kw)
        assert e.value.status == status, kw
    call(n_seq=0)  # nothing to do


def test_binding_rejects_lengths_beyond_the_table(llmk, reference_case):
    d = OnDevice(reference_case)
    bad = reference_case["lens"].copy()
    bad[0] = reference_case["max_pages"] * 16 + 1
    out = torch.empty(d.n_out, dtype=torch.float16, device=DEV)
    with pytest.raises(llmk.LlmkError):
        llmk.attention_decode_fast(d.q, d.kp, d.vp, d.tables, dev_i32(bad), out, None,
                                   reference_case["n_seq"], reference_case["max_pages"], 16, 32,
                                   8, 64, 1, check_indices=True)
    llmk.set_check_indices(True)  # the same through the module-wide default
    try:
        with pytest.raises(llmk.LlmkError):
            llmk.attention_decode_fast(d.q, d.kp, d.vp, d.tables, dev_i32(bad), out, None,
                                       reference_case["n_seq"], reference_case["max_pages"], 16,
                                       32, 8, 64, 1)
    finally:
        llmk.set_check_indices(False)


def test_on_a_side_stream(llmk, orc, reference_case):
    d = OnDevice(reference_case)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        got = d.run(llmk, 4, stream=s)
    assert_tol(orc.compare(got, oracle_out(orc, reference_case)), EXACT_FLOOR, "side stream")


def test_decode_batch_of_256_sequences_up_to_2048(llmk, orc):
    """The decode workload: 256 sequences, lengths uniform in [1, 2048], shuffled pages, the
    split count the MI355X default picks, and the reference's default pick as well."""
    rng = np.random.default_rng(0x5EED0006)
    lens = rng.integers(1, 2049, 256)
    c = attention_case(rng, lens, max_pages=128)
    d = OnDevice(c)
    ref = oracle_out(orc, c)
    for splits in (llmk.choose_num_splits(256, 8, int(lens.max())),
                   llmk.choose_num_splits(256, 8, int(lens.max()), 64)):
        assert_tol(orc.compare(d.run(llmk, splits), ref), EXACT_FLOOR, f"batch 256 splits {splits}")


@pytest.mark.parametrize("nkv", [1, 2, 4, 8, 16])
def test_page_balanced_runs_weigh_sequence_starts(llmk, orc, nkv):
    """The page-balanced grid cuts units of work, not pages: a sequence's start weighs 32 / KVW
    pages. With 1 or 2 kv heads per row (a start worth 32 or 16 pages) and many one- to
    three-page sequences, whole runs fall on start units and hold no page, runs end inside a
    start, and a sequence's page 0 opens a run; 16 kv heads take two kv groups of blocks. Empty
    sequences sit in between."""
    rng = np.random.default_rng(0xB1A5 + nkv)
    lens = rng.integers(1, 49, 400)
    lens[rng.choice(400, 40, replace=False)] = 0
    lens[::97] = 2048 // nkv  # a few long ones, split over several runs
    c = attention_case(rng, lens, n_heads=4 * nkv, n_kv_heads=nkv)
    d = OnDevice(c)
    ref = oracle_out(orc, c).reshape(400, -1)
    empty = c["lens"] <= 0
    for splits in (3, 8, 32):
        got = d.run(llmk, splits).reshape(400, -1)
        assert np.all(np.isnan(got[empty].view(np.float16))), f"n_kv {nkv} splits {splits}"
        assert_tol(orc.compare(got[~empty].reshape(-1), ref[~empty].reshape(-1)), EXACT_FLOOR,
                   f"n_kv {nkv} splits {splits}")


def test_many_short_sequences_share_a_block(llmk, orc):
    """Page-balanced runs that cover many whole sequences and pieces of others: 300 sequences
    of 1 to 40 positions, plus runs of a single page (every length <= 16, max_pages 1)."""
    rng = np.random.default_rng(7)
    c = attention_case(rng, rng.integers(1, 41, 300))
    d = OnDevice(c)
    ref = oracle_out(orc, c)
    for splits in (3, 8, 32):
        assert_tol(orc.compare(d.run(llmk, splits), ref), EXACT_FLOOR, f"short seqs splits {splits}")
    c1 = attention_case(rng, rng.integers(0, 17, 64))
    assert c1["max_pages"] == 1
    d1 = OnDevice(c1)
    ref1 = oracle_out(orc, c1).reshape(64, -1)
    empty = c1["lens"] <= 0
    for splits in (1, 8):
        got = d1.run(llmk, splits).reshape(64, -1)
        assert np.all(np.isnan(got[empty].view(np.float16)))
        assert_tol(orc.compare(got[~empty].reshape(-1), ref1[~empty].reshape(-1)), EXACT_FLOOR,
                   f"one-page sequences splits {splits}")
