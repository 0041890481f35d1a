"""The allocation-free attention entry point (llmk_attention_decode_fast_noalloc) against the
entry point it stands for (llmk_attention_decode_fast with a caller workspace): both run the
same kernels, so the outputs must be bit-identical. Two calls in a row through the C-ABI, the
second with a smaller batch (the library's scratch keeps the first call's contents), for each
of the three partial layouts the scratch holds: the page-balanced grid (k_attn_balanced, merged
by k_attn_merge from the segment count), the sequence-split grid of one or two splits
(k_attn_split, merged by k_attn_merge per split), and the short-run grid of the smallest batches
(k_attn_split in 2-wave blocks, merged by k_attn_merge_many). Every output slot is checked, and
the bytes past the output stay untouched. A last test captures the entry point in a HIP graph."""
import ctypes

import numpy as np
import pytest
import torch

from _helpers import ATTN_LENS, attention_case

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
NH, NKV, HD, PS = 32, 8, 64, 16


def dev_u16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(DEV)


def dev_i32(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(DEV)


class Case:
    def __init__(self, c):
        self.c = c
        self.q, self.kp, self.vp = dev_u16(c["q"]), dev_u16(c["k_pool"]), dev_u16(c["v_pool"])
        self.tables, self.lens = dev_i32(c["tables"]), dev_i32(c["lens"])

    def run(self, lib, splits, noalloc, n_seq=None):
        c = self.c
        n = c["n_seq"] if n_seq is None else n_seq
        n_out = n * NH * HD
        out = torch.full((n_out + 64,), 0x7F7F, dtype=torch.int16, device=DEV)
        args = [self.q.data_ptr(), self.kp.data_ptr(), self.vp.data_ptr(),
                self.tables.data_ptr(), self.lens.data_ptr(), out.data_ptr()]
        tail = [n, c["max_pages"], PS, NH, NKV, HD, splits, torch.cuda.current_stream().cuda_stream]
        if noalloc:
            st = lib.llmk_attention_decode_fast_noalloc(*args, *tail)
        else:
            floats = lib.llmk_attention_decode_fast_workspace_floats(n, NH, splits)
            ws = torch.full((max(floats, 4),), float("nan"), dtype=torch.float32, device=DEV)
            st = lib.llmk_attention_decode_fast(*args, ws.data_ptr(), *tail)
        assert st == 0, st
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        assert np.all(got[n_out:] == 0x7F7F), "write past the output"
        return got[:n_out]


def check_pair(lib, case, first, second):
    """`first` and `second` are (splits, n_seq): two calls in a row of each entry point."""
    for splits, n_seq in (first, second):
        ref = case.run(lib, splits, noalloc=False, n_seq=n_seq)
        got = case.run(lib, splits, noalloc=True, n_seq=n_seq)
        assert np.array_equal(got, ref), (splits, n_seq, int((got != ref).sum()))
        assert not np.isnan(got.view(np.float16)[: n_seq * NH * HD]).all()


def test_noalloc_page_balanced_grid_reference_lengths(llmk):
    """The reference test's lengths (128-page tables) with 8 splits, then the first 3 sequences
    with 3 splits: both calls take the page-balanced grid (splits of 16 and 43 pages are too
    long for the short-run grid) and its merge."""
    case = Case(attention_case(np.random.default_rng(7001), ATTN_LENS))
    check_pair(llmk.lib(), case, (8, 8), (3, 3))


def test_noalloc_sequence_split_grid_then_a_smaller_batch(llmk):
    """Two splits: the sequence-split grid (k_attn_split, 64-page splits) writing each split's
    partial into the scratch and k_attn_merge combining them per split; the reference test's
    8 sequences, then the first 5."""
    case = Case(attention_case(np.random.default_rng(7006), ATTN_LENS))
    check_pair(llmk.lib(), case, (2, 8), (2, 5))


def test_noalloc_short_run_grid_then_one_sequence(llmk):
    """32 splits of 128-page tables (4-page runs) over two sequences, then one: the short-run
    grid in 2-wave blocks of kv groups of 2 heads, and k_attn_merge_many over up to 32 pieces
    per sequence."""
    lens = np.array([2048, 1500], np.int32)
    case = Case(attention_case(np.random.default_rng(7007), lens, max_pages=128))
    check_pair(llmk.lib(), case, (32, 2), (32, 1))


def test_noalloc_page_balanced_grid_then_a_smaller_batch(llmk):
    """64 sequences of lengths uniform in [1, 2048] with 32 splits, then the first 17 with 20
    splits: the page-balanced grid and its merge both times."""
    lens = np.random.default_rng(7002).integers(1, 2049, 64)
    case = Case(attention_case(np.random.default_rng(7003), lens, max_pages=128))
    check_pair(llmk.lib(), case, (32, 64), (20, 17))


def test_noalloc_at_its_size_limit(llmk):
    """256 sequences x 32 heads x 32 splits is exactly the scratch; one sequence more is refused
    before anything is launched."""
    lib = llmk.lib()
    lens = np.random.default_rng(7004).integers(1, 257, 256)
    case = Case(attention_case(np.random.default_rng(7005), lens, max_pages=16))
    assert lib.llmk_attention_decode_fast_workspace_floats(256, NH, 32) == \
        llmk.ATTN_NOALLOC_MAX_FLOATS
    check_pair(lib, case, (32, 256), (5, 100))
    p = case.q.data_ptr()
    assert lib.llmk_attention_decode_fast_noalloc(p, p, p, p, p, p, 257, 16, PS, NH, NKV, HD, 32,
                                                  None) == llmk.LLMK_ERR_SCRATCH


def test_noalloc_in_a_graph_replayed_with_new_inputs(llmk):
    """The entry point captured in a HIP graph on a side stream (after one eager call on the
    device, which resolves the scratch's address: that first call must not be made under
    capture) and replayed with new query and length contents copied into the captured
    buffers in between, with eager work between replays; every replay gives the bits of an
    eager allocation-free call on the same inputs. 16 sequences, 32 splits (page-balanced
    grid)."""
    lib = llmk.lib()
    rng = np.random.default_rng(7008)
    lens0 = rng.integers(1, 2049, 16).astype(np.int32)
    case = Case(attention_case(np.random.default_rng(7009), lens0, max_pages=128))
    c = case.c
    n, splits = c["n_seq"], 32
    out = torch.full((n * NH * HD,), 0x7F7F, dtype=torch.int16, device=DEV)

    def call(stream):
        st = lib.llmk_attention_decode_fast_noalloc(
            case.q.data_ptr(), case.kp.data_ptr(), case.vp.data_ptr(), case.tables.data_ptr(),
            case.lens.data_ptr(), out.data_ptr(), n, c["max_pages"], PS, NH, NKV, HD, splits,
            stream)
        assert st == 0, st

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        call(s.cuda_stream)  # eager: resolves the scratch address outside capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call(torch.cuda.current_stream().cuda_stream)
    for i in range(3):
        # new contents in the captured buffers: another query, other lengths (within the
        # tables' pages, so the pool slots read stay the ones the case wrote)
        q_new = torch.from_numpy(
            (rng.uniform(-1, 1, n * NH * HD)).astype(np.float16).view(np.int16)).to(DEV)
        lens_new = np.minimum(lens0, rng.integers(1, 2049, n)).astype(np.int32)
        case.q.view(-1).copy_(q_new)
        case.lens.view(-1).copy_(torch.from_numpy(lens_new).to(DEV))
        torch.cuda.synchronize()
        out.fill_(0x7F7F)
        g.replay()
        torch.cuda.synchronize()
        got = out.cpu().numpy().copy()
        _ = torch.randn(1 << 20, device=DEV).sum().item()  # eager work between replays
        out.fill_(0x7F7F)
        call(torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        ref = out.cpu().numpy()
        assert np.array_equal(got, ref), (i, int((got != ref).sum()))
        assert not np.isnan(got.view(np.float16)).any()
