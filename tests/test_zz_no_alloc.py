"""The allocation-free attention entry point (llmk_attention_decode_fast_noalloc) against the
entry point it stands for (llmk_attention_decode_fast with a caller workspace): both run the
same kernels, so the outputs must be bit-identical. Two calls in a row through the C-ABI, the
second with a smaller batch (the library's scratch keeps the first call's contents), for the
sequence-split grid and the page-balanced grid; every output slot is checked, and the bytes
past the output stay untouched."""
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


def test_noalloc_sequence_split_grid_then_a_smaller_batch(llmk):
    """The reference test's lengths with 8 splits (sequence-split grid and merge), then the
    first 3 sequences with 3 splits."""
    case = Case(attention_case(np.random.default_rng(7001), ATTN_LENS))
    check_pair(llmk.lib(), case, (8, 8), (3, 3))


def test_noalloc_page_balanced_grid_then_a_smaller_batch(llmk):
    """64 sequences of lengths uniform in [1, 2048] with 32 splits (the page-balanced grid and
    its merge), then the first 17 with 20 splits."""
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
