"""CPU-side tests of the C-ABI boundary: the library loads, exports every entry point that
include/llmk.h declares, rejects bad arguments before launching anything, and its host-side
function (the Llama-3 rotation-speed table) equals the oracle bit for bit. Nothing here touches
a GPU: every call below returns from argument validation before any HIP call."""
import ctypes
import os
import subprocess

import numpy as np
import pytest
import torch

from _helpers import ROPE

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_every_declared_symbol(llmk):
    declared = llmk.exported_symbols_declared_in_header()
    assert len(declared) >= 14
    out = subprocess.run(["nm", "-D", "--defined-only", llmk.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = [s for s in declared if s not in exported]
    assert not missing, f"declared in include/llmk.h but not exported: {missing}"
    for s in declared:
        getattr(llmk.lib(), s)  # resolvable through ctypes as well
    assert [s for s in exported if s.startswith("llmk_")] and \
        all(s in declared for s in exported if s.startswith("llmk_"))


def test_library_has_gfx950_code_only(llmk, tmp_path):
    """The fat binary embedded in libllmk holds one device code object, for gfx950."""
    fatbin = tmp_path / "fatbin.bin"
    subprocess.run(["objcopy", f"--dump-section=.hip_fatbin={fatbin}", llmk.LIB_PATH,
                    str(tmp_path / "copy.so")], check=True)
    out = subprocess.run(["/opt/rocm/llvm/bin/clang-offload-bundler", "--list", "--type=o",
                          f"--input={fatbin}"], capture_output=True, text=True, check=True).stdout
    targets = [t for t in out.split() if t.startswith("hip")]
    assert targets == ["hipv4-amdgcn-amd-amdhsa--gfx950"], out


def test_version_and_error_strings(llmk):
    assert llmk.version() == 100
    assert llmk.error_string(0) == "success"
    for code in (llmk.LLMK_ERR_INVALID_VALUE, llmk.LLMK_ERR_SHAPE, llmk.LLMK_ERR_ALIGNMENT,
                 llmk.LLMK_ERR_UNSUPPORTED):
        assert llmk.error_string(code).startswith("llmk: ")
    assert llmk.error_string(1)  # a hipError_t value is named by HIP


def test_inv_freq_host_function_equals_oracle(llmk, orc):
    for hd in (64, 128, 32, 2):
        mine = np.array(llmk.compute_rope_inv_freq(hd, ROPE["theta"], ROPE["factor"],
                                                   ROPE["low"], ROPE["high"], ROPE["orig"]),
                        np.float32)
        ref = orc.compute_rope_inv_freq(hd, ROPE["theta"], ROPE["factor"], ROPE["low"],
                                        ROPE["high"], ROPE["orig"])
        assert np.array_equal(mine.view(np.uint32), ref.view(np.uint32)), hd
    # another parameter set (llama3.1-8B style: factor 8)
    mine = np.array(llmk.compute_rope_inv_freq(128, 500000.0, 8.0, 1.0, 4.0, 8192.0), np.float32)
    ref = orc.compute_rope_inv_freq(128, 500000.0, 8.0, 1.0, 4.0, 8192.0)
    assert np.array_equal(mine.view(np.uint32), ref.view(np.uint32))


FAKE = 0x10000  # 16-byte aligned, never dereferenced: every call below fails validation first
MIS = FAKE + 2  # 2-byte aligned


def test_argument_validation_without_launch(llmk):
    L = llmk.lib()
    E = llmk
    # zero-sized calls are no-ops
    assert L.llmk_rmsnorm(None, None, None, 0, 2048, 1e-5, None) == 0
    assert L.llmk_residual_add(None, None, None, 0, None) == 0
    assert L.llmk_swiglu(None, None, None, 0, None) == 0
    assert L.llmk_embedding_lookup(None, None, None, 0, 2048, None) == 0
    assert L.llmk_kv_scatter(None, None, None, 0, 0, 16, 512, None) == 0
    assert L.llmk_kv_scatter_batch(None, None, None, None, 0, 8, 16, 512, None) == 0
    assert L.llmk_rope_apply(None, None, None, None, 0, 32, 8, 64, None) == 0
    assert L.llmk_copy_bytes(None, None, 0, None) == 0
    # NULL pointers and negative sizes
    assert L.llmk_rmsnorm(None, FAKE, FAKE, 1, 2048, 1e-5, None) == E.LLMK_ERR_INVALID_VALUE
    assert L.llmk_rmsnorm(FAKE, FAKE, FAKE, -1, 2048, 1e-5, None) == E.LLMK_ERR_INVALID_VALUE
    assert L.llmk_add_rmsnorm(None, FAKE, FAKE, FAKE, 4, 2048, 1e-5, None) == E.LLMK_ERR_INVALID_VALUE
    assert L.llmk_residual_add(FAKE, None, FAKE, 10, None) == E.LLMK_ERR_INVALID_VALUE
    assert L.llmk_kv_scatter(FAKE, FAKE, FAKE, -1, 4, 16, 512, None) == E.LLMK_ERR_INVALID_VALUE
    assert L.llmk_kv_scatter_batch(FAKE, FAKE, FAKE, None, 4, 8, 16, 512, None) == E.LLMK_ERR_INVALID_VALUE
    assert L.llmk_rope_apply(FAKE, FAKE, None, FAKE, 4, 32, 8, 64, None) == E.LLMK_ERR_INVALID_VALUE
    assert L.llmk_decode_nongemm_pass(None, None) == E.LLMK_ERR_INVALID_VALUE
    # layout preconditions (ref: kernels/rmsnorm.cuh:5, embedding.cuh:5, kv_scatter.cuh:5)
    assert L.llmk_rmsnorm(FAKE, FAKE, FAKE, 4, 2044, 1e-5, None) == E.LLMK_ERR_SHAPE
    assert L.llmk_embedding_lookup(FAKE, FAKE, FAKE, 4, 100, None) == E.LLMK_ERR_SHAPE
    assert L.llmk_kv_scatter(FAKE, FAKE, FAKE, 0, 4, 16, 500, None) == E.LLMK_ERR_SHAPE
    assert L.llmk_rope_apply(FAKE, FAKE, FAKE, FAKE, 4, 32, 8, 63, None) == E.LLMK_ERR_SHAPE
    assert L.llmk_rope_kv_scatter_batch(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 4, 8, 16,
                                        32, 8, 40, None) == E.LLMK_ERR_SHAPE
    assert L.llmk_copy_bytes(FAKE, FAKE, 24, None) == E.LLMK_ERR_SHAPE
    # 16-byte alignment of the vector paths
    assert L.llmk_rmsnorm(MIS, FAKE, FAKE, 4, 2048, 1e-5, None) == E.LLMK_ERR_ALIGNMENT
    assert L.llmk_add_rmsnorm(MIS, FAKE, FAKE, FAKE, 4, 2048, 1e-5, None) == E.LLMK_ERR_ALIGNMENT
    assert L.llmk_embedding_lookup(FAKE, FAKE, MIS, 4, 2048, None) == E.LLMK_ERR_ALIGNMENT
    assert L.llmk_kv_scatter_batch(FAKE, MIS, FAKE, FAKE, 4, 8, 16, 512, None) == E.LLMK_ERR_ALIGNMENT
    assert L.llmk_rope_kv_scatter_batch(FAKE, FAKE, MIS, FAKE, FAKE, FAKE, FAKE, FAKE, 4, 8, 16,
                                        32, 8, 64, None) == E.LLMK_ERR_ALIGNMENT
    assert L.llmk_copy_bytes(MIS, FAKE, 32, None) == E.LLMK_ERR_ALIGNMENT
    assert L.llmk_compute_rope_inv_freq(63, 1e4, 1, 1, 4, 8192, None) == E.LLMK_ERR_INVALID_VALUE
    # split-KV attention: the reference's preconditions (kernels/attention_decode_fast.cu:160-163)
    A = L.llmk_attention_decode_fast
    assert A(None, None, None, None, None, None, None, 0, 8, 16, 32, 8, 64, 4, None) == 0
    assert A(*[FAKE] * 7, 4, 8, 32, 32, 8, 64, 4, None) == E.LLMK_ERR_SHAPE
    assert A(*[FAKE] * 7, 4, 8, 16, 32, 8, 128, 4, None) == E.LLMK_ERR_SHAPE
    assert A(*[FAKE] * 7, 4, 8, 16, 24, 8, 64, 4, None) == E.LLMK_ERR_SHAPE
    assert A(*[FAKE] * 7, 65536, 8, 16, 32, 8, 64, 4, None) == E.LLMK_ERR_UNSUPPORTED
    assert A(*[FAKE] * 7, 4, 8, 16, 32, 8, 64, 0, None) == E.LLMK_ERR_INVALID_VALUE
    assert A(*[FAKE] * 6, None, 4, 8, 16, 32, 8, 64, 2, None) == E.LLMK_ERR_INVALID_VALUE
    assert A(MIS, *[FAKE] * 6, 4, 8, 16, 32, 8, 64, 2, None) == E.LLMK_ERR_ALIGNMENT
    assert L.llmk_attention_decode_fast_workspace_floats(256, 32, 32) == 256 * 32 * 32 * 66
    # the allocation-free variant: same checks, and a batch past its scratch is refused
    N = L.llmk_attention_decode_fast_noalloc
    assert N(None, None, None, None, None, None, 0, 8, 16, 32, 8, 64, 4, None) == 0
    assert N(*[FAKE] * 6, 4, 8, 32, 32, 8, 64, 4, None) == E.LLMK_ERR_SHAPE
    assert N(*[FAKE] * 5, None, 4, 8, 16, 32, 8, 64, 4, None) == E.LLMK_ERR_INVALID_VALUE
    assert N(MIS, *[FAKE] * 5, 4, 8, 16, 32, 8, 64, 2, None) == E.LLMK_ERR_ALIGNMENT
    assert N(*[FAKE] * 6, 257, 8, 16, 32, 8, 64, 32, None) == E.LLMK_ERR_SCRATCH
    assert N(*[FAKE] * 6, 3, 8, 16, 4096, 1024, 64, 32, None) == E.LLMK_ERR_SCRATCH
    assert E.ATTN_NOALLOC_MAX_FLOATS == L.llmk_attention_decode_fast_workspace_floats(256, 32, 32)
    assert L.llmk_attention_decode_fast_workspace_floats(0, 32, 32) == 0
    assert L.llmk_argmax_rows(None, None, 0, 128256, None) == 0
    # measurement kernels
    P = L.llmk_bw_probe
    assert P(E.PROBE_COPY, None, None, None, 0, 0, 4, None) == 0
    assert P(5, FAKE, FAKE, FAKE, 32, 0, 4, None) == E.LLMK_ERR_INVALID_VALUE
    assert P(E.PROBE_READ2, FAKE, None, FAKE, 32, 0, 4, None) == E.LLMK_ERR_INVALID_VALUE
    assert P(E.PROBE_COPY, FAKE, None, FAKE, 32, -1, 4, None) == E.LLMK_ERR_INVALID_VALUE
    assert P(E.PROBE_COPY, FAKE, None, FAKE, 24, 0, 4, None) == E.LLMK_ERR_SHAPE
    assert P(E.PROBE_INPLACE, None, None, MIS, 32, 0, 4, None) == E.LLMK_ERR_ALIGNMENT
    assert P(E.PROBE_COPY, FAKE, None, FAKE, 32, 0, 3, None) == E.LLMK_ERR_INVALID_VALUE
    assert L.llmk_empty_launch(0, 64, None) == E.LLMK_ERR_INVALID_VALUE
    assert L.llmk_empty_launch(4, 2048, None) == E.LLMK_ERR_INVALID_VALUE
    assert L.llmk_argmax_rows(FAKE, FAKE, 4, 0, None) == E.LLMK_ERR_INVALID_VALUE
    assert L.llmk_argmax_rows(None, FAKE, 4, 100, None) == E.LLMK_ERR_INVALID_VALUE


def test_decode_pass_descriptor_validation_without_launch(llmk):
    """The decode-pass descriptor: the second add + RMSNorm is all or nothing, in both passes,
    refused before any launch (no pointer here is dereferenced)."""
    import ctypes
    L, E = llmk._lib, llmk
    arr = (ctypes.c_void_p * 1)(FAKE)
    parr = ctypes.cast(arr, ctypes.POINTER(ctypes.c_void_p))

    def desc(**second):
        d = E.DecodePass()
        d.n_seqs, d.n_layers, d.hidden, d.n_heads, d.n_kv_heads = 4, 1, 2048, 32, 8
        d.head_dim, d.inter, d.page_size, d.max_pages, d.eps = 64, 8192, 16, 8, 1e-5
        for f in ("embed_table", "token_ids", "residual", "block_tables", "positions",
                  "inv_freq"):
            setattr(d, f, FAKE)
        for f in ("x", "norm_w", "normed", "q", "k", "v", "k_pool", "v_pool", "gate", "up",
                  "act"):
            setattr(d, f, parr)
        for f, v in second.items():
            setattr(d, f, v)
        return ctypes.byref(d)

    for fn in (L.llmk_decode_nongemm_pass, L.llmk_decode_nongemm_pass_layers,
               L.llmk_decode_nongemm_pass_fused):
        assert fn(desc(x2=parr), None) == E.LLMK_ERR_INVALID_VALUE
        assert fn(desc(x2=parr, norm_w2=parr), None) == E.LLMK_ERR_INVALID_VALUE
        assert fn(desc(normed2=parr), None) == E.LLMK_ERR_INVALID_VALUE
        assert fn(None, None) == E.LLMK_ERR_INVALID_VALUE
    assert ctypes.sizeof(E.DecodePass) == 10 * 4 + 6 * 8 + 14 * 8


def test_split_count_rule_and_its_default(llmk):
    """choose_num_splits restates the reference's rule (kernels/attention_decode_fast.cuh:22-29);
    the Python default equals LLMK_ATTN_TARGET_BLOCKS of the C header."""
    import re
    with open(llmk.HEADER_PATH) as f:
        m = re.search(r"#define LLMK_ATTN_TARGET_BLOCKS (\d+)", f.read())
    assert m and int(m.group(1)) == llmk.ATTN_TARGET_BLOCKS
    assert llmk.choose_num_splits(16, 8, 2048, 64) == 1  # reference defaults: 64 // 128 -> 0 -> 1
    assert llmk.choose_num_splits(2, 8, 2048, 64) == 4
    assert llmk.choose_num_splits(1, 8, 30, 64) == 2    # capped by the page count
    assert llmk.choose_num_splits(1, 1, 4096, 64) == 32  # capped at 32
    assert llmk.choose_num_splits(256, 8, 2048) == 32
    assert llmk.choose_num_splits(1024, 8, 2048) == 8


def test_python_wrapper_rejects_host_tensors_and_short_buffers(llmk):
    x = torch.zeros(4, 2048, dtype=torch.float16)
    with pytest.raises(llmk.LlmkError, match="CUDA tensor"):
        llmk.rmsnorm(x, x[0], x, 4, 2048, 1e-5)
    if not torch.cuda.is_available():
        return
    d = torch.zeros(4, 2048, dtype=torch.float16, device="cuda")
    with pytest.raises(llmk.LlmkError, match="touches"):
        llmk.rmsnorm(d, d[0], d, 5, 2048, 1e-5)


def test_dropin_binary_is_built_and_resolves_its_libraries():
    exe = os.path.join(ROOT, "tests", "cpp", "llmk_dropin_test")
    assert os.path.exists(exe), "run __graft_entry__.build() first"
    out = subprocess.run(["ldd", exe], capture_output=True, text=True, check=True).stdout
    assert "not found" not in out, out
    assert "libllmk.so" in out and "liboracle.so" in out


def test_no_oracle_in_the_product():
    """The product (package + library sources) never refers to the oracle."""
    pkg = os.path.join(ROOT, "cuda-llm-engine_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".cpp", ".hpp", ".h")):
                text = open(os.path.join(dirpath, f), encoding="utf-8").read()
                assert "oracle" not in text.lower(), f
    with open(os.path.join(ROOT, "include", "llmk.h")) as fh:
        assert "oracle" not in fh.read().lower()
    out = subprocess.run(["ldd", os.path.join(pkg, "libllmk.so")], capture_output=True,
                         text=True, check=True).stdout
    assert "oracle" not in out


def test_attention_workspace_size_saturates_instead_of_wrapping(llmk):
    """llmk_attention_decode_fast_workspace_floats returns SIZE_MAX when the product does not fit
    a size_t (it would wrap to 0 for 32768 sequences x 2^18 heads x 2^29 splits x 66); the
    allocation-free entry point then refuses the call (LLMK_ERR_SCRATCH) and the workspace one
    as well (LLMK_ERR_INVALID_VALUE), before anything is launched."""
    lib = llmk.lib()
    size_max = (1 << 64) - 1
    assert lib.llmk_attention_decode_fast_workspace_floats(1 << 15, 1 << 18, 1 << 29) == size_max
    assert lib.llmk_attention_decode_fast_workspace_floats(256, 32, 32) == 256 * 32 * 32 * 66
    fake = 0x10000  # 16-byte aligned; never dereferenced: both calls return before any launch
    args = [fake] * 6
    n_seq, n_kv, splits = 1 << 15, 1 << 16, 1 << 29
    assert lib.llmk_attention_decode_fast_noalloc(*args, n_seq, 128, 16, 4 * n_kv, n_kv, 64,
                                                  splits, None) == llmk.LLMK_ERR_SCRATCH
    assert lib.llmk_attention_decode_fast(*args, fake, n_seq, 128, 16, 4 * n_kv, n_kv, 64,
                                          splits, None) == llmk.LLMK_ERR_INVALID_VALUE


def test_index_checks_are_opt_in(llmk):
    """The binding validates index values only when asked (per call, or module-wide), as the
    reference's launchers check nothing; off by default unless LLMK_CHECK_INDICES is set."""
    import os
    env_on = os.environ.get("LLMK_CHECK_INDICES", "") not in ("", "0")
    assert llmk._want_checks(None) == env_on
    assert llmk._want_checks(True) and not llmk._want_checks(False)
    llmk.set_check_indices(True)
    try:
        assert llmk._want_checks(None)
    finally:
        llmk.set_check_indices(env_on)
