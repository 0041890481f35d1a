"""llmk -- Python face of libllmk, the MI355X (gfx950) non-GEMM layer kernels.

The functions below carry the names and argument lists of the reference engine's C++ launchers
(JayeshNikam36/cuda-llm-engine, kernels/*.cuh) and call libllmk's C-ABI (include/llmk.h)
through ctypes. Tensors are torch CUDA tensors (torch provides device memory and streams only;
all compute is libllmk's HIP kernels). ``stream=None`` means torch's current stream.

Errors: a violated precondition raises ``LlmkError`` before anything is launched. Besides the
C-ABI's own checks, every function verifies here that each tensor holds at least the elements
the kernel will touch. Checking the values inside the index tensors -- that token ids, page
numbers and positions address only rows that exist -- reads them back, a device
synchronisation per call, so it is off by default, as in the reference, whose launchers check
nothing (kernels/embedding.cuh:5). Turn it on per call (``check_indices=True``), for every call
(``set_check_indices(True)``, or ``LLMK_CHECK_INDICES=1`` in the environment), or build a
``DecodeNonGemmPass``, which validates its indices once, when it is built.

There is no CPU fallback: if libllmk.so is missing, importing this package raises.
"""
from __future__ import annotations

import ctypes
import os
import re

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_CHECK_INDICES = os.environ.get("LLMK_CHECK_INDICES", "") not in ("", "0")


def set_check_indices(on: bool) -> None:
    """Default of every function's ``check_indices`` argument (initially off, or on with
    ``LLMK_CHECK_INDICES=1``): validate the index tensors' values on the host before launching."""
    global _CHECK_INDICES
    _CHECK_INDICES = bool(on)


def _want_checks(flag) -> bool:
    return _CHECK_INDICES if flag is None else bool(flag)
LIB_PATH = os.path.join(_HERE, "libllmk.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "llmk.h")

LLMK_OK = 0
LLMK_ERR_INVALID_VALUE = 10001
LLMK_ERR_SHAPE = 10002
LLMK_ERR_ALIGNMENT = 10003
LLMK_ERR_UNSUPPORTED = 10004
LLMK_ERR_BLAS = 10005
LLMK_ERR_IO = 10006
LLMK_ERR_CAPACITY = 10007
LLMK_ERR_SCRATCH = 10008


class LlmkError(RuntimeError):
    def __init__(self, fn: str, status: int, msg: str):
        super().__init__(f"{fn}: {msg} (status {status})")
        self.status = status


if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"libllmk.so not found at {LIB_PATH}: build it first (python -c "
        "'import __graft_entry__; __graft_entry__.build()')")

_vp = ctypes.c_void_p
_i = ctypes.c_int
_sz = ctypes.c_size_t
_f = ctypes.c_float
_d = ctypes.c_double


class DecodePass(ctypes.Structure):
    """Mirror of ``struct llmk_decode_pass`` (include/llmk.h)."""
    _fields_ = [
        ("n_seqs", _i), ("n_layers", _i), ("hidden", _i), ("n_heads", _i),
        ("n_kv_heads", _i), ("head_dim", _i), ("inter", _i), ("page_size", _i),
        ("max_pages", _i), ("eps", _f),
        ("embed_table", _vp), ("token_ids", _vp), ("residual", _vp),
        ("block_tables", _vp), ("positions", _vp), ("inv_freq", _vp),
        ("x", ctypes.POINTER(_vp)), ("norm_w", ctypes.POINTER(_vp)),
        ("normed", ctypes.POINTER(_vp)), ("q", ctypes.POINTER(_vp)),
        ("k", ctypes.POINTER(_vp)), ("v", ctypes.POINTER(_vp)),
        ("k_pool", ctypes.POINTER(_vp)), ("v_pool", ctypes.POINTER(_vp)),
        ("gate", ctypes.POINTER(_vp)), ("up", ctypes.POINTER(_vp)),
        ("act", ctypes.POINTER(_vp)),
        ("x2", ctypes.POINTER(_vp)), ("norm_w2", ctypes.POINTER(_vp)),
        ("normed2", ctypes.POINTER(_vp)),
    ]


class ModelConfig(ctypes.Structure):
    """Mirror of ``struct llmk_model_config`` (include/llmk.h). Defaults: Llama-3.2-1B
    (ref: engine/layer.h:6-9, engine/model.h:7, engine/model.cu:20)."""
    _fields_ = [
        ("n_layers", _i), ("hidden", _i), ("n_heads", _i), ("n_kv_heads", _i),
        ("head_dim", _i), ("inter", _i), ("vocab", _i), ("eps", _f),
        ("rope_theta", _d), ("rope_factor", _d), ("rope_low_freq_factor", _d),
        ("rope_high_freq_factor", _d), ("rope_original_max_pos", _d),
    ]

    def __init__(self, **kw):
        base = dict(n_layers=16, hidden=2048, n_heads=32, n_kv_heads=8, head_dim=64,
                    inter=8192, vocab=128256, eps=1e-5, rope_theta=500000.0, rope_factor=32.0,
                    rope_low_freq_factor=1.0, rope_high_freq_factor=4.0,
                    rope_original_max_pos=8192.0)
        unknown = set(kw) - set(base)
        if unknown:
            raise TypeError(f"unknown ModelConfig fields {sorted(unknown)}")
        base.update(kw)
        super().__init__(**base)

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


class LayerWeights(ctypes.Structure):
    """Mirror of ``struct llmk_layer_weights`` (ref: engine/layer.h:11-13)."""
    NAMES = ("attn_norm", "wq", "wk", "wv", "wo", "mlp_norm", "w_gate", "w_up", "w_down")
    _fields_ = [(n, _vp) for n in NAMES]


_i32p = ctypes.POINTER(ctypes.c_int32)


class Request(ctypes.Structure):
    """Mirror of ``struct llmk_request`` (ref: engine/scheduler.h:6-14)."""
    _fields_ = [("id", _i), ("prompt", _i32p), ("prompt_len", _i), ("max_new", _i),
                ("arrival_step", _i), ("output", _i32p), ("n_output", _i),
                ("t_arrive_ms", _d), ("t_first_ms", _d), ("t_done_ms", _d)]


class SchedStats(ctypes.Structure):
    """Mirror of ``struct llmk_sched_stats`` (ref: engine/scheduler.h:16-22)."""
    _fields_ = [("decode_steps", _i), ("total_words", _i), ("prefills", _i), ("max_batch", _i),
                ("iterations", _i), ("total_ms", _d), ("mean_batch", _d), ("prefill_ms", _d),
                ("decode_ms", _d), ("prep_ms", _d), ("gpu_ms", _d), ("copy_ms", _d),
                ("convert_ms", _d), ("argmax_ms", _d)]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


PREFILL_FN = ctypes.CFUNCTYPE(_i, _vp, _i32p, _i, _i32p, _i, _i32p)
class StepTimes(ctypes.Structure):
    """Mirror of ``struct llmk_step_times`` (ref: engine/batched.h:6-11 StepTimes)."""
    _fields_ = [("prep_ms", _d), ("gpu_ms", _d), ("copy_ms", _d), ("convert_ms", _d),
                ("argmax_ms", _d)]


DECODE_FN = ctypes.CFUNCTYPE(_i, _vp, _i, _i32p, _i32p, _i32p, _i, _i32p,
                             ctypes.POINTER(StepTimes))


class SchedModel(ctypes.Structure):
    """Mirror of ``struct llmk_sched_model``: the scheduler's view of the model."""
    _fields_ = [("user", _vp), ("prefill", PREFILL_FN), ("decode", DECODE_FN)]


_SIGS = {
    "llmk_error_string": (ctypes.c_char_p, [_i]),
    "llmk_version": (_i, []),
    "llmk_embedding_lookup": (_i, [_vp, _vp, _vp, _i, _i, _vp]),
    "llmk_residual_add": (_i, [_vp, _vp, _vp, _sz, _vp]),
    "llmk_rmsnorm": (_i, [_vp, _vp, _vp, _i, _i, _f, _vp]),
    "llmk_add_rmsnorm": (_i, [_vp, _vp, _vp, _vp, _i, _i, _f, _vp]),
    "llmk_compute_rope_inv_freq": (_i, [_i, _d, _d, _d, _d, _d, ctypes.POINTER(_f)]),
    "llmk_rope_apply": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "llmk_swiglu": (_i, [_vp, _vp, _vp, _sz, _vp]),
    "llmk_kv_scatter": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "llmk_kv_scatter_batch": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "llmk_rope_kv_scatter_batch": (_i, [_vp] * 8 + [_i] * 6 + [_vp]),
    "llmk_copy_bytes": (_i, [_vp, _vp, _sz, _vp]),
    "llmk_bw_probe": (_i, [_i, _vp, _vp, _vp, _sz, _i, _i, _vp]),
    "llmk_empty_launch": (_i, [_i, _i, _vp]),
    "llmk_attention_decode_fast_workspace_floats": (_sz, [_i, _i, _i]),
    "llmk_argmax_rows": (_i, [_vp, _vp, _i, _i, _vp]),
    "llmk_attention_decode_fast": (_i, [_vp] * 7 + [_i] * 7 + [_vp]),
    "llmk_attention_decode_fast_noalloc": (_i, [_vp] * 6 + [_i] * 7 + [_vp]),
    "llmk_decode_nongemm_pass": (_i, [ctypes.POINTER(DecodePass), _vp]),
    "llmk_decode_nongemm_pass_layers": (_i, [ctypes.POINTER(DecodePass), _vp]),
    "llmk_decode_nongemm_pass_fused": (_i, [ctypes.POINTER(DecodePass), _vp]),
    "llmk_blas_create": (_i, [ctypes.POINTER(_vp)]),
    "llmk_blas_destroy": (None, [_vp]),
    "llmk_linear": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "llmk_linear_rows": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "llmk_linear_rows_norm": (_i, [_vp, _vp, _f, _vp, _vp, _i, _i, _i, _vp]),
    "llmk_engine_set_option": (_i, [_vp, _i, _i]),
    "llmk_linear_rows_residual": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "llmk_linear_rows_swiglu": (_i, [_vp, _vp, _f, _vp, _vp, _i, _i, _i, _vp]),
    "llmk_linear_rows_qkv_rope_scatter": (_i, [_vp, _vp, _f, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                               _i, _i, _i, _i, _i, _vp]),
    "llmk_qkv_rope_scatter": (_i, [_vp, _i] + [_vp] * 6 + [_i] * 6 + [_vp]),
    "llmk_swiglu_rows": (_i, [_vp, _vp, _i, _i, _vp]),
    "llmk_engine_create": (_i, [ctypes.POINTER(ModelConfig), _i, _i, _i, ctypes.POINTER(_vp)]),
    "llmk_engine_destroy": (None, [_vp]),
    "llmk_engine_set_weights": (_i, [_vp, _vp, _vp, ctypes.POINTER(LayerWeights)]),
    "llmk_engine_load_weights": (_i, [_vp, ctypes.c_char_p]),
    "llmk_engine_set_rows": (_i, [_vp, _i, _vp, _vp, _vp, _i, _vp, _vp]),
    "llmk_engine_forward": (_i, [_vp, _i, _i, _i, _vp]),
    "llmk_engine_buffer": (_vp, [_vp, _i, _i]),
    "llmk_engine_reset_pools": (_i, [_vp, _vp]),
    "llmk_engine_forward_graph": (_i, [_vp, _i, _i, _i, _vp]),
    "llmk_engine_tune": (_i, [_vp, _i, _i, _vp]),
    "llmk_blas_tune": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "llmk_pages_create": (_i, [_i, ctypes.POINTER(_vp)]),
    "llmk_pages_destroy": (None, [_vp]),
    "llmk_pages_total": (_i, [_vp]),
    "llmk_pages_num_free": (_i, [_vp]),
    "llmk_pages_alloc": (_i, [_vp]),
    "llmk_pages_release": (_i, [_vp, _i]),
    "llmk_pages_set_free_list": (_i, [_vp, _i32p, _i]),
    "llmk_scheduler_run": (_i, [ctypes.POINTER(Request), _i, _i, _i, _i, _vp,
                                ctypes.POINTER(SchedModel), ctypes.POINTER(SchedStats)]),
    "llmk_engine_sched_model": (_i, [_vp, _vp, ctypes.POINTER(SchedModel)]),
}

_lib = ctypes.CDLL(LIB_PATH)
for _name, (_res, _args) in _SIGS.items():
    _fn = getattr(_lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args


def lib() -> ctypes.CDLL:
    return _lib


def exported_symbols_declared_in_header() -> list[str]:
    """Names of every function declared in include/llmk.h."""
    with open(HEADER_PATH) as f:
        text = f.read()
    return re.findall(r"LLMK_API\s+[\w\s\*]*?\b(llmk_\w+)\s*\(", text)


def error_string(status: int) -> str:
    return _lib.llmk_error_string(status).decode()


def version() -> int:
    return _lib.llmk_version()


def _check(fn: str, status: int) -> None:
    if status != LLMK_OK:
        raise LlmkError(fn, status, error_string(status))


def _fail(fn: str, msg: str):
    raise LlmkError(fn, LLMK_ERR_INVALID_VALUE, msg)


def _dev(fn: str, t: torch.Tensor, dtype: torch.dtype, min_numel: int, name: str) -> int:
    if not isinstance(t, torch.Tensor):
        _fail(fn, f"{name} must be a torch tensor")
    if not t.is_cuda:
        _fail(fn, f"{name} must be a CUDA tensor, got {t.device}")
    if t.dtype != dtype:
        _fail(fn, f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        _fail(fn, f"{name} must be contiguous")
    if t.numel() < min_numel:
        _fail(fn, f"{name} holds {t.numel()} elements, the call touches {min_numel}")
    return t.data_ptr()


def _stream(stream) -> int:
    if stream is None:
        return torch._C._cuda_getCurrentRawStream(torch.cuda.current_device())
    if isinstance(stream, torch.cuda.Stream):
        return stream.cuda_stream
    return int(stream)


def _range_check(fn: str, t: torch.Tensor, n: int, lo: int, hi: int, name: str) -> None:
    if n == 0:
        return
    v = t.reshape(-1)[:n]
    mn, mx = int(v.min()), int(v.max())
    if mn < lo or mx >= hi:
        _fail(fn, f"{name} values must lie in [{lo}, {hi}), got [{mn}, {mx}]")


# ---------------------------------------------------------------------------------------------
# operators (ref: kernels/*.cuh)
# ---------------------------------------------------------------------------------------------
def embedding_lookup(table, ids, out, n_tokens: int, hidden: int, stream=None,
                     check_indices: bool | None = None) -> None:
    """out[t] = table[ids[t]] (ref: kernels/embedding.cuh:6-7)."""
    fn = "embedding_lookup"
    if table.dim() != 2 or table.shape[1] != hidden:
        _fail(fn, f"table must be [vocab, {hidden}]")
    pt = _dev(fn, table, torch.float16, 0, "table")
    pi = _dev(fn, ids, torch.int32, n_tokens, "ids")
    po = _dev(fn, out, torch.float16, n_tokens * hidden, "out")
    if _want_checks(check_indices):
        _range_check(fn, ids, n_tokens, 0, table.shape[0], "ids")
    _check(fn, _lib.llmk_embedding_lookup(pt, pi, po, n_tokens, hidden, _stream(stream)))


def residual_add(a, b, out, n: int, stream=None) -> None:
    """out = a + b in fp16, out may be a (ref: kernels/residual_add.cuh:6)."""
    fn = "residual_add"
    pa = _dev(fn, a, torch.float16, n, "a")
    pb = _dev(fn, b, torch.float16, n, "b")
    po = _dev(fn, out, torch.float16, n, "out")
    _check(fn, _lib.llmk_residual_add(pa, pb, po, n, _stream(stream)))


def rmsnorm(x, w, out, n_rows: int, hidden: int, eps: float, stream=None) -> None:
    """RMSNorm of n_rows rows (ref: kernels/rmsnorm.cuh:6-7)."""
    fn = "rmsnorm"
    px = _dev(fn, x, torch.float16, n_rows * hidden, "x")
    pw = _dev(fn, w, torch.float16, hidden, "w")
    po = _dev(fn, out, torch.float16, n_rows * hidden, "out")
    _check(fn, _lib.llmk_rmsnorm(px, pw, po, n_rows, hidden, eps, _stream(stream)))


def add_rmsnorm(residual, x, w, out, n_rows: int, hidden: int, eps: float, stream=None) -> None:
    """residual += x (fp16, in place), out = rmsnorm(residual)."""
    fn = "add_rmsnorm"
    pr = _dev(fn, residual, torch.float16, n_rows * hidden, "residual")
    px = _dev(fn, x, torch.float16, n_rows * hidden, "x")
    pw = _dev(fn, w, torch.float16, hidden, "w")
    po = _dev(fn, out, torch.float16, n_rows * hidden, "out")
    _check(fn, _lib.llmk_add_rmsnorm(pr, px, pw, po, n_rows, hidden, eps, _stream(stream)))


def compute_rope_inv_freq(head_dim: int, theta: float, factor: float, low_freq_factor: float,
                          high_freq_factor: float, original_max_pos: float) -> list[float]:
    """Host function: head_dim/2 llama3-scaled rotation speeds (ref: kernels/rope.cuh:7-9)."""
    if head_dim <= 0 or head_dim % 2:
        _fail("compute_rope_inv_freq", "head_dim must be even and positive")
    buf = (ctypes.c_float * (head_dim // 2))()
    _check("compute_rope_inv_freq",
           _lib.llmk_compute_rope_inv_freq(head_dim, theta, factor, low_freq_factor,
                                           high_freq_factor, original_max_pos, buf))
    return list(buf)


def rope_apply(q, k, positions, inv_freq, n_tokens: int, n_heads: int, n_kv_heads: int,
               head_dim: int, stream=None) -> None:
    """In-place RoPE of q and k (ref: kernels/rope.cuh:13-15)."""
    fn = "rope_apply"
    pq = _dev(fn, q, torch.float16, n_tokens * n_heads * head_dim, "q") if n_heads else 0
    pk = _dev(fn, k, torch.float16, n_tokens * n_kv_heads * head_dim, "k") if n_kv_heads else 0
    pp = _dev(fn, positions, torch.int32, n_tokens, "positions")
    pf = _dev(fn, inv_freq, torch.float32, head_dim // 2, "inv_freq")
    _check(fn, _lib.llmk_rope_apply(pq, pk, pp, pf, n_tokens, n_heads, n_kv_heads, head_dim,
                                    _stream(stream)))


def swiglu(gate, up, out, n: int, stream=None) -> None:
    """out = silu(gate) * up (ref: kernels/swiglu.cuh:6)."""
    fn = "swiglu"
    pg = _dev(fn, gate, torch.float16, n, "gate")
    pu = _dev(fn, up, torch.float16, n, "up")
    po = _dev(fn, out, torch.float16, n, "out")
    _check(fn, _lib.llmk_swiglu(pg, pu, po, n, _stream(stream)))


def _pool_rows(fn: str, pool, kvdim: int) -> int:
    if pool.numel() % kvdim:
        _fail(fn, f"pool size {pool.numel()} is not a whole number of {kvdim}-wide rows")
    return pool.numel() // kvdim


def kv_scatter(src, pool, block_table, start_pos: int, T: int, page_size: int, kvdim: int,
               stream=None, check_indices: bool | None = None) -> None:
    """Prefill scatter of T rows into pages (ref: kernels/kv_scatter.cuh:7-8)."""
    fn = "kv_scatter"
    if T > 0 and (start_pos < 0 or page_size <= 0):
        _fail(fn, "start_pos must be >= 0 and page_size > 0")
    n_table = (start_pos + T - 1) // page_size + 1 if T > 0 else 0
    ps = _dev(fn, src, torch.float16, T * kvdim, "src")
    pp = _dev(fn, pool, torch.float16, 0, "pool")
    pt = _dev(fn, block_table, torch.int32, n_table, "block_table")
    if _want_checks(check_indices) and T > 0:
        rows = _pool_rows(fn, pool, kvdim)
        first = start_pos // page_size
        _range_check(fn, block_table[first:n_table], n_table - first, 0, rows // page_size,
                     "block_table")
    _check(fn, _lib.llmk_kv_scatter(ps, pp, pt, start_pos, T, page_size, kvdim, _stream(stream)))


def _check_batch_tables(fn, block_tables, positions, pools, n, max_pages, page_size, kvdim):
    _range_check(fn, positions, n, 0, max_pages * page_size, "positions")
    rows = min(_pool_rows(fn, p, kvdim) for p in pools)
    pos = positions[:n].long()
    pages = block_tables.reshape(-1)[:n * max_pages].view(n, max_pages)
    used = pages.gather(1, (pos // page_size).unsqueeze(1)).squeeze(1)
    _range_check(fn, used, n, 0, rows // page_size, "block_tables (addressed entries)")


def kv_scatter_batch(src, pool, block_tables, positions, n: int, max_pages: int,
                     page_size: int, kvdim: int, stream=None,
                     check_indices: bool | None = None) -> None:
    """Decode scatter, one row per sequence (ref: kernels/kv_scatter.cuh:12-13)."""
    fn = "kv_scatter_batch"
    ps = _dev(fn, src, torch.float16, n * kvdim, "src")
    pp = _dev(fn, pool, torch.float16, 0, "pool")
    pt = _dev(fn, block_tables, torch.int32, n * max_pages, "block_tables")
    pq = _dev(fn, positions, torch.int32, n, "positions")
    if _want_checks(check_indices) and n > 0:
        _check_batch_tables(fn, block_tables, positions, [pool], n, max_pages, page_size, kvdim)
    _check(fn, _lib.llmk_kv_scatter_batch(ps, pp, pt, pq, n, max_pages, page_size, kvdim,
                                          _stream(stream)))


def rope_kv_scatter_batch(q, k, v, k_pool, v_pool, block_tables, positions, inv_freq, n: int,
                          max_pages: int, page_size: int, n_heads: int, n_kv_heads: int,
                          head_dim: int, stream=None, check_indices: bool | None = None) -> None:
    """Fused decode RoPE of q (in place) and k, with k and v scattered into their pools."""
    fn = "rope_kv_scatter_batch"
    kvdim = n_kv_heads * head_dim
    pq = _dev(fn, q, torch.float16, n * n_heads * head_dim, "q") if n_heads else 0
    pk = _dev(fn, k, torch.float16, n * kvdim, "k")
    pv = _dev(fn, v, torch.float16, n * kvdim, "v")
    pkp = _dev(fn, k_pool, torch.float16, 0, "k_pool")
    pvp = _dev(fn, v_pool, torch.float16, 0, "v_pool")
    pt = _dev(fn, block_tables, torch.int32, n * max_pages, "block_tables")
    pp = _dev(fn, positions, torch.int32, n, "positions")
    pf = _dev(fn, inv_freq, torch.float32, head_dim // 2, "inv_freq")
    if _want_checks(check_indices) and n > 0:
        _check_batch_tables(fn, block_tables, positions, [k_pool, v_pool], n, max_pages,
                            page_size, kvdim)
    _check(fn, _lib.llmk_rope_kv_scatter_batch(pq, pk, pv, pkp, pvp, pt, pp, pf, n, max_pages,
                                               page_size, n_heads, n_kv_heads, head_dim,
                                               _stream(stream)))


# Default of choose_num_splits; the same value as LLMK_ATTN_TARGET_BLOCKS in include/llmk.h.
ATTN_TARGET_BLOCKS = 65536
# Scratch floats of llmk_attention_decode_fast_noalloc (LLMK_ATTN_NOALLOC_MAX_FLOATS).
ATTN_NOALLOC_MAX_FLOATS = 256 * 32 * 32 * 66


def choose_num_splits(n_seq: int, n_kv_heads: int, max_seq_len: int,
                      target_blocks: int = ATTN_TARGET_BLOCKS) -> int:
    """Split count for attention_decode_fast (ref: kernels/attention_decode_fast.cuh:22-29)."""
    splits = target_blocks // (n_seq * n_kv_heads)
    splits = min(splits, (max_seq_len + 15) // 16, 32)
    return max(splits, 1)


def attention_decode_fast_workspace_floats(n_seq: int, n_heads: int, num_splits: int) -> int:
    """ref: kernels/attention_decode_fast.cuh:6"""
    return int(_lib.llmk_attention_decode_fast_workspace_floats(n_seq, n_heads, num_splits))


def attention_decode_fast(q, k_pool, v_pool, block_tables, seq_lens, out, workspace, n_seq: int,
                          max_pages: int, page_size: int, n_heads: int, n_kv_heads: int,
                          head_dim: int, num_splits: int, stream=None,
                          check_indices: bool | None = None) -> None:
    """Split-KV decode attention over the paged pool (ref: kernels/attention_decode_fast.cuh:14-18).

    With ``check_indices`` the binding also checks, on the host, that every sequence length
    fits the block table (seq_lens <= max_pages * page_size) and that every page number a
    cached position reads lies inside both pools."""
    fn = "attention_decode_fast"
    kvdim = n_kv_heads * head_dim
    pq = _dev(fn, q, torch.float16, n_seq * n_heads * head_dim, "q")
    pk = _dev(fn, k_pool, torch.float16, 0, "k_pool")
    pv = _dev(fn, v_pool, torch.float16, 0, "v_pool")
    pt = _dev(fn, block_tables, torch.int32, n_seq * max_pages, "block_tables")
    pl = _dev(fn, seq_lens, torch.int32, n_seq, "seq_lens")
    po = _dev(fn, out, torch.float16, n_seq * n_heads * head_dim, "out")
    ws_need = attention_decode_fast_workspace_floats(n_seq, n_heads, num_splits)
    pw = 0
    if workspace is not None:
        pw = _dev(fn, workspace, torch.float32, ws_need if num_splits > 1 else 0, "workspace")
    if (_want_checks(check_indices) and n_seq > 0 and max_pages > 0 and page_size > 0
            and kvdim > 0):
        _range_check(fn, seq_lens, n_seq, -(1 << 31), max_pages * page_size + 1, "seq_lens")
        lens = seq_lens[:n_seq].long().clamp(min=0)
        npages = (lens + page_size - 1) // page_size
        tables = block_tables.reshape(-1)[:n_seq * max_pages].view(n_seq, max_pages)
        used = torch.arange(max_pages, device=tables.device)[None, :] < npages[:, None]
        if bool(used.any()):
            rows = min(_pool_rows(fn, k_pool, kvdim), _pool_rows(fn, v_pool, kvdim))
            pages = tables[used]
            _range_check(fn, pages, pages.numel(), 0, rows // page_size,
                         "block_tables (entries of cached positions)")
    _check(fn, _lib.llmk_attention_decode_fast(pq, pk, pv, pt, pl, po, pw, n_seq, max_pages,
                                               page_size, n_heads, n_kv_heads, head_dim,
                                               num_splits, _stream(stream)))


def argmax_rows(logits, out, n_rows: int, vocab: int, stream=None) -> None:
    """out[r] = index of the largest value of row r, lowest index on ties
    (ref: kernels/argmax.cuh:5-7)."""
    fn = "argmax_rows"
    if n_rows < 0 or vocab <= 0:
        _fail(fn, "n_rows must be >= 0 and vocab > 0")
    pl = _dev(fn, logits, torch.float16, n_rows * vocab, "logits")
    po = _dev(fn, out, torch.int32, n_rows, "out")
    _check(fn, _lib.llmk_argmax_rows(pl, po, n_rows, vocab, _stream(stream)))


def copy_bytes(src, dst, nbytes: int, stream=None) -> None:
    """16-byte vector device copy (bandwidth probe)."""
    fn = "copy_bytes"
    if src.numel() * src.element_size() < nbytes or dst.numel() * dst.element_size() < nbytes:
        _fail(fn, "buffers smaller than nbytes")
    if src.device.type != "cuda" or dst.device.type != "cuda":
        _fail(fn, "buffers must be CUDA tensors")
    _check(fn, _lib.llmk_copy_bytes(src.data_ptr(), dst.data_ptr(), nbytes, _stream(stream)))


PROBE_READ, PROBE_COPY, PROBE_READ2, PROBE_INPLACE, PROBE_WRITE = range(5)


def bw_probe(mode: int, dst, nbytes: int, a=None, b=None, blocks: int = 0, unroll: int = 4,
             stream=None) -> None:
    """Bandwidth probe of one traffic mix (``llmk_bw_probe``; PROBE_READ reads `a`, PROBE_COPY
    a -> dst, PROBE_READ2 a, b -> dst, PROBE_INPLACE rewrites dst, PROBE_WRITE fills dst)."""
    fn = "bw_probe"
    for name, t in (("dst", dst), ("a", a), ("b", b)):
        if t is None:
            continue
        if t.device.type != "cuda":
            _fail(fn, f"{name} must be a CUDA tensor")
        if t.numel() * t.element_size() < nbytes:
            _fail(fn, f"{name} holds fewer than nbytes")
    _check(fn, _lib.llmk_bw_probe(mode, None if a is None else a.data_ptr(),
                                  None if b is None else b.data_ptr(), dst.data_ptr(), nbytes,
                                  blocks, unroll, _stream(stream)))


def empty_launch(blocks: int, threads: int, stream=None) -> None:
    """An empty kernel of blocks x threads (``llmk_empty_launch``): the launch floor."""
    _check("empty_launch", _lib.llmk_empty_launch(blocks, threads, _stream(stream)))


class DecodeNonGemmPass:
    """The non-GEMM decode pass over caller-owned tensors: embedding into ``residual``, then per
    layer add+RMSNorm, fused RoPE + K/V scatter, and SwiGLU (``llmk_decode_nongemm_pass``).

    ``layers`` is a list of dicts with the per-layer tensors x, norm_w, normed, q, k, v,
    k_pool, v_pool, gate, up, act; with x2, norm_w2 and normed2 in every layer as well, each
    layer also runs its second add + RMSNorm (after the RoPE + K/V scatter, before the SwiGLU),
    as the reference layer does. The descriptor (host pointer arrays) is built once; ``run``
    enqueues the whole pass on one stream and can be captured into a CUDA/HIP graph.
    """

    def __init__(self, embed_table, token_ids, residual, block_tables, positions, inv_freq,
                 layers, *, n_heads: int, n_kv_heads: int, head_dim: int, inter: int,
                 page_size: int, max_pages: int, eps: float, check_indices: bool = True):
        fn = "decode_nongemm_pass"
        n = token_ids.numel()
        hidden = residual.shape[-1]
        kvdim = n_kv_heads * head_dim
        self._keep = [embed_table, token_ids, residual, block_tables, positions, inv_freq,
                      layers]
        d = DecodePass()
        d.n_seqs, d.n_layers, d.hidden = n, len(layers), hidden
        d.n_heads, d.n_kv_heads, d.head_dim, d.inter = n_heads, n_kv_heads, head_dim, inter
        d.page_size, d.max_pages, d.eps = page_size, max_pages, eps
        if embed_table.dim() != 2 or embed_table.shape[1] != hidden:
            _fail(fn, f"embed_table must be [vocab, {hidden}]")
        d.embed_table = _dev(fn, embed_table, torch.float16, 0, "embed_table")
        d.token_ids = _dev(fn, token_ids, torch.int32, n, "token_ids")
        d.residual = _dev(fn, residual, torch.float16, n * hidden, "residual")
        d.block_tables = _dev(fn, block_tables, torch.int32, n * max_pages, "block_tables")
        d.positions = _dev(fn, positions, torch.int32, n, "positions")
        d.inv_freq = _dev(fn, inv_freq, torch.float32, head_dim // 2, "inv_freq")
        need = {"x": n * hidden, "norm_w": hidden, "normed": n * hidden,
                "q": n * n_heads * head_dim, "k": n * kvdim, "v": n * kvdim, "k_pool": 0,
                "v_pool": 0, "gate": n * inter, "up": n * inter, "act": n * inter}
        present = [sum(k in layer for k in ("x2", "norm_w2", "normed2")) for layer in layers]
        second = [c == 3 for c in present]
        if any(c not in (0, 3) for c in present) or (any(second) and not all(second)):
            _fail(fn, "x2, norm_w2 and normed2 go in every layer or in none")
        if layers and all(second):
            need.update({"x2": n * hidden, "norm_w2": hidden, "normed2": n * hidden})
        self._arrays = {}
        for key, cnt in need.items():
            arr = (_vp * max(1, len(layers)))()
            for l, layer in enumerate(layers):
                arr[l] = _dev(fn, layer[key], torch.float16, cnt, f"layers[{l}].{key}")
            self._arrays[key] = arr
            setattr(d, key, ctypes.cast(arr, ctypes.POINTER(_vp)))
        if check_indices and n > 0:
            _range_check(fn, token_ids, n, 0, embed_table.shape[0], "token_ids")
            pools = [layer[p] for layer in layers for p in ("k_pool", "v_pool")]
            if pools:
                _check_batch_tables(fn, block_tables, positions, pools, n, max_pages,
                                    page_size, kvdim)
        self._desc = d

    def run(self, stream=None) -> None:
        _check("decode_nongemm_pass",
               _lib.llmk_decode_nongemm_pass(ctypes.byref(self._desc), _stream(stream)))

    def run_layers(self, stream=None) -> None:
        """The same pass with one launch per layer (``llmk_decode_nongemm_pass_layers``)."""
        _check("decode_nongemm_pass_layers",
               _lib.llmk_decode_nongemm_pass_layers(ctypes.byref(self._desc), _stream(stream)))

    def run_fused(self, stream=None) -> None:
        """The same pass in one launch per 16 layers (``llmk_decode_nongemm_pass_fused``)."""
        _check("decode_nongemm_pass_fused",
               _lib.llmk_decode_nongemm_pass_fused(ctypes.byref(self._desc), _stream(stream)))


# ---------------------------------------------------------------------------------------------
# the decode step: projections, fused layouts, engine
# ---------------------------------------------------------------------------------------------
class Blas:
    """A GEMM handle (``llmk_blas``): hipBLASLt handle, 32 MiB workspace, per-shape plans.
    Stands where the reference passes a cublasHandle_t (ref: kernels/linear.cuh:7)."""

    def __init__(self):
        h = _vp()
        _check("blas_create", _lib.llmk_blas_create(ctypes.byref(h)))
        self._h = h

    @property
    def handle(self) -> int:
        return self._h.value

    def close(self) -> None:
        if self._h:
            _lib.llmk_blas_destroy(self._h)
            self._h = _vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def linear(handle: Blas, x, w, y, T: int, in_features: int, out_features: int,
           stream=None) -> None:
    """y[T, out] = x[T, in] W^T, W [out, in] row-major (ref: kernels/linear.cuh:5-7)."""
    fn = "linear"
    if T < 0 or in_features <= 0 or out_features <= 0:
        _fail(fn, "T must be >= 0 and the feature counts > 0")
    px = _dev(fn, x, torch.float16, T * in_features, "x")
    pw = _dev(fn, w, torch.float16, out_features * in_features, "w")
    py = _dev(fn, y, torch.float16, T * out_features, "y")
    _check(fn, _lib.llmk_linear(handle.handle, px, pw, py, T, in_features, out_features,
                                _stream(stream)))


LINEAR_ROWS_MAX = 8  # LLMK_LINEAR_ROWS_MAX
ENGINE_FUSE_FEW_ROWS = 1  # LLMK_ENGINE_FUSE_FEW_ROWS
ENGINE_HOST_ARGMAX = 2  # LLMK_ENGINE_HOST_ARGMAX


def linear_rows(x, w, y, T: int, in_features: int, out_features: int, stream=None) -> None:
    """linear() for T <= 8 rows with this library's weight-streaming kernel
    (``llmk_linear_rows``); in_features % 512 == 0."""
    fn = "linear_rows"
    if T < 0 or in_features <= 0 or out_features <= 0:
        _fail(fn, "T must be >= 0 and the feature counts > 0")
    px = _dev(fn, x, torch.float16, T * in_features, "x")
    pw = _dev(fn, w, torch.float16, out_features * in_features, "w")
    py = _dev(fn, y, torch.float16, T * out_features, "y")
    _check(fn, _lib.llmk_linear_rows(px, pw, py, T, in_features, out_features, _stream(stream)))


def _norm_ptr(fn, norm_w, in_features):
    return None if norm_w is None else _dev(fn, norm_w, torch.float16, in_features, "norm_w")


def linear_rows_norm(x, norm_w, eps: float, w, y, T: int, in_features: int, out_features: int,
                     stream=None) -> None:
    """y = rmsnorm(x) W^T for T <= 8 rows; norm_w None: y = x W^T (``llmk_linear_rows_norm``)."""
    fn = "linear_rows_norm"
    px = _dev(fn, x, torch.float16, T * in_features, "x")
    pw = _dev(fn, w, torch.float16, out_features * in_features, "w")
    py = _dev(fn, y, torch.float16, T * out_features, "y")
    _check(fn, _lib.llmk_linear_rows_norm(px, _norm_ptr(fn, norm_w, in_features), eps, pw, py, T,
                                          in_features, out_features, _stream(stream)))


def linear_rows_residual(x, w, residual, T: int, in_features: int, out_features: int,
                         stream=None) -> None:
    """residual += x W^T, rounded as linear then residual_add (``llmk_linear_rows_residual``)."""
    fn = "linear_rows_residual"
    px = _dev(fn, x, torch.float16, T * in_features, "x")
    pw = _dev(fn, w, torch.float16, out_features * in_features, "w")
    pr = _dev(fn, residual, torch.float16, T * out_features, "residual")
    _check(fn, _lib.llmk_linear_rows_residual(px, pw, pr, T, in_features, out_features,
                                              _stream(stream)))


def linear_rows_swiglu(x, norm_w, eps: float, w_gate_up, act, T: int, in_features: int,
                       inter: int, stream=None) -> None:
    """act = swiglu of the gate and up projections of rmsnorm(x) (``llmk_linear_rows_swiglu``)."""
    fn = "linear_rows_swiglu"
    px = _dev(fn, x, torch.float16, T * in_features, "x")
    pw = _dev(fn, w_gate_up, torch.float16, 2 * inter * in_features, "w_gate_up")
    pa = _dev(fn, act, torch.float16, T * inter, "act")
    _check(fn, _lib.llmk_linear_rows_swiglu(px, _norm_ptr(fn, norm_w, in_features), eps, pw, pa,
                                            T, in_features, inter, _stream(stream)))


def linear_rows_qkv_rope_scatter(x, norm_w, eps: float, w_qkv, q_out, k_pool, v_pool,
                                 block_tables, positions, inv_freq, T: int, in_features: int,
                                 n_heads: int, n_kv_heads: int, max_pages: int,
                                 stream=None) -> None:
    """The QKV projection of rmsnorm(x) with RoPE and the KV scatter in its epilogue (head_dim
    64, page size 16; ``llmk_linear_rows_qkv_rope_scatter``). The tables and positions are not
    checked against the pools here; the caller owns that."""
    fn = "linear_rows_qkv_rope_scatter"
    out = (n_heads + 2 * n_kv_heads) * 64
    px = _dev(fn, x, torch.float16, T * in_features, "x")
    pw = _dev(fn, w_qkv, torch.float16, out * in_features, "w_qkv")
    pq = _dev(fn, q_out, torch.float16, T * n_heads * 64, "q_out")
    pk = _dev(fn, k_pool, torch.float16, n_kv_heads * 64, "k_pool")
    pv = _dev(fn, v_pool, torch.float16, n_kv_heads * 64, "v_pool")
    pt = _dev(fn, block_tables, torch.int32, T * max_pages, "block_tables")
    pp = _dev(fn, positions, torch.int32, T, "positions")
    pf = _dev(fn, inv_freq, torch.float32, 32, "inv_freq")
    _check(fn, _lib.llmk_linear_rows_qkv_rope_scatter(
        px, _norm_ptr(fn, norm_w, in_features), eps, pw, pq, pk, pv, pt, pp, pf, T, in_features,
        n_heads, n_kv_heads, max_pages, _stream(stream)))


def blas_tune(handle: Blas, x, w, y, T: int, in_features: int, out_features: int,
              stream=None) -> None:
    """Chooses the algorithm of one projection shape by timing (``llmk_blas_tune``)."""
    fn = "blas_tune"
    px = _dev(fn, x, torch.float16, T * in_features, "x")
    pw = _dev(fn, w, torch.float16, out_features * in_features, "w")
    py = _dev(fn, y, torch.float16, T * out_features, "y")
    _check(fn, _lib.llmk_blas_tune(handle.handle, px, pw, py, T, in_features, out_features,
                                   _stream(stream)))


def qkv_rope_scatter(qkv, ld: int, q_out, k_pool, v_pool, block_tables, positions, inv_freq,
                     n: int, max_pages: int, page_size: int, n_heads: int, n_kv_heads: int,
                     head_dim: int, stream=None, check_indices: bool | None = None) -> None:
    """RoPE + KV scatter from the rows of a fused QKV projection (``llmk_qkv_rope_scatter``)."""
    fn = "qkv_rope_scatter"
    kvdim = n_kv_heads * head_dim
    if n < 0 or ld < (n_heads + 2 * n_kv_heads) * head_dim:
        _fail(fn, "n must be >= 0 and ld >= (n_heads + 2 n_kv_heads) head_dim")
    width = (n_heads + 2 * n_kv_heads) * head_dim
    pqkv = _dev(fn, qkv, torch.float16, (n - 1) * ld + width if n else 0, "qkv")
    pq = _dev(fn, q_out, torch.float16, n * n_heads * head_dim, "q_out")
    pk = _dev(fn, k_pool, torch.float16, 0, "k_pool")
    pv = _dev(fn, v_pool, torch.float16, 0, "v_pool")
    pt = _dev(fn, block_tables, torch.int32, n * max_pages, "block_tables")
    pp = _dev(fn, positions, torch.int32, n, "positions")
    pi = _dev(fn, inv_freq, torch.float32, head_dim // 2, "inv_freq")
    if _want_checks(check_indices) and n > 0:
        _check_batch_tables(fn, block_tables, positions, [k_pool, v_pool], n, max_pages,
                            page_size, kvdim)
    _check(fn, _lib.llmk_qkv_rope_scatter(pqkv, ld, pq, pk, pv, pt, pp, pi, n, max_pages,
                                          page_size, n_heads, n_kv_heads, head_dim,
                                          _stream(stream)))


def swiglu_rows(gate_up, out, n_rows: int, inter: int, stream=None) -> None:
    """out[r] = swiglu(gate_up[r, :inter], gate_up[r, inter:]) (``llmk_swiglu_rows``)."""
    fn = "swiglu_rows"
    if n_rows < 0 or inter <= 0:
        _fail(fn, "n_rows must be >= 0 and inter > 0")
    pg = _dev(fn, gate_up, torch.float16, n_rows * 2 * inter, "gate_up")
    po = _dev(fn, out, torch.float16, n_rows * inter, "out")
    _check(fn, _lib.llmk_swiglu_rows(pg, po, n_rows, inter, _stream(stream)))


BUF_LOGITS, BUF_NEXT_TOKENS, BUF_RESIDUAL, BUF_K_POOL, BUF_V_POOL, BUF_EMBED = range(6)

_hip = None


def _hip_memcpy(dst: int, src: int, nbytes: int) -> None:
    """Synchronous device/host copy through the HIP runtime (hipMemcpyDefault)."""
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        _hip.hipMemcpy.restype = _i
        _hip.hipMemcpy.argtypes = [_vp, _vp, _sz, _i]
    st = _hip.hipMemcpy(dst, src, nbytes, 4)
    if st != 0:
        raise LlmkError("hipMemcpy", st, error_string(st))


class Engine:
    """The decode-step engine (``llmk_engine``): a Llama-3 forward pass over batches of token
    rows, each row one new token of a sequence at a position, with the sequence's block table.
    It owns the weights (fused layout), the paged K/V pools of every layer, the activations and
    a GEMM handle. ref: engine/batched.cu:44-120, engine/model.cu:9-33, engine/paged.cu:15-28.
    """

    def __init__(self, cfg: ModelConfig, max_rows: int, max_pages: int, num_pages: int):
        self.cfg = cfg
        self.max_rows, self.max_pages, self.num_pages = max_rows, max_pages, num_pages
        e = _vp()
        _check("engine_create", _lib.llmk_engine_create(ctypes.byref(cfg), max_rows, max_pages,
                                                        num_pages, ctypes.byref(e)))
        self._e = e
        self.page_size = 16

    @property
    def handle(self) -> int:
        return self._e.value

    def close(self) -> None:
        if self._e:
            _lib.llmk_engine_destroy(self._e)
            self._e = _vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_weights(self, embed, final_norm, layers) -> None:
        """Copies the weights in (torch tensors, device or CPU, fp16, contiguous). ``layers`` is a
        list of dicts keyed by LayerWeights.NAMES, in the reference's [out, in] layout."""
        fn = "engine_set_weights"
        c = self.cfg
        qdim, kvdim, H, I = c.n_heads * c.head_dim, c.n_kv_heads * c.head_dim, c.hidden, c.inter
        shapes = {"attn_norm": (H,), "wq": (qdim, H), "wk": (kvdim, H), "wv": (kvdim, H),
                  "wo": (H, qdim), "mlp_norm": (H,), "w_gate": (I, H), "w_up": (I, H),
                  "w_down": (H, I)}

        def ptr(t, shape, name):
            if tuple(t.shape) != tuple(shape) or t.dtype != torch.float16 or not t.is_contiguous():
                _fail(fn, f"{name} must be a contiguous float16 tensor of shape {shape}, got "
                          f"{tuple(t.shape)} {t.dtype}")
            return t.data_ptr()

        if len(layers) != c.n_layers:
            _fail(fn, f"{len(layers)} layers given, the model has {c.n_layers}")
        arr = (LayerWeights * max(1, c.n_layers))()
        for l, w in enumerate(layers):
            for name in LayerWeights.NAMES:
                setattr(arr[l], name, ptr(w[name], shapes[name], f"layers[{l}].{name}"))
        pe = ptr(embed, (c.vocab, H), "embed")
        pf = ptr(final_norm, (H,), "final_norm")
        _check(fn, _lib.llmk_engine_set_weights(self._e, pe, pf, arr))

    def load_weights(self, path: str) -> None:
        _check("engine_load_weights", _lib.llmk_engine_load_weights(self._e, path.encode()))

    def set_rows(self, tokens, positions, block_tables, logit_rows=None, stream=None) -> None:
        """Uploads one batch of rows from host arrays (numpy/int sequences): tokens[n],
        positions[n], block_tables[n, max_pages] (or [n, <= max_pages], zero-padded here), and
        optionally the rows whose logits are wanted."""
        import numpy as np
        tok = np.ascontiguousarray(tokens, np.int32).reshape(-1)
        pos = np.ascontiguousarray(positions, np.int32).reshape(-1)
        n = tok.size
        if pos.size != n:
            _fail("engine_set_rows", "tokens and positions differ in length")
        tab = np.asarray(block_tables, np.int32).reshape(n, -1)
        if tab.shape[1] < self.max_pages:
            tab = np.concatenate([tab, np.zeros((n, self.max_pages - tab.shape[1]), np.int32)], 1)
        tab = np.ascontiguousarray(tab[:, :self.max_pages])
        lr = None if logit_rows is None else np.ascontiguousarray(logit_rows, np.int32).reshape(-1)
        self._rows = (tok, pos, tab, lr)  # keep the host arrays alive until the copy is staged
        _check("engine_set_rows", _lib.llmk_engine_set_rows(
            self._e, n, tok.ctypes.data, pos.ctypes.data, tab.ctypes.data,
            0 if lr is None else lr.size, None if lr is None else lr.ctypes.data,
            _stream(stream)))

    def forward(self, n_rows: int, n_logit_rows: int = -1, num_splits: int = 0,
                stream=None) -> None:
        _check("engine_forward", _lib.llmk_engine_forward(self._e, n_rows, n_logit_rows,
                                                          num_splits, _stream(stream)))

    def forward_graph(self, n_rows: int, n_logit_rows: int = -1, num_splits: int = 0,
                      stream=None) -> None:
        """forward() through the engine's HIP graph cache (``llmk_engine_forward_graph``);
        `stream` must not be the null stream."""
        _check("engine_forward_graph", _lib.llmk_engine_forward_graph(
            self._e, n_rows, n_logit_rows, num_splits, _stream(stream)))

    def tune(self, n_rows: int, n_logit_rows: int = -1, stream=None) -> None:
        """Times hipBLASLt's candidates for this row count's GEMM shapes (``llmk_engine_tune``)."""
        _check("engine_tune", _lib.llmk_engine_tune(self._e, n_rows, n_logit_rows,
                                                    _stream(stream)))

    def sched_model(self, stream) -> "SchedModel":
        """Scheduler callbacks that run this engine on `stream` (``llmk_engine_sched_model``)."""
        m = SchedModel()
        _check("engine_sched_model", _lib.llmk_engine_sched_model(self._e, _stream(stream),
                                                                  ctypes.byref(m)))
        m._engine = self  # keep the engine alive while the callbacks may run
        return m

    def reset_pools(self, stream=None) -> None:
        _check("engine_reset_pools", _lib.llmk_engine_reset_pools(self._e, _stream(stream)))

    def set_option(self, option: int, value: int) -> None:
        """``llmk_engine_set_option`` (ENGINE_FUSE_FEW_ROWS, ENGINE_HOST_ARGMAX)."""
        _check("engine_set_option", _lib.llmk_engine_set_option(self._e, option, value))

    def buffer_ptr(self, which: int, layer: int = 0) -> int:
        p = _lib.llmk_engine_buffer(self._e, which, layer)
        if not p:
            _fail("engine_buffer", f"no buffer {which} for layer {layer}")
        return p

    def _read(self, which: int, layer: int, shape, dtype) -> torch.Tensor:
        out = torch.empty(shape, dtype=dtype)
        nbytes = out.numel() * out.element_size()
        if nbytes:
            torch.cuda.synchronize()
            _hip_memcpy(out.data_ptr(), self.buffer_ptr(which, layer), nbytes)
        return out

    def logits(self, n: int) -> torch.Tensor:
        """Host copy of the last forward's logit rows, fp16 [n, vocab]."""
        return self._read(BUF_LOGITS, 0, (n, self.cfg.vocab), torch.float16)

    def next_tokens(self, n: int) -> torch.Tensor:
        return self._read(BUF_NEXT_TOKENS, 0, (n,), torch.int32)

    def residual(self, n: int) -> torch.Tensor:
        return self._read(BUF_RESIDUAL, 0, (n, self.cfg.hidden), torch.float16)

    def pool(self, which: int, layer: int) -> torch.Tensor:
        """Host copy of one layer's K (BUF_K_POOL) or V (BUF_V_POOL) pool."""
        c = self.cfg
        return self._read(which, layer, (self.num_pages, self.page_size, c.n_kv_heads,
                                         c.head_dim), torch.float16)

    def write_pool(self, which: int, layer: int, src: torch.Tensor) -> None:
        """Overwrites one layer's pool with a tensor of its size (device or host)."""
        c = self.cfg
        n = self.num_pages * self.page_size * c.n_kv_heads * c.head_dim
        if src.dtype != torch.float16 or src.numel() != n or not src.is_contiguous():
            _fail("engine_write_pool", f"src must be a contiguous float16 tensor of {n} elements")
        torch.cuda.synchronize()
        _hip_memcpy(self.buffer_ptr(which, layer), src.data_ptr(), 2 * n)


# ---------------------------------------------------------------------------------------------
# continuous batching (ref: engine/paging.h, engine/scheduler.h)
# ---------------------------------------------------------------------------------------------
class PageAllocator:
    """Page numbers from a free list (``llmk_page_allocator``; ref: engine/paging.h:7-23)."""

    def __init__(self, num_pages: int):
        a = _vp()
        _check("pages_create", _lib.llmk_pages_create(num_pages, ctypes.byref(a)))
        self._a = a

    @property
    def handle(self) -> int:
        return self._a.value

    @property
    def total(self) -> int:
        return _lib.llmk_pages_total(self._a)

    def num_free(self) -> int:
        return _lib.llmk_pages_num_free(self._a)

    def alloc(self) -> int:
        return _lib.llmk_pages_alloc(self._a)

    def release(self, page: int) -> None:
        _check("pages_release", _lib.llmk_pages_release(self._a, page))

    def set_free_list(self, order) -> None:
        import numpy as np
        o = np.ascontiguousarray(order, np.int32)
        _check("pages_set_free_list", _lib.llmk_pages_set_free_list(
            self._a, o.ctypes.data_as(_i32p), o.size))

    def close(self) -> None:
        if self._a:
            _lib.llmk_pages_destroy(self._a)
            self._a = _vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def python_sched_model(prefill, decode) -> SchedModel:
    """Wraps Python callables as scheduler callbacks: prefill(table: np.ndarray[max_pages],
    prompt: np.ndarray) -> int and decode(tokens, positions, tables [n, max_pages]) -> sequence
    of n ints. An exception ends the run with LLMK_ERR_INVALID_VALUE (and is re-raised by
    run_scheduler)."""
    import numpy as np
    m = SchedModel()
    m._errors = []

    def _prefill(user, table, max_pages, prompt, n, out):
        try:
            t = np.ctypeslib.as_array(table, (max_pages,)).copy()
            pr = np.ctypeslib.as_array(prompt, (n,)).copy()
            out[0] = int(prefill(t, pr))
            return 0
        except BaseException as exc:  # noqa: BLE001 - reported after the run
            m._errors.append(exc)
            return LLMK_ERR_INVALID_VALUE

    def _decode(user, n, tokens, positions, tables, max_pages, out, times):
        try:
            tok = np.ctypeslib.as_array(tokens, (n,)).copy()
            pos = np.ctypeslib.as_array(positions, (n,)).copy()
            tab = np.ctypeslib.as_array(tables, (n * max_pages,)).reshape(n, max_pages).copy()
            res = list(decode(tok, pos, tab))
            if len(res) != n:
                raise ValueError(f"decode returned {len(res)} tokens for {n} rows")
            for i, v in enumerate(res):
                out[i] = int(v)
            return 0
        except BaseException as exc:  # noqa: BLE001 - reported after the run
            m._errors.append(exc)
            return LLMK_ERR_INVALID_VALUE

    m._fns = (PREFILL_FN(_prefill), DECODE_FN(_decode))
    m.prefill, m.decode = m._fns
    return m


def run_scheduler(requests, max_running: int, max_pages: int, page_size: int,
                  pages: PageAllocator, model: SchedModel):
    """Runs ``llmk_scheduler_run``. requests: list of dicts with prompt (ints), max_new,
    arrival_step and optionally id, sorted by arrival_step. Returns (outputs: list of lists,
    stats: dict, times: list of (t_arrive, t_first, t_done) ms)."""
    import numpy as np
    n = len(requests)
    arr = (Request * max(1, n))()
    keep = []
    for i, r in enumerate(requests):
        pr = np.ascontiguousarray(r["prompt"], np.int32)
        out = np.zeros(max(1, int(r["max_new"])), np.int32)
        keep += [pr, out]
        arr[i].id = int(r.get("id", i))
        arr[i].prompt = pr.ctypes.data_as(_i32p)
        arr[i].prompt_len = pr.size
        arr[i].max_new = int(r["max_new"])
        arr[i].arrival_step = int(r.get("arrival_step", 0))
        arr[i].output = out.ctypes.data_as(_i32p)
    st = SchedStats()
    status = _lib.llmk_scheduler_run(arr, n, max_running, max_pages, page_size, pages.handle,
                                     ctypes.byref(model), ctypes.byref(st))
    errors = getattr(model, "_errors", [])
    if errors:
        raise errors[0]
    _check("scheduler_run", status)
    outputs = [list(keep[2 * i + 1][:arr[i].n_output]) for i in range(n)]
    times = [(arr[i].t_arrive_ms, arr[i].t_first_ms, arr[i].t_done_ms) for i in range(n)]
    return outputs, st.as_dict(), times
