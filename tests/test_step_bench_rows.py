"""The rows file bench.py hands to llmk_step_bench (the decode step timed from a C++ process):
its layout against the C struct the program reads, and the program's refusals of bad input,
which happen before any HIP call (CPU only)."""
import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402
from __graft_entry__ import load_llmk  # noqa: E402

EXE = os.path.join(ROOT, "cuda-llm-engine_amd", "llmk_step_bench")


@pytest.fixture(scope="module")
def llmk():
    return load_llmk()


def test_rows_file_layout(llmk, tmp_path):
    cfg = llmk.ModelConfig()
    n, max_pages, num_pages = 5, 8, 40
    rng = np.random.default_rng(3)
    tokens = rng.integers(0, cfg.vocab, n)
    pos = rng.integers(0, 100, n)
    tables = rng.integers(0, num_pages, (n, 3))  # narrower than max_pages: zero-padded
    path = tmp_path / "r.rows"
    bench.write_step_rows(str(path), cfg, tokens, pos, tables, num_pages, max_pages)
    raw = path.read_bytes()
    assert raw[:8] == b"LLMKROWS"
    size = ctypes.sizeof(llmk.ModelConfig)
    assert size == 72  # 7 int32 + float + 5 double, as llmk_model_config
    back = llmk.ModelConfig.from_buffer_copy(raw[8:8 + size])
    assert (back.n_layers, back.hidden, back.vocab) == (cfg.n_layers, cfg.hidden, cfg.vocab)
    assert back.rope_theta == cfg.rope_theta and back.eps == cfg.eps
    body = np.frombuffer(raw[8 + size:], np.int32)
    assert body[:3].tolist() == [n, max_pages, num_pages]
    assert body[3:3 + n].tolist() == tokens.tolist()
    assert body[3 + n:3 + 2 * n].tolist() == pos.tolist()
    tab = body[3 + 2 * n:].reshape(n, max_pages)
    assert tab[:, :3].tolist() == tables.tolist() and not tab[:, 3:].any()
    assert body.size == 3 + 2 * n + n * max_pages


def test_rows_file_rejects_mismatched_lengths(llmk, tmp_path):
    with pytest.raises(ValueError):
        bench.write_step_rows(str(tmp_path / "r.rows"), llmk.ModelConfig(), [1, 2], [0],
                              [[0], [0]], 4, 2)


@pytest.mark.skipif(not os.path.exists(EXE), reason="llmk_step_bench is not built")
def test_step_bench_refuses_bad_input(tmp_path):
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "usage" in r.stderr
    r = subprocess.run([EXE, str(tmp_path / "missing.rows")], capture_output=True, text=True,
                       timeout=60)
    assert r.returncode == 1 and "open rows file" in r.stderr
    bad = tmp_path / "bad.rows"
    bad.write_bytes(b"NOTROWS!" + bytes(200))
    r = subprocess.run([EXE, str(bad)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "read rows header" in r.stderr
    short = tmp_path / "short.rows"
    short.write_bytes(b"LLMKROWS" + bytes(10))
    r = subprocess.run([EXE, str(short)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "read rows header" in r.stderr
