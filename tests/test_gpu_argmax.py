"""GPU parity of the row argmax (llmk_argmax_rows) against the CPU oracle: the rows of the
reference's own test (ref: tests/test_argmax.cu:10-25) -- many exact ties, a constant row, the
maximum at the last index, two equal maxima at 0 and 77777 -- plus NaN, +-inf and +-0 rows, a
decode batch of 256 rows, and the scalar path (unaligned rows, vocab not a multiple of 8,
short rows). Bar: bit-exact (integer indices)."""
import numpy as np
import pytest
import torch

from test_oracle import argmax_reference_rows

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
V = 128256


def run(llmk, rows_bits: np.ndarray, offset: int = 0) -> np.ndarray:
    n, vocab = rows_bits.shape
    flat = np.zeros(n * vocab + offset, np.uint16)
    flat[offset:] = rows_bits.reshape(-1)
    t = torch.from_numpy(flat.view(np.float16)).to(DEV)
    out = torch.full((n + 1,), -7, dtype=torch.int32, device=DEV)
    llmk.argmax_rows(t[offset:], out, n, vocab)
    got = out.cpu().numpy()
    assert got[n] == -7, "write past the output"
    return got[:n]


def test_reference_rows(llmk, orc):
    rows = argmax_reference_rows(np.random.default_rng(3))
    got = run(llmk, rows)
    assert np.array_equal(got, orc.argmax_rows(rows, 8, V))
    assert got[4] == 0 and got[5] == V - 1 and got[6] == 0


def special_rows(vocab):
    nan, inf = np.float16(np.nan), np.float16(np.inf)
    rng = np.random.default_rng(11)
    rows = rng.uniform(-3, 3, (8, vocab)).astype(np.float16)
    rows[0, ::7] = nan                  # NaN never wins
    rows[0, vocab // 2] = 50
    rows[1, :] = nan                    # nothing above -inf: INT_MAX
    rows[2, :] = -inf
    rows[3, :] = -1
    rows[3, [5, vocab - 3]] = 0.0       # +0 and -0 tie: the first
    rows[3, 5] = -0.0
    rows[4, :] = -inf
    rows[4, vocab - 1] = -60000         # one finite value
    rows[5, [17, vocab - 2]] = inf      # equal +inf maxima
    rows[6, :] = nan
    rows[6, 3] = -inf
    rows[6, vocab - 1] = -65504
    rows[7, :] = 0                      # all zero: index 0
    return rows.view(np.uint16)


@pytest.mark.parametrize("vocab", [V, 8192, 32000, 8191, 100])
def test_nan_inf_and_signed_zero(llmk, orc, vocab):
    rows = special_rows(vocab)
    got = run(llmk, rows)
    exp = orc.argmax_rows(rows, 8, vocab)
    assert np.array_equal(got, exp)
    assert got[1] == 0x7FFFFFFF and got[2] == 0x7FFFFFFF and got[3] == 5 and got[5] == 17
    assert got[6] == vocab - 1


def test_decode_batch_with_ties(llmk, orc):
    rng = np.random.default_rng(12)
    rows = (rng.integers(-40, 41, (256, V)) * 0.25).astype(np.float16).view(np.uint16)
    assert np.array_equal(run(llmk, rows), orc.argmax_rows(rows, 256, V))


@pytest.mark.parametrize("offset,vocab", [(1, V), (0, V - 1), (3, 4099)])
def test_scalar_path(llmk, orc, offset, vocab):
    rng = np.random.default_rng(offset * 7 + vocab)
    rows = (rng.integers(-20, 21, (5, vocab)) * 0.5).astype(np.float16).view(np.uint16)
    assert np.array_equal(run(llmk, rows, offset), orc.argmax_rows(rows, 5, vocab))


def test_zero_rows_and_bad_arguments(llmk):
    t = torch.zeros(16, dtype=torch.float16, device=DEV)
    out = torch.zeros(1, dtype=torch.int32, device=DEV)
    llmk.argmax_rows(t, out, 0, 16)
    with pytest.raises(llmk.LlmkError):
        llmk.argmax_rows(t, out, 1, 0)
    with pytest.raises(llmk.LlmkError):
        llmk.argmax_rows(t, out, 2, 16)  # logits too short


@pytest.mark.parametrize("vocab", [8200, 32008, V, 131080])
def test_maxima_in_the_last_vector(llmk, orc, vocab):
    """Past the row's end the 16-byte kernel reloads the last vector instead of masking, so a
    copy of it shows up at indices >= vocab: every maximum placed in that vector must still
    come back at its own index (8200 and 32008 leave thousands of copies; 131080 needs a second
    pass over the row)."""
    rng = np.random.default_rng(vocab)
    rows = rng.uniform(-3, 3, (8, vocab)).astype(np.float16)
    nan, inf = np.float16(np.nan), np.float16(np.inf)
    rows[0, vocab - 1] = 9                       # last element
    rows[1, vocab - 8] = 9                       # first element of the last vector
    rows[2, [vocab - 5, vocab - 1]] = 9          # tie inside the last vector
    rows[3, [3, vocab - 1]] = 9                  # tie with the start of the row
    rows[4, :] = nan                             # no value above -inf anywhere
    rows[4, vocab - 8:] = -inf
    rows[5, vocab - 8:] = 9                      # the whole last vector ties
    rows[6, vocab - 8:] = inf
    rows[6, vocab // 3] = inf                    # +inf earlier in the row wins the tie
    rows[7, :] = -2
    rows[7, vocab - 2] = -0.0                    # -0 and +0 tie: the first
    rows[7, vocab - 1] = 0.0
    bits = rows.view(np.uint16)
    got = run(llmk, bits)
    assert np.array_equal(got, orc.argmax_rows(bits, 8, vocab))
    assert list(got) == [vocab - 1, vocab - 8, vocab - 5, 3, 0x7FFFFFFF, vocab - 8, vocab // 3,
                         vocab - 2]
