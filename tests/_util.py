"""Small helpers shared by the tests."""
import numpy as np

# Attention tolerance of the hot path: fp32 accumulation
# on both sides, max-abs 2e-3 plus relative 1e-3 of the reference value.
ATOL = 2e-3
RTOL = 1e-3

# Worst error-to-bound ratio per full-size check, printed at the end of the
# session (conftest.pytest_terminal_summary): name -> (outputs, max abs err,
# max err / bound).
MARGINS = {}


def make_values(count, seed):
    """The reference tests' input generator (test_attention.cpp:12-21): a
    32-bit LCG, value = ((state >> 8) & 0xFFFF) / 32768 - 1, times 0.25."""
    out = np.empty(count, np.float32)
    state = (seed | 1) & 0xFFFFFFFF
    for i in range(count):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = (np.float32((state >> 8) & 0xFFFF) / np.float32(32768.0) - np.float32(1.0)) \
            * np.float32(0.25)
    return out


def assert_attention_close(got, want, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = np.abs(got - want)
    bound = ATOL + RTOL * np.abs(want)
    worst = np.unravel_index(np.argmax(err - bound), err.shape)
    assert np.all(err <= bound), (
        f"{what}: max abs err {err.max():.3e} at {worst}: got {got[worst]:.6f} want {want[worst]:.6f}")
    return float(err.max())


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a
