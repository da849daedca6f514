"""The Q8_1 kernels' division-free rounding, restated in f32 numpy (CPU).

rq_kernels.hip (q8_codes) computes rint(x * (1 / d)) and keeps it only when
x * (1 / d) is farther than 2^-14 from every half-integer; elsewhere it
divides. These tests check on the CPU, with IEEE f32 arithmetic, that the
window never keeps a code that differs from rint(x / d), on the inputs that
stress it: quotients on and next to ties, subnormal and zero d, huge and
infinite amax. The GPU tests then check the kernels themselves against the
oracle on the same inputs.
"""
import numpy as np
import pytest

from q8_inputs import near_tie_rows

F32 = np.float32
WINDOW = F32(0.5 - 2.0 ** -14)


def _codes(x: np.ndarray):
    """(window codes, division codes, kept-by-window mask, |t - x/d| max)."""
    xb = x.reshape(-1, 32).astype(F32)
    amax = np.abs(xb).max(1).astype(F32)
    d = (amax / F32(127)).astype(F32)
    with np.errstate(all="ignore"):
        r = (F32(1) / d).astype(F32)
        t = (xb * r[:, None]).astype(F32)
        rt = np.rint(t).astype(F32)
        kept = np.abs((t - rt).astype(F32)) < WINDOW
        div = np.where(d[:, None] > 0, np.rint((xb / d[:, None]).astype(F32)), F32(0))
        exact = xb.astype(np.float64) / d[:, None].astype(np.float64)
        err = np.where(kept, np.abs(t.astype(np.float64) - exact), 0.0)
    return rt, div, kept, float(err.max())


@pytest.mark.parametrize("seed", range(6))
def test_window_matches_division_near_ties(seed):
    x = near_tie_rows(64, 4096, seed)
    rt, div, kept, err = _codes(x)
    assert not np.any(kept & (rt != div))
    assert err < 2.3e-5  # the bound the kernel's comment derives
    assert kept.mean() < 0.2  # the inputs do sit in the fallback window


@pytest.mark.parametrize("scale", [1e-44, 1e-40, 1e-38, 1e-3, 1.0, 1e30, 3e38])
def test_window_matches_division_random(scale):
    rng = np.random.default_rng(int(np.log10(scale) + 50))
    with np.errstate(over="ignore"):
        x = (rng.standard_normal(32 * 4096) * scale).astype(F32)
    rt, div, kept, err = _codes(x)
    assert not np.any(kept & (rt != div))
    assert err < 2.3e-5
    if 1e-30 < scale < 1e30:
        assert kept.mean() > 0.999  # the fast path is the common case


def test_window_falls_back_on_zero_and_subnormal_d():
    x = np.zeros(64, F32)
    x[33] = F32(1e-44)  # d = 0 after rounding amax / 127
    rt, div, kept, _ = _codes(x)
    assert not kept.any()
    assert not np.any(div)
