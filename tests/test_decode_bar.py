"""The shared decode bar (decode_bar.py) on planted differences, CPU only: it excuses exactly a one-step rounding of a
near-tie and nothing wider."""
import numpy as np
import pytest

import decode_bar as D


def bits(x):
    return (np.asarray(x, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def val(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def case(unrounded):
    """oracle pair for the given unrounded values: bf16 bits rounded to nearest even, and the f32 values."""
    f = np.asarray(unrounded, np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r, f


def quiet(*a):
    pass


def test_identical_and_small_differences_pass():
    wb, wf = case(np.linspace(-3, 3, 64))
    D.check(wb, (wb, wf), "same", quiet)
    g = wb.copy(); g[5] += 1                                  # one step at |x| < 4 is below 2e-2
    D.check(g, (wb, wf), "one step small", quiet)


def test_near_tie_flip_at_large_magnitude_passes():
    mid = np.float32(4.0 + 2 ** -6)                           # midpoint between bf16 4.0 and 4.03125
    wf = np.array([mid * (1 - 1e-5)] + [0.1] * 63, np.float32)
    wb, _ = case(wf)
    assert val(wb[0]) == 4.0
    g = wb.copy(); g[0] += 1                                  # the other side of the near-tie: 4.03125
    _, _, nt = D.check(g, (wb, wf), "near tie", quiet)
    assert nt == 1


def test_flip_away_from_a_tie_fails():
    wf = np.array([4.0 + 2 ** -8] + [0.1] * 63, np.float32)   # a quarter step above 4.0: no tie
    wb, _ = case(wf)
    g = wb.copy(); g[0] += 1
    with pytest.raises(AssertionError):
        D.check(g, (wb, wf), "not a tie", quiet)


def test_two_steps_at_a_tie_fails():
    mid = np.float32(4.0 + 2 ** -6)
    wf = np.array([mid] + [0.1] * 63, np.float32)
    wb, _ = case(wf)
    g = wb.copy(); g[0] += 2
    with pytest.raises(AssertionError):
        D.check(g, (wb, wf), "two steps", quiet)


def test_mean_abs_bar_and_float_input():
    wb, wf = case(np.full(64, 0.5, np.float32))
    g = wb.copy(); g[:] += 1                                  # every element one step (2^-8) off: mean 3.9e-3
    with pytest.raises(AssertionError):
        D.check(g, (wb, wf), "mean", quiet)
    D.check(val(wb), (wb, wf), "float form", quiet)
    with pytest.raises(AssertionError):
        D.check(val(wb) + np.float32(1e-6), (wb, wf), "not bf16", quiet)
