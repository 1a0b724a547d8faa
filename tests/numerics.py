"""Shared tolerance checks for the parity tests.

bf16 activations/logits: |gpu - oracle| <= 2e-2 * |oracle| + 2e-2 * rms(oracle)
element-wise (rel 2e-2 as the product tolerance states, with an absolute floor
scaled by the tensor's RMS so that values near zero are judged against the
tensor's magnitude). fp32 recurrent state: the same form at 1e-3.
"""
import numpy as np

BF16_REL = 2e-2
STATE_REL = 1e-3


def assert_close(got, want, rel, what=""):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    scale = float(np.sqrt(np.mean(want * want))) if want.size else 0.0
    err = np.abs(got - want)
    bound = rel * np.abs(want) + rel * scale
    bad = err > bound
    if bad.any():
        i = int(np.argmax(err - bound))
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{err.size} elements out of tolerance; worst at {np.unravel_index(i, err.shape)}"
            f" got={got.reshape(-1)[i]!r} want={want.reshape(-1)[i]!r} rms={scale:.4g} max_err={err.max():.4g}")
    return float(err.max() / max(scale, 1e-30))


def assert_bf16_close(got, want, what=""):
    return assert_close(got, want, BF16_REL, what)


def assert_state_close(got, want, what=""):
    return assert_close(got, want, STATE_REL, what)
