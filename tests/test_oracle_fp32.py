"""The FP32 forms of the oracle's 4-bit products (the CPU baseline's timing
path) agree with the FP64 restatement to f32 accuracy: one matrix over a token
batch, and the grouped form over experts (every expert's routed tokens, experts
with no tokens, repeated experts across a token's slots)."""
import numpy as np
import pytest

import oracle


def _q4(rng, *shape):
    n, k = shape[-2], shape[-1]
    w = rng.integers(0, 2 ** 32, size=shape[:-1] + (k // 8,), dtype=np.uint64).astype(np.uint32)
    s = (rng.standard_normal(shape[:-1] + (k // 64,)) * 0.02).astype(np.float32)
    b = (rng.standard_normal(shape[:-1] + (k // 64,)) * 0.02).astype(np.float32)
    return w, s, b


def _rel(a, b):
    return float(np.max(np.abs(a - b)) / np.sqrt(np.mean(b * b)))


@pytest.mark.parametrize("M,N,K", [(1, 64, 64), (5, 48, 1024), (37, 512, 2048)])
def test_qmm4_f32_matches_fp64(M, N, K):
    rng = np.random.default_rng(M * 131 + K)
    w, s, b = _q4(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    assert _rel(oracle.qmm4_f32(x, w, s, b), oracle.qmm(x, w, s, b)) < 1e-5


def test_gather_qmm4_f32_matches_fp64():
    rng = np.random.default_rng(7)
    E, N, K, M, top = 9, 96, 512, 23, 3
    w, s, b = _q4(rng, E, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    idx = rng.integers(0, E - 2, size=(M, top)).astype(np.int32)  # experts E-2, E-1 get no tokens
    idx[0] = [4, 4, 4]                                            # one token routed to an expert thrice
    got, want = oracle.gather_qmm4_f32(x, w, s, b, idx), oracle.gather_qmm(x, w, s, b, idx)
    assert got.shape == want.shape
    assert _rel(got, want) < 1e-5


def test_fp32_forms_refuse_bad_shapes():
    rng = np.random.default_rng(1)
    w, s, b = _q4(rng, 16, 96)
    with pytest.raises(Exception):
        oracle.qmm4_f32(np.zeros((2, 96), np.float32), w, s, b)  # K not a multiple of 64
    w, s, b = _q4(rng, 3, 16, 64)
    with pytest.raises(Exception):
        oracle.gather_qmm4_f32(np.zeros((2, 64), np.float32), w, s, b, np.array([[0], [3]], np.int32))
