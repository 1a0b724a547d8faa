"""The chunked statement of the gated delta rule (gdn_chunk_ref, the form the
device's chunked prefill kernel computes) against the token-serial rule of
native/qwen_model.inc:191-200, in FP64: any dropped decay factor, wrong
triangle or misplaced beta in the closed form breaks the equality."""
import numpy as np
import pytest

import gdn_chunk_ref as ref

DK = DV = 16


def inputs(T, seed):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((T, DK))
    k = rng.standard_normal((T, DK))
    q /= np.linalg.norm(q, axis=1, keepdims=True) * np.sqrt(DK)
    k /= np.linalg.norm(k, axis=1, keepdims=True)
    v = rng.standard_normal((T, DV))
    g = np.exp(-rng.uniform(0.0, 1.0, T) * np.log1p(np.exp(rng.standard_normal(T))))
    beta = 1 / (1 + np.exp(-rng.standard_normal(T)))
    S = rng.standard_normal((DV, DK)) * 0.1
    return q, k, v, g, beta, S


@pytest.mark.parametrize("T", [1, 2, 15, 16, 17, 63, 64, 65, 130, 200])
def test_chunked_equals_serial(T):
    q, k, v, g, beta, S = inputs(T, T)
    o_s, S_s = ref.serial(q, k, v, g, beta, S)
    o_c, S_c = ref.chunked(q, k, v, g, beta, S)
    assert np.allclose(S_c, S_s, rtol=0, atol=1e-12 * np.abs(S_s).max())
    assert np.allclose(o_c, o_s, rtol=0, atol=1e-12 * max(np.abs(o_s).max(), 1e-30))


def test_chunk_with_strong_decay():
    # decays near zero make L span many orders of magnitude; the ratios
    # exp(L_t - L_i) are formed from differences and stay finite
    q, k, v, g, beta, S = inputs(64, 7)
    g[::5] = 1e-6
    o_s, S_s = ref.serial(q, k, v, g, beta, S)
    o_c, S_c = ref.chunk(q, k, v, g, beta, S)
    assert np.allclose(S_c, S_s, rtol=0, atol=1e-12 * np.abs(S_s).max())
    assert np.allclose(o_c, o_s, rtol=0, atol=1e-12 * np.abs(o_s).max())


def test_unit_decay_zero_beta_is_identity():
    # beta = 0 and g = 1 (the kernel's padding of a partial chunk) leaves the
    # state unchanged and reads o = S q
    q, k, v, g, beta, S = inputs(10, 3)
    o, S2 = ref.chunk(q, k, v, np.ones(10), np.zeros(10), S)
    assert np.array_equal(S2, S)
    assert np.allclose(o, q @ S.T, rtol=1e-14, atol=0)
