"""CPU pins for the expert permutation of the oracle (orc_expert_permute).

The reference sorts the flattened (token, slot) expert ids with mx::argsort
(native/qwen_model.inc:81) and gathers by the inverse; MLX does not document
that sort's stability, so the build defines it stable. These checks fix the
oracle against three independent statements of a stable sort by expert:
numpy's stable argsort, a per-expert brute-force scan, and the counting
identities (inverse is the inverse permutation; offsets are the exclusive
prefix sum of the per-expert counts)."""
import numpy as np
import pytest

import oracle


def brute_force(flat, experts):
    order, offsets = [], [0]
    for e in range(experts):
        order += [p for p, x in enumerate(flat) if x == e]
        offsets.append(len(order))
    return order, offsets


@pytest.mark.parametrize("seed,tokens,top,experts", [(0, 1, 1, 1), (1, 7, 2, 8), (2, 64, 10, 512), (3, 256, 10, 512),
                                                     (4, 33, 3, 5), (5, 16, 4, 64)])
def test_permute_is_stable_sort_by_expert(seed, tokens, top, experts):
    rng = np.random.default_rng(seed)
    # a hot expert, an unused range and a uniform remainder, so zero-token
    # experts and long runs of one expert both occur
    hot = int(rng.integers(0, experts))
    idx = rng.integers(0, max(1, experts // 2), (tokens, top)).astype(np.int32)
    idx[rng.random((tokens, top)) < 0.3] = hot
    flat = idx.reshape(-1)
    order, inverse, offsets = oracle.expert_permute(idx, experts)
    assert np.array_equal(order, np.argsort(flat, kind="stable"))
    assert np.array_equal(inverse, np.argsort(order))
    assert np.array_equal(order[inverse], np.arange(flat.size))
    want_off = np.concatenate([[0], np.cumsum(np.bincount(flat, minlength=experts))])
    assert np.array_equal(offsets, want_off)
    bf_order, bf_off = brute_force(flat.tolist(), experts)
    assert order.tolist() == bf_order and offsets.tolist() == bf_off
    assert np.all(np.diff(flat[order]) >= 0)
    if experts > 1:
        assert np.any(np.diff(offsets) == 0), "case must hold an expert with no tokens"


def test_permute_rejects_out_of_range():
    with pytest.raises(oracle.OracleError):
        oracle.expert_permute(np.array([[0, 8]], np.int32), 8)
    with pytest.raises(oracle.OracleError):
        oracle.expert_permute(np.array([[-1]], np.int32), 8)
