"""The graph API's fused operators, rs_mlx_kernel ops 1-6 (native/mlx_bridge.cpp:
141-167, built by src/serving/native_ops.rs:53-244), through
rs_mlx_input / rs_mlx_kernel / rs_mlx_finish:

- the reference's own closed forms (tests/native_execution.rs:129-209):
  rope(1, 0; offset 1) = (cos 1, sin 1); causal means [2, 4, 4, 6];
  gated delta y = [0.5, 1, 1.5, 2], S = [0.5, 3, 1, 4];
  route -> gather -> mix = 32 (1 + 2e) / (1 + e), and the out-of-range
  expert index refused;
- seeded shapes against the oracle's FP64 restatements (rope, paged
  attention, the gated delta rule, route top-k, gather_qmm at every
  bits x group, the expert mix), f32 tolerance 1e-5 of the RMS;
- malformed descriptors fail with the callers' messages and add no node.
"""
import numpy as np
import pytest

import oracle
from numerics import assert_close

pytestmark = pytest.mark.gpu
F32_REL = 1e-5


@pytest.fixture
def graph(bridge):
    return bridge.GraphHandle(1)


def test_rope_closed_form(graph):
    x = graph.input(np.array([1.0, 0.0], np.float32).reshape(1, 1, 1, 2))
    y = graph.kernel(1, [x], ints=[2, 1], floats=[10000.0])
    got = graph.finish(y, (2,))
    np.testing.assert_allclose(got, [np.cos(1.0), np.sin(1.0)], rtol=1e-6, atol=1e-7)


def test_causal_attention_closed_form(graph):
    q = graph.input(np.zeros((1, 2, 2, 2), np.float32))
    k = graph.input(np.zeros((1, 1, 2, 2), np.float32))
    v = graph.input(np.array([2.0, 4.0, 6.0, 8.0], np.float32).reshape(1, 1, 2, 2))
    y = graph.kernel(2, [q, k, v], ints=[1], floats=[1.0])
    np.testing.assert_allclose(graph.finish(y, (8,)), [2, 4, 4, 6, 2, 4, 4, 6], rtol=1e-6)


def test_gated_delta_closed_form(graph):
    q = graph.input(np.array([0.5, 0, 0, 0.5], np.float32).reshape(1, 2, 1, 2))
    k = graph.input(np.array([1, 0, 0, 1], np.float32).reshape(1, 2, 1, 2))
    v = graph.input(np.array([2, 4, 6, 8], np.float32).reshape(1, 2, 2, 1))
    decay = graph.input(np.full((1, 2, 2), 0.5, np.float32))
    beta = graph.input(np.full((1, 2, 2), 0.5, np.float32))
    state = graph.input(np.zeros((1, 2, 1, 2), np.float32))
    y, s = graph.kernel(3, [q, k, v, decay, beta, state], outputs=2)
    np.testing.assert_allclose(graph.finish(y, (4,)), [0.5, 1, 1.5, 2], rtol=1e-6)
    np.testing.assert_allclose(graph.finish(s, (4,)), [0.5, 3, 1, 4], rtol=1e-6)


def test_route_gather_mix_closed_form_and_oob(graph):
    from hip_bridge import HipBridgeError

    logits = graph.input(np.array([[-10.0, 0.0, 1.0]], np.float32))
    idx, scores = graph.kernel(4, [logits], ints=[2], outputs=2)
    x = graph.input(np.ones((1, 32), np.float32))
    w = graph.input(np.zeros((3, 1, 4), np.uint32))
    sc = graph.input(np.ones((3, 1, 1), np.float32))
    bi = graph.input(np.array([0.0, 1.0, 2.0], np.float32).reshape(3, 1, 1))
    unsafe = graph.input(np.array([[3]], np.uint32))
    before = graph.count
    with pytest.raises(HipBridgeError, match="out-of-range expert"):
        graph.kernel(5, [x, w, sc, bi, unsafe], ints=[32, 4])
    graph.count = before  # the failed call added no node
    experts = graph.kernel(5, [x, w, sc, bi, idx], ints=[32, 4])
    y = graph.kernel(6, [experts, scores])
    e = np.e
    np.testing.assert_allclose(graph.finish(y, (1,)), [32 * (1 + 2 * e) / (1 + e)], rtol=1e-6)
    got_idx = graph.finish(idx, (2,), np.uint32)
    assert list(got_idx) == [2, 1]
    np.testing.assert_allclose(graph.finish(scores, (2,)), [e / (1 + e), 1 / (1 + e)], rtol=1e-6)


@pytest.mark.parametrize("seed,offset", [(0, 3), (1, 40), (2, 4000)])
def test_rope_matches_oracle(graph, seed, offset):
    """Angles (offset + l) * base^(-2i/dims) are formed in f32, as MLX's
    fast::rope forms them, so an angle a carries ~a * 2^-23 of rounding: the
    tolerance is 1e-5 plus (offset + L) * 2^-20 relative to the RMS."""
    rng = np.random.default_rng(seed)
    B, H, L, D, dims = 2, 3, 7, 64, [64, 32, 16][seed]
    x = rng.standard_normal((B, H, L, D)).astype(np.float32)
    y = graph.kernel(1, [graph.input(x)], ints=[dims, offset], floats=[1e6])
    got = graph.finish(y, x.shape)
    # oracle layout: [tokens][heads][dim] with one position per token
    xt = x.transpose(2, 0, 1, 3).reshape(L, B * H, D)
    want = oracle.rope(xt, offset + np.arange(L), dims, 1e6).reshape(L, B, H, D).transpose(1, 2, 0, 3)
    assert_close(got, want, F32_REL + (offset + L) * 2.0 ** -20, "rope")


@pytest.mark.parametrize("causal,Tq,Tk", [(True, 5, 5), (True, 3, 41), (False, 4, 19), (True, 1, 300)])
def test_attention_matches_oracle(graph, causal, Tq, Tk):
    rng = np.random.default_rng(Tq * 100 + Tk)
    B, Hq, Hkv, D = 2, 4, 2, 32
    q = rng.standard_normal((B, Hq, Tq, D)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, Tk, D)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, Tk, D)).astype(np.float32)
    scale = 1 / np.sqrt(D)
    y = graph.kernel(2, [graph.input(q), graph.input(k), graph.input(v)], ints=[int(causal)], floats=[scale])
    got = graph.finish(y, (B, Hq, Tq, D))
    if causal:
        # the oracle's paged attention: row b holds Tk tokens of context, its
        # Tq queries are the last Tq positions (bottom-right causal alignment)
        page = 16
        pages = (Tk + page - 1) // page
        kc = np.zeros((B * pages, Hkv, page, D), np.float32)
        vc = np.zeros_like(kc)
        for b in range(B):
            for j in range(Tk):
                kc[b * pages + j // page, :, j % page] = k[b, :, j]
                vc[b * pages + j // page, :, j % page] = v[b, :, j]
        bt = np.arange(B * pages, dtype=np.int32).reshape(B, pages)
        want = oracle.paged_attention(q.transpose(0, 2, 1, 3).reshape(B * Tq, Hq, D), kc, vc, bt,
                                      np.arange(B + 1, dtype=np.int32) * Tq, np.full(B, Tk, np.int32), scale)
        want = want.reshape(B, Tq, Hq, D).transpose(0, 2, 1, 3)
    else:
        rep = Hq // Hkv
        s = np.einsum("bhqd,bhkd->bhqk", q.astype(np.float64), np.repeat(k, rep, 1).astype(np.float64)) * scale
        p = np.exp(s - s.max(-1, keepdims=True))
        want = np.einsum("bhqk,bhkd->bhqd", p / p.sum(-1, keepdims=True), np.repeat(v, rep, 1).astype(np.float64))
    assert_close(got, want, F32_REL, "sdpa")


@pytest.mark.parametrize("seed", range(3))
def test_gated_delta_matches_oracle(graph, seed):
    rng = np.random.default_rng(10 + seed)
    B, T, Hk, Hv, Dk, Dv = 2, [1, 5, 16][seed], 2, 4, 32, 16
    q = rng.standard_normal((B, T, Hk, Dk)).astype(np.float32) * 0.2
    k = rng.standard_normal((B, T, Hk, Dk)).astype(np.float32) * 0.2
    v = rng.standard_normal((B, T, Hv, Dv)).astype(np.float32)
    decay = rng.uniform(0.5, 1.0, (B, T, Hv)).astype(np.float32)
    beta = rng.uniform(0, 1, (B, T, Hv)).astype(np.float32)
    state = rng.standard_normal((B, Hv, Dv, Dk)).astype(np.float32) * 0.1
    ids = [graph.input(a) for a in (q, k, v, decay, beta, state)]
    y, s = graph.kernel(3, ids, outputs=2)
    want_y, want_s = oracle.gated_delta(q, k, v, decay, beta, state)
    assert_close(graph.finish(y, (B, T, Hv, Dv)), want_y, F32_REL, "gated delta output")
    assert_close(graph.finish(s, (B, Hv, Dv, Dk)), want_s, F32_REL, "gated delta state")


def test_route_matches_oracle(graph):
    rng = np.random.default_rng(21)
    rows, E, top = 33, 256, 8
    lg = rng.standard_normal((rows, E)).astype(np.float32)
    lg[0, 10] = lg[0, 20] = 9.0  # a tie inside the top-k: both taken, lower index first
    idx, sc = graph.kernel(4, [graph.input(lg)], ints=[top], outputs=2)
    gi = graph.finish(idx, (rows, top), np.uint32).astype(np.int32)
    gs = graph.finish(sc, (rows, top))
    wi, ws = oracle.route_topk(lg, top)
    for r in range(rows):  # MLX's argpartition order is unspecified: compare as sets
        assert sorted(gi[r]) == sorted(wi[r]), f"row {r}"
        order = np.argsort(gi[r])
        assert_close(gs[r][order], ws[r][np.argsort(wi[r])], 1e-6, f"scores row {r}")
    assert list(gi[0][:2]) == [10, 20]


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("group", [32, 64, 128])
def test_gather_qmm_and_mix_match_oracle(graph, bits, group):
    rng = np.random.default_rng(bits * 1000 + group)
    rows, top, E, N, K = 5, 3, 7, 24, group * 3
    x = rng.standard_normal((rows, K)).astype(np.float32)
    w = rng.integers(0, 2**32, (E, N, K * bits // 32), dtype=np.uint64).astype(np.uint32)
    s = (rng.standard_normal((E, N, K // group)) * 0.05).astype(np.float32)
    b = (rng.standard_normal((E, N, K // group)) * 0.05).astype(np.float32)
    idx = rng.integers(0, E, (rows, top)).astype(np.uint32)
    scores = rng.uniform(0, 1, (rows, top)).astype(np.float32)
    ex = graph.kernel(5, [graph.input(x), graph.input(w), graph.input(s), graph.input(b), graph.input(idx)],
                      ints=[group, bits])
    y = graph.kernel(6, [ex, graph.input(scores)])
    want = oracle.gather_qmm(x, w, s, b, idx.astype(np.int32), group, bits)
    got = graph.finish(ex, (rows, top, N))
    assert_close(got, want, F32_REL, f"gather_qmm bits {bits} group {group}")
    assert_close(graph.finish(y, (rows, N)), oracle.mix(got, scores), F32_REL, "mix")


def test_malformed_descriptors_fail_without_a_node(graph):
    from hip_bridge import HipBridgeError

    x4 = graph.input(np.zeros((1, 1, 2, 4), np.float32))
    x2 = graph.input(np.zeros((2, 4), np.float32))
    u = graph.input(np.zeros((2, 2), np.uint32))
    n0 = graph.count
    cases = [
        (1, [x4], [3, 0], [1e4], "invalid RoPE"),      # odd dims
        (1, [x4], [8, 0], [1e4], "invalid RoPE"),      # dims beyond D
        (1, [x4], [2], [1e4], "integer missing"),
        (2, [x4, x2, x4], [1], [1.0], "attention dtype/rank"),
        (2, [x4, x4, x4], [1], [-1.0], "attention shape/scale"),
        (3, [x4, x4, x4, x2, x2, x4], [], [], "gated-delta"),
        (4, [x2], [5], [], "invalid expert top-k"),
        (4, [x4], [1], [], "invalid expert top-k"),
        (5, [x2, u, x2, x2, u], [32, 4], [], "expert dtype/rank"),
        (5, [x2, u, x2, x2, u], [32, 7], [], "unsupported expert quantization"),
        (6, [x2, x2], [], [], "expert mix"),
        (9, [x2], [], [], "unsupported native kernel"),
        (7, [u], [], [], "floating point"),
    ]
    for op, ins, ints, floats, msg in cases:
        with pytest.raises(HipBridgeError, match=msg):
            graph.kernel(op, ins, ints=ints, floats=floats)
        graph.count = n0
    # the graph still works and its next node id is unchanged
    y = graph.kernel(7, [x2])
    assert y == n0
    np.testing.assert_array_equal(graph.finish(y, (2, 4)), np.zeros((2, 4), np.float32))
