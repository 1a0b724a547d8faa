"""CPU pins for the whole-model oracle composition (oracle/model.py):

- the one-token decode restatement (DecodeStepCPU) from an empty context
  equals the full-sequence layer (HybridModel.layer) on that token, for both
  mixers (attention and Gated DeltaNet) and the MoE, and equals it again for a
  second token once the first token's K/V, state and conv history are in place;
- the MoE of the decode restatement (one gather_qmm per matrix) equals the
  per-token loop of HybridModel.moe;
- the mixer of the last m tokens alone equals the whole-sequence mixer's last
  m rows bit for bit;
- a shuffled expert order in the fused gate/up rows is detected (the
  8-gate/8-up tile interleave matters).
Weights are random checkpoint-layout tensors from the oracle quantiser."""
import numpy as np
import pytest

import oracle
from oracle.model import (A_LOG, CONV_W, DOWN, DT_BIAS, GATE_UP, G_NORM, IN_NORM, IN_PROJ, K_NORM, OUT_PROJ,
                          POST_NORM, Q_NORM, ROUTER, DecodeStepCPU, HybridModel, layer_tensor)

D = dict(hidden=256, layers=4, vocab=64, q_heads=8, kv_heads=1, head_dim=256, key_heads=2, value_heads=4,
         key_dim=128, value_dim=128, conv=4, interval=4, experts=8, top=2, intermediate=128, rope_dims=64,
         epsilon=1e-6, theta=1e7)


def r16(n):
    return (n + 15) // 16 * 16


def shapes(d):
    H, E, I = d["hidden"], d["experts"], d["intermediate"]
    hq, hkv, Dh = d["q_heads"], d["kv_heads"], d["head_dim"]
    hk, hv, dk, dv = d["key_heads"], d["value_heads"], d["key_dim"], d["value_dim"]
    C = 2 * hk * dk + hv * dv

    def shape(tid):
        if tid < 16:
            return {0: (d["vocab"], H, 1), 1: (H, 0, 0), 2: (d["vocab"], H, 1)}[tid]
        layer, slot = divmod(tid - 16, 16)
        attn = (layer + 1) % d["interval"] == 0
        return {IN_NORM: (H, 0, 0), POST_NORM: (H, 0, 0),
                IN_PROJ: ((hq * 2 * Dh + 2 * hkv * Dh) if attn else r16(C + hv * dv + 2 * hv), H, 1),
                OUT_PROJ: (H, hq * Dh if attn else hv * dv, 1), CONV_W: (C * d["conv"], 0, 0), A_LOG: (hv, 0, 0),
                DT_BIAS: (hv, 0, 0), G_NORM: (dv, 0, 0), Q_NORM: (Dh, 0, 0), K_NORM: (Dh, 0, 0),
                ROUTER: (r16(E + 1), H, 1), GATE_UP: ((E + 1) * 2 * I, H, 1), DOWN: ((E + 1) * H, I, 1)}[slot]
    return shape


@pytest.fixture(scope="module")
def model():
    shape = shapes(D)
    cache = {}

    def tensors(tid):
        if tid not in cache:
            rng = np.random.default_rng(1000 + tid)
            n, k, q = shape(tid)
            if q:
                p, s, b = oracle.quantize_affine(rng.standard_normal((n, k)).astype(np.float32) * 0.05)
                cache[tid] = (p, oracle.to_bf16_bits(s), oracle.to_bf16_bits(b))
            elif (tid - 16) % 16 == A_LOG:
                cache[tid] = rng.uniform(0, 1, n).astype(np.float32)
            elif (tid - 16) % 16 == DT_BIAS:
                cache[tid] = np.zeros(n, np.float32)
            elif (tid - 16) % 16 == CONV_W:
                cache[tid] = (0.3 * rng.standard_normal(n)).astype(np.float32)
            else:
                cache[tid] = (1 + 0.05 * rng.standard_normal(n)).astype(np.float32)
        return cache[tid]

    return HybridModel(dict(D), tensors)


@pytest.mark.parametrize("layer", [0, 3])  # a DeltaNet layer and the attention layer
def test_decode_restatement_equals_sequence_layer(model, layer):
    rng = np.random.default_rng(layer)
    x = rng.standard_normal((2, D["hidden"])).astype(np.float32)  # token 0 and token 1 of one row
    want = model.layer(layer, x)
    step = DecodeStepCPU(model, [layer], [0], zero=True)
    got0 = step.layer(layer, x[:1])
    np.testing.assert_allclose(got0, want[:1], rtol=1e-5, atol=1e-5)
    step.ctx = step.ctx + 1  # the first token is now part of the context
    got1 = step.layer(layer, x[1:])
    np.testing.assert_allclose(got1, want[1:], rtol=1e-4, atol=1e-4)


def test_gathered_moe_equals_token_loop(model):
    rng = np.random.default_rng(7)
    h = oracle.bf16_round(rng.standard_normal((5, D["hidden"])).astype(np.float32))
    step = DecodeStepCPU(model, [0], [0] * 5, zero=True)
    np.testing.assert_allclose(step.moe(h, 0), model.moe(h, 0), rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(model.moe_per_token(h, 0), model.moe(h, 0), rtol=1e-6, atol=1e-6)


def test_near_tie_alternative_swaps_the_boundary_expert(model):
    """With a window wider than every gap, each token gets an alternative whose
    routed set differs from the primary one in exactly the boundary expert:
    recomputing the MoE with the router's top-th logit lowered below the
    (top+1)-th must reproduce it."""
    rng = np.random.default_rng(9)
    h = oracle.bf16_round(rng.standard_normal((4, D["hidden"])).astype(np.float32))
    model.tie_window = np.inf
    try:
        model.moe(h, 2)
        alts = dict(model.moe_alternatives)
    finally:
        model.tie_window = 0.0
    assert sorted(alts) == [0, 1, 2, 3]
    logits = model.w(layer_tensor(2, ROUTER))(h).astype(np.float32)
    E, top = D["experts"], D["top"]
    for t, alt in alts.items():
        idx, _ = oracle.route_topk(np.ascontiguousarray(logits[t:t + 1, :E]), top + 1)
        lowered = logits[t:t + 1, :E].copy()
        lowered[0, idx[0, top - 1]] = lowered[0, idx[0, top]] - 1.0  # force the swap
        i2, w2 = oracle.route_topk(np.ascontiguousarray(lowered), top)
        # weights of the swapped set come from the original logits
        sel = logits[t, i2[0]].astype(np.float64)
        w2 = np.exp(sel - sel.max()) / np.exp(sel - sel.max()).sum()
        want = model._experts(h[t:t + 1], 2, i2, w2[None], logits[t:t + 1, E])
        np.testing.assert_allclose(alt, want[0], rtol=1e-12, atol=1e-12)
        assert not np.allclose(alt, model.moe(h[t:t + 1], 2)[0], rtol=1e-3, atol=1e-3)


def test_gate_up_interleave_is_load_bearing(model):
    rng = np.random.default_rng(8)
    h = oracle.bf16_round(rng.standard_normal((3, D["hidden"])).astype(np.float32))
    base = model.moe(h, 1)
    gu = model.w(layer_tensor(1, GATE_UP))
    saved = gu.w.copy()
    rows = np.arange(gu.w.shape[0]).reshape(-1, 16)
    gu.w[:] = saved[np.concatenate([rows[:, 8:], rows[:, :8]], axis=1).reshape(-1)]  # swap gate and up halves
    try:
        assert not np.allclose(model.moe(h, 1), base, rtol=1e-3, atol=1e-3)
    finally:
        gu.w[:] = saved


@pytest.mark.parametrize("layer", [0, 3])  # a DeltaNet layer and the attention layer
def test_mixer_of_the_last_tokens_equals_the_whole_sequence(model, layer):
    # layer_mixer(..., last=m) forms q, gate and the output projection for the
    # last m rows only; every projected row is computed on its own, so its rows
    # are bit-identical to those of the whole-sequence form
    rng = np.random.default_rng(10 + layer)
    x = rng.standard_normal((37, D["hidden"])).astype(np.float32)
    full = model.layer_mixer(layer, x)
    for m in (1, 4, 37):
        assert np.array_equal(model.layer_mixer(layer, x, last=m), full[-m:]), m
