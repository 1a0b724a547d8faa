"""Known-answer tests that pin the C oracle to the reference's own test vectors.

Every case below is transcribed from a reference test (cited file:line) and is
checked against the closed form that test states, never against the oracle's
own formula re-typed.
"""
import math

import numpy as np
import pytest

import oracle
from oracle import OracleError


def set_value(packed, row, width, col, bits, value):
    """Bit-at-a-time packing, independent of the oracle's word extraction
    (judges/projection_reference.cpp:7-13)."""
    row_words = width * bits // 32
    for bit in range(bits):
        if value & (1 << bit):
            pos = col * bits + bit
            packed[row * row_words + pos // 32] |= np.uint32(1 << (pos % 32))


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("group", [32, 64, 128])
@pytest.mark.parametrize("rows", [1, 8])
def test_projection_all_widths(orc, bits, group, rows):
    # judges/projection_reference.cpp:16-27
    width, outputs = group * 2, 8
    x = np.array([((i % 19) - 9) * 0.125 for i in range(rows * width)], np.float32)
    scale = np.array([(-0.25 if i % 2 else 0.125) for i in range(outputs * 2)], np.float32)
    bias = np.array([float((i % 7) - 3) * 0.5 for i in range(outputs * 2)], np.float32)
    packed = np.zeros(outputs * width * bits // 32, np.uint32)
    expected = np.zeros(rows * outputs)
    expected_w = np.zeros(outputs * width)
    for out in range(outputs):
        for col in range(width):
            q = (col * 17 + out * 3) & ((1 << bits) - 1)
            set_value(packed, out, width, col, bits, q)
            w = float(scale[out * 2 + col // group]) * q + float(bias[out * 2 + col // group])
            expected_w[out * width + col] = w
            for r in range(rows):
                expected[r * outputs + out] += float(x[r * width + col]) * w
    y = orc.qmm(x.reshape(rows, width), packed.reshape(outputs, -1), scale.reshape(outputs, 2),
                bias.reshape(outputs, 2), group, bits)
    assert np.array_equal(y.reshape(-1), expected)
    d = orc.dequant(packed.reshape(outputs, -1), scale.reshape(outputs, 2), bias.reshape(outputs, 2), width,
                    group, bits)
    assert np.array_equal(d.reshape(-1), expected_w)


def test_projection_full_tile_3bit(orc):
    # judges/projection_reference.cpp:29-34: every output equals 3584
    width, outputs, rows = 1024, 256, 8
    packed = np.zeros(outputs * width * 3 // 32, np.uint32)
    for out in range(outputs):
        for col in range(width):
            set_value(packed, out, width, col, 3, (col + out) % 8)
    y = orc.qmm(np.ones((rows, width), np.float32), packed.reshape(outputs, -1), np.ones((outputs, 8), np.float32),
                np.zeros((outputs, 8), np.float32), 128, 3)
    assert np.all(y == 3584)


def test_literal_3bit_stream(orc):
    # judges/projection_reference.cpp:35-37: 0x00fac688 holds codes 0..7
    literal = np.array([[0x00FAC688, 0, 0]], np.uint32)
    for col in range(8):
        x = np.zeros((1, 32), np.float32)
        x[0, col] = 1
        y = orc.qmm(x, literal, np.ones((1, 1), np.float32), np.zeros((1, 1), np.float32), 32, 3)
        assert y[0, 0] == col


def test_projection_rejections(orc):
    # judges/projection_reference.cpp:38-51 (geometry the C oracle also rejects)
    L = orc.lib()
    x = np.ones(32, np.float32)
    packed = np.zeros(4, np.uint32)
    one, zero = np.ones(1, np.float32), np.zeros(1, np.float32)
    y = np.zeros(64, np.float64)
    assert L.orc_qmm(x, 0, packed, one, zero, 1, 32, 32, 4, y, 1) == -1
    assert L.orc_qmm(x, 1, packed, one, zero, 1, 32, 0, 4, y, 1) == -1
    assert L.orc_qmm(x, 1, packed, one, zero, 1, 32, 32, 7, y, 1) == -1
    assert L.orc_qmm(x, 1, packed, one, zero, 1, 31, 32, 4, y, 1) == -1
    assert L.orc_qmm(x, 1, packed, np.array([np.nan], np.float32), zero, 1, 32, 32, 4, y, 1) == -1
    bad = x.copy()
    bad[0] = np.inf
    assert L.orc_qmm(bad, 1, packed, one, zero, 1, 32, 32, 4, y, 1) == -1
    assert L.orc_qmm(x, 1, packed, one, np.array([np.inf], np.float32), 1, 32, 32, 4, y, 1) == -1


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("group", [32, 64, 128])
def test_all_ones_packing_oracle(orc, bits, group):
    # tests/native_execution.rs:103-128: u32::MAX codes, s=0.125, b=-0.25
    x = np.ones((2, group), np.float32)
    w = np.full((3, group * bits // 32), 0xFFFFFFFF, np.uint32)
    y = orc.qmm(x, w, np.full((3, 1), 0.125, np.float32), np.full((3, 1), -0.25, np.float32), group, bits)
    assert np.allclose(y, group * (((1 << bits) - 1) * 0.125 - 0.25), rtol=0, atol=1e-12)


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("group", [32, 64, 128])
def test_mixed_bitstream(orc, bits, group):
    # tests/native_execution.rs:286-322: one continuous LSB-first stream over 3 rows
    k = group * 2
    packed = np.zeros(3 * k * bits // 32, np.uint64)
    x = np.array([((j % 11) - 5) / 8 for j in range(2 * k)], np.float32)
    expected = np.zeros(6)
    for row in range(3):
        for j in range(k):
            q = (j * 7 + row * 3) % (1 << bits)
            bit = (row * k + j) * bits
            word, shift = bit // 32, bit % 32
            packed[word] |= (q << shift) & 0xFFFFFFFF
            if shift + bits > 32:
                packed[word + 1] |= q >> (32 - shift)
            for b in range(2):
                expected[b * 3 + row] += float(x[b * k + j]) * (q * 0.125 - 0.25)
    y = orc.qmm(x.reshape(2, k), packed.astype(np.uint32).reshape(3, -1), np.full((3, 2), 0.125, np.float32),
                np.full((3, 2), -0.25, np.float32), group, bits)
    assert np.allclose(y.reshape(-1), expected, rtol=1e-12, atol=1e-12)


def test_operator_closed_forms(orc):
    # judges/operator_reference.cpp:7-10
    r = orc.rms(np.array([[3, 4]], np.float32), np.array([2, 0.5], np.float32), eps=1.0)
    assert r[0, 0] == pytest.approx(6 / math.sqrt(13.5), rel=1e-11)
    assert r[0, 1] == pytest.approx(2 / math.sqrt(13.5), rel=1e-11)
    s = orc.silu(np.array([-1000, 0, 1000], np.float32))
    assert abs(s[0]) < 1e-11 and s[1] == 0 and s[2] == pytest.approx(1000, rel=1e-11)
    y = orc.rope(np.array([[[1, 2, 9, 10]]], np.float32), [1], rotary=2, theta=10000)[0, 0]
    assert y[0] == pytest.approx(math.cos(1) - 2 * math.sin(1), abs=1e-11)
    assert y[1] == pytest.approx(math.sin(1) + 2 * math.cos(1), abs=1e-11)
    assert y[2] == 9 and y[3] == 10
    y = orc.rope(np.array([[[1, 2, 3, 4]]], np.float32), [3], rotary=4, theta=10000)[0, 0]
    assert y[0] == pytest.approx(math.cos(3) - 3 * math.sin(3), abs=1e-11)
    assert y[1] == pytest.approx(2 * math.cos(0.03) - 4 * math.sin(0.03), abs=1e-11)
    assert y[2] == pytest.approx(math.sin(3) + 3 * math.cos(3), abs=1e-11)
    assert y[3] == pytest.approx(2 * math.sin(0.03) + 4 * math.cos(0.03), abs=1e-11)
    # tests/native_execution.rs:141-149: rope((1,0), offset 1, dims 2) = (cos 1, sin 1)
    y = orc.rope(np.array([[[1, 0]]], np.float32), [1], rotary=2, theta=10000)[0, 0]
    assert y[0] == pytest.approx(math.cos(1), abs=1e-7) and y[1] == pytest.approx(math.sin(1), abs=1e-7)


def test_operator_rejections(orc):
    # judges/operator_reference.cpp:21-24
    with pytest.raises(OracleError):
        orc.rms(np.array([[np.nan]], np.float32))
    with pytest.raises(OracleError):
        orc.rms(np.array([[1.0]], np.float32), eps=0.0)
    with pytest.raises(OracleError):
        orc.silu(np.array([np.inf], np.float32))
    with pytest.raises(OracleError):
        orc.rope(np.array([[[1, 2]]], np.float32), [0], rotary=1, theta=10000)


def test_gdn_shared_key_head(orc):
    # judges/operator_reference.cpp:11-16: two value heads share one key head, decay=beta=1/2
    qkv = np.array([[1, 1, 2, 3]], np.float32)
    cw = np.array([0, 1, 0, 1, 0, 1, 0, 1], np.float32).reshape(4, 2)
    act, hist, out, st = orc.gdn(qkv, np.zeros((1, 4), np.float32), cw, np.zeros((1, 2), np.float32),
                                 np.zeros((1, 2), np.float32), np.zeros(2, np.float32), np.zeros(2, np.float32),
                                 np.array([2, 4], np.float32).reshape(2, 1, 1), 1, 2, 1, 1)
    q = 1 / (1 + math.exp(-1.0))
    q /= math.sqrt(q * q + 1e-6)
    for h in range(2):
        v = (h + 2.0) / (1 + math.exp(-(h + 2.0)))
        old = h + 1.0
        expected = old + 0.5 * (v - old * q) * q
        assert st.reshape(-1)[h] == pytest.approx(expected, rel=1e-11)
        assert out.reshape(-1)[h] == pytest.approx(expected * q, rel=1e-11)
    assert np.array_equal(hist.reshape(-1), qkv.reshape(-1))


def test_gdn_conv_taps(orc):
    # judges/operator_reference.cpp:17-19: history and both taps reach each channel
    qkv = np.array([[1, 1, 2, 3]], np.float32)
    cw = np.array([0.25, 0.75] * 4, np.float32).reshape(4, 2)
    act, _, _, _ = orc.gdn(qkv, np.array([[4, 5, 6, 7]], np.float32), cw, np.zeros((1, 2), np.float32),
                           np.zeros((1, 2), np.float32), np.zeros(2, np.float32), np.zeros(2, np.float32),
                           np.zeros((2, 1, 1), np.float32), 1, 2, 1, 1)
    for i in range(4):
        x = 0.25 * (i + 4) + 0.75 * float(qkv[0, i])
        assert act[0, i] == pytest.approx(x / (1 + math.exp(-x)), rel=1e-11)


def test_gated_delta_multi_output(orc):
    # tests/native_execution.rs:153-182
    q = np.array([0.5, 0, 0, 0.5], np.float32).reshape(1, 2, 1, 2)
    k = np.array([1, 0, 0, 1], np.float32).reshape(1, 2, 1, 2)
    v = np.array([2, 4, 6, 8], np.float32).reshape(1, 2, 2, 1)
    half = np.full((1, 2, 2), 0.5, np.float32)
    y, s = orc.gated_delta(q, k, v, half, half, np.zeros((1, 2, 1, 2), np.float32))
    assert np.allclose(y.reshape(-1), [0.5, 1, 1.5, 2], atol=1e-12)
    assert np.allclose(s.reshape(-1), [0.5, 3, 1, 4], atol=1e-12)


def test_recurrent_bank_rows(orc):
    # tests/native_execution.rs:210-285: two one-dimensional rows evolve independently
    ones = np.ones((2, 1, 1, 1), np.float32)
    y, s = orc.gated_delta(ones, ones, np.array([4, 2], np.float32).reshape(2, 1, 1, 1),
                           np.ones((2, 1, 1), np.float32), np.full((2, 1, 1), 0.5, np.float32),
                           np.zeros((2, 1, 1, 1), np.float32))
    assert np.allclose(y.reshape(-1), [2, 1])
    # reorder: row 10 then row 20
    state = np.array([s.reshape(-1)[1], s.reshape(-1)[0]], np.float32).reshape(2, 1, 1, 1)
    y, s = orc.gated_delta(ones, ones, np.array([3, 8], np.float32).reshape(2, 1, 1, 1),
                           np.full((2, 1, 1), 0.5, np.float32), np.full((2, 1, 1), 0.5, np.float32), state)
    assert np.allclose(y.reshape(-1), [1.75, 4.5])


def test_routing_weights(orc):
    # judges/operator_reference.cpp:25-26
    idx, w = orc.route_topk(np.array([[0, 1, 2]], np.float32), 2)
    assert list(idx[0]) == [2, 1]
    e = math.e
    assert w[0, 0] == pytest.approx(e / (e + 1), rel=1e-11) and w[0, 1] == pytest.approx(1 / (e + 1), rel=1e-11)
    idx, w = orc.route_topk(np.array([[1, 1, 1]], np.float32), 2)
    assert list(idx[0]) == [0, 1]  # deterministic tie: lower index first
    assert np.allclose(w, 0.5)


def test_route_gather_mix(orc):
    # tests/native_execution.rs:183-209: mix = 32 (1 + 2e) / (1 + e)
    idx, scores = orc.route_topk(np.array([[-10, 0, 1]], np.float32), 2)
    x = np.ones((1, 32), np.float32)
    w = np.zeros((3, 1, 4), np.uint32)
    s = np.ones((3, 1, 1), np.float32)
    b = np.array([0, 1, 2], np.float32).reshape(3, 1, 1)
    experts = orc.gather_qmm(x, w, s, b, idx, group=32, bits=4)
    y = orc.mix(experts.astype(np.float32), scores.astype(np.float32))
    e = math.e
    assert y[0, 0] == pytest.approx(32 * (1 + 2 * e) / (1 + e), rel=1e-6)
    with pytest.raises(OracleError):
        orc.gather_qmm(x, w, s, b, np.array([[3]], np.int32), group=32, bits=4)


def _contiguous_paged(k, v, page=16):
    """Place contiguous [hkv][n][dim] keys/values into one row of pages."""
    hkv, n, dim = k.shape
    pages = (n + page - 1) // page
    kc = np.zeros((pages, hkv, page, dim), np.float32)
    vc = np.zeros_like(kc)
    for j in range(n):
        kc[j // page, :, j % page] = k[:, j]
        vc[j // page, :, j % page] = v[:, j]
    return kc, vc, np.arange(pages, dtype=np.int32).reshape(1, pages)


def test_attention_causal_means(orc):
    # tests/native_execution.rs:129-140: q=0, k=0, v=[2,4,6,8] causal -> [2,4,4,6] per head
    k = np.zeros((1, 2, 2), np.float32)
    v = np.array([2, 4, 6, 8], np.float32).reshape(1, 2, 2)
    kc, vc, bt = _contiguous_paged(k, v)
    y = orc.paged_attention(np.zeros((2, 2, 2), np.float32), kc, vc, bt, [0, 2], [2], 1.0)
    # y is [tokens][heads][dim]; reference layout is [heads][tokens][dim]
    assert np.allclose(y.transpose(1, 0, 2).reshape(-1), [2, 4, 4, 6, 2, 4, 4, 6])


def test_attention_causal_isolation(orc):
    # judges/metal_reference_attention.cpp:33-36: row 0 sees only 1, row 1 sees mean 4
    k = np.zeros((2, 2, 256), np.float32)
    v = np.concatenate([np.ones((2, 1, 256), np.float32), np.full((2, 1, 256), 7, np.float32)], 1)
    kc, vc, bt = _contiguous_paged(k, v)
    y = orc.paged_attention(np.zeros((2, 16, 256), np.float32), kc, vc, bt, [0, 2], [2], 1 / 16)
    assert np.all(y[0] == 1) and np.all(y[1] == 4)


def test_total_order_argmax(orc):
    # judges/device_selection.cpp:7-11
    f = np.float32(np.finfo(np.float32).smallest_subnormal)
    rows = np.array([[-0.0, 0.0, -f, -0.0], [0.0, -0.0, -f, -f], [-2, -1, -1, -3], [f, 0.0, f, -f]], np.float32)
    assert [orc.winner(r)[0] for r in rows] == [1, 0, 1, 0]
    # src/serving/native_speculative.rs:349, 408-415
    assert orc.winner(np.array([-0.0, 0.0, -1.0], np.float32))[0] == 1
    tok, margin = orc.winner(np.array([0.5, 3.25, 1.75, -2.0], np.float32))
    assert tok == 1 and abs(margin - 1.5) < 1e-6
    tok, margin = orc.winner(np.array([2.0, 4.0, 4.0], np.float32))
    assert tok == 1 and margin == 0.0


def test_selection_gate_vectors(orc):
    # judges/native_cpp_selection_gate.cpp:13-21
    logits = np.full(248320, -1, np.float32)
    logits[17] = logits[23] = 2
    assert orc.winner(logits)[0] == 17
    logits[:] = -1
    logits[0], logits[1] = -0.0, 0.0
    assert orc.winner(logits)[0] == 1
    logits[0] = 0.0
    assert orc.winner(logits)[0] == 0
    for index in (0, logits.size - 1):
        for value in (np.nan, np.inf, -np.inf):
            bad = logits.copy()
            bad[index] = value
            with pytest.raises(OracleError):
                orc.winner(bad)
    with pytest.raises(OracleError):
        orc.winner(np.zeros(0, np.float32))


def test_selection_tie_break_pressure(orc):
    # src/serving/native_speculative.rs:357-373 against choices::select (first strict max)
    for n in range(1, 513):
        values = np.array([((i * 17 + n * 31) % 23) - 11.0 for i in range(n)], np.float32)
        best = 0
        for i in range(1, n):
            if values[i] > values[best]:
                best = i
        assert orc.winner(values)[0] == best


def row(token):
    r = np.full(12, -1.0, np.float32)
    r[token] = 1.0
    return r


def test_plan_every_boundary():
    # src/serving/native_speculative.rs:319-355
    for n in range(1, 9):
        for accepted in range(n + 1):
            draft = [1] * n
            if accepted < n:
                draft[accepted] = 2
            rows = [row(1)] * n
            emitted, acc, term = oracle.plan(row(1), draft, np.stack(rows), [11], 9)
            assert acc == accepted and emitted == [1] * (accepted + 1) and not term
            for stop in range(min(accepted, n - 1) + 1):
                rs = list(rows)
                initial = row(1)
                if stop == 0:
                    initial = row(11)
                else:
                    rs[stop - 1] = row(11)
                emitted, acc, term = oracle.plan(initial, draft, np.stack(rs), [11], 9)
                assert term and len(emitted) == stop + 1 and emitted[stop] == 11
        emitted, _, _ = oracle.plan(row(1), [1] * n, np.stack([row(1)] * n), [], n)
        assert len(emitted) == n
    assert oracle.plan(row(1), [], None, [], 1)[0] == [1]
    emitted, acc, term = oracle.plan(row(11), [11, 2], np.stack([row(1), row(1)]), [11], 4)
    assert term and acc == 1 and emitted == [11]


def test_plan_malformed_rejected():
    # src/serving/native_speculative.rs:374-385
    cases = [
        (row(1), [2], np.full((1, 12), np.nan, np.float32), [], 8),
        (row(1), [2], np.full((1, 12), np.inf, np.float32), [], 8),
        (row(1), [12], np.stack([row(1)]), [], 8),
        (row(1), [], None, [12], 8),
        (np.zeros(0, np.float32), [], None, [], 8),
        (row(1), [1] * 9, np.stack([row(1)] * 9), [], 10),
        (row(1), [1], np.stack([row(1)]), [], 0),
    ]
    for args in cases:
        with pytest.raises(OracleError):
            oracle.plan(*args)
    with pytest.raises(OracleError):
        oracle.plan(row(1), [2], np.zeros((1, 11), np.float32), [], 8)  # wrong vocabulary
    with pytest.raises(OracleError):
        oracle.plan(row(1), [1], np.zeros((0, 12), np.float32), [], 8)  # missing rows
