"""Parity of the Gated DeltaNet kernels (hb_gdn_prep + hb_gdn_recurrence) with
the CPU oracle (oracle.gdn, pinned to native/operator_reference.h:20-44).
Configuration-3 shapes: 16 key heads x 128, 32 value heads x 128, fp32 state
~N(0, 0.01), conv width 4, A_log ~U[0,1], a, b ~N(0,1)."""
import numpy as np
import pytest

import oracle
from numerics import assert_bf16_close, assert_state_close

pytestmark = pytest.mark.gpu

HK, HV, DK, DV, CONV = 16, 32, 128, 128, 4
C = 2 * HK * DK + HV * DV


@pytest.fixture(scope="module")
def hb(bridge):
    import hip_bridge.quant  # noqa: F401

    return bridge


class Layer:
    """Seeded DeltaNet layer parameters and per-row state on the device."""

    def __init__(self, hb, rows, max_tokens, seed):
        from hip_bridge import DeviceBuffer

        self.hb, self.rows, self.maxt = hb, rows, max_tokens
        rng = np.random.default_rng(seed)
        self.rng = rng
        self.conv_w = (rng.standard_normal((C, CONV)) * 0.5).astype(np.float32)
        self.alog = rng.uniform(0, 1, HV).astype(np.float32)
        self.dt = np.zeros(HV, np.float32)
        self.norm_w = (1 + 0.1 * rng.standard_normal(DV)).astype(np.float32)
        self.state0 = (rng.standard_normal((rows, HV, DV, DK)) * 0.01).astype(np.float32)
        hist = hb.quant.bf16_bits(rng.standard_normal((rows, CONV - 1, C), dtype=np.float32))
        win = np.zeros((rows, CONV - 1 + max_tokens, C), np.uint16)
        win[:, :CONV - 1] = hist
        self.hist0 = hb.quant.bf16_value(hist)
        self.d = dict(conv_w=DeviceBuffer.from_array(self.conv_w), alog=DeviceBuffer.from_array(self.alog),
                      dt=DeviceBuffer.from_array(self.dt), norm=DeviceBuffer.from_array(self.norm_w),
                      state=DeviceBuffer.from_array(np.ascontiguousarray(self.state0.transpose(0, 1, 3, 2))),
                      win=DeviceBuffer.from_array(win),
                      lk=DeviceBuffer(rows * 4 * HV * DK * 4), ld=DeviceBuffer(rows * 4 * HV * DV * 4),
                      lg=DeviceBuffer(rows * 4 * HV * 4))

    def inputs(self, row_tokens):
        hb, rng = self.hb, self.rng
        T = int(sum(row_tokens))
        qkv = hb.quant.bf16_bits(rng.standard_normal((T, C), dtype=np.float32))
        ab = hb.quant.bf16_bits(rng.standard_normal((T, 2 * HV), dtype=np.float32))
        z = hb.quant.bf16_bits(rng.standard_normal((T, HV * DV), dtype=np.float32))
        return qkv, ab, z

    def step(self, row_tokens, qkv, ab, z, hist_off, log_count, speculative):
        from hip_bridge import DeviceBuffer

        hb = self.hb
        T = int(sum(row_tokens))
        cu = np.concatenate([[0], np.cumsum(row_tokens)]).astype(np.int32)
        d = dict(qkv=DeviceBuffer.from_array(qkv), ab=DeviceBuffer.from_array(ab), z=DeviceBuffer.from_array(z),
                 cu=DeviceBuffer.from_array(cu), hoff=DeviceBuffer.from_array(np.asarray(hist_off, np.int32)),
                 lcnt=DeviceBuffer.from_array(np.asarray(log_count, np.int32)),
                 q=DeviceBuffer(T * HK * DK * 4), k=DeviceBuffer(T * HK * DK * 4), v=DeviceBuffer(T * HV * DV * 4),
                 g=DeviceBuffer(T * HV * 4), b=DeviceBuffer(T * HV * 4), o=DeviceBuffer(T * HV * DV * 4),
                 y=DeviceBuffer(T * HV * DV * 2))
        ab_ptr = d["ab"].ptr
        hb.call("hb_gdn_prep", d["qkv"], C, d["ab"], hb._p(ab_ptr + 2 * HV), 2 * HV, self.d["conv_w"],
                self.d["alog"], self.d["dt"], self.d["win"], d["hoff"], None, None, d["cu"], self.rows, HK, HV, DK,
                DV, CONV, self.maxt, d["q"], d["k"], d["v"], d["g"], d["b"], None)
        hb.call("hb_gdn_recurrence", d["q"], d["k"], d["v"], d["g"], d["b"], d["cu"], self.rows, HK, HV, DK, DV,
                self.d["state"], None, None, self.d["lk"], self.d["ld"], self.d["lg"], d["lcnt"], 4, speculative,
                d["o"], d["z"], HV * DV, self.d["norm"], d["y"], None)
        hb.synchronize()
        return (d["o"].download(np.float32, (T, HV, DV)), hb.quant.bf16_value(d["y"].download(np.uint16, (T, HV * DV))))

    def state(self):
        # the device keeps each head's state key-major ([key][value])
        st = self.d["state"].download(np.float32, (self.rows, HV, DK, DV))
        return np.ascontiguousarray(st.transpose(0, 1, 3, 2))

    def window(self):
        return self.hb.quant.bf16_value(self.d["win"].download(np.uint16, (self.rows, CONV - 1 + self.maxt, C)))


def oracle_row(layer, r, qkv, ab, hist, state):
    a = ab[:, :HV].copy()
    b = ab[:, HV:].copy()
    return oracle.gdn(qkv, hist, layer.conv_w, a, b, layer.alog, layer.dt, state, HK, HV, DK, DV)


def test_decode_step_config3(hb):
    rows = 32
    L = Layer(hb, rows, 4, 31)
    row_tokens = [1] * rows
    qkv, ab, z = L.inputs(row_tokens)
    print("case: gdn decode 32 rows T=1", flush=True)
    o, y = L.step(row_tokens, qkv, ab, z, [0] * rows, [0] * rows, 0)
    st = L.state()
    qv, abv, zv = (hb.quant.bf16_value(t) for t in (qkv, ab, z))
    for r in range(rows):
        act, hist, out, s = oracle_row(L, r, qv[r:r + 1], abv[r:r + 1], L.hist0[r], L.state0[r])
        assert_state_close(st[r], s, f"state row {r}")
        assert_state_close(o[r], out[0], f"output row {r}")
        ref_y = oracle.rms(out.astype(np.float32).reshape(HV, DV), L.norm_w) * oracle.silu(
            zv[r].reshape(HV, DV))
        assert_bf16_close(y[r].reshape(HV, DV), ref_y, f"gated norm row {r}")


def test_prefill_chunks_ragged(hb):
    rows = 6
    L = Layer(hb, rows, 64, 32)
    row_tokens = [64, 1, 17, 33, 64, 5]
    qkv, ab, z = L.inputs(row_tokens)
    print("case: gdn prefill chunks", flush=True)
    o, _ = L.step(row_tokens, qkv, ab, z, [0] * rows, [0] * rows, 0)
    st = L.state()
    win = L.window()
    qv, abv = hb.quant.bf16_value(qkv), hb.quant.bf16_value(ab)
    cu = np.concatenate([[0], np.cumsum(row_tokens)])
    for r in range(rows):
        sl = slice(cu[r], cu[r + 1])
        act, hist, out, s = oracle_row(L, r, qv[sl], abv[sl], L.hist0[r], L.state0[r])
        assert_state_close(st[r], s, f"state row {r}")
        assert_state_close(o[sl], out, f"outputs row {r}")
        # window = [history | new rows]; the last conv-1 rows equal the oracle's rolled history
        n = row_tokens[r]
        assert np.array_equal(win[r, n:n + CONV - 1], hist.astype(np.float32)), f"conv history row {r}"


def test_speculative_log_replay(hb):
    rows = 8
    rng = np.random.default_rng(5)
    L = Layer(hb, rows, 4, 33)
    t4 = [4] * rows
    qkv1, ab1, z1 = L.inputs(t4)
    print("case: gdn speculative verify + replay", flush=True)
    o1, _ = L.step(t4, qkv1, ab1, z1, [0] * rows, [0] * rows, 1)
    assert np.array_equal(L.state(), L.state0), "speculative step must write back the committed state"
    accepted = rng.integers(1, 5, size=rows).astype(np.int32)
    t1 = [1] * rows
    qkv2, ab2, z2 = L.inputs(t1)
    o2, _ = L.step(t1, qkv2, ab2, z2, accepted, accepted, 0)
    st = L.state()
    q1, a1, q2, a2 = (hb.quant.bf16_value(t) for t in (qkv1, ab1, qkv2, ab2))
    for r in range(rows):
        n = int(accepted[r])
        _, _, out_v, _ = oracle_row(L, r, q1[4 * r:4 * r + 4], a1[4 * r:4 * r + 4], L.hist0[r], L.state0[r])
        assert_state_close(o1[4 * r:4 * r + 4], out_v, f"verify outputs row {r}")
        seq_q = np.concatenate([q1[4 * r:4 * r + n], q2[r:r + 1]])
        seq_a = np.concatenate([a1[4 * r:4 * r + n], a2[r:r + 1]])
        _, _, out, s = oracle_row(L, r, seq_q, seq_a, L.hist0[r], L.state0[r])
        assert_state_close(st[r], s, f"state after replay row {r} (accepted {n})")
        assert_state_close(o2[r], out[-1], f"output after replay row {r}")

    # the replayed state is bit-identical to stepping the accepted tokens directly
    M = Layer(hb, rows, 4, 33)  # same seed: same parameters, state and history
    qkv_acc = np.concatenate([qkv1[4 * r:4 * r + int(accepted[r])] for r in range(rows)])
    ab_acc = np.concatenate([ab1[4 * r:4 * r + int(accepted[r])] for r in range(rows)])
    z_acc = np.concatenate([z1[4 * r:4 * r + int(accepted[r])] for r in range(rows)])
    M.step(list(accepted), qkv_acc, ab_acc, z_acc, [0] * rows, [0] * rows, 0)
    M.step(t1, qkv2, ab2, z2, accepted, [0] * rows, 0)
    assert np.array_equal(M.state(), st)
