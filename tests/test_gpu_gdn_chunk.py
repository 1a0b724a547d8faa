"""Chunked DeltaNet prefill (hb_gdn_chunked: 64-token chunks as matrix
products on MFMA) against the CPU oracle (oracle.gdn, pinned to
native/operator_reference.h:20-44) on ragged rows, and against the
token-serial kernel (hb_gdn_recurrence) across many chunks at the prefill
workload: 32 prompts of U[64, 2048] tokens, 16 key heads / 32 value heads x
128, fp32 state ~N(0, 0.01). The fp32 state and the outputs are held to the
state tolerance (1e-3); the gated norm to the bf16 one."""
import numpy as np
import pytest

from numerics import assert_bf16_close, assert_state_close
from test_gpu_deltanet import CONV, DK, DV, HK, HV, Layer, C, oracle, oracle_row

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hb(bridge):
    import hip_bridge.quant  # noqa: F401

    return bridge


def prep(hb, L, row_tokens, qkv, ab, z):
    """gdn_prep of a ragged step: device buffers of q_hat, k_hat, v, decay, beta."""
    from hip_bridge import DeviceBuffer

    T = int(sum(row_tokens))
    cu = np.concatenate([[0], np.cumsum(row_tokens)]).astype(np.int32)
    d = dict(qkv=DeviceBuffer.from_array(qkv), ab=DeviceBuffer.from_array(ab), z=DeviceBuffer.from_array(z),
             cu=DeviceBuffer.from_array(cu), hoff=DeviceBuffer.from_array(np.zeros(L.rows, np.int32)),
             q=DeviceBuffer(T * HK * DK * 4), k=DeviceBuffer(T * HK * DK * 4), v=DeviceBuffer(T * HV * DV * 4),
             g=DeviceBuffer(T * HV * 4), b=DeviceBuffer(T * HV * 4), o=DeviceBuffer(T * HV * DV * 4),
             y=DeviceBuffer(T * HV * DV * 2))
    hb.call("hb_gdn_prep", d["qkv"], C, d["ab"], hb._p(d["ab"].ptr + 2 * HV), 2 * HV, L.d["conv_w"], L.d["alog"],
            L.d["dt"], L.d["win"], d["hoff"], None, None, d["cu"], L.rows, HK, HV, DK, DV, CONV, L.maxt, d["q"],
            d["k"], d["v"], d["g"], d["b"], None)
    return d


def chunked(hb, d, rows, state, norm, src=None, dst=None):
    hb.call("hb_gdn_chunked", d["q"], d["k"], d["v"], d["g"], d["b"], d["cu"], rows, HK, HV, DK, DV, state, src, dst,
            d["o"], d["z"], HV * DV, norm, d["y"], None)


def test_chunked_ragged_vs_oracle(hb):
    rows = 8
    L = Layer(hb, rows, 200, 41)
    row_tokens = [1, 17, 64, 65, 130, 0, 200, 128]
    qkv, ab, z = L.inputs(row_tokens)
    print("case: gdn chunked ragged rows", row_tokens, flush=True)
    d = prep(hb, L, row_tokens, qkv, ab, z)
    chunked(hb, d, rows, L.d["state"], L.d["norm"])
    hb.synchronize()
    T = int(sum(row_tokens))
    o = d["o"].download(np.float32, (T, HV, DV))
    y = hb.quant.bf16_value(d["y"].download(np.uint16, (T, HV * DV)))
    st = L.state()
    qv, abv, zv = (hb.quant.bf16_value(t) for t in (qkv, ab, z))
    cu = np.concatenate([[0], np.cumsum(row_tokens)])
    for r in range(rows):
        if row_tokens[r] == 0:
            assert np.array_equal(st[r], L.state0[r]), "an empty row keeps its state"
            continue
        sl = slice(cu[r], cu[r + 1])
        _, _, out, s = oracle_row(L, r, qv[sl], abv[sl], L.hist0[r], L.state0[r])
        assert_state_close(st[r], s, f"state row {r} ({row_tokens[r]} tokens)")
        assert_state_close(o[sl], out, f"outputs row {r}")
        ref_y = oracle.rms(out.astype(np.float32).reshape(-1, DV), L.norm_w).reshape(out.shape) * oracle.silu(
            zv[sl].reshape(-1, HV, DV))
        assert_bf16_close(y[sl].reshape(-1, HV, DV), ref_y, f"gated norm row {r}")


def test_chunked_slots(hb):
    """Row r reads its state at src[r] and writes dst[r]; the source stays intact."""
    from hip_bridge import DeviceBuffer

    rows = 3
    L = Layer(hb, rows, 80, 42)
    row_tokens = [80, 3, 64]
    qkv, ab, z = L.inputs(row_tokens)
    print("case: gdn chunked slots", flush=True)
    d = prep(hb, L, row_tokens, qkv, ab, z)
    km = np.ascontiguousarray(L.state0.transpose(0, 1, 3, 2))
    both = DeviceBuffer.from_array(np.concatenate([np.zeros_like(km), km]))  # slots 0..2 empty, 3..5 the states
    src = DeviceBuffer.from_array(np.array([3, 4, 5], np.int32))
    dst = DeviceBuffer.from_array(np.array([2, 0, 1], np.int32))
    chunked(hb, d, rows, both, L.d["norm"], src, dst)
    chunked(hb, d, rows, L.d["state"], L.d["norm"])  # in place, slot r
    hb.synchronize()
    got = both.download(np.float32, (2 * rows, HV, DK, DV))
    want = L.d["state"].download(np.float32, (rows, HV, DK, DV))
    assert np.array_equal(got[rows:], km), "source slots untouched"
    for r, s in enumerate([2, 0, 1]):
        assert np.array_equal(got[s], want[r]), f"row {r} written at slot {s}"


def test_chunked_equals_serial_prefill_workload(hb):
    """32 prompts of U[64, 2048] tokens (up to 32 chunks each): the chunked
    kernel's final states and outputs against the token-serial kernel's."""
    from hip_bridge import DeviceBuffer

    rng = np.random.default_rng(2048)
    rows = 32
    row_tokens = rng.integers(64, 2049, rows)
    T = int(row_tokens.sum())
    maxt = int(row_tokens.max())
    cu = np.concatenate([[0], np.cumsum(row_tokens)]).astype(np.int32)
    print(f"case: gdn chunked vs serial, {rows} prompts, {T} tokens", flush=True)
    conv_w = (rng.standard_normal((C, CONV)) * 0.5).astype(np.float32)
    alog = rng.uniform(0, 1, HV).astype(np.float32)
    norm_w = (1 + 0.1 * rng.standard_normal(DV)).astype(np.float32)
    state0 = (rng.standard_normal((rows, HV, DK, DV)) * 0.01).astype(np.float32)  # key-major on the device
    dev = dict(conv_w=DeviceBuffer.from_array(conv_w), alog=DeviceBuffer.from_array(alog),
               dt=DeviceBuffer.from_array(np.zeros(HV, np.float32)), norm=DeviceBuffer.from_array(norm_w),
               win=DeviceBuffer(rows * (CONV - 1 + maxt) * C * 2), cu=DeviceBuffer.from_array(cu),
               hoff=DeviceBuffer.from_array(np.zeros(rows, np.int32)), qkv=DeviceBuffer(T * C * 2),
               ab=DeviceBuffer(T * 2 * HV * 2), z=DeviceBuffer(T * HV * DV * 2),
               q=DeviceBuffer(T * HK * DK * 4), k=DeviceBuffer(T * HK * DK * 4), v=DeviceBuffer(T * HV * DV * 4),
               g=DeviceBuffer(T * HV * 4), b=DeviceBuffer(T * HV * 4))
    dev["win"].zero()
    hb.call("hb_random_normal", 71, T * C, 1.0, 0.0, 4, dev["qkv"], None)
    hb.call("hb_random_normal", 72, T * 2 * HV, 1.0, 0.0, 4, dev["ab"], None)
    hb.call("hb_random_normal", 73, T * HV * DV, 1.0, 0.0, 4, dev["z"], None)
    hb.call("hb_gdn_prep", dev["qkv"], C, dev["ab"], hb._p(dev["ab"].ptr + 2 * HV), 2 * HV, dev["conv_w"],
            dev["alog"], dev["dt"], dev["win"], dev["hoff"], None, None, dev["cu"], rows, HK, HV, DK, DV, CONV, maxt,
            dev["q"], dev["k"], dev["v"], dev["g"], dev["b"], None)
    results = {}
    for name in ("serial", "chunked"):
        st = DeviceBuffer.from_array(state0)
        o, y = DeviceBuffer(T * HV * DV * 4), DeviceBuffer(T * HV * DV * 2)
        if name == "serial":
            hb.call("hb_gdn_recurrence", dev["q"], dev["k"], dev["v"], dev["g"], dev["b"], dev["cu"], rows, HK, HV,
                    DK, DV, st, None, None, None, None, None, None, 0, 0, o, dev["z"], HV * DV, dev["norm"], y, None)
        else:
            hb.call("hb_gdn_chunked", dev["q"], dev["k"], dev["v"], dev["g"], dev["b"], dev["cu"], rows, HK, HV, DK,
                    DV, st, None, None, o, dev["z"], HV * DV, dev["norm"], y, None)
        hb.synchronize()
        results[name] = (st, o, y)
        print(f"  {name} done", flush=True)
    s_ser = results["serial"][0].download(np.float32, state0.shape)
    s_chk = results["chunked"][0].download(np.float32, state0.shape)
    assert not np.array_equal(s_ser, state0)
    for r in range(rows):
        assert_state_close(s_chk[r], s_ser[r], f"state row {r} ({row_tokens[r]} tokens)")
    # outputs of the longest prompt, the shortest and two more
    for r in sorted({int(np.argmax(row_tokens)), int(np.argmin(row_tokens)), 0, rows - 1}):
        n, off = int(row_tokens[r]), int(cu[r])
        o_ser = results["serial"][1].download(np.float32, (n, HV, DV), off * HV * DV * 4)
        o_chk = results["chunked"][1].download(np.float32, (n, HV, DV), off * HV * DV * 4)
        assert_state_close(o_chk, o_ser, f"outputs row {r}")
        y_ser = hb.quant.bf16_value(results["serial"][2].download(np.uint16, (n, HV * DV), off * HV * DV * 2))
        y_chk = hb.quant.bf16_value(results["chunked"][2].download(np.uint16, (n, HV * DV), off * HV * DV * 2))
        assert_bf16_close(y_chk, y_ser, f"gated norm row {r}")
