"""The fused DeltaNet decode step (hb_gdn_decode: the prep and the recurrence in
one launch) against hb_gdn_prep followed by hb_gdn_recurrence on copies of the
same layer state: outputs, gated norm, recurrent state, speculative logs and
the conv window are compared bit for bit (the fused kernel runs the same
arithmetic, wave for wave). The two-kernel path itself is checked against the
oracle in test_gpu_deltanet.py.

Cases: a config-3 decode step (32 rows, one token each, in place); ragged
speculative rows (0 to 8 tokens) followed by a step that replays their
accepted prefixes (pending logs, history offsets), including a row with only a
pending log; and rows that read one set of slots and write another (the parent
slots must stay untouched)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

HK, HV, DK, DV, CONV = 16, 32, 128, 128, 4
C = 2 * HK * DK + HV * DV


class Pair:
    """Two device copies of one layer's slots: one stepped by the fused kernel,
    one by prep + recurrence."""

    def __init__(self, hb, slots, max_tokens, log_cap, seed):
        import hip_bridge.quant  # noqa: F401
        from hip_bridge import DeviceBuffer

        self.hb, self.slots, self.maxt, self.cap = hb, slots, max_tokens, log_cap
        rng = np.random.default_rng(seed)
        self.rng = rng
        win = np.zeros((slots, CONV - 1 + max_tokens, C), np.uint16)
        win[:, :] = hb.quant.bf16_bits(rng.standard_normal((slots, CONV - 1 + max_tokens, C), dtype=np.float32))
        state = (rng.standard_normal((slots, HV, DK, DV)) * 0.01).astype(np.float32)
        logs = dict(lk=rng.standard_normal((slots, log_cap, HV, DK)).astype(np.float32),
                    ld=rng.standard_normal((slots, log_cap, HV, DV)).astype(np.float32),
                    lg=rng.uniform(0.5, 1.0, (slots, log_cap, HV)).astype(np.float32))
        self.params = dict(conv_w=DeviceBuffer.from_array((rng.standard_normal((C, CONV)) * 0.5).astype(np.float32)),
                           alog=DeviceBuffer.from_array(rng.uniform(0, 1, HV).astype(np.float32)),
                           dt=DeviceBuffer.from_array((0.1 * rng.standard_normal(HV)).astype(np.float32)),
                           norm=DeviceBuffer.from_array((1 + 0.1 * rng.standard_normal(DV)).astype(np.float32)))
        self.sides = []
        for _ in range(2):
            self.sides.append(dict(win=DeviceBuffer.from_array(win), state=DeviceBuffer.from_array(state),
                                   **{k: DeviceBuffer.from_array(v) for k, v in logs.items()}))

    def step(self, row_tokens, hist_off, log_count, speculative, src=None, dst=None):
        from hip_bridge import DeviceBuffer

        hb, rng = self.hb, self.rng
        rows, T = len(row_tokens), int(sum(row_tokens))
        n = max(T, 1)
        qkv = hb.quant.bf16_bits(rng.standard_normal((n, C), dtype=np.float32))
        ab = hb.quant.bf16_bits(rng.standard_normal((n, 2 * HV), dtype=np.float32))
        z = hb.quant.bf16_bits(rng.standard_normal((n, HV * DV), dtype=np.float32))
        cu = np.concatenate([[0], np.cumsum(row_tokens)]).astype(np.int32)
        d = dict(qkv=DeviceBuffer.from_array(qkv), ab=DeviceBuffer.from_array(ab), z=DeviceBuffer.from_array(z),
                 cu=DeviceBuffer.from_array(cu), hoff=DeviceBuffer.from_array(np.asarray(hist_off, np.int32)),
                 lcnt=DeviceBuffer.from_array(np.asarray(log_count, np.int32)),
                 src=None if src is None else DeviceBuffer.from_array(np.asarray(src, np.int32)),
                 dst=None if dst is None else DeviceBuffer.from_array(np.asarray(dst, np.int32)))
        b_ptr = hb._p(d["ab"].ptr + 2 * HV)
        p = self.params
        outs = []
        for k, sd in enumerate(self.sides):
            o, y = DeviceBuffer(n * HV * DV * 4), DeviceBuffer(n * HV * DV * 2)
            o.zero()
            y.zero()
            if k == 0:
                hb.call("hb_gdn_decode", d["qkv"], C, d["ab"], b_ptr, 2 * HV, p["conv_w"], p["alog"], p["dt"],
                        sd["win"], d["hoff"], d["src"], d["dst"], d["cu"], rows, HK, HV, DK, DV, CONV, self.maxt,
                        sd["state"], sd["lk"], sd["ld"], sd["lg"], d["lcnt"], self.cap, speculative, o, d["z"],
                        HV * DV, p["norm"], y, None)
            else:
                q, kk = DeviceBuffer(n * HK * DK * 4), DeviceBuffer(n * HK * DK * 4)
                v, g, b = DeviceBuffer(n * HV * DV * 4), DeviceBuffer(n * HV * 4), DeviceBuffer(n * HV * 4)
                hb.call("hb_gdn_prep", d["qkv"], C, d["ab"], b_ptr, 2 * HV, p["conv_w"], p["alog"], p["dt"],
                        sd["win"], d["hoff"], d["src"], d["dst"], d["cu"], rows, HK, HV, DK, DV, CONV, self.maxt,
                        q, kk, v, g, b, None)
                hb.call("hb_gdn_recurrence", q, kk, v, g, b, d["cu"], rows, HK, HV, DK, DV, sd["state"], d["src"],
                        d["dst"], sd["lk"], sd["ld"], sd["lg"], d["lcnt"], self.cap, speculative, o, d["z"],
                        HV * DV, p["norm"], y, None)
            hb.synchronize()
            outs.append((o.download(np.uint32, (n, HV * DV)), y.download(np.uint16, (n, HV * DV))))
        return outs

    def compare(self, outs, what):
        (o0, y0), (o1, y1) = outs
        assert np.array_equal(o0, o1), f"{what}: outputs differ"
        assert np.array_equal(y0, y1), f"{what}: gated norm differs"
        a, b = self.sides
        shapes = dict(win=(np.uint16, (self.slots, CONV - 1 + self.maxt, C)),
                      state=(np.uint32, (self.slots, HV, DK, DV)), lk=(np.uint32, (self.slots, self.cap, HV, DK)),
                      ld=(np.uint32, (self.slots, self.cap, HV, DV)), lg=(np.uint32, (self.slots, self.cap, HV)))
        for k, (dt, shp) in shapes.items():
            assert np.array_equal(a[k].download(dt, shp), b[k].download(dt, shp)), f"{what}: {k} differs"


def test_decode_step_32_rows_in_place(bridge):
    P = Pair(bridge, 32, 4, 4, 7)
    print("case: gdn decode fused vs prep+recurrence, 32 rows T=1", flush=True)
    P.compare(P.step([1] * 32, [0] * 32, [0] * 32, 0), "decode")
    print("case: second decode step (history offset 1)", flush=True)
    P.compare(P.step([1] * 32, [1] * 32, [0] * 32, 0), "second decode")


def test_ragged_speculative_then_replay(bridge):
    P = Pair(bridge, 8, 8, 8, 8)
    rt = [4, 1, 8, 0, 3, 2, 5, 4]
    print(f"case: gdn fused speculative rows {rt}", flush=True)
    P.compare(P.step(rt, [0, 1, 2, 0, 4, 8, 3, 1], [0] * 8, 1), "speculative")
    acc = [2, 1, 5, 0, 3, 1, 0, 4]
    rt2 = [1, 1, 1, 0, 2, 1, 1, 1]
    rt2[6] = 0  # a row that only replays its log
    acc[6] = 3
    print(f"case: gdn fused replay of accepted prefixes {acc}", flush=True)
    P.compare(P.step(rt2, rt, acc, 0), "replay")
    print("case: gdn fused speculative step after a replay", flush=True)
    P.compare(P.step([4] * 8, rt2, [0] * 8, 1), "speculative again")


def test_distinct_slots_keep_the_parents(bridge):
    rows = 6
    P = Pair(bridge, 2 * rows, 4, 4, 9)
    before = P.sides[0]["state"].download(np.uint32, (2 * rows, HV, DK, DV))[:rows].copy()
    src, dst = list(range(rows)), list(range(rows, 2 * rows))
    print("case: gdn fused with distinct source and destination slots", flush=True)
    P.compare(P.step([1, 2, 4, 1, 3, 1], [0, 1, 2, 3, 4, 0], [0] * rows, 1, src=src, dst=dst), "distinct slots")
    after = P.sides[0]["state"].download(np.uint32, (2 * rows, HV, DK, DV))[:rows]
    assert np.array_equal(before, after), "parent states must stay untouched"
