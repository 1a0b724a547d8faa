"""The decode engine at the full benchmark geometry against the CPU oracle.

Geometry: hidden 2048, vocab 151936, 16/2 x 256 gated GQA heads (64 rotary
dims), 16/32 x 128 Gated-DeltaNet heads, 512 experts top-10 of width 512 plus
the shared expert, 4-bit g64 everywhere, the single-layer MTP head; one
period of the layer program (3 DeltaNet layers, then 1 attention layer),
i.e. layers 0-3 of the 48-layer model.

- a ragged prefill of rows of 1..64 tokens, teacher-forced layer by layer:
  the oracle layer applied to the engine's own residual stream must give the
  engine's next residual (rel 2e-2); the final norm, lm_head and device
  selection for the last token of every row;
- one decode step, one speculative verify of 4 tokens per row, a partial
  commit and the step after it;
- the MTP head over (target hidden, next token) pairs;
- two rows prefilled to 1,100 and 1,023 tokens in 64-token chunks, then a
  decode step and a 4-token verify: the attention layer's mixer over more
  than four of the engine's 256-key splits, and its MoE, for the new tokens;
- RMSNorm and the embedding gather at hidden 2048 directly.

Each layer is judged in two teacher-forced halves (mixer, then MoE) with
near-tie routing judged against the swapped experts (layer_check.py). Top-10
of 512 routing makes near-ties common; the number of such tokens is printed.
"""
import numpy as np
import pytest

import oracle
from layer_check import Row, check_layer, check_layers
from numerics import assert_bf16_close, assert_close
from oracle.model import MTP_NORM, HybridModel

pytestmark = pytest.mark.gpu

MAX_ROWS, MAX_CTX, MAX_ROW_T, MAX_STEP_T = 8, 1280, 64, 192
# Router-logit gap below which a top-k boundary counts as a near-tie. The
# MoE half starts from the engine's own residual, so the router inputs differ
# only where a bf16 rounding of the normalised input flips (~2e-4 on a logit
# whose spread is ~0.9).
TIE = 2e-3


@pytest.fixture(scope="module")
def eng(bridge):
    from hip_bridge.engine import Engine, hybrid_config

    cfg = hybrid_config(layers=4)
    print("case: full-width engine create (4 layers, 512 experts, vocab 151936)", flush=True)
    e = Engine(cfg, MAX_ROWS, MAX_CTX, MAX_ROW_T, MAX_STEP_T, seed=29, mtp=True)
    e.trace(True)
    model = HybridModel(cfg.dims(), e.export)
    model.tie_window = TIE
    yield e, model
    print(f"smallest routing gap seen by the oracle: {model.min_route_gap:.3g}", flush=True)
    e.close()


def check_head(model, e, hidden_rows, logits_rows, winners, x_last, what, norm=None):
    """Hidden and logits of the given rows against the oracle head; winners
    bit-exact against the total-order argmax of the device logits, and equal to
    the oracle's winner wherever the oracle's margin exceeds twice the
    observed logit error."""
    hn, want = model.head(x_last) if norm is None else model.head(x_last, norm=norm)
    assert_bf16_close(hidden_rows, hn, f"{what} hidden")
    assert_bf16_close(logits_rows, want, f"{what} logits")
    for i in range(len(logits_rows)):
        w, _ = oracle.winner(logits_rows[i])
        assert winners[i] == w, f"{what} row {i}: device winner {winners[i]} != argmax of device logits {w}"
        ow, om = oracle.winner(want[i].astype(np.float32))
        err = float(np.max(np.abs(logits_rows[i] - want[i])))
        if om > 2 * err:
            assert winners[i] == ow, f"{what} row {i}: winner {winners[i]} != oracle {ow} (margin {om}, err {err})"


def prefill(e, seqs, rows):
    lens = [len(s) for s in seqs]
    T = sum(lens)
    e.forward(lens, [0] * len(seqs), rows, np.concatenate(seqs), logit_rows=list(range(T)))
    return e.read("logits", T), e.read("hidden", T), e.read("winners", T), np.cumsum([0] + lens)


def test_rmsnorm_and_embedding_at_hidden_2048(eng):
    import hip_bridge as hb
    from hip_bridge import DeviceBuffer, quant
    from oracle.model import EMBED, IN_NORM, layer_tensor

    e, model = eng
    H = e.config.hidden
    rng = np.random.default_rng(41)
    rows = 37
    x = (rng.standard_normal((rows, H)) * rng.uniform(0.1, 30, (rows, 1))).astype(np.float32)
    w = model.w(layer_tensor(0, IN_NORM))
    dx, dw = DeviceBuffer.from_array(x), DeviceBuffer.from_array(w)
    out, out32 = DeviceBuffer(rows * H * 2), DeviceBuffer(rows * H * 4)
    print("case: hb_rmsnorm rows 37 hidden 2048", flush=True)
    hb.call("hb_rmsnorm", dx, H, dw, rows, H, 1e-6, out, H, out32, None)
    hb.synchronize()
    want = oracle.rms(x, w, 1e-6)
    assert_close(out32.download(np.float32, (rows, H)), want, 1e-5, "rmsnorm f32")
    got = quant.bf16_value(out.download(np.uint16, (rows, H)))
    # bf16 output: within one bf16 rounding of the exact value
    assert np.all(np.abs(got - want) <= np.abs(want) * 2.0 ** -8 * (1 + 1e-4) + 1e-30), "rmsnorm bf16 beyond one rounding"

    tokens = np.concatenate([[0, e.config.vocab - 1], rng.integers(0, e.config.vocab, 62)]).astype(np.uint32)
    ew, es, eb = e.export(EMBED)
    dt = DeviceBuffer.from_array(tokens)
    dwt, dst, dbt = DeviceBuffer.from_array(ew), DeviceBuffer.from_array(es), DeviceBuffer.from_array(eb)
    dout = DeviceBuffer(len(tokens) * H * 4)
    print("case: hb_embed_gather 64 tokens hidden 2048", flush=True)
    hb.call("hb_embed_gather", dt, len(tokens), dwt, dst, dbt, H, dout, None)
    hb.synchronize()
    assert_close(dout.download(np.float32, (len(tokens), H)), model.embed(tokens), 1e-6, "embedding")


def test_prefill_matches_oracle_layer_by_layer(eng):
    e, model = eng
    V, L, H = e.config.vocab, e.config.layers, e.config.hidden
    rng = np.random.default_rng(1)
    seqs = [rng.integers(0, V, n).astype(np.uint32) for n in (1, 64, 17, 40, 5, 33)]
    print("case: full-width ragged prefill rows 1,64,17,40,5,33", flush=True)
    logits, hidden, winners, cu = prefill(e, seqs, list(range(len(seqs))))
    trace, mid = e.read("trace", int(cu[-1])), e.read("mid_trace", int(cu[-1]))
    ties = 0
    last = [int(c) - 1 for c in cu[1:]]
    xs = []
    for r, s in enumerate(seqs):
        row = Row(L, H)
        row.extend(trace[:, cu[r]:cu[r + 1]], mid[:, cu[r]:cu[r + 1]])
        ties += check_layers(model, row, len(s), s, f"row {r}")
        xs.append(row.x[L][-1:])
    check_head(model, e, hidden[last], logits[last], winners[last], np.concatenate(xs), "prefill last tokens")
    for i in range(len(winners)):  # every row's selection, bit-exact on the device logits
        assert winners[i] == oracle.winner(logits[i])[0], f"token {i}: device winner differs"
    print(f"prefill: {ties} near-tie tokens judged against the swapped routing", flush=True)


def test_decode_verify_and_partial_commit(eng):
    e, model = eng
    V, L, H = e.config.vocab, e.config.layers, e.config.hidden
    rng = np.random.default_rng(2)
    seqs = [rng.integers(0, V, n).astype(np.uint32) for n in (9, 30, 3)]
    rows = [5, 6, 7]
    _, _, _, cu = prefill(e, seqs, rows)
    trace, mid = e.read("trace", int(cu[-1])), e.read("mid_trace", int(cu[-1]))
    rs = [Row(L, H) for _ in seqs]
    for r in range(3):
        rs[r].extend(trace[:, cu[r]:cu[r + 1]], mid[:, cu[r]:cu[r + 1]])
    ties = 0
    nxt = rng.integers(0, V, 3).astype(np.uint32)
    pos = [len(s) for s in seqs]
    print("case: full-width decode step", flush=True)
    e.forward([1, 1, 1], pos, rows, nxt, hist_off=pos, logit_rows=[0, 1, 2])
    got, hid, win, trace = e.read("logits", 3), e.read("hidden", 3), e.read("winners", 3), e.read("trace", 3)
    mid = e.read("mid_trace", 3)
    seqs = [np.append(s, t) for s, t in zip(seqs, nxt)]
    for r, s in enumerate(seqs):
        rs[r].extend(trace[:, r:r + 1], mid[:, r:r + 1])
        ties += check_layers(model, rs[r], 1, s, f"decode row {r}")
    check_head(model, e, hid, got, win, np.concatenate([x.x[L][-1:] for x in rs]), "decode")

    block = rng.integers(0, V, (3, 4)).astype(np.uint32)
    pos = [len(s) for s in seqs]
    print("case: full-width speculative verify", flush=True)
    e.forward([4, 4, 4], pos, rows, block.reshape(-1), hist_off=[1, 1, 1], speculative=True,
              logit_rows=list(range(12)))
    ver, vw, trace = e.read("logits", 12), e.read("winners", 12), e.read("trace", 12)
    mid = e.read("mid_trace", 12)
    keep = [1, 4, 2]
    for r, s in enumerate(seqs):
        trial = rs[r].copy()
        trial.extend(trace[:, 4 * r:4 * r + 4], mid[:, 4 * r:4 * r + 4])
        ties += check_layers(model, trial, 4, np.concatenate([s, block[r]]), f"verify row {r}")
        _, want = model.head(trial.x[L][-4:])
        assert_bf16_close(ver[4 * r:4 * r + 4], want, f"verify logits row {r}")
        rs[r].extend(trace[:, 4 * r:4 * r + keep[r]], mid[:, 4 * r:4 * r + keep[r]])
    for i in range(12):
        assert vw[i] == oracle.winner(ver[i])[0], f"verify token {i}: device winner differs"
    seqs = [np.concatenate([s, block[r, :keep[r]]]) for r, s in enumerate(seqs)]
    nxt = rng.integers(0, V, 3).astype(np.uint32)
    print("case: full-width step after partial acceptance", flush=True)
    e.forward([1, 1, 1], [len(s) for s in seqs], rows, nxt, hist_off=keep, log_count=keep, speculative=True,
              logit_rows=[0, 1, 2])
    got, hid, win, trace = e.read("logits", 3), e.read("hidden", 3), e.read("winners", 3), e.read("trace", 3)
    mid = e.read("mid_trace", 3)
    for r, s in enumerate(seqs):
        rs[r].extend(trace[:, r:r + 1], mid[:, r:r + 1])
        ties += check_layers(model, rs[r], 1, np.append(s, nxt[r]), f"after commit row {r}")
    check_head(model, e, hid, got, win, np.concatenate([x.x[L][-1:] for x in rs]), "after commit")
    print(f"decode/verify: {ties} near-tie tokens judged against the swapped routing", flush=True)


def test_mtp_head_matches_oracle(eng):
    e, model = eng
    V, L = e.config.vocab, e.config.layers
    rng = np.random.default_rng(4)
    seqs = [rng.integers(0, V, n).astype(np.uint32) for n in (11, 26)]
    logits, hidden, _, cu = prefill(e, seqs, [0, 1])
    nxt = [np.append(s[1:], np.uint32(oracle.winner(logits[cu[r + 1] - 1])[0])) for r, s in enumerate(seqs)]
    T = int(cu[-1])
    print("case: full-width MTP head", flush=True)
    e.mtp_forward([len(s) for s in seqs], [0, 0], [0, 1], np.concatenate(nxt), list(range(T)),
                  logit_rows=list(range(T)))
    got, got_h, trace = e.read("logits", T), e.read("mtp_hidden", T), e.read("trace", T)
    win, mid = e.read("winners", T), e.read("mid_trace", T)
    ties = 0
    for r in range(len(seqs)):
        sl = slice(cu[r], cu[r + 1])
        assert_bf16_close(trace[0, sl], model.mtp_input(nxt[r], hidden[sl]), f"MTP fc row {r}")
        ties += check_layer(model, L, trace[0, sl], mid[L, sl], trace[1, sl], cu[r + 1] - cu[r], f"MTP row {r}")
        last = cu[r + 1] - 1
        check_head(model, e, got_h[last:last + 1], got[last:last + 1], win[last:last + 1], trace[1, last:last + 1],
                   f"MTP row {r}", norm=MTP_NORM)
    print(f"MTP: {ties} near-tie tokens judged against the swapped routing", flush=True)


def test_long_context_attention_layer(eng):
    """Rows of 1,100 and 1,023 tokens, prefilled 64 tokens per row per step
    (the chunked DeltaNet form runs where a step's longest row has 64), then
    one decode token and one 4-token speculative verify. The attention layer
    (layer 3) is checked teacher-forced against the oracle for the new tokens:
    at 1,101 / 1,024 keys (the second row's last split is whole) and at
    1,105 / 1,028 (a 4-key last split), with 8-step pieces over five splits."""
    e, model = eng
    V, L, H = e.config.vocab, e.config.layers, e.config.hidden
    attn = [layer for layer in range(L) if (layer + 1) % e.config.interval == 0]
    rng = np.random.default_rng(12)
    lens, rows = [1100, 1023], [2, 3]
    seqs = [rng.integers(0, V, n).astype(np.uint32) for n in lens]
    rs = [Row(L, H) for _ in seqs]
    done, prev = [0, 0], [0, 0]
    print(f"case: full-width long-context prefill rows {lens} in 64-token chunks", flush=True)
    while any(d < n for d, n in zip(done, lens)):
        live = [r for r in range(2) if done[r] < lens[r]]
        take = [min(MAX_ROW_T, lens[r] - done[r]) for r in live]
        toks = np.concatenate([seqs[r][done[r]:done[r] + t] for r, t in zip(live, take)])
        e.forward(take, [done[r] for r in live], [rows[r] for r in live], toks, hist_off=[prev[r] for r in live])
        n = int(sum(take))
        trace, mid = e.read("trace", n), e.read("mid_trace", n)
        at = 0
        for r, t in zip(live, take):
            rs[r].extend(trace[:, at:at + t], mid[:, at:at + t])
            done[r] += t
            prev[r] = t
            at += t
    ties = 0
    nxt = rng.integers(0, V, 2).astype(np.uint32)
    print("case: full-width long-context decode step (contexts 1101, 1024)", flush=True)
    e.forward([1, 1], done, rows, nxt, hist_off=prev)
    trace, mid = e.read("trace", 2), e.read("mid_trace", 2)
    seqs = [np.append(s, t) for s, t in zip(seqs, nxt)]
    for r in range(2):
        rs[r].extend(trace[:, r:r + 1], mid[:, r:r + 1])
        for layer in attn:
            ties += check_layer(model, layer, rs[r].x[layer], rs[r].mid[layer], rs[r].x[layer + 1], 1,
                                f"long decode row {r} ({len(seqs[r])} keys)")
    block = rng.integers(0, V, (2, 4)).astype(np.uint32)
    pos = [len(s) for s in seqs]
    print("case: full-width long-context verify of 4 tokens (contexts 1105, 1028)", flush=True)
    e.forward([4, 4], pos, rows, block.reshape(-1), hist_off=[1, 1], speculative=True)
    trace, mid = e.read("trace", 8), e.read("mid_trace", 8)
    for r in range(2):
        trial = rs[r].copy()
        trial.extend(trace[:, 4 * r:4 * r + 4], mid[:, 4 * r:4 * r + 4])
        for layer in attn:
            ties += check_layer(model, layer, trial.x[layer], trial.mid[layer], trial.x[layer + 1], 4,
                                f"long verify row {r} ({len(seqs[r]) + 4} keys)")
    print(f"long context: {ties} near-tie tokens judged against the swapped routing", flush=True)
