"""The decode engine against the CPU composition of the hybrid decoder
(oracle/model.py, restating qwen_forward_core, native/qwen_model.inc:277-373),
on a small geometry of the same family: 3 Gated-DeltaNet layers + 1 gated
GQA layer, 8 experts top-2 plus the shared expert, an MTP head.

- every layer of a ragged prefill, teacher-forced: the oracle layer applied
  to the engine's own residual stream (trace) must give the engine's next
  residual (rel 2e-2), then the final norm and lm_head;
- decode and speculative steps continue the state exactly like the full
  sequence (the chunked == full-sequence invariant of qwen_tests.rs:294-306);
- the MTP head over (target hidden, next token) pairs;
- the speculative decode loop emits the target's greedy stream bit-exactly,
  with acceptance counts fixed by the plan for perfect and corrupted drafts.
"""
import numpy as np
import pytest

import oracle
from layer_check import Row, check_layer, check_layers
from numerics import assert_bf16_close
from oracle.model import MTP_NORM, HybridModel

pytestmark = pytest.mark.gpu

MAX_ROWS, MAX_CTX, MAX_ROW_T, MAX_STEP_T = 4, 256, 64, 160
# Router-logit gap below which a top-k boundary counts as a near-tie (the MoE
# half starts from the engine's own residual, so router inputs differ only by
# the rounding of the normalised input and of the mixer's projections).
TIE = 2e-3


@pytest.fixture(scope="module")
def eng(bridge):
    from hip_bridge.engine import Engine, tiny_config

    cfg = tiny_config()
    print("case: engine tiny config create", flush=True)
    e = Engine(cfg, MAX_ROWS, MAX_CTX, MAX_ROW_T, MAX_STEP_T, seed=11, mtp=True)
    e.trace(True)
    model = HybridModel(cfg.dims(), e.export)
    model.tie_window = TIE
    yield e, model
    e.close()


def well_conditioned(model):
    # A near-tie in top-k routing lets rounding pick another expert, which the
    # comparisons above would report as a mismatch; once they have passed, a
    # small gap only means the data came close to one.
    print(f"smallest routing gap seen by the oracle: {model.min_route_gap:.3g}", flush=True)


def prompts(seed, lengths, vocab):
    rng = np.random.default_rng(seed)
    return [rng.integers(0, vocab, n).astype(np.uint32) for n in lengths]


def prefill(e, seqs, rows=None):
    rows = list(range(len(seqs))) if rows is None else rows
    lens = [len(s) for s in seqs]
    T = sum(lens)
    e.forward(lens, [0] * len(seqs), rows, np.concatenate(seqs), logit_rows=list(range(T)))
    return e.read("logits", T), e.read("hidden", T), np.cumsum([0] + lens)


def test_prefill_matches_oracle_layer_by_layer(eng):
    e, model = eng
    V, L, H = e.config.vocab, e.config.layers, e.config.hidden
    seqs = prompts(1, [7, 1, 23, 12], V)
    print("case: engine prefill rows 7,1,23,12", flush=True)
    logits, hidden, cu = prefill(e, seqs)
    trace, mid = e.read("trace", int(cu[-1])), e.read("mid_trace", int(cu[-1]))
    for r, s in enumerate(seqs):
        row = Row(L, H)
        row.extend(trace[:, cu[r]:cu[r + 1]], mid[:, cu[r]:cu[r + 1]])
        check_layers(model, row, len(s), s, f"row {r}")
        hn, want = model.head(row.x[L])
        assert_bf16_close(hidden[cu[r]:cu[r + 1]], hn, f"hidden row {r}")
        assert_bf16_close(logits[cu[r]:cu[r + 1]], want, f"logits row {r}")
    well_conditioned(model)


def test_decode_and_speculative_steps_continue_state(eng):
    e, model = eng
    V, L, H = e.config.vocab, e.config.layers, e.config.hidden
    seqs = prompts(2, [9, 16, 3], V)
    _, _, cu = prefill(e, seqs)
    trace, mid = e.read("trace", int(cu[-1])), e.read("mid_trace", int(cu[-1]))
    rows = [Row(L, H) for _ in seqs]
    for r in range(3):
        rows[r].extend(trace[:, cu[r]:cu[r + 1]], mid[:, cu[r]:cu[r + 1]])
    rng = np.random.default_rng(5)
    # plain decode step: one token per row
    nxt = rng.integers(0, V, 3).astype(np.uint32)
    pos = [len(s) for s in seqs]
    print("case: engine decode step", flush=True)
    e.forward([1, 1, 1], pos, [0, 1, 2], nxt, hist_off=pos, logit_rows=[0, 1, 2])
    got, trace, mid = e.read("logits", 3), e.read("trace", 3), e.read("mid_trace", 3)
    seqs = [np.append(s, t) for s, t in zip(seqs, nxt)]
    for r, s in enumerate(seqs):
        rows[r].extend(trace[:, r:r + 1], mid[:, r:r + 1])
        check_layers(model, rows[r], 1, s, f"decode row {r}")
        assert_bf16_close(got[r], model.head(rows[r].x[L][-1:])[1][0], f"decode logits row {r}")
    # speculative verify of 4 tokens per row, then commit 1..4 of them via the log
    block = rng.integers(0, V, (3, 4)).astype(np.uint32)
    pos = [len(s) for s in seqs]
    print("case: engine speculative verify", flush=True)
    e.forward([4, 4, 4], pos, [0, 1, 2], block.reshape(-1), hist_off=[1, 1, 1], speculative=True,
              logit_rows=list(range(12)))
    ver, trace, mid = e.read("logits", 12).reshape(3, 4, V), e.read("trace", 12), e.read("mid_trace", 12)
    keep = [1, 4, 2]
    for r, s in enumerate(seqs):
        trial = rows[r].copy()
        trial.extend(trace[:, 4 * r:4 * r + 4], mid[:, 4 * r:4 * r + 4])
        check_layers(model, trial, 4, np.concatenate([s, block[r]]), f"verify row {r}")
        assert_bf16_close(ver[r], model.head(trial.x[L][-4:])[1], f"verify logits row {r}")
        rows[r].extend(trace[:, 4 * r:4 * r + keep[r]], mid[:, 4 * r:4 * r + keep[r]])
    seqs = [np.concatenate([s, block[r, :keep[r]]]) for r, s in enumerate(seqs)]
    nxt = rng.integers(0, V, 3).astype(np.uint32)
    print("case: engine step after partial acceptance", flush=True)
    e.forward([1, 1, 1], [len(s) for s in seqs], [0, 1, 2], nxt, hist_off=keep, log_count=keep,
              speculative=True, logit_rows=[0, 1, 2])
    got, trace, mid = e.read("logits", 3), e.read("trace", 3), e.read("mid_trace", 3)
    for r, s in enumerate(seqs):
        rows[r].extend(trace[:, r:r + 1], mid[:, r:r + 1])
        check_layers(model, rows[r], 1, np.append(s, nxt[r]), f"after commit row {r}")
        assert_bf16_close(got[r], model.head(rows[r].x[L][-1:])[1][0], f"after commit logits row {r}")
    well_conditioned(model)


def test_prefill_in_chunks_equals_full_sequence(eng):
    # Both chunks have more than 16 tokens, so every projection takes the same
    # streaming kernel as the full sequence (a step of at most 16 tokens uses the
    # GEMV kernel, whose accumulation order differs): bit-exact equality.
    e, _ = eng
    V = e.config.vocab
    (s,) = prompts(3, [40], V)
    full, _, _ = prefill(e, [s], rows=[3])
    e.forward([20], [0], [3], s[:20])
    e.forward([20], [20], [3], s[20:], hist_off=[20], logit_rows=list(range(20)))
    chunked = e.read("logits", 20)
    assert np.array_equal(chunked, full[20:]), "chunked prefill differs from the full sequence"


def test_prefill_with_chunked_recurrence_matches_oracle(eng):
    # A row of 64 tokens sends the whole step's DeltaNet layers through the
    # chunked MFMA recurrence; a plain decode step (token-serial) continues it.
    e, model = eng
    V, L, H = e.config.vocab, e.config.layers, e.config.hidden
    seqs = prompts(7, [64, 5, 50], V)
    print("case: engine prefill rows 64,5,50 (chunked recurrence)", flush=True)
    logits, hidden, cu = prefill(e, seqs)
    trace, mid = e.read("trace", int(cu[-1])), e.read("mid_trace", int(cu[-1]))
    rows = []
    for r, s in enumerate(seqs):
        row = Row(L, H)
        row.extend(trace[:, cu[r]:cu[r + 1]], mid[:, cu[r]:cu[r + 1]])
        check_layers(model, row, len(s), s, f"row {r}")
        hn, want = model.head(row.x[L])
        assert_bf16_close(hidden[cu[r]:cu[r + 1]], hn, f"hidden row {r}")
        assert_bf16_close(logits[cu[r]:cu[r + 1]], want, f"logits row {r}")
        rows.append(row)
    nxt = np.random.default_rng(8).integers(0, V, 3).astype(np.uint32)
    pos = [len(s) for s in seqs]
    e.forward([1, 1, 1], pos, [0, 1, 2], nxt, hist_off=pos, logit_rows=[0, 1, 2])
    got, trace, mid = e.read("logits", 3), e.read("trace", 3), e.read("mid_trace", 3)
    for r, s in enumerate(seqs):
        rows[r].extend(trace[:, r:r + 1], mid[:, r:r + 1])
        check_layers(model, rows[r], 1, np.append(s, nxt[r]), f"decode after chunked prefill row {r}")
        assert_bf16_close(got[r], model.head(rows[r].x[L][-1:])[1][0], f"decode logits row {r}")
    well_conditioned(model)


def test_mtp_head_matches_oracle(eng):
    e, model = eng
    V, L = e.config.vocab, e.config.layers
    seqs = prompts(4, [11, 5], V)
    logits, hidden, cu = prefill(e, seqs)
    nxt = [np.append(s[1:], np.uint32(np.argmax(logits[cu[r + 1] - 1]))) for r, s in enumerate(seqs)]
    T = int(cu[-1])
    print("case: engine MTP refresh", flush=True)
    e.mtp_forward([len(s) for s in seqs], [0, 0], [0, 1], np.concatenate(nxt), list(range(T)),
                  logit_rows=list(range(T)))
    got, got_h, trace = e.read("logits", T), e.read("mtp_hidden", T), e.read("trace", T)
    mid = e.read("mid_trace", T)
    for r in range(len(seqs)):
        sl = slice(cu[r], cu[r + 1])
        assert_bf16_close(trace[0, sl], model.mtp_input(nxt[r], hidden[sl]), f"MTP fc row {r}")
        check_layer(model, L, trace[0, sl], mid[L, sl], trace[1, sl], cu[r + 1] - cu[r], f"MTP row {r}")
        mh, want = model.head(trace[1, sl], norm=MTP_NORM)
        assert_bf16_close(got_h[sl], mh, f"MTP hidden row {r}")
        assert_bf16_close(got[sl], want, f"MTP logits row {r}")
    well_conditioned(model)


def run_loop(e, seqs, width, budget, drafts=None):
    """Prefill `seqs`, seed the MTP KV over the prompt, decode `budget` tokens per row."""
    from hip_bridge.engine import DecodeLoop

    logits, _, cu = prefill(e, seqs)
    pend = [int(oracle.winner(logits[cu[r + 1] - 1])[0]) for r in range(len(seqs))]
    nxt = [np.append(s[1:], np.uint32(p)) for s, p in zip(seqs, pend)]
    T = int(cu[-1])
    e.mtp_forward([len(s) for s in seqs], [0] * len(seqs), list(range(len(seqs))), np.concatenate(nxt),
                  list(range(T)))
    loop = DecodeLoop(e, width=width, gate_margin=1.25)
    for r, s in enumerate(seqs):
        loop.admit(r, len(s), pend[r], budget, hist_off=len(s))
    steps = 0
    while loop.stats()["live"]:
        if drafts is not None:
            drafts(loop)
        loop.step()
        steps += 1
        assert steps <= budget + 1
    outs = [loop.output(r)[0] for r in range(len(seqs))]
    stats = loop.stats()
    loop.close()
    return outs, stats


def test_speculative_loop_emits_greedy_stream(eng):
    e, _ = eng
    V = e.config.vocab
    seqs = prompts(6, [13, 30, 4, 21], V)
    print("case: decode loop greedy width 1", flush=True)
    greedy, gs = run_loop(e, seqs, 1, 24)
    assert gs["steps"] == 24 and gs["emitted"] == 4 * 24
    print("case: decode loop MTP width 4", flush=True)
    spec, ss = run_loop(e, seqs, 4, 24)
    for r in range(4):
        assert np.array_equal(spec[r], greedy[r]), f"row {r}: speculative stream differs from greedy"
    assert ss["mtp_calls"] >= ss["steps"] - 1  # every step but the last refreshes the MTP head
    print("MTP stats", ss, flush=True)

    # external drafts: rows 0/2 get the true continuation, rows 1/3 a corrupted second draft
    def oracle_drafts(loop):
        for r in range(4):
            out, _ = loop.output(r)
            n = len(out)
            if n >= len(greedy[r]):
                continue
            d = [int(t) for t in greedy[r][n:n + 3]]
            if r % 2 and len(d) >= 2:
                d[1] = (d[1] + 1) % V
            loop.set_drafts(r, d)

    print("case: decode loop external drafts", flush=True)
    ext, es = run_loop(e, seqs, 4, 24, drafts=oracle_drafts)
    for r in range(4):
        assert np.array_equal(ext[r], greedy[r]), f"row {r}: stream with external drafts differs"
    # perfect rows emit 4 tokens per step (3 accepted + bonus), corrupted rows 2 (1 accepted + correction)
    print("external-draft stats", es, flush=True)
    assert es["accepted"] > 0 and es["steps"] < gs["steps"]
