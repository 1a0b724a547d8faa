"""Properties of the benchmark's own engine: the random-init 48-layer hybrid
decoder (36 Gated-DeltaNet + 12 gated GQA layers, hidden 2048, 512 experts
top-10 + shared, vocab 151936, MTP head) with 64 rows of synthetic context of
U[256, 8192] tokens, the exact configuration bench.py times.

Greedy decoding is lossless under speculation (src/serving/native_mtp_decode.rs:
124-295 emits the target's winners whatever the drafts were), so these three
loops over the same starting state must emit bit-identical streams:
- width 1 (no drafts: 64 target tokens per step);
- width 4 with the reference's margin gate 1.25 (the benchmark's headline);
- width 4 with the gate at 0, so every row proposes all 3 drafts and each
  step verifies 4 tokens per row (256 target tokens per step).
Every step also requires finite target and MTP logits and well-formed
acceptance rows (the loop raises otherwise)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROWS, BUDGET = 64, 8


@pytest.fixture(scope="module")
def bench_engine(bridge):
    from hip_bridge.engine import Engine, hybrid_config

    cfg = hybrid_config()
    rng = np.random.default_rng(20261201)
    contexts = rng.integers(256, 8193, ROWS).astype(np.int32)
    max_context = (8192 + 256 + 4 + 15) // 16 * 16
    print("case: 48-layer benchmark engine create (64 rows)", flush=True)
    e = Engine(cfg, ROWS, max_context, 8, ROWS * 4, seed=20261201, mtp=True)
    pending = rng.integers(0, cfg.vocab, ROWS).astype(np.uint32)
    yield e, contexts, pending
    e.close()


def run(e, contexts, pending, width, gate):
    from hip_bridge.engine import DecodeLoop

    e.synthetic_context(contexts, seed=20261202)  # the same starting state for every loop
    loop = DecodeLoop(e, width=width, gate_margin=gate)
    for r in range(ROWS):
        loop.admit(r, int(contexts[r]), int(pending[r]), BUDGET)
    steps = 0
    while loop.stats()["live"]:
        loop.step()
        steps += 1
        assert steps <= BUDGET
    outs = [loop.output(r)[0] for r in range(ROWS)]
    stats = loop.stats()
    loop.close()
    return outs, stats


def test_speculation_is_lossless_on_the_bench_engine(bench_engine):
    e, contexts, pending = bench_engine
    print("case: bench engine width 1", flush=True)
    greedy, gs = run(e, contexts, pending, 1, 1.25)
    assert gs["steps"] == BUDGET and gs["target_tokens"] == ROWS * BUDGET and gs["emitted"] == ROWS * BUDGET
    print("case: bench engine width 4 gate 1.25", flush=True)
    spec, ss = run(e, contexts, pending, 4, 1.25)
    print("case: bench engine width 4 forced (gate 0)", flush=True)
    forced, fs = run(e, contexts, pending, 4, 0.0)
    print("width 1:", gs, "\nwidth 4 gate 1.25:", ss, "\nwidth 4 gate 0:", fs, flush=True)
    for r in range(ROWS):
        assert len(greedy[r]) == BUDGET + 1  # pending first, then the budget
        assert np.array_equal(spec[r], greedy[r]), f"row {r}: width-4 stream differs from greedy"
        assert np.array_equal(forced[r], greedy[r]), f"row {r}: forced width-4 stream differs from greedy"
    # the forced loop really verifies full blocks: 3 drafts for every row with budget left
    first = ROWS * 1  # step 0 has no drafts yet
    assert fs["target_tokens"] >= first + (fs["steps"] - 1) * ROWS * 2
    assert fs["proposed"] >= ss["proposed"]
