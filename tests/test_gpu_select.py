"""Device greedy selection (hb_argmax_margin) and MTP acceptance (hb_mtp_plan)
against the CPU oracle: bit-exact winners, accept counts and emitted tokens,
exact margins, on the reference's own vectors (judges/device_selection.cpp:7-11,
src/serving/native_speculative.rs:319-415) and on seeded vocabulary-sized rows."""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def select(hb, logits, chunked=False):
    """chunked: with a workspace, rows longer than one chunk take the two-level kernels."""
    from hip_bridge import DeviceBuffer

    logits = np.ascontiguousarray(logits, np.float32)
    rows, vocab = logits.shape
    d = dict(x=DeviceBuffer.from_array(logits), w=DeviceBuffer(4 * rows), m=DeviceBuffer(4 * rows),
             s=DeviceBuffer(4 * rows))
    ws = DeviceBuffer(hb.load().hb_argmax_workspace_bytes(rows, vocab)) if chunked else None
    hb.call("hb_argmax_margin", d["x"], vocab, rows, vocab, d["w"], d["m"], d["s"], ws, None)
    hb.synchronize()
    return d["w"].download(np.uint32, rows), d["m"].download(np.float32, rows), d["s"].download(np.int32, rows)


def test_reference_total_order_vectors(bridge):
    f = np.float32(1.4e-45)  # denorm_min
    x = np.array([[-0.0, +0.0, -f, -0.0], [+0.0, -0.0, -f, -f], [-2, -1, -1, -3], [f, 0.0, f, -f]], np.float32)
    w, _, s = select(bridge, x)
    assert list(w) == [1, 0, 1, 0] and not s.any()
    w, m, _ = select(bridge, np.array([[0.5, 3.25, 1.75, -2.0]], np.float32))
    assert w[0] == 1 and m[0] == np.float32(1.5)
    w, m, _ = select(bridge, np.array([[2.0, 4.0, 4.0]], np.float32))
    assert w[0] == 1 and m[0] == 0.0
    w, m, _ = select(bridge, np.array([[-0.0, 0.0, -1.0]], np.float32))
    assert w[0] == 1
    w, m, _ = select(bridge, np.array([[7.0]], np.float32))
    assert w[0] == 0 and np.isinf(m[0])


def test_tie_break_under_pressure(bridge):
    for n in (1, 2, 63, 64, 65, 255, 256, 257, 511, 512):
        v = np.array([[((i * 17 + n * 31) % 23) - 11.0 for i in range(n)]], np.float32)
        w, m, _ = select(bridge, v)
        tok, marg = oracle.winner(v[0])
        assert w[0] == tok and (m[0] == np.float32(marg) or (np.isinf(m[0]) and np.isinf(marg)))


@pytest.mark.parametrize("chunked", [False, True])
def test_vocabulary_rows_match_oracle(bridge, chunked):
    rng = np.random.default_rng(3)
    rows, vocab = 48, 151936
    x = rng.standard_normal((rows, vocab), dtype=np.float32)
    for r in range(0, rows, 3):  # exact ties at the top, between far-apart columns
        a, b = sorted(rng.choice(vocab, 2, replace=False))
        x[r, a] = x[r, b] = x[r].max() + 1
    x[5, 100] = np.float32(-0.0)
    # ties straddling the 8192-column chunk boundaries of the two-level path
    x[1, 8191] = x[1, 8192] = x[1].max() + 2
    x[4, 3] = x[4, 151935] = x[4].max() + 2
    print(f"case: argmax 48 x 151936 chunked={chunked}", flush=True)
    w, m, s = select(bridge, x, chunked)
    assert not s.any()
    for r in range(rows):
        tok, marg = oracle.winner(x[r])
        assert w[r] == tok, r
        assert m[r] == np.float32(marg), r


def test_nonfinite_rows_flagged(bridge):
    x = np.zeros((3, 20000), np.float32)
    x[0, 17] = np.nan
    x[1, 19999] = np.inf
    for chunked in (False, True):
        _, _, s = select(bridge, x, chunked)
        assert list(s) == [1, 1, 0]


def plan_device(hb, cases, max_draft=8, eos=()):
    """cases: list of (initial winner, draft list, verify-row winners, remaining)."""
    from hip_bridge import DeviceBuffer

    rows = len(cases)
    draft = np.zeros((rows, max_draft), np.uint32)
    nd = np.zeros(rows, np.int32)
    target = np.zeros((rows, max_draft + 1), np.uint32)
    rem = np.zeros(rows, np.int32)
    for r, (init, dr, wins, remaining) in enumerate(cases):
        draft[r, :len(dr)] = dr
        nd[r] = len(dr)
        target[r, 0] = init
        target[r, 1:1 + len(wins)] = wins
        rem[r] = remaining
    eos = np.asarray(eos, np.uint32)
    d = dict(draft=DeviceBuffer.from_array(draft), nd=DeviceBuffer.from_array(nd),
             target=DeviceBuffer.from_array(target), rem=DeviceBuffer.from_array(rem),
             eos=DeviceBuffer.from_array(eos if len(eos) else np.zeros(1, np.uint32)),
             emitted=DeviceBuffer(rows * (max_draft + 1) * 4), n=DeviceBuffer(rows * 4), acc=DeviceBuffer(rows * 4),
             term=DeviceBuffer(rows * 4), st=DeviceBuffer(rows * 4))
    hb.call("hb_mtp_plan", d["draft"], d["nd"], max_draft, d["target"], d["eos"], len(eos), d["rem"], rows, 12,
            d["emitted"], d["n"], d["acc"], d["term"], d["st"], None)
    hb.synchronize()
    em = d["emitted"].download(np.uint32, (rows, max_draft + 1))
    n = d["n"].download(np.int32, rows)
    return ([list(em[r, :n[r]]) for r in range(rows)], d["acc"].download(np.int32, rows),
            d["term"].download(np.int32, rows), d["st"].download(np.int32, rows))


def row(token):
    r = np.full(12, -1.0, np.float32)
    r[token] = 1.0
    return r


def test_plan_matches_oracle_every_boundary(bridge):
    cases, want = [], []
    for n in range(0, 9):
        for accepted in range(0, n + 1):
            for stop in range(-1, n + 1):
                for remaining in (n, n + 1, 9):
                    if remaining == 0:
                        continue
                    draft = [1] * n
                    if accepted < n:
                        draft[accepted] = 2
                    wins = [1] * n
                    init = 1
                    if stop == 0:
                        init = 11
                    elif stop > 0:
                        wins[stop - 1] = 11
                    cases.append((init, draft, wins, remaining))
                    want.append(oracle.plan(row(init), draft, [row(w) for w in wins], [11], remaining))
    print(f"case: mtp plan {len(cases)} boundary rows", flush=True)
    emitted, acc, term, st = plan_device(bridge, cases, eos=[11])
    assert not st.any()
    for r, (em, a, t) in enumerate(want):
        assert emitted[r] == em and acc[r] == a and bool(term[r]) == t, (cases[r], want[r])


def test_plan_random_rows_match_oracle(bridge):
    rng = np.random.default_rng(11)
    cases, want = [], []
    for _ in range(2000):
        n = int(rng.integers(0, 9))
        remaining = int(rng.integers(max(n, 1), 12))
        draft = list(rng.integers(0, 4, n))
        wins = list(rng.integers(0, 4, n))
        init = int(rng.integers(0, 4))
        cases.append((init, draft, wins, remaining))
        want.append(oracle.plan(row(init), draft, [row(w) for w in wins], [3], remaining))
    emitted, acc, term, st = plan_device(bridge, cases, eos=[3])
    assert not st.any()
    for r, (em, a, t) in enumerate(want):
        assert emitted[r] == em and acc[r] == a and bool(term[r]) == t, (cases[r], want[r])


def test_plan_malformed_rows_flagged(bridge):
    # more drafts than the budget, an empty budget, tokens outside the vocabulary
    cases = [(1, [1, 1], [1, 1], 1), (1, [], [], 0), (1, [12], [1], 8), (1, [1], [1], 8)]
    _, _, _, st = plan_device(bridge, cases)
    assert list(st) == [1, 1, 1, 0]
