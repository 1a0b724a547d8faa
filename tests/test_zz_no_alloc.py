"""The allocation-free selection entry point, hb_argmax_margin_noalloc,
against hb_argmax_margin with a caller-allocated workspace (the same
multi-workgroup scan): winners, margins and statuses bit-identical, on two
calls in a row, the second with a smaller input than the first (the static
scratch still holds the first call's summaries beyond the second call's
entries). Also its size limit: a call that needs more than the 1 MiB scratch
fails before any device work and leaves the outputs untouched."""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def select(hb, logits, ld, rows, vocab, noalloc):
    from hip_bridge import DeviceBuffer

    win, mar, st = DeviceBuffer(rows * 4), DeviceBuffer(rows * 4), DeviceBuffer(rows * 4)
    if noalloc:
        hb.call("hb_argmax_margin_noalloc", logits, ld, rows, vocab, win, mar, st, None)
    else:
        ws = DeviceBuffer(hb.load().hb_argmax_workspace_bytes(rows, vocab))
        hb.call("hb_argmax_margin", logits, ld, rows, vocab, win, mar, st, ws, None)
    hb.synchronize()
    return win.download(np.uint32, rows), mar.download(np.float32, rows), st.download(np.int32, rows)


def planted_logits(rng, rows, vocab, ld):
    lg = rng.standard_normal((rows, ld)).astype(np.float32)
    lg[0, 5], lg[0, vocab - 1] = 50.0, 50.0  # a tie across chunks: the lower index wins
    lg[1, :] = -0.0
    lg[1, vocab // 2] = 0.0  # +0 above -0 under the total order
    lg[2, vocab - 3] = np.nan  # status 1
    lg[3, ld - 1] = 1e9  # beyond the vocabulary: ignored
    return lg


@pytest.mark.parametrize("order", ["large-then-small"])
def test_noalloc_matches_workspace_selection(bridge, order):
    from hip_bridge import DeviceBuffer

    hb = bridge
    rng = np.random.default_rng(17)
    for rows, vocab, ld in [(96, 151936, 152064), (7, 20000, 20008)]:
        print(f"case: noalloc selection rows {rows} vocab {vocab}", flush=True)
        lg = planted_logits(rng, rows, vocab, ld)
        dl = DeviceBuffer.from_array(lg)
        want = select(hb, dl, ld, rows, vocab, noalloc=False)
        got = select(hb, dl, ld, rows, vocab, noalloc=True)
        assert np.array_equal(got[0], want[0]), "winners differ"
        assert np.array_equal(got[1].view(np.uint32), want[1].view(np.uint32)), "margins differ"
        assert np.array_equal(got[2], want[2]), "statuses differ"
        assert got[0][0] == 5 and got[1][0] == 0.0
        assert got[2][2] == 1 and got[2].sum() == 1
        for r in (0, 1, 3, rows - 1):
            w, m = oracle.winner(lg[r, :vocab])
            assert got[0][r] == w and got[1][r] == np.float32(m)


def test_noalloc_rejects_more_than_its_scratch(bridge):
    from hip_bridge import DeviceBuffer, HipBridgeError

    hb = bridge
    limit = int(hb.load().hb_argmax_noalloc_limit_bytes())
    vocab = 151936
    chunks = (vocab + 8191) // 8192
    rows = limit // 16 // chunks + 1  # one row more than the scratch holds
    assert rows * chunks * 16 > limit
    sentinel = np.full(4, 0x5A5A5A5A, np.uint32)
    win, mar, st = (DeviceBuffer.from_array(sentinel) for _ in range(3))
    dl = DeviceBuffer(16)  # never read: the size check fails first
    with pytest.raises(HipBridgeError, match="static"):
        hb.call("hb_argmax_margin_noalloc", dl, vocab, rows, vocab, win, mar, st, None)
    hb.synchronize()
    for b in (win, mar, st):
        assert np.array_equal(b.download(np.uint32, 4), sentinel)
