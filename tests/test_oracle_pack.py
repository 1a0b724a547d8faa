"""CPU pins for the packing-table oracle: an independent brute-force expansion
and the invariants the packed step relies on (closed form of the ragged
generalisation of native/qwen_batch.inc:2-50)."""
import numpy as np
import pytest

import oracle


def brute_force(row_tokens, positions, block_table, page):
    cu, rows_of, pos_of, slot_of = [0], [], [], []
    for r, (t, p0) in enumerate(zip(row_tokens, positions)):
        for j in range(t):
            p = p0 + j
            rows_of.append(r)
            pos_of.append(p)
            slot_of.append(int(block_table[r][p // page]) * page + p % page)
        cu.append(cu[-1] + t)
    return cu, rows_of, pos_of, slot_of


@pytest.mark.parametrize("seed", range(5))
def test_pack_tables_brute_force(seed):
    rng = np.random.default_rng(seed)
    rows, page, max_pages = 64, 16, 40
    row_tokens = rng.choice([0, 1, 4, 64], size=rows)
    positions = rng.integers(0, max_pages * page - 64, size=rows)
    bt = rng.permutation(rows * max_pages).reshape(rows, max_pages).astype(np.int32)
    got = oracle.pack_tables(row_tokens, positions, bt, page)
    cu, rows_of, pos_of, slot_of = brute_force(row_tokens, positions, bt, page)
    assert list(got["cu_seqlens"]) == cu
    assert list(got["token_row"]) == rows_of and list(got["token_pos"]) == pos_of
    assert list(got["kv_slot"]) == slot_of
    assert list(got["context"]) == list(positions + row_tokens)
    # invariants: sorted, contiguous per row, slots unique across the step
    assert np.all(np.diff(got["cu_seqlens"]) >= 0)
    assert len(set(got["kv_slot"].tolist())) == len(got["kv_slot"])


def test_pack_tables_rejects_overrun():
    with pytest.raises(oracle.OracleError):
        oracle.pack_tables([4], [14], np.zeros((1, 1), np.int32), 16)  # 14 + 4 > 16
    with pytest.raises(oracle.OracleError):
        oracle.pack_tables([-1], [0], np.zeros((1, 1), np.int32), 16)
