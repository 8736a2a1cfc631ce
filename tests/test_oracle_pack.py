"""Pins the oracle's step packing (Engine::step, src/engine.rs:376-402) and table
padding (PaddedDecodeTables, src/model.rs:71-111)."""
import numpy as np
import pytest

import oracle


def test_hand_packed_step():
    bs = 4
    # decode at position 5 (table [7, 3]); chunk of 3 starting at 0 (table [9]);
    # chunk of 2 starting at 6 (table [1, 2]) -- plan order as given.
    tables = np.array([7, 3, 9, 1, 2], np.uint32)
    tokens = np.arange(100, 130, dtype=np.uint32)  # arena: seq histories back to back
    plan = np.array([[5, 1, 0, 2, 0],
                     [0, 3, 2, 1, 10],
                     [6, 2, 3, 2, 20]], np.uint32)
    out = oracle.pack_step(plan, tokens, tables, bs)
    np.testing.assert_array_equal(out["cu_seqlens"], [0, 1, 4, 6])
    np.testing.assert_array_equal(out["positions"], [5, 0, 1, 2, 6, 7])
    np.testing.assert_array_equal(out["seq_of_query"], [0, 1, 1, 1, 2, 2])
    np.testing.assert_array_equal(out["tokens"], [105, 110, 111, 112, 126, 127])
    # slot = table[pos // bs] * bs + pos % bs
    np.testing.assert_array_equal(out["slot_mapping"], [3 * 4 + 1, 36, 37, 38, 2 * 4 + 2, 2 * 4 + 3])
    np.testing.assert_array_equal(out["context_lens"], [6, 3, 8])
    # max_blocks = max ceil(ctx/bs) = 2; short table padded with its last needed block
    assert out["max_blocks"] == 2
    np.testing.assert_array_equal(out["block_tables"].reshape(3, 2), [[7, 3], [9, 9], [1, 2]])


def test_random_plans_invariants():
    rng = np.random.default_rng(0)
    for _ in range(50):
        bs = int(rng.choice([2, 4, 16]))
        S = int(rng.integers(1, 30))
        plan, tables, off = [], [], 0
        for s in range(S):
            q_len = 1 if rng.random() < 0.6 else int(rng.integers(2, 40))
            start = int(rng.integers(0, 200))
            need = (start + q_len + bs - 1) // bs
            extra = int(rng.integers(0, 3))
            tables.extend(rng.integers(0, 10000, need + extra))
            plan.append([start, q_len, off, need + extra, s * 300])
            off += need + extra
        plan = np.array(plan, np.uint32)
        tables = np.array(tables, np.uint32)
        arena = rng.integers(0, 50000, S * 300).astype(np.uint32)
        out = oracle.pack_step(plan, arena, tables, bs)
        cu = out["cu_seqlens"]
        assert (np.diff(cu) == plan[:, 1]).all()
        for s in range(S):
            st, ql, to, tl, ko = (int(v) for v in plan[s])
            tab = tables[to:to + tl]
            rows = slice(cu[s], cu[s + 1])
            pos = np.arange(st, st + ql)
            np.testing.assert_array_equal(out["positions"][rows], pos)
            np.testing.assert_array_equal(out["slot_mapping"][rows], tab[pos // bs].astype(np.int64) * bs + pos % bs)
            np.testing.assert_array_equal(out["tokens"][rows], arena[ko + pos])
            need = max((st + ql + bs - 1) // bs, 1)
            row = out["block_tables"].reshape(S, -1)[s]
            np.testing.assert_array_equal(row[:need], tab[:need])
            assert (row[need:] == tab[need - 1]).all()


def test_short_table_is_an_error():
    plan = np.array([[15, 2, 0, 1, 0]], np.uint32)  # positions 15, 16 need 2 blocks of 16
    with pytest.raises(ValueError):
        oracle.pack_step(plan, np.zeros(64, np.uint32), np.array([3], np.uint32), 16)
