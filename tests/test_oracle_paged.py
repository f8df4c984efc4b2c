"""Pins the oracle's paged-KV addressing (crates/engine/src/backend/paged.rs).

Known answers are the reference's own unit tests (paged.rs:220-318); the
rest are closed forms and brute-force enumeration that a wrong index, a
swapped div/mod or an off-by-one in the coverage check would fail.
"""
import itertools

import numpy as np
import pytest

import oracle
from oracle import OracleError


# ---- paged.rs:220-228 slot_of_follows_block_table ---------------------------
def test_slot_of_kat():
    table = [7, 2, 5]
    assert oracle.slot_of(table, 0, 4) == 28  # block 7, offset 0
    assert oracle.slot_of(table, 3, 4) == 31  # block 7, offset 3
    assert oracle.slot_of(table, 4, 4) == 8   # block 2, offset 0
    assert oracle.slot_of(table, 9, 4) == 21  # block 5, offset 1


def test_slot_of_brute_force_is_a_bijection_onto_the_tables_blocks():
    rng = np.random.default_rng(5)
    for bs in (1, 2, 3, 4, 16):
        table = rng.permutation(40)[:7]
        slots = [oracle.slot_of(table, p, bs) for p in range(7 * bs)]
        # every position lands in its own block, offsets in order
        want = [int(table[p // bs]) * bs + p % bs for p in range(7 * bs)]
        assert slots == want
        assert len(set(slots)) == len(slots)
        assert sorted(s // bs for s in slots) == sorted(np.repeat(table, bs).tolist())


def test_slot_of_wraps_in_u32_like_the_reference():
    # block * bs is u32 arithmetic in the reference (paged.rs:51)
    assert oracle.slot_of([0x40000001], 3, 4) == ((0x40000001 * 4 + 3) & 0xFFFFFFFF)


# ---- paged.rs:230-261 prefill_meta_flattens_a_batch -----------------------------
def test_prefill_meta_kat():
    m = oracle.prefill_meta([(0, 5, [3, 0]), (6, 3, [1, 4, 6])], 4)
    assert m["seq_row_starts"].tolist() == [0, 5, 8]
    assert m["positions"].tolist() == [0, 1, 2, 3, 4, 6, 7, 8]
    assert m["slot_mapping"].tolist() == [12, 13, 14, 15, 0, 18, 19, 24]
    assert m["row_seq"].tolist() == [0, 0, 0, 0, 0, 1, 1, 1]
    assert m["row_num_keys"].tolist() == [1, 2, 3, 4, 5, 7, 8, 9]
    assert m["last_rows"].tolist() == [4, 7]


# ---- paged.rs:263-285 decode_meta_one_row_per_sequence --------------------------
def test_decode_meta_kat():
    m = oracle.decode_meta([(0, [9]), (6, [2, 5])], 4)
    assert m["positions"].tolist() == [0, 6]
    assert m["slot_mapping"].tolist() == [36, 22]
    assert m["row_seq"].tolist() == [0, 1]
    assert m["row_num_keys"].tolist() == [1, 7]


# ---- paged.rs:287-318 short_block_table_is_rejected -----------------------------
def test_short_block_table_kat():
    with pytest.raises(OracleError) as e:
        oracle.prefill_meta([(0, 5, [0])], 4)
    assert e.value.code == oracle.BLOCK_TABLE_TOO_SHORT
    assert (e.value.tokens, e.value.needed, e.value.have) == (5, 2, 1)
    with pytest.raises(OracleError) as e:
        oracle.decode_meta([(4, [0])], 4)
    assert e.value.needed == 2


def test_coverage_boundary_brute_force():
    # needed = ceil(tokens / bs): exactly-full tables pass, one token more fails
    for bs in (1, 3, 4, 16):
        for n_blocks in range(0, 4):
            table = list(range(n_blocks))
            for tokens in range(0, n_blocks * bs + 2):
                ok = tokens <= n_blocks * bs
                if ok:
                    if tokens:
                        oracle.prefill_meta([(0, tokens, table)], bs)
                else:
                    with pytest.raises(OracleError) as e:
                        oracle.prefill_meta([(0, tokens, table)], bs)
                    assert e.value.needed == -(-tokens // bs)
                    assert e.value.have == n_blocks


def test_prefill_meta_matches_enumeration_on_random_batches():
    rng = np.random.default_rng(11)
    for _ in range(50):
        bs = int(rng.choice([1, 2, 4, 16]))
        nseq = int(rng.integers(1, 6))
        seqs = []
        for _ in range(nseq):
            ctx, new = int(rng.integers(0, 40)), int(rng.integers(0, 20))
            nb = -(-(ctx + new) // bs) + int(rng.integers(0, 3))
            seqs.append((ctx, new, rng.integers(0, 1000, nb).tolist()))
        m = oracle.prefill_meta(seqs, bs)
        rows = [(s, p) for s, (c, n, _) in enumerate(seqs) for p in range(c, c + n)]
        assert m["positions"].tolist() == [p for _, p in rows]
        assert m["row_seq"].tolist() == [s for s, _ in rows]
        assert m["row_num_keys"].tolist() == [p + 1 for _, p in rows]
        assert m["slot_mapping"].tolist() == [seqs[s][2][p // bs] * bs + p % bs for s, p in rows]
        starts = np.concatenate([[0], np.cumsum([n for _, n, _ in seqs])])
        assert m["seq_row_starts"].tolist() == starts.tolist()


def test_prefill_row_equals_decode_row():
    # A prefill row at position p and a decode at context p address the same slot.
    table = [5, 9, 2, 7]
    for p in range(16):
        pm = oracle.prefill_meta([(p, 1, table)], 4)
        dm = oracle.decode_meta([(p, table)], 4)
        for k in ("positions", "slot_mapping", "row_num_keys"):
            assert pm[k].tolist() == dm[k].tolist()
