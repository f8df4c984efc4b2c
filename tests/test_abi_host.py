"""C-ABI library on the host (no GPU needed).

* libvo_paged_attention.so loads and exports every function that
  include/*.h declares;
* the product's own restatement of paged.rs (slot_of, PrefillMeta::new,
  DecodeMeta::new, last_rows) matches the oracle bit for bit, including the
  reference's known answers (paged.rs:220-318) and its error fields.
"""
import ctypes
import pathlib
import re

import numpy as np
import pytest

import oracle

ROOT = pathlib.Path(__file__).resolve().parents[1]


def _declared_functions():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"\b(vo_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return sorted(names)


def test_library_exports_every_declared_symbol(vo):
    declared = _declared_functions()
    assert len(declared) >= 20
    missing = [n for n in declared if not hasattr(vo.lib, n)]
    assert not missing, missing
    # and the Python binding types every one of them
    assert set(declared) == set(vo.SIGNATURES)


def test_integration_extern_block_binds_every_declared_function():
    """The Rust FFI block of the integration guide (section 2) has one
    `pub fn` per function the header declares, and no other."""
    text = (ROOT / "INTEGRATION.md").read_text()
    start = text.index("## 2.")
    block = text[start:text.index("## 3.", start)]
    bound = set(re.findall(r"pub fn (vo_[a-z0-9_]+)\(", block))
    assert bound == set(_declared_functions())
    statuses = set(re.findall(r"pub const (VO_(?:OK|ERR_[A-Z_]+)): i32", block))
    header = (ROOT / "include" / "vo_paged_attention.h").read_text()
    enum = header[header.index("typedef enum vo_status"):header.index("} vo_status;")]
    assert statuses == set(re.findall(r"\b(VO_(?:OK|ERR_[A-Z_]+)) =", enum))


def test_version_and_status_names(vo):
    assert b"gfx950" in vo.lib.vo_version()
    assert vo.lib.vo_status_name(vo.VO_ERR_BLOCK_OUT_OF_RANGE) == b"VO_ERR_BLOCK_OUT_OF_RANGE"


def test_layout_helpers(vo):
    L = vo.KvLayout(num_layers=2, num_blocks=20000, block_size=16, kv_heads=8, head_dim=128)
    assert L.num_slots() == 320000
    assert L.layer_elems() == 320000 * 8 * 128


# ---- paged.rs known answers through the product library -----------------------
def test_slot_of_kat(vo):
    table = [7, 2, 5]
    assert [vo.slot_of(table, p, 4) for p in (0, 3, 4, 9)] == [28, 31, 8, 21]


def test_slot_of_past_table_is_an_error(vo):
    with pytest.raises(vo.BlockTableTooShort) as e:
        vo.slot_of([7, 2, 5], 12, 4)
    assert (e.value.needed, e.value.have) == (4, 3)


def test_prefill_meta_kat(vo):
    m = vo.PrefillMeta.new([vo.PrefillSeq(0, 5, [3, 0]), vo.PrefillSeq(6, 3, [1, 4, 6])], 4)
    assert m.seq_row_starts.tolist() == [0, 5, 8]
    assert m.positions.tolist() == [0, 1, 2, 3, 4, 6, 7, 8]
    assert m.slot_mapping.tolist() == [12, 13, 14, 15, 0, 18, 19, 24]
    assert m.row_seq.tolist() == [0, 0, 0, 0, 0, 1, 1, 1]
    assert m.row_num_keys.tolist() == [1, 2, 3, 4, 5, 7, 8, 9]
    assert m.last_rows().tolist() == [4, 7]


def test_decode_meta_kat(vo):
    m = vo.DecodeMeta.new([vo.DecodeSeq(0, [9]), vo.DecodeSeq(6, [2, 5])], 4)
    assert m.positions.tolist() == [0, 6]
    assert m.slot_mapping.tolist() == [36, 22]
    assert m.row_seq.tolist() == [0, 1]
    assert m.row_num_keys.tolist() == [1, 7]


def test_short_block_table_error_fields(vo):
    with pytest.raises(vo.BlockTableTooShort) as e:
        vo.PrefillMeta.new([vo.PrefillSeq(0, 5, [0])], 4)
    err = e.value
    assert (err.op, err.tokens, err.needed, err.have) == ("prefill", 5, 2, 1)
    assert err.message == "prefill: block table too short: 5 tokens need 2 blocks, table has 1"
    with pytest.raises(vo.BlockTableTooShort) as e:
        vo.DecodeMeta.new([vo.DecodeSeq(4, [0])], 4)
    assert (e.value.op, e.value.needed) == ("decode", 2)


# ---- bit-exact against the oracle on random batches ---------------------------
def test_metadata_bit_exact_vs_oracle_random(vo):
    rng = np.random.default_rng(2024)
    for trial in range(200):
        bs = int(rng.choice([1, 2, 4, 16, 32]))
        nseq = int(rng.integers(0, 9))
        pseqs, dseqs = [], []
        for _ in range(nseq):
            ctx, new = int(rng.integers(0, 300)), int(rng.integers(0, 40))
            # covers ctx + new for prefill and ctx + 1 for decode
            nb = -(-(ctx + max(new, 1)) // bs) + int(rng.integers(0, 2))
            table = rng.integers(0, 1 << 20, max(nb, 1)).tolist()
            pseqs.append((ctx, new, table))
            dseqs.append((ctx, table))
        got = vo.PrefillMeta.new([vo.PrefillSeq(c, n, t) for c, n, t in pseqs], bs)
        want = oracle.prefill_meta(pseqs, bs)
        for k in ("seq_row_starts", "positions", "slot_mapping", "row_seq", "row_num_keys"):
            assert np.array_equal(getattr(got, k).astype(np.uint64), want[k].astype(np.uint64)), k
        if nseq and all(new > 0 for _, new, _ in pseqs):
            assert np.array_equal(got.last_rows(), want["last_rows"])
        gd = vo.DecodeMeta.new([vo.DecodeSeq(c, t) for c, t in dseqs], bs)
        wd = oracle.decode_meta(dseqs, bs)
        for k in ("positions", "slot_mapping", "row_seq", "row_num_keys"):
            assert np.array_equal(getattr(gd, k).astype(np.uint64), wd[k].astype(np.uint64)), k


def test_metadata_errors_match_oracle(vo):
    rng = np.random.default_rng(7)
    for _ in range(100):
        bs = int(rng.choice([2, 4, 16]))
        seqs = [(int(rng.integers(0, 50)), int(rng.integers(1, 30)),
                 rng.integers(0, 99, int(rng.integers(0, 6))).tolist()) for _ in range(3)]
        try:
            want = oracle.prefill_meta(seqs, bs)
            want_err = None
        except oracle.OracleError as e:
            want_err = e
        try:
            vo.PrefillMeta.new([vo.PrefillSeq(*s) for s in seqs], bs)
            got_err = None
        except vo.BlockTableTooShort as e:
            got_err = e
        assert (want_err is None) == (got_err is None)
        if got_err is not None:
            assert (got_err.seq, got_err.tokens, got_err.needed, got_err.have) == (
                want_err.seq, want_err.tokens, want_err.needed, want_err.have)


def test_step_metas_are_immutable(vo):
    """A PrefillMeta / DecodeMeta holds read-only copies of its arrays and
    rejects attribute assignment, so HipBackend's one upload per meta object
    cannot go stale; a changed step is a new object (dataclasses.replace)."""
    import dataclasses
    table = np.array([3, 1], np.uint32)
    pm = vo.PrefillMeta.new([vo.PrefillSeq(5, 4, table)], 16)
    dm = vo.DecodeMeta.new([vo.DecodeSeq(20, table)], 16)
    table[0] = 7  # the caller's array is not the meta's
    assert pm.block_tables[0][0] == 3 and dm.block_tables[0][0] == 3
    for meta in (pm, dm):
        for name in ("positions", "slot_mapping", "row_seq", "row_num_keys"):
            with pytest.raises(ValueError):
                getattr(meta, name)[0] = 1
        with pytest.raises(ValueError):
            meta.block_tables[0][0] = 1
        with pytest.raises(dataclasses.FrozenInstanceError):
            meta.positions = np.zeros(1, np.uint32)
    changed = dataclasses.replace(pm, slot_mapping=[80, 81, 82, 83])
    assert changed is not pm and list(changed.slot_mapping) == [80, 81, 82, 83]
    assert not changed.slot_mapping.flags.writeable

