"""The oracle against the committed golden fixtures (tests/golden/)."""
import json
import pathlib
import sys

import numpy as np
import pytest

import oracle

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
import make_golden  # noqa: E402


def test_paged_kats_from_fixture():
    k = json.loads((GOLDEN / "paged_kats.json").read_text())
    s = k["slot_of"]
    for pos, want in s["cases"]:
        assert oracle.slot_of(s["table"], pos, s["block_size"]) == want
    p = k["prefill_meta"]
    m = oracle.prefill_meta([tuple(x) for x in p["seqs"]], p["block_size"])
    for key in ("seq_row_starts", "positions", "slot_mapping", "row_seq", "row_num_keys",
                "last_rows"):
        assert m[key].tolist() == p[key], key
    d = k["decode_meta"]
    m = oracle.decode_meta([tuple(x) for x in d["seqs"]], d["block_size"])
    for key in ("positions", "slot_mapping", "row_seq", "row_num_keys"):
        assert m[key].tolist() == d[key], key
    sp = k["short_table"]["prefill"]
    with pytest.raises(oracle.OracleError) as e:
        oracle.prefill_meta([tuple(x) for x in sp["seqs"]], sp["block_size"])
    assert (e.value.tokens, e.value.needed, e.value.have) == (sp["tokens"], sp["needed"], sp["have"])


@pytest.mark.parametrize("kind", ["prefill", "decode"])
def test_attention_scenarios_from_fixture(kind):
    g = np.load(GOLDEN / "attention_scenarios.npz")
    now = make_golden.scenario(kind)
    # inputs regenerate exactly; outputs agree to f32 round-off (glibc may pick
    # a different expf variant on another host, so not bitwise)
    for key in ("q", "k", "v", "row_seq", "row_num_keys"):
        assert np.array_equal(now[key], g[f"{kind}_{key}"]), key
    assert oracle.max_rel_diff(now["out"], g[f"{kind}_out"]) < 1e-6
    assert oracle.max_rel_diff(g[f"{kind}_out"], g[f"{kind}_naive"]) < 1e-5
