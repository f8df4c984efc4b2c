"""Writes the golden fixtures of tests/golden/ (run from the repository root:
`python tests/golden/make_golden.py`).

* paged_kats.json -- the known answers of the reference's paged.rs unit tests
  (crates/engine/src/backend/paged.rs:220-318), as data.
* attention_scenarios.npz -- the reference's two paged-attention scenarios
  (crates/engine/src/backend/cpu/tests.rs:232-334): inputs regenerated from
  the restated LCG, the oracle's f32 outputs and the naive f64 outputs.

The reference itself (Rust) cannot run here; the outputs are the oracle's,
pinned by tests/test_oracle_attention.py.  The fixtures catch regressions of
the oracle build (flags, compiler) and give GPU-free known answers.
"""
import json
import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
import oracle  # noqa: E402

HEADS, KV_HEADS, HD, BS, NUM_BLOCKS = 6, 2, 8, 4, 16
W = KV_HEADS * HD


def kats():
    return {
        "slot_of": {"table": [7, 2, 5], "block_size": 4,
                    "cases": [[0, 28], [3, 31], [4, 8], [9, 21]]},
        "prefill_meta": {"seqs": [[0, 5, [3, 0]], [6, 3, [1, 4, 6]]], "block_size": 4,
                         "seq_row_starts": [0, 5, 8], "positions": [0, 1, 2, 3, 4, 6, 7, 8],
                         "slot_mapping": [12, 13, 14, 15, 0, 18, 19, 24],
                         "row_seq": [0, 0, 0, 0, 0, 1, 1, 1],
                         "row_num_keys": [1, 2, 3, 4, 5, 7, 8, 9], "last_rows": [4, 7]},
        "decode_meta": {"seqs": [[0, [9]], [6, [2, 5]]], "block_size": 4,
                        "positions": [0, 6], "slot_mapping": [36, 22], "row_seq": [0, 1],
                        "row_num_keys": [1, 7]},
        "short_table": {"prefill": {"seqs": [[0, 5, [0]]], "block_size": 4, "tokens": 5,
                                    "needed": 2, "have": 1},
                        "decode": {"seqs": [[4, [0]]], "block_size": 4, "needed": 2}},
    }


def scenario(kind):
    if kind == "prefill":
        shape = [(5, 6), (0, 3), (8, 4)]
        tables = [[9, 2, 14], [7], [0, 11, 5]]
        kvs = [(oracle.rand_vec(100 + i, (c + n) * W), oracle.rand_vec(200 + i, (c + n) * W))
               for i, (c, n) in enumerate(shape)]
        meta = oracle.prefill_meta([(c, n, t) for (c, n), t in zip(shape, tables)], BS)
        q = oracle.rand_vec(300, len(meta["positions"]) * HEADS * HD).reshape(-1, HEADS * HD)
        lens = [c + n for c, n in shape]
        layer = 1
    else:
        ctx = [0, 3, 10]
        tables = [[15], [4], [12, 1, 8]]
        kvs = [(oracle.rand_vec(400 + i, (c + 1) * W), oracle.rand_vec(500 + i, (c + 1) * W))
               for i, c in enumerate(ctx)]
        meta = oracle.decode_meta([(c, t) for c, t in zip(ctx, tables)], BS)
        q = oracle.rand_vec(600, 3 * HEADS * HD).reshape(3, HEADS * HD)
        lens = [c + 1 for c in ctx]
        layer = 0
    pool = oracle.Pool(2, NUM_BLOCKS, BS, KV_HEADS, HD)
    for i, n in enumerate(lens):
        slots = [oracle.slot_of(tables[i], p, BS) for p in range(n)]
        pool.write_kv(layer, kvs[i][0].reshape(-1, W), kvs[i][1].reshape(-1, W), slots)
    out = pool.attention(q, layer, tables, meta["row_seq"], meta["row_num_keys"], threads=1)
    naive = []
    for row in range(q.shape[0]):
        s = int(meta["row_seq"][row])
        pos = int(meta["row_num_keys"][row]) - 1
        naive.append(oracle.naive_attend_f64(q[row], *kvs[s], pos, HEADS, KV_HEADS, HD))
    return dict(q=q, out=out, naive=np.stack(naive),
                k=np.concatenate([k for k, _ in kvs]), v=np.concatenate([v for _, v in kvs]),
                row_seq=np.asarray(meta["row_seq"]), row_num_keys=np.asarray(meta["row_num_keys"]))


def main():
    (HERE / "paged_kats.json").write_text(json.dumps(kats(), indent=1) + "\n")
    arrays = {}
    for kind in ("prefill", "decode"):
        for k, v in scenario(kind).items():
            arrays[f"{kind}_{k}"] = v
    np.savez_compressed(HERE / "attention_scenarios.npz", **arrays)
    print("wrote", sorted(p.name for p in HERE.iterdir() if p.suffix in (".json", ".npz")))


if __name__ == "__main__":
    main()
