"""Pins the oracle's CPU attention (crates/engine/src/backend/cpu/attention.rs,
cpu/mod.rs dot/write_kv) and its test helpers (testutil.rs).

* The reference's own scenarios (cpu/tests.rs:232-334), with inputs regenerated
  from the restated LCG, against the reference's naive f64 oracle
  (cpu/tests.rs:184-208) at the reference's tolerance, max_rel_diff < 1e-5.
* An independent numpy float64 attention (vectorised, dense softmax), so the
  naive oracle is not the only check.
* Closed forms and invariants: a single key returns V exactly, identical keys
  return the mean of V, prefill row p == decode at context p bitwise,
  batch invariance bitwise, block relabelling invariance, aliased tables.
* Error classes of cpu/tests.rs:336-362.
"""
import math

import numpy as np
import pytest

import oracle
from oracle import OracleError

HEADS, KV_HEADS, HD, BS, NUM_BLOCKS = 6, 2, 8, 4, 16  # cpu/tests.rs:161-165
W = KV_HEADS * HD


# ---- testutil.rs ------------------------------------------------------------
def _lcg_bigint(seed, n):
    """testutil.rs:34-44 restated with Python integers (explicit mod 2^64)."""
    M = 1 << 64
    s = (seed * 0x9E3779B97F4A7C15 + 1) % M
    out = []
    for _ in range(n):
        s = (s * 6364136223846793005 + 1442695040888963407) % M
        out.append(np.float32((s >> 40) / float(1 << 24)) * np.float32(2.0) - np.float32(1.0))
    return np.array(out, np.float32)


def test_rand_vec_matches_bigint_restatement_and_range():
    for seed in (0, 1, 7, 300, 2**63 + 5):
        v = oracle.rand_vec(seed, 257)
        assert np.array_equal(v, _lcg_bigint(seed, 257))
        assert v.min() >= -1.0 and v.max() < 1.0
        # values are k/2^23 - 1 for integer k (24 random bits scaled into [-1, 1))
        k = (v.astype(np.float64) + 1.0) * 2**23
        assert np.array_equal(k, np.round(k))
    big = oracle.rand_vec(42, 200_000)
    assert abs(big.mean()) < 0.01 and abs(big.var() - 1 / 3) < 0.01


def test_max_rel_diff_closed_form():
    a = np.array([1.0, 2.0, -3.0], np.float32)
    b = np.array([1.5, 2.0, -4.0], np.float32)
    assert oracle.max_rel_diff(a, b) == pytest.approx(1.0 / 4.0)
    assert oracle.max_rel_diff(np.zeros(3), np.zeros(3)) == 0.0


# ---- cpu/tests.rs:27-34 dot_matches_naive_for_odd_lengths -------------------------
@pytest.mark.parametrize("n", [0, 1, 15, 16, 17, 33, 2048])
def test_dot_matches_naive(n):
    a, b = oracle.rand_vec(1, n), oracle.rand_vec(2, n)
    want = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
    assert abs(oracle.dot(a, b) - want) < 1e-4


def test_dot_lane_order_is_the_references():
    # 16 partial sums, summed in lane order, then the remainder (cpu/mod.rs:95-110).
    a, b = oracle.rand_vec(3, 37), oracle.rand_vec(4, 37)
    partial = np.zeros(16, np.float32)
    for c in range(2):
        partial = partial + a[16 * c:16 * c + 16] * b[16 * c:16 * c + 16]
    s = np.float32(-0.0)
    for x in partial:
        s = np.float32(s + x)
    for i in range(32, 37):
        s = np.float32(s + np.float32(a[i] * b[i]))
    assert oracle.dot(a, b) == s


# ---- the reference scenarios ----------------------------------------------------
def _write_positions(pool, layer, k, v, table, lo, hi):
    """cpu/tests.rs:210-230."""
    if hi <= lo:
        return
    slots = [oracle.slot_of(table, p, BS) for p in range(lo, hi)]
    pool.write_kv(layer, k[lo * W:hi * W].reshape(-1, W), v[lo * W:hi * W].reshape(-1, W), slots)


def _numpy_attention_f64(q, k, v, pos, heads, kv_heads, hd):
    """Dense float64 attention for one row over a contiguous sequence."""
    group = heads // kv_heads
    q = q.reshape(heads, hd).astype(np.float64)
    k = k.reshape(-1, kv_heads, hd)[: pos + 1].astype(np.float64)
    v = v.reshape(-1, kv_heads, hd)[: pos + 1].astype(np.float64)
    out = np.zeros((heads, hd))
    for h in range(heads):
        s = k[:, h // group, :] @ q[h] / math.sqrt(hd)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ v[:, h // group, :]
    return out.ravel().astype(np.float32)


def prefill_scenario():
    """cpu/tests.rs:232-292: shapes, tables and seeds of the reference test."""
    shape = [(5, 6), (0, 3), (8, 4)]
    tables = [[9, 2, 14], [7], [0, 11, 5]]
    kvs = [(oracle.rand_vec(100 + i, (c + n) * W), oracle.rand_vec(200 + i, (c + n) * W))
           for i, (c, n) in enumerate(shape)]
    meta = oracle.prefill_meta([(c, n, t) for (c, n), t in zip(shape, tables)], BS)
    t_rows = len(meta["positions"])
    q = oracle.rand_vec(300, t_rows * HEADS * HD).reshape(t_rows, HEADS * HD)
    return shape, tables, kvs, meta, q


def decode_scenario():
    """cpu/tests.rs:294-334."""
    ctx = [0, 3, 10]
    tables = [[15], [4], [12, 1, 8]]
    kvs = [(oracle.rand_vec(400 + i, (c + 1) * W), oracle.rand_vec(500 + i, (c + 1) * W))
           for i, c in enumerate(ctx)]
    meta = oracle.decode_meta([(c, t) for c, t in zip(ctx, tables)], BS)
    q = oracle.rand_vec(600, 3 * HEADS * HD).reshape(3, HEADS * HD)
    return ctx, tables, kvs, meta, q


def test_paged_prefill_attention_matches_naive_with_shuffled_blocks():
    shape, tables, kvs, meta, q = prefill_scenario()
    pool = oracle.Pool(2, NUM_BLOCKS, BS, KV_HEADS, HD)
    layer = 1
    for i, (c, n) in enumerate(shape):
        _write_positions(pool, layer, *kvs[i], tables[i], 0, c)
        _write_positions(pool, layer, *kvs[i], tables[i], c, c + n)
    got = pool.attention(q, layer, tables, meta["row_seq"], meta["row_num_keys"])
    want, want_np = [], []
    for i, (c, n) in enumerate(shape):
        for j in range(n):
            row = int(meta["seq_row_starts"][i]) + j
            want.append(oracle.naive_attend_f64(q[row], *kvs[i], c + j, HEADS, KV_HEADS, HD))
            want_np.append(_numpy_attention_f64(q[row], *kvs[i], c + j, HEADS, KV_HEADS, HD))
    assert oracle.max_rel_diff(got, np.stack(want)) < 1e-5
    assert oracle.max_rel_diff(got, np.stack(want_np)) < 1e-5
    # the two f64 oracles agree far below the f32 tolerance
    assert oracle.max_rel_diff(np.stack(want), np.stack(want_np)) < 1e-6


def test_paged_decode_attention_matches_naive_with_shuffled_blocks():
    ctx, tables, kvs, meta, q = decode_scenario()
    pool = oracle.Pool(2, NUM_BLOCKS, BS, KV_HEADS, HD)
    for i, c in enumerate(ctx):
        _write_positions(pool, 0, *kvs[i], tables[i], 0, c + 1)
    got = pool.attention(q, 0, tables, meta["row_seq"], meta["row_num_keys"])
    want = np.stack([oracle.naive_attend_f64(q[i], *kvs[i], ctx[i], HEADS, KV_HEADS, HD)
                     for i in range(3)])
    want_np = np.stack([_numpy_attention_f64(q[i], *kvs[i], ctx[i], HEADS, KV_HEADS, HD)
                        for i in range(3)])
    assert oracle.max_rel_diff(got, want) < 1e-5
    assert oracle.max_rel_diff(got, want_np) < 1e-5


def test_single_key_returns_v0_exactly():
    # exp(0) = 1, 1/1 = 1: the output is V[0] bit for bit, for every head of the group.
    _, tables, kvs, meta, q = decode_scenario()
    pool = oracle.Pool(1, NUM_BLOCKS, BS, KV_HEADS, HD)
    _write_positions(pool, 0, *kvs[0], tables[0], 0, 1)
    got = pool.attention(q[:1], 0, tables[:1], [0], [1])
    v0 = kvs[0][1][:W].reshape(KV_HEADS, HD)
    want = np.concatenate([v0[h // (HEADS // KV_HEADS)] for h in range(HEADS)])
    assert np.array_equal(got[0], want)


def test_identical_keys_give_the_mean_of_values():
    pool = oracle.Pool(1, 4, BS, KV_HEADS, HD)
    n = 11
    table = [3, 1, 2]
    k = np.tile(oracle.rand_vec(9, W), n).reshape(n, W)
    v = oracle.rand_vec(10, n * W).reshape(n, W)
    pool.write_kv(0, k, v, [oracle.slot_of(table, p, BS) for p in range(n)])
    q = oracle.rand_vec(11, HEADS * HD).reshape(1, -1)
    got = pool.attention(q, 0, [table], [0], [n])[0].reshape(HEADS, HD)
    mean = v.reshape(n, KV_HEADS, HD).astype(np.float64).mean(0)
    for h in range(HEADS):
        np.testing.assert_allclose(got[h], mean[h // 3], rtol=1e-5, atol=1e-6)


def test_prefill_row_equals_decode_bitwise():
    shape, tables, kvs, meta, q = prefill_scenario()
    pool = oracle.Pool(1, NUM_BLOCKS, BS, KV_HEADS, HD)
    for i, (c, n) in enumerate(shape):
        _write_positions(pool, 0, *kvs[i], tables[i], 0, c + n)
    full = pool.attention(q, 0, tables, meta["row_seq"], meta["row_num_keys"])
    for row in range(q.shape[0]):
        s = int(meta["row_seq"][row])
        one = pool.attention(q[row:row + 1], 0, [tables[s]], [0], [meta["row_num_keys"][row]])
        assert np.array_equal(one[0], full[row])


def test_batch_invariance_and_thread_count_invariance_bitwise():
    shape, tables, kvs, meta, q = prefill_scenario()
    pool = oracle.Pool(1, NUM_BLOCKS, BS, KV_HEADS, HD)
    for i, (c, n) in enumerate(shape):
        _write_positions(pool, 0, *kvs[i], tables[i], 0, c + n)
    a = pool.attention(q, 0, tables, meta["row_seq"], meta["row_num_keys"], threads=1)
    b = pool.attention(q, 0, tables, meta["row_seq"], meta["row_num_keys"], threads=7)
    assert np.array_equal(a, b)


def test_block_relabelling_and_aliasing_do_not_change_outputs():
    rng = np.random.default_rng(3)
    n = 29
    k = oracle.rand_vec(21, n * W).reshape(n, W)
    v = oracle.rand_vec(22, n * W).reshape(n, W)
    q = oracle.rand_vec(23, 2 * HEADS * HD).reshape(2, -1)
    outs = []
    for _ in range(3):
        table = rng.permutation(NUM_BLOCKS)[:8].tolist()
        pool = oracle.Pool(1, NUM_BLOCKS, BS, KV_HEADS, HD)
        pool.write_kv(0, k, v, [oracle.slot_of(table, p, BS) for p in range(n)])
        # two rows aliasing the same table (prefix sharing) == two copies of it
        outs.append(pool.attention(q, 0, [table, list(table)], [0, 1], [n, n]))
        alias = pool.attention(q, 0, [table], [0, 0], [n, n])
        assert np.array_equal(alias, outs[-1])
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[1], outs[2])


# ---- cpu/tests.rs:336-362 out_of_range_blocks_and_slots_are_errors ---------------
def test_out_of_range_blocks_and_slots_are_errors():
    pool = oracle.Pool(2, NUM_BLOCKS, BS, KV_HEADS, HD)
    q = oracle.rand_vec(1, HEADS * HD).reshape(1, -1)
    with pytest.raises(OracleError) as e:
        pool.attention(q, 0, [[NUM_BLOCKS]], [0], [1])
    assert e.value.code == oracle.BLOCK_OUT_OF_RANGE
    assert (e.value.value, e.value.limit) == (NUM_BLOCKS, NUM_BLOCKS)
    k = oracle.rand_vec(1, W).reshape(1, W)
    v = oracle.rand_vec(2, W).reshape(1, W)
    with pytest.raises(OracleError) as e:
        pool.write_kv(0, k, v, [NUM_BLOCKS * BS])
    assert e.value.code == oracle.SLOT_OUT_OF_RANGE
    assert (e.value.value, e.value.limit) == (NUM_BLOCKS * BS, NUM_BLOCKS * BS)


def test_block_check_covers_whole_table_not_just_used_prefix():
    # attention.rs:132-147 scans every entry, even past the keys a row reads.
    pool = oracle.Pool(1, NUM_BLOCKS, BS, KV_HEADS, HD)
    q = oracle.rand_vec(1, HEADS * HD).reshape(1, -1)
    with pytest.raises(OracleError):
        pool.attention(q, 0, [[0, 1, 99]], [0], [1])


def test_write_kv_checks_all_slots_before_writing_and_later_row_wins():
    pool = oracle.Pool(1, NUM_BLOCKS, BS, KV_HEADS, HD)
    k = oracle.rand_vec(5, 3 * W).reshape(3, W)
    v = oracle.rand_vec(6, 3 * W).reshape(3, W)
    with pytest.raises(OracleError):
        pool.write_kv(0, k, v, [1, 2, NUM_BLOCKS * BS + 7])
    assert not pool.keys[0].any()  # nothing written
    pool.write_kv(0, k, v, [5, 9, 5])
    assert np.array_equal(pool.keys[0][5], k[2]) and np.array_equal(pool.keys[0][9], k[1])


# ---- split-K combine ----------------------------------------------------------------
def test_splitk_combine_identity_and_equals_one_pass():
    rng = np.random.default_rng(8)
    hd, n = 16, 40
    s = rng.standard_normal(n)
    vv = rng.standard_normal((n, hd))
    p = np.exp(s - s.max())
    whole = (p / p.sum()) @ vv
    # one split: identity
    m1 = np.array([s.max()], np.float32)
    l1 = np.array([p.sum()], np.float32)
    a1 = (p @ vv)[None].astype(np.float32)
    np.testing.assert_allclose(oracle.splitk_combine(m1, l1, a1), whole, rtol=1e-5, atol=1e-6)
    # uneven splits, plus an empty one (m = -inf)
    cuts = [0, 3, 17, 17, 40]
    ms, ls, accs = [], [], []
    for a, b in zip(cuts, cuts[1:]):
        if a == b:
            ms.append(-np.inf); ls.append(0.0); accs.append(np.zeros(hd)); continue
        mm = s[a:b].max()
        pp = np.exp(s[a:b] - mm)
        ms.append(mm); ls.append(pp.sum()); accs.append(pp @ vv[a:b])
    got = oracle.splitk_combine(np.array(ms, np.float32), np.array(ls, np.float32),
                                np.array(accs, np.float32))
    np.testing.assert_allclose(got, whole, rtol=1e-5, atol=1e-6)
