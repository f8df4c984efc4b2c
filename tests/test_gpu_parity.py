"""GPU parity: the HIP path through the C ABI against the CPU oracle.

Bars:
* slot mappings and block gathers: bit-exact;
* attention outputs: |gpu - oracle| <= atol + rtol*|oracle| with rtol 1e-2,
  atol 2e-3 (bf16 I/O, fp32 accumulation), on identical seeded inputs.
Plus size-independent properties at full BASELINE sizes: batch invariance and
block-relabelling invariance (bitwise), single key -> V exactly.
"""
import os

import numpy as np
import pytest

import oracle as orc
import workloads as W

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-2, 2e-3


def _say(msg):
    print(f"[gpu-test] {msg}", flush=True)


def _assert_close(got, want, what):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    err = np.abs(got - want)
    bad = err > ATOL + RTOL * np.abs(want)
    assert not np.isnan(got).any(), f"{what}: NaN in GPU output"
    assert not bad.any(), (f"{what}: {bad.sum()} of {bad.size} outside rtol {RTOL}/atol {ATOL}; "
                           f"max err {err.max():.3e}")


def _bits(t):
    import torch
    return t.contiguous().view(torch.int16).cpu().numpy()


def _out(wl, backend):
    if wl.kind == "decode":
        return backend.decode_attention(wl.q, wl.pool, wl.layer, wl.meta)
    return backend.prefill_attention(wl.q, wl.pool, wl.layer, wl.meta)


# ---------------------------------------------------------------------------
# reshape_and_cache + gather: bit-exact
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("hd,bs,kvh", [(128, 16, 8), (64, 16, 2), (8, 4, 2), (96, 8, 3)])
def test_reshape_and_cache_and_gather_bit_exact(vo, gpu_backend, hd, bs, kvh):
    import torch
    _say(f"reshape_and_cache hd={hd} bs={bs} kvh={kvh}")
    wl = W.build(vo, gpu_backend, kind="prefill", heads=kvh, kv_heads=kvh, head_dim=hd,
                 block_size=bs, num_blocks=97, context_lens=[0, 5, 33, 16],
                 num_new=[3, 11, 7, 17], seed=hd + bs, layer=1, num_layers=2)
    # slot mapping from the product equals the oracle's, bit for bit
    want_meta = orc.prefill_meta([(int(c), int(n), t) for c, n, t in
                                  zip(wl.context_lens, wl.num_new, wl.tables)], bs)
    assert np.array_equal(wl.meta.slot_mapping, want_meta["slot_mapping"])
    row = 0
    for s in range(len(wl.tables)):
        c, n = int(wl.context_lens[s]), int(wl.num_new[s])
        k, v = gpu_backend.read_kv(wl.pool, 1, wl.meta, s, c + n)
        want_k = torch.cat([wl.ctx_kv[s][0], wl.k_new[row:row + n]])
        want_v = torch.cat([wl.ctx_kv[s][1], wl.v_new[row:row + n]])
        assert np.array_equal(_bits(k), _bits(want_k)), f"K of seq {s}"
        assert np.array_equal(_bits(v), _bits(want_v)), f"V of seq {s}"
        row += n
    # layer 0 was never written: still the zero fill
    k0, v0 = gpu_backend.read_kv(wl.pool, 0, wl.meta, 1, 5)
    assert not _bits(k0).any() and not _bits(v0).any()


def test_write_kv_later_row_wins_on_repeated_slot(vo, gpu_backend):
    import torch
    _say("write_kv duplicate slots")
    layout = vo.KvLayout(1, 8, 16, 2, 64)
    pool = gpu_backend.alloc_kv_pool(layout)
    g = torch.Generator(device="cuda:0").manual_seed(9)
    k = torch.randn((3, 128), generator=g, device="cuda:0").to(torch.bfloat16)
    v = torch.randn((3, 128), generator=g, device="cuda:0").to(torch.bfloat16)
    gpu_backend.write_kv(pool, 0, k, v, [5, 9, 5])
    meta = vo.DecodeMeta.new([vo.DecodeSeq(15, [0])], 16)  # covers slots 0..15 of block 0
    kk, vv = gpu_backend.read_kv(pool, 0, meta, 0, 16)
    assert np.array_equal(_bits(kk[5]), _bits(k[2])) and np.array_equal(_bits(kk[9]), _bits(k[1]))
    assert np.array_equal(_bits(vv[5]), _bits(v[2]))


# ---------------------------------------------------------------------------
# The reference's own scenarios (cpu/tests.rs:232-334) on the generic kernel
# ---------------------------------------------------------------------------
def _bf16_round(x):
    import torch
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.bfloat16)


def test_reference_prefill_scenario(vo, gpu_backend):
    """cpu/tests.rs:232-292: H 6, KVH 2, hd 8, bs 4, layer 1, shuffled tables."""
    import torch
    _say("reference prefill scenario (hd 8, bs 4)")
    H, KVH, HD, BS, NB = 6, 2, 8, 4, 16
    Wd = KVH * HD
    shape = [(5, 6), (0, 3), (8, 4)]
    tables = [[9, 2, 14], [7], [0, 11, 5]]
    kvs = [(_bf16_round(orc.rand_vec(100 + i, (c + n) * Wd).reshape(-1, Wd)),
            _bf16_round(orc.rand_vec(200 + i, (c + n) * Wd).reshape(-1, Wd)))
           for i, (c, n) in enumerate(shape)]
    meta = vo.PrefillMeta.new([vo.PrefillSeq(c, n, t) for (c, n), t in zip(shape, tables)], BS)
    T = meta.num_rows()
    q = _bf16_round(orc.rand_vec(300, T * H * HD).reshape(T, H * HD))
    pool = gpu_backend.alloc_kv_pool(vo.KvLayout(2, NB, BS, KVH, HD))
    opool = orc.Pool(2, NB, BS, KVH, HD)
    for i, (c, n) in enumerate(shape):
        for lo, hi in ((0, c), (c, c + n)):  # "earlier steps", then this step
            if hi > lo:
                slots = [orc.slot_of(tables[i], p, BS) for p in range(lo, hi)]
                k, v = kvs[i][0][lo:hi], kvs[i][1][lo:hi]
                gpu_backend.write_kv(pool, 1, k.cuda().contiguous(), v.cuda().contiguous(), slots)
                opool.write_kv(1, k.float().numpy(), v.float().numpy(), slots)
    out = gpu_backend.prefill_attention(q.cuda(), pool, 1, meta)
    want = opool.attention(q.float().numpy(), 1, tables, meta.row_seq, meta.row_num_keys)
    _assert_close(out.float().cpu().numpy(), want, "reference prefill scenario")


def test_reference_decode_scenario(vo, gpu_backend):
    """cpu/tests.rs:294-334: ctx 0 / 3 / 10 (one key, one full block, spanning)."""
    _say("reference decode scenario (hd 8, bs 4)")
    H, KVH, HD, BS, NB = 6, 2, 8, 4, 16
    Wd = KVH * HD
    ctx = [0, 3, 10]
    tables = [[15], [4], [12, 1, 8]]
    kvs = [(_bf16_round(orc.rand_vec(400 + i, (c + 1) * Wd).reshape(-1, Wd)),
            _bf16_round(orc.rand_vec(500 + i, (c + 1) * Wd).reshape(-1, Wd)))
           for i, c in enumerate(ctx)]
    meta = vo.DecodeMeta.new([vo.DecodeSeq(c, t) for c, t in zip(ctx, tables)], BS)
    q = _bf16_round(orc.rand_vec(600, 3 * H * HD).reshape(3, H * HD))
    pool = gpu_backend.alloc_kv_pool(vo.KvLayout(2, NB, BS, KVH, HD))
    opool = orc.Pool(2, NB, BS, KVH, HD)
    for i, c in enumerate(ctx):
        slots = [orc.slot_of(tables[i], p, BS) for p in range(c + 1)]
        gpu_backend.write_kv(pool, 0, kvs[i][0].cuda().contiguous(), kvs[i][1].cuda().contiguous(),
                             slots)
        opool.write_kv(0, kvs[i][0].float().numpy(), kvs[i][1].float().numpy(), slots)
    out = gpu_backend.decode_attention(q.cuda(), pool, 0, meta)
    want = opool.attention(q.float().numpy(), 0, tables, meta.row_seq, meta.row_num_keys)
    _assert_close(out.float().cpu().numpy(), want, "reference decode scenario")
    # ctx 0: a single key, so every head of a group returns that key's V exactly
    v0 = kvs[0][1][0].reshape(KVH, HD)
    got0 = out[0].cpu().reshape(H, HD)
    for h in range(H):
        assert np.array_equal(_bits(got0[h]), _bits(v0[h // 3]))


# ---------------------------------------------------------------------------
# MFMA decode kernel
# ---------------------------------------------------------------------------
EDGE_CTX = [0, 1, 15, 16, 17, 31, 32, 33, 47, 63, 64, 100, 255, 256, 511, 512, 513, 1000, 1500]


@pytest.mark.parametrize("hd,heads,kvh", [(128, 32, 8), (128, 64, 8), (64, 4, 2), (128, 8, 8),
                                          (64, 48, 3), (128, 16, 1)])
def test_decode_mfma_edge_lengths(vo, gpu_backend, hd, heads, kvh):
    _say(f"decode mfma hd={hd} heads={heads} kvh={kvh}")
    wl = W.build(vo, gpu_backend, kind="decode", heads=heads, kv_heads=kvh, head_dim=hd,
                 block_size=16, num_blocks=1200, context_lens=EDGE_CTX, seed=hd * 7 + heads)
    out = _out(wl, gpu_backend)
    want = W.oracle_attention(orc, wl)
    _assert_close(out.float().cpu().numpy(), want, f"decode hd={hd} H={heads} KVH={kvh}")


@pytest.mark.parametrize("hd", [64, 128])
def test_decode_mfma_many_short_rows(vo, gpu_backend, hd):
    """Rows with 1..48 keys put the softmax weight on few keys, where rounding
    P to bf16 alone would break the tolerance; 256 rows per head_dim."""
    _say(f"decode short rows hd={hd}")
    ctx = np.random.default_rng(hd).integers(0, 48, 256)
    wl = W.build(vo, gpu_backend, kind="decode", heads=32, kv_heads=8, head_dim=hd,
                 block_size=16, num_blocks=1200, context_lens=ctx, seed=hd + 1)
    out = _out(wl, gpu_backend)
    want = W.oracle_attention(orc, wl)
    _assert_close(out.float().cpu().numpy(), want, f"short rows hd={hd}")


@pytest.mark.parametrize("split,waves", [("32", "1"), ("64", "2"), ("96", "4"), ("512", "1"),
                                         ("512", "2"), ("512", "4"), ("1024", "4"), ("2048", "4"),
                                         ("4096", "4"), ("32", "4"), ("768", "8"), ("4096", "8")])
def test_decode_mfma_split_and_wave_variants(vo, monkeypatch, split, waves):
    """Every split size and wavefront count gives the same results within
    tolerance, and a repeated call is bitwise identical."""
    monkeypatch.setenv("VO_DECODE_SPLIT", split)
    monkeypatch.setenv("VO_DECODE_WAVES", waves)
    _say(f"decode split={split} waves={waves}")
    backend = vo.HipBackend(device=0, max_seqs=64, max_rows=W.FILL_ROWS, max_table_entries=4096,
                            max_query_heads=32)
    wl = W.build(vo, backend, kind="decode", heads=32, kv_heads=8, head_dim=128, block_size=16,
                 num_blocks=1500, context_lens=EDGE_CTX, seed=int(split) + int(waves))
    out = _out(wl, backend)
    want = W.oracle_attention(orc, wl)
    _assert_close(out.float().cpu().numpy(), want, f"decode split={split} waves={waves}")
    again = _out(wl, backend)
    assert np.array_equal(_bits(again), _bits(out))


def test_decode_streaming_loads_bitwise_equal(vo, monkeypatch):
    """The non-temporal (streaming) and cached K/V load variants of the decode
    kernel differ only in cache policy: the outputs are bitwise equal, on
    disjoint tables (where the planner picks streaming) and on aliased ones
    (where it picks cached loads)."""
    _say("decode streaming vs cached loads")
    backend = vo.HipBackend(device=0, max_seqs=64, max_rows=W.FILL_ROWS, max_table_entries=8192,
                            max_query_heads=32)
    for shared in (0, 640):
        ctx = [shared + c for c in EDGE_CTX]
        wl = W.build(vo, backend, kind="decode", heads=32, kv_heads=8, head_dim=128,
                     block_size=16, num_blocks=3000, context_lens=ctx, seed=77,
                     shared_prefix=shared, shared_count=len(ctx) if shared else 0)
        outs = []
        for nt in ("0", "1"):
            monkeypatch.setenv("VO_DECODE_NT", nt)
            outs.append(_bits(_out(wl, backend)))
        monkeypatch.delenv("VO_DECODE_NT")
        auto = _bits(_out(wl, backend))
        assert np.array_equal(outs[0], outs[1]), f"shared={shared}"
        assert np.array_equal(auto, outs[0]), f"shared={shared}"
        want = W.oracle_attention(orc, wl)
        got = backend.decode_attention(wl.q, wl.pool, 0, wl.meta).float().cpu().numpy()
        _assert_close(got, want, f"streaming shared={shared}")


def test_decode_cfg2_full_size(vo, gpu_backend):
    """BASELINE config 2 at full size: 64 seqs, ctx U[512, 4096], 20000-block pool."""
    _say("decode cfg2 full size")
    ctx = W.cfg2_context_lens()
    wl = W.build(vo, gpu_backend, kind="decode", heads=32, kv_heads=8, head_dim=128,
                 block_size=16, num_blocks=20000, context_lens=ctx, seed=2)
    out = _out(wl, gpu_backend)
    want = W.oracle_attention(orc, wl)
    _assert_close(out.float().cpu().numpy(), want, "cfg2")


def test_decode_cfg5_prefix_shared_full_size(vo, gpu_backend):
    """H 64 / KVH 8, 64 seqs aliasing a 4096-token prefix,
    suffixes U[256, 1024], plus one 32768-context sequence (deep split-K)."""
    _say("decode cfg5 full size")
    ctx = W.cfg5_context_lens()
    wl = W.build(vo, gpu_backend, kind="decode", heads=64, kv_heads=8, head_dim=128,
                 block_size=16, num_blocks=40000, context_lens=ctx, seed=5, shared_prefix=4096,
                 shared_count=64)
    # aliased entries really are shared
    assert all(np.array_equal(wl.tables[0][:256], wl.tables[i][:256]) for i in range(64))
    out = _out(wl, gpu_backend)
    want = W.oracle_attention(orc, wl)
    _assert_close(out.float().cpu().numpy(), want, "cfg5")


def test_decode_batch_invariance_bitwise(vo, gpu_backend):
    """A row's output is identical alone or in a batch (the reference's
    batch-invariance invariant, CLAUDE.md; model.rs:539-584)."""
    import torch
    _say("decode batch invariance")
    ctx = W.cfg2_context_lens(seed=12, num_seqs=24)
    wl = W.build(vo, gpu_backend, kind="decode", heads=32, kv_heads=8, head_dim=128,
                 block_size=16, num_blocks=4000, context_lens=ctx, seed=12, keep_host=False)
    full = _out(wl, gpu_backend)
    for s in (0, 5, 23):
        meta1 = vo.DecodeMeta.new([vo.DecodeSeq(int(ctx[s]), wl.tables[s])], 16)
        one = gpu_backend.decode_attention(wl.q[s:s + 1].contiguous(), wl.pool, 0, meta1)
        assert np.array_equal(_bits(one[0]), _bits(full[s])), f"row {s}"


def test_decode_block_relabelling_invariance_bitwise(vo, gpu_backend):
    """Moving a sequence's blocks to other physical blocks changes nothing."""
    import torch
    _say("decode relabelling invariance")
    ctx = [700, 1333]
    wl = W.build(vo, gpu_backend, kind="decode", heads=32, kv_heads=8, head_dim=128,
                 block_size=16, num_blocks=600, context_lens=ctx, seed=21, keep_host=False)
    a = _out(wl, gpu_backend)
    # copy every key into fresh blocks of a second pool through a different permutation
    rng = np.random.default_rng(99)
    perm = rng.permutation(600).astype(np.uint32)
    pool2 = gpu_backend.alloc_kv_pool(vo.KvLayout(1, 600, 16, 8, 128))
    new_tables, off = [], 0
    for s, c in enumerate(ctx):
        n = len(wl.tables[s])
        new_tables.append(perm[off:off + n])
        off += n
        k, v = gpu_backend.read_kv(wl.pool, 0, wl.meta, s, c + 1)
        slots = [int(new_tables[s][p // 16]) * 16 + p % 16 for p in range(c + 1)]
        gpu_backend.write_kv(pool2, 0, k.contiguous(), v.contiguous(), slots)
    meta2 = vo.DecodeMeta.new([vo.DecodeSeq(c, t) for c, t in zip(ctx, new_tables)], 16)
    b = gpu_backend.decode_attention(wl.q, pool2, 0, meta2)
    assert np.array_equal(_bits(a), _bits(b))


# ---------------------------------------------------------------------------
# Prefill
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("hd,heads,kvh", [(128, 32, 8), (64, 4, 2), (128, 64, 8), (128, 16, 8),
                                          (64, 12, 3)])
def test_prefill_chunked_with_context(vo, gpu_backend, hd, heads, kvh):
    """Chunks that start at position 0, mid-block and on block boundaries;
    chunk lengths of 1, non-multiples of the 32-row tile, and > 64 rows."""
    _say(f"prefill hd={hd} heads={heads}")
    wl = W.build(vo, gpu_backend, kind="prefill", heads=heads, kv_heads=kvh, head_dim=hd,
                 block_size=16, num_blocks=800, context_lens=[0, 37, 256, 1000, 5],
                 num_new=[64, 100, 1, 77, 129], seed=hd + heads)
    out = _out(wl, gpu_backend)
    want = W.oracle_attention(orc, wl)
    _assert_close(out.float().cpu().numpy(), want, f"prefill hd={hd}")


def test_prefill_cfg3_full_size_sampled_rows(vo, gpu_backend):
    """8 seqs x 512-row chunks on context U[0, 8192]; every
    row is computed on the GPU, a sample of rows by the oracle."""
    _say("prefill cfg3 full size")
    ctx = W.cfg3_context_lens()
    wl = W.build(vo, gpu_backend, kind="prefill", heads=32, kv_heads=8, head_dim=128,
                 block_size=16, num_blocks=12000, context_lens=ctx, num_new=[512] * 8, seed=3)
    out = _out(wl, gpu_backend).float().cpu().numpy()
    starts = np.asarray(wl.meta.seq_row_starts, dtype=np.int64)
    rows = np.unique(np.concatenate([np.arange(0, wl.rows, 29), starts[1:] - 1, starts[:-1]]))
    want = W.oracle_attention(orc, wl, rows=rows)
    _assert_close(out[rows], want, "cfg3")


def test_prefill_row_matches_decode_within_tolerance(vo, gpu_backend):
    """A prefill row at position p and a decode at context p see the same keys."""
    _say("prefill row vs decode")
    wl = W.build(vo, gpu_backend, kind="prefill", heads=32, kv_heads=8, head_dim=128,
                 block_size=16, num_blocks=300, context_lens=[900], num_new=[40], seed=33)
    pre = _out(wl, gpu_backend).float().cpu().numpy()
    for i in (0, 17, 39):
        meta = vo.DecodeMeta.new([vo.DecodeSeq(900 + i, wl.tables[0])], 16)
        dec = gpu_backend.decode_attention(wl.q[i:i + 1].contiguous(), wl.pool, 0, meta)
        _assert_close(dec.float().cpu().numpy()[0], pre[i], f"row {i}")


# ---------------------------------------------------------------------------
# Errors through the GPU path: checked on the host, nothing launched
# ---------------------------------------------------------------------------
def test_errors_match_reference_classes(vo, gpu_backend):
    import torch
    _say("error classes")
    H, KVH, HD, BS, NB = 6, 2, 8, 4, 16
    pool = gpu_backend.alloc_kv_pool(vo.KvLayout(2, NB, BS, KVH, HD))
    q = torch.zeros((1, H * HD), dtype=torch.bfloat16, device="cuda:0")
    meta = vo.DecodeMeta.new([vo.DecodeSeq(0, [NB])], BS)  # cpu/tests.rs:340-348
    with pytest.raises(vo.BlockOutOfRange) as e:
        gpu_backend.decode_attention(q, pool, 0, meta)
    assert (e.value.value, e.value.limit, e.value.op) == (NB, NB, "decode_attention")
    k = torch.zeros((1, KVH * HD), dtype=torch.bfloat16, device="cuda:0")
    with pytest.raises(vo.SlotOutOfRange) as e:
        gpu_backend.write_kv(pool, 0, k, k.clone(), [NB * BS])  # cpu/tests.rs:355-360
    assert (e.value.value, e.value.limit) == (NB * BS, NB * BS)
    ok = vo.DecodeMeta.new([vo.DecodeSeq(0, [3])], BS)
    with pytest.raises(vo.ShapeError):  # layer out of range (arena/ops.rs:204)
        gpu_backend.decode_attention(q, pool, 2, ok)
    with pytest.raises(vo.ShapeError):  # cols not a multiple of kv_heads*hd groups
        gpu_backend.decode_attention(torch.zeros((1, 3 * HD), dtype=torch.bfloat16,
                                                 device="cuda:0"), pool, 0, ok)
    with pytest.raises(vo.ShapeError):  # rows != metadata rows
        gpu_backend.decode_attention(torch.zeros((2, H * HD), dtype=torch.bfloat16,
                                                 device="cuda:0"), pool, 0, ok)
    pm = vo.PrefillMeta.new([vo.PrefillSeq(0, 1, [3])], BS)
    with pytest.raises(vo.ShapeError):  # decode op given prefill metadata
        gpu_backend.decode_attention(q, pool, 0, pm)
    torch.cuda.synchronize()
