"""GPU parity: the HIP path through the C ABI against the CPU oracle.

Bars:
* slot mappings and block gathers: bit-exact;
* attention outputs: |gpu - oracle| <= atol + rtol*|oracle| with rtol 1e-2,
  atol 2e-3 (bf16 I/O, fp32 accumulation), on identical seeded inputs.
Plus size-independent properties at full BASELINE sizes: batch invariance and
block-relabelling invariance (bitwise), single key -> V exactly.
"""
import dataclasses
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


def _out_with_prefill_instances(vo, wl, backend):
    """_out with per-launch timing on; also the set of prefill kernel
    instances that ran (the library times each launch under its instance's
    name: prefill_pipe = the pipelined 4-wavefront kernel for 64-row
    workgroups at head_dim 128 / GQA 4, prefill_dma = the 8-wavefront kernel
    for other 64-row workgroups, prefill_dma_narrow = 32-row workgroups,
    prefill_regs = the register-staged kernel)."""
    import torch
    vo.profile_reset()
    vo.enable_profiling(True)
    try:
        out = _out(wl, backend)
        torch.cuda.synchronize()
    finally:
        vo.enable_profiling(False)
    return out, {k for k in vo.profile() if k.startswith("prefill_")}


def _out_replanned(wl, backend):
    """_out after uploading the metadata again, so that the launch plan is
    rebuilt under the current VO_DECODE_* settings (an unchanged meta object
    is otherwise not uploaded twice)."""
    backend.step_meta(wl.pool).holds = None
    return _out(wl, backend)


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
            outs.append(_bits(_out_replanned(wl, backend)))
        monkeypatch.delenv("VO_DECODE_NT")
        auto = _bits(_out_replanned(wl, backend))
        assert np.array_equal(outs[0], outs[1]), f"shared={shared}"
        assert np.array_equal(auto, outs[0]), f"shared={shared}"
        want = W.oracle_attention(orc, wl)
        got = backend.decode_attention(wl.q, wl.pool, 0, wl.meta).float().cpu().numpy()
        _assert_close(got, want, f"streaming shared={shared}")


_PACK_CASES = [
    (128, 64, 8, "1024", "4", 1, 12),  # cfg5's shape: group 8, two rows per item
    (128, 64, 8, "1024", "4", 2, 12),  # shared packs: 2 rows per tile
    (128, 64, 8, "2048", "4", 2, 2),   # a shared pack of 2 rows
    (128, 64, 8, "2048", "4", 2, 1),   # no two rows share a split: nothing packed
    (128, 64, 8, "64", "4", 2, 12),    # 2 chunks per split: states 2 and 3 stay empty
    (128, 64, 8, "96", "4", 2, 12),    # 3 chunks: the pairs' last step has one chunk
    (128, 32, 8, "512", "1", 1, 12),   # group 4, four rows per item, no LDS merge
    (128, 32, 8, "512", "1", 2, 12),   # one wavefront: shared packs fall back to one tile
    (128, 32, 8, "512", "8", 2, 12),   # 8 wavefronts: shared packs fall back to one tile
    (128, 32, 8, "512", "4", 2, 12),   # 4 rows per tile: a short last pack
    (64, 6, 2, "256", "2", 1, 12),     # group 3, five rows per item, a short last pack
    (64, 6, 2, "256", "4", 2, 12),     # group 3, shared: 5 rows per tile
]


@pytest.mark.parametrize("hd,heads,kvh,split,waves,mode,nalias,pairs",
                         [c + ("1",) for c in _PACK_CASES] +
                         [c + ("0",) for c in _PACK_CASES if c[5] == 2 and c[4] == "4"])
def test_decode_row_packing_bitwise(vo, monkeypatch, hd, heads, kvh, split, waves, mode,
                                    nalias, pairs):
    """Rows whose full splits read the same physical blocks (an aliased
    prefix) share one work item, each row in its own head columns: one
    16-column MFMA tile per item (VO_DECODE_PACK=1), or a shared pack over
    chunks staged once in LDS (=2, the default) whose tiles have two
    wavefronts each, one per pair of softmax states (VO_DECODE_SHARED_PAIRS=1,
    the default), or one wavefront each (=0).  The outputs are bitwise those
    of the unpacked plan (VO_DECODE_PACK=0) and within tolerance of the
    oracle; the plan really packs: each of the two shared prefix splits of the
    aliasing rows runs as ceil(rows / P) items, with P rows per item for the
    mode."""
    monkeypatch.setenv("VO_DECODE_SPLIT", split)
    monkeypatch.setenv("VO_DECODE_WAVES", waves)
    monkeypatch.setenv("VO_DECODE_SHARED_PAIRS", pairs)
    _say(f"decode row packing hd={hd} heads={heads} kvh={kvh} split={split} waves={waves} "
         f"mode={mode} aliasing rows={nalias} pairs={pairs}")
    L = int(split)
    backend = vo.HipBackend(device=0, max_seqs=64, max_rows=W.FILL_ROWS, max_table_entries=8192,
                            max_query_heads=heads)
    shared = 2 * L
    extra = [0, 1, 17, 100, L - 1, L, L + 5, 5, 2 * L + 3, 64, 700 % L, 31][:nalias]
    ctx = [shared + e for e in extra] + [3 * L, 50]
    wl = W.build(vo, backend, kind="decode", heads=heads, kv_heads=kvh, head_dim=hd,
                 block_size=16, num_blocks=4000, context_lens=ctx, seed=L + heads,
                 shared_prefix=shared, shared_count=len(extra))
    group = heads // kvh
    one_tile = 16 // group
    if mode == 2 and int(waves) != 4:
        mode = 1  # shared packs need 4 wavefronts
    if mode == 1:
        P = one_tile
    else:
        P = (2 if pairs == "1" else 4) * (16 // group)
        if min(P, len(extra)) < 2:
            P = 1  # nothing to share
    parts = sum(-(-(c + 1) // L) for c in ctx)
    meta = backend.step_meta(wl.pool)

    monkeypatch.setenv("VO_DECODE_PACK", "0")
    plain = _out_replanned(wl, backend)
    assert meta.decode_plan() == (parts, parts, 1)
    monkeypatch.setenv("VO_DECODE_PACK", str(mode))
    packed = _out_replanned(wl, backend)
    packs = -(-len(extra) // P)
    assert meta.decode_plan() == (parts - 2 * (len(extra) - packs), parts, P)
    assert np.array_equal(_bits(packed), _bits(plain))
    again = _out(wl, backend)
    assert np.array_equal(_bits(again), _bits(packed))
    want = W.oracle_attention(orc, wl)
    _assert_close(packed.float().cpu().numpy(), want, f"packed hd={hd} H={heads} mode={mode}")


@pytest.mark.parametrize("hd,heads,kvh,shared,fixed", [
    (128, 32, 8, 0, False),     # disjoint tables: one launch
    (64, 4, 2, 0, False),
    (128, 16, 1, 640, False),   # blocks shared, none holding a new slot: one launch
    (128, 32, 8, 2048, False),  # shared blocks that the plan packs: one launch
    (128, 32, 8, 0, True),      # fixed launch shapes: the two ops
])
def test_decode_attention_write_kv_bitwise(vo, hd, heads, kvh, shared, fixed):
    """vo_decode_attention_write_kv equals write_kv then decode_attention,
    bitwise: the output and the cached new keys.  The new slots hold other
    values before the call, so the launch must cache the keys itself; the
    kernel profile shows whether it ran as one launch."""
    import torch
    _say(f"decode+write_kv hd={hd} heads={heads} kvh={kvh} shared={shared}")
    backend = vo.HipBackend(device=0, max_seqs=64, max_rows=W.FILL_ROWS, max_table_entries=8192,
                            max_query_heads=heads)
    ctx = [shared + c for c in EDGE_CTX]
    wl = W.build(vo, backend, kind="decode", heads=heads, kv_heads=kvh, head_dim=hd,
                 block_size=16, num_blocks=3000, context_lens=ctx, seed=31 + hd + heads,
                 shared_prefix=shared, shared_count=len(ctx) if shared else 0)
    backend.write_kv(wl.pool, 0, wl.k_new, wl.v_new, wl.meta)
    want = _bits(backend.decode_attention(wl.q, wl.pool, 0, wl.meta))
    gen = torch.Generator(device="cuda:0").manual_seed(5)
    junk_k = torch.randn(wl.k_new.shape, generator=gen, device="cuda:0").to(torch.bfloat16)
    junk_v = torch.randn(wl.v_new.shape, generator=gen, device="cuda:0").to(torch.bfloat16)
    backend.write_kv(wl.pool, 0, junk_k, junk_v, wl.meta)
    if fixed:
        backend.step_meta(wl.pool).fix_launch(len(ctx), 0)
    else:
        work, parts, _ = backend.step_meta(wl.pool).decode_plan()
        assert (work < parts) == (shared >= 2048), (work, parts)  # packed items over the prefix
    vo.profile_reset()
    vo.enable_profiling(True)
    got = backend.decode_attention_write_kv(wl.q, wl.k_new, wl.v_new, wl.pool, 0, wl.meta)
    torch.cuda.synchronize()
    vo.enable_profiling(False)
    kernels = set(vo.profile())
    assert ("reshape_and_cache" in kernels) == fixed, kernels
    assert np.array_equal(_bits(got), want)
    for s_, c in enumerate(ctx):
        k, v = backend.read_kv(wl.pool, 0, wl.meta, s_, c + 1)
        assert np.array_equal(_bits(k[c]), _bits(wl.k_new[s_])), f"K of seq {s_}"
        assert np.array_equal(_bits(v[c]), _bits(wl.v_new[s_])), f"V of seq {s_}"
    if fixed:
        backend.step_meta(wl.pool).unfix_launch()


@pytest.mark.parametrize("case", ["two_rows_one_seq", "slot_not_last_key", "zero_keys",
                                  "tail_block_shared", "repeated_slot"])
def test_decode_attention_write_kv_noncanonical_falls_back(vo, case):
    """vo_decode_attention_write_kv on decode metadata that DecodeMeta::new
    would not build (its fields are public, paged.rs:173-186): two rows of one
    sequence, a slot that is not the row's last key, a row with no keys, a new
    slot in a block another sequence reads, a repeated slot.  Each must run as
    write_kv then decode_attention (reshape_and_cache shows in the profile)
    and give bitwise their output and pool contents."""
    import torch
    _say(f"decode+write_kv non-canonical: {case}")
    heads, kvh, hd, bs = 32, 8, 128, 16
    ctx = [40, 100, 17, 300]
    runs = []
    for _ in range(2):
        backend = vo.HipBackend(device=0, max_seqs=8, max_rows=W.FILL_ROWS,
                                max_table_entries=512, max_query_heads=heads)
        wl = W.build(vo, backend, kind="decode", heads=heads, kv_heads=kvh, head_dim=hd,
                     block_size=bs, num_blocks=200, context_lens=ctx, seed=77)
        runs.append((backend, wl))
    base = runs[0][1].meta
    tables = [np.array(t, np.uint32) for t in base.block_tables]
    rseq = np.array(base.row_seq, np.uint64)
    rkeys = np.array(base.row_num_keys, np.uint64)
    slots = np.array(base.slot_mapping, np.uint32)
    pos = np.array(base.positions, np.uint32)
    used = {int(b) for t in tables for b in t}
    spare = next(b for b in range(200) if b not in used)
    if case == "two_rows_one_seq":
        rseq[1], rkeys[1] = 0, 30            # a second row of sequence 0, inside its keys
        slots[1] = int(tables[0][29 // bs]) * bs + 29 % bs
    elif case == "slot_not_last_key":
        slots[2] = spare * bs + 3            # a block no table holds
    elif case == "zero_keys":
        rkeys[3] = 0
    elif case == "tail_block_shared":
        tables[1] = tables[1].copy()
        tables[1][0] = tables[0][40 // bs]   # sequence 1 reads the block of sequence 0's new slot
    elif case == "repeated_slot":
        slots[3] = slots[2]
    meta = vo.DecodeMeta(bs, tables, pos, slots, rseq, rkeys)
    results = []
    for i, (backend, wl) in enumerate(runs):
        # The new slots first hold other values, so a launch that skipped the
        # cache write, or read a slot it also writes, would differ.
        gen = torch.Generator(device="cuda:0").manual_seed(9)
        junk_k = torch.randn(wl.k_new.shape, generator=gen, device="cuda:0").to(torch.bfloat16)
        junk_v = torch.randn(wl.v_new.shape, generator=gen, device="cuda:0").to(torch.bfloat16)
        backend.write_kv(wl.pool, 0, junk_k, junk_v, wl.meta)
        vo.profile_reset()
        vo.enable_profiling(True)
        if i == 0:
            backend.write_kv(wl.pool, 0, wl.k_new, wl.v_new, meta)
            out = backend.decode_attention(wl.q, wl.pool, 0, meta)
        else:
            out = backend.decode_attention_write_kv(wl.q, wl.k_new, wl.v_new, wl.pool, 0, meta)
        torch.cuda.synchronize()
        vo.enable_profiling(False)
        kernels = set(vo.profile())
        assert "reshape_and_cache" in kernels, (case, kernels)
        pool_bits = []
        for s_ in range(len(ctx)):
            k, v = backend.read_kv(wl.pool, 0, meta, s_, ctx[s_] + 1)
            pool_bits.append((_bits(k), _bits(v)))
        results.append((_bits(out), pool_bits))
    assert np.array_equal(results[0][0], results[1][0]), case
    for s_ in range(len(ctx)):
        assert np.array_equal(results[0][1][s_][0], results[1][1][s_][0]), (case, "K", s_)
        assert np.array_equal(results[0][1][s_][1], results[1][1][s_][1]), (case, "V", s_)


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


@pytest.mark.parametrize("name", ["cfg2", "cfg5"])
def test_decode_attention_write_kv_full_size(vo, name):
    """The call the decode benchmark times, vo_decode_attention_write_kv, at
    BASELINE config 2 and config 5's full sizes: one launch, bitwise equal to
    write_kv then decode_attention (the output, and every key and value each
    sequence reads back from the pool), and within rtol/atol of the oracle.
    Layer 0 runs the two ops, layer 1 the fused call, on the same cached
    context; both layers' new slots hold other values first."""
    import torch
    _say(f"decode+write_kv full size {name}")
    if name == "cfg2":
        ctx, heads, blocks, seed, shared = W.cfg2_context_lens(), 32, 20000, 2, 0
    else:
        ctx, heads, blocks, seed, shared = W.cfg5_context_lens(), 64, 40000, 5, 4096
    backend = vo.HipBackend(device=0, max_seqs=len(ctx), max_rows=W.FILL_ROWS,
                            max_table_entries=blocks, max_query_heads=heads)
    wl = W.build(vo, backend, kind="decode", heads=heads, kv_heads=8, head_dim=128,
                 block_size=16, num_blocks=blocks, context_lens=ctx, seed=seed,
                 shared_prefix=shared, shared_count=64 if shared else 0, num_layers=2,
                 fill_layers=[0, 1])
    gen = torch.Generator(device="cuda:0").manual_seed(13)
    junk_k = torch.randn(wl.k_new.shape, generator=gen, device="cuda:0").to(torch.bfloat16)
    junk_v = torch.randn(wl.v_new.shape, generator=gen, device="cuda:0").to(torch.bfloat16)
    for layer in (0, 1):
        backend.write_kv(wl.pool, layer, junk_k, junk_v, wl.meta)
    backend.write_kv(wl.pool, 0, wl.k_new, wl.v_new, wl.meta)
    want = backend.decode_attention(wl.q, wl.pool, 0, wl.meta)
    vo.profile_reset()
    vo.enable_profiling(True)
    got = backend.decode_attention_write_kv(wl.q, wl.k_new, wl.v_new, wl.pool, 1, wl.meta)
    torch.cuda.synchronize()
    vo.enable_profiling(False)
    kernels = set(vo.profile())
    assert "reshape_and_cache" not in kernels and "decode_splitk" in kernels, kernels
    assert np.array_equal(_bits(got), _bits(want)), name
    for s_, c in enumerate(ctx):
        k0, v0 = backend.read_kv(wl.pool, 0, wl.meta, s_, c + 1)
        k1, v1 = backend.read_kv(wl.pool, 1, wl.meta, s_, c + 1)
        assert np.array_equal(_bits(k1), _bits(k0)), f"{name}: K of seq {s_}"
        assert np.array_equal(_bits(v1), _bits(v0)), f"{name}: V of seq {s_}"
        assert np.array_equal(_bits(k1[c]), _bits(wl.k_new[s_])), f"{name}: new K of seq {s_}"
    oracle_want = W.oracle_attention(orc, wl)
    _assert_close(got.float().cpu().numpy(), oracle_want, name)


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


@pytest.mark.parametrize("pipe", ["1", "0"])
@pytest.mark.parametrize("offset", ["fixed", "running"])
def test_prefill_64_row_workgroups_edge_shapes(vo, gpu_backend, monkeypatch, offset, pipe):
    """The 64-row workgroups at GQA 4, head_dim 128 -- the pipelined
    4-wavefront kernel and the 8-wavefront one (VO_PREFILL_PIPE=0) -- with
    the fixed tile-0 softmax offset and with the running max
    (VO_PREFILL_OFFSET), on a grid small enough that the 32-row workgroups
    would otherwise serve it (VO_PREFILL_NARROW=0): chunks starting at 0,
    mid-block, on and next to tile boundaries; items of 2, 31, 32, 33, 64
    and 65 rows; one row per block of a 2047-key context."""
    _say(f"prefill 64-row workgroups ({offset} offset, pipe {pipe})")
    monkeypatch.setenv("VO_PREFILL_NARROW", "0")
    monkeypatch.setenv("VO_PREFILL_OFFSET", offset)
    monkeypatch.setenv("VO_PREFILL_PIPE", pipe)
    wl = W.build(vo, gpu_backend, kind="prefill", heads=32, kv_heads=8, head_dim=128,
                 block_size=16, num_blocks=1200,
                 context_lens=[0, 5, 63, 64, 65, 1000, 2047, 31],
                 num_new=[2, 31, 32, 33, 64, 65, 129, 200], seed=61)
    gpu_backend.step_meta(wl.pool).holds = None
    out, ran = _out_with_prefill_instances(vo, wl, gpu_backend)
    # the settings are honoured: 64-row workgroups of the chosen kernel ran
    assert ran == ({"prefill_pipe"} if pipe == "1" else {"prefill_dma"}), ran
    want = W.oracle_attention(orc, wl)
    _assert_close(out.float().cpu().numpy(), want, f"prefill 64-row workgroups ({offset})")


@pytest.mark.parametrize("narrow,pipe,slots", [("1", "1", ""), ("0", "1", ""), ("0", "1", "1"),
                                               ("0", "0", "")])
@pytest.mark.parametrize("factor", [4.0, 10.0])
def test_prefill_key_far_above_tile0_max(vo, gpu_backend, monkeypatch, narrow, pipe, slots, factor):
    """The prefill kernel first keeps each row's tile-0 max as its softmax
    offset.  Key 200 of sequence 0 (cached, KV tile 3) is set to factor x
    query row 0's head-0 vector (KV head 0 serves heads 0..3), so that row's
    score for it is ~factor |q|^2 / sqrt(128): ~65 log2 units above the rest
    at factor 4 (row sum past the 2^40 bound, no overflow yet) and ~163 at
    factor 10, where 2^163 overflows f32 and only the recompute with the
    running max gives finite output.  Every row must match the oracle, in
    32-row (narrow) and 64-row workgroups (the pipelined kernel and the
    8-wavefront one).  slots "1": the pipelined kernel's five items run back
    to back in one workgroup per KV head, the recomputed one third, between
    items whose tiles it prefetched and that prefetched its own."""
    import torch
    _say(f"prefill key far above tile-0 max (factor {factor}, narrow {narrow}, pipe {pipe}, "
         f"slots {slots or 'default'})")
    monkeypatch.setenv("VO_PREFILL_NARROW", narrow)
    monkeypatch.setenv("VO_PREFILL_PIPE", pipe)
    monkeypatch.setenv("VO_PREFILL_PIPE_SLOTS", slots)
    ctx, new = [300, 0, 900], [64, 128, 100]
    wl = W.build(vo, gpu_backend, kind="prefill", heads=32, kv_heads=8, head_dim=128,
                 block_size=16, num_blocks=200, context_lens=ctx, num_new=new, seed=62)
    q0 = wl.q[0, :128].float()
    k_big = (factor * q0).to(torch.bfloat16)
    keys = wl.ctx_kv[0][0].clone()
    keys[200, :128] = k_big
    slot = int(wl.tables[0][200 // 16]) * 16 + 200 % 16
    gpu_backend.write_kv(wl.pool, 0, keys[200:201].contiguous(),
                         wl.ctx_kv[0][1][200:201].contiguous(), [slot])
    wl.ctx_kv[0] = (keys, wl.ctx_kv[0][1])
    wl.host["ctx"][0] = (keys.float().cpu().numpy(), wl.host["ctx"][0][1])
    gpu_backend.step_meta(wl.pool).holds = None
    out, ran = _out_with_prefill_instances(vo, wl, gpu_backend)
    assert ran == ({"prefill_dma_narrow"} if narrow == "1"
                   else {"prefill_pipe"} if pipe == "1" else {"prefill_dma"}), ran
    want = W.oracle_attention(orc, wl)
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    _assert_close(got, want, f"prefill key far above tile-0 max (factor {factor})")


@pytest.mark.parametrize("with_long", [False, True])
def test_prefill_batch_invariance_bitwise(vo, gpu_backend, with_long):
    """A sequence's prefill rows are bitwise the same alone and in a batch
    (the reference's batch invariance, CLAUDE.md; model.rs:539-584), where
    the batch changes how the kernels are launched:
    - alone, sequence A (100 rows: two items) has fewer items x KV heads
      than CUs and runs in 32-row workgroups; in the batch (with B's 32
      items) it runs in 64-row workgroups.  Key 200 of A is set to 4 x the
      head-0 query of A's row 40, ~65 log2 units above that row's other
      scores (and ~17 at most for the other rows), which puts that row's sum
      past the fixed offset's range, so row group 1 of A's first item is
      recomputed with the running max while group 0 keeps the fixed offset,
      in both;
    - with_long adds C, whose rows see more keys than the DMA kernel's LDS
      block table holds: C's item runs on the register-staged kernel, A's
      and B's items on the DMA kernel, in the batch as alone.
    A and C also match the oracle (C: sampled rows; its 65,600 cached keys
    are the only test of that path)."""
    import torch
    _say(f"prefill batch invariance (long sequence {with_long})")
    ctx, new = [300, 500], [100, 2048]
    if with_long:
        ctx.append(4096 * 16 + 64)  # past the DMA kernel's 4096-block LDS table
        new.append(40)
    num_blocks = sum(-(-(c + n) // 16) for c, n in zip(ctx, new)) + 8
    wl = W.build(vo, gpu_backend, kind="prefill", heads=32, kv_heads=8, head_dim=128,
                 block_size=16, num_blocks=num_blocks, context_lens=ctx, num_new=new, seed=71)
    q40 = wl.q[40, :128].float()
    keys = wl.ctx_kv[0][0].clone()
    keys[200, :128] = (4.0 * q40).to(torch.bfloat16)
    slot = int(wl.tables[0][200 // 16]) * 16 + 200 % 16
    gpu_backend.write_kv(wl.pool, 0, keys[200:201].contiguous(),
                         wl.ctx_kv[0][1][200:201].contiguous(), [slot])
    wl.ctx_kv[0] = (keys, wl.ctx_kv[0][1])
    wl.host["ctx"][0] = (keys.float().cpu().numpy(), wl.host["ctx"][0][1])
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    items = [-(-n // 64) for n in new]
    assert items[0] * 8 < cus <= sum(items) * 8, "A alone narrow, the batch wide"

    full = _out(wl, gpu_backend)
    starts = np.concatenate([[0], np.cumsum(new)])
    checked = [0, 2] if with_long else [0]
    for s in checked:
        a, b = int(starts[s]), int(starts[s + 1])
        meta1 = vo.PrefillMeta.new([vo.PrefillSeq(int(ctx[s]), int(new[s]), wl.tables[s])], 16)
        one = gpu_backend.prefill_attention(wl.q[a:b].contiguous(), wl.pool, 0, meta1)
        assert np.array_equal(_bits(one), _bits(full[a:b])), f"sequence {s}"
    rows = list(range(100))
    if with_long:
        c0 = int(starts[2])
        rows += [c0, c0 + 17, c0 + 39]
    got = full.float().cpu().numpy()[rows]
    assert np.isfinite(got).all()
    _assert_close(got, W.oracle_attention(orc, wl, rows=rows), "prefill batch invariance rows")


@pytest.mark.parametrize("hd,heads,kvh", [(64, 32, 8), (128, 16, 8), (128, 64, 8), (64, 8, 4)])
def test_prefill_batch_invariance_bitwise_shapes(vo, gpu_backend, hd, heads, kvh):
    """The batch invariance above at the other prefill kernel instances:
    head_dim 64 with GQA 4 (DMA kernel, 32- or 64-row workgroups), GQA 2
    (head_dim 128: register-staged kernel; head_dim 64: DMA kernel) and
    GQA 8 (one row group per workgroup), with the same planted key."""
    import torch
    _say(f"prefill batch invariance hd {hd} heads {heads}/{kvh}")
    ctx, new = [300, 500], [100, 2048]  # alone: 2 items; in the batch: 34 (x KV heads >= CUs at kvh 8)
    num_blocks = sum(-(-(c + n) // 16) for c, n in zip(ctx, new)) + 8
    wl = W.build(vo, gpu_backend, kind="prefill", heads=heads, kv_heads=kvh, head_dim=hd,
                 block_size=16, num_blocks=num_blocks, context_lens=ctx, num_new=new, seed=72,
                 keep_host=False)
    keys = wl.ctx_kv[0][0].clone()
    keys[200, :hd] = (4.0 * wl.q[40, :hd].float()).to(torch.bfloat16)
    slot = int(wl.tables[0][200 // 16]) * 16 + 200 % 16
    gpu_backend.write_kv(wl.pool, 0, keys[200:201].contiguous(),
                         wl.ctx_kv[0][1][200:201].contiguous(), [slot])
    full = _out(wl, gpu_backend)
    meta1 = vo.PrefillMeta.new([vo.PrefillSeq(ctx[0], new[0], wl.tables[0])], 16)
    one = gpu_backend.prefill_attention(wl.q[:new[0]].contiguous(), wl.pool, 0, meta1)
    assert np.isfinite(one.float().cpu().numpy()).all()
    assert np.array_equal(_bits(one), _bits(full[:new[0]]))


def _oracle_renumbered(vo, wl):
    """The oracle's output for wl with the physical block ids renumbered
    0, 1, .. in order of first use (aliasing kept): the attention does not
    depend on which blocks hold the keys, and the oracle's f32 pool then
    stays small for a workload on a huge device pool."""
    import copy
    ids = {}
    tables = [np.array([ids.setdefault(int(b), len(ids)) for b in t], np.uint32) for t in wl.tables]
    small = copy.copy(wl)
    small.tables = tables
    small.num_blocks = len(ids)
    bs = wl.block_size
    if wl.kind == "decode":
        small.meta = vo.DecodeMeta.new(
            [vo.DecodeSeq(int(c), t) for c, t in zip(wl.context_lens, tables)], bs)
    else:
        small.meta = vo.PrefillMeta.new(
            [vo.PrefillSeq(int(c), int(n), t) for c, n, t in zip(wl.context_lens, wl.num_new, tables)],
            bs)
    return W.oracle_attention(orc, small)


# 8 KV heads x 16 keys x head_dim 128 x bf16 = 32 KiB of a layer's K per block:
# 131,071 blocks keep the layer's K under 4 GiB, 131,080 put it past.
_BLOCK_BYTES_8x128 = 8 * 16 * 128 * 2


@pytest.mark.parametrize("num_blocks", [(1 << 32) // _BLOCK_BYTES_8x128 - 1,
                                        (1 << 32) // _BLOCK_BYTES_8x128 + 8])
def test_prefill_pool_at_and_past_4_gib(vo, num_blocks):
    """The LDS-DMA prefill kernel addresses a block by a 32-bit byte offset
    into the layer (one buffer resource per pool), so it serves layers of
    K (and V) under 4 GiB; a larger layer runs the register-staged kernel
    with 64-bit addresses.  Both, with tables that use the pool's last blocks
    (offsets just under and past 2^32), match the oracle."""
    _say(f"prefill on a {num_blocks}-block pool")
    rng = np.random.default_rng(71)
    ctx, new = [700, 130, 2000], [64, 100, 33]
    need = [-(-(c + n) // 16) for c, n in zip(ctx, new)]
    top = list(range(num_blocks - 1, num_blocks - 1 - need[0], -1))
    low = list(range(5, 5 + need[1] // 2))
    high = list(range(num_blocks - 1 - need[0], num_blocks - 1 - need[0] - (need[1] - len(low)), -1))
    mixed = [b for pair in zip(low, high) for b in pair] + low[len(high):] + high[len(low):]
    used = set(top) | set(mixed)
    rest = [int(b) for b in rng.permutation(num_blocks)[:need[2] + len(used)] if int(b) not in used]
    tables = [top, mixed, rest[:need[2]]]
    backend = vo.HipBackend(device=0, max_seqs=8, max_rows=W.FILL_ROWS, max_table_entries=1024,
                            max_query_heads=32)
    wl = W.build(vo, backend, kind="prefill", heads=32, kv_heads=8, head_dim=128,
                 block_size=16, num_blocks=num_blocks, context_lens=ctx, num_new=new, seed=71,
                 tables=tables)
    out = _out(wl, backend)
    _assert_close(out.float().cpu().numpy(), _oracle_renumbered(vo, wl),
                  f"prefill on a {num_blocks}-block pool")
    del wl, out
    import torch
    torch.cuda.empty_cache()


@pytest.mark.parametrize("num_blocks", [(1 << 32) // _BLOCK_BYTES_8x128 - 1,
                                        (1 << 32) // _BLOCK_BYTES_8x128 + 8])
def test_decode_shared_packs_pool_at_and_past_4_gib(vo, num_blocks):
    """Decode with shared packs (8 rows on an aliased 4096-key prefix, group
    8) and a long row, on pools whose last blocks sit just under and past
    4 GiB of a layer's K: the packs' LDS DMA and the register path both
    address those blocks right (oracle tolerance)."""
    _say(f"decode shared packs on a {num_blocks}-block pool")
    rng = np.random.default_rng(72)
    shared = 4096
    ctx = [shared + e for e in (3, 100, 257, 900, 31, 64, 1000, 5)] + [9000]
    pre = list(range(num_blocks - 1, num_blocks - 1 - shared // 16, -1))
    nxt = num_blocks - 1 - shared // 16
    tables = []
    for c in ctx[:8]:
        own = -(-(c + 1) // 16) - shared // 16
        tables.append(pre + list(range(nxt, nxt - own, -1)))
        nxt -= own
    long_need = -(-(ctx[8] + 1) // 16)
    tables.append([int(b) for b in rng.permutation(nxt)[:long_need]])
    backend = vo.HipBackend(device=0, max_seqs=16, max_rows=W.FILL_ROWS, max_table_entries=4096,
                            max_query_heads=64)
    wl = W.build(vo, backend, kind="decode", heads=64, kv_heads=8, head_dim=128,
                 block_size=16, num_blocks=num_blocks, context_lens=ctx, seed=72,
                 shared_prefix=shared, shared_count=8, tables=tables)
    out = _out(wl, backend)
    # 8 rows x 3 splits + 5 for the long row; each of the 8 rows' two prefix
    # splits runs as two shared packs of 4 rows.
    assert backend.step_meta(wl.pool).decode_plan() == (29 - 2 * 6, 29, 4)
    _assert_close(out.float().cpu().numpy(), _oracle_renumbered(vo, wl),
                  f"decode shared packs on a {num_blocks}-block pool")
    del wl, out
    import torch
    torch.cuda.empty_cache()


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


@pytest.mark.parametrize("case,slots", [("cfg3", ""), ("cfg3", "1"), ("edges", ""), ("edges", "1"),
                                        ("edges", "3")])
def test_prefill_pipe_kernel_bitwise_equals_dma_kernel(vo, gpu_backend, monkeypatch, case, slots):
    """The pipelined 4-wavefront kernel computes each row with the 32-row
    kernels' operations in their order, so its output is bitwise the
    8-wavefront DMA kernel's (VO_PREFILL_PIPE=0): at BASELINE config 3's full
    size, and on items that end before, at and past tile and 32-row-group
    boundaries (so that the pipelined loop runs 0, 1, 2 and many tiles and
    the masked tiles follow it in either S buffer).  The kernel is
    persistent: slots "1" and "3" deal all items to one or three workgroups
    per KV head, so that items of every length follow each other through
    the LDS ring (tile 0 at every stage, prefetched or not)."""
    _say(f"prefill pipelined kernel vs DMA kernel bitwise ({case}, slots {slots or 'default'})")
    monkeypatch.setenv("VO_PREFILL_NARROW", "0")
    monkeypatch.setenv("VO_PREFILL_PIPE_SLOTS", slots)
    if case == "cfg3":
        ctx, new = W.cfg3_context_lens(), [512] * 8
        nb = 12000
    else:
        ctx = [0, 63, 64, 127, 128, 130, 191, 192, 255, 1000, 3001, 4095]
        new = [64, 1, 65, 2, 64, 31, 33, 1, 129, 40, 77, 64]
        nb = 1200
    wl = W.build(vo, gpu_backend, kind="prefill", heads=32, kv_heads=8, head_dim=128,
                 block_size=16, num_blocks=nb, context_lens=ctx, num_new=new, seed=71)
    outs = {}
    for pipe in ("1", "0"):
        monkeypatch.setenv("VO_PREFILL_PIPE", pipe)
        out, ran = _out_with_prefill_instances(vo, wl, gpu_backend)
        assert ran == ({"prefill_pipe"} if pipe == "1" else {"prefill_dma"}), ran
        outs[pipe] = out.clone()
    assert np.array_equal(_bits(outs["1"]), _bits(outs["0"]))


MIXED_CTX = [0, 1, 15, 16, 17, 63, 64, 65, 700, 1023, 1024, 1025, 3000, 0, 100, 700, 5, 2047]
MIXED_NEW = [1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 64, 100, 200, 2, 33]


def test_mixed_step_matches_oracle(vo, gpu_backend):
    """One prefill_attention call carrying decode sequences (one new row, run
    on the split-K decode kernel) and chunks (run on the MFMA prefill
    kernel), as a continuous-batching step does (model.rs:312-319)."""
    _say("mixed step vs oracle")
    wl = W.build(vo, gpu_backend, kind="prefill", heads=32, kv_heads=8, head_dim=128,
                 block_size=16, num_blocks=1500, context_lens=MIXED_CTX, num_new=MIXED_NEW,
                 seed=41)
    out = _out(wl, gpu_backend)
    want = W.oracle_attention(orc, wl)
    _assert_close(out.float().cpu().numpy(), want, "mixed step")


def test_mixed_step_decode_rows_bitwise_equal_decode_call(vo, gpu_backend):
    """A sequence with one new row gets, inside a mixed prefill call, bitwise
    the output decode_attention gives it: its arithmetic does not depend on
    the rest of the batch (CLAUDE.md batch invariance, model.rs:539-584)."""
    import torch
    _say("mixed step decode rows == decode call")
    wl = W.build(vo, gpu_backend, kind="prefill", heads=32, kv_heads=8, head_dim=128,
                 block_size=16, num_blocks=1500, context_lens=MIXED_CTX, num_new=MIXED_NEW,
                 seed=42)
    mixed = _bits(_out(wl, gpu_backend))
    starts = np.asarray(wl.meta.seq_row_starts, dtype=np.int64)
    dec_seqs = [s for s in range(len(MIXED_CTX)) if MIXED_NEW[s] == 1]
    rows = [int(starts[s]) for s in dec_seqs]
    meta = vo.DecodeMeta.new([vo.DecodeSeq(MIXED_CTX[s], wl.tables[s]) for s in dec_seqs], 16)
    q = wl.q[torch.tensor(rows, device=wl.q.device)].contiguous()
    dec = _bits(gpu_backend.decode_attention(q, wl.pool, 0, meta))
    assert np.array_equal(dec, mixed[rows])


def test_mixed_step_routing_off_matches_oracle(vo, monkeypatch):
    """With the decode-row routing switched off (VO_PREFILL_DECODE_ROWS=0)
    every row runs on the prefill kernel; results agree within tolerance."""
    monkeypatch.setenv("VO_PREFILL_DECODE_ROWS", "0")
    _say("mixed step, routing off")
    backend = vo.HipBackend(device=0, max_seqs=64, max_rows=W.FILL_ROWS, max_table_entries=4096,
                            max_query_heads=32)
    wl = W.build(vo, backend, kind="prefill", heads=32, kv_heads=8, head_dim=128,
                 block_size=16, num_blocks=1500, context_lens=MIXED_CTX, num_new=MIXED_NEW,
                 seed=43)
    out = _out(wl, backend)
    want = W.oracle_attention(orc, wl)
    _assert_close(out.float().cpu().numpy(), want, "mixed step, routing off")


def test_mixed_step_cfg4_attention_full_size(vo):
    """BASELINE config 4's attention shape: 256 decode sequences (lognormal
    context, median 1024) + two 512-row chunks in one prefill_attention call;
    every row on the GPU, a sample of rows by the oracle."""
    _say("mixed step cfg4 attention shape")
    ctx, new = W.cfg4_attention_lens()
    backend = vo.HipBackend(device=0, max_seqs=300, max_rows=W.FILL_ROWS,
                            max_table_entries=30000, max_query_heads=32)
    wl = W.build(vo, backend, kind="prefill", heads=32, kv_heads=8, head_dim=128,
                 block_size=16, num_blocks=30000, context_lens=ctx, num_new=new, seed=4)
    out = _out(wl, backend).float().cpu().numpy()
    starts = np.asarray(wl.meta.seq_row_starts, dtype=np.int64)
    rows = np.unique(np.concatenate([np.arange(0, 256, 5), np.arange(256, wl.rows, 37),
                                     starts[-3:] - 1]))
    want = W.oracle_attention(orc, wl, rows=rows)
    _assert_close(out[rows], want, "cfg4 attention")


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


# ---------------------------------------------------------------------------
# Step metadata built on the device (PrefillMeta::new / DecodeMeta::new)
# ---------------------------------------------------------------------------
def _device_rows(vo, seq_row_starts, context_lens, tables, block_size):
    import torch
    off = np.concatenate([[0], np.cumsum([len(t) for t in tables])]).astype(np.int64)
    flat = np.concatenate([np.asarray(t, np.uint32) for t in tables] + [np.zeros(1, np.uint32)])
    d = lambda a: torch.tensor(np.asarray(a, np.int64).astype(np.uint32).view(np.int32),
                               device="cuda:0")
    T = int(seq_row_starts[-1])
    pos, slot, rseq, rkeys, err = vo.prefill_meta_build_device(
        d(seq_row_starts), d(context_lens), d(off), d(flat), block_size, T)
    torch.cuda.synchronize()
    u = lambda t: t.cpu().numpy().view(np.uint32)
    return u(pos), u(slot), u(rseq), u(rkeys), int(err.cpu()[0])


def test_device_meta_reference_kats(vo):
    """paged.rs:230-285 known answers, built on the device."""
    _say("device meta KATs")
    pos, slot, rseq, rkeys, err = _device_rows(vo, [0, 5, 8], [0, 6], [[3, 0], [1, 4, 6]], 4)
    assert err == 0
    assert list(pos) == [0, 1, 2, 3, 4, 6, 7, 8]
    assert list(slot) == [12, 13, 14, 15, 0, 18, 19, 24]
    assert list(rseq) == [0, 0, 0, 0, 0, 1, 1, 1]
    assert list(rkeys) == [1, 2, 3, 4, 5, 7, 8, 9]
    pos, slot, rseq, rkeys, err = _device_rows(vo, [0, 1, 2], [0, 6], [[9], [2, 5]], 4)
    assert err == 0
    assert list(pos) == [0, 6] and list(slot) == [36, 22]
    assert list(rseq) == [0, 1] and list(rkeys) == [1, 7]


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_device_meta_bit_exact_vs_oracle(vo, seed):
    """Random batches (empty sequences, chunks ending on and off block
    boundaries, decode-shaped steps): the device arrays equal the oracle's
    PrefillMeta / DecodeMeta bit for bit."""
    _say(f"device meta vs oracle seed={seed}")
    rng = np.random.default_rng(seed)
    for trial in range(20):
        S = int(rng.integers(1, 40))
        bs = int(rng.choice([1, 4, 16, 32]))
        decode = trial % 4 == 0
        ctx = rng.integers(0, 3000, S)
        new = np.ones(S, np.int64) if decode else rng.integers(0, 300, S)
        hi = (1 << 32) - 1 if trial % 5 == 1 else 1 << 20  # u32 slot arithmetic wraps
        tables = [rng.integers(0, hi, -(-int(c + n) // bs) + int(rng.integers(0, 3)),
                               dtype=np.uint64).astype(np.uint32) for c, n in zip(ctx, new)]
        starts = np.concatenate([[0], np.cumsum(new)])
        pos, slot, rseq, rkeys, err = _device_rows(vo, starts, ctx, tables, bs)
        assert err == 0
        if decode:
            want = orc.decode_meta([(int(c), t) for c, t in zip(ctx, tables)], bs)
        else:
            want = orc.prefill_meta([(int(c), int(n), t) for c, n, t in zip(ctx, new, tables)],
                                    bs)
        assert np.array_equal(pos, np.asarray(want["positions"], np.uint32))
        assert np.array_equal(slot, np.asarray(want["slot_mapping"], np.uint32))
        assert np.array_equal(rseq, np.asarray(want["row_seq"], np.uint32))
        assert np.array_equal(rkeys, np.asarray(want["row_num_keys"], np.uint32))


def test_device_meta_flags_uncovered_rows(vo):
    """paged.rs:287-318: 5 tokens on a one-block table of block size 4 are not
    covered; the device build flags it and marks the uncovered row's slot."""
    _say("device meta coverage flag")
    pos, slot, rseq, rkeys, err = _device_rows(vo, [0, 5], [0], [[7]], 4)
    assert err == 1
    assert list(slot[:4]) == [28, 29, 30, 31] and slot[4] == 0xffffffff



# ---------------------------------------------------------------------------
# RoPE (rope.rs) alone and fused with the cache write
# ---------------------------------------------------------------------------
def _bf16_bits_of(x):
    """Round f32 -> bf16 (nearest even), as uint16 bit patterns."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r


def _as_f32(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("hd,theta,cols_heads", [(128, 500000.0, 32), (64, 10000.0, 4),
                                                 (8, 10000.0, 6), (128, 10000.0, 8)])
def test_rope_bit_exact_vs_oracle(vo, gpu_backend, hd, theta, cols_heads):
    """Backend::rope on bf16 rows equals the oracle's f32 rotation of the same
    values, rounded to bf16, bit for bit (cpu/mod.rs:231-255, rope.rs:86-100)."""
    import torch
    _say(f"rope hd={hd} theta={theta}")
    max_len = 9000
    table = vo.RopeTable(hd, theta, max_len)
    rng = np.random.default_rng(hd)
    ctx = [0, 5, 700, 4095, 8000]
    new = [40, 1, 33, 1, 999]
    wl = W.build(vo, gpu_backend, kind="prefill", heads=cols_heads, kv_heads=2 if hd == 8 else 1,
                 head_dim=hd, block_size=16, num_blocks=1000, context_lens=ctx, num_new=new,
                 seed=hd + 1, keep_host=False)
    x = torch.tensor(rng.standard_normal((wl.rows, cols_heads * hd)), dtype=torch.float32,
                     device="cuda:0").to(torch.bfloat16)
    x0 = _as_f32(x)
    gpu_backend.rope(table, x, wl.pool, wl.meta, hd)
    torch.cuda.synchronize()
    c, s = orc.rope_table(orc.rope_inv_freq(hd, theta), max_len)
    want = _bf16_bits_of(orc.rope_apply(x0, wl.meta.positions, c, s))
    assert np.array_equal(_bits(x).view(np.uint16), want)


def test_rope_errors_match_reference(vo, gpu_backend):
    """PositionOutOfRange {pos, max} for the first position past the table
    (cpu/mod.rs:241-246); Shape for a head_dim the table was not built for."""
    import torch
    _say("rope errors")
    table = vo.RopeTable(64, 10000.0, 100)
    wl = W.build(vo, gpu_backend, kind="prefill", heads=2, kv_heads=1, head_dim=64,
                 block_size=16, num_blocks=64, context_lens=[90], num_new=[20], seed=5,
                 keep_host=False)
    x = torch.zeros((20, 128), dtype=torch.bfloat16, device="cuda:0")
    with pytest.raises(vo.PositionOutOfRange) as e:
        gpu_backend.rope(table, x, wl.pool, wl.meta, 64)
    assert e.value.value == 100 and e.value.limit == 100
    with pytest.raises(vo.ShapeError):
        gpu_backend.rope(table, x, wl.pool, wl.meta, 32)


@pytest.mark.parametrize("hd,heads,kvh", [(128, 32, 8), (64, 4, 2), (128, 64, 8)])
def test_rope_write_kv_fused_matches_unfused(vo, gpu_backend, hd, heads, kvh):
    """The fused launch leaves q and the pool bitwise as rope(q); rope(k);
    write_kv(k, v) does (model.rs:307-311), on a mixed step (chunks that start
    mid-block, whole blocks, decode rows)."""
    import torch
    _say(f"rope_write_kv hd={hd} heads={heads}")
    table = vo.RopeTable(hd, 500000.0, 6000)
    ctx = [0, 3, 16, 100, 2000, 777, 15]
    new = [70, 1, 33, 1, 129, 1, 17]
    wl = W.build(vo, gpu_backend, kind="prefill", heads=heads, kv_heads=kvh, head_dim=hd,
                 block_size=16, num_blocks=900, context_lens=ctx, num_new=new, seed=hd + heads,
                 num_layers=2, keep_host=False)
    k = wl.k_new.clone()
    v = wl.v_new.clone()
    q_ref = wl.q.clone()
    gpu_backend.rope(table, q_ref, wl.pool, wl.meta, hd)
    k_rot = k.clone()
    gpu_backend.rope(table, k_rot, wl.pool, wl.meta, hd)
    gpu_backend.write_kv(wl.pool, 0, k_rot, v, wl.meta)
    q_fused = wl.q.clone()
    gpu_backend.rope_write_kv(wl.pool, 1, table, q_fused, k, v, wl.meta)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(q_fused), _bits(q_ref))
    assert np.array_equal(_bits(k), _bits(wl.k_new))  # the caller's keys stay unrotated
    for s in range(len(ctx)):
        n = ctx[s] + new[s]
        meta = wl.meta
        k0, v0 = gpu_backend.read_kv(wl.pool, 0, meta, s, n)
        k1, v1 = gpu_backend.read_kv(wl.pool, 1, meta, s, n)
        lo = ctx[s]
        assert np.array_equal(_bits(k1[lo:]), _bits(k0[lo:])), s
        assert np.array_equal(_bits(v1[lo:]), _bits(v0[lo:])), s


def test_rope_write_kv_repeated_slot_rotates_every_q_row(vo, gpu_backend):
    """A slot given twice keeps the later row in the cache (cpu/mod.rs:277-283)
    while both rows' q are rotated."""
    import torch
    _say("rope_write_kv repeated slot")
    hd, heads, kvh = 128, 8, 2
    table = vo.RopeTable(hd, 500000.0, 64)
    layout = vo.KvLayout(1, 8, 16, kvh, hd)
    pool = gpu_backend.alloc_kv_pool(layout)
    meta = dataclasses.replace(vo.PrefillMeta.new([vo.PrefillSeq(0, 3, [5])], 16),
                               slot_mapping=[80, 81, 80])
    g = torch.Generator(device="cuda:0")
    g.manual_seed(9)
    q = torch.randn((3, heads * hd), generator=g, device="cuda:0").to(torch.bfloat16)
    k = torch.randn((3, kvh * hd), generator=g, device="cuda:0").to(torch.bfloat16)
    v = torch.randn((3, kvh * hd), generator=g, device="cuda:0").to(torch.bfloat16)
    q_ref = q.clone()
    gpu_backend.rope(table, q_ref, pool, meta, hd)
    gpu_backend.rope_write_kv(pool, 0, table, q, k, v, meta)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(q), _bits(q_ref))
    kc, vc = gpu_backend.read_kv(pool, 0, meta, 0, 2)
    c, s = orc.rope_table(orc.rope_inv_freq(hd, 500000.0), 64)
    k_rot = _bf16_bits_of(orc.rope_apply(_as_f32(k), [0, 1, 2], c, s))
    assert np.array_equal(_bits(kc[0:1]).view(np.uint16), k_rot[2:3])
    assert np.array_equal(_bits(kc[1:2]).view(np.uint16), k_rot[1:2])
    assert np.array_equal(_bits(vc[0:1]), _bits(v[2:3]))


# ---------------------------------------------------------------------------
# Block manager + prefix cache feeding the GPU path
# ---------------------------------------------------------------------------
def test_copy_blocks_bitwise(vo, gpu_backend):
    """vo_kv_copy_blocks copies whole blocks of every layer's K and V."""
    import torch
    _say("copy_blocks")
    hd, kvh, bs = 128, 8, 16
    pool = gpu_backend.alloc_kv_pool(vo.KvLayout(3, 64, bs, kvh, hd))
    g = torch.Generator(device="cuda:0")
    g.manual_seed(3)
    slots = np.arange(64 * bs, dtype=np.uint32)
    k = torch.randn((64 * bs, kvh * hd), generator=g, device="cuda:0").to(torch.bfloat16)
    v = torch.randn((64 * bs, kvh * hd), generator=g, device="cuda:0").to(torch.bfloat16)
    for layer in range(3):
        gpu_backend.write_kv(pool, layer, k, v, slots)
    pairs = [(5, 40), (6, 41), (63, 0)]
    gpu_backend.copy_blocks(pool, pairs)
    for layer in range(3):
        for src, dst in pairs:
            a = gpu_backend.read_kv(pool, layer, vo.DecodeMeta.new([vo.DecodeSeq(0, [src])], bs), 0, bs)
            b = gpu_backend.read_kv(pool, layer, vo.DecodeMeta.new([vo.DecodeSeq(0, [dst])], bs), 0, bs)
            assert np.array_equal(_bits(a[0]), _bits(b[0])) and np.array_equal(_bits(a[1]), _bits(b[1]))
    with pytest.raises(vo.BlockOutOfRange):
        gpu_backend.copy_blocks(pool, [(64, 1)])
    with pytest.raises(vo.ShapeError):
        gpu_backend.copy_blocks(pool, [(1, 2), (2, 3)])


def test_block_manager_prefix_cache_and_fork_decode(vo, gpu_backend):
    """The block manager builds a prefix-shared batch (the prefix's KV is
    written once, by the first sequence), then forks a sequence and appends
    to both copies (copy on write through vo_kv_copy_blocks).  Decode
    attention over the manager's tables matches the oracle run on the same
    KV laid out in private, unshared tables."""
    import torch
    _say("block manager -> decode")
    hd, heads, kvh, bs = 128, 32, 8, 16
    width = kvh * hd
    bm = vo.BlockManager(600, bs)
    pool = gpu_backend.alloc_kv_pool(vo.KvLayout(1, 600, bs, kvh, hd))
    g = torch.Generator(device="cuda:0")
    g.manual_seed(11)
    rnd = lambda n: torch.randn((n, width), generator=g, device="cuda:0").to(torch.bfloat16)
    prefix = list(range(1000))
    kv = {}          # seq -> (k, v) for every position, host f32 (what the oracle reads)
    prompts = {s: prefix + [2000 + s] * (37 * s + 5) for s in range(6)}
    prefix_kv = (rnd(1000), rnd(1000))
    for s, toks in prompts.items():
        cached = bm.add_sequence(s, toks)
        assert cached == (0 if s == 0 else 992)
        table = bm.block_table(s)
        n = len(toks)
        k_all = torch.cat([prefix_kv[0], rnd(n - 1000)])
        v_all = torch.cat([prefix_kv[1], rnd(n - 1000)])
        lo = cached
        slots = np.array([table[p // bs] * bs + p % bs for p in range(lo, n)], np.uint32)
        gpu_backend.write_kv(pool, 0, k_all[lo:].contiguous(), v_all[lo:].contiguous(), slots)
        kv[s] = [k_all, v_all]
    # fork sequence 3 and append one token to each copy
    bm.fork(3, 9)
    kv[9] = [t.clone() for t in kv[3]]
    for s in (3, 9):
        slot, copy = bm.append_token(s, 7)
        if copy is not None:
            gpu_backend.copy_blocks(pool, [copy])
        kn, vn = rnd(1), rnd(1)
        gpu_backend.write_kv(pool, 0, kn, vn, np.array([slot], np.uint32))
        kv[s][0] = torch.cat([kv[s][0], kn])
        kv[s][1] = torch.cat([kv[s][1], vn])
    bm.check()
    seqs = sorted(kv)
    tables = [bm.block_table(s) for s in seqs]
    ctx = [bm.num_tokens(s) - 1 for s in seqs]
    meta = vo.DecodeMeta.new([vo.DecodeSeq(c, t) for c, t in zip(ctx, tables)], bs)
    q = torch.randn((len(seqs), heads * hd), generator=g, device="cuda:0").to(torch.bfloat16)
    out = gpu_backend.decode_attention(q, pool, 0, meta).float().cpu().numpy()
    # oracle: each sequence's keys in private consecutive blocks
    opool = orc.Pool(1, 2000, bs, kvh, hd)
    otables, base = [], 0
    for s in seqs:
        n = kv[s][0].shape[0]
        nb = -(-n // bs)
        t = np.arange(base, base + nb, dtype=np.uint32)
        base += nb
        otables.append(t)
        opool.write_kv(0, kv[s][0].float().cpu().numpy(), kv[s][1].float().cpu().numpy(),
                       [int(t[p // bs]) * bs + p % bs for p in range(n)])
    want = opool.attention(q.float().cpu().numpy(), 0, otables, np.arange(len(seqs)),
                           np.asarray(ctx) + 1)
    _assert_close(out, want, "block manager decode")
