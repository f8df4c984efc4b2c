"""vo_decode_attention_static, the decode entry point that allocates nothing,
against vo_decode_attention through the C ABI: two calls in a row, the second
with a smaller input, each bitwise equal to the existing entry point's
output; then the checks it runs on the device (a block id past the pool, a
table that does not cover a row's keys) and on the host (capacity)."""
import ctypes

import numpy as np
import pytest

import workloads as W

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-test] {msg}", flush=True)


def _bits(t):
    import torch
    return t.contiguous().view(torch.int16).cpu().numpy()


def _device_meta(wl):
    """DecodeMeta's tables and key counts as device u32 arrays (int32 tensors)."""
    import torch
    off = np.zeros(len(wl.tables) + 1, np.uint32)
    off[1:] = np.cumsum([len(t) for t in wl.tables])
    flat = np.concatenate([np.asarray(t, np.uint32) for t in wl.tables])
    keys = np.asarray(wl.meta.row_num_keys, np.uint32)
    dev = [torch.from_numpy(a.view(np.int32)).to("cuda:0") for a in (off, flat, keys)]
    return dev, int(flat.size)


def _static(vo, wl, q, dmeta, entries, max_keys, errors, out=None):
    import torch
    if out is None:
        out = torch.full_like(q, 7.0)
    off, flat, keys = dmeta
    rc = vo.lib.vo_decode_attention_static(
        vo._vp(q.data_ptr()), q.shape[0], q.shape[1], wl.pool.handle, wl.layer,
        vo._vp(off.data_ptr()), vo._vp(flat.data_ptr()), entries, vo._vp(keys.data_ptr()),
        max_keys, vo._vp(out.data_ptr()), vo._vp(errors.data_ptr()),
        vo._stream_ptr(None))
    return rc, out


@pytest.mark.parametrize("heads", [32, 64])
def test_static_decode_equals_decode_attention_two_calls(vo, heads):
    import torch
    backend = vo.HipBackend(device=0, max_seqs=64, max_rows=W.FILL_ROWS, max_table_entries=20000,
                            max_query_heads=heads)
    errors = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    # First call: 64 sequences, contexts U[512, 4096] (BASELINE config 2's).
    # Second call, smaller: 16 sequences, contexts 0 .. 3000 (one empty, edge
    # lengths around the 2048-key split).
    cases = [("64 seqs", W.cfg2_context_lens(), 20000, 4097),
             ("16 seqs", np.array([0, 1, 15, 16, 17, 33, 500, 2047, 2048, 2049, 2500, 3000,
                                   64, 100, 1024, 4000]), 4000, 4001)]
    for name, ctx, nblocks, max_keys in cases:
        _say(f"static decode heads={heads}: {name}")
        wl = W.build(vo, backend, kind="decode", heads=heads, kv_heads=8, head_dim=128,
                     block_size=16, num_blocks=nblocks, context_lens=ctx, seed=len(ctx) + heads,
                     keep_host=False)
        want = backend.decode_attention(wl.q, wl.pool, 0, wl.meta)
        dmeta, entries = _device_meta(wl)
        rc, got = _static(vo, wl, wl.q, dmeta, entries, max_keys, errors)
        vo._check(rc)
        torch.cuda.synchronize()
        assert int(errors.item()) == 0
        assert np.array_equal(_bits(got), _bits(want)), name
        # the same call again on the same scratch gives the same bits
        rc, again = _static(vo, wl, wl.q, dmeta, entries, max_keys, errors)
        vo._check(rc)
        assert np.array_equal(_bits(again), _bits(want)), name + " (repeated)"


@pytest.mark.parametrize("case", ["3000 short rows", "shared prefix"])
def test_static_decode_many_rows_and_shared_prefix(vo, case):
    """Two more shapes, each bitwise equal to vo_decode_attention: 3000
    short rows (more rows than the plan kernel's 1024 threads, so each thread
    plans several), and 24 rows aliasing a 2048-key prefix, where
    vo_decode_attention runs the shared-pack kernel and the static call the
    register path.  The second call is the smaller one."""
    import torch
    rng = np.random.default_rng(17)
    if case == "3000 short rows":
        heads, ctx, shared = 16, rng.integers(0, 300, 3000), 0
        nblocks = int(sum(-(-(int(c) + 1) // 16) for c in ctx)) + 16
    else:
        heads, ctx, shared = 32, 2048 + rng.integers(1, 600, 24), 2048
        nblocks = 4000
    _say(f"static decode: {case}")
    backend = vo.HipBackend(device=0, max_seqs=len(ctx), max_rows=W.FILL_ROWS,
                            max_table_entries=nblocks, max_query_heads=heads)
    wl = W.build(vo, backend, kind="decode", heads=heads, kv_heads=8, head_dim=128,
                 block_size=16, num_blocks=nblocks, context_lens=ctx, seed=19,
                 shared_prefix=shared, shared_count=len(ctx) if shared else 0, keep_host=False)
    want = backend.decode_attention(wl.q, wl.pool, 0, wl.meta)
    work, parts, _ = backend.step_meta(wl.pool).decode_plan()
    assert (work < parts) == bool(shared), (work, parts)   # packed items over the prefix
    dmeta, entries = _device_meta(wl)
    errors = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    rc, got = _static(vo, wl, wl.q, dmeta, entries, int(max(ctx)) + 1, errors)
    vo._check(rc)
    torch.cuda.synchronize()
    assert int(errors.item()) == 0
    assert np.array_equal(_bits(got), _bits(want)), case


def test_static_decode_device_checks_and_capacity(vo):
    import torch
    backend = vo.HipBackend(device=0, max_seqs=8, max_rows=W.FILL_ROWS, max_table_entries=512,
                            max_query_heads=32)
    ctx = [40, 100, 17, 300]
    wl = W.build(vo, backend, kind="decode", heads=32, kv_heads=8, head_dim=128, block_size=16,
                 num_blocks=64, context_lens=ctx, seed=3, keep_host=False)
    (off, flat, keys), entries = _device_meta(wl)

    def run(off_, flat_, keys_, max_keys=4096):
        errors = torch.zeros(1, dtype=torch.int32, device="cuda:0")
        rc, out = _static(vo, wl, wl.q, (off_, flat_, keys_), entries, max_keys, errors)
        torch.cuda.synchronize()
        return rc, out, int(errors.item())

    rc, out, e = run(off, flat, keys)
    assert rc == 0 and e == 0
    # A block id past the pool (attention.rs:130-147): flagged, zero rows, no pool read.
    bad = flat.clone()
    bad[5] = 64
    rc, out, e = run(off, bad, keys)
    assert rc == 0 and e == 1 and not out.float().abs().sum().item()
    # A row whose table does not cover its keys (paged.rs:64-80).
    short = keys.clone()
    short[1] = 16 * 7 + 1  # 7 blocks in its table
    rc, out, e = run(off, flat, short)
    assert rc == 0 and e == 1 and not out.float().abs().sum().item()
    # Keys above max_keys.
    rc, out, e = run(off, flat, keys, max_keys=100)
    assert rc == 0 and e == 1
    # Past the scratch's size: refused on the host, nothing enqueued.
    errors = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    rc, _ = _static(vo, wl, wl.q, (off, flat, keys), entries, 1 << 30, errors)
    assert rc == vo.VO_ERR_CAPACITY
    info = vo.vo_error_info()
    vo.lib.vo_last_error(ctypes.byref(info))
    assert b"static decode scratch" in info.op
