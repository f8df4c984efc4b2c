"""Llama::forward's op order with the trait's own arguments, over the C ABI.

crates/engine/src/model.rs:294-345 calls, in every layer, rope(q, positions),
rope(k, positions), write_kv(k, v, slots) and then prefill_attention or
decode_attention(meta), and after the layers of a prefill step
gather_rows(residual, meta.last_rows()).  Each of those ops receives host
arrays (mod.rs:105, :107-119, :121-149, :167).  The model here hands every
op exactly those arrays and uploads nothing ahead of the op that carries
them: vo_rope_positions, vo_write_kv_slots, vo_step_meta_sync_* and
vo_gather_rows take them.  The decode steps refill the same host buffers in
place, as an engine that keeps its step vectors would, so a library that
keyed its uploads on (pointer, length) would run on stale values.  Logits
are compared with the oracle's on config 1.
"""
import ctypes

import numpy as np
import pytest

import oracle as orc
import workloads as W
from test_gpu_abi_only import AbiModel, _check_logits

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-test] {msg}", flush=True)


class StepHost:
    """The host arrays of one step (PrefillMeta / DecodeMeta fields,
    paged.rs:97-114 and :173-186), kept in buffers that a step of the same
    sizes refills in place."""

    def __init__(self):
        self.bufs = {}

    def _put(self, name, values, dtype):
        a = np.asarray(values, dtype=dtype).reshape(-1)
        if a.size == 0:
            a = np.zeros(0, dtype)
        b = self.bufs.get(name)
        if b is not None and b.shape == a.shape:
            b[...] = a
        else:
            b = self.bufs[name] = a.copy()
        return b

    def fill(self, vo, meta, prefill):
        off, flat = vo._csr(meta.block_tables)
        self.block_size = meta.block_size
        self.num_seqs = meta.num_seqs()
        self.table_off = self._put("table_off", off, np.uint64)
        self.tables = self._put("tables", flat, np.uint32)
        self.positions = self._put("positions", meta.positions, np.uint32)
        self.slots = self._put("slots", meta.slot_mapping, np.uint32)
        self.row_seq = self._put("row_seq", meta.row_seq, np.uint64)
        self.row_num_keys = self._put("row_num_keys", meta.row_num_keys, np.uint64)
        if prefill:
            self.context_lens = self._put("context_lens", meta.context_lens, np.uint64)
            self.seq_row_starts = self._put("seq_row_starts", meta.seq_row_starts, np.uint64)
            self.last_rows = self._put("last_rows", meta.last_rows(), np.uint32)
        return self

    def addresses(self):
        return {k: v.ctypes.data for k, v in self.bufs.items()}


def _p32(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32))


def _p64(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64))


class TraitModel(AbiModel):
    """AbiModel's forward with each op taking the trait's own host arrays,
    and the element types of a backend that sees only the trait's calls:
    every GEMM output is bf16 except the tied LM head's f32 logits, and add
    widens bf16 into the f32 residual."""

    def _sync(self, h, prefill):
        lib = self.lib
        if prefill:
            return lib.vo_step_meta_sync_prefill(
                self.meta, h.block_size, h.num_seqs, _p64(h.table_off), _p32(h.tables),
                _p64(h.context_lens), _p64(h.seq_row_starts), len(h.positions),
                _p32(h.positions), _p32(h.slots), _p64(h.row_seq), _p64(h.row_num_keys), None)
        return lib.vo_step_meta_sync_decode(
            self.meta, h.block_size, h.num_seqs, _p64(h.table_off), _p32(h.tables),
            _p32(h.positions), _p32(h.slots), _p64(h.row_seq), _p64(h.row_num_keys), None)

    def forward_trait(self, tokens, h, prefill):
        """model.rs:294-345 with host arrays h; returns (ids, logits)."""
        vo, lib, cfg, A = self.vo, self.lib, self.cfg, self.arena
        chk, bf, f32 = vo._check, vo.VO_DTYPE_BF16, vo.VO_DTYPE_F32
        T, S = len(tokens), h.num_seqs
        H, hd, V, F = cfg.hidden_size, cfg.head_dim, cfg.vocab_size, cfg.intermediate_size
        qd, kvd = cfg.num_attention_heads * hd, cfg.num_key_value_heads * hd
        eps = float(cfg.rms_norm_eps)
        toks = vo._u32(tokens)
        P = A.ptr
        with A.scope():
            residual = A.alloc(T, H)                                      # f32
            chk(lib.vo_step_meta_upload_tokens(self.meta, vo._p32(toks), T, None))
            chk(lib.vo_embed(self.embed.ptr, V, H, self.meta, T, P(residual), None))
            for li, L in enumerate(self.layers):
                with A.scope():
                    normed = A.alloc(T, H)                                # bf16
                    chk(lib.vo_rmsnorm(P(residual), T, H, L["attn_norm"].ptr, H, eps,
                                       P(normed), None))
                    q, k, v = A.alloc(T, qd), A.alloc(T, kvd), A.alloc(T, kvd)
                    for out, wname, n in ((q, "wq", qd), (k, "wk", kvd), (v, "wv", kvd)):
                        chk(lib.vo_matmul(self.gemm, P(normed), T, H, L[wname].ptr, n, H, P(out),
                                          bf, 0, None))
                    # rope(q, positions); rope(k, positions)       model.rs:307-308
                    chk(lib.vo_rope_positions(self.rope, P(q), T, qd, hd, _p32(h.positions),
                                              len(h.positions), self.meta, None))
                    chk(lib.vo_rope_positions(self.rope, P(k), T, kvd, hd, _p32(h.positions),
                                              len(h.positions), self.meta, None))
                    # write_kv(k, v, slots)                          model.rs:311
                    chk(lib.vo_write_kv_slots(self.pool, li, P(k), P(v), T, kvd, _p32(h.slots),
                                              len(h.slots), self.meta, None))
                    # prefill_attention / decode_attention(meta)     model.rs:312-319
                    attn = A.alloc(T, qd)
                    chk(self._sync(h, prefill))
                    fn = lib.vo_prefill_attention if prefill else lib.vo_decode_attention
                    chk(fn(P(q), T, qd, self.pool, li, self.meta, P(attn), None))
                    attn_out = A.alloc(T, H)                              # bf16
                    chk(lib.vo_matmul(self.gemm, P(attn), T, qd, L["wo"].ptr, H, qd,
                                      P(attn_out), bf, 0, None))
                    chk(lib.vo_add(P(residual), P(attn_out), bf, T, H, None))
                with A.scope():
                    normed = A.alloc(T, H)
                    chk(lib.vo_rmsnorm(P(residual), T, H, L["mlp_norm"].ptr, H, eps,
                                       P(normed), None))
                    gate, up = A.alloc(T, F), A.alloc(T, F)
                    chk(lib.vo_matmul(self.gemm, P(normed), T, H, L["w_gate"].ptr, F, H, P(gate),
                                      bf, 0, None))
                    chk(lib.vo_matmul(self.gemm, P(normed), T, H, L["w_up"].ptr, F, H, P(up),
                                      bf, 0, None))
                    chk(lib.vo_silu_mul(P(gate), F, P(up), F, T, F, P(gate), F, None))
                    down = A.alloc(T, H)                                  # bf16
                    chk(lib.vo_matmul(self.gemm, P(gate), T, F, L["w_down"].ptr, H, F, P(down),
                                      bf, 0, None))
                    chk(lib.vo_add(P(residual), P(down), bf, T, H, None))
            normed = A.alloc(S, H)
            if prefill:
                # gather_rows(residual, meta.last_rows()); rmsnorm   model.rs:337-340
                last = A.alloc(S, H)                                      # f32
                chk(lib.vo_gather_rows(P(residual), f32, T, H, _p32(h.last_rows),
                                       len(h.last_rows), self.meta, P(last), None))
                chk(lib.vo_rmsnorm(P(last), S, H, self.final_norm.ptr, H, eps, P(normed), None))
            else:
                # rmsnorm(residual)                                   model.rs:341
                chk(lib.vo_rmsnorm(P(residual), S, H, self.final_norm.ptr, H, eps, P(normed),
                                   None))
            logits = A.alloc(S, V)                                        # f32
            chk(lib.vo_matmul(self.gemm, P(normed), S, H, self.embed.ptr, V, H, P(logits),
                              f32, 0, None))
            ids_dev = A.alloc(S, 1)
            ids = np.zeros(S, np.uint32)
            chk(lib.vo_argmax(P(logits), f32, S, V,
                              ctypes.cast(P(ids_dev), ctypes.POINTER(ctypes.c_uint32)),
                              vo._p32(ids), None))
            out = self.ws.read(logits, f32)
        assert A.top == 0
        return ids, out


def test_trait_order_cfg1_prefill_then_decodes_match_oracle(vo):
    """Config 1 in Llama::forward's order with the trait's arguments: one
    batched prefill of four prompts, then five decode steps of four
    sequences whose host arrays refill the previous step's buffers; every
    step's logits against the oracle's."""
    cfg = W.cfg1_config()
    w = W.bf16_weights(W.normal_weights(cfg, 103))
    rng = np.random.default_rng(3)
    lens = [17, 33, 64, 100]
    steps = 5
    prompts = [list(map(int, rng.integers(0, cfg.vocab_size, n))) for n in lens]
    tables = [list(map(int, t))
              for t in W.split_tables(rng, [-(-(n + steps + 1) // 16) for n in lens], 64)]
    om = orc.Llama(cfg, w, num_blocks=64, block_size=16, max_len=256)
    gm = TraitModel(vo, cfg, w, max_tokens=256, max_seqs=4, num_blocks=64, block_size=16,
                    max_len=256)
    try:
        _say("trait order cfg1: prefill")
        want_ids, want = om.prefill(sum(prompts, []), [(0, n, t) for n, t in zip(lens, tables)], 16)
        meta = vo.PrefillMeta.new([vo.PrefillSeq(0, n, t) for n, t in zip(lens, tables)], 16)
        host = StepHost().fill(vo, meta, prefill=True)
        ids, got = gm.forward_trait(sum(prompts, []), host, prefill=True)
        worst = _check_logits(ids, got, want_ids, want, "prefill")
        ctx = list(lens)
        dhost = StepHost()
        addresses = None
        for step in range(steps):
            toks = [int(i) for i in want_ids]
            want_ids, want = om.decode(toks, [(c, t) for c, t in zip(ctx, tables)], 16)
            dmeta = vo.DecodeMeta.new([vo.DecodeSeq(c, t) for c, t in zip(ctx, tables)], 16)
            dhost.fill(vo, dmeta, prefill=False)
            if addresses is None:
                addresses = dhost.addresses()
            else:
                # the same host buffers, refilled with this step's values
                assert dhost.addresses() == addresses
            ids, got = gm.forward_trait(toks, dhost, prefill=False)
            worst = max(worst, _check_logits(ids, got, want_ids, want, f"decode {step}"))
            ctx = [c + 1 for c in ctx]
        _say(f"trait order cfg1: worst err/tolerance {worst:.3f}")
    finally:
        gm.close()


def test_gather_rows_matches_indexing(vo, gpu_backend):
    """Backend::gather_rows (cpu/mod.rs:360-368): bitwise row copies of f32
    and bf16 rows, repeated and out-of-order indices, the meta's last rows
    and other rows; the first index past x fails (arena/ops.rs:242-244)."""
    import torch
    layout = vo.KvLayout(1, 8, 16, 2, 64)
    pool = gpu_backend.alloc_kv_pool(layout)
    meta = vo.PrefillMeta.new([vo.PrefillSeq(0, 5, [0]), vo.PrefillSeq(3, 4, [1])], 16)
    gpu_backend.step_meta(pool).sync(meta)
    g = torch.Generator(device="cuda").manual_seed(7)
    for dtype, cols in ((torch.float32, 4096), (torch.float32, 37), (torch.bfloat16, 4096),
                        (torch.bfloat16, 38)):
        x = torch.randn((9, cols), generator=g, device="cuda").to(dtype)
        for rows in (list(meta.last_rows()), [8, 0, 8, 3, 1], [2]):
            out = gpu_backend.gather_rows(x, rows, pool)
            torch.cuda.synchronize()
            want = x[torch.tensor(rows, device="cuda").long()]
            assert torch.equal(out.view(torch.int16 if dtype == torch.bfloat16 else torch.int32),
                               want.view(torch.int16 if dtype == torch.bfloat16 else torch.int32))
    x = torch.zeros((3, 8), device="cuda")
    with pytest.raises(vo.ShapeError, match=r"gather_rows: row 3 of x \[3, 8\]"):
        gpu_backend.gather_rows(x, [0, 3], pool)
    xb = torch.zeros((3, 7), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(vo.InvalidArgument):
        gpu_backend.gather_rows(xb, [0], pool)


def test_rope_positions_matches_meta_rope(vo, gpu_backend):
    """vo_rope_positions is vo_rope on the caller's positions: bitwise equal
    on the meta's own positions and on others (the aux copy, refilled when
    the values change), with vo_rope's errors."""
    import torch
    layout = vo.KvLayout(1, 16, 16, 2, 128)
    pool = gpu_backend.alloc_kv_pool(layout)
    table = vo.RopeTable(128, 500000.0, 64, device=0)
    g = torch.Generator(device="cuda").manual_seed(9)
    x = torch.randn((6, 512), generator=g, device="cuda").to(torch.bfloat16)
    meta_a = vo.PrefillMeta.new([vo.PrefillSeq(0, 6, [0])], 16)             # positions 0..5
    meta_b = vo.PrefillMeta.new([vo.PrefillSeq(40, 6, [0, 1, 2, 3])], 16)    # positions 40..45
    m = gpu_backend.step_meta(pool)
    for want_meta, other in ((meta_a, meta_b), (meta_b, meta_a)):
        m.upload(want_meta)
        ref = x.clone()
        gpu_backend.rope(table, ref, pool, want_meta, 128)
        same = x.clone()
        gpu_backend.rope_positions(table, same, pool, want_meta.positions, 128)
        m.upload(other)          # the meta now holds the other positions: aux path
        aux = x.clone()
        gpu_backend.rope_positions(table, aux, pool, want_meta.positions, 128)
        aux2 = x.clone()         # the aux copy again, unchanged values
        gpu_backend.rope_positions(table, aux2, pool, want_meta.positions, 128)
        torch.cuda.synchronize()
        for got in (same, aux, aux2):
            assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    with pytest.raises(vo.PositionOutOfRange) as e:
        gpu_backend.rope_positions(table, x, pool, [0, 1, 70, 2, 80, 3], 128)
    assert e.value.value == 70 and e.value.limit == 64
    with pytest.raises(vo.ShapeError):
        gpu_backend.rope_positions(table, x, pool, [0, 1, 2], 128)
    table.close()


def test_write_kv_slots_checks_before_uploading(vo, gpu_backend):
    """vo_write_kv_slots refuses rows != slots before it uploads anything:
    the meta still holds its step, and attention on it is unchanged."""
    import torch
    layout = vo.KvLayout(1, 8, 16, 2, 64)
    pool = gpu_backend.alloc_kv_pool(layout)
    g = torch.Generator(device="cuda").manual_seed(11)
    kv = [torch.randn((20, 128), generator=g, device="cuda").to(torch.bfloat16)
          for _ in range(2)]
    meta = vo.PrefillMeta.new([vo.PrefillSeq(0, 20, [2, 5])], 16)
    m = gpu_backend.step_meta(pool)
    m.sync(meta)
    lib = vo.lib
    slots = vo._u32(meta.slot_mapping)
    vo._check(lib.vo_write_kv_slots(pool.handle, 0, vo._dev_ptr(kv[0]), vo._dev_ptr(kv[1]), 20,
                                    128, vo._p32(slots), 20, m.handle, vo._stream_ptr(None)))
    q = torch.randn((20, 256), generator=g, device="cuda").to(torch.bfloat16)
    before = gpu_backend.prefill_attention(q, pool, 0, meta)
    with pytest.raises(vo.ShapeError):
        vo._check(lib.vo_write_kv_slots(pool.handle, 0, vo._dev_ptr(kv[0]), vo._dev_ptr(kv[1]),
                                        20, 128, vo._p32(slots), 19, m.handle,
                                        vo._stream_ptr(None)))
    after = torch.empty_like(q)
    vo._check(lib.vo_prefill_attention(vo._dev_ptr(q), 20, 256, pool.handle, 0, m.handle,
                                       vo._dev_ptr(after), vo._stream_ptr(None)))
    torch.cuda.synchronize()
    assert torch.equal(before.view(torch.int16), after.view(torch.int16))
