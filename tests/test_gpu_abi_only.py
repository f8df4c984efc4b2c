"""The C ABI alone runs the model: no torch allocation anywhere.

This is what a Rust ``HipBackend`` in crates/kernels would do through
``extern "C"``: every byte of device memory comes from the library --
the activation workspace (Backend::alloc_workspace, mod.rs:76-77), the
weights (Backend::upload, mod.rs:69-70), the KV pool, the step metadata, the
RoPE table and the GEMM handle -- and every op takes device addresses of
workspace Regions (mod.rs:31-38) handed out by a bump arena that follows
arena.rs (scopes free their temporaries) and is sized by model::arena_elems
(model.rs:76-90).  The op order is Llama::forward's (model.rs:269-356): q/k/v
as three GEMMs, rope(q), rope(k), write_kv, attention, o_proj, add, then the
SwiGLU block.  The logits are read back with Backend::read (mod.rs:177-181)
and compared with the oracle's on config 1.
"""
import ctypes

import numpy as np
import pytest

import oracle as orc
import workloads as W

pytestmark = pytest.mark.gpu

# Config-1 logit tolerance, as in test_gpu_layer (bf16 weights and
# activations against the f32 oracle on the same bf16-rounded weights).
LOGIT_ATOL, LOGIT_RTOL = 1e-2, 2e-2


def _say(msg):
    print(f"[gpu-test] {msg}", flush=True)


def arena_elems(cfg, max_tokens, max_seqs):
    """model.rs:76-90."""
    h, hd = cfg.hidden_size, cfg.head_dim
    q_dim, kv_dim = cfg.num_attention_heads * hd, cfg.num_key_value_heads * hd
    residual = max_tokens * h
    attention = max_tokens * (2 * h + 2 * q_dim + 2 * kv_dim)
    mlp = max_tokens * (2 * h + 2 * cfg.intermediate_size)
    last_rows = max_seqs * (2 * h + cfg.vocab_size)
    return residual + max(attention, mlp, last_rows)


class Arena:
    """arena.rs: a bump allocator over the workspace; ``scope`` frees what was
    allocated inside it."""

    def __init__(self, vo, ws):
        self.vo, self.ws = vo, ws
        self.capacity = ws.elems()
        self.top = 0
        self.high_water = 0

    def alloc(self, rows, cols):
        need = rows * cols
        if self.top + need > self.capacity:
            raise AssertionError("arena exhausted")
        r = self.vo.Region(self.top, rows, cols)
        self.top += need
        self.high_water = max(self.high_water, self.top)
        return r

    def ptr(self, r):
        return self.ws.ptr(r)

    class _Scope:
        def __init__(self, arena):
            self.arena = arena

        def __enter__(self):
            self.mark = self.arena.top
            return self.arena

        def __exit__(self, *exc):
            self.arena.top = self.mark
            return False

    def scope(self):
        return Arena._Scope(self)


class AbiModel:
    """Llama<HipBackend> over the C ABI only."""

    def __init__(self, vo, cfg, weights, max_tokens, max_seqs, num_blocks, block_size, max_len):
        self.vo, self.cfg = vo, cfg
        lib = vo.lib
        self.lib = lib
        self.ws = vo.Workspace(arena_elems(cfg, max_tokens, max_seqs))
        self.arena = Arena(vo, self.ws)
        up = vo.Weight
        self.embed = up(weights["embed"])
        self.final_norm = up(weights["final_norm"])
        self.layers = [{k: up(v) for k, v in L.items()} for L in weights["layers"]]
        hd = cfg.head_dim
        layout = vo.vo_kv_layout(cfg.num_hidden_layers, num_blocks, block_size,
                                 cfg.num_key_value_heads, hd)
        self.pool = vo._vp()
        vo._check(lib.vo_kv_pool_create(ctypes.byref(layout), 0, ctypes.byref(self.pool)))
        self.meta = vo._vp()
        vo._check(lib.vo_step_meta_create(self.pool, max_seqs, max_tokens, 4096,
                                          cfg.num_attention_heads, ctypes.byref(self.meta)))
        rs = cfg.rope_scaling
        rc = vo.vo_rope_config(hd, cfg.rope_theta, rs["factor"], rs["low_freq_factor"],
                               rs["high_freq_factor"], rs["original_max_position_embeddings"])
        self.rope = vo._vp()
        vo._check(lib.vo_rope_table_create(ctypes.byref(rc), max_len, 0, ctypes.byref(self.rope)))
        self.gemm = vo._vp()
        vo._check(lib.vo_gemm_create(0, 32 << 20, ctypes.byref(self.gemm)))
        self.block_size = block_size

    def close(self):
        lib = self.lib
        lib.vo_gemm_destroy(self.gemm)
        lib.vo_rope_table_destroy(self.rope)
        lib.vo_step_meta_destroy(self.meta)
        lib.vo_kv_pool_destroy(self.pool)
        for L in self.layers:
            for w in L.values():
                w.close()
        self.embed.close()
        self.final_norm.close()
        self.ws.close()

    def _upload(self, meta, prefill):
        vo = self.vo
        off, flat = vo._csr(meta.block_tables)
        if prefill:
            vo._check(self.lib.vo_step_meta_upload_prefill(
                self.meta, meta.block_size, meta.num_seqs(), vo._p64(off), vo._p32(flat),
                vo._p64(vo._u64a(meta.context_lens)), vo._p64(vo._u64a(meta.seq_row_starts)),
                meta.num_rows(), vo._p32(vo._u32(meta.positions)),
                vo._p32(vo._u32(meta.slot_mapping)), vo._p64(vo._u64a(meta.row_seq)),
                vo._p64(vo._u64a(meta.row_num_keys)), None))
        else:
            vo._check(self.lib.vo_step_meta_upload_decode(
                self.meta, meta.block_size, meta.num_seqs(), vo._p64(off), vo._p32(flat),
                vo._p32(vo._u32(meta.positions)), vo._p32(vo._u32(meta.slot_mapping)),
                vo._p64(vo._u64a(meta.row_seq)), vo._p64(vo._u64a(meta.row_num_keys)), None))

    def forward(self, tokens, meta, prefill):
        """model.rs:269-356; returns (next ids, logits [S, vocab])."""
        vo, lib, cfg, A = self.vo, self.lib, self.cfg, self.arena
        chk, bf, f32 = vo._check, vo.VO_DTYPE_BF16, vo.VO_DTYPE_F32
        T, S = len(tokens), meta.num_seqs()
        H, hd, V, F = cfg.hidden_size, cfg.head_dim, cfg.vocab_size, cfg.intermediate_size
        qd, kvd = cfg.num_attention_heads * hd, cfg.num_key_value_heads * hd
        eps = float(cfg.rms_norm_eps)
        self._upload(meta, prefill)
        toks = vo._u32(tokens)
        chk(lib.vo_step_meta_upload_tokens(self.meta, vo._p32(toks), T, None))
        P = A.ptr
        with A.scope():
            residual = A.alloc(T, H)                                      # f32
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
                    chk(lib.vo_rope(self.rope, P(q), T, qd, hd, self.meta, None))
                    chk(lib.vo_rope(self.rope, P(k), T, kvd, hd, self.meta, None))
                    chk(lib.vo_write_kv(self.pool, li, P(k), P(v), T, kvd, self.meta, None))
                    attn = A.alloc(T, qd)
                    fn = lib.vo_prefill_attention if prefill else lib.vo_decode_attention
                    chk(fn(P(q), T, qd, self.pool, li, self.meta, P(attn), None))
                    attn_out = A.alloc(T, H)                              # f32
                    chk(lib.vo_matmul(self.gemm, P(attn), T, qd, L["wo"].ptr, H, qd,
                                      P(attn_out), f32, 0, None))
                    chk(lib.vo_add(P(residual), P(attn_out), f32, T, H, None))
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
                    down = A.alloc(T, H)                                  # f32
                    chk(lib.vo_matmul(self.gemm, P(gate), T, F, L["w_down"].ptr, H, F, P(down),
                                      f32, 0, None))
                    chk(lib.vo_add(P(residual), P(down), f32, T, H, None))
            # gather_rows(last_rows) + rmsnorm (model.rs:336-342), one pass.
            normed = A.alloc(S, H)
            chk(lib.vo_rmsnorm_last_rows(P(residual), T, H, self.final_norm.ptr, H, eps,
                                         self.meta, P(normed), None))
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


def _check_logits(got_ids, got, want_ids, want, what):
    err = np.abs(got - want)
    tol = LOGIT_ATOL + LOGIT_RTOL * np.abs(want)
    assert (err <= tol).all(), f"{what}: max logit err {err.max():.3e}"
    top2 = np.sort(want, axis=1)[:, -2:]
    for s in range(want.shape[0]):
        if top2[s, 1] - top2[s, 0] > 2 * (LOGIT_ATOL + LOGIT_RTOL * abs(top2[s, 1])):
            assert got_ids[s] == want_ids[s], f"{what}: seq {s} id differs"
    return float((err / tol).max())


def test_abi_only_cfg1_prefill_and_decode_match_oracle(vo):
    """Config 1 through the C ABI only: one batched prefill of the four
    prompts and two decode steps, logits read back from the workspace and
    compared with the oracle's."""
    cfg = W.cfg1_config()
    w = W.bf16_weights(W.normal_weights(cfg, 101))
    rng = np.random.default_rng(1)
    lens = [17, 33, 64, 100]
    prompts = [list(map(int, rng.integers(0, cfg.vocab_size, n))) for n in lens]
    tables = [list(map(int, t)) for t in W.split_tables(rng, [-(-(n + 4) // 16) for n in lens], 64)]
    om = orc.Llama(cfg, w, num_blocks=64, block_size=16, max_len=256)
    gm = AbiModel(vo, cfg, w, max_tokens=256, max_seqs=4, num_blocks=64, block_size=16,
                  max_len=256)
    try:
        _say("abi-only cfg1: prefill")
        want_ids, want = om.prefill(sum(prompts, []), [(0, n, t) for n, t in zip(lens, tables)], 16)
        meta = vo.PrefillMeta.new([vo.PrefillSeq(0, n, t) for n, t in zip(lens, tables)], 16)
        ids, got = gm.forward(sum(prompts, []), meta, prefill=True)
        worst = _check_logits(ids, got, want_ids, want, "prefill")
        ctx = list(lens)
        for step in range(2):
            toks = [int(i) for i in want_ids]
            want_ids, want = om.decode(toks, [(c, t) for c, t in zip(ctx, tables)], 16)
            dmeta = vo.DecodeMeta.new([vo.DecodeSeq(c, t) for c, t in zip(ctx, tables)], 16)
            ids, got = gm.forward(toks, dmeta, prefill=False)
            worst = max(worst, _check_logits(ids, got, want_ids, want, f"decode {step}"))
            ctx = [c + 1 for c in ctx]
        # the arena's high-water mark is model::arena_elems' bound (arena.rs tests)
        assert gm.arena.high_water <= gm.ws.elems()
        _say(f"abi-only cfg1: worst err/tolerance {worst:.3f}; arena high water "
             f"{gm.arena.high_water} of {gm.ws.elems()} elements")
    finally:
        gm.close()


def test_abi_workspace_and_weight_errors(vo):
    """OutsideWorkspace for a region past the end (cpu/mod.rs:57-62), the
    weight's shape round trip (mod.rs:71-72), and bf16 upload rounding."""
    ws = vo.Workspace(1000)
    assert ws.elems() == 1000
    ws.ptr(vo.Region(990, 2, 5))
    with pytest.raises(vo.OutsideWorkspace):
        ws.ptr(vo.Region(991, 2, 5))
    with pytest.raises(vo.OutsideWorkspace):
        ws.read(vo.Region(0, 1001, 1))
    # 1 + 2^-8 is a tie (rounds to even: 1.0); 1 + 3 * 2^-9 rounds up.
    a = np.array([[1.0, 1.00390625, -2.5e-3, 1.005859375],
                  [3.0e38, np.inf, -0.0, np.nan]], np.float32)
    wt = vo.Weight(a)
    assert wt.shape() == (2, 4) and wt.dtype() == vo.VO_DTYPE_BF16
    both = vo.Weight.concat_rows([wt, wt])
    assert both.shape() == (4, 4)
    wf = vo.Weight(a, dtype=vo.VO_DTYPE_F32)
    assert wf.shape() == (2, 4)
    # Read the stacked bf16 weight back through embed (rows of a bf16 table,
    # widened exactly): it holds round-to-nearest-even of the f32 data.
    lib = vo.lib
    layout = vo.vo_kv_layout(1, 4, 16, 1, 8)
    pool, meta = vo._vp(), vo._vp()
    vo._check(lib.vo_kv_pool_create(ctypes.byref(layout), 0, ctypes.byref(pool)))
    vo._check(lib.vo_step_meta_create(pool, 4, 8, 16, 1, ctypes.byref(meta)))
    toks = vo._u32([0, 1, 2, 3])
    vo._check(lib.vo_step_meta_upload_tokens(meta, vo._p32(toks), 4, None))
    r = vo.Region(0, 4, 4)
    vo._check(lib.vo_embed(both.ptr, 4, 4, meta, 4, ws.ptr(r), None))
    got = ws.read(r)
    want = W.round_bf16(np.concatenate([a, a]))
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32))
    assert got[0, 1] == 1.0 and got[0, 3] == 1.0078125
    lib.vo_step_meta_destroy(meta)
    lib.vo_kv_pool_destroy(pool)
    for x in (wt, both, wf):
        x.close()
    ws.close()
