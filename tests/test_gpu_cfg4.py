"""BASELINE config 4 on the GPU: one full mixed continuous-batching step of the
random-init Llama-3-8B-shaped model (32 layers, hidden 4096, 32 q / 8 kv
heads, head_dim 128, FFN 14336, vocab 128256, theta 500000, bf16 weights
~ N(0, 0.02)): 256 decode sequences (context lognormal, median 1024, sigma 1,
clipped to [128, 8192]) plus two 512-token prefill chunks, block size 16.

Llama::forward (crates/engine/src/model.rs:269-356) is checked three ways:
* the mixed step's logits are finite; its decode rows' logits are within
  SAME_GPU_ATOL of a decode-only step of the same rows, and their greedy ids
  equal wherever the top-1 / top-2 gap exceeds twice that (hipBLASLt may pick
  another algorithm for another row count, so the bar is the gap-aware one of
  hf_match.rs:139-155, not bitwise);
* the decode-only step replayed from a HIP graph equals the eager step bitwise;
* one decoder layer at this exact shape (plus the final norm and the LM head)
  against the oracle's Llama on a sample of the step's rows: 8 decode rows with
  their cached contexts and 24 rows of a chunk continuing a 2024-token context
  (the sample bench.py's CPU baseline times), logits within the bf16
  activation-rounding error measured for this shape (CFG4_LAYER_*).
"""
import importlib

import numpy as np
import pytest

import oracle as orc
import workloads as W

pytestmark = pytest.mark.gpu

LOGIT_ATOL, LOGIT_RTOL = 1e-2, 2e-2
# Mixed step vs decode-only step of the same rows, both on the GPU with the
# same bf16 weights: only hipBLASLt's algorithm choice for the row count
# differs (measured: at most 8.1e-6 in the logits).
SAME_GPU_ATOL = 1e-4
# One cfg4-shaped layer against the f32 oracle on the same bf16 weights.  The
# GPU rounds activations to bf16 where the oracle keeps f32 (normed rows, q/k/v,
# the attention output, gate/up and their product).  At hidden 4096 and vocab
# 128256 the logit error is that rounding: repeating the oracle's step with
# bf16 rounding at exactly those points gives max |dlogit| 0.053 and RMS
# 0.0091 on these inputs (logit std 1.28), the GPU max 0.047.  The bar is
# about twice both.
CFG4_LAYER_ATOL, CFG4_LAYER_RMS = 0.1, 0.02


def _say(msg):
    print(f"[gpu-test] {msg}", flush=True)


@pytest.fixture(scope="module")
def M(vo):
    return importlib.import_module("vllm_oxide_amd.model")


def _model_config(M, cfg):
    return M.ModelConfig(cfg.hidden_size, cfg.intermediate_size, cfg.num_hidden_layers,
                         cfg.num_attention_heads, cfg.num_key_value_heads, cfg.vocab_size,
                         cfg.max_position_embeddings, cfg.rms_norm_eps, cfg.rope_theta,
                         dict(cfg.rope_scaling))


def test_cfg4_full_mixed_step(vo, M):
    import torch
    cfg = W.llama3_8b_config(32)
    hd, H, F, V = cfg.head_dim, cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size
    qd, kvd = cfg.num_attention_heads * hd, cfg.num_key_value_heads * hd
    ctx, new = W.cfg4_attention_lens()
    S, T = len(ctx), int(np.sum(new))
    num_blocks = 30000
    backend = vo.HipBackend(device=0, max_seqs=S, max_rows=W.FILL_ROWS,
                            max_table_entries=num_blocks, max_query_heads=cfg.num_attention_heads)
    _say("cfg4: cached context of 32 layers")
    wl = W.build(vo, backend, kind="prefill", heads=cfg.num_attention_heads,
                 kv_heads=cfg.num_key_value_heads, head_dim=hd, block_size=16,
                 num_blocks=num_blocks, context_lens=ctx, num_new=new, seed=4,
                 num_layers=cfg.num_hidden_layers, fill_layers=range(cfg.num_hidden_layers),
                 keep_host=False)
    del wl.ctx_kv[:]
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(44)

    def nrm(o, i):
        return (torch.randn((o, i), generator=gen, device="cuda:0", dtype=torch.float32)
                * 0.02).to(torch.bfloat16)

    ones = torch.ones(H, dtype=torch.bfloat16, device="cuda:0")
    weights = dict(embed=nrm(V, H), final_norm=ones, layers=[
        dict(attn_norm=ones, wq=nrm(qd, H), wk=nrm(kvd, H), wv=nrm(kvd, H), wo=nrm(H, qd),
             mlp_norm=ones, w_gate=nrm(F, H), w_up=nrm(F, H), w_down=nrm(H, F))
        for _ in range(cfg.num_hidden_layers)])
    ec = M.EngineConfig(max_batch_tokens=T, max_seqs=S, max_model_len=8192 + 1024,
                        block_size=16, num_blocks=num_blocks)
    model = M.Llama(backend, _model_config(M, cfg), ec, weights)
    del weights
    torch.cuda.empty_cache()
    tokens = [int(t) for t in np.random.default_rng(4).integers(0, V, T)]

    _say("cfg4: mixed step (256 decode rows + 2 x 512-row chunks)")
    mixed = model.prefill(wl.pool, tokens, wl.meta, want_logits=True)
    assert mixed.logits.shape == (S, V)
    assert np.isfinite(mixed.logits).all()
    dec = np.nonzero(np.asarray(new) == 1)[0]
    assert len(dec) == 256
    starts = np.asarray(wl.meta.seq_row_starts)
    dec_tokens = [tokens[int(starts[s])] for s in dec]
    dmeta = vo.DecodeMeta.new([vo.DecodeSeq(int(ctx[s]), wl.tables[s]) for s in dec], 16)

    _say("cfg4: decode-only step of the same 256 rows")
    alone = model.decode(wl.pool, dec_tokens, dmeta, want_logits=True)
    a = mixed.logits[dec]
    b = alone.logits
    err = np.abs(a - b)
    assert (err <= SAME_GPU_ATOL).all(), (
        f"decode rows: mixed vs decode-only max |dlogit| {err.max():.3e}")
    top2 = np.sort(b, axis=1)[:, -2:]
    checked = 0
    for i in range(len(dec)):
        if top2[i, 1] - top2[i, 0] > 2 * SAME_GPU_ATOL:
            assert mixed.tokens[dec[i]] == alone.tokens[i], f"decode row {i}: id differs"
            checked += 1
    _say(f"cfg4: mixed vs decode-only max |dlogit| {err.max():.3e}; {checked} of 256 ids "
         f"compared (gap above tolerance), bitwise equal rows "
         f"{int(np.all(a == b, axis=1).sum())}")
    assert checked >= 200

    _say("cfg4: decode step as a HIP graph")
    graph = model.capture_decode(wl.pool, dec_tokens, dmeta)
    replay = graph.run(dec_tokens, dmeta, want_logits=True)
    assert replay.tokens == alone.tokens
    assert np.array_equal(replay.logits, alone.logits)
    replay2 = graph.run(dec_tokens, dmeta, want_logits=True)
    assert np.array_equal(replay2.logits, alone.logits)
    model.close()


def test_cfg4_one_layer_vs_oracle_on_sampled_rows(vo, M):
    """One decoder layer of the cfg4 model shape, the final norm and the tied LM
    head on 32 rows: the first 8 decode sequences of cfg4 (their lognormal
    contexts) and 24 chunk rows continuing a 2024-token context.  Weights
    ~ N(0, 0.02) drawn in f32 and rounded to bf16 for both sides; cached K/V
    ~ N(0, 1) written identically into both pools."""
    import torch
    cfg = W.llama3_8b_config(1)
    hd, H, F, V = cfg.head_dim, cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size
    qd, kvd = cfg.num_attention_heads * hd, cfg.num_key_value_heads * hd
    rng = np.random.default_rng(14)

    def nrm(o, i):
        return W.round_bf16((rng.standard_normal((o, i), np.float32) * np.float32(0.02)))

    w = dict(embed=nrm(V, H), final_norm=np.ones(H, np.float32), layers=[dict(
        attn_norm=np.ones(H, np.float32), wq=nrm(qd, H), wk=nrm(kvd, H), wv=nrm(kvd, H),
        wo=nrm(H, qd), mlp_norm=np.ones(H, np.float32), w_gate=nrm(F, H), w_up=nrm(F, H),
        w_down=nrm(H, F))])
    dctx, _ = W.cfg4_attention_lens()
    seqs = [(int(c), 1) for c in dctx[:8]] + [(2024, 24)]
    bs = 16
    nblk = [-(-(c + n) // bs) for c, n in seqs]
    num_blocks = sum(nblk) + 8
    perm = rng.permutation(num_blocks).astype(np.uint32)
    tables, at = [], 0
    for b in nblk:
        tables.append(perm[at:at + b])
        at += b
    backend = vo.HipBackend(device=0, max_seqs=16, max_rows=W.FILL_ROWS,
                            max_table_entries=num_blocks, max_query_heads=cfg.num_attention_heads)
    ec = M.EngineConfig(max_batch_tokens=64, max_seqs=16, max_model_len=8192 + 1024,
                        block_size=bs, num_blocks=num_blocks)
    model = M.Llama(backend, _model_config(M, cfg), ec, w)
    pool = model.alloc_kv_pool()
    om = orc.Llama(cfg, w, num_blocks=num_blocks, block_size=bs, max_len=8192 + 1024)
    _say("cfg4 layer: cached contexts")
    for (c, _), t in zip(seqs, tables):
        k = rng.standard_normal((c, kvd), np.float32)
        v = rng.standard_normal((c, kvd), np.float32)
        kb, vb = W.round_bf16(k), W.round_bf16(v)
        slots = np.array([int(t[p // bs]) * bs + p % bs for p in range(c)], np.uint32)
        om.pool.write_kv(0, kb, vb, slots)
        kt = torch.from_numpy(kb).to("cuda:0", torch.bfloat16)
        vt = torch.from_numpy(vb).to("cuda:0", torch.bfloat16)
        backend.write_kv(pool, 0, kt.contiguous(), vt.contiguous(), slots)
    rows = sum(n for _, n in seqs)
    tokens = [int(x) for x in rng.integers(0, V, rows)]
    _say("cfg4 layer: oracle step")
    want_ids, want = om.prefill(tokens, [(c, n, t) for (c, n), t in zip(seqs, tables)], bs)
    _say("cfg4 layer: GPU step")
    meta = vo.PrefillMeta.new([vo.PrefillSeq(c, n, t) for (c, n), t in zip(seqs, tables)], bs)
    got = model.prefill(pool, tokens, meta, want_logits=True)
    err = np.abs(got.logits - want)
    rms = float(np.sqrt(np.mean(err.astype(np.float64) ** 2)))
    _say(f"cfg4 layer: max |dlogit| {err.max():.3e}, RMS {rms:.3e} (logit std "
         f"{want.std():.3f}, max |logit| {np.abs(want).max():.3f})")
    assert err.max() <= CFG4_LAYER_ATOL and rms <= CFG4_LAYER_RMS
    top2 = np.sort(want, axis=1)[:, -2:]
    checked = 0
    for s in range(len(seqs)):
        if top2[s, 1] - top2[s, 0] > 2 * CFG4_LAYER_ATOL:
            assert got.tokens[s] == int(want_ids[s]), f"seq {s}"
            checked += 1
    _say(f"cfg4 layer: ids compared {checked} of {len(seqs)}")
    model.close()
