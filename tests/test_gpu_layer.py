"""GPU parity of the layer around attention and of the whole Llama forward,
through the C ABI, against the CPU oracle.

Ops (cpu/tests.rs:36-141 restated on the GPU, plus full-size shapes):
* embed, add, gather-by-last-rows and argmax: bit-exact (integer or exact
  float work);
* matmul with f32 output: max relative difference to a float64 product of the
  same bf16 inputs below 1e-5 (fp32 accumulation);
* outputs rounded to bf16 (rmsnorm, silu_mul, bf16 matmul): within one bf16
  ulp (2^-7 relative, bf16's largest relative spacing) of the oracle's f32
  result on the same inputs (a bf16 matmul output: two ulps of the float64
  product, one ulp for 99.9% of outputs -- see the test).

Model (BASELINE config 1 and the reference's own tiny test model): the GPU
model holds bf16 weights and bf16 activations around an f32 residual; the
oracle runs the same bf16-valued weights in f32.  Logits agree within the
tolerance written in each test; greedy ids agree wherever the oracle's top-1
/ top-2 gap exceeds the logit tolerance (the gap-aware comparison of the
reference's HF check, tests/hf_match.rs).
"""
import math

import numpy as np
import pytest

import oracle as orc
import workloads as W

pytestmark = pytest.mark.gpu

ULP = 2.0 ** -7  # largest relative spacing of bf16 (8 significand bits)


def _say(msg):
    print(f"[gpu-test] {msg}", flush=True)


def _dev(a, dtype):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0").to(dtype).contiguous()


def _np(t):
    return t.float().cpu().numpy()


def _within_ulp(got, want, what, ulps=1.0, atol=1e-6):
    """|got - want| within `ulps` bf16 ulps, an ulp measured at the larger
    magnitude (so a result that rounds up across a power of two counts as one
    ulp, not two)."""
    err = np.abs(got - want)
    lim = ulps * ULP * np.maximum(np.abs(want), np.abs(got)) + atol
    assert not np.isnan(got).any(), f"{what}: NaN"
    assert (err <= lim).all(), f"{what}: max err {err.max():.3e} ({(err > lim).sum()} over)"


@pytest.fixture(scope="module")
def M(vo):
    import importlib
    return importlib.import_module("vllm_oxide_amd.model")


# ---------------------------------------------------------------------------
# Ops
# ---------------------------------------------------------------------------
def test_matmul_reference_shape_generic_kernel(vo, gpu_backend):
    """cpu/tests.rs:36-59 shape: 21 inputs and 37 outputs are not whole
    16-byte rows, so the generic kernel runs; f32 out vs float64."""
    import torch
    _say("matmul 7x21x37 (generic)")
    x = W.round_bf16(orc.rand_vec(3, 7 * 21).reshape(7, 21))
    w = W.round_bf16(orc.rand_weight(4, (37, 21), 1.0))
    got = gpu_backend.matmul(_dev(x, torch.bfloat16), _dev(w, torch.bfloat16),
                             out_dtype=torch.float32)
    assert tuple(got.shape) == (7, 37)
    want = x.astype(np.float64) @ w.astype(np.float64).T
    assert orc.max_rel_diff(_np(got), want) < 1e-6


@pytest.mark.parametrize("rows,n,k", [(1, 4096, 4096), (3, 1024, 14336), (7, 6144, 4096),
                                      (16, 1024, 14336), (300, 1024, 14336), (1280, 512, 4096),
                                      (4, 1024, 256), (17, 512, 4096)])
def test_matmul_vs_float64(vo, gpu_backend, rows, n, k):
    """Up to 4 rows run on the weight-streaming kernel (K a multiple of
    2048), the rest on hipBLASLt."""
    import torch
    _say(f"matmul {rows}x{k} . {n}x{k}^T")
    rng = np.random.default_rng(rows + n + k)
    x = W.round_bf16(rng.standard_normal((rows, k), np.float32))
    w = W.round_bf16(rng.standard_normal((n, k), np.float32) * np.float32(0.02))
    xd, wd = _dev(x, torch.bfloat16), _dev(w, torch.bfloat16)
    want = x.astype(np.float64) @ w.astype(np.float64).T
    got32 = gpu_backend.matmul(xd, wd, out_dtype=torch.float32)
    assert orc.max_rel_diff(_np(got32), want) < 1e-5
    got16 = gpu_backend.matmul(xd, wd, out_dtype=torch.bfloat16)
    # bf16 output: the tuned algorithm may differ per output type, and a
    # split-K candidate rounds its partial sums, so the bar is two bf16 ulps
    # of the exact product everywhere and one ulp for 99.9% of the outputs.
    g16, w32 = _np(got16), want.astype(np.float32)
    _within_ulp(g16, w32, "bf16 out", ulps=2.0, atol=1e-6)
    one = np.abs(g16 - w32) <= ULP * np.maximum(np.abs(w32), np.abs(g16)) + 1e-6
    assert one.mean() >= 0.999, f"bf16 out: {1 - one.mean():.2e} of outputs beyond one ulp"
    # accumulate: out += x . w^T into an f32 residual (the model's add)
    base = rng.standard_normal((rows, n), np.float32)
    acc = _dev(base, torch.float32)
    gpu_backend.matmul(xd, wd, out=acc, accumulate=True)
    assert orc.max_rel_diff(_np(acc), base.astype(np.float64) + want) < 1e-5


def test_skinny_matmul_rows_independent_of_batch(vo, gpu_backend):
    """The weight-streaming kernel's output for a row does not depend on the
    other rows of the batch: each of 4 rows equals, bitwise, the same row
    computed alone (and the 3-row prefix equals the 4-row call's)."""
    import torch
    _say("skinny matmul batch independence")
    rng = np.random.default_rng(9)
    x = W.round_bf16(rng.standard_normal((4, 4096), np.float32))
    w = W.round_bf16(rng.standard_normal((6144, 4096), np.float32) * np.float32(0.02))
    xd, wd = _dev(x, torch.bfloat16), _dev(w, torch.bfloat16)
    full = _np(gpu_backend.matmul(xd, wd, out_dtype=torch.float32))
    for r in (0, 1, 3):
        one = _np(gpu_backend.matmul(xd[r:r + 1].contiguous(), wd, out_dtype=torch.float32))
        assert np.array_equal(one[0], full[r]), r
    part = _np(gpu_backend.matmul(xd[:3].contiguous(), wd, out_dtype=torch.float32))
    assert np.array_equal(part, full[:3])


def test_matmul_rejects_mismatched_shapes(vo, gpu_backend):
    """cpu/tests.rs:61-72: x [2, 8] against a weight [5, 9]."""
    import torch
    x = torch.zeros((2, 8), dtype=torch.bfloat16, device="cuda:0")
    w = torch.zeros((5, 9), dtype=torch.bfloat16, device="cuda:0")
    with pytest.raises(vo.ShapeError) as e:
        gpu_backend.matmul(x, w, out_dtype=torch.float32)
    assert e.value.op == "matmul"


@pytest.mark.parametrize("t,h", [(5, 19), (33, 4096), (7, 256), (3, 2056), (2, 8192), (2, 8200)])
def test_rmsnorm_matches_oracle(vo, gpu_backend, t, h):
    """cpu/tests.rs:74-96 shape first (the scalar path), then 16-byte rows:
    held in registers up to 8192 columns (2056: one live lane in the second
    pass of eight columns), read twice beyond (8200)."""
    import torch
    _say(f"rmsnorm {t}x{h}")
    x = orc.rand_vec(5, t * h).reshape(t, h) * np.float32(3.0)
    w = W.round_bf16(orc.rand_weight(6, (h,), 1.0))
    got = gpu_backend.rmsnorm(_dev(x, torch.float32), _dev(w, torch.bfloat16), 1e-5)
    _within_ulp(_np(got), orc.rmsnorm(x, w, 1e-5), "rmsnorm", ulps=1.0)
    with pytest.raises(vo.ShapeError):
        gpu_backend.rmsnorm(_dev(x, torch.float32), _dev(w[:-1], torch.bfloat16), 1e-5)


def test_rmsnorm_last_rows_is_gather_then_rmsnorm(vo, gpu_backend):
    """model.rs:334-343 for a prefill step (each sequence's last row) and a
    decode step (every row)."""
    import torch
    _say("rmsnorm over last rows")
    layout = vo.KvLayout(1, 64, 16, 2, 64)
    pool = gpu_backend.alloc_kv_pool(layout)
    seqs = [vo.PrefillSeq(0, 5, [1]), vo.PrefillSeq(3, 9, [2]), vo.PrefillSeq(0, 1, [3])]
    meta = vo.PrefillMeta.new(seqs, 16)
    h = 256
    x = orc.rand_vec(9, 15 * h).reshape(15, h)
    w = W.round_bf16(orc.rand_weight(10, (h,), 1.0))
    got = gpu_backend.rmsnorm_last_rows(_dev(x, torch.float32), _dev(w, torch.bfloat16), 1e-5,
                                        pool, meta)
    last = orc.gather_rows(x, [4, 13, 14])
    _within_ulp(_np(got), orc.rmsnorm(last, w, 1e-5), "last rows")
    dmeta = vo.DecodeMeta.new([vo.DecodeSeq(4, [1]), vo.DecodeSeq(7, [2])], 16)
    got = gpu_backend.rmsnorm_last_rows(_dev(x[:2], torch.float32), _dev(w, torch.bfloat16),
                                        1e-5, pool, dmeta)
    _within_ulp(_np(got), orc.rmsnorm(x[:2], w, 1e-5), "decode rows")


def test_silu_mul_add_gather_reference_and_fused_layout(vo, gpu_backend):
    """cpu/tests.rs:97-126, then a [64, 2 x 14336] gate|up projection output."""
    import torch
    _say("silu_mul / add")
    t, c = 3, 7
    g = W.round_bf16(orc.rand_vec(7, t * c).reshape(t, c))
    u = W.round_bf16(orc.rand_vec(8, t * c).reshape(t, c))
    gd, ud = _dev(g, torch.bfloat16), _dev(u, torch.bfloat16)
    got = gpu_backend.silu_mul(gd, ud)
    want = orc.silu_mul(g, u)
    _within_ulp(_np(got), want, "silu_mul 3x7")
    # add: f32 sum += bf16 x is exact f32 addition
    total = _dev(want, torch.float32)
    gpu_backend.add(total, ud)
    assert np.array_equal(_np(total), want + u)
    # in place on gate (the reference's form)
    gpu_backend.silu_mul(gd, ud, out=gd)
    _within_ulp(_np(gd), want, "silu_mul in place")
    F = 14336
    rng = np.random.default_rng(5)
    gu = W.round_bf16(rng.standard_normal((64, 2 * F), np.float32) * np.float32(4.0))
    gud = _dev(gu, torch.bfloat16)
    got = gpu_backend.silu_mul(gud[:, :F], gud[:, F:])
    _within_ulp(_np(got), orc.silu_mul(gu[:, :F], gu[:, F:]), "silu_mul fused layout")


def test_argmax_reference_cases_and_full_vocab(vo, gpu_backend):
    """cpu/tests.rs:128-141, then 258 rows x 128256 (cfg4's LM head) bit-exact."""
    import torch
    _say("argmax")
    x = np.array([1.0, 5.0, 5.0, -1.0, 0.0, 0.0, 0.0, 0.0, -3.0, -2.0, -2.0, -9.0],
                 np.float32).reshape(3, 4)
    assert list(gpu_backend.argmax(_dev(x, torch.float32))) == [1, 0, 1]
    with pytest.raises(vo.NaNError) as e:
        gpu_backend.argmax(_dev(np.array([[0.0, np.nan]], np.float32), torch.float32))
    assert e.value.op == "argmax" and e.value.message == "argmax: NaN in input"
    sp = np.array([[-np.inf, -np.inf, -np.inf], [-0.0, 0.0, -0.0], [np.inf, 1.0, np.inf]],
                  np.float32)
    assert list(gpu_backend.argmax(_dev(sp, torch.float32))) == [0, 0, 0]
    rng = np.random.default_rng(7)
    big = rng.standard_normal((258, 128256), np.float32)
    big[5, 77] = big[5, 100000] = 10.0  # a tie: the first index wins
    assert np.array_equal(gpu_backend.argmax(_dev(big, torch.float32)), orc.argmax(big))
    b16 = W.round_bf16(big[:16, :1001])
    assert np.array_equal(gpu_backend.argmax(_dev(b16, torch.bfloat16)), orc.argmax(b16))


def test_embed_exact_and_vocab_check(vo, gpu_backend):
    import torch
    _say("embed")
    layout = vo.KvLayout(1, 8, 16, 1, 64)
    pool = gpu_backend.alloc_kv_pool(layout)
    m = gpu_backend.step_meta(pool, "embed-test")
    table = W.round_bf16(np.random.default_rng(3).standard_normal((1024, 256), np.float32))
    td = _dev(table, torch.bfloat16)
    toks = [5, 1023, 0, 5, 17]
    got = gpu_backend.embed(td, toks, m)
    assert np.array_equal(_np(got), orc.embed(table, toks))
    with pytest.raises(vo.ShapeError) as e:
        gpu_backend.embed(td, [3, 1024], m)
    assert e.value.message == "embed: token 1024 >= vocab 1024"


# ---------------------------------------------------------------------------
# The whole forward
# ---------------------------------------------------------------------------
def _gpu_model(vo, M, backend, cfg, weights, num_blocks, block_size, max_tokens=512, max_seqs=8,
               max_len=256):
    mc = M.ModelConfig(cfg.hidden_size, cfg.intermediate_size, cfg.num_hidden_layers,
                       cfg.num_attention_heads, cfg.num_key_value_heads, cfg.vocab_size,
                       cfg.max_position_embeddings, cfg.rms_norm_eps, cfg.rope_theta,
                       dict(cfg.rope_scaling))
    ec = M.EngineConfig(max_batch_tokens=max_tokens, max_seqs=max_seqs, max_model_len=max_len,
                        block_size=block_size, num_blocks=num_blocks)
    model = M.Llama(backend, mc, ec, weights)
    return model, model.alloc_kv_pool()


def test_tiny_reference_model_prefill_then_decode(vo, M, gpu_backend):
    """model.rs:447-495 on the GPU with the reference's tiny model (head_dim
    8, block size 4: the unfused RoPE/write path and the generic attention
    kernel): full prefill vs prefill + 5 decode steps, and both against the
    oracle on the same bf16 weights."""
    cfg = W.tiny_config()
    w = W.bf16_weights(orc.random_weights(cfg, 7))
    n, k = 13, 5
    p = W.ref_prompt(n, 3)
    table = [6, 1, 9, 3]
    _say("tiny model: full prefill")
    m1, kv1 = _gpu_model(vo, M, gpu_backend, cfg, w, 32, 4, max_len=128)
    full = m1.prefill(kv1, p, vo.PrefillMeta.new([vo.PrefillSeq(0, n, table)], 4), True)
    _say("tiny model: prefill + decode")
    m2, kv2 = _gpu_model(vo, M, gpu_backend, cfg, w, 32, 4, max_len=128)
    out = m2.prefill(kv2, p[:n - k], vo.PrefillMeta.new([vo.PrefillSeq(0, n - k, table)], 4), True)
    for pos in range(n - k, n):
        out = m2.decode(kv2, p[pos:pos + 1], vo.DecodeMeta.new([vo.DecodeSeq(pos, table)], 4), True)
    om = orc.Llama(cfg, w, num_blocks=32, block_size=4, max_len=128)
    want_ids, want_logits = om.prefill(p, [(0, n, table)], 4)
    d_steps = orc.max_rel_diff(out.logits, full.logits)
    d_oracle = orc.max_rel_diff(full.logits, want_logits)
    _say(f"tiny model: rel diff decode-vs-prefill {d_steps:.2e}, gpu-vs-oracle {d_oracle:.2e}")
    assert out.tokens == full.tokens == list(want_ids)
    assert d_steps < 2e-2 and d_oracle < 2e-2


def test_tiny_reference_model_batched_prefill(vo, M, gpu_backend):
    """model.rs:541-583: two sequences prefilled together vs each alone.  The
    reference's bar is bitwise; here the attention kernels are row-invariant
    but hipBLASLt picks its algorithm per batch size, so the bar is the
    tolerance, and the ids must agree."""
    cfg = W.tiny_config()
    w = W.bf16_weights(orc.random_weights(cfg, 7))
    pa, pb = W.ref_prompt(7, 1), W.ref_prompt(10, 2)
    ta, tb = [3, 5], [0, 8, 1]

    def alone(p, t):
        m, kv = _gpu_model(vo, M, gpu_backend, cfg, w, 32, 4, max_len=128)
        return m.prefill(kv, p, vo.PrefillMeta.new([vo.PrefillSeq(0, len(p), t)], 4), True)

    a, b = alone(pa, ta), alone(pb, tb)
    m, kv = _gpu_model(vo, M, gpu_backend, cfg, w, 32, 4, max_len=128)
    both = m.prefill(kv, pa + pb, vo.PrefillMeta.new(
        [vo.PrefillSeq(0, 7, ta), vo.PrefillSeq(0, 10, tb)], 4), True)
    assert both.tokens == [a.tokens[0], b.tokens[0]]
    da = orc.max_rel_diff(both.logits[0], a.logits[0])
    db = orc.max_rel_diff(both.logits[1], b.logits[0])
    _say(f"tiny batched prefill: rel diff {da:.2e} {db:.2e} "
         f"(bitwise: {np.array_equal(both.logits[0], a.logits[0])})")
    assert da < 1e-2 and db < 1e-2


def _cfg1_setup(seed=1):
    cfg = W.cfg1_config()
    w = W.bf16_weights(W.normal_weights(cfg, 100 + seed))
    rng = np.random.default_rng(seed)
    lens = [17, 33, 64, 100]
    prompts = [list(map(int, rng.integers(0, cfg.vocab_size, n))) for n in lens]
    steps = 32
    need = [-(-(n + steps) // 16) for n in lens]
    tables = [list(map(int, t)) for t in W.split_tables(rng, need, 64)]
    return cfg, w, prompts, tables, steps


# Logit tolerance of config 1 (bf16 weights and activations against the f32
# oracle on the same weights): |gpu - oracle| <= LOGIT_ATOL + LOGIT_RTOL * |oracle|.
LOGIT_ATOL, LOGIT_RTOL = 1e-2, 2e-2


def test_cfg1_teacher_forced_logits_and_gap_aware_ids(vo, M, gpu_backend):
    """4 sequences (prompts 17/33/64/100), one batched
    prefill, then 32 greedy decode steps, block size 16 over 64 blocks.  The
    oracle generates; the GPU model is fed the oracle's tokens (teacher
    forcing) so both caches hold the same sequence, and every step's logits
    are compared.  Where the oracle's top-1 / top-2 gap is above twice the
    tolerance the GPU's greedy id must be the oracle's."""
    cfg, w, prompts, tables, steps = _cfg1_setup()
    om = orc.Llama(cfg, w, num_blocks=64, block_size=16, max_len=256)
    gm, kv = _gpu_model(vo, M, gpu_backend, cfg, w, 64, 16)
    lens = [len(p) for p in prompts]
    ids, want = om.prefill(sum(prompts, []), [(0, n, t) for n, t in zip(lens, tables)], 16)
    _say("cfg1: prefill")
    got = gm.prefill(kv, sum(prompts, []), vo.PrefillMeta.new(
        [vo.PrefillSeq(0, n, t) for n, t in zip(lens, tables)], 16), True)
    worst, checked, gapped = 0.0, 0, 0
    ctx = list(lens)
    for step in range(steps + 1):
        err = np.abs(got.logits - want)
        worst = max(worst, float((err / (LOGIT_ATOL + LOGIT_RTOL * np.abs(want))).max()))
        assert (err <= LOGIT_ATOL + LOGIT_RTOL * np.abs(want)).all(), (
            f"step {step}: max logit err {err.max():.3e}")
        top2 = np.sort(want, axis=1)[:, -2:]
        gap = top2[:, 1] - top2[:, 0]
        for s in range(4):
            if gap[s] > 2 * (LOGIT_ATOL + LOGIT_RTOL * abs(top2[s, 1])):
                assert got.tokens[s] == ids[s], f"step {step} seq {s}: id differs at gap {gap[s]:.3e}"
                checked += 1
            else:
                gapped += 1
        if step == steps:
            break
        toks = [int(i) for i in ids]
        ids, want = om.decode(toks, [(c, t) for c, t in zip(ctx, tables)], 16)
        got = gm.decode(kv, toks, vo.DecodeMeta.new(
            [vo.DecodeSeq(c, t) for c, t in zip(ctx, tables)], 16), True)
        ctx = [c + 1 for c in ctx]
    _say(f"cfg1: worst err/tolerance {worst:.3f}; ids checked {checked}, near-ties {gapped}")


def test_cfg1_free_running_greedy_matches_until_a_near_tie(vo, M, gpu_backend):
    """The GPU model generates on its own; per sequence, the generated ids
    equal the oracle's up to the first difference, and that first difference
    (if any) is at a step where the oracle's top-1 / top-2 gap is within the
    logit tolerance (hf_match.rs's gap-aware report)."""
    cfg, w, prompts, tables, steps = _cfg1_setup(seed=2)
    lens = [len(p) for p in prompts]

    def run_oracle():
        om = orc.Llama(cfg, w, num_blocks=64, block_size=16, max_len=256)
        ids, lg = om.prefill(sum(prompts, []), [(0, n, t) for n, t in zip(lens, tables)], 16)
        out, logits, ctx = [list(map(int, ids))], [lg], list(lens)
        for _ in range(steps):
            ids, lg = om.decode(out[-1], [(c, t) for c, t in zip(ctx, tables)], 16)
            out.append(list(map(int, ids)))
            logits.append(lg)
            ctx = [c + 1 for c in ctx]
        return np.array(out), logits

    want, want_logits = run_oracle()
    gm, kv = _gpu_model(vo, M, gpu_backend, cfg, w, 64, 16)
    _say("cfg1 free-running")
    o = gm.prefill(kv, sum(prompts, []), vo.PrefillMeta.new(
        [vo.PrefillSeq(0, n, t) for n, t in zip(lens, tables)], 16))
    got, ctx = [o.tokens], list(lens)
    for _ in range(steps):
        o = gm.decode(kv, got[-1], vo.DecodeMeta.new(
            [vo.DecodeSeq(c, t) for c, t in zip(ctx, tables)], 16))
        got.append(o.tokens)
        ctx = [c + 1 for c in ctx]
    got = np.array(got)
    for s in range(4):
        diff = np.nonzero(got[:, s] != want[:, s])[0]
        if len(diff) == 0:
            _say(f"seq {s}: all {steps + 1} ids equal")
            continue
        i = int(diff[0])
        row = want_logits[i][s]
        top2 = np.sort(row)[-2:]
        gap = float(top2[1] - top2[0])
        _say(f"seq {s}: first difference at id {i}, oracle gap {gap:.3e}")
        assert gap <= 2 * (LOGIT_ATOL + LOGIT_RTOL * abs(top2[1])), (
            f"seq {s} diverges at id {i} where the oracle's gap is {gap:.3e}")


# Config 1 as BASELINE states it: the oracle runs the f32 N(0, 0.02) weights,
# the GPU holds them rounded to bf16.  On the CPU, the oracle on bf16-rounded
# weights differs from the oracle on the f32 ones by at most 0.0065 in the
# logits over prefill + 32 steps (0.55 of LOGIT_ATOL + LOGIT_RTOL * |x|, seeds
# 1 and 2), and the GPU's bf16 activations add at most 0.55 of it against
# the oracle on bf16 weights; the sum stays within twice that tolerance.
F32W_ATOL, F32W_RTOL = 2 * LOGIT_ATOL, 2 * LOGIT_RTOL


def test_cfg1_f32_weights_logits_and_gap_aware_greedy(vo, M, gpu_backend):
    """BASELINE config 1 with its f32 weights on the oracle side.  Teacher
    forced: every step's logits within F32W_ATOL + F32W_RTOL * |oracle| and the
    ids equal wherever the oracle's top-1 / top-2 gap exceeds twice that.
    Free running (hf_match.rs:139-155): per sequence the first id that differs,
    if any, sits where the oracle's gap is within the tolerance."""
    cfg = W.cfg1_config()
    w32 = W.normal_weights(cfg, 101)
    rng = np.random.default_rng(1)
    lens = [17, 33, 64, 100]
    prompts = [list(map(int, rng.integers(0, cfg.vocab_size, n))) for n in lens]
    steps = 32
    tables = [list(map(int, t)) for t in
              W.split_tables(rng, [-(-(n + steps) // 16) for n in lens], 64)]
    seqs0 = [(0, n, t) for n, t in zip(lens, tables)]
    om = orc.Llama(cfg, w32, num_blocks=64, block_size=16, max_len=256)
    ids, want = om.prefill(sum(prompts, []), seqs0, 16)
    want_ids, want_logits = [list(map(int, ids))], [want]
    ctx = list(lens)
    for _ in range(steps):
        ids, lg = om.decode(want_ids[-1], [(c, t) for c, t in zip(ctx, tables)], 16)
        want_ids.append(list(map(int, ids)))
        want_logits.append(lg)
        ctx = [c + 1 for c in ctx]
    want_ids = np.array(want_ids)

    def tol(x):
        return F32W_ATOL + F32W_RTOL * np.abs(x)

    _say("cfg1 f32 weights: teacher forced")
    gm, kv = _gpu_model(vo, M, gpu_backend, cfg, w32, 64, 16)  # rounds to bf16 on upload
    got = gm.prefill(kv, sum(prompts, []), vo.PrefillMeta.new(
        [vo.PrefillSeq(*s) for s in seqs0], 16), True)
    worst_abs, worst_rel, checked, near = 0.0, 0.0, 0, 0
    ctx = list(lens)
    for step in range(steps + 1):
        want = want_logits[step]
        err = np.abs(got.logits - want)
        worst_abs = max(worst_abs, float(err.max()))
        worst_rel = max(worst_rel, float((err / tol(want)).max()))
        assert (err <= tol(want)).all(), f"step {step}: max logit err {err.max():.3e}"
        top2 = np.sort(want, axis=1)[:, -2:]
        for s in range(4):
            if top2[s, 1] - top2[s, 0] > 2 * tol(top2[s, 1]):
                assert got.tokens[s] == want_ids[step][s], f"step {step} seq {s}"
                checked += 1
            else:
                near += 1
        if step == steps:
            break
        got = gm.decode(kv, list(want_ids[step]), vo.DecodeMeta.new(
            [vo.DecodeSeq(c, t) for c, t in zip(ctx, tables)], 16), True)
        ctx = [c + 1 for c in ctx]
    _say(f"cfg1 f32 weights: worst |dlogit| {worst_abs:.3e} ({worst_rel:.3f} of the tolerance); "
         f"ids checked {checked}, near-ties {near}")

    _say("cfg1 f32 weights: free running")
    gm, kv = _gpu_model(vo, M, gpu_backend, cfg, w32, 64, 16)
    o = gm.prefill(kv, sum(prompts, []), vo.PrefillMeta.new([vo.PrefillSeq(*s) for s in seqs0], 16))
    gen, ctx = [o.tokens], list(lens)
    for _ in range(steps):
        o = gm.decode(kv, gen[-1], vo.DecodeMeta.new(
            [vo.DecodeSeq(c, t) for c, t in zip(ctx, tables)], 16))
        gen.append(o.tokens)
        ctx = [c + 1 for c in ctx]
    gen = np.array(gen)
    for s in range(4):
        diff = np.nonzero(gen[:, s] != want_ids[:, s])[0]
        if len(diff) == 0:
            _say(f"cfg1 f32 weights seq {s}: all {steps + 1} ids equal")
            continue
        i = int(diff[0])
        top2 = np.sort(want_logits[i][s])[-2:]
        gap = float(top2[1] - top2[0])
        _say(f"cfg1 f32 weights seq {s}: first difference at id {i}, oracle gap {gap:.3e}")
        assert gap <= 2 * tol(top2[1]), f"seq {s} diverges at id {i} where the gap is {gap:.3e}"


def test_cfg1_mixed_step_matches_oracle(vo, M, gpu_backend):
    """A continuous-batching step: two sequences decode one token while a
    third prefills a 40-token chunk onto 24 cached tokens, one prefill call
    (the decode rows take the split-K decode kernel)."""
    cfg, w, prompts, tables, _ = _cfg1_setup(seed=3)
    om = orc.Llama(cfg, w, num_blocks=64, block_size=16, max_len=256)
    gm, kv = _gpu_model(vo, M, gpu_backend, cfg, w, 64, 16)
    p = [prompts[0][:17], prompts[1][:30], prompts[3][:64]]
    t = [tables[0], tables[1], tables[3]]
    first = [(0, 17, t[0]), (0, 30, t[1]), (0, 24, t[2])]
    om.prefill(p[0] + p[1] + p[2][:24], first, 16)
    gm.prefill(kv, p[0] + p[1] + p[2][:24], vo.PrefillMeta.new(
        [vo.PrefillSeq(*f) for f in first], 16))
    step = [(17, 1, t[0]), (30, 1, t[1]), (24, 40, t[2])]
    toks = [3, 900] + p[2][24:64]
    ids, want = om.prefill(toks, step, 16)
    _say("cfg1 mixed step")
    got = gm.prefill(kv, toks, vo.PrefillMeta.new([vo.PrefillSeq(*s) for s in step], 16), True)
    err = np.abs(got.logits - want)
    assert (err <= LOGIT_ATOL + LOGIT_RTOL * np.abs(want)).all(), f"max err {err.max():.3e}"


def test_batch_checks(vo, M, gpu_backend):
    """model.rs:245-267 and :422-444: token count vs metadata, and capacity."""
    cfg = W.tiny_config()
    w = W.bf16_weights(orc.random_weights(cfg, 7))
    m, kv = _gpu_model(vo, M, gpu_backend, cfg, w, 32, 4, max_tokens=64, max_seqs=4, max_len=128)
    table = list(range(17))
    with pytest.raises(vo.CapacityError) as e:
        m.prefill(kv, W.ref_prompt(65, 0), vo.PrefillMeta.new([vo.PrefillSeq(0, 65, table)], 4))
    assert (e.value.value, e.value.limit) == (65, 64)
    with pytest.raises(vo.ShapeError):
        m.prefill(kv, W.ref_prompt(5, 0), vo.PrefillMeta.new([vo.PrefillSeq(0, 6, table)], 4))


def test_decode_graph_replays_equal_eager_steps(vo, M, gpu_backend):
    """A decode step recorded as a HIP graph (fixed launch shapes) and
    replayed for 16 later steps gives bitwise the eager step's logits and ids;
    eager work and syncs run between the replays.  Block tables grow as the
    engine's do (each step passes the blocks its keys need); a step whose
    table outgrows the fixed capacity is refused (CapacityError) and runs
    after recording again."""
    cfg, w, prompts, tables, _ = _cfg1_setup(seed=4)
    lens = [len(p) for p in prompts]
    ga, kva = _gpu_model(vo, M, gpu_backend, cfg, w, 64, 16)
    gb, kvb = _gpu_model(vo, M, gpu_backend, cfg, w, 64, 16)
    pm = vo.PrefillMeta.new([vo.PrefillSeq(0, n, t) for n, t in zip(lens, tables)], 16)
    a = ga.prefill(kva, sum(prompts, []), pm)
    b = gb.prefill(kvb, sum(prompts, []), pm)
    assert a.tokens == b.tokens
    toks, ctx = a.tokens, list(lens)
    graph = None
    refits = 0
    for step in range(16):
        meta = vo.DecodeMeta.new([vo.DecodeSeq(c, t[:(c + 16) // 16]) for c, t in zip(ctx, tables)],
                                 16)
        _say(f"graph decode step {step}")
        want = ga.decode(kva, toks, meta, want_logits=True)
        if graph is None:
            # no table headroom: the first block boundary forces a new recording
            graph = gb.capture_decode(kvb, toks, meta, entry_headroom=0)
        try:
            got = graph.run(toks, meta, want_logits=True)
        except vo.CapacityError:
            refits += 1
            graph = gb.capture_decode(kvb, toks, meta, entry_headroom=0)
            got = graph.run(toks, meta, want_logits=True)
        assert got.tokens == want.tokens, f"step {step}"
        assert np.array_equal(got.logits, want.logits), f"step {step}"
        toks, ctx = want.tokens, [c + 1 for c in ctx]
    _say(f"graph decode: 16 steps bitwise equal, {refits} re-recordings")
    assert refits >= 1
