"""Pins the oracle's restatement of the layer around attention
(crates/engine/src/backend/cpu/mod.rs: embed, rmsnorm, matmul, silu_mul,
add, gather_rows, argmax) and of Llama::forward (model.rs:269-356).

The reference's own op tests (cpu/tests.rs:37-141) and model tests
(model.rs:450-583) are restated on the reference's inputs (its LCG,
tiny_config, random_weights(seed 7), its prompts and block tables).  The
model is further checked against an independent float64 dense Llama written
here from the architecture (full causal attention over contiguous K/V, no
paging, no 16-lane dot), so that a dropped residual, a wrong GQA head
mapping or a rotation of the wrong half fails.
"""
import math

import numpy as np
import pytest

import oracle as orc
import workloads as W


def _f64_naive_matmul(x, w):
    return (x.astype(np.float64) @ w.astype(np.float64).T).astype(np.float32)


def test_reference_matmul_matches_naive():
    """cpu/tests.rs:36-59: 37 outputs (two 16-row tasks + a partial), 21 inputs
    (one 16-lane chunk + remainder)."""
    t, n_in, n_out = 7, 21, 37
    x = orc.rand_vec(3, t * n_in).reshape(t, n_in)
    w = orc.rand_weight(4, (n_out, n_in), 1.0)
    got = orc.matmul(x, w)
    assert got.shape == (t, n_out)
    assert orc.max_rel_diff(got, _f64_naive_matmul(x, w)) < 1e-6


def test_matmul_is_each_element_one_dot_for_any_thread_count():
    x = orc.rand_vec(11, 5 * 40).reshape(5, 40)
    w = orc.rand_weight(12, (67, 40), 0.5)
    one = orc.matmul(x, w, threads=1)
    for th in (2, 3, 8, 67):
        assert np.array_equal(orc.matmul(x, w, threads=th), one)
    for r in range(5):
        for o in (0, 16, 66):
            assert one[r, o] == np.float32(orc.dot(x[r], w[o]))


def test_reference_rmsnorm_matches_naive():
    """cpu/tests.rs:74-96."""
    t, h, eps = 5, 19, 1e-5
    x = orc.rand_vec(5, t * h).reshape(t, h)
    w = orc.rand_weight(6, (h,), 1.0)
    want = np.zeros((t, h), np.float32)
    for i in range(t):
        r = x[i].astype(np.float64)
        ms = (r * r).sum() / h
        want[i] = (w.astype(np.float64) * r / math.sqrt(ms + eps)).astype(np.float32)
    got = orc.rmsnorm(x, w, eps)
    assert orc.max_rel_diff(got, want) < 1e-6


def test_rmsnorm_is_scale_invariant_and_weighted():
    """rmsnorm(c x) = rmsnorm(x) for c > 0 up to eps; the weight scales columns."""
    x = orc.rand_vec(21, 3 * 64).reshape(3, 64)
    ones = np.ones(64, np.float32)
    a = orc.rmsnorm(x, ones, 0.0)
    b = orc.rmsnorm(x * np.float32(8.0), ones, 0.0)
    assert np.allclose(a, b, rtol=1e-6, atol=1e-7)
    assert np.allclose((a.astype(np.float64) ** 2).mean(axis=1), 1.0, rtol=1e-5)
    w = np.arange(64, dtype=np.float32) / 8
    assert np.allclose(orc.rmsnorm(x, w, 0.0), a * w, rtol=1e-6, atol=1e-7)


def test_reference_silu_mul_add_gather():
    """cpu/tests.rs:97-126."""
    t, c = 3, 7
    g = orc.rand_vec(7, t * c).reshape(t, c)
    u = orc.rand_vec(8, t * c).reshape(t, c)
    got = orc.silu_mul(g, u)
    x = g.astype(np.float64)
    want = x / (1.0 + np.exp(-x)) * u.astype(np.float64)
    assert np.abs(got - want).max() < 1e-6
    got2 = orc.add(got, u)
    assert np.array_equal(got2, got + u)
    p = orc.gather_rows(u, [2, 0])
    assert np.array_equal(p[0], u[2]) and np.array_equal(p[1], u[0])


def test_reference_argmax_first_max_wins_and_nan_errors():
    """cpu/tests.rs:128-141."""
    x = np.array([1.0, 5.0, 5.0, -1.0, 0.0, 0.0, 0.0, 0.0, -3.0, -2.0, -2.0, -9.0],
                 np.float32).reshape(3, 4)
    assert list(orc.argmax(x)) == [1, 0, 1]
    with pytest.raises(orc.OracleError) as e:
        orc.argmax(np.array([[0.0, np.nan]], np.float32))
    assert e.value.code == orc.NAN


def test_argmax_special_values():
    x = np.array([[-np.inf, -np.inf], [-0.0, 0.0], [np.inf, np.inf]], np.float32)
    assert list(orc.argmax(x)) == [0, 0, 0]
    with pytest.raises(orc.OracleError):
        orc.argmax(np.array([[1.0, 2.0], [np.nan, 0.0]], np.float32))


def test_embed_and_random_weights_follow_testutil():
    """testutil.rs:46-91: embed is rand_weight(seed*1000, [vocab, h], 1.0); the
    layer matrices are scaled by 1/sqrt(in); norms are 1 + 0.1 x."""
    cfg = W.tiny_config()
    w = orc.random_weights(cfg, 7)
    assert np.array_equal(w["embed"].ravel(), orc.rand_vec(7000, 37 * 48))
    wq = w["layers"][1]["wq"]
    assert wq.shape == (48, 48)
    assert np.array_equal(wq.ravel(), orc.rand_vec(7000 + 21, 48 * 48) * np.float32(1 / math.sqrt(48)))
    assert np.allclose(w["final_norm"], 1 + 0.1 * orc.rand_vec(7999, 48), rtol=0, atol=1e-7)
    e = orc.embed(w["embed"], [3, 0, 36])
    assert np.array_equal(e, w["embed"][[3, 0, 36]])


# ---- Llama::forward ------------------------------------------------------------

def _tiny_model():
    """model.rs:366-383: tiny_config, random_weights(seed 7), block size 4,
    32 blocks, max_model_len 128."""
    cfg = W.tiny_config()
    return orc.Llama(cfg, orc.random_weights(cfg, 7), num_blocks=32, block_size=4, max_len=128)


def test_reference_prefill_then_decode_matches_full_prefill():
    """model.rs:447-495."""
    n, k = 13, 5
    p = W.ref_prompt(n, 3)
    table = [6, 1, 9, 3]
    ids_full, logits_full = _tiny_model().prefill(p, [(0, n, table)], 4)
    m2 = _tiny_model()
    ids, logits = m2.prefill(p[:n - k], [(0, n - k, table)], 4)
    for pos in range(n - k, n):
        ids, logits = m2.decode(p[pos:pos + 1], [(pos, table)], 4)
    assert list(ids) == list(ids_full)
    assert orc.max_rel_diff(logits, logits_full) < 1e-5


def test_reference_prefill_with_context_matches_full_prefill():
    """model.rs:497-539."""
    n = 11
    p = W.ref_prompt(n, 5)
    table = [2, 0, 7]
    ids_full, logits_full = _tiny_model().prefill(p, [(0, n, table)], 4)
    m2 = _tiny_model()
    m2.prefill(p[:6], [(0, 6, table)], 4)
    ids, logits = m2.prefill(p[6:], [(6, 5, table)], 4)
    assert list(ids) == list(ids_full)
    assert orc.max_rel_diff(logits, logits_full) < 1e-5


def test_reference_batched_prefill_is_batch_invariant():
    """model.rs:541-583: bitwise."""
    pa, pb = W.ref_prompt(7, 1), W.ref_prompt(10, 2)
    ta, tb = [3, 5], [0, 8, 1]
    ia, la = _tiny_model().prefill(pa, [(0, 7, ta)], 4)
    ib, lb = _tiny_model().prefill(pb, [(0, 10, tb)], 4)
    ids, logits = _tiny_model().prefill(pa + pb, [(0, 7, ta), (0, 10, tb)], 4)
    assert list(ids) == [ia[0], ib[0]]
    assert np.array_equal(logits[0], la[0]) and np.array_equal(logits[1], lb[0])


def _dense_llama_f64(cfg, w, tokens):
    """Llama from the architecture, in float64: contiguous K/V, full causal
    attention, HF rotate-half RoPE with float64 llama3 frequencies.  Returns
    the logits of every position."""
    hd, H = cfg.head_dim, cfg.num_attention_heads
    KVH = cfg.num_key_value_heads
    grp = H // KVH
    eps = cfg.rms_norm_eps
    rs = cfg.rope_scaling
    half = hd // 2
    inv = np.zeros(half)
    old = rs["original_max_position_embeddings"]
    for i in range(half):
        f = 1.0 / cfg.rope_theta ** (2 * i / hd)
        wl = 2 * math.pi / f
        if wl < old / rs["high_freq_factor"]:
            inv[i] = f
        elif wl > old / rs["low_freq_factor"]:
            inv[i] = f / rs["factor"]
        else:
            sm = (old / wl - rs["low_freq_factor"]) / (rs["high_freq_factor"] - rs["low_freq_factor"])
            inv[i] = (1 - sm) * f / rs["factor"] + sm * f
    T = len(tokens)
    ang = np.arange(T)[:, None] * inv[None, :]
    cos, sin = np.cos(ang), np.sin(ang)

    def norm(x, g):
        return g * x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)

    def rope(x, nh):
        x = x.reshape(T, nh, hd)
        a, b = x[..., :half], x[..., half:]
        c, s = cos[:, None, :], sin[:, None, :]
        return np.concatenate([a * c - b * s, b * c + a * s], axis=-1).reshape(T, nh * hd)

    f64 = {k: np.asarray(v, np.float64) for k, v in w.items() if k != "layers"}
    x = f64["embed"][tokens]
    mask = np.tril(np.ones((T, T), bool))
    for L in w["layers"]:
        L = {k: np.asarray(v, np.float64) for k, v in L.items()}
        n = norm(x, L["attn_norm"])
        q, k, v = rope(n @ L["wq"].T, H), rope(n @ L["wk"].T, KVH), n @ L["wv"].T
        out = np.zeros((T, H * hd))
        for h in range(H):
            kh = h // grp
            qh, kk, vv = q[:, h * hd:(h + 1) * hd], k[:, kh * hd:(kh + 1) * hd], v[:, kh * hd:(kh + 1) * hd]
            sc = qh @ kk.T / math.sqrt(hd)
            sc = np.where(mask, sc, -np.inf)
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            p /= p.sum(axis=1, keepdims=True)
            out[:, h * hd:(h + 1) * hd] = p @ vv
        x = x + out @ L["wo"].T
        n = norm(x, L["mlp_norm"])
        g, u = n @ L["w_gate"].T, n @ L["w_up"].T
        x = x + (g / (1 + np.exp(-g)) * u) @ L["w_down"].T
    return norm(x, f64["final_norm"]) @ f64["embed"].T


@pytest.mark.parametrize("which", ["tiny", "cfg1"])
def test_llama_matches_dense_float64_model(which):
    if which == "tiny":
        cfg, w = W.tiny_config(), None
        w = orc.random_weights(cfg, 7)
        tokens, bs, table = W.ref_prompt(13, 3), 4, [6, 1, 9, 3]
    else:
        cfg = W.cfg1_config()
        w = W.normal_weights(cfg, 11)
        tokens = list(np.random.default_rng(1).integers(0, cfg.vocab_size, 40))
        bs, table = 16, [5, 2, 9]
    want = _dense_llama_f64(cfg, w, tokens)
    m = orc.Llama(cfg, w, num_blocks=16, block_size=bs, max_len=128)
    # Prefill of all but the last two tokens, then two decode steps: the
    # logits of the last row of each step against the dense model's.
    n = len(tokens)
    _, l0 = m.prefill(tokens[:n - 2], [(0, n - 2, table)], bs)
    _, l1 = m.decode(tokens[n - 2:n - 1], [(n - 2, table)], bs)
    _, l2 = m.decode(tokens[n - 1:], [(n - 1, table)], bs)
    for got, row in ((l0[0], n - 3), (l1[0], n - 2), (l2[0], n - 1)):
        scale = np.abs(want[row]).max()
        assert np.abs(got - want[row]).max() <= 2e-5 * scale + 1e-6, row
