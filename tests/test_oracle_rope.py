"""Pins the oracle's RoPE restatement (crates/engine/src/backend/cpu/rope.rs).

The reference's own tests (rope.rs:104-157) are restated first; the rest
check the same functions against what the mathematics fixes, computed
independently in float64: HF's llama3 frequency formula, cos/sin of the f32
angle, and the rotation as an orthogonal map.
"""
import math

import numpy as np
import pytest

import oracle as orc

HD_1B = 64          # LLAMA_3_2_1B head_dim (config.rs:41-56)
THETA_1B = 500000.0


def _inv_f64(head_dim, theta, factor=32.0, low=1.0, high=4.0, old_ctx=8192):
    """HF _compute_llama3_parameters in float64 (no f32 rounding)."""
    out = []
    low_wl, high_wl = old_ctx / low, old_ctx / high
    for i in range(head_dim // 2):
        inv = 1.0 / theta ** (2 * i / head_dim)
        wl = 2 * math.pi / inv
        if wl < high_wl:
            out.append(inv)
        elif wl > low_wl:
            out.append(inv / factor)
        else:
            sm = (old_ctx / wl - low) / (high - low)
            out.append((1 - sm) * inv / factor + sm * inv)
    return np.array(out)


def test_reference_llama3_scaling_bands():
    """rope.rs:108-128."""
    inv = orc.rope_inv_freq(HD_1B, THETA_1B)
    assert inv.shape == (32,)
    assert inv[0] == 1.0
    raw = np.float32(1.0) / np.float32(THETA_1B) ** np.float32(62.0 / 64.0)
    assert abs(inv[31] - raw / 32) <= raw * 1e-6
    for i in range(32):
        raw = np.float32(1.0) / np.float32(THETA_1B) ** np.float32(2 * i / 64.0)
        assert inv[i] <= raw and inv[i] >= raw / 32 * (1 - 1e-6), i
        if i:
            assert inv[i] < inv[i - 1]


def test_reference_rotation_matches_direct_formula_and_preserves_norm():
    """rope.rs:130-150: position 37, two heads of width 64."""
    inv = orc.rope_inv_freq(HD_1B, THETA_1B)
    c, s = orc.rope_table(inv, 40)
    row0 = np.array([((i * 37 % 11) - 5.0) / 3.0 for i in range(128)], np.float32)
    row = orc.rope_apply(row0[None, :], [37], c, s)[0]
    for head in range(2):
        for i in range(32):
            th = np.float32(37.0) * inv[i]
            a, b = row0[head * 64 + i], row0[head * 64 + 32 + i]
            e1 = a * np.cos(th) - b * np.sin(th)
            e2 = b * np.cos(th) + a * np.sin(th)
            assert abs(row[head * 64 + i] - e1) < 1e-6
            assert abs(row[head * 64 + 32 + i] - e2) < 1e-6
    n0, n1 = float((row0 ** 2).sum()), float((row ** 2).sum())
    assert abs(n0 - n1) < 1e-3 * n0


def test_reference_position_zero_is_identity():
    """rope.rs:152-157."""
    inv = orc.rope_inv_freq(HD_1B, THETA_1B)
    c, s = orc.rope_table(inv, 1)
    row0 = np.arange(64, dtype=np.float32)[None, :]
    assert np.array_equal(orc.rope_apply(row0, [0], c, s), row0)


@pytest.mark.parametrize("hd,theta", [(64, 500000.0), (128, 500000.0), (64, 10000.0),
                                      (128, 10000.0), (8, 10000.0)])
def test_inv_freq_matches_float64_formula(hd, theta):
    """Every band (unscaled, fully scaled, interpolated) within f32 rounding of
    the float64 formula; a dropped branch or a swapped factor is off by >= 2x."""
    got = orc.rope_inv_freq(hd, theta).astype(np.float64)
    want = _inv_f64(hd, theta)
    assert np.all(np.abs(got - want) <= 4e-6 * want)


def test_inv_freq_covers_all_three_bands():
    """At theta 500000, head_dim 128 the pairs fall in all three bands, so the
    float64 comparison above checks each branch."""
    inv = _inv_f64(128, 500000.0)
    wl = 2 * math.pi / np.array([1.0 / 500000.0 ** (2 * i / 128) for i in range(64)])
    assert (wl < 8192 / 4).any() and (wl > 8192).any() and ((wl >= 2048) & (wl <= 8192)).any()
    assert len(inv) == 64


def test_table_is_cos_sin_of_the_f32_angle():
    inv = orc.rope_inv_freq(128, 500000.0)
    c, s = orc.rope_table(inv, 3000)
    p = np.arange(3000, dtype=np.float32)[:, None]
    th = (p * inv[None, :]).astype(np.float32).astype(np.float64)
    assert np.max(np.abs(c - np.cos(th))) < 2e-6
    assert np.max(np.abs(s - np.sin(th))) < 2e-6


def test_apply_is_the_rotation_and_inverts():
    """x1' = a cos - b sin, x2' = b cos + a sin against float64 on random rows
    and positions; rotating back with -sin recovers the input; norms kept."""
    rng = np.random.default_rng(7)
    inv = orc.rope_inv_freq(128, 500000.0)
    c, s = orc.rope_table(inv, 5000)
    x = rng.standard_normal((50, 4 * 128)).astype(np.float32)
    pos = rng.integers(0, 5000, 50).astype(np.uint32)
    y = orc.rope_apply(x, pos, c, s)
    xs = x.reshape(50, 4, 2, 64).astype(np.float64)
    cc = c[pos][:, None, :].astype(np.float64)
    ss = s[pos][:, None, :].astype(np.float64)
    w1 = xs[:, :, 0] * cc - xs[:, :, 1] * ss
    w2 = xs[:, :, 1] * cc + xs[:, :, 0] * ss
    want = np.stack([w1, w2], axis=2).reshape(50, 512)
    assert np.max(np.abs(y - want)) < 1e-5
    back = orc.rope_apply(y, pos, c, -s)
    assert np.max(np.abs(back - x)) < 1e-5
    assert np.allclose((y ** 2).sum(1), (x ** 2).sum(1), rtol=1e-5)
