"""Pins for the oracle's QK RMSNorm + RoPE restatement (qwen3.py:59-78,286-296).

The reference cannot run here (no JAX), so the restatement is checked against
closed forms: the bf16 rounding of positions and of theta, RoPE at position 0,
RoPE as a complex multiplication of interleaved pairs (a half-split "NeoX"
rotation fails it), norm preservation, and RMSNorm's unit RMS and scale
invariance.
"""
from __future__ import annotations

import numpy as np

from oracle import paged_attention_oracle as ora


def _bf16(x):
    return ora.f32_to_bf16(np.asarray(x, np.float32))


def test_rope_positions_round_to_bf16():
    # bf16 keeps 8 significant bits: 257 is a tie between 256 and 258 -> 256 (even)
    got = ora.rope_positions([0, 1, 255, 256, 257, 259, 1000, 32000, 32001])
    assert got.tolist() == [0, 1, 255, 256, 256, 260, 1000, 32000, 32000]
    # linear scaling divides first (in float32), then rounds
    assert ora.rope_positions([10, 301], {"type": "linear", "factor": 2.0}).tolist() == [5.0, 150.0]


def test_inv_freq_closed_form():
    inv = ora.rope_inv_freq(128, 1e6)
    assert inv.shape == (64,)
    assert inv[0] == 1.0
    assert np.all(np.diff(inv) < 0)
    # theta is a bf16 value (1e6 -> 999424); each result within one bf16 ulp of the exact power
    theta = 999424.0
    exact = theta ** (-np.arange(0, 128, 2) / 128.0)
    assert np.all(np.abs(inv - exact) <= 2.0 ** -7 * exact)
    # every entry is a bf16 value
    assert np.array_equal(ora.round_bf16(inv), inv)


def test_rope_at_position_zero_is_identity():
    rng = np.random.default_rng(0)
    x = _bf16(rng.standard_normal((3, 4, 128)))
    c, s = ora.rope_cos_sin(np.zeros(3, np.int32), 128, 1e6)
    assert np.array_equal(ora.apply_rope(x, c, s), x)


def test_rope_is_complex_rotation_of_interleaved_pairs():
    rng = np.random.default_rng(1)
    t, h, d = 5, 3, 128
    x = _bf16(rng.standard_normal((t, h, d)))
    pos = np.array([0, 7, 300, 4097, 31999], np.int32)
    c, s = ora.rope_cos_sin(pos, d, 1e6)
    got = ora.bf16_to_f32(ora.apply_rope(x, c, s)).astype(np.float64)
    xf = ora.bf16_to_f32(x).astype(np.float64)
    z = (xf[..., 0::2] + 1j * xf[..., 1::2]) * (c[:, None, :] + 1j * s[:, None, :])
    want = np.empty_like(xf)
    want[..., 0::2], want[..., 1::2] = z.real, z.imag
    assert np.abs(got - want).max() <= 2.0 ** -8 * np.abs(want).max()
    # a half-split rotation (pairs (x[i], x[i + d/2])) is a different map
    half = np.concatenate([xf[..., :d // 2] * c[:, None] - xf[..., d // 2:] * s[:, None],
                           xf[..., :d // 2] * s[:, None] + xf[..., d // 2:] * c[:, None]], axis=-1)
    assert np.abs(half - want).max() > 0.1
    # the rotation keeps each pair's length (up to the bf16 roundings)
    n_in = np.hypot(xf[..., 0::2], xf[..., 1::2])
    n_out = np.hypot(got[..., 0::2], got[..., 1::2])
    assert np.abs(n_out - n_in).max() <= 0.02 * max(1.0, n_in.max())


def test_rope_cos_sin_match_float64_at_bf16_angles():
    pos = np.array([1, 2, 3, 100, 256, 20000], np.int32)
    c, s = ora.rope_cos_sin(pos, 128, 1e6)
    f = ora.round_bf16(ora.rope_positions(pos)[:, None] * ora.rope_inv_freq(128, 1e6)[None, :])
    assert np.abs(c - np.cos(f.astype(np.float64))).max() <= 2.0 ** -8
    assert np.abs(s - np.sin(f.astype(np.float64))).max() <= 2.0 ** -8


def test_rms_norm_unit_rms_and_scale_invariance():
    rng = np.random.default_rng(2)
    x = _bf16(rng.standard_normal((6, 5, 128)) * 3.0)
    ones = _bf16(np.ones(128))
    y = ora.bf16_to_f32(ora.rms_norm(x, ones, 1e-6)).astype(np.float64)
    assert np.abs(np.sqrt((y * y).mean(-1)) - 1.0).max() < 5e-3
    x2 = _bf16(ora.bf16_to_f32(x) * 4.0)  # exact scaling by a power of two
    assert np.array_equal(ora.rms_norm(x2, ones, 0.0), ora.rms_norm(x, ones, 0.0))
    w = _bf16(rng.uniform(0.5, 2.0, 128))
    yw = ora.bf16_to_f32(ora.rms_norm(x, w, 1e-6)).astype(np.float64)
    assert np.abs(yw - y * ora.bf16_to_f32(w)).max() <= 2.0 ** -7 * np.abs(yw).max()


def test_fused_step_stores_rotated_k_and_raw_v():
    rng = np.random.default_rng(3)
    t, h, hkv, d, nb, bs = 9, 4, 2, 128, 4, 8
    q = _bf16(rng.standard_normal((t, h, d)))
    k = _bf16(rng.standard_normal((t, hkv, d)))
    v = _bf16(rng.standard_normal((t, hkv, d)))
    qw, kw = _bf16(rng.uniform(0.5, 1.5, d)), _bf16(rng.uniform(0.5, 1.5, d))
    pos = rng.integers(0, 5000, t).astype(np.int32)
    slots = rng.permutation(nb * bs)[:t].astype(np.int32)
    slots[2] = -1
    kc0 = _bf16(rng.standard_normal((nb, bs, hkv, d)))
    vc0 = _bf16(rng.standard_normal((nb, bs, hkv, d)))
    q_out, kc, vc = ora.qk_norm_rope_store(q, k, v, qw, kw, pos, slots, kc0, vc0, eps=1e-6, rope_theta=1e6)
    c, s = ora.rope_cos_sin(pos, d, 1e6)
    assert np.array_equal(q_out, ora.apply_rope(ora.rms_norm(q, qw, 1e-6), c, s))
    k_rot = ora.apply_rope(ora.rms_norm(k, kw, 1e-6), c, s)
    fk, fv = kc.reshape(nb * bs, hkv, d), vc.reshape(nb * bs, hkv, d)
    for i in range(t):
        if slots[i] >= 0:
            assert np.array_equal(fk[slots[i]], k_rot[i]) and np.array_equal(fv[slots[i]], v[i])
    untouched = np.setdiff1d(np.arange(nb * bs), slots[slots >= 0])
    assert np.array_equal(fk[untouched], kc0.reshape(nb * bs, hkv, d)[untouched])
