"""The kernels' soft-cap evaluation, c - 2c / (2^(x*s2) + 1) in float32
(soft_cap_log2 in csrc/pa_common.h), against cap * log2(e) * tanh(x * scale /
cap) in float64 (the reference's cap * tanh(logit / cap),
decode_paged_attention.py:82-84, in the kernels' log2 units).  float32 numpy
stands in for v_exp_f32 / v_rcp_f32 (each within about 1 ulp of it)."""
import numpy as np
import pytest

LOG2E = 1.4426950408889634


def soft_cap_f32(x, scale, cap):
    x = np.asarray(x, np.float32)
    s2 = np.float32(2.0 * np.float32(LOG2E) * np.float32(scale) / np.float32(cap))
    c = np.float32(np.float32(cap) * np.float32(LOG2E))
    with np.errstate(over="ignore"):
        e = np.exp2(x * s2, dtype=np.float32)
    r = (np.float32(1.0) / (e + np.float32(1.0))).astype(np.float32)
    return (c - (np.float32(2.0) * c) * r).astype(np.float32)


@pytest.mark.parametrize("cap,scale", [(50.0, 128 ** -0.5), (30.0, 256 ** -0.5), (5.0, 1.0), (1.0, 64 ** -0.5)])
def test_soft_cap_matches_tanh(cap, scale):
    x = np.concatenate([np.linspace(-4000, 4000, 200001), np.linspace(-1e-3, 1e-3, 2001),
                        [0.0, 1e-30, -1e-30, 3e38, -3e38]]).astype(np.float32)
    got = soft_cap_f32(x, scale, cap).astype(np.float64)
    want = cap * LOG2E * np.tanh(x.astype(np.float64) * scale / cap)
    err = np.abs(got - want)
    # a few float32 ulps of c = cap * log2 e, far below the bf16 rounding of P
    assert err.max() <= 8 * 2.0 ** -24 * cap * LOG2E, err.max()
    assert np.all(np.isfinite(got))
    # saturates to exactly +-c, keeps the sign and is monotone
    c = np.float32(np.float32(cap) * np.float32(LOG2E))
    assert soft_cap_f32([3e38], scale, cap)[0] == c and soft_cap_f32([-3e38], scale, cap)[0] == -c
    assert np.all(np.sign(got[np.abs(want) > 1e-5]) == np.sign(want[np.abs(want) > 1e-5]))
    order = np.argsort(x[:200001], kind="stable")
    assert np.all(np.diff(got[:200001][order]) >= 0)
