"""Pins of the CPU oracle (oracle/paged_attention_oracle.py).

The reference (JAX/Pallas) cannot run here, so every oracle function is
checked against something independent of its own formula:

* bf16 conversion    -- torch's float32 -> bfloat16 cast (round to nearest even);
* kv_store / gather  -- their closed forms, element by element;
* prefill / decode   -- float64 brute force on tiny inputs, special cases that
                        reduce to textbook results (one key -> v_0, equal keys
                        -> mean(v), empty -> 0), and invariants (block
                        relabelling, split count, prefix truncation,
                        prefill-last-row == decode);
* mutation checks    -- a planted mistake (wrong kv head, missing scale,
                        swapped K/V, wrong block) must fail the same checks.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import paged_attention_oracle as ora

TOL = 2e-2   # bf16 output tolerance of the path
BRUTE_TOL = 1.2e-2  # oracle (bf16 P and partials, reference algebra) vs float64


def _bf16(rng, shape, scale=0.5):
    return ora.f32_to_bf16(rng.standard_normal(shape).astype(np.float32) * scale)


def _pool(rng, nb, bs, hkv, d=128):
    return _bf16(rng, (nb, bs, hkv, d)), _bf16(rng, (nb, bs, hkv, d))


def _tables(rng, lens, bs, nb):
    p = max(1, max(-(-int(n) // bs) for n in lens))
    perm = rng.permutation(nb)
    bt = np.full((len(lens), p), -1, np.int32)
    c = 0
    for b, n in enumerate(lens):
        k = -(-int(n) // bs)
        bt[b, :k] = perm[c:c + k]
        c += k
    return bt


# ---------------------------------------------------------------------------
# bf16
# ---------------------------------------------------------------------------
def test_bf16_matches_torch_round_to_nearest_even():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-30, 30, 20000),
        np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 65504.0, 3.3895314e38, 1e-40, -1e-40,
                  np.inf, -np.inf], np.float32),
        # exact ties between two bf16 values: must round to even
        (np.arange(1, 2000, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
    ])
    ours = ora.f32_to_bf16(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    assert np.array_equal(ora.bf16_to_f32(ours), torch.from_numpy(x).to(torch.bfloat16).float().numpy())


def test_bf16_nan_stays_nan():
    x = np.array([np.nan, -np.nan], np.float32)
    assert np.isnan(ora.bf16_to_f32(ora.f32_to_bf16(x))).all()


# ---------------------------------------------------------------------------
# KV store and gather: closed forms
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("nb,bs,hkv,t", [(8, 16, 2, 50), (4, 256, 8, 300), (3, 5, 1, 15)])
def test_kv_store_closed_form(nb, bs, hkv, t):
    rng = np.random.default_rng(t)
    kc, vc = _pool(rng, nb, bs, hkv)
    k = _bf16(rng, (t, hkv, 128))
    v = _bf16(rng, (t, hkv, 128))
    slots = rng.permutation(nb * bs)[:t].astype(np.int32)
    slots[::5] = -1                    # padding tokens
    slots[1] = nb * bs + 3             # past the pool: dropped
    k2, v2 = ora.kv_store(kc, vc, k, v, slots)
    written = np.zeros(nb * bs, bool)
    for i, s in enumerate(slots):
        if 0 <= s < nb * bs:
            assert np.array_equal(k2[s // bs, s % bs], k[i])
            assert np.array_equal(v2[s // bs, s % bs], v[i])
            written[s] = True
    keep = ~written.reshape(nb, bs)
    assert np.array_equal(k2[keep], kc[keep]) and np.array_equal(v2[keep], vc[keep])
    # inputs untouched
    assert not np.shares_memory(k2, kc)


def test_gather_closed_form():
    rng = np.random.default_rng(1)
    nb, bs, hkv = 16, 16, 2
    cache, _ = _pool(rng, nb, bs, hkv)
    lens = np.array([0, 1, 16, 17, 45], np.int32)
    bt = _tables(rng, lens, bs, nb)
    bt[0, 0] = -1
    ctx = ora.gather_kv(cache, bt, lens)
    for b, n in enumerate(lens):
        for j in range(bt.shape[1] * bs):
            want = cache[max(bt[b, j // bs], 0), j % bs] if j < n else np.zeros((hkv, 128), np.uint16)
            assert np.array_equal(ctx[b, j], want)


# ---------------------------------------------------------------------------
# prefill / decode vs float64 brute force
# ---------------------------------------------------------------------------
def _prefill_case(rng, lens, h, hkv, bs, prefix=None):
    lens = np.asarray(lens)
    prefix = np.zeros_like(lens) if prefix is None else np.asarray(prefix)
    kv_lens = lens + prefix
    nb = int(sum(-(-int(n) // bs) for n in kv_lens)) + 2
    kc, vc = _pool(rng, nb, bs, hkv)
    bt = _tables(rng, kv_lens, bs, nb)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    cuk = np.concatenate([[0], np.cumsum(kv_lens)]).astype(np.int32)
    pos = np.concatenate([np.arange(p, p + n) for p, n in zip(prefix, lens)]).astype(np.int32)
    q = _bf16(rng, (int(cu[-1]), h, 128))
    return q, kc, vc, bt, cu, cuk, pos, kv_lens


@pytest.mark.parametrize("lens,h,hkv,bs", [
    ([5, 1, 33], 4, 2, 16), ([40], 8, 8, 32), ([17, 30], 16, 2, 8), ([64, 3], 4, 1, 64)])
def test_prefill_vs_brute_force(lens, h, hkv, bs):
    rng = np.random.default_rng(sum(lens) + h)
    q, kc, vc, bt, cu, cuk, pos, kvl = _prefill_case(rng, lens, h, hkv, bs)
    got = ora.bf16_to_f32(ora.prefill_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3),
                                                bt, cu, pos))
    kctx, vctx = ora.gather_kv(kc, bt, kvl), ora.gather_kv(vc, bt, kvl)
    # the reference scales q in bf16 by bf16(1/sqrt(d)) (prefill...:60)
    sc = float(ora.round_bf16(np.float32(1 / math.sqrt(128))).reshape(-1)[0])
    qs = ora.f32_to_bf16(ora.round_bf16(ora.bf16_to_f32(q) * np.float32(sc)))
    want = ora.dense_prefill_f64(qs, kctx, vctx, cu, pos, scale=1.0)
    assert np.abs(got - want).max() <= BRUTE_TOL


def test_prefill_prefix_vs_brute_force():
    rng = np.random.default_rng(7)
    q, kc, vc, bt, cu, cuk, pos, kvl = _prefill_case(rng, [12, 30, 1], 8, 2, 16, prefix=[0, 20, 47])
    got = ora.bf16_to_f32(ora.prefill_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3),
                                                bt, cu, pos, cu_seqlens_k=cuk))
    kctx, vctx = ora.gather_kv(kc, bt, kvl), ora.gather_kv(vc, bt, kvl)
    sc = float(ora.round_bf16(np.float32(1 / math.sqrt(128))).reshape(-1)[0])
    qs = ora.f32_to_bf16(ora.round_bf16(ora.bf16_to_f32(q) * np.float32(sc)))
    want = ora.dense_prefill_f64(qs, kctx, vctx, cu, pos, cu_seqlens_k=cuk, scale=1.0)
    assert np.abs(got - want).max() <= BRUTE_TOL


@pytest.mark.parametrize("lens,h,hkv,bs", [([1, 15, 16, 17, 60, 0], 8, 2, 16), ([300, 40], 32, 8, 256)])
def test_decode_vs_brute_force(lens, h, hkv, bs):
    rng = np.random.default_rng(len(lens) + h)
    nb = int(sum(-(-int(n) // bs) for n in lens)) + 1
    kc, vc = _pool(rng, nb, bs, hkv)
    bt = _tables(rng, lens, bs, nb)
    q = _bf16(rng, (len(lens), h, 128))
    got = ora.bf16_to_f32(ora.decode_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, lens))
    want = ora.dense_decode_f64(q, ora.gather_kv(kc, bt, lens), ora.gather_kv(vc, bt, lens), lens)
    assert np.abs(got - want).max() <= BRUTE_TOL
    assert not got[np.asarray(lens) == 0].any()


def test_decode_soft_cap_vs_brute_force():
    rng = np.random.default_rng(3)
    lens = [100, 7]
    kc, vc = _pool(rng, 8, 16, 2)
    bt = _tables(rng, lens, 16, 8)
    q = _bf16(rng, (2, 4, 128), scale=2.0)
    got = ora.bf16_to_f32(ora.decode_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, lens,
                                               soft_cap=3.0))
    want = ora.dense_decode_f64(q, ora.gather_kv(kc, bt, lens), ora.gather_kv(vc, bt, lens), lens, soft_cap=3.0)
    assert np.abs(got - want).max() <= BRUTE_TOL


# ---------------------------------------------------------------------------
# special cases
# ---------------------------------------------------------------------------
def test_decode_single_key_returns_v0_exactly():
    rng = np.random.default_rng(4)
    kc, vc = _pool(rng, 4, 16, 2)
    bt = np.array([[2], [0]], np.int32)
    q = _bf16(rng, (2, 4, 128), scale=3.0)
    got = ora.decode_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, [1, 1])
    for b in range(2):
        for hh in range(4):
            assert np.array_equal(got[b, hh], vc[bt[b, 0], 0, hh // 2])


def test_prefill_first_row_returns_v0_exactly():
    rng = np.random.default_rng(5)
    q, kc, vc, bt, cu, cuk, pos, kvl = _prefill_case(rng, [9, 4], 4, 2, 16)
    got = ora.prefill_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, cu, pos)
    for b in range(2):
        row = cu[b]
        for hh in range(4):
            assert np.array_equal(got[row, hh], vc[bt[b, 0], 0, hh // 2])


def test_prefill_rows_at_the_first_position_see_only_kv0():
    """Every row of a sequence at the first row's position: kv j is visible
    iff j + pos0 <= pos_i, so each row sees kv 0 alone and returns V[0]
    exactly (prefill_paged_attention.py:79-82,108-115)."""
    rng = np.random.default_rng(8)
    q, kc, vc, bt, cu, cuk, pos, kvl = _prefill_case(rng, [9, 30], 4, 2, 16)
    pos = pos.copy()
    for b in range(2):
        pos[cu[b]:cu[b + 1]] = 100 + 7 * b
    got = ora.prefill_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, cu, pos)
    for b in range(2):
        for row in range(cu[b], cu[b + 1]):
            for hh in range(4):
                assert np.array_equal(got[row, hh], vc[bt[b, 0], 0, hh // 2])


def test_prefill_rows_past_the_end_see_the_whole_sequence():
    """Rows after the first at position pos0 + L - 1 see every kv token of
    their sequence: non-causal attention, computed here in float64 from the
    gathered K/V (q pre-scaled in bf16 as prefill_paged_attention.py:60)."""
    rng = np.random.default_rng(9)
    lens = [13, 40]
    q, kc, vc, bt, cu, cuk, pos_rows, kvl = _prefill_case(rng, lens, 4, 2, 16)
    pos = pos_rows.copy()
    for b, n in enumerate(lens):
        pos[cu[b] + 1:cu[b + 1]] = pos[cu[b]] + n - 1
    got = ora.bf16_to_f32(ora.prefill_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3),
                                                bt, cu, pos))
    # planted mistake: masking by row index (the contiguous positions) instead
    bad = ora.bf16_to_f32(ora.prefill_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3),
                                                bt, cu, pos_rows))
    bad_err = 0.0
    kctx = ora.bf16_to_f32(ora.gather_kv(kc, bt, kvl)).astype(np.float64)
    vctx = ora.bf16_to_f32(ora.gather_kv(vc, bt, kvl)).astype(np.float64)
    sc = float(ora.round_bf16(np.float32(1 / math.sqrt(128))).reshape(-1)[0])
    qs = ora.round_bf16(ora.bf16_to_f32(q) * np.float32(sc)).astype(np.float64)
    for b, n in enumerate(lens):
        for row in range(cu[b] + 1, cu[b + 1]):
            for hh in range(4):
                logits = kctx[b, :n, hh // 2] @ qs[row, hh]
                w = np.exp(logits - logits.max())
                want = (w / w.sum()) @ vctx[b, :n, hh // 2]
                assert np.abs(got[row, hh] - want).max() <= BRUTE_TOL
                bad_err = max(bad_err, float(np.abs(bad[row, hh] - want).max()))
    assert bad_err > 0.05


def test_prefill_rows_before_the_first_kv_position_are_zero():
    """A row whose position precedes its sequence's first kv position sees no
    key.  Contract: the row is 0, as the reference's dense definition gives it
    (prefill_paged_attention.py:502, qwen3.py:166); the Pallas kernel's finite
    mask_value (prefill...:62-64,109-117) would give a mean of V over its
    loaded blocks instead.  Both oracle forms must agree on 0, and the other
    rows must still match float64 attention."""
    rng = np.random.default_rng(12)
    lens = [20, 9]
    q, kc, vc, bt, cu, cuk, pos, kvl = _prefill_case(rng, lens, 4, 2, 16)
    pos = pos.copy()
    # sequence 0: row 0 keeps position 50; rows 5..9 drop below it (no key)
    pos[cu[0]:cu[1]] = 50 + np.arange(20)
    pos[cu[0] + 5:cu[0] + 10] = 40 + np.arange(5)
    blind = np.arange(cu[0] + 5, cu[0] + 10)
    got = ora.prefill_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, cu, pos)
    assert not got[blind].any()
    kctx, vctx = ora.gather_kv(kc, bt, kvl), ora.gather_kv(vc, bt, kvl)
    sc = float(ora.round_bf16(np.float32(1 / math.sqrt(128))).reshape(-1)[0])
    qs = ora.f32_to_bf16(ora.round_bf16(ora.bf16_to_f32(q) * np.float32(sc)))
    want = ora.dense_prefill_f64(qs, kctx, vctx, cu, pos, scale=1.0)
    assert not want[blind].any()
    assert np.abs(ora.bf16_to_f32(got) - want).max() <= BRUTE_TOL
    # the kernel-faithful alternative (finite mask value, no zeroing) is
    # what the contract rules out: it gives a nonzero mean of V there
    mean_v = ora.bf16_to_f32(vc[bt[0, :2]].reshape(32, 2, 128))[:20].mean(axis=0)
    assert np.abs(mean_v).max() > 0.05


def test_equal_keys_give_mean_of_values():
    rng = np.random.default_rng(6)
    kc, vc = _pool(rng, 2, 64, 1)
    kc[:] = kc[0, 0]                     # every key identical
    q = _bf16(rng, (1, 2, 128))
    bt = np.array([[1, 0]], np.int32)
    n = 100
    got = ora.bf16_to_f32(ora.decode_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, [n]))
    ctx = ora.bf16_to_f32(ora.gather_kv(vc, bt, [n]))[0, :n, 0]
    assert np.abs(got[0] - ctx.mean(0)[None]).max() <= 1e-2


def test_rows_outside_sequences_are_zero():
    rng = np.random.default_rng(8)
    q, kc, vc, bt, cu, cuk, pos, kvl = _prefill_case(rng, [5, 6], 4, 2, 16)
    qpad = np.concatenate([q, _bf16(rng, (5, 4, 128))])
    pos = np.concatenate([pos, np.zeros(5, np.int32)])
    got = ora.prefill_attention(qpad, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, cu, pos)
    assert not got[11:].any() and got[:11].any()


# ---------------------------------------------------------------------------
# invariants
# ---------------------------------------------------------------------------
def test_block_relabelling_is_bit_identical():
    rng = np.random.default_rng(9)
    q, kc, vc, bt, cu, cuk, pos, kvl = _prefill_case(rng, [50, 70], 8, 2, 16)
    a = ora.prefill_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, cu, pos)
    perm = rng.permutation(kc.shape[0])
    kc2, vc2 = np.empty_like(kc), np.empty_like(vc)
    kc2[perm], vc2[perm] = kc, vc
    bt2 = np.where(bt >= 0, perm[np.maximum(bt, 0)], -1).astype(np.int32)
    b = ora.prefill_attention(q, kc2.transpose(2, 0, 1, 3), vc2.transpose(2, 0, 1, 3), bt2, cu, pos)
    assert np.array_equal(a, b)


def test_split_count_changes_only_rounding():
    rng = np.random.default_rng(10)
    lens = [700, 300]
    kc, vc = _pool(rng, 12, 128, 2)
    bt = _tables(rng, lens, 128, 12)
    bt = np.concatenate([bt, np.full((2, 8 - bt.shape[1]), -1, np.int32)], 1)
    q = _bf16(rng, (2, 4, 128))
    outs = [ora.bf16_to_f32(ora.decode_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, lens,
                                                 k_splits=ks)) for ks in (1, 2, 4, 8)]
    for o in outs[1:]:
        assert np.abs(o - outs[0]).max() <= TOL


def test_prefix_truncation_does_not_change_earlier_rows():
    rng = np.random.default_rng(11)
    q, kc, vc, bt, cu, cuk, pos, kvl = _prefill_case(rng, [40], 4, 2, 16)
    a = ora.prefill_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, cu, pos)
    kc2, vc2 = kc.copy(), vc.copy()
    # scramble every kv token at index >= 25 (rows < 25 must not see them)
    for j in range(25, 40):
        kc2[bt[0, j // 16], j % 16] = _bf16(rng, (2, 128))
        vc2[bt[0, j // 16], j % 16] = _bf16(rng, (2, 128))
    b = ora.prefill_attention(q, kc2.transpose(2, 0, 1, 3), vc2.transpose(2, 0, 1, 3), bt, cu, pos)
    assert np.array_equal(a[:25], b[:25]) and not np.array_equal(a[25:], b[25:])


def test_prefill_last_row_matches_decode():
    rng = np.random.default_rng(12)
    q, kc, vc, bt, cu, cuk, pos, kvl = _prefill_case(rng, [200], 8, 2, 16)
    bt = np.concatenate([bt, np.full((1, 16 - bt.shape[1]), -1, np.int32)], 1)  # decode splits need 16 | width
    pre = ora.bf16_to_f32(ora.prefill_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, cu, pos))
    sc = float(ora.round_bf16(np.float32(1 / math.sqrt(128))).reshape(-1)[0])
    qs = ora.f32_to_bf16(ora.round_bf16(ora.bf16_to_f32(q[-1:]) * np.float32(sc)))
    dec = ora.bf16_to_f32(ora.decode_attention(qs, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, [200]))
    assert np.abs(pre[-1] - dec[0]).max() <= TOL


def test_gqa_mapping_matches_repeat():
    """q head h reads kv head h // G, i.e. the same as jnp.repeat of K/V over heads (qwen3.py:81-86)."""
    rng = np.random.default_rng(13)
    q, kc, vc, bt, cu, cuk, pos, kvl = _prefill_case(rng, [30], 8, 2, 16)
    a = ora.prefill_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, cu, pos)
    kr, vr = np.repeat(kc, 4, axis=2), np.repeat(vc, 4, axis=2)
    b = ora.prefill_attention(q, kr.transpose(2, 0, 1, 3), vr.transpose(2, 0, 1, 3), bt, cu, pos)
    assert np.array_equal(a, b)


# ---------------------------------------------------------------------------
# mutation checks: a planted mistake must fail the pins above
# ---------------------------------------------------------------------------
def test_planted_mistakes_are_caught():
    rng = np.random.default_rng(14)
    q, kc, vc, bt, cu, cuk, pos, kvl = _prefill_case(rng, [40, 20], 8, 2, 16)
    kctx, vctx = ora.gather_kv(kc, bt, kvl), ora.gather_kv(vc, bt, kvl)
    sc = float(ora.round_bf16(np.float32(1 / math.sqrt(128))).reshape(-1)[0])
    qs = ora.f32_to_bf16(ora.round_bf16(ora.bf16_to_f32(q) * np.float32(sc)))
    want = ora.dense_prefill_f64(qs, kctx, vctx, cu, pos, scale=1.0)

    def err(out):
        return np.abs(ora.bf16_to_f32(out) - want).max()

    good = ora.prefill_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, cu, pos)
    assert err(good) <= BRUTE_TOL
    # swapped K and V
    assert err(ora.prefill_attention(q, vc.transpose(2, 0, 1, 3), kc.transpose(2, 0, 1, 3), bt, cu, pos)) > 0.1
    # wrong GQA mapping (kv heads swapped)
    assert err(ora.prefill_attention(q, kc[:, :, ::-1].transpose(2, 0, 1, 3), vc[:, :, ::-1].transpose(2, 0, 1, 3),
                                     bt, cu, pos)) > 0.1
    # wrong block (tables shifted by one entry)
    bt_bad = np.roll(bt, 1, axis=1)
    assert err(ora.prefill_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt_bad, cu, pos)) > 0.1
    # missing 1/sqrt(d) scale (q pre-multiplied by sqrt(d))
    q_big = ora.f32_to_bf16(ora.bf16_to_f32(q) * np.float32(math.sqrt(128)))
    assert err(ora.prefill_attention(q_big, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, cu, pos)) > 0.1
    # off-by-one causal mask: every row but a sequence's first sees one key fewer
    pos_bad = pos.copy()
    first = np.zeros(len(pos), bool)
    first[cu[:-1]] = True
    pos_bad[~first] -= 1
    assert err(ora.prefill_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, cu, pos_bad)) > 0.05
    # a uniform shift of all positions is NOT a mistake: the mask is relative
    assert err(ora.prefill_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, cu, pos + 5)) <= BRUTE_TOL


def test_visible_pairs_closed_form():
    cu = np.array([0, 17, 145, 445, 956])
    assert ora.prefill_visible_pairs(cu) == sum(n * (n + 1) // 2 for n in (17, 128, 300, 511)) == 184375
    cuk = np.array([0, 27, 155, 455, 966])  # first sequence: prefix 10
    assert ora.prefill_visible_pairs(cu, cuk) == 184375 + 17 * 10


# ---------------------------------------------------------------------------
# mixed step (decode sequences first, then prefill sequences)
# ---------------------------------------------------------------------------
def _mixed_case(rng, dec_lens, pre_q, pre_prefix, h, hkv, bs, pad_rows=0):
    kv = list(dec_lens) + [p + n for p, n in zip(pre_prefix, pre_q)]
    nb = int(sum(-(-int(n) // bs) for n in kv)) + 2
    kc, vc = _pool(rng, nb, bs, hkv)
    bt = _tables(rng, kv, bs, nb)
    q_lens = [1] * len(dec_lens) + list(pre_q)
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    pos = np.concatenate([[max(n - 1, 0)] for n in dec_lens] +
                         [np.arange(p, p + n) for p, n in zip(pre_prefix, pre_q)]).astype(np.int32)
    pos = np.concatenate([pos, np.zeros(pad_rows, np.int32)])
    q = _bf16(rng, (int(cu[-1]) + pad_rows, h, 128))
    return q, kc, vc, bt, cu, np.asarray(kv, np.int32), pos


def test_mixed_vs_brute_force():
    rng = np.random.default_rng(11)
    dec, pre_q, pre_p = [1, 40, 0, 70], [5, 33, 1], [0, 12, 50]
    q, kc, vc, bt, cu, kv, pos = _mixed_case(rng, dec, pre_q, pre_p, 8, 2, 16, pad_rows=3)
    nd = len(dec)
    got = ora.bf16_to_f32(ora.mixed_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, cu, kv,
                                              pos, nd))
    kctx, vctx = ora.gather_kv(kc, bt, kv), ora.gather_kv(vc, bt, kv)
    # decode rows: q pre-scaled in bf16 by 1/bf16(sqrt(d)) (qwen3.py:207)
    qd = ora.f32_to_bf16(ora.round_bf16(ora.bf16_to_f32(q[cu[:nd]]) / np.float32(11.3125)))
    want_d = ora.dense_decode_f64(qd, kctx[:nd], vctx[:nd], kv[:nd])
    assert np.abs(got[cu[:nd]] - want_d).max() <= BRUTE_TOL
    assert not got[cu[2]].any()                       # kv length 0
    # prefill rows: q scaled by bf16(1/sqrt(d)) in bf16 (prefill...:60)
    sc = float(ora.round_bf16(np.float32(1 / math.sqrt(128))).reshape(-1)[0])
    base = int(cu[nd])
    qp = ora.f32_to_bf16(ora.round_bf16(ora.bf16_to_f32(q[base:cu[-1]]) * np.float32(sc)))
    cup = cu[nd:] - base
    cuk = np.concatenate([[0], np.cumsum(kv[nd:])])
    want_p = ora.dense_prefill_f64(qp, kctx[nd:], vctx[nd:], cup, pos[base:cu[-1]], cu_seqlens_k=cuk, scale=1.0)
    assert np.abs(got[base:cu[-1]] - want_p).max() <= BRUTE_TOL
    assert not got[cu[-1]:].any()                     # rows outside every sequence
    # mutation: treating the first prefill sequence as a decode sequence drops
    # its causal mask on row 0 and its later rows
    wrong = ora.bf16_to_f32(ora.mixed_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, cu, kv,
                                                pos, nd + 1))
    assert np.abs(wrong[base:cu[-1]] - want_p).max() > BRUTE_TOL


def test_mixed_decode_row_equals_prefill_last_row():
    """A decode sequence and a one-row prefill sequence over the same context
    differ only in how q is scaled; with the scales made equal they agree."""
    rng = np.random.default_rng(12)
    q, kc, vc, bt, cu, kv, pos = _mixed_case(rng, [90], [1], [89], 4, 2, 16)
    bt[1] = bt[0]                                     # same context pages
    q[1] = q[0]                                       # same query
    kp, vp = kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3)
    both = ora.bf16_to_f32(ora.mixed_attention(q, kp, vp, bt, cu, kv, pos, 1))
    assert np.abs(both[0] - both[1]).max() <= 2e-2 * max(1.0, np.abs(both).max())


# ---------------------------------------------------------------------------
# float8 e4m3fn pages
# ---------------------------------------------------------------------------
def test_fp8_tables_match_torch_float8():
    codes = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = ora.fp8_e4m3_decode(codes)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin], want[fin]) and np.isnan(got[~fin]).all()
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(50000) * 10.0 ** rng.uniform(-4, 2.6, 50000),
                        ora.fp8_e4m3_decode(codes[np.isfinite(want)]),            # exact codes
                        (ora.fp8_e4m3_decode(codes[:126]) + ora.fp8_e4m3_decode(codes[1:127])) / 2]  # ties
                       ).astype(np.float32)
    x = x[np.abs(x) <= 448]
    want_c = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ora.fp8_e4m3_encode(x), want_c)


def test_fp8_row_quantiser():
    rng = np.random.default_rng(1)
    x = _bf16(rng, (50, 128), scale=3.0)
    x[3] = 0
    codes, sc = ora.quantize_fp8_rows(x)
    xf = ora.bf16_to_f32(x)
    back = ora.fp8_e4m3_decode(codes) * sc[:, None]
    assert sc[3] == 1.0 and not codes[3].any()
    amax = np.abs(xf).max(axis=1)
    # scales are powers of two, the smallest that keep the row within 448:
    # the row maximum lands in (224, 448] before rounding
    m, _ = np.frexp(sc)
    assert np.all(m == 0.5)
    assert np.all(amax[amax > 0] / sc[amax > 0] <= 448.0) and np.all(amax[amax > 0] / sc[amax > 0] > 224.0)
    # every element within half an e4m3 step of its value (relative 2^-4 of the row maximum)
    rel = np.abs(back - xf) / np.maximum(amax[:, None], 1e-30)
    assert rel.max() <= 2.0 ** -4 * 1.0001
    # edge cases of the scale rule: a maximum of exactly 448 * 2^k and one
    # just above (next bf16), and a tiny row whose scale stops at 2^-126
    edge = ora.f32_to_bf16(np.array([[448.0, 1.0], [450.0, 1.0], [2.0 ** -130, 0.0], [1.75 * 2 ** 10, -3.0]],
                                    dtype=np.float32))
    ce, se = ora.quantize_fp8_rows(edge)
    assert list(se) == [1.0, 2.0, 2.0 ** -126, 4.0]
    assert ora.fp8_e4m3_decode(ce[0, :1])[0] == 448.0 and ora.fp8_e4m3_decode(ce[3, :1])[0] == 448.0


def test_decode_fp8_vs_brute_force():
    """Quantized decode == float64 attention over the dequantised context."""
    rng = np.random.default_rng(13)
    lens, h, hkv, bs = [5, 40, 0, 33], 8, 2, 16
    nb = int(sum(-(-n // bs) for n in lens)) + 1
    kf, vf = _pool(rng, nb, bs, hkv)
    kq, ks = ora.quantize_fp8_rows(kf)            # ks [NB, BS, Hkv]
    vq, vs = ora.quantize_fp8_rows(vf)
    bt = _tables(rng, lens, bs, nb)
    bt = np.concatenate([bt, np.full((len(lens), 4 - bt.shape[1]), -1, np.int32)], axis=1)
    q = _bf16(rng, (len(lens), h, 128))
    got = ora.bf16_to_f32(ora.decode_attention(q, kq.transpose(2, 0, 1, 3), vq.transpose(2, 0, 1, 3), bt, lens,
                                               k_scales_pages=ks.transpose(2, 0, 1),
                                               v_scales_pages=vs.transpose(2, 0, 1)))
    kd = ora.f32_to_bf16(ora.fp8_e4m3_decode(kq))                       # exact in bf16
    # V dequantised exactly in float32 is what the reference's f32 PV sees; compare in f64
    vd64 = ora.fp8_e4m3_decode(vq).astype(np.float64) * vs[..., None]
    kd64 = ora.bf16_to_f32(kd).astype(np.float64) * ks[..., None]
    want = np.zeros_like(got, dtype=np.float64)
    for b, n in enumerate(lens):
        if n == 0:
            continue
        pages = bt[b, :(n + bs - 1) // bs]
        kc = kd64[pages].reshape(-1, hkv, 128)[:n]
        vc = vd64[pages].reshape(-1, hkv, 128)[:n]
        for hh in range(h):
            kh = hh // (h // hkv)
            lg = kc[:, kh] @ ora.bf16_to_f32(q[b, hh]).astype(np.float64)
            w = np.exp(lg - lg.max())
            want[b, hh] = (w / w.sum()) @ vc[:, kh]
    assert np.abs(got - want).max() <= BRUTE_TOL
    assert not got[2].any()


def test_prefill_fp8_vs_brute_force():
    """Quantized prefill == float64 attention over the dequantised context."""
    rng = np.random.default_rng(14)
    q, kc, vc, bt, cu, cuk, pos, kvl = _prefill_case(rng, [12, 30, 1], 8, 2, 16, prefix=[0, 20, 47])
    kq, ks = ora.quantize_fp8_rows(kc)
    vq, vs = ora.quantize_fp8_rows(vc)
    got = ora.bf16_to_f32(ora.prefill_attention(q, kq.transpose(2, 0, 1, 3), vq.transpose(2, 0, 1, 3), bt, cu, pos,
                                                cu_seqlens_k=cuk, k_scales_pages=ks.transpose(2, 0, 1),
                                                v_scales_pages=vs.transpose(2, 0, 1)))
    sc = float(ora.round_bf16(np.float32(1 / math.sqrt(128))).reshape(-1)[0])
    qs = ora.bf16_to_f32(ora.f32_to_bf16(ora.round_bf16(ora.bf16_to_f32(q) * np.float32(sc)))).astype(np.float64)
    kd = ora.fp8_e4m3_decode(kq).astype(np.float64) * ks[..., None]
    vd = ora.fp8_e4m3_decode(vq).astype(np.float64) * vs[..., None]
    want = np.zeros_like(got, dtype=np.float64)
    for b in range(len(cu) - 1):
        lq, lk = cu[b + 1] - cu[b], cuk[b + 1] - cuk[b]
        pages = bt[b, :(lk + 15) // 16]
        kctx = kd[pages].reshape(-1, 2, 128)[:lk]
        vctx = vd[pages].reshape(-1, 2, 128)[:lk]
        for i in range(lq):
            row = cu[b] + i
            vis = np.arange(lk) + pos[cu[b]] - (lk - lq) <= pos[row]
            for hh in range(8):
                lg = kctx[vis, hh // 4] @ qs[row, hh]
                w = np.exp(lg - lg.max())
                want[row, hh] = (w / w.sum()) @ vctx[vis, hh // 4]
    assert np.abs(got - want).max() <= BRUTE_TOL


# ---------------------------------------------------------------------------
# integer pages (int8 / uint8 codes): the reference's astype keeps the integer
# ---------------------------------------------------------------------------
def test_code_values_follow_the_reference_cast():
    """int8 / uint8 codes are the integers (jnp.astype of an integer page to
    bf16 or float32, decode...:72-75,108-115), e4m3 codes their float8 value;
    either integer kind may come as its uint8 bit pattern."""
    raw = np.arange(256, dtype=np.uint8)
    assert np.array_equal(ora.code_values(raw, "uint8"), np.arange(256, dtype=np.float32))
    assert np.array_equal(ora.code_values(raw, "int8"), raw.view(np.int8).astype(np.float32))
    assert np.array_equal(ora.code_values(raw.view(np.int8), "int8"), ora.code_values(raw, "int8"))
    assert ora.code_values(np.array([0x80, 0x7F, 0xFF], np.uint8), "int8").tolist() == [-128.0, 127.0, -1.0]
    fin = np.isfinite(ora.fp8_e4m3_decode(raw))
    assert np.array_equal(ora.code_values(raw, "e4m3")[fin], ora.fp8_e4m3_decode(raw)[fin])
    # every integer code is exact in bf16
    for kind in ("int8", "uint8"):
        v = ora.code_values(raw, kind)
        assert np.array_equal(ora.bf16_to_f32(ora.f32_to_bf16(v)), v)


@pytest.mark.parametrize("kind", ["int8", "uint8"])
def test_integer_pages_vs_brute_force(kind):
    """Decode and prefill over integer codes with per-token scales == float64
    attention over code * scale (K and V), within the oracle's bf16 bar."""
    rng = np.random.default_rng(31 if kind == "int8" else 32)
    lens, h, hkv, bs = [5, 40, 0, 33], 8, 2, 16
    nb = int(sum(-(-n // bs) for n in lens)) + 1
    lo, hi = (-128, 128) if kind == "int8" else (0, 256)
    dt = np.int8 if kind == "int8" else np.uint8
    kq = rng.integers(lo, hi, (nb, bs, hkv, 128)).astype(dt)
    vq = rng.integers(lo, hi, (nb, bs, hkv, 128)).astype(dt)
    ks = (rng.uniform(0.5, 1.5, (nb, bs, hkv)) / 256).astype(np.float32)
    vs = (rng.uniform(0.5, 1.5, (nb, bs, hkv)) / 256).astype(np.float32)
    bt = _tables(rng, lens, bs, nb)
    bt = np.concatenate([bt, np.full((len(lens), 4 - bt.shape[1]), -1, np.int32)], axis=1)
    q = _bf16(rng, (len(lens), h, 128))
    got = ora.bf16_to_f32(ora.decode_attention(q, kq.transpose(2, 0, 1, 3), vq.transpose(2, 0, 1, 3), bt, lens,
                                               k_scales_pages=ks.transpose(2, 0, 1),
                                               v_scales_pages=vs.transpose(2, 0, 1), code_type=kind))
    kd64 = kq.astype(np.float64) * ks[..., None]
    vd64 = vq.astype(np.float64) * vs[..., None]
    want = np.zeros_like(got, dtype=np.float64)
    for b, n in enumerate(lens):
        if n == 0:
            continue
        pages = bt[b, :(n + bs - 1) // bs]
        kc = kd64[pages].reshape(-1, hkv, 128)[:n]
        vc = vd64[pages].reshape(-1, hkv, 128)[:n]
        for hh in range(h):
            kh = hh // (h // hkv)
            lg = kc[:, kh] @ ora.bf16_to_f32(q[b, hh]).astype(np.float64)
            w = np.exp(lg - lg.max())
            want[b, hh] = (w / w.sum()) @ vc[:, kh]
    assert np.abs(got - want).max() <= BRUTE_TOL
    assert not got[2].any()
    # prefill over the same pool, one sequence with a cached prefix
    cu = np.array([0, 12], np.int32)
    cuk = np.array([0, 40], np.int32)
    pos = np.arange(28, 40, dtype=np.int32)
    qp = _bf16(rng, (12, h, 128))
    btp = bt[1:2]
    gp = ora.bf16_to_f32(ora.prefill_attention(qp, kq.transpose(2, 0, 1, 3), vq.transpose(2, 0, 1, 3), btp, cu, pos,
                                               cu_seqlens_k=cuk, k_scales_pages=ks.transpose(2, 0, 1),
                                               v_scales_pages=vs.transpose(2, 0, 1), code_type=kind))
    sc = float(ora.round_bf16(np.float32(1 / math.sqrt(128))).reshape(-1)[0])
    qs = ora.bf16_to_f32(ora.f32_to_bf16(ora.round_bf16(ora.bf16_to_f32(qp) * np.float32(sc)))).astype(np.float64)
    kctx = kd64[btp[0, :3]].reshape(-1, hkv, 128)[:40]
    vctx = vd64[btp[0, :3]].reshape(-1, hkv, 128)[:40]
    wantp = np.zeros_like(gp, dtype=np.float64)
    for i in range(12):
        vis = np.arange(40) <= pos[i]
        for hh in range(h):
            lg = kctx[vis, hh // 4] @ qs[i, hh]
            w = np.exp(lg - lg.max())
            wantp[i, hh] = (w / w.sum()) @ vctx[vis, hh // 4]
    assert np.abs(gp - wantp).max() <= BRUTE_TOL
