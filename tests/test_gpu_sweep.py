"""Seeded random sweep of the device entries against the oracle.

Every case draws its shape from one seed: the q heads per kv head
(G in 1, 2, 4, 8, 16, 20, 32), the kv heads, the page size (aligned and unaligned
to the 64-token prefill tile and the 16-token decode step), the batch, q
lengths including 0 and 1, cached prefixes and the soft cap.  The prefill
cases run through the kernel entry, hence with the work list.  Bar as in the
per-entry tests: max-abs 2e-2 on bf16 outputs, zero rows exactly zero.
A last sweep draws head sizes other than 128 (multiples of 16 up to 256) for
the generic kernels, taking prefill, decode and the mixed launch in turn.
PA_SWEEP_SEEDS=n runs n seeds per sweep instead of the default counts.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

import vllm_jax_amd.workloads as wl
from conftest import from_u16, u16
from oracle import paged_attention_oracle as ora

pytestmark = pytest.mark.gpu
TOL = 2e-2
PAGE_SIZES = [16, 24, 32, 48, 64, 128, 256]


def _heads(rng, max_g=32, groups=(1, 2, 4, 8, 16, 20, 32)):
    g = int(rng.choice([g for g in groups if g <= max_g]))
    hkv = int(rng.choice([1, 2, 4, 8] if g <= 8 else [1, 2, 4]))
    return g * hkv, hkv


def _seeds(default):
    n = os.environ.get("PA_SWEEP_SEEDS")
    return range(int(n) if n else default)


def _prefill_case(seed):
    rng = np.random.default_rng(1000 + seed)
    h, hkv = _heads(rng)
    bs = int(rng.choice(PAGE_SIZES))
    batch = int(rng.integers(1, 13))
    new = rng.integers(1, 400, batch)
    new[rng.random(batch) < 0.15] = 1
    new[rng.random(batch) < 0.1] = 0
    new[0] = max(new[0], 1)
    prefix = np.where(rng.random(batch) < 0.5, rng.integers(0, 700, batch), 0)
    cap = 6.0 if rng.random() < 0.25 else None
    return h, hkv, bs, new.tolist(), prefix.tolist(), cap


def _decode_case(seed):
    rng = np.random.default_rng(2000 + seed)
    h, hkv = _heads(rng)
    bs = int(rng.choice(PAGE_SIZES))
    batch = int(rng.integers(1, 17))
    lens = rng.integers(1, 5000, batch)
    lens[rng.random(batch) < 0.1] = 0
    lens[rng.random(batch) < 0.1] = 1
    cap = 6.0 if rng.random() < 0.25 else None
    return h, hkv, bs, lens.tolist(), cap


@pytest.mark.parametrize("seed", _seeds(16))
def test_prefill_sweep(pkg, dev, seed):
    import torch
    h, hkv, bs, new, prefix, cap = _prefill_case(seed)
    print(f"prefill sweep seed {seed}: H {h} Hkv {hkv} page {bs} new {new} prefix {prefix} cap {cap}", flush=True)
    pb = wl.make_prefix_prefill(prefix, new, num_heads=h, num_kv_heads=hkv, page_size=bs,
                                rng=np.random.default_rng(seed))
    t = wl.materialize_prefill(pb, seed, dev)
    before = u16(t["kv_cache"])
    kv = pkg.update_kv_cache(t["kv_cache"], t["slot_mapping"], t["k"], t["v"])
    out = pkg.prefill_paged_attention(t["q"], kv[0].permute(2, 0, 1, 3), kv[1].permute(2, 0, 1, 3),
                                      t["block_tables"], t["cu_seqlens_q"], t["slot_mapping"],
                                      t["input_positions"], max_seqlen_bucket=pb.max_seqlen_bucket,
                                      cu_seqlens_k=t["cu_seqlens_k"], attn_logits_soft_cap=cap)
    torch.cuda.synchronize()
    kc, vc = ora.kv_store(before[0], before[1], u16(t["k"]), u16(t["v"]), pb.slot_mapping)
    assert np.array_equal(u16(kv[0]), kc) and np.array_equal(u16(kv[1]), vc)
    ref = ora.prefill_attention(u16(t["q"]), kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3),
                                pb.block_tables, pb.cu_seqlens_q, pb.input_positions,
                                cu_seqlens_k=pb.cu_seqlens_k, soft_cap=cap)
    got = ora.bf16_to_f32(u16(out))
    err = float(np.abs(got - ora.bf16_to_f32(ref)).max())
    print(f"  max-abs err {err:.3e}")
    assert err <= TOL and np.isfinite(got).all()


@pytest.mark.parametrize("seed", _seeds(16))
def test_decode_sweep(pkg, dev, seed):
    import torch
    h, hkv, bs, lens, cap = _decode_case(seed)
    print(f"decode sweep seed {seed}: H {h} Hkv {hkv} page {bs} lens {lens} cap {cap}", flush=True)
    # power-of-two table width: the oracle keeps the reference's split divisibility rules
    width = 1 << (max(1, max(-(-n // bs) for n in lens)) - 1).bit_length()
    db = wl.make_decode(lens, num_heads=h, num_kv_heads=hkv, page_size=bs, rng=np.random.default_rng(seed),
                        table_width=width)
    d = wl.materialize_decode(db, seed, dev)
    kv = d["kv_cache"]
    # the reference's caller pre-scales q in bf16 (qwen3.py:207); the kernel entry applies no scale
    q = (d["q"] / torch.tensor(float(np.sqrt(128)), dtype=torch.bfloat16)).to(torch.bfloat16)
    out = pkg.decode_paged_attention(q, kv[0].permute(2, 0, 1, 3), kv[1].permute(2, 0, 1, 3),
                                     d["block_tables"], d["context_lens"], attn_logits_soft_cap=cap)
    torch.cuda.synchronize()
    kvh = u16(kv)
    ref = ora.decode_attention(u16(q), kvh[0].transpose(2, 0, 1, 3), kvh[1].transpose(2, 0, 1, 3),
                               db.block_tables, db.context_lens, soft_cap=cap)
    got = ora.bf16_to_f32(u16(out))
    err = float(np.abs(got - ora.bf16_to_f32(ref)).max())
    print(f"  max-abs err {err:.3e}")
    assert err <= TOL and np.isfinite(got).all()
    assert not got[np.asarray(lens) == 0].any()


@pytest.mark.parametrize("seed", _seeds(8))
def test_mixed_sweep(pkg, dev, seed):
    import torch
    from test_gpu_mixed import _case, _run
    rng = np.random.default_rng(3000 + seed)
    h, hkv = _heads(rng)
    bs = int(rng.choice(PAGE_SIZES))
    nd, npre = int(rng.integers(0, 9)), int(rng.integers(0 if seed % 4 else 1, 6))
    nd = max(nd, 1 - npre)  # at least one sequence
    dec = rng.integers(0, 5000, nd).tolist()
    pre_q = rng.integers(1, 300, npre).tolist()
    pre_p = np.where(rng.random(npre) < 0.5, rng.integers(0, 500, npre), 0).tolist()
    cap = 6.0 if rng.random() < 0.25 else None
    pad = int(rng.integers(0, 3))
    print(f"mixed sweep seed {seed}: H {h} Hkv {hkv} page {bs} dec {dec} pre_q {pre_q} pre_p {pre_p} cap {cap} "
          f"pad {pad}", flush=True)
    q, kc, vc, bt, cu, kv, pos = _case(rng, dec, pre_q, pre_p, h, hkv, bs, pad_rows=pad)
    max_q = max(pre_q) if pre_q else 0
    got = _run(pkg, dev, q, kc, vc, bt, cu, kv, pos, nd, max_q, soft_cap=cap)
    want = ora.mixed_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, cu, kv, pos, nd,
                               soft_cap=cap)
    err = float(np.abs(ora.bf16_to_f32(got) - ora.bf16_to_f32(want)).max())
    print(f"  max-abs err {err:.3e}")
    assert err <= TOL
    zero = np.ones(q.shape[0], bool)
    zero[cu[:nd]] = False
    for b in range(nd, len(kv)):
        zero[cu[b]:cu[b + 1]] = False
    zero[cu[:nd][kv[:nd] == 0]] = True
    assert not got[zero].any()


@pytest.mark.parametrize("seed", _seeds(6))
def test_fp8_sweep(pkg, dev, seed):
    """Quantized decode and prefill over the same random float8 pool."""
    import torch
    from test_gpu_fp8 import _quantized_pool
    rng = np.random.default_rng(4000 + seed)
    h, hkv = _heads(rng)
    bs = int(rng.choice([16, 32, 48, 64, 128, 256]))
    batch = int(rng.integers(1, 9))
    new = rng.integers(1, 300, batch)
    prefix = np.where(rng.random(batch) < 0.5, rng.integers(0, 600, batch), 0)
    kvl = prefix + new
    print(f"fp8 sweep seed {seed}: H {h} Hkv {hkv} page {bs} new {new.tolist()} prefix {prefix.tolist()}", flush=True)
    pages = [(int(n) + bs - 1) // bs for n in kvl]
    nb = sum(pages) + 2
    width = 1 << (max(pages) - 1).bit_length()
    kq, vq, ks, vs = _quantized_pool(rng, nb, bs, hkv)
    perm = rng.permutation(nb)
    bt = np.full((batch, width), -1, np.int32)
    c = 0
    for b, p in enumerate(pages):
        bt[b, :p] = perm[c:c + p]
        c += p
    i32 = lambda x: torch.as_tensor(np.ascontiguousarray(x, dtype=np.int32), device=dev)
    kd = torch.from_numpy(kq).to(dev).view(torch.float8_e4m3fn)
    vd = torch.from_numpy(vq).to(dev).view(torch.float8_e4m3fn)
    ksd, vsd = torch.from_numpy(ks).to(dev), torch.from_numpy(vs).to(dev)
    # decode: one q row per sequence over the whole context (q already scaled, as the caller does)
    qd = ora.f32_to_bf16(rng.standard_normal((batch, h, 128)).astype(np.float32) * 0.5 * 0.125)
    out = pkg.decode_paged_attention(from_u16(qd, dev), kd.permute(2, 0, 1, 3), vd.permute(2, 0, 1, 3), i32(bt),
                                     i32(kvl), k_scales_pages=ksd, v_scales_pages=vsd)
    # prefill: the new rows after their cached prefixes
    cu = np.concatenate([[0], np.cumsum(new)]).astype(np.int32)
    cuk = np.concatenate([[0], np.cumsum(kvl)]).astype(np.int32)
    pos = np.concatenate([np.arange(p, p + n) for p, n in zip(prefix, new)]).astype(np.int32)
    qp = ora.f32_to_bf16(rng.standard_normal((int(cu[-1]), h, 128)).astype(np.float32) * 0.5)
    outp = pkg.prefill_paged_attention(from_u16(qp, dev), kd.permute(2, 0, 1, 3), vd.permute(2, 0, 1, 3), i32(bt),
                                       i32(cu), None, i32(pos), max_seqlen_bucket=int(new.max()),
                                       cu_seqlens_k=i32(cuk), k_scales_pages=ksd, v_scales_pages=vsd)
    torch.cuda.synchronize()
    kqt, vqt = kq.transpose(2, 0, 1, 3), vq.transpose(2, 0, 1, 3)
    want_d = ora.decode_attention(qd, kqt, vqt, bt, kvl, k_scales_pages=ks, v_scales_pages=vs)
    want_p = ora.prefill_attention(qp, kqt, vqt, bt, cu, pos, cu_seqlens_k=cuk, k_scales_pages=ks,
                                   v_scales_pages=vs)
    err_d = float(np.abs(ora.bf16_to_f32(u16(out)) - ora.bf16_to_f32(want_d)).max())
    err_p = float(np.abs(ora.bf16_to_f32(u16(outp)) - ora.bf16_to_f32(want_p)).max())
    print(f"  max-abs err decode {err_d:.3e} prefill {err_p:.3e}")
    assert err_d <= TOL and err_p <= TOL


ANY_DIMS = [d for d in range(16, 257, 16) if d != 128]


@pytest.mark.parametrize("seed", _seeds(12))
def test_head_dim_sweep(pkg, dev, seed):
    """Head sizes other than 128 (the generic kernels): each seed draws the
    size from the multiples of 16 up to 256, the entry (prefill, decode or
    the mixed launch, in turn) and a shape as the sweeps above."""
    from test_gpu_decode import _run_and_check
    from test_gpu_mixed import _case, _run
    from test_gpu_prefill import _prefill
    rng = np.random.default_rng(4000 + seed)
    d = int(rng.choice(ANY_DIMS))
    kind = ("prefill", "decode", "mixed")[seed % 3]
    h, hkv = _heads(rng)
    bs = int(rng.choice(PAGE_SIZES))
    cap = 6.0 if rng.random() < 0.25 else None
    print(f"head-dim sweep seed {seed}: {kind} d {d} H {h} Hkv {hkv} page {bs} cap {cap}", flush=True)
    if kind == "prefill":
        batch = int(rng.integers(1, 9))
        new = rng.integers(1, 300, batch).tolist()
        prefix = np.where(rng.random(batch) < 0.5, rng.integers(0, 500, batch), 0).tolist()
        pb = wl.make_prefix_prefill(prefix, new, num_heads=h, num_kv_heads=hkv, page_size=bs, head_dim=d,
                                    rng=np.random.default_rng(seed))
        _prefill(pkg, dev, pb, seed, soft_cap=cap, use_seam=cap is None)
    elif kind == "decode":
        lens = rng.integers(0, 4000, int(rng.integers(1, 13))).tolist()
        width = 1 << (max(max(-(-n // bs) for n in lens), 1) - 1).bit_length()
        db = wl.make_decode(lens, num_heads=h, num_kv_heads=hkv, page_size=bs, head_dim=d,
                            rng=np.random.default_rng(seed), table_width=width)
        _run_and_check(pkg, dev, db, seed, soft_cap=cap)
    else:
        nd, npre = int(rng.integers(1, 6)), int(rng.integers(0, 4))
        dec = rng.integers(0, 3000, nd).tolist()
        pre_q = rng.integers(1, 200, npre).tolist()
        pre_p = np.where(rng.random(npre) < 0.5, rng.integers(0, 400, npre), 0).tolist()
        q, kc, vc, bt, cu, kv, pos = _case(rng, dec, pre_q, pre_p, h, hkv, bs, pad_rows=1, d=d)
        root = float(ora.round_bf16(np.float32(np.sqrt(d))).reshape(-1)[0])
        got = _run(pkg, dev, q, kc, vc, bt, cu, kv, pos, nd, max(pre_q) if pre_q else 0, soft_cap=cap,
                   decode_scale=1.0 / root)
        want = ora.mixed_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, cu, kv, pos, nd,
                                   soft_cap=cap)
        err = float(np.abs(ora.bf16_to_f32(got) - ora.bf16_to_f32(want)).max())
        print(f"  max-abs err {err:.3e}")
        assert err <= TOL
        zero = np.ones(q.shape[0], bool)
        zero[cu[:nd]] = False
        for b in range(nd, len(kv)):
            zero[cu[b]:cu[b + 1]] = False
        zero[cu[:nd][kv[:nd] == 0]] = True
        assert not got[zero].any()
