"""Golden vectors (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle still reproduces every stored answer.
GPU: the HIP path matches them -- KV store bit-exact, attention within 2e-2.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

from conftest import ROOT, from_u16, u16
from oracle import paged_attention_oracle as ora

GOLDEN = os.path.join(ROOT, "tests", "golden")
TOL = 2e-2


def _load(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _pool(f, nb, bs, hkv):
    if f["pool_k"].size:
        return f["pool_k"], f["pool_v"]
    z = np.zeros((nb, bs, hkv, 128), np.uint16)
    return z, z.copy()


@pytest.mark.parametrize("name", ["prefill_small", "prefix_small"])
def test_oracle_reproduces_prefill_golden(name):
    f = _load(name)
    nb, bs, hkv = int(f["num_pages"]), int(f["page_size"]), f["k"].shape[1]
    kc, vc = _pool(f, nb, bs, hkv)
    kc, vc = ora.kv_store(kc, vc, f["k"], f["v"], f["slot_mapping"])
    out = ora.prefill_attention(f["q"], kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), f["block_tables"],
                                f["cu_seqlens_q"], f["input_positions"], cu_seqlens_k=f["cu_seqlens_k"])
    # identical up to BLAS summation order (at most one bf16 step on rare elements)
    d = np.abs(ora.bf16_to_f32(out) - ora.bf16_to_f32(f["out"]))
    assert d.max() <= 8e-3 and (d > 0).mean() < 1e-3


def test_oracle_reproduces_decode_golden():
    f = _load("decode_small")
    out = ora.decode_attention(f["q_scaled"], f["pool_k"].transpose(2, 0, 1, 3), f["pool_v"].transpose(2, 0, 1, 3),
                               f["block_tables"], f["lengths"])
    d = np.abs(ora.bf16_to_f32(out) - ora.bf16_to_f32(f["out"]))
    assert d.max() <= 8e-3 and (d > 0).mean() < 1e-3


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["prefill_small", "prefix_small"])
def test_gpu_matches_prefill_golden(pkg, dev, name):
    import torch
    f = _load(name)
    nb, bs, hkv = int(f["num_pages"]), int(f["page_size"]), f["k"].shape[1]
    kc, vc = _pool(f, nb, bs, hkv)
    kv = torch.stack([from_u16(kc, dev), from_u16(vc, dev)])
    i32 = lambda a: torch.as_tensor(a, dtype=torch.int32, device=dev)
    meta = pkg.PrefillAttentionMetadata(i32(f["input_positions"]), i32(f["slot_mapping"]), i32(f["block_tables"]),
                                        i32(f["cu_seqlens_q"]), i32(f["cu_seqlens_k"]), None, None,
                                        int(f["max_seqlen_bucket"]))
    kv, out = pkg.attention(kv, from_u16(f["q"], dev), from_u16(f["k"], dev), from_u16(f["v"], dev), meta)
    torch.cuda.synchronize()
    kce, vce = ora.kv_store(kc, vc, f["k"], f["v"], f["slot_mapping"])
    assert np.array_equal(u16(kv[0]), kce) and np.array_equal(u16(kv[1]), vce)
    err = np.abs(ora.bf16_to_f32(u16(out)) - ora.bf16_to_f32(f["out"])).max()
    print(f"{name}: max-abs err vs golden {err:.3e}")
    assert err <= TOL


@pytest.mark.gpu
def test_gpu_matches_decode_golden(pkg, dev):
    import torch
    f = _load("decode_small")
    kp = from_u16(f["pool_k"], dev).permute(2, 0, 1, 3)
    vp = from_u16(f["pool_v"], dev).permute(2, 0, 1, 3)
    i32 = lambda a: torch.as_tensor(a, dtype=torch.int32, device=dev)
    out = pkg.decode_paged_attention(from_u16(f["q_scaled"], dev), kp, vp, i32(f["block_tables"]), i32(f["lengths"]))
    torch.cuda.synchronize()
    got = ora.bf16_to_f32(u16(out))
    err = np.abs(got - ora.bf16_to_f32(f["out"])).max()
    print(f"decode_small: max-abs err vs golden {err:.3e}")
    assert err <= TOL
    assert not got[4].any()
