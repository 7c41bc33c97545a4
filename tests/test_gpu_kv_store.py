"""KV store and block-table gather on gfx950: bit-exact against the oracle."""
from __future__ import annotations

import numpy as np
import pytest

import vllm_jax_amd.workloads as wl
from conftest import u16
from oracle import paged_attention_oracle as ora

pytestmark = pytest.mark.gpu


def _pool(torch, shape, seed, dev):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    return (torch.randn(shape, generator=g, device=dev) * 0.5).to(torch.bfloat16)


@pytest.mark.parametrize("nb,bs,hkv,t,seed", [
    (64, 256, 8, 956, 0),       # qwen3-0.6B prefill shape
    (16, 16, 2, 100, 1),        # small pages (the reference's test.py uses 16)
    (8, 256, 8, 1, 2),          # single token
    (4, 32, 4, 0, 3),           # empty batch
])
def test_kv_store_bit_exact(pkg, dev, nb, bs, hkv, t, seed):
    import torch
    rng = np.random.default_rng(seed)
    cache = _pool(torch, (2, nb, bs, hkv, 128), seed, dev)
    before = cache.cpu()
    k = _pool(torch, (t, hkv, 128), seed + 100, dev)
    v = _pool(torch, (t, hkv, 128), seed + 200, dev)
    slots = rng.permutation(nb * bs)[:t].astype(np.int32)
    if t > 4:
        slots[::7] = -1                      # padding tokens
    sm = torch.as_tensor(slots, device=dev)
    pkg.update_kv_cache(cache, sm, k, v)
    torch.cuda.synchronize()
    kc, vc = ora.kv_store(u16(before[0]), u16(before[1]), u16(k), u16(v), slots)
    assert np.array_equal(u16(cache[0]), kc)
    assert np.array_equal(u16(cache[1]), vc)


def test_kv_store_strided_inputs_and_out_of_range_slots(pkg, dev):
    """k/v as non-contiguous views of a fused qkv buffer; slots past the pool are dropped."""
    import torch
    nb, bs, hkv, t = 8, 64, 4, 50
    cache = _pool(torch, (2, nb, bs, hkv, 128), 5, dev)
    before = cache.cpu()
    qkv = _pool(torch, (t, 3 * hkv, 128), 6, dev)
    k, v = qkv[:, hkv:2 * hkv], qkv[:, 2 * hkv:]
    slots = np.random.default_rng(7).permutation(nb * bs)[:t].astype(np.int32)
    slots[3] = nb * bs + 5
    slots[9] = -1
    pkg.update_kv_cache(cache, torch.as_tensor(slots, device=dev), k, v)
    torch.cuda.synchronize()
    kc, vc = ora.kv_store(u16(before[0]), u16(before[1]), u16(k), u16(v), slots)
    assert np.array_equal(u16(cache[0]), kc)
    assert np.array_equal(u16(cache[1]), vc)


def test_kv_store_full_size_roundtrip(pkg, dev):
    """Qwen3-32B long prefill size (~164k tokens): store then gather is the identity."""
    import torch
    pb = wl.qwen3_32b_long_prefill()
    nb, bs = pb.num_pages, pb.page_size
    cache = torch.zeros((2, nb, bs, 8, 128), dtype=torch.bfloat16, device=dev)
    t = pb.num_tokens
    k = _pool(torch, (t, 8, 128), 11, dev)
    v = _pool(torch, (t, 8, 128), 12, dev)
    pkg.update_kv_cache(cache, torch.as_tensor(pb.slot_mapping, device=dev), k, v)
    bt = torch.as_tensor(pb.block_tables, device=dev)
    lens = torch.as_tensor(np.diff(pb.cu_seqlens_q).astype(np.int32), device=dev)
    for cache_i, src in ((cache[0], k), (cache[1], v)):
        ctx = pkg.gather_kv(cache_i, bt, lens)
        for b in range(pb.batch):
            q0, q1 = int(pb.cu_seqlens_q[b]), int(pb.cu_seqlens_q[b + 1])
            assert torch.equal(ctx[b, :q1 - q0], src[q0:q1])
            assert not ctx[b, q1 - q0:].any()


def test_gather_bit_exact(pkg, dev):
    import torch
    rng = np.random.default_rng(9)
    nb, bs, hkv = 32, 16, 2
    cache = _pool(torch, (nb, bs, hkv, 128), 9, dev)
    lens = np.array([0, 1, 16, 17, 100, 5], np.int32)
    p = 8
    bt = np.full((len(lens), p), -1, np.int32)
    perm = rng.permutation(nb)
    c = 0
    for b, n in enumerate(lens):
        k = -(-int(n) // bs)
        bt[b, :k] = perm[c:c + k]
        c += k
    out = pkg.gather_kv(cache, torch.as_tensor(bt, device=dev), torch.as_tensor(lens, device=dev))
    torch.cuda.synchronize()
    assert np.array_equal(u16(out), ora.gather_kv(u16(cache), bt, lens))


def test_kv_store_duplicate_slot_check(pkg, dev, monkeypatch):
    """With PA_CHECK_SLOTS=1 the stores refuse a slot mapping that writes one
    slot twice, before any device write; without it the store runs (the
    winner of the duplicated slot is unspecified, as in the reference)."""
    import torch
    cache = torch.zeros((2, 4, 16, 2, 128), dtype=torch.bfloat16, device=dev)
    k = torch.ones((3, 2, 128), dtype=torch.bfloat16, device=dev)
    v = torch.ones_like(k)
    sm = torch.tensor([5, 9, 5], dtype=torch.int32, device=dev)
    monkeypatch.setenv("PA_CHECK_SLOTS", "1")
    with pytest.raises(ValueError, match="slot 5 from tokens"):
        pkg.update_kv_cache(cache, sm, k, v)
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(cache)) == 0
    pkg.update_kv_cache(cache, torch.tensor([5, 9, 6], dtype=torch.int32, device=dev), k, v)
    monkeypatch.delenv("PA_CHECK_SLOTS")
    pkg.update_kv_cache(cache, sm, k, v)
    torch.cuda.synchronize()
