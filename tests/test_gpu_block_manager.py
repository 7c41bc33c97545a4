"""Block tables from the native block manager driving the gfx950 kernels:
copy-on-write page copies (bit-exact), a prefix-cached prefill and a forked
decode, each against the oracle over the sequence's full context."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import from_u16, u16
from oracle import paged_attention_oracle as ora

pytestmark = pytest.mark.gpu
TOL = 2e-2
KV = __import__("vllm_jax_amd.kv_cache_manager", fromlist=["KVCacheManager"])


class Req:
    def __init__(self, token_ids, rid):
        self.token_ids, self.id = list(token_ids), rid

    def __len__(self):
        return len(self.token_ids)


def _bf16(rng, shape):
    return ora.f32_to_bf16(rng.standard_normal(shape).astype(np.float32) * 0.5)


def test_copy_blocks_bit_exact(pkg, dev):
    import torch
    rng = np.random.default_rng(0)
    nb, bs, hkv = 12, 64, 4
    pool = _bf16(rng, (2, nb, bs, hkv, 128))
    cache = from_u16(pool, dev)
    src, dst = [3, 7, 0, 11], [5, 1, 9, 2]
    KV.copy_blocks(cache, src, dst)
    torch.cuda.synchronize()
    want = pool.copy()
    want[:, dst] = pool[:, src]
    assert np.array_equal(u16(cache), want)


def _slots(table, positions, bs):
    return np.asarray([table[p // bs] * bs + p % bs for p in positions], np.int32)


def test_prefix_cached_prefill_matches_full_context(pkg, dev):
    """Request B shares a 600-token prefix with A; with prefix caching it
    computes only its tokens after the cached blocks."""
    import torch
    rng = np.random.default_rng(1)
    bs, nb, h, hkv = 256, 16, 16, 8
    m = KV.KVCacheManager(nb, bs, enable_prefix_caching=True)
    prefix = list(rng.integers(0, 50000, 600))
    a = Req(prefix + list(rng.integers(0, 50000, 100)), 1)
    b = Req(prefix + list(rng.integers(0, 50000, 150)), 2)
    # K/V of a token depend on the token sequence up to it: equal prefixes give equal K/V
    kv_a = _bf16(rng, (2, len(a), hkv, 128))
    kv_b = np.concatenate([kv_a[:, :600], _bf16(rng, (2, 150, hkv, 128))], axis=1)
    cache = torch.zeros((2, nb, bs, hkv, 128), dtype=torch.bfloat16, device=dev)
    i32 = lambda x: torch.as_tensor(np.ascontiguousarray(x, dtype=np.int32), device=dev)

    def step(req, kvs):
        m.allocate_slots(req, True)
        cached = m.num_cached_tokens(req)
        table = m.block_ids(req)
        n = len(req)
        new = np.arange(cached, n)
        pkg.update_kv_cache(cache, i32(_slots(table, new, bs)), from_u16(kvs[0, cached:], dev),
                            from_u16(kvs[1, cached:], dev))
        q = _bf16(rng, (len(new), h, 128))
        bt = np.asarray([table], np.int32)
        cu_q, cu_k = np.array([0, len(new)], np.int32), np.array([0, n], np.int32)
        out = pkg.prefill_paged_attention(from_u16(q, dev), cache[0].permute(2, 0, 1, 3), cache[1].permute(2, 0, 1, 3),
                                          i32(bt), i32(cu_q), None, i32(new), max_seqlen_bucket=1024,
                                          cu_seqlens_k=i32(cu_k))
        torch.cuda.synchronize()
        # oracle over the full context held in dense form
        kc = np.zeros((1, bs, hkv, 128), np.uint16).repeat(len(table), 0)
        vc = kc.copy()
        for p in range(n):
            kc[p // bs, p % bs], vc[p // bs, p % bs] = kvs[0, p], kvs[1, p]
        want = ora.prefill_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3),
                                     np.arange(len(table), dtype=np.int32)[None], cu_q, new, cu_seqlens_k=cu_k)
        return cached, u16(out), want

    ca, got_a, want_a = step(a, kv_a)
    cb, got_b, want_b = step(b, kv_b)
    assert ca == 0 and cb == 512
    assert m.block_ids(b)[:2] == m.block_ids(a)[:2]
    for got, want in ((got_a, want_a), (got_b, want_b)):
        assert np.abs(ora.bf16_to_f32(got) - ora.bf16_to_f32(want)).max() <= TOL


def test_forked_decode_copies_on_write(pkg, dev):
    import torch
    rng = np.random.default_rng(2)
    bs, nb, h, hkv = 16, 8, 8, 2
    m = KV.KVCacheManager(nb, bs)
    parent = Req(range(20), 1)
    m.allocate_slots(parent, True)
    cache = torch.zeros((2, nb, bs, hkv, 128), dtype=torch.bfloat16, device=dev)
    i32 = lambda x: torch.as_tensor(np.ascontiguousarray(x, dtype=np.int32), device=dev)
    kv_p = _bf16(rng, (2, 21, hkv, 128))
    pkg.update_kv_cache(cache, i32(_slots(m.block_ids(parent), range(20), bs)), from_u16(kv_p[0, :20], dev),
                        from_u16(kv_p[1, :20], dev))
    child = Req(range(20), 2)
    m.fork(parent, child)
    kv_c = _bf16(rng, (2, 1, hkv, 128))
    for req, kv_new in ((child, kv_c[:, 0]), (parent, kv_p[:, 20])):
        req.token_ids.append(0)
        m.allocate_slots(req, False)
        src, dst = m.take_block_copies()
        KV.copy_blocks(cache, src, dst)
        pkg.update_kv_cache(cache, i32(_slots(m.block_ids(req), [20], bs)), from_u16(kv_new[0][None], dev),
                            from_u16(kv_new[1][None], dev))
    assert m.block_ids(child)[1] != m.block_ids(parent)[1]
    q = _bf16(rng, (2, h, 128))
    bt = np.asarray([m.block_ids(parent), m.block_ids(child)], np.int32)
    lens = np.array([21, 21], np.int32)
    out = pkg.decode_paged_attention(from_u16(q, dev), cache[0].permute(2, 0, 1, 3), cache[1].permute(2, 0, 1, 3),
                                     i32(bt), i32(lens))
    torch.cuda.synchronize()
    ctx_p = kv_p
    ctx_c = np.concatenate([kv_p[:, :20], kv_c], axis=1)
    for i, ctx in enumerate((ctx_p, ctx_c)):
        kc = np.zeros((2, bs, hkv, 128), np.uint16)
        vc = kc.copy()
        for p in range(21):
            kc[p // bs, p % bs], vc[p // bs, p % bs] = ctx[0, p], ctx[1, p]
        want = ora.decode_attention(q[i:i + 1], kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3),
                                    np.array([[0, 1]], np.int32), lens[:1])
        err = np.abs(ora.bf16_to_f32(u16(out)[i]) - ora.bf16_to_f32(want[0])).max()
        assert err <= TOL, (i, err)
