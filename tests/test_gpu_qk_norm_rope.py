"""Fused q/k RMSNorm + RoPE + KV store on gfx950 against the oracle.

Tolerance: the kernel and the oracle both round the normalised row and the
rotated row to bf16, but their float32 sums, sqrt and cos/sin differ in the
last bits, so an element may land one bf16 step away.  The test requires
|got - want| <= 2**-7 * max(1, |want|) + 2**-8 (about two bf16 steps of an
O(1) value) for every element and bit-exact equality for at least 97% of
them; V and the untouched slots are compared bit-exact.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import from_u16, u16
from oracle import paged_attention_oracle as ora

pytestmark = pytest.mark.gpu


def _close(got_u16, want_u16):
    got = ora.bf16_to_f32(got_u16).astype(np.float64)
    want = ora.bf16_to_f32(want_u16).astype(np.float64)
    err = np.abs(got - want)
    bound = 2.0 ** -7 * np.maximum(1.0, np.abs(want)) + 2.0 ** -8
    assert np.all(np.isfinite(got))
    assert np.all(err <= bound), f"max err {err.max()} at {np.unravel_index(err.argmax(), err.shape)}"
    exact = np.mean(got_u16 == want_u16)
    assert exact >= 0.97, f"only {exact:.4f} of the elements are bit-exact"


def _bf16(rng, shape, scale=1.0):
    return ora.f32_to_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


@pytest.mark.parametrize("t,h,hkv,nb,bs,scaling,seed", [
    (956, 16, 8, 8, 256, None, 0),                              # Qwen3-0.6B prefill shape
    (37, 32, 8, 4, 16, None, 1),                                # 8B heads, small pages
    (1, 16, 8, 2, 256, None, 2),                                # one decode token
    (200, 8, 2, 4, 64, {"type": "linear", "factor": 4.0}, 3),   # linear rope scaling
])
def test_qk_norm_rope_store_matches_oracle(pkg, dev, t, h, hkv, nb, bs, scaling, seed):
    import torch
    rng = np.random.default_rng(seed)
    d = 128
    q, k, v = _bf16(rng, (t, h, d), 2.0), _bf16(rng, (t, hkv, d), 2.0), _bf16(rng, (t, hkv, d))
    qw = ora.f32_to_bf16(rng.uniform(0.5, 1.5, d).astype(np.float32))
    kw = ora.f32_to_bf16(rng.uniform(0.5, 1.5, d).astype(np.float32))
    pos = rng.integers(0, 40960, t).astype(np.int32)
    pos[: min(t, 4)] = np.arange(min(t, 4))             # includes position 0
    slots = rng.permutation(nb * bs)[:t].astype(np.int32)
    if t > 8:
        slots[::9] = -1                                  # padding tokens
        slots[5] = nb * bs + 3                           # past the pool: dropped
    kc0, vc0 = _bf16(rng, (nb, bs, hkv, d)), _bf16(rng, (nb, bs, hkv, d))
    q_want, kc_want, vc_want = ora.qk_norm_rope_store(q, k, v, qw, kw, pos, slots, kc0, vc0, eps=1e-6,
                                                      rope_theta=1e6, rope_scaling=scaling)

    cache = torch.stack([from_u16(kc0, dev), from_u16(vc0, dev)])
    q_out, cache2 = pkg.qk_norm_rope_store(
        from_u16(q, dev), from_u16(k, dev), from_u16(v, dev), from_u16(qw, dev), from_u16(kw, dev),
        torch.as_tensor(pos, device=dev), torch.as_tensor(slots, device=dev), cache,
        eps=1e-6, rope_theta=1e6, rope_scaling=scaling)
    torch.cuda.synchronize()
    assert cache2 is cache
    _close(u16(q_out), q_want)
    got_k = u16(cache[0])
    _close(got_k, kc_want)
    assert np.array_equal(u16(cache[1]), vc_want)
    # slots nobody wrote keep their bits
    flat = np.setdiff1d(np.arange(nb * bs), slots[(slots >= 0) & (slots < nb * bs)])
    assert np.array_equal(got_k.reshape(nb * bs, hkv, d)[flat], kc0.reshape(nb * bs, hkv, d)[flat])


def test_qk_norm_rope_store_strided_qkv_and_in_place(pkg, dev):
    """q/k/v as views of one fused projection buffer; q rotated in place."""
    import torch
    rng = np.random.default_rng(11)
    t, h, hkv, nb, bs, d = 70, 16, 8, 4, 32, 128
    qkv = _bf16(rng, (t, h + 2 * hkv, d), 1.5)
    q, k, v = qkv[:, :h], qkv[:, h:h + hkv], qkv[:, h + hkv:]
    qw = ora.f32_to_bf16(rng.uniform(0.5, 1.5, d).astype(np.float32))
    kw = ora.f32_to_bf16(rng.uniform(0.5, 1.5, d).astype(np.float32))
    pos = np.arange(t, dtype=np.int32) + 1000
    slots = np.arange(t, dtype=np.int32) * 3 % (nb * bs)
    kc0, vc0 = _bf16(rng, (nb, bs, hkv, d)), _bf16(rng, (nb, bs, hkv, d))
    q_want, kc_want, vc_want = ora.qk_norm_rope_store(np.ascontiguousarray(q), np.ascontiguousarray(k),
                                                      np.ascontiguousarray(v), qw, kw, pos, slots, kc0, vc0,
                                                      eps=1e-6, rope_theta=1e6)
    g = from_u16(qkv, dev)
    gq, gk, gv = g[:, :h], g[:, h:h + hkv], g[:, h + hkv:]
    cache = torch.stack([from_u16(kc0, dev), from_u16(vc0, dev)])
    q_out, _ = pkg.qk_norm_rope_store(gq, gk, gv, from_u16(qw, dev), from_u16(kw, dev),
                                      torch.as_tensor(pos, device=dev), torch.as_tensor(slots, device=dev),
                                      cache, eps=1e-6, rope_theta=1e6, out=gq)
    torch.cuda.synchronize()
    assert q_out.data_ptr() == gq.data_ptr()
    _close(u16(gq), q_want)
    _close(u16(cache[0]), kc_want)
    assert np.array_equal(u16(cache[1]), vc_want)
    assert np.array_equal(u16(gv), np.ascontiguousarray(v))   # v is read, never written


def test_qwen3_attention_core_matches_separate_steps(pkg, dev):
    """Fused step + attention equals the oracle's rope/norm followed by attention."""
    import torch
    rng = np.random.default_rng(21)
    lens = [300, 5, 129]
    h, hkv, d, bs = 16, 8, 128, 64
    t = sum(lens)
    pages = [(n + bs - 1) // bs for n in lens]
    nb = sum(pages) + 1
    width = max(pages)
    bt = np.zeros((len(lens), width), np.int32)
    perm = rng.permutation(nb)
    c = 0
    for b, p in enumerate(pages):
        bt[b, :p] = perm[c:c + p]
        c += p
    slots = np.concatenate([bt[b, np.arange(n) // bs] * bs + np.arange(n) % bs for b, n in enumerate(lens)])
    slots = slots.astype(np.int32)
    pos = np.concatenate([np.arange(n) for n in lens]).astype(np.int32)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    q, k, v = _bf16(rng, (t, h, d)), _bf16(rng, (t, hkv, d)), _bf16(rng, (t, hkv, d))
    qw = ora.f32_to_bf16(rng.uniform(0.5, 1.5, d).astype(np.float32))
    kw = ora.f32_to_bf16(rng.uniform(0.5, 1.5, d).astype(np.float32))
    kc0 = np.zeros((nb, bs, hkv, d), np.uint16)
    q_rot, kc, vc = ora.qk_norm_rope_store(q, k, v, qw, kw, pos, slots, kc0, kc0.copy(), eps=1e-6,
                                           rope_theta=1e6)
    want = ora.prefill_attention(q_rot, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, cu, pos)

    cache = torch.zeros((2, nb, bs, hkv, d), dtype=torch.bfloat16, device=dev)
    meta = pkg.PrefillAttentionMetadata(torch.as_tensor(pos, device=dev), torch.as_tensor(slots, device=dev),
                                        torch.as_tensor(bt, device=dev), torch.as_tensor(cu, device=dev),
                                        torch.as_tensor(cu, device=dev), None, None, 512)
    cache, out = pkg.qwen3_attention_core(cache, from_u16(q, dev), from_u16(k, dev), from_u16(v, dev),
                                          from_u16(qw, dev), from_u16(kw, dev), meta, eps=1e-6, rope_theta=1e6)
    torch.cuda.synchronize()
    err = np.abs(ora.bf16_to_f32(u16(out)) - ora.bf16_to_f32(want)).max()
    assert err <= 2e-2, err


def test_qk_norm_rope_store_qwen3_32b_long_workload(pkg, dev):
    """The Qwen3-32B long-prefill step the bench times: 213 732 tokens of
    8 sequences (positions 0 .. L-1 each), 64 q / 8 kv heads, into its
    256-token-page pool.  Every q and k row of 384 sampled tokens (the first
    and last token of every sequence among them) against the oracle; V of
    every token and every slot no token writes, bit-exact, on the device."""
    import torch
    import vllm_jax_amd.workloads as wl
    pb = wl.qwen3_32b_long_prefill(seed=4)
    t = wl.materialize_prefill(pb, seed=4, device=dev, fill_pool=True)
    rng = np.random.default_rng(17)
    d, h, hkv = pb.head_dim, pb.num_heads, pb.num_kv_heads
    qw = ora.f32_to_bf16(rng.uniform(0.5, 1.5, d).astype(np.float32))
    kw = ora.f32_to_bf16(rng.uniform(0.5, 1.5, d).astype(np.float32))
    kv = t["kv_cache"]
    before = kv.clone()
    q_out, _ = pkg.qk_norm_rope_store(t["q"], t["k"], t["v"], from_u16(qw, dev), from_u16(kw, dev),
                                      t["input_positions"], t["slot_mapping"], kv, eps=1e-6, rope_theta=1e6)
    torch.cuda.synchronize()
    n_tok = pb.num_tokens
    slots = torch.as_tensor(pb.slot_mapping, dtype=torch.long, device=dev)
    flat_k, flat_v = kv[0].reshape(-1, hkv, d), kv[1].reshape(-1, hkv, d)
    assert torch.equal(flat_v[slots], t["v"]), "V rows not stored bit-exact"
    untouched = torch.ones(flat_k.shape[0], dtype=torch.bool, device=dev)
    untouched[slots] = False
    for i in range(2):
        assert torch.equal(kv[i].reshape(-1, hkv, d)[untouched], before[i].reshape(-1, hkv, d)[untouched]), \
            "a slot no token writes changed"
    cu = pb.cu_seqlens_q
    sel = np.unique(np.concatenate([cu[:-1], cu[1:] - 1, rng.integers(0, n_tok, 384 - 2 * pb.batch)]))
    print(f"qk norm + rope + store: {n_tok} tokens, {sel.size} sampled", flush=True)
    idx = torch.as_tensor(sel, dtype=torch.long, device=dev)
    q_s, k_s, v_s = u16(t["q"][idx]), u16(t["k"][idx]), u16(t["v"][idx])
    pos = pb.input_positions[sel].astype(np.int32)
    # the oracle's store into a compact cache of one slot per sampled token
    kc0 = np.zeros((sel.size, 1, hkv, d), np.uint16)
    q_want, kc_want, _ = ora.qk_norm_rope_store(q_s, k_s, v_s, qw, kw, pos, np.arange(sel.size, dtype=np.int32),
                                                kc0, kc0.copy(), eps=1e-6, rope_theta=1e6)
    _close(u16(q_out[idx]), q_want)
    _close(u16(flat_k[slots[idx]]), kc_want.reshape(sel.size, hkv, d))
