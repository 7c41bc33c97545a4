"""Writes the golden vectors under tests/golden/ from the CPU oracle.

Each fixture holds its inputs (bf16 as uint16 bit patterns, int32 metadata)
and the oracle's expected outputs, so GPU tests need neither the oracle's
generator nor a random stream that matches across devices.  The reference
itself cannot run here (no JAX); these vectors pin the oracle against
regressions and give the HIP path fixed known answers.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import paged_attention_oracle as ora  # noqa: E402


def _bf16(rng, shape, scale=0.5):
    return ora.f32_to_bf16(rng.standard_normal(shape).astype(np.float32) * scale)


def _tables(lens, bs, perm, width=None):
    pages = [-(-int(n) // bs) for n in lens]
    width = width or max(pages)
    bt = np.full((len(lens), width), -1, np.int32)
    c = 0
    for b, k in enumerate(pages):
        bt[b, :k] = perm[c:c + k]
        c += k
    return bt


def prefill_small():
    """Qwen3-0.6B heads (16 q / 8 kv), lengths [17, 40, 100], 4 x 256-token pages, engine padding."""
    rng = np.random.default_rng(100)
    h, hkv, bs, nb = 16, 8, 256, 4
    lens = [17, 40, 100]
    perm = rng.permutation(nb).astype(np.int32)
    bt = _tables(lens, bs, perm)
    bt = np.concatenate([bt, np.full((1, bt.shape[1]), -1, np.int32)])          # padded batch row
    cu = np.array([0, 17, 57, 157, 157], np.int32)
    pos = np.concatenate([np.arange(n) for n in lens] + [np.zeros(3, int)]).astype(np.int32)
    slots = np.concatenate([bt[b, np.arange(n) // bs] * bs + np.arange(n) % bs for b, n in enumerate(lens)]
                           + [np.full(3, -1)]).astype(np.int32)                 # 3 padding tokens
    t = len(slots)
    q, k, v = _bf16(rng, (t, h, 128)), _bf16(rng, (t, hkv, 128)), _bf16(rng, (t, hkv, 128))
    kc = np.zeros((nb, bs, hkv, 128), np.uint16)
    kc, vc = ora.kv_store(kc, kc.copy(), k, v, slots)
    out = ora.prefill_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, cu, pos)
    return dict(q=q, k=k, v=v, slot_mapping=slots, block_tables=bt, cu_seqlens_q=cu, cu_seqlens_k=cu,
                input_positions=pos, num_pages=np.int32(nb), page_size=np.int32(bs), max_seqlen_bucket=np.int32(128),
                pool_k=np.zeros(0, np.uint16), pool_v=np.zeros(0, np.uint16), out=out)


def prefix_small():
    """32 q / 8 kv heads, 16-token pages; cached prefixes [40, 17] followed by new chunks [20, 9]."""
    rng = np.random.default_rng(101)
    h, hkv, bs = 32, 8, 16
    prefix, new = np.array([40, 17]), np.array([20, 9])
    kvl = prefix + new
    nb = int(sum(-(-int(n) // bs) for n in kvl)) + 1
    perm = rng.permutation(nb).astype(np.int32)
    bt = _tables(kvl, bs, perm)
    pool_k, pool_v = _bf16(rng, (nb, bs, hkv, 128)), _bf16(rng, (nb, bs, hkv, 128))
    cu = np.concatenate([[0], np.cumsum(new)]).astype(np.int32)
    cuk = np.concatenate([[0], np.cumsum(kvl)]).astype(np.int32)
    pos = np.concatenate([np.arange(p, p + n) for p, n in zip(prefix, new)]).astype(np.int32)
    slots = np.concatenate([bt[b, np.arange(p, p + n) // bs] * bs + np.arange(p, p + n) % bs
                            for b, (p, n) in enumerate(zip(prefix, new))]).astype(np.int32)
    t = len(slots)
    q, k, v = _bf16(rng, (t, h, 128)), _bf16(rng, (t, hkv, 128)), _bf16(rng, (t, hkv, 128))
    kc, vc = ora.kv_store(pool_k, pool_v, k, v, slots)
    out = ora.prefill_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, cu, pos,
                                cu_seqlens_k=cuk)
    return dict(q=q, k=k, v=v, slot_mapping=slots, block_tables=bt, cu_seqlens_q=cu, cu_seqlens_k=cuk,
                input_positions=pos, num_pages=np.int32(nb), page_size=np.int32(bs),
                max_seqlen_bucket=np.int32(32), pool_k=pool_k, pool_v=pool_v, out=out)


def decode_small():
    """8 q / 2 kv heads, 16-token pages, contexts [1, 33, 300, 256, 0]; q pre-scaled as qwen3.py:207 does."""
    rng = np.random.default_rng(102)
    h, hkv, bs = 8, 2, 16
    lens = np.array([1, 33, 300, 256, 0], np.int32)
    nb = int(sum(-(-int(n) // bs) for n in lens)) + 1
    perm = rng.permutation(nb).astype(np.int32)
    bt = _tables(lens, bs, perm, width=32)
    pool_k, pool_v = _bf16(rng, (nb, bs, hkv, 128)), _bf16(rng, (nb, bs, hkv, 128))
    q = _bf16(rng, (len(lens), h, 128))
    q_scaled = ora.f32_to_bf16(ora.round_bf16(ora.bf16_to_f32(q) / np.float32(11.3125)))
    out = ora.decode_attention(q_scaled, pool_k.transpose(2, 0, 1, 3), pool_v.transpose(2, 0, 1, 3), bt, lens)
    return dict(q_scaled=q_scaled, block_tables=bt, lengths=lens, num_pages=np.int32(nb), page_size=np.int32(bs),
                pool_k=pool_k, pool_v=pool_v, out=out)


FIXTURES = {"prefill_small": prefill_small, "prefix_small": prefix_small, "decode_small": decode_small}


def main():
    for name, fn in FIXTURES.items():
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **fn())
        print(path, os.path.getsize(path))


if __name__ == "__main__":
    main()
