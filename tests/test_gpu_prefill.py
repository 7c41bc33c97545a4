"""Ragged causal GQA paged prefill on gfx950 against the oracle (max-abs <= 2e-2)."""
from __future__ import annotations

import numpy as np
import pytest

import vllm_jax_amd.workloads as wl
from conftest import u16
from oracle import paged_attention_oracle as ora

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _prefill(pkg, dev, pb, seed, *, rows=None, soft_cap=None, use_seam=True):
    """KV store + prefill on the GPU; the oracle replays both on the host."""
    import torch
    t = wl.materialize_prefill(pb, seed, dev)
    before = u16(t["kv_cache"])
    if use_seam:
        meta = pkg.PrefillAttentionMetadata(t["input_positions"], t["slot_mapping"], t["block_tables"],
                                            t["cu_seqlens_q"], t["cu_seqlens_k"], None, None,
                                            pb.max_seqlen_bucket)
        kv, out = pkg.attention(t["kv_cache"], t["q"], t["k"], t["v"], meta)
    else:
        kv = pkg.update_kv_cache(t["kv_cache"], t["slot_mapping"], t["k"], t["v"])
        out = pkg.prefill_paged_attention(
            t["q"], kv[0].permute(2, 0, 1, 3), kv[1].permute(2, 0, 1, 3), t["block_tables"],
            t["cu_seqlens_q"], t["slot_mapping"], t["input_positions"],
            max_seqlen_bucket=pb.max_seqlen_bucket, cu_seqlens_k=t["cu_seqlens_k"],
            attn_logits_soft_cap=soft_cap)
    torch.cuda.synchronize()
    kc, vc = ora.kv_store(before[0], before[1], u16(t["k"]), u16(t["v"]), pb.slot_mapping)
    assert np.array_equal(u16(kv[0]), kc), "kv store (K) not bit-exact"
    assert np.array_equal(u16(kv[1]), vc), "kv store (V) not bit-exact"
    ref = ora.prefill_attention(u16(t["q"]), kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3),
                                pb.block_tables, pb.cu_seqlens_q, pb.input_positions,
                                cu_seqlens_k=pb.cu_seqlens_k, soft_cap=soft_cap, rows=rows)
    got = ora.bf16_to_f32(u16(out))
    want = ora.bf16_to_f32(ref)
    sel = slice(None) if rows is None else np.asarray(rows)
    err = float(np.abs(got[sel] - want[sel]).max())
    print(f"prefill max-abs err {err:.3e} over {got[sel].shape[0]} rows")
    assert err <= TOL, err
    assert np.isfinite(got).all()
    return got, t


def test_prefill_qwen3_06b_config(pkg, dev):
    """The CPU-runnable reference case: lengths [17,128,300,511], 16q/8kv, 64 x 256-token pool, seed 0."""
    _prefill(pkg, dev, wl.qwen3_06b_prefill(), seed=0)


@pytest.mark.parametrize("lens,h,hkv,bs", [
    ([1, 2, 3, 64, 65, 130], 8, 2, 16),        # tiny sequences, small pages
    ([200, 37], 32, 8, 256),                   # G = 4
    ([150, 300], 64, 8, 256),                  # G = 8 (Qwen3-32B heads)
    ([100, 33], 8, 8, 32),                     # MHA
    ([257, 40], 16, 1, 64),                    # G = 16
    ([129], 4, 4, 256),
])
def test_prefill_shapes(pkg, dev, lens, h, hkv, bs):
    pb = wl.make_prefill(lens, num_heads=h, num_kv_heads=hkv, page_size=bs,
                         rng=np.random.default_rng(sum(lens)))
    _prefill(pkg, dev, pb, seed=1)


def test_prefill_engine_padding(pkg, dev):
    """Engine layout: tokens padded to a power of two (slot -1), batch padded with repeated cu_seqlens."""
    pb = wl.make_prefill([100, 23, 7], num_heads=16, num_kv_heads=8, page_size=16, num_pages=20,
                         rng=np.random.default_rng(3), pad_tokens_to=256, pad_batch_to=4)
    got, _ = _prefill(pkg, dev, pb, seed=3)
    assert not got[130:].any()


def test_prefill_soft_cap_kernel_entry(pkg, dev):
    pb = wl.make_prefill([90, 300], num_heads=16, num_kv_heads=8, page_size=256, rng=np.random.default_rng(4))
    _prefill(pkg, dev, pb, seed=4, soft_cap=8.0, use_seam=False)


def test_prefill_prefix_cached_small(pkg, dev):
    """Cached prefixes in shared blocks (copy-on-write tail) followed by new chunks."""
    pb = wl.make_prefix_prefill([0, 300, 512, 40], [130, 64, 200, 1], num_heads=32, num_kv_heads=8,
                                rng=np.random.default_rng(5), shared_prefix_tokens=600)
    assert pb.refcounts.max() >= 2
    _prefill(pkg, dev, pb, seed=5)


def test_prefill_qwen3_8b_prefix_workload(pkg, dev):
    """Full Qwen3-8B prefix-cached workload; oracle on sampled rows (incl. every sequence's last row)."""
    pb = wl.qwen3_8b_prefix_prefill()
    rng = np.random.default_rng(0)
    rows = np.unique(np.concatenate([pb.cu_seqlens_q[1:] - 1, rng.integers(0, pb.num_tokens, 32)]))
    _prefill(pkg, dev, pb, seed=3, rows=rows)


def test_prefill_qwen3_06b_mixed_prefill_half(pkg, dev):
    pre, _ = wl.qwen3_06b_mixed()
    rng = np.random.default_rng(1)
    rows = np.unique(np.concatenate([pre.cu_seqlens_q[1:] - 1, pre.cu_seqlens_q[:-1], rng.integers(0, pre.num_tokens, 64)]))
    _prefill(pkg, dev, pre, seed=1, rows=rows)


def test_prefill_qwen3_32b_long(pkg, dev):
    """Full Qwen3-32B long-context workload (8 seqs of 8k-32k tokens).

    Oracle on sampled rows of two sequences, plus a full-size property: the
    last row of every sequence must equal a decode over that sequence's
    whole context with the same q (both on the GPU).
    """
    import torch
    pb = wl.qwen3_32b_long_prefill()
    cu = pb.cu_seqlens_q
    b_small = int(np.argmin(pb.q_lens))
    rows = np.array([cu[b_small], cu[b_small] + 1, cu[b_small] + 700, cu[b_small + 1] - 1, cu[1] - 1])
    got, t = _prefill(pkg, dev, pb, seed=4, rows=rows)
    kv = t["kv_cache"]
    last = torch.as_tensor(cu[1:] - 1, dtype=torch.long, device=dev)
    lens = torch.as_tensor(pb.q_lens.astype(np.int32), device=dev)
    dec = pkg.decode_paged_attention(t["q"][last], kv[0].permute(2, 0, 1, 3), kv[1].permute(2, 0, 1, 3),
                                     t["block_tables"], lens, scale=0.08837890625)
    torch.cuda.synchronize()
    diff = float(np.abs(ora.bf16_to_f32(u16(dec)) - got[cu[1:] - 1]).max())
    print(f"prefill last rows vs decode max-abs diff {diff:.3e}")
    assert diff <= TOL


def test_prefill_many_sequences(pkg, dev):
    """A batch of 70 short ragged sequences (most q tiles of the launch grid
    fall outside their sequence)."""
    rng = np.random.default_rng(22)
    lens = rng.integers(1, 200, 70).tolist()
    pb = wl.make_prefill(lens, num_heads=16, num_kv_heads=8, page_size=64, rng=rng)
    rows = np.unique(np.concatenate([pb.cu_seqlens_q[1:] - 1, rng.integers(0, pb.num_tokens, 64)]))
    _prefill(pkg, dev, pb, seed=22, rows=rows)
