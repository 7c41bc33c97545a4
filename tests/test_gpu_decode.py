"""Split-K paged decode on gfx950 against the oracle (max-abs <= 2e-2, bf16)."""
from __future__ import annotations

import numpy as np
import pytest

import vllm_jax_amd.workloads as wl
from conftest import from_u16, u16
from oracle import paged_attention_oracle as ora

pytestmark = pytest.mark.gpu

TOL = 2e-2  # max-abs, bf16 outputs (the parity bar for attention outputs)


def _run_and_check(pkg, dev, db, seed, *, seqs=None, soft_cap=None):
    import torch
    d = wl.materialize_decode(db, seed, dev)
    kv = d["kv_cache"]
    # the reference's caller pre-scales q in bf16 (qwen3.py:207); the kernel entry applies no scale
    q_scaled = (d["q"] / torch.tensor(float(np.sqrt(db.head_dim)), dtype=torch.bfloat16)).to(torch.bfloat16)
    out = pkg.decode_paged_attention(q_scaled, kv[0].permute(2, 0, 1, 3), kv[1].permute(2, 0, 1, 3),
                                     d["block_tables"], d["context_lens"], attn_logits_soft_cap=soft_cap)
    torch.cuda.synchronize()
    kvh = u16(kv)
    ref = ora.decode_attention(u16(q_scaled), kvh[0].transpose(2, 0, 1, 3), kvh[1].transpose(2, 0, 1, 3),
                               db.block_tables, db.context_lens, soft_cap=soft_cap, seqs=seqs)
    got = ora.bf16_to_f32(u16(out))
    want = ora.bf16_to_f32(ref)
    sel = slice(None) if seqs is None else np.asarray(seqs)
    err = float(np.abs(got[sel] - want[sel]).max())
    print(f"decode max-abs err {err:.3e}")
    assert err <= TOL, err
    assert np.isfinite(got).all()
    return out, d


@pytest.mark.parametrize("lens,h,hkv,bs", [
    ([1, 15, 16, 17, 60, 100, 0, 31], 8, 2, 16),          # small pages, length 0
    ([1, 255, 256, 257, 600, 1000, 33, 512], 32, 8, 256),  # Qwen3-8B heads
    ([300, 4000, 17], 16, 8, 256),                          # Qwen3-0.6B heads
    ([70, 500], 16, 16, 32),                                # MHA (G = 1)
    ([129, 1024], 16, 1, 64),                               # G = 16
    ([1100, 2049, 64, 1024], 8, 2, 16),                     # 16-token pages: 64 page ids per chunk
    ([5, 40, 1500, 2100], 8, 2, 24),                        # page size not a multiple of 16
    ([2048, 2049, 4097, 6000], 32, 8, 256),                 # chunk boundaries
    ([1, 70, 2049, 300], 40, 2, 256),                       # G = 20: two blocks of q heads, the second partial
    ([17, 1100, 2050], 32, 1, 16),                          # G = 32, 16-token pages, several chunks
    ([0, 5, 600], 17, 1, 24),                               # G = 17, unaligned pages, length 0
    ([32768], 32, 8, 256),                                  # one long sequence: 512-token items, 64 partials
    ([511, 512, 513, 1025, 9000], 32, 8, 16),               # a few sequences: 512-token items, 16-token pages
])
def test_decode_small(pkg, dev, lens, h, hkv, bs):
    # power-of-two table width: the oracle keeps the reference's split divisibility rules
    width = 1 << (max(-(-n // bs) for n in lens) - 1).bit_length()
    db = wl.make_decode(lens, num_heads=h, num_kv_heads=hkv, page_size=bs, rng=np.random.default_rng(len(lens)),
                        table_width=width)
    _run_and_check(pkg, dev, db, seed=3)


def test_decode_soft_cap(pkg, dev):
    db = wl.make_decode([40, 300, 700], num_heads=16, num_kv_heads=8, page_size=256, rng=np.random.default_rng(4))
    _run_and_check(pkg, dev, db, seed=4, soft_cap=5.0)


def test_decode_length_one_is_v0(pkg, dev):
    """Context length 1: the softmax weight is exactly 1, so out == v_0 bit for bit."""
    import torch
    db = wl.make_decode([1, 1, 1], num_heads=32, num_kv_heads=8, page_size=256, rng=np.random.default_rng(5))
    d = wl.materialize_decode(db, 5, dev)
    kv = d["kv_cache"]
    out = pkg.decode_paged_attention(d["q"], kv[0].permute(2, 0, 1, 3), kv[1].permute(2, 0, 1, 3),
                                     d["block_tables"], d["context_lens"])
    torch.cuda.synchronize()
    v0 = kv[1][torch.as_tensor(db.block_tables[:, 0].astype(np.int64), device=dev), 0]  # [B, Hkv, d]
    want = v0.repeat_interleave(4, dim=1)
    assert torch.equal(out, want)


def test_decode_block_relabel_invariance(pkg, dev):
    """Permuting physical blocks and rewriting tables consistently gives a bit-identical result."""
    import torch
    db = wl.make_decode([700, 2000, 256, 9], num_heads=32, num_kv_heads=8, page_size=256, num_pages=24,
                        rng=np.random.default_rng(6))
    d = wl.materialize_decode(db, 6, dev)
    kv = d["kv_cache"]
    out1 = pkg.decode_paged_attention(d["q"], kv[0].permute(2, 0, 1, 3), kv[1].permute(2, 0, 1, 3),
                                      d["block_tables"], d["context_lens"])
    perm = np.random.default_rng(7).permutation(db.num_pages)
    kv2 = torch.empty_like(kv)
    kv2[:, torch.as_tensor(perm, device=dev)] = kv
    bt2 = np.where(db.block_tables >= 0, perm[np.maximum(db.block_tables, 0)], -1).astype(np.int32)
    out2 = pkg.decode_paged_attention(d["q"], kv2[0].permute(2, 0, 1, 3), kv2[1].permute(2, 0, 1, 3),
                                      torch.as_tensor(bt2, device=dev), d["context_lens"])
    torch.cuda.synchronize()
    assert torch.equal(out1, out2)


def test_decode_reference_layout_and_no_lengths(pkg, dev):
    """k_pages in the reference's contiguous [Hkv, NB, BS, d] layout; lengths=None attends to the full table."""
    import torch
    db = wl.make_decode([512, 512], num_heads=8, num_kv_heads=2, page_size=256, rng=np.random.default_rng(8))
    d = wl.materialize_decode(db, 8, dev)
    kp = d["kv_cache"][0].permute(2, 0, 1, 3).contiguous()
    vp = d["kv_cache"][1].permute(2, 0, 1, 3).contiguous()
    out = pkg.decode_paged_attention(d["q"], kp, vp, d["block_tables"], None)
    torch.cuda.synchronize()
    ref = ora.decode_attention(u16(d["q"]), u16(kp), u16(vp), db.block_tables, np.array([512, 512]))
    err = float(np.abs(ora.bf16_to_f32(u16(out)) - ora.bf16_to_f32(ref)).max())
    assert err <= TOL, err


def test_decode_qwen3_8b_full(pkg, dev):
    """Full Qwen3-8B decode workload (256 seqs, ctx U[512,8192]); every sequence against the oracle."""
    db = wl.qwen3_8b_decode()
    _run_and_check(pkg, dev, db, seed=2)


def test_decode_qwen3_8b_full_soft_cap(pkg, dev):
    """The full Qwen3-8B decode workload with a logit soft cap of 30 (the
    kernels' exp2 / reciprocal evaluation of cap * tanh(logit / cap));
    every sequence against the oracle's float64 tanh."""
    db = wl.qwen3_8b_decode()
    _run_and_check(pkg, dev, db, seed=2, soft_cap=30.0)


def test_decode_through_attention_seam(pkg, dev):
    """attention() with DecodeAttentionMetadata: KV store of the new token, then decode."""
    import torch
    db = wl.make_decode([5, 256, 1000, 0], num_heads=16, num_kv_heads=8, page_size=256,
                        rng=np.random.default_rng(10))
    d = wl.materialize_decode(db, 10, dev)
    before = u16(d["kv_cache"])
    meta = pkg.DecodeAttentionMetadata(d["input_positions"], d["slot_mapping"], d["block_tables"],
                                       d["context_lens"])
    kv, out = pkg.attention(d["kv_cache"], d["q"], d["k"], d["v"], meta)
    torch.cuda.synchronize()
    kc, vc = ora.kv_store(before[0], before[1], u16(d["k"]), u16(d["v"]), db.slot_mapping)
    assert np.array_equal(u16(kv[0]), kc) and np.array_equal(u16(kv[1]), vc)
    qs = ora.round_bf16(ora.bf16_to_f32(u16(d["q"])) / np.float32(11.3125))
    ref = ora.decode_attention(ora.f32_to_bf16(qs), kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3),
                               db.block_tables, db.context_lens)
    got = ora.bf16_to_f32(u16(out))
    assert float(np.abs(got - ora.bf16_to_f32(ref)).max()) <= TOL
    assert not got[3].any()  # length-0 (padded) sequence


def test_decode_work_list_all_sequences(pkg, dev):
    """A launch large enough for the decode work list (96 sequences x 4
    chunks of 2048 tokens x 8 kv heads = 3072 workgroups; with 4096-token
    chunks it would hold only 1536, so it keeps the 2048-token ones), every
    sequence against the oracle: lengths 0 and 1, chunk boundaries, ragged
    rest."""
    rng = np.random.default_rng(31)
    lens = rng.integers(2, 6000, 96)
    lens[:8] = [0, 1, 2047, 2048, 2049, 4096, 4097, 6000]
    width = 1 << (int(-(-6000 // 256)) - 1).bit_length()
    db = wl.make_decode(lens.tolist(), num_heads=32, num_kv_heads=8, page_size=256, rng=rng, table_width=width)
    print(f"decode work list: {db.batch} sequences, table width {width}", flush=True)
    out, _ = _run_and_check(pkg, dev, db, seed=31)
    assert not u16(out)[0].any()


@pytest.mark.parametrize("bs,width,cap", [(256, 64, None), (64, 256, None), (80, 256, None), (8192, 2, None),
                                          (256, 64, 5.0), (16, 1024, None), (32, 512, None), (48, 384, None),
                                          (16, 1024, 5.0)])
def test_decode_long_chunks_all_sequences(pkg, dev, bs, width, cap):
    """A launch that still holds 2048 items of 4096 tokens (160 sequences x
    4+ chunks of the widest table row x 8 kv heads), so the split kernel runs
    4096-token chunks; every sequence against the oracle: lengths 0 and 1 and
    both sides of the 4096 and 8192 chunk boundaries.  64-token pages put 64
    page ids in a chunk (one per lane), 80-token ones chunks that start
    inside a page, 8192-token ones two chunks per page; then the soft cap.
    16-, 32- and 48-token pages put 256, 128 and up to 87 page ids in a chunk
    (the kernels that hold four per lane; 48-token chunks start inside a
    page), with and without the soft cap."""
    rng = np.random.default_rng(37)
    lens = rng.integers(2, 16384, 160)
    lens[:10] = [0, 1, 4095, 4096, 4097, 8191, 8192, 8193, 12289, 16384]
    db = wl.make_decode(lens.tolist(), num_heads=32, num_kv_heads=8, page_size=bs, rng=rng, table_width=width)
    print(f"decode long chunks: {db.batch} sequences, {bs}-token pages, table width {width}, soft cap {cap}",
          flush=True)
    out, _ = _run_and_check(pkg, dev, db, seed=37, soft_cap=cap)
    assert not u16(out)[0].any()


def test_decode_work_list_many_q_heads_per_kv_head(pkg, dev):
    """G = 64 (blocks of 32 q heads as separate work items, in the generic
    kernel that takes more than 16 q heads per kv head over bf16 pages) on a
    launch large enough for the work list (64 sequences x 4 chunks of the
    widest table row x 4 kv heads x 2 blocks = 2048 items); every sequence
    against the oracle."""
    rng = np.random.default_rng(57)
    lens = rng.integers(1, 6000, 64)
    lens[:4] = [0, 1, 2048, 4097]
    width = 1 << (int(-(-6000 // 256)) - 1).bit_length()
    db = wl.make_decode(lens.tolist(), num_heads=256, num_kv_heads=4, page_size=256, rng=rng, table_width=width)
    print(f"decode G=64: {db.batch} sequences, table width {width}", flush=True)
    out, _ = _run_and_check(pkg, dev, db, seed=57)
    assert not u16(out)[0].any()
