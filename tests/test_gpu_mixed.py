"""One launch for a mixed decode + prefill step on gfx950 against the oracle.

Tolerance: max-abs 2e-2 on bf16 outputs, as for the separate entries.  Rows
no sequence computes must be exactly zero, and the prefill rows must equal
the prefill entry's output bit for bit (same kernel body).
"""
from __future__ import annotations

import numpy as np
import pytest

import vllm_jax_amd.workloads as wl
from conftest import boundary_rows, from_u16, u16
from oracle import paged_attention_oracle as ora

pytestmark = pytest.mark.gpu
TOL = 2e-2
DECODE_SCALE = 1.0 / 11.3125   # 1/bf16(sqrt(128)): the decode caller's scale (qwen3.py:207)


def _bf16(rng, shape, scale=0.5):
    return ora.f32_to_bf16(rng.standard_normal(shape).astype(np.float32) * scale)


def _case(rng, dec_lens, pre_q, pre_prefix, h, hkv, bs, pad_rows=0, empty_decode_row=None, d=128):
    kv = list(dec_lens) + [p + n for p, n in zip(pre_prefix, pre_q)]
    nb = int(sum(-(-int(n) // bs) for n in kv)) + 3
    width = max(1, max(-(-int(n) // bs) for n in kv))
    width = 1 << (width - 1).bit_length()   # a power of two: the oracle's split count divides it
    perm = rng.permutation(nb)
    bt = np.full((len(kv), width), -1, np.int32)
    c = 0
    for b, n in enumerate(kv):
        k = -(-int(n) // bs)
        bt[b, :k] = perm[c:c + k]
        c += k
    q_lens = [1] * len(dec_lens) + list(pre_q)
    if empty_decode_row is not None:
        q_lens[empty_decode_row] = 0
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    pos = np.concatenate([[max(n - 1, 0)] * q for n, q in zip(dec_lens, q_lens[:len(dec_lens)])] +
                         [np.arange(p, p + n) for p, n in zip(pre_prefix, pre_q)]).astype(np.int32)
    pos = np.concatenate([pos, np.zeros(pad_rows, np.int32)])
    q = _bf16(rng, (int(cu[-1]) + pad_rows, h, d))
    kc, vc = _bf16(rng, (nb, bs, hkv, d)), _bf16(rng, (nb, bs, hkv, d))
    return q, kc, vc, bt, cu, np.asarray(kv, np.int32), pos


def _run(pkg, dev, q, kc, vc, bt, cu, kv, pos, nd, max_q, soft_cap=None, decode_scale=DECODE_SCALE):
    import torch
    i32 = lambda a: torch.as_tensor(np.ascontiguousarray(a), dtype=torch.int32, device=dev)
    kcd, vcd = from_u16(kc, dev), from_u16(vc, dev)
    out = pkg.mixed_paged_attention(from_u16(q, dev), kcd.permute(2, 0, 1, 3), vcd.permute(2, 0, 1, 3), i32(bt),
                                    i32(cu), i32(kv), i32(pos), nd, max_seqlen_q=max_q, decode_scale=decode_scale,
                                    attn_logits_soft_cap=soft_cap)
    torch.cuda.synchronize()
    return u16(out)


@pytest.mark.parametrize("dec,pre_q,pre_p,h,hkv,bs,pad", [
    ([1, 40, 0, 70, 300], [5, 33, 1, 200], [0, 12, 50, 0], 8, 2, 16, 3),   # small pages, empty context
    ([1000, 2000, 513], [130, 257], [0, 100], 16, 8, 256, 0),              # Qwen3-0.6B heads
    ([5, 4097, 9000], [64, 300], [0, 0], 32, 8, 256, 0),                   # decode over several chunks
    ([700, 30], [100], [0], 64, 8, 64, 0),                                 # G = 8
    ([50, 60], [70], [10], 8, 8, 32, 2),                                   # MHA
    ([100, 30], [50, 20], [0, 5], 8, 2, 24, 0),                            # pages not 16-aligned
    ([3000, 5000, 100], [90], [0], 8, 2, 48, 0),                           # 48-token pages, 4080-token chunks (85 ids)
    ([5000, 4096, 4097, 1500], [100, 30], [0, 40], 16, 8, 16, 0),          # 16-token pages, 4096-token chunks (256 ids)
    ([9000, 4100], [64], [0], 32, 8, 32, 0),                               # 32-token pages, 4096-token chunks (128 ids)
    ([], [17, 128, 300], [0, 0, 0], 16, 8, 256, 0),                        # no decode sequence
    ([10, 600, 4096], [], [], 16, 8, 256, 1),                              # no prefill sequence
    ([700, 30, 0], [100, 7], [0, 20], 40, 2, 64, 0),                       # G = 20: a 16 + 4 head split
    ([5000, 300], [90, 1], [0, 0], 32, 1, 256, 0),                         # G = 32 (one kv head), 2 chunks
    ([9000, 4500, 100], [300], [0], 16, 8, 4096, 0),                       # 4096-token pages: chunk = page
    ([9000, 5000, 4097], [100], [0], 16, 8, 8192, 0),                      # 8192-token pages: chunks start mid-page
    ([20000, 300], [64], [0], 16, 8, 256, 0),                              # 5 decode chunks: the workgroup-wide merge
])
def test_mixed_matches_oracle(pkg, dev, dec, pre_q, pre_p, h, hkv, bs, pad):
    rng = np.random.default_rng(len(dec) * 100 + h + bs)
    q, kc, vc, bt, cu, kv, pos = _case(rng, dec, pre_q, pre_p, h, hkv, bs, pad_rows=pad)
    nd = len(dec)
    max_q = max(pre_q) if pre_q else 0
    got = _run(pkg, dev, q, kc, vc, bt, cu, kv, pos, nd, max_q)
    want = ora.mixed_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, cu, kv, pos, nd)
    err = np.abs(ora.bf16_to_f32(got) - ora.bf16_to_f32(want)).max()
    print(f"mixed max-abs err {err:.3e}")
    assert err <= TOL
    zero = np.ones(q.shape[0], bool)
    zero[cu[:nd]] = False
    for b in range(nd, len(kv)):
        zero[cu[b]:cu[b + 1]] = False
    zero[cu[:nd][kv[:nd] == 0]] = True      # empty decode context
    assert not got[zero].any()


def test_mixed_work_list_many_q_heads_per_kv_head(pkg, dev):
    """1100 decode sequences with 32 q heads on one kv head and three prefill
    sequences: 2 200 decode items of 16 q heads (two per sequence) put the
    launch on the work-list path, which lists each block of 16 q heads as
    its own entry."""
    rng = np.random.default_rng(77)
    dec = rng.integers(0, 400, 1100).tolist()
    pre_q, pre_p = [150, 9, 260], [0, 40, 300]
    q, kc, vc, bt, cu, kv, pos = _case(rng, dec, pre_q, pre_p, 32, 1, 32)
    nd = len(dec)
    got = _run(pkg, dev, q, kc, vc, bt, cu, kv, pos, nd, max(pre_q))
    want = ora.mixed_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, cu, kv, pos, nd)
    err = np.abs(ora.bf16_to_f32(got) - ora.bf16_to_f32(want)).max()
    print(f"mixed (work list, G = 32) max-abs err {err:.3e}")
    assert err <= TOL
    assert not got[cu[:nd][kv[:nd] == 0]].any()


def test_mixed_prefill_noncontiguous_positions(pkg, dev):
    """Prefill rows of the mixed launch with permuted positions inside their
    sequences (the first row keeps the smallest): every row has its own kv
    limit, so the prefill items' masked tiles vary row by row."""
    rng = np.random.default_rng(21)
    q, kc, vc, bt, cu, kv, pos = _case(rng, [300, 1000, 5], [200, 70, 129], [0, 90, 300], 32, 8, 64)
    nd = 3
    pos = pos.copy()
    for b in range(nd, len(kv)):
        q0, n = int(cu[b]), int(cu[b + 1] - cu[b])
        pos[q0 + 1:q0 + n] = pos[q0] + 1 + rng.permutation(n - 1)
    got = _run(pkg, dev, q, kc, vc, bt, cu, kv, pos, nd, 200)
    want = ora.mixed_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, cu, kv, pos, nd)
    err = np.abs(ora.bf16_to_f32(got) - ora.bf16_to_f32(want)).max()
    print(f"mixed max-abs err {err:.3e}")
    assert err <= TOL


def test_mixed_soft_cap_and_empty_decode_row(pkg, dev):
    """A decode sequence without a q row writes nothing (its cu_seqlens entry
    is the next sequence's row)."""
    rng = np.random.default_rng(5)
    q, kc, vc, bt, cu, kv, pos = _case(rng, [80, 90, 33], [40, 7], [0, 3], 8, 2, 16, empty_decode_row=1)
    got = _run(pkg, dev, q, kc, vc, bt, cu, kv, pos, 3, 40, soft_cap=4.0)
    want = ora.mixed_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, cu, kv, pos, 3,
                               soft_cap=4.0)
    assert np.abs(ora.bf16_to_f32(got) - ora.bf16_to_f32(want)).max() <= TOL


def test_mixed_prefill_rows_bit_exact_with_prefill_entry(pkg, dev):
    import torch
    rng = np.random.default_rng(9)
    q, kc, vc, bt, cu, kv, pos = _case(rng, [300, 700, 2], [129, 64, 500], [0, 40, 0], 16, 8, 64)
    nd = 3
    got = _run(pkg, dev, q, kc, vc, bt, cu, kv, pos, nd, 500)
    i32 = lambda a: torch.as_tensor(np.ascontiguousarray(a), dtype=torch.int32, device=dev)
    base = int(cu[nd])
    cup = cu[nd:] - base
    cuk = np.concatenate([[0], np.cumsum(kv[nd:])]).astype(np.int32)
    kcd, vcd = from_u16(kc, dev), from_u16(vc, dev)
    ref = pkg.prefill_paged_attention(from_u16(q[base:], dev), kcd.permute(2, 0, 1, 3), vcd.permute(2, 0, 1, 3),
                                      i32(bt[nd:]), i32(cup), None, i32(pos[base:]), max_seqlen_bucket=500,
                                      cu_seqlens_k=i32(cuk))
    torch.cuda.synchronize()
    assert np.array_equal(got[base:], u16(ref))


def test_mixed_qwen3_06b_step_through_seam(pkg, dev):
    """The Qwen3-0.6B mixed step (96 decode + 32 prefill sequences, seed 1)
    through attention() with MixedAttentionMetadata, sampled against the
    oracle and compared with the two separate entries."""
    import torch
    pre, dec = wl.qwen3_06b_mixed(1)
    mb = wl.make_mixed(pre, dec)
    t = wl.materialize_mixed(mb, seed=1, device=dev)
    meta = pkg.MixedAttentionMetadata(t["input_positions"], t["slot_mapping"], t["block_tables"],
                                      t["cu_seqlens_q"], t["kv_lens"], mb.num_decodes, mb.max_seqlen_q)
    kv_cache, out = pkg.attention(t["kv_cache"], t["q"], t["k"], t["v"], meta)
    torch.cuda.synchronize()
    got = u16(out)
    kc, vc = u16(kv_cache[0]), u16(kv_cache[1])
    qh = u16(t["q"])
    nd = mb.num_decodes
    # every decode row, and >= 256 prefill rows: each prefill sequence's first,
    # last and middle rows and rows on q-tile / kv-tile / page edges
    dseq = np.arange(nd)
    pr = boundary_rows(mb.cu_seqlens_q[nd:], None, np.random.default_rng(1),
                       tile_tokens=256 // (pre.num_heads // pre.num_kv_heads), per_seq=10)
    assert pr.size >= 256
    want = ora.mixed_attention(qh, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), mb.block_tables,
                               mb.cu_seqlens_q, mb.kv_lens, mb.input_positions, nd, prefill_rows=pr,
                               decode_seqs=dseq)
    rows = np.concatenate([mb.cu_seqlens_q[dseq], pr])
    err = np.abs(ora.bf16_to_f32(got[rows]) - ora.bf16_to_f32(want[rows])).max()
    print(f"mixed step max-abs err {err:.3e} over {nd} decode rows and {pr.size} prefill rows", flush=True)
    assert err <= TOL
    # against the separate decode and prefill entries on the whole step
    kp, vp = kv_cache[0].permute(2, 0, 1, 3), kv_cache[1].permute(2, 0, 1, 3)
    base = int(mb.cu_seqlens_q[nd])
    qd = t["q"][:nd]
    od = pkg.decode_paged_attention(qd, kp, vp, t["block_tables"][:nd], t["kv_lens"][:nd], scale=DECODE_SCALE)
    cup = t["cu_seqlens_q"][nd:] - base
    cuk = torch.as_tensor(np.concatenate([[0], np.cumsum(mb.kv_lens[nd:])]).astype(np.int32), device=dev)
    op = pkg.prefill_paged_attention(t["q"][base:], kp, vp, t["block_tables"][nd:], cup, None,
                                     t["input_positions"][base:], max_seqlen_bucket=mb.max_seqlen_q,
                                     cu_seqlens_k=cuk)
    torch.cuda.synchronize()
    assert np.array_equal(got[base:], u16(op))
    derr = np.abs(ora.bf16_to_f32(got[:nd]) - ora.bf16_to_f32(u16(od))).max()
    assert derr <= TOL, derr
