"""Head sizes other than 128 on gfx950 against the oracle (max-abs <= 2e-2).

pa_prefill, pa_decode and pa_mixed take any head size that is a multiple of 16 from
16 to 256 (the reference only asks q and the pages to agree,
prefill_paged_attention.py:199-203, decode_paged_attention.py:356-360);
sizes other than 128 run the kernels of csrc/any_head.hip.  The cases cover
the head sizes of common model families (64, 80, 96, 256) and the edges
(16, 48, 240), head groups from 1 to 40, page sizes that do and do not
divide 32-token steps, the soft cap, cached prefixes, rows that see no key,
decode chunks, length 0, the mixed launch and the no-alloc decode entry.
"""
from __future__ import annotations

import numpy as np
import pytest

import vllm_jax_amd.workloads as wl
from conftest import u16
from oracle import paged_attention_oracle as ora
from test_gpu_decode import _run_and_check
from test_gpu_mixed import _case as _mixed_case
from test_gpu_mixed import _run as _mixed_run
from test_gpu_prefill import _prefill

pytestmark = pytest.mark.gpu

TOL = 2e-2


@pytest.mark.parametrize("lens,h,hkv,bs,d", [
    ([300, 97, 64, 1], 32, 8, 64, 64),        # G = 4, d = 64
    ([200, 33], 32, 32, 16, 80),              # MHA, d = 80, 16-token pages
    ([129, 260], 32, 4, 256, 96),             # G = 8, d = 96
    ([150, 41, 7], 16, 8, 24, 256),           # G = 2, d = 256, pages not a multiple of 16
    ([90, 300], 40, 2, 32, 16),               # G = 20, d = 16
    ([70, 33], 64, 1, 48, 48),                # G = 64 (one kv head), d = 48
    ([120], 8, 8, 128, 240),                  # MHA, d = 240
    ([100, 45], 16, 8, 8, 64),                # 8-token pages: paged per lane (below 16)
    ([77, 130], 16, 4, 4, 256),               # 4-token pages at d = 256
    ([50, 200], 32, 8, 17, 96),               # 17-token pages: a 32-token step spans up to 3 pages
])
def test_prefill_head_dims(pkg, dev, lens, h, hkv, bs, d):
    pb = wl.make_prefill(lens, num_heads=h, num_kv_heads=hkv, page_size=bs, head_dim=d,
                         rng=np.random.default_rng(sum(lens) + d))
    _prefill(pkg, dev, pb, seed=d)


def test_prefill_head_dim_soft_cap_kernel_entry(pkg, dev):
    pb = wl.make_prefill([90, 300], num_heads=16, num_kv_heads=8, page_size=256, head_dim=64,
                         rng=np.random.default_rng(4))
    _prefill(pkg, dev, pb, seed=4, soft_cap=8.0, use_seam=False)


def test_prefill_head_dim_prefix_cached(pkg, dev):
    """Cached prefixes in shared blocks, then new chunks, at head_dim 256."""
    pb = wl.make_prefix_prefill([0, 300, 512, 40], [130, 64, 200, 1], num_heads=16, num_kv_heads=4,
                                head_dim=256, rng=np.random.default_rng(5), shared_prefix_tokens=600)
    assert pb.refcounts.max() >= 2
    _prefill(pkg, dev, pb, seed=5)


def test_prefill_head_dim_rows_without_keys_are_zero(pkg, dev):
    """Rows whose position precedes the sequence's first kv position are zeros
    at head_dim 96, as at 128."""
    pb = wl.make_prefill([300, 97, 40], num_heads=32, num_kv_heads=8, page_size=64, head_dim=96,
                         rng=np.random.default_rng(13))
    cu = pb.cu_seqlens_q
    blind = []
    for b in range(len(cu) - 1):
        q0, n = int(cu[b]), int(cu[b + 1] - cu[b])
        p0 = 1000 * (b + 1)
        pb.input_positions[q0:q0 + n] = p0 + np.arange(n)
        lo = q0 + n // 3
        hi = lo + max(1, n // 5)
        pb.input_positions[lo:hi] = p0 - 1 - np.arange(hi - lo)
        blind.extend(range(lo, hi))
    got, _ = _prefill(pkg, dev, pb, seed=6, use_seam=False)
    assert not got[np.asarray(blind)].any()


def test_prefill_head_dim_engine_padding(pkg, dev):
    """Tokens padded to a power of two (slot -1) and a padded batch: padding rows are zero."""
    pb = wl.make_prefill([100, 23, 7], num_heads=16, num_kv_heads=8, page_size=16, num_pages=20, head_dim=64,
                         rng=np.random.default_rng(3), pad_tokens_to=256, pad_batch_to=4)
    got, _ = _prefill(pkg, dev, pb, seed=3)
    assert not got[130:].any()


@pytest.mark.parametrize("lens,h,hkv,bs,d", [
    ([1, 15, 16, 17, 60, 100, 0, 31], 8, 2, 16, 64),      # small pages, length 0, d = 64
    ([1, 255, 2049, 4100, 600], 32, 8, 256, 64),          # several 2048-token chunks
    ([300, 33, 1025], 32, 32, 32, 80),                    # MHA, d = 80
    ([700, 2100], 24, 8, 24, 96),                         # G = 3, pages not a multiple of 16
    ([40, 3000, 1], 16, 4, 256, 256),                     # d = 256
    ([129, 1024, 5], 40, 1, 64, 16),                      # G = 40: blocks of 32 q heads, d = 16
    ([77, 500], 8, 8, 48, 240),                           # d = 240
])
def test_decode_head_dims(pkg, dev, lens, h, hkv, bs, d):
    width = 1 << (max(-(-n // bs) for n in lens) - 1).bit_length()
    db = wl.make_decode(lens, num_heads=h, num_kv_heads=hkv, page_size=bs, head_dim=d,
                        rng=np.random.default_rng(len(lens) + d), table_width=width)
    out, _ = _run_and_check(pkg, dev, db, seed=3)
    got = ora.bf16_to_f32(u16(out))
    assert not got[np.asarray(lens) == 0].any()


@pytest.mark.parametrize("d", [64, 96, 256])
def test_decode_head_dims_work_list(pkg, dev, d):
    """A batch large enough for pa_decode's work list (640 sequences x 4 kv
    heads: 2 560 items), which the generic decode then follows, ranks dealt
    over the XCDs; every sequence against the oracle."""
    rng = np.random.default_rng(40 + d)
    lens = rng.integers(0, 700, size=640)
    lens[:6] = [0, 1, 63, 64, 65, 699]
    width = 1 << (max(-(-int(n) // 64) for n in lens) - 1).bit_length()
    db = wl.make_decode(lens, num_heads=16, num_kv_heads=4, page_size=64, head_dim=d,
                        rng=np.random.default_rng(41 + d), table_width=width)
    out, _ = _run_and_check(pkg, dev, db, seed=6)
    assert not ora.bf16_to_f32(u16(out))[lens == 0].any()


@pytest.mark.parametrize("d,hi,bs,width,edges", [
    (96, 5000, 256, 32, [1023, 1024, 1025, 2048, 3073]),     # 1024-token items
    (48, 5000, 256, 32, [1023, 1024, 1025, 2048, 3073]),     # 1024-token items
    (256, 16384, 256, 64, [4095, 4096, 4097, 8192, 12289]),  # 4096-token items (a launch of 2 048+ of them)
    (256, 16384, 16, 1024, [4095, 4096, 4097, 8192, 12289]),  # the same over 16-token pages
])
def test_decode_head_dims_item_lengths(pkg, dev, d, hi, bs, width, edges):
    """The generic decode's item lengths by head size over contexts of
    several items (160 sequences x 8 kv heads, on the work list): lengths 0
    and 1 and both sides of the item boundaries; every sequence against the
    oracle."""
    rng = np.random.default_rng(60 + d)
    lens = rng.integers(2, hi, size=160)
    lens[:2 + len(edges)] = [0, 1] + edges
    db = wl.make_decode(lens.tolist(), num_heads=32, num_kv_heads=8, page_size=bs, head_dim=d,
                        rng=np.random.default_rng(61 + d), table_width=width)
    print(f"generic decode d={d}: {db.batch} sequences, contexts up to {hi}, {bs}-token pages", flush=True)
    out, _ = _run_and_check(pkg, dev, db, seed=9)
    assert not ora.bf16_to_f32(u16(out))[0].any()


def test_decode_head_dim_soft_cap(pkg, dev):
    db = wl.make_decode([40, 300, 2700], num_heads=16, num_kv_heads=8, page_size=256, head_dim=64,
                        rng=np.random.default_rng(4), table_width=16)
    _run_and_check(pkg, dev, db, seed=4, soft_cap=5.0)


def test_decode_head_dim_noalloc_matches_pa_decode(pkg, dev):
    """pa_decode_noalloc at head_dim 64 equals pa_decode with a caller
    workspace bit for bit, on two calls in a row (the second smaller)."""
    import torch
    for lens, seed in (([2100, 64, 4000, 1, 700], 7), ([30, 5], 8)):
        width = 1 << (max(-(-n // 64) for n in lens) - 1).bit_length()
        db = wl.make_decode(lens, num_heads=16, num_kv_heads=4, page_size=64, head_dim=64,
                            rng=np.random.default_rng(seed), table_width=width)
        d = wl.materialize_decode(db, seed, dev)
        kv = d["kv_cache"]
        kp, vp = kv[0].permute(2, 0, 1, 3), kv[1].permute(2, 0, 1, 3)
        hs, ps, ss, _ = kp.stride()
        q, bt, ln = d["q"], d["block_tables"], d["context_lens"]
        args = [q.data_ptr(), q.stride(0), q.stride(1), kp.data_ptr(), vp.data_ptr(), db.num_pages,
                db.page_size, ps, ss, hs, bt.data_ptr(), bt.stride(0), bt.shape[1], ln.data_ptr(), db.batch,
                db.num_heads, db.num_kv_heads, 64, 1.0, 0.0]
        stream = torch.cuda.current_stream().cuda_stream
        got = torch.full_like(q, 3.0)
        pkg._lib.call("pa_decode_noalloc", *args, got.data_ptr(), got.stride(0), got.stride(1), stream)
        need = pkg._lib.load().pa_decode_workspace_size(db.batch, db.num_heads, 64, bt.shape[1], db.page_size)
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        ref = torch.full_like(q, 5.0)
        pkg._lib.call("pa_decode", *args, ref.data_ptr(), ref.stride(0), ref.stride(1), ws.data_ptr(), need,
                      stream)
        torch.cuda.synchronize()
        assert torch.equal(got, ref)
        kvh = u16(kv)
        want = ora.decode_attention(u16(q), kvh[0].transpose(2, 0, 1, 3), kvh[1].transpose(2, 0, 1, 3),
                                    db.block_tables, db.context_lens)
        err = float(np.abs(ora.bf16_to_f32(u16(got)) - ora.bf16_to_f32(want)).max())
        print(f"no-alloc decode at head_dim 64: max-abs err {err:.3e}", flush=True)
        assert err <= TOL


@pytest.mark.parametrize("dec,pre_q,pre_p,h,hkv,bs,d,cap", [
    ([1000, 2000, 513, 0], [130, 257], [0, 100], 16, 8, 256, 64, None),   # d = 64, an empty decode context
    ([5, 4097, 9000], [64, 300], [0, 0], 32, 8, 64, 96, 6.0),             # several chunks, soft cap
    ([700, 30], [100, 5], [0, 40], 40, 2, 48, 256, None),                 # G = 20, 48-token pages
    ([], [17, 128, 300], [0, 0, 0], 16, 8, 16, 80, None),                 # no decode sequence
    ([10, 600, 4096], [], [], 16, 4, 80, 112, None),                      # no prefill sequence, 80-token pages
    ([5000, 2000], [100], [0], 16, 8, 16, 96, None),                       # 16-token pages, 4096-token chunks
])
def test_mixed_head_dims(pkg, dev, dec, pre_q, pre_p, h, hkv, bs, d, cap):
    rng = np.random.default_rng(len(dec) * 100 + h + d)
    q, kc, vc, bt, cu, kv, pos = _mixed_case(rng, dec, pre_q, pre_p, h, hkv, bs, pad_rows=2, d=d)
    nd = len(dec)
    root = float(ora.round_bf16(np.float32(np.sqrt(d))).reshape(-1)[0])
    got = _mixed_run(pkg, dev, q, kc, vc, bt, cu, kv, pos, nd, max(pre_q) if pre_q else 0, soft_cap=cap,
                     decode_scale=1.0 / root)
    want = ora.mixed_attention(q, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), bt, cu, kv, pos, nd,
                               soft_cap=cap)
    err = np.abs(ora.bf16_to_f32(got) - ora.bf16_to_f32(want)).max()
    print(f"mixed at head_dim {d}: max-abs err {err:.3e}", flush=True)
    assert err <= TOL
    zero = np.ones(q.shape[0], bool)
    zero[cu[:nd]] = False
    for b in range(nd, len(kv)):
        zero[cu[b]:cu[b + 1]] = False
    zero[cu[:nd][kv[:nd] == 0]] = True      # empty decode context
    assert not got[zero].any()
