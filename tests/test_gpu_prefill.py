"""Ragged causal GQA paged prefill on gfx950 against the oracle (max-abs <= 2e-2)."""
from __future__ import annotations

import numpy as np
import pytest

import vllm_jax_amd.workloads as wl
from conftest import boundary_rows, u16
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
    ([300, 41], 40, 2, 64),                    # G = 20: 12-token q tiles, rows 240-255 idle
    ([200, 77], 32, 1, 256),                   # G = 32 (one kv head)
    ([90, 3], 64, 1, 16),                      # G = 64: 4-token q tiles
    ([129], 4, 4, 256),
])
def test_prefill_shapes(pkg, dev, lens, h, hkv, bs):
    pb = wl.make_prefill(lens, num_heads=h, num_kv_heads=hkv, page_size=bs,
                         rng=np.random.default_rng(sum(lens)))
    _prefill(pkg, dev, pb, seed=1)


@pytest.mark.parametrize("kind", ["permuted", "gapped", "reversed"])
def test_prefill_noncontiguous_positions(pkg, dev, kind):
    """Positions that are not contiguous inside a sequence.  kv index j of
    sequence b is visible to row i iff j + positions[cu[b]] <= positions[i]
    (prefill_paged_attention.py:79-82,108-115), so the rows of one q tile have
    different kv limits and most tiles straddle them.  The first row keeps the
    smallest position, so every row sees at least kv index 0."""
    pb = wl.make_prefill([300, 97, 64, 1], num_heads=32, num_kv_heads=8, page_size=64,
                         rng=np.random.default_rng(7))
    rng = np.random.default_rng(11)
    cu = pb.cu_seqlens_q
    for b in range(len(cu) - 1):
        q0, n = int(cu[b]), int(cu[b + 1] - cu[b])
        p0 = int(pb.input_positions[q0])
        if kind == "permuted":
            rel = np.concatenate([[0], 1 + rng.permutation(n - 1)])
        elif kind == "gapped":
            rel = 2 * np.arange(n)
        else:
            rel = np.concatenate([[0], np.arange(n - 1, 0, -1)])
        pb.input_positions[q0:q0 + n] = p0 + rel
    _prefill(pkg, dev, pb, seed=5, use_seam=False)


def test_prefill_rows_before_the_first_kv_position_are_zero(pkg, dev):
    """Rows whose position precedes their sequence's first kv position see no
    key and are written as zeros (the contract of the reference's dense
    definition, prefill_paged_attention.py:502); every other row matches the
    oracle.  Covers q tiles where such rows sit next to rows that see keys."""
    pb = wl.make_prefill([300, 97, 40], num_heads=32, num_kv_heads=8, page_size=64,
                         rng=np.random.default_rng(13))
    cu = pb.cu_seqlens_q
    blind = []
    for b in range(len(cu) - 1):
        q0, n = int(cu[b]), int(cu[b + 1] - cu[b])
        p0 = 1000 * (b + 1)
        pb.input_positions[q0:q0 + n] = p0 + np.arange(n)
        lo = q0 + n // 3
        hi = lo + max(1, n // 5)
        pb.input_positions[lo:hi] = p0 - 1 - np.arange(hi - lo)   # before kv position p0
        blind.extend(range(lo, hi))
    got, _ = _prefill(pkg, dev, pb, seed=6, use_seam=False)
    assert not got[np.asarray(blind)].any()


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
    """Full Qwen3-8B prefix-cached workload (64 sequences, cached prefixes
    U[0, 4096], new chunks U[128, 1024]); oracle on the first and last new row
    of every sequence plus rows on q-tile, kv-tile and page edges."""
    pb = wl.qwen3_8b_prefix_prefill()
    rng = np.random.default_rng(0)
    prefix = np.diff(pb.cu_seqlens_k) - np.diff(pb.cu_seqlens_q)
    rows = boundary_rows(pb.cu_seqlens_q, prefix, rng, tile_tokens=256 // (pb.num_heads // pb.num_kv_heads),
                         per_seq=6)
    cu = pb.cu_seqlens_q
    assert set(cu[:-1]) <= set(rows) and set(cu[1:] - 1) <= set(rows)
    print(f"qwen3-8b prefix-cached: {rows.size} rows over {pb.batch} sequences", flush=True)
    _prefill(pkg, dev, pb, seed=3, rows=rows)


def test_prefill_qwen3_8b_prefix_workload_soft_cap(pkg, dev):
    """The full Qwen3-8B prefix-cached workload with a logit soft cap of 30
    (the soft-capped prefill kernel): first, last and edge rows of every
    sequence against the oracle's float64 tanh."""
    pb = wl.qwen3_8b_prefix_prefill()
    prefix = np.diff(pb.cu_seqlens_k) - np.diff(pb.cu_seqlens_q)
    rows = boundary_rows(pb.cu_seqlens_q, prefix, np.random.default_rng(6),
                         tile_tokens=256 // (pb.num_heads // pb.num_kv_heads), per_seq=4)
    print(f"qwen3-8b prefix-cached, soft cap 30: {rows.size} rows over {pb.batch} sequences", flush=True)
    _prefill(pkg, dev, pb, seed=3, rows=rows, soft_cap=30.0, use_seam=False)


def test_prefill_qwen3_06b_mixed_prefill_half(pkg, dev):
    """The 32 prefill sequences of the Qwen3-0.6B mixed step: first, last and
    edge rows of every sequence (>= 256 rows)."""
    pre, _ = wl.qwen3_06b_mixed()
    rng = np.random.default_rng(1)
    rows = boundary_rows(pre.cu_seqlens_q, None, rng, tile_tokens=256 // (pre.num_heads // pre.num_kv_heads),
                         per_seq=10)
    assert rows.size >= 256
    _prefill(pkg, dev, pre, seed=1, rows=rows)


def test_prefill_qwen3_32b_long(pkg, dev):
    """Full Qwen3-32B long-context workload (8 seqs of 8k-32k tokens).

    Oracle on 10 rows of every sequence (first, second, middle, last, rows on
    both sides of 32-token q-tile, 64-token kv-tile and 256-token page edges,
    random interior rows), plus a full-size property: the last row of every
    sequence must equal a decode over that sequence's whole context with the
    same q (both on the GPU).
    """
    import torch
    pb = wl.qwen3_32b_long_prefill()
    cu = pb.cu_seqlens_q
    rows = boundary_rows(cu, None, np.random.default_rng(4), tile_tokens=256 // (pb.num_heads // pb.num_kv_heads),
                         per_seq=10)
    assert rows.size >= 64
    print(f"qwen3-32b long prefill: {rows.size} rows over {pb.batch} sequences", flush=True)
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


def _raw_prefill(pkg, t, pb, workspace, max_seqlen=None):
    """pa_prefill through the C ABI, with a caller workspace or none."""
    import torch
    kv = t["kv_cache"]
    kp, vp = kv[0].permute(2, 0, 1, 3), kv[1].permute(2, 0, 1, 3)
    hs, ps, ss, _ = kp.stride()
    q, bt = t["q"], t["block_tables"]
    out = torch.full_like(q, 7.0)
    cuk = t["cu_seqlens_k"]
    ws = (None, 0) if workspace is None else (workspace.data_ptr(), workspace.numel())
    pkg._lib.call("pa_prefill", q.data_ptr(), q.stride(0), q.stride(1), kp.data_ptr(), vp.data_ptr(), pb.num_pages,
                  pb.page_size, ps, ss, hs, bt.data_ptr(), bt.stride(0), bt.shape[1], t["cu_seqlens_q"].data_ptr(),
                  cuk.data_ptr() if cuk is not None else None, t["input_positions"].data_ptr(), pb.batch,
                  q.shape[0], int(max_seqlen or pb.max_seqlen_bucket), pb.num_heads, pb.num_kv_heads, 128,
                  0.08837890625, 0.0, out.data_ptr(), out.stride(0), out.stride(1), *ws,
                  torch.cuda.current_stream().cuda_stream)
    return out


def _expected_list(pb, num_tokens, max_seqlen):
    """Per (sequence, q tile) pair with rows: its geometry and kv-tile cost
    class (contiguous-position estimate, classes of 16 kv tiles), as the
    work list must hold them."""
    g = pb.num_heads // pb.num_kv_heads
    tt = 256 // g
    nq = -(-max_seqlen // tt)
    cu = pb.cu_seqlens_q.astype(np.int64)
    cuk = pb.cu_seqlens_k if pb.cu_seqlens_k is not None else cu
    span = pb.block_tables.shape[1] * pb.page_size
    want = {}
    for b in range(pb.batch):
        q0, lq = int(cu[b]), int(cu[b + 1] - cu[b])
        rows = 0 if (q0 < 0 or q0 >= num_tokens) else min(lq, max_seqlen, num_tokens - q0)
        lk = min(int(cuk[b + 1] - cuk[b]), span)
        for qt in range(nq):
            if qt * tt >= rows:
                continue
            off = int(pb.input_positions[q0]) - (lk - lq)
            hi = min(lk, lk - lq + min(qt * tt + tt, rows))
            cost = min((-(-hi // 64) if hi > 0 else 0) // 16 + 1, 4095)
            want[(b, qt)] = (q0, rows, lk, off, cost)
    return want


@pytest.mark.parametrize("case", ["prefix", "many", "padded", "pooled"])
def test_prefill_work_list(pkg, dev, case):
    """The work list (caller workspace) holds every (sequence, q tile) pair
    with rows once, with its geometry, in non-increasing cost class, the
    pairs of one class and one 64-pair planner run adjacent with their q
    tiles descending; and the output with
    the list is bit-identical to the grid-order output without.  "pooled"
    is the smallest launch that runs the pooled kernel (16 384 items: 16
    sequences of 4 096 tokens, 64 q / 8 kv heads): a pool item dropped or
    run twice would change the output, and every XCD's pool counter must
    have reached its pool size (a quarter of that XCD's items)."""
    import torch
    if case == "pooled":
        pb = wl.make_prefill([4096] * 16, num_heads=64, num_kv_heads=8, rng=np.random.default_rng(13))
    elif case == "prefix":
        pb = wl.make_prefix_prefill([0, 300, 512, 40, 1500, 3, 900, 64, 2000, 10, 700, 1200],
                                    [130, 64, 200, 1, 700, 260, 333, 1000, 45, 600, 17, 400], num_heads=32,
                                    num_kv_heads=8, rng=np.random.default_rng(7), shared_prefix_tokens=2100)
    elif case == "many":
        rng = np.random.default_rng(23)
        pb = wl.make_prefill(rng.integers(1, 300, 90).tolist(), num_heads=16, num_kv_heads=8, page_size=64, rng=rng)
    else:
        pb = wl.make_prefill([100, 23, 7, 1000, 640, 64, 65, 300, 999, 1, 512, 130], num_heads=32, num_kv_heads=8,
                             page_size=16, rng=np.random.default_rng(3), pad_tokens_to=8192, pad_batch_to=16)
    nq = -(-pb.max_seqlen_bucket // (256 // (pb.num_heads // pb.num_kv_heads)))
    assert pb.batch * nq * pb.num_kv_heads >= 1024, "below the work list's launch size"
    t = wl.materialize_prefill(pb, 11, dev)
    pkg.update_kv_cache(t["kv_cache"], t["slot_mapping"], t["k"], t["v"])
    need = pkg._lib.load().pa_prefill_workspace_size(pb.batch, pb.max_seqlen_bucket, pb.num_heads,
                                                     pb.num_kv_heads)
    ws = torch.full((need,), 0xAB, dtype=torch.uint8, device=dev)
    print(f"case {case}: batch {pb.batch} tokens {pb.num_tokens} workspace {need} B", flush=True)
    got = _raw_prefill(pkg, t, pb, ws)
    base = _raw_prefill(pkg, t, pb, None)
    torch.cuda.synchronize()
    assert np.array_equal(u16(got), u16(base)), "work-list order changed the output"
    plan = ws.view(torch.int32).cpu().numpy()
    want = _expected_list(pb, t["q"].shape[0], pb.max_seqlen_bucket)
    count = int(plan[0])
    assert count == len(want)
    if case == "pooled":
        items_per_xcd = count * (pb.num_kv_heads // 8)
        assert count * pb.num_kv_heads >= 16384, "the launch is below the pooled kernel's threshold"
        counters = plan[8:16]
        print(f"pool counters {counters.tolist()} (pool size {items_per_xcd // 4})", flush=True)
        assert (counters >= items_per_xcd // 4).all(), counters
    rec = plan[64:64 + 8 * count].reshape(count, 8)
    seen = set()
    costs = []
    for r in rec:
        key = (int(r[0]), int(r[1]))
        assert key in want and key not in seen, key
        seen.add(key)
        q0, rows, lk, off, cost = want[key]
        assert tuple(int(x) for x in r[2:6]) == (q0, rows, lk, off), (key, r)
        costs.append(cost)
    assert all(a >= b for a, b in zip(costs, costs[1:])), "work list not in non-increasing cost class"
    # The planner walks pair i = b * nq + (nq - 1 - qt) (a sequence's q tiles
    # in a row, costliest first) in runs of 64, one run per wave, and each run
    # reserves its pairs of one class with one atomic: so the pairs of one
    # (class, run) are adjacent in the list, in lane order (ascending pair
    # index: a sequence's q tiles descending).
    nq = -(-pb.max_seqlen_bucket // (256 // (pb.num_heads // pb.num_kv_heads)))
    groups = {}
    for rank, (r, c) in enumerate(zip(rec, costs)):
        run = (int(r[0]) * nq + nq - 1 - int(r[1])) // 64
        groups.setdefault((c, run), []).append((rank, int(r[0]) * nq + nq - 1 - int(r[1])))
    for key, members in groups.items():
        ranks = [m[0] for m in members]
        pair_ids = [m[1] for m in members]
        assert ranks == list(range(ranks[0], ranks[0] + len(ranks))), ("run not contiguous", key, ranks[:8])
        assert all(a < b for a, b in zip(pair_ids, pair_ids[1:])), ("run not in lane order", key, pair_ids[:8])


def test_prefill_more_sequences_than_the_planner_holds(pkg, dev):
    """2100 sequences of 1-3 tokens: above the work list's 2048-sequence
    limit pa_prefill runs in grid order; every row against the oracle."""
    rng = np.random.default_rng(41)
    lens = rng.integers(1, 4, 2100).tolist()
    pb = wl.make_prefill(lens, num_heads=16, num_kv_heads=8, page_size=16, rng=rng)
    print(f"prefill {pb.batch} sequences, {pb.num_tokens} tokens", flush=True)
    _prefill(pkg, dev, pb, seed=41, use_seam=False)


@pytest.mark.parametrize("with_list", [True, False])
def test_prefill_rows_past_max_seqlen_are_zero(pkg, dev, with_list):
    """max_seqlen_q below a sequence's length: its rows at offset >=
    max_seqlen_q are written as zeros (the reference's scatter covers only
    the first max_seqlen_bucket rows, prefill...:384-388); the rows before
    are unchanged by the truncation (causal rows see only earlier kv).  128
    sequences of one 128-token q tile x 8 kv heads = 1024 items: with a
    workspace the launch builds its work list and the list's launch zeroes
    the rows; without, the prefill kernel's last workgroups do."""
    import torch
    pb = wl.make_prefill([100, 300, 40] + [50] * 125, num_heads=16, num_kv_heads=8, page_size=64,
                         rng=np.random.default_rng(51))
    t = wl.materialize_prefill(pb, 51, dev)
    kv = pkg.update_kv_cache(t["kv_cache"], t["slot_mapping"], t["k"], t["v"])
    ws = None
    if with_list:
        ws = torch.empty(pkg._lib.load().pa_prefill_workspace_size(pb.batch, 128, 16, 8), dtype=torch.uint8,
                         device=dev)
    out = _raw_prefill(pkg, t, pb, ws, max_seqlen=128)
    torch.cuda.synchronize()
    got = ora.bf16_to_f32(u16(out))
    cu = pb.cu_seqlens_q
    kept = np.concatenate([np.arange(cu[b], min(cu[b + 1], cu[b] + 128)) for b in range(pb.batch)])
    dropped = np.setdiff1d(np.arange(pb.num_tokens), kept)
    assert len(dropped) == 300 - 128
    assert not got[dropped].any()
    kh = u16(kv)
    ref = ora.prefill_attention(u16(t["q"]), kh[0].transpose(2, 0, 1, 3), kh[1].transpose(2, 0, 1, 3),
                                pb.block_tables, pb.cu_seqlens_q, pb.input_positions, rows=kept)
    err = float(np.abs(got[kept] - ora.bf16_to_f32(ref)[kept]).max())
    print(f"truncated prefill max-abs err {err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("prefix", [False, True])
def test_prefill_page_sizes_bit_identical(pkg, dev, prefix):
    """The same tokens over 16-, 32-, 48-, 64- and 256-token pages: the three
    ways the tile loads find their pages (per lane at 48, one base per wave
    and tile at 16 and 32, one per tile at 64 and 256) read the same K / V
    rows, so the outputs are bit-identical; the 16-token one is also checked
    against the oracle.  With cached prefixes the kv ranges end inside pages
    and tiles, and rows past a kv length take the clamped last row."""
    import torch
    pre = [0, 5, 300, 1111, 64] if prefix else [0] * 6
    new = [700, 1, 129, 64, 333] if prefix else [1, 63, 64, 65, 700, 1500]
    gen = np.random.default_rng(74)
    bf = lambda *shape: torch.as_tensor(ora.round_bf16(0.5 * gen.standard_normal(shape).astype(np.float32)),
                                        device=dev).to(torch.bfloat16)
    doc_k, doc_v = bf(max(pre) + 1, 8, 128), bf(max(pre) + 1, 8, 128)   # the cached document's K / V
    q, k, v = bf(sum(new), 32, 128), bf(sum(new), 8, 128), bf(sum(new), 8, 128)
    outs = {}
    for bs in (16, 32, 48, 64, 256):
        rng = np.random.default_rng(71)
        if prefix:
            pb = wl.make_prefix_prefill(pre, new, num_heads=32, num_kv_heads=8, page_size=bs, rng=rng,
                                        shared_prefix_tokens=max(pre) + 1)
        else:
            pb = wl.make_prefill(new, num_heads=32, num_kv_heads=8, page_size=bs, rng=rng)
        kv = torch.zeros((2, pb.num_pages, bs, 8, 128), dtype=torch.bfloat16, device=dev)
        # the cached tokens: every prefix slot once (shared pages hold the same document tokens)
        slots = {}
        for b, p in enumerate(pre):
            for j in range(p):
                slots.setdefault(int(pb.block_tables[b, j // bs]) * bs + j % bs, j)
        if slots:
            sl = torch.as_tensor(list(slots), dtype=torch.int32, device=dev)
            pos = torch.as_tensor(list(slots.values()), dtype=torch.long, device=dev)
            kv = pkg.update_kv_cache(kv, sl, doc_k[pos], doc_v[pos])
        kv = pkg.update_kv_cache(kv, torch.as_tensor(pb.slot_mapping, dtype=torch.int32, device=dev), k, v)
        i32 = lambda a: torch.as_tensor(np.ascontiguousarray(a), dtype=torch.int32, device=dev)
        out = pkg.prefill_paged_attention(q, kv[0].permute(2, 0, 1, 3), kv[1].permute(2, 0, 1, 3),
                                          i32(pb.block_tables), i32(pb.cu_seqlens_q), i32(pb.slot_mapping),
                                          i32(pb.input_positions), max_seqlen_bucket=pb.max_seqlen_bucket,
                                          cu_seqlens_k=i32(pb.cu_seqlens_k))
        torch.cuda.synchronize()
        outs[bs] = u16(out)
        if bs == 16:
            kvh = u16(kv)
            ref = ora.prefill_attention(u16(q), kvh[0].transpose(2, 0, 1, 3), kvh[1].transpose(2, 0, 1, 3),
                                        pb.block_tables, pb.cu_seqlens_q, pb.input_positions,
                                        cu_seqlens_k=pb.cu_seqlens_k)
            err = float(np.abs(ora.bf16_to_f32(outs[16]) - ora.bf16_to_f32(ref)).max())
            print(f"16-token pages vs oracle: max-abs err {err:.3e}", flush=True)
            assert err <= TOL
    for bs in (32, 48, 64, 256):
        assert np.array_equal(outs[bs], outs[16]), bs
