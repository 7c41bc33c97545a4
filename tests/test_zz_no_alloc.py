"""pa_decode_noalloc (decode with its workspace in a static device array)
against pa_decode with a caller workspace, through the C ABI.

Two calls in a row on the same GPU, the second with a smaller input: the
first leaves its partials and work list in the shared array, and the second
must not depend on them.  Both must be bit-identical to pa_decode (same
kernels) and within the 2e-2 bar of the oracle on sampled sequences."""
from __future__ import annotations

import numpy as np
import pytest

import vllm_jax_amd.workloads as wl
from conftest import u16
from oracle import paged_attention_oracle as ora

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _decode(pkg, d, db, *, noalloc):
    import torch
    kv = d["kv_cache"]
    kp, vp = kv[0].permute(2, 0, 1, 3), kv[1].permute(2, 0, 1, 3)
    hs, ps, ss, _ = kp.stride()
    q, bt, lens = d["q"], d["block_tables"], d["context_lens"]
    out = torch.full_like(q, 3.0)
    stream = torch.cuda.current_stream().cuda_stream
    args = [q.data_ptr(), q.stride(0), q.stride(1), kp.data_ptr(), vp.data_ptr(), db.num_pages, db.page_size,
            ps, ss, hs, bt.data_ptr(), bt.stride(0), bt.shape[1], lens.data_ptr(), db.batch, db.num_heads,
            db.num_kv_heads, 128, 1.0 / 11.3125, 0.0, out.data_ptr(), out.stride(0), out.stride(1)]
    if noalloc:
        pkg._lib.call("pa_decode_noalloc", *args, stream)
    else:
        need = pkg._lib.load().pa_decode_workspace_size(db.batch, db.num_heads, 128, bt.shape[1], db.page_size)
        ws = torch.empty(need, dtype=torch.uint8, device=q.device)
        pkg._lib.call("pa_decode", *args, ws.data_ptr(), need, stream)
    torch.cuda.synchronize()
    return out


def _case(pkg, dev, db, seed):
    import torch
    d = wl.materialize_decode(db, seed, dev)
    need = pkg._lib.load().pa_decode_workspace_size(db.batch, db.num_heads, 128, db.block_tables.shape[1],
                                                      db.page_size)
    print(f"no-alloc decode: {db.batch} sequences, workspace {need} bytes", flush=True)
    got = _decode(pkg, d, db, noalloc=True)
    ref = _decode(pkg, d, db, noalloc=False)
    assert torch.equal(got, ref), "pa_decode_noalloc differs from pa_decode"
    return got, d


def test_decode_noalloc_two_calls_match_pa_decode(pkg, dev):
    import torch
    lib = pkg._lib.load()
    assert lib.pa_decode_noalloc_max_workspace() == 64 << 20
    # 1) a launch with the work list (64 x 4 chunks x 8 kv heads = 2048 workgroups)
    rng = np.random.default_rng(41)
    lens = rng.integers(1, 8192, 64)
    lens[:4] = [1, 2048, 2049, 8192]
    big = wl.make_decode(lens.tolist(), num_heads=32, num_kv_heads=8, page_size=256, rng=rng, table_width=32)
    got1, d1 = _case(pkg, dev, big, 41)
    # 2) a smaller launch right after (grid order, 6 sequences, some over several
    # chunks so the merge reads partials): nothing of call 1 may leak in
    small = wl.make_decode([5, 3000, 1000, 0, 4500, 2049], num_heads=32, num_kv_heads=8, page_size=256,
                           rng=np.random.default_rng(42), table_width=32)
    got2, d2 = _case(pkg, dev, small, 42)
    assert not u16(got2)[3].any()          # length 0: zero row
    # both against the oracle, with q pre-scaled as the reference's caller does (qwen3.py:207)
    for db, d, got, seqs in ((big, d1, got1, [0, 1, 2, 3, 10, 63]), (small, d2, got2, None)):
        kvh = u16(d["kv_cache"])
        qs = ora.f32_to_bf16(ora.round_bf16(ora.bf16_to_f32(u16(d["q"])) / np.float32(11.3125)))
        want = ora.decode_attention(qs, kvh[0].transpose(2, 0, 1, 3), kvh[1].transpose(2, 0, 1, 3),
                                    db.block_tables, db.context_lens, seqs=seqs)
        sel = slice(None) if seqs is None else np.asarray(seqs)
        err = float(np.abs(ora.bf16_to_f32(u16(got))[sel] - ora.bf16_to_f32(want)[sel]).max())
        print(f"no-alloc decode vs oracle max-abs err {err:.3e}", flush=True)
        assert err <= TOL, err
    torch.cuda.synchronize()


def test_decode_noalloc_replays_from_a_hip_graph(pkg, dev):
    """The use the entry is for: a caller that captures its decode step in a
    HIP graph.  The first call on a device looks up the scratch address
    (hipGetSymbolAddress), so it is made before the capture; the captured
    call then allocates nothing and records no memset.  Every replay, with a
    new q written into the captured buffer and eager pa_decode work between
    replays, must equal pa_decode on that q bit for bit."""
    import torch
    rng = np.random.default_rng(44)
    lens = rng.integers(1, 8192, 64)
    lens[:3] = [1, 2049, 8192]
    db = wl.make_decode(lens.tolist(), num_heads=32, num_kv_heads=8, page_size=256, rng=rng, table_width=32)
    d = wl.materialize_decode(db, 44, dev)
    _decode(pkg, d, db, noalloc=True)          # first call on this device, outside the capture
    kv = d["kv_cache"]
    kp, vp = kv[0].permute(2, 0, 1, 3), kv[1].permute(2, 0, 1, 3)
    hs, ps, ss, _ = kp.stride()
    q, bt, lens_d = d["q"], d["block_tables"], d["context_lens"]
    out = torch.full_like(q, 3.0)
    args = [q.data_ptr(), q.stride(0), q.stride(1), kp.data_ptr(), vp.data_ptr(), db.num_pages, db.page_size,
            ps, ss, hs, bt.data_ptr(), bt.stride(0), bt.shape[1], lens_d.data_ptr(), db.batch, db.num_heads,
            db.num_kv_heads, 128, 1.0 / 11.3125, 0.0, out.data_ptr(), out.stride(0), out.stride(1)]
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        pkg._lib.call("pa_decode_noalloc", *args, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    gen = torch.Generator(device="cpu").manual_seed(45)
    for replay in range(3):
        q.copy_((torch.randn(q.shape, generator=gen) * 0.5).to(torch.bfloat16))
        out.fill_(3.0)
        graph.replay()
        torch.cuda.synchronize()
        ref = _decode(pkg, d, db, noalloc=False)   # eager work between replays
        same = torch.equal(out, ref)
        print(f"graph replay {replay}: bit-identical to pa_decode {same}", flush=True)
        assert same, f"replay {replay} differs from pa_decode"
    del graph
    torch.cuda.synchronize()
