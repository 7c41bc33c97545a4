"""The attention entries under HIP graph capture.

Every entry launches its kernels on the caller's stream with no allocation,
no host synchronisation and no memset (work lists and counters are written
by the launches themselves), so a step can be captured once and replayed.
Each case captures one call, then replays it three times with new q copied
into the captured buffer between replays (eager work and synchronisations in
between), and checks every replay against an eager call on the same inputs,
bit for bit.
"""
from __future__ import annotations

import numpy as np
import pytest

import vllm_jax_amd.workloads as wl

pytestmark = pytest.mark.gpu


def _check_replays(fn, q, outs, seed):
    import torch
    gen = torch.Generator(device=q.device)
    gen.manual_seed(seed)
    fn()  # the first call on a device may load code objects: not under capture
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    for r in range(3):
        q.copy_((0.5 * torch.randn(q.shape, generator=gen, device=q.device)).to(q.dtype))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        replayed = [o.clone() for o in outs]
        fn()
        torch.cuda.synchronize()
        for a, b in zip(replayed, outs):
            assert torch.equal(a, b), f"replay {r} differs from the eager call"
        print(f"replay {r}: bit-identical to the eager call", flush=True)


def test_prefill_graph_replays(pkg, dev):
    """Prefix-cached prefill with its work list built inside the graph."""
    import torch
    rng = np.random.default_rng(81)
    pb = wl.make_prefix_prefill(rng.integers(0, 2049, 24), rng.integers(64, 700, 24), num_heads=32,
                                num_kv_heads=8, rng=rng, shared_prefix_tokens=2048)
    t = wl.materialize_prefill(pb, seed=81, device=dev)
    kv = pkg.update_kv_cache(t["kv_cache"], t["slot_mapping"], t["k"], t["v"])
    kp, vp = kv[0].permute(2, 0, 1, 3), kv[1].permute(2, 0, 1, 3)
    need = pkg._lib.load().pa_prefill_workspace_size(pb.batch, int(pb.max_seqlen_bucket), pb.num_heads,
                                                     pb.num_kv_heads)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    out = torch.empty_like(t["q"])

    def fn():
        pkg.prefill_paged_attention(t["q"], kp, vp, t["block_tables"], t["cu_seqlens_q"], t["slot_mapping"],
                                    t["input_positions"], max_seqlen_bucket=pb.max_seqlen_bucket,
                                    cu_seqlens_k=t["cu_seqlens_k"], workspace=ws, out=out)
    _check_replays(fn, t["q"], [out], seed=82)


@pytest.mark.parametrize("bs", [256, 16])
def test_decode_graph_replays(pkg, dev, bs):
    """A decode launch with the work list, 4096-token items (one page id per
    lane at 256-token pages, four at 16-token ones), plan and merge kernels
    inside the graph."""
    import torch
    rng = np.random.default_rng(83)
    lens = rng.integers(1, 9000, 160)
    db = wl.make_decode(lens.tolist(), num_heads=32, num_kv_heads=8, page_size=bs, rng=rng)
    d = wl.materialize_decode(db, seed=83, device=dev)
    kv = d["kv_cache"]
    kp, vp = kv[0].permute(2, 0, 1, 3), kv[1].permute(2, 0, 1, 3)
    need = pkg._lib.load().pa_decode_workspace_size(db.batch, db.num_heads, db.head_dim,
                                                    db.block_tables.shape[1], db.page_size)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    out = torch.empty_like(d["q"])

    def fn():
        pkg.decode_paged_attention(d["q"], kp, vp, d["block_tables"], d["context_lens"], scale=1 / 11.3125,
                                   workspace=ws, out=out)
    _check_replays(fn, d["q"], [out], seed=84)


def test_mixed_graph_replays(pkg, dev):
    """The Qwen3-0.6B mixed step (96 decode + 32 prefill sequences) as one
    captured launch with its work list."""
    import torch
    pre, dec = wl.qwen3_06b_mixed(1)
    mb = wl.make_mixed(pre, dec)
    t = wl.materialize_mixed(mb, seed=1, device=dev)
    kv = pkg.update_kv_cache(t["kv_cache"], t["slot_mapping"], t["k"], t["v"])
    kp, vp = kv[0].permute(2, 0, 1, 3), kv[1].permute(2, 0, 1, 3)
    lib = pkg._lib.load()
    need = lib.pa_mixed_workspace_size(mb.batch, mb.num_decodes, mb.max_seqlen_q, pre.num_heads,
                                       pre.num_kv_heads, pre.head_dim, mb.block_tables.shape[1], pre.page_size)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
    out = torch.empty_like(t["q"])

    def fn():
        pkg.mixed_paged_attention(t["q"], kp, vp, t["block_tables"], t["cu_seqlens_q"], t["kv_lens"],
                                  t["input_positions"], mb.num_decodes, max_seqlen_q=mb.max_seqlen_q,
                                  workspace=ws, out=out)
    _check_replays(fn, t["q"], [out], seed=85)
