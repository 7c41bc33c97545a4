"""Synthetic workloads reproduce the engine's metadata layout
(model_runner.py:204-301) and the stated configurations."""
from __future__ import annotations

import numpy as np
import pytest

import vllm_jax_amd.workloads as wl


def _check_prefill_layout(pb):
    bs = pb.page_size
    for b in range(pb.batch):
        q0, q1 = int(pb.cu_seqlens_q[b]), int(pb.cu_seqlens_q[b + 1])
        p = int(pb.prefix_lens[b])
        for i in range(q0, q1):
            pos = int(pb.input_positions[i])
            assert pos == p + i - q0                                   # model_runner.py:228
            slot = int(pb.slot_mapping[i])
            assert slot // bs == pb.block_tables[b, pos // bs]         # model_runner.py:233-236
            assert slot % bs == pos % bs
        n_pages = -(-(p + q1 - q0) // bs)
        assert (pb.block_tables[b, :n_pages] >= 0).all()
        assert (pb.block_tables[b, n_pages:] == -1).all()              # pad_block_tables
    assert len(set(pb.slot_mapping[pb.slot_mapping >= 0].tolist())) == int((pb.slot_mapping >= 0).sum())


def test_qwen3_06b_prefill_config():
    pb = wl.qwen3_06b_prefill()
    assert pb.cu_seqlens_q.tolist() == [0, 17, 145, 445, 956]
    assert pb.num_pages == 64 and pb.page_size == 256 and pb.num_heads == 16 and pb.num_kv_heads == 8
    assert pb.block_tables.shape == (4, 2)
    assert pb.visible_pairs() == 184375
    assert pb.flops() == 4 * 128 * 16 * 184375
    _check_prefill_layout(pb)


def test_every_named_workload_is_consistent():
    for name, fn in wl.WORKLOADS.items():
        w = fn()
        batches = w if isinstance(w, tuple) else (w,)
        for b in batches:
            if isinstance(b, wl.PrefillBatch):
                _check_prefill_layout(b)
            else:
                lens = b.context_lens
                assert (b.input_positions == np.maximum(lens - 1, 0)).all()   # model_runner.py:276
                for i, n in enumerate(lens):
                    if n > 0:
                        last = b.block_tables[i, (n - 1) // b.page_size]
                        assert b.slot_mapping[i] == last * b.page_size + (n - 1) % b.page_size


def test_mixed_step_blocks_never_collide():
    pre, dec = wl.qwen3_06b_mixed()
    a = pre.block_tables[pre.block_tables >= 0]
    b = dec.block_tables[dec.block_tables >= 0]
    assert len(np.intersect1d(a, b)) == 0
    assert len(np.unique(a)) == len(a) and len(np.unique(b)) == len(b)
    assert pre.batch == 32 and dec.batch == 96
    assert 64 <= pre.q_lens.min() and pre.q_lens.max() <= 2048
    assert 256 <= dec.context_lens.min() and dec.context_lens.max() <= 4096


def test_prefix_workload_shares_full_blocks_and_copies_tails():
    pb = wl.qwen3_8b_prefix_prefill()
    assert pb.refcounts.max() > 1
    shared = set(pb.doc_blocks.tolist())
    for b in range(pb.batch):
        p = int(pb.prefix_lens[b])
        full = p // pb.page_size
        assert set(pb.block_tables[b, :full].tolist()) <= shared
        # new tokens never land in a shared block
        q0, q1 = int(pb.cu_seqlens_q[b]), int(pb.cu_seqlens_q[b + 1])
        assert not (set((pb.slot_mapping[q0:q1] // pb.page_size).tolist()) & shared)
    assert (np.diff(pb.cu_seqlens_k) == pb.prefix_lens + pb.q_lens).all()


def test_decode_workload_bytes():
    db = wl.qwen3_8b_decode()
    assert db.batch == 256 and db.num_pages == 16384
    assert 512 <= db.context_lens.min() and db.context_lens.max() <= 8192
    kv = int(db.context_lens.sum()) * 2 * 8 * 128 * 2
    assert db.kv_bytes() == kv
    assert db.hbm_bytes() > kv


def test_engine_padding_layout():
    pb = wl.make_prefill([100, 23, 7], num_heads=16, num_kv_heads=8, page_size=16, num_pages=20,
                         rng=np.random.default_rng(3), pad_tokens_to=256, pad_batch_to=4)
    assert len(pb.slot_mapping) == 256 and (pb.slot_mapping[130:] == -1).all()
    assert pb.cu_seqlens_q.tolist() == [0, 100, 123, 130, 130]
    assert pb.max_seqlen_bucket == 128
