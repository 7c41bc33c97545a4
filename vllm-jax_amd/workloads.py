"""Synthetic paged-attention workloads with the engine's metadata layout.

Metadata is built the way the reference runner builds it
(vllm/src/model_runner.py:217-301): per-sequence block tables padded with -1
(``pad_block_tables`` :204-214), flat slots ``block_id * page_size + offset``
(:233-236, :283-284), positions restarting at 0 per sequence (:228), decode
``context_lens = len`` including the new token and ``input_positions =
len - 1`` (:276-278).  Physical block ids are handed out in order from
``rng.permutation(num_pages)``.

Randomness: metadata (lengths, block permutation) comes from
``numpy.random.default_rng(seed)``; tensor values (q, new k/v, existing pool
contents) are ``0.5 * N(0, 1)`` rounded to bf16 from a ``torch.Generator``
seeded with the same seed on the target device.

The five named workloads are the paged-attention shapes of Qwen3-0.6B,
Qwen3-8B and Qwen3-32B (16/8, 32/8 and 64/8 q/kv heads, head_dim 128,
256-token pages).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

HEAD_DIM = 128
PAGE_SIZE = 256


@dataclass
class PrefillBatch:
    """Ragged prefill batch (optionally with cached prefixes)."""
    num_heads: int
    num_kv_heads: int
    head_dim: int
    page_size: int
    num_pages: int
    q_lens: np.ndarray            # [B] new tokens per sequence
    prefix_lens: np.ndarray       # [B] cached tokens per sequence (0 = none)
    block_tables: np.ndarray      # [B, P] int32, -1 padded
    cu_seqlens_q: np.ndarray      # [B+1] int32
    cu_seqlens_k: np.ndarray      # [B+1] int32 (kv lengths = prefix + new)
    input_positions: np.ndarray   # [T] int32
    slot_mapping: np.ndarray      # [T] int32
    max_seqlen_bucket: int
    refcounts: np.ndarray = field(default=None)  # [num_pages] references per block

    @property
    def num_tokens(self) -> int:
        return int(self.cu_seqlens_q[-1])

    @property
    def batch(self) -> int:
        return len(self.q_lens)

    def visible_pairs(self) -> int:
        n = self.q_lens.astype(np.int64)
        p = self.prefix_lens.astype(np.int64)
        return int((n * p + n * (n + 1) // 2).sum())

    def flops(self) -> int:
        """Algorithmic FLOP: QK^T and PV over causal-visible pairs, 2 flop/MAC."""
        return 4 * self.head_dim * self.num_heads * self.visible_pairs()


@dataclass
class DecodeBatch:
    num_heads: int
    num_kv_heads: int
    head_dim: int
    page_size: int
    num_pages: int
    context_lens: np.ndarray      # [B] int32, includes the new token
    block_tables: np.ndarray      # [B, P] int32, -1 padded
    input_positions: np.ndarray   # [B] = len - 1
    slot_mapping: np.ndarray      # [B] slot of the new token

    @property
    def batch(self) -> int:
        return len(self.context_lens)

    def kv_bytes(self) -> int:
        return int(np.sum(self.context_lens, dtype=np.int64)) * 2 * self.num_kv_heads * self.head_dim * 2

    def hbm_bytes(self) -> int:
        """Algorithmic bytes: K+V context, q in, o out, block tables, lengths."""
        b = self.batch
        pages = np.ceil(self.context_lens / self.page_size).astype(np.int64)
        return (self.kv_bytes() + 2 * b * self.num_heads * self.head_dim * 2
                + 4 * int(pages.sum()) + 4 * b)

    def flops(self) -> int:
        return 4 * self.head_dim * self.num_heads * int(np.sum(self.context_lens, dtype=np.int64))


@dataclass
class MixedBatch:
    """One scheduler step, unpadded: the decode sequences of ``decode`` first
    (one q row each), then the prefill sequences of ``prefill``."""
    prefill: PrefillBatch
    decode: DecodeBatch
    block_tables: np.ndarray      # [B, P] int32, decode rows first
    cu_seqlens_q: np.ndarray      # [B+1] int32
    kv_lens: np.ndarray           # [B] int32
    input_positions: np.ndarray   # [T] int32
    slot_mapping: np.ndarray      # [T] int32

    @property
    def num_decodes(self) -> int:
        return self.decode.batch

    @property
    def batch(self) -> int:
        return len(self.kv_lens)

    @property
    def num_tokens(self) -> int:
        return int(self.cu_seqlens_q[-1])

    @property
    def max_seqlen_q(self) -> int:
        return int(self.prefill.q_lens.max()) if self.prefill.batch else 0

    def flops(self) -> int:
        return self.prefill.flops() + self.decode.flops()


def make_mixed(pre: PrefillBatch, dec: DecodeBatch) -> MixedBatch:
    """Concatenate a decode batch and a prefill batch over one pool."""
    assert (pre.num_heads, pre.num_kv_heads, pre.page_size, pre.num_pages) == \
        (dec.num_heads, dec.num_kv_heads, dec.page_size, dec.num_pages)
    width = max(pre.block_tables.shape[1], dec.block_tables.shape[1])
    bt = np.full((dec.batch + pre.batch, width), -1, np.int32)
    bt[:dec.batch, :dec.block_tables.shape[1]] = dec.block_tables
    bt[dec.batch:, :pre.block_tables.shape[1]] = pre.block_tables
    q_lens = np.concatenate([np.ones(dec.batch, np.int64), pre.q_lens.astype(np.int64)])
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    kv = np.concatenate([dec.context_lens, np.diff(pre.cu_seqlens_k)]).astype(np.int32)
    pos = np.concatenate([dec.input_positions, pre.input_positions[:pre.num_tokens]]).astype(np.int32)
    slots = np.concatenate([dec.slot_mapping, pre.slot_mapping[:pre.num_tokens]]).astype(np.int32)
    return MixedBatch(pre, dec, bt, cu, kv, pos, slots)


def _bucket(v: int) -> int:
    return 1 if v <= 1 else 1 << (int(v) - 1).bit_length()


def _tables(lens_in_pages, perm, width):
    tables = np.full((len(lens_in_pages), width), -1, np.int32)
    cursor = 0
    for i, n in enumerate(lens_in_pages):
        tables[i, :n] = perm[cursor:cursor + n]
        cursor += n
    return tables, cursor


def make_prefill(q_lens, *, num_heads, num_kv_heads, page_size=PAGE_SIZE, num_pages=None,
                 head_dim=HEAD_DIM, rng=None, perm=None, pad_batch_to=None, pad_tokens_to=None,
                 table_width=None) -> PrefillBatch:
    """Fresh (prefix-free) ragged prefill, as ``prepare_prefill`` lays it out.

    ``perm`` (optional) supplies the physical block ids to deal out; by
    default ``rng.permutation(num_pages)``.
    """
    rng = np.random.default_rng(0) if rng is None else rng
    q_lens = np.asarray(q_lens, np.int64)
    pages = [-(-int(n) // page_size) for n in q_lens]
    if num_pages is None:
        num_pages = max(1, sum(pages))
    if sum(pages) > num_pages:
        raise ValueError(f"{sum(pages)} pages needed, pool has {num_pages}")
    width = table_width or max(1, max(pages))
    if perm is None:
        perm = rng.permutation(num_pages).astype(np.int32)
    tables, _ = _tables(pages, perm, width)
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    positions = np.concatenate([np.arange(n) for n in q_lens]).astype(np.int32) if len(q_lens) else np.zeros(0, np.int32)
    slots = np.concatenate([
        tables[b, np.arange(n) // page_size].astype(np.int64) * page_size + np.arange(n) % page_size
        for b, n in enumerate(q_lens)]).astype(np.int32) if len(q_lens) else np.zeros(0, np.int32)
    total = int(cu[-1])
    if pad_tokens_to is not None and pad_tokens_to > total:
        pad = pad_tokens_to - total
        positions = np.concatenate([positions, np.zeros(pad, np.int32)])
        slots = np.concatenate([slots, np.full(pad, -1, np.int32)])
    if pad_batch_to is not None and pad_batch_to > len(q_lens):
        extra = pad_batch_to - len(q_lens)
        cu = np.concatenate([cu, np.full(extra, cu[-1], np.int32)])
        tables = np.concatenate([tables, np.full((extra, width), -1, np.int32)])
    n_b = len(cu) - 1
    q_pad = np.concatenate([q_lens, np.zeros(n_b - len(q_lens), np.int64)])
    refc = np.zeros(num_pages, np.int32)
    used = tables[tables >= 0]
    np.add.at(refc, used, 1)
    return PrefillBatch(num_heads, num_kv_heads, head_dim, page_size, num_pages, q_pad,
                        np.zeros(n_b, np.int64), tables, cu, cu.copy(), positions, slots,
                        _bucket(int(q_lens.max()) if len(q_lens) else 1), refc)


def make_prefix_prefill(prefix_lens, new_lens, *, num_heads, num_kv_heads, page_size=PAGE_SIZE,
                        head_dim=HEAD_DIM, rng=None, shared_prefix_tokens=None) -> PrefillBatch:
    """Prefill of new chunks after cached prefixes held in shared blocks.

    Every sequence's prefix is the first ``P_b`` tokens of one common cached
    document.  Its full pages are shared: the same physical block id appears
    in every table whose prefix covers it, with ``refcount`` = number of such
    tables.  A partial last prefix page is copy-on-write: the sequence gets a
    private block (filled with a copy of the shared page by
    :func:`materialize_prefill`) so its new tokens never touch shared blocks.
    q positions are ``P_b + i``; kv length is ``P_b + N_b``.
    """
    rng = np.random.default_rng(0) if rng is None else rng
    prefix_lens = np.asarray(prefix_lens, np.int64)
    new_lens = np.asarray(new_lens, np.int64)
    doc = int(shared_prefix_tokens or (prefix_lens.max() if len(prefix_lens) else 0))
    doc_pages = -(-doc // page_size)
    private_pages = [-(-int(p + n) // page_size) - int(p) // page_size for p, n in zip(prefix_lens, new_lens)]
    num_pages = doc_pages + sum(private_pages)
    perm = rng.permutation(num_pages).astype(np.int32)
    doc_blocks = perm[:doc_pages]
    cursor = doc_pages
    width = max(-(-int(p + n) // page_size) for p, n in zip(prefix_lens, new_lens))
    tables = np.full((len(new_lens), width), -1, np.int32)
    cow_src = []  # (private block, shared block, tokens to copy)
    for b, (p, n) in enumerate(zip(prefix_lens, new_lens)):
        full = int(p) // page_size
        tables[b, :full] = doc_blocks[:full]
        k = private_pages[b]
        tables[b, full:full + k] = perm[cursor:cursor + k]
        if p % page_size:
            cow_src.append((int(perm[cursor]), int(doc_blocks[full]), int(p % page_size)))
        cursor += k
    cu_q = np.concatenate([[0], np.cumsum(new_lens)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(prefix_lens + new_lens)]).astype(np.int32)
    positions = np.concatenate([np.arange(p, p + n) for p, n in zip(prefix_lens, new_lens)]).astype(np.int32)
    slots = np.concatenate([
        tables[b, np.arange(p, p + n) // page_size].astype(np.int64) * page_size + np.arange(p, p + n) % page_size
        for b, (p, n) in enumerate(zip(prefix_lens, new_lens))]).astype(np.int32)
    refc = np.zeros(num_pages, np.int32)
    np.add.at(refc, tables[tables >= 0], 1)
    pb = PrefillBatch(num_heads, num_kv_heads, head_dim, page_size, num_pages, new_lens, prefix_lens,
                      tables, cu_q, cu_k, positions, slots, _bucket(int(new_lens.max())), refc)
    pb.cow = cow_src
    pb.doc_blocks = doc_blocks
    return pb


def make_decode(context_lens, *, num_heads, num_kv_heads, page_size=PAGE_SIZE, num_pages=None,
                head_dim=HEAD_DIM, rng=None, perm=None, table_width=None) -> DecodeBatch:
    """Decode batch: one new token per sequence at position len-1 (model_runner.py:268-292)."""
    rng = np.random.default_rng(0) if rng is None else rng
    lens = np.asarray(context_lens, np.int64)
    pages = [-(-int(n) // page_size) for n in lens]
    if num_pages is None:
        num_pages = max(1, sum(pages))
    if perm is None:
        perm = rng.permutation(num_pages).astype(np.int32)
    width = table_width or max(1, max(pages))
    tables, _ = _tables(pages, perm, width)
    last = np.maximum(lens - 1, 0)
    slots = np.where(lens > 0, tables[np.arange(len(lens)), last // page_size].astype(np.int64) * page_size
                     + last % page_size, -1).astype(np.int32)
    return DecodeBatch(num_heads, num_kv_heads, head_dim, page_size, num_pages, lens.astype(np.int32),
                       tables, last.astype(np.int32), slots)


# ---------------------------------------------------------------------------
# the named workloads
# ---------------------------------------------------------------------------
def qwen3_06b_prefill(seed=0) -> PrefillBatch:
    """4 sequences [17,128,300,511], 16q/8kv, 64-block pool of 256-token pages."""
    rng = np.random.default_rng(seed)
    return make_prefill([17, 128, 300, 511], num_heads=16, num_kv_heads=8, num_pages=64, rng=rng)


def qwen3_06b_mixed(seed=1):
    """32 prefill seqs L~U[64,2048] + 96 decode seqs ctx~U[256,4096]; 4096-block pool."""
    rng = np.random.default_rng(seed)
    p_lens = rng.integers(64, 2049, size=32)
    d_lens = rng.integers(256, 4097, size=96)
    num_pages = 4096
    # one permutation dealt to the prefill sequences first, then to decode
    perm = rng.permutation(num_pages).astype(np.int32)
    used = pool_pages_needed(p_lens)
    pre = make_prefill(p_lens, num_heads=16, num_kv_heads=8, num_pages=num_pages, perm=perm)
    dec = make_decode(d_lens, num_heads=16, num_kv_heads=8, num_pages=num_pages, perm=perm[used:])
    return pre, dec


def qwen3_8b_decode(seed=2) -> DecodeBatch:
    """256 seqs ctx~U[512,8192], 32q/8kv, 16384-block pool, shuffled blocks."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(512, 8193, size=256)
    return make_decode(lens, num_heads=32, num_kv_heads=8, num_pages=16384, rng=rng)


def qwen3_8b_prefix_prefill(seed=3) -> PrefillBatch:
    """64 seqs, cached prefix P~U[0,4096] in shared blocks + new N~U[128,1024]; 32q/8kv."""
    rng = np.random.default_rng(seed)
    prefix = rng.integers(0, 4097, size=64)
    new = rng.integers(128, 1025, size=64)
    return make_prefix_prefill(prefix, new, num_heads=32, num_kv_heads=8, rng=rng,
                               shared_prefix_tokens=4096)


def qwen3_32b_long_prefill(seed=4) -> PrefillBatch:
    """8 seqs L~U[8192,32768], 64q/8kv, pool sized to fit."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(8192, 32769, size=8)
    return make_prefill(lens, num_heads=64, num_kv_heads=8, rng=rng)


def qwen3_8b_long_prefill(seed=4) -> PrefillBatch:
    """The long prefill's 8 sequence lengths (L~U[8192,32768], same draws)
    at Qwen3-8B's heads: 32q/8kv, pool sized to fit."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(8192, 32769, size=8)
    return make_prefill(lens, num_heads=32, num_kv_heads=8, rng=rng)


def g32_decode(seed=2) -> DecodeBatch:
    """The Qwen3-8B decode batch (256 seqs, ctx~U[512,8192], same draws) with
    32 q heads per kv head: 64q/2kv, so every kv head is read by two blocks
    of 16 q heads."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(512, 8193, size=256)
    return make_decode(lens, num_heads=64, num_kv_heads=2, num_pages=16384, rng=rng)


WORKLOADS = {
    "qwen3_0.6b_prefill": qwen3_06b_prefill,
    "qwen3_0.6b_mixed": qwen3_06b_mixed,
    "qwen3_8b_decode": qwen3_8b_decode,
    "qwen3_8b_prefix_prefill": qwen3_8b_prefix_prefill,
    "qwen3_32b_long_prefill": qwen3_32b_long_prefill,
    "qwen3_8b_long_prefill": qwen3_8b_long_prefill,
    "g32_decode": g32_decode,
}


# ---------------------------------------------------------------------------
# device tensors
# ---------------------------------------------------------------------------
def _randn_bf16(shape, gen, device):
    import torch
    t = torch.empty(shape, dtype=torch.bfloat16, device=device)
    # chunked so that the float32 staging buffer stays small
    flat = t.view(-1)
    step = 1 << 28
    for s in range(0, flat.numel(), step):
        e = min(s + step, flat.numel())
        flat[s:e] = (torch.randn(e - s, generator=gen, device=device, dtype=torch.float32) * 0.5).to(torch.bfloat16)
    return t


def materialize_prefill(pb: PrefillBatch, seed: int, device, fill_pool=True):
    """Device tensors for a prefill batch.

    Returns dict with kv_cache [2, NB, BS, Hkv, d] (pre-existing tokens
    random; copy-on-write tail pages copied from their shared source), q
    [T, H, d], k/v [T, Hkv, d] (new tokens, not yet stored) and int32
    metadata tensors.
    """
    import torch
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    t = len(pb.slot_mapping)
    shape = (2, pb.num_pages, pb.page_size, pb.num_kv_heads, pb.head_dim)
    if fill_pool:
        kv_cache = _randn_bf16(shape, gen, device)
    else:
        kv_cache = torch.zeros(shape, dtype=torch.bfloat16, device=device)
    for dst, src, ntok in getattr(pb, "cow", []):
        kv_cache[:, dst, :ntok] = kv_cache[:, src, :ntok]
    q = _randn_bf16((t, pb.num_heads, pb.head_dim), gen, device)
    k = _randn_bf16((t, pb.num_kv_heads, pb.head_dim), gen, device)
    v = _randn_bf16((t, pb.num_kv_heads, pb.head_dim), gen, device)
    i32 = lambda a: torch.as_tensor(np.ascontiguousarray(a), dtype=torch.int32, device=device)
    return dict(kv_cache=kv_cache, q=q, k=k, v=v, block_tables=i32(pb.block_tables),
                cu_seqlens_q=i32(pb.cu_seqlens_q), cu_seqlens_k=i32(pb.cu_seqlens_k),
                input_positions=i32(pb.input_positions), slot_mapping=i32(pb.slot_mapping))


def materialize_decode(db: DecodeBatch, seed: int, device, kv_cache=None):
    """Device tensors for a decode batch (pool contents random unless given)."""
    import torch
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    if kv_cache is None:
        kv_cache = _randn_bf16((2, db.num_pages, db.page_size, db.num_kv_heads, db.head_dim), gen, device)
    q = _randn_bf16((db.batch, db.num_heads, db.head_dim), gen, device)
    k = _randn_bf16((db.batch, db.num_kv_heads, db.head_dim), gen, device)
    v = _randn_bf16((db.batch, db.num_kv_heads, db.head_dim), gen, device)
    i32 = lambda a: torch.as_tensor(np.ascontiguousarray(a), dtype=torch.int32, device=device)
    return dict(kv_cache=kv_cache, q=q, k=k, v=v, block_tables=i32(db.block_tables),
                context_lens=i32(db.context_lens), input_positions=i32(db.input_positions),
                slot_mapping=i32(db.slot_mapping))


def materialize_mixed(mb: MixedBatch, seed: int, device):
    """Device tensors for a mixed step: random pool (the decode contexts),
    q and new k/v for every row (decode rows first), int32 metadata."""
    import torch
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    pre = mb.prefill
    t = mb.num_tokens
    kv_cache = _randn_bf16((2, pre.num_pages, pre.page_size, pre.num_kv_heads, pre.head_dim), gen, device)
    q = _randn_bf16((t, pre.num_heads, pre.head_dim), gen, device)
    k = _randn_bf16((t, pre.num_kv_heads, pre.head_dim), gen, device)
    v = _randn_bf16((t, pre.num_kv_heads, pre.head_dim), gen, device)
    i32 = lambda a: torch.as_tensor(np.ascontiguousarray(a), dtype=torch.int32, device=device)
    return dict(kv_cache=kv_cache, q=q, k=k, v=v, block_tables=i32(mb.block_tables),
                cu_seqlens_q=i32(mb.cu_seqlens_q), kv_lens=i32(mb.kv_lens),
                input_positions=i32(mb.input_positions), slot_mapping=i32(mb.slot_mapping))


def pool_pages_needed(lens, page_size=PAGE_SIZE) -> int:
    return int(sum(math.ceil(int(n) / page_size) for n in lens))
