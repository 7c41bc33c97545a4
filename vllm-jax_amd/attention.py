"""The layer seam: ``attention(kv_cache, q, k, v, metadata) -> (kv_cache, out)``.

Drop-in for ``vllm/model/qwen3.py:attention`` (qwen3.py:172-218) and its
metadata types (qwen3.py:17-37), with torch tensors on a HIP device.
Per layer it (1) stores the new K/V tokens into the paged pool through the
slot mapping (``_update_kv_cache``, qwen3.py:105-111) and (2) runs the paged
prefill or decode kernel.  Differences from the reference, all deliberate:

* the pool is updated in place and the same tensor is returned (the
  reference is functional and copies the pool every step without donation);
* no ``[NB, BS, Hkv, d] -> [Hkv, NB, BS, d]`` transpose (qwen3.py:177-178,
  196-197): the kernels read the native layout through strides;
* decode folds ``1/bf16(sqrt(d))`` into the kernel instead of pre-scaling q
  in bf16 (qwen3.py:207);
* prefill passes ``cu_seqlens_k`` so a cached prefix can precede the new
  tokens (with ``cu_seqlens_k == cu_seqlens_q``, the engine's case, the
  semantics are the reference's);
* a third metadata type, ``MixedAttentionMetadata``, runs a step's decode
  and prefill sequences together in one unpadded launch (the reference runs
  them as two padded jitted calls, model_runner.py:310-333).
"""
from __future__ import annotations

import os
from dataclasses import dataclass, field
from typing import Optional, Tuple, Union

import torch

from . import _lib
from .kernels._common import bf16_round, require_bf16, require_device, stream_handle
from .kernels.decode_paged_attention import decode_paged_attention
from .kernels.mixed_paged_attention import mixed_paged_attention
from .kernels.prefill_paged_attention import prefill_paged_attention

USE_DECODE_PAGED_ATTENTION_KERNEL = True
USE_PREFILL_PAGED_ATTENTION_KERNEL = True


@dataclass
class DecodeAttentionMetadata:
    """qwen3.py:17-22."""
    input_positions: torch.Tensor
    slot_mapping: torch.Tensor
    block_tables: torch.Tensor
    context_lens: torch.Tensor


@dataclass
class PrefillAttentionMetadata:
    """qwen3.py:25-34 (``max_seqlen_bucket`` is static in the reference)."""
    input_positions: torch.Tensor
    slot_mapping: torch.Tensor
    block_tables: torch.Tensor
    cu_seqlens_q: torch.Tensor
    cu_seqlens_k: torch.Tensor
    max_seqlen_q: torch.Tensor
    max_seqlen_k: torch.Tensor
    max_seqlen_bucket: int = field(default=0)


@dataclass
class MixedAttentionMetadata:
    """One scheduler step, unpadded: sequences ``0 .. num_decodes-1`` are
    decode sequences (one q row, ``kv_lens`` = context length including the
    new token, as ``context_lens`` of qwen3.py:17-22), the rest prefill
    sequences (q rows ``cu_seqlens_q[b] .. cu_seqlens_q[b+1]``, kv length
    ``kv_lens[b]``, positions as qwen3.py:25-34).  ``max_seqlen_q`` bounds
    every prefill q length."""
    input_positions: torch.Tensor
    slot_mapping: torch.Tensor
    block_tables: torch.Tensor
    cu_seqlens_q: torch.Tensor
    kv_lens: torch.Tensor
    num_decodes: int
    max_seqlen_q: int


AttentionMetadata = Union[DecodeAttentionMetadata, PrefillAttentionMetadata, MixedAttentionMetadata]


def check_slot_mapping(slot_mapping: torch.Tensor, num_slots: int) -> None:
    """Debug check of the store's contract: no two tokens may write one slot.

    The reference's scatter (``.at[slot].set(..., mode="drop")``,
    qwen3.py:109-110) leaves the winner of a duplicated slot unspecified, and
    so do the store kernels here (the tokens' rows race).  Slots outside
    ``[0, num_slots)`` are skipped by the store and ignored here.  Raises
    ``ValueError`` naming the first duplicated slot.  It synchronises the
    device, so the stores run it only when the environment sets
    ``PA_CHECK_SLOTS=1``.
    """
    s = slot_mapping.reshape(-1).to(torch.int64)
    s = s[(s >= 0) & (s < num_slots)]
    if s.numel() < 2:
        return
    u, counts = torch.unique(s, return_counts=True)
    dup = u[counts > 1]
    if dup.numel():
        first = int(dup[0])
        tokens = torch.nonzero(slot_mapping.reshape(-1).to(torch.int64) == first).reshape(-1)[:4].tolist()
        raise ValueError(f"slot_mapping writes {dup.numel()} slot(s) more than once: slot {first} "
                         f"from tokens {tokens}")


def _checking_slots() -> bool:
    return os.environ.get("PA_CHECK_SLOTS", "") == "1"


def update_kv_cache(kv_cache: torch.Tensor, slot_mapping: torch.Tensor, k: torch.Tensor,
                    v: torch.Tensor) -> torch.Tensor:
    """In-place KV store: ``kv_cache[0].flat[slot[t]] = k[t]``, same for v.

    ``kv_cache`` is ``[2, NB, BS, Hkv, d]`` (model_runner.py:195); ``k``/``v``
    are ``[T, Hkv, d]``.  Slots < 0 (padding tokens) and slots past the pool
    are skipped (qwen3.py:109-110 uses ``mode="drop"``).
    """
    for name, t in (("kv_cache", kv_cache), ("slot_mapping", slot_mapping), ("k", k), ("v", v)):
        require_device(name, t)
    require_bf16("kv_cache", kv_cache)
    require_bf16("k", k)
    require_bf16("v", v)
    if kv_cache.dim() != 5 or kv_cache.shape[0] != 2:
        raise ValueError(f"kv_cache must be [2, NB, BS, Hkv, d], got {tuple(kv_cache.shape)}")
    _, nb, bs, hkv, d = kv_cache.shape
    if k.dim() != 3 or tuple(k.shape[1:]) != (hkv, d) or tuple(v.shape) != tuple(k.shape):
        raise ValueError(f"k/v must be [T, {hkv}, {d}], got {tuple(k.shape)} and {tuple(v.shape)}")
    if slot_mapping.dtype != torch.int32 or tuple(slot_mapping.shape) != (k.shape[0],):
        raise ValueError("slot_mapping must be int32 of shape [T]")
    if _checking_slots():
        check_slot_mapping(slot_mapping, nb * bs)
    kc, vc = kv_cache[0], kv_cache[1]
    sm = slot_mapping if slot_mapping.is_contiguous() else slot_mapping.contiguous()
    _lib.call(
        "pa_kv_store",
        k.data_ptr(), k.stride(0), k.stride(1),
        v.data_ptr(), v.stride(0), v.stride(1),
        sm.data_ptr(), k.shape[0], hkv, d,
        kc.data_ptr(), vc.data_ptr(), nb, bs,
        kc.stride(0), kc.stride(1), kc.stride(2),
        stream_handle(k))
    return kv_cache


# reference name (qwen3.py:105)
_update_kv_cache = update_kv_cache


def qk_norm_rope_store(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_norm_weight: torch.Tensor,
                       k_norm_weight: torch.Tensor, positions: torch.Tensor, slot_mapping: torch.Tensor,
                       kv_cache: torch.Tensor, *, eps: float, rope_theta: float,
                       rope_scaling: Optional[dict] = None,
                       out: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """The layer step between the projections and attention, in one kernel:
    ``q = rope(q_norm(q))``, ``k = rope(k_norm(k))`` (qwen3.py:286-296 with
    apply_rope qwen3.py:59-78) and the K/V store of ``_update_kv_cache``
    (qwen3.py:105-111), in place.  Returns ``(q_out, kv_cache)``; ``out``
    may be ``q`` itself.  ``rope_scaling`` of type linear/dynamic divides the
    positions by its factor (qwen3.py:48-56); other types leave them as is.
    """
    for name, t in (("q", q), ("k", k), ("v", v), ("q_norm_weight", q_norm_weight),
                    ("k_norm_weight", k_norm_weight), ("positions", positions),
                    ("slot_mapping", slot_mapping), ("kv_cache", kv_cache)):
        require_device(name, t)
    for name, t in (("q", q), ("k", k), ("v", v), ("q_norm_weight", q_norm_weight),
                    ("k_norm_weight", k_norm_weight), ("kv_cache", kv_cache)):
        require_bf16(name, t)
    if kv_cache.dim() != 5 or kv_cache.shape[0] != 2:
        raise ValueError(f"kv_cache must be [2, NB, BS, Hkv, d], got {tuple(kv_cache.shape)}")
    _, nb, bs, hkv, d = kv_cache.shape
    if q.dim() != 3 or q.shape[-1] != d:
        raise ValueError(f"q must be [T, H, {d}], got {tuple(q.shape)}")
    t_count, h = q.shape[0], q.shape[1]
    if tuple(k.shape) != (t_count, hkv, d) or tuple(v.shape) != (t_count, hkv, d):
        raise ValueError(f"k/v must be [{t_count}, {hkv}, {d}], got {tuple(k.shape)} and {tuple(v.shape)}")
    if tuple(q_norm_weight.shape) != (d,) or tuple(k_norm_weight.shape) != (d,):
        raise ValueError("norm weights must be [head_dim]")
    for name, t in (("positions", positions), ("slot_mapping", slot_mapping)):
        if t.dtype != torch.int32 or tuple(t.shape) != (t_count,):
            raise ValueError(f"{name} must be int32 of shape [T]")
    factor = 1.0
    if rope_scaling is not None and rope_scaling.get("type") in {"linear", "dynamic"}:
        factor = float(rope_scaling.get("factor", 1.0))
    if _checking_slots():
        check_slot_mapping(slot_mapping, nb * bs)
    if out is None:
        out = torch.empty_like(q)
    kc, vc = kv_cache[0], kv_cache[1]
    pos = positions.contiguous()
    sm = slot_mapping.contiguous()
    qw, kw = q_norm_weight.contiguous(), k_norm_weight.contiguous()
    _lib.call(
        "pa_qk_norm_rope_store",
        q.data_ptr(), q.stride(0), q.stride(1),
        k.data_ptr(), k.stride(0), k.stride(1),
        v.data_ptr(), v.stride(0), v.stride(1),
        qw.data_ptr(), kw.data_ptr(), float(eps), float(rope_theta), factor,
        pos.data_ptr(), sm.data_ptr(), t_count, h, hkv, d,
        out.data_ptr(), out.stride(0), out.stride(1),
        kc.data_ptr(), vc.data_ptr(), nb, bs, kc.stride(0), kc.stride(1), kc.stride(2),
        stream_handle(q))
    return out, kv_cache


def update_kv_cache_fp8(kv_codes: torch.Tensor, kv_scales: torch.Tensor, slot_mapping: torch.Tensor,
                        k: torch.Tensor, v: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Quantising KV store into float8 pages, in place: ``kv_codes`` is the
    pool ``[2, NB, BS, Hkv, d]`` of float8_e4m3fn codes and
    ``kv_scales`` ``[2, Hkv, NB, BS]`` float32 (index 0 = K, 1 = V; each half
    is the reference's ``k_scales_pages`` layout).  Each (token, kv head) row
    is divided by its scale s and rounded to e4m3 (round to nearest even); s
    is the smallest power of two with max|row| / s <= 448 (at least 2^-126).
    Slots outside the pool are skipped.
    Returns ``(kv_codes, kv_scales)``."""
    if kv_codes.dim() != 5 or kv_codes.shape[0] != 2 or kv_codes.dtype != torch.float8_e4m3fn:
        raise ValueError("kv_codes must be a [2, NB, BS, Hkv, d] float8_e4m3fn pool")
    for name, t in (("kv_codes", kv_codes), ("kv_scales", kv_scales), ("slot_mapping", slot_mapping),
                    ("k", k), ("v", v)):
        require_device(name, t)
    require_bf16("k", k)
    require_bf16("v", v)
    _, nb, bs, hkv, d = kv_codes.shape
    if tuple(kv_scales.shape) != (2, hkv, nb, bs) or kv_scales.dtype != torch.float32:
        raise ValueError(f"kv_scales must be float32 [2, {hkv}, {nb}, {bs}]")
    if tuple(k.shape[1:]) != (hkv, d) or tuple(v.shape) != tuple(k.shape):
        raise ValueError("k / v must be [T, Hkv, d]")
    t_count = k.shape[0]
    if slot_mapping.dtype != torch.int32 or tuple(slot_mapping.shape) != (t_count,):
        raise ValueError("slot_mapping must be int32 of shape [T]")
    if _checking_slots():
        check_slot_mapping(slot_mapping, nb * bs)
    kc, vc = kv_codes[0], kv_codes[1]
    ks, vs = kv_scales[0], kv_scales[1]
    sm = slot_mapping.contiguous()
    _lib.call("pa_kv_store_fp8", k.data_ptr(), k.stride(0), k.stride(1), v.data_ptr(), v.stride(0), v.stride(1),
              sm.data_ptr(), t_count, hkv, d, kc.data_ptr(), vc.data_ptr(), ks.data_ptr(), vs.data_ptr(),
              nb, bs, kc.stride(0), kc.stride(1), kc.stride(2), ks.stride(1), ks.stride(2), ks.stride(0),
              stream_handle(k))
    return kv_codes, kv_scales


def attention(kv_cache: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
              metadata: AttentionMetadata) -> Tuple[torch.Tensor, torch.Tensor]:
    """qwen3.py:172-218 on gfx950 kernels; returns ``(kv_cache, out)``."""
    kv_cache = update_kv_cache(kv_cache, metadata.slot_mapping, k, v)
    return kv_cache, attention_stored(kv_cache, q, metadata)


def qwen3_attention_core(kv_cache: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                         q_norm_weight: torch.Tensor, k_norm_weight: torch.Tensor,
                         metadata: AttentionMetadata, *, eps: float, rope_theta: float,
                         rope_scaling: Optional[dict] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Everything of ``Qwen3Attention.__call__`` between the q/k/v
    projections and o_proj (qwen3.py:287-299): q/k RMSNorm + RoPE and the KV
    store in one fused kernel, then paged attention.  Returns
    ``(kv_cache, out)``."""
    q_rot, kv_cache = qk_norm_rope_store(q, k, v, q_norm_weight, k_norm_weight, metadata.input_positions,
                                         metadata.slot_mapping, kv_cache, eps=eps, rope_theta=rope_theta,
                                         rope_scaling=rope_scaling)
    return kv_cache, attention_stored(kv_cache, q_rot, metadata)


def attention_stored(kv_cache: torch.Tensor, q: torch.Tensor, metadata: AttentionMetadata) -> torch.Tensor:
    """The attention part of qwen3.py:175-218 for K/V already in the pool."""
    if not (USE_PREFILL_PAGED_ATTENTION_KERNEL and USE_DECODE_PAGED_ATTENTION_KERNEL):
        raise NotImplementedError("the dense fallbacks of qwen3.py:120-169 are not part of this library")
    k_pages = kv_cache[0].permute(2, 0, 1, 3)   # [Hkv, NB, BS, d] view
    v_pages = kv_cache[1].permute(2, 0, 1, 3)
    if isinstance(metadata, MixedAttentionMetadata):
        head_dim = q.shape[-1]
        outputs = mixed_paged_attention(
            q, k_pages, v_pages, metadata.block_tables, metadata.cu_seqlens_q, metadata.kv_lens,
            metadata.input_positions, metadata.num_decodes, max_seqlen_q=metadata.max_seqlen_q,
            decode_scale=1.0 / bf16_round(float(head_dim) ** 0.5))
    elif isinstance(metadata, PrefillAttentionMetadata):
        outputs = prefill_paged_attention(
            q, k_pages, v_pages, metadata.block_tables, metadata.cu_seqlens_q,
            metadata.slot_mapping, metadata.input_positions,
            max_seqlen_bucket=metadata.max_seqlen_bucket,
            cu_seqlens_k=metadata.cu_seqlens_k)
    else:
        head_dim = q.shape[-1]
        outputs = decode_paged_attention(
            q, k_pages, v_pages, metadata.block_tables, metadata.context_lens,
            scale=1.0 / bf16_round(float(head_dim) ** 0.5))
    return outputs


def gather_kv(cache: torch.Tensor, block_tables: torch.Tensor, lengths: torch.Tensor) -> torch.Tensor:
    """Dense ``[B, P*BS, Hkv, d]`` context of each sequence through its block
    table (test/debug helper; the address math of prefill...:79-82)."""
    for name, t in (("cache", cache), ("block_tables", block_tables), ("lengths", lengths)):
        require_device(name, t)
    require_bf16("cache", cache)
    nb, bs, hkv, d = cache.shape
    b, p = block_tables.shape
    bt = block_tables.contiguous()
    ln = lengths.contiguous()
    out = torch.empty((b, p * bs, hkv, d), dtype=cache.dtype, device=cache.device)
    _lib.call("pa_gather_kv", cache.data_ptr(), nb, bs, cache.stride(0), cache.stride(1), cache.stride(2),
              bt.data_ptr(), bt.stride(0), p, ln.data_ptr(), b, hkv, d, out.data_ptr(), stream_handle(cache))
    return out
