"""Split-K paged GQA decode on gfx950 -- drop-in for
``vllm/kernels/decode_paged_attention.py:decode_paged_attention``.

Same arguments, shapes and ``ValueError`` checks as the reference entry
(decode_paged_attention.py:300-372).  Quantized pages
(``k_scales_pages`` / ``v_scales_pages``, decode...:158-159,206-217) are float8
e4m3fn codes, or int8 / uint8 integers, with float32 per-token scales
``[Hkv, NB, BS]``.  As in the reference, q is expected to
be pre-scaled (the caller divides by sqrt(d), qwen3.py:207) and no scale is
applied inside; the extra keyword ``scale`` lets a caller fold the scale into
the kernel instead.  ``lengths=None`` attends to every slot of the block
table, like the reference's unmasked path (decode...:133-134).

The Pallas tuning knobs are accepted and ignored; the reference's assertion
that the table width divides ``k_splits`` (decode...:175-177) is a limitation
of its grid, not of the operation, and is not reproduced.
"""
from __future__ import annotations

import torch

from .. import _lib
from ._common import (DEFAULT_MASK_VALUE, as_i32, check_quantized_pages, pages_strides, require_bf16,
                      require_device, stream_handle)


def decode_workspace_bytes(batch: int, num_heads: int, head_dim: int, pages_per_seq: int,
                           page_size: int) -> int:
    return int(_lib.load().pa_decode_workspace_size(batch, num_heads, head_dim, pages_per_seq, page_size))


def decode_paged_attention(
        q: torch.Tensor,
        k_pages: torch.Tensor,
        v_pages: torch.Tensor,
        block_tables: torch.Tensor,
        lengths: torch.Tensor | None,
        k_scales_pages: torch.Tensor | None = None,
        v_scales_pages: torch.Tensor | None = None,
        *,
        block_h: int = 16,
        pages_per_compute_block: int = 8,
        k_splits: int = 16,
        num_warps: int = 8,
        num_stages: int = 2,
        interpret: bool = False,
        debug: bool = False,
        mask_value: float = DEFAULT_MASK_VALUE,
        attn_logits_soft_cap: float | None = None,
        scale: float = 1.0,
        workspace: torch.Tensor | None = None,
        out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Paged decode attention; q ``[B, H, d]`` -> ``[B, H, d]`` bf16."""
    del pages_per_compute_block, k_splits, num_warps, num_stages, interpret, debug, mask_value
    batch_size, num_heads, head_dim = q.shape
    num_kv_heads, total_num_pages, page_size, head_dim_k = k_pages.shape
    batch_size_paged_indices, pages_per_sequence = block_tables.shape

    if tuple(k_pages.shape) != tuple(v_pages.shape):
        raise ValueError(
            f"k_pages and v_pages must have the same shape. Got {tuple(k_pages.shape)} and"
            f" {tuple(v_pages.shape)}")
    if num_heads % num_kv_heads != 0:
        raise ValueError(
            "Number of Q heads must be divisible by number of KV heads. Got"
            f" {num_heads} and {num_kv_heads}.")
    if head_dim_k != head_dim:
        raise ValueError(
            "head_dim of Q must be the same as that of K/V. Got"
            f" {head_dim} and {head_dim_k}.")
    if batch_size_paged_indices != batch_size:
        raise ValueError("`block_tables` and `q` must have the same batch size")
    if lengths is not None:
        if tuple(lengths.shape) != (batch_size,):
            raise ValueError("`lengths` and `q` must have the same batch size")
        if lengths.dtype != torch.int32:
            raise ValueError(f"The dtype of `lengths` must be int32. Got {lengths.dtype}")
    if block_h % 16:
        raise ValueError(f"block_h must divisible by 16, but is {block_h}.")
    code_type = check_quantized_pages(k_pages, v_pages, k_scales_pages, v_scales_pages)
    quantized = code_type is not None

    for name, t in (("q", q), ("k_pages", k_pages), ("v_pages", v_pages), ("block_tables", block_tables)):
        require_device(name, t)
    require_bf16("q", q)
    if not quantized:
        require_bf16("k_pages", k_pages)
        require_bf16("v_pages", v_pages)
    if block_tables.dtype != torch.int32:
        raise ValueError("block_tables must be int32")
    if tuple(k_pages.stride()) != tuple(v_pages.stride()):
        raise ValueError("k_pages and v_pages must share strides")
    bt = block_tables if block_tables.stride(-1) == 1 else block_tables.contiguous()
    if lengths is None:
        lens = torch.full((batch_size,), pages_per_sequence * page_size, dtype=torch.int32, device=q.device)
    else:
        require_device("lengths", lengths)
        lens = as_i32("lengths", lengths)
    if out is None:
        out = torch.empty_like(q, memory_format=torch.contiguous_format)
    else:
        require_device("out", out)
        require_bf16("out", out)
        if tuple(out.shape) != tuple(q.shape):
            raise ValueError(f"out must have shape {tuple(q.shape)}")
    need = decode_workspace_bytes(batch_size, num_heads, head_dim, max(pages_per_sequence, 1), page_size)
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    soft_cap = 0.0 if attn_logits_soft_cap is None else float(attn_logits_soft_cap)
    ps, ss, hs = pages_strides(k_pages)
    if quantized:
        _lib.call(
            "pa_decode_quant", code_type,
            q.data_ptr(), q.stride(0), q.stride(1),
            k_pages.data_ptr(), v_pages.data_ptr(), k_scales_pages.data_ptr(), v_scales_pages.data_ptr(),
            total_num_pages, page_size, ps, ss, hs,
            k_scales_pages.stride(1), k_scales_pages.stride(0),
            bt.data_ptr(), bt.stride(0), pages_per_sequence,
            lens.data_ptr(), batch_size,
            num_heads, num_kv_heads, head_dim,
            float(scale), soft_cap,
            out.data_ptr(), out.stride(0), out.stride(1),
            workspace.data_ptr(), workspace.numel() * workspace.element_size(),
            stream_handle(q))
        return out
    _lib.call(
        "pa_decode",
        q.data_ptr(), q.stride(0), q.stride(1),
        k_pages.data_ptr(), v_pages.data_ptr(), total_num_pages, page_size,
        ps, ss, hs,
        bt.data_ptr(), bt.stride(0), pages_per_sequence,
        lens.data_ptr(), batch_size,
        num_heads, num_kv_heads, head_dim,
        float(scale), soft_cap,
        out.data_ptr(), out.stride(0), out.stride(1),
        workspace.data_ptr(), workspace.numel() * workspace.element_size(),
        stream_handle(q))
    return out
