"""Ragged causal GQA paged prefill on gfx950 -- drop-in for
``vllm/kernels/prefill_paged_attention.py:prefill_paged_attention``.

Same positional arguments, keywords, shapes and ``ValueError`` checks as the
reference entry (prefill_paged_attention.py:391-453, checks :189-207,
:430-431).  Tensors are torch tensors on a HIP device; ``k_pages`` /
``v_pages`` are ``[Hkv, NB, BS, d]`` *views* -- any strides with a unit last
stride -- so the engine's native pool ``kv_cache[i]`` (``[NB, BS, Hkv, d]``)
is passed as ``kv_cache[i].permute(2, 0, 1, 3)`` without the full-pool
transpose the reference performs (qwen3.py:177-178).

The Pallas tuning knobs (``block_m``, ``block_h``, ``pages_per_compute_block``,
``k_splits``, ``num_warps``, ``num_stages``, ``interpret``, ``debug``) are
accepted and ignored.  ``mask_value`` only matters for rows with no visible
key, which this implementation returns as zeros.
"""
from __future__ import annotations

import torch

from .. import _lib
from ._common import (DEFAULT_MASK_VALUE, as_i32, check_quantized_pages, inv_sqrt_head_dim_bf16, pages_strides,
                      require_bf16, require_device, stream_handle)


def prefill_paged_attention(
        q: torch.Tensor,
        k_pages: torch.Tensor,
        v_pages: torch.Tensor,
        block_tables: torch.Tensor,
        cu_seqlens: torch.Tensor,
        slot_mapping: torch.Tensor,
        input_positions: torch.Tensor,
        *,
        max_seqlen_bucket: int,
        k_scales_pages: torch.Tensor | None = None,
        v_scales_pages: torch.Tensor | None = None,
        block_m: int = 16,
        block_h: int = 16,
        pages_per_compute_block: int = 8,
        k_splits: int = 8,
        num_warps: int = 8,
        num_stages: int = 2,
        interpret: bool = False,
        debug: bool = False,
        mask_value: float = DEFAULT_MASK_VALUE,
        attn_logits_soft_cap: float | None = None,
        cu_seqlens_k: torch.Tensor | None = None,
        scale: float | None = None,
        out: torch.Tensor | None = None,
        workspace: torch.Tensor | None = None,
) -> torch.Tensor:
    """Paged prefill attention; returns ``[T, H, d]`` bf16.

    Extensions beyond the reference signature (all keyword-only, defaulting
    to the reference behaviour):
      * ``cu_seqlens_k`` -- per-sequence kv lengths including a cached prefix;
        kv index j then sits at position ``j + pos0 - (Lk - Lq)``;
      * ``scale`` -- logit scale (default: bf16(1/sqrt(d)) as prefill...:60);
      * ``out`` -- preallocated output;
      * ``workspace`` -- device bytes for the work list that orders the
        kernel's items by kv length (``pa_prefill_workspace_size``) and, for
        quantized pages (float8 e4m3fn codes, or int8 / uint8 integers, with
        float32 ``[Hkv, NB, BS]`` per-token scales), the pages widened to bf16 ahead of it
        (``pa_prefill_fp8_workspace_size``); allocated when absent or too small.
    """
    del slot_mapping, block_m, pages_per_compute_block, k_splits, num_warps, num_stages
    del interpret, debug, mask_value
    if block_h % 16:
        raise ValueError(f"block_h must divisible by 16, but is {block_h}.")
    total_tokens, num_heads, head_dim = q.shape
    num_kv_heads, total_num_pages, page_size, head_dim_k = k_pages.shape
    batch, pages_per_sequence = block_tables.shape
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
    if tuple(cu_seqlens.shape) != (batch + 1,):
        raise ValueError("cu_seqlens must have shape [batch + 1]")
    if block_tables.dtype != torch.int32:
        raise ValueError("block_tables must be int32")
    if cu_seqlens_k is not None and tuple(cu_seqlens_k.shape) != (batch + 1,):
        raise ValueError("cu_seqlens_k must have shape [batch + 1]")

    code_type = check_quantized_pages(k_pages, v_pages, k_scales_pages, v_scales_pages)
    quantized = code_type is not None
    for name, t in (("q", q), ("k_pages", k_pages), ("v_pages", v_pages), ("block_tables", block_tables),
                    ("cu_seqlens", cu_seqlens), ("input_positions", input_positions)):
        require_device(name, t)
    require_bf16("q", q)
    if not quantized:
        require_bf16("k_pages", k_pages)
        require_bf16("v_pages", v_pages)
    if tuple(k_pages.stride()) != tuple(v_pages.stride()):
        raise ValueError("k_pages and v_pages must share strides")
    bt = block_tables if block_tables.stride(-1) == 1 else block_tables.contiguous()
    cu = as_i32("cu_seqlens", cu_seqlens)
    cuk = as_i32("cu_seqlens_k", cu_seqlens_k) if cu_seqlens_k is not None else None
    pos = as_i32("input_positions", input_positions)
    if out is None:
        out = torch.empty_like(q, memory_format=torch.contiguous_format)
    else:
        require_device("out", out)
        require_bf16("out", out)
        if tuple(out.shape) != tuple(q.shape):
            raise ValueError(f"out must have shape {tuple(q.shape)}")
    if scale is None:
        scale = inv_sqrt_head_dim_bf16(head_dim)
    soft_cap = 0.0 if attn_logits_soft_cap is None else float(attn_logits_soft_cap)
    ps, ss, hs = pages_strides(k_pages)
    lib = _lib.load()
    if quantized:
        need = int(lib.pa_prefill_fp8_workspace_size(batch, pages_per_sequence, page_size, num_kv_heads, head_dim,
                                                     int(max_seqlen_bucket), num_heads))
    else:
        need = int(lib.pa_prefill_workspace_size(batch, int(max_seqlen_bucket), num_heads, num_kv_heads))
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    ws_bytes = workspace.numel() * workspace.element_size()
    if quantized:
        _lib.call(
            "pa_prefill_quant", code_type,
            q.data_ptr(), q.stride(0), q.stride(1),
            k_pages.data_ptr(), v_pages.data_ptr(), k_scales_pages.data_ptr(), v_scales_pages.data_ptr(),
            total_num_pages, page_size, ps, ss, hs,
            k_scales_pages.stride(1), k_scales_pages.stride(0),
            bt.data_ptr(), bt.stride(0), pages_per_sequence,
            cu.data_ptr(), cuk.data_ptr() if cuk is not None else None, pos.data_ptr(),
            batch, total_tokens, int(max_seqlen_bucket),
            num_heads, num_kv_heads, head_dim,
            float(scale), soft_cap,
            out.data_ptr(), out.stride(0), out.stride(1),
            workspace.data_ptr(), ws_bytes,
            stream_handle(q))
        return out
    _lib.call(
        "pa_prefill",
        q.data_ptr(), q.stride(0), q.stride(1),
        k_pages.data_ptr(), v_pages.data_ptr(), total_num_pages, page_size,
        ps, ss, hs,
        bt.data_ptr(), bt.stride(0), pages_per_sequence,
        cu.data_ptr(), cuk.data_ptr() if cuk is not None else None, pos.data_ptr(),
        batch, total_tokens, int(max_seqlen_bucket),
        num_heads, num_kv_heads, head_dim,
        float(scale), soft_cap,
        out.data_ptr(), out.stride(0), out.stride(1),
        workspace.data_ptr(), ws_bytes,
        stream_handle(q))
    return out
