"""One launch for a scheduler step that mixes decode and prefill sequences.

The reference engine runs such a step as two jitted calls, decode then
prefill, each padded to a power-of-two bucket (vllm/src/model_runner.py:
310-333; padding 243-255, 286-292).  This entry takes the step unpadded:
sequences ``0 .. num_decodes-1`` are decode sequences (one q row each, the
semantics of decode_paged_attention.py:300-397) and the others are prefill
sequences (prefill_paged_attention.py:407-453, with an explicit kv length
per sequence so a decode-style cached context is allowed).  Both halves run
in a single gfx950 kernel launch.
"""
from __future__ import annotations

import torch

from .. import _lib
from ._common import (as_i32, inv_sqrt_head_dim_bf16, pages_strides, require_bf16, require_device,
                      stream_handle)


def mixed_workspace_bytes(batch: int, num_decodes: int, max_seqlen_q: int, num_heads: int, num_kv_heads: int,
                          head_dim: int, pages_per_seq: int, page_size: int) -> int:
    """Workspace ``mixed_paged_attention`` needs: decode partials (when a
    decode context can span more than one 4096-token chunk) and the work list."""
    return int(_lib.load().pa_mixed_workspace_size(batch, num_decodes, max_seqlen_q, num_heads, num_kv_heads,
                                                   head_dim, pages_per_seq, page_size))


def mixed_paged_attention(
        q: torch.Tensor,
        k_pages: torch.Tensor,
        v_pages: torch.Tensor,
        block_tables: torch.Tensor,
        cu_seqlens_q: torch.Tensor,
        kv_lens: torch.Tensor,
        input_positions: torch.Tensor,
        num_decodes: int,
        *,
        max_seqlen_q: int,
        prefill_scale: float | None = None,
        decode_scale: float = 1.0,
        attn_logits_soft_cap: float | None = None,
        workspace: torch.Tensor | None = None,
        out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Mixed ragged paged attention; q ``[T, H, d]`` -> ``[T, H, d]`` bf16.

    ``k_pages`` / ``v_pages`` are ``[Hkv, NB, BS, d]`` views (any strides);
    ``block_tables [B, P]``, ``cu_seqlens_q [B+1]``, ``kv_lens [B]`` and
    ``input_positions [T]`` are int32.  ``prefill_scale`` defaults to the
    reference prefill's bf16 ``1/sqrt(d)``; ``decode_scale`` defaults to 1
    (the reference decode takes q pre-scaled).  ``max_seqlen_q`` bounds the
    q length of every prefill sequence.
    """
    t_count, num_heads, head_dim = q.shape
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
        raise ValueError(f"head_dim of Q must be the same as that of K/V. Got {head_dim} and {head_dim_k}.")
    if tuple(cu_seqlens_q.shape) != (batch + 1,):
        raise ValueError("cu_seqlens_q must have shape [batch + 1]")
    if tuple(kv_lens.shape) != (batch,):
        raise ValueError("kv_lens must have shape [batch]")
    if tuple(input_positions.shape) != (t_count,):
        raise ValueError("input_positions must have shape [num_tokens]")
    if block_tables.dtype != torch.int32:
        raise ValueError("block_tables must be int32")
    if not 0 <= int(num_decodes) <= batch:
        raise ValueError(f"num_decodes must lie in [0, {batch}], got {num_decodes}")
    for name, t in (("q", q), ("k_pages", k_pages), ("v_pages", v_pages), ("block_tables", block_tables),
                    ("cu_seqlens_q", cu_seqlens_q), ("kv_lens", kv_lens), ("input_positions", input_positions)):
        require_device(name, t)
    require_bf16("q", q)
    require_bf16("k_pages", k_pages)
    require_bf16("v_pages", v_pages)
    if tuple(k_pages.stride()) != tuple(v_pages.stride()):
        raise ValueError("k_pages and v_pages must share strides")
    bt = block_tables if block_tables.stride(-1) == 1 else block_tables.contiguous()
    cu = as_i32("cu_seqlens_q", cu_seqlens_q)
    kl = as_i32("kv_lens", kv_lens)
    pos = as_i32("input_positions", input_positions)
    if out is None:
        out = torch.empty_like(q, memory_format=torch.contiguous_format)
    else:
        require_device("out", out)
        require_bf16("out", out)
        if tuple(out.shape) != tuple(q.shape):
            raise ValueError(f"out must have shape {tuple(q.shape)}")
    need = mixed_workspace_bytes(batch, int(num_decodes), int(max_seqlen_q), num_heads, num_kv_heads, head_dim,
                                 pages_per_sequence, page_size)
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    ws_ptr = workspace.data_ptr()
    ws_bytes = workspace.numel() * workspace.element_size()
    if prefill_scale is None:
        prefill_scale = inv_sqrt_head_dim_bf16(head_dim)
    soft_cap = 0.0 if attn_logits_soft_cap is None else float(attn_logits_soft_cap)
    ps, ss, hs = pages_strides(k_pages)
    _lib.call(
        "pa_mixed",
        q.data_ptr(), q.stride(0), q.stride(1),
        k_pages.data_ptr(), v_pages.data_ptr(), total_num_pages, page_size,
        ps, ss, hs,
        bt.data_ptr(), bt.stride(0), pages_per_sequence,
        cu.data_ptr(), kl.data_ptr(), pos.data_ptr(),
        batch, int(num_decodes), t_count, int(max_seqlen_q),
        num_heads, num_kv_heads, head_dim,
        float(prefill_scale), float(decode_scale), soft_cap,
        out.data_ptr(), out.stride(0), out.stride(1),
        ws_ptr, ws_bytes,
        stream_handle(q))
    return out
