"""Shared argument plumbing for the kernel entry points (torch tensors -> C ABI)."""
from __future__ import annotations

import math

import numpy as np
import torch

# prefill_paged_attention.py:15 / decode_paged_attention.py:31
DEFAULT_MASK_VALUE = -0.7 * float(np.finfo(np.dtype("float32")).max)


def bf16_round(x: float) -> float:
    """The value a Python float takes when JAX weak-types it into bf16."""
    return float(torch.tensor(x, dtype=torch.float32).to(torch.bfloat16).float())


def inv_sqrt_head_dim_bf16(head_dim: int) -> float:
    """``1/sqrt(d)`` as the reference prefill applies it to bf16 q (prefill...:60)."""
    return bf16_round(1.0 / math.sqrt(head_dim))


def require_device(name: str, t: torch.Tensor) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must live on a HIP device (got {t.device}); "
                         "the paged-attention path has no CPU implementation")


def require_bf16(name: str, t: torch.Tensor) -> None:
    if t.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bfloat16, got {t.dtype}")
    if t.stride(-1) != 1:
        raise ValueError(f"{name} must be contiguous in its last dimension")


def as_i32(name: str, t: torch.Tensor) -> torch.Tensor:
    """int32 metadata, contiguous (copies only if it is not already)."""
    if t.dtype != torch.int32:
        raise ValueError(f"{name} must be int32, got {t.dtype}")
    return t if t.is_contiguous() else t.contiguous()


def stream_handle(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def pages_strides(k_pages: torch.Tensor):
    """(page, slot, head) element strides of a [Hkv, NB, BS, d] view."""
    hs, ps, ss, ds = k_pages.stride()
    if ds != 1:
        raise ValueError("k_pages must be contiguous in head_dim")
    return ps, ss, hs
