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


# dtype of quantized pages -> code type of pa_decode_quant / pa_prefill_quant
_CODE_TYPES = {torch.float8_e4m3fn: 0, torch.int8: 1, torch.uint8: 2}


def check_quantized_pages(k_pages: torch.Tensor, v_pages: torch.Tensor, k_scales_pages, v_scales_pages):
    """Validate quantized pages with per-token scales (the k_scales_pages /
    v_scales_pages arguments of the reference kernels, decode...:206-217 and
    prefill...:255-266).  Returns None for unquantized pages, else the code
    type of the pages: float8_e4m3fn codes, or int8 / uint8 integers, which
    the reference casts to q's dtype as integers (decode...:72-75,
    prefill...:84-85)."""
    if k_scales_pages is None and v_scales_pages is None:
        return None
    if k_scales_pages is None or v_scales_pages is None:
        raise ValueError("k_scales_pages and v_scales_pages must be given together")
    num_kv_heads, total_num_pages, page_size = k_pages.shape[:3]
    for name, t in (("k_scales_pages", k_scales_pages), ("v_scales_pages", v_scales_pages)):
        if tuple(t.shape) != (num_kv_heads, total_num_pages, page_size):
            raise ValueError(f"{name} must have shape {(num_kv_heads, total_num_pages, page_size)}, "
                             f"got {tuple(t.shape)}")
        if t.dtype != torch.float32:
            raise ValueError(f"{name} must be float32, got {t.dtype}")
        if t.stride(2) != 1:
            raise ValueError(f"{name} must be contiguous over the slots of a page")
    if tuple(k_scales_pages.stride()) != tuple(v_scales_pages.stride()):
        raise ValueError("k_scales_pages and v_scales_pages must share strides")
    for name, t in (("k_pages", k_pages), ("v_pages", v_pages)):
        if t.dtype not in _CODE_TYPES:
            # The reference casts pages of any dtype to q's dtype before the
            # dot; the kernels take 1-byte codes only.
            raise NotImplementedError(f"{name} of quantized pages must be float8_e4m3fn, int8 or uint8, "
                                      f"got {t.dtype}")
        if t.stride(-1) != 1:
            raise ValueError(f"{name} must be contiguous in its last dimension")
    if k_pages.dtype != v_pages.dtype:
        raise ValueError(f"k_pages and v_pages must have the same dtype, got {k_pages.dtype} and {v_pages.dtype}")
    require_device("k_scales_pages", k_scales_pages)
    require_device("v_scales_pages", v_scales_pages)
    return _CODE_TYPES[k_pages.dtype]
