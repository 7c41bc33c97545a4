"""ctypes binding of libpaged_attention.so (the gfx950 C ABI).

The signatures mirror ``include/paged_attention.h``.  Loading fails loudly:
there is no CPU or PyTorch fallback for any entry point.
"""
from __future__ import annotations

import ctypes
import os
import threading

from . import build as _build

_LOCK = threading.Lock()
_LIB = None
ABI_VERSION = 2  # pa_abi_version() of a library these bindings fit

c_i32, c_i64, c_f32, c_sz, c_vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_size_t, ctypes.c_void_p

# name -> (restype, argtypes)
SIGNATURES = {
    "pa_last_error": (ctypes.c_char_p, []),
    "pa_abi_version": (ctypes.c_int, []),  # must equal ABI_VERSION
    "pa_kv_store": (ctypes.c_int, [
        c_vp, c_i64, c_i64,            # k, k_tok_stride, k_head_stride
        c_vp, c_i64, c_i64,            # v, ...
        c_vp, c_i32,                   # slot_mapping, num_tokens
        c_i32, c_i32,                  # num_kv_heads, head_dim
        c_vp, c_vp,                    # k_cache, v_cache
        c_i32, c_i32,                  # num_pages, page_size
        c_i64, c_i64, c_i64,           # page/slot/head strides
        c_vp,                          # stream
    ]),
    "pa_gather_kv": (ctypes.c_int, [
        c_vp, c_i32, c_i32, c_i64, c_i64, c_i64,
        c_vp, c_i64, c_i32,
        c_vp, c_i32,
        c_i32, c_i32, c_vp, c_vp,
    ]),
    "pa_decode_workspace_size": (c_sz, [c_i32, c_i32, c_i32, c_i32, c_i32]),
    "pa_decode": (ctypes.c_int, [
        c_vp, c_i64, c_i64,            # q
        c_vp, c_vp, c_i32, c_i32,      # caches, num_pages, page_size
        c_i64, c_i64, c_i64,           # strides
        c_vp, c_i64, c_i32,            # block_tables, bt_stride, pages_per_seq
        c_vp, c_i32,                   # lengths, batch
        c_i32, c_i32, c_i32,           # heads, kv heads, head_dim
        c_f32, c_f32,                  # scale, soft_cap
        c_vp, c_i64, c_i64,            # out
        c_vp, c_sz, c_vp,              # workspace, bytes, stream
    ]),
    "pa_decode_noalloc": (ctypes.c_int, [
        c_vp, c_i64, c_i64,            # q
        c_vp, c_vp, c_i32, c_i32,      # caches, num_pages, page_size
        c_i64, c_i64, c_i64,           # strides
        c_vp, c_i64, c_i32,            # block_tables, bt_stride, pages_per_seq
        c_vp, c_i32,                   # lengths, batch
        c_i32, c_i32, c_i32,           # heads, kv heads, head_dim
        c_f32, c_f32,                  # scale, soft_cap
        c_vp, c_i64, c_i64,            # out
        c_vp,                          # stream (no workspace)
    ]),
    "pa_decode_noalloc_max_workspace": (c_sz, []),
    "pa_prefill": (ctypes.c_int, [
        c_vp, c_i64, c_i64,            # q
        c_vp, c_vp, c_i32, c_i32,      # caches, num_pages, page_size
        c_i64, c_i64, c_i64,           # strides
        c_vp, c_i64, c_i32,            # block_tables, bt_stride, pages_per_seq
        c_vp, c_vp, c_vp,              # cu_seqlens_q, cu_seqlens_k, input_positions
        c_i32, c_i32, c_i32,           # batch, num_tokens, max_seqlen_q
        c_i32, c_i32, c_i32,           # heads, kv heads, head_dim
        c_f32, c_f32,                  # scale, soft_cap
        c_vp, c_i64, c_i64,            # out
        c_vp, c_sz,                    # workspace (work list, may be NULL), bytes
        c_vp,                          # stream
    ]),
    "pa_prefill_workspace_size": (c_sz, [c_i32, c_i32, c_i32, c_i32]),
    "pa_qk_norm_rope_store": (ctypes.c_int, [
        c_vp, c_i64, c_i64,            # q
        c_vp, c_i64, c_i64,            # k
        c_vp, c_i64, c_i64,            # v
        c_vp, c_vp,                    # q_norm_weight, k_norm_weight
        c_f32, c_f32, c_f32,           # eps, rope_theta, rope_scaling_factor
        c_vp, c_vp,                    # positions, slot_mapping
        c_i32, c_i32, c_i32, c_i32,    # num_tokens, num_heads, num_kv_heads, head_dim
        c_vp, c_i64, c_i64,            # q_out
        c_vp, c_vp, c_i32, c_i32,      # caches, num_pages, page_size
        c_i64, c_i64, c_i64,           # page/slot/head strides
        c_vp,                          # stream
    ]),
    "pa_kv_store_fp8": (ctypes.c_int, [
        c_vp, c_i64, c_i64,            # k
        c_vp, c_i64, c_i64,            # v
        c_vp, c_i32,                   # slot_mapping, num_tokens
        c_i32, c_i32,                  # num_kv_heads, head_dim
        c_vp, c_vp, c_vp, c_vp,        # k/v code pools, k/v scale pools
        c_i32, c_i32,                  # num_pages, page_size
        c_i64, c_i64, c_i64,           # code page/slot/head strides (bytes)
        c_i64, c_i64, c_i64,           # scale page/slot/head strides (floats)
        c_vp,                          # stream
    ]),
    "pa_decode_fp8": (ctypes.c_int, [
        c_vp, c_i64, c_i64,            # q
        c_vp, c_vp, c_vp, c_vp,        # k/v codes, k/v scales
        c_i32, c_i32,                  # num_pages, page_size
        c_i64, c_i64, c_i64,           # code strides (bytes)
        c_i64, c_i64,                  # scale page/head strides (floats)
        c_vp, c_i64, c_i32,            # block_tables, bt_stride, pages_per_seq
        c_vp, c_i32,                   # lengths, batch
        c_i32, c_i32, c_i32,           # heads, kv heads, head_dim
        c_f32, c_f32,                  # scale, soft_cap
        c_vp, c_i64, c_i64,            # out
        c_vp, c_sz, c_vp,              # workspace, bytes, stream
    ]),
    "pa_prefill_fp8_workspace_size": (c_sz, [c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32]),
    "pa_prefill_fp8": (ctypes.c_int, [
        c_vp, c_i64, c_i64,            # q
        c_vp, c_vp, c_vp, c_vp,        # k/v codes, k/v scales
        c_i32, c_i32,                  # num_pages, page_size
        c_i64, c_i64, c_i64,           # code strides (bytes)
        c_i64, c_i64,                  # scale page/head strides (floats)
        c_vp, c_i64, c_i32,            # block_tables, bt_stride, pages_per_seq
        c_vp, c_vp, c_vp,              # cu_seqlens_q, cu_seqlens_k, input_positions
        c_i32, c_i32, c_i32,           # batch, num_tokens, max_seqlen_q
        c_i32, c_i32, c_i32,           # heads, kv heads, head_dim
        c_f32, c_f32,                  # scale, soft_cap
        c_vp, c_i64, c_i64,            # out
        c_vp, c_sz, c_vp,              # workspace, bytes, stream
    ]),
    # block manager (include/block_manager.h)
    "pa_bm_create": (c_vp, [c_i32, c_i32, c_i32]),
    "pa_bm_destroy": (None, [c_vp]),
    "pa_bm_num_free_blocks": (c_i32, [c_vp]),
    "pa_bm_can_allocate": (ctypes.c_int, [c_vp, c_i64, c_vp, c_i32, c_i32]),
    "pa_bm_allocate": (ctypes.c_int, [c_vp, c_i64, c_vp, c_i32, c_i32]),
    "pa_bm_num_cached_tokens": (c_i32, [c_vp, c_i64]),
    "pa_bm_block_table": (c_i32, [c_vp, c_i64, c_vp, c_i32]),
    "pa_bm_fork": (ctypes.c_int, [c_vp, c_i64, c_i64]),
    "pa_bm_deallocate": (ctypes.c_int, [c_vp, c_i64]),
    "pa_bm_ref_count": (c_i32, [c_vp, c_i32]),
    "pa_bm_take_copies": (c_i32, [c_vp, c_vp, c_vp, c_i32]),
    "pa_copy_blocks": (ctypes.c_int, [
        c_vp, c_vp, c_i32, c_i32,      # caches, num_pages, page_size
        c_i64, c_i64, c_i64,           # page/slot/head strides
        c_i32, c_i32,                  # num_kv_heads, head_dim
        c_vp, c_vp, c_i32,             # src, dst, num_copies
        c_vp,                          # stream
    ]),
    "pa_mixed_workspace_size": (c_sz, [c_i32] * 8),
    "pa_mixed": (ctypes.c_int, [
        c_vp, c_i64, c_i64,            # q
        c_vp, c_vp, c_i32, c_i32,      # caches, num_pages, page_size
        c_i64, c_i64, c_i64,           # strides
        c_vp, c_i64, c_i32,            # block_tables, bt_stride, pages_per_seq
        c_vp, c_vp, c_vp,              # cu_seqlens_q, kv_lens, input_positions
        c_i32, c_i32, c_i32, c_i32,    # batch, num_decodes, num_tokens, max_seqlen_q
        c_i32, c_i32, c_i32,           # heads, kv heads, head_dim
        c_f32, c_f32, c_f32,           # prefill_scale, decode_scale, soft_cap
        c_vp, c_i64, c_i64,            # out
        c_vp, c_sz, c_vp,              # workspace, bytes, stream
    ]),
}
# pa_decode_quant / pa_prefill_quant: a code_type (PA_CODE_*) before the
# arguments of pa_decode_fp8 / pa_prefill_fp8
SIGNATURES["pa_decode_quant"] = (ctypes.c_int, [c_i32] + SIGNATURES["pa_decode_fp8"][1])
SIGNATURES["pa_prefill_quant"] = (ctypes.c_int, [c_i32] + SIGNATURES["pa_prefill_fp8"][1])
PA_CODE_E4M3, PA_CODE_INT8, PA_CODE_UINT8 = 0, 1, 2


class PagedAttentionError(RuntimeError):
    """A non-zero return code from the C ABI."""

    def __init__(self, func: str, code: int, message: str):
        super().__init__(f"{func} returned {code}: {message}")
        self.code = code


def lib_path() -> str:
    return _build.LIB_PATH


def load():
    """Load (once) and return the ctypes library handle.

    Raises ``RuntimeError`` if the library has not been built.
    """
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is not None:
            return _LIB
        path = lib_path()
        if not os.path.exists(path):
            raise RuntimeError(
                f"{path} is missing: build the gfx950 library first "
                "(python vllm-jax_amd/build.py or __graft_entry__.build())")
        lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.pa_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{path} has ABI version {lib.pa_abi_version()}, these bindings expect "
                               f"{ABI_VERSION}: rebuild the library")
        _LIB = lib
    return _LIB


def check(func: str, code: int) -> None:
    if code != 0:
        msg = load().pa_last_error().decode(errors="replace")
        raise PagedAttentionError(func, code, msg)


def call(func: str, *args) -> None:
    """Call a C-ABI entry point and raise on a non-zero return code."""
    check(func, getattr(load(), func)(*args))
