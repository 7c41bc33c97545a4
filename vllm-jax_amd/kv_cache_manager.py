"""KV block manager -- drop-in for ``vllm/src/kv_cache_manager.py:KVCacheManager``.

The block bookkeeping runs in the native library (``csrc/block_manager.cpp``
through ``include/block_manager.h``).  With ``enable_prefix_caching=False``
(the default) and no forks, every method returns what the reference returns
for the same calls: same block ids, order, reference counts and free-queue
order (kv_cache_manager.py:14-70).  Additions:

* ``enable_prefix_caching=True``: a prompt's leading full blocks that match
  cached blocks (same tokens after the same predecessor block) are shared;
  ``num_cached_tokens(request)`` tells the runner how many prompt tokens need
  no recomputation (their K/V are already in the pool);
* ``fork(parent, child)`` and copy-on-write: the first decode write into a
  shared block moves the writer to a fresh block; ``take_block_copies()``
  returns the queued (src, dst) page copies and ``copy_blocks`` executes them
  on the device before the step's KV store.

A request is anything with ``.id``, ``.token_ids`` and ``len()`` (the
reference's ``Request``).  ``get_block_table`` returns a snapshot list of
``Block`` records, where the reference returns its live list.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import List, Sequence, Tuple

import numpy as np

from . import _lib


@dataclass
class Block:
    """kv_cache_manager.py:9-12 (a snapshot)."""
    block_id: int
    ref_count: int


def _tokens(request) -> np.ndarray:
    toks = getattr(request, "token_ids", None)
    if toks is None:
        return np.zeros(0, np.int32)
    return np.ascontiguousarray(np.asarray(toks, dtype=np.int64).astype(np.int32))


class KVCacheManager:
    """kv_cache_manager.py:14-70 on the native block manager."""

    def __init__(self, num_blocks: int, block_size: int, enable_prefix_caching: bool = False):
        self.num_blocks = int(num_blocks)
        self.block_size = int(block_size)
        self.enable_prefix_caching = bool(enable_prefix_caching)
        self._lib = _lib.load()
        handle = self._lib.pa_bm_create(self.num_blocks, self.block_size, int(self.enable_prefix_caching))
        if not handle:
            raise ValueError(self._lib.pa_last_error().decode(errors="replace"))
        self._h = ctypes.c_void_p(handle)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            self._lib.pa_bm_destroy(h)
            self._h = None

    # ---- the reference's methods
    @property
    def num_free_blocks(self) -> int:
        """``len(self.free_block_queue)``."""
        return int(self._lib.pa_bm_num_free_blocks(self._h))

    def block_ids(self, request) -> List[int]:
        n = self._lib.pa_bm_block_table(self._h, int(request.id), None, 0)
        if n < 0:
            _lib.check("pa_bm_block_table", n)
        out = np.zeros(max(n, 1), np.int32)
        self._lib.pa_bm_block_table(self._h, int(request.id), out.ctypes.data, n)
        return out[:n].tolist()

    def get_block_table(self, request) -> List[Block]:
        """kv_cache_manager.py:24-27."""
        return [Block(b, int(self._lib.pa_bm_ref_count(self._h, b))) for b in self.block_ids(request)]

    def can_allocate(self, request, is_prefill: bool) -> bool:
        """kv_cache_manager.py:29-41."""
        toks = _tokens(request) if self.enable_prefix_caching else None
        rc = self._lib.pa_bm_can_allocate(self._h, int(request.id), toks.ctypes.data if toks is not None else None,
                                          len(request), int(bool(is_prefill)))
        if rc < 0:
            raise AssertionError(self._lib.pa_last_error().decode(errors="replace"))
        return bool(rc)

    def allocate_slots(self, request, is_prefill: bool) -> None:
        """kv_cache_manager.py:43-60 (IndexError when the free queue runs dry,
        as ``deque.popleft`` raises in the reference)."""
        toks = _tokens(request) if self.enable_prefix_caching else None
        rc = self._lib.pa_bm_allocate(self._h, int(request.id), toks.ctypes.data if toks is not None else None,
                                      len(request), int(bool(is_prefill)))
        if rc != 0:
            msg = self._lib.pa_last_error().decode(errors="replace")
            raise IndexError(msg) if "free" in msg or "needed" in msg else RuntimeError(msg)

    def deallocate(self, request) -> None:
        """kv_cache_manager.py:62-70."""
        _lib.check("pa_bm_deallocate", self._lib.pa_bm_deallocate(self._h, int(request.id)))

    # ---- additions
    def num_cached_tokens(self, request) -> int:
        """Prompt tokens whose K/V were found in cached blocks at the last prefill."""
        return int(self._lib.pa_bm_num_cached_tokens(self._h, int(request.id)))

    def fork(self, parent, child) -> None:
        """``child`` shares every block of ``parent`` (copy-on-write)."""
        _lib.check("pa_bm_fork", self._lib.pa_bm_fork(self._h, int(parent.id), int(child.id)))

    def ref_count(self, block_id: int) -> int:
        return int(self._lib.pa_bm_ref_count(self._h, int(block_id)))

    def take_block_copies(self) -> Tuple[List[int], List[int]]:
        """Queued copy-on-write page copies (src, dst); the queue is cleared."""
        n = self._lib.pa_bm_take_copies(self._h, None, None, 0)
        if n < 0:
            _lib.check("pa_bm_take_copies", n)
        if n == 0:
            return [], []
        src, dst = np.zeros(n, np.int32), np.zeros(n, np.int32)
        got = self._lib.pa_bm_take_copies(self._h, src.ctypes.data, dst.ctypes.data, n)
        assert got == n
        return src.tolist(), dst.tolist()


def copy_blocks(kv_cache, src: Sequence[int], dst: Sequence[int]) -> None:
    """Execute page copies ``kv_cache[:, dst[i]] <- kv_cache[:, src[i]]`` on
    the device (copy-on-write), in place; ``kv_cache`` is one layer's
    ``[2, NB, BS, Hkv, d]`` bf16 pool."""
    import torch

    from .kernels._common import require_bf16, require_device, stream_handle
    require_device("kv_cache", kv_cache)
    require_bf16("kv_cache", kv_cache)
    if kv_cache.dim() != 5 or kv_cache.shape[0] != 2:
        raise ValueError(f"kv_cache must be [2, NB, BS, Hkv, d], got {tuple(kv_cache.shape)}")
    if len(src) != len(dst):
        raise ValueError("src and dst must have the same length")
    if len(src) == 0:
        return
    _, nb, bs, hkv, d = kv_cache.shape
    idx = torch.as_tensor(np.stack([np.asarray(src, np.int32), np.asarray(dst, np.int32)]), device=kv_cache.device)
    kc, vc = kv_cache[0], kv_cache[1]
    _lib.call("pa_copy_blocks", kc.data_ptr(), vc.data_ptr(), nb, bs, kc.stride(0), kc.stride(1), kc.stride(2),
              hkv, d, idx[0].data_ptr(), idx[1].data_ptr(), len(src), stream_handle(kv_cache))
