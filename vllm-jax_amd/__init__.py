"""MI355X (gfx950) paged-attention path for vllm-jax-style serving.

Public surface (mirrors simpissa/vllm-jax):

* ``attention(kv_cache, q, k, v, metadata)`` plus ``PrefillAttentionMetadata``
  / ``DecodeAttentionMetadata`` -- the layer seam of vllm/model/qwen3.py;
* ``prefill_paged_attention`` / ``decode_paged_attention`` -- the kernel
  entries of vllm/kernels/;
* ``update_kv_cache`` -- the KV store;
* ``qk_norm_rope_store`` / ``qwen3_attention_core`` -- the q/k RMSNorm +
  RoPE + KV store step before attention, fused into one kernel;
* ``MixedAttentionMetadata`` / ``mixed_paged_attention`` -- a step's decode
  and prefill sequences in one unpadded launch;
* ``KVCacheManager`` / ``copy_blocks`` -- the block manager of
  vllm/src/kv_cache_manager.py on a native allocator, with optional prefix
  caching and fork / copy-on-write.

All device work runs in ``libpaged_attention.so`` (hand-written HIP for
gfx950, built by ``build.py``) through a C ABI; there is no CPU fallback.
The directory name contains a hyphen, so it is imported by path under the
module name ``vllm_jax_amd``::

    spec = importlib.util.spec_from_file_location(
        "vllm_jax_amd", "<repo>/vllm-jax_amd/__init__.py",
        submodule_search_locations=["<repo>/vllm-jax_amd"])
"""
from .attention import (DecodeAttentionMetadata, MixedAttentionMetadata, PrefillAttentionMetadata,  # noqa: F401
                        attention, attention_stored, gather_kv, qk_norm_rope_store, qwen3_attention_core,
                        update_kv_cache, update_kv_cache_fp8)
from .kernels.decode_paged_attention import decode_paged_attention  # noqa: F401
from .kernels.mixed_paged_attention import mixed_paged_attention  # noqa: F401
from .kernels.prefill_paged_attention import prefill_paged_attention  # noqa: F401
from .kv_cache_manager import Block, KVCacheManager, copy_blocks  # noqa: F401
