"""Kernel entry points with the reference's signatures (vllm/kernels/)."""
from .decode_paged_attention import decode_paged_attention  # noqa: F401
from .prefill_paged_attention import prefill_paged_attention  # noqa: F401
from .mixed_paged_attention import mixed_paged_attention  # noqa: F401
