"""Host-side behaviour of the reference-compatible entry points: argument
checks raise the reference's ValueError messages (prefill_paged_attention.py:
189-207,430-431; decode_paged_attention.py:346-372) before any device work,
and CPU tensors are refused rather than computed on the host."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import PKG


def _prefill_args(t=10, h=16, hkv=8, d=128, nb=4, bs=16, b=2):
    q = torch.zeros(t, h, d, dtype=torch.bfloat16)
    kp = torch.zeros(hkv, nb, bs, d, dtype=torch.bfloat16)
    vp = torch.zeros_like(kp)
    bt = torch.zeros(b, 2, dtype=torch.int32)
    cu = torch.tensor([0, 4, t][:b + 1], dtype=torch.int32)
    sm = torch.zeros(t, dtype=torch.int32)
    pos = torch.zeros(t, dtype=torch.int32)
    return [q, kp, vp, bt, cu, sm, pos]


def test_prefill_shape_errors_match_reference():
    a = _prefill_args()
    with pytest.raises(ValueError, match="k_pages and v_pages must have the same shape"):
        PKG.prefill_paged_attention(a[0], a[1], a[2][:, :2], *a[3:], max_seqlen_bucket=8)
    with pytest.raises(ValueError, match="Number of Q heads must be divisible by number of KV heads"):
        b = _prefill_args(h=12, hkv=8)
        PKG.prefill_paged_attention(*b, max_seqlen_bucket=8)
    with pytest.raises(ValueError, match="head_dim of Q must be the same as that of K/V"):
        b = _prefill_args()
        PKG.prefill_paged_attention(b[0][..., :64], *b[1:], max_seqlen_bucket=8)
    with pytest.raises(ValueError, match=r"cu_seqlens must have shape \[batch \+ 1\]"):
        b = _prefill_args()
        PKG.prefill_paged_attention(*b[:4], b[4][:2], *b[5:], max_seqlen_bucket=8)
    with pytest.raises(ValueError, match="block_tables must be int32"):
        b = _prefill_args()
        PKG.prefill_paged_attention(*b[:3], b[3].long(), *b[4:], max_seqlen_bucket=8)
    with pytest.raises(ValueError, match="block_h must divisible by 16"):
        PKG.prefill_paged_attention(*_prefill_args(), max_seqlen_bucket=8, block_h=8)
    with pytest.raises(ValueError, match="must be given together"):
        PKG.prefill_paged_attention(*_prefill_args(), max_seqlen_bucket=8, k_scales_pages=torch.zeros(1))


def test_prefill_refuses_host_tensors():
    with pytest.raises(ValueError, match="HIP device"):
        PKG.prefill_paged_attention(*_prefill_args(), max_seqlen_bucket=8)


def _decode_args(b=3, h=32, hkv=8, d=128, nb=8, bs=16, p=4):
    q = torch.zeros(b, h, d, dtype=torch.bfloat16)
    kp = torch.zeros(hkv, nb, bs, d, dtype=torch.bfloat16)
    bt = torch.zeros(b, p, dtype=torch.int32)
    lens = torch.ones(b, dtype=torch.int32)
    return [q, kp, kp.clone(), bt, lens]


def test_decode_shape_errors_match_reference():
    a = _decode_args()
    with pytest.raises(ValueError, match="k_pages and v_pages must have the same shape"):
        PKG.decode_paged_attention(a[0], a[1], a[2][:, :3], a[3], a[4])
    with pytest.raises(ValueError, match="Number of Q heads must be divisible"):
        PKG.decode_paged_attention(*_decode_args(h=30))
    with pytest.raises(ValueError, match="head_dim of Q must be the same"):
        PKG.decode_paged_attention(a[0][..., :64], *a[1:])
    with pytest.raises(ValueError, match="`block_tables` and `q` must have the same batch size"):
        PKG.decode_paged_attention(a[0], a[1], a[2], a[3][:2], a[4])
    with pytest.raises(ValueError, match="`lengths` and `q` must have the same batch size"):
        PKG.decode_paged_attention(*a[:4], a[4][:2])
    with pytest.raises(ValueError, match="The dtype of `lengths` must be int32"):
        PKG.decode_paged_attention(*a[:4], a[4].long())
    with pytest.raises(ValueError, match="block_h must divisible by 16"):
        PKG.decode_paged_attention(*a, block_h=24)
    with pytest.raises(ValueError, match="must be given together"):
        PKG.decode_paged_attention(*a, k_scales_pages=torch.zeros(1))
    hkv, nb, bs = a[1].shape[:3]
    sc = torch.ones(hkv, nb, bs)
    with pytest.raises(NotImplementedError, match="float8_e4m3fn, int8 or uint8"):   # bf16 pages with scales
        PKG.decode_paged_attention(*a, k_scales_pages=sc, v_scales_pages=sc)
    with pytest.raises(ValueError, match="k_scales_pages must have shape"):
        PKG.decode_paged_attention(*a, k_scales_pages=sc[:, :1], v_scales_pages=sc)


def test_decode_refuses_host_tensors():
    with pytest.raises(ValueError, match="HIP device"):
        PKG.decode_paged_attention(*_decode_args())


def test_kv_store_validates_shapes_and_device():
    cache = torch.zeros(2, 4, 16, 8, 128, dtype=torch.bfloat16)
    k = torch.zeros(5, 8, 128, dtype=torch.bfloat16)
    sm = torch.zeros(5, dtype=torch.int32)
    with pytest.raises(ValueError, match="HIP device"):
        PKG.update_kv_cache(cache, sm, k, k)


def test_attention_metadata_types_mirror_reference():
    import dataclasses
    d = [f.name for f in dataclasses.fields(PKG.DecodeAttentionMetadata)]
    assert d == ["input_positions", "slot_mapping", "block_tables", "context_lens"]      # qwen3.py:17-22
    p = [f.name for f in dataclasses.fields(PKG.PrefillAttentionMetadata)]
    assert p == ["input_positions", "slot_mapping", "block_tables", "cu_seqlens_q", "cu_seqlens_k",
                 "max_seqlen_q", "max_seqlen_k", "max_seqlen_bucket"]                        # qwen3.py:25-34


def test_bf16_scale_constants():
    from vllm_jax_amd.kernels._common import inv_sqrt_head_dim_bf16, bf16_round
    assert inv_sqrt_head_dim_bf16(128) == 0.08837890625        # bf16(1/sqrt(128))
    assert bf16_round(128 ** 0.5) == 11.3125                    # bf16(sqrt(128)), qwen3.py:207


def test_check_slot_mapping_finds_duplicates():
    """The debug check of the store's contract (qwen3.py:109-110 leaves the
    winner of a duplicated slot unspecified): slots outside the pool are
    ignored, a slot written twice is named with its tokens."""
    from vllm_jax_amd.attention import check_slot_mapping
    check_slot_mapping(torch.tensor([3, 1, -1, -1, 7, 100], dtype=torch.int32), 64)  # -1 twice, 100 outside
    check_slot_mapping(torch.tensor([], dtype=torch.int32), 64)
    with pytest.raises(ValueError, match=r"1 slot\(s\) more than once: slot 5 from tokens \[1, 4\]"):
        check_slot_mapping(torch.tensor([0, 5, 6, 7, 5], dtype=torch.int32), 64)
    with pytest.raises(ValueError, match="2 slot"):
        check_slot_mapping(torch.tensor([9, 9, 2, 2, 63], dtype=torch.int32), 64)
    check_slot_mapping(torch.tensor([9, 9, 64, 64], dtype=torch.int32)[2:], 64)  # both past the pool


@pytest.mark.parametrize("dtype", [torch.uint8, torch.int8])
def test_integer_pages_pass_the_dtype_check(dtype):
    """The reference casts quantized pages of any dtype to q's dtype
    (decode_paged_attention.py:72-75,108-115; prefill_paged_attention.py:
    84-85,118-123), so uint8 / int8 pages mean integer values: the entries
    take them as such (code types PA_CODE_UINT8 / PA_CODE_INT8), and these
    host tensors then stop at the device check.  The library's own quantising
    store writes float8 codes only."""
    from vllm_jax_amd.kernels._common import _CODE_TYPES
    q, kp, _, bt, lens = _decode_args()
    hkv, nb, bs, d = kp.shape
    pages = torch.zeros(hkv, nb, bs, d, dtype=dtype)
    sc = torch.ones(hkv, nb, bs)
    assert _CODE_TYPES[dtype] == (PKG._lib.PA_CODE_INT8 if dtype == torch.int8 else PKG._lib.PA_CODE_UINT8)
    with pytest.raises(ValueError, match="HIP device"):
        PKG.decode_paged_attention(q, pages, pages, bt, lens, k_scales_pages=sc, v_scales_pages=sc)
    a = _prefill_args(hkv=hkv, nb=nb, bs=bs)
    with pytest.raises(ValueError, match="HIP device"):
        PKG.prefill_paged_attention(a[0], pages, pages, *a[3:], max_seqlen_bucket=8,
                                    k_scales_pages=sc, v_scales_pages=sc)
    with pytest.raises(ValueError, match="float8_e4m3fn pool"):
        PKG.update_kv_cache_fp8(torch.zeros(2, nb, bs, hkv, d, dtype=dtype), torch.ones(2, hkv, nb, bs),
                                torch.zeros(5, dtype=torch.int32), torch.zeros(5, hkv, d, dtype=torch.bfloat16),
                                torch.zeros(5, hkv, d, dtype=torch.bfloat16))


def test_other_quantized_page_dtypes_are_refused():
    """Pages with scales must be 1-byte codes (float8_e4m3fn, int8, uint8);
    K and V of one dtype."""
    from vllm_jax_amd.kernels._common import check_quantized_pages
    q, kp, _, bt, lens = _decode_args()
    hkv, nb, bs, d = kp.shape
    sc = torch.ones(hkv, nb, bs)
    for dt in (torch.float16, torch.bfloat16, torch.int16):
        pages = torch.zeros(hkv, nb, bs, d, dtype=dt)
        with pytest.raises(NotImplementedError, match="float8_e4m3fn, int8 or uint8"):
            check_quantized_pages(pages, pages, sc, sc)
    with pytest.raises(ValueError, match="same dtype"):
        check_quantized_pages(torch.zeros(hkv, nb, bs, d, dtype=torch.int8),
                              torch.zeros(hkv, nb, bs, d, dtype=torch.uint8), sc, sc)
