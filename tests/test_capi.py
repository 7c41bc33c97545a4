"""The C-ABI library: it loads, exports every entry point the header declares,
and rejects bad arguments with error codes before touching a device."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest

from conftest import PKG, ROOT

HEADER = os.path.join(ROOT, "include", "paged_attention.h")
HEADERS = sorted(os.path.join(ROOT, "include", f) for f in os.listdir(os.path.join(ROOT, "include")) if f.endswith(".h"))


def _declared():
    text = "".join(open(h).read() for h in HEADERS)
    return sorted(set(re.findall(r"\b(pa_[a-z_0-9]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib_path = PKG._lib.lib_path()
    assert os.path.exists(lib_path), "build the library first (__graft_entry__.build())"
    out = subprocess.run(["nm", "-D", "--defined-only", lib_path], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (pa_\w+)$", out, re.M))
    declared = _declared()
    assert declared, "no declarations parsed"
    missing = [s for s in declared if s not in exported]
    assert not missing, missing
    # and the ctypes table covers them all
    assert set(declared) <= set(PKG._lib.SIGNATURES)


def test_library_has_no_phase_stamps():
    """The per-workgroup phase stamps live only in the opt-in measurement
    build (``build.py --phases``); the library proper carries none."""
    proper = subprocess.run(["nm", "-D", "--defined-only", PKG._lib.lib_path()], capture_output=True, text=True,
                            check=True).stdout
    assert "pa_prefill_phases" not in proper


def test_phase_timestamp_build_exports_its_readers():
    """When the measurement build exists it carries the prefill entry points
    and the stamp readers that ``prefill_phases.py`` binds."""
    path = os.path.join(ROOT, "libpaged_attention_phases.so")
    if not os.path.exists(path):
        pytest.skip("opt-in measurement build not present (python vllm-jax_amd/build.py --phases)")
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (pa_\w+)$", out, re.M))
    assert {"pa_prefill", "pa_prefill_workspace_size", "pa_prefill_phases_read", "pa_prefill_phases_clear"} <= exported


def test_error_codes_match_header():
    text = open(HEADER).read()
    codes = dict(re.findall(r"#define (PA_(?:OK|ERR_\w+)) \(?(-?\d+)\)?", text))
    assert codes == {"PA_OK": "0", "PA_ERR_INVALID_ARGUMENT": "-1", "PA_ERR_UNSUPPORTED": "-2",
                     "PA_ERR_WORKSPACE": "-3", "PA_ERR_LAUNCH": "-4"}


def test_abi_version():
    assert PKG._lib.load().pa_abi_version() == PKG._lib.ABI_VERSION == 2


def _decode_args(**over):
    a = dict(q=None, q_bs=128 * 32, q_hs=128, k=None, v=None, num_pages=16, page_size=256,
             ps=256 * 8 * 128, ss=8 * 128, hs=128, bt=None, bt_stride=4, pps=4, lens=None, batch=2,
             heads=32, kv_heads=8, head_dim=128, scale=1.0, cap=0.0, out=None, o_bs=128 * 32, o_hs=128,
             ws=None, ws_bytes=0, stream=None)
    a.update(over)
    return list(a.values())


def test_decode_rejects_bad_arguments_without_a_device():
    lib = PKG._lib.load()
    rc = lib.pa_decode(*_decode_args(heads=30))
    assert rc == -1
    assert "divisible" in lib.pa_last_error().decode()
    # head sizes other than 128 go to the generic kernels: multiples of 16 up to 256
    assert lib.pa_decode(*_decode_args(head_dim=100)) == -2
    assert "head_dim" in lib.pa_last_error().decode()
    assert lib.pa_decode(*_decode_args(head_dim=272)) == -2
    assert lib.pa_decode(*_decode_args(head_dim=64)) == -1       # accepted; fails on the null pointers
    assert "null pointer" in lib.pa_last_error().decode()
    # 32 q heads per kv head are accepted (two blocks of 16 per work item):
    # these arguments then fail only on their null pointers
    assert lib.pa_decode(*_decode_args(heads=64, kv_heads=2)) == -1
    assert "null pointer" in lib.pa_last_error().decode()
    assert lib.pa_decode(*_decode_args(batch=0)) == 0                  # nothing to do
    assert lib.pa_decode(*_decode_args(page_size=0)) == -1


def test_decode_refuses_a_merge_grid_past_2_31_without_a_device():
    """The decode merge takes up to one workgroup per (sequence, q head): a
    launch with more than 2^31 - 1 such rows is refused before anything is
    launched.  The pointers are placeholders (16-byte aligned, never
    dereferenced on the host); without a workspace a launch of ordinary
    size stops at the workspace check instead."""
    lib = PKG._lib.load()
    fake = dict(q=0x10000, k=0x10000, v=0x10000, bt=0x10000, lens=0x10000, out=0x10000)
    rc = lib.pa_decode(*_decode_args(batch=1 << 25, heads=64, kv_heads=8, **fake))
    assert rc == -2
    assert "(sequence, q head) rows" in lib.pa_last_error().decode()
    assert lib.pa_decode(*_decode_args(**fake)) == -3


def test_decode_noalloc_refuses_oversized_launch_without_a_device():
    """pa_decode_noalloc checks its workspace need against the static
    scratch (64 MiB) before it touches a device: a launch that would need
    more returns PA_ERR_WORKSPACE with the sizes in the message."""
    lib = PKG._lib.load()
    # 4096 sequences x 64 q heads x 64 chunks of 2048 tokens: ~8.7 GB of partials
    a = _decode_args(batch=4096, heads=64, kv_heads=8, pps=512, bt_stride=512)
    need = lib.pa_decode_workspace_size(4096, 64, 128, 512, 256)
    assert need > lib.pa_decode_noalloc_max_workspace()
    rc = lib.pa_decode_noalloc(*a[:-2], a[-1])
    assert rc == -3
    msg = lib.pa_last_error().decode()
    assert "more than the 67108864 bytes" in msg and str(need) in msg, msg


def test_quant_entries_reject_unknown_code_types_without_a_device():
    """pa_decode_quant / pa_prefill_quant take PA_CODE_E4M3 (0), PA_CODE_INT8
    (1) or PA_CODE_UINT8 (2); any other code type is refused before the
    device is touched (null pointers here)."""
    lib = PKG._lib.load()
    text = open(HEADER).read()
    assert dict(re.findall(r"#define (PA_CODE_\w+) (\d+)", text)) == {"PA_CODE_E4M3": "0", "PA_CODE_INT8": "1",
                                                                    "PA_CODE_UINT8": "2"}
    d = [None, 128 * 32, 128, None, None, None, None, 16, 256, 256 * 8 * 128, 8 * 128, 128, 256 * 8, 256,
         None, 4, 4, None, 2, 32, 8, 128, 1.0, 0.0, None, 128 * 32, 128, None, 0, None]
    for code in (3, -1, 7):
        assert lib.pa_decode_quant(code, *d) == -1
        assert "code_type" in lib.pa_last_error().decode()
    p = [None, 2048, 128, None, None, None, None, 16, 256, 256 * 8 * 128, 8 * 128, 128, 256 * 8, 256,
         None, 4, 4, None, None, None, 2, 100, 64, 16, 8, 128, 0.088, 0.0, None, 2048, 128, None, 0, None]
    assert lib.pa_prefill_quant(5, *p) == -1
    assert "code_type" in lib.pa_last_error().decode()
    # a valid code type gets as far as the null pointers
    assert lib.pa_decode_quant(1, *d) == -1
    assert "null pointer" in lib.pa_last_error().decode()


def test_prefill_rejects_bad_arguments_without_a_device():
    lib = PKG._lib.load()
    args = [None, 2048, 128, None, None, 16, 256, 262144, 1024, 128, None, 4, 4, None, None, None,
            2, 100, 64, 16, 8, 128, 0.088, 0.0, None, 2048, 128, None, 0, None]
    bad_div = list(args)
    bad_div[19] = 15
    assert lib.pa_prefill(*bad_div) == -1
    bad_dim = list(args)
    bad_dim[21] = 100
    assert lib.pa_prefill(*bad_dim) == -2
    assert "head_dim" in lib.pa_last_error().decode()
    other_dim = list(args)   # a multiple of 16: accepted, then fails on the null pointers
    other_dim[21] = 96
    assert lib.pa_prefill(*other_dim) == -1
    empty = list(args)
    empty[17] = 0   # num_tokens == 0: nothing to write
    assert lib.pa_prefill(*empty) == 0
    nulls = list(args)  # valid sizes but null pointers
    assert lib.pa_prefill(*nulls) == -1
    assert "null" in lib.pa_last_error().decode()
    # Non-null (never dereferenced) pointers: the work-list checks come first.
    fake = list(args)
    for i in (0, 3, 4, 10, 13, 15, 24):
        fake[i] = 1 << 20
    need = lib.pa_prefill_workspace_size(2, 64, 16, 8)
    small = list(fake)
    small[27], small[28] = 1 << 20, need - 1
    assert lib.pa_prefill(*small) == -3
    assert "workspace" in lib.pa_last_error().decode()
    misaligned = list(fake)
    misaligned[27], misaligned[28] = (1 << 20) + 16, need
    assert lib.pa_prefill(*misaligned) == -3


def test_prefill_workspace_size():
    lib = PKG._lib.load()
    # G = 2: 128-token q tiles; 2 sequences x ceil(300 / 128) = 6 pairs; a
    # 256-byte header, then a 32-byte record per pair
    assert lib.pa_prefill_workspace_size(2, 300, 16, 8) == 256 + 32 * 6
    # G = 8: 32-token q tiles
    assert lib.pa_prefill_workspace_size(64, 1024, 64, 8) == 256 + 32 * 64 * 32
    assert lib.pa_prefill_workspace_size(0, 1024, 64, 8) == 256
    assert lib.pa_prefill_workspace_size(2, 300, 15, 8) == 0   # heads not a multiple of kv heads
    fp8 = lib.pa_prefill_fp8_workspace_size(2, 4, 256, 8, 128, 300, 16)
    widened = 2 * 8 * 256 * 8 * 128 * 2 + (2 * 8 + 1) * 4   # pages, then table, owners, count
    assert fp8 == (widened + 255) // 256 * 256 + 256 + 32 * 6


def test_kv_store_edge_arguments_without_a_device():
    lib = PKG._lib.load()
    base = [None, 1024, 128, None, 1024, 128, None, 0, 8, 128, None, None, 16, 256, 262144, 1024, 128, None]
    assert lib.pa_kv_store(*base) == 0                 # zero tokens
    neg = list(base)
    neg[7] = -1
    assert lib.pa_kv_store(*neg) == -1
    nulls = list(base)
    nulls[7] = 5
    assert lib.pa_kv_store(*nulls) == -1


def test_decode_workspace_size():
    lib = PKG._lib.load()
    # 2048-token work items: ceil(32 pages * 256 / 2048) = 4 chunks per sequence
    r256 = lambda n: (n + 255) // 256 * 256
    r8 = lambda n: (n + 7) // 8 * 8
    # partials (256-byte aligned), then a 256-byte header and one int per (sequence, chunk) pair
    assert lib.pa_decode_workspace_size(256, 32, 128, 32, 256) == r256(256 * 32 * 4 * (128 + 2) * 4) + 256 + 4 * 1024
    # a small launch halves its chunk (down to 512 tokens) until it has 64 (sequence, chunk) pairs:
    # 4 x 1600-token rows of 16-token pages -> 512-token items, ceil(1600 / 512) = 4 chunks
    assert lib.pa_decode_workspace_size(4, 8, 128, 100, 16) == r256(4 * 8 * 4 * (128 + 2) * 4) + 256 + 4 * r8(16)
    assert lib.pa_decode_workspace_size(3, 8, 128, 100, 16) == r256(3 * 8 * 4 * (128 + 2) * 4) + 256 + 4 * r8(12)
    # one 32 768-token row: 2048 -> 512-token items (64 pairs), 64 chunks
    assert lib.pa_decode_workspace_size(1, 32, 128, 128, 256) == r256(32 * 64 * (128 + 2) * 4) + 256 + 4 * r8(64)
    # 8 x 8192-token rows: 1024-token items (64 pairs); 16 of them keep 2048-token ones
    assert lib.pa_decode_workspace_size(8, 32, 128, 32, 256) == r256(8 * 32 * 8 * (128 + 2) * 4) + 256 + 4 * 64
    assert lib.pa_decode_workspace_size(16, 32, 128, 32, 256) == r256(16 * 32 * 4 * (128 + 2) * 4) + 256 + 4 * 64
    assert lib.pa_decode_workspace_size(0, 32, 128, 32, 256) == 0
    # the generic decode's 1024-token items at head sizes below 128 other than 64
    assert lib.pa_decode_workspace_size(4, 8, 96, 32, 256) == r256(4 * 8 * 8 * (96 + 2) * 4) + 256 + 4 * r8(32)
    assert lib.pa_decode_workspace_size(4, 8, 64, 32, 256) == r256(4 * 8 * 4 * (64 + 2) * 4) + 256 + 4 * r8(16)


def test_mixed_workspace_size():
    lib = PKG._lib.load()
    r256 = lambda n: (n + 255) // 256 * 256
    # Qwen3-0.6B step: 96 decode + 32 prefill sequences, 16-page tables of 256-token pages:
    # one 4096-token chunk per decode sequence (no partials); G = 2 -> 128-token q tiles,
    # 16 per prefill sequence; a 256-byte header, 32 bytes per pair (count rounded up to 8)
    assert lib.pa_mixed_workspace_size(128, 96, 2048, 16, 8, 128, 16, 256) == 256 + 32 * (96 + 32 * 16)
    # 40-page tables: 3 chunks per decode sequence, partials for 3 sequences x 16 heads
    part = r256(3 * 16 * 3 * (128 + 2) * 4)
    assert lib.pa_mixed_workspace_size(5, 3, 300, 16, 8, 128, 40, 256) == part + 256 + 32 * 16
    assert lib.pa_mixed_workspace_size(5, 6, 300, 16, 8, 128, 40, 256) == 0   # more decodes than sequences
    assert lib.pa_mixed_workspace_size(5, 3, 300, 15, 8, 128, 40, 256) == 0   # heads not a multiple of kv heads
    # pages above 4096 tokens: 4096-token chunks inside one page (2 per 8192-token page)
    part = r256(2 * 16 * 2 * (128 + 2) * 4)
    assert lib.pa_mixed_workspace_size(4, 2, 100, 16, 8, 128, 1, 8192) == part + 256 + 32 * 8
    assert lib.pa_mixed_workspace_size(4, 2, 100, 16, 8, 128, 1, 4096) == 256 + 32 * 8
    # 16-token pages: 4096-token chunks too (256 page ids, four per lane): a 400-page
    # table is 2 chunks; pairs 3 x 2 decode + 2 x 3 prefill (128-token q tiles) = 12
    part = r256(3 * 16 * 2 * (128 + 2) * 4)
    assert lib.pa_mixed_workspace_size(5, 3, 300, 16, 8, 128, 400, 16) == part + 256 + 32 * 16
    # G = 32: two decode pairs per (sequence, chunk), one per block of 16 q heads;
    # 8-token q tiles (13 per prefill sequence)
    assert lib.pa_mixed_workspace_size(4, 2, 100, 32, 1, 128, 8, 256) == 256 + 32 * 32
    # more q heads per kv head than the 256 rows of a prefill item is refused
    assert lib.pa_mixed_workspace_size(4, 2, 100, 512, 1, 128, 8, 256) == 0


def test_large_slot_stride_is_refused_by_the_aligned_tile_loads():
    # The aligned prefill tile loads use 32-bit per-lane offsets of up to
    # 63 * slot_stride + 127 elements: a larger stride (e.g. a [BS, NB, Hkv, d]
    # pool view with NB >= 32768) must be refused, not wrapped.
    lib = PKG._lib.load()
    fake = 1 << 20
    big = 0x7fffffff // 63 + 8          # first multiple-of-8 stride past the limit
    big -= big % 8
    ok = (0x7fffffff - 127) // 63 // 8 * 8
    def prefill(ss, page_size=256):
        args = [fake, 2048, 128, fake, fake, 16, page_size, 262144, ss, 128, fake, 4, 4, fake, None, fake,
                2, 100, 64, 16, 8, 128, 0.088, 0.0, fake, 2048, 128, None, 0, None]
        return lib.pa_prefill(*args)
    assert prefill(big) == -2
    assert "slot stride" in lib.pa_last_error().decode()
    assert prefill(-8) == -2
    def mixed(ss):
        return lib.pa_mixed(fake, 2048, 128, fake, fake, 16, 256, 262144, ss, 128, fake, 4, 4, fake, fake, fake,
                            3, 1, 100, 64, 16, 8, 128, 0.088, 1.0, 0.0, fake, 2048, 128, fake, 0, None)
    assert mixed(big) == -2
    assert "slot stride" in lib.pa_last_error().decode()
    # the largest stride that fits passes this check and stops at the next one (workspace)
    assert mixed(ok) == -3


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    """No silent fallback: a missing .so is an error, not a CPU path."""
    import importlib
    lib_mod = importlib.import_module("vllm_jax_amd._lib")
    monkeypatch.setattr(lib_mod, "_LIB", None)
    monkeypatch.setattr(lib_mod, "lib_path", lambda: str(tmp_path / "missing.so"))
    with pytest.raises(RuntimeError, match="missing"):
        lib_mod.load()


def test_generic_head_sizes_at_the_boundary():
    """Head sizes other than 128: multiples of 16 up to 256 are taken by
    pa_prefill / pa_decode / pa_mixed and by the quantized-page entries
    (they then fail here only on their null pointers), other sizes are
    refused, and the mixed workspace of a generic size holds the decode
    partials of every chunk after 256 bytes."""
    lib = PKG._lib.load()
    r256 = lambda n: (n + 255) // 256 * 256
    # 2 decodes, 16 heads, 40-page tables of 256-token pages: 3 chunks of 4096 tokens
    assert lib.pa_mixed_workspace_size(5, 2, 300, 16, 8, 64, 40, 256) == 256 + r256(2 * 16 * 3 * (64 + 2) * 4)
    assert lib.pa_mixed_workspace_size(5, 0, 300, 16, 8, 96, 40, 256) == 256          # no decode sequence
    assert lib.pa_mixed_workspace_size(5, 2, 300, 16, 8, 100, 40, 256) == 0           # not a multiple of 16
    assert lib.pa_mixed_workspace_size(5, 2, 300, 16, 8, 272, 40, 256) == 0           # above 256
    # quantized decode: head size 64 is taken (then the null pointers fail),
    # 100 and 272 are refused before any pointer is looked at
    fp8 = [None, 2048, 64, None, None, None, None, 16, 256, 131072, 512, 64, 4096, 256, None, 4, 4, None, 2,
           32, 8, 64, 1.0, 0.0, None, 2048, 64, None, 0, None]
    assert lib.pa_decode_fp8(*fp8) == -1
    assert "null pointer" in lib.pa_last_error().decode()
    for code in (0, 1, 2):
        assert lib.pa_decode_quant(code, *fp8) == -1
    for d in (100, 272):
        bad = list(fp8)
        bad[21] = d
        assert lib.pa_decode_fp8(*bad) == -2
        assert "head_dim" in lib.pa_last_error().decode()
    # quantized prefill: the same sizes
    pre = [None, 2048, 64, None, None, None, None, 16, 256, 131072, 512, 64, 4096, 256, None, 4, 4, None, None, None,
           2, 100, 64, 32, 8, 64, 0.125, 0.0, None, 2048, 64, None, 0, None]
    assert lib.pa_prefill_fp8(*pre) == -1
    assert "null pointer" in lib.pa_last_error().decode()
    for d in (100, 272):
        bad = list(pre)
        bad[25] = d
        assert lib.pa_prefill_quant(1, *bad) == -2
        assert "head_dim" in lib.pa_last_error().decode()
    # the quantising store: multiples of 16 from 16 to 256
    st = [None, 512, 64, None, 512, 64, None, 4, 8, 64, None, None, None, None, 16, 256, 131072, 512, 64,
          4096, 1, 256, None]
    assert lib.pa_kv_store_fp8(*st) == -1
    assert "null pointer" in lib.pa_last_error().decode()
    for d in (8, 100, 272):
        bad = list(st)
        bad[9] = d
        assert lib.pa_kv_store_fp8(*bad) == -2
        assert "head_dim" in lib.pa_last_error().decode()
