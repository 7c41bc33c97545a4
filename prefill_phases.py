"""Per-workgroup phase table of the prefill kernel.

Runs ``pa_prefill`` from ``libpaged_attention_phases.so`` (the prefill
entry points built with ``PA_PREFILL_PHASES``; ``python3
vllm-jax_amd/build.py --phases`` makes it next to this script, and the
package never loads it) on one of the benchmark workloads and prints where each workgroup's time goes.  The
kernel stamps ``s_memrealtime`` (100 MHz) at five points of every item:

    T0 item start          T1 kv range and tile count known
    T2 first tile in LDS   T3 loop done (all tiles)   T4 output stored

and records the workgroup's CU (HW_ID, XCC_ID), tile count and item.  From these
the script reports the mean / median / p90 of each phase, the gap between one
workgroup's T4 and the next workgroup's T0 on the same CU (one 8-wave
workgroup fills a CU), each CU's first start and last end, the last end per
XCD, and the share of CU time that is not tile work (phases T0-T2 and
T3-T4 plus the gaps).  A table per XCD gives the workgroups and kv tiles it
ran, its loop time per tile and its CUs' last ends.

Usage (one GPU)::

    python3 vllm-jax_amd/build.py --phases         # once, on the build machine
    python3 prefill_phases.py long     # Qwen3-32B, 8 x ~26.7k tokens
    python3 prefill_phases.py prefix   # Qwen3-8B prefix-cached
    python3 prefill_phases.py short    # 64 x 1024 tokens, 16/8 heads
    python3 prefill_phases.py prefix --dump stamps.npy

``--dump FILE`` also saves the raw records (one row of 8 uint64 per
workgroup that ran an item: T0..T4, HW_ID | XCC_ID << 32, tiles,
sequence | q tile << 24 | kv head << 48) with numpy.save.

The instrumented kernel is timed too; the stamps add a few stores per
workgroup and the run is within a percent of the library proper.
"""
from __future__ import annotations

import collections
import ctypes
import importlib
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PHASES_LIB = os.path.join(ROOT, "libpaged_attention_phases.so")
SLOTS = 1 << 17  # workgroup ids the kernel records (8 words each)


def _load(pkg):
    if not os.path.exists(PHASES_LIB):
        raise RuntimeError(f"{PHASES_LIB} is missing: run python3 vllm-jax_amd/build.py --phases first")
    lib = ctypes.CDLL(PHASES_LIB)
    for name in ("pa_prefill", "pa_prefill_workspace_size", "pa_last_error"):
        res, args = pkg._lib.SIGNATURES[name]
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    lib.pa_prefill_phases_read.restype = ctypes.c_int
    lib.pa_prefill_phases_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    lib.pa_prefill_phases_clear.restype = ctypes.c_int
    lib.pa_prefill_phases_clear.argtypes = []
    return lib


def _workload(wl, name):
    if name == "long":
        return "Qwen3-32B long prefill", wl.qwen3_32b_long_prefill(seed=4), 4
    if name == "prefix":
        return "Qwen3-8B prefix-cached prefill", wl.qwen3_8b_prefix_prefill(seed=3), 3
    if name == "short":
        return ("64 x 1024-token prefill, 16 q / 8 kv heads",
                wl.make_prefill([1024] * 64, num_heads=16, num_kv_heads=8, rng=np.random.default_rng(5)), 5)
    raise SystemExit(f"unknown workload {name!r}: long, prefix or short")


def _pct(a, q):
    return float(np.percentile(a, q))


def main(argv):
    import torch

    sys.path.insert(0, ROOT)
    import __graft_entry__ as ge

    pkg = ge.load_package()
    wl = importlib.import_module(pkg.__name__ + ".workloads")
    lib = _load(pkg)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    dump = None
    if "--dump" in argv:
        i = argv.index("--dump")
        if i + 1 >= len(argv):
            raise SystemExit("--dump needs a file name")
        dump = argv[i + 1]
        argv = argv[:i] + argv[i + 2:]
    title, pb, seed = _workload(wl, argv[0] if argv else "prefix")
    t = wl.materialize_prefill(pb, seed=seed, device=dev, fill_pool=True)
    kv = t["kv_cache"]
    kp, vp = kv[0].permute(2, 0, 1, 3), kv[1].permute(2, 0, 1, 3)
    ps, ss, hs = kp.stride(1), kp.stride(2), kp.stride(0)
    q, bt, cuk = t["q"], t["block_tables"], t["cu_seqlens_k"]
    need = int(lib.pa_prefill_workspace_size(pb.batch, int(pb.max_seqlen_bucket), pb.num_heads, pb.num_kv_heads))
    ws = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
    out = torch.empty_like(q)
    scale = float(torch.tensor(q.shape[-1] ** -0.5, dtype=torch.bfloat16))

    def run():
        rc = lib.pa_prefill(q.data_ptr(), q.stride(0), q.stride(1), kp.data_ptr(), vp.data_ptr(), kp.shape[1],
                            kp.shape[2], ps, ss, hs, bt.data_ptr(), bt.stride(0), bt.shape[1],
                            t["cu_seqlens_q"].data_ptr(), cuk.data_ptr() if cuk is not None else None,
                            t["input_positions"].data_ptr(), pb.batch, q.shape[0], int(pb.max_seqlen_bucket),
                            pb.num_heads, pb.num_kv_heads, q.shape[-1], scale, 0.0, out.data_ptr(),
                            out.stride(0), out.stride(1), ws.data_ptr(), ws.numel(),
                            torch.cuda.current_stream().cuda_stream)
        if rc != 0:
            raise RuntimeError(f"pa_prefill returned {rc}: {lib.pa_last_error().decode(errors='replace')}")

    for _ in range(3):
        run()
    torch.cuda.synchronize()
    ref = pkg.prefill_paged_attention(q, kp, vp, bt, t["cu_seqlens_q"], t["slot_mapping"], t["input_positions"],
                                      max_seqlen_bucket=pb.max_seqlen_bucket, cu_seqlens_k=cuk)
    diff = (out.float() - ref.float()).abs().max().item()
    if lib.pa_prefill_phases_clear() != 0:
        raise RuntimeError(lib.pa_last_error().decode(errors="replace"))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    run()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    buf = np.zeros(8 * SLOTS, dtype=np.uint64)
    if lib.pa_prefill_phases_read(buf.ctypes.data, buf.size) != 0:
        raise RuntimeError(lib.pa_last_error().decode(errors="replace"))
    g = buf.reshape(-1, 8)
    g = g[g[:, 0] > 0]
    if dump:
        np.save(dump, g)
    T = (g[:, :5].astype(np.float64) - float(g[:, 0].min())) / 100.0  # microseconds from the first start
    ph = np.diff(T, axis=1)
    tiles = g[:, 6].astype(np.float64)
    hw = g[:, 5]
    xcc = (hw >> np.uint64(32)).astype(np.int64)
    low = (hw & np.uint64(0xFFFFFFFF)).astype(np.int64)
    cu = (low >> 8) & 15
    sh = (low >> 12) & 1
    se = (low >> 13) & 7
    key = ((xcc * 8 + se) * 2 + sh) * 16 + cu

    gaps, busy, firsts, lasts = [], [], [], []
    xcd_last = collections.defaultdict(list)
    for k in np.unique(key):
        sel = np.where(key == k)[0]
        o = sel[np.argsort(T[sel, 0])]
        if len(o) > 1:
            gaps.extend((T[o[1:], 0] - T[o[:-1], 4]).tolist())
        busy.append(float((T[o, 4] - T[o, 0]).sum()))
        firsts.append(float(T[o, 0].min()))
        lasts.append(float(T[o, 4].max()))
        xcd_last[int(k) // 256].append(lasts[-1])
    gaps = np.array(gaps) if gaps else np.zeros(1)
    span = float(T[:, 4].max())

    print(f"## {title}")
    print(f"{pb.batch} sequences, {q.shape[0]} query tokens, {pb.num_heads} q / {pb.num_kv_heads} kv heads; "
          f"instrumented launch {ms * 1e3:.1f} us (events), stamped span {span:.1f} us; "
          f"{len(g)} workgroups on {len(busy)} CUs; max |out - library| = {diff:.3g}")
    print()
    print("| phase | mean us | median us | p90 us |")
    print("|---|---|---|---|")
    names = ["T0-T1 item start to kv range", "T1-T2 to first tile in LDS", "T2-T3 tile loop",
             "T3-T4 epilogue (normalise, store)"]
    for i, nm in enumerate(names):
        print(f"| {nm} | {ph[:, i].mean():.2f} | {np.median(ph[:, i]):.2f} | {_pct(ph[:, i], 90):.2f} |")
    print(f"| gap to the next workgroup on the CU | {gaps.mean():.2f} | {np.median(gaps):.2f} | "
          f"{_pct(gaps, 90):.2f} |")
    print()
    per_tile = ph[:, 2].sum() / max(tiles.sum(), 1.0)
    fixed = ph[:, 0].sum() + ph[:, 1].sum() + ph[:, 3].sum()
    total = float((T[:, 4] - T[:, 0]).sum() + gaps.sum())
    print(f"- tiles per workgroup: mean {tiles.mean():.1f}, min {tiles.min():.0f}, max {tiles.max():.0f}; "
          f"loop time per tile {per_tile:.3f} us")
    print(f"- fixed cost per workgroup (T0-T2 + T3-T4) {(fixed / len(g)):.2f} us; fixed + gaps = "
          f"{(fixed + gaps.sum()) / total * 100:.1f} % of CU time between first start and last end")
    print(f"- CU first start: max {max(firsts):.1f} us; CU last end: min {min(lasts):.1f}, "
          f"p50 {np.median(lasts):.1f}, max {max(lasts):.1f} us; CU busy mean {np.mean(busy):.1f} us of {span:.1f}")
    print()
    print("| XCD | workgroups | kv tiles | loop us per tile | last end us (min / max over its CUs) |")
    print("|---|---|---|---|---|")
    for x, v in sorted(xcd_last.items()):
        sel = xcc == x
        nt = max(float(tiles[sel].sum()), 1.0)
        print(f"| {x} | {int(sel.sum())} | {int(tiles[sel].sum())} | {ph[sel, 2].sum() / nt:.3f} | "
              f"{min(v):.0f} / {max(v):.0f} |")
    sys.stdout.flush()
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
