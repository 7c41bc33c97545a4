"""Benchmark of the gfx950 paged-attention path on one MI355X.

Default run (``python bench.py``): one step = one pass of each headline
workload, inputs resident in HBM:

* Qwen3-32B long-context ragged prefill (8 sequences, L ~ U[8192, 32768],
  64 q / 8 kv heads, head_dim 128, 256-token pages, seed 4):
  KV store of all new tokens + causal GQA paged prefill.
  ``value`` = algorithmic prefill TFLOP/s (causal-visible pairs only).
* Qwen3-8B decode (256 sequences, ctx ~ U[512, 8192], 32 q / 8 kv heads,
  16384-page pool, seed 2): KV store of the new token + split-K decode.
  Reported under ``"decode"`` in GB/s of algorithmic HBM traffic.
* The Qwen3-8B prefix-cached prefill (64 sequences, cached prefixes
  U[0, 4096] in shared blocks, new chunks U[128, 1024], 32 q / 8 kv heads,
  seed 3): reported under ``"prefix_prefill"`` in TFLOP/s.
* The prefix-cached prefill over float8 e4m3 pages (the same pool quantised
  on the device): each distinct page widened once, then the bf16 prefill;
  reported under ``"prefill_fp8"`` in TFLOP/s with the widening included,
  next to the bf16 time of the same batch.
* The Qwen3-8B decode over float8 e4m3 pages with per-token scales (the same
  pool quantised on the device): reported under ``"decode_fp8"`` in GB/s of
  its own algorithmic bytes (codes + scales), with the bf16 decode time of
  the same batch for comparison.
* The Qwen3-0.6B mixed scheduler step (96 decode sequences ctx ~ U[256,
  4096] + 32 prefill sequences L ~ U[64, 2048], seed 1) as one unpadded
  ``pa_mixed`` launch against the separate decode and prefill launches
  (timed in its own loop): reported under ``"mixed"``.
* The Qwen3-0.6B single-layer prefill (4 sequences [17, 128, 300, 511], the
  configuration the reference runs on its CPU path): GPU step time next to
  the CPU oracle over the same whole configuration, under
  ``"qwen3_06b_prefill"``.
* The fused q/k RMSNorm + RoPE + KV store over the prefill workload's tokens
  (timed in its own loop after the step): reported under ``"qk_norm_rope"``
  in GB/s of algorithmic HBM traffic, (2 H + 4 Hkv) * 256 + 8 bytes a token.

Prints ONE JSON line.  ``roofline`` (prefill, MFMA-bound) and
``decode.roofline`` (HBM-bound) use the average duration of the attention
call measured with HIP events on the launch stream.  ``cpu_baseline`` times
the CPU oracle on a bounded sample of the same workload (rank 0 only).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

MFMA_BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16
HBM_PEAK_GBS = 8000.0            # MI355X HBM3E
METRIC = "prefill attn TFLOP/s (% bf16 MFMA peak); decode attn GB/s (% HBM peak)"


def _load_traffic():
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE,
    scaled by a copy-kernel calibration), committed under profiles/."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return {}
    with open(path) as f:
        return json.load(f)


def _events(torch, n):
    return [torch.cuda.Event(enable_timing=True) for _ in range(n)]


def run_copy(args):
    """A plain 1 GiB device-to-device copy, K times: the calibration kernel for
    the FETCH_SIZE / WRITE_SIZE counters (1 GiB read + 1 GiB written per launch)."""
    import torch
    dev = torch.device("cuda:0")
    src = torch.ones(1 << 29, dtype=torch.bfloat16, device=dev)
    dst = torch.empty_like(src)
    for _ in range(args.warmup):
        dst.copy_(src)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(args.steps):
        dst.copy_(src)
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    return {"metric": "device copy GB/s (calibration)", "value": round(2 * src.numel() * 2 / ms / 1e6, 1),
            "unit": "GB/s", "bytes_read_per_launch": src.numel() * 2, "bytes_written_per_launch": src.numel() * 2,
            "ms_per_step": round(ms, 4), "steps": args.steps}


def run_head_dims(args):
    """Prefill and decode at head sizes 64, 96, 128 and 256 on the same
    shapes: 16 sequences of 2 048 new tokens (32 q / 8 kv heads, 256-token
    pages) and the Qwen3-8B-shaped decode batch (256 sequences, contexts
    U[512, 8192], pool sized to the batch).  128 runs the tuned kernels, the
    other sizes the generic ones.  Attention only (the pages are filled
    beforehand); HIP events, the median of three rounds of `steps` launches
    after at least 150 ms of warm-up launches per case."""
    import torch
    import __graft_entry__ as ge
    pkg = ge.load_package()
    import vllm_jax_amd.workloads as wl
    dev = torch.device("cuda:0")
    lens_d = np.random.default_rng(2).integers(512, 8193, size=256)
    pre, dec = [], []
    for d in (64, 96, 128, 256):
        pb = wl.make_prefill([2048] * 16, num_heads=32, num_kv_heads=8, head_dim=d, rng=np.random.default_rng(9))
        t = wl.materialize_prefill(pb, seed=9, device=dev, fill_pool=True)
        kp, vp = t["kv_cache"][0].permute(2, 0, 1, 3), t["kv_cache"][1].permute(2, 0, 1, 3)
        out = torch.empty_like(t["q"])

        def attn():
            pkg.prefill_paged_attention(t["q"], kp, vp, t["block_tables"], t["cu_seqlens_q"], t["slot_mapping"],
                                        t["input_positions"], max_seqlen_bucket=pb.max_seqlen_bucket,
                                        cu_seqlens_k=t["cu_seqlens_k"], out=out)
        ms = _time_ms_warm(torch, attn, args)
        tf = pb.flops() / (ms * 1e-3) / 1e12
        pre.append({"head_dim": d, "ms": round(ms, 4), "tflops": round(tf, 1),
                    "frac_of_mfma_peak": round(tf / MFMA_BF16_PEAK_TFLOPS, 4)})
        del t, kp, vp, out
        db = wl.make_decode(lens_d, num_heads=32, num_kv_heads=8, head_dim=d, rng=np.random.default_rng(2))
        dd = wl.materialize_decode(db, seed=2, device=dev)
        kv = dd["kv_cache"]
        kpd, vpd = kv[0].permute(2, 0, 1, 3), kv[1].permute(2, 0, 1, 3)
        outd = torch.empty_like(dd["q"])

        def dec_call():
            pkg.decode_paged_attention(dd["q"], kpd, vpd, dd["block_tables"], dd["context_lens"], out=outd)
        ms = _time_ms_warm(torch, dec_call, args)
        gbs = db.hbm_bytes() / (ms * 1e-3) / 1e9
        dec.append({"head_dim": d, "ms": round(ms, 4), "gbs": round(gbs, 1),
                    "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)})
        del dd, kv, kpd, vpd, outd
        torch.cuda.empty_cache()
    return {"metric": "attention at head sizes 64 / 96 / 128 / 256 (128: tuned kernels; others: generic)",
            "prefill": {"workload": "16 x 2048 new tokens, 32 q / 8 kv heads, causal", "results": pre},
            "decode": {"workload": "256 sequences, contexts U[512, 8192], 32 q / 8 kv heads", "results": dec},
            "steps": args.steps, "warmup": args.warmup}


def run_soft_cap(args):
    """Attention with and without the logit soft cap (cap 50) on the
    head-size shapes: prefill of 16 sequences of 2 048 new tokens and the
    Qwen3-8B-shaped decode batch (256 sequences, contexts U[512, 8192]),
    32 q / 8 kv heads, at head size 128 (tuned kernels) and 256 (generic
    kernels).  Attention only; HIP events, the median of three rounds of
    `steps` launches after at least 150 ms of warm-up launches per case."""
    import torch
    import __graft_entry__ as ge
    pkg = ge.load_package()
    import vllm_jax_amd.workloads as wl
    dev = torch.device("cuda:0")
    lens_d = np.random.default_rng(2).integers(512, 8193, size=256)
    pre, dec = [], []
    for d in (128, 256):
        pb = wl.make_prefill([2048] * 16, num_heads=32, num_kv_heads=8, head_dim=d, rng=np.random.default_rng(9))
        t = wl.materialize_prefill(pb, seed=9, device=dev, fill_pool=True)
        kp, vp = t["kv_cache"][0].permute(2, 0, 1, 3), t["kv_cache"][1].permute(2, 0, 1, 3)
        out = torch.empty_like(t["q"])
        row = {"head_dim": d}
        for cap in (None, 50.0):
            def attn():
                pkg.prefill_paged_attention(t["q"], kp, vp, t["block_tables"], t["cu_seqlens_q"], t["slot_mapping"],
                                            t["input_positions"], max_seqlen_bucket=pb.max_seqlen_bucket,
                                            cu_seqlens_k=t["cu_seqlens_k"], attn_logits_soft_cap=cap, out=out)
            ms = _time_ms_warm(torch, attn, args)
            tf = pb.flops() / (ms * 1e-3) / 1e12
            row["soft_cap_ms" if cap else "ms"] = round(ms, 4)
            row["soft_cap_tflops" if cap else "tflops"] = round(tf, 1)
        row["soft_cap_over_plain"] = round(row["soft_cap_ms"] / row["ms"], 3)
        pre.append(row)
        del t, kp, vp, out
        db = wl.make_decode(lens_d, num_heads=32, num_kv_heads=8, head_dim=d, rng=np.random.default_rng(2))
        dd = wl.materialize_decode(db, seed=2, device=dev)
        kv = dd["kv_cache"]
        kpd, vpd = kv[0].permute(2, 0, 1, 3), kv[1].permute(2, 0, 1, 3)
        outd = torch.empty_like(dd["q"])
        row = {"head_dim": d}
        for cap in (None, 50.0):
            def dec_call():
                pkg.decode_paged_attention(dd["q"], kpd, vpd, dd["block_tables"], dd["context_lens"],
                                           attn_logits_soft_cap=cap, out=outd)
            ms = _time_ms_warm(torch, dec_call, args)
            gbs = db.hbm_bytes() / (ms * 1e-3) / 1e9
            row["soft_cap_ms" if cap else "ms"] = round(ms, 4)
            row["soft_cap_gbs" if cap else "gbs"] = round(gbs, 1)
        row["soft_cap_over_plain"] = round(row["soft_cap_ms"] / row["ms"], 3)
        dec.append(row)
        del dd, kv, kpd, vpd, outd
        torch.cuda.empty_cache()
    return {"metric": "attention with the logit soft cap (50) against without, head sizes 128 and 256",
            "prefill": {"workload": "16 x 2048 new tokens, 32 q / 8 kv heads, causal", "results": pre},
            "decode": {"workload": "256 sequences, contexts U[512, 8192], 32 q / 8 kv heads", "results": dec},
            "steps": args.steps, "warmup": args.warmup}


def run_page_sizes(args):
    """Prefill and decode over pages of 16, 32, 64 and 256 tokens, the same
    tokens each time: the Qwen3-8B prefix-cached prefill (seed 3's lengths)
    and the Qwen3-8B-shaped decode batch (256 sequences, contexts U[512,
    8192]), 32 q / 8 kv heads, head size 128.  Attention only; timed like
    the other short lines (`_time_ms_warm`)."""
    import torch
    import __graft_entry__ as ge
    pkg = ge.load_package()
    import vllm_jax_amd.workloads as wl
    dev = torch.device("cuda:0")
    lens_d = np.random.default_rng(2).integers(512, 8193, size=256)
    rng = np.random.default_rng(3)
    prefix, new = rng.integers(0, 4097, size=64), rng.integers(128, 1025, size=64)
    pre, dec = [], []
    for bs in (256, 64, 32, 16):
        pb = wl.make_prefix_prefill(prefix, new, num_heads=32, num_kv_heads=8, page_size=bs,
                                    rng=np.random.default_rng(3), shared_prefix_tokens=4096)
        t = wl.materialize_prefill(pb, seed=3, device=dev, fill_pool=True)
        kp, vp = t["kv_cache"][0].permute(2, 0, 1, 3), t["kv_cache"][1].permute(2, 0, 1, 3)
        out = torch.empty_like(t["q"])

        def attn():
            pkg.prefill_paged_attention(t["q"], kp, vp, t["block_tables"], t["cu_seqlens_q"], t["slot_mapping"],
                                        t["input_positions"], max_seqlen_bucket=pb.max_seqlen_bucket,
                                        cu_seqlens_k=t["cu_seqlens_k"], out=out)
        ms = _time_ms_warm(torch, attn, args)
        tf = pb.flops() / (ms * 1e-3) / 1e12
        pre.append({"page_size": bs, "ms": round(ms, 4), "tflops": round(tf, 1),
                    "frac_of_mfma_peak": round(tf / MFMA_BF16_PEAK_TFLOPS, 4)})
        del t, kp, vp, out
        db = wl.make_decode(lens_d, num_heads=32, num_kv_heads=8, page_size=bs, rng=np.random.default_rng(2))
        dd = wl.materialize_decode(db, seed=2, device=dev)
        kv = dd["kv_cache"]
        kpd, vpd = kv[0].permute(2, 0, 1, 3), kv[1].permute(2, 0, 1, 3)
        outd = torch.empty_like(dd["q"])

        def dec_call():
            pkg.decode_paged_attention(dd["q"], kpd, vpd, dd["block_tables"], dd["context_lens"],
                                       scale=1 / 11.3125, out=outd)
        ms = _time_ms_warm(torch, dec_call, args)
        gbs = db.hbm_bytes() / (ms * 1e-3) / 1e9
        dec.append({"page_size": bs, "ms": round(ms, 4), "gbs": round(gbs, 1),
                    "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)})
        del dd, kv, kpd, vpd, outd
        torch.cuda.empty_cache()
    return {"metric": "attention over pages of 256 / 64 / 32 / 16 tokens (head size 128, tuned kernels)",
            "prefill": {"workload": "Qwen3-8B prefix-cached prefill (seed 3's lengths)", "results": pre},
            "decode": {"workload": "256 sequences, contexts U[512, 8192], 32 q / 8 kv heads", "results": dec},
            "steps": args.steps, "warmup": args.warmup}


def run_small_decode(args):
    """Decode of a few long sequences (32 q / 8 kv heads, head size 128,
    256-token pages): 1 x 32 768, 1 x 131 072, 2 x 16 384, 4 x 32 768 and
    8 x 8 192 context tokens, the whole entry call (split, merge) timed like
    the other short lines (`_time_ms_warm`)."""
    import torch
    import __graft_entry__ as ge
    pkg = ge.load_package()
    import vllm_jax_amd.workloads as wl
    dev = torch.device("cuda:0")
    res = []
    for batch, ctx in ((1, 32768), (1, 131072), (2, 16384), (4, 32768), (8, 8192)):
        db = wl.make_decode([ctx] * batch, num_heads=32, num_kv_heads=8, page_size=256,
                            rng=np.random.default_rng(1))
        d = wl.materialize_decode(db, seed=1, device=dev)
        kv = d["kv_cache"]
        kp, vp = kv[0].permute(2, 0, 1, 3), kv[1].permute(2, 0, 1, 3)
        out = torch.empty_like(d["q"])
        ws = torch.empty(pkg._lib.load().pa_decode_workspace_size(db.batch, 32, 128, db.block_tables.shape[1], 256),
                         dtype=torch.uint8, device=dev)

        def call():
            pkg.decode_paged_attention(d["q"], kp, vp, d["block_tables"], d["context_lens"], scale=1 / 11.3125,
                                       workspace=ws, out=out)
        ms = _time_ms_warm(torch, call, args)
        gbs = db.hbm_bytes() / (ms * 1e-3) / 1e9
        res.append({"seqs": batch, "context": ctx, "gb": round(db.hbm_bytes() / 1e9, 4), "us": round(ms * 1e3, 1),
                    "gbs": round(gbs, 1), "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)})
        del d, kv, kp, vp, out, ws
        torch.cuda.empty_cache()
    return {"metric": "decode attn GB/s, a few long sequences (head size 128, 32 q / 8 kv heads)",
            "results": res, "steps": args.steps, "warmup": args.warmup}


def _time_ms(torch, fn, args):
    for _ in range(args.warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / args.steps


def _time_ms_warm(torch, fn, args, warm_ms=150.0, rounds=3):
    """`_time_ms` for short launches timed in a fresh process: launches run
    back to back until at least `warm_ms` of GPU time has passed (the part's
    clock ramps up over its first milliseconds of work), then the median of
    `rounds` timings of `steps` launches."""
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    spent = 0.0
    while spent < warm_ms:
        e0.record()
        for _ in range(max(args.warmup, 1)):
            fn()
        e1.record()
        torch.cuda.synchronize()
        spent += e0.elapsed_time(e1)
    times = []
    for _ in range(rounds):
        e0.record()
        for _ in range(args.steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) / args.steps)
    return float(np.median(times))


def run_gpu(args):
    import torch
    import __graft_entry__ as ge
    pkg = ge.load_package()
    import vllm_jax_amd.workloads as wl

    pkg._lib.load()  # fail loudly if the HIP library is missing
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    # ---------------- prefill: Qwen3-32B long context
    pb = wl.qwen3_32b_long_prefill(seed=4)
    pt = wl.materialize_prefill(pb, seed=4, device=dev, fill_pool=False) \
        if args.only not in ("decode", "mixed", "decode_fp8", "prefix", "prefill_fp8", "long8", "g32") else None
    if pt is None:  # decode-only profiling run: keep the prefill half tiny
        pb = wl.make_prefill([64], num_heads=64, num_kv_heads=8, rng=np.random.default_rng(0))
        pt = wl.materialize_prefill(pb, seed=4, device=dev, fill_pool=False)
    kv_p = pt["kv_cache"]
    kp_p, vp_p = kv_p[0].permute(2, 0, 1, 3), kv_p[1].permute(2, 0, 1, 3)
    out_p = torch.empty_like(pt["q"])

    def prefill_step():
        pkg.update_kv_cache(kv_p, pt["slot_mapping"], pt["k"], pt["v"])

    def prefill_attn():
        pkg.prefill_paged_attention(pt["q"], kp_p, vp_p, pt["block_tables"], pt["cu_seqlens_q"],
                                    pt["slot_mapping"], pt["input_positions"],
                                    max_seqlen_bucket=pb.max_seqlen_bucket, out=out_p)

    # ---------------- decode: Qwen3-8B
    db = wl.qwen3_8b_decode(seed=2) if args.only not in ("prefill", "rope", "mixed", "prefix", "long8", "g32") else \
        wl.make_decode([64], num_heads=32, num_kv_heads=8, rng=np.random.default_rng(0))
    dt_ = wl.materialize_decode(db, seed=2, device=dev)
    kv_d = dt_["kv_cache"]
    kp_d, vp_d = kv_d[0].permute(2, 0, 1, 3), kv_d[1].permute(2, 0, 1, 3)
    out_d = torch.empty_like(dt_["q"])
    from vllm_jax_amd.kernels.decode_paged_attention import decode_workspace_bytes
    ws = torch.empty(decode_workspace_bytes(db.batch, db.num_heads, db.head_dim, db.block_tables.shape[1],
                                            db.page_size), dtype=torch.uint8, device=dev)
    dscale = 1.0 / 11.3125  # 1/bf16(sqrt(128)), folded into the kernel

    def decode_step():
        pkg.update_kv_cache(kv_d, dt_["slot_mapping"], dt_["k"], dt_["v"])

    def decode_attn():
        pkg.decode_paged_attention(dt_["q"], kp_d, vp_d, dt_["block_tables"], dt_["context_lens"],
                                   scale=dscale, workspace=ws, out=out_d)

    run_p = args.only in (None, "prefill")
    run_d = args.only in (None, "decode")
    run_r = args.only in (None, "rope")
    run_m = args.only in (None, "mixed")
    run_f = args.only in (None, "decode_fp8")
    run_x = args.only in (None, "prefix", "prefill_fp8")
    nop = lambda: None
    if not run_p:
        prefill_step = prefill_attn = nop
    if not run_d:
        decode_step = decode_attn = nop
    for _ in range(args.warmup):
        prefill_step(); prefill_attn(); decode_step(); decode_attn()
    torch.cuda.synchronize()

    k = args.steps
    ev = [_events(torch, 6) for _ in range(k)]
    t_begin, t_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    t_begin.record()
    for i in range(k):
        e = ev[i]
        e[0].record(); prefill_step(); e[1].record(); prefill_attn(); e[2].record()
        decode_step(); e[3].record(); decode_attn(); e[4].record()
    t_end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0

    total_ms = t_begin.elapsed_time(t_end)
    p_store = np.array([e[0].elapsed_time(e[1]) for e in ev])
    p_attn = np.array([e[1].elapsed_time(e[2]) for e in ev])
    d_store = np.array([e[2].elapsed_time(e[3]) for e in ev])
    d_attn = np.array([e[3].elapsed_time(e[4]) for e in ev])

    p_flops = pb.flops()
    d_bytes = db.hbm_bytes()
    prefill_step_ms = float((p_store + p_attn).mean())
    decode_step_ms = float((d_store + d_attn).mean())
    rate = lambda work, ms, unit: work / (ms * 1e-3) / unit if ms > 0 else 0.0
    p_tflops_step = rate(p_flops, prefill_step_ms, 1e12)
    p_tflops_kernel = rate(p_flops, float(p_attn.mean()), 1e12)
    d_gbs_step = rate(d_bytes, decode_step_ms, 1e9)
    d_gbs_kernel = rate(d_bytes, float(d_attn.mean()), 1e9)

    rope = run_rope(args, torch, pkg, pb, pt, kv_p) if run_r else None
    c1 = run_c1(args, torch, pkg, wl, dev, cpu=not args.no_cpu_baseline) if args.only is None else None
    mixed = run_mixed(args, torch, pkg, wl, dev) if run_m else None
    prefix, pre8 = run_prefix(args, torch, pkg, wl, dev, fp8=args.only in (None, "prefill_fp8")) \
        if run_x else (None, None)
    if prefix is not None:
        prefix["roofline"]["traffic"] = _load_traffic().get("prefill_kernel_prefix_cached")
    dec8 = run_decode_fp8(args, torch, pkg, db, dt_, ws, dscale, float(d_attn.mean()) if run_d else None) \
        if run_f else None

    long8 = run_long8(args, torch, pkg, wl, dev) if args.only in (None, "long8") else None
    g32 = run_g32(args, torch, pkg, wl, dev) if args.only in (None, "g32") else None

    traffic = _load_traffic()
    res = {
        "metric": METRIC,
        "value": round(p_tflops_step, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": k,
        "warmup": args.warmup,
        "ms_per_step": round(total_ms / k, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (0.5*N(0,1) bf16 q/k/v, seeded block-table permutations)",
        "config": {
            "workload": "qwen3_32b_long_prefill (seed 4) + qwen3_8b_decode (seed 2)",
            "prefill": {"seqs": int(pb.batch), "q_lens": [int(x) for x in pb.q_lens], "num_heads": 64,
                        "num_kv_heads": 8, "head_dim": 128, "page_size": 256, "tokens": pb.num_tokens,
                        "algorithmic_tflop": round(p_flops / 1e12, 4)},
            "decode": {"seqs": int(db.batch), "num_heads": 32, "num_kv_heads": 8, "head_dim": 128,
                       "page_size": 256, "pool_pages": db.num_pages,
                       "context_tokens": int(db.context_lens.sum()),
                       "algorithmic_gb": round(d_bytes / 1e9, 4)},
            "parallelism": "single GPU",
        },
        "prefill": {
            "step_ms": round(prefill_step_ms, 4),
            "kv_store_ms": round(float(p_store.mean()), 4),
            "attn_ms": round(float(p_attn.mean()), 4),
            "attn_tflops": round(p_tflops_kernel, 2),
            "frac_of_mfma_peak": round(p_tflops_kernel / MFMA_BF16_PEAK_TFLOPS, 4),
        },
        "roofline": {
            "kernel": "prefill_kernel_pooled",
            "bound": "mfma",
            "achieved": round(p_tflops_kernel, 2),
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(p_tflops_kernel / MFMA_BF16_PEAK_TFLOPS, 4),
            "traffic": traffic.get("prefill_kernel"),
        },
        "decode": {
            "metric": "decode attn GB/s",
            "value": round(d_gbs_step, 1),
            "unit": "GB/s",
            "step_ms": round(decode_step_ms, 4),
            "kv_store_ms": round(float(d_store.mean()), 4),
            "attn_ms": round(float(d_attn.mean()), 4),
            "roofline": {
                "kernel": "decode_split_kernel + decode_merge_kernel",
                "bound": "hbm",
                "achieved": round(d_gbs_kernel, 1),
                "peak": HBM_PEAK_GBS,
                "unit": "GB/s",
                "frac": round(d_gbs_kernel / HBM_PEAK_GBS, 4),
                "traffic": (traffic["decode_split_kernel"] + traffic["decode_merge_kernel"]
                            if "decode_split_kernel" in traffic and "decode_merge_kernel" in traffic else None),
            },
        },
        "wall_s_timed": round(wall, 3),
    }
    if rope is not None:
        rope["roofline"]["traffic"] = traffic.get("qk_norm_rope_store_kernel")
        res["qk_norm_rope"] = rope
    if mixed is not None:
        mixed["roofline"]["traffic"] = traffic.get("mixed_kernel")
        res["mixed"] = mixed
    if c1 is not None:
        res["qwen3_06b_prefill"] = c1
    if prefix is not None:
        res["prefix_prefill"] = prefix
    if pre8 is not None:
        pre8["roofline"]["traffic"] = traffic.get("prefill_fp8_path")
        res["prefill_fp8"] = pre8
    if dec8 is not None:
        dec8["roofline"]["traffic"] = traffic.get("decode_fp8_split_kernel")
        res["decode_fp8"] = dec8
    if long8 is not None:
        long8["roofline"]["traffic"] = traffic.get("prefill_kernel_qwen3_8b_long")
        res["qwen3_8b_long_prefill"] = long8
    if g32 is not None:
        g32["roofline"]["traffic"] = traffic.get("decode_any_kernel_g32")
        res["decode_g32"] = g32
    return res, (pb, pt, db, dt_)


def run_long8(args, torch, pkg, wl, dev):
    """Time a plain Qwen3-8B-shaped prefill: the long prefill's 8 sequence
    lengths (213 732 tokens) at 32 q / 8 kv heads (64-token q tiles of 4
    heads), attention only."""
    pb = wl.qwen3_8b_long_prefill(seed=4)
    t = wl.materialize_prefill(pb, seed=4, device=dev, fill_pool=True)
    kp, vp = t["kv_cache"][0].permute(2, 0, 1, 3), t["kv_cache"][1].permute(2, 0, 1, 3)
    out = torch.empty_like(t["q"])

    def attn():
        pkg.prefill_paged_attention(t["q"], kp, vp, t["block_tables"], t["cu_seqlens_q"], t["slot_mapping"],
                                    t["input_positions"], max_seqlen_bucket=pb.max_seqlen_bucket, out=out)
    quick = argparse.Namespace(warmup=min(args.warmup, 2), steps=min(max(args.steps, 3), 5))
    ms = _time_ms(torch, attn, quick)
    tf = pb.flops() / (ms * 1e-3) / 1e12
    del t, kp, vp, out
    torch.cuda.empty_cache()
    return {
        "metric": "Qwen3-8B-shaped long prefill attn TFLOP/s",
        "seqs": int(pb.batch), "tokens": int(pb.num_tokens), "num_heads": 32, "num_kv_heads": 8,
        "algorithmic_tflop": round(pb.flops() / 1e12, 4), "attn_ms": round(ms, 4), "steps": quick.steps,
        "roofline": {"kernel": "prefill_kernel_pooled", "bound": "mfma", "achieved": round(tf, 2),
                     "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
                     "traffic": None},
    }


def run_g32(args, torch, pkg, wl, dev):
    """Time decode with 32 q heads per kv head (64 q / 2 kv heads, the
    Qwen3-8B decode batch's contexts): pa_decode runs the generic kernel,
    one item of 32 q heads per (sequence, chunk, kv head)."""
    db = wl.g32_decode(seed=2)
    d = wl.materialize_decode(db, seed=2, device=dev)
    kv = d["kv_cache"]
    kp, vp = kv[0].permute(2, 0, 1, 3), kv[1].permute(2, 0, 1, 3)
    out = torch.empty_like(d["q"])
    from vllm_jax_amd.kernels.decode_paged_attention import decode_workspace_bytes
    ws = torch.empty(decode_workspace_bytes(db.batch, db.num_heads, db.head_dim, db.block_tables.shape[1],
                                            db.page_size), dtype=torch.uint8, device=dev)

    def call():
        pkg.decode_paged_attention(d["q"], kp, vp, d["block_tables"], d["context_lens"], scale=1.0 / 11.3125,
                                   workspace=ws, out=out)
    ms = _time_ms_warm(torch, call, args)
    gbs = db.hbm_bytes() / (ms * 1e-3) / 1e9
    del d, kv, kp, vp, out, ws
    torch.cuda.empty_cache()
    return {
        "metric": "decode attn GB/s, 32 q heads per kv head",
        "seqs": int(db.batch), "num_heads": 64, "num_kv_heads": 2, "algorithmic_gb": round(db.hbm_bytes() / 1e9, 4),
        "attn_ms": round(ms, 4),
        "roofline": {"kernel": "decode_any_kernel<128, false, true, false, true> + decode_any_merge_kernel",
                     "bound": "hbm",
                     "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None},
    }


def run_decode_fp8(args, torch, pkg, db, dt_, ws, dscale, bf16_ms):
    """Quantise the decode pool to float8 pages on the device and time the
    quantized split-K decode of the same batch."""
    kv = dt_["kv_cache"]
    nb, bs, hkv, d = kv.shape[1:]
    codes = torch.empty((2, nb, bs, hkv, d), dtype=torch.float8_e4m3fn, device=kv.device)
    scales = torch.empty((2, hkv, nb, bs), dtype=torch.float32, device=kv.device)
    pkg.update_kv_cache_fp8(codes, scales, torch.arange(nb * bs, dtype=torch.int32, device=kv.device),
                            kv[0].reshape(-1, hkv, d), kv[1].reshape(-1, hkv, d))
    out = torch.empty_like(dt_["q"])
    kp, vp = codes[0].permute(2, 0, 1, 3), codes[1].permute(2, 0, 1, 3)

    def call():
        pkg.decode_paged_attention(dt_["q"], kp, vp, dt_["block_tables"], dt_["context_lens"],
                                   k_scales_pages=scales[0], v_scales_pages=scales[1], scale=dscale,
                                   workspace=ws, out=out)

    ms = _time_ms_warm(torch, call, args)
    ctx = int(db.context_lens.sum())
    pages = int(np.ceil(db.context_lens / db.page_size).sum())
    nbytes = ctx * hkv * (2 * d + 8) + 2 * db.batch * db.num_heads * d * 2 + 4 * pages + 4 * db.batch
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {
        "metric": "decode attn GB/s over float8 e4m3 pages",
        "algorithmic_gb": round(nbytes / 1e9, 4),
        "attn_ms": round(ms, 4),
        "bf16_attn_ms": round(bf16_ms, 4) if bf16_ms else None,
        "speedup_vs_bf16": round(bf16_ms / ms, 3) if bf16_ms else None,
        "roofline": {"kernel": "decode_split_kernel<true, false, true> + decode_merge_kernel", "bound": "hbm",
                     "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None},
    }


def run_prefix(args, torch, pkg, wl, dev, fp8=False):
    """Time the Qwen3-8B prefix-cached prefill: new tokens stored, then the
    causal prefill over cached + new K/V.  With ``fp8``, also the same batch
    over float8 pages (``run_prefix_fp8``)."""
    pb = wl.qwen3_8b_prefix_prefill(seed=3)
    t = wl.materialize_prefill(pb, seed=3, device=dev, fill_pool=True)
    kv = t["kv_cache"]
    kp, vp = kv[0].permute(2, 0, 1, 3), kv[1].permute(2, 0, 1, 3)
    out = torch.empty_like(t["q"])

    def store():
        pkg.update_kv_cache(kv, t["slot_mapping"], t["k"], t["v"])

    def attn():
        pkg.prefill_paged_attention(t["q"], kp, vp, t["block_tables"], t["cu_seqlens_q"], t["slot_mapping"],
                                    t["input_positions"], max_seqlen_bucket=pb.max_seqlen_bucket,
                                    cu_seqlens_k=t["cu_seqlens_k"], out=out)

    for _ in range(args.warmup):
        store(); attn()
    torch.cuda.synchronize()
    n = max(args.steps, 10)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for e in ev:
        e[0].record(); store(); e[1].record()
    torch.cuda.synchronize()
    st = float(np.mean([e[0].elapsed_time(e[1]) for e in ev]))
    # the attention launch (work list + kernel) on a warm clock, like the
    # other short lines: back-to-back launches, median of three rounds
    at = _time_ms_warm(torch, attn, argparse.Namespace(steps=n, warmup=args.warmup))
    flops = pb.flops()
    tf = flops / (at * 1e-3) / 1e12
    pre8 = run_prefix_fp8(args, torch, pkg, pb, t) if fp8 else None
    return {
        "metric": "prefix-cached prefill attn TFLOP/s",
        "seqs": int(pb.batch), "new_tokens": int(pb.num_tokens),
        "cached_tokens": int(pb.prefix_lens.sum()), "algorithmic_tflop": round(flops / 1e12, 4),
        "kv_store_ms": round(st, 4), "attn_ms": round(at, 4),
        "timing": "attention launches back to back after 150 ms of warm-up launches, median of 3 rounds",
        "attn_tflops": round(tf, 2), "frac_of_mfma_peak": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
        "roofline": {"kernel": "prefill_kernel", "bound": "mfma", "achieved": round(tf, 2),
                     "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
                     "traffic": None},
    }, pre8


def run_prefix_fp8(args, torch, pkg, pb, t):
    """The prefix-cached prefill over float8 e4m3 pages: the bf16 pool
    quantised on the device, then per call every distinct page in use
    widened once to bf16 and the bf16 prefill over the remapped table."""
    kv = t["kv_cache"]
    nb, bs, hkv, d = kv.shape[1:]
    codes = torch.empty((2, nb, bs, hkv, d), dtype=torch.float8_e4m3fn, device=kv.device)
    scales = torch.empty((2, hkv, nb, bs), dtype=torch.float32, device=kv.device)
    pkg.update_kv_cache_fp8(codes, scales, torch.arange(nb * bs, dtype=torch.int32, device=kv.device),
                            kv[0].reshape(-1, hkv, d), kv[1].reshape(-1, hkv, d))
    kp, vp = codes[0].permute(2, 0, 1, 3), codes[1].permute(2, 0, 1, 3)
    bt = t["block_tables"]
    lib = pkg._lib.load()
    need = lib.pa_prefill_fp8_workspace_size(pb.batch, bt.shape[1], bs, hkv, d, int(pb.max_seqlen_bucket),
                                             pb.num_heads)
    ws = torch.empty(need, dtype=torch.uint8, device=kv.device)
    out = torch.empty_like(t["q"])

    def call():
        pkg.prefill_paged_attention(t["q"], kp, vp, bt, t["cu_seqlens_q"], t["slot_mapping"],
                                    t["input_positions"], max_seqlen_bucket=pb.max_seqlen_bucket,
                                    cu_seqlens_k=t["cu_seqlens_k"], k_scales_pages=scales[0],
                                    v_scales_pages=scales[1], workspace=ws, out=out)

    out16 = torch.empty_like(t["q"])
    kp16, vp16 = kv[0].permute(2, 0, 1, 3), kv[1].permute(2, 0, 1, 3)

    def call16():
        pkg.prefill_paged_attention(t["q"], kp16, vp16, bt, t["cu_seqlens_q"], t["slot_mapping"],
                                    t["input_positions"], max_seqlen_bucket=pb.max_seqlen_bucket,
                                    cu_seqlens_k=t["cu_seqlens_k"], out=out16)

    def timed(fn):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    # The part is power-limited, so the float8 and bf16 prefills alternate
    # (order swapped every round) and each reports the median of its rounds.
    for _ in range(args.warmup):
        call(); call16()
    torch.cuda.synchronize()
    n = max(args.steps, 10)
    t8, t16 = [], []
    for r in range(4):
        for fn, acc in (((call, t8), (call16, t16)) if r % 2 == 0 else ((call16, t16), (call, t8))):
            acc.append(timed(fn))
    ms, bf16_ms = float(np.median(t8)), float(np.median(t16))
    # the widening leaves its page count after the widened pages, the
    # remapped table and the pages' owner entries
    entries = pb.batch * bt.shape[1]
    at = 2 * entries * bs * hkv * d * 2 + 2 * entries * 4
    widened = int(ws[at:at + 4].cpu().numpy().view(np.int32)[0])
    kv_lens = (pb.prefix_lens + pb.q_lens).astype(np.int64)
    in_use = int(np.sum(-(-kv_lens // bs)))
    tf = pb.flops() / (ms * 1e-3) / 1e12
    return {
        "metric": "prefix-cached prefill attn TFLOP/s over float8 e4m3 pages (widening included)",
        "attn_ms": round(ms, 4), "bf16_attn_ms": round(bf16_ms, 4),
        "timing": "float8 and bf16 launches alternate over 4 rounds of max(steps, 10); medians",
        "widened_pages": widened, "table_entries_in_use": in_use,
        "attn_tflops": round(tf, 2), "frac_of_mfma_peak": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
        "roofline": {"kernel": "fp8_pages_widen_kernel + prefill_kernel", "bound": "mfma", "achieved": round(tf, 2),
                     "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
                     "traffic": None},
    }


def run_mixed(args, torch, pkg, wl, dev):
    """Time the Qwen3-0.6B mixed step: one pa_mixed launch vs pa_decode + pa_prefill."""
    pre, dec = wl.qwen3_06b_mixed(1)
    mb = wl.make_mixed(pre, dec)
    t = wl.materialize_mixed(mb, seed=1, device=dev)
    kv = t["kv_cache"]
    pkg.update_kv_cache(kv, t["slot_mapping"], t["k"], t["v"])
    kp, vp = kv[0].permute(2, 0, 1, 3), kv[1].permute(2, 0, 1, 3)
    nd, base = mb.num_decodes, int(mb.cu_seqlens_q[mb.num_decodes])
    from vllm_jax_amd.kernels.decode_paged_attention import decode_workspace_bytes
    ws = torch.empty(decode_workspace_bytes(nd, mb.prefill.num_heads, 128, mb.block_tables.shape[1],
                                            mb.prefill.page_size), dtype=torch.uint8, device=dev)
    out = torch.empty_like(t["q"])
    qd = t["q"][:nd].contiguous()
    od = torch.empty_like(qd)
    op = torch.empty_like(t["q"][base:])
    cup = t["cu_seqlens_q"][nd:] - base
    cuk = torch.as_tensor(np.concatenate([[0], np.cumsum(mb.kv_lens[nd:])]).astype(np.int32), device=dev)
    dscale = 1.0 / 11.3125

    def one():
        pkg.mixed_paged_attention(t["q"], kp, vp, t["block_tables"], t["cu_seqlens_q"], t["kv_lens"],
                                  t["input_positions"], nd, max_seqlen_q=mb.max_seqlen_q, decode_scale=dscale,
                                  out=out)

    def two():
        pkg.decode_paged_attention(qd, kp, vp, t["block_tables"][:nd], t["kv_lens"][:nd], scale=dscale,
                                   workspace=ws, out=od)
        pkg.prefill_paged_attention(t["q"][base:], kp, vp, t["block_tables"][nd:], cup, None,
                                    t["input_positions"][base:], max_seqlen_bucket=mb.max_seqlen_q,
                                    cu_seqlens_k=cuk, out=op)

    def timed(fn):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(max(args.steps, 10)):   # launches queue ahead of the host
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / max(args.steps, 10)

    # The part is power-limited, so a launch's speed depends on what ran just
    # before it: the two paths alternate, the order swapped every round, and
    # each reports the median of its rounds.
    for _ in range(args.warmup):
        one(); two()
    torch.cuda.synchronize()
    t_one, t_two = [], []
    for r in range(6):
        for fn, acc in (((one, t_one), (two, t_two)) if r % 2 == 0 else ((two, t_two), (one, t_one))):
            acc.append(timed(fn))
    ms_one, ms_two = float(np.median(t_one)), float(np.median(t_two))
    flops, dbytes = pre.flops(), dec.hbm_bytes()
    # The step is a prefill half bound by the matrix cores and a decode half
    # bound by HBM; the serial roof is the time of each half at its own peak,
    # added (a kernel that overlapped the halves perfectly could beat it).
    roof_ms = (flops / (MFMA_BF16_PEAK_TFLOPS * 1e12) + dbytes / (HBM_PEAK_GBS * 1e9)) * 1e3
    return {
        "metric": "mixed step ms (one launch vs decode + prefill launches)",
        "decode_seqs": int(nd), "prefill_seqs": int(pre.batch), "tokens": int(mb.num_tokens),
        "prefill_gflop": round(flops / 1e9, 3), "decode_gb": round(dbytes / 1e9, 4),
        "one_launch_ms": round(ms_one, 4), "two_launches_ms": round(ms_two, 4),
        "speedup": round(ms_two / ms_one, 3) if ms_one > 0 else None,
        "roofline": {"kernel": "mixed_kernel", "bound": "mfma+hbm (serial: prefill flops at the bf16 MFMA peak "
                     "plus decode bytes at the HBM peak)", "achieved": round(ms_one, 4),
                     "peak": round(roof_ms, 4), "unit": "ms", "frac": round(roof_ms / ms_one, 4) if ms_one > 0 else None,
                     "traffic": None},
    }


def run_c1(args, torch, pkg, wl, dev, cpu):
    """The Qwen3-0.6B single-layer prefill, the configuration the reference
    can run on its CPU path: 4 sequences [17, 128, 300, 511], 16 q / 8 kv
    heads, a 64 x 256-token pool, seed 0.  One step = KV store of the 956 new
    tokens + the causal prefill, on the GPU (median of the timed steps) and in
    the CPU oracle (median of 5 runs of the same full step)."""
    pb = wl.qwen3_06b_prefill()
    t = wl.materialize_prefill(pb, seed=0, device=dev)
    kv = t["kv_cache"]
    kp, vp = kv[0].permute(2, 0, 1, 3), kv[1].permute(2, 0, 1, 3)
    out = torch.empty_like(t["q"])

    def step():
        pkg.update_kv_cache(kv, t["slot_mapping"], t["k"], t["v"])
        pkg.prefill_paged_attention(t["q"], kp, vp, t["block_tables"], t["cu_seqlens_q"], t["slot_mapping"],
                                    t["input_positions"], max_seqlen_bucket=pb.max_seqlen_bucket, out=out)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    n = max(args.steps, 20)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for e in ev:
        e[0].record(); step(); e[1].record()
    torch.cuda.synchronize()
    gpu_ms = float(np.median([e[0].elapsed_time(e[1]) for e in ev]))
    flops = pb.flops()
    res = {"metric": "Qwen3-0.6B single-layer prefill step (KV store + attention) TFLOP/s",
           "q_lens": [int(x) for x in pb.q_lens], "algorithmic_gflop": round(flops / 1e9, 4),
           "gpu_step_ms": round(gpu_ms, 4), "gpu_tflops": round(flops / (gpu_ms * 1e-3) / 1e12, 3)}
    if cpu:
        from oracle import paged_attention_oracle as ora
        u16 = lambda x: x.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
        kc0, vc0 = u16(kv[0]), u16(kv[1])
        qh, kh, vh = u16(t["q"]), u16(t["k"]), u16(t["v"])
        times = []
        for _ in range(5):
            t0 = time.perf_counter()
            kc, vc = ora.kv_store(kc0, vc0, kh, vh, pb.slot_mapping)
            ora.prefill_attention(qh, kc.transpose(2, 0, 1, 3), vc.transpose(2, 0, 1, 3), pb.block_tables,
                                  pb.cu_seqlens_q, pb.input_positions)
            times.append(time.perf_counter() - t0)
        cpu_s = float(np.median(times))
        threads = _blas_threads()
        res["cpu_baseline"] = {"value": round(flops / cpu_s / 1e12, 6), "unit": "TFLOP/s", "cores": threads,
                               "kind": "port", "step_ms": round(cpu_s * 1e3, 2),
                               "sample": f"the whole configuration: CPU oracle (numpy, {threads} BLAS threads of "
                                         f"{os.cpu_count()} host CPUs) KV store + prefill, median of 5 runs "
                                         f"({', '.join(f'{x * 1e3:.0f}' for x in times)} ms)"}
        res["gpu_over_cpu"] = round(cpu_s * 1e3 / gpu_ms, 1)
    return res


def _blas_threads() -> int:
    try:
        from threadpoolctl import threadpool_info
        return int(max([i.get("num_threads", 1) for i in threadpool_info()] or [1]))
    except Exception:  # pragma: no cover
        return 1


def run_rope(args, torch, pkg, pb, pt, kv):
    """Time the fused q/k RMSNorm + RoPE + KV store on the prefill tokens."""
    g = torch.Generator(device=kv.device)
    g.manual_seed(7)
    d = pb.head_dim
    qw = (1.0 + 0.1 * torch.randn(d, generator=g, device=kv.device)).to(torch.bfloat16)
    kw = (1.0 + 0.1 * torch.randn(d, generator=g, device=kv.device)).to(torch.bfloat16)
    q_out = torch.empty_like(pt["q"])

    def call():
        pkg.qk_norm_rope_store(pt["q"], pt["k"], pt["v"], qw, kw, pt["input_positions"], pt["slot_mapping"], kv,
                               eps=1e-6, rope_theta=1e6, out=q_out)

    for _ in range(args.warmup):
        call()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(args.steps):
        call()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    t = pb.num_tokens
    nbytes = t * ((2 * pb.num_heads + 4 * pb.num_kv_heads) * d * 2 + 8)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {
        "metric": "fused qk rmsnorm + rope + kv store GB/s",
        "tokens": int(t), "num_heads": int(pb.num_heads), "num_kv_heads": int(pb.num_kv_heads),
        "algorithmic_gb": round(nbytes / 1e9, 4),
        "ms": round(ms, 4),
        "roofline": {"kernel": "qk_norm_rope_store_kernel", "bound": "hbm", "achieved": round(gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None},
    }


def cpu_baseline(pb, pt, db, dt_, budget_s):
    """Time the CPU oracle on bounded samples of the two workloads (host
    cores).  Each sample is sized so that one run takes about a sixth of the
    budget, then run 3 times; the median is reported."""
    import torch
    from oracle import paged_attention_oracle as ora
    threads = _blas_threads()
    u16 = lambda x: x.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
    runs = 3
    per_run = budget_s / (2 * runs)

    # prefill sample: the last R q rows of the shortest sequence, against its whole context
    b = int(np.argmin(pb.q_lens))
    q0, q1 = int(pb.cu_seqlens_q[b]), int(pb.cu_seqlens_q[b + 1])
    n_pages = -(-(q1 - q0) // pb.page_size)
    blocks = torch.as_tensor(pb.block_tables[b, :n_pages].astype(np.int64), device=pt["q"].device)
    kv = pt["kv_cache"]
    kp = u16(kv[0][blocks]).transpose(2, 0, 1, 3)
    vp = u16(kv[1][blocks]).transpose(2, 0, 1, 3)
    qh = u16(pt["q"][q0:q1])
    bt = np.arange(n_pages, dtype=np.int32)[None]
    cu = np.array([0, q1 - q0], np.int32)
    pos = pb.input_positions[q0:q1]
    rows_n = 8
    while True:
        rows = np.arange(q1 - q0 - rows_n, q1 - q0)
        t0 = time.perf_counter()
        ora.prefill_attention(qh, kp, vp, bt, cu, pos, rows=rows)
        dt = time.perf_counter() - t0
        if dt * 2.2 > per_run or rows_n >= 4096:
            break
        rows_n *= 2
    times = [dt]
    for _ in range(runs - 1):
        t0 = time.perf_counter()
        ora.prefill_attention(qh, kp, vp, bt, cu, pos, rows=rows)
        times.append(time.perf_counter() - t0)
    spent = float(np.median(times))
    flops = 4 * pb.head_dim * pb.num_heads * int((pos[rows] + 1).sum())
    p_val = flops / spent / 1e12

    # decode sample: the first S sequences
    s_n = 2
    kvd = dt_["kv_cache"]
    qd = dt_["q"]
    while True:
        used = sorted(set(int(x) for x in db.block_tables[:s_n].ravel() if x >= 0))
        remap = {blk: i for i, blk in enumerate(used)}
        bt_s = np.array([[remap.get(int(x), 0) if x >= 0 else -1 for x in row] for row in db.block_tables[:s_n]],
                        np.int32)
        idx = torch.as_tensor(used, dtype=torch.long, device=qd.device)
        kp_s = u16(kvd[0][idx]).transpose(2, 0, 1, 3)
        vp_s = u16(kvd[1][idx]).transpose(2, 0, 1, 3)
        qs = u16(qd[:s_n])
        t0 = time.perf_counter()
        ora.decode_attention(qs, kp_s, vp_s, bt_s, db.context_lens[:s_n])
        dt = time.perf_counter() - t0
        if dt * 2.2 > per_run or s_n >= db.batch:
            break
        s_n = min(s_n * 2, db.batch)
    d_times = [dt]
    for _ in range(runs - 1):
        t0 = time.perf_counter()
        ora.decode_attention(qs, kp_s, vp_s, bt_s, db.context_lens[:s_n])
        d_times.append(time.perf_counter() - t0)
    d_spent = float(np.median(d_times))
    d_bytes = int(db.context_lens[:s_n].sum()) * 2 * db.num_kv_heads * db.head_dim * 2
    d_val = d_bytes / d_spent / 1e9
    ncpu = os.cpu_count()
    fmt = lambda ts: ", ".join(f"{x:.2f}" for x in ts)
    return (
        {"value": round(p_val, 6), "unit": "TFLOP/s", "cores": int(threads), "kind": "port",
         "sample": f"CPU oracle (numpy, {threads} BLAS threads of {ncpu} host CPUs): prefill of the last "
                   f"{rows_n} q rows of the {q1 - q0}-token sequence against its whole causal context, "
                   f"{flops / 1e9:.1f} GFLOP, median of {runs} runs ({fmt(times)} s)"},
        {"value": round(d_val, 4), "unit": "GB/s", "cores": int(threads), "kind": "port",
         "sample": f"CPU oracle decode of the first {s_n} sequences ({d_bytes / 1e9:.3f} GB KV), median of "
                   f"{runs} runs ({fmt(d_times)} s)"},
    )


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--cpu-budget", type=float, default=24.0, help="seconds of CPU oracle work (total)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", choices=["prefill", "decode", "rope", "mixed", "decode_fp8", "prefix", "prefill_fp8",
                                       "long8", "g32",
                                       "copy", "head_dims", "page_sizes", "small_decode", "soft_cap"],
                    default=None,
                    help="profiling aid: run one kernel family only (the JSON line then covers that part)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this paged-attention path is built and measured on a single "
              "MI355X (it would shard over kv heads or sequences with no exchange between GPUs). "
              f"--gpus {args.gpus} is not supported.", file=sys.stderr)
        sys.exit(2)
    if args.only == "copy":
        print(json.dumps(run_copy(args)), flush=True)
        return
    if args.only == "head_dims":
        print(json.dumps(run_head_dims(args)), flush=True)
        return
    if args.only == "soft_cap":
        print(json.dumps(run_soft_cap(args)), flush=True)
        return
    if args.only == "page_sizes":
        print(json.dumps(run_page_sizes(args)), flush=True)
        return
    if args.only == "small_decode":
        print(json.dumps(run_small_decode(args)), flush=True)
        return
    res, ctx = run_gpu(args)
    if args.only is not None:
        res["only"] = args.only
    if not args.no_cpu_baseline and args.only is None:
        pcb, dcb = cpu_baseline(*ctx, budget_s=args.cpu_budget)
        res["cpu_baseline"] = pcb
        res["decode"]["cpu_baseline"] = dcb
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
