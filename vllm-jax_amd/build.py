"""Build recipe for libpaged_attention.so (gfx950).

Compiles every HIP/C++ source under ``csrc/`` with hipcc into one shared
library next to this file.  Run ``python vllm-jax_amd/build.py`` or call
:func:`build`.  hipcc cross-compiles for gfx950 without a GPU present.

``python vllm-jax_amd/build.py --phases`` (or ``build(phases=True)``) builds
only ``libpaged_attention_phases.so`` at the repository root instead: the
prefill entry points compiled with ``PA_PREFILL_PHASES``, whose kernel
records per-workgroup phase timestamps for the measurement script
``prefill_phases.py``.  The package never loads it, and the default build
does not make it.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_NAME = "libpaged_attention.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
PHASES_LIB_PATH = os.path.join(os.path.dirname(PKG_DIR), "libpaged_attention_phases.so")
ARCH = "gfx950"

SOURCES = ["pa_errors.cpp", "block_manager.cpp", "kv_store.hip", "decode.hip", "prefill.hip", "qk_norm_rope.hip",
           "mixed.hip", "any_head.hip"]
PHASES_SOURCES = ["pa_errors.cpp", "prefill.hip", "any_head.hip"]  # any_head: the head-size check of the quantized entries

# Packed-FP32 VALU forms are disabled for every device compile: the build
# relies on scalar/float2 code only.  Without NaN semantics, fmaxf lowers to a
# single v_max (no canonicalising v_max x,x before each operand).
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                # inputs are finite; -inf is still used (and honoured) for masking
                "-fno-honor-nans"]
COMMON_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-result"]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: cannot build the gfx950 paged-attention library")


def build(verbose: bool = False, jobs: int = 4, phases: bool = False) -> str:
    """Compile all sources and link ``libpaged_attention.so``; returns its
    path.  With ``phases`` build only the phase-timestamp prefill library."""
    hipcc = _hipcc()
    with tempfile.TemporaryDirectory(prefix="pa_build_") as tmp:
        procs = []
        libs = ((PHASES_SOURCES, PHASES_LIB_PATH, ["-DPA_PREFILL_PHASES"]),) if phases else ((SOURCES, LIB_PATH, []),)
        for i, (sources, _, defines) in enumerate(libs):
            for src in sources:
                obj = os.path.join(tmp, f"{i}_{src}.o")
                cmd = [hipcc, *COMMON_FLAGS, *defines, "-c", os.path.join(CSRC, src), "-o", obj]
                if src.endswith(".hip"):
                    cmd[1:1] = [f"--offload-arch={ARCH}", *DEVICE_FLAGS]
                procs.append((src, cmd))
        running = []
        for src, cmd in procs:
            if verbose:
                print(" ".join(cmd), flush=True)
            running.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
            if len(running) >= jobs:
                _wait(running.pop(0), verbose)
        for r in running:
            _wait(r, verbose)
        for i, (sources, lib_path, _) in enumerate(libs):
            tmp_lib = os.path.join(tmp, os.path.basename(lib_path))
            objs = [os.path.join(tmp, f"{i}_{src}.o") for src in sources]
            link = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined", "-o", tmp_lib, *objs]
            if verbose:
                print(" ".join(link), flush=True)
            res = subprocess.run(link, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
            if res.returncode != 0:
                raise RuntimeError("link failed:\n" + res.stdout.decode(errors="replace"))
            # Replace atomically so a process that has the old library mapped keeps it.
            shutil.copyfile(tmp_lib, lib_path + ".tmp")
            os.replace(lib_path + ".tmp", lib_path)
    return libs[0][1]


def _wait(item, verbose):
    src, proc = item
    out, _ = proc.communicate()
    text = out.decode(errors="replace")
    # hipcc's host pass does not know the device-only feature flag; that note is noise.
    lines = [ln for ln in text.splitlines() if "packed-fp32-ops" not in ln]
    if proc.returncode != 0:
        raise RuntimeError(f"compiling {src} failed:\n" + "\n".join(lines))
    if verbose and lines:
        print("\n".join(lines), flush=True)


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv, phases="--phases" in sys.argv))
