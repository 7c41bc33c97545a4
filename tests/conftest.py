"""Shared test setup: import path, the ``gpu`` marker, common helpers."""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import __graft_entry__  # noqa: E402

PKG = __graft_entry__.load_package()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); parity tests of the gfx950 kernels")


def _has_gpu() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:  # pragma: no cover
        return False


def pytest_collection_modifyitems(config, items):
    if _has_gpu():
        return
    skip = pytest.mark.skip(reason="no HIP device in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def pkg():
    return PKG


@pytest.fixture(scope="session")
def dev():
    import torch
    return torch.device("cuda:0")


def u16(t):
    """bf16 torch tensor -> numpy uint16 bit patterns (on the host)."""
    import torch
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def from_u16(a, device):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(device)


def boundary_rows(cu_seqlens, prefix_lens, rng, *, tile_tokens, page_size=256, kv_tile=64, per_seq=10):
    """q rows to check at full size, spread over every sequence.

    For each sequence (q rows cu[b] .. cu[b+1]-1, kv position of row i is
    prefix_b + i): its first, second, middle and last row; the rows on both
    sides of a q-tile edge (offsets k*tile_tokens - 1 and k*tile_tokens) and
    of a kv page edge and a 64-token kv tile edge (position % page_size and
    % kv_tile in {size - 1, 0}), a few of each picked at random; and random
    interior rows, up to ``per_seq`` rows per sequence in total."""
    cu = np.asarray(cu_seqlens, np.int64)
    out = []
    for b in range(len(cu) - 1):
        q0, n = int(cu[b]), int(cu[b + 1] - cu[b])
        if n <= 0:
            continue
        p = int(prefix_lens[b]) if prefix_lens is not None else 0
        fixed = {0, min(1, n - 1), n // 2, n - 1}
        cand = set()
        for step, base in ((tile_tokens, 0), (page_size, p), (kv_tile, p)):
            # offsets o with (base + o) % step in {step - 1, 0}
            first = (-base) % step
            edges = np.arange(first, n, step)
            edges = np.concatenate([edges, edges - 1])
            edges = edges[(edges >= 0) & (edges < n)]
            if edges.size:
                cand.update(int(x) for x in rng.choice(edges, size=min(2, edges.size), replace=False))
        rows = sorted(fixed | cand)
        extra = max(0, per_seq - len(rows))
        if extra and n > len(rows):
            rows = sorted(set(rows) | set(int(x) for x in rng.integers(0, n, extra)))
        out.extend(q0 + r for r in rows)
    return np.unique(np.asarray(out, np.int64))
