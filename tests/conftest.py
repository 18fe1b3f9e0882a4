import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def pytest_collection_modifyitems(config, items):
    try:
        import torch
        have_gpu = torch.cuda.is_available()
    except Exception:
        have_gpu = False
    if have_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)


def two_chain_ids(rng, B, L, lo_frac=0.25, hi_frac=0.75):
    """Two contiguous chains per sample, split point ~ U[lo, hi] * L."""
    cid = np.zeros((B, L), dtype=np.int32)
    for b in range(B):
        s = int(rng.integers(int(lo_frac * L), max(int(lo_frac * L) + 1, int(hi_frac * L) + 1)))
        cid[b, s:] = 1
    return cid


def multi_chain_ids(rng, B, L, n):
    """n contiguous chains per sample with random cut points."""
    cid = np.zeros((B, L), dtype=np.int32)
    for b in range(B):
        cuts = np.sort(rng.choice(np.arange(1, L), size=n - 1, replace=False)) if n > 1 else []
        c = 0
        for i in range(L):
            while c < len(cuts) and i >= cuts[c]:
                c += 1
            cid[b, i] = c
    return cid


def tail_padding(rng, B, L, max_frac=0.1):
    pad = np.zeros((B, L), dtype=bool)
    for b in range(B):
        n = int(rng.integers(0, int(max_frac * L) + 1))
        if n:
            pad[b, L - n:] = True
    return pad
