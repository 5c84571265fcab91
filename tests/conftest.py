"""pytest configuration: import paths, the `gpu` marker, shared helpers."""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "axs-6_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built libaxs6.so")
    config.addinivalue_line("markers", "slow: long-running CPU test")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this container")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def bits_equal(a, b) -> bool:
    """Bitwise equality of float arrays, with NaN matched by position only."""
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    if a.shape != b.shape or a.dtype != b.dtype:
        return False
    if a.dtype.kind != "f":
        return np.array_equal(a, b)
    na, nb = np.isnan(a), np.isnan(b)
    if not np.array_equal(na, nb):
        return False
    iv = {2: np.uint16, 4: np.uint32, 8: np.uint64}[a.dtype.itemsize]
    return np.array_equal(a.view(iv)[~na], b.view(iv)[~nb])


def first_mismatch(a, b) -> str:
    a = np.asarray(a).ravel()
    b = np.asarray(b).ravel()
    both_nan = np.isnan(a) & np.isnan(b) if a.dtype.kind == "f" else np.zeros(a.shape, bool)
    iv = {2: np.uint16, 4: np.uint32, 8: np.uint64}.get(a.dtype.itemsize, None)
    if a.dtype.kind == "f" and iv is not None:
        diff = (a.view(iv) != b.view(iv)) & ~both_nan
    else:
        diff = a != b
    idx = np.nonzero(diff)[0]
    if idx.size == 0:
        return "no mismatch"
    i = idx[0]
    return f"{idx.size} mismatches; first at flat {i}: got {a[i]!r} want {b[i]!r}"


def load_golden(name: str):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)
