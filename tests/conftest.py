"""Test configuration: import paths, the ``gpu`` marker, shared helpers.

``-m "not gpu"`` runs here without a GPU: the oracle against the golden
fixtures and the mathematics, host logic, and the C ABI's exports and
argument checks.  ``-m gpu`` runs on an MI355X: every kernel through the C
ABI against the oracle, and the Python API end to end.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG_PARENT = ROOT / "distributed-training-framework_amd"
for p in (str(ROOT), str(PKG_PARENT)):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def load_golden(name: str) -> dict:
    with np.load(GOLDEN / name, allow_pickle=False) as d:
        return {k: d[k] for k in d.files}


def same_bits(a: np.ndarray, b: np.ndarray) -> bool:
    """Bitwise equality, except that any NaN equals any NaN (payloads are not compared)."""
    a = np.asarray(a)
    b = np.asarray(b)
    if a.shape != b.shape or a.dtype != b.dtype:
        return False
    if a.dtype == np.float32:
        na, nb = np.isnan(a), np.isnan(b)
        if not np.array_equal(na, nb):
            return False
        return np.array_equal(a.view(np.uint32)[~na], b.view(np.uint32)[~nb])
    if a.dtype == np.uint16:  # bf16 bits
        na = (a & 0x7FFF) > 0x7F80
        nb = (b & 0x7FFF) > 0x7F80
        if not np.array_equal(na, nb):
            return False
        return np.array_equal(a[~na], b[~nb])
    if a.dtype == np.float16:
        na, nb = np.isnan(a), np.isnan(b)
        if not np.array_equal(na, nb):
            return False
        return np.array_equal(a.view(np.uint16)[~na], b.view(np.uint16)[~nb])
    return np.array_equal(a, b)


def first_mismatch(a: np.ndarray, b: np.ndarray) -> str:
    a = np.asarray(a).reshape(-1)
    b = np.asarray(b).reshape(-1)
    if a.shape != b.shape:
        return f"shape {a.shape} vs {b.shape}"
    bits = {np.dtype(np.float32): np.uint32, np.dtype(np.float16): np.uint16}
    ua = a.view(bits[a.dtype]) if a.dtype in bits else a
    ub = b.view(bits[b.dtype]) if b.dtype in bits else b
    idx = np.nonzero(ua != ub)[0]
    if idx.size == 0:
        return "no mismatch"
    i = int(idx[0])
    return f"{idx.size} mismatches; first at {i}: {a[i]!r} ({int(ua[i]):#x}) vs {b[i]!r} ({int(ub[i]):#x})"


def bf16_bits_torch(u):
    """The oracle's fp32 -> bf16 rounding (round to nearest even, NaN -> 0xFFFF) on int64
    tensors of fp32 bit patterns in [0, 2^32), as torch integer ops, so that it can be
    evaluated on the device over all 2^32 patterns.  Returns int64 values in [0, 0xFFFF].
    test_oracle.py checks it against oracle.gradpath.bf16_from_f32."""
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    return r.masked_fill(nan, 0xFFFF)


@pytest.fixture(scope="session")
def rng():
    return np.random.default_rng(1234)
