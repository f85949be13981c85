"""Helpers shared by the parity tests (seeds, uploads, tolerance checks)."""
from __future__ import annotations

import numpy as np

import oracle as O

# Tolerances from the benchmark contract: float outputs with fp32
# accumulation and fp32 output within max relative error 1e-3, fp16 outputs
# within 2e-2, both as max|y - r| / max|r| against the float64 reference.
TOL_F32 = 1e-3
TOL_F16 = 2e-2


def seed_for(cfg: int, sub: int = 0) -> int:
    """Seed rule of the benchmark configurations: 1000 + 10*config + sub."""
    return 1000 + 10 * cfg + sub


def to_dev(a: np.ndarray, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def bits_equal(a: np.ndarray, b: np.ndarray) -> bool:
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    if a.shape != b.shape or a.dtype.itemsize != b.dtype.itemsize:
        return False
    u = {2: np.uint16, 4: np.uint32, 1: np.uint8}[a.dtype.itemsize]
    return bool(np.array_equal(a.view(u), b.view(u)))


def first_mismatch(a: np.ndarray, b: np.ndarray) -> str:
    a = np.ascontiguousarray(a).reshape(-1)
    b = np.ascontiguousarray(b).reshape(-1)
    u = {2: np.uint16, 4: np.uint32, 1: np.uint8}[a.dtype.itemsize]
    idx = np.nonzero(a.view(u) != b.view(u))[0]
    if idx.size == 0:
        return "equal"
    i = int(idx[0])
    return f"{idx.size} mismatches, first at {i}: got {a[i]!r} expected {b[i]!r}"


def rel_err(y, r) -> float:
    return O.max_rel_err(y, r)
