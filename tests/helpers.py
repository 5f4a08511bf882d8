"""Shared helpers for the parity tests (numpy <-> device tensors, tolerances)."""
from __future__ import annotations

import numpy as np


def to_dev(a: np.ndarray, dev):
    """Device tensor holding the same bytes (unsigned dtypes via signed views)."""
    import torch

    a = np.ascontiguousarray(a)
    view = {np.dtype(np.uint8): np.uint8, np.dtype(np.uint16): np.int16, np.dtype(np.uint32): np.int32,
            np.dtype(np.float32): np.float32, np.dtype(np.float16): np.float16,
            np.dtype(np.int32): np.int32}[a.dtype]
    return torch.from_numpy(a.view(view).copy()).to(dev)


def to_np(t, dtype) -> np.ndarray:
    import torch

    torch.cuda.synchronize()
    return t.detach().cpu().numpy().view(dtype)


def rel_err_normwise(y: np.ndarray, ref: np.ndarray) -> float:
    """max|y - ref| / max|ref| (the fp32-accumulation tolerance metric, 1e-3)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(y - ref)) / max(np.max(np.abs(ref)), 1e-30))


def bf16_close(y_bits: np.ndarray, ref_bits: np.ndarray, rtol: float = 2e-2):
    """bf16 tolerance: |y - ref| <= rtol * (|ref| + rms(ref)) elementwise.
    Returns (ok, worst ratio, fraction bit-exact)."""
    from nerve_amd.workloads import bf16_bits_to_f32

    y = bf16_bits_to_f32(y_bits).astype(np.float64)
    r = bf16_bits_to_f32(ref_bits).astype(np.float64)
    floor = np.sqrt(np.mean(r * r)) if r.size else 0.0
    ratio = np.abs(y - r) / (rtol * (np.abs(r) + floor) + 1e-30)
    exact = float(np.mean(np.asarray(y_bits) == np.asarray(ref_bits))) if r.size else 1.0
    worst = float(np.max(ratio)) if r.size else 0.0
    return worst <= 1.0, worst, exact
