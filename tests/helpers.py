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


def bf16_close(y_bits: np.ndarray, ref_bits: np.ndarray, rtol: float = 2e-2, atol=0.0, name: str | None = None):
    """bf16 tolerance, elementwise: |y - ref| <= rtol |ref| + atol, with atol
    a scalar or an array of per-element floors (tests/bounds.py derives them
    from each output's own accumulation magnitude).  Returns (ok, worst
    ratio, fraction bit-exact).  With NERVE_BOUNDS_REPORT set, prints, under
    `name`, the accumulation error the check had to absorb (the part of
    |y - ref| above rtol |ref|, per unit of atol / ACC_EPS)."""
    import os

    from nerve_amd.workloads import bf16_bits_to_f32

    y = bf16_bits_to_f32(y_bits).astype(np.float64)
    r = bf16_bits_to_f32(ref_bits).astype(np.float64)
    a = np.broadcast_to(np.asarray(atol, np.float64), r.shape)
    ratio = np.abs(y - r) / (rtol * np.abs(r) + a + 1e-30)
    exact = float(np.mean(np.asarray(y_bits) == np.asarray(ref_bits))) if r.size else 1.0
    worst = float(np.max(ratio)) if r.size else 0.0
    if os.environ.get("NERVE_BOUNDS_REPORT") and r.size:
        from bounds import ACC_EPS

        excess = np.maximum(np.abs(y - r) - rtol * np.abs(r), 0.0)
        mag = a / ACC_EPS
        need = float(np.max(np.where(mag > 0, excess / np.maximum(mag, 1e-300), np.where(excess > 0, np.inf, 0.0))))
        print(f"[bounds] {name or '?'}: worst ratio {worst:.3g}, accumulation error needed {need:.3g} "
              f"(ACC_EPS {ACC_EPS:.3g}), bit-exact {exact:.4f}", flush=True)
    return worst <= 1.0, worst, exact
