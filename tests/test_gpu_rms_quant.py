"""GPU parity: RMSNorm + blockwise e4m3 prequantization
(rms_norm_quantize_fp8_e4m3.comp.template:70-129) through the C ABI, against
the CPU oracle.  y may differ from the oracle's in the last bf16 place (the
sum of squares is added in another order); q and the scales are checked
bit-exactly as the quantization of the GPU's own y, and against the oracle
wherever the y block agrees."""
import numpy as np
import pytest

import oracle
from nerve_amd import workloads as wl

from helpers import to_dev, to_np

pytestmark = pytest.mark.gpu


def _spec(H, block, pow2, rows, eps, offset):
    batch = f"_batch{rows}" if rows > 1 else ""
    return (f"rms_norm_quantize{batch}_fp8_e4m3{'_spow2' if pow2 else ''}_b{block}_h{H}"
            f"_eps{eps}_offset{offset}.comp")


@pytest.mark.parametrize("H,block,rows", [(2880, 32, 1), (2880, 64, 4), (4096, 128, 16), (512, 512, 3), (96, 32, 2)])
@pytest.mark.parametrize("pow2", [False, True])
@pytest.mark.parametrize("in_place", [False, True])
def test_rms_norm_quantize(ctx, dev, H, block, rows, pow2, in_place):
    import torch

    rng = np.random.default_rng(H + block + rows + 2 * pow2 + in_place)
    x = wl.bf16_normal(rng, (rows, H))
    w = wl.bf16_normal(rng, (H,), 0.4)
    eps, offset = 1e-05, 1.0
    xd = to_dev(x, dev)
    yd = xd if in_place else torch.zeros(rows, H, dtype=torch.int16, device=dev)
    qd = torch.zeros(rows, H, dtype=torch.uint8, device=dev)
    sd = torch.zeros(rows, H // block, dtype=torch.float32, device=dev)
    ctx.rms_norm_quantize_fp8_e4m3(_spec(H, block, pow2, rows, eps, offset), xd, to_dev(w, dev), yd, qd, sd, rows)
    y, q, s = to_np(yd, np.uint16), to_np(qd, np.uint8), to_np(sd, np.float32)
    yr, qr, sr = oracle.rms_norm_quantize(x, w, block, pow2, eps, offset)
    # y: within one bf16 place of the oracle, almost always equal
    d = np.abs(y.astype(np.int32) - yr.astype(np.int32))
    assert d.max() <= 1 and np.mean(d == 0) > 0.99
    # q, s: the quantization of the GPU's own y (blockwise, bit-exact)
    for r in range(rows):
        for b in range(H // block):
            cols = slice(b * block, (b + 1) * block)
            yb = wl.bf16_bits_to_f32(y[r, cols])
            amax = np.float32(np.max(np.abs(yb)))
            sc = oracle.pow2_fp8_scale(amax) if pow2 else oracle.amax_fp8_scale(amax)
            assert s[r, b] == np.float32(sc)
            assert np.array_equal(q[r, cols], oracle.f32_to_e4m3(yb / np.float32(sc)))
            if np.array_equal(y[r, cols], yr[r, cols]):
                assert s[r, b] == sr[r, b] and np.array_equal(q[r, cols], qr[r, cols])


@pytest.mark.parametrize("H,rows", [(2880, 1), (4096, 16), (96, 3)])
@pytest.mark.parametrize("in_place", [False, True])
def test_rms_norm_quantize_int8_pairpacked(ctx, dev, H, rows, in_place):
    """The int8 form (rms_norm_quantize_int8_pairpacked.comp.template:60-151):
    y as for the fp8 form, then the pair-packed INT8 quantization of the
    GPU's own y, bit-exact."""
    import torch

    rng = np.random.default_rng(H + rows + in_place)
    x = wl.bf16_normal(rng, (rows, H))
    w = wl.bf16_normal(rng, (H,), 0.4)
    xd = to_dev(x, dev)
    yd = xd if in_place else torch.zeros(rows, H, dtype=torch.int16, device=dev)
    qd = torch.zeros(rows, H, dtype=torch.uint8, device=dev)
    sd = torch.zeros(rows, H // 32, dtype=torch.float32, device=dev)
    md = torch.zeros(rows, H // 32, dtype=torch.int32, device=dev)
    batch = f"_batch{rows}" if rows > 1 else ""
    spec = f"rms_norm_quantize{batch}_int8_pairpacked_b32_h{H}_eps1e-06_offset0.comp"
    ctx.rms_norm_quantize_int8_pairpacked(spec, xd, to_dev(w, dev), yd, qd, sd, md, rows)
    y = to_np(yd, np.uint16)
    yr, _, _ = oracle.rms_norm_quantize(x, w, 32, False, 1e-06, 0.0)
    d = np.abs(y.astype(np.int32) - yr.astype(np.int32))
    assert d.max() <= 1 and np.mean(d == 0) > 0.99
    qr, sr, sumr = oracle.quantize_i8_pairpacked(y)
    assert np.array_equal(to_np(qd, np.uint8), qr)
    assert np.array_equal(to_np(sd, np.float32), sr)
    assert np.array_equal(to_np(md, np.int32), sumr)
