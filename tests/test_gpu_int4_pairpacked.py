"""GPU parity: pair-packed INT8 activations and the INT8 x GPTQ INT4 linear
(quantize_int8_symmetric_pairpacked.comp.template:22-72,
linear_prequant_pairpacked_int4_gptq.comp.template:56-128) through the C ABI,
against the CPU oracle: the quantizer bit-exact, the linear within bf16
tolerance (only the f32 accumulation order differs)."""
import numpy as np
import pytest

import oracle
from nerve_amd import workloads as wl

from bounds import gptq_dequant, linear_atol
from helpers import bf16_close, to_dev, to_np

pytestmark = pytest.mark.gpu


def _quant(ctx, dev, x):
    import torch

    B, K = x.shape
    q = torch.zeros(B, K, dtype=torch.uint8, device=dev)
    s = torch.zeros(B, K // 32, dtype=torch.float32, device=dev)
    sums = torch.zeros(B, K // 32, dtype=torch.int32, device=dev)
    spec = f"quantize{'_batch%d' % B if B > 1 else ''}_int8_symmetric_pairpacked_b32_h{K}.comp"
    ctx.quantize_int8_pairpacked(spec, to_dev(x, dev), q, s, sums, B)
    return q, s, sums


@pytest.mark.parametrize("B,K", [(1, 4096), (5, 2880), (16, 96)])
def test_quantize_int8_pairpacked_bit_exact(ctx, dev, B, K):
    rng = np.random.default_rng(B + K)
    x = wl.bf16_normal(rng, (B, K))
    x[0, 32:64] = 0
    q, s, sums = _quant(ctx, dev, x)
    qr, sr, sumr = oracle.quantize_i8_pairpacked(x)
    assert np.array_equal(to_np(q, np.uint8), qr)
    assert np.array_equal(to_np(s, np.float32), sr)
    assert np.array_equal(to_np(sums, np.int32), sumr)


@pytest.mark.parametrize("M,K,N,G", [(1, 4096, 14336, 128), (4, 1024, 512, 32), (16, 512, 96, 256)])
@pytest.mark.parametrize("finalize", [0, 1, 2])
@pytest.mark.parametrize("bf16_scales", [False, True])
def test_int4_linear_pairpacked(ctx, dev, M, K, N, G, finalize, bf16_scales):
    import torch

    rng = np.random.default_rng(M + K + N + finalize + bf16_scales)
    d = wl.int4_gptq(rng, K, N, G, True)
    sc = d["scales"].view(np.uint16)
    if bf16_scales:
        sc = wl.f32_to_bf16_bits(d["scales"].astype(np.float32))
    x = wl.bf16_normal(rng, (M, K))
    aux = wl.bf16_normal(rng, (M, N)) if finalize == 2 else wl.bf16_normal(rng, (N,)) if finalize == 1 else None
    q, s, sums = _quant(ctx, dev, x)
    y = torch.zeros(M, N, dtype=torch.int16, device=dev)
    op = ["linear", "linear_bias", "linear_residual"][finalize]
    spec = (f"{op}_prequant_pairpacked{'_batch%d' % M if M > 1 else ''}_int4_gptq_s{'bf16' if bf16_scales else 'f16'}"
            f"_g{G}_{K}x{N}.comp")
    ctx.int4_linear_pairpacked(spec, q, s, sums, to_dev(d["qweight"], dev), to_dev(sc, dev),
                               None if aux is None else to_dev(aux, dev), y, M)
    qr, sr, sumr = oracle.quantize_i8_pairpacked(x)
    ref = oracle.int4_linear_pairpacked(qr, sr, sumr, d["qweight"], sc, G, scale_bf16=bf16_scales,
                                        finalize=finalize, aux=aux)
    ok, worst, exact = bf16_close(to_np(y, np.uint16), ref, atol=linear_atol(x, gptq_dequant(d), finalize),
                                  name="pairpacked")
    assert ok and exact > 0.9, (worst, exact)


@pytest.mark.parametrize("B,N", [(1, 14336), (4, 2880), (16, 96)])
def test_silu_multiply_quantize_int8_pairpacked(ctx, dev, B, N):
    import torch

    rng = np.random.default_rng(B * 7 + N)
    g = wl.bf16_normal(rng, (B, N), 2.0)
    u = wl.bf16_normal(rng, (B, N))
    y = torch.zeros(B, N, dtype=torch.int16, device=dev)
    q = torch.zeros(B, N, dtype=torch.uint8, device=dev)
    s = torch.zeros(B, N // 32, dtype=torch.float32, device=dev)
    sums = torch.zeros(B, N // 32, dtype=torch.int32, device=dev)
    spec = f"silu_multiply_quantize{'_batch%d' % B if B > 1 else ''}_int8_pairpacked_b32_h{N}.comp"
    ctx.silu_multiply_quantize_int8_pairpacked(spec, to_dev(g, dev), to_dev(u, dev), y, q, s, sums, B)
    yg = to_np(y, np.uint16)
    yr = oracle.silu_multiply_bf16(g, u)
    d = np.abs(yg.astype(np.int32) - yr.astype(np.int32))
    assert d.max() <= 1 and np.mean(d == 0) > 0.99      # exp may differ in its last place
    qr, sr, sumr = oracle.quantize_i8_pairpacked(yg)
    assert np.array_equal(to_np(q, np.uint8), qr)
    assert np.array_equal(to_np(s, np.float32), sr)
    assert np.array_equal(to_np(sums, np.int32), sumr)


def test_silu_multiply_quantize_rejects_aliased_output(ctx, dev):
    """y written over gate or up is refused on the host (the kernel reads its
    inputs through restrict pointers)."""
    import torch

    from nerve_amd.hip import NerveHipError

    B, N = 2, 256
    rng = np.random.default_rng(11)
    gd = to_dev(wl.bf16_normal(rng, (B, N)), dev)
    ud = to_dev(wl.bf16_normal(rng, (B, N)), dev)
    q = torch.zeros(B, N, dtype=torch.uint8, device=dev)
    s = torch.zeros(B, N // 32, dtype=torch.float32, device=dev)
    sums = torch.zeros(B, N // 32, dtype=torch.int32, device=dev)
    spec = f"silu_multiply_quantize_batch{B}_int8_pairpacked_b32_h{N}.comp"
    for y in (gd, ud, gd[1:]):
        with pytest.raises(NerveHipError):
            ctx.silu_multiply_quantize_int8_pairpacked(spec, gd, ud, y, q, s, sums, B)


# --------------------------------------------------------------------------
# Unpaired INT8 input: quantize_int8_symmetric + linear_prequant_int4_{gptq,ct}
# --------------------------------------------------------------------------

def _quant_unpaired(ctx, dev, x):
    import torch

    B, K = x.shape
    q = torch.zeros(B, K, dtype=torch.uint8, device=dev)
    s = torch.zeros(B, K // 32, dtype=torch.float32, device=dev)
    spec = f"quantize{'_batch%d' % B if B > 1 else ''}_int8_symmetric_b32_h{K}.comp"
    ctx.quantize_int8_pairpacked(spec, to_dev(x, dev), q, s, None, B)
    return q, s


@pytest.mark.parametrize("B,K", [(1, 4096), (5, 2880), (16, 96)])
def test_quantize_int8_unpaired_bit_exact(ctx, dev, B, K):
    rng = np.random.default_rng(B + 3 * K)
    x = wl.bf16_normal(rng, (B, K))
    x[0, :32] = 0
    q, s = _quant_unpaired(ctx, dev, x)
    qr, sr = oracle.quantize_i8(x)
    assert np.array_equal(to_np(q, np.uint8), qr)
    assert np.array_equal(to_np(s, np.float32), sr)


def _ct_layout(d, K, N):
    qt = np.ascontiguousarray(d["q"].T)
    qw = np.zeros((N, K // 8), np.uint32)
    for j in range(8):
        qw |= qt[:, j::8] << np.uint32(4 * j)
    return qw, np.ascontiguousarray(d["scales"].T)


# config 1's shape (K = 4096, N = 14336) and small shapes with groups of 32 /
# 64 / 256, both layouts, every finalize form, f16 and bf16 scales.
@pytest.mark.parametrize("M,K,N,G", [(1, 4096, 14336, 128), (4, 1024, 512, 32), (16, 512, 96, 256), (3, 768, 64, 64)])
@pytest.mark.parametrize("layout", ["gptq", "ct"])
@pytest.mark.parametrize("finalize", [0, 1, 2])
def test_int4_linear_prequant_unpaired(ctx, dev, M, K, N, G, layout, finalize):
    import torch

    rng = np.random.default_rng(M + K + N + G + finalize + len(layout))
    d = wl.int4_gptq(rng, K, N, G, True)
    bf16_scales = (finalize + G) % 2 == 1
    if layout == "gptq":
        qw, sc = d["qweight"], d["scales"]
    else:
        qw, sc = _ct_layout(d, K, N)
    sc_bits = wl.f32_to_bf16_bits(sc.astype(np.float32)) if bf16_scales else sc.view(np.uint16)
    x = wl.bf16_normal(rng, (M, K))
    aux = wl.bf16_normal(rng, (M, N)) if finalize == 2 else wl.bf16_normal(rng, (N,)) if finalize == 1 else None
    q, s = _quant_unpaired(ctx, dev, x)
    y = torch.zeros(M, N, dtype=torch.int16, device=dev)
    op = ["linear", "linear_bias", "linear_residual"][finalize]
    spec = (f"{op}_prequant{'_batch%d' % M if M > 1 else ''}_int4_{layout}_s{'bf16' if bf16_scales else 'f16'}"
            f"_g{G}_{K}x{N}.comp")
    ctx.int4_linear_pairpacked(spec, q, s, None, to_dev(qw, dev), to_dev(sc_bits, dev),
                               None if aux is None else to_dev(aux, dev), y, M)
    qr, sr = oracle.quantize_i8(x)
    ref = oracle.int4_linear_prequant(layout, qr, sr, qw, sc_bits, G, scale_bf16=bf16_scales, finalize=finalize,
                                      aux=aux)
    ok, worst, exact = bf16_close(to_np(y, np.uint16), ref, atol=linear_atol(x, gptq_dequant(d), finalize),
                                  name="prequant unpaired")
    assert ok and exact > 0.9, (worst, exact)
