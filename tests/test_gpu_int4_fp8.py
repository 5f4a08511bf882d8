"""GPU parity: group-scaled INT4 linear (a9), FP8 output projection (a10) and
greedy argmax (a11), through the C ABI, against the CPU oracle."""
import numpy as np
import pytest

import oracle
from nerve_amd import workloads as wl

from bounds import fp8_head_dequant, gptq_dequant, linear_atol
from helpers import bf16_close, to_dev, to_np

pytestmark = pytest.mark.gpu


def _torch():
    import torch

    return torch


def _ct_from_gptq(d, K, N, group):
    """CT layout of the same codes: qweight [N, K/8], scales [N, K/G]."""
    q = d["q"]  # [K, N]
    qt = np.ascontiguousarray(q.T)
    qw = np.zeros((N, K // 8), np.uint32)
    for j in range(8):
        qw |= qt[:, j::8] << np.uint32(4 * j)
    return qw, np.ascontiguousarray(d["scales"].T)


def _run_int4(ctx, dev, spec, x, qw, scales, zeros, aux, B, N):
    torch = _torch()
    y = torch.zeros(B, N, dtype=torch.int16, device=dev)
    ctx.int4_linear(spec, to_dev(x, dev), to_dev(qw, dev), to_dev(scales.view(np.uint16), dev),
                    None if zeros is None else to_dev(zeros, dev), None if aux is None else to_dev(aux, dev), y, B)
    return to_np(y, np.uint16)


# (K, N) pairs cover both column-tile widths (16 columns when N % 64 != 0),
# groups that straddle load batches and grids of many XCD-remapped tiles.
@pytest.mark.parametrize("K,N", [(1024, 512), (512, 48), (256, 16384), (256, 32768)])
@pytest.mark.parametrize("M", [1, 4, 16, 20])
@pytest.mark.parametrize("symmetric", [True, False])
def test_int4_gptq_parity(ctx, dev, M, symmetric, K, N):
    G = 128
    rng = np.random.default_rng(M + 10 * symmetric + N)
    d = wl.int4_gptq(rng, K, N, G, symmetric)
    x = wl.bf16_normal(rng, (M, K))
    spec = f"linear_batch16_int4_gptq_sf16_g{G}_{K}x{N}.comp"
    y = _run_int4(ctx, dev, spec, x, d["qweight"], d["scales"], None if symmetric else d["qzeros"], None, M, N)
    ref = oracle.int4_linear("gptq", x, d["qweight"], d["scales"].view(np.uint16), G,
                             zeros=None if symmetric else d["qzeros"])
    ok, worst, exact = bf16_close(y, ref, atol=linear_atol(x, gptq_dequant(d)), name="int4 gptq")
    assert ok and exact > 0.9, (worst, exact)


# Group lengths with a compile-time kernel (32, 64, 128, 256) and one served
# by the generic kernel (96), at both column-tile widths.
# M = 2 takes the vector-ALU decode kernel where N % 64 == 0, M = 5 the MFMA one.
@pytest.mark.parametrize("G", [32, 64, 96, 256])
@pytest.mark.parametrize("N", [512, 48])
@pytest.mark.parametrize("M", [2, 3, 5])
def test_int4_gptq_group_lengths(ctx, dev, G, N, M):
    K = 768
    rng = np.random.default_rng(G * 7 + N + M)
    d = wl.int4_gptq(rng, K, N, G, False)
    x = wl.bf16_normal(rng, (M, K))
    spec = f"linear_batch16_int4_gptq_sf16_g{G}_{K}x{N}.comp"
    y = _run_int4(ctx, dev, spec, x, d["qweight"], d["scales"], d["qzeros"], None, M, N)
    ref = oracle.int4_linear("gptq", x, d["qweight"], d["scales"].view(np.uint16), G, zeros=d["qzeros"])
    ok, worst, exact = bf16_close(y, ref, atol=linear_atol(x, gptq_dequant(d)), name="int4 group lengths")
    assert ok and exact > 0.9, (worst, exact)


@pytest.mark.parametrize("M", [1, 4, 16])
def test_int4_config1_full_size(ctx, dev, M):
    d = wl.config1(M=M)
    K, N, G = d["K"], d["N"], d["group"]
    spec = f"linear_batch16_int4_gptq_sf16_g{G}_{K}x{N}.comp"
    y = _run_int4(ctx, dev, spec, d["x"], d["qweight"], d["scales"], d["qzeros"], None, M, N)
    ref = oracle.int4_linear("gptq", d["x"], d["qweight"], d["scales"].view(np.uint16), G, zeros=d["qzeros"])
    ok, worst, exact = bf16_close(y, ref, atol=linear_atol(d["x"], gptq_dequant(d)), name="int4 config1")
    assert ok and exact > 0.9, (worst, exact)


@pytest.mark.parametrize("finalize", [0, 1, 2])
@pytest.mark.parametrize("bf16_scales", [False, True])
def test_int4_ct_and_finalize(ctx, dev, finalize, bf16_scales):
    K, N, G, M = 512, 256, 128, 5
    rng = np.random.default_rng(finalize * 7 + bf16_scales)
    d = wl.int4_gptq(rng, K, N, G, True)
    x = wl.bf16_normal(rng, (M, K))
    qw, sc = _ct_from_gptq(d, K, N, G)
    if bf16_scales:
        sc = wl.f32_to_bf16_bits(sc.astype(np.float32))
    aux = None
    op = ["linear", "linear_bias", "linear_residual"][finalize]
    if finalize == 1:
        aux = wl.bf16_normal(rng, (N,))
    elif finalize == 2:
        aux = wl.bf16_normal(rng, (M, N))
    sdt = "bf16" if bf16_scales else "f16"
    spec = f"{op}_batch16_int4_ct_s{sdt}_g{G}_{K}x{N}.comp"
    sc_bits = sc.view(np.uint16)
    y = _run_int4(ctx, dev, spec, x, qw, sc_bits, None, aux, M, N)
    ref = oracle.int4_linear("ct", x, qw, sc_bits, G, scale_bf16=bf16_scales, finalize=finalize, aux=aux)
    atol = linear_atol(x, gptq_dequant(d), finalize)
    ok, worst, exact = bf16_close(y, ref, atol=atol, name="int4 ct finalize")
    assert ok and exact > 0.9, (worst, exact)
    # the same codes in the GPTQ layout give the same result
    gspec = f"{op}_batch16_int4_gptq_s{sdt}_g{G}_{K}x{N}.comp"
    g_sc = np.ascontiguousarray(sc_bits.T)
    y2 = _run_int4(ctx, dev, gspec, x, d["qweight"], g_sc, None, aux, M, N)
    ok, worst, _ = bf16_close(y2, ref, atol=atol)
    assert ok, worst


def _head(ctx, dev, d, spec, want_f32=True, want_bf16=True):
    torch = _torch()
    M, N = d["M"], d["N"]
    lf = torch.zeros(M, N, dtype=torch.float32, device=dev) if want_f32 else None
    lb = torch.zeros(M, N, dtype=torch.int16, device=dev) if want_bf16 else None
    am = torch.zeros(M, dtype=torch.int32, device=dev)
    ctx.fp8_output_projection(spec, to_dev(d["x"], dev), to_dev(d["W"], dev), to_dev(d["scale_inv"], dev), lf, lb,
                              am, M)
    return (None if lf is None else to_np(lf, np.float32), None if lb is None else to_np(lb, np.uint16),
            to_np(am, np.uint32))


def _argmax_ok(ids, ref_logits, tol):
    """Argmax parity: the same id, or (on a near-tie) one whose oracle logit is
    within `tol` of the oracle maximum."""
    for m, i in enumerate(ids):
        row = ref_logits[m]
        j = int(np.argmax(row))
        if int(i) != j and row[j] - row[int(i)] > tol:
            return False
    return True


# M <= 32 with per-row scales and K <= 3072 takes the stream kernel (1 or 2
# token tiles of 16, a partial last 16-row group at N % 16 != 0, fewer
# groups than blocks at small N); an odd N * nblk or K > 3072 falls back to
# the register form (M <= 16) or the GEMM; other M > 16 take the LDS-staged
# GEMM (token tiles of 64 / 128 / 256 rows;
# partial token and vocabulary tiles, N % 4 != 0, the 64-column K tail,
# K = 4096) or, with fewer K chunks than its ring has stages, the register
# form; K > 4096 takes the tiled fallback (fp8_head_kernel).  When the
# GEMM's items leave a part of a round, the rows past the last whole round
# take smaller tiles in a second launch.
@pytest.mark.parametrize("M,N,K", [(1, 1000, 256), (7, 4096, 2880), (64, 2048, 512), (130, 600, 384),
                                   (16, 2000, 4096), (2, 777, 64), (5, 1001, 384), (3, 30010, 2880),
                                   (20, 1000, 2880), (64, 4099, 640), (100, 777, 1024), (128, 3000, 2880),
                                   (300, 1300, 640), (257, 2051, 4096), (512, 5000, 2880),
                                   # stream form with 2 token tiles (partial last tile); M = 33: the GEMM
                                   (17, 2002, 384), (32, 3000, 2880), (33, 1500, 1024),
                                   # K > 4096: the tiled fallback kernel
                                   (5, 1000, 5120), (70, 1500, 5120),
                                   # 64-token tiles past one round of 256-row tiles per CU: the
                                   # rest in 64-row tiles (a partial last one; exactly one)
                                   (40, 66000, 384), (64, 65600, 256),
                                   # the same for 128-token tiles (tail in 128 x 64 tiles) and
                                   # 256-token tiles (tail in 128 x 128 tiles, 4 token tiles)
                                   (100, 33000, 384), (300, 16500, 640)])
def test_fp8_head_parity(ctx, dev, M, N, K):
    rng = np.random.default_rng(M * N + K)
    d = wl.fp8_head(rng, N, K, M)
    spec = f"tied_output_projection_batch4_fp8_e4m3_b1x128_{N}x{K}_scale1_to_f32.comp"
    lf, lb, am = _head(ctx, dev, d, spec)
    ref = oracle.fp8_output_projection(d["x"], d["W"], d["scale_inv"], 1, 1.0)
    err = np.max(np.abs(lf.astype(np.float64) - ref)) / np.max(np.abs(ref))
    assert err <= 1e-3, err
    ok, worst, _ = bf16_close(lb, wl.f32_to_bf16_bits(ref), atol=linear_atol(d["x"], fp8_head_dequant(d["W"], d["scale_inv"])),
                              name="fp8 head")
    assert ok, worst
    assert np.array_equal(lb, wl.f32_to_bf16_bits(lf))
    assert np.array_equal(am, oracle.argmax(lf))       # fused argmax == argmax of its own logits
    assert _argmax_ok(am, ref, 2e-3 * np.max(np.abs(ref)))


# M = 3: the register form; M = 50 / 200: the GEMM's general form (scales
# that vary along K, staged per tile), with one tile of uniform rows.
@pytest.mark.parametrize("M", [3, 50, 200])
def test_fp8_head_block_rows_and_output_scale(ctx, dev, M):
    N, K, BR = 1024, 640, 128
    rng = np.random.default_rng(5)
    d = wl.fp8_head(rng, N, K, M)
    nblk = K // 128
    grid = wl.bf16_normal(rng, ((N + BR - 1) // BR, nblk), 0.001)
    grid = wl.f32_to_bf16_bits(np.abs(wl.bf16_bits_to_f32(grid)) + np.float32(1e-4))
    grid[2, :] = grid[2, 0]          # rows 256..383 (one GEMM tile): one scale along K
    d["scale_inv"] = grid
    spec = f"tied_output_projection_batch4_fp8_e4m3_b{BR}x128_{N}x{K}_scale0.5_to_f32.comp"
    lf, _, am = _head(ctx, dev, d, spec, want_bf16=False)
    ref = oracle.fp8_output_projection(d["x"], d["W"], grid, BR, 0.5)
    assert np.max(np.abs(lf - ref)) / np.max(np.abs(ref)) <= 1e-3
    assert np.array_equal(am, oracle.argmax(lf))


def test_argmax_ties_lower_id(ctx, dev):
    torch = _torch()
    V = 201088
    rng = np.random.default_rng(3)
    lg = rng.standard_normal((4, V)).astype(np.float32)
    lg[0, [5, 77777, 200000]] = 50.0         # three-way tie -> 5
    lg[1, :] = -1.0                           # all equal -> 0
    lg[2, [V - 1, V - 2]] = 9.0               # tie at the end -> V-2
    lg[3, 123456] = np.float32(np.inf)
    out = torch.zeros(4, dtype=torch.int32, device=dev)
    ctx.argmax_f32(to_dev(lg, dev), 4, V, out)
    got = to_np(out, np.uint32)
    assert list(got) == [5, 0, V - 2, 123456]
    assert np.array_equal(got, oracle.argmax(lg))


@pytest.mark.parametrize("layout", ["gptq", "ct"])
def test_int4_finalize_rounding_closed_form(ctx, dev, layout):
    """The GPU finalize forms by closed form: bias rounds once (0x3F81),
    residual rounds the sum first and ties to even (0x3F80); see the CPU
    twin in test_oracle_paths.py for the derivation."""
    K, N, G, M = 128, 16, 128, 2
    x = np.zeros((M, K), np.uint16)
    x[:, 0], x[:, 1], x[:, 2] = 0x3F80, 0x3B00, 0x3A80
    if layout == "gptq":
        qw = np.full((K // 8, N), 0x99999999, np.uint32)
        sc = np.full((K // G, N), 0x3C00, np.uint16)
    else:
        qw = np.full((N, K // 8), 0x99999999, np.uint32)
        sc = np.full((N, K // G), 0x3C00, np.uint16)
    b = np.full((N,), 0x3B80, np.uint16)
    r = np.full((M, N), 0x3B80, np.uint16)
    for op, aux, want in (("linear", None, 0x3F80), ("linear_bias", b, 0x3F81), ("linear_residual", r, 0x3F80)):
        spec = f"{op}_batch16_int4_{layout}_sf16_g{G}_{K}x{N}.comp"
        y = _run_int4(ctx, dev, spec, x, qw, sc, None, aux, M, N)
        assert np.all(y == want), (op, y[0, :4])


# linear_batch_cooperative_int4.comp.template: batch-64 tiles; one and two
# tiles of tokens, both layouts, groups of 128 (and 32 for GPTQ).
@pytest.mark.parametrize("B", [64, 100])
@pytest.mark.parametrize("layout,G", [("gptq", 128), ("gptq", 32), ("ct", 128)])
@pytest.mark.parametrize("finalize", [0, 2])
def test_int4_cooperative_batch64(ctx, dev, B, layout, G, finalize):
    K, N = 1024, 384
    rng = np.random.default_rng(B + G + finalize + len(layout))
    d = wl.int4_gptq(rng, K, N, G, True)
    x = wl.bf16_normal(rng, (B, K))
    if layout == "gptq":
        qw, sc = d["qweight"], d["scales"]
    else:
        qw, sc = _ct_from_gptq(d, K, N, G)
    aux = wl.bf16_normal(rng, (B, N)) if finalize == 2 else None
    op = ["linear", "linear_bias", "linear_residual"][finalize]
    spec = f"{op}_batch64_cooperative_int4_{layout}_sf16_g{G}_{K}x{N}.comp"
    y = _run_int4(ctx, dev, spec, x, qw, sc.view(np.uint16), None, aux, B, N)
    ref = oracle.int4_linear(layout, x, qw, sc.view(np.uint16), G, finalize=finalize, aux=aux)
    ok, worst, exact = bf16_close(y, ref, atol=linear_atol(x, gptq_dequant(d), finalize), name="int4 cooperative")
    assert ok and exact > 0.9, (worst, exact)
