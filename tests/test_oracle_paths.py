"""Pins the oracle's hot-path functions (a3-a11) against the reference's known
answers, closed forms, brute force and invariants -- independently of the
oracle's own code paths."""
import math

import numpy as np
import pytest

import oracle
from nerve_amd import workloads as wl


def f(bits):
    return wl.bf16_bits_to_f32(bits)


# --------------------------------------------------------------------------
# a3 / a4 MXFP4 projections
# --------------------------------------------------------------------------

def _const_bank(E, H, I, nib, scale):
    return dict(gate_w=np.full((E, I, H // 2), nib, np.uint8), gate_s=np.full((E, I, H // 32), scale, np.uint8),
                up_w=np.full((E, I, H // 2), nib, np.uint8), up_s=np.full((E, I, H // 32), scale, np.uint8),
                down_w=np.full((E, H, I // 2), nib, np.uint8), down_s=np.full((E, H, I // 32), scale, np.uint8))


def _one_route(weight=1.0, expert=0):
    return np.array([[(int(wl.f32_to_bf16_bits(np.float32(weight))) << 16) | expert]], np.uint32)


def test_gate_up_known_answer_mxfp4_tests_rs():
    # runtime-rs/src/vulkan_compute/mxfp4_tests.rs:67-216
    d = _const_bank(1, 128, 128, 0x22, 120)
    routes = _one_route()
    h = oracle.moe_gate_up(np.full((1, 128), 0x3F80, np.uint16), routes, np.array([0], np.uint32), 1, 1,
                           d["gate_w"], d["gate_s"], d["up_w"], d["up_s"], 10.0)
    assert np.all(h == 0x3F3B)


def test_down_known_answers_every_code_and_route_weight():
    values = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, 0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]
    inter = np.full((1, 1, 128), 0x3F80, np.uint16)
    for nib, v in enumerate(values):
        d = _const_bank(1, 128, 128, nib | (nib << 4), 120)
        out = oracle.moe_down(inter, _one_route(), np.array([0], np.uint32), 1, d["down_w"], d["down_s"])
        assert np.all(out == wl.f32_to_bf16_bits(np.float32(v))), nib
    # the route weight is applied once, after the linear map (mxfp4_tests.rs:11-36)
    d = _const_bank(1, 128, 128, 0x77, 120)  # 6.0
    out = oracle.moe_down(inter, _one_route(0.375), np.array([0], np.uint32), 1, d["down_w"], d["down_s"])
    assert np.all(f(out) == np.float32(6.0 * 0.375))


def test_swiglu_clamp_closed_form():
    # hidden 1.0, weights 1.0 * 2^-3 over 128 columns -> g = u = 16 > limit 7:
    # gate = min(16, 7), up = clamp(16, -7, 7); h = bf16(7 / (1 + e^-7) * 7).
    d = _const_bank(1, 128, 128, 0x22, 124)
    h = oracle.moe_gate_up(np.full((1, 128), 0x3F80, np.uint16), _one_route(), np.array([0], np.uint32), 1, 1,
                           d["gate_w"], d["gate_s"], d["up_w"], d["up_s"], 7.0)
    g = np.float32(7.0)
    expect = wl.f32_to_bf16_bits((g / (np.float32(1.0) + np.exp(-g))) * np.float32(7.0))
    assert np.all(h == expect)
    # negative up side clamps to -limit; no limit (0) passes through
    d["up_w"][:] = 0xAA  # -1.0
    h = oracle.moe_gate_up(np.full((1, 128), 0x3F80, np.uint16), _one_route(), np.array([0], np.uint32), 1, 1,
                           d["gate_w"], d["gate_s"], d["up_w"], d["up_s"], 7.0)
    assert np.all(h == wl.f32_to_bf16_bits((g / (np.float32(1.0) + np.exp(-g))) * np.float32(-7.0)))


def test_gemv_one_hot_pins_nibble_and_scale_indexing():
    # A single nonzero activation at column c picks exactly W[n, c] * S[n, c/32].
    rng = np.random.default_rng(0)
    K, N = 256, 16
    W, S = wl.mxfp4_matrix(rng, N, K, 110, 140)
    for c in (0, 1, 31, 32, 63, 130, 255):
        x = np.zeros((1, K), np.uint16)
        x[0, c] = 0x3F80  # 1.0 -> e4m3 256 * 2^-8
        q, s = oracle.quantize_blocks(x, True)
        y = oracle.mxfp4_gemv(q, s, W, S)[0]
        for n in range(N):
            nib = (W[n, c // 2] >> 4) if c & 1 else (W[n, c // 2] & 15)
            assert y[n] == np.float32(oracle.mxfp4_value(int(nib), int(S[n, c // 32]))), (c, n)


def test_gemv_against_float64_ideal():
    rng = np.random.default_rng(1)
    for M, K, N in ((1, 2880, 64), (3, 160, 32), (5, 4096, 16)):
        W, S = wl.mxfp4_matrix(rng, N, K)
        x = wl.bf16_normal(rng, (M, K))
        q, s = oracle.quantize_blocks(x, True)
        y = oracle.mxfp4_gemv(q, s, W, S)
        ideal = oracle.mxfp4_gemv_f64(q, s, W, S)
        assert np.max(np.abs(y - ideal)) / np.max(np.abs(ideal)) < 1e-5
        # quantization error budget against the unquantized bf16 input
        xf = f(x).astype(np.float64)
        wf = np.array([[oracle.mxfp4_value(int((W[n, k // 2] >> (4 * (k & 1))) & 15), int(S[n, k // 32]))
                        for k in range(K)] for n in range(N)])
        exact = xf @ wf.T
        assert np.max(np.abs(ideal - exact)) / np.max(np.abs(exact)) < 0.1


def test_moe_chain_matches_per_route_gemv():
    # gate_up on a routed token == the GEMV of that token against the expert's
    # gate and up rows followed by the SwiGLU epilogue.
    rng = np.random.default_rng(2)
    E, k, B, H, I = 4, 2, 3, 160, 96
    d = wl.moe_experts(rng, E, H, I)
    logits = wl.bf16_normal(rng, (B, E))
    routes, _ = oracle.topk(logits, k, telemetry=False)
    hidden = wl.bf16_normal(rng, (B, H))
    cmap, _ = oracle.route_compact(routes, k, 3, B)
    h = oracle.moe_gate_up(hidden, routes, cmap, B * k, k, d["gate_w"], d["gate_s"], d["up_w"], d["up_s"], 7.0)
    q, s = oracle.quantize_blocks(hidden, True)
    for b in range(B):
        for r in range(k):
            e = int(routes[b, r] & 0xFFFF)
            g = oracle.mxfp4_gemv(q[b:b + 1], s[b:b + 1], d["gate_w"][e], d["gate_s"][e])[0]
            u = oracle.mxfp4_gemv(q[b:b + 1], s[b:b + 1], d["up_w"][e], d["up_s"][e])[0]
            gb = np.minimum(f(wl.f32_to_bf16_bits(g)), np.float32(7))
            ub = np.clip(f(wl.f32_to_bf16_bits(u)), np.float32(-7), np.float32(7))
            ref = wl.f32_to_bf16_bits((gb / (np.float32(1) + np.exp(-gb))) * ub)
            diff = np.abs(f(h[b, r]).astype(np.float64) - f(ref))
            assert np.max(diff) <= 2.0 ** -6 * (np.max(np.abs(f(ref))) + 1e-3)


# --------------------------------------------------------------------------
# a5 router, a6 top-k, a7 compaction, a8 combine
# --------------------------------------------------------------------------

def test_router_linear_float64():
    rng = np.random.default_rng(3)
    x = wl.bf16_normal(rng, (5, 2880))
    w = wl.bf16_normal(rng, (32, 2880), 0.02)
    got = f(oracle.router_linear(x, w)).astype(np.float64)
    ideal = f(x).astype(np.float64) @ f(w).astype(np.float64).T
    assert np.all(np.abs(got - ideal) <= np.abs(ideal) * 2.0 ** -8 + 1e-6)


def _brute_topk(row, k, bias=None, sigmoid=False, normalize=True):
    """Spec restated independently: stable arg-max by (-score, index), ascending
    sort, softmax over the selected logits (float64)."""
    lg = f(row).astype(np.float64)
    sc = 1 / (1 + np.exp(-lg)) if sigmoid else lg.copy()
    if bias is not None:
        sc = sc + bias
    order = sorted(range(len(row)), key=lambda e: (-sc[e], e))[:k]
    sel = sorted(order)
    if sigmoid:
        w = 1 / (1 + np.exp(-lg[sel]))
        if normalize:
            w = w / w.sum()
    else:
        top = lg[order[0]]
        w = np.exp(lg[sel] - top)
        w = w / (w.sum() if normalize else np.exp(lg - lg.max()).sum() * np.exp(lg.max() - top))
    return sel, w


@pytest.mark.parametrize("sigmoid,normalize", [(False, True), (True, True), (False, False), (True, False)])
def test_topk_brute_force(sigmoid, normalize):
    rng = np.random.default_rng(4)
    B, E, k = 40, 32, 4
    logits = wl.bf16_normal(rng, (B, E), 1.5)
    logits[0, [2, 9, 30, 31]] = wl.f32_to_bf16_bits(np.float32(5.0))   # four-way tie
    logits[1, :] = wl.f32_to_bf16_bits(np.float32(1.0))                 # all tied
    bias = rng.standard_normal(E).astype(np.float32) * np.float32(0.05)
    routes, tel = oracle.topk(logits, k, activation=int(sigmoid), normalize=int(normalize), bias=bias)
    counts = np.zeros(E, np.int64)
    pairs = {}
    for b in range(B):
        sel, w = _brute_topk(logits[b], k, bias.astype(np.float64), sigmoid, normalize)
        idx = routes[b] & 0xFFFF
        assert list(idx) == sel, b
        assert np.allclose(f((routes[b] >> 16).astype(np.uint16)), w, rtol=1e-2, atol=1e-7)
        for e in sel:
            counts[e] += 1
        for i in range(k):
            for j in range(i + 1, k):
                pairs[(sel[i], sel[j])] = pairs.get((sel[i], sel[j]), 0) + 1
    assert np.array_equal(tel[:E], counts)
    pair_tel = tel[E:]
    for (l, r), c in pairs.items():
        assert pair_tel[l * (2 * E - l - 1) // 2 + r - l - 1] == c
    assert pair_tel.sum() == sum(pairs.values())


def test_score_router_brute_force_softmax():
    rng = np.random.default_rng(5)
    B, E, k, A = 6, 20, 3, 2
    logits = wl.bf16_normal(rng, (B, E))
    bias = np.zeros(E, np.float32)
    routes, _ = oracle.topk(logits, k, mode=1, activation=1, normalize=1, routed_scale=2.0, always_count=A,
                            always_weight=0.25, bias=bias)
    for b in range(B):
        lg = f(logits[b]).astype(np.float64)
        p = np.exp(lg - lg.max()) / np.exp(lg - lg.max()).sum()
        sel = sorted(sorted(range(E), key=lambda e: (-p[e], e))[:k])
        w = p[sel] / p[sel].sum() * 2.0
        idx = list(routes[b] & 0xFFFF)
        assert idx == sel + [E, E + 1]
        wts = f((routes[b] >> 16).astype(np.uint16))
        assert np.allclose(wts[:k], w, rtol=1e-2) and np.all(wts[k:] == 0.25)


def test_route_compact_closed_forms():
    rng = np.random.default_rng(6)
    B, k, E = 37, 4, 16
    routes, _ = oracle.topk(wl.bf16_normal(rng, (B, E)), k, telemetry=False)
    m, ctl = oracle.route_compact(routes, k, 90, B)
    assert np.array_equal(m, np.argsort(routes.reshape(-1) & 0xFFFF, kind="stable"))
    assert list(ctl) == [B, 0, 0, B * k, k * 90, B, 1]
    m, ctl = oracle.route_compact(routes, k, 45, B, 4, 5)
    ex = routes.reshape(-1) & 0xFFFF
    owned = np.nonzero((ex >= 4) & (ex < 9))[0]
    assert ctl[3] == len(owned) and np.array_equal(m[:len(owned)], owned)
    assert list(ctl[4:]) == [len(owned) * 45, 1, 1]


def test_reduce_properties():
    rng = np.random.default_rng(7)
    # small integers: bf16 sums are exact
    ints = rng.integers(-20, 20, size=(3, 4, 64)).astype(np.float32)
    out = oracle.moe_reduce(wl.f32_to_bf16_bits(ints), 1.0)
    assert np.array_equal(f(out), ints.sum(axis=1))
    # k = 1 is bf16(x * scale)
    x = wl.bf16_normal(rng, (2, 1, 50))
    assert np.array_equal(oracle.moe_reduce(x, 0.5), wl.f32_to_bf16_bits(f(x)[:, 0] * np.float32(0.5)))
    # sequential bf16 rounding: within k/2 bf16 ulps of the exact sum
    v = wl.bf16_normal(rng, (8, 6, 100))
    got = f(oracle.moe_reduce(v, 1.0)).astype(np.float64)
    exact = f(v).astype(np.float64).sum(axis=1)
    scale = np.abs(f(v)).astype(np.float64).sum(axis=1)
    assert np.all(np.abs(got - exact) <= scale * 2.0 ** -8 * 6)


# --------------------------------------------------------------------------
# a9 INT4
# --------------------------------------------------------------------------

def test_int4_closed_form_asymmetric():
    rng = np.random.default_rng(8)
    K, N, G, B = 256, 64, 128, 3
    d = wl.int4_gptq(rng, K, N, G, symmetric=False)
    x = wl.bf16_normal(rng, (B, K))
    y = f(oracle.int4_linear("gptq", x, d["qweight"], d["scales"].view(np.uint16), G, zeros=d["qzeros"]))
    wdq = (d["q"].astype(np.float64) - np.repeat(d["zeros"], G, axis=0)) * np.repeat(d["scales"].astype(np.float64), G, axis=0)
    ideal = f(x).astype(np.float64) @ wdq
    assert np.all(np.abs(y - ideal) <= np.abs(ideal) * 2.0 ** -7 + 1e-3 * np.max(np.abs(ideal)))


def _int4_producer(values, group):
    """Reference INT4 producer restated (nerve/representation_optimizer/
    providers/group_scaled_int4/toolchain.py:400-418): s = bf16(amax/7),
    q = clip(rint(x/s), -7, 7) + 8, 8 codes per u32 along K, row-major
    [N, K/8] (the CT layout)."""
    N, K = values.shape
    blocks = values.reshape(N, K // group, group)
    amax = np.max(np.abs(blocks), axis=2)
    sc = np.where(amax > 0, amax / 7.0, 1.0).astype(np.float32)
    s_bits = wl.f32_to_bf16_bits(sc)
    s = f(s_bits)
    q = (np.clip(np.rint(blocks / s[:, :, None]), -7, 7).astype(np.int16) + 8).astype(np.uint32).reshape(N, K)
    qw = np.zeros((N, K // 8), np.uint32)
    for j in range(8):
        qw |= q[:, j::8] << np.uint32(4 * j)
    return qw, s_bits


def test_int4_reference_producer_round_trip_ct():
    rng = np.random.default_rng(9)
    N, K, G, B = 32, 512, 128, 2
    wf = f(wl.bf16_normal(rng, (N, K), 0.05))
    qw, s_bits = _int4_producer(wf, G)
    x = wl.bf16_normal(rng, (B, K))
    y = f(oracle.int4_linear("ct", x, qw, s_bits, G, scale_bf16=True)).astype(np.float64)
    # decode the producer's codes independently: code j of word p is k = 8p + j
    codes = np.stack([(qw >> np.uint32(4 * j)) & 15 for j in range(8)], axis=2).reshape(N, K).astype(np.float64)
    sc = np.repeat(f(s_bits).astype(np.float64), G, axis=1)
    wdq = (codes - 8) * sc
    assert np.all(np.abs(wdq - wf) <= sc / 2 + 1e-9)          # round-to-nearest within half a step
    ideal = f(x).astype(np.float64) @ wdq.T
    assert np.max(np.abs(y - ideal)) <= 2.0 ** -7 * np.max(np.abs(ideal))
    # GPTQ layout of the same codes agrees
    codes = np.stack([(qw >> np.uint32(4 * j)) & 15 for j in range(8)], axis=2).reshape(N, K).T  # [K, N]
    gq = np.zeros((K // 8, N), np.uint32)
    for j in range(8):
        gq |= codes[j::8, :] << np.uint32(4 * j)
    y2 = f(oracle.int4_linear("gptq", x, gq, np.ascontiguousarray(s_bits.T), G, scale_bf16=True))
    assert np.max(np.abs(y2 - y)) <= 2.0 ** -7 * np.max(np.abs(y))


# --------------------------------------------------------------------------
# a10 / a11 FP8 head and argmax
# --------------------------------------------------------------------------

def test_fp8_producer_matches_reference_rules():
    # nerve/model_package_tensors.py:1044-1075: RNE, saturation, subnormal clip to 7
    v = np.array([0.0, 1.0, 448.0, 500.0, -1e9, 2.0 ** -9, 2.0 ** -6, 0.0155, 1.0625, 1.1875], np.float32)
    got = wl.f32_to_e4m3fn_producer(v)
    assert list(got) == [0x00, 0x38, 0x7E, 0x7E, 0xFE, 0x01, 0x08, 0x07, 0x38, 0x3A]


def test_fp8_head_float64_and_one_hot():
    rng = np.random.default_rng(10)
    d = wl.fp8_head(rng, 64, 384, 3)
    out = oracle.fp8_output_projection(d["x"], d["W"], d["scale_inv"], 1, 1.0)
    q, s = oracle.quantize_blocks(d["x"], False)
    qf = oracle.e4m3_to_f32(q).astype(np.float64) * np.repeat(s, 128, axis=1)[:, :384]
    wf = oracle.e4m3_to_f32(d["W"]).astype(np.float64) * d["scale_f32"][:, None]
    ideal = qf @ wf.T
    assert np.max(np.abs(out - ideal)) / np.max(np.abs(ideal)) < 1e-5
    # one-hot input: logit = e4m3(448) * s_x * W[n, c] * s_w[n]
    x = np.zeros((1, 384), np.uint16)
    x[0, 200] = 0x4000  # 2.0
    out = oracle.fp8_output_projection(x, d["W"], d["scale_inv"], 1, 1.0)[0]
    sx = np.float32(2.0) / np.float32(448.0)
    expect = np.float32(448.0) * oracle.e4m3_to_f32(d["W"][:, 200]) * (sx * d["scale_f32"])
    assert np.allclose(out, expect, rtol=1e-6, atol=0)


def test_argmax_tie_rule():
    lg = np.array([[1, 3, 3, 2], [-np.inf, -np.inf, -np.inf, -np.inf], [0, 0, 5, 5]], np.float32)
    assert list(oracle.argmax(lg)) == [1, 0, 2]


def test_int4_finalize_rounding_closed_form():
    """The INT4 finalize forms by closed form
    (nerve/model_package_shader_selection.py:2504-2525): bias adds to the f32
    sum and rounds once, y = bf16(b + S); residual rounds the sum first,
    y = bf16(r + bf16(S)).  With every code 9 (weight 1), scale 1 and
    x = (1, 2^-9, 2^-10, 0, ...) the sum is exactly S = 1 + 2^-9 + 2^-10, so
    bf16(S) = 1; with b = r = 2^-8 the single rounding gives 1 + 2^-7
    (0x3F81) and the double rounding ties to even at 1.0 (0x3F80)."""
    K, N, G = 128, 16, 128
    x = np.zeros((1, K), np.uint16)
    x[0, 0] = 0x3F80                       # 1.0
    x[0, 1] = 0x3B00                       # 2^-9
    x[0, 2] = 0x3A80                       # 2^-10
    qw = np.full((K // 8, N), 0x99999999, np.uint32)
    sc = np.full((K // G, N), 0x3C00, np.uint16)          # f16 1.0
    b = np.full((N,), 0x3B80, np.uint16)                  # 2^-8
    y0 = oracle.int4_linear("gptq", x, qw, sc, G)
    assert np.all(y0 == 0x3F80)                            # bf16(S) = 1.0
    y1 = oracle.int4_linear("gptq", x, qw, sc, G, finalize=1, aux=b)
    assert np.all(y1 == 0x3F81)
    y2 = oracle.int4_linear("gptq", x, qw, sc, G, finalize=2, aux=np.tile(b, (1, 1)))
    assert np.all(y2 == 0x3F80)
    # the CT layout of the same codes gives the same bits
    qct = np.full((N, K // 8), 0x99999999, np.uint32)
    sct = np.full((N, K // G), 0x3C00, np.uint16)
    assert np.array_equal(oracle.int4_linear("ct", x, qct, sct, G, finalize=1, aux=b), y1)
    assert np.array_equal(oracle.int4_linear("ct", x, qct, sct, G, finalize=2, aux=np.tile(b, (1, 1))), y2)
