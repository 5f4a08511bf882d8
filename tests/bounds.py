"""Per-element error bounds for the bf16 parity checks.

A GPU output and the oracle's differ by the order of their fp32 sums (MFMA
blocks against the shaders' fma chains) and, where the algorithm rounds an
intermediate to bf16, by a one-place flip of that rounding.  The sum-order
difference of an output is bounded by ACC_EPS times its accumulation
magnitude sum_k |a_k| |w_k| (the dequantized operands of that output); the
flips are carried to the output by first-order propagation.  bf16_close then
allows |y - ref| <= 2e-2 |ref| + atol elementwise with atol from here: an
output near zero gets only the floor its own accumulation justifies, not a
fraction of the whole tensor's size.
"""
from __future__ import annotations

import numpy as np

# fp32 sum-order bound per unit of accumulation magnitude.  With
# NERVE_BOUNDS_REPORT=1 the GPU tests print, per check, the error above
# rtol |ref| per unit of magnitude: at most 1.6e-5 for every single-sum
# family (down projections, INT4, FP8 head) and 4.8e-4 for the gate_up
# checks, whose bound also carries the bf16 flips of g and u; the worst
# ratio |y - ref| / (rtol |ref| + atol) over the whole suite is 0.83.
ACC_EPS = 2.0 ** -12

_E2M1 = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6, -0.0, -0.5, -1, -1.5, -2, -3, -4, -6], np.float64)


def bf16_f64(bits) -> np.ndarray:
    b = np.asarray(bits).astype(np.uint32) << np.uint32(16)
    return b.view(np.float32).astype(np.float64)


def bf16_ulp(v) -> np.ndarray:
    """Spacing of bf16 values at |v| (one place of the 8-bit significand)."""
    a = np.maximum(np.abs(np.asarray(v, np.float64)), 2.0 ** -126)
    return 2.0 ** (np.floor(np.log2(a)) - 7)


def mxfp4_dequant(w_packed, s_bytes) -> np.ndarray:
    """[R, K/2] e2m1 bytes (low nibble first) with [R, K/32] e8m0 scales -> f64 [R, K]."""
    w = np.asarray(w_packed, np.uint8)
    R, K2 = w.shape
    v = np.empty((R, 2 * K2), np.float64)
    v[:, 0::2] = _E2M1[w & 0xF]
    v[:, 1::2] = _E2M1[w >> 4]
    sc = 2.0 ** (np.asarray(s_bytes, np.float64) - 127.0)
    return v * np.repeat(sc, 32, axis=1)


def _route_experts(routes):
    r = np.asarray(routes, np.uint32)
    return (r & 0xFFFF).astype(np.int64), bf16_f64((r >> 16).astype(np.uint16))


def _swiglu_atol(x, wg, wu, limit, act_rounded):
    """Bound on h = silu(g) u for g = x wg^T, u = x wu^T (f64 operands):
    |silu'(g) u| dg + |silu(g)| du (+ |u| ulp(silu(g)) when the activation
    is rounded to bf16 before the product), dg = ACC_EPS G + ulp(g)."""
    g, u = x @ wg.T, x @ wu.T
    G, U = np.abs(x) @ np.abs(wg).T, np.abs(x) @ np.abs(wu).T
    dg = ACC_EPS * G + bf16_ulp(g)
    du = ACC_EPS * U + bf16_ulp(u)
    if limit > 0:
        dg = np.where(g > limit, 0.0, dg)                 # clamped: no sensitivity
        du = np.where(np.abs(u) > limit, 0.0, du)
        g = np.minimum(g, limit)
        u = np.clip(u, -limit, limit)
    sg = 1.0 / (1.0 + np.exp(-g))
    silu, dsilu = g * sg, sg * (1.0 + g * (1.0 - sg))
    out = np.abs(dsilu * u) * dg + np.abs(silu) * du
    if act_rounded:
        out += np.abs(u) * bf16_ulp(silu)
    return out


def _per_expert(routes, valid, E, fn, width):
    e, wr = _route_experts(routes)
    B, k = e.shape
    out = np.zeros((B, k, width), np.float64)
    for ex in np.unique(e):
        if ex >= E:
            continue
        sel = (e == ex) if valid is None else ((e == ex) & valid)
        bb, jj = np.nonzero(sel)
        if len(bb):
            out[bb, jj] = fn(int(ex), bb, jj, wr[bb, jj])
    return out


def moe_gate_up_atol(hidden, routes, gw, gs, uw, us, limit, valid=None):
    """atol [B, k, I] of the MXFP4 gate_up h = bf16(silu(g) u), g and u the
    bf16-rounded, clamped sums over the pow2-scaled e4m3 activation blocks
    both sides contract.  valid [B, k] (optional) selects routes."""
    import oracle

    q, sc = oracle.quantize_blocks(np.asarray(hidden, np.uint16), True)
    x = oracle.e4m3_to_f32(q).astype(np.float64) * np.repeat(sc.astype(np.float64), 128, axis=1)[:, : q.shape[1]]
    E, I, _ = gw.shape
    return _per_expert(routes, valid, E, lambda ex, bb, jj, wr: _swiglu_atol(
        x[bb], mxfp4_dequant(gw[ex], gs[ex]), mxfp4_dequant(uw[ex], us[ex]), limit, False), I)


def moe_down_atol(inter_bits, routes, dw, ds, valid=None):
    """atol [B, k, H] of the MXFP4 down projection x route weight: ACC_EPS
    times w_route sum |h| |w_down| (the GPU's own h is the input of both
    sides; the bf16 roundings of y and y w_route are covered by rtol)."""
    h = bf16_f64(inter_bits)
    E, H, _ = dw.shape
    return _per_expert(routes, valid, E, lambda ex, bb, jj, wr: ACC_EPS * np.abs(wr)[:, None] * (
        np.abs(h[bb, jj]) @ np.abs(mxfp4_dequant(dw[ex], ds[ex])).T), H)


def int4_ct_dequant(W, S, group, scale_bf16) -> np.ndarray:
    """Sparse INT4-CT rows: W u32 [R, K/8] (nibble j of word c is column
    8c + j, value code - 8), S u16 [R, K/group] -> f64 [R, K]."""
    W = np.asarray(W, np.uint32)
    R, K8 = W.shape
    codes = np.empty((R, 8 * K8), np.float64)
    for j in range(8):
        codes[:, j::8] = ((W >> np.uint32(4 * j)) & np.uint32(15)).astype(np.float64) - 8.0
    S = np.asarray(S, np.uint16)
    sc = bf16_f64(S) if scale_bf16 else S.view(np.float16).astype(np.float64)
    return codes * np.repeat(sc, group, axis=1)


def int4_moe_gate_up_atol(hidden, routes, W, S, group, scale_bf16):
    """atol [B, k, I] of the sparse INT4-CT gate_up
    h = bf16(bf16(silu(bf16 g)) bf16 u) (W [E, 2I, H/8] gate rows then up rows)."""
    x = bf16_f64(hidden)
    E, I2, _ = W.shape
    I = I2 // 2

    def one(ex, bb, jj, wr):
        w = int4_ct_dequant(W[ex], S[ex], group, scale_bf16)
        return _swiglu_atol(x[bb], w[:I], w[I:], 0.0, True)

    return _per_expert(routes, None, E, one, I)


def int4_moe_down_atol(inter_bits, routes, W, S, group, scale_bf16):
    """atol [B, k, H] of the sparse INT4-CT down bf16(bf16(y) w_route)."""
    h = bf16_f64(inter_bits)
    E, H, _ = W.shape
    return _per_expert(routes, None, E, lambda ex, bb, jj, wr: ACC_EPS * np.abs(wr)[:, None] * (
        np.abs(h[bb, jj]) @ np.abs(int4_ct_dequant(W[ex], S[ex], group, scale_bf16)).T), H)


def linear_atol(x, w_kn, finalize=0):
    """atol [M, N] of y = x W for x [M, K] (bf16 bits or f64) and W [K, N]
    f64: ACC_EPS |x| |W|, plus, for the residual form residual + bf16(x W),
    a one-place flip of that rounding."""
    xf = bf16_f64(x) if np.asarray(x).dtype == np.uint16 else np.asarray(x, np.float64)
    a = ACC_EPS * (np.abs(xf) @ np.abs(w_kn))
    if finalize == 2:
        a = a + bf16_ulp(xf @ w_kn)
    return a


def gptq_dequant(d) -> np.ndarray:
    """workloads.int4_gptq's codes -> f64 [K, N] ((code - zero) x scale)."""
    q = np.asarray(d["q"], np.float64)
    group = q.shape[0] // d["scales"].shape[0]
    s = np.repeat(np.asarray(d["scales"], np.float64), group, axis=0)
    z = np.repeat(np.asarray(d["zeros"], np.float64), group, axis=0)
    return (q - z) * s


def fp8_head_dequant(W, scale_inv, block_rows=1) -> np.ndarray:
    """e4m3 W [N, K] with bf16 scale_inv [ceil(N/BR), ceil(K/128)] -> f64 [K, N]."""
    import oracle

    w = oracle.e4m3_to_f32(np.asarray(W, np.uint8)).astype(np.float64)
    N, K = w.shape
    sc = bf16_f64(scale_inv)
    sc = np.repeat(np.repeat(sc, block_rows, axis=0)[:N], 128, axis=1)[:, :K]
    return (w * sc).T
