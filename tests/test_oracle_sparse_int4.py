"""CPU checks of the sparse INT4-CT expert oracle
(sparse_moe_gate_up_int4_ct.comp.template:97-227,
sparse_moe_down_int4_ct.comp.template:106-193) against what the mathematics
fixes: one-hot activations pick (code - 8) * scale of one code exactly
(nibble order, gate/up row split, scale group index), a float64 dense
dequantize-then-matmul with the shaders' rounding points agrees within f32
summation error, and the route selection (map, owned expert range, unbound
experts, out-of-range ids) skips exactly the routes it should."""
import numpy as np
import pytest

import oracle
from nerve_amd import workloads as wl


def _route_words(experts, weights):
    return (wl.f32_to_bf16_bits(np.asarray(weights, np.float32)).astype(np.uint32) << np.uint32(16)) | \
        np.asarray(experts, np.uint32)


def _dense(W, S, group, scale_bf16):
    """float64 [E, rows, K] of (code - 8) * scale, unpacked independently."""
    E, R, KW = W.shape
    codes = np.stack([(W >> np.uint32(4 * j)) & np.uint32(15) for j in range(8)], axis=-1).reshape(E, R, KW * 8)
    sc = wl.bf16_bits_to_f32(S) if scale_bf16 else S.view(np.float16).astype(np.float32)
    return (codes.astype(np.float64) - 8.0) * np.repeat(sc.astype(np.float64), group, axis=2)


def _bf(v):
    return wl.bf16_bits_to_f32(wl.f32_to_bf16_bits(np.asarray(v, np.float32))).astype(np.float64)


@pytest.mark.parametrize("scale_bf16", [True, False])
@pytest.mark.parametrize("group", [16, 32, 64])
def test_one_hot_picks_one_code(scale_bf16, group):
    """x = e_j (value 1): g = (code_g[i, j] - 8) * s_g[i, j / G] exactly."""
    rng = np.random.default_rng(3)
    E, H, I = 2, 128, 32
    d = wl.int4_ct_experts(rng, E, 2 * I, H, group, scale_bf16, keep_codes=True)
    dense = _dense(d["W"], d["S"], group, scale_bf16)
    for j in (0, 1, 7, 8, 37, H - 1):
        x = np.zeros((1, H), np.float32)
        x[0, j] = 1.0
        routes = _route_words([[1]], [[1.0]])
        h = oracle.sparse_int4_gate_up(wl.f32_to_bf16_bits(x), routes, None, 1, d["W"], d["S"], group,
                                       scale_bf16=scale_bf16)
        code = d["q"][1, :, j].astype(np.float64) - 8.0
        assert np.array_equal(dense[1, :, j], code * np.repeat(
            (wl.bf16_bits_to_f32(d["S"]) if scale_bf16 else d["S"].view(np.float16).astype(np.float32))[1],
            group, axis=1)[:, j])
        g = _bf(dense[1, :I, j])
        u = _bf(dense[1, I:, j])
        ref = _bf(_bf(g / (1.0 + np.exp(-g))) * u)
        got = wl.bf16_bits_to_f32(h[0, 0]).astype(np.float64)
        assert np.array_equal(got, ref), j


def test_gate_up_and_down_match_float64_dense():
    rng = np.random.default_rng(4)
    E, H, I, k, B, G = 6, 256, 96, 3, 2, 32
    gu = wl.int4_ct_experts(rng, E, 2 * I, H, G, True)
    dn = wl.int4_ct_experts(rng, E, H, I, G, False)
    x = wl.bf16_normal(rng, (B, H))
    experts = np.array([[0, 3, 5], [3, 1, 0]])
    weights = rng.uniform(0.1, 1.0, size=(B, k))
    routes = _route_words(experts, weights)
    h = oracle.sparse_int4_gate_up(x, routes, None, B * k, gu["W"], gu["S"], G)
    y = oracle.sparse_int4_down(h, routes, None, B * k, dn["W"], dn["S"], G, scale_bf16=False)
    dg = _dense(gu["W"], gu["S"], G, True)
    dd = _dense(dn["W"], dn["S"], G, False)
    xf = wl.bf16_bits_to_f32(x).astype(np.float64)
    for b in range(B):
        for r in range(k):
            e = experts[b, r]
            gl = dg[e, :I] @ xf[b]
            ul = dg[e, I:] @ xf[b]
            g, u = _bf(gl), _bf(ul)
            href = _bf(g / (1.0 + np.exp(-g))) * u
            got = wl.bf16_bits_to_f32(h[b, r]).astype(np.float64)
            scale = np.abs(href) + np.sqrt(np.mean(href ** 2))
            assert np.max(np.abs(got - href) / scale) < 2e-2
            # down on the oracle's own h (so only down's arithmetic is judged)
            yl = dd[e] @ wl.bf16_bits_to_f32(h[b, r]).astype(np.float64)
            wr = wl.bf16_bits_to_f32(wl.f32_to_bf16_bits(np.float32(weights[b, r]))).astype(np.float64)
            yref = _bf(yl) * wr
            goty = wl.bf16_bits_to_f32(y[b, r]).astype(np.float64)
            sc = np.abs(yref) + np.sqrt(np.mean(yref ** 2))
            assert np.max(np.abs(goty - yref) / sc) < 2e-2


def test_down_closed_form_route_weight():
    """All codes 9 (value 1), scales 1: y = sum(h) exactly for small integer h;
    out = bf16(bf16(y) * w)."""
    E, H, I, G = 2, 64, 64, 32
    W = np.full((E, H, I // 8), 0x99999999, np.uint32)
    S = np.full((E, H, I // G), 0x3F80, np.uint16)
    h = np.zeros((1, 2, I), np.float32)
    h[0, 0] = np.arange(I) % 5
    h[0, 1] = 2.0
    routes = _route_words([[1, 0]], [[0.75, 3.0]])
    y = oracle.sparse_int4_down(wl.f32_to_bf16_bits(h), routes, None, 2, W, S, G)
    got = wl.bf16_bits_to_f32(y)
    assert np.all(got[0, 0] == _bf(_bf(np.sum(np.arange(I) % 5)) * 0.75))
    assert np.all(got[0, 1] == _bf(2.0 * I * 3.0))


def test_route_selection():
    """Map order, owned range, unbound experts and out-of-range ids."""
    rng = np.random.default_rng(5)
    E, H, I, k, B, G = 4, 64, 32, 2, 3, 32
    d = wl.int4_ct_experts(rng, E, 2 * I, H, G)
    x = wl.bf16_normal(rng, (B, H))
    experts = np.array([[0, 1], [2, 3], [1, 7]])          # 7 >= E: skipped
    routes = _route_words(experts, np.ones((B, k)))
    sentinel = np.full((B, k, I), 0x7FC1, np.uint16)
    full = oracle.sparse_int4_gate_up(x, routes, None, B * k, d["W"], d["S"], G, inter=sentinel)
    assert np.all(full[2, 1] == 0x7FC1)
    assert not np.any(full[:2] == 0x7FC1)
    # each route alone equals its slice of the full run
    for c in range(B * k - 1):
        one = oracle.sparse_int4_gate_up(x, routes, np.array([c], np.uint32), 1, d["W"], d["S"], G,
                                         inter=sentinel)
        b, r = divmod(c, k)
        assert np.array_equal(one[b, r], full[b, r])
        mask = np.ones((B, k), bool)
        mask[b, r] = False
        assert np.all(one[mask] == 0x7FC1)
    # owned range [1, 3): routes of experts 1 and 2 only
    own = oracle.sparse_int4_gate_up(x, routes, None, B * k, d["W"], d["S"], G, expert_start=1, expert_count=2,
                                     inter=sentinel)
    for b in range(B):
        for r in range(k):
            e = experts[b, r]
            if 1 <= e < 3:
                assert np.array_equal(own[b, r], full[b, r])
            else:
                assert np.all(own[b, r] == 0x7FC1)
    # unbound expert 3
    ub = oracle.sparse_int4_gate_up(x, routes, None, B * k, d["W"], d["S"], G, bound=[1, 1, 1, 0],
                                    inter=sentinel)
    assert np.all(ub[1, 1] == 0x7FC1) and np.array_equal(ub[1, 0], full[1, 0])
