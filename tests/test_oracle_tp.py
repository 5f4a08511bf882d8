"""Pins the oracle's tensor-parallel down slice (o_moe_down_tp,
…down_batch1_mxfp4.comp.template:421-505) by the closed form and against the
whole down projection: the slices' f32 partials add up to the float64
dequantize-then-matmul sum, scaling their sum by the route weight gives the
whole projection's bf16 output within one place, and a token's routes after
its first out-of-range expert are left untouched."""
import numpy as np

import oracle
from nerve_amd import workloads as wl

import bounds


def _case(seed, B=3, k=2, E=3, H=64, I=256):
    rng = np.random.default_rng(seed)
    d = wl.moe_experts(rng, E, H, I)
    inter = wl.bf16_normal(rng, (B, k, I))
    ex = rng.integers(0, E, size=(B, k))
    wts = rng.uniform(0.1, 0.9, size=(B, k)).astype(np.float32)
    routes = ((wl.f32_to_bf16_bits(wts).astype(np.uint32) << np.uint32(16)) | ex.astype(np.uint32))
    return d, inter, routes


def test_down_tp_slices_sum_to_the_closed_form():
    d, inter, routes = _case(1)
    B, k, I = inter.shape
    E, H, _ = d["down_w"].shape
    total = np.zeros((B, k, H), np.float64)
    for start, count in [(0, 128), (128, 128)]:
        part = oracle.moe_down_tp(inter[:, :, start:start + count], routes, start, d["down_w"], d["down_s"])
        # closed form of the slice: pow2 block quantization of the slice,
        # float64 products with the dequantized slice columns
        q, s = oracle.quantize_blocks(inter[:, :, start:start + count].reshape(B * k, count), True)
        x = oracle.e4m3_to_f32(q).astype(np.float64) * np.repeat(s.astype(np.float64), 128, axis=1)
        for b in range(B):
            for r in range(k):
                e = int(routes[b, r] & 0xFFFF)
                w = bounds.mxfp4_dequant(d["down_w"][e], d["down_s"][e])[:, start:start + count]
                ref = w @ x[b * k + r]
                mag = np.abs(w) @ np.abs(x[b * k + r])
                assert np.all(np.abs(part[b, r].astype(np.float64) - ref) <= 1e-6 * mag + 1e-30)
        total += part
    # the slices' sum, scaled by the route weight, is the whole projection
    wr = bounds.bf16_f64((routes >> 16).astype(np.uint16))
    got = bounds.bf16_f64(wl.f32_to_bf16_bits((total * wr[:, :, None]).astype(np.float32)))
    whole = bounds.bf16_f64(oracle.moe_down(inter, routes, np.arange(B * k, dtype=np.uint32), B * k,
                                            d["down_w"], d["down_s"]))
    assert np.all(np.abs(got - whole) <= 2.0 ** -7 * np.abs(whole) + 1e-30)


def test_down_tp_first_invalid_route_ends_the_token():
    d, inter, routes = _case(2, B=2, k=3)
    routes[1, 1] = (routes[1, 1] & np.uint32(0xFFFF0000)) | np.uint32(7)   # expert 7 >= E = 3
    sentinel = np.full((2, 3, d["down_w"].shape[1]), 12.5, np.float32)
    part = oracle.moe_down_tp(inter[:, :, :128], routes, 0, d["down_w"], d["down_s"], out=sentinel)
    assert np.all(part[1, 1:] == 12.5)       # route 1 and every later route of token 1
    assert not np.any(part[1, 0] == 12.5) and not np.any(part[0] == 12.5)
