"""Tensor-parallel expert slices on one GPU (…gate_up_batch1_mxfp4.comp.
template:487-641, …down_batch1_mxfp4.comp.template:421-505): each rank's
share is its own call.  gate_up slices are checked against the oracle on the
rank's weight rows, down slices (f32 partials, not scaled by the route
weight) against oracle.moe_down_tp on the GPU's own local intermediates, and
the ranks' partials summed and scaled against the whole down projection.  A
token's routes after its first out-of-range expert keep their outputs, as in
the reference."""
import numpy as np
import pytest

import oracle
from nerve_amd import workloads as wl
from nerve_amd.hip import check_specialization
from nerve_amd.moe import address_record, down_spec, gate_up_spec, u32_tensor

from bounds import ACC_EPS, bf16_f64, moe_down_atol, moe_gate_up_atol, mxfp4_dequant
from helpers import bf16_close, to_dev, to_np

pytestmark = pytest.mark.gpu

SENTINEL = 0x7F7F


def _block_major(w, s):
    """Row-major down parameters [E, H, I/2], [E, H, I/32] -> input-block-major
    [E, I/128, H, 64], [E, I/128, H, 4] (…down_batch1_mxfp4.comp.template:
    229-233, :260-263)."""
    E, H, RB = w.shape
    wb = np.ascontiguousarray(w.reshape(E, H, RB // 64, 64).transpose(0, 2, 1, 3))
    sb = np.ascontiguousarray(s.reshape(E, H, RB // 64, 4).transpose(0, 2, 1, 3))
    return wb, sb


class Rank:
    """One rank's parameter slices and address tables: gate/up rows [i0, i1)
    and the down weights' 128-column blocks [i0 / 128, i1 / 128)."""

    def __init__(self, dev, d, i0, i1):
        self.i0, self.i1, self.L = i0, i1, i1 - i0
        E = d["gate_w"].shape[0]
        wb, sb = _block_major(d["down_w"], d["down_s"])
        b0, b1 = i0 // 128, i1 // 128
        self.t = {n: to_dev(np.ascontiguousarray(d[n][:, i0:i1]), dev) for n in ("gate_w", "gate_s", "up_w", "up_s")}
        self.t["down_w"] = to_dev(np.ascontiguousarray(wb[:, b0:b1]), dev)
        self.t["down_s"] = to_dev(np.ascontiguousarray(sb[:, b0:b1]), dev)
        recs, gslots, dslots = [], [], []
        for e in range(E):
            for n in ("gate_w", "gate_s", "up_w", "up_s"):
                gslots.append(len(recs) // 8)
                recs += address_record(self.t[n][e])
            for n in ("down_w", "down_s"):
                dslots.append(len(recs) // 8)
                recs += address_record(self.t[n][e])
        self.addresses = u32_tensor(recs, dev)
        self.gate_slots = u32_tensor(gslots, dev)
        self.down_slots = u32_tensor(dslots, dev)


def _routes(rng, B, k, E):
    ex = np.stack([rng.permutation(E)[:k] for _ in range(B)])
    wts = rng.uniform(0.1, 0.6, size=(B, k)).astype(np.float32)
    return ((wl.f32_to_bf16_bits(wts).astype(np.uint32) << np.uint32(16)) | ex.astype(np.uint32))


@pytest.mark.parametrize("E,k,B,H,I,ranks", [(8, 4, 5, 384, 512, 2), (32, 4, 16, 2880, 2816, 2), (6, 2, 3, 256, 384, 3)])
def test_tensor_parallel_slices(ctx, dev, E, k, B, H, I, ranks):
    import torch

    rng = np.random.default_rng(E + B + H)
    d = wl.moe_experts(rng, E, H, I)
    hidden = wl.bf16_normal(rng, (B, H))
    routes = _routes(rng, B, k, E)
    limit = 7.0
    gspec = gate_up_spec(H, I, E, k, limit, tensor_parallel=True)
    dspec = down_spec(H, I, E, k, tensor_parallel=True)
    assert check_specialization(gspec) == 0 and check_specialization(dspec) == 0
    cut = [I * r // ranks // 128 * 128 for r in range(ranks)] + [I]
    hd, rd = to_dev(hidden, dev), to_dev(routes, dev)
    dummy = to_dev(np.zeros(8, np.uint32), dev)
    cmap = np.arange(B * k, dtype=np.uint32)
    partial_sum = np.zeros((B, k, H), np.float32)
    h_all = []
    for r in range(ranks):
        rk = Rank(dev, d, cut[r], cut[r + 1])
        L = rk.L
        h = torch.full((B * k * L,), SENTINEL, dtype=torch.int16, device=dev)
        ctx.mxfp4_moe_gate_up(gspec, hd, None, rd, h, rk.addresses, rk.gate_slots, dummy, B)
        h_np = to_np(h, np.uint16).reshape(B, k, L)
        sl = {n: np.ascontiguousarray(d[n][:, rk.i0:rk.i1]) for n in ("gate_w", "gate_s", "up_w", "up_s")}
        h_ref = oracle.moe_gate_up(hidden, routes, cmap, B * k, k, sl["gate_w"], sl["gate_s"], sl["up_w"],
                                   sl["up_s"], limit)
        ok, worst, exact = bf16_close(h_np, h_ref, atol=moe_gate_up_atol(hidden, routes, sl["gate_w"], sl["gate_s"],
                                                                         sl["up_w"], sl["up_s"], limit),
                                      name=f"tp gate_up rank {r}")
        assert ok and exact > 0.9, (r, worst, exact)
        # the same slice from prequantized hidden rows: identical bytes
        q, s = oracle.quantize_blocks(hidden, True)
        h2 = torch.full((B * k * L,), SENTINEL, dtype=torch.int16, device=dev)
        ctx.mxfp4_moe_gate_up(gate_up_spec(H, I, E, k, limit, prequant=True, tensor_parallel=True), to_dev(q, dev),
                              to_dev(s, dev), rd, h2, rk.addresses, rk.gate_slots, dummy, B)
        assert np.array_equal(to_np(h2, np.uint16).reshape(B, k, L), h_np)
        # down: the GPU's own local intermediates, f32 partials
        y = torch.full((B * k * H,), 3.25, dtype=torch.float32, device=dev)
        rng_dev = to_dev(np.array([rk.i0, L], np.uint32), dev)
        ctx.mxfp4_moe_down(dspec, h, rd, y, rk.addresses, rk.down_slots, rng_dev, B)
        y_np = to_np(y, np.float32).reshape(B, k, H)
        y_ref = oracle.moe_down_tp(h_np, routes, rk.i0, d["down_w"], d["down_s"])
        # f32 sum order only: ACC_EPS times each output's accumulation magnitude
        qh, sh = oracle.quantize_blocks(h_np.reshape(B * k, L), True)
        xh = oracle.e4m3_to_f32(qh).astype(np.float64) * np.repeat(sh.astype(np.float64), 128, axis=1)
        mag = np.zeros((B, k, H))
        for b in range(B):
            for j in range(k):
                e = int(routes[b, j] & 0xFFFF)
                w = np.abs(mxfp4_dequant(d["down_w"][e], d["down_s"][e])[:, rk.i0:rk.i1])
                mag[b, j] = w @ np.abs(xh[b * k + j])
        err = np.abs(y_np.astype(np.float64) - y_ref.astype(np.float64))
        assert np.all(err <= ACC_EPS * mag + 1e-30), float(np.max(err / (ACC_EPS * mag + 1e-30)))
        partial_sum += y_np
        h_all.append(h_np)
    # the ranks' partials, summed and scaled by the route weight, are the
    # whole down projection of the concatenated intermediates
    h_full = np.concatenate(h_all, axis=2)
    wr = bf16_f64((routes >> 16).astype(np.uint16))
    got = wl.f32_to_bf16_bits((partial_sum.astype(np.float64) * wr[:, :, None]).astype(np.float32))
    whole = oracle.moe_down(h_full, routes, cmap, B * k, d["down_w"], d["down_s"])
    ok, worst, exact = bf16_close(got, whole, atol=2 * moe_down_atol(h_full, routes, d["down_w"], d["down_s"]),
                                  name="tp down, ranks summed")
    assert ok and exact > 0.9, (worst, exact)


def test_tensor_parallel_first_invalid_route_ends_the_token(ctx, dev):
    import torch

    E, k, B, H, I = 4, 3, 2, 256, 256
    rng = np.random.default_rng(11)
    d = wl.moe_experts(rng, E, H, I)
    hidden = wl.bf16_normal(rng, (B, H))
    routes = _routes(rng, B, k, E)
    routes[1, 1] = (routes[1, 1] & np.uint32(0xFFFF0000)) | np.uint32(E)      # out of range
    rk = Rank(dev, d, 0, I)
    rd = to_dev(routes, dev)
    dummy = to_dev(np.zeros(8, np.uint32), dev)
    h = torch.full((B * k * I,), SENTINEL, dtype=torch.int16, device=dev)
    ctx.mxfp4_moe_gate_up(gate_up_spec(H, I, E, k, 7.0, tensor_parallel=True), to_dev(hidden, dev), None, rd, h,
                          rk.addresses, rk.gate_slots, dummy, B)
    h_np = to_np(h, np.uint16).reshape(B, k, I)
    assert np.all(h_np[1, 1:] == SENTINEL)                       # route 1 and every later route of token 1
    assert not np.all(h_np[1, 0] == SENTINEL) and not np.all(h_np[0] == SENTINEL)
    y = torch.full((B * k * H,), 3.25, dtype=torch.float32, device=dev)
    ctx.mxfp4_moe_down(down_spec(H, I, E, k, tensor_parallel=True), h, rd, y, rk.addresses, rk.down_slots,
                       to_dev(np.array([0, I], np.uint32), dev), B)
    y_np = to_np(y, np.float32).reshape(B, k, H)
    assert np.all(y_np[1, 1:] == 3.25)
    y_ref = oracle.moe_down_tp(h_np, routes, 0, d["down_w"], d["down_s"], out=np.full((B, k, H), 3.25, np.float32))
    assert np.all(y_ref[1, 1:] == 3.25)
    assert np.allclose(y_np, y_ref, rtol=1e-3, atol=1e-3 * np.max(np.abs(y_ref)))


def test_tensor_parallel_down_refuses_the_count_stage(ctx, dev):
    import torch

    E, k, B, H, I = 2, 1, 1, 128, 128
    t = torch.zeros(64, dtype=torch.int32, device=dev)
    with pytest.raises(Exception):
        ctx.mxfp4_moe_down_counted(down_spec(H, I, E, k, tensor_parallel=True), t, t, t, t, t, t, B)
