"""GPU parity: sparse INT4-CT expert gate/up + SwiGLU and down + route
weight (sparse_moe_{gate_up,down}_int4_ct.comp.template) through the C ABI,
against the CPU oracle: the real geometry of the reference's compiler test
(h3072 i1024 e256 k10, g32 bf16 scales), the batched (route map) and
unbatched forms, every lane split of the kernel, group sizes below 32, owned
expert ranges and the slots that skip a route."""
import numpy as np
import pytest

import oracle
from nerve_amd import workloads as wl
from nerve_amd.hip import NerveHipError
from nerve_amd.moe import Int4CtExpertBank, address_record, gate_up_spec, int4_ct_spec, u32_tensor

from bounds import int4_moe_down_atol, int4_moe_gate_up_atol
from helpers import bf16_close, to_dev, to_np

pytestmark = pytest.mark.gpu

SENTINEL = 0x7FC1


def _torch():
    import torch

    return torch


def _route_words(experts, weights):
    return (wl.f32_to_bf16_bits(np.asarray(weights, np.float32)).astype(np.uint32) << np.uint32(16)) | \
        np.asarray(experts, np.uint32)


class Rig:
    """Device buffers of one gate_up -> down run over an INT4-CT expert bank
    of nb stored experts shared by E model experts (expert e -> bank e % nb)."""

    def __init__(self, dev, H, I, E, k, G, scale_bf16, nb, seed):
        torch = _torch()
        rng = np.random.default_rng(seed)
        self.H, self.I, self.E, self.k, self.G, self.sbf = H, I, E, k, G, scale_bf16
        self.gu = wl.int4_ct_experts(rng, nb, 2 * I, H, G, scale_bf16)
        self.dn = wl.int4_ct_experts(rng, nb, H, I, G, scale_bf16)
        self.nb = nb
        self.bank = Int4CtExpertBank(to_dev(self.gu["W"], dev), to_dev(self.gu["S"], dev), to_dev(self.dn["W"], dev),
                                     to_dev(self.dn["S"], dev), experts=E, bank_of=[e % nb for e in range(E)])
        self.rng = rng
        self.dev = dev
        self.torch = torch

    def oracle_routes(self, routes):
        """Route words with expert ids replaced by their bank ids (ids >= E keep
        an out-of-range id)."""
        e = routes & 0xFFFF
        mapped = np.where(e < self.E, e % self.nb, 0xFFFF)
        return (routes & np.uint32(0xFFFF0000)) | mapped.astype(np.uint32)


def _frames_to_h(frames, B, k, I):
    return frames.reshape(B, -1)[:, : k * I // 2].copy().view(np.uint16).reshape(B, k, I)


def _run_batched(ctx, rig, x, routes, B, start=0, count=0):
    torch = rig.torch
    dev = rig.dev
    k, I, H = rig.k, rig.I, rig.H
    gspec = int4_ct_spec("gate_up", H, I, rig.E, k, rig.G, scale_bf16=rig.sbf)
    dspec = int4_ct_spec("down", H, I, rig.E, k, rig.G, scale_bf16=rig.sbf)
    fw = k * I // 2 + k
    frames = np.zeros((B, fw), np.uint32)
    frames[:, : k * I // 2] = (SENTINEL << 16) | SENTINEL
    inter = to_dev(frames, dev)
    control = to_dev(np.array([B, start, count, 0, 0, 0, 0, 0], np.uint32), dev)
    r_dev = to_dev(routes, dev)
    ctx.moe_route_compact(gspec, r_dev, inter, control, B)
    ctl = to_np(control, np.uint32)[:7].copy()
    ctx.int4_moe_gate_up(gspec, to_dev(x, dev), r_dev, inter, rig.bank.addresses, rig.bank.gate_slots, control, B)
    out = torch.full((B, k, H), SENTINEL, dtype=torch.int16, device=dev)
    ctx.moe_route_compact(dspec, r_dev, None, control, B)
    ctl_down = to_np(control, np.uint32)[:7].copy()
    ctx.int4_moe_down(dspec, inter, r_dev, out, rig.bank.addresses, rig.bank.down_slots, control, B)
    fr = to_np(inter, np.uint32)
    return _frames_to_h(fr, B, k, I), to_np(out, np.uint16).reshape(B, k, H), ctl, ctl_down


def _check(rig, x, routes, h, y, start=0, count=0):
    B, k = routes.shape
    oroutes = rig.oracle_routes(routes)
    # ownership is decided on the model expert ids, so select the routes here
    e = routes & 0xFFFF
    sel = (e < rig.E) & ((count == 0) | ((e >= start) & (e < start + count)))
    cmap = np.flatnonzero(sel.reshape(-1)).astype(np.uint32)
    sent = np.full((B, k, rig.I), SENTINEL, np.uint16)
    href = oracle.sparse_int4_gate_up(x, oroutes, cmap, len(cmap), rig.gu["W"], rig.gu["S"], rig.G,
                                      scale_bf16=rig.sbf, inter=sent)
    atol = int4_moe_gate_up_atol(x, oroutes, rig.gu["W"], rig.gu["S"], rig.G, rig.sbf)
    ok, worst, exact = bf16_close(h[sel], href[sel], atol=atol[sel], name="int4-ct gate_up")
    assert ok and exact > 0.9, ("gate_up", worst, exact)
    assert np.all(h[~sel] == SENTINEL)
    # down on the GPU's own h so that only down's arithmetic is compared
    ysent = np.full((B, k, rig.H), SENTINEL, np.uint16)
    yref = oracle.sparse_int4_down(h, oroutes, cmap, len(cmap), rig.dn["W"], rig.dn["S"], rig.G,
                                   scale_bf16=rig.sbf, out=ysent)
    atol = int4_moe_down_atol(h, oroutes, rig.dn["W"], rig.dn["S"], rig.G, rig.sbf)
    ok, worst, exact = bf16_close(y[sel], yref[sel], atol=atol[sel], name="int4-ct down")
    assert ok and exact > 0.9, ("down", worst, exact)
    assert np.all(y[~sel] == SENTINEL)


def test_real_geometry_h3072_i1024_e256_k10(ctx, dev):
    """The geometry of the reference's compiler test (tests/test_model_package_
    moe_components.py:979-1108): 640 gate_up and 1920 down workgroups, i.e.
    16-row tiles; batched decode of 4 tokens."""
    rig = Rig(dev, 3072, 1024, 256, 10, 32, True, nb=12, seed=11)
    B = 4
    logits = wl.bf16_normal(rig.rng, (B, 256))
    routes, _ = oracle.topk(logits, 10, telemetry=False)
    routes = routes.astype(np.uint32)
    x = wl.bf16_normal(rig.rng, (B, 3072))
    h, y, ctl, ctl_down = _run_batched(ctx, rig, x, routes, B)
    assert ctl[4] == 10 * 64 and ctl_down[4] == 10 * 192
    _check(rig, x, routes, h, y)


@pytest.mark.parametrize("H,I,G,sbf,B", [
    (2048, 512, 128, False, 3),     # gate_up 64 lanes per row, down 16
    (2880, 2880, 32, True, 2),      # 90 chunks per row: 32 lanes per row
    (256, 96, 16, False, 5),        # groups below 32 (one scale per word)
    (1024, 1024, 64, True, 16),     # a full decode batch; repeated experts
    (4096, 256, 8, True, 1),
])
def test_batched_shapes(ctx, dev, H, I, G, sbf, B):
    E, k = 16, 4
    rig = Rig(dev, H, I, E, k, G, sbf, nb=E, seed=H + I + G)
    logits = wl.bf16_normal(rig.rng, (B, E))
    routes, _ = oracle.topk(logits, k, telemetry=False)
    routes = routes.astype(np.uint32)
    x = wl.bf16_normal(rig.rng, (B, H))
    h, y, _, _ = _run_batched(ctx, rig, x, routes, B)
    _check(rig, x, routes, h, y)


@pytest.mark.parametrize("start,count", [(4, 6), (0, 1), (15, 1)])
def test_owned_expert_range(ctx, dev, start, count):
    E, k, B, H, I, G = 16, 4, 6, 512, 256, 32
    rig = Rig(dev, H, I, E, k, G, True, nb=E, seed=start * 31 + count)
    logits = wl.bf16_normal(rig.rng, (B, E))
    routes, _ = oracle.topk(logits, k, telemetry=False)
    routes = routes.astype(np.uint32)
    x = wl.bf16_normal(rig.rng, (B, H))
    h, y, ctl, _ = _run_batched(ctx, rig, x, routes, B, start, count)
    e = routes & 0xFFFF
    assert ctl[3] == np.count_nonzero((e >= start) & (e < start + count))
    _check(rig, x, routes, h, y, start, count)


@pytest.mark.parametrize("use_range", [False, True])
def test_unbatched_form(ctx, dev, use_range):
    """Unbatched specialization: one token, intermediates [k][I/2] words with
    no route map, control NULL (every expert) or an owned range."""
    torch = _torch()
    E, k, H, I, G = 32, 6, 1024, 512, 32
    rig = Rig(dev, H, I, E, k, G, False, nb=8, seed=7 + use_range)
    experts = rig.rng.choice(E, size=(1, k), replace=False)
    experts[0, -1] = 40                                   # id >= E: skipped
    routes = _route_words(experts, rig.rng.uniform(0.1, 1, (1, k)))
    x = wl.bf16_normal(rig.rng, (1, H))
    start, count = (8, 16) if use_range else (0, 0)
    control = to_dev(np.array([1, start, count, 0, 0, 0, 0, 0], np.uint32), dev) if use_range else None
    gspec = int4_ct_spec("gate_up", H, I, E, k, G, scale_bf16=False, batch1=False)
    dspec = int4_ct_spec("down", H, I, E, k, G, scale_bf16=False, batch1=False)
    inter = torch.full((k * I,), SENTINEL, dtype=torch.int16, device=dev)
    out = torch.full((k, H), SENTINEL, dtype=torch.int16, device=dev)
    r_dev = to_dev(routes, dev)
    ctx.int4_moe_gate_up(gspec, to_dev(x, dev), r_dev, inter, rig.bank.addresses, rig.bank.gate_slots, control, 1)
    ctx.int4_moe_down(dspec, inter, r_dev, out, rig.bank.addresses, rig.bank.down_slots, control, 1)
    h = to_np(inter, np.uint16).reshape(1, k, I)
    y = to_np(out, np.uint16).reshape(1, k, H)
    _check(rig, x, routes, h, y, start, count)
    with pytest.raises(NerveHipError):
        ctx.int4_moe_gate_up(gspec, to_dev(x, dev), r_dev, inter, rig.bank.addresses, rig.bank.gate_slots, control,
                             2)


def test_invalid_slots_skip_the_route(ctx, dev):
    """Unbound slot, slot beyond the table, short byte count, null address and
    a weight address that is not 16-byte aligned: that expert's routes are
    skipped; the others are unaffected."""
    E, k, B, H, I, G = 8, 2, 4, 256, 128, 32
    rig = Rig(dev, H, I, E, k, G, True, nb=E, seed=99)
    experts = np.array([[0, 1], [2, 3], [4, 5], [6, 7]])
    routes = _route_words(experts, np.full((B, k), 0.5))
    x = wl.bf16_normal(rig.rng, (B, H))
    base_h, base_y, _, _ = _run_batched(ctx, rig, x, routes, B)
    _check(rig, x, routes, base_h, base_y)
    recs = np.array(rig.bank.records, np.uint64).reshape(-1, 8).astype(np.uint32)
    gslots = to_np(rig.bank.gate_slots, np.uint32).copy()
    dslots = to_np(rig.bank.down_slots, np.uint32).copy()
    cases = []
    g1 = gslots.copy(); g1[2 * 1 + 0] = 0xFFFFFFFF; cases.append((1, recs, g1))
    g2 = gslots.copy(); g2[2 * 3 + 1] = 10_000; cases.append((3, recs, g2))
    r3 = recs.copy(); r3[gslots[2 * 5 + 0], 2] -= 1; cases.append((5, r3, gslots))
    r4 = recs.copy(); r4[gslots[2 * 6 + 1], 0:2] = 0; cases.append((6, r4, gslots))
    # a weight record 4-byte but not 16-byte aligned (rows are read in 16-byte pieces)
    r5 = recs.copy(); r5[gslots[2 * 7 + 0], 0] += 4; cases.append((7, r5, gslots))
    for bad, rec, gs in cases:
        bank = rig.bank
        saved = (bank.addresses, bank.gate_slots)
        bank.addresses = u32_tensor(rec.reshape(-1), dev)
        bank.gate_slots = u32_tensor(gs, dev)
        try:
            h, _, _, _ = _run_batched(ctx, rig, x, routes, B)
        finally:
            bank.addresses, bank.gate_slots = saved
        skipped = (experts == bad)
        assert np.all(h[skipped] == SENTINEL), bad
        assert np.array_equal(h[~skipped], base_h[~skipped]), bad


def test_entry_points_reject_other_families(ctx, dev):
    torch = _torch()
    z = torch.zeros(64, dtype=torch.int32, device=dev)
    spec_int4 = int4_ct_spec("gate_up", 256, 128, 8, 2, 32)
    with pytest.raises(NerveHipError):
        ctx.mxfp4_moe_gate_up(spec_int4, z, None, z, z, z, z, z, 1)
    with pytest.raises(NerveHipError):
        ctx.int4_moe_gate_up(gate_up_spec(256, 128, 8, 2, 7.0), z, z, z, z, z, z, 1)
    with pytest.raises(NerveHipError):
        ctx.int4_moe_down(spec_int4, z, z, z, z, z, z, 1)


def test_address_record_helper_layout():
    """Records the bank builds point at the tensors with their byte counts."""
    torch = _torch()
    t = torch.zeros(10, dtype=torch.int32, device="cuda:0")
    r = address_record(t)
    assert (r[0] | (r[1] << 32)) == t.data_ptr() and r[2] == 40 and r[6] == 1
