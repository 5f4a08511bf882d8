"""GPU parity: router projection (a5), top-k (a6) and route compaction (a7),
through the C ABI, against the CPU oracle.  Expert indices and permutations
are compared bit for bit; route weights within bf16 tolerance."""
import numpy as np
import pytest

import oracle
from nerve_amd import workloads as wl
from nerve_amd.moe import down_spec, gate_up_spec, topk_spec

from helpers import to_dev, to_np

pytestmark = pytest.mark.gpu


def _torch():
    import torch

    return torch


@pytest.mark.parametrize("B,H,E", [(16, 2880, 32), (2048, 2880, 128), (3, 100, 5)])
def test_router_linear(ctx, dev, B, H, E):
    torch = _torch()
    rng = np.random.default_rng(B + E)
    x = wl.bf16_normal(rng, (B, H))
    w = wl.bf16_normal(rng, (E, H), 0.02)
    out = torch.zeros(B, E, dtype=torch.int16, device=dev)
    ctx.router_linear_bf16(to_dev(x, dev), to_dev(w, dev), out, B, H, E)
    got = wl.bf16_bits_to_f32(to_np(out, np.uint16)).astype(np.float64)
    ref = wl.bf16_bits_to_f32(oracle.router_linear(x, w)).astype(np.float64)
    ideal = wl.bf16_bits_to_f32(x).astype(np.float64) @ wl.bf16_bits_to_f32(w).astype(np.float64).T
    # bf16 outputs: within one bf16 ulp of the oracle (and of the f64 ideal)
    ulp = np.maximum(np.abs(ref), 1e-30) * 2.0 ** -7
    assert np.all(np.abs(got - ref) <= ulp + 1e-6)
    assert np.all(np.abs(got - ideal) <= 2 * ulp + 1e-5)


def test_topk_config3_prefill_logits(ctx, dev):
    """The prefill bench's own top-k: config 3's Zipf-skewed logits (B = 2048,
    E = 128, k = 4) through topk_kernel; indices and telemetry bit-exact."""
    torch = _torch()
    d = wl.config3()
    logits, B, E, k = d["logits"], d["B"], d["E"], d["k"]
    spec = topk_spec(E, k)
    T = E + E * (E - 1) // 2
    routes = torch.zeros(B, k, dtype=torch.int32, device=dev)
    tel = torch.zeros(T, dtype=torch.int32, device=dev)
    ctx.moe_router_topk(spec, to_dev(logits, dev), None, routes, tel, B)
    ref, ref_tel = oracle.topk(logits, k)
    gi, gw = _route_split(to_np(routes, np.uint32))
    ri, rw = _route_split(ref)
    assert np.array_equal(gi, ri)
    assert np.allclose(gw, rw, rtol=2e-2, atol=1e-6)
    assert np.array_equal(to_np(tel, np.uint32), ref_tel)
    # the skew the bench relies on: the busiest expert takes > 1000 routes
    assert np.bincount(ri.reshape(-1), minlength=E).max() > 1000


def _route_split(routes):
    r = np.asarray(routes, np.uint32)
    return r & 0xFFFF, wl.bf16_bits_to_f32((r >> 16).astype(np.uint16))


@pytest.mark.parametrize("B,E,k,sigmoid,normalize,softcap,bias", [
    (16, 32, 4, False, True, 0.0, "nobias"),
    (64, 128, 8, False, True, 0.0, "biasf32"),
    (9, 256, 6, True, True, 0.0, "biasbf16"),
    (5, 64, 2, False, False, 30.0, "nobias"),
    (7, 16, 3, True, False, 0.0, "nobias"),
])
def test_topk_routed(ctx, dev, B, E, k, sigmoid, normalize, softcap, bias):
    torch = _torch()
    rng = np.random.default_rng(E + k)
    logits = wl.bf16_normal(rng, (B, E), 2.0)
    logits[0, 3] = logits[0, 7] = logits[0, 11] = wl.f32_to_bf16_bits(np.float32(9.0))  # ties -> lower index
    b = None
    bias_np = None
    if bias == "biasf32":
        bias_np = rng.standard_normal(E).astype(np.float32) * np.float32(0.1)
        b = to_dev(bias_np, dev)
    elif bias == "biasbf16":
        bb = wl.bf16_normal(rng, (E,), 0.1)
        bias_np = wl.bf16_bits_to_f32(bb)
        b = to_dev(bb, dev)
    spec = topk_spec(E, k, sigmoid=sigmoid, normalize=normalize, softcap=softcap, bias=bias)
    T = E + E * (E - 1) // 2
    routes = torch.zeros(B, k, dtype=torch.int32, device=dev)
    tel = torch.zeros(T, dtype=torch.int32, device=dev)
    ctx.moe_router_topk(spec, to_dev(logits, dev), b, routes, tel, B)
    ref, ref_tel = oracle.topk(logits, k, mode=0, activation=int(sigmoid), normalize=int(normalize),
                               softcap=softcap, bias=bias_np)
    got = to_np(routes, np.uint32)
    gi, gw = _route_split(got)
    ri, rw = _route_split(ref)
    assert np.array_equal(gi, ri)                        # indices bit-exact
    assert np.all(np.diff(gi.astype(np.int64), axis=1) > 0)   # ascending
    assert np.allclose(gw, rw, rtol=2e-2, atol=1e-6)     # weights in bf16 tolerance
    assert np.array_equal(to_np(tel, np.uint32), ref_tel)  # telemetry counts exact


@pytest.mark.parametrize("act", ["sigmoid", "softmax", "sqrtsoftplus"])
def test_score_router(ctx, dev, act):
    torch = _torch()
    B, E, k, A = 11, 64, 4, 2
    rng = np.random.default_rng(len(act))
    logits = wl.bf16_normal(rng, (B, E), 1.5)
    bias = rng.standard_normal(E).astype(np.float32) * np.float32(0.01)
    spec = f"moe_router_batch1_score_topk_{act}_bf16_r{E}_k{k}_a{A}w0.5_norm1_scale2.5_biasf32.comp"
    T = E + A
    routes = torch.zeros(B, k + A, dtype=torch.int32, device=dev)
    tel = torch.zeros(T + T * (T - 1) // 2, dtype=torch.int32, device=dev)
    ctx.moe_router_topk(spec, to_dev(logits, dev), to_dev(bias, dev), routes, tel, B)
    ref, ref_tel = oracle.topk(logits, k, mode=1, activation=["sigmoid", "softmax", "sqrtsoftplus"].index(act),
                               normalize=1, routed_scale=2.5, always_count=A, always_weight=0.5, bias=bias)
    gi, gw = _route_split(to_np(routes, np.uint32))
    ri, rw = _route_split(ref)
    assert np.array_equal(gi, ri)
    assert np.allclose(gw, rw, rtol=2e-2, atol=1e-6)
    assert np.array_equal(to_np(tel, np.uint32), ref_tel)


# n = B k routes: one wave's ballot ranks (n <= 64), the counting sort with
# each wave's segment in registers (1024 < n <= 8192; 8192 fills them), its
# looped form (n > 8192), and the rank loop (64 < n <= 1024).
@pytest.mark.parametrize("B,k,E", [(16, 4, 32), (2048, 4, 128), (1, 1, 8), (300, 6, 64), (2100, 4, 128),
                                   (100, 4, 32)])
@pytest.mark.parametrize("partition", [None, (8, 20)])
def test_route_compact(ctx, dev, B, k, E, partition):
    torch = _torch()
    rng = np.random.default_rng(B * k + E)
    logits = wl.bf16_normal(rng, (B, E))
    routes, _ = oracle.topk(logits, k, telemetry=False)
    I, H = 256, 128
    spec = gate_up_spec(H, I, E, k, 7.0)
    frame_words = k * I // 2 + k
    inter = torch.zeros(B * frame_words, dtype=torch.int32, device=dev)
    start, count = partition or (0, 0)
    control = to_dev(np.array([B, start, count, 0, 0, 0, 0, 0], np.uint32), dev)
    ctx.moe_route_compact(spec, to_dev(routes, dev), inter, control, B)
    fr = to_np(inter, np.uint32).reshape(B, frame_words)[:, k * I // 2:].reshape(-1)
    cmap, ctl = oracle.route_compact(routes, k, (I + 31) // 32, B, start, count)
    got_ctl = to_np(control, np.uint32)[:7]
    assert np.array_equal(got_ctl, ctl)
    n = int(ctl[3])
    assert np.array_equal(fr[:n], cmap[:n])
    if partition is None:
        # closed form: the stable argsort of the expert ids
        assert np.array_equal(fr, np.argsort(routes.reshape(-1) & 0xFFFF, kind="stable"))


@pytest.mark.parametrize("B,k,E", [(16, 4, 32), (2048, 4, 128), (1, 1, 8), (300, 6, 64)])
@pytest.mark.parametrize("partition", [None, (8, 20), (0, 1)])
def test_route_count_control_words(ctx, dev, B, k, E, partition):
    """The count stage before down (no intermediates): control words only,
    with the down projection's 64-row tiles per route."""
    rng = np.random.default_rng(B + 3 * k + E)
    routes, _ = oracle.topk(wl.bf16_normal(rng, (B, E)), k, telemetry=False)
    I, H = 256, 320
    start, count = partition or (0, 0)
    control = to_dev(np.array([B, start, count, 9, 9, 9, 9, 9], np.uint32), dev)
    ctx.moe_route_compact(down_spec(H, I, E, k), to_dev(routes, dev), None, control, B)
    _, ctl = oracle.route_compact(routes, k, (H + 63) // 64, B, start, count)
    got = to_np(control, np.uint32)
    assert np.array_equal(got[:7], ctl)
    assert got[7] == 9


def test_route_compact_expert_ids_beyond_spec(ctx, dev):
    """Garbage expert ids (>= E) still sort by the full 16-bit key, as the
    reference's rank loop does."""
    torch = _torch()
    B, k, E, I, H = 400, 4, 32, 64, 64
    rng = np.random.default_rng(11)
    ex = rng.integers(0, E, size=(B, k)).astype(np.uint32)
    ex[3, 1] = 200
    ex[17, 0] = 65535
    routes = ex | (np.uint32(0x3F80) << np.uint32(16))
    spec = gate_up_spec(H, I, E, k, 7.0)
    frame_words = k * I // 2 + k
    inter = torch.zeros(B * frame_words, dtype=torch.int32, device=dev)
    control = to_dev(np.array([B, 0, 0, 0, 0, 0, 0, 0], np.uint32), dev)
    ctx.moe_route_compact(spec, to_dev(routes, dev), inter, control, B)
    fr = to_np(inter, np.uint32).reshape(B, frame_words)[:, k * I // 2:].reshape(-1)
    assert np.array_equal(fr, np.argsort(ex.reshape(-1), kind="stable"))


@pytest.mark.parametrize("B,H,E,k,kind", [
    (16, 2880, 32, 4, "softmax"),          # the MoE decode block (config 2)
    (1, 2880, 32, 4, "softmax"),
    (64, 512, 128, 8, "sigmoid_biasbf16"),
    (5, 160, 48, 3, "score_softmax"),      # E not a multiple of 32, always-selected experts
    (3, 96, 16, 2, "softmax"),             # one block (it quantizes at its end); q 4 bytes off 16: 32-lane units
])
def test_route_fused_matches_separate(ctx, dev, B, H, E, k, kind):
    """nerve_hip_moe_route_fused: logits within one bf16 ulp of the router linear's
    (and of the oracle's); routes, telemetry, route map and control words
    bit-identical to top-k + compaction run on its own logits; the quantized
    hidden rows bit-identical to the standalone pow2 quantizer's and the
    oracle's."""
    torch = _torch()
    rng = np.random.default_rng(B * E + k)
    x = wl.bf16_normal(rng, (B, H))
    w = wl.bf16_normal(rng, (E, H), 0.05)
    bias, A = None, 0
    if kind == "softmax":
        tspec = topk_spec(E, k)
    elif kind == "sigmoid_biasbf16":
        bias = to_dev(wl.bf16_normal(rng, (E,), 0.1), dev)
        tspec = topk_spec(E, k, sigmoid=True, bias="biasbf16")
    else:
        A = 2
        bias = to_dev(rng.standard_normal(E).astype(np.float32) * np.float32(0.01), dev)
        tspec = f"moe_router_batch1_score_topk_softmax_bf16_r{E}_k{k}_a{A}w0.5_norm1_scale2.5_biasf32.comp"
    kt = k + A
    I = 256
    mspec = gate_up_spec(H, I, E, kt, 7.0)
    T = (E + A) + (E + A) * (E + A - 1) // 2
    frame_words = kt * I // 2 + kt

    def bufs():
        return dict(logits=torch.zeros(B, E, dtype=torch.int16, device=dev),
                    routes=torch.zeros(B, kt, dtype=torch.int32, device=dev),
                    tel=torch.zeros(T, dtype=torch.int32, device=dev),
                    inter=torch.zeros(B * frame_words, dtype=torch.int32, device=dev),
                    control=to_dev(np.array([B, 0, 0, 0, 0, 0, 0, 0], np.uint32), dev))

    xd, wd = to_dev(x, dev), to_dev(w, dev)
    f = bufs()
    nblk = (H + 127) // 128
    off = 4 if H == 96 else 0
    hq = torch.full((B * H + off,), 0x55, dtype=torch.uint8, device=dev)[off:].view(B, H)
    hs = torch.full((B, nblk), -1.0, dtype=torch.float32, device=dev)
    assert ctx.moe_route_fused(tspec, mspec, xd, wd, f["logits"], bias, f["routes"], f["tel"], f["inter"],
                               f["control"], B, hidden_q=hq, hidden_scales=hs)
    sq = torch.zeros(B, H, dtype=torch.uint8, device=dev)
    ss = torch.zeros(B, nblk, dtype=torch.float32, device=dev)
    ctx.quantize_fp8_e4m3(f"quantize_fp8_e4m3_spow2_b128_h{H}.comp", xd, B, sq, ss)
    oq, os_ = oracle.quantize_blocks(x, True)
    assert np.array_equal(to_np(hq, np.uint8), to_np(sq, np.uint8))
    assert np.array_equal(to_np(hs, np.float32), to_np(ss, np.float32))
    assert np.array_equal(to_np(hq, np.uint8), oq) and np.array_equal(to_np(hs, np.float32), os_)
    lin = torch.zeros(B, E, dtype=torch.int16, device=dev)
    ctx.router_linear_bf16(xd, wd, lin, B, H, E)
    got = wl.bf16_bits_to_f32(to_np(f["logits"], np.uint16)).astype(np.float64)
    ref = wl.bf16_bits_to_f32(oracle.router_linear(x, w)).astype(np.float64)
    ulp = np.maximum(np.abs(ref), 1e-30) * 2.0 ** -7
    assert np.all(np.abs(got - ref) <= ulp + 1e-6)
    assert np.all(np.abs(got - wl.bf16_bits_to_f32(to_np(lin, np.uint16))) <= ulp + 1e-6)
    # the separate top-k and compaction on the fused logits
    s = bufs()
    ctx.moe_router_topk(tspec, f["logits"], bias, s["routes"], s["tel"], B)
    ctx.moe_route_compact(mspec, s["routes"], s["inter"], s["control"], B)
    for name, dt in (("routes", np.uint32), ("tel", np.uint32), ("inter", np.uint32), ("control", np.uint32)):
        assert np.array_equal(to_np(f[name], dt), to_np(s[name], dt)), name
    if kind == "softmax":
        ref, _ = oracle.topk(to_np(f["logits"], np.uint16), k)
        assert np.array_equal(to_np(f["routes"], np.uint32) & 0xFFFF, ref & 0xFFFF)


def test_route_fused_quantized_rows_need_both_buffers(ctx, dev):
    from nerve_amd.hip import NerveHipError

    torch = _torch()
    B, H, E, k = 4, 256, 8, 2
    routes = torch.zeros(B, k, dtype=torch.int32, device=dev)
    control = to_dev(np.array([B, 0, 0, 0, 0, 0, 0, 0], np.uint32), dev)
    x = torch.zeros(B, H, dtype=torch.int16, device=dev)
    w = torch.zeros(E, H, dtype=torch.int16, device=dev)
    inter = torch.zeros(B * (k * 64 // 2 + k), dtype=torch.int32, device=dev)
    hq = torch.zeros(B, H, dtype=torch.uint8, device=dev)
    with pytest.raises(NerveHipError, match="INVALID_ARGUMENT"):
        ctx.moe_route_fused(topk_spec(E, k), gate_up_spec(H, 64, E, k, 7.0), x, w, None, None, routes, None, inter,
                            control, B, hidden_q=hq)


def test_route_fused_declines_large_batches(ctx, dev):
    torch = _torch()
    B, H, E, k = 65, 64, 8, 2
    routes = torch.zeros(B, k, dtype=torch.int32, device=dev)
    control = to_dev(np.array([B, 0, 0, 0, 0, 0, 0, 0], np.uint32), dev)
    x = torch.zeros(B, H, dtype=torch.int16, device=dev)
    w = torch.zeros(E, H, dtype=torch.int16, device=dev)
    assert not ctx.moe_route_fused(topk_spec(E, k), gate_up_spec(H, 64, E, k, 7.0), x, w, None, None, routes, None,
                                   None, control, B)


@pytest.mark.parametrize("E", [32, 100])
def test_topk_fewer_selectable_than_k(ctx, dev, E):
    """A row with only two non-NaN logits (experts 0 and 5) and k = 4: the
    rounds that find nothing select expert 0, which sorts first, so the
    route list is 0, 0, 0, 5 with expert 0's weight three times; expert 0 is
    counted three times and the pair (0, 5) three times.  E = 32 takes the
    lane-parallel form, E = 100 the round-by-round one: both must agree."""
    torch = _torch()
    k = 4
    lg = np.full((1, E), 0x7FC0, np.uint16)            # bf16 NaN
    lg[0, 0] = wl.f32_to_bf16_bits(np.float32(1.0))
    lg[0, 5] = wl.f32_to_bf16_bits(np.float32(2.0))
    T = E + E * (E - 1) // 2
    routes = torch.full((1, k), -1, dtype=torch.int32, device=dev)
    tel = torch.zeros(T, dtype=torch.int32, device=dev)
    ctx.moe_router_topk(topk_spec(E, k), to_dev(lg, dev), None, routes, tel, 1)
    got = to_np(routes, np.uint32)[0]
    assert list(got & 0xFFFF) == [0, 0, 0, 5]
    e1 = np.exp(np.float32(-1.0))
    den = np.float32(1.0) + e1 + e1 + e1
    w = wl.bf16_bits_to_f32((got >> 16).astype(np.uint16))
    assert np.allclose(w, [e1 / den, e1 / den, e1 / den, 1.0 / den], rtol=1e-2)
    assert len(set(got[:3].tolist())) == 1
    t = to_np(tel, np.uint32)
    assert t[0] == 3 and t[5] == 1 and t[E + 5 - 1] == 3 and t.sum() == 7
    if E == 32:
        # the same row through the fused decode routing (two tokens per wave)
        H, I = 64, 64
        x = np.zeros((1, H), np.uint16)
        w = np.zeros((E, H), np.uint16)
        x[0, 0] = wl.f32_to_bf16_bits(np.float32(1.0))
        w[:, 0] = lg[0]                                   # logit e = 1 * w[e, 0]
        frame_words = k * I // 2 + k
        r2 = torch.full((1, k), -1, dtype=torch.int32, device=dev)
        t2 = torch.zeros(T, dtype=torch.int32, device=dev)
        inter = torch.zeros(frame_words, dtype=torch.int32, device=dev)
        control = to_dev(np.array([1, 0, 0, 0, 0, 0, 0, 0], np.uint32), dev)
        assert ctx.moe_route_fused(topk_spec(E, k), gate_up_spec(H, I, E, k, 7.0), to_dev(x, dev), to_dev(w, dev),
                                   None, None, r2, t2, inter, control, 1)
        assert np.array_equal(to_np(r2, np.uint32)[0], got)
        assert np.array_equal(to_np(t2, np.uint32), t)
