"""GPU parity at the benchmarked shapes: the FP8 LM head at config 4's own
shape (N = 201088, K = 2880, M = 1 / 64 / 512), the whole decode MoE block
(MoEBlock.forward, the bench's exact launch sequence) at config 2, the
reference's real MXFP4 geometry (H = 4096, I = 2048, E = 256, k = 6;
runtime-rs/src/vulkan_compute/mxfp4_tests.rs:316-420), and the
PREQUANTIZED_INPUT gate_up fed by the standalone and RMSNorm quantizers."""
import numpy as np
import pytest

import oracle
from nerve_amd import workloads as wl
from nerve_amd.hip import check_specialization
from nerve_amd.moe import ExpertBank, MoEBlock, address_record, down_spec, gate_up_spec, u32_tensor

from bounds import moe_down_atol, moe_gate_up_atol
from helpers import bf16_close, rel_err_normwise, to_dev, to_np

pytestmark = pytest.mark.gpu


def _torch():
    import torch

    return torch


# --------------------------------------------------------------------------
# Config 4: FP8 LM head at N = 201088, K = 2880
# --------------------------------------------------------------------------

def _head_weights_on_device(dev, N, K, seed):
    """N(0, 0.02) rows, per-row scale bf16(amax/448), e4m3 by torch's RNE
    cast (|w / s| <= 448 (1 + 2^-8), so no value saturates) -- bench.py's
    generator; the grid repeats each row's scale over the K blocks."""
    torch = _torch()
    g = torch.Generator(device=dev).manual_seed(seed)
    W = torch.empty(N, K, dtype=torch.uint8, device=dev)
    sc = torch.empty(N, dtype=torch.float32, device=dev)
    for r0 in range(0, N, 16384):
        wf = torch.randn(min(16384, N - r0), K, generator=g, device=dev) * 0.02
        s = (wf.abs().amax(dim=1) / 448.0).to(torch.bfloat16).float()
        sc[r0:r0 + wf.shape[0]] = s
        W[r0:r0 + wf.shape[0]] = (wf / s[:, None]).to(torch.float8_e4m3fn).view(torch.uint8)
    nblk = (K + 127) // 128
    grid = sc.to(torch.bfloat16).view(torch.int16)[:, None].repeat(1, nblk).contiguous()
    return W, grid


@pytest.mark.parametrize("M", [1, 64, 512])
def test_fp8_head_config4_full_shape(ctx, dev, M):
    """tied_output_projection_batch_fp8_e4m3.comp.template:94-186 followed by
    greedy_sampler_f32.comp.template:25-109 at config 4.  The oracle runs on
    2048 sampled vocabulary rows plus every token's GPU argmax row (a row's
    logits depend only on that row); the argmax is checked against the argmax
    of the full GPU logits, and the chosen row's oracle logit against the
    oracle maximum over the sample (near-ties allowed)."""
    torch = _torch()
    N, K = 201088, 2880
    W, grid = _head_weights_on_device(dev, N, K, 20260004 + M)
    rng = np.random.default_rng(4000 + M)
    x = wl.bf16_normal(rng, (M, K))
    lf = torch.zeros(M, N, dtype=torch.float32, device=dev)
    lb = torch.zeros(M, N, dtype=torch.int16, device=dev)
    am = torch.zeros(M, dtype=torch.int32, device=dev)
    spec = f"tied_output_projection_batch4_fp8_e4m3_b1x128_{N}x{K}_scale1_to_f32.comp"
    ctx.fp8_output_projection(spec, to_dev(x, dev), W, grid, lf, lb, am, M)
    ids = to_np(am, np.uint32)
    lf_np = to_np(lf, np.float32)
    assert np.array_equal(ids, oracle.argmax(lf_np))
    assert np.array_equal(to_np(lb, np.uint16), wl.f32_to_bf16_bits(lf_np))
    rows = np.unique(np.concatenate([rng.choice(N, 2048, replace=False), ids.astype(np.int64),
                                     np.array([0, N - 1])]))
    rows_d = torch.from_numpy(rows).to(dev)
    W_s = to_np(W[rows_d].contiguous(), np.uint8)
    g_s = to_np(grid[rows_d].contiguous(), np.uint16)
    ref = oracle.fp8_output_projection(x, W_s, g_s, 1, 1.0)
    got = lf_np[:, rows]
    assert rel_err_normwise(got, ref) <= 1e-3
    # per token as well (rows of very different magnitude would hide in the norm)
    for m in range(0, M, max(1, M // 16)):
        assert rel_err_normwise(got[m], ref[m]) <= 1e-3, m
    pos = np.searchsorted(rows, ids)
    tol = 2e-3 * np.max(np.abs(ref), axis=1)
    assert np.all(ref.max(axis=1) - ref[np.arange(M), pos] <= tol)


# --------------------------------------------------------------------------
# Config 2: the bench's MoE decode block, end to end
# --------------------------------------------------------------------------

def _dv(a, dev):
    return to_dev(np.ascontiguousarray(a), dev)


@pytest.mark.parametrize("pad", [600, 6000])
def test_moe_block_package_wide_address_table(ctx, dev, pad):
    """A package-wide address table (pad unrelated records ahead of the
    block's, slots rebased): past 512 records the token-form gate_up reads
    its experts' records from memory instead of staging the table, past what
    its LDS holds the down's small plan does the same; the block's outputs
    are bit-identical to those with the block's own table."""
    torch = _torch()
    rng = np.random.default_rng(77 + pad)
    E, k, B, H, I = 32, 4, 16, 512, 512
    d = wl.moe_experts(rng, E, H, I)
    router = _dv(wl.bf16_normal(rng, (E, H), 0.02), dev)
    hidden = _dv(wl.bf16_normal(rng, (B, H)), dev)
    bank = ExpertBank(*(_dv(d[n], dev) for n in ("gate_w", "gate_s", "up_w", "up_s", "down_w", "down_s")))
    ref_block = MoEBlock(ctx, router, bank, k)
    ref = to_np(ref_block.forward(hidden), np.uint16).copy()
    ref_inter = to_np(ref_block.buffers(B)["inter"], np.uint32).copy()
    big = ExpertBank(*(_dv(d[n], dev) for n in ("gate_w", "gate_s", "up_w", "up_s", "down_w", "down_s")))
    junk = rng.integers(0, 2 ** 32, size=pad * 8, dtype=np.uint64).astype(np.uint32)
    big.addresses = torch.cat([to_dev(junk, dev).view(torch.int32), big.addresses])
    big.gate_slots = big.gate_slots + pad
    big.down_slots = big.down_slots + pad
    block = MoEBlock(ctx, router, big, k)
    out = to_np(block.forward(hidden), np.uint16)
    torch.cuda.synchronize()
    assert np.array_equal(to_np(block.buffers(B)["inter"], np.uint32), ref_inter)
    assert np.array_equal(out, ref)


def test_moe_block_forward_config2(ctx, dev):
    """MoEBlock.forward at config 2 (E = 32, k = 4, B = 16, H = I = 2880):
    fused routing (router partials + top-k + compaction), token-form gate_up,
    down with the count stage folded in, combine -- against the oracle chain
    router_linear -> topk -> route_compact -> gate_up -> down -> reduce.
    Logits within one bf16 ulp; routes, route map and control words bit-exact
    given the GPU's logits; h and expert outputs elementwise within the bf16
    tolerance stage by stage; the block output bit-exact from the GPU's expert
    outputs and normwise against the composed oracle chain."""
    d = wl.config2()
    B, E, k, H, I = d["B"], d["E"], d["k"], d["H"], d["I"]
    bank = ExpertBank(*(_dv(d[n], dev) for n in ("gate_w", "gate_s", "up_w", "up_s", "down_w", "down_s")))
    block = MoEBlock(ctx, _dv(d["router_w"], dev), bank, k)
    out = to_np(block.forward(_dv(d["hidden"], dev)), np.uint16)
    b = block.buffers(B)
    logits = to_np(b["logits"], np.uint16)
    ref_logits = oracle.router_linear(d["hidden"], d["router_w"])
    dl = np.abs(logits.astype(np.int32) - ref_logits.astype(np.int32))
    assert dl.max() <= 1 and np.mean(dl == 0) > 0.95
    routes = to_np(b["routes"], np.uint32)
    ref_routes, _ = oracle.topk(logits, k, telemetry=False)
    assert np.array_equal(routes & 0xFFFF, ref_routes & 0xFFFF)
    ok, worst, _ = bf16_close((routes >> 16).astype(np.uint16), (ref_routes >> 16).astype(np.uint16), name="route weights")
    assert ok, worst
    frame = k * I // 2 + k
    frames = to_np(b["inter"], np.uint32).reshape(B, frame)
    cmap, _ = oracle.route_compact(routes, k, (I + 31) // 32, B)
    assert np.array_equal(frames[:, k * I // 2:].reshape(-1), cmap)
    _, ctl_down = oracle.route_compact(routes, k, (H + 63) // 64, B)
    assert np.array_equal(to_np(b["control"], np.uint32)[:7], ctl_down)
    h = frames[:, : k * I // 2].copy().view(np.uint16).reshape(B, k, I)
    h_ref = oracle.moe_gate_up(d["hidden"], routes, cmap, B * k, k, d["gate_w"], d["gate_s"], d["up_w"], d["up_s"],
                               7.0)
    ok, worst, exact = bf16_close(h, h_ref, atol=moe_gate_up_atol(d["hidden"], routes, d["gate_w"], d["gate_s"], d["up_w"], d["up_s"], 7.0), name="config2 gate_up")
    assert ok and exact > 0.9, (worst, exact)
    eo = to_np(b["expert_out"], np.uint16)
    eo_ref = oracle.moe_down(h, routes, cmap, B * k, d["down_w"], d["down_s"])
    ok, worst, exact = bf16_close(eo, eo_ref, atol=moe_down_atol(h, routes, d["down_w"], d["down_s"]),
                                  name="config2 down")
    assert ok and exact > 0.9, (worst, exact)
    assert np.array_equal(out, oracle.moe_reduce(eo, 1.0))
    eo_chain = oracle.moe_down(h_ref, routes, cmap, B * k, d["down_w"], d["down_s"])
    out_chain = wl.bf16_bits_to_f32(oracle.moe_reduce(eo_chain, 1.0))
    assert rel_err_normwise(wl.bf16_bits_to_f32(out), out_chain) <= 2e-2
    # gate_up ran in its prequantized form on the routing launch's quantized
    # hidden rows: the bf16-input form on the same routes writes the same h
    torch = _torch()
    inter2 = b["inter"].clone()
    ctx.mxfp4_moe_gate_up(block.gate_up, _dv(d["hidden"], dev), None, b["routes"], inter2, bank.addresses,
                          bank.gate_slots, b["control"], B)
    torch.cuda.synchronize()
    assert np.array_equal(to_np(inter2, np.uint32), frames.reshape(-1))


# --------------------------------------------------------------------------
# The reference's real MXFP4 geometry: H = 4096, I = 2048, E = 256, k = 6
# --------------------------------------------------------------------------

@pytest.mark.parametrize("B", [1, 6])
def test_moe_real_geometry_e256_k6(ctx, dev, B):
    """mxfp4_tests.rs:316-420: E = 256 experts, six selected per token
    ([2, 17, 63, 127, 191, 255], B in 1..6), H = 4096, I = 2048.  Only the
    selected experts hold distinct random weights; every other expert's
    records point at one shared expert (valid, never selected).  Each token
    here routes to a rotation of the six experts with distinct weights."""
    torch = _torch()
    E, k, H, I = 256, 6, 4096, 2048
    sel = np.array([2, 17, 63, 127, 191, 255])
    rng = np.random.default_rng(316 + B)
    d = wl.moe_experts(rng, len(sel) + 1, H, I)          # six selected experts + one shared filler
    names = ("gate_w", "gate_s", "up_w", "up_s", "down_w", "down_s")
    dd = {n: _dv(d[n], dev) for n in names}
    slot_of = {int(e): i for i, e in enumerate(sel)}
    recs, gslots, dslots = [], [], []
    for e in range(E):
        j = slot_of.get(e, len(sel))
        for n in names[:4]:
            gslots.append(len(recs) // 8)
            recs += address_record(dd[n][j])
        for n in names[4:]:
            dslots.append(len(recs) // 8)
            recs += address_record(dd[n][j])
    addresses, gate_slots, down_slots = u32_tensor(recs, dev), u32_tensor(gslots, dev), u32_tensor(dslots, dev)
    ex = np.stack([np.roll(sel, t) for t in range(B)])
    wts = rng.uniform(0.05, 0.4, size=(B, k)).astype(np.float32)
    routes = ((wl.f32_to_bf16_bits(wts).astype(np.uint32) << np.uint32(16)) | ex.astype(np.uint32))
    hidden = wl.bf16_normal(rng, (B, H))
    gu, dn = gate_up_spec(H, I, E, k, 7.0), down_spec(H, I, E, k)
    assert check_specialization(gu) == 0 and check_specialization(dn) == 0
    frame = k * I // 2 + k
    inter = torch.zeros(B * frame, dtype=torch.int32, device=dev)
    control = to_dev(np.array([B, 0, 0, 0, 0, 0, 0, 0], np.uint32), dev)
    eo_d = torch.zeros(B, k, H, dtype=torch.int16, device=dev)
    out_d = torch.zeros(B, H, dtype=torch.int16, device=dev)
    routes_d = to_dev(routes, dev)
    ctx.moe_route_compact(gu, routes_d, inter, control, B)
    ctx.mxfp4_moe_gate_up(gu, to_dev(hidden, dev), None, routes_d, inter, addresses, gate_slots, control, B)
    ctx.moe_route_compact(dn, routes_d, None, control, B)
    ctx.mxfp4_moe_down(dn, inter, routes_d, eo_d, addresses, down_slots, control, B)
    ctx.moe_reduce(eo_d, out_d, B, H, k, 1.0)
    # oracle on the compact bank: expert ids remapped to their bank index
    remap = np.array([slot_of.get(int(e), len(sel)) for e in range(E)], np.uint32)
    routes_c = (routes & np.uint32(0xFFFF0000)) | remap[routes & 0xFFFF]
    cmap, _ = oracle.route_compact(routes_c, k, (I + 31) // 32, B)
    cmap_gpu, _ = oracle.route_compact(routes, k, (I + 31) // 32, B)
    frames = to_np(inter, np.uint32).reshape(B, frame)
    assert np.array_equal(frames[:, k * I // 2:].reshape(-1), cmap_gpu)
    h = frames[:, : k * I // 2].copy().view(np.uint16).reshape(B, k, I)
    h_ref = oracle.moe_gate_up(hidden, routes_c, cmap, B * k, k, d["gate_w"], d["gate_s"], d["up_w"], d["up_s"], 7.0)
    ok, worst, exact = bf16_close(h, h_ref, atol=moe_gate_up_atol(hidden, routes_c, d["gate_w"], d["gate_s"], d["up_w"], d["up_s"], 7.0), name="e256 gate_up")
    assert ok and exact > 0.9, (worst, exact)
    eo = to_np(eo_d, np.uint16)
    eo_ref = oracle.moe_down(h, routes_c, cmap, B * k, d["down_w"], d["down_s"])
    ok, worst, exact = bf16_close(eo, eo_ref, atol=moe_down_atol(h, routes_c, d["down_w"], d["down_s"]),
                                  name="e256 down")
    assert ok and exact > 0.9, (worst, exact)
    assert np.array_equal(to_np(out_d, np.uint16), oracle.moe_reduce(eo, 1.0))


# --------------------------------------------------------------------------
# PREQUANTIZED_INPUT gate_up fed by the standalone and RMSNorm quantizers
# --------------------------------------------------------------------------

# The RMSNorm quantizer needs whole 128-column blocks (H % 128 == 0), so its
# decode case uses H = 4096; B = 160 takes the preparation launch and the
# grouped GEMM, the other shapes the token-form kernel.
@pytest.mark.parametrize("source,E,k,B,H,I", [("quantize_spow2", 32, 4, 16, 2880, 2880),
                                              ("quantize_spow2", 8, 2, 5, 512, 256),
                                              ("quantize_spow2", 8, 4, 160, 384, 256),
                                              ("rms_norm", 32, 4, 16, 4096, 2880),
                                              ("rms_norm", 8, 2, 5, 512, 256),
                                              ("rms_norm", 8, 4, 160, 384, 256)])
def test_prequant_gate_up(ctx, dev, source, E, k, B, H, I):
    """independent_sparse_moe_gate_up_batch1_prequant_mxfp4 (…gate_up_batch1_
    mxfp4.comp.template:21-38, 325): hidden frames e4m3 [B, H] plus f32 block
    scales [B, H/128] in place of bf16 hidden.  Fed by nerve_hip_quantize_fp8_
    e4m3 ("_spow2") or nerve_hip_rms_norm_quantize_fp8_e4m3 ("_spow2",
    block 128) output; the result must equal, bit for bit, the bf16-input
    gate_up on the bf16 rows those bytes quantize (the same e4m3 bytes and
    power-of-two scales), and match the oracle on the quantized rows."""
    torch = _torch()
    rng = np.random.default_rng(E + B + H + len(source))
    d = wl.moe_experts(rng, E, H, I)
    logits = wl.bf16_normal(rng, (B, E))
    routes, _ = oracle.topk(logits, k, telemetry=False)
    x = wl.bf16_normal(rng, (B, H))
    xd = to_dev(x, dev)
    nblk = (H + 127) // 128
    q = torch.zeros(B, H, dtype=torch.uint8, device=dev)
    s = torch.zeros(B, nblk, dtype=torch.float32, device=dev)
    if source == "quantize_spow2":
        ctx.quantize_fp8_e4m3(f"quantize_batch{B}_fp8_e4m3_spow2_b128_h{H}.comp", xd, B, q, s)
        rows_bf16 = x
    else:
        w = wl.bf16_normal(rng, (H,), 0.4)
        y = torch.zeros(B, H, dtype=torch.int16, device=dev)
        ctx.rms_norm_quantize_fp8_e4m3(f"rms_norm_quantize_batch{B}_fp8_e4m3_spow2_b128_h{H}_eps1e-05_offset1.comp",
                                       xd, to_dev(w, dev), y, q, s, B)
        rows_bf16 = to_np(y, np.uint16)
    # the bytes are the oracle quantization of those bf16 rows
    qr, sr = oracle.quantize_blocks(rows_bf16, True)
    assert np.array_equal(to_np(q, np.uint8), qr)
    assert np.array_equal(to_np(s, np.float32).view(np.uint32), sr.view(np.uint32))

    bank = ExpertBank(*(_dv(d[n], dev) for n in ("gate_w", "gate_s", "up_w", "up_s", "down_w", "down_s")))
    routes_d = to_dev(routes.astype(np.uint32), dev)
    frame = k * I // 2 + k
    gu = gate_up_spec(H, I, E, k, 7.0)
    gu_pq = gate_up_spec(H, I, E, k, 7.0, prequant=True)
    assert check_specialization(gu_pq) == 0

    def run(spec, hidden, scales):
        inter = torch.zeros(B * frame, dtype=torch.int32, device=dev)
        control = to_dev(np.array([B, 0, 0, 0, 0, 0, 0, 0], np.uint32), dev)
        ctx.moe_route_compact(gu, routes_d, inter, control, B)
        ctx.mxfp4_moe_gate_up(spec, hidden, scales, routes_d, inter, bank.addresses, bank.gate_slots, control, B)
        return to_np(inter, np.uint32).reshape(B, frame)

    fr_pq = run(gu_pq, q, s)
    fr_bf = run(gu, to_dev(rows_bf16, dev), None)
    assert np.array_equal(fr_pq, fr_bf)
    cmap, _ = oracle.route_compact(routes, k, (I + 31) // 32, B)
    h = fr_pq[:, : k * I // 2].copy().view(np.uint16).reshape(B, k, I)
    h_ref = oracle.moe_gate_up(rows_bf16, routes, cmap, B * k, k, d["gate_w"], d["gate_s"], d["up_w"], d["up_s"], 7.0)
    ok, worst, exact = bf16_close(h, h_ref, atol=moe_gate_up_atol(rows_bf16, routes, d["gate_w"], d["gate_s"], d["up_w"], d["up_s"], 7.0), name="prequant gate_up")
    assert ok and exact > 0.9, (worst, exact)
