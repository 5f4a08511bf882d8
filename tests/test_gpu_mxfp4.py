"""GPU parity: activation quantization (a2), raw MXFP4 GEMV, MXFP4 expert
gate_up/down (a3/a4), route compaction (a7), combine (a8), all through the
C ABI, against the CPU oracle."""
import numpy as np
import pytest

import oracle
from nerve_amd import workloads as wl
from nerve_amd.hip import NerveHipError, check_specialization
from nerve_amd.moe import ExpertBank, address_record, down_spec, gate_up_spec, u32_tensor

from bounds import moe_down_atol, moe_gate_up_atol
from helpers import bf16_close, rel_err_normwise, to_dev, to_np

pytestmark = pytest.mark.gpu


def _torch():
    import torch

    return torch


@pytest.mark.parametrize("cols", [128, 2880, 4096, 96])
@pytest.mark.parametrize("pow2", [True, False])
def test_quantize_bit_exact(ctx, dev, cols, pow2):
    torch = _torch()
    rng = np.random.default_rng(cols + pow2)
    rows = 7
    x = rng.standard_normal((rows, cols)).astype(np.float32) * rng.uniform(1e-3, 50, (rows, 1)).astype(np.float32)
    x[0, :40] = 0.0  # zero-amax block edge
    x[1, 5] = 3e4
    xb = wl.f32_to_bf16_bits(x)
    xb[2, :] = 0  # all-zero row -> floor scale
    nblk = (cols + 127) // 128
    q = torch.zeros(rows, cols, dtype=torch.uint8, device=dev)
    s = torch.zeros(rows, nblk, dtype=torch.float32, device=dev)
    spec = f"quantize_fp8_e4m3{'_spow2' if pow2 else ''}_b128_h{cols}.comp"
    ctx.quantize_fp8_e4m3(spec, to_dev(xb, dev), rows, q, s)
    qr, sr = oracle.quantize_blocks(xb, pow2)
    assert np.array_equal(to_np(q, np.uint8), qr)
    assert np.array_equal(to_np(s, np.float32).view(np.uint32), sr.view(np.uint32))


def _gemv(ctx, dev, q, s, W, S):
    torch = _torch()
    M, K = q.shape
    N = W.shape[0]
    y = torch.zeros(M, N, dtype=torch.float32, device=dev)
    ctx.mxfp4_gemv(to_dev(q, dev), to_dev(s, dev), M, K, to_dev(W, dev), to_dev(S, dev), N, y)
    return to_np(y, np.float32)


def test_gemv_config0_parity(ctx, dev):
    d = wl.config0()
    q, s = oracle.quantize_blocks(d["x_bf16"], pow2=True)
    y = _gemv(ctx, dev, q, s, d["W"], d["S"])
    ref = oracle.mxfp4_gemv(q, s, d["W"], d["S"])
    assert rel_err_normwise(y, ref) <= 1e-3


@pytest.mark.parametrize("M,K,N", [(1, 128, 16), (4, 256, 64), (16, 2880, 256), (33, 4096, 128), (64, 160, 32),
                                   # rows per block sized to one block per CU: 24 rows with a 16-row
                                   # last block, 32 rows
                                   (3, 2880, 5776), (1, 1024, 7168)])
def test_gemv_shapes(ctx, dev, M, K, N):
    rng = np.random.default_rng(M * K + N)
    W, S = wl.mxfp4_matrix(rng, N, K, 118, 130)
    x = wl.bf16_normal(rng, (M, K))
    q, s = oracle.quantize_blocks(x, pow2=True)
    y = _gemv(ctx, dev, q, s, W, S)
    ideal = oracle.mxfp4_gemv_f64(q, s, W, S)
    ref = oracle.mxfp4_gemv(q, s, W, S)
    assert rel_err_normwise(y, ref) <= 1e-3
    assert rel_err_normwise(y, ideal) <= 1e-3


# --------------------------------------------------------------------------
# MoE chain helpers
# --------------------------------------------------------------------------

class MoeRig:
    """Device buffers of one gate_up -> down -> reduce run in package layouts."""

    def __init__(self, dev, d, routes_np):
        torch = _torch()
        self.dev = dev
        self.B, self.k = routes_np.shape
        self.E, self.I, _ = d["gate_w"].shape
        self.H = d["down_w"].shape[1]
        self.d = d
        self.bank = ExpertBank(*(to_dev(d[n], dev) for n in ("gate_w", "gate_s", "up_w", "up_s", "down_w", "down_s")))
        self.routes = to_dev(routes_np.astype(np.uint32), dev)
        self.frame_words = self.k * self.I // 2 + self.k
        self.inter = torch.zeros(self.B * self.frame_words, dtype=torch.int32, device=dev)
        self.control = to_dev(np.array([self.B, 0, 0, 0, 0, 0, 0, 0], np.uint32), dev)
        self.expert_out = torch.zeros(self.B, self.k, self.H, dtype=torch.int16, device=dev)
        self.out = torch.zeros(self.B, self.H, dtype=torch.int16, device=dev)
        self.gu = gate_up_spec(self.H, self.I, self.E, self.k, d.get("limit", 7.0))
        self.dn = down_spec(self.H, self.I, self.E, self.k)

    def frames_np(self):
        return to_np(self.inter, np.uint32).reshape(self.B, self.frame_words)

    def h_np(self):
        fr = self.frames_np()[:, : self.k * self.I // 2].copy()
        return fr.view(np.uint16).reshape(self.B, self.k, self.I)

    def map_np(self):
        return self.frames_np()[:, self.k * self.I // 2:].reshape(-1)

    def run(self, ctx, hidden_np, addresses=None, gate_slots=None, down_slots=None):
        hidden = to_dev(hidden_np, self.dev)
        bank = self.bank
        ctx.moe_route_compact(self.gu, self.routes, self.inter, self.control, self.B)
        ctx.mxfp4_moe_gate_up(self.gu, hidden, None, self.routes, self.inter,
                              bank.addresses if addresses is None else addresses,
                              bank.gate_slots if gate_slots is None else gate_slots, self.control, self.B)
        ctx.moe_route_compact(self.dn, self.routes, None, self.control, self.B)
        ctx.mxfp4_moe_down(self.dn, self.inter, self.routes, self.expert_out,
                           bank.addresses if addresses is None else addresses,
                           bank.down_slots if down_slots is None else down_slots, self.control, self.B)
        ctx.moe_reduce(self.expert_out, self.out, self.B, self.H, self.k, 1.0)


def _route_words(experts: np.ndarray, weights: np.ndarray) -> np.ndarray:
    return ((wl.f32_to_bf16_bits(weights).astype(np.uint32) << np.uint32(16)) | experts.astype(np.uint32))


def test_known_answers_mxfp4_tests_rs(ctx, dev):
    """runtime-rs/src/vulkan_compute/mxfp4_tests.rs:67-216: H = I = 128, all
    nibbles 0x22 (1.0), scale byte 120 (2^-7), hidden 1.0, route weight 1.0."""
    torch = _torch()
    W = 128
    d = dict(gate_w=np.full((1, W, W // 2), 0x22, np.uint8), gate_s=np.full((1, W, W // 32), 120, np.uint8),
             up_w=np.full((1, W, W // 2), 0x22, np.uint8), up_s=np.full((1, W, W // 32), 120, np.uint8),
             down_w=np.full((1, W, W // 2), 0x22, np.uint8), down_s=np.full((1, W, W // 32), 120, np.uint8),
             limit=10.0)
    routes = _route_words(np.zeros((1, 1)), np.ones((1, 1), np.float32))
    rig = MoeRig(dev, d, routes)
    hidden = np.full((1, W), 0x3F80, np.uint16)
    rig.run(ctx, hidden)
    expected = int(wl.f32_to_bf16_bits(np.float32(1.0) / (np.float32(1.0) + np.exp(np.float32(-1.0)))))
    assert expected == 0x3F3B
    assert np.all(rig.h_np() == expected)
    # down with intermediate 1.0 -> 1.0 per code; every e2m1 code reproduces its value
    fr = rig.frames_np()
    fr[:, : W // 2] = 0x3F803F80
    values = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, 0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]
    for nib, val in enumerate(values):
        rig.bank.down_w.fill_(nib | (nib << 4))
        rig.inter.copy_(to_dev(fr.reshape(-1), dev))
        ctx.moe_route_compact(rig.dn, rig.routes, None, rig.control, 1)
        ctx.mxfp4_moe_down(rig.dn, rig.inter, rig.routes, rig.expert_out, rig.bank.addresses, rig.bank.down_slots,
                           rig.control, 1)
        got = to_np(rig.expert_out, np.uint16)
        assert np.all(got == wl.f32_to_bf16_bits(np.float32(val))), (nib, got[0, 0, :4])


def _moe_case(E, k, B, H, I, seed):
    rng = np.random.default_rng(seed)
    d = wl.moe_experts(rng, E, H, I)
    d["limit"] = 7.0
    logits = wl.bf16_normal(rng, (B, E))
    routes, _ = oracle.topk(logits, k)
    hidden = wl.bf16_normal(rng, (B, H))
    return d, routes, hidden


@pytest.mark.parametrize("E,k,B,H,I", [(8, 2, 4, 256, 256), (4, 4, 3, 160, 96), (32, 4, 16, 2880, 2880),
                                       (16, 1, 40, 512, 384),
                                       # streaming kernel at a second shape (K >= 512 on both stages)
                                       (8, 2, 6, 1024, 512), (12, 3, 9, 4096, 1024),
                                       # >= 512 routes: the LDS-staged grouped GEMM path
                                       (16, 4, 160, 512, 384), (8, 2, 300, 2880, 160), (64, 8, 70, 224, 288),
                                       # grouped GEMM at K = 1344 / 1408 (below the persistent kernel's 7 chunks)
                                       (16, 4, 140, 1344, 1408),
                                       # persistent grouped GEMM on both stages: K tails of 64 / 128 and
                                       # 32 / 32 bytes, partial row blocks, experts with several 128-route tiles
                                       (16, 4, 140, 1856, 1664), (4, 2, 300, 1856, 1664), (8, 2, 280, 2080, 1568)])
def test_moe_chain_parity(ctx, dev, E, k, B, H, I):
    d, routes, hidden = _moe_case(E, k, B, H, I, seed=E * 100 + B)
    rig = MoeRig(dev, d, routes)
    rig.run(ctx, hidden)
    cmap, ctl = oracle.route_compact(routes, k, (I + 31) // 32, B)
    assert np.array_equal(rig.map_np(), cmap)
    ctl_gpu = to_np(rig.control, np.uint32)[:7]
    # after the down-stage count the dispatch geometry is the down projection's
    _, ctl_down = oracle.route_compact(routes, k, (H + 63) // 64, B)
    assert np.array_equal(ctl_gpu, ctl_down)
    h_ref = oracle.moe_gate_up(hidden, routes, cmap, B * k, k, d["gate_w"], d["gate_s"], d["up_w"], d["up_s"], 7.0)
    ok, worst, exact = bf16_close(rig.h_np(), h_ref, atol=moe_gate_up_atol(hidden, routes, d["gate_w"], d["gate_s"], d["up_w"], d["up_s"], 7.0), name="mxfp4 gate_up")
    assert ok and exact > 0.9, (worst, exact)
    # down on the GPU's own h (isolates a4 from a3 rounding differences)
    eo_ref = oracle.moe_down(rig.h_np(), routes, cmap, B * k, d["down_w"], d["down_s"])
    ok, worst, exact = bf16_close(to_np(rig.expert_out, np.uint16), eo_ref,
                                  atol=moe_down_atol(rig.h_np(), routes, d["down_w"], d["down_s"]), name="mxfp4 down")
    assert ok and exact > 0.9, (worst, exact)
    out_ref = oracle.moe_reduce(to_np(rig.expert_out, np.uint16), 1.0)
    assert np.array_equal(to_np(rig.out, np.uint16), out_ref)
    # End to end against the oracle chain.  A one-ulp bf16 difference in h can
    # move its e4m3 re-quantization in the down stage by one e4m3 step (~6%),
    # so the composed chain is held to the bf16 tolerance normwise; each stage
    # above is held to it elementwise.
    eo_chain = oracle.moe_down(h_ref, routes, cmap, B * k, d["down_w"], d["down_s"])
    out_chain = wl.bf16_bits_to_f32(oracle.moe_reduce(eo_chain, 1.0))
    assert rel_err_normwise(wl.bf16_bits_to_f32(to_np(rig.out, np.uint16)), out_chain) <= 2e-2


@pytest.mark.parametrize("counts", [(1, 32, 33, 64, 65, 128, 129, 260), (200, 300, 3, 17, 0, 45, 60, 91)])
def test_prefill_route_count_groups(ctx, dev, counts):
    """Persistent grouped GEMM: experts on both sides of the 32- and 64-route
    group boundaries, several 128-route tiles (with a short last tile) and an
    expert without routes, against the oracle on both stages."""
    E, k, H, I = 8, 2, 1856, 1664
    rng = np.random.default_rng(sum(counts))
    ex = np.repeat(np.arange(E), counts)
    rng.shuffle(ex)
    B = len(ex) // k
    assert B * k == len(ex) and B * k >= 512
    d = wl.moe_experts(rng, E, H, I)
    d["limit"] = 7.0
    routes = _route_words(ex.reshape(B, k), rng.uniform(0.05, 1.0, (B, k)).astype(np.float32))
    hidden = wl.bf16_normal(rng, (B, H))
    rig = MoeRig(dev, d, routes)
    rig.run(ctx, hidden)
    cmap, _ = oracle.route_compact(routes, k, (I + 31) // 32, B)
    h_ref = oracle.moe_gate_up(hidden, routes, cmap, B * k, k, d["gate_w"], d["gate_s"], d["up_w"], d["up_s"], 7.0)
    ok, worst, exact = bf16_close(rig.h_np(), h_ref, atol=moe_gate_up_atol(hidden, routes, d["gate_w"], d["gate_s"], d["up_w"], d["up_s"], 7.0), name="prefill gate_up")
    assert ok and exact > 0.9, (worst, exact)
    eo_ref = oracle.moe_down(rig.h_np(), routes, cmap, B * k, d["down_w"], d["down_s"])
    ok, worst, exact = bf16_close(to_np(rig.expert_out, np.uint16), eo_ref,
                                  atol=moe_down_atol(rig.h_np(), routes, d["down_w"], d["down_s"]), name="prefill down")
    assert ok and exact > 0.9, (worst, exact)


# H = 128: the span kernels; H = 512: the token-form gate_up kernel and the
# streaming down kernel.
@pytest.mark.parametrize("H,I", [(128, 128), (512, 256)])
def test_fail_closed_invalid_metadata(ctx, dev, H, I):
    """mxfp4_tests.rs:218-315: invalid expert ids, unbound slots, non-resident
    records, zero generation and short byte counts write nothing."""
    torch = _torch()
    E, k, B = 4, 2, 2
    d, _, hidden = _moe_case(E, k, B, H, I, seed=7)
    # token 0: expert 0 (valid) and expert 9 (>= E); token 1: expert 1 (to be
    # invalidated) and expert 2 (valid)
    routes = _route_words(np.array([[0, 9], [1, 2]]), np.full((2, 2), 0.5, np.float32))
    rig = MoeRig(dev, d, routes)
    bad = np.array(rig.bank.records, np.uint64).reshape(-1, 8)
    e_bad = 1
    gslots = to_np(rig.bank.gate_slots, np.uint32).copy()
    dslots = to_np(rig.bank.down_slots, np.uint32).copy()
    cases = []
    r1 = bad.copy(); r1[gslots[e_bad * 4 + 0], 6] = 0; cases.append(("non-resident", r1, gslots, dslots))
    r2 = bad.copy(); r2[gslots[e_bad * 4 + 1], 4:6] = 0; cases.append(("zero generation", r2, gslots, dslots))
    r3 = bad.copy(); r3[gslots[e_bad * 4 + 2], 2] -= 1; cases.append(("short byte count", r3, gslots, dslots))
    g4 = gslots.copy(); g4[e_bad * 4 + 3] = 0xFFFFFFFF; cases.append(("unbound slot", bad, g4, dslots))
    g5 = gslots.copy(); g5[e_bad * 4 + 0] = 10_000; cases.append(("slot out of table", bad, g5, dslots))
    for name, rec, gs_, ds_ in cases:
        rig.inter.fill_(0x7F7F7F7F)  # sentinel bf16 pair
        rig.run(ctx, hidden, addresses=u32_tensor(rec.reshape(-1), dev), gate_slots=u32_tensor(gs_, dev),
                down_slots=u32_tensor(ds_, dev))
        h = rig.h_np()
        sentinel = np.uint16(0x7F7F)
        assert np.all(h[0, 1] == sentinel), name           # invalid expert id
        assert np.all(h[1, 0] == sentinel), name           # invalidated expert record
        assert not np.any(h[0, 0] == sentinel), name       # valid routes still computed
        assert not np.any(h[1, 1] == sentinel), name
    # A record table that is 4-byte but not 16-byte aligned is refused before
    # any launch (records are read as 16-byte pieces).
    flat = np.concatenate([np.zeros(1, np.uint32), bad.reshape(-1).astype(np.uint32)])
    shifted = u32_tensor(flat, dev)[1:]
    assert shifted.data_ptr() % 16 == 4
    with pytest.raises(NerveHipError):
        rig.run(ctx, hidden, addresses=shifted)


# E <= 64: the token-form gate_up kernel; E = 80: the streaming kernel's tiles.
@pytest.mark.parametrize("E", [8, 80])
def test_gate_up_repeated_expert_in_a_token(ctx, dev, E):
    """A token may list one expert in several slots (top-k padding of an
    all-NaN row repeats expert 0): every such route gets its own frame."""
    k, B, H, I = 3, 5, 512, 256
    d, _, hidden = _moe_case(E, k, B, H, I, seed=31 + E)
    ex = np.array([[0, 0, 3], [1, 2, 0], [5, 5, 5], [7, 1, 0], [2, 3, 4]])
    routes = _route_words(ex, np.full((B, k), 0.25, np.float32))
    rig = MoeRig(dev, d, routes)
    rig.run(ctx, hidden)
    cmap, _ = oracle.route_compact(routes, k, (I + 31) // 32, B)
    h_ref = oracle.moe_gate_up(hidden, routes, cmap, B * k, k, d["gate_w"], d["gate_s"], d["up_w"], d["up_s"], 7.0)
    ok, worst, exact = bf16_close(rig.h_np(), h_ref, atol=moe_gate_up_atol(hidden, routes, d["gate_w"], d["gate_s"], d["up_w"], d["up_s"], 7.0), name="gate_up repeated expert")
    assert ok and exact > 0.9, (worst, exact)
    h = rig.h_np()
    assert np.array_equal(h[0, 0], h[0, 1]) and np.array_equal(h[2, 0], h[2, 2])


@pytest.mark.parametrize("E,start,count", [(32, 8, 12), (80, 30, 40)])
def test_owned_expert_range_gate_up_down(ctx, dev, E, start, count):
    """Expert-parallel ownership (BatchControl expert_start/expert_count,
    moe_route_compact_batch1.comp.template:27-59): only routes of owned
    experts are computed; every other frame and output row is left as it was."""
    k, B, H, I = 4, 16, 512, 256
    d, routes, hidden = _moe_case(E, k, B, H, I, seed=E + start)
    rig = MoeRig(dev, d, routes)
    rig.control = to_dev(np.array([B, start, count, 0, 0, 0, 0, 0], np.uint32), dev)
    rig.inter.fill_(0x7F7F7F7F)
    rig.expert_out.fill_(0x7F7F)
    rig.run(ctx, hidden)
    cmap, ctl = oracle.route_compact(routes, k, (I + 31) // 32, B, start, count)
    n = int(ctl[3])
    assert 0 < n < B * k
    sentinel_h = np.full((B, k, I), 0x7F7F, np.uint16)
    h_ref = oracle.moe_gate_up(hidden, routes, cmap, n, k, d["gate_w"], d["gate_s"], d["up_w"], d["up_s"], 7.0,
                               inter=sentinel_h)
    owned = ((routes & 0xFFFF) >= start) & ((routes & 0xFFFF) < start + count)
    h = rig.h_np()
    assert np.all(h[~owned] == 0x7F7F)
    ok, worst, exact = bf16_close(h[owned], h_ref[owned],       # compared on owned routes only
                                  atol=moe_gate_up_atol(hidden, routes, d["gate_w"], d["gate_s"], d["up_w"], d["up_s"], 7.0)[owned], name="owned gate_up")
    assert ok and exact > 0.9, (worst, exact)
    eo_ref = oracle.moe_down(h, routes, cmap, n, d["down_w"], d["down_s"], out=np.full((B, k, H), 0x7F7F, np.uint16))
    eo = to_np(rig.expert_out, np.uint16)
    assert np.all(eo[~owned] == 0x7F7F)
    ok, worst, exact = bf16_close(eo[owned], eo_ref[owned],
                                  atol=moe_down_atol(h, routes, d["down_w"], d["down_s"])[owned], name="owned down")
    assert ok and exact > 0.9, (worst, exact)


# Decode token/stream path, owned expert ranges and a prefill-sized batch
# (the grouped path, where the count is its own launch).
@pytest.mark.parametrize("E,k,B,H,I,start,count", [(32, 4, 16, 2880, 2880, 0, 0), (32, 4, 16, 512, 256, 8, 12),
                                                   (8, 2, 4, 256, 256, 2, 3), (8, 4, 160, 256, 256, 0, 0)])
def test_down_counted_matches_count_then_down(ctx, dev, E, k, B, H, I, start, count):
    """nerve_hip_mxfp4_moe_down_counted == moe_route_compact (count form) then
    mxfp4_moe_down: the same expert outputs and the same control words."""
    d, routes, hidden = _moe_case(E, k, B, H, I, seed=B + E + start)
    rig = MoeRig(dev, d, routes)
    rig.control = to_dev(np.array([B, start, count, 0, 0, 0, 0, 0], np.uint32), dev)
    rig.run(ctx, hidden)
    ref_ctl = to_np(rig.control, np.uint32).copy()
    ref_eo = to_np(rig.expert_out, np.uint16).copy()
    rig.expert_out.fill_(0x7F7F)
    rig.control = to_dev(np.array([B, start, count, 0, 0, 0, 0, 0], np.uint32), dev)
    ctx.moe_route_compact(rig.gu, rig.routes, rig.inter, rig.control, B)
    ctx.mxfp4_moe_gate_up(rig.gu, to_dev(hidden, dev), None, rig.routes, rig.inter, rig.bank.addresses,
                          rig.bank.gate_slots, rig.control, B)
    ctx.mxfp4_moe_down_counted(rig.dn, rig.inter, rig.routes, rig.expert_out, rig.bank.addresses,
                               rig.bank.down_slots, rig.control, B)
    assert np.array_equal(to_np(rig.control, np.uint32), ref_ctl)
    if count:
        owned = ((routes & 0xFFFF) >= start) & ((routes & 0xFFFF) < start + count)
        assert np.array_equal(to_np(rig.expert_out, np.uint16)[owned], ref_eo[owned])
    else:
        assert np.array_equal(to_np(rig.expert_out, np.uint16), ref_eo)


def _block_major(w, s):
    """Row-major down parameters -> input_block_major_b128 (W [E, I/128, H,
    64], S [E, I/128, H, 4]): byte (row r, packed column j) goes to
    ((j / 64) H + r) 64 + j % 64, scale byte (r, group q) to ((q / 4) H + r) 4
    + q % 4 (independent_sparse_moe_down_batch1_mxfp4.comp.template:229-233,
    :260-263)."""
    E, H, RB = w.shape
    wb = np.ascontiguousarray(w.reshape(E, H, RB // 64, 64).transpose(0, 2, 1, 3))
    sb = np.ascontiguousarray(s.reshape(E, H, RB // 64, 4).transpose(0, 2, 1, 3))
    return wb, sb


@pytest.mark.parametrize("E,k,B,H,I,start,count", [(8, 4, 16, 512, 256, 0, 0), (32, 4, 16, 2880, 2816, 0, 0),
                                                   (32, 4, 16, 384, 512, 4, 20), (8, 4, 3, 160, 256, 0, 0)])
def test_down_input_block_major(ctx, dev, E, k, B, H, I, start, count):
    """input_block_major_b128 down weights give the row-major result bit for
    bit (the same products, only the addresses differ), and match the oracle
    on the row-major copy; prefill-sized batches are refused."""
    d, routes, hidden = _moe_case(E, k, B, H, I, seed=H + I + start)
    rig = MoeRig(dev, d, routes)
    rig.control = to_dev(np.array([B, start, count, 0, 0, 0, 0, 0], np.uint32), dev)
    rig.run(ctx, hidden)
    ref_eo = to_np(rig.expert_out, np.uint16).copy()
    wb, sb = _block_major(d["down_w"], d["down_s"])
    bank = ExpertBank(rig.bank.gate_w, rig.bank.gate_s, rig.bank.up_w, rig.bank.up_s, to_dev(wb, dev), to_dev(sb, dev))
    spec = rig.dn.replace("_mxfp4_e2m1", "_input_block_major_b128_mxfp4_e2m1")
    assert check_specialization(spec) == 0
    rig.expert_out.fill_(0x7F7F)
    ctx.mxfp4_moe_down(spec, rig.inter, rig.routes, rig.expert_out, bank.addresses, bank.down_slots, rig.control, B)
    eo = to_np(rig.expert_out, np.uint16)
    owned = np.ones(routes.shape, bool) if not count else \
        ((routes & 0xFFFF) >= start) & ((routes & 0xFFFF) < start + count)
    assert np.array_equal(eo[owned], ref_eo[owned])
    cmap, ctl = oracle.route_compact(routes, k, (H + 63) // 64, B, start, count)
    eo_ref = oracle.moe_down(rig.h_np(), routes, cmap, int(ctl[3]), d["down_w"], d["down_s"])
    ok, worst, exact = bf16_close(eo[owned], eo_ref[owned],
                                  atol=moe_down_atol(rig.h_np(), routes, d["down_w"], d["down_s"])[owned],
                                  name="block-major down")
    assert ok and exact > 0.9, (worst, exact)


def test_down_input_block_major_prefill(ctx, dev):
    """Prefill-sized batches with block-major down weights take the
    register-fed kernel after the preparation launch; they match the
    row-major result within bf16 tolerance (another accumulation order)."""
    E, k, B, H, I = 8, 4, 160, 256, 256
    d, routes, hidden = _moe_case(E, k, B, H, I, seed=7)
    rig = MoeRig(dev, d, routes)
    rig.run(ctx, hidden)
    ref_eo = to_np(rig.expert_out, np.uint16).copy()
    wb, sb = _block_major(d["down_w"], d["down_s"])
    bank = ExpertBank(rig.bank.gate_w, rig.bank.gate_s, rig.bank.up_w, rig.bank.up_s, to_dev(wb, dev), to_dev(sb, dev))
    spec = rig.dn.replace("_mxfp4_e2m1", "_input_block_major_b128_mxfp4_e2m1")
    rig.expert_out.fill_(0x7F7F)
    ctx.moe_route_compact(rig.dn, rig.routes, None, rig.control, B)
    ctx.mxfp4_moe_down(spec, rig.inter, rig.routes, rig.expert_out, bank.addresses, bank.down_slots, rig.control, B)
    # two GPU sum orders, each within the bound of the exact sum
    ok, worst, exact = bf16_close(to_np(rig.expert_out, np.uint16), ref_eo,
                                  atol=2 * moe_down_atol(rig.h_np(), routes, d["down_w"], d["down_s"]),
                                  name="block-major prefill down")
    assert ok and exact > 0.9, (worst, exact)


_E2M1_E4M3 = np.array([0x00, 0x30, 0x38, 0x3C, 0x40, 0x44, 0x48, 0x4C], np.uint8)


def _expand_e4m3(w):
    """Compact MXFP4 bytes [..., K/2] -> the e4m3 bytes [..., K] of the same
    values (mxfp4_e4m3_bits, …gate_up_batch1_mxfp4.comp.template:246-248)."""
    lo, hi = w & 0x0F, w >> 4
    out = np.empty(w.shape[:-1] + (2 * w.shape[-1],), np.uint8)
    out[..., 0::2] = _E2M1_E4M3[lo & 7] | ((lo & 8) << 4)
    out[..., 1::2] = _E2M1_E4M3[hi & 7] | ((hi & 8) << 4)
    return out


def _bank_tables(dev, per_expert):
    """Address table and slots from per-expert (tensor, representation)
    lists: gate_up slots (gw, gs, uw, us) and down slots (dw, ds)."""
    recs, gate_slots, down_slots = [], [], []
    keep = []
    for gate, down in per_expert:
        for tt, rep in gate:
            gate_slots.append(len(recs) // 8)
            recs += address_record(tt, representation=rep)
            keep.append(tt)
        for tt, rep in down:
            down_slots.append(len(recs) // 8)
            recs += address_record(tt, representation=rep)
            keep.append(tt)
    return u32_tensor(recs, dev), u32_tensor(gate_slots, dev), u32_tensor(down_slots, dev), keep


@pytest.mark.parametrize("mode", ["resident", "adaptive", "native"])
@pytest.mark.parametrize("E,k,B,H,I", [(8, 4, 16, 512, 256), (8, 2, 40, 384, 640), (32, 4, 16, 2880, 2880)])
def test_e4m3_expert_banks(ctx, dev, mode, E, k, B, H, I):
    """Resident / adaptive pre-expanded MXFP4 and native FP8 experts
    (…gate_up_batch1_mxfp4.comp.template:173-229, :299-355): the same values
    as a compact bank give the compact bank's outputs.  Native experts get
    128 x 128 scale blocks (the compact twin repeats each block's scale) and
    one all-zero scale block, whose weights count as zero (the compact twin
    has zero codes there)."""
    d, routes, hidden = _moe_case(E, k, B, H, I, seed=E + B + H + len(mode))
    nf = E // 2 if mode == "native" else E
    orig = {n: d[n].copy() for n in ("gate_w", "up_w", "down_w")}   # native weights keep the zero-scale block's codes
    if mode == "native":
        for wn, sn, R, C in (("gate_w", "gate_s", I, H), ("up_w", "up_s", I, H), ("down_w", "down_s", H, I)):
            s = d[sn].reshape(E, R, C // 32)
            for e in range(nf, E):
                blk = s[e, ::128, ::4][:, :(C + 127) // 128].copy()                  # [ceil(R/128), ceil(C/128)]
                s[e] = np.repeat(np.repeat(blk, 128, 0)[:R], 4, 1)[:, :C // 32]
            d[wn][nf, :128, :64] = 0                                                  # the zero-scale block
    rig = MoeRig(dev, d, routes)
    rig.run(ctx, hidden)
    ref_h, ref_eo = rig.h_np().copy(), to_np(rig.expert_out, np.uint16).copy()

    exp = {n: to_dev(_expand_e4m3(orig[n] if mode == "native" else d[n]), dev) for n in ("gate_w", "up_w", "down_w")}
    comp = {n: to_dev(d[n], dev) for n in ("gate_w", "up_w", "down_w", "gate_s", "up_s", "down_s")}
    nat_s = {}
    if mode == "native":
        for sn, R, C in (("gate_s", I, H), ("up_s", I, H), ("down_s", H, I)):
            s = d[sn].reshape(E, R, C // 32)
            blk = np.ascontiguousarray(s[:, ::128, ::4][:, :, :(C + 127) // 128])
            blk[nf, 0, 0] = 0
            nat_s[sn] = to_dev(blk, dev)
    per_expert = []
    for e in range(E):
        if mode == "native" and e >= nf:
            g = [(exp["gate_w"][e], 0), (nat_s["gate_s"][e], 0), (exp["up_w"][e], 0), (nat_s["up_s"][e], 0)]
            dn = [(exp["down_w"][e], 0), (nat_s["down_s"][e], 0)]
        elif mode == "resident" or (mode == "adaptive" and e % 2 == 1):
            rep = 1 if mode == "adaptive" else 0
            g = [(exp["gate_w"][e], rep), (comp["gate_s"][e], 0), (exp["up_w"][e], rep), (comp["up_s"][e], 0)]
            dn = [(exp["down_w"][e], rep), (comp["down_s"][e], 0)]
        else:
            g = [(comp["gate_w"][e], 0), (comp["gate_s"][e], 0), (comp["up_w"][e], 0), (comp["up_s"][e], 0)]
            dn = [(comp["down_w"][e], 0), (comp["down_s"][e], 0)]
        per_expert.append((g, dn))
    addresses, gate_slots, down_slots, _keep = _bank_tables(dev, per_expert)
    tok = {"resident": "_resident_fp8_e4m3", "adaptive": "_adaptive_fp8_e4m3", "native": ""}[mode]
    nat = f"_native_fp8_e4m3_se8m0_b128_nf{nf}" if mode == "native" else ""
    gu = rig.gu.replace("_mxfp4_e2m1_g32_", f"_mxfp4_e2m1{tok}_g32{nat}_")
    dn = rig.dn.replace("_mxfp4_e2m1_g32_", f"_mxfp4_e2m1{tok}_g32{nat}_")
    assert check_specialization(gu) == 0 and check_specialization(dn) == 0
    hidden_d = to_dev(hidden, dev)
    rig.inter.zero_()
    rig.expert_out.fill_(0x7F7F)
    ctx.moe_route_compact(rig.gu, rig.routes, rig.inter, rig.control, B)
    ctx.mxfp4_moe_gate_up(gu, hidden_d, None, rig.routes, rig.inter, addresses, gate_slots, rig.control, B)
    h = rig.h_np()
    # against the compact bank's GPU result: two sum orders, each within the bound
    ok, worst, exact = bf16_close(h, ref_h, atol=2 * moe_gate_up_atol(hidden, routes, d["gate_w"], d["gate_s"],
                                                                     d["up_w"], d["up_s"], 7.0), name="e4m3 bank gate_up")
    assert ok and exact > 0.97, (worst, exact)
    # down from the reference h, so its check does not inherit gate_up's rounding
    fr = rig.frames_np().copy()
    fr[:, : k * I // 2] = ref_h.reshape(B, k * I).view(np.uint32).reshape(B, k * I // 2)
    rig.inter.copy_(to_dev(fr.reshape(-1).view(np.int32), dev))
    ctx.moe_route_compact(rig.dn, rig.routes, None, rig.control, B)
    ctx.mxfp4_moe_down(dn, rig.inter, rig.routes, rig.expert_out, addresses, down_slots, rig.control, B)
    ok, worst, exact = bf16_close(to_np(rig.expert_out, np.uint16), ref_eo,
                                  atol=2 * moe_down_atol(ref_h, routes, d["down_w"], d["down_s"]), name="e4m3 bank down")
    assert ok and exact > 0.97, (worst, exact)


def test_moe_prefill_config3_subset(ctx, dev):
    """Config 3 (2048 tokens, 128 Zipf-loaded experts, H = I = 2880) on the GPU;
    24 tokens re-computed by the oracle (each token's result depends only on
    its own row and routes)."""
    torch = _torch()
    d = wl.config3()
    B, E, k, H, I = d["B"], d["E"], d["k"], d["H"], d["I"]
    routes, _ = oracle.topk(d["logits"], k, telemetry=False)
    rig = MoeRig(dev, d, routes)
    rig.run(ctx, d["hidden"])
    counts = np.bincount((routes & 0xFFFF).ravel(), minlength=E)
    assert counts.max() > 256 and (counts > 0).sum() > 100      # Zipf skew is present
    sel = np.random.default_rng(0).choice(B, 24, replace=False)
    rs, hs = routes[sel], d["hidden"][sel]
    cm, _ = oracle.route_compact(rs, k, (I + 31) // 32, 24)
    h_ref = oracle.moe_gate_up(hs, rs, cm, 24 * k, k, d["gate_w"], d["gate_s"], d["up_w"], d["up_s"], 7.0)
    h = rig.h_np()[sel]
    ok, worst, exact = bf16_close(h, h_ref, atol=moe_gate_up_atol(hs, rs, d["gate_w"], d["gate_s"], d["up_w"], d["up_s"], 7.0), name="config3 gate_up")
    assert ok and exact > 0.9, (worst, exact)
    eo_ref = oracle.moe_down(h, rs, cm, 24 * k, d["down_w"], d["down_s"])
    ok, worst, exact = bf16_close(to_np(rig.expert_out, np.uint16)[sel], eo_ref,
                                  atol=moe_down_atol(h, rs, d["down_w"], d["down_s"]), name="config3 down")
    assert ok and exact > 0.9, (worst, exact)
    assert np.array_equal(to_np(rig.out, np.uint16)[sel], oracle.moe_reduce(to_np(rig.expert_out, np.uint16)[sel], 1.0))
