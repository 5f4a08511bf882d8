"""Benchmarks of NERVE's quantized-matmul hot path on one MI355X.

Default workload (the metric's MoE decode block):
32 experts, top-4, hidden = intermediate = 2880, 16 bf16 tokens, MXFP4
gate/up/down experts, SwiGLU limit 7.  One step is one full pass of the
reference node chain (router linear -> top-k -> compact -> gate_up -> count
-> down -> reduce) through libnerve_hip's C ABI with inputs resident in HBM.
Steps alternate between two MoE layers with distinct weights (2 x 423 MB,
beyond the 256 MB Infinity Cache), so weights stream from HBM as they do
when a model runs consecutive layers.

`value` = routed (token, expert) pairs per second.  The line also carries the
prefill block as a sub-object, since the metric names prefill
MXFP4 TFLOPS.  Other workloads (--workload) report their own rate with the
same JSON shape.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

METRIC = "MoE expert tokens/s; decode HBM GB/s + prefill MXFP4 TFLOPS as % of peak"
HBM_PEAK_GBS = 8000.0
MXFP4_PEAK_TFLOPS = 10100.0
FP8_PEAK_TFLOPS = 5000.0
BF16_PEAK_TFLOPS = 2500.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--workload", default="moe_decode",
                   choices=["moe_decode", "moe_prefill", "mxfp4_gemv", "int4_gemv", "int4_moe", "fp8_head",
                            "hbm_copy", "hbm_read"])
    p.add_argument("--summarize-traffic", nargs=4, metavar="DIR",
                   help="FETCH_SIZE and WRITE_SIZE rocprofv3 CSV dirs of a run, then of the hbm_copy run")
    p.add_argument("--m", type=int, default=1, help="batch rows for int4_gemv / int4_moe / fp8_head")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-prefill", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    return p.parse_args()


def to_dev(a, dev):
    import torch

    a = np.ascontiguousarray(a)
    view = {np.dtype(np.uint8): np.uint8, np.dtype(np.uint16): np.int16, np.dtype(np.uint32): np.int32,
            np.dtype(np.float16): np.int16, np.dtype(np.float32): np.float32}[a.dtype]
    return torch.from_numpy(a.view(view).copy()).to(dev)


def event_ms(fn, n, stream):
    """Median duration (ms) of fn() over n calls, each bracketed by HIP events
    on `stream` (the stream the kernels are launched on)."""
    import torch

    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for i in range(n):
        ev[i][0].record(stream)
        fn(i)
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    return float(np.median([a.elapsed_time(b) for a, b in ev]))


def batch_event_ms(fn, n, stream, warmup=5):
    """Average duration (ms) of fn() over n back-to-back calls between one
    pair of HIP events on `stream` (launch latency overlaps the previous
    call, as it does inside a model step)."""
    import torch

    for i in range(warmup):
        fn(i)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for i in range(n):
        fn(i)
    b.record(stream)
    torch.cuda.synchronize()
    return float(a.elapsed_time(b)) / n


def graph_event_ms(fn, n, reps=10):
    """Average duration (ms) of one fn(i, stream) call, for kernels shorter
    than the host's per-call cost: n calls (i = 0..n-1) are captured once
    into a HIP graph, and `reps` replays run back to back between one pair of
    HIP events on the replaying stream.  fn must launch on the stream it is
    given and must not allocate (one eager call per i runs first, so the
    library's workspace has its final size before the capture)."""
    import torch

    for i in range(n):
        fn(i, torch.cuda.current_stream())
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        s = torch.cuda.current_stream()
        for i in range(n):
            fn(i, s)
    st = torch.cuda.current_stream()
    g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(st)
    for _ in range(reps):
        g.replay()
    b.record(st)
    torch.cuda.synchronize()
    return float(a.elapsed_time(b)) / (n * reps)


def traffic_for(kernel_key):
    """HBM bytes per launch of `kernel_key` from profiles/traffic.json (two
    rocprofv3 --pmc runs, FETCH_SIZE and WRITE_SIZE, each scaled by what the
    counter reads for a copy of known size; see --summarize-traffic), or None."""
    path = os.path.join(HERE, "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
        return float(t["kernels"][kernel_key]["hbm_bytes"])
    except (OSError, KeyError, ValueError):
        return None


def wall_ms(fn, steps, warmup):
    import torch

    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        fn(i)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def base_line(args, value, unit, ms, dtype, config, higher=True):
    return {"metric": METRIC, "value": value, "unit": unit, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": ms, "higher_is_better": higher, "scaling": "weak", "vs_baseline": None, "dtype": dtype,
            "data": "synthetic (seeded, package layouts, random-init weights)", "config": config}


# --------------------------------------------------------------------------
# MoE decode (default)
# --------------------------------------------------------------------------

def moe_decode(args, ctx, dev):
    import torch

    from nerve_amd import workloads as wl
    from nerve_amd.moe import ExpertBank, MoEBlock

    layers, hidden, data = [], [], []
    for layer in range(2):
        d = wl.config2(layer=layer)
        bank = ExpertBank(*(to_dev(d[n], dev) for n in ("gate_w", "gate_s", "up_w", "up_s", "down_w", "down_s")))
        layers.append(MoEBlock(ctx, to_dev(d["router_w"], dev), bank, d["k"], limit=d["limit"]))
        hidden.append(to_dev(d["hidden"], dev))
        data.append(d)
    d = data[0]
    B, E, k, H, I = d["B"], d["E"], d["k"], d["H"], d["I"]
    stream = torch.cuda.current_stream()
    U = []
    for L in range(2):
        layers[L].forward(hidden[L])
        torch.cuda.synchronize()
        r = layers[L].buffers(B)["routes"].cpu().numpy().view(np.uint32)
        U.append(len(np.unique(r & 0xFFFF)))
    mat = I * H // 2 + I * H // 32                 # one MXFP4 matrix + scales
    # gate_up reads the hidden rows as the routing launch quantized them
    # (e4m3 bytes + f32 block scales)
    gate_up_bytes = [u * 2 * mat + B * H + B * ((H + 127) // 128) * 4 + B * k * I * 2 for u in U]
    down_bytes = [u * mat + B * k * I * 2 + B * k * H * 2 for u in U]
    # + router weights, hidden in and block output out, the quantized rows the
    # routing launch writes, the expert outputs the combine reads
    step_bytes = float(np.mean([g + dn + E * H * 2 + 2 * B * H * 2 + B * H + B * ((H + 127) // 128) * 4
                                + B * k * H * 2 for g, dn in zip(gate_up_bytes, down_bytes)]))

    ms = wall_ms(lambda i: layers[i % 2].forward(hidden[i % 2]), args.steps, args.warmup)

    def gate_up(i):
        # the launch MoEBlock.forward makes: the prequantized form on the
        # routing launch's e4m3 rows
        L = layers[i % 2]
        b = L.buffers(B)
        ctx.mxfp4_moe_gate_up(L.gate_up_pq, b["hidden_q"], b["hidden_s"], b["routes"], b["inter"], L.bank.addresses,
                              L.bank.gate_slots, b["control"], B, stream)

    # routes / maps of both layers are in their own buffers already
    gu_ms = batch_event_ms(gate_up, max(100, args.steps), stream)
    achieved = float(np.mean(gate_up_bytes)) / (gu_ms * 1e-3) / 1e9
    out = base_line(args, B * k / (ms * 1e-3), "expert-tokens/s", ms, "e4m3xe2m1->f32",
                    {"workload": "moe_decode_e32_k4_h2880_i2880_b16", "experts": E, "top_k": k, "hidden": H,
                     "intermediate": I, "batch_tokens": B, "layers_rotated": 2, "distinct_experts": U})
    out["tokens_per_s"] = B / (ms * 1e-3)
    out["step_hbm_gbs"] = step_bytes / (ms * 1e-3) / 1e9
    out["step_hbm_frac"] = out["step_hbm_gbs"] / HBM_PEAK_GBS
    out["roofline"] = {"bound": "hbm", "kernel": "mx_tokens_kernel<3, 8> (nerve_hip_mxfp4_moe_gate_up, one launch)",
                       "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                       "traffic": traffic_for("mx_tokens_kernel<3, 8>"),
                       "algorithmic_bytes_per_launch": float(np.mean(gate_up_bytes)), "launch_ms": gu_ms}
    return out, data[0]


# --------------------------------------------------------------------------
# MoE prefill
# --------------------------------------------------------------------------

class Prefill:
    def __init__(self, ctx, dev):
        import torch

        from nerve_amd import workloads as wl
        from nerve_amd.moe import ExpertBank, down_spec, gate_up_spec, topk_spec

        d = wl.config3()
        self.d = d
        B, E, k, H, I = d["B"], d["E"], d["k"], d["H"], d["I"]
        self.ctx = ctx
        self.bank = ExpertBank(*(to_dev(d[n], dev) for n in ("gate_w", "gate_s", "up_w", "up_s", "down_w", "down_s")))
        self.logits = to_dev(d["logits"], dev)
        self.hidden = to_dev(d["hidden"], dev)
        self.routes = torch.zeros(B, k, dtype=torch.int32, device=dev)
        self.inter = torch.zeros(B * (k * I // 2 + k), dtype=torch.int32, device=dev)
        self.control = torch.tensor([B, 0, 0, 0, 0, 0, 0, 0], dtype=torch.int32, device=dev)
        self.eo = torch.zeros(B, k, H, dtype=torch.int16, device=dev)
        self.out = torch.zeros(B, H, dtype=torch.int16, device=dev)
        self.gu, self.dn, self.tk = gate_up_spec(H, I, E, k, 7.0), down_spec(H, I, E, k), topk_spec(E, k)

    def step(self, _i=0, stream=None):
        c, d = self.ctx, self.d
        B, k, H = d["B"], d["k"], d["H"]
        c.moe_router_topk(self.tk, self.logits, None, self.routes, None, B, stream)
        c.moe_route_compact(self.gu, self.routes, self.inter, self.control, B, stream)
        c.mxfp4_moe_gate_up(self.gu, self.hidden, None, self.routes, self.inter, self.bank.addresses,
                            self.bank.gate_slots, self.control, B, stream)
        c.moe_route_compact(self.dn, self.routes, None, self.control, B, stream)
        c.mxfp4_moe_down(self.dn, self.inter, self.routes, self.eo, self.bank.addresses, self.bank.down_slots,
                         self.control, B, stream)
        c.moe_reduce(self.eo, self.out, B, H, k, 1.0, stream)

    def figures(self, ms):
        d = self.d
        B, E, k, H, I = d["B"], d["E"], d["k"], d["H"], d["I"]
        flop = 2.0 * B * k * 3 * H * I
        mat = I * H // 2 + I * H // 32
        hbm = 3 * E * mat + B * H * 2 + 2 * B * k * I * 2 + 2 * B * k * H * 2 + B * H * 2
        # the compulsory minimum: every weight and scale byte once, the hidden
        # rows in and the block output out (the expert-output round trip and
        # the intermediates are not counted)
        compulsory = 3 * E * mat + B * H * 2 + B * H * 2
        tf = flop / (ms * 1e-3) / 1e12
        return {"workload": "moe_prefill_e128_k4_b2048_zipf1.1", "ms": ms, "tflops": tf,
                "mxfp4_peak_frac": tf / MXFP4_PEAK_TFLOPS, "fp8_peak_frac": tf / FP8_PEAK_TFLOPS,
                "hbm_gbs": hbm / (ms * 1e-3) / 1e9, "hbm_frac": hbm / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                "compulsory_bytes": compulsory,
                "hbm_frac_compulsory": compulsory / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                "algorithmic_flop": flop, "algorithmic_bytes": hbm,
                "note": "HBM-bound shape: ~240 FLOP/B is below the MXFP4 ridge, so the MFMA fraction is capped "
                        "near 19% of the MXFP4 peak"}


def prefill_sub(ctx, dev, n=10):
    import torch

    pf = Prefill(ctx, dev)
    stream = torch.cuda.current_stream()
    for _ in range(3):
        pf.step()
    torch.cuda.synchronize()
    ms = event_ms(lambda i: pf.step(i, stream), n, stream)
    return pf.figures(ms)


# --------------------------------------------------------------------------
# single-kernel workloads (configs 0, 1, 4)
# --------------------------------------------------------------------------

def mxfp4_gemv(args, ctx, dev):
    import torch

    from nerve_amd import workloads as wl

    d = wl.config0()
    K, N = 2880, 5760
    nbytes = N * K // 2 + N * K // 32
    copies = -(-512 * 2 ** 20 // nbytes) + 1   # rotate past the Infinity Cache
    W = to_dev(np.tile(d["W"], (copies, 1)), dev).view(copies, N, K // 2)
    S = to_dev(np.tile(d["S"], (copies, 1)), dev).view(copies, N, K // 32)
    x = to_dev(d["x_bf16"], dev)
    q = torch.zeros(1, K, dtype=torch.uint8, device=dev)
    s = torch.zeros(1, (K + 127) // 128, dtype=torch.float32, device=dev)
    y = torch.zeros(1, N, dtype=torch.float32, device=dev)
    ctx.quantize_fp8_e4m3(f"quantize_fp8_e4m3_spow2_b128_h{K}.comp", x, 1, q, s)
    call = lambda i, st: ctx.mxfp4_gemv(q, s, 1, K, W[i % copies], S[i % copies], N, y, st)
    ms = wall_ms(lambda i: call(i, torch.cuda.current_stream()), args.steps, args.warmup)
    # one launch per call, shorter than the host's per-call cost: graph replay
    kms = graph_event_ms(call, copies)
    alg = nbytes + K + 4 * 23 + N * 4
    gbs = alg / (kms * 1e-3) / 1e9
    out = base_line(args, gbs, "GB/s", ms, "e4m3xe2m1->f32",
                    {"workload": "mxfp4_gemv_m1_k2880_n5760", "weight_copies_rotated": copies})
    out["roofline"] = {"bound": "hbm", "kernel": "mx_span_kernel<0,1,2,8>", "achieved": gbs, "peak": HBM_PEAK_GBS,
                       "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS, "traffic": traffic_for("mx_span_kernel<0, 1, 2, 8>"),
                       "algorithmic_bytes_per_launch": alg, "launch_ms": kms}
    return out


def int4_gemv(args, ctx, dev):
    import torch

    from nerve_amd import workloads as wl

    M = args.m
    d = wl.config1(M=M)
    K, N, G = d["K"], d["N"], d["group"]
    nbytes = K * N // 2 + (K // G) * N * 2 + (K // G) * N // 2
    copies = -(-512 * 2 ** 20 // nbytes) + 1
    qw = to_dev(np.tile(d["qweight"], (copies, 1)), dev).view(copies, K // 8, N)
    sc = to_dev(np.tile(d["scales"], (copies, 1)), dev).view(copies, K // G, N)
    qz = to_dev(np.tile(d["qzeros"], (copies, 1)), dev).view(copies, K // G, N // 8)
    x = to_dev(d["x"], dev)
    y = torch.zeros(M, N, dtype=torch.int16, device=dev)
    spec = f"linear_batch16_int4_gptq_sf16_g{G}_{K}x{N}.comp"
    call = lambda i, st: ctx.int4_linear(spec, x, qw[i % copies], sc[i % copies], qz[i % copies], None, y, M, st)
    ms = wall_ms(lambda i: call(i, torch.cuda.current_stream()), args.steps, args.warmup)
    # one launch per call, shorter than the host's per-call cost: graph replay
    kms = graph_event_ms(call, copies)
    alg = nbytes + M * K * 2 + M * N * 2
    gbs = alg / (kms * 1e-3) / 1e9
    out = base_line(args, gbs, "GB/s", ms, "bf16xint4->f32",
                    {"workload": f"int4_gptq_g128_asym_m{M}_k4096_n14336", "weight_copies_rotated": copies})
    kname = ("int4_gptq_gemv_kernel<16, 128, true, 1u>" if M == 1 else "int4_gptq_gemv_kernel<16, 128, true, 4u>"
             if M <= 4 else "int4_gptq_fixed_kernel<16, 4, 4>")
    out["roofline"] = {"bound": "hbm", "kernel": kname, "achieved": gbs, "peak": HBM_PEAK_GBS,
                       "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS, "traffic": traffic_for(kname),
                       "algorithmic_bytes_per_launch": alg, "launch_ms": kms}
    return out


def int4_moe(args, ctx, dev):
    """Sparse INT4-CT experts at the geometry of the reference's compiler test
    (h3072 i1024 e256 k10, g32 bf16 scales): one step = route compaction ->
    gate_up -> count -> down -> reduce for a batch of --m tokens.  The whole
    256-expert bank (1.36 GB) is drawn on the GPU, and every step routes the
    tokens to fresh random experts, so weights stream from HBM."""
    import torch

    from nerve_amd.moe import Int4CtExpertBank, int4_ct_spec

    B, H, I, E, k, G = args.m, 3072, 1024, 256, 10, 32
    g = torch.Generator(device=dev).manual_seed(20260005)

    def words(*shape):
        return torch.randint(-2 ** 31, 2 ** 31 - 1, shape, generator=g, device=dev, dtype=torch.int64).to(torch.int32)

    def scales(*shape):
        return (torch.rand(shape, generator=g, device=dev) * 0.018 + 0.002).to(torch.bfloat16).view(torch.int16)

    bank = Int4CtExpertBank(words(E, 2 * I, H // 8), scales(E, 2 * I, H // G), words(E, H, I // 8),
                            scales(E, H, I // G))
    rng = np.random.default_rng(5)
    R = 64
    sets = np.stack([np.stack([rng.choice(E, size=k, replace=False) for _ in range(B)]) for _ in range(R)])
    wbits = np.uint32(0x3DCC) << np.uint32(16)                       # bf16 0.1
    routes = [to_dev(sets[i].astype(np.uint32) | wbits, dev) for i in range(R)]
    x = (torch.randn(B, H, generator=g, device=dev)).to(torch.bfloat16).view(torch.int16)
    gspec = int4_ct_spec("gate_up", H, I, E, k, G)
    dspec = int4_ct_spec("down", H, I, E, k, G)
    fw = k * I // 2 + k
    inter = torch.zeros(B * fw, dtype=torch.int32, device=dev)
    control = to_dev(np.array([B, 0, 0, 0, 0, 0, 0, 0], np.uint32), dev)
    eo = torch.zeros(B, k, H, dtype=torch.int16, device=dev)
    y = torch.zeros(B, H, dtype=torch.int16, device=dev)

    def step(i, st=None):
        r = routes[i % R]
        ctx.moe_route_compact(gspec, r, inter, control, B, st)
        ctx.int4_moe_gate_up(gspec, x, r, inter, bank.addresses, bank.gate_slots, control, B, st)
        ctx.moe_route_compact(dspec, r, None, control, B, st)
        ctx.int4_moe_down(dspec, inter, r, eo, bank.addresses, bank.down_slots, control, B, st)
        ctx.moe_reduce(eo, y, B, H, k, 1.0, st)

    stream = torch.cuda.current_stream()
    ms = wall_ms(lambda i: step(i, stream), args.steps, args.warmup)
    step_ms = graph_event_ms(step, R)
    for i in range(R):
        ctx.moe_route_compact(gspec, routes[i], inter, control, B, stream)
    gu_ms = graph_event_ms(lambda i, st: ctx.int4_moe_gate_up(gspec, x, routes[i % R], inter, bank.addresses,
                                                              bank.gate_slots, control, B, st), R)
    dn_ms = graph_event_ms(lambda i, st: ctx.int4_moe_down(dspec, inter, routes[i % R], eo, bank.addresses,
                                                           bank.down_slots, control, B, st), R)
    distinct = np.mean([len(np.unique(s)) for s in sets])
    gu_alg = distinct * (2 * I * H // 2 + 2 * I * (H // G) * 2) + B * H * 2 + B * k * I * 2
    dn_alg = distinct * (H * I // 2 + H * (I // G) * 2) + B * k * I * 2 + B * k * H * 2
    gu_gbs = gu_alg / (gu_ms * 1e-3) / 1e9
    dn_gbs = dn_alg / (dn_ms * 1e-3) / 1e9
    out = base_line(args, B * k / (step_ms * 1e-3), "expert-tokens/s", ms, "bf16xint4->f32",
                    {"workload": f"int4_ct_sparse_moe_b{B}_h3072_i1024_e256_k10_g32"})
    out["roofline"] = {"bound": "hbm", "kernel": "sparse_int4_kernel<true, 32, false> (gate_up)", "achieved": gu_gbs,
                       "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": gu_gbs / HBM_PEAK_GBS,
                       "traffic": traffic_for("sparse_int4_kernel<true, 32u, false>"),
                       "algorithmic_bytes_per_launch": gu_alg, "launch_ms": gu_ms}
    out["down"] = {"kernel": "sparse_int4_kernel<false, 32, false>", "hbm_gbs": dn_gbs, "frac": dn_gbs / HBM_PEAK_GBS,
                   "algorithmic_bytes_per_launch": dn_alg, "launch_ms": dn_ms}
    out["step_ms_graph"] = step_ms
    return out


def fp8_head(args, ctx, dev):
    """Weights are drawn on the GPU (N(0,0.02), per-row bf16 amax/448 scale,
    torch's e4m3fn cast): 579 MB exceeds the Infinity Cache on its own."""
    import torch

    M, K, N = args.m, 2880, 201088
    g = torch.Generator(device=dev).manual_seed(20260004)
    W = torch.empty(N, K, dtype=torch.uint8, device=dev)
    sc = torch.empty(N, dtype=torch.float32, device=dev)
    for r0 in range(0, N, 16384):
        wf = torch.randn(min(16384, N - r0), K, generator=g, device=dev) * 0.02
        s = (wf.abs().amax(dim=1) / 448.0).to(torch.bfloat16).float()
        sc[r0:r0 + wf.shape[0]] = s
        W[r0:r0 + wf.shape[0]] = (wf / s[:, None]).to(torch.float8_e4m3fn).view(torch.uint8)
    nblk = (K + 127) // 128
    grid = sc.to(torch.bfloat16).view(torch.int16)[:, None].repeat(1, nblk).contiguous()
    x = (torch.randn(M, K, generator=g, device=dev)).to(torch.bfloat16).view(torch.int16)
    lb = torch.zeros(M, N, dtype=torch.int16, device=dev)
    am = torch.zeros(M, dtype=torch.int32, device=dev)
    spec = f"tied_output_projection_batch4_fp8_e4m3_b1x128_{N}x{K}_scale1_to_f32.comp"
    stream = torch.cuda.current_stream()
    fn = lambda i: ctx.fp8_output_projection(spec, x, W, grid, None, lb, am, M, stream)
    ms = wall_ms(fn, args.steps, args.warmup)
    kms = batch_event_ms(fn, max(50, args.steps), stream)
    alg = N * K + N * nblk * 2 + M * K * 2 + M * N * 2 + M * 4
    flop = 2.0 * M * N * K
    gbs = alg / (kms * 1e-3) / 1e9
    tf = flop / (kms * 1e-3) / 1e12
    out = base_line(args, M / (kms * 1e-3), "tokens/s", ms, "e4m3xe4m3->f32",
                    {"workload": f"fp8_lm_head_m{M}_k2880_n201088_argmax"})
    mfma_bound = M >= 512
    kname = ("fp8_head_stream_kernel<2, 1 or 2> (+ row quantization, argmax of the partials)" if M <= 32
             else "fp8_head_gemm_kernel (+ row quantization, scale scan, argmax of the partials)")
    tkey = ("fp8_head_stream_kernel<2, 1>" if M <= 16 else "fp8_head_stream_kernel<2, 2>" if M <= 32
            else "fp8_head_gemm_kernel<2, 4, 2, 4, 3>" if M <= 64
            else "fp8_head_gemm_kernel<2, 4, 4, 2, 4>" if M <= 128 else "fp8_head_gemm_kernel<4, 2, 4, 4, 3>")
    out["roofline"] = {"bound": "mfma" if mfma_bound else "hbm", "kernel": kname,
                       "achieved": tf if mfma_bound else gbs, "peak": FP8_PEAK_TFLOPS if mfma_bound else HBM_PEAK_GBS,
                       "unit": "TFLOP/s" if mfma_bound else "GB/s",
                       "frac": (tf / FP8_PEAK_TFLOPS) if mfma_bound else (gbs / HBM_PEAK_GBS),
                       "traffic": traffic_for(tkey),
                       "hbm_gbs": gbs, "tflops": tf, "launch_ms": kms}
    return out


def hbm_copy(args, ctx, dev):
    """Calibration workload for the HBM traffic counters: a device-to-device
    copy of 512 MiB (read 512 MiB, write 512 MiB per launch)."""
    import torch

    n = 512 * 2 ** 20
    src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(7)
    dst = torch.empty(n, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream()
    fn = lambda i: dst.copy_(src)
    ms = wall_ms(fn, args.steps, args.warmup)
    kms = batch_event_ms(fn, max(20, args.steps), stream)
    gbs = 2 * n / (kms * 1e-3) / 1e9
    out = base_line(args, gbs, "GB/s", ms, "u8", {"workload": "hbm_copy_512MiB", "bytes_read": n, "bytes_written": n})
    out["roofline"] = {"bound": "hbm", "kernel": "device copy", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                       "frac": gbs / HBM_PEAK_GBS, "traffic": 2 * n, "launch_ms": kms}
    return out


HBM_READ_MODES = {0: "register loads, nontemporal (1 KB per wave load)", 1: "register loads, temporal",
                  2: "global_load_lds copies, contiguous 1 KB", 3: "global_load_lds copies, 16 rows x 64 B (prefill weights)",
                  4: "register loads, nontemporal, 48 KB items, 2 in flight per CU (decode streams)",
                  5: "global_load_lds copies, 48 KB items, 2 ahead in a 3-slot ring",
                  6: "global_load_lds copies, 8 rows x 128 B (whole lines of the prefill weight rows)",
                  7: "global_load_lds copies, contiguous 1 KB, 2 MB L2-resident window (on-chip rate)",
                  8: "register loads, nontemporal, 2 MB L2-resident window (on-chip rate)",
                  9: "register loads in the MFMA operand layout (16 rows x 64 B of 1440-byte rows), 2 items in flight",
                  10: "global_load_lds copies, 16 rows x 64 B, 2 MB L2-resident window (on-chip rate)",
                  11: "global_load_lds copies, 8 rows x 128 B, 2 MB L2-resident window (on-chip rate)",
                  12: "FP8-head GEMM chunks: weight rows by global_load_lds + L2 token rows by register loads (both counted)",
                  13: "FP8-head GEMM chunks: weight rows + L2 token rows, both by global_load_lds (both counted)",
                  14: "register loads written to the LDS ring, 8 rows x 128 B, 2 MB L2-resident window (mode 11's depth)",
                  15: "register loads written to the LDS ring, 16 rows x 64 B, 2 MB L2-resident window (mode 10's depth)",
                  16: "register loads written to the LDS ring, 8 rows x 128 B (mode 6's depth)",
                  17: "register loads written to the LDS ring, contiguous 1 KB, 2 MB L2-resident window (mode 7's depth)"}


def hbm_read(args, ctx, dev):
    """Read-only calibration: the kernels of libnerve_calib.so stream a 1 GiB
    buffer once per launch (larger than the 256 MB Infinity Cache), one line
    per read mode; the headline is the fastest mode."""
    import ctypes

    import torch

    from nerve_amd import build as nb

    lib = ctypes.CDLL(nb.CALIB_LIB)
    lib.nerve_calib_read.restype = ctypes.c_int
    lib.nerve_calib_read.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                                     ctypes.c_void_p]
    n = 2 ** 30
    buf = torch.empty(n, dtype=torch.uint8, device=dev).random_(0, 255)
    sink = torch.zeros(4096, dtype=torch.int32, device=dev)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    stream = torch.cuda.current_stream()
    modes = {}
    for mode, what in HBM_READ_MODES.items():
        # the row pattern reads 22 of every 22.5 64-byte columns: count what it reads
        rows_bytes = (n // (cus * 16384)) * cus * 16384
        gemm_steps = (n // (128 * 2880) // cus) * 22
        nbytes = {3: rows_bytes, 6: rows_bytes, 7: rows_bytes, 10: rows_bytes, 11: rows_bytes, 14: rows_bytes,
                  15: rows_bytes, 16: rows_bytes, 17: rows_bytes,
                  12: gemm_steps * cus * 49152, 13: gemm_steps * cus * 49152, 4: (n // 49152) * 49152, 5: (n // 49152) * 49152,
                  9: (n // 46080) * 46080}.get(mode, n)
        fn = lambda i, m=mode: lib.nerve_calib_read(ctypes.c_void_p(buf.data_ptr()), n, m,
                                                    ctypes.c_void_p(sink.data_ptr()), cus,
                                                    ctypes.c_void_p(stream.cuda_stream))
        assert fn(0) == 0, f"nerve_calib_read mode {mode} failed"
        kms = batch_event_ms(fn, max(20, args.steps), stream)
        modes[mode] = {"mode": what, "ms": kms, "gbs": nbytes / (kms * 1e-3) / 1e9}
    # the headline is an HBM rate: the modes reading an L2-resident window (7,
    # 8, 10-15, 17) are reported only
    best = max((v for m, v in modes.items() if m not in (7, 8, 10, 11, 12, 13, 14, 15, 17)), key=lambda v: v["gbs"])
    out = base_line(args, best["gbs"], "GB/s", best["ms"], "u8", {"workload": "hbm_read_1GiB"})
    out["modes"] = list(modes.values())
    out["roofline"] = {"bound": "hbm", "kernel": "nerve_calib_read (" + best["mode"] + ")", "achieved": best["gbs"],
                       "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": best["gbs"] / HBM_PEAK_GBS, "traffic": None,
                       "launch_ms": best["ms"]}
    return out


def _pmc_per_dispatch(csv_dirs, counter):
    """{kernel name: mean counter value per dispatch} from rocprofv3 CSVs
    under the comma-separated directories `csv_dirs`."""
    import csv
    import glob

    vals = {}
    files = [f for d in csv_dirs.split(",")
             for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)]
    for f in files:
        with open(f) as fh:
            for row in csv.DictReader(fh):
                if row.get("Counter_Name") != counter:
                    continue
                name = row["Kernel_Name"].replace("(anonymous namespace)::", "").split("(")[0].strip()
                if name.startswith("void "):
                    name = name[5:]
                vals.setdefault(name, []).append(float(row["Counter_Value"]))
    return {k: sum(v) / len(v) for k, v in vals.items()}


def summarize_traffic(dirs):
    """--summarize-traffic FETCH_DIRS WRITE_DIRS COPY_FETCH_DIR COPY_WRITE_DIR
    (FETCH_DIRS / WRITE_DIRS: comma-separated, one run per workload):
    per-dispatch FETCH_SIZE / WRITE_SIZE (KiB) of every kernel, scaled by the
    copy calibration (512 MiB read and written per dispatch), written to
    profiles/traffic.json and printed as a markdown table."""
    fetch, write, cf, cw = (_pmc_per_dispatch(d, c) for d, c in
                            zip(dirs, ("FETCH_SIZE", "WRITE_SIZE", "FETCH_SIZE", "WRITE_SIZE")))
    copy_name = max(cf, key=lambda k: cf[k])
    n_kib = 512 * 1024
    ff, wf = n_kib / cf[copy_name], n_kib / cw[copy_name]
    out = {"copy_kernel": copy_name, "copy_fetch_kib": cf[copy_name], "copy_write_kib": cw[copy_name],
           "fetch_factor": ff, "write_factor": wf, "kernels": {}}
    for k in fetch:
        fk, wk = fetch[k], write.get(k, 0.0)
        out["kernels"][k] = {"fetch_kib": fk, "write_kib": wk, "hbm_bytes": (fk * ff + wk * wf) * 1024}
    with open(os.path.join(HERE, "profiles", "traffic.json"), "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
    print(f"copy calibration ({copy_name}): FETCH_SIZE {cf[copy_name]:.0f} KiB, WRITE_SIZE {cw[copy_name]:.0f} KiB "
          f"for 524288 KiB each -> factors {ff:.4f} / {wf:.4f}\n")
    print("| kernel | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM bytes (scaled) |\n|---|---|---|---|")
    for k, v in sorted(out["kernels"].items(), key=lambda kv: -kv[1]["hbm_bytes"]):
        print(f"| {k} | {v['fetch_kib']:.0f} | {v['write_kib']:.0f} | {v['hbm_bytes']:.4g} |")


def cpu_baseline(d, budget_s):
    """The C oracle (a per-lane restatement of the reference shaders, OpenMP
    over rows) timed on this host's cores on the same workload: whole MoE
    decode blocks of 16 tokens, repeated until `budget_s` elapses."""
    import oracle

    B, k = d["B"], d["k"]
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    done = 0
    t0 = time.perf_counter()
    while True:
        logits = oracle.router_linear(d["hidden"], d["router_w"])
        routes, _ = oracle.topk(logits, k)
        cmap, _ = oracle.route_compact(routes, k, (d["I"] + 31) // 32, B)
        h = oracle.moe_gate_up(d["hidden"], routes, cmap, B * k, k, d["gate_w"], d["gate_s"], d["up_w"], d["up_s"],
                               d["limit"])
        eo = oracle.moe_down(h, routes, cmap, B * k, d["down_w"], d["down_s"])
        oracle.moe_reduce(eo, 1.0)
        done += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    el = time.perf_counter() - t0
    return {"value": done * B * k / el, "unit": "expert-tokens/s", "cores": threads, "kind": "port",
            "sample": f"{done} full MoE decode block(s) of {B} tokens x top-{k} in {el:.1f} s (C oracle, OpenMP)"}


def main():
    args = parse()
    if args.summarize_traffic:
        summarize_traffic(args.summarize_traffic)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    import torch

    from nerve_amd.hip import Context

    dev = torch.device("cuda:0")
    ctx = Context(0)
    if args.workload == "moe_decode":
        out, d0 = moe_decode(args, ctx, dev)
        if not args.no_prefill:
            out["prefill"] = prefill_sub(ctx, dev)
        if not args.no_cpu_baseline:
            out["cpu_baseline"] = cpu_baseline(d0, args.cpu_seconds)
    elif args.workload == "moe_prefill":
        pf = Prefill(ctx, dev)
        stream = torch.cuda.current_stream()
        ms = wall_ms(pf.step, args.steps, args.warmup)
        kms = event_ms(lambda i: pf.step(i, stream), max(20, args.steps), stream)
        fig = pf.figures(kms)
        out = base_line(args, pf.d["B"] * pf.d["k"] / (kms * 1e-3), "expert-tokens/s", ms, "e4m3xe2m1->f32",
                        {"workload": fig["workload"]})
        out["roofline"] = {"bound": "hbm", "kernel": "MoE prefill block", "achieved": fig["hbm_gbs"],
                           "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": fig["hbm_frac"], "traffic": None,
                           "tflops": fig["tflops"], "mxfp4_peak_frac": fig["mxfp4_peak_frac"]}
    elif args.workload == "mxfp4_gemv":
        out = mxfp4_gemv(args, ctx, dev)
    elif args.workload == "int4_gemv":
        out = int4_gemv(args, ctx, dev)
    elif args.workload == "int4_moe":
        out = int4_moe(args, ctx, dev)
    elif args.workload == "hbm_copy":
        out = hbm_copy(args, ctx, dev)
    elif args.workload == "hbm_read":
        out = hbm_read(args, ctx, dev)
    else:
        out = fp8_head(args, ctx, dev)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
