"""Benchmark of the MXFP4 routed-MoE hot path on one MI355X.

Workload: one MoE decode block, 32 experts, top-4,
hidden = intermediate = 2880, 16 bf16 tokens, MXFP4 gate/up/down experts,
SwiGLU limit 7.  A step is one full pass of the reference node chain
(router linear -> top-k -> compact -> gate_up -> count -> down -> reduce)
through libnerve_hip's C ABI, inputs resident in HBM.

Prints one JSON line.  `value` = routed (token, expert) pairs processed per
second (16 tokens x 4 experts per step).
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


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    return p.parse_args()


def to_dev(a, dev):
    import torch

    a = np.ascontiguousarray(a)
    view = {np.dtype(np.uint8): np.uint8, np.dtype(np.uint16): np.int16, np.dtype(np.uint32): np.int32}[a.dtype]
    return torch.from_numpy(a.view(view).copy()).to(dev)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    import torch

    from nerve_amd import workloads as wl
    from nerve_amd.hip import Context
    from nerve_amd.moe import ExpertBank, MoEBlock

    dev = torch.device("cuda:0")
    d = wl.config2()
    B, E, k, H, I = d["B"], d["E"], d["k"], d["H"], d["I"]
    ctx = Context(0)
    bank = ExpertBank(*(to_dev(d[n], dev) for n in ("gate_w", "gate_s", "up_w", "up_s", "down_w", "down_s")))
    block = MoEBlock(ctx, to_dev(d["router_w"], dev), bank, k, limit=d["limit"])
    hidden = to_dev(d["hidden"], dev)
    stream = torch.cuda.current_stream()

    # Routing of this seeded batch (distinct experts U fixes the algorithmic bytes).
    block.forward(hidden)
    torch.cuda.synchronize()
    bufs = block.buffers(B)
    routes = bufs["routes"].cpu().numpy().view(np.uint32)
    U = len(np.unique(routes & 0xFFFF))
    expert_bytes = I * H // 2 + I * H // 32            # one MXFP4 matrix + its scales
    gate_up_bytes = U * 2 * expert_bytes + B * H * 2 + B * k * I * 2
    down_bytes = U * expert_bytes + B * k * I * 2 + B * k * H * 2
    step_bytes = gate_up_bytes + down_bytes + E * H * 2 + B * H * 2 * 2 + B * k * H * 2

    for _ in range(args.warmup):
        block.forward(hidden)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        block.forward(hidden)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1e3 / args.steps

    # Dominant kernel: the gate_up entry (act quant + tile build + MFMA GEMV),
    # timed with HIP events on the stream it is launched on.
    c = bufs["control"]
    n_ev = max(50, args.steps)
    ev0 = [torch.cuda.Event(enable_timing=True) for _ in range(n_ev)]
    ev1 = [torch.cuda.Event(enable_timing=True) for _ in range(n_ev)]
    for i in range(n_ev):
        ev0[i].record(stream)
        ctx.mxfp4_moe_gate_up(block.gate_up, hidden, None, bufs["routes"], bufs["inter"], bank.addresses,
                              bank.gate_slots, c, B, stream)
        ev1[i].record(stream)
    torch.cuda.synchronize()
    gu_ms = float(np.median([a.elapsed_time(b) for a, b in zip(ev0, ev1)]))
    achieved = gate_up_bytes / (gu_ms * 1e-3) / 1e9

    result = {
        "metric": METRIC,
        "value": B * k / (ms_per_step * 1e-3),
        "unit": "expert-tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "e4m3xe2m1->f32",
        "data": "synthetic (seeded, package layouts, random-init MXFP4 experts)",
        "config": {"workload": "moe_decode_e32_k4_h2880_i2880_b16", "experts": E, "top_k": k, "hidden": H,
                   "intermediate": I, "batch_tokens": B, "distinct_experts": U},
        "tokens_per_s": B / (ms_per_step * 1e-3),
        "step_hbm_gbs": step_bytes / (ms_per_step * 1e-3) / 1e9,
        "roofline": {"bound": "hbm", "kernel": "mxfp4_moe_gate_up", "achieved": achieved, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS, "traffic": None,
                     "algorithmic_bytes": gate_up_bytes, "launch_ms": gu_ms},
    }

    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(d, args.cpu_seconds)
    print(json.dumps(result))


def cpu_baseline(d, budget_s):
    """The C oracle (a scalar-per-lane restatement of the reference shaders,
    OpenMP over rows) timed on this host on the same workload: whole MoE
    blocks of 16 tokens, repeated until `budget_s` elapses."""
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


if __name__ == "__main__":
    main()
