"""Host-side MoE block over libnerve_hip, mirroring the reference node chain.

The compiler lowers one sparse-expert FFN to ``linear`` (router) ->
``moe_route`` -> ``independent_sparse_moe_gate_up`` ->
``independent_sparse_moe_down`` -> ``moe_reduce``
(nerve/circuit_lowering_sparse_experts.py:7-211), with a route-scheduling
stage (``moe_route_compact`` before gate_up, ``moe_route_count`` before down;
nerve/model_package_batching.py:265-284, nerve/model_package_manifest.py:
1539-1570).  ``MoEBlock.forward`` issues exactly that sequence of C-ABI calls.

Expert weights are reached the way the reference reaches demand-resident
weights: through a table of 8-word address records and per-expert parameter
slots (…gate_up_batch1_mxfp4.comp.template:126-166).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .hip import Context

UNBOUND_SLOT = 0xFFFFFFFF


def float_token(v: float) -> str:
    """Float literal as the manifest writes it (nerve/model_package_common.py:145-146)."""
    return format(v, ".9g")


def gate_up_spec(H: int, I: int, E: int, k: int, limit: float, batch1: bool = True, prequant: bool = False,
                 tensor_parallel: bool = False) -> str:
    """independent_sparse_moe_gate_up specialization; tensor_parallel names
    one rank's slice (nerve/model_package_physical_experts.py:228-260)."""
    return (f"independent_sparse_moe_gate_up{'_batch1' if batch1 else ''}"
            f"{'_tensor_parallel' if tensor_parallel else ''}{'_prequant' if prequant else ''}"
            f"_mxfp4_e2m1_g32_h{H}_i{I}_e{E}_k{k}_limit{float_token(limit)}.comp")


def down_spec(H: int, I: int, E: int, k: int, batch1: bool = True, block_major: bool = False,
              tensor_parallel: bool = False) -> str:
    """independent_sparse_moe_down specialization; a tensor-parallel slice
    reads input-block-major weights (nerve/model_package_physical_experts.py:
    262-330)."""
    return (f"independent_sparse_moe_down{'_batch1' if batch1 else ''}"
            f"{'_tensor_parallel' if tensor_parallel else ''}"
            f"{'_input_block_major_b128' if (block_major or tensor_parallel) else ''}"
            f"_mxfp4_e2m1_g32_h{H}_i{I}_e{E}_k{k}.comp")


def int4_ct_spec(stage: str, H: int, I: int, E: int, k: int, group: int, *, scale_bf16: bool = True,
                 batch1: bool = True) -> str:
    """sparse_moe_{gate_up|down}[_batch1]_int4_ct_… specialization
    (nerve/model_package_sparse_projection_shaders.py:80-84)."""
    return (f"sparse_moe_{stage}{'_batch1' if batch1 else ''}_int4_ct_s{'bf16' if scale_bf16 else 'f16'}"
            f"_g{group}_h{H}_i{I}_e{E}_k{k}.comp")


def topk_spec(E: int, k: int, *, sigmoid: bool = False, normalize: bool = True, softcap: float = 0.0,
              bias: str = "nobias") -> str:
    return (f"moe_topk_batch1_{'sigmoid' if sigmoid else 'softmax'}_bf16_e{E}_k{k}_norm{int(normalize)}"
            f"_cap{float_token(softcap)}_{bias}.comp")


def address_record(t: torch.Tensor | None, *, byte_count: int | None = None, generation: int = 1,
                   resident: int = 1, representation: int = 0) -> list[int]:
    """One 8 x u32 address record {addr_lo, addr_hi, bytes_lo, bytes_hi, gen_lo, gen_hi, resident, repr}."""
    addr = 0 if t is None else t.data_ptr()
    n = (0 if t is None else t.numel() * t.element_size()) if byte_count is None else byte_count
    return [addr & 0xFFFFFFFF, addr >> 32, n & 0xFFFFFFFF, n >> 32, generation & 0xFFFFFFFF, generation >> 32,
            resident, representation]


def u32_tensor(values, device) -> torch.Tensor:
    """u32 words stored in an int32 tensor (bit patterns preserved)."""
    import numpy as np

    arr = np.asarray(values, dtype=np.uint64).astype(np.uint32).view(np.int32)
    return torch.from_numpy(arr.copy()).to(device)


@dataclass
class ExpertBank:
    """Per-expert MXFP4 parameters and their address table.

    gate_w/up_w: u8 [E, I, H/2]; gate_s/up_s: u8 [E, I, H/32];
    down_w: u8 [E, H, I/2]; down_s: u8 [E, H, I/32] (package layouts).
    """

    gate_w: torch.Tensor
    gate_s: torch.Tensor
    up_w: torch.Tensor
    up_s: torch.Tensor
    down_w: torch.Tensor
    down_s: torch.Tensor

    def __post_init__(self):
        self.rebuild_tables()

    @property
    def experts(self) -> int:
        return self.gate_w.shape[0]

    def rebuild_tables(self) -> None:
        E = self.experts
        dev = self.gate_w.device
        recs: list[int] = []
        gate_slots: list[int] = []
        down_slots: list[int] = []
        for e in range(E):
            for t in (self.gate_w[e], self.gate_s[e], self.up_w[e], self.up_s[e]):
                gate_slots.append(len(recs) // 8)
                recs += address_record(t)
            for t in (self.down_w[e], self.down_s[e]):
                down_slots.append(len(recs) // 8)
                recs += address_record(t)
        self.records = recs
        self.addresses = u32_tensor(recs, dev)
        self.gate_slots = u32_tensor(gate_slots, dev)
        self.down_slots = u32_tensor(down_slots, dev)


class Int4CtExpertBank:
    """Sparse INT4-CT expert parameters and their address table.

    gate_up_w: u32 [Eb, 2I, H/8] (as int32), gate_up_s: u16 [Eb, 2I, H/G];
    down_w: u32 [Eb, H, I/8], down_s: u16 [Eb, H, I/G].  Expert e of an
    E-expert model reads bank bank_of[e] (default e), so several experts may
    share one stored tensor; per expert two parameter slots per stage
    (weight, scales), as the shaders' DYNAMIC_PARAMETER_COUNT = 2.
    """

    def __init__(self, gate_up_w, gate_up_s, down_w, down_s, experts: int | None = None, bank_of=None):
        self.gate_up_w, self.gate_up_s, self.down_w, self.down_s = gate_up_w, gate_up_s, down_w, down_s
        nb = gate_up_w.shape[0]
        self.experts = nb if experts is None else experts
        self.bank_of = list(range(self.experts)) if bank_of is None else [int(b) for b in bank_of]
        dev = gate_up_w.device
        recs: list[int] = []
        gu_rec, dn_rec = [], []
        for b in range(nb):
            gu_rec.append((len(recs) // 8, len(recs) // 8 + 1))
            recs += address_record(gate_up_w[b]) + address_record(gate_up_s[b])
            dn_rec.append((len(recs) // 8, len(recs) // 8 + 1))
            recs += address_record(down_w[b]) + address_record(down_s[b])
        gs, ds = [], []
        for e in range(self.experts):
            gs += list(gu_rec[self.bank_of[e]])
            ds += list(dn_rec[self.bank_of[e]])
        self.records = recs
        self.addresses = u32_tensor(recs, dev)
        self.gate_slots = u32_tensor(gs, dev)
        self.down_slots = u32_tensor(ds, dev)


class MoEBlock:
    """One routed-MoE FFN: router linear -> top-k -> compact -> gate_up -> count -> down -> reduce."""

    def __init__(self, ctx: Context, router_w: torch.Tensor, bank: ExpertBank, k: int, *, limit: float = 7.0,
                 routed_scale: float = 1.0, normalize: bool = True, sigmoid: bool = False):
        self.ctx = ctx
        self.router_w = router_w  # bf16 bits in int16 [E, H]
        self.bank = bank
        self.E, self.H = router_w.shape
        self.I = bank.gate_w.shape[1]
        self.k = k
        self.limit = limit
        self.routed_scale = routed_scale
        self.gate_up = gate_up_spec(self.H, self.I, self.E, k, limit)
        # The same projection on hidden rows the fused routing launch has
        # already quantized (bit-identical to its own quantization).
        self.gate_up_pq = gate_up_spec(self.H, self.I, self.E, k, limit, prequant=True)
        self.down = down_spec(self.H, self.I, self.E, k)
        self.topk = topk_spec(self.E, k, sigmoid=sigmoid, normalize=normalize)
        self.fuse_routing = True
        self._bufs = {}

    def buffers(self, B: int) -> dict:
        if B not in self._bufs:
            dev = self.router_w.device
            k, I, H, E = self.k, self.I, self.H, self.E
            frame_words = k * I // 2 + k
            T = E + E * (E - 1) // 2
            self._bufs[B] = dict(
                logits=torch.empty(B, E, dtype=torch.int16, device=dev),
                routes=torch.empty(B, k, dtype=torch.int32, device=dev),
                telemetry=torch.zeros(T, dtype=torch.int32, device=dev),
                inter=torch.zeros(B * frame_words, dtype=torch.int32, device=dev),
                # BatchControl {batch_width, expert_start=0, expert_count=0, ...}
                control=torch.tensor([B, 0, 0, 0, 0, 0, 0, 0], dtype=torch.int32, device=dev),
                expert_out=torch.empty(B, k, H, dtype=torch.int16, device=dev),
                out=torch.empty(B, H, dtype=torch.int16, device=dev),
                # the hidden rows' e4m3 blocks and pow2 scales (fused routing)
                hidden_q=torch.empty(B, H, dtype=torch.uint8, device=dev),
                hidden_s=torch.empty(B, (H + 127) // 128, dtype=torch.float32, device=dev),
            )
        return self._bufs[B]

    def forward(self, hidden: torch.Tensor, stream=None) -> torch.Tensor:
        """hidden: bf16 bits (int16) [B, H] on the device; returns bf16 bits [B, H]."""
        B = hidden.shape[0]
        c = self.ctx
        b = self.buffers(B)
        bank = self.bank
        # Decode-sized batches: router linear + top-k + compaction in one
        # launch, which also quantizes the hidden rows for gate_up.
        fused = self.fuse_routing and c.moe_route_fused(
            self.topk, self.gate_up, hidden, self.router_w, b["logits"], None, b["routes"], b["telemetry"],
            b["inter"], b["control"], B, stream, hidden_q=b["hidden_q"], hidden_scales=b["hidden_s"])
        if fused:
            c.mxfp4_moe_gate_up(self.gate_up_pq, b["hidden_q"], b["hidden_s"], b["routes"], b["inter"], bank.addresses,
                                bank.gate_slots, b["control"], B, stream)
        else:
            c.router_linear_bf16(hidden, self.router_w, b["logits"], B, self.H, self.E, stream)
            c.moe_router_topk(self.topk, b["logits"], None, b["routes"], b["telemetry"], B, stream)
            c.moe_route_compact(self.gate_up, b["routes"], b["inter"], b["control"], B, stream)
            c.mxfp4_moe_gate_up(self.gate_up, hidden, None, b["routes"], b["inter"], bank.addresses,
                                bank.gate_slots, b["control"], B, stream)
        if self.fuse_routing:
            # Count stage folded into the down launch (same control words).
            c.mxfp4_moe_down_counted(self.down, b["inter"], b["routes"], b["expert_out"], bank.addresses,
                                     bank.down_slots, b["control"], B, stream)
        else:
            c.moe_route_compact(self.down, b["routes"], None, b["control"], B, stream)
            c.mxfp4_moe_down(self.down, b["inter"], b["routes"], b["expert_out"], bank.addresses, bank.down_slots,
                             b["control"], B, stream)
        c.moe_reduce(b["expert_out"], b["out"], B, self.H, self.k, self.routed_scale, stream)
        return b["out"]
