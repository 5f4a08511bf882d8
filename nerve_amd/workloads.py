"""Seeded synthetic inputs for the five BASELINE configurations, in the
compiled package's layouts.

Generation rules: numpy PCG64 with seed 20260000 + config index; bf16 values
are produced by round-to-nearest-even from f32.  Weights are generated
directly in the packed layouts (there is no checkpoint to convert).
"""
from __future__ import annotations

import numpy as np

SEED_BASE = 20260000


def rng_for(config: int, salt: int = 0) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(SEED_BASE + config + 1000 * salt))


def f32_to_bf16_bits(x) -> np.ndarray:
    b = np.asarray(x, dtype=np.float32).view(np.uint32)
    return ((b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


def bf16_bits_to_f32(h) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def mxfp4_matrix(rng: np.random.Generator, rows: int, K: int, scale_lo: int = 120, scale_hi: int = 128):
    """Uniform e2m1 nibbles packed low-first along K ([rows, K/2] u8) and e8m0
    scale bytes uniform in [scale_lo, scale_hi) ([rows, K/32] u8)."""
    nib = rng.integers(0, 16, size=(rows, K), dtype=np.uint8)
    w = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    s = rng.integers(scale_lo, scale_hi, size=(rows, K // 32), dtype=np.uint8)
    return w, s


def bf16_normal(rng: np.random.Generator, shape, std: float = 1.0) -> np.ndarray:
    return f32_to_bf16_bits(rng.standard_normal(size=shape, dtype=np.float32) * np.float32(std))


def config0(K: int = 2880, N: int = 5760, M: int = 1):
    """MXFP4 GEMV: gate rows 0..N/2 | up rows N/2..N of one expert."""
    rng = rng_for(0)
    w, s = mxfp4_matrix(rng, N, K)
    x = rng.standard_normal(size=(M, K), dtype=np.float32)
    return dict(W=w, S=s, x_f32=x, x_bf16=f32_to_bf16_bits(x))


def moe_experts(rng: np.random.Generator, E: int, H: int, I: int):
    gw = np.empty((E, I, H // 2), np.uint8)
    gs = np.empty((E, I, H // 32), np.uint8)
    uw = np.empty_like(gw)
    us = np.empty_like(gs)
    dw = np.empty((E, H, I // 2), np.uint8)
    ds = np.empty((E, H, I // 32), np.uint8)
    for e in range(E):
        gw[e], gs[e] = mxfp4_matrix(rng, I, H)
        uw[e], us[e] = mxfp4_matrix(rng, I, H)
        dw[e], ds[e] = mxfp4_matrix(rng, H, I)
    return dict(gate_w=gw, gate_s=gs, up_w=uw, up_s=us, down_w=dw, down_s=ds)


def config2(B: int = 16, E: int = 32, k: int = 4, H: int = 2880, I: int = 2880, layer: int = 0):
    """MoE decode block: bf16 router N(0, 0.02), tokens N(0, 1), MXFP4 experts.
    `layer` > 0 draws another layer's router, experts and input tokens."""
    rng = rng_for(2, salt=layer)
    router = bf16_normal(rng, (E, H), 0.02)
    tokens = bf16_normal(rng, (B, H), 1.0)
    d = dict(router_w=router, hidden=tokens, B=B, E=E, k=k, H=H, I=I, limit=7.0)
    d.update(moe_experts(rng, E, H, I))
    return d


def zipf_router_logits(rng: np.random.Generator, B: int, E: int, k: int, s: float = 1.1) -> np.ndarray:
    """bf16 logits whose Gumbel top-k draws experts with Zipf(s) popularity:
    logit = log p_e + Gumbel(0,1), p_e ~ rank_e^-s over a seeded rank
    permutation.  Rows with a bf16 tie at the k/k+1 boundary are redrawn."""
    ranks = rng.permutation(E) + 1
    logp = (-s * np.log(ranks.astype(np.float64))).astype(np.float32)
    out = np.empty((B, E), np.uint16)
    for b in range(B):
        while True:
            g = rng.gumbel(size=E).astype(np.float32)
            row = f32_to_bf16_bits(logp + g)
            vals = np.sort(bf16_bits_to_f32(row))[::-1]
            if vals[k - 1] != vals[k]:
                out[b] = row
                break
    return out


def config3(B: int = 2048, E: int = 128, k: int = 4, H: int = 2880, I: int = 2880):
    """MoE prefill: Zipf(1.1)-skewed router logits, MXFP4 experts."""
    rng = rng_for(3)
    logits = zipf_router_logits(rng, B, E, k)
    tokens = bf16_normal(rng, (B, H), 1.0)
    d = dict(logits=logits, hidden=tokens, B=B, E=E, k=k, H=H, I=I, limit=7.0)
    d.update(moe_experts(rng, E, H, I))
    return d


def int4_gptq(rng: np.random.Generator, K: int, N: int, group: int, symmetric: bool):
    """GPTQ layout: qweight u32 [K/8, N] (8 codes along K per word, low first),
    f16 scales U(0.002, 0.02) [K/g, N], qzeros u32 [K/g, N/8] (8 codes along N)."""
    q = rng.integers(0, 16, size=(K, N), dtype=np.uint32)
    qw = np.zeros((K // 8, N), np.uint32)
    for j in range(8):
        qw |= q[j::8, :] << np.uint32(4 * j)
    scales = rng.uniform(0.002, 0.02, size=(K // group, N)).astype(np.float16)
    if symmetric:
        z = np.full((K // group, N), 8, np.uint32)
    else:
        z = rng.integers(0, 16, size=(K // group, N), dtype=np.uint32)
    qz = np.zeros((K // group, N // 8), np.uint32)
    for j in range(8):
        qz |= z[:, j::8] << np.uint32(4 * j)
    return dict(q=q, qweight=qw, scales=scales, zeros=z, qzeros=qz)


def int4_ct_experts(rng: np.random.Generator, E: int, rows: int, K: int, group: int, scale_bf16: bool = True,
                    keep_codes: bool = False):
    """Sparse INT4-CT expert bank: W u32 [E, rows, K/8] (8 codes along K per
    word, low nibble first, value code - 8) and scale bits u16 [E, rows,
    K/group] (bf16 or f16 values in U(0.002, 0.02)); the layout of
    experts.gate_up / experts.down (tests/test_model_package_moe_components.py:
    1012-1049 in the reference)."""
    q = rng.integers(0, 16, size=(E, rows, K), dtype=np.uint8)
    qq = q.reshape(E, rows, K // 8, 8).astype(np.uint32)
    W = np.zeros((E, rows, K // 8), np.uint32)
    for j in range(8):
        W |= qq[..., j] << np.uint32(4 * j)
    sv = rng.uniform(0.002, 0.02, size=(E, rows, K // group)).astype(np.float32)
    S = f32_to_bf16_bits(sv) if scale_bf16 else sv.astype(np.float16).view(np.uint16)
    d = dict(W=W, S=S)
    if keep_codes:
        d["q"] = q
    return d


def config1(M: int = 1, K: int = 4096, N: int = 14336, group: int = 128, symmetric: bool = False):
    rng = rng_for(1)
    d = int4_gptq(rng, K, N, group, symmetric)
    d["x"] = bf16_normal(rng_for(1, salt=M), (M, K), 1.0)
    d.update(M=M, K=K, N=N, group=group)
    return d


def f32_to_e4m3fn_producer(values) -> np.ndarray:
    """The package's weight producer, f32_to_e4m3fn
    (nerve/model_package_tensors.py:1044-1075), restated: RNE, saturation at
    448, and its subnormal branch that clips rint(x*512) to 7."""
    x = np.asarray(values, dtype=np.float32)
    sign = np.where(np.signbit(x), 0x80, 0).astype(np.uint8)
    ax = np.minimum(np.nan_to_num(np.abs(x), nan=0.0, posinf=448.0, neginf=448.0), np.float32(448.0))
    enc = np.zeros(ax.shape, np.uint8)
    nz = ax > 0.0
    sub = nz & (ax < np.float32(2.0 ** -6))
    if np.any(sub):
        m = np.clip(np.rint(ax[sub] * np.float32(512.0)).astype(np.int32), 0, 7)
        enc[sub] = m.astype(np.uint8)
    nrm = nz & ~sub
    if np.any(nrm):
        v = ax[nrm]
        e = np.floor(np.log2(v)).astype(np.int32)
        sc = v / np.exp2(e.astype(np.float32))
        m = np.rint((sc - np.float32(1.0)) * np.float32(8.0)).astype(np.int32)
        of = m == 8
        e[of] += 1
        m[of] = 0
        ef = e + 7
        sat = (ef > 15) | ((ef == 15) & (m > 6))
        ef = np.where(sat, 15, ef)
        m = np.where(sat, 6, m)
        enc[nrm] = ((ef << 3) | m).astype(np.uint8)
    return enc | sign


def fp8_head(rng: np.random.Generator, N: int, K: int, M: int):
    """e4m3 weights from N(0, 0.02) with per-row scale bf16(amax/448)
    (nerve/representation_optimizer/providers/output_fp8/toolchain.py:628-637
    with one block row); scale_inv grid bf16 [N, ceil(K/128)]."""
    wf = (rng.standard_normal(size=(N, K), dtype=np.float32) * np.float32(0.02))
    amax = np.max(np.abs(wf), axis=1)
    s = np.where(amax > 0, amax / np.float32(448.0), np.float32(1.0)).astype(np.float32)
    s_bf16 = f32_to_bf16_bits(s)
    s_f32 = bf16_bits_to_f32(s_bf16)
    wq = f32_to_e4m3fn_producer(wf / s_f32[:, None])
    nblk = (K + 127) // 128
    grid = np.repeat(s_bf16[:, None], nblk, axis=1)
    x = bf16_normal(rng, (M, K), 1.0)
    return dict(W=wq, scale_inv=grid, scale_f32=s_f32, x=x, N=N, K=K, M=M)


def config4(M: int = 1, K: int = 2880, N: int = 201088):
    return fp8_head(rng_for(4, salt=M), N, K, M)
