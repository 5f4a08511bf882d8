"""CPU oracle for NERVE's quantized-matmul hot path -- TEST INFRASTRUCTURE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the checker (or the
timed CPU baseline).  The product path never imports it.

The arithmetic lives in ``oracle/nerve_oracle.c`` (built into
``oracle/liboracle.so`` by ``oracle/Makefile``); this module wraps it with
numpy arrays.  Each wrapped function names the reference shader it restates.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE, "-B", "liboracle.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


P = ctypes.c_void_p
I = ctypes.c_int
F = ctypes.c_float
L = ctypes.c_long


def _declare(l) -> None:
    sig = {
        "o_f32_to_bf16": (ctypes.c_uint16, [F]),
        "o_bf16_to_f32": (F, [ctypes.c_uint16]),
        "o_e4m3_to_f32": (F, [ctypes.c_uint8]),
        "o_f32_to_e4m3": (ctypes.c_uint8, [F]),
        "o_e2m1_to_e4m3_bits": (ctypes.c_uint8, [ctypes.c_uint8]),
        "o_e2m1_to_sint8": (ctypes.c_int8, [ctypes.c_uint8]),
        "o_e8m0_scale": (F, [ctypes.c_uint8]),
        "o_mxfp4_value": (F, [ctypes.c_uint8, ctypes.c_uint8]),
        "o_pow2_fp8_scale": (F, [F]),
        "o_amax_fp8_scale": (F, [F]),
        "o_quantize_blocks": (None, [P, L, I, I, I, P, P]),
        "o_rms_norm_quantize": (None, [P, P, I, I, I, I, F, F, P, P, P]),
        "o_mxfp4_gemv": (None, [P, P, I, I, P, P, I, P]),
        "o_mxfp4_gemv_f64": (None, [P, P, I, I, P, P, I, P]),
        "o_router_linear": (None, [P, P, I, I, I, P]),
        "o_topk": (None, [P, I, I, I, I, I, I, F, F, I, F, P, P, P]),
        "o_route_compact": (None, [P, I, ctypes.c_uint32, P, P]),
        "o_moe_gate_up": (None, [P, P, P, I, I, I, I, I, I, F, P, P, P, P, P]),
        "o_moe_down": (None, [P, P, P, I, I, I, I, I, I, P, P, P]),
        "o_moe_down_tp": (None, [P, P, I, I, I, I, I, I, I, P, P, P]),
        "o_moe_reduce": (None, [P, I, I, I, F, P]),
        "o_int4_linear": (None, [I, P, P, P, I, P, I, I, I, I, I, P, P]),
        "o_quantize_i8_pairpacked": (None, [P, I, I, P, P, P]),
        "o_silu_multiply_bf16": (None, [P, P, L, P]),
        "o_int4_linear_pairpacked": (None, [P, P, P, P, P, I, I, I, I, I, I, P, P]),
        "o_quantize_i8": (None, [P, I, I, P, P]),
        "o_int4_linear_prequant": (None, [I, P, P, P, P, I, I, I, I, I, I, P, P]),
        "o_fp8_output_projection": (None, [P, I, I, P, P, I, I, F, P]),
        "o_argmax": (None, [P, I, I, P]),
        "o_sparse_int4_gate_up": (None, [P, P, P, I, I, I, I, I, I, I, I, ctypes.c_uint32, ctypes.c_uint32, P, P, P,
                                         P]),
        "o_sparse_int4_down": (None, [P, P, P, I, I, I, I, I, I, I, I, ctypes.c_uint32, ctypes.c_uint32, P, P, P,
                                      P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(l, name)
        fn.restype = res
        fn.argtypes = args


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# --------------------------------------------------------------------------
# scalar numerics (vectorised through numpy where cheap)
# --------------------------------------------------------------------------

def f32_to_bf16(x) -> np.ndarray:
    """bf16 RNE, ``...gate_up_batch1_mxfp4.comp.template:92-96``."""
    b = np.asarray(x, dtype=np.float32).view(np.uint32)
    return ((b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


def bf16_to_f32(h) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


_E4M3_TABLE = None


def e4m3_table() -> np.ndarray:
    global _E4M3_TABLE
    if _E4M3_TABLE is None:
        _E4M3_TABLE = np.array([lib().o_e4m3_to_f32(i) for i in range(256)], dtype=np.float32)
    return _E4M3_TABLE


def e4m3_to_f32(q) -> np.ndarray:
    return e4m3_table()[np.asarray(q, dtype=np.uint8)]


def f32_to_e4m3(x) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    f = lib().o_f32_to_e4m3
    return np.array([f(float(v)) for v in x.ravel()], dtype=np.uint8).reshape(x.shape)


def e8m0_scale(byte: int) -> float:
    return lib().o_e8m0_scale(byte)


def mxfp4_value(nibble: int, scale_byte: int) -> float:
    return lib().o_mxfp4_value(nibble, scale_byte)


def e2m1_to_e4m3_bits(nibble: int) -> int:
    return lib().o_e2m1_to_e4m3_bits(nibble)


def e2m1_to_sint8(nibble: int) -> int:
    return lib().o_e2m1_to_sint8(nibble)


def pow2_fp8_scale(amax: float) -> float:
    return lib().o_pow2_fp8_scale(amax)


def amax_fp8_scale(amax: float) -> float:
    return lib().o_amax_fp8_scale(amax)


# --------------------------------------------------------------------------
# a2 .. a11
# --------------------------------------------------------------------------

def quantize_blocks(x_bf16: np.ndarray, pow2: bool):
    """a2: blockwise e4m3 activation quantization.  Returns (q [R,C] u8, s [R,nblk] f32)."""
    x = _c(x_bf16, np.uint16)
    rows, cols = x.shape
    nblk = (cols + 127) // 128
    q = np.zeros((rows, cols), np.uint8)
    s = np.zeros((rows, nblk), np.float32)
    lib().o_quantize_blocks(_p(x), cols, rows, cols, int(pow2), _p(q), _p(s))
    return q, s


def rms_norm_quantize(x_bf16: np.ndarray, w_bf16: np.ndarray, block: int, pow2: bool, eps: float, offset: float):
    """RMSNorm + blockwise e4m3 quantization (rms_norm_quantize_fp8_e4m3.comp.template:70-129).
    Returns (y bf16 bits [R, H], q u8 [R, H], s f32 [R, H/block])."""
    x = _c(x_bf16, np.uint16)
    w = _c(w_bf16, np.uint16)
    rows, H = x.shape
    y = np.zeros((rows, H), np.uint16)
    q = np.zeros((rows, H), np.uint8)
    s = np.zeros((rows, H // block), np.float32)
    lib().o_rms_norm_quantize(_p(x), _p(w), rows, H, block, int(pow2), float(eps), float(offset), _p(y), _p(q), _p(s))
    return y, q, s


def mxfp4_gemv(q, s, W, S) -> np.ndarray:
    """Raw MXFP4 GEMV on pre-quantized activations (config 0 entry)."""
    q = _c(q, np.uint8); s = _c(s, np.float32); W = _c(W, np.uint8); S = _c(S, np.uint8)
    M, K = q.shape
    N = W.shape[0]
    assert W.shape == (N, K // 2) and S.shape == (N, K // 32)
    y = np.zeros((M, N), np.float32)
    lib().o_mxfp4_gemv(_p(q), _p(s), M, K, _p(W), _p(S), N, _p(y))
    return y


def mxfp4_gemv_f64(q, s, W, S) -> np.ndarray:
    q = _c(q, np.uint8); s = _c(s, np.float32); W = _c(W, np.uint8); S = _c(S, np.uint8)
    M, K = q.shape
    N = W.shape[0]
    y = np.zeros((M, N), np.float64)
    lib().o_mxfp4_gemv_f64(_p(q), _p(s), M, K, _p(W), _p(S), N, _p(y))
    return y


def router_linear(x_bf16, w_bf16) -> np.ndarray:
    """a5: ``linear_bf16.comp.template:40-98``."""
    x = _c(x_bf16, np.uint16); w = _c(w_bf16, np.uint16)
    B, H = x.shape
    E = w.shape[0]
    out = np.zeros((B, E), np.uint16)
    lib().o_router_linear(_p(x), _p(w), B, H, E, _p(out))
    return out


def topk(logits_bf16, k, *, mode=0, activation=0, normalize=1, softcap=0.0,
         routed_scale=1.0, always_count=0, always_weight=0.0, bias=None,
         telemetry=True):
    """a6: top-k routing.  mode 0 = ``moe_topk_routed`` (activation = sigmoid flag),
    mode 1 = ``moe_router_score_topk`` (activation 0/1/2 = sigmoid/softmax/sqrtsoftplus)."""
    lg = _c(logits_bf16, np.uint16)
    B, E = lg.shape
    total_sel = k + (always_count if mode == 1 else 0)
    total_res = E + (always_count if mode == 1 else 0)
    routes = np.zeros((B, total_sel), np.uint32)
    tel = np.zeros(total_res + total_res * (total_res - 1) // 2, np.uint32) if telemetry else None
    b = None if bias is None else _c(bias, np.float32)
    lib().o_topk(_p(lg), B, E, k, mode, activation, normalize, softcap, routed_scale,
                 always_count, always_weight, _p(b), _p(routes), _p(tel))
    return routes, tel


def route_compact(routes, k, tiles_per_route, batch_width, expert_start=0, expert_count=0):
    """a7: returns (map u32 [B*k], control u32[7])."""
    r = _c(routes, np.uint32).ravel()
    m = np.full(batch_width * k, 0xFFFFFFFF, np.uint32)
    ctl = np.array([batch_width, expert_start, expert_count, 0, 0, 0, 0], np.uint32)
    lib().o_route_compact(_p(r), k, tiles_per_route, _p(m), _p(ctl))
    return m, ctl


def moe_gate_up(hidden, routes, cmap, n_routes, k, gw, gs, uw, us, limit, inter=None):
    """a2 + a3.  Expert banks gw/uw [E, I, H/2] u8, gs/us [E, I, H/32] u8.
    Returns bf16 intermediates [B, k, I]."""
    h = _c(hidden, np.uint16)
    B, H = h.shape
    E, I, _ = gw.shape
    out = np.zeros((B, k, I), np.uint16) if inter is None else _c(inter, np.uint16).copy()
    lib().o_moe_gate_up(_p(h), _p(_c(routes, np.uint32)), _p(_c(cmap, np.uint32)), n_routes,
                        B, k, E, H, I, limit, _p(_c(gw, np.uint8)), _p(_c(gs, np.uint8)),
                        _p(_c(uw, np.uint8)), _p(_c(us, np.uint8)), _p(out))
    return out


def moe_down(inter, routes, cmap, n_routes, dw, ds, out=None):
    """a2 + a4.  dw [E, H, I/2], ds [E, H, I/32].  Returns bf16 [B, k, H]."""
    it = _c(inter, np.uint16)
    B, k, I = it.shape
    E, H, _ = dw.shape
    o = np.zeros((B, k, H), np.uint16) if out is None else _c(out, np.uint16).copy()
    lib().o_moe_down(_p(it), _p(_c(routes, np.uint32)), _p(_c(cmap, np.uint32)), n_routes,
                     B, k, E, H, I, _p(_c(dw, np.uint8)), _p(_c(ds, np.uint8)), _p(o))
    return o


def moe_down_tp(inter_slice, routes, start, dw, ds, out=None):
    """Tensor-parallel down slice: inter_slice bf16 [B, k, count] = columns
    [start, start + count) of the intermediates; dw [E, H, I/2], ds [E, H,
    I/32] (row layout).  Returns f32 [B, k, H], not scaled by the route
    weight; routes of a token after its first out-of-range expert keep
    ``out``'s values."""
    it = _c(inter_slice, np.uint16)
    B, k, count = it.shape
    E, H, I2 = dw.shape
    o = np.zeros((B, k, H), np.float32) if out is None else _c(out, np.float32).copy()
    lib().o_moe_down_tp(_p(it), _p(_c(routes, np.uint32)), B, k, E, H, 2 * I2, int(start), count,
                        _p(_c(dw, np.uint8)), _p(_c(ds, np.uint8)), _p(o))
    return o


def moe_reduce(expert_out, routed_scale=1.0):
    """a8: ``moe_reduce_batch1_bf16.comp.template:29-54``."""
    eo = _c(expert_out, np.uint16)
    B, k, H = eo.shape
    out = np.zeros((B, H), np.uint16)
    lib().o_moe_reduce(_p(eo), B, k, H, routed_scale, _p(out))
    return out


def int4_linear(layout, x_bf16, qweight, scales, group, *, scale_bf16=False, zeros=None,
                finalize=0, aux=None):
    """a9: layout "gptq" (qweight [K/8, N]) or "ct" (qweight [N, K/8])."""
    x = _c(x_bf16, np.uint16)
    B, K = x.shape
    qw = _c(qweight, np.uint32)
    lay = {"gptq": 0, "ct": 1}[layout]
    N = qw.shape[1] if lay == 0 else qw.shape[0]
    y = np.zeros((B, N), np.uint16)
    lib().o_int4_linear(lay, _p(x), _p(qw), _p(_c(scales, np.uint16)), int(scale_bf16),
                        _p(None if zeros is None else _c(zeros, np.uint32)), group, K, N, B,
                        finalize, _p(None if aux is None else _c(aux, np.uint16)), _p(y))
    return y


def quantize_i8_pairpacked(x_bf16):
    """Pair-packed symmetric INT8 activations per 32 columns.
    Returns (q u8 [R, C] in pair-packed byte order, s f32 [R, C/32], sums i32 [R, C/32])."""
    x = _c(x_bf16, np.uint16)
    rows, cols = x.shape
    q = np.zeros((rows, cols), np.uint8)
    s = np.zeros((rows, cols // 32), np.float32)
    sums = np.zeros((rows, cols // 32), np.int32)
    lib().o_quantize_i8_pairpacked(_p(x), rows, cols, _p(q), _p(s), _p(sums))
    return q, s, sums


def silu_multiply_bf16(g_bf16, u_bf16):
    """y = bf16(bf16(silu(g)) * u), elementwise (bf16 bits in, bf16 bits out)."""
    g = _c(g_bf16, np.uint16)
    u = _c(u_bf16, np.uint16)
    y = np.zeros(g.shape, np.uint16)
    lib().o_silu_multiply_bf16(_p(g), _p(u), g.size, _p(y))
    return y


def int4_linear_pairpacked(q, s, sums, qweight, scales, group, *, scale_bf16=False, finalize=0, aux=None):
    """Pair-packed INT8 x GPTQ INT4 (qweight [K/8, N], scales [K/G, N])."""
    q = _c(q, np.uint8)
    B, K = q.shape
    qw = _c(qweight, np.uint32)
    N = qw.shape[1]
    y = np.zeros((B, N), np.uint16)
    lib().o_int4_linear_pairpacked(_p(q), _p(_c(s, np.float32)), _p(_c(sums, np.int32)), _p(qw),
                                   _p(_c(scales, np.uint16)), int(scale_bf16), group, K, N, B, finalize,
                                   _p(None if aux is None else _c(aux, np.uint16)), _p(y))
    return y


def fp8_output_projection(x_bf16, w_e4m3, scale_inv_bf16, block_rows=1, output_scale=1.0):
    """a10: returns f32 logits [M, N]."""
    x = _c(x_bf16, np.uint16)
    M, K = x.shape
    w = _c(w_e4m3, np.uint8)
    N = w.shape[0]
    out = np.zeros((M, N), np.float32)
    lib().o_fp8_output_projection(_p(x), M, K, _p(w), _p(_c(scale_inv_bf16, np.uint16)),
                                  block_rows, N, output_scale, _p(out))
    return out


def argmax(logits) -> np.ndarray:
    """a11: ``greedy_sampler_f32.comp.template:25-109`` (ties -> lower id)."""
    lg = _c(logits, np.float32)
    M, N = lg.shape
    ids = np.zeros(M, np.uint32)
    lib().o_argmax(_p(lg), M, N, _p(ids))
    return ids


def quantize_i8(x_bf16):
    """Symmetric INT8 activations per 32 columns, natural byte order.
    Returns (q u8 [R, C], s f32 [R, C/32])."""
    x = _c(x_bf16, np.uint16)
    rows, cols = x.shape
    q = np.zeros((rows, cols), np.uint8)
    s = np.zeros((rows, cols // 32), np.float32)
    lib().o_quantize_i8(_p(x), rows, cols, _p(q), _p(s))
    return q, s


def int4_linear_prequant(layout, q, s, qweight, scales, group, *, scale_bf16=False, finalize=0, aux=None):
    """INT8-prequant INT4 linear, unpaired input: layout "gptq" (qweight
    [K/8, N], scales [K/G, N]) or "ct" (qweight [N, K/8], scales [N, K/G])."""
    q = _c(q, np.uint8)
    B, K = q.shape
    qw = _c(qweight, np.uint32)
    lay = {"gptq": 0, "ct": 1}[layout]
    N = qw.shape[1] if lay == 0 else qw.shape[0]
    y = np.zeros((B, N), np.uint16)
    lib().o_int4_linear_prequant(lay, _p(q), _p(_c(s, np.float32)), _p(qw), _p(_c(scales, np.uint16)),
                                 int(scale_bf16), group, K, N, B, finalize,
                                 _p(None if aux is None else _c(aux, np.uint16)), _p(y))
    return y


def _ct_bound(bound, E):
    return None if bound is None else _c(np.asarray(bound, np.uint8), np.uint8)


def sparse_int4_gate_up(hidden, routes, cmap, n_pos, W, S, group, *, scale_bf16=True, expert_start=0,
                        expert_count=0, bound=None, inter=None):
    """Sparse INT4-CT gate/up (``sparse_moe_gate_up_int4_ct.comp.template:97-227``).
    hidden bf16 [B, H]; routes u32 [B, k]; cmap: compacted positions -> route
    index (None: identity); W u32 [E, 2I, H/8]; S u16 [E, 2I, H/group].
    Returns bf16 intermediates [B, k, I] (``inter`` supplies the untouched
    values)."""
    h = _c(hidden, np.uint16)
    r = _c(routes, np.uint32)
    B, H = h.shape
    k = r.shape[1]
    E, R2, _ = W.shape
    I = R2 // 2
    out = np.zeros((B, k, I), np.uint16) if inter is None else _c(inter, np.uint16).copy()
    m = None if cmap is None else _c(cmap, np.uint32)
    bd = _ct_bound(bound, E)
    lib().o_sparse_int4_gate_up(_p(h), _p(r), None if m is None else _p(m), n_pos, B, k, E, H, I, group,
                                int(scale_bf16), expert_start, expert_count, None if bd is None else _p(bd),
                                _p(_c(W, np.uint32)), _p(_c(S, np.uint16)), _p(out))
    return out


def sparse_int4_down(inter, routes, cmap, n_pos, W, S, group, *, scale_bf16=True, expert_start=0,
                     expert_count=0, bound=None, out=None):
    """Sparse INT4-CT down (``sparse_moe_down_int4_ct.comp.template:106-193``).
    inter bf16 [B, k, I]; W u32 [E, H, I/8]; S u16 [E, H, I/group].  Returns
    bf16 expert outputs [B, k, H]."""
    it = _c(inter, np.uint16)
    r = _c(routes, np.uint32)
    B, k, I = it.shape
    E, H, _ = W.shape
    o = np.zeros((B, k, H), np.uint16) if out is None else _c(out, np.uint16).copy()
    m = None if cmap is None else _c(cmap, np.uint32)
    bd = _ct_bound(bound, E)
    lib().o_sparse_int4_down(_p(it), _p(r), None if m is None else _p(m), n_pos, B, k, E, H, I, group,
                             int(scale_bf16), expert_start, expert_count, None if bd is None else _p(bd),
                             _p(_c(W, np.uint32)), _p(_c(S, np.uint16)), _p(o))
    return o
