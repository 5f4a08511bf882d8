"""ctypes binding of libnerve_hip (the C ABI declared in include/nerve_hip.h).

Torch is used only as device-memory and stream plumbing: every call passes raw
device pointers.  The library must be present: there is no CPU fallback, and a
missing or unloadable library raises ``NerveHipUnavailable``.
"""
from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libnerve_hip.so")

# include/nerve_hip.h, in declaration order.
EXPORTS = (
    "nerve_hip_abi_version",
    "nerve_hip_last_error",
    "nerve_hip_open",
    "nerve_hip_close",
    "nerve_hip_check_specialization",
    "nerve_hip_quantize_fp8_e4m3",
    "nerve_hip_rms_norm_quantize_fp8_e4m3",
    "nerve_hip_rms_norm_quantize_int8_pairpacked",
    "nerve_hip_mxfp4_gemv",
    "nerve_hip_router_linear_bf16",
    "nerve_hip_moe_router_topk",
    "nerve_hip_moe_route_compact",
    "nerve_hip_moe_route_fused",
    "nerve_hip_mxfp4_moe_gate_up",
    "nerve_hip_mxfp4_moe_down",
    "nerve_hip_mxfp4_moe_down_counted",
    "nerve_hip_moe_reduce",
    "nerve_hip_int4_moe_gate_up",
    "nerve_hip_int4_moe_down",
    "nerve_hip_int4_linear",
    "nerve_hip_quantize_int8_pairpacked",
    "nerve_hip_silu_multiply_quantize_int8_pairpacked",
    "nerve_hip_int4_linear_pairpacked",
    "nerve_hip_fp8_output_projection",
    "nerve_hip_fp8_output_projection_noalloc",
    "nerve_hip_argmax_f32",
)

STATUS = {
    0: "OK",
    1: "INVALID_ARGUMENT",
    2: "INVALID_SPEC",
    3: "UNSUPPORTED",
    4: "DEVICE_ERROR",
    5: "OUT_OF_MEMORY",
}


UNSUPPORTED = 3


class NerveHipUnavailable(RuntimeError):
    """libnerve_hip.so is missing or cannot be loaded."""


class NerveHipError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS.get(status, status)}: {message}")
        self.status = status
        self.message = message


_lib = None
_lock = threading.Lock()

P = ctypes.c_void_p
U32 = ctypes.c_uint32
S = ctypes.c_char_p


def _declare(lib) -> None:
    sig = {
        "nerve_hip_abi_version": (ctypes.c_int, []),
        "nerve_hip_last_error": (ctypes.c_char_p, []),
        "nerve_hip_open": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(P)]),
        "nerve_hip_close": (None, [P]),
        "nerve_hip_check_specialization": (ctypes.c_int, [S]),
        "nerve_hip_quantize_fp8_e4m3": (ctypes.c_int, [P, S, P, U32, P, P, P]),
        "nerve_hip_rms_norm_quantize_fp8_e4m3": (ctypes.c_int, [P, S, P, P, P, P, P, U32, P]),
        "nerve_hip_rms_norm_quantize_int8_pairpacked": (ctypes.c_int, [P, S, P, P, P, P, P, P, U32, P]),
        "nerve_hip_mxfp4_gemv": (ctypes.c_int, [P, P, P, U32, U32, P, P, U32, P, P]),
        "nerve_hip_router_linear_bf16": (ctypes.c_int, [P, P, P, P, U32, U32, U32, P]),
        "nerve_hip_moe_router_topk": (ctypes.c_int, [P, S, P, P, P, P, U32, P]),
        "nerve_hip_moe_route_compact": (ctypes.c_int, [P, S, P, P, P, U32, P]),
        "nerve_hip_moe_route_fused": (ctypes.c_int, [P, S, S, P, P, P, P, P, P, P, P, P, P, U32, P]),
        "nerve_hip_mxfp4_moe_gate_up": (ctypes.c_int, [P, S, P, P, P, P, P, U32, P, U32, P, U32, P]),
        "nerve_hip_mxfp4_moe_down": (ctypes.c_int, [P, S, P, P, P, P, U32, P, U32, P, U32, P]),
        "nerve_hip_mxfp4_moe_down_counted": (ctypes.c_int, [P, S, P, P, P, P, U32, P, U32, P, U32, P]),
        "nerve_hip_moe_reduce": (ctypes.c_int, [P, P, P, U32, U32, U32, ctypes.c_float, P]),
        "nerve_hip_int4_moe_gate_up": (ctypes.c_int, [P, S, P, P, P, P, U32, P, U32, P, U32, P]),
        "nerve_hip_int4_moe_down": (ctypes.c_int, [P, S, P, P, P, P, U32, P, U32, P, U32, P]),
        "nerve_hip_int4_linear": (ctypes.c_int, [P, S, P, P, P, P, P, P, U32, P]),
        "nerve_hip_quantize_int8_pairpacked": (ctypes.c_int, [P, S, P, P, P, P, U32, P]),
        "nerve_hip_silu_multiply_quantize_int8_pairpacked": (ctypes.c_int, [P, S, P, P, P, P, P, P, U32, P]),
        "nerve_hip_int4_linear_pairpacked": (ctypes.c_int, [P, S, P, P, P, P, P, P, P, U32, P]),
        "nerve_hip_fp8_output_projection": (ctypes.c_int, [P, S, P, P, P, P, P, P, U32, P]),
        "nerve_hip_fp8_output_projection_noalloc": (ctypes.c_int, [P, S, P, P, P, P, P, P, U32, P]),
        "nerve_hip_argmax_f32": (ctypes.c_int, [P, P, U32, U32, P, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args


def load():
    """Loads libnerve_hip.so (raises NerveHipUnavailable if it is absent)."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise NerveHipUnavailable(
                    f"{LIB_PATH} is not built; run `python -m nerve_amd.build` (hipcc, gfx950)")
            try:
                lib = ctypes.CDLL(LIB_PATH)
            except OSError as exc:
                raise NerveHipUnavailable(f"cannot load {LIB_PATH}: {exc}") from exc
            _declare(lib)
            _lib = lib
    return _lib


def last_error() -> str:
    return load().nerve_hip_last_error().decode()


def check_specialization(spec: str) -> int:
    """Host-only validation of a specialization string (0 = accepted)."""
    return load().nerve_hip_check_specialization(spec.encode())


def _check(status: int) -> None:
    if status != 0:
        raise NerveHipError(status, last_error())


def ptr(t) -> int | None:
    """Raw device pointer of a torch tensor (None passes NULL)."""
    if t is None:
        return None
    return t.data_ptr()


def _spec(s: str | None) -> bytes | None:
    return None if s is None else s.encode()


def _stream(stream) -> int | None:
    if stream is None:
        import torch

        return torch.cuda.current_stream().cuda_stream
    return stream if isinstance(stream, int) else stream.cuda_stream


class Context:
    """A nerve_hip_ctx bound to one device (nerve_hip_open / nerve_hip_close)."""

    def __init__(self, device: int = 0):
        self.lib = load()
        h = P()
        _check(self.lib.nerve_hip_open(device, ctypes.byref(h)))
        self.handle = h
        self.device = device

    def close(self) -> None:
        if self.handle:
            self.lib.nerve_hip_close(self.handle)
            self.handle = P()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- a2
    def quantize_fp8_e4m3(self, spec, x, rows, q, scales, stream=None):
        _check(self.lib.nerve_hip_quantize_fp8_e4m3(self.handle, _spec(spec), ptr(x), rows, ptr(q), ptr(scales),
                                                    _stream(stream)))

    # ---- RMSNorm + FP8 prequantization
    def rms_norm_quantize_fp8_e4m3(self, spec, x, weight, y, q, scales, rows, stream=None):
        _check(self.lib.nerve_hip_rms_norm_quantize_fp8_e4m3(self.handle, _spec(spec), ptr(x), ptr(weight), ptr(y),
                                                             ptr(q), ptr(scales), rows, _stream(stream)))

    def rms_norm_quantize_int8_pairpacked(self, spec, x, weight, y, q, scales, sums, rows, stream=None):
        _check(self.lib.nerve_hip_rms_norm_quantize_int8_pairpacked(self.handle, _spec(spec), ptr(x), ptr(weight),
                                                                    ptr(y), ptr(q), ptr(scales), ptr(sums), rows,
                                                                    _stream(stream)))

    # ---- raw MXFP4 GEMV
    def mxfp4_gemv(self, q, scales, M, K, weight, weight_scale, N, y, stream=None):
        _check(self.lib.nerve_hip_mxfp4_gemv(self.handle, ptr(q), ptr(scales), M, K, ptr(weight), ptr(weight_scale), N,
                                             ptr(y), _stream(stream)))

    # ---- a5
    def router_linear_bf16(self, x, weight, logits, batch_width, hidden, experts, stream=None):
        _check(self.lib.nerve_hip_router_linear_bf16(self.handle, ptr(x), ptr(weight), ptr(logits), batch_width, hidden,
                                                     experts, _stream(stream)))

    # ---- a6
    def moe_router_topk(self, spec, logits, bias, routes, telemetry, batch_width, stream=None):
        _check(self.lib.nerve_hip_moe_router_topk(self.handle, _spec(spec), ptr(logits), ptr(bias), ptr(routes),
                                                  ptr(telemetry), batch_width, _stream(stream)))

    # ---- a7
    def moe_route_compact(self, spec, routes, intermediates, control, batch_width, stream=None):
        _check(self.lib.nerve_hip_moe_route_compact(self.handle, _spec(spec), ptr(routes), ptr(intermediates),
                                                    ptr(control), batch_width, _stream(stream)))

    # ---- a5 + a6 + a7
    def moe_route_fused(self, topk_spec, moe_spec, x, router_weight, logits, bias, routes, telemetry, intermediates,
                        control, batch_width, stream=None, hidden_q=None, hidden_scales=None) -> bool:
        """One launch for router linear + top-k + compaction (and, with
        hidden_q / hidden_scales, the hidden rows quantized for the gate/up
        projection's prequantized form).  Returns False (nothing launched)
        when the batch is too large for the fused form."""
        st = self.lib.nerve_hip_moe_route_fused(self.handle, _spec(topk_spec), _spec(moe_spec), ptr(x),
                                                ptr(router_weight), ptr(logits), ptr(bias), ptr(routes),
                                                ptr(telemetry), ptr(intermediates), ptr(control), ptr(hidden_q),
                                                ptr(hidden_scales), batch_width, _stream(stream))
        if st == UNSUPPORTED:
            return False
        _check(st)
        return True

    # ---- a3
    def mxfp4_moe_gate_up(self, spec, hidden, hidden_scales, routes, intermediates, addresses, param_slots, control,
                          batch_width, stream=None):
        _check(self.lib.nerve_hip_mxfp4_moe_gate_up(
            self.handle, _spec(spec), ptr(hidden), ptr(hidden_scales), ptr(routes), ptr(intermediates),
            ptr(addresses), addresses.numel() // 8, ptr(param_slots), param_slots.numel(), ptr(control), batch_width,
            _stream(stream)))

    # ---- a4
    def mxfp4_moe_down(self, spec, intermediates, routes, expert_outputs, addresses, param_slots, control,
                       batch_width, stream=None):
        _check(self.lib.nerve_hip_mxfp4_moe_down(
            self.handle, _spec(spec), ptr(intermediates), ptr(routes), ptr(expert_outputs), ptr(addresses),
            addresses.numel() // 8, ptr(param_slots), param_slots.numel(), ptr(control), batch_width,
            _stream(stream)))

    # ---- sparse INT4-CT experts
    def int4_moe_gate_up(self, spec, hidden, routes, intermediates, addresses, param_slots, control, batch_width,
                         stream=None):
        _check(self.lib.nerve_hip_int4_moe_gate_up(
            self.handle, _spec(spec), ptr(hidden), ptr(routes), ptr(intermediates), ptr(addresses),
            addresses.numel() // 8, ptr(param_slots), param_slots.numel(), ptr(control), batch_width,
            _stream(stream)))

    def int4_moe_down(self, spec, intermediates, routes, expert_outputs, addresses, param_slots, control,
                      batch_width, stream=None):
        _check(self.lib.nerve_hip_int4_moe_down(
            self.handle, _spec(spec), ptr(intermediates), ptr(routes), ptr(expert_outputs), ptr(addresses),
            addresses.numel() // 8, ptr(param_slots), param_slots.numel(), ptr(control), batch_width,
            _stream(stream)))

    # ---- count stage + a4 in one launch
    def mxfp4_moe_down_counted(self, spec, intermediates, routes, expert_outputs, addresses, param_slots, control,
                               batch_width, stream=None):
        _check(self.lib.nerve_hip_mxfp4_moe_down_counted(
            self.handle, _spec(spec), ptr(intermediates), ptr(routes), ptr(expert_outputs), ptr(addresses),
            addresses.numel() // 8, ptr(param_slots), param_slots.numel(), ptr(control), batch_width,
            _stream(stream)))

    # ---- pair-packed INT8 x INT4
    def quantize_int8_pairpacked(self, spec, x, q, scales, sums, rows, stream=None):
        _check(self.lib.nerve_hip_quantize_int8_pairpacked(self.handle, _spec(spec), ptr(x), ptr(q), ptr(scales),
                                                           ptr(sums), rows, _stream(stream)))

    def silu_multiply_quantize_int8_pairpacked(self, spec, gate, up, y, q, scales, sums, rows, stream=None):
        _check(self.lib.nerve_hip_silu_multiply_quantize_int8_pairpacked(
            self.handle, _spec(spec), ptr(gate), ptr(up), ptr(y), ptr(q), ptr(scales), ptr(sums), rows,
            _stream(stream)))

    def int4_linear_pairpacked(self, spec, q, scales_f32, sums, qweight, scales, aux, y, batch_width, stream=None):
        _check(self.lib.nerve_hip_int4_linear_pairpacked(self.handle, _spec(spec), ptr(q), ptr(scales_f32), ptr(sums),
                                                         ptr(qweight), ptr(scales), ptr(aux), ptr(y), batch_width,
                                                         _stream(stream)))

    # ---- a8
    def moe_reduce(self, expert_outputs, out, batch_width, hidden, experts_per_token, routed_scale=1.0, stream=None):
        _check(self.lib.nerve_hip_moe_reduce(self.handle, ptr(expert_outputs), ptr(out), batch_width, hidden,
                                             experts_per_token, routed_scale, _stream(stream)))

    # ---- a9
    def int4_linear(self, spec, x, qweight, scales, zeros, aux, y, batch_width, stream=None):
        _check(self.lib.nerve_hip_int4_linear(self.handle, _spec(spec), ptr(x), ptr(qweight), ptr(scales), ptr(zeros),
                                              ptr(aux), ptr(y), batch_width, _stream(stream)))

    # ---- a10 + a11
    def fp8_output_projection(self, spec, x, weight, scale_inv, logits_f32, logits_bf16, argmax, batch_width,
                              stream=None):
        _check(self.lib.nerve_hip_fp8_output_projection(self.handle, _spec(spec), ptr(x), ptr(weight), ptr(scale_inv),
                                                        ptr(logits_f32), ptr(logits_bf16), ptr(argmax), batch_width,
                                                        _stream(stream)))

    def fp8_output_projection_noalloc(self, spec, x, weight, scale_inv, logits_f32, logits_bf16, argmax, batch_width,
                                      stream=None):
        """The projection with the library's static per-GPU scratch: no device allocation."""
        _check(self.lib.nerve_hip_fp8_output_projection_noalloc(self.handle, _spec(spec), ptr(x), ptr(weight),
                                                                ptr(scale_inv), ptr(logits_f32), ptr(logits_bf16),
                                                                ptr(argmax), batch_width, _stream(stream)))

    def argmax_f32(self, logits, batch_width, vocab, out, stream=None):
        _check(self.lib.nerve_hip_argmax_f32(self.handle, ptr(logits), batch_width, vocab, ptr(out), _stream(stream)))
