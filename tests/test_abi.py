"""C-ABI checks that need no GPU: the library loads, exports every symbol the
header declares, and its host-side validation behaves like the reference's
specialization grammar."""
import ctypes
import os
import re

import pytest

from nerve_amd import hip
from nerve_amd.moe import down_spec, gate_up_spec, topk_spec

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    src = open(os.path.join(ROOT, "include", "nerve_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(nerve_hip_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    lib = hip.load()
    syms = header_symbols()
    assert len(syms) >= 16
    for s in syms:
        assert hasattr(lib, s), s
    assert set(syms) == set(hip.EXPORTS)


def test_abi_version():
    assert hip.load().nerve_hip_abi_version() == 1


def test_open_without_device_fails_cleanly():
    # This container has no GPU: open must report an error, not crash.
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    h = ctypes.c_void_p()
    st = hip.load().nerve_hip_open(0, ctypes.byref(h))
    assert st != 0 and not h.value
    assert hip.last_error()


def test_null_context_is_rejected():
    lib = hip.load()
    st = lib.nerve_hip_moe_reduce(None, None, None, 1, 1, 1, 1.0, None)
    assert st == 1 and "ctx" in hip.last_error()


@pytest.mark.parametrize("spec,status", [
    (gate_up_spec(2880, 2880, 32, 4, 7.0), 0),
    (down_spec(2880, 2880, 128, 4), 0),
    ("independent_sparse_moe_gate_up_batch1_prequant_mxfp4_e2m1_g32_h4096_i2048_e256_k6_limit7.comp", 0),
    # sparse INT4-CT experts (nerve/model_package_sparse_projection_shaders.py:80-125)
    ("sparse_moe_gate_up_int4_ct_sbf16_g32_h3072_i1024_e256_k10.comp", 0),
    ("sparse_moe_down_batch1_int4_ct_sf16_g32_h3072_i1024_e256_k10.comp", 0),
    ("sparse_moe_gate_up_batch1_int4_ct_sbf16_g8_h256_i96_e4_k2.comp", 0),
    ("sparse_moe_gate_up_batch2_int4_ct_sbf16_g32_h3072_i1024_e256_k10.comp", 2),
    ("sparse_moe_gate_up_int4_ct_sbf16_g12_h96_i96_e4_k2.comp", 2),
    ("sparse_moe_down_int4_ct_sbf16_g32_h64_i16_e4_k2.comp", 2),
    ("sparse_moe_gate_up_int4_ct_sbf16_g32_h64_i15_e4_k2.comp", 2),
    ("sparse_moe_gate_up_int4_ct_sbf16_g32_h64_i16_e5000_k2.comp", 2),
    ("sparse_moe_gate_up_int4_ct_sbf16_g32_h64_i16_e4_k5.comp", 2),
    ("sparse_moe_gate_up_int4_ct_sbf16_g16_h48_i16_e4_k2.comp", 3),
    ("sparse_moe_gate_up_int4_ct_sbf8_g32_h64_i16_e4_k2.comp", 2),
    ("independent_sparse_moe_gate_up_mxfp4_e2m1_g32_h128_i128_e1_k1_limit10.comp", 0),
    # shape rules (the 128 rule relaxed to 32)
    ("independent_sparse_moe_gate_up_batch1_mxfp4_e2m1_g32_h2890_i2880_e32_k4_limit7.comp", 2),
    ("independent_sparse_moe_gate_up_batch1_mxfp4_e2m1_g32_h2880_i2880_e4_k5_limit7.comp", 2),
    ("independent_sparse_moe_down_batch1_mxfp4_e2m1_g32_h2880_i2880_e32_k4_limit7.comp", 2),
    ("independent_sparse_moe_gate_up_batch1_mxfp4_e2m1_g32_h2880_i2880_e32_k4.comp", 2),
    # tensor-parallel slices: down needs the block-major layout, gate_up must
    # not have it, no native FP8 banks
    ("independent_sparse_moe_down_batch1_tensor_parallel_input_block_major_b128_mxfp4_e2m1_g32_h128_i128_e2_k1.comp", 0),
    ("independent_sparse_moe_gate_up_batch1_tensor_parallel_mxfp4_e2m1_g32_h128_i128_e2_k1_limit7.comp", 0),
    ("independent_sparse_moe_gate_up_batch1_tensor_parallel_prequant_mxfp4_e2m1_g32_h128_i128_e2_k1_limit7.comp", 0),
    ("independent_sparse_moe_down_batch1_tensor_parallel_mxfp4_e2m1_g32_h128_i128_e2_k1.comp", 2),
    ("independent_sparse_moe_down_batch1_tensor_parallel_input_block_major_b128_mxfp4_e2m1_g32_native_fp8_e4m3_se8m0_b128_nf1_h128_i128_e2_k1.comp", 2),
    # e4m3 expert banks (resident / adaptive pre-expanded, native FP8 experts)
    ("independent_sparse_moe_gate_up_batch1_mxfp4_e2m1_resident_fp8_e4m3_g32_h128_i128_e2_k1_limit7.comp", 0),
    ("independent_sparse_moe_down_batch1_mxfp4_e2m1_adaptive_fp8_e4m3_g32_h128_i128_e2_k1.comp", 0),
    ("independent_sparse_moe_down_batch1_mxfp4_e2m1_g32_native_fp8_e4m3_se8m0_b128_nf1_h128_i128_e2_k1.comp", 0),
    ("independent_sparse_moe_down_batch1_mxfp4_e2m1_g32_native_fp8_e4m3_se8m0_b128_nf2_h128_i128_e2_k1.comp", 2),
    ("independent_sparse_moe_down_batch1_mxfp4_e2m1_g32_native_fp8_e4m3_se8m0_b128_nf0_h128_i128_e2_k1.comp", 2),
    (topk_spec(32, 4), 0),
    ("moe_topk_batch1_sigmoid_bf16_e256_k8_norm1_cap0_biasf32.comp", 0),
    ("moe_topk_batch4_softmax_bf16_e32_k4_norm1_cap0_nobias.comp", 2),
    ("moe_topk_batch1_softmax_bf16_e4_k5_norm1_cap0_nobias.comp", 2),
    ("moe_router_batch1_score_topk_sqrtsoftplus_bf16_r64_k4_a2w0.5_norm1_scale2.5_biasbf16.comp", 0),
    ("linear_batch16_int4_gptq_sf16_g128_4096x14336.comp", 0),
    ("linear_residual_int4_ct_sbf16_g128_4096x4096.comp", 0),
    ("linear_int4_ct_sf16_g32_4096x4096.comp", 3),
    ("linear_batch16_int4_gptq_sf16_g100_4000x14336.comp", 2),
    ("linear_prequant_pairpacked_batch16_int4_gptq_sf16_g128_4096x14336.comp", 0),
    ("linear_residual_prequant_pairpacked_int4_gptq_sbf16_g32_4096x4096.comp", 0),
    ("linear_prequant_pairpacked_int4_ct_sf16_g128_4096x4096.comp", 2),
    ("linear_prequant_int4_gptq_sf16_g128_4096x4096.comp", 0),
    ("linear_bias_prequant_batch4_int4_ct_sbf16_g64_4096x4096.comp", 0),
    ("quantize_batch16_int8_symmetric_b32_h4096.comp", 0),
    ("linear_batch64_cooperative_int4_gptq_sf16_g128_4096x14336.comp", 0),
    ("linear_residual_batch64_cooperative_int4_ct_sbf16_g128_4096x4096.comp", 0),
    ("linear_batch64_cooperative_int4_ct_sf16_g64_4096x4096.comp", 3),
    ("linear_batch32_cooperative_int4_gptq_sf16_g128_4096x4096.comp", 2),
    ("quantize_int8_symmetric_b64_h4096.comp", 2),
    ("silu_multiply_quantize_int8_b32_h4096.comp", 2),
    ("quantize_batch4_int8_symmetric_pairpacked_b32_h4096.comp", 0),
    ("quantize_int8_symmetric_pairpacked_b64_h4096.comp", 2),
    ("silu_multiply_quantize_int8_pairpacked_b32_h14336.comp", 0),
    ("silu_multiply_quantize_batch16_int8_pairpacked_b32_h14336.comp", 0),
    ("tied_output_projection_fp8_e4m3_b1x128_201088x2880_scale1_to_f32.comp", 0),
    ("tied_output_projection_batch4_fp8_e4m3_b128x128_151936x4096_scale0.0333333351_to_f32.comp", 0),
    ("tied_output_projection_fp8_e4m3_b1x64_201088x2880_scale1_to_f32.comp", 2),
    ("quantize_fp8_e4m3_spow2_b128_h2880.comp", 0),
    ("rms_norm_quantize_fp8_e4m3_spow2_b64_h2880_eps1e-05_offset1.comp", 0),
    ("rms_norm_quantize_fp8_e4m3_spow2_b128_h2880_eps1e-05_offset1.comp", 2),
    ("rms_norm_quantize_batch16_fp8_e4m3_b32_h4096_eps1e-06_offset0.comp", 0),
    ("rms_norm_quantize_fp8_e4m3_b100_h2800_eps1e-05_offset1.comp", 2),
    ("rms_norm_quantize_batch8_int8_pairpacked_b32_h4096_eps1e-06_offset0.comp", 0),
    ("rms_norm_quantize_int8_pairpacked_b64_h4096_eps1e-06_offset0.comp", 2),
    ("quantize_batch4_fp8_e4m3_b128_h4096.comp", 0),
    ("quantize_fp8_e4m3_b64_h4096.comp", 2),
    ("rms_norm_bf16_h4096.comp", 2),
])
def test_check_specialization(spec, status):
    assert hip.check_specialization(spec) == status, hip.last_error()


def test_product_path_fails_loudly_without_library(tmp_path, monkeypatch):
    monkeypatch.setattr(hip, "LIB_PATH", str(tmp_path / "missing.so"))
    monkeypatch.setattr(hip, "_lib", None)
    with pytest.raises(hip.NerveHipUnavailable):
        hip.load()
