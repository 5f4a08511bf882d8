"""CPU checks of the RMSNorm + FP8 quantizer oracle
(rms_norm_quantize_fp8_e4m3.comp.template:70-129) by what the mathematics
fixes: the quantization of y is exactly the blockwise quantizer's (itself
pinned by the quantizer tests), a constant row normalizes to sign(x)(w + o),
and scaling x by a power of two leaves y unchanged when eps = 0."""
import numpy as np
import pytest

import oracle
from nerve_amd import workloads as wl


@pytest.mark.parametrize("pow2", [False, True])
def test_quantization_is_the_block_quantizer(pow2):
    rng = np.random.default_rng(11 + pow2)
    x = wl.bf16_normal(rng, (3, 640))
    w = wl.bf16_normal(rng, (640,), 0.5)
    y, q, s = oracle.rms_norm_quantize(x, w, 128, pow2, 1e-6, 1.0)
    q2, s2 = oracle.quantize_blocks(y, pow2)
    assert np.array_equal(q, q2) and np.array_equal(s, s2)


def test_constant_row_normalizes_to_the_weight():
    H = 256
    x = np.full((2, H), wl.f32_to_bf16_bits(np.float32(3.0)), np.uint16)
    x[1] = wl.f32_to_bf16_bits(np.float32(-0.25))
    rng = np.random.default_rng(2)
    w = wl.bf16_normal(rng, (H,), 0.3)
    y, _, _ = oracle.rms_norm_quantize(x, w, 64, False, 0.0, 1.0)
    want = wl.bf16_bits_to_f32(w).astype(np.float64) + 1.0
    got = wl.bf16_bits_to_f32(y).astype(np.float64)
    assert np.allclose(got[0], want, rtol=2 ** -7) and np.allclose(got[1], -want, rtol=2 ** -7)


def test_power_of_two_scaling_invariance():
    rng = np.random.default_rng(5)
    x = wl.bf16_normal(rng, (4, 512))
    w = wl.bf16_normal(rng, (512,), 0.5)
    x4 = wl.f32_to_bf16_bits(wl.bf16_bits_to_f32(x) * np.float32(4.0))
    y, q, s = oracle.rms_norm_quantize(x, w, 32, True, 0.0, 0.0)
    y4, q4, s4 = oracle.rms_norm_quantize(x4, w, 32, True, 0.0, 0.0)
    assert np.array_equal(y, y4) and np.array_equal(q, q4) and np.array_equal(s, s4)
