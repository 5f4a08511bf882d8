"""CPU checks of the pair-packed INT8 x INT4 oracle
(quantize_int8_symmetric_pairpacked.comp.template:22-72,
linear_prequant_pairpacked_int4_gptq.comp.template:56-95) against what the
mathematics fixes: the quantized codes dequantize to x within half a step,
the block sums are the sums of the codes, the byte order pairs column 8p + j
with nibble j, and the INT4 product equals the bf16 INT4 oracle (itself
pinned) applied to the dequantized activations, up to f32 rounding."""
import numpy as np

import oracle
from nerve_amd import workloads as wl


def _unpack(q):
    """Pair-packed bytes -> int8 codes in column order."""
    R, C = q.shape
    v = q.view(np.int8).reshape(R, C // 8, 2, 4)           # [.., even/odd word, byte]
    out = np.empty((R, C // 8, 8), np.int8)
    out[:, :, 0::2] = v[:, :, 0, :]
    out[:, :, 1::2] = v[:, :, 1, :]
    return out.reshape(R, C)


def test_quantizer_codes_sums_and_order():
    rng = np.random.default_rng(1)
    x = wl.bf16_normal(rng, (3, 256))
    x[0, :32] = 0                                    # an all-zero block: scale 1, codes 0
    q, s, sums = oracle.quantize_i8_pairpacked(x)
    codes = _unpack(q).astype(np.int64)
    xf = wl.bf16_bits_to_f32(x).astype(np.float64)
    step = np.repeat(s.astype(np.float64), 32, axis=1)
    assert np.all(np.abs(codes * step - xf) <= step / 2 + 1e-12)
    assert np.array_equal(sums, codes.reshape(3, 8, 32).sum(axis=2))
    assert s[0, 0] == 1.0 and np.all(codes[0, :32] == 0)
    assert np.max(np.abs(codes)) == 127                # the block max maps to +-127


def test_linear_matches_bf16_oracle_on_dequantized_input():
    rng = np.random.default_rng(2)
    K, N, G, B = 512, 64, 128, 3
    d = wl.int4_gptq(rng, K, N, G, True)
    x = wl.bf16_normal(rng, (B, K))
    q, s, sums = oracle.quantize_i8_pairpacked(x)
    y = oracle.int4_linear_pairpacked(q, s, sums, d["qweight"], d["scales"].view(np.uint16), G)
    # dequantized activations are exact bf16 values here only approximately, so
    # compare in f64 against the closed form sum_k x_q s (q - 8) s_w
    codes = _unpack(q).astype(np.float64) * np.repeat(s.astype(np.float64), 32, axis=1)
    wq = d["q"].astype(np.float64) - 8.0                                   # [K, N]
    sw = np.repeat(d["scales"].astype(np.float64), G, axis=0)
    ref = codes @ (wq * sw)
    got = wl.bf16_bits_to_f32(y).astype(np.float64)
    assert np.max(np.abs(got - ref) / (np.abs(ref) + np.sqrt(np.mean(ref ** 2)))) < 1e-2


def test_silu_multiply_closed_forms():
    """silu(0) = 0, silu(x) -> x for large x, silu(x) - silu(-x) = x, and the
    product with u (all up to the two bf16 roundings)."""
    g = wl.f32_to_bf16_bits(np.array([0.0, 30.0, -30.0, 1.5, -1.5, 3.0, -3.0], np.float32))
    one = wl.f32_to_bf16_bits(np.ones(7, np.float32))
    y = wl.bf16_bits_to_f32(oracle.silu_multiply_bf16(g, one)).astype(np.float64)
    assert y[0] == 0.0 and abs(y[1] - 30.0) <= 30.0 * 2 ** -7 and abs(y[2]) < 1e-9
    for i in (3, 5):
        xv = wl.bf16_bits_to_f32(g[i])
        assert abs((y[i] - y[i + 1]) - xv) <= abs(xv) * 2 ** -6
    u = wl.f32_to_bf16_bits(np.full(7, -2.0, np.float32))
    y2 = wl.bf16_bits_to_f32(oracle.silu_multiply_bf16(g, u)).astype(np.float64)
    assert np.array_equal(y2, -2.0 * y)                   # a power-of-two factor is exact


# --------------------------------------------------------------------------
# Unpaired INT8 input (quantize_int8_symmetric.comp.template:38-58,
# linear_prequant_int4_{gptq,ct}.comp.template)
# --------------------------------------------------------------------------

def test_unpaired_quantizer_is_the_pairpacked_codes_in_column_order():
    """Both quantizers apply the same rule per 32 columns; only the byte order
    differs (the pair-packed one is pinned above)."""
    rng = np.random.default_rng(3)
    x = wl.bf16_normal(rng, (4, 384))
    x[1, 64:96] = 0
    q, s = oracle.quantize_i8(x)
    qp, sp, sums = oracle.quantize_i8_pairpacked(x)
    assert np.array_equal(q.view(np.int8), _unpack(qp))
    assert np.array_equal(s, sp)


def test_unpaired_gptq_linear_equals_pairpacked_on_the_same_codes():
    """block_dot = sum q (code - 8) = sum q code - 8 sum q: the unpaired and the
    pair-packed GPTQ forms hold the same integers and the same fma order, so
    their outputs are bit-identical; finalize forms included."""
    rng = np.random.default_rng(4)
    K, N, G, B = 512, 48, 128, 3
    d = wl.int4_gptq(rng, K, N, G, True)
    x = wl.bf16_normal(rng, (B, K))
    q, s = oracle.quantize_i8(x)
    qp, sp, sums = oracle.quantize_i8_pairpacked(x)
    sc = d["scales"].view(np.uint16)
    for fin, aux in ((0, None), (1, wl.bf16_normal(rng, (N,))), (2, wl.bf16_normal(rng, (B, N)))):
        y = oracle.int4_linear_prequant("gptq", q, s, d["qweight"], sc, G, finalize=fin, aux=aux)
        yp = oracle.int4_linear_pairpacked(qp, sp, sums, d["qweight"], sc, G, finalize=fin, aux=aux)
        assert np.array_equal(y, yp), fin


def test_unpaired_ct_linear_closed_form():
    """The CT form against sum_k x_q s_x (code - 8) s_w in float64 (its f32
    chains differ from the GPTQ order only by rounding), and against the
    GPTQ form on the same codes in the transposed layout."""
    rng = np.random.default_rng(5)
    K, N, G, B = 1024, 32, 128, 2
    d = wl.int4_gptq(rng, K, N, G, True)
    x = wl.bf16_normal(rng, (B, K))
    q, s = oracle.quantize_i8(x)
    qt = np.ascontiguousarray(d["q"].T)                          # [N, K]
    qct = np.zeros((N, K // 8), np.uint32)
    for j in range(8):
        qct |= qt[:, j::8] << np.uint32(4 * j)
    sct = np.ascontiguousarray(d["scales"].T).view(np.uint16)
    y = wl.bf16_bits_to_f32(oracle.int4_linear_prequant("ct", q, s, qct, sct, G)).astype(np.float64)
    xq = q.view(np.int8).astype(np.float64) * np.repeat(s.astype(np.float64), 32, axis=1)
    ref = xq @ ((d["q"].astype(np.float64) - 8.0) * np.repeat(d["scales"].astype(np.float64), G, axis=0))
    assert np.max(np.abs(y - ref) / (np.abs(ref) + 1e-3 * np.sqrt(np.mean(ref ** 2)))) <= 2 ** -7
    yg = wl.bf16_bits_to_f32(oracle.int4_linear_prequant("gptq", q, s, d["qweight"], d["scales"].view(np.uint16),
                                                          G)).astype(np.float64)
    assert np.mean(yg == y) > 0.9
