// Blockwise e4m3 quantization of bf16 rows (a2), shared by the expert
// projections' own quantization and the fused routing launch, which hands
// the decode gate/up its prequantized hidden rows.
#pragma once

#include <cstdint>

#include "common.h"

namespace {

// ---------------------------------------------------------------------------
// a2: blockwise e4m3 quantization of bf16 rows.
// Row r lives at element offset (r / k) * frame_elems + (r % k) * seg_elems,
// which covers plain [rows, cols] tensors (k = 1) and the per-route slices of
// the intermediate frames.  One 32-lane cluster per 128-column block, as in
// quantize_hidden (…gate_up_batch1_mxfp4.comp.template:366-382).
// ---------------------------------------------------------------------------
struct QuantArgs {
    const uint16_t* x;
    uint32_t k;              // rows are grouped k per frame
    uint64_t frame_elems;    // elements per frame
    uint64_t seg_elems;      // elements between rows of one frame
    uint32_t cols, rows;
    uint8_t* q;              // e4m3 [rows, ldq]: row r's cols bytes at r * ldq
    float* s;                // f32 [rows, ceil(cols/128)]
    uint32_t* zero_word;     // set to 0 by the standalone quantizer (a counter of the next kernel), or null
    uint32_t vec8 = 0;       // x rows, frames and q rows 16-byte aligned: quant_units8_pow2 may be used
    uint32_t ldq = 0;        // q row stride in bytes, >= cols and a multiple of 4
};

// One 32-lane cluster quantizes one (row, 128-column block) unit.  All 32
// lanes of the cluster must call it (the amax is a cluster reduction).
template <bool POW2>
__device__ __forceinline__ void quant_unit(const QuantArgs& Q, uint32_t unit, uint32_t cl) {
    const uint32_t nblk = (Q.cols + 127) / 128;
    const uint32_t row = unit / nblk, blk = unit % nblk;
    const bool unit_ok = row < Q.rows;
    const uint32_t col = blk * 128 + cl * 4;
    const bool valid = unit_ok && col < Q.cols;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (valid) {
        const uint16_t* xr = Q.x + (uint64_t)(row / Q.k) * Q.frame_elems + (uint64_t)(row % Q.k) * Q.seg_elems;
        const uint32_t* p = reinterpret_cast<const uint32_t*>(xr + col);
        const uint32_t w0 = p[0], w1 = p[1];
        v[0] = bf16_to_f32(w0); v[1] = bf16_to_f32(w0 >> 16);
        v[2] = bf16_to_f32(w1); v[3] = bf16_to_f32(w1 >> 16);
    }
    float m = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    m = wave_max32(m);
    if (!valid) return;
    const float sc = POW2 ? pow2_fp8_scale(m) : amax_fp8_scale(m);
    if (cl == 0) Q.s[(uint64_t)row * nblk + blk] = sc;
    const uint32_t packed = f32_to_e4m3(v[0] / sc) | (f32_to_e4m3(v[1] / sc) << 8) |
                            (f32_to_e4m3(v[2] / sc) << 16) | (f32_to_e4m3(v[3] / sc) << 24);
    *reinterpret_cast<uint32_t*>(Q.q + (uint64_t)row * Q.ldq + col) = packed;
}

// Power-of-two block quantization of QU units per 16-lane cluster with all
// QU loads issued before any arithmetic, and the hardware e4m3 conversion:
// x * (1 / s) is exact for a power-of-two s, every quotient of a finite
// block lies in [-448, 448] where v_cvt_pk_fp8_f32 rounds exactly like
// f32_to_e4m3, and a block with a NaN code or an infinite max takes the
// software conversion.  Unit i of the call is unit u0 + i * ustride.
// Requires Q.vec8.
template <uint32_t QU>
__device__ __forceinline__ void quant_units8_pow2(const QuantArgs& Q, uint64_t u0, uint32_t ustride, uint32_t cl) {
    const uint32_t nblk = (Q.cols + 127) / 128;
    const uint64_t units = (uint64_t)Q.rows * nblk;
    v4i w[QU];
    uint32_t row[QU], blk[QU];
    bool valid[QU];
#pragma unroll
    for (uint32_t i = 0; i < QU; i++) {
        const uint64_t u = u0 + (uint64_t)i * ustride;
        const uint32_t uu = (uint32_t)(u < units ? u : 0u);
        row[i] = uu / nblk;
        blk[i] = uu % nblk;
        const uint32_t col = blk[i] * 128 + cl * 8;
        valid[i] = u < units && col < Q.cols;
        const uint16_t* xr = Q.x + (uint64_t)(row[i] / Q.k) * Q.frame_elems + (uint64_t)(row[i] % Q.k) * Q.seg_elems;
        w[i] = *reinterpret_cast<const v4i*>(xr + (valid[i] ? col : blk[i] * 128));
    }
#pragma unroll
    for (uint32_t i = 0; i < QU; i++) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            v[2 * j] = valid[i] ? bf16_to_f32((uint32_t)w[i][j]) : 0.f;
            v[2 * j + 1] = valid[i] ? bf16_to_f32((uint32_t)w[i][j] >> 16) : 0.f;
        }
        float m = 0.f;
#pragma unroll
        for (int j = 0; j < 8; j++) m = fmaxf(m, fabsf(v[j]));
        m = fmaxf(m, __shfl_xor(m, 8));
        m = fmaxf(m, __shfl_xor(m, 4));
        m = fmaxf(m, __shfl_xor(m, 2));
        m = fmaxf(m, __shfl_xor(m, 1));
        if (!valid[i]) continue;
        const float sc = pow2_fp8_scale(m);
        uint32_t p[2];
        bool soft = !(m <= 3.4028235e38f);
        if (!soft) {
            const float inv = __uint_as_float((254u << 23) - __float_as_uint(sc));
            uint32_t nan_bytes = 0;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                int t = __builtin_amdgcn_cvt_pk_fp8_f32(v[4 * h] * inv, v[4 * h + 1] * inv, 0, false);
                t = __builtin_amdgcn_cvt_pk_fp8_f32(v[4 * h + 2] * inv, v[4 * h + 3] * inv, t, true);
                p[h] = (uint32_t)t;
                nan_bytes |= ((p[h] & 0x7f7f7f7fu) + 0x01010101u) & 0x80808080u;
            }
            soft = nan_bytes != 0;
        }
        if (soft) {
#pragma unroll
            for (int h = 0; h < 2; h++)
                p[h] = f32_to_e4m3(v[4 * h] / sc) | (f32_to_e4m3(v[4 * h + 1] / sc) << 8) |
                       (f32_to_e4m3(v[4 * h + 2] / sc) << 16) | (f32_to_e4m3(v[4 * h + 3] / sc) << 24);
        }
        if (cl == 0) Q.s[(uint64_t)row[i] * nblk + blk[i]] = sc;
        *reinterpret_cast<v2i*>(Q.q + (uint64_t)row[i] * Q.ldq + blk[i] * 128 + cl * 8) = v2i{(int)p[0], (int)p[1]};
    }
}

}  // namespace
