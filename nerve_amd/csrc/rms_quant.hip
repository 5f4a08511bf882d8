// RMSNorm + blockwise e4m3 quantization of bf16 activation rows: the
// prequantization step in front of the "_prequant" expert kernels.
//
// Reference: rms_norm_quantize_fp8_e4m3.comp.template:70-129 (one row) and
// rms_norm_quantize_batch_fp8_e4m3 (rows of a batch, in place); scale
// expression nerve/model_package_shader_templates.py:21-28.
//   inv_rms = inversesqrt(sum(x^2) / H + eps)
//   y       = bf16(x * inv_rms * (w + offset))        (written back, bf16)
//   s_b     = pow2 ? 2^ceil(log2(max(amax_b, 1e-4) / 448)) : (amax_b > 0 ? amax_b / 448 : 1)
//   q       = e4m3(y / s_b)                            per block of `block` columns
// inversesqrt is taken as 1 / sqrt (correctly rounded); the sum of squares
// is a per-thread fma chain, a wave tree and the 4 waves in order.
#include "common.h"

namespace {

struct RmsArgs {
    const uint16_t* x;      // bf16 [rows, H]
    const uint16_t* w;      // bf16 [H]
    uint16_t* y;            // bf16 [rows, H] (may alias x)
    uint8_t* q;             // e4m3 [rows, H]
    float* s;               // f32 [rows, H / block]
    int32_t* sums;          // int8 form: i32 [rows, H / 32]
    uint32_t H, block;
    float eps, offset;
    int pow2;
};

// One 256-thread block per row; a thread owns 8 consecutive columns per
// 2048-column step, so the block/8 lanes of one quantization block are
// consecutive lanes of one wave.
template <bool I8>
__global__ __launch_bounds__(256) void rms_quant_kernel(RmsArgs A) {
    __shared__ float wsum[4];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t H = A.H;
    const uint16_t* xr = A.x + (uint64_t)blockIdx.x * H;
    float ss = 0.0f;
    for (uint32_t c = tid * 8; c < H; c += 256 * 8) {
        const v4i v = *reinterpret_cast<const v4i*>(xr + c);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float lo = bf16_to_f32((uint32_t)v[e]), hi = bf16_to_f32((uint32_t)v[e] >> 16);
            ss = fmaf(lo, lo, ss);
            ss = fmaf(hi, hi, ss);
        }
    }
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) ss += __shfl_xor(ss, d);
    if (lane == 0) wsum[wave] = ss;
    __syncthreads();
    const float total = ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3];
    const float inv = 1.0f / sqrtf(total / (float)H + A.eps);
    const uint32_t lanes_per_block = A.block / 8;
    for (uint32_t c = tid * 8; c < H; c += 256 * 8) {
        const v4i v = *reinterpret_cast<const v4i*>(xr + c);
        const v4i wv = *reinterpret_cast<const v4i*>(A.w + c);
        float y[8];
        uint32_t yb[8];
        float m = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const uint32_t xs = (uint32_t)v[e / 2] >> (16 * (e & 1)), ws = (uint32_t)wv[e / 2] >> (16 * (e & 1));
            yb[e] = f32_to_bf16(bf16_to_f32(xs) * inv * (bf16_to_f32(ws) + A.offset)) & 0xffffu;
            y[e] = bf16_to_f32(yb[e]);
            m = fmaxf(m, fabsf(y[e]));
        }
        // Block max over the block's consecutive lanes (block/8 of them).
        for (uint32_t d = 1; d < lanes_per_block; d <<= 1) m = fmaxf(m, __shfl_xor(m, (int)d));
        uint16_t* yr = A.y + (uint64_t)blockIdx.x * H + c;
        *reinterpret_cast<v4i*>(yr) = v4i{(int)(yb[0] | (yb[1] << 16)), (int)(yb[2] | (yb[3] << 16)),
                                          (int)(yb[4] | (yb[5] << 16)), (int)(yb[6] | (yb[7] << 16))};
        uint32_t q0 = 0, q1 = 0;
        float sc;
        if (I8) {
            // rms_norm_quantize_int8_pairpacked.comp.template:95-150: s =
            // amax / 127, q = round-half-even(clamp(y / s)), pair-packed
            // words (even columns, then odd), and the block's sum of q.
            sc = m > 0.0f ? m / 127.0f : 1.0f;
            int sum = 0;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int iv = (int)__builtin_rintf(fminf(fmaxf(y[e] / sc, -127.0f), 127.0f));
                sum += iv;
                if (e & 1) q1 |= (uint32_t)(iv & 255) << (8 * (e / 2));
                else q0 |= (uint32_t)(iv & 255) << (8 * (e / 2));
            }
            sum += __shfl_xor(sum, 1);
            sum += __shfl_xor(sum, 2);
            if (c % 32 == 0) A.sums[(uint64_t)blockIdx.x * (H / 32) + c / 32] = sum;
        } else {
            sc = A.pow2 ? pow2_fp8_scale(m) : amax_fp8_scale(m);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                q0 |= f32_to_e4m3(y[e] / sc) << (8 * e);
                q1 |= f32_to_e4m3(y[4 + e] / sc) << (8 * e);
            }
        }
        *reinterpret_cast<uint2*>(A.q + (uint64_t)blockIdx.x * H + c) = uint2{q0, q1};
        if (c % A.block == 0) A.s[(uint64_t)blockIdx.x * (H / A.block) + c / A.block] = sc;
    }
}

}  // namespace

static nerve_hip_status rms_quant_launch(nerve_hip_ctx* ctx, const char* spec, bool int8pp, const void* x_bf16,
                                         const void* weight_bf16, void* y_bf16, void* q, void* scales_f32,
                                         void* sums_i32, uint32_t rows, void* stream) {
    nerve_hip_status st = nh::enter(ctx);
    if (st) return st;
    nh::RmsQuantSpec rs;
    if ((st = nh::parse_rms_quant_spec(spec, &rs))) return st;
    if (rs.int8pp != int8pp)
        return nh::fail(NERVE_HIP_INVALID_SPEC, int8pp ? "not an int8_pairpacked RMSNorm quantizer"
                                                       : "not an fp8_e4m3 RMSNorm quantizer");
    if (!x_bf16 || !weight_bf16 || !y_bf16 || !q || !scales_f32 || (int8pp && !sums_i32))
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "null buffer");
    if (rs.batch_tile == 0 && rows > 1)
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "unbatched RMSNorm quantizer takes one row");
    if ((((uintptr_t)x_bf16) | ((uintptr_t)weight_bf16) | ((uintptr_t)y_bf16)) & 15 || ((uintptr_t)q & 7))
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "x, weight and y must be 16-byte aligned, q 8-byte aligned");
    if (rows == 0) return nh::ok();
    RmsArgs A;
    A.x = static_cast<const uint16_t*>(x_bf16);
    A.w = static_cast<const uint16_t*>(weight_bf16);
    A.y = static_cast<uint16_t*>(y_bf16);
    A.q = static_cast<uint8_t*>(q);
    A.s = static_cast<float*>(scales_f32);
    A.sums = static_cast<int32_t*>(sums_i32);
    A.H = rs.hidden;
    A.block = rs.block;
    A.eps = rs.eps;
    A.offset = rs.offset;
    A.pow2 = rs.pow2 ? 1 : 0;
    if (int8pp) rms_quant_kernel<true><<<rows, 256, 0, (hipStream_t)stream>>>(A);
    else rms_quant_kernel<false><<<rows, 256, 0, (hipStream_t)stream>>>(A);
    return nh::check_launch("rms_norm_quantize");
}

extern "C" nerve_hip_status nerve_hip_rms_norm_quantize_int8_pairpacked(nerve_hip_ctx* ctx, const char* spec,
                                                                       const void* x_bf16, const void* weight_bf16,
                                                                       void* y_bf16, void* q_i8, void* scales_f32,
                                                                       void* sums_i32, uint32_t rows, void* stream) {
    return rms_quant_launch(ctx, spec, true, x_bf16, weight_bf16, y_bf16, q_i8, scales_f32, sums_i32, rows, stream);
}

extern "C" nerve_hip_status nerve_hip_rms_norm_quantize_fp8_e4m3(nerve_hip_ctx* ctx, const char* spec,
                                                                const void* x_bf16, const void* weight_bf16,
                                                                void* y_bf16, void* q_e4m3, void* scales_f32,
                                                                uint32_t rows, void* stream) {
    return rms_quant_launch(ctx, spec, false, x_bf16, weight_bf16, y_bf16, q_e4m3, scales_f32, nullptr, rows, stream);
}
