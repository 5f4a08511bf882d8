// Group-scaled INT4 linear (a9) on gfx950 bf16 MFMA.
//
// Reference: linear_int4_gptq.comp.template:95-119 / linear_int4_ct.comp.
// template:95-124 compute y[n] = sum over packed words of
// fma(dot8(x, q - 8), scale[group, n], sum) in f32 and round to bf16.
//
// Here each 4-bit code is turned into the bf16 value 128 + q with one and-or
// per two codes (bf16 0x4300 | q), the MFMA contracts x against those values,
// and a second MFMA against bf16 ones yields sum(x) over the same k, so that
//   sum_k x (q - z) = sum_k x (128 + q) - (128 + z) sum_k x
// per group, which is then scaled by the group scale.  Products are exact in
// f32; only the accumulation order differs from the shader.
//
// MFMA v_mfma_f32_16x16x32_bf16: lane (g = l/16, r = l%16) supplies 8 bf16 of
// A row r and of B column r for its k-slice; both operands are loaded in the
// same per-lane k order, so A/B pairing is the identity.  Result lane (g, r)
// holds D[4g+i][r].
#include "common.h"

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

namespace {

__device__ __forceinline__ v4f mfma_bf16(v4i a, v4i b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, a), __builtin_bit_cast(v8bf, b), c, 0, 0, 0);
}

// 8 codes of one word (low nibble first along k) as bf16 (128 + q) pairs in
// k order (0,4),(1,5),(2,6),(3,7).
__device__ __forceinline__ v4i dequant_word(uint32_t w) {
    return v4i{(int)((w & 0x000F000Fu) | 0x43004300u), (int)(((w >> 4) & 0x000F000Fu) | 0x43004300u),
               (int)(((w >> 8) & 0x000F000Fu) | 0x43004300u), (int)(((w >> 12) & 0x000F000Fu) | 0x43004300u)};
}

// 8 contiguous bf16 activations reordered to the same (0,4),(1,5),(2,6),(3,7) order.
__device__ __forceinline__ v4i permute_act(v4i a) {
    uint32_t d0 = (uint32_t)a.x, d1 = (uint32_t)a.y, d2 = (uint32_t)a.z, d3 = (uint32_t)a.w;
    return v4i{(int)((d0 & 0xFFFFu) | (d2 << 16)), (int)((d0 >> 16) | (d2 & 0xFFFF0000u)),
               (int)((d1 & 0xFFFFu) | (d3 << 16)), (int)((d1 >> 16) | (d3 & 0xFFFF0000u))};
}

__device__ __forceinline__ float load_scale(const uint16_t* p, bool bf16) {
    uint16_t v = *p;
    if (bf16) return bf16_to_f32(v);
    return (float)__builtin_bit_cast(_Float16, v);
}

constexpr uint32_t ONES_BF16 = 0x3F803F80u;

struct Int4Args {
    const uint16_t* x;
    const uint32_t* qw;
    const uint16_t* scales;
    const uint32_t* qzeros;   // gptq only, may be null (zero = 8)
    const uint16_t* aux;      // bias [N] or residual [B, N]
    uint16_t* y;
    uint32_t B, K, N, G;
    int scale_bf16, finalize;
};

__device__ __forceinline__ void finalize_store(const Int4Args& A, uint32_t t, uint32_t n, float sum) {
    // nerve/model_package_shader_selection.py:2504-2533
    float v = sum;
    if (A.finalize == 1) v = bf16_to_f32(A.aux[n]) + sum;
    else if (A.finalize == 2) v = bf16_to_f32(A.aux[(uint64_t)t * A.N + n]) + round_bf16(sum);
    A.y[(uint64_t)t * A.N + n] = (uint16_t)f32_to_bf16(v);
}

// GPTQ layout: qweight [K/8, N].  A wave owns 64 columns (4 MFMA column tiles,
// lane r takes columns n0 + 4r .. n0 + 4r + 3 so one 16-byte load feeds all
// four) and 16 tokens; the block's KS waves split the groups.
template <int KS>
__global__ __launch_bounds__(64 * KS) void int4_gptq_kernel(Int4Args A) {
    __shared__ v4f part[KS][4][64];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t g = lane >> 4, rr = lane & 15;
    const uint32_t n0 = blockIdx.x * 64;
    const uint32_t m0 = blockIdx.y * 16;
    const uint32_t tok = m0 + rr;
    const uint32_t ngroups = A.K / A.G, steps = A.G / 32;
    const uint32_t per = (ngroups + KS - 1) / KS;
    const uint32_t g0 = min(ngroups, wave * per), g1 = min(ngroups, g0 + per);
    const uint32_t col = n0 + 4 * rr;
    const bool tv = tok < A.B;
    const uint16_t* xrow = A.x + (uint64_t)(tv ? tok : 0) * A.K;
    v4f acc[4] = {v4f{0.f, 0.f, 0.f, 0.f}, v4f{0.f, 0.f, 0.f, 0.f}, v4f{0.f, 0.f, 0.f, 0.f}, v4f{0.f, 0.f, 0.f, 0.f}};
    for (uint32_t grp = g0; grp < g1; grp++) {
        v4f ag[4] = {v4f{0.f, 0.f, 0.f, 0.f}, v4f{0.f, 0.f, 0.f, 0.f}, v4f{0.f, 0.f, 0.f, 0.f}, v4f{0.f, 0.f, 0.f, 0.f}};
        v4f as = v4f{0.f, 0.f, 0.f, 0.f};
        for (uint32_t s = 0; s < steps; s++) {
            const uint32_t kb = grp * A.G + 32 * s;
            const uint32_t p = kb / 8 + g;
            v4i wv = *reinterpret_cast<const v4i*>(A.qw + (uint64_t)p * A.N + col);
            v4i av = tv ? *reinterpret_cast<const v4i*>(xrow + kb + 8 * g) : v4i{0, 0, 0, 0};
            v4i ap = permute_act(av);
            ag[0] = mfma_bf16(ap, dequant_word((uint32_t)wv.x), ag[0]);
            ag[1] = mfma_bf16(ap, dequant_word((uint32_t)wv.y), ag[1]);
            ag[2] = mfma_bf16(ap, dequant_word((uint32_t)wv.z), ag[2]);
            ag[3] = mfma_bf16(ap, dequant_word((uint32_t)wv.w), ag[3]);
            as = mfma_bf16(ap, v4i{(int)ONES_BF16, (int)ONES_BF16, (int)ONES_BF16, (int)ONES_BF16}, as);
        }
        const uint16_t* sp = A.scales + (uint64_t)grp * A.N + col;
        uint32_t zw = A.qzeros ? A.qzeros[(uint64_t)grp * (A.N / 8) + col / 8] >> (4 * (col % 8)) : 0x8888u;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float sc = load_scale(sp + j, A.scale_bf16);
            float off = 128.0f + (float)((zw >> (4 * j)) & 15u);
#pragma unroll
            for (int i = 0; i < 4; i++) acc[j][i] = fmaf(sc, ag[j][i] - off * as[i], acc[j][i]);
        }
    }
#pragma unroll
    for (int j = 0; j < 4; j++) part[wave][j][lane] = acc[j];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        v4f t = part[0][j][lane];
#pragma unroll
        for (int w = 1; w < KS; w++) t += part[w][j][lane];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint32_t tt = m0 + 4 * g + i;
            if (tt < A.B) finalize_store(A, tt, col + j, t[i]);
        }
    }
}

// CT layout: qweight [N, K/8], scales [N, K/G], G % 128 == 0.  A wave owns 16
// columns; per 128-k step lane (g, r) loads 4 consecutive words of column r
// (k-slices 4g..4g+3) and MFMA j contracts slice 4g+j of every lane group.
template <int KS>
__global__ __launch_bounds__(64 * KS) void int4_ct_kernel(Int4Args A) {
    __shared__ v4f part[KS][64];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t g = lane >> 4, rr = lane & 15;
    const uint32_t n = blockIdx.x * 16 + rr;
    const uint32_t m0 = blockIdx.y * 16;
    const uint32_t tok = m0 + rr;
    const uint32_t ngroups = A.K / A.G, steps = A.G / 128;
    const uint32_t per = (ngroups + KS - 1) / KS;
    const uint32_t g0 = min(ngroups, wave * per), g1 = min(ngroups, g0 + per);
    const bool tv = tok < A.B;
    const uint16_t* xrow = A.x + (uint64_t)(tv ? tok : 0) * A.K;
    const uint32_t* wrow = A.qw + (uint64_t)n * (A.K / 8);
    v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
    for (uint32_t grp = g0; grp < g1; grp++) {
        v4f ag = v4f{0.f, 0.f, 0.f, 0.f}, as = v4f{0.f, 0.f, 0.f, 0.f};
        for (uint32_t s = 0; s < steps; s++) {
            const uint32_t kb = grp * A.G + 128 * s;
            v4i wv = *reinterpret_cast<const v4i*>(wrow + kb / 8 + 4 * g);
            const uint16_t* xa = xrow + kb + 32 * g;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                v4i av = tv ? *reinterpret_cast<const v4i*>(xa + 8 * j) : v4i{0, 0, 0, 0};
                v4i ap = permute_act(av);
                uint32_t wj = (uint32_t)(j == 0 ? wv.x : j == 1 ? wv.y : j == 2 ? wv.z : wv.w);
                ag = mfma_bf16(ap, dequant_word(wj), ag);
                as = mfma_bf16(ap, v4i{(int)ONES_BF16, (int)ONES_BF16, (int)ONES_BF16, (int)ONES_BF16}, as);
            }
        }
        float sc = load_scale(A.scales + (uint64_t)n * ngroups + grp, A.scale_bf16);
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] = fmaf(sc, ag[i] - 136.0f * as[i], acc[i]);
    }
    part[wave][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    v4f t = part[0][lane];
#pragma unroll
    for (int w = 1; w < KS; w++) t += part[w][lane];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t tt = m0 + 4 * g + i;
        if (tt < A.B) finalize_store(A, tt, n, t[i]);
    }
}

}  // namespace

extern "C" nerve_hip_status nerve_hip_int4_linear(nerve_hip_ctx* ctx, const char* spec, const void* x_bf16,
                                                  const void* qweight, const void* scales, const void* zeros,
                                                  const void* aux_bf16, void* y_bf16, uint32_t batch_width,
                                                  void* stream) {
    nerve_hip_status st = nh::enter(ctx);
    if (st) return st;
    nh::Int4Spec s;
    if ((st = nh::parse_int4_spec(spec, &s))) return st;
    if (!x_bf16 || !qweight || !scales || !y_bf16) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "null buffer");
    if (s.op != 0 && !aux_bf16) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "bias/residual specialization needs aux");
    if (s.batch_tile == 0 && batch_width > 1)
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "unbatched INT4 specialization takes batch_width 1");
    if (batch_width == 0) return nh::ok();
    if ((((uintptr_t)x_bf16) | ((uintptr_t)qweight)) & 15)
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "x and qweight must be 16-byte aligned");
    Int4Args A;
    A.x = static_cast<const uint16_t*>(x_bf16);
    A.qw = static_cast<const uint32_t*>(qweight);
    A.scales = static_cast<const uint16_t*>(scales);
    A.qzeros = static_cast<const uint32_t*>(zeros);
    A.aux = static_cast<const uint16_t*>(aux_bf16);
    A.y = static_cast<uint16_t*>(y_bf16);
    A.B = batch_width;
    A.K = s.in;
    A.N = s.out;
    A.G = s.group;
    A.scale_bf16 = s.scale_bf16;
    A.finalize = s.op;
    hipStream_t strm = (hipStream_t)stream;
    if (s.layout == 0) {
        if (A.N % 64) return nh::fail(NERVE_HIP_UNSUPPORTED, "GPTQ INT4 kernel needs N % 64 == 0");
        if (zeros && A.N % 8) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "qzeros need N % 8 == 0");
        dim3 grid(A.N / 64, (batch_width + 15) / 16);
        int4_gptq_kernel<8><<<grid, 512, 0, strm>>>(A);
        return nh::check_launch("int4_linear_gptq");
    }
    if (zeros) return nh::fail(NERVE_HIP_UNSUPPORTED, "asymmetric zeros are supported for the GPTQ layout only");
    if (A.G % 128 || A.N % 16) return nh::fail(NERVE_HIP_UNSUPPORTED, "CT INT4 kernel needs group % 128 == 0 and N % 16 == 0");
    dim3 grid(A.N / 16, (batch_width + 15) / 16);
    int4_ct_kernel<8><<<grid, 512, 0, strm>>>(A);
    return nh::check_launch("int4_linear_ct");
}
