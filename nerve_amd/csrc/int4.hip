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

__device__ __forceinline__ float decode_scale(uint16_t v, bool bf16) {
    if (bf16) return bf16_to_f32(v);
    return (float)__builtin_bit_cast(_Float16, v);
}

__device__ __forceinline__ float load_scale(const uint16_t* p, bool bf16) { return decode_scale(*p, bf16); }

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

// J consecutive packed words of one qweight row (J = 1, 2 or 4).
template <int J>
__device__ __forceinline__ void load_words(const uint32_t* p, uint32_t (&w)[J]) {
    if constexpr (J == 4) {
        v4i v = *reinterpret_cast<const v4i*>(p);
        w[0] = (uint32_t)v.x; w[1] = (uint32_t)v.y; w[2] = (uint32_t)v.z; w[3] = (uint32_t)v.w;
    } else if constexpr (J == 2) {
        v2i v = *reinterpret_cast<const v2i*>(p);
        w[0] = (uint32_t)v.x; w[1] = (uint32_t)v.y;
    } else {
        w[0] = *p;
    }
}

// GPTQ layout: qweight [K/8, N].  A wave owns 16 J columns (J MFMA column
// tiles; lane r takes columns n0 + J r .. n0 + J r + J - 1 so one load feeds
// all J) and 16 tokens; the block's KS waves split the groups.
template <int KS, int J, uint32_t GQ_BATCH>
__global__ __launch_bounds__(64 * KS) void int4_gptq_kernel(Int4Args A) {
    __shared__ v4f part[KS][J][64];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t g = lane >> 4, rr = lane & 15;
    // XCD-aware order: the hardware deals consecutive workgroups to the 8
    // XCDs in turn; remapping gives each XCD a contiguous run of column tiles
    // so partial cache lines shared by neighbouring tiles hit its L2.  The
    // grid is padded to a multiple of 8; padding blocks exit.
    const uint32_t per_xcd = gridDim.x / 8;
    const uint32_t tile = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    const uint32_t n0 = tile * (16 * J);
    if (n0 >= A.N) return;
    const uint32_t m0 = blockIdx.y * 16;
    const uint32_t tok = m0 + rr;
    const uint32_t ngroups = A.K / A.G, steps = A.G / 32;
    const uint32_t per = (ngroups + KS - 1) / KS;
    const uint32_t g0 = min(ngroups, wave * per), g1 = min(ngroups, g0 + per);
    const uint32_t col = n0 + J * rr;
    const bool tv = tok < A.B;
    const uint16_t* xrow = A.x + (uint64_t)(tv ? tok : 0) * A.K;
    v4f acc[J], ag[J];
#pragma unroll
    for (int j = 0; j < J; j++) acc[j] = ag[j] = v4f{0.f, 0.f, 0.f, 0.f};
    v4f as = v4f{0.f, 0.f, 0.f, 0.f};
    // The wave's 32-k steps run in batches of GQ_BATCH: every weight and
    // activation load of a batch is issued before its first MFMA, so the wave
    // waits for memory once per batch.  A group's partial sums are scaled and
    // folded into acc when its last step has been contracted.
    const uint32_t first = g0 * steps, last = g1 * steps;
    for (uint32_t base = first; base < last; base += GQ_BATCH) {
        uint32_t wbuf[GQ_BATCH][J], zbuf[GQ_BATCH];
        uint16_t sbuf[GQ_BATCH][J];
        v4i abuf[GQ_BATCH];
#pragma clang loop unroll(full)
        for (uint32_t u = 0; u < GQ_BATCH; u++) {
            const uint32_t i = min(base + u, last - 1);
            const uint32_t kb = i * 32;
            const uint32_t p = kb / 8 + g;
            load_words<J>(A.qw + (uint64_t)p * A.N + col, wbuf[u]);
            abuf[u] = tv ? *reinterpret_cast<const v4i*>(xrow + kb + 8 * g) : v4i{0, 0, 0, 0};
            // The group's scales and zero codes ride with its last step, so
            // the fold below does not wait on a dependent load.
            if ((i + 1) % steps == 0) {
                const uint32_t grp = i / steps;
                const uint16_t* sp = A.scales + (uint64_t)grp * A.N + col;
#pragma unroll
                for (int j = 0; j < J; j++) sbuf[u][j] = sp[j];
                zbuf[u] = A.qzeros ? A.qzeros[(uint64_t)grp * (A.N / 8) + col / 8] >> (4 * (col % 8)) : 0x8888u;
            }
        }
#pragma clang loop unroll(full)
        for (uint32_t u = 0; u < GQ_BATCH; u++) {
            const uint32_t i = base + u;
            if (i >= last) continue;
            v4i ap = permute_act(abuf[u]);
#pragma unroll
            for (int j = 0; j < J; j++) ag[j] = mfma_bf16(ap, dequant_word(wbuf[u][j]), ag[j]);
            as = mfma_bf16(ap, v4i{(int)ONES_BF16, (int)ONES_BF16, (int)ONES_BF16, (int)ONES_BF16}, as);
            if ((i + 1) % steps == 0) {
                const uint32_t zw = zbuf[u];
#pragma unroll
                for (int j = 0; j < J; j++) {
                    float sc = decode_scale(sbuf[u][j], A.scale_bf16);
                    float off = 128.0f + (float)((zw >> (4 * j)) & 15u);
#pragma unroll
                    for (int q = 0; q < 4; q++) acc[j][q] = fmaf(sc, ag[j][q] - off * as[q], acc[j][q]);
                    ag[j] = v4f{0.f, 0.f, 0.f, 0.f};
                }
                as = v4f{0.f, 0.f, 0.f, 0.f};
            }
        }
    }
#pragma unroll
    for (int j = 0; j < J; j++) part[wave][j][lane] = acc[j];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int j = 0; j < J; j++) {
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

// GPTQ layout with the group length fixed at compile time (STEPS = G / 32).
// Same tile and lane mapping as int4_gptq_kernel; a load batch holds GPB whole
// groups (GPB * STEPS 32-k steps), so the per-group fold needs no per-step
// test, and the wave's group range is derived from a scalar wave index so
// that all step and group addressing stays on the scalar unit.
template <int KS, int J, int STEPS>
__global__ __launch_bounds__(64 * KS) void int4_gptq_fixed_kernel(Int4Args A) {
    constexpr int GPB = STEPS >= 8 ? 1 : 8 / STEPS;
    __shared__ v4f part[KS][J][64];
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t g = lane >> 4, rr = lane & 15;
    const uint32_t per_xcd = gridDim.x / 8;
    const uint32_t tile = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    const uint32_t n0 = tile * (16 * J);
    if (n0 >= A.N) return;
    const uint32_t m0 = blockIdx.y * 16;
    const uint32_t tok = m0 + rr;
    const uint32_t N = A.N;
    const uint32_t ngroups = A.K / (32 * STEPS);
    const uint32_t per = (ngroups + KS - 1) / KS;
    const uint32_t g0 = min(ngroups, wave * per), g1 = min(ngroups, g0 + per);
    const uint32_t col = n0 + J * rr;
    const bool tv = tok < A.B;
    // Lane bases: packed row 4 i + g of step i is wq + i * 4 N; activations
    // of step i start at xq + 32 i.
    const uint32_t* wq = A.qw + (uint64_t)g * N + col;
    const uint16_t* xq = A.x + (uint64_t)(tv ? tok : 0) * A.K + 8 * g;
    const uint16_t* sq = A.scales + col;
    const uint32_t* zq = A.qzeros ? A.qzeros + col / 8 : nullptr;
    const uint32_t zshift = 4 * (col % 8);
    v4f acc[J];
#pragma unroll
    for (int j = 0; j < J; j++) acc[j] = v4f{0.f, 0.f, 0.f, 0.f};
    const v4i ones = v4i{(int)ONES_BF16, (int)ONES_BF16, (int)ONES_BF16, (int)ONES_BF16};
    for (uint32_t grp = g0; grp < g1; grp += GPB) {
        uint32_t wbuf[GPB][STEPS][J], zbuf[GPB];
        uint16_t sbuf[GPB][J];
        v4i abuf[GPB][STEPS];
#pragma unroll
        for (int gb = 0; gb < GPB; gb++) {
            const uint32_t gi = min(grp + gb, g1 - 1);
#pragma unroll
            for (int st = 0; st < STEPS; st++) {
                const uint32_t i = gi * STEPS + st;
                load_words<J>(wq + (uint64_t)i * 4 * N, wbuf[gb][st]);
                abuf[gb][st] = tv ? *reinterpret_cast<const v4i*>(xq + 32 * i) : v4i{0, 0, 0, 0};
            }
#pragma unroll
            for (int j = 0; j < J; j++) sbuf[gb][j] = sq[(uint64_t)gi * N + j];
            zbuf[gb] = zq ? zq[(uint64_t)gi * (N / 8)] >> zshift : 0x8888u;
        }
#pragma unroll
        for (int gb = 0; gb < GPB; gb++) {
            if (grp + gb >= g1) continue;
            v4f ag[J], as = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < J; j++) ag[j] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < STEPS; st++) {
                v4i ap = permute_act(abuf[gb][st]);
#pragma unroll
                for (int j = 0; j < J; j++) ag[j] = mfma_bf16(ap, dequant_word(wbuf[gb][st][j]), ag[j]);
                as = mfma_bf16(ap, ones, as);
            }
#pragma unroll
            for (int j = 0; j < J; j++) {
                const float sc = decode_scale(sbuf[gb][j], A.scale_bf16);
                const float off = 128.0f + (float)((zbuf[gb] >> (4 * j)) & 15u);
#pragma unroll
                for (int q = 0; q < 4; q++) acc[j][q] = fmaf(sc, ag[j][q] - off * as[q], acc[j][q]);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < J; j++) part[wave][j][lane] = acc[j];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int j = 0; j < J; j++) {
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

// Decode-sized GPTQ linear (M <= GEMV_MAX_M tokens).  The kernel is shaped
// for the weight stream: a block owns 64 columns and its 16 waves split the
// packed rows in batches of 32, each wave issuing every load of its batch up
// front.  Weights are read 16 bytes per lane: lane (q = l / 16, c = l % 16)
// loads columns 4c..4c+3 of packed rows 4i + q (i = 0..7) of the batch, so one
// load instruction covers four whole 256-byte row segments (a dword per lane
// would take four times the instructions and memory requests for the bytes).
//
// The loaded words are exactly the B operand of v_mfma_f32_16x16x32_bf16
// (lane (q, c) = k-slice q of column c) once each 4-bit code is turned into
// the bf16 value 128 + q (one and-or per two codes), so MFMA j of step i
// contracts columns 4c + j; A row c is token min(c, M - 1), and only result
// rows t < M are read.  The matrix core does the multiply-adds that would
// otherwise cost four v_dot2 per word per token; the vector ALU is left with
// the code expansion.  As in the other kernels
//   sum_k x (q - z) = sum_k x (128 + q) - (128 + z) sum_k x
// per group, with sum_k x from shuffles over the activation slice.
//
// Loads go oldest first in the order they are needed (the wave's activation
// slice, group scales and zero codes, then the packed words), so the wave
// waits for the slice alone and then contracts each load as it lands.  The
// slice is permuted into pair order and parked in the wave's own LDS region;
// the 16 waves' partial sums meet in LDS.
constexpr uint32_t GEMV_MAX_M = 4;
constexpr uint32_t GEMV_ROWS = 32;       // packed rows per wave batch (256 k)

typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2bf, a), __builtin_bit_cast(v2bf, b), c, false);
}

__device__ __forceinline__ float sum8_bf16(v4i v) {
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < 4; q++)
        s += bf16_to_f32((uint16_t)((uint32_t)v[q] & 0xFFFFu)) + bf16_to_f32((uint16_t)((uint32_t)v[q] >> 16));
    return s;
}

template <int KS, int G, bool ZP, uint32_t MT>
__global__ __launch_bounds__(64 * KS) void int4_gptq_gemv_kernel(Int4Args A) {
    constexpr uint32_t GR = G / 8;                 // packed rows per group
    constexpr uint32_t GPB = GEMV_ROWS / GR;       // groups per batch
    constexpr uint32_t LR = GEMV_ROWS / 4;         // packed rows per lane per batch
    static_assert(GR % 4 == 0 && GR <= GEMV_ROWS && GEMV_ROWS % GR == 0, "group length must divide the batch");
    __shared__ v4i xw[KS][MT][GEMV_ROWS];
    __shared__ v4f part[KS][MT][16];
    const uint32_t K = A.K, N = A.N, M = A.B, prow = K / 8;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lane = threadIdx.x & 63, lr = lane & (GEMV_ROWS - 1);
    const uint32_t q = lane >> 4, c = lane & 15;
    const uint32_t per_xcd = gridDim.x / 8;
    const uint32_t tile = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    const uint32_t n0 = tile * 64;
    if (n0 >= N) return;
    const uint32_t col = n0 + 4 * c;               // first of the lane's 4 columns
    const uint32_t ngroups = K / G;
    const uint32_t nbatch = (ngroups + GPB - 1) / GPB;
    const uint32_t per = (nbatch + KS - 1) / KS;
    const uint32_t b0 = min(nbatch, wave * per), b1 = min(nbatch, b0 + per);
    const uint32_t zshift = 4 * (col % 8);
    v4f acc[MT];
#pragma unroll
    for (uint32_t t = 0; t < MT; t++) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
    for (uint32_t b = b0; b < b1; b++) {
        const uint32_t grp0 = b * GPB, row0 = grp0 * GR;
        // Loads, oldest first.
        v4i xl[MT];
#pragma unroll
        for (uint32_t t = 0; t < MT; t++)
            xl[t] = *reinterpret_cast<const v4i*>(A.x + (uint64_t)min(t, M - 1) * K + 8 * min(row0 + lr, prow - 1));
        v2i sb[GPB];
        uint32_t zb[GPB];
#pragma unroll
        for (uint32_t gb = 0; gb < GPB; gb++) {
            const uint32_t gi = min(grp0 + gb, ngroups - 1);
            sb[gb] = *reinterpret_cast<const v2i*>(A.scales + (uint64_t)gi * N + col);
            zb[gb] = ZP ? A.qzeros[(uint64_t)gi * (N / 8) + col / 8] >> zshift : 0x8888u;
        }
        // Scheduling fences keep the issue order (the compiler would otherwise
        // hoist the packed-word loads ahead and then drain them all for the
        // slice).
        __builtin_amdgcn_sched_barrier(0);
        v4i w[LR];
#pragma unroll
        for (uint32_t i = 0; i < LR; i++)
            w[i] = *reinterpret_cast<const v4i*>(A.qw + (uint64_t)min(row0 + 4 * i + q, prow - 1) * N + col);
        __builtin_amdgcn_sched_barrier(0);
        // Activation slice: pair order into LDS (lane lr holds row row0 + lr;
        // lanes 32..63 mirror lanes 0..31), and per-group sums of the slice.
        float gsum[MT][GPB];
#pragma unroll
        for (uint32_t t = 0; t < MT; t++) {
            if (lane < GEMV_ROWS) xw[wave][t][lr] = permute_act(xl[t]);
            float v = sum8_bf16(xl[t]);
            v = lanes_sum_up<GR>(v);   // the __shfl_xor butterfly 1, 2, ..., GR / 2
#pragma unroll
            for (uint32_t gb = 0; gb < GPB; gb++) gsum[t][gb] = lane_bcast(v, gb * GR);
        }
        __builtin_amdgcn_wave_barrier();
        // MFMA j of step i contracts packed rows 4 i .. 4 i + 3 (k-slice q)
        // of columns 4 c + j against the activations: A row c is token
        // min(c, M - 1), so result rows t < M are the tokens and the rest are
        // never read.  Result lane (0, c) holds D[t][4 c + j] in element t.
        const uint32_t tsel = min(c, M - 1);
#pragma unroll
        for (uint32_t gb = 0; gb < GPB; gb++) {
            if (grp0 + gb >= ngroups) continue;
            v4f ag[4];
#pragma unroll
            for (uint32_t j = 0; j < 4; j++) ag[j] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (uint32_t i = gb * (GR / 4); i < (gb + 1) * (GR / 4); i++) {
                const v4i xv = xw[wave][tsel][4 * i + q];
#pragma unroll
                for (uint32_t j = 0; j < 4; j++) ag[j] = mfma_bf16(xv, dequant_word((uint32_t)w[i][j]), ag[j]);
            }
#pragma unroll
            for (uint32_t j = 0; j < 4; j++) {
                const uint32_t sbits = (uint32_t)sb[gb][j / 2] >> (16 * (j % 2));
                const float sc = decode_scale((uint16_t)(sbits & 0xFFFFu), A.scale_bf16);
                const float off = 128.0f + (float)((zb[gb] >> (4 * j)) & 15u);
#pragma unroll
                for (uint32_t t = 0; t < MT; t++) acc[t][j] = fmaf(sc, ag[j][t] - off * gsum[t][gb], acc[t][j]);
            }
        }
        __builtin_amdgcn_wave_barrier();
    }
#pragma unroll
    for (uint32_t t = 0; t < MT; t++)
        if (lane < 16) part[wave][t][lane] = acc[t];
    __syncthreads();
    if (wave != 0) return;
    const float* pf = reinterpret_cast<const float*>(&part[0][0][0]);
    for (uint32_t t = 0; t < M; t++) {
        float v = pf[t * 64 + lane];
#pragma unroll
        for (int w2 = 1; w2 < KS; w2++) v += pf[(w2 * MT + t) * 64 + lane];
        finalize_store(A, t, n0 + lane, v);
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
    v4f ag = v4f{0.f, 0.f, 0.f, 0.f}, as = v4f{0.f, 0.f, 0.f, 0.f};
    // 128-k steps run in batches of CT_BATCH with every load of a batch issued
    // before its first MFMA; a group is scaled and folded into acc after its
    // last step.
    constexpr uint32_t CT_BATCH = 4;
    const uint32_t first = g0 * steps, last = g1 * steps;
    for (uint32_t base = first; base < last; base += CT_BATCH) {
        v4i wbuf[CT_BATCH], abuf[CT_BATCH][4];
#pragma unroll
        for (uint32_t u = 0; u < CT_BATCH; u++) {
            const uint32_t kb = min(base + u, last - 1) * 128;
            wbuf[u] = *reinterpret_cast<const v4i*>(wrow + kb / 8 + 4 * g);
            const uint16_t* xa = xrow + kb + 32 * g;
#pragma unroll
            for (int j = 0; j < 4; j++) abuf[u][j] = tv ? *reinterpret_cast<const v4i*>(xa + 8 * j) : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (uint32_t u = 0; u < CT_BATCH; u++) {
            const uint32_t i = base + u;
            if (i >= last) break;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                v4i ap = permute_act(abuf[u][j]);
                uint32_t wj = (uint32_t)(j == 0 ? wbuf[u].x : j == 1 ? wbuf[u].y : j == 2 ? wbuf[u].z : wbuf[u].w);
                ag = mfma_bf16(ap, dequant_word(wj), ag);
                as = mfma_bf16(ap, v4i{(int)ONES_BF16, (int)ONES_BF16, (int)ONES_BF16, (int)ONES_BF16}, as);
            }
            if ((i + 1) % steps == 0) {
                float sc = load_scale(A.scales + (uint64_t)n * ngroups + i / steps, A.scale_bf16);
#pragma unroll
                for (int q = 0; q < 4; q++) acc[q] = fmaf(sc, ag[q] - 136.0f * as[q], acc[q]);
                ag = v4f{0.f, 0.f, 0.f, 0.f};
                as = v4f{0.f, 0.f, 0.f, 0.f};
            }
        }
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

// ---------------------------------------------------------------------------
// Pair-packed INT8 activations (quantize_int8_symmetric_pairpacked.comp.
// template:22-72): per 32 columns s = amax > 0 ? amax / 127 : 1,
// q = round-half-even(clamp(x / s, -127, 127)) and the block sum of q.  A
// thread owns 8 columns c..c+7 and writes the words (q[c], q[c+2], q[c+4],
// q[c+6]) and (q[c+1], q[c+3], q[c+5], q[c+7]); the 4 threads of a block are
// consecutive lanes.
// ---------------------------------------------------------------------------
// SILU: silu_multiply_quantize_int8_pairpacked.comp.template: the values are
// y = bf16(bf16(g / (1 + exp(-g))) * u) of the gate (x) and up rows, and y is
// written out as well.
template <bool SILU, bool PAIRED = true>
__global__ __launch_bounds__(256) void quant_i8pp_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ up,
                                                         uint16_t* __restrict__ y, uint32_t rows, uint32_t cols,
                                                         uint32_t* __restrict__ q, float* __restrict__ s,
                                                         int32_t* __restrict__ sums) {
    const uint32_t oct = blockIdx.x * 256 + threadIdx.x, per_row = cols / 8;
    const bool ok = oct < rows * per_row;
    const uint32_t o = ok ? oct : 0u;
    const v4i v = *reinterpret_cast<const v4i*>(x + (uint64_t)o * 8);
    float f[8];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        f[2 * e] = bf16_to_f32((uint32_t)v[e]);
        f[2 * e + 1] = bf16_to_f32((uint32_t)v[e] >> 16);
    }
    if (SILU) {
        const v4i uv = *reinterpret_cast<const v4i*>(up + (uint64_t)o * 8);
        uint32_t yb[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float act = round_bf16(f[e] / (1.0f + expf(-f[e])));
            yb[e] = f32_to_bf16(act * bf16_to_f32((uint32_t)uv[e / 2] >> (16 * (e & 1)))) & 0xffffu;
            f[e] = bf16_to_f32(yb[e]);
        }
        if (ok)
            *reinterpret_cast<v4i*>(y + (uint64_t)o * 8) = v4i{(int)(yb[0] | (yb[1] << 16)), (int)(yb[2] | (yb[3] << 16)),
                                                               (int)(yb[4] | (yb[5] << 16)), (int)(yb[6] | (yb[7] << 16))};
    }
    float m = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) m = fmaxf(m, fabsf(f[e]));
    m = fmaxf(m, __shfl_xor(m, 1));
    m = fmaxf(m, __shfl_xor(m, 2));
    const float sc = m > 0.0f ? m / 127.0f : 1.0f;
    int iv[8], sum = 0;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        iv[e] = (int)__builtin_rintf(fminf(fmaxf(f[e] / sc, -127.0f), 127.0f));
        sum += iv[e];
    }
    sum += __shfl_xor(sum, 1);
    sum += __shfl_xor(sum, 2);
    if (!ok) return;
    // pair-packed: (q[c], q[c+2], q[c+4], q[c+6]), (q[c+1], ...); unpaired:
    // the 8 codes in column order
    const int a0 = PAIRED ? 0 : 0, a1 = PAIRED ? 2 : 1, a2 = PAIRED ? 4 : 2, a3 = PAIRED ? 6 : 3;
    const int b0 = PAIRED ? 1 : 4, b1 = PAIRED ? 3 : 5, b2 = PAIRED ? 5 : 6, b3 = PAIRED ? 7 : 7;
    const uint32_t w0 = (uint32_t)(iv[a0] & 255) | ((uint32_t)(iv[a1] & 255) << 8) | ((uint32_t)(iv[a2] & 255) << 16) |
                        ((uint32_t)(iv[a3] & 255) << 24);
    const uint32_t w1 = (uint32_t)(iv[b0] & 255) | ((uint32_t)(iv[b1] & 255) << 8) | ((uint32_t)(iv[b2] & 255) << 16) |
                        ((uint32_t)(iv[b3] & 255) << 24);
    *reinterpret_cast<uint2*>(q + (uint64_t)o * 2) = uint2{w0, w1};
    if ((o & 3u) == 0) {
        s[o / 4] = sc;
        if (sums) sums[o / 4] = sum;
    }
}

// ---------------------------------------------------------------------------
// Pair-packed INT8 x GPTQ INT4 linear (linear_prequant_pairpacked_int4_gptq.
// comp.template:56-95).  Lane = output column (64 per block), the 4 waves
// split the weight groups; per 32-column block the integer dot is exact
// (v_dot4_i32_i8 on the bytes (q - 0) of the packed word's low and high
// nibbles against the even and odd activation words, minus 8 times the block
// sum), then acc = fma(dot, s_x * s_w, acc).  Only the f32 accumulation order
// differs from the shader (per-wave partials added in wave order).
// ---------------------------------------------------------------------------
struct PpArgs {
    const uint32_t* q;          // int8 words [B, K/4], pair-packed
    const float* s;             // [B, K/32]
    const int32_t* sums;        // [B, K/32]
    Int4Args L;                 // qweight, scales, aux, y, shapes
};

// Unpaired input (linear_prequant_int4_{gptq,ct}.comp.template): the int8
// words hold columns in order, so each packed weight word becomes the signed
// bytes (code - 8) of nibbles 0..3 and 4..7 for two v_dot4_i32_i8.
__device__ __forceinline__ int nibbles_to_i8x4(uint32_t t16) {
    uint32_t b = (t16 & 0xFu) | ((t16 & 0xF0u) << 4) | ((t16 & 0xF00u) << 8) | ((t16 & 0xF000u) << 12);
    b ^= 0x08080808u;                       // code - 8 as a 4-bit two's complement value
    return (int)(b | ((b & 0x08080808u) * 0x1Eu));   // sign-extend each byte
}

template <bool PAIRED, bool CT>
__global__ __launch_bounds__(256) void int4_pp_kernel(PpArgs P) {
    __shared__ float red[4][64];
    const Int4Args& A = P.L;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const uint32_t K = A.K, N = A.N, G = A.G, ngroups = K / G, bpg = G / 32, nblk = K / 32;
    const uint32_t n = blockIdx.x * 64 + lane;
    const uint32_t nc = n < N ? n : N - 1;
    const uint32_t per = (ngroups + 3) / 4, g0 = min(ngroups, wave * per), g1 = min(ngroups, g0 + per);
    for (uint32_t t = 0; t < A.B; t++) {
        const uint32_t* qt = P.q + (uint64_t)t * (K / 4);
        float acc = 0.0f;
        for (uint32_t g = g0; g < g1; g++) {
            const float sw = decode_scale(CT ? A.scales[(uint64_t)nc * ngroups + g] : A.scales[(uint64_t)g * N + nc],
                                          A.scale_bf16);
            for (uint32_t b = g * bpg; b < (g + 1) * bpg; b++) {
                int dot = PAIRED ? -8 * P.sums[(uint64_t)t * nblk + b] : 0;
#pragma unroll
                for (uint32_t p = 0; p < 4; p++) {
                    const uint32_t word = CT ? A.qw[(uint64_t)nc * (K / 8) + b * 4 + p] : A.qw[(uint64_t)(b * 4 + p) * N + nc];
                    if (PAIRED) {
                        dot = __builtin_amdgcn_sdot4((int)qt[(b * 4 + p) * 2], (int)(word & 0x0f0f0f0fu), dot, false);
                        dot = __builtin_amdgcn_sdot4((int)qt[(b * 4 + p) * 2 + 1], (int)((word >> 4) & 0x0f0f0f0fu), dot,
                                                     false);
                    } else {
                        dot = __builtin_amdgcn_sdot4((int)qt[(b * 4 + p) * 2], nibbles_to_i8x4(word & 0xffffu), dot, false);
                        dot = __builtin_amdgcn_sdot4((int)qt[(b * 4 + p) * 2 + 1], nibbles_to_i8x4(word >> 16), dot, false);
                    }
                }
                acc = fmaf((float)dot, P.s[(uint64_t)t * nblk + b] * sw, acc);
            }
        }
        red[wave][lane] = acc;
        __syncthreads();
        if (wave == 0 && n < N) finalize_store(A, t, n, ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane]);
        __syncthreads();
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
    if (s.input != 0)
        return nh::fail(NERVE_HIP_INVALID_SPEC, "INT8-prequantized input goes through nerve_hip_int4_linear_pairpacked");
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
        if (A.N % 16) return nh::fail(NERVE_HIP_UNSUPPORTED, "GPTQ INT4 kernel needs N % 16 == 0");
        if (zeros && A.N % 8) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "qzeros need N % 8 == 0");
        // 64-column tiles (8 KiB of weights in flight per wave per batch);
        // N % 64 != 0 uses 16-column tiles with deeper batches.
        const uint32_t row_tiles = (batch_width + 15) / 16;
        const bool wide = A.N % 64 == 0;
        const uint32_t tiles = wide ? A.N / 64 : A.N / 16;
        dim3 grid((tiles + 7) / 8 * 8, row_tiles);
        const uint32_t steps = A.G / 32;
        // Decode-sized batches go to the vector-ALU kernel.
        if (wide && batch_width <= GEMV_MAX_M && (A.G == 32 || A.G == 64 || A.G == 128 || A.G == 256) &&
            ((uintptr_t)scales & 7) == 0) {
            dim3 g1((tiles + 7) / 8 * 8);
            const bool zp = zeros != nullptr;
#define NERVE_INT4_GEMV(GG)                                                                   \
    (batch_width == 1 ? (zp ? int4_gptq_gemv_kernel<16, GG, true, 1><<<g1, 1024, 0, strm>>>(A)   \
                            : int4_gptq_gemv_kernel<16, GG, false, 1><<<g1, 1024, 0, strm>>>(A)) \
                      : (zp ? int4_gptq_gemv_kernel<16, GG, true, 4><<<g1, 1024, 0, strm>>>(A)   \
                            : int4_gptq_gemv_kernel<16, GG, false, 4><<<g1, 1024, 0, strm>>>(A)))
            if (A.G == 128) NERVE_INT4_GEMV(128);
            else if (A.G == 64) NERVE_INT4_GEMV(64);
            else if (A.G == 32) NERVE_INT4_GEMV(32);
            else NERVE_INT4_GEMV(256);
#undef NERVE_INT4_GEMV
            return nh::check_launch("int4_linear_gptq_gemv");
        }
        // Few column tiles (decode-sized N): 16 waves split K so that each
        // wave's share is one load batch.
        const bool deep = tiles * row_tiles < 2u * (uint32_t)ctx->cu_count;
        if (wide && steps == 4 && deep) int4_gptq_fixed_kernel<16, 4, 4><<<grid, 1024, 0, strm>>>(A);
        else if (wide && steps == 4) int4_gptq_fixed_kernel<8, 4, 4><<<grid, 512, 0, strm>>>(A);
        else if (wide && steps == 1) int4_gptq_fixed_kernel<8, 4, 1><<<grid, 512, 0, strm>>>(A);
        else if (wide && steps == 2) int4_gptq_fixed_kernel<8, 4, 2><<<grid, 512, 0, strm>>>(A);
        else if (wide && steps == 8) int4_gptq_fixed_kernel<8, 4, 8><<<grid, 512, 0, strm>>>(A);
        else if (!wide && steps == 4) int4_gptq_fixed_kernel<8, 1, 4><<<grid, 512, 0, strm>>>(A);
        else if (wide) int4_gptq_kernel<8, 4, 8><<<grid, 512, 0, strm>>>(A);
        else int4_gptq_kernel<8, 1, 16><<<grid, 512, 0, strm>>>(A);
        return nh::check_launch("int4_linear_gptq");
    }
    if (zeros) return nh::fail(NERVE_HIP_UNSUPPORTED, "asymmetric zeros are supported for the GPTQ layout only");
    if (A.G % 128 || A.N % 16) return nh::fail(NERVE_HIP_UNSUPPORTED, "CT INT4 kernel needs group % 128 == 0 and N % 16 == 0");
    dim3 grid(A.N / 16, (batch_width + 15) / 16);
    int4_ct_kernel<8><<<grid, 512, 0, strm>>>(A);
    return nh::check_launch("int4_linear_ct");
}

extern "C" nerve_hip_status nerve_hip_quantize_int8_pairpacked(nerve_hip_ctx* ctx, const char* spec, const void* x_bf16,
                                                              void* q_i8, void* scales_f32, void* sums_i32,
                                                              uint32_t rows, void* stream) {
    nerve_hip_status st = nh::enter(ctx);
    if (st) return st;
    nh::QuantI8Spec qs;
    if ((st = nh::parse_quant_i8_spec(spec, &qs))) return st;
    if (qs.silu) return nh::fail(NERVE_HIP_INVALID_SPEC, "silu_multiply_quantize goes through its own entry point");
    if (!x_bf16 || !q_i8 || !scales_f32 || (qs.paired && !sums_i32))
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "null buffer");
    if (qs.batch_tile == 0 && rows > 1)
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "unbatched pair-packed quantizer takes one row");
    if (((uintptr_t)x_bf16 & 15) || ((uintptr_t)q_i8 & 7))
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "x must be 16-byte and q 8-byte aligned");
    if (rows == 0) return nh::ok();
    const uint64_t octs = (uint64_t)rows * qs.elements / 8;
    const uint32_t grid = (uint32_t)((octs + 255) / 256);
    if (qs.paired)
        quant_i8pp_kernel<false, true><<<grid, 256, 0, (hipStream_t)stream>>>(
            static_cast<const uint16_t*>(x_bf16), nullptr, nullptr, rows, qs.elements, static_cast<uint32_t*>(q_i8),
            static_cast<float*>(scales_f32), static_cast<int32_t*>(sums_i32));
    else
        quant_i8pp_kernel<false, false><<<grid, 256, 0, (hipStream_t)stream>>>(
            static_cast<const uint16_t*>(x_bf16), nullptr, nullptr, rows, qs.elements, static_cast<uint32_t*>(q_i8),
            static_cast<float*>(scales_f32), static_cast<int32_t*>(sums_i32));
    return nh::check_launch("quantize_int8");
}

extern "C" nerve_hip_status nerve_hip_silu_multiply_quantize_int8_pairpacked(nerve_hip_ctx* ctx, const char* spec,
                                                                            const void* gate_bf16, const void* up_bf16,
                                                                            void* y_bf16, void* q_i8, void* scales_f32,
                                                                            void* sums_i32, uint32_t rows,
                                                                            void* stream) {
    nerve_hip_status st = nh::enter(ctx);
    if (st) return st;
    nh::QuantI8Spec qs;
    if ((st = nh::parse_quant_i8_spec(spec, &qs))) return st;
    if (!qs.silu) return nh::fail(NERVE_HIP_INVALID_SPEC, "not a silu_multiply_quantize specialization");
    if (!gate_bf16 || !up_bf16 || !y_bf16 || !q_i8 || !scales_f32 || !sums_i32)
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "null buffer");
    if (qs.batch_tile == 0 && rows > 1)
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "unbatched pair-packed quantizer takes one row");
    if ((((uintptr_t)gate_bf16) | ((uintptr_t)up_bf16) | ((uintptr_t)y_bf16)) & 15 || ((uintptr_t)q_i8 & 7))
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "gate, up and y must be 16-byte and q 8-byte aligned");
    if (rows == 0) return nh::ok();
    // The kernel reads gate and up through restrict pointers while it writes
    // y: y may not overlap either input.
    const uintptr_t bytes = (uintptr_t)rows * qs.elements * 2, yb = (uintptr_t)y_bf16;
    auto overlaps = [&](const void* p) { const uintptr_t a = (uintptr_t)p; return a < yb + bytes && yb < a + bytes; };
    if (overlaps(gate_bf16) || overlaps(up_bf16))
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "y must not overlap gate or up");
    const uint64_t octs = (uint64_t)rows * qs.elements / 8;
    quant_i8pp_kernel<true><<<(uint32_t)((octs + 255) / 256), 256, 0, (hipStream_t)stream>>>(
        static_cast<const uint16_t*>(gate_bf16), static_cast<const uint16_t*>(up_bf16), static_cast<uint16_t*>(y_bf16),
        rows, qs.elements, static_cast<uint32_t*>(q_i8), static_cast<float*>(scales_f32),
        static_cast<int32_t*>(sums_i32));
    return nh::check_launch("silu_multiply_quantize_int8_pairpacked");
}

extern "C" nerve_hip_status nerve_hip_int4_linear_pairpacked(nerve_hip_ctx* ctx, const char* spec, const void* q_i8,
                                                            const void* scales_f32, const void* sums_i32,
                                                            const void* qweight, const void* scales,
                                                            const void* aux_bf16, void* y_bf16, uint32_t batch_width,
                                                            void* stream) {
    nerve_hip_status st = nh::enter(ctx);
    if (st) return st;
    nh::Int4Spec s;
    if ((st = nh::parse_int4_spec(spec, &s))) return st;
    if (s.input == 0) return nh::fail(NERVE_HIP_INVALID_SPEC, "not a _prequant[_pairpacked] INT4 specialization");
    const bool paired = s.input == 2;
    if (!q_i8 || !scales_f32 || (paired && !sums_i32) || !qweight || !scales || !y_bf16)
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "null buffer");
    if (s.op != 0 && !aux_bf16) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "bias/residual specialization needs aux");
    if (s.batch_tile == 0 && batch_width > 1)
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "unbatched INT4 specialization takes batch_width 1");
    if (((uintptr_t)q_i8 & 3) || ((uintptr_t)qweight & 3))
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "q and qweight must be 4-byte aligned");
    if (batch_width == 0) return nh::ok();
    PpArgs P;
    P.q = static_cast<const uint32_t*>(q_i8);
    P.s = static_cast<const float*>(scales_f32);
    P.sums = static_cast<const int32_t*>(sums_i32);
    P.L.x = nullptr;
    P.L.qw = static_cast<const uint32_t*>(qweight);
    P.L.scales = static_cast<const uint16_t*>(scales);
    P.L.qzeros = nullptr;
    P.L.aux = static_cast<const uint16_t*>(aux_bf16);
    P.L.y = static_cast<uint16_t*>(y_bf16);
    P.L.B = batch_width;
    P.L.K = s.in;
    P.L.N = s.out;
    P.L.G = s.group;
    P.L.scale_bf16 = s.scale_bf16;
    P.L.finalize = s.op;
    const uint32_t grid = (s.out + 63) / 64;
    hipStream_t strm = (hipStream_t)stream;
    if (paired) int4_pp_kernel<true, false><<<grid, 256, 0, strm>>>(P);
    else if (s.layout == 0) int4_pp_kernel<false, false><<<grid, 256, 0, strm>>>(P);
    else int4_pp_kernel<false, true><<<grid, 256, 0, strm>>>(P);
    return nh::check_launch("int4_linear_prequant");
}
