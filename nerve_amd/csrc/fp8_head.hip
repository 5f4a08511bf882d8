// FP8 e4m3 output projection (a10) with fused greedy argmax (a11).
//
// Reference: tied_output_projection_fp8_e4m3.comp.template:87-144 (and the
// _batch twin :94-186): the bf16 input is quantized per 128-column block with
// s = amax/448 (not a power of two), and
//   logit[n] = OUTPUT_SCALE * sum_b fma(dot(qx_b, W[n]_b), s_x[b] * s_w[n/BR, b])
// Here each 128-column block is one v_mfma_scale_f32_16x16x128_f8f6f4 with
// unit scales (e8m0 127); its f32 result is multiplied by s_x * s_w and
// accumulated, which is the same contraction with a different summation order.
// fp8 x fp8 operand pairing is the identity (both operands use the same lane
// layout), so each lane loads 32 contiguous bytes of its row for both.
//
// Argmax follows greedy_sampler_f32.comp.template:25-109: larger f32 logit
// wins, ties go to the lower token id.
#include <algorithm>
#include <cfloat>

#include "async_copy.h"
#include "common.h"

namespace nh {
nerve_hip_status quantize_rows(const uint16_t* x, uint32_t cols, uint32_t rows, bool pow2, uint8_t* q, float* s,
                               hipStream_t st, uint32_t* zero_word = nullptr);
}

namespace {

constexpr int HEAD_WAVES = 8;     // 8 waves x 16 columns = 128 columns per block
constexpr int HEAD_MT = 4;        // token sub-tiles (of 16) per wave

struct HeadArgs {
    const uint8_t* xq;            // e4m3 [M, K]
    const float* xs;              // f32 [M, nblk]
    const uint8_t* W;             // e4m3 [N, K]
    const uint16_t* scale_inv;    // bf16 [ceil(N/BR), nblk]
    uint32_t M, K, N, BR;
    float out_scale;
    float* logits_f32;            // [M, N] or null
    uint16_t* logits_bf16;        // [M, N] or null
    float* part_val;              // [M, nblocks] or null
    uint32_t* part_idx;
    uint32_t nblocks;
};

__device__ __forceinline__ bool better(float v, uint32_t i, float bv, uint32_t bi) {
    return v > bv || (v == bv && i < bi);
}

__global__ __launch_bounds__(64 * HEAD_WAVES) void fp8_head_kernel(HeadArgs A) {
    __shared__ float red_v[HEAD_WAVES][HEAD_MT * 16];
    __shared__ uint32_t red_i[HEAD_WAVES][HEAD_MT * 16];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t g = lane >> 4, rr = lane & 15;
    const uint32_t col = blockIdx.x * (16 * HEAD_WAVES) + wave * 16 + rr;
    const bool cv = col < A.N;
    const uint32_t m_base = blockIdx.y * (16 * HEAD_MT);
    const uint32_t K = A.K, nblk = (K + 127) / 128;
    const uint8_t* wrow = A.W + (uint64_t)(cv ? col : 0) * K;
    const uint16_t* srow = A.scale_inv + (uint64_t)((cv ? col : 0) / A.BR) * nblk;
    const uint8_t* arow[HEAD_MT];
    bool av[HEAD_MT];
#pragma unroll
    for (int mt = 0; mt < HEAD_MT; mt++) {
        uint32_t t = m_base + mt * 16 + rr;
        av[mt] = t < A.M;
        arow[mt] = A.xq + (uint64_t)(av[mt] ? t : 0) * K;
    }
    v4f acc[HEAD_MT];
#pragma unroll
    for (int mt = 0; mt < HEAD_MT; mt++) acc[mt] = v4f{0.f, 0.f, 0.f, 0.f};
    for (uint32_t c = 0; c < nblk; c++) {
        const uint32_t k0 = c * 128 + 32 * g;
        const bool kv = k0 < K;
        v4i b0 = v4i{0, 0, 0, 0}, b1 = v4i{0, 0, 0, 0};
        if (cv && kv) {
            b0 = *reinterpret_cast<const v4i*>(wrow + k0);
            b1 = *reinterpret_cast<const v4i*>(wrow + k0 + 16);
        }
        v8i b = v8i{b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
        const float sw = cv ? bf16_to_f32(srow[c]) : 0.0f;
#pragma unroll
        for (int mt = 0; mt < HEAD_MT; mt++) {
            if (m_base + mt * 16 >= A.M) break;
            v4i a0 = v4i{0, 0, 0, 0}, a1 = v4i{0, 0, 0, 0};
            if (av[mt] && kv) {
                a0 = *reinterpret_cast<const v4i*>(arow[mt] + k0);
                a1 = *reinterpret_cast<const v4i*>(arow[mt] + k0 + 16);
            }
            v8i a = v8i{a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
            v4f p = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, 127, 0,
                                                                     127);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                uint32_t t = m_base + mt * 16 + 4 * g + i;
                float sx = t < A.M ? A.xs[(uint64_t)t * nblk + c] : 0.0f;
                acc[mt][i] = fmaf(p[i], sx * sw, acc[mt][i]);
            }
        }
    }
    // Epilogue: logits and per-block argmax partials.
#pragma unroll
    for (int mt = 0; mt < HEAD_MT; mt++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t tl = mt * 16 + 4 * g + i;
            const uint32_t t = m_base + tl;
            const float v = acc[mt][i] * A.out_scale;
            if (t < A.M && cv) {
                if (A.logits_f32) A.logits_f32[(uint64_t)t * A.N + col] = v;
                if (A.logits_bf16) A.logits_bf16[(uint64_t)t * A.N + col] = (uint16_t)f32_to_bf16(v);
            }
            if (A.part_val) {
                float bv = cv ? v : -INFINITY;
                uint32_t bi = cv ? col : 0xffffffffu;
#pragma unroll
                for (int d = 1; d < 16; d <<= 1) {
                    float ov = __shfl_xor(bv, d);
                    uint32_t oi = __shfl_xor(bi, d);
                    if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
                }
                if (rr == 0) {
                    red_v[wave][tl] = bv;
                    red_i[wave][tl] = bi;
                }
            }
        }
    }
    if (!A.part_val) return;
    __syncthreads();
    if (threadIdx.x < HEAD_MT * 16) {
        const uint32_t tl = threadIdx.x, t = m_base + tl;
        if (t < A.M) {
            float bv = red_v[0][tl];
            uint32_t bi = red_i[0][tl];
            for (int w = 1; w < HEAD_WAVES; w++)
                if (better(red_v[w][tl], red_i[w][tl], bv, bi)) { bv = red_v[w][tl]; bi = red_i[w][tl]; }
            A.part_val[(uint64_t)t * A.nblocks + blockIdx.x] = bv;
            A.part_idx[(uint64_t)t * A.nblocks + blockIdx.x] = bi;
        }
    }
}


// ---------------------------------------------------------------------------
// Skinny form (M <= 16, the decode LM head): a pure weight stream.  A block of
// 4 waves owns one group of 16 vocabulary rows at a time and the waves split
// its K chunks; each wave holds its whole K slice of the group's weights in
// registers (two sets: the next group's loads are in flight while this one
// is contracted), the block's activations and block scales sit in LDS, and
// the 4 partial sums meet in LDS.  The grid is persistent (groups strided
// over the blocks).
// ---------------------------------------------------------------------------
constexpr int SK_WAVES = 4;

template <int CHW>
struct SkSet {
    v4i w[CHW][2];
    uint32_t s[CHW];
};

template <int CHW>
__global__ __launch_bounds__(64 * SK_WAVES) void fp8_head_skinny_kernel(HeadArgs A, uint32_t groups) {
    extern __shared__ __attribute__((aligned(16))) uint8_t sk_lds[];
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, rr = lane & 15;
    const uint32_t K = A.K, M = A.M, N = A.N, nblk = (K + 127) / 128;
    uint8_t* xa = sk_lds;
    float* xs = reinterpret_cast<float*>(sk_lds + (M * K + 15) / 16 * 16);
    float* red = xs + (M * nblk + 3) / 4 * 4;          // [3][64][4]
    for (uint32_t i = tid * 16; i < M * K; i += 64 * SK_WAVES * 16)
        *reinterpret_cast<v4i*>(xa + i) = *reinterpret_cast<const v4i*>(A.xq + i);
    for (uint32_t i = tid; i < M * nblk; i += 64 * SK_WAVES) xs[i] = A.xs[i];
    __syncthreads();
    float best_v[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    uint32_t best_i[4] = {0xffffffffu, 0xffffffffu, 0xffffffffu, 0xffffffffu};

    const uint32_t per = (nblk + SK_WAVES - 1) / SK_WAVES;
    const uint32_t c0 = min(nblk, wave * per), nc = min(per, nblk - c0);
    // Loads of one group's K slice (unconditional, clamped: out-of-range
    // pieces are zeroed after the fact, so every load is always issued).
    auto load = [&](SkSet<CHW>& S, uint32_t grp) __attribute__((always_inline)) {
        const uint32_t gg = grp < groups ? grp : groups - 1;
        const uint32_t n = min(gg * 16 + rr, N - 1);
        const uint8_t* wrow = A.W + (uint64_t)n * K;
        const uint16_t* srow = A.scale_inv + (uint64_t)(n / A.BR) * nblk;
#pragma unroll
        for (int q = 0; q < CHW; q++) {
            const uint32_t c = c0 + min((uint32_t)q, nc ? nc - 1 : 0u);
            const uint32_t k = min(c * 128 + 32 * g, K - 32);
            S.w[q][0] = *reinterpret_cast<const v4i*>(wrow + k);
            S.w[q][1] = *reinterpret_cast<const v4i*>(wrow + k + 16);
            S.s[q] = srow[c < nblk ? c : 0];
        }
    };
    auto compute = [&](const SkSet<CHW>& S, uint32_t grp) __attribute__((always_inline)) {
        const uint32_t n = grp * 16 + rr;
        v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int q = 0; q < CHW; q++) {
            if ((uint32_t)q >= nc) break;
            const uint32_t c = c0 + q, k = c * 128 + 32 * g;
            const bool kv = k < K;
            v4i a0 = v4i{0, 0, 0, 0}, a1 = v4i{0, 0, 0, 0};
            if (rr < M && kv) {
                a0 = *reinterpret_cast<const v4i*>(xa + rr * K + k);
                a1 = *reinterpret_cast<const v4i*>(xa + rr * K + k + 16);
            }
            const v4i b0 = kv ? S.w[q][0] : v4i{0, 0, 0, 0}, b1 = kv ? S.w[q][1] : v4i{0, 0, 0, 0};
            const v4f p = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                v8i{a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w}, v8i{b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w},
                v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, 127, 0, 127);
            const float sw = bf16_to_f32(S.s[q]);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t t = 4 * g + i;
                const float sx = t < M ? xs[t * nblk + c] : 0.0f;
                acc[i] = fmaf(p[i], sx * sw, acc[i]);
            }
        }
        if (wave > 0) *reinterpret_cast<v4f*>(red + ((wave - 1) * 64 + lane) * 4) = acc;
        __syncthreads();
        if (wave == 0) {
#pragma unroll
            for (int w = 0; w < SK_WAVES - 1; w++) {
                const v4f o = *reinterpret_cast<const v4f*>(red + (w * 64 + lane) * 4);
                acc += o;
            }
            const bool cv = n < N;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t t = 4 * g + i;
                const float v = acc[i] * A.out_scale;
                if (t < M && cv) {
                    if (A.logits_f32) A.logits_f32[(uint64_t)t * N + n] = v;
                    if (A.logits_bf16) A.logits_bf16[(uint64_t)t * N + n] = (uint16_t)f32_to_bf16(v);
                }
                if (A.part_val) {
                    float bv = cv ? v : -INFINITY;
                    uint32_t bi = cv ? n : 0xffffffffu;
#pragma unroll
                    for (int d = 1; d < 16; d <<= 1) {
                        const float ov = __shfl_xor(bv, d);
                        const uint32_t oi = __shfl_xor(bi, d);
                        if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
                    }
                    if (better(bv, bi, best_v[i], best_i[i])) {
                        best_v[i] = bv;
                        best_i[i] = bi;
                    }
                }
            }
        }
        __syncthreads();
    };
    const uint32_t G = gridDim.x;
    SkSet<CHW> s0, s1;
    load(s0, blockIdx.x);
    for (uint32_t grp = blockIdx.x; grp < groups; grp += 2 * G) {
        load(s1, grp + G);
        compute(s0, grp);
        load(s0, grp + 2 * G);
        if (grp + G < groups) compute(s1, grp + G);
    }
    if (!A.part_val) return;
    // One argmax partial per block and token (wave 0's lanes hold token
    // 4 g + i's best); argmax_partials_kernel reduces them.
    if (wave == 0 && rr == 0) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t t = 4 * g + i;
            if (t < M) {
                A.part_val[(uint64_t)t * G + blockIdx.x] = best_v[i];
                A.part_idx[(uint64_t)t * G + blockIdx.x] = best_i[i];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Stream form (M <= 16, per-row weight scales): one 8-wave block per CU over
// a contiguous range of 16-row vocabulary groups.  A group's weights are one
// contiguous 16 K-byte span of W and its scales one contiguous 32 nblk-byte
// span of scale_inv; both are copied into an NBUF-slot LDS ring by
// global_load_lds (1 KiB and 256 B per wave instruction), so every wave keeps
// NBUF - 1 groups of copies in flight while it contracts the current one.
// The tokens are the MFMA A operand and stay in registers for the whole
// range; each wave contracts its share of the K chunks of every group and the
// 8 partial sums meet in LDS, where waves 0..3 finalize token 4 g + wave.
// ---------------------------------------------------------------------------
constexpr int HS_NW = 8;
constexpr uint32_t HS_CH = 4;        // K chunks per wave (K <= 4096; the LDS wait below names 4)
constexpr uint32_t HS_LWMAX = 8;     // weight copies per wave per group (16 K <= 64 KiB)

struct HeadStream {
    uint32_t groups;
    uint32_t lw;                     // weight copies per wave per group
    uint32_t cpi;                    // copies per wave per group (weights + one scale copy)
    uint32_t slot_bytes, s_off;      // ring slot size; scale region offset in a slot
};

template <int NBUF>
__device__ __forceinline__ void fp8_head_stream_body(const HeadArgs& A, const HeadStream& S) {
    extern __shared__ __attribute__((aligned(16))) uint8_t ring[];
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lane = threadIdx.x & 63, g = lane >> 4, rr = lane & 15;
    const uint32_t K = A.K, M = A.M, N = A.N, nblk = (K + 127) / 128;
    const uint32_t G = gridDim.x, b = blockIdx.x;
    const uint32_t i0 = (uint32_t)((uint64_t)S.groups * b / G), i1 = (uint32_t)((uint64_t)S.groups * (b + 1) / G);
    uint8_t* red = ring + NBUF * S.slot_bytes;      // [wave][lane] v4f partial sums

    // ---- copy plan: piece t of this wave starts at byte wpos[t] of the
    // group's span (waves past the last piece repeat their first one, so
    // every wave issues lw copies).  The last piece is aligned to the span's
    // end and overlaps its neighbour with identical bytes.
    const uint32_t span = 16 * K, sspan = 32 * nblk;
    const uint32_t npw = (span + 1023) / 1024, nps = (sspan + 255) / 256;
    uint32_t wpos[HS_LWMAX], woff[HS_LWMAX];
#pragma unroll
    for (uint32_t t = 0; t < HS_LWMAX; t++) {
        uint32_t pc = wave + HS_NW * t;
        if (pc >= npw) pc = wave < npw ? wave : 0;
        wpos[t] = min(pc * 1024, span - 1024);
        woff[t] = wpos[t] + lane * 16;
    }
    const uint32_t spc = wave < nps ? wave : 0;
    const uint32_t spos = sspan >= 256 ? min(spc * 256, sspan - 256) : 0u;
    const uint32_t soff = spos + lane * 4;

    auto issue = [&](uint32_t item, uint32_t slot) __attribute__((always_inline)) {
        const uint32_t n0 = item * 16, rows = min(16u, N - n0);
        const uint32_t wbytes = rows * K, sbytes = (rows * nblk * 2 + 3) & ~3u;
        const uint8_t* ws = A.W + (uint64_t)n0 * K;
        uint8_t* dst = ring + slot * S.slot_bytes;
#pragma unroll
        for (uint32_t t = 0; t < HS_LWMAX; t++)
            if (t < S.lw)
                __builtin_amdgcn_global_load_lds(ws + (woff[t] < wbytes ? woff[t] : 0u), dst + wpos[t], 16, 0, 0);
        const uint8_t* ss = reinterpret_cast<const uint8_t*>(A.scale_inv) + (uint64_t)n0 * nblk * 2;
        __builtin_amdgcn_global_load_lds(ss + (soff < sbytes ? soff : 0u), dst + S.s_off + spos, 4, 0, 0);
    };

    // ---- this wave's K chunks and their LDS offsets
    const uint32_t per = (nblk + HS_NW - 1) / HS_NW;
    const uint32_t c0 = min(nblk, wave * per), c1 = min(nblk, c0 + per);
    uint32_t rw[HS_CH], rs[HS_CH];
    bool kvalid[HS_CH];
#pragma unroll
    for (uint32_t q = 0; q < HS_CH; q++) {
        const uint32_t c = c0 + q, kb = c * 128 + g * 32;
        kvalid[q] = c < c1 && kb < K;
        rw[q] = rr * K + (kvalid[q] ? kb : 0u);
        rs[q] = S.s_off + (rr * nblk + (c < c1 ? c : 0u)) * 2;
    }

    // ---- tokens: e4m3 operand pieces and block scales, loaded with
    // untracked loads before the first copies and waited for together with
    // the first group's copies (loads retire in issue order).  Quantizing
    // the tokens here instead would repeat the whole M x K quantization in
    // every block, vector-ALU work that outlasts the ring's first groups.
    const bool arow = rr < M;
    v4i xlo[HS_CH], xhi[HS_CH];
    uint32_t sxr[HS_CH][4];
    {
        const uint8_t* xr = A.xq + (uint64_t)(arow ? rr : 0u) * K;
#pragma unroll
        for (uint32_t q = 0; q < HS_CH; q++) {
            if (c0 + q >= c1) continue;                 // wave-uniform
            const uint32_t kb = kvalid[q] ? (c0 + q) * 128 + g * 32 : 0u;
            xlo[q] = gload16_untracked(xr + kb);
            xhi[q] = gload16_untracked(xr + kb + 16);
#pragma unroll
            for (uint32_t i = 0; i < 4; i++) {
                const uint32_t tk = 4 * g + i;
                sxr[q][i] = gload4_untracked(A.xs + (tk < M ? tk * nblk + c0 + q : 0u));
            }
        }
    }
    if (i0 >= i1) {
        wait_vm_imm<0>();
    } else {
        issue(i0, 0);
        wait_vm(S.cpi);
    }
    v8i av[HS_CH];
    float sx[HS_CH][4];
#pragma unroll
    for (uint32_t q = 0; q < HS_CH; q++) {
        av[q] = v8i{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) sx[q][i] = 0.0f;
        if (c0 + q >= c1) continue;
        asm volatile("" : "+v"(xlo[q]), "+v"(xhi[q]));
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) asm volatile("" : "+v"(sxr[q][i]));
        if (arow && kvalid[q])
            av[q] = v8i{xlo[q].x, xlo[q].y, xlo[q].z, xlo[q].w, xhi[q].x, xhi[q].y, xhi[q].z, xhi[q].w};
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) sx[q][i] = 4 * g + i < M ? __uint_as_float(sxr[q][i]) : 0.0f;
    }
    const uint32_t pro = min((uint32_t)NBUF, i1 - i0);
#pragma unroll
    for (uint32_t j = 1; j < NBUF; j++)
        if (j < pro) issue(i0 + j, j);

    const uint32_t tok = 4 * g + wave;                  // finalized token (waves 0..3)
    float best_v = -INFINITY;
    uint32_t best_i = 0xffffffffu;
    for (uint32_t i = i0; i < i1; i++) {
        const uint32_t slot = (i - i0) % NBUF;
        if (i > i0 && i + NBUF - 1 < i1) issue(i + NBUF - 1, (i - i0 + NBUF - 1) % NBUF);
        wait_vm(S.cpi * min((uint32_t)(NBUF - 1), i1 - 1 - i));
        __builtin_amdgcn_s_barrier();
        const uint8_t* buf = ring + slot * S.slot_bytes;
        v4i w0[HS_CH], w1[HS_CH];
        uint32_t sw[HS_CH];
#pragma unroll
        for (uint32_t q = 0; q < HS_CH; q++) {
            if (c0 + q >= c1) continue;
            w0[q] = lds_read16(buf + rw[q]);
            w1[q] = lds_read16(buf + rw[q] + 16);
            sw[q] = lds_read_u16(buf + rs[q]);
        }
        // The wait takes the read results as operands, so no copy of them
        // is scheduled in front of it.
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(w0[0]), "+v"(w1[0]), "+v"(sw[0]), "+v"(w0[1]), "+v"(w1[1]), "+v"(sw[1]), "+v"(w0[2]),
                       "+v"(w1[2]), "+v"(sw[2]), "+v"(w0[3]), "+v"(w1[3]), "+v"(sw[3])
                     :
                     : "memory");
        v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (uint32_t q = 0; q < HS_CH; q++) {
            if (c0 + q >= c1) continue;
            v4i b0 = w0[q], b1 = w1[q];
            uint32_t s16 = sw[q];
            if (!kvalid[q]) b0 = b1 = v4i{0, 0, 0, 0};
            const v4f p = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                av[q], v8i{b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w}, v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, 127,
                0, 127);
            const float s = bf16_to_f32(s16);
#pragma unroll
            for (int e = 0; e < 4; e++) acc[e] = fmaf(p[e], sx[q][e] * s, acc[e]);
        }
        // An MFMA result read by inline asm needs software wait states the
        // compiler does not add: the nops take the sums as operands.
        asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(acc));
        lds_write16(red + (wave * 64 + lane) * 16, acc);
        lds_drain();
        __builtin_amdgcn_s_barrier();
        if (wave >= 4) continue;
        uint32_t v[HS_NW];
#pragma unroll
        for (int w2 = 0; w2 < HS_NW; w2++) v[w2] = lds_read_b32(red + (w2 * 64 + lane) * 16 + 4 * wave);
        lds_drain();
        float sum = 0.0f;
#pragma unroll
        for (int w2 = 0; w2 < HS_NW; w2++) {
            asm volatile("" : "+v"(v[w2]));
            sum += __uint_as_float(v[w2]);
        }
        const float val = sum * A.out_scale;
        const uint32_t n = i * 16 + rr;
        const bool cv = n < N;
        if (tok < M && cv) {
            if (A.logits_f32) A.logits_f32[(uint64_t)tok * N + n] = val;
            if (A.logits_bf16) A.logits_bf16[(uint64_t)tok * N + n] = (uint16_t)f32_to_bf16(val);
        }
        if (A.part_val) {
            float bv = cv ? val : -INFINITY;
            uint32_t bi = cv ? n : 0xffffffffu;
#pragma unroll
            for (int d = 1; d < 16; d <<= 1) {
                const float ov = __shfl_xor(bv, d);
                const uint32_t oi = __shfl_xor(bi, d);
                if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
            }
            if (better(bv, bi, best_v, best_i)) {
                best_v = bv;
                best_i = bi;
            }
        }
    }
    if (A.part_val && wave < 4 && rr == 0 && tok < M) {
        A.part_val[(uint64_t)tok * G + b] = best_v;
        A.part_idx[(uint64_t)tok * G + b] = best_i;
    }
}

template <int NBUF>
__global__ __launch_bounds__(64 * HS_NW) void fp8_head_stream_kernel(HeadArgs A, HeadStream S) {
    fp8_head_stream_body<NBUF>(A, S);
}

// Second pass: one block per row over the partials (argmax_candidate_reduce.
// comp.template:10-37).
__global__ __launch_bounds__(256) void argmax_partials_kernel(const float* __restrict__ pv, const uint32_t* __restrict__ pi,
                                                              uint32_t n, uint32_t* __restrict__ out) {
    __shared__ float sv[256];
    __shared__ uint32_t si[256];
    const uint32_t row = blockIdx.x;
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
    for (uint32_t j = threadIdx.x; j < n; j += 256) {
        float v = pv[(uint64_t)row * n + j];
        uint32_t i = pi[(uint64_t)row * n + j];
        if (better(v, i, bv, bi)) { bv = v; bi = i; }
    }
    sv[threadIdx.x] = bv;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (uint32_t s = 128; s > 0; s >>= 1) {
        if (threadIdx.x < s && better(sv[threadIdx.x + s], si[threadIdx.x + s], sv[threadIdx.x], si[threadIdx.x])) {
            sv[threadIdx.x] = sv[threadIdx.x + s];
            si[threadIdx.x] = si[threadIdx.x + s];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) out[row] = si[0];
}

// Standalone greedy argmax over f32 logits: each lane starts from its own
// logit as the shader does, then strided candidates and a block reduction.
__global__ __launch_bounds__(1024) void argmax_f32_kernel(const float* __restrict__ logits, uint32_t vocab,
                                                          uint32_t* __restrict__ out) {
    __shared__ float sv[1024];
    __shared__ uint32_t si[1024];
    const uint32_t row = blockIdx.x, lane = threadIdx.x;
    const float* lg = logits + (uint64_t)row * vocab;
    uint32_t bi = lane;
    float bv = lane < vocab ? lg[lane] : -FLT_MAX;
    for (uint32_t t = lane + 1024; t < vocab; t += 1024) {
        float v = lg[t];
        if (better(v, t, bv, bi)) { bv = v; bi = t; }
    }
    sv[lane] = bv;
    si[lane] = bi;
    __syncthreads();
    for (uint32_t s = 512; s > 0; s >>= 1) {
        if (lane < s && better(sv[lane + s], si[lane + s], sv[lane], si[lane])) {
            sv[lane] = sv[lane + s];
            si[lane] = si[lane + s];
        }
        __syncthreads();
    }
    if (lane == 0) out[row] = si[0];
}

}  // namespace

extern "C" {

nerve_hip_status nerve_hip_fp8_output_projection(nerve_hip_ctx* ctx, const char* spec, const void* x_bf16,
                                                 const void* weight_e4m3, const void* scale_inv_bf16, void* logits_f32,
                                                 void* logits_bf16, void* argmax_u32, uint32_t batch_width,
                                                 void* stream) {
    nerve_hip_status st = nh::enter(ctx);
    if (st) return st;
    nh::Fp8HeadSpec s;
    if ((st = nh::parse_fp8_head_spec(spec, &s))) return st;
    if (!x_bf16 || !weight_e4m3 || !scale_inv_bf16) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "null buffer");
    if (!logits_f32 && !logits_bf16 && !argmax_u32) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "no output requested");
    if (s.batch_tile == 0 && batch_width > 1)
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "unbatched FP8 projection takes batch_width 1");
    if (batch_width == 0) return nh::ok();
    if ((uintptr_t)weight_e4m3 & 15) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "weight must be 16-byte aligned");
    const uint32_t M = batch_width, K = s.in, N = s.vocab, nblk = (K + 127) / 128;
    const uint32_t nblocks = (N + 16 * HEAD_WAVES - 1) / (16 * HEAD_WAVES);
    // Skinny form: <= 16 tokens, K <= 4096 in 32-byte pieces.
    const bool skinny = M <= 16 && K <= 4096 && K % 32 == 0 && K >= 32;
    const uint32_t groups = (N + 15) / 16;
    // Skinny grid: groups strided over 4 blocks per CU.
    const uint32_t sk_grid = std::min<uint32_t>(groups, 4u * (uint32_t)ctx->cu_count);
    // Stream form: per-row scales (whole groups' scale spans are contiguous
    // and 4-byte aligned), 64 <= K <= 4096, the ring fits in LDS.
    HeadStream hs{};
    hs.groups = groups;
    hs.s_off = 16 * K;
    const uint32_t sspan = 32 * nblk;
    hs.slot_bytes = hs.s_off + ((sspan < 256 ? 256 : sspan) + 15) / 16 * 16;
    hs.lw = (16 * K + 1023) / 1024 / HS_NW + ((16 * K + 1023) / 1024 % HS_NW ? 1 : 0);
    hs.cpi = hs.lw + 1;
    const size_t hs_red = HS_NW * 64 * 16;
    const int hs_nbuf = (3 * (size_t)hs.slot_bytes + hs_red <= 160 * 1024) ? 3 : 2;
    const bool stream_form = skinny && s.block_rows == 1 && K >= 64 && ((uint64_t)N * nblk) % 2 == 0 &&
                             ((uintptr_t)scale_inv_bf16 & 3) == 0 && hs.lw <= HS_LWMAX &&
                             hs_nbuf * (size_t)hs.slot_bytes + hs_red <= 160 * 1024 && hs.cpi * hs_nbuf <= 63;
    const uint32_t hs_grid = (uint32_t)ctx->cu_count;
    const uint32_t nparts = stream_form ? hs_grid : skinny ? sk_grid : nblocks;
    nh::Carver cv;
    size_t o_q = cv.take<uint8_t>((size_t)M * K);
    size_t o_s = cv.take<float>((size_t)M * nblk);
    size_t o_pv = cv.take<float>(argmax_u32 ? (size_t)M * nparts : 0);
    size_t o_pi = cv.take<uint32_t>(argmax_u32 ? (size_t)M * nparts : 0);
    void* ws = nullptr;
    if ((st = nh::workspace(ctx, cv.offset, &ws))) return st;
    uint8_t* base = static_cast<uint8_t*>(ws);
    hipStream_t strm = (hipStream_t)stream;
    HeadArgs A;
    A.xq = base + o_q;
    A.xs = reinterpret_cast<float*>(base + o_s);
    if ((st = nh::quantize_rows(static_cast<const uint16_t*>(x_bf16), K, M, false, const_cast<uint8_t*>(A.xq),
                                const_cast<float*>(A.xs), strm)))
        return st;
    A.W = static_cast<const uint8_t*>(weight_e4m3);
    A.scale_inv = static_cast<const uint16_t*>(scale_inv_bf16);
    A.M = M;
    A.K = K;
    A.N = N;
    A.BR = s.block_rows;
    A.out_scale = s.output_scale;
    A.logits_f32 = static_cast<float*>(logits_f32);
    A.logits_bf16 = static_cast<uint16_t*>(logits_bf16);
    A.part_val = argmax_u32 ? reinterpret_cast<float*>(base + o_pv) : nullptr;
    A.part_idx = argmax_u32 ? reinterpret_cast<uint32_t*>(base + o_pi) : nullptr;
    A.nblocks = nblocks;
    if (stream_form) {
        A.nblocks = hs_grid;
        const size_t lds = hs_nbuf * (size_t)hs.slot_bytes + hs_red;
        static bool attr_set = false;
        if (!attr_set) {
            if (hipFuncSetAttribute((const void*)fp8_head_stream_kernel<3>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    160 * 1024) != hipSuccess ||
                hipFuncSetAttribute((const void*)fp8_head_stream_kernel<2>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    160 * 1024) != hipSuccess)
                return nh::fail(NERVE_HIP_DEVICE_ERROR, "hipFuncSetAttribute failed for fp8_head_stream_kernel");
            attr_set = true;
        }
        if (hs_nbuf == 3) fp8_head_stream_kernel<3><<<hs_grid, 64 * HS_NW, lds, strm>>>(A, hs);
        else fp8_head_stream_kernel<2><<<hs_grid, 64 * HS_NW, lds, strm>>>(A, hs);
    } else if (skinny) {
        A.nblocks = sk_grid;
        const uint32_t per = (nblk + SK_WAVES - 1) / SK_WAVES;
        const size_t lds = ((size_t)M * K + 15) / 16 * 16 + ((size_t)M * nblk + 3) / 4 * 4 * 4 + 3 * 64 * 4 * 4;
        const uint32_t grid = sk_grid;
        if (per <= 2) fp8_head_skinny_kernel<2><<<grid, 64 * SK_WAVES, lds, strm>>>(A, groups);
        else if (per <= 4) fp8_head_skinny_kernel<4><<<grid, 64 * SK_WAVES, lds, strm>>>(A, groups);
        else if (per <= 6) fp8_head_skinny_kernel<6><<<grid, 64 * SK_WAVES, lds, strm>>>(A, groups);
        else fp8_head_skinny_kernel<8><<<grid, 64 * SK_WAVES, lds, strm>>>(A, groups);
    } else {
        dim3 grid(nblocks, (M + 16 * HEAD_MT - 1) / (16 * HEAD_MT));
        fp8_head_kernel<<<grid, 64 * HEAD_WAVES, 0, strm>>>(A);
    }
    if ((st = nh::check_launch("fp8_output_projection"))) return st;
    if (argmax_u32) {
        argmax_partials_kernel<<<M, 256, 0, strm>>>(A.part_val, A.part_idx, A.nblocks, static_cast<uint32_t*>(argmax_u32));
        return nh::check_launch("fp8_output_projection_argmax");
    }
    return nh::ok();
}

nerve_hip_status nerve_hip_argmax_f32(nerve_hip_ctx* ctx, const void* logits_f32, uint32_t batch_width, uint32_t vocab,
                                      void* argmax_u32, void* stream) {
    nerve_hip_status st = nh::enter(ctx);
    if (st) return st;
    if (!logits_f32 || !argmax_u32) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "null buffer");
    if (vocab == 0) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "empty vocabulary");
    if (batch_width == 0) return nh::ok();
    argmax_f32_kernel<<<batch_width, 1024, 0, (hipStream_t)stream>>>(static_cast<const float*>(logits_f32), vocab,
                                                                    static_cast<uint32_t*>(argmax_u32));
    return nh::check_launch("argmax_f32");
}

}  // extern "C"
