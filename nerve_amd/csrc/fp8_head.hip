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
// Stream form (M <= 32, per-row weight scales, K <= 3072): one 8-wave block per CU over
// a contiguous range of 16-row vocabulary groups.  A group's weights are one
// contiguous 16 K-byte span of W and its scales one contiguous 32 nblk-byte
// span of scale_inv; both are read with nontemporal loads (1 KiB and 256 B
// per wave instruction) into a register set, written to one of two LDS slots
// when the group comes up, and every wave keeps the next group's loads in
// flight while it contracts the current one.
// The tokens are the MFMA A operand and stay in registers for the whole
// range; each wave contracts its share of the K chunks of every group and the
// 8 partial sums meet in LDS, where waves 0..3 finalize token 16 t + 4 g +
// wave of each token tile t.
// ---------------------------------------------------------------------------
constexpr int HS_NW = 8;
constexpr uint32_t HS_CH = 3;        // K chunks per wave (K <= 3072: 24 chunks over 8 waves)
constexpr uint32_t HS_LWMAX = 6;     // weight pieces per wave per group (16 K <= 48 KiB: K <= 3072)

struct HeadStream {
    uint32_t groups;
    uint32_t lw;                     // weight copies per wave per group
    uint32_t cpi;                    // copies per wave per group (weights + one scale copy)
    uint32_t slot_bytes, s_off;      // ring slot size; scale region offset in a slot
};

// MT token tiles of 16 (M <= 16 MT): each group's weights are contracted
// against all of them, so the weight stream is read once for up to 32 tokens.
// (Four tiles, with the token scales moved to LDS to fit the registers, took
// 186 us at M = 64 against the tiled GEMM's 161.)
template <int NBUF, int MT>
__device__ __forceinline__ void fp8_head_stream_body(const HeadArgs& A, const HeadStream& S) {
    extern __shared__ __attribute__((aligned(16))) uint8_t ring[];
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lane = threadIdx.x & 63, g = lane >> 4, rr = lane & 15;
    const uint32_t K = A.K, M = A.M, N = A.N, nblk = (K + 127) / 128;
    const uint32_t G = gridDim.x, b = blockIdx.x;
    const uint32_t i0 = (uint32_t)((uint64_t)S.groups * b / G), i1 = (uint32_t)((uint64_t)S.groups * (b + 1) / G);
    uint8_t* red = ring + 2 * S.slot_bytes;         // [wave][MT][lane] v4f partial sums

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

    // Group `item`'s pieces are loaded with nontemporal loads into a register
    // set and written to an LDS slot when the group comes up (streaming
    // reads from registers sustain ~7 TB/s over the chip where copies
    // straight into LDS sustain ~6.1).
    struct GroupRegs {
        v4i w[HS_LWMAX];
        uint32_t s;
    };
    // The loads are tracked by the compiler, which waits for each before its
    // LDS store.  Every wave issues HS_LWMAX + 1 per group on every path
    // (groups past the block's range re-read one of it, L2-resident), so
    // those waits count the other register set's loads rather than draining.
    auto load_group = [&](uint32_t item, GroupRegs& R) __attribute__((always_inline)) {
        item = item < i1 ? item : i1 > i0 ? i1 - 1 : S.groups - 1;
        const uint32_t n0 = item * 16, rows = min(16u, N - n0);
        const uint32_t wbytes = rows * K, sbytes = (rows * nblk * 2 + 3) & ~3u;
        const uint8_t* ws = A.W + (uint64_t)n0 * K;
#pragma unroll
        for (uint32_t t = 0; t < HS_LWMAX; t++)
            R.w[t] = gload16_nt(ws + (woff[t] < wbytes ? woff[t] : 0u));
        const uint8_t* ss = reinterpret_cast<const uint8_t*>(A.scale_inv) + (uint64_t)n0 * nblk * 2;
        R.s = gload4_nt(ss + (soff < sbytes ? soff : 0u));
    };
    auto store_group = [&](const GroupRegs& R, uint32_t slot) __attribute__((always_inline)) {
        uint8_t* dst = ring + slot * S.slot_bytes;
#pragma unroll
        for (uint32_t t = 0; t < HS_LWMAX; t++) *reinterpret_cast<v4i*>(dst + woff[t]) = R.w[t];
        *reinterpret_cast<uint32_t*>(dst + S.s_off + soff) = R.s;
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

    // ---- tokens: e4m3 operand pieces and block scales, loaded before the
    // first group's weights.  Quantizing the tokens here instead would repeat
    // the whole M x K quantization in every block, vector-ALU work that
    // outlasts the ring's first groups.
    v4i xlo[MT][HS_CH], xhi[MT][HS_CH];
    uint32_t sxr[MT][HS_CH][4];
#pragma unroll
    for (uint32_t mt = 0; mt < (uint32_t)MT; mt++) {
        const bool arow = 16 * mt + rr < M;
        const uint8_t* xr = A.xq + (uint64_t)(arow ? 16 * mt + rr : 0u) * K;
#pragma unroll
        for (uint32_t q = 0; q < HS_CH; q++) {
            if (c0 + q >= c1) continue;                 // wave-uniform
            const uint32_t kb = kvalid[q] ? (c0 + q) * 128 + g * 32 : 0u;
            xlo[mt][q] = *reinterpret_cast<const v4i*>(xr + kb);
            xhi[mt][q] = *reinterpret_cast<const v4i*>(xr + kb + 16);
#pragma unroll
            for (uint32_t i = 0; i < 4; i++) {
                const uint32_t tk = 16 * mt + 4 * g + i;
                sxr[mt][q][i] = __float_as_uint(A.xs[tk < M ? tk * nblk + c0 + q : 0u]);
            }
        }
    }
    GroupRegs R0, R1;
    load_group(i0, R0);
    v8i av[MT][HS_CH];
    float sx[MT][HS_CH][4];
#pragma unroll
    for (uint32_t mt = 0; mt < (uint32_t)MT; mt++) {
        const bool arow = 16 * mt + rr < M;
#pragma unroll
        for (uint32_t q = 0; q < HS_CH; q++) {
            av[mt][q] = v8i{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
            for (uint32_t i = 0; i < 4; i++) sx[mt][q][i] = 0.0f;
            if (c0 + q >= c1) continue;
            if (arow && kvalid[q])
                av[mt][q] = v8i{xlo[mt][q].x, xlo[mt][q].y, xlo[mt][q].z, xlo[mt][q].w,
                                xhi[mt][q].x, xhi[mt][q].y, xhi[mt][q].z, xhi[mt][q].w};
#pragma unroll
            for (uint32_t i = 0; i < 4; i++) sx[mt][q][i] = 16 * mt + 4 * g + i < M ? __uint_as_float(sxr[mt][q][i]) : 0.0f;
        }
    }
    load_group(i0 + 1, R1);

    const uint32_t tok = 4 * g + wave;                  // finalized token of tile 0 (waves 0..3)
    float best_v[MT];
    uint32_t best_i[MT];
#pragma unroll
    for (uint32_t mt = 0; mt < (uint32_t)MT; mt++) {
        best_v[mt] = -INFINITY;
        best_i[mt] = 0xffffffffu;
    }
    // One group: its registers go to LDS slot (i - i0) % 2 (last read by the
    // group two back, whose reduction barrier every wave has passed), the
    // group two ahead is loaded into the same registers, a barrier, then the
    // contraction, the cross-wave reduction and the finalization.
    auto group_step = [&](uint32_t i, GroupRegs& R) __attribute__((always_inline)) {
        const uint32_t slot = (i - i0) & 1u;
        store_group(R, slot);
        load_group(i + 2, R);
        __syncthreads();
        // Plain LDS reads: nothing but ds_writes fills the slots, so the
        // compiler's own waits cover them (inline-asm reads would leave it
        // free to copy their results before the wait).
        const uint8_t* buf = ring + slot * S.slot_bytes;
        v4i w0[HS_CH], w1[HS_CH];
        uint32_t sw[HS_CH];
#pragma unroll
        for (uint32_t q = 0; q < HS_CH; q++) {
            if (c0 + q >= c1) continue;
            w0[q] = *reinterpret_cast<const v4i*>(buf + rw[q]);
            w1[q] = *reinterpret_cast<const v4i*>(buf + rw[q] + 16);
            sw[q] = *reinterpret_cast<const uint16_t*>(buf + rs[q]);
        }
        v4f acc[MT];
#pragma unroll
        for (uint32_t mt = 0; mt < (uint32_t)MT; mt++) acc[mt] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (uint32_t q = 0; q < HS_CH; q++) {
            if (c0 + q >= c1) continue;
            v4i b0 = w0[q], b1 = w1[q];
            uint32_t s16 = sw[q];
            if (!kvalid[q]) b0 = b1 = v4i{0, 0, 0, 0};
            const v8i bw = v8i{b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
            const float s = bf16_to_f32(s16);
#pragma unroll
            for (uint32_t mt = 0; mt < (uint32_t)MT; mt++) {
                const v4f p = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av[mt][q], bw, v4f{0.f, 0.f, 0.f, 0.f},
                                                                                0, 0, 0, 127, 0, 127);
#pragma unroll
                for (int e = 0; e < 4; e++) acc[mt][e] = fmaf(p[e], sx[mt][q][e] * s, acc[mt][e]);
            }
        }
#pragma unroll
        for (uint32_t mt = 0; mt < (uint32_t)MT; mt++)
            *reinterpret_cast<v4f*>(red + ((wave * MT + mt) * 64 + lane) * 16) = acc[mt];
        __syncthreads();
        if (wave >= 4) return;
        const uint32_t n = i * 16 + rr;
        const bool cv = n < N;
#pragma unroll
        for (uint32_t mt = 0; mt < (uint32_t)MT; mt++) {
            float sum = 0.0f;
#pragma unroll
            for (int w2 = 0; w2 < HS_NW; w2++)
                sum += *reinterpret_cast<const float*>(red + ((w2 * MT + mt) * 64 + lane) * 16 + 4 * wave);
            const float val = sum * A.out_scale;
            const uint32_t tk = 16 * mt + tok;
            if (tk < M && cv) {
                if (A.logits_f32) A.logits_f32[(uint64_t)tk * N + n] = val;
                if (A.logits_bf16) A.logits_bf16[(uint64_t)tk * N + n] = (uint16_t)f32_to_bf16(val);
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
                if (better(bv, bi, best_v[mt], best_i[mt])) {
                    best_v[mt] = bv;
                    best_i[mt] = bi;
                }
            }
        }
    };
    // Both register sets are stepped on every path back to the loop head, so
    // the compiler's waits before the stores count the other set's loads.
    for (uint32_t i = i0; i < i1;) {
        group_step(i, R0);
        if (++i >= i1) break;
        group_step(i, R1);
        ++i;
    }
    wait_vm_imm<0>();   // the last re-read groups
#pragma unroll
    for (uint32_t mt = 0; mt < (uint32_t)MT; mt++) {
        const uint32_t tk = 16 * mt + tok;
        if (A.part_val && wave < 4 && rr == 0 && tk < M) {
            A.part_val[(uint64_t)tk * G + b] = best_v[mt];
            A.part_idx[(uint64_t)tk * G + b] = best_i[mt];
        }
    }
}

template <int NBUF, int MT>
__global__ __launch_bounds__(64 * HS_NW) void fp8_head_stream_kernel(HeadArgs A, HeadStream S) {
    fp8_head_stream_body<NBUF, MT>(A, S);
}

// ---------------------------------------------------------------------------
// Tiled form (M > 32, or M > 16 where the stream form does not apply): an
// LDS-staged FP8 GEMM.
//
// Item = (vocabulary tile of TN rows, token tile of TM rows).  Items are
// listed with token tiles fastest and dealt to the persistent blocks so that
// consecutive items run on one XCD: the token tiles of one vocabulary tile
// read the same weight rows while they sit in that XCD's L2, so the weights
// come from HBM about once.  A block of WM x WN waves (two per SIMD) streams
// every 128-column chunk of its items through an NS-stage LDS ring with
// global_load_lds: the chunk's token rows (TM x 128 B), weight rows (TN x
// 128 B) and token block scales (TM x 4 B); the ring runs across item
// boundaries.  The tokens are quantized beforehand into a chunk-major
// workspace layout ([chunk][token][128 B], 16-byte pieces already in their
// LDS positions), so their copies are contiguous 1 KiB reads, which the
// texture path serves at twice the rate of the 8-row weight pieces.  Each
// 16-byte piece p of a row R sits at piece p ^ f(R), f(R) = (R mod 8) ^
// (bit 3 of R), so the operand reads of 16 lanes hit 16 distinct bank groups.
// Every wave issues the same number of copies per chunk (plus one at an
// item's first chunk for the waves that copy the tile's row scales and
// flags), so "chunk s has landed" is a vmcnt wait for the copies issued
// after it.
//
// Wave (wm, wn) contracts tokens [wm 16 TT, +16 TT) against weight rows
// [wn 16 NJ, +16 NJ): per chunk, TT x NJ v_mfma_scale 16x16x128 e4m3 x e4m3
// (unit scales; the weights are the first operand, so a lane holds 4
// consecutive vocabulary rows of one token), each result accumulated as
// acc += p * s_x[token, chunk] and, at the end, multiplied by the row's
// scale: a reassociation of sum_b dot_b * (s_x[b] * s_w[n, b]) that holds
// when every row of the tile has one scale across K (per-channel grids; a
// scan before the launch flags the rows that do not).  A tile with any such
// row takes the general form, acc += p * (s_x * s_w[n, chunk]), with its
// scale block staged in LDS.  The epilogue writes logits and one (max, id)
// per token and tile for the argmax pass.
// ---------------------------------------------------------------------------
struct HeadGemmArgs {
    const uint8_t* xq;            // e4m3 [nblk][Mpad][128], pieces swizzled per row
    const float* xs;              // f32 [nblk][Mpad]
    const uint8_t* W;             // e4m3 [N, K]
    const uint16_t* scale_inv;    // bf16 [ceil(N/BR), nblk]
    const float* sw_row;          // f32 [N]: each row's first-block scale
    const uint8_t* nonuni;        // u8 [nvt * TN]: 1 = the row's scale varies along K
    uint32_t M, Mpad, K, N, BR, nblk;
    uint32_t ntt, n_items, nvt;
    // Item i covers vocabulary rows row0 + (i / ntt) TN ..; its argmax
    // partial is column part0 + i / ntt of the nvt per token.
    uint32_t row0, part0;
    float out_scale;
    float* logits_f32;            // [M, N] or null
    uint16_t* logits_bf16;        // [M, N] or null
    float* part_val;              // [M, nvt] or null
    uint32_t* part_idx;
};

__device__ __attribute__((aligned(16))) const uint8_t kHeadZero[1024] = {0};

template <int WM, int WN, int TT, int NJ, int NS>
struct HgLayout {
    static constexpr uint32_t NW = WM * WN;
    static constexpr uint32_t TM = 16 * WM * TT, TN = 16 * WN * NJ;
    static constexpr uint32_t A_BYTES = TM * 128, B_BYTES = TN * 128, SX_BYTES = TM * 4;
    static constexpr uint32_t STAGE = A_BYTES + B_BYTES + SX_BYTES;
    static constexpr uint32_t SWROW = NS * STAGE;           // [2][TN] f32, by item parity
    static constexpr uint32_t FLAGS = SWROW + 2 * TN * 4;   // [2][TN] u8, by item parity
    // [nblk <= 32][TN] bf16 scale block of a general-form tile; in the
    // epilogue, the argmax exchange [WN][TM] {f32, u32}
    static constexpr uint32_t SWB = FLAGS + 2 * TN;
    static constexpr uint32_t SWB_BYTES = 32 * TN * 2 > WN * TM * 8 ? 32 * TN * 2 : WN * TM * 8;
    static constexpr uint32_t BYTES = SWB + SWB_BYTES;
    static constexpr uint32_t AC = TM / 8 / NW;             // token copies per wave per chunk (1 KiB each)
    static constexpr uint32_t BC = TN / 8 / NW;             // weight copies per wave per chunk
    static constexpr uint32_t CB = AC + BC;                 // (+ 1 for wave 0: the block scales)
    static constexpr uint32_t XW = TN / 64 + 1;             // waves with an item-start copy
    static constexpr uint32_t F32_STRIDE = NJ * 64 + 16, BF16_STRIDE = NJ * 32 + 16;   // epilogue staging rows
    static_assert(AC * 8 * NW == TM && BC * 8 * NW == TN && AC >= 1 && BC >= 1, "copy split");
    static_assert(NW * 16 * F32_STRIDE <= STAGE, "staging fits a stage");
    static_assert(XW <= NW && TM % 64 == 0, "item-start copies");
};

// Piece swizzle of row r: (r mod 8) ^ bit 3 of r.  Rows 16 apart share it
// (the operand reads of tile t are those of tile 0 plus an immediate), and
// the 16 rows a read touches land on 16 distinct 16-byte bank groups.
__host__ __device__ __forceinline__ uint32_t hg_swz(uint32_t r) { return (r & 7u) ^ ((r >> 3) & 1u); }

// NPW = 0: every wave copies its share of each chunk and contracts; NPW > 0:
// NPW extra waves (NW .. NW + NPW - 1) only copy, three chunks ahead, and
// the NW waves only contract, so a copy that stalls at issue (the CU's miss
// queue full) holds up no MFMA.  The copy waves take part in every barrier
// of the contracting waves (their item starts and epilogues included).
template <int WM, int WN, int TT, int NJ, int NS, int NPW>
__device__ __forceinline__ void fp8_head_gemm_body(const HeadGemmArgs& A) {
    using L = HgLayout<WM, WN, TT, NJ, NS>;
    constexpr uint32_t TM = L::TM, TN = L::TN, NW = L::NW;
    // copy issuers and each one's share of a chunk
    constexpr uint32_t NI = NPW > 0 ? NPW : NW;
    constexpr uint32_t ACI = TM / 8 / NI, BCI = TN / 8 / NI, CBI = ACI + BCI;
    static_assert(ACI * 8 * NI == TM && BCI * 8 * NI == TN && ACI >= 1 && BCI >= 2 && BCI % 2 == 0, "copy split");
    extern __shared__ __attribute__((aligned(16))) uint8_t hg_lds[];
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t g = lane >> 4, rr = lane & 15;
    const uint32_t K = A.K, M = A.M, N = A.N, nblk = A.nblk, Mpad = A.Mpad;
    const uint32_t G = gridDim.x;
    const uint32_t ring = lds_addr(hg_lds);
    // Slot q of the item list; the hardware deals consecutive blocks to the
    // 8 XCDs in turn, so slot (b % 8) (G / 8) + b / 8 puts consecutive items
    // on one XCD.
    const uint32_t slot = G % 8 == 0 ? (blockIdx.x % 8) * (G / 8) + blockIdx.x / 8 : blockIdx.x;
    const uint32_t n_my = (A.n_items - slot + G - 1) / G;     // >= 1: G <= n_items
    const uint32_t tail_cols = K - (nblk - 1) * 128;          // columns of the last chunk (32..128)

    const bool producer = NPW > 0 && wave >= NW;
    const uint32_t wi = NPW > 0 ? (producer ? wave - NW : 0u) : wave;   // issuer index
    // item-start copies q < XW (q < TN / 64: 64 row scales; q = TN / 64: the
    // row flags) go to issuers q % NI
    auto xw_count = [&]() -> uint32_t {
        uint32_t n = 0;
        for (uint32_t q = wi; q < L::XW; q += NI) n++;
        return n;
    };
    const uint32_t n_xw = xw_count();
    // ---- issue side --------------------------------------------------------
    // Weight copy j of an issuer fills 8 rows (group wi BCI + j) with 8 pieces
    // each: lane l copies piece (l & 7) ^ f(row) of row l >> 3, where
    // f(row) = (l >> 3) ^ (group parity), so the lane part of every weight
    // copy address is one of two values; rows past N (last tile) are
    // redirected to the tile's first row.  Token copies are contiguous.
    const uint32_t lr = lane >> 3, sp0 = (lane & 7u) ^ lr;
    const uint32_t lane_off[2] = {lr * K + sp0 * 16, lr * K + (sp0 ^ 1u) * 16};
    const bool tail_ok[2] = {sp0 * 16 < tail_cols, (sp0 ^ 1u) * 16 < tail_cols};
    uint32_t i_item = slot, i_ord = 0, ic = 0, i_t0 = 0, i_n0 = 0;
    bool issuing = true;
    auto setup_issue = [&]() __attribute__((always_inline)) {
        i_t0 = (i_item % A.ntt) * TM;
        i_n0 = A.row0 + (i_item / A.ntt) * TN;
    };
    auto issue_chunk = [&](uint32_t ST) __attribute__((always_inline)) {
        uint8_t* const dA = hg_lds + ST * L::STAGE + wi * ACI * 1024;
        uint8_t* const dB = hg_lds + ST * L::STAGE + L::A_BYTES + wi * BCI * 1024;
        uint8_t* const dS = hg_lds + ST * L::STAGE + L::A_BYTES + L::B_BYTES;
        const bool last = ic + 1 == nblk;
        const uint8_t* a = A.xq + ((uint64_t)ic * Mpad + i_t0) * 128 + wi * ACI * 1024 + lane * 16;
        const uint8_t* w = A.W + (uint64_t)(i_n0 + wi * BCI * 8) * K + ic * 128;
        const bool wpart = i_n0 + TN > N;                        // last vocabulary tile
        static_for<ACI>([&](auto ji) __attribute__((always_inline)) {
            constexpr uint32_t j = decltype(ji)::value;
            __builtin_amdgcn_global_load_lds(a + j * 1024, dA + j * 1024, 16, 0, 0);
        });
        static_for<BCI>([&](auto ji) __attribute__((always_inline)) {
            constexpr uint32_t j = decltype(ji)::value;
            const uint8_t* src = w + j * 8 * K + lane_off[j & 1];
            if (wpart && i_n0 + (wi * BCI + j) * 8 + lr >= N) src = A.W + (uint64_t)i_n0 * K + ic * 128;
            __builtin_amdgcn_global_load_lds((!last || tail_ok[j & 1]) ? src : kHeadZero, dB + j * 1024, 16, 0, 0);
        });
        if (wi == 0 && lane < TM / 4)   // the chunk's TM block scales: one 16-byte piece per lane
            __builtin_amdgcn_global_load_lds(A.xs + (uint64_t)ic * Mpad + i_t0 + lane * 4, dS, 16, 0, 0);
        if (ic == 0) {
            // Item start: the tile's row scales (copies q < TN/64) and its
            // row flags (copy TN/64), into the slot of the item's parity.
            const uint32_t par = i_ord & 1u;
            for (uint32_t q = wi; q < L::XW; q += NI) {
                if (q < TN / 64) {
                    const uint32_t row = i_n0 + 64 * q + lane;
                    __builtin_amdgcn_global_load_lds(A.sw_row + (row < N ? row : N - 1),
                                                     hg_lds + L::SWROW + par * TN * 4 + 64 * q * 4, 4, 0, 0);
                } else if (lane < TN / 4) {
                    __builtin_amdgcn_global_load_lds(A.nonuni + i_n0 + 4 * lane, hg_lds + L::FLAGS + par * TN, 4, 0, 0);
                }
            }
        }
    };
    auto issue_next = [&](uint32_t ST) __attribute__((always_inline)) {
        if (!issuing) return;
        issue_chunk(ST);
        if (++ic == nblk) {
            ic = 0;
            i_ord++;
            i_item += G;
            issuing = i_ord < n_my;
            if (issuing) setup_issue();
        }
    };

    // ---- compute side --------------------------------------------------------
    const uint32_t wm = wave / WN, wn = wave % WN;
    const uint32_t RA = wm * 16 * TT + rr, RB = wn * 16 * NJ + rr;
    const uint32_t LA_lo = ring + RA * 128 + (((2 * g) ^ hg_swz(RA)) * 16);
    const uint32_t LA_hi = ring + RA * 128 + (((2 * g + 1) ^ hg_swz(RA)) * 16);
    const uint32_t LB_lo = ring + L::A_BYTES + RB * 128 + (((2 * g) ^ hg_swz(RB)) * 16);
    const uint32_t LB_hi = ring + L::A_BYTES + RB * 128 + (((2 * g + 1) ^ hg_swz(RB)) * 16);
    const uint32_t LSX = ring + L::A_BYTES + L::B_BYTES + RA * 4;
    uint32_t c = 0, c_ord = 0, c_item = slot;
    bool general = false;
    v4f acc[TT][NJ];

    auto start_item = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < TT; t++)
#pragma unroll
            for (int j = 0; j < NJ; j++) acc[t][j] = v4f{0.f, 0.f, 0.f, 0.f};
        // Row flags of the tile (landed with chunk 0): one ballot per wave,
        // the same decision in every wave.
        uint32_t f = 0;
        if (lane < TN / 4) f = lds_read_b32(hg_lds + L::FLAGS + (c_ord & 1u) * TN + 4 * lane);
        lds_drain();
        asm volatile("" : "+v"(f));
        general = __ballot(f != 0u) != 0ull;
        if (general) {
            // The tile's scale block, transposed to [chunk][row] bf16.  Plain
            // loads: the compiler drains the copies in flight before their use
            // (a pipeline bubble on this form only).
            const uint32_t n0 = A.row0 + (c_item / A.ntt) * TN;
            for (uint32_t e = tid; e < nblk * TN; e += 64 * NW) {
                const uint32_t ch = e / TN, R = e % TN, n = n0 + R < N ? n0 + R : N - 1;
                const uint32_t v = A.scale_inv[(uint64_t)(n / A.BR) * nblk + ch];
                const uint32_t a = ring + L::SWB + e * 2;
                asm volatile("ds_write_b16 %0, %1" : : "v"(a), "v"(v) : "memory");
            }
            lds_drain();
            __builtin_amdgcn_s_barrier();
        }
    };

    auto compute = [&](uint32_t stb, auto gen_tag) __attribute__((always_inline)) {
        constexpr bool general = decltype(gen_tag)::value;
        v4i blo[NJ], bhi[NJ], alo[2], ahi[2];
        uint32_t sxv[2];
        v2i swp[NJ];
        static_for<NJ>([&](auto ji) __attribute__((always_inline)) {
            constexpr uint32_t j = decltype(ji)::value;
            blo[j] = lds_rd128<j * 2048>(LB_lo + stb);
            bhi[j] = lds_rd128<j * 2048>(LB_hi + stb);
        });
        if constexpr (general) {
            // scales of rows 4 g .. 4 g + 3 of each weight tile at this chunk
            const uint32_t a = ring + L::SWB + (c * TN + wn * 16 * NJ + 4 * g) * 2;
            v2i* sp = swp;
            static_for<NJ>([&](auto ji) __attribute__((always_inline)) {
                constexpr uint32_t j = decltype(ji)::value;
                v2i r;
                asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(r) : "v"(a), "i"(j * 32));
                sp[j] = r;
            });
        }
        alo[0] = lds_rd128<0>(LA_lo + stb);
        ahi[0] = lds_rd128<0>(LA_hi + stb);
        sxv[0] = lds_rd32<0>(LSX + stb);
        // Software pipeline over the token tiles: each inline-asm group issues
        // the MFMA of (tile t, weight tile j) and then the scale-and-accumulate
        // of (tile t - 1, weight tile j), whose MFMA result was produced NJ
        // MFMAs earlier (past its latency), so the vector ALU works while the
        // matrix core is busy.  (Compiler scheduling placed each accumulate
        // right behind its own MFMA and waited for it.)
        v4f pring[NJ + 1];         // fast form: ring of MFMA results
        float sxp[2];
        const uint32_t unit = 127u;                 // e8m0 1.0: unscaled e4m3 x e4m3
        static_for<TT + 1>([&](auto ti) __attribute__((always_inline)) {
            constexpr uint32_t t = decltype(ti)::value;
            constexpr uint32_t cur = t & 1u, nxt = cur ^ 1u;
            if constexpr (t < (uint32_t)TT) {
                if constexpr (t + 1 < (uint32_t)TT) {
                    alo[nxt] = lds_rd128<(t + 1) * 2048>(LA_lo + stb);
                    ahi[nxt] = lds_rd128<(t + 1) * 2048>(LA_hi + stb);
                    sxv[nxt] = lds_rd32<(t + 1) * 64>(LSX + stb);
                    asm volatile("s_waitcnt lgkmcnt(3)" : "+v"(alo[cur]), "+v"(ahi[cur]), "+v"(sxv[cur]) : : "memory");
                } else {
                    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(alo[cur]), "+v"(ahi[cur]), "+v"(sxv[cur]) : : "memory");
                }
                if constexpr (t == 0) {
#pragma unroll
                    for (uint32_t j = 0; j < (uint32_t)NJ; j++) asm volatile("" : "+v"(blo[j]), "+v"(bhi[j]));
                    if constexpr (general) {
#pragma unroll
                        for (uint32_t j = 0; j < (uint32_t)NJ; j++) asm volatile("" : "+v"(swp[j]));
                    }
                }
                const v8i bt = v8i{alo[cur].x, alo[cur].y, alo[cur].z, alo[cur].w,
                                   ahi[cur].x, ahi[cur].y, ahi[cur].z, ahi[cur].w};
                sxp[cur] = __uint_as_float(sxv[cur]);
#pragma unroll
                for (uint32_t j = 0; j < (uint32_t)NJ; j++) {
                    const v8i bw = v8i{blo[j].x, blo[j].y, blo[j].z, blo[j].w, bhi[j].x, bhi[j].y, bhi[j].z, bhi[j].w};
                    // MFMA number m = t NJ + j writes ring slot m % (NJ + 1); the
                    // accumulate reads the slot of MFMA m - NJ.
                    const uint32_t m = t * NJ + j, wslot = m % (NJ + 1), rslot = (m + 1) % (NJ + 1);
                    if constexpr (!general && NJ >= 2 && t >= 1) {
                        v4f& a4 = acc[t - 1][j];
                        const v4f po = pring[rslot];
                        asm volatile(
                            "v_mfma_scale_f32_16x16x128_f8f6f4 %0, %5, %6, 0, %7, %7 op_sel_hi:[0,0,0]\n\t"
                            "v_fmac_f32 %1, %8, %12\n\t"
                            "v_fmac_f32 %2, %9, %12\n\t"
                            "v_fmac_f32 %3, %10, %12\n\t"
                            "v_fmac_f32 %4, %11, %12"
                            : "=&v"(pring[wslot]), "+v"(a4[0]), "+v"(a4[1]), "+v"(a4[2]), "+v"(a4[3])
                            : "v"(bw), "v"(bt), "v"(unit), "v"(po[0]), "v"(po[1]), "v"(po[2]), "v"(po[3]),
                              "v"(sxp[cur ^ 1u])
                            : );
                    } else if constexpr (!general && NJ >= 2) {
                        asm volatile("v_mfma_scale_f32_16x16x128_f8f6f4 %0, %1, %2, 0, %3, %3 op_sel_hi:[0,0,0]"
                                     : "=&v"(pring[wslot])
                                     : "v"(bw), "v"(bt), "v"(unit));
                    } else if constexpr (!general) {
                        // NJ = 1: no second MFMA to cover the first one's
                        // latency; the compiler places the wait states.
                        const v4f p = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bw, bt, v4f{0.f, 0.f, 0.f, 0.f},
                                                                                       0, 0, 0, 127, 0, 127);
#pragma unroll
                        for (int i = 0; i < 4; i++) acc[t][j][i] = fmaf(p[i], sxp[cur], acc[t][j][i]);
                    } else {
                        // general form (tiles with rows whose scale varies along
                        // K): accumulate each result right away, which keeps
                        // one result live instead of two rows of them
                        const v4f p = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bw, bt, v4f{0.f, 0.f, 0.f, 0.f},
                                                                                       0, 0, 0, 127, 0, 127);
                        const float sx = sxp[cur];
                        const uint32_t w0 = (uint32_t)swp[j].x, w1 = (uint32_t)swp[j].y;
                        acc[t][j][0] = fmaf(p[0], sx * __uint_as_float(w0 << 16), acc[t][j][0]);
                        acc[t][j][1] = fmaf(p[1], sx * __uint_as_float(w0 & 0xffff0000u), acc[t][j][1]);
                        acc[t][j][2] = fmaf(p[2], sx * __uint_as_float(w1 << 16), acc[t][j][2]);
                        acc[t][j][3] = fmaf(p[3], sx * __uint_as_float(w1 & 0xffff0000u), acc[t][j][3]);
                    }
                }
            }
            if constexpr (!general && NJ >= 2 && t == (uint32_t)TT) {
                // The last tile's accumulate: its MFMAs were the last issued, so
                // wait out their latency first (inline-asm results get no
                // compiler-inserted wait states).
                constexpr uint32_t pp = (TT - 1) & 1u;
                asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7"
                             : "+v"(pring[(TT * NJ - 1) % (NJ + 1)]), "+v"(pring[(TT * NJ - NJ) % (NJ + 1)]));
#pragma unroll
                for (uint32_t j = 0; j < (uint32_t)NJ; j++) {
                    v4f& a4 = acc[TT - 1][j];
                    const v4f po = pring[((TT - 1) * NJ + j) % (NJ + 1)];
                    asm volatile(
                        "v_fmac_f32 %0, %4, %8\n\t"
                        "v_fmac_f32 %1, %5, %8\n\t"
                        "v_fmac_f32 %2, %6, %8\n\t"
                        "v_fmac_f32 %3, %7, %8"
                        : "+v"(a4[0]), "+v"(a4[1]), "+v"(a4[2]), "+v"(a4[3])
                        : "v"(po[0]), "v"(po[1]), "v"(po[2]), "v"(po[3]), "v"(sxp[pp]));
                }
            }
        });
    };

    // Epilogue of the item: logits and the per-token (max, id) of the tile.
    // After a barrier (every wave done with stage ST and the scale block),
    // stage ST stages each wave's 16-token slices so the stores write whole
    // row segments, 16 bytes per lane, and the scale-block region carries
    // the argmax exchange between the WN waves of a token range.
    auto epilogue = [&](uint32_t ST) __attribute__((always_inline)) {
        const uint32_t vt = A.part0 + c_item / A.ntt, t0 = (c_item % A.ntt) * TM, n0 = A.row0 + (c_item / A.ntt) * TN;
        const uint32_t nw0 = n0 + wn * 16 * NJ;                  // first vocabulary row of this wave
        if (!general) {
            v4i r[NJ];
            const uint32_t a = ring + L::SWROW + (c_ord & 1u) * TN * 4 + (wn * 16 * NJ + 4 * g) * 4;
            static_for<NJ>([&](auto ji) __attribute__((always_inline)) {
                constexpr uint32_t j = decltype(ji)::value;
                r[j] = lds_rd128<j * 64>(a);
            });
            lds_drain();
#pragma unroll
            for (uint32_t j = 0; j < (uint32_t)NJ; j++) {
                asm volatile("" : "+v"(r[j]));
#pragma unroll
                for (uint32_t t = 0; t < (uint32_t)TT; t++)
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[t][j][i] *= __int_as_float(r[j][i]) * A.out_scale;
            }
        } else {
#pragma unroll
            for (uint32_t t = 0; t < (uint32_t)TT; t++)
#pragma unroll
                for (uint32_t j = 0; j < (uint32_t)NJ; j++)
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[t][j][i] *= A.out_scale;
        }
        lds_drain();
        __builtin_amdgcn_s_barrier();        // stage ST and the scale block are free
        if (A.part_val) {
            const bool whole = nw0 + 16 * NJ <= N;
#pragma unroll
            for (uint32_t t = 0; t < (uint32_t)TT; t++) {
                // A lane's 4 NJ candidates in ascending row order: a strictly
                // larger value wins, so ties keep the lower row.
                float bv = -INFINITY;
                uint32_t bi = 0xffffffffu;
#pragma unroll
                for (uint32_t j = 0; j < (uint32_t)NJ; j++) {
                    const uint32_t n = nw0 + j * 16 + 4 * g;
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const float v = acc[t][j][i];
                        const bool take = (v > bv || bi == 0xffffffffu) && (whole || n + i < N);
                        bv = take ? v : bv;
                        bi = take ? n + i : bi;
                    }
                }
                // lanes rr, rr + 16, rr + 32, rr + 48 hold one token: combine
                // them with row swaps (vector ALU; an LDS-routed shuffle would
                // queue behind the ring's copies)
                {
                    const auto v16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(bv), __float_as_uint(bv), false, false);
                    const auto i16 = __builtin_amdgcn_permlane16_swap(bi, bi, false, false);
                    const float ov = __uint_as_float((lane & 16u) ? v16[0] : v16[1]);
                    const uint32_t oi = (lane & 16u) ? i16[0] : i16[1];
                    if (better(ov, oi, bv, bi)) {
                        bv = ov;
                        bi = oi;
                    }
                    const auto v32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(bv), __float_as_uint(bv), false, false);
                    const auto i32 = __builtin_amdgcn_permlane32_swap(bi, bi, false, false);
                    const float ov2 = __uint_as_float((lane & 32u) ? v32[0] : v32[1]);
                    const uint32_t oi2 = (lane & 32u) ? i32[0] : i32[1];
                    if (better(ov2, oi2, bv, bi)) {
                        bv = ov2;
                        bi = oi2;
                    }
                }
                if (g == 0) {
                    const uint32_t a = ring + L::SWB + (wn * TM + wm * 16 * TT + t * 16 + rr) * 8;
                    asm volatile("ds_write_b64 %0, %1" : : "v"(a), "v"(v2i{(int)__float_as_uint(bv), (int)bi}) : "memory");
                }
            }
        }
        // Whole slices with 16-byte-aligned rows go through the stage; the
        // last tile's partial slice and N not a multiple of 8 (4 for f32) are
        // stored from registers.
        const bool full = nw0 + 16 * NJ <= N;
        const uint32_t sbase = ring + ST * L::STAGE + wave * 16 * L::F32_STRIDE;
        if (A.logits_bf16) {
            // (NJ = 1: two lanes per row would need 32 rows per read; the
            // register path stores those slices)
            if (full && (N & 7u) == 0 && NJ >= 2) {
                constexpr uint32_t LPR = 2 * NJ, RPR = NJ >= 2 ? 64 / LPR : 16;   // lanes per row, rows per read
#pragma unroll
                for (uint32_t t = 0; t < (uint32_t)TT; t++) {
#pragma unroll
                    for (uint32_t j = 0; j < (uint32_t)NJ; j++) {
                        const v2i w = v2i{(int)(f32_to_bf16(acc[t][j][0]) | (f32_to_bf16(acc[t][j][1]) << 16)),
                                          (int)(f32_to_bf16(acc[t][j][2]) | (f32_to_bf16(acc[t][j][3]) << 16))};
                        asm volatile("ds_write_b64 %0, %1" : : "v"(sbase + rr * L::BF16_STRIDE + (j * 16 + 4 * g) * 2), "v"(w) : "memory");
                    }
                    v4i r[16 / RPR];
                    const uint32_t ra = sbase + (lane / LPR) * L::BF16_STRIDE + (lane % LPR) * 16;
                    static_for<16 / RPR>([&](auto hi) __attribute__((always_inline)) {
                        constexpr uint32_t h = decltype(hi)::value;
                        r[h] = lds_rd128<h * RPR * L::BF16_STRIDE>(ra);
                    });
                    lds_drain();
                    const uint32_t col = nw0 + (lane % LPR) * 8;
#pragma unroll
                    for (uint32_t h = 0; h < 16 / RPR; h++) {
                        asm volatile("" : "+v"(r[h]));
                        const uint32_t tk = t0 + wm * 16 * TT + t * 16 + h * RPR + lane / LPR;
                        if (tk < M) *reinterpret_cast<v4i*>(A.logits_bf16 + (uint64_t)tk * N + col) = r[h];
                    }
                }
            } else {
#pragma unroll
                for (uint32_t t = 0; t < (uint32_t)TT; t++) {
                    const uint32_t tok = t0 + wm * 16 * TT + t * 16 + rr;
                    if (tok >= M) continue;
#pragma unroll
                    for (uint32_t j = 0; j < (uint32_t)NJ; j++) {
                        const uint32_t n = nw0 + j * 16 + 4 * g;
#pragma unroll
                        for (int i = 0; i < 4; i++)
                            if (n + i < N) A.logits_bf16[(uint64_t)tok * N + n + i] = (uint16_t)f32_to_bf16(acc[t][j][i]);
                    }
                }
            }
        }
        if (A.logits_f32) {
            if (full && (N & 3u) == 0) {
                constexpr uint32_t LPR = 4 * NJ, RPR = 64 / LPR;
#pragma unroll
                for (uint32_t t = 0; t < (uint32_t)TT; t++) {
#pragma unroll
                    for (uint32_t j = 0; j < (uint32_t)NJ; j++)
                        asm volatile("ds_write_b128 %0, %1" : : "v"(sbase + rr * L::F32_STRIDE + (j * 16 + 4 * g) * 4), "v"(acc[t][j]) : "memory");
                    v4i r[16 / RPR];
                    const uint32_t ra = sbase + (lane / LPR) * L::F32_STRIDE + (lane % LPR) * 16;
                    static_for<16 / RPR>([&](auto hi) __attribute__((always_inline)) {
                        constexpr uint32_t h = decltype(hi)::value;
                        r[h] = lds_rd128<h * RPR * L::F32_STRIDE>(ra);
                    });
                    lds_drain();
                    const uint32_t col = nw0 + (lane % LPR) * 4;
#pragma unroll
                    for (uint32_t h = 0; h < 16 / RPR; h++) {
                        asm volatile("" : "+v"(r[h]));
                        const uint32_t tk = t0 + wm * 16 * TT + t * 16 + h * RPR + lane / LPR;
                        if (tk < M) *reinterpret_cast<v4i*>(A.logits_f32 + (uint64_t)tk * N + col) = r[h];
                    }
                }
            } else {
#pragma unroll
                for (uint32_t t = 0; t < (uint32_t)TT; t++) {
                    const uint32_t tok = t0 + wm * 16 * TT + t * 16 + rr;
                    if (tok >= M) continue;
#pragma unroll
                    for (uint32_t j = 0; j < (uint32_t)NJ; j++) {
                        const uint32_t n = nw0 + j * 16 + 4 * g;
#pragma unroll
                        for (int i = 0; i < 4; i++)
                            if (n + i < N) A.logits_f32[(uint64_t)tok * N + n + i] = acc[t][j][i];
                    }
                }
            }
        }
        if (A.part_val) {
            lds_drain();
            __builtin_amdgcn_s_barrier();    // the exchange is complete
            // waves wn == 0: the best of the WN entries of each token
            if (wn == 0 && lane < 16 * TT) {
                const uint32_t tl = wm * 16 * TT + lane, tok = t0 + tl;
                float bv = -INFINITY;
                uint32_t bi = 0xffffffffu;
#pragma unroll
                for (uint32_t w2 = 0; w2 < (uint32_t)WN; w2++) {
                    v2i o;
                    asm volatile("ds_read_b64 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(o) : "v"(ring + L::SWB + (w2 * TM + tl) * 8));
                    if (better(__uint_as_float((uint32_t)o.x), (uint32_t)o.y, bv, bi)) {
                        bv = __uint_as_float((uint32_t)o.x);
                        bi = (uint32_t)o.y;
                    }
                }
                if (tok < M) {
                    A.part_val[(uint64_t)tok * A.nvt + vt] = bv;
                    A.part_idx[(uint64_t)tok * A.nvt + vt] = bi;
                }
            }
        }
    };

    // ---- pipeline ----------------------------------------------------------------
    // Chunk s of the block's sequence sits in stage s % NS.  Before
    // contracting chunk s, the copies of chunks s + 1 .. s + NS - 2 may still
    // be in flight: CB copies each, plus one at an item's first chunk for
    // waves below XW.
    const uint32_t total = n_my * nblk;
    // copies an issuer puts in flight with chunk s2 of the sequence
    auto copies_of = [&](uint32_t s2) -> uint32_t {
        return CBI + (wi == 0 ? 1u : 0u) + (s2 % nblk == 0 ? n_xw : 0u);
    };
    if (producer) {
        // Copy waves: wait for chunk sidx, join its barrier, issue chunk
        // sidx + NS - 1 into the stage chunk sidx - 1 left, and join the
        // contracting waves' barriers of this step (item start of the
        // general form, epilogue).
        setup_issue();
        for (uint32_t k = 0; k + 1 < (uint32_t)NS; k++) issue_next(k);
        uint32_t st = 0, pc = 0, pord = 0;
        for (uint32_t sidx = 0;; sidx++) {
            uint32_t x = 0;
            for (uint32_t k = 1; k + 1 < (uint32_t)NS; k++) {
                const uint32_t s2 = sidx + k;
                if (s2 < total) x += copies_of(s2);
            }
            wait_vm(x);
            __builtin_amdgcn_s_barrier();
            issue_next(st == 0 ? NS - 1 : st - 1);
            if (pc == 0) {
                // the item's row flags landed with its chunk 0: the same
                // decision as the contracting waves' start_item
                uint32_t f = 0;
                if (lane < TN / 4) f = lds_read_b32(hg_lds + L::FLAGS + (pord & 1u) * TN + 4 * lane);
                lds_drain();
                asm volatile("" : "+v"(f));
                if (__ballot(f != 0u) != 0ull) __builtin_amdgcn_s_barrier();
            }
            if (++pc == nblk) {
                __builtin_amdgcn_s_barrier();                   // epilogue: the stage is free
                if (A.part_val) __builtin_amdgcn_s_barrier();   // epilogue: the argmax exchange
                if (++pord == n_my) break;
                pc = 0;
            }
            st = st + 1 == (uint32_t)NS ? 0 : st + 1;
        }
        return;
    }
    if constexpr (NPW == 0) {
        setup_issue();
        for (uint32_t k = 0; k + 1 < (uint32_t)NS; k++) issue_next(k);
    }
    uint32_t st = 0;
    for (uint32_t sidx = 0;; sidx++) {
        if constexpr (NPW == 0) {
            uint32_t x = 0;
            for (uint32_t k = 1; k + 1 < (uint32_t)NS; k++) {
                const uint32_t s2 = sidx + k;
                if (s2 < total) x += copies_of(s2);
            }
            wait_vm(x);
        }
        __builtin_amdgcn_s_barrier();
        // Half the waves issue their copies before contracting, half after:
        // the copies queue at the texture unit, and a wave waiting to issue
        // them leaves its SIMD to the other wave, which is contracting.
        const bool early = wave < NW / 2;
        if (NPW == 0 && early) issue_next(st == 0 ? NS - 1 : st - 1);
        if (c == 0) start_item();
        const uint32_t stb = __builtin_amdgcn_readfirstlane(st * L::STAGE);
        if (general) compute(stb, std::true_type{});
        else compute(stb, std::false_type{});
        if (NPW == 0 && !early) issue_next(st == 0 ? NS - 1 : st - 1);
        if (++c == nblk) {
            epilogue(st);
            if (++c_ord == n_my) break;
            c = 0;
            c_item += G;
        }
        st = st + 1 == (uint32_t)NS ? 0 : st + 1;
    }
}

template <int WM, int WN, int TT, int NJ, int NS, int NPW>
__global__ __launch_bounds__(64 * (WM * WN + NPW), 1) void fp8_head_gemm_kernel(HeadGemmArgs A) {
    fp8_head_gemm_body<WM, WN, TT, NJ, NS, NPW>(A);
}

// Activation quantization for the tiled form (tied_output_projection_batch_
// fp8_e4m3.comp.template:94-120: per 128-column block s = amax > 0 ?
// amax / 448 : 1, q = e4m3(x / s)), written chunk-major for the GEMM's
// contiguous copies: q[chunk][row][128 B] with 16-byte piece p of row r at
// piece p ^ f(r), s[chunk][row]; rows M .. Mpad are zeros.  One 32-lane
// cluster per (row, chunk), 4 columns per lane.
__device__ __forceinline__ void head_quant_body(uint32_t bid, const uint16_t* __restrict__ x, uint32_t M, uint32_t Mpad,
                                                uint32_t K, uint8_t* __restrict__ q, float* __restrict__ s) {
    const uint32_t nblk = (K + 127) / 128;
    const uint32_t unit = bid * 8 + (threadIdx.x >> 5), cl = threadIdx.x & 31;
    const uint32_t row = unit / nblk, blk = unit % nblk;
    if (row >= Mpad) return;                     // uniform per cluster
    const uint32_t col = blk * 128 + cl * 4;
    const bool valid = row < M && col < K;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (valid) {
        const uint32_t* p = reinterpret_cast<const uint32_t*>(x + (uint64_t)row * K + col);
        const uint32_t w0 = p[0], w1 = p[1];
        v[0] = bf16_to_f32(w0); v[1] = bf16_to_f32(w0 >> 16);
        v[2] = bf16_to_f32(w1); v[3] = bf16_to_f32(w1 >> 16);
    }
    float m = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    m = wave_max32(m);
    const float sc = amax_fp8_scale(m);
    uint32_t packed = 0;
    if (valid)
        packed = f32_to_e4m3(v[0] / sc) | (f32_to_e4m3(v[1] / sc) << 8) | (f32_to_e4m3(v[2] / sc) << 16) |
                 (f32_to_e4m3(v[3] / sc) << 24);
    const uint32_t piece = (cl >> 2) ^ hg_swz(row), within = (cl & 3u) * 4;
    *reinterpret_cast<uint32_t*>(q + ((uint64_t)blk * Mpad + row) * 128 + piece * 16 + within) = packed;
    if (cl == 0) s[(uint64_t)blk * Mpad + row] = row < M ? sc : 0.0f;
}

// Per vocabulary row: its first-block scale as f32 and whether its scale
// varies across the K blocks (rows of the last tile past N: flag 0).  A block
// covers 256 rows; their scale rows are one contiguous span, read coalesced
// into LDS and checked there (nblk <= 32).
__device__ __forceinline__ void head_scale_scan_body(uint32_t bid, const uint16_t* __restrict__ scale_inv, uint32_t N,
                                                     uint32_t rows_pad, uint32_t BR, uint32_t nblk,
                                                     float* __restrict__ sw_row, uint8_t* __restrict__ nonuni) {
    __shared__ __attribute__((aligned(16))) uint16_t sh[256 * 32];
    const uint32_t n0 = bid * 256, tid = threadIdx.x;
    if (n0 >= N) {
        if (n0 + tid < rows_pad) nonuni[n0 + tid] = 0;
        return;
    }
    const uint32_t last = min(n0 + 255, N - 1);
    const uint32_t r0 = n0 / BR, r1 = last / BR;
    const uint32_t elems = (r1 - r0 + 1) * nblk;           // <= 256 * 32
    const uint16_t* src = scale_inv + (uint64_t)r0 * nblk;
    if ((((uintptr_t)src) & 15) == 0) {
        // 16-byte pieces (a few per thread), then the ragged tail
        const uint32_t nv = elems / 8;
        const v4i* s4 = reinterpret_cast<const v4i*>(src);
        v4i* d4 = reinterpret_cast<v4i*>(sh);
        for (uint32_t e = tid; e < nv; e += 256) d4[e] = s4[e];
        for (uint32_t e = nv * 8 + tid; e < elems; e += 256) sh[e] = src[e];
    } else {
        for (uint32_t e = tid; e < elems; e += 256) sh[e] = src[e];
    }
    __syncthreads();
    const uint32_t n = n0 + tid;
    if (n >= rows_pad) return;
    if (n >= N) {
        nonuni[n] = 0;
        return;
    }
    const uint16_t* row = sh + (n / BR - r0) * nblk;
    const uint32_t s0 = row[0];
    uint32_t diff = 0;
    for (uint32_t c = 1; c < nblk; c++) diff |= row[c] ^ s0;
    sw_row[n] = bf16_to_f32(s0);
    nonuni[n] = diff ? 1 : 0;
}

// The GEMM form's two preparation passes in one launch: blocks < qblocks
// quantize the token rows (head_quant_body), the others scan the vocabulary
// rows' scales (head_scale_scan_body).
__global__ __launch_bounds__(256) void head_prep_kernel(const uint16_t* __restrict__ x, uint32_t M, uint32_t Mpad,
                                                        uint32_t K, uint8_t* __restrict__ q, float* __restrict__ s,
                                                        uint32_t qblocks, const uint16_t* __restrict__ scale_inv,
                                                        uint32_t N, uint32_t rows_pad, uint32_t BR,
                                                        float* __restrict__ sw_row, uint8_t* __restrict__ nonuni) {
    if (blockIdx.x < qblocks) head_quant_body(blockIdx.x, x, M, Mpad, K, q, s);
    else head_scale_scan_body(blockIdx.x - qblocks, scale_inv, N, rows_pad, BR, (K + 127) / 128, sw_row, nonuni);
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

template <int WM, int WN, int TT, int NJ, int NS, int NPW>
nerve_hip_status launch_head_gemm_t(const HeadGemmArgs& G, uint32_t grid, hipStream_t st) {
    constexpr uint32_t lds = HgLayout<WM, WN, TT, NJ, NS>::BYTES;
    static_assert(lds <= 160 * 1024, "LDS");
    static bool attr_set = false;
    if (!attr_set) {
        if (hipFuncSetAttribute((const void*)fp8_head_gemm_kernel<WM, WN, TT, NJ, NS, NPW>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, lds) != hipSuccess)
            return nh::fail(NERVE_HIP_DEVICE_ERROR, "hipFuncSetAttribute failed for fp8_head_gemm_kernel");
        attr_set = true;
    }
    fp8_head_gemm_kernel<WM, WN, TT, NJ, NS, NPW><<<grid, 64 * (WM * WN + NPW), lds, st>>>(G);
    return nh::check_launch("fp8_head_gemm_kernel");
}

// Tiled-form configurations: token tiles of 64 / 128 / 256 rows with 256 /
// 128 / 128 vocabulary rows per tile, 8 contracting waves; and the tail
// configurations that take the rows past the last whole round of each
// (64 x 64, 128 x 64, 128 x 128 tiles: configurations 3, 4 and 1).
struct HgConfig {
    uint32_t tm, tn, ns;
};
constexpr HgConfig kHgConfigs[3] = {{64, 256, 3}, {128, 128, 4}, {256, 128, 3}};
constexpr HgConfig kHgTail[3] = {{64, 64, 3}, {128, 64, 4}, {128, 128, 4}};
constexpr int kHgTailCfg[3] = {3, 4, 1};

nerve_hip_status launch_head_gemm(int cfg, const HeadGemmArgs& G, uint32_t grid, hipStream_t st) {
    // 64- and 128-token tiles: four copy waves beside the 8 contracting
    // ones (measured 159 against 164 us at M = 64, 194 against 211 at
    // M = 128).  The 256-token tile keeps the copies in its contracting
    // waves: its ~250 registers per wave do not fit 12 waves per CU.
    constexpr int NPW = 4;
    if (cfg == 0) return launch_head_gemm_t<2, 4, 2, 4, 3, NPW>(G, grid, st);
    if (cfg == 1) return launch_head_gemm_t<2, 4, 4, 2, 4, NPW>(G, grid, st);
    if (cfg == 3) return launch_head_gemm_t<2, 4, 2, 1, 3, NPW>(G, grid, st);   // cfg 0's tail: 64 x 64
    if (cfg == 4) return launch_head_gemm_t<2, 4, 4, 1, 4, NPW>(G, grid, st);   // cfg 1's tail: 128 x 64
    return launch_head_gemm_t<4, 2, 4, 4, 3, 0>(G, grid, st);
}

}  // namespace

namespace {
// The projection with its scratch either from the context workspace
// (fixed == nullptr; may grow it with hipMalloc) or from `fixed`, a buffer of
// `fixed_bytes` that is never resized (calls needing more are refused).
nerve_hip_status fp8_projection(nerve_hip_ctx* ctx, const char* spec, const void* x_bf16, const void* weight_e4m3,
                                const void* scale_inv_bf16, void* logits_f32, void* logits_bf16, void* argmax_u32,
                                uint32_t batch_width, void* stream, void* fixed, size_t fixed_bytes) {
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
    hs.cpi = HS_LWMAX + 1;   // every wave loads HS_LWMAX pieces (repeats past lw) and one scale dword
    // Up to 32 tokens in 1 or 2 tiles of 16 (the weight stream is read once
    // for all of them).
    const uint32_t hs_mt = M <= 16 ? 1u : 2u;
    const size_t hs_red = (size_t)HS_NW * hs_mt * 64 * 16;
    const int hs_nbuf = 2;   // LDS slots; one more group is in flight in registers
    const bool stream_form = M <= 32 && K <= 4096 && K % 32 == 0 && s.block_rows == 1 && K >= 64 &&
                             ((uint64_t)N * nblk) % 2 == 0 && ((uintptr_t)scale_inv_bf16 & 3) == 0 &&
                             hs.lw <= HS_LWMAX && (nblk + HS_NW - 1) / HS_NW <= HS_CH &&
                             hs_nbuf * (size_t)hs.slot_bytes + hs_red <= 160 * 1024 && hs.cpi * hs_nbuf <= 63;
    const uint32_t hs_grid = (uint32_t)ctx->cu_count;
    // Tiled GEMM form (M > 16 without the stream form): token tiles of 64 / 128 / 256 rows, 128
    // vocabulary rows per tile; K <= 4096 (the general form's scale block
    // fits its LDS region) with at least NS chunks.
    const int hg_cfg = M <= 64 ? 0 : M <= 128 ? 1 : 2;
    const uint32_t hg_tm = kHgConfigs[hg_cfg].tm, hg_ns = kHgConfigs[hg_cfg].ns, hg_tn = kHgConfigs[hg_cfg].tn;
    const bool gemm_form = !stream_form && !skinny && K <= 4096 && K % 32 == 0 && nblk >= hg_ns;
    const uint32_t hg_nvt = (N + hg_tn - 1) / hg_tn, hg_ntt = (M + hg_tm - 1) / hg_tm;
    const uint32_t hg_items = hg_nvt * hg_ntt;
    const uint32_t hg_grid = std::min<uint32_t>(hg_items, (uint32_t)ctx->cu_count);
    // When the items leave a last round for a few blocks, the main launch
    // takes the vocabulary tiles of the whole rounds and a second launch the
    // remaining rows in smaller tiles, one round over more blocks.
    const uint32_t cu = (uint32_t)ctx->cu_count;
    const HgConfig hg_tc = kHgTail[hg_cfg];
    const uint32_t hg_mpad = hg_ntt * hg_tm;
    const uint32_t hg_main = hg_items / cu * cu / hg_ntt;        // vocabulary tiles of the whole rounds
    const uint32_t hg_tail_rows = N > hg_main * hg_tn ? N - hg_main * hg_tn : 0u;
    const uint32_t hg_tail_vt = (hg_tail_rows + hg_tc.tn - 1) / hg_tc.tn, hg_tail_ntt = hg_mpad / hg_tc.tm;
    const bool hg_tail = gemm_form && hg_main > 0 && hg_tail_vt > 0 && hg_mpad % hg_tc.tm == 0 &&
                         hg_tail_vt * hg_tail_ntt <= cu && nblk >= hg_tc.ns;
    const uint32_t hg_nparts = hg_tail ? hg_main + hg_tail_vt : hg_nvt;
    const uint32_t nparts = stream_form ? hs_grid : skinny ? sk_grid : gemm_form ? hg_nparts : nblocks;
    nh::Carver cv;
    // The GEMM form reads whole token tiles: rows up to the padded count.
    const size_t m_rows = gemm_form ? (size_t)hg_ntt * hg_tm : M;
    size_t o_q = cv.take<uint8_t>(gemm_form ? m_rows * nblk * 128 : m_rows * K);   // chunk-major pads K to 128
    size_t o_s = cv.take<float>(m_rows * nblk);
    size_t o_pv = cv.take<float>(argmax_u32 ? (size_t)M * nparts : 0);
    size_t o_pi = cv.take<uint32_t>(argmax_u32 ? (size_t)M * nparts : 0);
    size_t o_swr = cv.take<float>(gemm_form ? (size_t)N : 0);
    size_t o_nu = cv.take<uint8_t>(gemm_form ? (size_t)hg_nvt * hg_tn : 0);
    void* ws = fixed;
    if (fixed) {
        if (cv.offset > fixed_bytes)
            return nh::fail(NERVE_HIP_INVALID_ARGUMENT,
                            "FP8 projection needs " + std::to_string(cv.offset) + " bytes of scratch; the static scratch holds " +
                                std::to_string(fixed_bytes));
    } else if ((st = nh::workspace(ctx, cv.offset, &ws))) {
        return st;
    }
    uint8_t* base = static_cast<uint8_t*>(ws);
    hipStream_t strm = (hipStream_t)stream;
    HeadArgs A;
    A.xq = base + o_q;
    A.xs = reinterpret_cast<float*>(base + o_s);
    if (gemm_form) {
        // chunk-major, swizzled token rows padded to whole tiles, and the
        // vocabulary rows' scale scan, in one launch
        const uint32_t mpad = hg_ntt * hg_tm;
        const uint32_t qblocks = (uint32_t)(((uint64_t)mpad * nblk + 7) / 8);
        const uint32_t rows_pad = hg_nvt * hg_tn;
        head_prep_kernel<<<qblocks + (rows_pad + 255) / 256, 256, 0, strm>>>(
            static_cast<const uint16_t*>(x_bf16), M, mpad, K, const_cast<uint8_t*>(A.xq), const_cast<float*>(A.xs),
            qblocks, static_cast<const uint16_t*>(scale_inv_bf16), N, rows_pad, s.block_rows,
            reinterpret_cast<float*>(base + o_swr), base + o_nu);
        if ((st = nh::check_launch("head_prep"))) return st;
    } else if ((st = nh::quantize_rows(static_cast<const uint16_t*>(x_bf16), K, M, false, const_cast<uint8_t*>(A.xq),
                                       const_cast<float*>(A.xs), strm))) {
        return st;
    }
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
            if (hipFuncSetAttribute((const void*)fp8_head_stream_kernel<2, 1>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    160 * 1024) != hipSuccess ||
                hipFuncSetAttribute((const void*)fp8_head_stream_kernel<2, 2>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    160 * 1024) != hipSuccess)
                return nh::fail(NERVE_HIP_DEVICE_ERROR, "hipFuncSetAttribute failed for fp8_head_stream_kernel");
            attr_set = true;
        }
        if (hs_mt == 1) fp8_head_stream_kernel<2, 1><<<hs_grid, 64 * HS_NW, lds, strm>>>(A, hs);
        else fp8_head_stream_kernel<2, 2><<<hs_grid, 64 * HS_NW, lds, strm>>>(A, hs);
    } else if (skinny) {
        A.nblocks = sk_grid;
        const uint32_t per = (nblk + SK_WAVES - 1) / SK_WAVES;
        const size_t lds = ((size_t)M * K + 15) / 16 * 16 + ((size_t)M * nblk + 3) / 4 * 4 * 4 + 3 * 64 * 4 * 4;
        const uint32_t grid = sk_grid;
        if (per <= 2) fp8_head_skinny_kernel<2><<<grid, 64 * SK_WAVES, lds, strm>>>(A, groups);
        else if (per <= 4) fp8_head_skinny_kernel<4><<<grid, 64 * SK_WAVES, lds, strm>>>(A, groups);
        else if (per <= 6) fp8_head_skinny_kernel<6><<<grid, 64 * SK_WAVES, lds, strm>>>(A, groups);
        else fp8_head_skinny_kernel<8><<<grid, 64 * SK_WAVES, lds, strm>>>(A, groups);
    } else if (gemm_form) {
        HeadGemmArgs G;
        G.xq = A.xq;
        G.xs = A.xs;
        G.W = A.W;
        G.scale_inv = A.scale_inv;
        G.sw_row = reinterpret_cast<const float*>(base + o_swr);
        G.nonuni = base + o_nu;
        G.M = M;
        G.Mpad = hg_ntt * hg_tm;
        G.K = K;
        G.N = N;
        G.BR = s.block_rows;
        G.nblk = nblk;
        G.ntt = hg_ntt;
        G.n_items = hg_items;
        G.nvt = hg_nvt;
        G.row0 = 0;
        G.part0 = 0;
        G.out_scale = s.output_scale;
        G.logits_f32 = A.logits_f32;
        G.logits_bf16 = A.logits_bf16;
        G.part_val = A.part_val;
        G.part_idx = A.part_idx;
        A.nblocks = hg_nvt;
        if (hg_tail) {
            // Whole rounds of tiles, then the rest of the vocabulary in
            // smaller tiles over more blocks (a last round of a few whole
            // tiles would hold up the launch for a whole tile).
            G.n_items = hg_main * hg_ntt;
            G.nvt = hg_nparts;
            if ((st = launch_head_gemm(hg_cfg, G, std::min<uint32_t>(G.n_items, cu), strm))) return st;
            G.row0 = hg_main * hg_tn;
            G.part0 = hg_main;
            G.ntt = hg_tail_ntt;
            G.n_items = hg_tail_vt * hg_tail_ntt;
            if ((st = launch_head_gemm(kHgTailCfg[hg_cfg], G, std::min<uint32_t>(G.n_items, cu), strm))) return st;
            A.nblocks = hg_nparts;
        } else if ((st = launch_head_gemm(hg_cfg, G, hg_grid, strm))) {
            return st;
        }
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

}  // namespace

extern "C" {

nerve_hip_status nerve_hip_fp8_output_projection(nerve_hip_ctx* ctx, const char* spec, const void* x_bf16,
                                                 const void* weight_e4m3, const void* scale_inv_bf16, void* logits_f32,
                                                 void* logits_bf16, void* argmax_u32, uint32_t batch_width,
                                                 void* stream) {
    return fp8_projection(ctx, spec, x_bf16, weight_e4m3, scale_inv_bf16, logits_f32, logits_bf16, argmax_u32,
                          batch_width, stream, nullptr, 0);
}

nerve_hip_status nerve_hip_fp8_output_projection_noalloc(nerve_hip_ctx* ctx, const char* spec, const void* x_bf16,
                                                         const void* weight_e4m3, const void* scale_inv_bf16,
                                                         void* logits_f32, void* logits_bf16, void* argmax_u32,
                                                         uint32_t batch_width, void* stream) {
    if (!ctx) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "null nerve_hip_ctx");
    if (!ctx->static_scratch) return nh::fail(NERVE_HIP_DEVICE_ERROR, "the static scratch of this device was not resolved");
    return fp8_projection(ctx, spec, x_bf16, weight_e4m3, scale_inv_bf16, logits_f32, logits_bf16, argmax_u32,
                          batch_width, stream, ctx->static_scratch, nh::kStaticScratchBytes);
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
