// MoE routing on gfx950: router projection (a5), top-k (a6), expert-sorted
// route compaction (a7) and the weighted combine (a8).
#include <cmath>

#include "common.h"

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

namespace {

// ---------------------------------------------------------------------------
// a5: logits[b, e] = bf16(sum_k x[b,k] W[e,k]) (linear_bf16.comp.template:
// 40-98).  One block = 16 tokens x 16 experts; its 8 waves split K and reduce
// through LDS.  Each wave issues v_mfma_f32_16x16x32_bf16 with both operands
// loaded in the same per-lane k order (8 contiguous values per lane), so the
// pairing of A and B elements is the identity whatever the hardware's k
// numbering is.
// ---------------------------------------------------------------------------
constexpr int RL_WAVES = 8;

// One 16-token x 16-expert tile computed by 8 waves (wave8 = 0..7) that split
// K; `part` is the tile's [8][64] LDS reduction area.  Every thread of the
// block must call it (it synchronizes the block); out (global or LDS) gets
// the bf16 logits at [token * out_stride + expert].
__device__ __forceinline__ void router_tile(const uint16_t* __restrict__ x, const uint16_t* __restrict__ W, uint32_t B,
                                            uint32_t H, uint32_t E, uint32_t b0, uint32_t e0, uint32_t wave8, bool active,
                                            v4f (*part)[64], uint16_t* out, uint32_t out_stride) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t g = lane >> 4, rr = lane & 15;
    const uint32_t tok = b0 + rr, ex = e0 + rr;
    const uint32_t nsteps = (H + 31) / 32;
    const uint32_t per = (nsteps + RL_WAVES - 1) / RL_WAVES;
    const uint32_t s0 = min(nsteps, wave8 * per), s1 = active ? min(nsteps, s0 + per) : s0;
    v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
    const bool H8 = (H % 8) == 0;
    auto operands = [&](uint32_t s, v4i& av, v4i& bv) {
        const uint32_t k0 = s * 32 + g * 8;
        av = v4i{0, 0, 0, 0};
        bv = v4i{0, 0, 0, 0};
        if (H8) {
            if (tok < B && k0 < H) av = *reinterpret_cast<const v4i*>(x + (uint64_t)tok * H + k0);
            if (ex < E && k0 < H) bv = *reinterpret_cast<const v4i*>(W + (uint64_t)ex * H + k0);
        } else {
            uint16_t at[8], bt[8];
            for (int j = 0; j < 8; j++) {
                at[j] = (tok < B && k0 + j < H) ? x[(uint64_t)tok * H + k0 + j] : 0;
                bt[j] = (ex < E && k0 + j < H) ? W[(uint64_t)ex * H + k0 + j] : 0;
            }
            av = *reinterpret_cast<v4i*>(at);
            bv = *reinterpret_cast<v4i*>(bt);
        }
    };
    // Eight steps of operands are loaded before any of them is consumed, so a
    // wave waits for memory once per eight MFMAs.
    constexpr uint32_t U = 8;
    for (uint32_t s = s0; s < s1; s += U) {
        v4i av[U], bv[U];
#pragma unroll
        for (uint32_t u = 0; u < U; u++) {
            if (s + u < s1) operands(s + u, av[u], bv[u]);
            else av[u] = bv[u] = v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (uint32_t u = 0; u < U; u++)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, av[u]),
                                                          __builtin_bit_cast(v8bf, bv[u]), acc, 0, 0, 0);
    }
    part[wave8][lane] = acc;
    __syncthreads();
    if (wave8 == 0 && active) {
        v4f t = part[0][lane];
#pragma unroll
        for (int w = 1; w < RL_WAVES; w++) t += part[w][lane];
        // Result lane (g, rr) holds D[token 4g+i][expert rr].
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint32_t bt = b0 + 4 * g + i;
            if (bt < B && ex < E) out[(uint64_t)bt * out_stride + ex] = (uint16_t)f32_to_bf16(t[i]);
        }
    }
}

__global__ __launch_bounds__(64 * RL_WAVES) void router_linear_kernel(const uint16_t* __restrict__ x,
                                                                       const uint16_t* __restrict__ W, uint32_t B,
                                                                       uint32_t H, uint32_t E,
                                                                       uint16_t* __restrict__ logits) {
    __shared__ v4f part[RL_WAVES][64];
    router_tile(x, W, B, H, E, blockIdx.x * 16, blockIdx.y * 16, threadIdx.x >> 6, true, part, logits, E);
}

// ---------------------------------------------------------------------------
// a6: top-k.  One wave per token.
// ---------------------------------------------------------------------------
struct TopkParams {
    uint32_t E, k, always_count;
    int mode, activation, normalize, bias;
    float softcap, routed_scale, always_weight;
};

__device__ __forceinline__ bool better(float s, uint32_t i, float bs, uint32_t bi) {
    return s > bs || (s == bs && i < bi);
}

__device__ __forceinline__ float sigmoidf_(float v) { return 1.0f / (1.0f + expf(-v)); }

// Route words and telemetry (…topk_routed_batch1_bf16.comp.template:168-179),
// spread over the wave: lane r writes route r, lanes take one counter each.
// With tel_lds the counts go to that LDS copy of the telemetry array instead.
__device__ __forceinline__ void topk_publish(uint32_t b, uint32_t lane, const uint32_t* top, const float* wts,
                                             uint32_t total_sel, uint32_t total_res, uint32_t* routes,
                                             uint32_t* telemetry, uint32_t* tel_lds) {
    auto count = [&](uint32_t i) {
        if (tel_lds) atomicAdd(&tel_lds[i], 1u);
        else __hip_atomic_fetch_add(&telemetry[i], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    if (lane < total_sel) {
        routes[(uint64_t)b * total_sel + lane] = (f32_to_bf16(wts[lane]) << 16) | top[lane];
        if (telemetry) count(top[lane]);
    }
    if (!telemetry) return;
    const uint32_t pairs = total_sel * (total_sel - 1) / 2;
    for (uint32_t p = lane; p < pairs; p += 64) {
        // p -> (l, r), l < r, in row-major order of the upper triangle
        uint32_t l = 0, rem = p;
        while (rem >= total_sel - 1 - l) {
            rem -= total_sel - 1 - l;
            l++;
        }
        const uint32_t r = l + 1 + rem;
        const uint32_t left = top[l], right = top[r];
        if (left < right) {
            const uint32_t preceding = left * (2u * total_res - left - 1u) / 2u;
            count(total_res + preceding + right - left - 1u);
        }
    }
}

// LDS work area of one token's top-k (one wave).
struct TopkScratch {
    float* raw;          // [E] router values (after softcap / activation)
    uint32_t* sel;       // [E]
    uint32_t* top;       // [128]
    float* wts;          // [128]
    float* smax;
    float* sden;
    uint32_t* sel_total;
    uint32_t* res_total;
};

// Top-k of token b from its E bf16 logits `lg` (global or LDS) by one wave.
// It synchronizes the block: every wave of the block calls it the same
// number of times (`valid` false writes nothing).
__device__ void topk_token(const uint16_t* lg, const void* bias, uint32_t* routes, uint32_t* telemetry, uint32_t b,
                           bool valid, const TopkParams& P, const TopkScratch& S, uint32_t* tel_lds = nullptr) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t E = P.E;
    float* raw = S.raw;
    uint32_t* sel = S.sel;
    uint32_t* top = S.top;
    float* wts = S.wts;
    for (uint32_t e = lane; e < E; e += 64) {
        float v = bf16_to_f32(lg[e]);
        if (P.mode == 0 && P.softcap > 0.0f) v = tanhf(v / P.softcap) * P.softcap;
        raw[e] = v;
        sel[e] = 0;
    }
    __syncthreads();
    if (P.mode == 1) {
        // initialize_softmax + activate_router_value
        // (moe_router_score_topk_batch1_bf16.comp.template:62-107).
        if (P.activation == 1) {
            float m = -INFINITY;
            for (uint32_t e = lane; e < E; e += 64) m = fmaxf(m, raw[e]);
            for (int d = 32; d > 0; d >>= 1) m = fmaxf(m, __shfl_xor(m, d));
            float s = 0.0f;
            for (uint32_t e = lane; e < E; e += 64) s += expf(raw[e] - m);
            for (int d = 32; d > 0; d >>= 1) s += __shfl_xor(s, d);
            if (lane == 0) { *S.smax = m; *S.sden = s; }
        }
        __syncthreads();
        for (uint32_t e = lane; e < E; e += 64) {
            float v = raw[e];
            if (P.activation == 0) v = sigmoidf_(v);
            else if (P.activation == 1) v = expf(v - *S.smax) / *S.sden;
            else v = sqrtf(fmaxf(v, 0.0f) + logf(1.0f + expf(-fabsf(v))));
            raw[e] = v;
        }
        __syncthreads();
    }
    for (uint32_t r = 0; r < P.k; r++) {
        float best = -INFINITY;
        uint32_t bi = 0xffffffffu;
        for (uint32_t e = lane; e < E; e += 64) {
            float s = (P.mode == 0 && P.activation) ? sigmoidf_(raw[e]) : raw[e];
            if (P.bias == 1) s = s + static_cast<const float*>(bias)[e];
            else if (P.bias == 2) s = s + bf16_to_f32(static_cast<const uint16_t*>(bias)[e]);
            if (!sel[e] && better(s, e, best, bi)) { best = s; bi = e; }
        }
        for (int d = 32; d > 0; d >>= 1) {
            float os = __shfl_xor(best, d);
            uint32_t oi = __shfl_xor(bi, d);
            if (better(os, oi, best, bi)) { best = os; bi = oi; }
        }
        if (lane == 0) {
            top[r] = bi;
            if (bi < E) sel[bi] = 1;
        }
        __syncthreads();
    }
    if (lane == 0) {
        // All-NaN rows leave no selectable expert; index 0 keeps every LDS read in
        // bounds (the reference shader would read past its array there).
        for (uint32_t r = 0; r < P.k; r++)
            if (top[r] >= E) top[r] = 0;
        const uint32_t ks = P.k;
        uint32_t total_sel = ks, total_res = E;
        if (P.mode == 0) {
            // moe_topk_routed_batch1_bf16.comp.template:133-167
            const bool sig = P.activation != 0;
            float maximum = raw[top[0]];
            float den = 0.0f;
            if (P.normalize) {
                for (uint32_t r = 0; r < ks; r++) {
                    float l = raw[top[r]];
                    den += sig ? sigmoidf_(l) : expf(l - maximum);
                }
            } else if (!sig) {
                maximum = -INFINITY;
                for (uint32_t e = 0; e < E; e++) maximum = fmaxf(maximum, raw[e]);
                for (uint32_t e = 0; e < E; e++) den += expf(raw[e] - maximum);
            }
            for (uint32_t r = 1; r < ks; r++) {
                uint32_t ex = top[r];
                uint32_t ins = r;
                while (ins > 0 && top[ins - 1] > ex) { top[ins] = top[ins - 1]; ins--; }
                top[ins] = ex;
            }
            for (uint32_t r = 0; r < ks; r++) {
                float l = raw[top[r]];
                float w = sig ? sigmoidf_(l) : expf(l - maximum);
                if (P.normalize || !sig) w /= den;
                wts[r] = w;
            }
        } else {
            // moe_router_score_topk_batch1_bf16.comp.template:169-205
            total_sel = ks + P.always_count;
            total_res = E + P.always_count;
            float den = 0.0f;
            if (P.normalize) for (uint32_t r = 0; r < ks; r++) den += raw[top[r]];
            for (uint32_t r = 0; r < ks; r++) {
                float w = raw[top[r]];
                wts[r] = P.normalize ? w / den * P.routed_scale : w * P.routed_scale;
            }
            for (uint32_t a = 0; a < P.always_count; a++) {
                top[ks + a] = E + a;
                wts[ks + a] = P.always_weight;
            }
            for (uint32_t r = 1; r < total_sel; r++) {
                uint32_t ex = top[r];
                float w = wts[r];
                uint32_t ins = r;
                while (ins > 0 && top[ins - 1] > ex) {
                    top[ins] = top[ins - 1];
                    wts[ins] = wts[ins - 1];
                    ins--;
                }
                top[ins] = ex;
                wts[ins] = w;
            }
        }
        *S.sel_total = total_sel;
        *S.res_total = total_res;
    }
    __syncthreads();
    if (valid) topk_publish(b, lane, top, wts, *S.sel_total, *S.res_total, routes, telemetry, tel_lds);
}

// Lane-parallel top-k for moe_topk with E <= 64 (lane e holds expert e):
// the result of topk_token's k arg-max rounds, bit for bit.  Each lane's rank
// is the number of experts that beat it under the same strict order (value
// descending, index ascending; a NaN never beats and is never selected), so
// round r selects the expert of rank r.  Weights use the same formulas and
// summation orders (selection order, or expert order for the full softmax),
// carried out identically in every lane.  The block is not synchronized;
// s_sh is the wave's own 16-byte aligned LDS scratch of at least E rounded
// up to 4 floats.
__device__ void topk_token_fast(const uint16_t* lg, const void* bias, uint32_t* routes, uint32_t* telemetry, uint32_t b,
                                bool valid, const TopkParams& P, uint32_t* tel_lds, float* s_sh) {
    const uint32_t lane = threadIdx.x & 63, E = P.E, k = P.k;
    const bool have = lane < E;
    float raw = 0.0f, s = -INFINITY;
    if (have) {
        raw = bf16_to_f32(lg[lane]);
        if (P.softcap > 0.0f) raw = tanhf(raw / P.softcap) * P.softcap;
        s = P.activation ? sigmoidf_(raw) : raw;
        if (P.bias == 1) s = s + static_cast<const float*>(bias)[lane];
        else if (P.bias == 2) s = s + bf16_to_f32(static_cast<const uint16_t*>(bias)[lane]);
    }
    const bool nan = have && !(s == s);
    auto lane_f = [](float v, uint32_t j) __attribute__((always_inline)) {
        return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), j));
    };
    // Every lane compares against all E scores, read back from the wave's
    // LDS row as broadcasts (a readlane per comparison would serialize on
    // its hazard waits).
    if (lane < (E + 3) / 4 * 4) s_sh[lane] = s;     // -inf pads the row to whole float4s
    __builtin_amdgcn_wave_barrier();
    uint32_t rank = 0;
    const uint32_t E4 = (E + 3) / 4;
#pragma unroll 4
    for (uint32_t j4 = 0; j4 < E4; j4++) {
        const float4 v = *reinterpret_cast<const float4*>(s_sh + 4 * j4);
        const uint32_t j = 4 * j4;
        rank += better(v.x, j, s, lane) ? 1u : 0u;
        rank += better(v.y, j + 1, s, lane) ? 1u : 0u;
        rank += better(v.z, j + 2, s, lane) ? 1u : 0u;
        rank += better(v.w, j + 3, s, lane) ? 1u : 0u;
    }
    __builtin_amdgcn_wave_barrier();
    const bool chosen = have && !nan && rank < k;
    const uint64_t chosen_mask = __ballot(chosen);
    // Expert selected in round r (rounds past the selectable experts pick 0,
    // as topk_token does).
    auto top_of = [&](uint32_t r) -> uint32_t {
        const uint64_t m = __ballot(chosen && rank == r);
        return m ? (uint32_t)__builtin_ctzll(m) : 0u;
    };
    const bool sig = P.activation != 0;
    float maximum = lane_f(raw, top_of(0));
    float den = 0.0f;
    if (P.normalize) {
        // Per-lane terms, then added in selection order.
        const float term = sig ? sigmoidf_(raw) : expf(raw - maximum);
        for (uint32_t r = 0; r < k; r++) den += lane_f(term, top_of(r));
    } else if (!sig) {
        maximum = -INFINITY;
        for (uint32_t e = 0; e < E; e++) maximum = fmaxf(maximum, lane_f(raw, e));
        const float term = expf(raw - maximum);
        for (uint32_t e = 0; e < E; e++) den += lane_f(term, e);
    }
    // Rounds that found nothing select expert 0 with expert 0's logit.
    const uint32_t nsel = __popcll(chosen_mask);
    if (!valid) return;
    if (chosen || (lane == 0 && nsel < k)) {
        // Position in ascending expert order (the reference's insertion
        // sort); missing selections are expert 0 and sort first.
        const uint32_t pos0 = chosen ? (uint32_t)__popcll(chosen_mask & ((1ull << lane) - 1ull)) + (k - nsel) : 0u;
        const uint32_t copies = chosen ? 1u : k - nsel;
        float w = sig ? sigmoidf_(raw) : expf(raw - maximum);
        if (P.normalize || !sig) w /= den;
        const uint32_t word = (f32_to_bf16(w) << 16) | lane;
        for (uint32_t c = 0; c < copies; c++) routes[(uint64_t)b * k + pos0 + c] = word;
    }
    if (!telemetry) return;
    auto count = [&](uint32_t i) {
        if (tel_lds) atomicAdd(&tel_lds[i], 1u);
        else __hip_atomic_fetch_add(&telemetry[i], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    // counts[expert] per selection, and every pair of selections (left < right
    // in the sorted list; equal experts are not counted as a pair).
    if (chosen) count(lane);
    if (lane == 0 && nsel < k)
        for (uint32_t c = 0; c < k - nsel; c++) count(0);
    if (chosen) {
        uint64_t higher = chosen_mask & ~((2ull << lane) - 1ull);
        while (higher) {
            const uint32_t right = (uint32_t)__builtin_ctzll(higher);
            higher &= higher - 1ull;
            count(E + lane * (2u * E - lane - 1u) / 2u + right - lane - 1u);
        }
    }
    if (lane == 0 && nsel < k && nsel > 0) {
        // Pairs (0, right) between the padding zeros and real selections.
        for (uint32_t c = 0; c < k - nsel; c++) {
            uint64_t m = chosen_mask & ~1ull;
            while (m) {
                const uint32_t right = (uint32_t)__builtin_ctzll(m);
                m &= m - 1ull;
                count(E + right - 1u);
            }
        }
    }
}

__global__ __launch_bounds__(64) void topk_kernel(const uint16_t* __restrict__ logits, const void* __restrict__ bias,
                                                  uint32_t* __restrict__ routes, uint32_t* __restrict__ telemetry,
                                                  uint32_t B, TopkParams P) {
    extern __shared__ __attribute__((aligned(16))) float sh[];
    __shared__ uint32_t top[128];
    __shared__ float wts[128];
    __shared__ float smax_sh, sden_sh;
    __shared__ uint32_t sel_total, res_total;
    const uint32_t b = blockIdx.x;
    if (b >= B) return;
    if (P.mode == 0 && P.E <= 64) {
        topk_token_fast(logits + (uint64_t)b * P.E, bias, routes, telemetry, b, true, P, nullptr, sh);
        return;
    }
    TopkScratch S{sh, reinterpret_cast<uint32_t*>(sh + P.E), top, wts, &smax_sh, &sden_sh, &sel_total, &res_total};
    topk_token(logits + (uint64_t)b * P.E, bias, routes, telemetry, b, true, P, S);
}

// ---------------------------------------------------------------------------
// a7: route compaction (moe_route_compact_batch1.comp.template:26-106,
// moe_route_count_batch1.comp.template:21-58) in one 1024-thread block.
// With expert_count == 0 the map is the stable sort of the routes by expert
// (key = (expert, source index)); otherwise it lists the owned experts'
// routes in source order.  The control words are written either way.
// ---------------------------------------------------------------------------
constexpr uint32_t COMPACT_LDS_ROUTES = 8192;
constexpr uint32_t COUNT_MAX_EXPERTS = 512;

struct CompactArgs {
    const uint32_t* routes;
    uint32_t n, k, E;
    uint32_t* frames;        // may be null (count-only form)
    uint64_t frame_words;
    uint32_t data_words;
    uint32_t* control;
    uint32_t tiles_per_route;
};

__device__ __forceinline__ void put_map(const CompactArgs& A, uint32_t pos, uint32_t src) {
    A.frames[(uint64_t)(pos / A.k) * A.frame_words + A.data_words + pos % A.k] = src;
}

// Rank of each route by the full 16-bit key: O(n) per route from LDS.
__device__ void compact_rank_loop(const CompactArgs& A, uint16_t* ex) {
    const bool staged = A.n <= COMPACT_LDS_ROUTES;
    if (staged)
        for (uint32_t i = threadIdx.x; i < A.n; i += blockDim.x) ex[i] = (uint16_t)(A.routes[i] & 0xffffu);
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < A.n; i += blockDim.x) {
        const uint32_t e = staged ? ex[i] : (A.routes[i] & 0xffffu);
        uint32_t rank = 0;
        for (uint32_t c = 0; c < A.n; c++) {
            const uint32_t ce = staged ? ex[c] : (A.routes[c] & 0xffffu);
            rank += (ce < e || (ce == e && c < i)) ? 1u : 0u;
        }
        put_map(A, rank, i);
    }
}

// Stable counting sort for large n: wave w owns a contiguous segment; per-
// wave expert histograms give each (expert, wave) its output offset, then
// each wave places its routes in order, ranking equal experts inside a
// 64-lane group with shuffles.  Returns false (nothing written) if an
// expert id is outside [0, E).
__device__ bool compact_counting(const CompactArgs& A, uint32_t* cnt, uint32_t* wave_tot, uint32_t* flag) {
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, nw = blockDim.x >> 6;
    const uint32_t E = A.E, n = A.n;
    if (tid == 0) *flag = 0;
    for (uint32_t i = tid; i < nw * E; i += blockDim.x) cnt[i] = 0;
    __syncthreads();
    const uint32_t seg = (n + nw - 1) / nw;
    const uint32_t s0 = min(n, wave * seg), s1 = min(n, s0 + seg);
    for (uint32_t i = s0 + lane; i < s1; i += 64) {
        const uint32_t e = A.routes[i] & 0xffffu;
        if (e < E) atomicAdd(&cnt[wave * E + e], 1u);
        else *flag = 1;
    }
    __syncthreads();
    if (*flag) return false;
    uint32_t t = 0;
    if (tid < E)
        for (uint32_t w = 0; w < nw; w++) t += cnt[w * E + tid];
    uint32_t inc = t;
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t u = __shfl_up(inc, d);
        if (lane >= (uint32_t)d) inc += u;
    }
    if (lane == 63) wave_tot[wave] = inc;
    __syncthreads();
    if (tid == 0) {
        uint32_t run = 0;
        for (uint32_t w = 0; w < nw; w++) {
            const uint32_t u = wave_tot[w];
            wave_tot[w] = run;
            run += u;
        }
    }
    __syncthreads();
    if (tid < E) {
        uint32_t run = wave_tot[wave] + inc - t;
        for (uint32_t w = 0; w < nw; w++) {
            const uint32_t c = cnt[w * E + tid];
            cnt[w * E + tid] = run;
            run += c;
        }
    }
    __syncthreads();
    for (uint32_t base = s0; base < s1; base += 64) {
        const uint32_t i = base + lane;
        const bool valid = i < s1;
        const uint32_t e = valid ? (A.routes[i] & 0xffffu) : 0xffffffffu;
        uint32_t before = 0, after = 0;
        for (uint32_t j = 0; j < 64; j++) {
            const uint32_t ej = __shfl(e, j);
            before += (j < lane && ej == e) ? 1u : 0u;
            after += (j > lane && ej == e) ? 1u : 0u;
        }
        if (valid) {
            const uint32_t pos = cnt[wave * E + e] + before;
            put_map(A, pos, i);
            if (after == 0) cnt[wave * E + e] = pos + 1;
        }
    }
    return true;
}

// Partitioned form: owned routes in source order (block-wide prefix sums).
__device__ uint32_t compact_owned(const CompactArgs& A, uint32_t* wave_tot, uint32_t* base_sh) {
    const uint32_t start = A.control[1], end = A.control[1] + A.control[2];
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if (threadIdx.x == 0) *base_sh = 0;
    __syncthreads();
    for (uint32_t c0 = 0; c0 < A.n; c0 += blockDim.x) {
        const uint32_t i = c0 + threadIdx.x;
        uint32_t flag = 0;
        if (i < A.n) {
            const uint32_t e = A.routes[i] & 0xffffu;
            flag = (e >= start && e < end) ? 1u : 0u;
        }
        uint32_t inc = flag;
        for (int d = 1; d < 64; d <<= 1) {
            const uint32_t t = __shfl_up(inc, d);
            if (lane >= (uint32_t)d) inc += t;
        }
        if (lane == 63) wave_tot[wave] = inc;
        __syncthreads();
        if (threadIdx.x == 0) {
            uint32_t run = 0;
            for (uint32_t w = 0; w < nw; w++) {
                const uint32_t t = wave_tot[w];
                wave_tot[w] = run;
                run += t;
            }
        }
        __syncthreads();
        const uint32_t pos = *base_sh + wave_tot[wave] + inc - flag;
        if (flag && A.frames) put_map(A, pos, i);
        __syncthreads();
        if (threadIdx.x == blockDim.x - 1) *base_sh = pos + flag;
        __syncthreads();
    }
    return *base_sh;
}

// The whole compaction by one block of up to 1024 threads (scratch: 16 *
// COUNT_MAX_EXPERTS words, wave_tot: 16, misc: 2).
// pre: control[0] and control[2] already read by the caller (values, so
// that no generic load of an LDS copy is needed), when `have_ctl` is set.
__device__ void compact_body(const CompactArgs& A, uint32_t* scratch, uint32_t* wave_tot, uint32_t* misc,
                             bool have_ctl = false, uint32_t ctl2 = 0, uint32_t ctl0 = 0) {
    uint32_t* control = A.control;
    if ((have_ctl ? ctl2 : control[2]) != 0u) {
        const uint32_t owned = compact_owned(A, wave_tot, &misc[0]);
        if (threadIdx.x == 0) {
            control[3] = owned;
            control[4] = owned * A.tiles_per_route;
            control[5] = 1;
            control[6] = 1;
        }
        return;
    }
    if (threadIdx.x == 0) {
        control[3] = A.n;
        control[4] = A.k * A.tiles_per_route;
        control[5] = have_ctl ? ctl0 : control[0];
        control[6] = 1;
    }
    if (!A.frames || A.n == 0) return;
    if (A.n <= 64) {
        // One wave: route i's rank by the same key from ballots, most
        // significant key bit first: the routes that agree with it on the
        // higher bits and have a 0 where it has a 1 are smaller; those that
        // agree on every bit and sit at a lower index come before it.
        if (threadIdx.x < 64) {
            const uint32_t lane = threadIdx.x;
            const uint32_t e = lane < A.n ? (A.routes[lane] & 0xffffu) : 0u;
            uint64_t eq = __ballot(lane < A.n);
            uint32_t rank = 0;
#pragma unroll
            for (int bit = 15; bit >= 0; bit--) {
                const bool one = (e >> bit) & 1u;
                const uint64_t m = __ballot(one);
                if (one) rank += (uint32_t)__popcll(eq & ~m);
                eq &= one ? m : ~m;
            }
            rank += (uint32_t)__popcll(eq & ((1ull << lane) - 1ull));
            if (lane < A.n) put_map(A, rank, lane);
        }
        return;
    }
    if (A.n > blockDim.x && A.E <= COUNT_MAX_EXPERTS) {
        if (compact_counting(A, scratch, wave_tot, &misc[1])) return;
        __syncthreads();
    }
    compact_rank_loop(A, reinterpret_cast<uint16_t*>(scratch));
}

__global__ __launch_bounds__(1024) void compact_kernel(CompactArgs A) {
    __shared__ __attribute__((aligned(16))) uint32_t scratch[16 * COUNT_MAX_EXPERTS];
    __shared__ uint32_t wave_tot[16];
    __shared__ uint32_t misc[2];
    compact_body(A, scratch, wave_tot, misc);
}

// The control words alone (no intermediates to map), by one wave: what
// compact_body writes when A.frames is null, with the control words read in
// one round of loads and the owned routes counted by ballots.
__global__ __launch_bounds__(64) void route_count_kernel(CompactArgs A) {
    const uint32_t lane = threadIdx.x;
    const uint32_t c0 = A.control[0], c1 = A.control[1], c2 = A.control[2];
    uint32_t owned = 0;
    if (c2 != 0u) {
        for (uint32_t i0 = 0; i0 < A.n; i0 += 64) {
            const uint32_t i = i0 + lane;
            const uint32_t e = i < A.n ? (A.routes[i] & 0xffffu) : 0xffffffffu;
            owned += (uint32_t)__popcll(__ballot(e >= c1 && e < c1 + c2));
        }
    }
    if (lane == 0) {
        const bool part = c2 != 0u;
        A.control[3] = part ? owned : A.n;
        A.control[4] = part ? owned * A.tiles_per_route : A.k * A.tiles_per_route;
        A.control[5] = part ? 1u : c0;
        A.control[6] = 1;
    }
}

// ---------------------------------------------------------------------------
// Router projection + top-k + compaction for decode-sized batches in two
// launches.  router_partial_kernel spreads the projection over many blocks:
// block (expert tile, K slice) writes f32 partial sums of its 16 experts over
// its K slice for every token.  route_fused_kernel (one block) adds the
// slices in slice order, rounds to bf16 (the logits), then runs the top-k
// (one token per wave) and the compaction with the same code as topk_kernel
// and compact_kernel.
// ---------------------------------------------------------------------------
constexpr uint32_t FR_MAX_TOKENS = 64;
constexpr uint32_t FR_MAX_EXPERTS = 256;
constexpr uint32_t FR_SLICES = 16;

__global__ __launch_bounds__(256) void router_partial_kernel(const uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ W, uint32_t B, uint32_t H,
                                                             uint32_t E, float* __restrict__ part) {
    __shared__ v4f red[4][64];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t g = lane >> 4, rr = lane & 15;
    const uint32_t e0 = blockIdx.x * 16, slice = blockIdx.y;
    const uint32_t nsteps = (H + 31) / 32, per = (nsteps + FR_SLICES - 1) / FR_SLICES;
    const uint32_t s0 = min(nsteps, slice * per), s1 = min(nsteps, s0 + per);
    const uint32_t ex = e0 + rr;
    const bool H8 = (H % 8) == 0;
    for (uint32_t b0 = 0; b0 < B; b0 += 16) {
        const uint32_t tok = b0 + rr;
        v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
        for (uint32_t s = s0 + wave; s < s1; s += 4) {
            const uint32_t k0 = s * 32 + g * 8;
            v4i av = v4i{0, 0, 0, 0}, bv = v4i{0, 0, 0, 0};
            if (H8) {
                if (tok < B && k0 < H) av = *reinterpret_cast<const v4i*>(x + (uint64_t)tok * H + k0);
                if (ex < E && k0 < H) bv = *reinterpret_cast<const v4i*>(W + (uint64_t)ex * H + k0);
            } else {
                uint16_t at[8], bt[8];
                for (int j = 0; j < 8; j++) {
                    at[j] = (tok < B && k0 + j < H) ? x[(uint64_t)tok * H + k0 + j] : 0;
                    bt[j] = (ex < E && k0 + j < H) ? W[(uint64_t)ex * H + k0 + j] : 0;
                }
                av = *reinterpret_cast<v4i*>(at);
                bv = *reinterpret_cast<v4i*>(bt);
            }
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, av), __builtin_bit_cast(v8bf, bv),
                                                          acc, 0, 0, 0);
        }
        red[wave][lane] = acc;
        __syncthreads();
        if (wave == 0) {
            const v4f t = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t bt = b0 + 4 * g + i;
                if (bt < B && ex < E) part[((uint64_t)slice * B + bt) * E + ex] = t[i];
            }
        }
        __syncthreads();
    }
}

struct FusedRouteArgs {
    const float* part;     // [FR_SLICES][B][E] router partial sums
    uint32_t B;
    uint16_t* logits;      // optional global copy of the logits
    const void* bias;
    uint32_t* routes;
    uint32_t* telemetry;
    TopkParams P;
    CompactArgs C;
};

constexpr uint32_t FR_LDS_TELEMETRY = 4096;   // telemetry arrays up to this size are counted in LDS

__global__ __launch_bounds__(1024) void route_fused_kernel(FusedRouteArgs F) {
    __shared__ uint16_t lg[FR_MAX_TOKENS * FR_MAX_EXPERTS];
    __shared__ __attribute__((aligned(16))) float t_raw[16][FR_MAX_EXPERTS];
    __shared__ uint32_t t_sel[16][FR_MAX_EXPERTS];
    __shared__ uint32_t t_top[16][128];
    __shared__ float t_wts[16][128];
    __shared__ float t_f[16][2];
    __shared__ uint32_t t_u[16][2];
    __shared__ uint32_t rl[1024];                  // route words, [B][total_sel]
    __shared__ uint32_t tel[FR_LDS_TELEMETRY];
    __shared__ uint32_t wave_tot[16];
    __shared__ uint32_t misc[2];
    __shared__ uint32_t ctl2, ctl0;
    const uint32_t wave = threadIdx.x >> 6, E = F.P.E, B = F.B;
    const uint32_t total_sel = F.P.k + F.P.always_count, total_res = E + F.P.always_count;
    const uint32_t T = total_res + total_res * (total_res - 1) / 2;
    const bool tel_in_lds = F.telemetry && T <= FR_LDS_TELEMETRY;
    if (threadIdx.x == 0) {
        ctl2 = F.C.control[2];
        ctl0 = F.C.control[0];
    }
    if (tel_in_lds)
        for (uint32_t i = threadIdx.x; i < T; i += blockDim.x) tel[i] = 0;
    // Logits: the slices added in slice order, rounded to bf16.
    for (uint32_t i = threadIdx.x; i < B * E; i += blockDim.x) {
        float s = 0.0f;
#pragma unroll
        for (uint32_t sl = 0; sl < FR_SLICES; sl++) s += F.part[(uint64_t)sl * B * E + i];
        lg[i] = (uint16_t)f32_to_bf16(s);
    }
    __syncthreads();
    // Top-k, one token per wave; routes and counts stay in LDS so that no
    // barrier below waits for global stores or atomics.
    TopkScratch S{t_raw[wave], t_sel[wave], t_top[wave], t_wts[wave], &t_f[wave][0], &t_f[wave][1], &t_u[wave][0],
                  &t_u[wave][1]};
    const bool fast = F.P.mode == 0 && E <= 64;
    for (uint32_t b0 = 0; b0 < B; b0 += 16) {
        const uint32_t b = b0 + wave;
        uint32_t* telp = F.telemetry ? (tel_in_lds ? tel : F.telemetry) : nullptr;
        if (fast)
            topk_token_fast(lg + (b < B ? b : 0) * E, F.bias, rl, telp, b, b < B, F.P, tel_in_lds ? tel : nullptr,
                            t_raw[wave]);
        else topk_token(lg + (b < B ? b : 0) * E, F.bias, rl, telp, b, b < B, F.P, S, tel_in_lds ? tel : nullptr);
    }
    __syncthreads();
    CompactArgs C = F.C;
    C.routes = rl;
    compact_body(C, reinterpret_cast<uint32_t*>(&t_raw[0][0]), wave_tot, misc, true, ctl2, ctl0);
    __syncthreads();
    // Global outputs last: logits, route words, telemetry counts.
    if (F.logits)
        for (uint32_t i = threadIdx.x; i < B * E; i += blockDim.x) F.logits[i] = lg[i];
    for (uint32_t i = threadIdx.x; i < B * total_sel; i += blockDim.x) F.routes[i] = rl[i];
    if (tel_in_lds)
        for (uint32_t i = threadIdx.x; i < T; i += blockDim.x)
            if (tel[i]) __hip_atomic_fetch_add(&F.telemetry[i], tel[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// a8: weighted combine (moe_reduce_batch1_bf16.comp.template:29-54).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void reduce_kernel(const uint16_t* __restrict__ eo, uint16_t* __restrict__ out,
                                                     uint32_t B, uint32_t H, uint32_t k, float routed_scale) {
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (uint64_t)B * H) return;
    const uint32_t b = (uint32_t)(idx / H), j = (uint32_t)(idx % H);
    float acc = 0.0f;
    for (uint32_t r = 0; r < k; r++) acc = round_bf16(acc + bf16_to_f32(eo[((uint64_t)b * k + r) * H + j]));
    out[idx] = (uint16_t)f32_to_bf16(acc * routed_scale);
}


}  // namespace

extern "C" {

nerve_hip_status nerve_hip_router_linear_bf16(nerve_hip_ctx* ctx, const void* x_bf16, const void* weight_bf16,
                                              void* logits_bf16, uint32_t batch_width, uint32_t hidden,
                                              uint32_t experts, void* stream) {
    nerve_hip_status st = nh::enter(ctx);
    if (st) return st;
    if (!x_bf16 || !weight_bf16 || !logits_bf16) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "null buffer");
    if (hidden == 0 || experts == 0) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "empty router shape");
    if (batch_width == 0) return nh::ok();
    if (hidden % 8 == 0 && (((uintptr_t)x_bf16 | (uintptr_t)weight_bf16) & 15))
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "router buffers must be 16-byte aligned");
    dim3 grid((batch_width + 15) / 16, (experts + 15) / 16);
    router_linear_kernel<<<grid, 64 * RL_WAVES, 0, (hipStream_t)stream>>>(
        static_cast<const uint16_t*>(x_bf16), static_cast<const uint16_t*>(weight_bf16), batch_width, hidden, experts,
        static_cast<uint16_t*>(logits_bf16));
    return nh::check_launch("router_linear_bf16");
}

nerve_hip_status nerve_hip_moe_router_topk(nerve_hip_ctx* ctx, const char* spec, const void* logits_bf16,
                                           const void* bias, void* routes_u32, void* telemetry_u32,
                                           uint32_t batch_width, void* stream) {
    nerve_hip_status st = nh::enter(ctx);
    if (st) return st;
    nh::TopkSpec ts;
    if ((st = nh::parse_topk_spec(spec, &ts))) return st;
    if (!logits_bf16 || !routes_u32) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "null buffer");
    if (ts.bias != 0 && !bias) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "specialization requires a selection bias");
    if (batch_width == 0) return nh::ok();
    TopkParams P;
    P.E = ts.experts;
    P.k = ts.k;
    P.always_count = ts.always_count;
    P.mode = ts.mode;
    P.activation = ts.activation;
    P.normalize = ts.normalize;
    P.bias = ts.bias;
    P.softcap = ts.softcap;
    P.routed_scale = ts.routed_scale;
    P.always_weight = ts.always_weight;
    size_t lds = (size_t)(ts.experts + 3) / 4 * 4 * 8;   // >= E floats rounded up to float4s, twice
    topk_kernel<<<batch_width, 64, lds, (hipStream_t)stream>>>(static_cast<const uint16_t*>(logits_bf16), bias,
                                                               static_cast<uint32_t*>(routes_u32),
                                                               static_cast<uint32_t*>(telemetry_u32), batch_width, P);
    return nh::check_launch("moe_router_topk");
}

nerve_hip_status nerve_hip_moe_route_compact(nerve_hip_ctx* ctx, const char* spec, const void* routes_u32,
                                             void* intermediates, void* control_u32, uint32_t batch_width,
                                             void* stream) {
    nerve_hip_status st = nh::enter(ctx);
    if (st) return st;
    nh::MoeSpec ms;
    if ((st = nh::parse_moe_spec(spec, &ms))) return st;
    if (!routes_u32 || !control_u32) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "null buffer");
    const uint32_t n = batch_width * ms.k;
    if (ms.family == 1 && !ms.batch1)
        return nh::fail(NERVE_HIP_INVALID_SPEC, "the unbatched INT4 expert form reads no route map");
    // TILES_PER_ROUTE of the consuming projection.
    const uint32_t tiles = nh::moe_tiles_per_route(ms);
    const uint64_t frame_words = (uint64_t)ms.k * ms.inter / 2 + ms.k;
    const uint32_t data_words = ms.k * ms.inter / 2;
    CompactArgs A;
    A.routes = static_cast<const uint32_t*>(routes_u32);
    A.n = n;
    A.k = ms.k;
    A.E = ms.experts;
    A.frames = static_cast<uint32_t*>(intermediates);
    A.frame_words = frame_words;
    A.data_words = data_words;
    A.control = static_cast<uint32_t*>(control_u32);
    A.tiles_per_route = tiles;
    if (intermediates) compact_kernel<<<1, 1024, 0, (hipStream_t)stream>>>(A);
    else route_count_kernel<<<1, 64, 0, (hipStream_t)stream>>>(A);
    return nh::check_launch("moe_route_compact");
}

nerve_hip_status nerve_hip_moe_route_fused(nerve_hip_ctx* ctx, const char* topk_spec, const char* moe_spec,
                                           const void* x_bf16, const void* router_weight_bf16, void* logits_bf16,
                                           const void* bias, void* routes_u32, void* telemetry_u32,
                                           void* intermediates, void* control_u32, uint32_t batch_width,
                                           void* stream) {
    nerve_hip_status st = nh::enter(ctx);
    if (st) return st;
    nh::TopkSpec ts;
    nh::MoeSpec ms;
    if ((st = nh::parse_topk_spec(topk_spec, &ts))) return st;
    if ((st = nh::parse_moe_spec(moe_spec, &ms))) return st;
    if (ms.family == 1 && !ms.batch1)
        return nh::fail(NERVE_HIP_INVALID_SPEC, "the unbatched INT4 expert form reads no route map");
    if (!x_bf16 || !router_weight_bf16 || !routes_u32 || !control_u32) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "null buffer");
    if (ts.bias != 0 && !bias) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "specialization requires a selection bias");
    if (ts.experts != ms.experts || ts.k + ts.always_count != ms.k)
        return nh::fail(NERVE_HIP_INVALID_SPEC, "top-k and projection specializations disagree on experts or k");
    if (batch_width == 0) return nh::ok();
    const uint32_t H = ms.hidden;
    if (batch_width > FR_MAX_TOKENS || ts.experts > FR_MAX_EXPERTS || batch_width * ms.k > 1024 || ts.k > 128 ||
        ms.k > 128)
        return nh::fail(NERVE_HIP_UNSUPPORTED, "fused routing takes <= 64 tokens, <= 256 experts, <= 1024 routes");
    if (H % 8 == 0 && (((uintptr_t)x_bf16 | (uintptr_t)router_weight_bf16) & 15))
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "router buffers must be 16-byte aligned");
    nh::Carver cv;
    const size_t o_part = cv.take<float>((size_t)FR_SLICES * batch_width * ts.experts);
    void* ws = nullptr;
    if ((st = nh::workspace(ctx, cv.offset, &ws))) return st;
    float* part = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + o_part);
    router_partial_kernel<<<dim3((ts.experts + 15) / 16, FR_SLICES), 256, 0, (hipStream_t)stream>>>(
        static_cast<const uint16_t*>(x_bf16), static_cast<const uint16_t*>(router_weight_bf16), batch_width, H,
        ts.experts, part);
    if ((st = nh::check_launch("moe_route_fused (router)"))) return st;
    FusedRouteArgs F;
    F.part = part;
    F.B = batch_width;
    F.logits = static_cast<uint16_t*>(logits_bf16);
    F.bias = bias;
    F.routes = static_cast<uint32_t*>(routes_u32);
    F.telemetry = static_cast<uint32_t*>(telemetry_u32);
    F.P.E = ts.experts;
    F.P.k = ts.k;
    F.P.always_count = ts.always_count;
    F.P.mode = ts.mode;
    F.P.activation = ts.activation;
    F.P.normalize = ts.normalize;
    F.P.bias = ts.bias;
    F.P.softcap = ts.softcap;
    F.P.routed_scale = ts.routed_scale;
    F.P.always_weight = ts.always_weight;
    CompactArgs& A = F.C;
    A.routes = F.routes;
    A.n = batch_width * ms.k;
    A.k = ms.k;
    A.E = ms.experts;
    A.frames = static_cast<uint32_t*>(intermediates);
    A.frame_words = (uint64_t)ms.k * ms.inter / 2 + ms.k;
    A.data_words = ms.k * ms.inter / 2;
    A.control = static_cast<uint32_t*>(control_u32);
    A.tiles_per_route = nh::moe_tiles_per_route(ms);
    route_fused_kernel<<<1, 1024, 0, (hipStream_t)stream>>>(F);
    return nh::check_launch("moe_route_fused");
}

nerve_hip_status nerve_hip_moe_reduce(nerve_hip_ctx* ctx, const void* expert_outputs, void* out_bf16,
                                      uint32_t batch_width, uint32_t hidden, uint32_t experts_per_token,
                                      float routed_scale, void* stream) {
    nerve_hip_status st = nh::enter(ctx);
    if (st) return st;
    if (!expert_outputs || !out_bf16) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "null buffer");
    if (experts_per_token == 0) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "experts_per_token must be positive");
    const uint64_t total = (uint64_t)batch_width * hidden;
    if (total == 0) return nh::ok();
    reduce_kernel<<<(unsigned)((total + 255) / 256), 256, 0, (hipStream_t)stream>>>(
        static_cast<const uint16_t*>(expert_outputs), static_cast<uint16_t*>(out_bf16), batch_width, hidden,
        experts_per_token, routed_scale);
    return nh::check_launch("moe_reduce");
}

}  // extern "C"
