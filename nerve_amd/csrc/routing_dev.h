// Device code of the MoE routing steps shared by the routing launches and
// by the expert kernels that fold the routing into their own launch: top-k
// (a6) and expert-sorted route compaction (a7).
#pragma once

#include <cmath>

#include "common.h"

namespace {

// An LDS count.  The telemetry pointer of the forms below may address LDS
// or global memory, so the compiler would emit a flat atomic (the slow path
// through the vector memory unit); the explicit LDS address space makes it
// a ds_add.
typedef __attribute__((address_space(3))) uint32_t lds_u32_t;
__device__ __forceinline__ void lds_count(uint32_t* p) { __atomic_fetch_add((lds_u32_t*)p, 1u, __ATOMIC_RELAXED); }
// A device-memory count (agent scope), as a global atomic rather than a flat one.
typedef __attribute__((address_space(1))) uint32_t global_u32_t;
__device__ __forceinline__ void global_count(uint32_t* p) {
    __hip_atomic_fetch_add((global_u32_t*)p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
        if (tel_lds) lds_count(&tel_lds[i]);
        else global_count(&telemetry[i]);
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
        // sort); missing selections are expert 0 and sort first, before
        // expert 0's own selection.
        float w = sig ? sigmoidf_(raw) : expf(raw - maximum);
        if (P.normalize || !sig) w /= den;
        const uint32_t word = (f32_to_bf16(w) << 16) | lane;
        if (lane == 0)
            for (uint32_t c = 0; c < k - nsel; c++) routes[(uint64_t)b * k + c] = word;
        if (chosen) routes[(uint64_t)b * k + (uint32_t)__popcll(chosen_mask & ((1ull << lane) - 1ull)) + (k - nsel)] = word;
    }
    if (!telemetry) return;
    auto count = [&](uint32_t i) {
        if (tel_lds) lds_count(&tel_lds[i]);
        else global_count(&telemetry[i]);
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

// Top-k of two tokens per wave for E <= 32 in the moe_topk form (mode 0):
// lanes 32 h + e hold expert e of token b0 + h (h = 0, 1).  The selection,
// the weights, their summation orders, the route words and the telemetry
// counts are those of topk_token_fast; only the lane layout differs, so a
// wave settles two tokens with the same short chain of steps (one LDS row
// for the ranks, shuffles within each half for the selected experts).
// s_sh: the wave's 16-byte aligned LDS scratch of 64 floats; telemetry may be
// an LDS copy of the counts (tel_is_lds).
__device__ void topk_pair32(const uint16_t* lg, uint32_t stride, const void* bias, uint32_t* routes,
                            uint32_t* telemetry, uint32_t b0, uint32_t B, const TopkParams& P, float* s_sh,
                            bool tel_is_lds = false) {
    const uint32_t lane = threadIdx.x & 63, h = lane >> 5, e = lane & 31, E = P.E, k = P.k;
    const uint32_t b = b0 + h, base = 32 * h;
    const bool valid = b < B;
    const bool have = valid && e < E;
    float raw = 0.0f, s = -INFINITY;
    if (have) {
        raw = bf16_to_f32(lg[(uint64_t)b * stride + e]);
        if (P.softcap > 0.0f) raw = tanhf(raw / P.softcap) * P.softcap;
        s = P.activation ? sigmoidf_(raw) : raw;
        if (P.bias == 1) s = s + static_cast<const float*>(bias)[e];
        else if (P.bias == 2) s = s + bf16_to_f32(static_cast<const uint16_t*>(bias)[e]);
    }
    const bool nan = have && !(s == s);
    s_sh[lane] = s;
    __builtin_amdgcn_wave_barrier();
    uint32_t rank = 0;
    const uint32_t E4 = (E + 3) / 4;
    for (uint32_t j4 = 0; j4 < E4; j4++) {
        const float4 v = *reinterpret_cast<const float4*>(s_sh + base + 4 * j4);
        const uint32_t j = 4 * j4;
        rank += better(v.x, j, s, e) ? 1u : 0u;
        rank += better(v.y, j + 1, s, e) ? 1u : 0u;
        rank += better(v.z, j + 2, s, e) ? 1u : 0u;
        rank += better(v.w, j + 3, s, e) ? 1u : 0u;
    }
    __builtin_amdgcn_wave_barrier();
    const bool chosen = have && !nan && rank < k;
    const uint32_t hm = (uint32_t)(__ballot(chosen) >> base);
    // Expert of this half selected in round r (0 when the round found none).
    auto top_of = [&](uint32_t r) -> uint32_t {
        const uint32_t m = (uint32_t)(__ballot(chosen && rank == r) >> base);
        return m ? (uint32_t)__builtin_ctz(m) : 0u;
    };
    // Value of expert x of this lane's token: x is uniform within each half
    // of the wave, so two lane reads and a select instead of a shuffle.
    auto from = [&](float v, uint32_t x) -> float {
        const uint32_t x0 = (uint32_t)__builtin_amdgcn_readlane((int)x, 0), x1 = (uint32_t)__builtin_amdgcn_readlane((int)x, 32);
        const float lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), (int)x0));
        const float hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), (int)(32 + x1)));
        return h ? hi : lo;
    };
    const bool sig = P.activation != 0;
    float maximum = from(raw, top_of(0));
    float den = 0.0f;
    if (P.normalize) {
        const float term = sig ? sigmoidf_(raw) : expf(raw - maximum);
        for (uint32_t r = 0; r < k; r++) den += from(term, top_of(r));
    } else if (!sig) {
        float m = e < E ? raw : -INFINITY;
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        maximum = m;
        const float term = expf(raw - maximum);
        for (uint32_t x = 0; x < E; x++) den += from(term, x);
    }
    const uint32_t nsel = (uint32_t)__popc(hm);
    if (!valid) return;
    if (chosen || (e == 0 && nsel < k)) {
        // missing selections (expert 0) first, then the selected experts
        float w = sig ? sigmoidf_(raw) : expf(raw - maximum);
        if (P.normalize || !sig) w /= den;
        const uint32_t word = (f32_to_bf16(w) << 16) | e;
        if (e == 0)
            for (uint32_t c = 0; c < k - nsel; c++) routes[(uint64_t)b * k + c] = word;
        if (chosen) routes[(uint64_t)b * k + (uint32_t)__popc(hm & ((1u << e) - 1u)) + (k - nsel)] = word;
    }
    if (!telemetry) return;
    auto count = [&](uint32_t i) {
        if (tel_is_lds) lds_count(&telemetry[i]);
        else global_count(&telemetry[i]);
    };
    if (chosen) count(e);
    if (e == 0 && nsel < k)
        for (uint32_t c = 0; c < k - nsel; c++) count(0);
    if (chosen) {
        uint32_t higher = hm & ~(uint32_t)((2ull << e) - 1ull);
        while (higher) {
            const uint32_t right = (uint32_t)__builtin_ctz(higher);
            higher &= higher - 1u;
            count(E + e * (2u * E - e - 1u) / 2u + right - e - 1u);
        }
    }
    if (e == 0 && nsel < k && nsel > 0) {
        for (uint32_t c = 0; c < k - nsel; c++) {
            uint32_t m = hm & ~1u;
            while (m) {
                const uint32_t right = (uint32_t)__builtin_ctz(m);
                m &= m - 1u;
                count(E + right - 1u);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// a7: route compaction (moe_route_compact_batch1.comp.template:26-106,
// moe_route_count_batch1.comp.template:21-58) in one 1024-thread block.
// With expert_count == 0 the map is the stable sort of the routes by expert
// (key = (expert, source index)); otherwise it lists the owned experts'
// routes in source order.  The control words are written either way.
// ---------------------------------------------------------------------------
constexpr uint32_t COMPACT_LDS_ROUTES = 8192;
constexpr uint32_t COMPACT_RPL = 8;            // 64-route chunks per wave held in registers
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
// 64-route chunk with ballots.  Returns false (nothing written) if an
// expert id is outside [0, E).
__device__ bool compact_counting(const CompactArgs& A, uint32_t* cnt, uint32_t* wave_tot, uint32_t* flag) {
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, nw = blockDim.x >> 6;
    const uint32_t E = A.E, n = A.n;
    if (tid == 0) *flag = 0;
    for (uint32_t i = tid; i < nw * E; i += blockDim.x) cnt[i] = 0;
    __syncthreads();
    const uint32_t seg = (n + nw - 1) / nw;
    const uint32_t s0 = min(n, wave * seg), s1 = min(n, s0 + seg);
    // Segments of up to COMPACT_RPL * 64 routes: every route word loaded at
    // once into registers, each 64-route chunk's lanes grouped by expert with
    // one ballot per key bit (E <= 512), one LDS add per group.  The same
    // groups give each route's rank within its chunk for the placement.
    const bool regs = seg <= COMPACT_RPL * 64;
    uint32_t er[COMPACT_RPL], before_r[COMPACT_RPL], after_r[COMPACT_RPL];
    if (regs) {
#pragma unroll
        for (uint32_t c = 0; c < COMPACT_RPL; c++) {
            const uint32_t i = s0 + 64 * c + lane;
            er[c] = i < s1 ? (A.routes[i] & 0xffffu) : 0xffffffffu;
        }
#pragma unroll
        for (uint32_t c = 0; c < COMPACT_RPL; c++) {
            if (s0 + 64 * c >= s1) break;   // wave-uniform
            const uint32_t e = er[c];
            const bool valid = e != 0xffffffffu;
            if (valid && e >= E) *flag = 1;
            uint64_t eq = __ballot(valid && e < E);
#pragma unroll
            for (int bit = 0; bit < 9; bit++) {
                const bool one = (e >> bit) & 1u;
                const uint64_t m = __ballot(one);
                eq &= one ? m : ~m;
            }
            before_r[c] = (uint32_t)__popcll(eq & ((1ull << lane) - 1ull));
            after_r[c] = (uint32_t)__popcll(eq >> lane) - 1u;
            if (valid && e < E && before_r[c] == 0) __atomic_fetch_add((lds_u32_t*)&cnt[wave * E + e], (uint32_t)__popcll(eq), __ATOMIC_RELAXED);
        }
    } else {
        for (uint32_t i = s0 + lane; i < s1; i += 64) {
            const uint32_t e = A.routes[i] & 0xffffu;
            if (e < E) atomicAdd(&cnt[wave * E + e], 1u);
            else *flag = 1;
        }
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
    if (regs) {
        // Chunks in order: a chunk's group reads its expert's running
        // position, its last lane advances it (a wave's LDS accesses
        // complete in order).
#pragma unroll
        for (uint32_t c = 0; c < COMPACT_RPL; c++) {
            if (s0 + 64 * c >= s1) break;   // wave-uniform
            const uint32_t e = er[c], i = s0 + 64 * c + lane;
            if (e != 0xffffffffu) {
                const uint32_t pos = cnt[wave * E + e] + before_r[c];
                put_map(A, pos, i);
                if (after_r[c] == 0) cnt[wave * E + e] = pos + 1;
            }
        }
        return true;
    }
    for (uint32_t base = s0; base < s1; base += 64) {
        const uint32_t i = base + lane;
        const bool valid = i < s1;
        const uint32_t e = valid ? (A.routes[i] & 0xffffu) : 0xffffffffu;
        // Lanes holding the same expert, from one ballot per key bit (E <= 512).
        uint64_t eq = __ballot(valid);
#pragma unroll
        for (int bit = 0; bit < 9; bit++) {
            const bool one = (e >> bit) & 1u;
            const uint64_t m = __ballot(one);
            eq &= one ? m : ~m;
        }
        const uint32_t before = (uint32_t)__popcll(eq & ((1ull << lane) - 1ull));
        const uint32_t after = (uint32_t)__popcll(eq >> lane) - 1u;
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

}  // namespace
