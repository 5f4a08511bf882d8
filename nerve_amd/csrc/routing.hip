// MoE routing on gfx950: router projection (a5), top-k (a6), expert-sorted
// route compaction (a7) and the weighted combine (a8).
#include <algorithm>
#include <cmath>

#include "common.h"
#include "quant_dev.h"
#include "routing_dev.h"

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
// Router projection + top-k + compaction for decode-sized batches in one
// launch.  Block (expert tile, K slice) computes f32 partial sums of its 16
// experts over its slice for every token (16 waves split the slice's 32-k
// steps) and stores them device-coherently; the last block to arrive (an
// arrival counter that the last block resets) adds the slices in slice order,
// rounds to bf16 (the logits), then runs the top-k and the compaction with the
// same code as topk_kernel and compact_kernel.
// ---------------------------------------------------------------------------
constexpr uint32_t FR_MAX_TOKENS = 64;
constexpr uint32_t FR_MAX_EXPERTS = 256;
constexpr uint32_t FR_MAX_SLICES = 16;

struct FusedRouteArgs {
    const uint16_t* x;     // hidden bf16 [B, H]
    const uint16_t* W;     // router weight bf16 [E, H]
    uint32_t H, slices;
    float* part;           // [slices][B][E] router partial sums
    uint32_t* arrive;      // arrival counter, zero between launches
    uint32_t B;
    uint16_t* logits;      // optional global copy of the logits
    const void* bias;
    uint32_t* routes;
    uint32_t* telemetry;
    TopkParams P;
    CompactArgs C;
    QuantArgs Q;           // the hidden rows' e4m3 blocks, when quant is set
    uint32_t quant;
};

// The hidden rows' e4m3 blocks (pow2 scales, the gate/up projection's own
// quantization): worker w of `workers` takes units w U, w U + workers U, ...
// (U units per block pass).
__device__ __forceinline__ void route_quant_rows(const QuantArgs& Q, uint32_t w, uint32_t workers) {
    const uint64_t units = (uint64_t)Q.rows * ((Q.cols + 127) / 128);
    if (Q.vec8) {
        for (uint64_t u0 = (uint64_t)w * 64; u0 < units; u0 += (uint64_t)workers * 64)   // block-uniform bound
            quant_units8_pow2<1>(Q, u0 + (threadIdx.x >> 4), 0, threadIdx.x & 15);
    } else {
        for (uint64_t u0 = (uint64_t)w * 32; u0 < units; u0 += (uint64_t)workers * 32)
            quant_unit<true>(Q, (uint32_t)(u0 + (threadIdx.x >> 5)), threadIdx.x & 31);
    }
}

constexpr uint32_t FR_LDS_TELEMETRY = 4096;   // telemetry arrays up to this size are counted in LDS

__device__ __forceinline__ void coherent_store_f(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float coherent_load_f(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

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
    __shared__ uint32_t ctl2, ctl0, is_last, arrival;
    __shared__ v4f red[16][64];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63, E = F.P.E, B = F.B;
    // ---- partial sums of expert tile blockIdx.x over K slice blockIdx.y
    {
        const uint32_t g = lane >> 4, rr = lane & 15, H = F.H;
        const uint32_t e0 = blockIdx.x * 16, slice = blockIdx.y, ex = e0 + rr;
        const uint32_t nsteps = (H + 31) / 32, per = (nsteps + F.slices - 1) / F.slices;
        const uint32_t s0 = min(nsteps, slice * per), s1 = min(nsteps, s0 + per);
        const bool H8 = (H % 8) == 0;
        for (uint32_t b0 = 0; b0 < B; b0 += 16) {
            const uint32_t tok = b0 + rr;
            v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
            for (uint32_t st = s0 + wave; st < s1; st += 16) {
                const uint32_t k0 = st * 32 + g * 8;
                v4i av = v4i{0, 0, 0, 0}, bv = v4i{0, 0, 0, 0};
                if (H8) {
                    if (tok < B && k0 < H) av = *reinterpret_cast<const v4i*>(F.x + (uint64_t)tok * H + k0);
                    if (ex < E && k0 < H) bv = *reinterpret_cast<const v4i*>(F.W + (uint64_t)ex * H + k0);
                } else {
                    uint16_t at[8], bt[8];
                    for (int j = 0; j < 8; j++) {
                        at[j] = (tok < B && k0 + j < H) ? F.x[(uint64_t)tok * H + k0 + j] : 0;
                        bt[j] = (ex < E && k0 + j < H) ? F.W[(uint64_t)ex * H + k0 + j] : 0;
                    }
                    av = *reinterpret_cast<v4i*>(at);
                    bv = *reinterpret_cast<v4i*>(bt);
                }
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, av),
                                                              __builtin_bit_cast(v8bf, bv), acc, 0, 0, 0);
            }
            red[wave][lane] = acc;
            __syncthreads();
            if (wave == 0) {
                v4f t = red[0][lane];
#pragma unroll
                for (int w = 1; w < 16; w++) t += red[w][lane];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t bt = b0 + 4 * g + i;
                    if (bt < B && ex < E) coherent_store_f(F.part + ((uint64_t)slice * B + bt) * E + ex, t[i]);
                }
            }
            __syncthreads();
        }
    }
    // ---- arrival: the block's partial sums are released before thread 0
    // counts in, and the last block acquires every other block's.  The
    // counter wraps to 0 in the same atomic that counts the last block, so
    // no separate reset store can interleave with another arrival.
    if (threadIdx.x == 0) {
        const uint32_t nb = gridDim.x * gridDim.y;
        const uint32_t old = __builtin_amdgcn_atomic_inc32(F.arrive, nb - 1, __ATOMIC_ACQ_REL, "agent");
        is_last = old == nb - 1 ? 1u : 0u;
        arrival = old;
        ctl2 = F.C.control[2];
        ctl0 = F.C.control[0];
    }
    __syncthreads();
    // The blocks done before the last one quantize the hidden rows for the
    // gate/up projection, off the routing's critical path (a one-block grid
    // does it at its end).
    const uint32_t nb = gridDim.x * gridDim.y;
    if (!is_last) {
        if (F.quant) route_quant_rows(F.Q, arrival, nb - 1);
        return;
    }
    const uint32_t total_sel = F.P.k + F.P.always_count, total_res = E + F.P.always_count;
    const uint32_t T = total_res + total_res * (total_res - 1) / 2;
    const bool tel_in_lds = F.telemetry && T <= FR_LDS_TELEMETRY;
    if (tel_in_lds)
        for (uint32_t i = threadIdx.x; i < T; i += blockDim.x) tel[i] = 0;
    // Logits: the slices added in slice order, rounded to bf16.
    for (uint32_t i = threadIdx.x; i < B * E; i += blockDim.x) {
        float v[FR_MAX_SLICES];
#pragma unroll
        for (uint32_t sl = 0; sl < FR_MAX_SLICES; sl++)
            v[sl] = sl < F.slices ? coherent_load_f(F.part + (uint64_t)sl * B * E + i) : 0.0f;
        float sum = 0.0f;
#pragma unroll
        for (uint32_t sl = 0; sl < FR_MAX_SLICES; sl++)
            if (sl < F.slices) sum += v[sl];
        lg[i] = (uint16_t)f32_to_bf16(sum);
    }
    __syncthreads();
    // Top-k; routes and counts stay in LDS so that no barrier below waits for
    // global stores or atomics.  E <= 32 in the moe_topk form: two tokens per
    // wave; otherwise one token per wave.
    uint32_t* telp = F.telemetry ? (tel_in_lds ? tel : F.telemetry) : nullptr;
    if (F.P.mode == 0 && E <= 32) {
        // Waves without a token skip the call (it synchronizes nothing but
        // the wave): at B <= 16 the other half of the block would only add
        // to each SIMD's vector-ALU queue.
        for (uint32_t b0 = 0; b0 < B; b0 += 32)
            if (b0 + 2 * wave < B)
                topk_pair32(lg, E, F.bias, rl, telp, b0 + 2 * wave, B, F.P, t_raw[wave], tel_in_lds);
    } else {
        TopkScratch S{t_raw[wave], t_sel[wave], t_top[wave], t_wts[wave], &t_f[wave][0], &t_f[wave][1],
                      &t_u[wave][0], &t_u[wave][1]};
        const bool fast = F.P.mode == 0 && E <= 64;
        for (uint32_t b0 = 0; b0 < B; b0 += 16) {
            const uint32_t b = b0 + wave;
            if (fast) {
                if (b < B)   // wave-level only, like topk_pair32
                    topk_token_fast(lg + b * E, F.bias, rl, telp, b, true, F.P, tel_in_lds ? tel : nullptr, t_raw[wave]);
            }
            else topk_token(lg + (b < B ? b : 0) * E, F.bias, rl, telp, b, b < B, F.P, S, tel_in_lds ? tel : nullptr);
        }
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
    if (F.quant && nb == 1) route_quant_rows(F.Q, 0, 1);
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

// The same combine, 8 columns per thread with 16-byte loads and stores
// (H % 8 == 0, 16-byte aligned buffers).
__global__ __launch_bounds__(256) void reduce8_kernel(const uint16_t* __restrict__ eo, uint16_t* __restrict__ out,
                                                      uint32_t B, uint32_t H, uint32_t k, float routed_scale) {
    const uint32_t H8 = H / 8;
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (uint64_t)B * H8) return;
    const uint32_t b = (uint32_t)(idx / H8), j = (uint32_t)(idx % H8) * 8;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (uint32_t r = 0; r < k; r++) {
        const v4i v = *reinterpret_cast<const v4i*>(eo + ((uint64_t)b * k + r) * H + j);
        const uint32_t w[4] = {(uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
            acc[2 * q] = round_bf16(acc[2 * q] + bf16_to_f32(w[q] & 0xffffu));
            acc[2 * q + 1] = round_bf16(acc[2 * q + 1] + bf16_to_f32(w[q] >> 16));
        }
    }
    uint32_t o[4];
#pragma unroll
    for (int q = 0; q < 4; q++)
        o[q] = f32_to_bf16(acc[2 * q] * routed_scale) | (f32_to_bf16(acc[2 * q + 1] * routed_scale) << 16);
    *reinterpret_cast<v4i*>(out + (uint64_t)b * H + j) = v4i{(int)o[0], (int)o[1], (int)o[2], (int)o[3]};
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
                                           void* intermediates, void* control_u32, void* hidden_e4m3,
                                           void* hidden_scales_f32, uint32_t batch_width, void* stream) {
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
    if (!hidden_e4m3 != !hidden_scales_f32)
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "the quantized hidden rows need both the e4m3 and the scale buffer");
    if (hidden_scales_f32 && ((uintptr_t)hidden_scales_f32 & 3))
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "hidden scales must be 4-byte aligned");
    if (hidden_e4m3 && (ms.hidden % 4 || (((uintptr_t)hidden_e4m3 | (uintptr_t)x_bf16) & 3)))
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT,
                        "quantized hidden rows need hidden % 4 == 0 and 4-byte aligned hidden and e4m3 buffers");
    if (ts.experts != ms.experts || ts.k + ts.always_count != ms.k)
        return nh::fail(NERVE_HIP_INVALID_SPEC, "top-k and projection specializations disagree on experts or k");
    if (batch_width == 0) return nh::ok();
    const uint32_t H = ms.hidden;
    if (batch_width > FR_MAX_TOKENS || ts.experts > FR_MAX_EXPERTS || batch_width * ms.k > 1024 || ts.k > 128 ||
        ms.k > 128)
        return nh::fail(NERVE_HIP_UNSUPPORTED, "fused routing takes <= 64 tokens, <= 256 experts, <= 1024 routes");
    if (H % 8 == 0 && (((uintptr_t)x_bf16 | (uintptr_t)router_weight_bf16) & 15))
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "router buffers must be 16-byte aligned");
    // K slices: about 16 of the 32-k steps per slice (one per wave), at most 16.
    const uint32_t nsteps = (H + 31) / 32;
    const uint32_t slices = std::min<uint32_t>(FR_MAX_SLICES, std::max<uint32_t>(1u, (nsteps + 15) / 16));
    nh::Carver cv;
    const size_t o_part = cv.take<float>((size_t)slices * batch_width * ts.experts);
    void* ws = nullptr;
    if ((st = nh::workspace(ctx, cv.offset, &ws))) return st;
    float* part = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + o_part);
    FusedRouteArgs F;
    F.x = static_cast<const uint16_t*>(x_bf16);
    F.W = static_cast<const uint16_t*>(router_weight_bf16);
    F.H = H;
    F.slices = slices;
    F.arrive = ctx->sync_words;
    F.part = part;
    F.B = batch_width;
    F.logits = static_cast<uint16_t*>(logits_bf16);
    F.bias = bias;
    F.routes = static_cast<uint32_t*>(routes_u32);
    F.telemetry = static_cast<uint32_t*>(telemetry_u32);
    F.quant = hidden_e4m3 ? 1u : 0u;
    F.Q = QuantArgs{};
    F.Q.x = F.x;
    F.Q.k = 1;
    F.Q.frame_elems = H;
    F.Q.seg_elems = 0;
    F.Q.cols = H;
    F.Q.rows = batch_width;
    F.Q.q = static_cast<uint8_t*>(hidden_e4m3);
    F.Q.s = static_cast<float*>(hidden_scales_f32);
    F.Q.zero_word = nullptr;
    F.Q.ldq = H;
    F.Q.vec8 = ((((uintptr_t)F.Q.x | (uintptr_t)F.Q.q) & 15) == 0 && H % 8 == 0) ? 1u : 0u;
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
    route_fused_kernel<<<dim3((ts.experts + 15) / 16, slices), 1024, 0, (hipStream_t)stream>>>(F);
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
    if (hidden % 8 == 0 && (((uintptr_t)expert_outputs | (uintptr_t)out_bf16) & 15) == 0)
        reduce8_kernel<<<(unsigned)((total / 8 + 255) / 256), 256, 0, (hipStream_t)stream>>>(
            static_cast<const uint16_t*>(expert_outputs), static_cast<uint16_t*>(out_bf16), batch_width, hidden,
            experts_per_token, routed_scale);
    else
        reduce_kernel<<<(unsigned)((total + 255) / 256), 256, 0, (hipStream_t)stream>>>(
            static_cast<const uint16_t*>(expert_outputs), static_cast<uint16_t*>(out_bf16), batch_width, hidden,
            experts_per_token, routed_scale);
    return nh::check_launch("moe_reduce");
}

}  // extern "C"
