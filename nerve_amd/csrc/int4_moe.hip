// Sparse-expert INT4 (compressed-tensors) projections on gfx950:
// gate/up + SwiGLU and down + route weight.
//
// Reference: sparse_moe_gate_up_int4_ct.comp.template:97-227 and
// sparse_moe_down_int4_ct.comp.template:106-193 (rendered by
// nerve/model_package_sparse_projection_shaders.py:80-232).  Per route the
// shaders compute, for every output row, the f32 sum over packed words of
// fma(dot8(x, q - 8), scale[row, group], sum) with a 64-lane strided loop and
// subgroupAdd; gate/up then give bf16(bf16(silu(bf16 g)) * bf16 u) and down
// gives bf16(bf16(y) * route_weight).
//
// Work here is HBM-bound weight streaming (one activation row per route), so
// the kernel is organised around keeping 16-byte weight loads in flight:
//   * a block (4 waves) owns one route position and a tile of output rows;
//     each wave owns 8 weight rows (gate/up: 4 gate + the 4 matching up rows;
//     down: 8 rows) and issues all of its weight and scale loads of a pass
//     before the first arithmetic;
//   * lanes split a row into 16-byte chunks (32 codes), LU lanes per row, so
//     rows whose chunk count is not a multiple of 64 still fill the lanes;
//   * the activation row is staged once per block in LDS (4-byte loads: route
//     slices of the intermediate frames are only 4-byte aligned);
//   * codes become bf16 (128 + q) pairs with one and-or per two codes and
//     v_dot2_f32_bf16 contracts them with the activation pairs; the per-word
//     term 136 * sum(x) restores (q - 8).  Products are exact in f32; only the
//     summation order differs from the shader's (whose subgroupAdd order is
//     itself unspecified).
// Blocks are dealt to the XCDs in contiguous runs of (tile, position) work
// with positions fastest, so the routes of one expert (adjacent in the
// compacted map, which sorts routes by expert) read its rows through one L2.
#include "common.h"

namespace {

typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

constexpr uint32_t SM_WAVES = 4;
constexpr uint32_t SM_WROWS = 8;            // weight rows per wave
constexpr uint32_t SM_MAX_K = 16384;        // activation row staged in LDS
constexpr uint32_t SM_UNBOUND = 0xffffffffu;
constexpr uint32_t SM_ONES = 0x3F803F80u;   // bf16 (1, 1)

struct SmArgs {
    const uint16_t* x;          // gate_up: hidden bf16 [B, H]; down: the frames as bf16
    const uint32_t* routes;     // [B * k] route words
    const uint32_t* frames;     // intermediate frames (route map in the tails)
    uint16_t* out;              // gate_up: the frames as bf16; down: expert_outputs [B * k, H]
    const uint32_t* addr;
    const uint32_t* slots;
    const uint32_t* control;    // BatchControl, or null (unbatched form without an expert range)
    uint32_t n_records, n_slot_words;
    uint32_t batch_width, k, E;
    uint32_t K, N, I, G;        // contraction, output rows, intermediate size, group
    uint64_t frame_words;       // u32 words per frame (k * I / 2, + k route-map words when batched)
    uint32_t data_words;        // k * I / 2
    uint32_t tiles;             // row tiles per route
    uint32_t npos;              // route positions in the grid
    uint32_t per_xcd;           // grid / 8
    uint64_t w_bytes, s_bytes;  // bytes one expert's weight / scale tensor must span
    int batched, scale_bf16;
};

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2bf, a), __builtin_bit_cast(v2bf, b), c, false);
}

__device__ __forceinline__ float decode_scale(uint32_t v, int bf16) {
    return bf16 ? bf16_to_f32(v) : (float)__builtin_bit_cast(_Float16, (uint16_t)v);
}

// Pairs (0,4),(1,5),(2,6),(3,7) of 8 contiguous bf16: the order in which
// sm_word_dot decodes the codes of one packed word.
__device__ __forceinline__ v4i sm_permute(v4i a) {
    const uint32_t d0 = (uint32_t)a.x, d1 = (uint32_t)a.y, d2 = (uint32_t)a.z, d3 = (uint32_t)a.w;
    return v4i{(int)((d0 & 0xFFFFu) | (d2 << 16)), (int)((d0 >> 16) | (d2 & 0xFFFF0000u)),
               (int)((d1 & 0xFFFFu) | (d3 << 16)), (int)((d1 >> 16) | (d3 & 0xFFFF0000u))};
}

// sum_{i<8} x_i (128 + q_i) of one word (codes low nibble first along k)
// against permuted activations.
__device__ __forceinline__ float sm_word_dot(uint32_t w, v4i xp) {
    float d = dot2_bf16((uint32_t)xp.x, (w & 0x000F000Fu) | 0x43004300u, 0.0f);
    d = dot2_bf16((uint32_t)xp.y, ((w >> 4) & 0x000F000Fu) | 0x43004300u, d);
    d = dot2_bf16((uint32_t)xp.z, ((w >> 8) & 0x000F000Fu) | 0x43004300u, d);
    return dot2_bf16((uint32_t)xp.w, ((w >> 12) & 0x000F000Fu) | 0x43004300u, d);
}

__device__ __forceinline__ float sm_word_sum(v4i xp) {
    float s = dot2_bf16((uint32_t)xp.x, SM_ONES, 0.0f);
    s = dot2_bf16((uint32_t)xp.y, SM_ONES, s);
    s = dot2_bf16((uint32_t)xp.z, SM_ONES, s);
    return dot2_bf16((uint32_t)xp.w, SM_ONES, s);
}

// One 8-word address record (u32 {addr_lo, addr_hi, bytes_lo, bytes_hi, ...})
// behind parameter slot `idx`, or null.  The shaders only skip unbound slots
// (…gate_up_int4_ct.comp.template:163-166); slots beyond the table, null
// addresses, misaligned addresses and records shorter than the expert's tensor
// are treated the same way here instead of being read out of bounds.
__device__ __forceinline__ const void* sm_param(const SmArgs& A, uint32_t idx, uint64_t need, uint32_t align) {
    if (idx >= A.n_slot_words) return nullptr;
    const uint32_t slot = A.slots[idx];
    if (slot == SM_UNBOUND || slot >= A.n_records) return nullptr;
    const uint32_t* rec = A.addr + (uint64_t)slot * 8;
    const uint64_t a = (uint64_t)rec[0] | ((uint64_t)rec[1] << 32);
    const uint64_t bytes = (uint64_t)rec[2] | ((uint64_t)rec[3] << 32);
    if (a == 0 || (a & (align - 1)) || bytes < need) return nullptr;
    return reinterpret_cast<const void*>(a);
}

// LU: lanes per weight row (64, 32 or 16).  SPW: one scale per packed word
// (group sizes that are not a multiple of 32) instead of one per chunk.
template <bool GATE_UP, uint32_t LU, bool SPW>
__global__ __launch_bounds__(64 * SM_WAVES) void sparse_int4_kernel(SmArgs A) {
    constexpr uint32_t RS = 64 / LU;                  // rows loaded side by side
    constexpr uint32_t RPL = SM_WROWS / RS;           // rows per lane
    constexpr uint32_t NUP = 16 / RPL;                // chunks per lane per pass
    constexpr uint32_t OR = GATE_UP ? SM_WROWS / 2 : SM_WROWS;   // output rows per wave
    constexpr uint32_t NSC = SPW ? 4 : 1;
    extern __shared__ __attribute__((aligned(16))) uint16_t xs[];   // K activations

    // Work item: position fastest; contiguous runs of items per XCD.
    const uint32_t w = (blockIdx.x % 8) * A.per_xcd + blockIdx.x / 8;
    const uint32_t pos = w % A.npos, tile = w / A.npos;
    if (tile >= A.tiles) return;

    // Route of this position (…gate_up_int4_ct.comp.template:142-166 with
    // the batched ROUTE_MAPPING of nerve/model_package_sparse_projection_
    // shaders.py:194-212).
    // The map word and the control words are read together (every position
    // below B * k has a map word), so the chain of dependent loads before the
    // weights is map -> route -> slots -> records.
    const uint32_t cap = A.batch_width * A.k;
    uint32_t c = pos;
    uint32_t start = 0, count = 0, owned = cap;
    if (A.batched) c = A.frames[(uint64_t)(pos / A.k) * A.frame_words + A.data_words + pos % A.k];
    if (A.control) {
        start = A.control[1];
        count = A.control[2];
        if (A.batched) owned = A.control[3];
    }
    if (A.batched && count != 0u && pos >= owned) return;
    if (c >= cap) return;
    const uint32_t rw = A.routes[c];
    const uint32_t e = rw & 0xffffu;
    if (e >= A.E || (count != 0u && (e < start || e - start >= count))) return;
    const uint32_t* W = static_cast<const uint32_t*>(sm_param(A, 2 * e, A.w_bytes, 16));
    const uint16_t* S = static_cast<const uint16_t*>(sm_param(A, 2 * e + 1, A.s_bytes, 2));
    if (!W || !S) return;
    const uint32_t b = c / A.k, r = c % A.k;

    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t rsub = lane / LU, cl = lane % LU;
    const uint32_t K = A.K, kw = K / 8, units = K / 32, ng = K / A.G;
    const uint32_t orow0 = tile * (SM_WAVES * OR) + wave * OR;

    // Weight rows of this lane (clamped into the matrix; results of rows past
    // N are not stored).
    const uint32_t* wrow[RPL];
    const uint16_t* srow[RPL];
#pragma unroll
    for (uint32_t j = 0; j < RPL; j++) {
        const uint32_t li = rsub * RPL + j;
        uint32_t row;
        if constexpr (GATE_UP) row = min(orow0 + (li % OR), A.N - 1) + (li >= OR ? A.I : 0u);
        else row = min(orow0 + li, A.N - 1);
        wrow[j] = W + (uint64_t)row * kw;
        srow[j] = S + (uint64_t)row * ng;
    }

    // Activation row -> LDS.
    const uint16_t* xg = GATE_UP ? A.x + (uint64_t)b * K : A.x + (uint64_t)b * A.frame_words * 2 + (uint64_t)r * A.I;
    {
        const uint32_t* xg32 = reinterpret_cast<const uint32_t*>(xg);
        uint32_t* xs32 = reinterpret_cast<uint32_t*>(xs);
        for (uint32_t i = tid; i < K / 2; i += 64 * SM_WAVES) xs32[i] = xg32[i];
    }
    bool staged = false;

    float acc[RPL];
#pragma unroll
    for (uint32_t j = 0; j < RPL; j++) acc[j] = 0.0f;

    for (uint32_t u0 = 0; u0 < units; u0 += LU * NUP) {
        v4i wv[NUP][RPL];
        uint16_t sv[NUP][RPL][NSC];
#pragma unroll
        for (uint32_t i = 0; i < NUP; i++) {
            if (u0 + i * LU >= units) break;      // chunk slots past the row (uniform)
            const uint32_t un = min(u0 + i * LU + cl, units - 1);
            uint32_t gi[NSC];
#pragma unroll
            for (uint32_t q = 0; q < NSC; q++) gi[q] = (un * 32 + 8 * q) / A.G;
#pragma unroll
            for (uint32_t j = 0; j < RPL; j++) {
                wv[i][j] = *reinterpret_cast<const v4i*>(wrow[j] + un * 4);
#pragma unroll
                for (uint32_t q = 0; q < NSC; q++) sv[i][j][q] = srow[j][gi[q]];
            }
        }
        if (!staged) {
            __syncthreads();
            staged = true;
        }
#pragma unroll
        for (uint32_t i = 0; i < NUP; i++) {
            const uint32_t un = u0 + i * LU + cl;
            if (un >= units) continue;
            v4i xp[4];
            float sx[4];
#pragma unroll
            for (uint32_t q = 0; q < 4; q++) {
                xp[q] = sm_permute(*reinterpret_cast<const v4i*>(xs + un * 32 + 8 * q));
                sx[q] = -136.0f * sm_word_sum(xp[q]);
            }
#pragma unroll
            for (uint32_t j = 0; j < RPL; j++) {
                const uint32_t wj[4] = {(uint32_t)wv[i][j].x, (uint32_t)wv[i][j].y, (uint32_t)wv[i][j].z,
                                        (uint32_t)wv[i][j].w};
                if constexpr (SPW) {
#pragma unroll
                    for (uint32_t q = 0; q < 4; q++)
                        acc[j] = fmaf(sm_word_dot(wj[q], xp[q]) + sx[q], decode_scale(sv[i][j][q], A.scale_bf16), acc[j]);
                } else {
                    const float sc = decode_scale(sv[i][j][0], A.scale_bf16);
#pragma unroll
                    for (uint32_t q = 0; q < 4; q++) acc[j] = fmaf(sm_word_dot(wj[q], xp[q]) + sx[q], sc, acc[j]);
                }
            }
        }
    }

    // Row sums across the LU lanes of each row.
#pragma unroll
    for (uint32_t j = 0; j < RPL; j++) {
        acc[j] = lanes_sum_down<LU>(acc[j]);   // the __shfl_xor butterfly LU / 2, ..., 1
    }

    if constexpr (GATE_UP) {
        // Output row orow0 + t (t < OR) on lane t: gate = weight row t, up =
        // weight row OR + t.
        float gate = 0.0f, up = 0.0f;
#pragma unroll
        for (uint32_t li = 0; li < SM_WROWS; li++) {
            // lanes of row group li / RPL hold row li in acc[li % RPL]
            const float v = lane_bcast(acc[li % RPL], (li / RPL) * LU);
            if (li < OR && lane == li) gate = v;
            if (li >= OR && lane == li - OR) up = v;
        }
        const uint32_t row = orow0 + lane;
        if (lane < OR && row < A.N) {
            // …gate_up_int4_ct.comp.template:205-213
            const float g = round_bf16(gate), u = round_bf16(up);
            const float act = round_bf16(round_bf16(g / (1.0f + expf(-g))) * u);
            A.out[(uint64_t)b * A.frame_words * 2 + (uint64_t)r * A.I + row] = (uint16_t)f32_to_bf16(act);
        }
    } else {
        float y = 0.0f;
#pragma unroll
        for (uint32_t li = 0; li < SM_WROWS; li++) {
            const float v = lane_bcast(acc[li % RPL], (li / RPL) * LU);
            if (lane == li) y = v;
        }
        const uint32_t row = orow0 + lane;
        if (lane < OR && row < A.N) {
            // …down_int4_ct.comp.template:176-181
            const float wr = bf16_to_f32(rw >> 16);
            A.out[(uint64_t)c * A.N + row] = (uint16_t)f32_to_bf16(round_bf16(round_bf16(y) * wr));
        }
    }
}

template <bool GATE_UP>
nerve_hip_status launch_sparse(const SmArgs& A, hipStream_t stream) {
    const uint32_t units = A.K / 32;
    const bool spw = A.G % 32 != 0;
    const uint32_t lu = units % 64 == 0 ? 64u : (units % 32 == 0 || units > 32) ? 32u : 16u;
    const dim3 grid(A.per_xcd * 8), block(64 * SM_WAVES);
#define SM_LAUNCH(LU, SPW) sparse_int4_kernel<GATE_UP, LU, SPW><<<grid, block, A.K * 2, stream>>>(A)
    if (spw) {
        if (lu == 64) SM_LAUNCH(64, true);
        else if (lu == 32) SM_LAUNCH(32, true);
        else SM_LAUNCH(16, true);
    } else {
        if (lu == 64) SM_LAUNCH(64, false);
        else if (lu == 32) SM_LAUNCH(32, false);
        else SM_LAUNCH(16, false);
    }
#undef SM_LAUNCH
    return nh::check_launch(GATE_UP ? "int4_moe_gate_up" : "int4_moe_down");
}

nerve_hip_status sparse_common(nerve_hip_ctx* ctx, const char* spec, bool gate_up, const void* x,
                               const void* routes, void* intermediates, void* expert_outputs,
                               const void* addresses, uint32_t address_records, const void* slots,
                               uint32_t slot_words, const void* control, uint32_t batch_width, void* stream) {
    nerve_hip_status st = nh::enter(ctx);
    if (st) return st;
    nh::MoeSpec ms;
    if ((st = nh::parse_moe_spec(spec, &ms))) return st;
    if (ms.family != 1) return nh::fail(NERVE_HIP_INVALID_SPEC, std::string("not an INT4 sparse expert kernel: ") + spec);
    if (ms.gate_up != gate_up)
        return nh::fail(NERVE_HIP_INVALID_SPEC, gate_up ? "gate_up entry given a down specialization"
                                                        : "down entry given a gate_up specialization");
    if (!x || !routes || !intermediates || !addresses || !slots || (gate_up ? false : !expert_outputs) ||
        (ms.batch1 && !control))
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "null buffer");
    const uint32_t H = ms.hidden, I = ms.inter, k = ms.k;
    const uint32_t K = gate_up ? H : I, N = gate_up ? I : H;
    if (K % 32) return nh::fail(NERVE_HIP_UNSUPPORTED, "INT4 sparse experts need an input width that is a multiple of 32");
    if (K > SM_MAX_K) return nh::fail(NERVE_HIP_UNSUPPORTED, "INT4 sparse experts take input widths up to 16384");
    if (!ms.batch1 && batch_width != 1)
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "the unbatched INT4 expert form runs one token (batch_width 1)");
    if (((uintptr_t)x | (uintptr_t)intermediates) & 3) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "activation buffers must be 4-byte aligned");
    const uint64_t cap = (uint64_t)batch_width * k;
    if (cap == 0) return nh::ok();
    if (cap > (1u << 24)) return nh::fail(NERVE_HIP_UNSUPPORTED, "too many routes");
    SmArgs A{};
    A.x = static_cast<const uint16_t*>(x);
    A.routes = static_cast<const uint32_t*>(routes);
    A.frames = static_cast<const uint32_t*>(intermediates);
    A.out = static_cast<uint16_t*>(gate_up ? intermediates : expert_outputs);
    A.addr = static_cast<const uint32_t*>(addresses);
    A.slots = static_cast<const uint32_t*>(slots);
    A.control = static_cast<const uint32_t*>(control);
    A.n_records = address_records;
    A.n_slot_words = slot_words;
    A.batch_width = batch_width;
    A.k = k;
    A.E = ms.experts;
    A.K = K;
    A.N = N;
    A.I = I;
    A.G = ms.group;
    A.data_words = k * I / 2;
    A.frame_words = (uint64_t)A.data_words + (ms.batch1 ? k : 0u);
    A.tiles = (N + SM_WAVES * (gate_up ? SM_WROWS / 2 : SM_WROWS) - 1) / (SM_WAVES * (gate_up ? SM_WROWS / 2 : SM_WROWS));
    A.npos = (uint32_t)cap;
    A.per_xcd = (uint32_t)(((uint64_t)A.npos * A.tiles + 7) / 8);
    const uint64_t wrows = gate_up ? 2ull * I : (uint64_t)H;
    A.w_bytes = wrows * K / 2;
    A.s_bytes = wrows * (K / ms.group) * 2;
    A.batched = ms.batch1 ? 1 : 0;
    A.scale_bf16 = ms.scale_bf16;
    return gate_up ? launch_sparse<true>(A, (hipStream_t)stream) : launch_sparse<false>(A, (hipStream_t)stream);
}

}  // namespace

extern "C" {

nerve_hip_status nerve_hip_int4_moe_gate_up(nerve_hip_ctx* ctx, const char* spec, const void* hidden_bf16,
                                            const void* routes_u32, void* intermediates, const void* addresses_u32,
                                            uint32_t address_records, const void* param_slots_u32,
                                            uint32_t param_slot_words, const void* control_u32, uint32_t batch_width,
                                            void* stream) {
    return sparse_common(ctx, spec, true, hidden_bf16, routes_u32, intermediates, nullptr, addresses_u32,
                         address_records, param_slots_u32, param_slot_words, control_u32, batch_width, stream);
}

nerve_hip_status nerve_hip_int4_moe_down(nerve_hip_ctx* ctx, const char* spec, const void* intermediates,
                                         const void* routes_u32, void* expert_outputs, const void* addresses_u32,
                                         uint32_t address_records, const void* param_slots_u32,
                                         uint32_t param_slot_words, const void* control_u32, uint32_t batch_width,
                                         void* stream) {
    return sparse_common(ctx, spec, false, intermediates, routes_u32, const_cast<void*>(intermediates),
                         expert_outputs, addresses_u32, address_records, param_slots_u32, param_slot_words,
                         control_u32, batch_width, stream);
}

}  // extern "C"
