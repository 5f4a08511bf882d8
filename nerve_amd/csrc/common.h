// Shared device numerics and host plumbing for libnerve_hip (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/nerve_hip.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------------------
// Device numerics.  Each helper restates one rounding rule of the reference
// shaders bit for bit.
// ---------------------------------------------------------------------------

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float((h & 0xffffu) << 16); }

// bf16 round-to-nearest-even as the templates do it
// (independent_sparse_moe_gate_up_batch1_mxfp4.comp.template:92-96).
__device__ __forceinline__ uint32_t f32_to_bf16(float v) {
    uint32_t b = __float_as_uint(v);
    return (b + 0x7fffu + ((b >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ float round_bf16(float v) { return bf16_to_f32(f32_to_bf16(v)); }

// f32 -> OCP e4m3 with round-to-nearest-even and saturation at +-448: the
// GLSL fe4m3vec4(x) conversion of the activation quantizers
// (…gate_up_batch1_mxfp4.comp.template:380).
// Written without branches (both paths computed, then selected), which keeps
// per-lane quantization loops free of divergent control flow.
__device__ __forceinline__ uint32_t f32_to_e4m3(float x) {
    const uint32_t b = __float_as_uint(x), sign = (b >> 24) & 0x80u, a = b & 0x7fffffffu;
    // below 2^-6: the subnormal grid of 2^-9 (clamped so the conversion is
    // always in range; the value is only selected below 2^-6)
    const uint32_t sub = (uint32_t)__builtin_rintf(fminf(__uint_as_float(a) * 512.0f, 8.0f));
    const uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);
    const uint32_t e4 = (r >> 23) - 120u, m = (r >> 20) & 7u;
    const uint32_t nrm = (e4 > 15u && e4 < 0x80000000u) || (e4 == 15u && m == 7u) ? 0x7eu : ((e4 << 3) | m) & 0x7fu;
    const uint32_t v = a > 0x7f800000u ? 0x7fu : a < 0x3c800000u ? sub : nrm;
    return sign | v;
}

// rounded_fp8_scale (…gate_up_batch1_mxfp4.comp.template:357-363).
__device__ __forceinline__ float pow2_fp8_scale(float block_max) {
    float ratio = fmaxf(block_max, 1e-4f) / 448.0f;
    uint32_t bits = __float_as_uint(ratio);
    int exponent = (int)((bits >> 23) & 0xffu) - 127;
    if ((bits & 0x7fffffu) != 0u) exponent++;
    return __uint_as_float((uint32_t)(exponent + 127) << 23);
}

// amax/448 scale (tied_output_projection_fp8_e4m3.comp.template:99).
__device__ __forceinline__ float amax_fp8_scale(float block_max) {
    return block_max > 0.0f ? block_max / 448.0f : 1.0f;
}

// e8m0 byte of a power-of-two f32 scale (its biased exponent field).
__device__ __forceinline__ uint32_t pow2_to_e8m0(float s) { return (__float_as_uint(s) >> 23) & 0xffu; }

// Lane sums over aligned groups of lanes without the LDS-routed shuffles:
// DPP row operations within 16-lane rows and the gfx950 row swaps across
// rows.  At every step the partner lane holds the value the __shfl_xor
// butterfly would pair (an xor partner, or one holding the same value once
// the previous steps made the smaller groups uniform), and each lane adds
// own + partner, so the results are those of that butterfly bit for bit.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float sum_xor16(float v) {   // v + v of lane ^ 16
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float v) {   // v + v of lane ^ 32
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// The butterfly with partners lane ^ 1, ^ 2, ..., ^ (L / 2) (L = 2 .. 32).
template <uint32_t L>
__device__ __forceinline__ float lanes_sum_up(float v) {
    if constexpr (L >= 2) v += dpp_f32<0xB1>(v);    // quad_perm [1,0,3,2]: lane ^ 1
    if constexpr (L >= 4) v += dpp_f32<0x4E>(v);    // quad_perm [2,3,0,1]: lane ^ 2
    if constexpr (L >= 8) v += dpp_f32<0x141>(v);   // row_half_mirror: the other quad of the 8
    if constexpr (L >= 16) v += dpp_f32<0x140>(v);  // row_mirror: the other 8 of the row
    if constexpr (L >= 32) v = sum_xor16(v);
    return v;
}
// The butterfly with partners lane ^ (L / 2), ..., ^ 2, ^ 1 (L = 16, 32, 64).
template <uint32_t L>
__device__ __forceinline__ float lanes_sum_down(float v) {
    static_assert(L == 16 || L == 32 || L == 64, "lane group");
    if constexpr (L >= 64) v = sum_xor32(v);
    if constexpr (L >= 32) v = sum_xor16(v);
    v += dpp_f32<0x128>(v);   // row_ror:8 = lane ^ 8
    v += dpp_f32<0x124>(v);   // row_ror:4 (pairs {i, i ^ 8} uniform)
    v += dpp_f32<0x122>(v);   // row_ror:2
    v += dpp_f32<0x121>(v);   // row_ror:1
    return v;
}
// Lane `src` (a compile-time or uniform index) to every lane.
__device__ __forceinline__ float lane_bcast(float v, uint32_t src) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src));
}

__device__ __forceinline__ float wave_max32(float v) {
    // Reduction inside each 32-lane half of the wave (subgroupClusteredMax(v, 32)).
    v = fmaxf(v, __shfl_xor(v, 16));
    v = fmaxf(v, __shfl_xor(v, 8));
    v = fmaxf(v, __shfl_xor(v, 4));
    v = fmaxf(v, __shfl_xor(v, 2));
    v = fmaxf(v, __shfl_xor(v, 1));
    return v;
}

// ---------------------------------------------------------------------------
// Host side: context, errors, workspace.
// ---------------------------------------------------------------------------

struct nerve_hip_ctx {
    int device;
    int cu_count;
    void* workspace;
    size_t workspace_bytes;
    void* static_scratch;         // device address of this device's static scratch array
    uint32_t* sync_words;         // arrival counters of single-launch reductions (zeroed at open)
};

namespace nh {

// Size of the file-scope device array behind the no-allocation entry point.
constexpr size_t kStaticScratchBytes = 4u << 20;

nerve_hip_status fail(nerve_hip_status code, const std::string& msg);
nerve_hip_status ok();
// Makes ctx's device current and validates ctx itself.
nerve_hip_status enter(nerve_hip_ctx* ctx);
// Grows the context workspace to at least `bytes` (may synchronize the device
// when it has to grow).  Returns the device pointer through `out`.
nerve_hip_status workspace(nerve_hip_ctx* ctx, size_t bytes, void** out);
// Checks the launch status of the last kernel.
nerve_hip_status check_launch(const char* what);

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Carves aligned sub-buffers out of one workspace allocation.
struct Carver {
    size_t offset = 0;
    template <typename T>
    size_t take(size_t count) {
        offset = align_up(offset, 256);
        size_t at = offset;
        offset += count * sizeof(T);
        return at;
    }
};

// ---- specialization strings (reference grammar, nerve/model_package_shader_templates.py) ----

struct MoeSpec {
    bool gate_up = false;       // gate_up vs down
    bool batch1 = false;
    bool tensor_parallel = false;
    bool prequant = false;
    bool input_block_major = false;
    int weight_repr = 0;        // 0 compact, 1 resident_fp8_e4m3, 2 adaptive_fp8_e4m3
    int native_fp8_start = -1;
    uint32_t hidden = 0, inter = 0, experts = 0, k = 0;
    bool has_limit = false;
    float limit = 0.0f;
    // 0: independent_sparse_moe_*_mxfp4 (demand-addressed MXFP4 experts);
    // 1: sparse_moe_*_int4_ct (compressed-tensors INT4 experts, bf16 or f16
    //    group scales, 16-row tiles).
    int family = 0;
    int scale_bf16 = 0;
    uint32_t group = 0;
};
nerve_hip_status parse_moe_spec(const char* spec, MoeSpec* out);

// TILES_PER_ROUTE of an expert projection: the rows one reference workgroup
// produces per route (MXFP4: 32-row gate_up and 64-row down tiles,
// nerve/model_package_shader_templates.py:4836; INT4-CT: 16-row tiles,
// nerve/model_package_common.py:64).
inline uint32_t moe_tiles_per_route(const MoeSpec& m) {
    if (m.family == 1) return ((m.gate_up ? m.inter : m.hidden) + 15) / 16;
    return m.gate_up ? (m.inter + 31) / 32 : (m.hidden + 63) / 64;
}

struct TopkSpec {
    int mode = 0;               // 0 moe_topk, 1 moe_router_score_topk
    int activation = 0;         // mode 0: 1 = sigmoid; mode 1: 0 sigmoid, 1 softmax, 2 sqrtsoftplus
    uint32_t experts = 0, k = 0, always_count = 0;
    float always_weight = 0.0f;
    int normalize = 0;
    float softcap = 0.0f;
    float routed_scale = 1.0f;
    int bias = 0;               // 0 none, 1 f32, 2 bf16
};
nerve_hip_status parse_topk_spec(const char* spec, TopkSpec* out);

struct Int4Spec {
    int op = 0;                 // 0 linear, 1 linear_bias, 2 linear_residual
    int batch_tile = 0;         // 0 = unbatched form
    int layout = 0;             // 0 gptq, 1 ct
    int scale_bf16 = 0;
    int input = 0;              // 0 bf16, 1 "_prequant" int8, 2 "_prequant_pairpacked" int8
    bool cooperative = false;   // "_batch64_cooperative_" (batch-64 tiles of group sums)
    uint32_t group = 0, in = 0, out = 0;
};
nerve_hip_status parse_int4_spec(const char* spec, Int4Spec* out);

struct QuantI8Spec {
    int batch_tile = 0;
    bool paired = true;         // pair-packed byte order (with block sums) vs columns in order
    bool silu = false;          // silu_multiply_quantize_* (two bf16 inputs, bf16 output)
    uint32_t block = 0, elements = 0;
};
nerve_hip_status parse_quant_i8_spec(const char* spec, QuantI8Spec* out);

struct Fp8HeadSpec {
    int batch_tile = 0;
    uint32_t block_rows = 0, block_cols = 0, vocab = 0, in = 0;
    float output_scale = 1.0f;
};
nerve_hip_status parse_fp8_head_spec(const char* spec, Fp8HeadSpec* out);

struct QuantSpec {
    int batch_tile = 0;
    bool pow2 = false;
    uint32_t block = 0, elements = 0;
};
nerve_hip_status parse_quant_spec(const char* spec, QuantSpec* out);

struct RmsQuantSpec {
    int batch_tile = 0;
    bool int8pp = false;        // int8_pairpacked output instead of fp8_e4m3
    bool pow2 = false;
    uint32_t block = 0, hidden = 0;
    float eps = 0.0f, offset = 0.0f;
};
nerve_hip_status parse_rms_quant_spec(const char* spec, RmsQuantSpec* out);

}  // namespace nh
