// Context lifecycle, thread-local errors, workspace and specialization-string
// parsing for libnerve_hip.
#include <cstdarg>
#include <cstdlib>
#include <regex>
#include <string>
#include <unordered_map>

#include "common.h"

namespace {
thread_local std::string g_last_error;
}

// Scratch of nerve_hip_fp8_output_projection_noalloc: every device holds its
// own copy of this array until the process ends.  In host code the name is
// only a stand-in; nerve_hip_open resolves each device's copy to a device
// address with hipGetSymbolAddress, and only that address is ever used.
static __device__ __align__(256) uint8_t scratch[nh::kStaticScratchBytes];

namespace nh {

nerve_hip_status fail(nerve_hip_status code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

nerve_hip_status ok() { return NERVE_HIP_OK; }

nerve_hip_status enter(nerve_hip_ctx* ctx) {
    if (!ctx) return fail(NERVE_HIP_INVALID_ARGUMENT, "null nerve_hip_ctx");
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return fail(NERVE_HIP_DEVICE_ERROR, std::string("hipSetDevice: ") + hipGetErrorString(e));
    return NERVE_HIP_OK;
}

nerve_hip_status workspace(nerve_hip_ctx* ctx, size_t bytes, void** out) {
    if (bytes == 0) bytes = 256;
    if (ctx->workspace_bytes < bytes) {
        if (ctx->workspace) {
            // hipFree waits for work that may still use the old allocation.
            (void)hipDeviceSynchronize();
            (void)hipFree(ctx->workspace);
            ctx->workspace = nullptr;
            ctx->workspace_bytes = 0;
        }
        size_t grow = align_up(bytes + bytes / 4, 1 << 20);
        hipError_t e = hipMalloc(&ctx->workspace, grow);
        if (e != hipSuccess) {
            ctx->workspace = nullptr;
            return fail(NERVE_HIP_OUT_OF_MEMORY, std::string("workspace hipMalloc: ") + hipGetErrorString(e));
        }
        ctx->workspace_bytes = grow;
    }
    *out = ctx->workspace;
    return NERVE_HIP_OK;
}

nerve_hip_status check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(NERVE_HIP_DEVICE_ERROR, std::string(what) + ": " + hipGetErrorString(e));
    return NERVE_HIP_OK;
}

static bool parse_float(const std::string& s, float* out) {
    char* end = nullptr;
    float v = strtof(s.c_str(), &end);
    if (!end || *end != '\0' || s.empty()) return false;
    *out = v;
    return true;
}

static bool parse_u32(const std::string& s, uint32_t* out) {
    if (s.empty() || s.size() > 9) return false;
    *out = (uint32_t)strtoul(s.c_str(), nullptr, 10);
    return true;
}

// nerve/model_package_shader_templates.py:4773-4846
// nerve/model_package_sparse_projection_shaders.py:80-125
static nerve_hip_status parse_int4_moe_spec(const char* spec, MoeSpec* out) {
    static const std::regex re(
        "sparse_moe_(gate_up|down)(?:_batch(\\d+))?_int4_ct_s(f16|bf16)_g(\\d+)_"
        "h(\\d+)_i(\\d+)_e(\\d+)_k(\\d+)\\.comp");
    std::cmatch m;
    if (!std::regex_match(spec, m, re)) return NERVE_HIP_UNSUPPORTED;
    MoeSpec s;
    s.family = 1;
    s.gate_up = m[1].str() == "gate_up";
    if (m[2].matched && m[2].str() != "1")
        return fail(NERVE_HIP_INVALID_SPEC, "INT4 sparse experts support only frame-parallel batch tiles");
    s.batch1 = m[2].matched;
    s.scale_bf16 = m[3].str() == "bf16";
    if (!parse_u32(m[4].str(), &s.group) || !parse_u32(m[5].str(), &s.hidden) || !parse_u32(m[6].str(), &s.inter) ||
        !parse_u32(m[7].str(), &s.experts) || !parse_u32(m[8].str(), &s.k))
        return fail(NERVE_HIP_INVALID_SPEC, std::string("bad shape in ") + spec);
    const uint32_t in_w = s.gate_up ? s.hidden : s.inter, out_w = s.gate_up ? s.inter : s.hidden;
    if (s.group == 0 || s.group % 8 || in_w == 0 || in_w % s.group || in_w % 8 || out_w == 0 || out_w % 2 ||
        !(0 < s.k && s.k <= s.experts && s.experts <= 4096))
        return fail(NERVE_HIP_INVALID_SPEC, std::string("invalid INT4 sparse expert geometry ") + spec);
    *out = s;
    return NERVE_HIP_OK;
}

static nerve_hip_status parse_moe_spec_uncached(const char* spec, MoeSpec* out) {
    if (!spec) return fail(NERVE_HIP_INVALID_SPEC, "null specialization");
    {
        nerve_hip_status st = parse_int4_moe_spec(spec, out);
        if (st != NERVE_HIP_UNSUPPORTED) return st;
    }
    static const std::regex re(
        "independent_sparse_moe_(gate_up|down)(?:_(batch1))?"
        "(?:_(tensor_parallel))?"
        "(?:_(prequant))?_"
        "(?:(input_block_major_b128)_)?"
        "mxfp4_e2m1(?:_(resident_fp8_e4m3|adaptive_fp8_e4m3))?_g32"
        "(?:_native_fp8_e4m3_se8m0_b128_nf(\\d+))?_"
        "h(\\d+)_i(\\d+)_e(\\d+)_k(\\d+)"
        "(?:_limit([0-9eE+.-]+))?\\.comp");
    std::cmatch m;
    if (!std::regex_match(spec, m, re)) return fail(NERVE_HIP_INVALID_SPEC, std::string("not an MXFP4 expert kernel: ") + spec);
    MoeSpec s;
    s.gate_up = m[1].str() == "gate_up";
    s.batch1 = m[2].matched;
    s.tensor_parallel = m[3].matched;
    s.prequant = m[4].matched;
    s.input_block_major = m[5].matched;
    s.weight_repr = !m[6].matched ? 0 : (m[6].str() == "resident_fp8_e4m3" ? 1 : 2);
    uint32_t nf = 0;
    if (m[7].matched) { parse_u32(m[7].str(), &nf); s.native_fp8_start = (int)nf; }
    if (!parse_u32(m[8].str(), &s.hidden) || !parse_u32(m[9].str(), &s.inter) ||
        !parse_u32(m[10].str(), &s.experts) || !parse_u32(m[11].str(), &s.k))
        return fail(NERVE_HIP_INVALID_SPEC, std::string("bad shape in ") + spec);
    s.has_limit = m[12].matched;
    if (s.has_limit && !parse_float(m[12].str(), &s.limit)) return fail(NERVE_HIP_INVALID_SPEC, std::string("bad limit in ") + spec);
    // Reference validation, with the 128-multiple rule relaxed to 32 (the
    // MX group) under zero-padded tail-block semantics.
    if (s.hidden == 0 || s.hidden % 32 || s.inter == 0 || s.inter % 32 || !(0 < s.k && s.k <= s.experts) ||
        s.gate_up != s.has_limit || s.experts > 65536)
        return fail(NERVE_HIP_INVALID_SPEC, std::string("invalid demand-addressed MXFP4 expert kernel ") + spec);
    // Native FP8 banks: 0 < start < E, not with tensor-parallel partials or
    // the block-major layout (nerve/model_package_shader_templates.py:4809-4817).
    if (s.native_fp8_start >= 0 && (s.native_fp8_start == 0 || (uint32_t)s.native_fp8_start >= s.experts ||
                                    s.input_block_major || s.tensor_parallel))
        return fail(NERVE_HIP_INVALID_SPEC, std::string("invalid native FP8 expert range in ") + spec);
    // input_block_major_b128 is a down-weight layout
    // (nerve/model_package_independent_experts.py:164-170) and needs whole
    // 128-column blocks.
    if (s.input_block_major && (s.gate_up || s.inter % 128))
        return fail(NERVE_HIP_INVALID_SPEC, std::string("input_block_major_b128 needs a down kernel with I % 128 == 0: ") + spec);
    if (s.prequant && !s.gate_up) return fail(NERVE_HIP_INVALID_SPEC, "prequant applies to gate_up only");
    // A tensor-parallel down slice reads block-major weights, and only it
    // (nerve/model_package_shader_templates.py:4818-4821).
    if (s.tensor_parallel && s.gate_up == s.input_block_major)
        return fail(NERVE_HIP_INVALID_SPEC, std::string("tensor-parallel slices: down needs input_block_major_b128, gate_up must not have it: ") + spec);
    *out = s;
    return NERVE_HIP_OK;
}

// nerve/model_package_shader_templates.py:4850-4915 and :5003-5060
static nerve_hip_status parse_topk_spec_uncached(const char* spec, TopkSpec* out) {
    if (!spec) return fail(NERVE_HIP_INVALID_SPEC, "null specialization");
    static const std::regex topk(
        "moe_topk(?:_batch(\\d+))?_(sigmoid|softmax)_bf16_e(\\d+)_k(\\d+)_"
        "norm([01])_cap([0-9eE+.-]+)_(biasf32|biasbf16|nobias)\\.comp");
    static const std::regex score(
        "moe_router(?:_(batch1))?_score_topk_(sigmoid|softmax|sqrtsoftplus)_bf16_r(\\d+)_k(\\d+)_"
        "a(\\d+)w([0-9eE+.-]+)_norm([01])_scale([0-9eE+.-]+)_bias(f32|bf16)\\.comp");
    std::cmatch m;
    TopkSpec s;
    if (std::regex_match(spec, m, topk)) {
        if (m[1].matched && m[1].str() != "1") return fail(NERVE_HIP_INVALID_SPEC, "sparse routing supports only frame-parallel batch tiles");
        s.mode = 0;
        s.activation = m[2].str() == "sigmoid" ? 1 : 0;
        parse_u32(m[3].str(), &s.experts);
        parse_u32(m[4].str(), &s.k);
        s.normalize = m[5].str() == "1";
        if (!parse_float(m[6].str(), &s.softcap)) return fail(NERVE_HIP_INVALID_SPEC, "bad softcap");
        std::string b = m[7].str();
        s.bias = b == "nobias" ? 0 : (b == "biasf32" ? 1 : 2);
    } else if (std::regex_match(spec, m, score)) {
        s.mode = 1;
        std::string a = m[2].str();
        s.activation = a == "sigmoid" ? 0 : (a == "softmax" ? 1 : 2);
        parse_u32(m[3].str(), &s.experts);
        parse_u32(m[4].str(), &s.k);
        parse_u32(m[5].str(), &s.always_count);
        if (!parse_float(m[6].str(), &s.always_weight)) return fail(NERVE_HIP_INVALID_SPEC, "bad always-selected weight");
        s.normalize = m[7].str() == "1";
        if (!parse_float(m[8].str(), &s.routed_scale)) return fail(NERVE_HIP_INVALID_SPEC, "bad routed scale");
        s.bias = m[9].str() == "f32" ? 1 : 2;
    } else {
        return fail(NERVE_HIP_INVALID_SPEC, std::string("not a top-k routing kernel: ") + spec);
    }
    if (!(0 < s.k && s.k <= s.experts && s.experts <= 4096) || s.experts + s.always_count > 4096 || s.k + s.always_count > 64)
        return fail(NERVE_HIP_INVALID_SPEC, std::string("invalid sparse expert routing ") + spec);
    *out = s;
    return NERVE_HIP_OK;
}

// nerve/model_package_shader_templates.py:3219-3276, and the batch-64
// cooperative form (:3148-3215), which computes the same group sums.
static nerve_hip_status parse_int4_spec_uncached(const char* spec, Int4Spec* out) {
    if (!spec) return fail(NERVE_HIP_INVALID_SPEC, "null specialization");
    static const std::regex re(
        "(linear|linear_bias|linear_residual)(_prequant_pairpacked|_prequant)?(?:_batch(\\d+))?_int4_(gptq|ct)_s(f16|bf16)_g(\\d+)_"
        "(\\d+)x(\\d+)\\.comp");
    static const std::regex coop(
        "(linear|linear_bias|linear_residual)_batch64_cooperative_int4_(gptq|ct)_s(f16|bf16)_g(\\d+)_(\\d+)x(\\d+)\\.comp");
    std::cmatch m;
    if (std::regex_match(spec, m, coop)) {
        Int4Spec s;
        std::string op = m[1].str();
        s.op = op == "linear" ? 0 : (op == "linear_bias" ? 1 : 2);
        s.batch_tile = 64;
        s.cooperative = true;
        s.layout = m[2].str() == "gptq" ? 0 : 1;
        s.scale_bf16 = m[3].str() == "bf16";
        parse_u32(m[4].str(), &s.group);
        parse_u32(m[5].str(), &s.in);
        parse_u32(m[6].str(), &s.out);
        if (s.group == 0 || s.group % 32 || s.in == 0 || s.in % s.group || s.out == 0 || s.out % 2)
            return fail(NERVE_HIP_INVALID_SPEC, std::string("invalid cooperative INT4 shape ") + spec);
        *out = s;
        return NERVE_HIP_OK;
    }
    if (!std::regex_match(spec, m, re)) return fail(NERVE_HIP_INVALID_SPEC, std::string("not an INT4 linear kernel: ") + spec);
    Int4Spec s;
    std::string op = m[1].str();
    s.op = op == "linear" ? 0 : (op == "linear_bias" ? 1 : 2);
    s.input = !m[2].matched ? 0 : (m[2].str() == "_prequant" ? 1 : 2);
    uint32_t bt = 0;
    if (m[3].matched) parse_u32(m[3].str(), &bt);
    s.batch_tile = (int)bt;
    s.layout = m[4].str() == "gptq" ? 0 : 1;
    s.scale_bf16 = m[5].str() == "bf16";
    parse_u32(m[6].str(), &s.group);
    parse_u32(m[7].str(), &s.in);
    parse_u32(m[8].str(), &s.out);
    if (s.group == 0 || s.group % 32 || s.in == 0 || s.in % s.group || s.out == 0 || s.out % 2 ||
        (m[3].matched && bt == 0))
        return fail(NERVE_HIP_INVALID_SPEC, std::string("invalid native INT4 shape ") + spec);
    // nerve/model_package_shader_templates.py:3231-3235
    if (s.input == 2 && s.layout != 0)
        return fail(NERVE_HIP_INVALID_SPEC, std::string("pair-packed INT8 input requires GPTQ weights: ") + spec);
    *out = s;
    return NERVE_HIP_OK;
}

// nerve/model_package_shader_templates.py:2419-2465 (the output-scale token is
// accepted as any float literal: the manifest writes it with format ".9g",
// nerve/model_package_manifest.py:530-545).
static nerve_hip_status parse_fp8_head_spec_uncached(const char* spec, Fp8HeadSpec* out) {
    if (!spec) return fail(NERVE_HIP_INVALID_SPEC, "null specialization");
    static const std::regex re(
        "tied_output_projection(?:_batch(\\d+))?_fp8_e4m3_b(\\d+)x(\\d+)_(\\d+)x(\\d+)_scale([0-9eE+.-]+)_to_f32\\.comp");
    std::cmatch m;
    if (!std::regex_match(spec, m, re)) return fail(NERVE_HIP_INVALID_SPEC, std::string("not an FP8 output projection: ") + spec);
    Fp8HeadSpec s;
    uint32_t bt = 0;
    if (m[1].matched) parse_u32(m[1].str(), &bt);
    s.batch_tile = (int)bt;
    parse_u32(m[2].str(), &s.block_rows);
    parse_u32(m[3].str(), &s.block_cols);
    parse_u32(m[4].str(), &s.vocab);
    parse_u32(m[5].str(), &s.in);
    if (!parse_float(m[6].str(), &s.output_scale)) return fail(NERVE_HIP_INVALID_SPEC, "bad output scale");
    if ((m[1].matched && bt == 0) || s.block_rows == 0 || s.block_cols != 128 || s.in == 0 || s.in % 32 || s.vocab == 0)
        return fail(NERVE_HIP_INVALID_SPEC, std::string("invalid FP8 output projection shader shape ") + spec);
    *out = s;
    return NERVE_HIP_OK;
}

// nerve/model_package_shader_templates.py:1513-1545
static nerve_hip_status parse_quant_spec_uncached(const char* spec, QuantSpec* out) {
    if (!spec) return fail(NERVE_HIP_INVALID_SPEC, "null specialization");
    static const std::regex re("quantize(?:_batch(\\d+))?_fp8_e4m3(?:_(spow2))?_b(\\d+)_h(\\d+)\\.comp");
    std::cmatch m;
    if (!std::regex_match(spec, m, re)) return fail(NERVE_HIP_INVALID_SPEC, std::string("not an FP8 activation quantizer: ") + spec);
    QuantSpec s;
    uint32_t bt = 0;
    if (m[1].matched) parse_u32(m[1].str(), &bt);
    s.batch_tile = (int)bt;
    s.pow2 = m[2].matched;
    parse_u32(m[3].str(), &s.block);
    parse_u32(m[4].str(), &s.elements);
    if ((m[1].matched && bt == 0) || s.block != 128 || s.elements == 0 || s.elements % 32)
        return fail(NERVE_HIP_INVALID_SPEC, std::string("invalid FP8 activation-quantizer shape ") + spec);
    *out = s;
    return NERVE_HIP_OK;
}


// nerve/model_package_shader_templates.py:3530-3553
static nerve_hip_status parse_rms_quant_spec_uncached(const char* spec, RmsQuantSpec* out) {
    if (!spec) return fail(NERVE_HIP_INVALID_SPEC, "null specialization");
    static const std::regex re(
        "rms_norm_quantize(?:_batch(\\d+))?_(?:fp8_e4m3(?:_(spow2))?|(int8_pairpacked))_b(\\d+)_h(\\d+)_eps([0-9eE+.-]+)"
        "_offset([0-9eE+.-]+)\\.comp");
    std::cmatch m;
    if (!std::regex_match(spec, m, re))
        return fail(NERVE_HIP_INVALID_SPEC, std::string("not an RMSNorm FP8/INT8 quantizer: ") + spec);
    RmsQuantSpec s;
    uint32_t bt = 0;
    if (m[1].matched) parse_u32(m[1].str(), &bt);
    s.batch_tile = (int)bt;
    s.pow2 = m[2].matched;
    s.int8pp = m[3].matched;
    parse_u32(m[4].str(), &s.block);
    parse_u32(m[5].str(), &s.hidden);
    if (!parse_float(m[6].str(), &s.eps) || !parse_float(m[7].str(), &s.offset))
        return fail(NERVE_HIP_INVALID_SPEC, std::string("bad eps/offset in ") + spec);
    // The pair-packed INT8 output feeds the INT4 linear's 32-column blocks.
    if (s.int8pp && s.block != 32)
        return fail(NERVE_HIP_INVALID_SPEC, std::string("pair-packed INT8 RMSNorm quantizer needs b32: ") + spec);
    // Whole blocks of 32..512 columns (BLOCK_COUNT = HIDDEN / BLOCK_COLUMNS).
    if ((m[1].matched && bt == 0) || s.hidden == 0 || s.hidden % 32 || s.block < 32 || s.block > 512 ||
        (s.block & (s.block - 1)) || s.hidden % s.block)
        return fail(NERVE_HIP_INVALID_SPEC, std::string("invalid RMSNorm FP8 quantizer shape ") + spec);
    *out = s;
    return NERVE_HIP_OK;
}

// nerve/model_package_shader_templates.py:1440-1474 (Q8_0 groups of 32)
static nerve_hip_status parse_quant_i8_spec_uncached(const char* spec, QuantI8Spec* out) {
    if (!spec) return fail(NERVE_HIP_INVALID_SPEC, "null specialization");
    // and silu_multiply_quantize[_batch{T}]_int8_pairpacked_b{B}_h{N}
    // (nerve/model_package_shader_templates.py:3376-3380).
    // and quantize[_batch{T}]_int8_symmetric_b{B}_h{N}, the unpaired form
    // (nerve/model_package_shader_templates.py:1478-1506).
    static const std::regex re(
        "(?:quantize(?:_batch(\\d+))?_int8_symmetric|(silu_multiply)_quantize(?:_batch(\\d+))?_int8)(_pairpacked)?_b(\\d+)"
        "_h(\\d+)\\.comp");
    std::cmatch m;
    if (!std::regex_match(spec, m, re))
        return fail(NERVE_HIP_INVALID_SPEC, std::string("not an INT8 activation quantizer: ") + spec);
    QuantI8Spec s;
    uint32_t bt = 0;
    s.silu = m[2].matched;
    s.paired = m[4].matched;
    if (s.silu && !s.paired) return fail(NERVE_HIP_INVALID_SPEC, std::string("not an INT8 activation quantizer: ") + spec);
    const int bi = s.silu ? 3 : 1;
    if (m[bi].matched) parse_u32(m[bi].str(), &bt);
    s.batch_tile = (int)bt;
    parse_u32(m[5].str(), &s.block);
    parse_u32(m[6].str(), &s.elements);
    if ((m[bi].matched && bt == 0) || s.block != 32 || s.elements == 0 || s.elements % 32)
        return fail(NERVE_HIP_INVALID_SPEC, std::string("invalid INT8 quantizer shape ") + spec);
    *out = s;
    return NERVE_HIP_OK;
}

// Specialization strings are parsed once per thread: a dispatch looks its
// string up here (a hash of ~60 bytes) instead of running the grammar again,
// which costs more host time than a decode-sized kernel takes on the device.
// Only accepted strings are cached, so rejections keep their messages.
template <class S, nerve_hip_status (*Parse)(const char*, S*)>
static nerve_hip_status parse_cached(const char* spec, S* out) {
    if (!spec) return Parse(spec, out);
    thread_local std::unordered_map<std::string, S> cache;
    std::string key(spec);
    auto it = cache.find(key);
    if (it != cache.end()) {
        *out = it->second;
        return NERVE_HIP_OK;
    }
    nerve_hip_status st = Parse(spec, out);
    if (st == NERVE_HIP_OK) {
        if (cache.size() >= 4096) cache.clear();
        cache.emplace(std::move(key), *out);
    }
    return st;
}

nerve_hip_status parse_moe_spec(const char* spec, MoeSpec* out) {
    return parse_cached<MoeSpec, parse_moe_spec_uncached>(spec, out);
}
nerve_hip_status parse_topk_spec(const char* spec, TopkSpec* out) {
    return parse_cached<TopkSpec, parse_topk_spec_uncached>(spec, out);
}
nerve_hip_status parse_int4_spec(const char* spec, Int4Spec* out) {
    return parse_cached<Int4Spec, parse_int4_spec_uncached>(spec, out);
}
nerve_hip_status parse_fp8_head_spec(const char* spec, Fp8HeadSpec* out) {
    return parse_cached<Fp8HeadSpec, parse_fp8_head_spec_uncached>(spec, out);
}
nerve_hip_status parse_quant_spec(const char* spec, QuantSpec* out) {
    return parse_cached<QuantSpec, parse_quant_spec_uncached>(spec, out);
}
nerve_hip_status parse_quant_i8_spec(const char* spec, QuantI8Spec* out) {
    return parse_cached<QuantI8Spec, parse_quant_i8_spec_uncached>(spec, out);
}
nerve_hip_status parse_rms_quant_spec(const char* spec, RmsQuantSpec* out) {
    return parse_cached<RmsQuantSpec, parse_rms_quant_spec_uncached>(spec, out);
}

}  // namespace nh

extern "C" {

int nerve_hip_abi_version(void) { return NERVE_HIP_ABI_VERSION; }

const char* nerve_hip_last_error(void) { return g_last_error.c_str(); }

nerve_hip_status nerve_hip_open(int device_ordinal, nerve_hip_ctx** out) {
    if (!out) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "null output pointer");
    *out = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count == 0) return nh::fail(NERVE_HIP_DEVICE_ERROR, "no HIP device available");
    if (device_ordinal < 0 || device_ordinal >= count) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "device ordinal out of range");
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device_ordinal);
    if (e != hipSuccess) return nh::fail(NERVE_HIP_DEVICE_ERROR, std::string("hipGetDeviceProperties: ") + hipGetErrorString(e));
    if (std::string(prop.gcnArchName).rfind("gfx950", 0) != 0)
        return nh::fail(NERVE_HIP_UNSUPPORTED, std::string("libnerve_hip is built for gfx950, device is ") + prop.gcnArchName);
    // The no-allocation entry point's scratch: this device's copy of the
    // array, resolved with the device current (once per context).
    e = hipSetDevice(device_ordinal);
    if (e != hipSuccess) return nh::fail(NERVE_HIP_DEVICE_ERROR, std::string("hipSetDevice: ") + hipGetErrorString(e));
    void* scratch_ptr = nullptr;
    e = hipGetSymbolAddress(&scratch_ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !scratch_ptr)
        return nh::fail(NERVE_HIP_DEVICE_ERROR, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    // Arrival counters of launches whose last block finishes the work; zeroed
    // once here, each launch leaves its counter at zero.
    uint32_t* sync_words = nullptr;
    e = hipMalloc(&sync_words, 256);
    if (e != hipSuccess) return nh::fail(NERVE_HIP_OUT_OF_MEMORY, std::string("hipMalloc: ") + hipGetErrorString(e));
    e = hipMemset(sync_words, 0, 256);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        (void)hipFree(sync_words);
        return nh::fail(NERVE_HIP_DEVICE_ERROR, std::string("hipMemset: ") + hipGetErrorString(e));
    }
    nerve_hip_ctx* ctx = new nerve_hip_ctx();
    ctx->device = device_ordinal;
    ctx->sync_words = sync_words;
    ctx->cu_count = prop.multiProcessorCount;
    ctx->workspace = nullptr;
    ctx->workspace_bytes = 0;
    ctx->static_scratch = scratch_ptr;
    *out = ctx;
    return NERVE_HIP_OK;
}

nerve_hip_status nerve_hip_check_specialization(const char* spec) {
    if (!spec) return nh::fail(NERVE_HIP_INVALID_SPEC, "null specialization");
    std::string s(spec);
    if (s.rfind("independent_sparse_moe_", 0) == 0) {
        nh::MoeSpec m;
        return nh::parse_moe_spec(spec, &m);
    }
    if (s.rfind("sparse_moe_", 0) == 0) {
        nh::MoeSpec m;
        nerve_hip_status st = nh::parse_moe_spec(spec, &m);
        if (st) return st;
        if (m.family != 1) return nh::fail(NERVE_HIP_INVALID_SPEC, std::string("not an INT4 sparse expert kernel: ") + spec);
        if ((m.gate_up ? m.hidden : m.inter) % 32)
            return nh::fail(NERVE_HIP_UNSUPPORTED, "INT4 sparse experts need an input width that is a multiple of 32");
        return NERVE_HIP_OK;
    }
    if (s.rfind("moe_topk", 0) == 0 || s.rfind("moe_router", 0) == 0) {
        nh::TopkSpec t;
        return nh::parse_topk_spec(spec, &t);
    }
    if (s.rfind("tied_output_projection", 0) == 0) {
        nh::Fp8HeadSpec f;
        return nh::parse_fp8_head_spec(spec, &f);
    }
    if (s.rfind("rms_norm_quantize", 0) == 0) {
        nh::RmsQuantSpec r;
        return nh::parse_rms_quant_spec(spec, &r);
    }
    if ((s.rfind("quantize", 0) == 0 && s.find("_int8_symmetric_") != std::string::npos) ||
        s.rfind("silu_multiply_quantize", 0) == 0) {
        nh::QuantI8Spec q;
        return nh::parse_quant_i8_spec(spec, &q);
    }
    if (s.rfind("quantize", 0) == 0) {
        nh::QuantSpec q;
        return nh::parse_quant_spec(spec, &q);
    }
    if (s.rfind("linear", 0) == 0) {
        nh::Int4Spec i;
        nerve_hip_status st = nh::parse_int4_spec(spec, &i);
        if (st) return st;
        if (i.input != 0) return NERVE_HIP_OK;   // INT8-prequant inputs: any group of 32k columns, N even
        if (i.layout == 1 && i.group % 128)
            return nh::fail(NERVE_HIP_UNSUPPORTED, "CT INT4 kernel needs group % 128 == 0");
        if (i.layout == 0 && i.out % 16) return nh::fail(NERVE_HIP_UNSUPPORTED, "GPTQ INT4 kernel needs N % 16 == 0");
        if (i.layout == 1 && i.out % 16) return nh::fail(NERVE_HIP_UNSUPPORTED, "CT INT4 kernel needs N % 16 == 0");
        return NERVE_HIP_OK;
    }
    return nh::fail(NERVE_HIP_INVALID_SPEC, std::string("no kernel family matches ") + spec);
}

void nerve_hip_close(nerve_hip_ctx* ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    (void)hipDeviceSynchronize();
    if (ctx->workspace) (void)hipFree(ctx->workspace);
    if (ctx->sync_words) (void)hipFree(ctx->sync_words);
    delete ctx;
}

}  // extern "C"
