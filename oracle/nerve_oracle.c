/*
 * nerve_oracle.c -- CPU restatement of NERVE's quantized-matmul hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load this library, and only as the checker
 * (or as the timed CPU baseline).  The product path (nerve_amd/, libnerve_hip)
 * never links or calls it.
 *
 * Every function restates the arithmetic of one reference shader step by
 * step: the same rounding points (bf16 RNE, e4m3 RNE), the same scale rules and
 * the same accumulation structure (per-lane strided fma chains followed by a
 * subgroup tree reduction, emulated here with a 64-lane subgroup).  Paths are
 * relative to the reference repository root.
 *
 * Shape extension: the reference compiler rejects hidden/intermediate sizes
 * that are not multiples of 128 (nerve/model_package_shader_templates.py:
 * 4805-4807).  This restatement accepts multiples of 32 with "zero-padded tail
 * block" semantics: the last 128-column activation block is only as wide as
 * the data, and its amax is taken over the real columns.  This equals running
 * the reference on K padded with zero activations and zero weights.
 *
 * Pinning status of each function is recorded in oracle/README.md.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define SUBGROUP 64

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------ */
/* Scalar numerics                                                      */
/* ------------------------------------------------------------------ */

/* bf16 RNE: independent_sparse_moe_gate_up_batch1_mxfp4.comp.template:92-96 */
uint16_t o_f32_to_bf16(float v) {
    uint32_t b = f2u(v);
    uint32_t lsb = (b >> 16) & 1u;
    return (uint16_t)((b + 0x7fffu + lsb) >> 16);
}

/* ...gate_up_batch1_mxfp4.comp.template:90 */
float o_bf16_to_f32(uint16_t v) { return u2f(((uint32_t)v) << 16); }

static inline float round_bf16(float v) { return o_bf16_to_f32(o_f32_to_bf16(v)); }

/* e4m3 (OCP "fn") decode; nerve/quantized_transforms.py:113-125.  0x7f/0xff
 * are NaN in e4m3fn; the Python decoder treats them as 480 but no path on
 * this hot path produces them. */
float o_e4m3_to_f32(uint8_t b) {
    int s = b >> 7, e = (b >> 3) & 15, m = b & 7;
    float v = e ? ldexpf((float)(8 + m), e - 10) : ldexpf((float)m, -9);
    if (e == 15 && m == 7) v = NAN;
    return s ? -v : v;
}

/* f32 -> e4m3 with round-to-nearest-even and saturation at +-448.  This is
 * the GLSL `fe4m3vec4(x)` conversion used by every activation quantizer
 * (…gate_up_batch1_mxfp4.comp.template:380, tied_output_projection_fp8_e4m3.
 * comp.template:103).  The quantizers never feed it |x| > 448 (the scale is
 * chosen so that |x/s| <= 448), so the saturation rule is only reached by the
 * weight producer (nerve/model_package_tensors.py:1044-1075), whose subnormal
 * quirk is restated separately in nerve_amd/workloads.py (f32_to_e4m3fn_producer). */
uint8_t o_f32_to_e4m3(float x) {
    uint32_t b = f2u(x);
    uint8_t sign = (uint8_t)((b >> 24) & 0x80u);
    uint32_t a = b & 0x7fffffffu;
    if (a > 0x7f800000u) return sign | 0x7f;          /* NaN */
    if (a < 0x3c800000u) {                             /* |x| < 2^-6: subnormal grid 2^-9 */
        float y = u2f(a) * 512.0f;                     /* exact */
        int m = (int)nearbyintf(y);                    /* RNE (default rounding mode) */
        return sign | (uint8_t)m;                      /* m == 8 encodes 2^-6 exactly */
    }
    uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);      /* RNE to 3 mantissa bits */
    int e4 = (int)(r >> 23) - 120;
    uint32_t m = (r >> 20) & 7u;
    if (e4 > 15 || (e4 == 15 && m == 7)) return sign | 0x7e;   /* saturate to 448 */
    return sign | (uint8_t)((e4 << 3) | m);
}

/* E2M1 -> E4M3 bits: nerve/quantized_transforms.py:34-51;
 * GLSL mxfp4_e4m3_bits …gate_up_batch1_mxfp4.comp.template:246-248. */
static const uint8_t E2M1_E4M3[8] = {0x00, 0x30, 0x38, 0x3c, 0x40, 0x44, 0x48, 0x4c};
uint8_t o_e2m1_to_e4m3_bits(uint8_t nibble) {
    return (uint8_t)(E2M1_E4M3[nibble & 7] | ((nibble & 8) << 4));
}

/* E2M1 -> SINT8 (value * 2): nerve/quantized_transforms.py:12-29 */
static const int8_t E2M1_SINT8[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};
int8_t o_e2m1_to_sint8(uint8_t nibble) { return E2M1_SINT8[nibble & 15]; }

/* E8M0 scale: byte 0 -> 2^-127 (0x00400000), else bits(byte << 23).
 * …gate_up_batch1_mxfp4.comp.template:293-297; nerve/quantized_transforms.py:86-91 */
float o_e8m0_scale(uint8_t byte) {
    if (byte == 0) return u2f(0x00400000u);
    return u2f(((uint32_t)byte) << 23);
}

/* Dequantized MXFP4 value through the resident e4m3 form (a1).
 * nerve/quantized_transforms.py:128-130 */
float o_mxfp4_value(uint8_t nibble, uint8_t scale_byte) {
    return o_e4m3_to_f32(o_e2m1_to_e4m3_bits(nibble)) * o_e8m0_scale(scale_byte);
}

/* Power-of-two activation scale: rounded_fp8_scale,
 * …gate_up_batch1_mxfp4.comp.template:357-363 */
float o_pow2_fp8_scale(float block_max) {
    float ratio = fmaxf(block_max, 1e-4f) / 448.0f;
    uint32_t bits = f2u(ratio);
    int exponent = (int)((bits >> 23) & 0xffu) - 127;
    if ((bits & 0x7fffffu) != 0u) exponent++;
    return u2f((uint32_t)(exponent + 127) << 23);
}

/* amax/448 activation scale: tied_output_projection_fp8_e4m3.comp.template:99 */
float o_amax_fp8_scale(float block_max) {
    return block_max > 0.0f ? block_max / 448.0f : 1.0f;
}

/* ------------------------------------------------------------------ */
/* a2: blockwise activation quantization                                */
/* ------------------------------------------------------------------ */

/* x: bf16 [rows, cols] (row stride x_stride elements).  q: e4m3 [rows, cols]
 * (row stride cols), s: f32 [rows, ceil(cols/128)].  pow2 != 0 selects
 * rounded_fp8_scale (quantize_hidden …gate_up_batch1_mxfp4.comp.template:
 * 366-382; quantize_intermediate …down_batch1_mxfp4.comp.template:332-353),
 * pow2 == 0 selects amax/448 (tied_output_projection_fp8_e4m3.comp.template:
 * 91-104; quantize_fp8_e4m3.comp.template:41-59). */
void o_quantize_blocks(const uint16_t* x, long x_stride, int rows, int cols,
                       int pow2, uint8_t* q, float* s) {
    int nblk = (cols + 127) / 128;
    for (int r = 0; r < rows; r++) {
        const uint16_t* xr = x + (long)r * x_stride;
        for (int b = 0; b < nblk; b++) {
            int c0 = b * 128, c1 = c0 + 128 < cols ? c0 + 128 : cols;
            float amax = 0.0f;
            for (int c = c0; c < c1; c++) amax = fmaxf(amax, fabsf(o_bf16_to_f32(xr[c])));
            float sc = pow2 ? o_pow2_fp8_scale(amax) : o_amax_fp8_scale(amax);
            s[(long)r * nblk + b] = sc;
            for (int c = c0; c < c1; c++)
                q[(long)r * cols + c] = o_f32_to_e4m3(o_bf16_to_f32(xr[c]) / sc);
        }
    }
}

/* RMSNorm + blockwise e4m3 quantization of bf16 rows
 * (rms_norm_quantize_fp8_e4m3.comp.template:70-129): sum of squares by
 * fma, inv_rms = 1 / sqrt(sum / H + eps) (the shader's inversesqrt, taken
 * as the correctly rounded form), y = bf16(x * inv_rms * (w + offset)),
 * then per `block` columns s = pow2 / amax/448 scale of max |y| and
 * q = e4m3(y / s).  The sum is taken in index order here; the shader's
 * order is its subgroup layout's, so y may differ in the last bf16 place. */
void o_rms_norm_quantize(const uint16_t* x, const uint16_t* w, int rows, int H, int block, int pow2, float eps,
                         float offset, uint16_t* y, uint8_t* q, float* s) {
    int nblk = H / block;
    for (int r = 0; r < rows; r++) {
        const uint16_t* xr = x + (long)r * H;
        float ss = 0.0f;
        for (int c = 0; c < H; c++) {
            float v = o_bf16_to_f32(xr[c]);
            ss = fmaf(v, v, ss);
        }
        float inv = 1.0f / sqrtf(ss / (float)H + eps);
        for (int b = 0; b < nblk; b++) {
            float amax = 0.0f;
            for (int c = b * block; c < (b + 1) * block; c++) {
                float v = o_bf16_to_f32(xr[c]) * inv * (o_bf16_to_f32(w[c]) + offset);
                uint16_t yb = o_f32_to_bf16(v);
                y[(long)r * H + c] = yb;
                amax = fmaxf(amax, fabsf(o_bf16_to_f32(yb)));
            }
            float sc = pow2 ? o_pow2_fp8_scale(amax) : o_amax_fp8_scale(amax);
            s[(long)r * nblk + b] = sc;
            for (int c = b * block; c < (b + 1) * block; c++)
                q[(long)r * H + c] = o_f32_to_e4m3(o_bf16_to_f32(y[(long)r * H + c]) / sc);
        }
    }
}

/* ------------------------------------------------------------------ */
/* Shared MXFP4 dot: one output row, emulating the shader's lane loop.  */
/* ------------------------------------------------------------------ */

/* fp8_dot4_acc32(a, b, 0.0): four exact e4m3 x e4m3 products summed in f32. */
static inline float dot4(const float* a, const float* b) {
    return ((a[0] * b[0] + a[1] * b[1]) + a[2] * b[2]) + a[3] * b[3];
}

/* Subgroup tree reduction (subgroupAdd) over SUBGROUP partials. */
static float subgroup_add(float* v, int n) {
    for (int step = n / 2; step > 0; step /= 2)
        for (int i = 0; i < step; i++) v[i] = v[i] + v[i + step];
    return v[0];
}

/* y = sum_w fma(dot4(q[w], W[row, w]), sx[blk(w)] * se8m0[row, w/8], acc)
 * in lane-strided order (…gate_up_batch1_mxfp4.comp.template:759-787,
 * …down_batch1_mxfp4.comp.template:560-585).  qf: activation values decoded
 * to f32 (length K), sx: per-128 scales.  wrow: packed MXFP4 row (K/2 bytes),
 * srow: e8m0 bytes (K/32). */
static float mxfp4_row_dot(const float* qf, const float* sx, int K,
                           const uint8_t* wrow, const uint8_t* srow) {
    float lanes[SUBGROUP];
    int words = K / 4;
    for (int lane = 0; lane < SUBGROUP; lane++) {
        float acc = 0.0f;
        for (int w = lane; w < words; w += SUBGROUP) {
            int col = w * 4;
            float wv[4];
            uint8_t lo = wrow[col / 2], hi = wrow[col / 2 + 1];
            wv[0] = o_e4m3_to_f32(o_e2m1_to_e4m3_bits(lo & 15));
            wv[1] = o_e4m3_to_f32(o_e2m1_to_e4m3_bits(lo >> 4));
            wv[2] = o_e4m3_to_f32(o_e2m1_to_e4m3_bits(hi & 15));
            wv[3] = o_e4m3_to_f32(o_e2m1_to_e4m3_bits(hi >> 4));
            acc = fmaf(dot4(qf + col, wv), sx[col / 128] * o_e8m0_scale(srow[col / 32]), acc);
        }
        lanes[lane] = acc;
    }
    return subgroup_add(lanes, SUBGROUP);
}

static void decode_q(const uint8_t* q, int K, float* out) {
    for (int k = 0; k < K; k++) out[k] = o_e4m3_to_f32(q[k]);
}

/* Raw MXFP4 GEMV (config 0 entry): y[m, n] for pre-quantized activations.
 * q: e4m3 [M, K], s: f32 [M, ceil(K/128)], W: [N, K/2], S: [N, K/32]. */
void o_mxfp4_gemv(const uint8_t* q, const float* s, int M, int K,
                  const uint8_t* W, const uint8_t* S, int N, float* y) {
    int nblk = (K + 127) / 128;
    float* qf = (float*)malloc(sizeof(float) * (size_t)K * M);
    for (int m = 0; m < M; m++) decode_q(q + (long)m * K, K, qf + (long)m * K);
    #pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++)
        for (int m = 0; m < M; m++)
            y[(long)m * N + n] = mxfp4_row_dot(qf + (long)m * K, s + (long)m * nblk, K,
                                               W + (long)n * (K / 2), S + (long)n * (K / 32));
    free(qf);
}

/* float64 "ideal" of the same contraction (no intermediate rounding) for
 * pinning the order-dependent f32 result. */
void o_mxfp4_gemv_f64(const uint8_t* q, const float* s, int M, int K,
                      const uint8_t* W, const uint8_t* S, int N, double* y) {
    int nblk = (K + 127) / 128;
    #pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++)
        for (int m = 0; m < M; m++) {
            double acc = 0.0;
            for (int k = 0; k < K; k++) {
                uint8_t byte = W[(long)n * (K / 2) + k / 2];
                uint8_t nib = (k & 1) ? byte >> 4 : byte & 15;
                acc += (double)o_e4m3_to_f32(q[(long)m * K + k]) * (double)s[(long)m * nblk + k / 128]
                     * (double)o_mxfp4_value(nib, S[(long)n * (K / 32) + k / 32]);
            }
            y[(long)m * N + n] = acc;
        }
}

/* ------------------------------------------------------------------ */
/* a5: router projection, linear_bf16.comp.template:40-98                */
/* ------------------------------------------------------------------ */

/* logits[b, e] = bf16(sum_k x[b,k] * W[e,k]); lanes take word pairs with
 * fma(lo), fma(hi) (linear_bf16.comp.template:52-61), then a 64-lane add. */
void o_router_linear(const uint16_t* x, const uint16_t* W, int B, int H, int E, uint16_t* logits) {
    int words = (H + 1) / 2;
    #pragma omp parallel for schedule(static)
    for (int be = 0; be < B * E; be++) {
        int b = be / E, e = be % E;
        float lanes[64];
        for (int lane = 0; lane < 64; lane++) {
            float acc = 0.0f;
            for (int w = lane; w < words; w += 64) {
                float xl = o_bf16_to_f32(x[(long)b * H + 2 * w]);
                float xh = 2 * w + 1 < H ? o_bf16_to_f32(x[(long)b * H + 2 * w + 1]) : 0.0f;
                float wl = o_bf16_to_f32(W[(long)e * H + 2 * w]);
                float wh = 2 * w + 1 < H ? o_bf16_to_f32(W[(long)e * H + 2 * w + 1]) : 0.0f;
                acc = fmaf(xl, wl, acc);
                acc = fmaf(xh, wh, acc);
            }
            lanes[lane] = acc;
        }
        logits[(long)b * E + e] = o_f32_to_bf16(subgroup_add(lanes, 64));
    }
}

/* ------------------------------------------------------------------ */
/* a6: top-k routing                                                     */
/* ------------------------------------------------------------------ */

/* moe_topk_routed_batch1_bf16.comp.template:71-182.
 * mode: 0 = moe_topk (sigmoid flag, normalize flag, softcap, bias)
 *       1 = moe_router_score_topk (activation 0 sigmoid /1 softmax /2 sqrtsoftplus;
 *           moe_router_score_topk_batch1_bf16.comp.template:57-219)
 * bias: NULL or f32[E].  routes: u32 [B, k_total]; telemetry: u32
 * [T + T(T-1)/2] (T = total resource count) or NULL. */
void o_topk(const uint16_t* logits, int B, int E, int k, int mode,
            int activation, int normalize, float softcap, float routed_scale,
            int always_count, float always_weight, const float* bias,
            uint32_t* routes, uint32_t* telemetry) {
    int total_sel = k + (mode == 1 ? always_count : 0);
    int total_res = E + (mode == 1 ? always_count : 0);
    float* raw = (float*)malloc(sizeof(float) * E);
    float* val = (float*)malloc(sizeof(float) * E);
    uint8_t* sel = (uint8_t*)malloc(E);
    uint32_t idx[4096 + 64];
    float wts[4096 + 64];
    for (int b = 0; b < B; b++) {
        for (int e = 0; e < E; e++) {
            float v = o_bf16_to_f32(logits[(long)b * E + e]);
            if (mode == 0 && softcap > 0.0f) v = tanhf(v / softcap) * softcap;
            raw[e] = v;
            sel[e] = 0;
        }
        float smax = -INFINITY, sden = 0.0f;
        if (mode == 1 && activation == 1) {
            for (int e = 0; e < E; e++) smax = fmaxf(smax, raw[e]);
            for (int e = 0; e < E; e++) sden += expf(raw[e] - smax);
        }
        for (int e = 0; e < E; e++) {
            float v = raw[e];
            if (mode == 0) {
                val[e] = v;
            } else if (activation == 0) {
                val[e] = 1.0f / (1.0f + expf(-v));
            } else if (activation == 1) {
                val[e] = expf(v - smax) / sden;
            } else {
                float sp = fmaxf(v, 0.0f) + logf(1.0f + expf(-fabsf(v)));
                val[e] = sqrtf(sp);
            }
        }
        for (int r = 0; r < k; r++) {
            float best = -INFINITY;
            uint32_t bi = 0xffffffffu;
            for (int e = 0; e < E; e++) {
                float score;
                if (mode == 0 && activation) score = 1.0f / (1.0f + expf(-val[e]));
                else score = val[e];
                if (bias) score = score + bias[e];
                if (!sel[e] && (score > best || (score == best && (uint32_t)e < bi))) {
                    best = score;
                    bi = (uint32_t)e;
                }
            }
            idx[r] = bi;
            if (bi < (uint32_t)E) sel[bi] = 1;
        }
        if (mode == 0) {
            /* …topk_routed_batch1_bf16.comp.template:133-167 */
            int sig = activation;
            float maximum = val[idx[0]];
            float den = 0.0f;
            if (normalize) {
                for (int r = 0; r < k; r++) {
                    float l = val[idx[r]];
                    den += sig ? 1.0f / (1.0f + expf(-l)) : expf(l - maximum);
                }
            } else if (!sig) {
                maximum = -INFINITY;
                for (int e = 0; e < E; e++) maximum = fmaxf(maximum, val[e]);
                for (int e = 0; e < E; e++) den += expf(val[e] - maximum);
            }
            for (int r = 1; r < k; r++) {
                uint32_t ex = idx[r];
                int ins = r;
                while (ins > 0 && idx[ins - 1] > ex) { idx[ins] = idx[ins - 1]; ins--; }
                idx[ins] = ex;
            }
            for (int r = 0; r < k; r++) {
                float l = val[idx[r]];
                float w = sig ? 1.0f / (1.0f + expf(-l)) : expf(l - maximum);
                if (normalize || !sig) w /= den;
                wts[r] = w;
            }
        } else {
            /* …router_score_topk_batch1_bf16.comp.template:169-205 */
            float den = 0.0f;
            if (normalize) for (int r = 0; r < k; r++) den += val[idx[r]];
            for (int r = 0; r < k; r++) {
                float w = val[idx[r]];
                wts[r] = normalize ? w / den * routed_scale : w * routed_scale;
            }
            for (int a = 0; a < always_count; a++) {
                idx[k + a] = (uint32_t)(E + a);
                wts[k + a] = always_weight;
            }
            for (int r = 1; r < total_sel; r++) {
                uint32_t ex = idx[r];
                float w = wts[r];
                int ins = r;
                while (ins > 0 && idx[ins - 1] > ex) {
                    idx[ins] = idx[ins - 1];
                    wts[ins] = wts[ins - 1];
                    ins--;
                }
                idx[ins] = ex;
                wts[ins] = w;
            }
        }
        for (int r = 0; r < total_sel; r++) {
            routes[(long)b * total_sel + r] = ((uint32_t)o_f32_to_bf16(wts[r]) << 16) | idx[r];
            if (telemetry) telemetry[idx[r]]++;
        }
        if (telemetry)
            for (int l = 0; l < total_sel; l++)
                for (int r = l + 1; r < total_sel; r++) {
                    uint32_t left = idx[l], right = idx[r];
                    if (left < right) {
                        uint32_t preceding = left * (2u * (uint32_t)total_res - left - 1u) / 2u;
                        telemetry[total_res + preceding + right - left - 1u]++;
                    }
                }
    }
    free(raw); free(val); free(sel);
}

/* ------------------------------------------------------------------ */
/* a7: route compaction                                                  */
/* ------------------------------------------------------------------ */

/* moe_route_compact_batch1.comp.template:26-106.  map: u32 [B*k] indexed by
 * compact position (the frame-tail words, flattened).  control: u32[7]
 * BatchControl {batch_width, expert_start, expert_count, owned_route_count,
 * dispatch_x, dispatch_y, dispatch_z}; fields 0..2 are inputs. */
void o_route_compact(const uint32_t* routes, int k, uint32_t tiles_per_route,
                     uint32_t* map, uint32_t* control) {
    uint32_t B = control[0], start = control[1], count = control[2];
    uint32_t n = B * (uint32_t)k;
    if (count != 0) {
        uint32_t owned = 0, end = start + count;
        for (uint32_t i = 0; i < n; i++) {
            uint32_t e = routes[i] & 0xffffu;
            if (e < start || e >= end) continue;
            map[owned++] = i;
        }
        control[3] = owned;
        control[4] = owned * tiles_per_route;
        control[5] = 1;
        control[6] = 1;
        return;
    }
    control[3] = n;
    control[4] = (uint32_t)k * tiles_per_route;
    control[5] = B;
    control[6] = 1;
    for (uint32_t i = 0; i < n; i++) {
        uint32_t e = routes[i] & 0xffffu, rank = 0;
        for (uint32_t c = 0; c < n; c++) {
            uint32_t ce = routes[c] & 0xffffu;
            if (ce < e || (ce == e && c < i)) rank++;
        }
        map[rank] = i;
    }
}

/* ------------------------------------------------------------------ */
/* a3 / a4: MoE expert projections                                       */
/* ------------------------------------------------------------------ */

/* Expert weights are passed as contiguous banks: gate/up/down W [E, rows, K/2]
 * and S [E, rows, K/32].  The address-table indirection and its fail-closed
 * validation are host-side concerns tested against the HIP library only.
 *
 * Gate/up (…gate_up_batch1_mxfp4.comp.template:643-802): for compact
 * position c < n_routes: r = map[c]; token b = r / k, expert = routes[r] &
 * 0xffff; h[b, r%k, i] = bf16(silu(g) * u) with g, u rounded to bf16 and
 * clamped when limit > 0.  inter: bf16 [B, k, I].  Routes whose expert is out
 * of range are skipped (their output is left untouched). */
void o_moe_gate_up(const uint16_t* hidden, const uint32_t* routes, const uint32_t* map,
                   int n_routes, int B, int k, int E, int H, int I, float limit,
                   const uint8_t* gw, const uint8_t* gs, const uint8_t* uw, const uint8_t* us,
                   uint16_t* inter) {
    int nblk = (H + 127) / 128;
    uint8_t* q = (uint8_t*)malloc((size_t)B * H);
    float* s = (float*)malloc(sizeof(float) * (size_t)B * nblk);
    float* qf = (float*)malloc(sizeof(float) * (size_t)B * H);
    o_quantize_blocks(hidden, H, B, H, 1, q, s);
    for (int b = 0; b < B; b++) decode_q(q + (long)b * H, H, qf + (long)b * H);
    for (int c = 0; c < n_routes; c++) {
        uint32_t r = map[c];
        if (r >= (uint32_t)(B * k)) continue;
        int b = (int)(r / (uint32_t)k), route = (int)(r % (uint32_t)k);
        uint32_t e = routes[r] & 0xffffu;
        if (e >= (uint32_t)E) continue;
        const uint8_t* gwe = gw + (size_t)e * I * (H / 2);
        const uint8_t* gse = gs + (size_t)e * I * (H / 32);
        const uint8_t* uwe = uw + (size_t)e * I * (H / 2);
        const uint8_t* use = us + (size_t)e * I * (H / 32);
        #pragma omp parallel for schedule(static)
        for (int i = 0; i < I; i++) {
            float g = mxfp4_row_dot(qf + (long)b * H, s + (long)b * nblk, H,
                                    gwe + (size_t)i * (H / 2), gse + (size_t)i * (H / 32));
            float u = mxfp4_row_dot(qf + (long)b * H, s + (long)b * nblk, H,
                                    uwe + (size_t)i * (H / 2), use + (size_t)i * (H / 32));
            float gv = round_bf16(g), uv = round_bf16(u);
            if (limit > 0.0f) {
                gv = fminf(gv, limit);
                uv = fminf(fmaxf(uv, -limit), limit);
            }
            inter[((size_t)b * k + route) * I + i] = o_f32_to_bf16((gv / (1.0f + expf(-gv))) * uv);
        }
    }
    free(q); free(s); free(qf);
}

/* Down (…down_batch1_mxfp4.comp.template:507-610): quantize h per (token,
 * route) with pow2 scales, y = dot, out[b, route, j] = bf16(y * w_route). */
void o_moe_down(const uint16_t* inter, const uint32_t* routes, const uint32_t* map,
                int n_routes, int B, int k, int E, int H, int I,
                const uint8_t* dw, const uint8_t* ds, uint16_t* out) {
    int nblk = (I + 127) / 128;
    uint8_t* q = (uint8_t*)malloc((size_t)I);
    float* s = (float*)malloc(sizeof(float) * (size_t)nblk);
    float* qf = (float*)malloc(sizeof(float) * (size_t)I);
    for (int c = 0; c < n_routes; c++) {
        uint32_t r = map[c];
        if (r >= (uint32_t)(B * k)) continue;
        int b = (int)(r / (uint32_t)k), route = (int)(r % (uint32_t)k);
        uint32_t packed = routes[r];
        uint32_t e = packed & 0xffffu;
        if (e >= (uint32_t)E) continue;
        float wr = o_bf16_to_f32((uint16_t)(packed >> 16));
        o_quantize_blocks(inter + ((size_t)b * k + route) * I, I, 1, I, 1, q, s);
        decode_q(q, I, qf);
        const uint8_t* dwe = dw + (size_t)e * H * (I / 2);
        const uint8_t* dse = ds + (size_t)e * H * (I / 32);
        #pragma omp parallel for schedule(static)
        for (int j = 0; j < H; j++) {
            float y = mxfp4_row_dot(qf, s, I, dwe + (size_t)j * (I / 2), dse + (size_t)j * (I / 32));
            out[((size_t)b * k + route) * H + j] = o_f32_to_bf16(y * wr);
        }
    }
    free(q); free(s); free(qf);
}

/* Tensor-parallel down slice (…down_batch1_mxfp4.comp.template:421-505,
 * with INPUT_BLOCK_MAJOR addressing :229-233, :260-263): the local slice
 * h [B, k, count] holds intermediate columns [start, start + count); each
 * route's slice is quantized per 128-column block (pow2 scales) and
 * contracted against the same columns of the down weights; out f32
 * [B, k, H] = y, not scaled by the route weight.  A token's routes run in
 * order and the first one with an out-of-range expert ends the token (the
 * shader's `return`; later outputs untouched).  dw / ds are given in the
 * package row layout [E, H, I/2], [E, H, I/32]; block-major storage only
 * changes where a byte lives. */
void o_moe_down_tp(const uint16_t* inter, const uint32_t* routes, int B, int k, int E, int H, int I,
                   int start, int count, const uint8_t* dw, const uint8_t* ds, float* out) {
    int nblk = (count + 127) / 128;
    uint8_t* q = (uint8_t*)malloc((size_t)(count > 0 ? count : 1));
    float* s = (float*)malloc(sizeof(float) * (size_t)(nblk > 0 ? nblk : 1));
    float* qf = (float*)malloc(sizeof(float) * (size_t)(count > 0 ? count : 1));
    for (int b = 0; b < B; b++) {
        for (int route = 0; route < k; route++) {
            uint32_t e = routes[(size_t)b * k + route] & 0xffffu;
            if (e >= (uint32_t)E) break;
            o_quantize_blocks(inter + ((size_t)b * k + route) * count, count, 1, count, 1, q, s);
            decode_q(q, count, qf);
            const uint8_t* dwe = dw + (size_t)e * H * (I / 2);
            const uint8_t* dse = ds + (size_t)e * H * (I / 32);
            #pragma omp parallel for schedule(static)
            for (int j = 0; j < H; j++)
                out[((size_t)b * k + route) * H + j] =
                    mxfp4_row_dot(qf, s, count, dwe + (size_t)j * (I / 2) + start / 2, dse + (size_t)j * (I / 32) + start / 32);
        }
    }
    free(q); free(s); free(qf);
}

/* a8: moe_reduce_batch1_bf16.comp.template:29-54 */
void o_moe_reduce(const uint16_t* expert_out, int B, int k, int H, float routed_scale, uint16_t* out) {
    for (int b = 0; b < B; b++)
        for (int j = 0; j < H; j++) {
            float acc = 0.0f;
            for (int r = 0; r < k; r++)
                acc = round_bf16(acc + o_bf16_to_f32(expert_out[((size_t)b * k + r) * H + j]));
            out[(size_t)b * H + j] = o_f32_to_bf16(acc * routed_scale);
        }
}

/* ------------------------------------------------------------------ */
/* a9: group-scaled INT4                                                 */
/* ------------------------------------------------------------------ */

static float f16_to_f32(uint16_t h) {
    int s = h >> 15, e = (h >> 10) & 31, m = h & 1023;
    float v;
    if (e == 0) v = ldexpf((float)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexpf((float)(m + 1024), e - 25);
    return s ? -v : v;
}

/* linear_int4_gptq.comp.template:95-119 (layout 0: qweight [K/8, N], scales
 * [K/g, N]) and linear_int4_ct.comp.template:95-124 (layout 1: qweight
 * [N, K/8], scales [N, K/g]).  Per packed word: sum = fma(dot(x_lo, w_lo) +
 * dot(x_hi, w_hi), scale, sum).  The GPTQ form is a sequential loop over
 * groups (one lane per row); the CT form is 64 lane-strided chains plus a
 * subgroup add.  zeros: NULL (symmetric, code - 8) or the build's asymmetric
 * extension, AutoGPTQ qzeros [K/g, N/8] (8 zero codes per word along N).
 * finalize: 0 plain, 1 bias (bf16 [N], added to the f32 sum), 2 residual
 * (bf16 [B, N]: residual + bf16(sum)); nerve/model_package_shader_selection.py:
 * 2504-2533.  scale_bf16 selects bf16 scales instead of f16. */
void o_int4_linear(int layout, const uint16_t* x, const uint32_t* qw, const uint16_t* scales,
                   int scale_bf16, const uint32_t* zeros, int group, int K, int N, int B,
                   int finalize, const uint16_t* aux, uint16_t* y) {
    int G = K / group;
    #pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++) {
        for (int b = 0; b < B; b++) {
            const uint16_t* xb = x + (size_t)b * K;
            float lanes[64];
            int nl = layout == 0 ? 1 : 64;
            for (int lane = 0; lane < nl; lane++) {
                float sum = 0.0f;
                for (int p = lane; p < K / 8; p += nl) {
                    int g = (p * 8) / group;
                    uint16_t sr = layout == 0 ? scales[(size_t)g * N + n] : scales[(size_t)n * G + g];
                    float sc = scale_bf16 ? o_bf16_to_f32(sr) : f16_to_f32(sr);
                    uint32_t word = layout == 0 ? qw[(size_t)p * N + n] : qw[(size_t)n * (K / 8) + p];
                    int z = 8;
                    if (zeros) z = (int)((zeros[(size_t)g * (N / 8) + n / 8] >> (4 * (n % 8))) & 15u);
                    float wv[8], xv[8];
                    for (int j = 0; j < 8; j++) {
                        wv[j] = (float)((int)((word >> (4 * j)) & 15u) - z);
                        xv[j] = o_bf16_to_f32(xb[p * 8 + j]);
                    }
                    float d0 = ((xv[0] * wv[0] + xv[1] * wv[1]) + xv[2] * wv[2]) + xv[3] * wv[3];
                    float d1 = ((xv[4] * wv[4] + xv[5] * wv[5]) + xv[6] * wv[6]) + xv[7] * wv[7];
                    sum = fmaf(d0 + d1, sc, sum);
                }
                lanes[lane] = sum;
            }
            float total = nl == 1 ? lanes[0] : subgroup_add(lanes, 64);
            float v = total;
            if (finalize == 1) v = o_bf16_to_f32(aux[n]) + total;
            else if (finalize == 2) v = o_bf16_to_f32(aux[(size_t)b * N + n]) + round_bf16(total);
            y[(size_t)b * N + n] = o_f32_to_bf16(v);
        }
    }
}

/* Pair-packed symmetric INT8 activations (quantize_int8_symmetric_pairpacked.
 * comp.template:22-72): per 32-column block s = amax > 0 ? amax / 127 : 1,
 * q = round(clamp(x / s, -127, 127)) (GLSL round, taken here as round half
 * to even), sum = sum of the block's q.  Each 8 columns c..c+7 become two
 * words: bytes (q[c], q[c+2], q[c+4], q[c+6]) then (q[c+1], q[c+3], q[c+5],
 * q[c+7]), low byte first. */
void o_quantize_i8_pairpacked(const uint16_t* x, int rows, int cols, uint8_t* q, float* s, int32_t* sums) {
    int nblk = cols / 32;
    for (int r = 0; r < rows; r++) {
        const uint16_t* xr = x + (long)r * cols;
        for (int b = 0; b < nblk; b++) {
            float amax = 0.0f;
            for (int c = b * 32; c < b * 32 + 32; c++) amax = fmaxf(amax, fabsf(o_bf16_to_f32(xr[c])));
            float sc = amax > 0.0f ? amax / 127.0f : 1.0f;
            int sum = 0;
            for (int e = 0; e < 32; e++) {
                int c = b * 32 + e;
                float v = o_bf16_to_f32(xr[c]) / sc;
                v = v < -127.0f ? -127.0f : (v > 127.0f ? 127.0f : v);
                int iv = (int)rintf(v);
                sum += iv;
                int oct = e / 8, j = e % 8;
                int pos = b * 32 + oct * 8 + (j % 2) * 4 + j / 2;
                q[(long)r * cols + pos] = (uint8_t)(iv & 255);
            }
            s[(long)r * nblk + b] = sc;
            sums[(long)r * nblk + b] = sum;
        }
    }
}

/* silu(g) * u in bf16 (silu_multiply_quantize_int8_pairpacked.comp.template:
 * rounded_silu and main): y = bf16(bf16(g / (1 + exp(-g))) * u). */
void o_silu_multiply_bf16(const uint16_t* g, const uint16_t* u, long n, uint16_t* y) {
    for (long i = 0; i < n; i++) {
        float gv = o_bf16_to_f32(g[i]);
        float act = o_bf16_to_f32(o_f32_to_bf16(gv / (1.0f + expf(-gv))));
        y[i] = o_f32_to_bf16(act * o_bf16_to_f32(u[i]));
    }
}

/* Pair-packed INT8 x GPTQ INT4 linear (linear_prequant_pairpacked_int4_gptq.
 * comp.template:56-95): per output row, for each weight group and each
 * 32-column block of it, block_dot = -8 * sum + sum of the exact int8 x u4
 * products, then sum = fma(block_dot, s_x * s_w, sum) in group, block order. */
void o_int4_linear_pairpacked(const uint8_t* q, const float* s, const int32_t* sums, const uint32_t* qw,
                              const uint16_t* scales, int scale_bf16, int group, int K, int N, int B, int finalize,
                              const uint16_t* aux, uint16_t* y) {
    int nblk = K / 32;
    #pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++) {
        for (int b = 0; b < B; b++) {
            const int8_t* qb = (const int8_t*)(q + (size_t)b * K);
            float sum = 0.0f;
            for (int g = 0; g < K / group; g++) {
                uint16_t sr = scales[(size_t)g * N + n];
                float sw = scale_bf16 ? o_bf16_to_f32(sr) : f16_to_f32(sr);
                for (int blk = g * (group / 32); blk < (g + 1) * (group / 32); blk++) {
                    int dot = -8 * sums[(size_t)b * nblk + blk];
                    for (int p = blk * 4; p < blk * 4 + 4; p++) {
                        uint32_t word = qw[(size_t)p * N + n];
                        for (int j = 0; j < 8; j++) {
                            int pos = p * 8 + (j % 2) * 4 + j / 2;   /* pair-packed position of column 8p + j */
                            dot += (int)qb[pos] * (int)((word >> (4 * j)) & 15u);
                        }
                    }
                    sum = fmaf((float)dot, s[(size_t)b * nblk + blk] * sw, sum);
                }
            }
            float v = sum;
            if (finalize == 1) v = o_bf16_to_f32(aux[n]) + sum;
            else if (finalize == 2) v = o_bf16_to_f32(aux[(size_t)b * N + n]) + round_bf16(sum);
            y[(size_t)b * N + n] = o_f32_to_bf16(v);
        }
    }
}

/* Symmetric INT8 activations in natural byte order (quantize_int8_symmetric.
 * comp.template:38-58): per 32 columns s = amax > 0 ? amax / 127 : 1,
 * q = round(clamp(x / s, -127, 127)) (ties to even here; the GLSL round()
 * leaves the direction of exact .5 ties to the implementation). */
void o_quantize_i8(const uint16_t* x, int rows, int cols, uint8_t* q, float* s) {
    int nblk = cols / 32;
    for (int r = 0; r < rows; r++) {
        const uint16_t* xr = x + (long)r * cols;
        for (int b = 0; b < nblk; b++) {
            float amax = 0.0f;
            for (int c = b * 32; c < b * 32 + 32; c++) amax = fmaxf(amax, fabsf(o_bf16_to_f32(xr[c])));
            float sc = amax > 0.0f ? amax / 127.0f : 1.0f;
            for (int c = b * 32; c < b * 32 + 32; c++) {
                float v = o_bf16_to_f32(xr[c]) / sc;
                v = v < -127.0f ? -127.0f : (v > 127.0f ? 127.0f : v);
                q[(long)r * cols + c] = (uint8_t)((int)rintf(v) & 255);
            }
            s[(long)r * nblk + b] = sc;
        }
    }
}

/* INT8-prequant INT4 linear, unpaired input (q in natural byte order).
 * layout 0, linear_prequant_int4_gptq.comp.template:65-103: per output row,
 * for each weight group and each 32-column block of it, the exact integer
 * block_dot = sum of q * (code - 8), then sum = fma(block_dot, s_x * s_w,
 * sum).  layout 1, linear_prequant_int4_ct.comp.template:66-108: 64 lanes
 * take packed words (8 columns) lane, lane + 64, ...; each adds
 * fma(packed_dot, s_x[block] * s_w[group], lane_sum); then a subgroup add.
 * finalize as o_int4_linear. */
void o_int4_linear_prequant(int layout, const uint8_t* q, const float* s, const uint32_t* qw,
                            const uint16_t* scales, int scale_bf16, int group, int K, int N, int B, int finalize,
                            const uint16_t* aux, uint16_t* y) {
    int nblk = K / 32, G = K / group;
    #pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++) {
        for (int b = 0; b < B; b++) {
            const int8_t* qb = (const int8_t*)(q + (size_t)b * K);
            float sum = 0.0f;
            if (layout == 0) {
                for (int g = 0; g < G; g++) {
                    uint16_t sr = scales[(size_t)g * N + n];
                    float sw = scale_bf16 ? o_bf16_to_f32(sr) : f16_to_f32(sr);
                    for (int blk = g * (group / 32); blk < (g + 1) * (group / 32); blk++) {
                        int dot = 0;
                        for (int p = blk * 4; p < blk * 4 + 4; p++) {
                            uint32_t word = qw[(size_t)p * N + n];
                            for (int j = 0; j < 8; j++) dot += (int)qb[p * 8 + j] * ((int)((word >> (4 * j)) & 15u) - 8);
                        }
                        sum = fmaf((float)dot, s[(size_t)b * nblk + blk] * sw, sum);
                    }
                }
            } else {
                float lanes[64];
                for (int lane = 0; lane < 64; lane++) {
                    float ls = 0.0f;
                    for (int p = lane; p < K / 8; p += 64) {
                        uint32_t word = qw[(size_t)n * (K / 8) + p];
                        int dot = 0;
                        for (int j = 0; j < 8; j++) dot += (int)qb[p * 8 + j] * ((int)((word >> (4 * j)) & 15u) - 8);
                        uint16_t sr = scales[(size_t)n * G + (p * 8) / group];
                        float sw = scale_bf16 ? o_bf16_to_f32(sr) : f16_to_f32(sr);
                        ls = fmaf((float)dot, s[(size_t)b * nblk + (p * 8) / 32] * sw, ls);
                    }
                    lanes[lane] = ls;
                }
                sum = subgroup_add(lanes, 64);
            }
            float v = sum;
            if (finalize == 1) v = o_bf16_to_f32(aux[n]) + sum;
            else if (finalize == 2) v = o_bf16_to_f32(aux[(size_t)b * N + n]) + round_bf16(sum);
            y[(size_t)b * N + n] = o_f32_to_bf16(v);
        }
    }
}

/* ------------------------------------------------------------------ */
/* a10 / a11: FP8 output projection + argmax                             */
/* ------------------------------------------------------------------ */

/* tied_output_projection_fp8_e4m3.comp.template:87-144 (and the _batch twin
 * :94-186): input quantized per 128 block with amax/448 scale; logit[n] =
 * OUTPUT_SCALE * sum over 32-lane row clusters of fma(dot4, sx[b] *
 * s_w[n/BR, b], acc).  scale_inv: bf16 [ceil(N/BR), K/128]. */
void o_fp8_output_projection(const uint16_t* x, int M, int K, const uint8_t* W,
                             const uint16_t* scale_inv, int block_rows, int N,
                             float output_scale, float* logits) {
    int nblk = (K + 127) / 128;
    uint8_t* q = (uint8_t*)malloc((size_t)M * K);
    float* s = (float*)malloc(sizeof(float) * (size_t)M * nblk);
    float* qf = (float*)malloc(sizeof(float) * (size_t)M * K);
    o_quantize_blocks(x, K, M, K, 0, q, s);
    for (int m = 0; m < M; m++) decode_q(q + (size_t)m * K, K, qf + (size_t)m * K);
    #pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++) {
        const uint8_t* wr = W + (size_t)n * K;
        float wf[8192];
        int kk = K < 8192 ? K : 8192;
        for (int c = 0; c < kk; c++) wf[c] = o_e4m3_to_f32(wr[c]);
        for (int m = 0; m < M; m++) {
            float lanes[32];
            for (int lane = 0; lane < 32; lane++) {
                float acc = 0.0f;
                for (int w = lane; w < K / 4; w += 32) {
                    int c = w * 4, b = c / 128;
                    float sw = o_bf16_to_f32(scale_inv[(size_t)(n / block_rows) * nblk + b]);
                    acc = fmaf(dot4(qf + (size_t)m * K + c, wf + c), s[(size_t)m * nblk + b] * sw, acc);
                }
                lanes[lane] = acc;
            }
            logits[(size_t)m * N + n] = subgroup_add(lanes, 32) * output_scale;
        }
    }
    free(q); free(s); free(qf);
}

/* greedy_sampler_f32.comp.template:25-109: argmax, ties -> lower id. */
void o_argmax(const float* logits, int M, int N, uint32_t* ids) {
    for (int m = 0; m < M; m++) {
        float best = -3.4028234663852886e38f;
        uint32_t bi = 0;
        for (int n = 0; n < N; n++) {
            float v = logits[(size_t)m * N + n];
            if (v > best || (v == best && (uint32_t)n < bi)) { best = v; bi = (uint32_t)n; }
        }
        ids[m] = bi;
    }
}

/* ------------------------------------------------------------------ */
/* Sparse INT4 (compressed-tensors) experts                             */
/* ------------------------------------------------------------------ */

/* project_row (sparse_moe_gate_up_int4_ct.comp.template:124-149; the down
 * template's inner loop :156-174 is the same): 64 lane-strided chains of
 * sum = fma(dot(x[8c..8c+3], lo(w)) + dot(x[8c+4..8c+7], hi(w)), scale, sum)
 * over the packed words c of the row, then subgroupAdd.  lo/hi: codes 0-3 and
 * 4-7 of the word (low nibble first), each minus 8; scale[row, 8c / G]. */
static float ct_row_dot(const float* x, const uint32_t* wrow, const uint16_t* srow, int K, int G, int scale_bf16) {
    float lanes[SUBGROUP];
    int pc = K / 8;
    for (int lane = 0; lane < SUBGROUP; lane++) {
        float sum = 0.0f;
        for (int c = lane; c < pc; c += SUBGROUP) {
            uint32_t w = wrow[c];
            float lo[4], hi[4];
            for (int i = 0; i < 4; i++) {
                lo[i] = (float)((int)((w >> (4 * i)) & 15u) - 8);
                hi[i] = (float)((int)((w >> (16 + 4 * i)) & 15u) - 8);
            }
            uint16_t sb = srow[c * 8 / G];
            float sc = scale_bf16 ? o_bf16_to_f32(sb) : f16_to_f32(sb);
            sum = fmaf(dot4(x + 8 * c, lo) + dot4(x + 8 * c + 4, hi), sc, sum);
        }
        lanes[lane] = sum;
    }
    return subgroup_add(lanes, SUBGROUP);
}

/* Route selection shared by both stages (…gate_up_int4_ct.comp.template:
 * 142-166): position p < n_pos names route c = map[p] (map NULL: c = p);
 * routes whose expert is out of range or (expert_count != 0) outside
 * [expert_start, expert_start + expert_count) are skipped, as are experts
 * whose bank entry is marked unbound (bound[e] == 0; bound NULL: all bound). */
static int ct_route(const uint32_t* routes, const uint32_t* map, int p, int cap, int E, uint32_t start,
                    uint32_t count, const uint8_t* bound, uint32_t* c_out, uint32_t* e_out) {
    uint32_t c = map ? map[p] : (uint32_t)p;
    if (c >= (uint32_t)cap) return 0;
    uint32_t e = routes[c] & 0xffffu;
    if (e >= (uint32_t)E) return 0;
    if (count != 0 && (e < start || e - start >= count)) return 0;
    if (bound && !bound[e]) return 0;
    *c_out = c;
    *e_out = e;
    return 1;
}

/* Gate/up (…gate_up_int4_ct.comp.template:168-227): W u32 [E, 2I, H/8] (gate
 * rows then up rows), S [E, 2I, H/G]; inter bf16 [B, k, I] gets
 * bf16(bf16(silu(bf16 g)) * bf16 u) for each selected route. */
void o_sparse_int4_gate_up(const uint16_t* hidden, const uint32_t* routes, const uint32_t* map, int n_pos,
                           int B, int k, int E, int H, int I, int G, int scale_bf16, uint32_t start,
                           uint32_t count, const uint8_t* bound, const uint32_t* W, const uint16_t* S,
                           uint16_t* inter) {
    float* x = (float*)malloc(sizeof(float) * (size_t)H);
    for (int p = 0; p < n_pos; p++) {
        uint32_t c, e;
        if (!ct_route(routes, map, p, B * k, E, start, count, bound, &c, &e)) continue;
        int b = (int)(c / (uint32_t)k);
        for (int j = 0; j < H; j++) x[j] = o_bf16_to_f32(hidden[(size_t)b * H + j]);
        const uint32_t* we = W + (size_t)e * 2 * I * (H / 8);
        const uint16_t* se = S + (size_t)e * 2 * I * (H / G);
        #pragma omp parallel for schedule(static)
        for (int i = 0; i < I; i++) {
            float g = ct_row_dot(x, we + (size_t)i * (H / 8), se + (size_t)i * (H / G), H, G, scale_bf16);
            float u = ct_row_dot(x, we + (size_t)(I + i) * (H / 8), se + (size_t)(I + i) * (H / G), H, G,
                                 scale_bf16);
            g = round_bf16(g);
            u = round_bf16(u);
            inter[(size_t)c * I + i] = o_f32_to_bf16(round_bf16(g / (1.0f + expf(-g))) * u);
        }
    }
    free(x);
}

/* Down (…down_int4_ct.comp.template:131-193): W u32 [E, H, I/8], S [E, H,
 * I/G]; out bf16 [B, k, H] = bf16(bf16(y) * route_weight) for each selected
 * route, reading that route's intermediate slice inter [B, k, I]. */
void o_sparse_int4_down(const uint16_t* inter, const uint32_t* routes, const uint32_t* map, int n_pos, int B,
                        int k, int E, int H, int I, int G, int scale_bf16, uint32_t start, uint32_t count,
                        const uint8_t* bound, const uint32_t* W, const uint16_t* S, uint16_t* out) {
    float* x = (float*)malloc(sizeof(float) * (size_t)I);
    for (int p = 0; p < n_pos; p++) {
        uint32_t c, e;
        if (!ct_route(routes, map, p, B * k, E, start, count, bound, &c, &e)) continue;
        for (int j = 0; j < I; j++) x[j] = o_bf16_to_f32(inter[(size_t)c * I + j]);
        float wr = o_bf16_to_f32((uint16_t)(routes[c] >> 16));
        const uint32_t* we = W + (size_t)e * H * (I / 8);
        const uint16_t* se = S + (size_t)e * H * (I / G);
        #pragma omp parallel for schedule(static)
        for (int j = 0; j < H; j++) {
            float y = ct_row_dot(x, we + (size_t)j * (I / 8), se + (size_t)j * (I / G), I, G, scale_bf16);
            out[(size_t)c * H + j] = o_f32_to_bf16(round_bf16(round_bf16(y) * wr));
        }
    }
    free(x);
}
