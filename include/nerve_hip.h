/*
 * nerve_hip.h -- C ABI of the MI355X (gfx950) backend for NERVE's
 * quantized-matmul hot path.
 *
 * Conventions
 *   - Every device buffer is owned by the caller and passed as a raw device
 *     pointer; sizes are element counts given by the shape arguments.
 *   - Every operation enqueues on the caller's `stream` (a hipStream_t passed
 *     as void*; NULL = the default stream) and returns without synchronizing.
 *   - Host-side validation failures (bad specialization string, shape,
 *     alignment, NULL pointer) return a nonzero nerve_hip_status and set a
 *     thread-local message readable through nerve_hip_last_error().  This
 *     mirrors the reference's Result<_, String> error style
 *     (execution-contracts/src/lib.rs:8-17).
 *   - Device-side conditions fail closed exactly as the reference shaders do:
 *     an out-of-range expert id, an unbound parameter slot, a non-resident or
 *     too-short address record makes the affected route write nothing
 *     (runtime-rs/shaders/independent_sparse_moe_gate_up_batch1_mxfp4.
 *     comp.template:135-228).
 *   - A context is bound to one device.  Calls on one context must be
 *     externally serialized (the reference runs its tests and queues
 *     single-threaded: runtime-rs/.cargo/config.toml, AGENTS.md:3-9).  The
 *     context owns a device workspace that calls reuse; two calls on one
 *     context must not overlap on different streams.
 *
 * Buffer encodings are the compiled package's, unchanged:
 *   bf16 tensors       uint16 bit patterns, row-major ("words" of two, low half
 *                      = even element, as the templates read them)
 *   MXFP4 weight       u8 [rows, K/2], low nibble first along K
 *                      (nerve/quantized_layouts.py:4-7)
 *   MXFP4 scale        e8m0 u8 [rows, K/32]
 *   route word         (bf16(weight) << 16) | expert
 *   intermediates      u32 frames [B][k*I/2 + k]: bf16 h, then k route-map words
 *   BatchControl       u32[7] {batch_width, expert_start, expert_count,
 *                      owned_route_count, dispatch_x, dispatch_y, dispatch_z}
 *   address record     u32[8] {addr_lo, addr_hi, bytes_lo, bytes_hi, gen_lo,
 *                      gen_hi, resident(==1), representation}; the record
 *                      table passed to the MXFP4 projections must be 16-byte
 *                      aligned (NERVE_HIP_INVALID_ARGUMENT otherwise)
 *
 * Shape extension: the reference compiler requires hidden/intermediate/K to
 * be multiples of 128 (nerve/model_package_shader_templates.py:4805-4807,
 * 2437-2440).  This library also accepts multiples of 32 and treats the last
 * 128-column activation block as zero-padded (its amax is taken over the real
 * columns), which is the reference's result on zero-padded K.
 */
#ifndef NERVE_HIP_H
#define NERVE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NERVE_HIP_ABI_VERSION 1

typedef struct nerve_hip_ctx nerve_hip_ctx;

typedef enum {
    NERVE_HIP_OK = 0,
    NERVE_HIP_INVALID_ARGUMENT = 1,
    NERVE_HIP_INVALID_SPEC = 2,
    NERVE_HIP_UNSUPPORTED = 3,
    NERVE_HIP_DEVICE_ERROR = 4,
    NERVE_HIP_OUT_OF_MEMORY = 5
} nerve_hip_status;

/* ---- lifecycle --------------------------------------------------------- */

/* ABI version of the loaded library (NERVE_HIP_ABI_VERSION it was built with). */
int nerve_hip_abi_version(void);

/* Thread-local message for the last failing call on this thread ("" if none). */
const char* nerve_hip_last_error(void);

/* Opens a context on a HIP device ordinal.  Replaces the Vulkan device handle
 * the reference mounts kernels on (runtime-rs/src/vulkan_compute/
 * compute_device_dispatch.rs:2-249). */
nerve_hip_status nerve_hip_open(int device_ordinal, nerve_hip_ctx** out);

/* Releases the context and its workspace.  NULL is accepted. */
void nerve_hip_close(nerve_hip_ctx* ctx);

/* Validates a specialization string on the host, without a device: returns
 * NERVE_HIP_OK when some entry point of this library accepts it, else the
 * status that entry point would return (message via nerve_hip_last_error).
 * This is the check the reference compiler performs when it renders a
 * template (nerve/model_package_shader_templates.py:4773-5060, 2419-2465,
 * 3219-3276, 1513-1545), extended to shapes that are multiples of 32. */
nerve_hip_status nerve_hip_check_specialization(const char* spec);

/* ---- RMSNorm + FP8 prequantization -------------------------------------- */

/* Replaces rms_norm_quantize[_batch{T}]_fp8_e4m3[_spow2]_b{BLOCK}_h{H}_eps{E}
 * _offset{O}.comp (rms_norm_quantize_fp8_e4m3.comp.template:70-129; grammar
 * nerve/model_package_shader_templates.py:3530-3553): per row,
 * y = bf16(x * inversesqrt(mean(x^2) + eps) * (w + offset)) and, per BLOCK
 * columns, s = pow2 ("_spow2") or amax/448 scale of max |y|, q = e4m3(y / s).
 * x, y bf16 [rows, H] (y may be x: the batch form is in place); weight bf16
 * [H]; q e4m3 [rows, H]; scales f32 [rows, H / BLOCK].  The sum of squares
 * is a fixed tree of per-thread fma chains, so y can differ from the
 * shader's (whose order follows its subgroups) in the last bf16 place. */
nerve_hip_status nerve_hip_rms_norm_quantize_fp8_e4m3(nerve_hip_ctx* ctx, const char* spec,
                                                     const void* x_bf16, const void* weight_bf16,
                                                     void* y_bf16, void* q_e4m3, void* scales_f32,
                                                     uint32_t rows, void* stream);

/* Replaces rms_norm_quantize[_batch{T}]_int8_pairpacked_b32_h{H}_eps{E}
 * _offset{O}.comp (rms_norm_quantize_int8_pairpacked.comp.template:60-151;
 * grammar nerve/model_package_shader_templates.py:3357-3375): the same y as
 * above, then the pair-packed INT8 quantization of
 * nerve_hip_quantize_int8_pairpacked applied to y (q int8 [rows, H], scales
 * f32 and sums i32 [rows, H/32]), feeding nerve_hip_int4_linear_pairpacked. */
nerve_hip_status nerve_hip_rms_norm_quantize_int8_pairpacked(nerve_hip_ctx* ctx, const char* spec,
                                                            const void* x_bf16, const void* weight_bf16,
                                                            void* y_bf16, void* q_i8, void* scales_f32,
                                                            void* sums_i32, uint32_t rows, void* stream);

/* ---- a2: activation block quantization -------------------------------- */

/* Replaces quantize_fp8_e4m3[_spow2]_b128_h{N}.comp
 * (runtime-rs/shaders/quantize_fp8_e4m3.comp.template:41-59; specialization
 * nerve/model_package_shader_templates.py:1513-1545), batched over `rows`.
 * x: bf16 [rows, N]; q: e4m3 [rows, N]; scales: f32 [rows, ceil(N/128)].
 * "_spow2" uses the power-of-two scale of the MXFP4 expert kernels
 * (…gate_up_batch1_mxfp4.comp.template:357-363), otherwise amax/448. */
nerve_hip_status nerve_hip_quantize_fp8_e4m3(nerve_hip_ctx* ctx, const char* spec,
                                             const void* x_bf16, uint32_t rows,
                                             void* q_e4m3, void* scales_f32, void* stream);

/* ---- raw MXFP4 GEMV (config-0 entry; parity and measurement) ----------- */

/* y[m, n] = sum_k e4m3(x)[m,k] * sx[m,k/128] * e2m1(W)[n,k] * e8m0(S)[n,k/32]
 * in f32, for pre-quantized activations (the a2 output).  This is the
 * accumulation of …gate_up_batch1_mxfp4.comp.template:759-787 without the
 * SwiGLU epilogue.  q: e4m3 [M, K]; sx: f32 [M, ceil(K/128)]; W: u8 [N, K/2];
 * S: u8 [N, K/32]; y: f32 [M, N].  M <= 64. */
nerve_hip_status nerve_hip_mxfp4_gemv(nerve_hip_ctx* ctx, const void* q_e4m3,
                                      const void* scales_f32, uint32_t M, uint32_t K,
                                      const void* weight, const void* weight_scale,
                                      uint32_t N, void* y_f32, void* stream);

/* ---- a5: router projection --------------------------------------------- */

/* Replaces linear_bf16.comp.template:40-98 for the router node
 * (nerve/circuit_lowering_sparse_experts.py:82-88), batched:
 * logits[b, e] = bf16(sum_k x[b,k] * W[e,k]).  x: bf16 [B, H]; W: bf16 [E, H];
 * logits: bf16 [B, E]. */
nerve_hip_status nerve_hip_router_linear_bf16(nerve_hip_ctx* ctx, const void* x_bf16,
                                              const void* weight_bf16, void* logits_bf16,
                                              uint32_t batch_width, uint32_t hidden,
                                              uint32_t experts, void* stream);

/* ---- a6: top-k routing -------------------------------------------------- */

/* Replaces moe_topk[_batch1]_{sigmoid|softmax}_bf16_e{E}_k{k}_norm{0|1}_cap{c}_
 * {nobias|biasf32|biasbf16}.comp (moe_topk_routed_batch1_bf16.comp.template:
 * 71-182) and moe_router[_batch1]_score_topk_{sigmoid|softmax|sqrtsoftplus}_
 * bf16_r{E}_k{k}_a{A}w{w}_norm{0|1}_scale{s}_bias{f32|bf16}.comp
 * (moe_router_score_topk_batch1_bf16.comp.template:109-219); grammar in
 * nerve/model_package_shader_templates.py:4850-5060.
 * logits: bf16 [B, E]; bias: f32 [E] or bf16 [E] per spec, or NULL for
 * "nobias"; routes: u32 [B, k(+A)]; telemetry: u32 [T + T(T-1)/2] counters
 * (T = E(+A)), incremented atomically, or NULL to skip them. */
nerve_hip_status nerve_hip_moe_router_topk(nerve_hip_ctx* ctx, const char* spec,
                                           const void* logits_bf16, const void* bias,
                                           void* routes_u32, void* telemetry_u32,
                                           uint32_t batch_width, void* stream);

/* ---- a5 + a6 + a7 in one launch (decode-sized batches) ------------------- */

/* One launch in place of the router linear (linear_bf16.comp.template:
 * 47-68), the top-k (moe_topk_routed_batch1_bf16.comp.template:71-182 or
 * moe_router_score_topk_batch1_bf16.comp.template:109-219) and the route
 * compaction for `moe_spec`'s projection (moe_route_compact_batch1.comp.
 * template:26-106): the node pair linear -> moe_route of
 * nerve/circuit_lowering_sparse_experts.py:82-88 plus the route-scheduling
 * stage before gate_up (nerve/model_package_batching.py:265-284).  The
 * logits (f32 sums over up to 16 K slices added in slice order, rounded to
 * bf16; the last block of the launch to finish its slice does the rest)
 * are within one bf16 ulp of nerve_hip_router_linear_bf16's; routes,
 * telemetry, the route map and the control words are exactly what
 * nerve_hip_moe_router_topk + nerve_hip_moe_route_compact produce from
 * those logits.  logits_bf16 may be NULL.  hidden comes from moe_spec; the
 * top-k experts and k (plus always-selected experts) must match moe_spec.
 * hidden_e4m3 / hidden_scales_f32 (both or neither; u8 [B, H], f32
 * [B, ceil(H/128)]): the hidden rows quantized as the gate/up projection
 * quantizes them (quantize_hidden, …gate_up_batch1_mxfp4.comp.template:
 * 366-382: pow2 block scales), bit for bit, for its `_prequant` form; the
 * blocks that finish their partial sums before the last one write them.
 * Returns NERVE_HIP_UNSUPPORTED (nothing launched) above 64 tokens, 256
 * experts or 1024 routes: use the three entry points then.  Calls on one
 * context must not overlap (other streams, parallel graph branches): they
 * share the context's partial-sum buffer and arrival counter. */
nerve_hip_status nerve_hip_moe_route_fused(nerve_hip_ctx* ctx, const char* topk_spec,
                                           const char* moe_spec, const void* x_bf16,
                                           const void* router_weight_bf16, void* logits_bf16,
                                           const void* bias, void* routes_u32,
                                           void* telemetry_u32, void* intermediates,
                                           void* control_u32, void* hidden_e4m3,
                                           void* hidden_scales_f32, uint32_t batch_width,
                                           void* stream);

/* ---- a7: expert-sorted route permutation -------------------------------- */

/* Replaces moe_route_compact_batch1 (moe_route_compact_batch1.comp.template:
 * 26-106) and, when `intermediates` is NULL, moe_route_count_batch1
 * (moe_route_count_batch1.comp.template:21-58).  `spec` is the consuming
 * projection's specialization (it fixes I, k and the tile count per route).
 * control: device BatchControl; fields 0..2 are read, 3..6 are written.
 * The route map goes to the tail k words of each intermediate frame.  With
 * expert_count == 0 the map is the stable sort of routes by expert; otherwise
 * it lists the routes of experts in [expert_start, expert_start+expert_count)
 * in source order. */
nerve_hip_status nerve_hip_moe_route_compact(nerve_hip_ctx* ctx, const char* spec,
                                             const void* routes_u32, void* intermediates,
                                             void* control_u32, uint32_t batch_width,
                                             void* stream);

/* ---- a2+a3: MXFP4 gate/up + SwiGLU -------------------------------------- */

/* Replaces independent_sparse_moe_gate_up[_batch1][_prequant]_mxfp4_e2m1_g32_
 * h{H}_i{I}_e{E}_k{k}_limit{L}.comp (…gate_up_batch1_mxfp4.comp.template:
 * 643-802; grammar nerve/model_package_shader_templates.py:4773-4846).
 * Inputs follow the template's bindings: hidden bf16 [B, H] (or, for
 * "_prequant", hidden = e4m3 [B, H] and hidden_scales = f32 [B, H/128]),
 * routes u32 [B, k], intermediates (frames, map read from the tails),
 * addresses u32 [8 * address_records], param_slots u32 [4 * E]
 * (gate_w, gate_s, up_w, up_s).  control: device BatchControl (batch_width
 * given on the host; expert_count and owned_route_count read on the device).
 * The grid is sized for batch_width * k routes; routes past the owned count
 * exit on the device, which replaces the reference's indirect dispatch.
 * e4m3 expert banks (…_mxfp4_e2m1_{resident,adaptive}_fp8_e4m3_g32 and
 * …_g32_native_fp8_e4m3_se8m0_b128_nf{N}; gate_up template :173-229,
 * :299-355) take e4m3 weights [I, H] with the per-32 scales (pre-expanded)
 * or a [ceil(I/128), ceil(H/128)] e8m0 grid (experts >= N); adaptive banks
 * pick compact or expanded per expert by address-record word 7.  Both
 * projection entry points accept them for E <= 1024.
 * Tensor-parallel slices (…gate_up_batch1[_tensor_parallel][_prequant]_…,
 * template :487-641): one rank's share; the expert's four records cover its
 * rows [0, L) of the intermediate, L = gate weight record bytes / (H / 2),
 * and intermediates receives bf16 route-major local rows [B, k, L]; routes
 * are read per token in order (no route map) and control is not read (any
 * non-null buffer).  A token's routes after its first out-of-range or
 * invalid expert are left untouched.  Compact MXFP4 only, H <= 4096. */
nerve_hip_status nerve_hip_mxfp4_moe_gate_up(nerve_hip_ctx* ctx, const char* spec,
                                             const void* hidden, const void* hidden_scales,
                                             const void* routes_u32, void* intermediates,
                                             const void* addresses_u32, uint32_t address_records,
                                             const void* param_slots_u32, uint32_t param_slot_words,
                                             const void* control_u32, uint32_t batch_width,
                                             void* stream);

/* ---- a2+a4: MXFP4 down + route weight ----------------------------------- */

/* Replaces independent_sparse_moe_down[_batch1]_mxfp4_e2m1_g32_h{H}_i{I}_e{E}_
 * k{k}.comp (…down_batch1_mxfp4.comp.template:507-610).  Reads h from the
 * intermediate frames (map in the tails), writes expert_outputs bf16
 * [B, k, H] = bf16(y * route_weight); param_slots u32 [2 * E]
 * (down_w, down_s).  With an input_block_major_b128 spec the down
 * parameters are W [I/128, H, 64] and S [I/128, H, 4] bytes
 * (…down_batch1_mxfp4.comp.template:229-233, :260-263); decode-sized
 * batches stream that layout, larger ones read it through the preparation
 * launch and a register-fed kernel (E <= 1024).
 * Tensor-parallel slice (…down_batch1_tensor_parallel_input_block_major_b128_
 * …, template :421-505): control points to the device push constants
 * {input_start, input_count}; intermediates holds the local slice bf16
 * [B, k, input_count] (input_count a multiple of 32, at most I, else nothing
 * is written), the records the slice's blocks [I-blocks, H, 64] / [.., H, 4];
 * expert_outputs receives f32 [B, k, H] partial sums, not scaled by the route
 * weight (the ranks' partials are summed, then scaled, by the caller).
 * A token's routes after its first invalid expert are left untouched.
 * Compact MXFP4 only, I <= 4096; the counted form refuses it. */
nerve_hip_status nerve_hip_mxfp4_moe_down(nerve_hip_ctx* ctx, const char* spec,
                                          const void* intermediates, const void* routes_u32,
                                          void* expert_outputs,
                                          const void* addresses_u32, uint32_t address_records,
                                          const void* param_slots_u32, uint32_t param_slot_words,
                                          const void* control_u32, uint32_t batch_width,
                                          void* stream);

/* Count stage + down in one launch: nerve_hip_moe_route_compact(spec,
 * routes, NULL, control) followed by nerve_hip_mxfp4_moe_down (the reference
 * runs moe_route_count_batch1 then the down shader,
 * nerve/model_package_batching.py:265-284).  It requires that control[3],
 * [5] and [6] already hold what the count stage writes, which is the case
 * after a compaction (nerve_hip_moe_route_compact or
 * nerve_hip_moe_route_fused) of the same routes and control[0..2]; it then
 * writes control[4] = (expert_count ? control[3] : k) * ceil(H / 64), the one
 * word the count stage changes, and the same expert_outputs as the down
 * entry point. */
nerve_hip_status nerve_hip_mxfp4_moe_down_counted(nerve_hip_ctx* ctx, const char* spec,
                                                  const void* intermediates, const void* routes_u32,
                                                  void* expert_outputs,
                                                  const void* addresses_u32, uint32_t address_records,
                                                  const void* param_slots_u32, uint32_t param_slot_words,
                                                  void* control_u32, uint32_t batch_width,
                                                  void* stream);

/* ---- a8: weighted combine ----------------------------------------------- */

/* Replaces moe_reduce[_batch1]_bf16 (moe_reduce_batch1_bf16.comp.template:
 * 29-54): out[b, j] = bf16(bf16-sequential-sum_r expert_outputs[b, r, j] *
 * routed_scale).  expert_outputs bf16 [B, k, H]; out bf16 [B, H]. */
nerve_hip_status nerve_hip_moe_reduce(nerve_hip_ctx* ctx, const void* expert_outputs,
                                      void* out_bf16, uint32_t batch_width, uint32_t hidden,
                                      uint32_t experts_per_token, float routed_scale,
                                      void* stream);

/* ---- sparse INT4 (compressed-tensors) experts --------------------------- */

/* Replace sparse_moe_gate_up[_batch1]_int4_ct_s{f16|bf16}_g{G}_h{H}_i{I}_e{E}_
 * k{k}.comp (sparse_moe_gate_up_int4_ct.comp.template:97-227) and
 * sparse_moe_down[_batch1]_int4_ct_….comp (sparse_moe_down_int4_ct.comp.
 * template:106-193; grammar and rendering nerve/model_package_sparse_
 * projection_shaders.py:80-232).  Per expert two parameter slots
 * (param_slots u32 [2 * E]): CT-packed weights u32 [rows, K/8] (codes low
 * nibble first, value code - 8) and f16/bf16 scales [rows, K/G]; gate_up rows
 * are the I gate rows then the I up rows (K = H), down rows are H (K = I).
 * gate_up writes h = bf16(bf16(silu(bf16 g)) * bf16 u) into the intermediate
 * slices; down writes expert_outputs bf16 [B, k, H] = bf16(bf16(y) *
 * route_weight).
 * "_batch1" (frame-parallel) form: frames [B][k*I/2 + k] with the route map
 * in the tails (nerve_hip_moe_route_compact with this spec writes it) and
 * control = BatchControl, exactly as the MXFP4 entry points.  Unbatched form:
 * batch_width 1, intermediates [k][I/2] words without a map, and control
 * either NULL (every expert) or a BatchControl whose words 1 and 2 give the
 * owned expert range (DispatchControl {expert_start, expert_count}).
 * Slots that are unbound, beyond the table, or whose record has a null or
 * misaligned address (weights: 16-byte aligned, scales: 2-byte aligned) or
 * fewer bytes than the expert's tensor skip the route
 * (the reference skips unbound slots only).  Needs K % 32 == 0 and
 * K <= 16384. */
nerve_hip_status nerve_hip_int4_moe_gate_up(nerve_hip_ctx* ctx, const char* spec, const void* hidden_bf16,
                                            const void* routes_u32, void* intermediates,
                                            const void* addresses_u32, uint32_t address_records,
                                            const void* param_slots_u32, uint32_t param_slot_words,
                                            const void* control_u32, uint32_t batch_width, void* stream);
nerve_hip_status nerve_hip_int4_moe_down(nerve_hip_ctx* ctx, const char* spec, const void* intermediates,
                                         const void* routes_u32, void* expert_outputs,
                                         const void* addresses_u32, uint32_t address_records,
                                         const void* param_slots_u32, uint32_t param_slot_words,
                                         const void* control_u32, uint32_t batch_width, void* stream);

/* ---- a9: group-scaled INT4 linear --------------------------------------- */

/* Replaces {linear|linear_bias|linear_residual}[_batch{T}]_int4_{gptq|ct}_
 * s{f16|bf16}_g{G}_{K}x{N}.comp (linear_int4_gptq.comp.template:47-135,
 * linear_int4_ct.comp.template:49-150; replacements nerve/model_package_
 * shader_selection.py:2469-2549).  x: bf16 [B, K]; qweight: u32 [K/8, N]
 * (gptq) or [N, K/8] (ct); scales: f16/bf16 [K/G, N] (gptq) or [N, K/G]
 * (ct); zeros: NULL for the reference's symmetric code-8 ABI, or (gptq only,
 * an extension outside the reference ABI) AutoGPTQ qzeros u32 [K/G, N/8];
 * aux: bias bf16 [N] (linear_bias) or residual bf16 [B, N] (linear_residual),
 * else NULL; y: bf16 [B, N].  Also replaces {op}_batch64_cooperative_int4_
 * {gptq|ct}_s{f16|bf16}_g{G}_{K}x{N}.comp (linear_batch_cooperative_int4.
 * comp.template:85-233; grammar nerve/model_package_shader_templates.py:
 * 3148-3215): per group, the bf16 MFMA sum of (code - 8) x, then
 * fma(group_sum, scale, acc), any batch_width (the CT layout with group % 128
 * != 0 returns NERVE_HIP_UNSUPPORTED). */
nerve_hip_status nerve_hip_int4_linear(nerve_hip_ctx* ctx, const char* spec,
                                       const void* x_bf16, const void* qweight,
                                       const void* scales, const void* zeros,
                                       const void* aux_bf16, void* y_bf16,
                                       uint32_t batch_width, void* stream);

/* ---- pair-packed INT8 x INT4 (the int8-prequant GPTQ linear) ------------ */

/* Replaces quantize[_batch{T}]_int8_symmetric_pairpacked_b32_h{N}.comp
 * (quantize_int8_symmetric_pairpacked.comp.template:22-72; grammar
 * nerve/model_package_shader_templates.py:1440-1474): per 32 columns
 * s = amax > 0 ? amax / 127 : 1, q = round(clamp(x / s, -127, 127)) (round
 * half to even), sums = the block's sum of q; columns c..c+7 become the words
 * (q[c], q[c+2], q[c+4], q[c+6]), (q[c+1], q[c+3], q[c+5], q[c+7]).
 * x bf16 [rows, N]; q int8 [rows, N]; scales f32 and sums i32 [rows, N/32].
 * Also replaces the unpaired quantize[_batch{T}]_int8_symmetric_b32_h{N}.comp
 * (quantize_int8_symmetric.comp.template:38-58; grammar :1478-1506): the same
 * codes and scales with q in column order; sums may then be NULL (written
 * when given). */
nerve_hip_status nerve_hip_quantize_int8_pairpacked(nerve_hip_ctx* ctx, const char* spec, const void* x_bf16,
                                                   void* q_i8, void* scales_f32, void* sums_i32, uint32_t rows,
                                                   void* stream);

/* Replaces silu_multiply_quantize[_batch{T}]_int8_pairpacked_b32_h{N}.comp
 * (silu_multiply_quantize_int8_pairpacked.comp.template): y = bf16(bf16(
 * g / (1 + exp(-g))) * u) for gate and up bf16 [rows, N], written to y, and
 * the pair-packed INT8 quantization of y as above.  y must not overlap gate
 * or up (NERVE_HIP_INVALID_ARGUMENT otherwise). */
nerve_hip_status nerve_hip_silu_multiply_quantize_int8_pairpacked(nerve_hip_ctx* ctx, const char* spec,
                                                                 const void* gate_bf16, const void* up_bf16,
                                                                 void* y_bf16, void* q_i8, void* scales_f32,
                                                                 void* sums_i32, uint32_t rows, void* stream);

/* Replaces {linear,linear_bias,linear_residual}_prequant_pairpacked[_batch{T}]
 * _int4_gptq_s{f16,bf16}_g{G}_{K}x{N}.comp
 * (linear_prequant_pairpacked_int4_gptq.comp.template:56-128): y = bf16 of
 * sum over groups and 32-column blocks of fma(-8 sums + sum_k q (code),
 * s_x * s_w), with the bias / residual finalize of nerve_hip_int4_linear.
 * q, scales_f32, sums as nerve_hip_quantize_int8_pairpacked writes them;
 * qweight u32 [K/8, N], scales [K/G, N].
 * Also replaces the unpaired {linear,linear_bias,linear_residual}_prequant
 * [_batch{T}]_int4_{gptq,ct}_s{f16,bf16}_g{G}_{K}x{N}.comp
 * (linear_prequant_int4_gptq.comp.template:65-103, linear_prequant_int4_ct.
 * comp.template:66-108): q in column order (the unpaired quantizer), sums
 * unused (NULL), block_dot = sum_k q (code - 8); the CT layout takes qweight
 * u32 [N, K/8] and scales [N, K/G]. */
nerve_hip_status nerve_hip_int4_linear_pairpacked(nerve_hip_ctx* ctx, const char* spec, const void* q_i8,
                                                 const void* scales_f32, const void* sums_i32,
                                                 const void* qweight, const void* scales, const void* aux_bf16,
                                                 void* y_bf16, uint32_t batch_width, void* stream);

/* ---- a10+a11: FP8 output projection + fused argmax ----------------------- */

/* Replaces tied_output_projection[_batch{T}]_fp8_e4m3_b{BR}x128_{N}x{K}_
 * scale{S}_to_f32.comp (tied_output_projection_fp8_e4m3.comp.template:87-144,
 * …_batch_fp8_e4m3.comp.template:94-186) followed by greedy_sampler_f32
 * (greedy_sampler_f32.comp.template:25-109) / argmax_candidate_reduce.
 * x: bf16 [B, K]; weight: e4m3 [N, K]; scale_inv: bf16 [ceil(N/BR), K/128];
 * logits_f32: f32 [B, N] (the reference's output) or NULL; logits_bf16:
 * bf16 [B, N] or NULL; argmax: u32 [B] (ties -> lower id, on the f32 logits)
 * or NULL. */
nerve_hip_status nerve_hip_fp8_output_projection(nerve_hip_ctx* ctx, const char* spec,
                                                 const void* x_bf16, const void* weight_e4m3,
                                                 const void* scale_inv_bf16, void* logits_f32,
                                                 void* logits_bf16, void* argmax_u32,
                                                 uint32_t batch_width, void* stream);

/* No counterpart in the reference: the FP8 output projection of
 * nerve_hip_fp8_output_projection (same arguments, same results, same
 * kernels) for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  Its
 * scratch (quantized activations, per-row scale flags, argmax partials) is a
 * file-scope device array of 4 MiB per GPU, resolved once per device by
 * nerve_hip_open; it calls no hipMalloc/hipFree.  A call whose scratch would
 * exceed 4 MiB returns NERVE_HIP_INVALID_ARGUMENT without launching (e.g.
 * N = 201088, K = 2880 fits up to M = 128).  Calls on one GPU share the array:
 * two that overlap (other streams, other contexts on the same device) race;
 * nothing is kept between calls. */
nerve_hip_status nerve_hip_fp8_output_projection_noalloc(nerve_hip_ctx* ctx, const char* spec,
                                                         const void* x_bf16, const void* weight_e4m3,
                                                         const void* scale_inv_bf16, void* logits_f32,
                                                         void* logits_bf16, void* argmax_u32,
                                                         uint32_t batch_width, void* stream);

/* Standalone greedy argmax over f32 logits [B, N] (greedy_sampler_f32.comp.
 * template:25-109 without its stream-control bookkeeping). */
nerve_hip_status nerve_hip_argmax_f32(nerve_hip_ctx* ctx, const void* logits_f32,
                                      uint32_t batch_width, uint32_t vocab, void* argmax_u32,
                                      void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NERVE_HIP_H */
