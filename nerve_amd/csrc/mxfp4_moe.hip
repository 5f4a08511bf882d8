// MXFP4 expert projections on gfx950 scaled MFMA.
//
// The reference (independent_sparse_moe_{gate_up,down}_batch1_mxfp4.comp.
// template) quantizes each 128-column activation block to e4m3 with a
// power-of-two scale and accumulates fp8_dot4(e4m3 act, e4m3(e2m1 weight)) *
// (act_scale * e8m0_weight_scale).  That is exactly the contraction computed
// by V_MFMA_SCALE_F32_16X16X128_F8F6F4 with A = e4m3 activations (scale =
// e8m0 of the pow2 block scale) and B = e2m1 weights straight from the packed
// package bytes (scale = the package's e8m0 byte).  No dequantization runs on
// the VALU: each lane streams 16 bytes of one weight row (one MX block of 32
// values) per MFMA.
//
// Operand layout of the 16x16x128 f8f6f4 MFMA (lane l, g = l/16, r = l%16),
// measured on gfx950:
//   fp8 operand: bytes 0-15 hold k = 16g..16g+15, bytes 16-31 hold
//                k = 64+16g..64+16g+15 of row r;
//   fp4 operand: 16 bytes hold k = 32g..32g+31 (low nibble first) of row r;
//   scale operand: lane (g, r) supplies the e8m0 scale of row r, k-block g;
//   result: lane (g, r) holds D[4g+i][r], i = 0..3.
#include "common.h"

namespace {

constexpr uint32_t UNBOUND_SLOT = 0xffffffffu;

// ---------------------------------------------------------------------------
// a2: blockwise e4m3 quantization of bf16 rows.
// Row r lives at element offset (r / k) * frame_elems + (r % k) * seg_elems,
// which covers plain [rows, cols] tensors (k = 1) and the per-route slices of
// the intermediate frames.  One 32-lane cluster per 128-column block, as in
// quantize_hidden (…gate_up_batch1_mxfp4.comp.template:366-382).
// ---------------------------------------------------------------------------
template <bool POW2>
__global__ __launch_bounds__(256) void quant_rows_kernel(const uint16_t* __restrict__ x, uint32_t k,
                                                          uint64_t frame_elems, uint64_t seg_elems,
                                                          uint32_t cols, uint32_t rows,
                                                          uint8_t* __restrict__ q, float* __restrict__ s) {
    const uint32_t row = blockIdx.y;
    if (row >= rows) return;
    const uint32_t nblk = (cols + 127) / 128;
    const uint32_t blk = blockIdx.x * 8 + (threadIdx.x >> 5);
    const uint32_t cl = threadIdx.x & 31;
    const uint32_t col = blk * 128 + cl * 4;
    const bool valid = blk < nblk && col < cols;
    const uint16_t* xr = x + (uint64_t)(row / k) * frame_elems + (uint64_t)(row % k) * seg_elems;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (valid) {
        const uint32_t* p = reinterpret_cast<const uint32_t*>(xr + col);
        uint32_t w0 = p[0], w1 = p[1];
        v[0] = bf16_to_f32(w0); v[1] = bf16_to_f32(w0 >> 16);
        v[2] = bf16_to_f32(w1); v[3] = bf16_to_f32(w1 >> 16);
    }
    float m = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    m = wave_max32(m);
    if (!valid) return;
    float sc = POW2 ? pow2_fp8_scale(m) : amax_fp8_scale(m);
    if (cl == 0) s[(uint64_t)row * nblk + blk] = sc;
    uint32_t packed = f32_to_e4m3(v[0] / sc) | (f32_to_e4m3(v[1] / sc) << 8) |
                      (f32_to_e4m3(v[2] / sc) << 16) | (f32_to_e4m3(v[3] / sc) << 24);
    *reinterpret_cast<uint32_t*>(q + (uint64_t)row * cols + col) = packed;
}

// ---------------------------------------------------------------------------
// MFMA operand loaders.
// ---------------------------------------------------------------------------

// Weight operand for chunk `c` (128 K): lane group g takes MX block 4c+g of
// its row: 16 packed bytes + 1 e8m0 byte.
__device__ __forceinline__ void load_w(const uint8_t* __restrict__ wrow, const uint8_t* __restrict__ srow,
                                       uint32_t K, uint32_t c, uint32_t g, v4i& w, uint32_t& sc) {
    const uint32_t k0 = c * 128 + g * 32;
    if (k0 < K) {
        w = *reinterpret_cast<const v4i*>(wrow + k0 / 2);
        sc = srow[k0 / 32];
    } else {
        w = v4i{0, 0, 0, 0};
        sc = 127;
    }
}

// Activation operand for chunk `c`: k = 16g.. and 64+16g.. of the token row
// (the fp8 "halves" layout), scale = e8m0 of the row's pow2 block scale.
__device__ __forceinline__ void load_a(const uint8_t* __restrict__ arow, const float* __restrict__ ascale,
                                       uint32_t K, uint32_t c, uint32_t g, v8i& a, uint32_t& sc) {
    const uint32_t k0 = c * 128 + g * 16;
    v4i lo = v4i{0, 0, 0, 0}, hi = v4i{0, 0, 0, 0};
    sc = 127;
    if (arow) {
        if (k0 < K) lo = *reinterpret_cast<const v4i*>(arow + k0);
        if (k0 + 64 < K) hi = *reinterpret_cast<const v4i*>(arow + k0 + 64);
        sc = pow2_to_e8m0(ascale[c]);
    }
    a = v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
}

__device__ __forceinline__ v4f mfma_fp8_fp4(const v8i& a, const v4i& w, uint32_t sa, uint32_t sw, v4f acc) {
    v8i b = v8i{w.x, w.y, w.z, w.w, 0, 0, 0, 0};
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, acc, 0, 4, 0, (int)sa, 0, (int)sw);
}

// Contraction of one 16-row weight tile against one 16-token activation tile
// over chunks [c0, c1), four chunks in flight per iteration.
template <int NMAT>
__device__ __forceinline__ void mx_tile_loop(const uint8_t* __restrict__ arow, const float* __restrict__ ascale,
                                             const uint8_t* const* wrow, const uint8_t* const* srow, uint32_t K,
                                             uint32_t c0, uint32_t c1, uint32_t g, v4f* acc) {
    uint32_t c = c0;
    for (; c + 4 <= c1; c += 4) {
        v8i a[4];
        uint32_t sa[4];
        v4i w[NMAT][4];
        uint32_t sw[NMAT][4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
#pragma unroll
            for (int m = 0; m < NMAT; m++) load_w(wrow[m], srow[m], K, c + u, g, w[m][u], sw[m][u]);
        }
#pragma unroll
        for (int u = 0; u < 4; u++) load_a(arow, ascale, K, c + u, g, a[u], sa[u]);
#pragma unroll
        for (int u = 0; u < 4; u++) {
#pragma unroll
            for (int m = 0; m < NMAT; m++) acc[m] = mfma_fp8_fp4(a[u], w[m][u], sa[u], sw[m][u], acc[m]);
        }
    }
    for (; c < c1; c++) {
        v8i a;
        uint32_t sa;
        load_a(arow, ascale, K, c, g, a, sa);
#pragma unroll
        for (int m = 0; m < NMAT; m++) {
            v4i w;
            uint32_t sw;
            load_w(wrow[m], srow[m], K, c, g, w, sw);
            acc[m] = mfma_fp8_fp4(a, w, sa, sw, acc[m]);
        }
    }
}

// ---------------------------------------------------------------------------
// Raw GEMV (config-0 entry): y[M, N] f32.  One block = 16 weight rows; its
// KSPLIT waves split the K chunks and reduce through LDS.
// ---------------------------------------------------------------------------
template <int KSPLIT>
__global__ __launch_bounds__(64 * KSPLIT) void mxfp4_gemv_kernel(const uint8_t* __restrict__ q, const float* __restrict__ qs,
                                                                  uint32_t M, uint32_t K, const uint8_t* __restrict__ W,
                                                                  const uint8_t* __restrict__ S, uint32_t N,
                                                                  float* __restrict__ y) {
    __shared__ v4f part[KSPLIT][64];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t g = lane >> 4, rr = lane & 15;
    const uint32_t n0 = blockIdx.x * 16;
    const uint32_t nchunk = (K + 127) / 128, nblk = nchunk;
    const uint32_t per = (nchunk + KSPLIT - 1) / KSPLIT;
    const uint32_t c0 = min(nchunk, wave * per), c1 = min(nchunk, c0 + per);
    const uint8_t* wrow[1] = {W + (uint64_t)(n0 + rr) * (K / 2)};
    const uint8_t* srow[1] = {S + (uint64_t)(n0 + rr) * (K / 32)};
    for (uint32_t m0 = 0; m0 < M; m0 += 16) {
        const uint32_t tok = m0 + rr;
        const uint8_t* arow = tok < M ? q + (uint64_t)tok * K : nullptr;
        const float* ascale = qs + (uint64_t)(tok < M ? tok : 0) * nblk;
        v4f acc[1] = {v4f{0.f, 0.f, 0.f, 0.f}};
        mx_tile_loop<1>(arow, ascale, wrow, srow, K, c0, c1, g, acc);
        part[wave][lane] = acc[0];
        __syncthreads();
        if (wave == 0) {
            v4f t = part[0][lane];
#pragma unroll
            for (int w = 1; w < KSPLIT; w++) t += part[w][lane];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                uint32_t m = m0 + 4 * g + i;
                if (m < M) y[(uint64_t)m * N + n0 + rr] = t[i];
            }
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Route -> expert tile lists (replaces the per-route workgroups of the
// reference's indirect dispatch).  One 1024-thread block.
// ---------------------------------------------------------------------------
constexpr uint32_t MAX_EXPERTS = 4096;

__device__ bool param_valid(const uint32_t* __restrict__ addr, uint32_t n_records, const uint32_t* __restrict__ slots,
                            uint32_t n_slot_words, uint32_t idx, uint64_t required, uint32_t align) {
    // dynamic_parameter_record_is_valid / address_record_is_resident,
    // …gate_up_batch1_mxfp4.comp.template:135-158.
    if (idx >= n_slot_words) return false;
    uint32_t slot = slots[idx];
    if (slot == UNBOUND_SLOT || slot >= n_records) return false;
    const uint32_t* rec = addr + (uint64_t)slot * 8;
    uint64_t address = (uint64_t)rec[0] | ((uint64_t)rec[1] << 32);
    uint64_t bytes = (uint64_t)rec[2] | ((uint64_t)rec[3] << 32);
    return address != 0 && (address & (uint64_t)(align - 1)) == 0 && bytes >= required && (rec[4] | rec[5]) != 0 &&
           rec[6] == 1u;
}

__device__ __forceinline__ const uint8_t* param_ptr(const uint32_t* __restrict__ addr, const uint32_t* __restrict__ slots,
                                                    uint32_t idx) {
    const uint32_t* rec = addr + (uint64_t)slots[idx] * 8;
    return reinterpret_cast<const uint8_t*>((uint64_t)rec[0] | ((uint64_t)rec[1] << 32));
}

__device__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* wave_tot, uint32_t* total) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwave = blockDim.x >> 6;
    uint32_t inc = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        uint32_t t = __shfl_up(inc, d);
        if (lane >= (uint32_t)d) inc += t;
    }
    if (lane == 63) wave_tot[wave] = inc;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t run = 0;
        for (uint32_t w = 0; w < nwave; w++) {
            uint32_t t = wave_tot[w];
            wave_tot[w] = run;
            run += t;
        }
        *total = run;
    }
    __syncthreads();
    uint32_t r = wave_tot[wave] + inc - v;
    __syncthreads();
    return r;
}

struct TileArgs {
    const uint32_t* frames;     // intermediate frames (u32 words)
    uint64_t frame_words;       // k*I/2 + k
    uint32_t data_words;        // k*I/2
    const uint32_t* routes;
    const uint32_t* control;
    uint32_t batch_width, k, E;
    const uint32_t* addr;
    uint32_t n_records;
    const uint32_t* slots;
    uint32_t n_slot_words, P;
    uint64_t req_w, req_s;
    uint32_t TM, max_tiles;
    uint32_t* seg_list;
    uint32_t* tile_expert;
    uint32_t* tile_begin;
    uint32_t* tile_count;
    uint32_t* n_tiles;
};

__global__ __launch_bounds__(1024) void moe_build_tiles_kernel(TileArgs A) {
    __shared__ uint32_t cnt[MAX_EXPERTS];
    __shared__ uint32_t cur[MAX_EXPERTS];
    __shared__ uint32_t tst[MAX_EXPERTS];
    __shared__ uint8_t valid[MAX_EXPERTS];
    __shared__ uint32_t wave_tot[16];
    __shared__ uint32_t total;
    const uint32_t tid = threadIdx.x, nt = blockDim.x;
    for (uint32_t e = tid; e < A.E; e += nt) {
        bool ok = true;
        for (uint32_t p = 0; p < A.P; p++) {
            bool is_weight = (p % 2) == 0;
            ok = ok && param_valid(A.addr, A.n_records, A.slots, A.n_slot_words, e * A.P + p,
                                   is_weight ? A.req_w : A.req_s, is_weight ? 16u : 4u);
        }
        valid[e] = ok ? 1 : 0;
        cnt[e] = 0;
    }
    __syncthreads();
    const uint32_t cap = A.batch_width * A.k;
    uint32_t n = A.control[2] != 0u ? A.control[3] : cap;
    if (n > cap) n = cap;
    for (uint32_t c = tid; c < n; c += nt) {
        uint32_t r = A.frames[(uint64_t)(c / A.k) * A.frame_words + A.data_words + c % A.k];
        if (r >= cap) continue;
        uint32_t e = A.routes[r] & 0xffffu;
        if (e < A.E && valid[e]) atomicAdd(&cnt[e], 1u);
    }
    __syncthreads();
    // Exclusive scans of route counts and tile counts over experts.
    const uint32_t per = (A.E + nt - 1) / nt;
    const uint32_t e0 = min(A.E, tid * per), e1 = min(A.E, e0 + per);
    uint32_t lc = 0, lt = 0;
    for (uint32_t e = e0; e < e1; e++) {
        lc += cnt[e];
        lt += (cnt[e] + A.TM - 1) / A.TM;
    }
    uint32_t oc = block_exclusive_scan(lc, wave_tot, &total);
    uint32_t ot = block_exclusive_scan(lt, wave_tot, &total);
    const uint32_t tiles_total = total;
    for (uint32_t e = e0; e < e1; e++) {
        cur[e] = oc;
        tst[e] = ot;
        oc += cnt[e];
        ot += (cnt[e] + A.TM - 1) / A.TM;
    }
    __syncthreads();
    for (uint32_t e = tid; e < A.E; e += nt) {
        uint32_t nte = (cnt[e] + A.TM - 1) / A.TM;
        for (uint32_t t = 0; t < nte; t++) {
            uint32_t idx = tst[e] + t;
            if (idx < A.max_tiles) {
                A.tile_expert[idx] = e;
                A.tile_begin[idx] = cur[e] + t * A.TM;
                A.tile_count[idx] = min(A.TM, cnt[e] - t * A.TM);
            }
        }
    }
    __syncthreads();
    for (uint32_t c = tid; c < n; c += nt) {
        uint32_t r = A.frames[(uint64_t)(c / A.k) * A.frame_words + A.data_words + c % A.k];
        if (r >= cap) continue;
        uint32_t e = A.routes[r] & 0xffffu;
        if (e < A.E && valid[e]) {
            uint32_t pos = atomicAdd(&cur[e], 1u);
            A.seg_list[pos] = r;
        }
    }
    if (tid == 0) *A.n_tiles = min(tiles_total, A.max_tiles);
}

// ---------------------------------------------------------------------------
// Decode-shaped expert projections: one block = (expert tile of <= 16 routes,
// 64 output rows); wave w owns rows [16w, 16w+16).
// ---------------------------------------------------------------------------
struct ExpertArgs {
    const uint8_t* aq;          // e4m3 activations, row stride K
    const float* as;            // pow2 scales, row stride nblk
    uint32_t a_row_div;         // activation row of route r = r / a_row_div
    uint32_t K, N;              // contraction and output rows of each matrix
    uint32_t k;
    const uint32_t* addr;
    const uint32_t* slots;
    uint32_t P;
    const uint32_t* routes;
    const uint32_t* seg_list;
    const uint32_t* tile_expert;
    const uint32_t* tile_begin;
    const uint32_t* tile_count;
    const uint32_t* n_tiles;
    uint16_t* out;              // gate_up: frames as u16; down: expert_outputs
    uint64_t frame_elems;       // gate_up only
    float limit;
};

__global__ __launch_bounds__(256) void moe_gate_up_kernel(ExpertArgs A) {
    const uint32_t tile = blockIdx.x;
    if (tile >= *A.n_tiles) return;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t g = lane >> 4, rr = lane & 15;
    const uint32_t n0 = blockIdx.y * 64 + wave * 16;
    if (n0 >= A.N) return;
    const uint32_t e = A.tile_expert[tile], begin = A.tile_begin[tile], cnt = A.tile_count[tile];
    const uint32_t K = A.K, nblk = (K + 127) / 128;
    const uint8_t* gw = param_ptr(A.addr, A.slots, e * 4 + 0);
    const uint8_t* gs = param_ptr(A.addr, A.slots, e * 4 + 1);
    const uint8_t* uw = param_ptr(A.addr, A.slots, e * 4 + 2);
    const uint8_t* us = param_ptr(A.addr, A.slots, e * 4 + 3);
    const uint8_t* wrow[2] = {gw + (uint64_t)(n0 + rr) * (K / 2), uw + (uint64_t)(n0 + rr) * (K / 2)};
    const uint8_t* srow[2] = {gs + (uint64_t)(n0 + rr) * (K / 32), us + (uint64_t)(n0 + rr) * (K / 32)};
    const uint8_t* arow = nullptr;
    const float* ascale = A.as;
    if (rr < cnt) {
        uint32_t row = A.seg_list[begin + rr] / A.a_row_div;
        arow = A.aq + (uint64_t)row * K;
        ascale = A.as + (uint64_t)row * nblk;
    }
    v4f acc[2] = {v4f{0.f, 0.f, 0.f, 0.f}, v4f{0.f, 0.f, 0.f, 0.f}};
    mx_tile_loop<2>(arow, ascale, wrow, srow, K, 0, nblk, g, acc);
    // SwiGLU epilogue, …gate_up_batch1_mxfp4.comp.template:776-786.
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t t = 4 * g + i;
        if (t < cnt) {
            uint32_t r = A.seg_list[begin + t];
            uint32_t b = r / A.k, route = r % A.k;
            float gv = round_bf16(acc[0][i]);
            float uv = round_bf16(acc[1][i]);
            if (A.limit > 0.0f) {
                gv = fminf(gv, A.limit);
                uv = fminf(fmaxf(uv, -A.limit), A.limit);
            }
            float h = (gv / (1.0f + expf(-gv))) * uv;
            A.out[(uint64_t)b * A.frame_elems + (uint64_t)route * A.N + n0 + rr] = (uint16_t)f32_to_bf16(h);
        }
    }
}

__global__ __launch_bounds__(256) void moe_down_kernel(ExpertArgs A) {
    const uint32_t tile = blockIdx.x;
    if (tile >= *A.n_tiles) return;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t g = lane >> 4, rr = lane & 15;
    const uint32_t n0 = blockIdx.y * 64 + wave * 16;
    if (n0 >= A.N) return;
    const uint32_t e = A.tile_expert[tile], begin = A.tile_begin[tile], cnt = A.tile_count[tile];
    const uint32_t K = A.K, nblk = (K + 127) / 128;
    const uint8_t* dw = param_ptr(A.addr, A.slots, e * 2 + 0);
    const uint8_t* ds = param_ptr(A.addr, A.slots, e * 2 + 1);
    const uint8_t* wrow[1] = {dw + (uint64_t)(n0 + rr) * (K / 2)};
    const uint8_t* srow[1] = {ds + (uint64_t)(n0 + rr) * (K / 32)};
    const uint8_t* arow = nullptr;
    const float* ascale = A.as;
    if (rr < cnt) {
        uint32_t row = A.seg_list[begin + rr] / A.a_row_div;
        arow = A.aq + (uint64_t)row * K;
        ascale = A.as + (uint64_t)row * nblk;
    }
    v4f acc[1] = {v4f{0.f, 0.f, 0.f, 0.f}};
    mx_tile_loop<1>(arow, ascale, wrow, srow, K, 0, nblk, g, acc);
    // Route weight applied once before the bf16 boundary,
    // …down_batch1_mxfp4.comp.template:588-607.
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t t = 4 * g + i;
        if (t < cnt) {
            uint32_t r = A.seg_list[begin + t];
            float wr = bf16_to_f32(A.routes[r] >> 16);
            A.out[(uint64_t)r * A.N + n0 + rr] = (uint16_t)f32_to_bf16(acc[0][i] * wr);
        }
    }
}


// ---------------------------------------------------------------------------
// Prefill-shaped grouped GEMM: one block = (expert tile of <= 64 routes,
// 128 weight rows).  For gate_up the 128 rows are 64 gate and 64 up rows of
// the same channels; for down they are 128 output rows.  Every 128-k chunk
// of activations (64 x 128 B e4m3) and weights (128 x 64 B e2m1) is staged in
// LDS, double-buffered: the next chunk's global loads are in flight while the
// MFMAs consume the current one.  Wave (wm, wn) of the 2 x 2 wave grid owns
// tokens [32 wm, 32 wm + 32) and a quarter of the weight rows.
// ---------------------------------------------------------------------------
constexpr int GT_M = 64;
constexpr int GT_ROWS = 128;
constexpr int A_STRIDE = 144;   // 128-byte token chunk + 16 bytes of bank padding
constexpr int B_STRIDE = 80;    // 64-byte weight-row chunk + 16 bytes of bank padding

template <int NMAT>
__global__ __launch_bounds__(256) void moe_grouped_kernel(ExpertArgs A) {
    __shared__ __attribute__((aligned(16))) uint8_t lds_a[2][GT_M * A_STRIDE];
    __shared__ __attribute__((aligned(16))) uint8_t lds_b[2][GT_ROWS * B_STRIDE];
    __shared__ uint32_t lds_sb[2][GT_ROWS];
    __shared__ uint32_t lds_sa[2][GT_M];
    __shared__ uint32_t tok_route[GT_M];
    const uint32_t tile = blockIdx.x;
    if (tile >= *A.n_tiles) return;
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t g = lane >> 4, rr = lane & 15;
    const uint32_t e = A.tile_expert[tile], begin = A.tile_begin[tile], cnt = A.tile_count[tile];
    const uint32_t K = A.K, N = A.N, nch = (K + 127) / 128, nblk = nch;
    const uint32_t rows_per_mat = GT_ROWS / NMAT;
    const uint32_t row0 = blockIdx.y * rows_per_mat;
    if (tid < GT_M) tok_route[tid] = tid < cnt ? A.seg_list[begin + tid] : 0xffffffffu;
    __syncthreads();

    // loader roles
    const uint32_t ta = tid >> 2, apart = tid & 3;
    const uint8_t* a_src = nullptr;
    if (ta < cnt) a_src = A.aq + (uint64_t)(tok_route[ta] / A.a_row_div) * K;
    const uint32_t rb = tid >> 1, bhalf = tid & 1;
    const uint32_t mat = rb / rows_per_mat, lrow = rb % rows_per_mat;
    const uint32_t n = row0 + lrow;
    const uint8_t* w_src = nullptr;
    const uint8_t* s_src = nullptr;
    if (n < N) {
        const uint8_t* wbase = param_ptr(A.addr, A.slots, e * A.P + 2 * mat);
        const uint8_t* sbase = param_ptr(A.addr, A.slots, e * A.P + 2 * mat + 1);
        w_src = wbase + (uint64_t)n * (K / 2);
        s_src = sbase + (uint64_t)n * (K / 32);
    }

    v4i ra0, ra1, rb0, rb1;
    uint32_t rsb = 0, rsa = 127;
    auto load = [&](uint32_t c) {
        const uint32_t ka = c * 128 + apart * 32;
        ra0 = v4i{0, 0, 0, 0};
        ra1 = v4i{0, 0, 0, 0};
        if (a_src && ka < K) {
            ra0 = *reinterpret_cast<const v4i*>(a_src + ka);
            ra1 = *reinterpret_cast<const v4i*>(a_src + ka + 16);
        }
        const uint32_t kb = c * 128 + bhalf * 64;
        rb0 = v4i{0, 0, 0, 0};
        rb1 = v4i{0, 0, 0, 0};
        if (w_src && kb < K) {
            rb0 = *reinterpret_cast<const v4i*>(w_src + kb / 2);
            rb1 = *reinterpret_cast<const v4i*>(w_src + kb / 2 + 16);
        }
        if (bhalf == 0) {
            rsb = 0x7f7f7f7fu;
            if (s_src) {
                uint32_t v = 0;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    uint32_t blk = c * 4 + j;
                    v |= (blk * 32 < K ? (uint32_t)s_src[blk] : 127u) << (8 * j);
                }
                rsb = v;
            }
        }
        if (tid < GT_M) rsa = (tid < cnt) ? pow2_to_e8m0(A.as[(uint64_t)(tok_route[tid] / A.a_row_div) * nblk + c]) : 127u;
    };
    auto store = [&](uint32_t buf) {
        uint8_t* pa = &lds_a[buf][ta * A_STRIDE + apart * 32];
        *reinterpret_cast<v4i*>(pa) = ra0;
        *reinterpret_cast<v4i*>(pa + 16) = ra1;
        uint8_t* pb = &lds_b[buf][rb * B_STRIDE + bhalf * 32];
        *reinterpret_cast<v4i*>(pb) = rb0;
        *reinterpret_cast<v4i*>(pb + 16) = rb1;
        if (bhalf == 0) lds_sb[buf][rb] = rsb;
        if (tid < GT_M) lds_sa[buf][tid] = rsa;
    };

    const uint32_t wm = wave >> 1, wn = wave & 1;
    // B sub-tile row bases (LDS rows) of this wave: 4 sub-tiles of 16 rows.
    uint32_t brow[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        if (NMAT == 2) brow[j] = (j >> 1) * 64 + wn * 32 + (j & 1) * 16;   // gate0, gate1, up0, up1
        else brow[j] = wn * 64 + j * 16;
    }
    v4f acc[2][4];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[a][j] = v4f{0.f, 0.f, 0.f, 0.f};

    load(0);
    store(0);
    __syncthreads();
    for (uint32_t c = 0; c < nch; c++) {
        const uint32_t buf = c & 1;
        if (c + 1 < nch) load(c + 1);
        v8i av[2];
        uint32_t sa[2];
#pragma unroll
        for (int a = 0; a < 2; a++) {
            const uint32_t t = wm * 32 + a * 16 + rr;
            const uint8_t* p = &lds_a[buf][t * A_STRIDE + 16 * g];
            v4i lo = *reinterpret_cast<const v4i*>(p);
            v4i hi = *reinterpret_cast<const v4i*>(p + 64);
            av[a] = v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
            sa[a] = lds_sa[buf][t];
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t r = brow[j] + rr;
            v4i w = *reinterpret_cast<const v4i*>(&lds_b[buf][r * B_STRIDE + 16 * g]);
            uint32_t sw = (lds_sb[buf][r] >> (8 * g)) & 0xffu;
#pragma unroll
            for (int a = 0; a < 2; a++) acc[a][j] = mfma_fp8_fp4(av[a], w, sa[a], sw, acc[a][j]);
        }
        if (c + 1 < nch) store(buf ^ 1);
        __syncthreads();
    }

#pragma unroll
    for (int a = 0; a < 2; a++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t t = wm * 32 + a * 16 + 4 * g + i;
            if (t >= cnt) continue;
            const uint32_t r = tok_route[t];
            if (NMAT == 2) {
#pragma unroll
                for (int h2 = 0; h2 < 2; h2++) {
                    const uint32_t ch = row0 + wn * 32 + h2 * 16 + rr;
                    if (ch >= N) continue;
                    float gv = round_bf16(acc[a][h2][i]);
                    float uv = round_bf16(acc[a][2 + h2][i]);
                    if (A.limit > 0.0f) {
                        gv = fminf(gv, A.limit);
                        uv = fminf(fmaxf(uv, -A.limit), A.limit);
                    }
                    float h = (gv / (1.0f + expf(-gv))) * uv;
                    const uint32_t b = r / A.k, route = r % A.k;
                    A.out[(uint64_t)b * A.frame_elems + (uint64_t)route * N + ch] = (uint16_t)f32_to_bf16(h);
                }
            } else {
                const float wr = bf16_to_f32(A.routes[r] >> 16);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t row = row0 + brow[j] + rr;
                    if (row < N) A.out[(uint64_t)r * N + row] = (uint16_t)f32_to_bf16(acc[a][j][i] * wr);
                }
            }
        }
    }
}

nerve_hip_status launch_quant(const uint16_t* x, uint32_t k, uint64_t frame_elems, uint64_t seg_elems, uint32_t cols,
                              uint32_t rows, bool pow2, uint8_t* q, float* s, hipStream_t st) {
    if (rows == 0) return nh::ok();
    const uint32_t nblk = (cols + 127) / 128;
    dim3 grid((nblk + 7) / 8, rows);
    if (pow2)
        quant_rows_kernel<true><<<grid, 256, 0, st>>>(x, k, frame_elems, seg_elems, cols, rows, q, s);
    else
        quant_rows_kernel<false><<<grid, 256, 0, st>>>(x, k, frame_elems, seg_elems, cols, rows, q, s);
    return nh::check_launch("quantize_fp8_e4m3");
}

}  // namespace

namespace nh {
nerve_hip_status quantize_rows(const uint16_t* x, uint32_t cols, uint32_t rows, bool pow2, uint8_t* q, float* s,
                               hipStream_t st) {
    return launch_quant(x, 1, cols, cols, cols, rows, pow2, q, s, st);
}
}  // namespace nh

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" {

nerve_hip_status nerve_hip_quantize_fp8_e4m3(nerve_hip_ctx* ctx, const char* spec, const void* x_bf16, uint32_t rows,
                                             void* q_e4m3, void* scales_f32, void* stream) {
    nerve_hip_status st = nh::enter(ctx);
    if (st) return st;
    nh::QuantSpec qs;
    if ((st = nh::parse_quant_spec(spec, &qs))) return st;
    if (!x_bf16 || !q_e4m3 || !scales_f32) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "null buffer");
    return launch_quant(static_cast<const uint16_t*>(x_bf16), 1, qs.elements, qs.elements, qs.elements, rows, qs.pow2,
                        static_cast<uint8_t*>(q_e4m3), static_cast<float*>(scales_f32), (hipStream_t)stream);
}

nerve_hip_status nerve_hip_mxfp4_gemv(nerve_hip_ctx* ctx, const void* q_e4m3, const void* scales_f32, uint32_t M,
                                      uint32_t K, const void* weight, const void* weight_scale, uint32_t N, void* y_f32,
                                      void* stream) {
    nerve_hip_status st = nh::enter(ctx);
    if (st) return st;
    if (!q_e4m3 || !scales_f32 || !weight || !weight_scale || !y_f32) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "null buffer");
    if (M == 0 || M > 64 || K == 0 || K % 32 || N == 0 || N % 16)
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "mxfp4_gemv needs 1 <= M <= 64, K % 32 == 0, N % 16 == 0");
    if (((uintptr_t)weight & 15) || ((uintptr_t)q_e4m3 & 15))
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "weight and activation buffers must be 16-byte aligned");
    mxfp4_gemv_kernel<8><<<N / 16, 512, 0, (hipStream_t)stream>>>(
        static_cast<const uint8_t*>(q_e4m3), static_cast<const float*>(scales_f32), M, K,
        static_cast<const uint8_t*>(weight), static_cast<const uint8_t*>(weight_scale), N, static_cast<float*>(y_f32));
    return nh::check_launch("mxfp4_gemv");
}

static nerve_hip_status moe_common(nerve_hip_ctx* ctx, const nh::MoeSpec& ms, bool gate_up, const void* act_bf16,
                                   const void* pre_q, const void* pre_s, const void* routes, void* intermediates,
                                   void* expert_outputs, const void* addresses, uint32_t address_records,
                                   const void* slots, uint32_t slot_words, const void* control, uint32_t batch_width,
                                   hipStream_t stream) {
    const uint32_t H = ms.hidden, I = ms.inter, k = ms.k, E = ms.experts;
    const uint32_t cap = batch_width * k;
    if (cap == 0) return nh::ok();
    const uint32_t K = gate_up ? H : I;       // contraction
    const uint32_t N = gate_up ? I : H;       // output rows per matrix
    const uint32_t nblk = (K + 127) / 128;
    const uint32_t arows = gate_up ? batch_width : cap;
    // Decode-shaped batches stream each expert's weights once per <= 16
    // routes; prefill-shaped batches use the LDS-staged grouped GEMM with
    // 64-route tiles.
    const bool grouped = cap >= 512;
    const uint32_t TM = grouped ? 64 : 16;
    const uint32_t max_tiles = (cap + TM - 1) / TM + (E < cap ? E : cap);
    nh::Carver cv;
    size_t o_aq = cv.take<uint8_t>((size_t)arows * K);
    size_t o_as = cv.take<float>((size_t)arows * nblk);
    size_t o_seg = cv.take<uint32_t>(cap);
    size_t o_te = cv.take<uint32_t>(max_tiles);
    size_t o_tb = cv.take<uint32_t>(max_tiles);
    size_t o_tc = cv.take<uint32_t>(max_tiles);
    size_t o_nt = cv.take<uint32_t>(1);
    void* ws = nullptr;
    nerve_hip_status st = nh::workspace(ctx, cv.offset, &ws);
    if (st) return st;
    uint8_t* base = static_cast<uint8_t*>(ws);
    uint8_t* aq = base + o_aq;
    float* as = reinterpret_cast<float*>(base + o_as);
    const uint64_t frame_words = (uint64_t)k * I / 2 + k;
    const uint16_t* frames16 = static_cast<const uint16_t*>(intermediates);

    if (gate_up) {
        if (ms.prequant) {
            aq = const_cast<uint8_t*>(static_cast<const uint8_t*>(pre_q));
            as = const_cast<float*>(static_cast<const float*>(pre_s));
        } else {
            st = launch_quant(static_cast<const uint16_t*>(act_bf16), 1, H, H, H, batch_width, true, aq, as, stream);
            if (st) return st;
        }
    } else {
        // quantize_intermediate (…down_batch1_mxfp4.comp.template:332-353) for every route slice.
        st = launch_quant(frames16, k, frame_words * 2, I, I, cap, true, aq, as, stream);
        if (st) return st;
    }
    TileArgs ta;
    ta.frames = static_cast<const uint32_t*>(intermediates);
    ta.frame_words = frame_words;
    ta.data_words = k * I / 2;
    ta.routes = static_cast<const uint32_t*>(routes);
    ta.control = static_cast<const uint32_t*>(control);
    ta.batch_width = batch_width;
    ta.k = k;
    ta.E = E;
    ta.addr = static_cast<const uint32_t*>(addresses);
    ta.n_records = address_records;
    ta.slots = static_cast<const uint32_t*>(slots);
    ta.n_slot_words = slot_words;
    ta.P = gate_up ? 4 : 2;
    ta.req_w = (uint64_t)N * K / 2;
    ta.req_s = (uint64_t)N * K / 32;
    ta.TM = TM;
    ta.max_tiles = max_tiles;
    ta.seg_list = reinterpret_cast<uint32_t*>(base + o_seg);
    ta.tile_expert = reinterpret_cast<uint32_t*>(base + o_te);
    ta.tile_begin = reinterpret_cast<uint32_t*>(base + o_tb);
    ta.tile_count = reinterpret_cast<uint32_t*>(base + o_tc);
    ta.n_tiles = reinterpret_cast<uint32_t*>(base + o_nt);
    moe_build_tiles_kernel<<<1, 1024, 0, stream>>>(ta);
    if ((st = nh::check_launch("moe_build_tiles"))) return st;

    ExpertArgs ea;
    ea.aq = aq;
    ea.as = as;
    ea.a_row_div = gate_up ? k : 1;
    ea.K = K;
    ea.N = N;
    ea.k = k;
    ea.addr = ta.addr;
    ea.slots = ta.slots;
    ea.P = ta.P;
    ea.routes = ta.routes;
    ea.seg_list = ta.seg_list;
    ea.tile_expert = ta.tile_expert;
    ea.tile_begin = ta.tile_begin;
    ea.tile_count = ta.tile_count;
    ea.n_tiles = ta.n_tiles;
    ea.frame_elems = frame_words * 2;
    ea.limit = ms.limit;
    if (grouped) {
        const uint32_t rows_per_block = gate_up ? 64 : 128;
        dim3 ggrid(max_tiles, (N + rows_per_block - 1) / rows_per_block);
        if (gate_up) {
            ea.out = static_cast<uint16_t*>(intermediates);
            moe_grouped_kernel<2><<<ggrid, 256, 0, stream>>>(ea);
            return nh::check_launch("moe_gate_up_grouped");
        }
        ea.out = static_cast<uint16_t*>(expert_outputs);
        moe_grouped_kernel<1><<<ggrid, 256, 0, stream>>>(ea);
        return nh::check_launch("moe_down_grouped");
    }
    dim3 grid(max_tiles, (N + 63) / 64);
    if (gate_up) {
        ea.out = static_cast<uint16_t*>(intermediates);
        moe_gate_up_kernel<<<grid, 256, 0, stream>>>(ea);
        return nh::check_launch("moe_gate_up");
    }
    ea.out = static_cast<uint16_t*>(expert_outputs);
    moe_down_kernel<<<grid, 256, 0, stream>>>(ea);
    return nh::check_launch("moe_down");
}

nerve_hip_status nerve_hip_mxfp4_moe_gate_up(nerve_hip_ctx* ctx, const char* spec, const void* hidden,
                                             const void* hidden_scales, const void* routes_u32, void* intermediates,
                                             const void* addresses_u32, uint32_t address_records,
                                             const void* param_slots_u32, uint32_t param_slot_words,
                                             const void* control_u32, uint32_t batch_width, void* stream) {
    nerve_hip_status st = nh::enter(ctx);
    if (st) return st;
    nh::MoeSpec ms;
    if ((st = nh::parse_moe_spec(spec, &ms))) return st;
    if (!ms.gate_up) return nh::fail(NERVE_HIP_INVALID_SPEC, "gate_up entry given a down specialization");
    if (!hidden || !routes_u32 || !intermediates || !addresses_u32 || !param_slots_u32 || !control_u32 ||
        (ms.prequant && !hidden_scales))
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "null buffer");
    if (ms.prequant && ((uintptr_t)hidden & 15)) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "prequantized hidden must be 16-byte aligned");
    return moe_common(ctx, ms, true, hidden, hidden, hidden_scales, routes_u32, intermediates, nullptr, addresses_u32,
                      address_records, param_slots_u32, param_slot_words, control_u32, batch_width,
                      (hipStream_t)stream);
}

nerve_hip_status nerve_hip_mxfp4_moe_down(nerve_hip_ctx* ctx, const char* spec, const void* intermediates,
                                          const void* routes_u32, void* expert_outputs, const void* addresses_u32,
                                          uint32_t address_records, const void* param_slots_u32,
                                          uint32_t param_slot_words, const void* control_u32, uint32_t batch_width,
                                          void* stream) {
    nerve_hip_status st = nh::enter(ctx);
    if (st) return st;
    nh::MoeSpec ms;
    if ((st = nh::parse_moe_spec(spec, &ms))) return st;
    if (ms.gate_up) return nh::fail(NERVE_HIP_INVALID_SPEC, "down entry given a gate_up specialization");
    if (!intermediates || !routes_u32 || !expert_outputs || !addresses_u32 || !param_slots_u32 || !control_u32)
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "null buffer");
    return moe_common(ctx, ms, false, nullptr, nullptr, nullptr, routes_u32, const_cast<void*>(intermediates),
                      expert_outputs, addresses_u32, address_records, param_slots_u32, param_slot_words, control_u32,
                      batch_width, (hipStream_t)stream);
}

}  // extern "C"
