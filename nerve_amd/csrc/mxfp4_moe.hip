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
#include <algorithm>
#include <type_traits>
#include <utility>

#include "common.h"
#include "async_copy.h"
#include "quant_dev.h"

namespace {

constexpr uint32_t UNBOUND_SLOT = 0xffffffffu;

// a2 standalone: blockwise e4m3 quantization of bf16 rows (quantize_hidden,
// …gate_up_batch1_mxfp4.comp.template:366-382; quantize_fp8_e4m3.comp.
// template:41-59).  8 clusters of 32 lanes per 256-thread block.
template <bool POW2>
__global__ __launch_bounds__(256) void quant_rows_kernel(QuantArgs Q) {
    if (Q.zero_word && blockIdx.x == 0 && threadIdx.x == 0) *Q.zero_word = 0u;
    quant_unit<POW2>(Q, blockIdx.x * 8 + (threadIdx.x >> 5), threadIdx.x & 31);
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

// Exclusive prefix sums of four per-thread values over the block in thread
// order, with one barrier: each wave scans its lanes, then every thread adds
// the totals of the waves before its own.  `tot` receives the block totals.
// wave_tot must not be rewritten until every thread has returned (the
// caller's next barrier).
__device__ uint4 block_exclusive_scan4(uint4 v, uint4* wave_tot, uint4& tot) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwave = blockDim.x >> 6;
    uint4 inc = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t a = __shfl_up(inc.x, d), b = __shfl_up(inc.y, d), c = __shfl_up(inc.z, d),
                       e = __shfl_up(inc.w, d);
        if (lane >= (uint32_t)d) {
            inc.x += a;
            inc.y += b;
            inc.z += c;
            inc.w += e;
        }
    }
    if (lane == 63) wave_tot[wave] = inc;
    __syncthreads();
    uint4 pre = make_uint4(0, 0, 0, 0), all = make_uint4(0, 0, 0, 0);
    for (uint32_t w = 0; w < nwave; w++) {
        const uint4 t = wave_tot[w];
        if (w < wave) {
            pre.x += t.x;
            pre.y += t.y;
            pre.z += t.z;
            pre.w += t.w;
        }
        all.x += t.x;
        all.y += t.y;
        all.z += t.z;
        all.w += t.w;
    }
    tot = all;
    return make_uint4(pre.x + inc.x - v.x, pre.y + inc.y - v.y, pre.z + inc.z - v.z, pre.w + inc.w - v.w);
}

// One unit of expert work: up to TM routes of one expert, with the expert's
// weight/scale pointers already resolved through the address table, so a
// consuming block needs a single round of independent loads to start
// streaming.
struct TileRec {
    uint32_t expert, begin, count, pad;
    const uint8_t* w[2];
    const uint8_t* s[2];
};

// One work item of the persistent grouped GEMM: row block `rb` of tile
// `tile` (count routes) with its expert's pointers.
struct ItemRec {
    uint32_t rb, count, tile, pad;
    const uint8_t* w[2];
    const uint8_t* s[2];
};

// Route list of one 128-route tile of the persistent grouped GEMM, in the
// order the tile's rows are laid out: route id, activation row and route
// weight.  Entries past the tile's count are never written (they hold
// whatever the workspace held), so readers clamp positions >= count to
// entry 0.  2 KB, so a tile is copied into LDS by two 1 KB wave copies.
constexpr uint32_t PG_TILE = 128;
struct PgList {
    uint32_t route[PG_TILE];
    uint32_t arow[PG_TILE];
    float wr[PG_TILE];
    uint32_t pad[PG_TILE];
};

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
    // Weight representations (…gate_up_batch1_mxfp4.comp.template:173-229):
    // wmode 0 compact MXFP4 only, 1 every MXFP4 expert pre-expanded to e4m3
    // bytes, 2 per expert by address-record word 7 (0 compact, 1 expanded);
    // experts >= native_start are native e4m3 with a 128 x 128 e8m0 grid.
    // req_w8 / req_sn: expanded weight bytes, native scale bytes.
    uint32_t wmode, native_start;
    uint64_t req_w8, req_sn;
    uint32_t TM, max_tiles;
    uint32_t* seg_list;
    TileRec* recs;
    uint32_t* n_tiles;
    ItemRec* items;             // persistent grouped GEMM work items, or null
    PgList* lists;              // its per-tile route lists
    uint32_t item_nrb;          // row blocks per tile for the work items
    uint32_t a_row_div;         // activation row of route r = r / a_row_div
};

// Validity of one parameter from its (already loaded) slot word and address
// record; the same rules as param_valid().
__device__ __forceinline__ bool record_valid(uint32_t slot, uint32_t n_records, const uint32_t (&rec)[8],
                                             uint64_t required, uint32_t align) {
    if (slot == UNBOUND_SLOT || slot >= n_records) return false;
    const uint64_t address = (uint64_t)rec[0] | ((uint64_t)rec[1] << 32);
    const uint64_t bytes = (uint64_t)rec[2] | ((uint64_t)rec[3] << 32);
    return address != 0 && (address & (uint64_t)(align - 1)) == 0 && bytes >= required && (rec[4] | rec[5]) != 0 &&
           rec[6] == 1u;
}

constexpr uint32_t PREP_R = 8;                 // slots per thread whose route ids stay in registers
constexpr uint16_t NO_EXPERT = 0xffffu;
constexpr uint32_t PREP_QU = 4;                // quantization units per 16-lane cluster per pass

// atomicAdd(&cnt[e], 1) for every lane of the wave with e != NO_EXPERT,
// one LDS atomic per distinct expert of the wave (routes come in expert
// order from the compaction, so a wave mostly holds one or two experts and
// the hot experts' counters would otherwise serialize 64-way).  Returns the
// lane's old count plus its rank among the wave's lanes of the same expert.
__device__ __forceinline__ uint32_t wave_add_one(uint32_t* cnt, uint32_t e, bool want_old) {
    const uint32_t lane = threadIdx.x & 63;
    uint64_t todo = __ballot(e != NO_EXPERT);
    uint32_t mine = 0;
    while (todo) {
        const uint32_t leader = (uint32_t)__ffsll((unsigned long long)todo) - 1u;
        const uint32_t el = (uint32_t)__builtin_amdgcn_readlane((int)e, (int)leader);   // leader: wave-uniform
        const uint64_t m = __ballot(e == el);
        uint32_t base = 0;
        if (lane == leader) {
            if (want_old) base = atomicAdd(&cnt[el], (uint32_t)__popcll(m));
            else atomicAdd(&cnt[el], (uint32_t)__popcll(m));
        }
        if (want_old) base = (uint32_t)__builtin_amdgcn_readlane((int)base, (int)leader);
        if (e == el) mine = base + (uint32_t)__popcll(m & ((1ull << lane) - 1ull));
        todo &= ~m;
    }
    return mine;
}


// Latency matters here (decode runs this once per projection), so the block
// needs only two rounds of dependent global loads: (1) slot words of every
// expert's parameters, the compacted route map entries and the control
// words; (2) the address records and the route words.  Everything after that
// is LDS work; a thread keeps its first expert's resolved pointers in
// registers for the tile records.
template <uint32_t MAXE>
__device__ void build_tiles(const TileArgs& A) {
    __shared__ uint32_t cnt[MAXE];
    __shared__ uint32_t cur[MAXE];
    __shared__ uint32_t tst[MAXE];
    __shared__ uint32_t est[MAXE];
    __shared__ uint8_t valid[MAXE];
    __shared__ uint32_t gst[MAXE];
    __shared__ uint4 wave_tot4[16];
    // Expert pointers (w0, s0, w1, s1) for the work-item expansion, when
    // every expert has its own thread.
    constexpr bool EPTR = MAXE <= 1024;
    __shared__ const uint8_t* eptr[EPTR ? MAXE : 1][4];
    const uint32_t tid = threadIdx.x, nt = blockDim.x;
    const uint32_t cap = A.batch_width * A.k;
    const uint32_t P = A.P;   // 4 (gate, gate scales, up, up scales) or 2 (down, down scales)

    // ---- round 1: slot words of expert tid, route map entry tid, control
    // Every load of the two rounds is issued unconditionally (from a clamped
    // index, its value discarded where it does not apply): a load under a
    // lane condition makes the compiler wait for all loads in flight at the
    // branch's end, which turned the rounds into a dozen round trips.
    uint32_t slot[4] = {UNBOUND_SLOT, UNBOUND_SLOT, UNBOUND_SLOT, UNBOUND_SLOT};
    if (A.n_slot_words != 0) {
#pragma unroll
        for (uint32_t p = 0; p < 4; p++) {
            const uint32_t idx = tid * P + p;
            const uint32_t v = A.slots[min(idx, A.n_slot_words - 1)];
            if (tid < A.E && p < P && idx < A.n_slot_words) slot[p] = v;
        }
    }
    // Slots c = tid + i nt for i < PREP_R keep their route index and route
    // word in registers, loaded in these two rounds.  (Slots beyond PREP_R nt
    // take a plain loop.)
    uint32_t rw_r[PREP_R], rt_r[PREP_R];
#pragma unroll
    for (uint32_t i = 0; i < PREP_R; i++) {
        const uint32_t c = tid + i * nt;
        const uint32_t cc = c < cap ? c : 0u;
        const uint32_t v = A.frames[(uint64_t)(cc / A.k) * A.frame_words + A.data_words + cc % A.k];
        rw_r[i] = c < cap ? v : 0xffffffffu;
    }
    const uint32_t rword = rw_r[0];
    const uint32_t c2 = A.control[2], c3 = A.control[3];
    // ---- round 2: address records, route word
    uint32_t rec[4][8] = {};
    if (A.n_records != 0) {
#pragma unroll
        for (uint32_t p = 0; p < 4; p++) {
            const bool has = slot[p] != UNBOUND_SLOT && slot[p] < A.n_records;
            const v4i* r4 = reinterpret_cast<const v4i*>(A.addr + (uint64_t)(has ? slot[p] : 0u) * 8);
            const v4i lo = r4[0], hi = r4[1];
            const uint32_t w8[8] = {(uint32_t)lo.x, (uint32_t)lo.y, (uint32_t)lo.z, (uint32_t)lo.w,
                                    (uint32_t)hi.x, (uint32_t)hi.y, (uint32_t)hi.z, (uint32_t)hi.w};
#pragma unroll
            for (uint32_t j = 0; j < 8; j++) rec[p][j] = has ? w8[j] : 0u;
        }
    }
    uint32_t rv[PREP_R];
#pragma unroll
    for (uint32_t i = 0; i < PREP_R; i++) rv[i] = A.routes[rw_r[i] < cap ? rw_r[i] : 0u];
#pragma unroll
    for (uint32_t i = 0; i < PREP_R; i++) {
        const uint32_t c = tid + i * nt;
        rt_r[i] = (c < cap && rw_r[i] < cap) ? rv[i] : 0u;
    }
    const uint32_t route = rt_r[0];

    uint32_t n = c2 != 0u ? c3 : cap;
    if (n > cap) n = cap;
    const uint8_t* my_w[2] = {nullptr, nullptr};
    const uint8_t* my_s[2] = {nullptr, nullptr};
    uint32_t my_fmt = 0;
    if (tid < A.E) {
        bool ok = true;
        // Format of this expert: 0 compact, 1 expanded, 2 native e4m3
        // (dynamic_expert_is_valid, …gate_up_batch1_mxfp4.comp.template:190-229).
        const bool native = tid >= A.native_start;
        const uint32_t repr0 = rec[0][7], repr2 = P > 2 ? rec[2][7] : repr0;
        const bool pre0 = !native && (A.wmode == 1 || (A.wmode == 2 && repr0 == 1u));
        const bool pre2 = !native && (A.wmode == 1 || (A.wmode == 2 && repr2 == 1u));
        if (native) ok = repr0 == 0u && repr2 == 0u;
        else if (A.wmode == 2) ok = repr0 <= 1u && repr2 <= 1u && pre0 == pre2;
        my_fmt = native ? 2u : pre0 ? 1u : 0u;
        const uint64_t rw = my_fmt ? A.req_w8 : A.req_w, rs = native ? A.req_sn : A.req_s;
#pragma unroll
        for (uint32_t p = 0; p < 4; p++) {
            if (p >= P) continue;
            const bool is_weight = (p % 2) == 0;
            ok = record_valid(slot[p], A.n_records, rec[p], is_weight ? rw : rs, is_weight ? 16u : native ? 1u : 4u) && ok;
        }
        valid[tid] = ok ? 1 : 0;
        cnt[tid] = 0;
#pragma unroll
        for (uint32_t m = 0; m < 2; m++) {
            if (2 * m >= P) continue;
            my_w[m] = reinterpret_cast<const uint8_t*>((uint64_t)rec[2 * m][0] | ((uint64_t)rec[2 * m][1] << 32));
            my_s[m] = reinterpret_cast<const uint8_t*>((uint64_t)rec[2 * m + 1][0] | ((uint64_t)rec[2 * m + 1][1] << 32));
        }
        if constexpr (EPTR) {
            eptr[tid][0] = my_w[0];
            eptr[tid][1] = my_s[0];
            eptr[tid][2] = my_w[1];
            eptr[tid][3] = my_s[1];
        }
    }
    // Experts beyond the block size (E > 1024) take the plain path (compact
    // MXFP4 only: the host sends the other representations here only with
    // E <= the block size).
    for (uint32_t e = tid + nt; e < A.E; e += nt) {
        bool ok = true;
        for (uint32_t p = 0; p < P; p++) {
            const bool is_weight = (p % 2) == 0;
            ok = param_valid(A.addr, A.n_records, A.slots, A.n_slot_words, e * P + p, is_weight ? A.req_w : A.req_s,
                             is_weight ? 16u : 4u) && ok;
        }
        valid[e] = ok ? 1 : 0;
        cnt[e] = 0;
    }
    __syncthreads();
    // Expert of every compacted slot c < n (NO_EXPERT when invalid).
    auto slot_expert = [&](uint32_t c, uint32_t rw, uint32_t rt) -> uint32_t {
        if (c >= n || rw >= cap) return NO_EXPERT;
        const uint32_t e = rt & 0xffffu;
        return (e < A.E && valid[e]) ? e : NO_EXPERT;
    };
    wave_add_one(cnt, tid < cap ? slot_expert(tid, rword, route) : NO_EXPERT, false);
#pragma unroll
    for (uint32_t i = 1; i < PREP_R; i++) {
        const uint32_t c = tid + i * nt;
        if (c - tid >= cap) break;   // uniform: no lane of the block has slots this far
        wave_add_one(cnt, c < cap ? slot_expert(c, rw_r[i], rt_r[i]) : NO_EXPERT, false);
    }
    for (uint32_t c0 = PREP_R * nt; c0 < cap; c0 += nt) {
        const uint32_t c = c0 + tid;
        uint32_t e = NO_EXPERT;
        if (c < cap) {
            const uint32_t rw = A.frames[(uint64_t)(c / A.k) * A.frame_words + A.data_words + c % A.k];
            e = slot_expert(c, rw, rw < cap ? A.routes[rw] : 0u);
        }
        wave_add_one(cnt, e, false);
    }
    __syncthreads();
    // Exclusive scans over experts, in one pass: route counts, tile counts,
    // and the tiles of the route-count groups of the persistent grouped GEMM
    // (experts with more than 64 routes, 33-64, then 1-32: it contracts 128,
    // 64 or 32 routes per tile for them) -- the first two packed as 16-bit
    // halves.
    auto group_of = [](uint32_t c) -> uint32_t { return c > 64 ? 0u : c > 32 ? 1u : 2u; };
    const uint32_t per = (A.E + nt - 1) / nt;
    const uint32_t e0 = min(A.E, tid * per), e1 = min(A.E, e0 + per);
    uint4 lv = make_uint4(0, 0, 0, 0);
    for (uint32_t e = e0; e < e1; e++) {
        const uint32_t nte = (cnt[e] + A.TM - 1) / A.TM, gr = group_of(cnt[e]);
        lv.x += cnt[e];
        lv.y += nte;
        if (gr == 0) lv.z += nte;
        else if (gr == 1) lv.z += nte << 16;
        else lv.w += nte;
    }
    uint4 tot;
    uint4 o = block_exclusive_scan4(lv, wave_tot4, tot);
    const uint32_t tiles_total = tot.y;
    const uint32_t nt0 = tot.z & 0xffffu, nt1 = tot.z >> 16;
    for (uint32_t e = e0; e < e1; e++) {
        const uint32_t nte = (cnt[e] + A.TM - 1) / A.TM, gr = group_of(cnt[e]);
        cur[e] = o.x;
        est[e] = o.x;
        tst[e] = o.y;
        // first tile of expert e among its group's tiles
        gst[e] = gr == 0 ? (o.z & 0xffffu) : gr == 1 ? (o.z >> 16) : o.w;
        o.x += cnt[e];
        o.y += nte;
        if (gr == 0) o.z += nte;
        else if (gr == 1) o.z += nte << 16;
        else o.w += nte;
    }
    __syncthreads();
    // From here on every phase only writes global memory (and the route
    // counters in cur[]), so the phases run without barriers between them.
    for (uint32_t e = tid; e < A.E; e += nt) {
        const uint32_t nte = (cnt[e] + A.TM - 1) / A.TM;
        for (uint32_t t = 0; t < nte; t++) {
            const uint32_t idx = tst[e] + t;
            if (idx < A.max_tiles) {
                TileRec rec_out;
                // Bits 16-17: the expert's weight format (known to its own
                // thread; experts past the block size are compact).
                rec_out.expert = e | ((e == tid ? my_fmt : 0u) << 16);
                rec_out.begin = est[e] + t * A.TM;
                rec_out.count = min(A.TM, cnt[e] - t * A.TM);
                rec_out.pad = (t << 16) | nte;   // tile index within the expert, expert's tile count
                for (uint32_t m = 0; m < 2; m++) {
                    const bool has = 2 * m < P;
                    if (e == tid) {
                        rec_out.w[m] = my_w[m];
                        rec_out.s[m] = my_s[m];
                    } else {
                        rec_out.w[m] = has ? param_ptr(A.addr, A.slots, e * P + 2 * m) : nullptr;
                        rec_out.s[m] = has ? param_ptr(A.addr, A.slots, e * P + 2 * m + 1) : nullptr;
                    }
                }
                A.recs[idx] = rec_out;
            }
        }
    }
    // Route slots in expert order.  For the persistent grouped GEMM the slot
    // also goes into its tile's route list (position rank % TM of tile
    // tst[e] + rank / TM), with its activation row and route weight.
    // Called by every lane of the wave (e = NO_EXPERT places nothing).
    auto place = [&](uint32_t e, uint32_t r, uint32_t rt) {
        const uint32_t pos = wave_add_one(cur, e, true);
        if (e == NO_EXPERT) return;
        A.seg_list[pos] = r;
        if (A.lists) {
            const uint32_t rank = pos - est[e], t = tst[e] + rank / A.TM, j = rank % A.TM;
            if (t < A.max_tiles) {
                PgList& L = A.lists[t];
                L.route[j] = r;
                L.arow[j] = r / A.a_row_div;
                L.wr[j] = bf16_to_f32(rt >> 16);
            }
        }
    };
#pragma unroll
    for (uint32_t i = 0; i < PREP_R; i++) {
        const uint32_t c = tid + i * nt;
        if (c - tid >= n) break;     // uniform
        place(c < n ? slot_expert(c, rw_r[i], rt_r[i]) : NO_EXPERT, rw_r[i], rt_r[i]);
    }
    for (uint32_t c0 = PREP_R * nt; c0 < n; c0 += nt) {
        const uint32_t c = c0 + tid;
        uint32_t r = 0, rt = 0, e = NO_EXPERT;
        if (c < n) {
            r = A.frames[(uint64_t)(c / A.k) * A.frame_words + A.data_words + c % A.k];
            rt = r < cap ? A.routes[r] : 0u;
            e = slot_expert(c, r, rt);
        }
        place(e, r, rt);
    }
    if (tid == 0) *A.n_tiles = min(tiles_total, A.max_tiles);
    if (A.items) {
        // Work items (expert, row block, tile) with tiles fastest, grouped by
        // the expert's route count (gst[]: the expert's first tile among its
        // group's tiles); n_tiles[1], n_tiles[2] the first two groups' tile
        // counts.
        if (tid == 0) {
            A.n_tiles[1] = nt0;
            A.n_tiles[2] = nt1;
        }
        // Without per-expert pointers in LDS the items copy them from the
        // tile records: wait until every record is written.
        if constexpr (!EPTR) __syncthreads();
        // One thread per (expert, row block): its tiles' items.
        const uint32_t nrb = A.item_nrb;
        for (uint32_t pr = tid; pr < A.E * nrb; pr += nt) {
            const uint32_t e = pr / nrb, rb = pr % nrb;
            const uint32_t nte = (cnt[e] + A.TM - 1) / A.TM;
            if (nte == 0) continue;
            const uint32_t gr = group_of(cnt[e]);
            const uint32_t gbase = gr == 0 ? 0u : gr == 1 ? nt0 * nrb : (nt0 + nt1) * nrb;
            const uint32_t base = gbase + gst[e] * nrb + rb * nte;
            for (uint32_t kk = 0; kk < nte; kk++) {
                const uint32_t t = tst[e] + kk;
                ItemRec o;
                o.rb = rb;
                o.count = min(A.TM, cnt[e] - kk * A.TM);
                o.tile = t;
                o.pad = 0;
                if constexpr (EPTR) {
                    o.w[0] = eptr[e][0];
                    o.s[0] = eptr[e][1];
                    o.w[1] = eptr[e][2];
                    o.s[1] = eptr[e][3];
                } else {
                    o.w[0] = A.recs[t].w[0];
                    o.w[1] = A.recs[t].w[1];
                    o.s[0] = A.recs[t].s[0];
                    o.s[1] = A.recs[t].s[1];
                }
                A.items[base + kk] = o;
            }
        }
    }
}

// Preparation launch of one MoE projection: block 0 turns the route map into
// tile records while the other blocks quantize the activation rows (32
// (row, 128-column) units per block).
template <uint32_t MAXE>
__global__ __launch_bounds__(1024) void moe_prep_kernel(TileArgs T, QuantArgs Q) {
    if (blockIdx.x == 0) {
        build_tiles<MAXE>(T);
        return;
    }
    // Quantization blocks stride over the (row, 128-column) units, 64 per
    // pass with 16-byte loads (32 per pass otherwise).
    const uint64_t nblk = (Q.cols + 127) / 128, units = (uint64_t)Q.rows * nblk;
    if (Q.vec8) {
        for (uint64_t u = (uint64_t)(blockIdx.x - 1) * 64 * PREP_QU; u < units; u += (uint64_t)(gridDim.x - 1) * 64 * PREP_QU)
            quant_units8_pow2<PREP_QU>(Q, u + (threadIdx.x >> 4), 64, threadIdx.x & 15);
        return;
    }
    for (uint64_t u = (uint64_t)(blockIdx.x - 1) * 32; u < units; u += (uint64_t)(gridDim.x - 1) * 32)
        quant_unit<true>(Q, (uint32_t)u + (threadIdx.x >> 5), threadIdx.x & 31);
}

// ---------------------------------------------------------------------------
// Arguments shared by the grouped (prefill-shaped) kernels.
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
    const TileRec* recs;
    const uint32_t* n_tiles;
    uint32_t max_tiles;         // tile slots in the grid
    uint32_t work_items;        // max_tiles x row blocks (grouped kernels)
    uint16_t* out;              // gate_up: frames as u16; down: expert_outputs
    uint64_t frame_elems;       // gate_up only
    float limit;
};

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
    const uint32_t n_tiles = *A.n_tiles;
    const TileRec rec = A.recs[tile];
    if (tile >= n_tiles) return;
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t g = lane >> 4, rr = lane & 15;
    const uint32_t begin = rec.begin, cnt = rec.count;
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
        w_src = rec.w[mat] + (uint64_t)n * (K / 2);
        s_src = rec.s[mat] + (uint64_t)n * (K / 32);
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


// ---------------------------------------------------------------------------
// Grouped GEMM with an asynchronous LDS pipeline.  Same tile as
// moe_grouped_kernel (64 routes x 128 weight rows, 2 x 2 waves), but every
// chunk is copied global -> LDS with global_load_lds_dwordx4 (no register
// staging) into a ring of GS_STAGES buffers, so GS_STAGES - 1 chunks are in
// flight while one is consumed.  The block's e8m0 weight scales and the
// activation block scales are staged in LDS once per tile.  Rows are stored
// with an XOR swizzle of their 16-byte pieces so the MFMA operand reads
// spread over the LDS banks: 16 lanes reading one operand touch 16
// distinct 16-byte bank groups.  Synchronization is s_barrier plus explicit
// vmcnt waits (a fenced __syncthreads would drain the pipeline).
// ---------------------------------------------------------------------------
constexpr uint32_t GS_MAX_K = 4096;

__device__ __attribute__((aligned(16))) const uint8_t kZero16[16] = {0};


__device__ __forceinline__ void lds_wait(v4i& a0, v4i& a1, v4i& a2, v4i& a3, v4i& b0, v4i& b1, v4i& b2, v4i& b3) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3), "+v"(b0), "+v"(b1), "+v"(b2), "+v"(b3));
}

template <int NMAT>
__global__ __launch_bounds__(256) void moe_grouped_async_kernel(ExpertArgs A) {
    // One LDS object per pipeline stage: the compiler tracks asynchronous LDS
    // writes per object, so reads of the current stage wait only for the
    // copies into that stage.
    __shared__ __attribute__((aligned(16))) uint8_t st_a0[GT_M * 128];
    __shared__ __attribute__((aligned(16))) uint8_t st_a1[GT_M * 128];
    __shared__ __attribute__((aligned(16))) uint8_t st_a2[GT_M * 128];
    __shared__ __attribute__((aligned(16))) uint8_t st_b0[GT_ROWS * 64];
    __shared__ __attribute__((aligned(16))) uint8_t st_b1[GT_ROWS * 64];
    __shared__ __attribute__((aligned(16))) uint8_t st_b2[GT_ROWS * 64];
    __shared__ uint8_t sc_b[GT_ROWS * (GS_MAX_K / 32)];
    __shared__ uint8_t sc_a[GT_M * (GS_MAX_K / 128)];
    __shared__ uint32_t tok_route[GT_M];
    // XCD-aware work order: the hardware deals consecutive workgroups to the
    // 8 XCDs in turn; remap so that each XCD walks a contiguous range of
    // (tile, row-block) work with tiles fastest.  Tiles of one expert at one
    // row block then run back to back on one XCD and share its L2 copy of
    // the weight rows.
    const uint32_t per_xcd = gridDim.x / 8;   // the grid is a multiple of 8
    const uint32_t w = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (w >= A.work_items) return;
    const uint32_t tile = w % A.max_tiles;
    const uint32_t n_tiles = *A.n_tiles;
    const TileRec rec = A.recs[tile];
    if (tile >= n_tiles) return;
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t g = lane >> 4, rr = lane & 15;
    const uint32_t begin = rec.begin, cnt = rec.count;
    const uint32_t K = A.K, N = A.N, nch = (K + 127) / 128, nmx = K / 32;
    const uint32_t rows_per_mat = GT_ROWS / NMAT;
    const uint32_t row0 = (w / A.max_tiles) * rows_per_mat;
    if (tid < GT_M) tok_route[tid] = tid < cnt ? A.seg_list[begin + tid] : 0xffffffffu;
    __syncthreads();

    const uint8_t* wbase[NMAT];
    const uint8_t* sbase[NMAT];
#pragma unroll
    for (int m = 0; m < NMAT; m++) {
        wbase[m] = rec.w[m];
        sbase[m] = rec.s[m];
    }
    // Stage all scales of the tile.
    for (uint32_t i = tid; i < GT_ROWS * nmx; i += blockDim.x) {
        const uint32_t r = i / nmx, b = i % nmx;
        const uint32_t m = r / rows_per_mat, n = row0 + r % rows_per_mat;
        sc_b[r * nmx + b] = n < N ? sbase[m][(uint64_t)n * nmx + b] : 127;
    }
    for (uint32_t i = tid; i < GT_M * nch; i += blockDim.x) {
        const uint32_t t = i / nch, c = i % nch;
        sc_a[t * nch + c] =
            t < cnt ? (uint8_t)pow2_to_e8m0(A.as[(uint64_t)(tok_route[t] / A.a_row_div) * nch + c]) : 127;
    }

    // Per-lane source rows of the two A and two B copy instructions.  Copy
    // instruction q of a stage fills LDS bytes [q*1024, q*1024+1024): for A
    // the 128-byte chunks of tokens 8q..8q+7, for B the 64-byte chunks of
    // rows 16q..16q+15, each lane one 16-byte piece (XOR-swizzled slot).
    const uint8_t* a_row[2];
    uint32_t a_piece[2];
    const uint8_t* b_row[2];
    uint32_t b_piece[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const uint32_t q = wave * 2 + j;
        const uint32_t t = 8 * q + (lane >> 3);
        const uint32_t tt = t < cnt ? t : 0;
        a_row[j] = A.aq + (uint64_t)(tok_route[tt] / A.a_row_div) * K;
        a_piece[j] = (lane & 7) ^ ((t ^ (t >> 3)) & 7);
        const uint32_t r = 16 * q + (lane >> 2);
        const uint32_t m = r / rows_per_mat, n = row0 + r % rows_per_mat;
        b_row[j] = wbase[m] + (uint64_t)(n < N ? n : 0) * (K / 2);
        b_piece[j] = (lane & 3) ^ ((r ^ (r >> 2)) & 3);
    }
    auto issue = [&](uint32_t c, uint8_t* sa, uint8_t* sb) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint32_t q = wave * 2 + j;
            const uint32_t ka = c * 128 + a_piece[j] * 16;
            const uint8_t* src = ka < K ? a_row[j] + ka : kZero16;
            __builtin_amdgcn_global_load_lds(src, sa + q * 1024, 16, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint32_t q = wave * 2 + j;
            const uint32_t kb = c * 128 + b_piece[j] * 32;
            const uint8_t* src = kb < K ? b_row[j] + kb / 2 : kZero16;
            __builtin_amdgcn_global_load_lds(src, sb + q * 1024, 16, 0, 0);
        }
    };

    const uint32_t wm = wave >> 1, wn = wave & 1;
    uint32_t brow[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        if (NMAT == 2) brow[j] = (j >> 1) * 64 + wn * 32 + (j & 1) * 16;
        else brow[j] = wn * 64 + j * 16;
    }
    v4f acc[2][4];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[a][j] = v4f{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](uint32_t c, const uint8_t* sa_lds, const uint8_t* sb_lds) {
        const uint32_t t0 = wm * 32 + rr, t1 = t0 + 16;
        const uint32_t f0 = (t0 ^ (t0 >> 3)) & 7, f1 = (t1 ^ (t1 >> 3)) & 7;
        v4i lo0 = lds_read16(sa_lds + t0 * 128 + ((g ^ f0) * 16));
        v4i hi0 = lds_read16(sa_lds + t0 * 128 + (((g + 4) ^ f0) * 16));
        v4i lo1 = lds_read16(sa_lds + t1 * 128 + ((g ^ f1) * 16));
        v4i hi1 = lds_read16(sa_lds + t1 * 128 + (((g + 4) ^ f1) * 16));
        v4i w[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t r = brow[j] + rr;
            w[j] = lds_read16(sb_lds + r * 64 + ((g ^ ((r ^ (r >> 2)) & 3)) * 16));
        }
        lds_wait(lo0, hi0, lo1, hi1, w[0], w[1], w[2], w[3]);
        const v8i av[2] = {v8i{lo0.x, lo0.y, lo0.z, lo0.w, hi0.x, hi0.y, hi0.z, hi0.w},
                           v8i{lo1.x, lo1.y, lo1.z, lo1.w, hi1.x, hi1.y, hi1.z, hi1.w}};
        const uint32_t sa[2] = {sc_a[t0 * nch + c], sc_a[t1 * nch + c]};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t r = brow[j] + rr;
            const uint32_t blk = c * 4 + g;
            uint32_t sw = blk < nmx ? sc_b[r * nmx + blk] : 127u;
#pragma unroll
            for (int a = 0; a < 2; a++) acc[a][j] = mfma_fp8_fp4(av[a], w[j], sa[a], sw, acc[a][j]);
        }
    };
    // One pipeline step: refill the stage freed last step with chunk c + 2,
    // wait for chunk c, consume it.
    auto step = [&](uint32_t c, const uint8_t* ca, const uint8_t* cb, uint8_t* na, uint8_t* nb) {
        __builtin_amdgcn_s_barrier();
        if (c + 2 < nch) {
            issue(c + 2, na, nb);
            wait_vm(8);
        } else if (c + 1 < nch) {
            wait_vm(4);
        } else {
            wait_vm(0);
        }
        __builtin_amdgcn_s_barrier();
        compute(c, ca, cb);
    };

    __syncthreads();  // scales staged; nothing asynchronous is in flight yet
    issue(0, st_a0, st_b0);
    if (1 < nch) issue(1, st_a1, st_b1);
    for (uint32_t c = 0; c < nch; c += 3) {
        step(c, st_a0, st_b0, st_a2, st_b2);
        if (c + 1 < nch) step(c + 1, st_a1, st_b1, st_a0, st_b0);
        if (c + 2 < nch) step(c + 2, st_a2, st_b2, st_a1, st_b1);
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


// ---------------------------------------------------------------------------
// Span-streaming expert GEMV (decode-shaped batches and the raw GEMV).
//
// A block owns 16*NSUB consecutive rows of NMAT weight matrices of one expert
// and <= 16 routes.  Those rows are contiguous in the package layout
// ([rows, K/2] bytes), so the block copies each matrix's row span and its
// e8m0 scale span straight into LDS with global_load_lds (1 KB per wave
// instruction, all issued up front), while each lane also prefetches its
// activation operands.  DRAM therefore sees long sequential runs instead of
// one 64-byte stream per weight row.  After a single wait the NWS waves split
// the K chunks, contract from LDS on the scaled MFMA, and reduce through LDS.
// ---------------------------------------------------------------------------
enum SpanMode { SPAN_RAW = 0, SPAN_GATE_UP = 1, SPAN_DOWN = 2 };
constexpr uint32_t SPAN_MAX_CHUNKS_PER_WAVE = 8;   // K <= 4096

struct SpanArgs {
    const uint8_t* aq;
    const float* as;
    uint32_t a_row_div;
    uint32_t K, N, k, M;
    const uint8_t* w_direct;    // raw mode
    const uint8_t* s_direct;
    const uint32_t* addr;
    const uint32_t* slots;
    uint32_t P;
    const uint32_t* routes;
    const uint32_t* seg_list;
    const TileRec* recs;
    const uint32_t* n_tiles;
    uint16_t* out16;
    float* out32;
    uint64_t frame_elems;
    float limit;
    uint32_t w_region, s_region;   // LDS bytes per matrix (padded)
    uint32_t block_major;          // mx_wfmt_kernel: compact weights in the input-block-major layout
    uint32_t rpb;                  // mx_span_kernel: weight rows per block (<= 16 NSUB; 0: 16 NSUB)
};

__host__ __device__ inline uint32_t span_w_region(uint32_t rows, uint32_t K) { return (rows * (K / 2) + 1023) / 1024 * 1024; }
__host__ __device__ inline uint32_t span_s_region(uint32_t rows, uint32_t K) { return (rows * (K / 32) + 255) / 256 * 256; }

template <int MODE, int NMAT, int NSUB, int NWS = 4>
__global__ __launch_bounds__(64 * NWS) void mx_span_kernel(SpanArgs A) {
    extern __shared__ __attribute__((aligned(16))) uint8_t span_lds[];
    constexpr uint32_t R = 16 * NSUB;
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t g = lane >> 4, rr = lane & 15;
    const uint32_t K = A.K, N = A.N, RB = K / 2, SB = K / 32, nch = (K + 127) / 128;
    const uint32_t rpb = A.rpb ? A.rpb : R;
    const uint32_t n0 = blockIdx.x * rpb;
    if (n0 >= N) return;
    const uint32_t rows = min(rpb, N - n0);   // rows of this block (the subtiles past them are not stored)
    uint32_t cnt, begin = 0;
    TileRec rec;
    if (MODE == SPAN_RAW) {
        cnt = min(16u, A.M - blockIdx.y * 16);
        rec.w[0] = A.w_direct;
        rec.s[0] = A.s_direct;
        rec.w[1] = rec.s[1] = nullptr;
    } else {
        const uint32_t tile = blockIdx.y;
        const uint32_t n_tiles = *A.n_tiles;   // independent of the record load
        rec = A.recs[tile];
        if (tile >= n_tiles) return;
        begin = rec.begin;
        cnt = rec.count;
    }
    // ---- asynchronous copies of the weight and scale spans
#pragma unroll
    for (int m = 0; m < NMAT; m++) {
        const uint8_t* wb = rec.w[m];
        const uint8_t* sb = rec.s[m];
        const uint8_t* wsrc = wb + (uint64_t)n0 * RB;
        const uint32_t wbytes = rows * RB;
        uint8_t* wdst = span_lds + m * A.w_region;
        for (uint32_t pc = wave; pc * 1024 < wbytes; pc += NWS) {
            uint32_t off = pc * 1024 + lane * 16;
            __builtin_amdgcn_global_load_lds(wsrc + (off < wbytes ? off : 0), wdst + pc * 1024, 16, 0, 0);
        }
        const uint8_t* ssrc = sb + (uint64_t)n0 * SB;
        const uint32_t sbytes = rows * SB;
        uint8_t* sdst = span_lds + NMAT * A.w_region + m * A.s_region;
        for (uint32_t pc = wave; pc * 256 < sbytes; pc += NWS) {
            uint32_t off = pc * 256 + lane * 4;
            __builtin_amdgcn_global_load_lds(ssrc + (off < sbytes ? off : 0), sdst + pc * 256, 4, 0, 0);
        }
    }
    // ---- activation operands of this wave's chunks, prefetched to registers
    const uint32_t per = (nch + NWS - 1) / NWS;
    const uint32_t c0 = min(nch, wave * per), c1 = min(nch, c0 + per);
    const uint8_t* arow = nullptr;
    const float* ascale = nullptr;
    if (rr < cnt) {
        uint32_t row;
        if (MODE == SPAN_RAW) row = blockIdx.y * 16 + rr;
        else row = A.seg_list[begin + rr] / A.a_row_div;
        arow = A.aq + (uint64_t)row * K;
        ascale = A.as + (uint64_t)row * nch;
    }
    v8i av[SPAN_MAX_CHUNKS_PER_WAVE];
    uint32_t sa[SPAN_MAX_CHUNKS_PER_WAVE];
#pragma unroll
    for (uint32_t i = 0; i < SPAN_MAX_CHUNKS_PER_WAVE; i++) {
        if (c0 + i < c1) load_a(arow, ascale, K, c0 + i, g, av[i], sa[i]);
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): spans and operands have landed
    __syncthreads();

    v4f acc[NMAT][NSUB];
#pragma unroll
    for (int m = 0; m < NMAT; m++)
#pragma unroll
        for (int j = 0; j < NSUB; j++) acc[m][j] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (uint32_t i = 0; i < SPAN_MAX_CHUNKS_PER_WAVE; i++) {
        const uint32_t c = c0 + i;
        if (c >= c1) break;
        const uint32_t kb = c * 128 + g * 32;
        const bool kv = kb < K;
#pragma unroll
        for (int m = 0; m < NMAT; m++) {
#pragma unroll
            for (int j = 0; j < NSUB; j++) {
                const uint32_t row = j * 16 + rr;
                v4i w = v4i{0, 0, 0, 0};
                uint32_t sw = 127;
                if (kv) {
                    w = *reinterpret_cast<const v4i*>(span_lds + m * A.w_region + row * RB + kb / 2);
                    sw = span_lds[NMAT * A.w_region + m * A.s_region + row * SB + kb / 32];
                }
                acc[m][j] = mfma_fp8_fp4(av[i], w, sa[i], sw, acc[m][j]);
            }
        }
    }
    // ---- cross-wave reduction through LDS (the span region is free now)
    __syncthreads();
    v4f* red = reinterpret_cast<v4f*>(span_lds);
#pragma unroll
    for (int m = 0; m < NMAT; m++)
#pragma unroll
        for (int j = 0; j < NSUB; j++) red[((wave * NMAT + m) * NSUB + j) * 64 + lane] = acc[m][j];
    __syncthreads();
    // Wave w finalizes the sub-tiles j with j % NWS == w (all matrices).
#pragma unroll
    for (int j = 0; j < NSUB; j++) {
        if ((uint32_t)(j % NWS) != wave) continue;
        v4f t[NMAT];
#pragma unroll
        for (int m = 0; m < NMAT; m++) {
            t[m] = red[((0 * NMAT + m) * NSUB + j) * 64 + lane];
#pragma unroll
            for (int w = 1; w < NWS; w++) t[m] += red[((w * NMAT + m) * NSUB + j) * 64 + lane];
        }
        const uint32_t n = n0 + j * 16 + rr;
        if (j * 16 + rr >= rows) continue;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t tl = 4 * g + i;
            if (tl >= cnt) continue;
            if (MODE == SPAN_RAW) {
                A.out32[(uint64_t)(blockIdx.y * 16 + tl) * N + n] = t[0][i];
            } else if (MODE == SPAN_GATE_UP) {
                const uint32_t r = A.seg_list[begin + tl];
                float gv = round_bf16(t[0][i]);
                float uv = round_bf16(t[NMAT - 1][i]);
                if (A.limit > 0.0f) {
                    gv = fminf(gv, A.limit);
                    uv = fminf(fmaxf(uv, -A.limit), A.limit);
                }
                float h = (gv / (1.0f + expf(-gv))) * uv;
                A.out16[(uint64_t)(r / A.k) * A.frame_elems + (uint64_t)(r % A.k) * N + n] = (uint16_t)f32_to_bf16(h);
            } else {
                const uint32_t r = A.seg_list[begin + tl];
                const float wr = bf16_to_f32(A.routes[r] >> 16);
                A.out16[(uint64_t)r * N + n] = (uint16_t)f32_to_bf16(t[0][i] * wr);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Expert banks with e4m3 weights (resident/adaptive pre-expanded MXFP4 and
// native FP8 experts, …gate_up_batch1_mxfp4.comp.template:173-229, :299-355;
// …down_batch1_mxfp4.comp.template:151-183, :355-418).  One block = 16
// weight rows of one tile (<= 16 routes) of the preparation launch; its 4
// waves split the 128-column chunks.  The tile's format (bits 16-17 of its
// record's expert word) picks the operands per block:
//  - 0 compact MXFP4: fp4 weights, the fp8 x fp4 operand layout of load_a;
//  - 1 expanded: e4m3 weights in the activation operand's layout, with the
//    row's per-32 e8m0 scales (lane group g carries block g's);
//  - 2 native: e4m3 bytes with the e8m0 byte of the weight's 128 x 128 block
//    (a zero byte is the scale 0.0, so the weights are zeroed).
// The weights are read straight from global memory into registers.
// ---------------------------------------------------------------------------
template <int MODE, int NMAT>
__global__ __launch_bounds__(256) void mx_wfmt_kernel(SpanArgs A) {
    __shared__ v4f red[4][NMAT][64];
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t g = lane >> 4, rr = lane & 15;
    const uint32_t K = A.K, N = A.N, nch = (K + 127) / 128, SB = K / 32;
    const uint32_t n0 = blockIdx.x * 16;
    const uint32_t tile = blockIdx.y;
    if (n0 >= N || tile >= *A.n_tiles) return;
    const TileRec rec = A.recs[tile];
    const uint32_t fmt = (rec.expert >> 16) & 3u, begin = rec.begin, cnt = rec.count;
    const uint32_t n = min(n0 + rr, N - 1);
    const uint8_t* arow = nullptr;
    const float* ascale = nullptr;
    if (rr < cnt) {
        const uint32_t row = A.seg_list[begin + rr] / A.a_row_div;
        arow = A.aq + (uint64_t)row * K;
        ascale = A.as + (uint64_t)row * nch;
    }
    const uint32_t per = (nch + 3) / 4;
    const uint32_t c0 = min(nch, wave * per), c1 = min(nch, c0 + per);
    v4f acc[NMAT];
#pragma unroll
    for (int m = 0; m < NMAT; m++) acc[m] = v4f{0.f, 0.f, 0.f, 0.f};
    for (uint32_t c = c0; c < c1; c++) {
        const uint32_t kb = c * 128 + g * 32;
        const bool kv = kb < K;
        if (fmt == 0) {
            v8i a;
            uint32_t sa;
            load_a(arow, ascale, K, c, g, a, sa);
#pragma unroll
            for (int m = 0; m < NMAT; m++) {
                v4i w = v4i{0, 0, 0, 0};
                uint32_t sw = 127;
                if (A.block_major) {
                    // W [K/128, N, 64], S [K/128, N, 4]: chunk c of row n is
                    // 64 contiguous bytes, its 4 scales one dword.
                    if (kv) {
                        w = *reinterpret_cast<const v4i*>(rec.w[m] + ((uint64_t)c * N + n) * 64 + g * 16);
                        sw = rec.s[m][((uint64_t)c * N + n) * 4 + g];
                    }
                } else {
                    load_w(rec.w[m] + (uint64_t)n * (K / 2), rec.s[m] + (uint64_t)n * SB, K, c, g, w, sw);
                }
                acc[m] = mfma_fp8_fp4(a, w, sa, sw, acc[m]);
            }
        } else {
            // Both e4m3 operands in the activation layout (lane group g: k
            // 16 g.. and 64 + 16 g..); the scale of lane group g is that of
            // the chunk's 32-column block g, as for the fp4 weights.
            v8i a;
            uint32_t sa;
            load_a(arow, ascale, K, c, g, a, sa);
            const uint32_t k0 = c * 128 + g * 16;
#pragma unroll
            for (int m = 0; m < NMAT; m++) {
                const uint8_t* wr = rec.w[m] + (uint64_t)n * K;
                v4i wlo = v4i{0, 0, 0, 0}, whi = v4i{0, 0, 0, 0};
                if (k0 < K) wlo = *reinterpret_cast<const v4i*>(wr + k0);
                if (k0 + 64 < K) whi = *reinterpret_cast<const v4i*>(wr + k0 + 64);
                uint32_t sw = 127;
                if (fmt == 2) {
                    // One byte per 128 x 128 block; 0 is the scale 0.0.
                    sw = rec.s[m][(uint64_t)(n / 128) * nch + c];
                    if (sw == 0u) wlo = whi = v4i{0, 0, 0, 0};
                } else if (kv) {
                    sw = rec.s[m][(uint64_t)n * SB + kb / 32];
                }
                acc[m] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                    a, v8i{wlo.x, wlo.y, wlo.z, wlo.w, whi.x, whi.y, whi.z, whi.w}, acc[m], 0, 0, 0, (int)sa, 0,
                    (int)sw);
            }
        }
    }
#pragma unroll
    for (int m = 0; m < NMAT; m++) red[wave][m][lane] = acc[m];
    __syncthreads();
    if (wave != 0) return;
    v4f tsum[NMAT];
#pragma unroll
    for (int m = 0; m < NMAT; m++) tsum[m] = ((red[0][m][lane] + red[1][m][lane]) + red[2][m][lane]) + red[3][m][lane];
    const uint32_t nn = n0 + rr;
    if (nn >= N) return;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t tl = 4 * g + i;
        if (tl >= cnt) continue;
        const uint32_t r = A.seg_list[begin + tl];
        if (MODE == SPAN_GATE_UP) {
            float gv = round_bf16(tsum[0][i]);
            float uv = round_bf16(tsum[NMAT - 1][i]);
            if (A.limit > 0.0f) {
                gv = fminf(gv, A.limit);
                uv = fminf(fmaxf(uv, -A.limit), A.limit);
            }
            const float h = (gv / (1.0f + expf(-gv))) * uv;
            A.out16[(uint64_t)(r / A.k) * A.frame_elems + (uint64_t)(r % A.k) * N + nn] = (uint16_t)f32_to_bf16(h);
        } else {
            const float wr = bf16_to_f32(A.routes[r] >> 16);
            A.out16[(uint64_t)r * N + nn] = (uint16_t)f32_to_bf16(tsum[0][i] * wr);
        }
    }
}

template <int MODE, int NMAT, int NSUB, int NWS = 4>
nerve_hip_status launch_span(SpanArgs A, uint32_t tiles, hipStream_t st) {
    constexpr uint32_t R = 16 * NSUB;
    A.w_region = span_w_region(R, A.K);
    A.s_region = span_s_region(R, A.K);
    size_t lds = (size_t)NMAT * (A.w_region + A.s_region);
    size_t red = (size_t)NWS * NMAT * NSUB * 64 * sizeof(v4f);
    if (red > lds) lds = red;
    static bool attr_set = false;
    if (!attr_set) {
        (void)hipFuncSetAttribute((const void*)mx_span_kernel<MODE, NMAT, NSUB, NWS>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        attr_set = true;
    }
    const uint32_t rpb = A.rpb ? A.rpb : R;
    if (rpb > R) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "span rows per block exceed the kernel's tile");
    dim3 grid((A.N + rpb - 1) / rpb, tiles);
    mx_span_kernel<MODE, NMAT, NSUB, NWS><<<grid, 64 * NWS, lds, st>>>(A);
    return nh::check_launch("mx_span_kernel");
}

// ---------------------------------------------------------------------------
// Persistent span-streaming expert GEMV (decode-shaped batches).
//
// The span kernel above waits for its block's whole span before contracting
// it, so a CU holding ~3 such blocks spends much of its time with nothing in
// flight (record and activation round trips, MFMA, reduction, epilogue).  Here
// one block per CU walks a contiguous range of work items (tile, 16-row block)
// in tile-major order and keeps NBUF - 1 row spans in flight in a ring of LDS
// slots while it contracts the current one:
//   * activations of the current tile stay in registers (reloaded only when
//     the tile changes, at most a few times per block);
//   * every wave issues the same, fixed number of copies per item (short
//     waves re-copy one of their own pieces), so "item i has landed" is
//     vmcnt <= copies_per_item * (items issued after i).  Loads retire in
//     issue order; the epilogue's global stores may retire in any order but
//     can only hold the count up, so the wait never ends early;
//   * tile records are read with scalar loads and all LDS traffic of the loop
//     is inline ds_read/ds_write, so the compiler inserts no vmcnt drains.
// ---------------------------------------------------------------------------
struct StreamArgs {
    const uint8_t* aq;
    const float* as;
    uint32_t a_row_div;
    uint32_t K, N, k;
    const uint32_t* routes;
    const uint32_t* seg_list;
    const TileRec* recs;
    const uint32_t* n_tiles;
    uint16_t* out16;
    uint64_t frame_elems;
    float limit;
    uint32_t w_region, s_region, slot_bytes;   // LDS layout of one ring slot
    uint32_t lw, ls;                            // copies per wave per matrix (weights, scales)
    uint32_t copies_per_item;                   // per wave: NMAT * (lw + ls)
    // Fused set-up (no preparation launch): the route map and parameter
    // tables the block reads itself, and bf16 activation rows quantized in
    // registers.  Activation row of route r: x16 + (r / k) * x_frame + (r % k) * x_seg.
    TileArgs T;
    const uint16_t* x16;
    uint64_t x_frame, x_seg;
    uint32_t addr_lds_records;                   // address tables up to this many records are copied to LDS
    uint32_t small_plan;                         // fused set-up by one wave (E <= 64, B k <= 64, >= 64 blocks)
    // Count stage folded into the launch (down only): block 0 writes
    // control[4] = (expert_count ? control[3] : k) * count_tiles, the one
    // control word the count stage changes after a compaction of the same
    // routes.  No block of this launch reads control[4].
    uint32_t* count_control;
    uint32_t count_tiles;
    // Down weights in the input-block-major layout (W [K/128, N, 64] bytes,
    // S [K/128, N, 4]): byte (row r, packed column j) of row-major W sits at
    // ((j / 64) N + r) 64 + j % 64, scale byte (r, group q) at
    // ((q / 4) N + r) 4 + q % 4.
    uint32_t block_major;
};

// One tile as the streaming loop sees it: its parameter pointers, its route
// count, and per lane the route whose activations it loads (row rr) and the
// route whose output it writes (token 4 g + wave), with that route's word.
struct TileSrc {
    const uint8_t* w[2];
    const uint8_t* s[2];
    uint32_t count;
    uint32_t in_route, out_route, out_word;
};

// Blockwise e4m3 quantization of one lane's 32 bf16 values of a 128-column
// block (the same arithmetic as quant_unit: pow2 scale of the block amax,
// x / scale rounded to e4m3).  The four lanes of a row (g = 0..3, lanes
// l, l + 16, l + 32, l + 48) hold the block's 128 columns, so all 64 lanes
// must call it.  Outputs the MFMA operand and the scale's e8m0 byte.
__device__ __forceinline__ void quant_chunk_e4m3(const v4i (&x)[4], v8i& out, uint32_t& e8m0) {
    float v[32];
#pragma unroll
    for (int h = 0; h < 4; h++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t w = (uint32_t)x[h][j];
            v[h * 8 + 2 * j] = bf16_to_f32((uint16_t)(w & 0xFFFFu));
            v[h * 8 + 2 * j + 1] = bf16_to_f32((uint16_t)(w >> 16));
        }
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; j++) m = fmaxf(m, fabsf(v[j]));
    m = max_xor16(m);
    m = max_xor32(m);
    const float sc = pow2_fp8_scale(m);
    uint32_t pk[8];
    // sc is a power of two, so v * (1 / sc) equals v / sc.  For a finite
    // block max every quotient lies in [-448, 448], where v_cvt_pk_fp8_f32
    // rounds exactly like f32_to_e4m3; a NaN input (its code 0x7f / 0xff) or
    // an infinite max takes the software conversion instead.
    bool soft = !(m <= 3.4028235e38f);
    if (!soft) {
        const float inv = __uint_as_float((254u << 23) - __float_as_uint(sc));
        uint32_t nan_bytes = 0;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            int w = __builtin_amdgcn_cvt_pk_fp8_f32(v[4 * j] * inv, v[4 * j + 1] * inv, 0, false);
            w = __builtin_amdgcn_cvt_pk_fp8_f32(v[4 * j + 2] * inv, v[4 * j + 3] * inv, w, true);
            pk[j] = (uint32_t)w;
            nan_bytes |= ((pk[j] & 0x7f7f7f7fu) + 0x01010101u) & 0x80808080u;
        }
        soft = nan_bytes != 0;
    }
    if (soft) {
#pragma unroll
        for (int j = 0; j < 8; j++)
            pk[j] = f32_to_e4m3(v[4 * j] / sc) | (f32_to_e4m3(v[4 * j + 1] / sc) << 8) |
                    (f32_to_e4m3(v[4 * j + 2] / sc) << 16) | (f32_to_e4m3(v[4 * j + 3] / sc) << 24);
    }
    out = v8i{(int)pk[0], (int)pk[1], (int)pk[2], (int)pk[3], (int)pk[4], (int)pk[5], (int)pk[6], (int)pk[7]};
    e8m0 = pow2_to_e8m0(sc);
}


typedef uint32_t u4s __attribute__((ext_vector_type(4)));
typedef uint32_t u8s __attribute__((ext_vector_type(8)));

// A tile record through the scalar cache (begin, count, matrix and scale
// pointers), so that reading it adds nothing to vmcnt.
__device__ __forceinline__ void sload_rec(const TileRec* rec, uint32_t& begin, uint32_t& count,
                                          const uint8_t* (&w)[2], const uint8_t* (&s)[2]) {
    u4s h;
    u8s p;
    asm volatile("s_load_dwordx4 %0, %2, 0x0\n\ts_load_dwordx8 %1, %2, 0x10\n\ts_waitcnt lgkmcnt(0)"
                 : "=&s"(h), "=&s"(p)
                 : "s"(rec));
    begin = h.y;
    count = h.z;
    w[0] = reinterpret_cast<const uint8_t*>(((uint64_t)p[1] << 32) | p[0]);
    w[1] = reinterpret_cast<const uint8_t*>(((uint64_t)p[3] << 32) | p[2]);
    s[0] = reinterpret_cast<const uint8_t*>(((uint64_t)p[5] << 32) | p[4]);
    s[1] = reinterpret_cast<const uint8_t*>(((uint64_t)p[7] << 32) | p[6]);
}

// x * sigmoid(x) with e^-x from the hardware base-2 exponential
// (v_exp_f32, ~1 ulp): e^-x = 2^(-x log2 e).
__device__ __forceinline__ float silu_fast(float x) {
    const float e = __builtin_amdgcn_exp2f(-x * 1.4426950408889634f);
    return x / (1.0f + e);
}

typedef uint32_t u16s __attribute__((ext_vector_type(16)));

// 16 consecutive words through the scalar cache (the buffer must extend 64
// bytes past p).
__device__ __forceinline__ u16s sload_x16(const uint32_t* p) {
    u16s v;
    asm volatile("s_load_dwordx16 %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p));
    return v;
}

__device__ __forceinline__ uint32_t sload_u32(const uint32_t* p) {
    uint32_t v;
    asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p));
    return v;
}

// One contiguous range of work items [i0, i1) of one tile, run by NW waves
// that split each item's K chunks.  An item is RI = 16 NSUB rows of each of
// the NMAT matrices.
template <int MODE, int NMAT, int NBUF, int NW, int NSUB, bool FUSED>
__device__ __forceinline__ void stream_range(const StreamArgs& A, uint32_t i0, uint32_t i1, uint32_t nrb,
                                             const TileSrc& ts) {
    constexpr uint32_t RI = 16 * NSUB;
    constexpr uint32_t CH = 32 / NW;                            // max K chunks per wave (K <= 4096)
    constexpr uint32_t LWMAX = (32 * NSUB + NW - 1) / NW;       // max weight copies per wave per matrix
    constexpr uint32_t LSMAX = (8 * NSUB + NW - 1) / NW;
    extern __shared__ __attribute__((aligned(16))) uint8_t ring[];
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lane = threadIdx.x & 63, g = lane >> 4, rr = lane & 15;
    const uint32_t K = A.K, N = A.N, RB = K / 2, SB = K / 32, nch = (K + 127) / 128;
    const uint32_t lw = A.lw, ls = A.ls;

    // Ranges run back to back in one block: every wave has finished the
    // previous one (ring slots and the reduction area are reused).
    __builtin_amdgcn_s_barrier();
    uint8_t* red = ring + 2 * A.slot_bytes;   // [wave][NMAT * NSUB][lane] v4f partial sums
    const uint32_t npw = (RI * RB + 1023) / 1024, nps = (RI * SB + 255) / 256;

    // ---- copy plan, fixed for the range: piece t of this wave starts at
    // byte wpos(t) of the RI-row span (short waves repeat their first piece
    // so every wave issues lw + ls copies per matrix).  The last piece is
    // aligned to the span's end, overlapping its neighbour with identical
    // bytes, so LDS regions need no padding.
    uint32_t wpos[LWMAX], spos[LSMAX], woff[LWMAX], soff[LSMAX];
#pragma unroll
    for (uint32_t t = 0; t < LWMAX; t++) {
        uint32_t pc = wave + NW * t;
        if (pc >= npw) pc = wave < npw ? wave : 0;
        wpos[t] = min(pc * 1024, RI * RB - 1024);
        woff[t] = wpos[t] + lane * 16;
    }
#pragma unroll
    for (uint32_t t = 0; t < LSMAX; t++) {
        uint32_t pc = wave + NW * t;
        if (pc >= nps) pc = wave < nps ? wave : 0;
        spos[t] = min(pc * 256, RI * SB - 256);
        soff[t] = spos[t] + lane * 4;
    }

    // Source offsets of the same LDS pieces (relative to the item's first
    // row): the row-major span, or gathered from the input-block-major
    // layout (a 16-byte piece never straddles a 64-byte block row, a scale
    // dword never straddles a 4-byte one, since K % 128 == 0 there).
    uint32_t wsrc[LWMAX], ssrc[LSMAX];
#pragma unroll
    for (uint32_t t = 0; t < LWMAX; t++)
        wsrc[t] = A.block_major ? ((woff[t] % RB) / 64) * N * 64 + (woff[t] / RB) * 64 + woff[t] % 64 : woff[t];
#pragma unroll
    for (uint32_t t = 0; t < LSMAX; t++)
        ssrc[t] = A.block_major ? ((soff[t] % SB) / 4) * N * 4 + (soff[t] / SB) * 4 : soff[t];
    const uint32_t wrow = A.block_major ? 64u : RB, srow = A.block_major ? 4u : SB;

    // ---- issue side: item `item`'s pieces are loaded with nontemporal
    // loads into a register set and written to an LDS slot when the item
    // comes up (streaming reads from registers sustain ~7 TB/s over the chip
    // where copies straight into LDS sustain ~6.1).
    const uint32_t tile_base = (i0 / nrb) * nrb;
    struct ItemRegs {
        v4i w[NMAT][LWMAX];
        uint32_t s[NMAT][LSMAX];
    };
    auto load_item = [&](uint32_t item, ItemRegs& R) __attribute__((always_inline)) {
        const uint32_t n0 = (item - tile_base) * RI;
        const uint32_t rows = min(RI, N - n0);
        const uint32_t wbytes = rows * RB, sbytes = rows * SB;
#pragma unroll
        for (int m = 0; m < NMAT; m++) {
            const uint8_t* ws = ts.w[m] + (uint64_t)n0 * wrow;
#pragma unroll
            for (uint32_t t = 0; t < LWMAX; t++)
                if (t < lw) R.w[m][t] = gload16_nt_untracked(ws + (woff[t] < wbytes ? wsrc[t] : 0));
            const uint8_t* ss = ts.s[m] + (uint64_t)n0 * srow;
#pragma unroll
            for (uint32_t t = 0; t < LSMAX; t++)
                if (t < ls) R.s[m][t] = gload4_nt_untracked(ss + (soff[t] < sbytes ? ssrc[t] : 0));
        }
    };
    auto store_item = [&](const ItemRegs& R, uint32_t slot) __attribute__((always_inline)) {
        uint8_t* dst = ring + slot * A.slot_bytes;
#pragma unroll
        for (int m = 0; m < NMAT; m++) {
#pragma unroll
            for (uint32_t t = 0; t < LWMAX; t++)
                if (t < lw) *reinterpret_cast<v4i*>(dst + m * A.w_region + woff[t]) = R.w[m][t];
#pragma unroll
            for (uint32_t t = 0; t < LSMAX; t++)
                if (t < ls) *reinterpret_cast<uint32_t*>(dst + NMAT * A.w_region + m * A.s_region + soff[t]) = R.s[m][t];
        }
    };

    // ---- compute side: this wave's K chunks and their LDS offsets
    const uint32_t per = (nch + NW - 1) / NW;
    const uint32_t c0 = min(nch, wave * per), c1 = min(nch, c0 + per);
    uint32_t rw[CH], rs[CH];
    bool kvalid[CH];
#pragma unroll
    for (uint32_t q = 0; q < CH; q++) {
        const uint32_t c = c0 + q, kb = c * 128 + g * 32;
        kvalid[q] = c < c1 && kb < K;
        const uint32_t kk = kvalid[q] ? kb : 0;
        rw[q] = rr * RB + kk / 2;
        rs[q] = NMAT * A.w_region + rr * SB + kk / 32;
    }

    // ---- activations of the tile.  Loads are issued after the prologue
    // copies and converted after one wait (the empty asm in the conversion
    // keeps the compiler from folding it into the loads' branches, which
    // would wait for each load there).
    const bool arow_ok = rr < ts.count;
    const bool ovalid = wave < 4 && 4 * g + wave < ts.count;
    v8i av[CH];
    uint32_t sa[CH];
    v4i lo[CH], hi[CH];          // e4m3 operand halves (pre-quantized input)
    float sraw[CH];
    v4i xb[CH][4];               // bf16 operand halves (fused quantization)
    // Which of this lane's activation pieces exist (k0 < K covers a whole
    // 16-column half since K % 32 == 0).
    auto piece_ok = [&](uint32_t q, int h) __attribute__((always_inline)) {
        const uint32_t c = c0 + q, k0 = c * 128 + g * 16 + (h >= 2 ? 64u : 0u);
        return arow_ok && c < c1 && k0 < K;
    };
    auto act_request = [&]() __attribute__((always_inline)) {
        if (FUSED) {
            // Inline-asm loads: the compiler does not count them, so it adds
            // no wait for them in front of the weight copies issued next.
            // Every piece is loaded (absent ones from the row start, which
            // exists) and zeroed after the wait, so no load sits in a branch.
            const uint16_t* xr = A.x16 + (uint64_t)(ts.in_route / A.k) * A.x_frame + (uint64_t)(ts.in_route % A.k) * A.x_seg;
#pragma unroll
            for (uint32_t q = 0; q < CH; q++) {
                if (c0 + q >= c1) continue;   // wave-uniform: chunks this wave never contracts
                const uint32_t k0 = (c0 + q) * 128 + g * 16;
#pragma unroll
                for (int h = 0; h < 4; h++) {
                    const uint32_t off = k0 + (h >= 2 ? 64u : 0u) + (h & 1 ? 8u : 0u);
                    xb[q][h] = gload16_untracked(xr + (piece_ok(q, h) ? off : 0u));
                }
            }
        } else {
            const uint32_t row = ts.in_route / A.a_row_div;
            const uint8_t* arow = A.aq + (uint64_t)(arow_ok ? row : 0) * K;
            const float* ascale = A.as + (uint64_t)(arow_ok ? row : 0) * nch;
#pragma unroll
            for (uint32_t q = 0; q < CH; q++) {
                const uint32_t c = c0 + q, k0 = c * 128 + g * 16;
                lo[q] = hi[q] = v4i{0, 0, 0, 0};
                sraw[q] = 1.0f;
                if (arow_ok && c < c1) {
                    if (k0 < K) lo[q] = *reinterpret_cast<const v4i*>(arow + k0);
                    if (k0 + 64 < K) hi[q] = *reinterpret_cast<const v4i*>(arow + k0 + 64);
                    sraw[q] = ascale[c];
                }
            }
        }
    };
    auto act_finish = [&]() {
        if (FUSED) {
            // Blockwise e4m3 quantization of this lane's 32 values of each
            // 128-column block (the same arithmetic as quant_unit: pow2
            // scale of the block amax, x / scale rounded to e4m3).  The four
            // lanes of a row (g = 0..3) hold the block's 128 columns.
#pragma unroll
            for (uint32_t q = 0; q < CH; q++) {
                // Chunks past this wave's share are neither loaded nor contracted.
                if (c0 + q >= c1) {
                    av[q] = v8i{0, 0, 0, 0, 0, 0, 0, 0};
                    sa[q] = 127u;
                    continue;
                }
#pragma unroll
                for (int h = 0; h < 4; h++) {
                    asm volatile("" : "+v"(xb[q][h]));
                    if (!piece_ok(q, h)) xb[q][h] = v4i{0, 0, 0, 0};
                }
                uint32_t e8;
                quant_chunk_e4m3(xb[q], av[q], e8);
                sa[q] = arow_ok ? e8 : 127u;
            }
        } else {
#pragma unroll
            for (uint32_t q = 0; q < CH; q++) asm volatile("" : "+v"(lo[q]), "+v"(hi[q]), "+v"(sraw[q]));
#pragma unroll
            for (uint32_t q = 0; q < CH; q++) {
                av[q] = v8i{lo[q].x, lo[q].y, lo[q].z, lo[q].w, hi[q].x, hi[q].y, hi[q].z, hi[q].w};
                sa[q] = arow_ok ? pow2_to_e8m0(sraw[q]) : 127u;
            }
        }
    };
    uint64_t obase = 0;        // output element offset of this lane's token (component `wave`)
    if (MODE == SPAN_GATE_UP)
        obase = (uint64_t)(ts.out_route / A.k) * A.frame_elems + (uint64_t)(ts.out_route % A.k) * N;
    else
        obase = (uint64_t)ts.out_route * N;
    const float wr = bf16_to_f32(ts.out_word >> 16);

    // Prologue: the tile's activations, then the first item's loads.  Loads
    // retire in issue order, so waiting until only that item's loads are in
    // flight lands the activations, which are quantized while the item
    // streams; the second item is loaded after that (issuing it first would
    // stall this wave until the CU's miss queue drains).
    act_request();
    // Every wave's activation loads enter the CU's memory pipeline before
    // any weight load: behind those they would wait for HBM-bound traffic.
    __builtin_amdgcn_s_barrier();
    ItemRegs R0{}, R1{};
    load_item(i0, R0);
    wait_vm(A.copies_per_item);
    act_finish();
    if (i0 + 1 < i1) load_item(i0 + 1, R1);

    // One item: its registers go to LDS slot (i - i0) % 2 (last read by the
    // item two back, whose reduction barrier every wave has passed), the
    // item two ahead is loaded into the same registers, a barrier, then the
    // contraction and the cross-wave reduction.
    auto item_step = [&](uint32_t i, ItemRegs& R) __attribute__((always_inline)) {
        const uint32_t slot = (i - i0) & 1u;
        // With only the next item's loads allowed in flight this item's have landed.
        wait_vm(i + 1 < i1 ? A.copies_per_item : 0u);
#pragma unroll
        for (int m = 0; m < NMAT; m++) {
#pragma unroll
            for (uint32_t t = 0; t < LWMAX; t++) asm volatile("" : "+v"(R.w[m][t]));
#pragma unroll
            for (uint32_t t = 0; t < LSMAX; t++) asm volatile("" : "+v"(R.s[m][t]));
        }
        store_item(R, slot);
        if (i + 2 < i1) load_item(i + 2, R);
        __syncthreads();
        const uint32_t n0 = (i - tile_base) * RI;
        // ---- contract this wave's chunks of the slot
        const uint8_t* buf = ring + slot * A.slot_bytes;
        v4f acc[NMAT][NSUB];
#pragma unroll
        for (int m = 0; m < NMAT; m++)
#pragma unroll
            for (int j = 0; j < NSUB; j++) acc[m][j] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (uint32_t q0 = 0; q0 < CH; q0 += 4) {
            if (c0 + q0 >= c1) continue;
            v4i w[4][NMAT][NSUB];
            uint32_t sw[4][NMAT][NSUB];
#pragma unroll
            for (uint32_t u = 0; u < 4; u++) {
#pragma unroll
                for (int m = 0; m < NMAT; m++) {
#pragma unroll
                    for (int j = 0; j < NSUB; j++) {
                        w[u][m][j] = lds_read16(buf + m * A.w_region + j * 16 * RB + rw[q0 + u]);
                        sw[u][m][j] = lds_read_u8(buf + m * A.s_region + j * 16 * SB + rs[q0 + u]);
                    }
                }
            }
            lds_drain();
#pragma unroll
            for (uint32_t u = 0; u < 4; u++) {
                if (c0 + q0 + u >= c1) continue;
#pragma unroll
                for (int m = 0; m < NMAT; m++) {
#pragma unroll
                    for (int j = 0; j < NSUB; j++) {
                        // Operands of a drained read are opaque to the
                        // compiler; launder them through an empty asm so
                        // their use stays after the wait.
                        v4i wv = w[u][m][j];
                        uint32_t s8 = sw[u][m][j];
                        asm volatile("" : "+v"(wv), "+v"(s8));
                        if (!kvalid[q0 + u]) {
                            wv = v4i{0, 0, 0, 0};
                            s8 = 127;
                        }
                        acc[m][j] = mfma_fp8_fp4(av[q0 + u], wv, sa[q0 + u], s8, acc[m][j]);
                    }
                }
            }
        }
        // ---- cross-wave reduction; waves 0..3 finalize component `wave`.
        // An MFMA result read by another instruction needs software wait
        // states, which the compiler does not add in front of inline asm: the
        // nops take the accumulators as operands so they sit between the last
        // MFMA and the LDS write.
#pragma unroll
        for (int m = 0; m < NMAT; m++)
#pragma unroll
            for (int j = 0; j < NSUB; j++) asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(acc[m][j]));
#pragma unroll
        for (int m = 0; m < NMAT; m++)
#pragma unroll
            for (int j = 0; j < NSUB; j++)
                lds_write16(red + ((wave * NMAT * NSUB + m * NSUB + j) * 64 + lane) * 16, acc[m][j]);
        lds_drain();
        __builtin_amdgcn_s_barrier();
        if (wave >= 4) return;
#pragma unroll
        for (int j = 0; j < NSUB; j++) {
            float t[NMAT];
#pragma unroll
            for (int m = 0; m < NMAT; m++) {
                uint32_t v[NW];
#pragma unroll
                for (int w2 = 0; w2 < NW; w2++)
                    v[w2] = lds_read_b32(red + ((w2 * NMAT * NSUB + m * NSUB + j) * 64 + lane) * 16 + 4 * wave);
                lds_drain();
                float sum = 0.0f;
#pragma unroll
                for (int w2 = 0; w2 < NW; w2++) {
                    asm volatile("" : "+v"(v[w2]));
                    sum += __uint_as_float(v[w2]);
                }
                t[m] = sum;
            }
            const uint32_t n = n0 + j * 16 + rr;
            if (ovalid && n < N) {
                if (MODE == SPAN_GATE_UP) {
                    float gv = round_bf16(t[0]);
                    float uv = round_bf16(t[NMAT - 1]);
                    if (A.limit > 0.0f) {
                        gv = fminf(gv, A.limit);
                        uv = fminf(fmaxf(uv, -A.limit), A.limit);
                    }
                    const float h = silu_fast(gv) * uv;
                    A.out16[obase + n] = (uint16_t)f32_to_bf16(h);
                } else {
                    A.out16[obase + n] = (uint16_t)f32_to_bf16(t[0] * wr);
                }
            }
        }
    };
    for (uint32_t i = i0; i < i1; i += 2) {
        item_step(i, R0);
        if (i + 1 < i1) item_step(i + 1, R1);
    }
}

// Fused set-up tables (in the LDS ring, before any copy is issued).
constexpr uint32_t FUSED_MAX_EXPERTS = 512;
constexpr uint32_t FUSED_MAX_SLOTS = 1024;
constexpr uint32_t FUSED_MAX_WAVES = 8;

// A block's whole work as the one-wave set-up publishes it: the tile's
// parameter pointers, its route ids and words, and the block's row-block
// range (lo_rb == hi_rb: no work).
struct SmallPlan {
    uint64_t ptr[4];
    uint32_t count, tile, lo_rb, hi_rb;
    uint32_t route[16];
    uint32_t word[16];
    uint32_t cnt[64];                     // valid routes per expert (scratch)
};

struct FusedTables {
    SmallPlan plan;                       // the one-wave set-up's result
    uint64_t eptr[FUSED_MAX_EXPERTS][4];  // resolved parameter pointers of each expert
    uint32_t cnt[FUSED_MAX_EXPERTS];      // valid routes per expert
    uint32_t rw[FUSED_MAX_SLOTS];         // route index of compacted slot c
    uint32_t rword[FUSED_MAX_SLOTS];      // its route word
    uint32_t rtab[FUSED_MAX_SLOTS];       // route word of route index r
    uint16_t eslot[FUSED_MAX_SLOTS];      // its expert (NO_EXPERT: skipped)
    uint16_t rank[FUSED_MAX_SLOTS];       // its position among its expert's slots
    uint8_t valid[FUSED_MAX_EXPERTS];
    uint32_t wlist[FUSED_MAX_WAVES][16];  // per wave: slots of the tile being set up
};


// Route -> tile tables of one projection, built by every streaming block for
// itself (the same rules as build_tiles: invalid parameters or expert ids
// skip a route; 16 routes per tile).  One round of independent global loads
// (slot words, route map, route words, control words and the whole address
// table, copied into LDS after the tables), then LDS work.  Each slot's rank
// among its expert's slots comes from the counting atomic.  The launch has a
// thread per expert and per compacted slot.
template <int NW>
__device__ __forceinline__ void fused_tables(const TileArgs& A, FusedTables& F, uint32_t* addr_lds) {
    static_assert(NW <= (int)FUSED_MAX_WAVES, "per-wave lists");
    const uint32_t tid = threadIdx.x, nt = 64 * NW;
    const uint32_t cap = A.batch_width * A.k, P = A.P;
    uint32_t sl[4] = {UNBOUND_SLOT, UNBOUND_SLOT, UNBOUND_SLOT, UNBOUND_SLOT};
#pragma unroll
    for (uint32_t p = 0; p < 4; p++) {
        const uint32_t idx = tid * P + p;
        if (tid < A.E && p < P && idx < A.n_slot_words) sl[p] = A.slots[idx];
    }
    const uint32_t r0 = tid < cap ? A.frames[(uint64_t)(tid / A.k) * A.frame_words + A.data_words + tid % A.k] : 0u;
    const uint32_t rt0 = tid < cap ? A.routes[tid] : 0u;
    const uint32_t c2 = A.control[2], c3 = A.control[3];
    {
        const v4i* src = reinterpret_cast<const v4i*>(A.addr);
        v4i* dst = reinterpret_cast<v4i*>(addr_lds);
        for (uint32_t i = tid; i < 2 * A.n_records; i += nt) dst[i] = src[i];
    }
    if (tid < cap) {
        F.rw[tid] = r0;
        F.rtab[tid] = rt0;
    }
    __syncthreads();
    if (tid < A.E) {
        bool ok = true;
#pragma unroll
        for (uint32_t p = 0; p < 4; p++) {
            const bool has = sl[p] != UNBOUND_SLOT && sl[p] < A.n_records;
            const v4i* r = reinterpret_cast<const v4i*>(addr_lds + (has ? sl[p] : 0u) * 8);
            const v4i lo = r[0], hi = r[1];
            uint32_t rec[8];
#pragma unroll
            for (uint32_t j = 0; j < 4; j++) {
                rec[j] = has ? (uint32_t)lo[j] : 0u;
                rec[4 + j] = has ? (uint32_t)hi[j] : 0u;
            }
            if (p < P) {
                const bool is_weight = (p % 2) == 0;
                ok = record_valid(sl[p], A.n_records, rec, is_weight ? A.req_w : A.req_s, is_weight ? 16u : 4u) && ok;
            }
            F.eptr[tid][p] = (uint64_t)rec[0] | ((uint64_t)rec[1] << 32);
        }
        F.valid[tid] = ok ? 1 : 0;
        F.cnt[tid] = 0;
    }
    uint32_t n = c2 != 0u ? c3 : cap;
    if (n > cap) n = cap;
    __syncthreads();
    for (uint32_t c = tid; c < cap; c += nt) {
        const uint32_t r = F.rw[c], w = r < cap ? F.rtab[r] : 0u, e = w & 0xffffu;
        F.rword[c] = w;
        const bool ok = c < n && r < cap && e < A.E && F.valid[e];
        F.eslot[c] = ok ? (uint16_t)e : NO_EXPERT;
        if (ok) F.rank[c] = (uint16_t)atomicAdd(&F.cnt[e], 1u);
    }
    __syncthreads();
}

// Tiles of the fused tables, computed by each wave on its own (no barrier):
// expert e owns tiles [first(e), first(e) + ceil(cnt[e] / 16)), first() being
// the exclusive prefix sum in expert order.  Returns the tile count; for
// t < count also the tile's expert and its index among the expert's tiles.
__device__ __forceinline__ uint32_t fused_tile_scan(const FusedTables& F, uint32_t E, uint32_t t, uint32_t& te,
                                                    uint32_t& tk) {
    const uint32_t lane = threadIdx.x & 63;
    const uint64_t below = (1ull << lane) - 1ull;
    uint32_t base = 0;
    te = 0;
    tk = 0;
    for (uint32_t e0 = 0; e0 < E; e0 += 64) {
        const uint32_t e = e0 + lane;
        const uint32_t nte = e < E ? (F.cnt[e] + 15u) / 16u : 0u;   // <= 64 (slots <= 1024)
        uint32_t excl = 0, tot = 0;
#pragma unroll
        for (uint32_t bit = 0; bit < 7; bit++) {
            const uint64_t m = __ballot((nte >> bit) & 1u);
            excl += (uint32_t)__popcll(m & below) << bit;
            tot += (uint32_t)__popcll(m) << bit;
        }
        const uint32_t first = base + excl;
        const uint64_t hit = __ballot(nte != 0u && t >= first && t < first + nte);
        if (hit) {
            const uint32_t l = (uint32_t)__builtin_ctzll(hit);
            te = e0 + l;
            tk = t - (uint32_t)__builtin_amdgcn_readlane((int)first, (int)l);
        }
        base += tot;
    }
    return base;
}

// Tile `t` of the fused tables: its expert's pointers, its routes and this
// lane's route ids.  Ends with a block barrier, after which the ring may be
// overwritten.
template <int NW>
__device__ __forceinline__ TileSrc fused_tile(const StreamArgs& A, FusedTables& F, uint32_t t) {
    const TileArgs& T = A.T;
    const uint32_t cap = T.batch_width * T.k;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t e, kk;
    fused_tile_scan(F, T.E, t, e, kk);
    // The tile's slots: ranks 16 kk .. 16 kk + 15 of the expert, listed by
    // this wave for itself (a wave's LDS accesses complete in order).
    uint32_t* wl = F.wlist[wave];
    for (uint32_t c = lane; c < cap; c += 64) {
        const uint32_t rk = F.rank[c];
        if (F.eslot[c] == e && rk >= 16 * kk && rk < 16 * kk + 16) wl[rk - 16 * kk] = c;
    }
    TileSrc ts;
    ts.w[0] = reinterpret_cast<const uint8_t*>(F.eptr[e][0]);
    ts.s[0] = reinterpret_cast<const uint8_t*>(F.eptr[e][1]);
    ts.w[1] = reinterpret_cast<const uint8_t*>(F.eptr[e][2]);
    ts.s[1] = reinterpret_cast<const uint8_t*>(F.eptr[e][3]);
    ts.count = min(16u, F.cnt[e] - 16 * kk);
    const uint32_t rr = lane & 15, tl = 4 * (lane >> 4) + wave;
    ts.in_route = rr < ts.count ? F.rw[wl[rr]] : 0u;
    const bool ov = wave < 4 && tl < ts.count;
    ts.out_route = ov ? F.rw[wl[tl]] : 0u;
    ts.out_word = ov ? F.rword[wl[tl]] : 0u;
    __syncthreads();
    return ts;
}

// Row-block range of block b when there are at least as many blocks as
// tiles: tile t gets q or q + 1 blocks, which split its row blocks evenly.
__device__ __forceinline__ void block_share(uint32_t G, uint32_t b, uint32_t n_tiles, uint32_t nrb, uint32_t& tile,
                                            uint32_t& lo_rb, uint32_t& hi_rb) {
    const uint32_t q = G / n_tiles, r = G % n_tiles;
    // Blocks [0, r (q + 1)) serve tiles 0..r-1 with q + 1 blocks each.
    uint32_t part, parts;
    if (b < r * (q + 1)) {
        tile = b / (q + 1);
        part = b % (q + 1);
        parts = q + 1;
    } else {
        tile = r + (b - r * (q + 1)) / q;
        part = (b - r * (q + 1)) % q;
        parts = q;
    }
    lo_rb = nrb * part / parts;
    hi_rb = nrb * (part + 1) / parts;
}

// The fused set-up for small decode batches (E <= 64 experts, B k <= 64
// routes, at least 64 blocks): wave 0 alone computes the block's plan with
// one lane per expert and one per compacted slot, the same rules as
// fused_tables (a slot counts when it is below the owned count, its route
// index and expert are in range and every parameter record of its expert is
// valid; 16 routes per tile in expert order), while the other waves wait at
// one barrier.  Routes of a tile are taken in slot order.  The address table
// is staged in LDS by all waves first (a table the LDS does not hold is read
// from memory, its experts' records only, after the slot words).
__device__ __forceinline__ void fused_small_plan(const TileArgs& A, SmallPlan& S, uint32_t* addr_lds, uint32_t nrb,
                                                 bool big_table) {
    const uint32_t tid = threadIdx.x, nt = blockDim.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t cap = A.batch_width * A.k, P = A.P, E = A.E;
    uint32_t sl[4] = {UNBOUND_SLOT, UNBOUND_SLOT, UNBOUND_SLOT, UNBOUND_SLOT};
    uint32_t r0 = 0, rt0 = 0, c2 = 0, c3 = 0;
    if (wave == 0) {
#pragma unroll
        for (uint32_t p = 0; p < 4; p++) {
            const uint32_t idx = lane * P + p;
            if (lane < E && p < P && idx < A.n_slot_words) sl[p] = A.slots[idx];
        }
        r0 = lane < cap ? A.frames[(uint64_t)(lane / A.k) * A.frame_words + A.data_words + lane % A.k] : 0u;
        rt0 = lane < cap ? A.routes[lane] : 0u;
        c2 = A.control[2];
        c3 = A.control[3];
    }
    // A table the LDS does not hold (a package-wide one) is not staged: wave
    // 0 reads its experts' records from memory after the slot words.
    if (!big_table) {
        const v4i* src = reinterpret_cast<const v4i*>(A.addr);
        v4i* dst = reinterpret_cast<v4i*>(addr_lds);
        for (uint32_t i = tid; i < 2 * A.n_records; i += nt) dst[i] = src[i];
    }
    __syncthreads();
    if (wave == 0) {
        // Records of expert `lane`: all eight 16-byte reads first.
        v4i lo[4], hi[4];
        if (big_table) {
#pragma unroll
            for (uint32_t p = 0; p < 4; p++) {
                const bool has = sl[p] != UNBOUND_SLOT && sl[p] < A.n_records;
                const v4i* r = reinterpret_cast<const v4i*>(A.addr + (uint64_t)(has ? sl[p] : 0u) * 8);
                lo[p] = r[0];
                hi[p] = r[1];
            }
        } else {
#pragma unroll
            for (uint32_t p = 0; p < 4; p++) {
                const bool has = sl[p] != UNBOUND_SLOT && sl[p] < A.n_records;
                const v4i* r = reinterpret_cast<const v4i*>(addr_lds + (has ? sl[p] : 0u) * 8);
                lo[p] = r[0];
                hi[p] = r[1];
            }
        }
        bool valid = lane < E;
        uint64_t ptr[4];
#pragma unroll
        for (uint32_t p = 0; p < 4; p++) {
            const bool has = sl[p] != UNBOUND_SLOT && sl[p] < A.n_records;
            uint32_t rec[8];
#pragma unroll
            for (uint32_t j = 0; j < 4; j++) {
                rec[j] = has ? (uint32_t)lo[p][j] : 0u;
                rec[4 + j] = has ? (uint32_t)hi[p][j] : 0u;
            }
            if (p < P) {
                const bool is_weight = (p % 2) == 0;
                valid = record_valid(sl[p], A.n_records, rec, is_weight ? A.req_w : A.req_s, is_weight ? 16u : 4u) && valid;
            }
            ptr[p] = (uint64_t)rec[0] | ((uint64_t)rec[1] << 32);
        }
        const uint64_t vmask = __ballot(valid);
        // Slot `lane`: its route, expert and validity.
        uint32_t n = c2 != 0u ? c3 : cap;
        if (n > cap) n = cap;
        const uint32_t r = r0;
        // Every lane takes part in the shuffle (a lane reading from an inactive
        // lane gets 0), and the out-of-range routes are dropped afterwards.
        const uint32_t wsh = (uint32_t)__shfl((int)rt0, (int)(r & 63u));
        const uint32_t w = r < cap ? wsh : 0u;
        const uint32_t e = w & 0xffffu;
        const bool ok = lane < n && r < cap && e < E && ((vmask >> (e & 63u)) & 1ull);
        // Slots of the same expert (E <= 64: six bits), rank in slot order.
        uint64_t same = __ballot(ok);
#pragma unroll
        for (uint32_t bit = 0; bit < 6; bit++) {
            const uint64_t m = __ballot(ok && ((e >> bit) & 1u));
            same &= ((e >> bit) & 1u) ? m : ~m;
        }
        const uint64_t below = (1ull << lane) - 1ull;
        const uint32_t rank = (uint32_t)__popcll(same & below);
        // Per-expert counts through LDS (a wave's LDS accesses complete in order).
        S.cnt[lane] = 0;
        if (ok && rank == 0) S.cnt[e] = (uint32_t)__popcll(same);
        const uint32_t cnt = lane < E ? S.cnt[lane] : 0u;
        // Tiles in expert order: exclusive prefix of ceil(cnt / 16) by bits.
        const uint32_t nte = (cnt + 15u) / 16u;
        uint32_t first = 0, total = 0;
#pragma unroll
        for (uint32_t bit = 0; bit < 3; bit++) {       // nte <= 4 (cap <= 64)
            const uint64_t m = __ballot((nte >> bit) & 1u);
            first += (uint32_t)__popcll(m & below) << bit;
            total += (uint32_t)__popcll(m) << bit;
        }
        uint32_t tile = 0, lo_rb = 0, hi_rb = 0, te = 0, kk = 0;
        if (total) {
            block_share(gridDim.x, blockIdx.x, total, nrb, tile, lo_rb, hi_rb);
            const uint64_t hit = __ballot(nte != 0u && tile >= first && tile < first + nte);
            te = hit ? (uint32_t)__builtin_ctzll(hit) : 0u;
            kk = tile - (uint32_t)__builtin_amdgcn_readlane((int)first, (int)te);
        }
        const uint32_t tcnt = (uint32_t)__builtin_amdgcn_readlane((int)cnt, (int)te);
        if (ok && e == te && rank >= 16 * kk && rank < 16 * kk + 16) {
            S.route[rank - 16 * kk] = r;
            S.word[rank - 16 * kk] = w;
        }
#pragma unroll
        for (uint32_t p = 0; p < 4; p++) {
            const uint32_t plo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)ptr[p], (int)te);
            const uint32_t phi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(ptr[p] >> 32), (int)te);
            if (lane == 0) S.ptr[p] = ((uint64_t)phi << 32) | plo;
        }
        if (lane == 0) {
            S.count = total ? min(16u, tcnt - 16 * kk) : 0u;
            S.tile = tile;
            S.lo_rb = total ? lo_rb : 0u;
            S.hi_rb = total ? hi_rb : 0u;
        }
    }
    __syncthreads();
}

template <int MODE, int NMAT, int NBUF, int NW, int NSUB, bool FUSED>
__global__ __launch_bounds__(64 * NW) void mx_stream_kernel(StreamArgs A) {
    extern __shared__ __attribute__((aligned(16))) uint8_t ring[];
    if (A.count_control && blockIdx.x == 0 && threadIdx.x == 0) {
        const uint32_t c2 = A.count_control[2], c3 = A.count_control[3];
        A.count_control[4] = (c2 != 0u ? c3 : A.k) * A.count_tiles;
    }
    const uint32_t N = A.N;
    const uint32_t nrb = (N + 16 * NSUB - 1) / (16 * NSUB);
    FusedTables& F = *reinterpret_cast<FusedTables*>(ring);
    uint32_t n_tiles;
    uint32_t* addr_lds = reinterpret_cast<uint32_t*>(ring + (sizeof(FusedTables) + 15) / 16 * 16);
    if (FUSED && A.small_plan) {
        SmallPlan& S = F.plan;
        fused_small_plan(A.T, S, addr_lds, nrb, A.T.n_records > A.addr_lds_records);
        const uint32_t lo_rb = S.lo_rb, hi_rb = S.hi_rb, tile = S.tile;
        if (lo_rb >= hi_rb) return;
        TileSrc ts;
        ts.w[0] = reinterpret_cast<const uint8_t*>(S.ptr[0]);
        ts.s[0] = reinterpret_cast<const uint8_t*>(S.ptr[1]);
        ts.w[1] = reinterpret_cast<const uint8_t*>(S.ptr[2]);
        ts.s[1] = reinterpret_cast<const uint8_t*>(S.ptr[3]);
        ts.count = S.count;
        const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        const uint32_t rr = lane & 15, tl = 4 * (lane >> 4) + wave;
        ts.in_route = rr < ts.count ? S.route[rr] : 0u;
        const bool ov = wave < 4 && tl < ts.count;
        ts.out_route = ov ? S.route[tl] : 0u;
        ts.out_word = ov ? S.word[tl] : 0u;
        lds_drain();   // the plan is read before any copy can overwrite it
        stream_range<MODE, NMAT, NBUF, NW, NSUB, FUSED>(A, tile * nrb + lo_rb, tile * nrb + hi_rb, nrb, ts);
        return;
    }
    if (FUSED) {
        fused_tables<NW>(A.T, F, addr_lds);
        uint32_t te, tk;
        n_tiles = fused_tile_scan(F, A.T.E, ~0u, te, tk);
    } else {
        n_tiles = sload_u32(A.n_tiles);
    }
    auto tile_src = [&](uint32_t t) -> TileSrc {
        if (FUSED) return fused_tile<NW>(A, F, t);
        TileSrc ts;
        uint32_t begin, cnt;
        sload_rec(A.recs + t, begin, cnt, ts.w, ts.s);
        const u16s seg = sload_x16(A.seg_list + begin);
        const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        const uint32_t rr = lane & 15, tl = 4 * (lane >> 4) + wave;
        uint32_t in_r = 0, out_r = 0;
#pragma unroll
        for (uint32_t q = 0; q < 16; q++) {
            if (rr == q) in_r = seg[q];
            if (tl == q) out_r = seg[q];
        }
        ts.count = cnt;
        ts.in_route = in_r;
        ts.out_route = out_r;
        ts.out_word = (MODE == SPAN_DOWN && wave < 4 && tl < cnt) ? A.routes[out_r] : 0u;
        return ts;
    };
    // Work split that never crosses a tile inside a block when there are at
    // least as many blocks as tiles: tile t gets q or q + 1 blocks, which
    // split its row blocks evenly.  With fewer blocks than tiles a block
    // takes whole tiles (b, b + G, ...), each a separate range.
    const uint32_t G = gridDim.x, b = blockIdx.x;
    if (n_tiles == 0) return;
    if (G >= n_tiles) {
        uint32_t tile, lo_rb, hi_rb;
        block_share(G, b, n_tiles, nrb, tile, lo_rb, hi_rb);
        if (lo_rb >= hi_rb) return;
        const TileSrc ts = tile_src(tile);
        stream_range<MODE, NMAT, NBUF, NW, NSUB, FUSED>(A, tile * nrb + lo_rb, tile * nrb + hi_rb, nrb, ts);
    } else {
        for (uint32_t t = b; t < n_tiles; t += G) {
            // The tables share LDS with the ring: rebuild them after a range.
            if (FUSED && t != b) fused_tables<NW>(A.T, F, addr_lds);
            const TileSrc ts = tile_src(t);
            stream_range<MODE, NMAT, NBUF, NW, NSUB, FUSED>(A, t * nrb, (t + 1) * nrb, nrb, ts);
        }
    }
}

// Launches the streaming kernel, or returns UNSUPPORTED when the shape does
// not fit its LDS ring or copy-count limits (the caller then uses the span
// kernel).
template <int MODE, int NMAT, int NBUF, int NW, int NSUB, bool FUSED>
nerve_hip_status launch_stream(StreamArgs A, const nerve_hip_ctx* ctx, hipStream_t st) {
    constexpr uint32_t RI = 16 * NSUB;
    // Spans of at least one 1 KB weight piece and one 256 B scale piece.
    if (A.K > 4096 || A.K % 32 || RI * (A.K / 32) < 256) return NERVE_HIP_UNSUPPORTED;
    A.w_region = RI * (A.K / 2);
    A.s_region = RI * (A.K / 32);
    A.slot_bytes = NMAT * (A.w_region + A.s_region);
    const uint32_t npw = (A.w_region + 1023) / 1024, nps = (A.s_region + 255) / 256;
    A.lw = (npw + NW - 1) / NW;
    A.ls = (nps + NW - 1) / NW;
    A.copies_per_item = NMAT * (A.lw + A.ls);
    size_t lds = (size_t)2 * A.slot_bytes + (size_t)NW * NMAT * NSUB * 64 * 16;
    A.small_plan = FUSED && A.T.E <= 64 && A.T.batch_width * A.T.k <= 64 && ctx->cu_count >= 64 ? 1u : 0u;
    // The set-up tables and the staged address table share the ring's LDS
    // (short rings are extended to hold them, up to the LDS; the small plan
    // reads a larger table from memory instead).
    const size_t head = (sizeof(FusedTables) + 15) / 16 * 16;
    size_t tables = head + (size_t)A.T.n_records * 32;
    if (A.small_plan && tables > 160 * 1024) tables = head;
    if (FUSED && lds < tables) lds = tables;
    A.addr_lds_records = FUSED ? (uint32_t)((lds - head) / 32) : 0u;
    if (lds > 160 * 1024 || A.copies_per_item * 2 > 63) return NERVE_HIP_UNSUPPORTED;
    if (FUSED) {
        // Every compacted slot needs a thread in the tables, and activation
        // rows are read in 16-byte pieces.
        const uint32_t cap = A.T.batch_width * A.T.k;
        if (cap > 64 * NW || cap > FUSED_MAX_SLOTS || A.T.E > FUSED_MAX_EXPERTS || A.T.E > 64 * NW || A.T.P > 4 ||
            ((uintptr_t)A.x16 & 15) || A.x_frame % 8 || A.x_seg % 8 ||
            (A.T.n_records > A.addr_lds_records && !A.small_plan) ||   // the small plan reads a big table from memory
            ((uintptr_t)A.T.addr & 15))
            return NERVE_HIP_UNSUPPORTED;
    }
    static bool attr_set = false;
    if (!attr_set) {
        if (hipFuncSetAttribute((const void*)mx_stream_kernel<MODE, NMAT, NBUF, NW, NSUB, FUSED>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess)
            return nh::fail(NERVE_HIP_DEVICE_ERROR, "hipFuncSetAttribute failed for mx_stream_kernel");
        attr_set = true;
    }
    mx_stream_kernel<MODE, NMAT, NBUF, NW, NSUB, FUSED><<<ctx->cu_count, 64 * NW, lds, st>>>(A);
    return nh::check_launch("mx_stream_kernel");
}

// ---------------------------------------------------------------------------
// Decode gate/up in token form (at most 16 tokens, 64 experts, 64 routes).
//
// A route's gate/up activations are its token's hidden row, so the MFMA's 16
// activation rows are simply the batch's tokens: every active expert's weight
// rows are contracted against all tokens, and the epilogue writes the rows of
// the (token, slot) routes that select that expert.  The activations then do
// not depend on the routing, which takes the route tables off the critical
// path: wave 0 alone loads the routing inputs and builds the plan while waves
// 1.. load and quantize their K chunks of all tokens.  A work item is 16 rows
// of gate and up of one active expert; items are numbered expert-major and
// every block takes an equal contiguous share (no tiles, so shares may cross
// experts at no cost).  The streaming loop is the stream kernel's: a ring of
// NBUF LDS slots fed by global_load_lds, a fixed number of copies per wave
// and item, explicit vmcnt waits and an LDS cross-wave reduction.
// ---------------------------------------------------------------------------
constexpr uint32_t TOK_MAX_TOKENS = 16;
constexpr uint32_t TOK_MAX_EXPERTS = 64;

struct TokPlan {
    uint64_t ptr[TOK_MAX_EXPERTS][4];             // parameter pointers of active expert u
    uint32_t mask[TOK_MAX_EXPERTS][TOK_MAX_TOKENS];  // bit j: slot j of token t selects active expert u
    uint32_t flag[TOK_MAX_EXPERTS];                  // scratch: expert e has a valid slot
    uint32_t n_act;
};
constexpr uint32_t TOK_MAX_RECORDS = 512;            // address table staged by wave 0 in one round

// The body is a device function: the host pass instantiates kernel template
// bodies, and the gfx950-only builtins below would fail there.
template <int NBUF, int NW>
__device__ __forceinline__ void mx_tokens_body(const StreamArgs& A) {
    constexpr uint32_t RI = 16, NMAT = 2, NSUB = 1;
    constexpr uint32_t CH = 24 / NW;                              // chunks per wave (K <= NW CH 128)
    constexpr uint32_t LWMAX = (32 * NSUB + NW - 1) / NW;
    constexpr uint32_t LSMAX = (8 * NSUB + NW - 1) / NW;
    extern __shared__ __attribute__((aligned(16))) uint8_t ring[];
    TokPlan& S = *reinterpret_cast<TokPlan*>(ring);
    uint32_t* addr_lds = reinterpret_cast<uint32_t*>(ring + (sizeof(TokPlan) + 15) / 16 * 16);
    const TileArgs& T = A.T;
    const uint32_t tid = threadIdx.x, lane = tid & 63, g = lane >> 4, rr = lane & 15;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t K = A.K, N = A.N, RB = K / 2, SB = K / 32, nch = (K + 127) / 128;
    const uint32_t nrb = (N + RI - 1) / RI;
    const uint32_t B = T.batch_width, kr = T.k, cap = B * kr, E = T.E, P = T.P;
    // All waves split the K chunks; wave 0 also builds the plan (and loads
    // its activations after it).
    const uint32_t per = (nch + NW - 1) / NW;
    const uint32_t c0 = min(nch, wave * per), c1 = min(nch, c0 + per);
    const bool row_ok = rr < B;

    // ---- activations: token rr's pieces of this wave's chunks (inline-asm
    // loads, absent pieces from the row start and zeroed after the wait).
    v4i xb[CH][4];
    auto piece_ok = [&](uint32_t q, int h) __attribute__((always_inline)) {
        const uint32_t c = c0 + q, k0 = c * 128 + g * 16 + (h >= 2 ? 64u : 0u);
        return row_ok && c < c1 && k0 < K;
    };
    // ---- wave 0's routing inputs and address table go to memory first, so
    // they are not queued behind the activation loads of the other waves.
    const uint32_t n16 = 2 * T.n_records;
    // A table past TOK_MAX_RECORDS (a package-wide one) is not staged: the
    // plan reads its experts' records from memory after the slot words.
    const bool big_table = T.n_records > TOK_MAX_RECORDS;
    uint32_t sl[4] = {UNBOUND_SLOT, UNBOUND_SLOT, UNBOUND_SLOT, UNBOUND_SLOT};
    uint32_t r = 0, rt = 0, c2 = 0, c3 = 0;
    v4i tab[TOK_MAX_RECORDS * 2 / 64];
    if (wave == 0) {
#pragma unroll
        for (uint32_t p = 0; p < 4; p++) {
            const uint32_t idx = lane * P + p;
            if (lane < E && p < P && idx < T.n_slot_words) sl[p] = T.slots[idx];
        }
        r = lane < cap ? T.frames[(uint64_t)(lane / kr) * T.frame_words + T.data_words + lane % kr] : 0u;
        rt = lane < cap ? T.routes[lane] : 0u;
        c2 = T.control[2];
        c3 = T.control[3];
        const v4i* src = reinterpret_cast<const v4i*>(T.addr);
#pragma unroll
        for (uint32_t j = 0; j < TOK_MAX_RECORDS * 2 / 64; j++) {
            const uint32_t i = j * 64 + lane;
            tab[j] = i < n16 && !big_table ? src[i] : v4i{0, 0, 0, 0};
        }
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    const bool preq = A.aq != nullptr;   // wave-uniform: prequantized e4m3 rows + pow2 block scales
    auto act_loads = [&]() __attribute__((always_inline)) {
    if (!preq) {
        const uint16_t* xr = A.x16 + (uint64_t)(row_ok ? rr : 0u) * A.x_frame;
#pragma unroll
        for (uint32_t q = 0; q < CH; q++) {
            if (c0 + q >= c1) continue;
#pragma unroll
            for (int h = 0; h < 4; h++) {
                const uint32_t off = (c0 + q) * 128 + g * 16 + (h >= 2 ? 64u : 0u) + (h & 1 ? 8u : 0u);
                xb[q][h] = gload16_untracked(xr + (piece_ok(q, h) ? off : 0u));
            }
        }
    } else {
        // Prequantized hidden rows (PREQUANTIZED_INPUT): the operand pieces
        // are the e4m3 bytes k = 16 g.. and 64 + 16 g.. of the chunk, the
        // scale is the row's f32 block scale (its exponent is the e8m0).
        const uint8_t* xr = A.aq + (uint64_t)(row_ok ? rr : 0u) * K;
        const float* sr = A.as + (uint64_t)(row_ok ? rr : 0u) * nch;
#pragma unroll
        for (uint32_t q = 0; q < CH; q++) {
            if (c0 + q >= c1) continue;
            const uint32_t off = (c0 + q) * 128 + g * 16;
            xb[q][0] = gload16_untracked(xr + (piece_ok(q, 0) ? off : 0u));
            xb[q][1] = gload16_untracked(xr + (piece_ok(q, 2) ? off + 64u : 0u));
            xb[q][2].x = (int)gload4_untracked(sr + c0 + q);
        }
    }
    };
    if (wave != 0) act_loads();
    v8i av[CH];
    uint32_t sa[CH];
    if (wave == 0) {
        // ---- the plan: the same validity rules as fused_tables.
        if (!big_table) {
            v4i* dst = reinterpret_cast<v4i*>(addr_lds);
#pragma unroll
            for (uint32_t j = 0; j < TOK_MAX_RECORDS * 2 / 64; j++) {
                const uint32_t i = j * 64 + lane;
                if (i < n16) dst[i] = tab[j];
            }
        }
        {
            v4i* mz = reinterpret_cast<v4i*>(&S.mask[0][0]);
#pragma unroll
            for (uint32_t j = 0; j < TOK_MAX_EXPERTS * TOK_MAX_TOKENS / 4 / 64; j++) mz[j * 64 + lane] = v4i{0, 0, 0, 0};
            S.flag[lane] = 0;
        }
        // Records of expert `lane` (a wave's LDS accesses complete in order),
        // or from memory for a table that was not staged.
        v4i lo[4], hi[4];
        if (big_table) {
#pragma unroll
            for (uint32_t p = 0; p < 4; p++) {
                const bool has = sl[p] != UNBOUND_SLOT && sl[p] < T.n_records;
                const v4i* rp = reinterpret_cast<const v4i*>(T.addr + (uint64_t)(has ? sl[p] : 0u) * 8);
                lo[p] = rp[0];
                hi[p] = rp[1];
            }
        } else {
#pragma unroll
            for (uint32_t p = 0; p < 4; p++) {
                const bool has = sl[p] != UNBOUND_SLOT && sl[p] < T.n_records;
                const v4i* rp = reinterpret_cast<const v4i*>(addr_lds + (has ? sl[p] : 0u) * 8);
                lo[p] = rp[0];
                hi[p] = rp[1];
            }
        }
        bool valid = lane < E;
        uint64_t ptr[4];
#pragma unroll
        for (uint32_t p = 0; p < 4; p++) {
            const bool has = sl[p] != UNBOUND_SLOT && sl[p] < T.n_records;
            uint32_t rec[8];
#pragma unroll
            for (uint32_t j = 0; j < 4; j++) {
                rec[j] = has ? (uint32_t)lo[p][j] : 0u;
                rec[4 + j] = has ? (uint32_t)hi[p][j] : 0u;
            }
            if (p < P) {
                const bool is_weight = (p % 2) == 0;
                valid = record_valid(sl[p], T.n_records, rec, is_weight ? T.req_w : T.req_s, is_weight ? 16u : 4u) && valid;
            }
            ptr[p] = (uint64_t)rec[0] | ((uint64_t)rec[1] << 32);
        }
        const uint64_t vmask = __ballot(valid);
        // Slot `lane`: route r, its word, expert and validity.
        uint32_t n = c2 != 0u ? c3 : cap;
        if (n > cap) n = cap;
        // Every lane takes part in the shuffle (a lane reading from an inactive
        // lane gets 0), and the out-of-range routes are dropped afterwards.
        const uint32_t wsh = (uint32_t)__shfl((int)rt, (int)(r & 63u));
        const uint32_t w = r < cap ? wsh : 0u;
        const uint32_t e = w & 0xffffu;
        const bool ok = lane < n && r < cap && e < E && ((vmask >> (e & 63u)) & 1ull);
        // Active experts (at least one valid slot), numbered in expert order
        // (a wave's LDS accesses complete in order).
        if (ok) S.flag[e] = 1u;
        const uint64_t act = __ballot(lane < E && S.flag[lane] != 0u);
        const uint64_t below = (1ull << lane) - 1ull;
        const uint32_t u_of_lane = (uint32_t)__popcll(act & below);          // lane as an expert id
        const uint32_t u = (uint32_t)__shfl((int)u_of_lane, (int)(e & 63u)); // active index of this slot's expert
        if (ok) atomicOr(&S.mask[u][r / kr], 1u << (r % kr));
        if ((act >> lane) & 1ull) {
#pragma unroll
            for (uint32_t p = 0; p < 4; p++) S.ptr[u_of_lane][p] = ptr[p];
        }
        if (lane == 0) S.n_act = (uint32_t)__popcll(act);
        // Wave 0's activation loads go out after the plan's (the compiler's
        // waits for the plan's loads would otherwise also wait for them).
        act_loads();
    }
    __syncthreads();
    // ---- this block's share of the items, and the (at most two) experts it spans
    const uint32_t n_act = S.n_act;
    const uint64_t total = (uint64_t)n_act * nrb;
    const uint32_t i0 = (uint32_t)(total * blockIdx.x / gridDim.x), i1 = (uint32_t)(total * (blockIdx.x + 1) / gridDim.x);
    if (i0 >= i1) return;
    const uint32_t u0 = i0 / nrb;
    const uint32_t u1 = min(u0 + 1, n_act - 1);
    const uint8_t* wp[2][2];
    const uint8_t* sp[2][2];
    wp[0][0] = reinterpret_cast<const uint8_t*>(S.ptr[u0][0]);
    sp[0][0] = reinterpret_cast<const uint8_t*>(S.ptr[u0][1]);
    wp[0][1] = reinterpret_cast<const uint8_t*>(S.ptr[u0][2]);
    sp[0][1] = reinterpret_cast<const uint8_t*>(S.ptr[u0][3]);
    wp[1][0] = reinterpret_cast<const uint8_t*>(S.ptr[u1][0]);
    sp[1][0] = reinterpret_cast<const uint8_t*>(S.ptr[u1][1]);
    wp[1][1] = reinterpret_cast<const uint8_t*>(S.ptr[u1][2]);
    sp[1][1] = reinterpret_cast<const uint8_t*>(S.ptr[u1][3]);
    // Output token of this lane (waves 0..3 finalize component `wave`).
    const uint32_t tok = 4 * g + (wave & 3u);
    const uint32_t om0 = wave < 4 ? S.mask[u0][tok] : 0u, om1 = wave < 4 ? S.mask[u1][tok] : 0u;
    lds_drain();   // the plan is read before any copy can overwrite it
    __builtin_amdgcn_s_barrier();

    uint8_t* red = ring + 2 * A.slot_bytes;   // [wave][NMAT][lane] v4f partial sums
    const uint32_t npw = (RI * RB + 1023) / 1024, nps = (RI * SB + 255) / 256;
    const uint32_t lw = A.lw, ls = A.ls;
    uint32_t wpos[LWMAX], spos[LSMAX], woff[LWMAX], soff[LSMAX];
#pragma unroll
    for (uint32_t q = 0; q < LWMAX; q++) {
        uint32_t pc = wave + NW * q;
        if (pc >= npw) pc = wave < npw ? wave : 0;
        wpos[q] = min(pc * 1024, RI * RB - 1024);
        woff[q] = wpos[q] + lane * 16;
    }
#pragma unroll
    for (uint32_t q = 0; q < LSMAX; q++) {
        uint32_t pc = wave + NW * q;
        if (pc >= nps) pc = wave < nps ? wave : 0;
        spos[q] = min(pc * 256, RI * SB - 256);
        soff[q] = spos[q] + lane * 4;
    }
    // Item i: expert index i / nrb (u0 or u0 + 1), rows (i % nrb) * 16.
    // Its weight and scale bytes are loaded with nontemporal loads into a
    // register set (the same 1 KB / 256 B pieces per wave as a ring slot's
    // layout) and written to an LDS slot when the item comes up: streaming
    // reads from registers sustain ~7 TB/s over the chip where copies
    // straight into LDS (global_load_lds) sustain ~6.1.
    struct ItemRegs {
        v4i w[NMAT][LWMAX];
        uint32_t s[NMAT][LSMAX];
    };
    auto load_item = [&](uint32_t item, ItemRegs& R) __attribute__((always_inline)) {
        const uint32_t second = item / nrb != u0 ? 1u : 0u;
        const uint32_t n0 = (item - (u0 + second) * nrb) * RI;
        const uint32_t rows = min(RI, N - n0);
        const uint32_t wbytes = rows * RB, sbytes = rows * SB;
#pragma unroll
        for (uint32_t m = 0; m < NMAT; m++) {
            const uint8_t* ws = (second ? wp[1][m] : wp[0][m]) + (uint64_t)n0 * RB;
#pragma unroll
            for (uint32_t q = 0; q < LWMAX; q++)
                if (q < lw) R.w[m][q] = gload16_nt_untracked(ws + (woff[q] < wbytes ? woff[q] : 0));
            const uint8_t* ss = (second ? sp[1][m] : sp[0][m]) + (uint64_t)n0 * SB;
#pragma unroll
            for (uint32_t q = 0; q < LSMAX; q++)
                if (q < ls) R.s[m][q] = gload4_nt_untracked(ss + (soff[q] < sbytes ? soff[q] : 0));
        }
    };
    auto store_item = [&](const ItemRegs& R, uint32_t slot) __attribute__((always_inline)) {
        uint8_t* dst = ring + slot * A.slot_bytes;
#pragma unroll
        for (uint32_t m = 0; m < NMAT; m++) {
#pragma unroll
            for (uint32_t q = 0; q < LWMAX; q++)
                if (q < lw) *reinterpret_cast<v4i*>(dst + m * A.w_region + woff[q]) = R.w[m][q];
#pragma unroll
            for (uint32_t q = 0; q < LSMAX; q++)
                if (q < ls) *reinterpret_cast<uint32_t*>(dst + NMAT * A.w_region + m * A.s_region + soff[q]) = R.s[m][q];
        }
    };
    uint32_t rw[CH], rs[CH];
    bool kvalid[CH];
#pragma unroll
    for (uint32_t q = 0; q < CH; q++) {
        const uint32_t c = c0 + q, kb = c * 128 + g * 32;
        kvalid[q] = c < c1 && kb < K;
        const uint32_t kk = kvalid[q] ? kb : 0;
        rw[q] = rr * RB + kk / 2;
        rs[q] = NMAT * A.w_region + rr * SB + kk / 32;
    }

    // Prologue: the first item's loads, then the quantization while they
    // stream, then the second item's (issuing more up front stalls the wave
    // at issue until the CU's miss queue drains).
    ItemRegs R0{}, R1{};
    load_item(i0, R0);
    {
        // ---- quantize this wave's chunks of all tokens: loads retire in
        // issue order, so once only the first item's loads are in flight
        // the activations have landed.
        wait_vm(A.copies_per_item);
#pragma unroll
        for (uint32_t q = 0; q < CH; q++) {
            if (c0 + q >= c1) {
                av[q] = v8i{0, 0, 0, 0, 0, 0, 0, 0};
                sa[q] = 127u;
                continue;
            }
            if (preq) {
                asm volatile("" : "+v"(xb[q][0]), "+v"(xb[q][1]), "+v"(xb[q][2]));
                const v4i lo = piece_ok(q, 0) ? xb[q][0] : v4i{0, 0, 0, 0};
                const v4i hi = piece_ok(q, 2) ? xb[q][1] : v4i{0, 0, 0, 0};
                av[q] = v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
                sa[q] = row_ok ? pow2_to_e8m0(__int_as_float(xb[q][2].x)) : 127u;
                continue;
            }
#pragma unroll
            for (int h = 0; h < 4; h++) {
                asm volatile("" : "+v"(xb[q][h]));
                if (!piece_ok(q, h)) xb[q][h] = v4i{0, 0, 0, 0};
            }
            uint32_t e8;
            quant_chunk_e4m3(xb[q], av[q], e8);
            sa[q] = row_ok ? e8 : 127u;
        }
    }
    if (i0 + 1 < i1) load_item(i0 + 1, R1);

    // One item: its registers go to LDS slot `slot` (last read by the item
    // two back, whose reduction barrier every wave has passed), the item two
    // ahead is loaded into the same registers, a barrier, then the
    // contraction and the cross-wave reduction.  (Three items in flight
    // measured slower: 49.3 against 47.8 us at config 2.)
    auto item_step = [&](uint32_t i, ItemRegs& R) __attribute__((always_inline)) {
        const uint32_t slot = (i - i0) & 1u;
        // Loads retire in issue order: with only the next item's loads
        // allowed in flight this item's have landed.
        wait_vm(i + 1 < i1 ? A.copies_per_item : 0u);
#pragma unroll
        for (uint32_t m = 0; m < NMAT; m++) {
#pragma unroll
            for (uint32_t q = 0; q < LWMAX; q++) asm volatile("" : "+v"(R.w[m][q]));
#pragma unroll
            for (uint32_t q = 0; q < LSMAX; q++) asm volatile("" : "+v"(R.s[m][q]));
        }
        store_item(R, slot);
        if (i + 2 < i1) load_item(i + 2, R);
        __syncthreads();
        const uint32_t second = i / nrb != u0 ? 1u : 0u;
        const uint32_t n0 = (i - (u0 + second) * nrb) * RI;
        const uint8_t* buf = ring + slot * A.slot_bytes;
        v4f acc[NMAT];
#pragma unroll
        for (uint32_t m = 0; m < NMAT; m++) acc[m] = v4f{0.f, 0.f, 0.f, 0.f};
        if (c0 < c1) {
#pragma unroll
            for (uint32_t q0 = 0; q0 < CH; q0 += 4) {
                if (c0 + q0 >= c1) continue;
                v4i w[4][NMAT];
                uint32_t sw[4][NMAT];
#pragma unroll
                for (uint32_t q = 0; q < 4; q++)
#pragma unroll
                    for (uint32_t m = 0; m < NMAT; m++) {
                        w[q][m] = lds_read16(buf + m * A.w_region + rw[q0 + q]);
                        sw[q][m] = lds_read_u8(buf + m * A.s_region + rs[q0 + q]);
                    }
                lds_drain();
#pragma unroll
                for (uint32_t q = 0; q < 4; q++) {
                    if (c0 + q0 + q >= c1) continue;
#pragma unroll
                    for (uint32_t m = 0; m < NMAT; m++) {
                        v4i wv = w[q][m];
                        uint32_t s8 = sw[q][m];
                        asm volatile("" : "+v"(wv), "+v"(s8));
                        if (!kvalid[q0 + q]) {
                            wv = v4i{0, 0, 0, 0};
                            s8 = 127;
                        }
                        acc[m] = mfma_fp8_fp4(av[q0 + q], wv, sa[q0 + q], s8, acc[m]);
                    }
                }
            }
        }
        // Software wait states between the last MFMA and the inline-asm LDS
        // write of its result (see stream_range).
#pragma unroll
        for (uint32_t m = 0; m < NMAT; m++) asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(acc[m]));
#pragma unroll
        for (uint32_t m = 0; m < NMAT; m++) lds_write16(red + ((wave * NMAT + m) * 64 + lane) * 16, acc[m]);
        lds_drain();
        __builtin_amdgcn_s_barrier();
        if (wave < 4) {
            const uint32_t om = second ? om1 : om0;
            float tsum[NMAT];
#pragma unroll
            for (uint32_t m = 0; m < NMAT; m++) {
                uint32_t v[NW];
#pragma unroll
                for (uint32_t w2 = 0; w2 < NW; w2++)
                    v[w2] = lds_read_b32(red + ((w2 * NMAT + m) * 64 + lane) * 16 + 4 * wave);
                lds_drain();
                float sum = 0.0f;
#pragma unroll
                for (uint32_t w2 = 0; w2 < NW; w2++) {
                    asm volatile("" : "+v"(v[w2]));
                    sum += __uint_as_float(v[w2]);
                }
                tsum[m] = sum;
            }
            const uint32_t nrow = n0 + rr;
            if (om != 0u && nrow < N) {
                float gv = round_bf16(tsum[0]);
                float uv = round_bf16(tsum[1]);
                if (A.limit > 0.0f) {
                    gv = fminf(gv, A.limit);
                    uv = fminf(fmaxf(uv, -A.limit), A.limit);
                }
                const uint16_t h = (uint16_t)f32_to_bf16(silu_fast(gv) * uv);
                for (uint32_t bits = om; bits; bits &= bits - 1u) {
                    const uint32_t j = (uint32_t)__builtin_ctz(bits);
                    A.out16[(uint64_t)tok * A.frame_elems + (uint64_t)j * N + nrow] = h;
                }
            }
        }
    };
    for (uint32_t i = i0; i < i1; i += 2) {
        item_step(i, R0);
        if (i + 1 < i1) item_step(i + 1, R1);
    }
}

template <int NBUF, int NW>
__global__ __launch_bounds__(64 * NW) void mx_tokens_kernel(StreamArgs A) {
    mx_tokens_body<NBUF, NW>(A);
}

// Launches the token-form gate/up kernel, or returns UNSUPPORTED when the
// batch or the shape does not fit it.
template <int NBUF, int NW>
nerve_hip_status launch_tokens(StreamArgs A, const nerve_hip_ctx* ctx, hipStream_t st) {
    constexpr uint32_t RI = 16, CH = 24 / NW;
    const uint32_t nch = (A.K + 127) / 128;
    if (A.T.batch_width > TOK_MAX_TOKENS || A.T.E > TOK_MAX_EXPERTS || A.T.batch_width * A.T.k > 64 || A.T.P != 4 ||
        A.K % 32 || A.K > 4096 || (nch + NW - 1) / NW > CH || RI * (A.K / 32) < 256 || A.x_seg != 0 ||
        ((uintptr_t)A.x16 & 15) || A.x_frame % 8 || ((uintptr_t)A.T.addr & 15) || A.T.k > 32 ||
        (uint32_t)ctx->cu_count < A.T.E)   // >= E blocks: a block's share spans at most two experts
        return NERVE_HIP_UNSUPPORTED;
    A.w_region = RI * (A.K / 2);
    A.s_region = RI * (A.K / 32);
    A.slot_bytes = 2 * (A.w_region + A.s_region);
    const uint32_t npw = (A.w_region + 1023) / 1024, nps = (A.s_region + 255) / 256;
    A.lw = (npw + NW - 1) / NW;
    A.ls = (nps + NW - 1) / NW;
    A.copies_per_item = 2 * (A.lw + A.ls);
    const size_t lds = (size_t)2 * A.slot_bytes + (size_t)NW * 2 * 64 * 16;
    const size_t plan = (sizeof(TokPlan) + 15) / 16 * 16 + (A.T.n_records > TOK_MAX_RECORDS ? 0 : (size_t)A.T.n_records * 32);
    if (lds > 160 * 1024 || plan > lds || A.copies_per_item * 2 > 63) return NERVE_HIP_UNSUPPORTED;
    static bool attr_set = false;
    if (!attr_set) {
        if (hipFuncSetAttribute((const void*)mx_tokens_kernel<NBUF, NW>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                160 * 1024) != hipSuccess)
            return nh::fail(NERVE_HIP_DEVICE_ERROR, "hipFuncSetAttribute failed for mx_tokens_kernel");
        attr_set = true;
    }
    mx_tokens_kernel<NBUF, NW><<<ctx->cu_count, 64 * NW, lds, st>>>(A);
    return nh::check_launch("mx_tokens_kernel");
}

// ---------------------------------------------------------------------------
// Persistent grouped GEMM for prefill-shaped batches.
//
// Work item = (tile of <= 128 routes of one expert, block of 256 weight rows).
// For gate_up the 256 rows are 128 gate and 128 up rows of the same channels,
// so SwiGLU runs on the accumulators.  The preparation launch lists the items
// as (expert, row block, tile) with tiles fastest; every block takes every
// G-th item, with consecutive items on blocks of one XCD, so the tiles of one
// expert at one row block run side by side and read the same weight rows
// while they are in that XCD's L2.
//
// One 512-thread block per CU.  Each wave owns 32 of the item's weight rows
// (gate_up: 16 gate + the same 16 up channels) and contracts them against
// all of the tile's routes, so a weight byte is used by one wave only: the
// weights go from global memory straight into that wave's registers (16-byte
// loads in the MFMA's operand layout, three chunks in flight per wave), with
// no LDS round trip.  The activations (128 routes x 256 B
// e4m3 per 256-k chunk), the rows' e8m0 scale bytes and the routes' block
// scales are shared by all waves: they go global -> LDS with global_load_lds
// into a 3-stage ring that runs across item boundaries.  Per CU that keeps
// ~130 KB of weight and activation bytes in flight, and 256-row items read
// each route's activations once per 256 rows.
//
// Every wave issues a fixed set of copies and loads per stage (an SGPR base
// advanced per chunk plus fixed 32-bit lane offsets), so the vmcnt waits
// count them per stage; one barrier per chunk; the step body is unrolled
// over the 3 stages so every LDS operand read is a fixed register plus an
// immediate offset and every weight register set is a fixed variable.  The
// next item's descriptor (item record, then its tile's route list) also
// arrives by LDS copies issued by wave 0 inside the same pipeline.
// ---------------------------------------------------------------------------
constexpr uint32_t PG_TM = PG_TILE;
constexpr uint32_t PG_ROWS = 256;         // weight rows per item (gate_up: 128 gate + 128 up)
constexpr uint32_t PG_NST = 3;
constexpr uint32_t PG_KC = 256;           // k per chunk
// LDS map (bytes).  Regions are grouped by kind so a stage is an immediate.
constexpr uint32_t PG_A_OFF = 0;          // [3][128 routes][256 B], 16-byte pieces XOR-swizzled by route
constexpr uint32_t PG_SA_OFF = 98304;     // [3][128 routes][2] f32 block scales
constexpr uint32_t PG_REC_OFF = 101376;   // [2][256 B] item records (48 B used)
constexpr uint32_t PG_LIST_OFF = 101888;  // [2][2 KB] tile route lists
constexpr uint32_t PG_SPAN_OFF = 105984;  // [2][256 rows][K / 32 B]: the item's e8m0 scale rows, by item parity
// LDS bytes of a launch for contraction length K (the scale spans grow with K).
__host__ __device__ constexpr uint32_t pg_lds_bytes(uint32_t K) { return PG_SPAN_OFF + 2 * PG_ROWS * (K / 32); }
constexpr uint32_t PG_COPIES = 5;         // per-chunk LDS copy slots per wave
constexpr uint32_t PG_WLOADS = 4;         // weight register loads per wave per stage
// The item record rides on chunk 2's copies, the route list on chunk 4's,
// and the next item's copies are set up when chunk nch - 1 is issued (at
// chunk nch - 3), so an item needs at least 7 chunks.
constexpr uint32_t PG_MIN_CHUNKS = 7;

__device__ __attribute__((aligned(16))) const uint8_t kZeroPage[1024] = {0};

struct PgArgs {
    const uint8_t* aq;          // e4m3 activations, row stride lda
    uint32_t lda;               // K, or K rounded up to 128 so every 128-k chunk of a row is one cache line
    const float* as;            // pow2 scales, row stride ceil(K / 128)
    uint32_t K, N, k;
    const ItemRec* items;
    const PgList* lists;
    const uint32_t* n_tiles;
    uint16_t* out;              // gate_up: frames as u16; down: expert_outputs
    uint64_t frame_elems;
    float limit;
    uint32_t a_rows;            // activation rows (aq / as); list rows are clamped below it
    uint32_t routes;            // route slots (batch_width * k); larger route ids are skipped
};

template <uint32_t OFF>
__device__ __forceinline__ uint32_t lds_rd8(uint32_t a) {
    uint32_t r;
    asm volatile("ds_read_u8 %0, %1 offset:%2" : "=v"(r) : "v"(a), "i"(OFF));
    return r;
}
template <uint32_t OFF>
__device__ __forceinline__ v2i lds_rd64(uint32_t a) {
    v2i r;
    asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(r) : "v"(a), "i"(OFF));
    return r;
}

// 16-byte LDS read at any offset below 128 KiB (the immediate field holds 16 bits).
template <uint32_t OFF>
__device__ __forceinline__ v4i lds_rd128_far(uint32_t a) {
    if constexpr (OFF >= 65536u) return lds_rd128<OFF - 65536u>(a + 65536u);
    else return lds_rd128<OFF>(a);
}

// Item row of a wave's weight subtile j (16 rows): gate_up waves take gate
// rows 16 w.. and the same up channels (item rows 128 + 16 w..), down waves
// rows 32 w + 16 j...
template <int NMAT>
__host__ __device__ constexpr uint32_t pg_irow(uint32_t wave, uint32_t j) {
    return NMAT == 2 ? j * 128 + 16 * wave : 32 * wave + 16 * j;
}

// LDS dword read that waits for itself inside the same asm statement, so
// no use of the result can be scheduled ahead of the wait.
template <uint32_t OFF>
__device__ __forceinline__ uint32_t lds_rd32_sync(uint32_t a) {
    uint32_t r;
    asm volatile("ds_read_b32 %0, %1 offset:%2\n\ts_waitcnt lgkmcnt(0)" : "=v"(r) : "v"(a), "i"(OFF));
    return r;
}

// Issue-side state of the item whose chunks are being copied and loaded.
struct PgIssue {
    const uint8_t* sp[2];       // uniform: scale span of each matrix part of the item
    const uint8_t* wb[2];       // uniform: weight matrices of the wave's subtiles
    uint32_t off[PG_COPIES];    // per lane: copy source offsets
    uint32_t woff[2];           // per lane: weight row offset of subtile j (+ 16 g)
    uint32_t tail_ok;           // per lane: bit i = copy slot i lies inside K in the last chunk;
                                //   bits 8 + 2 j + h: weight piece (j, h) does
    uint32_t on;                // uniform: bit i = copy slot i is issued (routes that exist)
    uint32_t n;                 // uniform: copies + loads per chunk
    uint32_t slen[2];           // uniform: scale span bytes of each part
    uint32_t np0;               // uniform: 256-byte span pieces of part 0
    uint32_t nspan;             // uniform: this wave's span pieces (issued with chunk 0)
};

// Weight register set of one chunk: subtile j (0, 1), half h (0, 1).
struct PgW {
    v4i w[2][2];
};

// Items [i0, n_items) of one route-count group, NA route subtiles per tile.
template <int NMAT, int NA>
__device__ __forceinline__ void pg_range(const PgArgs& A, uint32_t i0, uint32_t n_items) {
    extern __shared__ __attribute__((aligned(16))) uint8_t pg_ring[];
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t g = lane >> 4, rr = lane & 15;
    const uint32_t K = A.K, N = A.N, RB = K / 2, SB = K / 32, nch = (K + PG_KC - 1) / PG_KC;
    const uint32_t nsa = (K + 127) / 128;             // activation scales per row
    constexpr uint32_t RPM = PG_ROWS / NMAT;           // rows per matrix in an item
    const uint32_t G = gridDim.x;
    const uint32_t ring = lds_addr(pg_ring);

    // ---- descriptor copies (wave 0): item record, then the tile's list ----
    auto copy_rec = [&](uint32_t item, uint32_t par) __attribute__((always_inline)) {
        const uint32_t idx = item < n_items ? item : i0;
        const uint32_t* src = reinterpret_cast<const uint32_t*>(A.items + idx) + (lane < 12 ? lane : 0);
        __builtin_amdgcn_global_load_lds(src, pg_ring + PG_REC_OFF + par * 256, 4, 0, 0);
    };
    auto copy_list = [&](uint32_t par) __attribute__((always_inline)) {
        const uint32_t tile = lds_rd32_sync<0>(ring + PG_REC_OFF + par * 256 + 8);
        const uint8_t* src = reinterpret_cast<const uint8_t*>(A.lists + __builtin_amdgcn_readfirstlane(tile)) + lane * 16;
        __builtin_amdgcn_global_load_lds(src, pg_ring + PG_LIST_OFF + par * 2048, 16, 0, 0);
        __builtin_amdgcn_global_load_lds(src + 1024, pg_ring + PG_LIST_OFF + par * 2048 + 1024, 16, 0, 0);
    };
    auto rec_word = [&](uint32_t par, uint32_t w) __attribute__((always_inline)) -> uint32_t {
        const uint32_t v = lds_rd32_sync<0>(ring + PG_REC_OFF + par * 256 + 4 * w);
        return __builtin_amdgcn_readfirstlane(v);
    };
    auto rec_ptr = [&](uint32_t par, uint32_t w) __attribute__((always_inline)) -> const uint8_t* {
        const uint64_t lo = rec_word(par, w), hi = rec_word(par, w + 1);
        return reinterpret_cast<const uint8_t*>(lo | (hi << 32));
    };

    // ---- issue side: set-up of an item's copies (after its descriptor landed) ----
    // Copy slots: 0-3 = activations of routes 32 i + 4 w.. (four 256-byte
    // rows per copy); 4, 5 = scale dwords of the wave's subtiles (16 rows x
    // 4 dwords); 6 = block scales of routes 32 w.. (waves 0-3).  Loads:
    // weight pieces (j, h) of the wave's two subtiles.
    auto setup_issue = [&](uint32_t par, PgIssue& S) __attribute__((always_inline)) {
        const uint32_t rb = rec_word(par, 0), count = rec_word(par, 1);
        const uint8_t* wp[2] = {rec_ptr(par, 4), rec_ptr(par, 6)};
        const uint8_t* sp[2] = {rec_ptr(par, 8), rec_ptr(par, 10)};
        const uint32_t list = ring + PG_LIST_OFF + par * 2048;
        const uint32_t last = nch - 1;
        uint32_t tail = 0, on = 0;
        // activations
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) {
            const uint32_t t = 32 * i + 4 * wave + (lane >> 4);
            const uint32_t p = (lane & 15) ^ (t & 15);
            const uint32_t row = lds_rd32_sync<512>(list + 4 * (t < count ? t : 0));
            S.off[i] = row * A.lda + p * 16;
            tail |= (last * PG_KC + p * 16 < K ? 1u : 0u) << i;
            on |= (32 * i + 4 * wave < count ? 1u : 0u) << i;
        }
        // the item's scale rows: per matrix part, the span of its existing
        // rows (contiguous in the package layout), copied once per item in
        // 256-byte pieces, the last one aligned to the span's end
        {
            uint32_t np = 0;
#pragma unroll
            for (uint32_t m = 0; m < (uint32_t)NMAT; m++) {
                const uint32_t rows = min(RPM, N - rb * RPM);
                S.sp[m] = sp[m] + (uint64_t)rb * RPM * SB;
                S.slen[m] = rows * SB;
                np += (rows * SB + 255) / 256;
                if (m == 0) S.np0 = np;
            }
            S.nspan = np > wave ? (np - wave + 7) / 8 : 0u;
        }
        // activation block scales: LDS word 2 t + h holds route t, block 2 c + h
        if (wave < 4) {
            const uint32_t t = 32 * wave + (lane >> 1), h = lane & 1u;
            const uint32_t row = lds_rd32_sync<512>(list + 4 * (t < count ? t : 0));
            S.off[4] = row * nsa * 4 + h * 4;
            tail |= (2 * last + h < nsa ? 1u : 0u) << 4;
            on |= (32 * wave < count ? 1u : 0u) << 4;
        } else {
            S.off[4] = 0;
        }
        // weights: lane (g, r) of subtile j loads bytes 64 h + 16 g of row r's
        // chunk piece (rows past N read row 0; pieces past K read the row start)
#pragma unroll
        for (uint32_t j = 0; j < 2; j++) {
            const uint32_t ir = pg_irow<NMAT>(wave, j), m = ir / RPM;
            const uint32_t n = rb * RPM + ir % RPM + rr;
            S.woff[j] = (n < N ? n : 0) * RB + 16 * g;
            S.wb[j] = wp[m];
#pragma unroll
            for (uint32_t h = 0; h < 2; h++) tail |= (last * (PG_KC / 2) + 64 * h + 16 * g < RB ? 1u : 0u) << (8 + 2 * j + h);
        }
        S.tail_ok = tail;
        S.on = on;
        S.n = __builtin_popcount(on) + PG_WLOADS;
    };

    // Issue unit U (0..7) of chunk c of the issue item into stage ST / set W:
    // units 0-3 load weight pieces (j, h) = (U / 2, U % 2), units 4-7 copy
    // activation rows 32 (U - 4) + 4 w.., unit 7 also the block scales.  The
    // loads are inline asm the compiler does not count (its wait pass would
    // otherwise wait for them, and for every copy in flight, before the next
    // LDS read): they are waited for by the per-stage vmcnt count and
    // laundered through an empty asm before use.  In the last chunk, pieces
    // past K come from the zero page (copies) or the row start (loads).
    auto issue_unit = [&](const PgIssue& S, uint32_t c, auto st_tag, PgW& W, auto u_tag) __attribute__((always_inline)) {
        constexpr uint32_t ST = decltype(st_tag)::value, U = decltype(u_tag)::value;
        const uint32_t ok = c + 1 < nch ? 0xffffu : S.tail_ok;
        if constexpr (U < 4) {
            constexpr uint32_t j = U / 2, h = U % 2;
            const uint32_t bo = (ok & (1u << (8 + 2 * j + h))) ? c * (PG_KC / 2) + 64 * h : 0u;
            W.w[j][h] = gload16_untracked(S.wb[j] + S.woff[j] + bo);
        } else {
            constexpr uint32_t i = U - 4;
            uint8_t* const dA = pg_ring + PG_A_OFF + ST * 32768 + wave * 1024 + i * 8192;
            if (S.on & (1u << i))
                __builtin_amdgcn_global_load_lds((ok & (1u << i)) ? A.aq + c * PG_KC + S.off[i] : kZeroPage, dA, 16, 0, 0);
            if constexpr (U == 7) {
                uint8_t* const dT = pg_ring + PG_SA_OFF + ST * 1024 + wave * 256;
                const uint8_t* sa = reinterpret_cast<const uint8_t*>(A.as) + c * 8;
                if (S.on & 16) __builtin_amdgcn_global_load_lds((ok & 16) ? sa + S.off[4] : kZeroPage, dT, 4, 0, 0);
            }
        }
    };

    // ---- first item: descriptor copied synchronously ----
    // Item s*G + q (of the whole item list, across the groups) goes to the
    // block in slot q, and the hardware deals consecutive blocks to the 8
    // XCDs in turn: slot q = (b % 8) * (G / 8) + b / 8 puts consecutive items
    // (the tiles of one expert row block) on one XCD, where they share its L2
    // copy of the weight rows.
    const uint32_t slot = G % 8 == 0 ? (blockIdx.x % 8) * (G / 8) + blockIdx.x / 8 : blockIdx.x;
    uint32_t item = i0 + (slot + G - i0 % G) % G;
    if (item >= n_items) return;
    if (wave == 0) copy_rec(item, 0);
    wait_vm_imm<0>();
    __syncthreads();
    if (wave == 0) copy_list(0);
    wait_vm_imm<0>();
    __syncthreads();

    PgIssue S;
    setup_issue(0, S);
    uint32_t ic = 0, ipar = 0, iitem = item;   // issue item: next chunk, descriptor slot, index
    bool issuing = true;
    // Issues the next chunk (one per stage: the item's scale spans at its
    // chunk 0, the weight loads, the copies) and moves to the next item after
    // the last chunk of the current one.  Past the block's last item the
    // weight loads are still issued (the last chunk again, unused) so every
    // register set is written on every path.
    uint32_t q0 = 0, q1 = 0, q2 = 0;   // copies + loads this wave issued into each stage
    // The item's scale spans, into the span slot of its parity: piece p of
    // the parts laid back to back (part m at byte m RPM K/32 of the slot).
    auto issue_span = [&](uint32_t par) __attribute__((always_inline)) {
        uint8_t* const dst = pg_ring + PG_SPAN_OFF + par * (PG_ROWS * SB);
        for (uint32_t t = 0; t < S.nspan; t++) {
            uint32_t q = wave + 8 * t, m = 0;
            if (NMAT == 2 && q >= S.np0) {
                m = 1;
                q -= S.np0;
            }
            const uint32_t o = min(q * 256, S.slen[m] - 256);
            __builtin_amdgcn_global_load_lds(S.sp[m] + o + lane * 4, dst + m * RPM * SB + o, 4, 0, 0);
        }
    };
    auto issue_next = [&](auto st_tag, PgW& W) __attribute__((always_inline)) {
        constexpr uint32_t ST = decltype(st_tag)::value;
        if (issuing && ic == 0) issue_span(ipar);
        const uint32_t nq = issuing ? S.n + (ic == 0 ? S.nspan : 0u) : PG_WLOADS;
        if (ST == 0) q0 = nq;
        if (ST == 1) q1 = nq;
        if (ST == 2) q2 = nq;
        if (!issuing) S.on = 0;
        const uint32_t ci = issuing ? ic : nch - 1;
        static_for<8>([&](auto u) __attribute__((always_inline)) { issue_unit(S, ci, st_tag, W, u); });
        if (issuing && ++ic == nch) {
            ic = 0;
            ipar ^= 1u;
            iitem += G;
            issuing = iitem < n_items;
            if (issuing) setup_issue(ipar, S);
        }
    };
    PgW W0, W1, W2;
    issue_next(std::integral_constant<uint32_t, 0>{}, W0);
    issue_next(std::integral_constant<uint32_t, 1>{}, W1);

    // ---- compute side ----
    // Activation operand of lane (g, r): route 16 a + r, k 16 g.. and
    // 64 + 16 g.. of each 128-k half h, at pieces (8 h + g) ^ r, (8 h + 4 + g) ^ r.
    uint32_t LA[4];
#pragma unroll
    for (uint32_t q = 0; q < 4; q++) LA[q] = ring + PG_A_OFF + rr * 256 + (((4 * q) + g) ^ rr) * 16;
    const uint32_t LSA = ring + PG_SA_OFF + rr * 8;

    uint32_t cpar = 0, c = 0;              // compute item descriptor slot, chunk
    uint32_t count = 0, rb = 0, alim = 0;
    uint32_t LSB[2];
    v4f acc[NA][2];
    auto start_item = [&]() __attribute__((always_inline)) {
        rb = rec_word(cpar, 0);
        count = rec_word(cpar, 1);
        alim = min((uint32_t)NA, (count + 15) / 16);
#pragma unroll
        for (uint32_t j = 0; j < 2; j++) {
            const uint32_t ir = pg_irow<NMAT>(wave, j);
            LSB[j] = ring + PG_SPAN_OFF + cpar * (PG_ROWS * SB) + (ir + rr) * SB + g;
        }
#pragma unroll
        for (int a = 0; a < NA; a++)
#pragma unroll
            for (int j = 0; j < 2; j++) acc[a][j] = v4f{0.f, 0.f, 0.f, 0.f};
    };
    start_item();
    bool cnext = item + G < n_items;        // is there an item after the compute item

    auto epilogue = [&]() __attribute__((always_inline)) {
        const uint32_t list = ring + PG_LIST_OFF + cpar * 2048;
#pragma unroll
        for (uint32_t a = 0; a < (uint32_t)NA; a++) {
            if (a >= alim) continue;
            // routes 16 a + 4 g .. + 3 (and their weights) in one read each
            v4i rt, wv;
            asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %2 offset:1024\n\ts_waitcnt lgkmcnt(0)"
                         : "=&v"(rt), "=&v"(wv)
                         : "v"(list + (16 * a + 4 * g) * 4));
            const uint32_t lim = count - 16 * a;   // routes of subtile a (a < alim: > 0)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                if (4 * g + i >= lim) continue;
                const uint32_t r = (uint32_t)rt[i];
                if (NMAT == 2) {
                    const uint64_t ob = (uint64_t)(r / A.k) * A.frame_elems + (uint64_t)(r % A.k) * N;
                    const uint32_t ch = rb * RPM + 16 * wave + rr;
                    if (ch >= N) continue;
                    float gv = round_bf16(acc[a][0][i]);
                    float uv = round_bf16(acc[a][1][i]);
                    if (A.limit > 0.0f) {
                        gv = fminf(gv, A.limit);
                        uv = fminf(fmaxf(uv, -A.limit), A.limit);
                    }
                    A.out[ob + ch] = (uint16_t)f32_to_bf16(silu_fast(gv) * uv);
                } else {
                    const float wr = __int_as_float(wv[i]);
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        const uint32_t row = rb * RPM + 32 * wave + 16 * j + rr;
                        if (row < N) A.out[(uint64_t)r * N + row] = (uint16_t)f32_to_bf16(acc[a][j][i] * wr);
                    }
                }
            }
        }
    };

    // One pipeline step on stage ST: wait for this chunk, barrier, issue the
    // chunk two ahead (wave 0 first copies the next item's record at chunk 0
    // and its route list at chunk 2), contract, and on the item's last chunk
    // write it out and switch items.  Returns false when the block has no
    // more work.
    auto step = [&](auto st_tag, PgW& Wc, PgW& Wn) __attribute__((always_inline)) -> bool {
        constexpr uint32_t ST = decltype(st_tag)::value;
        // Copies and loads issued after this chunk's: the next chunk's, plus
        // wave 0's descriptor copies issued in the previous step (record at
        // chunk 0, list at chunk 2).
        constexpr uint32_t S1 = (ST + 1) % PG_NST;
        uint32_t x = S1 == 0 ? q0 : S1 == 1 ? q1 : q2;
        if (wave == 0) x += (c == 1 ? 1u : 0u) + (c == 3 ? 2u : 0u);
        wait_vm(x);
        __builtin_amdgcn_s_barrier();
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int h = 0; h < 2; h++) asm volatile("" : "+v"(Wc.w[j][h]));
        if (wave == 0) {
            if (c == 0) copy_rec(item + G, cpar ^ 1u);
            else if (c == 2) copy_list(cpar ^ 1u);
        }
        // Chunk c + 2 (of this item or the next) goes into stage ST + 2.
        issue_next(std::integral_constant<uint32_t, (ST + 2) % PG_NST>{}, Wn);
        // ---- contract chunk c: scales, then the route subtiles two reads ahead ----
        // Subtiles past the item's routes contract stale LDS rows into
        // accumulators the epilogue never reads; the three forms (2, 4, 8
        // subtiles) keep every LDS read unconditional inside a form, so no
        // read result has to be merged across branches before its wait.
        auto contract = [&](auto n_tag) __attribute__((always_inline)) {
            constexpr uint32_t NC = decltype(n_tag)::value;
            uint32_t sbv[2][2];
            v2i sav[2];
            v4i av[2][4];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                sbv[j][0] = lds_rd8<0>(LSB[j] + 8 * c);
                sbv[j][1] = lds_rd8<4>(LSB[j] + 8 * c);
            }
            // Route subtile a's operands: 4 activation pieces and its block scales.
            auto read_a = [&](auto ai) __attribute__((always_inline)) {
                constexpr uint32_t a = decltype(ai)::value;
#pragma unroll
                for (int q = 0; q < 4; q++) av[a % 2][q] = lds_rd128_far<ST * 32768 + a * 4096>(LA[q]);
                sav[a % 2] = lds_rd64<ST * 1024 + a * 128>(LSA);
            };
            read_a(std::integral_constant<uint32_t, 0>{});
            static_for<NC>([&](auto ai) __attribute__((always_inline)) {
                constexpr uint32_t a = decltype(ai)::value;
                // Subtile a's reads are done when at most the next subtile's
                // five are in flight.
                if constexpr (a + 1 < NC) {
                    read_a(std::integral_constant<uint32_t, a + 1>{});
                    asm volatile("s_waitcnt lgkmcnt(5)"
                                 : "+v"(av[a % 2][0]), "+v"(av[a % 2][1]), "+v"(av[a % 2][2]), "+v"(av[a % 2][3]),
                                   "+v"(sav[a % 2]));
                } else {
                    asm volatile("s_waitcnt lgkmcnt(0)"
                                 : "+v"(av[a % 2][0]), "+v"(av[a % 2][1]), "+v"(av[a % 2][2]), "+v"(av[a % 2][3]),
                                   "+v"(sav[a % 2]));
                }
                if constexpr (a == 0) {
                    asm volatile("" : "+v"(sbv[0][0]), "+v"(sbv[0][1]), "+v"(sbv[1][0]), "+v"(sbv[1][1]));
                    // Scale blocks past K (last chunk) read bytes beyond the row.
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        const bool bvalid = c * 8 + 4 * h + g < SB;
#pragma unroll
                        for (int j = 0; j < 2; j++) sbv[j][h] = bvalid ? sbv[j][h] : 127u;
                    }
                }
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const v8i x8 = v8i{av[a % 2][2 * h].x, av[a % 2][2 * h].y, av[a % 2][2 * h].z, av[a % 2][2 * h].w,
                                       av[a % 2][2 * h + 1].x, av[a % 2][2 * h + 1].y, av[a % 2][2 * h + 1].z,
                                       av[a % 2][2 * h + 1].w};
                    const uint32_t se = ((uint32_t)sav[a % 2][h] >> 23) & 0xffu;
#pragma unroll
                    for (int j = 0; j < 2; j++) acc[a][j] = mfma_fp8_fp4(x8, Wc.w[j][h], se, sbv[j][h], acc[a][j]);
                }
            });
        };
        contract(std::integral_constant<uint32_t, NA>{});
        if (++c < nch) return true;
        // ---- end of the item ----
        epilogue();
        if (!cnext) return false;
        c = 0;
        cpar ^= 1u;
        item += G;
        cnext = item + G < n_items;
        start_item();
        return true;
    };
    while (true) {
        if (!step(std::integral_constant<uint32_t, 0>{}, W0, W2)) break;
        if (!step(std::integral_constant<uint32_t, 1>{}, W1, W0)) break;
        if (!step(std::integral_constant<uint32_t, 2>{}, W2, W1)) break;
    }
    // Loads past the last item may still be in flight into registers.
    wait_vm_imm<0>();
}

template <int NMAT>
__global__ __launch_bounds__(512) void moe_pgemm_kernel(PgArgs A) {
    constexpr uint32_t RPM = PG_ROWS / NMAT;
    const uint32_t nrb = (A.N + RPM - 1) / RPM;
    const uint32_t nt = __builtin_amdgcn_readfirstlane(A.n_tiles[0]);
    const uint32_t nt0 = __builtin_amdgcn_readfirstlane(A.n_tiles[1]);
    const uint32_t nt1 = __builtin_amdgcn_readfirstlane(A.n_tiles[2]);
    // The groups run one after the other; every wave finishes a group (its
    // descriptor slots and ring are reused) before the next starts.
    pg_range<NMAT, 8>(A, 0, nt0 * nrb);
    __syncthreads();
    pg_range<NMAT, 4>(A, nt0 * nrb, (nt0 + nt1) * nrb);
    __syncthreads();
    pg_range<NMAT, 2>(A, (nt0 + nt1) * nrb, nt * nrb);
}

// ---------------------------------------------------------------------------
// Prefill grouped GEMM, producer / consumer form (moe_pg2_kernel).
//
// One 768-thread block per CU walks the same work items as the form above
// (a tile of <= 128 routes of one expert x a 256-row weight block; gate_up:
// 128 gate + the same 128 up channels).  The waves have fixed roles:
//  - waves 8-11 (producers) only copy: each 128-k chunk of the item's weights
//    (256 rows x 64 B) and of its routes' e4m3 activations (<= 128 x 128 B)
//    goes global -> LDS with global_load_lds into a 4-stage ring, three
//    chunks ahead.  A producer that stalls at issue (the CU's miss queue
//    full) delays no MFMA;
//  - waves 0-7 (consumers) only read LDS and run the scaled MFMAs; each owns
//    a 64-route x 64-row (or 64 x 32, 32 x 32) block of the item, so every
//    16-byte operand read from LDS feeds two to four MFMAs.  They load their
//    rows' e8m0 bytes and their routes' block scales themselves, one chunk
//    ahead.
// One barrier per chunk joins both roles: the producers have waited for the
// next chunk's copies, the consumers are done with the stage the producers
// refill next.  The LDS layout is piece-major inside every 16-row (or
// 16-route) subtile, [piece][row] x 16 B, so lane (g, r) of an operand read
// takes the 16 bytes at lane * 16: every read is one contiguous 1 KB.
// ---------------------------------------------------------------------------
constexpr uint32_t P2_KC = 128;            // k per chunk (one MFMA)
constexpr uint32_t P2_W_BYTES = 16384;     // weights of a stage: 16 subtiles of 16 rows x 64 B
constexpr uint32_t P2_MAX_SB = 92;         // e8m0 bytes per weight row (K <= 2944)
constexpr uint32_t P2_SPAN_SLOT = PG_ROWS * P2_MAX_SB;   // an item's scale rows
constexpr uint32_t P2_LDS = 160 * 1024;
constexpr uint32_t P2_LIST_OFF = P2_LDS - 2 * sizeof(PgList);       // [2][2 KB] route lists by item parity
constexpr uint32_t P2_SPAN_OFF = P2_LIST_OFF - 2 * P2_SPAN_SLOT;    // [2] scale-row slots by item parity
constexpr uint32_t P2_RING = P2_SPAN_OFF;  // ring stages of (weights, activations, block scales)
// The next item's list is copied when chunk NS - 1 of an item is issued and
// read when its last chunk is issued, NS - 1 chunks before its end.
constexpr uint32_t P2_MIN_CHUNKS = 12;
// Ring stages of a route-count group (nat 16-route subtiles per tile): as
// many as fit.
__host__ __device__ constexpr uint32_t p2_stages(uint32_t nat) {
    return P2_RING / (P2_W_BYTES + nat * (16u * 128u + 16u * 4u));
}
static_assert(p2_stages(8) >= 3 && p2_stages(2) <= 6, "ring depth");

struct PgItem {
    uint32_t rb, count, tile;
    const uint8_t* w[2];
    const uint8_t* s[2];
};

// An item record through the scalar cache (reads only).
__device__ __forceinline__ PgItem p2_item(const ItemRec* rec) {
    u4s h;
    u8s p;
    asm volatile("s_load_dwordx4 %0, %2, 0x0\n\ts_load_dwordx8 %1, %2, 0x10\n\ts_waitcnt lgkmcnt(0)"
                 : "=&s"(h), "=&s"(p)
                 : "s"(rec));
    PgItem it;
    it.rb = h.x;
    it.count = h.y;
    it.tile = h.z;
    it.w[0] = reinterpret_cast<const uint8_t*>((uint64_t)p[0] | ((uint64_t)p[1] << 32));
    it.w[1] = reinterpret_cast<const uint8_t*>((uint64_t)p[2] | ((uint64_t)p[3] << 32));
    it.s[0] = reinterpret_cast<const uint8_t*>((uint64_t)p[4] | ((uint64_t)p[5] << 32));
    it.s[1] = reinterpret_cast<const uint8_t*>((uint64_t)p[6] | ((uint64_t)p[7] << 32));
    return it;
}

// LDS dword read that waits for itself.
__device__ __forceinline__ uint32_t p2_lds32(uint32_t a) {
    uint32_t r;
    asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(r) : "v"(a));
    return r;
}

// Item row of row subtile j of consumer wave w.  NJ = 4 (tiles of up to 128
// routes): waves (route half w / 4, row quarter w % 4), 64 rows each;
// NJ = 2: every wave takes all routes and 32 rows.  gate_up: the first NJ / 2
// subtiles are gate rows, the others the same up channels (item rows
// 128 + ...).
template <int NMAT, int NJ>
__device__ __forceinline__ uint32_t p2_irow(uint32_t w, uint32_t j) {
    if constexpr (NJ == 4) {
        const uint32_t q = w % 4;
        return NMAT == 2 ? (j < 2 ? 32 * q + 16 * j : 128 + 32 * q + 16 * (j - 2)) : 64 * q + 16 * j;
    } else {
        return NMAT == 2 ? j * 128 + 16 * w : 32 * w + 16 * j;
    }
}

// Items [i0, n_items) of one route-count group.  NAT: route subtiles the
// tile holds (8, 4, 2); NAW route subtiles and NJ row subtiles per consumer
// wave.
template <int NMAT, int NAT, int NAW, int NJ>
__device__ __forceinline__ void p2_range(const PgArgs& A, uint32_t i0, uint32_t n_items) {
    constexpr uint32_t NR = NAT * 16;                       // routes per tile
    constexpr uint32_t SBY = P2_W_BYTES + NR * 128 + NR * 4;  // stage: weights, activations, block scales
    constexpr uint32_t NS = p2_stages(NAT);                 // ring stages
    constexpr uint32_t NAI = 2 * NAT / 4;                   // activation copies per producer per chunk
    constexpr uint32_t NAS = (NR + 63) / 64;                // block-scale copies per chunk
    extern __shared__ __attribute__((aligned(16))) uint8_t p2_ring[];
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t g = lane >> 4, rr = lane & 15;
    const uint32_t K = A.K, N = A.N, RB = K / 2, SB = K / 32, nch = (K + P2_KC - 1) / P2_KC;
    const uint32_t nsa = (K + 127) / 128;
    constexpr uint32_t RPM = PG_ROWS / NMAT;
    const uint32_t G = gridDim.x;
    const uint32_t ring = lds_addr(p2_ring);

    // This block's items: s * G + slot (slot XCD-aware, as in pg_range).
    const uint32_t slot = G % 8 == 0 ? (blockIdx.x % 8) * (G / 8) + blockIdx.x / 8 : blockIdx.x;
    const uint32_t first = i0 + (slot + G - i0 % G) % G;
    if (first >= n_items) return;   // uniform over the block: no barrier below is reached
    const uint32_t n_mine = (n_items - first + G - 1) / G;
    const uint32_t T = n_mine * nch;   // steps (chunks) of this group for the block

    if (wave >= 8) {
        // ================= producers =================
        const uint32_t p = wave - 8;
        uint32_t pitem = first, pord = 0, pc = 0;      // item being issued, its ordinal, next chunk
        PgItem it = p2_item(A.items + pitem);
        // per-lane source offsets of the current issue item
        uint32_t woff[4], aoff[NAI], apc[NAI], soff = 0;
        const uint8_t* wb = nullptr;
        auto setup = [&]() __attribute__((always_inline)) {
            // weights: subtiles x = 4 p .. 4 p + 3 (16 rows each), lane (piece i / 16, row i % 16)
            // (selects, not a run-time index: an indexed record would live in
            // scratch memory, whose loads count in vmcnt)
            wb = (NMAT == 2 && p >= 2) ? it.w[1] : it.w[0];
#pragma unroll
            for (uint32_t u = 0; u < 4; u++) {
                const uint32_t irow = 16 * (4 * p + u) + rr;             // item row
                const uint32_t n = it.rb * RPM + irow % RPM;             // matrix row
                woff[u] = (n < N ? n : 0u) * RB + g * 16;
            }
            // activations: copy u = p * NAI + v covers the whole 128-byte
            // chunk of routes 8 (u % 2) .. + 7 of route subtile y = u / 2,
            // lane i route 8 (u % 2) + i / 8, slot i % 8 holding piece
            // (i % 8) ^ (route / 2); block scales: copy p < NAS covers
            // routes 64 p + i.  List entries past the tile's count are not
            // written: their positions read entry 0.
            const uint32_t list = ring + P2_LIST_OFF + (pord & 1u) * (uint32_t)sizeof(PgList);
#pragma unroll
            for (uint32_t v = 0; v < NAI; v++) {
                const uint32_t u = p * NAI + v, y = u / 2, rt = 8 * (u % 2) + lane / 8;
                const uint32_t pos = 16 * y + rt < it.count ? 16 * y + rt : 0u;
                const uint32_t arow = min(p2_lds32(list + 512 + 4 * pos), A.a_rows - 1);
                apc[v] = ((lane % 8) ^ (rt / 2)) * 16;
                aoff[v] = arow * A.lda + apc[v];
            }
            if (p < NAS) {
                const uint32_t pos = 64 * p + lane < it.count ? 64 * p + lane : 0u;
                soff = min(p2_lds32(list + 512 + 4 * pos), A.a_rows - 1) * nsa;
            }
        };
        // The scale rows of item `nx` (one contiguous span per matrix part,
        // rows * K / 32 bytes) into span slot `slot`: 256-byte pieces dealt
        // round-robin over the producers, the last piece of a part aligned
        // to its end.  Returns the copies issued.
        auto copy_span = [&](const PgItem& nx, uint32_t sslot) __attribute__((always_inline)) -> uint32_t {
            uint32_t cnt = 0;
            uint8_t* const base = p2_ring + P2_SPAN_OFF + sslot * P2_SPAN_SLOT;
#pragma unroll
            for (uint32_t m = 0; m < (uint32_t)NMAT; m++) {
                const uint32_t rows = min(RPM, N - nx.rb * RPM), slen = rows * SB;
                const uint8_t* src = (m == 0 ? nx.s[0] : nx.s[1]) + (uint64_t)nx.rb * RPM * SB;
                const uint32_t np = (slen + 255) / 256;
                for (uint32_t q = p; q < np; q += 4) {
                    const uint32_t o = min(q * 256, slen - 256);
                    __builtin_amdgcn_global_load_lds(src + o + lane * 4, base + m * RPM * SB + o, 4, 0, 0);
                    cnt++;
                }
            }
            return cnt;
        };
        bool issuing = true;
        // Issue the next chunk into its stage; returns the ops issued.
        auto issue = [&](uint32_t stage) __attribute__((always_inline)) -> uint32_t {
            if (!issuing) return 0u;
            uint32_t n = 0;
            const bool last = pc + 1 == nch;
            uint8_t* const st = p2_ring + stage * SBY;
#pragma unroll
            for (uint32_t u = 0; u < 4; u++) {
                const uint32_t bo = (!last || pc * 64 + g * 16 < RB) ? pc * 64 : 0u;
                __builtin_amdgcn_global_load_lds(wb + woff[u] + bo, st + (4 * p + u) * 1024, 16, 0, 0);
            }
            n += 4;
#pragma unroll
            for (uint32_t v = 0; v < NAI; v++) {
                const bool ok = !last || pc * P2_KC + apc[v] < K;
                __builtin_amdgcn_global_load_lds(ok ? A.aq + pc * P2_KC + aoff[v] : kZeroPage,
                                                 st + P2_W_BYTES + (p * NAI + v) * 1024, 16, 0, 0);
            }
            n += NAI;
            if (p < NAS) {
                // routes 64 p + lane (a tile of 32 routes: lanes < 32)
                if (NR >= 64 || lane < NR)
                    __builtin_amdgcn_global_load_lds(A.as + soff + pc, st + P2_W_BYTES + NR * 128 + p * 256, 4, 0, 0);
                n += 1;
            }
            // The next item's route list and scale rows, once the consumers
            // are done with the slots they go to (the item before this one).
            if (pc == NS - 1 && pord + 1 < n_mine) {
                const PgItem nx = p2_item(A.items + pitem + G);
                if (p < 2) {
                    const PgList* src = A.lists + nx.tile;
                    uint8_t* dst = p2_ring + P2_LIST_OFF + ((pord + 1) & 1u) * (uint32_t)sizeof(PgList) + p * 1024;
                    __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint8_t*>(src) + p * 1024 + lane * 16, dst,
                                                     16, 0, 0);
                    n += 1;
                }
                n += copy_span(nx, (pord + 1) & 1u);
            }
            if (++pc == nch) {
                pc = 0;
                pord++;
                pitem += G;
                issuing = pord < n_mine;
                if (issuing) {
                    it = p2_item(A.items + pitem);
                    setup();
                }
            }
            return n;
        };
        // prologue: the first item's list and scale rows (synchronously),
        // then chunks 0 .. NS - 2
        if (p < 2) {
            const PgList* src = A.lists + it.tile;
            __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint8_t*>(src) + p * 1024 + lane * 16,
                                             p2_ring + P2_LIST_OFF + p * 1024, 16, 0, 0);
        }
        copy_span(it, 0);
        wait_vm_imm<0>();
        __syncthreads();   // (1) the first list and scale rows are in LDS
        setup();
        // n[s]: ops this wave issued with the chunk of stage s (indexed by
        // compile-time constants only, so it stays in registers)
        uint32_t n[NS];
        static_for<NS>([&](auto s_) __attribute__((always_inline)) { n[decltype(s_)::value] = 0; });
        static_for<NS - 1>([&](auto s_) __attribute__((always_inline)) {
            constexpr uint32_t st = decltype(s_)::value;
            n[st] = issue(st);
        });
        {
            uint32_t x = 0;
            static_for<NS - 2>([&](auto q_) __attribute__((always_inline)) { x += n[decltype(q_)::value + 1]; });
            wait_vm(x);
        }
        __syncthreads();   // (2) chunk 0 landed
        // Step t issues chunk t + NS - 1 into stage (t + NS - 1) % NS and
        // waits for chunk t + 1: what was issued after it is the last NS - 2
        // batches.  A bare barrier: __syncthreads() would also wait for
        // every copy in flight (its release fence drains vmcnt).
        for (uint32_t t = 0; t < T; t += NS) {
            bool done = false;
            static_for<NS>([&](auto s_) __attribute__((always_inline)) {
                constexpr uint32_t sp = decltype(s_)::value;
                if (done || t + sp >= T) {
                    done = true;
                    return;
                }
                constexpr uint32_t sn = (sp + NS - 1) % NS;
                n[sn] = issue(sn);
                uint32_t x = 0;
                static_for<NS - 2>([&](auto q_) __attribute__((always_inline)) {
                    x += n[(sp + 2 + decltype(q_)::value) % NS];
                });
                wait_vm(x);
                __builtin_amdgcn_s_barrier();
            });
        }
        return;
    }

    // ================= consumers =================
    // Only LDS reads, MFMAs and the epilogue's stores: every operand and
    // scale of a chunk is in its ring stage or the item's scale-row slot.
    const uint32_t a0 = NJ == 4 ? 4 * (wave / 4) : 0u;   // first route subtile of this wave
    const uint32_t LW = ring + lane * 16;                  // + stage + subtile * 1 KB
    // + stage + subtile * 2 KB: route rr's chunk at (rr / 8) KB + (rr % 8) * 128,
    // piece x in slot x ^ (rr / 2); this lane reads pieces g and g + 4
    const uint32_t LA = ring + P2_W_BYTES + (rr / 8) * 1024 + (rr % 8) * 128;
    const uint32_t LAlo = LA + ((g ^ (rr / 2)) & 7) * 16, LAhi = LA + ((g ^ (rr / 2) ^ 4) & 7) * 16;
    const uint32_t LS = ring + P2_W_BYTES + NR * 128 + rr * 4;   // + stage + route subtile * 64
    uint32_t item = first, ord = 0;
    PgItem it = p2_item(A.items + item);
    uint32_t srow[NJ];   // LDS address of this lane's scale row of subtile j in the item's slot (+ 4 c + g)
    auto start_item = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (uint32_t j = 0; j < (uint32_t)NJ; j++)
            srow[j] = ring + P2_SPAN_OFF + (ord & 1u) * P2_SPAN_SLOT + (p2_irow<NMAT, NJ>(wave, j) + rr) * SB + g;
    };
    v4f acc[NAW][NJ];
#pragma unroll
    for (int a = 0; a < NAW; a++)
#pragma unroll
        for (int j = 0; j < NJ; j++) acc[a][j] = v4f{0.f, 0.f, 0.f, 0.f};
    __syncthreads();   // (1)
    start_item();
    __syncthreads();   // (2)
    uint32_t c = 0;
    for (uint32_t t = 0; t < T; t++) {
        const uint32_t so = (t % NS) * SBY;
        const bool item_end = c + 1 == nch;
        // operands and scales of chunk c
        v4i bw[NJ];
        v8i av[NAW];
        uint32_t sw[NJ], sa[NAW];
#pragma unroll
        for (uint32_t j = 0; j < (uint32_t)NJ; j++) {
            const uint32_t x = p2_irow<NMAT, NJ>(wave, j) / 16;
            asm volatile("ds_read_b128 %0, %1" : "=v"(bw[j]) : "v"(LW + so + x * 1024));
            asm volatile("ds_read_u8 %0, %1" : "=v"(sw[j]) : "v"(srow[j] + 4 * c));
        }
#pragma unroll
        for (uint32_t a = 0; a < (uint32_t)NAW; a++) {
            v4i lo, hi;
            const uint32_t ad = so + (a0 + a) * 2048;
            // early-clobber outputs: the second read must not find its address
            // register overwritten by the first read's data
            asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %3" : "=&v"(lo), "=&v"(hi) : "v"(LAlo + ad), "v"(LAhi + ad));
            av[a] = v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
            asm volatile("ds_read_b32 %0, %1" : "=v"(sa[a]) : "v"(LS + so + (a0 + a) * 64));
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (uint32_t j = 0; j < (uint32_t)NJ; j++) asm volatile("" : "+v"(bw[j]), "+v"(sw[j]));
#pragma unroll
        for (uint32_t a = 0; a < (uint32_t)NAW; a++) asm volatile("" : "+v"(av[a]), "+v"(sa[a]));
        uint32_t ew[NJ], ea[NAW];
        {
            const bool blk_ok = 4 * c + g < SB;   // scale blocks past K (last chunk): 2^0
#pragma unroll
            for (uint32_t j = 0; j < (uint32_t)NJ; j++) ew[j] = blk_ok ? sw[j] : 127u;
#pragma unroll
            for (uint32_t a = 0; a < (uint32_t)NAW; a++) ea[a] = (sa[a] >> 23) & 0xffu;
        }
#pragma unroll
        for (uint32_t a = 0; a < (uint32_t)NAW; a++)
#pragma unroll
            for (uint32_t j = 0; j < (uint32_t)NJ; j++) acc[a][j] = mfma_fp8_fp4(av[a], bw[j], ea[a], ew[j], acc[a][j]);
        if (item_end) {
            // ---- epilogue of the item ----
            const uint32_t list = ring + P2_LIST_OFF + (ord & 1u) * (uint32_t)sizeof(PgList);
            const uint32_t count = it.count;
#pragma unroll
            for (uint32_t a = 0; a < (uint32_t)NAW; a++) {
                const uint32_t tb = 16 * (a0 + a);
                if (tb >= count) continue;
                v4i rt, wv;
                asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %2 offset:1024\n\ts_waitcnt lgkmcnt(0)"
                             : "=&v"(rt), "=&v"(wv)
                             : "v"(list + (tb + 4 * g) * 4));
#pragma unroll
                for (uint32_t i = 0; i < 4; i++) {
                    const uint32_t r = (uint32_t)rt[i];
                    if (tb + 4 * g + i >= count || r >= A.routes) continue;
                    if constexpr (NMAT == 2) {
                        const uint64_t ob = (uint64_t)(r / A.k) * A.frame_elems + (uint64_t)(r % A.k) * N;
#pragma unroll
                        for (uint32_t j = 0; j < (uint32_t)NJ / 2; j++) {
                            const uint32_t ch = it.rb * RPM + p2_irow<NMAT, NJ>(wave, j) + rr;
                            if (ch >= N) continue;
                            float gv = round_bf16(acc[a][j][i]);
                            float uv = round_bf16(acc[a][j + NJ / 2][i]);
                            if (A.limit > 0.0f) {
                                gv = fminf(gv, A.limit);
                                uv = fminf(fmaxf(uv, -A.limit), A.limit);
                            }
                            A.out[ob + ch] = (uint16_t)f32_to_bf16(silu_fast(gv) * uv);
                        }
                    } else {
                        const float wr = __int_as_float(wv[i]);
#pragma unroll
                        for (uint32_t j = 0; j < (uint32_t)NJ; j++) {
                            const uint32_t row = it.rb * RPM + p2_irow<NMAT, NJ>(wave, j) + rr;
                            if (row < N) A.out[(uint64_t)r * N + row] = (uint16_t)f32_to_bf16(acc[a][j][i] * wr);
                        }
                    }
                }
            }
#pragma unroll
            for (int a = 0; a < NAW; a++)
#pragma unroll
                for (int j = 0; j < NJ; j++) acc[a][j] = v4f{0.f, 0.f, 0.f, 0.f};
            c = 0;
            ord++;
            item += G;
            if (ord < n_mine) {
                it = p2_item(A.items + item);
                start_item();
            }
        } else {
            c++;
        }
        __builtin_amdgcn_s_barrier();
    }
}

// ---------------------------------------------------------------------------
// Whole-line form of the producer / consumer loop, for tiles of <= 64 routes
// (the route-count groups where the weights are most of the copied bytes).
// A ring stage holds one half of the item's 256 rows (gate_up: the 128 gate
// or the 128 up rows; down: rows 0-127 or 128-255) over a k pair (256 k), so
// every weight copy takes whole 128-byte lines: 8 rows x 128 B per
// instruction.  Copying 64 bytes of 16 rows per instruction and the other
// half of each line a chunk later streams at ~5.0 TB/s over the chip; whole
// lines stream at ~6.0.  Row r's eight 16-byte pieces sit in its 128 LDS
// bytes XOR-swizzled by (r / 2) % 8 (r within its 16-row subtile), so the
// 16 lanes that read one piece column of a subtile hit distinct bank groups.
// The activations go by k pair as well: 4 routes x 256 B per instruction
// into an activation slot that both stages of the pair read, pieces
// swizzled by route % 16, with the pair's two block scales per route.
// Consumer wave w owns rows 16 w .. 16 w + 15 of each half (subtile j =
// half) for every route of the tile.
// ---------------------------------------------------------------------------
constexpr uint32_t WL_W_BYTES = 16384;   // weight stage: 128 rows x 128 B

template <int NMAT, int NAT>
__device__ __forceinline__ void p2_range_wl(const PgArgs& A, uint32_t i0, uint32_t n_items) {
    constexpr uint32_t NR = NAT * 16;                       // routes per tile
    constexpr uint32_t NSW = NAT <= 2 ? 4 : 3;              // weight stages
    constexpr uint32_t NSA = (NSW + 2) / 2;                 // activation slots: 2 NSA >= NSW + 1
    constexpr uint32_t ABY = NR * 256 + NR * 8;             // activation slot: pieces, then block scales
    constexpr uint32_t AOFF = NSW * WL_W_BYTES;
    static_assert(AOFF + NSA * ABY <= P2_RING, "whole-line ring");
    constexpr uint32_t NAI = NR / 16;                       // activation copies per producer per pair
    constexpr uint32_t NAS = NR / 32;                       // block-scale copies per pair (producers p < NAS)
    extern __shared__ __attribute__((aligned(16))) uint8_t p2_ring[];
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t g = lane >> 4, rr = lane & 15;
    const uint32_t K = A.K, N = A.N, RB = K / 2, SB = K / 32, nch = (K + P2_KC - 1) / P2_KC;
    const uint32_t NP2 = (nch + 1) / 2, SPI = 2 * NP2;      // k pairs and steps per item
    const uint32_t nsa = (K + 127) / 128;
    constexpr uint32_t RPM = PG_ROWS / NMAT;
    const uint32_t G = gridDim.x;
    const uint32_t ring = lds_addr(p2_ring);

    const uint32_t slot = G % 8 == 0 ? (blockIdx.x % 8) * (G / 8) + blockIdx.x / 8 : blockIdx.x;
    const uint32_t first = i0 + (slot + G - i0 % G) % G;
    if (first >= n_items) return;   // uniform over the block: no barrier below is reached
    const uint32_t n_mine = (n_items - first + G - 1) / G;
    const uint32_t T = n_mine * SPI;   // steps of this group for the block (even)

    if (wave >= 8) {
        // ================= producers =================
        const uint32_t p = wave - 8;
        uint32_t pitem = first, pord = 0, ps = 0;      // item being issued, its ordinal, next step in it
        PgItem it = p2_item(A.items + pitem);
        // row offsets of copy u in half 0 / half 1 (two arrays and a select:
        // an array indexed by the run-time half would live in scratch)
        uint32_t wo0[4], wo1[4], aoff[NAI], soff = 0;
        auto setup = [&]() __attribute__((always_inline)) {
#pragma unroll
            for (uint32_t u = 0; u < 4; u++) {
                const uint32_t hr = 32 * p + 8 * u + (lane >> 3);   // row within the half
                const uint32_t n0 = it.rb * RPM + hr;
                const uint32_t n1 = it.rb * RPM + (NMAT == 2 ? hr : 128 + hr);
                wo0[u] = (n0 < N ? n0 : 0u) * RB;
                wo1[u] = (n1 < N ? n1 : 0u) * RB;
            }
            // activation copy v: routes 4 (p NAI + v) + lane / 16; block
            // scales: routes 32 p + lane / 2.  List entries past the tile's
            // count are not written: their positions read entry 0.
            const uint32_t list = ring + P2_LIST_OFF + (pord & 1u) * (uint32_t)sizeof(PgList);
#pragma unroll
            for (uint32_t v = 0; v < NAI; v++) {
                const uint32_t route = 4 * (p * NAI + v) + (lane >> 4);
                const uint32_t pos = route < it.count ? route : 0u;
                aoff[v] = min(p2_lds32(list + 512 + 4 * pos), A.a_rows - 1) * A.lda;
            }
            if (p < NAS) {
                const uint32_t route = 32 * p + (lane >> 1);
                const uint32_t pos = route < it.count ? route : 0u;
                soff = min(p2_lds32(list + 512 + 4 * pos), A.a_rows - 1) * nsa;
            }
        };
        // The scale rows of item `nx` into span slot `sslot` (as p2_range).
        auto copy_span = [&](const PgItem& nx, uint32_t sslot) __attribute__((always_inline)) -> uint32_t {
            uint32_t cnt = 0;
            uint8_t* const base = p2_ring + P2_SPAN_OFF + sslot * P2_SPAN_SLOT;
#pragma unroll
            for (uint32_t m = 0; m < (uint32_t)NMAT; m++) {
                const uint32_t rows = min(RPM, N - nx.rb * RPM), slen = rows * SB;
                const uint8_t* src = (m == 0 ? nx.s[0] : nx.s[1]) + (uint64_t)nx.rb * RPM * SB;
                const uint32_t np = (slen + 255) / 256;
                for (uint32_t q = p; q < np; q += 4) {
                    const uint32_t o = min(q * 256, slen - 256);
                    __builtin_amdgcn_global_load_lds(src + o + lane * 4, base + m * RPM * SB + o, 4, 0, 0);
                    cnt++;
                }
            }
            return cnt;
        };
        bool issuing = true;
        // Issue the next step into weight stage `wst`; returns the ops issued.
        auto issue = [&](uint32_t wst) __attribute__((always_inline)) -> uint32_t {
            if (!issuing) return 0u;
            uint32_t n = 0;
            const uint32_t h = ps & 1u, cp = ps >> 1;
            const uint8_t* wb = (NMAT == 2 && h) ? it.w[1] : it.w[0];
            uint8_t* const st = p2_ring + wst * WL_W_BYTES;
#pragma unroll
            for (uint32_t u = 0; u < 4; u++) {
                // LDS piece slot lane % 8 of row 8 (u % 2) + lane / 8 of its subtile
                const uint32_t gp = (lane & 7u) ^ ((u & 1u) * 4u + (lane >> 4));
                const uint32_t bo = cp * 128 + gp * 16;
                const uint32_t wo = h ? wo1[u] : wo0[u];
                __builtin_amdgcn_global_load_lds(wb + wo + (bo < RB ? bo : 0u), st + (4 * p + u) * 1024, 16, 0, 0);
            }
            n += 4;
            if (h == 0) {
                // the pair's activations and block scales
                uint8_t* const as_ = p2_ring + AOFF + ((pord * NP2 + cp) % NSA) * ABY;
#pragma unroll
                for (uint32_t v = 0; v < NAI; v++) {
                    const uint32_t y = p * NAI + v;
                    const uint32_t gp = (lane & 15u) ^ ((4 * y + (lane >> 4)) & 15u);
                    const uint32_t kb = cp * 256 + gp * 16;
                    __builtin_amdgcn_global_load_lds(kb < K ? A.aq + aoff[v] + kb : kZeroPage, as_ + y * 1024, 16, 0, 0);
                }
                n += NAI;
                if (p < NAS) {
                    const uint32_t c = min(2 * cp + (lane & 1u), nsa - 1);
                    __builtin_amdgcn_global_load_lds(A.as + soff + c, as_ + NR * 256 + p * 256, 4, 0, 0);
                    n += 1;
                }
            }
            // The next item's route list and scale rows, once the consumers
            // are done with the slots they go to (the item before this one).
            if (ps == NSW - 1 && pord + 1 < n_mine) {
                const PgItem nx = p2_item(A.items + pitem + G);
                if (p < 2) {
                    const PgList* src = A.lists + nx.tile;
                    uint8_t* dst = p2_ring + P2_LIST_OFF + ((pord + 1) & 1u) * (uint32_t)sizeof(PgList) + p * 1024;
                    __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint8_t*>(src) + p * 1024 + lane * 16, dst,
                                                     16, 0, 0);
                    n += 1;
                }
                n += copy_span(nx, (pord + 1) & 1u);
            }
            if (++ps == SPI) {
                ps = 0;
                pord++;
                pitem += G;
                issuing = pord < n_mine;
                if (issuing) {
                    it = p2_item(A.items + pitem);
                    setup();
                }
            }
            return n;
        };
        if (p < 2) {
            const PgList* src = A.lists + it.tile;
            __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint8_t*>(src) + p * 1024 + lane * 16,
                                             p2_ring + P2_LIST_OFF + p * 1024, 16, 0, 0);
        }
        copy_span(it, 0);
        wait_vm_imm<0>();
        __syncthreads();   // (1) the first list and scale rows are in LDS
        setup();
        uint32_t n[NSW];
        static_for<NSW>([&](auto s_) __attribute__((always_inline)) { n[decltype(s_)::value] = 0; });
        static_for<NSW - 1>([&](auto s_) __attribute__((always_inline)) {
            constexpr uint32_t st = decltype(s_)::value;
            n[st] = issue(st);
        });
        {
            uint32_t x = 0;
            static_for<NSW - 2>([&](auto q_) __attribute__((always_inline)) { x += n[decltype(q_)::value + 1]; });
            wait_vm(x);
        }
        __syncthreads();   // (2) step 0 landed
        // Step t issues step t + NSW - 1 and waits for step t + 1 (what was
        // issued after it is the last NSW - 2 batches); a bare barrier.
        for (uint32_t t = 0; t < T; t += NSW) {
            bool done = false;
            static_for<NSW>([&](auto s_) __attribute__((always_inline)) {
                constexpr uint32_t sp = decltype(s_)::value;
                if (done || t + sp >= T) {
                    done = true;
                    return;
                }
                constexpr uint32_t sn = (sp + NSW - 1) % NSW;
                n[sn] = issue(sn);
                uint32_t x = 0;
                static_for<NSW - 2>([&](auto q_) __attribute__((always_inline)) {
                    x += n[(sp + 2 + decltype(q_)::value) % NSW];
                });
                wait_vm(x);
                __builtin_amdgcn_s_barrier();
            });
        }
        return;
    }

    // ================= consumers =================
    const uint32_t wsw = (rr >> 1) & 7u;                    // this lane's row swizzle
    const uint32_t LWr = ring + (16 * wave + rr) * 128;     // + stage + piece slot * 16
    const uint32_t LAr = ring + AOFF + rr * 256;            // + slot + subtile * 4 KB + piece slot * 16
    const uint32_t LSr = ring + AOFF + NR * 256 + rr * 8;   // + slot + subtile * 128 + 4 ch
    uint32_t item = first, ord = 0;
    PgItem it = p2_item(A.items + item);
    uint32_t srow0, srow1;   // this lane's scale row of subtile 0 / 1 in the item's slot (+ 4 c + g)
    auto start_item = [&]() __attribute__((always_inline)) {
        const uint32_t b = ring + P2_SPAN_OFF + (ord & 1u) * P2_SPAN_SLOT + g;
        srow0 = b + (16 * wave + rr) * SB;
        srow1 = b + (128 + 16 * wave + rr) * SB;
    };
    v4f acc0[NAT], acc1[NAT];
#pragma unroll
    for (int a = 0; a < NAT; a++) {
        acc0[a] = v4f{0.f, 0.f, 0.f, 0.f};
        acc1[a] = v4f{0.f, 0.f, 0.f, 0.f};
    }
    __syncthreads();   // (1)
    start_item();
    __syncthreads();   // (2)
    uint32_t cp = 0;
    // One step: half H of k pair cp from weight stage t % NSW.
    auto step = [&](uint32_t t, auto h_) __attribute__((always_inline)) {
        constexpr uint32_t H = decltype(h_)::value;
        const uint32_t wst = (t % NSW) * WL_W_BYTES;
        const uint32_t ab = ((ord * NP2 + cp) % NSA) * ABY;
        const bool ch1 = 2 * cp + 1 < nch;   // the pair's second chunk exists
        v4i bw[2], alo[NAT][2], ahi[NAT][2];
        uint32_t sw[2], sa[NAT][2];
#pragma unroll
        for (uint32_t ch = 0; ch < 2; ch++) {
            asm volatile("ds_read_b128 %0, %1" : "=v"(bw[ch]) : "v"(LWr + wst + (((4 * ch + g) ^ wsw) * 16)));
            asm volatile("ds_read_u8 %0, %1" : "=v"(sw[ch]) : "v"((H ? srow1 : srow0) + 4 * (2 * cp + ch)));
#pragma unroll
            for (uint32_t a = 0; a < (uint32_t)NAT; a++) {
                const uint32_t base = LAr + ab + a * 4096;
                asm volatile("ds_read_b128 %0, %1" : "=v"(alo[a][ch]) : "v"(base + (((8 * ch + g) ^ rr) * 16)));
                asm volatile("ds_read_b128 %0, %1" : "=v"(ahi[a][ch]) : "v"(base + (((8 * ch + 4 + g) ^ rr) * 16)));
                asm volatile("ds_read_b32 %0, %1" : "=v"(sa[a][ch]) : "v"(LSr + ab + a * 128 + 4 * ch));
            }
        }
        // every result is used (even copied) only after the wait and the
        // laundering asm
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        v8i av[NAT][2];
#pragma unroll
        for (uint32_t ch = 0; ch < 2; ch++) {
            asm volatile("" : "+v"(bw[ch]), "+v"(sw[ch]));
#pragma unroll
            for (uint32_t a = 0; a < (uint32_t)NAT; a++) {
                asm volatile("" : "+v"(alo[a][ch]), "+v"(ahi[a][ch]), "+v"(sa[a][ch]));
                const v4i lo = alo[a][ch], hi = ahi[a][ch];
                av[a][ch] = v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
            }
        }
#pragma unroll
        for (uint32_t ch = 0; ch < 2; ch++) {
            if (ch == 1 && !ch1) continue;
            const uint32_t c = 2 * cp + ch;
            const uint32_t ew = 4 * c + g < SB ? sw[ch] : 127u;   // scale blocks past K (last chunk): 2^0
#pragma unroll
            for (uint32_t a = 0; a < (uint32_t)NAT; a++) {
                const uint32_t ea = (sa[a][ch] >> 23) & 0xffu;
                if constexpr (H == 0) acc0[a] = mfma_fp8_fp4(av[a][ch], bw[ch], ea, ew, acc0[a]);
                else acc1[a] = mfma_fp8_fp4(av[a][ch], bw[ch], ea, ew, acc1[a]);
            }
        }
    };
    for (uint32_t t = 0; t < T; t += 2) {
        step(t, std::integral_constant<uint32_t, 0>{});
        __builtin_amdgcn_s_barrier();
        step(t + 1, std::integral_constant<uint32_t, 1>{});
        if (cp + 1 == NP2) {
            // ---- epilogue of the item ----
            const uint32_t list = ring + P2_LIST_OFF + (ord & 1u) * (uint32_t)sizeof(PgList);
            const uint32_t count = it.count;
#pragma unroll
            for (uint32_t a = 0; a < (uint32_t)NAT; a++) {
                const uint32_t tb = 16 * a;
                if (tb >= count) continue;
                v4i rt, wv;
                asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %2 offset:1024\n\ts_waitcnt lgkmcnt(0)"
                             : "=&v"(rt), "=&v"(wv)
                             : "v"(list + (tb + 4 * g) * 4));
#pragma unroll
                for (uint32_t i = 0; i < 4; i++) {
                    const uint32_t r = (uint32_t)rt[i];
                    if (tb + 4 * g + i >= count || r >= A.routes) continue;
                    if constexpr (NMAT == 2) {
                        const uint64_t ob = (uint64_t)(r / A.k) * A.frame_elems + (uint64_t)(r % A.k) * N;
                        const uint32_t ch = it.rb * RPM + 16 * wave + rr;
                        if (ch >= N) continue;
                        float gv = round_bf16(acc0[a][i]);
                        float uv = round_bf16(acc1[a][i]);
                        if (A.limit > 0.0f) {
                            gv = fminf(gv, A.limit);
                            uv = fminf(fmaxf(uv, -A.limit), A.limit);
                        }
                        A.out[ob + ch] = (uint16_t)f32_to_bf16(silu_fast(gv) * uv);
                    } else {
                        const float wr = __int_as_float(wv[i]);
                        const uint32_t row0 = it.rb * RPM + 16 * wave + rr, row1 = row0 + 128;
                        if (row0 < N) A.out[(uint64_t)r * N + row0] = (uint16_t)f32_to_bf16(acc0[a][i] * wr);
                        if (row1 < N) A.out[(uint64_t)r * N + row1] = (uint16_t)f32_to_bf16(acc1[a][i] * wr);
                    }
                }
            }
#pragma unroll
            for (int a = 0; a < NAT; a++) {
                acc0[a] = v4f{0.f, 0.f, 0.f, 0.f};
                acc1[a] = v4f{0.f, 0.f, 0.f, 0.f};
            }
            cp = 0;
            ord++;
            item += G;
            if (ord < n_mine) {
                it = p2_item(A.items + item);
                start_item();
            }
        } else {
            cp++;
        }
        __builtin_amdgcn_s_barrier();
    }
}

template <int NMAT>
__global__ __launch_bounds__(768) void moe_pg2_kernel(PgArgs A) {
    constexpr uint32_t RPM = PG_ROWS / NMAT;
    const uint32_t nrb = (A.N + RPM - 1) / RPM;
    const uint32_t nt = __builtin_amdgcn_readfirstlane(A.n_tiles[0]);
    const uint32_t nt0 = __builtin_amdgcn_readfirstlane(A.n_tiles[1]);
    const uint32_t nt1 = __builtin_amdgcn_readfirstlane(A.n_tiles[2]);
    p2_range<NMAT, 8, 4, 4>(A, 0, nt0 * nrb);
    __syncthreads();
    // Tiles of 33-64 and of 1-32 routes: the whole-line form (the 128-route
    // tiles' activation slots would not fit its LDS ring).
    p2_range_wl<NMAT, 4>(A, nt0 * nrb, (nt0 + nt1) * nrb);
    __syncthreads();
    p2_range_wl<NMAT, 2>(A, (nt0 + nt1) * nrb, nt * nrb);
}

template <int NMAT>
nerve_hip_status launch_pg2(const PgArgs& A, const nerve_hip_ctx* ctx, hipStream_t st) {
    static bool attr_set = false;
    if (!attr_set) {
        if (hipFuncSetAttribute((const void*)moe_pg2_kernel<NMAT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                P2_LDS) != hipSuccess)
            return nh::fail(NERVE_HIP_DEVICE_ERROR, "hipFuncSetAttribute failed for moe_pg2_kernel");
        attr_set = true;
    }
    moe_pg2_kernel<NMAT><<<ctx->cu_count, 768, P2_LDS, st>>>(A);
    return nh::check_launch("moe_pg2_kernel");
}

template <int NMAT>
nerve_hip_status launch_pgemm(const PgArgs& A, const nerve_hip_ctx* ctx, hipStream_t st) {
    static bool attr_set = false;
    if (!attr_set) {
        if (hipFuncSetAttribute((const void*)moe_pgemm_kernel<NMAT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                160 * 1024) != hipSuccess)
            return nh::fail(NERVE_HIP_DEVICE_ERROR, "hipFuncSetAttribute failed for moe_pgemm_kernel");
        attr_set = true;
    }
    moe_pgemm_kernel<NMAT><<<ctx->cu_count, 512, pg_lds_bytes(A.K), st>>>(A);
    return nh::check_launch("moe_pgemm_kernel");
}

nerve_hip_status launch_quant(const QuantArgs& Q, bool pow2, hipStream_t st) {
    if (Q.rows == 0) return nh::ok();
    const uint64_t units = (uint64_t)Q.rows * ((Q.cols + 127) / 128);
    const uint32_t blocks = (uint32_t)((units + 7) / 8);
    if (pow2)
        quant_rows_kernel<true><<<blocks, 256, 0, st>>>(Q);
    else
        quant_rows_kernel<false><<<blocks, 256, 0, st>>>(Q);
    return nh::check_launch("quantize_fp8_e4m3");
}

QuantArgs plain_rows(const uint16_t* x, uint32_t cols, uint32_t rows, uint8_t* q, float* s) {
    QuantArgs Q;
    Q.x = x;
    Q.k = 1;
    Q.frame_elems = cols;
    Q.seg_elems = cols;
    Q.cols = cols;
    Q.rows = rows;
    Q.q = q;
    Q.s = s;
    Q.zero_word = nullptr;
    Q.ldq = cols;
    return Q;
}

}  // namespace

namespace nh {
nerve_hip_status quantize_rows(const uint16_t* x, uint32_t cols, uint32_t rows, bool pow2, uint8_t* q, float* s,
                               hipStream_t st, uint32_t* zero_word) {
    QuantArgs Q = plain_rows(x, cols, rows, q, s);
    Q.zero_word = zero_word;
    return launch_quant(Q, pow2, st);
}
}  // namespace nh

// ---------------------------------------------------------------------------
// Tensor-parallel expert slices (…gate_up_batch1_mxfp4.comp.template:487-641,
// …down_batch1_mxfp4.comp.template:421-505): one rank's share of an expert
// projection.  On one GPU the ranks' shares are separate calls.
//  - gate_up: the expert's gate/up records cover the rank's rows [0, L) of
//    the intermediate, L = gate weight bytes / (H / 2); the output is bf16
//    route-major local rows [B][k][L].
//  - down: the local intermediate slice [B][k][count] (count = range[1])
//    against input-block-major down weights whose records start at the
//    slice's first 128-column block; the output is f32 [B][k][H], not scaled
//    by the route weight (the ranks' partials are summed, then scaled).
// Block = (tile of 32 gate_up / 64 down rows, token b), 4 waves of 16 rows
// (gate_up: waves 0-1 gate, 2-3 up).  The token's routes run in order; the
// first route whose expert is out of range or has an invalid record ends the
// block, as the reference's `return` does, so that token's later routes keep
// whatever their outputs held.  The activation row is quantized into LDS
// (pow2 block scales, zero past K); every lane of a wave feeds the same
// token to the MFMA's 16 activation rows.
// ---------------------------------------------------------------------------
constexpr uint32_t TP_MAX_K = 4096;   // contraction length staged in LDS

struct TpArgs {
    const uint16_t* x;        // gate_up: hidden bf16 [B, H]; down: local intermediates bf16 [B, k, count]
    const uint8_t* xq;        // gate_up with prequantized input: e4m3 [B, H]
    const float* xs;          //   and its pow2 block scales [B, ceil(H / 128)]
    const uint32_t* routes;   // [B, k]
    const uint32_t* addr;
    uint32_t n_records;
    const uint32_t* slots;
    uint32_t n_slot_words;
    const uint32_t* range;    // down: {input_start, input_count}
    uint16_t* out16;          // gate_up
    float* out32;             // down
    uint32_t H, I, E, k;
    float limit;
};

template <bool GU>
__device__ __forceinline__ void mx_tp_body(const TpArgs& A) {
    constexpr uint32_t TR = GU ? 32 : 64, P = GU ? 4 : 2;
    __shared__ __attribute__((aligned(16))) uint8_t q[TP_MAX_K];
    __shared__ float qs[TP_MAX_K / 128];
    __shared__ float gu[2][32];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, rr = lane & 15;
    const uint32_t b = blockIdx.y, first = blockIdx.x * TR;
    const uint32_t H = A.H;
    // contraction length: H, or the slice's column count (a multiple of 32,
    // at most I, else the launch writes nothing); it is also the row stride
    // of the local frames
    const uint32_t cnt = GU ? 0u : A.range[1];
    if (!GU && (cnt % 32 != 0 || cnt > A.I)) return;
    const uint32_t K = GU ? H : cnt;
    const uint32_t nch = (K + 127) / 128;
    const bool preq = GU && A.xq != nullptr;
    // Quantize bf16 row xr (K columns) into q / qs: one 32-lane cluster per
    // 128-column block, the same arithmetic as quant_unit.
    auto quantize = [&](const uint16_t* xr) {
        for (uint32_t blk = tid >> 5; blk < nch; blk += 8) {
            const uint32_t cl = tid & 31, col = blk * 128 + cl * 4;
            const bool valid = col < K;
            float v[4] = {0.f, 0.f, 0.f, 0.f};
            if (valid) {
                const uint32_t* p = reinterpret_cast<const uint32_t*>(xr + col);
                const uint32_t w0 = p[0], w1 = p[1];
                v[0] = bf16_to_f32(w0); v[1] = bf16_to_f32(w0 >> 16);
                v[2] = bf16_to_f32(w1); v[3] = bf16_to_f32(w1 >> 16);
            }
            float m = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
            m = wave_max32(m);
            const float sc = pow2_fp8_scale(m);
            if (cl == 0) qs[blk] = sc;
            const uint32_t packed = valid ? (f32_to_e4m3(v[0] / sc) | (f32_to_e4m3(v[1] / sc) << 8) |
                                             (f32_to_e4m3(v[2] / sc) << 16) | (f32_to_e4m3(v[3] / sc) << 24))
                                          : 0u;
            *reinterpret_cast<uint32_t*>(q + col) = packed;
        }
    };
    if (GU && !preq) {
        quantize(A.x + (uint64_t)b * H);
        __syncthreads();
    }
    for (uint32_t r = 0; r < A.k; r++) {
        const uint32_t e = A.routes[(uint64_t)b * A.k + r] & 0xffffu;
        // Validity of the expert's records (uniform over the block).  The
        // reference asks for one row (gate_up) or one 128-column block
        // (down); here every record must also cover what is read: the L
        // local rows of all four gate_up records (L from the gate weight
        // record), every block of the down slice.
        bool ok = e < A.E;
        uint32_t rec[P][8];
        uint32_t slot[P];
#pragma unroll
        for (uint32_t p = 0; p < P; p++) {
            const uint32_t idx = e * P + p;
            slot[p] = (ok && idx < A.n_slot_words) ? A.slots[idx] : UNBOUND_SLOT;
            const bool has = slot[p] != UNBOUND_SLOT && slot[p] < A.n_records;
#pragma unroll
            for (uint32_t j = 0; j < 8; j++) rec[p][j] = has ? A.addr[(uint64_t)slot[p] * 8 + j] : 0u;
        }
        const uint64_t gbytes = (uint64_t)rec[0][2] | ((uint64_t)rec[0][3] << 32);
        const uint64_t L64 = GU ? gbytes / (H / 2) : H;
        const uint32_t L = L64 > 0xffffffffull ? 0xffffffffu : (uint32_t)L64;
        const uint64_t nb = nch > 0 ? nch : 1u;
#pragma unroll
        for (uint32_t p = 0; p < P; p++) {
            const bool is_w = (p % 2) == 0;
            const uint64_t need = GU ? (is_w ? (uint64_t)(H / 2) : (uint64_t)((H + 31) / 32)) * (L64 > 0 ? L64 : 1u)
                                     : (is_w ? nb * H * 64 : nb * H * 4);
            ok = record_valid(slot[p], A.n_records, rec[p], need, is_w ? 16u : 4u) && ok;
        }
        if (!ok) return;
        auto ptr = [&](uint32_t p) {
            return reinterpret_cast<const uint8_t*>((uint64_t)rec[p][0] | ((uint64_t)rec[p][1] << 32));
        };
        if constexpr (!GU) {
            quantize(A.x + ((uint64_t)b * A.k + r) * cnt);
            __syncthreads();
        }
        const uint32_t m = GU ? (wave >> 1) : 0u;
        const uint32_t row = first + (GU ? 16 * (wave & 1u) : 16 * wave) + rr;
        const uint32_t lrow = row < L ? row : 0u;   // rows past the slice read row 0 and are not written
        const uint8_t* W = ptr(GU ? 2 * m : 0);
        const uint8_t* S = ptr(GU ? 2 * m + 1 : 1);
        v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
        if (first < L) {
            for (uint32_t c = 0; c < nch; c++) {
                v8i av;
                uint32_t sa;
                if (preq) {
                    load_a(A.xq + (uint64_t)b * H, A.xs + (uint64_t)b * nch, K, c, g, av, sa);
                } else {
                    const uint32_t k0 = c * 128 + g * 16;
                    const v4i lo = *reinterpret_cast<const v4i*>(q + k0);
                    const v4i hi = *reinterpret_cast<const v4i*>(q + k0 + 64);
                    av = v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
                    sa = pow2_to_e8m0(qs[c]);
                }
                v4i w;
                uint32_t sw;
                if constexpr (GU) {
                    load_w(W + (uint64_t)lrow * (H / 2), S + (uint64_t)lrow * ((H + 31) / 32), K, c, g, w, sw);
                } else {
                    // input-block-major: W [blocks][H][64 B], S [blocks][H][4 B]
                    if (c * 128 + g * 32 < K) {
                        w = *reinterpret_cast<const v4i*>(W + ((uint64_t)c * H + lrow) * 64 + g * 16);
                        sw = S[((uint64_t)c * H + lrow) * 4 + g];
                    } else {
                        w = v4i{0, 0, 0, 0};
                        sw = 127;
                    }
                }
                acc = mfma_fp8_fp4(av, w, sa, sw, acc);
            }
        }
        // every activation row is the token: D[0][rr] is row `row`'s sum
        if constexpr (GU) {
            if (g == 0) gu[m][16 * (wave & 1u) + rr] = acc[0];
            __syncthreads();
            if (tid < TR) {
                const uint32_t orow = first + tid;
                if (orow < L) {
                    float gv = round_bf16(gu[0][tid]);
                    float uv = round_bf16(gu[1][tid]);
                    if (A.limit > 0.0f) {
                        gv = fminf(gv, A.limit);
                        uv = fminf(fmaxf(uv, -A.limit), A.limit);
                    }
                    A.out16[((uint64_t)b * A.k + r) * L + orow] = (uint16_t)f32_to_bf16(silu_fast(gv) * uv);
                }
            }
        } else {
            if (g == 0 && row < H) A.out32[((uint64_t)b * A.k + r) * H + row] = acc[0];
        }
        __syncthreads();   // LDS (activations, exchange) reused by the next route
    }
}

__global__ __launch_bounds__(256) void mx_tp_gate_up_kernel(TpArgs A) { mx_tp_body<true>(A); }
__global__ __launch_bounds__(256) void mx_tp_down_kernel(TpArgs A) { mx_tp_body<false>(A); }

static nerve_hip_status moe_tensor_parallel(const nh::MoeSpec& ms, bool gate_up, const void* act, const void* pre_s,
                                            const void* routes, void* out, const void* addresses,
                                            uint32_t address_records, const void* slots, uint32_t slot_words,
                                            const void* range, uint32_t batch_width, hipStream_t stream) {
    if (ms.weight_repr != 0)
        return nh::fail(NERVE_HIP_UNSUPPORTED, "tensor-parallel slices are supported for compact MXFP4 experts");
    if ((gate_up ? ms.hidden : ms.inter) > TP_MAX_K)
        return nh::fail(NERVE_HIP_UNSUPPORTED, "tensor-parallel slices contract at most 4096 columns");
    if ((uintptr_t)addresses & 15)
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "the address record table must be 16-byte aligned");
    if (batch_width == 0) return nh::ok();
    if (batch_width > 65535) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "batch too large");
    TpArgs A{};
    A.routes = static_cast<const uint32_t*>(routes);
    A.addr = static_cast<const uint32_t*>(addresses);
    A.n_records = address_records;
    A.slots = static_cast<const uint32_t*>(slots);
    A.n_slot_words = slot_words;
    A.H = ms.hidden;
    A.I = ms.inter;
    A.E = ms.experts;
    A.k = ms.k;
    A.limit = ms.limit;
    if (gate_up) {
        if (ms.prequant) {
            A.xq = static_cast<const uint8_t*>(act);
            A.xs = static_cast<const float*>(pre_s);
        } else {
            if (((uintptr_t)act & 3) || ms.hidden % 2)
                return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "hidden rows must be 4-byte aligned");
            A.x = static_cast<const uint16_t*>(act);
        }
        A.out16 = static_cast<uint16_t*>(out);
        mx_tp_gate_up_kernel<<<dim3((ms.inter + 31) / 32, batch_width), 256, 0, stream>>>(A);
    } else {
        if ((uintptr_t)act & 3) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "intermediates must be 4-byte aligned");
        A.x = static_cast<const uint16_t*>(act);
        A.range = static_cast<const uint32_t*>(range);
        A.out32 = static_cast<float*>(out);
        mx_tp_down_kernel<<<dim3((ms.hidden + 63) / 64, batch_width), 256, 0, stream>>>(A);
    }
    return nh::check_launch(gate_up ? "mx_tp_gate_up_kernel" : "mx_tp_down_kernel");
}

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
    return launch_quant(plain_rows(static_cast<const uint16_t*>(x_bf16), qs.elements, rows, static_cast<uint8_t*>(q_e4m3),
                                   static_cast<float*>(scales_f32)),
                        qs.pow2, (hipStream_t)stream);
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
    if (K <= 4096 && ((uintptr_t)weight_scale & 3) == 0) {
        SpanArgs sa{};
        sa.aq = static_cast<const uint8_t*>(q_e4m3);
        sa.as = static_cast<const float*>(scales_f32);
        sa.a_row_div = 1;
        sa.K = K;
        sa.N = N;
        sa.k = 1;
        sa.M = M;
        sa.w_direct = static_cast<const uint8_t*>(weight);
        sa.s_direct = static_cast<const uint8_t*>(weight_scale);
        sa.out32 = static_cast<float*>(y_f32);
        // Rows per block: one block per CU when N allows (a multiple of 8 rows,
        // so every block's weight and scale spans keep 16- and 4-byte
        // alignment), 16 to 32 rows; 16-row blocks leave some CUs two blocks
        // while others have one.
        const uint32_t cu = (uint32_t)ctx->cu_count;
        const uint32_t want = ((N + cu - 1) / cu + 7) / 8 * 8;
        if (want > 16 && want <= 32 && (uint64_t)want * (K / 32) % 4 == 0) {
            sa.rpb = want;
            return launch_span<SPAN_RAW, 1, 2, 8>(sa, (M + 15) / 16, (hipStream_t)stream);
        }
        return launch_span<SPAN_RAW, 1, 1, 8>(sa, (M + 15) / 16, (hipStream_t)stream);
    }
    mxfp4_gemv_kernel<8><<<N / 16, 512, 0, (hipStream_t)stream>>>(
        static_cast<const uint8_t*>(q_e4m3), static_cast<const float*>(scales_f32), M, K,
        static_cast<const uint8_t*>(weight), static_cast<const uint8_t*>(weight_scale), N, static_cast<float*>(y_f32));
    return nh::check_launch("mxfp4_gemv");
}

// control[4] as the count stage writes it after a compaction of the same
// routes (control[3], [5] and [6] already hold its values).
__global__ __launch_bounds__(64) void count_control_kernel(uint32_t* control, uint32_t k, uint32_t tiles) {
    if (threadIdx.x == 0) control[4] = (control[2] != 0u ? control[3] : k) * tiles;
}

static nerve_hip_status moe_common(nerve_hip_ctx* ctx, const nh::MoeSpec& ms, bool gate_up, const void* act_bf16,
                                   const void* pre_q, const void* pre_s, const void* routes, void* intermediates,
                                   void* expert_outputs, const void* addresses, uint32_t address_records,
                                   const void* slots, uint32_t slot_words, const void* control, uint32_t batch_width,
                                   hipStream_t stream, uint32_t* count_control = nullptr) {
    const uint32_t H = ms.hidden, I = ms.inter, k = ms.k, E = ms.experts;
    const uint32_t cap = batch_width * k;
    if (cap == 0) {
        if (!count_control) return nh::ok();
        count_control_kernel<<<1, 64, 0, stream>>>(count_control, k, (H + 63) / 64);
        return nh::check_launch("moe_route_count");
    }
    // Address records are read as two 16-byte loads each.
    if ((uintptr_t)addresses & 15)
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "the address record table must be 16-byte aligned");
    const uint32_t K = gate_up ? H : I;       // contraction
    const uint32_t N = gate_up ? I : H;       // output rows per matrix
    const uint32_t nblk = (K + 127) / 128;
    const uint32_t arows = gate_up ? batch_width : cap;
    // Decode-shaped batches stream each expert's weights once per <= 16
    // routes; prefill-shaped batches use the LDS-staged grouped GEMM with
    // 64-route tiles.
    // Banks with e4m3 weights (pre-expanded or native FP8 experts) take the
    // preparation launch and mx_wfmt_kernel at every batch size.
    // The block-major down layout is streamed by the decode kernel and
    // otherwise takes the same register-fed kernel.
    const bool banks = ms.weight_repr != 0 || ms.native_fp8_start >= 0;
    const bool wf = banks || ms.input_block_major;
    if (wf && E > 1024)
        return nh::fail(NERVE_HIP_UNSUPPORTED, "e4m3 expert banks and block-major weights are supported for E <= 1024");
    const bool grouped = !wf && (cap >= 512 || K > 4096);
    // Persistent grouped GEMM: enough chunks per item for the descriptor
    // prefetch rounds, the item's scale spans fit the LDS, and every span is
    // a whole number of dwords of at least 256 bytes (copied in 256-byte
    // pieces, the last aligned to the span's end).
    const uint32_t pg_rpm = gate_up ? PG_ROWS / 2 : PG_ROWS, pg_tail = N % pg_rpm;
    const bool persistent = grouped && (K + PG_KC - 1) / PG_KC >= PG_MIN_CHUNKS && pg_lds_bytes(K) <= 160 * 1024 &&
                            (pg_tail * (K / 32)) % 4 == 0 && (pg_tail == 0 || pg_tail * (K / 32) >= 256);
    const uint32_t TM = persistent ? PG_TM : grouped ? 64 : 16;
    const uint32_t max_tiles = (cap + TM - 1) / TM + (E < cap ? E : cap);
    // The persistent GEMM copies activations in 128-byte row pieces: rows it
    // quantizes itself start on 128-byte boundaries (prequantized rows keep
    // the caller's stride K).
    const bool own_q = !(gate_up && ms.prequant);
    const uint32_t lda = persistent && own_q ? (K + 127) / 128 * 128 : K;
    nh::Carver cv;
    size_t o_aq = cv.take<uint8_t>((size_t)arows * lda);
    size_t o_as = cv.take<float>((size_t)arows * nblk);
    size_t o_seg = cv.take<uint32_t>(cap + 16);   // +16: the streaming kernel reads 16 entries at once
    size_t o_rec = cv.take<TileRec>(max_tiles);
    size_t o_nt = cv.take<uint32_t>(4);   // tiles; persistent GEMM: tiles of the first two route-count groups
    const uint32_t item_nrb = (N + (gate_up ? PG_ROWS / 2 : PG_ROWS) - 1) / (gate_up ? PG_ROWS / 2 : PG_ROWS);
    size_t o_items = cv.take<ItemRec>(persistent ? (size_t)max_tiles * item_nrb : 0);
    size_t o_lists = cv.take<PgList>(persistent ? max_tiles : 0);
    void* ws = nullptr;
    nerve_hip_status st = nh::workspace(ctx, cv.offset, &ws);
    if (st) return st;
    uint8_t* base = static_cast<uint8_t*>(ws);
    uint8_t* aq = base + o_aq;
    float* as = reinterpret_cast<float*>(base + o_as);
    const uint64_t frame_words = (uint64_t)k * I / 2 + k;
    const uint16_t* frames16 = static_cast<const uint16_t*>(intermediates);

    // Activation rows to quantize in the preparation launch: the hidden rows
    // for gate_up (quantize_hidden, …gate_up_batch1_mxfp4.comp.template:
    // 366-382), every route slice of the intermediate frames for down
    // (quantize_intermediate, …down_batch1_mxfp4.comp.template:332-353).
    QuantArgs Q;
    Q.zero_word = nullptr;
    if (gate_up) {
        Q = plain_rows(static_cast<const uint16_t*>(act_bf16), H, batch_width, aq, as);
        Q.ldq = lda;
        if (ms.prequant) {
            aq = const_cast<uint8_t*>(static_cast<const uint8_t*>(pre_q));
            as = const_cast<float*>(static_cast<const float*>(pre_s));
            Q.rows = 0;
        }
    } else {
        Q.x = frames16;
        Q.k = k;
        Q.frame_elems = frame_words * 2;
        Q.seg_elems = I;
        Q.cols = I;
        Q.rows = cap;
        Q.q = aq;
        Q.s = as;
        Q.ldq = lda;
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
    ta.wmode = (uint32_t)ms.weight_repr;
    ta.native_start = ms.native_fp8_start >= 0 ? (uint32_t)ms.native_fp8_start : 0xffffffffu;
    ta.req_w8 = (uint64_t)N * K;
    ta.req_sn = (uint64_t)((N + 127) / 128) * ((K + 127) / 128);
    ta.req_s = (uint64_t)N * K / 32;
    ta.TM = TM;
    ta.max_tiles = max_tiles;
    ta.seg_list = reinterpret_cast<uint32_t*>(base + o_seg);
    ta.recs = reinterpret_cast<TileRec*>(base + o_rec);
    ta.n_tiles = reinterpret_cast<uint32_t*>(base + o_nt);
    ta.items = persistent ? reinterpret_cast<ItemRec*>(base + o_items) : nullptr;
    ta.item_nrb = item_nrb;
    ta.lists = persistent ? reinterpret_cast<PgList*>(base + o_lists) : nullptr;
    ta.a_row_div = gate_up ? k : 1;
    // Decode-shaped batches: one streaming launch that builds its own tiles
    // and quantizes its own activation chunks (no preparation launch).
    if (!banks && !grouped) {
        StreamArgs fa{};
        fa.K = K;
        fa.N = N;
        fa.k = k;
        fa.a_row_div = gate_up ? k : 1;
        fa.routes = ta.routes;
        fa.frame_elems = frame_words * 2;
        fa.limit = ms.limit;
        fa.T = ta;
        if (gate_up) {
            fa.x16 = static_cast<const uint16_t*>(act_bf16);
            fa.x_frame = H;
            fa.x_seg = 0;
            fa.out16 = static_cast<uint16_t*>(intermediates);
            if (ms.prequant) {
                // Only the token form reads prequantized rows in its fused
                // set-up; other decode shapes take the preparation launch.
                fa.aq = static_cast<const uint8_t*>(pre_q);
                fa.as = static_cast<const float*>(pre_s);
                st = launch_tokens<3, 8>(fa, ctx, stream);
            } else {
                st = launch_tokens<3, 8>(fa, ctx, stream);
                if (st == NERVE_HIP_UNSUPPORTED) st = launch_stream<SPAN_GATE_UP, 2, 3, 8, 1, true>(fa, ctx, stream);
            }
        } else {
            fa.x16 = frames16;
            fa.x_frame = frame_words * 2;
            fa.x_seg = I;
            fa.out16 = static_cast<uint16_t*>(expert_outputs);
            fa.count_control = count_control;
            fa.count_tiles = (H + 63) / 64;
            fa.block_major = ms.input_block_major ? 1u : 0u;
            st = launch_stream<SPAN_DOWN, 1, 3, 8, 2, true>(fa, ctx, stream);
            if (st == NERVE_HIP_OK) count_control = nullptr;
        }
        if (st != NERVE_HIP_UNSUPPORTED) return st;
    }
    if (count_control) {
        // Count stage as its own launch (its one changed word, computed the
        // same way) for the other down paths.
        count_control_kernel<<<1, 64, 0, stream>>>(count_control, k, (H + 63) / 64);
        if ((st = nh::check_launch("moe_route_count"))) return st;
    }
    const uint64_t units = (uint64_t)Q.rows * ((Q.cols + 127) / 128);
    {
        // Block 0 builds the tiles; the others stride over the quantization
        // units (a few per CU keep the loads in flight).
        Q.vec8 = ((((uintptr_t)Q.x | (uintptr_t)Q.q) & 15) == 0 && Q.cols % 8 == 0 && Q.ldq % 8 == 0 &&
                  Q.frame_elems % 8 == 0 &&
                  Q.seg_elems % 8 == 0 && Q.rows > 0) ? 1u : 0u;
        const uint32_t per_pass = Q.vec8 ? 64 * PREP_QU : 32;
        const uint32_t qblocks =
            (uint32_t)std::min<uint64_t>((units + per_pass - 1) / per_pass, (uint64_t)4 * ctx->cu_count);
        if (E <= 1024) moe_prep_kernel<1024><<<1 + qblocks, 1024, 0, stream>>>(ta, Q);
        else moe_prep_kernel<MAX_EXPERTS><<<1 + qblocks, 1024, 0, stream>>>(ta, Q);
    }
    if ((st = nh::check_launch("moe_prep"))) return st;

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
    ea.recs = ta.recs;
    ea.n_tiles = ta.n_tiles;
    ea.frame_elems = frame_words * 2;
    ea.limit = ms.limit;
    if (wf) {
        SpanArgs wa{};
        wa.aq = aq;
        wa.as = as;
        wa.a_row_div = ea.a_row_div;
        wa.K = K;
        wa.N = N;
        wa.k = k;
        wa.routes = ea.routes;
        wa.seg_list = ea.seg_list;
        wa.recs = ea.recs;
        wa.n_tiles = ea.n_tiles;
        wa.frame_elems = ea.frame_elems;
        wa.limit = ea.limit;
        wa.block_major = ms.input_block_major ? 1u : 0u;
        const dim3 wgrid((N + 15) / 16, max_tiles);
        if (gate_up) {
            wa.out16 = static_cast<uint16_t*>(intermediates);
            mx_wfmt_kernel<SPAN_GATE_UP, 2><<<wgrid, 256, 0, stream>>>(wa);
        } else {
            wa.out16 = static_cast<uint16_t*>(expert_outputs);
            mx_wfmt_kernel<SPAN_DOWN, 1><<<wgrid, 256, 0, stream>>>(wa);
        }
        return nh::check_launch("mx_wfmt_kernel");
    }
    if (persistent) {
        // Producer / consumer form: the item's scale rows fit their LDS
        // slot and an item has enough chunks for the descriptor prefetch.
        const bool p2_ok = K % 32 == 0 && K / 32 <= P2_MAX_SB && (K + P2_KC - 1) / P2_KC >= P2_MIN_CHUNKS;
        PgArgs pa;
        pa.aq = aq;
        pa.lda = lda;
        pa.as = as;
        pa.a_rows = arows;
        pa.routes = cap;
        pa.K = K;
        pa.N = N;
        pa.k = k;
        pa.items = ta.items;
        pa.lists = ta.lists;
        pa.n_tiles = ta.n_tiles;
        pa.frame_elems = frame_words * 2;
        pa.limit = ms.limit;
        if (gate_up) {
            pa.out = static_cast<uint16_t*>(intermediates);
            if (p2_ok) return launch_pg2<2>(pa, ctx, stream);
            return launch_pgemm<2>(pa, ctx, stream);
        }
        pa.out = static_cast<uint16_t*>(expert_outputs);
        if (p2_ok) return launch_pg2<1>(pa, ctx, stream);
        return launch_pgemm<1>(pa, ctx, stream);
    }
    if (grouped) {
        const uint32_t rows_per_block = gate_up ? 64 : 128;
        dim3 ggrid(max_tiles, (N + rows_per_block - 1) / rows_per_block);
        const bool async_ok = K <= GS_MAX_K && K % 32 == 0;
        ea.max_tiles = max_tiles;
        ea.work_items = ggrid.x * ggrid.y;
        const uint32_t flat = (ea.work_items + 7) / 8 * 8;
        if (gate_up) {
            ea.out = static_cast<uint16_t*>(intermediates);
            if (async_ok) moe_grouped_async_kernel<2><<<flat, 256, 0, stream>>>(ea);
            else moe_grouped_kernel<2><<<ggrid, 256, 0, stream>>>(ea);
            return nh::check_launch("moe_gate_up_grouped");
        }
        ea.out = static_cast<uint16_t*>(expert_outputs);
        if (async_ok) moe_grouped_async_kernel<1><<<flat, 256, 0, stream>>>(ea);
        else moe_grouped_kernel<1><<<ggrid, 256, 0, stream>>>(ea);
        return nh::check_launch("moe_down_grouped");
    }
    {
        SpanArgs sa{};
        sa.aq = aq;
        sa.as = as;
        sa.a_row_div = ea.a_row_div;
        sa.K = K;
        sa.N = N;
        sa.k = k;
        sa.addr = ea.addr;
        sa.slots = ea.slots;
        sa.P = ea.P;
        sa.routes = ea.routes;
        sa.seg_list = ea.seg_list;
        sa.recs = ea.recs;
        sa.n_tiles = ea.n_tiles;
        sa.frame_elems = ea.frame_elems;
        sa.limit = ea.limit;
        StreamArgs qa{};
        qa.aq = aq;
        qa.as = as;
        qa.a_row_div = ea.a_row_div;
        qa.K = K;
        qa.N = N;
        qa.k = k;
        qa.routes = ea.routes;
        qa.seg_list = ea.seg_list;
        qa.recs = ea.recs;
        qa.n_tiles = ea.n_tiles;
        qa.frame_elems = ea.frame_elems;
        qa.limit = ea.limit;
        if (gate_up) {
            sa.out16 = qa.out16 = static_cast<uint16_t*>(intermediates);
            st = launch_stream<SPAN_GATE_UP, 2, 3, 8, 1, false>(qa, ctx, stream);
            if (st != NERVE_HIP_UNSUPPORTED) return st;
            return launch_span<SPAN_GATE_UP, 2, 1>(sa, max_tiles, stream);
        }
        sa.out16 = qa.out16 = static_cast<uint16_t*>(expert_outputs);
        st = launch_stream<SPAN_DOWN, 1, 3, 8, 2, false>(qa, ctx, stream);
        if (st != NERVE_HIP_UNSUPPORTED) return st;
        return launch_span<SPAN_DOWN, 1, 2>(sa, max_tiles, stream);
    }
    return nh::fail(NERVE_HIP_UNSUPPORTED, "no MXFP4 expert kernel for this shape");
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
    if (ms.family != 0) return nh::fail(NERVE_HIP_INVALID_SPEC, std::string("not an MXFP4 expert kernel: ") + spec);
    if (!ms.gate_up) return nh::fail(NERVE_HIP_INVALID_SPEC, "gate_up entry given a down specialization");
    if (!hidden || !routes_u32 || !intermediates || !addresses_u32 || !param_slots_u32 || !control_u32 ||
        (ms.prequant && !hidden_scales))
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "null buffer");
    if (ms.prequant && ((uintptr_t)hidden & 15)) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "prequantized hidden must be 16-byte aligned");
    if (ms.prequant && ((uintptr_t)hidden_scales & 3)) return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "hidden scales must be 4-byte aligned");
    if (ms.tensor_parallel)
        return moe_tensor_parallel(ms, true, hidden, hidden_scales, routes_u32, intermediates, addresses_u32,
                                   address_records, param_slots_u32, param_slot_words, nullptr, batch_width,
                                   (hipStream_t)stream);
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
    if (ms.family != 0) return nh::fail(NERVE_HIP_INVALID_SPEC, std::string("not an MXFP4 expert kernel: ") + spec);
    if (ms.gate_up) return nh::fail(NERVE_HIP_INVALID_SPEC, "down entry given a gate_up specialization");
    if (!intermediates || !routes_u32 || !expert_outputs || !addresses_u32 || !param_slots_u32 || !control_u32)
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "null buffer");
    if (ms.tensor_parallel)
        return moe_tensor_parallel(ms, false, intermediates, nullptr, routes_u32, expert_outputs, addresses_u32,
                                   address_records, param_slots_u32, param_slot_words, control_u32, batch_width,
                                   (hipStream_t)stream);
    return moe_common(ctx, ms, false, nullptr, nullptr, nullptr, routes_u32, const_cast<void*>(intermediates),
                      expert_outputs, addresses_u32, address_records, param_slots_u32, param_slot_words, control_u32,
                      batch_width, (hipStream_t)stream);
}

nerve_hip_status nerve_hip_mxfp4_moe_down_counted(nerve_hip_ctx* ctx, const char* spec, const void* intermediates,
                                                  const void* routes_u32, void* expert_outputs,
                                                  const void* addresses_u32, uint32_t address_records,
                                                  const void* param_slots_u32, uint32_t param_slot_words,
                                                  void* control_u32, uint32_t batch_width, void* stream) {
    nerve_hip_status st = nh::enter(ctx);
    if (st) return st;
    nh::MoeSpec ms;
    if ((st = nh::parse_moe_spec(spec, &ms))) return st;
    if (ms.family != 0) return nh::fail(NERVE_HIP_INVALID_SPEC, std::string("not an MXFP4 expert kernel: ") + spec);
    if (ms.gate_up) return nh::fail(NERVE_HIP_INVALID_SPEC, "down entry given a gate_up specialization");
    if (!intermediates || !routes_u32 || !expert_outputs || !addresses_u32 || !param_slots_u32 || !control_u32)
        return nh::fail(NERVE_HIP_INVALID_ARGUMENT, "null buffer");
    if (ms.tensor_parallel)
        return nh::fail(NERVE_HIP_INVALID_SPEC, "a tensor-parallel down slice takes no count stage (its push constants are the input range)");
    return moe_common(ctx, ms, false, nullptr, nullptr, nullptr, routes_u32, const_cast<void*>(intermediates),
                      expert_outputs, addresses_u32, address_records, param_slots_u32, param_slot_words, control_u32,
                      batch_width, (hipStream_t)stream, static_cast<uint32_t*>(control_u32));
}

}  // extern "C"
