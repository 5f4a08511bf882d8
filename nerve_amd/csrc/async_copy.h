// Device helpers of the asynchronous global -> LDS pipelines (gfx950):
// explicit vmcnt waits for copies issued with global_load_lds, inline-asm
// LDS and global accesses the compiler's wait insertion does not pair with
// those copies, and cross-lane maxima that stay off the LDS.
#pragma once

#include <utility>

#include "common.h"

namespace {

template <uint32_t N>
__device__ __forceinline__ void wait_vm_imm() {
    // gfx9 s_waitcnt: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8.
    __builtin_amdgcn_s_waitcnt((N & 15u) | ((N >> 4) << 14) | 0x0F70u);
}

template <uint32_t... I>
__device__ __forceinline__ void wait_vm_dispatch(uint32_t n, std::integer_sequence<uint32_t, I...>) {
    (void)((n == I ? (wait_vm_imm<I>(), true) : false) || ...);
}

// vmcnt(n) for a wave-uniform run-time n (clamped to the 6-bit counter).
__device__ __forceinline__ void wait_vm(uint32_t n) {
    wait_vm_dispatch(n > 63 ? 63 : n, std::make_integer_sequence<uint32_t, 64>{});
}

// LDS reads of pipeline stages are issued as inline asm so the compiler does
// not pair them with the asynchronous copies (its waitcnt insertion would
// otherwise drain every copy in flight before each read).  Their results are
// used only after lds_drain() (or a waitcnt asm that takes them as operands)
// and an empty asm that launders them.
typedef __attribute__((address_space(3))) const uint8_t lds_u8;

__device__ __forceinline__ v4i lds_read16(const uint8_t* p) {
    v4i r;
    uint32_t a = (uint32_t)(uintptr_t)(lds_u8*)p;
    asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(a));
    return r;
}

__device__ __forceinline__ uint32_t lds_read_u8(const uint8_t* p) {
    uint32_t r;
    uint32_t a = (uint32_t)(uintptr_t)(lds_u8*)p;
    asm volatile("ds_read_u8 %0, %1" : "=v"(r) : "v"(a));
    return r;
}

__device__ __forceinline__ uint32_t lds_read_b32(const uint8_t* p) {
    uint32_t r;
    uint32_t a = (uint32_t)(uintptr_t)(lds_u8*)p;
    asm volatile("ds_read_b32 %0, %1" : "=v"(r) : "v"(a));
    return r;
}

__device__ __forceinline__ void lds_write16(uint8_t* p, v4f v) {
    uint32_t a = (uint32_t)(uintptr_t)(lds_u8*)p;
    asm volatile("ds_write_b128 %0, %1" : : "v"(a), "v"(v) : "memory");
}

__device__ __forceinline__ uint32_t lds_read_u16(const uint8_t* p) {
    uint32_t r;
    uint32_t a = (uint32_t)(uintptr_t)(lds_u8*)p;
    asm volatile("ds_read_u16 %0, %1" : "=v"(r) : "v"(a));
    return r;
}

// Global loads the compiler's wait insertion does not see: the caller waits
// for them with wait_vm and passes the result through an empty asm before
// any use.
__device__ __forceinline__ v4i gload16_untracked(const void* p) {
    v4i v;
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(p));
    return v;
}

// Nontemporal global loads the compiler tracks (it waits for them itself);
// the explicit global address space keeps them off the FLAT path, whose
// loads also count against the LDS counter.
typedef __attribute__((address_space(1))) const v4i global_v4i;
typedef __attribute__((address_space(1))) const uint32_t global_u32;
__device__ __forceinline__ v4i gload16_nt(const void* p) {
    return __builtin_nontemporal_load(reinterpret_cast<global_v4i*>(reinterpret_cast<uintptr_t>(p)));
}
__device__ __forceinline__ uint32_t gload4_nt(const void* p) {
    return __builtin_nontemporal_load(reinterpret_cast<global_u32*>(reinterpret_cast<uintptr_t>(p)));
}

// Nontemporal forms (streamed once: whole-line reads at ~7 TB/s over the chip).
__device__ __forceinline__ v4i gload16_nt_untracked(const void* p) {
    v4i v;
    asm volatile("global_load_dwordx4 %0, %1, off nt" : "=v"(v) : "v"(p));
    return v;
}

__device__ __forceinline__ uint32_t gload4_nt_untracked(const void* p) {
    uint32_t v;
    asm volatile("global_load_dword %0, %1, off nt" : "=v"(v) : "v"(p));
    return v;
}

__device__ __forceinline__ uint32_t gload4_untracked(const void* p) {
    uint32_t v;
    asm volatile("global_load_dword %0, %1, off" : "=v"(v) : "v"(p));
    return v;
}

__device__ __forceinline__ void lds_drain() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// max(v, v of lane ^ 16) and max(v, v of lane ^ 32) with the gfx950 row swaps
// (VALU only: an LDS-routed shuffle would queue behind the LDS copies in
// flight).  With both operands v, the swap returns rows (0, 0, 2, 2) and
// (1, 1, 3, 3), resp. halves (lo, lo) and (hi, hi).  For the non-negative,
// NaN-free block maxima reduced here the order of the max is immaterial.
__device__ __forceinline__ float max_xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float max_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// LDS reads at a fixed register plus an immediate offset (< 64 KiB).
template <uint32_t OFF>
__device__ __forceinline__ v4i lds_rd128(uint32_t a) {
    v4i r;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(a), "i"(OFF));
    return r;
}
template <uint32_t OFF>
__device__ __forceinline__ uint32_t lds_rd32(uint32_t a) {
    uint32_t r;
    asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(r) : "v"(a), "i"(OFF));
    return r;
}

template <typename F, uint32_t... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<uint32_t, I...>) {
    (f(std::integral_constant<uint32_t, I>{}), ...);
}
// f(integral_constant<0>), ..., f(integral_constant<N-1>).
template <uint32_t N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<uint32_t, N>{});
}

__device__ __forceinline__ uint32_t lds_addr(const uint8_t* p) { return (uint32_t)(uintptr_t)(lds_u8*)p; }

}  // namespace
