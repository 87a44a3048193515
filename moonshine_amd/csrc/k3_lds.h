/*
 * LDS staging helpers shared by the MFMA kernels (k3_mfma.hip, k3_router.hip):
 * direct-to-LDS loads, wait counters, LDS fragment reads as inline asm, and
 * the XOR swizzle of 128-byte rows staged eight per 1 KB chunk.
 */
#pragma once

#include "k3_device.h"

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

namespace k3 {

/* XOR swizzle of the 16-byte pieces of row r of A chunk half h. */
__device__ __forceinline__ uint32_t a_swizzle(uint32_t r, uint32_t h) {
    return (r >> 1) | (h << 2);
}
/* Byte offset, inside a chunk pair (t, i), of 16-byte piece p of row c. */
__device__ __forceinline__ uint32_t a_slot(uint32_t c, uint32_t p) {
    const uint32_t h = c >> 3, r = c & 7u;
    return 1024u * h + 128u * r + 16u * (p ^ a_swizzle(r, h));
}
/* Row (within the chunk pair) and source piece of lane L of chunk half h. */
__device__ __forceinline__ uint32_t a_dma_row(uint32_t L, uint32_t h) { return 8u * h + (L >> 3); }
__device__ __forceinline__ uint32_t a_dma_piece(uint32_t L, uint32_t h) {
    return (L & 7u) ^ a_swizzle(L >> 3, h);
}

typedef __attribute__((address_space(3))) void lds_void;

template <int Bytes, int Aux = 0>
__device__ __forceinline__ void dma(const uint8_t *src, uint8_t *lds) {
    if constexpr (Bytes == 16)
        __builtin_amdgcn_global_load_lds((const void *)src, (lds_void *)lds, 16, 0, Aux);
    else
        __builtin_amdgcn_global_load_lds((const void *)src, (lds_void *)lds, 4, 0, Aux);
}

/* s_waitcnt vmcnt(N) (N < 64), other counters untouched. */
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)p;
}

/*
 * LDS reads of staged fragments are issued as inline asm: the compiler's
 * wait insertion cannot tell which ring buffer an in-flight direct-to-LDS
 * load targets and would drain them all before every read. The reads are
 * completed by one explicit lgkmcnt(0) wait (mfma_step) and the results are
 * passed through empty volatile asm after it, so no use can move above it.
 */
template <int OFF>
__device__ __forceinline__ u32x4_t ds_read16(uint32_t addr) {
    u32x4_t v;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
    return v;
}
template <int OFF>
__device__ __forceinline__ uint32_t ds_read4(uint32_t addr) {
    uint32_t v;
    asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
    return v;
}
template <class T>
__device__ __forceinline__ void after_wait(T &v) {
    asm volatile("" : "+v"(v));
}

/* s_waitcnt lgkmcnt(N) (N < 16), other counters untouched. */
template <int N>
__device__ __forceinline__ void wait_lgkm() {
    static_assert(N >= 0 && N < 16, "lgkmcnt");
    __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (N << 8) | (3 << 14));
}

/* f(integral_constant<int, i>) for i = 0 .. N - 1, unrolled */
template <int... Is, class Fn>
__device__ __forceinline__ void static_for_impl(std::integer_sequence<int, Is...>, Fn &&f) {
    (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, class Fn>
__device__ __forceinline__ void static_for(Fn &&f) {
    static_for_impl(std::make_integer_sequence<int, N>{}, f);
}

}  // namespace k3
