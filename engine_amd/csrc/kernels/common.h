// Shared device-side helpers for the gfx950 kernels of the hip backend.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lykuro_hip.h"

namespace lyk {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

__device__ __forceinline__ half2_t as_half2(uint32_t u) {
    return __builtin_bit_cast(half2_t, u);
}
__device__ __forceinline__ uint32_t as_u32(half2_t h) {
    return __builtin_bit_cast(uint32_t, h);
}

// v_dot2_f32_f16: c + a.x*b.x + a.y*b.y with fp32 accumulation.
__device__ __forceinline__ float dot2(half2_t a, half2_t b, float c) {
    return __builtin_amdgcn_fdot2(a, b, c, false);
}

__device__ __forceinline__ float h2f(uint16_t bits) {
    return (float)__builtin_bit_cast(half_t, bits);
}
__device__ __forceinline__ uint16_t f2h(float f) {
    return __builtin_bit_cast(uint16_t, (half_t)f);
}

// Wave-uniform value (kept in an SGPR).
__device__ __forceinline__ int uniform(int v) {
    return __builtin_amdgcn_readfirstlane(v);
}

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// CPU's RoPE rotation (qwen_model.cpp:49-52) with separately rounded
// products (no FMA), so equal inputs give equal bits.
__device__ __forceinline__ float rot_lo(float a, float b, float c, float s) {
#pragma clang fp contract(off)
    return a * c - b * s;
}
__device__ __forceinline__ float rot_hi(float a, float b, float c, float s) {
#pragma clang fp contract(off)
    return b * c + a * s;
}

// fp32 x as two fp16 parts, hi + lo == x to ~22 bits: an fp16 MFMA of an
// exact fp16 operand against both parts, accumulated in fp32, keeps the
// fp32 operand's precision.
__device__ __forceinline__ void split_f16(float x, uint16_t& hi, uint16_t& lo) {
    hi = f2h(x);
    lo = f2h(x - h2f(hi));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Lane pairs (l, l ^ 32) and (l, l ^ 16) combined through the gfx950
// permlane swaps: each lane receives both values of its pair in VGPRs, with
// no LDS round trip (a shuffle goes through ds_bpermute and waits for it).
// The combination is commutative, so both lanes of a pair get the same bits,
// the bits a shuffle exchange gives. Every lane of the wave must be active.
// Both swap operands start as v; the compiler folds the swap of one value
// with itself into two equal results (the hardware gives the two rows of
// each pair), so the copy and the results pass through empty asm it cannot
// see through.
template <bool Row32>
__device__ __forceinline__ void pair_of(float v, float& x, float& y) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    unsigned w;
    asm volatile("v_mov_b32 %0, %1" : "=v"(w) : "v"(u));
    const auto r = Row32 ? __builtin_amdgcn_permlane32_swap(u, w, false, false)
                         : __builtin_amdgcn_permlane16_swap(u, w, false, false);
    unsigned a = r[0], b = r[1];
    asm volatile("" : "+v"(a), "+v"(b));
    x = __builtin_bit_cast(float, a);
    y = __builtin_bit_cast(float, b);
}
__device__ __forceinline__ float pair32_sum(float v) {
    float x, y;
    pair_of<true>(v, x, y);
    return x + y;
}
__device__ __forceinline__ float pair16_sum(float v) {
    float x, y;
    pair_of<false>(v, x, y);
    return x + y;
}
__device__ __forceinline__ float pair32_max(float v) {
    float x, y;
    pair_of<true>(v, x, y);
    return fmaxf(x, y);
}
__device__ __forceinline__ float pair16_max(float v) {
    float x, y;
    pair_of<false>(v, x, y);
    return fmaxf(x, y);
}
// v + the value of the lane `CTRL` names within its 16-lane row (DPP).
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
// Sum over the wave without LDS: rotations by 8, 4, 2, 1 within each 16-lane
// row (after each, the lanes a rotation pairs hold equal bits), then the
// row pairs and halves through the permlane swaps. Every lane gets the same
// bits; the order is fixed. Every lane of the wave must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_max(float v) {
    return fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false)));
}
// Maximum over the wave without LDS (exact in any order), in every lane.
__device__ __forceinline__ float wave_top(float v) {
    v = dpp_max<0x128>(v);   // row_ror:8
    v = dpp_max<0x124>(v);   // row_ror:4
    v = dpp_max<0x122>(v);   // row_ror:2
    v = dpp_max<0x121>(v);   // row_ror:1
    return pair32_max(pair16_max(v));
}
__device__ __forceinline__ float wave_total(float v) {
    v = dpp_add<0x128>(v);   // row_ror:8
    v = dpp_add<0x124>(v);   // row_ror:4
    v = dpp_add<0x122>(v);   // row_ror:2
    v = dpp_add<0x121>(v);   // row_ror:1
    return pair32_sum(pair16_sum(v));
}

// Global-memory view of a generic pointer. Pointers that reach a kernel
// through a struct in device memory lose their address space; accesses
// through them would compile to flat instructions, which also count against
// the LDS wait counter and so serialize LDS reads behind outstanding global
// loads.
#define LYK_GLOBAL __attribute__((address_space(1)))
// LDS address space (the destination operand of LDS DMA).
#define LYK_LOCAL __attribute__((address_space(3)))
template <class T>
__device__ __forceinline__ LYK_GLOBAL T* gp(T* p) {
    return (LYK_GLOBAL T*)p;
}
template <class T>
__device__ __forceinline__ T ld(const T* p) {
    return *gp(p);
}
template <class T>
__device__ __forceinline__ void st(T* p, T v) {
    *gp(p) = v;
}

// Publishes this wave's earlier agent-scope (sc1) atomic stores before a
// following arrival counter update: s_waitcnt 0 returns only once those
// stores are performed at the device coherence point. (A workgroup-scope
// fence does not wait for them; an agent-scope fence would also write back
// the whole L2, which costs ~20 ns per workgroup.)
__device__ __forceinline__ void publish_sc1_stores() {
    __builtin_amdgcn_s_waitcnt(0);
}

// Arrival at a per-tile counter after publishing sc1 partial stores; true for
// the last of `expected` arrivals. Call with the whole wave; lane 0 counts.
__device__ __forceinline__ bool arrive_last(unsigned* counter, unsigned expected) {
    publish_sc1_stores();
    unsigned prev = 0;
    if ((threadIdx.x & 63) == 0)
        prev = __hip_atomic_fetch_add(gp(counter), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    prev = __shfl(prev, 0, 64);
    return prev == expected - 1;
}

template <class T>
__device__ __forceinline__ void store_sc1(T* p, T v) {
    __hip_atomic_store(gp(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
__device__ __forceinline__ T load_sc1(const T* p) {
    return __hip_atomic_load(gp(const_cast<T*>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

inline int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

}  // namespace lyk

#define LYK_LAUNCH_CHECK()                                   \
    do {                                                     \
        hipError_t e_ = hipGetLastError();                   \
        if (e_ != hipSuccess) return LYK_ERR_LAUNCH;         \
    } while (0)
