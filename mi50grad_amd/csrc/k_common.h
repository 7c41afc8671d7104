// Device helpers shared by the gfx950 kernels of libkvattn.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstdint>

namespace kva {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float h2f(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}
// Round-to-nearest-even fp32 -> fp16 (v_cvt_f16_f32 in the default mode).
__device__ __forceinline__ uint16_t f2h(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}
__device__ __forceinline__ float lo_f(uint32_t w) { return h2f(static_cast<uint16_t>(w & 0xffffu)); }
__device__ __forceinline__ float hi_f(uint32_t w) { return h2f(static_cast<uint16_t>(w >> 16)); }
__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
    return static_cast<uint32_t>(f2h(lo)) | (static_cast<uint32_t>(f2h(hi)) << 16);
}
// The same rounding in one v_cvt_pk_f16_f32 (gfx950), for softmax
// probabilities.  Outputs keep pack_h2: built with the vector form there,
// the gated prefill's outputs measured up to 2 ulps from the gate applied
// to the ungated outputs (1 with pack_h2), the compiled epilogues no longer
// rounding alike.
__device__ __forceinline__ uint32_t pack_p2(float lo, float hi) {
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    const f16x2_t v = {static_cast<_Float16>(lo), static_cast<_Float16>(hi)};
    return __builtin_bit_cast(uint32_t, v);
}

// v_dot2_f32_f16: acc + a.lo*b.lo + a.hi*b.hi, fp16 pairs packed in dwords.
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a), __builtin_bit_cast(half2_t, b),
                                  acc, false);
}

// DPP lane moves (row = 16 lanes).  The controls are the GCN DPP encodings.
enum : int {
    kDppQuadXor1 = 0xB1,       // quad_perm [1,0,3,2]
    kDppQuadXor2 = 0x4E,       // quad_perm [2,3,0,1]
    kDppRowHalfMirror = 0x141, // lane i <-> 7-i inside each 8 lanes
    kDppRowRor8 = 0x128,       // rotate a 16-lane row by 8
    kDppRowMirror = 0x140,     // lane i <-> 15-i inside each row
    kDppRowBcast15 = 0x142,    // lane 15 of a row -> all lanes of the next row
    kDppRowBcast31 = 0x143,    // lane 31 -> all lanes of rows 2 and 3
};
template <int Ctrl>
__device__ __forceinline__ float dpp_f(float x) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), Ctrl, 0xF, 0xF, false));
}
// DPP move restricted to the rows in RowMask; other rows keep x.
template <int Ctrl, int RowMask>
__device__ __forceinline__ float dpp_masked_f(float x) {
    const int xi = __builtin_bit_cast(int, x);
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(xi, xi, Ctrl, RowMask, 0xF, false));
}

// Sum over the 8 lanes of an aligned 8-lane group; every lane gets the sum.
__device__ __forceinline__ float group8_sum(float x) {
    x += dpp_f<kDppQuadXor1>(x);
    x += dpp_f<kDppQuadXor2>(x);
    x += dpp_f<kDppRowHalfMirror>(x);
    return x;
}

// Max / sum over the eight 8-lane groups of a wave (lanes of one group hold
// the same value on entry); every lane gets the result.
__device__ __forceinline__ float wave_groups_max(float x) {
    x = fmaxf(x, dpp_f<kDppRowRor8>(x));
    x = fmaxf(x, __shfl_xor(x, 16));
    x = fmaxf(x, __shfl_xor(x, 32));
    return x;
}
__device__ __forceinline__ float wave_groups_sum(float x) {
    x += dpp_f<kDppRowRor8>(x);
    x += __shfl_xor(x, 16);
    x += __shfl_xor(x, 32);
    return x;
}

// Wave-uniform read of read-only metadata (block-table entries, plans)
// through the scalar cache: a load in the constant address space with a
// uniform address becomes a scalar load, counted apart from the vector
// loads, so waiting for it does not also wait for K/V data in flight.
// floor(a * b / d) for 0 <= a, b and d > 0 (a stream-K share boundary): in
// 32 bits when the product fits, as it does for any realistic step (a 64-bit
// division is several times the instructions, and the combine kernels wait
// on these before their first loads); exact either way.
__device__ __forceinline__ int floor_muldiv(int a, int b, int d) {
    const uint64_t x = static_cast<uint64_t>(a) * static_cast<uint32_t>(b);
    return static_cast<int>(x <= 0xffffffffull ? static_cast<uint32_t>(x) / static_cast<uint32_t>(d)
                                               : x / static_cast<uint32_t>(d));
}

__device__ __forceinline__ int32_t ld_uniform(const int32_t *p) {
    return *reinterpret_cast<const __attribute__((address_space(4))) int32_t *>(
        reinterpret_cast<uintptr_t>(p));
}


typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) short4_t lds_short4_t;

// LDS byte address of a __shared__ location.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const lds_void_t *)p));
}

// One 16-byte-per-lane buffer load written straight to LDS: lane l's bytes
// go to lds + 16*l.  Written as inline assembly on purpose: the compiler
// would otherwise order every later LDS read of the kernel behind all such
// loads in flight (it cannot tell a ring's stages apart), which would drain
// the ring at every step.  Kernels do their own waiting (wait_vm + a
// barrier); to the compiler these loads are invisible, so its own load
// waits can only grow stricter, never too weak.
__device__ __forceinline__ void load_to_lds(__amdgpu_buffer_rsrc_t r, uint32_t lds, uint32_t voff) {
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %1, %2, 0 offen lds"
        :
        : "s"(lds), "v"(voff), "s"(r)
        : "memory", "m0");
}

// Wait until at most N of this wave's vector-memory operations are
// outstanding (they complete in order).
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt is six bits");
    // s_waitcnt fields: vmcnt[3:0], expcnt[6:4] (7 = no wait), lgkmcnt[11:8]
    // (15 = no wait), vmcnt[5:4] in bits [15:14].
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// The XCD (accelerator complex die) this wave runs on: CUs of one XCD
// share its L2.
__device__ __forceinline__ uint32_t xcc_id() {
    uint32_t x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
    return x & 0xfu;
}

// Read-only buffer resource over [base, base + bytes); bytes = 0 makes every
// access out of range (loads fetch nothing, and still count).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t ro_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, bytes, 0x00020000);
}

// Max / sum over the four 16-lane groups (every lane gets it): permlane
// swaps, VALU only (no LDS round trip).  v_permlane16_swap with both
// operands holding x leaves x of rows 0,0,2,2 in the first and of rows
// 1,1,3,3 in the second register; v_permlane32_swap likewise pairs the
// halves, so combining the two registers after each covers all four.
// Inline assembly: with one value in both operands the compiler's builtin
// has been seen to read the first result twice.
__device__ __forceinline__ void swap16(float &a, float &b) {
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap32(float &a, float &b) {
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ float group4_max(float x) {
    float a = x, b = x;
    swap16(a, b);
    a = fmaxf(a, b);
    b = a;
    swap32(a, b);
    return fmaxf(a, b);
}
__device__ __forceinline__ float group4_sum(float x) {
    float a = x, b = x;
    swap16(a, b);
    a += b;
    b = a;
    swap32(a, b);
    return a + b;
}

// Four attention output dims o0..o3 as fp16, through the optional output
// gate: the attention value is rounded to fp16 first and then multiplied by
// 1/(1+exp(-g)) in float32 (sigmoid_mul.hip:10-22 applied to the attention
// output, engine.py:2055-2056 after decode and :3120-3121 after prefill), so
// the fused result equals the reference's two launches.  g4: the four gate
// values (8-byte aligned) or null.
__device__ __forceinline__ uint2 out_fp16x4(float o0, float o1, float o2, float o3, const uint16_t *g4) {
    uint2 o;
    o.x = pack_h2(o0, o1);
    o.y = pack_h2(o2, o3);
    if (!g4) return o;
    const uint2 gw = *reinterpret_cast<const uint2 *>(g4);
    const float g[4] = {lo_f(gw.x), hi_f(gw.x), lo_f(gw.y), hi_f(gw.y)};
    const float a[4] = {lo_f(o.x), hi_f(o.x), lo_f(o.y), hi_f(o.y)};
    float r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = a[i] * (1.0f / (1.0f + expf(-g[i])));
    o.x = pack_h2(r[0], r[1]);
    o.y = pack_h2(r[2], r[3]);
    return o;
}

__device__ __forceinline__ uint4 ld16(const uint16_t *p) {
    return *reinterpret_cast<const uint4 *>(p);
}
__device__ __forceinline__ uint2 ld8(const uint16_t *p) {
    return *reinterpret_cast<const uint2 *>(p);
}
__device__ __forceinline__ void st16(uint16_t *p, uint4 v) {
    *reinterpret_cast<uint4 *>(p) = v;
}

}  // namespace kva
