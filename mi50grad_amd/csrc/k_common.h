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
__device__ __forceinline__ int32_t ld_uniform(const int32_t *p) {
    return *reinterpret_cast<const __attribute__((address_space(4))) int32_t *>(
        reinterpret_cast<uintptr_t>(p));
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
