// Per-head RMSNorm + interleaved partial RoPE of one 256-dim (or 128/64)
// row, shared by the append kernel and the projection epilogue so both
// produce the same bits.
//
// Math: qknorm_rope.hip:55-162 and qknorm_rope_cachew.hip:52-142 of the
// reference (RMSNorm with the stored weight, rotation of pairs (2i, 2i+1) for
// i < half_rotary, tail dims normalised only).  The operation order is the
// bit-exact contract mirrored by the CPU oracle: no FMA contraction,
// sequential 8-term lane sums, an xor butterfly across lanes, correctly
// rounded sqrt and divide, round-to-nearest-even fp16 stores.
#pragma once

#include "k_common.h"

namespace kva {

// The operands a row's norm + RoPE reads besides the row itself: this
// lane's 8 norm weights and its 4 cos/sin pairs.  Loaded apart from the
// math so a kernel can request them before it waits for the row.
struct NormRopeIn {
    uint4 w;
    uint2 c, s;
};

// The cos/sin half of norm_rope_in, for a caller that requests the weights
// earlier.
__device__ __forceinline__ void rope_in(NormRopeIn &in, const uint16_t *__restrict__ cos_row,
                                        const uint16_t *__restrict__ sin_row, int half_rot, int lane) {
    if (half_rot > 0) {
        const int cl = min(lane, half_rot / 4 - 1);
        in.c = ld8(cos_row + 4 * cl);
        in.s = ld8(sin_row + 4 * cl);
    } else {
        in.c = make_uint2(0, 0);
        in.s = make_uint2(0, 0);
    }
}

// Lanes past LANES get zero weights; lanes past the rotary pairs read the
// last lane's cos/sin (in bounds, never used).  half_rot % 4 == 0.
template <int LANES>
__device__ __forceinline__ NormRopeIn norm_rope_in(const uint16_t *__restrict__ w,
                                                   const uint16_t *__restrict__ cos_row,
                                                   const uint16_t *__restrict__ sin_row, int half_rot,
                                                   int lane) {
    NormRopeIn in;
    in.w = (lane < LANES) ? ld16(w + 8 * lane) : make_uint4(0, 0, 0, 0);
    rope_in(in, cos_row, sin_row, half_rot, lane);
    return in;
}

// rope_in without its branch, for a caller that must not wait for cos/sin
// before its next requests (a merge of loaded values after the branch makes
// the compiler wait for them there).  With no rotary part the loads read the
// weight row w instead (in bounds; norm_rope_apply uses c and s only on
// lanes that hold rotary pairs).
__device__ __forceinline__ void rope_in_flat(NormRopeIn &in, const uint16_t *__restrict__ w,
                                             const uint16_t *__restrict__ cos_row,
                                             const uint16_t *__restrict__ sin_row, int half_rot, int lane) {
    const bool rot = half_rot > 0;
    const int cl = rot ? min(lane, half_rot / 4 - 1) : 0;
    in.c = ld8((rot ? cos_row : w) + 4 * cl);
    in.s = ld8((rot ? sin_row : w) + 4 * cl);
}

// Normalise + rotate one row held as 8 fp16 per lane.  LANES = head_dim / 8
// lanes take part (lane < LANES); the butterfly stays inside them.
template <int LANES>
__device__ __forceinline__ uint4 norm_rope_apply(uint4 xin, const NormRopeIn &in, int half_rot, float eps,
                                                 int lane) {
#pragma clang fp contract(off)
    const uint32_t xw[4] = {xin.x, xin.y, xin.z, xin.w};
    float x[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        x[2 * i] = lo_f(xw[i]);
        x[2 * i + 1] = hi_f(xw[i]);
    }
    float s = x[0] * x[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) {
        const float sq = x[i] * x[i];
        s = s + sq;
    }
#pragma unroll
    for (int off = LANES / 2; off >= 1; off >>= 1) {
        const float other = __shfl_xor(s, off, 32);
        s = s + other;
    }
    const float ms = s * (1.0f / static_cast<float>(LANES * 8));
    const float var = ms + eps;
    const float inv = 1.0f / sqrtf(var);

    const uint32_t ww[4] = {in.w.x, in.w.y, in.w.z, in.w.w};
    float n[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float t0 = x[2 * i] * inv;
        const float t1 = x[2 * i + 1] * inv;
        n[2 * i] = t0 * lo_f(ww[i]);
        n[2 * i + 1] = t1 * hi_f(ww[i]);
    }
    if (8 * lane < 2 * half_rot) {
        // This lane holds pairs 4*lane .. 4*lane+3.
        const float c[4] = {lo_f(in.c.x), hi_f(in.c.x), lo_f(in.c.y), hi_f(in.c.y)};
        const float sn[4] = {lo_f(in.s.x), hi_f(in.s.x), lo_f(in.s.y), hi_f(in.s.y)};
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const float a = n[2 * p];
            const float b = n[2 * p + 1];
            const float ac = a * c[p];
            const float bs = b * sn[p];
            const float as = a * sn[p];
            const float bc = b * c[p];
            n[2 * p] = ac - bs;
            n[2 * p + 1] = as + bc;
        }
    }
    uint4 y;
    y.x = pack_h2(n[0], n[1]);
    y.y = pack_h2(n[2], n[3]);
    y.z = pack_h2(n[4], n[5]);
    y.w = pack_h2(n[6], n[7]);
    return y;
}

template <int LANES>
__device__ __forceinline__ uint4 norm_rope_row(uint4 xin, const uint16_t *__restrict__ w,
                                               const uint16_t *__restrict__ cos_row,
                                               const uint16_t *__restrict__ sin_row,
                                               int half_rot, float eps, int lane) {
    return norm_rope_apply<LANES>(xin, norm_rope_in<LANES>(w, cos_row, sin_row, half_rot, lane), half_rot, eps,
                                  lane);
}

}  // namespace kva
