// Fused per-head RMSNorm + interleaved partial RoPE + K/V append (gfx950).
//
// Math: norm_rope_row (k_normrope.h), the reference's qknorm_rope.hip:55-162
// and qknorm_rope_cachew.hip:52-142 under a fixed, bit-exact operation order.
//
// Layout: 32 lanes own one 256-dim row, 8 dims (16 bytes) per lane, so every
// load and store of a row is one coalesced 512-byte access of 16-byte lanes.
#include "k_common.h"
#include "k_normrope.h"
#include "kva_internal.h"

namespace kva {
namespace {

// One 32-lane group per row; rows of a token: H query heads, Hkv key heads,
// Hkv value heads.  8 rows per 256-thread workgroup, all of one token (the
// launch packs each token's rows into whole workgroups), so the token's
// position, sequence, slot and page id are workgroup-uniform scalar loads.
// Two memory round trips before the stores: first the token's position,
// sequence and slot with the group's row and norm weights; then cos/sin
// (at the position) and, in a workgroup holding key or value rows, the page
// id (at the sequence and slot).  Requested in source order the row waited
// for the position, and a key or value row's page id for the sequence and
// slot requested after it: four round trips before a cache store.
__global__ __launch_bounds__(256) void append_kernel(AppendArgs a) {
    const int nh = a.num_heads, hkv = a.num_kv_heads;
    const int rows_per_tok = nh + 2 * hkv;
    const int blocks_per_tok = (rows_per_tok + 7) / 8;
    const int t = blockIdx.x / blocks_per_tok;
    const int r0 = (blockIdx.x - t * blocks_per_tok) * 8;
    const int hr = r0 + (threadIdx.x >> 5);
    const int lane = threadIdx.x & 31;
    if (hr >= rows_per_tok) return;  // whole 32-lane group leaves
    const bool is_q = hr < nh, is_k = !is_q && hr < nh + hkv;
    uint16_t *const x = is_q   ? a.q + (static_cast<size_t>(t) * nh + hr) * kHeadDim
                        : is_k ? a.k + (static_cast<size_t>(t) * hkv + hr - nh) * kHeadDim
                               : const_cast<uint16_t *>(a.v) + (static_cast<size_t>(t) * hkv + hr - nh - hkv) * kHeadDim;
    const uint4 xin = ld16(x + 8 * lane);
    NormRopeIn nin;
    nin.w = ld16((is_q ? a.q_w : a.k_w) + 8 * lane);  // unused by a value row
    const int stride = a.table_stride, keep_k = a.keep_k;
    const int pos = ld_uniform(a.tok_pos + t);
    const int seq = ld_uniform(a.tok_seq + t);
    const int slot = ld_uniform(a.tok_slot + t);
    asm volatile("" ::"s"(pos), "s"(seq), "s"(slot), "s"(stride), "s"(keep_k));  // taken in together
    __builtin_amdgcn_sched_barrier(0);
    // Second round: cos/sin (branch-free, so nothing waits for them before
    // the page id goes out; a value row's are unused) and the page id.
    rope_in_flat(nin, a.k_w, a.cos_tab + static_cast<size_t>(pos) * a.half_rot,
                 a.sin_tab + static_cast<size_t>(pos) * a.half_rot, a.half_rot, lane);
    const bool any_kv = r0 + 7 >= nh;  // workgroup-uniform
    const int blk = any_kv ? ld_uniform(a.table + static_cast<size_t>(seq) * stride + (slot >> 4)) : 0;
    if (!is_q && !is_k) {
        const size_t row_base = (static_cast<size_t>(blk) * kBlockTokens + (slot & 15)) * hkv;
        st16(a.v_pool + (row_base + hr - nh - hkv) * kHeadDim + 8 * lane, xin);
        return;
    }
    const uint4 y = norm_rope_apply<32>(xin, nin, a.half_rot, a.eps, lane);
    if (is_q) {
        st16(x + 8 * lane, y);
        return;
    }
    const size_t row_base = (static_cast<size_t>(blk) * kBlockTokens + (slot & 15)) * hkv;
    if (!keep_k) st16(x + 8 * lane, y);
    st16(a.k_pool + (row_base + hr - nh) * kHeadDim + 8 * lane, y);
}

template <int LANES>
__global__ __launch_bounds__(256) void legacy_norm_kernel(LegacyNormArgs a) {
    const int row = blockIdx.x * 8 + (threadIdx.x >> 5);
    const int lane = threadIdx.x & 31;
    if (row >= a.num_heads) return;
    uint16_t *x = a.x + static_cast<size_t>(row) * a.head_dim;
    const uint4 xin = (lane < LANES) ? ld16(x + 8 * lane) : make_uint4(0, 0, 0, 0);
    const uint4 y = norm_rope_row<LANES>(xin, a.w, a.cos_row, a.sin_row, a.half_rot, a.eps, lane);
    if (lane < LANES) {
        st16(x + 8 * lane, y);
        if (a.cache_dst) st16(a.cache_dst + static_cast<size_t>(row) * a.head_dim + 8 * lane, y);
    }
}

}  // namespace

hipError_t launch_append(const AppendArgs &a, hipStream_t s) {
    if (a.n_tok <= 0) return hipSuccess;
    const int blocks_per_tok = (a.num_heads + 2 * a.num_kv_heads + 7) / 8;
    hipLaunchKernelGGL(append_kernel, dim3(a.n_tok * blocks_per_tok), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_legacy_norm(const LegacyNormArgs &a, hipStream_t s) {
    if (a.num_heads <= 0) return hipSuccess;
    const dim3 grid((a.num_heads + 7) / 8);
    switch (a.head_dim) {
        case 64: hipLaunchKernelGGL(legacy_norm_kernel<8>, grid, dim3(256), 0, s, a); break;
        case 128: hipLaunchKernelGGL(legacy_norm_kernel<16>, grid, dim3(256), 0, s, a); break;
        case 256: hipLaunchKernelGGL(legacy_norm_kernel<32>, grid, dim3(256), 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace kva
