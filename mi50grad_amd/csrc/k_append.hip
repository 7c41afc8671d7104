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
// position, sequence, slot and page id are workgroup-uniform scalar loads,
// and the norm weights and cos/sin rows go out with the row's own load.
__global__ __launch_bounds__(256) void append_kernel(AppendArgs a) {
    const int rows_per_tok = a.num_heads + 2 * a.num_kv_heads;
    const int blocks_per_tok = (rows_per_tok + 7) / 8;
    const int t = blockIdx.x / blocks_per_tok;
    const int hr = (blockIdx.x - t * blocks_per_tok) * 8 + (threadIdx.x >> 5);
    const int lane = threadIdx.x & 31;
    if (hr >= rows_per_tok) return;  // whole 32-lane group leaves
    const int hkv = a.num_kv_heads;
    const int pos = ld_uniform(a.tok_pos + t);
    const uint16_t *cos_row = a.cos_tab + static_cast<size_t>(pos) * a.half_rot;
    const uint16_t *sin_row = a.sin_tab + static_cast<size_t>(pos) * a.half_rot;

    if (hr < a.num_heads) {
        uint16_t *x = a.q + (static_cast<size_t>(t) * a.num_heads + hr) * kHeadDim;
        const uint4 xin = ld16(x + 8 * lane);
        const NormRopeIn nin = norm_rope_in<32>(a.q_w, cos_row, sin_row, a.half_rot, lane);
        st16(x + 8 * lane, norm_rope_apply<32>(xin, nin, a.half_rot, a.eps, lane));
        return;
    }
    const int seq = ld_uniform(a.tok_seq + t);
    const int slot = ld_uniform(a.tok_slot + t);
    const int blk = ld_uniform(a.table + static_cast<size_t>(seq) * a.table_stride + (slot >> 4));
    const size_t row_base = (static_cast<size_t>(blk) * kBlockTokens + (slot & 15)) * hkv;
    if (hr < a.num_heads + hkv) {
        const int kh = hr - a.num_heads;
        uint16_t *x = a.k + (static_cast<size_t>(t) * hkv + kh) * kHeadDim;
        const uint4 xin = ld16(x + 8 * lane);
        const NormRopeIn nin = norm_rope_in<32>(a.k_w, cos_row, sin_row, a.half_rot, lane);
        const uint4 y = norm_rope_apply<32>(xin, nin, a.half_rot, a.eps, lane);
        if (!a.keep_k) st16(x + 8 * lane, y);
        st16(a.k_pool + (row_base + kh) * kHeadDim + 8 * lane, y);
    } else {
        const int vh = hr - a.num_heads - hkv;
        const uint16_t *x = a.v + (static_cast<size_t>(t) * hkv + vh) * kHeadDim;
        st16(a.v_pool + (row_base + vh) * kHeadDim + 8 * lane, ld16(x + 8 * lane));
    }
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
