// Small bookkeeping kernels: block-table patches and tree rollback moves.
#include "k_common.h"
#include "kva_internal.h"

#include <algorithm>

namespace kva {
namespace {

__global__ void table_patch_kernel(int32_t *table, int32_t stride, const int32_t *patches,
                                   int32_t n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int32_t seq = patches[3 * i];
    const int32_t idx = patches[3 * i + 1];
    table[static_cast<size_t>(seq) * stride + idx] = patches[3 * i + 2];
}

// grid (sequence group, layer, K|V).  The moves of one sequence run in order
// and each thread copies the same 16-byte columns of every row, so a row read
// by an earlier move is read before a later move overwrites it (accepted
// rows only move towards lower slots: dst = k <= keep[k] = src).
__global__ __launch_bounds__(256) void rollback_kernel(RollbackArgs a) {
    const int grp = blockIdx.x;
    const int layer = blockIdx.y;
    uint16_t *pool = (blockIdx.z == 0 ? a.k_pools : a.v_pools) + a.layer_elems * layer;
    const size_t row_elems = static_cast<size_t>(a.num_kv_heads) * kHeadDim;
    for (int mv = a.move_off[grp]; mv < a.move_off[grp + 1]; ++mv) {
        const int32_t seq = a.moves[3 * mv];
        const int32_t src = a.moves[3 * mv + 1];
        const int32_t dst = a.moves[3 * mv + 2];
        const int32_t *trow = a.table + static_cast<size_t>(seq) * a.table_stride;
        const uint16_t *ps =
            pool + (static_cast<size_t>(trow[src >> 4]) * kBlockTokens + (src & 15)) * row_elems;
        uint16_t *pd =
            pool + (static_cast<size_t>(trow[dst >> 4]) * kBlockTokens + (dst & 15)) * row_elems;
        for (size_t e = 8 * threadIdx.x; e < row_elems; e += 8 * blockDim.x) st16(pd + e, ld16(ps + e));
    }
}

// Plain streaming copy: grid-stride over 4 x 16 bytes per lane, the four
// loads issued before the stores so each lane keeps 64 bytes in flight.
__global__ __launch_bounds__(256) void copy_kernel(uint4 *__restrict__ dst,
                                                   const uint4 *__restrict__ src, size_t n16) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const uint4 a = src[i], b = src[i + stride], c = src[i + 2 * stride], d = src[i + 3 * stride];
        dst[i] = a;
        dst[i + stride] = b;
        dst[i + 2 * stride] = c;
        dst[i + 3 * stride] = d;
    }
    for (; i < n16; i += stride) dst[i] = src[i];
}

// Read-only stream: workgroup w reads the contiguous w-th share of the
// buffer, four 16-byte loads per lane per pass, the next pass's loads issued
// before the current one is folded by XOR (the fastest of the shapes
// measured: contiguous shares beat a grid-stride walk by about 8 %).  A lane
// writes its fold only if it equals `magic` (data-dependent, so the loads
// stay; zero-filled input never writes).
constexpr int kReadDepth = 4;

__device__ __forceinline__ uint32_t fold16(uint4 v) { return v.x ^ v.y ^ v.z ^ v.w; }

__global__ __launch_bounds__(256) void read_kernel(const uint4 *__restrict__ src, size_t n16, uint32_t *sink,
                                                   uint32_t magic) {
    const size_t lo = blockIdx.x * n16 / gridDim.x;
    const size_t per = (blockIdx.x + 1) * n16 / gridDim.x - lo;
    const uint4 *p = src + lo;
    const size_t step = static_cast<size_t>(kReadDepth) * blockDim.x;
    uint32_t acc = 0;
    size_t o = 0;
    if (per >= 2 * step) {
        uint4 a[kReadDepth], b[kReadDepth];
#pragma unroll
        for (int k = 0; k < kReadDepth; ++k) a[k] = p[k * blockDim.x + threadIdx.x];
        for (o = step; o + 2 * step <= per; o += 2 * step) {
#pragma unroll
            for (int k = 0; k < kReadDepth; ++k) b[k] = p[o + k * blockDim.x + threadIdx.x];
#pragma unroll
            for (int k = 0; k < kReadDepth; ++k) acc ^= fold16(a[k]);
#pragma unroll
            for (int k = 0; k < kReadDepth; ++k) a[k] = p[o + step + k * blockDim.x + threadIdx.x];
#pragma unroll
            for (int k = 0; k < kReadDepth; ++k) acc ^= fold16(b[k]);
        }
#pragma unroll
        for (int k = 0; k < kReadDepth; ++k) acc ^= fold16(a[k]);  // [o - step, o)
    }
    for (size_t i = o + threadIdx.x; i < per; i += blockDim.x) acc ^= fold16(p[i]);
    if (acc == magic) sink[0] = acc;
}

// Paged read probe: the stream-K decode's loads without its arithmetic.
// Workgroup w of gridDim.x takes the pages [w*P/W, (w+1)*P/W) of the list;
// wave h (one per kv head) reads head h's 512-byte slice of every row of
// each page exactly as decode_mfma_kernel does (K: lane l reads 128
// contiguous bytes of row l%16 at byte 128*(l/16); V: 8 bytes at 8*l of every
// row), one page in flight while the previous one is folded.  Page ids are
// scalar loads, as in the decode.
__device__ __forceinline__ void fold_page(uint32_t &acc, const uint4 (&k)[8], const uint2 (&v)[kBlockTokens]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) acc ^= fold16(k[i]);
#pragma unroll
    for (int t = 0; t < kBlockTokens; ++t) acc ^= v[t].x ^ v[t].y;
}

__global__ __launch_bounds__(256) void page_read_kernel(const uint8_t *k_pool, const uint8_t *v_pool,
                                                        const int32_t *page_ids, int32_t n_pages, int32_t row_bytes,
                                                        uint32_t *sink, uint32_t magic) {
    const int w = blockIdx.x, W = gridDim.x;
    const int p0 = static_cast<int>(static_cast<int64_t>(w) * n_pages / W);
    const int p1 = static_cast<int>(static_cast<int64_t>(w + 1) * n_pages / W);
    const int h = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const size_t page_bytes = static_cast<size_t>(kBlockTokens) * row_bytes;
    const uint32_t koff = (lane & 15) * row_bytes + 128 * (lane >> 4);
    const uint32_t voff = 8 * lane;
    auto load = [&](uint4 (&k)[8], uint2 (&v)[kBlockTokens], int p) {
        const bool on = p < p1;
        const int id = on ? ld_uniform(page_ids + p) : 0;
        const size_t ofs = static_cast<size_t>(id) * page_bytes + h * kHeadDim * 2;
        const auto rk = ro_rsrc(k_pool + ofs, on ? page_bytes : 0u);
        const auto rv = ro_rsrc(v_pool + ofs, on ? page_bytes : 0u);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const auto x = __builtin_amdgcn_raw_buffer_load_b128(rk, koff + 16 * i, 0, 0);
            k[i] = make_uint4(x[0], x[1], x[2], x[3]);
        }
#pragma unroll
        for (int t = 0; t < kBlockTokens; ++t) {
            const auto x = __builtin_amdgcn_raw_buffer_load_b64(rv, voff + t * row_bytes, 0, 0);
            v[t] = make_uint2(x[0], x[1]);
        }
    };
    uint32_t acc = 0;
    uint4 ka[8], kb[8];
    uint2 va[kBlockTokens], vb[kBlockTokens];
    int p = p0;
    load(ka, va, p);
    while (p < p1) {
        load(kb, vb, p + 1);
        fold_page(acc, ka, va);
        if (++p >= p1) break;
        load(ka, va, p + 1);
        fold_page(acc, kb, vb);
        ++p;
    }
    if (acc == magic) sink[0] = acc;
}

}  // namespace

hipError_t launch_read_pages(const void *k_pool, const void *v_pool, const int32_t *page_ids, int32_t n_pages,
                             int32_t num_kv_heads, int32_t n_wg, uint32_t *sink, hipStream_t s) {
    if (n_pages <= 0) return hipSuccess;
    hipLaunchKernelGGL(page_read_kernel, dim3(n_wg), dim3(64 * num_kv_heads), 0, s,
                       static_cast<const uint8_t *>(k_pool), static_cast<const uint8_t *>(v_pool), page_ids, n_pages,
                       num_kv_heads * kHeadDim * 2, sink, 0x9e3779b9u);
    return hipGetLastError();
}

hipError_t launch_read(const void *src, size_t bytes, uint32_t *sink, hipStream_t s) {
    const size_t n16 = bytes / 16;
    if (n16 == 0) return hipSuccess;
    // 2048 shares of at least two passes each (fewer for small buffers).
    const size_t blocks = std::max<size_t>(1, std::min<size_t>(n16 / (2 * kReadDepth * 256), 2048));
    hipLaunchKernelGGL(read_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s,
                       static_cast<const uint4 *>(src), n16, sink, 0x9e3779b9u);
    return hipGetLastError();
}

hipError_t launch_copy(void *dst, const void *src, size_t bytes, hipStream_t s) {
    const size_t n16 = bytes / 16;
    if (n16 == 0) return hipSuccess;
    const size_t blocks = std::min<size_t>((n16 + 255) / 256, 256 * 32);
    hipLaunchKernelGGL(copy_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s,
                       static_cast<uint4 *>(dst), static_cast<const uint4 *>(src), n16);
    return hipGetLastError();
}

hipError_t launch_table_patch(int32_t *table, int32_t stride, const int32_t *patches,
                              int32_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(table_patch_kernel, dim3((n + 255) / 256), dim3(256), 0, s, table, stride,
                       patches, n);
    return hipGetLastError();
}

hipError_t launch_rollback(const RollbackArgs &a, hipStream_t s) {
    if (a.n_groups <= 0) return hipSuccess;
    hipLaunchKernelGGL(rollback_kernel, dim3(a.n_groups, a.n_layers, 2), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace kva
