// Multi-query attention over the paged cache with FP16 MFMA (gfx950):
// chunked causal prefill and tree verify.
//
// Semantics: softmax(q K^T / 16) V per query token and head, kv head =
// h*Hkv/H, where new token i of a sequence (slot s_i = len_before + i) sees
//   causal (prefill): keys [0, s_i]  — the reference's rule with the chunk
//       starting after an existing cache (flash_attn_256.hip:78,
//       flash_attn_256_v3.hip:252-255 assume a chunk at position 0);
//   tree:  keys [0, len_before) and the new tokens in its tree bit set
//       (flash_attn_tree.hip:72-175 under tree_attention.py:186-208).
//
// Unit = (sequence, tile of 16 new tokens, kv head); a 64*G-thread workgroup
// runs one wave per query head of the GQA group, so every K/V block staged
// in LDS serves G heads.  Work is split stream-K over 32-key blocks: the
// blocks of all units are laid end to end and each workgroup takes an equal
// share; units cut by a share boundary leave partials for mq_combine_kernel.
//
// Per 32-key block and wave (v_mfma_f32_16x16x32_f16, C layout: lane l holds
// rows 4*(l/16)+i, column l%16):
//   S^T[key][q] = K[key][:] . Q[q][:]   (A = K rows from LDS, B = Q^T held
//       in registers for the whole unit; 2 key tiles x 8 k-steps);
//   per query column: scale, mask, online softmax (max over the 4 lane
//       groups with two shuffles), P^T in fp16 — already the B operand of
//   O^T[dim][q] += V^T[dim][key] . P^T[key][q]   (A = V^T from LDS, stored
//       transposed when staged; 16 dim tiles).
// The k-index permutation of P^T (keys 4g..4g+3 and 16+4g..16+4g+3 in lane
// group g) is matched by the V^T reads, so the sum is over the right pairs.
#include "k_common.h"
#include "kva_internal.h"

namespace kva {
namespace {

constexpr int kKRow = kHeadDim + 8;  // K tile row stride (halves): 528 B, conflict-free b128 reads
constexpr int kVRow = kMqKeys + 8;   // V^T tile row stride (halves): 80 B
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ int mq_wg_start(int w, int n, int W) {
    return static_cast<int>(static_cast<int64_t>(w) * n / W);
}
__device__ __forceinline__ int mq_wg_of(int p, int n, int W) {
    int w = static_cast<int>(static_cast<int64_t>(p) * W / n);
    while (w + 1 < W && mq_wg_start(w + 1, n, W) <= p) ++w;
    return w;
}
// Largest i in [0, n) with pre[i] <= x (pre non-decreasing, pre[0] <= x).
__device__ __forceinline__ int upper_index(const int32_t *pre, int n, int x) {
    int lo = 0, hi = n - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (pre[mid] <= x) lo = mid; else hi = mid - 1;
    }
    return lo;
}

// Staged 32-key block.  K: 1024 chunks of 16 bytes (key = c/32, dims
// 8*(c%32)..+8) spread over the threads.  V: 256 tasks of 4 keys x 8 dims
// (keys 4*(v/32).., dims 8*(v%32)..), transposed in registers so each dim's
// 4 keys are stored to V^T with one 8-byte write.
template <int NT>
struct Stage {
    static constexpr int kPerK = (kMqKeys * 32 + NT - 1) / NT;
    static constexpr int kPerV = (kMqKeys / 4 * 32 + NT - 1) / NT;
    uint4 k[kPerK];
    uint4 v[kPerV][4];
};

// Page ids of a block's two 16-key pages (wave-uniform scalars).
struct BlockPages {
    int p0, p1;
};

// Scalar loads: waiting for a page id then never drains the K/V loads in
// flight (a vector load + readfirstlane would wait for every older load).
__device__ __forceinline__ BlockPages block_pages(const int32_t *trow, int blk, int ctx) {
    const int pg = 2 * blk;
    BlockPages bp;
    bp.p0 = ld_uniform(trow + pg);
    bp.p1 = (pg + 1) * kBlockTokens < ctx ? ld_uniform(trow + pg + 1) : bp.p0;
    return bp;
}

// Every lane issues every load of a stage (a key past the sequence, or a
// chunk beyond the block, reads the block's first key and is zeroed after):
// with the same loads on every path the compiler's load counters stay exact,
// so waiting for one stage never drains the next one in flight.
__device__ __forceinline__ uint4 zero_unless(bool keep, uint4 x) {
    return keep ? x : make_uint4(0, 0, 0, 0);
}

template <int NT>
__device__ __forceinline__ void stage_load(Stage<NT> &st, const MultiQueryArgs &a, BlockPages bp,
                                           int h, int key0, int ctx) {
    const int tid = threadIdx.x;
    const size_t row_elems = static_cast<size_t>(a.num_kv_heads) * kHeadDim;
    const size_t head_off = static_cast<size_t>(h) * kHeadDim;
#pragma unroll
    for (int i = 0; i < Stage<NT>::kPerK; ++i) {
        const int c = tid + i * NT;
        const int kk = c >> 5;
        const bool ok = c < kMqKeys * 32 && key0 + kk < ctx;
        const int kr = ok ? kk : 0;
        const int page = kr < 16 ? bp.p0 : bp.p1;
        const size_t off = (static_cast<size_t>(page) * kBlockTokens + (kr & 15)) * row_elems + head_off +
                           (ok ? (c & 31) * 8 : 0);
        st.k[i] = zero_unless(ok, ld16(a.k_pool + off));
    }
#pragma unroll
    for (int i = 0; i < Stage<NT>::kPerV; ++i) {
        const int v = tid + i * NT;
        const bool vin = v < kMqKeys / 4 * 32;
        const int kg = vin ? v >> 5 : 0;
        const int col = vin ? (v & 31) * 8 : 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int kk = 4 * kg + e;
            const bool ok = vin && key0 + kk < ctx;
            const int kr = ok ? kk : 0;
            const int page = kr < 16 ? bp.p0 : bp.p1;
            st.v[i][e] = zero_unless(ok, ld16(a.v_pool + (static_cast<size_t>(page) * kBlockTokens + (kr & 15)) *
                                                             row_elems + head_off + col));
        }
    }
}

template <int NT>
__device__ __forceinline__ void stage_store(const Stage<NT> &st, uint16_t *k_lds, uint16_t *vt_lds) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < Stage<NT>::kPerK; ++i) {
        const int c = tid + i * NT;
        if (c < kMqKeys * 32)
            *reinterpret_cast<uint4 *>(k_lds + (c >> 5) * kKRow + (c & 31) * 8) = st.k[i];
    }
#pragma unroll
    for (int i = 0; i < Stage<NT>::kPerV; ++i) {
        const int v = tid + i * NT;
        if (v < kMqKeys / 4 * 32) {
            const int key = 4 * (v >> 5);
            const int col = (v & 31) * 8;
            // word w of key e holds dims col+2w, col+2w+1
            const uint32_t w0[4] = {st.v[i][0].x, st.v[i][0].y, st.v[i][0].z, st.v[i][0].w};
            const uint32_t w1[4] = {st.v[i][1].x, st.v[i][1].y, st.v[i][1].z, st.v[i][1].w};
            const uint32_t w2[4] = {st.v[i][2].x, st.v[i][2].y, st.v[i][2].z, st.v[i][2].w};
            const uint32_t w3[4] = {st.v[i][3].x, st.v[i][3].y, st.v[i][3].z, st.v[i][3].w};
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                uint2 lo, hi;  // dims col+2w (low halves) and col+2w+1 (high halves), keys key..key+3
                lo.x = (w0[w] & 0xffffu) | (w1[w] << 16);
                lo.y = (w2[w] & 0xffffu) | (w3[w] << 16);
                hi.x = (w0[w] >> 16) | (w1[w] & 0xffff0000u);
                hi.y = (w2[w] >> 16) | (w3[w] & 0xffff0000u);
                *reinterpret_cast<uint2 *>(vt_lds + (col + 2 * w) * kVRow + key) = lo;
                *reinterpret_cast<uint2 *>(vt_lds + (col + 2 * w + 1) * kVRow + key) = hi;
            }
        }
    }
}

__device__ __forceinline__ half8_t as_h8(uint4 v) { return __builtin_bit_cast(half8_t, v); }

template <int G>
__global__ __launch_bounds__(64 * G) void mq_kernel(MultiQueryArgs a) {
    constexpr int NT = 64 * G;
    const int w = blockIdx.x;
    const int W = a.n_wg;
    const int NB = a.total_blocks;
    const int q0 = mq_wg_start(w, NB, W);
    const int q1 = mq_wg_start(w + 1, NB, W);
    if (q0 >= q1) return;  // uniform over the workgroup
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // head within the group
    const int lane = threadIdx.x & 63;
    const int col = lane & 15;   // query row of the tile (C/B column)
    const int grp = lane >> 4;   // lane group: keys 4*grp.. of a 16-key tile
    const int hkv = a.num_kv_heads;
    const int nh = a.num_heads;
    const float scale = kLog2e / 16.0f;

    // Two LDS tiles: block blk+1 is stored into one while block blk is read
    // from the other, so one barrier per block separates them.
    __shared__ uint16_t k_lds2[2][kMqKeys * kKRow];
    __shared__ uint16_t vt_lds2[2][kHeadDim * kVRow];

    int u = upper_index(a.mq_pre, a.n_units, q0);
    int p = q0;
    bool first_seg = true;
    while (p < q1) {
        const int ub = a.mq_pre[u];
        const int ue = a.mq_pre[u + 1];
        if (p >= ue) {  // empty or finished unit
            ++u;
            continue;
        }
        const int b = upper_index(a.upre, a.n_seqs, u);
        const int x = u - a.upre[b];
        const int tile = x / hkv;
        const int h = x - tile * hkv;
        const int seg_end = min(ue, q1);
        const int tok_base = a.tok_off[b];
        const int T = a.tok_off[b + 1] - tok_base;
        const int ns = a.new_start[b];
        const int ctx = a.ctx_lens[b];
        const int32_t *trow = a.table + static_cast<size_t>(a.seq_ids[b]) * a.table_stride;

        // This lane's query row (token qi of the sequence's new tokens).
        const int qi = tile * kMqRows + col;
        const bool qvalid = qi < T;
        const int qslot = ns + qi;
        const uint64_t qbits = (a.tree && qvalid) ? a.tok_bits[tok_base + qi] : 0ull;
        uint4 qb[8];  // B operand Q^T: dims 32*kk + 8*grp .. +8 of query qi, head h*G+wave
        {
            const uint16_t *qr = a.q + (static_cast<size_t>(tok_base + (qvalid ? qi : 0)) * nh + h * G + wave) * kHeadDim;
#pragma unroll
            for (int kk = 0; kk < 8; ++kk)
                qb[kk] = qvalid ? ld16(qr + 32 * kk + 8 * grp) : make_uint4(0, 0, 0, 0);
        }

        float m = -INFINITY, l = 0.0f;
        float4_t acc[16];
#pragma unroll
        for (int dt = 0; dt < 16; ++dt) acc[dt] = float4_t{0.f, 0.f, 0.f, 0.f};

        // Pipeline: two register stages, so blocks blk+1 and blk+2's K/V loads
        // (64 KB per workgroup) are in flight while block blk is computed from
        // LDS; the stage just stored is refilled with block blk+2 at once.
        // Loads past the segment repeat its last block (same loads on every
        // path, no use).
        // (A 64-thread workgroup, G = 1, holds a whole block per thread: one
        // stage.)
        constexpr int kAhead = G >= 2 ? 2 : 1;
        Stage<NT> stg[kAhead];
        const int blk0 = p - ub;
        const int blk1 = seg_end - ub;
        const int blast = blk1 - 1;
        stage_load<NT>(stg[0], a, block_pages(trow, blk0, ctx), h, blk0 * kMqKeys, ctx);
        if constexpr (kAhead == 2)
            stage_load<NT>(stg[1], a, block_pages(trow, min(blk0 + 1, blast), ctx), h,
                           min(blk0 + 1, blast) * kMqKeys, ctx);
        // Block blk0 to tile 0 now; its stage then fetches block blk0+kAhead.
        // (The previous segment ended on a barrier after its last reads.)
        stage_store<NT>(stg[0], k_lds2[0], vt_lds2[0]);
        stage_load<NT>(stg[0], a, block_pages(trow, min(blk0 + kAhead, blast), ctx), h,
                       min(blk0 + kAhead, blast) * kMqKeys, ctx);
        BlockPages nxt = block_pages(trow, min(blk0 + kAhead + 1, blast), ctx);
        __syncthreads();
        // One block: `cur` holds block blk+1; it goes to the other tile and
        // then fetches block blk+1+kAhead, while block blk is computed.
        auto do_block = [&](Stage<NT> &cur, int blk) {
            if (blk + 1 < blk1) {
                stage_store<NT>(cur, k_lds2[(blk + 1 - blk0) & 1], vt_lds2[(blk + 1 - blk0) & 1]);
                stage_load<NT>(cur, a, nxt, h, min(blk + 1 + kAhead, blast) * kMqKeys, ctx);
                nxt = block_pages(trow, min(blk + 2 + kAhead, blast), ctx);
            }
            const uint16_t *k_lds = k_lds2[(blk - blk0) & 1];  // block blk0 went to tile 0
            const uint16_t *vt_lds = vt_lds2[(blk - blk0) & 1];
            const int key0 = blk * kMqKeys;

            // S^T for keys key0 + 16*nt + 4*grp + i, query column `col`.
            float4_t s[2];
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                s[nt] = float4_t{0.f, 0.f, 0.f, 0.f};
                const uint16_t *kr = k_lds + (16 * nt + col) * kKRow + 8 * grp;
#pragma unroll
                for (int kk = 0; kk < 8; ++kk)
                    s[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        as_h8(*reinterpret_cast<const uint4 *>(kr + 32 * kk)), as_h8(qb[kk]), s[nt], 0, 0, 0);
            }
            float mx = -INFINITY;
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int key = key0 + 16 * nt + 4 * grp + i;
                    bool vis = qvalid && key < ctx;
                    if (a.tree)
                        vis = vis && (key < ns || ((qbits >> (key - ns)) & 1ull));
                    else
                        vis = vis && key <= qslot;
                    const float v = vis ? s[nt][i] * scale : -INFINITY;
                    s[nt][i] = v;
                    mx = fmaxf(mx, v);
                }
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const float mn = fmaxf(m, mx);
            const float mu = (mn == -INFINITY) ? 0.0f : mn;  // rows with nothing visible yet
            const float corr = __builtin_amdgcn_exp2f(m - mu);
            uint32_t pk[4];
            float psum = 0.0f;
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const uint32_t lo = pack_h2(__builtin_amdgcn_exp2f(s[nt][0] - mu), __builtin_amdgcn_exp2f(s[nt][1] - mu));
                const uint32_t hi = pack_h2(__builtin_amdgcn_exp2f(s[nt][2] - mu), __builtin_amdgcn_exp2f(s[nt][3] - mu));
                pk[2 * nt] = lo;
                pk[2 * nt + 1] = hi;
                psum += (lo_f(lo) + hi_f(lo)) + (lo_f(hi) + hi_f(hi));
            }
            l = l * corr + psum;
            m = mn;
            const half8_t pb = __builtin_bit_cast(half8_t, make_uint4(pk[0], pk[1], pk[2], pk[3]));
#pragma unroll
            for (int dt = 0; dt < 16; ++dt) {
                acc[dt] *= corr;
                const uint16_t *vr = vt_lds + (16 * dt + col) * kVRow + 4 * grp;
                const uint2 v0 = *reinterpret_cast<const uint2 *>(vr);
                const uint2 v1 = *reinterpret_cast<const uint2 *>(vr + 16);
                acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    __builtin_bit_cast(half8_t, make_uint4(v0.x, v0.y, v1.x, v1.y)), pb, acc[dt], 0, 0, 0);
            }
            __syncthreads();  // every wave is done with this tile and the next one is stored
        };
        for (int blk = blk0; blk < blk1; blk += 2) {
            do_block(stg[kAhead - 1], blk);
            if (blk + 1 >= blk1) break;
            do_block(stg[0], blk + 1);
        }

        // The four lane groups hold disjoint keys of each query column.
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
        const bool whole = p == ub && seg_end == ue;
        if (whole) {
            if (qvalid) {
                const float inv = 1.0f / l;
                uint16_t *orow = a.out + (static_cast<size_t>(tok_base + qi) * nh + h * G + wave) * kHeadDim;
#pragma unroll
                for (int dt = 0; dt < 16; ++dt) {
                    uint2 o;
                    o.x = pack_h2(acc[dt][0] * inv, acc[dt][1] * inv);
                    o.y = pack_h2(acc[dt][2] * inv, acc[dt][3] * inv);
                    *reinterpret_cast<uint2 *>(orow + 16 * dt + 4 * grp) = o;
                }
            }
        } else {
            const int slot = 2 * w + (first_seg ? 0 : 1);
            const size_t rowi = (static_cast<size_t>(slot) * G + wave) * kMqRows + col;
            float *ar = a.ws_acc + rowi * kHeadDim;
#pragma unroll
            for (int dt = 0; dt < 16; ++dt)
                *reinterpret_cast<float4 *>(ar + 16 * dt + 4 * grp) =
                    make_float4(acc[dt][0], acc[dt][1], acc[dt][2], acc[dt][3]);
            if (grp == 0) {
                a.ws_ml[rowi * 2] = m;
                a.ws_ml[rowi * 2 + 1] = l;
            }
        }
        p = seg_end;
        first_seg = false;
    }
}

// Merge the partials of units cut across workgroups: one workgroup per
// (unit, head of the group); thread = (query row, 16-dim slice).
template <int G>
__global__ __launch_bounds__(256) void mq_combine_kernel(MultiQueryArgs a) {
    const int u = blockIdx.x;
    const int wave = blockIdx.y;
    const int ub = a.mq_pre[u];
    const int ue = a.mq_pre[u + 1];
    if (ue == ub) return;
    const int W = a.n_wg;
    const int NB = a.total_blocks;
    const int w0 = mq_wg_of(ub, NB, W);
    const int w1 = mq_wg_of(ue - 1, NB, W);
    if (w0 == w1) return;  // written whole by one workgroup
    const int hkv = a.num_kv_heads;
    const int b = upper_index(a.upre, a.n_seqs, u);
    const int x = u - a.upre[b];
    const int tile = x / hkv;
    const int h = x - tile * hkv;
    const int row = threadIdx.x >> 4;
    const int d0 = (threadIdx.x & 15) * 16;
    const int T = a.tok_off[b + 1] - a.tok_off[b];
    const int qi = tile * kMqRows + row;
    if (qi >= T) return;
    float big = -INFINITY;
    for (int ww = w0; ww <= w1; ++ww) {
        const int slot = 2 * ww + (ub <= mq_wg_start(ww, NB, W) ? 0 : 1);
        big = fmaxf(big, a.ws_ml[((static_cast<size_t>(slot) * G + wave) * kMqRows + row) * 2]);
    }
    const float mu = (big == -INFINITY) ? 0.0f : big;
    float lt = 0.0f;
    float o[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) o[e] = 0.0f;
    for (int ww = w0; ww <= w1; ++ww) {
        const int slot = 2 * ww + (ub <= mq_wg_start(ww, NB, W) ? 0 : 1);
        const size_t rowi = (static_cast<size_t>(slot) * G + wave) * kMqRows + row;
        const float c = __builtin_amdgcn_exp2f(a.ws_ml[rowi * 2] - mu);
        lt += c * a.ws_ml[rowi * 2 + 1];
        const float4 *src = reinterpret_cast<const float4 *>(a.ws_acc + rowi * kHeadDim + d0);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float4 v = src[e];
            o[4 * e] += c * v.x;
            o[4 * e + 1] += c * v.y;
            o[4 * e + 2] += c * v.z;
            o[4 * e + 3] += c * v.w;
        }
    }
    const float inv = 1.0f / lt;
    uint16_t *orow = a.out + (static_cast<size_t>(a.tok_off[b] + qi) * a.num_heads + h * G + wave) * kHeadDim + d0;
    uint4 o0, o1;
    o0.x = pack_h2(o[0] * inv, o[1] * inv);
    o0.y = pack_h2(o[2] * inv, o[3] * inv);
    o0.z = pack_h2(o[4] * inv, o[5] * inv);
    o0.w = pack_h2(o[6] * inv, o[7] * inv);
    o1.x = pack_h2(o[8] * inv, o[9] * inv);
    o1.y = pack_h2(o[10] * inv, o[11] * inv);
    o1.z = pack_h2(o[12] * inv, o[13] * inv);
    o1.w = pack_h2(o[14] * inv, o[15] * inv);
    *reinterpret_cast<uint4 *>(orow) = o0;
    *reinterpret_cast<uint4 *>(orow + 8) = o1;
}

template <int G>
hipError_t launch_mq_g(const MultiQueryArgs &a, hipStream_t s) {
    hipLaunchKernelGGL(mq_kernel<G>, dim3(a.n_wg), dim3(64 * G), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(mq_combine_kernel<G>, dim3(a.n_units, G), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_multi_query(const MultiQueryArgs &a, hipStream_t s) {
    if (a.n_units <= 0 || a.total_blocks <= 0) return hipSuccess;
    switch (a.num_heads / a.num_kv_heads) {
        case 1: return launch_mq_g<1>(a, s);
        case 2: return launch_mq_g<2>(a, s);
        case 3: return launch_mq_g<3>(a, s);
        case 4: return launch_mq_g<4>(a, s);
        case 6: return launch_mq_g<6>(a, s);
        case 8: return launch_mq_g<8>(a, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace kva
