// Split-K GQA flash-decode over the paged FP16 cache (gfx950, VALU path).
//
// Semantics: flash_attn_256_decode (flash_attn_256_tuned.hip:198-350) —
// out = softmax(q K^T / sqrt(256)) V per query head, kv head = h*Hkv/H
// (:222) — generalised to a batch of sequences with ragged lengths read
// through a block table, and to any number of KV splits.
//
// Work unit: one 256-thread workgroup per (split, kv head, sequence).  The
// G = H/Hkv query heads of the KV head share every K/V byte the workgroup
// loads (the reference re-read each KV head G times, once per query head).
// The four waves take interleaved 16-token pages of the split, each with its
// own online-softmax state, and merge through LDS at the end.
//
// Per page, per wave (lane = 8*r + j):
//   QK: lanes of group r hold tokens r and r+8, 32 dims each (pieces
//       j, j+8, j+16, j+24 of 16 bytes), dot with the G query heads via
//       v_dot2_f32_f16; an 8-lane DPP sum finishes each score.
//   softmax: scores in the log2 domain; page max across the 8 groups with
//       DPP row rotate + two cross-row shuffles; v_exp_f32.
//   PV: lane owns dims 4*lane..4*lane+3 of all G heads; tokens r and r+8
//       are paired so one v_dot2_f32_f16 folds two tokens; the pair's
//       probabilities (fp16x2) come from group r via v_readlane (uniform).
// All K/V loads are 16- or 8-byte lane loads of 512-byte rows (coalesced).
#include "k_common.h"
#include "kva_internal.h"

namespace kva {
namespace {

constexpr float kLog2e = 1.4426950408889634f;

template <int G>
__global__ __launch_bounds__(256) void decode_kernel(DecodeArgs a) {
    const int split = blockIdx.x;
    const int h = blockIdx.y;
    const int b = blockIdx.z;
    const int hkv = a.num_kv_heads;
    const int nh = a.num_heads;
    const int ctx = a.ctx_lens ? a.ctx_lens[b] : a.ctx_len_const;
    const int tok_begin = split * a.split_tokens;
    if (tok_begin >= ctx) return;  // uniform over the workgroup
    const int tok_end = min(ctx, tok_begin + a.split_tokens);
    const int32_t *trow =
        a.table ? a.table + static_cast<size_t>(a.seq_ids[b]) * a.table_stride : nullptr;

    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int r = lane >> 3;
    const int j = lane & 7;
    const size_t row_elems = static_cast<size_t>(hkv) * kHeadDim;
    const size_t block_elems = kBlockTokens * row_elems;
    const float qk_scale = kLog2e / 16.0f;  // log2(e) / sqrt(256)

    uint4 qv[G][4];
    const uint16_t *qb = a.q + (static_cast<size_t>(b) * nh + static_cast<size_t>(h) * G) * kHeadDim;
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int k = 0; k < 4; ++k) qv[g][k] = ld16(qb + g * kHeadDim + 8 * (j + 8 * k));

    float m[G], l[G], acc[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[g][c] = 0.0f;
    }

    const int blk_begin = tok_begin >> 4;
    const int blk_end = (tok_end + 15) >> 4;
    for (int blk = blk_begin + wave; blk < blk_end; blk += kDecodeWaves) {
        const size_t page = trow ? static_cast<size_t>(trow[blk]) * block_elems
                                 : b * a.seq_stride + static_cast<size_t>(blk) * block_elems;
        const uint16_t *kb = a.k_pool + page + h * kHeadDim;
        const uint16_t *vb = a.v_pool + page + h * kHeadDim;
        const int page_tok = blk * kBlockTokens;
        const int lim = min(kBlockTokens, tok_end - page_tok);  // valid rows of this page
        uint4 k0[4], k1[4];
        uint2 vt[16];
        if (lim == kBlockTokens) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                k0[k] = ld16(kb + r * row_elems + 8 * (j + 8 * k));
                k1[k] = ld16(kb + (r + 8) * row_elems + 8 * (j + 8 * k));
            }
#pragma unroll
            for (int t = 0; t < 16; ++t) vt[t] = ld8(vb + t * row_elems + 4 * lane);
        } else {
            // Last page of the sequence: rows at or past the length are not
            // read (a contiguous cache may end there) and count as zeros.
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                k0[k] = (r < lim) ? ld16(kb + r * row_elems + 8 * (j + 8 * k)) : make_uint4(0, 0, 0, 0);
                k1[k] = (r + 8 < lim) ? ld16(kb + (r + 8) * row_elems + 8 * (j + 8 * k))
                                      : make_uint4(0, 0, 0, 0);
            }
#pragma unroll
            for (int t = 0; t < 16; ++t)
                vt[t] = (t < lim) ? ld8(vb + t * row_elems + 4 * lane) : make_uint2(0, 0);
        }

        float s0[G], s1[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float x0 = 0.0f, x1 = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                x0 = dot2(qv[g][k].x, k0[k].x, x0);
                x0 = dot2(qv[g][k].y, k0[k].y, x0);
                x0 = dot2(qv[g][k].z, k0[k].z, x0);
                x0 = dot2(qv[g][k].w, k0[k].w, x0);
                x1 = dot2(qv[g][k].x, k1[k].x, x1);
                x1 = dot2(qv[g][k].y, k1[k].y, x1);
                x1 = dot2(qv[g][k].z, k1[k].z, x1);
                x1 = dot2(qv[g][k].w, k1[k].w, x1);
            }
            s0[g] = group8_sum(x0) * qk_scale;
            s1[g] = group8_sum(x1) * qk_scale;
        }
        if (lim < kBlockTokens) {
            // Rows past the length get probability exactly 0 (their V is 0).
#pragma unroll
            for (int g = 0; g < G; ++g) {
                s0[g] = (r < lim) ? s0[g] : -INFINITY;
                s1[g] = (r + 8 < lim) ? s1[g] : -INFINITY;
            }
        }

        uint32_t pp[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float bm = wave_groups_max(fmaxf(s0[g], s1[g]));
            const float mn = fmaxf(m[g], bm);
            const float corr = __builtin_amdgcn_exp2f(m[g] - mn);
            const uint32_t p2 = pack_h2(__builtin_amdgcn_exp2f(s0[g] - mn),
                                        __builtin_amdgcn_exp2f(s1[g] - mn));
            pp[g] = p2;
            l[g] = l[g] * corr + (lo_f(p2) + hi_f(p2));
            m[g] = mn;
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[g][c] *= corr;
        }
#pragma unroll
        for (int rr = 0; rr < 8; ++rr) {
            const uint2 va = vt[rr];
            const uint2 vb2 = vt[rr + 8];
            const uint32_t v0 = (va.x & 0xffffu) | (vb2.x << 16);
            const uint32_t v1 = (va.x >> 16) | (vb2.x & 0xffff0000u);
            const uint32_t v2 = (va.y & 0xffffu) | (vb2.y << 16);
            const uint32_t v3 = (va.y >> 16) | (vb2.y & 0xffff0000u);
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const uint32_t pr = static_cast<uint32_t>(
                    __builtin_amdgcn_readlane(static_cast<int>(pp[g]), rr * 8));
                acc[g][0] = dot2(pr, v0, acc[g][0]);
                acc[g][1] = dot2(pr, v1, acc[g][1]);
                acc[g][2] = dot2(pr, v2, acc[g][2]);
                acc[g][3] = dot2(pr, v3, acc[g][3]);
            }
        }
    }

    // Merge the four waves (LDS), then write the split's partial state or,
    // with a single split, the normalised output.
    __shared__ float sm_ml[kDecodeWaves][G][2];
    __shared__ float4 sm_acc[kDecodeWaves][G][64];
    __shared__ int sm_last;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float lt = wave_groups_sum(l[g]);
        if (lane == 0) {
            sm_ml[wave][g][0] = m[g];
            sm_ml[wave][g][1] = lt;
        }
        sm_acc[wave][g][lane] = make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
    }
    __syncthreads();
    const int d = threadIdx.x;  // one output dim per thread
    const size_t unit0 = (static_cast<size_t>(b) * a.n_splits * hkv + h) * G;  // split 0, head 0
    const size_t split_stride = static_cast<size_t>(hkv) * G;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float mw[kDecodeWaves];
        float big = -INFINITY;
#pragma unroll
        for (int w = 0; w < kDecodeWaves; ++w) {
            mw[w] = sm_ml[w][g][0];
            big = fmaxf(big, mw[w]);
        }
        float lt = 0.0f, at = 0.0f;
#pragma unroll
        for (int w = 0; w < kDecodeWaves; ++w) {
            const float cw = (mw[w] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mw[w] - big);
            lt += cw * sm_ml[w][g][1];
            at += cw * reinterpret_cast<const float *>(&sm_acc[w][g][0])[d];
        }
        if (a.n_splits == 1) {
            a.out[(static_cast<size_t>(b) * nh + h * G + g) * kHeadDim + d] = f2h(at / lt);
        } else {
            const size_t unit = unit0 + split * split_stride + g;
            a.ws_acc[unit * kHeadDim + d] = at;
            if (d == 0) {
                a.ws_ml[unit * 2] = big;
                a.ws_ml[unit * 2 + 1] = lt;
            }
        }
    }
    if (a.n_splits == 1) return;

    // Split-K combine, fused: the last workgroup of this (sequence, KV head)
    // to finish merges every split.  Partials are released at agent scope
    // before the arrival count and acquired after it (the L2s of different
    // XCDs are not coherent without these fences); the last arrival resets
    // the counter for the next launch.
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        int *ctr = a.counters + static_cast<size_t>(b) * hkv + h;
        const int ns = (ctx + a.split_tokens - 1) / a.split_tokens;
        const int prev = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        const int last = prev == ns - 1;
        if (last) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sm_last = last;
    }
    __syncthreads();
    if (!sm_last) return;
    __threadfence();
    const int ns = (ctx + a.split_tokens - 1) / a.split_tokens;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float big = -INFINITY;
        for (int sp = 0; sp < ns; ++sp)
            big = fmaxf(big, a.ws_ml[(unit0 + sp * split_stride + g) * 2]);
        float lt = 0.0f, at = 0.0f;
        for (int sp = 0; sp < ns; ++sp) {
            const size_t u = unit0 + sp * split_stride + g;
            const float c = __builtin_amdgcn_exp2f(a.ws_ml[u * 2] - big);
            lt += c * a.ws_ml[u * 2 + 1];
            at += c * a.ws_acc[u * kHeadDim + d];
        }
        a.out[(static_cast<size_t>(b) * nh + h * G + g) * kHeadDim + d] = f2h(at / lt);
    }
}

template <int G>
hipError_t launch_g(const DecodeArgs &a, hipStream_t s) {
    const dim3 grid(a.n_splits, a.num_kv_heads, a.n_seqs);
    hipLaunchKernelGGL(decode_kernel<G>, grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_decode(const DecodeArgs &a, hipStream_t s) {
    if (a.n_seqs <= 0) return hipSuccess;
    switch (a.num_heads / a.num_kv_heads) {
        case 1: return launch_g<1>(a, s);
        case 2: return launch_g<2>(a, s);
        case 3: return launch_g<3>(a, s);
        case 4: return launch_g<4>(a, s);
        case 6: return launch_g<6>(a, s);
        case 8: return launch_g<8>(a, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace kva
