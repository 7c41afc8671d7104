// Split-K GQA flash-decode over the paged FP16 cache (gfx950, VALU path).
//
// Semantics: flash_attn_256_decode (flash_attn_256_tuned.hip:198-350) —
// out = softmax(q K^T / sqrt(256)) V per query head, kv head = h*Hkv/H
// (:222) — generalised to a batch of sequences with ragged lengths read
// through a block table, and to any number of KV splits.
//
// Work split: stream-K over pages (see decode_kernel).  A 256-thread
// workgroup processes (sequence, kv head) unit segments; the G = H/Hkv query
// heads of the KV head share every K/V byte it loads (the reference re-read
// each KV head G times, once per query head).  The four waves take
// interleaved 16-token pages of a segment, each with its own online-softmax
// state, and merge through LDS at the segment's end.
//
// Per page, per wave (lane = 16*r + j):
//   loads: the next page's K is prefetched into the second of two register
//       buffers (ping-pong) and the current page's V is issued before QK, so
//       every wave keeps 8-16 KB in flight during its arithmetic;
//   QK: the 16 lanes of row r hold tokens r, r+4, r+8, r+12, 16 dims each
//       (16-byte pieces j and j+16 of the 512-byte row: each load is 256
//       contiguous bytes per token), dot with the G query heads via
//       v_dot2_f32_f16; a 16-lane DPP sum finishes each score;
//   softmax: log2 domain; page max over the four rows with row-broadcast
//       DPP and one v_readlane (no LDS round trips); v_exp_f32;
//       probabilities rounded to fp16 pairs;
//   PV: lane owns dims 4*lane..4*lane+3 of all G heads; tokens t and t+4
//       are paired so one v_dot2_f32_f16 folds two tokens; the pair's
//       probabilities come from row t%4 via v_readlane (wave-uniform).
#include "k_common.h"
#include "kva_internal.h"

namespace kva {
namespace {

constexpr float kLog2e = 1.4426950408889634f;

// Sum over the 16 lanes of a DPP row; every lane gets the sum.
__device__ __forceinline__ float row16_sum(float x) {
    x += dpp_f<kDppQuadXor1>(x);
    x += dpp_f<kDppQuadXor2>(x);
    x += dpp_f<kDppRowHalfMirror>(x);
    x += dpp_f<kDppRowMirror>(x);
    return x;
}

struct KRegs {
    uint4 k[4][2];  // tokens r + 4*t4, pieces j and j+16
};
struct VRegs {
    uint2 v[16];    // all 16 tokens, dims 4*lane..4*lane+3
};

// Load a page's K (row stride row_bytes) into registers; rows >= lim read as 0.
template <bool kFull>
__device__ __forceinline__ void load_k(KRegs &p, const char *kb, uint32_t koff, int row_bytes,
                                       int r, int lim) {
#pragma unroll
    for (int t4 = 0; t4 < 4; ++t4) {
        const char *base = kb + t4 * 4 * row_bytes + koff;
        if (kFull || r + 4 * t4 < lim) {
            p.k[t4][0] = *reinterpret_cast<const uint4 *>(base);
            p.k[t4][1] = *reinterpret_cast<const uint4 *>(base + 256);
        } else {
            p.k[t4][0] = make_uint4(0, 0, 0, 0);
            p.k[t4][1] = make_uint4(0, 0, 0, 0);
        }
    }
}

template <bool kFull>
__device__ __forceinline__ void load_v(VRegs &p, const char *vb, uint32_t voff, int row_bytes,
                                       int lim) {
#pragma unroll
    for (int t = 0; t < 16; ++t) {
        if (kFull || t < lim)
            p.v[t] = *reinterpret_cast<const uint2 *>(vb + t * row_bytes + voff);
        else
            p.v[t] = make_uint2(0, 0);
    }
}

template <int G>
struct WaveState {
    float m[G], l[G], acc[G][4];
};

// Fold one page into the wave's online-softmax state.  lim < 16 masks rows.
template <int G, bool kFull>
__device__ __forceinline__ void compute_page(WaveState<G> &st, const KRegs &p, const VRegs &pv,
                                             const uint4 (&qv)[G][2], int r, int lim) {
    const float qk_scale = kLog2e / 16.0f;  // log2(e) / sqrt(256)
    float s[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4) {
            float x = 0.0f;
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                x = dot2(qv[g][q].x, p.k[t4][q].x, x);
                x = dot2(qv[g][q].y, p.k[t4][q].y, x);
                x = dot2(qv[g][q].z, p.k[t4][q].z, x);
                x = dot2(qv[g][q].w, p.k[t4][q].w, x);
            }
            s[g][t4] = row16_sum(x) * qk_scale;
        }
    if (!kFull) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int t4 = 0; t4 < 4; ++t4) s[g][t4] = (r + 4 * t4 < lim) ? s[g][t4] : -INFINITY;
    }
    // Page max per head: the 16 lanes of a row agree, so a row-broadcast DPP
    // max (rows 1,3 <- rows 0,2; then rows 2,3 <- row 1) leaves the wave max
    // in lane 63; all heads are reduced together to overlap the DPP hazards.
    float bm[G];
#pragma unroll
    for (int g = 0; g < G; ++g) bm[g] = fmaxf(fmaxf(s[g][0], s[g][1]), fmaxf(s[g][2], s[g][3]));
#pragma unroll
    for (int g = 0; g < G; ++g) bm[g] = fmaxf(bm[g], dpp_masked_f<kDppRowBcast15, 0xA>(bm[g]));
#pragma unroll
    for (int g = 0; g < G; ++g) bm[g] = fmaxf(bm[g], dpp_masked_f<kDppRowBcast31, 0xC>(bm[g]));
    uint32_t pa[G], pb[G];  // fp16 pairs: tokens (r, r+4) and (r+8, r+12)
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float mn = fmaxf(st.m[g], __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                                                __builtin_bit_cast(int, bm[g]), 63)));
        const float corr = __builtin_amdgcn_exp2f(st.m[g] - mn);
        pa[g] = pack_h2(__builtin_amdgcn_exp2f(s[g][0] - mn), __builtin_amdgcn_exp2f(s[g][1] - mn));
        pb[g] = pack_h2(__builtin_amdgcn_exp2f(s[g][2] - mn), __builtin_amdgcn_exp2f(s[g][3] - mn));
        st.l[g] = st.l[g] * corr + ((lo_f(pa[g]) + hi_f(pa[g])) + (lo_f(pb[g]) + hi_f(pb[g])));
        st.m[g] = mn;
#pragma unroll
        for (int c = 0; c < 4; ++c) st.acc[g][c] *= corr;
    }
#pragma unroll
    for (int pr = 0; pr < 8; ++pr) {
        // Pair pr: row rr = pr & 3, tokens (rr, rr+4) or (rr+8, rr+12).
        const int rr = pr & 3;
        const int t0 = rr + (pr >> 2) * 8;
        const uint2 va = pv.v[t0];
        const uint2 vb = pv.v[t0 + 4];
        const uint32_t v0 = (va.x & 0xffffu) | (vb.x << 16);
        const uint32_t v1 = (va.x >> 16) | (vb.x & 0xffff0000u);
        const uint32_t v2 = (va.y & 0xffffu) | (vb.y << 16);
        const uint32_t v3 = (va.y >> 16) | (vb.y & 0xffff0000u);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const uint32_t src = (pr >> 2) ? pb[g] : pa[g];
            const uint32_t pp =
                static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(src), rr * 16));
            st.acc[g][0] = dot2(pp, v0, st.acc[g][0]);
            st.acc[g][1] = dot2(pp, v1, st.acc[g][1]);
            st.acc[g][2] = dot2(pp, v2, st.acc[g][2]);
            st.acc[g][3] = dot2(pp, v3, st.acc[g][3]);
        }
    }
}

// First page of workgroup w when P pages are shared by W workgroups.
__device__ __forceinline__ int wg_start(int w, int P, int W) {
    return static_cast<int>(static_cast<int64_t>(w) * P / W);
}

// The workgroup whose page range holds page p.
__device__ __forceinline__ int wg_of_page(int p, int P, int W) {
    int w = static_cast<int>(static_cast<int64_t>(p) * W / P);
    while (w + 1 < W && wg_start(w + 1, P, W) <= p) ++w;
    return w;
}

// Pages of all (sequence, kv head) units before sequence b (units are
// ordered sequence-major, then kv head).
__device__ __forceinline__ int seq_page_base(const DecodeArgs &a, int b, int npg) {
    return a.pre_seq ? a.pre_seq[b] : b * a.num_kv_heads * npg;
}

// Stream-K decode: the pages of every (sequence, kv head) unit are laid end
// to end and workgroup w takes pages [wg_start(w), wg_start(w+1)) — equal
// shares, whatever the ragged lengths.  A workgroup walks the unit segments
// of its range; a unit it covers whole is written out directly, a unit cut
// by a range boundary leaves a partial (m, l, acc) in slot 2w (the range's
// first unit) or 2w+1 (its last unit) for combine_kernel.
template <int G>
__global__ __launch_bounds__(256) void decode_kernel(DecodeArgs a) {
    const int w = blockIdx.x;
    const int W = a.n_wg;
    const int P = a.total_pages;
    const int p_begin = wg_start(w, P, W);
    const int p_end = wg_start(w + 1, P, W);
    if (p_begin >= p_end) return;  // uniform over the workgroup
    const int hkv = a.num_kv_heads;
    const int nh = a.num_heads;

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int r = lane >> 4;
    const int j = lane & 15;
    const int row_bytes = hkv * kHeadDim * 2;
    const size_t page_bytes = static_cast<size_t>(kBlockTokens) * row_bytes;
    const uint32_t koff = r * row_bytes + 16 * j;
    const uint32_t voff = 8 * lane;

    // Sequence holding p_begin: the last b with base(b) <= p_begin.
    int b;
    if (a.pre_seq) {
        int lo = 0, hi = a.n_seqs - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (a.pre_seq[mid] <= p_begin) lo = mid; else hi = mid - 1;
        }
        b = lo;
    } else {
        b = p_begin / (hkv * ((a.ctx_len_const + 15) >> 4));
    }

    __shared__ float sm_ml[kDecodeWaves][G][2];
    __shared__ float4 sm_acc[kDecodeWaves][G][64];
    int p = p_begin;
    bool first_seg = true;
    while (p < p_end) {
        const int ctx = a.ctx_lens ? a.ctx_lens[b] : a.ctx_len_const;
        const int npg = (ctx + 15) >> 4;
        const int base_b = seq_page_base(a, b, npg);
        if (npg == 0 || p >= base_b + hkv * npg) {  // empty or finished sequence
            ++b;
            continue;
        }
        const int h = (p - base_b) / npg;
        const int pg0 = p - base_b - h * npg;
        const int seg_end = min(base_b + (h + 1) * npg, p_end);
        const int pg1 = pg0 + (seg_end - p);

        const int32_t *trow =
            a.table ? a.table + static_cast<size_t>(a.seq_ids[b]) * a.table_stride : nullptr;
        const size_t seq_base = a.table ? 0 : static_cast<size_t>(b) * a.seq_stride * 2;
        const char *kpool = reinterpret_cast<const char *>(a.k_pool) + seq_base + h * kHeadDim * 2;
        const char *vpool = reinterpret_cast<const char *>(a.v_pool) + seq_base + h * kHeadDim * 2;

        uint4 qv[G][2];
        const uint16_t *qb =
            a.q + (static_cast<size_t>(b) * nh + static_cast<size_t>(h) * G) * kHeadDim;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            qv[g][0] = ld16(qb + g * kHeadDim + 8 * j);
            qv[g][1] = ld16(qb + g * kHeadDim + 8 * (j + 16));
        }
        WaveState<G> st;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            st.m[g] = -INFINITY;
            st.l[g] = 0.0f;
#pragma unroll
            for (int c = 0; c < 4; ++c) st.acc[g][c] = 0.0f;
        }

        // This wave's pages of the segment: first, first+4, ...  All are full
        // except the unit's last page when the length is not a page multiple.
        const int first = pg0 + wave;
        const int n_pages = first < pg1 ? (pg1 - first + kDecodeWaves - 1) / kDecodeWaves : 0;
        const int last_lim = ctx - (npg - 1) * kBlockTokens;
        const bool owns_partial = last_lim < kBlockTokens && n_pages > 0 &&
                                  first + (n_pages - 1) * kDecodeWaves == npg - 1;
        const int n_full = n_pages - (owns_partial ? 1 : 0);
        auto page_off = [&](int blk) -> size_t {
            const int pb = trow ? __builtin_amdgcn_readfirstlane(trow[blk]) : blk;
            return static_cast<size_t>(pb) * page_bytes;
        };

        // K of the next page is prefetched into the idle one of two register
        // buffers; V of the current page is issued first and lands during QK.
        KRegs KA, KB;
        VRegs V;
#if KVA_DEEP_PREFETCH
        VRegs V2;
        if (n_full > 0) {
            load_k<true>(KA, kpool + page_off(first), koff, row_bytes, r, kBlockTokens);
            load_v<true>(V, vpool + page_off(first), voff, row_bytes, kBlockTokens);
        }
        for (int i = 0; i < n_full; i += 2) {
            if (i + 1 < n_full) {
                const size_t o = page_off(first + (i + 1) * kDecodeWaves);
                load_k<true>(KB, kpool + o, koff, row_bytes, r, kBlockTokens);
                load_v<true>(V2, vpool + o, voff, row_bytes, kBlockTokens);
            }
            compute_page<G, true>(st, KA, V, qv, r, kBlockTokens);
            if (i + 1 >= n_full) break;
            if (i + 2 < n_full) {
                const size_t o = page_off(first + (i + 2) * kDecodeWaves);
                load_k<true>(KA, kpool + o, koff, row_bytes, r, kBlockTokens);
                load_v<true>(V, vpool + o, voff, row_bytes, kBlockTokens);
            }
            compute_page<G, true>(st, KB, V2, qv, r, kBlockTokens);
        }
#else
        if (n_full > 0) load_k<true>(KA, kpool + page_off(first), koff, row_bytes, r, kBlockTokens);
        for (int i = 0; i < n_full; i += 2) {
            load_v<true>(V, vpool + page_off(first + i * kDecodeWaves), voff, row_bytes, kBlockTokens);
            if (i + 1 < n_full)
                load_k<true>(KB, kpool + page_off(first + (i + 1) * kDecodeWaves), koff, row_bytes, r,
                             kBlockTokens);
            compute_page<G, true>(st, KA, V, qv, r, kBlockTokens);
            if (i + 1 >= n_full) break;
            load_v<true>(V, vpool + page_off(first + (i + 1) * kDecodeWaves), voff, row_bytes,
                         kBlockTokens);
            if (i + 2 < n_full)
                load_k<true>(KA, kpool + page_off(first + (i + 2) * kDecodeWaves), koff, row_bytes, r,
                             kBlockTokens);
            compute_page<G, true>(st, KB, V, qv, r, kBlockTokens);
        }
#endif
        if (owns_partial) {
            const size_t o = page_off(npg - 1);
            load_k<false>(KA, kpool + o, koff, row_bytes, r, last_lim);
            load_v<false>(V, vpool + o, voff, row_bytes, last_lim);
            compute_page<G, false>(st, KA, V, qv, r, last_lim);
        }

        // Merge the four waves through LDS; write the output (whole unit) or
        // this range's partial for the unit.
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float lt = st.l[g];  // rows hold disjoint tokens: sum the four rows
            lt += __shfl_xor(lt, 16);
            lt += __shfl_xor(lt, 32);
            if (lane == 0) {
                sm_ml[wave][g][0] = st.m[g];
                sm_ml[wave][g][1] = lt;
            }
            sm_acc[wave][g][lane] = make_float4(st.acc[g][0], st.acc[g][1], st.acc[g][2], st.acc[g][3]);
        }
        __syncthreads();
        const bool whole = pg0 == 0 && pg1 == npg;
        const int slot = 2 * w + (first_seg ? 0 : 1);
        const int d = threadIdx.x;  // one output dim per thread
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float mw[kDecodeWaves];
            float big = -INFINITY;
#pragma unroll
            for (int wv = 0; wv < kDecodeWaves; ++wv) {
                mw[wv] = sm_ml[wv][g][0];
                big = fmaxf(big, mw[wv]);
            }
            float lt = 0.0f, at = 0.0f;
#pragma unroll
            for (int wv = 0; wv < kDecodeWaves; ++wv) {
                const float cw = (mw[wv] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mw[wv] - big);
                lt += cw * sm_ml[wv][g][1];
                at += cw * reinterpret_cast<const float *>(&sm_acc[wv][g][0])[d];
            }
            if (whole) {
                a.out[(static_cast<size_t>(b) * nh + h * G + g) * kHeadDim + d] = f2h(at / lt);
            } else {
                const size_t u = static_cast<size_t>(slot) * G + g;
                a.ws_acc[u * kHeadDim + d] = at;
                if (d == 0) {
                    a.ws_ml[u * 2] = big;
                    a.ws_ml[u * 2 + 1] = lt;
                }
            }
        }
        __syncthreads();  // LDS is reused by the next segment
        p = seg_end;
        first_seg = false;
    }
}

// Merge the partials of one (unit, query head of its group) whose pages were
// cut across workgroups: 64 lanes x 4 dims.  A separate launch (stream order
// makes the partials visible), so no cross-workgroup fences are needed: an
// agent-scope release on every decode workgroup costs an L2 writeback per
// workgroup on multi-XCD parts.
template <int G>
__global__ __launch_bounds__(64) void combine_kernel(DecodeArgs a) {
    const int u = blockIdx.x;
    const int g = blockIdx.y;
    const int hkv = a.num_kv_heads;
    const int b = u / hkv;
    const int h = u - b * hkv;
    const int lane = threadIdx.x;
    const int W = a.n_wg;
    const int P = a.total_pages;
    const int ctx = a.ctx_lens ? a.ctx_lens[b] : a.ctx_len_const;
    const int npg = (ctx + 15) >> 4;
    if (npg == 0) return;
    const int first = seq_page_base(a, b, npg) + h * npg;
    const int w0 = wg_of_page(first, P, W);
    const int w1 = wg_of_page(first + npg - 1, P, W);
    if (w0 == w1) return;  // one workgroup covered the unit and wrote it
    float big = -INFINITY;
    for (int w = w0; w <= w1; ++w) {
        const int slot = 2 * w + (first <= wg_start(w, P, W) ? 0 : 1);
        big = fmaxf(big, a.ws_ml[(static_cast<size_t>(slot) * G + g) * 2]);
    }
    float lt = 0.0f;
    float4 at = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int w = w0; w <= w1; ++w) {
        const int slot = 2 * w + (first <= wg_start(w, P, W) ? 0 : 1);
        const size_t s = static_cast<size_t>(slot) * G + g;
        const float c = __builtin_amdgcn_exp2f(a.ws_ml[s * 2] - big);
        lt += c * a.ws_ml[s * 2 + 1];
        const float4 v = reinterpret_cast<const float4 *>(a.ws_acc + s * kHeadDim)[lane];
        at.x += c * v.x;
        at.y += c * v.y;
        at.z += c * v.z;
        at.w += c * v.w;
    }
    const float inv = 1.0f / lt;
    uint2 o;
    o.x = pack_h2(at.x * inv, at.y * inv);
    o.y = pack_h2(at.z * inv, at.w * inv);
    *reinterpret_cast<uint2 *>(a.out + (static_cast<size_t>(b) * a.num_heads + h * G + g) * kHeadDim +
                               4 * lane) = o;
}

template <int G>
hipError_t launch_g(const DecodeArgs &a, hipStream_t s) {
    hipLaunchKernelGGL(decode_kernel<G>, dim3(a.n_wg), dim3(256), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !a.ws_acc) return e;
    hipLaunchKernelGGL(combine_kernel<G>, dim3(a.n_seqs * a.num_kv_heads, G), dim3(64), 0, s, a);
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
