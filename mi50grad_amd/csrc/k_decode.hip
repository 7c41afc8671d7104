// GQA flash-decode over the paged FP16 cache (gfx950).
//
// Semantics: flash_attn_256_decode (flash_attn_256_tuned.hip:198-350) —
// out = softmax(q K^T / sqrt(256)) V per query head, kv head = h*Hkv/H
// (:222) — generalised to a batch of sequences with ragged lengths read
// through a block table, and to any split of the keys.  The G = H/Hkv query
// heads of a kv head share every K/V byte a wave loads (the reference
// re-read each kv head G times, once per query head).
//
// Three launches:
//   decode_mfma_kernel + combine_kernel: stream-K over pages for long steps.
//       The pages of every sequence are laid end to end and workgroup w
//       takes [w*P/W, (w+1)*P/W), equal shares whatever the ragged lengths;
//       one wave per kv head walks every page of the share, QK on the
//       matrix cores, PV on v_dot2_f32_f16.  A sequence the share covers
//       whole is written out directly; a cut one leaves a partial (m, l,
//       acc) per head for combine_kernel.
//   whole_kernel: steps of short sequences (no combine): a workgroup walks
//       one sequence for one kv head and a group of its query heads, eight
//       waves on half pages with QK and PV on v_dot2_f32_f16 (below),
//       merged through LDS; optionally with the step's append fused in.
//
// The whole-sequence form's half page, per wave (lane = 16*r + j):
//   loads: a ring of register buffers; buffer loads through a per-page
//       resource whose range check zero-fills rows past a sequence's end
//       and turns a prefetch past the range into a no-op that still counts;
//   QK: the 16 lanes of row r hold tokens 8k+r and 8k+r+4, 16 dims each
//       (16-byte pieces j and j+16 of the 512-byte row), dot with the G query
//       rows (held in registers) via v_dot2_f32_f16; a 16-lane DPP sum
//       finishes each score;
//   softmax: log2 domain; max over the four rows with row-broadcast DPP and
//       one v_readlane (no LDS round trips); v_exp_f32; probabilities
//       rounded to fp16 pairs;
//   PV: lane owns dims 4*lane..4*lane+3 of all G heads; tokens t and t+4
//       are paired so one v_dot2_f32_f16 folds two tokens; the pair's
//       probabilities (row t's) reach every lane by an LDS broadcast.
#include "k_common.h"
#include "k_normrope.h"
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

constexpr int kHalf = kBlockTokens / 2;  // tokens per wave per page

// One wave's half page: K tokens 8k + r + 4*t4 (t4 = 0, 1), pieces j and
// j+16; V tokens 8k + t (t = 0..7), dims 4*lane..4*lane+3.
struct HalfPage {
    uint4 k[2][2];
    uint2 v[kHalf];
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t page_rsrc(const char *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(base), 0, bytes, 0x00020000);
}

// Load a half page (kb, vb: the page's first row, this head's 512 bytes;
// koff/voff already hold this wave's first row).  One branch-free form for
// every page: each row offset travels in voffset, and the resource's range
// (num_records = valid rows * row_bytes) makes the rows past the sequence's
// end read as zeros without touching memory; a disabled page (num_records =
// 0) fetches nothing.  Every step issues the same loads, so the compiler's
// load counters stay exact (a branch between two load forms made it drain
// the loads in flight).
__device__ __forceinline__ void load_half(HalfPage &p, const char *kb, const char *vb, int lim, bool on,
                                          uint32_t koff, uint32_t voff, int row_bytes) {
    const uint32_t n = on ? static_cast<uint32_t>(lim * row_bytes) : 0u;
    const auto rk = page_rsrc(kb, n), rv = page_rsrc(vb, n);
#pragma unroll
    for (int t4 = 0; t4 < 2; ++t4)
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const auto x = __builtin_amdgcn_raw_buffer_load_b128(rk, koff + t4 * 4 * row_bytes + 256 * q, 0, 0);
            p.k[t4][q] = make_uint4(x[0], x[1], x[2], x[3]);
        }
#pragma unroll
    for (int t = 0; t < kHalf; ++t) {
        const auto x = __builtin_amdgcn_raw_buffer_load_b64(rv, voff + t * row_bytes, 0, 0);
        p.v[t] = make_uint2(x[0], x[1]);
    }
}

// A use of every register of a half page (no instructions): a wave that
// skips a half page still waits for its loads there, so every path leaves
// the ring's registers in the same state and the compiler's load-counter
// waits stay exact (a path with loads still pending would make it wait for
// all loads in flight wherever those registers are reused).
__device__ __forceinline__ void consume(const HalfPage &p) {
#pragma unroll
    for (int t4 = 0; t4 < 2; ++t4)
#pragma unroll
        for (int q = 0; q < 2; ++q) asm volatile("" ::"v"(p.k[t4][q].x), "v"(p.k[t4][q].y), "v"(p.k[t4][q].z), "v"(p.k[t4][q].w));
#pragma unroll
    for (int t = 0; t < kHalf; ++t) asm volatile("" ::"v"(p.v[t].x), "v"(p.v[t].y));
}

// m is the running max of the raw scores q.k; probabilities are
// exp2((s - m) * log2(e)/16).
template <int G>
struct WaveState {
    float m[G], l[G], acc[G][4];
};

template <int G>
__device__ __forceinline__ void reset(WaveState<G> &st) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
        st.m[g] = -INFINITY;
        st.l[g] = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; ++c) st.acc[g][c] = 0.0f;
    }
}

// Fold a half page into the wave's online-softmax state; tokens r + 4*t4 >=
// lim (relative to the half) are masked, lim >= 1.  qv: this lane's 16-byte
// pieces j and j+16 of the G query rows.  pbuf: this wave's 32 dwords of LDS
// through which PV's probability pairs are broadcast: a v_readlane per pair
// and head would cost a VALU issue plus a dependent-SGPR stall each.
template <int G>
__device__ __forceinline__ void compute_half(WaveState<G> &st, const HalfPage &p, const uint4 (&qv)[G][2],
                                             int r, int j, int lim, uint32_t *pbuf) {
    const float qk_scale = kLog2e / 16.0f;  // log2(e) / sqrt(256)
    const uint32_t kOnes = 0x3c003c00u;     // fp16 pair (1, 1)
    float s[G][2];
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
        for (int t4 = 0; t4 < 2; ++t4) {
            float x = 0.0f;
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                x = dot2(qv[g][q].x, p.k[t4][q].x, x);
                x = dot2(qv[g][q].y, p.k[t4][q].y, x);
                x = dot2(qv[g][q].z, p.k[t4][q].z, x);
                x = dot2(qv[g][q].w, p.k[t4][q].w, x);
            }
            s[g][t4] = row16_sum(x);
        }
    }
    if (lim < kHalf) {  // the sequence's last page (wave-uniform)
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int t4 = 0; t4 < 2; ++t4) s[g][t4] = (r + 4 * t4 < lim) ? s[g][t4] : -INFINITY;
    }
    // Max per head: the 16 lanes of a row agree, so a row-broadcast DPP max
    // (rows 1,3 <- rows 0,2; then rows 2,3 <- row 1) leaves the wave max in
    // lane 63; all heads are reduced together to overlap the DPP hazards.
    float bm[G];
#pragma unroll
    for (int g = 0; g < G; ++g) bm[g] = fmaxf(s[g][0], s[g][1]);
#pragma unroll
    for (int g = 0; g < G; ++g) bm[g] = fmaxf(bm[g], dpp_masked_f<kDppRowBcast15, 0xA>(bm[g]));
#pragma unroll
    for (int g = 0; g < G; ++g) bm[g] = fmaxf(bm[g], dpp_masked_f<kDppRowBcast31, 0xC>(bm[g]));
    float mn[G];
    bool grew = false;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        mn[g] = fmaxf(st.m[g], __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, bm[g]), 63)));
        grew = grew || mn[g] > st.m[g];
    }
    // Rescale l and acc only when some head's max grew (wave-uniform test):
    // after the first pages of a sequence the max rarely moves.
    if (grew) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float corr = __builtin_amdgcn_exp2f((st.m[g] - mn[g]) * qk_scale);
            st.l[g] *= corr;
#pragma unroll
            for (int c = 0; c < 4; ++c) st.acc[g][c] *= corr;
            st.m[g] = mn[g];
        }
    }
    uint32_t pa[G];  // fp16 pair: tokens r and r+4 of the half
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float off = -mn[g] * qk_scale;
        pa[g] = pack_p2(__builtin_amdgcn_exp2f(__builtin_fmaf(s[g][0], qk_scale, off)),
                        __builtin_amdgcn_exp2f(__builtin_fmaf(s[g][1], qk_scale, off)));
        st.l[g] = dot2(pa[g], kOnes, st.l[g]);  // l sums the fp16 probabilities PV uses
    }
    // Row r's pairs (the same in all 16 lanes of the row) to pbuf[8r + g];
    // every lane then reads each row's pairs back as one broadcast. The
    // wave's LDS operations run in order, so the previous half page's reads
    // are done before these writes land.
    if (j == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) pbuf[8 * r + g] = pa[g];
    }
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
        uint32_t pp[8];
        *reinterpret_cast<uint4 *>(pp) = reinterpret_cast<const uint4 *>(pbuf)[2 * rr];
        if (G > 4) *reinterpret_cast<uint4 *>(pp + 4) = reinterpret_cast<const uint4 *>(pbuf)[2 * rr + 1];
        const uint2 va = p.v[rr];
        const uint2 vb = p.v[rr + 4];
        const uint32_t v0 = (va.x & 0xffffu) | (vb.x << 16);
        const uint32_t v1 = (va.x >> 16) | (vb.x & 0xffff0000u);
        const uint32_t v2 = (va.y & 0xffffu) | (vb.y << 16);
        const uint32_t v3 = (va.y >> 16) | (vb.y & 0xffff0000u);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            st.acc[g][0] = dot2(pp[g], v0, st.acc[g][0]);
            st.acc[g][1] = dot2(pp[g], v1, st.acc[g][1]);
            st.acc[g][2] = dot2(pp[g], v2, st.acc[g][2]);
            st.acc[g][3] = dot2(pp[g], v3, st.acc[g][3]);
        }
    }
}

__device__ __forceinline__ const uint16_t *gate_of(const DecodeArgs &a, int b, int hq, int lane) {
    return a.gate ? a.gate + static_cast<int64_t>(b) * a.gate_stride + hq * kHeadDim + 4 * lane : nullptr;
}

// First page of workgroup w when P pages are shared by W workgroups.
// kFast: floor_muldiv's 32-bit division when the product fits, for the
// combine, which waits on these before its first loads; the decode kernel
// keeps the 64-bit form (the extra branch cost it registers: one wave per
// SIMD instead of two, C3 114 -> 144 us).
template <bool kFast = false>
__device__ __forceinline__ int wg_start(int w, int P, int W) {
    return kFast ? floor_muldiv(w, P, W) : static_cast<int>(static_cast<int64_t>(w) * P / W);
}

// The workgroup whose page range holds page p.
template <bool kFast = false>
__device__ __forceinline__ int wg_of_page(int p, int P, int W) {
    int w = kFast ? floor_muldiv(p, W, P) : static_cast<int>(static_cast<int64_t>(p) * W / P);
    while (w + 1 < W && wg_start<kFast>(w + 1, P, W) <= p) ++w;
    return w;
}

// The stream-K shape of a launch: P pages over W workgroups.  Fixed by the
// host for an ordinary call; for a launch recorded into a graph it is derived
// here from the step plan (the same rule the host applies), so a replay after
// the lengths grew still shares the right page count.
__device__ __forceinline__ void stream_k_shape(const DecodeArgs &a, int &P, int &W) {
    if (!a.dyn) {
        P = a.total_pages;
        W = a.n_wg;
        return;
    }
    P = ld_uniform(a.pre_seq + a.n_seqs);
    int w = a.split_tokens > 0 ? (P * kBlockTokens + a.split_tokens - 1) / a.split_tokens : a.n_wg;
    w = min(w, (P + a.min_pages - 1) / a.min_pages);
    W = max(1, min(w, a.n_wg));
}

// Pages of all sequences before sequence b.
__device__ __forceinline__ int seq_page_base(const DecodeArgs &a, int b, int npg) {
    return a.pre_seq ? a.pre_seq[b] : b * npg;
}

// Per-sequence facts for sequences b0 .. b0+63, one per lane, so a sequence
// switch costs v_readlane instead of a chain of dependent loads.
struct SeqWindow {
    int b0;
    int base, ctx, sid;  // this lane's sequence: first page, length, cache slot
};

__device__ __forceinline__ void load_window(SeqWindow &win, const DecodeArgs &a, int b0, int lane) {
    const int i = b0 + lane;
    const bool ok = i < a.n_seqs;
    const int npg_c = (a.ctx_len_const + 15) >> 4;
    win.b0 = b0;
    win.ctx = ok ? (a.ctx_lens ? a.ctx_lens[i] : a.ctx_len_const) : 0;
    win.base = ok ? (a.pre_seq ? a.pre_seq[i] : i * npg_c) : INT32_MAX;  // lanes past n_seqs: unused
    win.sid = (ok && a.table) ? a.seq_ids[i] : 0;
}

// A page of the workgroup's range: sequence b (index in the step), page pg of
// it.  Every field is wave-uniform.
struct Cursor {
    int b, pg, npg, ctx, base, sid;
    bool ok;
};

__device__ __forceinline__ Cursor seq_cursor(const SeqWindow &win, int b) {
    Cursor c;
    const int k = b - win.b0;
    c.b = b;
    c.pg = 0;
    c.ctx = __builtin_amdgcn_readlane(win.ctx, k);
    c.base = __builtin_amdgcn_readlane(win.base, k);
    c.sid = __builtin_amdgcn_readlane(win.sid, k);
    c.npg = (c.ctx + 15) >> 4;
    c.ok = true;
    return c;
}

// ---- Stream-K decode with QK on the matrix cores ----
//
// One wave per kv head walks every page of the workgroup's share (16 token
// rows a step), so no waves merge inside the workgroup; at a sequence end the
// wave writes its head's output or the share's partial itself.
//   QK: S^T = K Q^T on v_mfma_f32_16x16x32_f16, the page's 16 rows as the A
//       operand and the G query rows as columns 0..G-1 of B (the others
//       zero).  The k order inside the product is free as long as A and B
//       agree, so lane group g's k-step s covers dims 64g + 8s .. +7: each
//       lane loads its row's 128 contiguous bytes, dims 64g .. 64g+63.
//   softmax: on the C layout (lane: head column l%16, rows 4(l/16)..+3);
//       the column max over the four lane groups by permlane swaps.
//   PV: the fp16 probability pairs go through 64 dwords of LDS per wave
//       ([token pair][head]) to every lane, which folds token pairs with
//       v_dot2_f32_f16 into dims 4l..4l+3 of every head (the whole-sequence
//       form's PV, over sixteen rows).
// Measured against the previous stream-K kernel (eight waves on half pages,
// QK and PV on the VALU), config 3 went from 130.8 to 120.0 us per call and
// ctx 8192 from 203 to 188: the VALU work per page of a kv head roughly
// halves, and one workgroup of four waves per CU (one wave per SIMD) beats
// two (126 us).
constexpr int kMfmaWaves = kDecodeHeadsPerWg;  // waves (kv heads) per workgroup, at most

struct Page {
    uint4 k[8];   // this lane's row (l%16), dims 64(l/16) .. +63
    uint2 v[16];  // rows 0..15, dims 4l .. 4l+3
};

__device__ __forceinline__ void load_page(Page &p, const char *kb, const char *vb, int lim, bool on, uint32_t koff,
                                          uint32_t voff, int row_bytes) {
    const uint32_t n = on ? static_cast<uint32_t>(lim * row_bytes) : 0u;
    const auto rk = page_rsrc(kb, n), rv = page_rsrc(vb, n);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        const auto x = __builtin_amdgcn_raw_buffer_load_b128(rk, koff + 16 * s, 0, 0);
        p.k[s] = make_uint4(x[0], x[1], x[2], x[3]);
    }
#pragma unroll
    for (int t = 0; t < kBlockTokens; ++t) {
        const auto x = __builtin_amdgcn_raw_buffer_load_b64(rv, voff + t * row_bytes, 0, 0);
        p.v[t] = make_uint2(x[0], x[1]);
    }
}

// m: the running max of this lane's head column (raw scores), l: the fp16
// probabilities of this lane's four rows summed, acc: dims 4l..4l+3 of every
// head of the group.
template <int G>
struct MfmaState {
    float m, l, acc[G][4];
};

template <int G>
__device__ __forceinline__ void reset(MfmaState<G> &st) {
    st.m = -INFINITY;
    st.l = 0.0f;
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int c = 0; c < 4; ++c) st.acc[g][c] = 0.0f;
}

// Fold a page into the state; rows >= lim are masked (lim >= 1).  qb: the B
// operand (this lane's column: query head l%16, zero past G).
template <int G>
__device__ __forceinline__ void compute_page(MfmaState<G> &st, const Page &p, const uint4 (&qb)[8], int lane, int lim,
                                             uint32_t *pbuf) {
    using half8 = _Float16 __attribute__((ext_vector_type(8)));
    const float qk_scale = kLog2e / 16.0f;
    const uint32_t kOnes = 0x3c003c00u;
    const int col = lane & 15;
    const int grp = lane >> 4;
    float4_t s = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < 8; ++k)
        s = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, p.k[k]), __builtin_bit_cast(half8, qb[k]),
                                                  s, 0, 0, 0);
    if (lim < kBlockTokens) {  // the sequence's last page (wave-uniform)
#pragma unroll
        for (int i = 0; i < 4; ++i) s[i] = (4 * grp + i < lim) ? s[i] : -INFINITY;
    }
    const float bm = group4_max(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])));
    const float mn = fmaxf(st.m, bm);
    // Rescale only when some head's max grew (wave-uniform).
    if (__builtin_amdgcn_ballot_w64(col < G && mn > st.m)) {
        const float corr = __builtin_amdgcn_exp2f((st.m - mn) * qk_scale);
        st.l *= corr;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float cg = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, corr), g));
#pragma unroll
            for (int c = 0; c < 4; ++c) st.acc[g][c] *= cg;
        }
        st.m = mn;
    }
    const float off = -st.m * qk_scale;
    const uint32_t pk0 = pack_p2(__builtin_amdgcn_exp2f(__builtin_fmaf(s[0], qk_scale, off)),
                                 __builtin_amdgcn_exp2f(__builtin_fmaf(s[1], qk_scale, off)));
    const uint32_t pk1 = pack_p2(__builtin_amdgcn_exp2f(__builtin_fmaf(s[2], qk_scale, off)),
                                 __builtin_amdgcn_exp2f(__builtin_fmaf(s[3], qk_scale, off)));
    st.l = dot2(pk1, kOnes, dot2(pk0, kOnes, st.l));  // l sums the fp16 probabilities PV uses
    // Rows 4grp, 4grp+1 are pair 2grp; rows 4grp+2, 4grp+3 pair 2grp+1.  The
    // wave's LDS operations run in order, so the previous page's reads are
    // done before these writes land.
    if (col < 8) {
        pbuf[(2 * grp) * 8 + col] = pk0;
        pbuf[(2 * grp + 1) * 8 + col] = pk1;
    }
#pragma unroll
    for (int t = 0; t < kBlockTokens / 2; ++t) {
        uint32_t pp[8];
        *reinterpret_cast<uint4 *>(pp) = reinterpret_cast<const uint4 *>(pbuf)[2 * t];
        if (G > 4) *reinterpret_cast<uint4 *>(pp + 4) = reinterpret_cast<const uint4 *>(pbuf)[2 * t + 1];
        const uint2 va = p.v[2 * t];
        const uint2 vb = p.v[2 * t + 1];
        const uint32_t v0 = (va.x & 0xffffu) | (vb.x << 16);
        const uint32_t v1 = (va.x >> 16) | (vb.x & 0xffff0000u);
        const uint32_t v2 = (va.y & 0xffffu) | (vb.y << 16);
        const uint32_t v3 = (va.y >> 16) | (vb.y & 0xffff0000u);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            st.acc[g][0] = dot2(pp[g], v0, st.acc[g][0]);
            st.acc[g][1] = dot2(pp[g], v1, st.acc[g][1]);
            st.acc[g][2] = dot2(pp[g], v2, st.acc[g][2]);
            st.acc[g][3] = dot2(pp[g], v3, st.acc[g][3]);
        }
    }
}

template <int G>
__global__ __launch_bounds__(64 * kMfmaWaves) void decode_mfma_kernel(DecodeArgs a) {
    // Query rows of the range's first kQSlots sequences, per wave (its kv
    // head); later ones are reloaded kQSlots at a time.
    constexpr int kQSlots = 4;
    __shared__ uint4 q_lds[kMfmaWaves * kQSlots * G * 32];
    __shared__ uint32_t p_lds[kMfmaWaves * 64];
    __shared__ uint64_t tl_t[2];
    if (a.timeline && threadIdx.x == 0) tl_t[0] = __builtin_amdgcn_s_memrealtime();

    const int w = blockIdx.x;
    int P, W;
    stream_k_shape(a, P, W);
    if (w >= W) return;
    const int p_begin = wg_start(w, P, W);
    const int p_end = wg_start(w + 1, P, W);
    if (p_begin >= p_end) return;
    const int hkv = a.num_kv_heads;
    const int nh = a.num_heads;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = __builtin_amdgcn_readfirstlane(blockIdx.y * (blockDim.x >> 6) + wave);
    const int lane = threadIdx.x & 63;
    const int col = lane & 15;
    const int grp = lane >> 4;
    const int row_bytes = hkv * kHeadDim * 2;
    const size_t page_bytes = static_cast<size_t>(kBlockTokens) * row_bytes;
    const uint32_t koff = col * row_bytes + 128 * grp;
    const uint32_t voff = 8 * lane;

    int b0, b1;
    if (a.pre_seq) {
        b0 = 0;
        b1 = 0;
        for (int c0 = 0; c0 < a.n_seqs; c0 += 64) {
            const int i = c0 + lane;
            const int end = i < a.n_seqs ? a.pre_seq[i + 1] : INT32_MAX;
            const uint64_t m0 = __ballot(end <= p_begin);
            const uint64_t m1 = __ballot(end <= p_end - 1);
            b0 += __popcll(m0);
            b1 += __popcll(m1);
            if (m1 != ~0ull) break;
        }
    } else {
        const int npg_c = (a.ctx_len_const + 15) >> 4;
        b0 = p_begin / npg_c;
        b1 = (p_end - 1) / npg_c;
    }
    b0 = __builtin_amdgcn_readfirstlane(b0);
    b1 = __builtin_amdgcn_readfirstlane(b1);
    SeqWindow win;
    load_window(win, a, b0, lane);

    // This wave's query rows of sequences b .. b+kQSlots-1 (up to b1) into its
    // own slots; q_hi is the last sequence loaded.  Only this wave reads them.
    uint4 *q_head = q_lds + wave * kQSlots * G * 32;
    int q_hi = 0;
    auto load_q = [&](int b) {
        q_hi = b + kQSlots - 1;
        const int n = min(kQSlots, b1 - b + 1);
        for (int k = 0; k < n; ++k) {
            const uint16_t *qb =
                a.q + (static_cast<size_t>(b + k) * nh + static_cast<size_t>(h) * G) * kHeadDim;
            const int slot = (b + k - b0) % kQSlots;
#pragma unroll
            for (int i = lane; i < G * 32; i += 64) q_head[slot * G * 32 + i] = ld16(qb + 8 * i);
        }
    };
    uint4 qb[8];
    auto fill_q = [&](int b) {
        const uint4 *qs = q_head + ((b - b0) % kQSlots) * G * 32;
#pragma unroll
        for (int k = 0; k < 8; ++k) qb[k] = col < G ? qs[col * 32 + 8 * grp + k] : make_uint4(0, 0, 0, 0);
    };
    load_q(b0);
    fill_q(b0);

    const char *kpool = reinterpret_cast<const char *>(a.k_pool) + h * kHeadDim * 2;
    const char *vpool = reinterpret_cast<const char *>(a.v_pool) + h * kHeadDim * 2;
    auto page_id = [&](const Cursor &c) -> int {
        return a.table ? ld_uniform(a.table + static_cast<size_t>(c.sid) * a.table_stride + c.pg) : c.pg;
    };
    auto page_ofs = [&](const Cursor &c, int id) -> size_t {
        const size_t seq = a.table ? 0 : static_cast<size_t>(c.b) * a.seq_stride * 2;
        return seq + static_cast<size_t>(id) * page_bytes;
    };
    auto lim_of = [](const Cursor &c) { return min(kBlockTokens, c.ctx - c.pg * kBlockTokens); };
    auto next = [&](Cursor c) -> Cursor {
        if (!c.ok) return c;
        if (c.base + c.pg + 1 >= p_end) {
            c.ok = false;
            return c;
        }
        if (c.pg + 1 < c.npg) {
            ++c.pg;
            return c;
        }
        int b = c.b;
        do {
            ++b;
            if (b - win.b0 >= 64) load_window(win, a, b, lane);
            c = seq_cursor(win, b);
        } while (c.npg == 0);
        return c;
    };

    MfmaState<G> st;
    reset(st);
    // End of sequence c.b in this range: the wave writes its head's output
    // (whole sequence) or this range's partial, then loads the next rows.
    auto finish = [&](const Cursor &c, int b_next) {
        const float qk_scale = kLog2e / 16.0f;
        const float lt = group4_sum(st.l);  // the four lane groups hold disjoint rows
        const bool whole = c.base >= p_begin && c.base + c.npg <= p_end;
        const int slot = 2 * w + (c.b == b0 ? 0 : 1);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float mg = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, st.m), g));
            const float lg = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lt), g));
            if (whole) {
                const float inv = 1.0f / lg;
                *reinterpret_cast<uint2 *>(a.out + (static_cast<size_t>(c.b) * nh + h * G + g) * kHeadDim +
                                           4 * lane) =
                    out_fp16x4(st.acc[g][0] * inv, st.acc[g][1] * inv, st.acc[g][2] * inv, st.acc[g][3] * inv,
                               gate_of(a, c.b, h * G + g, lane));
            } else {
                const size_t u = (static_cast<size_t>(slot) * hkv + h) * G + g;
                *reinterpret_cast<float4 *>(a.ws_acc + u * kHeadDim + 4 * lane) =
                    make_float4(st.acc[g][0], st.acc[g][1], st.acc[g][2], st.acc[g][3]);
                if (lane == 0) {
                    a.ws_ml[u * 2] = mg * qk_scale;  // log2 units
                    a.ws_ml[u * 2 + 1] = lg;
                }
            }
        }
        if (b_next > q_hi) load_q(b_next);
        reset(st);
    };

    // Two page buffers: while one is folded in, the next page is in flight.
    Page A, B;
    Cursor c0 = seq_cursor(win, b0);
    c0.pg = p_begin - c0.base;
    Cursor cq[2];
    cq[0] = c0;
    cq[1] = next(c0);
    int id_last = 0;
    {
        const int id = page_id(cq[0]);
        load_page(A, kpool + page_ofs(cq[0], id), vpool + page_ofs(cq[0], id), lim_of(cq[0]), true, koff, voff,
                  row_bytes);
        id_last = cq[1].ok ? page_id(cq[1]) : id;
    }
    if (a.timeline && threadIdx.x == 0) tl_t[1] = __builtin_amdgcn_s_memrealtime();
    uint32_t *pbuf = p_lds + 64 * wave;
    auto step = [&](Page &cr, Page &nr) -> bool {
        const Cursor cl = cq[1];
        const Cursor cn = next(cl);
        const int id_n = cn.ok ? page_id(cn) : id_last;
        load_page(nr, kpool + page_ofs(cl, id_last), vpool + page_ofs(cl, id_last), lim_of(cl), cl.ok, koff, voff,
                  row_bytes);
        __builtin_amdgcn_sched_barrier(0);
        const Cursor cur = cq[0];
        compute_page<G>(st, cr, qb, lane, lim_of(cur), pbuf);
        if (!cq[1].ok || cq[1].b != cur.b) {
            finish(cur, cq[1].ok ? cq[1].b : 0);
            if (cq[1].ok) fill_q(cq[1].b);
        }
        cq[0] = cq[1];
        cq[1] = cn;
        id_last = id_n;
        return cq[0].ok;
    };
    while (step(A, B) && step(B, A)) {
    }
    if (a.timeline && lane == 0) {
        // Per wave: entry, first K/V issue, end of its walk (100 MHz
        // s_memrealtime ticks), then the XCD (high word) and the share's
        // pages; eight records per workgroup row, zero for the waves this
        // workgroup does not have.
        const uint32_t xcc = xcc_id();
        uint64_t *rec = a.timeline + ((static_cast<size_t>(w) * gridDim.y + blockIdx.y) * 8 + wave) * kTimelineWords;
        rec[0] = tl_t[0];
        rec[1] = tl_t[1];
        rec[2] = __builtin_amdgcn_s_memrealtime();
        rec[3] = (static_cast<uint64_t>(xcc & 0xf) << 32) | static_cast<uint32_t>(p_end - p_begin);
        for (int v = wave + (blockDim.x >> 6); v < 8; v += blockDim.x >> 6)
            for (int i = 0; i < kTimelineWords; ++i)
                a.timeline[((static_cast<size_t>(w) * gridDim.y + blockIdx.y) * 8 + v) * kTimelineWords + i] = 0;
    }
}

// Merge the partials of one (sequence, kv head, query head of the group)
// whose pages were cut across workgroups: 64 lanes x 4 dims per wave.  A
// separate launch (stream order makes the partials visible), so no
// cross-workgroup fences are needed: an agent-scope release on every decode
// workgroup costs an L2 writeback per workgroup on multi-XCD parts.  The
// (m, l) pairs and acc rows of up to kChunk partials are all requested before
// any is used, so a sequence cut into at most kChunk pieces costs one memory
// round trip when the host passes each sequence's first piece and piece
// count with the launch arguments (DecodeArgs::crec), two otherwise (its
// length, then its partials).  A sequence cut into more pieces (one long
// sequence over every CU) has its chunks dealt to the four waves of its
// workgroup, which merge through LDS.
//
// kHeads (the host has shown that no sequence of the launch has more than
// kChunk pieces): a workgroup per (sequence, kv head), its G waves one
// query head each, where the general form has a workgroup of four waves per
// query head.
constexpr int kCombineWaves = 4;
template <int G, bool kHeads = false>
__global__ __launch_bounds__(64 * (kHeads ? G : kCombineWaves)) void combine_kernel(DecodeArgs a) {
    constexpr int kChunk = kCombineChunk;
    __shared__ float4 w_acc[kCombineWaves * 64];
    __shared__ float w_ml[kCombineWaves * 2];
    const int u = blockIdx.x;
    const int g = kHeads ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) : static_cast<int>(blockIdx.y);
    const int hkv = a.num_kv_heads;
    const int b = u / hkv;
    const int h = u - b * hkv;
    const int lane = threadIdx.x & 63;
    const int wave = kHeads ? 0 : __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // Partial i comes from workgroup w0 + i: slot 2w when the sequence began
    // at or before that workgroup's range, else 2w+1.  Only w0's range can
    // begin after the sequence's first page, so one division settles every
    // slot (one per piece kept the pieces' loads from going out together).
    int w0, n, slot0;
    if (a.n_crec > 0) {  // the host's figures, with the kernel arguments
        w0 = a.crec[b];
        if (w0 < 0) return;  // one workgroup covered the sequence and wrote it
        n = a.crec_n[b] >> 1;
        slot0 = 2 * w0 + (a.crec_n[b] & 1);
    } else {
        int P, W;
        stream_k_shape(a, P, W);
        const int ctx = a.ctx_lens ? a.ctx_lens[b] : a.ctx_len_const;
        const int npg = (ctx + 15) >> 4;
        if (npg == 0) return;
        const int first = seq_page_base(a, b, npg);
        w0 = wg_of_page<true>(first, P, W);
        const int w1 = wg_of_page<true>(first + npg - 1, P, W);
        if (w0 == w1) return;  // one workgroup covered the sequence and wrote it
        n = w1 - w0 + 1;
        slot0 = 2 * w0 + (first <= wg_start<true>(w0, P, W) ? 0 : 1);
    }
    const int nw = kHeads ? 1 : blockDim.x >> 6;  // 1 when the host knows no sequence has more than kChunk pieces
    const bool multi = n > kChunk;   // uniform over the workgroup
    if (!multi && wave != 0) return;
    auto row_of = [&](int i) -> size_t {
        const int slot = i == 0 ? slot0 : 2 * (w0 + i);
        return (static_cast<size_t>(slot) * hkv + h) * G + g;
    };
    // Running merge over this wave's chunks: (big, lt, at) is the merge of
    // the chunks so far (big = -inf, lt = 0 before any).
    float big = -INFINITY, lt = 0.0f;
    float4 at = make_float4(0.f, 0.f, 0.f, 0.f);
    const int step = multi ? nw * kChunk : kChunk;
    for (int c0 = (multi ? wave : 0) * kChunk; c0 < n; c0 += step) {
        const int cnt = min(kChunk, n - c0);
        float2 ml = make_float2(-INFINITY, 0.0f);
        if (lane < cnt) ml = *reinterpret_cast<const float2 *>(a.ws_ml + row_of(c0 + lane) * 2);
        float4 v[kChunk];
#pragma unroll
        for (int k = 0; k < kChunk; ++k)
            v[k] = k < cnt ? reinterpret_cast<const float4 *>(a.ws_acc + row_of(c0 + k) * kHeadDim)[lane]
                           : make_float4(0.f, 0.f, 0.f, 0.f);
        float cm = ml.x;
#pragma unroll
        for (int o = 8; o >= 1; o >>= 1) cm = fmaxf(cm, __shfl_xor(cm, o));
        cm = __shfl(cm, 0);
        const float nb = fmaxf(big, cm);
        const float keep = __builtin_amdgcn_exp2f(big - nb);  // 0 on the first chunk
        const float ci = lane < cnt ? __builtin_amdgcn_exp2f(ml.x - nb) : 0.0f;
        float ls = ci * ml.y;
#pragma unroll
        for (int o = 8; o >= 1; o >>= 1) ls += __shfl_xor(ls, o);
        lt = lt * keep + __shfl(ls, 0);
        at.x *= keep;
        at.y *= keep;
        at.z *= keep;
        at.w *= keep;
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            const float ck = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ci), k));
            at.x += ck * v[k].x;
            at.y += ck * v[k].y;
            at.z += ck * v[k].z;
            at.w += ck * v[k].w;
        }
        big = nb;
    }
    if (multi && nw > 1) {
        // Wave 0 always holds a chunk; a wave without one (fewer than nw
        // chunks) keeps big = -inf and weighs 0.
        w_acc[wave * 64 + lane] = at;
        if (lane == 0) {
            w_ml[wave * 2] = big;
            w_ml[wave * 2 + 1] = lt;
        }
        __syncthreads();
        if (wave != 0) return;
        float mm = -INFINITY;
#pragma unroll
        for (int v = 0; v < kCombineWaves; ++v)
            if (v < nw) mm = fmaxf(mm, w_ml[v * 2]);
        lt = 0.0f;
        at = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int v = 0; v < kCombineWaves; ++v) {
            if (v >= nw) break;
            const float c = __builtin_amdgcn_exp2f(w_ml[v * 2] - mm);  // 0 for a wave without chunks
            const float4 x = w_acc[v * 64 + lane];
            lt += w_ml[v * 2 + 1] * c;
            at.x += x.x * c;
            at.y += x.y * c;
            at.z += x.z * c;
            at.w += x.w * c;
        }
    }
    const float inv = 1.0f / lt;
    *reinterpret_cast<uint2 *>(a.out + (static_cast<size_t>(b) * a.num_heads + h * G + g) * kHeadDim +
                               4 * lane) =
        out_fp16x4(at.x * inv, at.y * inv, at.z * inv, at.w * inv, gate_of(a, b, h * G + g, lane));
}

// Whole-sequence decode for steps of short sequences: a workgroup walks one
// sequence for one kv head alone, its eight waves taking half pages w, w+8,
// w+16, ... (8 token rows each, up to three in flight per wave); the waves
// merge through LDS and write the output.  No partials and no combine
// launch: a step of a few pages per sequence is bound by its launches, its
// memory round trips and the VALU work of each CU, not by bandwidth.  The
// G query heads of a kv head are split among a.whole workgroups of GP heads
// each (GP = G / a.whole), so a step of few sequences still spreads its
// arithmetic over many CUs; workgroup w serves unit u = (sequence, kv head)
// and head group z with w % 8 == u % 8, so the groups of one unit run on one
// XCD and their reads of its K/V after the first come from that XCD's L2.
// Correct for any length (a recorded launch keeps this form when the lengths
// grow), fast while every sequence is a few hundred rows.
//
// kFused: the step's append runs in the same launch (DecodeArgs::fused).
// Half-wave k of the workgroup normalises and rotates query row k (k < GP),
// the kv head's new K row (k = GP) or carries its V row (k = GP + 1), with
// the append kernel's arithmetic (norm_rope_apply: the same bits); the walk
// covers the ctx - 1 cached rows and the new token enters the merge as one
// more partial (its score from the rounded K row, probability 1, its V row).
template <int GP, bool kFused>
__global__ __launch_bounds__(64 * kWholeWaves) void whole_kernel(DecodeArgs a) {
    __shared__ uint4 q_lds[GP * 32];
    __shared__ uint4 kv_new[kFused ? 64 : 1];  // fused: the new K (normalised) and V rows
    __shared__ uint32_t p_lds[kWholeWaves * 32];
    __shared__ float4 mrg_acc[kWholeWaves * GP * 64];
    __shared__ float mrg_ml[(kWholeWaves + 1) * GP * 2];
    __shared__ uint64_t tl_t[2];  // timeline: entry and first-issue times
    if (a.timeline && threadIdx.x == 0) tl_t[0] = __builtin_amdgcn_s_memrealtime();
    const int hkv = a.num_kv_heads;
    const int nh = a.num_heads;
    const int n_grp = a.whole;
    const int w = blockIdx.x;
    const int rest = w >> 3;
    const int z = rest % n_grp;
    const int u = (rest / n_grp) * 8 + (w & 7);
    if (u >= a.n_seqs * hkv) return;  // the grid rounds the units up to 8
    const int b = u / hkv;
    const int h = u - b * hkv;
    const int hq0 = h * (nh / hkv) + z * GP;  // this workgroup's first query head
    // First round: every request that needs only the kernel arguments (the
    // plan's page ids, this workgroup's q rows; fused: the new K and V rows
    // and the norm weights) goes out before the scalar loads of the length,
    // the sequence id and the position.  A wait for one scalar load waits
    // for every scalar load in flight, so an argument fetched after those
    // loads would hold back the requests that need it until they had
    // arrived.  The first K/V loads then wait for one round trip (the length
    // and the page ids), not two (the table row needs the sequence id).
    // Page ids: lane k holds page k's, for the sequence's first 64 pages;
    // past the 64th they come from the table.
    static_assert(kPlanPages == 64, "one plan page id per lane");
    const int lane = threadIdx.x & 63;
    // A buffer load over the sequence's 64 ids (an empty range without a
    // plan: zeros, no memory touched), so the compiler neither waits on a
    // branch nor folds it into the table read below.
    const int32_t *pid_p = a.plan_pages;
    const auto pid_rs = ro_rsrc(pid_p ? pid_p + static_cast<size_t>(b) * kPlanPages : nullptr,
                                pid_p ? kPlanPages * 4u : 0u);
    const int plan_ids = static_cast<int>(__builtin_amdgcn_raw_buffer_load_b32(pid_rs, 4 * lane, 0, 0));
    const int qi = threadIdx.x;
    const int hw = threadIdx.x >> 5;  // fused: the half-wave's row
    const int l32 = threadIdx.x & 31;
    uint4 qin = make_uint4(0, 0, 0, 0);
    uint4 win = make_uint4(0, 0, 0, 0);
    if constexpr (kFused) {
        const AppendArgs &ap = a.app;
        const uint16_t *src = hw < GP    ? ap.q + (static_cast<size_t>(b) * nh + hq0 + hw) * kHeadDim
                              : hw == GP ? ap.k + (static_cast<size_t>(b) * hkv + h) * kHeadDim
                                         : ap.v + (static_cast<size_t>(b) * hkv + h) * kHeadDim;
        if (hw <= GP + 1) qin = ld16(src + 8 * l32);
        win = ld16((hw < GP ? ap.q_w : ap.k_w) + 8 * l32);
    } else {
        if (qi < GP * 32) qin = ld16(a.q + (static_cast<size_t>(b) * nh + hq0) * kHeadDim + 8 * qi);
    }
    const int32_t *ctx_p = a.ctx_lens, *sid_p = a.seq_ids, *tab = a.table;
    const int32_t *pos_p = kFused ? a.app.tok_pos : nullptr;
    const int half_rot = kFused ? a.app.half_rot : 0;  // addresses this position's cos/sin
    asm volatile("" ::"s"(ctx_p), "s"(sid_p), "s"(tab), "s"(pos_p), "s"(half_rot));
    __builtin_amdgcn_sched_barrier(0);
    // The length, the sequence id and the position are requested together
    // (no branch on the length between them); an empty sequence walks
    // nothing and writes no output.
    const int ctx = ctx_p ? ld_uniform(ctx_p + b) : a.ctx_len_const;
    const int sid = tab ? ld_uniform(sid_p + b) : 0;
    const int pos = kFused ? ld_uniform(pos_p + b) : 0;
    // Taken in here, together: kernel arguments fetched after this point
    // then wait only for themselves.
    asm volatile("" ::"s"(ctx), "s"(sid), "s"(pos));
    __builtin_amdgcn_sched_barrier(0);
    const int walk = kFused ? ctx - 1 : ctx;  // cached rows the waves walk
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane >> 4;
    const int j = lane & 15;
    const int row_bytes = hkv * kHeadDim * 2;
    const size_t page_bytes = static_cast<size_t>(kBlockTokens) * row_bytes;
    const size_t seq_ofs = tab ? 0 : static_cast<size_t>(b) * a.seq_stride * 2;
    const char *kpool = reinterpret_cast<const char *>(a.k_pool) + seq_ofs + h * kHeadDim * 2;
    const char *vpool = reinterpret_cast<const char *>(a.v_pool) + seq_ofs + h * kHeadDim * 2;
    // Without the plan's ids (a contiguous cache has none to read), lane k
    // reads page k's from the table row.
    const int32_t *row = tab ? tab + static_cast<size_t>(sid) * a.table_stride : nullptr;
    const int npg = (max(ctx, 0) + kBlockTokens - 1) / kBlockTokens;
    const int ids = pid_p ? plan_ids : (row && lane < npg) ? row[lane] : 0;
    // Fused: this position's cos/sin, requested after the position arrives
    // and waited for only where the rows are normalised (after the first
    // K/V loads go out).
    NormRopeIn nin{};
    if constexpr (kFused) {
        const AppendArgs &ap = a.app;
        nin.w = win;
        rope_in_flat(nin, hw < GP ? ap.q_w : ap.k_w, ap.cos_tab + static_cast<size_t>(pos) * half_rot,
                     ap.sin_tab + static_cast<size_t>(pos) * half_rot, half_rot, l32);
    }

    const int n_hp = (max(walk, 0) + kHalf - 1) / kHalf;
    const int n_i = wave < n_hp ? (n_hp - wave + kWholeWaves - 1) / kWholeWaves : 0;
    const uint32_t koff = r * row_bytes + 16 * j;
    const uint32_t voff = 8 * lane;
    // Issue this wave's i-th half page into p (a no-op load past the list).
    // Block id of page pg (wave-uniform): the first 64 from the lanes' ids,
    // later ones from the table row by a vector load, which the compiler
    // keeps inside its branch (a scalar load it would issue for every page,
    // and the first K/V loads would wait for it).
    auto page_of = [&](int pg) -> int {
        if (!row) return pg;
        if (pg < 64) return __builtin_amdgcn_readlane(ids, pg);
        return __builtin_amdgcn_readfirstlane(row[pg]);
    };
    auto issue = [&](HalfPage &p, int i) {
        const bool on = i < n_i;
        const int hp = on ? wave + kWholeWaves * i : 0;
        const int pg = hp >> 1;
        const int id = page_of(pg);
        const size_t ofs = static_cast<size_t>(id) * page_bytes + static_cast<size_t>(hp & 1) * kHalf * row_bytes;
        load_half(p, kpool + ofs, vpool + ofs, min(kHalf, walk - hp * kHalf), on, koff, voff, row_bytes);
    };
    constexpr int kStages = GP <= 6 ? 3 : 2;
    HalfPage A, B, C;
    issue(A, 0);
    if (kStages == 3) issue(B, 1);
    if (a.timeline && threadIdx.x == 0) tl_t[1] = __builtin_amdgcn_s_memrealtime();
    if constexpr (kFused) {
        const AppendArgs &ap = a.app;
        // Every half-wave runs the arithmetic (the unused ones on zeros) so
        // the butterfly's lanes are all active; the results are kept by row.
        const uint4 y = norm_rope_apply<32>(qin, nin, ap.half_rot, ap.eps, l32);
        if (hw < GP) {
            q_lds[hw * 32 + l32] = y;
            st16(ap.q + (static_cast<size_t>(b) * nh + hq0 + hw) * kHeadDim + 8 * l32, y);
        } else if (hw == GP) {
            kv_new[l32] = y;
        } else if (hw == GP + 1) {
            kv_new[32 + l32] = qin;
        }
        // The first head group of (b, h) writes the new rows into slot ctx - 1.
        const int slot = ctx - 1;
        const int pg = max(slot, 0) >> 4;
        const int id = page_of(pg);
        if (z == 0 && ctx > 0 && (hw == GP || hw == GP + 1)) {
            const size_t at = ((static_cast<size_t>(id) * kBlockTokens + (slot & 15)) * hkv + h) * kHeadDim + 8 * l32;
            st16((hw == GP ? ap.k_pool : ap.v_pool) + at, hw == GP ? y : qin);
        }
    } else {
        if (qi < GP * 32) q_lds[qi] = qin;
    }
    __syncthreads();
    uint4 qv[GP][2];
#pragma unroll
    for (int g = 0; g < GP; ++g) {
        qv[g][0] = q_lds[g * 32 + j];
        qv[g][1] = q_lds[g * 32 + 16 + j];
    }

    WaveState<GP> st;
    reset(st);
    int i = 0;  // the half page folded in next
    auto step = [&](HalfPage &cr, HalfPage &nr) -> bool {
        issue(nr, i + kStages - 1);
        __builtin_amdgcn_sched_barrier(0);
        if (i < n_i) {
            compute_half<GP>(st, cr, qv, r, j, min(kHalf, walk - (wave + kWholeWaves * i) * kHalf),
                             p_lds + 32 * wave);
        } else {
            consume(cr);
        }
        ++i;
        return i < n_i;
    };
    if constexpr (kStages == 3) {
        while (step(A, C) && step(B, A) && step(C, B)) {
        }
    } else {
        while (step(A, B) && step(B, A)) {
        }
    }
    if (a.timeline && lane == 0) {
        // As decode_mfma_kernel's records, one row per workgroup of unit
        // u's group z: [n_units * n_grp][1][8 waves].
        const uint32_t xcc = xcc_id();
        uint64_t *rec =
            a.timeline + ((static_cast<size_t>(u) * n_grp + z) * kWholeWaves + wave) * kTimelineWords;
        rec[0] = tl_t[0];
        rec[1] = tl_t[1];
        rec[2] = __builtin_amdgcn_s_memrealtime();
        rec[3] = (static_cast<uint64_t>(xcc & 0xf) << 32) | static_cast<uint32_t>(npg);
    }

    // Merge the eight waves: each leaves (m, l, acc) in LDS; thread
    // (g, lane) merges head g's four dims 4*lane..4*lane+3.  A wave that had
    // no half page left m = -inf, l = acc = 0 and weighs nothing.  Fused:
    // wave g < GP adds head g's score of the new token as partial 8 (its V
    // row is read from LDS at the merge).
    const float qk_scale = kLog2e / 16.0f;
    if constexpr (kFused) {
        if (wave < GP) {
            const uint2 qq = reinterpret_cast<const uint2 *>(q_lds + wave * 32)[lane];
            const uint2 kk = reinterpret_cast<const uint2 *>(kv_new)[lane];
            float sc = dot2(qq.y, kk.y, dot2(qq.x, kk.x, 0.0f));
            sc = row16_sum(sc);
            sc += __shfl_xor(sc, 16);
            sc += __shfl_xor(sc, 32);
            if (lane == 0) {
                mrg_ml[(kWholeWaves * GP + wave) * 2] = sc;
                mrg_ml[(kWholeWaves * GP + wave) * 2 + 1] = 1.0f;
            }
        }
    }
#pragma unroll
    for (int g = 0; g < GP; ++g) {
        float lt = st.l[g];  // the four rows hold disjoint tokens
        lt += __shfl_xor(lt, 16);
        lt += __shfl_xor(lt, 32);
        mrg_acc[(wave * GP + g) * 64 + lane] = make_float4(st.acc[g][0], st.acc[g][1], st.acc[g][2], st.acc[g][3]);
        if (lane == 0) {
            mrg_ml[(wave * GP + g) * 2] = st.m[g];
            mrg_ml[(wave * GP + g) * 2 + 1] = lt;
        }
    }
    __syncthreads();
    if (ctx > 0 && qi < GP * 64) {
        const int g = qi >> 6;
        float mm = -INFINITY;
        constexpr int kParts = kFused ? kWholeWaves + 1 : kWholeWaves;
#pragma unroll
        for (int v = 0; v < kParts; ++v) mm = fmaxf(mm, mrg_ml[(v * GP + g) * 2]);
        float l = 0.0f;
        float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int v = 0; v < kParts; ++v) {
            const float c = __builtin_amdgcn_exp2f((mrg_ml[(v * GP + g) * 2] - mm) * qk_scale);
            float4 x;
            if (v < kWholeWaves) {
                x = mrg_acc[(v * GP + g) * 64 + lane];
            } else {
                const uint2 vv = reinterpret_cast<const uint2 *>(kv_new + 32)[lane];
                x = make_float4(lo_f(vv.x), hi_f(vv.x), lo_f(vv.y), hi_f(vv.y));
            }
            l += mrg_ml[(v * GP + g) * 2 + 1] * c;
            o.x += x.x * c;
            o.y += x.y * c;
            o.z += x.z * c;
            o.w += x.w * c;
        }
        const float inv = 1.0f / l;
        *reinterpret_cast<uint2 *>(a.out + (static_cast<size_t>(b) * nh + hq0 + g) * kHeadDim + 4 * lane) =
            out_fp16x4(o.x * inv, o.y * inv, o.z * inv, o.w * inv, gate_of(a, b, hq0 + g, lane));
    }
}

// The caller's timing events around the decode kernel itself (if any).
hipError_t mark(hipEvent_t ev, hipStream_t s) { return ev ? hipEventRecord(ev, s) : hipSuccess; }

template <int GP>
hipError_t launch_whole(const DecodeArgs &a, hipStream_t s) {
    const int units8 = (a.n_seqs * a.num_kv_heads + 7) / 8;
    const dim3 grid(units8 * 8 * a.whole), block(64 * kWholeWaves);
    hipError_t e = mark(a.ev_before, s);
    if (e != hipSuccess) return e;
    if (a.fused)
        hipLaunchKernelGGL((whole_kernel<GP, true>), grid, block, 0, s, a);
    else
        hipLaunchKernelGGL((whole_kernel<GP, false>), grid, block, 0, s, a);
    e = hipGetLastError();
    return e != hipSuccess ? e : mark(a.ev_after, s);
}

template <int G>
hipError_t launch_g(const DecodeArgs &a, hipStream_t s) {
    // Kv heads (one wave each) per workgroup: all of them up to kMfmaWaves,
    // else the largest divisor of Hkv that is at most that; grid rows split
    // the rest.
    int hpw = a.num_kv_heads <= kMfmaWaves ? a.num_kv_heads : kMfmaWaves;
    while (a.num_kv_heads % hpw) --hpw;
    hipError_t e = mark(a.ev_before, s);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(decode_mfma_kernel<G>, dim3(a.n_wg, a.num_kv_heads / hpw), dim3(64 * hpw), 0, s, a);
    if ((e = hipGetLastError()) != hipSuccess || (e = mark(a.ev_after, s)) != hipSuccess) return e;
    if (a.combine_waves == 1)
        hipLaunchKernelGGL((combine_kernel<G, true>), dim3(a.n_seqs * a.num_kv_heads), dim3(64 * G), 0, s, a);
    else
        hipLaunchKernelGGL((combine_kernel<G>), dim3(a.n_seqs * a.num_kv_heads, G), dim3(64 * kCombineWaves), 0, s,
                           a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_decode(const DecodeArgs &a, hipStream_t s) {
    if (a.n_seqs <= 0) return hipSuccess;
    if (a.whole) {
        const int G = a.num_heads / a.num_kv_heads;
        if (a.whole < 1 || G % a.whole) return hipErrorInvalidValue;
        switch (G / a.whole) {
            case 1: return launch_whole<1>(a, s);
            case 2: return launch_whole<2>(a, s);
            case 3: return launch_whole<3>(a, s);
            case 4: return launch_whole<4>(a, s);
            case 6: return launch_whole<6>(a, s);
            case 8: return launch_whole<8>(a, s);
            default: return hipErrorInvalidValue;
        }
    }
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
