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
// Unit = (sequence, tile of Q new tokens, kv head).  The tile's query rows
// are the Q x G (token, query head) pairs of the GQA group packed row after
// row — every head of the group attends to the same K/V — so four waves of
// 16 x NT rows each (Q = 64*NT/G) leave at most G-1 rows idle (the tree
// verify's 9 nodes x 6 heads fill 54 of 64 rows).  Work is split stream-K
// over key blocks (64 keys for prefill steps of eight-wave tiles, 32
// otherwise: mq_keys_for): the blocks of all units are laid end to end, head-major
// (kv head, sequence, tile), and each workgroup takes an equal share, the
// shares dealt out XCD by XCD so the tiles of one (sequence, head) run on
// one XCD and their repeated reads of its keys come from that XCD's L2;
// units cut by a share boundary leave partials for mq_combine_kernel.
//
// K/V blocks travel HBM -> LDS by buffer loads that write LDS directly (no
// register staging), through a ring of LDS stages: four of 32 keys (while
// block i is computed, blocks i+1..i+3, 96 KB, are in flight) or two of 64
// keys (block i+1, 64 KB).  Each wave issues the loads of KEYS/WAVES keys of
// every block; a wave waits for its own loads of block i (vmcnt) and one
// workgroup barrier makes all of them visible and frees the stage of block
// i-1 for the next issue.  Rows are stored with an XOR swizzle of
// their 16-byte granules so both read patterns below are conflict-free.
//
// Per block, wave and 16-row tile t (v_mfma_f32_16x16x32_f16, C layout:
// lane l holds rows 4*(l/16)+i, column l%16):
//   S^T[key][row] = K[key][:] . Q[row][:]   (A = K rows read from LDS once
//       for all NT tiles, B = Q^T held in registers for the whole unit);
//   per row: scale, mask, online softmax (max over the 4 lane groups with
//       two permlane swaps; the reference max moves, and acc is rescaled,
//       only when a block's max passes it by more than a slack), P^T in
//       fp16 — already the B operand of
//   O^T[dim][row] += V^T[dim][key] . P^T[key][row]   (A = V^T read with
//       ds_read_b64_tr_b16 from the row-major V tile; 16 dim tiles).
// The k-index permutation of P^T (keys 4g..4g+3 and 16+4g..16+4g+3 in lane
// group g) is matched by the V^T reads, so the sum is over the right pairs.
#include "k_common.h"
#include "kva_internal.h"

namespace kva {
namespace {

constexpr int kRowBytes = kHeadDim * 2;             // 512 B: one key of one head
constexpr int kPairBytes = 2 * kRowBytes + 32;      // two keys, then 32 B of padding
// LDS stages of the ring for blocks of KEYS keys: 4 x 33 KB or 2 x 66 KB.
template <int KEYS> constexpr int ring_stages() { return KEYS == 32 ? 4 : 2; }
template <int KEYS> constexpr int tile_bytes() { return KEYS / 2 * kPairBytes; }  // K or V of a block
constexpr float kLog2e = 1.4426950408889634f;


__device__ __forceinline__ int mq_wg_start(int w, int n, int W) { return floor_muldiv(w, n, W); }
__device__ __forceinline__ int mq_wg_of(int p, int n, int W) {
    int w = floor_muldiv(p, W, n);
    while (w + 1 < W && mq_wg_start(w + 1, n, W) <= p) ++w;
    return w;
}
// Largest i in [0, n) with pre[i] <= x (pre non-decreasing, pre[0] <= x;
// wave-uniform arguments).  Each round reads 64 evenly spaced entries of the
// remaining interval with one vector load and keeps the stretch between the
// last entry <= x and the next (a ballot: the entries <= x are a prefix of
// the lanes): two rounds up to 4096 entries, where a binary search by
// scalar loads took one dependent round trip per halving.
__device__ __forceinline__ int upper_index(const int32_t *pre, int n, int x, int lane) {
    int lo = 0, hi = n;  // the answer lies in [lo, hi)
    while (hi - lo > 1) {
        const int step = (hi - lo + 63) >> 6;  // entries between probes
        const int i = lo + lane * step;
        const uint64_t ok = __ballot(i < hi && pre[i] <= x);  // lane 0: pre[lo] <= x
        const int k = ok ? 63 - __clzll(ok) : 0;
        lo = __builtin_amdgcn_readfirstlane(lo + k * step);
        hi = __builtin_amdgcn_readfirstlane(min(hi, lo + step));
    }
    return lo;
}

// LDS layout of a K or V tile: keys in pairs (one 1 KB load each) 1056 B
// apart, and in odd keys the 16-byte granules swapped in twos (K) or fours
// (V).  The padding and the swaps spread both read patterns over all banks
// — K reads take 16 consecutive keys at one granule, V^T reads 4
// consecutive keys at two neighbouring granules — while every read of a
// lane stays at a fixed offset from one base, so the addresses are
// immediates (key = key index within the block).
__device__ __forceinline__ int key_off(int key) { return (key >> 1) * kPairBytes + (key & 1) * kRowBytes; }
__device__ __forceinline__ int k_granule(int key, int p) { return p ^ (key & 1); }
__device__ __forceinline__ int v_granule(int key, int p) { return p ^ ((key & 1) << 2); }

// The facts of one unit (all wave-uniform, read by scalar loads).
struct Unit {
    int u, ub, ue;        // unit index and its global block range [ub, ue)
    int b, h, tile;       // sequence (index in the step), kv head, query tile
    int ctx, ns, tok, T;  // keys visible, first new slot, first token, new tokens
    const int32_t *trow;  // block-table row
};

// Units are head-major: unit u is tile r = u % U1 of head u / U1 (U1 =
// upre[n_seqs], one head's units), and sequence b holds tiles
// [upre[b], upre[b+1]).  b is a hint (a sequence at or before the unit's
// within the same head), so a walk in unit order scans each sequence once.
template <int KEYS>
__device__ __forceinline__ Unit load_unit(const MultiQueryArgs &a, int u, int b) {
    Unit x;
    x.u = u;
    x.ub = ld_uniform(a.mq_pre + u) + mq_unit_cost(KEYS);  // its first block (positions before: the start cost)
    x.ue = ld_uniform(a.mq_pre + u + 1);
    const int U1 = ld_uniform(a.upre + a.n_seqs);
    x.h = u / U1;
    const int r = u - x.h * U1;
    if (r < ld_uniform(a.upre + b)) b = 0;  // the walk entered the next head
    while (ld_uniform(a.upre + b + 1) <= r) ++b;
    x.b = b;
    x.tile = r - ld_uniform(a.upre + b);
    x.ctx = ld_uniform(a.ctx_lens + b);
    x.ns = ld_uniform(a.new_start + b);
    x.tok = ld_uniform(a.tok_off + b);
    x.T = ld_uniform(a.tok_off + b + 1) - x.tok;
    x.trow = a.table + static_cast<size_t>(ld_uniform(a.seq_ids + b)) * a.table_stride;
    return x;
}

// Page of this wave's keys of block g of unit un (see issue_block).  (Read
// a block ahead, at the end of the previous block, it measured 10 % slower
// on config 4.)
template <int WAVES, int KEYS>
__device__ __forceinline__ int block_page(const Unit &un, int g, bool on, int wv) {
    const int key0 = (g - un.ub) * KEYS + KEYS / WAVES * wv;
    return on ? ld_uniform(un.trow + (min(key0, un.ctx - 1) >> 4)) : 0;
}

// Issue this wave's share of block g of unit un into LDS stage `st`: keys
// kPer*wv .. kPer*wv + kPer-1 of the block (kPer = 32/WAVES, within one
// page), K and V, one 1 KB load per two keys each (lane l writes granule
// l%32 of key 2i + l/32).  Keys past the sequence read its last key (finite
// data; the mask drops them).  A disabled issue (past the workgroup's share)
// goes through an empty resource: no memory access, but the same loads, so
// every wave's load counter advances alike.
template <int WAVES, int KEYS>
__device__ __forceinline__ void issue_block(uint8_t *st, const MultiQueryArgs &a, const Unit &un, int g, bool on,
                                            int page, int wv, int lane, int row_bytes) {
    constexpr int kPer = KEYS / WAVES;
    static_assert(kPer <= kBlockTokens && kBlockTokens % kPer == 0, "a wave's keys of a block lie in one page");
    const int key0 = (g - un.ub) * KEYS + kPer * wv;  // key of the unit
    const int last = un.ctx - 1;
    const size_t off = (static_cast<size_t>(page) * kBlockTokens * row_bytes + un.h * kRowBytes) / 2;
    const uint32_t n = on ? kBlockTokens * row_bytes : 0u;
    const auto rk = ro_rsrc(a.k_pool + off, n), rv = ro_rsrc(a.v_pool + off, n);
    const int q = lane & 31;
#pragma unroll
    for (int i = 0; i < kPer / 2; ++i) {
        const int kl = kPer * wv + 2 * i + (lane >> 5);  // key within the block
        const int row = min(key0 + 2 * i + (lane >> 5), last) & 15;
        const uint32_t dst = lds_addr(st + (kPer * wv / 2 + i) * kPairBytes);  // this load's two keys
        load_to_lds(rk, dst, row * row_bytes + 16 * k_granule(kl, q));
        load_to_lds(rv, dst + tile_bytes<KEYS>(), row * row_bytes + 16 * v_granule(kl, q));
    }
}

// Block i's loads have landed in LDS when at most the loads of the blocks
// issued after it and before this wait (ring stages - 2 of them, KEYS/WAVES
// loads each per wave) are outstanding.
template <int WAVES, int KEYS>
__device__ __forceinline__ void wait_block() { wait_vm<KEYS / WAVES * (ring_stages<KEYS>() - 2)>(); }

__device__ __forceinline__ half8_t as_h8(uint4 v) { return __builtin_bit_cast(half8_t, v); }

// A row's reference max moves only when a block's max exceeds it by more
// than this (log2 units): probabilities then stay below 2^8 (fp16 holds
// them to the same relative precision) and the accumulators are rescaled
// only on such jumps, not at every block where some row's max grew.
constexpr float kRescaleSlack = 8.0f;

// Stream-K share of workgroup i.  Workgroup i runs on XCD i % 8, so with
// W a multiple of 8 the shares are dealt out XCD by XCD: XCD x takes shares
// [x*W/8, (x+1)*W/8), consecutive in unit order.  With head-major units the
// tiles of one (sequence, head), which all read that head's keys, then run
// together on one XCD and share its L2.
__device__ __forceinline__ int mq_share_of(int i, int W) {
    return (W & 7) == 0 ? (i & 7) * (W >> 3) + (i >> 3) : i;
}

template <int NT, int WAVES, bool TREE, int KEYS>
__global__ __launch_bounds__(64 * WAVES) void mq_kernel(MultiQueryArgs a) {
    constexpr int kRing = ring_stages<KEYS>();
    constexpr int kTileBytes = tile_bytes<KEYS>();
    constexpr int kKT = KEYS / 16;  // 16-key tiles of a block (QK)
    constexpr int kKS = KEYS / 32;  // 32-key steps of a block (PV)
    __shared__ __attribute__((aligned(16))) uint8_t ring[kRing][2 * kTileBytes];
    const int w = mq_share_of(blockIdx.x, a.n_wg);  // this workgroup's share (and partial slots)
    const int W = a.n_wg;
    const int NB = a.total_blocks;
    const int q0 = mq_wg_start(w, NB, W);
    const int q1 = mq_wg_start(w + 1, NB, W);
    if (q0 >= q1) return;  // uniform over the workgroup
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int col = lane & 15;  // this lane's row within each 16-row tile (C/B column)
    const int grp = lane >> 4;  // lane group: keys 4*grp.. of a 16-key tile
    const int hkv = a.num_kv_heads;
    const int nh = a.num_heads;
    const int G = nh / hkv;
    const int Q = a.q_tile;
    const int row_bytes = hkv * kRowBytes;
    const float scale = kLog2e / 16.0f;

    // This lane's query row in each of the wave's NT tiles: (token iq, head gq).
    int iq[NT], gq[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int rho = 16 * (wv * NT + t) + col;
        iq[t] = rho / G;
        gq[t] = rho - iq[t] * G;
    }

    // Issue side: the unit and block of the next load, kRing-1 blocks ahead
    // of the compute side, across unit boundaries.
    const int u0 = upper_index(a.mq_pre, a.n_units, q0, lane);
    const int U1 = ld_uniform(a.upre + a.n_seqs);
    Unit iu = load_unit<KEYS>(a, u0, upper_index(a.upre, a.n_seqs, u0 % U1, lane));
    int ig = max(q0, iu.ub);
    if (ig >= q1) return;  // the share holds only a unit's start cost
    int ipage = 0;  // page of the next issue
    auto fetch_page = [&]() { ipage = block_page<WAVES, KEYS>(iu, ig, ig < q1, wv); };
    auto issue = [&](int slot) {
        const bool on = ig < q1;
        issue_block<WAVES, KEYS>(ring[slot], a, iu, ig, on, ipage, wv, lane, row_bytes);
        if (on && ++ig < q1 && ig >= iu.ue) {
            iu = load_unit<KEYS>(a, iu.u + 1, iu.b);
            ig = iu.ub;
        }
    };
    Unit cu = iu;
    int g = ig;
#pragma unroll
    for (int s = 0; s + 1 < kRing; ++s) {
        fetch_page();
        issue(s);
    }

    int n_done = 0;  // blocks computed by this workgroup (ring position)
    while (true) {
        const int seg_end = min(cu.ue, q1);
        const bool whole = g == cu.ub && seg_end == cu.ue;
        // Query rows of this unit.
        bool qvalid[NT];
        int qslot[NT];
        uint64_t qbits[NT];
        uint4 qb[NT][8];  // B operand Q^T: dims 32*kk + 8*grp .. +8
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int qi = cu.tile * Q + iq[t];
            qvalid[t] = iq[t] < Q && qi < cu.T;
            qslot[t] = cu.ns + qi;
            qbits[t] = (TREE && qvalid[t]) ? a.tok_bits[cu.tok + qi] : 0ull;
            const uint16_t *qr =
                a.q + (static_cast<size_t>(cu.tok + (qvalid[t] ? qi : 0)) * nh + cu.h * G + gq[t]) * kHeadDim;
#pragma unroll
            for (int kk = 0; kk < 8; ++kk)
                qb[t][kk] = qvalid[t] ? ld16(qr + 32 * kk + 8 * grp) : make_uint4(0, 0, 0, 0);
        }
        // Take delivery of the query rows here, once per unit: left to the
        // compiler, the wait for them would sit inside the block loop and
        // (not seeing the LDS loads) drain the ring at every block.
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            asm volatile("" : "+v"(qbits[t]));
#pragma unroll
            for (int kk = 0; kk < 8; ++kk)
                asm volatile("" : "+v"(qb[t][kk].x), "+v"(qb[t][kk].y), "+v"(qb[t][kk].z), "+v"(qb[t][kk].w));
        }
        float m[NT], l[NT];
        float4_t acc[NT][16];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            m[t] = -INFINITY;
            l[t] = 0.0f;
#pragma unroll
            for (int dt = 0; dt < 16; ++dt) acc[t][dt] = float4_t{0.f, 0.f, 0.f, 0.f};
        }

        for (; g < seg_end; ++g) {
            wait_block<WAVES, KEYS>();
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
            fetch_page();
            issue((n_done + kRing - 1) % kRing);
            __builtin_amdgcn_sched_barrier(0);
            const uint8_t *kt = ring[n_done % kRing];
            const uint8_t *kbase = kt + key_off(col) + 16 * k_granule(col, grp);
            const int key0 = (g - cu.ub) * KEYS;

            // S^T for keys key0 + 16*nt + 4*grp + i, row `col` of each tile.
            float4_t s[NT][kKT];
#pragma unroll
            for (int nt = 0; nt < kKT; ++nt) {
#pragma unroll
                for (int t = 0; t < NT; ++t) s[t][nt] = float4_t{0.f, 0.f, 0.f, 0.f};
                // key 16*nt + col, granule 4*kk + grp: kbase + nt*8 pairs + 64*kk
                const uint8_t *kr = kbase + 8 * nt * kPairBytes;
#pragma unroll
                for (int kk = 0; kk < 8; ++kk) {
                    const uint4 ka = *reinterpret_cast<const uint4 *>(kr + 64 * kk);
#pragma unroll
                    for (int t = 0; t < NT; ++t)
                        s[t][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(ka), as_h8(qb[t][kk]), s[t][nt],
                                                                        0, 0, 0);
                }
            }
            half8_t pb[NT][kKS];
            float corr[NT];
            bool rescale = false;
            // A block wholly before the step's first new slot is visible to
            // every row (wave-uniform test); otherwise mask key by key.  Rows
            // past the unit's tokens are never written, so the open case
            // needs no mask at all.
            const bool open = key0 + KEYS <= cu.ns;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                // Masked scores become -inf; the max is taken over the raw
                // scores and scaled once (scale > 0 keeps the order and the
                // rounding of the largest), and the probabilities below
                // fold the scale into one fma.
                if (!open) {  // wave-uniform: blocks of the cache prefix skip this
#pragma unroll
                    for (int nt = 0; nt < kKT; ++nt)
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            bool vis;
                            if constexpr (TREE) {
                                // The cache before the step, then the new rows
                                // in the node's bit set (bits only for the
                                // step's nodes, so keys past the sequence drop
                                // out).  Bitwise, so no lane branches.
                                const int rel = key0 + 16 * nt + 4 * grp + i - cu.ns;
                                const bool bit = ((qbits[t] >> (rel & 63)) & 1ull) != 0;
                                vis = qvalid[t] & ((rel < 0) | ((rel < 64) & bit));
                            } else {
                                // key0 + 16nt + 4grp + i <= qslot (qslot < ctx)
                                vis = qvalid[t] & (16 * nt + i <= qslot[t] - key0 - 4 * grp);
                            }
                            s[t][nt][i] = vis ? s[t][nt][i] : -INFINITY;
                        }
                }
                float mx = -INFINITY;
#pragma unroll
                for (int nt = 0; nt < kKT; ++nt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[t][nt][i]);
                mx = group4_max(mx) * scale;
                // Move the reference max only on a jump past the slack (or
                // from -inf, where acc and l are still zero).
                const bool jump = mx > m[t] + kRescaleSlack;
                const float mn = jump ? mx : m[t];
                const float mu = (mn == -INFINITY) ? 0.0f : mn;  // rows with nothing visible yet
                corr[t] = __builtin_amdgcn_exp2f(m[t] - mu);
                rescale = rescale || (jump && m[t] != -INFINITY);
                uint32_t pk[2 * kKT];
#pragma unroll
                for (int nt = 0; nt < kKT; ++nt) {
                    pk[2 * nt] = pack_p2(__builtin_amdgcn_exp2f(fmaf(s[t][nt][0], scale, -mu)),
                                         __builtin_amdgcn_exp2f(fmaf(s[t][nt][1], scale, -mu)));
                    pk[2 * nt + 1] = pack_p2(__builtin_amdgcn_exp2f(fmaf(s[t][nt][2], scale, -mu)),
                                             __builtin_amdgcn_exp2f(fmaf(s[t][nt][3], scale, -mu)));
                }
                // l sums the fp16 probabilities PV uses.
                constexpr uint32_t kOnes = 0x3c003c00u;  // fp16 pair (1, 1)
                float psum = 0.0f;
#pragma unroll
                for (int i = 0; i < 2 * kKT; ++i) psum = dot2(pk[i], kOnes, psum);
                l[t] = l[t] * corr[t] + psum;
                m[t] = mn;
#pragma unroll
                for (int ks = 0; ks < kKS; ++ks)
                    pb[t][ks] = __builtin_bit_cast(half8_t, make_uint4(pk[4 * ks], pk[4 * ks + 1], pk[4 * ks + 2],
                                                                      pk[4 * ks + 3]));
            }
            // Rescale only when some row's reference max moved (wave-uniform).
            if (__builtin_amdgcn_ballot_w64(rescale)) {
#pragma unroll
                for (int t = 0; t < NT; ++t)
#pragma unroll
                    for (int dt = 0; dt < 16; ++dt) acc[t][dt] *= corr[t];
            }
            // V^T operand of dim tile dt: ds_read_b64_tr_b16 gives lane c of
            // a 16-lane group column c of the 4 x 16 block whose row r the
            // group's lanes 4r..4r+3 address, 8 bytes each: here key
            // 4*grp + r (then 16 + 4*grp + r), dims 16*dt + 4*(lane%4) ...
            // Key 16*hh + 4*grp + vr, granule 2*dt + vs/2: for odd keys the
            // swap of fours moves dims 32*dt.. by +-64 B, + when bit 1 of dt
            // is clear, - when set, so two bases cover every dt.
            const int vr = (lane & 15) >> 2;
            const int vs = lane & 3;
            const uint8_t *vb = kt + kTileBytes + key_off(4 * grp + vr) + 16 * (vs >> 1) + 8 * (vs & 1);
            const uint8_t *vbase[2] = {vb + 64 * (vr & 1), vb - 64 * (vr & 1)};
#pragma unroll
            for (int dt = 0; dt < 16; ++dt) {
#pragma unroll
                for (int ks = 0; ks < kKS; ++ks) {  // keys 32*ks ..: 16 pairs on
                    short4_t part[2];
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        const uint8_t *src = vbase[(dt >> 1) & 1] + (16 * ks + 8 * hh) * kPairBytes + 32 * dt;
                        part[hh] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t *)src);
                    }
                    const uint2 v0 = __builtin_bit_cast(uint2, part[0]);
                    const uint2 v1 = __builtin_bit_cast(uint2, part[1]);
                    const half8_t va = __builtin_bit_cast(half8_t, make_uint4(v0.x, v0.y, v1.x, v1.y));
#pragma unroll
                    for (int t = 0; t < NT; ++t)
                        acc[t][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb[t][ks], acc[t][dt], 0, 0, 0);
                }
            }
            ++n_done;
        }

        // The four lane groups hold disjoint keys of each row.
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const float lt = group4_sum(l[t]);
            const int rho = 16 * (wv * NT + t) + col;
            if (whole) {
                if (qvalid[t]) {
                    const float inv = 1.0f / lt;
                    const size_t tq = static_cast<size_t>(cu.tok + cu.tile * Q + iq[t]);
                    uint16_t *orow = a.out + (tq * nh + cu.h * G + gq[t]) * kHeadDim;
                    const uint16_t *grow = a.gate ? a.gate + tq * a.gate_stride + (cu.h * G + gq[t]) * kHeadDim : nullptr;
#pragma unroll
                    for (int dt = 0; dt < 16; ++dt)
                        *reinterpret_cast<uint2 *>(orow + 16 * dt + 4 * grp) =
                            out_fp16x4(acc[t][dt][0] * inv, acc[t][dt][1] * inv, acc[t][dt][2] * inv,
                                       acc[t][dt][3] * inv, grow ? grow + 16 * dt + 4 * grp : nullptr);
                }
            } else {
                // Slot 2w: the unit began at or before this share (its first
                // segment); slot 2w+1: the share's last segment.
                const int slot = 2 * w + (cu.ub <= q0 ? 0 : 1);
                const size_t rowi = static_cast<size_t>(slot) * kMqSlotRows + rho;
                float *ar = a.ws_acc + rowi * kHeadDim;
#pragma unroll
                for (int dt = 0; dt < 16; ++dt)
                    *reinterpret_cast<float4 *>(ar + 16 * dt + 4 * grp) =
                        make_float4(acc[t][dt][0], acc[t][dt][1], acc[t][dt][2], acc[t][dt][3]);
                if (grp == 0) {
                    a.ws_ml[rowi * 2] = m[t];
                    a.ws_ml[rowi * 2 + 1] = lt;
                }
            }
        }
        if (g >= q1) break;
        cu = load_unit<KEYS>(a, cu.u + 1, cu.b);
        g = cu.ub;
        if (g >= q1) break;  // the share ends inside the next unit's start cost
    }
    // Loads past the share write LDS too: none may land after the
    // workgroup's LDS is handed on.
    __builtin_amdgcn_s_waitcnt(0);
}

// Merge the partials of units cut across workgroups: one workgroup per
// (cut unit, 16 rows of its tile); thread = (row, 16-dim slice).  The step
// plan holds a record per cut unit (kva_step_begin finds them from the same
// shares as the launch), so a workgroup waits for two memory round trips:
// its record, then every piece's (m, l) and acc slice, requested before any
// is used and merged online.  (Found here, from the unit positions, the
// tile's sequence and token range, the pieces took four, and the launch
// held a row of workgroups for every unit, cut or not.)
__global__ __launch_bounds__(256) void mq_combine_kernel(MultiQueryArgs a) {
    constexpr int kMaxP = 4;  // pieces requested together
    const int32_t *rec = a.mq_cut + static_cast<size_t>(blockIdx.x) * kMqCutWords;
    const int h = ld_uniform(rec);
    const int tq0 = ld_uniform(rec + 1);      // the tile's first new token (step order)
    const int n_valid = ld_uniform(rec + 2);  // its tokens
    const int w0 = ld_uniform(rec + 3);
    const int w1 = ld_uniform(rec + 4);
    const int slot0 = ld_uniform(rec + 5);
    const int G = a.num_heads / a.num_kv_heads;
    const int rho = 16 * blockIdx.y + (threadIdx.x >> 4);
    const int d0 = (threadIdx.x & 15) * 16;
    const int iq = rho / G;
    const int gq = rho - iq * G;
    if (iq >= n_valid) return;
    // Running merge: (big, lt, o) over the pieces so far; m in log2 units.
    float big = -INFINITY, lt = 0.0f;
    float o[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) o[e] = 0.0f;
    for (int wb = w0; wb <= w1; wb += kMaxP) {
        float2 ml[kMaxP];
        float4 v[kMaxP][4];
#pragma unroll
        for (int i = 0; i < kMaxP; ++i) {
            const int ww = wb + i;
            if (ww <= w1) {
                const int slot = ww == w0 ? slot0 : 2 * ww;
                const size_t rowi = static_cast<size_t>(slot) * kMqSlotRows + rho;
                ml[i] = *reinterpret_cast<const float2 *>(a.ws_ml + rowi * 2);
                const float4 *src = reinterpret_cast<const float4 *>(a.ws_acc + rowi * kHeadDim + d0);
#pragma unroll
                for (int e = 0; e < 4; ++e) v[i][e] = src[e];
            } else {
                ml[i] = make_float2(-INFINITY, 0.0f);
#pragma unroll
                for (int e = 0; e < 4; ++e) v[i][e] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
        float nb = big;
#pragma unroll
        for (int i = 0; i < kMaxP; ++i) nb = fmaxf(nb, ml[i].x);
        const float mu = (nb == -INFINITY) ? 0.0f : nb;  // rows that see no key of these pieces
        const float keep = (big == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(big - mu);
        lt *= keep;
#pragma unroll
        for (int e = 0; e < 16; ++e) o[e] *= keep;
#pragma unroll
        for (int i = 0; i < kMaxP; ++i) {
            const float c = (ml[i].x == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(ml[i].x - mu);
            lt += c * ml[i].y;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                o[4 * e] += c * v[i][e].x;
                o[4 * e + 1] += c * v[i][e].y;
                o[4 * e + 2] += c * v[i][e].z;
                o[4 * e + 3] += c * v[i][e].w;
            }
        }
        big = nb;
    }
    const float inv = 1.0f / lt;
    const size_t tq = static_cast<size_t>(tq0 + iq);
    uint16_t *orow = a.out + (tq * a.num_heads + h * G + gq) * kHeadDim + d0;
    const uint16_t *grow = a.gate ? a.gate + tq * a.gate_stride + (h * G + gq) * kHeadDim + d0 : nullptr;
    uint2 p[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
        p[e] = out_fp16x4(o[4 * e] * inv, o[4 * e + 1] * inv, o[4 * e + 2] * inv, o[4 * e + 3] * inv,
                          grow ? grow + 4 * e : nullptr);
    *reinterpret_cast<uint4 *>(orow) = make_uint4(p[0].x, p[0].y, p[1].x, p[1].y);
    *reinterpret_cast<uint4 *>(orow + 8) = make_uint4(p[2].x, p[2].y, p[3].x, p[3].y);
}

template <int NT, int WAVES>
hipError_t launch_mq(const MultiQueryArgs &a, hipStream_t s) {
    // 64-key blocks only for eight-wave causal tiles (mq_keys_for).
    const bool k64 = a.keys == 64 && WAVES == 8 && !a.tree;
    if (a.keys != 32 && !k64) return hipErrorInvalidValue;
    if (a.ev_before) {
        const hipError_t e = hipEventRecord(a.ev_before, s);
        if (e != hipSuccess) return e;
    }
    if (a.tree) {
        hipLaunchKernelGGL((mq_kernel<NT, WAVES, true, 32>), dim3(a.n_wg), dim3(64 * WAVES), 0, s, a);
    } else if (k64) {
        if constexpr (WAVES == 8)
            hipLaunchKernelGGL((mq_kernel<NT, WAVES, false, 64>), dim3(a.n_wg), dim3(64 * WAVES), 0, s, a);
    } else {
        hipLaunchKernelGGL((mq_kernel<NT, WAVES, false, 32>), dim3(a.n_wg), dim3(64 * WAVES), 0, s, a);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (a.ev_after && (e = hipEventRecord(a.ev_after, s)) != hipSuccess) return e;
    if (a.n_cut > 0) hipLaunchKernelGGL(mq_combine_kernel, dim3(a.n_cut, WAVES * NT), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_multi_query(const MultiQueryArgs &a, hipStream_t s) {
    if (a.n_units <= 0 || a.total_blocks <= 0) return hipSuccess;
    const int G = a.num_heads / a.num_kv_heads;
    if (G < 1 || G > kMqMaxGroup || a.num_heads % a.num_kv_heads) return hipErrorInvalidValue;
    if (a.q_tile != mq_tile_tokens(G, a.n_waves, a.n_t)) return hipErrorInvalidValue;
    if (a.n_t == 1 && a.n_waves == 4) return launch_mq<1, 4>(a, s);
    if (a.n_t == 1 && a.n_waves == 8) return launch_mq<1, 8>(a, s);
    return hipErrorInvalidValue;
}

}  // namespace kva
