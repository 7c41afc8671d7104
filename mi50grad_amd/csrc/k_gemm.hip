// Prefill-sized Q/K/V projection: one GEMM launch with the norm + RoPE +
// append epilogue fused (gfx950).
//
// The reference projects a prefill chunk with its batched FP16 GEMM once
// seq_len >= 32 (gemm_fp16_prefill.hip:47, launched through
// _launch_gemm_fp16 at engine.py:3061-3068 into [Q | Q_gate] and [K | V]),
// then normalises, rotates and appends per token.  Here
//   Y[t][n] = sum_k X[t][k] W[n][k]   (X: [T][hidden], W: the stacked
//   weight rows [w_a; w_b], both k-contiguous)
// runs as tiles of 256 tokens x 256 weight rows.  256 rows are exactly one
// head of one kind (Q, Q_gate, K or V), so the workgroup that finishes a
// tile holds complete head rows for its 256 tokens and does the epilogue of
// proj_finish_kernel itself: each value rounded to fp16 (what the
// reference's GEMM stores), then Q -> RMSNorm + RoPE -> q_out, Q_gate ->
// gate_out, K -> RMSNorm + RoPE -> its page slot (and K, V as projected ->
// kv_out), V -> its page slot.  No [T][N] intermediate and no second launch.
//
// Main loop.  Eight waves in a 2 x 4 grid, each 128 tokens x 64 rows as
// 8 x 4 tiles of v_mfma_f32_16x16x32_f16 (A = X rows, B = W rows; lane l
// holds row l%16 and k-slots 8*(l/16)..+7 of both, C: tokens 4*(l/16)+i,
// row l%16).  K goes in chunks of 64 through two LDS stages (X 32 KB + W
// 32 KB each): buffer loads write LDS directly, chunk c+1 is issued while
// chunk c is multiplied, one barrier per chunk makes a chunk visible and
// frees the stage of chunk c-1.  A chunk of 64 k is one whole 128-byte line
// per row, which the load path moves markedly faster than half lines (a
// 32-wide chunk in four stages is slower although more of it is in
// flight).  Rows sit 128 bytes apart in LDS with their 16-byte granules
// XOR-swizzled (g_swizzle), chosen by which global granule each lane
// fetches, so the 16 rows an MFMA operand read touches fall in different
// banks.  A chunk issued past the end goes through an empty buffer
// resource: the same loads, no memory access, so every wave's load counter
// advances alike and the waits stay exact.
//
// What bounds it: the global -> LDS path.  A 256 x 256 tile needs 1/64 byte
// per MAC, about 67 GB/s per CU to keep the MFMA pipes full at the clock
// this kernel runs at; the load path alone moves ~45-51 GB/s per CU here.
//
// Tile order.  Tiles are numbered head-major (head, token tile) and dealt
// out XCD by XCD (workgroup i runs on XCD i % 8): each XCD takes a
// contiguous run of heads with all their token tiles, so a head's weight
// rows are read by one XCD and reused from its L2 by the token tiles
// running beside each other.
#include "k_common.h"
#include "k_normrope.h"
#include "kva_internal.h"

// Chunk width in k, LDS stages, waves per workgroup (tuning builds may
// override all three together).
#ifndef KVA_GEMM_KC
#define KVA_GEMM_KC 64
#define KVA_GEMM_S 2
#define KVA_GEMM_W 8
#endif

namespace kva {
namespace {

constexpr int kGTok = kBigTileTokens;      // tokens per tile
constexpr int kGRows = kHeadDim;           // weight rows per tile: one head
constexpr int kGWaveTok = kGTok / 2;       // tokens per wave (waves in a 2 x (W/2) grid)
constexpr int kGTM = kGWaveTok / 16;       // 16-token MFMA tiles per wave
// The epilogue's fp16 tile, rows padded against bank conflicts: half the
// tile's tokens at a time, in the ring.
constexpr int kGEpiRow = kGRows * 2 + 16;  // 528 B

// Geometry of the ring for KC k per stage (64 or 32) and W waves.
template <int KC, int W>
struct GRing {
    static constexpr int kWaves = W;
    static constexpr int kWaveRows = kGRows / (W / 2);         // weight rows per wave
    static constexpr int kTN = kWaveRows / 16;                // 16-row MFMA tiles per wave
    static constexpr int kRowBytes = KC * 2;                 // one row of one stage
    static constexpr int kGran = KC / 8;                      // 16-byte granules per row
    static constexpr int kStageX = kGTok * kRowBytes;
    static constexpr int kStageW = kGRows * kRowBytes;
    static constexpr int kStage = kStageX + kStageW;
    static constexpr int kLoadsX = kStageX / 1024 / W;  // 1 KB loads per wave per stage
    static constexpr int kLoadsW = kStageW / 1024 / W;
    static constexpr int kLoads = kLoadsX + kLoadsW;
};

// The granule swizzle of row r.  The 16 rows one MFMA operand read touches
// at one logical granule must land on distinct 16-byte bank groups whether
// the LDS serves 8 lanes per 128-byte cycle or 16 per 256-byte cycle.  With
// 128-byte rows (KC = 64) two rows share a 256-byte cycle, so the even rows
// take granules 0..7 and the odd rows the same set XORed by 4; with 64-byte
// rows (KC = 32) four rows share one.  The counters read zero bank
// conflicts for both.
template <int KC>
__device__ __forceinline__ int g_swizzle(int r) {
    if constexpr (KC == 64)
        return ((r >> 1) ^ ((r & 1) << 2)) & 7;
    else
        return ((r >> 1) ^ (r >> 2)) & (KC / 8 - 1);
}

// LDS byte offset of row r's 16-byte granule g within a stage's X or W part.
template <int KC>
__device__ __forceinline__ uint32_t g_swz(int r, int g) {
    return r * (KC * 2) + 16 * (g ^ g_swizzle<KC>(r));
}

// Issue one chunk's loads of this wave into `stage`: load j of the wave
// covers LDS granule slots 64*(W*j + wv) + lane of the X part, then of the
// W part; slot p holds row p / kGran at stored granule p % kGran, i.e.
// global granule (p % kGran) ^ swizzle(row) of that row.
template <int KC, int W>
__device__ __forceinline__ void g_issue(uint32_t stage, __amdgpu_buffer_rsrc_t rx, __amdgpu_buffer_rsrc_t rw,
                                        uint32_t k_byte, int wv, int lane, uint32_t row_bytes) {
    using R = GRing<KC, W>;
#pragma unroll
    for (int j = 0; j < R::kLoadsX; ++j) {
        const int ins = W * j + wv;
        const int p = 64 * ins + lane;
        const int row = p / R::kGran, g = (p % R::kGran) ^ g_swizzle<KC>(row);
        load_to_lds(rx, stage + 1024 * ins, row * row_bytes + k_byte + 16 * g);
    }
#pragma unroll
    for (int j = 0; j < R::kLoadsW; ++j) {
        const int ins = W * j + wv;
        const int p = 64 * ins + lane;
        const int row = p / R::kGran, g = (p % R::kGran) ^ g_swizzle<KC>(row);
        load_to_lds(rw, stage + R::kStageX + 1024 * ins, row * row_bytes + k_byte + 16 * g);
    }
}

__device__ __forceinline__ half8_t g_h8(uint4 v) { return __builtin_bit_cast(half8_t, v); }

template <int KC, int S, int W>
__global__ __launch_bounds__(64 * W) void proj_big_kernel(ProjectArgs a) {
    using R = GRing<KC, W>;
    constexpr int kTN = R::kTN;
    static_assert(kGWaveTok * kGEpiRow <= S * R::kStage, "half the epilogue tile must fit the ring");
    __shared__ __attribute__((aligned(16))) uint8_t ring[S * R::kStage];
    __shared__ int32_t meta[4][kGTok];  // per token of the tile: RoPE position, sequence, slot, page id

    const int n_heads = (a.n_a + a.n_b) / kGRows;
    const int n_mt = (a.n_tok + kGTok - 1) / kGTok;
    const int n_tiles = n_heads * n_mt;
    const int i = blockIdx.x;
    const int tau = (n_tiles & 7) == 0 ? (i & 7) * (n_tiles >> 3) + (i >> 3) : i;
    const int head = tau / n_mt;
    const int t0 = (tau - head * n_mt) * kGTok;  // first token of the tile within the launch
    const int n0 = head * kGRows;                // first stacked weight row
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int hidden = a.hidden;
    const uint32_t row_bytes = static_cast<uint32_t>(hidden) * 2;

    // The tile's tokens' facts, for the epilogue (requested first, used last).
    if (threadIdx.x < kGTok) {
        const int tl = t0 + threadIdx.x;
        const int t = a.tok0 + min(tl, a.n_tok - 1);
        const int pos = a.tok_pos[t], seq = a.tok_seq[t], slot = a.tok_slot[t];
        meta[0][threadIdx.x] = pos;
        meta[1][threadIdx.x] = seq;
        meta[2][threadIdx.x] = slot;
        meta[3][threadIdx.x] = a.table[static_cast<size_t>(seq) * a.table_stride + (slot >> 4)];
    }

    const uint16_t *wbase = n0 < a.n_a ? a.w_a + static_cast<size_t>(n0) * hidden
                                       : a.w_b + static_cast<size_t>(n0 - a.n_a) * hidden;
    const uint16_t *xbase = a.x + static_cast<size_t>(t0) * hidden;
    // X rows past the launch's tokens read as zeros (the resource's range).
    const uint32_t x_bytes = static_cast<uint32_t>(max(0, min(kGTok, a.n_tok - t0))) * row_bytes;
    const auto rx = ro_rsrc(xbase, x_bytes), rw = ro_rsrc(wbase, kGRows * row_bytes);
    const auto rx0 = ro_rsrc(xbase, 0u), rw0 = ro_rsrc(wbase, 0u);
    const uint32_t lds0 = lds_addr(ring);
    const int nc = hidden / KC;
    auto issue = [&](int c) {
        const bool on = c < nc;
        g_issue<KC, W>(lds0 + (c % S) * R::kStage, on ? rx : rx0, on ? rw : rw0,
                    static_cast<uint32_t>(on ? c : 0) * R::kRowBytes, wv, lane, row_bytes);
    };

    const int wm = wv / (W / 2), wn = wv % (W / 2);  // this wave's kGWaveTok tokens and kWaveRows rows
    const int col = lane & 15, grp = lane >> 4;
    float4_t acc[kGTM][kTN];
#pragma unroll
    for (int m = 0; m < kGTM; ++m)
#pragma unroll
        for (int n = 0; n < kTN; ++n) acc[m][n] = float4_t{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int s = 0; s + 1 < S; ++s) issue(s);
    for (int c = 0; c < nc; ++c) {
        // Chunk c has landed once no more than S - 2 later chunks' loads
        // are outstanding; the barrier then also frees chunk c-1's stage.
        wait_vm<R::kLoads * (S - 2)>();
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        issue(c + S - 1);
        __builtin_amdgcn_sched_barrier(0);
        const uint8_t *sx = ring + (c % S) * R::kStage;
        const uint8_t *sw = sx + R::kStageX;
        // Every k step's operands requested before the first product: the
        // later step's reads land while the earlier step multiplies (the
        // compiler, left alone, kept only 2-6 reads ahead of the products:
        // 295-298 against 289-291 us per layer at config 4).
        uint4 av[KC / 32][kGTM], bv[KC / 32][kTN];
#pragma unroll
        for (int ks = 0; ks < KC / 32; ++ks) {
            const int g = 4 * ks + grp;
#pragma unroll
            for (int n = 0; n < kTN; ++n)
                bv[ks][n] = *reinterpret_cast<const uint4 *>(sw + g_swz<KC>(R::kWaveRows * wn + 16 * n + col, g));
#pragma unroll
            for (int m = 0; m < kGTM; ++m)
                av[ks][m] = *reinterpret_cast<const uint4 *>(sx + g_swz<KC>(kGWaveTok * wm + 16 * m + col, g));
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ks = 0; ks < KC / 32; ++ks)
#pragma unroll
            for (int m = 0; m < kGTM; ++m)
#pragma unroll
                for (int n = 0; n < kTN; ++n)
                    acc[m][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(g_h8(av[ks][m]), g_h8(bv[ks][n]), acc[m][n],
                                                                     0, 0, 0);
    }
    // Every load (the dummy ones past the end too) has landed before the
    // ring is reused for the epilogue tile.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    const int H = a.num_heads, hkv = a.num_kv_heads;
    const int hw = threadIdx.x >> 5;  // half-wave 0 .. 2W-1
    const int l32 = threadIdx.x & 31;
    const bool is_q = head < H, is_gate = !is_q && head < 2 * H;
    const int kv = head - 2 * H;  // K heads 0..hkv-1, then V heads
    const bool rot = is_q || (!is_gate && kv < hkv);
    uint16_t *epi = reinterpret_cast<uint16_t *>(ring);
    // The norm weights are the same for every row of the tile; each
    // half-wave's cos/sin rows are requested before the half is written, so
    // the finish loop waits on none of them row by row.
    constexpr int kRowsPerHw = kGWaveTok / (2 * W);
    NormRopeIn nin[kRowsPerHw];
    const uint4 wnorm = rot ? ld16((is_q ? a.q_w : a.k_w) + 8 * l32) : make_uint4(0, 0, 0, 0);
    const int cl = a.half_rot > 0 ? min(l32, a.half_rot / 4 - 1) : 0;
    // Two halves: the waves of token half `half` write their sums as fp16
    // (each rounded once: what the reference's GEMM stores) into the tile
    // [kGWaveTok tokens][256 rows]; tile (m, n), C row 4*grp + e is token
    // 16*m + 4*grp + e of the half, column col is row kWaveRows*wn + 16*n +
    // col.  Then every wave finishes the half's token rows.
    for (int half = 0; half < 2; ++half) {
#pragma unroll
        for (int j = 0; j < kRowsPerHw; ++j) {
            nin[j].w = wnorm;
            nin[j].c = make_uint2(0, 0);
            nin[j].s = make_uint2(0, 0);
            if (rot && a.half_rot > 0) {
                // Tokens past the launch's end carry the last token's
                // position, so these reads stay inside the tables.
                const size_t off = static_cast<size_t>(meta[0][half * kGWaveTok + hw + 2 * W * j]) * a.half_rot;
                nin[j].c = ld8(a.cos_tab + off + 4 * cl);
                nin[j].s = ld8(a.sin_tab + off + 4 * cl);
            }
        }
        if (wm == half) {
#pragma unroll
            for (int m = 0; m < kGTM; ++m)
#pragma unroll
                for (int n = 0; n < kTN; ++n)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int tok = 16 * m + 4 * grp + e;
                        epi[tok * (kGEpiRow / 2) + R::kWaveRows * wn + 16 * n + col] = f2h(acc[m][n][e]);
                    }
        }
        __syncthreads();
        // Finish: one 32-lane group per token row, 8 dims per lane, the
        // arithmetic of proj_finish_kernel (norm_rope_apply: the same bits).
#pragma unroll
        for (int j = 0; j < kRowsPerHw; ++j) {
            const int rr = hw + 2 * W * j;
            const int r = half * kGWaveTok + rr;
            const int tl = t0 + r;
            if (tl >= a.n_tok) break;
            const int t = a.tok0 + tl;
            const uint4 y = *reinterpret_cast<const uint4 *>(epi + rr * (kGEpiRow / 2) + 8 * l32);
            if (is_gate) {
                if (a.gate_out) st16(a.gate_out + (static_cast<size_t>(t) * H + head - H) * kHeadDim + 8 * l32, y);
                continue;
            }
            if (!is_q && a.kv_out) st16(a.kv_out + (static_cast<size_t>(t) * 2 * hkv + kv) * kHeadDim + 8 * l32, y);
            const uint4 o = rot ? norm_rope_apply<32>(y, nin[j], a.half_rot, a.eps, l32) : y;
            if (is_q) {
                st16(a.q_out + (static_cast<size_t>(t) * H + head) * kHeadDim + 8 * l32, o);
                continue;
            }
            const int slot = meta[2][r], blk = meta[3][r];
            const size_t row_base = (static_cast<size_t>(blk) * kBlockTokens + (slot & 15)) * hkv;
            if (kv < hkv)
                st16(a.k_pool + (row_base + kv) * kHeadDim + 8 * l32, o);
            else
                st16(a.v_pool + (row_base + kv - hkv) * kHeadDim + 8 * l32, y);
        }
        __syncthreads();  // the half's rows are read before the next half overwrites them
    }
}

}  // namespace

hipError_t launch_project_big(const ProjectArgs &a, hipStream_t s) {
    if (a.n_tok <= 0) return hipSuccess;
    if ((a.n_a + a.n_b) % kGRows != 0 || a.hidden % 64 != 0 || a.n_tok > kBigProjMaxTokens)
        return hipErrorInvalidValue;
    const int n_heads = (a.n_a + a.n_b) / kGRows;
    const int n_mt = (a.n_tok + kGTok - 1) / kGTok;
    if (a.ev_before) {
        const hipError_t e = hipEventRecord(a.ev_before, s);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL((proj_big_kernel<KVA_GEMM_KC, KVA_GEMM_S, KVA_GEMM_W>), dim3(n_heads * n_mt),
                       dim3(64 * KVA_GEMM_W), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && a.ev_after) e = hipEventRecord(a.ev_after, s);
    return e;
}

}  // namespace kva
