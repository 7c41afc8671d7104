// Q/K/V projection fused with QK-RMSNorm + RoPE + K/V append (gfx950).
//
// The reference projects the normed hidden state with FP16 GEMVs
// (gemv_fp16_v2.hip:22-85: fp32 accumulation, fp16 result) into [Q | Q_gate]
// and [K | V] buffers (engine.py:1366-1378 stack the weights that way), then
// normalises/rotates Q and K and copies K and V into the cache slot
// (engine.py:2000-2022, 2371-2432; c_dispatch.c:1042-1059 sends V's GEMV
// straight to the slot).  Here a step's tokens are projected together:
//
// proj_gemm_kernel: out[t][n] = sum_k W[n][k] x[t][k] as split-K MFMA tiles.
//   A workgroup owns a run of 16-row weight tiles and one of `splits`
//   slices of hidden; each of its waves takes an equal part of the slice for
//   all those rows and all tokens (up to four 16-token column
//   tiles), so every weight byte is read from HBM once and x (a few hundred
//   KB) comes from L2.  The k order inside a 32-wide MFMA step is free as long
//   as A and B agree: lane group g holds elements 8g..8g+7 of both, 16-byte
//   loads, 64 contiguous bytes of each weight row per load.  A ring of
//   register stages with fixed roles keeps several k-steps of loads in
//   flight ahead of the MFMAs; the last round's extra slots reload cached
//   weights against zero x instead of branching, so the compiler's
//   load-counter waits never drain the loads in flight.  The waves' sums
//   meet in LDS in a fixed order and go out as fp32 partials
//   [split][token][row].  proj_lds_kernel, the form for up to 32 tokens,
//   keeps x in registers and stages the weights through LDS instead.
// proj_finish_kernel: per (token, head), one 32-lane group sums the splits
//   in order, rounds to fp16 and then does what the append kernel does:
//   Q -> norm + RoPE -> q_out, Q_gate -> gate_out, K -> norm + RoPE -> its
//   page slot, V -> its page slot (and K, V as projected -> kv_out).
#include "k_common.h"
#include "k_normrope.h"
#include "kva_internal.h"

namespace kva {
namespace {

__device__ __forceinline__ half8_t as_h8(uint4 v) { return __builtin_bit_cast(half8_t, v); }

template <int NTB, int RT>
struct ProjStage {
    uint4 w[RT];   // 16-row weight tiles: row 16*i + lane%16, 8 elements
    uint4 x[NTB];  // 16-token tiles: token 16*j + lane%16, the same 8 elements
};

// This workgroup's weight row tiles: tile i holds rows 16*(grp*RT + i) ..
// +15 of the stacked [w_a; w_b] (a tile never straddles the two: n_a is a
// multiple of 16).  Tiles past the last one repeat it (live = false: loaded,
// never written), so every wave issues the same loads.  wt[i] points at
// this lane's row and first element.
template <int RT>
__device__ __forceinline__ void proj_tiles(const ProjectArgs &a, int grp, int lane_off,
                                           const uint16_t *(&wt)[RT], bool (&live)[RT]) {
    const int n_t16 = (a.n_a + a.n_b) / 16;
    const size_t hidden = static_cast<size_t>(a.hidden);
#pragma unroll
    for (int i = 0; i < RT; ++i) {
        const int t16 = grp * RT + i;
        live[i] = t16 < n_t16;
        const int row = 16 * min(t16, n_t16 - 1);
        const uint16_t *base = row < a.n_a ? a.w_a + static_cast<size_t>(row) * hidden
                                           : a.w_b + static_cast<size_t>(row - a.n_a) * hidden;
        wt[i] = base + lane_off;
    }
}

// Sum the waves' k ranges, one row tile at a time through LDS, in wave
// order; wave i % WAVES writes row tile i's partial [split][token][row].
template <int NTB, int WAVES, int RT>
__device__ __forceinline__ void proj_reduce_store(const ProjectArgs &a, float4_t (&acc)[RT][NTB],
                                                  float4_t (&red)[WAVES][NTB][64], const bool (&live)[RT],
                                                  int grp, int split, int wave, int lane) {
    const size_t N = static_cast<size_t>(a.n_a) + a.n_b;
    const int r = lane & 15, g = lane >> 4;
#pragma unroll
    for (int i = 0; i < RT; ++i) {
#pragma unroll
        for (int j = 0; j < NTB; ++j) red[wave][j][lane] = acc[i][j];
        __syncthreads();
        if (wave == i % WAVES && live[i]) {
#pragma unroll
            for (int j = 0; j < NTB; ++j) {
                float4_t sum = red[0][j][lane];
#pragma unroll
                for (int w = 1; w < WAVES; ++w) sum = sum + red[w][j][lane];
                const int t = 16 * j + r;
                if (t < a.n_tok) {
                    float *dst = a.part + (static_cast<size_t>(split) * a.n_tok + t) * N +
                                 16 * (grp * RT + i) + 4 * g;
                    *reinterpret_cast<float4_t *>(dst) = sum;
                }
            }
        }
        __syncthreads();
    }
}

// Load k-step `step` of this wave into a stage.  Steps past the wave's
// range (the ring's last round) reload the final step's weights (cache hits)
// and read x out of range (zeros), so their MFMAs add nothing and every
// round issues the same loads: no branch, exact load-counter waits.
template <int NTB, int RT>
__device__ __forceinline__ void proj_load(ProjStage<NTB, RT> &st, const uint16_t *const (&wt)[RT],
                                          __amdgpu_buffer_rsrc_t xr, const uint32_t (&xoff)[NTB], int step,
                                          int steps) {
    const int ks = min(step, steps - 1);
#pragma unroll
    for (int i = 0; i < RT; ++i) st.w[i] = ld16(wt[i] + 32 * ks);
#pragma unroll
    for (int j = 0; j < NTB; ++j) {
        const uint32_t off = step < steps ? xoff[j] + 64u * static_cast<uint32_t>(ks) : 0x80000000u;
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0);
        st.x[j] = make_uint4(v[0], v[1], v[2], v[3]);
    }
}

template <int NTB, int RT>
__device__ __forceinline__ void proj_mfma(float4_t (&acc)[RT][NTB], const ProjStage<NTB, RT> &st) {
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int j = 0; j < NTB; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(st.w[i]), as_h8(st.x[j]), acc[i][j], 0, 0, 0);
}

// General form.  Grid: ceil(rows / (16 * RT)) * splits workgroups of WAVES
// waves; each wave covers all 16 * RT rows of its workgroup for
// hidden / (splits * WAVES) elements of k.  The host checks
// hidden % (32 * WAVES * splits) == 0 and n_tok <= 16 * NTB.  A ring of
// DEPTH + 1 stages keeps DEPTH k-steps of loads in flight while one is
// multiplied.
template <int NTB, int WAVES, int DEPTH, int RT>
__global__ __launch_bounds__(64 * WAVES) void proj_gemm_kernel(ProjectArgs a) {
    constexpr int R = DEPTH + 1;
    __shared__ float4_t red[WAVES][NTB][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n_grp = ((a.n_a + a.n_b) / 16 + RT - 1) / RT;
    const int grp = blockIdx.x % n_grp;
    const int split = blockIdx.x / n_grp;
    const int steps = a.hidden / (32 * WAVES * a.splits);  // k-steps of this wave
    const int k0 = (split * WAVES + wave) * steps * 32;
    const int r = lane & 15, g = lane >> 4;
    const uint16_t *wt[RT];
    bool live[RT];
    proj_tiles<RT>(a, grp, r * a.hidden + k0 + 8 * g, wt, live);
    // x rows past n_tok lie outside the resource and load as zeros.
    const auto xr = ro_rsrc(a.x, static_cast<uint32_t>(a.n_tok) * static_cast<uint32_t>(a.hidden) * 2u);
    uint32_t xoff[NTB];
#pragma unroll
    for (int j = 0; j < NTB; ++j) xoff[j] = ((16 * j + r) * static_cast<uint32_t>(a.hidden) + k0 + 8 * g) * 2u;

    float4_t acc[RT][NTB];
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int j = 0; j < NTB; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

    // Slot j of round rr holds step rr*R + j.  Scheduling barriers keep each
    // group of loads ahead of the MFMAs after it; left alone, the scheduler
    // interleaves them and only a few loads stay in flight.
    ProjStage<NTB, RT> st[R];
#pragma unroll
    for (int j = 0; j < DEPTH; ++j) {
        __builtin_amdgcn_sched_barrier(0);
        proj_load(st[j], wt, xr, xoff, j, steps);
    }
    const int rounds = (steps + R - 1) / R;
    for (int rr = 0; rr < rounds; ++rr) {
#pragma unroll
        for (int j = 0; j < R; ++j) {
            __builtin_amdgcn_sched_barrier(0);
            proj_load(st[(j + DEPTH) % R], wt, xr, xoff, rr * R + j + DEPTH, steps);
            __builtin_amdgcn_sched_barrier(0);
            proj_mfma(acc, st[j]);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    proj_reduce_store<NTB, WAVES, RT>(a, acc, red, live, grp, split, wave, lane);
}

// The form for up to 32 tokens and STEPS k-steps per wave: each wave's x
// slice stays in registers for the whole kernel (loaded once at the start)
// and the weights stream one row tile at a time through LDS: a load
// instruction that writes LDS directly moves 8 rows x 128 contiguous bytes
// (two k-steps of one row tile), where a load into MFMA registers can carry
// only 64 bytes per row (4 lanes of a row x 16 B); each wave then reads its
// A operands back from its own ring of DEPTH + 1 two-step stages.  No wave
// reads another's ring, so a wave waits only for its own loads (no
// barrier).  Stage layout: row r's 16-byte granule g sits at granule
// g ^ ((r >> 1) & 7), so the 16 rows an A read takes at one granule fall in
// distinct banks.
template <int NTB, int WAVES, int RT, int STEPS, int DEPTH>
__global__ __launch_bounds__(64 * WAVES) void proj_lds_kernel(ProjectArgs a) {
    static_assert(STEPS % 2 == 0, "stages of two k-steps");
    constexpr int SPT = STEPS / 2;       // stages per row tile
    constexpr int N_ST = RT * SPT;       // stages of a wave
    constexpr int R = DEPTH + 1;
    constexpr int kStage = 16 * 128;     // 16 rows x 128 B
    __shared__ __attribute__((aligned(16))) uint8_t wlds[WAVES][R][kStage];
    __shared__ float4_t red[WAVES][NTB][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n_grp = ((a.n_a + a.n_b) / 16 + RT - 1) / RT;
    const int grp = blockIdx.x % n_grp;
    const int split = blockIdx.x / n_grp;
    const int k0 = (split * WAVES + wave) * STEPS * 32;
    const int r = lane & 15, g = lane >> 4;
    const int n_t16 = (a.n_a + a.n_b) / 16;
    const size_t hidden = static_cast<size_t>(a.hidden);
    // Row tile i's first row and first element of this wave (uniform), and
    // whether the tile exists (tiles past the end repeat the last one).
    const uint16_t *tb[RT];
    bool live[RT];
#pragma unroll
    for (int i = 0; i < RT; ++i) {
        const int t16 = grp * RT + i;
        live[i] = t16 < n_t16;
        const int row = 16 * min(t16, n_t16 - 1);
        tb[i] = (row < a.n_a ? a.w_a + static_cast<size_t>(row) * hidden
                             : a.w_b + static_cast<size_t>(row - a.n_a) * hidden) + k0;
    }
    // Load lane mapping: instruction h of a stage covers rows 8h + lane/8;
    // lane lands at physical granule lane%8, so it fetches logical granule
    // (lane%8) ^ ((row >> 1) & 7).
    uint32_t loff[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int row = 8 * h + (lane >> 3);
        const int gl = (lane & 7) ^ ((row >> 1) & 7);
        loff[h] = (row * static_cast<uint32_t>(a.hidden) + 8 * gl) * 2u;
    }
    const uint32_t rbytes = 16u * static_cast<uint32_t>(a.hidden) * 2u;
    auto issue = [&](int n) {
        const int i = n / SPT, q = n % SPT;
        const auto rs = ro_rsrc(tb[i] + 64 * q, rbytes);
        const uint32_t dst = lds_addr(&wlds[wave][n % R][0]);
        load_to_lds(rs, dst, loff[0]);
        load_to_lds(rs, dst + 1024, loff[1]);
    };

    // The first DEPTH weight stages go out before x: the weights come from
    // HBM and x from L2, so both are in flight together.  Taking delivery
    // of x below then also waits for these stages (loads complete in
    // order); the ring's waits are upper bounds and stay exact after that.
#pragma unroll
    for (int n = 0; n < DEPTH; ++n) issue(n);
    const auto xr = ro_rsrc(a.x, static_cast<uint32_t>(a.n_tok) * static_cast<uint32_t>(a.hidden) * 2u);
    uint4 xv[STEPS][NTB];
#pragma unroll
    for (int st = 0; st < STEPS; ++st)
#pragma unroll
        for (int j = 0; j < NTB; ++j) {
            const uint32_t off = ((16 * j + r) * static_cast<uint32_t>(a.hidden) + k0 + 8 * g + 32 * st) * 2u;
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0);
            xv[st][j] = make_uint4(v[0], v[1], v[2], v[3]);
        }
    // Take delivery of x before the ring starts: the compiler cannot see the
    // LDS loads, and a wait for x placed later would drain them.
#pragma unroll
    for (int st = 0; st < STEPS; ++st)
#pragma unroll
        for (int j = 0; j < NTB; ++j)
            asm volatile("" : "+v"(xv[st][j].x), "+v"(xv[st][j].y), "+v"(xv[st][j].z), "+v"(xv[st][j].w));
    float4_t acc[RT][NTB];
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int j = 0; j < NTB; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

    // A reads: row r at logical granule 4*s + g of a stage's two steps.
    const int sw = (r >> 1) & 7;
#pragma unroll
    for (int n = 0; n < N_ST; ++n) {
        __builtin_amdgcn_sched_barrier(0);
        if (n + DEPTH < N_ST) {  // resolved at compile time after unrolling
            issue(n + DEPTH);
            wait_vm<2 * DEPTH>();
        } else {
            wait_vm<0>();  // the last stages: everything is issued
        }
        __builtin_amdgcn_sched_barrier(0);
        const uint8_t *sb = &wlds[wave][n % R][0] + r * 128;
        const int i = n / SPT, q = n % SPT;
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
            const uint4 w4 = *reinterpret_cast<const uint4 *>(sb + 16 * ((4 * s2 + g) ^ sw));
#pragma unroll
            for (int j = 0; j < NTB; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(w4), as_h8(xv[2 * q + s2][j]), acc[i][j],
                                                                 0, 0, 0);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    proj_reduce_store<NTB, WAVES, RT>(a, acc, red, live, grp, split, wave, lane);
}

// Grid: (token, block of 8 head rows) per 256-thread workgroup; one 32-lane
// group per head row.  Head rows of a token: H query, H gate, Hkv key, Hkv
// value heads (the order of the weight rows).  The token's metadata and
// page id are workgroup-uniform, read through the scalar cache while the
// partials are in flight.
__global__ __launch_bounds__(256) void proj_finish_kernel(ProjectArgs a) {
    const int H = a.num_heads, hkv = a.num_kv_heads;
    const int rows_per_tok = 2 * H + 2 * hkv;
    const int blocks_per_tok = (rows_per_tok + 7) / 8;
    const int tc = blockIdx.x / blocks_per_tok;
    const int hr = (blockIdx.x - tc * blocks_per_tok) * 8 + (threadIdx.x >> 5);
    const int lane = threadIdx.x & 31;
    if (hr >= rows_per_tok) return;  // whole 32-lane group leaves
    const int t = a.tok0 + tc;
    // Two memory round trips before the stores.  First: every split's
    // partial (splits past a.splits reread split 0 and are not added) and
    // the norm weights, which need only the kernel arguments, with the
    // token's position, sequence and slot; then cos/sin and the page id.
    // (Requested in source order, the partials waited for the page id, which
    // waited for the sequence and slot: three round trips.)
    const size_t N = static_cast<size_t>(a.n_a) + a.n_b;
    const size_t row_at = static_cast<size_t>(tc) * N + static_cast<size_t>(hr) * kHeadDim + 8 * lane;
    const size_t split_stride = static_cast<size_t>(a.n_tok) * N;
    const int splits = a.splits;
    float4_t plo[kProjMaxSplits], phi[kProjMaxSplits];
#pragma unroll
    for (int s = 0; s < kProjMaxSplits; ++s) {
        const float *ps = a.part + row_at + (s < splits ? s : 0) * split_stride;
        plo[s] = *reinterpret_cast<const float4_t *>(ps);
        phi[s] = *reinterpret_cast<const float4_t *>(ps + 4);
    }
    const uint16_t *w = hr < H ? a.q_w : a.k_w;  // gate and value rows load and ignore them
    NormRopeIn nin;
    nin.w = ld16(w + 8 * lane);
    const int stride = a.table_stride, half_rot = a.half_rot;
    const int pos = ld_uniform(a.tok_pos + t);
    const int seq = ld_uniform(a.tok_seq + t);
    const int slot = ld_uniform(a.tok_slot + t);
    asm volatile("" ::"s"(pos), "s"(seq), "s"(slot), "s"(stride), "s"(half_rot));  // taken in together
    __builtin_amdgcn_sched_barrier(0);
    rope_in_flat(nin, w, a.cos_tab + static_cast<size_t>(pos) * half_rot, a.sin_tab + static_cast<size_t>(pos) * half_rot,
                 half_rot, lane);
    const int blk = ld_uniform(a.table + static_cast<size_t>(seq) * stride + (slot >> 4));
    uint4 y;
    {
        float4_t lo = plo[0], hi = phi[0];
#pragma unroll
        for (int s = 1; s < kProjMaxSplits; ++s) {
            lo = s < splits ? lo + plo[s] : lo;
            hi = s < splits ? hi + phi[s] : hi;
        }
        y.x = pack_h2(lo[0], lo[1]);
        y.y = pack_h2(lo[2], lo[3]);
        y.z = pack_h2(hi[0], hi[1]);
        y.w = pack_h2(hi[2], hi[3]);
    }

    if (hr < H) {
        const uint4 q = norm_rope_apply<32>(y, nin, a.half_rot, a.eps, lane);
        st16(a.q_out + (static_cast<size_t>(t) * H + hr) * kHeadDim + 8 * lane, q);
        return;
    }
    if (hr < 2 * H) {
        if (a.gate_out) st16(a.gate_out + (static_cast<size_t>(t) * H + hr - H) * kHeadDim + 8 * lane, y);
        return;
    }
    const int kv = hr - 2 * H;  // 0..2*Hkv-1: K heads, then V heads
    if (a.kv_out) st16(a.kv_out + (static_cast<size_t>(t) * 2 * hkv + kv) * kHeadDim + 8 * lane, y);
    const size_t row_base = (static_cast<size_t>(blk) * kBlockTokens + (slot & 15)) * hkv;
    if (kv < hkv) {
        const uint4 k = norm_rope_apply<32>(y, nin, a.half_rot, a.eps, lane);
        st16(a.k_pool + (row_base + kv) * kHeadDim + 8 * lane, k);
    } else {
        st16(a.v_pool + (row_base + kv - hkv) * kHeadDim + 8 * lane, y);
    }
}

// Grid: 8 consecutive output rows of one token per thread.  y = fp16(the
// split partials summed in split order + residual): one rounding after the
// residual add, the epilogue of the reference GEMV (gemv_fp16_v2.hip:81-86).
// A thread reads its residual before writing the same 16 bytes, so the
// residual may be the output (in place, d_hidden += o_proj(attn)).
__global__ __launch_bounds__(256) void oproj_finish_kernel(ProjectArgs a) {
    const int per_tok = a.n_a / 8;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= a.n_tok * per_tok) return;
    const int tc = i / per_tok;
    const size_t N = static_cast<size_t>(a.n_a);
    const size_t row = static_cast<size_t>(i - tc * per_tok) * 8;
    const size_t at = static_cast<size_t>(a.tok0 + tc) * N + row;
    const uint4 r = a.residual ? ld16(a.residual + at) : make_uint4(0, 0, 0, 0);
    const size_t split_stride = static_cast<size_t>(a.n_tok) * N;
    const float *p = a.part + static_cast<size_t>(tc) * N + row;
    float4_t plo[kProjMaxSplits], phi[kProjMaxSplits];
#pragma unroll
    for (int s = 0; s < kProjMaxSplits; ++s) {
        const float *ps = p + (s < a.splits ? s : 0) * split_stride;
        plo[s] = *reinterpret_cast<const float4_t *>(ps);
        phi[s] = *reinterpret_cast<const float4_t *>(ps + 4);
    }
    float4_t lo = plo[0], hi = phi[0];
#pragma unroll
    for (int s = 1; s < kProjMaxSplits; ++s) {
        lo = s < a.splits ? lo + plo[s] : lo;
        hi = s < a.splits ? hi + phi[s] : hi;
    }
    if (a.residual) {
        lo += float4_t{lo_f(r.x), hi_f(r.x), lo_f(r.y), hi_f(r.y)};
        hi += float4_t{lo_f(r.z), hi_f(r.z), lo_f(r.w), hi_f(r.w)};
    }
    uint4 y;
    y.x = pack_h2(lo[0], lo[1]);
    y.y = pack_h2(lo[2], lo[3]);
    y.z = pack_h2(hi[0], hi[1]);
    y.w = pack_h2(hi[2], hi[3]);
    st16(a.y_out + at, y);
}

// Split-K partials of x [n_tok][hidden] against the stacked weight rows.
hipError_t launch_proj_gemm(const ProjectArgs &a, hipStream_t s) {
    constexpr int W = kProjWaves, P = kProjDepth, RT = kProjRowTiles, LD = kProjLdsDepth;
    const int n_t16 = (a.n_a + a.n_b) / 16;
    const dim3 grid(static_cast<unsigned>((n_t16 + RT - 1) / RT * a.splits));
    const dim3 block(64 * W);
    const int ntb = (a.n_tok + 15) / 16;
    if (ntb <= 2 && a.hidden == kProjStreamSteps * 32 * W * a.splits) {
        constexpr int ST = kProjStreamSteps;
        if (ntb == 1) hipLaunchKernelGGL((proj_lds_kernel<1, W, RT, ST, LD>), grid, block, 0, s, a);
        else hipLaunchKernelGGL((proj_lds_kernel<2, W, RT, ST, LD>), grid, block, 0, s, a);
    } else if (ntb <= 2 && a.hidden == kProjStreamStepsB * 32 * W * a.splits) {
        constexpr int ST = kProjStreamStepsB, RB = kProjRowTilesB;
        const dim3 grid_b(static_cast<unsigned>((n_t16 + RB - 1) / RB * a.splits));
        if (ntb == 1) hipLaunchKernelGGL((proj_lds_kernel<1, W, RB, ST, LD>), grid_b, block, 0, s, a);
        else hipLaunchKernelGGL((proj_lds_kernel<2, W, RB, ST, LD>), grid_b, block, 0, s, a);
    } else switch (ntb) {
        case 1: hipLaunchKernelGGL((proj_gemm_kernel<1, W, P, RT>), grid, block, 0, s, a); break;
        case 2: hipLaunchKernelGGL((proj_gemm_kernel<2, W, P, RT>), grid, block, 0, s, a); break;
        case 3: hipLaunchKernelGGL((proj_gemm_kernel<3, W, P, RT>), grid, block, 0, s, a); break;
        case 4: hipLaunchKernelGGL((proj_gemm_kernel<4, W, P, RT>), grid, block, 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

// The GEMM of a launch pair between the caller's timing events (if any).
hipError_t launch_proj_gemm_timed(const ProjectArgs &a, hipStream_t s) {
    if (a.ev_before) {
        const hipError_t e = hipEventRecord(a.ev_before, s);
        if (e != hipSuccess) return e;
    }
    const hipError_t e = launch_proj_gemm(a, s);
    if (e != hipSuccess || !a.ev_after) return e;
    return hipEventRecord(a.ev_after, s);
}

hipError_t launch_project(const ProjectArgs &a, hipStream_t s) {
    if (a.n_tok <= 0) return hipSuccess;
    const hipError_t e = launch_proj_gemm_timed(a, s);
    if (e != hipSuccess) return e;
    const int blocks_per_tok = (2 * a.num_heads + 2 * a.num_kv_heads + 7) / 8;
    hipLaunchKernelGGL(proj_finish_kernel, dim3(a.n_tok * blocks_per_tok), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_out_project(const ProjectArgs &a, hipStream_t s) {
    if (a.n_tok <= 0) return hipSuccess;
    if (a.n_b != 0 || a.n_a % 16 != 0) return hipErrorInvalidValue;
    const hipError_t e = launch_proj_gemm_timed(a, s);
    if (e != hipSuccess) return e;
    const int threads = a.n_tok * (a.n_a / 8);
    hipLaunchKernelGGL(oproj_finish_kernel, dim3((threads + 255) / 256), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace kva
