// Internal interface between the host side of libkvattn (kva_host.cpp, built
// with g++) and the HIP kernels (k_*.hip, built with hipcc for gfx950).
// Only plain types cross this boundary: fp16 tensors are uint16_t pointers.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>

namespace kva {

constexpr int kHeadDim = 256;     // the only head_dim the paged kernels take
constexpr int kBlockTokens = 16;  // tokens per page
constexpr int kDecodeHeadsPerWg = 4;  // kv heads per stream-K decode workgroup (one wave each), at most
constexpr int kSplitQuantum = 16; // decode split sizes are whole pages
constexpr int kCombineRecs = 64;  // sequences whose combine facts travel in the decode arguments
constexpr int kPlanPages = 64;    // page ids per sequence in the step plan (one per lane)
constexpr int kCombineChunk = 16; // decode partials a combine wave requests together

// Fused QK-RMSNorm + RoPE + K/V append over all new tokens of a step.
struct AppendArgs {
    uint16_t *q;              // [T][H][256], normalised + rotated in place
    uint16_t *k;              // [T][Hkv][256], normalised + rotated in place
    const uint16_t *v;        // [T][Hkv][256]
    const uint16_t *q_w;      // [256]
    const uint16_t *k_w;      // [256]
    const uint16_t *cos_tab;  // [rows][half_rot]
    const uint16_t *sin_tab;
    uint16_t *k_pool;         // this layer's pool [blocks][16][Hkv][256]
    uint16_t *v_pool;
    const int32_t *table;     // [max_seqs][table_stride]
    int32_t table_stride;
    const int32_t *tok_seq;   // device: sequence id of each new token
    const int32_t *tok_slot;  // device: logical slot of each new token
    const int32_t *tok_pos;   // device: RoPE position of each new token
    int32_t n_tok;
    int32_t num_heads;
    int32_t num_kv_heads;
    int32_t half_rot;
    float eps;
    int32_t keep_k;           // 1: k is read only (the cache gets the normalised rows)
};
hipError_t launch_append(const AppendArgs &a, hipStream_t s);

// Q/K/V projection of a step's tokens fused with norm + RoPE + K/V append.
// Weight rows: w_a = [Q heads | Q_gate heads] (n_a = 2*H*256 rows), w_b =
// [K heads | V heads] (n_b = 2*Hkv*256 rows), each row `hidden` fp16.  One
// launch pair covers up to kProjTokens tokens: proj_gemm_kernel writes
// split-K fp32 partials, proj_finish_kernel sums them in split order, rounds
// to fp16 (the projection the reference's GEMV stores) and finishes each head.
constexpr int kProjTokens = 64;     // tokens per launch pair (4 MFMA column tiles)
constexpr int kProjMaxSplits = 4;   // hidden split among workgroups, at most
constexpr int kProjWaves = 8;       // waves per GEMM workgroup
constexpr int kProjRowTiles = 7;    // 16-row weight tiles per GEMM workgroup
constexpr int kProjDepth = 1;       // k-steps of loads in flight per wave (general form)
constexpr int kProjHiddenQuantum = 512;  // hidden must be a multiple of this
constexpr int kProjWgPerCu = 1;     // GEMM workgroups per CU the split aims for, at most
constexpr int kProjStreamSteps = 10;  // k-steps per wave of the x-resident form (up to 32 tokens)
constexpr int kProjLdsDepth = 6;      // two-step LDS stages in flight per wave there
// The same form over 6 k-steps per wave (hidden 6144 at four splits: the
// O-projection from 24 heads), with 5 row tiles per workgroup so that 5120
// output rows still make 256 workgroups.
constexpr int kProjStreamStepsB = 6;
constexpr int kProjRowTilesB = 5;
struct ProjectArgs {
    const uint16_t *x;        // [n_tok][hidden], this chunk's first token
    const uint16_t *w_a;
    const uint16_t *w_b;
    int32_t n_a, n_b;
    int32_t hidden;
    int32_t n_tok;            // tokens of this chunk, 1..kProjTokens
    int32_t splits;
    float *part;              // [splits][n_tok][n_a + n_b]
    int32_t tok0;             // the chunk's first token within the step
    uint16_t *q_out;          // [T][H][256]: normalised + rotated Q
    uint16_t *gate_out;       // [T][H][256]: Q_gate as projected (nullable)
    uint16_t *kv_out;         // [T][2][Hkv][256]: K, V as projected (nullable)
    const uint16_t *q_w;
    const uint16_t *k_w;
    const uint16_t *cos_tab;
    const uint16_t *sin_tab;
    uint16_t *k_pool;
    uint16_t *v_pool;
    const int32_t *table;
    int32_t table_stride;
    const int32_t *tok_seq;
    const int32_t *tok_slot;
    const int32_t *tok_pos;
    int32_t num_heads;
    int32_t num_kv_heads;
    int32_t half_rot;
    float eps;
    // Output projection (launch_out_project; w_a = W_o, n_b = 0): y_out =
    // fp16(x W_o^T + residual), both [T][n_a]; residual nullable, may be y_out.
    uint16_t *y_out;
    const uint16_t *residual;
    // Events around the GEMM kernel of a launch pair (null: none), as in
    // DecodeArgs.
    hipEvent_t ev_before, ev_after;
};
hipError_t launch_project(const ProjectArgs &a, hipStream_t s);
hipError_t launch_out_project(const ProjectArgs &a, hipStream_t s);
// Prefill-sized steps (more than kProjTokens tokens): one GEMM launch over
// every token, tiles of kBigTileTokens tokens x one head's 256 weight rows,
// with the finish kernel's epilogue (fp16 rounding, norm + RoPE, outputs,
// cache rows) done by the workgroup that computed the tile (k_gemm.hip).
// Needs (n_a + n_b) % 256 == 0 and hidden % 64 == 0; a.tok0 = 0.
constexpr int kBigTileTokens = 256;
constexpr int kBigProjMaxTokens = 1 << 24;
hipError_t launch_project_big(const ProjectArgs &a, hipStream_t s);

// Reference-compatible norm+RoPE on a contiguous [n_heads][head_dim] buffer.
struct LegacyNormArgs {
    uint16_t *x;
    const uint16_t *w;
    const uint16_t *cos_row;
    const uint16_t *sin_row;
    uint16_t *cache_dst;      // nullable
    int32_t num_heads;
    int32_t head_dim;         // 64, 128 or 256
    int32_t half_rot;
    float eps;
};
hipError_t launch_legacy_norm(const LegacyNormArgs &a, hipStream_t s);

// Split-K GQA decode over a paged (or contiguous) cache.
struct DecodeArgs {
    const uint16_t *q;        // [n_seqs][H][256]
    const uint16_t *k_pool;   // layer base (or contiguous K when table == null)
    const uint16_t *v_pool;
    const int32_t *table;     // device block table, null = contiguous cache
    int32_t table_stride;
    size_t seq_stride;        // contiguous cache: elements between sequences
    const int32_t *seq_ids;   // device [n_seqs] (ignored when table == null)
    const int32_t *ctx_lens;  // device [n_seqs] (null: use ctx_len_const)
    const int32_t *pre_seq;   // device [n_seqs+1]: pages of earlier sequences
                              // (null: every sequence has ctx_len_const)
    // Device [n_seqs][kPlanPages] (null: read the table): the block ids of
    // each sequence's first kPlanPages pages, copied from the table into the
    // step plan when the step began (zeros past its pages), so the
    // whole-sequence form reads them with the length instead of after the
    // sequence id.
    const int32_t *plan_pages;
    int32_t ctx_len_const;
    int32_t n_seqs;
    int32_t num_heads;
    int32_t num_kv_heads;
    int32_t total_pages;      // pages of all sequences (one page = 16 token rows)
    int32_t n_wg;             // workgroups sharing the pages (stream-K)
    // dyn = 1 (a launch recorded into a replayable graph): total_pages is
    // read from pre_seq[n_seqs] on the device and the workgroup count derived
    // there from split_tokens / min_pages, with n_wg as the cap (the grid).
    int32_t dyn;
    int32_t split_tokens;     // 0 = one workgroup per CU up to the cap
    int32_t min_pages;
    // 1 (the host has shown that no sequence is cut into more than
    // kCombineChunk pieces): the combine launch has a workgroup per
    // (sequence, kv head) with a wave per query head; else a workgroup of
    // four waves per (sequence, kv head, query head).
    int32_t combine_waves;
    // The combine's view of each sequence, in the kernel arguments so its
    // first loads are the partials (n_crec = n_seqs <= kCombineRecs; 0: it
    // reads the length from the step plan and derives these): crec[b] = the
    // workgroup of the sequence's first piece, -1 when one workgroup covered
    // it; crec_n[b] = 2 * pieces + 1 if the first piece's slot is 2*w0 + 1.
    int32_t n_crec;
    int32_t crec[kCombineRecs];
    int32_t crec_n[kCombineRecs];
    float *ws_acc;            // [2*n_wg][Hkv][G][256] partial slots
    float *ws_ml;             // [2*n_wg][Hkv][G][2]
    uint16_t *out;            // [n_seqs][H][256]
    // Output gate (null = none): out = fp16(fp16(attn) * sigmoid(gate)), the
    // gate row of sequence b, query head hq at gate + b*gate_stride + hq*256.
    const uint16_t *gate;
    int64_t gate_stride;
    // Per-workgroup timeline (null = off): record kTimelineWords words per
    // wave, [n_wg][grid rows][8 waves], see kva_timeline_read.
    uint64_t *timeline;
    // > 0: whole-sequence form, one workgroup per (sequence, kv head, group
    // of G / whole query heads): no partials, no combine; the stream-K
    // fields are unused.  G / whole must be 1, 2, 3, 4, 6 or 8.
    int32_t whole;
    // Events recorded on the stream right before and after the decode
    // kernel itself (null: none): the dominant kernel's own duration.
    hipEvent_t ev_before, ev_after;
    // 1 (whole form only): the step's append is done in the same launch
    // from `app` (one new token per sequence, token b of sequence b): each
    // workgroup normalises and rotates its query rows (written back in
    // place, q = app.q) and its kv head's new K row, the first group of each
    // (sequence, kv head) writes the new K and V rows to the cache, and the
    // new token joins the attention from registers, not from the cache.
    int32_t fused;
    AppendArgs app;
};
constexpr int kTimelineWords = 4;
constexpr int kWholeWaves = 8;  // waves per whole-sequence decode workgroup
hipError_t launch_decode(const DecodeArgs &a, hipStream_t s);

// Static device scratch of kva_legacy_decode_noalloc (k_noalloc.hip): the
// decode partial slots [2*n_wg][H][256] floats, then [2*n_wg][H][2].
constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
constexpr int kNoAllocMaxHeads = 128;  // query heads it serves, at most
// The current device's scratch address (fetched once per device with
// hipGetSymbolAddress) and its CU count.
hipError_t noalloc_scratch(void **ptr, int *n_cu);

// Apply block-table patches (seq, index, block) staged by a step.
hipError_t launch_table_patch(int32_t *table, int32_t table_stride,
                              const int32_t *patches, int32_t n_patches,
                              hipStream_t s);

// Streaming device copy (bytes multiple of 16): the HBM bandwidth probe.
hipError_t launch_copy(void *dst, const void *src, size_t bytes, hipStream_t s);
// Read-only stream over `bytes` (multiple of 16): the read-bandwidth probe.
// sink: one word, written only when the data's XOR fold hits a fixed value.
hipError_t launch_read(const void *src, size_t bytes, uint32_t *sink, hipStream_t s);
// Paged read probe: the pages page_ids[0 .. n_pages) (device array) of the
// K and V pools, [page][16][num_kv_heads][256] fp16, read with the stream-K
// decode's per-wave pattern by n_wg workgroups of one wave per kv head.
hipError_t launch_read_pages(const void *k_pool, const void *v_pool, const int32_t *page_ids, int32_t n_pages,
                             int32_t num_kv_heads, int32_t n_wg, uint32_t *sink, hipStream_t s);

// Move accepted rows of each sequence, in every layer (tree rollback).
struct RollbackArgs {
    uint16_t *k_pools;        // base of layer 0; layers are layer_elems apart
    uint16_t *v_pools;
    size_t layer_elems;
    int32_t n_layers;
    const int32_t *table;
    int32_t table_stride;
    const int32_t *moves;     // device [n_moves][3]: seq, src slot, dst slot
    const int32_t *move_off;  // device [n_groups+1]: moves of one sequence
    int32_t n_groups;
    int32_t num_kv_heads;
};
hipError_t launch_rollback(const RollbackArgs &a, hipStream_t s);

// Multi-query (prefill / tree) attention with MFMA tiles.
struct MultiQueryArgs {
    const uint16_t *q;        // [T][H][256]
    uint16_t *out;            // [T][H][256]
    const uint16_t *k_pool;
    const uint16_t *v_pool;
    const int32_t *table;
    int32_t table_stride;
    const int32_t *seq_ids;   // device [n_seqs]
    const int32_t *ctx_lens;  // device [n_seqs]: length after the step
    const int32_t *new_start; // device [n_seqs]: first new slot
    const int32_t *tok_off;   // device [n_seqs+1]: new-token ranges
    const uint64_t *tok_bits; // device [T] (tree mode) or null
    const int32_t *upre;      // device [n_seqs+1]: tiles of earlier sequences (units of one head)
    const int32_t *mq_pre;    // device [n_units+1]: positions of earlier units (blocks + mq_unit_cost each)
    // Device [n_cut][kMqCutWords]: the units cut across workgroups, as
    // kva_step_begin found them from the shares of n_wg (head, first new
    // token of the tile, its valid tokens, first and last share, first
    // piece's slot); the combine launch has one row of workgroups per cut unit.
    const int32_t *mq_cut;
    int32_t n_cut;
    int32_t n_seqs;
    int32_t n_units;          // (kv head, sequence, token tile) units, head-major
    int32_t total_blocks;     // positions of all units (blocks + mq_unit_cost each)
    int32_t keys;             // keys per block: mq_keys_for(n_waves, the step has tree bits)
    int32_t n_wg;             // workgroups sharing the blocks (stream-K)
    int32_t num_heads;
    int32_t num_kv_heads;
    int32_t tree;             // 0 = causal chunk, 1 = tree mask
    int32_t n_waves;          // waves per workgroup (4 or 8)
    int32_t n_t;              // 16-row MFMA tiles per wave (1: the form launched)
    int32_t q_tile;           // new tokens per unit tile: mq_tile_tokens(G, n_waves, n_t)
    float *ws_acc;            // [2*n_wg][kMqSlotRows][256] partial slots
    float *ws_ml;             // [2*n_wg][kMqSlotRows][2]
    // Output gate (null = none), as in DecodeArgs: new token t's row of
    // query head hq at gate + t*gate_stride + hq*256.
    const uint16_t *gate;
    int64_t gate_stride;
    // Events around mq_kernel itself (null: none), as in DecodeArgs.
    hipEvent_t ev_before, ev_after;
};
// Keys per multi-query block.  64 for a step of eight-wave prefill tiles
// (half the barriers, page lookups and softmax reductions per key, two LDS
// stages of 66 KB: config 4 115.5 -> 110.4 us per call); 32 otherwise, a
// four-stage ring that keeps 96 KB in flight for the HBM-bound tree verify
// (config 5 at 64 keys: 862 -> 888 us) and for small steps.  A step planned
// with tree bits uses 32 for kva_prefill too.
constexpr int mq_keys_for(int waves, bool tree_plan) { return (waves == 8 && !tree_plan) ? 64 : 32; }
// The stream-K split of the multi-query kernel counts each unit as the
// blocks of 128 more keys than it has (the cost of starting a unit: its
// query rows, its output), so a share full of short units gets fewer
// blocks.  Unit u's blocks sit at positions [mq_pre[u] + cost, mq_pre[u+1]).
// 128 keys: a unit start measured about two 32-key blocks' time, but with
// two the shares holding many short units still ended last (config 4 at 32
// keys per block, cost 2 -> 132 us, 3 -> 122, 4 -> 116, 5 and 6 -> 116-117).
constexpr int mq_unit_cost(int keys) { return 128 / keys; }
constexpr int kMqMaxGroup = 8;    // largest GQA group of the multi-query kernel
constexpr int kMqSlotRows = 128;  // query rows of a partial slot (waves x 16 x tiles at most)
constexpr int kMqCutWords = 8;    // int32 words of a cut-unit record (6 used)
// Workgroups of a multi-query launch over `blocks` positions: one per CU (the
// cap), at least 128 keys' blocks each.  kva_step_begin (the cut-unit
// records) and the launch must agree.
inline int32_t mq_wg_count(int64_t blocks, int32_t keys, int32_t cap) {
    const int64_t min_blocks = 128 / keys;
    const int64_t w = (blocks + min_blocks - 1) / min_blocks;
    return static_cast<int32_t>(w < 1 || cap < 1 ? 1 : (w > cap ? cap : w));
}
// First position of share w of W over n positions (the device's mq_wg_start).
inline int32_t mq_share_start(int64_t w, int64_t n, int64_t W) { return static_cast<int32_t>(w * n / W); }
// A unit's query rows are (token, head) pairs of the GQA group, 16 per
// MFMA tile, n_t tiles per wave: tokens per unit tile.
constexpr int mq_tile_tokens(int G, int n_waves, int n_t) { return 16 * n_waves * n_t / G; }
// Waves for a step whose longest new-token run is max_new: four (one per
// SIMD) when a whole run fits one unit of 64 rows (tree verify), else eight
// (128 rows; two waves per SIMD hide each other's softmax and LDS waits).
constexpr int mq_waves_for(int G, int max_new) { return max_new * G <= 64 ? 4 : 8; }
hipError_t launch_multi_query(const MultiQueryArgs &a, hipStream_t s);

}  // namespace kva
