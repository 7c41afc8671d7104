// Host side of libkvattn: the paged block pool, per-sequence block tables and
// lengths, per-step plans, argument validation and the C ABI of kvattn.h.
// Built with g++ against the HIP runtime API; kernels live in k_*.hip.
//
// Reference behaviour restated here:
//   - KVCache (engine.py:79-291): one contiguous [max_seq][kv_heads][256]
//     region per layer and batch slot, one shared current_len; here a pool of
//     16-token pages per layer with a block table and a length per sequence.
//   - the C dispatch loop's per-step argument patching (c_dispatch.c:426-456,
//     used at :1066-1103): here one host->device copy of a step plan that all
//     layers of the step read.
//   - HIP errors raise (hip_dispatch.py:267-269) -> here every call returns a
//     code and kva_last_error_string() says why; no silent fallbacks.
#include "../../include/kvattn.h"
#include "kva_internal.h"

#include <algorithm>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

namespace {

thread_local std::string g_err;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_fail(hipError_t e, const char *what) {
    return fail(static_cast<int>(e), "%s: %s (hipError %d)", what, hipGetErrorString(e),
                static_cast<int>(e));
}

#define KVA_HIP(call)                                         \
    do {                                                      \
        hipError_t e_ = (call);                               \
        if (e_ != hipSuccess) return hip_fail(e_, #call);     \
    } while (0)

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

constexpr int kStageSlots = 4;
constexpr int kDecodeWgPerCu = 1;   // stream-K decode workgroups per CU

constexpr int kMinPagesPerWg = 1;   // a short sequence still spreads over several CUs
// A decode step (automatic split) whose longest sequence has at most this
// many rows runs the whole-sequence form: one workgroup per sequence and kv
// head, no partials and no combine launch.
constexpr int kWholeMaxTokens = 1024;
// The CU count a host-only cache validates against (MI355X).
constexpr int kHostOnlyCus = 256;

}  // namespace

struct kva_cache {
    kva_config cfg{};
    bool host_only = false;
    int group = 0;  // query heads per KV head
    size_t row_elems = 0;
    size_t layer_elems = 0;

    // device memory
    uint16_t *d_k = nullptr;
    uint16_t *d_v = nullptr;
    int32_t *d_table = nullptr;
    uint8_t *d_step = nullptr;
    size_t step_bytes = 0;
    uint8_t *d_aux = nullptr;
    size_t aux_bytes = 0;
    float *d_ws_acc = nullptr;
    float *d_ws_ml = nullptr;
    uint64_t *d_timeline = nullptr;  // decode timeline records (kva_timeline_enable)
    float *d_mq_acc = nullptr;  // multi-query partial slots [2*mq_max_wg][8][16][256]
    float *d_mq_ml = nullptr;
    int32_t mq_max_wg = 0;
    float *d_proj = nullptr;    // projection partials [kProjMaxSplits][kProjTokens][(2H+2Hkv)*256]
    size_t proj_floats = 0;
    int32_t last_proj_path = 0;  // KVA_PROJECT_KERNELS or KVA_PROJECT_PREFILL_GEMM
    int32_t max_wg = 0;  // decode workgroups the partial workspace can serve
    size_t ws_rows = 0;  // 256-float rows in the decode partial workspace
    int32_t n_cu = 0;

    // pinned staging ring
    uint8_t *h_stage[kStageSlots] = {};
    hipEvent_t ev[kStageSlots] = {};
    bool ev_live[kStageSlots] = {};
    int stage_next = 0;
    size_t stage_bytes = 0;

    // host bookkeeping
    std::vector<int32_t> table;   // [max_seqs][max_blocks_per_seq]
    std::vector<int32_t> nblk;    // blocks held per sequence
    std::vector<int32_t> len;     // committed length per sequence
    std::vector<uint8_t> freed;   // sequence released by kva_seq_free
    std::vector<uint8_t> used;    // per block
    std::vector<int32_t> free_list;
    std::vector<int32_t> patches; // pending (seq, idx, block) triples

    // current step plan
    bool step_valid = false;
    int32_t st_n_seqs = 0, st_n_tok = 0, st_max_ctx = 0, st_max_new = 0, st_max_pos = 0;
    int32_t st_total_pages = 0;  // pages of all sequences of the step
    int32_t st_mq_units = 0;     // (sequence, token tile, kv head) units
    int32_t st_mq_wg = 0;        // workgroups of the step's multi-query launch
    int32_t st_mq_cut = 0;       // its units cut across workgroups (records at off_cut)
    int32_t st_mq_blocks = 0;    // key blocks (and unit start costs) of all multi-query units
    int32_t st_mq_waves = 4;     // waves per workgroup of the multi-query kernel
    int32_t st_mq_keys = 32;     // keys per multi-query block (mq_keys_for)
    int32_t st_mq_q = 0;         // new tokens per unit tile
    size_t off_upre = 0, off_mqpre = 0;
    bool st_all_one = false, st_has_bits = false;
    std::vector<int32_t> st_pre;  // pages of the step's earlier sequences, [n_seqs + 1]
    size_t off_seq = 0, off_ctx = 0, off_start = 0, off_tokoff = 0, off_tseq = 0,
           off_tslot = 0, off_tpos = 0, off_bits = 0, off_pre = 0, off_pids = 0, off_cut = 0;

    // Caller's timing events around the dominant kernel of each hot call
    // (kva_kernel_events); null: none.
    hipEvent_t kev_before = nullptr, kev_after = nullptr;

    int32_t split_user = 0;  // decode tokens per workgroup (0 = automatic)
    int32_t last_split = 0, last_nwg = 0;
    bool last_whole = false;  // the last decode ran the whole-sequence form

    // Graph recording (kva_graph_capture_begin .. _end) on `cap_stream`.
    bool capturing = false;
    bool capture_failed = false;
    hipStream_t cap_stream = nullptr;
    int32_t cap_table_rows = 0;  // fewest RoPE table rows any recorded append was given
};

// A recorded step: the launches of one step's per-layer calls, replayable for
// any later step of the same shape (the per-step values live in the device
// step plan, whose layout depends only on that shape).
struct kva_graph {
    kva_cache *cache = nullptr;
    hipGraphExec_t exec = nullptr;
    int32_t n_seqs = 0, n_tok = 0, table_rows = 0;
    bool all_one = false, has_bits = false;
    size_t offs[12] = {};
};

namespace {

int check_cfg(const kva_config *c) {
    if (!c) return fail(KVA_ERR_INVALID_ARG, "config is NULL");
    if (c->n_layers <= 0 || c->max_seqs <= 0 || c->max_blocks <= 0 ||
        c->max_blocks_per_seq <= 0 || c->max_step_tokens <= 0)
        return fail(KVA_ERR_INVALID_ARG, "n_layers, max_seqs, max_blocks, max_blocks_per_seq and "
                                         "max_step_tokens must be positive");
    if (c->head_dim != kva::kHeadDim)
        return fail(KVA_ERR_UNSUPPORTED, "head_dim %d unsupported (only 256)", c->head_dim);
    if (c->block_tokens != kva::kBlockTokens)
        return fail(KVA_ERR_UNSUPPORTED, "block_tokens %d unsupported (only 16)", c->block_tokens);
    if (c->num_heads <= 0 || c->num_kv_heads <= 0 || c->num_heads % c->num_kv_heads != 0)
        return fail(KVA_ERR_INVALID_ARG, "num_heads %d must be a positive multiple of num_kv_heads %d",
                    c->num_heads, c->num_kv_heads);
    const int g = c->num_heads / c->num_kv_heads;
    if (!(g == 1 || g == 2 || g == 3 || g == 4 || g == 6 || g == 8))
        return fail(KVA_ERR_UNSUPPORTED, "GQA group %d unsupported (1,2,3,4,6,8)", g);
    if (c->rotary_dim < 0 || c->rotary_dim > c->head_dim || c->rotary_dim % 8 != 0)
        return fail(KVA_ERR_UNSUPPORTED, "rotary_dim %d must be a multiple of 8 in [0, head_dim]",
                    c->rotary_dim);
    if (!(c->eps >= 0.0f)) return fail(KVA_ERR_INVALID_ARG, "eps must be >= 0");
    if (static_cast<int64_t>(c->max_blocks_per_seq) * kva::kBlockTokens > (1 << 30))
        return fail(KVA_ERR_INVALID_ARG, "max_blocks_per_seq too large");
    return KVA_OK;
}

int check_seq(const kva_cache *c, int32_t seq) {
    if (seq < 0 || seq >= c->cfg.max_seqs)
        return fail(KVA_ERR_BAD_SEQ, "sequence id %d out of range [0, %d)", seq, c->cfg.max_seqs);
    return KVA_OK;
}

// Take free blocks until `seq` holds `need` blocks.
int grow_seq(kva_cache *c, int32_t seq, int32_t need) {
    if (need > c->cfg.max_blocks_per_seq)
        return fail(KVA_ERR_CAPACITY, "sequence %d needs %d blocks > max_blocks_per_seq %d", seq,
                    need, c->cfg.max_blocks_per_seq);
    const int32_t have = c->nblk[seq];
    if (need <= have) return KVA_OK;
    if (static_cast<size_t>(need - have) > c->free_list.size())
        return fail(KVA_ERR_OUT_OF_BLOCKS, "pool exhausted: sequence %d needs %d more blocks, %zu free",
                    seq, need - have, c->free_list.size());
    for (int32_t i = have; i < need; ++i) {
        const int32_t blk = c->free_list.back();
        c->free_list.pop_back();
        c->used[blk] = 1;
        c->table[static_cast<size_t>(seq) * c->cfg.max_blocks_per_seq + i] = blk;
        c->patches.insert(c->patches.end(), {seq, i, blk});
    }
    c->nblk[seq] = need;
    c->freed[seq] = 0;
    return KVA_OK;
}

void release_blocks(kva_cache *c, int32_t seq) {
    const size_t base = static_cast<size_t>(seq) * c->cfg.max_blocks_per_seq;
    for (int32_t i = 0; i < c->nblk[seq]; ++i) {
        const int32_t blk = c->table[base + i];
        c->used[blk] = 0;
        c->free_list.push_back(blk);
        c->table[base + i] = -1;
    }
    c->nblk[seq] = 0;
}

// Next pinned staging slot, waiting until its previous copy has completed.
int acquire_stage(kva_cache *c, uint8_t **slot, int *idx) {
    const int i = c->stage_next;
    c->stage_next = (i + 1) % kStageSlots;
    if (c->ev_live[i]) {
        KVA_HIP(hipEventSynchronize(c->ev[i]));
        c->ev_live[i] = false;
    }
    *slot = c->h_stage[i];
    *idx = i;
    return KVA_OK;
}

int release_stage(kva_cache *c, int idx, hipStream_t s) {
    KVA_HIP(hipEventRecord(c->ev[idx], s));
    c->ev_live[idx] = true;
    return KVA_OK;
}

size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Upload pending block-table patches, in chunks that fit a staging slot.
int flush_patches(kva_cache *c, hipStream_t s) {
    if (c->host_only) {
        c->patches.clear();
        return KVA_OK;
    }
    const size_t per_chunk = c->aux_bytes / (3 * sizeof(int32_t));
    size_t done = 0;
    const size_t total = c->patches.size() / 3;
    while (done < total) {
        const size_t n = std::min(per_chunk, total - done);
        uint8_t *h;
        int idx;
        int rc = acquire_stage(c, &h, &idx);
        if (rc) return rc;
        std::memcpy(h, c->patches.data() + 3 * done, n * 3 * sizeof(int32_t));
        KVA_HIP(hipMemcpyAsync(c->d_aux, h, n * 3 * sizeof(int32_t), hipMemcpyHostToDevice, s));
        rc = release_stage(c, idx, s);
        if (rc) return rc;
        KVA_HIP(kva::launch_table_patch(c->d_table, c->cfg.max_blocks_per_seq,
                                        reinterpret_cast<const int32_t *>(c->d_aux),
                                        static_cast<int32_t>(n), s));
        done += n;
    }
    c->patches.clear();
    return KVA_OK;
}

int require_device(const kva_cache *c) {
    if (!c) return fail(KVA_ERR_INVALID_ARG, "cache is NULL");
    if (c->host_only) return fail(KVA_ERR_NO_DEVICE, "cache was created host-only");
    return KVA_OK;
}

int check_layer(const kva_cache *c, int32_t layer) {
    if (layer < 0 || layer >= c->cfg.n_layers)
        return fail(KVA_ERR_INVALID_ARG, "layer %d out of range [0, %d)", layer, c->cfg.n_layers);
    return KVA_OK;
}

template <class T>
T *at(uint8_t *base, size_t off) {
    return reinterpret_cast<T *>(base + off);
}

// Workgroups for a stream-K decode over `pages` pages: one per CU by default
// (each then streams long runs of pages), or pages*16/split_user when a
// token count per workgroup was set; never more than the workspace holds or
// than there are pages, and at least kMinPagesPerWg pages each.
int32_t choose_wg(const kva_cache *c, int64_t pages) {
    int64_t w;
    if (c->split_user > 0)
        w = (pages * kva::kBlockTokens + c->split_user - 1) / c->split_user;
    else
        w = static_cast<int64_t>(c->n_cu) * kDecodeWgPerCu;
    w = std::min<int64_t>(w, (pages + kMinPagesPerWg - 1) / kMinPagesPerWg);
    w = std::min<int64_t>(w, c->max_wg);
    return static_cast<int32_t>(std::max<int64_t>(1, w));
}

// While a graph is being recorded, a call on another stream would run now
// instead of being recorded, and a call that fails leaves a hole in the
// recording: both are refused or remembered, and kva_graph_capture_end
// reports them.
int capture_check(kva_cache *c, kva_stream_t stream) {
    if (c && c->capturing && static_cast<hipStream_t>(stream) != c->cap_stream)
        return fail(KVA_ERR_STATE, "call on another stream while a graph is being recorded");
    return KVA_OK;
}

int capture_note(kva_cache *c, int rc) {
    if (rc != KVA_OK && c && c->capturing) c->capture_failed = true;
    return rc;
}

// A call that cannot be recorded: its launch shape or its host work depends
// on the step (or it is the step change itself).
int refuse_while_capturing(const kva_cache *c, const char *what) {
    if (c && c->capturing) return fail(KVA_ERR_STATE, "%s cannot run while a graph is being recorded", what);
    return KVA_OK;
}

}  // namespace

extern "C" {

const char *kva_last_error_string(void) { return g_err.c_str(); }
const char *kva_version(void) { return "kvattn 0.1 gfx950"; }

int kva_create(const kva_config *cfg, kva_cache **out) {
    if (!out) return fail(KVA_ERR_INVALID_ARG, "out is NULL");
    *out = nullptr;
    int rc = check_cfg(cfg);
    if (rc) return rc;
    kva_cache *c = new kva_cache();
    c->cfg = *cfg;
    c->host_only = (cfg->flags & KVA_FLAG_HOST_ONLY) != 0;
    c->group = cfg->num_heads / cfg->num_kv_heads;
    c->row_elems = static_cast<size_t>(cfg->num_kv_heads) * cfg->head_dim;
    c->layer_elems = static_cast<size_t>(cfg->max_blocks) * kva::kBlockTokens * c->row_elems;
    const size_t mbps = cfg->max_blocks_per_seq;
    c->table.assign(static_cast<size_t>(cfg->max_seqs) * mbps, -1);
    c->nblk.assign(cfg->max_seqs, 0);
    c->len.assign(cfg->max_seqs, 0);
    c->freed.assign(cfg->max_seqs, 0);
    c->used.assign(cfg->max_blocks, 0);
    c->free_list.resize(cfg->max_blocks);
    for (int32_t i = 0; i < cfg->max_blocks; ++i) c->free_list[i] = cfg->max_blocks - 1 - i;
    // Step plan: 5 per-sequence arrays + 3 per-token arrays + bits + the
    // first kPlanPages block ids of each sequence.
    // Multi-query units: at most (tokens/Q + sequences) tiles per kv head,
    // Q >= the one-tile token count of the group.
    const size_t q_min = static_cast<size_t>(kva::mq_tile_tokens(cfg->num_heads / cfg->num_kv_heads, 4, 1));
    const size_t max_units =
        (static_cast<size_t>(cfg->max_step_tokens) / q_min + cfg->max_seqs) * cfg->num_kv_heads;
    c->step_bytes = round_up(sizeof(int32_t) * (6 * static_cast<size_t>(cfg->max_seqs) + 3), 256) +
                    round_up(sizeof(int32_t) * (max_units + 1), 256) +
                    round_up(sizeof(int32_t) * 3 * static_cast<size_t>(cfg->max_step_tokens), 256) +
                    round_up(sizeof(uint64_t) * static_cast<size_t>(cfg->max_step_tokens), 256) +
                    round_up(sizeof(int32_t) * kva::kPlanPages * static_cast<size_t>(cfg->max_seqs), 256) +
                    round_up(sizeof(int32_t) * kva::kMqCutWords * max_units, 256) + 1024;
    const size_t patch_cap = std::max<size_t>(4096, cfg->max_seqs + cfg->max_step_tokens);
    c->aux_bytes = round_up(std::max(patch_cap * 3 * sizeof(int32_t),
                                     (static_cast<size_t>(cfg->max_step_tokens) * 3 + cfg->max_seqs + 1) *
                                         sizeof(int32_t)),
                            256);
    c->stage_bytes = std::max(c->step_bytes, c->aux_bytes);
    // Projection partials: every split of one launch pair's tokens.  Sized
    // for host-only caches too, whose calls are validated exactly as on the
    // device (against a nominal MI355X CU count) before they are refused.
    c->proj_floats = static_cast<size_t>(kva::kProjMaxSplits) * kva::kProjTokens *
                     (2 * static_cast<size_t>(cfg->num_heads) + 2 * cfg->num_kv_heads) * kva::kHeadDim;
    c->n_cu = kHostOnlyCus;
    c->mq_max_wg = c->n_cu;  // the device's CU count below
    if (!c->host_only) {
        auto cleanup = [&](int code) {
            kva_destroy(c);
            return code;
        };
        hipError_t e;
        const size_t pool_bytes = c->layer_elems * cfg->n_layers * sizeof(uint16_t);
        if ((e = hipMalloc(&c->d_k, pool_bytes)) != hipSuccess) return cleanup(hip_fail(e, "hipMalloc(K pool)"));
        if ((e = hipMalloc(&c->d_v, pool_bytes)) != hipSuccess) return cleanup(hip_fail(e, "hipMalloc(V pool)"));
        // Zeroed pools: rows never written read as finite zeros.
        if ((e = hipMemset(c->d_k, 0, pool_bytes)) != hipSuccess) return cleanup(hip_fail(e, "hipMemset(K)"));
        if ((e = hipMemset(c->d_v, 0, pool_bytes)) != hipSuccess) return cleanup(hip_fail(e, "hipMemset(V)"));
        const size_t tbytes = c->table.size() * sizeof(int32_t);
        if ((e = hipMalloc(&c->d_table, tbytes)) != hipSuccess) return cleanup(hip_fail(e, "hipMalloc(table)"));
        if ((e = hipMemset(c->d_table, 0, tbytes)) != hipSuccess) return cleanup(hip_fail(e, "hipMemset(table)"));
        if ((e = hipMalloc(&c->d_step, c->step_bytes)) != hipSuccess) return cleanup(hip_fail(e, "hipMalloc(step)"));
        if ((e = hipMalloc(&c->d_aux, c->aux_bytes)) != hipSuccess) return cleanup(hip_fail(e, "hipMalloc(aux)"));
        int dev = 0, ncu = 0;
        if ((e = hipGetDevice(&dev)) != hipSuccess) return cleanup(hip_fail(e, "hipGetDevice"));
        if ((e = hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess)
            return cleanup(hip_fail(e, "hipDeviceGetAttribute(CU count)"));
        c->n_cu = std::max(1, ncu);
        // Partial slots: two per decode workgroup, each [heads][256] floats;
        // up to four workgroups per CU can be requested.
        c->max_wg = 4 * c->n_cu;
        c->ws_rows = static_cast<size_t>(2) * c->max_wg * c->cfg.num_heads;
        const size_t units = c->ws_rows;
        if ((e = hipMalloc(&c->d_ws_acc, units * kva::kHeadDim * sizeof(float))) != hipSuccess)
            return cleanup(hip_fail(e, "hipMalloc(workspace)"));
        if ((e = hipMalloc(&c->d_ws_ml, units * 2 * sizeof(float))) != hipSuccess)
            return cleanup(hip_fail(e, "hipMalloc(workspace ml)"));
        // Multi-query partial slots: two per workgroup, one workgroup per CU.
        c->mq_max_wg = c->n_cu;
        const size_t mq_rows = static_cast<size_t>(2) * c->mq_max_wg * kva::kMqSlotRows;
        if ((e = hipMalloc(&c->d_mq_acc, mq_rows * kva::kHeadDim * sizeof(float))) != hipSuccess)
            return cleanup(hip_fail(e, "hipMalloc(multi-query workspace)"));
        if ((e = hipMalloc(&c->d_mq_ml, mq_rows * 2 * sizeof(float))) != hipSuccess)
            return cleanup(hip_fail(e, "hipMalloc(multi-query workspace ml)"));
        if ((e = hipMalloc(&c->d_proj, c->proj_floats * sizeof(float))) != hipSuccess)
            return cleanup(hip_fail(e, "hipMalloc(projection workspace)"));
        for (int i = 0; i < kStageSlots; ++i) {
            if ((e = hipHostMalloc(reinterpret_cast<void **>(&c->h_stage[i]), c->stage_bytes,
                                   hipHostMallocDefault)) != hipSuccess)
                return cleanup(hip_fail(e, "hipHostMalloc(staging)"));
            if ((e = hipEventCreateWithFlags(&c->ev[i], hipEventDisableTiming)) != hipSuccess)
                return cleanup(hip_fail(e, "hipEventCreate"));
        }
        if ((e = hipDeviceSynchronize()) != hipSuccess) return cleanup(hip_fail(e, "hipDeviceSynchronize"));
    }
    *out = c;
    return KVA_OK;
}

int kva_destroy(kva_cache *c) {
    if (!c) return fail(KVA_ERR_INVALID_ARG, "cache is NULL");
    if (int rc = refuse_while_capturing(c, "kva_destroy")) return rc;
    if (!c->host_only) {
        (void)hipDeviceSynchronize();
        for (int i = 0; i < kStageSlots; ++i) {
            if (c->ev[i]) (void)hipEventDestroy(c->ev[i]);
            if (c->h_stage[i]) (void)hipHostFree(c->h_stage[i]);
        }
        (void)hipFree(c->d_k);
        (void)hipFree(c->d_v);
        (void)hipFree(c->d_table);
        (void)hipFree(c->d_step);
        (void)hipFree(c->d_aux);
        (void)hipFree(c->d_ws_acc);
        (void)hipFree(c->d_ws_ml);
        (void)hipFree(c->d_timeline);
        (void)hipFree(c->d_mq_acc);
        (void)hipFree(c->d_mq_ml);
        (void)hipFree(c->d_proj);
    }
    delete c;
    return KVA_OK;
}

int kva_get_layout(const kva_cache *c, kva_layout *out) {
    if (!c || !out) return fail(KVA_ERR_INVALID_ARG, "NULL argument");
    out->row_bytes = c->row_elems * sizeof(uint16_t);
    out->block_bytes = out->row_bytes * kva::kBlockTokens;
    out->layer_bytes = c->layer_elems * sizeof(uint16_t);
    out->block_tokens = kva::kBlockTokens;
    out->max_blocks_per_seq = c->cfg.max_blocks_per_seq;
    return KVA_OK;
}

int kva_layer_pools(const kva_cache *c, int32_t layer, void **k_pool, void **v_pool) {
    int rc = require_device(c);
    if (rc) return rc;
    if ((rc = check_layer(c, layer))) return rc;
    if (!k_pool || !v_pool) return fail(KVA_ERR_INVALID_ARG, "NULL output pointer");
    *k_pool = c->d_k + c->layer_elems * layer;
    *v_pool = c->d_v + c->layer_elems * layer;
    return KVA_OK;
}

int kva_seq_reserve(kva_cache *c, int32_t seq, int32_t n_tokens) {
    if (!c) return fail(KVA_ERR_INVALID_ARG, "cache is NULL");
    int rc = check_seq(c, seq);
    if (rc) return rc;
    if (n_tokens < 0) return fail(KVA_ERR_INVALID_ARG, "n_tokens %d < 0", n_tokens);
    const int64_t need = (static_cast<int64_t>(n_tokens) + kva::kBlockTokens - 1) / kva::kBlockTokens;
    if (need > c->cfg.max_blocks_per_seq)
        return fail(KVA_ERR_CAPACITY, "sequence %d: %d tokens exceed capacity %d", seq, n_tokens,
                    c->cfg.max_blocks_per_seq * kva::kBlockTokens);
    return grow_seq(c, seq, static_cast<int32_t>(need));
}

int kva_seq_set_blocks(kva_cache *c, int32_t seq, const int32_t *ids, int32_t n) {
    if (!c) return fail(KVA_ERR_INVALID_ARG, "cache is NULL");
    int rc = check_seq(c, seq);
    if (rc) return rc;
    if (n < 0 || (n > 0 && !ids)) return fail(KVA_ERR_INVALID_ARG, "bad block list");
    if (n > c->cfg.max_blocks_per_seq)
        return fail(KVA_ERR_CAPACITY, "%d blocks > max_blocks_per_seq %d", n, c->cfg.max_blocks_per_seq);
    if (static_cast<int64_t>(n) * kva::kBlockTokens < c->len[seq])
        return fail(KVA_ERR_CAPACITY, "%d blocks cannot hold the current length %d", n, c->len[seq]);
    // Validate: in range, distinct, free (or already this sequence's).
    const size_t base = static_cast<size_t>(seq) * c->cfg.max_blocks_per_seq;
    std::vector<uint8_t> mine(c->cfg.max_blocks, 0), seen(c->cfg.max_blocks, 0);
    for (int32_t i = 0; i < c->nblk[seq]; ++i) mine[c->table[base + i]] = 1;
    for (int32_t i = 0; i < n; ++i) {
        const int32_t b = ids[i];
        if (b < 0 || b >= c->cfg.max_blocks)
            return fail(KVA_ERR_BAD_BLOCK, "block id %d out of range [0, %d)", b, c->cfg.max_blocks);
        if (seen[b]) return fail(KVA_ERR_BAD_BLOCK, "block id %d listed twice", b);
        seen[b] = 1;
        if (c->used[b] && !mine[b]) return fail(KVA_ERR_BAD_BLOCK, "block id %d is in use", b);
    }
    release_blocks(c, seq);
    // Remove the new blocks from the free list.
    c->free_list.erase(std::remove_if(c->free_list.begin(), c->free_list.end(),
                                      [&](int32_t b) { return seen[b] != 0; }),
                       c->free_list.end());
    for (int32_t i = 0; i < n; ++i) {
        c->used[ids[i]] = 1;
        c->table[base + i] = ids[i];
        c->patches.insert(c->patches.end(), {seq, i, ids[i]});
    }
    c->nblk[seq] = n;
    c->freed[seq] = 0;
    c->step_valid = false;  // the step plan holds the old block ids
    return KVA_OK;
}

int kva_seq_free(kva_cache *c, int32_t seq) {
    if (!c) return fail(KVA_ERR_INVALID_ARG, "cache is NULL");
    int rc = check_seq(c, seq);
    if (rc) return rc;
    if (c->freed[seq]) return fail(KVA_ERR_DOUBLE_FREE, "sequence %d already freed", seq);
    release_blocks(c, seq);
    c->len[seq] = 0;
    c->freed[seq] = 1;
    c->step_valid = false;
    return KVA_OK;
}

int kva_seq_get_len(const kva_cache *c, int32_t seq, int32_t *len) {
    if (!c || !len) return fail(KVA_ERR_INVALID_ARG, "NULL argument");
    int rc = check_seq(c, seq);
    if (rc) return rc;
    *len = c->len[seq];
    return KVA_OK;
}

int kva_seq_set_len(kva_cache *c, int32_t seq, int32_t len) {
    if (!c) return fail(KVA_ERR_INVALID_ARG, "cache is NULL");
    int rc = check_seq(c, seq);
    if (rc) return rc;
    if (len < 0) return fail(KVA_ERR_ROLLBACK, "length %d < 0", len);
    if (static_cast<int64_t>(len) > static_cast<int64_t>(c->nblk[seq]) * kva::kBlockTokens)
        return fail(KVA_ERR_CAPACITY, "length %d exceeds reserved capacity %d", len,
                    c->nblk[seq] * kva::kBlockTokens);
    c->len[seq] = len;
    c->step_valid = false;
    return KVA_OK;
}

int kva_seq_get_blocks(const kva_cache *c, int32_t seq, int32_t *ids, int32_t cap, int32_t *n) {
    if (!c || !n) return fail(KVA_ERR_INVALID_ARG, "NULL argument");
    int rc = check_seq(c, seq);
    if (rc) return rc;
    *n = c->nblk[seq];
    if (ids) {
        const size_t base = static_cast<size_t>(seq) * c->cfg.max_blocks_per_seq;
        for (int32_t i = 0; i < std::min(cap, c->nblk[seq]); ++i) ids[i] = c->table[base + i];
    }
    return KVA_OK;
}

int kva_free_block_count(const kva_cache *c, int32_t *n) {
    if (!c || !n) return fail(KVA_ERR_INVALID_ARG, "NULL argument");
    *n = static_cast<int32_t>(c->free_list.size());
    return KVA_OK;
}

int kva_row_ptr(const kva_cache *c, int32_t layer, int32_t seq, int32_t slot, void **k_row,
                void **v_row) {
    int rc = require_device(c);
    if (rc) return rc;
    if ((rc = check_layer(c, layer))) return rc;
    if ((rc = check_seq(c, seq))) return rc;
    if (!k_row || !v_row) return fail(KVA_ERR_INVALID_ARG, "NULL output pointer");
    if (slot < 0 || slot >= c->nblk[seq] * kva::kBlockTokens)
        return fail(KVA_ERR_CAPACITY, "slot %d outside the %d reserved rows of sequence %d", slot,
                    c->nblk[seq] * kva::kBlockTokens, seq);
    const int32_t blk = c->table[static_cast<size_t>(seq) * c->cfg.max_blocks_per_seq + slot / kva::kBlockTokens];
    const size_t off = c->layer_elems * layer +
                       (static_cast<size_t>(blk) * kva::kBlockTokens + slot % kva::kBlockTokens) * c->row_elems;
    *k_row = c->d_k + off;
    *v_row = c->d_v + off;
    return KVA_OK;
}

int kva_sync_tables(kva_cache *c, kva_stream_t stream) {
    if (!c) return fail(KVA_ERR_INVALID_ARG, "cache is NULL");
    if (int rc = refuse_while_capturing(c, "kva_sync_tables")) return rc;
    return flush_patches(c, static_cast<hipStream_t>(stream));
}

int kva_step_begin(kva_cache *c, int32_t n_seqs, const int32_t *seq_ids, const int32_t *n_new,
                   const int32_t *rope_pos, const uint64_t *tree_bits, kva_stream_t stream) {
    if (!c) return fail(KVA_ERR_INVALID_ARG, "cache is NULL");
    if (int rc = refuse_while_capturing(c, "kva_step_begin")) return rc;
    c->step_valid = false;
    if (n_seqs <= 0 || n_seqs > c->cfg.max_seqs)
        return fail(KVA_ERR_INVALID_ARG, "n_seqs %d outside [1, %d]", n_seqs, c->cfg.max_seqs);
    if (!seq_ids || !n_new) return fail(KVA_ERR_INVALID_ARG, "seq_ids / n_new is NULL");
    std::vector<uint8_t> seen(c->cfg.max_seqs, 0);
    int64_t n_tok = 0;
    int64_t extra_blocks = 0;
    for (int32_t b = 0; b < n_seqs; ++b) {
        const int32_t s = seq_ids[b];
        int rc = check_seq(c, s);
        if (rc) return rc;
        if (seen[s]) return fail(KVA_ERR_INVALID_ARG, "sequence %d listed twice in one step", s);
        seen[s] = 1;
        if (n_new[b] < 0) return fail(KVA_ERR_INVALID_ARG, "n_new[%d] = %d < 0", b, n_new[b]);
        const int64_t end = static_cast<int64_t>(c->len[s]) + n_new[b];
        if (end > static_cast<int64_t>(c->cfg.max_blocks_per_seq) * kva::kBlockTokens)
            return fail(KVA_ERR_CAPACITY, "sequence %d: length %lld exceeds capacity %d", s,
                        static_cast<long long>(end), c->cfg.max_blocks_per_seq * kva::kBlockTokens);
        const int64_t need = (end + kva::kBlockTokens - 1) / kva::kBlockTokens;
        extra_blocks += std::max<int64_t>(0, need - c->nblk[s]);
        n_tok += n_new[b];
    }
    if (n_tok > c->cfg.max_step_tokens)
        return fail(KVA_ERR_CAPACITY, "step has %lld new tokens > max_step_tokens %d",
                    static_cast<long long>(n_tok), c->cfg.max_step_tokens);
    if (extra_blocks > static_cast<int64_t>(c->free_list.size()))
        return fail(KVA_ERR_OUT_OF_BLOCKS, "step needs %lld more blocks, %zu free",
                    static_cast<long long>(extra_blocks), c->free_list.size());
    if (rope_pos)
        for (int64_t i = 0; i < n_tok; ++i)
            if (rope_pos[i] < 0) return fail(KVA_ERR_INVALID_ARG, "rope_pos[%lld] < 0", static_cast<long long>(i));
    if (tree_bits) {
        int64_t t = 0;
        for (int32_t b = 0; b < n_seqs; ++b) {
            if (n_new[b] > 64) return fail(KVA_ERR_UNSUPPORTED, "tree of %d nodes > 64", n_new[b]);
            for (int32_t i = 0; i < n_new[b]; ++i, ++t) {
                const uint64_t bits = tree_bits[t];
                const uint64_t self = 1ull << i;
                if (!(bits & self) || (bits >> i) != 1ull)
                    return fail(KVA_ERR_INVALID_ARG,
                                "tree_bits of node %d of sequence %d must contain itself and only earlier nodes",
                                i, seq_ids[b]);
            }
        }
    }
    // Commit: reserve, assign slots, advance lengths.
    for (int32_t b = 0; b < n_seqs; ++b) {
        const int32_t s = seq_ids[b];
        const int64_t end = static_cast<int64_t>(c->len[s]) + n_new[b];
        int rc = grow_seq(c, s, static_cast<int32_t>((end + kva::kBlockTokens - 1) / kva::kBlockTokens));
        if (rc) return rc;
    }
    const size_t o_seq = 0;
    const size_t o_ctx = o_seq + sizeof(int32_t) * n_seqs;
    const size_t o_start = o_ctx + sizeof(int32_t) * n_seqs;
    const size_t o_tokoff = o_start + sizeof(int32_t) * n_seqs;
    const size_t o_pre = o_tokoff + sizeof(int32_t) * (n_seqs + 1);
    // Multi-query tiling: Q new tokens per unit tile (see mq_tiles_for).
    const int32_t group = c->cfg.num_heads / c->cfg.num_kv_heads;
    int32_t run_max = 0;
    for (int32_t b = 0; b < n_seqs; ++b) run_max = std::max(run_max, n_new[b]);
    const int32_t mq_waves = kva::mq_waves_for(group, run_max);
    const int32_t mq_q = kva::mq_tile_tokens(group, mq_waves, 1);
    int64_t n_units = 0;
    for (int32_t b = 0; b < n_seqs; ++b)
        n_units += static_cast<int64_t>((n_new[b] + mq_q - 1) / mq_q) * c->cfg.num_kv_heads;
    const size_t o_upre = o_pre + sizeof(int32_t) * (n_seqs + 1);
    const size_t o_mqpre = o_upre + sizeof(int32_t) * (n_seqs + 1);
    const size_t o_tseq = round_up(o_mqpre + sizeof(int32_t) * (n_units + 1), 16);
    const size_t o_tslot = round_up(o_tseq + sizeof(int32_t) * n_tok, 16);
    const size_t o_tpos = round_up(o_tslot + sizeof(int32_t) * n_tok, 16);
    const size_t o_bits = round_up(o_tpos + sizeof(int32_t) * n_tok, 16);
    const size_t o_pids = round_up(o_bits + (tree_bits ? sizeof(uint64_t) * n_tok : 0), 16);
    const size_t o_cut = round_up(o_pids + sizeof(int32_t) * kva::kPlanPages * n_seqs, 16);
    // The cut-unit records (below) take at most one per unit; only those
    // written are uploaded.
    const size_t total_max = o_cut + sizeof(int32_t) * kva::kMqCutWords * n_units;

    std::vector<uint8_t> local;
    uint8_t *h = nullptr;
    int idx = -1;
    if (c->host_only) {
        local.resize(total_max + 16);
        h = local.data();
    } else {
        int rc = acquire_stage(c, &h, &idx);
        if (rc) return rc;
    }
    int32_t *p_seq = at<int32_t>(h, o_seq), *p_ctx = at<int32_t>(h, o_ctx),
            *p_start = at<int32_t>(h, o_start), *p_off = at<int32_t>(h, o_tokoff),
            *p_tseq = at<int32_t>(h, o_tseq), *p_tslot = at<int32_t>(h, o_tslot),
            *p_tpos = at<int32_t>(h, o_tpos), *p_pre = at<int32_t>(h, o_pre);
    int32_t max_ctx = 0, max_new = 0, max_pos = 0;
    int64_t pages = 0;
    bool all_one = true;
    int32_t t = 0;
    for (int32_t b = 0; b < n_seqs; ++b) {
        const int32_t s = seq_ids[b];
        const int32_t start = c->len[s];
        p_seq[b] = s;
        p_start[b] = start;
        p_ctx[b] = start + n_new[b];
        p_off[b] = t;
        for (int32_t i = 0; i < n_new[b]; ++i, ++t) {
            p_tseq[t] = s;
            p_tslot[t] = start + i;
            p_tpos[t] = rope_pos ? rope_pos[t] : start + i;
            max_pos = std::max(max_pos, p_tpos[t]);
        }
        c->len[s] = start + n_new[b];
        max_ctx = std::max(max_ctx, p_ctx[b]);
        max_new = std::max(max_new, n_new[b]);
        p_pre[b] = static_cast<int32_t>(pages);
        pages += (p_ctx[b] + kva::kBlockTokens - 1) / kva::kBlockTokens;
        all_one = all_one && n_new[b] == 1;
    }
    p_off[n_seqs] = t;
    p_pre[n_seqs] = static_cast<int32_t>(pages);
    // The block ids of each sequence's first kPlanPages pages (the blocks the
    // step needs are reserved above), zeros past its pages.
    int32_t *p_pids = at<int32_t>(h, o_pids);
    for (int32_t b = 0; b < n_seqs; ++b) {
        const int32_t np =
            std::min<int32_t>((p_ctx[b] + kva::kBlockTokens - 1) / kva::kBlockTokens, kva::kPlanPages);
        const int32_t *row = c->table.data() + static_cast<size_t>(seq_ids[b]) * c->cfg.max_blocks_per_seq;
        int32_t *dst = p_pids + static_cast<size_t>(b) * kva::kPlanPages;
        std::copy(row, row + np, dst);
        std::fill(dst + np, dst + kva::kPlanPages, 0);
    }
    // Multi-query units in (kv head, sequence, tile) order with their key
    // blocks: a tree tile reads the whole cache, a causal tile reads up to
    // its last token's slot.  upre[b] counts the tiles of earlier sequences
    // (one head's units); unit u is head u / upre[n_seqs].  Head-major order
    // puts all tiles of one (sequence, head) in consecutive stream-K shares,
    // which the kernel places on one XCD, so the tiles' repeated reads of
    // that head's keys hit the XCD's L2.
    int32_t *p_upre = at<int32_t>(h, o_upre), *p_mqpre = at<int32_t>(h, o_mqpre);
    int64_t tiles_all = 0;
    for (int32_t b = 0; b < n_seqs; ++b) {
        p_upre[b] = static_cast<int32_t>(tiles_all);
        tiles_all += (n_new[b] + mq_q - 1) / mq_q;
    }
    p_upre[n_seqs] = static_cast<int32_t>(tiles_all);
    const int32_t mq_keys = kva::mq_keys_for(mq_waves, tree_bits != nullptr);
    const int32_t unit_cost = kva::mq_unit_cost(mq_keys);
    int64_t units = 0, blocks = 0;
    for (int32_t hh = 0; hh < c->cfg.num_kv_heads; ++hh) {
        for (int32_t b = 0; b < n_seqs; ++b) {
            const int32_t tiles = (n_new[b] + mq_q - 1) / mq_q;
            for (int32_t tl = 0; tl < tiles; ++tl) {
                const int64_t keys = tree_bits ? p_ctx[b] : p_start[b] + std::min(n_new[b], (tl + 1) * mq_q);
                const int64_t nb = (keys + mq_keys - 1) / mq_keys;
                p_mqpre[units++] = static_cast<int32_t>(blocks);
                blocks += unit_cost + nb;
            }
        }
    }
    p_mqpre[units] = static_cast<int32_t>(blocks);
    if (tree_bits) std::memcpy(h + o_bits, tree_bits, sizeof(uint64_t) * n_tok);
    // The units the multi-query launch will cut across workgroups (the same
    // shares: kva::mq_wg_count workgroups over the unit positions), one
    // record each for its combine: head, the tile's first new token, its
    // valid tokens, first and last share, and the first piece's slot (2w
    // when the unit begins at or before share w's start, else 2w+1; every
    // later share starts inside the unit, so its slot is 2w).
    const int32_t mq_wg = kva::mq_wg_count(blocks, mq_keys, c->mq_max_wg);
    // The share holding position p, for non-decreasing p (a cursor: one
    // division per share boundary passed, so large decode-only steps, which
    // build the records too, stay cheap).
    int32_t cur_w = 0;
    int64_t cur_next = mq_wg > 1 ? kva::mq_share_start(1, blocks, mq_wg) : blocks;
    auto share_of = [&](int64_t p) {
        while (cur_w + 1 < mq_wg && cur_next <= p) {
            ++cur_w;
            cur_next = kva::mq_share_start(cur_w + 1, blocks, mq_wg);
        }
        return cur_w;
    };
    int32_t *p_cut = at<int32_t>(h, o_cut);
    int32_t n_cut = 0;
    {
        int64_t u = 0;
        for (int32_t hh = 0; hh < c->cfg.num_kv_heads; ++hh) {
            for (int32_t b = 0; b < n_seqs; ++b) {
                const int32_t tiles = (n_new[b] + mq_q - 1) / mq_q;
                for (int32_t tl = 0; tl < tiles; ++tl, ++u) {
                    const int64_t ub = p_mqpre[u] + unit_cost, ue = p_mqpre[u + 1];
                    if (ue <= ub) continue;
                    const int32_t w0 = share_of(ub), w1 = share_of(ue - 1);
                    if (w0 == w1) continue;
                    int32_t *r = p_cut + static_cast<size_t>(n_cut++) * kva::kMqCutWords;
                    r[0] = hh;
                    r[1] = p_off[b] + tl * mq_q;
                    r[2] = std::min(mq_q, n_new[b] - tl * mq_q);
                    r[3] = w0;
                    r[4] = w1;
                    r[5] = 2 * w0 + (ub <= kva::mq_share_start(w0, blocks, mq_wg) ? 0 : 1);
                    r[6] = r[7] = 0;
                }
            }
        }
    }
    const size_t total = o_cut + sizeof(int32_t) * kva::kMqCutWords * n_cut;

    if (!c->host_only) {
        hipStream_t s = static_cast<hipStream_t>(stream);
        KVA_HIP(hipMemcpyAsync(c->d_step, h, total, hipMemcpyHostToDevice, s));
        int rc = release_stage(c, idx, s);
        if (rc) return rc;
        if ((rc = flush_patches(c, s))) return rc;
    } else {
        c->patches.clear();
    }
    c->off_seq = o_seq;
    c->off_ctx = o_ctx;
    c->off_start = o_start;
    c->off_tokoff = o_tokoff;
    c->off_tseq = o_tseq;
    c->off_tslot = o_tslot;
    c->off_tpos = o_tpos;
    c->off_bits = o_bits;
    c->off_pre = o_pre;
    c->off_pids = o_pids;
    c->off_cut = o_cut;
    c->st_mq_wg = mq_wg;
    c->st_mq_cut = n_cut;
    c->st_n_seqs = n_seqs;
    c->st_n_tok = static_cast<int32_t>(n_tok);
    c->st_max_ctx = max_ctx;
    c->st_max_new = max_new;
    c->st_max_pos = max_pos;
    c->st_total_pages = static_cast<int32_t>(pages);
    c->st_mq_units = static_cast<int32_t>(units);
    c->st_mq_blocks = static_cast<int32_t>(blocks);
    c->st_mq_waves = mq_waves;
    c->st_mq_keys = mq_keys;
    c->st_mq_q = mq_q;
    c->off_upre = o_upre;
    c->off_mqpre = o_mqpre;
    c->st_all_one = all_one;
    c->st_pre.assign(p_pre, p_pre + n_seqs + 1);
    c->st_has_bits = tree_bits != nullptr;
    c->step_valid = true;
    return KVA_OK;
}

// Check an append's operands (the step already begun) and fill its launch
// arguments.
static int make_append(kva_cache *c, int32_t layer, void *q, void *k, const void *v, const void *q_norm_w,
                       const void *k_norm_w, const void *cos_tab, const void *sin_tab, int32_t table_rows,
                       kva::AppendArgs &a) {
    if (!q || !k || !v || !q_norm_w || !k_norm_w || !cos_tab || !sin_tab)
        return fail(KVA_ERR_INVALID_ARG, "NULL tensor pointer");
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(q_norm_w) || !aligned16(k_norm_w))
        return fail(KVA_ERR_MISALIGNED, "q, k, v and norm weights must be 16-byte aligned");
    const int half_rot = c->cfg.rotary_dim / 2;
    if (half_rot > 0 && ((reinterpret_cast<uintptr_t>(cos_tab) | reinterpret_cast<uintptr_t>(sin_tab)) & 7u))
        return fail(KVA_ERR_MISALIGNED, "cos/sin tables must be 8-byte aligned");
    if (c->st_max_pos >= table_rows)
        return fail(KVA_ERR_INVALID_ARG, "RoPE position %d beyond the %d table rows", c->st_max_pos,
                    table_rows);
    a = kva::AppendArgs{};
    a.q = static_cast<uint16_t *>(q);
    a.k = static_cast<uint16_t *>(k);
    a.v = static_cast<const uint16_t *>(v);
    a.q_w = static_cast<const uint16_t *>(q_norm_w);
    a.k_w = static_cast<const uint16_t *>(k_norm_w);
    a.cos_tab = static_cast<const uint16_t *>(cos_tab);
    a.sin_tab = static_cast<const uint16_t *>(sin_tab);
    a.k_pool = c->d_k + c->layer_elems * layer;
    a.v_pool = c->d_v + c->layer_elems * layer;
    a.table = c->d_table;
    a.table_stride = c->cfg.max_blocks_per_seq;
    a.tok_seq = at<int32_t>(c->d_step, c->off_tseq);
    a.tok_slot = at<int32_t>(c->d_step, c->off_tslot);
    a.tok_pos = at<int32_t>(c->d_step, c->off_tpos);
    a.n_tok = c->st_n_tok;
    a.num_heads = c->cfg.num_heads;
    a.num_kv_heads = c->cfg.num_kv_heads;
    a.half_rot = half_rot;
    a.eps = c->cfg.eps;
    return KVA_OK;
}

static int append_impl(kva_cache *c, int32_t layer, void *q, void *k, const void *v, const void *q_norm_w,
                       const void *k_norm_w, const void *cos_tab, const void *sin_tab, int32_t table_rows,
                       kva_stream_t stream) {
    if (!c) return fail(KVA_ERR_INVALID_ARG, "cache is NULL");
    int rc = check_layer(c, layer);
    if (rc) return rc;
    if (!c->step_valid) return fail(KVA_ERR_STATE, "no step begun (kva_step_begin)");
    if (c->st_n_tok == 0) return require_device(c);
    kva::AppendArgs a;
    if ((rc = make_append(c, layer, q, k, v, q_norm_w, k_norm_w, cos_tab, sin_tab, table_rows, a))) return rc;
    if ((rc = require_device(c))) return rc;
    KVA_HIP(kva::launch_append(a, static_cast<hipStream_t>(stream)));
    return KVA_OK;
}

// Hidden split among projection workgroups: the most splits (up to
// kProjMaxSplits) that give every wave a whole number of 32-wide k-steps
// and keep the grid within kProjWgPerCu workgroups per CU (at hidden 5120,
// 24 + 4 heads and 256 CUs: 128 row groups x 2 splits, one per CU).
static int32_t project_splits(const kva_cache *c, int32_t hidden, int32_t n_rows) {
    const int64_t n_grp = (n_rows / 16 + kva::kProjRowTiles - 1) / kva::kProjRowTiles;
    int32_t best = 1;
    for (int32_t s = 2; s <= kva::kProjMaxSplits; s *= 2)
        if (hidden % (s * 32 * kva::kProjWaves) == 0 &&
            n_grp * s <= static_cast<int64_t>(kva::kProjWgPerCu) * c->n_cu)
            best = s;
    return best;
}

static int project_impl(kva_cache *c, int32_t layer, const void *x, int32_t hidden, const void *w_q_fused,
                        const void *w_kv_fused, const void *q_norm_w, const void *k_norm_w, const void *cos_tab,
                        const void *sin_tab, int32_t table_rows, void *q_out, void *q_gate_out, void *kv_out,
                        kva_stream_t stream) {
    if (!c) return fail(KVA_ERR_INVALID_ARG, "cache is NULL");
    int rc = check_layer(c, layer);
    if (rc) return rc;
    if (!c->step_valid) return fail(KVA_ERR_STATE, "no step begun (kva_step_begin)");
    if (c->st_n_tok == 0) return require_device(c);
    if (!x || !w_q_fused || !w_kv_fused || !q_norm_w || !k_norm_w || !cos_tab || !sin_tab || !q_out)
        return fail(KVA_ERR_INVALID_ARG, "NULL tensor pointer");
    if (!aligned16(x) || !aligned16(w_q_fused) || !aligned16(w_kv_fused) || !aligned16(q_norm_w) ||
        !aligned16(k_norm_w) || !aligned16(q_out) || !aligned16(q_gate_out) || !aligned16(kv_out))
        return fail(KVA_ERR_MISALIGNED, "x, weights, norm weights and outputs must be 16-byte aligned");
    if (hidden <= 0 || hidden % kva::kProjHiddenQuantum != 0)
        return fail(KVA_ERR_INVALID_ARG, "hidden %d must be a positive multiple of %d", hidden,
                    kva::kProjHiddenQuantum);
    if (static_cast<int64_t>(kva::kProjTokens) * hidden * 2 > INT32_MAX)
        return fail(KVA_ERR_INVALID_ARG, "hidden %d too large", hidden);
    const int half_rot = c->cfg.rotary_dim / 2;
    if (half_rot > 0 && ((reinterpret_cast<uintptr_t>(cos_tab) | reinterpret_cast<uintptr_t>(sin_tab)) & 7u))
        return fail(KVA_ERR_MISALIGNED, "cos/sin tables must be 8-byte aligned");
    if (c->st_max_pos >= table_rows)
        return fail(KVA_ERR_INVALID_ARG, "RoPE position %d beyond the %d table rows", c->st_max_pos,
                    table_rows);
    if ((rc = require_device(c))) return rc;
    kva::ProjectArgs a{};
    a.w_a = static_cast<const uint16_t *>(w_q_fused);
    a.w_b = static_cast<const uint16_t *>(w_kv_fused);
    a.n_a = 2 * c->cfg.num_heads * kva::kHeadDim;
    a.n_b = 2 * c->cfg.num_kv_heads * kva::kHeadDim;
    a.hidden = hidden;
    a.splits = project_splits(c, hidden, a.n_a + a.n_b);
    a.part = c->d_proj;
    a.q_out = static_cast<uint16_t *>(q_out);
    a.gate_out = static_cast<uint16_t *>(q_gate_out);
    a.kv_out = static_cast<uint16_t *>(kv_out);
    a.q_w = static_cast<const uint16_t *>(q_norm_w);
    a.k_w = static_cast<const uint16_t *>(k_norm_w);
    a.cos_tab = static_cast<const uint16_t *>(cos_tab);
    a.sin_tab = static_cast<const uint16_t *>(sin_tab);
    a.k_pool = c->d_k + c->layer_elems * layer;
    a.v_pool = c->d_v + c->layer_elems * layer;
    a.table = c->d_table;
    a.table_stride = c->cfg.max_blocks_per_seq;
    a.tok_seq = at<int32_t>(c->d_step, c->off_tseq);
    a.tok_slot = at<int32_t>(c->d_step, c->off_tslot);
    a.tok_pos = at<int32_t>(c->d_step, c->off_tpos);
    a.num_heads = c->cfg.num_heads;
    a.num_kv_heads = c->cfg.num_kv_heads;
    a.half_rot = half_rot;
    a.eps = c->cfg.eps;
    a.ev_before = c->kev_before;
    a.ev_after = c->kev_after;
    const auto *xs = static_cast<const uint16_t *>(x);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    // Prefill-sized steps: one GEMM launch whose tiles are whole heads, the
    // epilogue fused (the reference's batched path at seq_len >= 32,
    // engine.py:3051-3068), instead of 64-token launch pairs that would
    // each read all the weights.
    if (c->st_n_tok > kva::kProjTokens) {
        a.tok0 = 0;
        a.n_tok = c->st_n_tok;
        a.x = xs;
        KVA_HIP(kva::launch_project_big(a, s));
        c->last_proj_path = KVA_PROJECT_PREFILL_GEMM;
        return KVA_OK;
    }
    for (int32_t t0 = 0; t0 < c->st_n_tok; t0 += kva::kProjTokens) {
        a.tok0 = t0;
        a.n_tok = std::min(kva::kProjTokens, c->st_n_tok - t0);
        a.x = xs + static_cast<size_t>(t0) * hidden;
        KVA_HIP(kva::launch_project(a, s));
    }
    c->last_proj_path = KVA_PROJECT_KERNELS;
    return KVA_OK;
}

int kva_get_project_path(const kva_cache *c, int32_t *path) {
    if (!c || !path) return fail(KVA_ERR_INVALID_ARG, "NULL argument");
    *path = c->last_proj_path;
    return KVA_OK;
}

int kva_set_decode_split(kva_cache *c, int32_t split_tokens) {
    if (!c) return fail(KVA_ERR_INVALID_ARG, "cache is NULL");
    if (split_tokens < 0 || split_tokens % kva::kSplitQuantum != 0)
        return fail(KVA_ERR_INVALID_ARG, "split_tokens %d must be 0 or a positive multiple of %d",
                    split_tokens, kva::kSplitQuantum);
    c->split_user = split_tokens;
    return KVA_OK;
}

// Timeline records, eight waves each: every stream-K workgroup the workspace
// can serve times the grid rows of a cache's own heads, or one whole-form
// workgroup per sequence and query head (the most it launches), whichever is
// more.
static size_t timeline_words(const kva_cache *c) {
    const int32_t hpw = std::min(c->cfg.num_kv_heads, static_cast<int32_t>(kva::kDecodeHeadsPerWg));
    int32_t h = hpw;
    while (c->cfg.num_kv_heads % h) --h;
    const size_t wgs = std::max(static_cast<size_t>(c->max_wg) * (c->cfg.num_kv_heads / h),
                                static_cast<size_t>(c->cfg.max_seqs) * c->cfg.num_heads);
    return wgs * 8 * kva::kTimelineWords;
}

int kva_timeline_enable(kva_cache *c, int32_t on) {
    if (!c) return fail(KVA_ERR_INVALID_ARG, "cache is NULL");
    if (int rc = require_device(c)) return rc;
    if (int rc = refuse_while_capturing(c, "kva_timeline_enable")) return rc;
    if (!on) {
        if (c->d_timeline) KVA_HIP(hipFree(c->d_timeline));
        c->d_timeline = nullptr;
        return KVA_OK;
    }
    if (c->d_timeline) return KVA_OK;
    const size_t bytes = timeline_words(c) * sizeof(uint64_t);
    KVA_HIP(hipMalloc(&c->d_timeline, bytes));
    KVA_HIP(hipMemset(c->d_timeline, 0, bytes));
    return KVA_OK;
}

int kva_timeline_read(const kva_cache *c, uint64_t *dst, size_t cap_words, int32_t *n_wg, int32_t *grid_rows) {
    if (!c || !dst || !n_wg || !grid_rows) return fail(KVA_ERR_INVALID_ARG, "NULL argument");
    if (!c->d_timeline) return fail(KVA_ERR_STATE, "timeline not enabled (kva_timeline_enable)");
    int32_t h = std::min(c->cfg.num_kv_heads, static_cast<int32_t>(kva::kDecodeHeadsPerWg));
    while (c->cfg.num_kv_heads % h) --h;
    *n_wg = c->last_nwg;
    *grid_rows = c->last_whole ? 1 : c->cfg.num_kv_heads / h;
    const size_t words = static_cast<size_t>(c->last_nwg) * *grid_rows * 8 * kva::kTimelineWords;
    if (cap_words < words) return fail(KVA_ERR_CAPACITY, "timeline needs %zu words, %zu given", words, cap_words);
    KVA_HIP(hipDeviceSynchronize());
    KVA_HIP(hipMemcpy(dst, c->d_timeline, words * sizeof(uint64_t), hipMemcpyDeviceToHost));
    return KVA_OK;
}

int kva_kernel_events(kva_cache *c, kva_event_t before, kva_event_t after) {
    if (!c) return fail(KVA_ERR_INVALID_ARG, "cache is NULL");
    if ((before == nullptr) != (after == nullptr))
        return fail(KVA_ERR_INVALID_ARG, "give both events or neither");
    if (int rc = refuse_while_capturing(c, "kva_kernel_events")) return rc;
    if (before && c->host_only) return fail(KVA_ERR_NO_DEVICE, "cache was created host-only");
    c->kev_before = static_cast<hipEvent_t>(before);
    c->kev_after = static_cast<hipEvent_t>(after);
    return KVA_OK;
}

int kva_get_decode_split(const kva_cache *c, int32_t *split_tokens, int32_t *n_splits) {
    if (!c || !split_tokens || !n_splits) return fail(KVA_ERR_INVALID_ARG, "NULL argument");
    *split_tokens = c->last_split;
    *n_splits = c->last_nwg;
    return KVA_OK;
}

// The combine's form: 1 (a workgroup per sequence and kv head, a wave per
// query head) when no sequence can be cut into more than kCombineChunk
// pieces, else 4 (four waves per query head share the chunks of a sequence
// cut into more): npg pages meet at most floor(npg * W / P) + 2 of W shares
// of P pages.
static int32_t combine_waves_for(int64_t max_npg, int64_t pages, int32_t n_wg) {
    if (pages <= 0) return 4;
    return max_npg * n_wg / pages + 2 <= kva::kCombineChunk ? 1 : 4;
}

// The combine's per-sequence facts for a launch of a.n_wg shares over
// a.total_pages pages (pre: the pages of earlier sequences), computed as the
// kernels split the pages: share w starts at w*P/W.
static void set_combine_recs(const std::vector<int32_t> &pre, kva::DecodeArgs &a) {
    a.n_crec = 0;
    const int32_t n = a.n_seqs;
    if (n > kva::kCombineRecs || static_cast<int64_t>(pre.size()) != static_cast<int64_t>(n) + 1) return;
    const int64_t P = a.total_pages, W = a.n_wg;
    if (P <= 0 || W <= 0) return;
    auto start = [&](int64_t w) { return w * P / W; };
    auto wg_of = [&](int64_t p) {
        int64_t w = p * W / P;
        while (w + 1 < W && start(w + 1) <= p) ++w;
        return w;
    };
    for (int32_t b = 0; b < n; ++b) {
        const int64_t first = pre[b], npg = pre[b + 1] - pre[b];
        const int64_t w0 = npg > 0 ? wg_of(first) : 0, w1 = npg > 0 ? wg_of(first + npg - 1) : 0;
        a.crec[b] = (npg > 0 && w0 != w1) ? static_cast<int32_t>(w0) : -1;
        a.crec_n[b] = static_cast<int32_t>(2 * (w1 - w0 + 1) + (first <= start(w0) ? 0 : 1));
    }
    a.n_crec = n;
}

static void set_stream_k(kva_cache *c, kva::DecodeArgs &a, int64_t pages, int32_t num_heads) {
    a.total_pages = static_cast<int32_t>(pages);
    // Two partial slots of num_heads rows per workgroup must fit the workspace.
    const int64_t fit = static_cast<int64_t>(c->ws_rows / (2 * static_cast<size_t>(num_heads)));
    a.n_wg = static_cast<int32_t>(std::max<int64_t>(1, std::min<int64_t>(choose_wg(c, pages), fit)));
    a.ws_acc = c->d_ws_acc;
    a.ws_ml = c->d_ws_ml;
    a.timeline = c->d_timeline;
    c->last_nwg = a.n_wg;
    c->last_split = static_cast<int32_t>((pages * kva::kBlockTokens + a.n_wg - 1) / a.n_wg);
}

// Switch a decode launch to the whole-sequence form when the split is
// automatic and no sequence is longer than kWholeMaxTokens rows: returns the
// workgroups per (sequence, kv head), each serving group / n of its query
// heads, n as large as fits one workgroup per CU (0: stream-K instead).
static int32_t use_whole(kva_cache *c, int32_t split_user, int64_t max_ctx, int32_t n_seqs, int32_t num_heads,
                         int32_t num_kv_heads, int32_t n_cu) {
    const bool whole = split_user == 0 && max_ctx <= kWholeMaxTokens;
    if (c) c->last_whole = whole;
    if (!whole) return 0;
    const int32_t g = num_heads / num_kv_heads;
    const int64_t units = static_cast<int64_t>(n_seqs) * num_kv_heads;
    int32_t n = 1;
    for (int32_t d = g; d > 1; --d) {  // the most groups whose workgroups fit the CUs
        if (g % d == 0 && units * d <= n_cu) {
            n = d;
            break;
        }
    }
    if (c) {
        c->last_nwg = static_cast<int32_t>(units * n);
        c->last_split = 0;
    }
    return n;
}

// The output gate's layout: 8-byte aligned rows, a stride in whole 4-element
// groups covering one sequence's H heads.
static int check_gate(const void *gate, int64_t gate_stride, int32_t num_heads) {
    if (!gate) return KVA_OK;
    if (reinterpret_cast<uintptr_t>(gate) & 7u) return fail(KVA_ERR_MISALIGNED, "gate must be 8-byte aligned");
    if (gate_stride % 4 != 0 || gate_stride < static_cast<int64_t>(num_heads) * kva::kHeadDim)
        return fail(KVA_ERR_INVALID_ARG, "gate_stride %lld must be a multiple of 4 covering %d heads",
                    static_cast<long long>(gate_stride), num_heads);
    return KVA_OK;
}

// app (nullable): the step's append, fused into the launch when the decode
// runs the whole-sequence form, else launched first (k left unwritten).
static int decode_impl(kva_cache *c, int32_t layer, const void *q, const void *gate, int64_t gate_stride,
                       void *out, kva_stream_t stream, const kva::AppendArgs *app = nullptr) {
    if (!c) return fail(KVA_ERR_INVALID_ARG, "cache is NULL");
    int rc = check_layer(c, layer);
    if (rc) return rc;
    if (!c->step_valid) return fail(KVA_ERR_STATE, "no step begun (kva_step_begin)");
    if (!c->st_all_one) return fail(KVA_ERR_STATE, "kva_decode needs exactly one new token per sequence");
    if (!q || !out) return fail(KVA_ERR_INVALID_ARG, "NULL tensor pointer");
    if (!aligned16(q) || !aligned16(out)) return fail(KVA_ERR_MISALIGNED, "q/out must be 16-byte aligned");
    if ((rc = check_gate(gate, gate_stride, c->cfg.num_heads))) return rc;
    if ((rc = require_device(c))) return rc;
    kva::DecodeArgs a{};
    a.gate = static_cast<const uint16_t *>(gate);
    a.gate_stride = gate_stride;
    a.q = static_cast<const uint16_t *>(q);
    a.k_pool = c->d_k + c->layer_elems * layer;
    a.v_pool = c->d_v + c->layer_elems * layer;
    a.table = c->d_table;
    a.table_stride = c->cfg.max_blocks_per_seq;
    a.seq_ids = at<int32_t>(c->d_step, c->off_seq);
    a.ctx_lens = at<int32_t>(c->d_step, c->off_ctx);
    a.pre_seq = at<int32_t>(c->d_step, c->off_pre);
    a.plan_pages = at<int32_t>(c->d_step, c->off_pids);
    a.n_seqs = c->st_n_seqs;
    a.num_heads = c->cfg.num_heads;
    a.num_kv_heads = c->cfg.num_kv_heads;
    set_stream_k(c, a, c->st_total_pages, c->cfg.num_heads);
    if ((a.whole = use_whole(c, c->split_user, c->st_max_ctx, c->st_n_seqs, c->cfg.num_heads,
                             c->cfg.num_kv_heads, c->n_cu))) {
        // Every launch of this form reads the lengths from the step plan: a
        // recorded one stays correct when they grow.
    } else if (c->capturing) {
        // Recorded launch: the device derives the page count and workgroup
        // count from the step plan at replay; the grid is the cap.
        const int64_t fit = static_cast<int64_t>(c->ws_rows / (2 * static_cast<size_t>(c->cfg.num_heads)));
        const int64_t cap = c->split_user > 0 ? c->max_wg : static_cast<int64_t>(c->n_cu) * kDecodeWgPerCu;
        a.n_wg = static_cast<int32_t>(std::max<int64_t>(1, std::min(cap, fit)));
        a.dyn = 1;  // the shape is derived at replay, so the combine keeps four waves
        a.split_tokens = c->split_user;
        a.min_pages = kMinPagesPerWg;
    } else {
        a.combine_waves = combine_waves_for((c->st_max_ctx + kva::kBlockTokens - 1) / kva::kBlockTokens,
                                            a.total_pages, a.n_wg);
        set_combine_recs(c->st_pre, a);
    }
    a.out = static_cast<uint16_t *>(out);
    a.ev_before = c->kev_before;
    a.ev_after = c->kev_after;
    if (app) {
        kva::AppendArgs ap = *app;
        ap.keep_k = 1;
        if (a.whole) {
            a.fused = 1;
            a.app = ap;
        } else {
            KVA_HIP(kva::launch_append(ap, static_cast<hipStream_t>(stream)));
        }
    }
    KVA_HIP(kva::launch_decode(a, static_cast<hipStream_t>(stream)));
    return KVA_OK;
}

static int append_decode_impl(kva_cache *c, int32_t layer, void *q, const void *k, const void *v,
                              const void *q_norm_w, const void *k_norm_w, const void *cos_tab, const void *sin_tab,
                              int32_t table_rows, const void *gate, int64_t gate_stride, void *out,
                              kva_stream_t stream) {
    if (!c) return fail(KVA_ERR_INVALID_ARG, "cache is NULL");
    int rc = check_layer(c, layer);
    if (rc) return rc;
    if (!c->step_valid) return fail(KVA_ERR_STATE, "no step begun (kva_step_begin)");
    if (!c->st_all_one) return fail(KVA_ERR_STATE, "kva_append_decode needs exactly one new token per sequence");
    kva::AppendArgs ap;
    if ((rc = make_append(c, layer, q, const_cast<void *>(k), v, q_norm_w, k_norm_w, cos_tab, sin_tab, table_rows,
                          ap)))
        return rc;
    return decode_impl(c, layer, q, gate, gate_stride, out, stream, &ap);
}

int kva_append_decode(kva_cache *c, int32_t layer, void *q, const void *k, const void *v, const void *q_norm_w,
                      const void *k_norm_w, const void *cos_tab, const void *sin_tab, int32_t table_rows, void *out,
                      kva_stream_t stream) {
    int rc = capture_check(c, stream);
    if (rc) return capture_note(c, rc);
    rc = append_decode_impl(c, layer, q, k, v, q_norm_w, k_norm_w, cos_tab, sin_tab, table_rows, nullptr, 0, out,
                            stream);
    if (rc == KVA_OK && c->capturing)
        c->cap_table_rows = c->cap_table_rows ? std::min(c->cap_table_rows, table_rows) : table_rows;
    return capture_note(c, rc);
}

int kva_append_decode_gated(kva_cache *c, int32_t layer, void *q, const void *k, const void *v,
                            const void *q_norm_w, const void *k_norm_w, const void *cos_tab, const void *sin_tab,
                            int32_t table_rows, const void *gate, int64_t gate_stride, void *out,
                            kva_stream_t stream) {
    int rc = capture_check(c, stream);
    if (rc) return capture_note(c, rc);
    if (!gate) return capture_note(c, fail(KVA_ERR_INVALID_ARG, "NULL gate"));
    rc = append_decode_impl(c, layer, q, k, v, q_norm_w, k_norm_w, cos_tab, sin_tab, table_rows, gate, gate_stride,
                            out, stream);
    if (rc == KVA_OK && c->capturing)
        c->cap_table_rows = c->cap_table_rows ? std::min(c->cap_table_rows, table_rows) : table_rows;
    return capture_note(c, rc);
}

int kva_append_qknorm_rope(kva_cache *c, int32_t layer, void *q, void *k, const void *v,
                           const void *q_norm_w, const void *k_norm_w, const void *cos_tab,
                           const void *sin_tab, int32_t table_rows, kva_stream_t stream) {
    int rc = capture_check(c, stream);
    if (rc) return capture_note(c, rc);
    rc = append_impl(c, layer, q, k, v, q_norm_w, k_norm_w, cos_tab, sin_tab, table_rows, stream);
    if (rc == KVA_OK && c->capturing && c->st_n_tok > 0)
        c->cap_table_rows = c->cap_table_rows ? std::min(c->cap_table_rows, table_rows) : table_rows;
    return capture_note(c, rc);
}

int kva_project_append(kva_cache *c, int32_t layer, const void *x, int32_t hidden, const void *w_q_fused,
                       const void *w_kv_fused, const void *q_norm_w, const void *k_norm_w, const void *cos_tab,
                       const void *sin_tab, int32_t table_rows, void *q_out, void *q_gate_out, void *kv_out,
                       kva_stream_t stream) {
    int rc = capture_check(c, stream);
    if (rc) return capture_note(c, rc);
    rc = project_impl(c, layer, x, hidden, w_q_fused, w_kv_fused, q_norm_w, k_norm_w, cos_tab, sin_tab, table_rows,
                      q_out, q_gate_out, kv_out, stream);
    if (rc == KVA_OK && c->capturing && c->st_n_tok > 0)
        c->cap_table_rows = c->cap_table_rows ? std::min(c->cap_table_rows, table_rows) : table_rows;
    return capture_note(c, rc);
}

static int out_project_impl(kva_cache *c, const void *attn, int32_t n_tok, int32_t q_dim, const void *w_o,
                            int32_t n_out, const void *residual, void *out, kva_stream_t stream) {
    if (!c) return fail(KVA_ERR_INVALID_ARG, "cache is NULL");
    if (n_tok < 0) return fail(KVA_ERR_INVALID_ARG, "n_tok %d is negative", n_tok);
    if (n_tok == 0) return require_device(c);
    if (!attn || !w_o || !out) return fail(KVA_ERR_INVALID_ARG, "NULL tensor pointer");
    if (!aligned16(attn) || !aligned16(w_o) || !aligned16(residual) || !aligned16(out))
        return fail(KVA_ERR_MISALIGNED, "attn, w_o, residual and out must be 16-byte aligned");
    if (q_dim <= 0 || q_dim % kva::kProjHiddenQuantum != 0)
        return fail(KVA_ERR_INVALID_ARG, "q_dim %d must be a positive multiple of %d", q_dim,
                    kva::kProjHiddenQuantum);
    if (static_cast<int64_t>(kva::kProjTokens) * q_dim * 2 > INT32_MAX)
        return fail(KVA_ERR_INVALID_ARG, "q_dim %d too large", q_dim);
    if (n_out <= 0 || n_out % 16 != 0)
        return fail(KVA_ERR_INVALID_ARG, "n_out %d must be a positive multiple of 16", n_out);
    if (static_cast<int64_t>(n_tok) * n_out > INT32_MAX)
        return fail(KVA_ERR_INVALID_ARG, "n_tok x n_out too large");
    kva::ProjectArgs a{};
    a.w_a = static_cast<const uint16_t *>(w_o);
    a.w_b = a.w_a;
    a.n_a = n_out;
    a.n_b = 0;
    a.hidden = q_dim;
    a.splits = project_splits(c, q_dim, n_out);
    // One launch pair's partials: [splits][its tokens][n_out] floats.
    const int64_t chunk_tok = std::min(n_tok, kva::kProjTokens);
    if (static_cast<size_t>(a.splits) * chunk_tok * n_out > c->proj_floats)
        return fail(KVA_ERR_INVALID_ARG, "n_out %d x %lld tokens exceeds the projection workspace (%zu floats)", n_out,
                    static_cast<long long>(chunk_tok), c->proj_floats);
    if (int rc = require_device(c)) return rc;
    a.part = c->d_proj;
    a.ev_before = c->kev_before;
    a.ev_after = c->kev_after;
    a.y_out = static_cast<uint16_t *>(out);
    a.residual = static_cast<const uint16_t *>(residual);
    const auto *xs = static_cast<const uint16_t *>(attn);
    for (int32_t t0 = 0; t0 < n_tok; t0 += kva::kProjTokens) {
        a.tok0 = t0;
        a.n_tok = std::min(kva::kProjTokens, n_tok - t0);
        a.x = xs + static_cast<size_t>(t0) * q_dim;
        KVA_HIP(kva::launch_out_project(a, static_cast<hipStream_t>(stream)));
    }
    return KVA_OK;
}

int kva_out_project(kva_cache *c, const void *attn, int32_t n_tok, int32_t q_dim, const void *w_o, int32_t n_out,
                    const void *residual, void *out, kva_stream_t stream) {
    int rc = capture_check(c, stream);
    if (rc) return capture_note(c, rc);
    return capture_note(c, out_project_impl(c, attn, n_tok, q_dim, w_o, n_out, residual, out, stream));
}

int kva_decode(kva_cache *c, int32_t layer, const void *q, void *out, kva_stream_t stream) {
    int rc = capture_check(c, stream);
    if (rc) return capture_note(c, rc);
    return capture_note(c, decode_impl(c, layer, q, nullptr, 0, out, stream));
}

int kva_decode_gated(kva_cache *c, int32_t layer, const void *q, const void *gate, int64_t gate_stride,
                     void *out, kva_stream_t stream) {
    int rc = capture_check(c, stream);
    if (rc) return capture_note(c, rc);
    if (!gate) return capture_note(c, fail(KVA_ERR_INVALID_ARG, "NULL gate"));
    return capture_note(c, decode_impl(c, layer, q, gate, gate_stride, out, stream));
}

// Causal prefill or tree verify over the step; with `append`
// (kva_append_prefill) the step's append launch goes first.
static int multi_query(kva_cache *c, int32_t layer, const void *q, void *out, kva_stream_t stream,
                       bool tree, const void *gate = nullptr, int64_t gate_stride = 0,
                       const kva::AppendArgs *append = nullptr, const char *what = nullptr) {
    if (int rc = refuse_while_capturing(c, what ? what : tree ? "kva_tree_verify" : "kva_prefill")) return rc;
    if (!c) return fail(KVA_ERR_INVALID_ARG, "cache is NULL");
    int rc = check_layer(c, layer);
    if (rc) return rc;
    if (!c->step_valid) return fail(KVA_ERR_STATE, "no step begun (kva_step_begin)");
    if (tree && !c->st_has_bits) return fail(KVA_ERR_STATE, "tree verify needs tree_bits in kva_step_begin");
    if (!q || !out) return fail(KVA_ERR_INVALID_ARG, "NULL tensor pointer");
    if (!aligned16(q) || !aligned16(out)) return fail(KVA_ERR_MISALIGNED, "q/out must be 16-byte aligned");
    if ((rc = check_gate(gate, gate_stride, c->cfg.num_heads))) return rc;
    if ((rc = require_device(c))) return rc;
    if (c->st_n_tok == 0) return KVA_OK;
    if (append) KVA_HIP(kva::launch_append(*append, static_cast<hipStream_t>(stream)));
    kva::MultiQueryArgs a{};
    a.gate = static_cast<const uint16_t *>(gate);
    a.gate_stride = gate_stride;
    a.q = static_cast<const uint16_t *>(q);
    a.out = static_cast<uint16_t *>(out);
    a.k_pool = c->d_k + c->layer_elems * layer;
    a.v_pool = c->d_v + c->layer_elems * layer;
    a.table = c->d_table;
    a.table_stride = c->cfg.max_blocks_per_seq;
    a.seq_ids = at<int32_t>(c->d_step, c->off_seq);
    a.ctx_lens = at<int32_t>(c->d_step, c->off_ctx);
    a.new_start = at<int32_t>(c->d_step, c->off_start);
    a.tok_off = at<int32_t>(c->d_step, c->off_tokoff);
    a.tok_bits = tree ? at<uint64_t>(c->d_step, c->off_bits) : nullptr;
    a.upre = at<int32_t>(c->d_step, c->off_upre);
    a.mq_pre = at<int32_t>(c->d_step, c->off_mqpre);
    a.n_seqs = c->st_n_seqs;
    a.n_units = c->st_mq_units;
    a.total_blocks = c->st_mq_blocks;
    a.keys = c->st_mq_keys;
    // Stream-K share: one workgroup per CU, at least 128 keys' blocks each
    // (kva::mq_wg_count, as kva_step_begin found the cut units from it).
    a.n_wg = c->st_mq_wg;
    a.mq_cut = at<int32_t>(c->d_step, c->off_cut);
    a.n_cut = c->st_mq_cut;
    a.num_heads = c->cfg.num_heads;
    a.num_kv_heads = c->cfg.num_kv_heads;
    a.tree = tree ? 1 : 0;
    a.n_waves = c->st_mq_waves;
    a.n_t = 1;
    a.q_tile = c->st_mq_q;
    a.ws_acc = c->d_mq_acc;
    a.ws_ml = c->d_mq_ml;
    a.ev_before = c->kev_before;
    a.ev_after = c->kev_after;
    const hipError_t e = kva::launch_multi_query(a, static_cast<hipStream_t>(stream));
    if (e == hipErrorNotSupported)
        return fail(KVA_ERR_UNSUPPORTED, "multi-query attention kernel not available for this shape");
    if (e != hipSuccess) return hip_fail(e, "launch_multi_query");
    return KVA_OK;
}

int kva_prefill(kva_cache *c, int32_t layer, const void *q, void *out, kva_stream_t stream) {
    return multi_query(c, layer, q, out, stream, false);
}

int kva_tree_verify(kva_cache *c, int32_t layer, const void *q, void *out, kva_stream_t stream) {
    return multi_query(c, layer, q, out, stream, true);
}

int kva_prefill_gated(kva_cache *c, int32_t layer, const void *q, const void *gate, int64_t gate_stride,
                      void *out, kva_stream_t stream) {
    if (!gate) return fail(KVA_ERR_INVALID_ARG, "NULL gate");
    return multi_query(c, layer, q, out, stream, false, gate, gate_stride);
}

int kva_tree_verify_gated(kva_cache *c, int32_t layer, const void *q, const void *gate, int64_t gate_stride,
                          void *out, kva_stream_t stream) {
    if (!gate) return fail(KVA_ERR_INVALID_ARG, "NULL gate");
    return multi_query(c, layer, q, out, stream, true, gate, gate_stride);
}

static int append_prefill_impl(kva_cache *c, int32_t layer, void *q, const void *k, const void *v,
                               const void *q_norm_w, const void *k_norm_w, const void *cos_tab,
                               const void *sin_tab, int32_t table_rows, const void *gate, int64_t gate_stride,
                               void *out, kva_stream_t stream, const char *what) {
    if (int rc = refuse_while_capturing(c, what)) return rc;
    if (!c) return fail(KVA_ERR_INVALID_ARG, "cache is NULL");
    int rc = check_layer(c, layer);
    if (rc) return rc;
    if (!c->step_valid) return fail(KVA_ERR_STATE, "no step begun (kva_step_begin)");
    kva::AppendArgs ap;
    if ((rc = make_append(c, layer, q, const_cast<void *>(k), v, q_norm_w, k_norm_w, cos_tab, sin_tab, table_rows,
                          ap)))
        return rc;
    ap.keep_k = 1;  // k is only read; the cache gets the normalised rows
    return multi_query(c, layer, q, out, stream, false, gate, gate_stride, &ap, what);
}

int kva_append_prefill(kva_cache *c, int32_t layer, void *q, const void *k, const void *v,
                       const void *q_norm_w, const void *k_norm_w, const void *cos_tab, const void *sin_tab,
                       int32_t table_rows, void *out, kva_stream_t stream) {
    return append_prefill_impl(c, layer, q, k, v, q_norm_w, k_norm_w, cos_tab, sin_tab, table_rows, nullptr, 0,
                               out, stream, "kva_append_prefill");
}

int kva_append_prefill_gated(kva_cache *c, int32_t layer, void *q, const void *k, const void *v,
                             const void *q_norm_w, const void *k_norm_w, const void *cos_tab, const void *sin_tab,
                             int32_t table_rows, const void *gate, int64_t gate_stride, void *out,
                             kva_stream_t stream) {
    if (!gate) return fail(KVA_ERR_INVALID_ARG, "NULL gate");
    return append_prefill_impl(c, layer, q, k, v, q_norm_w, k_norm_w, cos_tab, sin_tab, table_rows, gate,
                               gate_stride, out, stream, "kva_append_prefill_gated");
}

int kva_rollback(kva_cache *c, int32_t n_seqs, const int32_t *seq_ids, const int32_t *base_len,
                 const int32_t *keep_off, const int32_t *keep_rows, kva_stream_t stream) {
    if (!c) return fail(KVA_ERR_INVALID_ARG, "cache is NULL");
    if (int rc = refuse_while_capturing(c, "kva_rollback")) return rc;
    if (n_seqs < 0 || n_seqs > c->cfg.max_seqs) return fail(KVA_ERR_INVALID_ARG, "bad n_seqs %d", n_seqs);
    if (n_seqs == 0) return KVA_OK;
    if (!seq_ids || !base_len || !keep_off) return fail(KVA_ERR_INVALID_ARG, "NULL index array");
    if (keep_off[0] != 0) return fail(KVA_ERR_INVALID_ARG, "keep_off[0] must be 0");
    std::vector<uint8_t> seen(c->cfg.max_seqs, 0);
    std::vector<int32_t> moves;
    std::vector<int32_t> move_off(1, 0);
    // Everything is checked, and the upload sized, before any length changes:
    // a refused call leaves the cache as it was.
    size_t n_moves_all = 0, n_groups_all = 0;
    for (int32_t b = 0; b < n_seqs; ++b) {
        const int32_t s = seq_ids[b];
        int rc = check_seq(c, s);
        if (rc) return rc;
        if (seen[s]) return fail(KVA_ERR_INVALID_ARG, "sequence %d listed twice", s);
        seen[s] = 1;
        const int32_t n = keep_off[b + 1] - keep_off[b];
        if (n < 0) return fail(KVA_ERR_INVALID_ARG, "keep_off must be non-decreasing");
        if (n > 0 && !keep_rows) return fail(KVA_ERR_INVALID_ARG, "keep_rows is NULL");
        if (base_len[b] < 0 || base_len[b] > c->len[s])
            return fail(KVA_ERR_ROLLBACK, "sequence %d: base length %d outside [0, %d]", s, base_len[b], c->len[s]);
        int32_t prev = -1;
        size_t n_moved = 0;
        for (int32_t j = 0; j < n; ++j) {
            const int32_t row = keep_rows[keep_off[b] + j];
            if (row <= prev) return fail(KVA_ERR_ROLLBACK, "keep_rows of sequence %d not strictly increasing", s);
            if (static_cast<int64_t>(base_len[b]) + row >= c->len[s])
                return fail(KVA_ERR_ROLLBACK, "sequence %d: kept row %d beyond length %d", s,
                            base_len[b] + row, c->len[s]);
            n_moved += row != j;
            prev = row;
        }
        n_moves_all += n_moved;
        n_groups_all += n_moved > 0;
    }
    if (n_moves_all > 0 &&
        round_up(n_moves_all * 3 * sizeof(int32_t), 16) + (n_groups_all + 1) * sizeof(int32_t) > c->aux_bytes)
        return fail(KVA_ERR_CAPACITY, "rollback moves %zu rows, more than the staging area holds (%zu bytes)",
                    n_moves_all, c->aux_bytes);
    for (int32_t b = 0; b < n_seqs; ++b) {
        const int32_t s = seq_ids[b];
        const int32_t n = keep_off[b + 1] - keep_off[b];
        for (int32_t j = 0; j < n; ++j) {
            const int32_t src = base_len[b] + keep_rows[keep_off[b] + j];
            const int32_t dst = base_len[b] + j;
            if (src != dst) moves.insert(moves.end(), {s, src, dst});
        }
        if (moves.size() / 3 > static_cast<size_t>(move_off.back())) move_off.push_back(static_cast<int32_t>(moves.size() / 3));
        c->len[s] = base_len[b] + n;
    }
    c->step_valid = false;
    const int32_t n_moves = static_cast<int32_t>(moves.size() / 3);
    if (n_moves == 0 || c->host_only) return KVA_OK;
    const int32_t n_groups = static_cast<int32_t>(move_off.size()) - 1;
    const size_t bytes_moves = moves.size() * sizeof(int32_t);
    const size_t o_off = round_up(bytes_moves, 16);
    const size_t total = o_off + move_off.size() * sizeof(int32_t);  // fits: checked above
    hipStream_t st = static_cast<hipStream_t>(stream);
    uint8_t *h;
    int idx;
    int rc = acquire_stage(c, &h, &idx);
    if (rc) return rc;
    std::memcpy(h, moves.data(), bytes_moves);
    std::memcpy(h + o_off, move_off.data(), move_off.size() * sizeof(int32_t));
    KVA_HIP(hipMemcpyAsync(c->d_aux, h, total, hipMemcpyHostToDevice, st));
    if ((rc = release_stage(c, idx, st))) return rc;
    kva::RollbackArgs a{};
    a.k_pools = c->d_k;
    a.v_pools = c->d_v;
    a.layer_elems = c->layer_elems;
    a.n_layers = c->cfg.n_layers;
    a.table = c->d_table;
    a.table_stride = c->cfg.max_blocks_per_seq;
    a.moves = reinterpret_cast<const int32_t *>(c->d_aux);
    a.move_off = reinterpret_cast<const int32_t *>(c->d_aux + o_off);
    a.n_groups = n_groups;
    a.num_kv_heads = c->cfg.num_kv_heads;
    KVA_HIP(kva::launch_rollback(a, st));
    return KVA_OK;
}

int kva_graph_capture_begin(kva_cache *c, kva_stream_t stream) {
    int rc = require_device(c);
    if (rc) return rc;
    if (c->capturing) return fail(KVA_ERR_STATE, "a graph is already being recorded");
    if (!c->step_valid) return fail(KVA_ERR_STATE, "no step begun (kva_step_begin)");
    if (!stream) return fail(KVA_ERR_INVALID_ARG, "recording needs a created stream, not the legacy default stream");
    hipStream_t s = static_cast<hipStream_t>(stream);
    KVA_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    c->capturing = true;
    c->capture_failed = false;
    c->cap_stream = s;
    c->cap_table_rows = 0;
    return KVA_OK;
}

int kva_graph_capture_end(kva_cache *c, kva_stream_t stream, kva_graph **out) {
    if (!c || !out) return fail(KVA_ERR_INVALID_ARG, "NULL argument");
    *out = nullptr;
    if (!c->capturing) return fail(KVA_ERR_STATE, "no graph is being recorded");
    if (static_cast<hipStream_t>(stream) != c->cap_stream)
        return fail(KVA_ERR_INVALID_ARG, "recording was begun on another stream");
    c->capturing = false;
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(c->cap_stream, &graph);
    if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
    if (c->capture_failed) {
        (void)hipGraphDestroy(graph);
        return fail(KVA_ERR_STATE, "a call failed while the graph was being recorded; nothing was kept");
    }
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
    auto *g = new kva_graph;
    g->cache = c;
    g->exec = exec;
    g->n_seqs = c->st_n_seqs;
    g->n_tok = c->st_n_tok;
    g->table_rows = c->cap_table_rows;
    g->all_one = c->st_all_one;
    g->has_bits = c->st_has_bits;
    const size_t offs[12] = {c->off_seq,  c->off_ctx,  c->off_start, c->off_tokoff, c->off_tseq,  c->off_tslot,
                             c->off_tpos, c->off_bits, c->off_pre,   c->off_upre,   c->off_mqpre, c->off_pids};
    std::memcpy(g->offs, offs, sizeof(offs));
    *out = g;
    return KVA_OK;
}

int kva_graph_launch(kva_graph *g, kva_stream_t stream) {
    if (!g || !g->cache) return fail(KVA_ERR_INVALID_ARG, "graph is NULL");
    kva_cache *c = g->cache;
    if (c->capturing) return fail(KVA_ERR_STATE, "a graph is being recorded");
    if (!c->step_valid) return fail(KVA_ERR_STATE, "no step begun (kva_step_begin)");
    const size_t offs[12] = {c->off_seq,  c->off_ctx,  c->off_start, c->off_tokoff, c->off_tseq,  c->off_tslot,
                             c->off_tpos, c->off_bits, c->off_pre,   c->off_upre,   c->off_mqpre, c->off_pids};
    if (c->st_n_seqs != g->n_seqs || c->st_n_tok != g->n_tok || c->st_all_one != g->all_one ||
        c->st_has_bits != g->has_bits || std::memcmp(offs, g->offs, sizeof(offs)) != 0)
        return fail(KVA_ERR_STATE, "the current step (%d sequences, %d tokens) is not the recorded shape (%d, %d)",
                    c->st_n_seqs, c->st_n_tok, g->n_seqs, g->n_tok);
    if (g->table_rows > 0 && c->st_max_pos >= g->table_rows)
        return fail(KVA_ERR_INVALID_ARG, "RoPE position %d beyond the %d table rows the graph was recorded with",
                    c->st_max_pos, g->table_rows);
    KVA_HIP(hipGraphLaunch(g->exec, static_cast<hipStream_t>(stream)));
    return KVA_OK;
}

int kva_graph_destroy(kva_graph *g) {
    if (!g) return fail(KVA_ERR_INVALID_ARG, "graph is NULL");
    hipError_t e = g->exec ? hipGraphExecDestroy(g->exec) : hipSuccess;
    delete g;
    if (e != hipSuccess) return hip_fail(e, "hipGraphExecDestroy");
    return KVA_OK;
}

int kva_legacy_qknorm_rope(void *x, const void *w, const void *cos_row, const void *sin_row,
                           void *cache_dst, int32_t num_heads, int32_t head_dim, int32_t half_rotary,
                           float eps, kva_stream_t stream) {
    if (!x || !w) return fail(KVA_ERR_INVALID_ARG, "x / w is NULL");
    if (num_heads < 0) return fail(KVA_ERR_INVALID_ARG, "num_heads %d < 0", num_heads);
    if (!(head_dim == 64 || head_dim == 128 || head_dim == 256))
        return fail(KVA_ERR_UNSUPPORTED, "head_dim %d unsupported (64, 128, 256)", head_dim);
    if (half_rotary < 0 || half_rotary % 4 != 0 || 2 * half_rotary > head_dim)
        return fail(KVA_ERR_UNSUPPORTED, "half_rotary %d must be a multiple of 4 with 2*half_rotary <= head_dim",
                    half_rotary);
    if (half_rotary > 0 && (!cos_row || !sin_row)) return fail(KVA_ERR_INVALID_ARG, "cos/sin row is NULL");
    if (!aligned16(x) || !aligned16(w) || (cache_dst && !aligned16(cache_dst)))
        return fail(KVA_ERR_MISALIGNED, "x, w and cache_dst must be 16-byte aligned");
    if (half_rotary > 0 && ((reinterpret_cast<uintptr_t>(cos_row) | reinterpret_cast<uintptr_t>(sin_row)) & 7u))
        return fail(KVA_ERR_MISALIGNED, "cos/sin rows must be 8-byte aligned");
    if (!(eps >= 0.0f)) return fail(KVA_ERR_INVALID_ARG, "eps must be >= 0");
    kva::LegacyNormArgs a{};
    a.x = static_cast<uint16_t *>(x);
    a.w = static_cast<const uint16_t *>(w);
    a.cos_row = static_cast<const uint16_t *>(cos_row);
    a.sin_row = static_cast<const uint16_t *>(sin_row);
    a.cache_dst = static_cast<uint16_t *>(cache_dst);
    a.num_heads = num_heads;
    a.head_dim = head_dim;
    a.half_rot = half_rotary;
    a.eps = eps;
    KVA_HIP(kva::launch_legacy_norm(a, static_cast<hipStream_t>(stream)));
    return KVA_OK;
}

// noalloc: take the split-K partials from the library's static device
// scratch (kva_legacy_decode_noalloc) instead of a cache's workspace.
static int legacy_decode(kva_cache *ws, const void *q, const void *gate, const void *k_base, const void *v_base,
                         void *out, int32_t kv_seq_len, int32_t batch, int64_t batch_stride,
                         int32_t num_heads, int32_t num_kv_heads, kva_stream_t stream,
                         bool noalloc = false) {
    if (!q || !k_base || !v_base || !out) return fail(KVA_ERR_INVALID_ARG, "NULL tensor pointer");
    if (kv_seq_len <= 0) return fail(KVA_ERR_INVALID_ARG, "kv_seq_len %d must be positive", kv_seq_len);
    if (batch <= 0 || batch > 65535) return fail(KVA_ERR_INVALID_ARG, "batch %d outside [1, 65535]", batch);
    if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0)
        return fail(KVA_ERR_INVALID_ARG, "num_heads %d must be a positive multiple of num_kv_heads %d",
                    num_heads, num_kv_heads);
    const int g = num_heads / num_kv_heads;
    if (!(g == 1 || g == 2 || g == 3 || g == 4 || g == 6 || g == 8))
        return fail(KVA_ERR_UNSUPPORTED, "GQA group %d unsupported", g);
    if (!aligned16(q) || !aligned16(k_base) || !aligned16(v_base) || !aligned16(out))
        return fail(KVA_ERR_MISALIGNED, "q, K, V and out must be 16-byte aligned");
    const int64_t row_bytes = static_cast<int64_t>(num_kv_heads) * kva::kHeadDim * 2;
    if (batch > 1 && (batch_stride % 16 != 0 || batch_stride < row_bytes * kv_seq_len))
        return fail(KVA_ERR_INVALID_ARG, "batch_stride %lld must be a multiple of 16 covering %d rows",
                    static_cast<long long>(batch_stride), kv_seq_len);
    if (ws && ws->host_only) return fail(KVA_ERR_NO_DEVICE, "workspace cache is host-only");
    if (int rc = check_gate(gate, static_cast<int64_t>(num_heads) * kva::kHeadDim, num_heads)) return rc;
    kva::DecodeArgs a{};
    a.gate = static_cast<const uint16_t *>(gate);
    a.gate_stride = static_cast<int64_t>(num_heads) * kva::kHeadDim;
    a.q = static_cast<const uint16_t *>(q);
    a.k_pool = static_cast<const uint16_t *>(k_base);
    a.v_pool = static_cast<const uint16_t *>(v_base);
    a.seq_stride = static_cast<size_t>(batch_stride / 2);
    a.ctx_len_const = kv_seq_len;
    a.n_seqs = batch;
    a.num_heads = num_heads;
    a.num_kv_heads = num_kv_heads;
    // Every sequence has the same length: the page prefix sums are implicit.
    const int64_t unit_pages = (kv_seq_len + kva::kBlockTokens - 1) / kva::kBlockTokens;
    const int64_t pages = unit_pages * batch;
    // Without a workspace (and not the allocation-free entry point) only the
    // whole-sequence form can run, which needs none: it gives each kv head
    // one workgroup, so a long cache would stream on a few CUs.  Such calls
    // are refused rather than run an order of magnitude below the split form.
    if (!ws && !noalloc && kv_seq_len > kWholeMaxTokens)
        return fail(KVA_ERR_STATE,
                    "kv_seq_len %d > %d needs a workspace cache (ws) for its split-K partials, or "
                    "kva_legacy_decode_noalloc",
                    kv_seq_len, kWholeMaxTokens);
    if (noalloc && num_heads > kva::kNoAllocMaxHeads)
        return fail(KVA_ERR_CAPACITY, "num_heads %d: the static decode scratch (%zu bytes) serves at most %d heads",
                    num_heads, kva::kNoAllocScratchBytes, kva::kNoAllocMaxHeads);
    int n_cu = ws ? ws->n_cu : 0;
    if (!ws) {
        int dev = 0;
        KVA_HIP(hipGetDevice(&dev));
        KVA_HIP(hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev));
    }
    if ((a.whole = use_whole(ws, ws ? ws->split_user : 0, kv_seq_len, batch, num_heads,
                             num_kv_heads, std::max(1, n_cu)))) {
    } else if (noalloc) {
        void *scratch = nullptr;
        int n_cu = 0;
        KVA_HIP(kva::noalloc_scratch(&scratch, &n_cu));
        // Two partial slots of num_heads rows (256 + 2 floats) per workgroup.
        const int64_t slot_bytes = static_cast<int64_t>(num_heads) * (kva::kHeadDim + 2) * sizeof(float);
        const int64_t fit = static_cast<int64_t>(kva::kNoAllocScratchBytes) / (2 * slot_bytes);
        a.total_pages = static_cast<int32_t>(pages);
        a.n_wg = static_cast<int32_t>(std::max<int64_t>(
            1, std::min<int64_t>({static_cast<int64_t>(n_cu) * kDecodeWgPerCu,
                                  (pages + kMinPagesPerWg - 1) / kMinPagesPerWg, fit})));
        a.ws_acc = static_cast<float *>(scratch);
        a.ws_ml = a.ws_acc + static_cast<size_t>(2) * a.n_wg * num_heads * kva::kHeadDim;
    } else {
        set_stream_k(ws, a, pages, num_heads);
    }
    if (!a.whole) a.combine_waves = combine_waves_for(unit_pages, pages, a.n_wg);
    a.out = static_cast<uint16_t *>(out);
    KVA_HIP(kva::launch_decode(a, static_cast<hipStream_t>(stream)));
    return KVA_OK;
}

int kva_legacy_decode_noalloc(const void *q, const void *k_base, const void *v_base, void *out,
                              int32_t kv_seq_len, int32_t num_heads, int32_t num_kv_heads,
                              kva_stream_t stream) {
    return legacy_decode(nullptr, q, nullptr, k_base, v_base, out, kv_seq_len, 1, 0, num_heads, num_kv_heads,
                         stream, true);
}

int kva_legacy_decode(kva_cache *ws, const void *q, const void *k_base, const void *v_base,
                      void *out, int32_t kv_seq_len, int32_t num_heads, int32_t num_kv_heads,
                      kva_stream_t stream) {
    return legacy_decode(ws, q, nullptr, k_base, v_base, out, kv_seq_len, 1, 0, num_heads, num_kv_heads, stream);
}

int kva_legacy_decode_batched(kva_cache *ws, const void *q, const void *k_base, const void *v_base,
                              void *out, int32_t kv_seq_len, int32_t batch, int64_t batch_stride,
                              int32_t num_heads, int32_t num_kv_heads, kva_stream_t stream) {
    return legacy_decode(ws, q, nullptr, k_base, v_base, out, kv_seq_len, batch, batch_stride, num_heads,
                         num_kv_heads, stream);
}

int kva_legacy_decode_gated(kva_cache *ws, const void *q, const void *gate, const void *k_base,
                            const void *v_base, void *out, int32_t kv_seq_len, int32_t num_heads,
                            int32_t num_kv_heads, kva_stream_t stream) {
    if (!gate) return fail(KVA_ERR_INVALID_ARG, "NULL gate");
    return legacy_decode(ws, q, gate, k_base, v_base, out, kv_seq_len, 1, 0, num_heads, num_kv_heads, stream);
}

int kva_hbm_copy(void *dst, const void *src, size_t bytes, kva_stream_t stream) {
    if (!dst || !src) return fail(KVA_ERR_INVALID_ARG, "NULL pointer");
    if (bytes % 16 != 0) return fail(KVA_ERR_INVALID_ARG, "bytes %zu not a multiple of 16", bytes);
    if (!aligned16(dst) || !aligned16(src)) return fail(KVA_ERR_MISALIGNED, "pointers must be 16-byte aligned");
    KVA_HIP(kva::launch_copy(dst, src, bytes, static_cast<hipStream_t>(stream)));
    return KVA_OK;
}

int kva_hbm_read(const void *src, size_t bytes, void *sink, kva_stream_t stream) {
    if (!src || !sink) return fail(KVA_ERR_INVALID_ARG, "NULL pointer");
    if (bytes % 16 != 0) return fail(KVA_ERR_INVALID_ARG, "bytes %zu not a multiple of 16", bytes);
    if (!aligned16(src) || (reinterpret_cast<uintptr_t>(sink) & 3u))
        return fail(KVA_ERR_MISALIGNED, "src must be 16-byte and sink 4-byte aligned");
    KVA_HIP(kva::launch_read(src, bytes, static_cast<uint32_t *>(sink), static_cast<hipStream_t>(stream)));
    return KVA_OK;
}

int kva_hbm_read_pages(const void *k_pool, const void *v_pool, const int32_t *page_ids, int32_t n_pages,
                       int32_t num_kv_heads, int32_t n_wg, void *sink, kva_stream_t stream) {
    if (!k_pool || !v_pool || !page_ids || !sink) return fail(KVA_ERR_INVALID_ARG, "NULL pointer");
    if (n_pages < 0) return fail(KVA_ERR_INVALID_ARG, "n_pages %d < 0", n_pages);
    if (num_kv_heads < 1 || num_kv_heads > 16)
        return fail(KVA_ERR_UNSUPPORTED, "num_kv_heads %d outside [1, 16]", num_kv_heads);
    if (n_wg < 1 || n_wg > 65535) return fail(KVA_ERR_INVALID_ARG, "n_wg %d outside [1, 65535]", n_wg);
    if (!aligned16(k_pool) || !aligned16(v_pool) || (reinterpret_cast<uintptr_t>(page_ids) & 3u) ||
        (reinterpret_cast<uintptr_t>(sink) & 3u))
        return fail(KVA_ERR_MISALIGNED, "pools must be 16-byte, page ids and sink 4-byte aligned");
    KVA_HIP(kva::launch_read_pages(k_pool, v_pool, page_ids, n_pages, num_kv_heads, n_wg, static_cast<uint32_t *>(sink),
                                   static_cast<hipStream_t>(stream)));
    return KVA_OK;
}

// ---- device helpers -------------------------------------------------------
int kva_dev_count(int32_t *n) {
    if (!n) return fail(KVA_ERR_INVALID_ARG, "NULL argument");
    int c = 0;
    KVA_HIP(hipGetDeviceCount(&c));
    *n = c;
    return KVA_OK;
}
int kva_dev_props(int32_t *n_cu, int32_t *clock_khz, int32_t *mem_clock_khz, int32_t *mem_bus_bits) {
    if (!n_cu || !clock_khz || !mem_clock_khz || !mem_bus_bits) return fail(KVA_ERR_INVALID_ARG, "NULL argument");
    int dev = 0;
    KVA_HIP(hipGetDevice(&dev));
    hipDeviceProp_t p{};
    KVA_HIP(hipGetDeviceProperties(&p, dev));
    *n_cu = p.multiProcessorCount;
    *clock_khz = p.clockRate;
    *mem_clock_khz = p.memoryClockRate;
    *mem_bus_bits = p.memoryBusWidth;
    return KVA_OK;
}
int kva_dev_set(int32_t d) {
    KVA_HIP(hipSetDevice(d));
    return KVA_OK;
}
int kva_dev_malloc(void **p, size_t n) {
    if (!p) return fail(KVA_ERR_INVALID_ARG, "NULL argument");
    KVA_HIP(hipMalloc(p, n));
    return KVA_OK;
}
int kva_dev_free(void *p) {
    KVA_HIP(hipFree(p));
    return KVA_OK;
}
int kva_memcpy_h2d(void *d, const void *s, size_t n) {
    KVA_HIP(hipMemcpy(d, s, n, hipMemcpyHostToDevice));
    return KVA_OK;
}
int kva_memcpy_d2h(void *d, const void *s, size_t n) {
    KVA_HIP(hipMemcpy(d, s, n, hipMemcpyDeviceToHost));
    return KVA_OK;
}
int kva_memcpy_d2d(void *d, const void *s, size_t n) {
    KVA_HIP(hipMemcpy(d, s, n, hipMemcpyDeviceToDevice));
    return KVA_OK;
}
int kva_memset(void *d, int32_t v, size_t n) {
    KVA_HIP(hipMemset(d, v, n));
    return KVA_OK;
}
int kva_dev_synchronize(void) {
    KVA_HIP(hipDeviceSynchronize());
    return KVA_OK;
}
int kva_stream_create(kva_stream_t *s) {
    if (!s) return fail(KVA_ERR_INVALID_ARG, "NULL argument");
    hipStream_t st;
    KVA_HIP(hipStreamCreate(&st));
    *s = st;
    return KVA_OK;
}
int kva_stream_destroy(kva_stream_t s) {
    KVA_HIP(hipStreamDestroy(static_cast<hipStream_t>(s)));
    return KVA_OK;
}
int kva_stream_synchronize(kva_stream_t s) {
    KVA_HIP(hipStreamSynchronize(static_cast<hipStream_t>(s)));
    return KVA_OK;
}
int kva_event_create(kva_event_t *ev) {
    if (!ev) return fail(KVA_ERR_INVALID_ARG, "NULL argument");
    hipEvent_t e;
    KVA_HIP(hipEventCreate(&e));
    *ev = e;
    return KVA_OK;
}
int kva_event_destroy(kva_event_t ev) {
    KVA_HIP(hipEventDestroy(static_cast<hipEvent_t>(ev)));
    return KVA_OK;
}
int kva_event_record(kva_event_t ev, kva_stream_t s) {
    KVA_HIP(hipEventRecord(static_cast<hipEvent_t>(ev), static_cast<hipStream_t>(s)));
    return KVA_OK;
}
int kva_event_synchronize(kva_event_t ev) {
    KVA_HIP(hipEventSynchronize(static_cast<hipEvent_t>(ev)));
    return KVA_OK;
}
int kva_event_elapsed_ms(float *ms, kva_event_t a, kva_event_t b) {
    if (!ms) return fail(KVA_ERR_INVALID_ARG, "NULL argument");
    KVA_HIP(hipEventElapsedTime(ms, static_cast<hipEvent_t>(a), static_cast<hipEvent_t>(b)));
    return KVA_OK;
}

}  // extern "C"
