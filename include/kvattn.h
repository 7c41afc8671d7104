/*
 * kvattn.h — C ABI of libkvattn.so, the MI355X (gfx950) full-attention
 * KV-cache path: paged FP16 K/V cache, fused QK-RMSNorm + RoPE + K/V append,
 * split-K GQA decode, chunked causal prefill and tree-verify attention.
 *
 * Conventions (the reference's host wrappers use the same ones):
 *   - every pointer argument named q, k, v, out, x, w, cos_*, sin_*, *_base,
 *     cache_dst is a DEVICE address; index arrays (seq_ids, n_new, ...) are
 *     HOST arrays unless stated otherwise;
 *   - fp16 tensors are passed as void* (IEEE binary16, little endian);
 *   - every call returns int: 0 = ok, > 0 = hipError_t from the HIP runtime,
 *     < 0 = one of the KVA_ERR_* validation codes below; kva_last_error_string
 *     gives detail for the calling thread; there are no silent fallbacks;
 *   - kva_stream_t is a hipStream_t (NULL = the legacy default stream); a
 *     cache is driven from one host thread and its calls are ordered on the
 *     stream they are given: calls on different streams must be ordered by
 *     the caller.  A cache owns one set of workspaces (decode, multi-query
 *     and projection partials, the step plan) shared by every call on it,
 *     so two calls on one cache that overlap on different streams race:
 *     use one stream per cache, or one cache per stream;
 *   - the library allocates device memory in kva_create and the kva_dev_*
 *     helpers, and in kva_timeline_enable (the timeline buffer).  No other
 *     call allocates; kva_legacy_decode_noalloc allocates nothing at all;
 *   - every call validates its arguments before it touches the device, so a
 *     host-only cache (KVA_FLAG_HOST_ONLY) reports the same refusals and
 *     answers a call that would pass them with KVA_ERR_NO_DEVICE.
 *
 * Reference citations are to larkinwc/mi50grad (file:line).
 */
#ifndef KVATTN_H
#define KVATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *kva_stream_t;
typedef void *kva_event_t;
typedef struct kva_cache kva_cache;
typedef struct kva_graph kva_graph;

enum {
    KVA_OK = 0,
    KVA_ERR_INVALID_ARG = -1,   /* null pointer, negative count, bad index  */
    KVA_ERR_UNSUPPORTED = -2,   /* shape outside what the kernels implement */
    KVA_ERR_NO_DEVICE = -3,     /* device call on a host-only cache         */
    KVA_ERR_OUT_OF_BLOCKS = -4, /* block pool exhausted                     */
    KVA_ERR_CAPACITY = -5,      /* length beyond max_blocks_per_seq * 16    */
    KVA_ERR_BAD_SEQ = -6,       /* sequence id out of range / not active    */
    KVA_ERR_BAD_BLOCK = -7,     /* block id out of range or already in use  */
    KVA_ERR_STATE = -8,         /* call order (no step begun, wrong mode)   */
    KVA_ERR_ROLLBACK = -9,      /* rollback past the base / unsorted rows   */
    KVA_ERR_MISALIGNED = -10,   /* device pointer not 16-byte aligned       */
    KVA_ERR_DOUBLE_FREE = -11   /* sequence freed twice                     */
};

/* Cache flags. */
#define KVA_FLAG_HOST_ONLY 0x1u /* no device memory: host bookkeeping only  */

/*
 * Cache configuration.  Replaces the constructor arguments of
 * KVCache(config, max_seq_len, device, tp_size, batch_size), engine.py:88-117,
 * whose contiguous [layers][batch][max_seq][kv_heads][256] layout becomes a
 * pool of 16-token pages per layer: [max_blocks][16][num_kv_heads][head_dim].
 */
typedef struct kva_config {
    int32_t n_layers;           /* full-attention layers held (16)          */
    int32_t num_heads;          /* query heads (24)                         */
    int32_t num_kv_heads;       /* KV heads (4); num_heads % this == 0      */
    int32_t head_dim;           /* 256 (the only supported value)           */
    int32_t rotary_dim;         /* 64; RoPE on interleaved pairs of [0,64)  */
    int32_t block_tokens;       /* 16 (the only supported value)            */
    int32_t max_seqs;           /* sequence slots                           */
    int32_t max_blocks;         /* physical blocks in each layer's pool     */
    int32_t max_blocks_per_seq; /* block-table width                        */
    int32_t max_step_tokens;    /* most new tokens in one step, all seqs    */
    float eps;                  /* RMSNorm epsilon (1e-6)                   */
    uint32_t flags;             /* KVA_FLAG_*                               */
} kva_config;

/* Byte layout of the pools, for callers that address rows themselves. */
typedef struct kva_layout {
    uint64_t row_bytes;   /* one token, all KV heads: kv_heads*head_dim*2   */
    uint64_t block_bytes; /* block_tokens * row_bytes                       */
    uint64_t layer_bytes; /* max_blocks * block_bytes (per K or V pool)     */
    int32_t block_tokens;
    int32_t max_blocks_per_seq;
} kva_layout;

/* ---- lifetime ---------------------------------------------------------- */
/* KVCache.__init__ (engine.py:88-117) and cleanup() (engine.py:288-290).   */
int kva_create(const kva_config *cfg, kva_cache **out);
int kva_destroy(kva_cache *cache);
const char *kva_last_error_string(void);
const char *kva_version(void);
int kva_get_layout(const kva_cache *cache, kva_layout *out);
/* Device base of layer `layer`'s K and V pools: KVCache.layer_k_ptr /
 * layer_v_ptr (engine.py:123-156) for the paged layout.                    */
int kva_layer_pools(const kva_cache *cache, int32_t layer, void **k_pool, void **v_pool);

/* ---- host block management (no device work) ---------------------------- */
/* Ensure sequence `seq_id` can hold n_tokens rows, taking free blocks from
 * the pool.  The reference pre-allocates max_seq_len rows per batch slot
 * (engine.py:101-117); here capacity grows a page at a time.               */
int kva_seq_reserve(kva_cache *cache, int32_t seq_id, int32_t n_tokens);
/* Give sequence `seq_id` an explicit block list (e.g. a permuted one).  The
 * blocks must be free; the sequence's previous blocks are released.  Ends
 * the current step (the step plan holds block ids), as kva_seq_set_len and
 * kva_seq_free do: begin a new one before the next hot-path call.          */
int kva_seq_set_blocks(kva_cache *cache, int32_t seq_id, const int32_t *block_ids,
                       int32_t n_blocks);
/* Release a sequence's blocks and set its length to 0: KVCache.reset()
 * (engine.py:228-230) for one sequence.                                    */
int kva_seq_free(kva_cache *cache, int32_t seq_id);
int kva_seq_get_len(const kva_cache *cache, int32_t seq_id, int32_t *len);
/* Set the committed length (the reference's `current_len`, engine.py:94,
 * written by callers at engine.py:3283 and tp_engine.py:1684).  Rows at or
 * beyond the new length become invisible; capacity must already exist.    */
int kva_seq_set_len(kva_cache *cache, int32_t seq_id, int32_t len);
int kva_seq_get_blocks(const kva_cache *cache, int32_t seq_id, int32_t *block_ids,
                       int32_t cap, int32_t *n_blocks);
int kva_free_block_count(const kva_cache *cache, int32_t *n_free);
/* Device address of one logical row: KVCache.get_kv_ptr (engine.py:158-176).
 * Valid for reads/writes of that single [num_kv_heads, head_dim] row.      */
int kva_row_ptr(const kva_cache *cache, int32_t layer, int32_t seq_id, int32_t slot,
                void **k_row, void **v_row);
/* Push block-table changes made by kva_seq_* calls to the device.          */
int kva_sync_tables(kva_cache *cache, kva_stream_t stream);

/* ---- per-step plan ----------------------------------------------------- */
/* Start a step that appends n_new[b] rows to each sequence seq_ids[b]
 * (b < n_seqs; a sequence appears at most once).  New rows take slots
 * len..len+n_new-1; the committed length becomes len+n_new (the reference
 * writes at current_len and then calls advance(), engine.py:220-226).
 * rope_pos (nullable, one per new token in sequence order) overrides the
 * RoPE position, which defaults to the slot; tree verify passes
 * len + depth.  tree_bits (nullable, one per new token) gives, for tree
 * verify, the set of new tokens of the same sequence that token sees
 * (bit j = j-th new token of that sequence; self and ancestors).  One
 * host->device copy on `stream` carries the plan (with the block ids of
 * each sequence's first 64 pages) and any block-table changes; every layer
 * of the step reuses it (the reference patches the same per-step arguments
 * for all layers: c_dispatch.c:426-456).                                   */
int kva_step_begin(kva_cache *cache, int32_t n_seqs, const int32_t *seq_ids,
                   const int32_t *n_new, const int32_t *rope_pos,
                   const uint64_t *tree_bits, kva_stream_t stream);

/* ---- hot path (device work, per layer) --------------------------------- */
/* Fused QK-RMSNorm + interleaved partial RoPE + K/V append for every new
 * token of the step.  Replaces qknorm_rope_fused (qknorm_rope.hip:55-162)
 * launched via _launch_qknorm_rope (engine.py:2371-2399) for Q,
 * qknorm_rope_cachew_fused (qknorm_rope_cachew.hip:52-142) via
 * _launch_qknorm_rope_cachew (engine.py:2401-2432) for K, and the V write
 * into the cache slot (engine.py:2012-2018 / append_kv_gpu :199-218).
 * q [T, num_heads, 256] and k [T, num_kv_heads, 256] are normalised and
 * rotated in place (as the reference kernels do); K is also stored to the
 * cache; v [T, num_kv_heads, 256] is copied to the cache.  T is the step's
 * token count, tokens in sequence order.  cos_tab/sin_tab: [table_rows,
 * rotary_dim/2] fp16 (the tables of _init_rope_tables, engine.py:1025-1046). */
int kva_append_qknorm_rope(kva_cache *cache, int32_t layer, void *q, void *k,
                           const void *v, const void *q_norm_w, const void *k_norm_w,
                           const void *cos_tab, const void *sin_tab, int32_t table_rows,
                           kva_stream_t stream);
/* The Q/K/V projection of every new token of the step, fused with the
 * append above: the producer side of the cache.  Replaces the FP16
 * attention projections (gemv_fp16_v2, gemv_fp16_v2.hip:22-85) launched at
 * engine.py:2000-2022 (per sequence at :1815-1828; from the launch cache at
 * :3367-3400 and c_dispatch.c:1042-1059, where V's GEMV writes into the
 * cache slot) plus the norm/RoPE/append launches of kva_append_qknorm_rope.
 * x: [T, hidden] fp16, the normed hidden states in step token order;
 * hidden a multiple of 512.  w_q_fused: [2*num_heads*256, hidden] fp16, Q
 * rows then Q_gate rows; w_kv_fused: [2*num_kv_heads*256, hidden] fp16, K
 * rows then V rows (the stacked weights of engine.py:1366-1378).  Each
 * projected value is the fp32 sum rounded to fp16 (what the reference's GEMV
 * stores); Q and K are then normalised and rotated exactly as
 * kva_append_qknorm_rope does, K and V go to the cache slots.  Outputs:
 * q_out [T, num_heads, 256] (normalised + rotated Q, the input of
 * kva_decode / kva_prefill / kva_tree_verify); q_gate_out [T, num_heads,
 * 256] (Q_gate as projected, the gate of kva_decode_gated with gate_stride
 * num_heads*256; may be NULL); kv_out [T, 2, num_kv_heads, 256] (K and V as
 * projected, the reference's d_kv_fused; may be NULL).  16-byte aligned.   */
int kva_project_append(kva_cache *cache, int32_t layer, const void *x, int32_t hidden,
                       const void *w_q_fused, const void *w_kv_fused,
                       const void *q_norm_w, const void *k_norm_w,
                       const void *cos_tab, const void *sin_tab, int32_t table_rows,
                       void *q_out, void *q_gate_out, void *kv_out, kva_stream_t stream);
/* How the last kva_project_append on this cache projected: steps of up to
 * 64 tokens through the split-K projection kernels and their finish kernel
 * (the weights are read once per 64 tokens); larger steps through one
 * prefill GEMM launch (the reference's batched prefill GEMM,
 * gemm_fp16_prefill.hip:47 at engine.py:3051-3068) whose tiles of 128
 * tokens x one head's 256 weight rows each finish their own rows: fp32 sums
 * rounded to fp16, then the same norm, RoPE and append.  The results
 * satisfy the same contract either way; this says which ran.               */
#define KVA_PROJECT_KERNELS 0
#define KVA_PROJECT_PREFILL_GEMM 1
int kva_get_project_path(const kva_cache *cache, int32_t *path);
/* Output projection of the (gated) attention rows, the consumer of
 * kva_decode_gated: out[t] = fp16(attn[t] . W_o^T + residual[t]) for
 * t < n_tok, accumulated in fp32 and rounded once after the residual add.
 * Replaces the single-GPU O-projection _launch_gemv_fp16(d_hidden,
 * d_attn_out, o_weight, q_dim, hidden, residual=d_hidden) (engine.py:2083-
 * 2085, launcher engine.py:2434-2455, kernel gemv_fp16_v2.hip:22-87) for
 * all n_tok rows at once.  attn [n_tok, q_dim], w_o [n_out, q_dim] (row
 * major), residual and out [n_tok, n_out], fp16, 16-byte aligned; residual
 * may be NULL (no add) or equal to out (in place).  q_dim a multiple of 512,
 * n_out a multiple of 16 and at most (2*num_heads + 2*num_kv_heads)*256
 * (the projection workspace).  Uses no step state.                        */
int kva_out_project(kva_cache *cache, const void *attn, int32_t n_tok, int32_t q_dim,
                    const void *w_o, int32_t n_out, const void *residual, void *out,
                    kva_stream_t stream);
/* GQA decode attention, one query token per sequence (every n_new == 1):
 * out[b] = softmax(q[b] K^T / 16) V over the sequence's rows [0, len).
 * Replaces flash_attn_256_decode (flash_attn_256_tuned.hip:198-350) as
 * launched by _launch_decode_attn_256 (engine.py:2760-2804) and the batched
 * launcher _launch_decode_attn_256_batched (engine.py:2806-2857), now with
 * ragged per-sequence lengths.  q, out: [n_seqs, num_heads, 256] fp16.     */
int kva_decode(kva_cache *cache, int32_t layer, const void *q, void *out,
               kva_stream_t stream);
/* kva_decode with the attention output gate fused into its epilogue:
 * out = fp16(fp16(attn) * 1/(1+exp(-gate))) elementwise, which is what
 * _launch_sigmoid_mul (sigmoid_mul.hip:10-22) does to the decode output at
 * engine.py:2055-2056, without the extra launch and round trip.  gate:
 * fp16, sequence b's row of num_heads*256 values at gate + b*gate_stride
 * (e.g. gate_stride = 2*num_heads*256 when it is the Q_gate half of a fused
 * [Q | Q_gate] projection output, engine.py:1069-1071); 8-byte aligned.     */
int kva_decode_gated(kva_cache *cache, int32_t layer, const void *q, const void *gate,
                     int64_t gate_stride, void *out, kva_stream_t stream);
/* kva_append_qknorm_rope followed by kva_decode for a step of one new token
 * per sequence, in one launch when the decode runs the whole-sequence form
 * (see kva_set_decode_split) and in two otherwise.  Replaces the decode
 * loop's qknorm_q, qknorm_k (cache write), K/V copy and decode_attn launches
 * (c_dispatch.c:1066-1103).  The same results as the two calls: q is
 * normalised and rotated in place and the cache rows are bit-identical;
 * out is the decode over every row including the new one (the new token's
 * score and V row enter from registers, so its rounding path differs from
 * kva_decode's: both are within the decode's tolerance).  Unlike
 * kva_append_qknorm_rope, k is only read.                                   */
int kva_append_decode(kva_cache *cache, int32_t layer, void *q, const void *k, const void *v,
                      const void *q_norm_w, const void *k_norm_w, const void *cos_tab,
                      const void *sin_tab, int32_t table_rows, void *out, kva_stream_t stream);
/* kva_append_decode with the output gate of kva_decode_gated (the decode
 * loop's sigmoid_mul launch, c_dispatch.c:1105).                           */
int kva_append_decode_gated(kva_cache *cache, int32_t layer, void *q, const void *k, const void *v,
                            const void *q_norm_w, const void *k_norm_w, const void *cos_tab,
                            const void *sin_tab, int32_t table_rows, const void *gate,
                            int64_t gate_stride, void *out, kva_stream_t stream);
/* Causal attention of each sequence's new rows over cache + new rows: new
 * token i (slot s) sees slots [0, s].  Replaces the prefill attention of
 * _prefill_full_attention (engine.py:3043-3139; flash_attn_256_fp16,
 * flash_attn_256.hip:38-137; flash_attn_256_v3_prefill,
 * flash_attn_256_v3.hip:189-404), which could only start from an empty
 * cache.  q, out: [T, num_heads, 256] fp16 in step token order.            */
int kva_prefill(kva_cache *cache, int32_t layer, const void *q, void *out,
                kva_stream_t stream);
/* Tree-verify attention: new token i sees the cache rows [0, len_before)
 * plus the new tokens in its tree_bits set.  Replaces flash_attn_tree_decode
 * (flash_attn_tree.hip:72-175) under the mask of TreeAttentionMask
 * (tree_attention.py:186-208), wired in decode_step_tree
 * (tp_engine.py:3186-3214).  q, out: [T, num_heads, 256] fp16.            */
int kva_tree_verify(kva_cache *cache, int32_t layer, const void *q, void *out,
                    kva_stream_t stream);
/* kva_prefill / kva_tree_verify with the attention output gate fused into
 * the epilogue, as kva_decode_gated: out = fp16(fp16(attn) * sigmoid(gate)),
 * the _launch_sigmoid_mul(d_pf_attn_out, d_pf_q_gate, seq_len*q_dim) that
 * follows the prefill attention at engine.py:3120-3121 (sigmoid_mul.hip:
 * 10-22).  gate: new token t's row of num_heads*256 values at
 * gate + t*gate_stride (num_heads*256 for the engine's d_pf_q_gate buffer,
 * 2*num_heads*256 for the Q_gate half of a fused [Q | Q_gate] row);
 * 8-byte aligned.                                                          */
int kva_prefill_gated(kva_cache *cache, int32_t layer, const void *q, const void *gate,
                      int64_t gate_stride, void *out, kva_stream_t stream);
int kva_tree_verify_gated(kva_cache *cache, int32_t layer, const void *q, const void *gate,
                          int64_t gate_stride, void *out, kva_stream_t stream);
/* kva_append_qknorm_rope followed by kva_prefill in one call: the
 * per-token qknorm_rope launches for Q and K, the K/V copy into the cache
 * and the causal flash attention of _prefill_full_attention
 * (engine.py:3087-3117; qknorm_rope.hip:55-162, flash_attn_256.hip:38-137).
 * Two launches on `stream`: the append (q normalised and rotated in place,
 * as kva_append_decode does; K normalised into its cache slots, k itself
 * only read; V copied) and the attention.  out and the cache rows are
 * bit-identical to kva_append_qknorm_rope + kva_prefill.  Arguments as
 * kva_append_qknorm_rope, out as kva_prefill.  Not while a graph is
 * recorded (as kva_prefill).                                               */
int kva_append_prefill(kva_cache *cache, int32_t layer, void *q, const void *k, const void *v,
                       const void *q_norm_w, const void *k_norm_w, const void *cos_tab,
                       const void *sin_tab, int32_t table_rows, void *out, kva_stream_t stream);
/* kva_append_prefill with the output gate of kva_prefill_gated (the
 * sigmoid_mul at engine.py:3120-3121).                                     */
int kva_append_prefill_gated(kva_cache *cache, int32_t layer, void *q, const void *k,
                             const void *v, const void *q_norm_w, const void *k_norm_w,
                             const void *cos_tab, const void *sin_tab, int32_t table_rows,
                             const void *gate, int64_t gate_stride, void *out,
                             kva_stream_t stream);
/* Keep accepted tree rows and drop the rest, in every layer: for sequence
 * seq_ids[b], rows base_len[b] + keep_rows[j] (j in [keep_off[b],
 * keep_off[b+1]), strictly increasing) move to base_len[b] + (j -
 * keep_off[b]) and the length becomes base_len[b] + count.  Replaces
 * rollback_kv_cache (tp_engine.py:1673-1687), which only moved the length.
 * All index arrays are host arrays.                                        */
int kva_rollback(kva_cache *cache, int32_t n_seqs, const int32_t *seq_ids,
                 const int32_t *base_len, const int32_t *keep_off,
                 const int32_t *keep_rows, kva_stream_t stream);

/* Split-K tuning for kva_decode: tokens per split (multiple of 16); 0 =
 * automatic.  Automatic runs a step whose longest sequence is at most 1024
 * rows in the whole-sequence form (each sequence walked whole by workgroups
 * that split its kv heads' query-head groups among them, no partials, no
 * combine launch; kva_get_decode_split then reports split 0 and the
 * workgroup count) and longer steps stream-K over all CUs.  A nonzero split
 * always runs stream-K.                                                     */
int kva_set_decode_split(kva_cache *cache, int32_t split_tokens);
int kva_get_decode_split(const kva_cache *cache, int32_t *split_tokens,
                         int32_t *n_splits);

/* Decode timeline (no counterpart in the reference, which has no tracer:
 * its timing is perf_counter around a device sync, bench_optimization_
 * baseline.py:54-69).  While enabled, every kva_decode on this cache records
 * per wave, in the kernel itself: its workgroup's entry time, the time the
 * first K/V loads were issued, the end of its page walk (100 MHz ticks of the
 * GPU's constant clock), and the XCD (bits 32-35) with the workgroup's page
 * count (bits 0-31).  kva_timeline_read copies the last decode's records,
 * [n_wg][grid_rows][8 waves][4] words (a synchronising call); the recorded
 * workload is otherwise unchanged.  The stream-K decode runs one wave per kv
 * head: the records of waves a workgroup does not have are zero.  A decode
 * in the whole-sequence form records its workgroups (n_wg of them,
 * grid_rows = 1; several per sequence and kv head), each with its
 * sequence's page count.  Off by default; costs one device buffer while on. */
/* Dominant-kernel timing (no counterpart in the reference, which times
 * perf_counter around a device sync, bench_optimization_baseline.py:54-69).
 * While set, each following hot-path call on this cache records `before` on
 * its stream right before its main kernel and `after` right after it, so
 * kva_event_elapsed_ms(before, after) is that kernel's own duration: the
 * decode kernel of kva_decode / kva_append_decode (without the combine
 * launch or the append), mq_kernel of kva_prefill / kva_tree_verify
 * (without its combine), the GEMM of kva_project_append / kva_out_project
 * (without the finish kernel).  A call that launches its main kernel more
 * than once (chunked projections) records around each, so the events hold
 * the last.  Both NULL: off.  Refused while a graph is being recorded.     */
int kva_kernel_events(kva_cache *cache, kva_event_t before, kva_event_t after);

int kva_timeline_enable(kva_cache *cache, int32_t on);
int kva_timeline_read(const kva_cache *cache, uint64_t *dst, size_t cap_words,
                      int32_t *n_wg, int32_t *grid_rows);

/* ---- recorded steps (hipGraph replay) ------------------------------------ */
/* Replaces the per-step kernel-node patching of the reference's graph
 * dispatch (c_graph_dispatch.c:392-414 update_mutable_params, which rewrote
 * cos/sin pointers, the K slot pointer and seq_len in every node) and the
 * C dispatch loop's patched arguments (c_dispatch.c:426-456).  Here every
 * per-step value already lives in the device step plan that kva_step_begin
 * uploads, so a recorded step needs no patching: record one step's
 * kva_append_qknorm_rope and kva_decode calls (any layers, in order) between
 * capture_begin and capture_end on one created stream, then for each later
 * step call kva_step_begin and kva_graph_launch.  A replay is valid while
 * the step has the recorded shape (same number of sequences, one new token
 * each) and its RoPE positions stay within the tables the recording used;
 * lengths may grow past page boundaries (the decode launch derives its
 * stream-K shape from the plan on the device).  While recording, calls that
 * cannot be recorded (kva_step_begin, kva_sync_tables, kva_prefill,
 * kva_tree_verify, kva_rollback, kva_destroy, calls on another stream) return
 * KVA_ERR_STATE; a failed call makes capture_end discard the recording.
 * Destroy a graph before its cache.                                        */
int kva_graph_capture_begin(kva_cache *cache, kva_stream_t stream);
int kva_graph_capture_end(kva_cache *cache, kva_stream_t stream, kva_graph **out);
int kva_graph_launch(kva_graph *graph, kva_stream_t stream);
int kva_graph_destroy(kva_graph *graph);

/* ---- reference-kernel-compatible entry points (contiguous caches) ------- */
/* qknorm_rope_fused / qknorm_rope_cachew_fused on a contiguous
 * [num_heads, head_dim] buffer, in place; cache_dst (nullable) also gets the
 * result (qknorm_rope.hip:55-162, qknorm_rope_cachew.hip:52-142).
 * cos_row/sin_row point at the position's table row (the reference passes
 * d_cos + position*half_rotary*2, engine.py:2387).  head_dim in {64, 128,
 * 256}; half_rotary a multiple of 4 with 2*half_rotary <= head_dim.       */
int kva_legacy_qknorm_rope(void *x, const void *w, const void *cos_row,
                           const void *sin_row, void *cache_dst, int32_t num_heads,
                           int32_t head_dim, int32_t half_rotary, float eps,
                           kva_stream_t stream);
/* flash_attn_256_decode semantics (flash_attn_256_tuned.hip:198-350) on a
 * contiguous cache K/V [kv_seq_len, num_kv_heads, 256]: one query row
 * q [num_heads, 256] -> out [num_heads, 256].  `ws` (nullable) lends its
 * split-K workspace and split setting.  With NULL the call runs the
 * whole-sequence form, which needs no workspace, and so takes caches of at
 * most 1024 rows: a longer one returns KVA_ERR_STATE (give it a workspace,
 * or call kva_legacy_decode_noalloc) instead of streaming on a few CUs.    */
int kva_legacy_decode(kva_cache *ws, const void *q, const void *k_base,
                      const void *v_base, void *out, int32_t kv_seq_len,
                      int32_t num_heads, int32_t num_kv_heads, kva_stream_t stream);
/* kva_legacy_decode without a workspace cache and without allocating: no
 * counterpart in the reference.  It is for callers that cannot allocate
 * device memory (code under graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Same arguments and results as kva_legacy_decode;
 * the split-K partials live in a static 16 MiB device array of the library
 * (one per GPU, held until the process ends), so num_heads is at most 128
 * (KVA_ERR_CAPACITY beyond).  Every call on a GPU shares that GPU's array:
 * calls that overlap on one GPU (other streams, other threads) race and must
 * be ordered by the caller.  Nothing in the array needs to start at zero.  */
int kva_legacy_decode_noalloc(const void *q, const void *k_base, const void *v_base,
                              void *out, int32_t kv_seq_len, int32_t num_heads,
                              int32_t num_kv_heads, kva_stream_t stream);
/* kva_legacy_decode followed by the output gate (as kva_decode_gated) in
 * one call: the engine's decode + _launch_sigmoid_mul pair
 * (engine.py:2047-2056).  gate: [num_heads, 256] fp16, 8-byte aligned.     */
int kva_legacy_decode_gated(kva_cache *ws, const void *q, const void *gate,
                            const void *k_base, const void *v_base, void *out,
                            int32_t kv_seq_len, int32_t num_heads, int32_t num_kv_heads,
                            kva_stream_t stream);
/* The intended semantics of _launch_decode_attn_256_batched
 * (engine.py:2806-2857; its kernel ignores the batch index, survey fact F9):
 * sequence b's contiguous cache starts at k_base/v_base + b*batch_stride
 * bytes; q, out: [batch, num_heads, 256]; all sequences have kv_seq_len
 * rows (the reference's shared current_len).                              */
int kva_legacy_decode_batched(kva_cache *ws, const void *q, const void *k_base,
                              const void *v_base, void *out, int32_t kv_seq_len,
                              int32_t batch, int64_t batch_stride,
                              int32_t num_heads, int32_t num_kv_heads,
                              kva_stream_t stream);

/* HBM stream-copy probe: one kernel copying `bytes` (a multiple of 16,
 * 16-byte aligned pointers) with 16-byte lanes.  The measured-bandwidth
 * counterpart of the reference's bench/micro/hbm_bandwidth.hip.cpp, and the
 * known-size kernel that calibrates FETCH_SIZE / WRITE_SIZE counters.      */
int kva_hbm_copy(void *dst, const void *src, size_t bytes, kva_stream_t stream);

/* HBM read-only stream probe: one kernel reading `bytes` (a multiple of 16,
 * src 16-byte aligned) with 16-byte lanes, eight loads in flight per lane;
 * `sink` (one 4-byte word) is written only when the data's XOR fold hits a
 * fixed value, so the reads cannot be dropped.  The read-side ceiling the
 * decode attention is measured against; like kva_hbm_copy, the measured
 * counterpart of the reference's bench/micro/hbm_bandwidth.hip.cpp.        */
int kva_hbm_read(const void *src, size_t bytes, void *sink, kva_stream_t stream);

/* Paged HBM read probe: the stream-K decode's own load pattern with no
 * arithmetic.  n_wg workgroups of num_kv_heads waves share the page list
 * page_ids[0 .. n_pages) (a DEVICE int32 array) in equal contiguous ranges;
 * wave h reads kv head h's 512-byte slice of every row of each page of K and
 * of V (pools [page][16][num_kv_heads][256] fp16), as decode_mfma_kernel
 * does, one page in flight while the previous is folded by XOR; `sink` (one
 * 4-byte word) is written only when the fold hits a fixed value.  The read
 * ceiling of the decode's access pattern, next to kva_hbm_read's contiguous
 * stream (bench/micro/hbm_bandwidth.hip.cpp is the reference's probe).     */
int kva_hbm_read_pages(const void *k_pool, const void *v_pool, const int32_t *page_ids, int32_t n_pages,
                       int32_t num_kv_heads, int32_t n_wg, void *sink, kva_stream_t stream);

/* ---- device helpers (the GPUDevice surface, hip_dispatch.py:594-703) ----- */
int kva_dev_count(int32_t *n);
/* The current device's compute units, peak shader clock (kHz), memory clock
 * (kHz) and memory bus width (bits), from hipGetDeviceProperties: what a
 * bench derives its peaks from next to the vendor figures.  No reference
 * counterpart (its benchmarks quote fixed MI50 peaks).                     */
int kva_dev_props(int32_t *n_cu, int32_t *clock_khz, int32_t *mem_clock_khz,
                  int32_t *mem_bus_bits);
int kva_dev_set(int32_t device);
int kva_dev_malloc(void **ptr, size_t bytes);
int kva_dev_free(void *ptr);
int kva_memcpy_h2d(void *dst, const void *src, size_t bytes);
int kva_memcpy_d2h(void *dst, const void *src, size_t bytes);
int kva_memcpy_d2d(void *dst, const void *src, size_t bytes);
int kva_memset(void *dst, int32_t value, size_t bytes);
int kva_dev_synchronize(void);
int kva_stream_create(kva_stream_t *stream);
int kva_stream_destroy(kva_stream_t stream);
int kva_stream_synchronize(kva_stream_t stream);
int kva_event_create(kva_event_t *ev);
int kva_event_destroy(kva_event_t ev);
int kva_event_record(kva_event_t ev, kva_stream_t stream);
int kva_event_synchronize(kva_event_t ev);
int kva_event_elapsed_ms(float *ms, kva_event_t start, kva_event_t stop);

#ifdef __cplusplus
}
#endif

#endif /* KVATTN_H */
