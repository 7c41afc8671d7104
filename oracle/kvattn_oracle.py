"""numpy restatement of mi50grad's full-attention KV-cache path (CPU oracle).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py``; never by ``mi50grad_amd``.

Every function cites the reference code it restates (paths relative to the
mi50grad repository).  Two kinds of functions live here:

* *Textbook* restatements (attention, masks, RoPE tables): what the reference
  computes, in float32, checked against closed forms, library routines and the
  reference's own known answers in ``tests/test_oracle.py``.
* The *bit-exact contract* ``qknorm_rope_exact``: the reference kernel's math
  (per-head RMSNorm then interleaved partial RoPE) with the operation order the
  HIP kernel commits to, mirrored op by op in IEEE float32 so the GPU result
  can be compared bit for bit.  Its tolerance-level agreement with the
  reference's float formula is checked separately.
"""
from __future__ import annotations

import numpy as np

# Model constants: qwen.py:32-38 (24/4 heads, head_dim 256, theta 1e7,
# eps 1e-6) and qwen.py:52 (partial_rotary_factor 0.25 -> 64 rotary dims).
NUM_HEADS = 24
NUM_KV_HEADS = 4
HEAD_DIM = 256
ROTARY_DIM = 64
HALF_ROTARY = 32
ROPE_THETA = 10000000.0
RMS_EPS = 1e-6
BLOCK_TOKENS = 16
# One token's K row [4,256] + V row [4,256] in fp16.
KV_ROW_BYTES = 2 * NUM_KV_HEADS * HEAD_DIM * 2


# ---------------------------------------------------------------------------
# a1: RoPE tables
# ---------------------------------------------------------------------------
def rope_tables(max_seq: int, head_dim: int = HEAD_DIM,
                partial_rotary_factor: float = 0.25,
                theta: float = ROPE_THETA):
    """cos/sin tables [max_seq, rotary_dim/2] fp16.

    Restates ``InferenceEngine._init_rope_tables`` (engine.py:1025-1046):
    float32 inverse frequencies, float32 outer product with the positions,
    float32 cos/sin, then a cast to fp16.
    """
    rotary_dim = int(head_dim * partial_rotary_factor)
    half = rotary_dim // 2
    freqs = 1.0 / (theta ** (np.arange(0, half, dtype=np.float32) * 2.0 / rotary_dim))
    positions = np.arange(max_seq, dtype=np.float32)
    angles = np.outer(positions, freqs)
    return np.cos(angles).astype(np.float16), np.sin(angles).astype(np.float16)


# ---------------------------------------------------------------------------
# producer: the FP16 attention projections
# ---------------------------------------------------------------------------
def project_fp16(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """out[t, n] = fp16(sum_k w[n, k] x[t, k]): the FP16 GEMV of
    gemv_fp16_v2.hip:22-85 (fp16 operands, fp32 accumulation, one fp16
    rounding of the sum) for every row t of x.

    The sum is taken in float64, in which every fp16 product is exact, so
    the result is the correctly rounded fp16 of a sum whose own error is far
    below the fp32 accumulation error of any GPU summation order: a GPU
    result may differ from this by at most one fp16 ulp, and by none when
    every partial sum is exactly representable in fp32.
    """
    acc = np.asarray(x, np.float64) @ np.asarray(w, np.float64).T
    return acc.astype(np.float16)


def out_project(attn: np.ndarray, w_o: np.ndarray, residual: np.ndarray | None = None) -> np.ndarray:
    """out[t, n] = fp16(sum_k w_o[n, k] attn[t, k] + residual[t, n]): the
    O-projection GEMV with its residual epilogue (gemv_fp16_v2.hip:81-84,
    called at engine.py:2083-2085 with residual = d_hidden), one fp16
    rounding after the add.  Summed in float64 as in project_fp16; without
    a residual it is project_fp16."""
    acc = np.asarray(attn, np.float64) @ np.asarray(w_o, np.float64).T
    if residual is not None:
        acc = acc + np.asarray(residual, np.float64)
    return acc.astype(np.float16)


def project_append(x, w_q_fused, w_kv_fused, q_w, k_w, cos_rows, sin_rows,
                   num_heads: int = NUM_HEADS, num_kv_heads: int = NUM_KV_HEADS):
    """The reference's producer for one step, token by token: the Q+Q_gate
    and K+V GEMVs (engine.py:2000-2022 over the stacked weights of
    engine.py:1366-1378), then QK-norm + RoPE of Q and K
    (engine.py:2371-2432).  Returns (q [T,H,256] normed + rotated,
    q_gate [T,H,256], k_raw [T,Hkv,256], k [T,Hkv,256] normed + rotated,
    v [T,Hkv,256])."""
    T = x.shape[0]
    qd, kd = num_heads * HEAD_DIM, num_kv_heads * HEAD_DIM
    qf = project_fp16(x, w_q_fused)
    kvf = project_fp16(x, w_kv_fused)
    q_raw = qf[:, :qd].reshape(T, num_heads, HEAD_DIM)
    gate = qf[:, qd:].reshape(T, num_heads, HEAD_DIM)
    k_raw = kvf[:, :kd].reshape(T, num_kv_heads, HEAD_DIM)
    v = kvf[:, kd:].reshape(T, num_kv_heads, HEAD_DIM)
    cq = np.repeat(cos_rows, num_heads, axis=0)
    sq = np.repeat(sin_rows, num_heads, axis=0)
    q = qknorm_rope_exact(q_raw.reshape(-1, HEAD_DIM), q_w, cq, sq).reshape(T, num_heads, HEAD_DIM)
    ck = np.repeat(cos_rows, num_kv_heads, axis=0)
    sk = np.repeat(sin_rows, num_kv_heads, axis=0)
    k = qknorm_rope_exact(k_raw.reshape(-1, HEAD_DIM), k_w, ck, sk).reshape(T, num_kv_heads, HEAD_DIM)
    return q, gate, k_raw, k, v


# ---------------------------------------------------------------------------
# a2/a3: fused per-head RMSNorm + interleaved partial RoPE
# ---------------------------------------------------------------------------
def qknorm_rope_exact(x: np.ndarray, w: np.ndarray, cos_rows: np.ndarray,
                      sin_rows: np.ndarray, eps: float = RMS_EPS) -> np.ndarray:
    """Bit-exact mirror of the build's norm+RoPE kernel.

    Math follows qknorm_rope.hip:55-162 (per-head RMSNorm with the stored
    weight, then rotation of interleaved pairs (2i, 2i+1) for i < half_rotary,
    tail dims normalised only; F4/F5 of the survey).  Operation order, which
    the HIP kernel reproduces exactly (no FMA contraction):

    1. lanes: head_dim/8 lanes hold 8 consecutive dims each; a lane sums
       x_i*x_i sequentially over its 8 dims;
    2. butterfly over lanes with offsets n/2, ..., 1: s = s + s[lane ^ off];
    3. ms = s * (1/head_dim)  (exact: power of two);  v = ms + eps;
    4. inv = 1 / sqrt(v)  (both correctly rounded);
    5. n_i = (x_i * inv) * w_i;
    6. pair p: y0 = n0*c - n1*s ; y1 = n0*s + n1*c  (each product rounded);
    7. fp16 round-to-nearest-even.

    x: [n, head_dim] fp16.  w: [head_dim] fp16.  cos_rows/sin_rows:
    [n, half_rotary] fp16 (the table row of each vector's position).
    """
    x = np.asarray(x, dtype=np.float16)
    n, d = x.shape
    assert d % 8 == 0 and (d // 8) & (d // 8 - 1) == 0, "head_dim/8 must be a power of two"
    cos_rows = np.asarray(cos_rows, dtype=np.float16)
    sin_rows = np.asarray(sin_rows, dtype=np.float16)
    half = cos_rows.size // n if n else 0
    cos_rows = cos_rows.reshape(n, half)
    sin_rows = sin_rows.reshape(n, half)
    assert 2 * half <= d
    xf = x.astype(np.float32)
    sq = (xf * xf).reshape(n, d // 8, 8)
    s = sq[:, :, 0].copy()
    for i in range(1, 8):
        s = s + sq[:, :, i]
    lanes = d // 8
    idx = np.arange(lanes)
    off = lanes // 2
    while off >= 1:
        s = s + s[:, idx ^ off]
        off //= 2
    total = s[:, 0]
    ms = total * np.float32(1.0 / d)
    v = ms + np.float32(eps)
    inv = np.float32(1.0) / np.sqrt(v)
    nrm = (xf * inv[:, None]) * np.asarray(w, dtype=np.float16).astype(np.float32)[None, :]
    c = cos_rows.astype(np.float32)
    sn = sin_rows.astype(np.float32)
    a = nrm[:, 0:2 * half:2]
    b = nrm[:, 1:2 * half:2]
    y0 = a * c - b * sn
    y1 = a * sn + b * c
    out = nrm.copy()
    out[:, 0:2 * half:2] = y0
    out[:, 1:2 * half:2] = y1
    return out.astype(np.float16)


def qknorm_rope_float(x, w, cos_row, sin_row, eps: float = RMS_EPS) -> np.ndarray:
    """The reference test's float formula (tests/test_qknorm_rope.py:55-90).

    rms = sqrt(mean(x^2) + eps); x / rms * w; interleaved rotation of the
    first 2*half dims.  Used for the tolerance-level check of the exact
    mirror (the reference test's bar is 2e-3).
    """
    xf = np.asarray(x, dtype=np.float32)
    wf = np.asarray(w, dtype=np.float16).astype(np.float32)
    c = np.asarray(cos_row, dtype=np.float16).astype(np.float32).reshape(xf.shape[0], -1)
    s = np.asarray(sin_row, dtype=np.float16).astype(np.float32).reshape(xf.shape[0], -1)
    out = np.empty_like(xf)
    for h in range(xf.shape[0]):
        vec = xf[h]
        rms = np.sqrt(np.mean(vec ** 2) + eps)
        vec = vec / rms * wf
        half = c.shape[1]
        x0 = vec[0:2 * half:2].copy()
        x1 = vec[1:2 * half:2].copy()
        vec[0:2 * half:2] = x0 * c[h] - x1 * s[h]
        vec[1:2 * half:2] = x0 * s[h] + x1 * c[h]
        out[h] = vec
    return out.astype(np.float16)


# ---------------------------------------------------------------------------
# a6-a9: attention
# ---------------------------------------------------------------------------
def kv_head_of(h: int, num_heads: int, num_kv_heads: int) -> int:
    """GQA map used by every reference kernel: flash_attn_256_tuned.hip:222."""
    return (h * num_kv_heads) // num_heads


def attention_fp32(q: np.ndarray, k: np.ndarray, v: np.ndarray,
                   visible: np.ndarray | None = None) -> np.ndarray:
    """softmax(q k^T / sqrt(d)) v in float32 with the GQA head map.

    Textbook restatement of the reference's numpy oracles
    (tests/test_flash_attn_v3.py:35-63, tests/test_attention.py:48-67).
    q: [M, H, D]; k, v: [N, Hkv, D]; visible: [M, N] bool (None = all).
    Returns [M, H, D] float32.  A row with no visible key returns zeros.
    """
    q = np.asarray(q)
    m, num_heads, d = q.shape
    n, num_kv, _ = k.shape
    scale = np.float32(1.0 / np.sqrt(d))
    out = np.zeros((m, num_heads, d), dtype=np.float32)
    kf = np.asarray(k, dtype=np.float32)
    vf = np.asarray(v, dtype=np.float32)
    for h in range(num_heads):
        kh = kv_head_of(h, num_heads, num_kv)
        qh = q[:, h, :].astype(np.float32) * scale
        scores = qh @ kf[:, kh, :].T
        if visible is not None:
            scores = np.where(visible, scores, -np.inf)
        mx = np.max(scores, axis=-1, keepdims=True)
        mx = np.where(np.isfinite(mx), mx, 0.0).astype(np.float32)
        e = np.exp(scores - mx)
        den = e.sum(axis=-1, keepdims=True)
        den = np.where(den > 0, den, 1.0)
        out[:, h, :] = (e / den) @ vf[:, kh, :]
    return out


def decode_attention(q: np.ndarray, ks, vs) -> np.ndarray:
    """Batched single-token decode over ragged caches.

    Per sequence b, ``attention_fp32(q[b:b+1], ks[b], vs[b])``: what
    flash_attn_256_decode (flash_attn_256_tuned.hip:198-350) computes for one
    sequence, applied to each sequence of the batch.  q: [B, H, D];
    ks[b], vs[b]: [L_b, Hkv, D].  Returns [B, H, D] float32.
    """
    return np.stack([attention_fp32(q[b:b + 1], ks[b], vs[b])[0] for b in range(len(ks))])


def sigmoid_gate(out: np.ndarray, gate: np.ndarray) -> np.ndarray:
    """The attention output gate, sigmoid_mul.hip:10-22 as used after decode
    at engine.py:2055-2056: each fp16 output element times sigmoid of the
    matching fp16 gate element (the gate half of the fused [Q | Q_gate]
    projection, engine.py:1069-1071), in float32, rounded to fp16:
    ``fp16(float(out) * (1 / (1 + exp(-float(gate)))))``."""
    o = np.asarray(out, np.float16).astype(np.float32)
    g = np.asarray(gate, np.float16).astype(np.float32)
    sig = np.float32(1.0) / (np.float32(1.0) + np.exp(-g, dtype=np.float32))
    return (o * sig).astype(np.float16)


def chunk_visibility(prefix_len: int, chunk_len: int) -> np.ndarray:
    """Causal rule for a chunk appended after ``prefix_len`` cached rows.

    Chunk row i sits at slot prefix_len+i and sees keys [0, prefix_len+i].
    With prefix_len=0 this is the reference's causal rule
    (flash_attn_256.hip:78, flash_attn_256_v3.hip:252-255 and 336-339).
    """
    n = prefix_len + chunk_len
    rows = prefix_len + np.arange(chunk_len)[:, None]
    return np.arange(n)[None, :] <= rows


def chunk_attention(q_chunk, k_all, v_all, prefix_len: int) -> np.ndarray:
    """Causal attention of a chunk over cache+chunk: [n, H, D] float32."""
    vis = chunk_visibility(prefix_len, q_chunk.shape[0])
    return attention_fp32(q_chunk, k_all, v_all, vis)


# ---------------------------------------------------------------------------
# a10/a11: tree masks, tree verify, rollback
# ---------------------------------------------------------------------------
def tree_depths(parents) -> np.ndarray:
    """Depth of each node; parents[i] < i (BFS order), root has parent -1."""
    parents = list(parents)
    depth = np.zeros(len(parents), dtype=np.int64)
    for i, p in enumerate(parents):
        if i == 0:
            assert p == -1, "node 0 must be the root"
        else:
            assert 0 <= p < i, "parents must precede children (BFS order)"
            depth[i] = depth[p] + 1
    return depth


def tree_ancestors(parents, i: int):
    """Ancestors of node i from the root down (TreeNode.get_ancestors,
    tree_attention.py:40-49)."""
    out = []
    p = parents[i]
    while p != -1:
        out.append(p)
        p = parents[p]
    return out[::-1]


def tree_mask_reference(parents, kv_len: int) -> np.ndarray:
    """``TreeAttentionMask._build_mask`` (tree_attention.py:186-208).

    [T, T+kv_len] bool; columns are tree nodes first, then the KV cache.
    """
    t = len(parents)
    mask = np.zeros((t, t + kv_len), dtype=bool)
    for i in range(t):
        mask[i, i] = True
        for a in tree_ancestors(parents, i):
            mask[i, a] = True
        if kv_len > 0:
            mask[i, t:t + kv_len] = True
    return mask


def tree_visibility_cache_order(parents, kv_len: int) -> np.ndarray:
    """Same mask with the cache-slot column order the build uses.

    The tree rows are appended at slots kv_len..kv_len+T-1, so columns are the
    cache [0, kv_len) first, then the tree nodes.
    """
    ref = tree_mask_reference(parents, kv_len)
    t = len(parents)
    return np.concatenate([ref[:, t:], ref[:, :t]], axis=1)


def tree_row_bits(parents) -> np.ndarray:
    """Per node, a uint64 bit set of the tree nodes it sees (self+ancestors)."""
    t = len(parents)
    assert t <= 64
    bits = np.zeros(t, dtype=np.uint64)
    for i in range(t):
        b = 1 << i
        for a in tree_ancestors(parents, i):
            b |= 1 << a
        bits[i] = np.uint64(b)
    return bits


def tree_attention(q_tree, k_cache, v_cache, k_tree, v_tree, parents) -> np.ndarray:
    """Tree verify: node i attends the cache plus its ancestors and itself.

    The semantics ``flash_attn_tree_decode`` implements with a bit mask
    (flash_attn_tree.hip:72-175) under the mask of tree_attention.py:186-208.
    q_tree: [T, H, D]; cache [L, Hkv, D]; tree K/V [T, Hkv, D].
    """
    kv_len = k_cache.shape[0]
    k_all = np.concatenate([k_cache, k_tree], axis=0)
    v_all = np.concatenate([v_cache, v_tree], axis=0)
    vis = tree_visibility_cache_order(parents, kv_len)
    return attention_fp32(q_tree, k_all, v_all, vis)


def rollback_rows(rows: np.ndarray, base_len: int, keep) -> tuple[np.ndarray, int]:
    """Compact accepted tree rows and roll back the rest.

    The reference only moves ``current_len`` back (tp_engine.py:1673-1687,
    survey fact F7); the intended semantics restated here: rows at
    base_len+keep[k] move to base_len+k in order, the new length is
    base_len+len(keep), rows below base_len are untouched.  ``rows`` is one
    sequence's logical cache [n, ...]; returns (new rows array, new length).
    """
    keep = list(keep)
    assert all(keep[i] < keep[i + 1] for i in range(len(keep) - 1))
    out = rows.copy()
    for k, src in enumerate(keep):
        out[base_len + k] = rows[base_len + src]
    return out, base_len + len(keep)


# ---------------------------------------------------------------------------
# a5: paged cache model
# ---------------------------------------------------------------------------
class PagedCacheModel:
    """Host model of the paged cache: pools [layer][block][16][Hkv][D] fp16.

    Logical slot s of a sequence lives in block table[s // 16], row s % 16.
    That is the reference's contiguous row layout (engine.py:79-117:
    [max_seq][Hkv][256] per batch slot) cut into 16-token pages.
    """

    def __init__(self, n_layers: int, n_blocks: int, num_kv_heads: int = NUM_KV_HEADS,
                 head_dim: int = HEAD_DIM, block_tokens: int = BLOCK_TOKENS):
        shape = (n_layers, n_blocks, block_tokens, num_kv_heads, head_dim)
        self.k = np.zeros(shape, dtype=np.float16)
        self.v = np.zeros(shape, dtype=np.float16)
        self.bt = block_tokens
        self.tables: dict[int, list[int]] = {}
        self.lens: dict[int, int] = {}

    def set_table(self, seq: int, blocks, length: int = 0):
        self.tables[seq] = list(blocks)
        self.lens[seq] = length

    def _where(self, seq: int, slot: int):
        return self.tables[seq][slot // self.bt], slot % self.bt

    def write(self, layer: int, seq: int, slot: int, k_row, v_row):
        blk, r = self._where(seq, slot)
        self.k[layer, blk, r] = k_row
        self.v[layer, blk, r] = v_row

    def gather(self, layer: int, seq: int, n: int):
        ks = np.empty((n,) + self.k.shape[3:], dtype=np.float16)
        vs = np.empty_like(ks)
        for s in range(n):
            blk, r = self._where(seq, s)
            ks[s] = self.k[layer, blk, r]
            vs[s] = self.v[layer, blk, r]
        return ks, vs


def merge_partials(ms, ls, accs):
    """Merge split-K online-softmax partials (m, l, acc) into one output.

    The 4-wave merge of flash_attn_256_tuned.hip:285-349, generalised to any
    number of partials: M = max m_s, L = sum l_s e^(m_s-M),
    out = sum acc_s e^(m_s-M) / L.  ms, ls: [S]; accs: [S, D].
    """
    ms = np.asarray(ms, dtype=np.float64)
    big = np.max(ms)
    c = np.exp(ms - big)
    den = np.sum(np.asarray(ls, dtype=np.float64) * c)
    return (np.asarray(accs, dtype=np.float64) * c[:, None]).sum(0) / den


def partial_softmax(q_row, k, v):
    """One split's partial state for a single query row (m, l, acc)."""
    s = (k.astype(np.float64) @ q_row.astype(np.float64)) / np.sqrt(q_row.shape[-1])
    m = np.max(s)
    e = np.exp(s - m)
    return m, e.sum(), e @ v.astype(np.float64)
