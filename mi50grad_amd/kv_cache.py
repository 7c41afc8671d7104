"""Paged FP16 KV cache (libkvattn) and the reference-compatible ``KVCache``.

``PagedKVCache`` is the full interface: ragged per-sequence lengths, a block
table per sequence, per-step plans shared by all layers, and the hot-path
calls (append, decode, prefill, tree verify, rollback).

``KVCache`` keeps the constructor, attributes and methods of the reference's
``KVCache`` (engine.py:79-291) so ``engine.py``-style callers can swap it in:
it gives every batch slot a run of consecutive pages, which makes each slot's
rows contiguous ``[max_seq][kv_heads][256]`` exactly as in the reference, and
the raw pointers it returns address real rows.
"""
from __future__ import annotations

import ctypes
from typing import Sequence

import numpy as np

from . import _lib
from .device import GPUDevice

BLOCK_TOKENS = 16
HEAD_DIM = 256


def _ptr(x) -> int:
    """Device address of an int pointer or a DeviceArray (None stays NULL)."""
    if x is None:
        return None
    return x if isinstance(x, int) else x.ptr


class PagedKVCache:
    """Owns a ``kva_cache``: K/V pools for ``n_layers`` layers plus metadata."""

    def __init__(self, n_layers: int, max_seqs: int, max_blocks: int, max_blocks_per_seq: int,
                 max_step_tokens: int = 4096, num_heads: int = 24, num_kv_heads: int = 4,
                 head_dim: int = HEAD_DIM, rotary_dim: int = 64, eps: float = 1e-6,
                 host_only: bool = False):
        cfg = _lib.KvaConfig(n_layers, num_heads, num_kv_heads, head_dim, rotary_dim, BLOCK_TOKENS,
                             max_seqs, max_blocks, max_blocks_per_seq, max_step_tokens, eps,
                             _lib.KVA_FLAG_HOST_ONLY if host_only else 0)
        self.cfg = cfg
        h = ctypes.c_void_p()
        _lib.call("kva_create", ctypes.byref(cfg), ctypes.byref(h))
        self.handle = h.value
        self.n_layers = n_layers
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.host_only = host_only
        lay = _lib.KvaLayout()
        _lib.call("kva_get_layout", self.handle, ctypes.byref(lay))
        self.row_bytes = lay.row_bytes
        self.block_bytes = lay.block_bytes
        self.layer_bytes = lay.layer_bytes

    # lifetime -------------------------------------------------------------
    def destroy(self) -> None:
        if self.handle:
            _lib.call("kva_destroy", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass

    # host block management ------------------------------------------------
    def reserve(self, seq: int, n_tokens: int) -> None:
        _lib.call("kva_seq_reserve", self.handle, seq, n_tokens)

    def set_blocks(self, seq: int, block_ids: Sequence[int]) -> None:
        ids = _lib.int_array(block_ids)
        _lib.call("kva_seq_set_blocks", self.handle, seq, ids, len(block_ids))

    def free_seq(self, seq: int) -> None:
        _lib.call("kva_seq_free", self.handle, seq)

    def seq_len(self, seq: int) -> int:
        n = ctypes.c_int32()
        _lib.call("kva_seq_get_len", self.handle, seq, ctypes.byref(n))
        return n.value

    def set_len(self, seq: int, length: int) -> None:
        _lib.call("kva_seq_set_len", self.handle, seq, length)

    def blocks(self, seq: int) -> list[int]:
        n = ctypes.c_int32()
        _lib.call("kva_seq_get_blocks", self.handle, seq, None, 0, ctypes.byref(n))
        buf = (ctypes.c_int32 * max(1, n.value))()
        _lib.call("kva_seq_get_blocks", self.handle, seq, buf, n.value, ctypes.byref(n))
        return list(buf[:n.value])

    def free_block_count(self) -> int:
        n = ctypes.c_int32()
        _lib.call("kva_free_block_count", self.handle, ctypes.byref(n))
        return n.value

    def sync_tables(self, stream=None) -> None:
        _lib.call("kva_sync_tables", self.handle, stream)

    # device addressing ----------------------------------------------------
    def layer_pools(self, layer: int) -> tuple[int, int]:
        k = ctypes.c_void_p()
        v = ctypes.c_void_p()
        _lib.call("kva_layer_pools", self.handle, layer, ctypes.byref(k), ctypes.byref(v))
        return k.value, v.value

    def row_ptr(self, layer: int, seq: int, slot: int) -> tuple[int, int]:
        k = ctypes.c_void_p()
        v = ctypes.c_void_p()
        _lib.call("kva_row_ptr", self.handle, layer, seq, slot, ctypes.byref(k), ctypes.byref(v))
        return k.value, v.value

    def download_pools(self, layer: int) -> tuple[np.ndarray, np.ndarray]:
        """Whole K and V pools of one layer as [blocks][16][Hkv][256] fp16."""
        kp, vp = self.layer_pools(layer)
        shape = (self.cfg.max_blocks, BLOCK_TOKENS, self.num_kv_heads, self.head_dim)
        out = []
        for p in (kp, vp):
            a = np.empty(shape, dtype=np.float16)
            _lib.call("kva_memcpy_d2h", a.ctypes.data, p, a.nbytes)
            out.append(a)
        return out[0], out[1]

    def gather(self, layer: int, seq: int, n: int) -> tuple[np.ndarray, np.ndarray]:
        """Logical rows [0, n) of one sequence (test helper; downloads the pool)."""
        kpool, vpool = self.download_pools(layer)
        ids = self.blocks(seq)
        rows = np.arange(n)
        blk = np.asarray(ids, dtype=np.int64)[rows // BLOCK_TOKENS]
        return kpool[blk, rows % BLOCK_TOKENS], vpool[blk, rows % BLOCK_TOKENS]

    # per-step plan and hot path ---------------------------------------------
    def begin_step(self, seq_ids: Sequence[int], n_new: Sequence[int], rope_pos=None,
                   tree_bits=None, stream=None) -> None:
        ids = _lib.int_array(seq_ids)
        nn = _lib.int_array(n_new)
        rp = _lib.int_array(rope_pos) if rope_pos is not None else None
        tb = _lib.u64_array(tree_bits) if tree_bits is not None else None
        _lib.call("kva_step_begin", self.handle, len(seq_ids), ids, nn, rp, tb, stream)

    def append(self, layer: int, q, k, v, q_norm_w, k_norm_w, cos_tab, sin_tab, table_rows: int,
               stream=None) -> None:
        _lib.call("kva_append_qknorm_rope", self.handle, layer, _ptr(q), _ptr(k), _ptr(v),
                  _ptr(q_norm_w), _ptr(k_norm_w), _ptr(cos_tab), _ptr(sin_tab), table_rows, stream)

    def append_decode(self, layer: int, q, k, v, q_norm_w, k_norm_w, cos_tab, sin_tab, table_rows: int, out,
                      stream=None, gate=None, gate_stride: int = 0) -> None:
        """append() then decode() for a step of one token per sequence, in
        one launch where the decode runs its whole-sequence form
        (kva_append_decode); k is only read."""
        if gate is None:
            _lib.call("kva_append_decode", self.handle, layer, _ptr(q), _ptr(k), _ptr(v), _ptr(q_norm_w),
                      _ptr(k_norm_w), _ptr(cos_tab), _ptr(sin_tab), table_rows, _ptr(out), stream)
        else:
            stride = gate_stride or self.num_heads * 256
            _lib.call("kva_append_decode_gated", self.handle, layer, _ptr(q), _ptr(k), _ptr(v), _ptr(q_norm_w),
                      _ptr(k_norm_w), _ptr(cos_tab), _ptr(sin_tab), table_rows, _ptr(gate), stride, _ptr(out),
                      stream)

    def append_prefill(self, layer: int, q, k, v, q_norm_w, k_norm_w, cos_tab, sin_tab, table_rows: int, out,
                       stream=None, gate=None, gate_stride: int = 0) -> None:
        """append() then prefill() in one call (kva_append_prefill): q is
        normalised in place, k only read; out and the cache rows are
        bit-identical to the two calls."""
        if gate is None:
            _lib.call("kva_append_prefill", self.handle, layer, _ptr(q), _ptr(k), _ptr(v), _ptr(q_norm_w),
                      _ptr(k_norm_w), _ptr(cos_tab), _ptr(sin_tab), table_rows, _ptr(out), stream)
        else:
            stride = gate_stride or self.num_heads * 256
            _lib.call("kva_append_prefill_gated", self.handle, layer, _ptr(q), _ptr(k), _ptr(v), _ptr(q_norm_w),
                      _ptr(k_norm_w), _ptr(cos_tab), _ptr(sin_tab), table_rows, _ptr(gate), stride, _ptr(out),
                      stream)

    def project_append(self, layer: int, x, hidden: int, w_q_fused, w_kv_fused, q_norm_w, k_norm_w,
                       cos_tab, sin_tab, table_rows: int, q_out, q_gate_out=None, kv_out=None,
                       stream=None) -> None:
        """Q/K/V projection of the step's tokens fused with norm + RoPE +
        append (the reference's FP16 GEMVs, engine.py:2000-2022, followed by
        its norm/RoPE/cache-write launches).  Writes q_out [T, H, 256] and,
        when given, q_gate_out [T, H, 256] and kv_out [T, 2, Hkv, 256]."""
        _lib.call("kva_project_append", self.handle, layer, _ptr(x), hidden, _ptr(w_q_fused),
                  _ptr(w_kv_fused), _ptr(q_norm_w), _ptr(k_norm_w), _ptr(cos_tab), _ptr(sin_tab),
                  table_rows, _ptr(q_out), _ptr(q_gate_out), _ptr(kv_out), stream)

    def project_path(self) -> str:
        """Which path the last project_append took: "kernels" (the split-K
        projection kernels, 64 tokens per launch pair) or "prefill_gemm" (one
        GEMM launch over every token, the epilogue fused)."""
        p = ctypes.c_int32()
        _lib.call("kva_get_project_path", self.handle, ctypes.byref(p))
        return {0: "kernels", 1: "prefill_gemm"}[p.value]

    def out_project(self, attn, n_tok: int, q_dim: int, w_o, n_out: int, out, residual=None,
                    stream=None) -> None:
        """O-projection of n_tok attention rows: out = fp16(attn . w_o^T +
        residual), the reference's _launch_gemv_fp16(d_hidden, d_attn_out,
        o_weight, q_dim, hidden, residual=d_hidden) (engine.py:2083-2085)
        for every row at once.  residual may be None or `out` itself."""
        _lib.call("kva_out_project", self.handle, _ptr(attn), n_tok, q_dim, _ptr(w_o), n_out,
                  _ptr(residual), _ptr(out), stream)

    def decode(self, layer: int, q, out, stream=None, gate=None, gate_stride: int = 0) -> None:
        """Decode attention; with `gate`, the output gate (out *= sigmoid(gate),
        sigmoid_mul.hip) is applied in the same launch."""
        if gate is None:
            _lib.call("kva_decode", self.handle, layer, _ptr(q), _ptr(out), stream)
        else:
            stride = gate_stride or self.num_heads * 256
            _lib.call("kva_decode_gated", self.handle, layer, _ptr(q), _ptr(gate), stride, _ptr(out), stream)

    def prefill(self, layer: int, q, out, stream=None, gate=None, gate_stride: int = 0) -> None:
        """Causal attention of the step's new rows; with `gate`, the output
        gate (out *= sigmoid(gate), engine.py:3120-3121) in the same launch."""
        if gate is None:
            _lib.call("kva_prefill", self.handle, layer, _ptr(q), _ptr(out), stream)
        else:
            stride = gate_stride or self.num_heads * 256
            _lib.call("kva_prefill_gated", self.handle, layer, _ptr(q), _ptr(gate), stride, _ptr(out), stream)

    def tree_verify(self, layer: int, q, out, stream=None, gate=None, gate_stride: int = 0) -> None:
        if gate is None:
            _lib.call("kva_tree_verify", self.handle, layer, _ptr(q), _ptr(out), stream)
        else:
            stride = gate_stride or self.num_heads * 256
            _lib.call("kva_tree_verify_gated", self.handle, layer, _ptr(q), _ptr(gate), stride, _ptr(out),
                      stream)

    def rollback(self, seq_ids: Sequence[int], base_len: Sequence[int],
                 keep_rows: Sequence[Sequence[int]], stream=None) -> None:
        off = [0]
        flat: list[int] = []
        for rows in keep_rows:
            flat.extend(int(r) for r in rows)
            off.append(len(flat))
        _lib.call("kva_rollback", self.handle, len(seq_ids), _lib.int_array(seq_ids),
                  _lib.int_array(base_len), _lib.int_array(off), _lib.int_array(flat), stream)

    def record_step(self, stream) -> "StepGraph":
        """Start recording this step's append/decode calls on `stream` (a
        created Stream's handle); end with StepGraph.end()."""
        _lib.call("kva_graph_capture_begin", self.handle, stream)
        return StepGraph(self, stream)

    def set_decode_split(self, split_tokens: int) -> None:
        _lib.call("kva_set_decode_split", self.handle, split_tokens)

    def decode_split(self) -> tuple[int, int]:
        s = ctypes.c_int32()
        n = ctypes.c_int32()
        _lib.call("kva_get_decode_split", self.handle, ctypes.byref(s), ctypes.byref(n))
        return s.value, n.value

    def kernel_events(self, before=None, after=None) -> None:
        """Record Events `before` / `after` around the main kernel of each
        following hot-path call (kva_kernel_events); None, None: off."""
        _lib.call("kva_kernel_events", self.handle, before.handle if before else None,
                  after.handle if after else None)

    def timeline_enable(self, on: bool = True) -> None:
        """Record per-wave timestamps in every decode launch (kva_timeline_enable)."""
        _lib.call("kva_timeline_enable", self.handle, 1 if on else 0)

    def timeline(self) -> np.ndarray:
        """The last decode's records: int64 [n_wg, grid_rows, 8 waves, 4]
        (entry, first K/V issue, walk end in 100 MHz ticks; XCD << 32 | pages)."""
        n_wg, rows = ctypes.c_int32(), ctypes.c_int32()
        cap = 1 << 22
        buf = (ctypes.c_uint64 * cap)()
        _lib.call("kva_timeline_read", self.handle, buf, cap, ctypes.byref(n_wg), ctypes.byref(rows))
        words = n_wg.value * rows.value * 8 * 4
        return np.frombuffer(buf, dtype=np.uint64, count=words).astype(np.int64).reshape(n_wg.value, rows.value, 8, 4)


class KVCache:
    """Drop-in for the reference ``KVCache`` (engine.py:79-291).

    Layout per full-attention layer is [batch][max_seq][kv_heads][256] fp16
    for K and, separately, V — the reference's own — realised as consecutive
    16-token pages of a ``PagedKVCache`` (batch slot b owns pages
    [b*n, (b+1)*n)).  ``current_len`` is one shared length, as in the
    reference; attention calls receive it explicitly (``seq_len``).
    """

    def __init__(self, config, max_seq_len: int, device: GPUDevice | None = None,
                 tp_size: int = 1, batch_size: int = 1):
        self.config = config
        self.max_seq_len = max_seq_len
        self.device = device
        self.batch_size = batch_size
        self.current_len = 0
        self.num_full_layers = config.num_full_attention_layers
        self.full_layer_indices = [i for i in range(config.num_hidden_layers)
                                   if config.is_full_attention(i)]
        self.local_num_kv_heads = config.num_key_value_heads // tp_size
        self.pos_size_per_batch = self.local_num_kv_heads * config.head_dim * 2
        self.pos_stride = self.pos_size_per_batch
        self._pages_per_slot = (max_seq_len + BLOCK_TOKENS - 1) // BLOCK_TOKENS
        self.batch_stride = self._pages_per_slot * BLOCK_TOKENS * self.pos_stride
        local_heads = config.num_attention_heads // tp_size
        self.paged = PagedKVCache(
            n_layers=self.num_full_layers, max_seqs=batch_size,
            max_blocks=batch_size * self._pages_per_slot,
            max_blocks_per_seq=self._pages_per_slot,
            max_step_tokens=max(16, batch_size * 16, max_seq_len),  # a prefill of up to max_seq_len tokens
            num_heads=local_heads, num_kv_heads=self.local_num_kv_heads,
            head_dim=config.head_dim, rotary_dim=int(config.head_dim * config.partial_rotary_factor),
            eps=config.rms_norm_eps)
        for b in range(batch_size):
            first = b * self._pages_per_slot
            self.paged.set_blocks(b, range(first, first + self._pages_per_slot))
        self.paged.sync_tables()
        self.d_k, self.d_v = self.paged.layer_pools(0)
        self.k_size = self.num_full_layers * batch_size * self.batch_stride
        self.v_size = self.k_size

    def _full_layer_slot(self, layer_idx: int) -> int:
        return self.full_layer_indices.index(layer_idx)

    def layer_k_ptr(self, layer_idx: int, batch_idx: int = 0) -> int:
        k, _ = self.paged.layer_pools(self._full_layer_slot(layer_idx))
        return k + batch_idx * self.batch_stride

    def layer_v_ptr(self, layer_idx: int, batch_idx: int = 0) -> int:
        _, v = self.paged.layer_pools(self._full_layer_slot(layer_idx))
        return v + batch_idx * self.batch_stride

    def get_kv_ptr(self, layer_idx: int, position: int, batch_idx: int = 0):
        return self.paged.row_ptr(self._full_layer_slot(layer_idx), batch_idx, position)

    def append_kv(self, layer_idx: int, k_data: bytes, v_data: bytes, batch_idx: int = 0):
        kp, vp = self.get_kv_ptr(layer_idx, self.current_len, batch_idx)
        n = self.pos_size_per_batch
        _lib.call("kva_memcpy_h2d", kp, bytes(k_data[:n]), n)
        _lib.call("kva_memcpy_h2d", vp, bytes(v_data[:n]), n)

    def append_kv_gpu(self, layer_idx: int, d_k_src: int, d_v_src: int, batch_idx: int = 0):
        kp, vp = self.get_kv_ptr(layer_idx, self.current_len, batch_idx)
        _lib.call("kva_memcpy_d2d", kp, d_k_src, self.pos_size_per_batch)
        _lib.call("kva_memcpy_d2d", vp, d_v_src, self.pos_size_per_batch)

    def append_kv_gpu_batch(self, layer_idx: int, d_k_src: int, d_v_src: int,
                            start_batch_idx: int = 0, num_positions: int = 1):
        kp, vp = self.get_kv_ptr(layer_idx, self.current_len, start_batch_idx)
        n = num_positions * self.pos_stride
        _lib.call("kva_memcpy_d2d", kp, d_k_src, n)
        _lib.call("kva_memcpy_d2d", vp, d_v_src, n)

    def append_kv_gpu_from_batch(self, layer_idx: int, d_k_src: int, d_v_src: int,
                                 batch_idx: int = 0):
        self.append_kv_gpu(layer_idx, d_k_src, d_v_src, batch_idx)

    def advance(self, num_positions: int = 1):
        self.current_len += num_positions

    def reset(self):
        self.current_len = 0

    def cleanup(self):
        self.paged.destroy()


class StepGraph:
    """A recorded step (kva_graph_*): replay it after each begin_step of the
    same shape instead of issuing the per-layer calls again."""

    def __init__(self, cache: PagedKVCache, stream):
        self.cache = cache
        self.stream = stream
        self.handle = None

    def end(self) -> "StepGraph":
        h = ctypes.c_void_p()
        _lib.call("kva_graph_capture_end", self.cache.handle, self.stream, ctypes.byref(h))
        self.handle = h.value
        return self

    def launch(self, stream=None) -> None:
        _lib.call("kva_graph_launch", self.handle, self.stream if stream is None else stream)

    def destroy(self) -> None:
        if self.handle:
            _lib.call("kva_graph_destroy", self.handle)
            self.handle = None
