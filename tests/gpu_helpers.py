"""Shared setup for the GPU parity tests: build a paged cache holding given
rows, run a step through libkvattn, and compute the oracle's expectation."""
from __future__ import annotations

import sys

import numpy as np

from mi50grad_amd import _lib
from mi50grad_amd.kv_cache import PagedKVCache
from mi50grad_amd.rope import rope_tables
from oracle import kvattn_oracle as orc

H, HKV, D = 24, 4, 256


def say(msg: str) -> None:
    """Name the case before a GPU step (flushed, so it survives a crash)."""
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


class Tables:
    def __init__(self, dev, rows: int):
        self.cos, self.sin = rope_tables(rows)
        self.rows = rows
        self.d_cos = dev.array(self.cos)
        self.d_sin = dev.array(self.sin)


def build_cache(lengths, block_ids, extra_rows, n_layers=1, num_heads=H, num_kv_heads=HKV,
                max_step_tokens=4096, rng=None, fill=True, max_blocks=None):
    """A PagedKVCache whose sequence b holds lengths[b] random rows in every
    layer (pages block_ids[b]); returns (cache, k_rows, v_rows) with the rows
    per layer and sequence as fp16 [L, Hkv, D] arrays."""
    rng = rng or np.random.default_rng(0)
    nb = max_blocks or (max(max(ids) for ids in block_ids) + 1)
    mbps = max(len(ids) for ids in block_ids)
    cache = PagedKVCache(n_layers=n_layers, max_seqs=len(lengths), max_blocks=nb,
                         max_blocks_per_seq=mbps, max_step_tokens=max_step_tokens,
                         num_heads=num_heads, num_kv_heads=num_kv_heads)
    k_rows = [[None] * len(lengths) for _ in range(n_layers)]
    v_rows = [[None] * len(lengths) for _ in range(n_layers)]
    extra = extra_rows if isinstance(extra_rows, (list, tuple)) else [extra_rows] * len(lengths)
    for b, ids in enumerate(block_ids):
        assert len(ids) * 16 >= lengths[b] + extra[b]
        cache.set_blocks(b, ids)
    for layer in range(n_layers):
        kimg = np.zeros((nb, 16, num_kv_heads, D), np.float16)
        vimg = np.zeros_like(kimg)
        for b, ids in enumerate(block_ids):
            n = int(lengths[b])
            k = rng.standard_normal((n, num_kv_heads, D), dtype=np.float32).astype(np.float16) if fill \
                else np.zeros((n, num_kv_heads, D), np.float16)
            v = rng.standard_normal((n, num_kv_heads, D), dtype=np.float32).astype(np.float16) if fill \
                else np.zeros((n, num_kv_heads, D), np.float16)
            k_rows[layer][b], v_rows[layer][b] = k, v
            slots = np.arange(n)
            blk = np.asarray(ids)[slots // 16]
            kimg[blk, slots % 16] = k
            vimg[blk, slots % 16] = v
        kp, vp = cache.layer_pools(layer)
        _lib.call("kva_memcpy_h2d", kp, kimg.ctypes.data, kimg.nbytes)
        _lib.call("kva_memcpy_h2d", vp, vimg.ctypes.data, vimg.nbytes)
    for b in range(len(lengths)):
        cache.set_len(b, int(lengths[b]))
    cache.sync_tables()
    return cache, k_rows, v_rows


def expected_norm(x, w, tables: Tables, positions):
    """Oracle norm+RoPE of rows x [n, heads, D] at per-row positions."""
    n, heads, d = x.shape
    pos = np.repeat(np.asarray(positions), heads)
    return orc.qknorm_rope_exact(x.reshape(n * heads, d), w, tables.cos[pos],
                                 tables.sin[pos]).reshape(n, heads, d)


def max_err(a, b) -> float:
    return float(np.max(np.abs(np.asarray(a, np.float32) - np.asarray(b, np.float32))))
