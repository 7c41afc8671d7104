"""Seeded synthetic inputs for the path's five measured configurations.

Draw order and distributions follow the measurement plan: values drawn in
float32 from ``np.random.default_rng(seed)`` and cast to fp16; stored norm
weights are fp16(1 + 0.02*N(0,1)) (the loader stores 1+w, weight_loader.py:
476-480); cache contents are drawn directly as K (already normed and rotated)
and V.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

H, HKV, D = 24, 4, 256
BLOCK = 16
# Config 5's draft tree: depth 3, branching up to 3, BFS order.
C5_PARENTS = [-1, 0, 0, 0, 1, 1, 2, 4, 4]


def normal_f16(rng: np.random.Generator, shape) -> np.ndarray:
    return rng.standard_normal(shape, dtype=np.float32).astype(np.float16)


def norm_weight(rng: np.random.Generator) -> np.ndarray:
    return (1.0 + 0.02 * rng.standard_normal(D, dtype=np.float32)).astype(np.float16)


@dataclass
class C1Inputs:
    q: np.ndarray        # [1, 24, 256]
    k_new: np.ndarray    # [1, 4, 256]
    v_new: np.ndarray    # [1, 4, 256]
    q_norm: np.ndarray   # [256]
    k_norm: np.ndarray   # [256]
    k_cache: np.ndarray  # [255, 4, 256]
    v_cache: np.ndarray  # [255, 4, 256]
    position: int = 255


def c1_inputs(seed: int = 0) -> C1Inputs:
    """Config 1: one layer, batch 1, 255 cached rows, append at position 255."""
    rng = np.random.default_rng(seed)
    q = normal_f16(rng, (1, H, D))
    k_new = normal_f16(rng, (1, HKV, D))
    v_new = normal_f16(rng, (1, HKV, D))
    qn = norm_weight(rng)
    kn = norm_weight(rng)
    kc = normal_f16(rng, (255, HKV, D))
    vc = normal_f16(rng, (255, HKV, D))
    return C1Inputs(q, k_new, v_new, qn, kn, kc, vc)


@dataclass
class RaggedSpec:
    lengths: np.ndarray      # cached rows per sequence before the step
    block_ids: list          # physical pages of each sequence
    n_blocks: int            # pool pages used


def ragged_spec(seed: int, batch: int, lo: int, hi: int, extra_rows: int = 1) -> RaggedSpec:
    """Lengths uniform in [lo, hi]; pages for lengths+extra_rows drawn as a
    random permutation of the pool, assigned to sequences in order."""
    rng = np.random.default_rng(seed)
    lengths = rng.integers(lo, hi + 1, batch)
    nblk = [(int(length) + extra_rows + BLOCK - 1) // BLOCK for length in lengths]
    perm = rng.permutation(sum(nblk))
    ids, o = [], 0
    for n in nblk:
        ids.append([int(x) for x in perm[o:o + n]])
        o += n
    return RaggedSpec(lengths=lengths, block_ids=ids, n_blocks=int(sum(nblk)))


def c3_spec(seed: int = 0, batch: int = 32, lo: int = 1024, hi: int = 8192) -> RaggedSpec:
    """Config 3: ragged batched decode, one appended row per sequence."""
    return ragged_spec(seed, batch, lo, hi, extra_rows=1)


def c5_spec(seed: int = 0, batch: int = 64, lo: int = 4096, hi: int = 32768) -> RaggedSpec:
    """Config 5: long-context tree verify, 9 tree rows per sequence."""
    return ragged_spec(seed, batch, lo, hi, extra_rows=len(C5_PARENTS))


C4_PREFIX = [0, 256, 1024, 2048]
C4_CHUNK = 512


def decode_bytes(ctx_lens) -> dict:
    """Algorithmic bytes of one decode layer-step (ctx = rows attended)."""
    ctx = np.asarray(ctx_lens, dtype=np.int64)
    b = len(ctx)
    kv = int(ctx.sum()) * 2 * HKV * D * 2
    return {"kv": kv, "q": b * H * D * 2, "out": b * H * D * 2, "append": b * 2 * HKV * D * 2}
