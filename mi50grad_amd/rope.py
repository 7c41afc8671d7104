"""RoPE cos/sin tables, computed on the host as the reference engine does.

``rope_tables`` follows ``InferenceEngine._init_rope_tables``
(engine.py:1025-1046): float32 inverse frequencies for the rotary half of
``head_dim * partial_rotary_factor`` dims, a float32 outer product with the
positions, float32 cos/sin, then fp16.  Row ``p`` is what the kernels read for
RoPE position ``p`` (the reference addresses it as d_cos + p*half*2 bytes,
engine.py:2387).
"""
from __future__ import annotations

import hashlib

import numpy as np


def rope_tables(max_seq: int, head_dim: int = 256, partial_rotary_factor: float = 0.25,
                theta: float = 10000000.0):
    rotary_dim = int(head_dim * partial_rotary_factor)
    half = rotary_dim // 2
    freqs = 1.0 / (theta ** (np.arange(0, half, dtype=np.float32) * 2.0 / rotary_dim))
    positions = np.arange(max_seq, dtype=np.float32)
    angles = np.outer(positions, freqs)
    return np.cos(angles).astype(np.float16), np.sin(angles).astype(np.float16)


def table_digest(cos: np.ndarray, sin: np.ndarray) -> str:
    """SHA-256 over the fp16 bytes of cos then sin (little endian)."""
    h = hashlib.sha256()
    h.update(np.ascontiguousarray(cos, dtype="<f2").tobytes())
    h.update(np.ascontiguousarray(sin, dtype="<f2").tobytes())
    return h.hexdigest()
