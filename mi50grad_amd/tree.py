"""Draft-tree topology helpers for tree-verify attention.

A tree is a parent array in BFS order (parents[0] == -1, parents[i] < i),
the flattening ``TreeTopology`` uses (tree_attention.py:58-92).  Node i sees
its ancestors and itself (``TreeAttentionMask._build_mask``,
tree_attention.py:186-208); ``tree_bits`` encodes that set as one uint64 per
node for ``kva_step_begin``.
"""
from __future__ import annotations

from typing import Sequence

import numpy as np


def validate_parents(parents: Sequence[int]) -> None:
    if len(parents) == 0 or parents[0] != -1:
        raise ValueError("parents[0] must be -1 (the root)")
    if len(parents) > 64:
        raise ValueError("trees of more than 64 nodes are not supported")
    for i, p in enumerate(parents[1:], start=1):
        if not 0 <= p < i:
            raise ValueError(f"parents[{i}] = {p}: a parent must precede its child (BFS order)")


def depths(parents: Sequence[int]) -> list[int]:
    validate_parents(parents)
    d = [0] * len(parents)
    for i in range(1, len(parents)):
        d[i] = d[parents[i]] + 1
    return d


def ancestors(parents: Sequence[int], i: int) -> list[int]:
    out = []
    p = parents[i]
    while p != -1:
        out.append(p)
        p = parents[p]
    return out[::-1]


def tree_bits(parents: Sequence[int]) -> list[int]:
    """Per node, bit j set when node j is node i itself or one of its ancestors."""
    validate_parents(parents)
    bits = []
    for i in range(len(parents)):
        b = 1 << i
        for a in ancestors(parents, i):
            b |= 1 << a
        bits.append(b)
    return bits


def tree_mask(parents: Sequence[int], kv_len: int = 0) -> np.ndarray:
    """[T, T+kv_len] bool mask, tree columns first (the reference's order)."""
    t = len(parents)
    mask = np.zeros((t, t + kv_len), dtype=bool)
    for i, b in enumerate(tree_bits(parents)):
        for j in range(t):
            mask[i, j] = bool((b >> j) & 1)
        mask[i, t:] = True
    return mask


def root_to_node_path(parents: Sequence[int], node: int) -> list[int]:
    """Node indices from the root to ``node`` inclusive (increasing)."""
    return ancestors(parents, node) + [node]
