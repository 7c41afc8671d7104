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


# ---- the reference's tree classes (tree_attention.py:20-268) --------------
# Same names, attributes and results, so speculative-decoding code written
# against the reference builds its trees and masks here unchanged; each
# topology also hands kva_step_begin its parent array and tree bits.

class TreeNode:
    """A draft token in the tree (tree_attention.py:20-57): token_id, parent,
    children, depth (root 0) and index (BFS position, set by the topology)."""

    def __init__(self, token_id: int, parent: "TreeNode | None" = None):
        self.token_id = token_id
        self.parent = parent
        self.children: list[TreeNode] = []
        self.depth = 0 if parent is None else parent.depth + 1
        self.index = 0
        if parent is not None:
            parent.children.append(self)

    def get_ancestors(self) -> list["TreeNode"]:
        """Root first, parent last (self excluded)."""
        chain = []
        node = self.parent
        while node is not None:
            chain.append(node)
            node = node.parent
        return chain[::-1]

    def get_path_from_root(self) -> list["TreeNode"]:
        return self.get_ancestors() + [self]

    def __repr__(self):
        return f"TreeNode(token={self.token_id}, depth={self.depth}, idx={self.index})"


class TreeTopology:
    """A draft tree numbered in insertion (BFS) order (tree_attention.py:
    60-145).  ``parents()`` is the parent array the kernels take."""

    def __init__(self, root_token: int):
        self.root = TreeNode(root_token)
        self.nodes: list[TreeNode] = [self.root]

    def add_child(self, parent_node: TreeNode, token_id: int) -> TreeNode:
        child = TreeNode(token_id, parent_node)
        child.index = len(self.nodes)
        self.nodes.append(child)
        return child

    def get_node_by_index(self, index: int) -> TreeNode:
        return self.nodes[index]

    def get_all_tokens(self) -> list[int]:
        return [n.token_id for n in self.nodes]

    def get_max_depth(self) -> int:
        return max(n.depth for n in self.nodes)

    def get_tree_size(self) -> int:
        return len(self.nodes)

    def get_nodes_at_depth(self, depth: int) -> list[TreeNode]:
        return [n for n in self.nodes if n.depth == depth]

    def parents(self) -> list[int]:
        return [-1 if n.parent is None else n.parent.index for n in self.nodes]

    def to_dict(self) -> dict:
        return {
            "root_token": self.root.token_id,
            "nodes": [{"index": n.index, "token_id": n.token_id, "depth": n.depth,
                       "parent_index": None if n.parent is None else n.parent.index,
                       "children_indices": [c.index for c in n.children]} for n in self.nodes],
            "tree_size": self.get_tree_size(),
            "max_depth": self.get_max_depth(),
        }

    @classmethod
    def from_parents(cls, parents: Sequence[int], tokens: Sequence[int] | None = None) -> "TreeTopology":
        validate_parents(parents)
        toks = list(tokens) if tokens is not None else list(range(len(parents)))
        tree = cls(toks[0])
        for i in range(1, len(parents)):
            tree.add_child(tree.nodes[parents[i]], toks[i])
        return tree


class TreeAttentionMask:
    """Tree attention mask (tree_attention.py:148-268): [T, T + kv_len] bool,
    tree columns first, then the KV cache; node i sees itself, its
    ancestors and every cache position.  ``tree_bits()`` is the same
    visibility over the tree rows as kva_step_begin takes it (the cache
    columns are implied: the kernels always see the whole cache)."""

    def __init__(self, tree_topology: TreeTopology, kv_len: int = 0):
        self.tree = tree_topology
        self.kv_len = kv_len
        self.tree_size = tree_topology.get_tree_size()
        self.mask = self._build_mask()

    def _build_mask(self) -> np.ndarray:
        return tree_mask(self.tree.parents(), self.kv_len)

    def get_mask(self) -> np.ndarray:
        return self.mask

    def get_causal_mask(self) -> np.ndarray:
        return self.mask[:, :self.tree_size]

    def update_kv_len(self, kv_len: int) -> None:
        self.kv_len = kv_len
        self.mask = self._build_mask()

    def to_dense_int(self) -> np.ndarray:
        return self.mask.astype(np.int32)

    def tree_bits(self) -> list[int]:
        return tree_bits(self.tree.parents())

    def visualize(self) -> str:
        t = self.tree_size
        head = "     " + " ".join(f"T{i:2d}" for i in range(t))
        if self.kv_len > 0:
            head += " " + " ".join(f"K{i:2d}" for i in range(self.kv_len))
        rows = [head]
        for i in range(t):
            cells = "".join("  1 " if v else "  0 " for v in self.mask[i])
            rows.append(f"T{i:2d}: " + cells)
        return "\n".join(rows)


def build_complete_binary_tree(root_token: int, depth: int,
                               token_ids: Sequence[int] | None = None) -> TreeTopology:
    """Complete binary tree of the given depth in BFS order
    (tree_attention.py:270-332): 2^(depth+1) - 1 nodes with token ids
    root_token, root_token+1, ...  Given token_ids (at least that many), the
    reference's construction keeps filling one level further while ids
    remain (its level loop runs through depth inclusive), so up to
    2^(depth+2) - 1 nodes are taken; so are they here."""
    if depth < 0:
        raise ValueError("depth must be non-negative")
    n = 2 ** (depth + 1) - 1
    if token_ids is not None and len(token_ids) < n:
        raise ValueError(f"token_ids must have at least {n} tokens for depth {depth}")
    if token_ids is None:
        toks = list(range(root_token, root_token + n))
    else:
        toks = list(token_ids[:2 ** (depth + 2) - 1])
    return TreeTopology.from_parents([-1] + [(i - 1) // 2 for i in range(1, len(toks))], toks)


def build_chain_tree(token_ids: Sequence[int]) -> TreeTopology:
    """A chain: each node the only child of the one before
    (tree_attention.py:335-356)."""
    if len(token_ids) == 0:
        raise ValueError("token_ids must not be empty")
    return TreeTopology.from_parents([-1] + list(range(len(token_ids) - 1)), token_ids)


def build_star_tree(root_token: int, children_tokens: Sequence[int]) -> TreeTopology:
    """A root with children and no grandchildren (tree_attention.py:359-380)."""
    return TreeTopology.from_parents([-1] + [0] * len(children_tokens), [root_token] + list(children_tokens))


def verify_tree_mask_correctness(mask: TreeAttentionMask, verbose: bool = False) -> bool:
    """The mask's invariants (tree_attention.py:387-460): self and every
    ancestor visible, every cache column visible, no other tree column, and
    lower triangular over the tree columns (BFS order)."""
    dense = mask.to_dense_int()
    t = mask.tree_size
    problems = []
    for node in mask.tree.nodes:
        i = node.index
        seen = {a.index for a in node.get_ancestors()} | {i}
        for j in range(t):
            if bool(dense[i, j]) != (j in seen):
                problems.append(f"node {i}, tree column {j}")
            if j > i and dense[i, j]:
                problems.append(f"node {i} sees later node {j}")
        if mask.kv_len > 0 and not dense[i, t:t + mask.kv_len].all():
            problems.append(f"node {i} misses a KV position")
    if verbose:
        print("\n".join(problems) if problems else "All tree mask correctness checks passed!")
    return not problems
