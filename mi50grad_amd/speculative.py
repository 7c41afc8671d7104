"""Tree speculative verification around the KV-cache path.

Covers the callers of ``kva_tree_verify`` / ``kva_rollback`` in the
reference's speculative driver:

* draft-tree topologies: complete binary, chain and star trees
  (tree_attention.py:271-380) and the trees of the Sequoia optimizer, all as
  parent arrays (``parents[0] == -1``, ``parents[i] < i``: the order new
  tokens take in the cache);
* ``SequoiaTreeOptimizer``: the dynamic program that picks the tree shape
  with the most expected accepted tokens for a node budget
  (tree_optimizer.py:52-330), with ``position_dependent_optimizer``
  (tree_optimizer.py:413-460);
* ``accept_tree_path``: the longest root path whose nodes the model agrees
  with (``TreeSpeculativeDecoder._accept_tree_path``,
  tree_speculative.py:328-383);
* ``TreeVerifyStep``: one verification step over a ``PagedKVCache``: the
  step plan (RoPE positions len + depth, tree bit sets), then, after the
  caller's per-layer append + tree verify and the model's predictions,
  acceptance and the rollback that keeps the accepted path's rows
  contiguous in every layer.

The acceptance rule is the reference's: node i is accepted when the model's
prediction at node i equals node i's draft token and its parent was
accepted; the walk starts at the root.
"""
from __future__ import annotations

from collections import deque
from dataclasses import dataclass
from typing import Iterator, Sequence

import numpy as np

from . import tree as tr

# ---------------------------------------------------------------------------
# topologies


def complete_binary_parents(depth: int, n_nodes: int | None = None) -> list[int]:
    """Parent array of the complete binary tree of the given depth
    (build_complete_binary_tree, tree_attention.py:271-332): BFS order, node
    i's children are 2i+1 and 2i+2.  With ``n_nodes`` (at least the full
    tree's 2^(depth+1)-1) the construction goes on level by level the way
    the reference's does with extra token ids."""
    if depth < 0:
        raise ValueError("depth must be non-negative")
    full = (1 << (depth + 1)) - 1
    n = full if n_nodes is None else n_nodes
    if n < full:
        raise ValueError(f"a depth-{depth} tree needs at least {full} nodes")
    # The reference adds two children to every node of levels 0..depth, in
    # BFS order, while node ids last: the first n nodes of the infinite
    # binary heap, but no node below level depth + 1.
    limit = (1 << (depth + 2)) - 1
    n = min(n, limit)
    return [-1] + [(i - 1) // 2 for i in range(1, n)]


def chain_parents(n_nodes: int) -> list[int]:
    """A chain of n nodes (build_chain_tree, tree_attention.py:335-356)."""
    if n_nodes <= 0:
        raise ValueError("a chain needs at least one node")
    return [-1] + list(range(n_nodes - 1))


def star_parents(n_children: int) -> list[int]:
    """A root with n children (build_star_tree, tree_attention.py:359-380)."""
    if n_children < 0:
        raise ValueError("n_children must be non-negative")
    return [-1] + [0] * n_children


def parents_from_edges(edges: Sequence[tuple[int, int]], num_nodes: int) -> list[int]:
    """Parent array of a tree given as (parent, child) edges over nodes
    0..num_nodes-1 rooted at 0 (the optimizer's output)."""
    parents = [-2] * num_nodes
    parents[0] = -1
    for p, c in edges:
        if not (0 <= p < num_nodes and 0 < c < num_nodes) or parents[c] != -2:
            raise ValueError(f"bad edge ({p}, {c})")
        parents[c] = p
    if -2 in parents:
        raise ValueError("edges do not reach every node")
    tr.validate_parents(parents)
    return parents


def children_of(parents: Sequence[int]) -> list[list[int]]:
    kids: list[list[int]] = [[] for _ in parents]
    for i, p in enumerate(parents):
        if p >= 0:
            kids[p].append(i)
    return kids


# ---------------------------------------------------------------------------
# Sequoia optimizer


@dataclass
class OptimalTree:
    """The optimizer's answer (TreeTopology, tree_optimizer.py:30-49)."""
    edges: list[tuple[int, int]]
    num_nodes: int
    expected_tokens: float

    def to_dict(self) -> dict:
        return {"edges": self.edges, "num_nodes": self.num_nodes, "expected_tokens": self.expected_tokens}

    def parents(self) -> list[int]:
        return parents_from_edges(self.edges, self.num_nodes)


class SequoiaTreeOptimizer:
    """Tree shape with the most expected accepted tokens for a node budget
    (SequoiaTreeOptimizer, tree_optimizer.py:52-330).

    Acceptance at depth d is p(d) = base * (1 - decay)^d up to max_depth and
    0 below.  A subtree rooted at depth d with child subtrees c_1..c_k has
    E = p(d) * (1 + sum E(c_j)) (tree_optimizer.py:149-178); the dynamic
    program tries 1..max_branching children and every split of the remaining
    budget among them (first child 1, 2, ... nodes, the rest recursively),
    keeping the first configuration that is strictly better than a leaf
    (tree_optimizer.py:180-246).  The verification cost is the reference's
    constant (all-reduces x latency, tree_optimizer.py:117-118), reported
    only.
    """

    def __init__(self, base_acceptance_rate: float = 0.54, max_depth: int = 4, max_branching: int = 2,
                 size_budget: int = 16, acceptance_decay: float = 0.0, allreduce_latency_us: float = 46.0,
                 num_allreduces: int = 64):
        if size_budget < 1 or max_depth < 0 or max_branching < 1:
            raise ValueError("size_budget >= 1, max_depth >= 0 and max_branching >= 1 are required")
        self.base_acceptance_rate = base_acceptance_rate
        self.max_depth = max_depth
        self.max_branching = max_branching
        self.size_budget = size_budget
        self.acceptance_decay = acceptance_decay
        self.allreduce_latency_us = allreduce_latency_us
        self.num_allreduces = num_allreduces
        self.verification_cost_ms = num_allreduces * allreduce_latency_us / 1000.0
        self._acceptance_probs = [
            base_acceptance_rate * ((1.0 - acceptance_decay) ** d) if acceptance_decay > 0 else base_acceptance_rate
            for d in range(max_depth + 1)
        ]
        self._memo: dict[tuple[int, int], tuple[float, list[int]]] = {}

    def get_acceptance_prob(self, depth: int) -> float:
        return self._acceptance_probs[depth] if 0 <= depth < len(self._acceptance_probs) else 0.0

    def acceptance_probs(self) -> list[float]:
        return list(self._acceptance_probs)

    def subtree_expectation(self, depth: int, children_expectations: Sequence[float]) -> float:
        return self.get_acceptance_prob(depth) * (1.0 + sum(children_expectations))

    @staticmethod
    def child_distributions(total: int, n_children: int) -> Iterator[tuple[int, ...]]:
        """Every split of ``total`` nodes among ``n_children`` subtrees of at
        least one node each, first child smallest first."""
        if n_children == 1:
            yield (total,)
            return
        for first in range(1, total - n_children + 2):
            for rest in SequoiaTreeOptimizer.child_distributions(total - first, n_children - 1):
                yield (first,) + rest

    def solve(self, budget: int, depth: int) -> tuple[float, list[int]]:
        """(best expectation, child subtree budgets) of a subtree of at most
        ``budget`` nodes rooted at ``depth``."""
        key = (budget, depth)
        if key in self._memo:
            return self._memo[key]
        if budget < 1 or depth > self.max_depth:
            return 0.0, []
        p = self.get_acceptance_prob(depth)
        best, best_sizes = p, []
        child_budget = budget - 1
        for k in range(1, min(self.max_branching, child_budget) + 1):
            for sizes in self.child_distributions(child_budget, k):
                e = self.subtree_expectation(depth, [self.solve(s, depth + 1)[0] for s in sizes])
                if e > best:
                    best, best_sizes = e, list(sizes)
        self._memo[key] = (best, best_sizes)
        return best, best_sizes

    def _build(self, budget: int, depth: int, next_id: int, edges: list[tuple[int, int]]) -> int:
        """Append the edges of the optimal subtree rooted at node ``next_id``;
        return the next free node id.  (The reference numbers a child by the
        next free id minus its budget, tree_optimizer.py:248-292, which names
        the child's root only when its subtree uses its whole budget; here
        the child's root id is taken before its subtree is built, which is
        the same whenever the reference's is well defined.)"""
        root = next_id
        next_id += 1
        if budget <= 1 or depth > self.max_depth:
            return next_id
        _, sizes = self.solve(budget, depth)
        for s in sizes:
            child = next_id
            edges.append((root, child))
            next_id = self._build(s, depth + 1, next_id, edges)
        return next_id

    def find_optimal_tree(self) -> OptimalTree:
        self._memo = {}
        e, _ = self.solve(self.size_budget, 0)
        edges: list[tuple[int, int]] = []
        n = self._build(self.size_budget, 0, 0, edges)
        return OptimalTree(edges=edges, num_nodes=n, expected_tokens=e)

    def compare_with_chain(self) -> dict:
        """The optimal tree against a chain of as many nodes
        (tree_optimizer.py:334-393)."""
        t = self.find_optimal_tree()
        chain, path = 0.0, 1.0
        for d in range(t.num_nodes):
            p = self.get_acceptance_prob(d)
            if p <= 0:
                break
            path *= p
            chain += path
        return {
            "optimal_tree": t.to_dict(),
            "chain": {"length": t.num_nodes, "expected_tokens": chain},
            "improvement": {"absolute": t.expected_tokens - chain,
                            "relative": (t.expected_tokens / chain - 1) * 100 if chain > 0 else 0},
            "efficiency": {"tree": t.expected_tokens / t.num_nodes, "chain": chain / t.num_nodes},
        }


def position_dependent_optimizer(code_domain: bool = False, repetitive_domain: bool = False) -> SequoiaTreeOptimizer:
    """The reference's per-domain settings (tree_optimizer.py:413-460)."""
    if repetitive_domain:
        return SequoiaTreeOptimizer(0.87, max_depth=4, max_branching=3, size_budget=16, acceptance_decay=0.05)
    if code_domain:
        return SequoiaTreeOptimizer(0.59, max_depth=4, max_branching=2, size_budget=16, acceptance_decay=0.05)
    return SequoiaTreeOptimizer(0.54, max_depth=4, max_branching=2, size_budget=16, acceptance_decay=0.0)


def tree_expectation(parents: Sequence[int], probs: Sequence[float]) -> float:
    """Expected accepted tokens of a tree: the sum over nodes of the product
    of p(depth) over the node and its ancestors."""
    d = tr.depths(parents)
    path = [0.0] * len(parents)
    for i, p in enumerate(parents):
        pi = probs[d[i]] if d[i] < len(probs) else 0.0
        path[i] = pi * (path[p] if p >= 0 else 1.0)
    return float(sum(path))


# ---------------------------------------------------------------------------
# acceptance


def accept_tree_path(parents: Sequence[int], draft_tokens: Sequence[int],
                     predicted: Sequence[int]) -> tuple[list[int], list[int]]:
    """(accepted tokens, accepted node indices) of the longest root path on
    which every node's prediction equals its draft token
    (tree_speculative.py:328-383): a breadth-first walk from the root that
    stops a path at its first mismatch; among equally long paths the first
    one the walk reaches wins.  ``predicted[i]`` is the model's choice at
    node i (argmax of its logits)."""
    tr.validate_parents(parents)
    if len(draft_tokens) != len(parents) or len(predicted) != len(parents):
        raise ValueError("draft_tokens and predicted need one entry per node")
    kids = children_of(parents)
    best_tok: list[int] = []
    best_idx: list[int] = []
    queue: deque[tuple[int, list[int], list[int]]] = deque([(0, [], [])])
    while queue:
        i, toks, idxs = queue.popleft()
        if int(predicted[i]) != int(draft_tokens[i]):
            continue
        toks, idxs = toks + [int(draft_tokens[i])], idxs + [i]
        if len(toks) > len(best_tok):
            best_tok, best_idx = toks, idxs
        for c in kids[i]:
            queue.append((c, toks, idxs))
    return best_tok, best_idx


def predictions_from_logits(logits: np.ndarray) -> list[int]:
    """argmax per node of [nodes, vocab] logits."""
    return [int(x) for x in np.asarray(logits).argmax(axis=-1)]


# ---------------------------------------------------------------------------
# one verification step on the cache


class TreeVerifyStep:
    """One tree-verification step of several sequences on a PagedKVCache.

    ``TreeVerifyStep(cache, seq_ids, trees)`` begins the step: the trees'
    nodes are the step's new tokens (node i of sequence b at slot
    len_b + i), RoPE positions are len_b + depth(i) and each node sees the
    cache and its own ancestor set.  The caller then runs, per layer,
    ``cache.append`` and ``cache.tree_verify`` with [sum(nodes)] rows of
    q/k/v in the same order, and the model turns the outputs into
    predictions.  ``finish(accepted_nodes)`` rolls every layer back to
    len_b + len(accepted path), the path's rows moved to slots
    len_b, len_b + 1, ... in path order (``kva_rollback``), which corrects
    the reference's rollback (tp_engine.py:1673-1687: a length cut that
    keeps the first n rows whatever the accepted branch was).
    """

    def __init__(self, cache, seq_ids: Sequence[int], trees: Sequence[Sequence[int]], stream=None):
        if len(seq_ids) != len(trees):
            raise ValueError("one tree per sequence")
        self.cache = cache
        self.seq_ids = [int(s) for s in seq_ids]
        self.trees = [list(t) for t in trees]
        for t in self.trees:
            tr.validate_parents(t)
        self.base_len = [cache.seq_len(s) for s in self.seq_ids]
        self.offsets = np.cumsum([0] + [len(t) for t in self.trees]).tolist()
        self.rope_pos = [L + d for L, t in zip(self.base_len, self.trees) for d in tr.depths(t)]
        self.bits = [b for t in self.trees for b in tr.tree_bits(t)]
        self.stream = stream
        cache.begin_step(self.seq_ids, [len(t) for t in self.trees], rope_pos=self.rope_pos,
                         tree_bits=self.bits, stream=stream)
        self.finished = False

    @property
    def n_tokens(self) -> int:
        return self.offsets[-1]

    def rows_of(self, b: int) -> slice:
        """The step rows (q/k/v/out) of sequence index b."""
        return slice(self.offsets[b], self.offsets[b + 1])

    def accept(self, draft_tokens: Sequence[Sequence[int]],
               predicted: Sequence[Sequence[int]]) -> list[tuple[list[int], list[int]]]:
        """``accept_tree_path`` per sequence."""
        return [accept_tree_path(t, d, p) for t, d, p in zip(self.trees, draft_tokens, predicted)]

    def finish(self, accepted_nodes: Sequence[Sequence[int]]) -> list[int]:
        """Keep each sequence's accepted root path (node indices, root
        first, each the parent of the next) and drop its other tree rows in
        every layer; returns the new lengths."""
        if self.finished:
            raise RuntimeError("step already finished")
        keep = []
        for t, nodes in zip(self.trees, accepted_nodes):
            nodes = [int(n) for n in nodes]
            for k, n in enumerate(nodes):
                want = -1 if k == 0 else nodes[k - 1]
                if not 0 <= n < len(t) or t[n] != want:
                    raise ValueError(f"accepted nodes {nodes} are not a root path of the tree")
            keep.append(nodes)
        self.cache.rollback(self.seq_ids, self.base_len, keep, stream=self.stream)
        self.finished = True
        return [L + len(k) for L, k in zip(self.base_len, keep)]
