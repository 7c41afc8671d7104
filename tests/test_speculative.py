"""Speculative tree driver on the CPU: the Sequoia optimizer, tree builders,
acceptance, and the verification step's plan and rollback on a host-only
cache.

Pins:
* the reference's own known answers (tests/test_tree_optimizer.py:33-200,
  277-400): configuration, the cost constant, acceptance probabilities
  (uniform and decayed), subtree expectations 0.5 / 0.75 / 1.0, the DP for
  budgets 1 and 2, E >= 2.0 for the default optimizer, the domain order
  repetitive > code > default, the tree never below the chain;
* brute force: the DP's optimum equals the best of every tree (parent
  array) within the budget, depth and branching limits, and the tree it
  builds has that expectation by direct summation of path products;
* acceptance against an exhaustive search over root paths with the
  reference's breadth-first tie rule (tree_speculative.py:328-383).
"""
import itertools
import math

import numpy as np
import pytest

from mi50grad_amd import speculative as sp
from mi50grad_amd import tree as tr
from mi50grad_amd.kv_cache import PagedKVCache
from mi50grad_amd.workloads import C5_PARENTS


# ---------------------------------------------------------------------------
# reference known answers

def test_optimizer_configuration_and_cost():
    o = sp.SequoiaTreeOptimizer()
    assert (o.base_acceptance_rate, o.max_depth, o.max_branching, o.size_budget, o.acceptance_decay) == \
        (0.54, 4, 2, 16, 0.0)
    assert abs(o.verification_cost_ms - 64 * 46.0 / 1000.0) < 1e-9
    c = sp.SequoiaTreeOptimizer(0.60, max_depth=5, max_branching=3, size_budget=32, acceptance_decay=0.1)
    assert (c.max_depth, c.max_branching, c.size_budget) == (5, 3, 32)
    assert len(c.acceptance_probs()) == 6


def test_acceptance_probabilities():
    o = sp.SequoiaTreeOptimizer(0.54)
    assert all(abs(o.get_acceptance_prob(d) - 0.54) < 1e-12 for d in range(5))
    d = sp.SequoiaTreeOptimizer(0.60, acceptance_decay=0.1, max_depth=5)
    assert abs(d.get_acceptance_prob(0) - 0.6) < 1e-9
    assert abs(d.get_acceptance_prob(1) - 0.54) < 1e-9
    assert abs(d.get_acceptance_prob(2) - 0.486) < 1e-9
    assert abs(d.get_acceptance_prob(5) - 0.6 * 0.9 ** 5) < 1e-9
    assert d.get_acceptance_prob(10) == 0.0


def test_subtree_expectation_and_small_budgets():
    o = sp.SequoiaTreeOptimizer(0.5, max_depth=3, max_branching=2, size_budget=4)
    assert abs(o.subtree_expectation(0, []) - 0.5) < 1e-12
    assert abs(o.subtree_expectation(0, [0.5]) - 0.75) < 1e-12
    assert abs(o.subtree_expectation(0, [0.5, 0.5]) - 1.0) < 1e-12
    assert o.solve(1, 0) == (0.5, [])
    e, ch = o.solve(2, 0)
    assert abs(e - 0.75) < 1e-12 and len(ch) == 1
    assert o.solve(3, 0) == o.solve(3, 0)


def test_default_targets_and_domain_order():
    t = sp.SequoiaTreeOptimizer().find_optimal_tree()
    assert t.expected_tokens >= 2.0 and t.expected_tokens > 0.54
    assert 1 <= t.num_nodes <= 16
    rep = sp.position_dependent_optimizer(repetitive_domain=True).find_optimal_tree()
    code = sp.position_dependent_optimizer(code_domain=True).find_optimal_tree()
    dflt = sp.position_dependent_optimizer().find_optimal_tree()
    assert rep.expected_tokens > code.expected_tokens > dflt.expected_tokens
    for opt in (sp.SequoiaTreeOptimizer(), sp.SequoiaTreeOptimizer(0.6, acceptance_decay=0.1)):
        cmp = opt.compare_with_chain()
        assert cmp["optimal_tree"]["expected_tokens"] >= cmp["chain"]["expected_tokens"] - 1e-12


def test_chain_closed_form():
    # A chain of L nodes under uniform p: p + p^2 + ... + p^L.
    p = 0.54
    o = sp.SequoiaTreeOptimizer(p, max_depth=10, max_branching=1, size_budget=6)
    t = o.find_optimal_tree()
    assert t.parents() == sp.chain_parents(6)
    assert abs(t.expected_tokens - p * (1 - p ** 6) / (1 - p)) < 1e-12


# ---------------------------------------------------------------------------
# brute force

def all_trees(n):
    """Every parent array of n nodes with parents[i] < i."""
    for rest in itertools.product(*[range(i) for i in range(1, n)]):
        yield [-1] + list(rest)


def brute_best(budget, probs, max_branching):
    best = 0.0
    for n in range(1, budget + 1):
        for par in all_trees(n):
            if max((list(par).count(i) for i in range(n)), default=0) > max_branching:
                continue
            best = max(best, sp.tree_expectation(par, probs))
    return best


@pytest.mark.parametrize("p,decay,depth,branch,budget", [
    (0.54, 0.0, 4, 2, 7), (0.5, 0.0, 2, 3, 6), (0.8, 0.1, 3, 2, 7), (0.3, 0.0, 4, 3, 6), (0.9, 0.2, 1, 4, 6),
])
def test_dp_optimum_matches_brute_force(p, decay, depth, branch, budget):
    o = sp.SequoiaTreeOptimizer(p, max_depth=depth, max_branching=branch, size_budget=budget, acceptance_decay=decay)
    t = o.find_optimal_tree()
    best = brute_best(budget, o.acceptance_probs(), branch)
    assert abs(t.expected_tokens - best) < 1e-12
    par = t.parents()
    assert len(par) <= budget
    assert abs(sp.tree_expectation(par, o.acceptance_probs()) - t.expected_tokens) < 1e-12
    assert max(tr.depths(par)) <= depth
    assert max((par.count(i) for i in range(len(par))), default=0) <= branch


def test_budget_beyond_depth_reach():
    # 16 nodes but depth 1 and branching 2: at most 3 useful nodes; the tree
    # built has only those and the same expectation.
    o = sp.SequoiaTreeOptimizer(0.54, max_depth=1, max_branching=2, size_budget=16)
    t = o.find_optimal_tree()
    assert t.parents() == [-1, 0, 0]
    assert abs(t.expected_tokens - 0.54 * (1 + 2 * 0.54)) < 1e-12


# ---------------------------------------------------------------------------
# builders

def test_builders():
    for d in range(4):
        par = sp.complete_binary_parents(d)
        assert len(par) == 2 ** (d + 1) - 1
        assert tr.depths(par) == [int(math.log2(i + 1)) for i in range(len(par))]
        kids = sp.children_of(par)
        assert all(len(k) in (0, 2) for k in kids)
    assert sp.complete_binary_parents(1, 5) == [-1, 0, 0, 1, 1]
    assert len(sp.complete_binary_parents(1, 100)) == 7  # no node below level depth + 1
    with pytest.raises(ValueError):
        sp.complete_binary_parents(2, 3)
    assert sp.chain_parents(4) == [-1, 0, 1, 2]
    assert sp.star_parents(3) == [-1, 0, 0, 0]
    assert sp.parents_from_edges([(0, 1), (1, 2), (0, 3)], 4) == [-1, 0, 1, 0]
    with pytest.raises(ValueError):
        sp.parents_from_edges([(0, 1)], 3)
    # The optimizer's pre-order trees are valid step trees.
    t = sp.SequoiaTreeOptimizer().find_optimal_tree()
    tr.validate_parents(t.parents())


# ---------------------------------------------------------------------------
# acceptance

def bfs_order(parents):
    kids = sp.children_of(parents)
    order, q = [], [0]
    while q:
        i = q.pop(0)
        order.append(i)
        q.extend(kids[i])
    return order


def brute_accept(parents, draft, pred):
    ok = [int(pred[i]) == int(draft[i]) for i in range(len(parents))]
    rank = {n: k for k, n in enumerate(bfs_order(parents))}
    best = None
    for n in range(len(parents)):
        path = tr.root_to_node_path(parents, n)
        if all(ok[i] for i in path):
            key = (-len(path), rank[n])
            if best is None or key < best[0]:
                best = (key, path)
    if best is None:
        return [], []
    return [int(draft[i]) for i in best[1]], best[1]


def test_acceptance_matches_exhaustive_search():
    rng = np.random.default_rng(0)
    trees = [C5_PARENTS, sp.complete_binary_parents(2), sp.chain_parents(6), sp.star_parents(4),
             sp.SequoiaTreeOptimizer().find_optimal_tree().parents()]
    for _ in range(400):
        par = trees[rng.integers(len(trees))]
        draft = rng.integers(0, 4, len(par))
        pred = np.where(rng.random(len(par)) < 0.7, draft, rng.integers(0, 4, len(par)))
        assert sp.accept_tree_path(par, draft, pred) == brute_accept(par, draft, pred)


def test_acceptance_cases():
    par = C5_PARENTS
    draft = list(range(10, 19))
    assert sp.accept_tree_path(par, draft, [0] * 9) == ([], [])  # the root is rejected
    toks, nodes = sp.accept_tree_path(par, draft, draft)  # everything agrees: the first deepest path
    assert nodes == [0, 1, 4, 7] and toks == [10, 11, 14, 17]
    pred = list(draft)
    pred[7] = -1
    assert sp.accept_tree_path(par, draft, pred)[1] == [0, 1, 4, 8]
    logits = np.zeros((9, 32))
    logits[np.arange(9), draft] = 1.0
    assert sp.predictions_from_logits(logits) == draft


# ---------------------------------------------------------------------------
# the verification step on a host-only cache

def test_verify_step_plan_and_rollback():
    cache = PagedKVCache(n_layers=2, max_seqs=4, max_blocks=40, max_blocks_per_seq=16, max_step_tokens=64,
                         host_only=True)
    base = [37, 5, 100]
    for s, n in enumerate(base):
        cache.reserve(s, n)
        cache.set_len(s, n)
    trees = [C5_PARENTS, sp.chain_parents(4), sp.complete_binary_parents(1)]
    step = sp.TreeVerifyStep(cache, [0, 1, 2], trees)
    assert step.n_tokens == 9 + 4 + 3
    assert step.rows_of(1) == slice(9, 13)
    assert step.rope_pos[:9] == [37 + d for d in tr.depths(C5_PARENTS)]
    assert step.bits[9:13] == tr.tree_bits(sp.chain_parents(4))
    assert [cache.seq_len(s) for s in range(3)] == [37 + 9, 5 + 4, 100 + 3]
    drafts = [list(range(9)), [5, 6, 7, 8], [1, 2, 3]]
    preds = [[0, 1, 2, 3, 4, 0, 0, 7, 0], [5, 6, 0, 0], [1, 0, 3]]
    acc = step.accept(drafts, preds)
    assert [a[1] for a in acc] == [[0, 1, 4, 7], [0, 1], [0, 2]]
    with pytest.raises(ValueError):
        sp.TreeVerifyStep.finish(step, [[0, 4], [0], [0]])  # not a root path
    assert step.finish([a[1] for a in acc]) == [41, 7, 102]
    assert [cache.seq_len(s) for s in range(3)] == [41, 7, 102]
    with pytest.raises(RuntimeError):
        step.finish([[0], [0], [0]])
    cache.destroy()
