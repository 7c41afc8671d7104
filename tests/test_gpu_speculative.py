"""GPU: two tree-speculative steps through mi50grad_amd.speculative.

Each sequence has its own tree shape: the config-5 tree, the Sequoia
optimizer's default tree (pre-order node numbering), a complete binary
tree, a chain and a star.  Per layer the step appends the tree rows
(norm + RoPE at len + depth) and runs tree verify.  Outputs are checked
against the fp32 oracle within 2e-3.  Predictions accept a chosen root path
per sequence (tree_speculative.py:328-383).  The rollback keeps that path's
rows, compacted, in every layer; they must be bit-equal to the appended
rows.  A second step then verifies new trees on top of the compacted cache,
so its attention must see exactly the kept rows.
"""
import numpy as np
import pytest

from mi50grad_amd import speculative as sp
from mi50grad_amd import tree as tr
from mi50grad_amd.workloads import C5_PARENTS
from oracle import kvattn_oracle as orc

from gpu_helpers import HKV, H, D, Tables, build_cache, expected_norm, max_err, say

pytestmark = pytest.mark.gpu
TOL = 2e-3

TREES = [C5_PARENTS, sp.SequoiaTreeOptimizer().find_optimal_tree().parents(),
         sp.complete_binary_parents(2), sp.chain_parents(5), sp.star_parents(4)]


def _ids(rng, nblk):
    perm = rng.permutation(sum(nblk))
    ids, o = [], 0
    for n in nblk:
        ids.append([int(x) for x in perm[o:o + n]])
        o += n
    return ids


def _run_step(device, cache, rng, tables, trees, n_layers, k_hist, v_hist):
    """One verify step; returns (step, appended normed K, V per layer) after
    checking every layer's output against the oracle over k_hist/v_hist
    (each sequence's rows before the step)."""
    step = sp.TreeVerifyStep(cache, list(range(len(trees))), trees)
    T = step.n_tokens
    # Expected RoPE positions len + depth from the oracle's depths; the
    # product's (which the kernels were given) must agree.
    exp_pos = [len(k_hist[0][b]) + int(d) for b, par in enumerate(trees) for d in orc.tree_depths(par)]
    assert list(step.rope_pos) == exp_pos
    kns, vs = [], []
    for layer in range(n_layers):
        q = rng.standard_normal((T, H, D), dtype=np.float32).astype(np.float16)
        k = rng.standard_normal((T, HKV, D), dtype=np.float32).astype(np.float16)
        v = rng.standard_normal((T, HKV, D), dtype=np.float32).astype(np.float16)
        qw = (1 + 0.02 * rng.standard_normal(D, dtype=np.float32)).astype(np.float16)
        kw = (1 + 0.02 * rng.standard_normal(D, dtype=np.float32)).astype(np.float16)
        dq, out = device.array(q), device.empty((T, H, D), np.float16)
        cache.append(layer, dq, device.array(k), device.array(v), device.array(qw), device.array(kw),
                     tables.d_cos, tables.d_sin, tables.rows)
        cache.tree_verify(layer, dq, out)
        device.synchronize()
        qn = expected_norm(q, qw, tables, exp_pos)
        kn = expected_norm(k, kw, tables, exp_pos)
        got = out.numpy()
        for b, par in enumerate(trees):
            s = step.rows_of(b)
            exp = orc.tree_attention(qn[s], k_hist[layer][b], v_hist[layer][b], kn[s], v[s], par)
            assert max_err(got[s], exp) <= TOL, (layer, b)
        kns.append(kn)
        vs.append(v)
    return step, kns, vs


def test_two_speculative_steps(device):
    rng = np.random.default_rng(23)
    B, n_layers = len(TREES), 2
    lengths = [int(x) for x in rng.integers(200, 3000, B)]
    room = 2 * max(len(t) for t in TREES)
    ids = _ids(rng, [(L + room + 15) // 16 for L in lengths])
    say("speculative: two verify steps with rollback")
    cache, kr, vr = build_cache(lengths, ids, extra_rows=room, n_layers=n_layers, rng=rng)
    tables = Tables(device, 4000)
    k_hist = [[kr[l][b] for b in range(B)] for l in range(n_layers)]
    v_hist = [[vr[l][b] for b in range(B)] for l in range(n_layers)]
    for rnd in range(2):
        step, kns, vs = _run_step(device, cache, rng, tables, TREES, n_layers, k_hist, v_hist)
        # Predictions agree with the drafts along one root path (to a random
        # node) and nowhere else, so that path is what gets accepted.
        drafts, preds, want = [], [], []
        for par in TREES:
            n = len(par)
            draft = rng.integers(0, 1000, n)
            target = int(rng.integers(0, n))
            path = tr.root_to_node_path(par, target)
            pred = draft + 1
            pred[path] = draft[path]
            drafts.append(draft)
            preds.append(pred)
            want.append(path)
        acc = step.accept(drafts, preds)
        for (toks, nodes), d, w in zip(acc, drafts, want):
            assert nodes == w and toks == [int(d[i]) for i in nodes]
        new_len = step.finish([a[1] for a in acc])
        device.synchronize()
        for b in range(B):
            keep = acc[b][1]
            L = lengths[b]
            assert cache.seq_len(b) == new_len[b] == L + len(keep)
            for layer in range(n_layers):
                s = step.rows_of(b)
                krow, vrow = cache.gather(layer, b, new_len[b])
                exp_k = np.concatenate([k_hist[layer][b], kns[layer][s][keep]])
                exp_v = np.concatenate([v_hist[layer][b], vs[layer][s][keep]])
                assert np.array_equal(krow.view(np.uint16), exp_k.view(np.uint16)), (rnd, b, layer)
                assert np.array_equal(vrow.view(np.uint16), exp_v.view(np.uint16)), (rnd, b, layer)
                k_hist[layer][b], v_hist[layer][b] = exp_k, exp_v
        lengths = new_len
    cache.destroy()

