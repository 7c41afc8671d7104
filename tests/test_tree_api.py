"""The reference's tree classes and the engine installer (CPU only).

Tree classes: the assertions of the reference's own tests
(tests/test_tree_attention_mask.py:33-231 and :270-340), restated against
mi50grad_amd.tree's TreeNode / TreeTopology / TreeAttentionMask and builders,
plus the link to the kernels' input (parent array, tree bits) checked
against the oracle's mask.

Installer: a stand-in engine class that defines the reference's launcher
names in its own body (as InferenceEngine does, engine.py:2371-2857) gets the
libkvattn versions after bind_methods, whatever its class defines.
"""
import json
from pathlib import Path

import numpy as np
import pytest

from mi50grad_amd import attention as att
from mi50grad_amd import tree as tr
from oracle import kvattn_oracle as orc

GOLD = Path(__file__).resolve().parent / "golden" / "golden.json"


def test_tree_node_and_topology_known_answers():
    root = tr.TreeNode(100)
    c1, c2 = tr.TreeNode(200, root), tr.TreeNode(300, root)
    assert root.depth == 0 and root.parent is None and root.children == [c1, c2]
    assert c1.depth == c2.depth == 1 and c1.get_ancestors() == [root]
    assert c1.get_path_from_root() == [root, c1]
    g = tr.TreeNode(400, c1)
    assert g.get_ancestors() == [root, c1]

    tree = tr.TreeTopology(100)
    a = tree.add_child(tree.root, 200)
    b = tree.add_child(tree.root, 300)
    gc = tree.add_child(a, 400)
    assert tree.get_tree_size() == 4 and tree.get_max_depth() == 2
    assert [tree.root.index, a.index, b.index, gc.index] == [0, 1, 2, 3]
    assert tree.get_all_tokens() == [100, 200, 300, 400]
    assert tree.get_nodes_at_depth(0) == [tree.root] and len(tree.get_nodes_at_depth(1)) == 2
    assert tree.get_nodes_at_depth(2) == [gc]
    d = tree.to_dict()
    assert d["tree_size"] == 4 and d["max_depth"] == 2 and len(d["nodes"]) == 4
    assert tree.parents() == [-1, 0, 0, 1]


def test_builders_known_answers():
    for depth, size in ((0, 1), (1, 3), (2, 7), (3, 15)):
        t = tr.build_complete_binary_tree(100, depth)
        assert t.get_tree_size() == size and t.get_max_depth() == depth
    assert tr.build_complete_binary_tree(100, 1).get_all_tokens() == [100, 101, 102]
    assert tr.build_complete_binary_tree(100, 2).get_all_tokens() == list(range(100, 107))
    custom = [10, 20, 30, 40, 50, 60, 70]
    assert tr.build_complete_binary_tree(10, 2, token_ids=custom).get_all_tokens() == custom
    with pytest.raises(ValueError):
        tr.build_complete_binary_tree(0, 2, token_ids=[1, 2, 3])
    chain = tr.build_chain_tree([100, 200, 300, 400])
    assert chain.get_tree_size() == 4 and chain.get_max_depth() == 3
    assert chain.root.children[0].token_id == 200 and chain.root.children[0].children[0].token_id == 300
    assert tr.build_chain_tree([999]).get_max_depth() == 0
    star = tr.build_star_tree(100, [200, 300, 400])
    assert star.get_tree_size() == 4 and star.get_max_depth() == 1
    assert [c.token_id for c in star.root.children] == [200, 300, 400]


def test_mask_known_answers_and_kernel_inputs():
    g = json.loads(GOLD.read_text())
    t3 = tr.build_star_tree(0, [1, 2])
    m3 = tr.TreeAttentionMask(t3, kv_len=g["tree3_kv_len"])
    assert m3.to_dense_int().tolist() == g["tree3_rows"]
    assert m3.get_mask().shape == (3, 5) and m3.get_causal_mask().shape == (3, 3)
    t7 = tr.build_complete_binary_tree(0, 2)
    m7 = tr.TreeAttentionMask(t7, kv_len=g["tree7_kv_len"])
    assert m7.to_dense_int()[0].tolist() == g["tree7_row0"]
    assert m7.to_dense_int()[3].tolist() == g["tree7_row3"]
    assert m7.to_dense_int()[:, :7].sum(1).tolist() == g["tree7_ancestor_counts"]
    assert tr.verify_tree_mask_correctness(m7)
    m7.update_kv_len(5)
    assert m7.mask.shape == (7, 12) and m7.mask[:, 7:].all()
    broken = tr.TreeAttentionMask(t7, 2)
    broken.mask[2, 1] = True  # a non-ancestor
    assert not tr.verify_tree_mask_correctness(broken)
    # What the kernels are given equals the oracle's visibility.
    par = [-1, 0, 0, 0, 1, 1, 2, 4, 4]
    m = tr.TreeAttentionMask(tr.TreeTopology.from_parents(par), kv_len=6)
    assert np.array_equal(m.mask, orc.tree_mask_reference(par, 6))
    assert m.tree_bits() == [int(x) for x in orc.tree_row_bits(par)]
    assert "T 0" in m.visualize()


class _ReferenceStyleEngine:
    """Defines the reference's launcher names in its own class body."""

    def _launch_qknorm_rope(self, *a):
        raise AssertionError("reference kernel called")

    _launch_qknorm_rope_cachew = _launch_decode_attn_256 = _launch_decode_attn_256_batched = \
        _prefill_full_attention = build_decode_launch_cache = set_direct_kv_write = \
        rollback_kv_cache = _launch_gemv_fp16 = _launch_qknorm_rope


def test_bind_methods_overrides_the_engine_class():
    eng = _ReferenceStyleEngine()
    att.bind_methods(eng)
    for name in att.ENGINE_METHODS:
        assert getattr(eng, name).__func__ is getattr(att.FullAttentionLaunchers, name), name
    # The engine's own GEMV stays unless asked for.
    assert eng._launch_gemv_fp16.__func__ is _ReferenceStyleEngine._launch_gemv_fp16
    att.bind_methods(eng, names=(), gemv=True)
    assert eng._launch_gemv_fp16.__func__ is att.FullAttentionLaunchers._launch_gemv_fp16
