"""Write the golden fixtures under tests/golden/ (run from the repo root).

    python tests/golden/make_golden.py

Fixtures:
* rope_0_255.npz       cos/sin fp16 rows for positions 0..255 (config 1/2).
* golden.json          SHA-256 of the full tables up to position 32776 (the
                       longest context of config 5), the numpy version that
                       made them, and the reference's literal known answers
                       for tree masks (tests/test_tree_attention_mask.py:
                       270-291 and 298-340) and ancestor counts
                       (tests/test_tree_vs_causal_attention.py:289-322),
                       transcribed as data.
* c1_golden.npz        config-1 inputs (seed 0) and the oracle's outputs:
                       normalised q/k (bit-exact contract) and the fp32
                       attention output over the 256-row cache.

Nothing here imports the reference; the known answers are data copied from
its tests.
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))

from oracle import kvattn_oracle as orc  # noqa: E402
from mi50grad_amd import workloads  # noqa: E402
from mi50grad_amd.rope import table_digest  # noqa: E402

MAX_POS = 32777  # positions 0..32776: config 5's longest cache plus its tree


def main() -> None:
    cos256, sin256 = orc.rope_tables(256)
    np.savez(HERE / "rope_0_255.npz", cos=cos256, sin=sin256)

    cos_full, sin_full = orc.rope_tables(MAX_POS)
    golden = {
        "numpy_version": np.__version__,
        "rope_rows": MAX_POS,
        "rope_sha256": table_digest(cos_full, sin_full),
        # tests/test_tree_attention_mask.py:270-291: root with two children,
        # kv_len = 2, columns tree-first.
        "tree3_parents": [-1, 0, 0],
        "tree3_kv_len": 2,
        "tree3_rows": [[1, 0, 0, 1, 1], [1, 1, 0, 1, 1], [1, 0, 1, 1, 1]],
        # tests/test_tree_attention_mask.py:298-340: complete binary tree of
        # depth 2 (BFS), kv_len = 2; row 3 sees root, parent 1, itself, KV.
        "tree7_parents": [-1, 0, 0, 1, 1, 2, 2],
        "tree7_kv_len": 2,
        "tree7_row0": [1, 0, 0, 0, 0, 0, 0, 1, 1],
        "tree7_row3": [1, 1, 0, 1, 0, 0, 0, 1, 1],
        # tests/test_tree_vs_causal_attention.py:289-322.
        "tree7_ancestor_counts": [1, 2, 2, 3, 3, 3, 3],
        # Node depths the reference's tests assert (TreeNode.depth =
        # parent.depth + 1, tree_attention.py:35; get_max_depth,
        # get_nodes_at_depth): tests/test_tree_attention_mask.py:44-54 (root
        # 0, children 1), :84-125 (root, two children, a grandchild under the
        # first: max depth 2, one/two/one nodes at depths 0/1/2), :145-170
        # (complete binary trees of depth 0..3), :185-212 (chains of 4 and of
        # 1) and :225-231 (a star of 3 children).  Parent arrays in the
        # reference's BFS numbering.
        "tree_depth_cases": [
            {"parents": [-1, 0, 0], "depths": [0, 1, 1]},
            {"parents": [-1, 0, 0, 1], "max_depth": 2, "nodes_per_depth": [1, 2, 1]},
            {"parents": [-1], "max_depth": 0},
            {"parents": [-1, 0, 0], "max_depth": 1},
            {"parents": [-1, 0, 0, 1, 1, 2, 2], "max_depth": 2},
            {"parents": [-1] + [(i - 1) // 2 for i in range(1, 15)], "max_depth": 3},
            {"parents": [-1, 0, 1, 2], "max_depth": 3},
            {"parents": [-1, 0, 0, 0], "max_depth": 1},
        ],
    }
    (HERE / "golden.json").write_text(json.dumps(golden, indent=1) + "\n")

    c1 = workloads.c1_inputs(0)
    pos = c1.position
    qn = orc.qknorm_rope_exact(c1.q[0], c1.q_norm, np.repeat(cos256[pos:pos + 1], 24, 0),
                               np.repeat(sin256[pos:pos + 1], 24, 0))
    kn = orc.qknorm_rope_exact(c1.k_new[0], c1.k_norm, np.repeat(cos256[pos:pos + 1], 4, 0),
                               np.repeat(sin256[pos:pos + 1], 4, 0))
    k_all = np.concatenate([c1.k_cache, kn[None]], 0)
    v_all = np.concatenate([c1.v_cache, c1.v_new], 0)
    out = orc.attention_fp32(qn[None], k_all, v_all)[0]
    np.savez(HERE / "c1_golden.npz", q=c1.q, k_new=c1.k_new, v_new=c1.v_new, q_norm=c1.q_norm,
             k_norm=c1.k_norm, k_cache=c1.k_cache, v_cache=c1.v_cache, q_normed=qn, k_normed=kn,
             out_fp32=out)
    print("wrote", sorted(p.name for p in HERE.iterdir() if p.suffix in (".npz", ".json")))


if __name__ == "__main__":
    main()
