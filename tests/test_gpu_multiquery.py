"""GPU parity: MFMA chunked prefill and tree verify, and tree rollback.

Oracle: fp32 attention with the causal-chunk rule (new row i sees slots
[0, len_before + i]) or the tree mask (tree_attention.py:186-208 in cache
column order); tolerance 2e-3.  Covers the config-4 workload (4 sequences,
512-token chunks after 0/256/1024/2048 cached rows, seed 0), ragged chunk
and prefix edge cases, the reference's own causal prefill shapes
(tests/test_flash_attn_v3.py:214-274, bar 1e-2 there), tree verify with the
config-5 tree, chain tree == causal, and rollback compaction in every layer.
"""
import numpy as np
import pytest

from mi50grad_amd import tree as tr
from mi50grad_amd.workloads import C4_CHUNK, C4_PREFIX, C5_PARENTS
from oracle import kvattn_oracle as orc

from gpu_helpers import HKV, H, D, Tables, build_cache, expected_norm, max_err, say

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _ids(rng, nblk):
    perm = rng.permutation(sum(nblk))
    ids, o = [], 0
    for n in nblk:
        ids.append([int(x) for x in perm[o:o + n]])
        o += n
    return ids


def run_prefilled(device, prefix, chunk, num_heads=H, num_kv_heads=HKV, seed=0, scale=1.0,
                  tree_parents=None, causal_on_tree_step=False):
    """Cache rows [0, prefix+chunk) pre-filled with random K/V (no append);
    attention of the chunk's queries through kva_prefill / kva_tree_verify
    (causal_on_tree_step: kva_prefill on a step begun with the tree's bits,
    compared with the causal rule)."""
    rng = np.random.default_rng(seed)
    B = len(prefix)
    total = [p + c for p, c in zip(prefix, chunk)]
    ids = _ids(rng, [(t + 15) // 16 for t in total])
    cache, kr, vr = build_cache(total, ids, extra_rows=0, num_heads=num_heads,
                                num_kv_heads=num_kv_heads, rng=rng)
    for b in range(B):
        cache.set_len(b, prefix[b])
    T = sum(chunk)
    q = (rng.standard_normal((T, num_heads, D), dtype=np.float32) * scale).astype(np.float16)
    dq, out = device.array(q), device.empty((T, num_heads, D), np.float16)
    if tree_parents is None:
        cache.begin_step(list(range(B)), chunk)
        cache.prefill(0, dq, out)
    else:
        bits = tr.tree_bits(tree_parents) * B
        cache.begin_step(list(range(B)), chunk, tree_bits=bits)
        if causal_on_tree_step:
            cache.prefill(0, dq, out)
        else:
            cache.tree_verify(0, dq, out)
    device.synchronize()
    got = out.numpy()
    exp = np.zeros((T, num_heads, D), np.float32)
    t = 0
    for b in range(B):
        n = chunk[b]
        if tree_parents is None or causal_on_tree_step:
            exp[t:t + n] = orc.chunk_attention(q[t:t + n], kr[0][b], vr[0][b], prefix[b])
        else:
            P = prefix[b]
            exp[t:t + n] = orc.tree_attention(q[t:t + n], kr[0][b][:P], vr[0][b][:P], kr[0][b][P:],
                                              vr[0][b][P:], tree_parents)
        t += n
    cache.destroy()
    return got, exp


@pytest.mark.parametrize("prefix,chunk", [
    ([0], [1]), ([0], [16]), ([0], [17]), ([5], [1]), ([15], [33]), ([31], [5]),
    ([100, 0, 7], [40, 3, 64]), ([0, 1000], [200, 31]),
])
def test_prefill_edges(device, prefix, chunk):
    say(f"prefill edges prefix={prefix} chunk={chunk}")
    got, exp = run_prefilled(device, prefix, chunk, seed=sum(prefix) + sum(chunk))
    assert max_err(got, exp) <= TOL


@pytest.mark.parametrize("S", [16, 64, 128, 512])
def test_prefill_reference_causal_shapes(device, S):
    """tests/test_flash_attn_v3.py:214-240 shapes: heads 4, kv heads 2, causal
    from position 0, queries x0.1 (the reference's bar was 1e-2)."""
    say(f"prefill reference shape S={S}")
    got, exp = run_prefilled(device, [0], [S], num_heads=4, num_kv_heads=2, seed=42, scale=0.1)
    assert max_err(got, exp) <= TOL


def test_prefill_c4_workload(device):
    """Config 4: 4 sequences, 512-token chunks after 0/256/1024/2048 cached rows,
    appended through the fused norm+RoPE kernel, then causal prefill."""
    rng = np.random.default_rng(0)
    prefix = list(C4_PREFIX)
    chunk = [C4_CHUNK] * 4
    ids = _ids(rng, [(p + c + 15) // 16 for p, c in zip(prefix, chunk)])
    say("prefill c4 workload")
    cache, kr, vr = build_cache(prefix, ids, extra_rows=chunk, rng=rng)
    tables = Tables(device, 4096)
    T = sum(chunk)
    q = rng.standard_normal((T, H, D), dtype=np.float32).astype(np.float16)
    k = rng.standard_normal((T, HKV, D), dtype=np.float32).astype(np.float16)
    v = rng.standard_normal((T, HKV, D), dtype=np.float32).astype(np.float16)
    qw = (1 + 0.02 * rng.standard_normal(D, dtype=np.float32)).astype(np.float16)
    kw = (1 + 0.02 * rng.standard_normal(D, dtype=np.float32)).astype(np.float16)
    dq, out = device.array(q), device.empty((T, H, D), np.float16)
    cache.begin_step([0, 1, 2, 3], chunk)
    cache.append(0, dq, device.array(k), device.array(v), device.array(qw), device.array(kw),
                 tables.d_cos, tables.d_sin, tables.rows)
    cache.prefill(0, dq, out)
    device.synchronize()
    pos = np.concatenate([np.arange(p, p + c) for p, c in zip(prefix, chunk)])
    qn = expected_norm(q, qw, tables, pos)
    kn = expected_norm(k, kw, tables, pos)
    got = out.numpy()
    t = 0
    for b in range(4):
        n = chunk[b]
        kall = np.concatenate([kr[0][b], kn[t:t + n]])
        vall = np.concatenate([vr[0][b], v[t:t + n]])
        exp = orc.chunk_attention(qn[t:t + n], kall, vall, prefix[b])
        assert max_err(got[t:t + n], exp) <= TOL, b
        t += n
    cache.destroy()


@pytest.mark.parametrize("heads,kv", [(8, 8), (12, 4), (16, 2), (8, 2)])
def test_multi_query_groups(device, heads, kv):
    """GQA groups 1, 3, 8 and 4: a unit's query rows pack (token, head)
    pairs, so the tile's token count and row layout depend on the group.
    Causal chunks long enough for two tiles per wave, and a 9-node tree
    (one tile per wave, except for a group of 8)."""
    say(f"multi-query groups heads={heads} kv={kv}")
    got, exp = run_prefilled(device, [37, 0, 130], [70, 9, 140], num_heads=heads, num_kv_heads=kv,
                             seed=heads * 10 + kv)
    assert max_err(got, exp) <= TOL
    got, exp = run_prefilled(device, [300, 20, 1], [9, 9, 9], num_heads=heads, num_kv_heads=kv,
                             seed=heads * 10 + kv + 1, tree_parents=C5_PARENTS)
    assert max_err(got, exp) <= TOL


def test_tree_verify_small(device):
    say("tree verify small")
    got, exp = run_prefilled(device, [100, 37, 2000, 0], [9, 9, 9, 9], seed=5, tree_parents=C5_PARENTS)
    assert max_err(got, exp) <= TOL


def test_chain_tree_equals_causal_prefill(device):
    parents = [-1, 0, 1, 2, 3, 4, 5]
    say("chain tree vs causal")
    tree_out, exp = run_prefilled(device, [300, 50], [7, 7], seed=9, tree_parents=parents)
    causal_out, _ = run_prefilled(device, [300, 50], [7, 7], seed=9)
    assert max_err(tree_out, exp) <= TOL
    assert max_err(tree_out, causal_out) <= 1e-3


def test_prefill_block_sizes(device):
    """An eight-wave prefill step plans 64-key blocks; kva_prefill on a step
    begun with tree bits runs the same causal rule on 32-key blocks, and the
    tree kernel verifies the chain tree on 32-key blocks: all three agree
    with the causal oracle, each other within its bar.  Contexts cover a
    block's end exactly (64, 128 rows) and one past it."""
    parents = [-1] + list(range(39))  # a chain of 40: 240 query rows, eight-wave tiles
    prefix, chunk = [24, 88, 0, 1000, 985], [40] * 5
    say("prefill block sizes")
    plain, exp = run_prefilled(device, prefix, chunk, seed=11)
    on_tree, exp_t = run_prefilled(device, prefix, chunk, seed=11, tree_parents=parents,
                                   causal_on_tree_step=True)
    tree_out, _ = run_prefilled(device, prefix, chunk, seed=11, tree_parents=parents)
    assert max_err(plain, exp) <= TOL
    assert max_err(on_tree, exp_t) <= TOL
    assert max_err(tree_out, exp) <= TOL
    assert max_err(plain, on_tree) <= 1e-3


def test_tree_verify_append_then_rollback(device):
    """Config-5 flow at reduced size: append 9 tree rows (RoPE at len+depth),
    verify, accept a root-to-node path, compact it and roll back the rest in
    every layer."""
    rng = np.random.default_rng(17)
    B = 6
    lengths = [int(x) for x in rng.integers(300, 5000, B)]
    n_layers = 2
    ids = _ids(rng, [(L + 9 + 15) // 16 for L in lengths])
    say("tree verify + rollback")
    cache, kr, vr = build_cache(lengths, ids, extra_rows=9, n_layers=n_layers, rng=rng)
    tables = Tables(device, 6000)
    # RoPE positions len + depth, from the oracle's depths (the kernel input
    # and the expectation alike; the product's own depths are checked in
    # test_gpu_speculative against these).
    depth = orc.tree_depths(C5_PARENTS).tolist()
    rope_pos = [L + d for L in lengths for d in depth]
    T = 9 * B
    outs, qns, kns, vs = [], [], [], []
    cache.begin_step(list(range(B)), [9] * B, rope_pos=rope_pos, tree_bits=tr.tree_bits(C5_PARENTS) * B)
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
        outs.append(out)
        qns.append(expected_norm(q, qw, tables, rope_pos))
        kns.append(expected_norm(k, kw, tables, rope_pos))
        vs.append(v)
    device.synchronize()
    for layer in range(n_layers):
        got = outs[layer].numpy()
        for b in range(B):
            s = slice(9 * b, 9 * b + 9)
            exp = orc.tree_attention(qns[layer][s], kr[layer][b], vr[layer][b], kns[layer][s],
                                     vs[layer][s], C5_PARENTS)
            assert max_err(got[s], exp) <= TOL, (layer, b)
    # Accept a different root-to-node path per sequence.
    accepted = [tr.root_to_node_path(C5_PARENTS, node) for node in (0, 1, 4, 7, 8, 6)]
    cache.rollback(list(range(B)), lengths, accepted)
    device.synchronize()
    for b in range(B):
        assert cache.seq_len(b) == lengths[b] + len(accepted[b])
        for layer in range(n_layers):
            krow, vrow = cache.gather(layer, b, lengths[b] + 9)
            L = lengths[b]
            assert np.array_equal(krow[:L].view(np.uint16), kr[layer][b].view(np.uint16))
            exp_k, _ = orc.rollback_rows(np.concatenate([kr[layer][b], kns[layer][9 * b:9 * b + 9]]), L,
                                         accepted[b])
            exp_v, _ = orc.rollback_rows(np.concatenate([vr[layer][b], vs[layer][9 * b:9 * b + 9]]), L,
                                         accepted[b])
            n = L + len(accepted[b])
            assert np.array_equal(krow[:n].view(np.uint16), exp_k[:n].view(np.uint16)), (b, layer)
            assert np.array_equal(vrow[:n].view(np.uint16), exp_v[:n].view(np.uint16)), (b, layer)
    cache.destroy()
