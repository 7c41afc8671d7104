"""GPU parity at the full sizes of configs 2 and 5, against the oracle.

Config 5 (long-context tree verify): 64 sequences with cached rows
U[4096, 32768] (``workloads.c5_spec(0)``: lengths, permuted pages), one
layer.  The 9-node tree of the config is appended with norm + RoPE at
len + depth (depths from the oracle), tree verify runs over the whole
cache, every sequence's output is compared with ``orc.tree_attention`` at
2e-3, the appended rows must be bit-exact, then a seeded root-to-node path
per sequence is kept (compacted) and the rest rolled back.  Cache rows are
N(0,1) fp16 drawn once into a 32768-row bank; each sequence takes a seeded
permutation of it, so the host holds the bank plus one pool image.

Config 2 (16 stacked layers, batch 1, 128 decode steps from a 128-row cache
to 256 rows): every step appends one row per layer (norm + RoPE at the
row's slot) and decodes; every layer's output of every step is compared
with ``orc.attention_fp32`` over the oracle's own copy of the rows.  The
same inputs run twice, eagerly and as one recorded step replayed 127 times
(the reference's graph replay, c_graph_dispatch.c:392-414); both must match
the oracle, and the replay must equal the eager run bit for bit, outputs
and cache rows alike.
"""
import numpy as np
import pytest

from mi50grad_amd import _lib
from mi50grad_amd import tree as tr
from mi50grad_amd import workloads as wl
from mi50grad_amd.device import Stream
from mi50grad_amd.kv_cache import PagedKVCache
from oracle import kvattn_oracle as orc

from gpu_helpers import HKV, H, D, Tables, build_cache, expected_norm, max_err, say

pytestmark = pytest.mark.gpu
TOL = 2e-3
BANK = 32768


def _f16(rng, shape):
    return rng.standard_normal(shape, dtype=np.float32).astype(np.float16)


def _path(parents, node):
    return orc.tree_ancestors(parents, node) + [node]


def test_c5_workload_tree_verify_and_rollback(device):
    spec = wl.c5_spec(0)
    lengths = [int(x) for x in spec.lengths]
    B = len(lengths)
    par = wl.C5_PARENTS
    T = len(par)
    say(f"config 5 full: B={B} ctx {min(lengths)}..{max(lengths)} pages={spec.n_blocks}")
    rng = np.random.default_rng(55)
    bank_k, bank_v = _f16(rng, (BANK, HKV, D)), _f16(rng, (BANK, HKV, D))
    picks = [rng.permutation(BANK)[:L] for L in lengths]
    cache = PagedKVCache(n_layers=1, max_seqs=B, max_blocks=spec.n_blocks,
                         max_blocks_per_seq=max(len(ids) for ids in spec.block_ids),
                         max_step_tokens=B * T)
    for b, ids in enumerate(spec.block_ids):
        cache.set_blocks(b, ids)
    for pool, bank in zip(cache.layer_pools(0), (bank_k, bank_v)):
        img = np.zeros((spec.n_blocks, 16, HKV, D), np.float16)
        for b, ids in enumerate(spec.block_ids):
            slots = np.arange(lengths[b])
            img[np.asarray(ids)[slots // 16], slots % 16] = bank[picks[b]]
        _lib.call("kva_memcpy_h2d", pool, img.ctypes.data, img.nbytes)
        del img
    for b, L in enumerate(lengths):
        cache.set_len(b, L)
    cache.sync_tables()

    depth = orc.tree_depths(par).tolist()
    rope_pos = [L + d for L in lengths for d in depth]
    tables = Tables(device, max(rope_pos) + 1)
    bits = tr.tree_bits(par)
    assert bits == [int(x) for x in orc.tree_row_bits(par)]
    q, k, v = _f16(rng, (B * T, H, D)), _f16(rng, (B * T, HKV, D)), _f16(rng, (B * T, HKV, D))
    qw, kw = wl.norm_weight(rng), wl.norm_weight(rng)
    dq, out = device.array(q), device.empty((B * T, H, D), np.float16)
    cache.begin_step(list(range(B)), [T] * B, rope_pos=rope_pos, tree_bits=bits * B)
    cache.append(0, dq, device.array(k), device.array(v), device.array(qw), device.array(kw),
                 tables.d_cos, tables.d_sin, tables.rows)
    cache.tree_verify(0, dq, out)
    device.synchronize()
    got = out.numpy()
    qn = expected_norm(q, qw, tables, rope_pos)
    kn = expected_norm(k, kw, tables, rope_pos)
    assert np.array_equal(dq.numpy().view(np.uint16), qn.view(np.uint16))

    def tree_rows(b, n):
        ks = np.empty((n, HKV, D), np.float16)
        vs = np.empty_like(ks)
        for i in range(n):
            kp, vp = cache.row_ptr(0, b, lengths[b] + i)
            _lib.call("kva_memcpy_d2h", ks[i].ctypes.data, kp, ks[i].nbytes)
            _lib.call("kva_memcpy_d2h", vs[i].ctypes.data, vp, vs[i].nbytes)
        return ks, vs

    worst = 0.0
    for b, L in enumerate(lengths):
        s = slice(T * b, T * b + T)
        ks, vs = tree_rows(b, T)
        assert np.array_equal(ks.view(np.uint16), kn[s].view(np.uint16)), b
        assert np.array_equal(vs.view(np.uint16), v[s].view(np.uint16)), b
        exp = orc.tree_attention(qn[s], bank_k[picks[b]], bank_v[picks[b]], kn[s], v[s], par)
        err = max_err(got[s], exp)
        worst = max(worst, err)
        assert err <= TOL, (b, L, err)
    say(f"config 5 tree verify: worst max-abs error {worst:.2e} over {B} sequences")

    # Keep a seeded root-to-node path per sequence, roll back the rest.
    keep = [_path(par, int(n)) for n in rng.integers(0, T, B)]
    cache.rollback(list(range(B)), lengths, keep)
    device.synchronize()
    for b, L in enumerate(lengths):
        assert cache.seq_len(b) == L + len(keep[b])
        s = slice(T * b, T * b + T)
        ks, vs = tree_rows(b, len(keep[b]))
        assert np.array_equal(ks.view(np.uint16), kn[s][keep[b]].view(np.uint16)), b
        assert np.array_equal(vs.view(np.uint16), v[s][keep[b]].view(np.uint16)), b
        kp, vp = cache.row_ptr(0, b, L - 1)  # the last cached row is untouched
        last = np.empty((HKV, D), np.float16)
        _lib.call("kva_memcpy_d2h", last.ctypes.data, kp, last.nbytes)
        assert np.array_equal(last.view(np.uint16), bank_k[picks[b][L - 1]].view(np.uint16)), b
    cache.destroy()


C2_LAYERS, C2_START, C2_STEPS = 16, 128, 128


def test_c2_workload_eager_and_replayed(device):
    """Config 2: 16 layers, batch 1, 128 steps from 128 cached rows to 256."""
    say("config 2 full: 16 layers x 128 steps, eager and recorded-step replay")
    rng = np.random.default_rng(0)
    pages = [int(x) for x in rng.permutation(16)]
    twins = []
    for _ in range(2):
        c, kr, vr = build_cache([C2_START], [pages], extra_rows=C2_STEPS, n_layers=C2_LAYERS,
                                max_step_tokens=16, rng=np.random.default_rng(1))
        twins.append(c)
    k_hist = [list(kr[layer][0]) for layer in range(C2_LAYERS)]
    v_hist = [list(vr[layer][0]) for layer in range(C2_LAYERS)]
    tables = Tables(device, C2_START + C2_STEPS)
    qw = [wl.norm_weight(rng) for _ in range(C2_LAYERS)]
    kw = [wl.norm_weight(rng) for _ in range(C2_LAYERS)]
    d_qw = [device.array(w) for w in qw]
    d_kw = [device.array(w) for w in kw]
    stream = Stream()
    bufs = [[dict(q=device.empty((1, H, D), np.float16), k=device.empty((1, HKV, D), np.float16),
                  v=device.empty((1, HKV, D), np.float16), out=device.empty((1, H, D), np.float16))
             for _ in range(C2_LAYERS)] for _ in range(2)]

    def calls(which, stream_h):
        for layer in range(C2_LAYERS):
            b = bufs[which][layer]
            twins[which].append(layer, b["q"], b["k"], b["v"], d_qw[layer], d_kw[layer], tables.d_cos,
                                tables.d_sin, tables.rows, stream=stream_h)
            twins[which].decode(layer, b["q"], b["out"], stream=stream_h)

    graph = None
    worst = 0.0
    for step in range(C2_STEPS):
        pos = C2_START + step
        ins = [dict(q=_f16(rng, (1, H, D)), k=_f16(rng, (1, HKV, D)), v=_f16(rng, (1, HKV, D)))
               for _ in range(C2_LAYERS)]
        for which in range(2):
            for layer in range(C2_LAYERS):
                for name in ("q", "k", "v"):
                    bufs[which][layer][name].copy_from(ins[layer][name])
        device.synchronize()
        twins[0].begin_step([0], [1])
        calls(0, None)
        twins[1].begin_step([0], [1], stream=stream.handle)
        if graph is None:
            graph = twins[1].record_step(stream.handle)
            calls(1, stream.handle)
            graph.end()
        graph.launch()
        stream.synchronize()
        device.synchronize()
        for layer in range(C2_LAYERS):
            qn = expected_norm(ins[layer]["q"], qw[layer], tables, [pos])
            kn = expected_norm(ins[layer]["k"], kw[layer], tables, [pos])
            k_hist[layer].append(kn[0])
            v_hist[layer].append(ins[layer]["v"][0])
            exp = orc.attention_fp32(qn, np.stack(k_hist[layer]), np.stack(v_hist[layer]))
            eager = bufs[0][layer]["out"].numpy()
            replay = bufs[1][layer]["out"].numpy()
            assert np.array_equal(bufs[0][layer]["q"].numpy().view(np.uint16), qn.view(np.uint16)), (step, layer)
            err = max_err(eager, exp)
            worst = max(worst, err)
            assert err <= TOL, (step, layer, err)
            assert max_err(replay, exp) <= TOL, (step, layer)
            assert np.array_equal(replay.view(np.uint16), eager.view(np.uint16)), (step, layer)
    say(f"config 2: worst max-abs error {worst:.2e} over {C2_STEPS} steps x {C2_LAYERS} layers")
    n = C2_START + C2_STEPS
    for which in range(2):
        assert twins[which].seq_len(0) == n
        for layer in range(C2_LAYERS):
            ks, vs = twins[which].gather(layer, 0, n)
            assert np.array_equal(ks.view(np.uint16), np.stack(k_hist[layer]).view(np.uint16)), (which, layer)
            assert np.array_equal(vs.view(np.uint16), np.stack(v_hist[layer]).view(np.uint16)), (which, layer)
    graph.destroy()
    stream.synchronize()
    stream.destroy()
    for c in twins:
        c.destroy()
