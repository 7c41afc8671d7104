"""GPU: the attention output gate fused into decode (kva_decode_gated,
kva_legacy_decode_gated) against sigmoid_mul.hip:10-22 applied after the
ungated decode, as the engine does (engine.py:2047-2056).

The gate is read from the Q_gate half of a fused [Q | Q_gate] buffer
(engine.py:1069-1071), so its row stride is twice the query row.  The fused
result must equal the oracle gate applied to the ungated GPU output within
one fp16 ulp (exp in float32 may round differently), and the gated
attention stays within 2e-3 of fp32 attention followed by the gate.
"""
import numpy as np
import pytest

from mi50grad_amd import _lib
from mi50grad_amd.kv_cache import PagedKVCache
from oracle import kvattn_oracle as orc

from gpu_helpers import HKV, H, D, Tables, build_cache, expected_norm, max_err, say

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _ordered(x):
    """fp16 bit patterns mapped to integers in value order: +0 and -0 both
    map to 0 and neighbouring values differ by one."""
    bits = np.asarray(x, np.float16).view(np.uint16).astype(np.int32)
    return np.where(bits & 0x8000, -(bits & 0x7FFF), bits)


def ulps(a, b):
    """fp16 ulp distance per element (finite values; -0 equals +0)."""
    return np.abs(_ordered(a) - _ordered(b))


@pytest.mark.parametrize("split,lengths", [(0, [1, 15, 16, 300, 2047]), (64, [1, 15, 16, 300, 2047]),
                                           (0, [1, 15, 16, 300, 511])])
def test_decode_gated_paged(device, split, lengths):
    """Stream-K (the first two cases) and the whole-sequence form (the last:
    every sequence at most 1024 rows at the automatic split)."""
    rng = np.random.default_rng(21 + split + (0 if lengths[-1] == 2047 else 1000))
    nblk = [(L + 1 + 15) // 16 for L in lengths]
    perm = rng.permutation(sum(nblk))
    ids, o = [], 0
    for n in nblk:
        ids.append([int(x) for x in perm[o:o + n]])
        o += n
    say(f"decode gated split={split} longest={lengths[-1]}")
    cache, kr, vr = build_cache(lengths, ids, extra_rows=1, rng=rng)
    cache.set_decode_split(split)
    tables = Tables(device, 4096)
    B = len(lengths)
    q = rng.standard_normal((B, H, D), dtype=np.float32).astype(np.float16)
    k = rng.standard_normal((B, HKV, D), dtype=np.float32).astype(np.float16)
    v = rng.standard_normal((B, HKV, D), dtype=np.float32).astype(np.float16)
    gate = (2 * rng.standard_normal((B, H, D), dtype=np.float32)).astype(np.float16)
    fused = np.concatenate([q.reshape(B, -1), gate.reshape(B, -1)], axis=1)  # [B, Q | Q_gate]
    qw = (1 + 0.02 * rng.standard_normal(D, dtype=np.float32)).astype(np.float16)
    kw = (1 + 0.02 * rng.standard_normal(D, dtype=np.float32)).astype(np.float16)
    dq, dk, dv = device.array(q), device.array(k), device.array(v)
    dfused = device.array(fused)
    plain, gated = device.empty((B, H, D), np.float16), device.empty((B, H, D), np.float16)
    cache.begin_step(list(range(B)), [1] * B)
    cache.append(0, dq, dk, dv, device.array(qw), device.array(kw), tables.d_cos, tables.d_sin, tables.rows)
    cache.decode(0, dq, plain)
    cache.decode(0, dq, gated, gate=dfused.ptr + H * D * 2, gate_stride=2 * H * D)
    device.synchronize()
    p, g = plain.numpy(), gated.numpy()
    assert ulps(g, orc.sigmoid_gate(p, gate)).max() <= 1
    pos = np.asarray(lengths)
    qn, kn = expected_norm(q, qw, tables, pos), expected_norm(k, kw, tables, pos)
    ks = [np.concatenate([kr[0][b], kn[b:b + 1]]) for b in range(B)]
    vs = [np.concatenate([vr[0][b], v[b:b + 1]]) for b in range(B)]
    ref = orc.sigmoid_gate(orc.decode_attention(qn, ks, vs).astype(np.float16), gate)
    assert max_err(g, ref) <= TOL
    cache.destroy()


def test_legacy_decode_gated(device):
    rng = np.random.default_rng(31)
    L = 700
    Q = rng.standard_normal((1, H, D), dtype=np.float32).astype(np.float16)
    Gt = (2 * rng.standard_normal((1, H, D), dtype=np.float32)).astype(np.float16)
    K = rng.standard_normal((L, HKV, D), dtype=np.float32).astype(np.float16)
    V = rng.standard_normal((L, HKV, D), dtype=np.float32).astype(np.float16)
    say("legacy decode gated")
    dq, dg, dk, dv = device.array(Q), device.array(Gt), device.array(K), device.array(V)
    plain, gated = device.empty((1, H, D), np.float16), device.empty((1, H, D), np.float16)
    ws = PagedKVCache(n_layers=1, max_seqs=1, max_blocks=1, max_blocks_per_seq=1, max_step_tokens=16)
    _lib.call("kva_legacy_decode", ws.handle, dq.ptr, dk.ptr, dv.ptr, plain.ptr, L, H, HKV, None)
    _lib.call("kva_legacy_decode_gated", ws.handle, dq.ptr, dg.ptr, dk.ptr, dv.ptr, gated.ptr, L, H, HKV, None)
    device.synchronize()
    ws.destroy()
    assert ulps(gated.numpy(), orc.sigmoid_gate(plain.numpy(), Gt)).max() <= 1
    ref = orc.sigmoid_gate(orc.attention_fp32(Q, K, V).astype(np.float16), Gt)
    assert max_err(gated.numpy(), ref) <= TOL


def _prefilled(rng, prefix, chunk):
    """A cache whose sequence b holds prefix[b] + chunk[b] random rows (pages
    permuted), its length set to prefix[b]: the chunk's keys are in place."""
    total = [p + c for p, c in zip(prefix, chunk)]
    nblk = [(t + 15) // 16 for t in total]
    perm = rng.permutation(sum(nblk))
    ids, o = [], 0
    for n in nblk:
        ids.append([int(x) for x in perm[o:o + n]])
        o += n
    cache, kr, vr = build_cache(total, ids, extra_rows=0, rng=rng)
    for b, p in enumerate(prefix):
        cache.set_len(b, p)
    return cache, kr[0], vr[0]


@pytest.mark.parametrize("tree", [False, True])
def test_multi_query_gated(device, tree):
    """kva_prefill_gated on config 4's shape (512-token chunks after 0/256/
    1024/2048 cached rows) and kva_tree_verify_gated (config 5's tree over
    ragged caches), the gate read from the Q_gate half of a fused
    [Q | Q_gate] buffer: the gate is applied in the epilogue of whole units
    and of units merged by the combine alike, so the result equals
    sigmoid_mul (engine.py:3120-3121) applied to the ungated output within
    one ulp, and the oracle's attention followed by the gate within 2e-3."""
    from mi50grad_amd import tree as tr
    from mi50grad_amd.workloads import C4_CHUNK, C4_PREFIX, C5_PARENTS
    rng = np.random.default_rng(90 + tree)
    if tree:
        prefix = [int(x) for x in rng.integers(300, 5000, 6)]
        chunk = [len(C5_PARENTS)] * 6
    else:
        prefix, chunk = list(C4_PREFIX), [C4_CHUNK] * 4
    say(f"multi-query gated tree={tree}")
    cache, kr, vr = _prefilled(rng, prefix, chunk)
    B, T = len(prefix), sum(chunk)
    q = rng.standard_normal((T, H, D), dtype=np.float32).astype(np.float16)
    gate = (2 * rng.standard_normal((T, H, D), dtype=np.float32)).astype(np.float16)
    fused = device.array(np.concatenate([q.reshape(T, -1), gate.reshape(T, -1)], axis=1))
    dq = device.array(q)
    plain, gated = device.empty((T, H, D), np.float16), device.empty((T, H, D), np.float16)
    bits = tr.tree_bits(C5_PARENTS) * B if tree else None
    cache.begin_step(list(range(B)), chunk, tree_bits=bits)
    run = cache.tree_verify if tree else cache.prefill
    run(0, dq, plain)
    run(0, dq, gated, gate=fused.ptr + H * D * 2, gate_stride=2 * H * D)
    device.synchronize()
    p, g = plain.numpy(), gated.numpy()
    assert ulps(g, orc.sigmoid_gate(p, gate)).max() <= 1
    t = 0
    for b in range(B):
        s = slice(t, t + chunk[b])
        if tree:
            P = prefix[b]
            att = orc.tree_attention(q[s], kr[b][:P], vr[b][:P], kr[b][P:], vr[b][P:], C5_PARENTS)
        else:
            att = orc.chunk_attention(q[s], kr[b], vr[b], prefix[b])
        assert max_err(g[s], orc.sigmoid_gate(att.astype(np.float16), gate[s])) <= TOL, b
        t += chunk[b]
    cache.destroy()
