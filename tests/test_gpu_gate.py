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
from oracle import kvattn_oracle as orc

from gpu_helpers import HKV, H, D, Tables, build_cache, expected_norm, max_err, say

pytestmark = pytest.mark.gpu
TOL = 2e-3


def ulps(a, b):
    """fp16 ulp distance per element (same-sign finite values)."""
    ai = np.asarray(a, np.float16).view(np.int16).astype(np.int32)
    bi = np.asarray(b, np.float16).view(np.int16).astype(np.int32)
    return np.abs(ai - bi)


@pytest.mark.parametrize("split", [0, 64])
def test_decode_gated_paged(device, split):
    rng = np.random.default_rng(21 + split)
    lengths = [1, 15, 16, 300, 2047]
    nblk = [(L + 1 + 15) // 16 for L in lengths]
    perm = rng.permutation(sum(nblk))
    ids, o = [], 0
    for n in nblk:
        ids.append([int(x) for x in perm[o:o + n]])
        o += n
    say(f"decode gated split={split}")
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
    _lib.call("kva_legacy_decode", None, dq.ptr, dk.ptr, dv.ptr, plain.ptr, L, H, HKV, None)
    _lib.call("kva_legacy_decode_gated", None, dq.ptr, dg.ptr, dk.ptr, dv.ptr, gated.ptr, L, H, HKV, None)
    device.synchronize()
    assert ulps(gated.numpy(), orc.sigmoid_gate(plain.numpy(), Gt)).max() <= 1
    ref = orc.sigmoid_gate(orc.attention_fp32(Q, K, V).astype(np.float16), Gt)
    assert max_err(gated.numpy(), ref) <= TOL
