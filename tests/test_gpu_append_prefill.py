"""GPU: kva_append_prefill, the append and the causal prefill in one call
(two launches on the caller's stream).

Against the two calls it replaces (kva_append_qknorm_rope, then
kva_prefill / kva_prefill_gated) on twin caches built from one seed: the
output bit-identical, every cache row bit-identical, q normalised in place
to the same bits, k untouched (only read).  Cases: the config-4 workload
(eight-wave tiles of 64-key blocks; also against the oracle within 2e-3),
small steps (four-wave tiles, 32-key blocks), GQA groups 1, 4 and 8, RoPE
positions other than the slots, and the gated form.
"""
import numpy as np
import pytest

from mi50grad_amd.workloads import C4_CHUNK, C4_PREFIX
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


def _twin(device, prefix, chunk, heads=H, kv=HKV, seed=0, gated=False, pos_shift=0):
    rng = np.random.default_rng(seed)
    B, T = len(prefix), sum(chunk)
    ids = _ids(rng, [(p + c + 15) // 16 for p, c in zip(prefix, chunk)])
    caches = []
    for _ in range(2):
        c, kr, vr = build_cache(prefix, ids, extra_rows=chunk, num_heads=heads, num_kv_heads=kv,
                                rng=np.random.default_rng(seed + 1))
        caches.append(c)
    two, fused = caches
    tables = Tables(device, 4096)
    q = rng.standard_normal((T, heads, D), dtype=np.float32).astype(np.float16)
    k = rng.standard_normal((T, kv, D), dtype=np.float32).astype(np.float16)
    v = rng.standard_normal((T, kv, D), dtype=np.float32).astype(np.float16)
    qw = (1 + 0.02 * rng.standard_normal(D, dtype=np.float32)).astype(np.float16)
    kw = (1 + 0.02 * rng.standard_normal(D, dtype=np.float32)).astype(np.float16)
    gate = rng.standard_normal((T, heads, D), dtype=np.float32).astype(np.float16) if gated else None
    dv, dqw, dkw = device.array(v), device.array(qw), device.array(kw)
    dgate = device.array(gate) if gated else None
    pos = np.concatenate([np.arange(p, p + c) for p, c in zip(prefix, chunk)]) + pos_shift
    rope_pos = [int(x) for x in pos] if pos_shift else None
    outs = []
    # The two calls: append (q and k normalised in place), then prefill.
    dq, dk, out = device.array(q), device.array(k), device.empty((T, heads, D), np.float16)
    two.begin_step(list(range(B)), chunk, rope_pos=rope_pos)
    two.append(0, dq, dk, dv, dqw, dkw, tables.d_cos, tables.d_sin, tables.rows)
    two.prefill(0, dq, out, gate=dgate)
    outs.append(out)
    # The one call on the same raw rows.
    fq, fk, fout = device.array(q), device.array(k), device.empty((T, heads, D), np.float16)
    fused.begin_step(list(range(B)), chunk, rope_pos=rope_pos)
    fused.append_prefill(0, fq, fk, dv, dqw, dkw, tables.d_cos, tables.d_sin, tables.rows, fout, gate=dgate)
    outs.append(fout)
    device.synchronize()
    got_two, got = outs[0].numpy(), outs[1].numpy()
    assert np.array_equal(got.view(np.uint16), got_two.view(np.uint16))
    assert np.array_equal(fq.numpy().view(np.uint16), dq.numpy().view(np.uint16)), "q normalised in place"
    assert np.array_equal(fk.numpy().view(np.uint16), k.view(np.uint16)), "k must be only read"
    kt, vt = two.download_pools(0)
    kf, vf = fused.download_pools(0)
    assert np.array_equal(kt.view(np.uint16), kf.view(np.uint16))
    assert np.array_equal(vt.view(np.uint16), vf.view(np.uint16))
    two.destroy()
    fused.destroy()
    return got, dict(q=q, k=k, v=v, qw=qw, kw=kw, kr=kr, vr=vr, tables=tables, pos=pos)


def test_append_prefill_c4_workload(device):
    """Config 4 through the fused call: equal to append + prefill bit for
    bit, and within 2e-3 of the oracle's chunk attention on the normalised
    rows."""
    prefix, chunk = list(C4_PREFIX), [C4_CHUNK] * 4
    say("append_prefill c4 workload")
    got, d = _twin(device, prefix, chunk, seed=0)
    qn = expected_norm(d["q"], d["qw"], d["tables"], d["pos"])
    kn = expected_norm(d["k"], d["kw"], d["tables"], d["pos"])
    t = 0
    for b, (P, n) in enumerate(zip(prefix, chunk)):
        kall = np.concatenate([d["kr"][0][b], kn[t:t + n]])
        vall = np.concatenate([d["vr"][0][b], d["v"][t:t + n]])
        exp = orc.chunk_attention(qn[t:t + n], kall, vall, P)
        assert max_err(got[t:t + n], exp) <= TOL, b
        t += n


@pytest.mark.parametrize("prefix,chunk", [([100, 7], [9, 5]), ([0], [1]), ([31, 0, 500], [40, 64, 3]),
                                          ([0, 1000], [300, 31])])
def test_append_prefill_shapes(device, prefix, chunk):
    """Four- and eight-wave tiles, 32- and 64-key blocks, one-token and
    ragged chunks."""
    say(f"append_prefill prefix={prefix} chunk={chunk}")
    _twin(device, prefix, chunk, seed=sum(prefix) + 3 * sum(chunk))


@pytest.mark.parametrize("heads,kv", [(8, 8), (8, 2), (16, 2)])
def test_append_prefill_groups(device, heads, kv):
    say(f"append_prefill heads={heads} kv={kv}")
    _twin(device, [37, 0, 130], [70, 9, 140], heads=heads, kv=kv, seed=heads + kv)


def test_append_prefill_gated_and_positions(device):
    """The gated form, with RoPE positions 700 past the slots."""
    say("append_prefill gated, shifted positions")
    _twin(device, [20, 300], [130, 77], seed=5, gated=True, pos_shift=700)
