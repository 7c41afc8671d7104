"""GPU parity: fused QK-norm + RoPE + K/V append is bit-exact against the oracle.

Checks the in-place q/k results, the K and V rows written into the paged
pool (permuted block tables, ragged lengths, several tokens per sequence,
RoPE positions decoupled from slots), and that no other byte of any pool
changed (canary).  The reference-compatible contiguous entry point is
checked the same way, plus against the reference test's recipe
(tests/test_qknorm_rope.py:55-114, tolerance 2e-3).
"""
import numpy as np
import pytest

from mi50grad_amd import _lib
from mi50grad_amd.workloads import c1_inputs
from oracle import kvattn_oracle as orc

from gpu_helpers import HKV, H, D, Tables, build_cache, expected_norm, say

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint16)


@pytest.mark.parametrize("rope_override,many", [(False, False), (True, False), (False, True), (True, True)])
def test_append_bitexact_with_canary(device, rope_override, many):
    """42 tokens, or (many) 306 tokens over 20 permuted blocks of four
    sequences, with RoPE positions from the slots or overridden."""
    rng = np.random.default_rng(21)
    if many:
        lengths, n_new = [0, 37, 250, 16], [1, 5, 200, 100]
        nblk = [(L + n + 15) // 16 for L, n in zip(lengths, n_new)]
        perm = [int(x) for x in rng.permutation(sum(nblk) + 3)]
        ids, o = [], 0
        for n in nblk:
            ids.append(perm[o:o + n])
            o += n
        max_blocks = sum(nblk) + 3
    else:
        lengths = [0, 37, 250, 16]
        n_new = [1, 5, 20, 16]
        ids = [[9, 2], [4, 11, 0], [13, 7, 1, 15, 5, 12, 3, 8, 10, 14, 6, 16, 17, 18, 19, 20, 21],
               [22, 23]]
        max_blocks = 24
    say(f"append canary rope_override={rope_override} many={many}")
    cache, _, _ = build_cache(lengths, ids, extra_rows=n_new, n_layers=2, rng=rng, max_blocks=max_blocks)
    tables = Tables(device, 1024)
    T = sum(n_new)
    q = rng.standard_normal((T, H, D), dtype=np.float32).astype(np.float16)
    k = rng.standard_normal((T, HKV, D), dtype=np.float32).astype(np.float16)
    v = rng.standard_normal((T, HKV, D), dtype=np.float32).astype(np.float16)
    qw = (1 + 0.02 * rng.standard_normal(D, dtype=np.float32)).astype(np.float16)
    kw = (1 + 0.02 * rng.standard_normal(D, dtype=np.float32)).astype(np.float16)
    slots = np.concatenate([np.arange(L, L + n) for L, n in zip(lengths, n_new)])
    pos = rng.integers(0, 1024, T) if rope_override else slots
    before = [cache.download_pools(layer) for layer in range(2)]
    dq, dk, dv = device.array(q), device.array(k), device.array(v)
    dqw, dkw = device.array(qw), device.array(kw)
    cache.begin_step([0, 1, 2, 3], n_new, rope_pos=pos if rope_override else None)
    cache.append(1, dq, dk, dv, dqw, dkw, tables.d_cos, tables.d_sin, tables.rows)
    device.synchronize()
    exp_q = expected_norm(q, qw, tables, pos)
    exp_k = expected_norm(k, kw, tables, pos)
    assert np.array_equal(_bits(dq.numpy()), _bits(exp_q))
    assert np.array_equal(_bits(dk.numpy()), _bits(exp_k))
    # Layer 0 untouched, layer 1 changed exactly at the new rows.
    after0 = cache.download_pools(0)
    assert all(np.array_equal(_bits(a), _bits(b)) for a, b in zip(before[0], after0))
    kpool, vpool = cache.download_pools(1)
    kexp, vexp = before[1][0].copy(), before[1][1].copy()
    t = 0
    for b, (L, n) in enumerate(zip(lengths, n_new)):
        for i in range(n):
            s = L + i
            blk = ids[b][s // 16]
            kexp[blk, s % 16] = exp_k[t]
            vexp[blk, s % 16] = v[t]
            t += 1
    assert np.array_equal(_bits(kpool), _bits(kexp))
    assert np.array_equal(_bits(vpool), _bits(vexp))
    assert [cache.seq_len(b) for b in range(4)] == [L + n for L, n in zip(lengths, n_new)]
    cache.destroy()


def test_append_c1_golden(device):
    """Config 1 inputs (seed 0): q and the appended K row match the fixture."""
    from pathlib import Path

    fx = np.load(Path(__file__).resolve().parent / "golden" / "c1_golden.npz")
    c1 = c1_inputs(0)
    assert np.array_equal(_bits(c1.q), _bits(fx["q"]))
    say("append c1 golden")
    cache, _, _ = build_cache([255], [list(range(16))], extra_rows=1, rng=np.random.default_rng(0))
    tables = Tables(device, 256)
    dq, dk, dv = device.array(c1.q), device.array(c1.k_new), device.array(c1.v_new)
    cache.begin_step([0], [1])
    cache.append(0, dq, dk, dv, device.array(c1.q_norm), device.array(c1.k_norm), tables.d_cos,
                 tables.d_sin, tables.rows)
    device.synchronize()
    assert np.array_equal(_bits(dq.numpy()[0]), _bits(fx["q_normed"]))
    krow, vrow = cache.gather(0, 0, 256)
    assert np.array_equal(_bits(krow[255]), _bits(fx["k_normed"]))
    assert np.array_equal(_bits(vrow[255]), _bits(c1.v_new[0]))
    cache.destroy()


@pytest.mark.parametrize("heads,head_dim,half", [(24, 256, 32), (4, 256, 32), (1, 256, 32),
                                                 (48, 256, 32), (8, 128, 32), (3, 64, 16),
                                                 (5, 256, 0)])
def test_legacy_qknorm_bitexact(device, heads, head_dim, half):
    rng = np.random.default_rng(heads * 7 + head_dim)
    x = (rng.standard_normal((heads, head_dim)) * 3).astype(np.float16)
    w = (1 + 0.05 * rng.standard_normal(head_dim)).astype(np.float16)
    rows = max(half, 1)
    c = np.cos(np.arange(rows, dtype=np.float32) * 0.37).astype(np.float16)
    s = np.sin(np.arange(rows, dtype=np.float32) * 0.37).astype(np.float16)
    say(f"legacy qknorm heads={heads} head_dim={head_dim} half={half}")
    dx, dw, dc, ds = device.array(x), device.array(w), device.array(c), device.array(s)
    dst = device.array(np.zeros_like(x))
    _lib.call("kva_legacy_qknorm_rope", dx.ptr, dw.ptr, dc.ptr, ds.ptr, dst.ptr, heads, head_dim,
              half, 1e-6, None)
    device.synchronize()
    exp = orc.qknorm_rope_exact(x, w, np.tile(c[:half], (heads, 1)), np.tile(s[:half], (heads, 1)))
    assert np.array_equal(_bits(dx.numpy()), _bits(exp))
    assert np.array_equal(_bits(dst.numpy()), _bits(exp))


def test_legacy_qknorm_reference_recipe(device):
    """tests/test_qknorm_rope.py:106-114 inputs; the reference's bar is 2e-3."""
    for heads, hd in [(8, 256), (1, 256), (48, 256), (8, 128)]:
        np.random.seed(42)
        x = (np.random.randn(heads, hd) * 0.3).astype(np.float16)
        w = (np.random.rand(hd) * 0.5 + 0.5).astype(np.float16)
        c = np.cos(np.arange(32, dtype=np.float32) * 0.1).astype(np.float16)
        s = np.sin(np.arange(32, dtype=np.float32) * 0.1).astype(np.float16)
        say(f"legacy qknorm reference recipe heads={heads} hd={hd}")
        dx, dw, dc, ds = device.array(x), device.array(w), device.array(c), device.array(s)
        _lib.call("kva_legacy_qknorm_rope", dx.ptr, dw.ptr, dc.ptr, ds.ptr, None, heads, hd, 32,
                  1e-6, None)
        device.synchronize()
        ref = orc.qknorm_rope_float(x, w, np.tile(c, (heads, 1)), np.tile(s, (heads, 1)))
        assert np.max(np.abs(dx.numpy().astype(np.float32) - ref.astype(np.float32))) < 2e-3
