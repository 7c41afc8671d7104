"""GPU: kva_project_append, the Q/K/V projection fused with norm + RoPE +
append, against the oracle's producer (oracle.project_append).

* Integer inputs whose partial sums are exact in fp32: every output is
  bit-exact (projected Q_gate, K, V; normed + rotated Q; the K and V cache
  rows), whatever the summation order.
* Random N(0,1) inputs: each projected value within one fp16 ulp plus the
  fp32 accumulation error of the correctly rounded sum (fp32 accumulation,
  gemv_fp16_v2.hip:22-85); the
  cache's K row is bit-exactly the norm + RoPE of the projected K and its V
  row the projected V; decode over the result within 2e-3 of fp32.
* Chunking (steps of more than 64 tokens), the hidden sizes that select 1, 2
  and 4 splits, one-token steps, and the validation errors.
* Prefill-sized steps (more than 64 tokens) go through the prefill GEMM
  (tiles of 256 tokens x one head, the norm/RoPE/append epilogue fused): the
  same contract (bit-exact on exact inputs, within one ulp plus the
  accumulation term on random ones) at 70-300 tokens and at 1024 tokens of
  hidden 5120 (two config-4 sequences), and the path taken is reported.
"""
import numpy as np
import pytest

from oracle import kvattn_oracle as orc

from gpu_helpers import HKV, H, D, Tables, build_cache, max_err, say

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _ids(rng, nblk):
    perm = rng.permutation(sum(nblk))
    ids, o = [], 0
    for n in nblk:
        ids.append([int(x) for x in perm[o:o + n]])
        o += n
    return ids


def _weights(rng, hidden, exact):
    nq, nkv = 2 * H * D, 2 * HKV * D
    if exact:
        wq = (rng.integers(-2, 3, (nq, hidden), dtype=np.int8) * 2.0 ** -7).astype(np.float16)
        wkv = (rng.integers(-2, 3, (nkv, hidden), dtype=np.int8) * 2.0 ** -7).astype(np.float16)
    else:
        s = np.float32(1 / np.sqrt(hidden))
        wq = (rng.standard_normal((nq, hidden), dtype=np.float32) * s).astype(np.float16)
        wkv = (rng.standard_normal((nkv, hidden), dtype=np.float32) * s).astype(np.float16)
    qw = (1 + 0.02 * rng.standard_normal(D, dtype=np.float32)).astype(np.float16)
    kw = (1 + 0.02 * rng.standard_normal(D, dtype=np.float32)).astype(np.float16)
    return wq, wkv, qw, kw


def _ulp(x):
    """fp16 spacing at |x| (subnormal spacing below the normal range)."""
    a = np.abs(np.asarray(x, np.float32))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
    return (2.0 ** (e - 10)).astype(np.float32)


def _run(device, rng, lengths, n_new, hidden, exact, tables):
    """One step through kva_project_append; returns everything to check."""
    B = len(lengths)
    T = int(sum(n_new))
    ids = _ids(rng, [(L + n + 15) // 16 for L, n in zip(lengths, n_new)])
    cache, kr, vr = build_cache(lengths, ids, extra_rows=list(n_new), rng=rng)
    wq, wkv, qw, kw = _weights(rng, hidden, exact)
    if exact:
        x = rng.integers(-3, 4, (T, hidden), dtype=np.int8).astype(np.float16)
    else:
        x = rng.standard_normal((T, hidden), dtype=np.float32).astype(np.float16)
    pos = [L + i for L, n in zip(lengths, n_new) for i in range(n)]
    cache.begin_step(list(range(B)), list(n_new))
    d = dict(q=device.empty((T, H, D), np.float16), g=device.empty((T, H, D), np.float16),
             kv=device.empty((T, 2, HKV, D), np.float16))
    cache.project_append(0, device.array(x), hidden, device.array(wq), device.array(wkv), device.array(qw),
                         device.array(kw), tables.d_cos, tables.d_sin, tables.rows, d["q"], d["g"], d["kv"])
    device.synchronize()
    exp = orc.project_append(x, wq, wkv, qw, kw, tables.cos[pos], tables.sin[pos])
    got = {k: v.numpy() for k, v in d.items()}
    return cache, kr, vr, exp, got, pos, qw, kw, tables


def _check_cache_rows(cache, kr, vr, lengths, n_new, k_new, v_new):
    """Old rows untouched; new rows equal k_new / v_new bit for bit."""
    o = 0
    for b, (L, n) in enumerate(zip(lengths, n_new)):
        krow, vrow = cache.gather(0, b, L + n)
        assert np.array_equal(krow[:L].view(np.uint16), kr[0][b].view(np.uint16)), b
        assert np.array_equal(vrow[:L].view(np.uint16), vr[0][b].view(np.uint16)), b
        assert np.array_equal(krow[L:].view(np.uint16), k_new[o:o + n].view(np.uint16)), b
        assert np.array_equal(vrow[L:].view(np.uint16), v_new[o:o + n].view(np.uint16)), b
        o += n


def test_project_exact_decode_step(device):
    """C3-shaped decode step (32 sequences, one token each, hidden 5120)
    with fp32-exact sums: every output bit-exact."""
    rng = np.random.default_rng(31)
    lengths = [int(x) for x in rng.integers(100, 1500, 32)]
    n_new = [1] * 32
    say("project_append exact, B=32, hidden 5120")
    tables = Tables(device, 2048)
    cache, kr, vr, exp, got, pos, qw, kw, _ = _run(device, rng, lengths, n_new, 5120, True, tables)
    q, gate, k_raw, k, v = exp
    assert np.array_equal(got["kv"][:, 0].view(np.uint16), k_raw.view(np.uint16))
    assert np.array_equal(got["kv"][:, 1].view(np.uint16), v.view(np.uint16))
    assert np.array_equal(got["g"].view(np.uint16), gate.view(np.uint16))
    assert np.array_equal(got["q"].view(np.uint16), q.view(np.uint16))
    _check_cache_rows(cache, kr, vr, lengths, n_new, k, v)
    cache.destroy()


def test_project_random_then_decode(device):
    """Random inputs: projections within one fp16 ulp (plus the fp32
    accumulation error) of the correctly rounded sum; cache rows bit-exact given the projected K/V; decode on the
    produced q and cache within 2e-3 of the fp32 oracle."""
    rng = np.random.default_rng(32)
    lengths = [int(x) for x in rng.integers(200, 3000, 32)]
    n_new = [1] * 32
    say("project_append random, B=32, hidden 5120, then decode")
    tables = Tables(device, 4096)
    cache, kr, vr, exp, got, pos, qw, kw, _ = _run(device, rng, lengths, n_new, 5120, False, tables)
    q, gate, k_raw, k, v = exp
    # One fp16 ulp, plus 2^-13 for fp32 accumulation over 5120 terms (its
    # typical size is ~4e-6; it only shows on values near zero, where the
    # fp16 spacing is finer).  A dropped 32-term k-step moves a value by ~0.1.
    for name, g, e in (("k", got["kv"][:, 0], k_raw), ("v", got["kv"][:, 1], v), ("gate", got["g"], gate)):
        diff = np.abs(g.astype(np.float32) - e.astype(np.float32))
        assert np.all(diff <= _ulp(e) + 2.0 ** -13), name
        assert np.mean(diff == 0) > 0.98, name
    T = len(pos)
    k_gpu = orc.qknorm_rope_exact(got["kv"][:, 0].reshape(-1, D), kw, np.repeat(tables.cos[pos], HKV, 0),
                                  np.repeat(tables.sin[pos], HKV, 0)).reshape(T, HKV, D)
    _check_cache_rows(cache, kr, vr, lengths, n_new, k_gpu, got["kv"][:, 1])
    diff = np.abs(got["q"].astype(np.float32) - q.astype(np.float32))
    assert np.all(diff <= 2 * _ulp(q) + 2.0 ** -12)
    out = device.empty((T, H, D), np.float16)
    cache.decode(0, device.array(got["q"]), out)
    device.synchronize()
    res = out.numpy()
    for b, L in enumerate(lengths):
        kc = np.concatenate([kr[0][b], k_gpu[b:b + 1]])
        vc = np.concatenate([vr[0][b], got["kv"][b:b + 1, 1]])
        ref = orc.attention_fp32(got["q"][b:b + 1], kc, vc)
        assert max_err(res[b:b + 1], ref) <= TOL, b
    cache.destroy()


@pytest.mark.parametrize("hidden,n_new", [(512, [1]), (1024, [30, 25, 15]), (1024, [20, 20]),
                                          (2048, [64, 1, 7]), (5120, [3, 70])])
def test_project_chunks_and_splits(device, hidden, n_new):
    """Steps of more than 64 tokens run in several launch pairs; hidden 512,
    1024 and 2048 select 1, 2 and 4 splits."""
    rng = np.random.default_rng(33 + hidden)
    lengths = [int(x) for x in rng.integers(0, 300, len(n_new))]
    say(f"project_append hidden {hidden}, n_new {n_new}")
    tables = Tables(device, 512)
    cache, kr, vr, exp, got, pos, qw, kw, _ = _run(device, rng, lengths, n_new, hidden, True, tables)
    q, gate, k_raw, k, v = exp
    assert np.array_equal(got["kv"][:, 0].view(np.uint16), k_raw.view(np.uint16))
    assert np.array_equal(got["kv"][:, 1].view(np.uint16), v.view(np.uint16))
    assert np.array_equal(got["g"].view(np.uint16), gate.view(np.uint16))
    assert np.array_equal(got["q"].view(np.uint16), q.view(np.uint16))
    _check_cache_rows(cache, kr, vr, lengths, n_new, k, v)
    assert cache.project_path() == ("prefill_gemm" if sum(n_new) > 64 else "kernels")
    cache.destroy()


def test_project_prefill_sized_step(device):
    """Two config-4 sequences (P = 256 and 1024) each appending a 512-token
    chunk, hidden 5120: 1024 tokens through the prefill GEMM; random inputs
    within one fp16 ulp (+ the fp32 accumulation term) of the correctly
    rounded projection, Q within two ulps after norm + RoPE, cache rows
    bit-exact given the projected K/V; then an exact-input step of 300
    tokens bit-exact everywhere."""
    rng = np.random.default_rng(35)
    lengths, n_new = [256, 1024], [512, 512]
    say("project_append prefill-sized: 2 x 512 tokens, hidden 5120")
    tables = Tables(device, 2048)
    cache, kr, vr, exp, got, pos, qw, kw, _ = _run(device, rng, lengths, n_new, 5120, False, tables)
    assert cache.project_path() == "prefill_gemm"
    q, gate, k_raw, k, v = exp
    for name, g, e in (("k", got["kv"][:, 0], k_raw), ("v", got["kv"][:, 1], v), ("gate", got["g"], gate)):
        diff = np.abs(g.astype(np.float32) - e.astype(np.float32))
        assert np.all(diff <= _ulp(e) + 2.0 ** -13), name
        assert np.mean(diff == 0) > 0.98, name
    T = len(pos)
    k_gpu = orc.qknorm_rope_exact(got["kv"][:, 0].reshape(-1, D), kw, np.repeat(tables.cos[pos], HKV, 0),
                                  np.repeat(tables.sin[pos], HKV, 0)).reshape(T, HKV, D)
    _check_cache_rows(cache, kr, vr, lengths, n_new, k_gpu, got["kv"][:, 1])
    # Q after norm + RoPE, per (token, head) row: a one-ulp difference in the
    # projected input moves every element by about one ulp of the row's
    # scale, which RoPE's sums can leave on elements much smaller than the
    # row (an element-wise ulp bound fails on some of 6.3 M values).
    diff = np.abs(got["q"].astype(np.float32) - q.astype(np.float32)).max(axis=2)
    assert np.all(diff <= 4 * _ulp(np.abs(q.astype(np.float32)).max(axis=2)) + 2.0 ** -12)
    cache.destroy()
    say("project_append prefill-sized exact: 300 tokens, hidden 1024")
    cache, kr, vr, exp, got, pos, qw, kw, _ = _run(device, rng, [40, 0, 700], [100, 150, 50], 1024, True,
                                                    Tables(device, 1024))
    assert cache.project_path() == "prefill_gemm"
    q, gate, k_raw, k, v = exp
    assert np.array_equal(got["kv"][:, 0].view(np.uint16), k_raw.view(np.uint16))
    assert np.array_equal(got["kv"][:, 1].view(np.uint16), v.view(np.uint16))
    assert np.array_equal(got["g"].view(np.uint16), gate.view(np.uint16))
    assert np.array_equal(got["q"].view(np.uint16), q.view(np.uint16))
    _check_cache_rows(cache, kr, vr, [40, 0, 700], [100, 150, 50], k, v)
    cache.destroy()


def test_project_optional_outputs(device):
    rng = np.random.default_rng(34)
    lengths = [40, 7]
    ids = _ids(rng, [4, 2])
    say("project_append optional outputs")
    cache, kr, vr = build_cache(lengths, ids, extra_rows=[1, 1], rng=rng)
    tables = Tables(device, 128)
    wq, wkv, qw, kw = _weights(rng, 512, True)
    x = rng.integers(-3, 4, (2, 512), dtype=np.int8).astype(np.float16)
    args = [device.array(x), 512, device.array(wq), device.array(wkv), device.array(qw), device.array(kw),
            tables.d_cos, tables.d_sin, tables.rows]
    q_out = device.empty((2, H, D), np.float16)
    cache.begin_step([0, 1], [1, 1])
    cache.project_append(0, *args, q_out)  # gate and kv outputs omitted
    device.synchronize()
    pos = [40, 7]
    q, gate, k_raw, k, v = orc.project_append(x, wq, wkv, qw, kw, tables.cos[pos], tables.sin[pos])
    assert np.array_equal(q_out.numpy().view(np.uint16), q.view(np.uint16))
    _check_cache_rows(cache, kr, vr, lengths, [1, 1], k, v)
    cache.destroy()


@pytest.mark.parametrize("n_new", [[2, 1, 5], [120, 1, 200]])
def test_project_other_head_shape(device, n_new):
    """8 query and 2 kv heads (G = 4): 5120 weight rows, so the last group
    of 7 row tiles is partial (its missing tiles are loaded, never
    written); every output still bit-exact on fp32-exact inputs.  321 new
    tokens take the prefill GEMM instead: 20 heads of four kinds, the second
    token tile 65 tokens long."""
    rng = np.random.default_rng(35)
    h, hkv, hidden = 8, 2, 1024
    lengths = [19, 250, 64]
    T = sum(n_new)
    ids = _ids(rng, [(L + n + 15) // 16 for L, n in zip(lengths, n_new)])
    say("project_append with 8 q / 2 kv heads")
    cache, kr, vr = build_cache(lengths, ids, extra_rows=n_new, num_heads=h, num_kv_heads=hkv, rng=rng)
    tables = Tables(device, 512)
    wq = (rng.integers(-2, 3, (2 * h * D, hidden), dtype=np.int8) * 2.0 ** -7).astype(np.float16)
    wkv = (rng.integers(-2, 3, (2 * hkv * D, hidden), dtype=np.int8) * 2.0 ** -7).astype(np.float16)
    qw = (1 + 0.02 * rng.standard_normal(D, dtype=np.float32)).astype(np.float16)
    kw = (1 + 0.02 * rng.standard_normal(D, dtype=np.float32)).astype(np.float16)
    x = rng.integers(-3, 4, (T, hidden), dtype=np.int8).astype(np.float16)
    pos = [L + i for L, n in zip(lengths, n_new) for i in range(n)]
    cache.begin_step(list(range(3)), n_new)
    q_out, g_out = device.empty((T, h, D), np.float16), device.empty((T, h, D), np.float16)
    kv_out = device.empty((T, 2, hkv, D), np.float16)
    cache.project_append(0, device.array(x), hidden, device.array(wq), device.array(wkv), device.array(qw),
                         device.array(kw), tables.d_cos, tables.d_sin, tables.rows, q_out, g_out, kv_out)
    device.synchronize()
    q, gate, k_raw, k, v = orc.project_append(x, wq, wkv, qw, kw, tables.cos[pos], tables.sin[pos], h, hkv)
    assert np.array_equal(q_out.numpy().view(np.uint16), q.view(np.uint16))
    assert np.array_equal(g_out.numpy().view(np.uint16), gate.view(np.uint16))
    kvo = kv_out.numpy()
    assert np.array_equal(kvo[:, 0].view(np.uint16), k_raw.view(np.uint16))
    assert np.array_equal(kvo[:, 1].view(np.uint16), v.view(np.uint16))
    _check_cache_rows(cache, kr, vr, lengths, n_new, k, v)
    assert cache.project_path() == ("prefill_gemm" if T > 64 else "kernels")
    cache.destroy()
