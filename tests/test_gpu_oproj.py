"""GPU: kva_out_project, the O-projection of the attention rows with the
residual add (engine.py:2083-2085, gemv_fp16_v2.hip:22-87), against the
oracle (oracle.out_project).

* Integer inputs whose sums are exact in fp32: bit-exact, whatever the
  summation order, with and without the residual.
* Random N(0,1) inputs: within one fp16 ulp plus 2^-13 of the correctly
  rounded result (fp32 accumulation in another order than the reference's),
  and equal to it for almost every element; in place (residual = out).
* The config-3 shape (32 rows, q_dim 6144, n_out 5120), chunking past 64
  rows, the x-resident LDS form (q_dim 5120, n_out 10240, <= 32 rows), and
  the validation errors.
"""
import numpy as np
import pytest

from oracle import kvattn_oracle as orc

from gpu_helpers import build_cache, say

pytestmark = pytest.mark.gpu


def _ulp(x):
    a = np.abs(np.asarray(x, np.float32))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
    return (2.0 ** (e - 10)).astype(np.float32)


def _cache():
    cache, _, _ = build_cache([8], [[0]], extra_rows=[1])
    return cache


def _inputs(rng, n_tok, q_dim, n_out, exact):
    if exact:
        x = rng.integers(-3, 4, (n_tok, q_dim), dtype=np.int8).astype(np.float16)
        w = (rng.integers(-2, 3, (n_out, q_dim), dtype=np.int8) * 2.0 ** -7).astype(np.float16)
        r = (rng.integers(-64, 65, (n_tok, n_out), dtype=np.int16) * 2.0 ** -3).astype(np.float16)
    else:
        s = np.float32(1 / np.sqrt(q_dim))
        x = rng.standard_normal((n_tok, q_dim), dtype=np.float32).astype(np.float16)
        w = (rng.standard_normal((n_out, q_dim), dtype=np.float32) * s).astype(np.float16)
        r = rng.standard_normal((n_tok, n_out), dtype=np.float32).astype(np.float16)
    return x, w, r


@pytest.mark.parametrize("n_tok,q_dim,n_out", [(32, 6144, 5120), (1, 6144, 5120), (100, 1024, 512),
                                               (20, 5120, 10240)])
def test_out_project_exact(device, n_tok, q_dim, n_out):
    rng = np.random.default_rng(n_tok * 7 + n_out)
    say(f"out_project exact n_tok={n_tok} q_dim={q_dim} n_out={n_out}")
    cache = _cache()
    x, w, r = _inputs(rng, n_tok, q_dim, n_out, True)
    dx, dw = device.array(x), device.array(w)
    out, out_nr = device.empty((n_tok, n_out), np.float16), device.empty((n_tok, n_out), np.float16)
    cache.out_project(dx, n_tok, q_dim, dw, n_out, out, residual=device.array(r))
    cache.out_project(dx, n_tok, q_dim, dw, n_out, out_nr)
    device.synchronize()
    assert np.array_equal(out.numpy().view(np.uint16), orc.out_project(x, w, r).view(np.uint16))
    assert np.array_equal(out_nr.numpy().view(np.uint16), orc.out_project(x, w).view(np.uint16))
    cache.destroy()


def test_out_project_random_in_place(device):
    rng = np.random.default_rng(41)
    n_tok, q_dim, n_out = 32, 6144, 5120
    say("out_project random, in place")
    cache = _cache()
    x, w, r = _inputs(rng, n_tok, q_dim, n_out, False)
    hid = device.array(r)  # d_hidden: the residual, overwritten with the result
    cache.out_project(device.array(x), n_tok, q_dim, device.array(w), n_out, hid, residual=hid)
    device.synchronize()
    got = hid.numpy().astype(np.float32)
    exp = orc.out_project(x, w, r).astype(np.float32)
    diff = np.abs(got - exp)
    assert np.all(diff <= _ulp(exp) + 2.0 ** -13), float(np.max(diff))
    assert np.mean(diff == 0) > 0.98
    cache.destroy()


def test_out_project_empty_and_residual(device):
    """No rows is a no-op; two exact rows with the residual are bit-exact.
    (The argument refusals are checked on a host-only cache in
    test_host_logic.py, before any device work.)"""
    rng = np.random.default_rng(42)
    say("out_project empty + residual")
    cache = _cache()
    x, w, r = _inputs(rng, 2, 512, 64, True)
    dx, dw, dr = device.array(x), device.array(w), device.array(r)
    out = device.empty((2, 64), np.float16)
    cache.out_project(dx, 0, 512, dw, 64, out)  # no rows: nothing to do
    cache.out_project(dx, 2, 512, dw, 64, out, residual=dr)
    device.synchronize()
    assert np.array_equal(out.numpy().view(np.uint16), orc.out_project(x, w, r).view(np.uint16))
    cache.destroy()
