"""The allocation-free decode entry point, kva_legacy_decode_noalloc.

It is kva_legacy_decode (flash_attn_256_decode semantics on a contiguous
cache) with the split-K partials in the library's static device scratch
instead of a cache workspace.  On the GPU it is called through the C ABI
twice in a row, the second call on a smaller cache (so it runs fewer
workgroups over the scratch the first call left behind), and each output
must equal kva_legacy_decode's on the same inputs bit for bit (the same
stream-K split, the same kernels) and lie within 2e-3 of the fp32 oracle.
On the CPU: the head-count limit is refused before any device work.
"""
import numpy as np
import pytest

from mi50grad_amd import _lib
from mi50grad_amd.kv_cache import PagedKVCache
from oracle import kvattn_oracle as orc

from gpu_helpers import HKV, H, D, max_err, say

TOL = 2e-3


def test_noalloc_refuses_too_many_heads():
    """num_heads beyond the static scratch's limit: KVA_ERR_CAPACITY, raised
    by argument checks that run before anything touches the device (the
    pointers are never dereferenced)."""
    fake = 1 << 20  # 16-byte aligned, never used
    with pytest.raises(_lib.KvaError) as e:
        _lib.call("kva_legacy_decode_noalloc", fake, fake, fake, fake, 256, 136, 17, None)
    assert e.value.code == -5 and "136" in str(e.value)


@pytest.mark.gpu
def test_noalloc_decode_matches_workspace_decode(device):
    rng = np.random.default_rng(70)
    ws = PagedKVCache(n_layers=1, max_seqs=1, max_blocks=1, max_blocks_per_seq=1, max_step_tokens=16)
    cases = []
    for L in (5000, 700):  # the second call is smaller
        q = rng.standard_normal((H, D), dtype=np.float32).astype(np.float16)
        k = rng.standard_normal((L, HKV, D), dtype=np.float32).astype(np.float16)
        v = rng.standard_normal((L, HKV, D), dtype=np.float32).astype(np.float16)
        cases.append(dict(L=L, q=q, k=k, v=v, dq=device.array(q), dk=device.array(k), dv=device.array(v),
                          got=device.empty((H, D), np.float16), ref=device.empty((H, D), np.float16)))
    device.synchronize()
    for c in cases:
        say(f"noalloc decode L={c['L']}")
        _lib.call("kva_legacy_decode_noalloc", c["dq"].ptr, c["dk"].ptr, c["dv"].ptr, c["got"].ptr, c["L"], H, HKV,
                  None)
    for c in cases:
        _lib.call("kva_legacy_decode", ws.handle, c["dq"].ptr, c["dk"].ptr, c["dv"].ptr, c["ref"].ptr, c["L"], H,
                  HKV, None)
    device.synchronize()
    for c in cases:
        got, ref = c["got"].numpy(), c["ref"].numpy()
        assert np.array_equal(got.view(np.uint16), ref.view(np.uint16)), c["L"]
        exp = orc.attention_fp32(c["q"][None], c["k"], c["v"])[0]
        assert max_err(got, exp) <= TOL, c["L"]
    ws.destroy()
