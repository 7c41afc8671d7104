"""The allocation-free decode entry point, kva_legacy_decode_noalloc.

It is kva_legacy_decode (flash_attn_256_decode semantics on a contiguous
cache) with the split-K partials in the library's static device scratch
instead of a cache workspace.  On the GPU it is called through the C ABI
three times in a row, the second call on a smaller cache (so it runs fewer
workgroups over the scratch the first call left behind) and the third with
so many heads that the scratch, not the CU count, caps its workgroups; each
output must equal kva_legacy_decode's on the same inputs bit for bit (the
same stream-K split, the same kernels) and lie within 2e-3 of the fp32
oracle.
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
    """Three calls in a row through the static scratch: 5000 rows (313
    pages over 256 workgroups), then 2000 rows (125 pages, 125 workgroups:
    a smaller stream-K launch over the partials the first call left), then
    128 query / 16 kv heads over 3000 rows, where the 16 MiB scratch holds
    the partials of only 63 workgroups (fewer than the CUs).  Each output
    equals kva_legacy_decode's bit for bit when the workspace cache runs
    the same split (the third with its split set to 48 tokens: 63
    workgroups), and lies within 2e-3 of the fp32 oracle."""
    rng = np.random.default_rng(70)
    ws = PagedKVCache(n_layers=1, max_seqs=1, max_blocks=1, max_blocks_per_seq=1, max_step_tokens=16)
    cases = []
    for h, hkv, L, split in ((H, HKV, 5000, 0), (H, HKV, 2000, 0), (128, 16, 3000, 48)):
        q = rng.standard_normal((h, D), dtype=np.float32).astype(np.float16)
        k = rng.standard_normal((L, hkv, D), dtype=np.float32).astype(np.float16)
        v = rng.standard_normal((L, hkv, D), dtype=np.float32).astype(np.float16)
        cases.append(dict(h=h, hkv=hkv, L=L, split=split, q=q, k=k, v=v, dq=device.array(q), dk=device.array(k),
                          dv=device.array(v), got=device.empty((h, D), np.float16),
                          ref=device.empty((h, D), np.float16)))
    device.synchronize()
    for c in cases:
        say(f"noalloc decode H={c['h']} Hkv={c['hkv']} L={c['L']}")
        _lib.call("kva_legacy_decode_noalloc", c["dq"].ptr, c["dk"].ptr, c["dv"].ptr, c["got"].ptr, c["L"], c["h"],
                  c["hkv"], None)
    for c in cases:
        ws.set_decode_split(c["split"])
        _lib.call("kva_legacy_decode", ws.handle, c["dq"].ptr, c["dk"].ptr, c["dv"].ptr, c["ref"].ptr, c["L"],
                  c["h"], c["hkv"], None)
        device.synchronize()
        assert ws.decode_split()[1] == {5000: 256, 2000: 125, 3000: 63}[c["L"]], ws.decode_split()
    device.synchronize()
    for c in cases:
        got, ref = c["got"].numpy(), c["ref"].numpy()
        assert np.array_equal(got.view(np.uint16), ref.view(np.uint16)), c["L"]
        exp = orc.attention_fp32(c["q"][None], c["k"], c["v"])[0]
        assert max_err(got, exp) <= TOL, c["L"]
    ws.destroy()
