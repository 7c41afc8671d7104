"""GPU: the bandwidth probes bench.py reports next to the vendor peak.

kva_hbm_copy must copy every byte (it is also the known-size kernel that
calibrates the FETCH_SIZE / WRITE_SIZE counters); kva_hbm_read must read
without writing, except for the one fold value that proves its loads are
kept: a single 16-byte row (0x9e3779b9, 0, 0, 0) folds to exactly that.
"""
import numpy as np
import pytest

from mi50grad_amd import _lib
from mi50grad_amd.device import GPUDevice

from gpu_helpers import say

pytestmark = pytest.mark.gpu


def test_copy_and_read_probes():
    dev = GPUDevice(0)
    say("copy probe: 4 MiB + a 48-byte tail")
    src = np.random.default_rng(0).integers(0, 2 ** 32, (1 << 20) + 12, dtype=np.uint32)
    a, b = dev.array(src), dev.array(np.zeros_like(src))
    _lib.call("kva_hbm_copy", b.ptr, a.ptr, src.nbytes, None)
    dev.synchronize()
    assert np.array_equal(b.numpy(), src)

    say("read probe: zeros leave the sink alone; the magic row writes it")
    sink = dev.array(np.full(4, 7, np.uint32))
    z = dev.array(np.zeros(1 << 18, np.uint32))
    _lib.call("kva_hbm_read", z.ptr, z.nbytes, sink.ptr, None)
    dev.synchronize()
    assert sink.numpy().tolist() == [7, 7, 7, 7]
    one = dev.array(np.array([0x9E3779B9, 0, 0, 0], np.uint32))
    _lib.call("kva_hbm_read", one.ptr, 16, sink.ptr, None)
    dev.synchronize()
    assert sink.numpy().tolist() == [0x9E3779B9, 7, 7, 7]
    with pytest.raises(_lib.KvaError, match="multiple of 16"):
        _lib.call("kva_hbm_read", z.ptr, 20, sink.ptr, None)
    for x in (a, b, sink, z, one):
        x.free()


def test_paged_read_probe():
    """kva_hbm_read_pages reads exactly the listed pages with the decode's
    per-wave pattern: zero pages leave the sink alone; a listed page holding
    the magic 16 bytes at K row 0, head 0 (lane 0 of wave 0's first load)
    writes it, the same page left off the list does not."""
    dev = GPUDevice(0)
    say("paged read probe")
    pages, hkv = 4, 4
    page_words = 16 * hkv * 256 // 2  # uint32 words of one page (fp16 rows)
    k = np.zeros(pages * page_words, np.uint32)
    k[2 * page_words] = 0x9E3779B9
    dk, dv = dev.array(k), dev.array(np.zeros_like(k))
    sink = dev.array(np.full(4, 7, np.uint32))
    for ids, hit in (([3, 0], False), ([3, 2, 0], True)):
        sink.copy_from(np.full(4, 7, np.uint32))
        d_ids = dev.array(np.asarray(ids, np.int32))
        for n_wg in (1, 2):
            _lib.call("kva_hbm_read_pages", dk.ptr, dv.ptr, d_ids.ptr, len(ids), hkv, n_wg, sink.ptr, None)
        dev.synchronize()
        assert sink.numpy().tolist() == ([0x9E3779B9, 7, 7, 7] if hit else [7, 7, 7, 7]), ids
        d_ids.free()
    for x in (dk, dv, sink):
        x.free()
