"""GPU: the decode timeline (kva_timeline_enable / kva_timeline_read).

The records must describe the launch that ran (one per wave of every
workgroup, zero for waves a workgroup does not have, entry <= first K/V
issue <= walk end, an XCD id below 8, page counts that add up to the step's
pages; for the whole-sequence form, one
workgroup per sequence and kv head with that sequence's pages) and recording
must not change the decode's output (bit-equal to the same decode with the
timeline off).  Refused before it is enabled.
"""
import numpy as np
import pytest

from mi50grad_amd import _lib
from mi50grad_amd.device import GPUDevice

from gpu_helpers import H, HKV, D, build_cache, say

pytestmark = pytest.mark.gpu


def test_timeline_records_the_launch_and_leaves_the_output_alone():
    dev = GPUDevice(0)
    rng = np.random.default_rng(11)
    lengths = [700, 1500, 33, 2049]
    npg = [(n + 1 + 15) // 16 for n in lengths]
    perm = rng.permutation(sum(npg))
    ids, o = [], 0
    for n in npg:
        ids.append([int(x) for x in perm[o:o + n]])
        o += n
    say("timeline: 4 ragged sequences, one layer")
    cache, _, _ = build_cache(lengths, ids, extra_rows=1, rng=rng)
    cache.begin_step([0, 1, 2, 3], [1, 1, 1, 1])
    q = dev.array(rng.standard_normal((4, H, D), dtype=np.float32).astype(np.float16))
    out_off, out_on = dev.empty((4, H, D), np.float16), dev.empty((4, H, D), np.float16)
    with pytest.raises(_lib.KvaError, match="not enabled"):
        cache.timeline()
    cache.decode(0, q, out_off)
    cache.timeline_enable(True)
    cache.decode(0, q, out_on)
    rec = cache.timeline()
    split, n_wg = cache.decode_split()
    assert rec.shape == (n_wg, 1, 8, 4)
    assert np.array_equal(out_on.numpy().view(np.uint16), out_off.numpy().view(np.uint16))
    ent, first, end, meta = (rec[..., i] for i in range(4))
    ran = ent > 0  # waves a workgroup does not have leave zero records
    assert ran[:, :, 0].all() and (rec[~ran] == 0).all()
    assert (ent[ran] <= first[ran]).all() and (first[ran] <= end[ran]).all()
    assert (((meta[ran] >> 32) & 0xF) < 8).all()
    pages = (meta & 0xFFFFFFFF)[:, 0, 0]
    assert int(pages.sum()) == sum(npg) and (pages > 0).all()
    same = np.broadcast_to(meta[:, :, :1], meta.shape)
    assert (meta[ran] == same[ran]).all()  # every wave of a workgroup reports the same range
    cache.timeline_enable(False)
    with pytest.raises(_lib.KvaError, match="not enabled"):
        cache.timeline()
    cache.destroy()


def test_timeline_of_the_whole_sequence_form():
    """A step of short sequences runs the whole-sequence form: one record per
    wave of each of its workgroups (sequence-major, several per sequence),
    carrying that sequence's page count; the output is again unchanged by
    recording."""
    dev = GPUDevice(0)
    rng = np.random.default_rng(12)
    lengths = [40, 0, 300, 17]
    npg = [(n + 1 + 15) // 16 for n in lengths]
    perm = rng.permutation(sum(npg))
    ids, o = [], 0
    for n in npg:
        ids.append([int(x) for x in perm[o:o + n]])
        o += n
    say("timeline: whole-sequence form, 4 short sequences")
    cache, _, _ = build_cache(lengths, ids, extra_rows=1, rng=rng)
    cache.begin_step([0, 1, 2, 3], [1, 1, 1, 1])
    q = dev.array(rng.standard_normal((4, H, D), dtype=np.float32).astype(np.float16))
    out_off, out_on = dev.empty((4, H, D), np.float16), dev.empty((4, H, D), np.float16)
    cache.decode(0, q, out_off)
    cache.timeline_enable(True)
    cache.decode(0, q, out_on)
    rec = cache.timeline()
    split, n_wg = cache.decode_split()
    per_seq = n_wg // 4  # workgroups per sequence: kv heads x query-head groups
    assert split == 0 and n_wg % (4 * HKV) == 0
    assert rec.shape == (n_wg, 1, 8, 4)
    assert np.array_equal(out_on.numpy().view(np.uint16), out_off.numpy().view(np.uint16))
    ent, first, end, meta = (rec[..., i] for i in range(4))
    assert (ent > 0).all() and (ent <= first).all() and (first <= end).all()
    assert (((meta >> 32) & 0xF) < 8).all()
    pages = (meta & 0xFFFFFFFF)[:, 0, 0]
    assert [int(x) for x in pages] == [n for n in npg for _ in range(per_seq)]
    assert (meta[:, :, :1] == meta).all()  # every wave of a workgroup reports the same
    cache.timeline_enable(False)
    cache.destroy()
