"""Host-side bookkeeping of libkvattn on a host-only cache (CPU only).

Covers the failure handling the C ABI validates before any launch: bad
arguments, capacity and pool exhaustion, double free, rollback past the
base, unsorted keep lists, call order.  No device memory is touched.
"""
import pytest

from mi50grad_amd import _lib
from mi50grad_amd._lib import KvaError
from mi50grad_amd.kv_cache import PagedKVCache


def make(**kw):
    args = dict(n_layers=2, max_seqs=4, max_blocks=20, max_blocks_per_seq=8, max_step_tokens=64,
                host_only=True)
    args.update(kw)
    return PagedKVCache(**args)


def code(excinfo):
    return excinfo.value.code


def test_config_validation():
    with pytest.raises(KvaError) as e:
        make(n_layers=0)
    assert code(e) == -1
    for bad in (dict(num_heads=24, num_kv_heads=5), dict(num_heads=20, num_kv_heads=4)):
        with pytest.raises(KvaError):
            make(**bad)
    with pytest.raises(KvaError) as e:
        make(head_dim=128)
    assert code(e) == -2


def test_reserve_grows_a_page_at_a_time():
    c = make()
    assert c.free_block_count() == 20
    c.reserve(0, 1)
    assert len(c.blocks(0)) == 1
    c.reserve(0, 16)
    assert len(c.blocks(0)) == 1
    c.reserve(0, 17)
    assert len(c.blocks(0)) == 2
    assert c.free_block_count() == 18
    with pytest.raises(KvaError) as e:
        c.reserve(0, 8 * 16 + 1)
    assert code(e) == -5


def test_pool_exhaustion_and_free():
    c = make(max_blocks=5)
    c.reserve(0, 64)
    with pytest.raises(KvaError) as e:
        c.reserve(1, 32)
    assert code(e) == -4
    c.free_seq(0)
    assert c.free_block_count() == 5
    with pytest.raises(KvaError) as e:
        c.free_seq(0)
    assert code(e) == -11
    c.reserve(1, 32)
    assert len(c.blocks(1)) == 2


def test_set_blocks_validation():
    c = make()
    c.set_blocks(0, [7, 3, 11])
    assert c.blocks(0) == [7, 3, 11]
    with pytest.raises(KvaError) as e:
        c.set_blocks(1, [3])                  # in use by sequence 0
    assert code(e) == -7
    with pytest.raises(KvaError) as e:
        c.set_blocks(1, [99])                 # out of range
    assert code(e) == -7
    with pytest.raises(KvaError) as e:
        c.set_blocks(1, [4, 4])               # duplicate
    assert code(e) == -7
    c.set_blocks(0, [3, 12])                  # re-plan: keeps 3, releases 7 and 11
    assert c.free_block_count() == 18


def test_set_blocks_ends_the_step():
    """The step plan holds the block ids of the step's first pages (the
    whole-sequence decode reads them with the lengths), so replacing a
    sequence's blocks ends the step, as setting a length does."""
    c = make()
    c.begin_step([0], [1])
    with pytest.raises(KvaError) as e:
        c.decode(0, 1 << 20, 1 << 20)
    assert code(e) == -3                      # past the step check: no device
    c.set_blocks(1, [5])
    with pytest.raises(KvaError) as e:
        c.decode(0, 1 << 20, 1 << 20)
    assert code(e) == -8                      # no step begun
    c.begin_step([0, 1], [1, 1])
    assert c.seq_len(0) == 2 and c.seq_len(1) == 1


def test_bad_sequence_ids():
    c = make()
    for s in (-1, 4):
        with pytest.raises(KvaError) as e:
            c.reserve(s, 1)
        assert code(e) == -6


def test_step_assigns_slots_and_lengths():
    c = make()
    c.begin_step([0, 2], [1, 5])
    assert c.seq_len(0) == 1 and c.seq_len(2) == 5
    c.begin_step([2], [12])
    assert c.seq_len(2) == 17 and len(c.blocks(2)) == 2
    with pytest.raises(KvaError) as e:
        c.begin_step([0, 0], [1, 1])          # a sequence twice
    assert code(e) == -1
    with pytest.raises(KvaError) as e:
        c.begin_step([1], [65])               # beyond max_step_tokens
    assert code(e) == -5
    with pytest.raises(KvaError) as e:
        c.begin_step([1], [-1])
    assert code(e) == -1


def test_step_capacity_checked_before_commit():
    c = make(max_blocks=3)
    c.begin_step([0], [16])
    with pytest.raises(KvaError) as e:
        c.begin_step([0, 1], [16, 32])        # needs 3 more blocks, 2 free
    assert code(e) == -4
    assert c.seq_len(0) == 16 and c.seq_len(1) == 0   # nothing committed


def test_tree_bits_validation():
    c = make()
    with pytest.raises(KvaError):
        c.begin_step([0], [3], tree_bits=[0b001, 0b001, 0b101])   # node 1 misses itself
    c2 = make()
    with pytest.raises(KvaError):
        c2.begin_step([0], [2], tree_bits=[0b11, 0b10])            # root sees a later node
    assert c.seq_len(0) == 0 and c2.seq_len(0) == 0
    c3 = make()
    c3.begin_step([0], [3], tree_bits=[0b001, 0b011, 0b101], rope_pos=[0, 1, 1])
    assert c3.seq_len(0) == 3


def test_hot_calls_need_a_device_and_a_step():
    """Validation comes first (here: no step begun), then the device."""
    c = make()
    with pytest.raises(KvaError) as e:
        c.decode(0, 1 << 20, 1 << 20)
    assert code(e) == -8
    c.begin_step([0], [1])
    with pytest.raises(KvaError) as e:
        c.decode(0, 1 << 20, 1 << 20)
    assert code(e) == -3


def test_rollback_validation_and_lengths():
    c = make()
    c.begin_step([0, 1], [20, 9])
    c.rollback([0, 1], [11, 0], [[0, 2, 3], []])
    assert c.seq_len(0) == 14 and c.seq_len(1) == 0
    c.begin_step([0], [9])                    # length 23
    with pytest.raises(KvaError) as e:
        c.rollback([0], [14], [[2, 1]])       # not increasing
    assert code(e) == -9
    with pytest.raises(KvaError) as e:
        c.rollback([0], [14], [[0, 9]])       # beyond the length
    assert code(e) == -9
    with pytest.raises(KvaError) as e:
        c.rollback([0], [24], [[]])           # base past the length
    assert code(e) == -9
    assert c.seq_len(0) == 23


def test_rollback_beyond_staging_leaves_lengths():
    """A rollback whose row moves do not fit the staging area (4096 moves at
    this configuration) is refused before any length changes, also when a
    valid sequence precedes the one that overflows."""
    c = make(max_blocks=600, max_blocks_per_seq=300)
    c.reserve(0, 4800)
    c.set_len(0, 4800)
    c.reserve(1, 32)
    c.set_len(1, 32)
    with pytest.raises(KvaError) as e:
        c.rollback([1, 0], [16, 0], [[1, 3], list(range(1, 4800))])   # 4799 moves of sequence 0
    assert code(e) == -5
    assert c.seq_len(0) == 4800 and c.seq_len(1) == 32
    c.rollback([1, 0], [16, 0], [[1, 3], list(range(1, 4001))])      # 4002 moves fit
    assert c.seq_len(0) == 4000 and c.seq_len(1) == 18


def test_set_len_bounds():
    c = make()
    c.reserve(0, 20)
    c.set_len(0, 32)
    with pytest.raises(KvaError) as e:
        c.set_len(0, 33)
    assert code(e) == -5
    with pytest.raises(KvaError) as e:
        c.set_len(0, -1)
    assert code(e) == -9


def test_decode_split_setting():
    c = make()
    c.set_decode_split(128)
    with pytest.raises(KvaError):
        c.set_decode_split(100)


def test_graph_recording_validation():
    """kva_graph_*: a host-only cache cannot record; NULL graphs and an end
    without a begin are refused before anything touches a device."""
    import ctypes

    from mi50grad_amd import _lib

    c = make()
    c.reserve(0, 3)
    c.begin_step([0], [1])
    with pytest.raises(KvaError) as e:
        _lib.call("kva_graph_capture_begin", c.handle, None)
    assert code(e) == -3
    h = ctypes.c_void_p()
    with pytest.raises(KvaError) as e:
        _lib.call("kva_graph_capture_end", c.handle, None, ctypes.byref(h))
    assert code(e) == -8
    with pytest.raises(KvaError) as e:
        _lib.call("kva_graph_launch", None, None)
    assert code(e) == -1
    with pytest.raises(KvaError) as e:
        _lib.call("kva_graph_destroy", None)
    assert code(e) == -1


# ---- argument refusals of the device entry points, on a host-only cache ----
# Every hot-path call validates its arguments before it touches the device,
# so the refusals are checked here with fake (aligned, never dereferenced)
# pointers; a call that passes every check answers KVA_ERR_NO_DEVICE.  The
# GPU tests then only ever hand the device buffers that cover what they ask
# for.
FAKE = 1 << 20


def _rows(c, seq_ids, lens):
    for s, n in zip(seq_ids, lens):
        c.reserve(s, n)
        c.set_len(s, n)


def test_out_project_refusals_before_device():
    c = make(num_heads=24, num_kv_heads=4)
    with pytest.raises(KvaError, match="q_dim 500") as e:
        c.out_project(FAKE, 2, 500, FAKE, 64, FAKE)
    assert code(e) == -1
    with pytest.raises(KvaError, match="n_out 60") as e:
        c.out_project(FAKE, 2, 512, FAKE, 60, FAKE)
    assert code(e) == -1
    # Beyond the projection workspace for 2 tokens: refused on the host.
    with pytest.raises(KvaError, match="workspace") as e:
        c.out_project(FAKE, 2, 512, FAKE, 1 << 24, FAKE)
    assert code(e) == -1
    with pytest.raises(KvaError) as e:
        c.out_project(FAKE, -1, 512, FAKE, 64, FAKE)
    assert code(e) == -1
    with pytest.raises(KvaError) as e:
        c.out_project(None, 2, 512, FAKE, 64, FAKE)
    assert code(e) == -1
    with pytest.raises(KvaError) as e:
        c.out_project(FAKE, 2, 512, FAKE, 64, FAKE, residual=FAKE + 2)
    assert code(e) == -10
    with pytest.raises(KvaError) as e:  # every check passed: only the device is missing
        c.out_project(FAKE, 2, 512, FAKE, 64, FAKE, residual=FAKE)
    assert code(e) == -3
    # The widest output one token can take (an lm_head's) passes the checks.
    with pytest.raises(KvaError) as e:
        c.out_project(FAKE, 1, 512, FAKE, 151936, FAKE)
    assert code(e) == -3
    c.destroy()


def test_project_append_refusals_before_device():
    c = make(num_heads=24, num_kv_heads=4)
    _rows(c, [0, 1], [40, 7])
    args = [FAKE, 512, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 128]
    with pytest.raises(KvaError) as e:
        c.project_append(0, *args, FAKE)  # no step begun
    assert code(e) == -8
    c.begin_step([0, 1], [1, 1])
    for i, val, want in ((1, 1000, -1), (0, FAKE + 2, -10), (8, 40, -1), (2, None, -1), (6, FAKE + 4, -10)):
        bad = list(args)
        bad[i] = val
        with pytest.raises(KvaError) as e:
            c.project_append(0, *bad, FAKE)
        assert code(e) == want, (i, val)
    with pytest.raises(KvaError) as e:
        c.project_append(5, *args, FAKE)  # layer out of range
    assert code(e) == -1
    with pytest.raises(KvaError) as e:
        c.project_append(0, *args, FAKE)
    assert code(e) == -3
    c.destroy()


def test_decode_and_append_refusals_before_device():
    c = make(num_heads=24, num_kv_heads=4)
    _rows(c, [0, 1], [10, 20])
    c.begin_step([0, 1], [2, 1])
    with pytest.raises(KvaError, match="one new token") as e:
        c.decode(0, FAKE, FAKE)
    assert code(e) == -8
    with pytest.raises(KvaError, match="one new token"):
        c.append_decode(0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 64, FAKE)
    c.begin_step([0, 1], [1, 1])
    with pytest.raises(KvaError, match="table rows"):
        c.append_decode(0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 5, FAKE)
    with pytest.raises(KvaError) as e:
        c.append(0, FAKE, FAKE + 8, FAKE, FAKE, FAKE, FAKE, FAKE, 64)
    assert code(e) == -10
    with pytest.raises(KvaError) as e:
        c.decode(0, FAKE, FAKE, gate=FAKE + 4)
    assert code(e) == -10
    with pytest.raises(KvaError) as e:
        c.decode(0, FAKE, FAKE, gate=FAKE, gate_stride=24 * 256 - 4)
    assert code(e) == -1
    with pytest.raises(KvaError, match="NULL gate"):
        _lib.call("kva_append_decode_gated", c.handle, 0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 64, None, 0,
                  FAKE, None)
    for call in (lambda: c.decode(0, FAKE, FAKE), lambda: c.append(0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 64),
                 lambda: c.append_decode(0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 64, FAKE)):
        with pytest.raises(KvaError) as e:
            call()
        assert code(e) == -3
    c.destroy()


def test_multi_query_refusals_before_device():
    c = make(num_heads=24, num_kv_heads=4)
    _rows(c, [0], [10])
    c.begin_step([0], [3])
    with pytest.raises(KvaError, match="tree_bits") as e:
        c.tree_verify(0, FAKE, FAKE)
    assert code(e) == -8
    with pytest.raises(KvaError) as e:
        c.prefill(0, FAKE + 2, FAKE)
    assert code(e) == -10
    with pytest.raises(KvaError) as e:
        c.prefill(0, FAKE, FAKE)
    assert code(e) == -3
    c.destroy()


def test_append_prefill_refusals_before_device():
    """kva_append_prefill validates the append's and the attention's
    arguments (pointers, alignment, table rows, gate) before the device
    check, which a valid call on a host-only cache reaches last."""
    c = make(num_heads=24, num_kv_heads=4)
    _rows(c, [0, 1], [10, 20])
    args = [FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 64]
    with pytest.raises(KvaError, match="no step") as e:
        c.append_prefill(0, *args, FAKE)
    assert code(e) == -8
    c.begin_step([0, 1], [3, 5])
    for i, val, want in ((0, None, -1), (1, FAKE + 8, -10), (3, FAKE + 2, -10), (5, FAKE + 4, -10), (7, 20, -1)):
        bad = list(args)
        bad[i] = val
        with pytest.raises(KvaError) as e:
            c.append_prefill(0, *bad, FAKE)
        assert code(e) == want, (i, val)
    with pytest.raises(KvaError) as e:
        c.append_prefill(0, *args, FAKE + 2)  # misaligned out
    assert code(e) == -10
    with pytest.raises(KvaError, match="NULL gate"):
        _lib.call("kva_append_prefill_gated", c.handle, 0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 64, None, 0,
                  FAKE, None)
    with pytest.raises(KvaError) as e:
        c.append_prefill(0, *args, FAKE, gate=FAKE, gate_stride=24 * 256 - 4)
    assert code(e) == -1
    with pytest.raises(KvaError) as e:
        c.append_prefill(5, *args, FAKE)  # layer out of range
    assert code(e) == -1
    with pytest.raises(KvaError) as e:
        c.append_prefill(0, *args, FAKE)
    assert code(e) == -3
    c.destroy()


def test_legacy_decode_without_workspace_refuses_long_caches():
    """kva_legacy_decode with no workspace cache runs only the whole-sequence
    form; past 1024 rows it refuses (KVA_ERR_STATE) instead of streaming a
    long cache on one workgroup per kv head.  Refused before any launch."""
    with pytest.raises(KvaError, match="workspace") as e:
        _lib.call("kva_legacy_decode", None, FAKE, FAKE, FAKE, FAKE, 1025, 24, 4, None)
    assert code(e) == -8
    with pytest.raises(KvaError, match="workspace") as e:
        _lib.call("kva_legacy_decode_batched", None, FAKE, FAKE, FAKE, FAKE, 5000, 2, 5000 * 2048, 24, 4, None)
    assert code(e) == -8


def test_paged_read_probe_refusals():
    """kva_hbm_read_pages validates before any launch (fake pointers)."""
    for args, want in (((FAKE, FAKE, FAKE, 4, 4, 0, FAKE), -1), ((FAKE, FAKE, FAKE, -1, 4, 8, FAKE), -1),
                       ((FAKE, FAKE, FAKE, 4, 17, 8, FAKE), -2), ((FAKE + 8, FAKE, FAKE, 4, 4, 8, FAKE), -10),
                       ((None, FAKE, FAKE, 4, 4, 8, FAKE), -1)):
        with pytest.raises(KvaError) as e:
            _lib.call("kva_hbm_read_pages", *args, None)
        assert code(e) == want, args
