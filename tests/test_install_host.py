"""Host-side behaviour of attention.install() (CPU only).

The RoPE tables an installed engine gets must cover every position its
callers can address: reference code indexes engine.d_cos directly
(engine.py:2741; tp_engine.py:169, 341, 2933) with no bounds check, so the
tables never shrink below the engine's cache length or the tables already
built, and the tables they replace are freed.
"""
from types import SimpleNamespace

import numpy as np

from mi50grad_amd import attention as att
from mi50grad_amd.config import AttnConfig
from mi50grad_amd.rope import rope_tables


class FakeDevice:
    """malloc/upload/free bookkeeping in host memory (no GPU)."""

    def __init__(self):
        self.live = {}
        self.freed = []
        self.next = 1 << 20

    def malloc(self, n):
        p = self.next
        self.next += (n + 255) // 256 * 256
        self.live[p] = b"\0" * n
        return p

    def upload(self, p, data):
        assert p in self.live and len(data) == len(self.live[p])
        self.live[p] = bytes(data)

    def free(self, p):
        assert p in self.live, "freed a pointer that was not allocated"
        del self.live[p]
        self.freed.append(p)


def test_rows_follow_a_non_drop_in_cache():
    """The reference's own KVCache (not this package's) with max_seq_len 4096:
    the tables get 4096 rows, not the 2048 default."""
    eng = SimpleNamespace(kv_cache=SimpleNamespace(max_seq_len=4096))
    assert att.rope_table_rows(eng) == 4096
    assert att.rope_table_rows(eng, 100) == 4096          # an explicit smaller request cannot shrink them
    assert att.rope_table_rows(eng, 8192) == 8192
    eng.rope_rows = 16384                                 # tables already built
    assert att.rope_table_rows(eng) == 16384
    assert att.rope_table_rows(SimpleNamespace()) == 2048
    assert att.rope_table_rows(SimpleNamespace(max_seq_len=3000, kv_cache=None)) == 3000


def test_init_rope_tables_replaces_and_frees():
    dev = FakeDevice()
    cfg = AttnConfig()
    eng = SimpleNamespace(config=cfg, device=dev, kv_cache=SimpleNamespace(max_seq_len=4096))
    # The engine's own tables (engine.py:1025-1046 allocates them at init).
    eng.d_cos, eng.d_sin = dev.malloc(2048 * 64), dev.malloc(2048 * 64)
    old = (eng.d_cos, eng.d_sin)
    att.FullAttentionLaunchers._init_rope_tables(eng, att.rope_table_rows(eng))
    assert eng.rope_rows >= 4096
    assert set(old) <= set(dev.freed) and set(old).isdisjoint(dev.live)
    cos, sin = rope_tables(eng.rope_rows)
    assert dev.live[eng.d_cos] == cos.tobytes() and dev.live[eng.d_sin] == sin.tobytes()
    # Positions up to 4095 are inside the tables the reference code indexes.
    assert eng.d_cos + 4095 * 64 + 64 <= eng.d_cos + len(dev.live[eng.d_cos])
    assert len(dev.live) == 2
