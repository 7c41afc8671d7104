"""libkvattn loads and exports every function include/kvattn.h declares (CPU only)."""
import ctypes
import re
from pathlib import Path

from mi50grad_amd import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "kvattn.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:int|const char \*)\s*(kva_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_abi():
    names = declared_functions()
    assert len(names) >= 40
    for must in ("kva_create", "kva_step_begin", "kva_append_qknorm_rope", "kva_decode",
                 "kva_prefill", "kva_tree_verify", "kva_rollback", "kva_legacy_decode"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_table_matches_header():
    declared = set(declared_functions())
    bound = set(_lib.SIGNATURES) | set(_lib.STRING_FUNCS)
    assert declared == bound, (declared - bound, bound - declared)


def test_config_struct_layout():
    # kva_config: 11 int32/float fields + uint32 flags, no padding.
    assert ctypes.sizeof(_lib.KvaConfig) == 12 * 4
    assert ctypes.sizeof(_lib.KvaLayout) == 3 * 8 + 2 * 4


def test_version_string():
    assert b"gfx950" in _lib.load().kva_version()
