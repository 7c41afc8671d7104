"""ctypes binding of libkvattn.so (the C ABI declared in include/kvattn.h).

The host convention follows the reference's ``hip_dispatch`` (ctypes over a
shared library, integer device addresses, a raised error for any nonzero
return code: hip_dispatch.py:267-269).  The library must have been built
(``python -m mi50grad_amd.build``); there is no fallback path.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_int64, c_size_t, c_uint32, c_uint64, c_void_p
from pathlib import Path

# KVA_LIB names another build of the library (the host-sanitized one of
# `python -m mi50grad_amd.build --sanitize`); by default the in-tree build.
LIB_PATH = Path(os.environ["KVA_LIB"]).resolve() if os.environ.get("KVA_LIB") \
    else Path(__file__).resolve().with_name("libkvattn.so")

KVA_FLAG_HOST_ONLY = 0x1
ERROR_NAMES = {
    -1: "KVA_ERR_INVALID_ARG", -2: "KVA_ERR_UNSUPPORTED", -3: "KVA_ERR_NO_DEVICE",
    -4: "KVA_ERR_OUT_OF_BLOCKS", -5: "KVA_ERR_CAPACITY", -6: "KVA_ERR_BAD_SEQ",
    -7: "KVA_ERR_BAD_BLOCK", -8: "KVA_ERR_STATE", -9: "KVA_ERR_ROLLBACK",
    -10: "KVA_ERR_MISALIGNED", -11: "KVA_ERR_DOUBLE_FREE",
}


class KvaError(RuntimeError):
    """A libkvattn call returned nonzero (validation code < 0, hipError_t > 0)."""

    def __init__(self, code: int, what: str, detail: str):
        self.code = code
        name = ERROR_NAMES.get(code, f"hipError {code}")
        super().__init__(f"{what} failed: {name}: {detail}")


class KvaConfig(ctypes.Structure):
    _fields_ = [
        ("n_layers", c_int32), ("num_heads", c_int32), ("num_kv_heads", c_int32),
        ("head_dim", c_int32), ("rotary_dim", c_int32), ("block_tokens", c_int32),
        ("max_seqs", c_int32), ("max_blocks", c_int32), ("max_blocks_per_seq", c_int32),
        ("max_step_tokens", c_int32), ("eps", c_float), ("flags", c_uint32),
    ]


class KvaLayout(ctypes.Structure):
    _fields_ = [
        ("row_bytes", c_uint64), ("block_bytes", c_uint64), ("layer_bytes", c_uint64),
        ("block_tokens", c_int32), ("max_blocks_per_seq", c_int32),
    ]


_P = c_void_p
_I = c_int32
_PI = POINTER(c_int32)
# name -> argtypes; every function returns int except the two string getters.
SIGNATURES = {
    "kva_create": [POINTER(KvaConfig), POINTER(c_void_p)],
    "kva_destroy": [_P],
    "kva_get_layout": [_P, POINTER(KvaLayout)],
    "kva_layer_pools": [_P, _I, POINTER(c_void_p), POINTER(c_void_p)],
    "kva_seq_reserve": [_P, _I, _I],
    "kva_seq_set_blocks": [_P, _I, _PI, _I],
    "kva_seq_free": [_P, _I],
    "kva_seq_get_len": [_P, _I, _PI],
    "kva_seq_set_len": [_P, _I, _I],
    "kva_seq_get_blocks": [_P, _I, _PI, _I, _PI],
    "kva_free_block_count": [_P, _PI],
    "kva_row_ptr": [_P, _I, _I, _I, POINTER(c_void_p), POINTER(c_void_p)],
    "kva_sync_tables": [_P, _P],
    "kva_step_begin": [_P, _I, _PI, _PI, _PI, POINTER(c_uint64), _P],
    "kva_append_qknorm_rope": [_P, _I, _P, _P, _P, _P, _P, _P, _P, _I, _P],
    "kva_project_append": [_P, _I, _P, _I, _P, _P, _P, _P, _P, _P, _I, _P, _P, _P, _P],
    "kva_out_project": [_P, _P, _I, _I, _P, _I, _P, _P, _P],
    "kva_decode": [_P, _I, _P, _P, _P],
    "kva_decode_gated": [_P, _I, _P, _P, c_int64, _P, _P],
    "kva_append_decode": [_P, _I, _P, _P, _P, _P, _P, _P, _P, _I, _P, _P],
    "kva_append_decode_gated": [_P, _I, _P, _P, _P, _P, _P, _P, _P, _I, _P, c_int64, _P, _P],
    "kva_prefill": [_P, _I, _P, _P, _P],
    "kva_tree_verify": [_P, _I, _P, _P, _P],
    "kva_prefill_gated": [_P, _I, _P, _P, c_int64, _P, _P],
    "kva_append_prefill": [_P, _I, _P, _P, _P, _P, _P, _P, _P, _I, _P, _P],
    "kva_append_prefill_gated": [_P, _I, _P, _P, _P, _P, _P, _P, _P, _I, _P, c_int64, _P, _P],
    "kva_tree_verify_gated": [_P, _I, _P, _P, c_int64, _P, _P],
    "kva_rollback": [_P, _I, _PI, _PI, _PI, _PI, _P],
    "kva_set_decode_split": [_P, _I],
    "kva_get_decode_split": [_P, _PI, _PI],
    "kva_kernel_events": [_P, _P, _P],
    "kva_hbm_read_pages": [_P, _P, _P, _I, _I, _I, _P, _P],
    "kva_timeline_enable": [_P, _I],
    "kva_get_project_path": [_P, _PI],
    "kva_timeline_read": [_P, POINTER(c_uint64), c_size_t, _PI, _PI],
    "kva_graph_capture_begin": [_P, _P],
    "kva_graph_capture_end": [_P, _P, POINTER(c_void_p)],
    "kva_graph_launch": [_P, _P],
    "kva_graph_destroy": [_P],
    "kva_legacy_qknorm_rope": [_P, _P, _P, _P, _P, _I, _I, _I, c_float, _P],
    "kva_legacy_decode": [_P, _P, _P, _P, _P, _I, _I, _I, _P],
    "kva_legacy_decode_noalloc": [_P, _P, _P, _P, _I, _I, _I, _P],
    "kva_legacy_decode_gated": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _P],
    "kva_legacy_decode_batched": [_P, _P, _P, _P, _P, _I, _I, c_int64, _I, _I, _P],
    "kva_hbm_copy": [_P, _P, c_size_t, _P],
    "kva_hbm_read": [_P, c_size_t, _P, _P],
    "kva_dev_count": [_PI],
    "kva_dev_props": [_PI, _PI, _PI, _PI],
    "kva_dev_set": [_I],
    "kva_dev_malloc": [POINTER(c_void_p), c_size_t],
    "kva_dev_free": [_P],
    "kva_memcpy_h2d": [_P, _P, c_size_t],
    "kva_memcpy_d2h": [_P, _P, c_size_t],
    "kva_memcpy_d2d": [_P, _P, c_size_t],
    "kva_memset": [_P, _I, c_size_t],
    "kva_dev_synchronize": [],
    "kva_stream_create": [POINTER(c_void_p)],
    "kva_stream_destroy": [_P],
    "kva_stream_synchronize": [_P],
    "kva_event_create": [POINTER(c_void_p)],
    "kva_event_destroy": [_P],
    "kva_event_record": [_P, _P],
    "kva_event_synchronize": [_P],
    "kva_event_elapsed_ms": [POINTER(c_float), _P, _P],
}
STRING_FUNCS = ("kva_last_error_string", "kva_version")

_lib = None


def load() -> ctypes.CDLL:
    """Load libkvattn.so once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m mi50grad_amd.build` "
                           "(no CPU or PyTorch fallback exists for this path)")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = c_int
    for name in STRING_FUNCS:
        fn = getattr(lib, name)
        fn.argtypes = []
        fn.restype = c_char_p
    _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        detail = load().kva_last_error_string().decode(errors="replace")
        raise KvaError(rc, what, detail)


def call(name: str, *args) -> None:
    """Call ``name`` and raise KvaError on a nonzero return code."""
    check(getattr(load(), name)(*args), name)


def int_array(values) -> ctypes.Array:
    vals = [int(v) for v in values]
    return (c_int32 * max(1, len(vals)))(*vals)


def u64_array(values) -> ctypes.Array:
    vals = [int(v) for v in values]
    return (c_uint64 * max(1, len(vals)))(*vals)
