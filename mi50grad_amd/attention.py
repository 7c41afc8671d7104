"""Engine-facing attention launchers with the reference's names and arguments.

``FullAttentionLaunchers`` provides the attention methods of the reference's
``InferenceEngine`` so engine code calls them unchanged:

* ``_init_rope_tables``            engine.py:1025-1046
* ``_launch_qknorm_rope``          engine.py:2371-2399 (qknorm_rope_fused)
* ``_launch_qknorm_rope_cachew``   engine.py:2401-2432 (qknorm_rope_cachew_fused)
* ``set_direct_kv_write``          engine.py:660-678
* ``_launch_decode_attn_256``      engine.py:2760-2804 (flash_attn_256_decode)
* ``_launch_decode_attn_256_batched`` engine.py:2806-2857

Pointers are integer device addresses, as in the reference.  Every launch
goes to libkvattn's gfx950 kernels; failures raise ``KvaError`` (the
reference's silent fallbacks, engine.py:2774-2803, are not reproduced).
"""
from __future__ import annotations

from . import _lib
from .device import GPUDevice
from .kv_cache import KVCache
from .rope import rope_tables


class FullAttentionLaunchers:
    def __init__(self, config, device: GPUDevice | None = None, max_seq_len: int = 2048,
                 tp_size: int = 1, kv_cache: KVCache | None = None, stream=None):
        self.config = config
        self.device = device if device is not None else GPUDevice(0)
        self.tp_size = tp_size
        self.local_num_attention_heads = config.num_attention_heads // tp_size
        self.local_num_kv_heads = config.num_key_value_heads // tp_size
        self.kv_cache = kv_cache
        self.stream = stream
        self._qknorm_rope_fused = True
        self._qknorm_rope_cachew = True
        self._direct_kv_write = False
        self._init_rope_tables(max_seq_len)

    def _init_rope_tables(self, max_seq_len: int):
        cfg = self.config
        cos, sin = rope_tables(max_seq_len, cfg.head_dim, cfg.partial_rotary_factor, cfg.rope_theta)
        self.rotary_dim = int(cfg.head_dim * cfg.partial_rotary_factor)
        self.rope_rows = max_seq_len
        self.d_cos = self.device.malloc(cos.nbytes)
        self.d_sin = self.device.malloc(sin.nbytes)
        self.device.upload(self.d_cos, cos.tobytes())
        self.device.upload(self.d_sin, sin.tobytes())

    def set_direct_kv_write(self, enabled: bool):
        self._direct_kv_write = bool(enabled)

    def _rope_rows(self, position: int) -> tuple[int, int]:
        if not 0 <= position < self.rope_rows:
            raise ValueError(f"position {position} outside the RoPE table [0, {self.rope_rows})")
        off = position * (self.rotary_dim // 2) * 2
        return self.d_cos + off, self.d_sin + off

    def _launch_qknorm_rope(self, x_ptr, norm_weight, position, num_heads, head_dim):
        c, s = self._rope_rows(position)
        _lib.call("kva_legacy_qknorm_rope", x_ptr, norm_weight, c, s, None, num_heads, head_dim,
                  self.rotary_dim // 2, self.config.rms_norm_eps, self.stream)

    def _launch_qknorm_rope_cachew(self, x_ptr, norm_weight, position, num_heads, head_dim,
                                   cache_dst):
        c, s = self._rope_rows(position)
        _lib.call("kva_legacy_qknorm_rope", x_ptr, norm_weight, c, s, cache_dst or None, num_heads,
                  head_dim, self.rotary_dim // 2, self.config.rms_norm_eps, self.stream)

    def _workspace(self):
        return self.kv_cache.paged.handle if self.kv_cache is not None else None

    def _launch_gemv_fp16(self, dst, src, weight, K, N, residual=0, stream=0):
        """FP16 GEMV dst[N] = weight[N, K] . src[K] (+ residual[N] when
        non-zero, one rounding after the add): the reference launcher
        (engine.py:2434-2455) as the O-projection uses it (engine.py:2083-
        2085, residual = d_hidden), through kva_out_project for one row.
        Needs the KV cache (its workspace); K a multiple of 512, N of 16."""
        _lib.call("kva_out_project", self._workspace(), src, 1, K, weight, N, residual or None, dst,
                  stream or self.stream)

    def _launch_decode_attn_256(self, out, q, k_cache, v_cache, seq_len):
        _lib.call("kva_legacy_decode", self._workspace(), q, k_cache, v_cache, out, seq_len,
                  self.local_num_attention_heads, self.local_num_kv_heads, self.stream)

    def _launch_decode_attn_256_gated(self, out, q, gate, k_cache, v_cache, seq_len):
        """The engine's decode + _launch_sigmoid_mul pair (engine.py:2047-2056)
        in one launch: out = fp16(fp16(attn) * sigmoid(gate))."""
        _lib.call("kva_legacy_decode_gated", self._workspace(), q, gate, k_cache, v_cache, out, seq_len,
                  self.local_num_attention_heads, self.local_num_kv_heads, self.stream)

    def _launch_decode_attn_256_batched(self, out_batch, q_batch, k_cache_base, v_cache_base,
                                        seq_len, batch_size, batch_stride: int | None = None):
        if batch_stride is None:
            if self.kv_cache is None:
                raise ValueError("batch_stride is needed without a KVCache")
            batch_stride = self.kv_cache.batch_stride
        _lib.call("kva_legacy_decode_batched", self._workspace(), q_batch, k_cache_base,
                  v_cache_base, out_batch, seq_len, batch_size, batch_stride,
                  self.local_num_attention_heads, self.local_num_kv_heads, self.stream)
