"""Engine-facing attention launchers with the reference's names and arguments.

``FullAttentionLaunchers`` provides the full-attention methods of the
reference's ``InferenceEngine`` (and the speculative engine's rollback) so
engine code calls them unchanged:

* ``_init_rope_tables``             engine.py:1025-1046
* ``_launch_qknorm_rope``           engine.py:2371-2399 (qknorm_rope_fused)
* ``_launch_qknorm_rope_cachew``    engine.py:2401-2432 (qknorm_rope_cachew_fused)
* ``set_direct_kv_write``           engine.py:660-678
* ``_launch_decode_attn_256``       engine.py:2760-2804 (flash_attn_256_decode)
* ``_launch_decode_attn_256_batched`` engine.py:2806-2857
* ``_prefill_full_attention``       engine.py:3043-3139
* ``_decode_full_attention``        engine.py:1943-2092
* ``_decode_full_attention_batched`` engine.py:1778-1876
* ``build_decode_launch_cache``     engine.py:3309-3555 (its qknorm_q, qknorm_k
  and decode_attn entries, with the same mutable parameter indices)
* ``rollback_kv_cache``             tp_engine.py:1673-1687

``install(engine)`` puts these on an existing engine instance.  That is the
supported way to swap them into the reference engine: the engine class
defines the same names in its own body, so a base class (mixin) would lose
to them in Python's method resolution order.

Pointers are integer device addresses, as in the reference.  Every launch
goes to libkvattn's gfx950 kernels; failures raise ``KvaError`` (the
reference's silent fallbacks, engine.py:2774-2803, are not reproduced).
"""
from __future__ import annotations

import ctypes
import types

from . import _lib
from .device import GPUDevice
from .kv_cache import KVCache, PagedKVCache
from .rope import rope_tables


class KvaLaunchSpec:
    """One pre-built launch of the decode launch cache.

    Keeps the reference LaunchSpec's surface (hip_dispatch.py:23-60): a list
    of ctypes values in ``params`` that callers update in place between
    launches (``spec.params[2].value = new_cos_ptr``) and a ``grid``/``block``
    for inspection.  ``launch(stream)`` reads the current values and calls
    the libkvattn entry point that replaces the reference kernel;
    ``GPUDevice.launch_cached(spec)`` does the same.
    """

    def __init__(self, kind: str, params: list, grid: tuple, block: tuple = (256, 1, 1),
                 num_heads: int = 0, workspace=None):
        self.kind = kind
        self.params = params
        self.grid = grid
        self.block = block
        self.num_heads = num_heads
        self.workspace = workspace

    def launch(self, stream=None) -> None:
        p = [x.value for x in self.params]
        if self.kind == "qknorm":        # x, w, cos, sin, head_dim, half_rotary, eps
            _lib.call("kva_legacy_qknorm_rope", p[0], p[1], p[2], p[3], None, self.num_heads, p[4], p[5],
                      p[6], stream)
        elif self.kind == "qknorm_cachew":  # x, w, cos, sin, cache_dst, head_dim, half_rotary, eps
            _lib.call("kva_legacy_qknorm_rope", p[0], p[1], p[2], p[3], p[4] or None, self.num_heads, p[5],
                      p[6], p[7], stream)
        elif self.kind == "decode":      # q, k, v, out, seq_len, num_heads, num_kv_heads
            _lib.call("kva_legacy_decode", self.workspace, p[0], p[1], p[2], p[3], p[4], p[5], p[6], stream)
        else:
            raise ValueError(f"unknown launch kind {self.kind!r}")


class FullAttentionLaunchers:
    def __init__(self, config, device: GPUDevice | None = None, max_seq_len: int = 2048,
                 tp_size: int = 1, kv_cache: KVCache | None = None, stream=None):
        self.config = config
        self.device = device if device is not None else GPUDevice(0)
        self.tp_size = tp_size
        self.kv_cache = kv_cache
        self._kva_stream = stream
        _setup(self, rope_table_rows(self, max_seq_len), tp_size)

    def _init_rope_tables(self, max_seq_len: int):
        """cos/sin tables of max_seq_len rows (the recipe of engine.py:1025-
        1046, so the fp16 bits are the reference's).  Tables this object
        already holds (the engine's own, or an earlier install's) are freed
        once the new ones are in place."""
        cfg = self.config
        cos, sin = rope_tables(max_seq_len, cfg.head_dim, cfg.partial_rotary_factor, cfg.rope_theta)
        old = [p for p in (getattr(self, "d_cos", 0), getattr(self, "d_sin", 0)) if p]
        self.rotary_dim = int(cfg.head_dim * cfg.partial_rotary_factor)
        self.rope_rows = max_seq_len
        self.d_cos = self.device.malloc(cos.nbytes)
        self.d_sin = self.device.malloc(sin.nbytes)
        self.device.upload(self.d_cos, cos.tobytes())
        self.device.upload(self.d_sin, sin.tobytes())
        for p in old:
            self.device.free(p)

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
                  self.rotary_dim // 2, self.config.rms_norm_eps, self._kva_stream)

    def _launch_qknorm_rope_cachew(self, x_ptr, norm_weight, position, num_heads, head_dim,
                                   cache_dst):
        c, s = self._rope_rows(position)
        _lib.call("kva_legacy_qknorm_rope", x_ptr, norm_weight, c, s, cache_dst or None, num_heads,
                  head_dim, self.rotary_dim // 2, self.config.rms_norm_eps, self._kva_stream)

    def _workspace(self):
        """The cache whose split-K workspace the contiguous-cache launches
        borrow: the engine's KVCache, or one the launchers own (made once,
        at set-up)."""
        if isinstance(self.kv_cache, KVCache):
            return self.kv_cache.paged.handle
        return self._kva_ws.handle

    def _launch_gemv_fp16(self, dst, src, weight, K, N, residual=0, stream=0):
        """FP16 GEMV dst[N] = weight[N, K] . src[K] (+ residual[N] when
        non-zero, one rounding after the add): the reference launcher
        (engine.py:2434-2455) as the O-projection uses it (engine.py:2083-
        2085, residual = d_hidden), through kva_out_project for one row.
        K must be a multiple of 512 and N of 16 (KvaError otherwise); any N
        that fits the projection workspace for one row, e.g. an lm_head's.
        ``install`` leaves the engine's own GEMV in place unless asked."""
        if K % 512 or N % 16:
            raise ValueError(f"_launch_gemv_fp16: K={K} must be a multiple of 512 and N={N} of 16 "
                             "for kva_out_project")
        _lib.call("kva_out_project", self._workspace(), src, 1, K, weight, N, residual or None, dst,
                  stream or self._kva_stream)

    def _launch_decode_attn_256(self, out, q, k_cache, v_cache, seq_len):
        _lib.call("kva_legacy_decode", self._workspace(), q, k_cache, v_cache, out, seq_len,
                  self.local_num_attention_heads, self.local_num_kv_heads, self._kva_stream)

    def _launch_decode_attn_256_gated(self, out, q, gate, k_cache, v_cache, seq_len):
        """The engine's decode + _launch_sigmoid_mul pair (engine.py:2047-2056)
        in one launch: out = fp16(fp16(attn) * sigmoid(gate))."""
        _lib.call("kva_legacy_decode_gated", self._workspace(), q, gate, k_cache, v_cache, out, seq_len,
                  self.local_num_attention_heads, self.local_num_kv_heads, self._kva_stream)

    def _launch_decode_attn_256_batched(self, out_batch, q_batch, k_cache_base, v_cache_base,
                                        seq_len, batch_size, batch_stride: int | None = None):
        if batch_stride is None:
            if self.kv_cache is None:
                raise ValueError("batch_stride is needed without a KVCache")
            batch_stride = self.kv_cache.batch_stride
        _lib.call("kva_legacy_decode_batched", self._workspace(), q_batch, k_cache_base,
                  v_cache_base, out_batch, seq_len, batch_size, batch_stride,
                  self.local_num_attention_heads, self.local_num_kv_heads, self._kva_stream)

    # ---- prefill (engine.py:3009-3139) -------------------------------------
    def _alloc_prefill_scratch(self, seq_len: int):
        """The prefill buffers of engine.py:3009-3041 this path uses
        (d_pf_hidden, d_pf_normed, d_pf_q, d_pf_q_gate, d_pf_attn_out), for an
        engine that does not allocate them itself."""
        if getattr(self, "_pf_seq_len", 0) >= seq_len:
            return
        for name in ("d_pf_hidden", "d_pf_normed", "d_pf_q", "d_pf_q_gate", "d_pf_attn_out"):
            if getattr(self, name, 0):
                self.device.free(getattr(self, name))
        h = self.config.hidden_size
        q_dim = self.local_num_attention_heads * self.config.head_dim
        self.d_pf_hidden = self.device.malloc(seq_len * h * 2)
        self.d_pf_normed = self.device.malloc(seq_len * h * 2)
        self.d_pf_q = self.device.malloc(seq_len * q_dim * 2)
        self.d_pf_q_gate = self.device.malloc(seq_len * q_dim * 2)
        self.d_pf_attn_out = self.device.malloc(seq_len * q_dim * 2)
        self._pf_seq_len = seq_len

    def _stacked_weights(self, lw) -> tuple[int, int]:
        """[Q; Q_gate] and [K; V] stacked weight bases (engine.py:1366-1378
        stack them at load and point q_weight / k_weight at the stack)."""
        h = self.config.hidden_size
        q_dim = self.local_num_attention_heads * self.config.head_dim
        kv_dim = self.local_num_kv_heads * self.config.head_dim
        wq = getattr(lw, "q_fused_weight", 0) or lw.q_weight
        wkv = getattr(lw, "kv_fused_weight", 0) or lw.k_weight
        if lw.q_gate_weight != wq + q_dim * h * 2 or lw.v_weight != wkv + kv_dim * h * 2:
            raise ValueError("_prefill_full_attention needs the stacked [Q; Q_gate] and [K; V] weights "
                             "of engine.py:1366-1378 (q_gate_weight right after q_weight, v_weight right "
                             "after k_weight)")
        return wq, wkv

    def _paged_kv(self, what: str) -> KVCache:
        if not isinstance(self.kv_cache, KVCache):
            raise ValueError(f"{what} needs a mi50grad_amd KVCache (the paged cache whose steps it appends to)")
        return self.kv_cache

    def _paged_step(self, layer_idx: int, n_new: int, lens: list[int], rope_pos: list[int] | None = None) -> None:
        """Begin the paged step of an engine step once, at its first
        full-attention layer: batch slots 0..len(lens)-1 hold lens[b] rows
        and append n_new each (RoPE positions rope_pos, default the slots).
        Later layers of the same engine step reuse it (every layer appends
        the same slots at the same positions); a layer seen again, or other
        lengths or positions, begin a new one."""
        kv = self.kv_cache
        key = (tuple(lens), n_new, tuple(rope_pos) if rope_pos is not None else None)
        if getattr(self, "_step_key", None) != key or layer_idx in self._step_layers:
            for b, n in enumerate(lens):
                kv.paged.set_len(b, n)
            pos = None if rope_pos is None else [p + i for p in rope_pos for i in range(n_new)]
            kv.paged.begin_step(list(range(len(lens))), [n_new] * len(lens), rope_pos=pos, stream=self._kva_stream)
            self._step_key = key
            self._step_layers = set()
        self._step_layers.add(layer_idx)

    def _prefill_full_attention(self, layer_idx: int, lw, seq_len: int):
        """Full-attention prefill of seq_len tokens of batch slot 0
        (engine.py:3043-3139), d_pf_hidden [seq_len, hidden] updated in place.

        Per token the engine's RMSNorm of the hidden state (its own kernel,
        as in the reference) into d_pf_normed; then, for all tokens at once
        through libkvattn: the Q/Q_gate/K/V projection with QK-norm + RoPE and
        the K/V append into the cache (kva_project_append), causal attention
        over the cache with the sigmoid gate the reference applies next
        (_launch_sigmoid_mul, engine.py:3120-3121) fused into its epilogue
        (kva_prefill_gated, same rounding), and the O-projection with the
        residual add into d_pf_hidden (kva_out_project, one rounding after
        the add where the reference's GEMM + residual_add round twice: the
        two differ by at most one fp16 ulp).  The chunk goes to slots [current_len,
        current_len + seq_len), attending causally over everything before
        it; the reference's prefill starts from an empty cache, which is the
        current_len = 0 case.  The caller sets current_len afterwards, as
        prefill_step does (engine.py:3283)."""
        self._paged_kv("_prefill_full_attention")
        cfg = self.config
        h = cfg.hidden_size
        q_dim = self.local_num_attention_heads * cfg.head_dim
        wq, wkv = self._stacked_weights(lw)
        for t in range(seq_len):
            self._launch_rmsnorm(self.d_pf_normed + t * h * 2, self.d_pf_hidden + t * h * 2, lw.attn_norm, h)
        self._paged_step(layer_idx, seq_len, [self.kv_cache.current_len])
        paged = self.kv_cache.paged
        layer = self.kv_cache._full_layer_slot(layer_idx)
        paged.project_append(layer, self.d_pf_normed, h, wq, wkv, lw.q_norm, lw.k_norm, self.d_cos,
                             self.d_sin, self.rope_rows, self.d_pf_q, q_gate_out=self.d_pf_q_gate,
                             stream=self._kva_stream)
        paged.prefill(layer, self.d_pf_q, self.d_pf_attn_out, stream=self._kva_stream, gate=self.d_pf_q_gate,
                      gate_stride=q_dim)
        paged.out_project(self.d_pf_attn_out, seq_len, q_dim, lw.o_weight, h, self.d_pf_hidden,
                          residual=self.d_pf_hidden, stream=self._kva_stream)

    # ---- decode (engine.py:1778-1876, 1943-2092) ------------------------------
    def _decode_full_attention(self, layer_idx: int, lw, position: int):
        """Full-attention decode of batch slot 0 (engine.py:1943-2092), FP16
        attention weights, d_hidden updated in place.

        The engine has RMS-normed the hidden state into d_normed.  Through
        libkvattn: the Q/Q_gate/K/V projection with QK-norm + RoPE at
        `position` and the K/V append into the cache row current_len
        (kva_project_append: Q -> d_q, Q_gate -> d_q_gate, K and V as
        projected -> d_kv_fused), decode attention over current_len + 1 rows
        with the sigmoid gate of _launch_sigmoid_mul (engine.py:2055-2056)
        fused into its epilogue (kva_decode_gated -> d_attn_out), and the
        O-projection (kva_out_project): with tp_size 1 into d_hidden with the
        residual add (engine.py:2083-2085), else into d_proj_out without it
        (engine.py:2086-2088, the all-reduce being the caller's).  The caller
        advances current_len after the step, as decode_step does
        (engine.py:1500)."""
        kv = self._paged_kv("_decode_full_attention")
        cfg = self.config
        h = cfg.hidden_size
        q_dim = self.local_num_attention_heads * cfg.head_dim
        wq, wkv = self._stacked_weights(lw)
        self._paged_step(layer_idx, 1, [kv.current_len], [position])
        paged = kv.paged
        layer = kv._full_layer_slot(layer_idx)
        st = self._kva_stream
        paged.project_append(layer, self.d_normed, h, wq, wkv, lw.q_norm, lw.k_norm, self.d_cos, self.d_sin,
                             self.rope_rows, self.d_q, q_gate_out=self.d_q_gate,
                             kv_out=getattr(self, "d_kv_fused", 0) or None, stream=st)
        paged.decode(layer, self.d_q, self.d_attn_out, stream=st, gate=self.d_q_gate, gate_stride=q_dim)
        if getattr(self, "tp_size", 1) <= 1:
            paged.out_project(self.d_attn_out, 1, q_dim, lw.o_weight, h, self.d_hidden, residual=self.d_hidden,
                              stream=st)
        else:
            paged.out_project(self.d_attn_out, 1, q_dim, lw.o_weight, h, self.d_proj_out, stream=st)

    def _decode_full_attention_batched(self, layer_idx: int, lw, position: int, batch_size: int):
        """Batched full-attention decode (engine.py:1778-1876): sequence b of
        batch_size is KV batch slot b, appends its row at `position` and
        attends over position + 1 rows, all in single launches instead of the
        reference's per-sequence loop: kva_project_append over the batch's
        rows of _d_normed_batch, kva_decode_gated, and kva_out_project of
        every row into _d_proj_out_batch with the residual _d_hidden_batch
        (engine.py:1872-1874).  Q, Q_gate and the attention output go to
        contiguous [batch, q_dim] buffers of the launchers' own, allocated
        once per batch size (the last one is also _d_attn_out_batch, the
        name the reference gives it)."""
        kv = self._paged_kv("_decode_full_attention_batched")
        cfg = self.config
        h = cfg.hidden_size
        q_dim = self.local_num_attention_heads * cfg.head_dim
        B = int(batch_size)
        if not 1 <= B <= kv.batch_size:
            raise ValueError(f"batch_size {B} outside the KVCache's {kv.batch_size} batch slots")
        wq, wkv = self._stacked_weights(lw)
        if getattr(self, "_kva_batch_bufs", (0,))[0] != B:
            for p in getattr(self, "_kva_batch_bufs", (0,))[1:]:
                self.device.free(p)
            self._kva_batch_bufs = (B, *(self.device.malloc(B * q_dim * 2) for _ in range(3)))
        _, d_q, d_gate, attn = self._kva_batch_bufs
        self._d_attn_out_batch = attn
        self._paged_step(layer_idx, 1, [int(position)] * B, [int(position)] * B)
        paged = kv.paged
        layer = kv._full_layer_slot(layer_idx)
        st = self._kva_stream
        paged.project_append(layer, self._d_normed_batch, h, wq, wkv, lw.q_norm, lw.k_norm, self.d_cos, self.d_sin,
                             self.rope_rows, d_q, q_gate_out=d_gate, stream=st)
        paged.decode(layer, d_q, attn, stream=st, gate=d_gate, gate_stride=q_dim)
        paged.out_project(attn, B, q_dim, lw.o_weight, h, self._d_proj_out_batch, residual=self._d_hidden_batch,
                          stream=st)

    # ---- decode launch cache (engine.py:3309-3555) ---------------------------
    def build_decode_launch_cache(self):
        """Per full-attention layer, the launches of the reference's decode
        launch cache that this path replaces, keyed like the reference:
        ``qknorm_q`` (params: d_q, q_norm, cos [2], sin [3], head_dim,
        half_rotary, eps), ``qknorm_k`` (the cache-write variant when direct
        KV write is on: d_k, k_norm, cos [2], sin [3], cache_dst [4], ...;
        else as qknorm_q) and ``decode_attn`` (d_q, k_cache, v_cache,
        d_attn_out, seq_len [4], num_heads, num_kv_heads).  Update the
        mutable values in place per step and launch with
        ``device.launch_cached(spec)`` or ``spec.launch()``.  Needs the
        engine's ``layers``, ``d_q``, ``d_k`` and ``d_attn_out``."""
        cfg = self.config
        half = self.rotary_dim // 2
        eps = cfg.rms_norm_eps
        u64, u32, f32 = ctypes.c_uint64, ctypes.c_uint32, ctypes.c_float
        out = {}
        for layer_idx, lw in enumerate(self.layers):
            if getattr(lw, "layer_type", "full_attention") != "full_attention":
                continue
            lc = {"qknorm_q": KvaLaunchSpec(
                "qknorm", [u64(self.d_q), u64(lw.q_norm), u64(self.d_cos), u64(self.d_sin), u32(cfg.head_dim),
                           u32(half), f32(eps)], grid=(self.local_num_attention_heads, 1, 1),
                num_heads=self.local_num_attention_heads)}
            if self._direct_kv_write and self._qknorm_rope_cachew:
                k0 = self.kv_cache.layer_k_ptr(layer_idx)
                lc["qknorm_k"] = KvaLaunchSpec(
                    "qknorm_cachew", [u64(self.d_k), u64(lw.k_norm), u64(self.d_cos), u64(self.d_sin), u64(k0),
                                      u32(cfg.head_dim), u32(half), f32(eps)],
                    grid=(self.local_num_kv_heads, 1, 1), num_heads=self.local_num_kv_heads)
                lc["_k_cache_base"] = k0
            else:
                lc["qknorm_k"] = KvaLaunchSpec(
                    "qknorm", [u64(self.d_k), u64(lw.k_norm), u64(self.d_cos), u64(self.d_sin), u32(cfg.head_dim),
                               u32(half), f32(eps)], grid=(self.local_num_kv_heads, 1, 1),
                    num_heads=self.local_num_kv_heads)
            lc["decode_attn"] = KvaLaunchSpec(
                "decode", [u64(self.d_q), u64(self.kv_cache.layer_k_ptr(layer_idx)),
                           u64(self.kv_cache.layer_v_ptr(layer_idx)), u64(self.d_attn_out), u32(1),
                           u32(self.local_num_attention_heads), u32(self.local_num_kv_heads)],
                grid=(self.local_num_attention_heads, 1, 1), workspace=self._workspace())
            out[layer_idx] = lc
        self._decode_launch_cache = out
        return out

    # ---- speculative rollback (tp_engine.py:1673-1687) -----------------------
    def rollback_kv_cache(self, num_tokens: int):
        """Drop the last num_tokens rows: current_len = max(0, current_len -
        num_tokens), as the reference does; the paged lengths of every batch
        slot follow, so later paged steps append at the rolled-back slot.
        (Compacting accepted tree rows is kva_rollback / TreeVerifyStep.)"""
        kv = self.kv_cache
        kv.current_len = max(0, kv.current_len - int(num_tokens))
        if isinstance(kv, KVCache):
            for b in range(kv.batch_size):
                if kv.paged.seq_len(b) > kv.current_len:
                    kv.paged.set_len(b, kv.current_len)


# Methods install() puts on an engine instance (the reference defines all of
# them in InferenceEngine's class body or in the speculative engine).
ENGINE_METHODS = (
    "_launch_qknorm_rope", "_launch_qknorm_rope_cachew", "_launch_decode_attn_256",
    "_launch_decode_attn_256_gated", "_launch_decode_attn_256_batched", "_prefill_full_attention",
    "_decode_full_attention", "_decode_full_attention_batched",
    "set_direct_kv_write", "build_decode_launch_cache", "rollback_kv_cache",
    # helpers the methods above call
    "_rope_rows", "_workspace", "_stacked_weights", "_paged_kv", "_paged_step",
)


def _setup(obj, max_seq_len: int, tp_size: int = 1) -> None:
    """State the launchers need on `obj` (a FullAttentionLaunchers or an
    installed engine): head counts, flags, RoPE tables (the reference's own
    recipe, so the bits match engine.py:1025-1046), and a split-K workspace
    of its own when there is no KVCache, made here once so that no decode
    call allocates or runs unsplit."""
    cfg = obj.config
    obj.local_num_attention_heads = cfg.num_attention_heads // tp_size
    obj.local_num_kv_heads = cfg.num_key_value_heads // tp_size
    obj._qknorm_rope_fused = True
    obj._qknorm_rope_cachew = True
    obj._direct_kv_write = getattr(obj, "_direct_kv_write", False)
    FullAttentionLaunchers._init_rope_tables(obj, max_seq_len)
    if not isinstance(getattr(obj, "kv_cache", None), KVCache):
        obj._kva_ws = PagedKVCache(n_layers=1, max_seqs=1, max_blocks=1, max_blocks_per_seq=1,
                                   max_step_tokens=16, num_heads=obj.local_num_attention_heads,
                                   num_kv_heads=obj.local_num_kv_heads, head_dim=cfg.head_dim,
                                   rotary_dim=int(cfg.head_dim * cfg.partial_rotary_factor),
                                   eps=cfg.rms_norm_eps)


def bind_methods(engine, names=ENGINE_METHODS, gemv: bool = False) -> None:
    """Bind the launchers' methods onto `engine` as instance attributes, which
    take precedence over the methods its class defines.  With gemv=True the
    engine's _launch_gemv_fp16 is replaced too (every GEMV call site then
    goes to kva_out_project, so K must be a multiple of 512)."""
    for name in tuple(names) + (("_launch_gemv_fp16",) if gemv else ()):
        setattr(engine, name, types.MethodType(getattr(FullAttentionLaunchers, name), engine))


def rope_table_rows(engine, max_seq_len: int | None = None) -> int:
    """Rows the RoPE tables of an installed engine need: every position any
    of its callers can address.  That is the largest of `max_seq_len`, the
    max_seq_len of the engine's KV cache (the reference's own KVCache has
    one too, engine.py:91) or of the engine itself, and the rows of tables
    already built (rope_rows): reference code indexes engine.d_cos directly
    (engine.py:2741; tp_engine.py:169, 341, 2933) without a bounds check, so
    the tables must never shrink.  2048 (the engine's default max_seq_len,
    engine.py:475) when none of these is known."""
    cands = (max_seq_len, getattr(getattr(engine, "kv_cache", None), "max_seq_len", None),
             getattr(engine, "max_seq_len", None), getattr(engine, "rope_rows", None))
    rows = max((int(c) for c in cands if c), default=0)
    return rows if rows > 0 else 2048


def install(engine, kv_cache: KVCache | None = None, max_seq_len: int | None = None, stream=None,
            gemv: bool = False):
    """Route an engine instance's full-attention calls through libkvattn.

    `engine` is the reference's InferenceEngine (or anything with its
    ``config``, ``device`` and, for prefill and the launch cache, its
    buffers and ``layers``).  `kv_cache` (a drop-in ``KVCache``) replaces
    ``engine.kv_cache`` when given.  With the engine's own reference
    KVCache kept, the contiguous-cache launches still work (on a split-K
    workspace made here, once) but the paged ones (_prefill_full_attention)
    refuse.  Launches go to `stream` (None: the legacy default stream).
    The RoPE tables are rebuilt with rope_table_rows(engine, max_seq_len)
    rows and the engine's previous tables freed.  Returns the engine."""
    if kv_cache is not None:
        engine.kv_cache = kv_cache
    engine._kva_stream = stream
    _setup(engine, rope_table_rows(engine, max_seq_len), getattr(engine, "tp_size", 1))
    bind_methods(engine, gemv=gemv)
    return engine
