"""GPU: the reference-compatible surface used the way engine.py uses it.

Mirrors InferenceEngine._decode_full_attention's direct-KV-write flow
(engine.py:2029-2053) for several decode steps and two batch slots: q norm+RoPE
in place, k norm+RoPE written into the slot from get_kv_ptr, V copied into the
cache, decode over layer_k_ptr/layer_v_ptr with seq_len = current_len + 1,
advance().  Also the batched launcher and the attribute contract of KVCache
(engine.py:88-117, tests/test_batch_kv_cache.py:41-84).
"""
import numpy as np
import pytest

from mi50grad_amd.attention import FullAttentionLaunchers
from mi50grad_amd.config import AttnConfig
from mi50grad_amd.kv_cache import KVCache
from oracle import kvattn_oracle as orc

from gpu_helpers import HKV, H, D, max_err, say

pytestmark = pytest.mark.gpu


def test_kvcache_attributes(device):
    cfg = AttnConfig(num_hidden_layers=8)
    kv = KVCache(cfg, 512, device, tp_size=1, batch_size=4)
    assert kv.num_full_layers == 2 and kv.full_layer_indices == [3, 7]
    assert kv.pos_stride == HKV * D * 2 == kv.pos_size_per_batch
    assert kv.batch_stride == 512 * kv.pos_stride
    for layer in kv.full_layer_indices:
        k0 = kv.layer_k_ptr(layer, 0)
        for b in range(4):
            assert kv.layer_k_ptr(layer, b) - k0 == b * kv.batch_stride
            assert kv.get_kv_ptr(layer, 17, b)[0] == k0 + b * kv.batch_stride + 17 * kv.pos_stride
    assert kv.layer_k_ptr(7, 0) - kv.layer_k_ptr(3, 0) == 4 * kv.batch_stride
    kv.cleanup()


def test_engine_style_decode_steps(device):
    say("engine-style decode steps")
    rng = np.random.default_rng(77)
    cfg = AttnConfig(num_hidden_layers=4)        # one full-attention layer: index 3
    max_seq, batch, steps = 256, 2, 5
    kv = KVCache(cfg, max_seq, device, batch_size=batch)
    eng = FullAttentionLaunchers(cfg, device, max_seq_len=max_seq, kv_cache=kv)
    eng.set_direct_kv_write(True)
    layer = 3
    qw = (1 + 0.02 * rng.standard_normal(D)).astype(np.float16)
    kw = (1 + 0.02 * rng.standard_normal(D)).astype(np.float16)
    d_qw, d_kw = device.array(qw), device.array(kw)
    # A prefix of 40 random rows per slot, written with append_kv (H2D).
    prefix = 40
    hist_k = [rng.standard_normal((prefix, HKV, D)).astype(np.float16) for _ in range(batch)]
    hist_v = [rng.standard_normal((prefix, HKV, D)).astype(np.float16) for _ in range(batch)]
    for t in range(prefix):
        for b in range(batch):
            kv.append_kv(layer, hist_k[b][t].tobytes(), hist_v[b][t].tobytes(), batch_idx=b)
        kv.advance()
    cos, sin = orc.rope_tables(max_seq)
    for step in range(steps):
        pos = kv.current_len
        for b in range(batch):
            q = rng.standard_normal((H, D)).astype(np.float16)
            k = rng.standard_normal((HKV, D)).astype(np.float16)
            v = rng.standard_normal((HKV, D)).astype(np.float16)
            dq, dk, dv = device.array(q), device.array(k), device.array(v)
            out = device.empty((H, D), np.float16)
            k_slot, v_slot = kv.get_kv_ptr(layer, pos, b)
            device.memcpy_d2d(v_slot, dv.ptr, v.nbytes)                       # V GEMV -> cache slot
            eng._launch_qknorm_rope(dq.ptr, d_qw.ptr, pos, H, D)
            eng._launch_qknorm_rope_cachew(dk.ptr, d_kw.ptr, pos, HKV, D, k_slot)
            eng._launch_decode_attn_256(out.ptr, dq.ptr, kv.layer_k_ptr(layer, b),
                                        kv.layer_v_ptr(layer, b), kv.current_len + 1)
            device.synchronize()
            qn = orc.qknorm_rope_exact(q, qw, np.repeat(cos[pos:pos + 1], H, 0), np.repeat(sin[pos:pos + 1], H, 0))
            kn = orc.qknorm_rope_exact(k, kw, np.repeat(cos[pos:pos + 1], HKV, 0),
                                       np.repeat(sin[pos:pos + 1], HKV, 0))
            assert np.array_equal(dq.numpy().view(np.uint16), qn.view(np.uint16))
            assert np.array_equal(dk.numpy().view(np.uint16), kn.view(np.uint16))
            hist_k[b] = np.concatenate([hist_k[b], kn[None]])
            hist_v[b] = np.concatenate([hist_v[b], v[None]])
            exp = orc.attention_fp32(qn[None], hist_k[b], hist_v[b])[0]
            assert max_err(out.numpy(), exp) <= 2e-3, (step, b)
        kv.advance()
    # Cache rows equal the history for both slots (bit-exact appends).
    n = kv.current_len
    for b in range(batch):
        rows = np.frombuffer(device.download(kv.layer_k_ptr(layer, b), n * kv.pos_stride),
                             dtype=np.float16).reshape(n, HKV, D)
        assert np.array_equal(rows.view(np.uint16), hist_k[b].view(np.uint16))
    # Batched launcher over both slots at the shared length.
    q = rng.standard_normal((batch, H, D)).astype(np.float16)
    dq, out = device.array(q), device.empty((batch, H, D), np.float16)
    eng._launch_decode_attn_256_batched(out.ptr, dq.ptr, kv.layer_k_ptr(layer, 0), kv.layer_v_ptr(layer, 0),
                                        n, batch)
    device.synchronize()
    exp = np.stack([orc.attention_fp32(q[b:b + 1], hist_k[b], hist_v[b])[0] for b in range(batch)])
    assert max_err(out.numpy(), exp) <= 2e-3
    kv.cleanup()


def test_gemv_fp16_o_projection(device):
    """engine.py:2083-2085: d_hidden = fp16(o_proj(attn) + d_hidden) in place
    through the reference-named launcher, then without the residual."""
    say("engine-style O-projection GEMV")
    rng = np.random.default_rng(78)
    cfg = AttnConfig(num_hidden_layers=4)
    kv = KVCache(cfg, 64, device, batch_size=1)
    eng = FullAttentionLaunchers(cfg, device, max_seq_len=64, kv_cache=kv)
    q_dim, hidden = H * D, 512
    attn = rng.integers(-3, 4, q_dim).astype(np.float16)
    w = (rng.integers(-2, 3, (hidden, q_dim)) * 2.0 ** -7).astype(np.float16)
    h0 = (rng.integers(-64, 65, hidden) * 2.0 ** -3).astype(np.float16)
    d_attn, d_w, d_hid = device.array(attn), device.array(w), device.array(h0)
    eng._launch_gemv_fp16(d_hid.ptr, d_attn.ptr, d_w.ptr, q_dim, hidden, residual=d_hid.ptr)
    d_out = device.empty((hidden,), np.float16)
    eng._launch_gemv_fp16(d_out.ptr, d_attn.ptr, d_w.ptr, q_dim, hidden)
    device.synchronize()
    exp = orc.out_project(attn[None], w, h0[None])[0]
    assert np.array_equal(d_hid.numpy().view(np.uint16), exp.view(np.uint16))
    assert np.array_equal(d_out.numpy().view(np.uint16), orc.out_project(attn[None], w)[0].view(np.uint16))
    kv.cleanup()


# ---- the engine surface through install(): prefill, launch cache, rollback --
class _Layer:
    def __init__(self, layer_type):
        self.layer_type = layer_type


class StubEngine:
    """What install() and the reference-named methods read from an
    InferenceEngine: config, device, kv_cache, layers with the stacked
    attention weights of engine.py:1366-1378, the decode buffers (d_q, d_k,
    d_attn_out), the prefill buffers, and the engine's own hidden-state
    RMSNorm (outside this path; here numpy on the host)."""

    _alloc_prefill_scratch = FullAttentionLaunchers._alloc_prefill_scratch

    def __init__(self, cfg, device, kv, rng, hidden):
        self.config, self.device, self.kv_cache = cfg, device, kv
        self.host = {}
        self.layers = []
        q_dim, kv_dim = H * D, HKV * D
        for i in range(cfg.num_hidden_layers):
            lw = _Layer("full_attention" if cfg.is_full_attention(i) else "linear_attention")
            if lw.layer_type == "full_attention":
                wq = (rng.standard_normal((2 * q_dim, hidden), dtype=np.float32) * hidden ** -0.5).astype(np.float16)
                wkv = (rng.standard_normal((2 * kv_dim, hidden), dtype=np.float32) * hidden ** -0.5).astype(np.float16)
                wo = (rng.standard_normal((hidden, q_dim), dtype=np.float32) * q_dim ** -0.5).astype(np.float16)
                qn = (1 + 0.02 * rng.standard_normal(D)).astype(np.float16)
                kn = (1 + 0.02 * rng.standard_normal(D)).astype(np.float16)
                an = (1 + 0.1 * rng.standard_normal(hidden)).astype(np.float16)
                self.host[i] = dict(wq=wq, wkv=wkv, wo=wo, qn=qn, kn=kn, an=an)
                lw.q_fused_weight = device.array(wq).ptr
                lw.q_weight, lw.q_gate_weight = lw.q_fused_weight, lw.q_fused_weight + q_dim * hidden * 2
                lw.kv_fused_weight = device.array(wkv).ptr
                lw.k_weight, lw.v_weight = lw.kv_fused_weight, lw.kv_fused_weight + kv_dim * hidden * 2
                lw.o_weight = device.array(wo).ptr
                lw.q_norm, lw.k_norm, lw.attn_norm = device.array(qn).ptr, device.array(kn).ptr, device.array(an).ptr
            self.layers.append(lw)
        # The decode buffers of engine.py:1063-1077: [Q | Q_gate] and [K | V]
        # contiguous, d_q / d_q_gate / d_k pointing into them.
        self.d_q_fused = device.malloc(2 * q_dim * 2)
        self.d_q, self.d_q_gate = self.d_q_fused, self.d_q_fused + q_dim * 2
        self.d_kv_fused = device.malloc(2 * kv_dim * 2)
        self.d_k = self.d_kv_fused
        self.d_attn_out = device.malloc(q_dim * 2)
        self.d_normed = device.malloc(hidden * 2)
        self.d_hidden = device.malloc(hidden * 2)
        self.d_proj_out = device.malloc(hidden * 2)
        self.tp_size = 1

    def _launch_rmsnorm(self, dst, src, weight, dim):
        x = np.frombuffer(self.device.download(src, dim * 2), np.float16).astype(np.float32)
        w = np.frombuffer(self.device.download(weight, dim * 2), np.float16).astype(np.float32)
        y = (x / np.sqrt(np.mean(x * x) + 1e-6) * w).astype(np.float16)
        self.device.upload(dst, y.tobytes())

    # The reference names, defined in the class body as InferenceEngine does.
    def _prefill_full_attention(self, *a):
        raise AssertionError("reference prefill called")

    _launch_qknorm_rope = _launch_decode_attn_256 = build_decode_launch_cache = rollback_kv_cache = \
        _decode_full_attention = _decode_full_attention_batched = _prefill_full_attention


def _ulp_close(got, exp, ulps=1):
    """Within `ulps` fp16 ulps of each expected element, plus 2^-12 for the
    fp32 accumulation of the projection (its error is absolute: a sum that
    cancels to a tiny value is not known to a few of ITS ulps)."""
    e = np.abs(np.asarray(exp, np.float32))
    return np.all(np.abs(np.asarray(got, np.float32) - exp.astype(np.float32)) <= ulps * np.maximum(e, 2.0 ** -14) * 2.0 ** -10 + 2.0 ** -12)


def _row_close(got, exp, ulps=4):
    """Normalised + rotated head rows: each element within `ulps` ulps of
    its row's largest element.  A projected value one ulp off moves the
    row's RMS and, through the rotation a*c - b*s, its partner element by an
    amount set by the pair's size, not by the (possibly cancelled) result."""
    g = np.asarray(got, np.float32)
    e = np.asarray(exp, np.float32)
    scale = np.max(np.abs(e), axis=-1, keepdims=True)
    return np.all(np.abs(g - e) <= ulps * scale * 2.0 ** -10 + 2.0 ** -12)


def test_installed_prefill_full_attention(device):
    """_prefill_full_attention (engine.py:3043-3139) on an installed engine:
    two full-attention layers (3 and 7), an 80-token prefill (two producer
    launch pairs) then a 48-token chunk after it.  Per layer: Q, Q_gate and
    the cache rows within the projection's rounding of
    oracle.project_append on the engine's normed rows (gate and V within
    one ulp, normalised + rotated Q and K within 4 ulps of each head row's
    largest element); the gated attention within 2e-3 of the
    oracle's causal attention over every row so far followed by the gate;
    the hidden rows within one ulp of oracle.out_project plus the residual."""
    from mi50grad_amd import attention as att
    say("installed _prefill_full_attention")
    rng = np.random.default_rng(81)
    cfg = AttnConfig(num_hidden_layers=8, hidden_size=512)
    kv = KVCache(cfg, 256, device, batch_size=1)
    eng = att.install(StubEngine(cfg, device, kv, rng, 512))
    assert eng._prefill_full_attention.__func__ is FullAttentionLaunchers._prefill_full_attention
    h, q_dim = 512, H * D
    cos, sin = orc.rope_tables(256)
    hist = {li: ([], []) for li in kv.full_layer_indices}
    for seq_len in (80, 48):
        start = kv.current_len
        pos = np.arange(start, start + seq_len)
        eng._alloc_prefill_scratch(seq_len)
        x0 = rng.standard_normal((seq_len, h), dtype=np.float32).astype(np.float16)
        device.upload(eng.d_pf_hidden, x0.tobytes())
        for li in kv.full_layer_indices:
            w = eng.host[li]
            before = np.frombuffer(device.download(eng.d_pf_hidden, seq_len * h * 2), np.float16).reshape(seq_len, h)
            eng._prefill_full_attention(li, eng.layers[li], seq_len)
            device.synchronize()
            rd = lambda p, shape: np.frombuffer(device.download(p, int(np.prod(shape)) * 2), np.float16).reshape(shape)
            normed = rd(eng.d_pf_normed, (seq_len, h))
            q_o, g_o, _, k_o, v_o = orc.project_append(normed, w["wq"], w["wkv"], w["qn"], w["kn"], cos[pos], sin[pos])
            q_g, g_g = rd(eng.d_pf_q, (seq_len, H, D)), rd(eng.d_pf_q_gate, (seq_len, H, D))
            assert _row_close(q_g, q_o) and _ulp_close(g_g, g_o), (seq_len, li)
            ks, vs = kv.paged.gather(kv._full_layer_slot(li), 0, start + seq_len)
            assert _row_close(ks[start:], k_o) and _ulp_close(vs[start:], v_o), (seq_len, li)
            hist[li][0].append(ks[start:])
            hist[li][1].append(vs[start:])
            kall, vall = np.concatenate(hist[li][0]), np.concatenate(hist[li][1])
            att_o = orc.chunk_attention(q_g, kall, vall, start)
            out_g = rd(eng.d_pf_attn_out, (seq_len, H, D))
            assert max_err(out_g, orc.sigmoid_gate(att_o.astype(np.float16), g_g)) <= 2e-3, (seq_len, li)
            x_exp = orc.out_project(out_g.reshape(seq_len, q_dim), w["wo"], before)
            assert _ulp_close(rd(eng.d_pf_hidden, (seq_len, h)), x_exp), (seq_len, li)
        kv.current_len = start + seq_len  # prefill_step's bookkeeping (engine.py:3283)
    kv.cleanup()


def _fill_slot(device, kv, layer_idx, b, k, v):
    """Rows [0, len(k)) of batch slot b: the KVCache's slot rows are
    contiguous (consecutive pages), as in the reference layout."""
    device.upload(kv.layer_k_ptr(layer_idx, b), k.tobytes())
    device.upload(kv.layer_v_ptr(layer_idx, b), v.tobytes())


def test_installed_decode_full_attention(device):
    """_decode_full_attention (engine.py:1943-2092) on an installed engine:
    two full-attention layers over a 40-row history, five decode steps at
    positions current_len (the caller advancing current_len after each,
    engine.py:1500).  Per layer and step, against the oracle chain
    project_append -> attention_fp32 -> sigmoid_gate -> out_project: Q and
    the appended K row within 4 ulps of each head row's largest element, Q_gate
    and the V row within one ulp (the projection's rounding), the gated
    attention within 2e-3 over every row so far, d_hidden within one ulp of
    the O-projection plus the residual (engine.py:2083-2085)."""
    from mi50grad_amd import attention as att
    say("installed _decode_full_attention")
    rng = np.random.default_rng(85)
    cfg = AttnConfig(num_hidden_layers=8, hidden_size=512)
    kv = KVCache(cfg, 128, device, batch_size=1)
    eng = att.install(StubEngine(cfg, device, kv, rng, 512))
    assert eng._decode_full_attention.__func__ is FullAttentionLaunchers._decode_full_attention
    h, q_dim = 512, H * D
    cos, sin = orc.rope_tables(128)
    prefix = 40
    for li in kv.full_layer_indices:
        k0 = rng.standard_normal((prefix, HKV, D), dtype=np.float32).astype(np.float16)
        v0 = rng.standard_normal((prefix, HKV, D), dtype=np.float32).astype(np.float16)
        _fill_slot(device, kv, li, 0, k0, v0)
    kv.current_len = prefix
    rd = lambda p, shape: np.frombuffer(device.download(p, int(np.prod(shape)) * 2), np.float16).reshape(shape)
    for step in range(5):
        pos = kv.current_len
        for li in kv.full_layer_indices:
            w = eng.host[li]
            normed = rng.standard_normal((1, h), dtype=np.float32).astype(np.float16)
            before = rng.standard_normal((1, h), dtype=np.float32).astype(np.float16)
            device.upload(eng.d_normed, normed.tobytes())
            device.upload(eng.d_hidden, before.tobytes())
            eng._decode_full_attention(li, eng.layers[li], pos)
            device.synchronize()
            q_o, g_o, _, k_o, v_o = orc.project_append(normed, w["wq"], w["wkv"], w["qn"], w["kn"], cos[[pos]],
                                                       sin[[pos]])
            q_g, g_g = rd(eng.d_q, (1, H, D)), rd(eng.d_q_gate, (1, H, D))
            assert _row_close(q_g, q_o) and _ulp_close(g_g, g_o), (step, li)
            ks, vs = kv.paged.gather(kv._full_layer_slot(li), 0, pos + 1)
            assert _row_close(ks[pos:], k_o) and _ulp_close(vs[pos:], v_o), (step, li)
            out_g = rd(eng.d_attn_out, (1, H, D))
            exp = orc.sigmoid_gate(orc.attention_fp32(q_g, ks, vs).astype(np.float16), g_g)
            assert max_err(out_g, exp) <= 2e-3, (step, li)
            x_exp = orc.out_project(out_g.reshape(1, q_dim), w["wo"], before)
            assert _ulp_close(rd(eng.d_hidden, (1, h)), x_exp), (step, li)
        kv.advance()
    kv.cleanup()


def test_installed_decode_full_attention_batched(device):
    """_decode_full_attention_batched (engine.py:1778-1876): three batch
    slots with their own 37-row histories append at position 37 and attend
    over 38 rows, two steps, each stage against the oracle as above, the
    O-projection of every row into _d_proj_out_batch with the residual
    _d_hidden_batch (engine.py:1872-1874)."""
    from mi50grad_amd import attention as att
    say("installed _decode_full_attention_batched")
    rng = np.random.default_rng(86)
    cfg = AttnConfig(num_hidden_layers=4, hidden_size=512)
    B, P, h, q_dim = 3, 37, 512, H * D
    kv = KVCache(cfg, 64, device, batch_size=4)
    eng = att.install(StubEngine(cfg, device, kv, rng, 512))
    eng._d_normed_batch = device.malloc(B * h * 2)
    eng._d_hidden_batch = device.malloc(B * h * 2)
    eng._d_proj_out_batch = device.malloc(B * h * 2)
    cos, sin = orc.rope_tables(64)
    li = kv.full_layer_indices[0]
    w = eng.host[li]
    for b in range(B):
        _fill_slot(device, kv, li, b, rng.standard_normal((P, HKV, D), dtype=np.float32).astype(np.float16),
                   rng.standard_normal((P, HKV, D), dtype=np.float32).astype(np.float16))
    rd = lambda p, shape: np.frombuffer(device.download(p, int(np.prod(shape)) * 2), np.float16).reshape(shape)
    for position in (P, P + 1):
        normed = rng.standard_normal((B, h), dtype=np.float32).astype(np.float16)
        hid = rng.standard_normal((B, h), dtype=np.float32).astype(np.float16)
        device.upload(eng._d_normed_batch, normed.tobytes())
        device.upload(eng._d_hidden_batch, hid.tobytes())
        eng._decode_full_attention_batched(li, eng.layers[li], position, B)
        device.synchronize()
        pos = [position] * B
        q_o, g_o, _, k_o, v_o = orc.project_append(normed, w["wq"], w["wkv"], w["qn"], w["kn"], cos[pos], sin[pos])
        _, d_q, d_gate, d_attn = eng._kva_batch_bufs
        q_g, g_g = rd(d_q, (B, H, D)), rd(d_gate, (B, H, D))
        assert _row_close(q_g, q_o) and _ulp_close(g_g, g_o), position
        out_g = rd(d_attn, (B, H, D))
        for b in range(B):
            ks, vs = kv.paged.gather(kv._full_layer_slot(li), b, position + 1)
            assert _row_close(ks[position:], k_o[b:b + 1]) and _ulp_close(vs[position:], v_o[b:b + 1]), (position, b)
            exp = orc.sigmoid_gate(orc.attention_fp32(q_g[b:b + 1], ks, vs).astype(np.float16), g_g[b:b + 1])
            assert max_err(out_g[b:b + 1], exp) <= 2e-3, (position, b)
        x_exp = orc.out_project(out_g.reshape(B, q_dim), w["wo"], hid)
        assert _ulp_close(rd(eng._d_proj_out_batch, (B, h)), x_exp), position
        assert np.array_equal(rd(eng._d_hidden_batch, (B, h)).view(np.uint16), hid.view(np.uint16))
    kv.cleanup()


def test_decode_launch_cache_and_rollback(device):
    """build_decode_launch_cache (engine.py:3309-3555): per step the caller
    moves cos/sin (params 2, 3), the K slot (qknorm_k params 4) and seq_len
    (decode_attn params 4) in place and launches with device.launch_cached,
    V going to its slot directly (engine.py:2012-2018); outputs against the
    oracle.  Then rollback_kv_cache(2) (tp_engine.py:1673-1687) and a step
    that overwrites the dropped rows must see the truncated history."""
    from mi50grad_amd import attention as att
    say("decode launch cache + rollback_kv_cache")
    rng = np.random.default_rng(83)
    cfg = AttnConfig(num_hidden_layers=4, hidden_size=512)
    kv = KVCache(cfg, 128, device, batch_size=1)
    eng = att.install(StubEngine(cfg, device, kv, rng, 512))
    eng.set_direct_kv_write(True)
    lc = eng.build_decode_launch_cache()
    assert list(lc) == [3] and {"qknorm_q", "qknorm_k", "decode_attn"} <= set(lc[3])
    w = eng.host[3]
    cos, sin = orc.rope_tables(128)
    hk, hv = [], []
    for step in range(12):
        if step == 9:
            eng.rollback_kv_cache(2)
            del hk[-2:], hv[-2:]
            assert kv.current_len == 7
        pos = kv.current_len
        q = rng.standard_normal((H, D)).astype(np.float16)
        k = rng.standard_normal((HKV, D)).astype(np.float16)
        v = rng.standard_normal((HKV, D)).astype(np.float16)
        device.upload(eng.d_q, q.tobytes())
        device.upload(eng.d_k, k.tobytes())
        k_slot, v_slot = kv.get_kv_ptr(3, pos)
        device.upload(v_slot, v.tobytes())
        off = pos * (eng.rotary_dim // 2) * 2
        for name in ("qknorm_q", "qknorm_k"):
            lc[3][name].params[2].value = eng.d_cos + off
            lc[3][name].params[3].value = eng.d_sin + off
        lc[3]["qknorm_k"].params[4].value = k_slot
        lc[3]["decode_attn"].params[4].value = pos + 1
        for name in ("qknorm_q", "qknorm_k", "decode_attn"):
            device.launch_cached(lc[3][name])
        device.synchronize()
        qn = orc.qknorm_rope_exact(q, w["qn"], np.repeat(cos[pos:pos + 1], H, 0), np.repeat(sin[pos:pos + 1], H, 0))
        kn = orc.qknorm_rope_exact(k, w["kn"], np.repeat(cos[pos:pos + 1], HKV, 0), np.repeat(sin[pos:pos + 1], HKV, 0))
        hk.append(kn)
        hv.append(v)
        out = np.frombuffer(device.download(eng.d_attn_out, H * D * 2), np.float16).reshape(H, D)
        assert max_err(out, orc.attention_fp32(qn[None], np.stack(hk), np.stack(hv))[0]) <= 2e-3, step
        kv.advance()
    kv.cleanup()


def test_gemv_fp16_lm_head_shape(device):
    """_launch_gemv_fp16 with an lm_head-like output width (the reference's
    vocab, 248320 rows) for one token: bit-exact on fp32-exact inputs."""
    say("GEMV with vocab-wide output")
    rng = np.random.default_rng(84)
    cfg = AttnConfig(num_hidden_layers=4)
    eng = FullAttentionLaunchers(cfg, device, max_seq_len=64)
    K, N = 512, 248320
    x = rng.integers(-3, 4, K).astype(np.float16)
    w = (rng.integers(-2, 3, (N, K)) * 2.0 ** -7).astype(np.float16)
    dx, dw, dy = device.array(x), device.array(w), device.empty((N,), np.float16)
    eng._launch_gemv_fp16(dy.ptr, dx.ptr, dw.ptr, K, N)
    device.synchronize()
    assert np.array_equal(dy.numpy().view(np.uint16), orc.out_project(x[None], w)[0].view(np.uint16))
    with pytest.raises(ValueError):
        eng._launch_gemv_fp16(dy.ptr, dx.ptr, dw.ptr, 500, N)


def test_tree_attention_mask_drives_tree_verify(device):
    """A TreeAttentionMask (tree_attention.py:148-268) built from the
    reference's classes gives kva_step_begin its tree bits; tree verify over
    its topology matches the oracle's masked attention."""
    from mi50grad_amd import tree as tr
    from gpu_helpers import build_cache
    say("TreeAttentionMask -> tree verify")
    rng = np.random.default_rng(85)
    topo = tr.build_complete_binary_tree(1000, 2)
    par = topo.parents()
    lengths = [300, 47]
    T = topo.get_tree_size()
    ids = [list(range(0, 20)), list(range(20, 24))]
    cache, kr, vr = build_cache([L + T for L in lengths], ids, extra_rows=0, rng=rng)
    for b, L in enumerate(lengths):
        cache.set_len(b, L)
    masks = [tr.TreeAttentionMask(topo, kv_len=L) for L in lengths]
    q = rng.standard_normal((2 * T, H, D), dtype=np.float32).astype(np.float16)
    dq, out = device.array(q), device.empty((2 * T, H, D), np.float16)
    cache.begin_step([0, 1], [T, T], tree_bits=masks[0].tree_bits() + masks[1].tree_bits())
    cache.tree_verify(0, dq, out)
    device.synchronize()
    got = out.numpy()
    for b, L in enumerate(lengths):
        s = slice(b * T, b * T + T)
        exp = orc.tree_attention(q[s], kr[0][b][:L], vr[0][b][:L], kr[0][b][L:], vr[0][b][L:], par)
        assert max_err(got[s], exp) <= 2e-3, b
    cache.destroy()
