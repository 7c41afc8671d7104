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
