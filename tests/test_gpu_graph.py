"""GPU: recorded steps (kva_graph_*) replay bit-identically to eager calls.

Two caches built from the same seed: one runs every step's per-layer
append + decode eagerly, the other records one step into a graph and replays
it for 20 more steps, with fresh inputs uploaded between replays (the eager
work and synchronizations between them), lengths crossing page boundaries
(so the decode's stream-K shape, derived on the device from the step plan,
changes under the recording) and a decode split set.  Every replayed step's
outputs and, at the end, every pool byte must equal the eager twin's, and
every replayed output is also compared with the oracle (attention over the
oracle's own copy of the rows within 2e-3; O-projection within one fp16 ulp
of ``orc.out_project`` on the replay's own gated rows).  Also: what
recording refuses, a replay whose step has another shape, and a
whole-sequence recording replayed past 64 pages (block ids beyond the step
plan's, read from the table).
"""
import numpy as np
import pytest

from mi50grad_amd._lib import KvaError
from mi50grad_amd.device import Stream
from oracle import kvattn_oracle as orc

from gpu_helpers import HKV, H, D, Tables, build_cache, expected_norm, max_err, say

pytestmark = pytest.mark.gpu
LAYERS = 3


def _twin(lengths, split, seed):
    ids, o = [], 0
    for L in lengths:
        n = (L + 40 + 15) // 16
        ids.append(list(range(o, o + n))[::-1])  # reversed: pages out of order
        o += n
    caches = []
    for _ in range(2):
        c, kr, vr = build_cache(lengths, ids, extra_rows=40, n_layers=LAYERS, rng=np.random.default_rng(seed))
        c.set_decode_split(split)
        caches.append(c)
    # The oracle's copy of every layer's rows, per sequence (appended to as
    # the steps run).
    hist = [[(list(kr[layer][b]), list(vr[layer][b])) for b in range(len(lengths))] for layer in range(LAYERS)]
    return caches, hist


@pytest.mark.parametrize("lengths,split,fused", [([14, 30], 0, False), ([200, 5, 77], 32, False),
                                                 ([14, 30], 0, True), ([200, 5, 77], 32, True)])
def test_graph_replay_matches_eager(device, lengths, split, fused):
    """fused: each layer is one kva_append_decode call (a single launch in
    the whole-sequence form at the automatic split; append + stream-K decode
    with the split set), recorded and replayed like the two-call form."""
    say(f"graph replay lengths={lengths} split={split} fused={fused}")
    _replay(device, lengths, split, fused, steps=21, same_outputs=True, other_shape=True)


@pytest.mark.parametrize("fused", [False, True])
def test_graph_whole_form_past_64_pages(device, fused):
    """A step recorded in the whole-sequence form (longest sequence 1021
    rows, 64 pages) keeps that form as the replays take the sequences past
    1024 rows: the walk then reads page 64, whose block id comes from the
    table rather than the step plan's 64 ids, and (fused) writes the new
    rows there.  The eager twin runs stream-K past 1024 rows, so replayed
    outputs are held to the oracle (2e-3) and the pools to the twin's bits."""
    say(f"graph replay past 64 pages fused={fused}")
    _replay(device, [1020, 300], 0, fused, steps=12, same_outputs=False, other_shape=False)


def _replay(device, lengths, split, fused, steps, same_outputs, other_shape):
    rng = np.random.default_rng(5)
    (eager, graphed), hist = _twin(lengths, split, seed=11)
    B = len(lengths)
    tables = Tables(device, max(512, max(lengths) + steps + 16))
    stream = Stream()
    h_qw = [(1 + 0.02 * rng.standard_normal(D)).astype(np.float16) for _ in range(LAYERS)]
    h_kw = [(1 + 0.02 * rng.standard_normal(D)).astype(np.float16) for _ in range(LAYERS)]
    qw = [device.array(w) for w in h_qw]
    kw = [device.array(w) for w in h_kw]

    def fresh(shape):
        return rng.standard_normal(shape, dtype=np.float32).astype(np.float16)

    # One set of device inputs and outputs per cache and layer; the graph
    # reads and writes the same buffers at every replay.
    bufs = []
    for _ in range(2):
        bufs.append([dict(q=device.empty((B, H, D), np.float16), k=device.empty((B, HKV, D), np.float16),
                          v=device.empty((B, HKV, D), np.float16), out=device.empty((B, H, D), np.float16))
                     for _ in range(LAYERS)])

    def upload(step_inputs):
        for which in range(2):
            for layer in range(LAYERS):
                for name in ("q", "k", "v"):
                    a = step_inputs[layer][name]
                    device.upload(bufs[which][layer][name].ptr, a.tobytes())

    def calls(cache, which, stream_h):
        for layer in range(LAYERS):
            b = bufs[which][layer]
            if fused:
                cache.append_decode(layer, b["q"], b["k"], b["v"], qw[layer], kw[layer], tables.d_cos,
                                    tables.d_sin, tables.rows, b["out"], stream=stream_h)
                continue
            cache.append(layer, b["q"], b["k"], b["v"], qw[layer], kw[layer], tables.d_cos, tables.d_sin,
                         tables.rows, stream=stream_h)
            cache.decode(layer, b["q"], b["out"], stream=stream_h)

    graph = None
    for step in range(steps):
        inputs = [dict(q=fresh((B, H, D)), k=fresh((B, HKV, D)), v=fresh((B, HKV, D))) for _ in range(LAYERS)]
        upload(inputs)
        device.synchronize()
        eager.begin_step(list(range(B)), [1] * B)
        calls(eager, 0, None)
        graphed.begin_step(list(range(B)), [1] * B, stream=stream.handle)
        if graph is None:
            graph = graphed.record_step(stream.handle)
            with pytest.raises(KvaError):  # the step cannot change while recording
                graphed.begin_step(list(range(B)), [1] * B, stream=stream.handle)
            with pytest.raises(KvaError):  # nor can a multi-query launch be recorded
                graphed.prefill(0, bufs[1][0]["q"], bufs[1][0]["out"], stream=stream.handle)
            calls(graphed, 1, stream.handle)
            graph.end()
        graph.launch()
        stream.synchronize()
        device.synchronize()
        pos = [L + step for L in lengths]
        for layer in range(LAYERS):
            got = bufs[1][layer]["out"].numpy()
            exp = bufs[0][layer]["out"].numpy()
            if same_outputs:
                assert np.array_equal(got.view(np.uint16), exp.view(np.uint16)), (step, layer)
            assert np.array_equal(bufs[1][layer]["q"].numpy().view(np.uint16),
                                  bufs[0][layer]["q"].numpy().view(np.uint16)), (step, layer)
            qn = expected_norm(inputs[layer]["q"], h_qw[layer], tables, pos)
            kn = expected_norm(inputs[layer]["k"], h_kw[layer], tables, pos)
            for b in range(B):
                hist[layer][b][0].append(kn[b])
                hist[layer][b][1].append(inputs[layer]["v"][b])
            ora = orc.decode_attention(qn, [np.stack(hist[layer][b][0]) for b in range(B)],
                                       [np.stack(hist[layer][b][1]) for b in range(B)])
            assert max_err(got, ora) <= 2e-3, (step, layer)
    for layer in range(LAYERS):
        ke, ve = eager.download_pools(layer)
        kg, vg = graphed.download_pools(layer)
        assert np.array_equal(ke.view(np.uint16), kg.view(np.uint16))
        assert np.array_equal(ve.view(np.uint16), vg.view(np.uint16))
    assert [graphed.seq_len(b) for b in range(B)] == [L + steps for L in lengths]
    if other_shape:  # a step of another shape is refused
        graphed.begin_step([0], [1], stream=stream.handle)
        with pytest.raises(KvaError):
            graph.launch()
    graph.destroy()
    stream.synchronize()
    stream.destroy()
    eager.destroy()
    graphed.destroy()


def test_graph_replay_project_append(device):
    """The producer path recorded too: per layer kva_project_append (fused
    projection + norm + RoPE + append), the gated decode, then the
    O-projection added into the hidden rows in place; one step recorded and
    replayed with fresh hidden states; every replay equals the eager twin
    bit for bit, and so do the pools at the end."""
    say("graph replay of project_append + gated decode")
    rng = np.random.default_rng(8)
    lengths, hidden = [30, 47, 3], 512
    (eager, graphed), hist = _twin(lengths, 0, seed=12)
    B = len(lengths)
    tables = Tables(device, 512)
    stream = Stream()

    def f16(shape, s=1.0):
        return (rng.standard_normal(shape, dtype=np.float32) * s).astype(np.float16)

    hw = [dict(wq=f16((2 * H * D, hidden), hidden ** -0.5), wkv=f16((2 * HKV * D, hidden), hidden ** -0.5),
               qw=(1 + 0.02 * rng.standard_normal(D)).astype(np.float16),
               kw=(1 + 0.02 * rng.standard_normal(D)).astype(np.float16),
               wo=f16((hidden, H * D), (H * D) ** -0.5)) for _ in range(LAYERS)]
    w = [{name: device.array(a) for name, a in p.items()} for p in hw]
    bufs = [[dict(x=device.empty((B, hidden), np.float16), q=device.empty((B, H, D), np.float16),
                  g=device.empty((B, H, D), np.float16), out=device.empty((B, H, D), np.float16))
             for _ in range(LAYERS)] for _ in range(2)]

    def calls(cache, which, stream_h):
        for layer in range(LAYERS):
            b, p = bufs[which][layer], w[layer]
            cache.project_append(layer, b["x"], hidden, p["wq"], p["wkv"], p["qw"], p["kw"], tables.d_cos,
                                 tables.d_sin, tables.rows, b["q"], b["g"], stream=stream_h)
            cache.decode(layer, b["q"], b["out"], stream=stream_h, gate=b["g"])
            cache.out_project(b["out"], B, H * D, p["wo"], hidden, b["x"], residual=b["x"], stream=stream_h)

    graph = None
    for step in range(12):
        xs = [f16((B, hidden)) for _ in range(LAYERS)]
        for which in range(2):
            for layer in range(LAYERS):
                device.upload(bufs[which][layer]["x"].ptr, xs[layer].tobytes())
        device.synchronize()
        eager.begin_step(list(range(B)), [1] * B)
        calls(eager, 0, None)
        graphed.begin_step(list(range(B)), [1] * B, stream=stream.handle)
        if graph is None:
            graph = graphed.record_step(stream.handle)
            calls(graphed, 1, stream.handle)
            graph.end()
        graph.launch()
        stream.synchronize()
        device.synchronize()
        for layer in range(LAYERS):
            for name in ("q", "g", "out", "x"):
                got = bufs[1][layer][name].numpy().view(np.uint16)
                exp = bufs[0][layer][name].numpy().view(np.uint16)
                assert np.array_equal(got, exp), (step, layer, name)
        # The replay against the oracle, layer 0: projection + norm + RoPE
        # (within one fp16 ulp: random sums), gated attention over the
        # oracle's rows (2e-3), and the O-projection of the replay's own
        # gated rows plus the residual (one ulp).
        pos = [L + step for L in lengths]
        cos, sin = tables.cos[pos], tables.sin[pos]
        p = hw[0]
        q_o, g_o, _, k_o, v_o = orc.project_append(xs[0], p["wq"], p["wkv"], p["qw"], p["kw"], cos, sin)
        q_g = bufs[1][0]["q"].numpy()
        assert max_err(q_g, q_o) <= 2 * np.max(np.abs(q_o.astype(np.float32))) * 2.0 ** -10 + 2.0 ** -12, step
        assert max_err(bufs[1][0]["g"].numpy(), g_o) <= np.max(np.abs(g_o.astype(np.float32))) * 2.0 ** -10 + 2.0 ** -12, step
        for b in range(B):
            hist[0][b][0].append(k_o[b])
            hist[0][b][1].append(v_o[b])
        att = orc.decode_attention(q_g, [np.stack(hist[0][b][0]) for b in range(B)],
                                   [np.stack(hist[0][b][1]) for b in range(B)])
        gated = orc.sigmoid_gate(att.astype(np.float16), bufs[1][0]["g"].numpy())
        out_g = bufs[1][0]["out"].numpy()
        assert max_err(out_g, gated) <= 2e-3, step
        x_exp = orc.out_project(out_g.reshape(B, H * D), p["wo"], xs[0])
        x_got = bufs[1][0]["x"].numpy()
        assert max_err(x_got, x_exp) <= np.max(np.abs(x_exp.astype(np.float32))) * 2.0 ** -10 + 2.0 ** -12, step
    for layer in range(LAYERS):
        ke, ve = eager.download_pools(layer)
        kg, vg = graphed.download_pools(layer)
        assert np.array_equal(ke.view(np.uint16), kg.view(np.uint16))
        assert np.array_equal(ve.view(np.uint16), vg.view(np.uint16))
    graph.destroy()
    stream.synchronize()
    stream.destroy()
    eager.destroy()
    graphed.destroy()


def test_graph_replay_prefill_sized_project(device):
    """A prefill-sized step (130 new tokens: kva_project_append takes the
    prefill GEMM, one launch with its norm/RoPE/append epilogue) recorded
    once and replayed for five more steps with fresh x: every replay's q,
    gate and K/V outputs equal the eager twin's and the oracle's bit for bit
    (fp32-exact inputs), and at the end so do the pools."""
    say("graph replay of a prefill-sized project_append")
    rng = np.random.default_rng(9)
    lengths, n_new, hidden, steps = [30, 47, 3], [50, 40, 40], 512, 6
    B, T = len(lengths), sum(n_new)
    ids, o = [], 0
    for L, n in zip(lengths, n_new):
        k = (L + steps * n + 15) // 16
        ids.append(list(range(o, o + k))[::-1])
        o += k
    eager, graphed = [build_cache(lengths, ids, extra_rows=[steps * n for n in n_new],
                                  rng=np.random.default_rng(13))[0] for _ in range(2)]
    tables = Tables(device, 512)
    stream = Stream()
    wq = (rng.integers(-2, 3, (2 * H * D, hidden), dtype=np.int8) * 2.0 ** -7).astype(np.float16)
    wkv = (rng.integers(-2, 3, (2 * HKV * D, hidden), dtype=np.int8) * 2.0 ** -7).astype(np.float16)
    qw = (1 + 0.02 * rng.standard_normal(D, dtype=np.float32)).astype(np.float16)
    kw = (1 + 0.02 * rng.standard_normal(D, dtype=np.float32)).astype(np.float16)
    w = [device.array(a) for a in (wq, wkv, qw, kw)]
    bufs = [dict(x=device.empty((T, hidden), np.float16), q=device.empty((T, H, D), np.float16),
                 g=device.empty((T, H, D), np.float16), kv=device.empty((T, 2, HKV, D), np.float16))
            for _ in range(2)]

    def call(cache, b, stream_h):
        cache.project_append(0, b["x"], hidden, *w, tables.d_cos, tables.d_sin, tables.rows, b["q"], b["g"],
                             b["kv"], stream=stream_h)

    graph = None
    for step in range(steps):
        x = rng.integers(-3, 4, (T, hidden), dtype=np.int8).astype(np.float16)
        for b in bufs:
            device.upload(b["x"].ptr, x.tobytes())
        device.synchronize()
        eager.begin_step(list(range(B)), n_new)
        call(eager, bufs[0], None)
        graphed.begin_step(list(range(B)), n_new, stream=stream.handle)
        if graph is None:
            graph = graphed.record_step(stream.handle)
            call(graphed, bufs[1], stream.handle)
            graph.end()
        graph.launch()
        stream.synchronize()
        device.synchronize()
        assert eager.project_path() == "prefill_gemm"
        pos = [L + step * n + i for L, n in zip(lengths, n_new) for i in range(n)]
        q, gate, k_raw, _, v = orc.project_append(x, wq, wkv, qw, kw, tables.cos[pos], tables.sin[pos])
        for name, exp in (("q", q), ("g", gate)):
            got = bufs[1][name].numpy().view(np.uint16)
            assert np.array_equal(got, bufs[0][name].numpy().view(np.uint16)), (step, name)
            assert np.array_equal(got, exp.view(np.uint16)), (step, name)
        kv = bufs[1]["kv"].numpy()
        assert np.array_equal(kv.view(np.uint16), bufs[0]["kv"].numpy().view(np.uint16)), step
        assert np.array_equal(kv[:, 0].view(np.uint16), k_raw.view(np.uint16)), step
        assert np.array_equal(kv[:, 1].view(np.uint16), v.view(np.uint16)), step
    ke, ve = eager.download_pools(0)
    kg, vg = graphed.download_pools(0)
    assert np.array_equal(ke.view(np.uint16), kg.view(np.uint16))
    assert np.array_equal(ve.view(np.uint16), vg.view(np.uint16))
    graph.destroy()
    stream.synchronize()
    stream.destroy()
    eager.destroy()
    graphed.destroy()
