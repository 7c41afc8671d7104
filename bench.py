#!/usr/bin/env python3
"""Benchmark of the full-attention KV-cache decode path on one MI355X.

Default workload (config 3 of the measurement plan): ragged batched decode,
B=32 sequences with cached lengths U[1024, 8192] (seed 0), 16 full-attention
layers of 24 query / 4 KV heads x 256 dims, FP16 cache in 16-token pages with
randomly permuted page ids.  One step = one decode step of the whole stack:
the step plan upload, then per layer the fused QK-norm+RoPE+K/V append and
the split-K GQA decode attention.  After each step the lengths are set back,
so every timed step is the same workload (append at position L_b, attend
over L_b+1 rows).

Prints ONE JSON line.  ``value`` is the KV bytes the decode attention reads
per second over the whole timed region (the metric's "decode-attn KV-read
HBM GB/s"); ``tok_per_s`` is sequences x steps / time.  The timed steps
carry no events (a marker costs the stream about 3 us).  ``roofline`` is one
kva_decode call: algorithmic bytes per launch (KV rows read + queries) over
its average duration, from HIP events recorded on the launch stream around
the 16 decode calls of each of as many further steps (their appends run
first), divided by 16; ``roofline.decode_kernel`` is the decode kernel
alone, from the library's events around each launch.  ``cpu_baseline`` is the
numpy oracle on a bounded sample of the same workload on this host.
The default line also carries the fixed ctx=8192 case (``ctx8192``), the
measured read and copy ceilings (``peaks``) and every other workload's own
figures (``other_configs``: c1, c2, c4, c5, proj, proj4); --no-extras drops
those three.

Other workloads: --workload c1 (the one-layer config-1 step: GPU latency
next to the numpy oracle's, 1 and all BLAS threads), ctx8192 (every
sequence at 8192 rows), c2
(16 layers, B=1, 128 decode steps growing 128 -> 256 rows), c2graph (the
same with the 16-layer step recorded once and replayed), c4 (chunked
prefill), c5 (tree verify + rollback), proj (config 3 with its producer:
the fused Q/K/V projection + append, then the gated decode), proj4 (the
config-4 producer: 2048 tokens through the tiled prefill GEMM with the
QK-norm/RoPE/append epilogue fused in), copy and read
(HBM stream probes: the measured bandwidth ceilings).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from mi50grad_amd import _lib  # noqa: E402
from mi50grad_amd.device import Event, GPUDevice, Stream, device_props  # noqa: E402
from mi50grad_amd.kv_cache import PagedKVCache  # noqa: E402
from mi50grad_amd.rope import rope_tables  # noqa: E402
from mi50grad_amd import workloads as wl  # noqa: E402

H, HKV, D, LAYERS = 24, 4, 256, 16
HBM_PEAK_GBS = 8000.0
ROW_BYTES = 2 * HKV * D * 2  # K + V of one token in one layer


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def fill_pools(dev: GPUDevice, cache: PagedKVCache, n_blocks: int, seed: int = 0) -> None:
    """Fill every layer's K/V pages [0, n_blocks) with N(0,1) fp16 data.

    A 64 MiB random tile is drawn on the host once and tiled on the device
    (values only matter for realism; timings do not depend on them)."""
    rng = np.random.default_rng(seed)
    tile = rng.standard_normal(32 * 1024 * 1024, dtype=np.float32).astype(np.float16)
    d_tile = dev.array(tile)
    need = n_blocks * cache.block_bytes
    for layer in range(cache.n_layers):
        for base in cache.layer_pools(layer):
            off = 0
            while off < need:
                n = min(tile.nbytes, need - off)
                _lib.call("kva_memcpy_d2d", base + off, d_tile.ptr, n)
                off += n
    d_tile.free()


class L2Flush:
    """Evicts L2 and the MALL between timed iterations: a 1 GiB device
    write (the MALL holds 256 MB), followed by a device synchronisation, so
    the next iteration reads its operands from HBM."""

    BYTES = 1 << 30

    def __init__(self, dev: GPUDevice):
        self.dev = dev
        self.ptr = dev.malloc(self.BYTES)
        self.n = 0

    def __call__(self) -> None:
        self.n += 1
        _lib.call("kva_memset", self.ptr, self.n & 0xff, self.BYTES)
        self.dev.synchronize()

    def free(self) -> None:
        self.dev.free(self.ptr)


def make_inputs(dev: GPUDevice, n_tok: int, seed: int = 1):
    rng = np.random.default_rng(seed)
    per_layer = []
    for _ in range(LAYERS):
        q = dev.array(wl.normal_f16(rng, (n_tok, H, D)))
        k = dev.array(wl.normal_f16(rng, (n_tok, HKV, D)))
        v = dev.array(wl.normal_f16(rng, (n_tok, HKV, D)))
        qw = dev.array(wl.norm_weight(rng))
        kw = dev.array(wl.norm_weight(rng))
        out = dev.empty((n_tok, H, D), np.float16)
        per_layer.append((q, k, v, qw, kw, out))
    return per_layer


def timeline_summary(rec: np.ndarray) -> dict:
    """Summary of one decode launch's timeline (kva_timeline_read records,
    [n_wg, rows, 8 waves, 4]): per workgroup, entry = first wave's entry,
    first issue = when its first K/V loads were out, end = its last wave's
    walk end; microseconds (100 MHz ticks)."""
    ran = rec[:, :, :, 0] > 0  # waves a workgroup does not have leave zero records
    ent = np.where(ran, rec[:, :, :, 0], np.iinfo(np.int64).max).min(axis=(1, 2))
    first = rec[:, :, :, 1].max(axis=(1, 2))
    end = rec[:, :, :, 2].max(axis=(1, 2))
    xcd = (rec[:, 0, 0, 3] >> 32) & 0xF
    t0 = ent.min()
    dur = (end - ent) / 100.0
    return {"workgroups": int(rec.shape[0]), "entry_spread_us": float((ent.max() - t0) / 100.0),
            "first_issue_us": {"median": float(np.median((first - ent) / 100.0)),
                               "max": float(((first - ent) / 100.0).max())},
            "wg_duration_us": {"min": float(dur.min()), "median": float(np.median(dur)), "max": float(dur.max())},
            "span_us": float((end.max() - t0) / 100.0),
            "xcd_mean_duration_us": [round(float(dur[xcd == x].mean()), 2) if (xcd == x).any() else None
                                     for x in range(8)]}


def decode_workload(dev, lengths, block_ids, n_blocks, steps, warmup, split, label, timeline=False):
    B = len(lengths)
    mbps = max(len(ids) for ids in block_ids)
    cache = PagedKVCache(n_layers=LAYERS, max_seqs=B, max_blocks=n_blocks, max_blocks_per_seq=mbps,
                         max_step_tokens=max(64, B))
    for b, ids in enumerate(block_ids):
        cache.set_blocks(b, ids)
    cache.sync_tables()
    fill_pools(dev, cache, n_blocks)
    if split:
        cache.set_decode_split(split)
    rows = int(max(lengths)) + 2
    cos, sin = rope_tables(rows)
    d_cos, d_sin = dev.array(cos), dev.array(sin)
    inputs = make_inputs(dev, B)
    seqs = list(range(B))
    ones = [1] * B

    def step(bracket=None, ev_pairs=None):
        # Plain: each layer's append, then its decode, no events (the timed
        # steps: an event marker costs the stream about 3 us, 95 us per step
        # when every call was bracketed).  bracket: the step's appends, then
        # its 16 decode calls between one pair of events (the per-call figure
        # is the pair's time over 16).  ev_pairs: the library's events around
        # each decode kernel alone (kva_kernel_events).
        for b in seqs:
            cache.set_len(b, int(lengths[b]))
        cache.begin_step(seqs, ones)
        if bracket is not None:
            for layer, (q, k, v, qw, kw, out) in enumerate(inputs):
                cache.append(layer, q, k, v, qw, kw, d_cos, d_sin, rows)
            bracket[0].record()
            for layer, (q, k, v, qw, kw, out) in enumerate(inputs):
                cache.decode(layer, q, out)
            bracket[1].record()
            return
        for layer, (q, k, v, qw, kw, out) in enumerate(inputs):
            cache.append(layer, q, k, v, qw, kw, d_cos, d_sin, rows)
            if ev_pairs is not None:
                cache.kernel_events(ev_pairs[layer][0], ev_pairs[layer][1])
            cache.decode(layer, q, out)
        if ev_pairs is not None:
            cache.kernel_events(None, None)

    log(f"{label}: B={B} sum_ctx={int(np.sum(lengths)) + B} warmup={warmup}")
    for _ in range(warmup):
        step()
    dev.synchronize()
    split_used, n_splits = cache.decode_split()
    t0 = time.perf_counter()
    for i in range(steps):
        step()
    dev.synchronize()
    wall = time.perf_counter() - t0
    # The per-call figure and the decode kernel's own duration, in steps of
    # their own after the timed ones.
    brackets = [[Event(), Event()] for _ in range(steps)]
    for i in range(steps):
        step(bracket=brackets[i])
    dev.synchronize()
    dec_ms = [p[0].elapsed_ms(p[1]) / LAYERS for p in brackets]
    evs = [[[Event(), Event()] for _ in range(LAYERS)] for _ in range(steps)]
    for i in range(steps):
        step(ev_pairs=evs[i])
    dev.synchronize()
    ker_ms = [e[0].elapsed_ms(e[1]) for per_step in evs for e in per_step]
    for pair in brackets + [pair for per_step in evs for pair in per_step]:
        for x in pair:
            x.destroy()
    log(f"{label}: {steps} steps in {wall * 1e3:.2f} ms; kva_decode avg {np.mean(dec_ms) * 1e3:.1f} us, "
        f"decode kernel avg {np.mean(ker_ms) * 1e3:.1f} us")
    tl = None
    if timeline:
        # Outside the timed region: one more step, each layer's decode
        # followed by a read of its timeline (the read synchronises).
        cache.timeline_enable(True)
        for b in seqs:
            cache.set_len(b, int(lengths[b]))
        cache.begin_step(seqs, ones)
        samples = []
        for layer, (q, k, v, qw, kw, out) in enumerate(inputs):
            cache.append(layer, q, k, v, qw, kw, d_cos, d_sin, rows)
            cache.decode(layer, q, out)
            samples.append(timeline_summary(cache.timeline()))
        cache.timeline_enable(False)
        med = lambda f: float(np.median([f(x) for x in samples]))
        tl = {"launches": len(samples),
              "first_issue_us_median": med(lambda x: x["first_issue_us"]["median"]),
              "wg_duration_us_median": med(lambda x: x["wg_duration_us"]["median"]),
              "wg_duration_us_max": med(lambda x: x["wg_duration_us"]["max"]),
              "span_us": med(lambda x: x["span_us"]),
              "xcd_mean_duration_us": [round(med(lambda x, i=i: x["xcd_mean_duration_us"][i]), 2) for i in range(8)],
              "per_launch": samples}
    cache.destroy()
    ctx = np.asarray(lengths, dtype=np.int64) + 1
    by = wl.decode_bytes(ctx)
    return {
        "wall_s": wall, "steps": steps, "B": B,
        "kv_bytes_per_layer": by["kv"], "alg_bytes_decode_launch": by["kv"] + by["q"],
        "alg_bytes_layer_step": by["kv"] + by["q"] + by["out"] + by["append"],
        "decode_avg_us": float(np.mean(dec_ms) * 1e3), "decode_min_us": float(np.min(dec_ms) * 1e3),
        "kernel_avg_us": float(np.mean(ker_ms) * 1e3),
        "split_tokens": split_used, "n_splits": n_splits, "timeline": tl,
    }


def proj_workload(dev, steps, warmup, hidden=5120):
    """The config-3 step with its producer and consumer: per layer,
    kva_project_append (the Q+Q_gate and K+V projections of the 32 new
    tokens from hidden 5120, norm + RoPE, K/V into the pages), then
    kva_decode_gated, then kva_out_project (the O-projection from 6144 back
    to 5120, added into the layer's hidden rows in place).  Each layer has
    its own weights (16 x 147 MB + 16 x 63 MB, so no layer's weights are
    still cached when it comes round again); their values are a 32 MiB
    random tile repeated on the device."""
    spec = wl.c3_spec(0)
    lengths, block_ids, n_blocks = spec.lengths, spec.block_ids, spec.n_blocks
    B = len(lengths)
    mbps = max(len(ids) for ids in block_ids)
    cache = PagedKVCache(n_layers=LAYERS, max_seqs=B, max_blocks=n_blocks, max_blocks_per_seq=mbps,
                         max_step_tokens=max(64, B))
    for b, ids in enumerate(block_ids):
        cache.set_blocks(b, ids)
    cache.sync_tables()
    fill_pools(dev, cache, n_blocks)
    rows = int(max(lengths)) + 2
    cos, sin = rope_tables(rows)
    d_cos, d_sin = dev.array(cos), dev.array(sin)
    rng = np.random.default_rng(2)
    tile = (rng.standard_normal(16 * 1024 * 1024, dtype=np.float32) / np.sqrt(hidden)).astype(np.float16)
    d_tile = dev.array(tile)
    nq, nkv = 2 * H * D * hidden * 2, 2 * HKV * D * hidden * 2  # bytes
    q_dim = H * D
    no = hidden * q_dim * 2  # O-projection weight bytes
    layers = []
    for layer in range(LAYERS):
        w = []
        for nbytes in (nq, nkv, no):
            d = dev.empty((nbytes // 2,), np.float16)
            off = 0
            while off < nbytes:
                n = min(tile.nbytes - 4096 * layer, nbytes - off)
                _lib.call("kva_memcpy_d2d", d.ptr + off, d_tile.ptr + 4096 * layer, n)
                off += n
            w.append(d)
        x = dev.array(wl.normal_f16(rng, (B, hidden)))
        qw, kw = dev.array(wl.norm_weight(rng)), dev.array(wl.norm_weight(rng))
        q, g, out = (dev.empty((B, H, D), np.float16) for _ in range(3))
        layers.append((x, w[0], w[1], w[2], qw, kw, q, g, out))
    d_tile.free()
    seqs, ones = list(range(B)), [1] * B

    def step(evs=None):
        # The 16 layers' projections, then their gated decodes, then their
        # O-projections (each layer has its own buffers), each group between
        # one pair of events: a per-call figure is the group's time over 16
        # (an event marker costs the stream about 3 us, too much to put one
        # around every call).
        for b in seqs:
            cache.set_len(b, int(lengths[b]))
        cache.begin_step(seqs, ones)
        if evs is not None:
            evs[0].record()
        for layer, (x, wq, wkv, wo, qw, kw, q, g, out) in enumerate(layers):
            cache.project_append(layer, x, hidden, wq, wkv, qw, kw, d_cos, d_sin, rows, q, g)
        if evs is not None:
            evs[1].record()
        for layer, (x, wq, wkv, wo, qw, kw, q, g, out) in enumerate(layers):
            cache.decode(layer, q, out, gate=g)
        if evs is not None:
            evs[2].record()
        for layer, (x, wq, wkv, wo, qw, kw, q, g, out) in enumerate(layers):
            cache.out_project(out, B, q_dim, wo, hidden, x, residual=x)  # hidden += o_proj(attn)
        if evs is not None:
            evs[3].record()

    for _ in range(warmup):
        step()
    dev.synchronize()
    evs = [[Event(), Event(), Event(), Event()] for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        step(evs[i])
    dev.synchronize()
    wall = time.perf_counter() - t0
    proj_ms = [e[0].elapsed_ms(e[1]) / LAYERS for e in evs]
    dec_ms = [e[1].elapsed_ms(e[2]) / LAYERS for e in evs]
    out_ms = [e[2].elapsed_ms(e[3]) / LAYERS for e in evs]
    for e in evs:
        for x in e:
            x.destroy()
    cache.destroy()
    alg = (nq + nkv) + B * hidden * 2 + 2 * B * H * D * 2 + B * 2 * HKV * D * 2
    alg_out = no + B * q_dim * 2 + 2 * B * hidden * 2  # W_o, attention rows, hidden read + written
    return {"wall_s": wall, "steps": steps, "B": B, "hidden": hidden, "alg_bytes_proj": alg,
            "weight_bytes": nq + nkv, "proj_avg_us": float(np.mean(proj_ms) * 1e3),
            "decode_avg_us": float(np.mean(dec_ms) * 1e3), "out_avg_us": float(np.mean(out_ms) * 1e3),
            "alg_bytes_out": alg_out}


def proj_prefill_workload(dev, steps, warmup, hidden=5120):
    """The config-4 step's producer: kva_project_append of the 2048 new
    tokens (4 sequences x 512 after 0/256/1024/2048 cached rows) from hidden
    5120, with norm + RoPE + append, per layer (16 layers, own weights)."""
    prefix, chunk = list(wl.C4_PREFIX), [wl.C4_CHUNK] * 4
    B, T = 4, sum(chunk)
    nblk = [(p + c + 15) // 16 for p, c in zip(prefix, chunk)]
    cache = PagedKVCache(n_layers=LAYERS, max_seqs=B, max_blocks=sum(nblk), max_blocks_per_seq=max(nblk),
                         max_step_tokens=T)
    o = 0
    for b, n in enumerate(nblk):
        cache.set_blocks(b, list(range(o, o + n)))
        o += n
    cache.sync_tables()
    cos, sin = rope_tables(4096)
    d_cos, d_sin = dev.array(cos), dev.array(sin)
    rng = np.random.default_rng(6)
    tile = (rng.standard_normal(16 * 1024 * 1024, dtype=np.float32) / np.sqrt(hidden)).astype(np.float16)
    d_tile = dev.array(tile)
    nq, nkv = 2 * H * D * hidden * 2, 2 * HKV * D * hidden * 2
    layers = []
    for layer in range(LAYERS):
        w = []
        for nbytes in (nq, nkv):
            d = dev.empty((nbytes // 2,), np.float16)
            off = 0
            while off < nbytes:
                n = min(tile.nbytes - 4096 * layer, nbytes - off)
                _lib.call("kva_memcpy_d2d", d.ptr + off, d_tile.ptr + 4096 * layer, n)
                off += n
            w.append(d)
        qw, kw = dev.array(wl.norm_weight(rng)), dev.array(wl.norm_weight(rng))
        layers.append((w[0], w[1], qw, kw))
    d_tile.free()
    x = dev.array(wl.normal_f16(rng, (T, hidden)))
    q, g = dev.empty((T, H, D), np.float16), dev.empty((T, H, D), np.float16)
    seqs = list(range(B))

    def step(evs=None):
        for b in seqs:
            cache.set_len(b, prefix[b])
        cache.begin_step(seqs, chunk)
        for layer, (wq, wkv, qw, kw) in enumerate(layers):
            if evs is not None:
                evs[layer][0].record()
            cache.project_append(layer, x, hidden, wq, wkv, qw, kw, d_cos, d_sin, 4096, q, g)
            if evs is not None:
                evs[layer][1].record()

    for _ in range(warmup):
        step()
    dev.synchronize()
    evs = [[[Event(), Event()] for _ in range(LAYERS)] for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        step(evs[i])
    dev.synchronize()
    wall = time.perf_counter() - t0
    ms = [e[0].elapsed_ms(e[1]) for s_ in evs for e in s_]
    path = cache.project_path()
    cache.destroy()
    return {"wall_s": wall, "steps": steps, "tokens": T, "hidden": hidden, "weight_bytes": nq + nkv,
            "flops": T * (nq + nkv), "proj_avg_us": float(np.mean(ms) * 1e3), "path": path}


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def c1_workload(dev, reps=200):
    """Config 1: one layer, batch 1, 255 cached rows; append at position 255
    (norm + RoPE of q and k, K/V into the cache) then decode over 256 rows.
    GPU: HIP events around kva_append_decode (one launch), and separately
    around kva_append_qknorm_rope + kva_decode, median of `reps` calls each,
    L2 and MALL flushed before each call (the layer's 1 MB would otherwise
    stay cached from the previous call).  CPU: the
    numpy oracle's same step (norm + RoPE of the 28 rows, then decode
    attention), median of 25 calls with 1 BLAS thread and with all of them."""
    from threadpoolctl import threadpool_limits

    from oracle import kvattn_oracle as orc

    x = wl.c1_inputs(0)
    cache = PagedKVCache(n_layers=1, max_seqs=1, max_blocks=16, max_blocks_per_seq=16, max_step_tokens=16)
    cache.reserve(0, 256)
    cache.sync_tables()
    ids = cache.blocks(0)
    kimg = np.zeros((16, 16, HKV, D), np.float16)
    vimg = np.zeros_like(kimg)
    for r in range(255):
        kimg[ids[r // 16], r % 16] = x.k_cache[r]
        vimg[ids[r // 16], r % 16] = x.v_cache[r]
    kp, vp = cache.layer_pools(0)
    dev.upload(kp, kimg.tobytes())
    dev.upload(vp, vimg.tobytes())
    cos, sin = rope_tables(256)
    d_cos, d_sin = dev.array(cos), dev.array(sin)
    qw, kw = dev.array(x.q_norm), dev.array(x.k_norm)
    q, k, v = dev.empty((1, H, D), np.float16), dev.array(x.k_new), dev.array(x.v_new)
    out = dev.empty((1, H, D), np.float16)
    flush = L2Flush(dev)
    ms = {"fused": [], "two_calls": []}
    for mode, times in ms.items():
        for i in range(reps + 10):
            cache.set_len(0, 255)
            cache.begin_step([0], [1])
            dev.upload(q.ptr, x.q.tobytes())
            dev.upload(k.ptr, x.k_new.tobytes())
            flush()
            a, b = Event(), Event()
            a.record()
            if mode == "fused":
                cache.append_decode(0, q, k, v, qw, kw, d_cos, d_sin, 256, out)
            else:
                cache.append(0, q, k, v, qw, kw, d_cos, d_sin, 256)
                cache.decode(0, q, out)
            b.record()
            b.synchronize()
            if i >= 10:
                times.append(a.elapsed_ms(b))
            a.destroy()
            b.destroy()
    cache.destroy()
    flush.free()

    pos = np.array([255])

    def cpu_step():
        qn = orc.qknorm_rope_exact(x.q.reshape(H, D), x.q_norm, np.repeat(cos[pos], H, 0), np.repeat(sin[pos], H, 0))
        kn = orc.qknorm_rope_exact(x.k_new.reshape(HKV, D), x.k_norm, np.repeat(cos[pos], HKV, 0),
                                   np.repeat(sin[pos], HKV, 0))
        kc = np.concatenate([x.k_cache, kn.reshape(1, HKV, D)])
        vc = np.concatenate([x.v_cache, x.v_new])
        return orc.decode_attention(qn.reshape(1, H, D), [kc], [vc])

    cpu = {}
    for label, n in (("1", 1), ("all", None)):
        with threadpool_limits(n):
            ts = []
            for _ in range(25):
                t0 = time.perf_counter()
                cpu_step()
                ts.append(time.perf_counter() - t0)
        cpu[label] = float(np.median(ts) * 1e6)
    return {"gpu_us": float(np.median(ms["fused"]) * 1e3), "gpu_min_us": float(np.min(ms["fused"]) * 1e3),
            "two_calls_us": float(np.median(ms["two_calls"]) * 1e3), "cpu_us_1": cpu["1"],
            "cpu_us_all": cpu["all"], "reps": reps}


def c2_workload(dev, steps_unused, warmup, graph=False, split=0, fused=True):
    """Config 2: B=1, 16 layers, 128 decode steps from a 128-row cache.  Each
    layer is one kva_append_decode call (fused=True: norm + RoPE, append and
    decode in one launch) or kva_append_qknorm_rope + kva_decode.  With
    graph=True the 16 layers' calls are recorded once (kva_graph_*) and
    replayed after each step's plan upload.

    Timed twice: back to back (wall clock over the 128 steps, the 16 MB of
    pages staying in the MALL), and per step between HIP events on the launch
    stream with L2 and the MALL flushed before each step (`step_us`, the
    reported value)."""
    B, start, n_steps = 1, 128, 128
    cache = PagedKVCache(n_layers=LAYERS, max_seqs=1, max_blocks=16, max_blocks_per_seq=16,
                         max_step_tokens=16)
    cache.reserve(0, 256)
    cache.sync_tables()
    cache.set_decode_split(split)
    fill_pools(dev, cache, 16)
    cos, sin = rope_tables(256)
    d_cos, d_sin = dev.array(cos), dev.array(sin)
    inputs = make_inputs(dev, B)
    stream = Stream() if graph else None
    sh = stream.handle if graph else None
    recorded = []

    def layers():
        for layer, (q, k, v, qw, kw, out) in enumerate(inputs):
            if fused:
                cache.append_decode(layer, q, k, v, qw, kw, d_cos, d_sin, 256, out, stream=sh)
            else:
                cache.append(layer, q, k, v, qw, kw, d_cos, d_sin, 256, stream=sh)
                cache.decode(layer, q, out, stream=sh)

    def run(evs=None, flush=None):
        cache.set_len(0, start)
        for i in range(n_steps):
            if flush is not None:
                if stream:
                    stream.synchronize()
                flush()
            if evs is not None:
                evs[i][0].record(sh)
            cache.begin_step([0], [1], stream=sh)
            if not graph:
                layers()
            else:
                if not recorded:
                    g = cache.record_step(sh)
                    layers()
                    recorded.append(g.end())
                recorded[0].launch()
            if evs is not None:
                evs[i][1].record(sh)

    for _ in range(max(1, warmup)):
        run()
    if stream:
        stream.synchronize()
    dev.synchronize()
    t0 = time.perf_counter()
    run()
    if stream:
        stream.synchronize()
    dev.synchronize()
    wall = time.perf_counter() - t0
    flush = L2Flush(dev)
    evs = [[Event(), Event()] for _ in range(n_steps)]
    run(evs, flush)
    if stream:
        stream.synchronize()
    dev.synchronize()
    step_ms = [a.elapsed_ms(b) for a, b in evs]
    for a, b in evs:
        a.destroy()
        b.destroy()
    flush.free()
    for g in recorded:
        g.destroy()
    if stream:
        stream.destroy()
    cache.destroy()
    kv = LAYERS * ROW_BYTES * sum(range(start + 1, start + n_steps + 1))
    return {"wall_s": wall, "steps": n_steps, "kv_bytes": kv, "step_us": float(np.mean(step_ms) * 1e3),
            "step_us_median": float(np.median(step_ms) * 1e3)}


MFMA_PEAK_TFLOPS = 2500.0  # dense fp16


def mfma_peak_derived() -> dict:
    """Dense fp16 MFMA peak from this device's CU count and peak clock: a
    v_mfma_f32_16x16x32_f16 does 16384 FLOPs in 16 cycles on each of a CU's
    4 SIMDs, 4096 FLOPs per CU per clock."""
    p = device_props()
    return {"tflops": p["n_cu"] * p["clock_khz"] * 1e3 * 4096 / 1e12, "n_cu": p["n_cu"],
            "clock_mhz": p["clock_khz"] / 1e3,
            "method": "kva_dev_props: CUs x peak shader clock x 4096 dense fp16 FLOP per CU per clock"}


def stored_mfma_busy() -> dict | None:
    """MFMA-busy fraction of the prefill kernel from its stored rocprofv3
    counter profile (not counted in this run)."""
    path = ROOT / "profiles" / "prefill_c4_mfma.json"
    if not path.exists():
        return None
    d = json.loads(path.read_text())["derived"]
    return {"fraction": d["mfma_busy_fraction"], "source": "profiles/prefill_c4_mfma.json: "
            "SQ_VALU_MFMA_BUSY_CYCLES per SIMD over the kernel's cycles (a stored profile)"}


def c4_workload(dev, steps, warmup, extras=True):
    """Config 4: 4 sequences append a 512-token chunk after 0/256/1024/2048
    cached rows (fused norm+RoPE+append), then causal prefill attention; 16
    layers per step.  Lengths are set back after each step."""
    prefix, chunk = list(wl.C4_PREFIX), [wl.C4_CHUNK] * 4
    B, T = 4, sum(chunk)
    nblk = [(p + c + 15) // 16 for p, c in zip(prefix, chunk)]
    cache = PagedKVCache(n_layers=LAYERS, max_seqs=B, max_blocks=sum(nblk), max_blocks_per_seq=max(nblk),
                         max_step_tokens=T)
    perm = np.random.default_rng(0).permutation(sum(nblk))
    o = 0
    for b, n in enumerate(nblk):
        cache.set_blocks(b, [int(x) for x in perm[o:o + n]])
        o += n
    cache.sync_tables()
    fill_pools(dev, cache, sum(nblk))
    cos, sin = rope_tables(4096)
    d_cos, d_sin = dev.array(cos), dev.array(sin)
    inputs = make_inputs(dev, T)
    seqs = list(range(B))

    def step(evs=None, kernel=False, mode="fused"):
        # fused: kva_append_prefill (append + attention, one call); two:
        # kva_append_qknorm_rope + kva_prefill; the 16 layers' calls between
        # one pair of events, evs[0] (per call: the pair's time over 16; an
        # event marker costs the stream about 3 us).  prefill: each layer's
        # append, then its kva_prefill between a pair of its own, evs[layer]
        # (how earlier lines were measured: the append just before leaves q
        # in the caches, which running all appends first would not).
        # kernel: each layer's fused call with the library's events
        # (evs[layer]) around mq_kernel alone.
        for b in seqs:
            cache.set_len(b, prefix[b])
        cache.begin_step(seqs, chunk)
        if kernel:
            for layer, (q, k, v, qw, kw, out) in enumerate(inputs):
                cache.kernel_events(evs[layer][0], evs[layer][1])
                cache.append_prefill(layer, q, k, v, qw, kw, d_cos, d_sin, 4096, out)
            cache.kernel_events(None, None)
            return
        if mode == "prefill":
            for layer, (q, k, v, qw, kw, out) in enumerate(inputs):
                cache.append(layer, q, k, v, qw, kw, d_cos, d_sin, 4096)
                if evs is not None:
                    evs[layer][0].record()
                cache.prefill(layer, q, out)
                if evs is not None:
                    evs[layer][1].record()
            return
        if evs is not None:
            evs[0][0].record()
        for layer, (q, k, v, qw, kw, out) in enumerate(inputs):
            if mode == "fused":
                cache.append_prefill(layer, q, k, v, qw, kw, d_cos, d_sin, 4096, out)
            else:
                cache.append(layer, q, k, v, qw, kw, d_cos, d_sin, 4096)
                cache.prefill(layer, q, out)
        if evs is not None:
            evs[0][1].record()

    for _ in range(warmup):
        step()
    dev.synchronize()
    flush = L2Flush(dev)

    # The modes take turns step by step, so each sees the same clock and
    # thermal state; mq_kernel's own duration comes from steps of their own.
    modes = (("fused", False), ("fused", True), ("two", False), ("prefill", False)) if extras else \
        (("fused", False),)
    evs = {m: [[[Event(), Event()] for _ in range(LAYERS)] for _ in range(steps)] for m in modes}
    wall = 0.0
    for i in range(steps):
        for m in modes:
            flush()  # each step starts from HBM: its 1.3 GB would not fit the MALL anyway
            t0 = time.perf_counter()
            step(evs[m][i], m[1], m[0])
            dev.synchronize()
            if m == modes[0]:
                wall += time.perf_counter() - t0
    per = {m: ([e[0].elapsed_ms(e[1]) for s in evs[m] for e in s] if m[1] or m[0] == "prefill" else
               [s[0][0].elapsed_ms(s[0][1]) / LAYERS for s in evs[m]]) for m in modes}
    ms = per[modes[0]]
    kms, two_ms, pre_ms = (per[m] for m in modes[1:]) if extras else (None, None, None)
    for m in modes:
        for s in evs[m]:
            for pair in s:
                for x in pair:
                    x.destroy()
    flush.free()
    cache.destroy()
    flops = 4 * H * D * sum(sum(p + i + 1 for i in range(c)) for p, c in zip(prefix, chunk))
    # Cache rows read, q read and out written, the new K/V rows read and
    # written to their slots.
    by = (sum(p + c for p, c in zip(prefix, chunk)) * ROW_BYTES + 2 * T * H * D * 2 + 4 * T * HKV * D * 2)
    return {"wall_s": wall, "steps": steps, "tokens": T, "flops_per_layer": flops, "bytes_per_layer": by,
            "prefill_avg_us": float(np.mean(ms) * 1e3),
            **{k: (float(np.mean(v) * 1e3) if v is not None else None)
               for k, v in (("kernel_avg_us", kms), ("two_calls_avg_us", two_ms), ("prefill_only_avg_us", pre_ms))}}


def c5_workload(dev, steps, warmup, layers=4, batch=64):
    """Config 5: 64 sequences with cached lengths U[4096, 32768] (seed 0)
    append the 9-node draft tree (RoPE at len+depth), run tree-verify
    attention, then keep a seeded root-to-node path and roll back the rest
    (all layers).  `layers` full-attention layers per step (the pools of 16
    layers would hold 77 GB; per-layer figures are what is reported)."""
    from mi50grad_amd import tree as tr

    spec = wl.c5_spec(0, batch=batch)
    lengths = [int(x) for x in spec.lengths]
    T = 9 * batch
    cache = PagedKVCache(n_layers=layers, max_seqs=batch, max_blocks=spec.n_blocks,
                         max_blocks_per_seq=max(len(i) for i in spec.block_ids), max_step_tokens=T)
    for b, ids in enumerate(spec.block_ids):
        cache.set_blocks(b, ids)
    cache.sync_tables()
    fill_pools(dev, cache, spec.n_blocks)
    rows = max(lengths) + 16
    cos, sin = rope_tables(rows)
    d_cos, d_sin = dev.array(cos), dev.array(sin)
    rng = np.random.default_rng(1)
    inputs = [tuple(dev.array(x) for x in (wl.normal_f16(rng, (T, H, D)), wl.normal_f16(rng, (T, HKV, D)),
                                          wl.normal_f16(rng, (T, HKV, D)), wl.norm_weight(rng),
                                          wl.norm_weight(rng))) + (dev.empty((T, H, D), np.float16),)
              for _ in range(layers)]
    depth = tr.depths(wl.C5_PARENTS)
    rope_pos = [L + d for L in lengths for d in depth]
    bits = tr.tree_bits(wl.C5_PARENTS) * batch
    accept = np.random.default_rng(2).integers(0, 9, batch)
    keep = [tr.root_to_node_path(wl.C5_PARENTS, int(n)) for n in accept]
    seqs = list(range(batch))

    def step(evs=None, kernel_evs=None):
        # evs: the step's appends, then its tree-verify calls between one
        # pair of events (per call: the pair's time over the layers), then
        # the rollback between another pair.  kernel_evs: each layer's append
        # and verify, with the library's events around mq_kernel alone.
        for b in seqs:
            cache.set_len(b, lengths[b])
        cache.begin_step(seqs, [9] * batch, rope_pos=rope_pos, tree_bits=bits)
        if kernel_evs is not None:
            for layer, (q, k, v, qw, kw, out) in enumerate(inputs):
                cache.append(layer, q, k, v, qw, kw, d_cos, d_sin, rows)
                cache.kernel_events(kernel_evs[layer][0], kernel_evs[layer][1])
                cache.tree_verify(layer, q, out)
            cache.kernel_events(None, None)
        else:
            for layer, (q, k, v, qw, kw, out) in enumerate(inputs):
                cache.append(layer, q, k, v, qw, kw, d_cos, d_sin, rows)
            if evs is not None:
                evs[0].record()
            for layer, (q, k, v, qw, kw, out) in enumerate(inputs):
                cache.tree_verify(layer, q, out)
            if evs is not None:
                evs[1].record()
        if evs is not None:
            evs[2].record()
        cache.rollback(seqs, lengths, keep)
        if evs is not None:
            evs[3].record()

    for _ in range(warmup):
        step()
    dev.synchronize()
    evs = [[Event() for _ in range(4)] for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        step(evs[i])
    dev.synchronize()
    wall = time.perf_counter() - t0
    verify_ms = [e[0].elapsed_ms(e[1]) / layers for e in evs]
    rb_ms = [e[2].elapsed_ms(e[3]) for e in evs]
    kevs = [[[Event(), Event()] for _ in range(layers)] for _ in range(steps)]
    for i in range(steps):  # mq_kernel's own duration, in steps of their own
        step(kernel_evs=kevs[i])
    dev.synchronize()
    kernel_ms = [e[0].elapsed_ms(e[1]) for s in kevs for e in s]
    for x in [x for e in evs for x in e] + [x for s in kevs for pair in s for x in pair]:
        x.destroy()
    cache.destroy()
    kv = sum(lengths) * ROW_BYTES + T * ROW_BYTES
    return {"wall_s": wall, "steps": steps, "layers": layers, "kv_bytes_per_layer": kv,
            "alg_bytes_per_layer": kv + 2 * T * H * D * 2, "verify_avg_us": float(np.mean(verify_ms) * 1e3),
            "kernel_avg_us": float(np.mean(kernel_ms) * 1e3),
            "rollback_avg_us": float(np.mean(rb_ms) * 1e3), "sum_len": sum(lengths)}


def copy_probe(dev, gib: float = 4.0, reps: int = 20):
    n = int(gib * (1 << 30)) // 16 * 16
    a, b = dev.malloc(n), dev.malloc(n)
    _lib.call("kva_memset", a, 0, n)
    s, e = Event(), Event()
    for _ in range(3):
        _lib.call("kva_hbm_copy", b, a, n, None)
    s.record()
    for _ in range(reps):
        _lib.call("kva_hbm_copy", b, a, n, None)
    e.record()
    e.synchronize()
    ms = s.elapsed_ms(e) / reps
    dev.free(a)
    dev.free(b)
    return {"bytes_per_launch": 2 * n, "avg_us": ms * 1e3, "gbs": 2 * n / (ms * 1e-3) / 1e9}


def page_read_probe(dev, reps: int = 20, copies: int = 4):
    """The read ceiling of the decode's own access pattern: kva_hbm_read_pages
    over config 3's pages (the same lengths, the same permuted page ids, 256
    workgroups of four waves), rotating over `copies` layers' pools so no
    launch finds the previous one's pages in the MALL; average of `reps`
    launches between HIP events."""
    spec = wl.c3_spec(0)
    ids = np.concatenate([np.asarray(b[:(int(L) + 1 + 15) // 16], np.int32)
                          for L, b in zip(spec.lengths, spec.block_ids)])
    cache = PagedKVCache(n_layers=copies, max_seqs=1, max_blocks=spec.n_blocks, max_blocks_per_seq=1,
                         max_step_tokens=16)
    d_ids, sink = dev.array(ids), dev.malloc(256)
    pools = [cache.layer_pools(i) for i in range(copies)]
    n_cu = device_props()["n_cu"]
    call = lambda i: _lib.call("kva_hbm_read_pages", pools[i % copies][0], pools[i % copies][1], d_ids.ptr,
                               len(ids), HKV, n_cu, sink, None)
    for i in range(copies):
        call(i)
    s, e = Event(), Event()
    s.record()
    for i in range(reps):
        call(i)
    e.record()
    e.synchronize()
    ms = s.elapsed_ms(e) / reps
    by = len(ids) * 16 * ROW_BYTES  # K and V of every row of every page
    dev.free(sink)
    d_ids.free()
    cache.destroy()
    return {"bytes_per_launch": by, "avg_us": ms * 1e3, "gbs": by / (ms * 1e-3) / 1e9, "pages": len(ids)}


def read_probe(dev, gib: float = 4.0, reps: int = 20):
    """The HBM read ceiling: kva_hbm_read over `gib` GiB, average of `reps`
    launches between HIP events."""
    n = int(gib * (1 << 30)) // 16 * 16
    a, sink = dev.malloc(n), dev.malloc(256)
    _lib.call("kva_memset", a, 0, n)
    s, e = Event(), Event()
    for _ in range(3):
        _lib.call("kva_hbm_read", a, n, sink, None)
    s.record()
    for _ in range(reps):
        _lib.call("kva_hbm_read", a, n, sink, None)
    e.record()
    e.synchronize()
    ms = s.elapsed_ms(e) / reps
    dev.free(a)
    dev.free(sink)
    return {"bytes_per_launch": n, "avg_us": ms * 1e3, "gbs": n / (ms * 1e-3) / 1e9}


def cpu_baseline(budget_s: float = 10.0):
    """The numpy oracle's decode attention on a slice of the config-3 workload.

    Sample: the first 4 sequences of config 3 (seed 0), one layer, one decode
    step (append excluded), single-threaded BLAS; repeated until ~budget_s.
    Reported as KV GB/s with the same algorithmic byte count as the GPU row.

    ``all_threads`` runs the first 16 sequences with one sequence per worker
    thread (1 BLAS thread each); numpy releases the interpreter lock in the
    conversions and products that take the time, so the workers overlap.  At
    most 8 workers: on the 16-CPU box host 1, 2, 4, 8, 12 and 16 workers gave
    1.5, 3.0, 3.4, 4.3, 3.7 and 3.9 GB/s (the oracle's per-head Python loop
    holds the lock between the numpy calls)."""
    from concurrent.futures import ThreadPoolExecutor

    from threadpoolctl import threadpool_limits

    from oracle import kvattn_oracle as orc

    spec = wl.c3_spec(0)
    lens = [int(x) + 1 for x in spec.lengths[:16]]
    rng = np.random.default_rng(3)
    q = wl.normal_f16(rng, (len(lens), H, D))
    ks = [wl.normal_f16(rng, (n, HKV, D)) for n in lens]
    vs = [wl.normal_f16(rng, (n, HKV, D)) for n in lens]

    def timed(step, n_seq):
        reps, t = 0, 0.0
        t0 = time.perf_counter()
        while t < budget_s:
            step()
            reps += 1
            t = time.perf_counter() - t0
        return sum(lens[:n_seq]) * ROW_BYTES * reps / t / 1e9, reps, t

    try:
        workers = min(len(os.sched_getaffinity(0)), 8)
    except AttributeError:
        workers = min(os.cpu_count() or 1, 8)
    with threadpool_limits(1):
        v1, r1, t1 = timed(lambda: orc.decode_attention(q[:4], ks[:4], vs[:4]), 4)
        with ThreadPoolExecutor(workers) as pool:
            def one(b):
                return orc.decode_attention(q[b:b + 1], ks[b:b + 1], vs[b:b + 1])
            va, ra, ta = timed(lambda: list(pool.map(one, range(len(lens)))), len(lens))
    return {"value": v1, "unit": "GB/s", "cores": 1, "kind": "port",
            "all_threads": {"value": va, "cores": workers, "reps": ra, "seconds": round(ta, 1),
                            "sample": f"config-3 sequences 0-{len(lens) - 1} (ctx {lens}), one sequence per "
                                      f"worker thread, 1 BLAS thread each"},
            "sample": f"numpy oracle decode_attention, config-3 sequences 0-3 "
                      f"(ctx {lens[:4]}), one layer, {r1} reps in {t1:.1f} s, 1 BLAS thread (value); "
                      f"all_threads: {workers} worker threads; host {os.cpu_count()} logical CPUs ({_cpu_model()})"}


def _median_cpu(fn, budget_s: float, threads):
    """Median time of fn() (3 warm-ups, then until ~budget_s or 20 calls,
    at least 5) under a BLAS thread limit (None = all)."""
    from threadpoolctl import threadpool_limits

    ts = []
    with threadpool_limits(threads):
        for _ in range(3):
            fn()
        t_end = time.perf_counter() + budget_s
        while len(ts) < 5 or (len(ts) < 20 and time.perf_counter() < t_end):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
    return float(np.median(ts)), len(ts)


def cpu_baseline_c4(budget_s: float = 8.0):
    """The numpy oracle's causal chunk attention for one config-4 sequence
    (P = 256: a 512-token chunk over 768 keys), one layer, 1 BLAS thread;
    reported as TFLOP/s on the unmasked pairs, as the GPU row."""
    from oracle import kvattn_oracle as orc

    rng = np.random.default_rng(4)
    P, C = 256, wl.C4_CHUNK
    q = wl.normal_f16(rng, (C, H, D))
    k = wl.normal_f16(rng, (P + C, HKV, D))
    v = wl.normal_f16(rng, (P + C, HKV, D))
    t, n = _median_cpu(lambda: orc.chunk_attention(q, k, v, P), budget_s, 1)
    flops = 4 * H * D * sum(P + i + 1 for i in range(C))
    return {"value": flops / t / 1e12, "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": f"numpy oracle chunk_attention, one config-4 sequence (P={P}, chunk {C}), one layer, "
                      f"median of {n} calls, 1 BLAS thread; host {os.cpu_count()} logical CPUs ({_cpu_model()})"}


def cpu_baseline_c5(budget_s: float = 8.0):
    """The numpy oracle's tree attention for one config-5 sequence (its
    first: the 9-node tree over the cached rows), one layer, 1 BLAS thread;
    reported as KV GB/s with the GPU row's byte count."""
    from oracle import kvattn_oracle as orc

    spec = wl.c5_spec(0)
    L = int(spec.lengths[0])
    rng = np.random.default_rng(5)
    q = wl.normal_f16(rng, (9, H, D))
    kc, vc = wl.normal_f16(rng, (L, HKV, D)), wl.normal_f16(rng, (L, HKV, D))
    kt, vt = wl.normal_f16(rng, (9, HKV, D)), wl.normal_f16(rng, (9, HKV, D))
    t, n = _median_cpu(lambda: orc.tree_attention(q, kc, vc, kt, vt, wl.C5_PARENTS), budget_s, 1)
    by = L * ROW_BYTES + 9 * ROW_BYTES + 2 * 9 * H * D * 2
    return {"value": by / t / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"numpy oracle tree_attention, config-5 sequence 0 (ctx {L}, 9-node tree), one layer, "
                      f"median of {n} calls, 1 BLAS thread; host {os.cpu_count()} logical CPUs ({_cpu_model()})"}


def load_traffic(name: str):
    p = ROOT / "profiles" / name
    if not p.exists():
        return None
    try:
        return json.loads(p.read_text()).get("traffic_bytes_per_launch")
    except (ValueError, OSError):
        return None


def workload_line(dev, args) -> dict:
    """The bench line (a dict) of every workload but the decode ones."""
    if args.workload in ("copy", "read", "pages"):
        r = {"copy": copy_probe, "read": read_probe, "pages": page_read_probe}[args.workload](dev)
        return ({"metric": f"HBM {'paged' if args.workload == 'pages' else 'stream'} read GB/s"
                 if args.workload != "copy" else "HBM stream copy GB/s", "value": r["gbs"], "unit": "GB/s",
                          "n_gpus": 1, "avg_us": r["avg_us"], "bytes_per_launch": r["bytes_per_launch"],
                          "higher_is_better": True})
    if args.workload == "c1":
        r = c1_workload(dev)
        by = 256 * ROW_BYTES + 2 * H * D * 2 + 2 * HKV * D * 2
        return ({
            "metric": "config-1 one-layer step latency (append at 255 + decode over 256, B=1)",
            "value": r["gpu_us"], "unit": "us", "n_gpus": 1, "steps": r["reps"], "higher_is_better": False,
            "dtype": "f16", "data": "synthetic (seed 0, the config-1 recipe)",
            "config": {"workload": "C1", "layers": 1, "rows": 256, "calls": "kva_append_decode"},
            "gpu_min_us": r["gpu_min_us"], "alg_bytes": by, "gpu_gbs": by / (r["gpu_us"] * 1e-6) / 1e9,
            "two_calls_us": r["two_calls_us"],
            "cpu_baseline": {"value": r["cpu_us_1"], "unit": "us", "cores": 1, "kind": "port",
                             "all_threads_us": r["cpu_us_all"], "host_logical_cpus": os.cpu_count(),
                             "cpu_model": _cpu_model(),
                             "sample": "the whole config-1 step in the numpy oracle, median of 25 calls, "
                                       "1 BLAS thread (value) and all BLAS threads"}})
    if args.workload in ("c2", "c2graph"):
        graph = args.workload == "c2graph"
        r = c2_workload(dev, args.steps, args.warmup, graph=graph, split=args.split)
        r2 = c2_workload(dev, args.steps, args.warmup, graph=graph, split=args.split, fused=False)
        ms = r["step_us"] * 1e-3
        warm_us = r["wall_s"] * 1e6 / r["steps"]
        return ({"metric": "config-2 decode step time (16 layers, B=1, 128->256 rows)",
                          "value": r["step_us"], "unit": "us/step", "n_gpus": 1, "steps": r["steps"],
                          "ms_per_step": ms, "higher_is_better": False,
                          "timing": "HIP events around each step (plan upload + 16 layers) on the launch "
                                    "stream, L2 and MALL flushed before each step",
                          "step_us_median": r["step_us_median"],
                          "kv_gbs": r["kv_bytes"] / r["steps"] / (r["step_us"] * 1e-6) / 1e9,
                          "back_to_back_us_per_step": warm_us, "dtype": "f16",
                          "data": "synthetic",
                          "launches_per_step": {"kernels": LAYERS, "plan_copies": 1,
                                                "two_calls_kernels": 2 * LAYERS},
                          "two_calls_per_layer": {"step_us": r2["step_us"],
                                                  "back_to_back_us_per_step": r2["wall_s"] * 1e6 / r2["steps"],
                                                  "calls": "kva_append_qknorm_rope + kva_decode"},
                          "config": {"workload": "C2", "calls": "kva_append_decode per layer",
                                     "dispatch": "recorded step replay" if graph else "per-layer calls"}})

    if args.workload == "proj":
        r = proj_workload(dev, args.steps, args.warmup)
        gbs = r["alg_bytes_proj"] / (r["proj_avg_us"] * 1e-6) / 1e9
        ms = r["wall_s"] * 1e3 / r["steps"]
        return ({
            "metric": "config-3 producer GB/s: fused Q/K/V projection + norm + RoPE + append (B=32, hidden 5120)",
            "value": gbs, "unit": "GB/s", "n_gpus": 1, "steps": r["steps"], "warmup": args.warmup,
            "ms_per_step": ms, "higher_is_better": True, "dtype": "f16", "data": "synthetic",
            "config": {"workload": "C3 + producer", "layers": LAYERS, "batch": r["B"], "hidden": r["hidden"]},
            "tok_per_s": r["B"] * r["steps"] / r["wall_s"], "decode_gated_avg_us": r["decode_avg_us"],
            "out_project": {"avg_us": r["out_avg_us"], "alg_bytes_per_launch": r["alg_bytes_out"],
                            "gbs": r["alg_bytes_out"] / (r["out_avg_us"] * 1e-6) / 1e9,
                            "traffic": load_traffic("out_project_c3_traffic.json"),
                            "kernel": "kva_out_project = proj_lds_kernel<2 token tiles, 8 waves, 5 row tiles, "
                                      "6 k-steps, 6 stages> + oproj_finish_kernel"},
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gbs / HBM_PEAK_GBS, "traffic": load_traffic("project_c3_traffic.json"),
                         "kernel": "kva_project_append = proj_lds_kernel<2 token tiles, 8 waves, 7 row tiles, "
                                   "10 k-steps, 6 stages> + proj_finish_kernel",
                         "timing": "HIP events around each step's 16 projections (then its 16 gated decodes, then "
                                   "its 16 O-projections, each group between its own pair), over 16",
                         "avg_us": r["proj_avg_us"], "alg_bytes_per_launch": r["alg_bytes_proj"]}})
    if args.workload == "proj4":
        r = proj_prefill_workload(dev, args.steps, args.warmup)
        us = r["proj_avg_us"]
        tflops = r["flops"] / (us * 1e-6) / 1e12
        alg = r["weight_bytes"] + r["tokens"] * r["hidden"] * 2 + 2 * r["tokens"] * (H + HKV) * D * 2
        return ({
            "metric": "config-4 producer: kva_project_append of 2048 tokens from hidden 5120 (norm + RoPE + append)",
            "value": tflops, "unit": "TFLOP/s", "n_gpus": 1, "steps": r["steps"], "warmup": args.warmup,
            "ms_per_step": r["wall_s"] * 1e3 / r["steps"], "higher_is_better": True, "dtype": "f16",
            "data": "synthetic", "config": {"workload": "C4 producer", "layers": LAYERS, "tokens": r["tokens"],
                                            "hidden": r["hidden"]},
            "path": r["path"], "avg_us_per_layer": us, "weight_bytes": r["weight_bytes"],
            "alg_bytes_per_layer": alg, "weights_gbs": r["weight_bytes"] / (us * 1e-6) / 1e9,
            "roofline": {"bound": "mfma", "achieved": tflops, "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": tflops / MFMA_PEAK_TFLOPS, "traffic": load_traffic("project_c4_traffic.json"),
                         "avg_us": us, "alg_flops_per_launch": r["flops"]}})
    if args.workload == "c4":
        r = c4_workload(dev, args.steps, args.warmup, extras=not args.no_extras)
        tflops = r["flops_per_layer"] / (r["prefill_avg_us"] * 1e-6) / 1e12
        kernel_tflops = (r["flops_per_layer"] / (r["kernel_avg_us"] * 1e-6) / 1e12) if r["kernel_avg_us"] else None
        ms = r["wall_s"] * 1e3 / r["steps"]
        extra = {} if args.no_cpu_baseline else {"cpu_baseline": cpu_baseline_c4()}
        return ({**extra, 
            "metric": "config-4 chunked prefill TFLOP/s, K/V append + causal attention (pp512 after 0/256/1024/2048 rows, B=4)",
            "value": tflops, "unit": "TFLOP/s", "n_gpus": 1, "steps": r["steps"], "warmup": args.warmup,
            "ms_per_step": ms, "higher_is_better": True, "dtype": "f16", "data": "synthetic",
            "config": {"workload": "C4", "layers": LAYERS, "tokens_per_step": r["tokens"]},
            "tok_per_s": r["tokens"] * r["steps"] / r["wall_s"],
            "roofline": {"bound": "mfma", "achieved": tflops, "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": tflops / MFMA_PEAK_TFLOPS, "traffic": load_traffic("prefill_c4_traffic.json"),
                         "kernel": "kva_append_prefill = append_kernel + mq_kernel<1 tile, 8 waves, causal, "
                                   "64-key blocks> + mq_combine_kernel",
                         "timing": "HIP events around each step's 16 calls (caches flushed before the step), "
                                   "over 16; the modes take turns step by step",
                         "two_calls_avg_us": r["two_calls_avg_us"],
                         "prefill_only_avg_us": r["prefill_only_avg_us"],
                         "prefill_only_timing": "each layer's append, then its kva_prefill between a pair of "
                                                "events of its own (the pair's markers in the figure)",
                         "mq_kernel": {"what": "mq_kernel alone: HIP events the library records around its launch "
                                               "(kva_kernel_events), in a second set of as many steps",
                                       "avg_us": r["kernel_avg_us"], "achieved": kernel_tflops,
                                       "frac": kernel_tflops / MFMA_PEAK_TFLOPS if kernel_tflops else None},
                         "avg_us": r["prefill_avg_us"], "alg_flops_per_launch": r["flops_per_layer"],
                         "alg_bytes_per_launch": r["bytes_per_layer"], "mfma_busy": stored_mfma_busy(),
                         "peak_derived": mfma_peak_derived()}})
    if args.workload == "c5":
        r = c5_workload(dev, args.steps, args.warmup)
        gbs = r["alg_bytes_per_layer"] / (r["verify_avg_us"] * 1e-6) / 1e9
        kernel_gbs = r["alg_bytes_per_layer"] / (r["kernel_avg_us"] * 1e-6) / 1e9
        ms = r["wall_s"] * 1e3 / r["steps"]
        extra = {} if args.no_cpu_baseline else {"cpu_baseline": cpu_baseline_c5()}
        return ({**extra, 
            "metric": "config-5 tree-verify attention GB/s (B=64, ctx U[4096,32768], 9-node tree)",
            "value": gbs, "unit": "GB/s", "n_gpus": 1, "steps": r["steps"], "warmup": args.warmup,
            "ms_per_step": ms, "higher_is_better": True, "dtype": "f16", "data": "synthetic",
            "config": {"workload": "C5", "layers": r["layers"], "sum_len": r["sum_len"]},
            "rollback_avg_us": r["rollback_avg_us"],
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gbs / HBM_PEAK_GBS, "traffic": load_traffic("tree_c5_traffic.json"),
                         "kernel": "kva_tree_verify = mq_kernel<1 tile, 4 waves, tree, 32-key blocks> + mq_combine_kernel",
                         "timing": "HIP events around each step's verify calls (its appends first), over the layers",
                         "mq_kernel": {"what": "mq_kernel alone: HIP events the library records around its launch "
                                               "(kva_kernel_events), in a second set of as many steps",
                                       "avg_us": r["kernel_avg_us"], "achieved": kernel_gbs,
                                       "frac": kernel_gbs / HBM_PEAK_GBS},
                         "avg_us": r["verify_avg_us"], "alg_bytes_per_launch": r["alg_bytes_per_layer"]}})
    raise ValueError(args.workload)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="c3", choices=["c1", "c3", "ctx8192", "c2", "c2graph", "c4", "c5", "proj", "proj4", "copy", "read", "pages"])
    ap.add_argument("--split", type=int, default=0, help="decode split tokens (0 = automatic)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="c3: leave out the ctx8192 variant, the bandwidth probes and the other configs; "
                         "c4: time the headline call only (no two-call, prefill-only or kernel-event steps)")
    ap.add_argument("--timeline", action="store_true",
                    help="c3/ctx8192: after the timed steps, record the decode kernels' per-workgroup "
                         "timeline (kva_timeline_enable) for one more step and add its summary")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build runs the path on a single MI355X "
              "(see the sharding design); run it with --gpus 1", file=sys.stderr)
        return 2
    dev = GPUDevice(0)

    if args.workload not in ("c3", "ctx8192"):
        print(json.dumps(workload_line(dev, args)), flush=True)
        return 0
    line = decode_line(dev, args.workload, args)
    if args.workload == "c3" and not args.no_extras:
        # The metric names the fixed ctx=8192 case too: the same step with
        # every sequence at 8192 cached rows.
        sub = decode_line(dev, "ctx8192", args)
        line["ctx8192"] = {k: sub[k] for k in ("value", "unit", "pct_of_hbm_peak", "tok_per_s", "ms_per_step")}
        line["ctx8192"]["config"] = sub["config"]["workload"]
        line["ctx8192"]["roofline"] = {k: sub["roofline"][k] for k in ("achieved", "frac", "avg_us",
                                                                         "alg_bytes_per_launch", "decode_kernel")}
        rd, cp, pr = read_probe(dev), copy_probe(dev), page_read_probe(dev)
        dk = line["roofline"]["decode_kernel"]["achieved"]
        line["peaks"] = {
            "vendor_hbm_gbs": HBM_PEAK_GBS,
            "measured_page_read_gbs": pr["gbs"],
            "measured_stream_read_gbs": rd["gbs"], "measured_stream_copy_gbs": cp["gbs"],
            "decode_kernel_frac_of_page_read": dk / pr["gbs"],
            "decode_call_frac_of_page_read": line["roofline"]["achieved"] / pr["gbs"],
            "method": "kva_hbm_read_pages over config 3's permuted pages (the decode kernel's own per-wave loads, "
                      "no arithmetic, 256 workgroups, four pools rotated); kva_hbm_read over 4 GiB (read-only: "
                      "2048 contiguous shares, two passes of 4 x 16-byte loads per lane in flight) and "
                      "kva_hbm_copy over 4 GiB (bytes read + written); averages of 20 launches between HIP "
                      "events; roofline.frac stays against the vendor 8 TB/s"}
    if args.workload == "c3" and not args.no_extras:
        line["other_configs"] = other_configs(dev, args)
    if not args.no_cpu_baseline:
        log("cpu baseline (numpy oracle, ~10 s at 1 thread + ~10 s at all threads)")
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)
    return 0


def other_configs(dev, args) -> dict:
    """The other configs' figures in the default line (each workload's own
    line, the CPU baselines left out), so one default run records them all."""
    pick = {
        "c1": lambda d: {"us_per_step": d["value"], "two_calls_us": d["two_calls_us"],
                         "gpu_min_us": d["gpu_min_us"], "calls": d["config"]["calls"]},
        "c2": lambda d: {"us_per_step": d["value"], "back_to_back_us_per_step": d["back_to_back_us_per_step"],
                         "two_calls_us_per_step": d["two_calls_per_layer"]["step_us"],
                         "launches_per_step": d["launches_per_step"], "timing": d["timing"]},
        "c4": lambda d: {"tflops": d["value"], "frac": d["roofline"]["frac"], "avg_us": d["roofline"]["avg_us"],
                         "two_calls_avg_us": d["roofline"]["two_calls_avg_us"],
                         "prefill_only_avg_us": d["roofline"]["prefill_only_avg_us"],
                         "mq_kernel_frac": d["roofline"]["mq_kernel"]["frac"],
                         "mq_kernel_avg_us": d["roofline"]["mq_kernel"]["avg_us"],
                         "tok_per_s": d["tok_per_s"], "mfma_busy": d["roofline"]["mfma_busy"]},
        "c5": lambda d: {"gbs": d["value"], "frac": d["roofline"]["frac"], "avg_us": d["roofline"]["avg_us"],
                         "mq_kernel_frac": d["roofline"]["mq_kernel"]["frac"],
                         "mq_kernel_avg_us": d["roofline"]["mq_kernel"]["avg_us"],
                         "rollback_avg_us": d["rollback_avg_us"]},
        "proj": lambda d: {"gbs": d["value"], "frac": d["roofline"]["frac"], "avg_us": d["roofline"]["avg_us"],
                           "out_project_avg_us": d["out_project"]["avg_us"],
                           "out_project_gbs": d["out_project"]["gbs"]},
        "proj4": lambda d: {"tflops": d["value"], "frac": d["roofline"]["frac"], "avg_us": d["roofline"]["avg_us"],
                            "path": d["path"]},
    }
    out = {}
    for w, f in pick.items():
        log(f"other config {w}")
        sub = argparse.Namespace(**{**vars(args), "workload": w, "no_cpu_baseline": True})
        d = workload_line(dev, sub)
        out[w] = {"metric": d["metric"], "unit": d["unit"], **f(d)}
    return out


def decode_line(dev, which, args):
    """The bench line of a decode workload: c3 (ragged) or ctx8192."""
    if which == "c3":
        spec = wl.c3_spec(0)
        lengths, ids, nb = spec.lengths, spec.block_ids, spec.n_blocks
        workload = ("C3 ragged batched decode: B=32, cached rows U[1024,8192] (seed 0), append 1 row "
                    "per sequence then attend over L+1; 16 layers, 24 q / 4 kv heads, d=256, fp16 "
                    "16-token pages with permuted ids")
    else:
        lengths = np.full(32, 8192)
        nblk = (8192 + 1 + 15) // 16
        perm = np.random.default_rng(0).permutation(32 * nblk)
        ids = [[int(x) for x in perm[b * nblk:(b + 1) * nblk]] for b in range(32)]
        nb = 32 * nblk
        workload = ("C3 at fixed ctx: B=32, every sequence 8192 cached rows, append 1 then attend over "
                    "8193; 16 layers, 24 q / 4 kv heads, d=256, fp16 16-token pages, permuted ids")
    r = decode_workload(dev, lengths, ids, nb, args.steps, args.warmup, args.split, which,
                        timeline=getattr(args, "timeline", False))
    kv_total = r["kv_bytes_per_layer"] * LAYERS * r["steps"]
    value = kv_total / r["wall_s"] / 1e9
    ms_step = r["wall_s"] * 1e3 / r["steps"]
    achieved = r["alg_bytes_decode_launch"] / (r["decode_avg_us"] * 1e-6) / 1e9
    kernel_gbs = r["alg_bytes_decode_launch"] / (r["kernel_avg_us"] * 1e-6) / 1e9
    traffic_file = f"decode_{which}_traffic.json"
    return {
        "metric": "decode-attn KV-read HBM GB/s (% of MI355X peak) + tok/s at B=32, ctx=8192",
        "value": value, "unit": "GB/s", "n_gpus": 1, "steps": r["steps"], "warmup": args.warmup,
        "ms_per_step": ms_step, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16", "data": "synthetic",
        "config": {"workload": workload, "layers": LAYERS, "batch": r["B"],
                   "split_tokens": r["split_tokens"], "n_splits": r["n_splits"],
                   "flush": "none: each layer-step reads its own layer's pages, 0.6-1.1 GB, past the 256 MB MALL"},
        "pct_of_hbm_peak": 100.0 * value / HBM_PEAK_GBS,
        "tok_per_s": r["B"] * r["steps"] / r["wall_s"],
        **({"timeline": r["timeline"]} if r["timeline"] else {}),
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS,
                     "traffic": load_traffic(traffic_file),
                     "traffic_source": f"profiles/{traffic_file}: rocprofv3 FETCH_SIZE and WRITE_SIZE of this "
                                       "workload (separate runs), scaled by the copy-kernel calibration stored "
                                       "there; a stored figure, not counted in this run",
                     "kernel": "kva_decode = decode_mfma_kernel<6> (stream-K, QK on MFMA) + combine_kernel<6> (one stream; "
                               "HIP events around each step's 16 calls, after its appends, over 16)",
                     "avg_us": r["decode_avg_us"],
                     "alg_bytes_per_launch": r["alg_bytes_decode_launch"],
                     "decode_kernel": {"what": "decode_mfma_kernel<6> alone: HIP events the library records right "
                                               "before and after its launch (kva_kernel_events), in a second set of "
                                               "as many steps",
                                       "avg_us": r["kernel_avg_us"], "achieved": kernel_gbs,
                                       "frac": kernel_gbs / HBM_PEAK_GBS}},
    }


if __name__ == "__main__":
    sys.exit(main())
