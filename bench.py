#!/usr/bin/env python3
"""HBM bandwidth of the gfx950 tensor-op library on one MI355X.

A step is one pass of the non-GEMM chain of a SmolLM2-360M decoder layer in
f16 at a 4096-token prefill (LayerChain): RMSNorm [4096, 960]; RoPE of Q
and K with the KV-cache append and repeat_kv 5 -> 15 heads, one launch;
causal scale/mask + softmax on [15, 4096, 4096] scores; SwiGLU [4096, 2560];
residual add -- 5 launches.  Inputs are resident in HBM before timing.  Step
i runs on buffer set i mod R (1.1 GB each, so every set is four times the
256 MB Infinity Cache); K steps are launched back to back on one stream with
events around them, after W warm-up steps.  GB/s = the step's algorithmic
bytes (each launch's inputs read once and outputs written once) / time per
step.  The same K steps then run again with the softmax -- 3/4 of the
step's time -- recording its own start and end in every step; its mean
launch duration gives the roofline fraction (a stamped launch adds ~6-7 us
to its step, which is why the step time comes from the unstamped pass).  The
CPU oracle runs the same chain on set 0's inputs (one core,
then every core), and every stage of the GPU's outputs is checked against
it.

The JSON line (stdout, one line) carries the headline, the roofline, the CPU
baseline, the [4096, 1536] batch step and a summary of the per-op table;
the full per-op table -- each op alone on rotated buffer copies, one launch
and sustained, at every configuration's shapes -- goes to stderr and to
--per-op-out.

    python bench.py [--steps K] [--warmup W] [--sets R] [--no-cpu] [--quick]
"""

from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from rustllm_amd import abi, synth  # noqa: E402

PEAK_GBS = 8000.0
PEAK_F16_TFLOPS = 2500.0  # MI355X dense f16 MFMA
PEAK_F32_TFLOPS = 157.3  # MI355X dense f32 MFMA
METRIC = "achieved HBM GB/s & % of MI355X peak per op (RMSNorm, softmax, SwiGLU, RoPE)"
F32, F16 = np.float32, np.float16
T, H = 4096, 1536


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


class Op:
    """One kernel launch on one buffer set: `launch(ctx, bufs)`, its bytes and
    the part of them it writes."""

    def __init__(self, name, dtype, shape, nbytes, launch, write=None):
        self.name, self.dtype, self.shape, self.nbytes, self.launch = (name, dtype, shape, nbytes,
                                                                       launch)
        self.write = write


def batch_inputs(seed_tag: str):
    """Host arrays of the [4096, 1536] elementwise batch (N(0,1) values)."""
    arrs = {}
    for dt in (F32, F16):
        tag = np.dtype(dt).name
        arrs[f"a_{tag}"] = synth.normal(synth.seed_for("c2", "a", tag, seed_tag), (T, H), 0, 1, dt)
        arrs[f"b_{tag}"] = synth.normal(synth.seed_for("c2", "b", tag, seed_tag), (T, H), 0, 1, dt)
        arrs[f"bias_{tag}"] = synth.normal(synth.seed_for("c2", "bias", tag, seed_tag), (H,), 0, 1,
                                           dt)
        arrs[f"view_{tag}"] = synth.normal(synth.seed_for("c2", "view", tag, seed_tag),
                                           (1, 4096, 9, 64), 0, 1, dt)
        arrs[f"kv_{tag}"] = synth.normal(synth.seed_for("c2", "kv", tag, seed_tag),
                                         (1, 3, 4096, 64), 0, 1, dt)
    return arrs


VIEW_DIMS = [1, 9, 4096, 64]
VIEW_STRIDES = [4096 * 9 * 64, 64, 9 * 64, 1]


def batch_ops():
    ops = []
    n = T * H
    for dt in (F32, F16):
        tag = np.dtype(dt).name
        es = np.dtype(dt).itemsize
        sfx = "f16" if dt == F16 else "f32"

        def mk(kind, tag=tag):
            return lambda c, b: kind(c, b, tag)

        ops.append(Op(f"add_{sfx}", sfx, [T, H], 3 * n * es,
                      mk(lambda c, b, t: c.add(b[f"a_{t}"], b[f"b_{t}"], b[f"o1_{t}"])), n * es))
        ops.append(Op(f"mul_{sfx}", sfx, [T, H], 3 * n * es,
                      mk(lambda c, b, t: c.mul(b[f"a_{t}"], b[f"b_{t}"], b[f"o2_{t}"])), n * es))
        ops.append(Op(f"silu_{sfx}", sfx, [T, H], 2 * n * es,
                      mk(lambda c, b, t: c.silu(b[f"a_{t}"], b[f"o3_{t}"])), n * es))
        ops.append(Op(f"swiglu_{sfx}", sfx, [T, H], 3 * n * es,
                      mk(lambda c, b, t: c.swiglu(b[f"a_{t}"], b[f"b_{t}"], b[f"o4_{t}"])),
                      n * es))
        ops.append(Op(f"add_broadcast_{sfx}", sfx, [T, H], 2 * n * es + H * es,
                      mk(lambda c, b, t: c.add_broadcast(b[f"a_{t}"], b[f"bias_{t}"],
                                                         b[f"o5_{t}"])), n * es))
    ops.append(Op("cast_f32_to_f16", "f32->f16", [T, H], n * 6,
                  lambda c, b: c.cast(b["a_float32"], F16, b["cast_h"]), n * 2))
    ops.append(Op("cast_f16_to_f32", "f16->f32", [T, H], n * 6,
                  lambda c, b: c.cast(b["a_float16"], F32, b["cast_f"]), n * 4))
    nv = 9 * 4096 * 64
    nkv = 3 * 4096 * 64
    for dt in (F32, F16):
        tag = np.dtype(dt).name
        es = np.dtype(dt).itemsize
        sfx = "f16" if dt == F16 else "f32"
        ops.append(Op(f"contiguous_{sfx}", sfx, VIEW_DIMS, 2 * nv * es,
                      lambda c, b, t=tag: c.contiguous(b[f"view_{t}"], VIEW_DIMS, VIEW_STRIDES,
                                                       b[f"vo_{t}"]), nv * es))
        ops.append(Op(f"repeat_kv_{sfx}", sfx, [1, 3, 4096, 64], (nkv + 3 * nkv) * es,
                      lambda c, b, t=tag: c.repeat_kv(b[f"kv_{t}"], 3, b[f"kvo_{t}"]),
                      3 * nkv * es))
    return ops


def batch_set(ctx, host):
    """Device buffers of one set: the inputs plus one output per op."""
    b = {k: ctx.upload(v) for k, v in host.items()}
    for dt in (F32, F16):
        tag = np.dtype(dt).name
        for i in range(1, 6):
            b[f"o{i}_{tag}"] = ctx.empty((T, H), dt)
        b[f"vo_{tag}"] = ctx.empty(VIEW_DIMS, dt)
        b[f"kvo_{tag}"] = ctx.empty((1, 9, 4096, 64), dt)
    b["cast_h"] = ctx.empty((T, H), F16)
    b["cast_f"] = ctx.empty((T, H), F32)
    return b


def set_bytes(b) -> int:
    return sum(v.byte_len for v in b.values())


# Graph-replayed figures: the sustained time of each op (back-to-back
# launches recorded in one graph and replayed), the chain and the batch step
# recorded as graphs.  On by default; `--no-graph-batch` leaves them out.
# Under `rocprofv3 --kernel-trace` a run that created, replayed and destroyed
# one graph per op once ended in a SIGSEGV inside hipGraphLaunch, so every
# graph is kept until the process exits rather than destroyed after use.
GRAPH_BATCH = True
_LIVE_GRAPHS = []


def time_graphs(ctx, graphs, launches_per_graph, reps, warmup=2):
    """Replays `graphs` round-robin `reps` times; returns ms per launch."""
    for i in range(warmup):
        ctx.graph_launch(graphs[i % len(graphs)])
    ctx.finish()
    start, end = ctx.event(), ctx.event()
    ctx.record(start)
    for i in range(reps):
        ctx.graph_launch(graphs[i % len(graphs)])
    ctx.record(end)
    ms = ctx.elapsed_ms(start, end)
    ctx.destroy_event(start)
    ctx.destroy_event(end)
    return ms / (reps * launches_per_graph)


def capture(ctx, fn):
    """fn's launches recorded as a graph, one kernel per op (the fusion of
    recorded streaming ops off: these graphs stand for a given sequence of
    launches)."""
    ctx.set_fusion(False)
    ctx.capture_begin()
    try:
        fn()
    finally:
        g = ctx.capture_end()
        ctx.set_fusion(True)
    return g


def time_step(ctx, ops, sets, steps, warmup):
    """ms per step of the [4096, 1536] batch: the steps over the buffer sets
    recorded in turn into one graph (a step per set, so a replay is
    len(sets) steps; `steps` is a multiple of the set count), replayed
    after `warmup` steps, events around the timed replays."""
    assert steps % len(sets) == 0
    ctx.capture_begin()
    try:
        for s in sets:
            for op in ops:
                op.launch(ctx, s)
    finally:
        graph = ctx.capture_end()
    _LIVE_GRAPHS.append(graph)
    ms = time_graphs(ctx, [graph], len(sets), steps // len(sets),
                     warmup=max(1, -(-warmup // len(sets))))
    ctx.finish()
    return ms


def kernel_times_us(ctx, launches, reps, batch=True):
    """Device time of `reps` launches (cycling through `launches`, one kernel
    each), every one bracketed by events that the kernel itself stamps at its
    start and end -- the same per-dispatch duration a kernel trace reports.
    Also returns the time per launch of a batch of back-to-back launches
    (recorded once as a graph and replayed, so host launch cost is out of
    it and the gaps between kernels are in), or None for ops that cannot be
    recorded."""
    for fn in launches:
        fn()
    ctx.finish()
    evs = [(ctx.event(), ctx.event()) for _ in range(reps)]
    for i, (start, stop) in enumerate(evs):
        ctx.time_next_kernel(start, stop)
        launches[i % len(launches)]()
    ctx.finish()
    us = [ctx.elapsed_ms(start, stop) * 1e3 for start, stop in evs]
    for e in [e for pair in evs for e in pair]:
        ctx.destroy_event(e)
    return us, (graph_batch_us(ctx, launches) if GRAPH_BATCH and batch else None), \
        len(launches) + reps


def call_times_us(ctx, calls, reps, groups=3):
    """Time per call of `reps` calls back to back (cycling through `calls`),
    events recorded on the context's stream around each group of them: for
    entry points that may enqueue more than one kernel (the per-launch stamps
    of kernel_times_us see only the first)."""
    for fn in calls:
        fn()
    ctx.finish()
    out = []
    for _ in range(groups):
        start, stop = ctx.event(), ctx.event()
        ctx.record(start)
        for i in range(reps):
            calls[i % len(calls)]()
        ctx.record(stop)
        ctx.finish()
        out.append(ctx.elapsed_ms(start, stop) * 1e3 / reps)
        ctx.destroy_event(start)
        ctx.destroy_event(stop)
    return out, None


def graph_batch_us(ctx, launches, min_per_graph=32, replays=8):
    """us per launch of back-to-back launches replayed as a graph: one launch
    on each of the op's buffer sets (>= 1 GiB in total, so a replay streams
    from HBM, not from the 256 MB Infinity Cache), at least `min_per_graph`.
    One kernel per launch: the fusion of recorded streaming ops is off here."""
    per_graph = max(min_per_graph, len(launches))
    ctx.set_fusion(False)
    ctx.capture_begin()
    failed = False
    try:
        for i in range(per_graph):
            launches[i % len(launches)]()
    except abi.RustLLMError:
        failed = True
    finally:
        graph = ctx.capture_end()
        ctx.set_fusion(True)
    _LIVE_GRAPHS.append(graph)
    if failed:
        return None
    ms = time_graphs(ctx, [graph], per_graph, replays)
    ctx.finish()
    return ms * 1e3


def op_row(name, dtype, shape, nbytes, timing, write=None):
    """One per-op line; `write` = the bytes of `nbytes` the op writes (None
    for ops that HBM does not bound: matrix-core and latency-bound rows)."""
    us_list, batch_us = timing[0], timing[1]
    us = float(np.mean(us_list))
    gbs = nbytes / (us * 1e-6) / 1e9
    batch = "   n/a" if batch_us is None else f"{batch_us:7.2f}"
    log(f"  {name:34s} {str(shape):20s} {us:9.2f} us {gbs:8.1f} GB/s ({100 * gbs / PEAK_GBS:5.1f}%)"
        f"  graph batch {batch} us/launch")
    row = {"op": name, "dtype": dtype, "shape": shape, "bytes": nbytes, "us": round(us, 3),
           "us_min": round(float(np.min(us_list)), 3),
           "GB/s": round(gbs, 1), "pct_peak": round(100 * gbs / PEAK_GBS, 1),
           "us_graph_batch": None, "GB/s_graph_batch": None, "pct_peak_graph_batch": None}
    if write is not None:
        row["read_bytes"], row["write_bytes"] = nbytes - write, write
    if len(timing) > 2:  # kernel dispatches of the one-launch timing: warm-up, then timed
        row["dispatches"] = timing[2]
        row["timed"] = len(us_list)
    if batch_us is not None:
        gb = nbytes / (batch_us * 1e-6) / 1e9
        row.update({"us_graph_batch": round(batch_us, 3), "GB/s_graph_batch": round(gb, 1),
                    "pct_peak_graph_batch": round(100 * gb / PEAK_GBS, 1)})
    return row


class _KeyProbe(dict):
    """A buffer set that records which buffers an op reads or writes."""

    def __init__(self, base):
        super().__init__(base)
        self.used = set()

    def __getitem__(self, key):
        self.used.add(key)
        return super().__getitem__(key)


class _NullContext:
    """Accepts any op call and does nothing (for _KeyProbe runs)."""

    def __getattr__(self, name):
        return lambda *args, **kwargs: None


def per_op_rows(ctx, ops, sets, reps):
    """Each op alone, cycling through copies of its own buffers: as many
    copies as make >= 1 GiB (4 .. 256), so its reads come from HBM."""
    rows = []
    for op in ops:
        probe = _KeyProbe(sets[0])
        op.launch(_NullContext(), probe)
        footprint = sum(sets[0][k].byte_len for k in probe.used)
        n = int(min(256, max(4, -(-(1 << 30) // footprint))))
        op_sets = [{k: (s[k] if i < len(sets) else ctx.clone(s[k])) for k in probe.used}
                   for i, s in ((i, sets[i % len(sets)]) for i in range(n))]
        launches = [lambda s=s, op=op: op.launch(ctx, s) for s in op_sets]
        rows.append(op_row(op.name, op.dtype, op.shape, op.nbytes,
                           kernel_times_us(ctx, launches, reps), op.write))
        del launches, op_sets
    return rows


# ------------------------------------------------------- the other shapes

def extra_rows(ctx, reps, quick):
    """RMSNorm over hidden {576, 768, 960} x tokens, scale/mask + softmax on
    [9, 2048, 2048] scores and each op of the SmolLM2-360M decoder layer
    alone -- same method, rotated buffer sets."""
    rows = []

    def measure(name, dtype, shape, nbytes, make_set, launch, write=None):
        # As many buffer sets as make >= 1 GiB in total (4 .. 256 sets).
        first = make_set(0)
        footprint = sum(b.byte_len for b in first)
        nsets = int(min(256, max(4, -(-(1 << 30) // max(footprint, 1)))))
        sets = [first] + [make_set(i) for i in range(1, nsets)]
        launches = [lambda s=s: launch(s) for s in sets]
        rows.append(op_row(name, dtype, shape, nbytes, kernel_times_us(ctx, launches, reps),
                           write))
        del sets, launches, first

    tokens_list = [4096, 16384] if quick else [1, 16, 256, 4096, 16384]
    for dt in (F32, F16):
        es = np.dtype(dt).itemsize
        sfx = "f16" if dt == F16 else "f32"
        for hidden in (576, 768, 960):
            w = ctx.upload(synth.uniform_range(synth.seed_for("w", hidden), (hidden,), 0.5, 1.5,
                                               dt))
            for tokens in tokens_list:
                x = synth.normal(synth.seed_for("rms", tokens, hidden, sfx), (tokens, hidden), 0,
                                 2.0, dt)
                nbytes = tokens * hidden * 2 * es + hidden * es
                measure(f"rmsnorm_{sfx}", sfx, [tokens, hidden], nbytes,
                        lambda i, x=x, tokens=tokens, hidden=hidden, dt=dt:
                        (ctx.upload(x), ctx.empty((tokens, hidden), dt)),
                        lambda s, w=w: ctx.rmsnorm(s[0], w, 1e-5, s[1]),
                        tokens * hidden * es)

    # attention scores: prefill [9, 2048, 2048] causal, scale 1/8; decode [9, 1, 2048]
    def logits(shape, dt=F32):
        x = synth.normal(synth.seed_for("logits", *shape), shape, 0, 4.0, F32)
        u = synth.uniform(synth.seed_for("spike", *shape), x.size).reshape(shape)
        x[u < 0.01] = 20.0
        return x.astype(dt)

    pre = logits((9, 2048, 2048))
    n = pre.size
    unmasked = 9 * (2048 * 2049 // 2)
    for name, nbytes, fn in [
        ("attention_softmax_f32", unmasked * 4 + n * 4,
         lambda s: ctx.attention_softmax(s[0], 0.125, 0, s[1])),
        ("attention_scale_mask_f32", unmasked * 4 + n * 4,
         lambda s: ctx.scale_mask(s[0], 0.125, 0, s[1])),
        ("softmax_f32", 2 * n * 4, lambda s: ctx.softmax(s[0], s[1])),
    ]:
        measure(name, "f32", [9, 2048, 2048], nbytes,
                lambda i: (ctx.upload(pre), ctx.empty(pre.shape, F32)), fn, n * 4)
    dec = logits((9, 1, 2048))
    measure("attention_softmax_f32", "f32", [9, 1, 2048], 2 * dec.size * 4,
            lambda i: (ctx.upload(dec), ctx.empty(dec.shape, F32)),
            lambda s: ctx.attention_softmax(s[0], 0.125, 2047, s[1]), dec.size * 4)

    # SmolLM2-360M decoder layer, f16, 4096 tokens
    hid, qh, kvh, hd, ffn, tok = 960, 15, 5, 64, 2560, 4096
    c, s_ = _rope_table(hd, tok)
    dc, ds = ctx.upload(c), ctx.upload(s_)
    wn = ctx.upload(synth.uniform_range(1, (hid,), 0.5, 1.5, F16))
    x = synth.normal(synth.seed_for("c5", "x"), (tok, hid), 0, 1, F16)
    measure("layer.1 rmsnorm_f16", "f16", [tok, hid], tok * hid * 4 + hid * 2,
            lambda i: (ctx.upload(x), ctx.empty((tok, hid), F16)),
            lambda s: ctx.rmsnorm(s[0], wn, 1e-5, s[1]), tok * hid * 2)
    for heads, label in ((qh, "Q"), (kvh, "K")):
        proj = synth.normal(synth.seed_for("c5", label), (1, tok, heads, hd), 0, 1, F16)
        dims, strides = [1, heads, tok, hd], [tok * heads * hd, hd, heads * hd, 1]
        nbytes = 2 * proj.size * 2 + 2 * tok * (hd // 2) * 4  # + cos/sin tables, once
        measure(f"layer.2 rope_{label}_f16 (fused gather)", "f16", dims, nbytes,
                lambda i, proj=proj, dims=dims: (ctx.upload(proj), ctx.empty(dims, F16)),
                lambda s, dims=dims, strides=strides: ctx.rope_strided(s[0], dims, strides, dc,
                                                                        ds, 0, s[1]),
                proj.size * 2)
        cont = np.ascontiguousarray(proj.transpose(0, 2, 1, 3))
        measure(f"layer.2 rope_{label}_f16", "f16", list(cont.shape), nbytes,
                lambda i, cont=cont: (ctx.upload(cont), ctx.empty(cont.shape, F16)),
                lambda s: ctx.rope(s[0], dc, ds, 0, s[1]), proj.size * 2)
    # K rotated straight into a [1, 5, 4096, 64] cache, V gathered into one
    proj_k = synth.normal(synth.seed_for("c5", "Kc"), (1, tok, kvh, hd), 0, 1, F16)
    kdims, kstrides = [1, kvh, tok, hd], [tok * kvh * hd, hd, kvh * hd, 1]
    measure("layer.2 rope_K_f16 -> KV cache (fused)", "f16", kdims,
            2 * proj_k.size * 2 + 2 * tok * (hd // 2) * 4,
            lambda i: (ctx.upload(proj_k), ctx.empty(kdims, F16)),
            lambda s: ctx.rope_kv_cache_write(s[0], kdims, kstrides, dc, ds, 0, s[1]),
            proj_k.size * 2)
    measure("layer.2 V_f16 -> KV cache (fused gather)", "f16", kdims, 2 * proj_k.size * 2,
            lambda i: (ctx.upload(proj_k), ctx.empty(kdims, F16)),
            lambda s: ctx.kv_cache_write_strided(s[0], kdims, kstrides, s[1], 0), proj_k.size * 2)
    # Q and K rotated, K and V appended, as one launch
    proj_q = synth.normal(synth.seed_for("c5", "Qc"), (1, tok, qh, hd), 0, 1, F16)
    qdims, qstrides = [1, qh, tok, hd], [tok * qh * hd, hd, qh * hd, 1]
    measure("layer.2 QKV rotate + KV append (one launch)", "f16", [1, qh + 2 * kvh, tok, hd],
            2 * (proj_q.size + 2 * proj_k.size) * 2 + 2 * tok * (hd // 2) * 4,
            lambda i: (ctx.upload(proj_q), ctx.upload(proj_k), ctx.upload(proj_k),
                       ctx.empty(qdims, F16), ctx.empty(kdims, F16), ctx.empty(kdims, F16)),
            lambda s: ctx.qkv_rope_kv_append((s[0], qdims, qstrides), (s[1], kdims, kstrides),
                                             (s[2], kdims, kstrides), dc, ds, 0, s[4], s[5],
                                             s[3]),
            (proj_q.size + 2 * proj_k.size) * 2)
    # ... and repeat_kv of both caches (5 -> 15 heads) in the same launch
    n_rep = qh // kvh
    measure("layer.2 QKV + KV append + repeat_kv (one launch)", "f16",
            [1, qh + 2 * kvh, tok, hd],
            2 * proj_q.size * 2 + 2 * proj_k.size * (1 + 1 + n_rep) * 2
            + 2 * tok * (hd // 2) * 4,
            lambda i: (ctx.upload(proj_q), ctx.upload(proj_k), ctx.upload(proj_k),
                       ctx.empty(qdims, F16), ctx.empty(kdims, F16), ctx.empty(kdims, F16),
                       ctx.empty(qdims, F16), ctx.empty(qdims, F16)),
            lambda s: ctx.qkv_rope_kv_append_repeat(
                (s[0], qdims, qstrides), (s[1], kdims, kstrides), (s[2], kdims, kstrides), dc,
                ds, 0, s[4], s[5], n_rep, s[3], s[6], s[7]),
            (proj_q.size + 2 * proj_k.size * (1 + n_rep)) * 2)
    # token embedding gather: 4096 ids into a [49152, 960] f16 table
    # (each set has its own 94 MB table, so the gathered rows come from HBM)
    vocab = 49152
    emb = synth.normal(synth.seed_for("c5", "emb"), (vocab, hid), 0, 1, F16)
    ids = (synth.uniform(synth.seed_for("c5", "ids"), tok) * vocab).astype(np.uint32)
    measure("layer.0 embedding_f16", "f16", [tok, hid], 2 * tok * hid * 2 + tok * 4,
            lambda i: (ctx.upload(emb), ctx.empty((tok, hid), F16)),
            lambda s: ctx.embedding(s[0], ids, s[1]), tok * hid * 2)
    kv = synth.normal(synth.seed_for("c5", "kv"), (1, kvh, tok, hd), 0, 1, F16)
    measure("layer.3 repeat_kv_f16", "f16", [1, kvh, tok, hd], (kv.size + 3 * kv.size) * 2,
            lambda i: (ctx.upload(kv), ctx.empty((1, qh, tok, hd), F16)),
            lambda s: ctx.repeat_kv(s[0], 3, s[1]), 3 * kv.size * 2)
    if not quick:
        rng = np.random.default_rng(5)
        sc = rng.standard_normal((qh, tok, tok), dtype=np.float32).astype(F16)
        n = sc.size
        unm = qh * (tok * (tok + 1) // 2)
        measure("layer.4 attention_softmax_f16", "f16", [qh, tok, tok], unm * 2 + n * 2,
                lambda i: (ctx.upload(sc), ctx.empty(sc.shape, F16)),
                lambda s: ctx.attention_softmax(s[0], 0.125, 0, s[1]), n * 2)
        del sc
    g = synth.normal(synth.seed_for("c5", "g"), (tok, ffn), 0, 1, F16)
    u = synth.normal(synth.seed_for("c5", "u"), (tok, ffn), 0, 1, F16)
    measure("layer.5 swiglu_f16", "f16", [tok, ffn], 3 * g.size * 2,
            lambda i: (ctx.upload(g), ctx.upload(u), ctx.empty(g.shape, F16)),
            lambda s: ctx.swiglu(s[0], s[1], s[2]), g.size * 2)
    r = synth.normal(synth.seed_for("c5", "r"), (tok, hid), 0, 1, F16)
    measure("layer.6 residual add_f16", "f16", [tok, hid], 3 * r.size * 2,
            lambda i: (ctx.upload(x), ctx.upload(r), ctx.empty(r.shape, F16)),
            lambda s: ctx.add(s[0], s[1], s[2]), r.size * 2)
    rows.extend(attention_rows(ctx, qh, kvh, hd, tok, reps))
    if not quick:
        rows.append(fused_layer_row(ctx, hid, qh, kvh, hd, ffn, tok, wn, dc, ds))
    # [64, 768] f32 (the reference's CPU-runnable case), fused add + RMSNorm
    # (writes the sum and the norm)
    x0 = synth.normal(1, (64, 768), 0, 1, F32)
    w0 = ctx.upload(synth.uniform_range(2, (768,), 0.5, 1.5, F32))
    measure("add_rmsnorm_f32", "f32", [64, 768], 64 * 768 * 4 * 4 + 768 * 4,
            lambda i: (ctx.upload(x0), ctx.upload(x0), ctx.empty(x0.shape, F32),
                       ctx.empty(x0.shape, F32)),
            lambda s: ctx.add_rmsnorm(s[0], s[1], w0, 1e-5, s[2], s[3]), 2 * x0.size * 4)
    return rows


def attention_flops(qh, q_len, kv_len, hd, start):
    """2 x 2 D flops per (query, visible key): QK^T and PV, causal."""
    keys = sum(min(kv_len, start + i + 1) for i in range(q_len))
    return 4.0 * hd * keys * qh


def attention_rows(ctx, qh, kvh, hd, tok, reps):
    """SmolLM2-360M attention core at 4096 tokens, f16: the fused pass
    (rl_attention_f16, matrix cores; TFLOP/s vs the 2.5 PF dense f16 peak; and
    rl_attention_f32 on the same inputs vs the 157.3 TF f32 peak),
    the reference's unfused calls (gqa_qk, scale/mask + softmax, gqa_pv) one
    by one and as one graph, and a decode step over a 4096-row cache."""
    rows = []
    q = synth.normal(synth.seed_for("c5", "attn-q"), (1, qh, tok, hd), 0, 1, F16)
    k = synth.normal(synth.seed_for("c5", "attn-k"), (1, kvh, tok, hd), 0, 1, F16)
    v = synth.normal(synth.seed_for("c5", "attn-v"), (1, kvh, tok, hd), 0, 1, F16)
    flops = attention_flops(qh, tok, tok, hd, 0)
    sets = [(ctx.upload(q), ctx.upload(k), ctx.upload(v), ctx.empty(q.shape, F16))
            for _ in range(4)]
    io_bytes = (q.size + 2 * k.size + q.size) * 2
    timing = kernel_times_us(ctx, [lambda s=s: ctx.attention(s[0], s[1], s[2], 0.125, 0, None,
                                                                s[3]) for s in sets], reps)
    row = op_row("layer.4 attention_f16 (fused, matrix cores)", "f16", [1, qh, tok, hd],
                 io_bytes, timing)
    us = row["us"]
    row.update({"flops": flops, "TFLOP/s": round(flops / (us * 1e-6) / 1e12, 1),
                "pct_peak_mfma": round(100 * flops / (us * 1e-6) / 1e12 / PEAK_F16_TFLOPS, 1)})
    log(f"    -> {row['TFLOP/s']} TFLOP/s ({row['pct_peak_mfma']}% of the dense f16 peak)")
    rows.append(row)
    # the same layer in f32 (the f32 matrix-core kernel; vs the 157.3 TFLOP/s f32 peak)
    sets32 = [tuple(ctx.upload(x.astype(np.float32)) for x in (q, k, v)) +
              (ctx.empty(q.shape, np.float32),) for _ in range(2)]
    timing = kernel_times_us(ctx, [lambda s=s: ctx.attention(s[0], s[1], s[2], 0.125, 0, None,
                                                                s[3]) for s in sets32], reps)
    row32 = op_row("layer.4 attention_f32 (fused, matrix cores)", "f32", [1, qh, tok, hd],
                   io_bytes * 2, timing)
    row32.update({"flops": flops, "TFLOP/s": round(flops / (row32["us"] * 1e-6) / 1e12, 1),
                  "pct_peak_mfma": round(100 * flops / (row32["us"] * 1e-6) / 1e12 /
                                         PEAK_F32_TFLOPS, 1)})
    log(f"    -> {row32['TFLOP/s']} TFLOP/s ({row32['pct_peak_mfma']}% of the dense f32 peak)")
    rows.append(row32)
    del sets32
    # a prefill of 512 tokens after 4096 - 512 cached ones (f16, the layer's K
    # and V): few 128-query tiles, so each tile's keys are split over
    # workgroups and merged by a second kernel; timed per whole call
    pre = tok // 8
    qp = synth.normal(synth.seed_for("c5", "attn-q-prefill"), (1, qh, pre, hd), 0, 1, F16)
    psets = [(ctx.upload(qp), ctx.empty(qp.shape, F16)) for _ in range(2)]
    pflops = attention_flops(qh, pre, tok, hd, tok - pre)
    rowp = op_row(f"layer.4 attention_f16 prefill of {pre} tokens after {tok - pre} cached "
                  "(key chunks, every launch of a call timed)", "f16", [1, qh, pre, hd],
                  (2 * qp.size + 2 * k.size) * 2,
                  call_times_us(ctx, [lambda s=s: ctx.attention(s[0], sets[0][1], sets[0][2], 0.125,
                                                                 tok - pre, None, s[1])
                                      for s in psets], reps))
    rowp.update({"flops": pflops, "TFLOP/s": round(pflops / (rowp["us"] * 1e-6) / 1e12, 1),
                 "pct_peak_mfma": round(100 * pflops / (rowp["us"] * 1e-6) / 1e12 /
                                        PEAK_F16_TFLOPS, 1)})
    log(f"    -> {rowp['TFLOP/s']} TFLOP/s ({rowp['pct_peak_mfma']}% of the dense f16 peak)")
    rows.append(rowp)
    del psets
    # the reference's calls: scores written (503 MB), softmaxed, read back
    n_scores = qh * tok * tok
    unmasked = qh * (tok * (tok + 1) // 2)
    s0 = sets[0]
    sc = [ctx.empty((1, qh, tok, tok), F16) for _ in range(2)]
    pr = [ctx.empty((1, qh, tok, tok), F16) for _ in range(2)]
    out = ctx.empty(q.shape, F16)
    qk_bytes = (q.size + k.size + n_scores) * 2
    rows.append(op_row("layer.4 gqa_qk_f16 (scores)", "f16", [1, qh, tok, tok], qk_bytes,
                       kernel_times_us(ctx, [lambda i=i: ctx.gqa_qk(s0[0], s0[1], None, sc[i])
                                             for i in range(2)], reps), n_scores * 2))
    pv_bytes = (n_scores + v.size + q.size) * 2
    rows.append(op_row("layer.4 gqa_pv_f16", "f16", [1, qh, tok, hd], pv_bytes,
                       kernel_times_us(ctx, [lambda i=i: ctx.gqa_pv(pr[i], s0[2], out)
                                             for i in range(2)], reps), q.size * 2))
    # the same two products in f32 (f32 matrix cores; 2 x 32.2 GFLOP over all keys)
    q32, k32, v32 = (ctx.upload(x.astype(np.float32)) for x in (q, k, v))
    sc32 = ctx.empty((1, qh, tok, tok), np.float32)
    out32 = ctx.empty(q.shape, np.float32)
    mm_flops = 2.0 * qh * tok * tok * hd
    for name, fn, nbytes in (
            ("layer.4 gqa_qk_f32 (scores)", lambda: ctx.gqa_qk(q32, k32, None, sc32),
             qk_bytes * 2),
            ("layer.4 gqa_pv_f32", lambda: ctx.gqa_pv(sc32, v32, out32), pv_bytes * 2)):
        r32 = op_row(name, "f32", [1, qh, tok, tok if "qk" in name else hd], nbytes,
                     kernel_times_us(ctx, [fn], max(10, reps // 5)))
        r32.update({"flops": mm_flops,
                    "TFLOP/s": round(mm_flops / (r32["us"] * 1e-6) / 1e12, 1),
                    "pct_peak_mfma": round(100 * mm_flops / (r32["us"] * 1e-6) / 1e12 /
                                           PEAK_F32_TFLOPS, 1)})
        log(f"    -> {r32['TFLOP/s']} TFLOP/s ({r32['pct_peak_mfma']}% of the dense f32 peak)")
        rows.append(r32)
    del q32, k32, v32, sc32, out32

    def chain(i):
        ctx.gqa_qk(s0[0], s0[1], None, sc[i])
        ctx.attention_softmax(sc[i], 0.125, 0, pr[i])
        ctx.gqa_pv(pr[i], s0[2], out)

    graphs = [capture(ctx, lambda i=i: chain(i)) for i in range(2)]
    ms = time_graphs(ctx, graphs, 1, 10)
    ctx.finish()
    for g in graphs:
        ctx.graph_destroy(g)
    chain_us = ms * 1e3
    chain_bytes = qk_bytes + unmasked * 2 + n_scores * 2 + pv_bytes
    log(f"  {'layer.4 unfused QK, softmax, PV (graph)':34s} {chain_us:9.2f} us "
        f"(fused: {us:.2f} us, {chain_us / us:.1f}x)")
    rows.append({"op": "layer.4 unfused gqa_qk + scale/mask softmax + gqa_pv (one graph)",
                 "dtype": "f16", "shape": [1, qh, tok, hd], "bytes": chain_bytes,
                 "us": round(chain_us, 3), "us_min": None,
                 "GB/s": round(chain_bytes / (chain_us * 1e-6) / 1e9, 1),
                 "pct_peak": round(100 * chain_bytes / (chain_us * 1e-6) / 1e9 / PEAK_GBS, 1),
                 "flops": flops, "TFLOP/s": round(flops / (chain_us * 1e-6) / 1e12, 1),
                 "fused_speedup": round(chain_us / us, 2),
                 "us_graph_batch": None, "GB/s_graph_batch": None, "pct_peak_graph_batch": None})
    del sc, pr
    # the same unfused calls at an odd length (4093 tokens): score rows that
    # start off the 16-byte grid
    rl_tok = tok - 3
    q_r = ctx.upload(np.ascontiguousarray(q[:, :, :rl_tok]))
    n_r = qh * rl_tok * rl_tok
    unmasked_r = qh * (rl_tok * (rl_tok + 1) // 2)
    sc_r = [ctx.empty((1, qh, rl_tok, rl_tok), F16) for _ in range(2)]
    pr_r = [ctx.empty((1, qh, rl_tok, rl_tok), F16) for _ in range(2)]
    out_r = ctx.empty((1, qh, rl_tok, hd), F16)
    kv_r = kvh * rl_tok * hd
    for name, fns, nbytes, write in (
            ("layer.4 ragged gqa_qk_f16 (4093 keys)",
             [lambda i=i: ctx.gqa_qk(q_r, s0[1], rl_tok, sc_r[i]) for i in range(2)],
             (qh * rl_tok * hd + kv_r + n_r) * 2, n_r * 2),
            ("layer.4 ragged attention_softmax_f16 (4093 keys)",
             [lambda i=i: ctx.attention_softmax(sc_r[i], 0.125, 0, pr_r[i]) for i in range(2)],
             (unmasked_r + n_r) * 2, n_r * 2),
            ("layer.4 ragged gqa_pv_f16 (4093 keys)",
             [lambda i=i: ctx.gqa_pv(pr_r[i], s0[2], out_r) for i in range(2)],
             (n_r + kv_r + qh * rl_tok * hd) * 2, qh * rl_tok * hd * 2)):
        shape = [1, qh, rl_tok, rl_tok if "pv" not in name else hd]
        rows.append(op_row(name, "f16", shape, nbytes, kernel_times_us(ctx, fns, reps), write))
    del sc_r, pr_r, out_r, q_r
    # decode: one new token of 15 heads over a 4096-row KV cache (one launch:
    # key splits whose last workgroup per KV head merges them), kernel-stamped
    # like every other line
    qd = ctx.upload(q[:, :, :1].copy())
    od = ctx.empty((1, qh, 1, hd), F16)
    dec_bytes = (2 * k.size + 2 * qh * hd) * 2
    rows.append(op_row("decode attention_f16 (1 token, 4096-row cache)", "f16", [1, qh, 1, hd],
                       dec_bytes,
                       kernel_times_us(ctx, [lambda: ctx.attention(qd, s0[1], s0[2], 0.125,
                                                                   tok - 1, None, od)], reps,
                                       batch=False)))
    # the same step through the allocation-free entry (same kernel, no pool
    # block, so a graph can record it): also the sustained figure, over
    # rotated copies of the cache (>= 1 GiB in all, so that every replay
    # reads K and V from HBM)
    n_dec = int(max(4, -(-(1 << 30) // (2 * k.size * 2))))
    dsets = [(ctx.upload(k), ctx.upload(v)) for _ in range(n_dec)]
    rows.append(op_row("decode attention_f16, allocation-free entry (1 token, 4096-row cache)",
                       "f16", [1, qh, 1, hd], dec_bytes,
                       kernel_times_us(ctx, [lambda s=s: ctx.attention_noalloc(
                           qd, s[0], s[1], 0.125, tok - 1, None, od) for s in dsets], reps)))
    del dsets
    return rows


def fused_layer_row(ctx, hid, qh, kvh, hd, ffn, tok, wn, dc, ds, sets=2, reps=20, per_graph=4):
    """One SmolLM2-360M layer's non-projection work with the attention fused:
    RMSNorm, Q/K rotation + K/V append (one launch), the fused attention core,
    SwiGLU, residual add -- 5 launches.  `us`: the layers launched back to
    back on rotated buffer sets, events around them (as the headline chain);
    `us_graph_batch`: the same recorded as graphs of `per_graph` layers (one
    kernel per op), replayed round-robin.  Bytes are the launches'
    algorithmic bytes (the attention counted by its inputs and output)."""
    qdims, qstrides = [1, qh, tok, hd], [tok * qh * hd, hd, qh * hd, 1]
    kdims, kstrides = [1, kvh, tok, hd], [tok * kvh * hd, hd, kvh * hd, 1]
    nbytes = (tok * hid * 4 + hid * 2                                    # RMSNorm
              + 2 * (qh + 2 * kvh) * tok * hd * 2 + 2 * tok * (hd // 2) * 4  # QKV rotate + append
              + (2 * qh + 2 * kvh) * tok * hd * 2                        # attention in/out
              + 3 * tok * ffn * 2 + 3 * tok * hid * 2)                   # SwiGLU, residual

    def make(i):
        key = ("fused-layer", i)
        b = {"x": ctx.upload(synth.normal(synth.seed_for(*key, "x"), (tok, hid), 0, 1, F16)),
             "q": ctx.upload(synth.normal(synth.seed_for(*key, "q"), (1, tok, qh, hd), 0, 1, F16)),
             "k": ctx.upload(synth.normal(synth.seed_for(*key, "k"), (1, tok, kvh, hd), 0, 1, F16)),
             "v": ctx.upload(synth.normal(synth.seed_for(*key, "v"), (1, tok, kvh, hd), 0, 1, F16)),
             "g": ctx.upload(synth.normal(synth.seed_for(*key, "g"), (tok, ffn), 0, 1, F16)),
             "u": ctx.upload(synth.normal(synth.seed_for(*key, "u"), (tok, ffn), 0, 1, F16)),
             "r": ctx.upload(synth.normal(synth.seed_for(*key, "r"), (tok, hid), 0, 1, F16))}
        b.update({"xn": ctx.empty((tok, hid), F16), "qr": ctx.empty(qdims, F16),
                  "kc": ctx.empty(kdims, F16), "vc": ctx.empty(kdims, F16),
                  "a": ctx.empty(qdims, F16), "h": ctx.empty((tok, ffn), F16),
                  "o": ctx.empty((tok, hid), F16)})
        return b

    def layer(b):
        ctx.rmsnorm(b["x"], wn, 1e-5, b["xn"])
        ctx.qkv_rope_kv_append((b["q"], qdims, qstrides), (b["k"], kdims, kstrides),
                               (b["v"], kdims, kstrides), dc, ds, 0, b["kc"], b["vc"], b["qr"])
        ctx.attention(b["qr"], b["kc"], b["vc"], 0.125, 0, None, b["a"])
        ctx.swiglu(b["g"], b["u"], b["h"])
        ctx.add(b["xn"], b["r"], b["o"])

    bufs = [make(i) for i in range(sets)]
    for i in range(2 * sets):  # warm-up
        layer(bufs[i % sets])
    ctx.finish()
    start, end = ctx.event(), ctx.event()
    ctx.record(start)
    for i in range(reps):
        layer(bufs[i % sets])
    ctx.record(end)
    us = ctx.elapsed_ms(start, end) * 1e3 / reps
    ctx.destroy_event(start)
    ctx.destroy_event(end)
    graphs = [capture(ctx, lambda g=g: [layer(bufs[(g + j) % sets]) for j in range(per_graph)])
              for g in range(sets)]
    us_graph = time_graphs(ctx, graphs, per_graph, max(1, reps // per_graph)) * 1e3
    ctx.finish()
    for g in graphs:
        ctx.graph_destroy(g)
    log(f"  {'layer with fused attention (5 launches)':34s} {us:9.2f} us  "
        f"graphs of {per_graph} layers {us_graph:7.2f} us/layer")
    gb, gbg = nbytes / (us * 1e-6) / 1e9, nbytes / (us_graph * 1e-6) / 1e9
    return {"op": "layer with fused attention (5 launches)", "dtype": "f16",
            "shape": [tok, hid], "bytes": nbytes, "us": round(us, 3), "us_min": None,
            "GB/s": round(gb, 1), "pct_peak": round(100 * gb / PEAK_GBS, 1),
            "us_graph_batch": round(us_graph, 3), "GB/s_graph_batch": round(gbg, 1),
            "pct_peak_graph_batch": round(100 * gbg / PEAK_GBS, 1)}


# ------------------------------------------- the headline: one layer's chain

class LayerChain:
    """The non-GEMM chain of one SmolLM2-360M decoder layer (hidden 960, 15 Q
    heads, 5 KV heads, head size 64, FFN 2560) in f16 at a 4096-token
    prefill, in the order of TransformerBlock::forward_with_cache_encode
    (nn/transformer_block.rs:128-158):

      1. RMSNorm [4096, 960] (eps 1e-5)                               x -> xn
      2. RoPE (theta 1e4, positions 0..4095) of Q [1, 15, 4096, 64] and
         K [1, 5, 4096, 64], read straight from strided views of xn (the
         rows the Q/K projections would produce), K and V appended to
         [1, 5, 4096, 64] caches, both caches repeated to 15 heads
      3. causal scale/mask (1/8) + softmax on [15, 4096, 4096]  scores -> p
      4. SwiGLU [4096, 2560]                                      g, u -> h
      5. residual add [4096, 960]                                xn, r -> o

    `prologue="one"`: stage 2 is one launch (rl_qkv_rope_kv_append_repeat_f16),
    5 launches in all.  `prologue="split"`: rope Q, rope K (into the K
    cache), repeat_kv of K and of V, 8 launches; V is then the cache itself.
    Where a GEMM sits between two stages (V, the scores, gate/up) the stage
    reads a seeded stand-in.  Bytes are the sum of the launches' algorithmic
    bytes (inputs read once, outputs written once; the masked scores are
    not read; the RoPE tables counted once per rotation)."""

    HID, QH, KVH, HD, FFN, TOK = 960, 15, 5, 64, 2560, 4096
    WORKLOAD = "SmolLM2-360M layer non-GEMM chain, f16, 4096 tokens"

    def __init__(self, ctx, prologue="one"):
        self.ctx = ctx
        self.fused = prologue == "one"
        hid, qh, kvh, hd, ffn, tok = (self.HID, self.QH, self.KVH, self.HD, self.FFN, self.TOK)
        self.qdims, self.qstrides = [1, qh, tok, hd], [tok * hid, hd, hid, 1]
        self.kdims, self.kstrides = [1, kvh, tok, hd], [tok * hid, hd, hid, 1]
        self.vdims, self.vstrides = [1, kvh, tok, hd], [kvh * tok * hd, tok * hd, hd, 1]
        self.cos, self.sin = _rope_table(hd, tok)
        self.dc, self.ds = ctx.upload(self.cos), ctx.upload(self.sin)
        self.w = synth.uniform_range(synth.seed_for("c5", "norm-w"), (hid,), 0.5, 1.5, F16)
        self.dw = ctx.upload(self.w)
        self.launches = 5 if self.fused else 8
        n_scores = qh * tok * tok
        unmasked = qh * (tok * (tok + 1) // 2)
        self.softmax_bytes = unmasked * 2 + n_scores * 2
        table = 2 * tok * (hd // 2) * 4
        stage = {
            "rmsnorm": tok * hid * 4 + hid * 2,
            "softmax": self.softmax_bytes,
            "swiglu": 3 * tok * ffn * 2,
            "residual_add": 3 * tok * hid * 2,
        }
        if self.fused:
            # Q in and out; K and V in, to the caches, repeated to 15 heads
            stage["prologue"] = (2 * qh * tok * hd * 2 + 2 * (kvh + kvh + qh) * tok * hd * 2
                                 + table)
        else:
            stage["rope_q"] = 2 * qh * tok * hd * 2 + table
            stage["rope_k"] = 2 * kvh * tok * hd * 2 + table
            stage["repeat_kv_k"] = (kvh + qh) * tok * hd * 2
            stage["repeat_kv_v"] = (kvh + qh) * tok * hd * 2
        self.stage_bytes = stage
        self.nbytes = sum(stage.values())
        # (bytes read, bytes written) of each launch of the 5-launch chain
        q, kv = qh * tok * hd * 2, kvh * tok * hd * 2
        self.stage_rw = {
            "rmsnorm": (tok * hid * 2 + hid * 2, tok * hid * 2),
            "prologue": (q + 2 * kv + table, q + 2 * kv + 2 * (qh // kvh) * kv),
            "softmax": (unmasked * 2, n_scores * 2),
            "swiglu": (2 * tok * ffn * 2, tok * ffn * 2),
            "residual_add": (2 * tok * hid * 2, tok * hid * 2),
        }
        self._scores = None

    def scores(self):
        """The stand-in for the QK^T output: N(0, 1) f16 scores, one array
        shared by every buffer set (each set holds its own device copy)."""
        if self._scores is None:
            rng = np.random.default_rng(synth.seed_for("c5", "scores") & 0xFFFFFFFF)
            s = rng.standard_normal((self.QH, self.TOK, self.TOK), dtype=np.float32)
            self._scores = s.astype(F16)
        return self._scores

    def host_inputs(self, i):
        hid, kvh, hd, ffn, tok = self.HID, self.KVH, self.HD, self.FFN, self.TOK
        key = ("c5-chain", i)
        return {"x": synth.normal(synth.seed_for(*key, "x"), (tok, hid), 0, 1, F16),
                "v": synth.normal(synth.seed_for(*key, "v"), (1, kvh, tok, hd), 0, 1, F16),
                "g": synth.normal(synth.seed_for(*key, "g"), (tok, ffn), 0, 1, F16),
                "u": synth.normal(synth.seed_for(*key, "u"), (tok, ffn), 0, 1, F16),
                "r": synth.normal(synth.seed_for(*key, "r"), (tok, hid), 0, 1, F16),
                "s": self.scores()}

    def device_set(self, host):
        ctx = self.ctx
        hid, qh, ffn, tok = self.HID, self.QH, self.FFN, self.TOK
        b = {k: ctx.upload(v) for k, v in host.items()}
        b.update({"xn": ctx.empty((tok, hid), F16), "qr": ctx.empty(self.qdims, F16),
                  "kc": ctx.empty(self.kdims, F16), "vc": ctx.empty(self.kdims, F16),
                  "kq": ctx.empty(self.qdims, F16), "vq": ctx.empty(self.qdims, F16),
                  "p": ctx.empty((qh, tok, tok), F16), "h": ctx.empty((tok, ffn), F16),
                  "o": ctx.empty((tok, hid), F16)})
        return b

    def launch(self, b, stamp=None):
        """Enqueues the chain on `b`; `stamp` = (start, stop) events that the
        softmax launch records its own start and end in."""
        ctx = self.ctx
        ctx.rmsnorm(b["x"], self.dw, 1e-5, b["xn"])
        self.launch_prologue(b)
        if stamp is not None:
            ctx.time_next_kernel(*stamp)
        ctx.attention_softmax(b["s"], 0.125, 0, b["p"])
        ctx.swiglu(b["g"], b["u"], b["h"])
        ctx.add(b["xn"], b["r"], b["o"])

    def launch_prologue(self, b):
        """Stage 2: RoPE of Q and K, the KV append, repeat_kv of both."""
        ctx, rep = self.ctx, self.QH // self.KVH
        if self.fused:
            ctx.qkv_rope_kv_append_repeat((b["xn"], self.qdims, self.qstrides),
                                          (b["xn"], self.kdims, self.kstrides),
                                          (b["v"], self.vdims, self.vstrides), self.dc, self.ds,
                                          0, b["kc"], b["vc"], rep, b["qr"], b["kq"], b["vq"])
        else:
            ctx.rope_strided(b["xn"], self.qdims, self.qstrides, self.dc, self.ds, 0, b["qr"])
            ctx.rope_strided(b["xn"], self.kdims, self.kstrides, self.dc, self.ds, 0, b["kc"])
            ctx.repeat_kv(b["kc"], rep, b["kq"])
            ctx.repeat_kv(b["v"], rep, b["vq"])


def time_chain(ctx, chain, sets, steps, warmup, stamped=False):
    """K chain steps launched back to back on the context's stream, step i
    on buffer set i mod len(sets), bracketed by stream events (after a
    synchronize).  With `stamped`, each step's softmax launch records its own
    start and end (the per-dispatch duration a kernel trace reports); a
    stamped launch goes out through hipExtLaunchKernelGGL with its events,
    which adds ~6-7 us to every step, so the step time of record comes from
    an unstamped pass.  Returns ms per step and the softmax launches'
    durations in us (empty without stamps)."""
    for i in range(warmup):
        chain.launch(sets[i % len(sets)])
    ctx.finish()
    stamps = [(ctx.event(), ctx.event()) for _ in range(steps)] if stamped else []
    start, end = ctx.event(), ctx.event()
    ctx.finish()
    ctx.record(start)
    for i in range(steps):
        chain.launch(sets[i % len(sets)], stamp=stamps[i] if stamped else None)
    ctx.record(end)
    ctx.finish()
    ms = ctx.elapsed_ms(start, end)
    sm_us = [ctx.elapsed_ms(a, b) * 1e3 for a, b in stamps]
    for e in [start, end] + [e for pair in stamps for e in pair]:
        ctx.destroy_event(e)
    return ms / steps, sm_us


def time_chain_graphs(ctx, chain, sets, steps, warmup, per_graph=4):
    """ms per step with the chain recorded as graphs of `per_graph` steps
    each (step j of a graph on set j mod len(sets); recorded streaming ops
    fused, the library's default) and the graphs replayed round-robin.  A
    graph launch costs ~9 us before its first kernel starts, so one step per
    graph would add that to every step.  The graphs stay alive until the
    process ends."""
    graphs = []
    for g in range(len(sets)):
        ctx.capture_begin()
        try:
            for j in range(per_graph):
                chain.launch(sets[(g + j) % len(sets)])
        finally:
            graphs.append(ctx.capture_end())
    _LIVE_GRAPHS.extend(graphs)
    ms = time_graphs(ctx, graphs, per_graph, max(1, steps // per_graph), warmup=warmup)
    ctx.finish()
    return ms


PROBE = os.path.join(ROOT, "rustllm_amd", "hbm_probe")


def probe_cases(pairs, timeout=120):
    """The probe's record of each (read, write) byte pair -- "us": back-to-back
    us per launch of a plain streaming kernel moving those bytes, "us_one":
    one launch between events (rustllm_amd/hbm_probe, a process of its own) --
    or None if the probe is missing or fails."""
    if not os.path.exists(PROBE):
        log(f"{PROBE} is missing (python -m rustllm_amd.build builds it)")
        return None
    try:
        res = subprocess.run([PROBE] + [f"{r}:{w}" for r, w in pairs], capture_output=True,
                             text=True, timeout=timeout)
    except subprocess.TimeoutExpired:
        log("hbm_probe timed out")
        return None
    if res.returncode != 0:
        log(f"hbm_probe failed ({res.returncode}): {res.stderr.strip()[-300:]}")
        return None
    return json.loads(res.stdout)["cases"]


def probe_streams(pairs, timeout=120):
    """Back-to-back us per launch of each (read, write) pair (probe_cases)."""
    cases = probe_cases(pairs, timeout)
    return None if cases is None else [c["us"] for c in cases]


def attach_attainable(rows, min_bytes=1 << 20, max_bytes=3 << 30):
    """Adds to each HBM-bound row (one with a read/write split) the probe's
    times for the same read and write bytes -- back to back
    ("attainable_us") and one launch between events ("attainable_one_us") --
    and the row's times as a percentage of them: sustained (graph batch)
    against back to back, one launch against one launch (a row with no
    graph-batch figure is compared one launch to one launch only).  100 = as
    fast as a plain streaming kernel moving those bytes; below 70 % of 8 TB/s
    at these sizes that figure, not the peak, says whether a kernel leaves
    time on the table."""
    todo = [r for r in rows if "write_bytes" in r and min_bytes <= r["bytes"] <= max_bytes]
    pairs = sorted({(r["read_bytes"], r["write_bytes"]) for r in todo})
    if not pairs:
        return
    cases = probe_cases(pairs)
    if cases is None:
        return
    b2b = {p: c["us"] for p, c in zip(pairs, cases)}
    single = {p: c["us_one"] for p, c in zip(pairs, cases)}
    for r in todo:
        key = (r["read_bytes"], r["write_bytes"])
        a, a1 = b2b[key], single[key]
        r["attainable_us"], r["attainable_one_us"] = round(a, 3), round(a1, 3)
        r["pct_of_attainable_one_launch"] = round(100 * a1 / r["us"], 1)
        if r["us_graph_batch"] is not None:
            r["pct_of_attainable_sustained"] = round(100 * a / r["us_graph_batch"], 1)
            what = f"sustained at {r['pct_of_attainable_sustained']:5.1f}% of it"
        else:
            what = f"one launch at {r['pct_of_attainable_one_launch']:5.1f}% of one launch"
        log(f"  {r['op']:34s} {str(r['shape']):20s} attainable {a:8.2f} us: {what}")


def oracle_chain(o, chain, host):
    """The chain on the CPU oracle (same stages, same order, f16 storage).
    V's cache is V itself (the append copies it)."""
    hid, qh, kvh, hd, tok = chain.HID, chain.QH, chain.KVH, chain.HD, chain.TOK
    rep = qh // kvh
    out = {"xn": o.rmsnorm(host["x"], chain.w, 1e-5)}
    out.update(oracle_after_norm(o, chain, host, out["xn"]))
    out["p"] = o.attention_softmax(host["s"], 0.125, 0)
    out["h"] = o.swiglu(host["g"], host["u"])
    return out


def oracle_after_norm(o, chain, host, xn):
    """The chain's stages that read xn (RoPE of its Q/K views, repeat_kv,
    the residual add), on the oracle."""
    qh, kvh, rep = chain.QH, chain.KVH, chain.QH // chain.KVH
    flat = xn.ravel()
    q = o.contiguous(flat, chain.qdims, chain.qstrides).reshape(chain.qdims)
    k = o.contiguous(flat, chain.kdims, chain.kstrides).reshape(chain.kdims)
    kc = o.rope(k, chain.cos, chain.sin, 0)
    return {"qr": o.rope(q, chain.cos, chain.sin, 0), "kc": kc,
            "kq": o.repeat_kv(kc, rep), "vq": o.repeat_kv(host["v"], rep),
            "o": o.add(xn, host["r"])}


def _ulp16(got, ref) -> int:
    gi = got.view(np.int16).astype(np.int32)
    ri = ref.view(np.int16).astype(np.int32)
    gi = np.where(gi < 0, -(gi & 0x7FFF), gi)
    ri = np.where(ri < 0, -(ri & 0x7FFF), ri)
    return int(np.max(np.abs(gi - ri)))


def check_chain(o, chain, b, host, ref) -> list[str]:
    """The GPU chain's outputs on buffer set `b` against the oracle's `ref`
    on the same inputs: f16 RMSNorm, softmax and SwiGLU within 2 ulp; the
    stages that read xn (RoPE, repeat_kv, residual add, the V cache)
    bit-exact against the oracle applied to the GPU's own xn.  Returns the
    stages that differ."""
    bad = []
    xn = b["xn"].numpy()
    if _ulp16(xn, ref["xn"]) > 2:
        bad.append("rmsnorm")
    if _ulp16(b["p"].numpy(), ref["p"]) > 2:
        bad.append("attention_softmax")
    if _ulp16(b["h"].numpy(), ref["h"]) > 2:
        bad.append("swiglu")
    exact = (oracle_after_norm(o, chain, host, xn) if not np.array_equal(xn, ref["xn"])
             else ref)
    for name in ("qr", "kc", "kq", "vq", "o"):
        if not np.array_equal(b[name].numpy().view(np.uint16), exact[name].view(np.uint16)):
            bad.append(name)
    if chain.fused and not np.array_equal(b["vc"].numpy().view(np.uint16),
                                          host["v"].view(np.uint16)):
        bad.append("v_cache")
    return bad


def _rope_table(head_dim, max_seq, theta=10000.0):
    """RotaryEmbedding::new's table (nn/rope.rs:44-62) in float32."""
    half = head_dim // 2
    pos = np.arange(max_seq, dtype=np.float32)[:, None]
    expo = (2 * np.arange(half, dtype=np.float32)) / np.float32(head_dim)
    inv = np.float32(1.0) / np.power(np.float32(theta), expo, dtype=np.float32)
    ang = (pos * inv[None, :]).astype(np.float32)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


# --------------------------------------------------------------- CPU leg

def cpu_threads() -> int:
    """Cores this process may use: its affinity set, capped by OMP_NUM_THREADS."""
    n = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS", "")
    return max(1, min(n, int(cap))) if cap.isdigit() and int(cap) > 0 else n


def _oracle():
    sys.path.insert(0, ROOT)
    from oracle import oracle as o
    return o


def cpu_chain(chain, host, budget_s: float, threads: int = 1):
    """The oracle (scalar C restatement of the reference ops; `threads` > 1
    splits each op's rows/elements over OpenMP threads) on whole passes of
    the layer chain over one buffer set's inputs, at least one pass and
    until `budget_s` seconds have run.  Returns passes, seconds, outputs."""
    o = _oracle()
    o.set_threads(threads)
    passes = 0
    t0 = time.perf_counter()
    while True:
        outs = oracle_chain(o, chain, host)
        passes += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    return passes, time.perf_counter() - t0, outs


def oracle_batch_step(host, threads):
    """One step of the [4096, 1536] batch on the oracle (its outputs)."""
    o = _oracle()
    o.set_threads(threads)
    a32, b32, a16, b16 = host["a_float32"], host["b_float32"], host["a_float16"], host["b_float16"]
    outs = {}
    for t, a, b in (("float32", a32, b32), ("float16", a16, b16)):
        outs[f"add_{t}"] = o.add(a, b)
        outs[f"mul_{t}"] = o.mul(a, b)
        outs[f"silu_{t}"] = o.silu(a)
        outs[f"swiglu_{t}"] = o.swiglu(a, b)
        outs[f"bias_{t}"] = o.add_broadcast(a, host[f"bias_{t}"])
        outs[f"view_{t}"] = o.contiguous(host[f"view_{t}"].ravel(), VIEW_DIMS, VIEW_STRIDES)
        outs[f"kv_{t}"] = o.repeat_kv(host[f"kv_{t}"], 3)
    outs["cast_h"] = o.cast(a32, F16)
    outs["cast_f"] = o.cast(a16, F32)
    return outs


def check_outputs(ctx, dev, outs) -> list[str]:
    """Compares the first buffer set's outputs with the oracle's; returns failures."""
    bad = []

    def same(name, got, ref, exact=True):
        if exact:
            ok = np.array_equal(got.view(np.uint8), ref.view(np.uint8))
        elif got.dtype == np.float16:
            gi = got.view(np.int16).astype(np.int32)
            ri = ref.view(np.int16).astype(np.int32)
            gi = np.where(gi < 0, -(gi & 0x7FFF), gi)
            ri = np.where(ri < 0, -(ri & 0x7FFF), ri)
            ok = int(np.max(np.abs(gi - ri))) <= 2
        else:
            ok = float(np.max(np.abs(got - ref) / np.maximum(np.abs(ref), 1.18e-38))) <= 1e-5
        if not ok:
            bad.append(name)

    for t in ("float32", "float16"):
        same(f"add_{t}", dev[f"o1_{t}"].numpy(), outs[f"add_{t}"])
        same(f"mul_{t}", dev[f"o2_{t}"].numpy(), outs[f"mul_{t}"])
        same(f"silu_{t}", dev[f"o3_{t}"].numpy(), outs[f"silu_{t}"], exact=False)
        same(f"swiglu_{t}", dev[f"o4_{t}"].numpy(), outs[f"swiglu_{t}"], exact=False)
        same(f"bias_{t}", dev[f"o5_{t}"].numpy(), outs[f"bias_{t}"])
        same(f"contiguous_{t}", dev[f"vo_{t}"].numpy(), outs[f"view_{t}"])
        same(f"repeat_kv_{t}", dev[f"kvo_{t}"].numpy(), outs[f"kv_{t}"])
    same("cast_f32_to_f16", dev["cast_h"].numpy(), outs["cast_h"])
    same("cast_f16_to_f32", dev["cast_f"].numpy(), outs["cast_f"])
    return bad


def probe(ctx, host, ops):
    """Hardware-counter probe: each op 3 times, then a plain copy of known
    size whose FETCH_SIZE / WRITE_SIZE readings calibrate the counters."""
    s = batch_set(ctx, host)
    for op in ops:
        for _ in range(3):
            ctx.begin()
            op.launch(ctx, s)
            ctx.finish()
        log(f"probe {op.name}: {op.nbytes} algorithmic bytes per launch")
    # the whole batch recorded as a graph: its ops in one fused launch
    ctx.capture_begin()
    try:
        for op in ops:
            op.launch(ctx, s)
    finally:
        step_graph = ctx.capture_end()
    for _ in range(3):
        ctx.graph_launch(step_graph)
        ctx.finish()
    ctx.graph_destroy(step_graph)
    log(f"probe fused step (the {len(ops)} ops in one launch): "
        f"{sum(op.nbytes for op in ops)} algorithmic bytes per launch")
    # The row ops at their benchmark shapes.
    hid, tok = 960, 4096
    x = ctx.upload(synth.normal(1, (tok, hid), 0, 2.0, F16))
    w = ctx.upload(synth.uniform_range(2, (hid,), 0.5, 1.5, F16))
    y = ctx.empty((tok, hid), F16)
    c, s_ = _rope_table(64, tok)
    dc, ds = ctx.upload(c), ctx.upload(s_)
    q = ctx.upload(synth.normal(3, (1, 15, tok, 64), 0, 1, F16))
    qo = ctx.empty((1, 15, tok, 64), F16)
    sc = ctx.upload(synth.normal(4, (9, 2048, 2048), 0, 4.0, F32))
    so = ctx.empty((9, 2048, 2048), F32)
    xl = ctx.upload(synth.normal(5, (16384, hid), 0, 2.0, F16))
    yl = ctx.empty((16384, hid), F16)
    kproj = ctx.upload(synth.normal(6, (1, tok, 5, 64), 0, 1, F16))
    kcache = ctx.empty((1, 5, tok, 64), F16)
    kdims, kstrides = [1, 5, tok, 64], [tok * 5 * 64, 64, 5 * 64, 1]
    vocab = 49152
    emb = ctx.upload(synth.normal(7, (vocab, hid), 0, 1, F16))
    ids = (synth.uniform(8, tok) * vocab).astype(np.uint32)
    # attention core at the SmolLM2 layer shape (Q [1,15,4096,64], K/V [1,5,4096,64])
    ka = ctx.upload(synth.normal(9, (1, 5, tok, 64), 0, 1, F16))
    va = ctx.upload(synth.normal(10, (1, 5, tok, 64), 0, 1, F16))
    scores = ctx.empty((1, 15, tok, tok), F16)
    attn_io = (2 * 15 + 2 * 5) * tok * 64 * 2
    n_scores = 15 * tok * tok
    # ragged scores (4093 keys: rows off the 16-byte grid)
    q_r = ctx.upload(synth.normal(11, (1, 15, 4093, 64), 0, 1, F16))
    k_r = ctx.upload(synth.normal(12, (1, 5, 4093, 64), 0, 1, F16))
    scores_r = ctx.empty((1, 15, 4093, 4093), F16)
    # the one-launch prologue: Q, K, V views of [1, S, H, D] projections
    qp = ctx.upload(synth.normal(13, (1, tok, 15, 64), 0, 1, F16))
    qd, qs = [1, 15, tok, 64], [tok * 15 * 64, 64, 15 * 64, 1]
    vcache = ctx.empty((1, 5, tok, 64), F16)
    krep, vrep = ctx.empty((1, 15, tok, 64), F16), ctx.empty((1, 15, tok, 64), F16)
    # one decode step over a 4096-row cache
    q1, o1 = ctx.upload(synth.normal(14, (1, 15, 1, 64), 0, 1, F16)), ctx.empty((1, 15, 1, 64), F16)
    # f32 operands of the same attention core
    q32 = ctx.upload(synth.normal(15, (1, 15, tok, 64), 0, 1, F32))
    k32 = ctx.upload(synth.normal(16, (1, 5, tok, 64), 0, 1, F32))
    v32 = ctx.upload(synth.normal(17, (1, 5, tok, 64), 0, 1, F32))
    o32 = ctx.empty((1, 15, tok, 64), F32)
    scores32 = ctx.empty((1, 15, tok, tok), F32)
    # the layer chain's other kernels at its shapes (LayerChain): the f16
    # scores' causal scale/mask + softmax, SwiGLU [4096, 2560], residual add
    chain = LayerChain(ctx)
    cb = chain.device_set(chain.host_inputs(0))
    for name, nbytes, fn in [
        ("attention_softmax_f16 [15,4096,4096] causal", chain.softmax_bytes,
         lambda: ctx.attention_softmax(cb["s"], 0.125, 0, cb["p"])),
        ("swiglu_f16 [4096,2560]", chain.stage_bytes["swiglu"],
         lambda: ctx.swiglu(cb["g"], cb["u"], cb["h"])),
        ("add_f16 [4096,960]", chain.stage_bytes["residual_add"],
         lambda: ctx.add(cb["x"], cb["r"], cb["o"])),
        ("chain prologue: qkv rope + KV append + repeat_kv f16", chain.stage_bytes["prologue"],
         lambda: chain.launch_prologue(cb)),
    ]:
        for _ in range(3):
            ctx.begin()
            fn()
            ctx.finish()
        log(f"probe {name}: {nbytes} algorithmic bytes per launch")
    for name, nbytes, fn in [
        ("attention_f16 fused [1,15,4096,64] causal (inputs + output)", attn_io,
         lambda: ctx.attention(q, ka, va, 0.125, 0, None, qo)),
        ("gqa_qk_f16 [1,15,4096,4096]", (15 + 5) * tok * 64 * 2 + n_scores * 2,
         lambda: ctx.gqa_qk(q, ka, None, scores)),
        ("gqa_pv_f16 [1,15,4096,64]", n_scores * 2 + (5 + 15) * tok * 64 * 2,
         lambda: ctx.gqa_pv(scores, va, qo)),
        ("rmsnorm_f16 [4096,960]", tok * hid * 4 + hid * 2, lambda: ctx.rmsnorm(x, w, 1e-5, y)),
        ("rmsnorm_f16 [16384,960]", 16384 * hid * 4 + hid * 2,
         lambda: ctx.rmsnorm(xl, w, 1e-5, yl)),
        ("rope_K_f16 -> KV cache [1,5,4096,64]", 2 * 5 * tok * 64 * 2 + 2 * tok * 32 * 4,
         lambda: ctx.rope_kv_cache_write(kproj, kdims, kstrides, dc, ds, 0, kcache)),
        ("embedding_f16 [4096 of 49152,960]", 2 * tok * hid * 2 + tok * 4,
         lambda: ctx.embedding(emb, ids, y)),
        ("rope_f16 [1,15,4096,64]", 2 * 15 * tok * 64 * 2 + 2 * tok * 32 * 4,
         lambda: ctx.rope(q, dc, ds, 0, qo)),
        ("attention_softmax_f32 [9,2048,2048]", 9 * (2048 * 2049 // 2) * 4 + 9 * 2048 * 2048 * 4,
         lambda: ctx.attention_softmax(sc, 0.125, 0, so)),
        ("gqa_qk_f16 ragged [1,15,4093,4093]", (15 + 5) * 4093 * 64 * 2 + 15 * 4093 * 4093 * 2,
         lambda: ctx.gqa_qk(q_r, k_r, None, scores_r)),
        ("qkv + KV append + repeat_kv f16 [1,25,4096,64]",
         2 * 15 * tok * 64 * 2 + 2 * 5 * tok * 64 * (1 + 1 + 3) * 2 + 2 * tok * 32 * 4,
         lambda: ctx.qkv_rope_kv_append_repeat((qp, qd, qs), (kproj, kdims, kstrides),
                                               (kproj, kdims, kstrides), dc, ds, 0, kcache,
                                               vcache, 3, qo, krep, vrep)),
        ("decode attention_f16 [1,15,1,64] over 4096 rows", 2 * 15 * 64 * 2 + 2 * 5 * tok * 64 * 2,
         lambda: ctx.attention_noalloc(q1, ka, va, 0.125, tok - 1, None, o1)),
        # the f32 matrix-core kernels at the same shape (Q/K/V as f32, f32 scores)
        ("gqa_qk_f32 [1,15,4096,4096]", (15 + 5) * tok * 64 * 4 + n_scores * 4,
         lambda: ctx.gqa_qk(q32, k32, None, scores32)),
        ("gqa_pv_f32 [1,15,4096,64]", n_scores * 4 + (5 + 15) * tok * 64 * 4,
         lambda: ctx.gqa_pv(scores32, v32, o32)),
        ("attention_f32 fused [1,15,4096,64] causal (inputs + output)", attn_io * 2,
         lambda: ctx.attention(q32, k32, v32, 0.125, 0, None, o32)),
    ]:
        for _ in range(3):
            ctx.begin()
            fn()
            ctx.finish()
        log(f"probe {name}: {nbytes} algorithmic bytes per launch")
    # A contiguous "view" of a contiguous buffer is a plain copy kernel.
    nbytes = 256 << 20
    n = nbytes // 4
    src = ctx.upload(np.ones(n, dtype=F32))
    dst = ctx.empty((n,), F32)
    for _ in range(3):
        ctx.begin()
        ctx.contiguous(src, [n], [1], dst)
        ctx.finish()
    log(f"probe copy (contiguous_f32 of a flat view): {nbytes} bytes read and {nbytes} bytes "
        f"written per launch")


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_batch.json")


def measured_traffic(op_name):
    """HBM bytes per launch of `op_name` as the hardware counters read it:
    FETCH_SIZE and WRITE_SIZE per dispatch from two `rocprofv3 --pmc` runs of
    `bench.py --probe`, each scaled by its reading on a copy of known size.
    The summary is committed text; None if it has no entry for the op."""
    try:
        with open(TRAFFIC_FILE) as f:
            data = json.load(f)
    except (OSError, ValueError):
        return None
    entry = data.get("ops", {}).get(op_name)
    return None if entry is None else entry["hbm_bytes"]


# ------------------------------------------------------------------ main

# The per-op rows the JSON line carries (the full table goes to stderr and
# to the --per-op-out file): the metric's four ops at the layer's shapes,
# the largest RMSNorm rows, the [9, 2048, 2048] softmax and the SwiGLU rows.
SUMMARY_ROWS = [
    ("layer.1 rmsnorm_f16", [4096, 960]),
    ("layer.2 rope_Q_f16 (fused gather)", [1, 15, 4096, 64]),
    ("layer.2 rope_K_f16 (fused gather)", [1, 5, 4096, 64]),
    ("layer.2 QKV + KV append + repeat_kv (one launch)", [1, 25, 4096, 64]),
    ("layer.4 attention_softmax_f16", [15, 4096, 4096]),
    ("layer.5 swiglu_f16", [4096, 2560]),
    ("layer.6 residual add_f16", [4096, 960]),
    ("rmsnorm_f16", [16384, 960]),
    ("rmsnorm_f32", [16384, 960]),
    ("attention_softmax_f32", [9, 2048, 2048]),
    ("softmax_f32", [9, 2048, 2048]),
    ("swiglu_f16", [4096, 1536]),
    ("swiglu_f32", [4096, 1536]),
    ("add_rmsnorm_f32", [64, 768]),
]


def summary(rows):
    """{"op shape": [us, GB/s, % of peak, sustained % of peak, sustained % of
    the probe's time for the same bytes]} for SUMMARY_ROWS."""
    out = {}
    for op, shape in SUMMARY_ROWS:
        for r in rows:
            if r["op"] == op and r["shape"] == shape:
                out[f"{op} {shape}"] = [r["us"], r["GB/s"], r["pct_peak"],
                                        r.get("pct_peak_graph_batch"),
                                        r.get("pct_of_attainable_sustained")]
                break
    return out


def write_side_file(path, payload):
    try:
        os.makedirs(os.path.dirname(path), exist_ok=True)
        with open(path, "w") as f:
            json.dump(payload, f, indent=1)
        return os.path.relpath(path, ROOT)
    except OSError as e:
        log(f"could not write {path}: {e}")
        return None


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--sets", type=int, default=2,
                    help="buffer sets of the layer chain rotated across steps (1.1 GB each)")
    ap.add_argument("--op-reps", type=int, default=100, help="timed launches per op line")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="CPU leg: at least one chain pass on one core, then passes on all "
                         "cores for half this long")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the per-op lines")
    ap.add_argument("--quick", action="store_true", help="fewer per-op shapes")
    ap.add_argument("--no-graph-batch", action="store_true",
                    help="leave out the graph-replayed figures (sustained per-op times, the "
                         "chain and the batch step as graphs)")
    ap.add_argument("--per-op-out", default=os.path.join(ROOT, "bench_out", "bench_per_op.json"),
                    help="file the full per-op table is written to")
    ap.add_argument("--per-op-only", action="store_true",
                    help="only the per-op table, written to --per-op-out (the child process "
                         "of a default run)")
    ap.add_argument("--probe", action="store_true",
                    help="no timing: run each op 3 times on one buffer set, then a "
                         "256 MiB device-to-device copy 3 times (for hardware-counter runs)")
    args = ap.parse_args()
    global GRAPH_BATCH
    GRAPH_BATCH = not args.no_graph_batch

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: every op runs on one MI355X and shards across GPUs "
              "without any exchange, so no multi-GPU figure is produced (use --gpus 1).",
              file=sys.stderr)
        sys.exit(2)

    ctx = abi.Context(0)
    if args.probe:
        probe(ctx, batch_inputs("bench"), batch_ops())
        return
    if args.per_op_only:
        host = batch_inputs("bench")
        sets = [batch_set(ctx, host) for _ in range(4)]
        log("per op ([4096, 1536] batch):")
        rows = per_op_rows(ctx, batch_ops(), sets, args.op_reps)
        del sets
        rows += extra_rows(ctx, args.op_reps, args.quick)
        log("per op against the HBM probe at the same read and write bytes:")
        attach_attainable(rows)
        write_side_file(args.per_op_out, {"per_op": rows})
        ctx.close()
        return

    # ---- the headline: the layer chain, 5 launches, over rotated buffer sets
    chain = LayerChain(ctx, "one")
    log(f"layer chain: {args.sets} buffer sets")
    host0 = chain.host_inputs(0)
    csets = [chain.device_set(host0)] + [chain.device_set(chain.host_inputs(i))
                                         for i in range(1, args.sets)]
    footprint = sum(set_bytes(s) for s in csets)
    ms_step, _ = time_chain(ctx, chain, csets, args.steps, args.warmup)
    value = chain.nbytes / (ms_step * 1e-3) / 1e9
    log(f"layer chain ({chain.launches} launches): {ms_step * 1e3:.2f} us per step, "
        f"{value:.1f} GB/s ({100 * value / PEAK_GBS:.1f}% of peak), footprint "
        f"{footprint / 2**30:.2f} GiB")
    # the roofline kernel's own durations: the same K steps again, each
    # softmax launch stamping its start and end
    ms_stamped, sm_us = time_chain(ctx, chain, csets, args.steps, args.warmup, stamped=True)
    sm_mean = float(np.mean(sm_us))
    sm_gbs = chain.softmax_bytes / (sm_mean * 1e-6) / 1e9
    log(f"  its softmax launches (a second pass, every softmax launch stamped: "
        f"{ms_stamped * 1e3:.2f} us per step): {sm_mean:.2f} us mean ({len(sm_us)} launches), "
        f"{sm_gbs:.1f} GB/s ({100 * sm_gbs / PEAK_GBS:.1f}%)")
    ms_graph = (time_chain_graphs(ctx, chain, csets, max(args.steps, 20), args.warmup)
                if GRAPH_BATCH else None)
    if ms_graph is not None:
        log(f"  the same chain recorded as graphs: {ms_graph * 1e3:.2f} us per step")
    split = LayerChain(ctx, "split")
    ms_split, _ = time_chain(ctx, split, csets, args.steps, args.warmup)
    log(f"layer chain, prologue as 4 launches ({split.launches} launches): "
        f"{ms_split * 1e3:.2f} us per step, {split.nbytes / (ms_split * 1e-3) / 1e9:.1f} GB/s")
    chain.launch(csets[0])  # set 0 holds the 5-launch chain's outputs again
    ctx.finish()

    # What HBM allows for the same bytes: a plain streaming kernel per stage
    probe_us = probe_streams(list(chain.stage_rw.values()))
    attain = None
    if probe_us is not None:
        attain = dict(zip(chain.stage_rw, probe_us))
        log("  a plain streaming kernel moving each stage's bytes (back to back): " +
            ", ".join(f"{k} {v:.2f} us" for k, v in attain.items()) +
            f"; {sum(probe_us):.2f} us in all")

    threads = cpu_threads()
    o = _oracle()
    cpu = None
    if not args.no_cpu:
        log(f"cpu baseline: oracle, 1 thread, >= 1 chain pass (~{args.cpu_seconds:.0f} s)")
        passes, elapsed, ref = cpu_chain(chain, host0, args.cpu_seconds, 1)
        cpu_gbs = chain.nbytes * passes / elapsed / 1e9
        cpu = {"value": round(cpu_gbs, 3), "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": f"{passes} whole pass(es) of the layer chain on buffer set 0's inputs "
                         f"in {elapsed:.1f} s ({1e3 * elapsed / passes:.0f} ms a pass)"}
        log(f"cpu (1 thread): {cpu_gbs:.3f} GB/s, {passes} pass(es) in {elapsed:.1f} s")
        if threads > 1:
            passes_n, elapsed_n, _ = cpu_chain(chain, host0, args.cpu_seconds / 2, threads)
            gbs_n = chain.nbytes * passes_n / elapsed_n / 1e9
            cpu["all_cores"] = {"value": round(gbs_n, 3), "cores": threads,
                                "sample": f"{passes_n} passes in {elapsed_n:.1f} s"}
            log(f"cpu ({threads} threads): {gbs_n:.3f} GB/s, {passes_n} passes in "
                f"{elapsed_n:.1f} s")
        else:
            cpu["all_cores"] = None
            cpu["note"] = "this process may use one core (affinity / OMP_NUM_THREADS)"
    else:
        o.set_threads(threads)
        ref = oracle_chain(o, chain, host0)
    bad = check_chain(o, chain, csets[0], host0, ref)
    log("layer chain: every stage matches the oracle" if not bad
        else f"layer chain: MISMATCH against the oracle in {bad}")
    if cpu is not None:
        cpu["gpu_outputs_match_oracle"] = not bad
    del csets, ref
    chain._scores = None

    # ---- the [4096, 1536] batch step (secondary): 16 ops over rotated sets
    host = batch_inputs("bench")
    ops = batch_ops()
    sets = [batch_set(ctx, host) for _ in range(4)]
    distinct = set_bytes(sets[0])  # every input and output of a step, each once
    c2_steps = 4 * max(1, -(-max(args.steps, 20) // 4))
    ms_c2 = time_step(ctx, ops, sets, c2_steps, args.warmup) if GRAPH_BATCH else None
    ctx.set_fusion(False)
    ms_c2_unfused = time_step(ctx, ops, sets, c2_steps, args.warmup) if GRAPH_BATCH else None
    ctx.set_fusion(True)
    c2_bad = check_outputs(ctx, sets[0], oracle_batch_step(host, threads))
    c2 = {"workload": "elementwise+broadcast batch [4096,1536], f32 and f16 (16 ops)",
          "distinct_bytes_per_step": distinct, "outputs_match_oracle": not c2_bad}
    if ms_c2 is not None:
        c2.update({"us_per_step_fused_launch": round(ms_c2 * 1e3, 2),
                   "GB/s_fused_launch": round(distinct / (ms_c2 * 1e-3) / 1e9, 1),
                   "us_per_step_kernel_per_op": round(ms_c2_unfused * 1e3, 2),
                   "GB/s_kernel_per_op": round(distinct / (ms_c2_unfused * 1e-3) / 1e9, 1)})
        log(f"batch step [4096,1536]: {ms_c2 * 1e3:.1f} us fused, {ms_c2_unfused * 1e3:.1f} us "
            f"one kernel per op ({distinct / 1e6:.1f} MB distinct bytes)")
    if c2_bad:
        log(f"batch step: MISMATCH against the oracle: {c2_bad}")

    del sets
    rows, per_op_status = [], "not run (--no-extra)"
    if not args.no_extra:
        # The per-op table runs in a child process (the same script with
        # --per-op-only), after this process has returned its buffers: a
        # failure there costs the table, not the headline.
        ctx.lib.rl_context_trim(ctx.handle)
        cmd = [sys.executable, os.path.abspath(__file__), "--per-op-only", "--op-reps",
               str(args.op_reps), "--per-op-out", args.per_op_out]
        cmd += ["--quick"] if args.quick else []
        cmd += ["--no-graph-batch"] if args.no_graph_batch else []
        try:
            os.remove(args.per_op_out)
        except OSError:
            pass
        rc = subprocess.run(cmd).returncode
        try:
            with open(args.per_op_out) as f:
                rows = json.load(f)["per_op"]
        except (OSError, ValueError, KeyError):
            rows = []
        per_op_status = "ok" if rc == 0 else f"per-op process exited with status {rc}"
        if rc != 0:
            log(f"per-op table: {per_op_status}")
    side = os.path.relpath(args.per_op_out, ROOT) if rows else None

    sm_traffic = measured_traffic("attention_softmax_f16 [15,4096,4096] causal")
    roofline = {"bound": "hbm", "kernel": "k_softmax_rows_h2<4, 128, true, false, false>",
                "op": "causal scale/mask + softmax f16 [15,4096,4096]",
                "achieved": round(sm_gbs, 1), "peak": PEAK_GBS, "unit": "GB/s",
                "frac": round(sm_gbs / PEAK_GBS, 4), "traffic": sm_traffic,
                "bytes_per_launch": chain.softmax_bytes, "us_per_launch": round(sm_mean, 3),
                "launches_timed": len(sm_us), "step_ms_stamped": round(ms_stamped, 5),
                "share_of_step": round(sm_mean / (ms_stamped * 1e3), 3)}
    if attain is not None:
        # the same bytes moved by a plain streaming kernel, back to back
        roofline["attainable_us"] = round(attain["softmax"], 3)
        roofline["attainable_GBps"] = round(chain.softmax_bytes / (attain["softmax"] * 1e-6) / 1e9,
                                            1)
        roofline["frac_of_attainable"] = round(attain["softmax"] / sm_mean, 4)
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": LayerChain.WORKLOAD,
                   "stages": "rmsnorm [4096,960] -> rope Q/K + KV append + repeat_kv 5->15 "
                             "(one launch) -> causal scale/mask+softmax [15,4096,4096] -> "
                             "swiglu [4096,2560] -> residual add [4096,960]",
                   "launches_per_step": chain.launches, "bytes_per_step": chain.nbytes,
                   "buffer_sets": args.sets, "footprint_gib": round(footprint / 2**30, 2),
                   "timing": "eager launches on one stream, events around the K steps "
                             "(the roofline's per-launch stamps in a second pass)",
                   "graph_replay_ms_per_step": None if ms_graph is None else round(ms_graph, 5),
                   "eight_launch_ms_per_step": round(ms_split, 5),
                   "attainable_ms_per_step": (None if attain is None
                                              else round(sum(attain.values()) * 1e-3, 5)),
                   "attainable_by_stage_us": (None if attain is None else
                                              {k: round(v, 2) for k, v in attain.items()}),
                   "outputs_match_oracle": not bad},
        "pct_of_peak": round(100 * value / PEAK_GBS, 1),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "per_op_summary": {"columns": ["us", "GB/s", "pct_peak", "pct_peak_sustained",
                                       "pct_of_attainable_sustained"],
                           **summary(rows)},
        "per_op_file": side,
        "per_op_status": per_op_status,
        "batch_step": c2,
    }
    ctx.close()
    text = json.dumps(line, separators=(",", ":"))
    if len(text) > 7500:  # keep the line short enough for the driver to parse
        line.pop("per_op_summary")
        text = json.dumps(line, separators=(",", ":"))
    print(text, flush=True)


if __name__ == "__main__":
    main()
