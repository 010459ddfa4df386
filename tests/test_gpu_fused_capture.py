"""Streaming ops recorded into a graph: runs of independent maps and bias adds
share one fused launch, dependent ones are split into successive launches.
Every replay must equal the same calls run eagerly, bit for bit (the fused
kernel runs each op's own body), with eager work between the replays."""

import numpy as np
import pytest

from helpers import assert_bitexact
from oracle import oracle as o
from rustllm_amd import synth

pytestmark = pytest.mark.gpu

F16, F32 = np.float16, np.float32
T, H = 512, 1536


def norm(tag, shape, dtype):
    return synth.normal(synth.seed_for("fused", tag, *shape, np.dtype(dtype).name), shape, 0, 1,
                        dtype)


def replay_and_compare(ctx, record, outs, reps=3):
    """Runs `record` eagerly, snapshots `outs`, clears them, records the same
    calls as a graph and replays it `reps` times (eager work and a wait in
    between), comparing every output with the eager run each time."""
    ctx.begin()
    record()
    ctx.finish()
    eager = [b.numpy() for b in outs]
    zeros = [np.zeros(e.shape, e.dtype) for e in eager]
    ctx.capture_begin()
    record()
    graph = ctx.capture_end()
    scratch = ctx.upload(np.ones((T, H), F32))
    for i in range(reps):
        for b, z in zip(outs, zeros):  # a replay must write every output again
            ctx.copy(ctx.upload(z), b)
        ctx.graph_launch(graph)
        ctx.finish()
        for j, (b, e) in enumerate(zip(outs, eager)):
            assert_bitexact(b.numpy(), e, f"replay {i}, output {j}")
        ctx.begin()
        ctx.mul(scratch, scratch)  # unrelated eager work between replays
        ctx.finish()
    ctx.graph_destroy(graph)
    return eager


VIEW_DIMS = [1, 9, 512, 64]                 # [1, 512, 9, 64] seen as [1, 9, 512, 64]
VIEW_STRIDES = [512 * 9 * 64, 64, 9 * 64, 1]


def test_independent_batch_matches_eager_and_oracle(ctx):
    """The C2-style batch: add, mul, SiLU, SwiGLU, bias add in f32 and f16,
    both casts, the transposed view's contiguous copy and repeat_kv 3 -> 9 in
    both dtypes, all independent -- one fused launch."""
    host, dev, outs, ops = {}, {}, [], []
    for dt in (F32, F16):
        a, b, bias = norm("a", (T, H), dt), norm("b", (T, H), dt), norm("bias", (H,), dt)
        host[dt] = (a, b, bias)
        da, db, dbias = ctx.upload(a), ctx.upload(b), ctx.upload(bias)
        dev[dt] = (da, db, dbias)
        o5 = [ctx.empty((T, H), dt) for _ in range(5)]
        outs += o5
        ops += [lambda da=da, db=db, x=o5[0]: ctx.add(da, db, x),
                lambda da=da, db=db, x=o5[1]: ctx.mul(da, db, x),
                lambda da=da, x=o5[2]: ctx.silu(da, x),
                lambda da=da, db=db, x=o5[3]: ctx.swiglu(da, db, x),
                lambda da=da, dbias=dbias, x=o5[4]: ctx.add_broadcast(da, dbias, x)]
    ch, cf = ctx.empty((T, H), F16), ctx.empty((T, H), F32)
    outs += [ch, cf]
    ops += [lambda: ctx.cast(dev[F32][0], F16, ch), lambda: ctx.cast(dev[F16][0], F32, cf)]
    moves = {}
    for dt in (F32, F16):
        view = norm("view", (1, 512, 9, 64), dt)
        kv = norm("kv", (1, 3, 512, 64), dt)
        dview, dkv = ctx.upload(view), ctx.upload(kv)
        vo, kvo = ctx.empty(VIEW_DIMS, dt), ctx.empty((1, 9, 512, 64), dt)
        moves[dt] = (view, kv)
        outs += [vo, kvo]
        ops += [lambda dview=dview, vo=vo: ctx.contiguous(dview, VIEW_DIMS, VIEW_STRIDES, vo),
                lambda dkv=dkv, kvo=kvo: ctx.repeat_kv(dkv, 3, kvo)]

    def record():
        for op in ops:
            op()

    eager = replay_and_compare(ctx, record, outs)
    k = 0
    for dt in (F32, F16):
        a, b, bias = host[dt]
        assert_bitexact(eager[k], o.add(a, b), "add")
        assert_bitexact(eager[k + 1], o.mul(a, b), "mul")
        assert_bitexact(eager[k + 4], o.add_broadcast(a, bias), "bias add")
        k += 5
    assert_bitexact(eager[k], o.cast(host[F32][0], F16), "cast f32 -> f16")
    assert_bitexact(eager[k + 1], o.cast(host[F16][0], F32), "cast f16 -> f32")
    k += 2
    for dt in (F32, F16):
        view, kv = moves[dt]
        assert_bitexact(eager[k], o.contiguous(view.ravel(), VIEW_DIMS, VIEW_STRIDES), "contiguous")
        assert_bitexact(eager[k + 1], o.repeat_kv(kv, 3), "repeat_kv")
        k += 2


def test_gathers_feeding_maps(ctx):
    """repeat_kv and a contiguous copy whose outputs later ops read (and an
    op writing a gather's source after the gather read it)."""
    kv = norm("fkv", (1, 3, 512, 64), F16)
    view = norm("fview", (1, 512, 9, 64), F16)
    dkv, dview = ctx.upload(kv), ctx.upload(view)
    src = ctx.empty((1, 512, 9, 64), F16)
    rep_out, cont, s1, s2 = (ctx.empty((1, 9, 512, 64), F16) for _ in range(4))

    def record():
        ctx.add(dview, dview, src)                              # src = 2 view
        ctx.repeat_kv(dkv, 3, rep_out)
        ctx.contiguous(src, VIEW_DIMS, VIEW_STRIDES, cont)      # reads src (after write)
        ctx.add(rep_out, cont, s1)                              # reads both gathers' outputs
        ctx.mul(dview, dview, src)                              # rewrites src after it was read
        ctx.add(cont, rep_out, s2)

    eager = replay_and_compare(ctx, record, [rep_out, cont, s1, s2, src])
    two = o.add(view, view)
    rc = o.contiguous(two.ravel(), VIEW_DIMS, VIEW_STRIDES)
    rr = o.repeat_kv(kv, 3)
    assert_bitexact(eager[0], rr, "repeat_kv")
    assert_bitexact(eager[1], rc, "contiguous of the written source")
    assert_bitexact(eager[2], o.add(rr, rc), "add of both")
    assert_bitexact(eager[4], o.mul(view, view), "source rewritten after the gather")


def test_dependent_ops_are_split(ctx):
    """Read-after-write, write-after-read and write-after-write between
    recorded ops: each must see its predecessor's result."""
    a, b = norm("da", (T, H), F32), norm("db", (T, H), F32)
    da, db, dz = ctx.upload(a), ctx.upload(b), ctx.upload(np.zeros((T, H), F32))
    c, d, e, w = (ctx.empty((T, H), F32) for _ in range(4))

    def record():
        ctx.add(da, dz, w)    # w = a
        ctx.add(da, db, c)    # c = a + b
        ctx.mul(c, da, d)     # reads c (after write)
        ctx.silu(w, e)        # reads w (after write)
        ctx.add(d, db, w)     # writes w after it was read; reads d (after write)
        ctx.swiglu(w, c, c)   # reads w (after write), writes c in place

    outs = [c, d, e, w]
    eager = replay_and_compare(ctx, record, outs, reps=1)
    rc = o.add(a, b)
    rd = o.mul(rc, a)
    rw = o.add(rd, b)
    assert_bitexact(eager[1], rd, "mul after add")
    assert_bitexact(eager[3], rw, "add into a buffer read before")
    np.testing.assert_allclose(eager[2], o.silu(a), rtol=1e-5, atol=1e-30)
    np.testing.assert_allclose(eager[0], o.swiglu(rw, rc), rtol=1e-5, atol=1e-30)


def test_more_ops_than_one_launch_holds(ctx):
    """Twenty independent adds: more than a fused launch takes."""
    a, b = norm("ma", (64, H), F16), norm("mb", (64, H), F16)
    da, db = ctx.upload(a), ctx.upload(b)
    outs = [ctx.empty((64, H), F16) for _ in range(20)]

    def record():
        for x in outs:
            ctx.add(da, db, x)

    eager = replay_and_compare(ctx, record, outs)
    for x in eager:
        assert_bitexact(x, o.add(a, b), "add")


def test_ragged_sizes_in_one_launch(ctx):
    """Sizes that end inside a block and inside a pack: each op's last block
    is partly past its array and the elements after the last whole pack are
    its tail, in both dtypes, beside a bias add over 1,000 columns."""
    shape, bshape = (333, 1001), (333, 1000)
    host, outs, ops = [], [], []
    for dt in (F32, F16):
        a, b = norm("ra", shape, dt), norm("rb", shape, dt)
        x, bias = norm("rx", bshape, dt), norm("rbias", (1000,), dt)
        da, db, dx, dbias = ctx.upload(a), ctx.upload(b), ctx.upload(x), ctx.upload(bias)
        bufs = [ctx.empty(shape, dt) for _ in range(4)] + [ctx.empty(bshape, dt)]
        host.append((a, b, x, bias))
        outs += bufs
        ops += [lambda da=da, db=db, y=bufs[0]: ctx.add(da, db, y),
                lambda da=da, db=db, y=bufs[1]: ctx.mul(da, db, y),
                lambda da=da, y=bufs[2]: ctx.silu(da, y),
                lambda da=da, db=db, y=bufs[3]: ctx.swiglu(da, db, y),
                lambda dx=dx, dbias=dbias, y=bufs[4]: ctx.add_broadcast(dx, dbias, y)]

    def record():
        for op in ops:
            op()

    eager = replay_and_compare(ctx, record, outs)
    for k, (a, b, x, bias) in enumerate(host):
        e = eager[5 * k:5 * k + 5]
        assert_bitexact(e[0], o.add(a, b), "add")
        assert_bitexact(e[1], o.mul(a, b), "mul")
        assert_bitexact(e[4], o.add_broadcast(x, bias), "bias add")


def test_other_kernels_between_fused_ops(ctx):
    """An op outside the fused set (RMSNorm) reading a deferred op's output,
    and a deferred op reading the RMSNorm's, in one recording."""
    a, b = norm("ra", (T, 960), F16), norm("rb", (T, 960), F16)
    w = synth.uniform_range(3, (960,), 0.5, 1.5, F16)
    da, db, dw = ctx.upload(a), ctx.upload(b), ctx.upload(w)
    s, y, z = (ctx.empty((T, 960), F16) for _ in range(3))

    def record():
        ctx.add(da, db, s)
        ctx.rmsnorm(s, dw, 1e-5, y)
        ctx.mul(y, da, z)

    eager = replay_and_compare(ctx, record, [s, y, z])
    assert_bitexact(eager[0], o.add(a, b), "add")
    assert_bitexact(eager[2], o.mul(eager[1], a), "mul of the RMSNorm output")
