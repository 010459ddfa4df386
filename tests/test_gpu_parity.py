"""HIP library vs the CPU oracle through the C ABI, on seeded inputs.

Bars (stated per test): bit-exact for add, mul, cast, broadcast add,
contiguous, repeat_kv, scale/mask and RoPE (FMA contraction is off on both
sides); f32 RMSNorm / softmax / SiLU / SwiGLU within a max relative error of
1e-5 with a FLT_MIN magnitude floor; every f16 output within 2 ulp.
Shapes cover the reference's own test vectors, ragged sizes that exercise
the tail and unaligned paths, and the full benchmark configurations.
"""

import os

import numpy as np
import pytest

from helpers import assert_bitexact, f16_ulp_distance, floats, kats, max_rel_err
from oracle import oracle as o
from rustllm_amd import abi, synth

pytestmark = pytest.mark.gpu

K = kats()
TINY = np.finfo(np.float32).tiny
F32_REL = 1e-5
F16_ULP = 2

o.set_threads(min(16, os.cpu_count() or 1))


def norm(key, shape, dtype, mu=0.0, sigma=1.0):
    return synth.normal(synth.seed_for(*key, *shape, np.dtype(dtype).name), shape, mu, sigma,
                        dtype)


def check_float(got, ref, what):
    if got.dtype == np.float16:
        d = f16_ulp_distance(got, ref)
        assert d <= F16_ULP, f"{what}: {d} ulp"
    else:
        e = max_rel_err(got, ref, TINY)
        assert e <= F32_REL, f"{what}: max rel err {e:.3g}"


def run(ctx, fn):
    """Runs one batch (begin .. finish) and returns fn's result."""
    ctx.begin()
    out = fn()
    ctx.finish()
    return out


DT = [np.float32, np.float16]
SIZES = [1, 3, 7, 8, 9, 1000, 100_003, 4096 * 1536]


# ------------------------------------------------------------ element-wise

@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("n", SIZES)
def test_add_mul_bitexact(ctx, dtype, n):
    a = norm(("add", "a"), (n,), dtype)
    b = norm(("add", "b"), (n,), dtype)
    da, db = ctx.upload(a), ctx.upload(b)
    got_add = run(ctx, lambda: ctx.add(da, db)).numpy()
    assert_bitexact(got_add, o.add(a, b), f"add {dtype.__name__} n={n}")
    got_mul = run(ctx, lambda: ctx.mul(da, db)).numpy()
    assert_bitexact(got_mul, o.mul(a, b), f"mul {dtype.__name__} n={n}")


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("n", SIZES)
def test_silu_swiglu(ctx, dtype, n):
    g = norm(("silu", "g"), (n,), dtype, 0.0, 3.0)
    u = norm(("silu", "u"), (n,), dtype)
    dg, du = ctx.upload(g), ctx.upload(u)
    check_float(run(ctx, lambda: ctx.silu(dg)).numpy(), o.silu(g), f"silu n={n}")
    check_float(run(ctx, lambda: ctx.swiglu(dg, du)).numpy(), o.swiglu(g, u), f"swiglu n={n}")


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("op,shape", [("swiglu", (4096, 2560)), ("silu", (4096, 2560)),
                                      ("add", (4096, 960)), ("mul", (4096, 960))])
def test_smollm_layer_shapes(ctx, dtype, op, shape):
    """The SmolLM2-360M layer's element-wise shapes at 4096 tokens: SwiGLU on
    the [4096, 2560] FFN activations, the residual add on [4096, 960]."""
    a = norm(("layer", op, "a"), shape, dtype)
    b = norm(("layer", op, "b"), shape, dtype)
    da, db = ctx.upload(a), ctx.upload(b)
    if op in ("add", "mul"):
        got = run(ctx, lambda: getattr(ctx, op)(da, db)).numpy()
        assert_bitexact(got, getattr(o, op)(a, b), f"{op} {shape}")
    elif op == "silu":
        check_float(run(ctx, lambda: ctx.silu(da)).numpy(), o.silu(a), f"silu {shape}")
    else:
        check_float(run(ctx, lambda: ctx.swiglu(da, db)).numpy(), o.swiglu(a, b),
                    f"swiglu {shape}")


def test_silu_extremes(ctx):
    x = np.array([-1e30, -100, -88.7, -20, -1, -1e-30, -0.0, 0.0, 1e-30, 1, 20, 88.7, 100, 1e30,
                  np.inf, -np.inf], dtype=np.float32)
    got = run(ctx, lambda: ctx.silu(ctx.upload(x))).numpy()
    ref = o.silu(x)
    fin = np.isfinite(ref)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert max_rel_err(got[fin], ref[fin], TINY) <= F32_REL
    xh = np.array([-65504, -20, -1, -0.0, 0, 1e-7, 1, 20, 65504], dtype=np.float16)
    got = run(ctx, lambda: ctx.silu(ctx.upload(xh))).numpy()
    assert f16_ulp_distance(got, o.silu(xh)) <= F16_ULP


@pytest.mark.parametrize("n", [1000, 100_003, 4096 * 1536 + 8 * 100 + 5])
def test_silu_f16_in_place(ctx, n):
    """SiLU f16 written over its own input (out == input, which the ABI
    accepts) at sizes whose last block of packs is partial: every pack is
    stored only by the lane that owns it, so the result is the oracle's SiLU
    of the original input (within 2 ulp) -- eagerly, and recorded into a
    graph (the fused launch of recorded ops) and replayed twice, each time
    onto a fresh copy of the input."""
    x = norm(("silu-inplace",), (n,), np.float16, 0.0, 3.0)
    ref = o.silu(x)
    d = ctx.upload(x)
    run(ctx, lambda: ctx.silu(d, d))
    check_float(d.numpy(), ref, f"in-place silu n={n}")
    src, d2 = ctx.upload(x), ctx.upload(x)
    ctx.capture_begin()
    ctx.silu(d2, d2)
    graph = ctx.capture_end()
    for i in range(2):
        ctx.copy(src, d2)
        ctx.graph_launch(graph)
        ctx.finish()
        check_float(d2.numpy(), ref, f"in-place silu n={n}, graph replay {i}")
    ctx.graph_destroy(graph)


@pytest.mark.parametrize("n", [8 << 20, 8 * ((1 << 20) + 1000) + 5, 4096 * 2560])
def test_swiglu_f16_large_launch_shape(ctx, n):
    """SwiGLU f16 from 2^20 packs of 8 on runs four packs a thread in three
    phases (clamped loads, results, stores of owned packs only): at an exact
    multiple of the block's packs, with a partial last block plus 5 elements
    past the last pack, and at the layer's [4096, 2560] -- out of place and
    written over the gate and over the up operand, each within 2 ulp of the
    oracle."""
    g = norm(("swiglu-big", "g"), (n,), np.float16, 0.0, 3.0)
    u = norm(("swiglu-big", "u"), (n,), np.float16, 0.0, 2.0)
    ref = o.swiglu(g, u)
    dg, du = ctx.upload(g), ctx.upload(u)
    check_float(run(ctx, lambda: ctx.swiglu(dg, du)).numpy(), ref, f"swiglu n={n}")
    run(ctx, lambda: ctx.swiglu(dg, du, dg))
    check_float(dg.numpy(), ref, f"swiglu over gate n={n}")
    dg = ctx.upload(g)
    run(ctx, lambda: ctx.swiglu(dg, du, du))
    check_float(du.numpy(), ref, f"swiglu over up n={n}")


def test_silu_swiglu_f16_every_half(ctx):
    """SiLU over all 65,536 halves (incl. +-inf, NaN, subnormals and the range
    where the sigmoid's reciprocal is subnormal), and SwiGLU with every half as
    the gate against a few up values."""
    xh = np.arange(65536, dtype=np.uint16).view(np.float16)
    ref = o.silu(xh)
    got = run(ctx, lambda: ctx.silu(ctx.upload(xh))).numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert f16_ulp_distance(got[~nan], ref[~nan]) <= F16_ULP
    dg = ctx.upload(xh)
    for u in (1.0, -3.5, 65504.0, 1e-3):
        uh = np.full(xh.shape, u, dtype=np.float16)
        ref = o.swiglu(xh, uh)
        got = run(ctx, lambda: ctx.swiglu(dg, ctx.upload(uh))).numpy()
        nan = np.isnan(ref)
        assert np.array_equal(np.isnan(got), nan), u
        assert f16_ulp_distance(got[~nan], ref[~nan]) <= F16_ULP, u


@pytest.mark.parametrize("n", SIZES)
def test_cast_bitexact(ctx, n):
    x = norm(("cast",), (n,), np.float32, 0.0, 2000.0)
    got = run(ctx, lambda: ctx.cast(ctx.upload(x), np.float16)).numpy()
    assert_bitexact(got, o.cast(x, np.float16), f"cast f32->f16 n={n}")
    h = x.astype(np.float16)
    got = run(ctx, lambda: ctx.cast(ctx.upload(h), np.float32)).numpy()
    assert_bitexact(got, o.cast(h, np.float32), f"cast f16->f32 n={n}")


def test_cast_rounding_probe(ctx):
    """Every sign/exponent/top-mantissa pattern with the rounding-deciding low
    bits, including subnormal results, overflow to inf and NaN."""
    high = np.arange(1 << 19, dtype=np.uint32) << np.uint32(13)
    lows = np.array([0, 1, 0x0FFF, 0x1000, 0x1001, 0x1FFF], dtype=np.uint32)
    x = (high[:, None] | lows[None, :]).ravel().view(np.float32)
    got = run(ctx, lambda: ctx.cast(ctx.upload(x), np.float16)).numpy()
    assert_bitexact(got, o.cast(x, np.float16), "cast probe")
    every = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    got = run(ctx, lambda: ctx.cast(ctx.upload(every), np.float32)).numpy()
    assert_bitexact(got, o.cast(every, np.float32), "f16->f32 exhaustive")


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("rows,cols", [(4096, 1536), (3, 5), (17, 24), (1, 8), (4095, 960),
                                       (6, 4096), (5, 8200), (2, 8192 + 8)])
def test_add_broadcast_bitexact(ctx, dtype, rows, cols):
    x = norm(("bias", "x"), (rows, cols), dtype)
    b = norm(("bias", "b"), (cols,), dtype)
    got = run(ctx, lambda: ctx.add_broadcast(ctx.upload(x), ctx.upload(b))).numpy()
    assert_bitexact(got, o.add_broadcast(x, b), f"bias add {rows}x{cols}")


# ------------------------------------------------------------ reference KATs

def test_reference_kats_elementwise(ctx):
    kat = K["add_f16"]
    a = np.array(kat["left"], np.float16).reshape(kat["shape"])
    b = np.array(kat["right"], np.float16).reshape(kat["shape"])
    got = run(ctx, lambda: ctx.add(ctx.upload(a), ctx.upload(b))).numpy()
    assert got.astype(np.float32).ravel().tolist() == kat["expected"]

    # Two ops in one batch, no wait in between (ops/add.rs:113-168, ops/mul.rs:132-203)
    kat = K["chained_add_f16"]
    da, db, dc = (ctx.upload(np.array(kat[k], np.float16)) for k in ("a", "b", "c"))
    got = run(ctx, lambda: ctx.add(ctx.add(da, db), dc)).numpy().astype(np.float32)
    assert np.all(np.abs(got - kat["expected"]) < kat["tol"])
    kat = K["add_then_mul_f16"]
    da, db, dc = (ctx.upload(np.array(kat[k], np.float16)) for k in ("a", "b", "c"))
    got = run(ctx, lambda: ctx.mul(ctx.add(da, db), dc)).numpy().astype(np.float32)
    assert np.all(np.abs(got - kat["expected"]) < kat["tol"])
    kat = K["silu_then_mul_f16"]
    dg, du = ctx.upload(np.array(kat["gate"], np.float16)), ctx.upload(np.array(kat["up"],
                                                                                   np.float16))
    got = run(ctx, lambda: ctx.mul(ctx.silu(dg), du)).numpy().astype(np.float32)
    assert np.all(np.abs(got - kat["expected"]) < kat["tol"])


# ------------------------------------------------------------ data movement

def _view_strides(arr):
    return [s // arr.itemsize for s in arr.strides]


@pytest.mark.parametrize("dtype", DT)
def test_contiguous_config_transpose(ctx, dtype):
    # [1, 9, 4096, 64] view of a contiguous [1, 4096, 9, 64] (permute [0, 2, 1, 3])
    base = norm(("contig",), (1, 4096, 9, 64), dtype)
    dims, strides = [1, 9, 4096, 64], [4096 * 9 * 64, 64, 9 * 64, 1]
    d = ctx.upload(base)
    got = run(ctx, lambda: ctx.contiguous(d, dims, strides)).numpy()
    assert_bitexact(got, o.contiguous(base.ravel(), dims, strides), "contiguous config")
    assert_bitexact(got, np.ascontiguousarray(base.transpose(0, 2, 1, 3)), "vs numpy")


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("seed", range(12))
def test_contiguous_random_permutations(ctx, dtype, seed):
    rng = np.random.default_rng(seed)
    rank = int(rng.integers(1, 6))
    shape = [int(v) for v in rng.integers(1, 9, rank)]
    base = norm(("perm", seed), tuple(shape), dtype)
    perm = [int(v) for v in rng.permutation(rank)]
    view = base.transpose(perm)
    dims, strides = list(view.shape), _view_strides(view)
    got = run(ctx, lambda: ctx.contiguous(ctx.upload(base), dims, strides)).numpy()
    assert_bitexact(got, np.ascontiguousarray(view), f"perm {shape} {perm}")


@pytest.mark.parametrize("dtype", DT)
def test_contiguous_dense_permutations_rowwise(ctx, dtype):
    """Permutations of dense tensors that keep the stride-1 dim innermost
    (copied in source order, whole rows) at ranks 3-5 with 16-byte packs and
    grids of many blocks, and permutes of a narrowed tensor (gaps between the
    rows: copied in output order) -- all bit-exact against numpy."""
    cases = [((7, 300, 64), (1, 0, 2)), ((2, 129, 5, 64), (0, 2, 1, 3)),
             ((3, 4, 50, 32), (2, 0, 1, 3)), ((2, 3, 4, 5, 16), (3, 1, 0, 2, 4)),
             ((64, 9, 128), (1, 0, 2))]
    for shape, perm in cases:
        base = norm(("dperm", shape), shape, dtype)
        view = base.transpose(perm)
        got = run(ctx, lambda: ctx.contiguous(ctx.upload(base), list(view.shape),
                                              _view_strides(view))).numpy()
        assert_bitexact(got, np.ascontiguousarray(view), f"dense {shape} {perm}")
    base = norm(("narrowed",), (6, 200, 64), dtype)
    for view in (base[:, 3:150].transpose(1, 0, 2), base[1:5].transpose(1, 0, 2)):
        offset = (view.__array_interface__["data"][0] - base.__array_interface__["data"][0]) \
            // base.itemsize
        src = ctx.upload(base.ravel()[offset:].copy())
        got = run(ctx, lambda: ctx.contiguous(src, list(view.shape), _view_strides(view))).numpy()
        assert_bitexact(got, np.ascontiguousarray(view), f"narrowed {view.shape}")


def test_contiguous_special_views(ctx):
    # stride-0 broadcast, transposed inner dims (per-element path), narrowed KV cache
    bias = norm(("b0",), (24,), np.float32)
    got = run(ctx, lambda: ctx.contiguous(ctx.upload(bias), [100, 24], [0, 1])).numpy()
    assert_bitexact(got, np.broadcast_to(bias, (100, 24)).copy())
    m = norm(("t",), (33, 65), np.float16)
    got = run(ctx, lambda: ctx.contiguous(ctx.upload(m), [65, 33], [1, 65])).numpy()
    assert_bitexact(got, m.T.copy())
    kat = K["kv_cache_narrow_contiguous"]
    _, heads, max_seq, hd = kat["cache_shape"]
    cache = np.zeros(kat["cache_shape"], np.float16)
    for pos, vals in enumerate(kat["appends"]):
        cache[:, :, pos, :] = np.array(vals, np.float16).reshape(heads, hd)
    n = kat["narrow_len"]
    got = run(ctx, lambda: ctx.contiguous(ctx.upload(cache), [1, heads, n, hd],
                                          [heads * max_seq * hd, max_seq * hd, hd, 1])).numpy()
    assert got.astype(np.float32).ravel().tolist() == kat["expected"]


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("shape,repeats", [((1, 3, 4096, 64), 3), ((1, 5, 4096, 64), 3),
                                           ((2, 2, 7, 5), 4), ((1, 2, 2, 2), 3),
                                           ((1, 1, 2, 2), 1)])
def test_repeat_kv_bitexact(ctx, dtype, shape, repeats):
    x = norm(("rkv",), shape, dtype)
    got = run(ctx, lambda: ctx.repeat_kv(ctx.upload(x), repeats)).numpy()
    assert_bitexact(got, o.repeat_kv(x, repeats), f"repeat_kv {shape} x{repeats}")


def test_repeat_kv_kat(ctx):
    kat = K["repeat_kv_r3"]
    for dt in (np.float32, np.float16):
        x = np.array(kat["input"], dt).reshape(kat["shape"])
        got = run(ctx, lambda: ctx.repeat_kv(ctx.upload(x), kat["repeats"])).numpy()
        assert list(got.shape) == kat["expected_shape"]
        assert got.astype(np.float32).ravel().tolist() == kat["expected"]


# ---------------------------------------------------------------- RMSNorm

@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("hidden", [576, 768, 960])
@pytest.mark.parametrize("tokens", [1, 16, 256, 4096, 16384])
def test_rmsnorm_config_grid(ctx, dtype, hidden, tokens):
    x = norm(("rms", "x"), (tokens, hidden), dtype, 0.0, 2.0)
    w = synth.uniform_range(synth.seed_for("rms", "w", hidden), (hidden,), 0.5, 1.5, dtype)
    got = run(ctx, lambda: ctx.rmsnorm(ctx.upload(x), ctx.upload(w), 1e-5)).numpy()
    check_float(got, o.rmsnorm(x, w, 1e-5), f"rmsnorm {tokens}x{hidden}")


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("rows,hidden", [(2, 4), (3, 5), (5, 4097), (2, 20000), (1, 1)])
def test_rmsnorm_odd_and_large_rows(ctx, dtype, rows, hidden):
    x = norm(("rms2", "x"), (rows, hidden), dtype, 0.0, 2.0)
    w = synth.uniform_range(synth.seed_for("rms2", "w", hidden), (hidden,), 0.5, 1.5, dtype)
    got = run(ctx, lambda: ctx.rmsnorm(ctx.upload(x), ctx.upload(w), 1e-5)).numpy()
    check_float(got, o.rmsnorm(x, w, 1e-5), f"rmsnorm {rows}x{hidden}")


# Row lengths in 16-byte packs that select each lane-group width x packs-per-
# lane kernel of the row planner (16/32/64 lanes per row, 1..16 packs each).
# Narrow groups are only chosen for launches of >= 4096 waves, hence the
# second row count; neither count is a multiple of a rows-per-block count.
RMS_PACKS = [2, 20, 48, 50, 70, 100, 120, 130, 150, 170, 180, 200, 240, 270, 300, 330, 360,
             400, 600, 700, 1000, 1024]
RMS_PLAN_CASES = [(p, 37) for p in RMS_PACKS] + [(p, 16411) for p in RMS_PACKS if p <= 352]


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("packs,rows", RMS_PLAN_CASES)
def test_rmsnorm_row_plans(ctx, dtype, packs, rows):
    hidden = packs * (16 // np.dtype(dtype).itemsize)
    x = norm(("rmsplan", "x"), (rows, hidden), dtype, 0.0, 2.0)
    r = norm(("rmsplan", "r"), (rows, hidden), dtype)
    w = synth.uniform_range(synth.seed_for("rmsplan", "w", hidden), (hidden,), 0.5, 1.5, dtype)
    dx, dr, dw = ctx.upload(x), ctx.upload(r), ctx.upload(w)
    got = run(ctx, lambda: ctx.rmsnorm(dx, dw, 1e-5)).numpy()
    check_float(got, o.rmsnorm(x, w, 1e-5), f"rmsnorm {rows}x{hidden}")
    s, y = run(ctx, lambda: ctx.add_rmsnorm(dx, dr, dw, 1e-5))
    rs, ry = o.add_rmsnorm(x, r, w, 1e-5)
    assert_bitexact(s.numpy(), rs, "residual sum")
    check_float(y.numpy(), ry, f"add_rmsnorm {rows}x{hidden}")


def test_rmsnorm_reference_kats(ctx):
    kat = K["rmsnorm_2x4"]
    x = np.array(kat["input"], np.float32)
    w = np.array(kat["weight"], np.float32)
    expected = o.cpu_rmsnorm_literal(x, w, kat["eps"])
    got = run(ctx, lambda: ctx.rmsnorm(ctx.upload(x), ctx.upload(w), kat["eps"])).numpy()
    assert np.max(np.abs(got - expected)) <= kat["tol_f32"]
    xh, wh = x.astype(np.float16), w.astype(np.float16)
    zeros = ctx.upload(np.zeros(8, np.float16))
    dx, dw = ctx.upload(xh), ctx.upload(wh)
    got = run(ctx, lambda: ctx.add(ctx.rmsnorm(dx, dw, kat["eps"]), zeros)).numpy()
    assert np.max(np.abs(got.astype(np.float32) - expected)) <= kat["tol_f16"]


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("rows,hidden", [(64, 768), (4096, 960), (3, 5), (2, 9000)])
def test_add_rmsnorm(ctx, dtype, rows, hidden):
    # the reference's CPU-runnable case: out = RMSNorm(x + r) * w on f32 [64, 768]
    x = norm(("arms", "x"), (rows, hidden), dtype)
    r = norm(("arms", "r"), (rows, hidden), dtype)
    w = synth.uniform_range(synth.seed_for("arms", "w", hidden), (hidden,), 0.5, 1.5, dtype)
    s, y = run(ctx, lambda: ctx.add_rmsnorm(ctx.upload(x), ctx.upload(r), ctx.upload(w), 1e-5))
    rs, ry = o.add_rmsnorm(x, r, w, 1e-5)
    assert_bitexact(s.numpy(), rs, "residual sum")
    check_float(y.numpy(), ry, f"add_rmsnorm {rows}x{hidden}")


# ---------------------------------------------------------------- softmax

def _logits(key, shape, dtype=np.float32):
    """N(0, 4) logits with 1% of entries set to +20 (spiky attention scores)."""
    x = synth.normal(synth.seed_for(*key, *shape), shape, 0.0, 4.0, np.float32)
    u = synth.uniform(synth.seed_for("spike", *key, *shape), x.size).reshape(shape)
    x[u < 0.01] = 20.0
    return x.astype(dtype)


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("rows,width", [(2, 3), (7, 33), (64, 2048), (9, 4096), (5, 5000),
                                        (3, 9000), (2, 70000), (1, 1),
                                        # widths off the pack grid: rows at every lead
                                        (13, 4093), (6, 1001), (4, 9003), (9, 130),
                                        (5, 2041)])
def test_softmax(ctx, dtype, rows, width):
    x = _logits(("sm",), (rows, width), dtype)
    got = run(ctx, lambda: ctx.softmax(ctx.upload(x))).numpy()
    check_float(got, o.softmax(x), f"softmax {rows}x{width}")


@pytest.mark.parametrize("width", [8, 3, 5000, 70000, 1001])
def test_softmax_special_rows(ctx, width):
    # all -inf: f32 NaN (no guard, softmax.metal:7-132), f16 zeros (:166-173);
    # a NaN score poisons its row; -inf entries get exact zeros; scores 85..110
    # below the max give subnormal probabilities, which must not flush to 0.
    x = np.zeros((5, width), np.float32)
    x[0] = -np.inf
    x[1, 0] = np.nan
    x[2, ::2] = -np.inf
    x[3] = np.linspace(-3, 3, width, dtype=np.float32)
    x[4] = -np.linspace(0, 110, width, dtype=np.float32)
    for dt in DT:
        xi = x.astype(dt)
        got = run(ctx, lambda: ctx.softmax(ctx.upload(xi))).numpy()
        ref = o.softmax(xi)
        assert np.array_equal(np.isnan(got), np.isnan(ref)), dt
        ok = ~np.isnan(ref)
        assert np.array_equal(got[ok] == 0, ref[ok] == 0), dt
        check_float(np.where(ok, got, 0).astype(dt), np.where(ok, ref, 0).astype(dt), "special")


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("shape,start", [((9, 2048, 2048), 0), ((9, 1, 2048), 2047),
                                         ((1, 1, 3, 3), 0), ((2, 5, 40), 11),
                                         ((3, 4, 6000), 100), ((1, 2, 70000), 3),
                                         # key lengths off the pack grid
                                         ((3, 7, 4093), 0), ((2, 9, 1001), 500),
                                         ((4, 5, 35), 30), ((1, 13, 1003), 990),
                                         ((2, 6, 2041), 7)])
def test_scale_mask_and_fused_softmax(ctx, dtype, shape, start):
    x = _logits(("att",), shape, dtype)
    scale = 1.0 / 8.0
    d = ctx.upload(x)
    ref_mask = o.scale_mask(x, scale, start)
    got_mask = run(ctx, lambda: ctx.scale_mask(d, scale, start)).numpy()
    assert_bitexact(got_mask, ref_mask, f"scale/mask {shape}")
    ref = o.softmax(ref_mask)  # the reference's two adjacent calls
    got = run(ctx, lambda: ctx.attention_softmax(d, scale, start)).numpy()
    check_float(got, ref, f"fused {shape}")
    masked = np.isinf(ref_mask)
    assert np.all(got[masked] == 0), "masked probabilities must be exact zeros"
    # and the unfused pair on the device agrees with the fused kernel's bar too
    got2 = run(ctx, lambda: ctx.softmax(ctx.scale_mask(d, scale, start))).numpy()
    check_float(got2, ref, f"unfused {shape}")


SCALES = [0.125, 1.0 / np.sqrt(80.0), 0.3, 1.0 / 3.0, 2.0, 1.0]


@pytest.mark.parametrize("scale", SCALES)
def test_scale_mask_f16_every_half(ctx, scale):
    """f16 scale/mask over all 65,536 halves (+-0, subnormals, +-inf, NaN) in
    one decode row (every key kept), bit-exact against the oracle's f32
    product rounded to f16 -- for scales that are f16 values (1/8, 2, 1) and
    scales that are not (1/sqrt(80), 0.3, 1/3), where the f32 product's own
    rounding matters."""
    xh = np.arange(65536, dtype=np.uint16).view(np.float16).reshape(1, 1, 65536)
    d = ctx.upload(xh)
    got = run(ctx, lambda: ctx.scale_mask(d, float(np.float32(scale)), 65535)).numpy()
    assert_bitexact(got, o.scale_mask(xh, float(np.float32(scale)), 65535), f"scale {scale}")


@pytest.mark.parametrize("scale", SCALES)
@pytest.mark.parametrize("shape,start", [((4, 64, 1000), 936), ((15, 256, 4096), 3840),
                                         ((3, 33, 4093), 100), ((2, 16, 512), 0)])
def test_fused_softmax_f16_scales(ctx, scale, shape, start):
    """Fused causal scale/mask + softmax in f16 at scales that are f16 values
    (the launch that scales pairs of halves) and scales that are not (the
    element-wise launch), on N(0, 2) scores with -0.0, +-inf and NaN planted
    in a few rows: within 2 ulp of the oracle, masked entries exactly 0, NaN
    and zero rows where the oracle has them."""
    x = norm(("fused-scales", start), shape, np.float16, 0.0, 2.0)
    flat = x.reshape(-1, shape[-1])
    flat[1, :7] = -0.0
    flat[2, 3] = np.inf
    flat[3, 0] = np.nan
    flat[4, :] = -np.inf
    flat[5, 2] = -np.inf
    s = float(np.float32(scale))
    got = run(ctx, lambda: ctx.attention_softmax(ctx.upload(x), s, start)).numpy()
    ref = o.attention_softmax(x, s, start)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan), "NaN positions"
    assert np.array_equal(got[~nan] == 0, ref[~nan] == 0), "zero positions"
    check_float(np.where(nan, 0, got).astype(np.float16), np.where(nan, 0, ref).astype(np.float16),
                f"fused softmax f16 scale {scale} {shape}")


def test_scale_mask_reference_kats(ctx):
    kat = K["scale_mask_prefill"]
    x = np.array(kat["input"], np.float32).reshape(kat["shape"])
    got = run(ctx, lambda: ctx.scale_mask(ctx.upload(x), kat["scale"], kat["start"])).numpy()
    assert_bitexact(got.ravel(), floats(kat["expected_f32"]))
    for name in ("scale_mask_decode", "scale_mask_intermediate"):
        kat = K[name]
        x = np.array(kat["input"], np.float16).reshape(kat["shape"])
        got = run(ctx, lambda: ctx.scale_mask(ctx.upload(x), kat["scale"], kat["start"]))
        assert_bitexact(got.numpy().astype(np.float32).ravel(), floats(kat["expected"]))
    kat = K["mask_softmax"]
    x = np.array(kat["input"], np.float32).reshape(kat["shape"])
    ref = o.attention_softmax(x, kat["scale"], kat["start"])
    for fused in (True, False):
        d = ctx.upload(x.astype(np.float16))
        if fused:
            got = run(ctx, lambda: ctx.attention_softmax(d, kat["scale"], kat["start"]))
        else:
            got = run(ctx, lambda: ctx.softmax(ctx.scale_mask(d, kat["scale"], kat["start"])))
        got = got.numpy().astype(np.float32)
        assert np.max(np.abs(got - ref)) < kat["tol_f16_vs_f32"]
        assert all(got.ravel()[i] == 0.0 for i in kat["zero_indices"])


def test_fused_softmax_smollm_layer_f16(ctx):
    """SmolLM2-360M layer at 4096 tokens: [15, 4096, 4096] f16 causal scores,
    scale 1/8."""
    rng = np.random.default_rng(synth.seed_for("c5", "scores"))
    x = rng.standard_normal((15, 4096, 4096), dtype=np.float32).astype(np.float16)
    d = ctx.upload(x)
    got = run(ctx, lambda: ctx.attention_softmax(d, 0.125, 0)).numpy()
    del d
    ref = o.attention_softmax(x, 0.125, 0)
    check_float(got, ref, "SmolLM2 layer fused softmax")
    del ref
    # size-independent invariants: each row sums to 1 and nothing past the diagonal
    sums = np.add.reduce(got, axis=-1, dtype=np.float32)
    assert np.all(np.abs(sums - 1.0) < 4e-3)
    upper = np.triu(np.ones((4096, 4096), bool), 1)
    for h in range(15):
        assert not got[h][upper].any()


@pytest.mark.parametrize("dtype,scale", [(np.float32, 0.125), (np.float16, 0.1)])
def test_fused_softmax_streamed_rows(ctx, dtype, scale):
    """Rows on the 16-byte grid are read plainly when a launch reads at most
    160 MB of kept keys and streamed above: 2048 queries after 2048 cached
    keys over 15 heads keep 377 MB (f32) / 189 MB (f16) -- the streamed
    variants of the row kernel (f32) and of the f16 rows at a scale that is
    not an f16 value (0.1), against the oracle."""
    rng = np.random.default_rng(synth.seed_for("streamed-rows", np.dtype(dtype).name))
    x = rng.standard_normal((15, 2048, 4096), dtype=np.float32).astype(dtype)
    d = ctx.upload(x)
    got = run(ctx, lambda: ctx.attention_softmax(d, scale, 2048)).numpy()
    del d
    check_float(got, o.attention_softmax(x, scale, 2048), f"streamed rows {np.dtype(dtype).name}")


# ------------------------------------------------------------------- RoPE

@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("shape,start,table", [((1, 15, 4096, 64), 0, 4096),
                                               ((1, 5, 4096, 64), 0, 4096),
                                               ((1, 1, 2, 4), 1, 8), ((2, 3, 7, 6), 5, 16),
                                               ((1, 2, 1, 64), 4000, 4096)])
def test_rope_bitexact(ctx, dtype, shape, start, table):
    head_dim = shape[-1]
    c, s = o.rope_table(head_dim, table, 10000.0)
    x = norm(("rope",), shape, dtype)
    dc, ds = ctx.upload(c), ctx.upload(s)
    got = run(ctx, lambda: ctx.rope(ctx.upload(x), dc, ds, start)).numpy()
    assert_bitexact(got, o.rope(x, c, s, start), f"rope {shape} start={start}")


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("seq,heads", [(4096, 15), (4096, 5), (3, 2), (1, 1)])
def test_rope_fused_transpose_gather(ctx, dtype, seq, heads):
    """ops::rope_encode on the [1, H, S, D] permute of a [1, S, H, D] projection
    (nn/attention.rs:403-407): gather + rotation in one pass equals
    contiguous() then rope()."""
    hd = 64
    c, s = o.rope_table(hd, max(seq, 8), 10000.0)
    base = norm(("ropeT",), (1, seq, heads, hd), dtype)
    dims, strides = [1, heads, seq, hd], [seq * heads * hd, hd, heads * hd, 1]
    ref = o.rope(o.contiguous(base.ravel(), dims, strides), c, s, 0)
    dc, ds = ctx.upload(c), ctx.upload(s)
    got = run(ctx, lambda: ctx.rope_strided(ctx.upload(base), dims, strides, dc, ds, 0)).numpy()
    assert_bitexact(got, ref, f"fused rope {seq}x{heads}")


ROW_BLOCK_DIMS = {"f16": [16, 32, 64, 128], "f32": [8, 16, 32, 64]}


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("lane_case", [0, 1, 2, 3])
@pytest.mark.parametrize("seq,start", [(1, 0), (33, 7), (300, 0)])
def test_rope_every_row_width(ctx, dtype, lane_case, seq, start):
    """Rows of 32, 64, 128 and 256 bytes (2, 4, 8 and 16 lanes of 16 bytes
    each), position counts that do and do not fill whole blocks, a start
    offset, a contiguous [2, 3, S, D] input and a rank-5 permuted view."""
    hd = ROW_BLOCK_DIMS["f16" if dtype == np.float16 else "f32"][lane_case]
    c, s = o.rope_table(hd, seq + start + 3, 10000.0)
    dc, ds = ctx.upload(c), ctx.upload(s)
    x = norm(("ropeW", hd), (2, 3, seq, hd), dtype)
    got = run(ctx, lambda: ctx.rope(ctx.upload(x), dc, ds, start)).numpy()
    assert_bitexact(got, o.rope(x, c, s, start), f"rope D={hd} S={seq} start={start}")
    # [2, S, 2, 3, D] seen as [2, 3, 2, S, D]
    base = norm(("ropeW5", hd), (2, seq, 2, 3, hd), dtype)
    dims = [2, 3, 2, seq, hd]
    strides = [seq * 6 * hd, hd, 3 * hd, 6 * hd, 1]
    ref = o.rope(o.contiguous(base.ravel(), dims, strides), c, s, start)
    got = run(ctx, lambda: ctx.rope_strided(ctx.upload(base), dims, strides, dc, ds,
                                            start)).numpy()
    assert_bitexact(got, ref, f"rank-5 view D={hd} S={seq}")


@pytest.mark.parametrize("dtype", DT)
def test_rope_rows_off_the_fast_layout(ctx, dtype):
    """Rows that the 16-byte-lane kernel does not take: f32 rows of 512 bytes,
    and a view whose row starts are 4 bytes apart from 16-byte alignment."""
    c, s = o.rope_table(128, 64, 10000.0)
    dc, ds = ctx.upload(c), ctx.upload(s)
    x = norm(("ropeF", 128), (1, 2, 33, 128), dtype)
    got = run(ctx, lambda: ctx.rope(ctx.upload(x), dc, ds, 5)).numpy()
    assert_bitexact(got, o.rope(x, c, s, 5), "D=128")
    c, s = o.rope_table(64, 64, 10000.0)
    dc, ds = ctx.upload(c), ctx.upload(s)
    base = norm(("ropeF", 66), (1, 40, 3, 66), dtype)
    dims, strides = [1, 3, 40, 64], [40 * 3 * 66, 66, 3 * 66, 1]
    ref = o.rope(o.contiguous(base.ravel(), dims, strides), c, s, 2)
    got = run(ctx, lambda: ctx.rope_strided(ctx.upload(base), dims, strides, dc, ds,
                                            2)).numpy()
    assert_bitexact(got, ref, "stride 66 view")


def test_rope_reference_kats(ctx):
    kat = K["rope_f16_vs_f32"]
    c, s = o.rope_table(kat["head_dim"], kat["max_seq_len"], kat["theta"])
    dc, ds = ctx.upload(c), ctx.upload(s)
    x = np.array(kat["input"], np.float32).reshape(kat["shape"])
    ref = run(ctx, lambda: ctx.rope(ctx.upload(x), dc, ds, kat["start"])).numpy()
    got = run(ctx, lambda: ctx.rope(ctx.upload(x.astype(np.float16)), dc, ds, kat["start"]))
    assert np.max(np.abs(got.numpy().astype(np.float32) - ref)) <= kat["tol_f16_vs_f32"]
    kat = K["rope_non_contiguous"]
    c, s = o.rope_table(kat["head_dim"], kat["max_seq_len"], kat["theta"])
    base = np.array(kat["input"], np.float16).reshape(kat["shape"])
    view = base.transpose(kat["permute"])
    got = run(ctx, lambda: ctx.rope_strided(ctx.upload(base), list(view.shape),
                                            _view_strides(view), ctx.upload(c), ctx.upload(s),
                                            kat["start"])).numpy()
    assert got.dtype == np.float16 and got.flags["C_CONTIGUOUS"]
    assert_bitexact(got, o.rope(np.ascontiguousarray(view), c, s, kat["start"]))


# ------------------------------------------------------ KV cache, embedding

# (kv_heads, max_seq, head_dim, seq_len, start)
KV_CASES = [(5, 4096, 64, 4096, 0), (5, 4096, 64, 1, 4095), (5, 4096, 64, 7, 100),
            (4, 300, 128, 77, 200), (3, 64, 16, 40, 10),
            (2, 8, 4, 1, 3), (3, 17, 6, 5, 12), (2, 9, 5, 4, 2)]


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("heads,max_seq,hd,seq,start", KV_CASES)
def test_kv_cache_write_bitexact(ctx, dtype, heads, max_seq, hd, seq, start):
    """ops::kv_cache_write_*: rows start.. of each head are replaced, every
    other row of the cache keeps its contents."""
    cache0 = norm(("kvc",), (1, heads, max_seq, hd), dtype)
    src = norm(("kvs",), (1, heads, seq, hd), dtype)
    dc = ctx.upload(cache0)
    run(ctx, lambda: ctx.kv_cache_write(dc, ctx.upload(src), start))
    assert_bitexact(dc.numpy(), o.kv_cache_write(cache0, src, start), "kv_cache_write")


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("heads,max_seq,hd,seq,start", KV_CASES)
def test_kv_cache_write_from_projection_view(ctx, dtype, heads, max_seq, hd, seq, start):
    """append_encode's contiguous + kv_cache_write in one pass, from the
    [1, H, S, D] permute of a [1, S, H, D] projection."""
    cache0 = norm(("kvc2",), (1, heads, max_seq, hd), dtype)
    proj = norm(("kvp",), (1, seq, heads, hd), dtype)
    dims, strides = [1, heads, seq, hd], [seq * heads * hd, hd, heads * hd, 1]
    dc = ctx.upload(cache0)
    run(ctx, lambda: ctx.kv_cache_write_strided(ctx.upload(proj), dims, strides, dc, start))
    ref = o.kv_cache_write(cache0, o.contiguous(proj.ravel(), dims, strides), start)
    assert_bitexact(dc.numpy(), ref, "strided kv_cache_write")


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("heads,max_seq,hd,seq,start",
                         [c for c in KV_CASES if c[2] % 2 == 0])
def test_rope_kv_cache_write_bitexact(ctx, dtype, heads, max_seq, hd, seq, start):
    """RoPE of the key view at positions start.. written straight into the
    cache equals contiguous -> rope -> kv_cache_write."""
    c, s = o.rope_table(hd, max_seq, 10000.0)
    cache0 = norm(("kvc3",), (1, heads, max_seq, hd), dtype)
    proj = norm(("kvr",), (1, seq, heads, hd), dtype)
    dims, strides = [1, heads, seq, hd], [seq * heads * hd, hd, heads * hd, 1]
    dc, dcos, dsin = ctx.upload(cache0), ctx.upload(c), ctx.upload(s)
    run(ctx, lambda: ctx.rope_kv_cache_write(ctx.upload(proj), dims, strides, dcos, dsin,
                                             start, dc))
    rotated = o.rope(o.contiguous(proj.ravel(), dims, strides), c, s, start)
    assert_bitexact(dc.numpy(), o.kv_cache_write(cache0, rotated, start), "rope+kv write")


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("qh,kvh,seq,hd,start,max_seq", [(15, 5, 4096, 64, 0, 4096),
                                                         (15, 5, 1, 64, 100, 4096),
                                                         (6, 2, 77, 32, 9, 90),
                                                         (4, 4, 40, 16, 0, 40),
                                                         (3, 1, 19, 128, 2, 30),
                                                         (4, 2, 7, 6, 3, 12),
                                                         (2, 2, 5, 2, 0, 5)])
def test_qkv_rope_kv_append_one_launch(ctx, dtype, qh, kvh, seq, hd, start, max_seq):
    """Q and K rotated, K and V appended to the caches, in one launch, equals
    contiguous -> rope (Q, K) and contiguous -> kv_cache_write (K, V)."""
    c, s = o.rope_table(hd, max_seq, 10000.0)
    qp = norm(("qkv", "q"), (1, seq, qh, hd), dtype)
    kp = norm(("qkv", "k"), (1, seq, kvh, hd), dtype)
    vp = norm(("qkv", "v"), (1, seq, kvh, hd), dtype)
    kc0 = norm(("qkv", "kc"), (1, kvh, max_seq, hd), dtype)
    vc0 = norm(("qkv", "vc"), (1, kvh, max_seq, hd), dtype)

    def view(h):
        return [1, h, seq, hd], [seq * h * hd, hd, h * hd, 1]

    qd, qs = view(qh)
    kd, ks = view(kvh)
    dkc, dvc = ctx.upload(kc0), ctx.upload(vc0)
    dcos, dsin = ctx.upload(c), ctx.upload(s)
    q_out = run(ctx, lambda: ctx.qkv_rope_kv_append(
        (ctx.upload(qp), qd, qs), (ctx.upload(kp), kd, ks), (ctx.upload(vp), kd, ks),
        dcos, dsin, start, dkc, dvc)).numpy()
    q_ref = o.rope(o.contiguous(qp.ravel(), qd, qs), c, s, start)
    k_ref = o.kv_cache_write(kc0, o.rope(o.contiguous(kp.ravel(), kd, ks), c, s, start), start)
    v_ref = o.kv_cache_write(vc0, o.contiguous(vp.ravel(), kd, ks), start)
    assert_bitexact(q_out, q_ref, "Q")
    assert_bitexact(dkc.numpy(), k_ref, "K cache")
    assert_bitexact(dvc.numpy(), v_ref, "V cache")


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("qh,kvh,seq,hd,start,max_seq", [(15, 5, 4096, 64, 0, 4096),
                                                         (15, 5, 1, 64, 100, 4096),
                                                         (6, 2, 77, 32, 9, 90),
                                                         (4, 4, 40, 16, 3, 50),
                                                         (3, 1, 19, 128, 2, 30),
                                                         (4, 2, 7, 6, 3, 12)])
def test_qkv_rope_kv_append_repeat_one_launch(ctx, dtype, qh, kvh, seq, hd, start, max_seq):
    """The QKV launch with repeat_kv of both caches' prefixes after the append
    equals rope (Q, K), kv_cache_write (K, V), then repeat_kv of the first
    start + S cache rows made contiguous (tensor/repeat_kv.rs:31-35)."""
    n_rep = qh // kvh
    c, s = o.rope_table(hd, max_seq, 10000.0)
    qp = norm(("qkvr", "q"), (1, seq, qh, hd), dtype)
    kp = norm(("qkvr", "k"), (1, seq, kvh, hd), dtype)
    vp = norm(("qkvr", "v"), (1, seq, kvh, hd), dtype)
    kc0 = norm(("qkvr", "kc"), (1, kvh, max_seq, hd), dtype)
    vc0 = norm(("qkvr", "vc"), (1, kvh, max_seq, hd), dtype)

    def view(h):
        return [1, h, seq, hd], [seq * h * hd, hd, h * hd, 1]

    qd, qs = view(qh)
    kd, ks = view(kvh)
    dkc, dvc = ctx.upload(kc0), ctx.upload(vc0)
    dcos, dsin = ctx.upload(c), ctx.upload(s)
    q_out, k_rep, v_rep = run(ctx, lambda: ctx.qkv_rope_kv_append_repeat(
        (ctx.upload(qp), qd, qs), (ctx.upload(kp), kd, ks), (ctx.upload(vp), kd, ks),
        dcos, dsin, start, dkc, dvc, n_rep))
    q_ref = o.rope(o.contiguous(qp.ravel(), qd, qs), c, s, start)
    k_ref = o.kv_cache_write(kc0, o.rope(o.contiguous(kp.ravel(), kd, ks), c, s, start), start)
    v_ref = o.kv_cache_write(vc0, o.contiguous(vp.ravel(), kd, ks), start)
    total = start + seq
    assert_bitexact(q_out.numpy(), q_ref, "Q")
    assert_bitexact(dkc.numpy(), k_ref, "K cache")
    assert_bitexact(dvc.numpy(), v_ref, "V cache")
    assert_bitexact(k_rep.numpy(), o.repeat_kv(np.ascontiguousarray(k_ref[:, :, :total]), n_rep),
                    "repeated K")
    assert_bitexact(v_rep.numpy(), o.repeat_kv(np.ascontiguousarray(v_ref[:, :, :total]), n_rep),
                    "repeated V")


def test_kv_cache_appends_reference_kat(ctx):
    """src/model/kv_cache.rs:213-258: two one-token f16 appends into a
    [1, 2, 8, 4] cache, then the narrowed [1, 2, 2, 4] prefix made
    contiguous."""
    kat = K["kv_cache_narrow_contiguous"]
    _, heads, max_seq, hd = kat["cache_shape"]
    cache = ctx.upload(np.zeros(kat["cache_shape"], np.float16))
    ctx.begin()
    for pos, vals in enumerate(kat["appends"]):
        key = np.array(vals, np.float16).reshape(kat["append_shape"])
        ctx.kv_cache_write(cache, ctx.upload(key), pos)
    n = kat["narrow_len"]
    got = ctx.contiguous(cache, [1, heads, n, hd], [heads * max_seq * hd, max_seq * hd, hd, 1])
    ctx.finish()
    assert got.numpy().astype(np.float32).ravel().tolist() == kat["expected"]


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("vocab,hidden,tokens", [(49152, 960, 4096), (1000, 576, 1),
                                                 (300, 7, 33), (64, 12, 5)])
def test_embedding_bitexact(ctx, dtype, vocab, hidden, tokens):
    w = norm(("emb",), (vocab, hidden), dtype)
    ids = (synth.uniform(synth.seed_for("ids", vocab, tokens), tokens) * vocab).astype(np.uint32)
    ids[0] = vocab - 1
    dw = ctx.upload(w)
    got = run(ctx, lambda: ctx.embedding(dw, ids)).numpy()
    assert_bitexact(got, o.embedding(w, ids), f"embedding {vocab}x{hidden} [{tokens}]")


def test_embedding_staging_reuse(ctx):
    """Token ids are copied in stream order: several gathers enqueued in one
    batch, with the host array overwritten between calls and growing past
    the staging size, each see their own ids."""
    vocab, hidden = 512, 64
    w = norm(("emb2",), (vocab, hidden), np.float32)
    dw = ctx.upload(w)
    ids = np.zeros(1, np.uint32)
    outs, expected = [], []
    ctx.begin()
    for k, n in enumerate([1, 3, 2000, 5, 9000]):
        ids = ((np.arange(n, dtype=np.uint64) * 7919 + k) % vocab).astype(np.uint32)
        outs.append(ctx.embedding(dw, ids))
        expected.append(w[ids])
        ids[:] = 0  # the library must not read the host array after the call
    ctx.finish()
    for got, ref in zip(outs, expected):
        assert_bitexact(got.numpy(), ref, "embedding batch")


def test_embedding_in_a_graph(ctx):
    """Up to 256 ids travel in the kernel arguments, so such a gather can be
    recorded and replayed; more ids would need a host copy, which a graph
    cannot hold, and are refused while recording."""
    vocab, hidden = 300, 96
    w = norm(("emb3",), (vocab, hidden), np.float16)
    dw = ctx.upload(w)
    ids = np.array([7, 299, 0, 7, 150], np.uint32)
    out = ctx.empty((ids.size, hidden), np.float16)
    ctx.capture_begin()
    try:
        ctx.embedding(dw, ids, out)
    finally:
        graph = ctx.capture_end()
    ids[:] = 1  # the recorded launch keeps the ids it was given
    for _ in range(3):
        ctx.begin()
        ctx.graph_launch(graph)
        ctx.finish()
        assert_bitexact(out.numpy(), w[[7, 299, 0, 7, 150]], "replayed embedding")
    ctx.graph_destroy(graph)
    big = np.zeros(257, np.uint32)
    big_out = ctx.empty((big.size, hidden), np.float16)
    ctx.capture_begin()
    try:
        with pytest.raises(abi.RustLLMError, match="graph"):
            ctx.embedding(dw, big, big_out)
    finally:
        ctx.graph_destroy(ctx.capture_end())


# ------------------------------------------------------- runtime behaviour

def test_one_batch_is_one_submission(ctx):
    """Submission counters (MetalDecodeProfile semantics): ops enqueued
    between begin and finish are one command buffer, one commit, one wait."""
    x = ctx.upload(norm(("prof",), (4, 64), np.float32))
    w = ctx.upload(np.ones(64, np.float32))
    ctx.profile_begin()
    ctx.begin()
    y = ctx.rmsnorm(x, w, 1e-5)
    z = ctx.add(y, x)
    ctx.silu(z)
    ctx.finish()
    prof = ctx.profile_take()
    assert prof["command_buffers"] == 1 and prof["commits"] == 1 and prof["waits"] == 1
    assert prof["kernel_dispatches"] == 3 and prof["compute_encoders"] == 3
    assert prof["buffer_allocations"] == 3
    assert ctx.dispatches("rmsnorm_f32") == 1 and ctx.dispatches("add_f32") == 1
    assert ctx.profile_take() is None


def test_graph_replay_matches_eager(ctx):
    """A recorded batch replayed several times, with eager work and waits in
    between, gives the eager result every time."""
    a = norm(("graph", "a"), (1000, 96), np.float16)
    b = norm(("graph", "b"), (1000, 96), np.float16)
    w = synth.uniform_range(7, (96,), 0.5, 1.5, np.float16)
    da, db, dw = ctx.upload(a), ctx.upload(b), ctx.upload(w)
    s_out, y_out = ctx.empty(a.shape, np.float16), ctx.empty(a.shape, np.float16)
    sm_out = ctx.empty(a.shape, np.float16)
    ctx.capture_begin()
    ctx.add_rmsnorm(da, db, dw, 1e-5, s_out, y_out)
    ctx.softmax(y_out, sm_out)
    graph = ctx.capture_end()
    rs, ry = o.add_rmsnorm(a, b, w, 1e-5)
    for i in range(4):
        ctx.graph_launch(graph)
        ctx.finish()
        assert_bitexact(s_out.numpy(), rs, f"replay {i}")
        check_float(y_out.numpy(), ry, f"replay {i}")
        check_float(sm_out.numpy(), o.softmax(y_out.numpy()), f"replay {i}")
        run(ctx, lambda: ctx.mul(da, db))  # unrelated eager work between replays
    ctx.graph_destroy(graph)


def test_forked_graph_over_two_streams_matches_eager(ctx):
    """Independent ops recorded on two contexts' streams (fork/join by events)
    replay correctly, every time, with eager work in between."""
    aux = abi.Context(0)
    try:
        a = norm(("fork", "a"), (2048, 256), np.float32)
        b = norm(("fork", "b"), (2048, 256), np.float32)
        h = norm(("fork", "h"), (2048, 256), np.float16)
        da, db, dh = ctx.upload(a), ctx.upload(b), ctx.upload(h)
        o1, o2, o3 = (ctx.empty(a.shape, np.float32), ctx.empty(a.shape, np.float32),
                      ctx.empty(a.shape, np.float16))
        fork, join = ctx.event(), ctx.event()
        ctx.capture_begin()
        ctx.record(fork)
        aux.wait(fork)
        ctx.add(da, db, o1)
        aux.swiglu(da, db, o2)
        aux.silu(dh, o3)
        aux.record(join)
        ctx.wait(join)
        graph = ctx.capture_end()
        for i in range(3):
            ctx.graph_launch(graph)
            ctx.finish()
            assert_bitexact(o1.numpy(), o.add(a, b), f"replay {i}")
            check_float(o2.numpy(), o.swiglu(a, b), f"replay {i}")
            check_float(o3.numpy(), o.silu(h), f"replay {i}")
            run(ctx, lambda: ctx.mul(da, db))
        ctx.graph_destroy(graph)
        ctx.destroy_event(fork)
        ctx.destroy_event(join)
    finally:
        aux.close()


def test_kernel_stamped_events_time_one_kernel(ctx):
    a = ctx.upload(norm(("evt",), (1 << 22,), np.float32))
    start, stop = ctx.event(), ctx.event()
    ctx.time_next_kernel(start, stop)
    out = ctx.silu(a)
    ctx.finish()
    us = ctx.elapsed_ms(start, stop) * 1e3
    assert 0.5 < us < 5000
    check_float(out.numpy(), o.silu(a.numpy()), "timed launch")
    ctx.destroy_event(start)
    ctx.destroy_event(stop)


def test_device_validation_matches_cpu(ctx):
    a, b = ctx.upload(np.ones(8, np.float32)), ctx.upload(np.ones(9, np.float32))
    with pytest.raises(abi.RustLLMError) as err:
        ctx.add(a, b, out=ctx.empty((8,), np.float32))
    assert err.value.kind == "InvalidShape"
    assert "equal buffer lengths, got 8 and 9" in str(err.value)


def test_pool_reuses_released_blocks(ctx):
    # A released block is handed out again for the same size class: drain the
    # class first so that the only free block of it is the one released here.
    n = (1 << 20) + 4097
    held = [ctx.empty((n,), np.float32) for _ in range(64)]
    first = ctx.empty((n,), np.float32)
    addr = first.ptr
    first.release()
    second = ctx.empty((n,), np.float32)
    assert second.ptr == addr
    del held


# ------------------------------------------------------ outputs over inputs

def _in_place_cases(ctx, dtype, rows, width):
    """(name, fresh-input factory, op on given buffers) for every op whose
    output may be the very buffer of an input: the element-wise maps, the
    bias add, and the row ops."""
    x = norm(("inplace-x",), (rows, width), dtype)
    y = norm(("inplace-y",), (rows, width), dtype)
    bias = norm(("inplace-b",), (width,), dtype)
    w = synth.uniform_range(synth.seed_for("inplace-w", width), (width,), 0.5, 1.5, dtype)
    s = norm(("inplace-s",), (rows, width), dtype, 0.0, 2.0)
    up = ctx.upload
    masks = [] if rows > width else [
        ("scale/mask", lambda: (up(s),),
         lambda a, out: ctx.scale_mask(a, 0.125, width - rows, out), 0),
        ("scale/mask + softmax", lambda: (up(s),),
         lambda a, out: ctx.attention_softmax(a, 0.125, width - rows, out), 0)]
    return masks + [
        ("add, out = a", lambda: (up(x), up(y)), lambda a, b, out: ctx.add(a, b, out), 0),
        ("add, out = b", lambda: (up(x), up(y)), lambda a, b, out: ctx.add(a, b, out), 1),
        ("mul, out = a", lambda: (up(x), up(y)), lambda a, b, out: ctx.mul(a, b, out), 0),
        ("SwiGLU, out = gate", lambda: (up(x), up(y)), lambda a, b, out: ctx.swiglu(a, b, out), 0),
        ("SwiGLU, out = up", lambda: (up(x), up(y)), lambda a, b, out: ctx.swiglu(a, b, out), 1),
        ("SiLU", lambda: (up(x),), lambda a, out: ctx.silu(a, out), 0),
        ("bias add", lambda: (up(x), up(bias)), lambda a, b, out: ctx.add_broadcast(a, b, out), 0),
        ("RMSNorm", lambda: (up(x), up(w)), lambda a, b, out: ctx.rmsnorm(a, b, 1e-5, out), 0),
        ("softmax", lambda: (up(s),), lambda a, out: ctx.softmax(a, out), 0),
    ]


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("rows,width", [(33, 1001), (16, 4096), (3, 9003), (4096, 1536)])
def test_outputs_over_inputs(ctx, dtype, rows, width):
    """An output passed as the very buffer of one of its inputs (out == a,
    which the ABI accepts for these ops) gives the same bits as a separate
    output: each lane group reads everything it writes before writing it
    (rows held in registers, packs stored by the lane that loaded them).
    Ragged widths, partial last blocks and the streaming softmax (9003 f32
    columns) included."""
    for name, make, op, which in _in_place_cases(ctx, dtype, rows, width):
        ins = make()
        ref = run(ctx, lambda: op(*ins, ctx.empty(ins[which].shape, dtype))).numpy()
        ins = make()
        run(ctx, lambda: op(*ins, ins[which]))
        assert_bitexact(ins[which].numpy(), ref, f"{name} in place, {dtype.__name__} [{rows}, {width}]")


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("shape", [(1, 15, 4096, 64), (2, 3, 7, 6), (1, 2, 33, 128)])
def test_rope_and_add_rmsnorm_over_inputs(ctx, dtype, shape):
    """RoPE written over its input, and add + RMSNorm writing the sum over x
    and the normalised rows over the residual: the same bits as separate
    outputs."""
    c, s = o.rope_table(shape[-1], shape[-2] + 8, 10000.0)
    dc, ds = ctx.upload(c), ctx.upload(s)
    x = norm(("inplace-rope",), shape, dtype)
    ref = run(ctx, lambda: ctx.rope(ctx.upload(x), dc, ds, 3)).numpy()
    d = ctx.upload(x)
    run(ctx, lambda: ctx.rope(d, dc, ds, 3, d))
    assert_bitexact(d.numpy(), ref, f"rope in place {shape}")
    h = shape[-1]
    rows = int(np.prod(shape[:-1]))
    a = norm(("inplace-ar-x",), (rows, h), dtype)
    r = norm(("inplace-ar-r",), (rows, h), dtype)
    wt = ctx.upload(synth.uniform_range(synth.seed_for("inplace-ar-w", h), (h,), 0.5, 1.5, dtype))
    s_ref, y_ref = run(ctx, lambda: ctx.add_rmsnorm(ctx.upload(a), ctx.upload(r), wt, 1e-5))
    s_ref, y_ref = s_ref.numpy(), y_ref.numpy()
    da, dr = ctx.upload(a), ctx.upload(r)
    run(ctx, lambda: ctx.add_rmsnorm(da, dr, wt, 1e-5, sum_out=da, norm_out=dr))
    assert_bitexact(da.numpy(), s_ref, f"add + rmsnorm sum over x {shape}")
    assert_bitexact(dr.numpy(), y_ref, f"add + rmsnorm rows over the residual {shape}")
