"""Buffers whose data pointer is not on the 16-byte grid, against the oracle.

An rl_buffer is a plain (pointer, length) pair, so a caller may pass one
that starts inside a larger allocation.  Every op then leaves its 16-byte
pack paths for the narrower ones (fewer elements a pack, per-element gathers,
the streaming softmax, the row kernels of the GQA matmuls and of the
attention core); these tests run each op on views that start 1 or 3
elements into an allocation and hold them to the bars of the aligned tests:
bit-exact for add, mul, cast, bias add, contiguous, repeat_kv, scale/mask,
RoPE, the KV-cache write and the embedding gather; f32 RMSNorm, softmax,
SiLU and SwiGLU within 1e-5 max relative error (FLT_MIN floor); every f16
output within 2 ulp; the GQA matmuls bit-exact on small integers and the
attention core under its float64 forward-error bound.
"""

import numpy as np
import pytest

from helpers import assert_bitexact, attention_bound, f16_ulp_distance, max_rel_err
from oracle import oracle as o
from rustllm_amd import abi, synth

pytestmark = pytest.mark.gpu

TINY = np.finfo(np.float32).tiny
DT = [np.float32, np.float16]


def view(ctx, array, offset):
    """`array` uploaded `offset` elements into an allocation (a few spare
    elements after it), as an rl_buffer that starts there and owns nothing."""
    a = np.ascontiguousarray(array)
    pad = np.zeros(offset + a.size + 16, dtype=a.dtype)
    pad[offset:offset + a.size] = a.ravel()
    parent = ctx.upload(pad)
    raw = abi.RlBuffer()
    raw.data = parent.ptr + offset * a.itemsize
    raw.len = a.size
    raw.byte_len = a.nbytes
    v = abi.DeviceBuffer(ctx, raw, a.dtype, a.shape)
    v.release = lambda: None  # the parent owns the memory
    v.parent = parent
    return v


def empty_view(ctx, shape, dtype, offset):
    return view(ctx, np.zeros(shape, dtype=dtype), offset)


def run(ctx, fn):
    ctx.begin()
    out = fn()
    ctx.finish()
    return out


def close(got, ref, what):
    if got.dtype == np.float16:
        d = f16_ulp_distance(got, ref)
        assert d <= 2, f"{what}: {d} ulp"
    else:
        fin = np.isfinite(ref)
        assert np.array_equal(np.isfinite(got), fin), f"{what}: non-finite positions differ"
        e = max_rel_err(got[fin], ref[fin], TINY)
        assert e <= 1e-5, f"{what}: max rel err {e:.3g}"


def norm(key, shape, dtype, sigma=1.0):
    return synth.normal(synth.seed_for(*key, *shape, np.dtype(dtype).name), shape, 0.0, sigma,
                        dtype)


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("offset", [1, 3])
@pytest.mark.parametrize("shape", [(7, 33), (64, 1000), (256, 1536)])
def test_elementwise_and_rows_off_the_grid(ctx, dtype, offset, shape):
    rows, width = shape
    x = norm(("off-x",), shape, dtype)
    y = norm(("off-y",), shape, dtype)
    bias = norm(("off-b",), (width,), dtype)
    w = synth.uniform_range(synth.seed_for("off-w", width), (width,), 0.5, 1.5, dtype)
    s = norm(("off-s",), shape, dtype, 2.0)
    tag = f"{np.dtype(dtype).name} {shape} +{offset}"
    v = lambda a: view(ctx, a, offset)  # noqa: E731
    e = lambda: empty_view(ctx, shape, dtype, offset)  # noqa: E731

    assert_bitexact(run(ctx, lambda: ctx.add(v(x), v(y), e())).numpy(), o.add(x, y), f"add {tag}")
    assert_bitexact(run(ctx, lambda: ctx.mul(v(x), v(y), e())).numpy(), o.mul(x, y), f"mul {tag}")
    close(run(ctx, lambda: ctx.silu(v(x), e())).numpy(), o.silu(x), f"silu {tag}")
    close(run(ctx, lambda: ctx.swiglu(v(x), v(y), e())).numpy(), o.swiglu(x, y), f"swiglu {tag}")
    assert_bitexact(run(ctx, lambda: ctx.add_broadcast(v(x), v(bias), e())).numpy(),
                    o.add_broadcast(x, bias), f"bias add {tag}")
    other = np.float16 if dtype == np.float32 else np.float32
    got = run(ctx, lambda: ctx.cast(v(x), other, empty_view(ctx, shape, other, offset))).numpy()
    assert_bitexact(got, o.cast(x, other), f"cast {tag}")
    close(run(ctx, lambda: ctx.rmsnorm(v(x), v(w), 1e-5, e())).numpy(), o.rmsnorm(x, w, 1e-5),
          f"rmsnorm {tag}")
    s_ref, y_ref = o.add_rmsnorm(x, y, w, 1e-5)
    s_got, y_got = run(ctx, lambda: ctx.add_rmsnorm(v(x), v(y), v(w), 1e-5, e(), e()))
    assert_bitexact(s_got.numpy(), s_ref, f"add + rmsnorm sum {tag}")
    close(y_got.numpy(), y_ref, f"add + rmsnorm {tag}")
    close(run(ctx, lambda: ctx.softmax(v(s), e())).numpy(), o.softmax(s), f"softmax {tag}")
    if rows <= width:
        start = width - rows
        assert_bitexact(run(ctx, lambda: ctx.scale_mask(v(s), 0.125, start, e())).numpy(),
                        o.scale_mask(s, 0.125, start), f"scale/mask {tag}")
        close(run(ctx, lambda: ctx.attention_softmax(v(s), 0.125, start, e())).numpy(),
              o.attention_softmax(s, 0.125, start), f"scale/mask + softmax {tag}")


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("offset", [1, 3])
def test_movement_and_rope_off_the_grid(ctx, dtype, offset):
    tag = f"{np.dtype(dtype).name} +{offset}"
    # contiguous of a [1, 9, 40, 64] view of [1, 40, 9, 64] storage
    base = norm(("off-perm",), (1, 40, 9, 64), dtype)
    dims, strides = (1, 9, 40, 64), (40 * 9 * 64, 64, 9 * 64, 1)
    got = run(ctx, lambda: ctx.contiguous(view(ctx, base, offset), dims, strides,
                                          empty_view(ctx, dims, dtype, offset))).numpy()
    assert_bitexact(got, o.contiguous(base.ravel(), dims, strides), f"contiguous {tag}")
    kv = norm(("off-kv",), (1, 3, 40, 64), dtype)
    got = run(ctx, lambda: ctx.repeat_kv(view(ctx, kv, offset), 3,
                                         empty_view(ctx, (1, 9, 40, 64), dtype, offset))).numpy()
    assert_bitexact(got, o.repeat_kv(kv, 3), f"repeat_kv {tag}")
    c, s = o.rope_table(64, 48, 10000.0)
    x = norm(("off-rope",), (1, 5, 40, 64), dtype)
    got = run(ctx, lambda: ctx.rope(view(ctx, x, offset), view(ctx, c, offset),
                                    view(ctx, s, offset), 3,
                                    empty_view(ctx, x.shape, dtype, offset))).numpy()
    assert_bitexact(got, o.rope(x, c, s, 3), f"rope {tag}")
    cache0 = norm(("off-cache",), (1, 3, 64, 64), dtype)
    cache = view(ctx, cache0, offset)
    run(ctx, lambda: ctx.kv_cache_write(cache, view(ctx, kv, offset), 7))
    assert_bitexact(cache.numpy(), o.kv_cache_write(cache0, kv, 7), f"kv cache write {tag}")
    table = norm(("off-emb",), (500, 96), dtype)
    ids = synth.splitmix64(5, 77).astype(np.uint64) % np.uint64(500)
    ids = ids.astype(np.uint32)
    got = run(ctx, lambda: ctx.embedding(view(ctx, table, offset), ids,
                                         empty_view(ctx, (77, 96), dtype, offset))).numpy()
    assert_bitexact(got, o.embedding(table, ids), f"embedding {tag}")


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("offset", [1, 3])
def test_attention_off_the_grid(ctx, dtype, offset):
    """GQA QK^T / PV on small integers (exact in every accumulation order)
    and the fused attention core under its float64 bound, on views off the
    16-byte grid (the row kernels)."""
    rng = np.random.default_rng(11 + offset)
    q = rng.integers(-3, 4, (1, 6, 40, 64)).astype(dtype)
    k = rng.integers(-3, 4, (1, 2, 40, 64)).astype(dtype)
    tag = f"{np.dtype(dtype).name} +{offset}"
    got = run(ctx, lambda: ctx.gqa_qk(view(ctx, q, offset), view(ctx, k, offset),
                                      out=empty_view(ctx, (1, 6, 40, 40), dtype, offset))).numpy()
    assert np.array_equal(got, o.gqa_qk(q, k)), f"gqa qk {tag}"
    p = (o.gqa_qk(q, k) / 64).astype(dtype)
    got = run(ctx, lambda: ctx.gqa_pv(view(ctx, p, offset), view(ctx, k, offset),
                                      out=empty_view(ctx, (1, 6, 40, 64), dtype, offset))).numpy()
    assert np.array_equal(got, o.gqa_pv(p, k)), f"gqa pv {tag}"
    qf = synth.normal(synth.seed_for("off-attn-q", offset), (1, 6, 40, 64)).astype(dtype)
    kf = synth.normal(synth.seed_for("off-attn-k", offset), (1, 2, 40, 64)).astype(dtype)
    vf = synth.normal(synth.seed_for("off-attn-v", offset), (1, 2, 40, 64)).astype(dtype)
    got = run(ctx, lambda: ctx.attention(view(ctx, qf, offset), view(ctx, kf, offset),
                                         view(ctx, vf, offset), 0.125, 0,
                                         out=empty_view(ctx, qf.shape, dtype, offset))).numpy()
    kind = "f16_fused" if dtype == np.float16 else "f32"
    exact, bound = attention_bound(qf, kf, vf, 0.125, 0, 40, kind)
    err = np.abs(got.astype(np.float64) - exact)
    assert np.all(err <= bound), f"attention {tag}: max error {err.max():.3g}"
