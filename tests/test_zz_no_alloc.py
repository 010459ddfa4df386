"""rl_attention_f16_noalloc (the allocation-free attention entry) against
rl_attention_f16 through the C ABI.

Both run the same kernels on the same inputs, so the bar is bit-identical
output; the first call is also held to the float64 forward error bound the
attention tests use.  Two calls in a row share the static scratch, the second
on a smaller decode shape (fewer splits and heads: the first call's partials
are still in the scratch and must not leak into the second); then a prefill
shape (the matrix-core path, which uses no scratch) and the decode call
recorded in a graph and replayed, every replay checked against the eager
result with eager work in between.
"""

import numpy as np
import pytest

from helpers import attention_bound
from rustllm_amd import synth

pytestmark = pytest.mark.gpu

F16 = np.float16


def inputs(tag, b, qh, kvh, ql, cap, hd):
    q = synth.normal(synth.seed_for("noalloc", tag, "q"), (b, qh, ql, hd)).astype(F16)
    k = synth.normal(synth.seed_for("noalloc", tag, "k"), (b, kvh, cap, hd)).astype(F16)
    v = synth.normal(synth.seed_for("noalloc", tag, "v"), (b, kvh, cap, hd)).astype(F16)
    return q, k, v


def both(ctx, q, k, v, start, kv_len):
    dq, dk, dv = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    ctx.begin()
    ref = ctx.attention(dq, dk, dv, 0.125, start, kv_len)
    got = ctx.attention_noalloc(dq, dk, dv, 0.125, start, kv_len)
    ctx.finish()
    return got.numpy(), ref.numpy()


def test_noalloc_decode_matches_the_pooled_entry_twice(ctx):
    # 1: one token of 15 heads over a full 4096-row cache (16 key splits)
    q, k, v = inputs("a", 1, 15, 5, 1, 4096, 64)
    got, ref = both(ctx, q, k, v, 4095, 4096)
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))
    exact, bound = attention_bound(q, k, v, 0.125, 4095, 4096, "f16_fused")
    assert np.all(np.abs(got.astype(np.float64) - exact) <= bound)
    # 2: smaller -- 6 heads over 1000 of 1100 cache rows (4 splits)
    q, k, v = inputs("b", 1, 6, 2, 1, 1100, 64)
    got, ref = both(ctx, q, k, v, 999, 1000)
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))
    exact, bound = attention_bound(q, k, v, 0.125, 999, 1000, "f16_fused")
    assert np.all(np.abs(got.astype(np.float64) - exact) <= bound)


def test_noalloc_prefill_matches_the_pooled_entry(ctx):
    q, k, v = inputs("c", 1, 6, 2, 130, 300, 64)
    got, ref = both(ctx, q, k, v, 170, 300)
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))


def test_noalloc_decode_recorded_in_a_graph(ctx):
    q, k, v = inputs("d", 2, 8, 2, 2, 1536, 128)  # batch 2, two query rows per head
    dq, dk, dv = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    ctx.begin()
    eager = ctx.attention(dq, dk, dv, 0.125, 1534, 1536).numpy()
    ctx.finish()
    out = ctx.empty(q.shape, F16)
    ctx.capture_begin()
    try:
        ctx.attention_noalloc(dq, dk, dv, 0.125, 1534, 1536, out)
    finally:
        graph = ctx.capture_end()
    try:
        for i in range(3):
            ctx.begin()  # eager work between the replays
            ctx.attention(dq, dk, dv, 0.125, 1534, 1536)
            ctx.attention_noalloc(ctx.upload(q[:, :, :1].copy()), dk, dv, 0.125, 1535, 1536)
            ctx.finish()
            ctx.begin()
            ctx.graph_launch(graph)
            ctx.finish()
            assert np.array_equal(out.numpy().view(np.uint16), eager.view(np.uint16)), i
    finally:
        ctx.graph_destroy(graph)
