"""The fused attention core (rl_attention_*) on the GPU against float64.

SelfAttention::attention_core_encode (nn/attention.rs:216-247) is QK^T,
scale/mask, softmax and PV; the fused pass keeps scores and probabilities in
f32, so it is compared with float64 attention under the forward error bound
of its own roundings (helpers.attention_bound, "f32" / "f16_fused"), and the
reference's four calls (the oracle) are held to the bound of theirs.  Shapes
cover every kernel (the f16 and f32 matrix-core kernels for head sizes
32..128 in steps of 32 in their three workgroup shapes, the split-key decode
kernel, the row kernel for other head sizes), grouped and plain heads,
batches, ragged query/key counts, a start offset (chunked prefill and decode)
and KV caches whose rows past kv_len hold NaN (never read).
"""

import ctypes

import numpy as np
import pytest

from helpers import attention_bound, attention_exact, kats
from oracle import oracle as o
from rustllm_amd import abi, synth

pytestmark = pytest.mark.gpu

K = kats()


def cache(seed, batch, heads, capacity, head_dim, kv_len, dtype):
    kv = synth.normal(seed, (batch, heads, capacity, head_dim)).astype(dtype)
    kv[:, :, kv_len:] = np.nan
    return kv


def run_attention(ctx, q, k, v, scale, start, kv_len):
    dq, dk, dv = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    ctx.begin()
    out = ctx.attention(dq, dk, dv, scale, start, kv_len)
    ctx.finish()
    return out.numpy()


def check(got, q, k, v, scale, start, kv_len, what):
    kind = "f16_fused" if got.dtype == np.float16 else "f32"
    exact, bound = attention_bound(q, k, v, scale, start, kv_len, kind)
    err = np.abs(got.astype(np.float64) - exact)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    worst = np.unravel_index(np.argmax(err / bound), err.shape)
    assert np.all(err <= bound), (f"{what}: error {err[worst]:.3g} > bound {bound[worst]:.3g} "
                                  f"at {worst}")
    return float(err.max())


# batch, q_heads, kv_heads, q_len, kv_len, capacity, head_dim, start
SHAPES = [
    (1, 6, 2, 5, 7, 9, 64, 2),          # grouped, tiny, cache with spare rows
    (1, 15, 5, 130, 130, 160, 64, 0),   # SmolLM2 heads, two ragged query tiles
    (2, 4, 4, 100, 357, 400, 64, 257),  # batch 2, plain heads, chunked prefill
    (1, 3, 1, 257, 257, 257, 32, 0),    # three query tiles (paired 0/2, 1 alone)
    (1, 2, 1, 64, 64, 64, 96, 0),
    (1, 2, 2, 200, 300, 300, 128, 100),
    (1, 8, 2, 256, 1500, 1536, 128, 1244),  # many key blocks per workgroup, D 128
    (1, 6, 3, 384, 2000, 2048, 32, 1616),   # many key blocks, D 32, ragged last block
    (1, 9, 3, 2048, 2048, 2048, 64, 0),     # 9 heads x 2048: 32-query tiles, 2 key shares
    (1, 6, 2, 1, 2048, 4096, 64, 2047),  # decode step from a half-full cache
    (1, 2, 1, 33, 40, 40, 48, 7),        # head size off the matrix-core path
    (1, 2, 2, 17, 17, 20, 80, 0),
    (1, 2, 1, 9, 300, 300, 256, 291),
    # f16: too few 128-query tile pairs, the key steps split over workgroups
    # (partials merged by a second kernel)
    (1, 15, 5, 512, 4096, 4096, 64, 3584),   # 8 key chunks: prefill after cached keys
    (1, 48, 8, 512, 2048, 2048, 128, 1536),  # 96 tile pairs, D 128: 2 key chunks
    (1, 6, 2, 256, 4096, 4096, 96, 3840),    # D 96 (register-staged blocks), 8 chunks
    (1, 4, 2, 300, 5000, 5000, 32, 4700),    # D 32, ragged query tile and key count
    (2, 4, 4, 200, 4100, 4160, 64, 3900),    # batch 2, cache rows past kv_len hold NaN
]

# Few query rows per KV head over long key ranges: the split-key path
# (rows per KV head 3..32, head sizes 64..256, f32 and f16).
DECODE_SHAPES = [
    (1, 15, 5, 1, 4096, 4096, 64, 4095),   # SmolLM2 decode at a full context
    (2, 6, 2, 2, 1000, 1024, 64, 998),     # two new tokens, batch 2, 6 rows per KV head
    (1, 8, 2, 4, 700, 800, 128, 696),      # 16 rows per KV head, D 128
    (1, 4, 4, 1, 3000, 3000, 256, 2999),   # plain heads, D 256
    (1, 32, 4, 4, 600, 600, 64, 596),      # 32 rows per KV head
    (1, 3, 1, 1, 513, 520, 96, 512),       # just past the split threshold, D 96
    (1, 15, 5, 1, 4093, 4096, 64, 4092),   # ragged last wave (4093 keys)
    (1, 8, 8, 1, 1500, 1536, 128, 1400),   # one row per KV head, keys past the causal limit
    (1, 12, 3, 3, 2100, 2100, 64, 2097),   # 12 rows per KV head, three new tokens
]


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
@pytest.mark.parametrize("shape", SHAPES)
def test_attention_within_float64_bound(ctx, dtype, shape):
    b, qh, kvh, ql, kl, cap, hd, start = shape
    q = synth.normal(synth.seed_for("attn-q", *shape), (b, qh, ql, hd)).astype(dtype)
    k = cache(synth.seed_for("attn-k", *shape), b, kvh, cap, hd, kl, dtype)
    v = cache(synth.seed_for("attn-v", *shape), b, kvh, cap, hd, kl, dtype)
    scale = 1.0 / np.sqrt(hd)
    got = run_attention(ctx, q, k, v, scale, start, kl)
    check(got, q, k, v, scale, start, kl, f"attention {np.dtype(dtype).name} {shape}")


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
@pytest.mark.parametrize("shape", DECODE_SHAPES)
def test_attention_decode_within_float64_bound(ctx, dtype, shape):
    test_attention_within_float64_bound(ctx, dtype, shape)


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_attention_core_reference_kat(ctx, dtype):
    """nn/attention.rs:590-668 (fused core == op-by-op calls within 1e-5):
    (2, 2) and (3, 1) heads, D 4, 3 new positions after 2 cached."""
    kat = K["attention_core"]
    d, sl, start = kat["head_dim"], kat["seq_len"], kat["start_pos"]
    for case in kat["cases"]:
        qh, kvh = case["heads"]
        q = (np.arange(qh * sl * d) % 5 - 2).astype(dtype).reshape(1, qh, sl, d)
        kv = (np.arange(kvh * (start + sl) * d) % 3 - 1).astype(dtype).reshape(1, kvh, start + sl, d)
        got = run_attention(ctx, q, kv, kv, 1.0 / np.sqrt(d), start, start + sl)
        expected = np.array(case["expected"]).reshape(got.shape)
        tol = kat["tol"] if dtype == np.float32 else 2.0 ** -10  # f16: the output's rounding
        assert np.max(np.abs(got.astype(np.float64) - expected)) < tol, case["heads"]


def test_attention_f16_is_closer_than_the_reference_composition(ctx):
    """Both within their bounds; the fused pass (no f16 scores in between) is
    the more accurate of the two on a SmolLM2-shaped block."""
    shape = (1, 15, 5, 256, 256, 256, 64, 0)
    b, qh, kvh, ql, kl, cap, hd, start = shape
    q = synth.normal(101, (b, qh, ql, hd)).astype(np.float16)
    k = synth.normal(102, (b, kvh, cap, hd)).astype(np.float16)
    v = synth.normal(103, (b, kvh, cap, hd)).astype(np.float16)
    got = run_attention(ctx, q, k, v, 0.125, start, kl)
    fused_err = check(got, q, k, v, 0.125, start, kl, "fused")
    ref = o.attention(q, k, v, 0.125, start)
    exact, bound = attention_bound(q, k, v, 0.125, start, kl, "f16_reference")
    ref_err = np.abs(ref.astype(np.float64) - exact)
    assert np.all(ref_err <= bound)
    assert fused_err <= float(ref_err.max())


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_attention_smollm_layer(ctx, dtype):
    """SmolLM2-360M layer at 4096 tokens: Q [1, 15, 4096, 64], K/V
    [1, 5, 4096, 64], causal, scale 1/8 (f16, and f32 for the f32 matrix-core
    kernel).  Every output is finite and sampled query rows of every head
    (first, last, tile edges, random) are within the float64 bound."""
    q = synth.normal(201, (1, 15, 4096, 64)).astype(dtype)
    k = synth.normal(202, (1, 5, 4096, 64)).astype(dtype)
    v = synth.normal(203, (1, 5, 4096, 64)).astype(dtype)
    kind = "f16_fused" if dtype == np.float16 else "f32"
    got = run_attention(ctx, q, k, v, 0.125, 0, 4096)
    assert np.isfinite(got).all()
    rows = sorted({0, 1, 31, 32, 127, 128, 2047, 2048, 4094, 4095} |
                  set(np.random.default_rng(204).integers(0, 4096, 12).tolist()))
    for r in rows:
        exact, bound = attention_bound(q[:, :, r:r + 1], k, v, 0.125, r, 4096, kind)
        err = np.abs(got[:, :, r:r + 1].astype(np.float64) - exact)
        assert np.all(err <= bound), f"row {r}: max error {err.max():.3g}"
    # row 0 attends to key 0 only: its output is V's first row of its KV head
    assert np.array_equal(got[0, :, 0], np.repeat(v[0, :, 0], 3, axis=0))


# ------------------------------------------------- the reference's GQA matmuls

U32 = 2.0 ** -24
GQA_SHAPES = [  # batch, q_heads, kv_heads, q_len, kv_len, capacity, head_dim
    (1, 15, 5, 130, 300, 320, 64),   # matrix-core path, ragged tiles, cache with spare rows
    (2, 4, 4, 33, 64, 64, 128),      # plain heads, batch 2
    (1, 6, 2, 7, 45, 50, 32),        # key count not a multiple of 8 (element stores)
    (1, 3, 1, 17, 200, 200, 96),
    (1, 8, 2, 300, 1000, 1024, 128),  # many key tiles and PV steps
    (1, 2, 1, 9, 70, 80, 48),        # row kernels
    (1, 15, 5, 200, 1001, 1024, 64),  # odd key count: rows off the 16-byte grid, 8 key tiles
    (2, 4, 2, 129, 259, 264, 128),    # batch 2, key count 3 mod 8, ragged query tiles
    (1, 6, 3, 33, 130, 136, 32),      # key count 2 mod 8: a last tile of 2 keys
    (1, 15, 5, 300, 1024, 1024, 64),  # rows on the line grid: PV walks 8 key steps from a
    (2, 6, 3, 129, 640, 704, 128),    # per-workgroup start (5 steps here), batch 2
]


def gqa_exact(q, k, kv_len):
    from helpers import gqa_expand
    ke = gqa_expand(k, q.shape[1], kv_len)
    q64 = q.astype(np.float64)
    return (np.matmul(q64, np.swapaxes(ke, -1, -2)),
            np.matmul(np.abs(q64), np.swapaxes(np.abs(ke), -1, -2)))


def ulp16(x):
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -14)))
    return 2.0 ** (e - 10)


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
@pytest.mark.parametrize("shape", GQA_SHAPES)
def test_gqa_qk_within_float64_bound(ctx, dtype, shape):
    """gqa_matmul.metal:7-322: f32 sums of the products (any order stays
    within D u sum|q k| of the exact dot), the f16 score rounded once."""
    b, qh, kvh, ql, kl, cap, hd = shape
    q = synth.normal(synth.seed_for("gqa-q", *shape), (b, qh, ql, hd)).astype(dtype)
    k = cache(synth.seed_for("gqa-k", *shape), b, kvh, cap, hd, kl, dtype)
    ctx.begin()
    got = ctx.gqa_qk(ctx.upload(q), ctx.upload(k), kl)
    ctx.finish()
    got = got.numpy().astype(np.float64)
    exact, dot_abs = gqa_exact(q, k, kl)
    bound = hd * U32 * dot_abs + (ulp16(exact) * 0.5001 if dtype == np.float16 else 0.0) + 1e-30
    assert np.all(np.abs(got - exact) <= bound)


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
@pytest.mark.parametrize("shape", GQA_SHAPES)
def test_gqa_pv_within_float64_bound(ctx, dtype, shape):
    """gqa_matmul.metal:323-629: sum over kv_len keys of p v in f32."""
    from helpers import gqa_expand
    b, qh, kvh, ql, kl, cap, hd = shape
    p = synth.uniform_range(synth.seed_for("gqa-p", *shape), (b, qh, ql, kl), 0.0, 1.0, dtype)
    v = cache(synth.seed_for("gqa-v", *shape), b, kvh, cap, hd, kl, dtype)
    ctx.begin()
    got = ctx.gqa_pv(ctx.upload(p), ctx.upload(v))
    ctx.finish()
    got = got.numpy().astype(np.float64)
    ve = gqa_expand(v, qh, kl)
    exact = np.matmul(p.astype(np.float64), ve)
    weight = np.matmul(p.astype(np.float64), np.abs(ve))
    bound = kl * U32 * weight + (ulp16(exact) * 0.5001 if dtype == np.float16 else 0.0) + 1e-30
    assert np.all(np.abs(got - exact) <= bound)


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_gqa_small_integers_match_the_oracle_bit_for_bit(ctx, dtype):
    """Small-integer operands make every sum exact: the library (matrix cores
    or row kernels) and the oracle agree exactly -- also where the key count
    puts the score rows off the 16-byte grid (every element in its place)."""
    for hd, ql, kl in ((64, 40, 72), (48, 40, 72), (64, 130, 301), (128, 70, 1003), (32, 5, 9),
                       (64, 300, 1024), (128, 130, 384)):  # line-grid rows, small grids: key order
        q = (np.arange(1 * 6 * ql * hd) % 7 - 3).reshape(1, 6, ql, hd).astype(dtype)
        k = (np.arange(1 * 2 * kl * hd) % 5 - 2).reshape(1, 2, kl, hd).astype(dtype)
        ctx.begin()
        s = ctx.gqa_qk(ctx.upload(q), ctx.upload(k))
        pv = ctx.gqa_pv(ctx.upload((o.gqa_qk(q, k) / 64).astype(dtype)), ctx.upload(k))
        ctx.finish()
        assert np.array_equal(s.numpy(), o.gqa_qk(q, k))
        assert np.array_equal(pv.numpy(), o.gqa_pv((o.gqa_qk(q, k) / 64).astype(dtype), k))


@pytest.mark.parametrize("kl,walk", [(2048, "rotated"), (1536, "key order, streamed")])
def test_gqa_pv_line_grid_walks_bit_for_bit(ctx, kl, walk):
    """P V f16 over probability rows on the 128-byte line grid at the sizes
    where the matrix-core kernel changes its walk: rows 4 KB apart with 480
    workgroups (16 heads x 30 query tiles, about two a CU) start each
    workgroup's key walk at its own step; 3 KB rows over 189 MB of
    probabilities walk in key order with streamed loads.  Small-integer
    operands make every sum exact, so the result is the float64 product
    rounded once to f16, element for element (the oracle's own arithmetic
    at this size would take minutes on the host)."""
    qh, kvh, ql, hd = 16, 4, 3840, 64
    p = ((np.arange(qh * ql * kl, dtype=np.int64) % 7 - 3) / 64).astype(np.float16)
    p = p.reshape(1, qh, ql, kl)
    v = (np.arange(kvh * kl * hd) % 5 - 2).reshape(1, kvh, kl, hd).astype(np.float16)
    ctx.begin()
    got = ctx.gqa_pv(ctx.upload(p), ctx.upload(v)).numpy()
    ctx.finish()
    for h in range(qh):
        want = (p[0, h].astype(np.float64) @ v[0, h // (qh // kvh)].astype(np.float64))
        assert np.array_equal(got[0, h], want.astype(np.float16)), f"{walk}: head {h}"


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
@pytest.mark.parametrize("hd,ql,kl", [(64, 2000, 1000), (128, 2048, 512), (32, 2048, 1032),
                                      (64, 200, 4093)])
def test_gqa_qk_large_grids_bit_for_bit(ctx, hd, ql, kl, dtype):
    """Grids of thousands of score tiles (16 heads x 2-16 query tiles x 4-32
    key tiles): small-integer operands make every sum exact, so the library
    and the oracle agree exactly -- with a partial last query tile, key counts
    off the 128-key tile (1000, 1032, 4093) and off the 128-byte line (1000:
    rows stored plainly; 4093: rows off the 16-byte grid, unaligned stores),
    and whole lines (512); in f32 the 4093-key rows are off the 16-byte grid
    too (unaligned 16-byte stores)."""
    q = (np.arange(1 * 16 * ql * hd) % 7 - 3).reshape(1, 16, ql, hd).astype(dtype)
    k = (np.arange(1 * 4 * kl * hd) % 5 - 2).reshape(1, 4, kl, hd).astype(dtype)
    ctx.begin()
    s = ctx.gqa_qk(ctx.upload(q), ctx.upload(k))
    ctx.finish()
    assert np.array_equal(s.numpy(), o.gqa_qk(q, k))


@pytest.mark.parametrize("hd", [32, 64, 128])
def test_gqa_qk_every_key_residue_bit_for_bit(ctx, hd):
    """f16 score rows of every key count residue mod 8 (a row then starts r
    scores past the 16-byte grid for r = row kv_len mod 8): each row segment
    goes out in the buffer's aligned chunks, the chunks it shares with the
    neighbouring segment element by element -- every score in its place and
    no neighbour overwritten, at partial query and key tiles."""
    for kl in (1024, 1025, 1026, 1027, 1028, 1029, 1030, 1031, 129, 250, 7):
        ql = 97 if kl > 200 else 40
        q = (np.arange(1 * 6 * ql * hd) % 7 - 3).reshape(1, 6, ql, hd).astype(np.float16)
        k = (np.arange(1 * 2 * kl * hd) % 5 - 2).reshape(1, 2, kl, hd).astype(np.float16)
        ctx.begin()
        s = ctx.gqa_qk(ctx.upload(q), ctx.upload(k))
        ctx.finish()
        assert np.array_equal(s.numpy(), o.gqa_qk(q, k)), f"hd {hd}, {kl} keys"


def test_unfused_chain_f16_within_the_reference_bound(ctx):
    """The reference's four calls on the library (gqa_qk, scale/mask +
    softmax, gqa_pv) with the reference's rounding points stay within the
    forward bound of those roundings, like the oracle's composition."""
    from helpers import attention_bound
    b, qh, kvh, ql, kl, hd, start = 1, 15, 5, 200, 200, 64, 0
    q = synth.normal(301, (b, qh, ql, hd)).astype(np.float16)
    k = synth.normal(302, (b, kvh, kl, hd)).astype(np.float16)
    v = synth.normal(303, (b, kvh, kl, hd)).astype(np.float16)
    ctx.begin()
    s = ctx.gqa_qk(ctx.upload(q), ctx.upload(k))
    p = ctx.attention_softmax(s, 0.125, start)
    got = ctx.gqa_pv(p, ctx.upload(v))
    ctx.finish()
    exact, bound = attention_bound(q, k, v, 0.125, start, kl, "f16_reference")
    assert np.all(np.abs(got.numpy().astype(np.float64) - exact) <= bound)


def test_gqa_qk_smollm_layer_f16_sampled_rows(ctx):
    """Full SmolLM2 shape (Q [1, 15, 4096, 64] x K [1, 5, 4096, 64]^T, a
    503 MB score tensor): sampled rows of every head against float64."""
    q = synth.normal(311, (1, 15, 4096, 64)).astype(np.float16)
    k = synth.normal(312, (1, 5, 4096, 64)).astype(np.float16)
    ctx.begin()
    s = ctx.gqa_qk(ctx.upload(q), ctx.upload(k))
    ctx.finish()
    got = s.numpy()
    for r in (0, 127, 128, 2049, 4095):
        exact, dot_abs = gqa_exact(q[:, :, r:r + 1], k, 4096)
        bound = 64 * U32 * dot_abs + ulp16(exact) * 0.5001
        assert np.all(np.abs(got[:, :, r:r + 1].astype(np.float64) - exact) <= bound), r


# ------------------------------------------------- recorded in a graph

@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_attention_in_a_graph_matches_eager(ctx, dtype):
    """A prefill and a decode step recorded in one graph, replayed several
    times with eager work in between: the prefill replays give the eager
    result bit for bit (same kernel); the decode step, which takes the
    matrix-core kernel while recording (the split-key kernel's partials live
    in a pool block that a replay could not own), stays within the float64
    bound on every replay."""
    pre = (1, 6, 2, 300, 300, 320, 64, 0)
    dec = (1, 15, 5, 1, 1024, 1024, 64, 1023)
    bufs = []
    for shape in (pre, dec):
        b, qh, kvh, ql, kl, cap, hd, start = shape
        q = synth.normal(synth.seed_for("graph-q", *shape), (b, qh, ql, hd)).astype(dtype)
        k = cache(synth.seed_for("graph-k", *shape), b, kvh, cap, hd, kl, dtype)
        v = cache(synth.seed_for("graph-v", *shape), b, kvh, cap, hd, kl, dtype)
        bufs.append((shape, q, k, v, ctx.upload(q), ctx.upload(k), ctx.upload(v),
                     ctx.empty(q.shape, dtype)))
    eager = []
    for shape, q, k, v, dq, dk, dv, out in bufs:
        ctx.begin()
        ctx.attention(dq, dk, dv, 0.125, shape[7], shape[4], out)
        ctx.finish()
        eager.append(out.numpy().copy())
    ctx.capture_begin()
    try:
        for shape, q, k, v, dq, dk, dv, out in bufs:
            ctx.attention(dq, dk, dv, 0.125, shape[7], shape[4], out)
    finally:
        graph = ctx.capture_end()
    for i in range(3):
        for _, _, _, _, _, _, _, out in bufs:  # a replay must write every element
            nan = ctx.upload(np.full(out.shape, np.nan, dtype))
            abi.check(ctx.lib.rl_buffer_copy(ctx.handle, ctypes.byref(nan.raw),
                                             ctypes.byref(out.raw), out.byte_len))
        ctx.graph_launch(graph)
        ctx.finish()
        (shape, q, k, v, *_, out_pre), (dshape, dq_, dk_, dv_, *_, out_dec) = bufs
        assert np.array_equal(out_pre.numpy(), eager[0]), f"prefill replay {i}"
        check(out_dec.numpy(), dq_, dk_, dv_, 0.125, dshape[7], dshape[4], f"decode replay {i}")
        ctx.begin()
        ctx.attention(bufs[1][4], bufs[1][5], bufs[1][6], 0.125, dshape[7], dshape[4])  # eager work
        ctx.finish()
    ctx.graph_destroy(graph)
