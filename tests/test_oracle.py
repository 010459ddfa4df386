"""Pins the CPU oracle before it is trusted as the checker.

Each oracle function is checked against something that does not restate its
own code: the reference's known-answer vectors (tests/golden), numpy's IEEE
float16/float32 arithmetic, float64 closed forms, complex multiplication for
RoPE, numpy stride tricks for the gathers, and algebraic invariants.  The
planted-mistake tests at the end show that these checks catch plausible bugs.
"""

import numpy as np
import pytest

from helpers import (U32, assert_bitexact, attention_bound, f16_ulp_distance, floats, gqa_expand,
                     kats, max_rel_err, ulp16)
from oracle import oracle as o
from rustllm_amd import synth

K = kats()


def f16(values):
    return np.asarray(values, dtype=np.float32).astype(np.float16)


# ------------------------------------------------------------ f16 <-> f32

def test_f16_to_f32_exhaustive_matches_numpy():
    all_bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    h = all_bits.view(np.float16)
    assert_bitexact(o.f16_to_f32(h), h.astype(np.float32), "f16->f32")


def _f32_rounding_probe():
    """Every exponent/sign/top-mantissa pattern with the low 13 bits set to
    the values that decide rounding (below, at and above the halfway point,
    both parities), plus all f32 specials."""
    high = np.arange(1 << 19, dtype=np.uint32) << np.uint32(13)
    lows = np.array([0, 1, 0x0FFF, 0x1000, 0x1001, 0x1FFF], dtype=np.uint32)
    pats = (high[:, None] | lows[None, :]).ravel()
    return pats.view(np.float32)


def test_f32_to_f16_rounding_probe_matches_numpy():
    x = _f32_rounding_probe()
    with np.errstate(over="ignore", invalid="ignore"):
        ref = x.astype(np.float16)
    got = o.f32_to_f16(x)
    assert_bitexact(got, ref, "f32->f16 (RNE, subnormals, overflow)")


def test_f32_to_f16_random_matches_numpy():
    u = synth.splitmix64(7, 2_000_000).astype(np.uint64)
    x = (u & np.uint64(0xFFFFFFFF)).astype(np.uint32).view(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        ref = x.astype(np.float16)
    assert_bitexact(o.f32_to_f16(x), ref, "f32->f16 random")


def test_f16_boundaries():
    assert o.f32_to_f16_bits(65504.0) == 0x7BFF
    assert o.f32_to_f16_bits(65519.99) == 0x7BFF  # below the halfway point to 65536
    assert o.f32_to_f16_bits(65520.0) == 0x7C00  # ties-to-even rounds up to inf
    assert o.f32_to_f16_bits(2.0 ** -24) == 0x0001
    assert o.f32_to_f16_bits(2.0 ** -25) == 0x0000  # tie to even (zero)
    assert o.f32_to_f16_bits(1.5 * 2.0 ** -25) == 0x0001
    assert o.f32_to_f16_bits(-0.0) == 0x8000
    assert o.f32_to_f16_bits(float("-inf")) == 0xFC00
    assert o.f16_bits_to_f32(0x3C00) == 1.0


# ------------------------------------------------------------ element-wise

def _inputs(n=100_003, dtype=np.float32, seed=1, sigma=3.0):
    a = synth.normal(synth.seed_for("a", n, seed), (n,), 0.0, sigma, dtype)
    b = synth.normal(synth.seed_for("b", n, seed), (n,), 0.0, sigma, dtype)
    return a, b


def test_add_mul_f32_match_numpy_ieee():
    a, b = _inputs()
    assert_bitexact(o.add(a, b), a + b, "add_f32")
    assert_bitexact(o.mul(a, b), a * b, "mul_f32")


def test_add_mul_f16_match_numpy_float16():
    # numpy's float16 arithmetic widens to float32, operates and rounds back.
    a, b = _inputs(dtype=np.float16)
    assert_bitexact(o.add(a, b), a + b, "add_f16")
    assert_bitexact(o.mul(a, b), a * b, "mul_f16")


def test_add_f16_kat():
    kat = K["add_f16"]
    got = o.add(f16(kat["left"]), f16(kat["right"]))
    assert got.astype(np.float32).tolist() == kat["expected"]


def test_chained_f16_kats():
    kat = K["chained_add_f16"]
    got = o.add(o.add(f16(kat["a"]), f16(kat["b"])), f16(kat["c"])).astype(np.float32)
    assert np.all(np.abs(got - np.array(kat["expected"])) < kat["tol"])
    kat = K["add_then_mul_f16"]
    got = o.mul(o.add(f16(kat["a"]), f16(kat["b"])), f16(kat["c"])).astype(np.float32)
    assert np.all(np.abs(got - np.array(kat["expected"])) < kat["tol"])
    kat = K["silu_then_mul_f16"]
    got = o.mul(o.silu(f16(kat["gate"])), f16(kat["up"])).astype(np.float32)
    assert np.all(np.abs(got - np.array(kat["expected"])) < kat["tol"])


def test_silu_against_float64_closed_form():
    x = synth.normal(3, (200_000,), 0.0, 6.0)
    exact = x.astype(np.float64) / (1.0 + np.exp(-x.astype(np.float64)))
    assert max_rel_err(o.silu(x), exact, np.finfo(np.float32).tiny) < 2e-6
    # f16: one rounding of a float computation, so within 1 ulp of the exact value.
    xh = x.astype(np.float16)
    exact_h = (xh.astype(np.float64) / (1.0 + np.exp(-xh.astype(np.float64)))).astype(np.float16)
    assert f16_ulp_distance(o.silu(xh), exact_h) <= 1


def test_silu_saturation():
    x = np.array([-100.0, -89.0, 0.0, 89.0, 100.0], dtype=np.float32)
    got = o.silu(x)
    assert got[0] == 0.0 and got[2] == 0.0  # exp(100) overflows: x * 0
    assert got[3] == 89.0 and got[4] == 100.0


def test_swiglu_is_silu_times_up():
    g, u = _inputs(dtype=np.float32, sigma=2.0)
    # f32 SwiGLU is the silu_f32 -> mul_f32 composition, bit for bit.
    assert_bitexact(o.swiglu(g, u), o.mul(o.silu(g), u), "swiglu_f32")
    gh, uh = g.astype(np.float16), u.astype(np.float16)
    exact = (gh.astype(np.float64) / (1.0 + np.exp(-gh.astype(np.float64))) *
             uh.astype(np.float64)).astype(np.float16)
    assert f16_ulp_distance(o.swiglu(gh, uh), exact) <= 1
    # one rounding (fused) differs from the two-rounding path on some inputs
    two = o.mul(o.silu(gh), uh)
    assert f16_ulp_distance(o.swiglu(gh, uh), two) <= 2


def test_cast_matches_numpy():
    x = synth.normal(5, (100_000,), 0.0, 1000.0)
    assert_bitexact(o.cast(x, np.float16), x.astype(np.float16), "cast f32->f16")
    h = x.astype(np.float16)
    assert_bitexact(o.cast(h, np.float32), h.astype(np.float32), "cast f16->f32")


def test_add_broadcast_matches_numpy():
    x = synth.normal(9, (37, 48))
    bias = synth.normal(10, (48,))
    assert_bitexact(o.add_broadcast(x, bias), x + bias[None, :], "bias f32")
    xh, bh = x.astype(np.float16), bias.astype(np.float16)
    assert_bitexact(o.add_broadcast(xh, bh), xh + bh[None, :], "bias f16")


# ------------------------------------------------------------ data movement

def test_contiguous_matches_numpy_strides():
    base = np.arange(1 * 7 * 3 * 8, dtype=np.float32)
    view = base.reshape(1, 7, 3, 8).transpose(0, 2, 1, 3)  # permute [0, 2, 1, 3]
    strides = [s // 4 for s in view.strides]
    assert_bitexact(o.contiguous(base, view.shape, strides), np.ascontiguousarray(view))
    # stride-0 broadcast of a row
    bias = np.arange(5, dtype=np.float16)
    got = o.contiguous(bias, [4, 5], [0, 1])
    assert_bitexact(got, np.broadcast_to(bias, (4, 5)).copy())
    # transposed last dims (inner stride != 1)
    m = np.arange(12, dtype=np.float32)
    assert_bitexact(o.contiguous(m, [4, 3], [1, 4]), m.reshape(3, 4).T.copy())


def test_contiguous_kv_cache_narrow_kat():
    kat = K["kv_cache_narrow_contiguous"]
    _, heads, max_seq, d = kat["cache_shape"]
    cache = np.zeros(kat["cache_shape"], dtype=np.float16)
    for pos, vals in enumerate(kat["appends"]):
        cache = o.kv_cache_write(cache, f16(vals).reshape(kat["append_shape"]), pos)
    # narrow(2, 0, len) keeps the parent strides (tensor.rs:283-306)
    n = kat["narrow_len"]
    strides = [heads * max_seq * d, max_seq * d, d, 1]
    got = o.contiguous(cache.ravel(), [1, heads, n, d], strides)
    assert got.astype(np.float32).ravel().tolist() == kat["expected"]


def test_repeat_kv_kats_and_numpy():
    for name in ("repeat_kv_r3", "repeat_kv_r1"):
        kat = K[name]
        x = np.array(kat["input"], dtype=np.float32).reshape(kat["shape"])
        for dt in kat["dtypes"]:
            xin = x.astype(np.float16 if dt == "f16" else np.float32)
            got = o.repeat_kv(xin, kat["repeats"])
            assert list(got.shape) == kat["expected_shape"]
            assert got.astype(np.float32).ravel().tolist() == kat["expected"]
    x = synth.normal(11, (2, 3, 5, 8), dtype=np.float16)
    assert_bitexact(o.repeat_kv(x, 4), np.repeat(x, 4, axis=1))


def test_embedding_and_kv_write_match_numpy():
    w = synth.normal(12, (50, 16))
    ids = np.array([3, 0, 49, 3, 7], dtype=np.uint32)
    assert_bitexact(o.embedding(w, ids), w[ids])
    cache = synth.normal(13, (1, 3, 10, 8), dtype=np.float16)
    src = synth.normal(14, (1, 3, 4, 8), dtype=np.float16)
    ref = cache.copy()
    ref[:, :, 5:9, :] = src
    assert_bitexact(o.kv_cache_write(cache, src, 5), ref)


# ---------------------------------------------------------------- RMSNorm

def _rms64(x, w, eps):
    x64 = x.astype(np.float64)
    inv = 1.0 / np.sqrt(np.mean(x64 * x64, axis=-1, keepdims=True) + eps)
    return x64 * inv * w.astype(np.float64)


def test_rmsnorm_reference_kat_against_cpu_rmsnorm():
    kat = K["rmsnorm_2x4"]
    x = np.array(kat["input"], dtype=np.float32)
    w = np.array(kat["weight"], dtype=np.float32)
    expected = o.cpu_rmsnorm_literal(x, w, kat["eps"])
    assert np.max(np.abs(o.rmsnorm(x, w, kat["eps"]) - expected)) <= kat["tol_f32"]
    got16 = o.rmsnorm(x.astype(np.float16), w.astype(np.float16), kat["eps"])
    assert np.max(np.abs(got16.astype(np.float32) - expected)) <= kat["tol_f16"]
    # RMSNorm then + 0 (rmsnorm.rs:442-530)
    plus0 = o.add(got16, np.zeros_like(got16)).astype(np.float32)
    assert np.max(np.abs(plus0 - expected)) <= kat["tol_f16"]
    kat = K["rmsnorm_f16_vs_f32"]
    x = np.array(kat["input"], dtype=np.float32)
    w = np.array(kat["weight"], dtype=np.float32)
    ref = o.rmsnorm(x, w, kat["eps"])
    got = o.rmsnorm(x.astype(np.float16), w.astype(np.float16), kat["eps"]).astype(np.float32)
    assert np.max(np.abs(got - ref)) <= kat["tol_f16_vs_f32"]


def test_rmsnorm_against_float64():
    x = synth.normal(21, (64, 960), 0.0, 2.0)
    w = synth.uniform_range(22, (960,), 0.5, 1.5)
    assert max_rel_err(o.rmsnorm(x, w, 1e-5), _rms64(x, w, 1e-5),
                       np.finfo(np.float32).tiny) < 1e-6
    xh, wh = x.astype(np.float16), w.astype(np.float16)
    exact = _rms64(xh, wh, 1e-5).astype(np.float16)
    assert f16_ulp_distance(o.rmsnorm(xh, wh, 1e-5), exact) <= 1


def test_rmsnorm_closed_forms():
    # constant row c: y = c / sqrt(c^2 + eps) * w
    x = np.full((3, 8), 3.0, dtype=np.float32)
    w = np.arange(1, 9, dtype=np.float32)
    got = o.rmsnorm(x, w, 1e-5)
    ref = 3.0 / np.sqrt(9.0 + 1e-5) * w
    assert np.allclose(got, ref, rtol=1e-6, atol=0)
    # zero row: y = 0 (inv = 1/sqrt(eps) is finite)
    assert np.all(o.rmsnorm(np.zeros((1, 8), np.float32), w, 1e-5) == 0)


def test_add_rmsnorm_is_add_then_rmsnorm():
    x = synth.normal(23, (16, 96))
    r = synth.normal(24, (16, 96))
    w = synth.uniform_range(25, (96,), 0.5, 1.5)
    s, y = o.add_rmsnorm(x, r, w, 1e-5)
    assert_bitexact(s, x + r)
    assert_bitexact(y, o.rmsnorm(x + r, w, 1e-5))


# ---------------------------------------------------------------- softmax

def _softmax64(x):
    # x - max is rounded to the input precision as in the reference kernel
    # (a float subtraction); exp and the sum are exact to float64.
    d = (x.astype(np.float32) - np.max(x.astype(np.float32), axis=-1, keepdims=True))
    e = np.exp(d.astype(np.float64))
    return e / np.sum(e, axis=-1, keepdims=True)


def test_softmax_against_float64_and_row_sums():
    x = synth.normal(31, (33, 257), 0.0, 4.0)
    got = o.softmax(x)
    assert max_rel_err(got, _softmax64(x), np.finfo(np.float32).tiny) < 1e-6
    assert np.allclose(got.astype(np.float64).sum(-1), 1.0, atol=1e-5)
    xh = x.astype(np.float16)
    assert f16_ulp_distance(o.softmax(xh), _softmax64(xh).astype(np.float16)) <= 1


def test_softmax_shift_invariance_and_special_rows():
    x = synth.normal(32, (4, 64))
    assert np.allclose(o.softmax(x), o.softmax(x + np.float32(7.0)), rtol=1e-5, atol=1e-9)
    ninf = np.full((2, 5), -np.inf, dtype=np.float32)
    assert np.isnan(o.softmax(ninf)).all()  # f32: no guard (softmax.metal:7-132)
    assert (o.softmax(ninf.astype(np.float16)) == 0).all()  # f16 guard (:166-173)


def test_softmax_kats():
    kat = K["softmax_rows"]
    x = np.array(kat["input"], dtype=np.float32).reshape(kat["shape"])
    ref = o.softmax(x)
    got = o.softmax(x.astype(np.float16)).astype(np.float32)
    assert np.max(np.abs(got - ref)) < kat["tol_f16_vs_f32"]
    assert np.all(np.abs(got.sum(-1) - 1.0) < kat["row_sum_tol"])


def test_scale_mask_kats():
    kat = K["scale_mask_prefill"]
    x = np.array(kat["input"], dtype=np.float32).reshape(kat["shape"])
    ref = o.scale_mask(x, kat["scale"], kat["start"])
    assert_bitexact(ref.ravel(), floats(kat["expected_f32"]))
    got = o.scale_mask(x.astype(np.float16), kat["scale"], kat["start"]).astype(np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(np.isinf(got), ~fin) and np.all(got[~fin] < 0)
    assert np.max(np.abs(got[fin] - ref[fin])) < kat["tol_f16_vs_f32"]
    for name in ("scale_mask_decode", "scale_mask_intermediate"):
        kat = K[name]
        x = np.array(kat["input"], dtype=np.float16).reshape(kat["shape"])
        got = o.scale_mask(x, kat["scale"], kat["start"]).astype(np.float32).ravel()
        assert_bitexact(got, floats(kat["expected"]))


def test_scale_mask_against_numpy_triangle():
    q, k, start, heads = 7, 12, 5, 3
    x = synth.normal(33, (heads, q, k))
    mask = np.arange(k)[None, :] > (start + np.arange(q))[:, None]
    ref = np.where(mask[None], np.float32(-np.inf), x * np.float32(0.125))
    assert_bitexact(o.scale_mask(x, 0.125, start), ref)


def test_mask_softmax_kat():
    kat = K["mask_softmax"]
    x = np.array(kat["input"], dtype=np.float32).reshape(kat["shape"])
    ref = o.attention_softmax(x, kat["scale"], kat["start"])
    got = o.attention_softmax(x.astype(np.float16), kat["scale"], kat["start"])
    got = got.astype(np.float32)
    assert np.max(np.abs(got - ref)) < kat["tol_f16_vs_f32"]
    assert all(got.ravel()[i] == 0.0 for i in kat["zero_indices"])


# ------------------------------------------------------------------- RoPE

def test_rope_table_against_float64():
    c, s = o.rope_table(64, 4096, 10000.0)
    pos = np.arange(4096, dtype=np.float64)[:, None]
    inv = 10000.0 ** (-(2.0 * np.arange(32)) / 64.0)
    ang = pos * inv[None, :]
    # float angles up to ~4096 rad: error ~ |angle| * 2^-24
    tol = np.maximum(ang, 1.0) * 3e-7
    assert np.all(np.abs(c - np.cos(ang)) <= tol)
    assert np.all(np.abs(s - np.sin(ang)) <= tol)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)


def test_rope_against_complex_rotation():
    c, s = o.rope_table(16, 32, 10000.0)
    x = synth.normal(41, (2, 3, 10, 16))
    start = 4
    got = o.rope(x, c, s, start)
    z = x[..., :8].astype(np.complex128) + 1j * x[..., 8:].astype(np.complex128)
    rot = c[start:start + 10].astype(np.float64) + 1j * s[start:start + 10].astype(np.float64)
    ref = z * rot[None, None]
    a, b = x[..., :8].astype(np.float64), x[..., 8:].astype(np.float64)
    cc, ss = c[start:start + 10].astype(np.float64), s[start:start + 10].astype(np.float64)
    # cancellation-safe magnitude of each output: |a c| + |b s| and |b c| + |a s|
    floor = np.concatenate([np.abs(a * cc) + np.abs(b * ss), np.abs(b * cc) + np.abs(a * ss)],
                           axis=-1) + 1e-30
    err = np.abs(got - np.concatenate([ref.real, ref.imag], axis=-1)) / floor
    assert err.max() < 2e-7


def test_rope_identity_at_position_zero_and_inverse():
    c, s = o.rope_table(8, 4, 10000.0)
    x = synth.normal(42, (1, 1, 1, 8))
    assert_bitexact(o.rope(x, c, s, 0), x)  # cos 1, sin 0
    y = o.rope(x.reshape(1, 1, 1, 8), c, s, 3)
    back = o.rope(y, c, -s, 3)  # rotate by -angle
    assert np.allclose(back, x, rtol=0, atol=1e-6)


def _rope_f16_ulp_where_conditioned(got, x16, c, s, start):
    """Max f16 ulp distance of `got` from the exact rotation of the f16 inputs
    by the f32 table (float64, rounded once to f16), over outputs whose value
    is at least 1/64 of the magnitude |a c| + |b s| (where an f32 evaluation
    is within 2^-17 relative of the exact value, so one rounding to f16 is
    off by at most 1 ulp)."""
    from helpers import f16_ulp_distance
    seq, half = x16.shape[-2], x16.shape[-1] // 2
    a = x16[..., :half].astype(np.float64)
    b = x16[..., half:].astype(np.float64)
    cc = c[start:start + seq].astype(np.float64)
    ss = s[start:start + seq].astype(np.float64)
    exact = np.concatenate([a * cc - b * ss, b * cc + a * ss], axis=-1)
    mag = np.concatenate([np.abs(a * cc) + np.abs(b * ss), np.abs(b * cc) + np.abs(a * ss)],
                         axis=-1)
    keep = np.abs(exact) >= mag / 64
    assert keep.mean() > 0.9
    return f16_ulp_distance(got[keep], exact.astype(np.float16)[keep])


def test_rope_f16_is_one_rounding_of_the_exact_rotation():
    """oracle_rope_f16 (rope.metal:66-97): halves widened, the rotation in
    f32, one rounding to f16 -- within 1 ulp of the correctly rounded exact
    rotation wherever cancellation is limited, at the SmolLM2 layer's table
    (head 64, theta 1e4) over positions 0..4095."""
    c, s = o.rope_table(64, 4096, 10000.0)
    for start, seq in ((0, 4096), (3000, 700)):
        x16 = synth.normal(synth.seed_for("rope-f16-pin", start), (1, 3, seq, 64),
                           0.0, 2.0).astype(np.float16)
        assert _rope_f16_ulp_where_conditioned(o.rope(x16, c, s, start), x16, c, s,
                                               start) <= 1


def test_rope_f16_pin_catches_an_extra_rounding():
    """A plausible slip -- each product rounded to f16 before the sum -- fails
    the same check on the same inputs."""
    c, s = o.rope_table(64, 4096, 10000.0)
    x16 = synth.normal(synth.seed_for("rope-f16-pin", 0), (1, 3, 4096, 64), 0.0,
                       2.0).astype(np.float16)
    half = 32
    a = x16[..., :half].astype(np.float32)
    b = x16[..., half:].astype(np.float32)
    cc, ss = c[:4096], s[:4096]
    h = np.float16
    slip = np.concatenate([(a * cc).astype(h).astype(np.float32) - (b * ss).astype(h),
                           (b * cc).astype(h).astype(np.float32) + (a * ss).astype(h)],
                          axis=-1).astype(h)
    assert _rope_f16_ulp_where_conditioned(slip, x16, c, s, 0) > 1


def test_rope_kat_f16_vs_f32():
    kat = K["rope_f16_vs_f32"]
    c, s = o.rope_table(kat["head_dim"], kat["max_seq_len"], kat["theta"])
    x = np.array(kat["input"], dtype=np.float32).reshape(kat["shape"])
    ref = o.rope(x, c, s, kat["start"])
    got = o.rope(x.astype(np.float16), c, s, kat["start"]).astype(np.float32)
    assert np.max(np.abs(got - ref)) <= kat["tol_f16_vs_f32"]


# ------------------------------------------------- planted mistakes are caught

# ------------------------------------------------------------ attention core

def _cache(seed, batch, heads, capacity, head_dim, kv_len, dtype=np.float32):
    """A [B, H, capacity, D] cache whose rows past kv_len hold NaN, so a read
    of an unused row shows up in every result."""
    kv = synth.normal(seed, (batch, heads, capacity, head_dim)).astype(dtype)
    kv[:, :, kv_len:] = np.nan
    return kv


GQA_CASES = [  # batch, q_heads, kv_heads, q_len, kv_len, capacity, head_dim
    (1, 6, 2, 5, 7, 9, 16),
    (2, 3, 3, 4, 4, 4, 8),
    (1, 15, 5, 3, 33, 40, 64),
]


@pytest.mark.parametrize("case", GQA_CASES)
def test_gqa_qk_against_float64(case):
    b, qh, kvh, ql, kl, cap, hd = case
    q = synth.normal(61, (b, qh, ql, hd))
    k = _cache(62, b, kvh, cap, hd, kl)
    exact = np.matmul(q.astype(np.float64), np.swapaxes(gqa_expand(k, qh, kl), -1, -2))
    dot_abs = np.matmul(np.abs(q.astype(np.float64)), np.swapaxes(np.abs(gqa_expand(k, qh, kl)), -1, -2))
    got = o.gqa_qk(q, k, kl)
    assert got.shape == (b, qh, ql, kl)
    assert np.all(np.abs(got - exact) <= hd * U32 * dot_abs + 1e-30)
    qh16, kh16 = q.astype(np.float16), k.astype(np.float16)
    exact16 = np.matmul(qh16.astype(np.float64), np.swapaxes(gqa_expand(kh16, qh, kl), -1, -2))
    got16 = o.gqa_qk(qh16, kh16, kl)
    dot16 = np.matmul(np.abs(qh16.astype(np.float64)),
                      np.swapaxes(np.abs(gqa_expand(kh16, qh, kl)), -1, -2))
    assert np.all(np.abs(got16 - exact16) <= hd * U32 * dot16 + ulp16(exact16) / 2 * 1.0001)


@pytest.mark.parametrize("case", GQA_CASES)
def test_gqa_pv_against_float64(case):
    b, qh, kvh, ql, kl, cap, hd = case
    p = synth.uniform_range(63, (b, qh, ql, kl), 0.0, 1.0)
    v = _cache(64, b, kvh, cap, hd, kl)
    ve = gqa_expand(v, qh, kl)
    exact = np.matmul(p.astype(np.float64), ve)
    weight = np.matmul(p.astype(np.float64), np.abs(ve))
    got = o.gqa_pv(p, v, kl)
    assert got.shape == (b, qh, ql, hd)
    assert np.all(np.abs(got - exact) <= kl * U32 * weight + 1e-30)
    p16, v16 = p.astype(np.float16), v.astype(np.float16)
    exact16 = np.matmul(p16.astype(np.float64), gqa_expand(v16, qh, kl))
    weight16 = np.matmul(p16.astype(np.float64), np.abs(gqa_expand(v16, qh, kl)))
    got16 = o.gqa_pv(p16, v16, kl)
    assert np.all(np.abs(got16 - exact16) <= kl * U32 * weight16 + ulp16(exact16) / 2 * 1.0001)


def test_gqa_small_integers_are_exact():
    """Small-integer operands: every product and partial sum is exact in
    float32 and in the f16 result, so any order gives the float64 value."""
    q = (np.arange(2 * 6 * 3 * 8) % 7 - 3).reshape(2, 6, 3, 8).astype(np.float32)
    k = (np.arange(2 * 2 * 5 * 8) % 5 - 2).reshape(2, 2, 5, 8).astype(np.float32)
    exact = np.matmul(q.astype(np.float64), np.swapaxes(gqa_expand(k, 6, 5), -1, -2))
    for dt in (np.float32, np.float16):
        assert np.array_equal(o.gqa_qk(q.astype(dt), k.astype(dt)).astype(np.float64), exact)
        assert np.array_equal(o.gqa_pv(exact.astype(dt) / 8, k.astype(dt)).astype(np.float64),
                              np.matmul(exact / 8, gqa_expand(k, 6, 5)))


def _composition_bounds(q, k, v, scale, start, kv_len, f16):
    return attention_bound(q, k, v, scale, start, kv_len, "f16_reference" if f16 else "f32")


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
@pytest.mark.parametrize("case", [(1, 6, 2, 5, 7, 9, 16, 2), (1, 15, 5, 17, 17, 24, 64, 0),
                                  (2, 4, 4, 1, 12, 12, 32, 11)])
def test_attention_composition_against_float64(case, dtype):
    """QK^T -> scale/mask -> softmax -> PV with the reference's rounding points
    stays within the forward error bound of those roundings."""
    b, qh, kvh, ql, kl, cap, hd, start = case
    q = synth.normal(65, (b, qh, ql, hd)).astype(dtype)
    k = _cache(66, b, kvh, cap, hd, kl, dtype)
    v = _cache(67, b, kvh, cap, hd, kl, dtype)
    scale = 1.0 / np.sqrt(hd)
    got = o.attention(q, k, v, scale, start, kl)
    exact, bound = _composition_bounds(q, k, v, scale, start, kl, dtype == np.float16)
    assert got.shape == exact.shape and np.isfinite(got).all()
    assert np.all(np.abs(got.astype(np.float64) - exact) <= bound)


def test_attention_core_kat():
    """nn/attention.rs:590-668: attention_core_encode == the op-by-op calls,
    (2, 2) and (3, 1) heads, D 4, 3 new positions after 2 cached, values
    (i % 5) - 2 and (i % 3) - 1, tolerance 1e-5."""
    kat = K["attention_core"]
    for case in kat["cases"]:
        qh, kvh = case["heads"]
        d, sl, start = kat["head_dim"], kat["seq_len"], kat["start_pos"]
        q = (np.arange(qh * sl * d) % 5 - 2).astype(np.float32).reshape(1, qh, sl, d)
        kv = (np.arange(kvh * (start + sl) * d) % 3 - 1).astype(np.float32)
        kv = kv.reshape(1, kvh, start + sl, d)
        got = o.attention(q, kv, kv, 1.0 / np.sqrt(d), start)
        expected = np.array(case["expected"], dtype=np.float64).reshape(got.shape)
        assert np.max(np.abs(got - expected)) < kat["tol"]


def test_planted_mistakes_fail_the_pins():
    """Plausible slips (a transposed operand, a dropped term, an off-by-one in
    the mask, double rounding) must fail the independent checks above."""
    x = synth.normal(51, (3, 9))
    mask = np.arange(9)[None, :] > (2 + np.arange(3))[:, None]
    ref = np.where(mask, np.float32(-np.inf), x * np.float32(0.5))
    off_by_one = o.scale_mask(x, 0.5, 3)  # start + 1
    assert not np.array_equal(np.isinf(off_by_one), np.isinf(ref))
    c, s = o.rope_table(8, 8, 10000.0)
    xr = synth.normal(52, (1, 1, 4, 8))
    wrong_sign = o.rope(xr, c, -s, 2)
    z = (xr[..., :4] + 1j * xr[..., 4:]) * (c[2:6] + 1j * s[2:6])
    assert not np.allclose(wrong_sign, np.concatenate([z.real, z.imag], -1), atol=1e-5)
    xn = synth.normal(53, (4, 32), 0.0, 2.0)
    w = synth.uniform_range(54, (32,), 0.5, 1.5)
    no_eps_in_mean = xn * (1.0 / np.sqrt(np.mean(xn.astype(np.float64) ** 2, -1,
                                                 keepdims=True) + 1.0)) * w
    assert max_rel_err(no_eps_in_mean, _rms64(xn, w, 1e-5), 1e-30) > 1e-3
    # swapped strides (a transposed operand) and tile-for-repeat are caught
    base = np.arange(24, dtype=np.float32)
    good = np.ascontiguousarray(base.reshape(2, 3, 4).transpose(1, 0, 2))
    swapped = o.contiguous(base, [3, 2, 4], [12, 4, 1])
    assert not np.array_equal(swapped, good)
    assert np.array_equal(o.contiguous(base, [3, 2, 4], [4, 12, 1]), good)
    kv = synth.normal(55, (1, 2, 3, 4))
    assert not np.array_equal(o.repeat_kv(kv, 2), np.tile(kv, (1, 2, 1, 1)))
    # attention: KV head h % KVH instead of h // (QH / KVH), and a mask start one too
    # late, both leave the float64 bound
    q = synth.normal(56, (1, 6, 4, 16))
    kc, vc = synth.normal(57, (1, 2, 8, 16)), synth.normal(58, (1, 2, 8, 16))
    exact, bound = _composition_bounds(q, kc, vc, 0.25, 3, 8, False)
    wrong_heads = np.concatenate([o.attention(q[:, h:h + 1], kc[:, h % 2:h % 2 + 1],
                                              vc[:, h % 2:h % 2 + 1], 0.25, 3)
                                  for h in range(6)], axis=1)
    assert np.all(np.abs(o.attention(q, kc, vc, 0.25, 3) - exact) <= bound)
    assert not np.all(np.abs(wrong_heads - exact) <= bound)
    assert not np.all(np.abs(o.attention(q, kc, vc, 0.25, 4) - exact) <= bound)
