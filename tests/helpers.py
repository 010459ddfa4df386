"""Comparison helpers shared by the tests: the reference's known-answer vectors, bit-exact
comparison, relative error above a magnitude floor, f16 ulp distance, and float64 attention
with forward error bounds for the attention products."""

from __future__ import annotations

import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def kats() -> dict:
    with open(os.path.join(GOLDEN, "reference_kats.json")) as f:
        data = json.load(f)
    return {k: v for k, v in data.items() if not k.startswith("_")}


def floats(values) -> np.ndarray:
    """JSON numbers with "inf"/"-inf"/"nan" strings -> float32."""
    return np.array([float(v) for v in values], dtype=np.float32)


def bits(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a)
    return a.view(np.uint16 if a.dtype == np.float16 else np.uint32)


def assert_bitexact(got, ref, what=""):
    """Identical bit patterns; NaNs only need to be NaN on both sides."""
    got, ref = np.asarray(got), np.asarray(ref)
    assert got.shape == ref.shape and got.dtype == ref.dtype, (got.shape, ref.shape, got.dtype)
    gn, rn = np.isnan(got), np.isnan(ref)
    assert np.array_equal(gn, rn), f"{what}: NaN positions differ"
    bad = (bits(got) != bits(ref)) & ~gn
    if bad.any():
        i = int(np.flatnonzero(bad.ravel())[0])
        raise AssertionError(f"{what}: {int(bad.sum())} mismatches, first at {i}: "
                             f"got {got.ravel()[i]!r} ref {ref.ravel()[i]!r}")


def max_rel_err(got, ref, floor) -> float:
    """max |got - ref| / max(|ref|, floor) over finite refs; inf and NaN must match exactly.
    `floor` may be an array (per-element magnitude floor)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape
    assert np.array_equal(np.isnan(got), np.isnan(ref)), "NaN positions differ"
    inf = np.isinf(ref)
    assert np.array_equal(got[inf], ref[inf]), "infinities differ"
    assert not np.isinf(got[~inf]).any(), "unexpected infinity"
    fin = np.isfinite(ref)
    if not fin.any():
        return 0.0
    denom = np.maximum(np.abs(ref), floor)
    if np.ndim(denom):
        denom = denom[fin]
    return float(np.max(np.abs(got[fin] - ref[fin]) / denom))


def f16_ulp_distance(got, ref) -> int:
    """Max distance in ordered binary16 encodings; infinities must match exactly."""
    got = np.ascontiguousarray(got, dtype=np.float16)
    ref = np.ascontiguousarray(ref, dtype=np.float16)
    assert got.shape == ref.shape
    assert np.array_equal(np.isnan(got), np.isnan(ref)), "NaN positions differ"
    inf = np.isinf(ref)
    assert np.array_equal(got[inf], ref[inf]), "infinities differ"

    def key(a):
        b = a.view(np.uint16).astype(np.int32)
        mag = b & 0x7FFF
        return np.where(b & 0x8000, -mag, mag)

    ok = ~np.isnan(ref)
    if not ok.any():
        return 0
    return int(np.max(np.abs(key(got)[ok] - key(ref)[ok])))


def gqa_expand(kv, q_heads: int, kv_len: int) -> np.ndarray:
    """[B, KVH, capacity, D] -> float64 [B, QH, kv_len, D]: query head h reads
    KV head h // (QH / KVH) (np.repeat, the textbook grouped-query layout)."""
    kv = np.asarray(kv, dtype=np.float64)[:, :, :kv_len]
    return np.repeat(kv, q_heads // kv.shape[1], axis=1)


def attention_exact(q, k, v, scale: float, start: int, kv_len=None):
    """Float64 causal attention, softmax(mask(scale * Q K^T)) V, computed with
    numpy matrix products.  Returns (out, weight, dot_abs): weight[..., i, d] =
    sum_j p_ij |v_jd| (the magnitude an error bound of the output scales with)
    and dot_abs[..., i] = max_j sum_d |q_id k_jd| (that of the scores)."""
    q = np.asarray(q, dtype=np.float64)
    kv_len = k.shape[2] if kv_len is None else kv_len
    ke = gqa_expand(k, q.shape[1], kv_len)
    ve = gqa_expand(v, q.shape[1], kv_len)
    s = np.matmul(q, np.swapaxes(ke, -1, -2)) * float(scale)
    q_len = q.shape[2]
    masked = np.arange(kv_len)[None, :] > (start + np.arange(q_len))[:, None]
    s = np.where(masked, -np.inf, s)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    out = np.matmul(p, ve)
    weight = np.matmul(p, np.abs(ve))
    dot_abs = np.max(np.where(masked, 0.0, np.matmul(np.abs(q), np.swapaxes(np.abs(ke), -1, -2))),
                     axis=-1)
    return out, weight, dot_abs


U32 = 2.0 ** -24


def ulp16(x):
    """Spacing of binary16 at |x| (2^-24 below the normal range)."""
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -14)))
    return 2.0 ** (e - 10)


def attention_bound(q, k, v, scale: float, start: int, kv_len=None, kind="f32"):
    """(exact, bound): float64 attention and a forward error bound per output
    element, from the roundings each evaluation makes.

    u = 2^-24, w = sum_j p_j |v_j| (the output's magnitude scale), S = max_j
    sum_d |q_d k_jd|, T = a bound on |logit - max|:
      f32           scores in f32 (D u S each, times scale, on two logits),
                    exp / subtraction (8 u (1 + T)), sums over kv_len keys:
                    (2 scale (D + 1) u S + 8 u (1 + T) + (kv_len + 2) u) w
      f16_fused     the same plus probabilities fed to the P V product as
                    f16 (2^-11, twice with the normaliser: 2^-10), f16
                    subnormal probabilities (kv_len 2^-25 max|v|) and the
                    final rounding (1 ulp)
      f16_reference the reference's four calls: scores and scaled scores
                    rounded to f16 (2^-11 |x| each on two logits: 2^-8
                    scale S), probabilities rounded (2^-9 with the sum),
                    then as f16_fused."""
    exact, weight, dot_abs = attention_exact(q, k, v, scale, start, kv_len)
    kv_len = k.shape[2] if kv_len is None else kv_len
    hd = q.shape[-1]
    s_term = dot_abs[..., None]
    tmax = 2.0 * scale * float(np.max(dot_abs)) + 1.0
    rel = (2.0 * scale * (hd + 1) * U32 * s_term + 8.0 * U32 * (1.0 + tmax)
           + (kv_len + 2) * U32)
    if kind == "f32":
        return exact, rel * weight + 1e-30
    vmax = float(np.max(np.abs(np.asarray(v, np.float64)[:, :, :kv_len])))
    if kind == "f16_fused":
        rel = rel + 2.0 ** -10
    elif kind == "f16_reference":
        rel = rel + 2.0 ** -8 * scale * s_term + 2.0 ** -9
    else:
        raise ValueError(kind)
    return exact, rel * weight + kv_len * 2.0 ** -25 * vmax + ulp16(exact)
