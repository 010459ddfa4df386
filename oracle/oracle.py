"""numpy front end of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: the checker the HIP library is compared against.
Only tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
bench.py may import this module.  Every function restates one reference
kernel; the C source (oracle/oracle.c) cites the file:line of each.

f16 arrays are ``numpy.float16`` (bit patterns are passed through as
uint16); f32 arrays are ``numpy.float32``.  Each function allocates and
returns its output.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

_P = ctypes.c_void_p
_S = ctypes.c_size_t
_F = ctypes.c_float


def build(force: bool = False) -> str:
    """Compile liboracle.so with gcc through oracle/Makefile."""
    if force or not os.path.exists(_LIB_PATH):
        args = ["make", "-s", "-C", _HERE] + (["-B"] if force else [])
        subprocess.run(args, check=True)
    return _LIB_PATH


def _load() -> ctypes.CDLL:
    if not os.path.exists(_LIB_PATH):
        build()
    lib = ctypes.CDLL(_LIB_PATH)
    sigs = {
        "oracle_f32_to_f16": ([_F], ctypes.c_uint16),
        "oracle_f16_to_f32": ([ctypes.c_uint16], _F),
        "oracle_f32_to_f16_array": ([_P, _P, _S], None),
        "oracle_f16_to_f32_array": ([_P, _P, _S], None),
        "oracle_set_threads": ([ctypes.c_int], None),
        "oracle_get_threads": ([], ctypes.c_int),
        "oracle_add_f32": ([_P, _P, _P, _S], None),
        "oracle_add_f16": ([_P, _P, _P, _S], None),
        "oracle_mul_f32": ([_P, _P, _P, _S], None),
        "oracle_mul_f16": ([_P, _P, _P, _S], None),
        "oracle_silu_f32": ([_P, _P, _S], None),
        "oracle_silu_f16": ([_P, _P, _S], None),
        "oracle_swiglu_f16": ([_P, _P, _P, _S], None),
        "oracle_swiglu_f32": ([_P, _P, _P, _S], None),
        "oracle_cast_f32_to_f16": ([_P, _P, _S], None),
        "oracle_cast_f16_to_f32": ([_P, _P, _S], None),
        "oracle_add_broadcast_f32": ([_P, _P, _P, _S, _S], None),
        "oracle_add_broadcast_f16": ([_P, _P, _P, _S, _S], None),
        "oracle_contiguous": ([_P, _P, _P, _P, ctypes.c_uint32, _S], None),
        "oracle_repeat_kv": ([_P, _P, _S, _S, _S, _S, _S, _S], None),
        "oracle_rmsnorm_f32": ([_P, _P, _P, _S, _S, _F], None),
        "oracle_rmsnorm_f16": ([_P, _P, _P, _S, _S, _F], None),
        "oracle_cpu_rmsnorm_literal": ([_P, _P, _P, _S, _S, _F], None),
        "oracle_add_rmsnorm_f32": ([_P, _P, _P, _P, _P, _S, _S, _F], None),
        "oracle_add_rmsnorm_f16": ([_P, _P, _P, _P, _P, _S, _S, _F], None),
        "oracle_softmax_f32": ([_P, _P, _S, _S], None),
        "oracle_softmax_f16": ([_P, _P, _S, _S], None),
        "oracle_scale_mask_f32": ([_P, _P, _S, _F, _S, _S, _S], None),
        "oracle_scale_mask_f16": ([_P, _P, _S, _F, _S, _S, _S], None),
        "oracle_rope_f32": ([_P, _P, _P, _P, _S, _S, _S, _S], None),
        "oracle_rope_f16": ([_P, _P, _P, _P, _S, _S, _S, _S], None),
        "oracle_rope_table": ([_S, _S, _F, _P, _P], None),
        "oracle_embedding": ([_P, _P, _P, _S, _S, _S], None),
        "oracle_kv_cache_write": ([_P, _P, _S, _S, _S, _S, _S, _S], None),
        "oracle_gqa_qk_f32": ([_P, _P, _P] + [_S] * 7, None),
        "oracle_gqa_qk_f16": ([_P, _P, _P] + [_S] * 7, None),
        "oracle_gqa_pv_f32": ([_P, _P, _P] + [_S] * 7, None),
        "oracle_gqa_pv_f16": ([_P, _P, _P] + [_S] * 7, None),
    }
    for name, (args, res) in sigs.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    return lib


_lib = _load()


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "oracle inputs must be C-contiguous"
    return a.ctypes.data


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _f16(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float16)


def set_threads(n: int) -> None:
    _lib.oracle_set_threads(int(n))


def get_threads() -> int:
    return int(_lib.oracle_get_threads())


# ------------------------------------------------------------------ f16

def f32_to_f16_bits(value: float) -> int:
    return int(_lib.oracle_f32_to_f16(float(value)))


def f16_bits_to_f32(bits: int) -> float:
    return float(_lib.oracle_f16_to_f32(int(bits)))


def f32_to_f16(a) -> np.ndarray:
    a = _f32(a)
    out = np.empty(a.shape, dtype=np.float16)
    _lib.oracle_f32_to_f16_array(_ptr(a), _ptr(out), a.size)
    return out


def f16_to_f32(a) -> np.ndarray:
    a = _f16(a)
    out = np.empty(a.shape, dtype=np.float32)
    _lib.oracle_f16_to_f32_array(_ptr(a), _ptr(out), a.size)
    return out


# ---------------------------------------------------------- element-wise

def _binary(name: str, a, b, conv):
    a, b = conv(a), conv(b)
    assert a.size == b.size
    out = np.empty(a.shape, dtype=a.dtype)
    getattr(_lib, name)(_ptr(a), _ptr(b), _ptr(out), a.size)
    return out


def _unary(name: str, a, conv, out_dtype=None):
    a = conv(a)
    out = np.empty(a.shape, dtype=out_dtype or a.dtype)
    getattr(_lib, name)(_ptr(a), _ptr(out), a.size)
    return out


def add(a, b):
    return _binary("oracle_add_f16", a, b, _f16) if np.asarray(a).dtype == np.float16 else \
        _binary("oracle_add_f32", a, b, _f32)


def mul(a, b):
    return _binary("oracle_mul_f16", a, b, _f16) if np.asarray(a).dtype == np.float16 else \
        _binary("oracle_mul_f32", a, b, _f32)


def silu(a):
    return _unary("oracle_silu_f16", a, _f16) if np.asarray(a).dtype == np.float16 else \
        _unary("oracle_silu_f32", a, _f32)


def swiglu(gate, up):
    """Fused silu(gate) * up: one f16 rounding (silu.metal:38-46); f32 is the
    silu_f32 -> mul_f32 composition (nn/swiglu.rs:15-37)."""
    if np.asarray(gate).dtype == np.float16:
        return _binary("oracle_swiglu_f16", gate, up, _f16)
    return _binary("oracle_swiglu_f32", gate, up, _f32)


def cast(a, dtype):
    a = np.asarray(a)
    if np.dtype(dtype) == a.dtype:
        return a.copy()
    if np.dtype(dtype) == np.float16:
        return _unary("oracle_cast_f32_to_f16", a, _f32, np.float16)
    return _unary("oracle_cast_f16_to_f32", a, _f16, np.float32)


def add_broadcast(x, bias):
    x = np.asarray(x)
    conv = _f16 if x.dtype == np.float16 else _f32
    x, bias = conv(x), conv(bias)
    cols = bias.size
    rows = x.size // cols
    out = np.empty(x.shape, dtype=x.dtype)
    name = "oracle_add_broadcast_f16" if x.dtype == np.float16 else "oracle_add_broadcast_f32"
    getattr(_lib, name)(_ptr(x), _ptr(bias), _ptr(out), rows, cols)
    return out


# --------------------------------------------------------- data movement

def contiguous(storage, dims, strides):
    """Gather a strided view of the flat ``storage`` array into a new
    contiguous array of shape ``dims`` (contiguous.metal:21-34)."""
    storage = np.ascontiguousarray(storage)
    d = np.asarray(dims, dtype=np.uint64)
    s = np.asarray(strides, dtype=np.uint64)
    out = np.empty(tuple(int(x) for x in dims), dtype=storage.dtype)
    _lib.oracle_contiguous(_ptr(storage), _ptr(out), _ptr(d), _ptr(s), len(dims),
                           storage.dtype.itemsize)
    return out


def repeat_kv(x, repeats: int):
    x = np.ascontiguousarray(x)
    b, kvh, s, d = x.shape
    out = np.empty((b, kvh * repeats, s, d), dtype=x.dtype)
    _lib.oracle_repeat_kv(_ptr(x), _ptr(out), b, kvh, s, d, repeats, x.dtype.itemsize)
    return out


def embedding(weight, ids):
    weight = np.ascontiguousarray(weight)
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    vocab, hidden = weight.shape
    assert int(ids.max(initial=0)) < vocab
    out = np.empty((ids.size, hidden), dtype=weight.dtype)
    _lib.oracle_embedding(_ptr(weight), _ptr(ids), _ptr(out), ids.size, hidden,
                          weight.dtype.itemsize)
    return out


def kv_cache_write(cache, src, start: int):
    """Returns a copy of ``cache`` [1, H, max, D] with ``src`` [1, H, S, D]
    written at sequence offset ``start``."""
    cache = np.array(cache, copy=True, order="C")
    src = np.ascontiguousarray(src, dtype=cache.dtype)
    _, heads, max_seq, head_dim = cache.shape
    _lib.oracle_kv_cache_write(_ptr(cache), _ptr(src), heads, src.shape[2], max_seq, head_dim,
                               start, cache.dtype.itemsize)
    return cache


# ------------------------------------------------------------ reductions

def rmsnorm(x, weight, eps: float):
    x = np.asarray(x)
    conv = _f16 if x.dtype == np.float16 else _f32
    x, weight = conv(x), conv(weight)
    hidden = weight.size
    rows = x.size // hidden
    out = np.empty(x.shape, dtype=x.dtype)
    name = "oracle_rmsnorm_f16" if x.dtype == np.float16 else "oracle_rmsnorm_f32"
    getattr(_lib, name)(_ptr(x), _ptr(weight), _ptr(out), rows, hidden, eps)
    return out


def cpu_rmsnorm_literal(x, weight, eps: float):
    x, weight = _f32(x), _f32(weight)
    hidden = weight.size
    out = np.empty(x.shape, dtype=np.float32)
    _lib.oracle_cpu_rmsnorm_literal(_ptr(x), _ptr(weight), _ptr(out), x.size // hidden, hidden,
                                    eps)
    return out


def add_rmsnorm(x, residual, weight, eps: float):
    """Returns (x + residual, rmsnorm(x + residual) * weight)."""
    x = np.asarray(x)
    conv = _f16 if x.dtype == np.float16 else _f32
    x, residual, weight = conv(x), conv(residual), conv(weight)
    hidden = weight.size
    rows = x.size // hidden
    s = np.empty(x.shape, dtype=x.dtype)
    y = np.empty(x.shape, dtype=x.dtype)
    name = "oracle_add_rmsnorm_f16" if x.dtype == np.float16 else "oracle_add_rmsnorm_f32"
    getattr(_lib, name)(_ptr(x), _ptr(residual), _ptr(weight), _ptr(s), _ptr(y), rows, hidden,
                        eps)
    return s, y


def softmax(x):
    x = np.asarray(x)
    conv = _f16 if x.dtype == np.float16 else _f32
    x = conv(x)
    width = x.shape[-1]
    out = np.empty(x.shape, dtype=x.dtype)
    name = "oracle_softmax_f16" if x.dtype == np.float16 else "oracle_softmax_f32"
    getattr(_lib, name)(_ptr(x), _ptr(out), x.size // width, width)
    return out


def scale_mask(x, scale: float, start: int):
    """attention_scale_mask on [..., q, k] scores."""
    x = np.asarray(x)
    conv = _f16 if x.dtype == np.float16 else _f32
    x = conv(x)
    q, k = x.shape[-2], x.shape[-1]
    out = np.empty(x.shape, dtype=x.dtype)
    name = "oracle_scale_mask_f16" if x.dtype == np.float16 else "oracle_scale_mask_f32"
    getattr(_lib, name)(_ptr(x), _ptr(out), x.size, scale, q, k, start)
    return out


def attention_softmax(x, scale: float, start: int):
    """The reference's two adjacent calls (nn/attention.rs:233-240)."""
    return softmax(scale_mask(x, scale, start))


def rope(x, cos_table, sin_table, start: int):
    """RoPE on a contiguous [..., S, D] array with f32 [rows, D/2] tables."""
    x = np.asarray(x)
    conv = _f16 if x.dtype == np.float16 else _f32
    x = conv(x)
    c, s = _f32(cos_table), _f32(sin_table)
    seq_len, head_dim = x.shape[-2], x.shape[-1]
    out = np.empty(x.shape, dtype=x.dtype)
    name = "oracle_rope_f16" if x.dtype == np.float16 else "oracle_rope_f32"
    getattr(_lib, name)(_ptr(x), _ptr(c), _ptr(s), _ptr(out), x.size, seq_len, head_dim, start)
    return out


def rope_table(head_dim: int, max_seq_len: int, theta: float):
    half = head_dim // 2
    c = np.empty((max_seq_len, half), dtype=np.float32)
    s = np.empty((max_seq_len, half), dtype=np.float32)
    _lib.oracle_rope_table(head_dim, max_seq_len, theta, _ptr(c), _ptr(s))
    return c, s


def _gqa_shapes(left, right, kv_len):
    batch, q_heads, q_len = left.shape[:3]
    r_batch, kv_heads, capacity, head_dim = right.shape
    kv_len = capacity if kv_len is None else kv_len
    assert r_batch == batch and q_heads % kv_heads == 0 and kv_len <= capacity
    return batch, q_heads, kv_heads, q_len, kv_len, head_dim, capacity


def gqa_qk(q, k, kv_len=None):
    """Q [B, QH, Q, D] x K^T with K [B, KVH, capacity, D], its first kv_len
    rows per head used: scores [B, QH, Q, kv_len] (gqa_matmul.metal:7-322)."""
    q = np.asarray(q)
    conv = _f16 if q.dtype == np.float16 else _f32
    q, k = conv(q), conv(k)
    b, qh, kvh, ql, kl, hd, cap = _gqa_shapes(q, k, kv_len)
    assert q.shape[3] == hd
    out = np.empty((b, qh, ql, kl), dtype=q.dtype)
    name = "oracle_gqa_qk_f16" if q.dtype == np.float16 else "oracle_gqa_qk_f32"
    getattr(_lib, name)(_ptr(q), _ptr(k), _ptr(out), b, qh, kvh, ql, kl, hd, cap)
    return out


def gqa_pv(probs, v, kv_len=None):
    """P [B, QH, Q, kv_len] x V with V [B, KVH, capacity, D]: [B, QH, Q, D]
    (gqa_matmul.metal:323-629)."""
    probs = np.asarray(probs)
    conv = _f16 if probs.dtype == np.float16 else _f32
    probs, v = conv(probs), conv(v)
    b, qh, kvh, ql, kl, hd, cap = _gqa_shapes(probs, v, kv_len)
    assert probs.shape[3] == kl
    out = np.empty((b, qh, ql, hd), dtype=probs.dtype)
    name = "oracle_gqa_pv_f16" if probs.dtype == np.float16 else "oracle_gqa_pv_f32"
    getattr(_lib, name)(_ptr(probs), _ptr(v), _ptr(out), b, qh, kvh, ql, kl, hd, cap)
    return out


def attention(q, k, v, scale: float, start: int, kv_len=None):
    """The reference's attention core (nn/attention.rs:216-247) as its four
    calls with their rounding points: QK^T, scale/mask, softmax, PV."""
    scores = gqa_qk(q, k, kv_len)
    probs = softmax(scale_mask(scores, scale, start))
    return gqa_pv(probs, v, scores.shape[-1])
