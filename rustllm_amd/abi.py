"""ctypes binding of the C ABI in include/rustllm_hip.h.

This is the Python-side equivalent of the `extern "C"` block the Rust crate
would declare.  It loads ``rustllm_amd/librustllm_hip.so`` (built in-tree by
``python -m rustllm_amd.build``) and raises if the library is missing: there
is no fallback path.

``Context`` wraps one rl_context and offers numpy upload/download plus one
method per op; ``DeviceBuffer`` owns one rl_buffer from the context's pool.
"""

from __future__ import annotations

import ctypes
import os
from typing import Sequence

import numpy as np

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "librustllm_hip.so")

RL_OK = 0
STATUS_NAMES = {
    1: "InvalidArgument",
    2: "InvalidShape",
    3: "ShapeMismatch",
    4: "InvalidDimension",
    5: "UnsupportedDType",
    6: "NonContiguousTensor",
    7: "PositionOutOfRange",
    8: "ModelFormat",
    9: "Device",
    10: "InvalidTokenId",
}


class RlBuffer(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("len", ctypes.c_uint64),
                ("byte_len", ctypes.c_uint64)]


class RlProfile(ctypes.Structure):
    _fields_ = [(name, ctypes.c_uint64) for name in (
        "command_buffers", "compute_encoders", "kernel_dispatches", "commits", "waits",
        "buffer_allocations", "allocated_bytes")]


ERROR_MAX_RANK = 16


class RlErrorPayload(ctypes.Structure):
    """rl_error_payload: the fields of the TinyError variants that carry data."""
    _fields_ = [("code", ctypes.c_int32), ("left_rank", ctypes.c_uint32),
                ("right_rank", ctypes.c_uint32), ("token_id", ctypes.c_uint32),
                ("left", ctypes.c_uint64 * ERROR_MAX_RANK),
                ("right", ctypes.c_uint64 * ERROR_MAX_RANK),
                ("start_pos", ctypes.c_uint64), ("seq_len", ctypes.c_uint64),
                ("max_seq_len", ctypes.c_uint64), ("vocab_size", ctypes.c_uint64)]


class RustLLMError(RuntimeError):
    """A non-zero rl_status, named after the TinyError variant it maps to.

    `fields` holds the variant's data for ShapeMismatch ({left, right}),
    PositionOutOfRange ({start_pos, seq_len, max_seq_len}) and InvalidTokenId
    ({token_id, vocab_size}); it is empty for the other variants."""

    def __init__(self, status: int, message: str, fields: dict | None = None):
        self.status = status
        self.kind = STATUS_NAMES.get(status, f"status{status}")
        self.fields = fields or {}
        super().__init__(f"{self.kind}: {message}")


_P = ctypes.c_void_p
_U64 = ctypes.c_uint64
_U32 = ctypes.c_uint32
_I32 = ctypes.c_int32
_F = ctypes.c_float
_BUF = ctypes.POINTER(RlBuffer)
_U64P = ctypes.POINTER(ctypes.c_uint64)

# name -> (argtypes, restype); every symbol include/rustllm_hip.h declares.
SIGNATURES: dict[str, tuple[list, object]] = {
    "rl_last_error_message": ([], ctypes.c_char_p),
    "rl_last_error_payload": ([ctypes.POINTER(RlErrorPayload)], _I32),
    "rl_version": ([], ctypes.c_char_p),
    "rl_context_create": ([_I32, ctypes.POINTER(_P)], _I32),
    "rl_context_create_on_stream": ([_I32, _P, ctypes.POINTER(_P)], _I32),
    "rl_context_destroy": ([_P], None),
    "rl_context_stream": ([_P], _P),
    "rl_device_count": ([], _I32),
    "rl_buffer_empty": ([_P, _U64, _U64, _BUF], _I32),
    "rl_buffer_from_host": ([_P, _P, _U64, _U64, _BUF], _I32),
    "rl_buffer_to_host": ([_P, _BUF, _P, _U64], _I32),
    "rl_buffer_copy": ([_P, _BUF, _BUF, _U64], _I32),
    "rl_buffer_release": ([_P, _BUF], None),
    "rl_context_trim": ([_P], _I32),
    "rl_execution_begin": ([_P], _I32),
    "rl_execution_finish": ([_P], _I32),
    "rl_graph_capture_begin": ([_P], _I32),
    "rl_context_set_fusion": ([_P, _I32], _I32),
    "rl_graph_capture_end": ([_P, ctypes.POINTER(_P)], _I32),
    "rl_graph_launch": ([_P, _P], _I32),
    "rl_graph_destroy": ([_P], None),
    "rl_event_create": ([_P, ctypes.POINTER(_P)], _I32),
    "rl_event_record": ([_P, _P], _I32),
    "rl_event_wait": ([_P, _P], _I32),
    "rl_event_elapsed_ms": ([_P, _P, ctypes.POINTER(_F)], _I32),
    "rl_event_destroy": ([_P], None),
    "rl_event_time_next_kernel": ([_P, _P, _P], _I32),
    "rl_profile_begin": ([_P], None),
    "rl_profile_take": ([_P, ctypes.POINTER(RlProfile)], _I32),
    "rl_profile_dispatches": ([_P, ctypes.c_char_p], _U64),
    "rl_add_f32": ([_P, _BUF, _BUF, _BUF], _I32),
    "rl_add_f16": ([_P, _BUF, _BUF, _BUF], _I32),
    "rl_mul_f32": ([_P, _BUF, _BUF, _BUF], _I32),
    "rl_mul_f16": ([_P, _BUF, _BUF, _BUF], _I32),
    "rl_silu_f32": ([_P, _BUF, _BUF], _I32),
    "rl_silu_f16": ([_P, _BUF, _BUF], _I32),
    "rl_swiglu_f16": ([_P, _BUF, _BUF, _BUF], _I32),
    "rl_swiglu_f32": ([_P, _BUF, _BUF, _BUF], _I32),
    "rl_cast_f32_to_f16": ([_P, _BUF, _BUF], _I32),
    "rl_cast_f16_to_f32": ([_P, _BUF, _BUF], _I32),
    "rl_add_broadcast_f32": ([_P, _BUF, _BUF, _U64, _U64, _BUF], _I32),
    "rl_add_broadcast_f16": ([_P, _BUF, _BUF, _U64, _U64, _BUF], _I32),
    "rl_contiguous_f32": ([_P, _BUF, _U64P, _U64P, _U32, _BUF], _I32),
    "rl_contiguous_f16": ([_P, _BUF, _U64P, _U64P, _U32, _BUF], _I32),
    "rl_repeat_kv_f32": ([_P, _BUF, _U64, _U64, _U64, _U64, _U64, _BUF], _I32),
    "rl_repeat_kv_f16": ([_P, _BUF, _U64, _U64, _U64, _U64, _U64, _BUF], _I32),
    "rl_rmsnorm_f32": ([_P, _BUF, _BUF, _U64, _U64, _F, _BUF], _I32),
    "rl_rmsnorm_f16": ([_P, _BUF, _BUF, _U64, _U64, _F, _BUF], _I32),
    "rl_add_rmsnorm_f32": ([_P, _BUF, _BUF, _BUF, _U64, _U64, _F, _BUF, _BUF], _I32),
    "rl_add_rmsnorm_f16": ([_P, _BUF, _BUF, _BUF, _U64, _U64, _F, _BUF, _BUF], _I32),
    "rl_softmax_f32": ([_P, _BUF, _U64, _U64, _BUF], _I32),
    "rl_softmax_f16": ([_P, _BUF, _U64, _U64, _BUF], _I32),
    "rl_attention_scale_mask_f32": ([_P, _BUF, _F, _U64, _U64, _U64, _BUF], _I32),
    "rl_attention_scale_mask_f16": ([_P, _BUF, _F, _U64, _U64, _U64, _BUF], _I32),
    "rl_attention_softmax_f32": ([_P, _BUF, _F, _U64, _U64, _U64, _BUF], _I32),
    "rl_attention_softmax_f16": ([_P, _BUF, _F, _U64, _U64, _U64, _BUF], _I32),
    "rl_rope_f32": ([_P, _BUF, _BUF, _BUF, _U64, _U64, _U64, _BUF], _I32),
    "rl_rope_f16": ([_P, _BUF, _BUF, _BUF, _U64, _U64, _U64, _BUF], _I32),
    "rl_rope_strided_f32": ([_P, _BUF, _U64P, _U64P, _U32, _BUF, _BUF, _U64, _U64, _BUF], _I32),
    "rl_rope_strided_f16": ([_P, _BUF, _U64P, _U64P, _U32, _BUF, _BUF, _U64, _U64, _BUF], _I32),
    "rl_kv_cache_write_f32": ([_P, _BUF, _U64, _U64, _U64, _BUF, _U64, _U64], _I32),
    "rl_kv_cache_write_f16": ([_P, _BUF, _U64, _U64, _U64, _BUF, _U64, _U64], _I32),
    "rl_kv_cache_write_strided_f32": ([_P, _BUF, _U64P, _U64P, _U32, _BUF, _U64, _U64], _I32),
    "rl_kv_cache_write_strided_f16": ([_P, _BUF, _U64P, _U64P, _U32, _BUF, _U64, _U64], _I32),
    "rl_rope_kv_cache_write_f32": ([_P, _BUF, _U64P, _U64P, _U32, _BUF, _BUF, _U64, _U64, _BUF,
                                    _U64], _I32),
    "rl_rope_kv_cache_write_f16": ([_P, _BUF, _U64P, _U64P, _U32, _BUF, _BUF, _U64, _U64, _BUF,
                                    _U64], _I32),
    "rl_qkv_rope_kv_append_f32": ([_P, _BUF, _U64P, _U64P, _BUF, _U64P, _U64P, _BUF, _U64P,
                                   _U64P, _BUF, _BUF, _U64, _U64, _BUF, _BUF, _BUF, _U64], _I32),
    "rl_qkv_rope_kv_append_f16": ([_P, _BUF, _U64P, _U64P, _BUF, _U64P, _U64P, _BUF, _U64P,
                                   _U64P, _BUF, _BUF, _U64, _U64, _BUF, _BUF, _BUF, _U64], _I32),
    "rl_qkv_rope_kv_append_repeat_f32": ([_P, _BUF, _U64P, _U64P, _BUF, _U64P, _U64P, _BUF,
                                          _U64P, _U64P, _BUF, _BUF, _U64, _U64, _BUF, _BUF,
                                          _BUF, _U64, _U64, _BUF, _BUF], _I32),
    "rl_qkv_rope_kv_append_repeat_f16": ([_P, _BUF, _U64P, _U64P, _BUF, _U64P, _U64P, _BUF,
                                          _U64P, _U64P, _BUF, _BUF, _U64, _U64, _BUF, _BUF,
                                          _BUF, _U64, _U64, _BUF, _BUF], _I32),
    "rl_embedding_f32": ([_P, _BUF, _U64, _U64, ctypes.POINTER(ctypes.c_uint32), _U64, _BUF],
                         _I32),
    "rl_embedding_f16": ([_P, _BUF, _U64, _U64, ctypes.POINTER(ctypes.c_uint32), _U64, _BUF],
                         _I32),
    "rl_attention_f32": ([_P, _BUF, _BUF, _BUF] + [_U64] * 7 + [_F, _U64, _BUF], _I32),
    "rl_attention_f16": ([_P, _BUF, _BUF, _BUF] + [_U64] * 7 + [_F, _U64, _BUF], _I32),
    "rl_attention_f16_noalloc": ([_P, _BUF, _BUF, _BUF] + [_U64] * 7 + [_F, _U64, _BUF], _I32),
    "rl_gqa_qk_matmul_f32": ([_P, _BUF, _BUF] + [_U64] * 7 + [_BUF], _I32),
    "rl_gqa_qk_matmul_f16": ([_P, _BUF, _BUF] + [_U64] * 7 + [_BUF], _I32),
    "rl_gqa_pv_matmul_f32": ([_P, _BUF, _BUF] + [_U64] * 7 + [_BUF], _I32),
    "rl_gqa_pv_matmul_f16": ([_P, _BUF, _BUF] + [_U64] * 7 + [_BUF], _I32),
}

_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Loads the in-tree library (no fallback: a missing library is an error)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing; build it with `python -m rustllm_amd.build`")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
    return _lib


def last_error() -> str:
    return load().rl_last_error_message().decode()


def last_error_fields() -> tuple[int, dict]:
    """The thread's last failure code and its variant's fields (see RustLLMError)."""
    p = RlErrorPayload()
    code = int(load().rl_last_error_payload(ctypes.byref(p)))
    fields: dict = {}
    if code == 3:
        fields = {"left": [int(v) for v in p.left[:min(p.left_rank, ERROR_MAX_RANK)]],
                  "right": [int(v) for v in p.right[:min(p.right_rank, ERROR_MAX_RANK)]]}
    elif code == 7:
        fields = {"start_pos": int(p.start_pos), "seq_len": int(p.seq_len),
                  "max_seq_len": int(p.max_seq_len)}
    elif code == 10:
        fields = {"token_id": int(p.token_id), "vocab_size": int(p.vocab_size)}
    return code, fields


def check(status: int) -> None:
    if status != RL_OK:
        code, fields = last_error_fields()
        raise RustLLMError(status, last_error(), fields if code == status else None)


def device_count() -> int:
    return int(load().rl_device_count())


_DTYPES = {np.dtype(np.float32): 4, np.dtype(np.float16): 2}


def _u64_array(values: Sequence[int]):
    arr = (ctypes.c_uint64 * max(1, len(values)))(*[int(v) for v in values])
    return arr


class DeviceBuffer:
    """One pooled rl_buffer with the dtype/shape it was created for."""

    def __init__(self, ctx: "Context", raw: RlBuffer, dtype, shape):
        self.ctx = ctx
        self.raw = raw
        self.dtype = np.dtype(dtype)
        self.shape = tuple(int(s) for s in shape)

    @property
    def len(self) -> int:
        return int(self.raw.len)

    @property
    def byte_len(self) -> int:
        return int(self.raw.byte_len)

    @property
    def ptr(self) -> int:
        return int(self.raw.data or 0)

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        if out.nbytes:
            check(self.ctx.lib.rl_buffer_to_host(self.ctx.handle, ctypes.byref(self.raw),
                                                  out.ctypes.data, out.nbytes))
        return out

    def release(self) -> None:
        if self.raw.data and self.ctx.handle:
            self.ctx.lib.rl_buffer_release(self.ctx.handle, ctypes.byref(self.raw))

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


class Context:
    """One rl_context: a device, an in-order stream and a buffer pool."""

    def __init__(self, device: int = 0):
        self.lib = load()
        handle = ctypes.c_void_p()
        check(self.lib.rl_context_create(device, ctypes.byref(handle)))
        self.handle = handle

    def close(self) -> None:
        if self.handle:
            self.lib.rl_context_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---------------------------------------------------------- buffers
    def empty(self, shape, dtype) -> DeviceBuffer:
        dtype = np.dtype(dtype)
        n = int(np.prod(shape, dtype=np.int64))
        raw = RlBuffer()
        check(self.lib.rl_buffer_empty(self.handle, n, dtype.itemsize, ctypes.byref(raw)))
        return DeviceBuffer(self, raw, dtype, shape)

    def clone(self, buf: DeviceBuffer) -> DeviceBuffer:
        """A new buffer with a stream-ordered device copy of `buf`."""
        out = self.empty(buf.shape, buf.dtype)
        check(self.lib.rl_buffer_copy(self.handle, ctypes.byref(buf.raw), ctypes.byref(out.raw),
                                      buf.byte_len))
        return out

    def copy(self, src: DeviceBuffer, dst: DeviceBuffer) -> None:
        """Stream-ordered device copy of src's bytes into dst."""
        check(self.lib.rl_buffer_copy(self.handle, ctypes.byref(src.raw), ctypes.byref(dst.raw),
                                      src.byte_len))

    def upload(self, array) -> DeviceBuffer:
        a = np.ascontiguousarray(array)
        if a.dtype not in _DTYPES and a.dtype != np.uint32:
            raise TypeError(f"unsupported dtype {a.dtype}")
        raw = RlBuffer()
        check(self.lib.rl_buffer_from_host(self.handle, a.ctypes.data, a.size, a.itemsize,
                                            ctypes.byref(raw)))
        return DeviceBuffer(self, raw, a.dtype, a.shape)

    def begin(self) -> None:
        check(self.lib.rl_execution_begin(self.handle))

    def finish(self) -> None:
        check(self.lib.rl_execution_finish(self.handle))

    # ---------------------------------------------------------- profile
    def profile_begin(self) -> None:
        self.lib.rl_profile_begin(self.handle)

    def profile_take(self) -> dict | None:
        p = RlProfile()
        if not self.lib.rl_profile_take(self.handle, ctypes.byref(p)):
            return None
        return {name: int(getattr(p, name)) for name, _ in RlProfile._fields_}

    def dispatches(self, kernel_name: str) -> int:
        return int(self.lib.rl_profile_dispatches(self.handle, kernel_name.encode()))

    # ---------------------------------------------------------- timing
    def event(self):
        e = ctypes.c_void_p()
        check(self.lib.rl_event_create(self.handle, ctypes.byref(e)))
        return e

    def record(self, event) -> None:
        check(self.lib.rl_event_record(self.handle, event))

    def wait(self, event) -> None:
        """Later work on this context waits for `event`."""
        check(self.lib.rl_event_wait(self.handle, event))

    def elapsed_ms(self, start, end) -> float:
        ms = ctypes.c_float()
        check(self.lib.rl_event_elapsed_ms(start, end, ctypes.byref(ms)))
        return float(ms.value)

    def destroy_event(self, event) -> None:
        self.lib.rl_event_destroy(event)

    def time_next_kernel(self, start, stop) -> None:
        """The next kernel launched records its own start/end in these events."""
        check(self.lib.rl_event_time_next_kernel(self.handle, start, stop))

    def capture_begin(self) -> None:
        check(self.lib.rl_graph_capture_begin(self.handle))

    def set_fusion(self, enabled: bool) -> None:
        """Whether streaming ops recorded into a graph share fused launches."""
        check(self.lib.rl_context_set_fusion(self.handle, 1 if enabled else 0))

    def capture_end(self):
        g = ctypes.c_void_p()
        check(self.lib.rl_graph_capture_end(self.handle, ctypes.byref(g)))
        return g

    def graph_launch(self, graph) -> None:
        check(self.lib.rl_graph_launch(self.handle, graph))

    def graph_destroy(self, graph) -> None:
        self.lib.rl_graph_destroy(graph)

    # ---------------------------------------------------------- ops
    @staticmethod
    def _sfx(buf: DeviceBuffer) -> str:
        return "f16" if buf.dtype == np.float16 else "f32"

    def _call(self, name: str, *args) -> None:
        conv = [ctypes.byref(a.raw) if isinstance(a, DeviceBuffer) else a for a in args]
        check(getattr(self.lib, name)(self.handle, *conv))

    def _binary(self, op: str, a: DeviceBuffer, b: DeviceBuffer, out=None) -> DeviceBuffer:
        out = out or self.empty(a.shape, a.dtype)
        self._call(f"rl_{op}_{self._sfx(a)}", a, b, out)
        return out

    def add(self, a, b, out=None):
        return self._binary("add", a, b, out)

    def mul(self, a, b, out=None):
        return self._binary("mul", a, b, out)

    def swiglu(self, gate, up, out=None):
        return self._binary("swiglu", gate, up, out)

    def silu(self, x, out=None):
        out = out or self.empty(x.shape, x.dtype)
        self._call(f"rl_silu_{self._sfx(x)}", x, out)
        return out

    def cast(self, x, dtype, out=None):
        dtype = np.dtype(dtype)
        out = out or self.empty(x.shape, dtype)
        name = "rl_cast_f32_to_f16" if dtype == np.float16 else "rl_cast_f16_to_f32"
        self._call(name, x, out)
        return out

    def add_broadcast(self, x, bias, out=None):
        out = out or self.empty(x.shape, x.dtype)
        cols = bias.len
        self._call(f"rl_add_broadcast_{self._sfx(x)}", x, bias, x.len // max(cols, 1), cols,
                   out)
        return out

    def contiguous(self, src, dims, strides, out=None):
        out = out or self.empty(dims, src.dtype)
        d, s = _u64_array(dims), _u64_array(strides)
        self._call(f"rl_contiguous_{self._sfx(src)}", src, d, s, len(dims), out)
        return out

    def repeat_kv(self, x, repeats: int, out=None):
        b, kvh, s, d = x.shape
        out = out or self.empty((b, kvh * repeats, s, d), x.dtype)
        self._call(f"rl_repeat_kv_{self._sfx(x)}", x, b, kvh, s, d, repeats, out)
        return out

    def rmsnorm(self, x, weight, eps: float, out=None):
        out = out or self.empty(x.shape, x.dtype)
        hidden = weight.len
        self._call(f"rl_rmsnorm_{self._sfx(x)}", x, weight, x.len // hidden, hidden,
                   ctypes.c_float(eps), out)
        return out

    def add_rmsnorm(self, x, residual, weight, eps: float, sum_out=None, norm_out=None):
        sum_out = sum_out or self.empty(x.shape, x.dtype)
        norm_out = norm_out or self.empty(x.shape, x.dtype)
        hidden = weight.len
        self._call(f"rl_add_rmsnorm_{self._sfx(x)}", x, residual, weight, x.len // hidden,
                   hidden, ctypes.c_float(eps), sum_out, norm_out)
        return sum_out, norm_out

    def softmax(self, x, out=None):
        out = out or self.empty(x.shape, x.dtype)
        width = x.shape[-1]
        self._call(f"rl_softmax_{self._sfx(x)}", x, x.len // width, width, out)
        return out

    def scale_mask(self, x, scale: float, start: int, out=None):
        out = out or self.empty(x.shape, x.dtype)
        q, k = x.shape[-2], x.shape[-1]
        self._call(f"rl_attention_scale_mask_{self._sfx(x)}", x, ctypes.c_float(scale), q, k,
                   start, out)
        return out

    def attention_softmax(self, x, scale: float, start: int, out=None):
        out = out or self.empty(x.shape, x.dtype)
        q, k = x.shape[-2], x.shape[-1]
        self._call(f"rl_attention_softmax_{self._sfx(x)}", x, ctypes.c_float(scale), q, k,
                   start, out)
        return out

    def rope(self, x, cos, sin, start: int, out=None):
        out = out or self.empty(x.shape, x.dtype)
        s, d = x.shape[-2], x.shape[-1]
        self._call(f"rl_rope_{self._sfx(x)}", x, cos, sin, s, d, start, out)
        return out

    def rope_strided(self, src, dims, strides, cos, sin, start: int, out=None):
        out = out or self.empty(dims, src.dtype)
        d, s = _u64_array(dims), _u64_array(strides)
        table_rows = cos.shape[0]
        self._call(f"rl_rope_strided_{self._sfx(src)}", src, d, s, len(dims), cos, sin,
                   table_rows, start, out)
        return out

    # ------------------------------------------------ KV cache, embedding
    def kv_cache_write(self, cache, source, start: int) -> None:
        """Writes a contiguous [1, H, S, D] `source` into rows start.. of the
        [1, H, max, D] `cache` (in place)."""
        _, heads, max_seq, head_dim = cache.shape
        seq = source.shape[2]
        self._call(f"rl_kv_cache_write_{self._sfx(cache)}", cache, heads, max_seq, head_dim,
                   source, seq, start)

    def kv_cache_write_strided(self, src, dims, strides, cache, start: int) -> None:
        d, s = _u64_array(dims), _u64_array(strides)
        self._call(f"rl_kv_cache_write_strided_{self._sfx(cache)}", src, d, s, len(dims), cache,
                   cache.shape[2], start)

    def rope_kv_cache_write(self, src, dims, strides, cos, sin, start: int, cache) -> None:
        d, s = _u64_array(dims), _u64_array(strides)
        self._call(f"rl_rope_kv_cache_write_{self._sfx(cache)}", src, d, s, len(dims), cos, sin,
                   cos.shape[0], start, cache, cache.shape[2])

    def qkv_rope_kv_append(self, q, k, v, cos, sin, start: int, k_cache, v_cache, q_out=None):
        """q/k/v: (buffer, dims, strides) of [1, H, S, D] views.  Returns the
        rotated contiguous Q; K (rotated) and V land in the caches at start."""
        (qb, qd, qs), (kb, kd, ks), (vb, vd, vs) = q, k, v
        q_out = q_out or self.empty(qd, qb.dtype)
        self._call(f"rl_qkv_rope_kv_append_{self._sfx(qb)}", qb, _u64_array(qd), _u64_array(qs),
                   kb, _u64_array(kd), _u64_array(ks), vb, _u64_array(vd), _u64_array(vs), cos,
                   sin, cos.shape[0], start, q_out, k_cache, v_cache, k_cache.shape[2])
        return q_out

    def qkv_rope_kv_append_repeat(self, q, k, v, cos, sin, start: int, k_cache, v_cache,
                                  n_rep: int, q_out=None, k_rep=None, v_rep=None):
        """qkv_rope_kv_append, then repeat_kv of the caches' first start + S
        rows into contiguous [1, KVH * n_rep, start + S, D] outputs, in one
        launch.  Returns (q_out, k_rep, v_rep)."""
        (qb, qd, qs), (kb, kd, ks), (vb, vd, vs) = q, k, v
        q_out = q_out or self.empty(qd, qb.dtype)
        rep_shape = (kd[0], kd[1] * max(n_rep, 1), start + kd[2], kd[3])
        k_rep = k_rep or self.empty(rep_shape, kb.dtype)
        v_rep = v_rep or self.empty(rep_shape, vb.dtype)
        self._call(f"rl_qkv_rope_kv_append_repeat_{self._sfx(qb)}", qb, _u64_array(qd),
                   _u64_array(qs), kb, _u64_array(kd), _u64_array(ks), vb, _u64_array(vd),
                   _u64_array(vs), cos, sin, cos.shape[0], start, q_out, k_cache, v_cache,
                   k_cache.shape[2], n_rep, k_rep, v_rep)
        return q_out, k_rep, v_rep

    def attention(self, q, k, v, scale: float, start: int, kv_len=None, out=None):
        """Fused attention core: q [B, QH, Q, D]; k, v [B, KVH, capacity, D]
        buffers of which the first kv_len rows per head are used."""
        b, qh, ql, hd = q.shape
        kvh, cap = k.shape[1], k.shape[2]
        kv_len = cap if kv_len is None else kv_len
        out = out or self.empty(q.shape, q.dtype)
        self._call(f"rl_attention_{self._sfx(q)}", q, k, v, b, qh, kvh, ql, kv_len, hd, cap,
                   ctypes.c_float(scale), start, out)
        return out

    def attention_noalloc(self, q, k, v, scale: float, start: int, kv_len=None, out=None):
        """rl_attention_f16_noalloc: as attention() (f16), the decode path's
        partials and counters in the library's static scratch (the caller
        still passes the output)."""
        b, qh, ql, hd = q.shape
        kvh, cap = k.shape[1], k.shape[2]
        kv_len = cap if kv_len is None else kv_len
        out = out or self.empty(q.shape, q.dtype)
        self._call("rl_attention_f16_noalloc", q, k, v, b, qh, kvh, ql, kv_len, hd, cap,
                   ctypes.c_float(scale), start, out)
        return out

    def gqa_qk(self, q, k, kv_len=None, out=None):
        """Scores [B, QH, Q, kv_len] = Q K^T; k is [B, KVH, capacity, D]."""
        b, qh, ql, hd = q.shape
        kvh, cap = k.shape[1], k.shape[2]
        kv_len = cap if kv_len is None else kv_len
        out = out or self.empty((b, qh, ql, kv_len), q.dtype)
        self._call(f"rl_gqa_qk_matmul_{self._sfx(q)}", q, k, b, qh, kvh, ql, kv_len, hd, cap, out)
        return out

    def gqa_pv(self, probs, v, out=None):
        """[B, QH, Q, D] = P V for P [B, QH, Q, kv_len]; v is [B, KVH, capacity, D]."""
        b, qh, ql, kv_len = probs.shape
        kvh, cap, hd = v.shape[1], v.shape[2], v.shape[3]
        out = out or self.empty((b, qh, ql, hd), probs.dtype)
        self._call(f"rl_gqa_pv_matmul_{self._sfx(probs)}", probs, v, b, qh, kvh, ql, kv_len, hd,
                   cap, out)
        return out

    def embedding(self, weight, token_ids, out=None):
        ids = np.ascontiguousarray(token_ids, dtype=np.uint32)
        vocab, hidden = weight.shape
        out = out or self.empty((ids.size, hidden), weight.dtype)
        self._call(f"rl_embedding_{self._sfx(weight)}", weight, vocab, hidden,
                   ids.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), ids.size, out)
        return out
