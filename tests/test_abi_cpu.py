"""The C ABI without a GPU: the library loads, exports every declared symbol,
and validates arguments in the reference's order before touching a device.

With ctx == NULL an op that passes validation reports RL_ERR_DEVICE, so the
validation result of every path is observable here.  The buffers below carry
fake device addresses: validation never dereferences them and nothing is
launched.
"""

import ctypes
import os
import re

import numpy as np
import pytest

from rustllm_amd import abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rustllm_hip.h")

OK, ARG, SHAPE, MISMATCH, DIM, DTYPE, NONCONTIG, POS, FORMAT, DEVICE = range(10)

lib = abi.load()
NULL = None


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rl_[a-z0-9_]+)\s*\(", text)))


def buf(n, es, addr=0x10000):
    return abi.RlBuffer(addr, n, n * es)


def call(name, *args):
    conv = [ctypes.byref(a) if isinstance(a, abi.RlBuffer) else a for a in args]
    status = getattr(lib, name)(NULL, *conv)
    return status, abi.last_error()


def u64s(*v):
    return (ctypes.c_uint64 * len(v))(*v)


def test_every_declared_symbol_is_exported_and_bound():
    names = declared_functions()
    assert len(names) >= 50
    for name in names:
        assert hasattr(lib, name), f"{name} not exported"
        assert name in abi.SIGNATURES, f"{name} has no ctypes signature"
    assert set(abi.SIGNATURES) == set(names)


def test_library_is_gfx950_only_and_versioned():
    assert b"gfx950" in lib.rl_version()


def test_context_create_without_gpu_reports_device_error():
    if abi.device_count() > 0:
        pytest.skip("a GPU is visible")
    handle = ctypes.c_void_p()
    assert lib.rl_context_create(0, ctypes.byref(handle)) == DEVICE
    assert "no HIP GPU" in abi.last_error()
    assert not handle


def test_null_context_after_valid_arguments_is_a_device_error():
    st, msg = call("rl_add_f32", buf(8, 4), buf(8, 4), buf(8, 4))
    assert st == DEVICE and "no HIP context" in msg


@pytest.mark.parametrize("name,es", [("rl_add_f32", 4), ("rl_mul_f32", 4), ("rl_mul_f16", 2)])
def test_binary_length_mismatch(name, es):
    st, msg = call(name, buf(8, es), buf(9, es), buf(8, es))
    assert st == SHAPE
    assert "equal buffer lengths, got 8 and 9" in msg


def test_add_f16_checks_element_size_like_the_reference():
    # src/ops/add.rs:120: a F32-sized buffer is rejected by the F16 add.
    st, msg = call("rl_add_f16", buf(8, 4), buf(8, 2), buf(8, 2))
    assert st == SHAPE and "F16 add requires equal F16 buffers" in msg
    st, msg = call("rl_swiglu_f16", buf(8, 2), buf(7, 2), buf(8, 2))
    assert st == SHAPE and "SwiGLU requires equal F16 buffers" in msg


def test_output_buffer_is_checked():
    st, msg = call("rl_add_f32", buf(8, 4), buf(8, 4), buf(7, 4))
    assert st == SHAPE and "output buffer" in msg
    st, _ = call("rl_cast_f32_to_f16", buf(8, 4), buf(8, 4))  # f16 output must be 2-byte
    assert st == SHAPE


def test_input_smaller_than_its_elements_is_rejected():
    # An F16 buffer passed to an F32 op would be read past its end.
    st, msg = call("rl_add_f32", buf(8, 2), buf(8, 2), buf(8, 4))
    assert st == SHAPE and "fewer than" in msg


def test_silu_empty_and_u32():
    st, msg = call("rl_silu_f32", buf(0, 4), buf(0, 4))
    assert st == SHAPE and "SiLU input cannot be empty" in msg
    big = 1 << 32
    st, msg = call("rl_silu_f32", buf(big, 4), buf(big, 4))
    assert st == SHAPE and "exceeds u32" in msg
    st, msg = call("rl_mul_f32", buf(big, 4), buf(big, 4), buf(big, 4))
    assert st == SHAPE and "multiply input size exceeds u32" in msg


def test_rmsnorm_validation_order():
    # src/ops/rmsnorm.rs:38-116: hidden 0, then input size, then weight size.
    assert call("rl_rmsnorm_f32", buf(8, 4), buf(4, 4), 2, 0, ctypes.c_float(1e-5),
                buf(8, 4))[0] == SHAPE
    st, msg = call("rl_rmsnorm_f32", buf(9, 4), buf(4, 4), 2, 4, ctypes.c_float(1e-5), buf(9, 4))
    assert st == SHAPE and "RMSNorm input has 9 elements, expected 8" in msg
    st, msg = call("rl_rmsnorm_f32", buf(8, 4), buf(5, 4), 2, 4, ctypes.c_float(1e-5), buf(8, 4))
    assert st == SHAPE and "RMSNorm weight has 5 elements, expected 4" in msg
    assert call("rl_rmsnorm_f16", buf(8, 2), buf(4, 2), 2, 4, ctypes.c_float(1e-5),
                buf(8, 2))[0] == DEVICE


@pytest.mark.parametrize("name,es", [("rl_rmsnorm_f32", 4), ("rl_rmsnorm_f16", 2),
                                     ("rl_add_rmsnorm_f32", 4), ("rl_add_rmsnorm_f16", 2)])
@pytest.mark.parametrize("eps", [0.0, -1.0, float("inf"), float("nan")])
def test_rmsnorm_buffer_level_accepts_any_epsilon(name, es, eps):
    # src/ops/rmsnorm.rs:38-116 checks no epsilon; only the Tensor-level
    # ops::rmsnorm (:226-230) and RmsNorm::new (nn/rmsnorm.rs:29-33) do.
    if "add" in name:
        args = (buf(8, es), buf(8, es), buf(4, es), 2, 4, ctypes.c_float(eps), buf(8, es),
                buf(8, es))
    else:
        args = (buf(8, es), buf(4, es), 2, 4, ctypes.c_float(eps), buf(8, es))
    st, msg = call(name, *args)
    assert st == DEVICE and "no HIP context" in msg


def test_add_rmsnorm_validation():
    st, msg = call("rl_add_rmsnorm_f32", buf(8, 4), buf(6, 4), buf(4, 4), 2, 4,
                   ctypes.c_float(1e-5), buf(8, 4), buf(8, 4))
    assert st == MISMATCH and msg == "left=[8], right=[6]"
    assert abi.last_error_fields() == (MISMATCH, {"left": [8], "right": [6]})
    st, _ = call("rl_add_rmsnorm_f32", buf(8, 4), buf(8, 4), buf(4, 4), 2, 4,
                 ctypes.c_float(1e-5), buf(8, 4), buf(8, 4))
    assert st == DEVICE


def test_softmax_validation():
    # src/ops/softmax.rs:91-108
    st, msg = call("rl_softmax_f32", buf(8, 4), 0, 8, buf(8, 4))
    assert st == SHAPE and "rows and width must be greater than zero" in msg
    st, msg = call("rl_softmax_f32", buf(8, 4), 3, 3, buf(8, 4))
    assert st == SHAPE and "Softmax input has 8 elements" in msg
    st, _ = call("rl_softmax_f16", buf(8, 4), 2, 4, buf(8, 2))  # f32-sized f16 input
    assert st == SHAPE
    assert call("rl_softmax_f16", buf(8, 2), 2, 4, buf(8, 2))[0] == DEVICE


@pytest.mark.parametrize("name", ["rl_attention_scale_mask_f32", "rl_attention_softmax_f32"])
def test_scale_mask_validation(name):
    f = ctypes.c_float
    # src/ops/attention_scale_mask.rs:120-161, in order
    st, msg = call(name, buf(9, 4), f(0.5), 0, 3, 0, buf(9, 4))
    assert st == SHAPE and "query/key length cannot be zero" in msg
    for bad in (0.0, -0.5, float("inf"), float("nan")):
        st, msg = call(name, buf(9, 4), f(bad), 3, 3, 0, buf(9, 4))
        assert st == SHAPE and "scale must be positive and finite" in msg
    st, msg = call(name, buf(9, 4), f(0.5), 3, 3, 1, buf(9, 4))
    assert st == SHAPE and "exceeds key length" in msg
    st, msg = call(name, buf(10, 4), f(0.5), 3, 3, 0, buf(10, 4))
    assert st == SHAPE and "incompatible with query_len=3" in msg
    st, _ = call(name, buf(18, 4), f(0.5), 3, 3, 0, buf(18, 4))
    assert st == DEVICE


def test_rope_validation():
    f = "rl_rope_f32"
    tab = buf(8 * 2, 4)  # [8, 2] f32 tables for head_dim 4
    st, msg = call(f, buf(8, 4), tab, tab, 2, 3, 0, buf(8, 4))
    assert st == SHAPE and "head dimension must be positive and even" in msg
    st, msg = call(f, buf(8, 4), tab, tab, 0, 4, 0, buf(8, 4))
    assert st == SHAPE and "sequence length cannot be zero" in msg
    st, msg = call(f, buf(10, 4), tab, tab, 2, 4, 0, buf(10, 4))
    assert st == SHAPE and "not divisible by head dimension" in msg
    st, msg = call(f, buf(12, 4), tab, tab, 2, 4, 0, buf(12, 4))
    assert st == SHAPE and "incompatible with sequence length" in msg
    st, msg = call(f, buf(8, 4), tab, tab, 2, 4, 7, buf(8, 4))  # 7 + 2 > 8 table rows
    assert st == SHAPE and "position range is invalid" in msg
    st, msg = call(f, buf(8, 4), buf(16, 2), buf(16, 2), 2, 4, 0, buf(8, 4))
    assert st == DTYPE and "F32 cos/sin tables" in msg
    assert call(f, buf(8, 4), tab, tab, 2, 4, 6, buf(8, 4))[0] == DEVICE


def test_rope_strided_validation():
    tab = buf(8 * 2, 4)
    st, _ = call("rl_rope_strided_f16", buf(8, 2), u64s(8), u64s(1), 1, tab, tab, 8, 0,
                 buf(8, 2))
    assert st == DIM
    st, msg = call("rl_rope_strided_f16", buf(8, 2), u64s(2, 4), u64s(1, 2), 2, tab, tab, 8, 0,
                   buf(8, 2))
    assert st == NONCONTIG and "unit innermost stride" in msg
    # [1, 2, 1, 4] permuted to [1, 1, 2, 4]: strides [8, 4, 4, 1] (rope.rs:211-233)
    assert call("rl_rope_strided_f16", buf(8, 2), u64s(1, 1, 2, 4), u64s(8, 4, 4, 1), 4, tab,
                tab, 8, 0, buf(8, 2))[0] == DEVICE
    st, msg = call("rl_rope_strided_f16", buf(8, 2), u64s(1, 1, 2, 4), u64s(8, 4, 8, 1), 4,
                   tab, tab, 8, 0, buf(8, 2))
    assert st == SHAPE and "past the end" in msg


def test_contiguous_validation():
    st, msg = call("rl_contiguous_f32", buf(6, 2), u64s(2, 3), u64s(3, 1), 2, buf(6, 4))
    assert st == SHAPE and "does not match contiguous materialization dtype" in msg
    st, msg = call("rl_contiguous_f32", buf(4, 4), u64s(2, 3), u64s(3, 1), 2, buf(6, 4))
    assert st == SHAPE and "reaches element 5 of a 4-element source" in msg
    st, msg = call("rl_contiguous_f32", buf(6, 4), u64s(2, 3), u64s(1 << 33, 1), 2, buf(6, 4))
    assert st == SHAPE and "stride exceeds u32" in msg
    st, msg = call("rl_contiguous_f32", buf(6, 4), u64s(2, 3), u64s(4, 1), 2, buf(6, 4))
    assert st == SHAPE and "reaches element 6" in msg
    assert call("rl_contiguous_f32", buf(6, 4), u64s(3, 2), u64s(1, 3), 2,
                buf(6, 4))[0] == DEVICE
    assert call("rl_contiguous_f16", buf(5, 2), u64s(4, 5), u64s(0, 1), 2,
                buf(20, 2))[0] == DEVICE  # stride-0 broadcast is a valid view


def test_repeat_kv_validation():
    st, msg = call("rl_repeat_kv_f32", buf(8, 4), 1, 2, 2, 2, 0, buf(8, 4))
    assert st == FORMAT and "repeats must be greater than zero" in msg
    st, _ = call("rl_repeat_kv_f32", buf(9, 4), 1, 2, 2, 2, 3, buf(24, 4))
    assert st == SHAPE
    assert call("rl_repeat_kv_f32", buf(8, 4), 1, 2, 2, 2, 3, buf(24, 4))[0] == DEVICE


def test_broadcast_validation():
    st, msg = call("rl_add_broadcast_f32", buf(12, 4), buf(5, 4), 3, 4, buf(12, 4))
    assert st == MISMATCH and msg == "left=[3, 4], right=[5]"
    assert abi.last_error_fields() == (MISMATCH, {"left": [3, 4], "right": [5]})
    assert call("rl_add_broadcast_f32", buf(12, 4), buf(4, 4), 3, 4, buf(12, 4))[0] == DEVICE


def test_buffer_calls_without_context():
    raw = abi.RlBuffer()
    assert lib.rl_buffer_empty(NULL, 0, 4, ctypes.byref(raw)) == SHAPE  # len must be > 0
    assert lib.rl_buffer_empty(NULL, 4, 4, ctypes.byref(raw)) == DEVICE
    assert lib.rl_execution_finish(NULL) == DEVICE
    assert lib.rl_profile_take(NULL, None) == 0
    assert lib.rl_context_set_fusion(NULL, 0) == DEVICE
    assert lib.rl_graph_capture_begin(NULL) == DEVICE


def _fastdiv(d):
    s = 0
    while (1 << s) < d:
        s += 1
    magic = ((1 << 32) * ((1 << s) - d)) // d + 1
    assert magic < (1 << 32)
    return magic, s


def test_fastdiv_magic_numbers():
    """The multiply-high division used by the kernels (FastDiv in common.hpp)
    against exact integer division, over divisors and numerators at the
    edges of the 32-bit range."""
    rng = np.random.default_rng(0)
    divisors = [1, 2, 3, 5, 7, 9, 15, 64, 576, 1536, 2047, 2048, 4096, 65535, 65537,
                (1 << 31) - 1, 1 << 31, (1 << 31) + 1, (1 << 32) - 1]
    divisors += [int(v) for v in rng.integers(1, 1 << 32, 200)]
    nums = np.concatenate([np.arange(0, 5000, dtype=np.uint64),
                           (1 << 32) - 1 - np.arange(0, 5000, dtype=np.uint64),
                           rng.integers(0, 1 << 32, 20000).astype(np.uint64)])
    for d in divisors:
        magic, s = _fastdiv(d)
        hi = (nums * np.uint64(magic)) >> np.uint64(32)
        q = (hi + nums) >> np.uint64(s)
        assert np.array_equal(q, nums // np.uint64(d)), d


TOKEN = 10  # RL_ERR_INVALID_TOKEN_ID


def test_kv_cache_write_validation():
    # src/ops/kv_cache_write.rs:79-135: dtype, shape, position range, u32 limits
    f = "rl_kv_cache_write_f16"
    cache = buf(2 * 8 * 4, 2)  # [1, 2, 8, 4]
    st, msg = call(f, buf(64, 4), 2, 8, 4, buf(8, 2), 1, 0)
    assert st == DTYPE and "kv_cache_write_f16 expects F16 cache and source" in msg
    st, msg = call(f, buf(63, 2), 2, 8, 4, buf(8, 2), 1, 0)
    assert st == SHAPE and "invalid KV cache write shape" in msg
    st, msg = call(f, cache, 2, 8, 4, buf(12, 2), 1, 0)  # source is not [1, 2, 1, 4]
    assert st == SHAPE and "invalid KV cache write shape" in msg
    st, msg = call(f, cache, 2, 8, 4, buf(0, 2), 0, 0)
    assert st == SHAPE and "greater than zero" in msg
    st, msg = call(f, cache, 2, 8, 4, buf(16, 2), 2, 7)
    assert st == POS and "position range [7, 9) exceeds max sequence length 8" in msg
    # TinyError::PositionOutOfRange { start_pos, seq_len, max_seq_len }
    # (src/ops/kv_cache_write.rs:101-110) crosses the ABI as integers
    assert abi.last_error_fields() == (POS, {"start_pos": 7, "seq_len": 2, "max_seq_len": 8})
    with pytest.raises(abi.RustLLMError) as err:
        abi.check(st)
    assert err.value.kind == "PositionOutOfRange"
    assert err.value.fields == {"start_pos": 7, "seq_len": 2, "max_seq_len": 8}
    assert call(f, cache, 2, 8, 4, buf(16, 2), 2, 6)[0] == DEVICE
    # a later failure without a payload replaces it
    assert abi.last_error_fields() == (DEVICE, {})


def test_kv_cache_write_strided_validation():
    f = "rl_kv_cache_write_strided_f32"
    cache = buf(2 * 8 * 4, 4)
    # [1, 2, 3, 4] permute of a [1, 3, 2, 4] projection: strides [24, 4, 8, 1]
    dims, strides = u64s(1, 2, 3, 4), u64s(24, 4, 8, 1)
    st, msg = call(f, buf(24, 4), u64s(2, 3, 4), u64s(12, 4, 1), 3, cache, 8, 0)
    assert st == SHAPE and "invalid KV cache write shape" in msg
    st, _ = call(f, buf(48, 4), u64s(2, 1, 3, 4), u64s(24, 24, 8, 1), 4, buf(8 * 4, 4), 8, 0)
    assert st == SHAPE  # batch 2
    st, msg = call(f, buf(23, 4), dims, strides, 4, cache, 8, 0)
    assert st == SHAPE and "past the end" in msg
    st, _ = call(f, buf(24, 4), dims, strides, 4, cache, 8, 6)
    assert st == POS
    assert call(f, buf(24, 4), dims, strides, 4, cache, 8, 5)[0] == DEVICE
    # any innermost stride is accepted (the gather handles it)
    assert call(f, buf(24, 4), u64s(1, 2, 3, 4), u64s(24, 1, 2, 6), 4, cache, 8, 0)[0] == DEVICE


def test_rope_kv_cache_write_validation():
    f = "rl_rope_kv_cache_write_f16"
    tab = buf(8 * 2, 4)  # [8, 2] tables, head_dim 4
    cache = buf(2 * 8 * 4, 2)
    dims, strides = u64s(1, 2, 3, 4), u64s(24, 4, 8, 1)
    # RoPE's checks first ...
    assert call(f, buf(24, 2), u64s(4), u64s(1), 1, tab, tab, 8, 0, cache, 8)[0] == DIM
    st, msg = call(f, buf(24, 2), u64s(1, 2, 4, 3), u64s(24, 12, 3, 1), 4, tab, tab, 8, 0,
                   cache, 8)
    assert st == SHAPE and "head dimension must be positive and even" in msg
    st, _ = call(f, buf(24, 2), dims, strides, 4, buf(16, 2), buf(16, 2), 8, 0, cache, 8)
    assert st == DTYPE
    st, msg = call(f, buf(24, 2), dims, u64s(24, 1, 2, 6), 4, tab, tab, 8, 0, cache, 8)
    assert st == NONCONTIG
    st, msg = call(f, buf(24, 2), dims, strides, 4, tab, tab, 8, 6, cache, 8)
    assert st == SHAPE and "position range is invalid" in msg  # 6 + 3 > 8 table rows
    # ... then the cache write's
    st, msg = call(f, buf(24, 2), dims, strides, 4, tab, tab, 8, 0, buf(2 * 8 * 4, 4), 8)
    assert st == DTYPE and "kv_cache_write_f16" in msg
    st, _ = call(f, buf(24, 2), dims, strides, 4, tab, tab, 8, 5, buf(2 * 6 * 4, 2), 6)
    assert st == POS
    assert call(f, buf(24, 2), dims, strides, 4, tab, tab, 8, 5, cache, 8)[0] == DEVICE


def test_embedding_validation():
    # src/ops/embedding.rs:119-149, then the u32 limits of :171-183
    ids = (ctypes.c_uint32 * 3)(0, 5, 9)
    f = "rl_embedding_f32"
    st, msg = call(f, buf(40, 4), 10, 4, ids, 0, buf(0, 4))
    assert st == SHAPE and "at least one token" in msg
    st, msg = call(f, buf(39, 4), 10, 4, ids, 3, buf(12, 4))
    assert st == SHAPE and "embedding weight has 39 elements" in msg
    st, msg = call("rl_embedding_f16", buf(40, 4), 10, 4, ids, 3, buf(12, 2))
    assert st == SHAPE and "of 2 bytes" in msg
    bad = (ctypes.c_uint32 * 3)(0, 10, 2)
    st, msg = call(f, buf(40, 4), 10, 4, bad, 3, buf(12, 4))
    assert st == TOKEN and "invalid token id 10: vocabulary size is 10" in msg
    # TinyError::InvalidTokenId { token_id, vocab_size } (src/ops/embedding.rs:129-136)
    assert abi.last_error_fields() == (TOKEN, {"token_id": 10, "vocab_size": 10})
    big = (ctypes.c_uint32 * 2)(1, 0xFFFFFFFF)
    assert call(f, buf(40, 4), 10, 4, big, 2, buf(8, 4))[0] == TOKEN
    assert abi.last_error_fields() == (TOKEN, {"token_id": 0xFFFFFFFF, "vocab_size": 10})
    st, msg = call(f, buf(40, 4), 10, 4, ids, 3, buf(11, 4))
    assert st == SHAPE and "output buffer" in msg
    assert call(f, buf(40, 4), 10, 4, ids, 3, buf(12, 4))[0] == DEVICE


def test_qkv_rope_kv_append_validation():
    f = "rl_qkv_rope_kv_append_f16"
    tab = buf(8 * 2, 4)  # [8, 2] tables, head_dim 4
    # Q: [1, 3, 2, 4] permute of [1, 2, 3, 4]; K, V: [1, 1, 2, 4] permutes of [1, 2, 1, 4]
    qd, qs = u64s(1, 3, 2, 4), u64s(24, 4, 12, 1)
    kd, ks = u64s(1, 1, 2, 4), u64s(8, 4, 4, 1)
    kc, vc = buf(1 * 8 * 4, 2), buf(1 * 8 * 4, 2)

    def go(q=None, k=None, v=None, start=0, tables=(tab, tab), q_out=None, kcache=None,
           vcache=None, max_seq=8):
        qb, qdd, qss = q or (buf(24, 2), qd, qs)
        kb, kdd, kss = k or (buf(8, 2), kd, ks)
        vb, vdd, vss = v or (buf(8, 2), kd, ks)
        return call(f, qb, qdd, qss, kb, kdd, kss, vb, vdd, vss, tables[0], tables[1], 8, start,
                    q_out or buf(24, 2), kcache or kc, vcache or vc, max_seq)

    assert go()[0] == DEVICE
    st, msg = go(q=(buf(24, 2), u64s(1, 3, 2, 4), u64s(24, 4, 12, 2)))
    assert st == NONCONTIG and "Q view" in msg
    st, msg = go(k=(buf(6, 2), u64s(1, 1, 2, 3), u64s(6, 3, 3, 1)))
    assert st == SHAPE and "head dimension" in msg
    assert go(tables=(buf(16, 2), buf(16, 2)))[0] == DTYPE
    st, msg = go(start=7)  # 7 + 2 > 8 table rows
    assert st == SHAPE and "position range is invalid" in msg
    st, _ = go(q_out=buf(23, 2))
    assert st == SHAPE
    st, msg = go(v=(buf(16, 2), u64s(1, 2, 2, 4), u64s(16, 8, 4, 1)))
    assert st == FORMAT and "key and value differ" in msg
    st, msg = go(kcache=buf(32, 4))
    assert st == DTYPE and "kv_cache_write_f16" in msg
    st, _ = go(start=5, max_seq=6, kcache=buf(24, 2), vcache=buf(24, 2))
    assert st == POS


def test_qkv_rope_kv_append_repeat_validation():
    # the append's checks first (same as rl_qkv_rope_kv_append_f16), then
    # repeat_kv's (src/tensor/repeat_kv.rs:21-25, :42-44), then the outputs
    f = "rl_qkv_rope_kv_append_repeat_f16"
    tab = buf(8 * 2, 4)
    qd, qs = u64s(1, 3, 2, 4), u64s(24, 4, 12, 1)
    kd, ks = u64s(1, 1, 2, 4), u64s(8, 4, 4, 1)

    def go(start=0, n_rep=3, k_rep=None, v_rep=None, max_seq=8, kcache=None):
        rep = 1 * 1 * n_rep * (start + 2) * 4
        return call(f, buf(24, 2), qd, qs, buf(8, 2), kd, ks, buf(8, 2), kd, ks, tab, tab, 8,
                    start, buf(24, 2), kcache or buf(32, 2), buf(32, 2), max_seq, n_rep,
                    k_rep or buf(rep, 2), v_rep or buf(rep, 2))

    assert go()[0] == DEVICE
    assert go(start=3)[0] == DEVICE
    st, msg = go(n_rep=0)
    assert st == FORMAT and "repeat_kv repeats must be greater than zero" in msg
    st, msg = go(n_rep=0, kcache=buf(32, 4))  # the cache write's check comes first
    assert st == DTYPE and "kv_cache_write_f16" in msg
    st, msg = go(n_rep=1 << 63)  # 1 head x 2^63 fits u64, not u32
    assert st == SHAPE and "exceeds u32" in msg
    kd2, ks2 = u64s(1, 2, 2, 4), u64s(16, 4, 8, 1)  # 2 KV heads: 2 x 2^63 overflows
    st, msg = call(f, buf(24, 2), qd, qs, buf(16, 2), kd2, ks2, buf(16, 2), kd2, ks2, tab, tab,
                   8, 0, buf(24, 2), buf(64, 2), buf(64, 2), 8, 1 << 63, buf(64, 2), buf(64, 2))
    assert st == FORMAT and "head count overflow" in msg
    st, msg = go(start=3, k_rep=buf(3 * 5 * 4 - 1, 2))
    assert st == SHAPE and "repeat_kv" in msg
    st, msg = go(start=3, v_rep=buf(3 * 5 * 4, 4))
    assert st == SHAPE and "repeat_kv" in msg


def test_attention_noalloc_rejects_decode_shapes_beyond_its_scratch():
    # rl_attention_f16_noalloc: the checks of rl_attention_f16, then the decode
    # path's needs against the static scratch (8 MiB - 256 KiB of partials,
    # 1024 counters), all before any device call
    def go(f, b, qh, kvh, kl, hd=64):
        cap = kl
        return call(f, buf(b * qh * hd, 2), buf(b * kvh * cap * hd, 2),
                    buf(b * kvh * cap * hd, 2), b, qh, kvh, 1, kl, hd, cap,
                    ctypes.c_float(0.125), kl - 1, buf(b * qh * hd, 2))

    f = "rl_attention_f16_noalloc"
    assert go(f, 1, 15, 5, 4096)[0] == DEVICE           # SmolLM2 decode: 63 KB of partials
    assert go(f, 64, 32, 1, 32768)[0] == SHAPE          # 2048 rows x 128 splits x 66 floats
    assert "allocation-free entry holds 8126464 bytes" in abi.last_error()
    assert go("rl_attention_f16", 64, 32, 1, 32768)[0] == DEVICE  # the pooled entry takes it
    assert go(f, 1025, 1, 1, 512, 32)[0] == SHAPE       # 1025 hand-off counters > 1024
    assert "1025 counters" in abi.last_error()
    assert go(f, 1024, 1, 1, 512, 32)[0] == DEVICE
    assert go(f, 64, 32, 1, 300)[0] == DEVICE           # < 512 keys: not the split path


@pytest.mark.parametrize("dt,es", [("f32", 4), ("f16", 2)])
def test_attention_validation(dt, es):
    # nn/attention.rs:216-247: gqa_matmul.rs head groups and u32 limits, then the
    # scale/mask checks of attention_scale_mask.rs:120-161, then the buffers
    f = f"rl_attention_{dt}"

    def go(b=1, qh=6, kvh=2, ql=3, kl=5, hd=64, cap=8, scale=0.125, start=2, qn=None, kn=None,
           vn=None, on=None):
        qn = b * qh * ql * hd if qn is None else qn
        kvn = b * kvh * cap * hd
        return call(f, buf(qn, es), buf(kvn if kn is None else kn, es),
                    buf(kvn if vn is None else vn, es), b, qh, kvh, ql, kl, hd, cap,
                    ctypes.c_float(scale), start, buf(b * qh * ql * hd if on is None else on, es))

    assert go()[0] == DEVICE
    assert go(hd=48)[0] == DEVICE and go(hd=512)[0] == DEVICE
    st, msg = go(ql=0)
    assert st == SHAPE and "greater than zero" in msg
    st, msg = go(kvh=4)
    assert st == FORMAT and "Q heads 6 must be divisible by non-zero KV heads 4" in msg
    assert go(kvh=0)[0] == FORMAT
    st, msg = go(kl=9)
    assert st == SHAPE and "KV capacity 8 is smaller than the key length 9" in msg
    st, msg = go(scale=0.0)
    assert st == SHAPE and "scale must be positive and finite" in msg
    assert go(scale=float("inf"))[0] == SHAPE
    st, msg = go(start=3)  # 3 + 3 > 5
    assert st == SHAPE and "query range [3, 6) exceeds key length 5" in msg
    st, msg = go(qn=6 * 3 * 64 - 1)
    assert st == SHAPE and "query buffer" in msg
    st, msg = go(kn=2 * 5 * 64)  # capacity rows, not kv_len rows
    assert st == SHAPE and "key buffer" in msg
    st, msg = go(vn=1)
    assert st == SHAPE and "value buffer" in msg
    st, msg = go(on=5)
    assert st == SHAPE and "attention output buffer" in msg
    st, msg = go(hd=520)
    assert st == SHAPE and "head size 520 exceeds 512" in msg
    st, msg = go(kl=1 << 33, cap=1 << 33, hd=1)
    assert st == SHAPE and "exceeds u32" in msg


@pytest.mark.parametrize("op", ["qk", "pv"])
@pytest.mark.parametrize("dt,es", [("f32", 4), ("f16", 2)])
def test_gqa_matmul_validation(op, dt, es):
    # gqa_matmul.rs: head groups (:174-182), the u32 limits of dispatch (:192-212),
    # then the buffers
    f = f"rl_gqa_{op}_matmul_{dt}"

    def go(b=1, qh=6, kvh=2, ql=3, kl=5, hd=64, cap=8, ln=None, rn=None, on=None):
        left = b * qh * ql * (hd if op == "qk" else kl)
        out = b * qh * ql * (kl if op == "qk" else hd)
        return call(f, buf(left if ln is None else ln, es),
                    buf(b * kvh * cap * hd if rn is None else rn, es), b, qh, kvh, ql, kl, hd,
                    cap, buf(out if on is None else on, es))

    assert go()[0] == DEVICE
    assert go(hd=48)[0] == DEVICE
    st, msg = go(kl=0)
    assert st == SHAPE and "greater than zero" in msg
    st, msg = go(kvh=4)
    assert st == FORMAT and "Q heads 6 must be divisible by non-zero KV heads 4" in msg
    st, msg = go(kl=9)
    assert st == SHAPE and "KV capacity 8 is smaller than the key length 9" in msg
    st, msg = go(ln=7)
    assert st == SHAPE and ("query buffer" in msg or "probability buffer" in msg)
    st, msg = go(rn=7)
    assert st == SHAPE and ("key buffer" in msg or "value buffer" in msg)
    st, msg = go(on=7)
    assert st == SHAPE and "output buffer" in msg
    st, msg = go(kl=1 << 33, cap=1 << 33, hd=1, ql=1, qh=2, kvh=1)
    assert st == SHAPE and "exceeds u32" in msg
