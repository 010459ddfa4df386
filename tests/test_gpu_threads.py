"""Contexts on several host threads at once (one context per thread, as
MetalContext is per thread: src/metal/context.rs:14-17).

Each thread owns a context -- its own stream and buffer pool -- and runs a
batch of ops over and over on its own inputs while the others do the same;
every thread's results must equal the oracle's (the bars of the parity
tests), and a validation error raised on one thread must leave the other
threads' last-error message and payload untouched (they are per thread).
"""

import threading

import numpy as np
import pytest

from helpers import assert_bitexact, f16_ulp_distance, max_rel_err
from oracle import oracle as o
from rustllm_amd import abi, synth

pytestmark = pytest.mark.gpu

TINY = np.finfo(np.float32).tiny


def _worker(index, rounds, failures, barrier):
    dtype = np.float16 if index % 2 else np.float32
    shape = (64 + 7 * index, 1000 + 3 * index)
    x = synth.normal(synth.seed_for("thread-x", index), shape, 0.0, 1.0, dtype)
    y = synth.normal(synth.seed_for("thread-y", index), shape, 0.0, 1.0, dtype)
    w = synth.uniform_range(synth.seed_for("thread-w", index), (shape[1],), 0.5, 1.5, dtype)
    ref_add, ref_rms = o.add(x, y), o.rmsnorm(o.add(x, y), w, 1e-5)
    ref_sm = o.attention_softmax(x, 0.125, shape[1] - shape[0])
    try:
        with abi.Context(0) as ctx:
            dx, dy, dw = ctx.upload(x), ctx.upload(y), ctx.upload(w)
            s, n, p = ctx.empty(shape, dtype), ctx.empty(shape, dtype), ctx.empty(shape, dtype)
            barrier.wait()
            for r in range(rounds):
                ctx.begin()
                ctx.add(dx, dy, s)
                ctx.rmsnorm(s, dw, 1e-5, n)
                ctx.attention_softmax(dx, 0.125, shape[1] - shape[0], p)
                ctx.finish()
                if index == 0 and r == rounds // 2:
                    # a validation error on this thread only: a scale that is
                    # not positive
                    with pytest.raises(abi.RustLLMError, match="scale must be positive"):
                        ctx.scale_mask(dx, -1.0, 0, p)
            assert_bitexact(s.numpy(), ref_add, f"thread {index}: add")
            got_n, got_p = n.numpy(), p.numpy()
            if dtype == np.float16:
                assert f16_ulp_distance(got_n, ref_rms) <= 2, f"thread {index}: rmsnorm"
                assert f16_ulp_distance(got_p, ref_sm) <= 2, f"thread {index}: softmax"
            else:
                assert max_rel_err(got_n, ref_rms, TINY) <= 1e-5, f"thread {index}: rmsnorm"
                assert max_rel_err(got_p, ref_sm, TINY) <= 1e-5, f"thread {index}: softmax"
            msg = abi.last_error()
            if index == 0:
                assert "scale must be positive" in msg, f"thread 0 lost its own error: {msg}"
            else:
                assert "scale must be positive" not in msg, \
                    f"thread {index} sees another thread's error: {msg}"
    except BaseException as e:  # reported by the main thread (pytest's Failed included)
        failures.append(f"thread {index}: {e!r}")


@pytest.mark.parametrize("threads", [2, 4])
def test_contexts_on_concurrent_threads(threads):
    failures: list[str] = []
    barrier = threading.Barrier(threads)
    pool = [threading.Thread(target=_worker, args=(i, 40, failures, barrier))
            for i in range(threads)]
    for t in pool:
        t.start()
    for t in pool:
        t.join(timeout=100)
    assert not any(t.is_alive() for t in pool), "a worker thread did not finish"
    assert not failures, "; ".join(failures)
