"""One SmolLM2-360M-shaped decoder layer's non-GEMM chain in f16 at a
4096-token prefill, run on device buffers with each stage's output feeding
the next, in the order of TransformerBlock::forward_encode
(nn/transformer_block.rs:128-158) and SelfAttention (nn/attention.rs:195-247):

  1. RMSNorm            x [4096, 960] -> xn
  2. RoPE (theta 1e4)   Q = xn seen as [1, 15, 4096, 64] and K = xn[:, 0:320]
                        seen as [1, 5, 4096, 64] (the projections' strided
                        views, rotated in place of their gather) -> qr, kr
  3. repeat_kv 5 -> 15  kr -> kq; V = xn[:, 320:640] gathered -> vc -> vq
     (QK^T on the matrix cores: qr x kq^T -> scores [15, 4096, 4096])
  4. scale/mask + softmax (causal, scale 1/8) -> p
     (PV -> [1, 15, 4096, 64], heads merged by contiguous -> attn [4096, 960])
  5. residual add       h = x + attn
  6. SwiGLU             [4096, 2560] -> act
  7. residual add       out = h + act[:, 0:960] (gathered)

The dense projections between the stages are out of scope, so the chain
takes views of its own tensors where a projection would sit (Q/K/V are
slices of xn; the down projection's output is a slice of act); the FFN's
gate/up projections are the one place with no such view, so SwiGLU reads
seeded N(0, 1) gate/up tensors.  Every stage is compared with the oracle
applied to that stage's actual GPU inputs, at the parity bars of the ops:
bit-exact RoPE, repeat_kv, gathers and adds; f16 RMSNorm, softmax and SwiGLU
within 2 ulp (masked probabilities exactly 0); the two products within the
float64 forward error bounds the attention tests use.
"""

import os

import numpy as np
import pytest

from helpers import U32, assert_bitexact, f16_ulp_distance, gqa_expand, ulp16
from oracle import oracle as o
from rustllm_amd import abi, synth

pytestmark = pytest.mark.gpu

o.set_threads(min(16, os.cpu_count() or 1))

T, HID, QH, KVH, HD, FFN = 4096, 960, 15, 5, 64, 2560
F16 = np.float16


def seeded(tag, shape, lo=None, hi=None):
    seed = synth.seed_for("c5-chain", tag, *shape)
    if lo is not None:
        return synth.uniform_range(seed, shape, lo, hi, F16)
    return synth.normal(seed, shape, 0.0, 1.0, F16)


def window(buf, first, count, shape):
    """A non-owning rl_buffer over elements first .. first + count of `buf`."""
    raw = abi.RlBuffer(buf.ptr + first * buf.dtype.itemsize, count, count * buf.dtype.itemsize)
    view = abi.DeviceBuffer.__new__(abi.DeviceBuffer)
    view.ctx, view.raw, view.dtype, view.shape = buf.ctx, raw, buf.dtype, tuple(shape)
    view.release = lambda: None
    return view


def step(ctx, fn):
    ctx.begin()
    out = fn()
    ctx.finish()
    return out


def ulp_ok(got, ref, what):
    d = f16_ulp_distance(got, ref)
    assert d <= 2, f"{what}: {d} ulp"


def test_smollm_layer_chain_f16(ctx):
    x = seeded("x", (T, HID))
    w = seeded("w", (HID,), 0.5, 1.5)
    gate, up = seeded("gate", (T, FFN)), seeded("up", (T, FFN))
    cos, sin = o.rope_table(HD, T, 10000.0)
    dx, dw = ctx.upload(x), ctx.upload(w)
    dcos, dsin = ctx.upload(cos), ctx.upload(sin)

    # 1. RMSNorm
    dxn = step(ctx, lambda: ctx.rmsnorm(dx, dw, 1e-5))
    xn = dxn.numpy()
    ulp_ok(xn, o.rmsnorm(x, w, 1e-5), "1 rmsnorm [4096, 960]")

    # 2. RoPE of the Q and K projections' [1, H, T, D] views of xn
    q_dims, q_strides = [1, QH, T, HD], [T * HID, HD, HID, 1]
    k_dims, k_strides = [1, KVH, T, HD], [T * HID, HD, HID, 1]
    dqr = step(ctx, lambda: ctx.rope_strided(dxn, q_dims, q_strides, dcos, dsin, 0))
    dkr = step(ctx, lambda: ctx.rope_strided(dxn, k_dims, k_strides, dcos, dsin, 0))
    q_view = np.ascontiguousarray(xn.reshape(1, T, QH, HD).transpose(0, 2, 1, 3))
    k_view = np.ascontiguousarray(xn[:, :KVH * HD].reshape(1, T, KVH, HD).transpose(0, 2, 1, 3))
    qr, kr = dqr.numpy(), dkr.numpy()
    assert_bitexact(qr, o.rope(q_view, cos, sin, 0), "2 rope Q [1, 15, 4096, 64]")
    assert_bitexact(kr, o.rope(k_view, cos, sin, 0), "2 rope K [1, 5, 4096, 64]")

    # 3. repeat_kv of K and of V (V gathered from its view of xn first)
    dv_view = window(dxn, KVH * HD, T * HID - KVH * HD, (T * HID - KVH * HD,))
    dvc = step(ctx, lambda: ctx.contiguous(dv_view, k_dims, k_strides))
    vc = dvc.numpy()
    assert_bitexact(vc, np.ascontiguousarray(
        xn[:, KVH * HD:2 * KVH * HD].reshape(1, T, KVH, HD).transpose(0, 2, 1, 3)),
        "3 V gather [1, 5, 4096, 64]")
    dkq = step(ctx, lambda: ctx.repeat_kv(dkr, QH // KVH))
    dvq = step(ctx, lambda: ctx.repeat_kv(dvc, QH // KVH))
    assert_bitexact(dkq.numpy(), o.repeat_kv(kr, QH // KVH), "3 repeat_kv K 5 -> 15")
    assert_bitexact(dvq.numpy(), o.repeat_kv(vc, QH // KVH), "3 repeat_kv V 5 -> 15")

    # QK^T of the rotated queries and repeated keys (sampled rows vs float64)
    dscores = step(ctx, lambda: ctx.gqa_qk(dqr, dkq))
    scores = dscores.numpy()
    kq64 = gqa_expand(kr, QH, T)
    for r in (0, 1, 127, 2048, 4095):
        q64 = qr[:, :, r:r + 1].astype(np.float64)
        exact = np.matmul(q64, np.swapaxes(kq64, -1, -2))
        dot_abs = np.matmul(np.abs(q64), np.swapaxes(np.abs(kq64), -1, -2))
        bound = HD * U32 * dot_abs + ulp16(exact) * 0.5001
        assert np.all(np.abs(scores[:, :, r:r + 1].astype(np.float64) - exact) <= bound), r

    # 4. causal scale/mask + softmax of those scores
    dp = step(ctx, lambda: ctx.attention_softmax(dscores, 0.125, 0))
    p = dp.numpy()
    ref = o.attention_softmax(scores, 0.125, 0)
    ulp_ok(p, ref, "4 scale/mask + softmax [15, 4096, 4096]")
    del ref
    upper = np.triu(np.ones((T, T), bool), 1)
    for h in range(QH):
        assert not p[0, h][upper].any(), f"4 masked probability non-zero in head {h}"
    del scores, dscores

    # PV with the repeated values, heads merged back to [4096, 960]
    dctx_out = step(ctx, lambda: ctx.gqa_pv(dp, dvq))
    ctx_out = dctx_out.numpy()
    ve = gqa_expand(vc, QH, T)
    for r in (0, 1, 127, 2048, 4095):
        pr = p[:, :, r:r + 1].astype(np.float64)
        exact = np.matmul(pr, ve)
        weight = np.matmul(pr, np.abs(ve))
        bound = T * U32 * weight + ulp16(exact) * 0.5001
        assert np.all(np.abs(ctx_out[:, :, r:r + 1].astype(np.float64) - exact) <= bound), r
    del p
    dattn = step(ctx, lambda: ctx.contiguous(dctx_out, [1, T, QH, HD],
                                             [QH * T * HD, HD, T * HD, 1]))
    attn = dattn.numpy().reshape(T, HID)
    assert_bitexact(attn, np.ascontiguousarray(ctx_out.transpose(0, 2, 1, 3)).reshape(T, HID),
                    "heads merged [4096, 960]")

    # 5. first residual add
    dh = step(ctx, lambda: ctx.add(dx, dattn))
    h = dh.numpy()
    assert_bitexact(h, o.add(x, attn), "5 residual add [4096, 960]")

    # 6. SwiGLU [4096, 2560]
    dact = step(ctx, lambda: ctx.swiglu(ctx.upload(gate), ctx.upload(up)))
    act = dact.numpy()
    ulp_ok(act, o.swiglu(gate, up), "6 swiglu [4096, 2560]")

    # 7. second residual add, with the first 960 columns of act in the down
    #    projection's place
    ddown = step(ctx, lambda: ctx.contiguous(dact, [T, HID], [FFN, 1]))
    down = ddown.numpy()
    assert_bitexact(down, np.ascontiguousarray(act[:, :HID]), "7 gather act[:, :960]")
    dout = step(ctx, lambda: ctx.add(dh, ddown))
    assert_bitexact(dout.numpy(), o.add(h, down), "7 residual add [4096, 960]")
