"""GPU parity: the SwiGLU gate SiLU(gate) * up and its backward through the C ABI, against the
float64 oracle with the reference's own inputs and tolerance (examples/silu_mul_tensor.rs:9,
25-44: |a-b| <= 2e-5 + 1e-4|b|), the shared-gate gradient (:51-53), the C5 feed-forward shape,
BF16 storage, unaligned and ragged tensors, the input checks of runtime/elementwise.rs:5-11 and
the swiglu_bf16_fp32 composition of src/nn/feed_forward.rs:24-42."""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import DEV, close, dev_bf16, dev_f32, host, mag_ok, rel_ok
from rust_ascend_hip import HipRuntime, HkError, nn

pytestmark = pytest.mark.gpu

TOL = (2e-5, 1e-4)


def reference_inputs(n):
    i = np.arange(n)
    x = ((i % 41).astype(np.float32) * np.float32(0.6) - np.float32(12.0)).astype(np.float32)
    u = ((i % 13).astype(np.float32) * np.float32(0.125) - np.float32(0.5)).astype(np.float32)
    dy = ((i % 7).astype(np.float32) * np.float32(0.25) - np.float32(0.75)).astype(np.float32)
    return x.reshape(1, n), u.reshape(1, n), dy.reshape(1, n)


@pytest.mark.parametrize("n", [0, 1, 65, 1025])
def test_silu_mul_reference_cases(n):
    x, u, dy = reference_inputs(n)
    y = HipRuntime.silu_mul(dev_f32(x), dev_f32(u))
    assert y.shape == (1, n) and y.dtype == torch.float32
    close(host(y), oracle.silu_mul_f64(x, u), *TOL, "Y")
    dg, du = HipRuntime.silu_mul_backward(dev_f32(x), dev_f32(u), dev_f32(dy))
    want_dg, want_du = oracle.silu_mul_backward_f64(x, u, dy)
    close(host(dg), want_dg, *TOL, "dGate")
    close(host(du), want_du, *TOL, "dUp")
    # through autograd: d/d(inputs) of sum(Y * dY)
    g = dev_f32(x).requires_grad_(True)
    up = dev_f32(u).requires_grad_(True)
    (nn.silu_mul(g, up) * dev_f32(dy)).sum().backward()
    close(host(g.grad), want_dg, *TOL, "autograd dGate")
    close(host(up.grad), want_du, *TOL, "autograd dUp")


def test_silu_mul_shared_gate():
    x, _, dy = reference_inputs(1025)
    g = dev_f32(x).requires_grad_(True)
    (nn.silu_mul(g, g) * dev_f32(dy)).sum().backward()
    a = x.astype(np.float64)
    s = 1 / (1 + np.exp(-a))
    want = dy.astype(np.float64) * (a * (s * (1 + a * (1 - s))) + a * s)  # silu_mul_tensor.rs:45
    close(host(g.grad), want, *TOL, "shared gate")


@pytest.mark.parametrize("shape", [(4096, 14336), (3, 1023), (7,), (2, 5, 9)])
def test_silu_mul_random_f32(shape):
    g = oracle.normal(shape, seed=sum(shape), stream=61, std=3.0)
    u = oracle.normal(shape, seed=sum(shape), stream=62)
    dy = oracle.normal(shape, seed=sum(shape), stream=63)
    y = host(HipRuntime.silu_mul(dev_f32(g), dev_f32(u)))
    close(y, oracle.silu_mul_f64(g, u), *TOL, "Y")
    dg, du = HipRuntime.silu_mul_backward(dev_f32(g), dev_f32(u), dev_f32(dy))
    want_dg, want_du = oracle.silu_mul_backward_f64(g, u, dy)
    close(host(dg), want_dg, *TOL, "dGate")
    close(host(du), want_du, *TOL, "dUp")


def test_silu_mul_bf16_storage():
    shape = (2048, 14336)  # C5's feed-forward activation for 2 x 2048 tokens
    g = oracle.bf16_round(oracle.normal(shape, seed=5, stream=64, std=2.0))
    u = oracle.bf16_round(oracle.normal(shape, seed=5, stream=65))
    dy = oracle.bf16_round(oracle.normal(shape, seed=5, stream=66))
    y = HipRuntime.silu_mul(dev_bf16(g), dev_bf16(u))
    assert y.dtype == torch.bfloat16
    # F32 arithmetic, one BF16 rounding of each output
    np.testing.assert_array_equal(host(y), oracle.bf16_round(host(HipRuntime.silu_mul(dev_f32(g), dev_f32(u)))))
    rel_ok(host(y), oracle.silu_mul_f64(g, u), 1e-2, "Y bf16")
    dg, du = HipRuntime.silu_mul_backward(dev_bf16(g), dev_bf16(u), dev_bf16(dy))
    want_dg, want_du = oracle.silu_mul_backward_f64(g, u, dy)
    rel_ok(host(dg), want_dg, 1e-2, "dGate bf16")
    rel_ok(host(du), want_du, 1e-2, "dUp bf16")


def test_silu_mul_unaligned_views():
    base = oracle.normal((4 * 1000 + 3,), seed=9, stream=67)
    g_all, u_all = dev_f32(base), dev_f32(base[::-1].copy())
    g, u = g_all[1:1001], u_all[3:1003]  # 4-byte aligned, not 16-byte aligned
    y = host(HipRuntime.silu_mul(g, u))
    close(y, oracle.silu_mul_f64(host(g), host(u)), *TOL, "unaligned")


def test_silu_mul_rejects_bad_inputs():
    a = torch.zeros((4, 8), device=DEV)
    with pytest.raises(HkError):
        HipRuntime.silu_mul(a, torch.zeros((4, 9), device=DEV))
    with pytest.raises(HkError):
        HipRuntime.silu_mul(a, a.to(torch.bfloat16))
    with pytest.raises(HkError):
        HipRuntime.silu_mul(a.half(), a.half())
    with pytest.raises(HkError):
        HipRuntime.silu_mul_backward(a, a, torch.zeros((8, 4), device=DEV))


def test_swiglu_bf16_fp32_composition():
    m, k, h, n = 64, 128, 256, 96
    x = oracle.normal((m, k), seed=3, stream=70)
    wg = oracle.normal((h, k), seed=3, stream=71, std=0.05)
    wu = oracle.normal((h, k), seed=3, stream=72, std=0.05)
    wd = oracle.normal((n, h), seed=3, stream=73, std=0.05)
    y = host(nn.swiglu_bf16_fp32(dev_f32(x), dev_f32(wg), dev_f32(wu), dev_f32(wd)))
    xb, gb, ub, db = (oracle.bf16_round(t) for t in (x, wg, wu, wd))
    gate = oracle.gemm_f64(xb, gb, 0, 1)
    up = oracle.gemm_f64(xb, ub, 0, 1)
    act = oracle.bf16_round(oracle.silu_mul_f64(gate.astype(np.float32), up.astype(np.float32)).astype(np.float32))
    # The activation is rounded to BF16 before the down projection, so a last-bit difference in
    # the F32 gate can move one term by a BF16 ulp (2^-8 of |act| |down|): where an output
    # cancels to ~0 that is unbounded relative to the output, hence the magnitude criterion.
    magnitude = np.abs(act).astype(np.float64) @ np.abs(db).T.astype(np.float64)
    mag_ok(y, oracle.gemm_f64(act, db, 0, 1), magnitude, 1e-2, "SwiGLU")
    with pytest.raises(ValueError):
        nn.swiglu_bf16_fp32(dev_f32(x[:, :120]), dev_f32(wg[:, :120]), dev_f32(wu[:, :120]), dev_f32(wd))
