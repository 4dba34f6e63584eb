"""GPU: the autograd mirrors of the reference's `nn` functions (rust_ascend_hip.nn) driven by
torch.autograd, on the reference's own autodiff cases, checking values, gradients and the saved
state of each backward node against src/nn.rs:

* linear_bf16_fp32 / matmul_bf16_fp32 save the BF16 snapshots of both operands
  (LinearBf16Fp32Backward / MatmulBf16Fp32Backward, src/nn.rs:375-453);
* rms_norm saves (x, w, rstd) (RmsNormBackward, src/nn.rs:203-232);
* rotary / rotary_prefix save only the tables (src/nn/rotary.rs:32-105);
* the attention function saves (q, k, v, o, lse).

Reference cases: examples/linear_tensor.rs:24-57 (two shapes, the output used twice, tolerance
5e-4 + 5e-4|b|), examples/rms_norm_tensor.rs:27-59 (18 shapes incl. empty, unaligned and wide rows,
the output used twice, same tolerance), examples/rotary_tensor.rs (tolerance 2e-5 + 1e-4|b|).
"""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import DEV, close, dev_bf16, dev_f32, host, mag_ok, randn_bf16, rel_ok, rows_ok
from rust_ascend_hip import RotaryLayout, Transpose, nn

pytestmark = pytest.mark.gpu


def saved(t):
    """The tensors a custom autograd node saved for its backward."""
    return t.grad_fn.saved_tensors


@pytest.mark.parametrize("m,n,k", [(16, 32, 16), (32, 48, 32)])
def test_linear_bf16_fp32_reference_cases(m, n, k):
    x = ((np.arange(m * k) % 17).astype(np.float32) - 8) * 0.125
    w = ((np.arange(n * k) % 13).astype(np.float32) - 6) * 0.25
    dy = ((np.arange(m * n) % 11).astype(np.float32) - 5) * 0.0625
    x, w, dy = x.reshape(m, k), w.reshape(n, k), dy.reshape(m, n)
    xt = dev_f32(x).requires_grad_()
    wt = dev_f32(w).requires_grad_()
    y = nn.linear_bf16_fp32(xt, wt)
    assert y.shape == (m, n) and y.dtype == torch.float32
    xb, wb = saved(y)
    assert xb.dtype == torch.bfloat16 and wb.dtype == torch.bfloat16
    np.testing.assert_array_equal(host(xb), oracle.bf16_round(x))
    np.testing.assert_array_equal(host(wb), oracle.bf16_round(w))
    up = dev_f32(dy)
    (y * up + y * up).sum().backward()  # the output used twice, as linear_tensor.rs:37
    x64, w64, g = x.astype(np.float64), w.astype(np.float64), 2 * dy.astype(np.float64)
    close(host(y), x64 @ w64.T, 5e-4, 5e-4, "Y")
    close(host(xt.grad), g @ w64, 5e-4, 5e-4, "shared dX")
    close(host(wt.grad), g.T @ x64, 5e-4, 5e-4, "shared dW")
    assert xt.grad.dtype == torch.float32 and wt.grad.shape == (n, k)


@pytest.mark.parametrize("batches", [0, 2])  # 0: rank 2
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_matmul_bf16_fp32_reference_cases(batches, ta, tb):
    """examples/matmul_tensor.rs:14-58: (m, n, k) = (32, 48, 16), dense and 2 batches, every
    transpose pair; gradients in the physical layouts of A and B."""
    m, n, k = 32, 48, 16
    nb = max(batches, 1)
    a = ((np.arange(nb * m * k) % 17).astype(np.float32) - 8) * 0.125
    b = ((np.arange(nb * k * n) % 13).astype(np.float32) - 6) * 0.25
    dy = ((np.arange(nb * m * n) % 11).astype(np.float32) - 5) * 0.0625
    lead = (batches,) if batches else ()
    a = a.reshape(lead + ((k, m) if ta else (m, k)))
    b = b.reshape(lead + ((n, k) if tb else (k, n)))
    dy = dy.reshape(lead + (m, n))
    at, bt = dev_f32(a).requires_grad_(), dev_f32(b).requires_grad_()
    out = nn.matmul_bf16_fp32(at, bt, Transpose(ta), Transpose(tb))
    assert out.shape == lead + (m, n) and out.dtype == torch.float32
    ab, bb = saved(out)
    np.testing.assert_array_equal(host(ab), oracle.bf16_round(a))
    np.testing.assert_array_equal(host(bb), oracle.bf16_round(b))
    out.backward(dev_f32(dy))
    tr = lambda x, t: np.swapaxes(x, -1, -2) if t else x
    a64, b64, g = a.astype(np.float64), b.astype(np.float64), dy.astype(np.float64)
    close(host(out), tr(a64, ta) @ tr(b64, tb), 5e-4, 5e-4, "Y")
    d_opa, d_opb = g @ np.swapaxes(tr(b64, tb), -1, -2), np.swapaxes(tr(a64, ta), -1, -2) @ g
    close(host(at.grad), tr(d_opa, ta), 5e-4, 5e-4, "dA")
    close(host(bt.grad), tr(d_opb, tb), 5e-4, 5e-4, "dB")
    assert at.grad.shape == at.shape and bt.grad.shape == bt.shape


@pytest.mark.parametrize("m,n,k", [(16, 32, 32), (32, 48, 16)])
def test_linear_frozen_bf16_fp32_reference_cases(m, n, k):
    """examples/frozen_bf16_tensor.rs:30-53: F32 X and a fixed BF16 W, the output used twice;
    dX = bf16(2 dY) W (the reference's expectation rounds the doubled upstream), no weight
    gradient, W left bit-identical, and the node keeps only W (src/nn/frozen.rs:59-70)."""
    x = ((np.arange(m * k) % 17) * 0.037 - 0.25).astype(np.float32).reshape(m, k)
    w = ((np.arange(n * k) % 13) * 0.019 - 0.125).astype(np.float32).reshape(n, k)
    dy = ((np.arange(m * n) % 11) * 0.017 - 0.0625).astype(np.float32).reshape(m, n)
    wt = dev_bf16(w)
    before = wt.clone()
    xt = dev_f32(x).requires_grad_()
    y = nn.linear_frozen_bf16_fp32(xt, wt)
    (sw,) = saved(y)
    assert sw.data_ptr() == wt.data_ptr()
    up = dev_f32(dy)
    (y * up + y * up).sum().backward()
    xr, wr = oracle.bf16_round(x).astype(np.float64), oracle.bf16_round(w).astype(np.float64)
    close(host(y), xr @ wr.T, 5e-4, 5e-4, "frozen linear Y")
    close(host(xt.grad), oracle.bf16_round(2 * dy).astype(np.float64) @ wr, 5e-4, 5e-4, "frozen linear shared dX")
    assert torch.equal(wt.view(torch.int16), before.view(torch.int16)) and wt.grad is None


def test_linear_bf16_autograd():
    x_t, x = randn_bf16((256, 384), seed=31)
    w_t, w = randn_bf16((512, 384), seed=32, std=0.05)
    x_t.requires_grad_()
    w_t.requires_grad_()
    y = nn.linear_bf16(x_t, w_t)
    sx, sw = saved(y)
    assert torch.equal(sx, x_t) and torch.equal(sw, w_t)
    dy_t, dy = randn_bf16((256, 512), seed=33)
    y.backward(dy_t)
    rel_ok(host(y), oracle.gemm_f64(x, w, 0, 1), 1e-2, "Y")
    rel_ok(host(x_t.grad), oracle.gemm_f64(dy, w, 0, 0), 1e-2, "dX")
    rel_ok(host(w_t.grad), oracle.gemm_f64(dy, x, 1, 0), 1e-2, "dW")
    assert x_t.grad.dtype == torch.bfloat16 and w_t.grad.dtype == torch.bfloat16


RMS_CASES = [(0, 32), (1, 32), (3, 96), (7, 256), (33, 4096), (0, 4128), (1, 8192), (3, 8224), (0, 7), (1, 1),
             (3, 2), (3, 7), (3, 31), (3, 33), (3, 65), (3, 4095), (3, 4097), (3, 8225)]


@pytest.mark.parametrize("rows,width", RMS_CASES)
def test_rms_norm_autograd_reference_cases(rows, width):
    eps = 1e-3
    w = (0.5 + (np.arange(width) % 7) / 9).astype(np.float32)
    x = ((np.arange(rows * width) % 31) / 7 - 1).astype(np.float32).reshape(1, rows, width)
    dy = ((np.arange(rows * width) % 11) / 5 - 0.7).astype(np.float32).reshape(1, rows, width)
    xt, wt = dev_f32(x).requires_grad_(), dev_f32(w).requires_grad_()
    y = nn.rms_norm(xt, wt, eps)
    sx, sw, rstd = saved(y)
    assert torch.equal(sx, xt) and torch.equal(sw, wt) and rstd.shape == (rows,) and rstd.dtype == torch.float32
    up = dev_f32(dy)
    (y * up + y * up).sum().backward()  # rms_norm_tensor.rs:41
    y_ref, r_ref = oracle.rms_norm_f64(x.reshape(rows, width), w, eps)
    dx_ref, dw_ref = oracle.rms_norm_backward_f64(x.reshape(rows, width), w, 2 * dy.reshape(rows, width), r_ref)
    close(host(y).reshape(rows, width), y_ref, 5e-4, 5e-4, "Y")
    close(host(rstd), r_ref, 1e-6, 1e-6, "saved rstd")
    close(host(xt.grad).reshape(rows, width), dx_ref, 5e-4, 5e-4, "dX")
    close(host(wt.grad), dw_ref, 5e-4, 5e-4, "dWeight")


def test_rms_norm_autograd_bf16_input():
    x_t, x = randn_bf16((64, 4096), seed=35)
    w = (1 + 0.1 * oracle.normal((4096,), 35, 2)).astype(np.float32)
    x_t.requires_grad_()
    wt = dev_f32(w).requires_grad_()
    y = nn.rms_norm(x_t, wt, 1e-6)
    dy_t, dy = randn_bf16((64, 4096), seed=36)
    y.backward(dy_t)
    y_ref, r_ref = oracle.rms_norm_f64(x, w, 1e-6)
    dx_ref, dw_ref = oracle.rms_norm_backward_f64(x, w, dy, r_ref)
    assert y.dtype == torch.bfloat16 and x_t.grad.dtype == torch.bfloat16 and wt.grad.dtype == torch.float32
    rel_ok(host(y), y_ref, 1e-2, "Y")
    rel_ok(host(x_t.grad), dx_ref, 1e-2, "dX")
    rel_ok(host(wt.grad), dw_ref, 1e-4, "dW", atol_frac=1e-3)


@pytest.mark.parametrize("rows,width", [(1, 2), (3, 6), (2, 96)])
@pytest.mark.parametrize("layout", [0, 1])
def test_rotary_autograd(rows, width, layout):
    x = oracle.normal((rows, width), 41, width)
    ang = ((np.arange(rows * width // 2) % 23) * 0.125).reshape(rows, width // 2)  # rotary_tensor.rs:23-30
    c, s = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    dy = oracle.normal((rows, width), 42, width)
    xt = dev_f32(x).requires_grad_()
    ct, st = dev_f32(c), dev_f32(s)
    y = nn.rotary(xt, ct, st, RotaryLayout(layout))
    assert [t.data_ptr() for t in saved(y)] == [ct.data_ptr(), st.data_ptr()]  # only the tables are kept
    y.backward(dev_f32(dy))
    close(host(y), oracle.rotary_f64(x, c, s, layout), 2e-5, 1e-4, "Y")
    close(host(xt.grad), oracle.rotary_f64(dy, c, s, layout, backward=True), 2e-5, 1e-4, "dX")


@pytest.mark.parametrize("layout", [0, 1])
def test_rotary_prefix_autograd_broadcast_tables(layout):
    x_t, x = randn_bf16((2, 4, 64, 96), seed=43)
    cos, sin = oracle.rope_tables(np.arange(64), 64, 5e5)
    ct, st = dev_f32(cos[None, None]), dev_f32(sin[None, None])
    x_t.requires_grad_()
    y = nn.rotary_prefix(x_t, ct, st, 64, RotaryLayout(layout))
    dy_t, dy = randn_bf16((2, 4, 64, 96), seed=44)
    y.backward(dy_t)
    rel_ok(host(y), oracle.rotary_prefix(x, cos[None, None], sin[None, None], 64, layout), 1e-2, "Y")
    rel_ok(host(x_t.grad), oracle.rotary_prefix(dy, cos[None, None], sin[None, None], 64, layout, True), 1e-2, "dX")
    np.testing.assert_array_equal(host(x_t.grad)[..., 64:], dy[..., 64:])  # the tail passes through


@pytest.mark.parametrize("causal", [False, True])
def test_attention_autograd_saved_state_and_grads(causal):
    B, H, HKV, M, N, D = 2, 8, 2, 192, 192, 128
    q_t, q = randn_bf16((B, H, M, D), seed=45)
    k_t, k = randn_bf16((B, HKV, N, D), seed=46)
    v_t, v = randn_bf16((B, HKV, N, D), seed=47)
    for t in (q_t, k_t, v_t):
        t.requires_grad_()
    scale = D ** -0.5
    if causal:
        o = nn.causal_grouped_query_attention_bf16(q_t, k_t, v_t, scale)
    else:
        o = nn.grouped_query_attention_bf16(q_t, k_t, v_t, scale)
    sq, sk, sv, so, slse = saved(o)
    assert torch.equal(sq, q_t) and torch.equal(sk, k_t) and torch.equal(sv, v_t) and torch.equal(so, o)
    assert slse.shape == (B, H, M) and slse.dtype == torch.float32
    do_t, do = randn_bf16((B, H, M, D), seed=48)
    o.backward(do_t)
    ref = oracle.attention_f64(q, k, v, do, scale=scale, causal=causal, magnitudes=True)
    mag_ok(host(o), ref["out"], ref["out_mag"], 1e-2, "O")
    rows_ok(host(o), ref["out"], 1e-2, "O rows")
    close(host(slse), ref["lse"], 1e-3, 1e-4, "saved lse")
    for name, t in (("dq", q_t), ("dk", k_t), ("dv", v_t)):
        assert t.grad.dtype == torch.bfloat16 and t.grad.shape == t.shape
        mag_ok(host(t.grad), ref[name], ref[name + "_mag"], 1e-2, name)
