"""GPU parity of the decoder layer's fused feed-forward GEMMs, through the C ABI:

* hk_linear_residual: y = residual + x W^T, the add in the GEMM epilogue;
* hk_swiglu_projection: gate and up as one GEMM over W_gu (gate and up rows interleaved in blocks
  of 16) with SiLU(gate) * up in the epilogue;
* hk_swiglu_projection_backward: dM = dY Wd with the SwiGLU backward in the epilogue, written as
  the interleaved [dgate | dup].

Where the unfused composition runs the same 256x256 tile kernel (grids of at least 256 tiles), the
fused results must equal it bit for bit: hk_gemm_into (BF16 output) followed by hk_bias_add,
hk_silu_mul or hk_silu_mul_backward, which themselves are pinned to the oracle (the reference's
silu_mul programs, rust-ascend-compiler/src/ascend/programs.rs:21-46, and affine add,
src/nn/affine.rs:14-25) in test_gpu_swiglu.py and test_gpu_embedding_bias.py. Smaller shapes run
another kernel in the unfused composition and are checked against the float64 oracle on the same
BF16 values: per row normwise <= 1e-2 (an element of a sum or a SiLU product can cancel to ~0 while
its rounding stays ~2^-9 of the terms)."""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import DEV, host
from rust_ascend_hip import HipRuntime, HkError, runtime

pytestmark = pytest.mark.gpu


def call(name, *tensors):
    runtime._call(name, *(runtime.desc(t) for t in tensors))


def randn(shape, seed, scale=1.0):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    return (torch.randn(shape, generator=g, device=DEV) * scale).to(torch.bfloat16)


def interleave(wg, wu):
    """W_gu [2F, H]: row 32 b + r = gate row 16 b + r (r < 16), up row 16 b + r - 16."""
    f, h = wg.shape
    return torch.stack([wg.view(f // 16, 16, h), wu.view(f // 16, 16, h)], dim=1).reshape(2 * f, h).contiguous()


def deinterleave(t, f):
    t = t.view(t.shape[0], f // 16, 2, 16)
    return t[:, :, 0].reshape(t.shape[0], f), t[:, :, 1].reshape(t.shape[0], f)


def row_ok(got, want, name):
    e = oracle.row_err(host(got), want)
    assert e <= 1e-2, (name, e)


# ------------------------------------------------------------------ projection + residual

@pytest.mark.parametrize("m,n,k", [(4096, 4096, 4096), (4096, 4096, 14336), (8192, 4096, 1000 + 8)])
def test_linear_residual_bit_exact_with_gemm_and_add(m, n, k):
    x, w, r = randn((m, k), m + k, k ** -0.5), randn((n, k), n + k + 1, 1.0), randn((m, n), m + n + 2)
    y = torch.empty((m, n), device=DEV, dtype=torch.bfloat16)
    print(f"linear residual {m}x{n}x{k}", flush=True)
    call("hk_linear_residual", x, w, r, y)
    a = torch.empty_like(y)
    HipRuntime.gemm_into(x, w, 0, 1, a)
    want = HipRuntime.bias_add(a, None, r)
    assert torch.equal(y, want)


@pytest.mark.parametrize("m,n,k", [(1, 16, 8), (100, 48, 200), (300, 256, 64)])
def test_linear_residual_small_vs_oracle(m, n, k):
    x, w, r = randn((m, k), m + k), randn((n, k), n + k + 1), randn((m, n), m + n + 2)
    y = torch.empty((m, n), device=DEV, dtype=torch.bfloat16)
    call("hk_linear_residual", x, w, r, y)
    want = oracle.bf16_round(oracle.gemm_f64(host(x), host(w), False, True)) + host(r)
    row_ok(y, want, "y")


# ------------------------------------------------------------------ SwiGLU forward

@pytest.mark.parametrize("t,f,h", [(4096, 14336, 4096), (8192, 2048, 1000 + 8)])
def test_swiglu_projection_bit_exact_with_gemms_and_silu_mul(t, f, h):
    x, wg, wu = randn((t, h), t + h, h ** -0.5), randn((f, h), f + h), randn((f, h), f + h + 1)
    w_gu = interleave(wg, wu)
    gate, up, act = (torch.empty((t, f), device=DEV, dtype=torch.bfloat16) for _ in range(3))
    print(f"swiglu projection {t}x{f}x{h}", flush=True)
    call("hk_swiglu_projection", x, w_gu, gate, up, act)
    g2, u2 = torch.empty_like(gate), torch.empty_like(up)
    HipRuntime.gemm_into(x, wg, 0, 1, g2)
    HipRuntime.gemm_into(x, wu, 0, 1, u2)
    assert torch.equal(gate, g2) and torch.equal(up, u2)
    assert torch.equal(act, HipRuntime.silu_mul(g2, u2))


@pytest.mark.parametrize("t,f,h", [(1, 16, 8), (100, 48, 200), (300, 160, 64)])
def test_swiglu_projection_small_vs_oracle(t, f, h):
    x, wg, wu = randn((t, h), t + h), randn((f, h), f + h), randn((f, h), f + h + 1)
    gate, up, act = (torch.empty((t, f), device=DEV, dtype=torch.bfloat16) for _ in range(3))
    call("hk_swiglu_projection", x, interleave(wg, wu), gate, up, act)
    gw = oracle.bf16_round(oracle.gemm_f64(host(x), host(wg), False, True))
    uw = oracle.bf16_round(oracle.gemm_f64(host(x), host(wu), False, True))
    row_ok(gate, gw, "gate")
    row_ok(up, uw, "up")
    row_ok(act, oracle.silu_mul_f64(gw, uw), "act")


# ------------------------------------------------------------------ SwiGLU backward

@pytest.mark.parametrize("t,f,h", [(4096, 14336, 4096), (8192, 2048, 1000 + 8)])
def test_swiglu_backward_bit_exact_with_gemm_and_silu_mul_backward(t, f, h):
    dy, wd = randn((t, h), t + h), randn((h, f), f + h, f ** -0.5)
    gate, up = randn((t, f), t + f), randn((t, f), t + f + 1)
    dgu = torch.empty((t, 2 * f), device=DEV, dtype=torch.bfloat16)
    print(f"swiglu projection backward {t}x{f}x{h}", flush=True)
    call("hk_swiglu_projection_backward", dy, wd, gate, up, dgu)
    dm = torch.empty((t, f), device=DEV, dtype=torch.bfloat16)
    HipRuntime.gemm_into(dy, wd, 0, 0, dm)
    dg, du = HipRuntime.silu_mul_backward(gate, up, dm)
    got_g, got_u = deinterleave(dgu, f)
    assert torch.equal(got_g, dg) and torch.equal(got_u, du)


@pytest.mark.parametrize("t,f,h", [(1, 16, 8), (100, 48, 200), (300, 160, 64)])
def test_swiglu_backward_small_vs_oracle(t, f, h):
    dy, wd = randn((t, h), t + h), randn((h, f), f + h)
    gate, up = randn((t, f), t + f), randn((t, f), t + f + 1)
    dgu = torch.empty((t, 2 * f), device=DEV, dtype=torch.bfloat16)
    call("hk_swiglu_projection_backward", dy, wd, gate, up, dgu)
    dm = oracle.bf16_round(oracle.gemm_f64(host(dy), host(wd), False, False))
    want_g, want_u = oracle.silu_mul_backward_f64(host(gate), host(up), dm)
    got_g, got_u = deinterleave(dgu, f)
    row_ok(got_g, want_g, "dgate")
    row_ok(got_u, want_u, "dup")


def test_fused_ffn_reject_bad_inputs():
    x = randn((64, 256), 1)
    w = randn((32 * 2, 256), 2)
    out = torch.empty((64, 32), device=DEV, dtype=torch.bfloat16)
    with pytest.raises(HkError):  # F % 16 != 0 (F = 24)
        call("hk_swiglu_projection", x, randn((48, 256), 3), out[:, :24].contiguous(), out[:, :24].contiguous(),
             out[:, :24].contiguous())
    with pytest.raises(HkError):  # residual shape
        call("hk_linear_residual", x, w, torch.empty((64, 32), device=DEV, dtype=torch.bfloat16),
             torch.empty((64, 64), device=DEV, dtype=torch.bfloat16))
    with pytest.raises(HkError):  # K % 8 != 0
        call("hk_linear_residual", randn((64, 20), 4), randn((64, 20), 5), randn((64, 64), 6),
             torch.empty((64, 64), device=DEV, dtype=torch.bfloat16))
    with pytest.raises(HkError):  # output aliases the residual
        r = randn((64, 64), 7)
        call("hk_linear_residual", x, w, r, r)
