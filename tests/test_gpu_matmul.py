"""GPU parity of the generic floating matmul (hk_tensor_matmul / hk_tensor_matmul_backward; the
reference's RudaAscend::float_matmul -> AscendRuntime::tensor_matmul, src/backend.rs:692-703,
rust-ascend-driver/src/tensor/runtime/generic_matrix.rs, worker.rs:128-162 KEEP_DTYPE) against the
f64 oracle: F32, F16 and BF16 in and out, batch dims broadcast at ranks 2 to 6, ragged M/N/K, an
empty contraction (zeros), empty outputs, more than 4096 batches, and the gradients with their
broadcast sums through torch autograd (nn.float_matmul).

Tolerances: F32 out 2e-5 (relative, FP32 products and sums over K <= 260); F16 out 2e-3 (its
2^-11 rounding); BF16 out max rel err 1e-2."""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import DEV, close, host, rel_ok
from rust_ascend_hip import HipRuntime, HkError, nn

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]
SHAPES = [((2, 1, 3, 5), (1, 4, 5, 7)), ((37, 45), (45, 29)), ((3, 64, 128), (128, 96)),
          ((2, 3, 1, 17, 33), (3, 1, 33, 9)), ((4, 512, 256), (4, 256, 384)), ((1, 1, 2, 1, 70, 130), (3, 130, 65)),
          ((2, 260, 16), (16, 260))]


def dev(shape, dtype, seed, std=1.0):
    x = np.random.default_rng(seed).standard_normal(shape).astype(np.float32) * std
    t = torch.from_numpy(x).to(DEV).to(dtype)
    return t, host(t)  # the device tensor and its exact values


def check(got, want, dtype, name):
    got = host(got)
    rms = float(np.sqrt(np.mean(want * want))) if want.size else 1.0
    if dtype == torch.float32:
        close(got, want, 2e-5 * rms, 2e-5, name)
    elif dtype == torch.float16:
        close(got, want, 2e-3 * rms, 2e-3, name)
    else:
        rel_ok(got, want, 1e-2, name)


@pytest.mark.parametrize("sa,sb", SHAPES)
@pytest.mark.parametrize("dtype", DTYPES)
def test_forward_vs_oracle(sa, sb, dtype):
    a, ah = dev(sa, dtype, 1, 1 / np.sqrt(sa[-1]))
    b, bh = dev(sb, dtype, 2)
    y = HipRuntime.tensor_matmul(a, b)
    assert y.dtype == dtype and tuple(y.shape) == oracle.matmul_shape(sa, sb)
    check(y, oracle.tensor_matmul_f64(ah, bh), dtype, f"{sa}@{sb} {dtype}")


@pytest.mark.parametrize("sa,sb", [SHAPES[0], SHAPES[1], SHAPES[3], SHAPES[5]])
@pytest.mark.parametrize("dtype", DTYPES)
def test_autograd_vs_oracle(sa, sb, dtype):
    a, ah = dev(sa, dtype, 3, 1 / np.sqrt(sa[-1]))
    b, bh = dev(sb, dtype, 4)
    out_shape = oracle.matmul_shape(sa, sb)
    dy, dyh = dev(out_shape, dtype, 5)
    a.requires_grad_()
    b.requires_grad_()
    y = nn.float_matmul(a, b)
    y.backward(dy)
    da, db = oracle.tensor_matmul_backward_f64(ah, bh, dyh)
    assert a.grad.dtype == dtype and a.grad.shape == a.shape and b.grad.shape == b.shape
    check(a.grad, da, dtype, f"dA {sa}@{sb} {dtype}")
    check(b.grad, db, dtype, f"dB {sa}@{sb} {dtype}")


@pytest.mark.parametrize("dtype", DTYPES)
def test_empty_contraction_and_empty_output(dtype):
    a = torch.empty((3, 0), dtype=dtype, device=DEV)
    b = torch.empty((0, 7), dtype=dtype, device=DEV)
    y = HipRuntime.tensor_matmul(a, b)
    assert y.shape == (3, 7) and float(y.float().abs().max()) == 0.0  # zeros, not stale memory
    y = HipRuntime.tensor_matmul(torch.empty((0, 5), dtype=dtype, device=DEV), torch.ones((5, 7), dtype=dtype,
                                                                                           device=DEV))
    assert y.shape == (0, 7)
    da, db = HipRuntime.tensor_matmul_backward(torch.ones((2, 0, 5), dtype=dtype, device=DEV),
                                               torch.ones((5, 7), dtype=dtype, device=DEV),
                                               torch.empty((2, 0, 7), dtype=dtype, device=DEV))
    assert float(db.float().abs().max()) == 0.0  # no output rows: dB is zero


def test_many_batches():
    a, ah = dev((4100, 16, 16), torch.float32, 6)
    b, bh = dev((16, 8), torch.float32, 7)
    check(HipRuntime.tensor_matmul(a, b), oracle.tensor_matmul_f64(ah, bh), torch.float32, "4100 batches")


def test_contract_errors_leave_the_context_healthy():
    a = torch.ones((3, 5), device=DEV)
    with pytest.raises(HkError, match="contraction"):
        HipRuntime.tensor_matmul(a, torch.ones((4, 7), device=DEV))
    with pytest.raises(HkError, match="matching floating dtypes"):
        HipRuntime.tensor_matmul(a, torch.ones((5, 7), device=DEV, dtype=torch.bfloat16))
    with pytest.raises(HkError, match="FP32"):
        HipRuntime.matmul_fp32(a.to(torch.bfloat16), torch.ones((5, 7), device=DEV, dtype=torch.bfloat16))
    y = HipRuntime.matmul_fp32(a, torch.ones((5, 7), device=DEV))
    assert float(y.min()) == 5.0 and float(y.max()) == 5.0
