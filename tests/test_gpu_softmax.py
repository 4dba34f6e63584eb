"""GPU parity: row softmax / log-softmax forward and backward (F32) through the C ABI against
the CPU oracle, with the reference's own inputs, shapes and tolerance
(examples/common_rows_validate.rs:7-9,100,121: |a-b| <= 5e-4 + 5e-4|b| against an f64 host
reference), plus random rows, widths off the fast path (not a multiple of 4, wider than 4096)
and the input checks of runtime/rows.rs:50-79."""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import close, dev_f32, host
from rust_ascend_hip import HipRuntime, HkError, nn

pytestmark = pytest.mark.gpu


def reference_inputs(rows, width):
    i = np.arange(rows * width)
    x = ((i % 41).astype(np.float32) / np.float32(7.0) - np.float32(2.0)).reshape(rows, width)
    dy = ((i % 13).astype(np.float32) / np.float32(9.0) - np.float32(0.5)).reshape(rows, width)
    return x.astype(np.float32), dy.astype(np.float32)


@pytest.mark.parametrize("rows,width", [(0, 32), (1, 32), (3, 96), (7, 256), (33, 4096)])
@pytest.mark.parametrize("logarithmic", [False, True])
def test_softmax_reference_cases(rows, width, logarithmic):
    x, dy = reference_inputs(rows, width)
    fwd = HipRuntime.log_softmax if logarithmic else HipRuntime.softmax
    bwd = HipRuntime.log_softmax_backward if logarithmic else HipRuntime.softmax_backward
    y = fwd(dev_f32(x))
    assert y.shape == x.shape and y.dtype == torch.float32
    y_ref = oracle.softmax_f64(x, logarithmic)
    close(host(y), y_ref, 5e-4, 5e-4, "Y")
    yh = host(y)
    dx = bwd(dev_f32(yh), dev_f32(dy))
    close(host(dx), oracle.softmax_backward_f64(yh, dy, logarithmic), 5e-4, 5e-4, "dX")


@pytest.mark.parametrize("shape", [(64, 4096), (5, 3, 128), (9, 4100), (2, 7), (4, 8224), (1000, 64), (3, 1),
                                   (3, 12000), (2, 20004), (5, 32000), (2, 32768), (2, 32772), (3, 4102)])
@pytest.mark.parametrize("logarithmic", [False, True])
def test_softmax_random_rows(shape, logarithmic):
    x = oracle.normal(shape, seed=sum(shape), stream=41, std=4.0)
    dy = oracle.normal(shape, seed=sum(shape), stream=42)
    fwd = HipRuntime.log_softmax if logarithmic else HipRuntime.softmax
    bwd = HipRuntime.log_softmax_backward if logarithmic else HipRuntime.softmax_backward
    y = fwd(dev_f32(x))
    close(host(y), oracle.softmax_f64(x, logarithmic), 1e-5, 1e-5, "Y")
    yh = host(y)
    dx = bwd(dev_f32(yh), dev_f32(dy))
    close(host(dx), oracle.softmax_backward_f64(yh, dy, logarithmic), 1e-5, 1e-5, "dX")


def test_softmax_autograd_wrapper_matches_torch():
    x = torch.tensor(oracle.normal((6, 300), seed=5, stream=43, std=2.0), device="cuda", requires_grad=True)
    g = torch.tensor(oracle.normal((6, 300), seed=5, stream=44), device="cuda")
    for ours, ref in [(nn.softmax, torch.softmax), (nn.log_softmax, torch.log_softmax)]:
        xr = x.detach().double().requires_grad_(True)
        y = ours(x)
        y.backward(g)
        yr = ref(xr, dim=-1)
        yr.backward(g.double())
        close(host(y), yr.detach().cpu().numpy(), 1e-5, 1e-5, "Y")
        close(host(x.grad), xr.grad.cpu().numpy(), 1e-5, 1e-5, "dX")
        x.grad = None


def test_softmax_rejects_invalid_inputs():
    with pytest.raises(HkError):
        HipRuntime.softmax(torch.zeros((2, 8), device="cuda", dtype=torch.bfloat16))  # F32 only
    with pytest.raises(HkError):
        HipRuntime.softmax(torch.zeros((2, 0), device="cuda"))  # zero width
    y = torch.zeros((2, 8), device="cuda")
    with pytest.raises(HkError):
        HipRuntime.softmax_backward(y, torch.zeros((2, 9), device="cuda"))  # shape mismatch
