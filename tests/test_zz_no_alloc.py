"""GPU: hk_rms_norm_backward_noalloc, the allocation-free form of hk_rms_norm_backward, called
through the C ABI. Its results must equal hk_rms_norm_backward's bit for bit (the same kernels,
with the dgamma partials in the library's fixed device scratch instead of the context workspace)
on two calls in a row, the second with a smaller input (so stale partials of the first call would
show), and it must reject shapes whose partials do not fit the scratch without touching the
context."""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import DEV, dev_f32, host, randn_bf16, rel_ok
from rust_ascend_hip import HipRuntime, HkError, runtime

pytestmark = pytest.mark.gpu


def backward(name, x, w, dy, rstd):
    dx = torch.full_like(x, float("nan"))
    dw = torch.full((w.shape[0],), float("nan"), dtype=torch.float32, device=DEV)
    runtime._call(name, runtime.desc(x), runtime.desc(w), runtime.desc(dy), runtime.desc(rstd), runtime.desc(dx),
                  runtime.desc(dw))
    return dx, dw


def bits(t):
    return t.view(torch.int16) if t.dtype == torch.bfloat16 else t.view(torch.int32)


def case(rows, width, dtype, seed):
    x_t, x = randn_bf16((rows, width), seed=seed)
    dy_t, dy = randn_bf16((rows, width), seed=seed + 1)
    w = (1 + 0.1 * oracle.normal((width,), seed, 2)).astype(np.float32)
    w_t = dev_f32(w)
    if dtype == torch.float32:
        x_t, dy_t = x_t.float(), dy_t.float()
    _, rstd = HipRuntime.rms_norm(x_t, w_t, 1e-6)
    return x_t, w_t, dy_t, rstd, (x, w, dy)


def test_noalloc_backward_equals_the_allocating_one_on_two_calls():
    # the C2 shape first (the fast path, 256 partial rows), then a smaller F32 input on the
    # general path (width 1000: 5 partial rows) into the same scratch
    cases = [case(16384, 4096, torch.bfloat16, 81), case(300, 1000, torch.float32, 83)]
    got = [backward("hk_rms_norm_backward_noalloc", *c[:4]) for c in cases]
    for (x_t, w_t, dy_t, rstd, (x, w, dy)), (dx, dw) in zip(cases, got):
        want_dx, want_dw = backward("hk_rms_norm_backward", x_t, w_t, dy_t, rstd)
        assert torch.equal(bits(dx), bits(want_dx)), x_t.shape
        assert torch.equal(bits(dw), bits(want_dw)), x_t.shape
        _, r_ref = oracle.rms_norm_f64(x, w, 1e-6)
        dx_ref, dw_ref = oracle.rms_norm_backward_f64(x, w, dy, r_ref)
        rel_ok(host(dx), dx_ref, 1e-2, "dX")
        rel_ok(host(dw), dw_ref, 1e-4, "dW", atol_frac=1e-3)


def test_noalloc_backward_takes_any_row_count_at_width_4096():
    # the row-split path keeps at most 256 partial rows (one per workgroup), so 32768 rows of
    # width 4096 fit the 8 MiB scratch as C2's 16384 do
    x_t, w_t, dy_t, rstd, _ = case(32768, 4096, torch.bfloat16, 87)
    a = backward("hk_rms_norm_backward_noalloc", x_t, w_t, dy_t, rstd)
    b = backward("hk_rms_norm_backward", x_t, w_t, dy_t, rstd)
    assert torch.equal(bits(a[0]), bits(b[0])) and torch.equal(bits(a[1]), bits(b[1]))


@pytest.mark.parametrize("width", [8192, 4100])
def test_noalloc_backward_rejects_partials_beyond_its_scratch(width):
    # width 8192 (the row-split path) with 32768 rows needs 256 x 8192 FP64 partials = 16 MiB;
    # width 4100 (not a multiple of 8: the general path) 512 x 4100 = 16.4 MB
    x_t = torch.zeros((32768, width), dtype=torch.bfloat16, device=DEV)
    w_t = torch.ones((width,), dtype=torch.float32, device=DEV)
    rstd = torch.ones((32768,), dtype=torch.float32, device=DEV)
    with pytest.raises(HkError, match="scratch"):
        backward("hk_rms_norm_backward_noalloc", x_t, w_t, x_t, rstd)
    del x_t
    x_t, w_t, dy_t, rstd, _ = case(64, 4096, torch.bfloat16, 85)  # the context stays usable
    a = backward("hk_rms_norm_backward_noalloc", x_t, w_t, dy_t, rstd)
    b = backward("hk_rms_norm_backward", x_t, w_t, dy_t, rstd)
    assert torch.equal(bits(a[0]), bits(b[0])) and torch.equal(bits(a[1]), bits(b[1]))
