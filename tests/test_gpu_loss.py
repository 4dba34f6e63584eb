"""GPU parity: NLLLoss forward/backward (hk_nll_loss, hk_nll_loss_backward) and the composed
cross entropy nll_loss(log_softmax(logits)) through the C ABI, against the f64 oracle.

Cases are the reference's (examples/cross_entropy_tensor.rs:17-59): rows = 5, twelve class widths
from 1 to 4129, all three reductions, with and without the ignore label -100, unweighted and
weighted, the loss used twice under upstream gradients 1.25 + n/4; tolerance 3e-5 + 2e-4|b| on the
loss and the logit gradient. Plus the direct NLLLoss known answer 19/4, BF16 log-probabilities at
BF16 tolerance, larger random cases, and an out-of-range label reported as an error.
"""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import DEV, close, dev_f32, host, rel_ok
from rust_ascend_hip import HipRuntime, HkError, LossReduction, nn

pytestmark = pytest.mark.gpu

WIDTHS = [1, 3, 7, 31, 32, 33, 65, 96, 4095, 4097, 4128, 4129]


@pytest.mark.parametrize("classes", WIDTHS)
@pytest.mark.parametrize("reduction", [0, 1, 2])
@pytest.mark.parametrize("ignore", [None, -100])
@pytest.mark.parametrize("weighted", [False, True])
def test_cross_entropy_reference_cases(classes, reduction, ignore, weighted):
    rows = 5
    x = ((np.arange(rows * classes) % 23).astype(np.float32) / 8 - 1000).reshape(rows, classes)
    labels = np.array([0, 31 % classes, 7 % classes, 0, 2 % classes], np.int64)
    if ignore is not None:
        labels[1] = ignore
    w = (0.5 + (np.arange(classes) % 7) / 4).astype(np.float32) if weighted else np.ones(classes, np.float32)
    logits = dev_f32(x).requires_grad_()
    tgt = torch.from_numpy(labels).to(DEV)
    if weighted:
        loss = nn.weighted_cross_entropy(logits, tgt, dev_f32(w), LossReduction(reduction), ignore)
    else:
        loss = nn.cross_entropy(logits, tgt, LossReduction(reduction), ignore)
    n_out = rows if reduction == 0 else 1
    up = (1.25 + np.arange(n_out) / 4).astype(np.float32)
    dy = dev_f32(up)
    ((loss * dy) + (loss * dy)).sum().backward()
    ii = -1 if ignore is None else ignore
    logp = oracle.softmax_f64(x, logarithmic=True)
    want, total = oracle.nll_loss_f64(logp, labels, w, reduction, ii)
    close(host(loss), want, 3e-5, 2e-4, "loss")
    dlogp = oracle.nll_loss_backward_f64(2 * up.astype(np.float64), x.shape, labels, w, total, reduction, ii)
    dlogits = dlogp - np.exp(logp) * dlogp.sum(-1, keepdims=True)
    close(host(logits.grad), dlogits, 3e-5, 2e-4, "logit gradient")


def test_direct_nll_known_answer():
    """examples/cross_entropy_tensor.rs:55-59: NLLLoss of given log-probabilities, I32 labels."""
    x = dev_f32(np.array([[-1.0, -2, -3], [-4, -5, -6]], np.float32))
    t = torch.tensor([0, 2], dtype=torch.int32, device=DEV)
    w = dev_f32(np.array([1.0, 2, 3], np.float32))
    loss = nn.nll_loss(x, t, w, LossReduction.Mean)
    close(host(loss), [19 / 4], 3e-5, 2e-4, "plain NLLLoss")
    out, total = HipRuntime.nll_loss(x, t, w, LossReduction.Sum)
    assert host(out).tolist() == [19.0] and host(total).tolist() == [4.0]
    out, total = HipRuntime.nll_loss(x, t, w, LossReduction.None_)
    assert host(out).tolist() == [1.0, 18.0]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("reduction", [0, 1, 2])
def test_nll_random_vs_oracle(dtype, reduction):
    rng = np.random.default_rng(reduction)
    n, c = 4096, 32000
    x = rng.standard_normal((n, c)).astype(np.float32) - 10
    labels = rng.integers(0, c, n)
    labels[::7] = -100
    w = rng.uniform(0.5, 2.0, c).astype(np.float32)
    xt = dev_f32(x).to(dtype)
    xr = host(xt)
    wt = dev_f32(w).to(dtype)
    wr = host(wt)
    out, total = HipRuntime.nll_loss(xt, torch.from_numpy(labels).to(DEV), wt, reduction, -100)
    want, tw = oracle.nll_loss_f64(xr, labels, wr, reduction, -100)
    tol = 1e-2 if dtype == torch.bfloat16 else 1e-5
    rel_ok(host(out), want, tol, "loss")
    rel_ok(host(total), [tw if reduction else 0.0], tol, "total weight")  # None reports 0, as torch's nll_loss
    g = (1.0 + np.arange(n if reduction == 0 else 1) / n).astype(np.float32)
    gt = dev_f32(g).to(dtype)
    dx = HipRuntime.nll_loss_backward(gt, xt, torch.from_numpy(labels).to(DEV), wt, total, reduction, -100)
    want_dx = oracle.nll_loss_backward_f64(host(gt), x.shape, labels, wr, float(host(total)[0]), reduction, -100)
    rows = np.arange(0, n, 97)
    rel_ok(host(dx)[rows], want_dx[rows], tol, "dinput rows")
    assert int((host(dx) != 0).sum()) == int((labels != -100).sum())  # one entry per non-ignored row


def test_out_of_range_label_is_reported():
    x = dev_f32(np.zeros((2, 3), np.float32))
    w = dev_f32(np.ones(3, np.float32))
    with pytest.raises(HkError):
        HipRuntime.nll_loss(x, torch.tensor([0, 3], device=DEV), w, LossReduction.Sum)
    out, _ = HipRuntime.nll_loss(x, torch.tensor([0, 2], device=DEV), w, LossReduction.Sum)  # context healthy
    assert host(out).tolist() == [0.0]


def test_nll_backward_past_32_bit_work_items():
    """The dense gradient of a [33000, 131072] BF16 input (4.33e9 elements, more than a dispatch's
    32-bit work-item count): every element is written, the last rows included. The output buffer
    starts as NaN so an element the kernel skipped would show."""
    from rust_ascend_hip import runtime
    rows, classes = 33000, 131072
    assert rows * classes > 1 << 32
    inp = torch.empty((rows, classes), dtype=torch.bfloat16, device=DEV)  # only its layout is read
    labels = torch.arange(rows, device=DEV, dtype=torch.int64) * 7919 % classes
    labels[5] = -100
    w = torch.ones((classes,), dtype=torch.bfloat16, device=DEV)
    g = (1 + torch.arange(rows, device=DEV, dtype=torch.float32) % 5).to(torch.bfloat16)
    total = torch.zeros((1,), dtype=torch.bfloat16, device=DEV)
    dx = torch.full((rows, classes), float("nan"), dtype=torch.bfloat16, device=DEV)
    runtime._call("hk_nll_loss_backward", runtime.desc(g), runtime.desc(inp), runtime.desc(labels), runtime.desc(w),
                  runtime.desc(total), int(LossReduction.None_), -100, runtime.desc(dx))
    del inp
    assert not bool(torch.isnan(dx).any())
    per_row = (dx != 0).sum(dim=1)
    keep = torch.arange(rows, device=DEV) != 5
    assert bool((per_row[keep] == 1).all()) and int(per_row[5]) == 0  # one entry per row but the ignored one
    picked = dx.gather(1, labels.clamp(min=0)[:, None])[:, 0]
    assert torch.equal(picked[keep], -g[keep])
    del dx
    torch.cuda.empty_cache()
