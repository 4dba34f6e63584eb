"""GPU parity: the padded BF16-compute GEMM for logical shapes that are not multiples of 16
(AscendRuntime::gemm_padded_bf16_fp32[_backward] and linear_frozen_padded_bf16_fp32[_backward],
rust-ascend-driver/src/tensor/runtime/padded_matrix.rs; nn::matmul_padded_bf16_fp32,
src/nn/padded.rs), through the C ABI.

Cases and tolerance are the reference's (examples/padded_matrix_tensor.rs): (m,n,k) in
{(1,1,1),(3,17,7),(17,33,65),(16,32,48)} x all transposes x rank 2 and batch-2 rank 3, output and
both gradients of sum(2Y * dY) against f64 sums of BF16-rounded products, |a-b| <= 5e-4 + 5e-4|b|;
the frozen linear on the reference's tail shape 3x19x35; an infinite activation whose NaN padding
channels are cropped away (padded_matrix_tensor.rs:91-97); larger tails on the 256-tile kernels
against the f64 oracle.
"""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import close, dev_f32, f32_close, host
from rust_ascend_hip import HipRuntime, HkError, Transpose, nn

pytestmark = pytest.mark.gpu

MNK = ["1x1x1", "3x17x7", "17x33x65", "16x32x48"]


@pytest.mark.parametrize("batch", [1, 2])
@pytest.mark.parametrize("mnk", MNK)
@pytest.mark.parametrize("ta", [0, 1])
@pytest.mark.parametrize("tb", [0, 1])
def test_padded_reference_cases(golden, batch, mnk, ta, tb):
    key = f"padded_{batch}_{mnk}_{'nt'[ta]}{'nt'[tb]}"
    a, b, dy = golden[key + "_a"], golden[key + "_b"], golden[key + "_dy"]
    # plain forward (padded_matrix_tensor.rs:32-35), with its saved snapshots
    y, ap, bp = HipRuntime.gemm_padded_bf16_fp32(dev_f32(a), dev_f32(b), Transpose(ta), Transpose(tb))
    assert y.dtype == torch.float32 and tuple(y.shape) == golden[key + "_y"].shape
    close(host(y), golden[key + "_y"], 5e-4, 5e-4, "padded Y")
    for snap, src in ((ap, a), (bp, b)):  # zero-padded BF16 roundings of the inputs
        want = np.zeros(snap.shape, np.float32)
        want[(Ellipsis, slice(0, src.shape[-2]), slice(0, src.shape[-1]))] = oracle.bf16_round(src)
        np.testing.assert_array_equal(host(snap), want)
    # autograd through the output used twice (padded_matrix_tensor.rs:36-44)
    x = dev_f32(a).requires_grad_()
    w = dev_f32(b).requires_grad_()
    out = nn.matmul_padded_bf16_fp32(x, w, Transpose(ta), Transpose(tb))
    ((out + out) * dev_f32(dy)).sum().backward()
    assert x.grad.shape == x.shape and w.grad.shape == w.shape
    close(host(x.grad), 2 * golden[key + "_da"], 5e-4, 5e-4, "padded dA")
    close(host(w.grad), 2 * golden[key + "_db"], 5e-4, 5e-4, "padded dB")


def test_frozen_padded_linear_tail():
    """The frozen tail shape of padded_matrix_tensor.rs:46-52 (3x19x35): input-only gradient, the
    fixed weight unchanged; an aligned weight is reused as the saved weight."""
    m, n, k = 3, 19, 35
    x = ((np.arange(m * k) % 7).astype(np.float32) - 3) / 64
    wv = ((np.arange(n * k) % 5).astype(np.float32) - 2) / 16
    dy = ((np.arange(m * n) % 7).astype(np.float32) - 3) / 8
    X = dev_f32(x.reshape(m, k)).requires_grad_()
    W = dev_f32(wv.reshape(n, k)).to(torch.bfloat16)
    before = W.clone()
    y = nn.linear_frozen_padded_bf16_fp32(X, W)
    xr, wr = oracle.bf16_round(x.reshape(m, k)), oracle.bf16_round(wv.reshape(n, k))
    close(host(y), oracle.gemm_f64(xr, wr, 0, 1), 5e-4, 5e-4, "frozen Y")
    (y * dev_f32(dy.reshape(m, n))).sum().backward()
    close(host(X.grad), oracle.gemm_f64(oracle.bf16_round(dy.reshape(m, n)), wr, 0, 0), 5e-4, 5e-4, "frozen dX")
    assert torch.equal(W, before)
    y2, wp = HipRuntime.linear_frozen_padded_bf16_fp32(X.detach(), W)
    assert tuple(wp.shape) == (32, 48) and torch.equal(y2, y.detach())
    aligned = torch.ones((32, 48), device=W.device, dtype=torch.bfloat16)
    y3, saved = HipRuntime.linear_frozen_padded_bf16_fp32(dev_f32(np.ones((3, 48), np.float32)), aligned)
    assert saved is aligned  # no copy of an aligned weight
    assert host(y3).tolist() == [[48.0] * 32] * 3


def test_infinite_activation_padding_is_cropped():
    """inf * 0 = NaN fills the padded output channels; the crop must discard them
    (padded_matrix_tensor.rs:91-97)."""
    x = dev_f32(np.array([[np.inf]], np.float32))
    one = dev_f32(np.ones((1, 1), np.float32))
    y, _, _ = HipRuntime.gemm_padded_bf16_fp32(x, one, Transpose.No, Transpose.Yes)
    assert host(y).tolist() == [[np.inf]]
    y = nn.linear_frozen_padded_bf16_fp32(x, one.to(torch.bfloat16))
    assert host(y).tolist() == [[np.inf]]


@pytest.mark.parametrize("m,n,k,ta,tb", [(1000, 1500, 700, 0, 1), (4100, 4090, 1030, 0, 1), (4100, 4090, 1030, 1, 0),
                                         (777, 2049, 3001, 1, 1)])
def test_padded_large_tails_vs_oracle(m, n, k, ta, tb):
    """Tails on the large-tile kernels: the padded problem (rounded to 16) runs the 256-tile GEMMs."""
    rng = np.random.default_rng(m + n + k)
    a = (rng.standard_normal((k, m) if ta else (m, k)) / np.sqrt(k)).astype(np.float32)
    b = rng.standard_normal((n, k) if tb else (k, n)).astype(np.float32)
    dy = rng.standard_normal((m, n)).astype(np.float32)
    x, w = dev_f32(a).requires_grad_(), dev_f32(b).requires_grad_()
    y = nn.matmul_padded_bf16_fp32(x, w, Transpose(ta), Transpose(tb))
    ar, br, dr = oracle.bf16_round(a), oracle.bf16_round(b), oracle.bf16_round(dy)
    rows = np.concatenate([np.arange(0, m, 37), [m - 1]])
    cols = np.concatenate([np.arange(0, n, 29), [n - 1]])
    r, c = np.meshgrid(rows, cols, indexing="ij")
    f32_close(host(y)[r.ravel(), c.ravel()], oracle.gemm_f64_sampled(ar, br, ta, tb, r.ravel(), c.ravel()), "Y")
    (y * dev_f32(dy)).sum().backward()
    # d op(A) = dY op(B)^T; d op(B) = op(A)^T dY, mapped back to the physical layouts
    opb = br.T if tb else br
    opa = ar.T if ta else ar
    d_opa = oracle.gemm_f64(dr, np.ascontiguousarray(opb), 0, 1)
    d_opb = oracle.gemm_f64(np.ascontiguousarray(opa), dr, 1, 0)
    f32_close(host(x.grad), d_opa.T if ta else d_opa, "dA")
    f32_close(host(w.grad), d_opb.T if tb else d_opb, "dB")


def _bits16(t):
    """uint16 bit patterns of a BF16 device tensor."""
    return t.detach().view(torch.int16).cpu().numpy().view(np.uint16)


def _specials(shape, seed):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal(shape).astype(np.float32)
    flat = a.reshape(-1)
    specials = np.array([np.inf, -np.inf, 1 + 2.0**-8, 1 + 3 * 2.0**-8, 1e-40, -1e-42, 3.4e38, 0.0], np.float32)
    flat[rng.choice(flat.size, 64, replace=False)] = np.resize(specials, 64)
    return a


def _assert_padded_bits(got, bits):
    want = np.zeros(tuple(got.shape), np.uint16)
    want[..., : bits.shape[-2], : bits.shape[-1]] = bits
    assert np.array_equal(_bits16(got), want)


@pytest.mark.parametrize("shape", [(1000, 777), (1001, 1024), (3, 600, 530), (640, 1024), (2, 520, 1536)])
def test_padded_snapshots_hold_exact_bits(shape):
    """The padded BF16 operand snapshots hold exactly the RNE BF16 bits of the F32 inputs inside and
    zero bits in the padding, rows and columns rounded up to multiples of 16: the row-wise pad kernel
    (padded rows of 512 columns or more) at 16-byte aligned and unaligned widths, with row padding
    and batches, and the element kernel for the narrow B; the inputs carry rounding ties,
    subnormals, the largest finite value and infinities."""
    a = _specials(shape, sum(shape))
    b = np.random.default_rng(len(shape)).standard_normal(shape[:-2] + (shape[-1], 20)).astype(np.float32)
    print(f"padded snapshots {shape}", flush=True)
    _, ap, bp = HipRuntime.gemm_padded_bf16_fp32(dev_f32(a), dev_f32(b))
    _assert_padded_bits(ap, oracle.bf16_bits(a))
    _assert_padded_bits(bp, oracle.bf16_bits(b))


@pytest.mark.parametrize("shape", [(1000, 777), (1001, 1024), (600, 530), (40, 2050)])
def test_frozen_padded_weight_copy_holds_exact_bits(shape):
    """A frozen BF16 weight whose axes are not multiples of 16 is copied bit for bit into its
    zero-padded snapshot (infinities and subnormals included): the row-wise pad kernel's BF16 path
    at 16-byte aligned and unaligned widths, and its element path at the row edges."""
    w = dev_f32(_specials(shape, 7 + sum(shape))).to(torch.bfloat16)
    x = dev_f32(np.random.default_rng(3).standard_normal((16, shape[1])).astype(np.float32))
    print(f"frozen padded weight {shape}", flush=True)
    _, wp = HipRuntime.linear_frozen_padded_bf16_fp32(x, w)
    _assert_padded_bits(wp, _bits16(w))


def test_padded_rejections_leave_the_context_healthy():
    a = dev_f32(np.ones((3, 7), np.float32))
    with pytest.raises(HkError):
        HipRuntime.gemm_padded_bf16_fp32(a, dev_f32(np.ones((8, 17), np.float32)))  # contraction mismatch
    with pytest.raises(HkError):
        HipRuntime.gemm_padded_bf16_fp32(a.to(torch.bfloat16), dev_f32(np.ones((7, 17), np.float32)))  # FP32 only
    y, _, _ = HipRuntime.gemm_padded_bf16_fp32(a, dev_f32(np.ones((7, 17), np.float32)))
    assert host(y).tolist() == [[7.0] * 17] * 3
