"""CPU checks of the generic floating matmul (RudaAscend::float_matmul -> AscendRuntime::tensor_matmul,
src/backend.rs:692-703, rust-ascend-driver/src/tensor/runtime/{mod.rs:156-158,generic_matrix.rs}):
the oracle pinned against the reference's own shape cases, numpy's float64 matmul and torch's float64
autograd; libhk.so's host-only layout check against the same cases."""
import numpy as np
import pytest
import torch

from rust_ascend_hip import HkError, runtime

# generic_matrix.rs:59-101 and tensor/tests.rs:56-69 (rank >= 2): (A, B, out) or (A, B, None) = error
REFERENCE_SHAPES = [
    ((2, 1, 3, 5), (1, 4, 5, 7), (2, 4, 3, 7)),
    ((0, 5), (5, 7), (0, 7)),
    ((3, 0), (0, 7), (3, 7)),
    ((7, 1, 2, 3), (4, 3, 5), (7, 4, 2, 5)),
    ((0, 3), (3, 4), (0, 4)),
    ((3, 5), (4, 7), None),
    ((2, 3, 4), (3, 4, 5), None),
]


@pytest.mark.parametrize("a,b,out", REFERENCE_SHAPES)
def test_reference_shape_cases(oracle, a, b, out):
    if out is None:
        with pytest.raises(ValueError):
            oracle.matmul_shape(a, b)
        for dtype in (torch.float32, torch.float16, torch.bfloat16):
            with pytest.raises(HkError):
                runtime.matmul_layout(a, b, dtype)
    else:
        assert oracle.matmul_shape(a, b) == out
        for dtype in (torch.float32, torch.float16, torch.bfloat16):  # half dtypes keep their storage
            assert runtime.matmul_layout(a, b, dtype) == out


def test_rank_limits(oracle):
    for a, b in (((5,), (5, 7)), ((2, 3), (3,)), ((1,) * 5 + (2, 3), (3, 4))):
        with pytest.raises(ValueError):
            oracle.matmul_shape(a, b)
        with pytest.raises(HkError):
            runtime.matmul_layout(a, b)
    assert runtime.matmul_layout((1, 1, 1, 1, 2, 3), (1, 3, 4)) == (1, 1, 1, 1, 2, 4)


CASES = [((2, 1, 3, 5), (1, 4, 5, 7)), ((4, 6), (6, 3)), ((3, 1, 2, 4, 5), (2, 1, 5, 3)),
         ((1, 2, 1, 1, 3, 2), (2, 1, 1, 2, 4)), ((5, 2, 3), (3, 4))]


@pytest.mark.parametrize("sa,sb", CASES)
def test_oracle_vs_numpy_and_autograd(oracle, sa, sb):
    rng = np.random.default_rng(len(sa) * 10 + len(sb))
    a = rng.standard_normal(sa).astype(np.float32)
    b = rng.standard_normal(sb).astype(np.float32)
    got = oracle.tensor_matmul_f64(a, b)
    want = np.matmul(a.astype(np.float64), b.astype(np.float64))
    assert got.shape == want.shape
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    dy = rng.standard_normal(want.shape)
    ta = torch.tensor(a, dtype=torch.float64, requires_grad=True)
    tb = torch.tensor(b, dtype=torch.float64, requires_grad=True)
    torch.matmul(ta, tb).backward(torch.tensor(dy))
    da, db = oracle.tensor_matmul_backward_f64(a, b, dy.astype(np.float32))
    np.testing.assert_allclose(da, ta.grad.numpy(), rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(db, tb.grad.numpy(), rtol=1e-6, atol=1e-6)


def test_oracle_gradient_catches_a_dropped_broadcast_sum(oracle):
    """A backward that keeps only the first broadcast batch (no sum) differs from the oracle."""
    rng = np.random.default_rng(3)
    a = rng.standard_normal((1, 3, 4)).astype(np.float32)
    b = rng.standard_normal((5, 4, 2)).astype(np.float32)
    dy = rng.standard_normal((5, 3, 2)).astype(np.float32)
    da, _ = oracle.tensor_matmul_backward_f64(a, b, dy)
    wrong = dy[0].astype(np.float64) @ b[0].astype(np.float64).T
    assert np.abs(da[0] - wrong).max() > 1e-2
