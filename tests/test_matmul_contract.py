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


# ------------------------------------------------------------------ module attention oracle

def _torch_module_attention(q, k, v, mask, bias, scale, softcap, causal):
    """Explicit torch float64 composition (independent of the oracle's numpy code)."""
    s = torch.matmul(q, k.transpose(-1, -2)) * scale
    if softcap:
        s = softcap * torch.tanh(s / softcap)
    if bias is not None:
        s = s + bias
    if causal:
        s = s.masked_fill(torch.ones(s.shape[-2:], dtype=torch.bool).triu(1), float("-inf"))
    if mask is not None:
        s = s.masked_fill(mask, float("-inf"))
    return torch.matmul(torch.softmax(s, dim=-1), v)


@pytest.mark.parametrize("softcap,causal,with_bias,with_mask", [(None, False, True, True), (None, True, False, False),
                                                                (5.0, False, True, False), (2.0, True, True, True)])
def test_module_attention_oracle(oracle, softcap, causal, with_bias, with_mask):
    rng = np.random.default_rng(11)
    B, H, Sq, Sk, D, Dv = 2, 3, 5, 7, 4, 6
    q, k = rng.standard_normal((B, H, Sq, D)), rng.standard_normal((B, H, Sk, D))
    v, dy = rng.standard_normal((B, H, Sk, Dv)), rng.standard_normal((B, H, Sq, Dv))
    bias = rng.standard_normal((1, H, Sq, Sk)) if with_bias else None
    mask = (rng.random((B, 1, Sq, Sk)) < 0.3) if with_mask else None
    if mask is not None:
        mask[..., 0] = False  # every query keeps a key
    ref = oracle.module_attention_f64(q, k, v, dy, mask=mask, bias=bias, scale=0.4, softcap=softcap, causal=causal)
    tq, tk, tv = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    tb = None if bias is None else torch.tensor(bias, requires_grad=True)
    tm = None if mask is None else torch.tensor(mask)
    o = _torch_module_attention(tq, tk, tv, tm, tb, 0.4, softcap, causal)
    o.backward(torch.tensor(dy))
    np.testing.assert_allclose(ref["out"], o.detach().numpy(), rtol=1e-10, atol=1e-12)
    for name, t in (("dq", tq), ("dk", tk), ("dv", tv)) + ((("dbias", tb),) if tb is not None else ()):
        np.testing.assert_allclose(ref[name], t.grad.numpy(), rtol=1e-9, atol=1e-11, err_msg=name)
    if not softcap:  # torch's own SDPA with the bias and mask folded into one float mask
        fm = torch.zeros((B, H, Sq, Sk), dtype=torch.float64)
        if bias is not None:
            fm = fm + torch.tensor(bias)
        if causal:
            fm = fm.masked_fill(torch.ones(Sq, Sk, dtype=torch.bool).triu(1), float("-inf"))
        if mask is not None:
            fm = fm.masked_fill(torch.tensor(mask), float("-inf"))
        sd = torch.nn.functional.scaled_dot_product_attention(torch.tensor(q), torch.tensor(k), torch.tensor(v),
                                                              attn_mask=fm, scale=0.4)
        np.testing.assert_allclose(ref["out"], sd.numpy(), rtol=1e-10, atol=1e-12)


def test_module_attention_closed_forms(oracle):
    """Orthogonal Q/K: uniform probabilities, so O is the mean of V (attention_tensor.rs:22-66);
    Q = K = 0 causal: O row i is the running mean of V[0..i] (causal_attention_tensor.rs:31-55)."""
    rng = np.random.default_rng(2)
    q = np.zeros((1, 1, 4, 8))
    q[0, 0, :, 0] = 1.0
    k = np.zeros((1, 1, 6, 8))
    k[0, 0, :, 1] = 1.0
    v = rng.standard_normal((1, 1, 6, 3))
    out = oracle.module_attention_f64(q, k, v)["out"]
    np.testing.assert_allclose(out[0, 0], np.broadcast_to(v[0, 0].mean(axis=0), (4, 3)), atol=1e-14)
    out = oracle.module_attention_f64(np.zeros((1, 1, 6, 8)), np.zeros((1, 1, 6, 8)), v, causal=True)["out"]
    want = np.cumsum(v[0, 0], axis=0) / np.arange(1, 7)[:, None]
    np.testing.assert_allclose(out[0, 0], want, atol=1e-14)
