"""GPU parity of the backend's module attention (RudaAscend's ModuleOps::attention,
src/backend.rs:1323-1333: the RUDA tensor library's fallback composed from the backend's own ops,
here hk_tensor_matmul, hk_swap_last_dims, hk_attention_scores and hk_softmax) against the float64
oracle, forward and gradients (Q, K, V and the broadcast bias), with boolean masks, causal masking,
softcap and broadcast bias/mask shapes. Parity with the RUDA library itself is unpinned (not
vendored); the oracle's formula is pinned on the CPU (tests/test_matmul_contract.py).

Tolerance: F32 throughout (FP32 matmul products and sums, F32 softmax): 1e-4 relative plus 1e-5
of the tensor's rms."""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import DEV, close, dev_f32, host
from rust_ascend_hip import HipRuntime, HkError, nn

pytestmark = pytest.mark.gpu


def f32_tight(got, want, name):
    rms = float(np.sqrt(np.mean(want * want))) if want.size else 1.0
    close(host(got), want, 1e-5 * rms, 1e-4, name)


CASES = [  # (B, H, Sq, Sk, D, Dv, softcap, causal, bias shape, mask shape)
    (2, 3, 5, 7, 4, 6, None, False, (1, 3, 5, 7), (2, 1, 5, 7)),
    (2, 4, 64, 96, 32, 48, None, True, None, None),
    (1, 2, 33, 33, 16, 16, 5.0, False, (1, 1, 33, 33), None),
    (2, 2, 40, 72, 64, 24, 2.0, True, (2, 2, 40, 72), (1, 1, 40, 72)),
    (1, 8, 128, 128, 64, 64, None, False, None, (1, 8, 1, 128)),
]


@pytest.mark.parametrize("case", CASES)
def test_module_attention_vs_oracle(case):
    B, H, Sq, Sk, D, Dv, softcap, causal, bshape, mshape = case
    rng = np.random.default_rng(Sq * 100 + Sk)
    q = rng.standard_normal((B, H, Sq, D)).astype(np.float32)
    k = rng.standard_normal((B, H, Sk, D)).astype(np.float32)
    v = rng.standard_normal((B, H, Sk, Dv)).astype(np.float32)
    dy = rng.standard_normal((B, H, Sq, Dv)).astype(np.float32)
    bias = None if bshape is None else rng.standard_normal(bshape).astype(np.float32)
    mask = None if mshape is None else rng.random(mshape) < 0.25
    if mask is not None:
        mask[..., 0] = False  # every query keeps a key
    scale = D ** -0.5
    tq, tk, tv = (dev_f32(x).requires_grad_() for x in (q, k, v))
    tb = None if bias is None else dev_f32(bias).requires_grad_()
    tm = None if mask is None else torch.from_numpy(mask).to(DEV)
    o = nn.module_attention(tq, tk, tv, mask=tm, attn_bias=tb, scale=scale, softcap=softcap, is_causal=causal)
    assert o.shape == (B, H, Sq, Dv) and o.dtype == torch.float32
    o.backward(dev_f32(dy))
    ref = oracle.module_attention_f64(q, k, v, dy, mask=mask, bias=bias, scale=scale, softcap=softcap, causal=causal)
    f32_tight(o, ref["out"], "out")
    for name, t in (("dq", tq), ("dk", tk), ("dv", tv)) + ((("dbias", tb),) if tb is not None else ()):
        f32_tight(t.grad, ref[name], name)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", [(70, 130), (3, 2, 64, 64), (5, 1, 129)])
def test_swap_last_dims_is_exact(dtype, shape):
    x = torch.randn(shape, device=DEV).to(dtype)
    y = HipRuntime.swap_last_dims(x)
    assert torch.equal(y.cpu(), x.cpu().transpose(-1, -2).contiguous())


def test_score_contract_errors():
    s = torch.zeros((1, 2, 4, 8), device=DEV)
    with pytest.raises(HkError, match="broadcast"):
        HipRuntime.attention_scores(s, 1.0, bias=torch.zeros((1, 2, 4, 4), device=DEV))
    with pytest.raises(HkError, match="BOOL"):
        HipRuntime.attention_scores(s, 1.0, mask=torch.zeros((1, 2, 4, 8), device=DEV))
    with pytest.raises(HkError, match="softcap"):
        HipRuntime.attention_scores(s, 1.0, softcap=-1.0)
    with pytest.raises(HkError, match="F32 rank-4"):
        nn.module_attention(s.to(torch.bfloat16), s.to(torch.bfloat16), s.to(torch.bfloat16))
    out = HipRuntime.attention_scores(s, 2.0, causal=True)
    want = torch.zeros((4, 8)).masked_fill(torch.ones(4, 8, dtype=torch.bool).triu(1), float("-inf"))
    assert torch.equal(out[0, 1].cpu(), want)
