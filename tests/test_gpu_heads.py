"""GPU parity: the composed-attention compatibility entry points (causal mask, KV-head
repetition and its backward) through the C ABI, on the reference's own cases
(examples/grouped_attention_tensor.rs:50-72) and the golden masks, bit-exact: the mask is a
pattern of 0 and -inf, the repeat a copy, and the backward adds in the reference's pairwise
level order, which the oracle restates (runtime/heads.rs:29-51)."""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import DEV, dev_f32, host
from rust_ascend_hip import HipRuntime, HkError

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def test_causal_mask_golden(golden):
    for ci in range(3):
        b, qn, kn, qs, ks = (int(x) for x in golden[f"mask_{ci}_spec"])
        out = HipRuntime.causal_mask(b, qn, kn, qs, ks, device=DEV)
        np.testing.assert_array_equal(_bits(host(out)), golden[f"mask_{ci}"].view(np.uint32))


@pytest.mark.parametrize("b,qn,kn,qs,ks", [(1, 1, 1, 0, 0), (2, 37, 129, 5, 0), (3, 64, 64, 0, 7),
                                           (1, 300, 1000, (1 << 40) + 700, 1 << 40), (2, 5, 9, 0, 1 << 63)])
def test_causal_mask_vs_oracle(b, qn, kn, qs, ks):
    out = HipRuntime.causal_mask(b, qn, kn, qs, ks, device=DEV)
    np.testing.assert_array_equal(_bits(host(out)), _bits(oracle.causal_mask(b, qn, kn, qs, ks)))


def _repeat_case(group):
    batch, kv, n, d = 2, 3, 5, 7
    heads = kv * group
    x = (np.arange(batch * kv * n * d, dtype=np.float32) / 8 - 1).reshape(batch, kv, n, d)
    dy = ((np.arange(batch * heads * n * d) % 11).astype(np.float32) / 8 - 0.25).reshape(batch, heads, n, d)
    return x, dy, heads


@pytest.mark.parametrize("group", [1, 2, 3, 5, 9])
def test_repeat_kv_reference_cases(group):
    x, dy, heads = _repeat_case(group)
    y = HipRuntime.repeat_kv_heads(dev_f32(x), heads)
    np.testing.assert_array_equal(_bits(host(y)), _bits(oracle.repeat_kv(x, heads)))
    dx = HipRuntime.repeat_kv_heads_backward(x.shape, heads, dev_f32(dy))
    np.testing.assert_array_equal(_bits(host(dx)), _bits(oracle.repeat_kv_backward(dy, x.shape[1])))


@pytest.mark.parametrize("b,kv,group,n,d", [(1, 1, 4, 1, 4), (2, 8, 4, 257, 128), (1, 2, 8, 64, 64),
                                            (3, 1, 7, 33, 5), (1, 4, 16, 16, 32), (2, 2, 6, 9, 128)])
def test_repeat_kv_random(b, kv, group, n, d):
    heads = kv * group
    x = oracle.normal((b, kv, n, d), seed=group, stream=51)
    dy = oracle.normal((b, heads, n, d), seed=group, stream=52, std=1e3)
    y = HipRuntime.repeat_kv_heads(dev_f32(x), heads)
    np.testing.assert_array_equal(_bits(host(y)), _bits(oracle.repeat_kv(x, heads)))
    dx = HipRuntime.repeat_kv_heads_backward(x.shape, heads, dev_f32(dy))
    np.testing.assert_array_equal(_bits(host(dx)), _bits(oracle.repeat_kv_backward(dy, kv)))


def test_repeat_kv_pairwise_order_on_device():
    dy = np.array([1.0, 1e8, -1e8, 1.0, 1.0], np.float32).reshape(1, 5, 1, 1)
    dx = HipRuntime.repeat_kv_heads_backward((1, 1, 1, 1), 5, dev_f32(dy))
    assert host(dx).item() == 1.0   # ((1 + 1e8) + (-1e8 + 1)) + 1 in float32


@pytest.mark.parametrize("shape", [(0, 3, 5, 7), (2, 3, 0, 7), (2, 3, 5, 0)])
def test_repeat_kv_empty(shape):
    x = torch.empty(shape, dtype=torch.float32, device=DEV)
    y = HipRuntime.repeat_kv_heads(x, 9)
    assert y.shape == (shape[0], 9, shape[2], shape[3]) and y.numel() == 0
    dx = HipRuntime.repeat_kv_heads_backward(shape, 9, torch.empty(y.shape, dtype=torch.float32, device=DEV))
    assert dx.shape == shape


def test_repeat_kv_rejects_bad_shapes():
    x = torch.zeros((1, 3, 4, 8), dtype=torch.float32, device=DEV)
    with pytest.raises(HkError):
        HipRuntime.repeat_kv_heads(x, 4)            # 4 query heads over 3 kv heads
    with pytest.raises(HkError):
        HipRuntime.repeat_kv_heads(x.to(torch.bfloat16), 6)
    with pytest.raises(HkError):
        HipRuntime.repeat_kv_heads_backward((1, 3, 4, 9), 6, torch.zeros((1, 6, 4, 8), device=DEV))
