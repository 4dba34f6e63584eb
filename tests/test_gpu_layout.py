"""GPU parity: the decoder layer's relayouts (no reference counterpart; they compose reference
ops). qkv_rope_split must equal, bit for bit, splitting the fused QKV rows into head planes and
applying hk_rotary_prefix with [1,1,S,D/2] tables (itself pinned to the oracle's rotation,
rotary_programs.rs:47-156); qkv_rope_merge must equal the rotation's backward followed by the
inverse split; heads_to_rows / rows_to_heads are exact transposes."""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import DEV, dev_bf16, dev_f32, host
from rust_ascend_hip import HipRuntime, HkError, RotaryLayout

pytestmark = pytest.mark.gpu

CASES = [(2, 64, 4, 2, 64), (1, 48, 8, 8, 128), (2, 2048, 32, 8, 128), (3, 5, 2, 1, 16)]


def planes_of(qkv, hq, hkv, d):
    """Reference split with torch views: [B,S,(Hq+2Hkv)D] -> three [B,H,S,D] planes."""
    b, s, _ = qkv.shape
    x = qkv.reshape(b, s, hq + 2 * hkv, d).permute(0, 2, 1, 3)
    return (x[:, :hq].contiguous(), x[:, hq:hq + hkv].contiguous(), x[:, hq + hkv:].contiguous())


@pytest.mark.parametrize("b,s,hq,hkv,d", CASES)
@pytest.mark.parametrize("layout", [0, 1])
def test_qkv_rope_split_matches_rotary_prefix(b, s, hq, hkv, d, layout):
    g = torch.Generator(device=DEV)
    g.manual_seed(b * 1000 + s + d)
    qkv = torch.randn((b, s, (hq + 2 * hkv) * d), generator=g, device=DEV).to(torch.bfloat16)
    cos, sin = oracle.rope_tables(np.arange(s), d, 5e5)
    c_t, s_t = dev_f32(cos), dev_f32(sin)
    q, k, v = HipRuntime.qkv_rope_split(qkv, c_t, s_t, hq, hkv, RotaryLayout(layout))
    pq, pk, pv = planes_of(qkv, hq, hkv, d)
    c4, s4 = c_t.reshape(1, 1, s, d // 2), s_t.reshape(1, 1, s, d // 2)
    assert torch.equal(q, HipRuntime.rotary_prefix(pq, c4, s4, d, RotaryLayout(layout)))
    assert torch.equal(k, HipRuntime.rotary_prefix(pk, c4, s4, d, RotaryLayout(layout)))
    assert torch.equal(v, pv)
    if b * s * hq * d <= 1 << 16:  # the oracle's rotation directly, one BF16 rounding
        want = oracle.rotary_prefix(host(pq), cos[None, None], sin[None, None], d, layout)
        np.testing.assert_array_equal(host(q), oracle.bf16_round(want))
    # merge is split's transpose: gradients rotate back and return to the fused rows
    dq = torch.randn(q.shape, generator=g, device=DEV).to(torch.bfloat16)
    dk = torch.randn(k.shape, generator=g, device=DEV).to(torch.bfloat16)
    dv = torch.randn(v.shape, generator=g, device=DEV).to(torch.bfloat16)
    dqkv = HipRuntime.qkv_rope_merge(dq, dk, dv, c_t, s_t, RotaryLayout(layout))
    gq = HipRuntime.rotary_prefix_backward(dq, c4, s4, d, RotaryLayout(layout))
    gk = HipRuntime.rotary_prefix_backward(dk, c4, s4, d, RotaryLayout(layout))
    want = torch.cat([gq, gk, dv], dim=1).permute(0, 2, 1, 3).reshape(b, s, -1)
    assert torch.equal(dqkv, want)


def test_qkv_rope_split_is_orthogonal():
    """<split(x), y> == <x, merge(y)> in float64 (RoPE rotations are orthogonal)."""
    b, s, hq, hkv, d = 1, 256, 4, 2, 128
    cos, sin = oracle.rope_tables(np.arange(s), d, 5e5)
    x = oracle.bf16_round(oracle.normal((b, s, (hq + 2 * hkv) * d), seed=1, stream=90))
    yq = oracle.bf16_round(oracle.normal((b, hq, s, d), seed=1, stream=91))
    yk = oracle.bf16_round(oracle.normal((b, hkv, s, d), seed=1, stream=92))
    yv = oracle.bf16_round(oracle.normal((b, hkv, s, d), seed=1, stream=93))
    q, k, v = HipRuntime.qkv_rope_split(dev_bf16(x), dev_f32(cos), dev_f32(sin), hq, hkv)
    lhs = sum(float((host(a).astype(np.float64) * c).sum()) for a, c in ((q, yq), (k, yk), (v, yv)))
    back = host(HipRuntime.qkv_rope_merge(dev_bf16(yq), dev_bf16(yk), dev_bf16(yv), dev_f32(cos), dev_f32(sin)))
    rhs = float((x.astype(np.float64) * back).sum())
    scale = float(np.abs(x).sum() * 3)
    assert abs(lhs - rhs) <= 2 ** -7 * scale / np.sqrt(x.size), (lhs, rhs)


@pytest.mark.parametrize("b,h,s,d", [(2, 32, 2048, 128), (1, 3, 7, 8), (4, 8, 64, 64)])
def test_heads_rows_round_trip(b, h, s, d):
    x = torch.randn((b, h, s, d), device=DEV).to(torch.bfloat16)
    rows = HipRuntime.heads_to_rows(x)
    assert torch.equal(rows, x.permute(0, 2, 1, 3).reshape(b, s, h * d))
    back = HipRuntime.rows_to_heads(rows, h)
    assert torch.equal(back, x)


def test_layout_rejects_bad_inputs():
    qkv = torch.zeros((1, 8, 8 * 64), device=DEV, dtype=torch.bfloat16)
    cos = torch.zeros((8, 32), device=DEV)
    with pytest.raises(HkError):
        HipRuntime.qkv_rope_split(qkv.float(), cos, cos, 4, 2)                 # F32 rows
    with pytest.raises(HkError):
        HipRuntime.qkv_rope_split(qkv, cos[:7], cos[:7], 4, 2)                 # tables must cover S
    with pytest.raises(HkError):
        HipRuntime.qkv_rope_split(torch.zeros((1, 8, 8 * 24), device=DEV, dtype=torch.bfloat16),
                                  torch.zeros((8, 12), device=DEV), torch.zeros((8, 12), device=DEV), 4, 2)  # D % 16
    flat = torch.zeros(1 + 8 * 8 * 64, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(HkError):
        HipRuntime.qkv_rope_split(flat[1:].reshape(1, 8, 512), cos, cos, 4, 2)  # not 16-byte aligned
    with pytest.raises(HkError):
        HipRuntime.heads_to_rows(torch.zeros((1, 2, 3, 12), device=DEV, dtype=torch.bfloat16))  # D % 8
