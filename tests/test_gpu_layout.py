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


# ------------------------------------------------------------------ fused QKV projection / backward rows

def projection_inputs(b, s, hq, hkv, hidden, seed):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    x = (torch.randn((b * s, hidden), generator=g, device=DEV) / hidden ** 0.25).to(torch.bfloat16)
    w = (torch.randn(((hq + 2 * hkv) * 128, hidden), generator=g, device=DEV) / hidden ** 0.25).to(torch.bfloat16)
    cos, sin = oracle.rope_tables(np.arange(s), 128, 5e5)
    return x, w, dev_f32(cos), dev_f32(sin)


# (B, S, Hq, Hkv, H): C5's projection (a grid of 384 256x256 tiles, so hk_gemm_into runs the same
# tile kernel and the two paths must agree bit for bit), the same grid with K % 64 != 0 (the
# partial-last-stage variant), then small and ragged shapes (fewer tiles: hk_gemm_into takes
# another kernel there, so they are compared within the BF16 tolerance).
PROJ_EXACT = [(2, 2048, 32, 8, 4096), (4, 1024, 32, 8, 1008)]
PROJ_SMALL = [(2, 64, 4, 2, 256), (1, 48, 2, 1, 512), (3, 100, 1, 1, 200)]


@pytest.mark.parametrize("b,s,hq,hkv,hidden", PROJ_EXACT)
@pytest.mark.parametrize("layout", [0, 1])
def test_qkv_projection_rope_bit_exact_with_gemm_and_split(b, s, hq, hkv, hidden, layout):
    x, w, cos, sin = projection_inputs(b, s, hq, hkv, hidden, seed=s + hidden + layout)
    print(f"qkv projection rope {b}x{s} tokens, {hq}/{hkv} heads, H {hidden}, layout {layout}", flush=True)
    q, k, v = HipRuntime.qkv_projection_rope(x, w, cos, sin, b, hq, hkv, RotaryLayout(layout))
    rows = torch.empty((b, s, w.shape[0]), device=DEV, dtype=torch.bfloat16)
    HipRuntime.gemm_into(x, w, 0, 1, rows.view(b * s, -1))
    q2, k2, v2 = HipRuntime.qkv_rope_split(rows, cos, sin, hq, hkv, RotaryLayout(layout))
    assert torch.equal(q, q2) and torch.equal(k, k2) and torch.equal(v, v2)


@pytest.mark.parametrize("b,s,hq,hkv,hidden", PROJ_SMALL)
@pytest.mark.parametrize("layout", [0, 1])
def test_qkv_projection_rope_small_shapes_vs_oracle(b, s, hq, hkv, hidden, layout):
    x, w, cos, sin = projection_inputs(b, s, hq, hkv, hidden, seed=3 * s + hidden + layout)
    q, k, v = HipRuntime.qkv_projection_rope(x, w, cos, sin, b, hq, hkv, RotaryLayout(layout))
    y = oracle.gemm_f64(host(x), host(w), False, True).reshape(b, s, hq + 2 * hkv, 128).transpose(0, 2, 1, 3)
    y = oracle.bf16_round(y)  # the product's storage, before the rotation
    c4, s4 = host(cos)[None, None], host(sin)[None, None]
    want_q = oracle.rotary_prefix(y[:, :hq], c4, s4, 128, layout)
    want_k = oracle.rotary_prefix(y[:, hq:hq + hkv], c4, s4, 128, layout)
    # per head row (128 values): the rotation keeps each pair's norm, but where a pair's two terms
    # cancel an element can be ~0 while its rounding error stays ~2^-9 of the pair
    for got, want, name in ((q, want_q, "q"), (k, want_k, "k"), (v, y[:, hq + hkv:], "v")):
        e = oracle.row_err(host(got), want)
        assert e <= 1e-2, (name, e)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("form", ["stored_ds", "recompute"])
def test_attention_backward_qkv_rows_bit_exact_with_merge(d, layout, causal, form, monkeypatch):
    """The rows form of the attention backward equals the plane form (BF16 gradients) followed by
    qkv_rope_merge bit for bit, on both dQ forms, GQA with ragged tiles."""
    if form == "recompute":
        monkeypatch.setenv("HK_ATTN_DS_BUDGET", "0")
    else:
        monkeypatch.delenv("HK_ATTN_DS_BUDGET", raising=False)
    b, hq, hkv, s = 2, 4, 2, 200
    g = torch.Generator(device=DEV)
    g.manual_seed(d + 10 * layout + causal)
    q, k, v, do = (torch.randn(shape, generator=g, device=DEV).to(torch.bfloat16)
                   for shape in ((b, hq, s, d), (b, hkv, s, d), (b, hkv, s, d), (b, hq, s, d)))
    cos, sin = (dev_f32(t) for t in oracle.rope_tables(np.arange(s), d, 5e5))
    scale = d ** -0.5
    o, lse = HipRuntime.attention_forward(q, k, v, scale, causal)
    rows = HipRuntime.attention_backward_qkv_rows(q, k, v, o, lse, do, cos, sin, scale, causal,
                                                  layout=RotaryLayout(layout))
    dq, dk, dv = HipRuntime.attention_backward(q, k, v, o, lse, do, scale, causal, grad_dtype=torch.bfloat16)
    want = HipRuntime.qkv_rope_merge(dq, dk, dv, cos, sin, RotaryLayout(layout))
    assert torch.equal(rows, want)


def test_fused_projection_and_rows_reject_bad_inputs():
    x, w, cos, sin = projection_inputs(1, 64, 2, 1, 256, seed=1)
    q = torch.empty((1, 2, 64, 128), device=DEV, dtype=torch.bfloat16)
    kv = torch.empty((1, 1, 64, 128), device=DEV, dtype=torch.bfloat16)
    from rust_ascend_hip import runtime
    with pytest.raises(HkError):  # tables must cover S
        runtime._call("hk_qkv_projection_rope", runtime.desc(x), runtime.desc(w), runtime.desc(cos[:32]),
                      runtime.desc(sin[:32]), 1, runtime.desc(q), runtime.desc(kv), runtime.desc(kv.clone()))
    with pytest.raises(HkError):  # heads of width 64 are not taken by the fused projection
        w64 = torch.empty((4 * 64, 256), device=DEV, dtype=torch.bfloat16)
        q64, kv64 = q[..., :64].contiguous(), kv[..., :64].contiguous()
        runtime._call("hk_qkv_projection_rope", runtime.desc(x), runtime.desc(w64), runtime.desc(cos[:, :32].contiguous()),
                      runtime.desc(sin[:, :32].contiguous()), 1, runtime.desc(q64), runtime.desc(kv64),
                      runtime.desc(kv64.clone()))
    o, lse = HipRuntime.attention_forward(q, kv, kv, 0.1, True)
    with pytest.raises(HkError):  # the rows form needs as many keys as queries
        k2 = torch.zeros((1, 1, 80, 128), device=DEV, dtype=torch.bfloat16)
        HipRuntime.attention_backward_qkv_rows(q, k2, k2, o, lse, q, cos, sin, 0.1, True)
