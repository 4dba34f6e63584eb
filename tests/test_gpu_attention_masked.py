"""GPU parity of the reference's FP32 attention surface (src/nn/attention.rs:10-80) through the C ABI:

* the materialized path with an additive mask and its gradient (hk_attention_masked_forward /
  _backward), on the reference's own GQA cases (examples/grouped_attention_tensor.rs:74-97,
  tolerance 2e-3 + 3e-3|b|, out/dQ/dK/dV/dMask against the stored torch-f64 golden vectors and
  against the oracle, which keeps the reference's BF16 rounding points), value widths other than
  the head width, head widths the fused kernels do not take, rank-3 SDPA;
* the fused kernels with F32 Q/K/V and F32 O (hk_attention_forward / _backward), where the
  backward's row term rowsum(dO * O) comes from the unrounded O.
"""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import DEV, close, dev_f32, host, mag_ok, rows_ok
from rust_ascend_hip import HipRuntime, HkError, nn

pytestmark = pytest.mark.gpu

MASKED_CASES = ["kv3_g1_n32_c0", "kv1_g3_n96_c0", "kv3_g2_n32_c0", "kv3_g5_n96_c0"]
REF_TOL = dict(atol=2e-3, rtol=3e-3)  # grouped_attention_tensor.rs:10


def golden_case(golden, case):
    return {k[len("attn_" + case) + 1:]: v for k, v in golden.items() if k.startswith("attn_" + case + "_")}


@pytest.mark.parametrize("case", MASKED_CASES)
def test_reference_gqa_cases_with_mask(golden, case):
    """nn::grouped_query_attention_bf16_fp32 with Some(mask): output and all four gradients,
    the mask's included (grouped_attention_tensor.rs:84-96)."""
    g = golden_case(golden, case)
    q, k, v, mask = (dev_f32(g[x]).requires_grad_() for x in ("q", "k", "v", "mask"))
    o = nn.grouped_query_attention_bf16_fp32(q, k, v, 0.25, mask)
    assert o.dtype == torch.float32
    o.backward(dev_f32(g["dy"]))
    ref = oracle.attention_f64(g["q"], g["k"], g["v"], g["dy"], scale=0.25, mask=g["mask"])
    for name, got in (("out", o), ("dq", q.grad), ("dk", k.grad), ("dv", v.grad), ("dmask", mask.grad)):
        close(host(got), g[name], REF_TOL["atol"], REF_TOL["rtol"], name + " vs golden")
        close(host(got), ref[name], REF_TOL["atol"], REF_TOL["rtol"], name + " vs oracle")


def test_reference_causal_case_fp32_surface(golden):
    """nn::causal_grouped_query_attention_bf16_fp32 on the reference's causal case (absolute starts
    2^40 + (n - m) and 2^40): the fused kernels with F32 in and out."""
    g = golden_case(golden, "kv3_g3_n96_c1")
    q, k, v = (dev_f32(g[x]).requires_grad_() for x in ("q", "k", "v"))
    o = nn.causal_grouped_query_attention_bf16_fp32(q, k, v, 0.25, (1 << 40) + 64, 1 << 40)
    assert o.dtype == torch.float32
    o.backward(dev_f32(g["dy"]))
    for name, got in (("out", o), ("dq", q.grad), ("dk", k.grad), ("dv", v.grad)):
        close(host(got), g[name], REF_TOL["atol"], REF_TOL["rtol"], name + " vs golden")


def test_materialized_causal_mask_equals_fused(golden):
    """The same causal case through the materialized path (the reference's own composition: a
    device-generated causal mask added to the scores) agrees with the fused kernels."""
    g = golden_case(golden, "kv3_g3_n96_c1")
    q, k, v, dy = (dev_f32(g[x]) for x in ("q", "k", "v", "dy"))
    mask = dev_f32(g["mask"])
    o = HipRuntime.attention_masked_forward(q, k, v, 0.25, mask)
    dq, dk, dv, _ = HipRuntime.attention_masked_backward(q, k, v, mask, dy, 0.25)
    for name, got in (("out", o), ("dq", dq), ("dk", dk), ("dv", dv)):
        close(host(got), g[name], REF_TOL["atol"], REF_TOL["rtol"], name + " (materialized) vs golden")


@pytest.mark.parametrize("d,dv,causal", [(64, 128, False), (48, 80, True), (80, 80, True), (96, 32, False),
                                         (128, 64, True)])
def test_value_and_head_widths_off_the_fused_path(d, dv, causal):
    """Value widths other than the head width and head widths other than 16/32/64/128 (any
    multiple of 16, src/nn/attention.rs:95-100) run the materialized path; against the oracle."""
    B, H, Hkv, M, N = 2, 4, 2, 64, 160
    rng = np.random.default_rng(d * 1000 + dv)
    q = oracle.bf16_round(rng.standard_normal((B, H, M, d)).astype(np.float32))
    k = oracle.bf16_round(rng.standard_normal((B, Hkv, N, d)).astype(np.float32))
    v = oracle.bf16_round(rng.standard_normal((B, Hkv, N, dv)).astype(np.float32))
    dy = oracle.bf16_round(rng.standard_normal((B, H, M, dv)).astype(np.float32))
    qt, kt, vt = (dev_f32(x).requires_grad_() for x in (q, k, v))
    scale = d ** -0.5
    if causal:
        o = nn.causal_grouped_query_attention_bf16_fp32(qt, kt, vt, scale, N - M, 0)
        ref = oracle.attention_f64(q, k, v, dy, scale=scale, causal=True, query_start=N - M, magnitudes=True)
    else:
        mask = (rng.standard_normal((B, H, M, N)) * 0.5).astype(np.float32)
        mask[:, :, 5, 40:100] = -np.inf
        o = nn.grouped_query_attention_bf16_fp32(qt, kt, vt, scale, dev_f32(mask))
        ref = oracle.attention_f64(q, k, v, dy, scale=scale, mask=mask, magnitudes=True)
    assert o.shape == (B, H, M, dv)
    o.backward(dev_f32(dy))
    mag_ok(host(o), ref["out"], ref["out_mag"], 1e-2, "O")
    rows_ok(host(o), ref["out"], 1e-2, "O rows")
    for name, t in (("dq", qt), ("dk", kt), ("dv", vt)):
        mag_ok(host(t.grad), ref[name], ref[name + "_mag"], 1e-2, name)
        rows_ok(host(t.grad), ref[name], 1e-2, name + " rows")


def test_rank3_sdpa_and_causal_attention():
    """nn::scaled_dot_product_attention_bf16_fp32 (with and without a mask) and
    nn::causal_attention_bf16_fp32 on rank-3 Q[B,M,D], K[B,N,D], V[B,N,Dv]."""
    B, M, N, D = 3, 32, 96, 32
    rng = np.random.default_rng(5)
    q = oracle.bf16_round(rng.standard_normal((B, M, D)).astype(np.float32))
    k = oracle.bf16_round(rng.standard_normal((B, N, D)).astype(np.float32))
    v = oracle.bf16_round(rng.standard_normal((B, N, D)).astype(np.float32))
    mask = (rng.standard_normal((B, M, N)) * 0.3).astype(np.float32)
    for name, fn, ref in (
            ("sdpa+mask", lambda: nn.scaled_dot_product_attention_bf16_fp32(dev_f32(q), dev_f32(k), dev_f32(v), 0.2,
                                                                            dev_f32(mask)),
             oracle.attention_f64(q[:, None], k[:, None], v[:, None], scale=0.2, mask=mask[:, None], magnitudes=True)),
            ("sdpa", lambda: nn.scaled_dot_product_attention_bf16_fp32(dev_f32(q), dev_f32(k), dev_f32(v), 0.2),
             oracle.attention_f64(q[:, None], k[:, None], v[:, None], scale=0.2, magnitudes=True)),
            ("causal", lambda: nn.causal_attention_bf16_fp32(dev_f32(q), dev_f32(k), dev_f32(v), 0.2, N - M, 0),
             oracle.attention_f64(q[:, None], k[:, None], v[:, None], scale=0.2, causal=True, query_start=N - M,
                                  magnitudes=True))):
        o = fn()
        assert o.shape == (B, M, D) and o.dtype == torch.float32, name
        mag_ok(host(o), ref["out"][:, 0], ref["out_mag"][:, 0], 1e-2, name)


def test_fp32_fused_path_row_term_from_unrounded_o():
    """F32 Q/K/V with F32 O on the fused kernels: the backward's row term uses the unrounded O,
    so dQ meets the per-row check on every row that sees a key (the BF16-O path needs >= 128
    keys per row for that, its row term carrying O's BF16 rounding)."""
    B, H, Hkv, S, D = 1, 8, 2, 1024, 128
    rng = np.random.default_rng(17)
    q, k, v, do = (oracle.bf16_round(rng.standard_normal(shape).astype(np.float32))
                   for shape in ((B, H, S, D), (B, Hkv, S, D), (B, Hkv, S, D), (B, H, S, D)))
    qt, kt, vt, dot = (dev_f32(x) for x in (q, k, v, do))
    o, lse = HipRuntime.attention_forward(qt, kt, vt, D ** -0.5, True, out_dtype=torch.float32)
    assert o.dtype == torch.float32
    o_b, _ = HipRuntime.attention_forward(qt.to(torch.bfloat16), kt.to(torch.bfloat16), vt.to(torch.bfloat16),
                                          D ** -0.5, True)
    assert torch.equal(o.to(torch.bfloat16).view(torch.int16), o_b.view(torch.int16))  # same kernel, one rounding
    dq, dk, dv = HipRuntime.attention_backward(qt, kt, vt, o, lse, dot, D ** -0.5, True)
    ref = oracle.attention_f64(q, k, v, do, scale=D ** -0.5, causal=True, magnitudes=True)
    rows_ok(host(o), ref["out"], 1e-2, "O rows")
    rows_ok(host(dq)[:, :, 16:], ref["dq"][:, :, 16:], 1e-2, "dq rows")
    for name, got in (("dq", dq), ("dk", dk), ("dv", dv)):
        mag_ok(host(got), ref[name], ref[name + "_mag"], 1e-2, name)
    rows_ok(host(dk), ref["dk"], 1e-2, "dk rows")
    rows_ok(host(dv), ref["dv"], 1e-2, "dv rows")


def test_masked_contract_errors_leave_the_context_healthy():
    q = dev_f32(np.zeros((1, 2, 16, 16), np.float32))
    k = dev_f32(np.zeros((1, 1, 48, 16), np.float32))  # N % 32 != 0
    with pytest.raises(HkError):
        HipRuntime.attention_masked_forward(q, k, k, 0.25)
    k = dev_f32(np.zeros((1, 1, 64, 16), np.float32))
    with pytest.raises(HkError):  # mask of the wrong shape
        HipRuntime.attention_masked_forward(q, k, k, 0.25, dev_f32(np.zeros((1, 2, 16, 32), np.float32)))
    with pytest.raises(HkError, match="mask gradient"):
        _dmask_without_mask(q, k)
    o = HipRuntime.attention_masked_forward(q, k, k, 0.25)
    assert float(torch.abs(o).max()) == 0.0


def _dmask_without_mask(q, k):
    from rust_ascend_hip import runtime
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(k)
    dmask = torch.empty((1, 2, 16, 64), dtype=torch.float32, device=DEV)
    runtime._call("hk_attention_masked_backward", runtime.desc(q), runtime.desc(k), runtime.desc(k), None,
                  runtime.desc(q), 0.25, runtime.desc(dq), runtime.desc(dk), runtime.desc(dv), runtime.desc(dmask))
