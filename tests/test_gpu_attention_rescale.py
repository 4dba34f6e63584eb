"""GPU parity of the fused attention on scores that rise across key tiles, so the forward's
lagging running max rescales O and l after the first tile (hk_attention.hip, tile_softmax: a
rescale when some query of a wave sees its tile max pass its running max + 8 in base 2).

N(0,1) inputs reach that branch after the first tile with probability ~1e-6 per row. Here each
32-query wave has one pattern (tests/attn_cases.py): scores rising 12 or 3 base-2 units per
64-key tile, falling 5 per tile, or rising 90 per tile (|scale * s| ~ 1e3 at the end). A CPU
replay of the kernel's rule on the same inputs (asserted below, and in test_oracle.py) shows at
least two rescales after the first tile on nearly every rising row; test_oracle.py also shows
that a wrong rescale (l or O left unscaled, the reciprocal factor) moves O far beyond the per-row
check used here.

Checks, against the float64 oracle (examples/grouped_attention_tensor.rs:14-44 with its BF16
rounding points): forward O by the magnitude check and per row (<= 1e-2), lse to 1e-3 + 1e-5|b|;
backward dQ/dK/dV by the magnitude check (<= 1e-2), whose dS term includes the row term
rowsum(dO o O) -- with scores this peaked a row's dS nearly cancels on its dominant keys, so the
BF16 O in that term (FlashAttention's form) is measured against the terms, not the cancelled
sum -- and dV per row on rows holding at least 1e-3 of the largest row's norm (dV = P^T dO has no
row term)."""
import numpy as np
import pytest
import torch

import oracle
from attn_cases import PATTERNS, base2_scores, rescale_counts, rising_inputs
from gpu_util import close, dev_bf16, host, mag_ok, rows_ok

pytestmark = pytest.mark.gpu

M = N = 1024
B, H, HKV = 1, 4, 2

DQ_FORMS = {"stored_ds": None, "recompute": "0"}


@pytest.fixture(params=sorted(DQ_FORMS))
def dq_form(request, monkeypatch):
    budget = DQ_FORMS[request.param]
    if budget is None:
        monkeypatch.delenv("HK_ATTN_DS_BUDGET", raising=False)
    else:
        monkeypatch.setenv("HK_ATTN_DS_BUDGET", budget)
    return request.param


def inputs(d, causal):
    q, k, v, do, names = rising_inputs(B, H, HKV, M, N, d, seed=100 + d)
    counts = rescale_counts(base2_scores(q, k, d ** -0.5, causal))
    seen = np.arange(M) + 1 if causal else np.full(M, N)
    rising = np.array([PATTERNS[nm] > 0 for nm in names]) & (seen >= 512)
    # the inputs do what they are for: rescales after the first tile on the rising rows
    assert np.mean(counts[..., rising] >= 2) >= 0.9
    return q, k, v, do


def significant_rows(ref):
    r = np.asarray(ref, np.float64).reshape(-1, ref.shape[-1])
    nrm = np.linalg.norm(r, axis=1)
    return nrm >= 1e-3 * nrm.max()


@pytest.mark.parametrize("d", [16, 32, 64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_forward_rising_scores_rescale(d, causal):
    from rust_ascend_hip import HipRuntime
    q, k, v, _ = inputs(d, causal)
    print(f"forward rising scores d={d} causal={causal}", flush=True)
    o, lse = HipRuntime.attention_forward(dev_bf16(q), dev_bf16(k), dev_bf16(v), d ** -0.5, causal)
    ref = oracle.attention_f64(q, k, v, scale=d ** -0.5, causal=causal, magnitudes=True)
    assert np.all(np.isfinite(host(o))) and np.all(np.isfinite(host(lse)))
    mag_ok(host(o), ref["out"], ref["out_mag"], 1e-2, "O")
    rows_ok(host(o), ref["out"], 1e-2, "O rows")
    close(host(lse), ref["lse"], 1e-3, 1e-5, "lse")


@pytest.mark.parametrize("d", [16, 32, 64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_backward_rising_scores(d, causal, dq_form):
    from rust_ascend_hip import HipRuntime
    q, k, v, do = inputs(d, causal)
    print(f"backward rising scores d={d} causal={causal} form={dq_form}", flush=True)
    q_t, k_t, v_t, do_t = dev_bf16(q), dev_bf16(k), dev_bf16(v), dev_bf16(do)
    o, lse = HipRuntime.attention_forward(q_t, k_t, v_t, d ** -0.5, causal)
    dq, dk, dv = HipRuntime.attention_backward(q_t, k_t, v_t, o, lse, do_t, d ** -0.5, causal)
    ref = oracle.attention_f64(q, k, v, do, scale=d ** -0.5, causal=causal, magnitudes=True)
    for name, got in (("dq", dq), ("dk", dk), ("dv", dv)):
        g = host(got)
        assert np.all(np.isfinite(g)), name
        mag_ok(g, ref[name], ref[name + "_mag"], 1e-2, name)
    sig = significant_rows(ref["dv"])
    rows_ok(host(dv).reshape(-1, d)[sig], ref["dv"].reshape(-1, d)[sig], 1e-2, "dv rows")


@pytest.mark.parametrize("d", [16, 64, 128])
def test_backward_keys_after_queries(d, dq_form):
    """key_start > query_start: the leading query rows see no key (lse = -inf, zero dQ) and the
    dK/dV kernel skips whole query steps. The workspace is filled first by a larger stored-dS
    call, so a stale dS block that reached dQ would show."""
    from rust_ascend_hip import HipRuntime
    from gpu_util import randn_bf16
    # a larger backward first: the stored-dS workspace then holds blocks of another problem
    qa, _ = randn_bf16((2, 4, 512, d), seed=d + 1)
    ka, _ = randn_bf16((2, 2, 512, d), seed=d + 2)
    oa, la = HipRuntime.attention_forward(qa, ka, ka, d ** -0.5, True)
    HipRuntime.attention_backward(qa, ka, ka, oa, la, qa, d ** -0.5, True)
    m, n, qs, ks = 200, 260, 1000, 1100  # rows 0..99 see no key; row i sees keys 0..i-100
    q_t, q = randn_bf16((1, 4, m, d), seed=d + 3)
    k_t, k = randn_bf16((1, 2, n, d), seed=d + 4)
    v_t, v = randn_bf16((1, 2, n, d), seed=d + 5)
    do_t, do = randn_bf16((1, 4, m, d), seed=d + 6)
    print(f"backward keys after queries d={d} form={dq_form}", flush=True)
    o, lse = HipRuntime.attention_forward(q_t, k_t, v_t, d ** -0.5, True, qs, ks)
    dq, dk, dv = HipRuntime.attention_backward(q_t, k_t, v_t, o, lse, do_t, d ** -0.5, True, qs, ks)
    ref = oracle.attention_f64(q, k, v, do, scale=d ** -0.5, causal=True, query_start=qs, key_start=ks,
                               magnitudes=True)
    blind = ks - qs
    assert torch.all(torch.isneginf(lse[:, :, :blind]))
    assert torch.count_nonzero(dq[:, :, :blind]) == 0
    for name, got in (("dq", dq), ("dk", dk), ("dv", dv)):
        g = host(got)
        assert np.all(np.isfinite(g)), name
        mag_ok(g, ref[name], ref[name + "_mag"], 1e-2, name)
    # keys past the last query's reach get no gradient at all
    last_key = qs + m - 1 - ks
    assert torch.count_nonzero(dk[:, :, last_key + 1:]) == 0 and torch.count_nonzero(dv[:, :, last_key + 1:]) == 0
    rows_ok(host(dv)[:, :, :last_key + 1], ref["dv"][:, :, :last_key + 1], 1e-2, "dv rows")
    rows_ok(host(dk)[:, :, :last_key + 1], ref["dk"][:, :, :last_key + 1], 1e-2, "dk rows")
