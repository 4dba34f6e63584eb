"""Pins the CPU oracle (oracle/) against the golden vectors, closed forms and
float64 autograd. CPU only. See oracle/oracle.py's header for what pins what."""
import numpy as np
import pytest
import torch


def close(actual, expected, atol, rtol):
    a = np.asarray(actual, dtype=np.float64)
    b = np.asarray(expected, dtype=np.float64)
    assert a.shape == b.shape, (a.shape, b.shape)
    bad = ~(np.abs(a - b) <= atol + rtol * np.abs(b))
    assert not bad.any(), f"{bad.sum()} mismatches, first at {np.argwhere(bad)[0]}: {a[bad][0]} vs {b[bad][0]}"


# ------------------------------------------------------------------ BF16

def test_bf16_rounding_bit_patterns(oracle):
    cases = {
        1.0: 0x3F80, 1.00390625: 0x3F80,          # tie -> even (down)
        1.01171875: 0x3F82,                        # tie -> even (up)
        -0.0: 0x8000, 3.0e38: 0x7F62, 3.4e38: 0x7F80,  # finite; overflow to +Inf
        float("inf"): 0x7F80, float("-inf"): 0xFF80,
    }
    for x, bits in cases.items():
        assert int(oracle.bf16_bits(np.array([x], np.float32))[0]) == bits, x
    nan = np.array([0x7FC01234], dtype=np.uint32).view(np.float32)
    assert int(oracle.bf16_bits(nan)[0]) == 0x7FC0  # NaN keeps top bits, stays NaN


def test_bf16_rounding_matches_torch(oracle):
    x = oracle.normal((1 << 16,), seed=3, stream=1, std=100.0)
    x[:64] = np.ldexp(np.float32(1.0) + np.arange(64, dtype=np.float32) / 256, -130)  # subnormals
    want = torch.tensor(x).to(torch.bfloat16).to(torch.float32).numpy()
    np.testing.assert_array_equal(oracle.bf16_round(x), want)


def test_normal_generator_is_deterministic_and_standard(oracle):
    a = oracle.normal((4096, 64), seed=0, stream=5)
    b = oracle.normal((4096, 64), seed=0, stream=5)
    c = oracle.normal((4096, 64), seed=0, stream=6)
    np.testing.assert_array_equal(a, b)
    assert not np.array_equal(a, c)
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1) < 0.01


# ------------------------------------------------------------------ GEMM

@pytest.mark.parametrize("batch", [1, 3])
@pytest.mark.parametrize("ta", [0, 1])
@pytest.mark.parametrize("tb", [0, 1])
def test_gemm_deepgemm_validate_cases(oracle, golden, batch, ta, tb):
    key = f"gemm_dv_b{batch}_{'tn'[ta]}{'tn'[tb]}"
    a, b, want = golden[key + "_a"], golden[key + "_b"], golden[key + "_out"]
    close(oracle.gemm_f64(a, b, ta, tb), want, 1e-12, 0)
    close(oracle.gemm_f32(a, b, ta, tb), want, 1e-4, 1e-5)


@pytest.mark.parametrize("shape", ["1x80x96x144", "3x16x32x16"])
@pytest.mark.parametrize("ta", [0, 1])
@pytest.mark.parametrize("tb", [0, 1])
def test_gemm_kernel_vm_cases(oracle, golden, shape, ta, tb):
    key = f"gemm_vm_{shape}_{'nt'[ta]}{'nt'[tb]}"
    a, b, want = golden[key + "_a"], golden[key + "_b"], golden[key + "_out"]
    close(oracle.gemm_f64(a, b, ta, tb), want, 1e-12, 0)
    # rust-ascend-kernels/src/tests.rs:117 compares at 1e-4 absolute
    close(oracle.gemm_f32(a, b, ta, tb), want, 1e-4, 0)


@pytest.mark.parametrize("case", ["vm", "dv"])
def test_gemm_grouped_reference_cases(oracle, golden, case):
    # rust-ascend-kernels/src/tests.rs:130-132 (two empty experts) and deepgemm_validate.rs:45-53
    a, w, ends = golden[f"grouped_{case}_a"], golden[f"grouped_{case}_w"], golden[f"grouped_{case}_ends"]
    close(oracle.gemm_grouped_nt_f64(a, w, ends), golden[f"grouped_{case}_out"], 1e-12, 0)


def test_gemm_grouped_identities(oracle):
    rng = np.random.default_rng(7)
    a = rng.standard_normal((512, 32)).astype(np.float32)
    w = rng.standard_normal((3, 48, 32)).astype(np.float32)
    # one group is the dense NT product
    close(oracle.gemm_grouped_nt_f64(a, w[:1], [512]), oracle.gemm_f64(a, w[0], 0, 1), 1e-12, 1e-12)
    # a leading and a middle empty expert take no rows; each row slice uses its own weights
    y = oracle.gemm_grouped_nt_f64(a, w, [0, 256, 512])
    close(y[:256], a[:256].astype(np.float64) @ w[1].T.astype(np.float64), 1e-10, 1e-12)
    close(y[256:], a[256:].astype(np.float64) @ w[2].T.astype(np.float64), 1e-10, 1e-12)
    y = oracle.gemm_grouped_nt_f64(a, w, [256, 256, 512])
    close(y[256:], a[256:].astype(np.float64) @ w[2].T.astype(np.float64), 1e-10, 1e-12)
    assert not np.allclose(y[256:], a[256:].astype(np.float64) @ w[1].T.astype(np.float64))


@pytest.mark.parametrize("batch", [1, 2])
@pytest.mark.parametrize("mnk", ["1x1x1", "3x17x7", "17x33x65", "16x32x48"])
@pytest.mark.parametrize("ta", [0, 1])
@pytest.mark.parametrize("tb", [0, 1])
def test_gemm_on_padded_reference_cases(oracle, golden, batch, mnk, ta, tb):
    # examples/padded_matrix_tensor.rs:12-45: logical shapes that are not multiples of 16; the
    # oracle's product of BF16-rounded operands is the padded GEMM's expectation
    key = f"padded_{batch}_{mnk}_{'nt'[ta]}{'nt'[tb]}"
    a, b = oracle.bf16_round(golden[key + "_a"]), oracle.bf16_round(golden[key + "_b"])
    close(oracle.gemm_f64(a, b, ta, tb), golden[key + "_y"], 1e-12, 1e-12)


def test_gemm_random_vs_numpy_and_transpose_identity(oracle):
    a = oracle.normal((3, 40, 24), 1, 1)
    b = oracle.normal((3, 24, 56), 1, 2)
    want = np.einsum("gik,gkj->gij", a.astype(np.float64), b.astype(np.float64))
    close(oracle.gemm_f64(a, b, 0, 0), want, 1e-10, 1e-12)
    # (A B)^T = B^T A^T, through the transposed addressing
    at = np.ascontiguousarray(a.transpose(0, 2, 1))
    bt = np.ascontiguousarray(b.transpose(0, 2, 1))
    close(oracle.gemm_f64(at, bt, 1, 1), want, 1e-10, 1e-12)
    close(oracle.gemm_f64(bt, at, 0, 0).transpose(0, 2, 1), want, 1e-10, 1e-12)
    rows = np.array([0, 5, 39, 17])
    cols = np.array([0, 55, 3, 28])
    close(oracle.gemm_f64_sampled(a[0], b[0], 0, 0, rows, cols), want[0][rows, cols], 1e-12, 0)
    close(oracle.gemm_f64_sampled(at[0], b[0], 1, 0, rows, cols), want[0][rows, cols], 1e-12, 0)


def test_linear_backward_gradient_identity(oracle, golden):
    """dX = dY W and dW = dY^T X (matrix_runtime.rs:70-77) and the finite-difference
    identity of tools/ascend/tests/test_adapter.py:89-93."""
    x, w, dy = golden["linbwd_x"], golden["linbwd_w"], golden["linbwd_dy"]
    dx = oracle.gemm_f64(dy, w, 0, 0)
    dw = oracle.gemm_f64(dy, x, 1, 0)
    close(dx, golden["linbwd_dx"], 1e-12, 0)
    close(dw, golden["linbwd_dw"], 1e-12, 0)
    y = oracle.gemm_f64(x, w, 0, 1)
    for p, q in [(0, 0), (8, 3), (31, 15)]:
        xx = x.astype(np.float64).copy()
        xx[p, q] += 1.0  # linear: the difference is exact
        yy = xx @ w.astype(np.float64).T
        assert abs(np.sum((yy - y) * dy) - dx[p, q]) < 1e-9


# ------------------------------------------------------------------ RMSNorm

@pytest.mark.parametrize("case", ["0x32", "1x32", "3x96", "7x256", "33x4096", "3x7", "2x4100"])
def test_rms_norm_f64_vs_autograd(oracle, golden, case):
    g = {k[len("rms_" + case) + 1:]: v for k, v in golden.items() if k.startswith("rms_" + case + "_")}
    y, rstd = oracle.rms_norm_f64(g["x"], g["w"], 1e-3)
    close(y, g["y"], 1e-12, 1e-12)
    close(rstd, g["rstd"], 1e-12, 1e-12)
    dx, dw = oracle.rms_norm_backward_f64(g["x"], g["w"], g["dy"], rstd)
    close(dx, g["dx"], 1e-11, 1e-11)
    close(dw, g["dw"], 1e-10, 1e-11)


@pytest.mark.parametrize("case", ["1x32", "3x96", "7x256", "33x4096"])
def test_rms_norm_lanes_f32_vs_autograd(oracle, golden, case):
    g = {k[len("rms_" + case) + 1:]: v for k, v in golden.items() if k.startswith("rms_" + case + "_")}
    y, rstd = oracle.rms_norm_lanes_f32(g["x"], g["w"], 1e-3)
    close(y, g["y"], 2e-6, 1e-5)
    close(rstd, g["rstd"], 0, 1e-6)
    dx, dw = oracle.rms_norm_backward_lanes_f32(g["x"], g["w"], g["dy"], rstd)
    close(dx, g["dx"], 2e-6, 1e-5)
    close(dw, g["dw"], 5e-5, 1e-5)


def test_rms_norm_gradients_rs_vectors(oracle, golden):
    x, w, dy = golden["rmsgrad_x"], golden["rmsgrad_w"], golden["rmsgrad_dy"]
    y, rstd = oracle.rms_norm_f64(x, w, 1e-5)
    close(y, golden["rmsgrad_y"], 1e-12, 1e-12)
    dx, dw = oracle.rms_norm_backward_f64(x, w, dy, rstd)
    close(dx, golden["rmsgrad_dx"], 1e-12, 1e-12)
    close(dw, golden["rmsgrad_dw"], 1e-12, 1e-12)


def test_rms_weight_contribution_known_answer(oracle, golden):
    """row_tests.rs:280-287: x = 2, dy = 3, rstd = [.5,.25,2] -> contributions [3,1.5,12].
    With width 32 and w = 1, the contribution of row r to dw is (x*rstd)*dy per column,
    so a one-row backward gives dw = 3, 1.5 and 12."""
    for r, want in zip(golden["rmskat_rstd"], golden["rmskat_contrib"]):
        x = np.full((1, 32), 2.0, np.float32)
        dy = np.full((1, 32), 3.0, np.float32)
        w = np.ones(32, np.float32)
        _, dw = oracle.rms_norm_backward_lanes_f32(x, w, dy, np.array([r], np.float32))
        np.testing.assert_array_equal(dw, np.full(32, want, np.float32))
        _, dw64 = oracle.rms_norm_backward_f64(x, w, dy, np.array([r], np.float64))
        np.testing.assert_array_equal(dw64, np.full(32, want))


def test_rms_constant_row_and_pairwise_tree(oracle):
    # test_row_reference.py:81-83: a constant 1000 row's mean is exactly 1000 -> y = w*sign
    x = np.full((3, 4096), 1000.0, np.float32)
    w = np.linspace(0.5, 1.5, 4096).astype(np.float32)
    y, rstd = oracle.rms_norm_lanes_f32(x, w, 1e-6)
    np.testing.assert_allclose(rstd, np.full(3, 1e-3), rtol=1e-6)
    np.testing.assert_allclose(y, np.broadcast_to(w, (3, 4096)), rtol=1e-6)
    # normalization.rs:95-114: odd rows are carried; rows == 0 gives zeros
    for rows in (0, 1, 2, 3, 5, 7, 16, 33):
        parts = np.arange(rows * 5, dtype=np.float32).reshape(rows, 5)
        np.testing.assert_array_equal(oracle.column_sum_pairwise(parts), parts.sum(0) if rows else np.zeros(5))


# ------------------------------------------------------------------ RoPE

@pytest.mark.parametrize("case", ["0x6", "1x2", "3x6", "2x96"])
@pytest.mark.parametrize("layout", [0, 1])
def test_rotary_vs_autograd(oracle, golden, case, layout):
    key = f"rope_{case}_l{layout}"
    x, dy, c, s = (golden[key + s_] for s_ in ("_x", "_dy", "_cos", "_sin"))
    close(oracle.rotary_f64(x, c, s, layout), golden[key + "_y"], 1e-12, 1e-12)
    close(oracle.rotary_f64(dy, c, s, layout, True), golden[key + "_dx"], 1e-12, 1e-12)
    # device order in f32 (rotary_tensor.rs:8: 2e-5 + 1e-4|b|)
    close(oracle.rotary(x, c, s, layout), golden[key + "_y"], 2e-6, 2e-6)
    close(oracle.rotary(dy, c, s, layout, True), golden[key + "_dx"], 2e-6, 2e-6)


def test_rotary_invariants(oracle):
    x = oracle.normal((5, 64), 0, 1)
    ang = oracle.normal((5, 32), 0, 2)
    c, s = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    for layout in (0, 1):
        y = oracle.rotary_f64(x, c, s, layout)
        # pair norms are preserved
        if layout == 0:
            na, nb = x[:, 0::2], x[:, 1::2]
            ya, yb = y[:, 0::2], y[:, 1::2]
        else:
            na, nb, ya, yb = x[:, :32], x[:, 32:], y[:, :32], y[:, 32:]
        np.testing.assert_allclose(ya ** 2 + yb ** 2, na.astype(np.float64) ** 2 + nb.astype(np.float64) ** 2, rtol=1e-5)
        # backward undoes forward (rotation is orthogonal)
        back = oracle.rotary_f64(y.astype(np.float32), c, s, layout, True)
        np.testing.assert_allclose(back, x, atol=1e-5)
        # angle 0 is the identity
        np.testing.assert_array_equal(oracle.rotary(x, np.ones_like(c), np.zeros_like(s), layout), x)


@pytest.mark.parametrize("ci", range(5))
@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("backward", [0, 1])
def test_rotary_prefix_golden(oracle, golden, ci, layout, backward):
    key = f"ropepre_{ci}_l{layout}_b{backward}"
    x, c, s, want = golden[key + "_x"], golden[key + "_cos"], golden[key + "_sin"], golden[key + "_y"]
    y = oracle.rotary_prefix(x, c, s, 6, layout, bool(backward))
    head = (slice(None),) * (x.ndim - 1) + (slice(0, 6),)
    tail = (slice(None),) * (x.ndim - 1) + (slice(6, None),)
    close(y[head], want[head], 3e-6, 3e-6)
    np.testing.assert_array_equal(y[tail].view(np.uint32), x[tail].view(np.uint32))


def test_rotary_prefix_full_width_equals_rotary(oracle):
    x = (np.arange(18, dtype=np.float32) / 8).reshape(3, 6)
    c = np.full((3, 3), 0.75, np.float32)
    s = np.full((3, 3), 0.25, np.float32)
    for layout in (0, 1):
        for bw in (False, True):
            np.testing.assert_array_equal(oracle.rotary_prefix(x, c, s, 6, layout, bw),
                                          oracle.rotary(x, c, s, layout, bw))
    for bad in (0, 5, 8):
        with pytest.raises(ValueError):
            oracle.rotary_prefix(x, c, s, bad, 0)


# ------------------------------------------------------------------ attention

@pytest.mark.parametrize("case", ["kv3_g1_n32_c0", "kv1_g3_n96_c0", "kv3_g2_n32_c0", "kv3_g5_n96_c0", "kv3_g3_n96_c1"])
def test_attention_reference_cases_vs_autograd(oracle, golden, case):
    g = {k[len("attn_" + case) + 1:]: v for k, v in golden.items() if k.startswith("attn_" + case + "_")}
    causal = case.endswith("c1")
    n = g["k"].shape[2]
    m = g["q"].shape[2]
    kw = dict(scale=0.25, causal=causal, query_start=(1 << 40) + n - m, key_start=1 << 40)
    if not causal:
        kw["mask"] = g["mask"]
    r = oracle.attention_f64(g["q"], g["k"], g["v"], g["dy"], **kw)
    tol = dict(atol=2e-3, rtol=3e-3)  # grouped_attention_tensor.rs:10
    close(r["out"], g["out"], **tol)
    close(r["lse"], g["lse"], 1e-9, 1e-12)  # no BF16 rounding enters the scores' lse
    close(r["dq"], g["dq"], **tol)
    close(r["dk"], g["dk"], **tol)
    close(r["dv"], g["dv"], **tol)
    if not causal:  # grouped_attention_tensor.rs:95: the mask gradient
        close(r["dmask"], g["dmask"], **tol)


@pytest.mark.parametrize("d,dv", [(16, 48), (48, 16), (32, 32)])
def test_attention_value_width_and_mask_grad_vs_autograd(oracle, d, dv):
    """A value width other than the head width (src/nn/attention.rs:49-52 allows any) and the
    mask gradient, against torch float64 autograd of softmax(scale QK^T + mask) V with GQA by
    repeated heads; inputs exactly representable in BF16, so only the oracle's BF16 rounding of
    P and dS separates the two (the reference's tolerance 2e-3 + 3e-3|b|)."""
    B, H, Hkv, M, N = 2, 4, 2, 16, 64
    # magnitudes like the reference's cases (|x| <= 0.5), where its absolute tolerance applies
    q = oracle.bf16_round(oracle.normal((B, H, M, d), 9, 1, std=0.25))
    k = oracle.bf16_round(oracle.normal((B, Hkv, N, d), 9, 2, std=0.25))
    v = oracle.bf16_round(oracle.normal((B, Hkv, N, dv), 9, 3, std=0.25))
    dy = oracle.bf16_round(oracle.normal((B, H, M, dv), 9, 4, std=0.25))
    mask = (oracle.normal((B, H, M, N), 9, 5) * 0.5).astype(np.float32)
    mask[:, :, 3, 10:40] = -np.inf
    r = oracle.attention_f64(q, k, v, dy, scale=0.3, mask=mask)
    tq, tk, tv, tm = (torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (q, k, v, mask))
    kk, vv = tk.repeat_interleave(H // Hkv, 1), tv.repeat_interleave(H // Hkv, 1)
    p = torch.softmax(0.3 * tq @ kk.transpose(-1, -2) + tm, -1)
    o = p @ vv
    (o * torch.tensor(dy, dtype=torch.float64)).sum().backward()
    tol = dict(atol=2e-3, rtol=3e-3)
    close(r["out"], o.detach().numpy(), **tol)
    for name, t in (("dq", tq), ("dk", tk), ("dv", tv), ("dmask", tm)):
        close(r[name], t.grad.numpy(), **tol)
    assert r["out"].shape == (B, H, M, dv) and r["dv"].shape == (B, Hkv, N, dv)


def test_attention_causal_equals_explicit_mask(oracle, golden):
    g = {k[len("attn_kv3_g3_n96_c1") + 1:]: v for k, v in golden.items() if k.startswith("attn_kv3_g3_n96_c1_")}
    a = oracle.attention_f64(g["q"], g["k"], g["v"], g["dy"], scale=0.25, causal=True,
                             query_start=(1 << 40) + 64, key_start=1 << 40)
    b = oracle.attention_f64(g["q"], g["k"], g["v"], g["dy"], scale=0.25, causal=False, mask=g["mask"])
    for key in ("out", "lse", "dq", "dk", "dv"):
        np.testing.assert_array_equal(a[key], b[key])


@pytest.mark.parametrize("n", [32, 256])
def test_attention_orthogonal_closed_form(oracle, golden, n):
    key = f"attnkat_orth_n{n}"
    q, k, v, dy = (golden[key + s][:, None] for s in ("_q", "_k", "_v", "_dy"))
    r = oracle.attention_f64(q, k, v, dy, scale=0.25)
    for name in ("out", "dq", "dk", "dv"):
        close(r[name][:, 0], golden[key + "_" + name], 5e-4, 5e-4)


@pytest.mark.parametrize("n", [32, 96])
@pytest.mark.parametrize("cached", [0, 1])
def test_attention_causal_closed_form(oracle, golden, n, cached):
    key = f"attnkat_causal_n{n}_c{cached}"
    v, dy, qs = golden[key + "_v"][:, None], golden[key + "_dy"][:, None], int(golden[key + "_qs"])
    q = np.zeros((2, 1, 32, 16), np.float32)
    k = np.zeros((2, 1, n, 16), np.float32)
    r = oracle.attention_f64(q, k, v, dy, scale=0.25, causal=True, query_start=qs, key_start=0)
    close(r["out"][:, 0], golden[key + "_out"], 5e-4, 5e-4)   # attention_tensor.rs close(): 5e-4+5e-4|b|
    close(r["dv"][:, 0], golden[key + "_dv"], 5e-4, 5e-4)
    assert np.all(r["dq"] == 0) and np.all(r["dk"] == 0)


def test_causal_mask_bit_patterns(oracle, golden):
    for ci in range(3):
        b, qn, kn, qs, ks = (int(x) for x in golden[f"mask_{ci}_spec"])
        np.testing.assert_array_equal(oracle.causal_mask(b, qn, kn, qs, ks).view(np.uint32),
                                      golden[f"mask_{ci}"].view(np.uint32))


def test_attention_fully_masked_rows_are_zero(oracle):
    q = oracle.normal((1, 1, 4, 16), 0, 1)
    k = oracle.normal((1, 1, 4, 16), 0, 2)
    v = oracle.normal((1, 1, 4, 16), 0, 3)
    dy = oracle.normal((1, 1, 4, 16), 0, 4)
    # key_start 2 > query_start 0: rows 0 and 1 see no key
    r = oracle.attention_f64(q, k, v, dy, causal=True, query_start=0, key_start=2)
    assert np.all(r["out"][0, 0, :2] == 0) and np.all(np.isneginf(r["lse"][0, 0, :2]))
    assert np.all(r["dq"][0, 0, :2] == 0)
    assert np.all(np.isfinite(r["out"]))


def test_attention_magnitudes_bound_the_outputs(oracle):
    """Each magnitude is the sum of |terms|: >= |value| everywhere, == value when every term
    is non-negative (V, dY >= 0 give O, dV >= 0), and it scales linearly with V."""
    q = oracle.normal((1, 2, 40, 32), 0, 1)
    k = oracle.normal((1, 1, 72, 32), 0, 2)
    v = oracle.normal((1, 1, 72, 32), 0, 3)
    dy = oracle.normal((1, 2, 40, 32), 0, 4)
    r = oracle.attention_f64(q, k, v, dy, scale=0.2, causal=True, query_start=32, magnitudes=True)
    for name in ("out", "dq", "dk", "dv"):  # the BF16-rounded terms may exceed theirs by 2^-8
        assert np.all(r[name + "_mag"] * (1 + 2.0 ** -8) >= np.abs(r[name]) - 1e-12), name
    rp = oracle.attention_f64(q, k, np.abs(v), np.abs(dy), scale=0.2, causal=True, query_start=32, magnitudes=True)
    np.testing.assert_allclose(rp["out_mag"], rp["out"], rtol=1e-12)
    np.testing.assert_allclose(rp["dv_mag"], rp["dv"], rtol=1e-12)
    r2 = oracle.attention_f64(q, k, 2 * v, dy, scale=0.2, causal=True, query_start=32, magnitudes=True)
    np.testing.assert_allclose(r2["out_mag"], 2 * r["out_mag"], rtol=1e-12)


def test_row_normwise_check_rejects_dropped_tiles(oracle):
    """The C4 attention checks (per-row normwise error <= 1e-2 next to the magnitude check) must
    reject a kernel that drops one 64-key tile from P V, or one 32-query tile from dK/dV, on long
    causal rows (S = 2048, D = 128): on a row that sees i keys, a tile holds ~64/i of the row's
    sum of |terms| (what the magnitude check measures against, so it passes such a tile on rows
    of C4's length, i ~ 4096) but ~sqrt(64/i) of the row's norm. The planted mistakes are built
    from the oracle's own outputs on the CPU."""
    S, D = 2048, 128
    q = oracle.bf16_round(oracle.normal((1, 1, S, D), 7, 1))
    k = oracle.bf16_round(oracle.normal((1, 1, S, D), 7, 2))
    v = oracle.bf16_round(oracle.normal((1, 1, S, D), 7, 3))
    dy = oracle.bf16_round(oracle.normal((1, 1, S, D), 7, 4))
    scale = D ** -0.5
    r = oracle.attention_f64(q, k, v, dy, scale=scale, causal=True)
    q2, k2, v2, dy2 = (x[0, 0].astype(np.float64) for x in (q, k, v, dy))
    s = scale * q2 @ k2.T
    s[np.triu_indices(S, 1)] = -np.inf
    p = np.exp(s - r["lse"][0, 0][:, None])
    keys = slice(1024, 1088)
    out_bad = r["out"][0, 0] - p[:, keys] @ v2[keys]
    dp = dy2 @ v2.T
    ds = p * (dp - (p * dp).sum(1, keepdims=True))
    rows = slice(1024, 1056)
    dv_bad = r["dv"][0, 0] - p[rows].T @ dy2[rows]
    dk_bad = r["dk"][0, 0] - scale * ds[rows].T @ q2[rows]
    for name, bad in (("out", out_bad), ("dv", dv_bad), ("dk", dk_bad)):
        want = r[name][0, 0]
        assert oracle.row_err(bad, want) > 1e-2, name             # the per-row check rejects it
        assert oracle.row_err(want, want) == 0.0
        # within rounding of the exact result, the per-row check passes
        assert oracle.row_err(want * (1 + 2.0 ** -9), want) <= 1e-2


def test_row_err_definition(oracle):
    b = np.array([[3.0, 4.0], [0.0, 0.0], [1.0, 0.0]])
    assert oracle.row_err(b, b) == 0.0
    assert abs(oracle.row_err(b + np.array([[0.05, 0.0], [0.0, 0.0], [0.0, 0.0]]), b) - 0.01) < 1e-15
    # an all-zero expected row is measured against the largest row norm (5)
    assert abs(oracle.row_err(b + np.array([[0.0, 0.0], [0.0, 0.1], [0.0, 0.0]]), b) - 0.02) < 1e-15
    assert oracle.row_err(np.array([[np.nan, 0.0]]), np.array([[1.0, 0.0]])) == float("inf")


@pytest.mark.parametrize("causal", [False, True])
def test_rising_score_inputs_drive_the_lagging_rescale(oracle, causal):
    """The GPU tests of the forward's lagging running max (test_gpu_attention_rescale.py) use
    these inputs. Replaying the kernel's rule (64-key tiles in order, waves of 32 queries, a
    rescale when some query's tile max passes its running max + 8 in base 2) shows that after the
    first tile the "jump", "creep" and "extreme" rows are rescaled at least twice -- every such
    row when nothing is masked, nearly every one that sees >= 512 keys when causal -- and that
    the "descending" rows never are (their first tile holds the max)."""
    from attn_cases import PATTERNS, base2_scores, rescale_counts, rising_inputs
    m = n = 1024
    for d in (16, 128):
        q, k, _, _, names = rising_inputs(1, 4, 2, m, n, d, seed=d)
        counts = rescale_counts(base2_scores(q, k, d ** -0.5, causal))[0]  # [H, M]
        seen = np.arange(m) + 1 if causal else np.full(m, n)
        for p in PATTERNS:
            rows = np.array([i for i, nm in enumerate(names) if nm == p and seen[i] >= 512])
            c = counts[:, rows]
            if p == "descending":
                assert np.all(c == 0), (d, p)
            else:
                frac = float(np.mean(c >= 2))
                assert frac >= (1.0 if not causal else 0.9), (d, p, frac)


@pytest.mark.parametrize("bug", ["keep_l", "keep_o", "alpha_inv"])
def test_lagging_softmax_replay_matches_exact_and_catches_rescale_mistakes(oracle, bug):
    """The kernel's tile-by-tile softmax with a lagging max, evaluated in float64, equals the
    exact softmax on the rising-score inputs (so the rule itself changes nothing), and each
    plausible mistake in the rescale (l or O left unscaled, the reciprocal factor) moves O by far
    more than the per-row check's 1e-2 on those inputs: a kernel with such a mistake fails the
    GPU tests, which apply that check."""
    from attn_cases import LOG2E, base2_scores, lagging_softmax_f64, rising_inputs
    m = n = 512
    d = 64
    q, k, v, _, _ = rising_inputs(1, 2, 1, m, n, d, seed=5)
    for causal in (False, True):
        s = base2_scores(q, k, d ** -0.5, causal)[0, 0]
        vv = v[0, 0].astype(np.float64)
        good, lse = lagging_softmax_f64(s, vv)
        ex = np.exp((s - s.max(axis=1, keepdims=True)) / LOG2E)
        exact = (ex @ vv) / ex.sum(axis=1, keepdims=True)
        exact_lse = s.max(axis=1) / LOG2E + np.log(ex.sum(axis=1))
        assert oracle.row_err(good, exact) < 1e-12
        np.testing.assert_allclose(lse, exact_lse, rtol=1e-12, atol=1e-9)
        bad, _ = lagging_softmax_f64(s, vv, bug=bug)
        assert oracle.row_err(bad, exact) > 1e-1, (bug, causal)


# ------------------------------------------------------------------ softmax rows

def _reference_row_inputs(rows, width):
    """The inputs of examples/common_rows_validate.rs:7-9."""
    i = np.arange(rows * width)
    x = ((i % 41).astype(np.float32) / np.float32(7.0) - np.float32(2.0)).reshape(rows, width)
    dy = ((i % 13).astype(np.float32) / np.float32(9.0) - np.float32(0.5)).reshape(rows, width)
    return x.astype(np.float32), dy.astype(np.float32)


def test_softmax_known_answers(oracle):
    x = np.log(np.array([[1.0, 2.0, 3.0], [5.0, 5.0, 5.0]], np.float64)).astype(np.float32)
    y = oracle.softmax_f64(x)
    close(y[0], [1 / 6, 2 / 6, 3 / 6], 1e-7, 1e-7)
    close(y[1], [1 / 3] * 3, 1e-15, 0)
    close(oracle.softmax_f64(np.zeros((2, 7), np.float32)), np.full((2, 7), 1 / 7), 1e-15, 0)
    close(np.exp(oracle.softmax_f64(x, True)), y, 1e-15, 1e-12)


@pytest.mark.parametrize("logarithmic", [False, True])
def test_softmax_invariants(oracle, logarithmic):
    x = oracle.normal((33, 257), seed=1, stream=40, std=3.0)
    y = oracle.softmax_f64(x, logarithmic)
    p = np.exp(y) if logarithmic else y
    close(p.sum(-1), np.ones(33), 1e-12, 0)                       # rows sum to one
    shifted = oracle.softmax_f64(x + np.float32(2.0), logarithmic)  # exact shift in float32 here
    close(shifted, y, 1e-6, 1e-6)


@pytest.mark.parametrize("rows,width", [(1, 32), (3, 96), (7, 256), (2, 33)])
@pytest.mark.parametrize("logarithmic", [False, True])
def test_softmax_vs_autograd_on_reference_inputs(oracle, rows, width, logarithmic):
    x, dy = _reference_row_inputs(rows, width)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    fn = torch.log_softmax if logarithmic else torch.softmax
    yt = fn(xt, dim=-1)
    yt.backward(torch.tensor(dy, dtype=torch.float64))
    y = oracle.softmax_f64(x, logarithmic)
    close(y, yt.detach().numpy(), 1e-12, 1e-12)
    # the backward takes the saved output, rounded to F32 as a device would store it
    dx = oracle.softmax_backward_f64(y.astype(np.float32), dy, logarithmic)
    close(dx, xt.grad.numpy(), 1e-6, 1e-6)


def test_softmax_backward_catches_planted_mistakes(oracle):
    """A sign or a dropped term in the backward breaks the vector-Jacobian identity."""
    x, dy = _reference_row_inputs(3, 96)
    y = oracle.softmax_f64(x).astype(np.float32)
    good = oracle.softmax_backward_f64(y, dy)
    assert abs(good.sum(-1)).max() < 1e-6             # softmax gradients sum to zero per row
    wrong = y.astype(np.float64) * dy                  # dropped "- dot" term
    assert abs(wrong.sum(-1)).max() > 1e-2


# ------------------------------------------------------------------ KV-head repetition

def _repeat_case(group):
    # examples/grouped_attention_tensor.rs:51-53
    batch, kv, n, d = 2, 3, 5, 7
    heads = kv * group
    x = (np.arange(batch * kv * n * d, dtype=np.float32) / 8 - 1).reshape(batch, kv, n, d)
    dy = ((np.arange(batch * heads * n * d) % 11).astype(np.float32) / 8 - 0.25).reshape(batch, heads, n, d)
    return x, dy, heads


@pytest.mark.parametrize("group", [1, 2, 3, 5, 9])
def test_repeat_kv_reference_cases(oracle, group):
    x, dy, heads = _repeat_case(group)
    y = oracle.repeat_kv(x, heads)
    b, kv, n, d = x.shape
    for h in range(heads):   # grouped_attention_tensor.rs:58-60: kv head = h / group
        np.testing.assert_array_equal(y[:, h], x[:, h // group])
    dx = oracle.repeat_kv_backward(dy, kv)
    want = dy.astype(np.float64).reshape(b, kv, group, n, d).sum(axis=2)
    close(dx, want, 5e-4, 5e-4)
    # the backward is the transpose of the repeat: <repeat(x), dy> == <x, backward(dy)>
    lhs = float(np.sum(y.astype(np.float64) * dy))
    rhs = float(np.sum(x.astype(np.float64) * dx))
    assert abs(lhs - rhs) <= 1e-6 * max(1.0, abs(lhs))


def test_repeat_kv_backward_follows_the_pairwise_order(oracle):
    # [1e8, 1, -1e8, 1]: pairwise (1e8+1) + (-1e8+1) == 0 in float32; left to right gives 1
    dy = np.array([1e8, 1.0, -1e8, 1.0], np.float32).reshape(1, 4, 1, 1)
    assert oracle.repeat_kv_backward(dy, 1).item() == 0.0
    # five groups: ((g0+g1) + (g2+g3)) + g4, the odd group carried through two levels
    dy = np.array([1.0, 1e8, -1e8, 1.0, 1.0], np.float32).reshape(1, 5, 1, 1)
    assert oracle.repeat_kv_backward(dy, 1).item() == np.float32(np.float32(1e8) + np.float32(-1e8)) + 1.0
    # a left-to-right sum (1 + 1e8) - 1e8 + 1 + 1 would give 2.0
    assert oracle.repeat_kv_backward(dy, 1).item() == 1.0


def test_repeat_kv_backward_catches_planted_mistakes(oracle):
    x, dy, heads = _repeat_case(3)
    dx = oracle.repeat_kv_backward(dy, 3)
    want = dy.astype(np.float64).reshape(2, 3, 3, 5, 7).sum(axis=2)
    wrong_map = dy.astype(np.float64).reshape(2, 3, 3, 5, 7).transpose(0, 2, 1, 3, 4).sum(axis=2)  # h % kv
    dropped = dy.astype(np.float64).reshape(2, 3, 3, 5, 7)[:, :, :2].sum(axis=2)                  # tail lost
    close(dx, want, 5e-4, 5e-4)
    for bad in (wrong_map, dropped):
        with pytest.raises(AssertionError):
            close(bad, want, 5e-4, 5e-4)


# ------------------------------------------------------------------ SwiGLU gate

def _silu_inputs(n):
    # examples/silu_mul_tensor.rs:25-27
    i = np.arange(n)
    x = ((i % 41).astype(np.float32) * np.float32(0.6) - np.float32(12.0)).astype(np.float32)
    u = ((i % 13).astype(np.float32) * np.float32(0.125) - np.float32(0.5)).astype(np.float32)
    dy = ((i % 7).astype(np.float32) * np.float32(0.25) - np.float32(0.75)).astype(np.float32)
    return x, u, dy


def test_silu_mul_known_answers(oracle):
    g = np.array([0.0, 40.0, -40.0, 1.0], np.float32)
    u = np.array([3.0, 2.0, 5.0, 1.0], np.float32)
    dy = np.array([2.0, 1.0, 1.0, 1.0], np.float32)
    y = oracle.silu_mul_f64(g, u)
    dg, du = oracle.silu_mul_backward_f64(g, u, dy)
    assert y[0] == 0.0 and dg[0] == 2.0 * 3.0 * 0.5 and du[0] == 0.0   # sigmoid(0) = 1/2
    close(y[1:3], [80.0, 0.0], 1e-12, 1e-12)                            # silu(g) -> g, -> 0
    close(dg[1:3], [2.0, 0.0], 1e-12, 1e-12)                            # derivative -> 1, -> 0
    s1 = 1.0 / (1.0 + np.exp(-1.0))
    close([y[3], dg[3], du[3]], [s1, s1 * (1 + (1 - s1)), s1], 1e-15, 1e-15)


@pytest.mark.parametrize("n", [1, 65, 1025])
def test_silu_mul_vs_autograd(oracle, n):
    x, u, dy = _silu_inputs(n)
    g64 = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    u64 = torch.tensor(u, dtype=torch.float64, requires_grad=True)
    y = torch.nn.functional.silu(g64) * u64
    y.backward(torch.tensor(dy, dtype=torch.float64))
    close(oracle.silu_mul_f64(x, u), y.detach().numpy(), 1e-13, 1e-12)
    dg, du = oracle.silu_mul_backward_f64(x, u, dy)
    close(dg, g64.grad.numpy(), 1e-13, 1e-12)
    close(du, u64.grad.numpy(), 1e-13, 1e-12)


def test_silu_mul_backward_catches_planted_mistakes(oracle):
    x, u, dy = _silu_inputs(1025)
    dg, du = oracle.silu_mul_backward_f64(x, u, dy)
    s = 1 / (1 + np.exp(-x.astype(np.float64)))
    wrong_derivative = dy * u * s                 # drops the x s (1 - s) term
    wrong_sign = dy * u * s * (1 - x * (1 - s))
    for bad in (wrong_derivative, wrong_sign):
        with pytest.raises(AssertionError):
            close(bad, dg, 2e-5, 1e-4)
    with pytest.raises(AssertionError):
        close(dy * u, du, 2e-5, 1e-4)             # dup must carry silu(g), not u


# ------------------------------------------------------------------ bias / residual add

from ref_cases import BIAS_SHAPES, bias_inputs, embedding_reference_inputs  # noqa: E402


@pytest.mark.parametrize("shape", BIAS_SHAPES)
def test_bias_add_reference_cases(oracle, shape):
    x, r, b, dy = bias_inputs(shape)
    x64, r64, b64 = (t.astype(np.float64) for t in (x, r, b))
    # every value is a multiple of 1/16, so float32 sums are exact: compare with float64 exactly
    np.testing.assert_array_equal(oracle.bias_add_f32(x, b), x64 + b64)
    np.testing.assert_array_equal(oracle.bias_add_f32(x, b, r), x64 + r64 + b64)
    np.testing.assert_array_equal(oracle.bias_add_f32(x, b, x), 2 * x64 + b64)
    width = shape[-1]
    want = dy.astype(np.float64).reshape(-1, width).sum(0) if dy.size else np.zeros(width)
    np.testing.assert_array_equal(oracle.bias_add_backward(dy), want)


def test_bias_add_order_and_nonfinite(oracle):
    # bias_tensor.rs:60-61: (1e20 + -1e20) + 1 == 1; x + (r + b) would give 0
    one = np.ones(1, np.float32)
    assert oracle.bias_add_f32(1e20 * one, one, -1e20 * one)[0] == 1.0
    # bias_tensor.rs:62-65: -0, NaN and infinities follow IEEE float32 addition
    data = np.array([0.0, -0.0, np.nan, np.inf, -np.inf, 1.0, -1.0], np.float32)
    got = oracle.bias_add_f32(data, np.ones(7, np.float32))
    np.testing.assert_array_equal(got, data + np.float32(1))


def test_column_sum_follows_the_halving_order(oracle):
    # runtime/normalization.rs:95-114 adds row i and row i + floor(r/2) per level; on these
    # columns that order decides the float32 result
    parts = np.array([[1e8], [-1e8], [1.0], [1.0]], np.float32)
    assert oracle.column_sum_pairwise(parts)[0] == 0.0          # (1e8+1) + (-1e8+1) -> 0
    assert np.float32(np.float32(np.float32(1e8) - np.float32(1e8)) + 1) + 1 == 2.0  # left to right
    parts5 = np.array([[1e8], [1.0], [-1e8], [1.0], [0.0]], np.float32)
    assert oracle.column_sum_pairwise(parts5)[0] == 2.0         # (1e8-1e8)+(1+1), then + 0
    seq = np.float32(0)
    for v in parts5[:, 0]:
        seq = np.float32(seq + v)
    assert seq == 1.0                                            # the sequential sum differs


# ------------------------------------------------------------------ embedding

def _torch_embedding(weights, ids, dy, padding_idx, scale):
    w = torch.tensor(weights, dtype=torch.float64, requires_grad=True)
    y = torch.nn.functional.embedding(torch.tensor(ids, dtype=torch.int64), w, padding_idx=padding_idx,
                                      scale_grad_by_freq=scale)
    y.backward(torch.tensor(dy, dtype=torch.float64))
    return y.detach().numpy(), w.grad.numpy()


@pytest.mark.parametrize("padding_idx", [None, 0])
@pytest.mark.parametrize("scale", [False, True])
def test_embedding_vs_torch_reference_cases(oracle, padding_idx, scale):
    weights, ids, upstream = embedding_reference_inputs()
    dy = 2 * upstream  # the example's loss y*dy + y*dy
    want_y, want_dw = _torch_embedding(weights, ids, dy, padding_idx, scale)
    np.testing.assert_array_equal(oracle.embedding(weights, ids), want_y)
    close(oracle.embedding_backward_f64(dy, ids, 7, padding_idx, scale), want_dw, 1e-12, 1e-12)


def test_embedding_random_and_empty(oracle):
    rng = np.random.default_rng(4)
    weights = rng.standard_normal((50, 24)).astype(np.float32)
    ids = rng.integers(0, 50, (6, 40))
    dy = rng.standard_normal((6, 40, 24)).astype(np.float32)
    for padding_idx, scale in [(None, False), (7, True), (ids[0, 0], False)]:
        want_y, want_dw = _torch_embedding(weights, ids, dy, padding_idx, scale)
        np.testing.assert_array_equal(oracle.embedding(weights, ids), want_y)
        close(oracle.embedding_backward_f64(dy, ids, 50, padding_idx, scale), want_dw, 1e-12, 1e-12)
    # embedding_tensor.rs:47-53: no IDs -> zero gradient
    empty = np.zeros((0, 3), np.int32)
    assert oracle.embedding(weights, empty).shape == (0, 3, 24)
    np.testing.assert_array_equal(oracle.embedding_backward_f64(np.zeros((0, 3, 24)), empty, 50), np.zeros((50, 24)))
    with pytest.raises(ValueError):
        oracle.embedding(weights, np.array([50]))


# ------------------------------------------------------------------ NLLLoss / cross entropy

def _ce_case(classes, ignore, weighted):
    # examples/cross_entropy_tensor.rs:19-24
    rows = 5
    x = ((np.arange(rows * classes) % 23).astype(np.float32) / 8 - 1000).reshape(rows, classes)
    labels = np.array([0, 31 % classes, 7 % classes, 0, 2 % classes], np.int64)
    if ignore is not None:
        labels[1] = ignore
    w = (0.5 + (np.arange(classes) % 7) / 4).astype(np.float32) if weighted else np.ones(classes, np.float32)
    return x, labels, w


@pytest.mark.parametrize("classes", [1, 3, 33, 4097])
@pytest.mark.parametrize("reduction", [0, 1, 2])
@pytest.mark.parametrize("ignore", [None, -100])
@pytest.mark.parametrize("weighted", [False, True])
def test_nll_oracle_vs_torch_cross_entropy(oracle, classes, reduction, ignore, weighted):
    x, labels, w = _ce_case(classes, ignore, weighted)
    ii = -1 if ignore is None else ignore
    tx = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    red = ["none", "mean", "sum"][reduction]
    want = torch.nn.functional.cross_entropy(tx, torch.tensor(labels), weight=torch.tensor(w, dtype=torch.float64),
                                             reduction=red, ignore_index=ii)
    logp = torch.log_softmax(tx.detach(), -1).numpy()
    got, total = oracle.nll_loss_f64(logp, labels, w, reduction, ii)
    close(got, np.atleast_1d(want.detach().numpy()), 1e-9, 1e-12)
    close([total], [sum(w[t] for t in labels if t != ii)], 0, 1e-12)
    # backward: the oracle's d/dlogp chained through log-softmax equals torch's d/dlogits
    grad = (1.25 + np.arange(5 if reduction == 0 else 1) / 4)
    (want * torch.tensor(grad)).sum().backward()
    dlogp = oracle.nll_loss_backward_f64(grad, x.shape, labels, w, total, reduction, ii)
    p = np.exp(logp)
    dlogits = dlogp - p * dlogp.sum(-1, keepdims=True)
    close(dlogits, tx.grad.numpy(), 1e-9, 1e-9)


def test_nll_known_answers(oracle):
    # examples/cross_entropy_tensor.rs:55-59: Mean over [-1,-2,-3],[-4,-5,-6], labels [0,2], w [1,2,3]
    got, total = oracle.nll_loss_f64(np.array([[-1.0, -2, -3], [-4, -5, -6]]), [0, 2], [1.0, 2, 3], 1, -1)
    assert got.tolist() == [19 / 4] and total == 4
    # every row ignored: Mean is 0/0
    got, total = oracle.nll_loss_f64(np.zeros((2, 3)), [-100, -100], np.ones(3), 1, -100)
    assert np.isnan(got[0]) and total == 0
