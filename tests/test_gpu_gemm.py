"""GPU parity: BF16 GEMM (all transposes, dense and batched, BF16/F32 out), the Linear backward
and the FP32-storage wrappers, through the C ABI, against the golden vectors and the oracle.

Tolerances: the reference acceptance check (deepgemm_validate.rs:16: 0.05 + 0.01|b|), bit
exactness where the reference's integer-formula inputs make every partial sum exact in F32
(rust-ascend-kernels/src/tests.rs:89-103), and max rel err <= 1e-2 vs the f64 oracle otherwise.
"""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import DEV, close, dev_bf16, dev_f32, f32_close, host, randn_bf16, rel_ok
from rust_ascend_hip import HipRuntime, HkError, Transpose

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("batch", [1, 3])
@pytest.mark.parametrize("ta", [0, 1])
@pytest.mark.parametrize("tb", [0, 1])
@pytest.mark.parametrize("out", [torch.bfloat16, torch.float32])
def test_gemm_deepgemm_validate_cases(golden, batch, ta, tb, out):
    key = f"gemm_dv_b{batch}_{'tn'[ta]}{'tn'[tb]}"
    a, b, want = golden[key + "_a"], golden[key + "_b"], golden[key + "_out"]
    at, bt = dev_bf16(a), dev_bf16(b)
    y = HipRuntime.gemm(at, bt, Transpose(ta), Transpose(tb), out)
    close(host(y), want, 0.05, 0.01, "GEMM")
    # gemm_into reuses the output storage (deepgemm_validate.rs:40-42)
    y.zero_()
    HipRuntime.gemm_into(at, bt, Transpose(ta), Transpose(tb), y)
    close(host(y), want, 0.05, 0.01, "GEMM output reuse")


@pytest.mark.parametrize("shape", ["1x80x96x144", "3x16x32x16"])
@pytest.mark.parametrize("ta", [0, 1])
@pytest.mark.parametrize("tb", [0, 1])
def test_gemm_exact_integer_cases(golden, shape, ta, tb):
    key = f"gemm_vm_{shape}_{'nt'[ta]}{'nt'[tb]}"
    a, b, want = golden[key + "_a"], golden[key + "_b"], golden[key + "_out"]
    at, bt = dev_bf16(a), dev_bf16(b)
    y32 = host(HipRuntime.gemm(at, bt, Transpose(ta), Transpose(tb), torch.float32))
    np.testing.assert_array_equal(y32, want.astype(np.float32))  # every partial sum is exact in F32
    y16 = host(HipRuntime.gemm(at, bt, Transpose(ta), Transpose(tb), torch.bfloat16))
    np.testing.assert_array_equal(y16, oracle.bf16_round(want.astype(np.float32)))


def test_linear_nt_backward_golden(golden):
    x, w, dy = golden["linbwd_x"], golden["linbwd_w"], golden["linbwd_dy"]
    dx, dw = HipRuntime.linear_nt_backward(dev_bf16(x), dev_bf16(w), dev_bf16(dy))
    assert dx.dtype == torch.bfloat16 and dw.dtype == torch.float32
    assert dx.shape == (32, 16) and dw.shape == (48, 16)
    # matrix_runtime.rs:21-22 tolerances (5e-4 + 4e-3|b| BF16, 5e-4|b| F32)
    close(host(dx), golden["linbwd_dx"], 5e-4, 4e-3, "dX")
    close(host(dw), golden["linbwd_dw"], 5e-4, 5e-4, "dW")


SHAPES = [(16, 16, 16), (48, 80, 144), (272, 528, 1040), (1024, 1024, 1024), (512, 1024, 1024), (2048, 4096, 512),
          (4096, 4096, 256)]


@pytest.mark.parametrize("m,n,k", SHAPES)
@pytest.mark.parametrize("ta,tb", [(0, 1), (0, 0), (1, 0), (1, 1)])
def test_gemm_random_vs_oracle(m, n, k, ta, tb):
    if (m * n * k > 1 << 31) and (ta, tb) != (0, 1):
        pytest.skip("large shapes run NT only (the others share the kernel after the transpose)")
    a_t, a = randn_bf16((k, m) if ta else (m, k), seed=m + n + k, std=1 / np.sqrt(k))
    b_t, b = randn_bf16((n, k) if tb else (k, n), seed=m * 3 + k, std=1.0)
    for out in (torch.bfloat16, torch.float32):
        y = host(HipRuntime.gemm(a_t, b_t, Transpose(ta), Transpose(tb), out))
        if m * n * k <= 1 << 28:
            want = oracle.gemm_f64(a, b, ta, tb)
        else:
            rows = np.arange(0, m, 7)[:512]
            cols = np.arange(0, n, 5)[:512]
            r, c = np.meshgrid(rows, cols, indexing="ij")
            want = oracle.gemm_f64_sampled(a, b, ta, tb, r.ravel(), c.ravel())
            y = y[r.ravel(), c.ravel()]
        if out == torch.bfloat16:
            rel_ok(y, want, 1e-2, f"GEMM {m}x{n}x{k} {ta}{tb} bf16")
        else:
            f32_close(y, want, f"GEMM {m}x{n}x{k} {ta}{tb} f32")


TILE_SHAPES = [(1, 4000, 4112, 512), (1, 4096, 4096, 64), (1, 4096, 4096, 128), (1, 4096, 4096, 96),
               (2, 2048, 4096, 320), (1, 4368, 3856, 1216), (1, 4096, 4112, 1040), (1, 4000, 4096, 2032)]
TRANSPOSES = [(0, 1), (0, 0), (1, 0), (1, 1)]


@pytest.mark.parametrize("batch,m,n,k", TILE_SHAPES)
@pytest.mark.parametrize("ta,tb", TRANSPOSES)
def test_gemm_256_tile_paths(batch, m, n, k, ta, tb):
    """Shapes that fill the GPU with 256x256 tiles: ragged M/N edges (rows past the matrix read as
    zero, outputs masked), one and two 64-deep K stages, K not a multiple of 64 (the 32-deep
    kernel), batches; every transpose pair, so the ping-pong kernel's MN-major operand reads
    (A stored [K,M], B stored [K,N]) are covered. Sampled rows/columns include the last ones."""
    if (ta, tb) != (0, 1) and (m, n, k) in ((4096, 4096, 64), (4096, 4096, 96)):
        pytest.skip("one and 1.5 stage cases run NT only")
    a_t, a = randn_bf16((batch, k, m) if ta else (batch, m, k), seed=m + k, std=1 / np.sqrt(k))
    b_t, b = randn_bf16((batch, n, k) if tb else (batch, k, n), seed=n + k, std=1.0)
    a_t, b_t = a_t.squeeze(0), b_t.squeeze(0)
    rows = np.concatenate([np.arange(0, m, 13)[:300], np.arange(m - 40, m)])
    cols = np.concatenate([np.arange(0, n, 11)[:300], np.arange(n - 40, n)])
    r, c = np.meshgrid(rows, cols, indexing="ij")
    for out in (torch.bfloat16, torch.float32):
        y = host(HipRuntime.gemm(a_t, b_t, Transpose(ta), Transpose(tb), out)).reshape(batch, m, n)
        for g in range(batch):
            want = oracle.gemm_f64_sampled(a[g], b[g], ta, tb, r.ravel(), c.ravel())
            got = y[g][r.ravel(), c.ravel()]
            if out == torch.bfloat16:
                rel_ok(got, want, 1e-2, f"GEMM {batch}x{m}x{n}x{k} {ta}{tb} bf16 [{g}]")
            else:
                f32_close(got, want, f"GEMM {batch}x{m}x{n}x{k} {ta}{tb} f32 [{g}]")


@pytest.mark.parametrize("n", [6144, 6128, 4112])
@pytest.mark.parametrize("ta,tb", TRANSPOSES)
def test_gemm_narrow_tiles_equal_square_tiles(n, ta, tb):
    """Grids whose square 256x256 tiles would take a part-empty extra round run 256x192 tiles:
    N = 6144 (384 -> 512 tiles, two full rounds), 6128 and 4112 (partial last tiles). An output
    element's K sum does not depend on the tile it belongs to, so the first 4096 columns are
    bit-identical to the same product with N = 4096 (256 square tiles), in both output types and
    every transpose (an MN-major B is staged 256 columns wide either way); plus the oracle on the
    last columns."""
    m, k = 4096, 320
    a_t, a = randn_bf16((k, m) if ta else (m, k), seed=n + ta, std=1 / np.sqrt(k))
    b_t, b = randn_bf16((n, k) if tb else (k, n), seed=n + 2 * tb + 1, std=1.0)
    b_sq = (b_t[:4096] if tb else b_t[:, :4096]).contiguous()
    for out in (torch.bfloat16, torch.float32):
        y = HipRuntime.gemm(a_t, b_t, Transpose(ta), Transpose(tb), out)
        y_sq = HipRuntime.gemm(a_t, b_sq, Transpose(ta), Transpose(tb), out)
        view = torch.int16 if out == torch.bfloat16 else torch.int32
        assert torch.equal(y[:, :4096].contiguous().view(view), y_sq.view(view)), (n, ta, tb, out)
    rows = np.concatenate([np.arange(0, m, 97), np.arange(m - 8, m)])
    cols = np.arange(n - 300, n)
    r, c = np.meshgrid(rows, cols, indexing="ij")
    want = oracle.gemm_f64_sampled(a, b, ta, tb, r.ravel(), c.ravel())
    rel_ok(host(y)[r.ravel(), c.ravel()], want, 1e-2, f"narrow tiles {m}x{n}x{k} {ta}{tb}")


@pytest.mark.parametrize("batch,k", [(1, 16), (1, 48), (1, 1040), (1, 2032), (1, 4000), (2, 48), (2, 1040)])
@pytest.mark.parametrize("ta,tb", TRANSPOSES)
def test_gemm_partial_last_stage_equals_zero_padded_k(batch, k, ta, tb):
    """K % 64 != 0 on the 256x256-tile kernel: the chunks or k-rows of the partial last stage
    past K read as zero, so the result is bit-identical to the same product with K zero-padded
    to a multiple of 64 (which runs whole stages only). With two batches, the MN-major k-rows
    past K of batch 0 must read as zero, not as batch 1's first k-rows."""
    m, n = 4096, 4352
    k64 = (k + 63) // 64 * 64
    a_t, _ = randn_bf16((batch, k, m) if ta else (batch, m, k), seed=k + 1, std=1 / np.sqrt(k))
    b_t, _ = randn_bf16((batch, n, k) if tb else (batch, k, n), seed=k + 2, std=1.0)
    if ta:
        a_p = torch.zeros((batch, k64, m), dtype=torch.bfloat16, device=DEV)
        a_p[:, :k] = a_t
    else:
        a_p = torch.zeros((batch, m, k64), dtype=torch.bfloat16, device=DEV)
        a_p[:, :, :k] = a_t
    if tb:
        b_p = torch.zeros((batch, n, k64), dtype=torch.bfloat16, device=DEV)
        b_p[:, :, :k] = b_t
    else:
        b_p = torch.zeros((batch, k64, n), dtype=torch.bfloat16, device=DEV)
        b_p[:, :k] = b_t
    if batch == 1:
        a_t, b_t, a_p, b_p = a_t[0], b_t[0], a_p[0], b_p[0]
    for out in (torch.bfloat16, torch.float32):
        got = HipRuntime.gemm(a_t, b_t, Transpose(ta), Transpose(tb), out)
        want = HipRuntime.gemm(a_p, b_p, Transpose(ta), Transpose(tb), out)
        assert torch.equal(got.view(torch.int16) if out == torch.bfloat16 else got.view(torch.int32),
                           want.view(torch.int16) if out == torch.bfloat16 else want.view(torch.int32)), (k, ta, tb, out)


def test_gemm_batched_vs_oracle():
    for ta, tb in [(0, 0), (0, 1), (1, 0), (1, 1)]:
        a_t, a = randn_bf16((5, 96, 64) if ta else (5, 64, 96), seed=1)
        b_t, b = randn_bf16((5, 112, 96) if tb else (5, 96, 112), seed=2)
        y = host(HipRuntime.gemm(a_t, b_t, Transpose(ta), Transpose(tb), torch.float32))
        f32_close(y, oracle.gemm_f64(a, b, ta, tb), f"batched {ta}{tb}")


C3_CASES = [(8192, 8192, 8192, 1), (8192, 8192, 8192, 0), (8192, 14336, 4096, 1), (8192, 4096, 14336, 1),
            (4096, 4096, 4096, 1), (4096, 4096, 4096, 0), (1024, 1024, 1024, 1), (1024, 1024, 1024, 0)]


@pytest.mark.parametrize("m,n,k,tb", C3_CASES)
def test_gemm_c3_full_size_sampled(m, n, k, tb):
    """BASELINE config C3, every shape and layout the sweep times: A, B ~N(0,1)/sqrt(K) BF16, NT
    (Linear weights [N,K]) or NN (B stored [K,N]), BF16 out; sampled parity on 4096 random (i, j)
    plus a full row and a full column (the last)."""
    a_t, a = randn_bf16((m, k), seed=1, std=1 / np.sqrt(k))
    b_t, b = randn_bf16((n, k) if tb else (k, n), seed=2, std=1 / np.sqrt(k))
    y_t = HipRuntime.gemm(a_t, b_t, Transpose.No, Transpose(tb), torch.bfloat16)
    rng = np.random.default_rng(0)
    rows = np.concatenate([rng.integers(0, m, 4096), np.full(n, m // 3), np.arange(m)])
    cols = np.concatenate([rng.integers(0, n, 4096), np.arange(n), np.full(m, n - 1)])
    y = host(y_t[torch.from_numpy(rows).to(DEV), torch.from_numpy(cols).to(DEV)])
    want = oracle.gemm_f64_sampled(a, b, 0, tb, rows, cols)
    rel_ok(y, want, 1e-2, f"C3 {m}x{n}x{k} {'NT' if tb else 'NN'}")


def test_c1_linear_forward():
    """X[512,1024] ~N(0,1), W[1024,1024] ~N(0,0.02), bias zeros, BF16 out."""
    x = oracle.normal((512, 1024), 0, 1)
    w = oracle.normal((1024, 1024), 0, 2, std=0.02)
    y = host(HipRuntime.gemm(dev_bf16(x), dev_bf16(w), Transpose.No, Transpose.Yes, torch.bfloat16))
    rel_ok(y, oracle.gemm_f64(oracle.bf16_round(x), oracle.bf16_round(w), 0, 1), 1e-2, "C1")


@pytest.mark.parametrize("ta", [0, 1])
@pytest.mark.parametrize("tb", [0, 1])
def test_gemm_bf16_fp32_forward_backward(ta, tb):
    m, n, k = 64, 48, 80
    a = oracle.normal((k, m) if ta else (m, k), 5, 1)
    b = oracle.normal((n, k) if tb else (k, n), 5, 2)
    out, ab, bb = HipRuntime.gemm_bf16_fp32(dev_f32(a), dev_f32(b), Transpose(ta), Transpose(tb))
    np.testing.assert_array_equal(host(ab), oracle.bf16_round(a))
    np.testing.assert_array_equal(host(bb), oracle.bf16_round(b))
    ar, br = oracle.bf16_round(a), oracle.bf16_round(b)
    f32_close(host(out), oracle.gemm_f64(ar, br, ta, tb), "fwd")
    dy = oracle.normal((m, n), 5, 3)
    da, db = HipRuntime.gemm_bf16_fp32_backward(ab, bb, dev_f32(dy), Transpose(ta), Transpose(tb))
    assert da.shape == ab.shape and db.shape == bb.shape
    dyr = oracle.bf16_round(dy)
    op_a = ar.T if ta else ar
    op_b = br.T if tb else br
    want_da = dyr.astype(np.float64) @ op_b.T.astype(np.float64)  # d op(A)
    want_db = op_a.T.astype(np.float64) @ dyr.astype(np.float64)  # d op(B)
    f32_close(host(da), want_da.T if ta else want_da, "dA")
    f32_close(host(db), want_db.T if tb else want_db, "dB")


def test_linear_bf16_fp32_matches_gemm():
    x = oracle.normal((32, 64), 6, 1)
    w = oracle.normal((48, 64), 6, 2)
    y, xb, wb = HipRuntime.linear_bf16_fp32(dev_f32(x), dev_f32(w))
    f32_close(host(y), oracle.gemm_f64(oracle.bf16_round(x), oracle.bf16_round(w), 0, 1), "linear")
    dy = oracle.normal((32, 48), 6, 3)
    dx, dw = HipRuntime.linear_bf16_fp32_backward(xb, wb, dev_f32(dy))
    dyr = oracle.bf16_round(dy).astype(np.float64)
    f32_close(host(dx), dyr @ oracle.bf16_round(w), "dX")
    f32_close(host(dw), dyr.T @ oracle.bf16_round(x), "dW")


def test_gemm_rejects_overlap_and_stays_healthy():
    a_t, a = randn_bf16((64, 64), seed=3)
    with pytest.raises(HkError):
        HipRuntime.gemm_into(a_t, a_t, Transpose.No, Transpose.No, a_t)  # in-place output overlaps inputs
    y = host(HipRuntime.gemm(a_t, a_t, Transpose.No, Transpose.No, torch.float32))
    f32_close(y, oracle.gemm_f64(a, a, 0, 0), "after rejection")
