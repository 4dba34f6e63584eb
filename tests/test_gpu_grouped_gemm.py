"""GPU parity: M-grouped (mixture-of-experts) NT GEMM through the C ABI
(hk_group_ends_upload + hk_gemm_grouped_nt_into; reference DeepGemm::upload_group_ends /
grouped_nt, rust-ascend-driver/src/tensor/deepgemm/mod.rs:61-78).

Cases: the reference's own grouped inputs (rust-ascend-kernels/src/tests.rs:130-132 with two
empty experts, rust-ascend-driver/examples/deepgemm_validate.rs:45-53), whose partial sums are
exact in F32 so the result is checked bit for bit; random expert layouts on each kernel path
(the 4-wave 256x256 kernel when the grid fills the GPU, the 64/128-tile global->LDS kernel, the
register-staged kernel for K % 32 != 0) against the f64 oracle at max rel err <= 1e-2 (BF16 out)
and the reference's F32 criterion 5e-4 + 5e-4|b| (F32 out).
"""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import DEV, dev_bf16, f32_close, host, randn_bf16, rel_ok
from rust_ascend_hip import HipRuntime, HkError, Transpose

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("case", ["vm", "dv"])
def test_grouped_reference_cases_bit_exact(golden, case):
    a, w, ends = golden[f"grouped_{case}_a"], golden[f"grouped_{case}_w"], golden[f"grouped_{case}_ends"]
    want = golden[f"grouped_{case}_out"]
    groups = HipRuntime.upload_group_ends(ends.tolist())
    try:
        at, wt = dev_bf16(a), dev_bf16(w)
        y32 = HipRuntime.grouped_nt(at, wt, groups, torch.float32)
        np.testing.assert_array_equal(host(y32), want.astype(np.float32))
        y16 = HipRuntime.grouped_nt(at, wt, groups, torch.bfloat16)
        np.testing.assert_array_equal(host(y16), oracle.bf16_round(want.astype(np.float32)))
        # output reuse (grouped_nt_into, mod.rs:74-78)
        y32.fill_(float("nan"))
        HipRuntime.grouped_nt_into(at, wt, groups, y32)
        np.testing.assert_array_equal(host(y32), want.astype(np.float32))
    finally:
        groups.close()


def _check_grouped(m, n, k, ends, seed, sampled):
    g = len(ends)
    a_t, a = randn_bf16((m, k), seed=seed, std=1 / np.sqrt(k))
    w_t, w = randn_bf16((g, n, k), seed=seed + 1, std=1.0)
    groups = HipRuntime.upload_group_ends(ends)
    try:
        for out in (torch.bfloat16, torch.float32):
            y = host(HipRuntime.grouped_nt(a_t, w_t, groups, out))
            if not sampled:
                want, got = oracle.gemm_grouped_nt_f64(a, w, ends), y
            else:  # a band of rows at the start and end of every non-empty group, sampled columns
                want, got, begin = [], [], 0
                cols = np.concatenate([np.arange(0, n, 7)[:256], np.arange(n - 16, n)])
                for e, end in enumerate(ends):
                    if end > begin:
                        rows = np.concatenate([np.arange(begin, min(begin + 8, end)), np.arange(max(end - 8, begin), end)])
                        r, c = np.meshgrid(rows, cols, indexing="ij")
                        want.append(oracle.gemm_f64_sampled(a[begin:end], w[e], 0, 1, r.ravel() - begin, c.ravel()))
                        got.append(y[r.ravel(), c.ravel()])
                    begin = end
                want, got = np.concatenate(want), np.concatenate(got)
            if out == torch.bfloat16:
                rel_ok(got, want, 1e-2, f"grouped {m}x{n}x{k} {ends} bf16")
            else:
                f32_close(got, want, f"grouped {m}x{n}x{k} {ends} f32")
    finally:
        groups.close()


@pytest.mark.parametrize("m,n,k,ends", [
    (2048, 256, 512, [512, 512, 1280, 2048]),      # 64x64 tiles, global->LDS kernel
    (4096, 1024, 256, [0, 1024, 3840, 4096]),      # 128x128 tiles
    (1024, 160, 48, [256, 768, 768, 1024]),        # K % 32 != 0: register-staged kernel, ragged N
])
def test_grouped_small_paths_vs_oracle(m, n, k, ends):
    _check_grouped(m, n, k, ends, seed=m + n + k, sampled=False)


@pytest.mark.parametrize("m,n,k,ends", [
    (8192, 2048, 1024, [1024, 1024, 3072, 3328, 5120, 8192]),   # 256x256 4-wave kernel, empty expert
    (16384, 1792, 4096, [2048 * (i + 1) for i in range(8)]),     # 8 experts, TP-8 Llama FFN width
    (8192, 2048, 1040, [1024, 1024, 3072, 3328, 5120, 8192]),   # K % 64 != 0: partial last K stage
])
def test_grouped_large_paths_vs_oracle_sampled(m, n, k, ends):
    _check_grouped(m, n, k, ends, seed=m + n, sampled=True)


def test_grouped_matches_dense_per_expert():
    """Each expert's rows equal the dense NT GEMM of that row slice with that expert's weights."""
    m, n, k, ends = 4096, 512, 512, [0, 1536, 1536, 4096]
    a_t, _ = randn_bf16((m, k), seed=11, std=1 / np.sqrt(k))
    w_t, _ = randn_bf16((4, n, k), seed=12)
    groups = HipRuntime.upload_group_ends(ends)
    try:
        y = HipRuntime.grouped_nt(a_t, w_t, groups, torch.float32)
    finally:
        groups.close()
    for e, (begin, end) in enumerate([(0, 0), (0, 1536), (1536, 1536), (1536, 4096)]):
        if end > begin:
            d = HipRuntime.gemm(a_t[begin:end].contiguous(), w_t[e].contiguous(), Transpose.No, Transpose.Yes,
                                torch.float32)
            f32_close(host(y[begin:end]), host(d).astype(np.float64), f"expert {e}")


def test_grouped_rejections_leave_the_context_healthy():
    a_t, _ = randn_bf16((512, 64), seed=3)
    w_t, _ = randn_bf16((3, 64, 64), seed=4)
    with pytest.raises(HkError):
        HipRuntime.upload_group_ends([256, 128])            # decreasing
    groups = HipRuntime.upload_group_ends([256, 256, 512])
    try:
        with pytest.raises(HkError):                        # group count != W's leading dim
            HipRuntime.grouped_nt(a_t, w_t[:2].contiguous(), groups)
        with pytest.raises(HkError):                        # output overlapping A
            HipRuntime.grouped_nt_into(a_t, w_t, groups, a_t.view(torch.bfloat16)[:, :64])
        y = host(HipRuntime.grouped_nt(a_t, w_t, groups, torch.float32))
        f32_close(y, oracle.gemm_grouped_nt_f64(host(a_t), host(w_t), [256, 256, 512]), "after rejection")
    finally:
        groups.close()
    with pytest.raises(HkError):
        HipRuntime.grouped_nt(a_t, w_t, groups)              # freed handle
