"""GPU parity of the GEMM device programs (hk_programs.hsaco, launched through
hk_launch_kernel_with_args with the reference's nine arguments; reference DeepGemm,
rust-ascend-driver/src/tensor/deepgemm/mod.rs:18-145, and the program ABI of
rust-ascend-kernels/src/ascend.rs:88-114):

* the reference's own cases (deepgemm_validate.rs:16 tolerance; the integer-formula cases of
  rust-ascend-kernels/src/tests.rs:89-103 and the grouped cases, bit for bit);
* bit-exact equality with libhk.so's GEMM (hk_gemm_into / hk_gemm_grouped_nt_into) on shapes
  where both run the 256x256-tile kernel: the programs are that kernel behind the reference's
  argument structs, with the group-end table read in place of libhk.so's per-block table;
* small and ragged shapes against the f64 oracle;
* operand slices past 32-bit byte offsets (2^30 elements: each program's wide companion), exact on
  integer-valued inputs;
* the launch contract: every argument checked before the launch, the context healthy after.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from gpu_util import DEV, close, dev_bf16, f32_close, host, randn_bf16, rel_ok
from rust_ascend_hip import DeepGemm, HipRuntime, HkError, Transpose, runtime
from rust_ascend_hip._lib import HkEpilogue, HkGm

pytestmark = pytest.mark.gpu

TRANSPOSES = [(0, 1), (0, 0), (1, 0), (1, 1)]


@pytest.fixture(scope="module")
def dg():
    provider = DeepGemm()
    yield provider
    provider.close()


@pytest.mark.parametrize("batch", [1, 3])
@pytest.mark.parametrize("ta,tb", TRANSPOSES)
@pytest.mark.parametrize("out", [torch.bfloat16, torch.float32])
def test_deepgemm_validate_cases(dg, golden, batch, ta, tb, out):
    key = f"gemm_dv_b{batch}_{'tn'[ta]}{'tn'[tb]}"
    a, b, want = golden[key + "_a"], golden[key + "_b"], golden[key + "_out"]
    at, bt = dev_bf16(a), dev_bf16(b)
    y = dg.gemm(at, bt, Transpose(ta), Transpose(tb), out)
    close(host(y), want, 0.05, 0.01, "program GEMM")
    y.zero_()
    dg.gemm_into(at, bt, Transpose(ta), Transpose(tb), y)
    close(host(y), want, 0.05, 0.01, "program GEMM output reuse")


@pytest.mark.parametrize("shape", ["1x80x96x144", "3x16x32x16"])
@pytest.mark.parametrize("ta,tb", TRANSPOSES)
def test_exact_integer_cases(dg, golden, shape, ta, tb):
    key = f"gemm_vm_{shape}_{'nt'[ta]}{'nt'[tb]}"
    a, b, want = golden[key + "_a"], golden[key + "_b"], golden[key + "_out"]
    at, bt = dev_bf16(a), dev_bf16(b)
    np.testing.assert_array_equal(host(dg.gemm(at, bt, Transpose(ta), Transpose(tb), torch.float32)),
                                  want.astype(np.float32))
    np.testing.assert_array_equal(host(dg.gemm(at, bt, Transpose(ta), Transpose(tb), torch.bfloat16)),
                                  oracle.bf16_round(want.astype(np.float32)))


@pytest.mark.parametrize("batch,m,n,k", [(1, 4096, 4096, 256), (1, 4000, 4112, 1040), (2, 2048, 4096, 320)])
@pytest.mark.parametrize("ta,tb", TRANSPOSES)
def test_bit_exact_with_the_library_gemm(dg, batch, m, n, k, ta, tb):
    """Shapes whose grid fills the GPU, where libhk.so also runs the 256x256-tile kernel: whole
    and partial last K stages, ragged M/N edges, batches."""
    a_t, _ = randn_bf16((batch, k, m) if ta else (batch, m, k), seed=m + k + ta, std=1 / np.sqrt(k))
    b_t, _ = randn_bf16((batch, n, k) if tb else (batch, k, n), seed=n + k + tb, std=1.0)
    if batch == 1:
        a_t, b_t = a_t[0], b_t[0]
    for out in (torch.bfloat16, torch.float32):
        want = HipRuntime.gemm(a_t, b_t, Transpose(ta), Transpose(tb), out)
        got = dg.gemm(a_t, b_t, Transpose(ta), Transpose(tb), out)
        assert torch.equal(got.view(torch.int16 if out == torch.bfloat16 else torch.int32),
                           want.view(torch.int16 if out == torch.bfloat16 else torch.int32)), (batch, m, n, k, ta, tb,
                                                                                               out)


@pytest.mark.parametrize("batch,m,n,k", [(1, 16, 16, 16), (1, 48, 80, 144), (1, 272, 528, 1040), (3, 48, 80, 144),
                                         (1, 512, 1024, 1024)])
@pytest.mark.parametrize("ta,tb", TRANSPOSES)
def test_small_and_ragged_shapes_vs_oracle(dg, batch, m, n, k, ta, tb):
    a_t, a = randn_bf16((batch, k, m) if ta else (batch, m, k), seed=m * 7 + k, std=1 / np.sqrt(k))
    b_t, b = randn_bf16((batch, n, k) if tb else (batch, k, n), seed=n * 5 + k, std=1.0)
    if batch == 1:
        a_t, b_t = a_t[0], b_t[0]
    for out in (torch.bfloat16, torch.float32):
        y = host(dg.gemm(a_t, b_t, Transpose(ta), Transpose(tb), out)).reshape(batch, m, n)
        for g in range(batch):
            want = oracle.gemm_f64(a[g], b[g], ta, tb)
            if out == torch.bfloat16:
                rel_ok(y[g], want, 1e-2, f"program {batch}x{m}x{n}x{k} {ta}{tb} bf16")
            else:
                f32_close(y[g], want, f"program {batch}x{m}x{n}x{k} {ta}{tb} f32")


def test_linear_nt_backward_golden(dg, golden):
    x, w, dy = golden["linbwd_x"], golden["linbwd_w"], golden["linbwd_dy"]
    dx, dw = dg.linear_nt_backward(dev_bf16(x), dev_bf16(w), dev_bf16(dy))
    close(host(dx), golden["linbwd_dx"], 5e-4, 4e-3, "dX")
    close(host(dw), golden["linbwd_dw"], 5e-4, 5e-4, "dW")


@pytest.mark.parametrize("case", ["vm", "dv"])
def test_grouped_reference_cases_bit_exact(dg, golden, case):
    a, w, ends = golden[f"grouped_{case}_a"], golden[f"grouped_{case}_w"], golden[f"grouped_{case}_ends"]
    want = golden[f"grouped_{case}_out"]
    groups = dg.upload_group_ends(ends.tolist())
    try:
        at, wt = dev_bf16(a), dev_bf16(w)
        np.testing.assert_array_equal(host(dg.grouped_nt(at, wt, groups, torch.float32)), want.astype(np.float32))
        y16 = dg.grouped_nt(at, wt, groups, torch.bfloat16)
        np.testing.assert_array_equal(host(y16), oracle.bf16_round(want.astype(np.float32)))
        y16.zero_()
        dg.grouped_nt_into(at, wt, groups, y16)
        np.testing.assert_array_equal(host(y16), oracle.bf16_round(want.astype(np.float32)))
    finally:
        groups.close()


@pytest.mark.parametrize("m,n,k,ends", [(4096, 4096, 320, [512, 512, 1536, 4096, 4096]),
                                        (768, 80, 144, [0, 256, 256, 768])])
def test_grouped_with_empty_experts(dg, m, n, k, ends):
    """Repeated ends (empty experts, first and last included): bit-exact with libhk.so's grouped
    GEMM where both run the 256x256 kernel, against the oracle otherwise."""
    g = len(ends)
    a_t, a = randn_bf16((m, k), seed=m + g, std=1 / np.sqrt(k))
    w_t, w = randn_bf16((g, n, k), seed=n + g, std=1.0)
    groups = dg.upload_group_ends(ends)
    try:
        for out in (torch.bfloat16, torch.float32):
            got = dg.grouped_nt(a_t, w_t, groups, out)
            if m * n >= 4096 * 4096:
                want = HipRuntime.grouped_nt(a_t, w_t, groups, out)
                assert torch.equal(got.float(), want.float())
            elif out == torch.bfloat16:
                rel_ok(host(got), oracle.gemm_grouped_nt_f64(a, w, ends), 1e-2, "grouped bf16")
            else:
                f32_close(host(got), oracle.gemm_grouped_nt_f64(a, w, ends), "grouped f32")
    finally:
        groups.close()


# ------------------------------------------------------------------ launch contract

def _argv(a, b, d, m, n, k, ends_ptr=None, groups=0, epilogue=None):
    keep = [a, b, d, ctypes.c_uint32(m), ctypes.c_uint32(n), ctypes.c_uint32(k), ctypes.c_void_p(ends_ptr),
            ctypes.c_uint32(groups), epilogue or HkEpilogue(1.0, 0, 0, 0, n, 0)]
    argv = (ctypes.c_void_p * 9)(*(ctypes.cast(ctypes.byref(x), ctypes.c_void_p) for x in keep))
    return argv, keep


def _launch(fn, argv):
    runtime._call("hk_launch_kernel_with_args", fn, 32, argv)


def _allocation_range(ptr):
    """(base, size) of the device allocation holding ptr, from the HIP runtime torch uses."""
    hip = ctypes.CDLL("libamdhip64.so")
    base, size = ctypes.c_void_p(), ctypes.c_size_t()
    rc = hip.hipMemGetAddressRange(ctypes.byref(base), ctypes.byref(size), ctypes.c_void_p(ptr))
    return rc, base.value or 0, size.value


def test_launch_contract_rejections_keep_the_context_healthy(dg):
    m, n, k = 256, 256, 64
    a_t, a = randn_bf16((m, k), seed=1, std=0.125)
    b_t, b = randn_bf16((n, k), seed=2, std=1.0)
    d_t = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    fn = dg.prepare("bf16_dense_nt_bf16")
    ga, gb, gd = HkGm(a_t.data_ptr(), k, 0), HkGm(b_t.data_ptr(), k, 0), HkGm(d_t.data_ptr(), n, 0)

    def rejected(match, *args, **kw):
        argv, _keep = _argv(*args, **kw)
        with pytest.raises(HkError, match=match):
            _launch(fn, argv)

    rejected("multiples of 16", ga, gb, gd, m, n, 40)
    rejected("epilogue", ga, gb, gd, m, n, k, epilogue=HkEpilogue(2.0, 0, 0, 0, n, 0))
    rejected("epilogue", ga, gb, gd, m, n, k, epilogue=HkEpilogue(1.0, 0, 0, 0, n + 16, 0))
    rejected("packed row-major", HkGm(a_t.data_ptr(), k + 16, 0), gb, gd, m, n, k)
    rejected("packed row-major", ga, gb, HkGm(d_t.data_ptr(), n, m * n), m, n, k)
    rejected("num_groups 0", ga, gb, gd, m, n, k, groups=1)
    rejected("overlaps", ga, gb, HkGm(a_t.data_ptr(), n, 0), m, n, k)
    rejected("16-byte aligned", HkGm(a_t.data_ptr() + 8, k, 0), gb, gd, m, n, k)
    # an operand range that runs past its device allocation (checked once the HIP runtime's own
    # range query is seen to work on this tensor)
    rc, base, size = _allocation_range(a_t.data_ptr())
    assert rc == 0 and base <= a_t.data_ptr() and a_t.data_ptr() + a_t.numel() * 2 <= base + size
    short = torch.empty((16, k), dtype=torch.bfloat16, device=DEV)
    rc, base, size = _allocation_range(short.data_ptr())
    assert rc == 0
    rows = (base + size - short.data_ptr()) // (2 * k) + 16  # rows reaching 16 past the allocation's end
    rows = (rows + 15) // 16 * 16
    assert rows * k * 2 < (1 << 30)
    big_d = torch.empty((rows, n), dtype=torch.bfloat16, device=DEV)
    argv, _keep = _argv(HkGm(short.data_ptr(), k, 0), gb, HkGm(big_d.data_ptr(), n, 0), rows, n, k)
    with pytest.raises(HkError, match="inside one device allocation|overlaps"):
        _launch(fn, argv)
    # an M-grouped program needs uploaded ends
    gfn = dg.prepare("bf16_mgrouped_nt_bf16")
    fake_ends = torch.tensor([256], dtype=torch.int32, device=DEV)
    argv, _keep = _argv(ga, gb, gd, m, n, k, ends_ptr=fake_ends.data_ptr(), groups=1)
    with pytest.raises(HkError, match="grouped_layout"):
        runtime._call("hk_launch_kernel_with_args", gfn, 32, argv)
    # unknown program names
    with pytest.raises(HkError, match="unknown device program"):
        dg.prepare("bf16_mgrouped_tn_bf16")
    # the context still computes
    y = dg.gemm(a_t, b_t, Transpose.No, Transpose.Yes, torch.float32)
    f32_close(host(y), oracle.gemm_f64(a, b, 0, 1), "after rejections")


# ------------------------------------------------------------------ operands past 32-bit offsets

def _small_ints(shape, seed):
    """BF16 integers in [-2, 2]: products and sums of up to 2^22 of them are exact in F32, so every
    summation order gives the same F32 bits and any addressing mistake shows."""
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    return torch.randint(-2, 3, shape, generator=g, device=DEV, dtype=torch.int16).to(torch.bfloat16)


# (ta, tb, m, n, k): an operand slice of 2^30 elements (2 GiB), past the 32-bit offsets of the
# plain programs, so the driver runs each program's wide companion. The reference accepts these
# (M/N/K <= INT32_MAX, plan.rs:72-77): e.g. a 131072-row vocabulary projection with K = 8192.
WIDE_SHAPES = [
    (0, 1, 256, 131072, 8192),  # NT: B [N, K], K-major
    (0, 0, 256, 131072, 8192),  # NN: B stored [K, N], MN-major
    (1, 0, 131072, 256, 8192),  # TN: A stored [K, M], MN-major
    (0, 1, 131072, 272, 8192),  # NT: A [M, K], K-major, ragged N
]


@pytest.mark.parametrize("ta,tb,m,n,k", WIDE_SHAPES)
def test_programs_past_32bit_offsets_are_exact(dg, ta, tb, m, n, k):
    print(f"wide program ta={ta} tb={tb} m={m} n={n} k={k}", flush=True)
    a_t = _small_ints((k, m) if ta else (m, k), seed=m + ta)
    b_t = _small_ints((n, k) if tb else (k, n), seed=n + tb + 1)
    af, bf = a_t.float(), b_t.float()
    want = (af.t() if ta else af) @ (bf.t() if tb else bf)  # exact: |sum| <= 4 K = 2^15
    del af, bf
    got = dg.gemm(a_t, b_t, Transpose(ta), Transpose(tb), torch.float32)
    assert torch.equal(got, want), float((got - want).abs().max())
    del got
    got16 = dg.gemm(a_t, b_t, Transpose(ta), Transpose(tb), torch.bfloat16)
    assert torch.equal(got16, want.to(torch.bfloat16))


def test_programs_reject_shapes_past_the_wide_reach(dg):
    """M*K >= 2^30 with K >= 2^22 (a K-major tile's 256 rows pass 2^31 bytes) is refused before any
    address is looked at; the context still computes."""
    fn = dg.prepare("bf16_dense_nt_bf16")
    m, n, k = 256, 256, 1 << 22
    t = torch.zeros((16, 16), dtype=torch.bfloat16, device=DEV)
    argv, _keep = _argv(HkGm(t.data_ptr(), k, 0), HkGm(t.data_ptr(), k, 0), HkGm(t.data_ptr(), n, 0), m, n, k)
    with pytest.raises(HkError, match="too large for the device programs"):
        _launch(fn, argv)
    a_t, a = randn_bf16((64, 32), seed=5)
    b_t, b = randn_bf16((48, 32), seed=6)
    f32_close(host(dg.gemm(a_t, b_t, Transpose.No, Transpose.Yes, torch.float32)), oracle.gemm_f64(a, b, 0, 1),
              "after the rejection")


def test_module_lifecycle_and_stats():
    before = HipRuntime.stats()["modules_loaded"]
    provider = DeepGemm()
    assert HipRuntime.stats()["modules_loaded"] == before + 1
    f1 = provider.prepare("bf16_dense_nn_f32")
    f2 = provider.prepare("bf16_dense_nn_f32")
    assert f1 is f2 and provider.stats()["modules_loaded"] == 1
    a_t, a = randn_bf16((64, 32), seed=3)
    b_t, b = randn_bf16((32, 48), seed=4)
    f32_close(host(provider.gemm(a_t, b_t, Transpose.No, Transpose.No, torch.float32)), oracle.gemm_f64(a, b, 0, 0),
              "lifecycle")
    assert provider.stats()["launches"] == 1
    provider.close()
    with pytest.raises(HkError, match="closed"):
        provider.gemm(a_t, b_t, Transpose.No, Transpose.No, torch.float32)
    # a stale function handle is rejected, not launched
    argv, _keep = _argv(HkGm(a_t.data_ptr(), 32, 0), HkGm(b_t.data_ptr(), 48, 0), HkGm(a_t.data_ptr(), 48, 0), 64, 48,
                        32)
    with pytest.raises(HkError, match="not a device program"):
        _launch(f1, argv)
