"""CPU tests of the C ABI: the library loads, exports every symbol include/hk.h declares, and
rejects invalid calls before any device work (the reference's host contract tests:
deepgemm/plan.rs:89-109, runtime/normalization.rs:188-221, rotary_programs.rs:277-297,
src/nn/attention.rs:105-133). No compute call is made here."""
import ctypes
import re

import pytest

import rust_ascend_hip as rh
from rust_ascend_hip import _lib
from rust_ascend_hip._lib import BF16, F16, F32, HkError, tensor_desc


def declared_functions():
    text = open(_lib.HEADER_PATH).read()
    return sorted(set(re.findall(r"^\s*(?:hk_status|const char\*|int32_t|void\*)\s+(hk_\w+)\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_functions()
    assert len(names) >= 29
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_lib.SIGNATURES), set(names) ^ set(_lib.SIGNATURES)
    assert lib.hk_abi_version() == 1


def fake(dtype, shape, ptr=1 << 20):
    return ctypes.byref(tensor_desc(ptr, dtype, shape))


def test_ops_without_context_report_not_initialized():
    lib = _lib.load()
    a, b = fake(BF16, (32, 48)), fake(BF16, (48, 64), ptr=1 << 30)
    out = fake(BF16, (32, 64), ptr=1 << 31)
    assert lib.hk_gemm_into(None, a, b, 0, 0, out) == _lib.NOT_INITIALIZED
    assert "not initialized" in _lib.last_error()
    assert lib.hk_sync(None) == _lib.NOT_INITIALIZED


def test_init_without_gpu_is_a_load_error():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    lib = _lib.load()
    h = ctypes.c_void_p()
    assert lib.hk_init(0, ctypes.byref(h)) == _lib.LOAD_ERROR


@pytest.mark.parametrize("ta", [0, 1])
@pytest.mark.parametrize("tb", [0, 1])
def test_four_transposes_share_the_logical_shape(ta, tb):
    # plan.rs:93-99
    a = (48, 32) if ta else (32, 48)
    b = (64, 48) if tb else (48, 64)
    p = rh.gemm_plan(a, b, ta, tb, out_dtype=__import__("torch").float32)
    assert (p["m"], p["n"], p["k"]) == (32, 64, 48)
    assert p["out_shape"] == (32, 64)
    assert p["key"] == f"bf16_dense_{'nt'[ta]}{'nt'[tb]}_f32"


def test_gemm_contract_rejections():
    import torch
    with pytest.raises(HkError):  # batch broadcast, plan.rs:100
        rh.gemm_plan((2, 16, 16), (1, 16, 16), 0, 0)
    for dims in [(0, 16), (17, 16), (16,), (1, 1, 16, 16)]:  # plan.rs:101-104
        with pytest.raises(HkError):
            rh.gemm_plan(dims, (16, 16), 0, 0)
    with pytest.raises(HkError):
        rh.gemm_plan((16, 16), (16, 16), 0, 0, a_dtype=torch.float16)
    with pytest.raises(HkError):  # contraction mismatch
        rh.gemm_plan((32, 48), (32, 64), 0, 0)
    with pytest.raises(HkError):  # batches 1..=4096
        rh.gemm_plan((4097, 16, 16), (4097, 16, 16), 0, 0)
    p = rh.gemm_plan((3, 16, 32), (3, 32, 48), 0, 0)
    assert p["kind"] == "batched" and p["out_shape"] == (3, 16, 48) and p["key"] == "bf16_batched_nn_bf16"
    # training dimension mapping (plan.rs:107): dY[32,64] . W[64,48] -> X shape, dY^T X -> W shape
    assert rh.gemm_plan((32, 64), (64, 48), 0, 0)["out_shape"] == (32, 48)
    assert rh.gemm_plan((32, 64), (32, 48), 1, 0)["out_shape"] == (64, 48)


def test_group_ends_contract():
    # GroupEnds::new, deepgemm/plan.rs:16-26 and its tests :105-106
    rh.check_group_ends([0, 256, 256, 768])
    rh.check_group_ends([256])
    for ends in ([1, 17], [256, 0], [0, 0], [], [-256, 256], [256] * 4097):
        with pytest.raises(HkError):
            rh.check_group_ends(ends)
    # GemmSpec::grouped_nt, plan.rs:61-67,105: A [768,64], W [4,128,64] -> [768,128]
    p = rh.grouped_gemm_plan((768, 64), (4, 128, 64), [0, 256, 256, 768])
    assert p["kind"] == "mgrouped" and p["groups"] == 4 and p["out_shape"] == (768, 128)
    assert (p["m"], p["n"], p["k"]) == (768, 128, 64) and p["key"] == "bf16_mgrouped_nt_bf16"
    import torch
    assert rh.grouped_gemm_plan((512, 48), (3, 64, 48), [256, 256, 512], torch.float32)["key"] == "bf16_mgrouped_nt_f32"
    for a, w, ends in [((768, 64), (3, 128, 64), [0, 256, 256, 768]),   # group count != W's
                       ((512, 64), (4, 128, 64), [0, 256, 256, 768]),   # rows != last end
                       ((768, 64), (4, 128, 48), [0, 256, 256, 768]),   # K mismatch
                       ((768, 64), (128, 64), [768]),                   # W rank
                       ((768, 64), (1, 120, 64), [768])]:               # N % 16
        with pytest.raises(HkError):
            rh.grouped_gemm_plan(a, w, ends)
    with pytest.raises(HkError):
        rh.grouped_gemm_plan((256, 64), (1, 128, 64), [256], a_dtype=torch.float32)
    lib = _lib.load()
    a, w = fake(BF16, (512, 48), 1 << 20), fake(BF16, (3, 64, 48), 1 << 24)
    out = fake(BF16, (512, 64), 1 << 28)
    assert lib.hk_gemm_grouped_nt_into(None, a, w, None, out) == _lib.INVALID_ARGUMENT  # no uploaded ends
    arr = (ctypes.c_int32 * 3)(256, 256, 512)
    assert lib.hk_group_ends_upload(None, arr, 3, ctypes.byref(ctypes.c_void_p())) == _lib.NOT_INITIALIZED
    bad = (ctypes.c_int32 * 2)(256, 128)
    assert lib.hk_group_ends_upload(None, bad, 2, ctypes.byref(ctypes.c_void_p())) == _lib.INVALID_ARGUMENT


def test_padded_gemm_contract():
    # deepgemm/padded.rs:54-80: tails are accepted; contract, batch, dtype and native-domain errors
    # are not disguised by padding. Valid calls reach the (missing) context.
    lib = _lib.load()

    def call(a, b, ta=0, tb=0, adt=F32, bdt=F32):
        ra, rb = len(a), len(b)
        m = a[-1] if ta else a[-2]
        n = b[-2] if tb else b[-1]
        out = a[:-2] + (m, n)
        pad = lambda s: tuple(s[:-2]) + tuple((d + 15) // 16 * 16 for d in s[-2:])
        return lib.hk_gemm_padded_bf16_fp32(None, fake(adt, a, 1 << 20), fake(bdt, b, 1 << 30), ta, tb,
                                            fake(F32, out, 1 << 34), fake(BF16, pad(a), 1 << 36),
                                            fake(BF16, pad(b), 1 << 38))

    for (m, n, k) in [(1, 1, 1), (3, 17, 7), (17, 33, 65), (16, 32, 48)]:
        for ta in (0, 1):
            for tb in (0, 1):
                a = (k, m) if ta else (m, k)
                b = (n, k) if tb else (k, n)
                assert call(a, b, ta, tb) == _lib.NOT_INITIALIZED, (m, n, k, ta, tb)
                assert call((2,) + a, (2,) + b, ta, tb) == _lib.NOT_INITIALIZED
    for a, b, adt in [((3, 7), (8, 17), F32), ((0, 7), (7, 17), F32), ((2, 3, 7), (1, 7, 17), F32),
                      ((3, 7), (7, 17), F16), ((2**31 - 1, 7), (7, 17), F32), ((4097, 3, 7), (4097, 7, 17), F32)]:
        assert call(a, b, adt=adt) == _lib.INVALID_ARGUMENT, (a, b)
    # the trainable form takes F32 inputs only (padded_matrix.rs:42)
    assert call((3, 7), (7, 17), bdt=BF16) == _lib.INVALID_ARGUMENT
    # snapshots must have the native (rounded) shapes
    assert lib.hk_gemm_padded_bf16_fp32(None, fake(F32, (3, 7), 1 << 20), fake(F32, (7, 17), 1 << 30), 0, 0,
                                        fake(F32, (3, 17), 1 << 34), fake(BF16, (3, 7), 1 << 36),
                                        fake(BF16, (16, 32), 1 << 38)) == _lib.INVALID_ARGUMENT
    # frozen form: rank-2 F32 input, BF16 weight; the padded weight may be omitted
    assert lib.hk_linear_frozen_padded_bf16_fp32(None, fake(F32, (3, 35), 1 << 20), fake(BF16, (19, 35), 1 << 30),
                                                 fake(F32, (3, 19), 1 << 34), None) == _lib.NOT_INITIALIZED
    assert lib.hk_linear_frozen_padded_bf16_fp32(None, fake(F32, (3, 35), 1 << 20), fake(F32, (19, 35), 1 << 30),
                                                 fake(F32, (3, 19), 1 << 34), None) == _lib.INVALID_ARGUMENT
    assert lib.hk_linear_frozen_padded_bf16_fp32_backward(None, fake(BF16, (32, 48), 1 << 20),
                                                          fake(F32, (3, 19), 1 << 30),
                                                          fake(F32, (3, 35), 1 << 34)) == _lib.NOT_INITIALIZED
    assert lib.hk_linear_frozen_padded_bf16_fp32_backward(None, fake(BF16, (19, 35), 1 << 20),
                                                          fake(F32, (3, 19), 1 << 30),
                                                          fake(F32, (3, 35), 1 << 34)) == _lib.INVALID_ARGUMENT


def test_nll_loss_contract():
    # tensor/loss.rs:64-99: layouts for every dtype, label width and reduction; invalid labels,
    # weights and upstream layouts are rejected before any device work
    from rust_ascend_hip._lib import I32, I64
    lib = _lib.load()

    def fwd(x, t, w, red, out, tot):
        return lib.hk_nll_loss(None, fake(*x, 1 << 20), fake(*t, 1 << 24), fake(*w, 1 << 26), red, -100,
                               fake(*out, 1 << 28), fake(*tot, 1 << 30))

    for dt in (F32, F16, BF16):
        for it in (I32, I64):
            for rows in (0, 3):
                for red in (0, 1, 2):
                    n_out = rows if red == 0 else 1
                    assert fwd((dt, (rows, 65)), (it, (rows,)), (dt, (65,)), red, (dt, (n_out,)),
                               (dt, (1,))) == _lib.NOT_INITIALIZED, (dt, it, rows, red)
    ok = ((F32, (3, 65)), (I64, (3,)), (F32, (65,)), 1, (F32, (1,)), (F32, (1,)))
    assert fwd(*ok) == _lib.NOT_INITIALIZED
    bad = [((F32, (3, 65)), (F32, (3,)), (F32, (65,))), ((F32, (3, 65)), (I64, (3, 1)), (F32, (65,))),
           ((F32, (3, 65)), (I64, (3,)), (F32, (64,))), ((F32, (3, 65)), (I64, (3,)), (BF16, (65,))),
           ((F32, (3, 0)), (I64, (3,)), (F32, (0,)))]
    for x, t, w in bad:
        assert fwd(x, t, w, 1, (F32, (1,)), (F32, (1,))) == _lib.INVALID_ARGUMENT, (x, t, w)
    assert fwd((F32, (3, 65)), (I64, (3,)), (F32, (65,)), 3, (F32, (1,)), (F32, (1,))) == _lib.INVALID_ARGUMENT
    assert fwd((F32, (3, 65)), (I64, (3,)), (F32, (65,)), 0, (F32, (1,)), (F32, (1,))) == _lib.INVALID_ARGUMENT

    def bwd(g, tot, red=1):
        return lib.hk_nll_loss_backward(None, fake(*g, 1 << 32), fake(F32, (3, 65), 1 << 20), fake(I64, (3,), 1 << 24),
                                        fake(F32, (65,), 1 << 26), fake(*tot, 1 << 30), red, -1,
                                        fake(F32, (3, 65), 1 << 34))
    assert bwd((F32, (1,)), (F32, (1,))) == _lib.NOT_INITIALIZED
    assert bwd((F32, (3,)), (F32, (1,))) == _lib.INVALID_ARGUMENT   # Mean takes a [1] upstream
    assert bwd((F32, (1,)), (BF16, (1,))) == _lib.INVALID_ARGUMENT  # total weight dtype
    assert bwd((F32, (3,)), (F32, (1,)), red=0) == _lib.NOT_INITIALIZED


def test_overlap_and_shape_checks_run_before_the_context():
    lib = _lib.load()
    a = fake(BF16, (32, 48), ptr=1 << 20)
    b = fake(BF16, (48, 64), ptr=1 << 24)
    # output overlapping A
    assert lib.hk_gemm_into(None, a, b, 0, 0, fake(BF16, (32, 64), ptr=(1 << 20) + 64)) == _lib.INVALID_ARGUMENT
    assert "overlap" in _lib.last_error()
    # wrong output layout
    assert lib.hk_gemm_into(None, a, b, 0, 0, fake(BF16, (64, 32), ptr=1 << 28)) == _lib.INVALID_ARGUMENT
    assert lib.hk_gemm_into(None, a, b, 0, 0, fake(F16, (32, 64), ptr=1 << 28)) == _lib.INVALID_ARGUMENT


def test_rms_norm_contract():
    lib = _lib.load()
    x = fake(F32, (3, 96), 1 << 20)
    w = fake(F32, (96,), 1 << 24)
    y = fake(F32, (3, 96), 1 << 26)
    r = fake(F32, (3,), 1 << 28)
    # normalization.rs:200, 217: epsilon must be positive and representable in FP32
    for eps in (0.0, -1.0, float("nan"), float("inf"), 1e300, 1e-100):
        assert lib.hk_rms_norm(None, x, w, eps, y, r) == _lib.INVALID_ARGUMENT, eps
    assert lib.hk_rms_norm(None, x, w, 1e-5, y, r) == _lib.NOT_INITIALIZED
    assert lib.hk_rms_norm(None, x, fake(F32, (95,), 1 << 24), 1e-5, y, r) == _lib.INVALID_ARGUMENT
    assert lib.hk_rms_norm(None, x, w, 1e-5, fake(BF16, (3, 96), 1 << 26), r) == _lib.INVALID_ARGUMENT
    assert lib.hk_rms_norm(None, x, w, 1e-5, y, fake(F32, (4,), 1 << 28)) == _lib.INVALID_ARGUMENT
    assert lib.hk_rms_norm(None, fake(F32, (3, 0), 1 << 20), w, 1e-5, y, r) == _lib.INVALID_ARGUMENT
    assert lib.hk_rms_norm(None, fake(F16, (3, 96), 1 << 20), w, 1e-5, y, r) == _lib.INVALID_ARGUMENT
    # empty batch is valid (normalization.rs:194)
    assert lib.hk_rms_norm(None, fake(F32, (0, 64), 0), fake(F32, (64,), 1 << 24), 1e-5,
                           fake(F32, (0, 64), 0), fake(F32, (0,), 0)) == _lib.NOT_INITIALIZED


def test_rotary_prefix_contract():
    # rotary_programs.rs:277-283: invalid broadcast and widths are rejected
    lib = _lib.load()
    x = fake(F32, (2, 3, 5, 11), 1 << 20)
    y = fake(F32, (2, 3, 5, 11), 1 << 26)

    def call(table, p):
        return lib.hk_rotary_prefix(None, x, fake(F32, table, 1 << 24), fake(F32, table, 1 << 25), p, 0, y)

    assert call((1, 1, 5, 3), 6) == _lib.NOT_INITIALIZED
    for table, p in [((5, 3), 6), ((1, 2, 5, 3), 6), ((1, 1, 5, 6), 6), ((1, 1, 5, 3), 0), ((1, 1, 5, 3), 5),
                     ((1, 1, 5, 6), 12)]:
        assert call(table, p) == _lib.INVALID_ARGUMENT, (table, p)
    # full rotation requires same-row tables and an even width
    assert lib.hk_rotary(None, fake(F32, (3, 6), 1 << 20), fake(F32, (3, 3), 1 << 24), fake(F32, (3, 3), 1 << 25),
                         1, fake(F32, (3, 6), 1 << 26)) == _lib.NOT_INITIALIZED
    assert lib.hk_rotary(None, fake(F32, (3, 7), 1 << 20), fake(F32, (3, 3), 1 << 24), fake(F32, (3, 3), 1 << 25),
                         1, fake(F32, (3, 7), 1 << 26)) == _lib.INVALID_ARGUMENT
    assert lib.hk_rotary(None, fake(F32, (3, 6), 1 << 20), fake(F32, (1, 3), 1 << 24), fake(F32, (1, 3), 1 << 25),
                         1, fake(F32, (3, 6), 1 << 26)) == _lib.INVALID_ARGUMENT


def test_attention_contract():
    # src/nn/attention.rs:120-132: head ratios, batches and lengths
    lib = _lib.load()

    def call(q, k, v, d_out=None, causal=1, scale=0.25):
        o = fake(BF16, q, 1 << 34)
        lse = fake(F32, q[:3], 1 << 35)
        return lib.hk_attention_forward(None, fake(BF16, q, 1 << 20), fake(BF16, k, 1 << 26), fake(BF16, v, 1 << 30),
                                        scale, causal, 0, 0, o, lse)

    for heads, kv in [(1, 1), (6, 6), (6, 3), (6, 1), (15, 3)]:
        assert call((2, heads, 32, 64), (2, kv, 96, 64), (2, kv, 96, 64)) == _lib.NOT_INITIALIZED
    for q, k, v in [((2, 5, 32, 64), (2, 3, 96, 64), (2, 3, 96, 64)), ((2, 6, 32, 64), (2, 3, 96, 64), (2, 2, 96, 64)),
                    ((2, 6, 32, 64), (2, 3, 96, 64), (1, 3, 96, 64)), ((2, 6, 32, 64), (2, 3, 96, 64), (2, 3, 32, 64)),
                    ((4096, 2, 32, 64), (4096, 1, 96, 64), (4096, 1, 96, 64)), ((2, 6, 32, 48), (2, 3, 96, 48), (2, 3, 96, 48))]:
        assert call(q, k, v) == _lib.INVALID_ARGUMENT, (q, k, v)
    assert call((2, 2, 32, 64), (2, 1, 96, 64), (2, 1, 96, 64), scale=float("nan")) == _lib.INVALID_ARGUMENT


def test_attention_oversized_shapes_are_invalid_arguments():
    """The fused kernels address one Q/K/V head with 32-bit byte offsets and launch at most 2^32
    work items per grid dimension: larger shapes are invalid arguments, reported before the
    context is touched (so they can never poison it)."""
    lib = _lib.load()

    def call(q, k):
        o = fake(BF16, q, 1 << 44)
        lse = fake(F32, q[:3], 1 << 45)
        return lib.hk_attention_forward(None, fake(BF16, q, 1 << 20), fake(BF16, k, 1 << 36), fake(BF16, k, 1 << 40),
                                        0.1, 1, 0, 0, o, lse)

    assert call((1, 1, 64, 128), (1, 1, (1 << 23) - 16, 128)) == _lib.NOT_INITIALIZED   # N*D*2 < 2^31
    assert call((1, 1, 64, 128), (1, 1, 1 << 23, 128)) == _lib.INVALID_ARGUMENT        # N*D*2 == 2^31
    assert "too large" in _lib.last_error()
    assert call((1, 1, 1 << 23, 128), (1, 1, 64, 128)) == _lib.INVALID_ARGUMENT        # M*D*2 == 2^31
    # D = 16: one head fits the offsets, but 4096 heads of 2^25 rows exceed 2^32 work items
    assert call((1, 1, 1 << 25, 16), (1, 1, 64, 16)) == _lib.NOT_INITIALIZED
    assert call((1, 4096, 1 << 25, 16), (1, 1, 64, 16)) == _lib.INVALID_ARGUMENT


def test_linear_frozen_contract():
    # matrix.rs:147-172: rank-2 F32 X with a fixed rank-2 BF16 W (aligned to 16), F32 Y; the
    # backward takes matching F32 dY and writes F32 dX in the input's shape
    lib = _lib.load()
    x, w = fake(F32, (32, 48), 1 << 20), fake(BF16, (64, 48), 1 << 24)
    assert lib.hk_linear_frozen_bf16_fp32(None, x, w, fake(F32, (32, 64), 1 << 28)) == _lib.NOT_INITIALIZED
    for xd, wd, yd in [((F32, (32, 48)), (F32, (64, 48)), (F32, (32, 64))),      # F32 weight
                       ((BF16, (32, 48)), (BF16, (64, 48)), (F32, (32, 64))),    # BF16 input
                       ((F32, (32, 40)), (BF16, (64, 40)), (F32, (32, 64))),     # K % 16
                       ((F32, (2, 32, 48)), (BF16, (64, 48)), (F32, (2, 32, 64))),  # rank 3
                       ((F32, (32, 48)), (BF16, (64, 48)), (BF16, (32, 64)))]:   # BF16 output
        assert lib.hk_linear_frozen_bf16_fp32(None, fake(*xd, 1 << 20), fake(*wd, 1 << 24),
                                              fake(*yd, 1 << 28)) == _lib.INVALID_ARGUMENT, (xd, wd, yd)
    assert lib.hk_linear_frozen_bf16_fp32_backward(None, w, fake(F32, (32, 64), 1 << 28),
                                                   fake(F32, (32, 48), 1 << 30)) == _lib.NOT_INITIALIZED
    assert lib.hk_linear_frozen_bf16_fp32_backward(None, w, fake(F32, (32, 60), 1 << 28),
                                                   fake(F32, (32, 48), 1 << 30)) == _lib.INVALID_ARGUMENT
    assert lib.hk_linear_frozen_bf16_fp32_backward(None, w, fake(F32, (32, 64), 1 << 28),
                                                   fake(F32, (32, 32), 1 << 30)) == _lib.INVALID_ARGUMENT
    assert lib.hk_linear_frozen_bf16_fp32_backward(None, w, fake(F32, (32, 64), 1 << 28),
                                                   fake(F32, (32, 48), (1 << 28) + 64)) == _lib.INVALID_ARGUMENT


def test_masked_attention_contract():
    # validate_dimensions / validate_gqa (src/nn/attention.rs:81-133): N % 32, M/D/Dv % 16, batches,
    # u32 scores; masks exactly [B,M,N] (rank 3) or [B,Hq,M,N] (rank 4), F32; Dv may differ from D
    lib = _lib.load()

    def call(q, k, v, mask=None, o=None, dt=F32):
        o = o or q[:-1] + (v[-1],)
        return lib.hk_attention_masked_forward(None, fake(dt, q, 1 << 20), fake(dt, k, 1 << 26), fake(dt, v, 1 << 30),
                                               0.25, None if mask is None else fake(F32, mask, 1 << 34),
                                               fake(F32, o, 1 << 38))

    assert call((2, 32, 16), (2, 8192, 16), (2, 8192, 32)) == _lib.NOT_INITIALIZED        # rank 3, Dv != D
    assert call((2, 6, 32, 16), (2, 3, 96, 16), (2, 3, 96, 48), mask=(2, 6, 32, 96)) == _lib.NOT_INITIALIZED
    assert call((2, 6, 32, 16), (2, 3, 96, 16), (2, 3, 96, 16), dt=BF16) == _lib.NOT_INITIALIZED
    for n in (0, 31, 4097):                                                                # attention.rs:111-113
        assert call((2, 32, 16), (2, n, 16), (2, n, 32)) == _lib.INVALID_ARGUMENT, n
    for q, k, v in [((2, 5, 32, 16), (2, 3, 96, 16), (2, 3, 96, 16)), ((2, 6, 32, 16), (2, 3, 96, 16), (2, 2, 96, 16)),
                    ((2, 6, 32, 16), (2, 3, 96, 16), (1, 3, 96, 16)), ((2, 6, 32, 16), (2, 3, 96, 16), (2, 3, 32, 16)),
                    ((4096, 2, 32, 16), (4096, 1, 96, 16), (4096, 1, 96, 16)), ((2, 6, 32, 24), (2, 3, 96, 24), (2, 3, 96, 24)),
                    ((4096, 65536, 16), (4096, 8192, 16), (4096, 8192, 16))]:              # attention.rs:114,127-130
        assert call(q, k, v) == _lib.INVALID_ARGUMENT, (q, k, v)
    assert call((2, 6, 32, 16), (2, 3, 96, 16), (2, 3, 96, 16), mask=(2, 6, 32, 64)) == _lib.INVALID_ARGUMENT
    assert call((2, 32, 16), (2, 96, 16), (2, 96, 16), mask=(2, 1, 32, 96)) == _lib.INVALID_ARGUMENT
    assert call((2, 32, 16), (2, 96, 16), (2, 96, 16), o=(2, 32, 32)) == _lib.INVALID_ARGUMENT  # O's value width
    # the backward: a mask gradient needs the mask and the mask's shape
    q, k = fake(F32, (1, 2, 16, 16), 1 << 20), fake(F32, (1, 1, 64, 16), 1 << 24)
    grads = [fake(F32, (1, 2, 16, 16), 1 << 28), fake(F32, (1, 1, 64, 16), 1 << 30), fake(F32, (1, 1, 64, 16), 1 << 32)]
    assert lib.hk_attention_masked_backward(None, q, k, k, None, fake(F32, (1, 2, 16, 16), 1 << 26), 0.25, *grads,
                                            fake(F32, (1, 2, 16, 64), 1 << 36)) == _lib.INVALID_ARGUMENT
    assert lib.hk_attention_masked_backward(None, q, k, k, fake(F32, (1, 2, 16, 64), 1 << 34),
                                            fake(F32, (1, 2, 16, 16), 1 << 26), 0.25, *grads,
                                            fake(F32, (1, 2, 16, 64), 1 << 36)) == _lib.NOT_INITIALIZED
    assert lib.hk_attention_masked_backward(None, q, k, k, fake(F32, (1, 2, 16, 64), 1 << 34),
                                            fake(F32, (1, 2, 16, 16), 1 << 26), 0.25, *grads,
                                            fake(F32, (1, 2, 16, 64), (1 << 20) + 1024)) == _lib.INVALID_ARGUMENT  # dMask overlaps Q


def test_integration_extern_blocks_match_the_exports():
    """Every function that the Rust `extern "C"` blocks of the repository's integration guide
    declare is exported by libhk.so, and every exported hk_* function is declared in one of those
    blocks (nm -D on the built library)."""
    import os
    import subprocess
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    text = open(os.path.join(root, "INTEGRATION.md")).read()
    blocks = re.findall(r'extern "C" \{(.*?)\n\}', text, re.S)
    assert blocks, "no extern block found"
    declared = set()
    for b in blocks:
        declared |= set(re.findall(r"pub fn (hk_\w+)\(", b))
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True, check=True)
    exported = {ln.split()[-1] for ln in out.stdout.splitlines() if ln.split() and ln.split()[-1].startswith("hk_")
                and ln.split()[-2] in ("T", "t")}
    assert declared - exported == set(), declared - exported
    assert exported - declared == set(), exported - declared
    assert exported == set(declared_functions())
