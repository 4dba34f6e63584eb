"""GPU parity: RMSNorm forward/backward, RoPE (full and prefix) and F32<->BF16 casts through
the C ABI, against the CPU oracle and the golden vectors.

Tolerances: the reference's own (rms_norm_runtime.rs:20: 5e-4 + 5e-4|b| for F32 I/O;
rotary_tensor.rs:8: 2e-5 + 1e-4|b|), and for BF16 I/O max rel err <= 1e-2 on BF16 outputs and
<= 1e-4 on the F32 weight gradient, rel err = max |a-b| / (|b| + 1e-3 rms(b)).
"""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import DEV, DW_ATOL_FRAC, close, dev_bf16, dev_f32, host, randn_bf16, rel_ok
from rust_ascend_hip import HipRuntime, HkError, RotaryLayout

pytestmark = pytest.mark.gpu

RMS_CASES = ["0x32", "1x32", "3x96", "7x256", "33x4096", "3x7", "2x4100"]


@pytest.mark.parametrize("case", RMS_CASES)
def test_rms_norm_f32_golden(golden, case):
    g = {k[len("rms_" + case) + 1:]: v for k, v in golden.items() if k.startswith("rms_" + case + "_")}
    x = dev_f32(g["x"])
    w = dev_f32(g["w"])
    y, rstd = HipRuntime.rms_norm(x, w, 1e-3)
    dx, dw = HipRuntime.rms_norm_backward(x, w, dev_f32(g["dy"]), rstd)
    assert y.shape == x.shape and rstd.shape == (x.shape[0],) and dw.shape == (x.shape[1],)
    close(host(y), g["y"], 5e-4, 5e-4, "Y")
    close(host(rstd), g["rstd"], 5e-4, 5e-4, "rstd")
    close(host(dx), g["dx"], 5e-4, 5e-4, "dX")
    close(host(dw), g["dw"], 5e-4, 5e-4, "dW")


@pytest.mark.parametrize("rows,width", [(1, 4096), (37, 4096), (300, 1024), (5, 8), (9, 520), (4, 4100), (3, 8224),
                                        (2, 3), (1000, 64)])
def test_rms_norm_bf16_vs_oracle(rows, width):
    x_t, x = randn_bf16((rows, width), seed=rows * 7 + width)
    dy_t, dy = randn_bf16((rows, width), seed=rows * 7 + width + 1)
    w = (1 + oracle.normal((width,), 0, 9, std=0.1)).astype(np.float32)
    y, rstd = HipRuntime.rms_norm(x_t, dev_f32(w), 1e-6)
    dx, dw = HipRuntime.rms_norm_backward(x_t, dev_f32(w), dy_t, rstd)
    y_ref, r_ref = oracle.rms_norm_f64(x, w, 1e-6)
    dx_ref, dw_ref = oracle.rms_norm_backward_f64(x, w, dy, r_ref)
    rel_ok(host(y), y_ref, 1e-2, "Y")
    rel_ok(host(rstd), r_ref, 1e-5, "rstd")
    rel_ok(host(dx), dx_ref, 1e-2, "dX")
    rel_ok(host(dw), dw_ref, 1e-4, "dW", atol_frac=DW_ATOL_FRAC)


# Row-split kernels: W = 8 * chunks is spread over QN waves of 64 lanes x CPL chunks (CPL 2 from
# W = 3072 on, W = 2048 keeps CPL 1 over four waves), G = 16 // QN row groups per workgroup of at
# most 256: the widths below cover QN = 1..16, a partly filled last wave (520, 12296) and full ones;
# the row counts leave row groups idle, walk uneven grid strides and reuse both posting slots.
SPLIT_CASES = [(5, 8), (4099, 512), (1000, 520), (4100, 1024), (1, 2048), (5, 2048), (2050, 2048), (3, 4096),
               (1023, 4096), (4099, 4096), (1300, 3072), (2, 5120), (1290, 5120), (900, 6144), (515, 8192),
               (300, 12296), (260, 16384), (7, 16384)]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("rows,width", SPLIT_CASES)
def test_rms_norm_split_path(dtype, rows, width):
    """Forward (above W = 4096) and backward (every W % 8 == 0 up to 16384) on the row-split
    kernels, against the float64 oracle; the backward bit-identical on a rerun."""
    seed = rows * 3 + width + (7 if dtype == "bf16" else 0)
    if dtype == "bf16":
        x_t, x = randn_bf16((rows, width), seed=seed)
        dy_t, dy = randn_bf16((rows, width), seed=seed + 1)
    else:
        x = oracle.normal((rows, width), 0, seed).astype(np.float32)
        dy = oracle.normal((rows, width), 0, seed + 1).astype(np.float32)
        x_t, dy_t = dev_f32(x), dev_f32(dy)
    w = (1 + oracle.normal((width,), 0, seed + 2, std=0.1)).astype(np.float32)
    w_t = dev_f32(w)
    y, rstd = HipRuntime.rms_norm(x_t, w_t, 1e-6)
    dx, dw = HipRuntime.rms_norm_backward(x_t, w_t, dy_t, rstd)
    dx2, dw2 = HipRuntime.rms_norm_backward(x_t, w_t, dy_t, rstd)
    assert torch.equal(dx, dx2) and torch.equal(dw, dw2), "backward must be deterministic"
    y_ref, r_ref = oracle.rms_norm_f64(x, w, 1e-6)
    rel_ok(host(rstd), r_ref, 1e-5, "rstd")
    # the backward is a function of the rstd it is given (the saved F32 tensor): its oracle takes
    # the same values, so F32 rounding of rstd (up to ~1.2e-4 on this dγ measure at W = 5120 F32)
    # is charged to the forward's rstd check above, not to the backward
    dx_ref, dw_ref = oracle.rms_norm_backward_f64(x, w, dy, host(rstd).astype(np.float64))
    if dtype == "bf16":
        rel_ok(host(y), y_ref, 1e-2, "Y")
        rel_ok(host(dx), dx_ref, 1e-2, "dX")
    else:
        close(host(y), y_ref, 5e-4, 5e-4, "Y")
        close(host(dx), dx_ref, 5e-4, 5e-4, "dX")
    rel_ok(host(dw), dw_ref, 1e-4, "dW", atol_frac=DW_ATOL_FRAC)


def test_rms_norm_c2_full_size_and_determinism():
    """x[16384,4096] bf16 ~N(0,1), w F32 ~1+N(0,0.1), eps 1e-6, dy bf16 ~N(0,1)."""
    x_t, x = randn_bf16((16384, 4096), seed=0)
    dy_t, dy = randn_bf16((16384, 4096), seed=1)
    w = (1 + oracle.normal((4096,), 0, 2, std=0.1)).astype(np.float32)
    w_t = dev_f32(w)
    y, rstd = HipRuntime.rms_norm(x_t, w_t, 1e-6)
    dx, dw = HipRuntime.rms_norm_backward(x_t, w_t, dy_t, rstd)
    dx2, dw2 = HipRuntime.rms_norm_backward(x_t, w_t, dy_t, rstd)
    assert torch.equal(dw, dw2) and torch.equal(dx, dx2), "backward must be deterministic"
    y_ref, r_ref = oracle.rms_norm_f64(x, w, 1e-6)
    dx_ref, dw_ref = oracle.rms_norm_backward_f64(x, w, dy, r_ref)
    rel_ok(host(y), y_ref, 1e-2, "Y")
    rel_ok(host(dx), dx_ref, 1e-2, "dX")
    rel_ok(host(dw), dw_ref, 1e-4, "dW", atol_frac=DW_ATOL_FRAC)
    # and the strict relative error over the components with |b| >= 1e-2 rms(b)
    big = np.abs(dw_ref) >= 1e-2 * np.sqrt(np.mean(dw_ref ** 2))
    strict = float(np.max(np.abs(host(dw)[big] - dw_ref[big]) / np.abs(dw_ref[big])))
    assert strict <= 1e-4, f"dW strict relative error {strict:.3e}"


@pytest.mark.parametrize("dtype,rows,width,offset", [
    (torch.bfloat16, 16384, 4096, 0),   # C2: the row-split kernel, two chunks per lane
    (torch.bfloat16, 37, 1000, 0),      # split kernel, partial lanes
    (torch.float32, 300, 4096, 0),      # F32 storage (the add is exact: no rounding in between)
    (torch.bfloat16, 64, 4100, 0),      # width not a multiple of 8: the general kernels
    (torch.bfloat16, 64, 512, 1),       # misaligned views: the general kernels
])
def test_rms_norm_backward_residual_bit_exact_with_backward_and_add(dtype, rows, width, offset):
    """hk_rms_norm_backward_residual = hk_rms_norm_backward then hk_bias_add(dx, no bias, residual),
    bit for bit, and the same dW."""
    g = torch.Generator(device=DEV)
    g.manual_seed(rows + width)

    def rand(shape, std=1.0):
        t = (torch.randn((shape[0] * shape[1] + offset,), generator=g, device=DEV) * std).to(dtype)
        return t[offset:].view(shape)

    x, dy, res = rand((rows, width)), rand((rows, width)), rand((rows, width), 0.5)
    w = (1 + 0.1 * torch.randn((width,), generator=g, device=DEV)).float()
    _, rstd = HipRuntime.rms_norm(x, w, 1e-6)
    print(f"rms backward residual {dtype} {rows}x{width} offset {offset}", flush=True)
    dx, dw = HipRuntime.rms_norm_backward_residual(x, w, dy, rstd, res)
    dx0, dw0 = HipRuntime.rms_norm_backward(x, w, dy, rstd)
    want = HipRuntime.bias_add(dx0, None, res)
    assert torch.equal(dx, want)
    assert torch.equal(dw, dw0)


def test_rms_norm_backward_residual_rejects_bad_residual():
    x, _ = randn_bf16((8, 64), seed=1)
    dy, _ = randn_bf16((8, 64), seed=2)
    w = torch.ones(64, device=DEV)
    _, rstd = HipRuntime.rms_norm(x, w, 1e-6)
    with pytest.raises(HkError, match="residual"):
        HipRuntime.rms_norm_backward_residual(x, w, dy, rstd, torch.zeros((8, 64), device=DEV))  # F32
    with pytest.raises(HkError, match="residual"):
        HipRuntime.rms_norm_backward_residual(x, w, dy, rstd, torch.zeros((8, 32), device=DEV, dtype=torch.bfloat16))
    dx, _ = HipRuntime.rms_norm_backward_residual(x, w, dy, rstd, torch.zeros_like(x))  # still healthy
    assert torch.equal(dx, HipRuntime.rms_norm_backward(x, w, dy, rstd)[0])


def test_rms_norm_empty_batch_and_known_answer(golden):
    w = dev_f32(np.ones(32, np.float32))
    x = torch.empty((0, 32), device=DEV)
    y, rstd = HipRuntime.rms_norm(x, w, 1e-5)
    dx, dw = HipRuntime.rms_norm_backward(x, w, x.clone(), rstd)
    assert y.shape == (0, 32) and torch.count_nonzero(dw) == 0
    # row_tests.rs:280-287: x = 2, dy = 3, rstd = [.5,.25,2] -> per-row contributions 3, 1.5, 12
    for r, want in zip(golden["rmskat_rstd"], golden["rmskat_contrib"]):
        xt = torch.full((1, 32), 2.0, device=DEV)
        _, dw = HipRuntime.rms_norm_backward(xt, w, torch.full((1, 32), 3.0, device=DEV),
                                             torch.tensor([r], device=DEV, dtype=torch.float32))
        assert torch.all(dw == float(want))


def test_rms_norm_misaligned_view_uses_general_path():
    base_t, base = randn_bf16((1, 4096 + 4), seed=5)
    x_t = base_t[0, 4:].reshape(16, 256)  # 8-byte offset: not 16-byte aligned
    assert x_t.data_ptr() % 16 != 0
    w = np.ones(256, np.float32)
    y, rstd = HipRuntime.rms_norm(x_t, dev_f32(w), 1e-6)
    y_ref, _ = oracle.rms_norm_f64(base[0, 4:].reshape(16, 256), w, 1e-6)
    rel_ok(host(y), y_ref, 1e-2, "Y")


def test_rms_norm_split_exchange_timeout_is_reported(monkeypatch):
    """The row-split kernels' waits for their partners' posts are bounded; a wait that runs out
    makes a synchronous call fail with HK_COMPLETION_ERROR (its results are invalid) instead of
    returning stale sums silently. Forced from the host: HK_ROW_SPIN_LIMIT=1 lets every wait poll
    once, so at width 16384 (16 waves per row) some wave reads a post its partner has not written
    yet; every wait still ends. The context stays usable and the next call is exact again."""
    rows, width = 4096, 16384
    x_t, x = randn_bf16((rows, width), seed=91)
    dy_t, dy = randn_bf16((rows, width), seed=92)
    w = (1 + 0.1 * oracle.normal((width,), 91, 2)).astype(np.float32)
    w_t = dev_f32(w)
    y0, rstd0 = HipRuntime.rms_norm(x_t, w_t, 1e-6)
    dx0, dw0 = HipRuntime.rms_norm_backward(x_t, w_t, dy_t, rstd0)
    monkeypatch.setenv("HK_ROW_SPIN_LIMIT", "1")
    print("rms_norm split exchange with a one-poll wait bound", flush=True)
    with pytest.raises(HkError, match="exchange wait ran out"):
        HipRuntime.rms_norm_backward(x_t, w_t, dy_t, rstd0)
    with pytest.raises(HkError, match="exchange wait ran out"):
        HipRuntime.rms_norm(x_t, w_t, 1e-6)
    monkeypatch.delenv("HK_ROW_SPIN_LIMIT")
    y1, rstd1 = HipRuntime.rms_norm(x_t, w_t, 1e-6)
    dx1, dw1 = HipRuntime.rms_norm_backward(x_t, w_t, dy_t, rstd1)
    for a, b in ((y0, y1), (rstd0, rstd1), (dx0, dx1), (dw0, dw1)):
        assert torch.equal(a, b)
    y_ref, r_ref = oracle.rms_norm_f64(x[:64], w, 1e-6)
    rel_ok(host(y1[:64]), y_ref, 1e-2, "Y")


@pytest.mark.parametrize("case", ["0x6", "1x2", "3x6", "2x96"])
@pytest.mark.parametrize("layout", [0, 1])
def test_rotary_f32_golden(golden, case, layout):
    key = f"rope_{case}_l{layout}"
    x, dy, c, s = (golden[key + s_] for s_ in ("_x", "_dy", "_cos", "_sin"))
    y = HipRuntime.rotary(dev_f32(x), dev_f32(c), dev_f32(s), RotaryLayout(layout))
    dx = HipRuntime.rotary_backward(dev_f32(dy), dev_f32(c), dev_f32(s), RotaryLayout(layout))
    close(host(y), golden[key + "_y"], 2e-5, 1e-4, "rotary Y")
    close(host(dx), golden[key + "_dx"], 2e-5, 1e-4, "rotary dX")


@pytest.mark.parametrize("ci", range(5))
@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("backward", [0, 1])
def test_rotary_prefix_golden_tail_bits(golden, ci, layout, backward):
    key = f"ropepre_{ci}_l{layout}_b{backward}"
    x, c, s, want = golden[key + "_x"], golden[key + "_cos"], golden[key + "_sin"], golden[key + "_y"]
    fn = HipRuntime.rotary_prefix_backward if backward else HipRuntime.rotary_prefix
    y = host(fn(dev_f32(x), dev_f32(c), dev_f32(s), 6, RotaryLayout(layout)))
    head = (slice(None),) * (x.ndim - 1) + (slice(0, 6),)
    tail = (slice(None),) * (x.ndim - 1) + (slice(6, None),)
    close(y[head], want[head], 3e-6, 3e-6, "prefix head")
    np.testing.assert_array_equal(y[tail].view(np.uint32), x[tail].view(np.uint32))


@pytest.mark.parametrize("layout", [0, 1])
def test_rotary_c4_shape_bf16(layout):
    """C4's RoPE: Q [4,32,4096,128] and K [4,8,4096,128] BF16 with [1,1,4096,64] tables, theta 5e5."""
    cos, sin = oracle.rope_tables(np.arange(4096), 128, 5e5)
    c_t, s_t = dev_f32(cos[None, None]), dev_f32(sin[None, None])
    for shape, seed in (((4, 32, 4096, 128), 11), ((4, 8, 4096, 128), 12)):
        x_t, x = randn_bf16(shape, seed)
        y = HipRuntime.rotary_prefix(x_t, c_t, s_t, 128, RotaryLayout(layout))
        want = oracle.rotary_prefix(x, cos[None, None], sin[None, None], 128, layout)
        rel_ok(host(y), want, 1e-2, f"rope {shape}")
        # transpose Jacobian on the BF16 result, F32 in and out
        yf = y.float().contiguous()
        back = HipRuntime.rotary_prefix_backward(yf, c_t, s_t, 128, RotaryLayout(layout))
        want_back = oracle.rotary_prefix(host(yf), cos[None, None], sin[None, None], 128, layout, True)
        close(host(back), want_back, 1e-6, 1e-6, "rope backward f32")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("shape,p", [((3, 5, 100, 128), 128), ((2, 3, 64), 48), ((1, 7, 9, 80), 64), ((4, 1, 33, 16), 16)])
def test_rotary_prefix_broadcast_tables_match_per_row_tables(dtype, layout, shape, p):
    """Tables [1, ..., 1, S, P/2] broadcast over the leading axes give exactly the bits of the same
    tables expanded to the input's leading shape (every row its own table row), forward and
    backward, tail columns included; and agree with the oracle."""
    S, half = shape[-2], p // 2
    g = torch.Generator(device=DEV)
    g.manual_seed(sum(shape) + p)
    x = torch.randn(shape, generator=g, device=DEV).to(dtype)
    ang = torch.rand((S, half), generator=g, device=DEV) * 6.0
    lead = (1,) * (len(shape) - 2)
    c, s = torch.cos(ang).reshape(lead + (S, half)), torch.sin(ang).reshape(lead + (S, half))
    full = shape[:-1] + (half,)
    c_full, s_full = c.expand(full).contiguous(), s.expand(full).contiguous()
    print(f"rope broadcast tables {shape} p {p} layout {layout} {dtype}", flush=True)
    for fn in (HipRuntime.rotary_prefix, HipRuntime.rotary_prefix_backward):
        got = fn(x, c, s, p, RotaryLayout(layout))
        want = fn(x, c_full, s_full, p, RotaryLayout(layout))
        assert torch.equal(got.view(torch.int16 if dtype == torch.bfloat16 else torch.int32),
                           want.view(torch.int16 if dtype == torch.bfloat16 else torch.int32))
    want64 = oracle.rotary_prefix(host(x).astype(np.float64), host(c), host(s), p, layout)
    close(host(HipRuntime.rotary_prefix(x, c, s, p, RotaryLayout(layout))), want64,
          1e-2 if dtype == torch.bfloat16 else 1e-5, 1e-2 if dtype == torch.bfloat16 else 1e-5, "rope broadcast")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("shape,tshape", [((3, 4, 10, 64), (3, 1, 10, 32)), ((2, 6, 5, 7, 32), (1, 6, 1, 7, 16)),
                                          ((5, 3, 128), (5, 1, 64)), ((6, 16, 256), (1, 16, 128)),
                                          ((3, 4, 10, 64), (1, 4, 10, 32)), ((2, 1, 5, 1, 9, 64), (1, 1, 5, 1, 9, 32)),
                                          ((4, 3, 1, 48), (4, 3, 1, 24))])
def test_rotary_general_table_maps_match_per_row_tables(dtype, layout, shape, tshape):
    """Tables broadcast over axes that do not leave a contiguous innermost run (the first three
    shapes: a middle or inner axis, so the table row is not the input row modulo a period and the
    kernel walks the leading axes per row) give exactly the bits of the same tables expanded per
    row, forward and backward. The other shapes are period patterns (the table row is the input row modulo the
    table's row count): at 16 threads per row, over two leading axes (period 40), with singleton
    axes inside the pattern, and a same-shape table at 3 threads per row (the general kernel)."""
    half = tshape[-1]
    g = torch.Generator(device=DEV)
    g.manual_seed(sum(shape) + half)
    x = torch.randn(shape, generator=g, device=DEV).to(dtype)
    c = torch.cos(torch.rand(tshape, generator=g, device=DEV) * 6.0)
    s = torch.sin(torch.rand(tshape, generator=g, device=DEV) * 6.0)
    full = shape[:-1] + (half,)
    c_full, s_full = c.expand(full).contiguous(), s.expand(full).contiguous()
    print(f"rope general table map {shape} tables {tshape} layout {layout} {dtype}", flush=True)
    bits = torch.int16 if dtype == torch.bfloat16 else torch.int32
    for fn in (HipRuntime.rotary_prefix, HipRuntime.rotary_prefix_backward):
        got = fn(x, c, s, 2 * half, RotaryLayout(layout))
        want = fn(x, c_full, s_full, 2 * half, RotaryLayout(layout))
        assert torch.equal(got.view(bits), want.view(bits))
    want64 = oracle.rotary_prefix(host(x).astype(np.float64), host(c_full), host(s_full), 2 * half, layout)
    close(host(HipRuntime.rotary_prefix(x, c, s, 2 * half, RotaryLayout(layout))), want64,
          1e-2 if dtype == torch.bfloat16 else 1e-5, 1e-2 if dtype == torch.bfloat16 else 1e-5, "rope general map")


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("width", [2, 6, 64, 96, 128])
def test_rotary_random_widths_vs_oracle(layout, width):
    rows = 37
    x = oracle.normal((rows, width), 3, width)
    ang = oracle.normal((rows, width // 2), 4, width)
    c, s = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    for bw in (False, True):
        fn = HipRuntime.rotary_backward if bw else HipRuntime.rotary
        y = host(fn(dev_f32(x), dev_f32(c), dev_f32(s), RotaryLayout(layout)))
        close(y, oracle.rotary(x, c, s, layout, bw), 1e-6, 1e-6, "rotary f32")
        yb = host(fn(dev_bf16(x), dev_f32(c), dev_f32(s), RotaryLayout(layout)))
        rel_ok(yb, oracle.rotary(oracle.bf16_round(x), c, s, layout, bw), 1e-2, "rotary bf16")


def test_cast_round_trip_bits():
    specials = np.array([0x80000000, 0x7FC01234, 0x7F800000, 0xFF800000, 0x00000001, 0x3F808000, 0x3F818000,
                         0x7F7FFFFF], dtype=np.uint32).view(np.float32)
    x = np.concatenate([specials, oracle.normal((100003,), 1, 1, std=50.0)]).astype(np.float32)
    b = HipRuntime.cast(dev_f32(x), torch.bfloat16)
    got = b.cpu().view(torch.int16).numpy().view(np.uint16)
    want = oracle.bf16_bits(x)
    finite = np.isfinite(x)
    np.testing.assert_array_equal(got[finite], want[finite])
    assert np.all(np.isnan(host(b)[np.isnan(x)]))
    assert np.array_equal(np.isinf(host(b)), np.isinf(oracle.bf16_round(x)))
    back = HipRuntime.cast(b, torch.float32)
    np.testing.assert_array_equal(host(back)[finite], oracle.bf16_round(x)[finite])


def test_invalid_call_raises_and_does_not_poison():
    x = dev_f32(np.ones((4, 32), np.float32))
    with pytest.raises(HkError):
        HipRuntime.rms_norm(x, dev_f32(np.ones(31, np.float32)), 1e-5)
    y, _ = HipRuntime.rms_norm(x, dev_f32(np.ones(32, np.float32)), 1e-5)
    assert torch.allclose(y, torch.ones_like(y), atol=1e-4)
    s = HipRuntime.stats()
    # modules_loaded: the library's own code plus every device-program code object loaded so far
    assert s["launches"] > 0 and s["synchronizations"] > 0 and s["modules_loaded"] >= 1
