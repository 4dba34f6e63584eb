"""Helpers shared by the GPU parity tests (imported by tests only)."""
import numpy as np
import torch

import oracle

DEV = torch.device("cuda:0") if torch.cuda.is_available() else None


def dev_f32(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(DEV)


def dev_bf16(a) -> torch.Tensor:
    """BF16 device tensor holding the RNE rounding of `a` (exactly the oracle's bf16_round)."""
    bits = oracle.bf16_bits(np.ascontiguousarray(a, dtype=np.float32))
    return torch.from_numpy(bits.view(np.int16)).to(DEV).view(torch.bfloat16)


def host(t: torch.Tensor) -> np.ndarray:
    """float32 numpy copy of a device tensor (BF16 widened exactly)."""
    return t.detach().float().cpu().numpy()


def randn_bf16(shape, seed: int, std: float = 1.0):
    """Seeded BF16 N(0, std^2) tensor generated on the GPU, plus its exact float32 host copy."""
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    t = (torch.randn(shape, generator=g, device=DEV, dtype=torch.float32) * std).to(torch.bfloat16)
    return t, host(t)


def close(actual, expected, atol, rtol, name=""):
    a = np.asarray(actual, dtype=np.float64)
    b = np.asarray(expected, dtype=np.float64)
    assert a.shape == b.shape, (name, a.shape, b.shape)
    ok = np.abs(a - b) <= atol + rtol * np.abs(b)
    ok &= np.isfinite(a) | ~np.isfinite(b)
    if not ok.all():
        i = np.argwhere(~ok)[0]
        raise AssertionError(f"{name}: {int((~ok).sum())} mismatches; first at {tuple(i)}: {a[tuple(i)]} vs {b[tuple(i)]}")


def rel_ok(actual, expected, tol, name="", atol_frac=1e-3):
    e = oracle.rel_err(actual, expected, atol_frac)
    assert e <= tol, f"{name}: max rel err {e:.3e} > {tol}"
    return e


# FP32 weight gradients: the rel err's absolute term is 1e-3*rms(dw), the path's own definition
# of the dγ tolerance (max |a-b| / (|b| + 1e-3 rms(b)) <= 1e-4). The kernels form each term
# x*dy exactly (BF16 significands) and round it once, with rstd, in a fused multiply-add; with the
# product rounded twice (x*rstd, then *dy) the C2 error was 1.04e-4 on this measure, 4.0e-5 now.
DW_ATOL_FRAC = 1e-3


def f32_close(actual, expected, name=""):
    """The reference's F32 GEMM criterion, examples/matrix_runtime.rs:21-22: 5e-4 + 5e-4|b|,
    with the absolute term scaled by rms(b) (the reference's values are O(1))."""
    b = np.asarray(expected, dtype=np.float64)
    rms = float(np.sqrt(np.mean(b * b))) if b.size else 1.0
    close(actual, expected, 5e-4 * rms, 5e-4, name)


def mag_ok(actual, expected, magnitude, tol, name=""):
    """Attention parity: max |a-b| / (sum of |terms|) <= tol. A one-pass fused kernel rounds P
    to BF16 before normalizing while the reference rounds the normalized P, so the two differ
    by up to ~2^-8 of sum_j p_j |v_j| (and likewise for the gradients): measured against the
    output itself that difference is unbounded where the output cancels to ~0."""
    e = oracle.mag_err(actual, expected, magnitude)
    assert e <= tol, f"{name}: max err / magnitude {e:.3e} > {tol}"
    return e


def rows_ok(actual, expected, tol, name=""):
    """Per-row normwise parity: max over rows (last axis) of ||a-b|| / ||b|| <= tol. Unlike
    mag_ok, this is measured against each row's own norm, so an error that is small next to the
    sum of |terms| but not next to the row (a dropped key or query tile) fails."""
    e = oracle.row_err(actual, expected)
    assert e <= tol, f"{name}: max per-row normwise err {e:.3e} > {tol}"
    return e
