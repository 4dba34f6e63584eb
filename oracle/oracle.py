"""CPU oracle for the BF16 transformer kernel path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
may import this module, and only as the checker or as the timed CPU baseline. The
product path (``libhk.so`` and the ``rust_ascend_hip`` package) never imports it.

This is a numpy/ctypes front end over ``hk_oracle.c`` (a C restatement of the
reference's host loops; every C function cites the reference file:line it follows),
plus the BF16 helpers and the counter-based input generator that tests and bench
share.

How each oracle function is pinned (tests/test_oracle.py), so that a dropped term,
a wrong sign or index, or a transposed operand fails at least one check:

* ``bf16_round``: bit patterns of hand-picked values (ties to even, Inf/NaN, -0,
  overflow to Inf) and agreement with torch's float32->bfloat16 conversion.
* ``gemm_grouped_nt_f64``: per-group numpy float64 matmul of the row slices on the reference's
  grouped cases (rust-ascend-kernels/src/tests.rs:89-103,130-132: 768x16x144 with ends
  [0,256,256,768], two empty experts; deepgemm_validate.rs:45-53: 512x64x48 with ends
  [256,256,512]), plus the identity with one group == the dense NT product.
* ``gemm_f64``/``gemm_f32``: numpy float64 matmul for all four transposes and
  batches; the reference's integer-formula cases of
  rust-ascend-kernels/src/tests.rs:89-103,124-129 (80x96x144 dense, 3x16x32x16
  batched, exact BF16 inputs), examples/matrix_runtime.rs:50-77 and
  rust-ascend-driver/examples/deepgemm_validate.rs:30-56, which are exact or
  near-exact in f64; the linear-gradient finite-difference identity of
  tools/ascend/tests/test_adapter.py:89-93.
* ``matmul_shape``/``tensor_matmul_f64``/``tensor_matmul_backward_f64``: the reference's own
  shape cases (generic_matrix.rs:59-101, tensor/tests.rs:56-69 for rank >= 2: broadcast
  [2,1,3,5] @ [1,4,5,7] -> [2,4,3,7], empty and zero-K outputs, contraction, broadcast and rank
  errors), numpy's float64 matmul (an independent implementation of the same broadcasting) and
  torch float64 autograd of torch.matmul for the gradients, on broadcast cases of rank 2 to 6.
* ``module_attention_f64``: parity unpinned against the RUDA library itself (not vendored); its
  formula is checked against torch float64 ``scaled_dot_product_attention`` with the bias and the
  boolean mask folded into a float mask (an independent implementation) and torch float64
  autograd of the explicit composition (softcap included), the orthogonal-Q/K closed form of
  examples/attention_tensor.rs:22-66 (uniform probabilities) and the causal running means of
  examples/causal_attention_tensor.rs:31-55.
* ``rms_norm_f64``/``rms_norm_backward_f64``: torch float64 autograd of
  x*rsqrt(mean(x^2)+eps)*w (the independent reference of
  tools/ascend/tests/test_row_reference.py:65-78); the weight-contribution known
  answer x=2, dy=3, rstd=[.5,.25,2] -> [3,1.5,12] (row_tests.rs:280-287); the
  six-element vectors of examples/gradients.rs:20-37.
* ``rms_norm_lanes_f32``/``rms_norm_backward_lanes_f32``: against the f64 oracle
  (1e-5) and the constant-row invariant of test_row_reference.py:81-83.
* ``rotary``/``rotary_f64``/``rotary_prefix``: torch float64 autograd (the backward
  must be the forward's vector-Jacobian product), pair-norm preservation,
  angle-zero identity, the prefix tail bit patterns (NaN/Inf/-0) of
  rotary_programs.rs:224-260, and prefix-with-full-width == full rotation
  (rotary_programs.rs:262-275).
* ``softmax_f64``/``softmax_backward_f64``: known answers (x = ln[1,2,3] -> [1,2,3]/6,
  a constant row -> 1/W), rows summing to one / log-sum-exp of zero, invariance to a
  per-row shift, and torch float64 autograd (the backward must be the forward's
  vector-Jacobian product) on the reference's own inputs and shapes
  (examples/common_rows_validate.rs:7-9,100).
* ``nll_loss_f64``/``nll_loss_backward_f64``: torch float64 ``nll_loss`` and ``cross_entropy`` (an
  independent implementation of the same semantics, with autograd for the backward) for all three
  reductions, with and without class weights and an ignore label, on the reference's inputs of
  examples/cross_entropy_tensor.rs:19-24; the direct known answer of :55-59 (19/4); a Mean over
  only ignored rows is 0/0 = NaN.
* ``silu_mul_f64``/``silu_mul_backward_f64``: torch float64 autograd of
  torch.nn.functional.silu(g) * u (an independent implementation; the backward must be its
  vector-Jacobian product), known answers at g = 0 (y = 0, dgate = dy*u/2, dup = 0) and for
  large |g| (silu(g) -> g or 0), on the reference's own inputs of examples/silu_mul_tensor.rs:25-27.
* ``bias_add_f32``/``bias_add_backward`` (and ``column_sum_pairwise``): the reference's own
  cases of examples/bias_tensor.rs (integer-formula inputs on seven shapes, exact results; the
  ordered case (1e20 + -1e20) + 1 == 1, which x + (r + b) gets wrong; -0, NaN and infinities), the
  exact integer column sum, and inputs on which the pairwise halving order decides the float32
  result ([1e8, -1e8, 1, 1] sums to 0 pairwise, to 2 left to right or in adjacent pairs).
* ``embedding``/``embedding_backward_f64``: torch float64 autograd of
  torch.nn.functional.embedding with the same padding_idx and scale_grad_by_freq (an independent
  implementation of these semantics) on the reference's inputs of
  examples/embedding_tensor.rs:20-24 (V = 7, H = 65, repeated IDs) for all four option pairs and on
  random cases; the empty-ID gradient is zero (embedding_tensor.rs:47-53).
* ``repeat_kv``/``repeat_kv_backward``: the backward is the repeat's transpose (inner products
  <repeat(x), dy> == <x, backward(dy)> in float64), equals the float64 group sum within
  rounding, and follows the pairwise level order exactly on inputs where the order decides the
  float32 result ([1e8, 1, -1e8, 1] sums to 0 pairwise, to 1 left to right).
* ``attention_f64``: the closed forms of examples/attention_tensor.rs:22-66
  (orthogonal Q/K -> uniform probabilities) and
  examples/causal_attention_tensor.rs:31-55 (Q=K=0 causal -> running means), the
  exact mask patterns of causal_attention_tensor.rs:23-30, and torch float64
  autograd of softmax(scale*QK^T+mask)V at the reference's tolerance
  (grouped_attention_tensor.rs:10, 2e-3+3e-3|b|) on the reference's five GQA cases,
  the mask gradient included, and on random cases with a value width other than the
  head width.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(dtype=np.int64, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64
_int = ctypes.c_int


def build() -> str:
    """Compile liboracle.so with oracle/Makefile (gcc, no GPU needed)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.or_bf16.argtypes = [ctypes.c_float]
        L.or_bf16.restype = ctypes.c_float
        L.or_round_bf16.argtypes = [_f32p, _f32p, _i64]
        L.or_num_threads.restype = _int
        L.or_set_num_threads.argtypes = [_int]
        L.or_gemm_f64.argtypes = [_f32p, _f32p, _i64, _i64, _i64, _i64, _int, _int, _f64p]
        L.or_gemm_f64_sampled.argtypes = [_f32p, _f32p, _i64, _i64, _i64, _int, _int, _i64p, _i64p, _i64, _f64p]
        L.or_gemm_f32.argtypes = [_f32p, _f32p, _i64, _i64, _i64, _i64, _int, _int, _f32p]
        L.or_gemm_grouped_nt_f64.argtypes = [_f32p, _f32p, _i64, _i64, _i64, _i32p, _i64, _f64p]
        L.or_rms_norm_f64.argtypes = [_f32p, _f32p, _i64, _i64, ctypes.c_double, _f64p, _f64p]
        L.or_rms_norm_backward_f64.argtypes = [_f32p, _f32p, _f32p, _f64p, _i64, _i64, _f64p, _f64p]
        L.or_rms_norm_lanes_f32.argtypes = [_f32p, _f32p, _i64, _i64, ctypes.c_float, _f32p, _f32p]
        L.or_rms_norm_lanes_f32.restype = _int
        L.or_rms_norm_backward_lanes_f32.argtypes = [_f32p, _f32p, _f32p, _f32p, _i64, _i64, _f32p, _f32p]
        L.or_rms_norm_backward_lanes_f32.restype = _int
        L.or_column_sum_pairwise.argtypes = [_f32p, _i64, _i64, _f32p]
        L.or_rotary.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, _int, _int, _f32p]
        L.or_rotary_f64.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, _int, _int, _f64p]
        L.or_rotary_prefix.argtypes = [_f32p, _i64p, _i64p, _int, _i64, _int, _int, _f32p, _f32p, _f32p]
        L.or_rotary_prefix.restype = _int
        _vp = ctypes.c_void_p
        L.or_attention_f64.argtypes = [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                       ctypes.c_double, _int, ctypes.c_uint64, ctypes.c_uint64,
                                       _vp, _vp, _vp, _vp, _vp, _vp, _vp]
        L.or_causal_mask.argtypes = [_i64, _i64, _i64, ctypes.c_uint64, ctypes.c_uint64, _f32p]
        L.or_softmax_f64.argtypes = [_f32p, _i64, _i64, _int, _f64p]
        L.or_repeat_kv_backward.argtypes = [_f32p, _i64, _i64, _i64, _f32p]
        L.or_softmax_backward_f64.argtypes = [_f32p, _f32p, _i64, _i64, _int, _f64p]
        _lib = L
    return _lib


def set_threads(n: int) -> None:
    lib().or_set_num_threads(int(n))


def num_threads() -> int:
    return int(lib().or_num_threads())


# ------------------------------------------------------------------ BF16 helpers

def bf16_round(x) -> np.ndarray:
    """float32 values rounded to the nearest BF16 (RNE), returned as float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().or_round_bf16(x.reshape(-1), out.reshape(-1), x.size)
    return out


def bf16_bits(x) -> np.ndarray:
    """uint16 BF16 bit patterns of float32 values (RNE)."""
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def bf16_decode(bits) -> np.ndarray:
    """float32 values of uint16 BF16 bit patterns."""
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    return (bits.astype(np.uint32) << 16).view(np.float32)


# ------------------------------------------------------------------ inputs

_MASK = (1 << 64) - 1


def _splitmix64(x: np.ndarray) -> np.ndarray:
    x = (x + np.uint64(0x9E3779B97F4A7C15)) & np.uint64(_MASK)
    z = x
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def normal(shape, seed: int, stream: int, std: float = 1.0, mean: float = 0.0) -> np.ndarray:
    """Counter-based N(mean, std^2) float32: SplitMix64 of (seed, stream, index), then
    Box-Muller. Deterministic for a given (seed, stream), independent of the platform."""
    n = int(np.prod(shape)) if len(shape) else 1
    pairs = (n + 1) // 2
    idx = np.arange(pairs, dtype=np.uint64)
    base = np.uint64(((seed & 0xFFFFFFFF) << 32) ^ ((stream & 0xFFFF) << 48))
    with np.errstate(over="ignore"):
        u1 = _splitmix64(base + idx * np.uint64(2))
        u2 = _splitmix64(base + idx * np.uint64(2) + np.uint64(1))
    f1 = ((u1 >> np.uint64(11)).astype(np.float64) + 1.0) / float(1 << 53)
    f2 = (u2 >> np.uint64(11)).astype(np.float64) / float(1 << 53)
    r = np.sqrt(-2.0 * np.log(f1))
    z = np.concatenate([r * np.cos(2 * np.pi * f2), r * np.sin(2 * np.pi * f2)])[:n]
    return (z * std + mean).astype(np.float32).reshape(shape)


# ------------------------------------------------------------------ GEMM

def _c32(x):
    return np.ascontiguousarray(x, dtype=np.float32)


def gemm_f64(a, b, ta: bool, tb: bool) -> np.ndarray:
    """op(A) @ op(B) in f64 over float32 inputs; rank 2 or rank 3 (batched)."""
    a = _c32(a)
    b = _c32(b)
    batched = a.ndim == 3
    if not batched:
        a = a[None]
        b = b[None]
    g = a.shape[0]
    m, k = (a.shape[2], a.shape[1]) if ta else (a.shape[1], a.shape[2])
    n = b.shape[1] if tb else b.shape[2]
    out = np.empty((g, m, n), dtype=np.float64)
    lib().or_gemm_f64(a.reshape(-1), b.reshape(-1), g, m, n, k, int(ta), int(tb), out.reshape(-1))
    return out if batched else out[0]


def gemm_f32(a, b, ta: bool, tb: bool) -> np.ndarray:
    a = _c32(a)
    b = _c32(b)
    batched = a.ndim == 3
    if not batched:
        a = a[None]
        b = b[None]
    g = a.shape[0]
    m, k = (a.shape[2], a.shape[1]) if ta else (a.shape[1], a.shape[2])
    n = b.shape[1] if tb else b.shape[2]
    out = np.empty((g, m, n), dtype=np.float32)
    lib().or_gemm_f32(a.reshape(-1), b.reshape(-1), g, m, n, k, int(ta), int(tb), out.reshape(-1))
    return out if batched else out[0]


def gemm_grouped_nt_f64(a, w, ends) -> np.ndarray:
    """M-grouped NT product in f64: rows [ends[g-1], ends[g]) of A times W[g]^T.
    A [M,K], W [G,N,K]; rows past the last end are NaN."""
    a = _c32(a)
    w = _c32(w)
    ends = np.ascontiguousarray(ends, dtype=np.int32)
    m, k = a.shape
    g, n, kw = w.shape
    assert kw == k and ends.shape == (g,)
    out = np.empty((m, n), dtype=np.float64)
    lib().or_gemm_grouped_nt_f64(a.reshape(-1), w.reshape(-1), m, n, k, ends, g, out.reshape(-1))
    return out


def gemm_f64_sampled(a, b, ta: bool, tb: bool, rows, cols) -> np.ndarray:
    a = _c32(a)
    b = _c32(b)
    m, k = (a.shape[1], a.shape[0]) if ta else (a.shape[0], a.shape[1])
    n = b.shape[0] if tb else b.shape[1]
    rows = np.ascontiguousarray(rows, dtype=np.int64)
    cols = np.ascontiguousarray(cols, dtype=np.int64)
    out = np.empty(rows.shape[0], dtype=np.float64)
    lib().or_gemm_f64_sampled(a.reshape(-1), b.reshape(-1), m, n, k, int(ta), int(tb), rows, cols, rows.shape[0], out)
    return out


def matmul_shape(a_shape, b_shape):
    """Output shape of the generic floating matmul: generic_matrix::output_layout
    (rust-ascend-driver/src/tensor/runtime/generic_matrix.rs:4-15) over layout::matmul_shape and
    layout::broadcast (tensor/layout.rs:106-142): rank 2..6 each, A [..., M, K] @ B [..., K, N],
    batch dims broadcast from the right. Raises ValueError with the reference's reason."""
    a_shape, b_shape = tuple(int(d) for d in a_shape), tuple(int(d) for d in b_shape)
    if not (2 <= len(a_shape) <= 6 and 2 <= len(b_shape) <= 6):
        raise ValueError("generic matmul requires matching floating dtypes and rank 2..6")
    if a_shape[-1] != b_shape[-2]:
        raise ValueError("matmul contraction dimensions differ")
    ba, bb = a_shape[:-2], b_shape[:-2]
    rank = max(len(ba), len(bb))
    out = []
    for i in range(rank):  # from the right
        x = ba[len(ba) - 1 - i] if i < len(ba) else 1
        y = bb[len(bb) - 1 - i] if i < len(bb) else 1
        if x == y or y == 1:
            out.append(x)
        elif x == 1:
            out.append(y)
        else:
            raise ValueError("incompatible broadcast dimensions")
    return tuple(reversed(out)) + (a_shape[-2], b_shape[-1])


def _batch_index(batch, shape):
    """Index of the operand batch that output batch multi-index `batch` reads (broadcast dims -> 0)."""
    shape = tuple(shape)
    lead = len(batch) - len(shape)
    return tuple(0 if shape[d] == 1 else batch[lead + d] for d in range(len(shape)))


def tensor_matmul_f64(a, b) -> np.ndarray:
    """A @ B in float64 over the operands' exact values (F32, F16 or BF16-valued), batch dims
    broadcast per matmul_shape; each batch's product is the C restatement of the GEMM sum
    (or_gemm_f64). The KEEP_DTYPE rounding of the output is the caller's."""
    a, b = np.asarray(a), np.asarray(b)
    out_shape = matmul_shape(a.shape, b.shape)
    out = np.empty(out_shape, dtype=np.float64)
    for batch in np.ndindex(*out_shape[:-2]):
        ia, ib = _batch_index(batch, a.shape[:-2]), _batch_index(batch, b.shape[:-2])
        out[batch] = gemm_f64(a[ia].astype(np.float32), b[ib].astype(np.float32), False, False)
    return out


def tensor_matmul_backward_f64(a, b, dy):
    """(dA, dB) of A @ B in float64: dY B^T and A^T dY, each summed over the output batches that
    broadcast onto the operand's batch (the autodiff of matmul)."""
    a, b, dy = np.asarray(a), np.asarray(b), np.asarray(dy)
    out_shape = matmul_shape(a.shape, b.shape)
    da = np.zeros(a.shape, dtype=np.float64)
    db = np.zeros(b.shape, dtype=np.float64)
    for batch in np.ndindex(*out_shape[:-2]):
        ia, ib = _batch_index(batch, a.shape[:-2]), _batch_index(batch, b.shape[:-2])
        g = dy[batch].astype(np.float32)
        da[ia] += gemm_f64(g, b[ib].astype(np.float32), False, True)
        db[ib] += gemm_f64(a[ia].astype(np.float32), g, True, False)
    return da, db


def module_attention_f64(q, k, v, dy=None, mask=None, bias=None, scale=None, softcap=None, causal=False):
    """The backend's module attention in float64 (ModuleOps::attention, src/backend.rs:1323-1333,
    via the RUDA tensor library's attention_fallback, git rev 126b1c78 -- not vendored; the step
    order is that library's published composition): x = scale * Q K^T (scale defaults to
    1/sqrt(D)); t = c tanh(x / c) with a softcap c, else x; z = t + bias; z = -inf where causal
    (key > query) or mask (True); P = softmax(z) over the keys; O = P V. Q [B,H,Sq,D], K [B,H,Sk,D],
    V [B,H,Sk,Dv]; mask and bias broadcast onto [B,H,Sq,Sk]. With dy, the gradients dq, dk, dv and
    dbias (summed to the bias shape) from the chain rule through those steps."""
    q, k, v = (np.asarray(t, dtype=np.float64) for t in (q, k, v))
    b, h, sq, d = q.shape
    sk = k.shape[2]
    scale = 1.0 / np.sqrt(d) if scale is None else float(scale)
    x = np.einsum("bhqd,bhkd->bhqk", q, k) * scale
    t = softcap * np.tanh(x / softcap) if softcap else x
    z = t + (0.0 if bias is None else np.broadcast_to(np.asarray(bias, dtype=np.float64), x.shape))
    masked = np.zeros(x.shape, dtype=bool)
    if causal:
        masked |= np.arange(sk)[None, :] > np.arange(sq)[:, None]
    if mask is not None:
        masked |= np.broadcast_to(np.asarray(mask, dtype=bool), x.shape)
    z = np.where(masked, -np.inf, z)
    zmax = z.max(axis=-1, keepdims=True)
    e = np.exp(z - zmax)
    p = e / e.sum(axis=-1, keepdims=True)
    out = {"out": np.einsum("bhqk,bhkd->bhqd", p, v)}
    if dy is not None:
        dy = np.asarray(dy, dtype=np.float64)
        out["dv"] = np.einsum("bhqk,bhqd->bhkd", p, dy)
        dp = np.einsum("bhqd,bhkd->bhqk", dy, v)
        dz = p * (dp - (dp * p).sum(axis=-1, keepdims=True))
        dz = np.where(masked, 0.0, dz)
        if bias is not None:
            bshape = np.asarray(bias).shape
            axes = tuple(i for i in range(4) if bshape[i] == 1 and x.shape[i] != 1)
            out["dbias"] = dz.sum(axis=axes, keepdims=True) if axes else dz.copy()
        dx = dz * (1.0 - np.tanh(x / softcap) ** 2) if softcap else dz
        dx = dx * scale
        out["dq"] = np.einsum("bhqk,bhkd->bhqd", dx, k)
        out["dk"] = np.einsum("bhqk,bhqd->bhkd", dx, q)
    return out


# ------------------------------------------------------------------ RMSNorm

def rms_norm_f64(x, w, eps: float):
    x = _c32(x)
    width = x.shape[-1]
    rows = x.size // width if width else 0
    y = np.empty(x.shape, dtype=np.float64)
    rstd = np.empty(x.shape[:-1], dtype=np.float64)
    lib().or_rms_norm_f64(x.reshape(-1), _c32(w), rows, width, float(eps), y.reshape(-1), rstd.reshape(-1))
    return y, rstd


def rms_norm_backward_f64(x, w, dy, rstd):
    x = _c32(x)
    width = x.shape[-1]
    rows = x.size // width if width else 0
    dx = np.empty(x.shape, dtype=np.float64)
    dw = np.empty(width, dtype=np.float64)
    r = np.ascontiguousarray(rstd, dtype=np.float64).reshape(-1)
    lib().or_rms_norm_backward_f64(x.reshape(-1), _c32(w), _c32(dy).reshape(-1), r, rows, width,
                                   dx.reshape(-1), dw)
    return dx, dw


def rms_norm_lanes_f32(x, w, eps: float):
    x = _c32(x)
    width = x.shape[-1]
    rows = x.size // width
    y = np.empty(x.shape, dtype=np.float32)
    rstd = np.empty(x.shape[:-1], dtype=np.float32)
    rc = lib().or_rms_norm_lanes_f32(x.reshape(-1), _c32(w), rows, width, float(eps), y.reshape(-1), rstd.reshape(-1))
    if rc != 0:
        raise ValueError("row program order needs width % 32 == 0")
    return y, rstd


def rms_norm_backward_lanes_f32(x, w, dy, rstd):
    x = _c32(x)
    width = x.shape[-1]
    rows = x.size // width
    dx = np.empty(x.shape, dtype=np.float32)
    dw = np.empty(width, dtype=np.float32)
    rc = lib().or_rms_norm_backward_lanes_f32(x.reshape(-1), _c32(w), _c32(dy).reshape(-1),
                                              _c32(rstd).reshape(-1), rows, width, dx.reshape(-1), dw)
    if rc != 0:
        raise ValueError("row program order needs width % 32 == 0")
    return dx, dw


def column_sum_pairwise(parts) -> np.ndarray:
    parts = np.array(parts, dtype=np.float32, copy=True, order="C")
    rows, width = parts.shape
    out = np.empty(width, dtype=np.float32)
    lib().or_column_sum_pairwise(parts.reshape(-1), rows, width, out)
    return out


# ------------------------------------------------------------------ RoPE

def rotary(x, cos_t, sin_t, layout: int, backward: bool = False) -> np.ndarray:
    x = _c32(x)
    width = x.shape[-1]
    rows = x.size // width if width else 0
    y = np.empty_like(x)
    lib().or_rotary(x.reshape(-1), _c32(cos_t).reshape(-1), _c32(sin_t).reshape(-1), rows, width,
                    int(layout), int(backward), y.reshape(-1))
    return y


def rotary_f64(x, cos_t, sin_t, layout: int, backward: bool = False) -> np.ndarray:
    x = _c32(x)
    width = x.shape[-1]
    rows = x.size // width if width else 0
    y = np.empty(x.shape, dtype=np.float64)
    lib().or_rotary_f64(x.reshape(-1), _c32(cos_t).reshape(-1), _c32(sin_t).reshape(-1), rows, width,
                        int(layout), int(backward), y.reshape(-1))
    return y


def rotary_prefix(x, cos_t, sin_t, width: int, layout: int, backward: bool = False) -> np.ndarray:
    x = _c32(x)
    cos_t = _c32(cos_t)
    sin_t = _c32(sin_t)
    ins = np.array(x.shape, dtype=np.int64)
    tabs = np.array(cos_t.shape, dtype=np.int64)
    y = np.empty_like(x)
    rc = lib().or_rotary_prefix(x.reshape(-1), ins, tabs, x.ndim, int(width), int(layout), int(backward),
                                cos_t.reshape(-1), sin_t.reshape(-1), y.reshape(-1))
    if rc != 0:
        raise ValueError("invalid rotary prefix spec")
    return y


def softmax_f64(x, logarithmic: bool = False) -> np.ndarray:
    """Last-axis softmax / log-softmax in float64 (common_rows_validate.rs:55-58)."""
    x = _c32(x)
    width = x.shape[-1]
    out = np.empty(x.shape, np.float64)
    lib().or_softmax_f64(x, x.size // width if width else 0, width, int(logarithmic), out)
    return out


def softmax_backward_f64(y, dy, logarithmic: bool = False) -> np.ndarray:
    """dX from the saved output (common_rows_validate.rs:82-85)."""
    y, dy = _c32(y), _c32(dy)
    width = y.shape[-1]
    out = np.empty(y.shape, np.float64)
    lib().or_softmax_backward_f64(y, dy, y.size // width if width else 0, width, int(logarithmic), out)
    return out


def nll_loss_f64(logp, target, weight, reduction: int, ignore_index: int):
    """NLLLoss in float64: row loss -w[t] * logp[n, t], 0 for rows labelled ignore_index;
    reduction 0 None ([N]), 1 Mean (sum / W), 2 Sum; returns (loss, W) with W the summed weight of
    the non-ignored labels. Restates the expectation loop of examples/cross_entropy_tensor.rs:38-52
    (the reference's NLLLoss itself is the closed aclnnNLLLoss, tensor/loss.rs:31-46)."""
    logp = np.asarray(logp, np.float64)
    w = np.asarray(weight, np.float64)
    t = np.asarray(target, np.int64)
    rows = np.zeros(t.shape[0], np.float64)
    total = 0.0
    for n, label in enumerate(t):
        if label == ignore_index:
            continue
        rows[n] = -w[label] * logp[n, label]
        total += w[label]
    if reduction == 0:
        return rows, total
    s = rows.sum()
    if reduction == 1:
        return np.array([s / total if total != 0 else np.nan]), total
    return np.array([s]), total


def nll_loss_backward_f64(grad, shape, target, weight, total, reduction: int, ignore_index: int) -> np.ndarray:
    """Dense d loss / d logp in float64: -w[t_n] g_n at (n, t_n), g_n = grad[n] (None), grad[0]
    (Sum), grad[0] / total (Mean) (the derivative of nll_loss_f64; cross_entropy_tensor.rs:48-50
    for the composed cross entropy)."""
    g = np.asarray(grad, np.float64)
    w = np.asarray(weight, np.float64)
    out = np.zeros(shape, np.float64)
    for n, label in enumerate(np.asarray(target, np.int64)):
        if label == ignore_index:
            continue
        gn = g[n] if reduction == 0 else (g[0] / total if reduction == 1 else g[0])
        out[n, label] = -w[label] * gn
    return out


def silu_mul_f64(gate, up) -> np.ndarray:
    """gate * sigmoid(gate) * up in float64 (examples/silu_mul_tensor.rs:40-42)."""
    g = np.asarray(gate, np.float64)
    s = 1.0 / (1.0 + np.exp(-g))
    return g * s * np.asarray(up, np.float64)


def silu_mul_backward_f64(gate, up, dy):
    """(dgate, dup) in float64: derivative = s (1 + g (1 - s)); dgate = dy u derivative,
    dup = dy g s (examples/silu_mul_tensor.rs:40-44)."""
    g = np.asarray(gate, np.float64)
    u = np.asarray(up, np.float64)
    d = np.asarray(dy, np.float64)
    s = 1.0 / (1.0 + np.exp(-g))
    return d * u * (s * (1.0 + g * (1.0 - s))), d * g * s


def bias_add_f32(x, bias, residual=None) -> np.ndarray:
    """(x + residual) + bias[c] in float32, in that order (src/nn/affine.rs:21-25; the
    reference's BiasAddSpec program, runtime/affine.rs:10-22)."""
    x = np.asarray(x, np.float32)
    s = x + np.asarray(residual, np.float32) if residual is not None else x
    return (s + np.asarray(bias, np.float32)).astype(np.float32)


def bias_add_backward(dy) -> np.ndarray:
    """dbias = dY summed over the leading axes by the pairwise tree of
    runtime/normalization.rs:95-114 (runtime/affine.rs:23-26)."""
    dy = np.asarray(dy, np.float32)
    width = dy.shape[-1]
    return column_sum_pairwise(dy.reshape(-1, width))


def embedding(weight, ids) -> np.ndarray:
    """weight[ids]: [ids..., H] in the table's dtype (embedding.rs:27-34, the aclnnEmbedding
    lookup). IDs must lie in [0, V)."""
    weight = np.asarray(weight)
    ids = np.asarray(ids, np.int64)
    if ids.size and (ids.min() < 0 or ids.max() >= weight.shape[0]):
        raise ValueError("embedding index outside the table")
    return weight[ids]


def embedding_backward_f64(grad, ids, num_weights: int, padding_idx=None, scale_grad_by_freq=False):
    """Dense weight gradient in float64 (embedding.rs:60-79, the aclnnEmbeddingDenseBackward
    semantics the reference's examples/embedding_tensor.rs:31-39 checks): every position adds its
    gradient row to its ID's row; the padding row stays zero; with frequency scaling each row is
    divided by how often its ID occurs."""
    grad = np.asarray(grad, np.float64)
    ids = np.asarray(ids, np.int64).reshape(-1)
    g = grad.reshape(ids.size, grad.shape[-1])
    dw = np.zeros((int(num_weights), g.shape[1]), np.float64)
    np.add.at(dw, ids, g)
    if scale_grad_by_freq:
        counts = np.bincount(ids, minlength=int(num_weights)).astype(np.float64)
        nz = counts > 0
        dw[nz] /= counts[nz, None]
    if padding_idx is not None:
        dw[padding_idx] = 0.0
    return dw


def repeat_kv(x, query_heads: int) -> np.ndarray:
    """[B,Hkv,N,D] -> [B,Hq,N,D], kv_head = q_head // (Hq/Hkv) (heads_programs.rs:42-55)."""
    x = np.asarray(x, np.float32)
    return np.repeat(x, query_heads // x.shape[1], axis=1)


def repeat_kv_backward(dy, kv_heads: int) -> np.ndarray:
    """[B,Hq,N,D] -> [B,Hkv,N,D], the replicas summed in F32 in the reference's level order
    (runtime/heads.rs:29-51)."""
    dy = _c32(dy)
    b, hq, n, d = dy.shape
    out = np.empty((b, kv_heads, n, d), np.float32)
    lib().or_repeat_kv_backward(dy, b * kv_heads, hq // kv_heads, n * d, out)
    return out


def rope_tables(positions, dim: int, theta: float):
    """cos/sin tables [len(positions), dim/2]: angle = pos * theta^(-2i/dim), computed in
    f64 and rounded to f32 (the reference has no frequency policy; the caller builds
    the tables, rotary_programs.rs:1)."""
    pos = np.asarray(positions, dtype=np.float64)[:, None]
    inv = theta ** (-np.arange(0, dim, 2, dtype=np.float64) / dim)
    ang = pos * inv[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


# ------------------------------------------------------------------ attention

def attention_f64(q, k, v, dy=None, scale=0.25, causal=False, query_start=0, key_start=0,
                  mask=None, want_grads=True, magnitudes=False):
    """Returns dict(out, lse[, dq, dk, dv[, dmask]]) in f64 for q [B,Hq,M,D], k [B,Hkv,N,D],
    v [B,Hkv,N,Dv]. With a mask (additive, [B,Hq,M,N], used when not causal) and dy, also dmask,
    the gradient of the masked scores. With magnitudes=True also out_mag/dq_mag/dk_mag/dv_mag:
    each output's sum over the absolute values of its terms (the scale against which a rounding
    of any term is measured)."""
    q = _c32(q)
    k = _c32(k)
    v = _c32(v)
    B, H, M, D = q.shape
    Hkv, N, Dv = k.shape[1], k.shape[2], v.shape[3]
    out = np.empty((B, H, M, Dv), dtype=np.float64)
    lse = np.empty((B, H, M), dtype=np.float64)
    res = {"out": out, "lse": lse}
    ptr = lambda a: None if a is None else a.ctypes.data
    dq = dk = dv = dmask = None
    dyc = None
    maskc = None if mask is None else _c32(mask)
    if dy is not None:
        dyc = _c32(dy)
        if want_grads:
            dq = np.empty((B, H, M, D), dtype=np.float64)
            dk = np.empty((B, Hkv, N, D), dtype=np.float64)
            dv = np.empty((B, Hkv, N, Dv), dtype=np.float64)
            res.update(dq=dq, dk=dk, dv=dv)
        if maskc is not None and not causal:
            dmask = np.empty((B, H, M, N), dtype=np.float64)
            res["dmask"] = dmask
    mag = None
    if magnitudes:
        mag = np.empty(B * H * M * (D + Dv) + B * Hkv * N * (D + Dv), dtype=np.float64)
    lib().or_attention_f64(ptr(q), ptr(k), ptr(v), ptr(dyc), ptr(maskc), B, H, Hkv, M, N, D, Dv,
                           float(scale), int(bool(causal)), int(query_start), int(key_start),
                           ptr(out), ptr(lse), ptr(dq), ptr(dk), ptr(dv), ptr(mag), ptr(dmask))
    if magnitudes:
        a, aq, c, cv = B * H * M * Dv, B * H * M * D, B * Hkv * N * D, B * Hkv * N * Dv
        res["out_mag"] = mag[:a].reshape(out.shape)
        res["dq_mag"] = mag[a:a + aq].reshape((B, H, M, D))
        res["dk_mag"] = mag[a + aq:a + aq + c].reshape((B, Hkv, N, D))
        res["dv_mag"] = mag[a + aq + c:a + aq + c + cv].reshape((B, Hkv, N, Dv))
    return res


def mag_err(actual, expected, magnitude) -> float:
    """max_i |a-b| / magnitude_i, magnitude = the sum of |terms| of each output (attention)."""
    a = np.asarray(actual, dtype=np.float64)
    b = np.asarray(expected, dtype=np.float64)
    mg = np.asarray(magnitude, dtype=np.float64)
    if a.size == 0:
        return 0.0
    if not np.all(np.isfinite(a)):
        return float("inf")
    floor = 1e-6 * max(float(np.max(mg)), 1e-30)
    return float(np.max(np.abs(a - b) / np.maximum(mg, floor)))


def causal_mask(batch, queries, keys, query_start, key_start) -> np.ndarray:
    out = np.empty((batch, queries, keys), dtype=np.float32)
    lib().or_causal_mask(batch, queries, keys, int(query_start), int(key_start), out.reshape(-1))
    return out


# ------------------------------------------------------------------ comparison

def rel_err(actual, expected, atol_frac: float = 1e-3) -> float:
    """max_i |a-b| / (|b| + atol), atol = atol_frac * rms(b) (1e-3 by default). Infinite when a
    has a non-finite value where b is finite."""
    a = np.asarray(actual, dtype=np.float64).reshape(-1)
    b = np.asarray(expected, dtype=np.float64).reshape(-1)
    if a.size == 0:
        return 0.0
    if not np.all(np.isfinite(a[np.isfinite(b)])):
        return float("inf")
    rms = float(np.sqrt(np.mean(b * b)))
    atol = atol_frac * rms if rms > 0 else 1e-30
    return float(np.max(np.abs(a - b) / (np.abs(b) + atol)))


def row_err(actual, expected) -> float:
    """max over rows (the last axis) of ||a_row - b_row||_2 / ||b_row||_2; a row whose expected
    norm is zero contributes ||a_row||_2 divided by the largest row norm (so an all-zero row must
    come back near zero). Infinite when a has a non-finite value."""
    a = np.asarray(actual, dtype=np.float64)
    b = np.asarray(expected, dtype=np.float64)
    if a.size == 0:
        return 0.0
    a = a.reshape(-1, a.shape[-1])
    b = b.reshape(-1, b.shape[-1])
    if not np.all(np.isfinite(a)):
        return float("inf")
    nb = np.sqrt(np.sum(b * b, axis=1))
    ne = np.sqrt(np.sum((a - b) ** 2, axis=1))
    floor = max(float(np.max(nb)), 1e-300)
    return float(np.max(np.where(nb > 0, ne / np.where(nb > 0, nb, 1.0), ne / floor)))
