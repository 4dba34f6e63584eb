"""HipRuntime: the MI355X counterpart of the reference's AscendRuntime static entry points
(rust-ascend-driver/src/tensor/runtime/mod.rs:147-435), over the C ABI of libhk.so.

Tensors are torch tensors on the GPU: torch provides device allocation and the current
stream, libhk.so does every computation. Each method validates through the C ABI (which
checks shapes before any device work), allocates outputs with torch (the reference's
allocating forms), and raises HkError on failure. Methods keep the reference's names,
argument meaning and return arity.
"""
from __future__ import annotations

import ctypes
import enum
import threading

import torch

from . import _lib
from ._lib import BF16, BOOL, F16, F32, I32, I64, NO_PADDING, HkError, check, tensor_desc


class Transpose(enum.IntEnum):
    """Reference: deepgemm::Transpose (rust-ascend-driver/src/tensor/deepgemm/plan.rs:7)."""
    No = 0
    Yes = 1


class LossReduction(enum.IntEnum):
    """Reference: LossReduction (rust-ascend-driver/src/tensor/loss.rs:3-6)."""
    None_ = 0
    Mean = 1
    Sum = 2


def _ignore(ignore_index):
    """NllLossOptions::ignore (tensor/loss.rs:10-12): the explicit ignore label, else -1."""
    return -1 if ignore_index is None else int(ignore_index)


class RotaryLayout(enum.IntEnum):
    """Reference: RotaryLayout (rust-ascend-compiler/src/ascend/rotary_programs.rs:5-6)."""
    Interleaved = 0
    SplitHalf = 1


_DTYPES = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16, torch.int32: I32, torch.int64: I64,
           torch.bool: BOOL}
_TORCH = {v: k for k, v in _DTYPES.items()}

_ctx = None
_ctx_lock = threading.Lock()


def _context():
    """The process-wide context (initialize_exclusive, runtime/mod.rs:424-435), created on
    first use on torch's current CUDA device."""
    global _ctx
    with _ctx_lock:
        if _ctx is None:
            lib = _lib.load()
            if not torch.cuda.is_available():
                raise HkError(_lib.LOAD_ERROR, "no GPU visible to torch; libhk.so has no CPU fallback")
            h = ctypes.c_void_p()
            check(lib.hk_init(torch.cuda.current_device(), ctypes.byref(h)))
            _ctx = h
        return _ctx


def _call(name: str, *args) -> None:
    lib = _lib.load()
    ctx = _context()
    check(lib.hk_set_stream(ctx, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    check(getattr(lib, name)(ctx, *args))


def desc(t: torch.Tensor):
    """hk_tensor descriptor of a contiguous GPU tensor."""
    if not isinstance(t, torch.Tensor):
        raise HkError(_lib.INVALID_ARGUMENT, f"expected a torch.Tensor, got {type(t).__name__}")
    if t.dtype not in _DTYPES:
        raise HkError(_lib.INVALID_ARGUMENT, f"unsupported dtype {t.dtype}")
    if not t.is_contiguous():
        raise HkError(_lib.INVALID_ARGUMENT, "native buffers must be contiguous")
    if t.numel() and not t.is_cuda:
        raise HkError(_lib.INVALID_ARGUMENT, "tensors must be on the GPU")
    return ctypes.byref(tensor_desc(t.data_ptr() if t.numel() else 0, _DTYPES[t.dtype], t.shape))


def _empty(shape, dtype, like: torch.Tensor) -> torch.Tensor:
    return torch.empty(tuple(shape), dtype=dtype, device=like.device)


def gemm_plan(a_shape, b_shape, ta, tb, out_dtype=torch.bfloat16, a_dtype=torch.bfloat16, b_dtype=torch.bfloat16):
    """Host-only GEMM contract check (GemmSpec::new, plan.rs:49-80); needs no GPU.
    Returns dict(kind, batch, m, n, k, out_shape, key) or raises HkError."""
    lib = _lib.load()
    ta_ = tensor_desc(0, _DTYPES[a_dtype], a_shape)
    tb_ = tensor_desc(0, _DTYPES[b_dtype], b_shape)
    # descriptors of non-empty tensors need a non-null pointer; the plan never dereferences it
    ta_.data = 256
    tb_.data = 256
    plan = _lib.HkGemmPlan()
    check(lib.hk_gemm_plan_check(ctypes.byref(ta_), ctypes.byref(tb_), int(ta), int(tb), _DTYPES[out_dtype],
                                 ctypes.byref(plan)))
    return {"kind": "dense" if plan.kind == 0 else "batched", "batch": plan.batch, "m": plan.m, "n": plan.n,
            "k": plan.k, "out_shape": tuple(plan.out_shape[:plan.out_rank]), "key": plan.key.decode()}


def _ends_array(ends):
    ends = [int(e) for e in ends]
    return (ctypes.c_int32 * max(len(ends), 1))(*ends), len(ends)


def grouped_gemm_plan(a_shape, w_shape, ends, out_dtype=torch.bfloat16, a_dtype=torch.bfloat16,
                      w_dtype=torch.bfloat16):
    """Host-only M-grouped NT contract check (GemmSpec::grouped_nt, plan.rs:61-67); needs no GPU."""
    lib = _lib.load()
    ta_ = tensor_desc(256, _DTYPES[a_dtype], a_shape)
    tw_ = tensor_desc(256, _DTYPES[w_dtype], w_shape)
    arr, count = _ends_array(ends)
    plan = _lib.HkGemmPlan()
    check(lib.hk_gemm_grouped_plan_check(ctypes.byref(ta_), ctypes.byref(tw_), arr, count, _DTYPES[out_dtype],
                                         ctypes.byref(plan)))
    return {"kind": "mgrouped", "groups": plan.batch, "m": plan.m, "n": plan.n, "k": plan.k,
            "out_shape": tuple(plan.out_shape[:plan.out_rank]), "key": plan.key.decode()}


def check_group_ends(ends) -> None:
    """Reference: GroupEnds::new (deepgemm/plan.rs:16-26): 1..=4096 nondecreasing multiples of
    256, not all zero. Raises HkError."""
    arr, count = _ends_array(ends)
    check(_lib.load().hk_group_ends_check(arr, count))


def matmul_layout(a_shape, b_shape, dtype=torch.float32):
    """Host-only output shape of the generic matmul (generic_matrix::output_layout,
    runtime/generic_matrix.rs:4-15): matching floating dtypes, rank 2..6, broadcast batch dims."""
    lib = _lib.load()
    ta_ = tensor_desc(256, _DTYPES[dtype], a_shape)
    tb_ = tensor_desc(256, _DTYPES[dtype], b_shape)
    out = _lib.HkTensor()
    check(lib.hk_matmul_layout(ctypes.byref(ta_), ctypes.byref(tb_), ctypes.byref(out)))
    return tuple(int(out.shape[i]) for i in range(out.rank))


class DeviceGroupEnds:
    """Checked group ends uploaded once (DeepGemm::upload_group_ends / DeviceGroupEnds,
    deepgemm/mod.rs:61-67); immutable, reused by every grouped call, freed on close()."""

    def __init__(self, ends):
        arr, count = _ends_array(ends)
        h = ctypes.c_void_p()
        _call("hk_group_ends_upload", arr, count, ctypes.byref(h))
        self.ends = tuple(int(e) for e in ends)
        self._handle = h

    @property
    def handle(self):
        if self._handle is None:
            raise HkError(_lib.INVALID_ARGUMENT, "group ends already freed")
        return self._handle

    def close(self) -> None:
        if self._handle is not None:
            _call("hk_group_ends_free", self._handle)
            self._handle = None


def _padded(shape):
    """Shape with its two matrix axes rounded up to multiples of 16 (deepgemm/padded.rs:26-31)."""
    shape = tuple(int(d) for d in shape)
    return shape[:-2] + tuple((d + 15) // 16 * 16 for d in shape[-2:])


class HipRuntime:
    """Static entry points mirroring AscendRuntime (runtime/mod.rs:147-435)."""

    # ---------------------------------------------------------------- runtime

    @staticmethod
    def initialize_exclusive():
        """Reference: AscendRuntime::initialize_exclusive (mod.rs:424-435)."""
        _context()

    @staticmethod
    def set_async(enabled: bool) -> None:
        """Benchmark mode: leave work queued instead of synchronizing after each op."""
        lib = _lib.load()
        check(lib.hk_set_async(_context(), 1 if enabled else 0))

    @staticmethod
    def synchronize() -> None:
        lib = _lib.load()
        ctx = _context()
        check(lib.hk_set_stream(ctx, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
        check(lib.hk_sync(ctx))

    @staticmethod
    def stats() -> dict:
        lib = _lib.load()
        s = _lib.HkStats()
        check(lib.hk_get_stats(_context(), ctypes.byref(s)))
        return {"modules_loaded": s.modules_loaded, "launches": s.launches, "synchronizations": s.synchronizations}

    @staticmethod
    def workspace_size() -> int:
        """Bytes of device scratch the context holds for later calls."""
        n = ctypes.c_uint64()
        check(_lib.load().hk_workspace_size(_context(), ctypes.byref(n)))
        return int(n.value)

    @staticmethod
    def trim_workspace(keep_bytes: int = 0) -> None:
        """Frees the context's scratch when it holds more than keep_bytes (after queued work)."""
        lib = _lib.load()
        ctx = _context()
        check(lib.hk_set_stream(ctx, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
        check(lib.hk_trim_workspace(ctx, ctypes.c_uint64(keep_bytes)))

    # ---------------------------------------------------------------- GEMM

    @staticmethod
    def gemm(a, b, ta=Transpose.No, tb=Transpose.No, dtype=torch.bfloat16):
        """Reference: AscendRuntime::gemm (mod.rs:344-348)."""
        plan = gemm_plan(a.shape, b.shape, ta, tb, dtype, a.dtype, b.dtype)
        out = _empty(plan["out_shape"], dtype, a)
        HipRuntime.gemm_into(a, b, ta, tb, out)
        return out

    @staticmethod
    def gemm_into(a, b, ta, tb, out) -> None:
        """Reference: AscendRuntime::gemm_into (mod.rs:350-354)."""
        _call("hk_gemm_into", desc(a), desc(b), int(ta), int(tb), desc(out))

    @staticmethod
    def upload_group_ends(ends) -> DeviceGroupEnds:
        """Reference: DeepGemm::upload_group_ends (deepgemm/mod.rs:61-67)."""
        return DeviceGroupEnds(ends)

    @staticmethod
    def grouped_nt(a, weights, groups: DeviceGroupEnds, dtype=torch.bfloat16):
        """out[M,N] = A[M,K] W[g]^T per aligned row group. Reference: DeepGemm::grouped_nt (mod.rs:68-73)."""
        plan = grouped_gemm_plan(a.shape, weights.shape, groups.ends, dtype, a.dtype, weights.dtype)
        out = _empty(plan["out_shape"], dtype, a)
        HipRuntime.grouped_nt_into(a, weights, groups, out)
        return out

    @staticmethod
    def grouped_nt_into(a, weights, groups: DeviceGroupEnds, out) -> None:
        """Reference: DeepGemm::grouped_nt_into (mod.rs:74-78)."""
        _call("hk_gemm_grouped_nt_into", desc(a), desc(weights), groups.handle, desc(out))

    @staticmethod
    def tensor_matmul(a, b):
        """A @ B in the inputs' dtype (F32, F16 or BF16), batch dims broadcast, any M/N/K.
        Reference: AscendRuntime::tensor_matmul (mod.rs:156-158), behind RudaAscend::float_matmul
        (src/backend.rs:692-703)."""
        if a.dtype != b.dtype:
            raise HkError(_lib.INVALID_ARGUMENT, "generic matmul requires matching floating dtypes and rank 2..6")
        out = _empty(matmul_layout(a.shape, b.shape, a.dtype), a.dtype, a)
        _call("hk_tensor_matmul", desc(a), desc(b), desc(out))
        return out

    @staticmethod
    def matmul_fp32(a, b):
        """Reference: AscendRuntime::matmul_fp32 (mod.rs:150-155): tensor_matmul on F32 inputs only."""
        if a.dtype != torch.float32 or b.dtype != torch.float32:
            raise HkError(_lib.INVALID_ARGUMENT, "matmul_fp32 requires FP32 inputs")
        return HipRuntime.tensor_matmul(a, b)

    @staticmethod
    def tensor_matmul_backward(a, b, grad):
        """[dA, dB] of A @ B: dY B^T and A^T dY, summed over each operand's broadcast batch dims."""
        da = _empty(a.shape, a.dtype, a)
        db = _empty(b.shape, b.dtype, a)
        _call("hk_tensor_matmul_backward", desc(a), desc(b), desc(grad), desc(da), desc(db))
        return da, db

    @staticmethod
    def swap_last_dims(x):
        """x with its last two dims swapped, materialized (float_swap_dims + contiguous,
        src/backend.rs:133-140,641)."""
        y = _empty(tuple(x.shape[:-2]) + (x.shape[-1], x.shape[-2]), x.dtype, x)
        _call("hk_swap_last_dims", desc(x), desc(y))
        return y

    @staticmethod
    def attention_scores(s, scale, softcap=0.0, bias=None, mask=None, causal=False):
        """masked ? -inf : softcap(s * scale) + bias over F32 scores [B, H, Sq, Sk] (module attention's
        score step, the fallback composition behind ModuleOps::attention, src/backend.rs:1323-1333)."""
        out = _empty(s.shape, torch.float32, s)
        _call("hk_attention_scores", desc(s), float(scale), float(softcap or 0.0),
              None if bias is None else desc(bias), None if mask is None else desc(mask), int(bool(causal)), desc(out))
        return out

    @staticmethod
    def attention_scores_backward(s, grad, scale, softcap=0.0, mask=None, causal=False, bias_shape=None):
        """[dS, dBias or None]: the score step's gradient (zero where masked) and, for a bias of
        bias_shape, its gradient summed over the broadcast dims."""
        ds = _empty(s.shape, torch.float32, s)
        dbias = None if bias_shape is None else _empty(bias_shape, torch.float32, s)
        _call("hk_attention_scores_backward", desc(s), desc(grad), float(scale), float(softcap or 0.0),
              None if mask is None else desc(mask), int(bool(causal)), desc(ds), None if dbias is None else desc(dbias))
        return ds, dbias

    @staticmethod
    def linear_nt_backward(x, w, dy):
        """[BF16 dX, F32 dW] for Y = X W^T. Reference: AscendRuntime::linear_nt_backward (mod.rs:357-362)."""
        dx = _empty(x.shape, torch.bfloat16, x)
        dw = _empty(w.shape, torch.float32, x)
        _call("hk_linear_nt_backward", desc(x), desc(w), desc(dy), desc(dx), desc(dw))
        return dx, dw

    @staticmethod
    def gemm_bf16_fp32(a, b, ta=Transpose.No, tb=Transpose.No):
        """[F32 out, saved BF16 A, saved BF16 B]. Reference: AscendRuntime::gemm_bf16_fp32 (mod.rs:388-392)."""
        plan = gemm_plan(a.shape, b.shape, ta, tb, torch.float32)
        out = _empty(plan["out_shape"], torch.float32, a)
        ab = _empty(a.shape, torch.bfloat16, a)
        bb = _empty(b.shape, torch.bfloat16, a)
        _call("hk_gemm_bf16_fp32", desc(a), desc(b), int(ta), int(tb), desc(out), desc(ab), desc(bb))
        return out, ab, bb

    @staticmethod
    def gemm_bf16_fp32_backward(a_bf16, b_bf16, grad, ta=Transpose.No, tb=Transpose.No):
        """[F32 dA, F32 dB] in the physical input layouts. Reference: mod.rs:395-399."""
        da = _empty(a_bf16.shape, torch.float32, a_bf16)
        db = _empty(b_bf16.shape, torch.float32, a_bf16)
        _call("hk_gemm_bf16_fp32_backward", desc(a_bf16), desc(b_bf16), desc(grad), int(ta), int(tb), desc(da),
              desc(db))
        return da, db

    @staticmethod
    def gemm_padded_bf16_fp32(a, b, ta=Transpose.No, tb=Transpose.No):
        """[F32 logical out, padded BF16 A snapshot, padded BF16 B snapshot] for any positive
        M/N/K. Reference: AscendRuntime::gemm_padded_bf16_fp32 (mod.rs:186-190)."""
        r = a.dim()
        if r not in (2, 3) or b.dim() != r:
            raise HkError(_lib.INVALID_ARGUMENT, "padded GEMM requires matching rank-2/3 FP32/BF16 inputs")
        m = a.shape[-1] if int(ta) else a.shape[-2]
        n = b.shape[-2] if int(tb) else b.shape[-1]
        lead = tuple(a.shape[:-2])
        out = _empty(lead + (m, n), torch.float32, a)
        ap = _empty(_padded(a.shape), torch.bfloat16, a)
        bp = _empty(_padded(b.shape), torch.bfloat16, a)
        _call("hk_gemm_padded_bf16_fp32", desc(a), desc(b), int(ta), int(tb), desc(out), desc(ap), desc(bp))
        return out, ap, bp

    @staticmethod
    def gemm_padded_bf16_fp32_backward(a_pad, b_pad, grad, a_shape, b_shape, ta=Transpose.No, tb=Transpose.No):
        """[F32 dA in a_shape, F32 dB in b_shape] (the original physical input shapes).
        Reference: AscendRuntime::gemm_padded_bf16_fp32_backward (mod.rs:191-195)."""
        da = _empty(tuple(a_shape), torch.float32, grad)
        db = _empty(tuple(b_shape), torch.float32, grad)
        _call("hk_gemm_padded_bf16_fp32_backward", desc(a_pad), desc(b_pad), desc(grad), int(ta), int(tb), desc(da),
              desc(db))
        return da, db

    @staticmethod
    def linear_frozen_bf16_fp32(x, weight):
        """F32 Y = bf16(X) W^T for a fixed BF16 weight used in place. Reference:
        AscendRuntime::linear_frozen_bf16_fp32 (mod.rs:379-382)."""
        if x.dim() != 2 or weight.dim() != 2:
            raise HkError(_lib.INVALID_ARGUMENT, "frozen BF16 linear requires rank-2 FP32 input and fixed BF16 weight")
        y = _empty((x.shape[0], weight.shape[0]), torch.float32, x)
        _call("hk_linear_frozen_bf16_fp32", desc(x), desc(weight), desc(y))
        return y

    @staticmethod
    def linear_frozen_bf16_fp32_backward(input_shape, weight, grad):
        """F32 dX in input_shape from the fixed BF16 weight and F32 dY. Reference:
        AscendRuntime::linear_frozen_bf16_fp32_backward (mod.rs:383-386)."""
        dx = _empty(tuple(input_shape), torch.float32, grad)
        _call("hk_linear_frozen_bf16_fp32_backward", desc(weight), desc(grad), desc(dx))
        return dx

    @staticmethod
    def linear_frozen_padded_bf16_fp32(x, weight):
        """[F32 Y, the BF16 weight the backward uses]: the weight itself when its axes are multiples
        of 16, else a zero-padded copy. Reference: AscendRuntime::linear_frozen_padded_bf16_fp32
        (mod.rs:196-200)."""
        if x.dim() != 2 or weight.dim() != 2:
            raise HkError(_lib.INVALID_ARGUMENT, "frozen padded linear requires rank-2 FP32 input and fixed BF16 weight")
        y = _empty((x.shape[0], weight.shape[0]), torch.float32, x)
        if tuple(weight.shape) == _padded(weight.shape):
            _call("hk_linear_frozen_padded_bf16_fp32", desc(x), desc(weight), desc(y), None)
            return y, weight
        wp = _empty(_padded(weight.shape), torch.bfloat16, x)
        _call("hk_linear_frozen_padded_bf16_fp32", desc(x), desc(weight), desc(y), desc(wp))
        return y, wp

    @staticmethod
    def linear_frozen_padded_bf16_fp32_backward(weight_pad, grad, input_shape, weight_shape=None):
        """F32 dX in input_shape. weight_shape (the logical [N, K]) is implied by grad and
        input_shape and only checked. Reference: linear_frozen_padded_bf16_fp32_backward (mod.rs:201-204)."""
        if weight_shape is not None and (tuple(weight_shape) != (grad.shape[-1], input_shape[-1])):
            raise HkError(_lib.INVALID_ARGUMENT, "frozen padded linear saved weight or dY layout mismatch")
        dx = _empty(tuple(input_shape), torch.float32, grad)
        _call("hk_linear_frozen_padded_bf16_fp32_backward", desc(weight_pad), desc(grad), desc(dx))
        return dx

    @staticmethod
    def linear_bf16_fp32(x, w):
        """[F32 Y, saved BF16 X, saved BF16 W]. Reference: AscendRuntime::linear_bf16_fp32 (mod.rs:364-370)."""
        y = _empty((x.shape[0], w.shape[0]) if x.dim() == 2 and w.dim() == 2 else (0,), torch.float32, x)
        xb = _empty(x.shape, torch.bfloat16, x)
        wb = _empty(w.shape, torch.bfloat16, x)
        _call("hk_linear_bf16_fp32", desc(x), desc(w), desc(y), desc(xb), desc(wb))
        return y, xb, wb

    @staticmethod
    def linear_bf16_fp32_backward(x_bf16, w_bf16, grad):
        """[F32 dX, F32 dW]. Reference: AscendRuntime::linear_bf16_fp32_backward (mod.rs:372-377)."""
        dx = _empty(x_bf16.shape, torch.float32, x_bf16)
        dw = _empty(w_bf16.shape, torch.float32, x_bf16)
        _call("hk_linear_bf16_fp32_backward", desc(x_bf16), desc(w_bf16), desc(grad), desc(dx), desc(dw))
        return dx, dw

    @staticmethod
    def cast(x, dtype):
        """Reference: AscendRuntime::cast (mod.rs:271-274)."""
        out = _empty(x.shape, dtype, x)
        HipRuntime.cast_into(x, out)
        return out

    @staticmethod
    def cast_into(x, out) -> None:
        """Reference: AscendRuntime::cast_into (mod.rs:276-279)."""
        _call("hk_cast_into", desc(x), desc(out))

    # ---------------------------------------------------------------- SwiGLU gate

    @staticmethod
    def silu_mul(gate, up):
        """SiLU(gate) * up. Reference: AscendRuntime::silu_mul (mod.rs:282-285)."""
        y = _empty(gate.shape, gate.dtype, gate)
        _call("hk_silu_mul", desc(gate), desc(up), desc(y))
        return y

    @staticmethod
    def silu_mul_backward(gate, up, grad):
        """[dGate, dUp]. Reference: AscendRuntime::silu_mul_backward (mod.rs:287-290)."""
        dg = _empty(gate.shape, gate.dtype, gate)
        du = _empty(gate.shape, gate.dtype, gate)
        _call("hk_silu_mul_backward", desc(gate), desc(up), desc(grad), desc(dg), desc(du))
        return dg, du

    # ---------------------------------------------------------------- bias and residual add

    @staticmethod
    def bias_add(x, bias, residual=None):
        """(X + residual) + bias over the last axis (residual optional; bias may be None when a
        residual is given). Reference: AscendRuntime::bias_add (mod.rs:177-181)."""
        y = _empty(x.shape, x.dtype, x)
        _call("hk_bias_add", desc(x), desc(bias) if bias is not None else None,
              desc(residual) if residual is not None else None, desc(y))
        return y

    # ---------------------------------------------------------------- decoder-layer relayouts

    @staticmethod
    def qkv_rope_split(qkv, cos, sin, q_heads: int, kv_heads: int, layout=None):
        """qkv [B,S,(Hq+2Hkv)D] -> (q [B,Hq,S,D], k, v [B,Hkv,S,D]) with RoPE on q and k; tables [S, D/2]."""
        layout = RotaryLayout.SplitHalf if layout is None else layout
        b, s, w = qkv.shape
        d = w // (q_heads + 2 * kv_heads)
        q = _empty((b, q_heads, s, d), qkv.dtype, qkv)
        k = _empty((b, kv_heads, s, d), qkv.dtype, qkv)
        v = _empty((b, kv_heads, s, d), qkv.dtype, qkv)
        _call("hk_qkv_rope_split", desc(qkv), desc(cos), desc(sin), int(layout), desc(q), desc(k), desc(v))
        return q, k, v

    @staticmethod
    def qkv_rope_merge(dq, dk, dv, cos, sin, layout=None):
        """(dq, dk, dv) -> dqkv [B,S,(Hq+2Hkv)D], the transpose of qkv_rope_split."""
        layout = RotaryLayout.SplitHalf if layout is None else layout
        b, hq, s, d = dq.shape
        out = _empty((b, s, (hq + 2 * dk.shape[1]) * d), dq.dtype, dq)
        _call("hk_qkv_rope_merge", desc(dq), desc(dk), desc(dv), desc(cos), desc(sin), int(layout), desc(out))
        return out

    @staticmethod
    def qkv_projection_rope(x, w, cos, sin, batch: int, q_heads: int, kv_heads: int, layout=None):
        """The fused QKV projection with RoPE: x [B*S, H] times w [(Hq+2Hkv)*128, H]^T straight into
        (q [B,Hq,S,128], k, v [B,Hkv,S,128]), q and k rotated (tables [S, 64])."""
        layout = RotaryLayout.SplitHalf if layout is None else layout
        d = w.shape[0] // (q_heads + 2 * kv_heads)
        s = x.shape[-2] if x.dim() == 3 else x.shape[0] // batch
        q = _empty((batch, q_heads, s, d), x.dtype, x)
        k = _empty((batch, kv_heads, s, d), x.dtype, x)
        v = _empty((batch, kv_heads, s, d), x.dtype, x)
        _call("hk_qkv_projection_rope", desc(x), desc(w), desc(cos), desc(sin), int(layout), desc(q), desc(k),
              desc(v))
        return q, k, v

    @staticmethod
    def attention_backward_qkv_rows(q, k, v, o, lse, grad, cos, sin, scale: float, causal: bool = True,
                                    query_start: int = 0, key_start: int = 0, layout=None):
        """The attention backward into the fused projection's gradient rows dqkv [B,S,(Hq+2Hkv)D]
        (BF16), dQ and dK rotated back."""
        layout = RotaryLayout.SplitHalf if layout is None else layout
        b, hq, s, d = q.shape
        out = _empty((b, s, (hq + 2 * k.shape[1]) * d), torch.bfloat16, q)
        _call("hk_attention_backward_qkv_rows", desc(q), desc(k), desc(v), desc(o), desc(lse), desc(grad),
              float(scale), int(bool(causal)), int(query_start), int(key_start), desc(cos), desc(sin), int(layout),
              desc(out))
        return out

    @staticmethod
    def heads_to_rows(x):
        """[B,H,S,D] -> [B,S,H*D]."""
        b, h, s, d = x.shape
        y = _empty((b, s, h * d), x.dtype, x)
        _call("hk_heads_to_rows", desc(x), desc(y))
        return y

    @staticmethod
    def rows_to_heads(x, heads: int):
        """[B,S,H*D] -> [B,H,S,D]."""
        b, s, w = x.shape
        y = _empty((b, heads, s, w // heads), x.dtype, x)
        _call("hk_rows_to_heads", desc(x), desc(y))
        return y

    @staticmethod
    def bias_add_backward(grad):
        """dbias = dY summed over the leading axes in the reference's pairwise order. Reference:
        AscendRuntime::bias_add_backward (mod.rs:182-185)."""
        db = _empty((grad.shape[-1],), torch.float32, grad)
        _call("hk_bias_add_backward", desc(grad), desc(db))
        return db

    # ---------------------------------------------------------------- embedding

    @staticmethod
    def nll_loss(input, target, weight, reduction=LossReduction.Mean, ignore_index=None):
        """[loss, total weight] from log-probabilities input [N, C], labels target [N] and class
        weights weight [C]; loss is [N] for None, [1] otherwise. Reference: AscendRuntime::nll_loss
        (mod.rs:226-228)."""
        red = LossReduction(reduction)
        rows = input.shape[0] if input.dim() == 2 else 0
        out = _empty((rows if red == LossReduction.None_ else 1,), input.dtype, input)
        total = _empty((1,), input.dtype, input)
        _call("hk_nll_loss", desc(input), desc(target), desc(weight), int(red), _ignore(ignore_index), desc(out),
              desc(total))
        return out, total

    @staticmethod
    def nll_loss_with_saved_inputs(input, target, weight, reduction=LossReduction.Mean, ignore_index=None):
        """[loss, total weight, saved labels, saved weights]: the forward plus independent device
        copies of the labels and weights. Reference: AscendRuntime::nll_loss_with_saved_inputs
        (mod.rs:229-231, runtime/loss.rs:21-26)."""
        t, w = target.clone(), weight.clone()
        out, total = HipRuntime.nll_loss(input, t, w, reduction, ignore_index)
        return out, total, t, w

    @staticmethod
    def nll_loss_backward(grad, input, target, weight, total_weight, reduction=LossReduction.Mean, ignore_index=None):
        """Dense derivative with respect to the log-probabilities. Reference:
        AscendRuntime::nll_loss_backward (mod.rs:232-236)."""
        dx = _empty(input.shape, input.dtype, input)
        _call("hk_nll_loss_backward", desc(grad), desc(input), desc(target), desc(weight), desc(total_weight),
              int(LossReduction(reduction)), _ignore(ignore_index), desc(dx))
        return dx

    @staticmethod
    def embedding(weight, ids):
        """weight[ids] -> [ids..., H]. Reference: AscendRuntime::embedding (mod.rs:237-241)."""
        out = _empty(tuple(ids.shape) + (weight.shape[1],), weight.dtype, weight)
        _call("hk_embedding", desc(weight), desc(ids), desc(out))
        return out

    @staticmethod
    def embedding_backward(grad, ids, num_weights: int, padding_idx=None, scale_grad_by_freq: bool = False):
        """Dense [num_weights, H] weight gradient. Reference: AscendRuntime::embedding_backward
        (mod.rs:252-256) with EmbeddingOptions {padding_idx, scale_grad_by_freq}."""
        if padding_idx is not None and (padding_idx < 0 or padding_idx >= num_weights):
            raise HkError(_lib.INVALID_ARGUMENT, "embedding padding index must be within the weight rows")
        dw = _empty((int(num_weights), grad.shape[-1]), grad.dtype, grad)
        _call("hk_embedding_backward", desc(grad), desc(ids), int(num_weights),
              NO_PADDING if padding_idx is None else int(padding_idx), int(bool(scale_grad_by_freq)), desc(dw))
        return dw

    # ---------------------------------------------------------------- composed-attention shims

    @staticmethod
    def causal_mask(batch: int, queries: int, keys: int, query_start: int = 0, key_start: int = 0, device=None):
        """F32 [B,Q,K] additive mask. Reference: AscendRuntime::causal_mask (mod.rs:205-206)."""
        out = torch.empty((batch, queries, keys), dtype=torch.float32, device=device or torch.device("cuda"))
        _call("hk_causal_mask", int(query_start), int(key_start), desc(out))
        return out

    @staticmethod
    def repeat_kv_heads(x, query_heads: int):
        """[B,Hkv,N,D] -> [B,Hq,N,D]. Reference: AscendRuntime::repeat_kv_heads (mod.rs:208-209)."""
        b, _, n, d = x.shape
        y = _empty((b, int(query_heads), n, d), x.dtype, x)
        _call("hk_repeat_kv_heads", desc(x), desc(y))
        return y

    @staticmethod
    def repeat_kv_heads_backward(input_shape, query_heads: int, grad):
        """dX [B,Hkv,N,D] from dY [B,Hq,N,D]. Reference: AscendRuntime::repeat_kv_heads_backward (mod.rs:210-213)."""
        if int(grad.shape[1]) != int(query_heads):
            raise ValueError("grad must have query_heads heads")
        dx = _empty(tuple(input_shape), grad.dtype, grad)
        _call("hk_repeat_kv_heads_backward", desc(grad), desc(dx))
        return dx

    # ---------------------------------------------------------------- RMSNorm

    # ---------------------------------------------------------------- softmax rows

    @staticmethod
    def softmax(x):
        """Row softmax over the last axis (F32). Reference: AscendRuntime::softmax (mod.rs:322-325)."""
        y = _empty(x.shape, x.dtype, x)
        _call("hk_softmax", desc(x), 0, desc(y))
        return y

    @staticmethod
    def log_softmax(x):
        """Reference: AscendRuntime::log_softmax (mod.rs:327-330)."""
        y = _empty(x.shape, x.dtype, x)
        _call("hk_softmax", desc(x), 1, desc(y))
        return y

    @staticmethod
    def softmax_backward(output, grad):
        """dX from the saved softmax output. Reference: AscendRuntime::softmax_backward (mod.rs:332-335)."""
        dx = _empty(output.shape, output.dtype, output)
        _call("hk_softmax_backward", desc(output), desc(grad), 0, desc(dx))
        return dx

    @staticmethod
    def log_softmax_backward(output, grad):
        """Reference: AscendRuntime::log_softmax_backward (mod.rs:338-341)."""
        dx = _empty(output.shape, output.dtype, output)
        _call("hk_softmax_backward", desc(output), desc(grad), 1, desc(dx))
        return dx

    # ---------------------------------------------------------------- RMSNorm

    @staticmethod
    def rms_norm(x, weight, epsilon: float):
        """[Y, rstd]. Reference: AscendRuntime::rms_norm (mod.rs:402-408); rstd has one F32 per row."""
        y = _empty(x.shape, x.dtype, x)
        rows = x.numel() // x.shape[-1] if x.dim() and x.shape[-1] else 0
        rstd = _empty((rows,), torch.float32, x)
        _call("hk_rms_norm", desc(x), desc(weight), float(epsilon), desc(y), desc(rstd))
        return y, rstd

    @staticmethod
    def rms_norm_backward(x, weight, grad, rstd):
        """[dX, F32 dW]. Reference: AscendRuntime::rms_norm_backward (mod.rs:410-415)."""
        dx = _empty(x.shape, x.dtype, x)
        dw = _empty((x.shape[-1],), torch.float32, x)
        _call("hk_rms_norm_backward", desc(x), desc(weight), desc(grad), desc(rstd), desc(dx), desc(dw))
        return dx, dw

    @staticmethod
    def rms_norm_backward_residual(x, weight, grad, rstd, residual):
        """[dX + residual, F32 dW] in one pass: the norm's backward with a residual branch's
        gradient added as dX is stored (hk_rms_norm_backward_residual)."""
        dx = _empty(x.shape, x.dtype, x)
        dw = _empty((x.shape[-1],), torch.float32, x)
        _call("hk_rms_norm_backward_residual", desc(x), desc(weight), desc(grad), desc(rstd), desc(residual),
              desc(dx), desc(dw))
        return dx, dw

    # ---------------------------------------------------------------- RoPE

    @staticmethod
    def rotary(x, cos, sin, layout=RotaryLayout.SplitHalf):
        """Reference: AscendRuntime::rotary (mod.rs:257-261)."""
        y = _empty(x.shape, x.dtype, x)
        _call("hk_rotary", desc(x), desc(cos), desc(sin), int(layout), desc(y))
        return y

    @staticmethod
    def rotary_backward(grad, cos, sin, layout=RotaryLayout.SplitHalf):
        """Reference: AscendRuntime::rotary_backward (mod.rs:264-268)."""
        dx = _empty(grad.shape, grad.dtype, grad)
        _call("hk_rotary_backward", desc(grad), desc(cos), desc(sin), int(layout), desc(dx))
        return dx

    @staticmethod
    def rotary_prefix(x, cos, sin, width: int, layout=RotaryLayout.SplitHalf):
        """Reference: AscendRuntime::rotary_prefix (mod.rs:214-217)."""
        y = _empty(x.shape, x.dtype, x)
        _call("hk_rotary_prefix", desc(x), desc(cos), desc(sin), int(width), int(layout), desc(y))
        return y

    @staticmethod
    def rotary_prefix_backward(grad, cos, sin, width: int, layout=RotaryLayout.SplitHalf):
        """Reference: AscendRuntime::rotary_prefix_backward (mod.rs:218-221)."""
        dx = _empty(grad.shape, grad.dtype, grad)
        _call("hk_rotary_prefix_backward", desc(grad), desc(cos), desc(sin), int(width), int(layout), desc(dx))
        return dx

    # ---------------------------------------------------------------- attention

    @staticmethod
    def attention_forward(q, k, v, scale: float, causal: bool = True, query_start: int = 0, key_start: int = 0,
                          out_dtype=torch.bfloat16):
        """Fused GQA attention forward: [O (out_dtype: BF16, or F32 for the reference's FP32
        surface), lse (F32 [B,Hq,M])]. Q/K/V all BF16 or all F32. Replaces the composed chain of
        src/nn/attention.rs:10-80."""
        o = _empty(q.shape, out_dtype, q)
        lse = _empty(q.shape[:3], torch.float32, q)
        _call("hk_attention_forward", desc(q), desc(k), desc(v), float(scale), int(bool(causal)), int(query_start),
              int(key_start), desc(o), desc(lse))
        return o, lse

    @staticmethod
    def attention_backward(q, k, v, o, lse, grad, scale: float, causal: bool = True, query_start: int = 0,
                           key_start: int = 0, grad_dtype=torch.float32):
        """[dQ, dK, dV] of the fused GQA attention (dK/dV summed over each KV group)."""
        dq = _empty(q.shape, grad_dtype, q)
        dk = _empty(k.shape, grad_dtype, q)
        dv = _empty(v.shape, grad_dtype, q)
        _call("hk_attention_backward", desc(q), desc(k), desc(v), desc(o), desc(lse), desc(grad), float(scale),
              int(bool(causal)), int(query_start), int(key_start), desc(dq), desc(dk), desc(dv))
        return dq, dk, dv

    @staticmethod
    def attention_masked_forward(q, k, v, scale: float, mask=None, out_dtype=torch.float32):
        """The reference's materialized attention with an optional additive F32 mask: rank 3
        (scaled_dot_product_attention_bf16_fp32) or rank 4 (grouped_query_attention_bf16_fp32),
        any value width (src/nn/attention.rs:10-67). Returns O [.., M, Dv]."""
        o = _empty(tuple(q.shape[:-1]) + (v.shape[-1],), out_dtype, q)
        _call("hk_attention_masked_forward", desc(q), desc(k), desc(v), float(scale),
              None if mask is None else desc(mask), desc(o))
        return o

    @staticmethod
    def attention_masked_backward(q, k, v, mask, grad, scale: float, grad_dtype=torch.float32, mask_grad=False):
        """[dQ, dK, dV, dMask or None] of attention_masked_forward; dMask = dS (F32, the mask's
        shape) when mask_grad is set."""
        dq = _empty(q.shape, grad_dtype, q)
        dk = _empty(k.shape, grad_dtype, q)
        dv = _empty(v.shape, grad_dtype, q)
        dmask = _empty(mask.shape, torch.float32, q) if mask_grad else None
        _call("hk_attention_masked_backward", desc(q), desc(k), desc(v), None if mask is None else desc(mask),
              desc(grad), float(scale), desc(dq), desc(dk), desc(dv), None if dmask is None else desc(dmask))
        return dq, dk, dv, dmask
