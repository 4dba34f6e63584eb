"""ctypes binding of libhk.so (the C ABI declared in include/hk.h).

The library is loaded from ``rust-ascend_amd/lib/libhk.so`` inside this repository (built by
``__graft_entry__.build()`` or ``make -C rust-ascend_amd/csrc``). A missing library is an error:
there is no CPU fallback, as in the reference (rust-ascend-driver/src/tensor/deepgemm/mod.rs:1-3).
"""
from __future__ import annotations

import ctypes
import os
import threading

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.normpath(os.path.join(_PKG, "..", "lib", "libhk.so"))
HEADER_PATH = os.path.normpath(os.path.join(_PKG, "..", "..", "include", "hk.h"))
# the GEMM device programs' code object (built with libhk.so, loaded by hk_module_load_data)
PROGRAMS_PATH = os.path.normpath(os.path.join(_PKG, "..", "lib", "hk_programs.hsaco"))

# Status codes (hk_status) and their reference counterparts (CannError, rust-ascend-driver/src/lib.rs:18-78).
OK, INVALID_ARGUMENT, HIP_ERROR, COMPLETION_ERROR, POISONED, NOT_INITIALIZED, LOAD_ERROR = range(7)
STATUS_NAMES = {OK: "OK", INVALID_ARGUMENT: "INVALID_ARGUMENT", HIP_ERROR: "HIP_ERROR",
                COMPLETION_ERROR: "COMPLETION_ERROR", POISONED: "POISONED",
                NOT_INITIALIZED: "NOT_INITIALIZED", LOAD_ERROR: "LOAD_ERROR"}

# Element type codes (reference DType codes, rust-ascend-driver/src/tensor/layout.rs:5-17).
F32, F16, BF16 = 0, 1, 27
I32, I64 = 3, 9
BOOL = 12
NO_PADDING = (1 << 64) - 1  # HK_NO_PADDING
MAX_RANK = 8


class HkError(RuntimeError):
    """A failed libhk.so call: `.status` is the hk_status code, the message is hk_last_error()."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status
        self.message = message


class HkTensor(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("dtype", ctypes.c_int32), ("rank", ctypes.c_int32),
                ("shape", ctypes.c_int64 * MAX_RANK)]


class HkStats(ctypes.Structure):
    _fields_ = [("modules_loaded", ctypes.c_uint64), ("launches", ctypes.c_uint64),
                ("synchronizations", ctypes.c_uint64)]


class HkGemmPlan(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int32), ("out_rank", ctypes.c_int32), ("batch", ctypes.c_int64),
                ("m", ctypes.c_int64), ("n", ctypes.c_int64), ("k", ctypes.c_int64),
                ("out_shape", ctypes.c_int64 * 3), ("key", ctypes.c_char * 32)]


class HkGm(ctypes.Structure):
    """hk_gm: the reference's RudaGm / GmPtr (deepgemm/native.rs:80-82), 24 bytes."""
    _fields_ = [("addr", ctypes.c_uint64), ("stride_outer", ctypes.c_uint64), ("stride_batch", ctypes.c_uint64)]


class HkEpilogue(ctypes.Structure):
    """hk_epilogue: the reference's RudaEpilogue / Epilogue (deepgemm/native.rs:83-85), 32 bytes."""
    _fields_ = [("alpha", ctypes.c_float), ("pad0", ctypes.c_uint32), ("sfd", ctypes.c_uint64),
                ("stride", ctypes.c_uint64), ("n", ctypes.c_uint32), ("pad1", ctypes.c_uint32)]


_T = ctypes.POINTER(HkTensor)
_CTX = ctypes.c_void_p
_i32 = ctypes.c_int32
_u64 = ctypes.c_uint64
_f32 = ctypes.c_float

# name -> argtypes (every function returns hk_status unless listed in _RESTYPE)
SIGNATURES = {
    "hk_init": [_i32, ctypes.POINTER(ctypes.c_void_p)],
    "hk_shutdown": [_CTX],
    "hk_set_stream": [_CTX, ctypes.c_void_p],
    "hk_get_stream": [_CTX],
    "hk_set_async": [_CTX, _i32],
    "hk_sync": [_CTX],
    "hk_get_stats": [_CTX, ctypes.POINTER(HkStats)],
    "hk_workspace_size": [_CTX, ctypes.POINTER(_u64)],
    "hk_trim_workspace": [_CTX, _u64],
    "hk_last_error": [],
    "hk_abi_version": [],
    "hk_alloc": [_CTX, ctypes.c_size_t, ctypes.POINTER(ctypes.c_void_p)],
    "hk_free": [_CTX, ctypes.c_void_p],
    "hk_upload": [_CTX, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t],
    "hk_download": [_CTX, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t],
    "hk_gemm_plan_check": [_T, _T, _i32, _i32, _i32, ctypes.POINTER(HkGemmPlan)],
    "hk_gemm_into": [_CTX, _T, _T, _i32, _i32, _T],
    "hk_group_ends_check": [ctypes.POINTER(_i32), _i32],
    "hk_group_ends_upload": [_CTX, ctypes.POINTER(_i32), _i32, ctypes.POINTER(ctypes.c_void_p)],
    "hk_group_ends_free": [_CTX, ctypes.c_void_p],
    "hk_group_ends_data": [_CTX, ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)],
    "hk_matmul_layout": [_T, _T, _T],
    "hk_tensor_matmul": [_CTX, _T, _T, _T],
    "hk_tensor_matmul_backward": [_CTX, _T, _T, _T, _T, _T],
    "hk_swap_last_dims": [_CTX, _T, _T],
    "hk_attention_scores": [_CTX, _T, _f32, _f32, _T, _T, _i32, _T],
    "hk_attention_scores_backward": [_CTX, _T, _T, _f32, _f32, _T, _i32, _T, _T],
    "hk_module_load_data": [_CTX, ctypes.c_void_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_void_p)],
    "hk_module_get_function": [_CTX, ctypes.c_void_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p)],
    "hk_launch_kernel_with_args": [_CTX, ctypes.c_void_p, ctypes.c_uint32, ctypes.POINTER(ctypes.c_void_p)],
    "hk_module_unload": [_CTX, ctypes.c_void_p],
    "hk_gemm_grouped_plan_check": [_T, _T, ctypes.POINTER(_i32), _i32, _i32, ctypes.POINTER(HkGemmPlan)],
    "hk_gemm_grouped_nt_into": [_CTX, _T, _T, ctypes.c_void_p, _T],
    "hk_linear_nt_backward": [_CTX, _T, _T, _T, _T, _T],
    "hk_gemm_bf16_fp32": [_CTX, _T, _T, _i32, _i32, _T, _T, _T],
    "hk_gemm_bf16_fp32_backward": [_CTX, _T, _T, _T, _i32, _i32, _T, _T],
    "hk_gemm_padded_bf16_fp32": [_CTX, _T, _T, _i32, _i32, _T, _T, _T],
    "hk_gemm_padded_bf16_fp32_backward": [_CTX, _T, _T, _T, _i32, _i32, _T, _T],
    "hk_linear_frozen_bf16_fp32": [_CTX, _T, _T, _T],
    "hk_linear_frozen_bf16_fp32_backward": [_CTX, _T, _T, _T],
    "hk_linear_frozen_padded_bf16_fp32": [_CTX, _T, _T, _T, _T],
    "hk_linear_frozen_padded_bf16_fp32_backward": [_CTX, _T, _T, _T],
    "hk_linear_bf16_fp32": [_CTX, _T, _T, _T, _T, _T],
    "hk_linear_bf16_fp32_backward": [_CTX, _T, _T, _T, _T, _T],
    "hk_cast_into": [_CTX, _T, _T],
    "hk_silu_mul": [_CTX, _T, _T, _T],
    "hk_silu_mul_backward": [_CTX, _T, _T, _T, _T, _T],
    "hk_bias_add": [_CTX, _T, _T, _T, _T],
    "hk_bias_add_backward": [_CTX, _T, _T],
    "hk_nll_loss": [_CTX, _T, _T, _T, _i32, ctypes.c_int64, _T, _T],
    "hk_nll_loss_backward": [_CTX, _T, _T, _T, _T, _T, _i32, ctypes.c_int64, _T],
    "hk_embedding": [_CTX, _T, _T, _T],
    "hk_embedding_backward": [_CTX, _T, _T, _u64, _u64, _i32, _T],
    "hk_qkv_rope_split": [_CTX, _T, _T, _T, _i32, _T, _T, _T],
    "hk_qkv_projection_rope": [_CTX, _T, _T, _T, _T, _i32, _T, _T, _T],
    "hk_linear_residual": [_CTX, _T, _T, _T, _T],
    "hk_swiglu_projection": [_CTX, _T, _T, _T, _T, _T],
    "hk_swiglu_projection_backward": [_CTX, _T, _T, _T, _T, _T],
    "hk_attention_backward_qkv_rows": [_CTX, _T, _T, _T, _T, _T, _T, _f32, _i32, _u64, _u64, _T, _T, _i32, _T],
    "hk_qkv_rope_merge": [_CTX, _T, _T, _T, _T, _T, _i32, _T],
    "hk_heads_to_rows": [_CTX, _T, _T],
    "hk_rows_to_heads": [_CTX, _T, _T],
    "hk_softmax": [_CTX, _T, _i32, _T],
    "hk_softmax_backward": [_CTX, _T, _T, _i32, _T],
    "hk_causal_mask": [_CTX, _u64, _u64, _T],
    "hk_repeat_kv_heads": [_CTX, _T, _T],
    "hk_repeat_kv_heads_backward": [_CTX, _T, _T],
    "hk_rms_norm": [_CTX, _T, _T, ctypes.c_double, _T, _T],
    "hk_rms_norm_backward": [_CTX, _T, _T, _T, _T, _T, _T],
    "hk_rms_norm_backward_noalloc": [_CTX, _T, _T, _T, _T, _T, _T],
    "hk_rms_norm_backward_residual": [_CTX, _T, _T, _T, _T, _T, _T, _T],
    "hk_rotary": [_CTX, _T, _T, _T, _i32, _T],
    "hk_rotary_backward": [_CTX, _T, _T, _T, _i32, _T],
    "hk_rotary_prefix": [_CTX, _T, _T, _T, _i32, _i32, _T],
    "hk_rotary_prefix_backward": [_CTX, _T, _T, _T, _i32, _i32, _T],
    "hk_attention_forward": [_CTX, _T, _T, _T, _f32, _i32, _u64, _u64, _T, _T],
    "hk_attention_backward": [_CTX, _T, _T, _T, _T, _T, _T, _f32, _i32, _u64, _u64, _T, _T, _T],
    "hk_attention_masked_forward": [_CTX, _T, _T, _T, _f32, _T, _T],
    "hk_attention_masked_backward": [_CTX, _T, _T, _T, _T, _T, _f32, _T, _T, _T, _T],
}
_RESTYPE = {"hk_last_error": ctypes.c_char_p, "hk_abi_version": ctypes.c_int32, "hk_get_stream": ctypes.c_void_p}

_lib = None
_lock = threading.Lock()


def load(path: str = None):
    """Load libhk.so (the module's LIB_PATH as it stands at the first call, or `path`) and bind
    every entry point; raises HkError(LOAD_ERROR) if absent."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if path is None:
            path = LIB_PATH
        if not os.path.exists(path):
            raise HkError(LOAD_ERROR, f"{path} is missing: build it with __graft_entry__.build() "
                                      "(no CPU fallback exists)")
        lib = ctypes.CDLL(path)
        for name, args in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = _RESTYPE.get(name, ctypes.c_int)
        _lib = lib
        return lib


def last_error() -> str:
    msg = load().hk_last_error()
    return msg.decode() if msg else ""


def check(status: int) -> None:
    if status != OK:
        raise HkError(status, last_error())


def tensor_desc(data_ptr: int, dtype: int, shape) -> HkTensor:
    shape = tuple(int(d) for d in shape)
    if len(shape) > MAX_RANK:
        raise HkError(INVALID_ARGUMENT, f"rank {len(shape)} exceeds {MAX_RANK}")
    t = HkTensor()
    t.data = int(data_ptr) if data_ptr else None
    t.dtype = int(dtype)
    t.rank = len(shape)
    for i, d in enumerate(shape):
        t.shape[i] = d
    return t
