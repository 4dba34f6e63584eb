"""DeepGemm: the reference's native GEMM provider over its ahead-of-time device programs
(rust-ascend-driver/src/tensor/deepgemm/mod.rs:18-145), here over libhk.so's code-object ABI.

The 18 programs ``ruda_rust_bf16_{dense,batched}_{n,t}{n,t}_{bf16,f32}`` and
``ruda_rust_bf16_mgrouped_nt_{bf16,f32}`` sit in one gfx950 code object
(``rust-ascend_amd/lib/hk_programs.hsaco``). ``DeepGemm(path)`` loads it
(``hk_module_load_data``; the reference's ``DeepGemm::load`` + ``Kernel::load``), ``prepare`` looks a
program up once per key (``hk_module_get_function``), and every call packs the reference's nine
arguments -- three ``hk_gm`` (RudaGm), M, N, K, the group-end pointer, the batch/group count and the
epilogue -- exactly as ``DeepGemm::execute_addresses`` does (mod.rs:122-132), then launches them with
``hk_launch_kernel_with_args`` (``aclrtLaunchKernelWithArgsArray``). Contract checks: the host-side
plan (``GemmSpec``, plan.rs:49-80) before any device work, then libhk.so's launch checks.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import HkEpilogue, HkError, HkGm
from .runtime import DeviceGroupEnds, Transpose, _call, gemm_plan, grouped_gemm_plan

_OUT = {torch.bfloat16: "bf16", torch.float32: "f32"}


class DeepGemm:
    """Reference: DeepGemm (deepgemm/mod.rs:18-145). Not thread-safe, like the reference's."""

    def __init__(self, path: str = _lib.PROGRAMS_PATH):
        """Reference: DeepGemm::load (mod.rs:26-35): the code object is read once and loaded."""
        with open(path, "rb") as f:
            data = f.read()
        self._image = ctypes.create_string_buffer(data, len(data))
        h = ctypes.c_void_p()
        _call("hk_module_load_data", self._image, len(data), ctypes.byref(h))
        self._module = h
        self._functions: dict[str, ctypes.c_void_p] = {}
        self._stats = {"modules_loaded": 0, "launches": 0, "synchronizations": 0}

    # ---------------------------------------------------------------- provider

    def stats(self) -> dict:
        """Reference: KernelStats (mod.rs:15-16): programs prepared, launches, synchronizations."""
        return dict(self._stats)

    def prepare(self, key: str):
        """Look the program for GemmSpec::key `key` up once (mod.rs:38-49)."""
        if self._module is None:
            raise HkError(_lib.INVALID_ARGUMENT, "DeepGemm provider is closed")
        fn = self._functions.get(key)
        if fn is None:
            fn = ctypes.c_void_p()
            _call("hk_module_get_function", self._module, ("ruda_rust_" + key).encode(), ctypes.byref(fn))
            self._functions[key] = fn
            self._stats["modules_loaded"] += 1
        return fn

    def close(self) -> None:
        """Unload the code object after queued work completes (Drop for Kernel, native.rs:66-76)."""
        if self._module is not None:
            _call("hk_module_unload", self._module)
            self._module = None
            self._functions.clear()

    # ---------------------------------------------------------------- GEMM

    def gemm(self, a, b, ta=Transpose.No, tb=Transpose.No, dtype=torch.bfloat16):
        """New output. Reference: DeepGemm::gemm (mod.rs:51-57)."""
        plan = gemm_plan(a.shape, b.shape, ta, tb, dtype, a.dtype, b.dtype)
        out = torch.empty(plan["out_shape"], dtype=dtype, device=a.device)
        self._run(plan, int(ta), int(tb), a, b, out, None)
        return out

    def gemm_into(self, a, b, ta, tb, out) -> None:
        """Reference: DeepGemm::gemm_into (mod.rs:58-61)."""
        plan = gemm_plan(a.shape, b.shape, ta, tb, out.dtype, a.dtype, b.dtype)
        self._check_out(plan, out)
        self._run(plan, int(ta), int(tb), a, b, out, None)

    def upload_group_ends(self, ends) -> DeviceGroupEnds:
        """Reference: DeepGemm::upload_group_ends (mod.rs:63-67)."""
        return DeviceGroupEnds(ends)

    def grouped_nt(self, a, weights, groups: DeviceGroupEnds, dtype=torch.bfloat16):
        """Reference: DeepGemm::grouped_nt (mod.rs:68-73)."""
        plan = grouped_gemm_plan(a.shape, weights.shape, groups.ends, dtype, a.dtype, weights.dtype)
        out = torch.empty(plan["out_shape"], dtype=dtype, device=a.device)
        self._run(plan, 0, 1, a, weights, out, groups)
        return out

    def grouped_nt_into(self, a, weights, groups: DeviceGroupEnds, out) -> None:
        """Reference: DeepGemm::grouped_nt_into (mod.rs:74-78)."""
        plan = grouped_gemm_plan(a.shape, weights.shape, groups.ends, out.dtype, a.dtype, weights.dtype)
        self._check_out(plan, out)
        self._run(plan, 0, 1, a, weights, out, groups)

    def linear_nt_backward(self, x, w, dy):
        """[BF16 dX, F32 dW] for Y = X W^T: dX = dY W, dW = dY^T X. Reference:
        DeepGemm::linear_nt_backward (mod.rs:82-92)."""
        fwd = gemm_plan(x.shape, w.shape, Transpose.No, Transpose.Yes, torch.bfloat16, x.dtype, w.dtype)
        if fwd["kind"] != "dense" or dy.dtype != torch.bfloat16 or tuple(dy.shape) != fwd["out_shape"]:
            raise HkError(_lib.INVALID_ARGUMENT, "linear backward requires dense BF16 dY matching X @ W^T")
        dx = self.gemm(dy, w, Transpose.No, Transpose.No, torch.bfloat16)
        dw = self.gemm(dy, x, Transpose.Yes, Transpose.No, torch.float32)
        return dx, dw

    # ---------------------------------------------------------------- launch

    @staticmethod
    def _check_out(plan, out) -> None:
        if tuple(out.shape) != tuple(plan["out_shape"]) or not out.is_contiguous():
            raise HkError(_lib.INVALID_ARGUMENT, "native GEMM tensor layout mismatch")

    def _run(self, plan, ta: int, tb: int, a, b, out, groups) -> None:
        """Pack the nine arguments as DeepGemm::execute_addresses does (mod.rs:122-132) and launch
        them on 32 blocks (the reference's core count; libhk.so sizes the grid from the shape)."""
        for name, t in (("A", a), ("B", b), ("D", out)):
            if not t.is_cuda or not t.is_contiguous():
                raise HkError(_lib.INVALID_ARGUMENT, f"{name} must be a contiguous GPU tensor")
        if out.dtype not in _OUT or a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16:
            raise HkError(_lib.INVALID_ARGUMENT, "native DeepGEMM accepts BF16 inputs and BF16/F32 output only")
        fn = self.prepare(plan["key"])
        m, n, k = int(plan["m"]), int(plan["n"]), int(plan["k"])
        kind = plan["kind"]
        batched = kind == "batched"
        ga = HkGm(a.data_ptr(), a.shape[-1], m * k if batched else 0)
        gb = HkGm(b.data_ptr(), b.shape[-1], n * k if batched else 0)
        gd = HkGm(out.data_ptr(), n, m * n if batched else 0)
        ends_ptr = ctypes.c_void_p(None)
        if kind == "mgrouped":
            _call("hk_group_ends_data", groups.handle, ctypes.byref(ends_ptr))
            count = len(groups.ends)
        else:
            count = int(plan["batch"]) if batched else 0
        cm, cn, ck, cg = (ctypes.c_uint32(x) for x in (m, n, k, count))
        ep = HkEpilogue(1.0, 0, 0, 0, n, 0)
        argv = (ctypes.c_void_p * 9)(*(ctypes.cast(ctypes.byref(x), ctypes.c_void_p)
                                       for x in (ga, gb, gd, cm, cn, ck, ends_ptr, cg, ep)))
        _call("hk_launch_kernel_with_args", fn, 32, argv)
        self._stats["launches"] += 1
        self._stats["synchronizations"] += 1
