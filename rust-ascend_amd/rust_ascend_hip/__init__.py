"""rust_ascend_hip — MI355X (gfx950) BF16 transformer kernel path, the drop-in counterpart of
rust-ascend's AscendRuntime / nn::* hot path, over libhk.so (include/hk.h)."""
from ._lib import HkError, LIB_PATH, load
from .runtime import (DeviceGroupEnds, HipRuntime, LossReduction, RotaryLayout, Transpose, check_group_ends, gemm_plan,
                      grouped_gemm_plan)
from .deepgemm import DeepGemm
from . import nn
from .decoder import DecoderConfig, DecoderLayer

__all__ = ["HkError", "LIB_PATH", "load", "HipRuntime", "RotaryLayout", "Transpose", "gemm_plan", "grouped_gemm_plan",
           "check_group_ends", "DeviceGroupEnds", "DeepGemm", "LossReduction", "nn", "DecoderConfig", "DecoderLayer"]
