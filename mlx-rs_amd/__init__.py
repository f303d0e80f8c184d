"""MI355X-native sparse-MoE block of mlxr-lm (router, dispatch, grouped
quantised expert GEMM, combine) behind the reference's op/module API.

The kernels live in libmlxr_moe.so (HIP, gfx950) behind the C ABI of
include/mlxr_moe.h.  This package is the Python view of that ABI:
    ops       gather_qmm / quantize / dequantize / argpartition_axis /
              softmax_axis / router_topk / dispatch / combine
    nn        QuantizedSwitchLinear / QuantizedLinear / SwigluMlp /
              SplitSwitchFfn / PackedSwitchFfn / Qwen35MoeBlock /
              GemmaRouter / GemmaMoe
    loader    one MoE layer of an mlxr checkpoint (safetensors) into nn
    workloads the benchmark configurations and seeded synthetic weights
"""
from . import _capi, loader, nn, ops, workloads
from ._capi import LIB_PATH, MlxrMoeError

__all__ = ["_capi", "loader", "nn", "ops", "workloads", "LIB_PATH", "MlxrMoeError"]
