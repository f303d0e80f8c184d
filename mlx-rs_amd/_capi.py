"""ctypes binding of libmlxr_moe.so (declarations in include/mlxr_moe.h).

Loading fails loudly when the library is missing: there is no CPU
fallback behind these functions.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import (POINTER, Structure, c_char_p, c_double, c_float, c_int, c_int32, c_int64,
                    c_size_t, c_void_p)
from pathlib import Path

# MLXR_MOE_LIB: another build of the same sources (e.g. a host-sanitizer copy)
LIB_PATH = Path(os.environ.get("MLXR_MOE_LIB", Path(__file__).resolve().parent / "libmlxr_moe.so"))

FLOAT32 = 0
BFLOAT16 = 1


class MlxrMoeError(RuntimeError):
    """An entry point returned a nonzero status (mlxr's Exception)."""


class OptionalInt(Structure):
    _fields_ = [("value", c_int32), ("has_value", c_int32)]

    @classmethod
    def of(cls, v):
        return cls(0, 0) if v is None else cls(int(v), 1)


class QLinear(Structure):
    _fields_ = [
        ("weight", c_void_p),
        ("scales", c_void_p),
        ("biases", c_void_p),
        ("num_experts", c_int64),
        ("output_dims", c_int64),
        ("input_dims", c_int64),
        ("group_size", c_int32),
        ("bits", c_int32),
    ]


class SwitchGlu(Structure):
    _fields_ = [("gate_proj", QLinear), ("up_proj", QLinear), ("down_proj", QLinear)]


class PackedSwitchGlu(Structure):
    _fields_ = [("gate_up_proj", QLinear), ("down_proj", QLinear), ("activation", c_int32)]


class GemmaRouter(Structure):
    _fields_ = [
        ("hidden_size", c_int64),
        ("num_experts", c_int64),
        ("top_k", c_int64),
        ("eps", c_float),
        ("norm_weight", c_void_p),
        ("proj_weight", c_void_p),
        ("proj_q", QLinear),
        ("per_expert_scale", c_void_p),
    ]


ACT_SWIGLU, ACT_GEGLU = 0, 1


class Block(Structure):
    _fields_ = [
        ("hidden_size", c_int64),
        ("num_experts", c_int64),
        ("num_experts_per_tok", c_int64),
        ("moe_intermediate_size", c_int64),
        ("shared_expert_intermediate_size", c_int64),
        ("gate_weight", c_void_p),
        ("gate_bias", c_void_p),
        ("switch_mlp", SwitchGlu),
        ("shared_gate_proj", QLinear),
        ("shared_up_proj", QLinear),
        ("shared_down_proj", QLinear),
        ("shared_expert_gate_weight", c_void_p),
        ("gate_q", QLinear),
        ("shared_expert_gate_q", QLinear),
    ]


P = c_void_p
OI = OptionalInt
# name -> (restype, argtypes); the exact set of symbols include/mlxr_moe.h
# declares.
SIGNATURES = {
    "mlxr_moe_last_error": (c_char_p, []),
    "mlxr_moe_version": (c_int, []),
    "mlxr_moe_quantize": (c_int, [P, c_int, c_int64, c_int64, OI, OI, c_char_p, P, P, P, P]),
    "mlxr_moe_dequantize": (c_int, [P, P, P, c_int, c_int64, c_int64, OI, OI, c_char_p, P, c_int, P]),
    "mlxr_moe_gather_qmm_workspace_size": (c_size_t, [c_int64, c_int64, c_int64]),
    "mlxr_moe_gather_qmm": (
        c_int,
        [P, c_int, c_int64, c_int64, c_int64, P, P, P, c_int, c_int64, c_int64, P, P, c_int64,
         c_int, OI, OI, c_char_p, c_int, P, c_int, P, c_size_t, P],
    ),
    "mlxr_moe_gather_mm_workspace_size": (c_size_t, [c_int64, c_int64, c_int64]),
    "mlxr_moe_gather_mm": (
        c_int,
        [P, c_int, c_int64, c_int64, c_int64, P, c_int, c_int64, c_int64, c_int, P, P, c_int64,
         c_int, P, c_int, P, c_size_t, P],
    ),
    "mlxr_moe_argpartition": (c_int, [P, c_int64, c_int64, c_int, c_int, P, P]),
    "mlxr_moe_softmax": (c_int, [P, c_int64, c_int64, c_int, c_int, P, P]),
    "mlxr_moe_router_workspace_size": (c_size_t, [c_int64, c_int64]),
    "mlxr_moe_router_topk": (c_int, [P, c_int64, c_int64, P, c_int64, c_int64, P, P, P, c_size_t, P]),
    "mlxr_moe_router_topk_quantized": (
        c_int, [P, c_int64, POINTER(QLinear), c_int64, P, P, P, c_size_t, P]),
    "mlxr_moe_dispatch_workspace_size": (c_size_t, [c_int64, c_int64]),
    "mlxr_moe_dispatch": (c_int, [P, c_int64, c_int64, P, P, P, P, P, c_size_t, P]),
    "mlxr_moe_combine": (c_int, [P, P, c_int64, c_int64, c_int64, P, P, P, P]),
    "mlxr_moe_switch_glu_workspace_size": (c_size_t, [POINTER(SwitchGlu), c_int64, c_int64]),
    "mlxr_moe_switch_glu_forward": (
        c_int, [POINTER(SwitchGlu), P, c_int64, P, P, c_int64, P, P, c_size_t, P]),
    "mlxr_moe_switch_glu_experts": (
        c_int, [POINTER(SwitchGlu), P, c_int64, P, c_int64, P, P, c_size_t, P]),
    "mlxr_moe_packed_switch_glu_workspace_size": (
        c_size_t, [POINTER(PackedSwitchGlu), c_int64, c_int64]),
    "mlxr_moe_packed_switch_glu_forward": (
        c_int, [POINTER(PackedSwitchGlu), P, c_int64, P, P, c_int, c_int64, P, P, c_size_t, P]),
    "mlxr_moe_packed_switch_glu_experts": (
        c_int, [POINTER(PackedSwitchGlu), P, c_int64, P, c_int64, P, P, c_size_t, P]),
    "mlxr_moe_gemma_router_workspace_size": (c_size_t, [POINTER(GemmaRouter), c_int64]),
    "mlxr_moe_gemma_router_forward": (
        c_int, [POINTER(GemmaRouter), P, c_int64, P, P, P, c_size_t, P]),
    "mlxr_moe_block_workspace_size": (c_size_t, [POINTER(Block), c_int64]),
    "mlxr_moe_block_forward": (c_int, [POINTER(Block), P, c_int64, P, P, P, P, c_size_t, P]),
    "mlxr_moe_rms_norm": (c_int, [P, c_int64, c_int64, P, c_float, P, P]),
    "mlxr_moe_block_residual_workspace_size": (c_size_t, [POINTER(Block), c_int64]),
    "mlxr_moe_block_forward_residual": (
        c_int, [POINTER(Block), P, c_float, P, c_int64, P, P, P, P, c_size_t, P]),
    "mlxr_moe_workspace_status": (c_int, [P, c_size_t, P]),
    "mlxr_moe_noalloc_scratch_size": (c_size_t, []),
    "mlxr_moe_block_forward_noalloc": (c_int, [POINTER(Block), P, c_int64, P, P, P, P]),
    "mlxr_moe_gather_qmm_tiled": (c_int, [c_int64, c_int64]),
    "mlxr_moe_router_matrix_order": (c_int, [c_int64, c_int64, c_int64]),
    "mlxr_moe_profile_start": (c_int, [c_char_p]),
    "mlxr_moe_profile_read": (c_int, [P, c_size_t, P, P]),
    "mlxr_moe_profile_stop": (c_int, [POINTER(c_int64), POINTER(c_double), POINTER(c_double),
                                      POINTER(c_double)]),
}

_lib = None


def lib() -> ctypes.CDLL:
    """The loaded library with typed entry points (loaded once)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise MlxrMoeError(
                f"{LIB_PATH} is missing: build it with `python mlx-rs_amd/build.py` "
                "(or __graft_entry__.build()); there is no fallback implementation")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        raise MlxrMoeError(lib().mlxr_moe_last_error().decode())


def last_error() -> str:
    return lib().mlxr_moe_last_error().decode()
