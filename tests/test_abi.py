"""The C-ABI library loads and exports every declared symbol, and rejects
bad arguments on the host with an mlxr-style error (no GPU needed: every
call here fails validation before touching the device)."""
import ctypes
import re
import threading
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "mlxr_moe.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mlxr_moe_\w+)\s*\(", text)))


def test_header_declares_the_boundary():
    syms = declared_symbols()
    for s in ["mlxr_moe_gather_qmm", "mlxr_moe_quantize", "mlxr_moe_dequantize",
              "mlxr_moe_argpartition", "mlxr_moe_router_topk", "mlxr_moe_dispatch",
              "mlxr_moe_combine", "mlxr_moe_switch_glu_forward", "mlxr_moe_block_forward",
              "mlxr_moe_last_error"]:
        assert s in syms


def test_library_exports_every_declared_symbol(pkg):
    lib = ctypes.CDLL(str(pkg.LIB_PATH))
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing
    assert sorted(pkg._capi.SIGNATURES) == declared_symbols()
    assert pkg._capi.lib().mlxr_moe_version() == 301


def _err(pkg):
    return pkg._capi.last_error()


def test_quantize_rejects_bad_bits_group_mode(pkg):
    lib, C = pkg._capi.lib(), pkg._capi
    OI = C.OptionalInt
    assert lib.mlxr_moe_quantize(None, C.BFLOAT16, 4, 64, OI.of(64), OI.of(3), b"affine",
                                 None, None, None, None) == -1
    assert "bits" in _err(pkg)
    assert lib.mlxr_moe_quantize(None, C.BFLOAT16, 4, 64, OI.of(48), OI.of(4), b"affine",
                                 None, None, None, None) == -1
    assert "group_size" in _err(pkg)
    assert lib.mlxr_moe_quantize(None, C.BFLOAT16, 4, 100, OI.of(None), OI.of(None), None,
                                 None, None, None, None) == -1
    assert "multiple of group_size 64" in _err(pkg)
    assert lib.mlxr_moe_quantize(None, C.BFLOAT16, 4, 64, OI.of(64), OI.of(4), b"mxfp4",
                                 None, None, None, None) == -1
    assert "mode" in _err(pkg)


def test_gather_qmm_rejects_unsupported(pkg):
    lib, C = pkg._capi.lib(), pkg._capi
    OI = C.OptionalInt
    args = lambda gs, bits, transpose: (  # noqa: E731
        None, C.BFLOAT16, 1, 1, 128, None, None, None, C.BFLOAT16, 4, 64, None, None, 1,
        transpose, OI.of(gs), OI.of(bits), b"affine", 0, None, C.BFLOAT16, None, 0, None)
    assert lib.mlxr_moe_gather_qmm(*args(32, 4, 1)) == -1
    assert "group_size must be 64" in _err(pkg)
    assert lib.mlxr_moe_gather_qmm(*args(64, 2, 1)) == -1
    assert "bits must be 4 or 8" in _err(pkg)
    assert lib.mlxr_moe_gather_qmm(*args(64, 4, 0)) == -1
    assert "transpose" in _err(pkg)


def test_argpartition_invalid_axis_and_kth(pkg):
    """crates/mlxr/src/ops/sort.rs:262-301: invalid axis / kth must error."""
    lib = pkg._capi.lib()
    assert lib.mlxr_moe_argpartition(None, 1, 5, 2, 2, None, None) == -1
    assert "axis" in _err(pkg)
    assert lib.mlxr_moe_argpartition(None, 1, 5, 5, 0 - 1, None, None) == -1
    assert "kth" in _err(pkg)
    assert lib.mlxr_moe_argpartition(None, 1, 5, -6, -1, None, None) == -1


def test_block_validation(pkg):
    C = pkg._capi
    lib = C.lib()
    blk = C.Block()
    blk.hidden_size, blk.num_experts, blk.num_experts_per_tok = 2048, 128, 0
    blk.moe_intermediate_size = 768
    assert lib.mlxr_moe_block_forward(ctypes.byref(blk), None, 1, None, None, None, None, 0,
                                      None) == -1
    assert "num_experts_per_tok" in _err(pkg)
    blk.num_experts_per_tok = 8
    assert lib.mlxr_moe_block_forward(ctypes.byref(blk), None, 1, None, None, None, None, 0,
                                      None) == -1
    assert "gate_weight" in _err(pkg)
    # a quantised router replaces the f32 one and must be 4/8-bit, group 64
    blk.gate_q = C.QLinear(1, 1, 1, 1, 128, 2048, 64, 3)
    assert lib.mlxr_moe_block_forward(ctypes.byref(blk), None, 1, None, None, None, None, 0,
                                      None) == -1
    assert "gate_q must be 4- or 8-bit" in _err(pkg)
    blk.gate_q = C.QLinear(4, 4, 4, 1, 64, 2048, 64, 8)
    assert lib.mlxr_moe_block_forward(ctypes.byref(blk), None, 1, None, None, None, None, 0,
                                      None) == -1
    assert "[num_experts, hidden_size]" in _err(pkg)
    blk.gate_q = C.QLinear(4, 4, 4, 1, 128, 2048, 64, 8)
    blk.gate_weight = 16
    assert lib.mlxr_moe_block_forward(ctypes.byref(blk), None, 1, None, None, None, None, 0,
                                      None) == -1
    assert "replaces gate_weight" in _err(pkg)


def test_router_topk_quantized_validation(pkg):
    C = pkg._capi
    lib = C.lib()
    g = C.QLinear(4, 4, 4, 1, 128, 2048, 64, 2)
    assert lib.mlxr_moe_router_topk_quantized(None, 1, ctypes.byref(g), 8, None, None, None,
                                              0, None) == -1
    assert "bits must be 4 or 8" in _err(pkg)
    g.bits, g.input_dims = 8, 2000
    assert lib.mlxr_moe_router_topk_quantized(None, 1, ctypes.byref(g), 8, None, None, None,
                                              0, None) == -1
    assert "multiple of 64" in _err(pkg)
    g.input_dims = 2048
    assert lib.mlxr_moe_router_topk_quantized(None, 1, ctypes.byref(g), 200, None, None, None,
                                              0, None) == -1
    assert "k must be" in _err(pkg)


def test_last_error_is_thread_local(pkg):
    lib = pkg._capi.lib()
    assert lib.mlxr_moe_argpartition(None, 1, 5, 2, 7, None, None) == -1
    seen = {}

    def other():
        seen["msg"] = pkg._capi.last_error()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["msg"] == ""
    assert "axis" in _err(pkg)


def test_python_mirror_axis_errors_without_gpu(pkg):
    torch = pytest.importorskip("torch")
    a = torch.zeros(5)
    with pytest.raises(pkg.MlxrMoeError):
        pkg.ops.argpartition_axis(a, 2, 1)


def test_gather_mm_rejects_unsupported(pkg):
    """gather_mm: only the [E, N, K] storage of SwitchLinear's weight, bf16
    operands, K and N multiples of 64; errors before any device work."""
    lib, C = pkg._capi.lib(), pkg._capi

    def call(a_dt=C.BFLOAT16, b_dt=C.BFLOAT16, K=128, N=64, bt=1, rhs=None):
        return lib.mlxr_moe_gather_mm(None, a_dt, 1, 1, K, None, b_dt, 4, N, bt, None, rhs, 1,
                                      0, None, C.BFLOAT16, None, 0, None)

    assert call(bt=0) == -1 and "b_transposed" in _err(pkg)
    assert call(b_dt=C.FLOAT32) == -1 and "bf16" in _err(pkg)
    assert call() == -1 and "rhs_indices" in _err(pkg)
    assert lib.mlxr_moe_gather_mm(None, C.BFLOAT16, 1, 1, 128, None, C.BFLOAT16, 4, 64, 1, None,
                                  None, 0, 0, None, C.BFLOAT16, None, 0, None) == -1
    assert "workspace" in _err(pkg)  # B = 0 needs no indices, only the (small) workspace
    assert call(K=96, rhs=8) == -1 and "multiples of 64" in _err(pkg)
    assert call(K=8192, rhs=8) == -1 and "K above" in _err(pkg)
    assert lib.mlxr_moe_gather_mm_workspace_size(8, 1, 4) == \
        lib.mlxr_moe_gather_qmm_workspace_size(8, 1, 4)


def test_dense_linear_descriptors_validation(pkg):
    """bits 16 marks a dense bf16 SwitchLinear / Linear: it takes no scales
    or biases, in the router entry and in the expert modules alike."""
    C = pkg._capi
    lib = C.lib()
    g = C.QLinear(16, 16, None, 1, 128, 2048, 0, 16)
    assert lib.mlxr_moe_router_topk_quantized(None, 1, ctypes.byref(g), 8, None, None, None,
                                              0, None) == -1
    assert "no scales" in _err(pkg)
    dense = C.QLinear(16, None, None, 8, 256, 512, 0, 16)
    with_scales = C.QLinear(16, 16, 16, 8, 256, 512, 0, 16)
    down = C.QLinear(16, None, None, 8, 512, 256, 0, 16)
    ffn = C.SwitchGlu(dense, with_scales, down)
    assert lib.mlxr_moe_switch_glu_forward(ctypes.byref(ffn), None, 1, None, None, 2, None,
                                           None, 0, None) == -1
    assert "dense (bits 16) weight takes no scales" in _err(pkg)
    mixed = C.SwitchGlu(dense, dense, C.QLinear(16, 16, 16, 8, 512, 256, 64, 4))
    assert lib.mlxr_moe_switch_glu_forward(ctypes.byref(mixed), None, 1, None, None, 2, None,
                                           None, 0, None) == -1
    assert "share bits" in _err(pkg)


def test_profile_read_validation(pkg):
    lib, C = pkg._capi.lib(), pkg._capi
    assert lib.mlxr_moe_profile_read(None, 1024, None, None) == -1
    assert "buf and sink" in _err(pkg)
    # a size that is not whole 16-byte vectors, an unaligned buffer
    assert lib.mlxr_moe_profile_read(16, 1000, 16, None) == -1
    assert "multiple of 16" in _err(pkg)
    assert lib.mlxr_moe_profile_read(8, 1024, 16, None) == -1
    assert "aligned" in _err(pkg)


def test_router_matrix_order_rule(pkg):
    """The router's summation order (host logic, no GPU): the matrix-core
    order from 512 tokens with d a multiple of 256 and at least 192 tiles of
    32 tokens x 32 logit columns, else the lane order; negative sizes
    rejected."""
    q = pkg._capi.lib().mlxr_moe_router_matrix_order
    assert q(1, 2048, 128) == 0 and q(300, 4096, 1024) == 0 and q(511, 2048, 1024) == 0
    # tiles: 4 x 64, 4 x 128, 4 x 512, 4 x 48 (the fewest taken)
    assert q(2048, 2048, 128) == 1 and q(4096, 2048, 128) == 1
    assert q(16384, 256, 128) == 1 and q(1536, 2048, 128) == 1
    # 4 x 32, 2 x 64, 4 x 47: too few tiles
    assert q(1024, 2048, 128) == 0 and q(2048, 2048, 64) == 0 and q(1504, 2048, 128) == 0
    # a shared-expert gate's column adds a column of tiles: 9 x 32, 17 x 16
    assert q(1024, 2048, 257) == 1 and q(512, 2048, 513) == 1 and q(1024, 2048, 256) == 1
    assert q(1024, 2048, 160) == 0 and q(1024, 2048, 161) == 1  # 5 x 32 / 6 x 32
    assert q(4096, 2052, 128) == 0 and q(4096, 320, 128) == 0 and q(4096, 64, 128) == 0
    assert q(-1, 64, 8) == -1 and q(64, -1, 8) == -1 and q(64, 64, -1) == -1
    assert pkg.ops.router_matrix_order(4096, 2048, 128) is True
    assert pkg.ops.router_matrix_order(1024, 2048, 128) is False
