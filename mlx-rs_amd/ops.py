"""mlxr ops on the MoE path, over the gfx950 C ABI.

Same names, argument meaning and error behaviour as the reference's Rust
op wrappers; torch tensors on a ROCm device stand in for mlx arrays (torch
is plumbing here: device memory and the current stream).  Every array op
runs a kernel of libmlxr_moe.so; there is no fallback.

    quantize          crates/mlxr/src/ops/quantization.rs:47-70
    dequantize        crates/mlxr/src/ops/quantization.rs:118-146
    gather_qmm        crates/mlxr/src/ops/quantization.rs:171-221
    argpartition_axis crates/mlxr/src/ops/sort.rs:211-226
    softmax_axis      crates/mlxr/src/ops/arithmetic.rs:1298-1311
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _capi as C
from ._capi import MlxrMoeError

DEFAULT_GROUP_SIZE = 64
DEFAULT_BITS = 4


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return C.FLOAT32
    if t.dtype == torch.bfloat16:
        return C.BFLOAT16
    raise MlxrMoeError(f"unsupported dtype {t.dtype} (float32 or bfloat16)")


def _dev(*ts):
    dev = None
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise MlxrMoeError("arrays must live on a ROCm device")
        if dev is not None and t.device != dev:
            raise MlxrMoeError("arrays live on different devices")
        dev = t.device
    return dev


def workspace(nbytes: int, device) -> torch.Tensor:
    """Device scratch for one call (torch's allocator aligns to 512 B)."""
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def _as_u32(idx: torch.Tensor) -> torch.Tensor:
    # mlx indices are uint32; int32 storage carries the same bits.
    if idx.dtype not in (torch.int32, torch.int64, torch.uint32):
        raise MlxrMoeError(f"indices must be integer, got {idx.dtype}")
    return idx.to(torch.int32).contiguous()


def _check_x_batch(name: str, x_batch_shape, idx_shape):
    """Without lhs indices the kernels take x's batch b as b // (B // x_batch)
    (B = the index count): right for x's batch shape equal to the index
    shape's leading axes followed by singletons (x [.., T, 1, 1, K] against
    indices [.., T, top_k], or one x batch for all).  Other broadcasts (a
    leading singleton against a larger index axis) would pick wrong rows:
    they are rejected."""
    xs = list(x_batch_shape)
    while len(xs) > len(idx_shape) and xs[0] == 1:
        xs.pop(0)
    ok = len(xs) <= len(idx_shape)
    if ok:
        pad = [1] * (len(idx_shape) - len(xs)) + xs
        j = 0
        while j < len(pad) and pad[j] == idx_shape[j]:
            j += 1
        ok = all(p == 1 for p in pad[j:])
    if not ok:
        raise MlxrMoeError(
            f"{name}: x batch shape {tuple(x_batch_shape)} must be the indices' leading axes "
            f"{tuple(idx_shape)} followed by singletons (or pass lhs_indices)")


def quantize(w: torch.Tensor, group_size=None, bits=None):
    """(w_q, scales, biases) of MLX affine quantisation along the last axis.
    w_q is int32 storage of mlx's uint32 words."""
    _dev(w)
    w = w.contiguous()
    gs = DEFAULT_GROUP_SIZE if group_size is None else group_size
    b = DEFAULT_BITS if bits is None else bits
    cols = w.shape[-1]
    rows = w.numel() // cols if cols else 0
    lead = tuple(w.shape[:-1])
    if b in (2, 4, 8) and cols * b % 32 == 0 and gs and cols % gs == 0:
        wq = torch.empty(lead + (cols * b // 32,), dtype=torch.int32, device=w.device)
        sc = torch.empty(lead + (cols // gs,), dtype=w.dtype, device=w.device)
        bi = torch.empty_like(sc)
    else:  # let the library produce the error message
        wq = sc = bi = torch.empty(1, device=w.device)
    C.check(C.lib().mlxr_moe_quantize(
        _p(w), _code(w), rows, cols, C.OptionalInt.of(group_size), C.OptionalInt.of(bits),
        b"affine", _p(wq), _p(sc), _p(bi), _stream(w)))
    return wq, sc, bi


def dequantize(w: torch.Tensor, scales: torch.Tensor, biases=None, group_size=None,
               bits=None, out_dtype=None):
    """code * scale + bias (one fused multiply-add, rounded once) in scales'
    dtype unless out_dtype is given."""
    _dev(w, scales, biases)
    b = DEFAULT_BITS if bits is None else bits
    cols = w.shape[-1] * 32 // b
    rows = w.numel() // w.shape[-1]
    out_dtype = out_dtype or scales.dtype
    out = torch.empty(tuple(w.shape[:-1]) + (cols,), dtype=out_dtype, device=w.device)
    C.check(C.lib().mlxr_moe_dequantize(
        _p(w.contiguous()), _p(scales.contiguous()),
        _p(None if biases is None else biases.contiguous()), _code(scales), rows, cols,
        C.OptionalInt.of(group_size), C.OptionalInt.of(bits), b"affine", _p(out),
        _code(out), _stream(w)))
    return out


def gather_qmm(x, w, scales, biases=None, lhs_indices=None, rhs_indices=None,
               transpose=True, group_size=None, bits=None, sorted_indices=False):
    """out[b] = x[xb(b)] @ dequant(w[rhs_indices[b]])^T.

    x [..., M, K] bf16; w [E, N, K*bits/32]; output rhs_indices.shape +
    [M, N].  Without lhs_indices, x's batch broadcasts over the trailing
    index axis (x [.., T, 1, 1, K] against indices [.., T, top_k])."""
    if rhs_indices is None:
        raise MlxrMoeError("gather_qmm: rhs_indices are required")
    if lhs_indices is None and rhs_indices.numel():
        _check_x_batch("gather_qmm", x.shape[:-2], tuple(rhs_indices.shape))
    _dev(x, w, scales, biases, lhs_indices, rhs_indices)
    b = DEFAULT_BITS if bits is None else bits
    x = x.contiguous()
    M, K = x.shape[-2], x.shape[-1]
    x_batch = math.prod(x.shape[:-2])
    E, N = w.shape[0], w.shape[1]
    if w.shape[-1] * 32 != K * b and transpose:
        raise MlxrMoeError(
            f"gather_qmm: w last dim {w.shape[-1]} does not match K={K} at {b} bits")
    rhs = _as_u32(rhs_indices)
    lhs = None if lhs_indices is None else _as_u32(lhs_indices)
    B = rhs.numel()
    if lhs is not None and lhs.numel() != B:
        raise MlxrMoeError("gather_qmm: lhs and rhs indices must have the same size")
    out = torch.empty(tuple(rhs.shape) + (M, N), dtype=torch.bfloat16, device=x.device)
    lib = C.lib()
    nbytes = lib.mlxr_moe_gather_qmm_workspace_size(B, M, E)
    ws = workspace(nbytes, x.device)
    C.check(lib.mlxr_moe_gather_qmm(
        _p(x), _code(x), x_batch, M, K, _p(w.contiguous()), _p(scales.contiguous()),
        _p(None if biases is None else biases.contiguous()), _code(scales), E, N,
        _p(lhs), _p(rhs), B, int(bool(transpose)), C.OptionalInt.of(group_size),
        C.OptionalInt.of(bits), b"affine", int(bool(sorted_indices)), _p(out), C.BFLOAT16,
        _p(ws), ws.numel(), _stream(x)))
    out._mlxr_workspace = ws  # keep the status word alive with the result
    return out


def gather_mm(a, b, lhs_indices=None, rhs_indices=None, sorted_indices=False,
              b_transposed=True):
    """gather_mm (ops/arithmetic.rs:1577-1613) as SwitchLinear::apply calls
    it (nn/switch.rs:84-93): out[i] = a[ab(i)] @ b[rhs_indices[i]]^T with b
    the SwitchLinear weight as stored, bf16 [E, N, K] (the reference passes
    swap_axes(weight, -1, -2), the same memory).  a [..., M, K] bf16; output
    rhs_indices.shape + [M, N] bf16, f32 accumulation.  Without lhs_indices,
    a's batch broadcasts over the trailing index axis."""
    if rhs_indices is None:
        raise MlxrMoeError("gather_mm: rhs_indices are required")
    if lhs_indices is None and rhs_indices.numel():
        _check_x_batch("gather_mm", a.shape[:-2], tuple(rhs_indices.shape))
    _dev(a, b, lhs_indices, rhs_indices)
    if not b_transposed:
        raise MlxrMoeError("gather_mm: only b stored [E, N, K] (b_transposed) is supported")
    if b.ndim != 3:
        raise MlxrMoeError("gather_mm: b must be [E, N, K]")
    a = a.contiguous()
    M, K = a.shape[-2], a.shape[-1]
    a_batch = math.prod(a.shape[:-2])
    E, N = b.shape[0], b.shape[1]
    if b.shape[2] != K:
        raise MlxrMoeError(f"gather_mm: b last dim {b.shape[2]} does not match K={K}")
    rhs = _as_u32(rhs_indices)
    lhs = None if lhs_indices is None else _as_u32(lhs_indices)
    B = rhs.numel()
    if lhs is not None and lhs.numel() != B:
        raise MlxrMoeError("gather_mm: lhs and rhs indices must have the same size")
    out = torch.empty(tuple(rhs.shape) + (M, N), dtype=torch.bfloat16, device=a.device)
    lib = C.lib()
    ws = workspace(lib.mlxr_moe_gather_mm_workspace_size(B, M, E), a.device)
    bc = b.contiguous()
    C.check(lib.mlxr_moe_gather_mm(
        _p(a), _code(a), a_batch, M, K, _p(bc), _code(bc), E, N, 1, _p(lhs), _p(rhs), B,
        int(bool(sorted_indices)), _p(out), C.BFLOAT16, _p(ws), ws.numel(), _stream(a)))
    out._mlxr_workspace = ws  # keep the status word alive with the result
    return out


def _check_axis(a: torch.Tensor, axis: int, what: str) -> int:
    if not -a.ndim <= axis < a.ndim:
        raise MlxrMoeError(
            f"[{what}] Received invalid axis {axis} for array with {a.ndim} dimensions.")
    return axis % a.ndim


def argpartition_axis(a: torch.Tensor, kth: int, axis: int):
    """Indices partitioning `a` along `axis` around position kth (uint32
    semantics in int32 storage).  The full ascending order is returned,
    which satisfies every kth."""
    ax = _check_axis(a, axis, "argpartition")
    _dev(a)
    n = a.shape[ax]
    if not -n <= kth < n:
        raise MlxrMoeError(
            f"[argpartition] Received invalid kth {kth} along axis {axis} for array with "
            f"shape: {tuple(a.shape)}")
    if a.dtype != torch.float32:
        raise MlxrMoeError("argpartition: float32 input only")
    src = a.movedim(ax, -1).contiguous()
    out = torch.empty(src.shape, dtype=torch.int32, device=a.device)
    rows = src.numel() // n if n else 0
    C.check(C.lib().mlxr_moe_argpartition(_p(src), rows, n, kth, -1, _p(out), _stream(a)))
    return out.movedim(-1, ax)


def argpartition(a: torch.Tensor, kth: int):
    """argpartition over the flattened array (sort.rs:250-258)."""
    return argpartition_axis(a.reshape(-1), kth, 0)


def softmax_axis(a: torch.Tensor, axis: int, precise=None):
    ax = _check_axis(a, axis, "softmax")
    _dev(a)
    if a.dtype != torch.float32:
        raise MlxrMoeError("softmax: float32 input only")
    src = a.movedim(ax, -1).contiguous()
    n = src.shape[-1]
    out = torch.empty_like(src)
    C.check(C.lib().mlxr_moe_softmax(_p(src), src.numel() // max(n, 1), n, -1,
                                     int(bool(precise)), _p(out), _stream(a)))
    return out.movedim(-1, ax)


def router_topk(x: torch.Tensor, gate_w: torch.Tensor, k: int):
    """softmax(x @ gate_w^T) -> top-k -> renormalise (moe.rs:122-138).
    Returns (indices int32 [T, k], weights f32 [T, k])."""
    _dev(x, gate_w)
    x2 = x.reshape(-1, x.shape[-1]).contiguous()
    T, d = x2.shape
    E = gate_w.shape[0]
    idx = torch.empty((T, k), dtype=torch.int32, device=x.device)
    wts = torch.empty((T, k), dtype=torch.float32, device=x.device)
    lib = C.lib()
    ws = workspace(lib.mlxr_moe_router_workspace_size(T, E), x.device)
    C.check(lib.mlxr_moe_router_topk(_p(x2), T, d, _p(gate_w.contiguous()), E, k, _p(idx),
                                     _p(wts), _p(ws), ws.numel(), _stream(x)))
    lead = tuple(x.shape[:-1])
    return idx.reshape(lead + (k,)), wts.reshape(lead + (k,))


def router_topk_quantized(x: torch.Tensor, gate, k: int):
    """router_topk with the router as a QuantizedLinear (nn.QuantizedLinear,
    4 or 8 bits, group 64; layers/quantized.rs:356-373) or a bf16 Linear
    (nn.Linear): bf16 logits and probabilities, top-k on the probabilities.
    Returns (indices int32 [T, k], weights [T, k] -- bf16 values held in
    f32)."""
    _dev(x, gate.weight)
    x2 = x.reshape(-1, x.shape[-1]).contiguous()
    T = x2.shape[0]
    idx = torch.empty((T, k), dtype=torch.int32, device=x.device)
    wts = torch.empty((T, k), dtype=torch.float32, device=x.device)
    lib = C.lib()
    ws = workspace(lib.mlxr_moe_router_workspace_size(T, gate.output_dims), x.device)
    desc = gate.descriptor()
    C.check(lib.mlxr_moe_router_topk_quantized(_p(x2), T, ctypes.byref(desc), k, _p(idx),
                                               _p(wts), _p(ws), ws.numel(), _stream(x)))
    lead = tuple(x.shape[:-1])
    return idx.reshape(lead + (k,)), wts.reshape(lead + (k,))


def dispatch(ids: torch.Tensor, num_experts: int):
    """Stable expert sort of flat ids (gather_sort, switch.rs:499-512).
    Returns (counts [E], offsets [E+1], order [n], inv_order [n])."""
    _dev(ids)
    flat = _as_u32(ids).reshape(-1)
    n = flat.numel()
    dev = ids.device
    counts = torch.empty(num_experts, dtype=torch.int32, device=dev)
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    order = torch.empty(n, dtype=torch.int32, device=dev)
    inv = torch.empty(n, dtype=torch.int32, device=dev)
    lib = C.lib()
    ws = workspace(lib.mlxr_moe_dispatch_workspace_size(n, num_experts), dev)
    C.check(lib.mlxr_moe_dispatch(_p(flat), n, num_experts, _p(counts), _p(offsets),
                                  _p(order), _p(inv), _p(ws), ws.numel(), _stream(ids)))
    order._mlxr_workspace = ws
    return counts, offsets, order, inv


def combine(y: torch.Tensor, weights: torch.Tensor, shared_y=None, shared_logit=None):
    """sum_k w * y over the top-k axis (combine_with_weights, switch.rs:
    223-234), plus shared_y * sigmoid(shared_logit) when given."""
    _dev(y, weights, shared_y, shared_logit)
    T, K, d = y.shape
    out = torch.empty((T, d), dtype=torch.float32, device=y.device)
    C.check(C.lib().mlxr_moe_combine(
        _p(y.contiguous()), _p(weights.contiguous()), T, K, d,
        _p(None if shared_y is None else shared_y.contiguous()),
        _p(None if shared_logit is None else shared_logit.contiguous()), _p(out),
        _stream(y)))
    return out


def gather_qmm_tiled(rows: int, num_experts: int) -> bool:
    """True when a gather_qmm of `rows` flat rows over `num_experts` experts
    runs the M-tiled kernel (weights dequantised to bf16 tiles, the
    gather_mm(x, dequantize(w)) numerics), False for the streaming kernel
    (weights dequantised in f32)."""
    rc = C.lib().mlxr_moe_gather_qmm_tiled(int(rows), int(num_experts))
    if rc < 0:
        raise MlxrMoeError("gather_qmm_tiled: negative size")
    return bool(rc)


def router_matrix_order(T: int, d: int, columns: int) -> bool:
    """True when a router's logits of T tokens over d inputs, `columns`
    logit columns (the experts, plus one for a shared-expert gate computed
    beside them), are summed in the matrix-core order (the oracle's
    router_logits(mfma=True)), False for the lane order."""
    rc = C.lib().mlxr_moe_router_matrix_order(int(T), int(d), int(columns))
    if rc < 0:
        raise MlxrMoeError("router_matrix_order: negative size")
    return bool(rc)


def workspace_status(ws: torch.Tensor) -> int:
    """Device status word of a call's workspace (1 = an index was out of
    range).  Synchronises the current stream."""
    rc = C.lib().mlxr_moe_workspace_status(_p(ws), ws.numel(), _stream(ws))
    if rc < 0:
        raise MlxrMoeError(C.last_error())
    return rc
