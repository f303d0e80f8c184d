"""numpy view of the CPU oracle (liboracle.so built from moe_oracle.c).

TEST INFRASTRUCTURE ONLY: the parity checker and the "port" CPU baseline.
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module.  bf16 arrays are numpy uint16 bit patterns.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from ctypes import POINTER, Structure, c_float, c_int, c_int32, c_int64, c_uint16, c_uint32, c_void_p
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
# MLXR_ORACLE_LIB: another build of the same source (the sanitizer copy)
LIB = Path(os.environ.get("MLXR_ORACLE_LIB", HERE / "liboracle.so"))
F32, BF16 = 0, 1


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def build_native(out_dir) -> Path:
    """A copy of the oracle compiled for this host's CPU (-march=native) in
    out_dir: the CPU baseline times it where it runs."""
    out = Path(out_dir) / "liboracle_native.so"
    subprocess.run(["make", "-s", "-C", str(HERE), f"NATIVE_OUT={out}", "native"], check=True)
    return out


_lib = None


def use_library(path) -> None:
    """Route every later oracle call through the library at `path` (built
    from the same source, e.g. by build_native)."""
    global _lib
    _lib = ctypes.CDLL(str(path))


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        _lib = ctypes.CDLL(str(LIB))
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(c_void_p)


# ----------------------------------------------------------------- bf16
def f32_to_bf16(a) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bits (NaN -> 0x7FC0)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r[nan] = 0x7FC0
    return r


def bf16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)


# ------------------------------------------------------------- wrappers
def quantize(w: np.ndarray, group_size=64, bits=4, bf16=True):
    """w: uint16 bf16 bits (bf16=True) or float32 [rows, cols]."""
    w = np.ascontiguousarray(w)
    rows, cols = int(np.prod(w.shape[:-1])), w.shape[-1]
    wq = np.zeros(w.shape[:-1] + (cols * bits // 32,), np.uint32)
    sdt = np.uint16 if bf16 else np.float32
    sc = np.zeros(w.shape[:-1] + (cols // group_size,), sdt)
    bi = np.zeros_like(sc)
    rc = lib().orc_quantize(_p(w), c_int(BF16 if bf16 else F32), c_int64(rows), c_int64(cols),
                            c_int(group_size), c_int(bits), _p(wq), _p(sc), _p(bi))
    if rc:
        raise ValueError("orc_quantize rejected the arguments")
    return wq, sc, bi


def dequantize(wq, scales, biases, group_size=64, bits=4, out_bf16=True):
    wq = np.ascontiguousarray(wq, np.uint32)
    sb_bf16 = scales.dtype == np.uint16
    cols = wq.shape[-1] * 32 // bits
    rows = int(np.prod(wq.shape[:-1]))
    out = np.zeros(wq.shape[:-1] + (cols,), np.uint16 if out_bf16 else np.float32)
    rc = lib().orc_dequantize(_p(wq), _p(np.ascontiguousarray(scales)),
                              _p(np.ascontiguousarray(biases)), c_int(BF16 if sb_bf16 else F32),
                              c_int64(rows), c_int64(cols), c_int(group_size), c_int(bits),
                              _p(out), c_int(BF16 if out_bf16 else F32))
    if rc:
        raise ValueError("orc_dequantize rejected the arguments")
    return out


def router_logits(x_bf16, w_f32, mfma=False):
    """logits [T, E] of an f32 router in the lane order (orc_router_logits),
    or with mfma in the matrix-core order (orc_router_logits_mfma, d a
    multiple of 64)."""
    x = np.ascontiguousarray(x_bf16, np.uint16)
    w = np.ascontiguousarray(w_f32, np.float32)
    T, d = x.shape
    E = w.shape[0]
    out = np.zeros((T, E), np.float32)
    if mfma:
        if lib().orc_router_logits_mfma(_p(x), _p(w), c_int64(T), c_int64(d), c_int64(E),
                                        _p(out)):
            raise ValueError("orc_router_logits_mfma: d must be a multiple of 64")
    else:
        lib().orc_router_logits(_p(x), _p(w), c_int64(T), c_int64(d), c_int64(E), _p(out))
    return out


def router_topk(logits, K):
    lg = np.ascontiguousarray(logits, np.float32)
    T, E = lg.shape
    idx = np.zeros((T, K), np.int32)
    w = np.zeros((T, K), np.float32)
    lib().orc_router_topk(_p(lg), c_int64(T), c_int64(E), c_int64(K), _p(idx), _p(w))
    return idx, w


def router_logits_q(x_bf16, wq, scales, biases, bits, mfma=False):
    """QuantizedLinear router (or, bits 16, a bf16 Linear: wq the bf16 bits
    [E, d], scales and biases None): bf16 logits (as f32) [T, E]; with mfma
    in the matrix-core order."""
    x = np.ascontiguousarray(x_bf16, np.uint16)
    wq = np.ascontiguousarray(wq, np.uint16 if bits == 16 else np.uint32)
    T, d = x.shape
    E = wq.shape[0]
    out = np.zeros((T, E), np.float32)
    sc = None if scales is None else np.ascontiguousarray(scales, np.uint16)
    bi = None if biases is None else np.ascontiguousarray(biases, np.uint16)
    fn = lib().orc_router_logits_q_mfma if mfma else lib().orc_router_logits_q
    rc = fn(_p(x), _p(wq), _p(sc), _p(bi), c_int(bits),
                                   c_int64(T), c_int64(d), c_int64(E), _p(out))
    if rc:
        raise ValueError("orc_router_logits_q rejected the arguments")
    return out


def router_topk_bf16(logits, K):
    """Top-K on the bf16 probabilities of bf16 logits; bf16 weights."""
    lg = np.ascontiguousarray(logits, np.float32)
    T, E = lg.shape
    idx = np.zeros((T, K), np.int32)
    w = np.zeros((T, K), np.float32)
    lib().orc_router_topk_bf16(_p(lg), c_int64(T), c_int64(E), c_int64(K), _p(idx), _p(w))
    return idx, w


def dispatch(ids, E):
    ids = np.ascontiguousarray(ids, np.int32).reshape(-1)
    n = ids.size
    counts = np.zeros(E, np.int32)
    offsets = np.zeros(E + 1, np.int32)
    srt = np.zeros(n, np.int32)
    inv = np.zeros(n, np.int32)
    rc = lib().orc_dispatch(_p(ids), c_int64(n), c_int64(E), _p(counts), _p(offsets), _p(srt),
                            _p(inv))
    if rc:
        raise ValueError("orc_dispatch: id out of range")
    return counts, offsets, srt, inv


def gather_qmm(x, wq, scales, biases, rhs, lhs=None, group_size=64, bits=4, nthreads=1,
               tiled=False):
    """x uint16 [x_batch, M, K]; wq uint32 [E, N, K*bits/32]; scales/biases
    uint16 [E, N, K/g]; rhs [B] -> out uint16 [B, M, N].  tiled: the
    bf16-dequantised (tiled) numerics instead of the f32 (vector) ones."""
    x = np.ascontiguousarray(x, np.uint16)
    xb, M, Kd = x.shape
    E, N = wq.shape[0], wq.shape[1]
    rhs = np.ascontiguousarray(rhs, np.int32).reshape(-1)
    lhs_a = None if lhs is None else np.ascontiguousarray(lhs, np.int32).reshape(-1)
    B = rhs.size
    out = np.zeros((B, M, N), np.uint16)
    rc = lib().orc_gather_qmm(_p(x), c_int64(xb), c_int64(M), c_int64(Kd),
                              _p(np.ascontiguousarray(wq, np.uint32)),
                              _p(np.ascontiguousarray(scales, np.uint16)),
                              _p(np.ascontiguousarray(biases, np.uint16)), c_int64(E),
                              c_int64(N), _p(lhs_a), _p(rhs), c_int64(B), c_int(group_size),
                              c_int(bits), c_int(1 if tiled else 0), _p(out), c_int(nthreads))
    if rc:
        raise ValueError("orc_gather_qmm rejected the arguments")
    return out


def gather_mm(x, w, rhs, lhs=None, nthreads=1):
    """x uint16 [x_batch, M, K]; w uint16 (bf16 bits) [E, N, K] -- the
    SwitchLinear weight as stored; rhs [B] -> out uint16 [B, M, N]."""
    x = np.ascontiguousarray(x, np.uint16)
    xb, M, Kd = x.shape
    w = np.ascontiguousarray(w, np.uint16)
    E, N = w.shape[0], w.shape[1]
    rhs = np.ascontiguousarray(rhs, np.int32).reshape(-1)
    lhs_a = None if lhs is None else np.ascontiguousarray(lhs, np.int32).reshape(-1)
    B = rhs.size
    out = np.zeros((B, M, N), np.uint16)
    rc = lib().orc_gather_mm(_p(x), c_int64(xb), c_int64(M), c_int64(Kd), _p(w), c_int64(E),
                             c_int64(N), _p(lhs_a), _p(rhs), c_int64(B), _p(out),
                             c_int(nthreads))
    if rc:
        raise ValueError("orc_gather_mm rejected the arguments")
    return out


def swiglu(g, u):
    g = np.ascontiguousarray(g, np.uint16)
    u = np.ascontiguousarray(u, np.uint16)
    out = np.zeros_like(g)
    lib().orc_swiglu(_p(g), _p(u), c_int64(g.size), _p(out))
    return out


def combine(y, w, shared_y=None, shared_logit=None):
    y = np.ascontiguousarray(y, np.uint16)
    T, K, d = y.shape
    out = np.zeros((T, d), np.float32)
    lib().orc_combine(_p(y), _p(np.ascontiguousarray(w, np.float32)), c_int64(T), c_int64(K),
                      c_int64(d),
                      _p(None if shared_y is None else np.ascontiguousarray(shared_y, np.uint16)),
                      _p(None if shared_logit is None
                         else np.ascontiguousarray(shared_logit, np.float32)),
                      _p(out))
    return out


def combine_bf16(y, w, shared_y=None, shared_logit=None):
    """Combine with bf16 routing weights; bf16 out (uint16 bits)."""
    y = np.ascontiguousarray(y, np.uint16)
    T, K, d = y.shape
    out = np.zeros((T, d), np.uint16)
    lib().orc_combine_bf16(_p(y), _p(np.ascontiguousarray(w, np.float32)), c_int64(T),
                           c_int64(K), c_int64(d),
                           _p(None if shared_y is None
                              else np.ascontiguousarray(shared_y, np.uint16)),
                           _p(None if shared_logit is None
                              else np.ascontiguousarray(shared_logit, np.float32)),
                           _p(out))
    return out


def geglu(g, u):
    g = np.ascontiguousarray(g, np.uint16)
    u = np.ascontiguousarray(u, np.uint16)
    out = np.zeros_like(g)
    lib().orc_geglu(_p(g), _p(u), c_int64(g.size), _p(out))
    return out


def rms_norm(x, w, eps):
    x = np.ascontiguousarray(x, np.uint16)
    T, d = x.shape
    out = np.zeros_like(x)
    lib().orc_rms_norm(_p(x), c_int64(T), c_int64(d), _p(np.ascontiguousarray(w, np.uint16)),
                       c_float(eps), _p(out))
    return out


def gemma_router(x, norm_w, eps, proj, pes, K, bits=0, mfma=False):
    """gemma4 Router::forward.  proj: bf16 [E, d] (uint16) when bits == 0,
    else (wq, scales, biases) of a QuantizedLinear; mfma: the scores in the
    matrix-core order.  Returns (idx [T, K], weights bf16 [T, K] as
    uint16)."""
    x = np.ascontiguousarray(x, np.uint16)
    T, d = x.shape
    keep = []
    if bits:
        wq, sc, bi = (np.ascontiguousarray(a, dt) for a, dt in
                      zip(proj, (np.uint32, np.uint16, np.uint16)))
        keep += [wq, sc, bi]
        E = wq.shape[0]
        ql = _QL(wq.ctypes.data, sc.ctypes.data, bi.ctypes.data)
        pb, pq = None, ctypes.byref(ql)
    else:
        pw = np.ascontiguousarray(proj, np.uint16)
        keep.append(pw)
        E = pw.shape[0]
        pb, pq = _p(pw), None
    idx = np.zeros((T, K), np.int32)
    w = np.zeros((T, K), np.uint16)
    rc = lib().orc_gemma_router(_p(x), c_int64(T), c_int64(d), c_int64(E), c_int64(K),
                                _p(np.ascontiguousarray(norm_w, np.uint16)), c_float(eps),
                                pb, pq, c_int(bits), _p(np.ascontiguousarray(pes, np.uint16)),
                                _p(idx), _p(w), c_int(1 if mfma else 0))
    if rc:
        raise ValueError("orc_gemma_router rejected the arguments")
    return idx, w


def packed_switch_glu(x, gate_up, down, idx, w, act=1, w_bf16=True, tiled=False, nthreads=1,
                      with_y=False):
    """PackedSwitchFfn::forward_with_combine.  gate_up = (wq [E, 2H, d*b/32],
    scales, biases); down likewise [E, d, H]; idx [T, K]; w [T, K] (f32, or
    bf16 values when w_bf16).  Returns out ([T, d] bf16 as uint16 when
    w_bf16, else f32) and, with_y, the per-expert rows [T, K, d]."""
    x = np.ascontiguousarray(x, np.uint16)
    T, d = x.shape

    def arrs(t):
        # (weight, scales, biases); dense bf16: (weight uint16 [E, N, K], None, None)
        if t[1] is None:
            return np.ascontiguousarray(t[0], np.uint16), None, None
        return tuple(np.ascontiguousarray(a, dt)
                     for a, dt in zip(t, (np.uint32, np.uint16, np.uint16)))

    gw, gs, gb = arrs(gate_up)
    dw, ds, db = arrs(down)
    E, H2 = gw.shape[0], gw.shape[1]
    bits = 16 if gs is None else gw.shape[2] * 32 // d
    idx = np.ascontiguousarray(idx, np.int32)
    K = idx.shape[1]
    wf = np.ascontiguousarray(w, np.float32)
    out = np.zeros((T, d), np.uint16 if w_bf16 else np.float32)
    y = np.zeros((T, K, d), np.uint16)
    rc = lib().orc_packed_switch_glu(_p(x), c_int64(T), c_int64(d), c_int64(H2 // 2),
                                     c_int64(E), _p(gw), _p(gs), _p(gb), _p(dw), _p(ds), _p(db),
                                     c_int(bits), c_int(act), _p(idx), _p(wf),
                                     c_int(1 if w_bf16 else 0), c_int64(K),
                                     c_int(1 if tiled else 0), _p(out), _p(y), c_int(nthreads))
    if rc:
        raise ValueError("orc_packed_switch_glu rejected the arguments")
    return (out, y) if with_y else out


class _QL(Structure):
    _fields_ = [("w", c_void_p), ("scales", c_void_p), ("biases", c_void_p)]


class _Block(Structure):
    _fields_ = [
        ("hidden", c_int64), ("num_experts", c_int64), ("top_k", c_int64),
        ("intermediate", c_int64), ("shared_intermediate", c_int64), ("bits", c_int32),
        ("group_size", c_int32), ("router_w", c_void_p), ("router_b", c_void_p),
        ("gate_proj", _QL), ("up_proj", _QL), ("down_proj", _QL),
        ("shared_gate", _QL), ("shared_up", _QL), ("shared_down", _QL),
        ("shared_gate_w", c_void_p), ("switch_tiled", c_int32), ("shared_tiled", c_int32),
        ("router_q", _QL), ("shared_gate_q", _QL), ("router_bits", c_int32),
        ("router_mfma", c_int32),
    ]


def _ql(t):
    if t is None:
        return _QL()
    return _QL(*(None if a is None else a.ctypes.data for a in t))


def block_forward_residual(p: dict, norm_w, eps, h, nthreads=1, tiled=(False, False),
                           router_mfma=False):
    """out = h + block(rms_norm(h, norm_w, eps)) (layer.rs:134-138), with
    block_forward's parameters.  Returns (out, idx, weights)."""
    return block_forward(p, h, nthreads, tiled, residual=(norm_w, eps),
                         router_mfma=router_mfma)


def block_forward(p: dict, x, nthreads=1, tiled=(False, False), residual=None,
                  router_mfma=False):
    """p: numpy block parameters -- d, E, K, f, fs, bits, group_size,
    router_w, router_b (or None), gate/up/down = (wq, scales, biases),
    shared_gate/shared_up/shared_down, shared_gate_w (None when fs == 0).
    A quantised router instead: router_q = (wq, scales, biases) [E, ...],
    shared_gate_q likewise [1, ...], router_bits; then the block is bf16.
    tiled: gather_qmm numerics of (routed experts, shared expert).
    router_mfma: an f32 router's logits (and the shared gate's) in
    router_logits(mfma=True)'s order.
    Returns (out [T, d] -- f32, or bf16 as uint16 with a quantised router --,
    idx [T, K], weights [T, K])."""
    keep = []

    def c(a, dt):
        if a is None:
            return None
        a = np.ascontiguousarray(a, dt)
        keep.append(a)
        return a

    def q(t):
        if t is None:
            return None
        if t[1] is None:  # dense bf16 weights
            return (c(t[0], np.uint16), None, None)
        return (c(t[0], np.uint32), c(t[1], np.uint16), c(t[2], np.uint16))

    x = c(x, np.uint16)
    T = x.shape[0]
    rq = p.get("router_q")
    rw, rb = c(p.get("router_w"), np.float32), c(p.get("router_b"), np.float32)
    sgw = c(p.get("shared_gate_w"), np.float32)
    blk = _Block(p["d"], p["E"], p["K"], p["f"], p.get("fs", 0), p["bits"], p["group_size"],
                 None if rw is None else rw.ctypes.data, None if rb is None else rb.ctypes.data,
                 _ql(q(p["gate"])), _ql(q(p["up"])), _ql(q(p["down"])),
                 _ql(q(p.get("shared_gate"))), _ql(q(p.get("shared_up"))),
                 _ql(q(p.get("shared_down"))), None if sgw is None else sgw.ctypes.data,
                 1 if tiled[0] else 0, 1 if tiled[1] else 0,
                 _ql(q(rq)), _ql(q(p.get("shared_gate_q"))), p.get("router_bits", 0),
                 1 if router_mfma else 0)
    out = np.zeros((T, p["d"]), np.uint16 if rq is not None else np.float32)
    idx = np.zeros((T, p["K"]), np.int32)
    w = np.zeros((T, p["K"]), np.float32)
    if residual is not None:
        nw = c(residual[0], np.uint16)
        rc = lib().orc_block_forward_residual(ctypes.byref(blk), _p(nw), c_float(residual[1]),
                                              _p(x), c_int64(T), _p(out), _p(idx), _p(w),
                                              c_int(nthreads))
    else:
        rc = lib().orc_block_forward(ctypes.byref(blk), _p(x), c_int64(T), _p(out), _p(idx),
                                     _p(w), c_int(nthreads))
    if rc:
        raise ValueError("orc_block_forward rejected the arguments")
    return out, idx, w


__all__ = ["build", "build_native", "use_library", "lib", "f32_to_bf16", "bf16_to_f32", "quantize", "dequantize",
           "router_logits", "router_topk", "router_logits_q", "router_topk_bf16", "dispatch",
           "gather_qmm", "gather_mm", "swiglu", "combine", "combine_bf16", "geglu", "rms_norm", "gemma_router",
           "packed_switch_glu",
           "block_forward", "block_forward_residual", "POINTER", "c_float", "c_uint16", "c_uint32"]


# ------------------------------------------------------- torch adapters
def to_np(t):
    """Device tensor -> numpy with bf16 as uint16 bits and packed int32
    words as uint32."""
    import torch

    t = t.detach()
    if t.dtype == torch.bfloat16:
        return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    if t.dtype == torch.int32:
        return t.contiguous().cpu().numpy().view(np.uint32)
    return t.contiguous().cpu().numpy()


def qlinear_np(lin):
    """(weight, scales, biases) numpy arrays of an nn module's projection:
    packed words uint32 [E, N, K*bits/32] with bf16 scales/biases, or for a
    dense SwitchLinear / Linear (bits 16) the bf16 bits [E, N, K] and None."""
    if lin.bits == 16:
        return (to_np(lin.weight), None, None)
    return (to_np(lin.weight).reshape(lin.weight.shape[0], lin.weight.shape[1], -1),
            to_np(lin.scales), to_np(lin.biases))


def block_params(bw) -> dict:
    """Numpy parameters for block_forward from a workloads.BlockWeights."""
    cfg = bw.cfg
    q = qlinear_np

    m = bw.switch_mlp
    p = dict(d=cfg.d, E=cfg.E, K=cfg.K, f=cfg.f, fs=cfg.fs, bits=cfg.bits,
             group_size=cfg.group_size,
             router_b=None if bw.gate_b is None else to_np(bw.gate_b),
             gate=q(m.gate_proj), up=q(m.up_proj), down=q(m.down_proj))
    if cfg.router_bits:  # QuantizedLinear or bf16 Linear router
        p.update(router_q=q(bw.gate_w), router_bits=cfg.router_bits)
    else:
        p.update(router_w=to_np(bw.gate_w))
    if cfg.fs:
        s = bw.shared_expert
        p.update(shared_gate=q(s.gate_proj), shared_up=q(s.up_proj), shared_down=q(s.down_proj))
        if cfg.router_bits:
            p.update(shared_gate_q=q(bw.shared_gate_w))
        else:
            p.update(shared_gate_w=to_np(bw.shared_gate_w))
    return p
