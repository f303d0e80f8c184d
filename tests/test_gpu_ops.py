"""GPU parity of the op-level entry points against the CPU oracle."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _bf16(orc, a, dev):
    return torch.from_numpy(orc.f32_to_bf16(a).view(np.int16)).view(torch.bfloat16).to(dev)


def _np(orc, t):
    return orc.to_np(t)


# ------------------------------------------------------- quantize
@pytest.mark.parametrize("shape,gs,bits", [
    ((8, 256), 64, 4), ((8, 256), 64, 8), ((8, 256), 64, 2), ((16, 512), 128, 4),
    ((16, 512), 32, 8), ((3, 64, 128), 64, 4)])
def test_quantize_bit_exact_bf16(pkg, orc, dev, shape, gs, bits):
    rng = np.random.default_rng(abs(hash((shape, gs, bits))) % 2 ** 32)
    w = (rng.standard_normal(shape) * 0.02).astype(np.float32)
    w[..., :64] *= 50  # a wide group next to narrow ones
    wt = _bf16(orc, w, dev)
    wq, sc, bi = pkg.ops.quantize(wt, gs, bits)
    rq, rs, rb = orc.quantize(_np(orc, wt), gs, bits, bf16=True)
    assert np.array_equal(_np(orc, wq).reshape(rq.shape), rq)
    assert np.array_equal(_np(orc, sc), rs)
    assert np.array_equal(_np(orc, bi), rb)
    deq = pkg.ops.dequantize(wq, sc, bi, gs, bits)
    assert np.array_equal(_np(orc, deq), orc.dequantize(rq, rs, rb, gs, bits))


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_quantize_reference_arange_f32(pkg, orc, dev, bits):
    """quantization.rs:299-315 on the GPU, f32 in, f32 scales."""
    x = torch.arange(0, 512, dtype=torch.float32, device=dev).expand(128, 512).contiguous()
    wq, sc, bi = pkg.ops.quantize(x, 128, bits)
    assert tuple(wq.shape) == (128, 512 // (32 // bits)) and tuple(sc.shape) == (128, 4)
    xh = pkg.ops.dequantize(wq, sc, bi, 128, bits)
    assert float((x - xh).abs().max()) <= 127.0 / (1 << bits)
    rq, rs, rb = orc.quantize(x.cpu().numpy(), 128, bits, bf16=False)
    assert np.array_equal(_np(orc, wq), rq)
    assert np.array_equal(sc.cpu().numpy(), rs) and np.array_equal(bi.cpu().numpy(), rb)


def test_quantize_full_expert_bank_bit_exact(pkg, orc, dev):
    """c2 gate_proj [128, 768, 2048] at 4 bits and a c5-sized 8-bit slice."""
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    for shape, bits in [((128, 768, 2048), 4), ((16, 1536, 4096), 8)]:
        w = (torch.randn(shape, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        wq, sc, bi = pkg.ops.quantize(w, 64, bits)
        rq, rs, rb = orc.quantize(_np(orc, w), 64, bits, bf16=True)
        assert np.array_equal(_np(orc, wq), rq)
        assert np.array_equal(_np(orc, sc), rs) and np.array_equal(_np(orc, bi), rb)
        del w, wq, sc, bi


# --------------------------------------------------------- router
@pytest.mark.parametrize("T,d,E,K", [(16, 512, 8, 2), (1, 2048, 128, 8), (64, 2048, 128, 8),
                                     (64, 2048, 512, 10), (300, 4096, 128, 8),
                                     (300, 2052, 128, 8), (2048, 2048, 128, 8),
                                     (3001, 4096, 513, 10), (2048, 2052, 128, 8),
                                     (1024, 2048, 256, 8), (1024, 2048, 128, 8),
                                     (520, 2048, 513, 10)])
def test_router_topk_bit_exact(pkg, orc, dev, T, d, E, K):
    rng = np.random.default_rng(T * 7 + E)
    print(f"  router_topk T={T} d={d} E={E} K={K}", flush=True)
    # x is the head of a buffer whose tail holds NaN bits: a kernel that
    # read past the last row (or past a row into the next) would turn a
    # logit into NaN
    buf = torch.full((T * d + 64,), float("nan"), dtype=torch.bfloat16, device=dev)
    buf[:T * d] = _bf16(orc, rng.standard_normal((T, d)).astype(np.float32), dev).reshape(-1)
    x = buf[:T * d].view(T, d)
    w = torch.from_numpy((rng.standard_normal((E, d)) * 0.02).astype(np.float32)).to(dev)
    idx, wts = pkg.ops.router_topk(x, w, K)
    # (many tokens with d a multiple of 64: the matrix-core order; the
    # rows past the last token hold NaN, as above, and a 513-column router
    # has a partial tile of columns)
    lg = orc.router_logits(_np(orc, x), w.cpu().numpy(), mfma=pkg.ops.router_matrix_order(T, d, E))
    ridx, rw = orc.router_topk(lg, K)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    assert np.allclose(wts.cpu().numpy(), rw, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("T,d,E,K,bits", [(1, 2048, 256, 8, 8), (40, 2048, 256, 8, 8),
                                          (1024, 2048, 256, 8, 8), (16, 512, 8, 2, 4),
                                          (300, 4096, 128, 8, 4), (7, 2048, 512, 10, 8),
                                          (2048, 2048, 256, 8, 8), (2100, 4096, 128, 8, 4)])
def test_router_topk_quantized_bit_exact(pkg, orc, dev, T, d, E, K, bits):
    """QuantizedLinear router (layers/quantized.rs:356-373): bf16 logits,
    top-K on the bf16 probabilities and bf16 weights, all bit for bit
    against the oracle, through each logits kernel (T <= 2, <= 256,
    tiled)."""
    rng = np.random.default_rng(T * 11 + E + bits)
    print(f"  router_topk_quantized T={T} d={d} E={E} K={K} bits={bits}", flush=True)
    x = _bf16(orc, rng.standard_normal((T, d)).astype(np.float32), dev)
    w = _bf16(orc, (rng.standard_normal((E, d)) * 0.05).astype(np.float32), dev)
    gate = pkg.nn.QuantizedLinear.try_from_linear(w, 64, bits)
    idx, wts = pkg.ops.router_topk_quantized(x, gate, K)
    wq, sc, bi = (_np(orc, t) for t in (gate.weight, gate.scales, gate.biases))
    lg = orc.router_logits_q(_np(orc, x), wq.reshape(E, -1), sc.reshape(E, -1),
                             bi.reshape(E, -1), bits, mfma=pkg.ops.router_matrix_order(T, d, E))
    ridx, rw = orc.router_topk_bf16(lg, K)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    assert np.array_equal(wts.cpu().numpy(), rw)


@pytest.mark.parametrize("T,d,E,K,bits", [(1, 2048, 128, 8, 16), (40, 2048, 128, 8, 16),
                                          (300, 2048, 128, 8, 16), (33, 2048, 256, 8, 8),
                                          (7, 512, 8, 2, 16), (300, 516, 64, 4, 16),
                                          (2048, 2048, 128, 8, 16), (2048, 2048, 256, 8, 8)])
def test_gemma_router_bit_exact(pkg, orc, dev, T, d, E, K, bits):
    """gemma4 Router::forward (text.rs:621-665): RMSNorm, bf16 (or 8-bit)
    projection, top-K of the bf16 scores, softmax of the K scores times
    per_expert_scale -- indices and bf16 weights bit for bit."""
    rng = np.random.default_rng(T + E + bits)
    print(f"  gemma_router T={T} d={d} E={E} K={K} bits={bits}", flush=True)
    x = _bf16(orc, rng.standard_normal((T, d)).astype(np.float32), dev)
    projf = _bf16(orc, rng.standard_normal((E, d)).astype(np.float32), dev)
    proj = pkg.nn.QuantizedLinear.try_from_linear(projf, 64, 8) if bits == 8 else projf
    scale = _bf16(orc, (rng.random(d) + 0.5).astype(np.float32), dev)
    pes = _bf16(orc, (rng.random(E) + 0.5).astype(np.float32), dev)
    r = pkg.nn.GemmaRouter(proj, scale, pes, K)
    idx, w = r(x)
    oproj = ((_np(orc, proj.weight).reshape(E, -1), _np(orc, proj.scales).reshape(E, -1),
              _np(orc, proj.biases).reshape(E, -1)) if bits == 8 else _np(orc, projf))
    ridx, rw = orc.gemma_router(_np(orc, x), _np(orc, r.norm_weight), r.eps, oproj,
                                _np(orc, pes), K, bits=8 if bits == 8 else 0,
                                mfma=pkg.ops.router_matrix_order(T, d, E))
    assert np.array_equal(idx.cpu().numpy(), ridx)
    assert np.array_equal(_np(orc, w), rw)


@pytest.mark.parametrize("T", [24, 512])
def test_packed_swiglu_equals_split(pkg, dev, T):
    """PackedSwitchFfn with gate_up = [gate; up] along the output rows and
    SwiGLU runs the same kernels as SplitSwitchFfn with the separate
    tensors: identical bits, per-expert rows and combine, on the decode
    (T=24) and prefill (T=512) paths."""
    W = pkg.workloads
    cfg = W.CONFIGS["c2"]
    bw = W.make_weights(cfg, dev)
    m = bw.switch_mlp
    cat = lambda a, b: torch.cat([a, b], dim=1).contiguous()  # noqa: E731
    gu = pkg.nn.QuantizedSwitchLinear(cat(m.gate_proj.weight, m.up_proj.weight),
                                      cat(m.gate_proj.scales, m.up_proj.scales),
                                      cat(m.gate_proj.biases, m.up_proj.biases), 64, cfg.bits)
    packed = pkg.nn.PackedSwitchFfn(gu, m.down_proj, "swiglu")
    g = torch.Generator().manual_seed(T)
    x = W.make_x(cfg, T, dev, seed=T)
    idx = torch.stack([torch.randperm(cfg.E, generator=g)[:cfg.K] for _ in range(T)]).int().to(dev)
    w = torch.rand((T, cfg.K), generator=g).to(dev)
    print(f"  packed vs split T={T}", flush=True)
    assert torch.equal(packed.forward(x, idx), m.forward(x, idx))
    assert torch.equal(packed.forward_with_combine(x, idx, w), m.forward_with_combine(x, idx, w))


@pytest.mark.parametrize("T", [6, 600])
def test_switch_status_cleared_per_call(pkg, orc, dev, T):
    """The switch FFN's dispatch clears the workspace status itself: an
    out-of-range expert id sets it to 1, and the next call with valid ids on
    the same workspace reads 0 again, with T*K below (one dispatch kernel)
    and above 1024 flat rows (the multi-kernel dispatch)."""
    E, d, f, K = 8, 256, 128, 2
    qs = [_qbank(pkg, orc, E, n, k, 4, dev, seed) for seed, (n, k) in
          enumerate([(f, d), (f, d), (d, f)])]
    sw = pkg.nn.SplitSwitchFfn(*[pkg.nn.QuantizedSwitchLinear(*q, 64, 4) for q in qs])
    g = torch.Generator().manual_seed(T)
    x = (torch.randn((T, d), generator=g) * 0.5).to(torch.bfloat16).to(dev)
    good = torch.randint(0, E, (T, K), generator=g, dtype=torch.int32).to(dev)
    bad = good.clone()
    bad[T // 2, 1] = E + 3
    print(f"  switch status T={T}", flush=True)
    sw.forward(x, bad)
    ws = sw.last_workspace
    assert pkg.ops.workspace_status(ws) == 1
    want = sw.forward(x, good)
    C, lib = pkg._capi, pkg._capi.lib()
    y = torch.empty((T, K, d), dtype=torch.bfloat16, device=dev)
    C.check(lib.mlxr_moe_switch_glu_experts(
        ctypes.byref(sw.descriptor()), x.data_ptr(), T, good.data_ptr(), K, y.data_ptr(),
        ws.data_ptr(), ws.numel(), pkg.ops._stream(x)))
    assert pkg.ops.workspace_status(ws) == 0
    assert torch.equal(y, want)


def test_router_ties_pick_lower_ids(pkg, dev):
    x = torch.zeros((4, 512), dtype=torch.bfloat16, device=dev)
    w = torch.randn((64, 512), device=dev)
    idx, wts = pkg.ops.router_topk(x, w, 4)
    assert idx.cpu().tolist() == [[0, 1, 2, 3]] * 4
    assert torch.allclose(wts, torch.full_like(wts, 0.25))


# ------------------------------------------------------- dispatch
@pytest.mark.parametrize("n,E", [(0, 8), (1, 1), (5, 3), (512, 128), (1000, 7), (4096, 128),
                                 (20480, 512), (32768, 128), (33000, 1024)])
def test_dispatch_is_stable_argsort(pkg, orc, dev, n, E):
    rng = np.random.default_rng(n + E)
    ids = rng.integers(0, E, n).astype(np.int32)
    if n > 100:
        ids[: n // 3] = E - 1  # a heavy expert spanning several workgroups
    counts, offsets, order, inv = pkg.ops.dispatch(torch.from_numpy(ids).to(dev), E)
    rc, ro, rs, ri = orc.dispatch(ids, E)
    assert np.array_equal(counts.cpu().numpy(), rc)
    assert np.array_equal(offsets.cpu().numpy(), ro)
    assert np.array_equal(order.cpu().numpy(), rs)
    assert np.array_equal(inv.cpu().numpy(), ri)
    assert pkg.ops.workspace_status(order._mlxr_workspace) == 0


def test_dispatch_flags_out_of_range(pkg, dev):
    ids = torch.tensor([0, 3, 9, 1], dtype=torch.int32, device=dev)
    counts, offsets, order, inv = pkg.ops.dispatch(ids, 4)
    assert pkg.ops.workspace_status(order._mlxr_workspace) == 1
    assert counts.cpu().tolist() == [1, 1, 0, 1]
    assert offsets.cpu().tolist()[-1] == 3


# ----------------------------------------------------- gather_qmm
def _qbank(pkg, orc, E, N, K, bits, dev, seed):
    rng = np.random.default_rng(seed)
    w = _bf16(orc, (rng.standard_normal((E, N, K)) * 0.02).astype(np.float32), dev)
    return pkg.ops.quantize(w, 64, bits)


def _close(got, want, what=""):
    got = got.astype(np.float64)
    want = want.astype(np.float64)
    rms = np.sqrt(np.mean(want ** 2)) + 1e-30
    err = np.abs(got - want)
    # bf16 outputs from two fp32 accumulation orders: a couple of ulps
    assert np.all(err <= 2 ** -7 * np.abs(want) + 1e-2 * rms), (what, err.max(), rms)


@pytest.mark.parametrize("bits", [4, 8])
def test_gather_qmm_reference_cases(pkg, orc, dev, bits):
    """quantization.rs:344-421 shapes: M=32, N=64, K=64; (lhs=(0,), rhs=(2,1))
    and (x batch 5, lhs=(0,2), rhs=(2,1))."""
    wq, sc, bi = _qbank(pkg, orc, 3, 64, 64, bits, dev, 11)
    rng = np.random.default_rng(12)
    for xb, lhs in [(1, [0, 0]), (5, [0, 2])]:
        x = _bf16(orc, rng.standard_normal((xb, 32, 64)).astype(np.float32), dev)
        l_t = torch.tensor(lhs, dtype=torch.int32, device=dev)
        r_t = torch.tensor([2, 1], dtype=torch.int32, device=dev)
        got = pkg.ops.gather_qmm(x, wq, sc, bi, l_t, r_t, True, 64, bits)
        assert tuple(got.shape) == (2, 32, 64)
        want = orc.gather_qmm(_np(orc, x), _np(orc, wq), _np(orc, sc), _np(orc, bi), [2, 1],
                              lhs, bits=bits, tiled=pkg.ops.gather_qmm_tiled(2 * 32, 3))
        _close(orc.bf16_to_f32(_np(orc, got)), orc.bf16_to_f32(want), (xb, bits))
        # gather_mm of the dequantised weights (fp64) as a second reference
        wd = orc.bf16_to_f32(_np(orc, pkg.ops.dequantize(wq, sc, bi, 64, bits))).astype(np.float64)
        xf = orc.bf16_to_f32(_np(orc, x)).astype(np.float64)
        mm = np.stack([xf[lhs[i]] @ wd[[2, 1][i]].T for i in range(2)])
        _close(orc.bf16_to_f32(_np(orc, got)), mm, "gather_mm")


@pytest.mark.parametrize("T,K,E,N,Kd,bits", [
    (1, 8, 128, 768, 2048, 4), (64, 8, 128, 768, 2048, 4), (64, 8, 128, 2048, 768, 4),
    (16, 2, 8, 256, 512, 4), (32, 8, 128, 1536, 4096, 8), (7, 10, 512, 512, 2048, 4),
    (300, 8, 16, 128, 256, 4), (40, 1, 2, 64, 64, 8),
    # many rows per expert: the M-tiled prefill kernel, ragged last tiles
    (1024, 4, 8, 256, 512, 8), (600, 8, 32, 384, 1024, 4),
    # 256-row M-tiles (experts averaging >= 192 rows)
    (2048, 2, 16, 256, 512, 4), (2048, 2, 16, 320, 1024, 8),
    # 128-row narrow tiles (128 columns) with a half last N-tile, and
    # 64-row tiles (256 columns) with a quarter last N-tile
    (1200, 4, 32, 320, 512, 4), (1024, 4, 100, 320, 512, 4),
    # more than 1024 ids (the multi-kernel dispatch) on the decode kernels:
    # its work list, long-form items first
    (200, 8, 128, 768, 2048, 4), (160, 8, 128, 256, 1024, 8)])
def test_gather_qmm_moe_unsorted_shapes(pkg, orc, dev, T, K, E, N, Kd, bits):
    """x [T, 1, 1, Kd] against indices [T, K] -> [T, K, 1, N]."""
    wq, sc, bi = _qbank(pkg, orc, E, N, Kd, bits, dev, T + E)
    rng = np.random.default_rng(T * 3 + K)
    x = _bf16(orc, rng.standard_normal((T, 1, 1, Kd)).astype(np.float32), dev)
    idx = rng.integers(0, E, (T, K)).astype(np.int32)
    if T > 4:
        idx[: T // 2, 0] = 3 % E  # one expert with many rows
    got = pkg.ops.gather_qmm(x, wq, sc, bi, None, torch.from_numpy(idx).to(dev), True, 64, bits)
    assert tuple(got.shape) == (T, K, 1, N)
    tiled = pkg.ops.gather_qmm_tiled(T * K, E)
    want = orc.gather_qmm(_np(orc, x).reshape(T, 1, Kd), _np(orc, wq), _np(orc, sc),
                          _np(orc, bi), idx.reshape(-1), bits=bits, nthreads=16, tiled=tiled)
    _close(orc.bf16_to_f32(_np(orc, got)).reshape(T * K, N),
           orc.bf16_to_f32(want).reshape(T * K, N), (T, K, E, N, Kd, bits))


@pytest.mark.parametrize("bits", [4, 16])
def test_gather_lhs_rows_beyond_gathered_count(pkg, orc, dev, bits):
    """lhs indices may pick x rows past B * M (x batch 20 x M 64 rows, B = 8
    gathers): the M-tiled kernel must bound x by x's own rows.  Regression
    test: it once bounded x by B * M rows and read zeros past them."""
    E, N, Kd, xb, M, B = 2, 128, 256, 20, 64, 8
    assert pkg.ops.gather_qmm_tiled(B * M, E)
    rng = np.random.default_rng(50 + bits)
    x = _bf16(orc, rng.standard_normal((xb, M, Kd)).astype(np.float32), dev)
    lhs = [19, 18, 0, 12, 19, 5, 17, 3]
    rhs = [1, 0, 0, 1, 1, 0, 1, 0]
    lt = torch.tensor(lhs, dtype=torch.int32, device=dev)
    rt = torch.tensor(rhs, dtype=torch.int32, device=dev)
    if bits == 16:
        w = _bf16(orc, (0.05 * rng.standard_normal((E, N, Kd))).astype(np.float32), dev)
        got = pkg.ops.gather_mm(x, w, lt, rt)
        want = orc.gather_mm(_np(orc, x), _np(orc, w), rhs, lhs)
    else:
        wq, sc, bi = _qbank(pkg, orc, E, N, Kd, bits, dev, 51)
        got = pkg.ops.gather_qmm(x, wq, sc, bi, lt, rt, True, 64, bits)
        want = orc.gather_qmm(_np(orc, x), _np(orc, wq), _np(orc, sc), _np(orc, bi), rhs, lhs,
                              bits=bits, tiled=True)
    assert tuple(got.shape) == (B, M, N)
    _close(orc.bf16_to_f32(_np(orc, got)), orc.bf16_to_f32(want), bits)


def test_gather_qmm_out_of_range_index(pkg, orc, dev):
    wq, sc, bi = _qbank(pkg, orc, 4, 64, 64, 4, dev, 3)
    x = torch.ones((3, 1, 64), dtype=torch.bfloat16, device=dev)
    idx = torch.tensor([1, 7, 2], dtype=torch.int32, device=dev)
    got = pkg.ops.gather_qmm(x, wq, sc, bi, None, idx)
    assert pkg.ops.workspace_status(got._mlxr_workspace) == 1
    assert torch.all(got[1] == 0)
    ok = pkg.ops.gather_qmm(x[[0, 2]], wq, sc, bi, None, idx[[0, 2]])
    assert torch.equal(got[[0, 2]], ok)


# ----------------------------------------------- gather_mm (dense bf16)
def test_gather_mm_reference_example(pkg, dev):
    """arithmetic.rs:1565-1575 at the kernels' 64-multiple sizes: a = ones
    [5, 64, 64], b = ones [3, 64, 64], lhs (0, 2), rhs (2, 1) -> all 64."""
    a = torch.ones((5, 64, 64), dtype=torch.bfloat16, device=dev)
    b = torch.ones((3, 64, 64), dtype=torch.bfloat16, device=dev)
    lhs = torch.tensor([0, 2], dtype=torch.int32, device=dev)
    rhs = torch.tensor([2, 1], dtype=torch.int32, device=dev)
    out = pkg.ops.gather_mm(a, b, lhs, rhs)
    assert tuple(out.shape) == (2, 64, 64)
    assert torch.all(out.float() == 64.0)


@pytest.mark.parametrize("T,K,E,N,Kd", [
    (1, 8, 128, 768, 2048), (64, 8, 128, 2048, 768), (7, 10, 512, 512, 2048),
    (300, 8, 16, 128, 256), (40, 1, 2, 64, 64), (1024, 4, 8, 256, 512),
    (600, 8, 32, 384, 1024), (5, 8, 256, 1024, 4096)])
def test_gather_mm_moe_shapes(pkg, orc, dev, T, K, E, N, Kd):
    """SwitchLinear::apply (switch.rs:84-93): x [T, 1, 1, Kd] against
    indices [T, K] -> [T, K, 1, N], against the oracle's gather_mm (f32
    accumulation in another order: the bf16 outputs agree within the
    block tolerance)."""
    print(f"  gather_mm T={T} K={K} E={E} N={N} Kd={Kd}", flush=True)
    rng = np.random.default_rng(T * 7 + E)
    w = _bf16(orc, (0.05 * rng.standard_normal((E, N, Kd))).astype(np.float32), dev)
    x = _bf16(orc, rng.standard_normal((T, 1, 1, Kd)).astype(np.float32), dev)
    idx = rng.integers(0, E, (T, K)).astype(np.int32)
    if T > 4:
        idx[: T // 2, 0] = 3 % E  # one expert with many rows
    lin = pkg.nn.SwitchLinear(w)
    got = lin.apply(x, torch.from_numpy(idx).to(dev))
    assert tuple(got.shape) == (T, K, 1, N)
    want = orc.gather_mm(_np(orc, x).reshape(T, 1, Kd), _np(orc, w), idx.reshape(-1),
                         nthreads=16)
    _close(orc.bf16_to_f32(_np(orc, got)).reshape(T * K, N),
           orc.bf16_to_f32(want).reshape(T * K, N), (T, K, E, N, Kd))


def test_gather_mm_edge_cases(pkg, orc, dev):
    """Empty index lists give empty outputs; an out-of-range expert id
    leaves its rows zero and sets the workspace status (the reference raises
    at eval time instead); the other rows are unaffected."""
    rng = np.random.default_rng(45)
    w = _bf16(orc, (0.05 * rng.standard_normal((4, 64, 128))).astype(np.float32), dev)
    x = _bf16(orc, rng.standard_normal((3, 1, 128)).astype(np.float32), dev)
    empty = pkg.ops.gather_mm(x, w, None, torch.zeros((0, 1), dtype=torch.int32, device=dev))
    assert tuple(empty.shape) == (0, 1, 1, 64)
    idx = torch.tensor([1, 9, 2], dtype=torch.int32, device=dev)
    got = pkg.ops.gather_mm(x, w, None, idx)
    assert pkg.ops.workspace_status(got._mlxr_workspace) == 1
    assert torch.all(got[1] == 0)
    ok = pkg.ops.gather_mm(x[[0, 2]], w, None, idx[[0, 2]])
    assert pkg.ops.workspace_status(ok._mlxr_workspace) == 0
    assert torch.equal(got[[0, 2]], ok)


@pytest.mark.parametrize("bits", [4, 8])
def test_gather_mm_is_tiled_gather_qmm_of_dequant(pkg, orc, dev, bits):
    """quantization.rs:344-421: gather_qmm(x, w) == gather_mm(x,
    dequantize(w)).  Where gather_qmm runs the M-tiled kernel (weights
    dequantised to bf16 tiles) the two calls multiply the same bf16 values
    in the same order: bit for bit."""
    E, N, Kd, T, K = 8, 256, 512, 1024, 4
    assert pkg.ops.gather_qmm_tiled(T * K, E)
    wq, sc, bi = _qbank(pkg, orc, E, N, Kd, bits, dev, 40 + bits)
    wd = pkg.ops.dequantize(wq, sc, bi, 64, bits)
    rng = np.random.default_rng(41)
    x = _bf16(orc, rng.standard_normal((T, 1, 1, Kd)).astype(np.float32), dev)
    idx = torch.from_numpy(rng.integers(0, E, (T, K)).astype(np.int32)).to(dev)
    q = pkg.ops.gather_qmm(x, wq, sc, bi, None, idx, True, 64, bits)
    m = pkg.ops.gather_mm(x, wd.reshape(E, N, Kd), None, idx)
    assert torch.equal(q, m)


@pytest.mark.parametrize("T,E", [(1, 256), (40, 256), (1024, 128), (2048, 256)])
def test_router_topk_bf16_linear_bit_exact(pkg, orc, dev, T, E):
    """A bf16 Linear router (an unquantised checkpoint's mlp.gate): bf16
    logits in the lane order (the matrix-core order from 2048 tokens), top-K
    on the bf16 probabilities, bit for bit, through each logits kernel."""
    rng = np.random.default_rng(T + E)
    d, K = 2048, 8
    x = _bf16(orc, rng.standard_normal((T, d)).astype(np.float32), dev)
    w = _bf16(orc, (rng.standard_normal((E, d)) * 0.05).astype(np.float32), dev)
    idx, wts = pkg.ops.router_topk_quantized(x, pkg.nn.Linear(w), K)
    lg = orc.router_logits_q(_np(orc, x), _np(orc, w), None, None, 16,
                             mfma=pkg.ops.router_matrix_order(T, d, E))
    ridx, rw = orc.router_topk_bf16(lg, K)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    assert np.array_equal(wts.cpu().numpy(), rw)


# ------------------------------------------------------- rms_norm
@pytest.mark.parametrize("T,d", [(1, 2048), (37, 2048), (300, 4096), (5, 516), (3, 6148)])
def test_rms_norm_bit_exact(pkg, orc, dev, T, d):
    """fast::rms_norm (layers/normalization.rs:272-276): bit for bit
    against the oracle (rows held in registers up to d = 4096; d = 6148
    takes the two-pass loop)."""
    rng = np.random.default_rng(T + d)
    x = _bf16(orc, (3 * rng.standard_normal((T, d))).astype(np.float32), dev)
    w = _bf16(orc, (1 + 0.2 * rng.standard_normal(d)).astype(np.float32), dev)
    got = pkg.nn.RmsNorm(w, 1e-6)(x)
    assert np.array_equal(_np(orc, got), orc.rms_norm(_np(orc, x), _np(orc, w), 1e-6))


# -------------------------------------------------------- combine
def test_combine_bit_exact(pkg, orc, dev):
    rng = np.random.default_rng(13)
    T, K, d = 33, 8, 2048
    y = _bf16(orc, rng.standard_normal((T, K, d)).astype(np.float32), dev)
    w = torch.from_numpy(rng.random((T, K)).astype(np.float32)).to(dev)
    got = pkg.ops.combine(y, w).cpu().numpy()
    assert np.array_equal(got, orc.combine(_np(orc, y), w.cpu().numpy()))
    sy = _bf16(orc, rng.standard_normal((T, d)).astype(np.float32), dev)
    sl = torch.from_numpy(rng.standard_normal(T).astype(np.float32)).to(dev)
    got = pkg.ops.combine(y, w, sy, sl).cpu().numpy()
    want = orc.combine(_np(orc, y), w.cpu().numpy(), _np(orc, sy), sl.cpu().numpy())
    assert np.allclose(got, want, rtol=1e-6, atol=1e-6)


# ------------------------------------------- argpartition / softmax
def test_argpartition_and_softmax(pkg, dev):
    a = torch.randn((37, 128), device=dev)
    a[0, 5] = a[0, 9]  # a tie
    for kth in (-8, 0, 64, 127):
        p = pkg.ops.argpartition_axis(a, kth, -1).long()
        vals = torch.gather(a, 1, p)
        k = kth % 128
        assert torch.all(vals[:, :k] <= vals[:, k:k + 1])
        assert torch.all(vals[:, k + 1:] >= vals[:, k:k + 1])
        assert torch.equal(p.sort(1).values, torch.arange(128, device=dev).expand(37, 128))
    pt = pkg.ops.argpartition_axis(a.t().contiguous(), 3, 0)
    assert pt.shape == (128, 37)
    s = pkg.ops.softmax_axis(a, -1, True)
    assert torch.allclose(s, torch.softmax(a, -1), rtol=1e-5, atol=1e-7)
    with pytest.raises(pkg.MlxrMoeError):
        pkg.ops.argpartition_axis(a, 128, -1)


# ------------------------------------------------------- read probe
def test_profile_read_times_one_launch_per_call(pkg, dev):
    """The plain read of the bench's read ceiling: one profiled launch per
    call, a positive time, the buffer unchanged, the sink written only on
    the sentinel (never for this data)."""
    C = pkg._capi
    lib = C.lib()
    buf = torch.arange(1 << 20, dtype=torch.int32, device=dev)  # 4 MiB
    keep = buf.clone()
    sink = torch.full((1,), 7, dtype=torch.int32, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    C.check(lib.mlxr_moe_profile_start(b"read_probe"))
    for _ in range(3):
        C.check(lib.mlxr_moe_profile_read(buf.data_ptr(), buf.numel() * 4, sink.data_ptr(),
                                          stream))
    n = ctypes.c_int64()
    tot, mn, mx = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
    C.check(lib.mlxr_moe_profile_stop(ctypes.byref(n), ctypes.byref(tot), ctypes.byref(mn),
                                      ctypes.byref(mx)))
    assert n.value == 3 and 0.0 < mn.value <= mx.value
    torch.cuda.synchronize(dev)
    assert torch.equal(buf, keep)
    assert sink.item() == 7
