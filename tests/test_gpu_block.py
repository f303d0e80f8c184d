"""GPU parity of the whole MoE block (Qwen35MoeBlock::forward) and of
SplitSwitchFfn against the CPU oracle on the benchmark configurations.

Bar: routing indices bit-exact; routing weights to 2e-6 relative (bit-exact
with a quantised router, whose weights are bf16); max |out - oracle| <=
2e-2 * RMS(oracle) with f32 accumulation.  A quantised router makes the
output bf16, and the GPU's and the oracle's f32 sums (in different orders)
can round to neighbouring bf16 values, so there each element may also
differ by one bf16 step of the oracle's value.  Every point prints (and,
with MLXR_PARITY_LOG set, logs) its max|err|/RMS and the count of elements
past 2e-2 * RMS; that count is held to the measured figure in PAST_BAR
(zero for the points it does not list)."""
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))

_WEIGHTS = {}


def weights(pkg, cfg_name, dev):
    if cfg_name not in _WEIGHTS:
        _WEIGHTS.clear()  # keep one config resident at a time
        torch.cuda.empty_cache()
        _WEIGHTS[cfg_name] = pkg.workloads.make_weights(pkg.workloads.CONFIGS[cfg_name], dev)
    return _WEIGHTS[cfg_name]


# Elements past the literal bar max|err| <= 2e-2 * RMS, per point, as measured
# on the MI355X (the rest of the points have none).  Each such element is
# within one step of a bf16 value it depends on: an intermediate (a SwiGLU
# activation or an expert row y_k, rounded the other way because the GPU's
# and the oracle's f32 sums run in different orders; f32-output blocks) or
# the bf16 output itself (a bf16 block: an element near 4*RMS has a step of
# ~3% of RMS).  The test holds each point to its measured count.
PAST_BAR = {
    "c4_e512_top10_shared T=64": 1, "c4_e512_top10_shared T=512": 1,
    "c4_e512_top10_shared T=2048": 3,
    "c6_qwen3_6_35b_a3b_q8router T=9": 1, "c6_qwen3_6_35b_a3b_q8router T=64": 2,
    "c6_qwen3_6_35b_a3b_q8router T=512": 2, "c6_qwen3_6_35b_a3b_q8router T=2048": 13,
    "c8_qwen3_6_35b_a3b_bf16 T=512": 1, "c8_qwen3_6_35b_a3b_bf16 T=2048": 11,
}


def router_mfma(pkg, cfg, T):
    """Whether the block's router sums its logits in the matrix-core order
    at T tokens (the library's own choice; the oracle then follows).  A
    shared expert's gate is one more logit column of the same pass."""
    return pkg.ops.router_matrix_order(T, cfg.d, cfg.E + (1 if cfg.fs else 0))


def record_parity(name, T, got, ref, rms, allowed=None):
    """Print the parity figures of one block point (max|err|/RMS, the count
    of elements past 2e-2 * RMS, p99.9 |err|/RMS) and, when MLXR_PARITY_LOG
    names a file, append them there as a JSON line."""
    import json
    import os
    diff = np.abs(np.asarray(got, np.float64) - np.asarray(ref, np.float64))
    rec = {"point": f"{name} T={T}", "max_err_over_rms": float(diff.max() / rms),
           "past_bar": int((diff > 2e-2 * rms).sum()), "elements": int(diff.size),
           "p999_over_rms": float(np.quantile(diff, 0.999) / rms)}
    if allowed is not None:
        rec["past_bar_allowed"] = allowed
    print("  PARITY " + json.dumps(rec), flush=True)
    path = os.environ.get("MLXR_PARITY_LOG")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(rec) + "\n")
    return rec


def check_gemma(pkg, orc, bw, x, nthreads=16):
    """gemma4 routed MoE (router + PackedSwitchFfn<Geglu>) against the
    oracle: routing bit-exact (indices and bf16 weights), bf16 out within
    2e-2 * RMS plus one bf16 step."""
    block = bw.block()
    out = block(x)
    torch.cuda.synchronize()
    T, cfg = x.shape[0], bw.cfg
    print(f"  gemma block {cfg.name} T={T}", flush=True)
    r = block.router
    ridx, rw = orc.gemma_router(orc.to_np(x), orc.to_np(r.norm_weight), r.eps, orc.to_np(r.proj),
                                orc.to_np(r.per_expert_scale), cfg.K,
                                mfma=pkg.ops.router_matrix_order(x.shape[0], cfg.d, cfg.E))
    assert np.array_equal(block.last_indices.cpu().numpy(), ridx), "routing indices differ"
    assert np.array_equal(orc.to_np(block.last_weights), rw)
    m = bw.switch_mlp
    q = orc.qlinear_np
    tiled = pkg.ops.gather_qmm_tiled(T * cfg.K, cfg.E)
    ref = orc.packed_switch_glu(orc.to_np(x), q(m.gate_up_proj), q(m.down_proj), ridx,
                                orc.bf16_to_f32(rw), act=1, w_bf16=True, tiled=tiled,
                                nthreads=nthreads)
    got = orc.bf16_to_f32(orc.to_np(out)).astype(np.float64)
    ref = orc.bf16_to_f32(ref).astype(np.float64)
    rms = np.sqrt(np.mean(ref ** 2))
    diff = np.abs(got - ref)
    print(f"  max|err| {diff.max():.3e}  rms {rms:.3e}", flush=True)
    rec = record_parity(cfg.name, T, got, ref, rms, PAST_BAR.get(f"{cfg.name} T={T}", 0))
    a = np.abs(ref)
    ulp = np.where(a > 0, 2.0 ** (np.floor(np.log2(np.maximum(a, 1e-38))) - 7), 0.0)
    assert np.all(diff <= 2e-2 * rms + ulp)
    assert rec["past_bar"] <= rec["past_bar_allowed"]
    assert pkg.ops.workspace_status(block.last_workspace) == 0


def _step(a):
    """One bf16 step (ulp) at each value of a (0 at 0)."""
    a = np.abs(np.asarray(a, np.float64))
    return np.where(a > 0, 2.0 ** (np.floor(np.log2(np.maximum(a, 1e-38))) - 7), 0.0)


def flip_allowance(pkg, orc, bw, x, ridx, rw, tiled, nthreads=16):
    """Per-element bound on what one-step flips of the block's bf16
    intermediates can move the f32 output by: sum_k |w_k| step(y_k) +
    sigmoid(g) step(y_s), from the oracle's own y [T, K, d] and shared y_s.
    Two implementations of the same op sequence whose f32 sums run in
    different orders round a small fraction of those bf16 values to
    neighbouring steps; at large T some fall on the largest values, and one
    step of a shared-expert output near 0.5 alone is ~2% of the block's RMS."""
    cfg, p = bw.cfg, orc.block_params(bw)
    T = x.shape[0]
    xs = orc.to_np(x)[:, None, :]
    ids = ridx.reshape(-1)
    gq = lambda a, t, i, tl: orc.gather_qmm(a, *t, i, bits=cfg.bits, nthreads=nthreads,  # noqa
                                            tiled=tl)
    a = orc.swiglu(gq(xs, p["gate"], ids, tiled[0]), gq(xs, p["up"], ids, tiled[0]))
    y = orc.bf16_to_f32(gq(a, p["down"], ids, tiled[0])).reshape(T, cfg.K, -1)
    bound = np.einsum("tk,tkd->td", np.abs(rw.astype(np.float64)), _step(y))
    if cfg.fs:
        z = np.zeros(T, np.int32)
        sa = orc.swiglu(gq(xs, p["shared_gate"], z, tiled[1]), gq(xs, p["shared_up"], z, tiled[1]))
        ys = orc.bf16_to_f32(gq(sa, p["shared_down"], z, tiled[1])).reshape(T, -1)
        if "shared_gate_q" in p:  # quantised shared gate (bf16 block)
            wq, sc, bi = p["shared_gate_q"]
            row = lambda a: None if a is None else a.reshape(1, -1)  # noqa: E731
            sl = orc.router_logits_q(orc.to_np(x), row(wq), row(sc), row(bi), cfg.router_bits,
                                     mfma=router_mfma(pkg, cfg, T))
        else:
            sl = orc.router_logits(orc.to_np(x), p["shared_gate_w"],
                                   mfma=router_mfma(pkg, cfg, T))
        sl = sl[:, 0].astype(np.float64)
        bound += (1.0 / (1.0 + np.exp(-sl)))[:, None] * _step(ys)
    return bound


def check_block(pkg, orc, bw, x, nthreads=16):
    if bw.cfg.layout == "gemma":
        return check_gemma(pkg, orc, bw, x, nthreads)
    block = bw.block()
    out = block(x)
    torch.cuda.synchronize()
    print(f"  block {bw.cfg.name} T={x.shape[0]}", flush=True)
    T, cfg = x.shape[0], bw.cfg
    # the gather_qmm numerics the library picks for each GEMM set
    tiled = (pkg.ops.gather_qmm_tiled(T * cfg.K, cfg.E), pkg.ops.gather_qmm_tiled(T, 1))
    ref, ridx, rw = orc.block_forward(orc.block_params(bw), orc.to_np(x), nthreads=nthreads,
                                      tiled=tiled, router_mfma=router_mfma(pkg, cfg, T))
    idx = block.last_indices.cpu().numpy()
    assert np.array_equal(idx, ridx), "routing indices differ"
    if cfg.router_bits:
        # bf16 block: bf16 routing weights, bit for bit; bf16 out
        assert out.dtype == torch.bfloat16
        assert np.array_equal(block.last_weights.cpu().numpy(), rw)
        got = orc.bf16_to_f32(orc.to_np(out)).astype(np.float64)
        ref = orc.bf16_to_f32(ref)
    else:
        assert np.allclose(block.last_weights.cpu().numpy(), rw, rtol=2e-6, atol=1e-7)
        got = out.cpu().numpy().astype(np.float64)
    rms = np.sqrt(np.mean(ref.astype(np.float64) ** 2))
    diff = np.abs(got - ref)
    err = diff.max()
    print(f"  max|err| {err:.3e}  rms {rms:.3e}  ratio {err / rms:.2e}", flush=True)
    rec = record_parity(cfg.name, T, got, ref, rms, PAST_BAR.get(f"{cfg.name} T={T}", 0))
    assert rec["past_bar"] <= rec["past_bar_allowed"]
    if cfg.router_bits:
        # bf16 block: past the bar by one step of the output element, or
        # where a one-step flip of a bf16 row the element sums (a routed y
        # or the shared expert's row) is carried through the bf16 combine,
        # by that row's step bound as well
        step = _step(ref)
        over = diff > 2e-2 * rms + step
        if over.any():
            allow = flip_allowance(pkg, orc, bw, x, ridx, rw, tiled, nthreads)
            print(f"  {int(over.sum())} elements past 2e-2*rms + one output step; max excess / "
                  f"flip bound {((diff - 2e-2 * rms - step) / allow)[over].max():.2f}",
                  flush=True)
            assert np.all(diff <= 2e-2 * rms + step + allow)
    elif err > 2e-2 * rms:
        # Past the bar only through one-step flips of bf16 intermediates
        # (as many elements as PAST_BAR lists), each within the bar plus the
        # step bound of the branch values it sums (the oracle's own).
        over = diff > 2e-2 * rms
        allow = flip_allowance(pkg, orc, bw, x, ridx, rw, tiled, nthreads)
        print(f"  {int(over.sum())} of {over.size} elements past 2e-2*rms; "
              f"max excess / flip bound {((diff - 2e-2 * rms) / allow)[over].max():.2f}",
              flush=True)
        assert np.all(diff <= 2e-2 * rms + allow)
    # the bulk of the elements sit well inside the bar
    q = np.quantile(diff, 0.999)
    print(f"  p99.9 |err| / rms {q / rms:.2e}", flush=True)
    assert q <= 1e-2 * rms
    assert pkg.ops.workspace_status(block.last_workspace) == 0
    return out, block


def test_c1_golden_fixture(pkg, orc, dev):
    """The committed c1 fixture (tests/golden/c1_block.npz), inputs rebuilt
    from numpy's seed-0 stream and uploaded as-is (no GPU quantisation)."""
    from make_golden import c1_inputs, digest
    z = np.load(Path(__file__).resolve().parent / "golden" / "c1_block.npz")
    x, p, dense = c1_inputs()
    assert digest(x) == str(z["x_sha"])
    assert digest(*p["gate"], *p["up"], *p["down"]) == str(z["packed_sha"])
    t = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a).view(dt)).to(dev)  # noqa: E731

    def bank(q):
        return pkg.nn.QuantizedSwitchLinear(t(q[0], np.int32), t(q[1], np.int16).view(torch.bfloat16),
                                            t(q[2], np.int16).view(torch.bfloat16), 64, 4)

    mlp = pkg.nn.SplitSwitchFfn(bank(p["gate"]), bank(p["up"]), bank(p["down"]))
    block = pkg.nn.Qwen35MoeBlock(t(p["router_w"], np.float32), mlp, 2)
    xt = t(x, np.int16).view(torch.bfloat16)
    out = block(xt).cpu().numpy()
    assert np.array_equal(block.last_indices.cpu().numpy(), z["idx"])
    assert np.allclose(block.last_weights.cpu().numpy(), z["weights"], rtol=2e-6)
    rms = np.sqrt(np.mean(z["out"].astype(np.float64) ** 2))
    assert np.abs(out - z["out"]).max() <= 2e-2 * rms
    # and the GPU quantiser reproduces the fixture's packed weights
    for name in ("gate", "up", "down"):
        wq, sc, bi = pkg.ops.quantize(t(dense[name], np.int16).view(torch.bfloat16), 64, 4)
        assert np.array_equal(orc.to_np(wq), p[name][0])
        assert np.array_equal(orc.to_np(sc), p[name][1])


# Besides the bench points: T = 2, 3, 5 on the streaming kernel with
# K-slices (4, 2, 1 of them as the grid grows), c5 T=1 and 4 (8-bit
# K-slices), c4/c6 at T = 3 and 9 (the folded shared expert with a partial
# item of rows; 9 > 8 rows: two shared items).  c4 and c6 at T = 2048 and
# c6 at T = 512 fold the shared expert into the M-tiled launches (c8: dense
# weights); c4 at T = 512 does not (10 routed rows per expert stay on the
# streaming kernel, the shared expert's 512 rows are M-tiled).  c2 at
# T = 256 (16 rows per expert) and c5 at T = 256 are M-tiled, c2 at T = 240
# (15) is not.
@pytest.mark.parametrize("cfg,T", [("c1", 16), ("c2", 1), ("c2", 2), ("c2", 3), ("c2", 5),
                                   ("c2", 8), ("c2", 32), ("c2", 64), ("c2", 240),
                                   ("c2", 256), ("c5", 256),
                                   ("c5", 1), ("c5", 4), ("c5", 32), ("c5", 512),
                                   ("c4", 1), ("c4", 3), ("c4", 9), ("c4", 64), ("c4", 512),
                                   ("c4", 2048),
                                   ("c3", 512), ("c3", 2048), ("c3", 4096),
                                   ("c6", 1), ("c6", 3), ("c6", 9), ("c6", 64),
                                   ("c6", 512), ("c6", 2048), ("c7", 1), ("c7", 64),
                                   ("c7", 512), ("c7", 2048), ("c8", 1), ("c8", 64),
                                   ("c8", 512), ("c8", 2048)])
def test_block_parity(pkg, orc, dev, cfg, T):
    """Every benchmark configuration (c1-c5) at every token count the bench
    reports, plus the Qwen3.6 (c6, c8) and gemma4 (c7) layouts."""
    bw = weights(pkg, cfg, dev)
    x = pkg.workloads.make_x(bw.cfg, T, dev, seed=T)
    check_block(pkg, orc, bw, x)


@pytest.mark.parametrize("T", [1, 64, 600])
def test_gemma_dense_experts(pkg, orc, dev, T):
    """gemma4's layout with unquantised experts: PackedSwitchFfn over dense
    bf16 gate_up [E, 2H, d] and down (gather_mm), GeGLU, gemma router."""
    W = pkg.workloads
    cfg = W.MoEConfig("gemma_dense", d=1024, E=32, K=4, f=512, bits=16, router_bits=16,
                      layout="gemma", tokens=(T,))
    bw = W.make_weights(cfg, dev)
    x = W.make_x(cfg, T, dev, seed=T)
    check_block(pkg, orc, bw, x)


def test_dense_block_equals_dequantised_4bit_block(pkg, dev):
    """The c1 block with its 4-bit experts replaced by their bf16
    dequantisation (dense SwitchLinear / Linear, gather_mm) gives the 4-bit
    block's output bit for bit where the 4-bit GEMMs run the M-tiled kernel
    (weights dequantised to bf16 tiles): T = 4096 over 8 experts."""
    W = pkg.workloads
    cfg = W.MoEConfig("c1_shared", d=512, E=8, K=2, f=256, fs=256, tokens=(4096,))
    bw = W.make_weights(cfg, dev)
    T = 4096
    assert pkg.ops.gather_qmm_tiled(T * cfg.K, cfg.E) and pkg.ops.gather_qmm_tiled(T, 1)
    x = W.make_x(cfg, T, dev, seed=7)
    q = bw.block()
    nn = pkg.nn

    def dq(lin):
        E, N = lin.weight.shape[0], lin.weight.shape[1]
        w = pkg.ops.dequantize(lin.weight, lin.scales, lin.biases, 64, lin.bits)
        return nn.SwitchLinear(w.reshape(E, N, -1))

    m = bw.switch_mlp
    mlp = nn.SplitSwitchFfn(dq(m.gate_proj), dq(m.up_proj), dq(m.down_proj))
    s = bw.shared_expert
    shared = nn.SwigluMlp(*(nn.Linear(dq(lin).weight[0])
                            for lin in (s.gate_proj, s.up_proj, s.down_proj)))
    dense = nn.Qwen35MoeBlock(bw.gate_w, mlp, cfg.K, shared, bw.shared_gate_w, bw.gate_b)
    a = q(x)
    b = dense(x)
    assert torch.equal(q.last_indices, dense.last_indices)
    assert torch.equal(a, b)


@pytest.mark.parametrize("cfg,T", [("c2", 64), ("c6", 1), ("c6", 64), ("c6", 512),
                                   ("c8", 64)])
def test_block_residual_parity(pkg, orc, dev, cfg, T):
    """The decoder layer's MoE half, out = h + block(rms_norm(h))
    (layer.rs:134-138), through mlxr_moe_block_forward_residual: routing
    bit-exact against the oracle, out within the block tolerance (on the
    block's part) plus one step of out's dtype; and bit-identical to the
    same three steps run as separate GPU calls."""
    bw = weights(pkg, cfg, dev)
    c = bw.cfg
    h = pkg.workloads.make_x(c, T, dev, seed=T + 1)
    g = torch.Generator(device=dev).manual_seed(T)
    nw = (1 + 0.1 * torch.randn(c.d, generator=g, device=dev)).to(torch.bfloat16)
    norm = pkg.nn.RmsNorm(nw, 1e-6)
    block = bw.block()
    print(f"  block_residual {c.name} T={T}", flush=True)
    out = block.forward_residual(h, norm)
    idx = block.last_indices.clone()
    # the same steps as separate calls
    m = block(norm(h))
    assert torch.equal(block.last_indices, idx)
    sep = (h + m) if c.router_bits else (h.float() + m)
    assert torch.equal(out, sep)
    tiled = (pkg.ops.gather_qmm_tiled(T * c.K, c.E), pkg.ops.gather_qmm_tiled(T, 1))
    p = orc.block_params(bw)
    ref, ridx, rw = orc.block_forward_residual(p, orc.to_np(nw), 1e-6, orc.to_np(h),
                                               nthreads=16, tiled=tiled,
                                               router_mfma=router_mfma(pkg, c, T))
    assert np.array_equal(idx.cpu().numpy(), ridx)
    mref, _, _ = orc.block_forward(p, orc.rms_norm(orc.to_np(h), orc.to_np(nw), 1e-6),
                                   nthreads=16, tiled=tiled, router_mfma=router_mfma(pkg, c, T))
    if c.router_bits:
        got, ref = orc.bf16_to_f32(orc.to_np(out)), orc.bf16_to_f32(ref)
        mref = orc.bf16_to_f32(mref)
    else:
        got = out.cpu().numpy()
    got, ref = got.astype(np.float64), ref.astype(np.float64)
    rms = np.sqrt(np.mean(mref.astype(np.float64) ** 2))
    a = np.abs(ref)
    step = 2.0 ** (np.floor(np.log2(np.maximum(a, 1e-38))) - (7 if c.router_bits else 23))
    if c.router_bits:
        # the bf16 chain rounds twice: the block's output (where the two
        # f32 sums can round to neighbouring bf16 values), then h + it
        step = step + _step(mref)
    diff = np.abs(got - ref)
    print(f"  max|err| {diff.max():.3e}  block rms {rms:.3e}", flush=True)
    assert np.all(diff <= 2e-2 * rms + step)
    assert pkg.ops.workspace_status(block.last_workspace) == 0


@pytest.mark.parametrize("cfg", ["c6", "c8"])
def test_block_residual_and_norm_empty_input(pkg, dev, cfg):
    """T = 0 through the layer-tail entry and the norm: empty outputs, no
    error, nothing launched that reads the input."""
    bw = weights(pkg, cfg, dev)
    d = bw.cfg.d
    h = torch.empty((0, d), dtype=torch.bfloat16, device=dev)
    norm = pkg.nn.RmsNorm(torch.ones(d, dtype=torch.bfloat16, device=dev))
    out = bw.block().forward_residual(h, norm)
    assert tuple(out.shape) == (0, d)
    assert tuple(norm(h).shape) == (0, d)


def test_block_token_permutation_equivariance(pkg, dev):
    """At full c2 size: permuting tokens permutes output rows bit for bit,
    and repeated runs are bit-identical (size-independent properties)."""
    bw = weights(pkg, "c2", dev)
    T = 64
    x = pkg.workloads.make_x(bw.cfg, T, dev, seed=99)
    block = bw.block()
    a = block(x).clone()
    b = block(x).clone()
    assert torch.equal(a, b)
    perm = torch.randperm(T, generator=torch.Generator().manual_seed(0)).to(dev)
    c = block(x[perm])
    assert torch.equal(c, a[perm])


@pytest.mark.parametrize("cfg", ["c2", "c4", "c6"])
def test_block_routing_counter_in_dirty_reused_workspace(pkg, dev, cfg):
    """Routing of 16 < T tokens whose T*K ids fit one workgroup runs as one
    launch whose last workgroup to finish sorts the ids; it counts finished
    workgroups in the workspace word after the status word, which the logits
    launch clears.  One workspace filled with garbage, then reused for
    forwards of T = 64, 17, 33 and 64 tokens, gives every forward's output,
    indices and weights bit for bit as a zeroed workspace of its own does."""
    bw = weights(pkg, cfg, dev)
    block = bw.block()
    Ts = [64, 17, 33, 64]
    xs = [pkg.workloads.make_x(bw.cfg, T, dev, seed=200 + i) for i, T in enumerate(Ts)]
    ws = pkg.ops.workspace(max(block.workspace_size(T) for T in Ts), dev)
    ws.fill_(0xA5)
    for T, x in zip(Ts, xs):
        ref = block(x, workspace=torch.zeros(block.workspace_size(T), dtype=torch.uint8,
                                             device=dev)).clone()
        ref_i, ref_w = block.last_indices.clone(), block.last_weights.clone()
        got = block(x, workspace=ws)
        assert torch.equal(got, ref), (cfg, T)
        assert torch.equal(block.last_indices, ref_i) and torch.equal(block.last_weights, ref_w)
        assert pkg.ops.workspace_status(ws) == 0


@pytest.mark.parametrize("E,K,T", [(1024, 1, 100), (1024, 4, 256), (1024, 8, 17),
                                   (300, 3, 333)])
def test_block_one_launch_routing_wide_routers(pkg, orc, dev, E, K, T):
    """The one-launch routing (16 < T, T*K <= 1024 ids) at its widest
    router (1024 experts: 16 logits per lane), with one expert per token (a
    workgroup per 4 tokens, up to 84 of them), with exactly 1024 ids, and
    at an expert count off the powers of two.  Indices bit for bit and
    weights to 2e-6 of the oracle's; the output bit for bit equal to the
    switch FFN's forward_with_combine given those indices and weights (its
    sort runs as separate launches)."""
    d, f = 256, 64
    gen = torch.Generator().manual_seed(1000 * K + T)

    def rnd(*shape, sd):
        return (torch.randn(*shape, generator=gen) * sd)

    router = rnd(E, d, sd=0.05).to(dev)
    bf = lambda t: t.to(torch.bfloat16).to(dev)  # noqa: E731
    mlp = pkg.nn.SplitSwitchFfn.from_dense(bf(rnd(E, f, d, sd=0.02)), bf(rnd(E, f, d, sd=0.02)),
                                           bf(rnd(E, d, f, sd=0.02)))
    block = pkg.nn.Qwen35MoeBlock(router, mlp, K)
    x = bf(rnd(T, d, sd=1.0))
    out = block(x).clone()
    idx, wts = block.last_indices.clone(), block.last_weights.clone()
    assert pkg.ops.workspace_status(block.last_workspace) == 0
    xb = x.cpu().view(torch.int16).numpy().view(np.uint16)
    ridx, rw = orc.router_topk(orc.router_logits(xb, router.cpu().numpy(),
                                                 mfma=pkg.ops.router_matrix_order(T, d, E)), K)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    assert np.allclose(wts.cpu().numpy(), rw, rtol=2e-6, atol=0)
    ref = mlp.forward_with_combine(x, idx, wts)
    assert torch.equal(out, ref)


@pytest.mark.parametrize("cfg", ["c2", "c5", "c4", "c6"])
def test_single_token_combine_in_down_launch(pkg, dev, cfg, monkeypatch):
    """At T = 1 the block and SplitSwitchFfn.forward_with_combine sum the
    routed rows inside their down launch; both equal, bit for bit, the
    separate launches of the same routing: the block run with the fusion
    switched off (MLXR_MOE_DOWN_COMBINE=0: routed y and, on c4/c6, the folded
    shared expert's y from the down launch, then the combine op with the
    shared gate logit), and the per-expert rows (SplitSwitchFfn.forward)
    with the combine op."""
    bw = weights(pkg, cfg, dev)
    block = bw.block()
    K, d = bw.cfg.K, bw.cfg.d
    for seed in (11, 12, 13):
        x = pkg.workloads.make_x(bw.cfg, 1, dev, seed=seed)
        print(f"  single-token combine {cfg} seed={seed}", flush=True)
        out = block(x).clone()
        idx, w = block.last_indices.clone(), block.last_weights.clone()
        monkeypatch.setenv("MLXR_MOE_DOWN_COMBINE", "0")
        sep = block(x).clone()
        monkeypatch.delenv("MLXR_MOE_DOWN_COMBINE")
        assert torch.equal(block.last_indices, idx)
        assert out.dtype == sep.dtype and torch.equal(out, sep), seed
        y = bw.switch_mlp.forward(x, idx)
        fused = bw.switch_mlp.forward_with_combine(x, idx, w)
        if not bw.cfg.fs:
            ref = pkg.ops.combine(y.reshape(1, K, d), w.reshape(1, K))
            assert out.dtype == ref.dtype and torch.equal(out, ref), seed
        monkeypatch.setenv("MLXR_MOE_DOWN_COMBINE", "0")
        sep_fwc = bw.switch_mlp.forward_with_combine(x, idx, w)
        monkeypatch.delenv("MLXR_MOE_DOWN_COMBINE")
        assert torch.equal(fused, sep_fwc), seed
        assert torch.equal(fused, pkg.ops.combine(y.reshape(1, K, d), w.reshape(1, K))), seed


@pytest.mark.parametrize("cfg,ids", [("c2", [3, 3, 3, 3, 3, 1, 2, 4]),
                                     ("c2", [7] * 8),
                                     ("c2", [5, 9, 5, 9, 5, 9, 5, 9]),
                                     ("c4", [2] * 10),
                                     ("c4", [4, 4, 4, 4, 4, 4, 1, 1, 1, 0])])
def test_single_token_combine_repeated_ids(pkg, dev, cfg, ids, monkeypatch):
    """forward_with_combine at T = 1 with caller indices that name one
    expert several times: an expert of more than 4 of the K rows runs in the
    8-token MFMA form (and, past 8 rows, in two work items), in the fused
    down + combine launch as in the separate down launch.  Equal bit for bit
    to SplitSwitchFfn.forward followed by the combine op, and to the
    separate launches."""
    bw = weights(pkg, cfg, dev)
    K, d = bw.cfg.K, bw.cfg.d
    assert len(ids) == K
    x = pkg.workloads.make_x(bw.cfg, 1, dev, seed=31)
    idx = torch.tensor([ids], dtype=torch.int32, device=dev)
    g = torch.Generator().manual_seed(5)
    w = torch.rand((1, K), generator=g).to(dev)
    print(f"  repeated ids {cfg} {ids}", flush=True)
    y = bw.switch_mlp.forward(x, idx)
    ref = pkg.ops.combine(y.reshape(1, K, d), w)
    fused = bw.switch_mlp.forward_with_combine(x, idx, w)
    torch.cuda.synchronize()
    # rows of one expert are equal to each other (same x, same weights)
    yr = y.reshape(K, d)
    for k in range(1, K):
        if ids[k] == ids[0]:
            assert torch.equal(yr[k], yr[0])
    assert torch.equal(fused, ref)
    monkeypatch.setenv("MLXR_MOE_DOWN_COMBINE", "0")
    sep = bw.switch_mlp.forward_with_combine(x, idx, w)
    monkeypatch.delenv("MLXR_MOE_DOWN_COMBINE")
    assert torch.equal(fused, sep)


def test_switch_glu_forward_matches_composition(pkg, orc, dev):
    """SplitSwitchFfn::forward (per-expert rows) and forward_with_combine
    against the oracle composition of gather_qmm / swiglu / combine."""
    bw = weights(pkg, "c2", dev)
    cfg = bw.cfg
    T = 24
    x = pkg.workloads.make_x(cfg, T, dev, seed=5)
    g = torch.Generator().manual_seed(3)
    idx = torch.stack([torch.randperm(cfg.E, generator=g)[:cfg.K] for _ in range(T)]).int().to(dev)
    w = torch.rand((T, cfg.K), generator=g).to(dev)
    mlp = bw.switch_mlp
    y = mlp.forward(x, idx)
    out = mlp.forward_with_combine(x, idx, w)
    p = orc.block_params(bw)
    xs = orc.to_np(x)[:, None, :]
    ids = idx.cpu().numpy().reshape(-1)
    tl = pkg.ops.gather_qmm_tiled(T * cfg.K, cfg.E)
    ga = orc.gather_qmm(xs, *p["gate"], ids, nthreads=16, tiled=tl)
    ua = orc.gather_qmm(xs, *p["up"], ids, nthreads=16, tiled=tl)
    ya = orc.gather_qmm(orc.swiglu(ga, ua), *p["down"], ids, nthreads=16,
                        tiled=tl).reshape(T, cfg.K, -1)
    yf = orc.bf16_to_f32(ya).astype(np.float64)
    rms = np.sqrt(np.mean(yf ** 2))
    assert np.abs(orc.bf16_to_f32(orc.to_np(y)) - yf).max() <= 2e-2 * rms
    ref = orc.combine(ya, w.cpu().numpy())
    rms = np.sqrt(np.mean(ref.astype(np.float64) ** 2))
    assert np.abs(out.cpu().numpy() - ref).max() <= 2e-2 * rms


@pytest.mark.parametrize("bits", [4, 8])
def test_switch_glu_tall_prefill_tile(pkg, orc, dev, bits):
    """The 256-row M-tiles of the prefill GEMMs (taken when the experts
    average 192 rows or more: here 4096 rows over 16 experts), gated
    (gate/up with the SwiGLU epilogue) and down, against the oracle's tiled
    gather_qmm numerics, one expert much fuller than the rest."""
    W = pkg.workloads
    cfg = W.MoEConfig("tall_tile", d=512, E=16, K=2, f=512, bits=bits, tokens=(2048,))
    bw = W.make_weights(cfg, dev)
    T = 2048
    assert T * cfg.K >= 192 * cfg.E and pkg.ops.gather_qmm_tiled(T * cfg.K, cfg.E)
    x = W.make_x(cfg, T, dev, seed=21)
    g = torch.Generator().manual_seed(21)
    idx = torch.stack([torch.randperm(cfg.E, generator=g)[:cfg.K] for _ in range(T)]).int()
    idx[: T // 2, 0] = 5  # expert 5: ~1100 rows, several tiles and a ragged last one
    idx[: T // 2, 1] = torch.where(idx[: T // 2, 1] == 5, 6, idx[: T // 2, 1])
    idx = idx.to(dev)
    w = torch.rand((T, cfg.K), generator=g).to(dev)
    print(f"  tall prefill tile bits={bits}", flush=True)
    mlp = bw.switch_mlp
    y = mlp.forward(x, idx)
    out = mlp.forward_with_combine(x, idx, w)
    p = orc.block_params(bw)
    xs = orc.to_np(x)[:, None, :]
    ids = idx.cpu().numpy().reshape(-1)
    ga = orc.gather_qmm(xs, *p["gate"], ids, bits=bits, nthreads=16, tiled=True)
    ua = orc.gather_qmm(xs, *p["up"], ids, bits=bits, nthreads=16, tiled=True)
    ya = orc.gather_qmm(orc.swiglu(ga, ua), *p["down"], ids, bits=bits, nthreads=16,
                        tiled=True).reshape(T, cfg.K, -1)
    yf = orc.bf16_to_f32(ya).astype(np.float64)
    rms = np.sqrt(np.mean(yf ** 2))
    dy = np.abs(orc.bf16_to_f32(orc.to_np(y)).reshape(yf.shape) - yf)
    print(f"  max|y err| {dy.max():.3e}  rms {rms:.3e}  "
          f"{int((dy > 2e-2 * rms).sum())} of {dy.size} past 2e-2*rms", flush=True)
    # bf16 y: one step of the oracle's value where the two f32 sums round
    # apart (a step of a value past ~3 RMS is itself 2e-2 * RMS)
    assert np.all(dy <= 2e-2 * rms + _step(yf))
    assert (dy > 2e-2 * rms).sum() <= 1e-4 * dy.size
    ref = orc.combine(ya, w.cpu().numpy())
    rms = np.sqrt(np.mean(ref.astype(np.float64) ** 2))
    do = np.abs(out.cpu().numpy() - ref)
    flips = np.einsum("tk,tkd->td", np.abs(w.cpu().numpy().astype(np.float64)), _step(yf))
    assert np.all(do <= 2e-2 * rms + flips)
    assert (do > 2e-2 * rms).sum() <= 1e-4 * do.size


def test_checkpoint_round_trip_forward(pkg, orc, dev, tmp_path):
    """A layer written as an mlxr checkpoint (the reference's key names,
    per-path 8-bit overrides for mlp.gate / mlp.shared_expert_gate) and read
    back by the loader runs bit-identically to the block it came from, and
    within tolerance of the oracle."""
    import json
    from safetensors.torch import save_file
    W = pkg.workloads
    cfg = W.MoEConfig("ckpt", d=512, E=8, K=2, f=256, fs=256, router_bits=8, tokens=(16,))
    bw = W.make_weights(cfg, dev)
    p = "model.language_model.layers.5.mlp."
    t = {}

    def put(name, lin, squeeze=False):
        w, s, b = lin.weight, lin.scales, lin.biases
        if squeeze:
            w, s, b = w[0], s[0], b[0]
        t[p + name + ".weight"] = w.contiguous().cpu().view(torch.uint32)
        t[p + name + ".scales"] = s.contiguous().cpu()
        t[p + name + ".biases"] = b.contiguous().cpu()
    m, se = bw.switch_mlp, bw.shared_expert
    put("switch_mlp.gate_proj", m.gate_proj)
    put("switch_mlp.up_proj", m.up_proj)
    put("switch_mlp.down_proj", m.down_proj)
    put("shared_expert.gate_proj", se.gate_proj, True)
    put("shared_expert.up_proj", se.up_proj, True)
    put("shared_expert.down_proj", se.down_proj, True)
    put("gate", bw.gate_w, True)
    put("shared_expert_gate", bw.shared_gate_w, True)
    g = torch.Generator(device=dev).manual_seed(9)
    norm_w = (1 + 0.1 * torch.randn(cfg.d, generator=g, device=dev)).to(torch.bfloat16)
    t["model.language_model.layers.5.post_attention_layernorm.weight"] = norm_w.cpu()
    d = tmp_path / "ck"
    d.mkdir()
    save_file(t, str(d / "model.safetensors"), metadata={"format": "mlx"})
    q = {"group_size": 64, "bits": 4, "mode": "affine",
         "language_model.model.layers.5.mlp.gate": {"group_size": 64, "bits": 8},
         "language_model.model.layers.5.mlp.shared_expert_gate": {"group_size": 64, "bits": 8}}
    (d / "config.json").write_text(json.dumps({"quantization": q,
                                               "text_config": {"num_experts_per_tok": 2,
                                                               "rms_norm_eps": 1e-6}}))
    loaded = pkg.loader.qwen35_moe_block(d, 5, dev)
    x = W.make_x(cfg, 40, dev, seed=3)
    print("  checkpoint round trip T=40", flush=True)
    assert torch.equal(loaded(x), bw.block()(x))
    check_block(pkg, orc, bw, x)
    # the layer tail from the same checkpoint (mlx format: the norm weight as
    # stored)
    norm = pkg.loader.post_attention_layernorm(d, 5, dev)
    assert torch.equal(norm.weight, norm_w)
    assert torch.equal(loaded.forward_residual(x, norm),
                       bw.block().forward_residual(x, pkg.nn.RmsNorm(norm_w, 1e-6)))


@pytest.mark.parametrize("cfg", ["c3", "c5"])
def test_zipf_routing_matches_fixture(pkg, dev, cfg):
    """The Zipf-skewed configurations route as committed: with the fixture's
    router bias, the block's realised per-expert row counts at every bench
    T equal tests/golden/zipf_routing.npz's (the routing itself is
    bit-exact against the oracle in test_block_parity)."""
    bw = weights(pkg, cfg, dev)
    block = bw.block()
    for T in bw.cfg.tokens:
        want = pkg.workloads.zipf_rows(bw.cfg, T)
        assert want is not None, f"no committed row counts for {cfg} T={T}"
        block(pkg.workloads.make_x(bw.cfg, T, dev, seed=T))
        got = torch.bincount(block.last_indices.reshape(-1).long(), minlength=bw.cfg.E)
        print(f"  zipf rows {cfg} T={T}: max {int(got.max())}", flush=True)
        assert np.array_equal(got.cpu().numpy(), want)


# Largest sizes of the suite, sampled: each token's output depends on its own
# row only (routing and every expert product are per token), so the oracle
# runs on a seeded sample of the rows, with the numerics the library picks at
# the full T.  (point, T, sampled tokens, elements past 2e-2 * RMS allowed:
# the measured count, as PAST_BAR)
LARGE_T = [("c2", 16384, 256, 0), ("c6", 8192, 256, 1)]


@pytest.mark.parametrize("cfg,T,n,allowed", LARGE_T)
def test_block_parity_large_T_sampled(pkg, orc, dev, cfg, T, n, allowed):
    """c2 at T = 16384 (131072 routed rows: the three-kernel dispatch, 512
    M-tiles of 256 rows, the largest x, activations and y buffers of the
    suite) and the Qwen3.6 block at T = 8192 (the folded shared expert,
    8-bit router) against the oracle on n of their tokens, the first and the
    last among them: routing bit-exact, values within check_block's bar."""
    bw = weights(pkg, cfg, dev)
    c = bw.cfg
    x = pkg.workloads.make_x(c, T, dev, seed=T)
    block = bw.block()
    print(f"  large T {cfg} T={T}", flush=True)
    out = block(x)
    torch.cuda.synchronize()
    rng = np.random.default_rng(T)
    sel = np.unique(np.concatenate([[0, T - 1], rng.choice(T, n - 2, replace=False)]))
    tiled = (pkg.ops.gather_qmm_tiled(T * c.K, c.E), pkg.ops.gather_qmm_tiled(T, 1))
    ref, ridx, rw = orc.block_forward(orc.block_params(bw), orc.to_np(x)[sel], nthreads=16,
                                      tiled=tiled, router_mfma=router_mfma(pkg, c, T))
    assert np.array_equal(block.last_indices.cpu().numpy()[sel], ridx), "routing indices differ"
    if c.router_bits:
        assert np.array_equal(block.last_weights.cpu().numpy()[sel], rw)
        got = orc.bf16_to_f32(orc.to_np(out)[sel]).astype(np.float64)
        ref = orc.bf16_to_f32(ref).astype(np.float64)
    else:
        assert np.allclose(block.last_weights.cpu().numpy()[sel], rw, rtol=2e-6, atol=1e-7)
        got = out.cpu().numpy()[sel].astype(np.float64)
    rms = np.sqrt(np.mean(ref ** 2))
    diff = np.abs(got - ref)
    rec = record_parity(c.name + " sampled", T, got, ref, rms, allowed)
    if c.router_bits:
        assert np.all(diff <= 2e-2 * rms + _step(ref))
    assert rec["past_bar"] <= rec["past_bar_allowed"]
    assert np.quantile(diff, 0.999) <= 1e-2 * rms
    assert pkg.ops.workspace_status(block.last_workspace) == 0
    del out, block, bw
    torch.cuda.empty_cache()


# Token counts off the benchmark grid, across the launch-shape boundaries:
# the routing kernels (one wave at T*K <= 64, one workgroup at T <= 16,
# top-k + dispatch above), the streaming decode GEMM's K-slices and blocks
# per wave, the switch to the M-tiled GEMM and its tile heights, the router
# logits' per-wave / tiled kernels (4 or 8 tokens per wave) and, on the
# Qwen3.6 block, its shared-gate column folded into the tiled grid or
# launched apart.  Elements past 2e-2 * RMS allowed per point: the measured
# count, as PAST_BAR.
SWEEP = {("c2", 4): 0, ("c2", 17): 0, ("c2", 33): 0, ("c2", 129): 0, ("c2", 257): 0,
         ("c2", 383): 0, ("c2", 777): 0,
         ("c6", 2): 0, ("c6", 17): 0, ("c6", 100): 0, ("c6", 257): 5, ("c6", 300): 2,
         ("c6", 700): 11, ("c6", 1100): 11,
         ("c4", 7): 0, ("c4", 130): 0, ("c4", 1000): 21,
         ("c5", 9): 0, ("c5", 100): 0, ("c5", 300): 0,
         ("c7", 9): 0, ("c7", 200): 0, ("c7", 1000): 0,
         ("c8", 9): 0, ("c8", 200): 2, ("c8", 1000): 10,
         ("c3", 1000): 0, ("c3", 1100): 0, ("c3", 3000): 0, ("c3", 3100): 0}


@pytest.mark.parametrize("cfg,T", sorted(SWEEP))
def test_block_parity_token_sweep(pkg, orc, dev, cfg, T, monkeypatch):
    """The block at token counts between the benchmark's, against the oracle
    (check_block's bar, with this point's measured allowance)."""
    bw = weights(pkg, cfg, dev)
    x = pkg.workloads.make_x(bw.cfg, T, dev, seed=3 * T + 1)
    monkeypatch.setitem(PAST_BAR, f"{bw.cfg.name} T={T}", SWEEP[(cfg, T)])
    check_block(pkg, orc, bw, x)
