"""MoE-block throughput on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2] [--tokens 64]

One step is one Qwen35MoeBlock forward (router -> dispatch -> grouped
quantised expert GEMMs -> combine) over T synthetic tokens, weights and
inputs already resident in HBM.  Steps run as replays of a captured HIP
graph holding several forwards (--forwards-per-graph, as a decoder's step
graph holds one block per layer); the same forward alone in its graph is
reported beside it.  Prints ONE JSON line: tokens/s through the
block, the dominant kernel's roofline (algorithmic bytes or FLOPs per launch
over its average launch time, from HIP events recorded on the stream it runs
on) and the CPU oracle timed on this host's cores on a bounded sample.

Only one GPU is used; --gpus N with N > 1 exits with a message.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

import __graft_entry__ as entry

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16 MFMA


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="c2", help="c1..c8 (default c2, the decode block)")
    ap.add_argument("--tokens", type=int, default=64, help="T of the headline line")
    ap.add_argument("--launch", choices=["graph", "eager"], default="graph",
                    help="replay one captured HIP graph per step, or launch eagerly")
    ap.add_argument("--sweep", default="c2:1,c2:1:cold,c2:8,c2:8:cold,c2:32,c2:32:cold,c3:512,"
                    "c3:2048,c3:4096,c4:64,c4:2048,c5:32,c5:512,c6:64,c6:2048,c6:64:res,"
                    "c6:2048:res,c7:64,c7:2048,c8:64,c8:2048",
                    help="extra cfg:T points timed after the headline ('' for none); "
                         "cfg:T:res times the decoder layer's MoE half (RMSNorm, block, "
                         "residual add); cfg:T:cold rotates copies of the weights so "
                         "every forward reads its experts from HBM")
    ap.add_argument("--forwards-per-graph", type=int, default=20,
                    help="forwards of the block one captured graph holds (warm graph "
                         "replays; a decoder's step graph holds one block per layer -- "
                         "48 in Qwen3-30B-A3B -- so the replay's own launch cost is "
                         "shared); the headline uses the largest count up to this that "
                         "divides --steps")
    ap.add_argument("--sweep-steps", type=int, default=50)
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="bound of the CPU-baseline sample (0 skips it)")
    ap.add_argument("--cpu-threads", type=int, default=0, help="0: the host cores, up to 16")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="only run a plain device copy of this many MiB, 20 times (the "
                         "known-size kernel that calibrates FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--dense-gemm", action="store_true",
                    help="only time the vendor library's dense bf16 batched GEMM "
                         "(torch.bmm) at --config/--tokens' expert shapes, the routed "
                         "rows spread evenly over the experts: the practical ceiling "
                         "the quantized prefill GEMMs are set beside")
    return ap.parse_args()


def dense_gemm_reference(cfg, T: int, reps: int = 50) -> None:
    """Event-timed torch.bmm (hipBLASLt) in bf16 at the expert shapes of one
    block forward: [E, rows, d] x [E, d, 2f] (gate and up as one product) and
    [E, rows, f] x [E, f, d], rows = T*K/E per expert, uniform -- no gather,
    no skew, no dequantisation, no SwiGLU -- and the same rows as one flat
    [E*rows, k] x [k, n] product of a single weight matrix (no expert
    structure).  One JSON line per projection and form."""
    import torch
    dev = torch.device("cuda:0")
    rows = max(1, T * cfg.K // cfg.E)
    for name, k, n in (("gate_up", cfg.d, 2 * cfg.f), ("down", cfg.f, cfg.d)):
        a = torch.randn(cfg.E, rows, k, device=dev, dtype=torch.bfloat16)
        b = torch.randn(cfg.E, k, n, device=dev, dtype=torch.bfloat16).contiguous()
        o = torch.empty(cfg.E, rows, n, device=dev, dtype=torch.bfloat16)
        a2, b2 = a.reshape(cfg.E * rows, k), b[0].contiguous()
        o2 = o.reshape(cfg.E * rows, n)
        flops = 2.0 * cfg.E * rows * k * n
        for form, fn, shape in (
                ("torch.bmm bf16", lambda: torch.bmm(a, b, out=o), [cfg.E, rows, k, n]),
                ("torch.mm bf16 flat", lambda: torch.mm(a2, b2, out=o2),
                 [cfg.E * rows, k, n])):
            for _ in range(5):
                fn()
            torch.cuda.synchronize()
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0.record()
            for _ in range(reps):
                fn()
            t1.record()
            torch.cuda.synchronize()
            us = t0.elapsed_time(t1) / reps * 1e3
            print(json.dumps({"library_gemm": form, "config": cfg.name, "tokens": T,
                              "projection": name, "shape": shape, "us": round(us, 1),
                              "tflops": round(flops / us / 1e6, 1),
                              "frac_of_bf16_peak": round(flops / us / 1e6 / BF16_PEAK_TFLOPS,
                                                         3)}),
                  flush=True)
        del a, b, o, a2, b2, o2
    torch.cuda.empty_cache()


def copy_calibration(mib: int) -> None:
    import torch
    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(20):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_per_launch": n * 4, "launches": 20}), flush=True)


def graph_forwards(steps: int, cap: int, launch: str) -> int:
    """Forwards one graph replay holds: the largest count up to `cap` that
    divides `steps`, so that exactly `steps` forwards are timed (1 for
    eager launches)."""
    if launch != "graph":
        return 1
    return max(c for c in range(1, max(1, cap) + 1) if steps % c == 0)


def host_cores() -> int:
    """The cores this process may run on (its affinity mask), within an
    OpenMP thread limit the host sets (OMP_NUM_THREADS)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    lim = os.environ.get("OMP_NUM_THREADS", "")
    if lim.isdigit() and int(lim) > 0:
        n = min(n, int(lim))
    return max(1, n)


class Runner:
    """One block at one T: eager or graph-replay steps on the current stream.
    residual: the decoder layer's MoE half instead (post-attention RMSNorm,
    the block, the residual add: Qwen35MoeBlock.forward_residual).
    banks: more copies of the weights in their own memory (a cold-cache
    measurement, like a decoder whose every step reads another layer's
    experts): one step is one forward on the next bank in turn.
    repeat: the forwards of one graph replay (or eager step) run the same
    weights this many times over (with banks: the bank cycle, repeated)."""

    def __init__(self, pkg, bw, T, dev, launch, residual=False, banks=(), repeat=1):
        import torch
        self.torch = torch
        self.T = T
        self.blocks = [b.block() for b in (bw, *banks)] * max(1, repeat)
        self.block = self.blocks[0]
        self.x = pkg.workloads.make_x(bw.cfg, T, dev, seed=T)
        self.out = torch.empty((T, bw.cfg.d), dtype=self.block.out_dtype, device=dev)
        self.norm = None
        if residual:
            g = torch.Generator(device=dev).manual_seed(T)
            w = (1 + 0.1 * torch.randn(bw.cfg.d, generator=g, device=dev)).to(torch.bfloat16)
            self.norm = pkg.nn.RmsNorm(w, 1e-6)
            self.ws = pkg.ops.workspace(self.block.residual_workspace_size(T), dev)
        else:
            self.ws = pkg.ops.workspace(self.block.workspace_size(T), dev)
        # one routed run: distinct experts for the byte count
        self.run(keep_routing=True)
        torch.cuda.synchronize()
        self.idx = self.block.last_indices.clone()
        self.ref = self.out.clone()
        self.graph = None
        if launch == "graph":
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                for _ in range(2):
                    self.eager()
            torch.cuda.current_stream().wait_stream(s)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self.eager()
            torch.cuda.synchronize()
            self.graph = g
            for _ in range(3):  # every replay reproduces the eager result
                g.replay()
                torch.cuda.synchronize()
                if not torch.equal(self.out, self.ref):
                    raise RuntimeError("graph replay differs from the eager forward")
                self.eager()
                torch.cuda.synchronize()

    def run(self, keep_routing, block=None):
        block = block or self.block
        if self.norm is not None:
            block.forward_residual(self.x, self.norm, out=self.out, workspace=self.ws,
                                   keep_routing=keep_routing)
        else:
            block(self.x, out=self.out, workspace=self.ws, keep_routing=keep_routing)

    def eager(self):
        # one forward per bank (the graph holds them all)
        for b in self.blocks:
            self.run(keep_routing=False, block=b)

    def step(self):
        if self.graph is not None:
            self.graph.replay()
        else:
            self.eager()

    def timed(self, steps, warmup):
        """Mean seconds per forward over `steps` steps."""
        return self.timed_regions(steps, warmup, 1)[0]

    def timed_regions(self, steps, warmup, repeats):
        """Seconds per forward of each of `repeats` timed regions, each
        `steps` steps bracketed by a synchronisation on both sides, after
        `warmup` untimed steps."""
        torch = self.torch
        for _ in range(warmup):
            self.step()
        torch.cuda.synchronize()
        out = []
        for _ in range(repeats):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                self.step()
            torch.cuda.synchronize()
            out.append((time.perf_counter() - t0) / steps / len(self.blocks))
        return out

    def median(self, steps):
        """Median seconds per forward, each step bracketed by events on the
        stream the forwards run on."""
        torch = self.torch
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
        ev[0].record()
        for i in range(steps):
            self.step()
            ev[i + 1].record()
        torch.cuda.synchronize()
        d = sorted(ev[i].elapsed_time(ev[i + 1]) for i in range(steps))
        return d[steps // 2] / 1e3 / len(self.blocks)

    def kernel_time(self, pkg, kernel, steps):
        """Average duration (s) of `kernel` over `steps` eager forwards, from
        HIP events the library records around each launch on its stream."""
        import ctypes
        C = pkg._capi
        lib = C.lib()
        self.torch.cuda.synchronize()
        C.check(lib.mlxr_moe_profile_start(kernel.encode()))
        for _ in range(steps):
            self.eager()
        n = ctypes.c_int64()
        tot, mn, mx = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
        C.check(lib.mlxr_moe_profile_stop(ctypes.byref(n), ctypes.byref(tot), ctypes.byref(mn),
                                          ctypes.byref(mx)))
        if n.value == 0:
            raise RuntimeError(f"kernel {kernel} was not launched")
        return tot.value / n.value / 1e3, n.value, mn.value / 1e3, mx.value / 1e3


def gated_bytes(cfg, T, U, shared_folded=False):
    """Algorithmic HBM bytes of one gate/up launch: the packed words plus
    bf16 scales and biases (or the dense bf16 weights) of the U distinct
    selected experts' gate and up rows (2*f*d weights each), x read once
    (T*d bf16) and the activations written (T*K*f bf16); with the shared
    expert folded into the launch (folds_shared) also its gate and up rows
    (2*fs*d) and its activations (T*fs bf16)."""
    per_w = 2.0 if cfg.bits == 16 else cfg.bits / 8 + 4 / cfg.group_size
    b = U * 2 * cfg.f * cfg.d * per_w + T * cfg.d * 2 + T * cfg.K * cfg.f * 2
    if shared_folded and cfg.fs:
        b += 2 * cfg.fs * cfg.d * per_w + T * cfg.fs * 2
    return int(b)


def gated_flops(cfg, T, shared_folded=False):
    """gate/up flops of one launch: 4*T*K*f*d, plus 4*T*fs*d with the
    shared expert folded in."""
    return 4 * T * (cfg.K * cfg.f + (cfg.fs if shared_folded and cfg.fs else 0)) * cfg.d


def tiled_path(rows, experts, bits):
    """Whether a grouped GEMM of `rows` rows over `experts` experts runs the
    M-tiled kernel: nn::use_prefill_path (csrc/nn.cpp), with its thresholds
    MLXR_QUANT_TILED_ROWS (16) and MLXR_DENSE_TILED_ROWS (2) rows per
    expert (csrc/nn.hpp), and at least 512 rows."""
    per = 2 if bits == 16 else 16
    return rows >= per * experts and rows >= 512


def folds_shared(cfg, T):
    """Whether the block folds its shared expert into the routed launches
    (SwitchFfn::can_fold, csrc/nn.cpp): same bits and hidden size, and both
    on the streaming decode kernel (quantised) or both M-tiled."""
    if not cfg.fs or cfg.fs != cfg.f:
        return False
    routed = tiled_path(T * cfg.K, cfg.E, cfg.bits)
    shared = tiled_path(T, 1, cfg.bits)
    if not routed and not shared:
        return cfg.bits != 16
    return routed and shared


def measured_traffic(workload: str, kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter
    summary (FETCH_SIZE + WRITE_SIZE, each scaled by a plain copy of known
    size), when it covers this workload; None otherwise."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        "qgemm_decode_c2_T64_traffic.json")
    try:
        with open(path) as fh:
            data = json.load(fh)
    except (OSError, ValueError):
        return None
    if data.get("workload") != workload:
        return None
    return data.get("kernels", {}).get(kernel, {}).get("traffic_bytes")


def read_ceiling(pkg, dev, chunk, reps=20):
    """Bytes per second of a plain streaming read (mlxr_moe_profile_read) of
    `chunk` bytes per launch, the launches rotating over eight chunks of one
    buffer (more than the 256 MB last-level cache holds, so each reads from
    HBM), event-timed like the GEMMs: the practical read ceiling of this
    GPU beside which the GEMMs' rates are set."""
    import ctypes
    import torch
    C = pkg._capi
    lib = C.lib()
    chunk = max(16, chunk // 256 * 256)
    buf = torch.empty(8 * chunk, dtype=torch.uint8, device=dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    base = buf.data_ptr()
    for i in range(2):
        C.check(lib.mlxr_moe_profile_read(base + i * chunk, chunk, sink.data_ptr(), stream))
    torch.cuda.synchronize()
    C.check(lib.mlxr_moe_profile_start(b"read_probe"))
    for i in range(reps):
        C.check(lib.mlxr_moe_profile_read(base + (i % 8) * chunk, chunk, sink.data_ptr(),
                                          stream))
    n = ctypes.c_int64()
    tot, mn, mx = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
    C.check(lib.mlxr_moe_profile_stop(ctypes.byref(n), ctypes.byref(tot), ctypes.byref(mn),
                                      ctypes.byref(mx)))
    del buf
    torch.cuda.empty_cache()
    return chunk / (tot.value / n.value / 1e3), chunk


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cold_banks(W, bw, T, U):
    """Copies of bw so that a bank is reused only after more than twice the
    256 MB of MI355X's last-level (Infinity) cache has streamed through:
    every forward then reads its experts from HBM."""
    per_step = W.algorithmic_bytes(bw.cfg, T, U)
    n = max(4, min(48, -(-2 * 256 * 2 ** 20 // max(per_step, 1)) + 1))
    return [W.clone_weights(bw) for _ in range(n - 1)]


def cpu_baseline(pkg, orc, bw, T, seconds, threads):
    """The oracle (plain C, OpenMP) on this host: whole block forwards of the
    same c-config at T tokens until `seconds` have passed (at least one)."""
    import torch
    p = orc.block_params(bw)
    x = orc.to_np(pkg.workloads.make_x(bw.cfg, T, torch.device("cuda:0"), seed=T))
    orc.block_forward(p, x[:1], nthreads=threads)  # page in
    n = 0
    t0 = time.perf_counter()
    while True:
        orc.block_forward(p, x, nthreads=threads)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return dict(value=round(n * T / el, 2), unit="tokens/s", cores=threads, kind="port",
                sample=f"{n} block forwards of {bw.cfg.name} at T={T} "
                       f"({el:.1f} s, oracle/moe_oracle.c -O3 -march=native, "
                       f"{threads} OpenMP threads)")


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one MI355X only (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE={world}); the MoE block is not sharded across GPUs here.",
              file=sys.stderr)
        sys.exit(2)

    if args.copy_mib:
        copy_calibration(args.copy_mib)
        return
    import torch
    pkg = entry.load_package()
    dev = torch.device("cuda:0")
    W = pkg.workloads
    cfg = W.CONFIGS[args.config]
    if args.dense_gemm:
        dense_gemm_reference(cfg, args.tokens)
        return
    T = args.tokens
    print(f"bench: {cfg.name} T={T} on {torch.cuda.get_device_name(dev)}", file=sys.stderr,
          flush=True)
    bw = W.make_weights(cfg, dev)
    fpg = graph_forwards(args.steps, args.forwards_per_graph, args.launch)
    r = Runner(pkg, bw, T, dev, args.launch, repeat=fpg)
    U = W.distinct(r.idx)
    # the timed region is exactly --steps forwards; it runs `repeats` times
    # (at least 10, and at least 50 timed forwards in all) after at least 10
    # warm-up forwards, and the median region gives ms_per_step
    repeats = max(10, -(-50 // max(1, args.steps)))
    warm = max(args.warmup, 10)
    regions = r.timed_regions(args.steps // fpg, -(-warm // fpg), repeats)
    sec = float(np.median(regions))
    tok_s = T / sec
    block_bytes = W.algorithmic_bytes(cfg, T, U)
    med = r.median(args.steps // fpg)
    print(f"bench: {sec * 1e6:.1f} us/step (median {med * 1e6:.1f}), {tok_s:.0f} tokens/s, "
          f"{fpg} forwards per graph", file=sys.stderr, flush=True)
    # the same forward alone in its graph (the replay's launch cost on every
    # forward)
    sec1 = None
    if fpg > 1:
        r1 = Runner(pkg, bw, T, dev, args.launch)
        sec1 = r1.timed(args.steps, args.warmup)
        del r1
        print(f"bench: one forward per graph {sec1 * 1e6:.1f} us/step", file=sys.stderr,
              flush=True)
    # the same forward with the weights rotated over banks in their own
    # memory: no step finds its experts in the caches
    rc = Runner(pkg, bw, T, dev, args.launch, banks=cold_banks(W, bw, T, U))
    sec_c = rc.timed(max(args.steps // len(rc.blocks), 10), 2)
    cold = dict(tokens_per_s=round(T / sec_c, 1), us_per_step=round(sec_c * 1e6, 2),
                us_per_step_median=round(rc.median(max(args.steps // len(rc.blocks), 10)) * 1e6, 2),
                banks=len(rc.blocks), bank_bytes=W.bank_bytes(bw),
                block_hbm_gbs=round(block_bytes / sec_c / 1e9, 1))
    del rc
    print(f"bench: cold {cold}", file=sys.stderr, flush=True)

    # dominant kernel: the fused gate/up gather_qmm
    kt, kn, kmin, kmax = r.kernel_time(pkg, "qgemm_gated", max(1, args.steps // fpg))
    decode = T * cfg.K < 2048
    if decode:
        traffic_alg = gated_bytes(cfg, T, U, folds_shared(cfg, T))
        achieved = traffic_alg / kt / 1e9
        roof = dict(bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                    frac=round(achieved / HBM_PEAK_GBS, 4),
                    traffic=measured_traffic(f"{cfg.name} T={T}", "qgemm_gated"),
                    algorithmic_bytes=traffic_alg)
        # the same byte count read by a kernel that only reads
        rate, nbytes = read_ceiling(pkg, dev, traffic_alg)
        roof["read_ceiling"] = dict(gbs=round(rate / 1e9, 1), bytes=nbytes,
                                    frac_of_ceiling=round(achieved / (rate / 1e9), 4))
        print(f"bench: plain read of {nbytes} bytes {rate / 1e9:.1f} GB/s", file=sys.stderr,
              flush=True)
    else:
        achieved = gated_flops(cfg, T, folds_shared(cfg, T)) / kt / 1e12
        roof = dict(bound="mfma", achieved=round(achieved, 2), peak=BF16_PEAK_TFLOPS,
                    unit="TFLOP/s", frac=round(achieved / BF16_PEAK_TFLOPS, 4), traffic=None)
    roof.update(kernel="qgemm_gated", kernel_us=round(kt * 1e6, 2), launches=kn,
                kernel_us_min=round(kmin * 1e6, 2), kernel_us_max=round(kmax * 1e6, 2))
    print(f"bench: qgemm_gated {kt * 1e6:.2f} us avg over {kn} launches", file=sys.stderr,
          flush=True)

    sweep = []
    banks = {cfg.name: bw}
    for item in [s for s in args.sweep.split(",") if s]:
        parts = item.split(":")
        cname, tt = parts[0], int(parts[1])
        res = len(parts) > 2 and parts[2] == "res"
        cold_pt = len(parts) > 2 and parts[2] == "cold"
        c2 = W.CONFIGS[cname]
        if c2.name not in banks:
            banks[c2.name] = W.make_weights(c2, dev)
        fpg2 = max(1, args.forwards_per_graph) if args.launch == "graph" else 1
        r2 = Runner(pkg, banks[c2.name], tt, dev, args.launch, residual=res, repeat=fpg2)
        U2 = W.distinct(r2.idx)
        if cold_pt:
            r2 = Runner(pkg, banks[c2.name], tt, dev, args.launch,
                        banks=cold_banks(W, banks[c2.name], tt, U2))
        steps2 = max(args.sweep_steps // len(r2.blocks), 10)
        s2 = r2.timed(steps2, 2)
        m2 = r2.median(steps2)
        # both rates for every point: the decode sizes and the small prefills
        # (c3 T=512, c4 T=2048, c5 T=512: arithmetic intensity below the
        # ridge) are HBM-bound, the large prefills MFMA-bound
        ent = dict(config=c2.name + (" layer tail" if res else "") + (" cold" if cold_pt else ""),
                   T=tt, tokens_per_s=round(tt / s2, 1),
                   us_per_step=round(s2 * 1e6, 2), us_per_step_median=round(m2 * 1e6, 2),
                   distinct_experts=U2,
                   block_hbm_gbs=round(W.algorithmic_bytes(c2, tt, U2) / s2 / 1e9, 1),
                   block_tflops=round(W.algorithmic_flops(c2, tt) / s2 / 1e12, 2),
                   rows_per_expert=W.rows_per_expert(r2.idx, c2.E),
                   forwards_per_graph=len(r2.blocks))
        if cold_pt:
            ent["banks"] = len(r2.blocks)
        sweep.append(ent)
        print(f"bench: sweep {ent}", file=sys.stderr, flush=True)
        del r2

    cpu = None
    if args.cpu_seconds > 0:
        import tempfile
        orc = entry.load_oracle()
        # the restatement compiled for this host's CPU, in a scratch dir
        tmp = tempfile.mkdtemp(prefix="mlxr_oracle_")
        orc.use_library(orc.build_native(tmp))
        threads = args.cpu_threads or host_cores()
        cpu = cpu_baseline(pkg, orc, bw, T, args.cpu_seconds, threads)
        # and on one core (a single-threaded run of the same restatement)
        one = cpu_baseline(pkg, orc, bw, T, args.cpu_seconds / 2, 1)
        cpu["value_1core"] = one["value"]
        cpu["sample_1core"] = one["sample"]
        cpu["host"] = dict(cpu_model=cpu_model(), nproc=os.cpu_count(),
                           affinity=len(os.sched_getaffinity(0)),
                           omp_num_threads=os.environ.get("OMP_NUM_THREADS"))
        print(f"bench: cpu baseline {cpu}", file=sys.stderr, flush=True)

    line = {
        "metric": "MoE-block tokens/sec (Qwen3-30B-A3B-shaped 4-bit block, decode)",
        "value": round(tok_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec * 1e3, 5),
        "timed_regions": {"repeats": repeats, "steps_each": args.steps,
                          "warmup_forwards": -(-warm // fpg) * fpg,
                          "ms_per_step_mean": round(float(np.mean(regions)) * 1e3, 5),
                          "ms_per_step_min": round(min(regions) * 1e3, 5),
                          "ms_per_step_max": round(max(regions) * 1e3, 5)},
        "ms_per_step_median": round(med * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) x, N(0,0.02) weights affine-quantised on the GPU)",
        "config": {"workload": f"{cfg.name} T={T}", "tokens": T, "d": cfg.d, "E": cfg.E,
                   "K": cfg.K, "f": cfg.f, "bits": cfg.bits, "group_size": cfg.group_size,
                   "distinct_experts": U, "launch": args.launch,
                   "forwards_per_graph": fpg,
                   "block_algorithmic_bytes": block_bytes,
                   "block_hbm_gbs": round(block_bytes / sec / 1e9, 1),
                   "rows_per_expert": W.rows_per_expert(r.idx, cfg.E)},
        "one_forward_per_graph": (None if sec1 is None else
                                  {"us_per_step": round(sec1 * 1e6, 2),
                                   "tokens_per_s": round(T / sec1, 1)}),
        "cold": cold,
        "roofline": roof,
        "cpu_baseline": cpu,
        "sweep": sweep,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
