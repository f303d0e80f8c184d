"""bench.py's contract on the CPU: one GPU only, the options the driver
passes, and the algorithmic byte counts the roofline divides by."""
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def _run(*args):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], cwd=ROOT,
                          capture_output=True, text=True, timeout=120)


def test_more_than_one_gpu_exits_with_a_message():
    r = _run("--gpus", "2", "--steps", "1", "--warmup", "0")
    assert r.returncode == 2
    assert "one MI355X" in r.stderr and r.stdout == ""


def test_help_lists_the_driver_options_and_the_sweep_forms():
    r = _run("--help")
    assert r.returncode == 0
    for opt in ("--gpus", "--steps", "--warmup", "--sweep", "--cpu-seconds",
                "--forwards-per-graph", "--dense-gemm"):
        assert opt in r.stdout
    assert "cfg:T:res" in r.stdout


def test_forwards_per_graph_divide_the_steps():
    """Graph replays hold the largest count of forwards up to the option
    that divides --steps, so exactly --steps forwards are timed."""
    import bench
    assert bench.graph_forwards(200, 8, "graph") == 8
    assert bench.graph_forwards(5, 8, "graph") == 5
    assert bench.graph_forwards(9, 8, "graph") == 3
    assert bench.graph_forwards(7, 8, "graph") == 7
    assert bench.graph_forwards(13, 8, "graph") == 1
    assert bench.graph_forwards(200, 8, "eager") == 1
    assert bench.graph_forwards(200, 0, "graph") == 1
    for steps in range(1, 60):
        f = bench.graph_forwards(steps, 8, "graph")
        assert steps % f == 0 and 1 <= f <= 8


def test_algorithmic_bytes(pkg):
    """Decode bytes per block forward (the distinct experts' weights, the
    router, x in, out, routing): 4-bit at 0.5 + 4/64 bytes per weight,
    dense bf16 at 2, with the router at its own width."""
    W = pkg.workloads
    c2, c8 = W.CONFIGS["c2"], W.CONFIGS["c8"]
    T, U = 64, 126
    want2 = (U * 3 * c2.f * c2.d * (0.5 + 4 / 64) + c2.E * c2.d * 4
             + T * c2.d * 2 + T * c2.d * 4 + T * c2.K * 8)
    assert W.algorithmic_bytes(c2, T, U) == int(want2)
    U8 = 218
    want8 = (U8 * 3 * c8.f * c8.d * 2 + c8.E * c8.d * 2 + 3 * c8.fs * c8.d * 2 + c8.d * 2
             + T * c8.d * 2 + T * c8.d * 2 + T * c8.K * 8)
    assert W.algorithmic_bytes(c8, T, U8) == int(want8)
    assert W.weight_bytes_per_element(c8) == 2.0
    assert W.weight_bytes_per_element(c2) == pytest.approx(0.5625)


def test_gated_bytes_with_folded_shared_expert(pkg):
    """The gate/up launch's bytes: the routed experts' gate and up rows, x in,
    activations out; the folded shared expert adds its own rows and
    activations (c6: E=256, f = fs = 512, 4-bit)."""
    import bench
    c6 = pkg.workloads.CONFIGS["c6"]
    T, U = 64, 219
    per_w = 0.5 + 4 / 64
    base = U * 2 * c6.f * c6.d * per_w + T * c6.d * 2 + T * c6.K * c6.f * 2
    assert bench.gated_bytes(c6, T, U) == int(base)
    assert bench.gated_bytes(c6, T, U, True) == int(base + 2 * c6.fs * c6.d * per_w + T * c6.fs * 2)


def test_shared_expert_fold_rule(pkg):
    """The bench's copy of the library's fold rule: c6 folds at T=64 (both
    streaming) and T=512 and 2048 (both M-tiled); c4 not at T=512 (routed
    rows on the streaming kernel, 10 per expert; the shared expert's 512
    rows M-tiled); dense c8 folds only M-tiled; c3 has no shared expert.
    The folded gate/up launch's flops count the shared expert's rows."""
    import bench
    C = pkg.workloads.CONFIGS
    c4, c6, c8 = C["c4"], C["c6"], C["c8"]
    assert bench.folds_shared(c6, 64) and bench.folds_shared(c6, 2048)
    assert bench.folds_shared(c6, 512) and not bench.folds_shared(c4, 512)
    assert not bench.folds_shared(c8, 64) and bench.folds_shared(c8, 2048)
    assert not bench.folds_shared(C["c3"], 4096)
    assert bench.tiled_path(2048 * c6.K, c6.E, c6.bits) == bool(pkg.ops.gather_qmm_tiled(2048 * c6.K, c6.E))
    assert bench.tiled_path(512 * c6.K, c6.E, c6.bits) == bool(pkg.ops.gather_qmm_tiled(512 * c6.K, c6.E))
    T = 2048
    assert bench.gated_flops(c6, T, True) == 4 * T * (c6.K * c6.f + c6.fs) * c6.d
    assert bench.gated_flops(c6, T) == 4 * T * c6.K * c6.f * c6.d
