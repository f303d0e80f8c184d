"""MoE block configurations and seeded synthetic weights/inputs.

The shapes the block is measured and tested on (c1 small CPU case, c2
Qwen3-30B-A3B-shaped decode, c3 the same shape at prefill with Zipf routing
skew, c4 high-expert-count with shared expert, c5 wide 8-bit), plus c6, the
Qwen3.6-35B-A3B block as its shipped checkpoint quantises it
(crates/mlxr-lm/tests/fixtures/qwen3_6_35b_a3b/config.json: d 2048, 256
experts, top-8, f 512, shared expert 512, 4-bit experts, mlp.gate and
mlp.shared_expert_gate at 8 bits, group 64), c7 gemma4's expert layout,
and c8, the same Qwen3.6 block unquantised (bf16 experts through gather_mm,
bf16 Linear router and shared gate).
Weights are drawn N(0, 0.02) in f32, rounded to bf16 and affine-quantised
on the device by this library's quantize kernel; x ~ N(0, 1) in bf16;
router weights N(0, 0.02) in f32 (unquantised), or for c6 N(0, 0.02) in
bf16 quantised at router_bits.  No checkpoint is read: everything is
synthetic, from torch generators seeded per tensor.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np
import torch

from . import nn, ops


@dataclass(frozen=True)
class MoEConfig:
    name: str
    d: int                 # hidden size
    E: int                 # routed experts
    K: int                 # experts per token
    f: int                 # expert intermediate size
    fs: int = 0            # shared-expert intermediate size (0: none)
    bits: int = 4          # 4/8: quantised experts; 16: dense bf16 experts (gather_mm)
    group_size: int = 64
    zipf_alpha: float | None = None   # routing skew via per-expert logit bias
    tokens: tuple = field(default_factory=tuple)
    seed: int = 0
    router_bits: int = 0   # 0: f32 router; 4/8: QuantizedLinear router (bf16 block);
                           # 16: bf16 Linear router (gemma4, or an unquantised block)
    layout: str = "split"  # "split": Qwen35MoeBlock; "gemma": gemma4 router +
                           # PackedSwitchFfn<Geglu> (GemmaMoe)


CONFIGS = {
    "c1": MoEConfig("c1_small_cpu", d=512, E=8, K=2, f=256, tokens=(16,)),
    "c2": MoEConfig("c2_qwen3_30b_a3b_decode", d=2048, E=128, K=8, f=768,
                    tokens=(1, 8, 32, 64)),
    "c3": MoEConfig("c3_qwen3_30b_a3b_prefill_zipf", d=2048, E=128, K=8, f=768,
                    zipf_alpha=1.1, tokens=(512, 2048, 4096)),
    "c4": MoEConfig("c4_e512_top10_shared", d=2048, E=512, K=10, f=512, fs=512,
                    tokens=(1, 64, 2048)),
    "c5": MoEConfig("c5_wide_8bit_zipf", d=4096, E=128, K=8, f=1536, bits=8,
                    zipf_alpha=1.1, tokens=(32, 512)),
    "c6": MoEConfig("c6_qwen3_6_35b_a3b_q8router", d=2048, E=256, K=8, f=512, fs=512,
                    router_bits=8, tokens=(1, 64, 2048)),
    # gemma4's layout at the c2 shape: RMSNorm router (bf16 Linear, per-expert
    # scales) and packed gate_up [E, 2f, d] experts with GeGLU
    "c7": MoEConfig("c7_gemma4_packed_geglu", d=2048, E=128, K=8, f=768, router_bits=16,
                    layout="gemma", tokens=(1, 64, 2048)),
    # the c6 block from an unquantised checkpoint: bf16 experts (gather_mm) and
    # bf16 Linear router / shared gate
    "c8": MoEConfig("c8_qwen3_6_35b_a3b_bf16", d=2048, E=256, K=8, f=512, fs=512, bits=16,
                    router_bits=16, tokens=(1, 64, 2048)),
}


def _gen(device, seed: int, stream: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed * 1000003 + stream)
    return g


def _normal(shape, std, device, seed, stream):
    return torch.randn(shape, generator=_gen(device, seed, stream), device=device,
                       dtype=torch.float32) * std


def make_x(cfg: MoEConfig, T: int, device, seed: int | None = None) -> torch.Tensor:
    seed = cfg.seed if seed is None else seed
    return _normal((T, cfg.d), 1.0, device, seed, 1).to(torch.bfloat16)


# The Zipf routing fixture (tests/golden/make_zipf_routing.py writes it):
# per configuration the router logit bias and the realised row counts.
ZIPF_FIXTURE = Path(__file__).resolve().parent.parent / "tests" / "golden" / "zipf_routing.npz"


def zipf_bias(cfg: MoEConfig, device) -> torch.Tensor:
    """Per-expert router bias giving `cfg` its Zipf(alpha) top-K load over a
    seeded permutation of the experts, from the committed fixture (the
    calibration that made it runs once, in make_zipf_routing.py)."""
    key = f"{cfg.name}__bias"
    with np.load(ZIPF_FIXTURE) as z:
        if key not in z.files:
            raise KeyError(f"{ZIPF_FIXTURE.name} has no bias for {cfg.name}: run "
                           "tests/golden/make_zipf_routing.py on a GPU")
        b = z[key]
    if b.shape != (cfg.E,):
        raise ValueError(f"{ZIPF_FIXTURE.name}: bias of {cfg.name} has shape {b.shape}")
    return torch.from_numpy(b.astype(np.float32)).to(device)


def zipf_rows(cfg: MoEConfig, T: int):
    """The committed per-expert row counts of `cfg` at T tokens (None when
    the fixture does not hold them)."""
    key = f"{cfg.name}__rows_T{T}"
    with np.load(ZIPF_FIXTURE) as z:
        return z[key].copy() if key in z.files else None


@dataclass
class BlockWeights:
    cfg: MoEConfig
    gate_w: torch.Tensor | nn.QuantizedLinear | nn.Linear
    gate_b: torch.Tensor | None
    switch_mlp: nn.SplitSwitchFfn
    shared_expert: nn.SwigluMlp | None
    shared_gate_w: torch.Tensor | nn.QuantizedLinear | nn.Linear | None

    gemma: object = None   # (scale, per_expert_scale) of the gemma4 router

    def block(self):
        if self.cfg.layout == "gemma":
            scale, pes = self.gemma
            router = nn.GemmaRouter(self.gate_w, scale, pes, self.cfg.K)
            return nn.GemmaMoe(router, self.switch_mlp)
        return nn.Qwen35MoeBlock(self.gate_w, self.switch_mlp, self.cfg.K, self.shared_expert,
                                 self.shared_gate_w, self.gate_b)


def make_weights(cfg: MoEConfig, device) -> BlockWeights:
    """Seeded weights for `cfg`, quantised on `device` by this library."""
    s = cfg.seed
    gate_w = _normal((cfg.E, cfg.d), 0.02, device, s, 2)
    gate_b = zipf_bias(cfg, device) if cfg.zipf_alpha else None

    def qrouter(w):
        if cfg.router_bits == 16:
            return nn.Linear(w.to(torch.bfloat16))
        return nn.QuantizedLinear.try_from_linear(w.to(torch.bfloat16), 64, cfg.router_bits)

    if cfg.router_bits in (4, 8) or (cfg.router_bits == 16 and cfg.layout == "split"):
        gate_w = qrouter(gate_w)

    def qbank(shape, stream):
        w = _normal(shape, 0.02, device, s, stream).to(torch.bfloat16)
        if cfg.bits == 16:
            return nn.SwitchLinear(w)
        return nn.QuantizedSwitchLinear.try_from_switch_linear(w, cfg.group_size, cfg.bits)

    if cfg.layout == "gemma":
        # scores ~ N(0, 1): the normed input has rms d^-1/2 (scale 1 * root_size)
        proj = _normal((cfg.E, cfg.d), 1.0, device, s, 2).to(torch.bfloat16)
        scale = torch.ones(cfg.d, device=device, dtype=torch.bfloat16)
        pes = (0.5 + torch.rand(cfg.E, generator=_gen(device, s, 13), device=device)).to(
            torch.bfloat16)
        mlp = nn.PackedSwitchFfn(qbank((cfg.E, 2 * cfg.f, cfg.d), 3),
                                 qbank((cfg.E, cfg.d, cfg.f), 5), "geglu")
        return BlockWeights(cfg, proj, None, mlp, None, None, (scale, pes))

    mlp = nn.SplitSwitchFfn(qbank((cfg.E, cfg.f, cfg.d), 3), qbank((cfg.E, cfg.f, cfg.d), 4),
                            qbank((cfg.E, cfg.d, cfg.f), 5))
    shared = sgw = None
    if cfg.fs:
        def qlin(shape, stream):
            w = _normal(shape, 0.02, device, s, stream).to(torch.bfloat16)
            if cfg.bits == 16:
                return nn.Linear(w)
            return nn.QuantizedLinear.try_from_linear(w, cfg.group_size, cfg.bits)
        shared = nn.SwigluMlp(qlin((cfg.fs, cfg.d), 8), qlin((cfg.fs, cfg.d), 9),
                              qlin((cfg.d, cfg.fs), 10))
        sgw = _normal((1, cfg.d), 0.02, device, s, 12)
        if cfg.router_bits:
            sgw = qrouter(sgw)
    return BlockWeights(cfg, gate_w, gate_b, mlp, shared, sgw)


def clone_weights(bw: BlockWeights) -> BlockWeights:
    """The same weights in new device memory: another layer's bank for a
    cold-cache measurement (every step reads weights no earlier step of
    the cycle left in the caches)."""
    def lin(x):
        if x is None:
            return None
        if isinstance(x, torch.Tensor):
            return x.clone()
        if isinstance(x, nn.QuantizedLinear):
            return nn.QuantizedLinear(x.weight[0].clone(), x.scales[0].clone(),
                                      x.biases[0].clone(), x.group_size, x.bits)
        if isinstance(x, nn.QuantizedSwitchLinear):
            return nn.QuantizedSwitchLinear(x.weight.clone(), x.scales.clone(), x.biases.clone(),
                                            x.group_size, x.bits)
        if isinstance(x, nn.Linear):
            return nn.Linear(x.weight[0].clone())
        if isinstance(x, nn.SwitchLinear):
            return nn.SwitchLinear(x.weight.clone())
        raise TypeError(type(x))

    m = bw.switch_mlp
    if isinstance(m, nn.PackedSwitchFfn):
        mlp = nn.PackedSwitchFfn(lin(m.gate_up_proj), lin(m.down_proj), m.activation)
    else:
        mlp = nn.SplitSwitchFfn(lin(m.gate_proj), lin(m.up_proj), lin(m.down_proj))
    se = bw.shared_expert
    shared = None if se is None else nn.SwigluMlp(lin(se.gate_proj), lin(se.up_proj),
                                                 lin(se.down_proj))
    gemma = None if bw.gemma is None else tuple(t.clone() for t in bw.gemma)
    return BlockWeights(bw.cfg, lin(bw.gate_w), lin(bw.gate_b), mlp, shared,
                        lin(bw.shared_gate_w), gemma)


def bank_bytes(bw: BlockWeights) -> int:
    """Device bytes of one bank's expert weights (what a layer holds)."""
    m = bw.switch_mlp
    lins = ([m.gate_up_proj, m.down_proj] if isinstance(m, nn.PackedSwitchFfn)
            else [m.gate_proj, m.up_proj, m.down_proj])
    tot = 0
    for x in lins:
        for t in (x.weight, getattr(x, "scales", None), getattr(x, "biases", None)):
            if t is not None:
                tot += t.numel() * t.element_size()
    return tot


def rows_per_expert(indices: torch.Tensor, E: int) -> dict:
    """The realised load: rows each expert received (max, min over all E,
    mean over the active ones, active count)."""
    c = torch.bincount(indices.reshape(-1).long(), minlength=E).cpu()
    act = c[c > 0]
    return dict(max=int(c.max()), min=int(c.min()), active=int(act.numel()),
                mean_active=round(float(act.float().mean()), 2) if act.numel() else 0.0)


def algorithmic_bytes(cfg: MoEConfig, T: int, distinct_experts: int) -> int:
    """HBM bytes one block forward must move at decode: the packed weights,
    scales and biases of the distinct selected experts (3 projections), the
    router weights (f32, or packed at router_bits with bf16 scales/biases
    per 64), x in, the output (f32, bf16 with a quantised router), and the
    routing (idx + weight)."""
    per_w = weight_bytes_per_element(cfg)
    per_r = (2 if cfg.router_bits == 16 else
             cfg.router_bits / 8 + 4 / 64 if cfg.router_bits else 4)
    b = distinct_experts * 3 * cfg.f * cfg.d * per_w + cfg.E * cfg.d * per_r
    if cfg.fs:
        b += 3 * cfg.fs * cfg.d * per_w + cfg.d * per_r
    b += T * cfg.d * 2 + T * cfg.d * (2 if cfg.router_bits else 4) + T * cfg.K * 8
    return int(b)


def algorithmic_flops(cfg: MoEConfig, T: int) -> int:
    """Expert matmul FLOPs of one forward: 6*T*K*f*d (+ shared expert)."""
    fl = 6 * T * cfg.K * cfg.f * cfg.d
    if cfg.fs:
        fl += 6 * T * cfg.fs * cfg.d + 2 * T * cfg.d
    return int(fl)


def distinct(indices: torch.Tensor) -> int:
    return int(torch.unique(indices.reshape(-1)).numel())


def weight_bytes_per_element(cfg: MoEConfig) -> float:
    """Expert weight bytes per element: the code plus the group's bf16 scale
    and bias, or 2 for dense bf16 weights."""
    return 2.0 if cfg.bits == 16 else cfg.bits / 8 + 4 / cfg.group_size


def expert_bytes_per_row(cfg: MoEConfig, K_dim: int) -> float:
    return K_dim * weight_bytes_per_element(cfg)


__all__ = ["MoEConfig", "CONFIGS", "make_x", "make_weights", "BlockWeights", "zipf_bias", "zipf_rows",
           "clone_weights", "bank_bytes", "rows_per_expert",
           "algorithmic_bytes", "weight_bytes_per_element", "algorithmic_flops", "distinct", "math", "ops"]
