"""Reading one MoE layer of an mlxr checkpoint (safetensors shards) into the
block's modules.

Follows the reference's loader for the keys this path uses:
  list_shards             crates/mlxr-lm/src/loader.rs:148-175
  sanitize_key            crates/mlxr-lm/src/qwen3_5/text/weights.rs:69-83
  rewrite_quantised_keys  crates/mlxr-lm/src/loader.rs:176-191 (a `.weight`
                          with a `.scales` sibling is a QuantizedLinear's)
  QuantizationConfig      crates/mlxr-lm/src/quantization.rs:20-101
                          (body group_size / bits, per-path overrides)
  post_attention_layernorm weights.rs:33-42, 119-165 (+1.0 in the
                          weight's dtype unless the shard says format "mlx")
  the packed HF expert tensor `mlp.experts.gate_up_proj [E, 2H, D]`, split
  along axis 1 into `switch_mlp.{gate,up}_proj` as mlxr-convert does
  (crates/mlxr-convert/src/qwen3_5.rs:96-147).
Only the tensors of the requested layer are read (safe_open, one key at a
time): a 35B checkpoint's other layers never reach host memory.
"""
from __future__ import annotations

import json
from pathlib import Path

import torch

from . import nn
from ._capi import MlxrMoeError


def list_shards(model_dir) -> list[Path]:
    """`model.safetensors`, or the files `model.safetensors.index.json`
    names, sorted (loader.rs:148-175)."""
    d = Path(model_dir)
    single = d / "model.safetensors"
    if single.is_file():
        return [single]
    index = d / "model.safetensors.index.json"
    if not index.is_file():
        raise MlxrMoeError(f"weights: neither model.safetensors nor "
                           f"model.safetensors.index.json in {d}")
    weight_map = json.loads(index.read_text())["weight_map"]
    return sorted({d / f for f in weight_map.values()})


def sanitize_key(key: str) -> str:
    """weights.rs:69-83 (the language-model keys)."""
    if "model.language_model" in key:
        return key.replace("model.language_model", "language_model.model")
    if "model.visual" in key:
        return key.replace("model.visual", "vision_tower")
    if key.startswith("lm_head"):
        return "language_model." + key
    if key.startswith("mtp."):
        return "language_model." + key
    return key


class QuantizationConfig:
    """The `quantization` (or `quantization_config`) block of config.json:
    body group_size / bits and per-path {group_size, bits} overrides keyed
    by the raw module prefix (quantization.rs:20-101)."""

    def __init__(self, cfg: dict):
        self.group_size = int(cfg["group_size"])
        self.bits = int(cfg["bits"])
        self.mode = cfg.get("mode", "affine")
        self.overrides = {}
        for k, v in cfg.items():
            if isinstance(v, dict) and "group_size" in v and "bits" in v:
                self.overrides[k] = (int(v["group_size"]), int(v["bits"]))

    def for_path(self, raw_prefix: str) -> tuple[int, int]:
        """quantization.rs:51-56."""
        return self.overrides.get(raw_prefix, (self.group_size, self.bits))

    @classmethod
    def from_config(cls, config: dict):
        q = config.get("quantization") or config.get("quantization_config")
        return None if q is None else cls(q)


def read_config(model_dir) -> dict:
    return json.loads((Path(model_dir) / "config.json").read_text())


def text_config(config: dict) -> dict:
    return config.get("text_config", config)


class LayerTensors:
    """The sanitised tensors under `language_model.model.layers.{layer}.mlp.`
    (CPU, as stored), read key by key from the shards."""

    def __init__(self, model_dir, layer: int):
        from safetensors import safe_open

        self.prefix = f"language_model.model.layers.{layer}.mlp."
        self.t = {}
        for path in list_shards(model_dir):
            with safe_open(str(path), framework="pt") as f:
                for k in f.keys():
                    sk = sanitize_key(k)
                    if sk.startswith(self.prefix):
                        self.t[sk[len(self.prefix):]] = f.get_tensor(k)
        # the HF packed expert tensor -> switch_mlp.{gate,up}_proj
        # (mlxr-convert/src/qwen3_5.rs:96-147)
        gu = self.t.pop("experts.gate_up_proj", None)
        if gu is not None:
            h = gu.shape[1] // 2
            self.t["switch_mlp.gate_proj.weight"] = gu[:, :h].contiguous()
            self.t["switch_mlp.up_proj.weight"] = gu[:, h:].contiguous()
        dn = self.t.pop("experts.down_proj", None)
        if dn is not None:
            self.t["switch_mlp.down_proj.weight"] = dn

    def has(self, name: str) -> bool:
        return name in self.t

    def quantised(self, module: str) -> bool:
        """rewrite_quantised_keys: a `.scales` sibling marks a quantised
        module (loader.rs:176-191)."""
        return f"{module}.scales" in self.t

    def get(self, name: str) -> torch.Tensor:
        if name not in self.t:
            raise MlxrMoeError(f"weights: {self.prefix}{name} is missing")
        return self.t[name]


def is_mlx_format(path) -> bool:
    """The shard's header metadata says format "mlx": its norm weights
    already carry the +1.0 shift (weights.rs:45-70)."""
    from safetensors import safe_open

    with safe_open(str(path), framework="pt") as f:
        meta = f.metadata() or {}
    return meta.get("format") == "mlx"


def post_attention_layernorm(model_dir, layer: int, device):
    """nn.RmsNorm of decoder layer `layer`'s post_attention_layernorm (the
    norm before the MoE block, layer.rs:137), eps = rms_norm_eps; the weight
    gets the +1.0 centring shift in its own dtype unless its shard is
    mlx-format (weights.rs:147-165)."""
    from safetensors import safe_open

    want = f"language_model.model.layers.{layer}.post_attention_layernorm.weight"
    tc = text_config(read_config(model_dir))
    for path in list_shards(model_dir):
        with safe_open(str(path), framework="pt") as f:
            for k in f.keys():
                if sanitize_key(k) == want:
                    w = f.get_tensor(k)
                    if not is_mlx_format(path) and w.ndim == 1 and w.is_floating_point():
                        w = w + torch.ones((), dtype=w.dtype)
                    return nn.RmsNorm(w.to(device), float(tc.get("rms_norm_eps", 1e-6)))
    raise MlxrMoeError(f"weights: {want} is missing")


def _u32_as_i32(t: torch.Tensor) -> torch.Tensor:
    # packed codes are stored as U32; the kernels read the same bits as int32
    return t.view(torch.int32) if t.dtype == torch.uint32 else t.to(torch.int32)


def qwen35_moe_block(model_dir, layer: int, device, quantize_dense=None):
    """The MoE block of decoder layer `layer` (Qwen3.5 / Qwen3.6 MoE
    naming: mlp.gate, mlp.switch_mlp.*, mlp.shared_expert.*,
    mlp.shared_expert_gate) as an nn.Qwen35MoeBlock on `device`.

    Quantised modules keep the checkpoint's codes, scales and biases bit for
    bit, with (group_size, bits) from the config's per-path overrides
    (quantization.rs:51-56).  Dense modules stay dense -- bf16
    SwitchLinear experts (gather_mm) and Linear projections, the
    MaybeQuantized::Original form -- unless quantize_dense = (group_size,
    bits) asks to quantise them on load (try_into_quantized,
    switch.rs:478-491).  A dense bf16 router computes in bf16 like the
    reference's (nn.Linear); an f32 one in f32."""
    config = read_config(model_dir)
    tc = text_config(config)
    qc = QuantizationConfig.from_config(config)
    lt = LayerTensors(model_dir, layer)
    raw = f"language_model.model.layers.{layer}.mlp."
    dev = torch.device(device)

    def qlinear(module, cls, expert_dims):
        if not lt.quantised(module):
            w = lt.get(f"{module}.weight").to(dev, torch.bfloat16)
            if quantize_dense is None:
                return nn.Linear(w) if cls is nn.QuantizedLinear else nn.SwitchLinear(w)
            gs, bits = quantize_dense
            if cls is nn.QuantizedLinear:
                return cls.try_from_linear(w, gs, bits)
            return cls.try_from_switch_linear(w, gs, bits)
        if qc is None:
            raise MlxrMoeError("weights: quantised tensors but no quantization config")
        gs, bits = qc.for_path(raw + module)
        wq = _u32_as_i32(lt.get(f"{module}.weight")).to(dev)
        sc = lt.get(f"{module}.scales").to(dev, torch.bfloat16)
        bi = lt.get(f"{module}.biases").to(dev, torch.bfloat16)
        return cls(wq, sc, bi, gs, bits)

    S = nn.QuantizedSwitchLinear
    mlp = nn.SplitSwitchFfn(qlinear("switch_mlp.gate_proj", S, 3),
                            qlinear("switch_mlp.up_proj", S, 3),
                            qlinear("switch_mlp.down_proj", S, 3))
    K = int(tc["num_experts_per_tok"])
    shared = sgate = None
    if lt.has("shared_expert.gate_proj.weight"):
        L = nn.QuantizedLinear
        shared = nn.SwigluMlp(qlinear("shared_expert.gate_proj", L, 2),
                              qlinear("shared_expert.up_proj", L, 2),
                              qlinear("shared_expert.down_proj", L, 2))
    f32_router = not lt.quantised("gate") and lt.get("gate.weight").dtype == torch.float32
    if not f32_router:
        # QuantizedLinear, or bf16 Linear (quantize_dense quantises the
        # expert and shared-expert projections only; a dense router stays
        # a bf16 Linear)
        def router(module):
            if lt.quantised(module):
                return qlinear(module, nn.QuantizedLinear, 2)
            return nn.Linear(lt.get(f"{module}.weight").to(dev, torch.bfloat16))
        gate = router("gate")
        if shared is not None:
            sgate = router("shared_expert_gate")
    else:
        gate = lt.get("gate.weight").to(dev, torch.float32)
        if shared is not None:
            sgate = lt.get("shared_expert_gate.weight").to(dev, torch.float32)
    return nn.Qwen35MoeBlock(gate, mlp, K, shared, sgate)


__all__ = ["list_shards", "sanitize_key", "QuantizationConfig", "read_config", "text_config",
           "LayerTensors", "qwen35_moe_block", "is_mlx_format", "post_attention_layernorm"]
