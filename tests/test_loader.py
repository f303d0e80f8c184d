"""The checkpoint reader (mlx-rs_amd/loader.py) on the reference's naming:
key sanitising, the per-path quantisation overrides of the shipped
Qwen3.6-35B-A3B config (tests/golden/qwen3_6_35b_a3b_config.json, the
quantization block of crates/mlxr-lm/tests/fixtures/qwen3_6_35b_a3b/
config.json), and a synthetic sharded checkpoint read back bit for bit.
CPU only."""
import json
from pathlib import Path

import numpy as np
import pytest

torch = pytest.importorskip("torch")
safetensors_torch = pytest.importorskip("safetensors.torch")

GOLDEN = Path(__file__).resolve().parent / "golden" / "qwen3_6_35b_a3b_config.json"


def test_sanitize_key(pkg):
    L = pkg.loader
    assert (L.sanitize_key("model.language_model.layers.3.mlp.gate.weight")
            == "language_model.model.layers.3.mlp.gate.weight")
    assert L.sanitize_key("model.visual.blocks.0.x") == "vision_tower.blocks.0.x"
    assert L.sanitize_key("lm_head.weight") == "language_model.lm_head.weight"
    assert L.sanitize_key("language_model.model.norm.weight") == "language_model.model.norm.weight"


def test_quantization_overrides_of_the_shipped_config(pkg):
    """quantization.rs:51-56 on the real config: the body is 4-bit g64, every
    layer's mlp.gate and mlp.shared_expert_gate are 8-bit g64."""
    cfg = json.loads(GOLDEN.read_text())
    q = pkg.loader.QuantizationConfig.from_config(cfg)
    assert (q.group_size, q.bits, q.mode) == (64, 4, "affine")
    n_layers = cfg["text_config"]["num_hidden_layers"]
    assert len(q.overrides) == 2 * n_layers
    for i in (0, n_layers - 1):
        p = f"language_model.model.layers.{i}.mlp."
        assert q.for_path(p + "gate") == (64, 8)
        assert q.for_path(p + "shared_expert_gate") == (64, 8)
        assert q.for_path(p + "switch_mlp.gate_proj") == (64, 4)
        assert q.for_path(p + "shared_expert.down_proj") == (64, 4)


def _write_checkpoint(d: Path, tensors: dict, config: dict, shards=1, fmt="mlx"):
    d.mkdir(parents=True, exist_ok=True)
    (d / "config.json").write_text(json.dumps(config))
    keys = sorted(tensors)
    if shards == 1:
        safetensors_torch.save_file(tensors, str(d / "model.safetensors"),
                                    metadata={"format": fmt})
        return
    weight_map = {}
    for s in range(shards):
        name = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
        part = {k: tensors[k] for k in keys[s::shards]}
        safetensors_torch.save_file(part, str(d / name), metadata={"format": fmt})
        weight_map.update({k: name for k in part})
    (d / "model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}))


def _synthetic(orc, rng, E=8, d=512, f=256, fs=256):
    def q(shape, bits):
        w = orc.f32_to_bf16((rng.standard_normal(shape) * 0.02).astype(np.float32))
        wq, sc, bi = orc.quantize(w.reshape(-1, shape[-1]), 64, bits)
        return (wq.reshape(shape[:-1] + (-1,)), sc.reshape(shape[:-1] + (-1,)),
                bi.reshape(shape[:-1] + (-1,)))
    mods = {"switch_mlp.gate_proj": q((E, f, d), 4), "switch_mlp.up_proj": q((E, f, d), 4),
            "switch_mlp.down_proj": q((E, d, f), 4), "shared_expert.gate_proj": q((fs, d), 4),
            "shared_expert.up_proj": q((fs, d), 4), "shared_expert.down_proj": q((d, fs), 4),
            "gate": q((E, d), 8), "shared_expert_gate": q((1, d), 8)}
    return mods


def _as_tensors(prefix, mods):
    out = {}
    for m, (wq, sc, bi) in mods.items():
        out[f"{prefix}{m}.weight"] = torch.from_numpy(wq.view(np.int32)).view(torch.uint32)
        out[f"{prefix}{m}.scales"] = torch.from_numpy(sc.view(np.int16)).view(torch.bfloat16)
        out[f"{prefix}{m}.biases"] = torch.from_numpy(bi.view(np.int16)).view(torch.bfloat16)
    return out


@pytest.mark.parametrize("shards", [1, 3])
def test_read_back_quantised_layer(pkg, orc, tmp_path, shards):
    """A Qwen3.6-style layer (4-bit experts, 8-bit router and shared gate by
    override) written under the checkpoint's own key prefix reads back into
    Qwen35MoeBlock modules with every code, scale and bias unchanged."""
    rng = np.random.default_rng(60)
    mods = _synthetic(orc, rng)
    t = _as_tensors("model.language_model.layers.2.mlp.", mods)
    t["model.language_model.layers.1.mlp.gate.weight"] = torch.zeros(4, dtype=torch.bfloat16)
    qcfg = {"group_size": 64, "bits": 4, "mode": "affine",
            "language_model.model.layers.2.mlp.gate": {"group_size": 64, "bits": 8},
            "language_model.model.layers.2.mlp.shared_expert_gate": {"group_size": 64, "bits": 8}}
    cfg = {"quantization": qcfg, "text_config": {"num_experts_per_tok": 2}}
    _write_checkpoint(tmp_path / "ck", t, cfg, shards)
    blk = pkg.loader.qwen35_moe_block(tmp_path / "ck", 2, "cpu")
    assert blk.quantised_router and blk.num_experts_per_tok == 2
    got = {"switch_mlp.gate_proj": blk.switch_mlp.gate_proj, "switch_mlp.up_proj": blk.switch_mlp.up_proj,
           "switch_mlp.down_proj": blk.switch_mlp.down_proj,
           "shared_expert.gate_proj": blk.shared_expert.gate_proj,
           "shared_expert.up_proj": blk.shared_expert.up_proj,
           "shared_expert.down_proj": blk.shared_expert.down_proj,
           "gate": blk.gate_weight, "shared_expert_gate": blk.shared_expert_gate_weight}
    for m, lin in got.items():
        wq, sc, bi = mods[m]
        assert lin.bits == (8 if m in ("gate", "shared_expert_gate") else 4), m
        assert np.array_equal(lin.weight.reshape(wq.shape).numpy().view(np.uint32), wq), m
        assert np.array_equal(lin.scales.reshape(sc.shape).view(torch.int16).numpy().view(np.uint16), sc)
        assert np.array_equal(lin.biases.reshape(bi.shape).view(torch.int16).numpy().view(np.uint16), bi)


def test_hf_packed_experts_split_and_loaded_dense(pkg, tmp_path):
    """mlp.experts.gate_up_proj [E, 2H, D] (an unconverted checkpoint) splits
    along axis 1 into gate and up (mlxr-convert/src/qwen3_5.rs:96-147); the
    dense experts load as bf16 SwitchLinears (gather_mm) and the bf16 router
    as a Linear (a bf16 block, as the reference computes it)."""
    E, d, H = 4, 256, 128
    g = torch.Generator().manual_seed(1)
    gu = (torch.randn((E, 2 * H, d), generator=g) * 0.02).to(torch.bfloat16)
    dn = (torch.randn((E, d, H), generator=g) * 0.02).to(torch.bfloat16)
    p = "model.language_model.layers.0.mlp."
    t = {p + "experts.gate_up_proj": gu, p + "experts.down_proj": dn,
         p + "gate.weight": torch.randn((E, d), generator=g).to(torch.bfloat16)}
    _write_checkpoint(tmp_path / "hf", t, {"text_config": {"num_experts_per_tok": 2}})
    lt = pkg.loader.LayerTensors(tmp_path / "hf", 0)
    assert torch.equal(lt.get("switch_mlp.gate_proj.weight"), gu[:, :H])
    assert torch.equal(lt.get("switch_mlp.up_proj.weight"), gu[:, H:])
    blk = pkg.loader.qwen35_moe_block(tmp_path / "hf", 0, "cpu")
    m = blk.switch_mlp
    assert all(isinstance(x, pkg.nn.SwitchLinear) for x in (m.gate_proj, m.up_proj, m.down_proj))
    assert torch.equal(m.gate_proj.weight, gu[:, :H]) and torch.equal(m.up_proj.weight, gu[:, H:])
    assert torch.equal(m.down_proj.weight, dn)
    assert isinstance(blk.gate_weight, pkg.nn.Linear) and blk.quantised_router
    assert blk.out_dtype == torch.bfloat16 and blk.shared_expert is None
    # an f32 router stays the f32 Linear path
    t[p + "gate.weight"] = t[p + "gate.weight"].float()
    _write_checkpoint(tmp_path / "hf32", t, {"text_config": {"num_experts_per_tok": 2}})
    blk = pkg.loader.qwen35_moe_block(tmp_path / "hf32", 0, "cpu")
    assert not blk.quantised_router and blk.gate_weight.dtype == torch.float32


@pytest.mark.parametrize("fmt", ["mlx", "pt"])
def test_post_attention_layernorm_shift(pkg, tmp_path, fmt):
    """weights.rs:147-165: a non-mlx-format checkpoint's norm weight gets
    +1.0 in its own dtype (bf16 here: 0.5 -> 1.5, 2^-9 -> 1.0 after
    rounding); an mlx-format one is taken as stored.  eps is rms_norm_eps."""
    p = "model.language_model.layers.3."
    w = torch.tensor([0.5, -0.25, 2.0 ** -9, 3.0], dtype=torch.bfloat16)
    t = {p + "post_attention_layernorm.weight": w,
         p + "input_layernorm.weight": torch.zeros(4, dtype=torch.bfloat16)}
    _write_checkpoint(tmp_path / fmt, t, {"text_config": {"rms_norm_eps": 1e-5}}, fmt=fmt)
    norm = pkg.loader.post_attention_layernorm(tmp_path / fmt, 3, "cpu")
    assert norm.eps == pytest.approx(1e-5)
    want = w if fmt == "mlx" else torch.tensor([1.5, 0.75, 1.0, 4.0], dtype=torch.bfloat16)
    assert torch.equal(norm.weight, want)
    with pytest.raises(pkg.MlxrMoeError):
        pkg.loader.post_attention_layernorm(tmp_path / fmt, 2, "cpu")
