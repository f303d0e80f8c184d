"""mlxr-lm MoE modules over the gfx950 C ABI.

    SwitchLinear           crates/mlxr-lm/src/nn/switch.rs:49-94 (dense)
    RmsNorm                crates/mlxr/src/layers/normalization.rs:254-276
    Linear                 crates/mlxr/src/layers/linear.rs (dense, bf16)
    QuantizedSwitchLinear  crates/mlxr-lm/src/nn/switch.rs:115-168
    QuantizedLinear        crates/mlxr/src/layers/quantized.rs:214-379
    SwigluMlp              crates/mlxr-lm/src/nn/swiglu_mlp.rs:24-75
    SplitSwitchFfn         crates/mlxr-lm/src/nn/switch.rs:366-491
    Qwen35MoeBlock         crates/mlxr-lm/src/qwen3_5/text/moe.rs:43-159

Each module keeps its device tensors (torch, for memory) and the C
descriptor that points at them; forward() is one C-ABI call whose kernels
run on the current stream.
"""
from __future__ import annotations

import ctypes

import torch

from . import _capi as C
from . import ops
from ._capi import MlxrMoeError


class SwitchLinear:
    """Expert-stacked dense linear (the unquantised MaybeQuantized slot):
    weight bf16 [E, out, in], applied with gather_mm (switch.rs:84-93).  No
    bias: the MoE blocks build theirs without (moe.rs:92-97,
    gemma4/text/text.rs:679)."""

    bits = 16
    group_size = 0

    def __init__(self, weight):
        if weight.ndim != 3:
            raise MlxrMoeError("SwitchLinear weight must be [E, out, in]")
        self.weight = weight.to(torch.bfloat16).contiguous()

    @property
    def num_experts(self):
        return self.weight.shape[0]

    @property
    def output_dims(self):
        return self.weight.shape[1]

    @property
    def input_dims(self):
        return self.weight.shape[2]

    def apply(self, x, indices, sorted=False):
        """SwitchLinear::apply (switch.rs:84-93)."""
        return ops.gather_mm(x, self.weight, None, indices, sorted)

    def try_into_quantized(self, group_size=64, bits=4):
        """Quantizable::try_into_quantized (switch.rs:96-113)."""
        return QuantizedSwitchLinear.try_from_switch_linear(self.weight, group_size, bits)

    def descriptor(self) -> C.QLinear:
        return C.QLinear(self.weight.data_ptr(), None, None, self.num_experts,
                         self.output_dims, self.input_dims, 0, 16)


class Linear(SwitchLinear):
    """A dense bf16 Linear without bias (weight [out, in]) seen as one expert:
    the router and shared-expert projections of an unquantised checkpoint."""

    def __init__(self, weight):
        super().__init__(weight.reshape((1,) + tuple(weight.shape)))

    def try_into_quantized(self, group_size=64, bits=4):
        return QuantizedLinear.try_from_linear(self.weight[0], group_size, bits)

    def forward(self, x):
        """x @ weight^T in bf16 (layers/linear.rs:91-95)."""
        lead = tuple(x.shape[:-1])
        x2 = x.reshape(-1, 1, x.shape[-1])
        idx = torch.zeros(x2.shape[0], dtype=torch.int32, device=x.device)
        y = ops.gather_mm(x2, self.weight, None, idx)
        return y.reshape(lead + (self.output_dims,))


class QuantizedSwitchLinear:
    """Expert-stacked quantised linear: weight [E, out, in*bits/32] (int32
    storage of uint32 words), scales/biases bf16 [E, out, in/group]."""

    def __init__(self, weight, scales, biases, group_size=64, bits=4):
        if weight.ndim != 3:
            raise MlxrMoeError("QuantizedSwitchLinear weight must be [E, out, packed_in]")
        self.weight = weight.contiguous()
        self.scales = scales.contiguous()
        self.biases = biases.contiguous()
        self.group_size = group_size
        self.bits = bits

    @classmethod
    def try_from_switch_linear(cls, weight, group_size=64, bits=4):
        """QuantizedSwitchLinear::try_from_switch_linear (switch.rs:129-145)."""
        wq, s, b = ops.quantize(weight, group_size, bits)
        return cls(wq, s, b, group_size, bits)

    @property
    def num_experts(self):
        return self.weight.shape[0]

    @property
    def output_dims(self):
        return self.weight.shape[1]

    @property
    def input_dims(self):
        return self.weight.shape[2] * 32 // self.bits

    def apply(self, x, indices, sorted=False):
        """QuantizedSwitchLinear::apply (switch.rs:148-167)."""
        return ops.gather_qmm(x, self.weight, self.scales, self.biases, None, indices, True,
                              self.group_size, self.bits, sorted)

    def descriptor(self) -> C.QLinear:
        return C.QLinear(self.weight.data_ptr(), self.scales.data_ptr(), self.biases.data_ptr(),
                         self.num_experts, self.output_dims, self.input_dims,
                         self.group_size, self.bits)


class QuantizedLinear(QuantizedSwitchLinear):
    """A single quantised linear (weight [out, in*bits/32]) seen as one
    expert."""

    def __init__(self, weight, scales, biases, group_size=64, bits=4):
        super().__init__(weight.reshape((1,) + tuple(weight.shape)),
                         scales.reshape((1,) + tuple(scales.shape)),
                         biases.reshape((1,) + tuple(biases.shape)), group_size, bits)

    @classmethod
    def try_from_linear(cls, weight, group_size=64, bits=4):
        """QuantizedLinear::try_from_linear (layers/quantized.rs:249-273)."""
        wq, s, b = ops.quantize(weight, group_size, bits)
        return cls(wq, s, b, group_size, bits)

    def forward(self, x):
        """quantized_matmul(x, w, transpose=true) (layers/quantized.rs:356-373)."""
        lead = tuple(x.shape[:-1])
        x2 = x.reshape(-1, 1, x.shape[-1])
        idx = torch.zeros(x2.shape[0], dtype=torch.int32, device=x.device)
        y = ops.gather_qmm(x2, self.weight, self.scales, self.biases, None, idx, True,
                           self.group_size, self.bits)
        return y.reshape(lead + (self.output_dims,))


def _ptr(t):
    return None if t is None else t.data_ptr()


def _check_x(name: str, x, d: int, dtype=torch.bfloat16):
    """x must be a `dtype` tensor whose last dim is d: the C ABI reads
    T * d elements of that type.  (Callers check the device after every
    shape check.)"""
    if x.dtype != dtype:
        raise MlxrMoeError(f"{name}: x must be {dtype}, got {x.dtype}")
    if x.ndim < 1 or x.shape[-1] != d:
        raise MlxrMoeError(f"{name}: x last dim must be {d}, got {tuple(x.shape)}")


def _check_out(name: str, out, T: int, d: int, dtype, device):
    """A caller's out must hold exactly T x d elements of `dtype`,
    contiguously, on the inputs' device (the kernels write T * d of them)."""
    if out.dtype != dtype:
        raise MlxrMoeError(f"{name}: out must be {dtype}, got {out.dtype}")
    if out.numel() != T * d or (out.ndim and out.shape[-1] != d):
        raise MlxrMoeError(f"{name}: out must have shape ({T}, {d}), got {tuple(out.shape)}")
    if not out.is_contiguous():
        raise MlxrMoeError(f"{name}: out must be contiguous")
    if out.device != device:
        raise MlxrMoeError(f"{name}: out must be on {device}, got {out.device}")


class SplitSwitchFfn:
    """SplitSwitchFfn<SwigluActivation>: gate_proj, up_proj [E, f, d],
    down_proj [E, d, f]; all three QuantizedSwitchLinear or all three dense
    SwitchLinear."""

    def __init__(self, gate_proj: QuantizedSwitchLinear | SwitchLinear,
                 up_proj: QuantizedSwitchLinear | SwitchLinear,
                 down_proj: QuantizedSwitchLinear | SwitchLinear):
        self.gate_proj, self.up_proj, self.down_proj = gate_proj, up_proj, down_proj
        self._desc = C.SwitchGlu(gate_proj.descriptor(), up_proj.descriptor(),
                                 down_proj.descriptor())

    @classmethod
    def from_dense(cls, gate_w, up_w, down_w, group_size=64, bits=4):
        """Quantise dense expert weights, as try_into_quantized does
        (switch.rs:478-491)."""
        q = QuantizedSwitchLinear.try_from_switch_linear
        return cls(q(gate_w, group_size, bits), q(up_w, group_size, bits),
                   q(down_w, group_size, bits))

    def descriptor(self) -> C.SwitchGlu:
        return self._desc

    def _prep(self, x, indices):
        d = self.gate_proj.input_dims
        _check_x("SplitSwitchFfn", x, d)
        ops._dev(x, indices)
        x2 = x.reshape(-1, d).contiguous()
        K = indices.shape[-1]
        idx = indices.reshape(-1, K).to(torch.int32).contiguous()
        if idx.shape[0] != x2.shape[0]:
            raise MlxrMoeError("SplitSwitchFfn: indices must be [..., T, K] over x [..., T, d]")
        return x2, idx, K

    def forward(self, x, indices):
        """Per-expert outputs [..., K, d] (switch.rs:417-442)."""
        x2, idx, K = self._prep(x, indices)
        T, d = x2.shape
        y = torch.empty((T, K, d), dtype=torch.bfloat16, device=x.device)
        lib = C.lib()
        ws = ops.workspace(lib.mlxr_moe_switch_glu_workspace_size(ctypes.byref(self._desc), T, K),
                           x.device)
        C.check(lib.mlxr_moe_switch_glu_experts(
            ctypes.byref(self._desc), _ptr(x2), T, _ptr(idx), K, _ptr(y), _ptr(ws), ws.numel(),
            ops._stream(x)))
        self.last_workspace = ws
        return y.reshape(tuple(indices.shape) + (d,))

    def forward_with_combine(self, x, indices, weights):
        """sum_k weights * expert_k(x) -> f32 [..., d] (switch.rs:446-474)."""
        x2, idx, K = self._prep(x, indices)
        T, d = x2.shape
        ops._dev(x, weights)
        w = weights.reshape(-1, K).to(torch.float32).contiguous()
        out = torch.empty((T, d), dtype=torch.float32, device=x.device)
        lib = C.lib()
        ws = ops.workspace(lib.mlxr_moe_switch_glu_workspace_size(ctypes.byref(self._desc), T, K),
                           x.device)
        C.check(lib.mlxr_moe_switch_glu_forward(
            ctypes.byref(self._desc), _ptr(x2), T, _ptr(idx), _ptr(w), K, _ptr(out), _ptr(ws),
            ws.numel(), ops._stream(x)))
        self.last_workspace = ws
        return out.reshape(tuple(x.shape[:-1]) + (d,))


class PackedSwitchFfn:
    """PackedSwitchFfn (switch.rs:236-335), gemma4's expert layout:
    gate_up_proj [E, 2H, d] (gate channels first, split_sections at H) and
    down_proj [E, d, H], with GeGLU (GemmaSwitchGlu, gemma4/text/mod.rs:27)
    or SwiGLU between them."""

    def __init__(self, gate_up_proj: QuantizedSwitchLinear | SwitchLinear,
                 down_proj: QuantizedSwitchLinear | SwitchLinear, activation: str = "geglu"):
        if activation not in ("geglu", "swiglu"):
            raise MlxrMoeError("PackedSwitchFfn: activation is 'geglu' or 'swiglu'")
        if gate_up_proj.output_dims % 2:
            raise MlxrMoeError("PackedSwitchFfn: gate_up_proj must have 2 * hidden_dims rows")
        self.gate_up_proj, self.down_proj = gate_up_proj, down_proj
        self.activation = activation
        self.hidden_dims = gate_up_proj.output_dims // 2
        self._desc = C.PackedSwitchGlu(gate_up_proj.descriptor(), down_proj.descriptor(),
                                       C.ACT_GEGLU if activation == "geglu" else C.ACT_SWIGLU)

    @classmethod
    def from_dense(cls, gate_up_w, down_w, group_size=64, bits=4, activation="geglu"):
        """Quantise dense expert weights (try_into_quantized, switch.rs:323-335)."""
        q = QuantizedSwitchLinear.try_from_switch_linear
        return cls(q(gate_up_w, group_size, bits), q(down_w, group_size, bits), activation)

    def descriptor(self) -> C.PackedSwitchGlu:
        return self._desc

    def _prep(self, x, indices):
        d = self.gate_up_proj.input_dims
        _check_x("PackedSwitchFfn", x, d)
        ops._dev(x, indices)
        x2 = x.reshape(-1, d).contiguous()
        K = indices.shape[-1]
        idx = indices.reshape(-1, K).to(torch.int32).contiguous()
        if idx.shape[0] != x2.shape[0]:
            raise MlxrMoeError("PackedSwitchFfn: indices must be [..., T, K] over x [..., T, d]")
        return x2, idx, K

    def workspace_size(self, T: int, K: int) -> int:
        return C.lib().mlxr_moe_packed_switch_glu_workspace_size(ctypes.byref(self._desc), T, K)

    def forward(self, x, indices):
        """Per-expert outputs [..., K, d] bf16 (switch.rs:290-315)."""
        x2, idx, K = self._prep(x, indices)
        T, d = x2.shape
        y = torch.empty((T, K, d), dtype=torch.bfloat16, device=x.device)
        ws = ops.workspace(self.workspace_size(T, K), x.device)
        C.check(C.lib().mlxr_moe_packed_switch_glu_experts(
            ctypes.byref(self._desc), _ptr(x2), T, _ptr(idx), K, _ptr(y), _ptr(ws), ws.numel(),
            ops._stream(x)))
        self.last_workspace = ws
        return y.reshape(tuple(indices.shape) + (d,))

    def forward_with_combine(self, x, indices, weights, out=None, workspace=None):
        """sum_k weights * expert_k(x) (switch.rs:316-335): f32 weights give
        an f32 [..., d], bf16 weights (gemma4's router) a bf16 one."""
        x2, idx, K = self._prep(x, indices)
        T, d = x2.shape
        bf16 = weights.dtype == torch.bfloat16
        w = weights.reshape(-1, K).contiguous()
        if not bf16:
            w = w.to(torch.float32)
        odt = torch.bfloat16 if bf16 else torch.float32
        ops._dev(x, weights)
        if out is None:
            out = torch.empty((T, d), dtype=odt, device=x.device)
        else:
            _check_out("PackedSwitchFfn", out, T, d, odt, x.device)
        if workspace is None:
            workspace = ops.workspace(self.workspace_size(T, K), x.device)
        C.check(C.lib().mlxr_moe_packed_switch_glu_forward(
            ctypes.byref(self._desc), _ptr(x2), T, _ptr(idx), _ptr(w),
            C.BFLOAT16 if bf16 else C.FLOAT32, K, _ptr(out), _ptr(workspace), workspace.numel(),
            ops._stream(x)))
        self.last_workspace = workspace
        return out.reshape(tuple(x.shape[:-1]) + (d,))

    __call__ = forward_with_combine


class GemmaRouter:
    """gemma4's Router (gemma4/text/text.rs:568-665): rms_norm(x, scale *
    root_size) -> proj (a bf16 Linear [E, d], or a QuantizedLinear) -> top-K
    of the bf16 scores -> softmax of the K scores * per_expert_scale; bf16
    throughout."""

    def __init__(self, proj, scale, per_expert_scale, top_k: int, eps: float = 1e-6):
        self.quantised = isinstance(proj, QuantizedLinear)
        if self.quantised:
            self.proj = proj
            E, d = proj.output_dims, proj.input_dims
        else:
            self.proj = proj.to(torch.bfloat16).contiguous()
            E, d = self.proj.shape
        self.top_k, self.eps, self.num_experts, self.hidden_size = top_k, eps, E, d
        # scale * root_size in scale's dtype, once (text.rs:626-637)
        scale = scale.to(torch.bfloat16)
        root = torch.tensor(d ** -0.5, dtype=torch.float32).to(torch.bfloat16)
        self.norm_weight = (scale * root.to(scale.device)).contiguous()
        self.per_expert_scale = per_expert_scale.to(torch.bfloat16).contiguous()
        z = C.QLinear()
        self._desc = C.GemmaRouter(
            d, E, top_k, eps, self.norm_weight.data_ptr(),
            None if self.quantised else self.proj.data_ptr(),
            self.proj.descriptor() if self.quantised else z, self.per_expert_scale.data_ptr())

    def descriptor(self) -> C.GemmaRouter:
        return self._desc

    def workspace_size(self, T: int) -> int:
        return C.lib().mlxr_moe_gemma_router_workspace_size(ctypes.byref(self._desc), T)

    def forward(self, x, idx=None, weights=None, workspace=None):
        """x bf16 [..., d] -> (indices int32 [..., K], weights bf16 [..., K])."""
        d = self.hidden_size
        _check_x("GemmaRouter", x, d)
        ops._dev(x)
        x2 = x.reshape(-1, d).contiguous()
        T, K = x2.shape[0], self.top_k
        if idx is None:
            idx = torch.empty((T, K), dtype=torch.int32, device=x.device)
        if weights is None:
            weights = torch.empty((T, K), dtype=torch.bfloat16, device=x.device)
        if workspace is None:
            workspace = ops.workspace(self.workspace_size(T), x.device)
        C.check(C.lib().mlxr_moe_gemma_router_forward(
            ctypes.byref(self._desc), _ptr(x2), T, _ptr(idx), _ptr(weights), _ptr(workspace),
            workspace.numel(), ops._stream(x)))
        lead = tuple(x.shape[:-1])
        return idx.reshape(lead + (K,)), weights.reshape(lead + (K,))

    __call__ = forward


class GemmaMoe:
    """The routed half of a gemma4 MoE layer (text.rs:901-917): router(h)
    and Experts(h2, indices, weights) = PackedSwitchFfn<Geglu>::
    forward_with_combine.  bf16 in and out.  (The layer's norms and the
    dense MLP branch around it are outside this path; here the experts see
    the router's input.)"""

    out_dtype = torch.bfloat16

    def __init__(self, router: GemmaRouter, experts: PackedSwitchFfn):
        self.router, self.experts = router, experts
        self.last_indices = self.last_weights = self.last_workspace = None
        self._ws = None

    def workspace_size(self, T: int) -> int:
        a = self.router.workspace_size(T)
        return ((a + 255) // 256) * 256 + self.experts.workspace_size(T, self.router.top_k)

    def forward(self, x, out=None, workspace=None, keep_routing=True):
        d = self.router.hidden_size
        _check_x("GemmaMoe", x, d)
        ops._dev(x)
        x2 = x.reshape(-1, d).contiguous()
        T, K = x2.shape[0], self.router.top_k
        if workspace is None:
            need = self.workspace_size(T)
            if self._ws is None or self._ws.numel() < need or self._ws.device != x.device:
                self._ws = ops.workspace(need, x.device)
            workspace = self._ws
        ra = ((self.router.workspace_size(T) + 255) // 256) * 256
        key = (T, x.device)
        if getattr(self, "_route_key", None) != key:
            self._route = (torch.empty((T, K), dtype=torch.int32, device=x.device),
                           torch.empty((T, K), dtype=torch.bfloat16, device=x.device))
            self._route_key = key
        idx, w = self._route
        self.router.forward(x2, idx, w, workspace[:ra])
        o = self.experts.forward_with_combine(x2, idx, w, out=out, workspace=workspace[ra:])
        self.last_indices = idx if keep_routing else None
        self.last_weights = w if keep_routing else None
        self.last_workspace = workspace[ra:]
        return o.reshape(tuple(x.shape[:-1]) + (d,))

    __call__ = forward


class SwigluMlp:
    """down(silu(gate(x)) * up(x)) with QuantizedLinear (or dense bf16 Linear)
    projections."""

    def __init__(self, gate_proj: QuantizedLinear, up_proj: QuantizedLinear,
                 down_proj: QuantizedLinear):
        self.gate_proj, self.up_proj, self.down_proj = gate_proj, up_proj, down_proj

    def forward(self, x):
        """SwigluMlp::forward (swiglu_mlp.rs:63-70); bf16 output.  Runs as
        a one-expert SplitSwitchFfn with routing weight 1 (exact)."""
        ffn = SplitSwitchFfn(self.gate_proj, self.up_proj, self.down_proj)
        lead = tuple(x.shape[:-1])
        T = x.numel() // x.shape[-1]
        idx = torch.zeros((T, 1), dtype=torch.int32, device=x.device)
        return ffn.forward(x.reshape(T, -1), idx).reshape(lead + (-1,))


class Qwen35MoeBlock:
    """Router -> softmax -> top-k -> renormalise -> SplitSwitchFfn, plus an
    optional sigmoid-gated shared SwigluMlp (moe.rs:43-159).

    The router (`gate_weight`) and the shared gate
    (`shared_expert_gate_weight`) are MaybeQuantized<Linear> as in the
    reference (moe.rs:57-58): an f32 weight tensor [E, d] / [1, d], or both a
    QuantizedLinear (the shipped Qwen3.6 checkpoints quantise them at 8 bits,
    moe.rs:255-284), or both a bf16 Linear (an unquantised checkpoint).  With
    a QuantizedLinear or bf16 Linear router the block is bf16 throughout
    (logits, probabilities, routing weights and the output).  The experts
    and the shared expert may be dense (SwitchLinear / Linear projections)."""

    def __init__(self, gate_weight, switch_mlp: SplitSwitchFfn, num_experts_per_tok: int,
                 shared_expert: SwigluMlp | None = None, shared_expert_gate_weight=None,
                 gate_bias=None):
        if (shared_expert is None) != (shared_expert_gate_weight is None):
            raise MlxrMoeError("shared_expert and shared_expert_gate_weight go together")
        def form(w):
            return ("q" if isinstance(w, QuantizedLinear) else
                    "bf16" if isinstance(w, Linear) else "f32")

        # the bf16 router: a QuantizedLinear or a bf16 Linear
        self.quantised_router = form(gate_weight) != "f32"
        if shared_expert_gate_weight is not None and (
                form(shared_expert_gate_weight) != form(gate_weight)):
            raise MlxrMoeError("gate and shared_expert_gate must take the same form "
                               "(both QuantizedLinear, both Linear or both f32 tensors)")
        if self.quantised_router and gate_bias is not None:
            raise MlxrMoeError("the router has no bias (moe.rs:89-91)")
        z = C.QLinear()
        if self.quantised_router:
            self.gate_weight = gate_weight
            self.gate_bias = None
            self.shared_expert_gate_weight = shared_expert_gate_weight
            E, d = gate_weight.output_dims, gate_weight.input_dims
            gate_ptr = sgw_ptr = None
            gate_q = gate_weight.descriptor()
            sg_q = z if shared_expert_gate_weight is None else shared_expert_gate_weight.descriptor()
        else:
            self.gate_weight = gate_weight.to(torch.float32).contiguous()
            self.gate_bias = (None if gate_bias is None
                              else gate_bias.to(torch.float32).contiguous())
            self.shared_expert_gate_weight = (
                None if shared_expert_gate_weight is None
                else shared_expert_gate_weight.to(torch.float32).contiguous())
            E, d = self.gate_weight.shape
            gate_ptr, sgw_ptr = self.gate_weight.data_ptr(), _ptr(self.shared_expert_gate_weight)
            gate_q = sg_q = z
        self.switch_mlp = switch_mlp
        self.shared_expert = shared_expert
        self.num_experts_per_tok = num_experts_per_tok
        self.out_dtype = torch.bfloat16 if self.quantised_router else torch.float32
        self.hidden_size = d
        f = switch_mlp.gate_proj.output_dims
        se = shared_expert
        self._desc = C.Block(
            d, E, num_experts_per_tok, f,
            0 if se is None else se.gate_proj.output_dims,
            gate_ptr, _ptr(self.gate_bias), switch_mlp.descriptor(),
            z if se is None else se.gate_proj.descriptor(),
            z if se is None else se.up_proj.descriptor(),
            z if se is None else se.down_proj.descriptor(),
            sgw_ptr, gate_q, sg_q)
        self._ws = None
        self.last_indices = None
        self.last_weights = None

    def descriptor(self) -> C.Block:
        return self._desc

    def workspace_size(self, T: int) -> int:
        return C.lib().mlxr_moe_block_workspace_size(ctypes.byref(self._desc), T)

    def forward(self, x, out=None, workspace=None, keep_routing=True):
        """Qwen35MoeBlock::forward (moe.rs:116-146): x bf16 [..., d] ->
        [..., d], f32 (bf16 with a quantised router)."""
        d = self.hidden_size
        _check_x("Qwen35MoeBlock", x, d)
        ops._dev(x)
        x2 = x.reshape(-1, d)
        if not x2.is_contiguous():
            x2 = x2.contiguous()
        T = x2.shape[0]
        K = self.num_experts_per_tok
        if out is None:
            out = torch.empty((T, d), dtype=self.out_dtype, device=x.device)
        else:
            _check_out("Qwen35MoeBlock", out, T, d, self.out_dtype, x.device)
        if workspace is not None:
            ops._dev(x, workspace)
        if workspace is None:
            need = self.workspace_size(T)
            if self._ws is None or self._ws.numel() < need or self._ws.device != x.device:
                self._ws = ops.workspace(need, x.device)
            workspace = self._ws
        idx = wts = None
        if keep_routing:
            idx = torch.empty((T, K), dtype=torch.int32, device=x.device)
            wts = torch.empty((T, K), dtype=torch.float32, device=x.device)
        C.check(C.lib().mlxr_moe_block_forward(
            ctypes.byref(self._desc), _ptr(x2), T, _ptr(out), _ptr(idx), _ptr(wts),
            _ptr(workspace), workspace.numel(), ops._stream(x)))
        self.last_indices, self.last_weights = idx, wts
        self.last_workspace = workspace
        return out.reshape(tuple(x.shape[:-1]) + (d,))

    __call__ = forward

    def residual_workspace_size(self, T: int) -> int:
        return C.lib().mlxr_moe_block_residual_workspace_size(ctypes.byref(self._desc), T)

    def forward_residual(self, h, norm: "RmsNorm", out=None, workspace=None,
                         keep_routing=True):
        """The decoder layer's MoE half (layer.rs:134-138): h + self(norm(h)),
        the norm (post_attention_layernorm) one kernel before the block and
        the add fused into its combine.  h bf16 [..., d]; out f32 (bf16 with
        a bf16 router)."""
        d = self.hidden_size
        _check_x("Qwen35MoeBlock.forward_residual", h, d)
        if norm.weight.numel() != d:
            raise MlxrMoeError(f"forward_residual: the norm weight must have {d} elements, "
                               f"got {norm.weight.numel()}")
        ops._dev(h, norm.weight)
        h2 = h.reshape(-1, d).contiguous()
        T, K = h2.shape[0], self.num_experts_per_tok
        if out is None:
            out = torch.empty((T, d), dtype=self.out_dtype, device=h.device)
        else:
            _check_out("Qwen35MoeBlock.forward_residual", out, T, d, self.out_dtype, h.device)
        if workspace is not None:
            ops._dev(h, workspace)
        if workspace is None:
            workspace = ops.workspace(self.residual_workspace_size(T), h.device)
        idx = wts = None
        if keep_routing:
            idx = torch.empty((T, K), dtype=torch.int32, device=h.device)
            wts = torch.empty((T, K), dtype=torch.float32, device=h.device)
        C.check(C.lib().mlxr_moe_block_forward_residual(
            ctypes.byref(self._desc), _ptr(norm.weight), norm.eps, _ptr(h2), T, _ptr(out),
            _ptr(idx), _ptr(wts), _ptr(workspace), workspace.numel(), ops._stream(h)))
        self.last_indices, self.last_weights = idx, wts
        self.last_workspace = workspace
        return out.reshape(tuple(h.shape[:-1]) + (d,))


class RmsNorm:
    """layers::RmsNorm (crates/mlxr/src/layers/normalization.rs:254-276):
    fast::rms_norm(x, weight, eps), bf16.  The weight is the one the model
    holds (a Qwen3.5 checkpoint's +1.0 shift already applied by the
    loader)."""

    def __init__(self, weight, eps: float = 1e-6):
        if weight.ndim != 1:
            raise MlxrMoeError("RmsNorm weight must be [d]")
        self.weight = weight.to(torch.bfloat16).contiguous()
        self.eps = float(eps)

    def forward(self, x):
        d = x.shape[-1]
        if d != self.weight.numel():
            raise MlxrMoeError("RmsNorm: last dim does not match the weight")
        _check_x("RmsNorm", x, d)
        x2 = x.reshape(-1, d).contiguous()
        ops._dev(x2, self.weight)
        out = torch.empty_like(x2, dtype=torch.bfloat16)
        C.check(C.lib().mlxr_moe_rms_norm(_ptr(x2), x2.shape[0], d, _ptr(self.weight), self.eps,
                                          _ptr(out), ops._stream(x)))
        return out.reshape(x.shape)

    __call__ = forward
