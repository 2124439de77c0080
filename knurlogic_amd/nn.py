"""Module mirrors of the layers that call the quantized ops.

- ``QuantizedLinear``: mlx's nn.QuantizedLinear as swapped in by the
  reference's loader (src/knurlogic/engine/model/load_model.py:124-144).
- ``QuantizedSwitchLinear`` / ``SwitchGLU``: mlx-lm's switch layers
  (vendored twin at src/knurlogic/engine/families/glm5/architecture/
  glm5_next/_mlx_vlm/models/switch_layers.py:24-86,156-193).
- ``VQSwitchLinear`` / ``VQSwitchGLU``: the codebook-decode experts VQ
  artifacts ship in their model.py (class named at tests/engine/
  test_deepseek_v4_mtp.py:249,360): 8-element vectors with byte or 16-bit
  indices, or the on-disk packed layout (2-8-element vectors, 8-12 or
  16-bit fields), fp16 codebook and scales.
- ``MLP`` / ``SparseMoeBlock``: Qwen3.5-MoE's expert block with the
  reference's rounding edits (src/knurlogic/engine/families/qwen/
  architecture/qwen3_5.py:35-40,108-118,151-192).

Tensors live in GPU memory (torch); every product and every elementwise
step runs in the HIP library -- the dense (unquantized) router and
shared-expert gate too (``Linear``, kmi_linear).
"""
from __future__ import annotations

import math

import torch

from .ops import (add_bias, gather_qmm, linear, moe_combine, moe_experts, moe_route,
                  moe_shared_add, quantize, quantized_matmul, swiglu, switch_glu, switch_glu_mx, vq_gather_qmm,
                  vq_experts, vq_glu, vq_packed_experts, vq_packed_gather_qmm, vq_packed_glu, vq_packed_switch_glu,
                  vq_switch_glu)


class Linear:
    """mlx's nn.Linear for a layer the loader left unquantized (the router,
    the shared-expert gate): x @ w^T, or addmm(bias, x, w^T), through
    kmi_linear."""

    def __init__(self, weight: torch.Tensor, bias: torch.Tensor | None = None):
        self.weight, self.bias = weight, bias

    def __call__(self, x):
        return linear(x, self.weight, self.bias)


class QuantizedLinear:
    """nn.QuantizedLinear: y = quantized_matmul(x, w, scales, biases) (+ bias)."""

    def __init__(self, weight, scales, biases, bias=None, group_size: int = 64, bits: int = 4,
                 mode: str = "affine"):
        self.weight, self.scales, self.biases, self.bias = weight, scales, biases, bias
        self.group_size, self.bits, self.mode = group_size, bits, mode

    @classmethod
    def from_float(cls, w: torch.Tensor, bias=None, group_size: int = 64, bits: int = 4):
        return cls(*quantize(w, group_size=group_size, bits=bits), bias, group_size, bits)

    @property
    def input_dims(self):
        return self.scales.shape[-1] * self.group_size

    @property
    def output_dims(self):
        return self.weight.shape[0]

    def __call__(self, x):
        y = quantized_matmul(x, self.weight, self.scales, self.biases, transpose=True,
                             group_size=self.group_size, bits=self.bits, mode=self.mode)
        return add_bias(y, self.bias) if self.bias is not None else y


class QuantizedSwitchLinear:
    """QuantizedSwitchLinear (switch_layers.py:24-86): per-row expert matmul
    through gather_qmm over weight [E, N, K*bits/32]."""

    def __init__(self, weight, scales, biases, bias=None, group_size: int = 64, bits: int = 4,
                 mode: str = "affine"):
        self.weight, self.scales, self.biases, self.bias = weight, scales, biases, bias
        self.group_size, self.bits, self.mode = group_size, bits, mode

    @classmethod
    def from_float(cls, w: torch.Tensor, bias=None, group_size: int = 64, bits: int = 4):
        """w [E, N, K] -> the quantized layer (mx.quantize per expert row)."""
        return cls(*quantize(w, group_size=group_size, bits=bits), bias, group_size, bits)

    @property
    def input_dims(self):
        return self.scales.shape[2] * self.group_size

    @property
    def output_dims(self):
        return self.weight.shape[1]

    @property
    def num_experts(self):
        return self.weight.shape[0]

    def __call__(self, x, indices, sorted_indices: bool = False):
        y = gather_qmm(x, self.weight, self.scales, self.biases, rhs_indices=indices,
                       transpose=True, group_size=self.group_size, bits=self.bits,
                       mode=self.mode, sorted_indices=sorted_indices)
        if self.bias is not None:
            y = add_bias(y, self.bias, indices)
        return y


def _stackable(a: QuantizedSwitchLinear, b: QuantizedSwitchLinear) -> bool:
    return (a.weight.shape == b.weight.shape and a.scales.shape == b.scales.shape
            and a.group_size == b.group_size and a.bits == b.bits and a.bias is None
            and b.bias is None and a.weight.dtype == b.weight.dtype and a.scales.dtype == b.scales.dtype
            and a.mode == b.mode and (a.biases is None) == (b.biases is None))


class SwitchGLU:
    """SwitchGLU (switch_layers.py:156-193) with Qwen3.5's _SwiGLU
    activation: per (token, slot) the expert's gate and up projections,
    round(round(silu_f32(gate)) * up), and the down projection.

    Gate and up are stacked into one [E, 2I, K] weight at construction, so
    one gather_qmm streams both (each routed expert's bytes read once per
    call); ``gate_proj`` / ``up_proj`` stay available as views of it.  The
    reference sorts pairs by expert when indices.size >= 64 (:175); the
    kernels group rows by expert on every call, and sorting only reorders
    rows, so the result is the same either way."""

    def __init__(self, gate_proj: QuantizedSwitchLinear, up_proj: QuantizedSwitchLinear,
                 down_proj: QuantizedSwitchLinear):
        self.down_proj = down_proj
        self.fused = None
        if _stackable(gate_proj, up_proj):
            cat = lambda a, b: None if a is None else torch.cat([a, b], dim=1).contiguous()
            mode = gate_proj.mode
            self.fused = QuantizedSwitchLinear(cat(gate_proj.weight, up_proj.weight),
                                               cat(gate_proj.scales, up_proj.scales),
                                               cat(gate_proj.biases, up_proj.biases),
                                               None, gate_proj.group_size, gate_proj.bits, mode)
            I = gate_proj.output_dims
            view = lambda t, lo: None if t is None else t[:, lo:lo + I]
            self.gate_proj = QuantizedSwitchLinear(view(self.fused.weight, 0), view(self.fused.scales, 0),
                                                   view(self.fused.biases, 0), None,
                                                   gate_proj.group_size, gate_proj.bits, mode)
            self.up_proj = QuantizedSwitchLinear(view(self.fused.weight, I), view(self.fused.scales, I),
                                                 view(self.fused.biases, I), None,
                                                 up_proj.group_size, up_proj.bits, mode)
        else:
            self.gate_proj, self.up_proj = gate_proj, up_proj

    @classmethod
    def from_float(cls, gate_w, up_w, down_w, group_size: int = 64, bits: int = 4):
        q = lambda w: QuantizedSwitchLinear.from_float(w, None, group_size, bits)
        return cls(q(gate_w), q(up_w), q(down_w))

    def _one_call(self, k: int) -> bool:
        f, d = self.fused, self.down_proj
        return (f is not None and d.bias is None and k <= 8 and f.bits == d.bits and f.mode == "affine"
                and d.mode == "affine" and f.group_size == d.group_size and f.scales.dtype == torch.bfloat16)

    def _one_call_mx(self, x: torch.Tensor, k: int) -> bool:
        """mxfp4 / mxfp8 experts in one call (kmi_switch_glu_mx)."""
        f, d = self.fused, self.down_proj
        return (f is not None and d.bias is None and k <= 8 and f.mode in ("mxfp4", "mxfp8")
                and d.mode == f.mode and x.dtype == torch.bfloat16
                and x.shape[-1] % 64 == 0 and (f.weight.shape[1] // 2) % 64 == 0)

    def __call__(self, x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        """x [..., H], indices [..., k] (int) -> [..., k, H]."""
        return self._experts(x, indices, None)

    def combine(self, x: torch.Tensor, indices: torch.Tensor, scores: torch.Tensor) -> torch.Tensor:
        """The experts' outputs weighted by ``scores`` and summed over the k
        slots (SparseMoeBlock's combine, qwen3_5.py:181-182) -> [..., H]."""
        return self._experts(x, indices, scores)

    def _experts(self, x, indices, scores):
        k = indices.shape[-1]
        f, d = self.fused, self.down_proj
        if self._one_call(k) and x.dtype == torch.bfloat16:
            return switch_glu(x, indices, f.weight, f.scales, f.biases, d.weight, d.scales, d.biases,
                              scores, f.group_size, f.bits)
        if self._one_call_mx(x, k):
            return switch_glu_mx(x, indices, f.weight, f.scales, d.weight, d.scales, scores, f.mode)
        y = self.gathered(x, indices)
        return y if scores is None else moe_combine(y, scores)

    def gathered(self, x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        """The same through separate gather_qmm calls (any layer mix)."""
        lead, H = x.shape[:-1], x.shape[-1]
        k = indices.shape[-1]
        T = math.prod(lead)
        P = T * k
        x3 = x.reshape(T, 1, H)
        rhs = indices.reshape(P).to(torch.int32)
        tok = torch.arange(P, device=x.device, dtype=torch.int32) // k
        if self.fused is not None:
            f = self.fused
            gu = gather_qmm(x3, f.weight, f.scales, f.biases, lhs_indices=tok, rhs_indices=rhs,
                            group_size=f.group_size, bits=f.bits, mode=f.mode)  # [P, 1, 2I]
            act = swiglu(gu)                                                   # [P, 1, I]
        else:
            g, u = self.gate_proj, self.up_proj
            gate = gather_qmm(x3, g.weight, g.scales, g.biases, lhs_indices=tok, rhs_indices=rhs,
                              group_size=g.group_size, bits=g.bits, mode=g.mode)
            up = gather_qmm(x3, u.weight, u.scales, u.biases, lhs_indices=tok, rhs_indices=rhs,
                            group_size=u.group_size, bits=u.bits, mode=u.mode)
            act = swiglu(gate, up)
        d = self.down_proj
        pairs = torch.arange(P, device=x.device, dtype=torch.int32)
        y = gather_qmm(act, d.weight, d.scales, d.biases, lhs_indices=pairs, rhs_indices=rhs,
                       group_size=d.group_size, bits=d.bits, mode=d.mode)      # [P, 1, H]
        return y.reshape(*lead, k, y.shape[-1])


class VQSwitchLinear:
    """VQ experts: weight[e, o, i] = scales[e, o, i / scale_group] *
    codebook[codes[e, o, i / dim]][i % dim] (scale_group 0: scales [E, N],
    one per output channel); the call is gather_qmm's.  ``pack_bits`` > 0:
    codes are the artifacts' packed layout, uint32 [E, N, ceil(in/dim/32) *
    pack_bits] of pack_bits-bit fields, with per-group scales
    (``scale_group`` inputs each), as the bundled runtime's class takes them
    (.../heads/deepseek_v4.py:126-129)."""

    def __init__(self, codes, codebook, scales, scale_group: int = 0, pack_bits: int = 0,
                 in_features: int | None = None):
        self.codes, self.codebook, self.scales, self.scale_group = codes, codebook, scales, scale_group
        self.pack_bits = int(pack_bits)
        if self.pack_bits and not scale_group:
            raise ValueError("VQSwitchLinear: packed codes carry per-group scales (scale_group > 0)")
        self.in_features = in_features

    @property
    def group_size(self):
        return self.scale_group

    @property
    def input_dims(self):
        if self.pack_bits:
            return self.in_features or self.scales.shape[2] * self.scale_group
        return self.codes.shape[2] * self.codebook.shape[1]

    @property
    def output_dims(self):
        return self.codes.shape[1]

    @property
    def num_experts(self):
        return self.codes.shape[0]

    def __call__(self, x, indices, sorted_indices: bool = False):
        if self.pack_bits:
            return vq_packed_gather_qmm(x, self.codes, self.codebook, self.scales, self.pack_bits,
                                        self.scale_group, rhs_indices=indices)
        return vq_gather_qmm(x, self.codes, self.codebook, self.scales, rhs_indices=indices,
                             scale_group=self.scale_group)


class VQSwitchGLU:
    """SwitchGLU over VQ experts with the _SwiGLU activation: the gate and up
    projections and the activation in one kernel, then the down projection
    (and the weighted combine)."""

    def __init__(self, gate_proj: VQSwitchLinear, up_proj: VQSwitchLinear, down_proj: VQSwitchLinear):
        self.gate_proj, self.up_proj, self.down_proj = gate_proj, up_proj, down_proj

    def _mats(self):
        return tuple((m.codes, m.codebook, m.scales) for m in (self.gate_proj, self.up_proj, self.down_proj))

    def _packed(self):
        return self.gate_proj.pack_bits or self.up_proj.pack_bits or self.down_proj.pack_bits

    def __call__(self, x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        """x [..., H], indices [..., k] -> [..., k, H]: one library call."""
        if self._packed():
            return self._packed_one_call(x, indices)
        return vq_switch_glu(x, indices, *self._mats(), self.gate_proj.scale_group)

    def combine(self, x, indices, scores):
        """(self(x, indices) * scores[..., None]).sum(-2) with the reference's
        roundings, in the same library call."""
        if self._packed():
            return self._packed_one_call(x, indices, scores)
        return vq_switch_glu(x, indices, *self._mats(), self.gate_proj.scale_group, scores=scores)

    def experts(self, x, logits, k: int):
        """Route (the router of ``moe_route``), SwitchGLU and the weighted
        combine from router logits in one library call.  Returns (out,
        inds, scores)."""
        if self._packed():
            g, u, d = self.gate_proj, self.up_proj, self.down_proj
            if not (g.pack_bits == u.pack_bits == d.pack_bits) or not (g.scale_group == u.scale_group == d.scale_group):
                raise ValueError("VQSwitchGLU: gate, up and down must share the packed layout")
            return vq_packed_experts(x, logits, k, (g.codes, g.codebook, g.scales), (u.codes, u.codebook, u.scales),
                                     (d.codes, d.codebook, d.scales), g.pack_bits, g.scale_group)
        return vq_experts(x, logits, k, *self._mats(), self.gate_proj.scale_group)

    def _packed_one_call(self, x, indices, scores=None):
        g, u, d = self.gate_proj, self.up_proj, self.down_proj
        if not (g.pack_bits == u.pack_bits == d.pack_bits) or not (g.scale_group == u.scale_group == d.scale_group):
            raise ValueError("VQSwitchGLU: gate, up and down must share the packed layout")
        return vq_packed_switch_glu(x, indices, (g.codes, g.codebook, g.scales), (u.codes, u.codebook, u.scales),
                                    (d.codes, d.codebook, d.scales), g.pack_bits, g.scale_group, scores=scores)

    def _packed_call(self, x, indices):
        """The packed SwitchGLU through the separate ops (gate/up + SwiGLU,
        then the down gather)."""
        g, u, d = self.gate_proj, self.up_proj, self.down_proj
        if not (g.pack_bits == u.pack_bits == d.pack_bits) or g.scale_group != u.scale_group:
            raise ValueError("VQSwitchGLU: gate, up and down must share the packed layout")
        act = vq_packed_glu(x, indices, (g.codes, g.codebook, g.scales), (u.codes, u.codebook, u.scales),
                            g.pack_bits, g.scale_group)                          # [..., k, I]
        lead, k = tuple(indices.shape[:-1]), indices.shape[-1]
        P = math.prod(lead) * k
        y = vq_packed_gather_qmm(act.reshape(P, 1, act.shape[-1]), d.codes, d.codebook, d.scales,
                                 d.pack_bits, d.scale_group, rhs_indices=indices.reshape(P),
                                 rows_are_pairs=True)
        return y.reshape(*lead, k, y.shape[-1])

    def separate(self, x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        """The same through the separate ops: vq_glu, then vq_gather_qmm over
        the (token, slot) rows."""
        g, u, d = self.gate_proj, self.up_proj, self.down_proj
        act = vq_glu(x, indices, (g.codes, g.codebook, g.scales), (u.codes, u.codebook, u.scales),
                     g.scale_group)                                           # [..., k, I]
        lead, k = tuple(indices.shape[:-1]), indices.shape[-1]
        P = math.prod(lead) * k
        a2 = act.reshape(P, 1, act.shape[-1])
        y = vq_gather_qmm(a2, d.codes, d.codebook, d.scales,
                          lhs_indices=torch.arange(P, device=x.device, dtype=torch.int32),
                          rhs_indices=indices.reshape(P).to(torch.int32), scale_group=d.scale_group)
        return y.reshape(*lead, k, y.shape[-1])


class MLP:
    """The shared expert (qwen3_5.py:115-118): down(_silu(gate(x)) * up(x))."""

    def __init__(self, gate_proj, up_proj, down_proj):
        self.gate_proj, self.up_proj, self.down_proj = gate_proj, up_proj, down_proj

    def __call__(self, x):
        return self.down_proj(swiglu(self.gate_proj(x), self.up_proj(x)))


class SparseMoeBlock:
    """Qwen3.5-MoE's SparseMoeBlock (qwen3_5.py:151-192): router (softmax in
    float32, top-k, renormalize, round), SwitchGLU experts, the weighted
    combine, plus the sigmoid-gated shared expert when present."""

    def __init__(self, gate, switch_mlp: SwitchGLU, top_k: int, shared_expert: MLP | None = None,
                 shared_expert_gate=None):
        self.gate, self.switch_mlp, self.top_k = gate, switch_mlp, top_k
        self.shared_expert, self.shared_expert_gate = shared_expert, shared_expert_gate
        self.norm_topk_prob = True

    def experts(self, x, logits):
        """The routed part from given router logits: route, experts, combine
        (one library call when the experts take it: the gate/up kernel then
        routes each token itself at decode sizes)."""
        sm = self.switch_mlp
        if (isinstance(sm, SwitchGLU) and sm._one_call(self.top_k) and x.dtype == torch.bfloat16
                and logits.dtype == torch.bfloat16 and logits.shape[-1] <= 1024):
            f, d = sm.fused, sm.down_proj
            out, _, _ = moe_experts(x, logits, self.top_k, f.weight, f.scales, f.biases, d.weight, d.scales,
                                    d.biases, f.group_size, f.bits)
            return out
        inds, scores = moe_route(logits, self.top_k)
        return sm.combine(x, inds, scores)

    def __call__(self, x):
        y = self.experts(x, self.gate(x))
        if self.shared_expert is not None:
            y = moe_shared_add(y, self.shared_expert_gate(x), self.shared_expert(x))
        return y
