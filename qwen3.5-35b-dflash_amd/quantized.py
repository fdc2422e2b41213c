"""The quantized-weights seam of the reference's stateful target, on this library's kernels.

``FusedTargetModel`` (``model/qwen35_moe_dflash/fused/model.py:96-125,197-204,296-307``)
takes a ``quantization`` object and calls exactly these members on it:

* ``device``, ``validate_shapes(shapes)``, ``has_weight(key)`` at construction;
* ``embedding(token_ids)`` -- fp32 rows (``fused/quantization.py:138-141``);
* ``linear(x, key)`` for every packed projection (``:154-165``);
* ``moe(x, prefix, top_k=)`` for the routed experts (``:181-202``); the model adds
  the shared expert itself through ``linear`` and its float ``shared_expert_gate``.

:class:`QuantizedWeights` implements that interface over :class:`PackedW4`
banks: ``linear`` is one ``dflash_qlinear_w4a16`` launch, ``moe`` one
``dflash_moe_w4a16`` sequence.  Like the vendor path it returns float16
(``fused/model.py`` checks fp16 projection and MoE outputs); activations enter
the kernels as bf16 (W4A16).  Errors are the reference adapter's
``ValueError`` messages.

The reference model also checks ``isinstance(quantization,
OriginalQuantizedWeights)`` (``fused/model.py:111-114``).  :func:`bind` takes
that class (the caller imports it; this package never imports the reference)
and returns a subclass whose members are this adapter's, so the unmodified
model binds it.
"""
from __future__ import annotations

from typing import Mapping, Optional

import torch
from torch import Tensor

from . import ops, plan
from .packing import PackedW4


class QuantizedWeights(torch.nn.Module):
    """Packed int4 projections, expert banks and the int8 embedding of one target."""

    def __init__(self, shapes: Mapping[str, tuple], banks: Mapping[str, PackedW4], embedding: tuple,
                 *, routers: Optional[Mapping[str, Tensor]] = None, layout: str = "tiled"):
        torch.nn.Module.__init__(self)      # not super(): a bound subclass's base takes other arguments
        self.shapes = {key: tuple(shape) for key, shape in shapes.items()}
        self.kinds = {key: plan.tensor_kind(key, shape) for key, shape in self.shapes.items()}
        weight, scale = embedding
        expected = self.shapes["target.embed_tokens.weight"]
        if (not isinstance(weight, Tensor) or weight.dtype != torch.int8 or tuple(weight.shape) != expected
                or not isinstance(scale, Tensor) or scale.dtype != torch.float32
                or tuple(scale.shape) != (expected[0], 1)):
            raise ValueError("embedding requires original INT8 [vocab,hidden] and FP32 [vocab,1]")
        if not torch.isfinite(scale).all():
            raise ValueError("embedding scale is nonfinite")
        device = weight.device
        self.register_buffer("embedding_weight", weight.detach().clone())
        self.register_buffer("embedding_scale", scale.detach().clone())
        self._banks: dict[str, PackedW4] = {}
        for key, bank in banks.items():
            kind = self.kinds.get(key)
            if kind not in ("linear_int4", "expert_int4"):
                raise ValueError(f"{key} is not an int4 tensor of this target")
            bank.validate(key)
            logical = (*bank.packed.shape[:-1], bank.cols)
            if logical != self.shapes[key] or bank.packed.device != device:
                raise ValueError(f"invalid packed descriptor: {key}")
            if layout == "tiled" and bank.layout != "tiled":
                bank = bank.tiled()
            self._banks[key] = bank
        self._routers: dict[str, Tensor] = {}
        for key, value in (routers or {}).items():
            if (plan.suffix_of(key) != plan.ROUTER_SUFFIX or tuple(value.shape) != self.shapes.get(key)
                    or value.dtype != torch.bfloat16 or value.device != device):
                raise ValueError(f"router {key} must be bfloat16 {self.shapes.get(key)} on {device}")
            self._routers[key] = value.contiguous()
        self.eval()

    @property
    def device(self) -> torch.device:
        return self.embedding_weight.device

    def has_weight(self, key: str) -> bool:
        return key == "target.embed_tokens.weight" or key in self._banks or key in self._routers

    def validate_shapes(self, shapes: Mapping[str, tuple]) -> None:
        if {key: tuple(shape) for key, shape in shapes.items()} != self.shapes:
            raise ValueError("original quant adapter geometry does not match target model")

    def embedding(self, token_ids: Tensor) -> Tensor:
        idx = token_ids.long()
        return self.embedding_weight[idx].float() * self.embedding_scale[idx]

    def linear(self, x: Tensor, key: str) -> Tensor:
        bank = self._banks.get(key)
        if bank is None or self.kinds[key] != "linear_int4" or x.shape[-1] != self.shapes[key][-1]:
            raise ValueError(f"invalid original quant linear invocation: {key}")
        out = ops.qlinear(x.reshape(-1, x.shape[-1]).to(torch.bfloat16), bank)
        return out.to(torch.float16).reshape(*x.shape[:-1], bank.rows)

    def router_logits(self, flat: Tensor, key: str) -> Tensor:
        """fp32 logits ``[T, E]``: the bf16 router's GEMV, or a packed router's qlinear, both the
        unrounded fp32 sums, so the top-k ranks exact logits (no bf16 ties at the k-th place)."""
        if key in self._routers:
            return ops.router_logits(flat, self._routers[key])
        if key in self._banks:
            return ops.qlinear(flat, self._banks[key], out_dtype=torch.float32)
        raise ValueError(f"invalid original quant linear invocation: {key}")

    def moe(self, x: Tensor, prefix: str, *, top_k: int) -> Tensor:
        gate_up, down = self._banks.get(prefix + ".experts.gate_up_proj"), self._banks.get(prefix + ".experts.down_proj")
        if gate_up is None or down is None:
            raise ValueError(f"invalid original quant MoE invocation: {prefix}")
        flat = x.reshape(-1, x.shape[-1]).to(torch.bfloat16)
        key = prefix + ".gate.weight"
        if key in self._routers:
            out = ops.moe_w4a16(flat, gate_up, down, top_k=top_k, router_weight=self._routers[key])
        else:
            out = ops.moe_w4a16(flat, gate_up, down, top_k=top_k, router_logits=self.router_logits(flat, key))
        return out.to(torch.float16).reshape(x.shape)


def bind(base: type) -> type:
    """A subclass of ``base`` (the reference's ``OriginalQuantizedWeights``) with this adapter's members.

    ``isinstance(bind(Base)(...), Base)`` holds, and every member the model calls resolves to
    :class:`QuantizedWeights` (it comes first in the method order); ``base.__init__`` is never
    run, so no vendor binding is required.
    """
    if not isinstance(base, type) or not issubclass(base, torch.nn.Module):
        raise TypeError("bind needs the reference's OriginalQuantizedWeights class (an nn.Module)")
    return type(f"{base.__name__}OnMI355X", (QuantizedWeights, base), {"__module__": __name__})


def from_target_weights(weights, *, layout: str = "tiled") -> QuantizedWeights:
    """The adapter over a :class:`target.TargetWeights` (synthetic or loaded), keyed by the reference's
    tensor names: stacked projections are split back into their per-key matrices."""
    c = weights.config
    shapes = plan.target_shapes(c)
    banks: dict[str, PackedW4] = {"target.lm_head.weight": weights.lm_head}
    routers = {}
    kw, vw = c.linear_key_heads * c.linear_key_dim, c.linear_value_heads * c.linear_value_dim
    for i, lw in enumerate(weights.layers):
        p = f"target.layers.{i}"
        if lw.kind == "linear_attention":
            parts = (("in_proj_qkv", 2 * kw + vw), ("in_proj_z", vw), ("in_proj_b", c.linear_value_heads),
                     ("in_proj_a", c.linear_value_heads))
            banks.update(_split_rows(lw.mixer_in, [(f"{p}.linear_attn.{n}.weight", r) for n, r in parts]))
            banks[f"{p}.linear_attn.out_proj.weight"] = lw.mixer_out
        else:
            d = c.head_dim
            parts = (("q_proj", 2 * c.heads * d), ("k_proj", c.kv_heads * d), ("v_proj", c.kv_heads * d))
            banks.update(_split_rows(lw.mixer_in, [(f"{p}.self_attn.{n}.weight", r) for n, r in parts]))
            banks[f"{p}.self_attn.o_proj.weight"] = lw.mixer_out
        banks[f"{p}.mlp.experts.gate_up_proj"] = lw.gate_up
        banks[f"{p}.mlp.experts.down_proj"] = lw.down
        banks.update(_split_rows(lw.shared.gate_up, [(f"{p}.mlp.shared_expert.gate_proj.weight", c.shared_inter),
                                                     (f"{p}.mlp.shared_expert.up_proj.weight", c.shared_inter)]))
        banks[f"{p}.mlp.shared_expert.down_proj.weight"] = lw.shared.down
        routers[f"{p}.mlp.gate.weight"] = lw.router
    return QuantizedWeights(shapes, banks, (weights.embedding, weights.embedding_scale), routers=routers,
                            layout=layout)


def _split_rows(bank: PackedW4, parts) -> dict:
    """Row blocks of a stacked matrix as separate banks (views; 16-row aligned in the tiled layout)."""
    out, row = {}, 0
    for key, rows in parts:
        if bank.layout == "tiled" and (row % 16 or rows % 16):
            raise ValueError(f"{key}: tiled banks split only at 16-row boundaries ({row}, {rows})")
        out[key] = PackedW4(bank.packed[row:row + rows].contiguous(), bank.scales[row:row + rows].contiguous(),
                            bank.group_size, bank.layout)
        row += rows
    return out
