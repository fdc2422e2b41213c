"""Tensor inventory of the Qwen3.5-MoE target: names, shapes and which ones are int4.

Restates the reference's canonical target inventory
(``model/qwen35_moe_dflash/target/weight_shapes.py:7-45``) and its per-tensor
quantization descriptor (``graph/quant_plan.py:25-101``): which tensors are
packed int4 linears or expert banks, which stay floating point, and the byte
layout of each packed tensor.  The group size is a parameter here (the
reference fixes 256; the W4A16 configs use 128, ``reference/quantization.py:87-89``).

``int4_keys`` lists what the qlinear / MoE kernels consume; the stack and the
quantized-weights adapter load exactly that set.
"""
from __future__ import annotations

import math
import re
from dataclasses import dataclass, field
from typing import Mapping

# packed int4 linears (graph/quant_plan.py:25-32) and expert banks
LINEAR_SUFFIXES = frozenset({
    "linear_attn.in_proj_qkv.weight", "linear_attn.in_proj_z.weight",
    "linear_attn.in_proj_a.weight", "linear_attn.in_proj_b.weight",
    "linear_attn.out_proj.weight", "self_attn.q_proj.weight",
    "self_attn.k_proj.weight", "self_attn.v_proj.weight", "self_attn.o_proj.weight",
    "mlp.gate.weight", "mlp.shared_expert.gate_proj.weight",
    "mlp.shared_expert.up_proj.weight", "mlp.shared_expert.down_proj.weight",
})
EXPERT_SUFFIXES = frozenset({"mlp.experts.gate_up_proj", "mlp.experts.down_proj"})
# floating tensors (graph/quant_plan.py:33-38)
FLOAT_SUFFIXES = frozenset({
    "input_layernorm.weight", "post_attention_layernorm.weight",
    "self_attn.q_norm.weight", "self_attn.k_norm.weight",
    "linear_attn.conv1d.weight", "linear_attn.dt_bias", "linear_attn.A_log",
    "linear_attn.norm.weight", "mlp.shared_expert_gate.weight",
})
# Tensors this build keeps floating although the inventory lists them as int4 linears: the
# router, whose fp32 logits decide the routing bit-exactly, stays bf16 (its logits are a
# kernel of the MoE layer, not a qlinear).  The DOPT W4A16 plan also keeps the vocabulary
# projection and the GDN a/b predictors floating (reference/quantization.py:95-96); pass
# them to int4_keys to follow that plan instead.
ROUTER_SUFFIX = "mlp.gate.weight"
DOPT_W4A16_FLOAT = frozenset({"target.lm_head.weight", "linear_attn.in_proj_a.weight",
                              "linear_attn.in_proj_b.weight", ROUTER_SUFFIX})


@dataclass(frozen=True)
class TargetConfig:
    """The text-model geometry the stack needs (``specs/target-config.json:7-90``)."""

    hidden: int = 2048
    layer_types: tuple = field(default_factory=lambda: tuple(
        "full_attention" if (i + 1) % 4 == 0 else "linear_attention" for i in range(40)))
    vocab: int = 248320
    heads: int = 16
    kv_heads: int = 2
    head_dim: int = 256
    linear_key_heads: int = 16
    linear_value_heads: int = 32
    linear_key_dim: int = 128
    linear_value_dim: int = 128
    conv_kernel: int = 4
    experts: int = 256
    top_k: int = 8
    moe_inter: int = 512
    shared_inter: int = 512
    rms_eps: float = 1e-6
    rope_theta: float = 10_000_000.0
    partial_rotary: float = 0.25

    @property
    def layers(self) -> int:
        return len(self.layer_types)

    @property
    def rotary_dim(self) -> int:
        return int(self.head_dim * self.partial_rotary)

    @property
    def conv_channels(self) -> int:
        return 2 * self.linear_key_heads * self.linear_key_dim + self.linear_value_heads * self.linear_value_dim

    def validate(self) -> None:
        if set(self.layer_types) - {"linear_attention", "full_attention"} or not self.layer_types:
            raise ValueError("layer_types must declare every full/linear attention layer")
        if self.heads % self.kv_heads or self.linear_value_heads % self.linear_key_heads:
            raise ValueError("query/value head counts must be multiples of KV/key heads")
        if not 0 < self.top_k <= self.experts:
            raise ValueError("top-k exceeds expert count")
        if self.rotary_dim < 2 or self.rotary_dim % 2:
            raise ValueError("RoPE requires positive even rotary width")


def target_shapes(c: TargetConfig) -> dict[str, tuple[int, ...]]:
    """Canonical ``target.*`` tensor names and shapes (``target/weight_shapes.py:7-45``)."""
    h, d = c.hidden, c.head_dim
    shapes = {"target.embed_tokens.weight": (c.vocab, h), "target.norm.weight": (h,),
              "target.lm_head.weight": (c.vocab, h)}
    kw, vw = c.linear_key_heads * c.linear_key_dim, c.linear_value_heads * c.linear_value_dim
    for i, kind in enumerate(c.layer_types):
        p = f"target.layers.{i}"
        shapes[p + ".input_layernorm.weight"] = (h,)
        shapes[p + ".post_attention_layernorm.weight"] = (h,)
        if kind == "linear_attention":
            q = p + ".linear_attn"
            shapes.update({q + ".in_proj_qkv.weight": (2 * kw + vw, h), q + ".in_proj_z.weight": (vw, h),
                           q + ".in_proj_b.weight": (c.linear_value_heads, h),
                           q + ".in_proj_a.weight": (c.linear_value_heads, h),
                           q + ".A_log": (c.linear_value_heads,), q + ".dt_bias": (c.linear_value_heads,),
                           q + ".conv1d.weight": (2 * kw + vw, 1, c.conv_kernel),
                           q + ".norm.weight": (c.linear_value_dim,), q + ".out_proj.weight": (h, vw)})
        else:
            q = p + ".self_attn"
            shapes.update({q + ".q_proj.weight": (c.heads * d * 2, h), q + ".k_proj.weight": (c.kv_heads * d, h),
                           q + ".v_proj.weight": (c.kv_heads * d, h), q + ".o_proj.weight": (h, c.heads * d),
                           q + ".q_norm.weight": (d,), q + ".k_norm.weight": (d,)})
        q = p + ".mlp"
        shapes.update({q + ".gate.weight": (c.experts, h),
                       q + ".experts.gate_up_proj": (c.experts, 2 * c.moe_inter, h),
                       q + ".experts.down_proj": (c.experts, h, c.moe_inter),
                       q + ".shared_expert.gate_proj.weight": (c.shared_inter, h),
                       q + ".shared_expert.up_proj.weight": (c.shared_inter, h),
                       q + ".shared_expert.down_proj.weight": (h, c.shared_inter),
                       q + ".shared_expert_gate.weight": (1, h)})
    return shapes


def tensor_kind(key: str, shape) -> str:
    """``linear_int4`` | ``expert_int4`` | ``embedding_int8`` | ``float`` (``graph/quant_plan.py:41-59``).

    Unknown names raise rather than falling into a default policy.
    """
    shape = tuple(shape)
    if not shape or any(type(n) is not int or n <= 0 for n in shape):
        raise ValueError(f"{key}: shape must contain positive integers")
    m = re.fullmatch(r"target\.layers\.([0-9]+)\.(.+)", key)
    suffix = m.group(2) if m else None
    if key == "target.embed_tokens.weight":
        return "embedding_int8"
    if key == "target.lm_head.weight" or suffix in LINEAR_SUFFIXES:
        return "linear_int4"
    if suffix in EXPERT_SUFFIXES:
        return "expert_int4"
    if key == "target.norm.weight" or suffix in FLOAT_SUFFIXES:
        return "float"
    raise ValueError(f"unrecognized target weight: {key}")


def describe(key: str, shape, group_size: int = 128) -> dict:
    """Byte layout of one tensor in the portable format (``graph/quant_plan.py:60-101``)."""
    shape = tuple(shape)
    kind = tensor_kind(key, shape)
    params = math.prod(shape)
    rec = {"key": key, "shape": list(shape), "kind": kind, "parameters": params, "group_size": None,
           "weight_shape": list(shape), "weight_dtype": "bfloat16", "weight_bytes": params * 2,
           "scale_shape": None, "scale_bytes": 0, "weight_transform": "CAST_ONLY_NO_OFFSET"}
    if kind in ("linear_int4", "expert_int4"):
        rank = 3 if kind == "expert_int4" else 2
        if len(shape) != rank or shape[-1] % group_size or group_size not in (128, 256):
            raise ValueError(f"{key}: INT4 requires rank {rank} and K divisible by {group_size}")
        scale_shape = [*shape[:-1], shape[-1] // group_size]
        rec.update(group_size=group_size, weight_shape=[*shape[:-1], shape[-1] // 2], weight_dtype="uint8",
                   weight_bytes=params // 2, scale_shape=scale_shape, scale_bytes=math.prod(scale_shape) * 2,
                   weight_transform="PORTABLE_SIGNED_INT4_K_LOW_NIBBLE_FIRST")
    elif kind == "embedding_int8":
        if len(shape) != 2:
            raise ValueError(f"{key}: embedding requires rank two")
        rec.update(weight_dtype="int8", weight_bytes=params, scale_shape=[shape[0], 1], scale_bytes=shape[0] * 4,
                   weight_transform="SYMMETRIC_INT8_PER_ROW")
    if key == "target.norm.weight" or (suffix_of(key) or "").endswith("norm.weight"):
        # main / q / k norms apply (1 + w); the gated GDN norm applies w (fused/model.py:206-225)
        rec["norm_weight_addend"] = 0 if suffix_of(key) == "linear_attn.norm.weight" else 1
    return rec


def suffix_of(key: str):
    m = re.fullmatch(r"target\.layers\.([0-9]+)\.(.+)", key)
    return m.group(2) if m else None


def int4_keys(shapes: Mapping[str, tuple], *, keep_float=frozenset({ROUTER_SUFFIX})) -> list[str]:
    """The tensors a kernel consumes packed: every int4 linear and expert bank of the inventory
    except those named in ``keep_float`` (full keys or per-layer suffixes)."""
    keys = []
    for key, shape in shapes.items():
        if tensor_kind(key, shape) not in ("linear_int4", "expert_int4"):
            continue
        if key in keep_float or suffix_of(key) in keep_float:
            continue
        keys.append(key)
    return keys
