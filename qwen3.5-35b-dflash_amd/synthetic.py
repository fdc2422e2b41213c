"""Seeded synthetic workloads for the W4A16 qlinear and the routed-MoE layer.

Distributions: activations ``N(0,1)`` cast to bf16; int4 values uniform in
[-8, 7]; group scales ``U(0.005, 0.02)`` cast to the scale dtype; router
weight ``N(0, 0.02)`` bf16.  Random numbers come from a CPU
``torch.Generator`` so the same seed gives the same data on any machine; the
tensors are then moved to the requested device.
"""
from __future__ import annotations

from typing import NamedTuple, Optional

import torch

from .packing import PackedW4, SharedExpert


def int4_weight(gen: torch.Generator, shape: tuple, group_size: int = 128,
                scale_dtype: torch.dtype = torch.bfloat16, device="cpu") -> PackedW4:
    """Random packed matrix/bank ``[*shape[:-1], K/2]`` with scales ``U(0.005, 0.02)``.

    A uniform random byte holds two independent nibbles, each uniform over the
    16 int4 values [-8, 7], so bytes are drawn directly in packed form.
    """
    packed = torch.randint(0, 256, (*shape[:-1], shape[-1] // 2), dtype=torch.uint8, generator=gen)
    scales = (torch.rand((*shape[:-1], shape[-1] // group_size), generator=gen) * 0.015 + 0.005).to(scale_dtype)
    return PackedW4(packed.to(device), scales.contiguous().to(device), group_size)


def device_bank(gen: torch.Generator, shape: tuple, device, group_size: int = 128) -> PackedW4:
    """Random packed bank generated on the device by ``gen`` (a device generator): uniform bytes
    (two uniform int4 values each), bf16 scales ``U(0.005, 0.02)``; for benchmark-sized banks."""
    packed = torch.randint(0, 256, (*shape[:-1], shape[-1] // 2), dtype=torch.uint8, device=device, generator=gen)
    scales = torch.rand((*shape[:-1], shape[-1] // group_size), device=device, generator=gen) * 0.015 + 0.005
    return PackedW4(packed, scales.to(torch.bfloat16).contiguous(), group_size)


class MoeLayer(NamedTuple):
    hidden: torch.Tensor          # bf16 [T, H]
    router_weight: torch.Tensor   # bf16 [E, H]
    gate_up: PackedW4             # [E, 2I, H]
    down: PackedW4                # [E, H, I]
    shared: Optional[SharedExpert]
    logit_bias: Optional[torch.Tensor]  # fp32 [E] added to the router logits (skewed routing), or None


def moe_layer(tokens: int, *, hidden: int = 2048, inter: int = 512, experts: int = 256, group_size: int = 128,
              seed: int = 0, shared: bool = True, scale_dtype: torch.dtype = torch.bfloat16,
              device="cpu", banks: bool = True) -> MoeLayer:
    """Hidden states, router and (unless ``banks=False``) packed expert banks of one MoE layer."""
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn((tokens, hidden), generator=gen).to(torch.bfloat16)
    router = (torch.randn((experts, hidden), generator=gen) * 0.02).to(torch.bfloat16)
    if not banks:
        return MoeLayer(x.to(device), router.to(device), None, None, None, None)
    gate_up = int4_weight(gen, (experts, 2 * inter, hidden), group_size, scale_dtype, device)
    down = int4_weight(gen, (experts, hidden, inter), group_size, scale_dtype, device)
    sh = None
    if shared:
        sgu = int4_weight(gen, (2 * inter, hidden), group_size, scale_dtype, device)
        sdn = int4_weight(gen, (hidden, inter), group_size, scale_dtype, device)
        gate_w = (torch.randn((hidden,), generator=gen) * 0.02).to(torch.bfloat16)
        sh = SharedExpert(sgu, sdn, gate_w.to(device))
    return MoeLayer(x.to(device), router.to(device), gate_up, down, sh, None)


def hot_expert_bias(logits: torch.Tensor, hot: torch.Tensor, top_k: int, target: float = 0.5) -> float:
    """Bias b (added to the hot experts' logits) giving the hot set ~``target`` of all assignments.

    Bisection on the given fp32 logits ``[T, E]``; ties resolved as in routing.
    """
    lo, hi = 0.0, 16.0
    for _ in range(40):
        b = 0.5 * (lo + hi)
        biased = logits.clone()
        biased[:, hot] += b
        ids = torch.topk(biased, top_k, dim=-1).indices
        frac = torch.isin(ids, hot).float().mean().item()
        if frac < target:
            lo = b
        else:
            hi = b
    return 0.5 * (lo + hi)


def skewed_bias(layer: MoeLayer, *, hot_count: int = 16, top_k: int = 8, target: float = 0.5,
                seed: int = 0) -> torch.Tensor:
    """fp32 ``[E]`` logit bias putting ~``target`` of the assignments on ``hot_count`` fixed experts."""
    experts = layer.router_weight.shape[0]
    gen = torch.Generator().manual_seed(seed + 7919)
    hot = torch.randperm(experts, generator=gen)[:hot_count]
    logits = layer.hidden.float().cpu() @ layer.router_weight.float().cpu().T
    b = hot_expert_bias(logits, hot, top_k, target)
    bias = torch.zeros(experts)
    bias[hot] = b
    return bias
