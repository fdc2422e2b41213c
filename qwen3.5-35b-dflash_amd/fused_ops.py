"""FusedOps ABI-v1 adapter module for MI355X (gfx950).

Drop-in for the reference's operator seam: a module with ``FUSED_OPS_ABI = 1``,
a ``BACKEND_ID`` and the seven callables that
``model/qwen35_moe_dflash/fused/ops.py:126-176`` (``ModuleFusedOps``) binds.
``moe`` and ``qlinear`` run on the hand-written HIP kernels of
``libdflash_hip.so``; the six non-hot operations are plain PyTorch
restatements of ``reference/fused_ops.py:28-145`` that run on whatever device
their inputs are on.

Physical format (the explicit adapter contract that
``fused/ops.py:117-122`` asks packed weights to have): ``gate_up`` and
``down`` are :class:`PackedW4` banks in the portable K-packed int4 layout with
group scales (``graph/quant_weights.py:147-148``).  Dense logical float banks
are not a physical format of this backend and are rejected; nothing is
quantised or dequantised implicitly.
"""
from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn.functional as F
from torch import Tensor

from . import ops
from .packing import PackedW4, SharedExpert

FUSED_OPS_ABI = 1
BACKEND_ID = "mi355x-hip"
IS_REFERENCE_BACKEND = False


# ------------------------------------------------------------------ non-hot ops
def rms_norm(x: Tensor, gamma: Tensor, eps: float) -> Tensor:
    """``x * rsqrt(mean(x^2) + eps)`` in fp32, cast back, times the given (effective) gamma."""
    if not math.isfinite(eps) or eps <= 0 or tuple(gamma.shape) != tuple(x.shape[-1:]):
        raise ValueError("RMSNorm needs positive epsilon and one gamma per feature")
    xf = x.float()
    scale = torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    return (xf * scale).to(x.dtype) * gamma


def conv_state_update(projected: Tensor, history: Tensor) -> tuple[Tensor, Tensor]:
    """``[B,S,C]`` + history ``[B,C,K-1]`` -> (new history ``[B,C,K-1]``, padded ``[B,C,S+K-1]``)."""
    if (projected.ndim != 3 or history.ndim != 3 or projected.shape[1] < 1
            or projected.shape[0] != history.shape[0] or projected.shape[2] != history.shape[1]
            or projected.dtype != history.dtype):
        raise ValueError("conv state requires projected [B,S,C] and matching history [B,C,K-1]")
    padded = torch.cat([history, projected.permute(0, 2, 1)], dim=2)
    keep = history.shape[2]
    new_history = padded[:, :, padded.shape[2] - keep:].clone() if keep else padded[:, :, :0].clone()
    return new_history, padded


def causal_conv1d(padded: Tensor, weight: Tensor) -> Tensor:
    """Depthwise causal conv ``[B,C,S+K-1]`` x ``[C,1,K]`` -> ``[B,S,C]`` (no activation)."""
    if (padded.ndim != 3 or weight.ndim != 3 or weight.shape[1] != 1
            or padded.shape[1] != weight.shape[0] or weight.shape[2] < 1
            or padded.shape[2] < weight.shape[2] or padded.dtype != weight.dtype):
        raise ValueError("depthwise conv requires [B,C,S+K-1] and [C,1,K]")
    out = F.conv1d(padded, weight, groups=weight.shape[0])
    return out.permute(0, 2, 1).contiguous()


def chunk_gated_delta_rule(query: Tensor, key: Tensor, value: Tensor, g: Tensor, beta: Tensor,
                           initial_state: Tensor, effective_length: Tensor, *, chunk_size: int,
                           use_qk_l2norm_in_kernel: bool) -> tuple[Tensor, Tensor]:
    """Gated delta rule, token by token; only the first ``effective_length`` tokens update state."""
    if isinstance(chunk_size, bool) or chunk_size not in (1, 64):
        raise ValueError("chunk_size must be 1 or 64")
    if not isinstance(use_qk_l2norm_in_kernel, bool):
        raise ValueError("use_qk_l2norm_in_kernel must be bool")
    if (query.ndim != 4 or key.shape != query.shape or value.ndim != 4
            or value.shape[:3] != query.shape[:3] or g.shape != query.shape[:3]
            or beta.shape != query.shape[:3] or min(query.shape) < 1 or value.shape[-1] < 1):
        raise ValueError("GDN requires compatible [B,S,H,D] tensors and [B,S,H] gates")
    b, s, h, dk = query.shape
    dv = value.shape[-1]
    if tuple(initial_state.shape) != (b, h, dk, dv) or initial_state.dtype not in (torch.float16, torch.float32):
        raise ValueError("initial_state must be FP16/FP32 [B,H,Dk,Dv]")
    if (effective_length.dtype != torch.int16 or tuple(effective_length.shape) != (b,)
            or bool(((effective_length < 0) | (effective_length > s)).any())):
        raise ValueError("effective_length must be INT16 [B] within [0,S]")
    if query.dtype not in (torch.float16, torch.float32) or any(t.dtype != query.dtype for t in (key, value, g, beta)):
        raise ValueError("GDN floating inputs must share FP16 or FP32 dtype")
    q, k, v, decay, gate = (t.float() for t in (query, key, value, g, beta))
    if use_qk_l2norm_in_kernel:
        q = q / torch.sqrt(q.pow(2).sum(-1, keepdim=True) + 1e-6)
        k = k / torch.sqrt(k.pow(2).sum(-1, keepdim=True) + 1e-6)
    q = q * (dk ** -0.5)
    state = initial_state.float().clone()
    length = effective_length.to(torch.int64)
    outs = []
    for i in range(s):
        active = (i < length)[:, None, None, None]
        st = state * torch.exp(decay[:, i])[:, :, None, None]
        ki = k[:, i]
        pred = (st * ki[:, :, :, None]).sum(dim=2)
        delta = (v[:, i] - pred) * gate[:, i][:, :, None]
        st = st + ki[:, :, :, None] * delta[:, :, None, :]
        state = torch.where(active, st, state)
        o = (state * q[:, i][:, :, :, None]).sum(dim=2)
        outs.append(torch.where(active[..., 0], o, torch.zeros_like(o)))
    return torch.stack(outs, dim=1).to(query.dtype), state.to(initial_state.dtype)


def cache_update(key: Optional[Tensor], value: Optional[Tensor], new_key: Tensor,
                 new_value: Tensor) -> tuple[Tensor, Tensor]:
    """Append ``[B,Hkv,S,D]`` keys/values; returns new, privately owned caches."""
    if ((key is None) != (value is None) or new_key.ndim != 4 or new_value.ndim != 4
            or new_key.shape[:3] != new_value.shape[:3]):
        raise ValueError("KV caches must appear together and use [B,H,T,D]")
    if key is None:
        return new_key.clone(), new_value.clone()
    for old, new in ((key, new_key), (value, new_value)):
        if old.ndim != 4 or old.shape[:2] != new.shape[:2] or old.shape[-1] != new.shape[-1] or old.dtype != new.dtype:
            raise ValueError("old and new KV cache dimensions/dtypes do not match")
    if key.shape[2] != value.shape[2]:
        raise ValueError("old key and value cache lengths differ")
    return torch.cat([key, new_key], dim=2), torch.cat([value, new_value], dim=2)


def attention(query: Tensor, key: Tensor, value: Tensor, *, query_start: int, scale: float) -> Tensor:
    """Causal GQA; query row i sees key positions ``<= query_start + i``.  fp32 math."""
    if (query.ndim != 4 or key.ndim != 4 or value.ndim != 4 or query.shape[0] != key.shape[0]
            or key.shape[:3] != value.shape[:3] or query.shape[-1] != key.shape[-1] or key.shape[1] < 1
            or query.shape[1] % key.shape[1] or isinstance(query_start, bool) or not isinstance(query_start, int)
            or query_start < 0 or query_start + query.shape[2] != key.shape[2]
            or not math.isfinite(scale) or scale <= 0):
        raise ValueError("attention requires causal append-only GQA [B,H,S,D] inputs")
    rep = query.shape[1] // key.shape[1]
    kf = key.float().repeat_interleave(rep, dim=1)
    vf = value.float().repeat_interleave(rep, dim=1)
    scores = torch.matmul(query.float(), kf.transpose(-1, -2).contiguous()) * scale
    qpos = torch.arange(query.shape[2], device=query.device) + query_start
    kpos = torch.arange(key.shape[2], device=query.device)
    scores = scores.masked_fill((kpos[None, :] > qpos[:, None])[None, None], float("-inf"))
    return torch.matmul(torch.softmax(scores, dim=-1), vf).to(query.dtype)


# ------------------------------------------------------------------ hot path (HIP)
def _bank(value, name: str) -> PackedW4:
    if isinstance(value, PackedW4):
        return value
    if isinstance(value, tuple) and len(value) == 3:
        return PackedW4(*value)
    raise ValueError(f"{BACKEND_ID} moe needs packed int4 {name} (PackedW4); dense logical banks are not "
                     "a physical format of this backend")


def moe(hidden: Tensor, router_weight: Optional[Tensor], gate_up, down, *, top_k: int,
        router_logits: Optional[Tensor] = None, shared: Optional[SharedExpert] = None) -> Tensor:
    """Routed experts on packed banks (reference signature, ``fused/ops.py:108-123``).

    ``hidden`` bf16 ``[B,S,H]``; ``router_weight`` bf16 ``[E,H]`` (or fp32
    ``router_logits [B*S,E]`` given instead); ``gate_up`` packed ``[E,2I,H]``,
    ``down`` packed ``[E,H,I]``; ``top_k`` in ``(0, E]``.  Selection ranks the
    fp32 logits (lowest id on ties), weights are the renormalised softmax of
    the selected logits, experts accumulate in fp32 and the result is rounded
    to bf16 once.  Routed experts only unless ``shared`` is given, in which
    case the gated shared expert (``fused/model.py:305-307``) is added in the
    same fp32 sum.  Returns a new tensor shaped like ``hidden``.
    """
    gate_up, down = _bank(gate_up, "gate_up"), _bank(down, "down")
    if (not isinstance(hidden, Tensor) or hidden.ndim != 3 or gate_up.packed.ndim != 3 or down.packed.ndim != 3
            or gate_up.rows % 2 or down.experts != gate_up.experts or gate_up.cols != hidden.shape[-1]
            or (down.rows, down.cols) != (hidden.shape[-1], gate_up.rows // 2)
            or isinstance(top_k, bool) or not isinstance(top_k, int) or not 0 < top_k <= gate_up.experts):
        raise ValueError("MoE needs compatible expert weights and a valid top_k")
    if router_logits is None:
        if (not isinstance(router_weight, Tensor) or router_weight.ndim != 2
                or tuple(router_weight.shape) != (gate_up.experts, hidden.shape[-1])):
            raise ValueError("MoE needs router_weight [E, H]")
    out = ops.moe_w4a16(hidden, gate_up, down, top_k=top_k, router_weight=router_weight,
                        router_logits=router_logits, shared=shared)
    return out.reshape(hidden.shape)


def qlinear(x: Tensor, packed: Tensor, scales: Tensor, *, group_size: int) -> Tensor:
    """W4A16 linear ``[..., K] -> [..., N]`` over a packed ``[N, K/2]`` matrix and ``[N, K/G]`` scales."""
    return ops.qlinear(x, PackedW4(packed, scales, group_size))
