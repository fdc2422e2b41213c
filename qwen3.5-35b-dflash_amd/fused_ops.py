"""FusedOps ABI-v1 adapter module for MI355X (gfx950).

Drop-in for the reference's operator seam: a module with ``FUSED_OPS_ABI = 1``,
a ``BACKEND_ID`` and the seven callables that
``model/qwen35_moe_dflash/fused/ops.py:126-176`` (``ModuleFusedOps``) binds.
``moe`` and ``qlinear`` run on the hand-written HIP kernels of
``libdflash_hip.so``; the six non-hot operations are batched PyTorch code of
this backend's own that runs on whatever device its inputs are on (the
protocol they satisfy is ``fused/ops.py:25-123``).

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
from torch import Tensor

from . import layers, ops
from .packing import PackedW4, SharedExpert

FUSED_OPS_ABI = 1
BACKEND_ID = "mi355x-hip"
IS_REFERENCE_BACKEND = False


# ------------------------------------------------------------------ non-hot ops
# The contract of each op (signature, shapes, dtypes and the ValueError messages a caller
# may match on) is the FusedOps protocol of ``fused/ops.py:25-123``; the bodies are this
# backend's own: batched tensor algebra that runs on the inputs' device in a handful of
# launches (no per-token Python loop, no materialised GQA repeat of the KV cache).

def _require(ok: bool, message: str) -> None:
    if not ok:
        raise ValueError(message)


def _is_int(v) -> bool:
    return isinstance(v, int) and not isinstance(v, bool)


def rms_norm(x: Tensor, gamma: Tensor, eps: float) -> Tensor:
    """``x / rms(x)`` computed in fp32 and rounded to ``x.dtype``, then times the effective gamma.

    The gamma given is the effective one (the caller adds any +1 offset).
    """
    _require(tuple(gamma.shape) == tuple(x.shape[-1:]) and math.isfinite(eps) and eps > 0,
             "RMSNorm needs positive epsilon and one gamma per feature")
    xf = x.float()
    mean_square = torch.linalg.vector_norm(xf, dim=-1, keepdim=True).square_().div_(x.shape[-1])
    return (xf * mean_square.add_(eps).rsqrt_()).to(x.dtype) * gamma


def conv_state_update(projected: Tensor, history: Tensor) -> tuple[Tensor, Tensor]:
    """``[B,S,C]`` + history ``[B,C,K-1]`` -> (new history ``[B,C,K-1]``, window ``[B,C,K-1+S]``).

    The window is the history followed by the new columns; the new history is its
    last ``K-1`` columns, returned as a tensor of its own.
    """
    _require(projected.ndim == 3 and history.ndim == 3 and projected.shape[1] >= 1
             and (projected.shape[0], projected.shape[2]) == tuple(history.shape[:2])
             and projected.dtype == history.dtype,
             "conv state requires projected [B,S,C] and matching history [B,C,K-1]")
    keep = history.shape[2]
    window = projected.new_empty((projected.shape[0], projected.shape[2], keep + projected.shape[1]))
    window[:, :, :keep] = history
    window[:, :, keep:] = projected.transpose(1, 2)
    return window[:, :, window.shape[2] - keep:].clone(), window


def causal_conv1d(padded: Tensor, weight: Tensor) -> Tensor:
    """Depthwise causal conv ``[B,C,K-1+S]`` with taps ``[C,1,K]`` -> ``[B,S,C]`` (no activation).

    Output column ``s`` of channel ``c`` is ``sum_j weight[c,0,j] * padded[c, s+j]``: the
    ``K`` taps are read as one strided window view and reduced in a single pass.
    """
    _require(padded.ndim == 3 and weight.ndim == 3 and weight.shape[1] == 1 and weight.shape[2] >= 1
             and padded.shape[1] == weight.shape[0] and padded.shape[2] >= weight.shape[2]
             and padded.dtype == weight.dtype,
             "depthwise conv requires [B,C,S+K-1] and [C,1,K]")
    taps = weight.shape[2]
    windows = padded.unfold(2, taps, 1)                      # [B, C, S, K] view, no copy
    out = (windows.float() * weight[:, 0, None, :].float()).sum(-1)
    return out.to(padded.dtype).transpose(1, 2).contiguous()


def chunk_gated_delta_rule(query: Tensor, key: Tensor, value: Tensor, g: Tensor, beta: Tensor,
                           initial_state: Tensor, effective_length: Tensor, *, chunk_size: int,
                           use_qk_l2norm_in_kernel: bool) -> tuple[Tensor, Tensor]:
    """Gated delta rule over ``[B,S,H,D]`` tokens; returns core ``[B,S,H,Dv]`` and the final state.

    Tokens at or past ``effective_length[b]`` leave the state unchanged and output zeros
    (they enter the chunk with ``g = 0`` and ``beta = 0``).  Math in fp32, in closed-form
    chunks of 16 tokens (``layers.delta_rule``; ``chunk_size`` is the caller's decode/prefill
    tag, 1 or 64, and does not change the result).  Q/K are L2-normalised here when asked to be
    (``q / sqrt(|q|^2 + 1e-6)``); q is scaled by ``Dk^-1/2``.
    """
    _require(_is_int(chunk_size) and chunk_size in (1, 64), "chunk_size must be 1 or 64")
    _require(isinstance(use_qk_l2norm_in_kernel, bool), "use_qk_l2norm_in_kernel must be bool")
    gates_shape = tuple(query.shape[:3])
    _require(query.ndim == 4 and key.shape == query.shape and value.ndim == 4
             and tuple(value.shape[:3]) == gates_shape and tuple(g.shape) == gates_shape
             and tuple(beta.shape) == gates_shape and min(query.shape) >= 1 and value.shape[-1] >= 1,
             "GDN requires compatible [B,S,H,D] tensors and [B,S,H] gates")
    b, s, h, dk = query.shape
    dv = value.shape[-1]
    _require(tuple(initial_state.shape) == (b, h, dk, dv) and initial_state.dtype in (torch.float16, torch.float32),
             "initial_state must be FP16/FP32 [B,H,Dk,Dv]")
    _require(effective_length.dtype == torch.int16 and tuple(effective_length.shape) == (b,)
             and bool(((effective_length >= 0) & (effective_length <= s)).all()),
             "effective_length must be INT16 [B] within [0,S]")
    _require(query.dtype in (torch.float16, torch.float32)
             and all(t.dtype == query.dtype for t in (key, value, g, beta)),
             "GDN floating inputs must share FP16 or FP32 dtype")
    # head-major fp32 [B, H, S, .]; layers.delta_rule normalises, scales q and chunks
    q, k, v, gf, bf = (t.float().transpose(1, 2) for t in (query, key, value, g, beta))
    valid = (torch.arange(s, device=query.device)[None, :] < effective_length.to(torch.int64)[:, None])[:, None, :]
    core, state, _ = layers.delta_rule(q, k, v, gf, bf, initial_state.float(), normalise=use_qk_l2norm_in_kernel,
                                       valid=valid)
    return core.transpose(1, 2).to(query.dtype).contiguous(), state.to(initial_state.dtype)


def cache_update(key: Optional[Tensor], value: Optional[Tensor], new_key: Tensor,
                 new_value: Tensor) -> tuple[Tensor, Tensor]:
    """Append ``[B,Hkv,S,D]`` keys/values along the sequence axis; new, privately owned caches."""
    _require((key is None) == (value is None) and new_key.ndim == 4 and new_value.ndim == 4
             and new_key.shape[:3] == new_value.shape[:3],
             "KV caches must appear together and use [B,H,T,D]")
    if key is None:
        return new_key.clone(), new_value.clone()
    _require(all(old.ndim == 4 and old.shape[:2] == new.shape[:2] and old.shape[3] == new.shape[3]
                 and old.dtype == new.dtype for old, new in ((key, new_key), (value, new_value))),
             "old and new KV cache dimensions/dtypes do not match")
    _require(key.shape[2] == value.shape[2], "old key and value cache lengths differ")
    return torch.cat((key, new_key), dim=2), torch.cat((value, new_value), dim=2)


def attention(query: Tensor, key: Tensor, value: Tensor, *, query_start: int, scale: float) -> Tensor:
    """Causal grouped-query attention in fp32: query row ``i`` sees key positions ``<= query_start + i``.

    The ``H / Hkv`` query heads that share a KV head are stacked into one block of rows and
    multiplied against that head's keys once, so the cache is never repeated per query head.
    """
    _require(query.ndim == 4 and key.ndim == 4 and value.ndim == 4 and query.shape[0] == key.shape[0]
             and key.shape[:3] == value.shape[:3] and query.shape[3] == key.shape[3] and key.shape[1] >= 1
             and query.shape[1] % key.shape[1] == 0 and _is_int(query_start) and query_start >= 0
             and query_start + query.shape[2] == key.shape[2] and math.isfinite(scale) and scale > 0,
             "attention requires causal append-only GQA [B,H,S,D] inputs")
    return layers.grouped_attention(query, key, value, query_start, scale).to(query.dtype)


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
