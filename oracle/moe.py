"""Oracle: routed-MoE expert FFN, weighted combine and the gated shared expert.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Semantics followed:

* router logits ``hidden @ router_weight.T`` kept in float32
  (``reference/fused_ops.py:161``; the logits enter ranking as fp32 so that
  selection is a function of the logits, see ``oracle/routing.py``);
* per hit expert, in ascending expert order: gather the expert's tokens,
  ``gate, up = (x @ gate_up[e].T).chunk(2)`` (gate rows first,
  ``reference/fused_ops.py:170``), ``h = silu(gate) * up`` rounded once to bf16
  (both reference conventions round this intermediate to the activation dtype:
  ``reference/fused_ops.py:171``, ``target/prefill_t64/cpu_reference.py:177``),
  ``y = h @ down[e].T``;
* combine in float32 over the k slots, one cast at the end
  (``target/prefill_t64/cpu_reference.py:180``);
* shared expert ``down(silu(gate(x)) * up(x)) * sigmoid(x . w_gate)``
  (``fused/model.py:305-307``, ``cpu_reference.py:165-169``), added in float32
  before the single cast.

``moe_reference_order`` mirrors the bf16 rounding order of
``reference/fused_ops.py:148-173`` (bf16 GEMM outputs, bf16 weights, bf16 ``+=``
in ascending expert order) for information only; it is not the golden.

Pinning: ``tests/test_oracle_moe.py`` checks ``moe`` against an independent
dense formulation (every token through every expert, masked by a one-hot
routing matrix), the E=1/k=1 reduction to a dense SwiGLU MLP, zero-weight
experts contributing nothing, and the golden MoE vectors written by the
pure-Python brute force in ``tests/golden/make_golden.py``.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from . import routing, w4


def router_logits(hidden: torch.Tensor, router_weight: torch.Tensor) -> np.ndarray:
    """fp32 logits ``[T, E]`` from bf16 hidden ``[..., H]`` and router weight ``[E, H]`` (fp64 sums)."""
    x = hidden.reshape(-1, hidden.shape[-1]).to(torch.float64)
    w = router_weight.to(torch.float64)
    return (x @ w.T).to(torch.float32).numpy()


def _bank(bank, index: int, group_size: int) -> torch.Tensor:
    """Dequantise one expert of a packed bank ``(uint8 [E,N,K/2], scales [E,N,K/G])``."""
    packed, scales = bank
    return torch.from_numpy(w4.dequantize(packed[index].cpu().numpy(), scales[index], group_size))


def _ffn(x: torch.Tensor, gate_up: torch.Tensor, down: torch.Tensor, round_hidden: bool) -> torch.Tensor:
    gate, up = (x @ gate_up.T).chunk(2, dim=-1)
    h = F.silu(gate) * up
    if round_hidden:
        h = h.to(torch.bfloat16).to(torch.float32)
    return h @ down.T


def shared_expert(hidden: torch.Tensor, shared, group_size: int, *, round_hidden: bool = True) -> torch.Tensor:
    """fp32 ``[T, H]`` shared-expert output already multiplied by ``sigmoid(x . w_gate)``.

    ``shared = ((gate_up_packed [2I, H/2], gate_up_scales), (down_packed, down_scales), gate_weight [H])``.
    """
    (gu_p, gu_s), (dn_p, dn_s), gate_w = shared
    x = hidden.reshape(-1, hidden.shape[-1]).to(torch.float32)
    gu = torch.from_numpy(w4.dequantize(gu_p.cpu().numpy(), gu_s, group_size))
    dn = torch.from_numpy(w4.dequantize(dn_p.cpu().numpy(), dn_s, group_size))
    y = _ffn(x, gu, dn, round_hidden)
    gate = torch.sigmoid(x @ gate_w.reshape(-1).to(torch.float32))
    return y * gate[:, None]


def moe(hidden: torch.Tensor, logits: np.ndarray, top_k: int, gate_up, down, group_size: int, *,
        shared=None, round_hidden: bool = True) -> dict:
    """Golden routed MoE (+ optional shared expert) over packed banks.

    Returns ``ids, weights, perm, inv, offsets`` (routing) and ``out_f32`` /
    ``out`` (bf16) of shape ``[T, H]``.
    """
    x = hidden.reshape(-1, hidden.shape[-1]).to(torch.float32)
    num_experts = gate_up[0].shape[0]
    ids, weights = routing.topk(np.asarray(logits, dtype=np.float32), top_k)
    perm, inv, offsets = routing.permutation(ids, num_experts)
    t = x.shape[0]
    routed = torch.zeros((t, top_k, x.shape[1]), dtype=torch.float32)
    for expert in np.unique(ids).tolist():
        rows, slots = np.nonzero(ids == expert)
        gu = _bank(gate_up, expert, group_size)
        dn = _bank(down, expert, group_size)
        routed[rows, slots] = _ffn(x[rows], gu, dn, round_hidden)
    out = (routed * torch.from_numpy(weights)[..., None]).sum(dim=1)
    if shared is not None:
        out = out + shared_expert(hidden, shared, group_size, round_hidden=round_hidden)
    return dict(ids=ids, weights=weights, perm=perm, inv=inv, offsets=offsets,
                out_f32=out, out=out.to(torch.bfloat16))


def moe_dense(hidden: torch.Tensor, logits: np.ndarray, top_k: int, gate_up, down, *, shared=None,
              dequantize=None) -> torch.Tensor:
    """Same routed MoE over dense banks ``[E,2I,H]`` / ``[E,H,I]`` (any float dtype).

    This is the CPU-baseline form: the reference's ``moe`` consumes dense
    logical banks (``reference/fused_ops.py:148-159``).  Math runs in the
    banks' dtype per expert, combine in float32.  ``shared`` = (gate_up
    ``[2I,H]``, down ``[H,I]``, gate vector ``[H]``) adds the gated shared expert
    (``fused/model.py:305-307``).  With ``dequantize`` (a function of an expert
    index returning its dense ``(gate_up, down)``), ``gate_up``/``down`` are
    ignored and each hit expert is dequantised inside the call.
    """
    dtype = gate_up.dtype if dequantize is None else torch.bfloat16
    x = hidden.reshape(-1, hidden.shape[-1]).to(dtype)
    ids, weights = routing.topk(np.asarray(logits, dtype=np.float32), top_k)
    routed = torch.zeros((x.shape[0], top_k, x.shape[1]), dtype=torch.float32)
    for expert in np.unique(ids).tolist():
        rows, slots = np.nonzero(ids == expert)
        gu, dn = (gate_up[expert], down[expert]) if dequantize is None else dequantize(expert)
        gate, up = F.linear(x[rows], gu).chunk(2, dim=-1)
        routed[rows, slots] = F.linear(F.silu(gate) * up, dn).to(torch.float32)
    out = (routed * torch.from_numpy(weights)[..., None]).sum(dim=1)
    if shared is not None:
        sgu, sdn, sgate = shared
        gate, up = F.linear(x, sgu).chunk(2, dim=-1)
        y = F.linear(F.silu(gate) * up, sdn).to(torch.float32)
        out = out + y * torch.sigmoid(x.to(torch.float32) @ sgate.to(torch.float32))[:, None]
    return out.to(hidden.dtype)


def moe_reference_order(hidden: torch.Tensor, logits: np.ndarray, top_k: int, gate_up: torch.Tensor,
                        down: torch.Tensor) -> torch.Tensor:
    """bf16 rounding order of ``reference/fused_ops.py:160-173`` over dense bf16 banks (informational)."""
    flat = hidden.reshape(-1, hidden.shape[-1])
    ids, weights = routing.topk(np.asarray(logits, dtype=np.float32), top_k)
    w = torch.from_numpy(weights).to(flat.dtype)
    result = torch.zeros_like(flat)
    selected = torch.from_numpy(ids.astype(np.int64))
    for expert in range(gate_up.shape[0]):
        tokens, slots = torch.where(selected == expert)
        if not tokens.numel():
            continue
        gate, up = F.linear(flat[tokens], gate_up[expert]).chunk(2, dim=-1)
        values = F.linear(F.silu(gate) * up, down[expert])
        result[tokens] += values * w[tokens, slots, None]
    return result
