"""Non-hot decoder arithmetic shared by the FusedOps module and the verify stack.

Plain PyTorch on the tensors' device (on MI355X: batched rocBLAS/elementwise
launches that a HIP graph can hold).  The qlinear and MoE layers are not here:
they are the HIP kernels of ``libdflash_hip.so``.

Gated delta rule (``model/qwen35_moe_dflash/fused/ops.py:54-71`` defines it by
the per-token recurrence ``S <- e^g S; u = beta (v - S^T k); S <- S + k u^T;
o = S^T q``): computed here chunk by chunk in closed form, see
:func:`delta_rule_chunk`.
"""
from __future__ import annotations

import math
from typing import NamedTuple, Optional

import torch
from torch import Tensor

# chunk length of the closed-form delta rule; the matmul-only inverse below is exact to fp32
# rounding at this length even for repeated keys (entries of (-A)^n stay below C(15,7))
CHUNK = 16


class DeltaChunk(NamedTuple):
    """What one chunk leaves behind: enough to rebuild the state after any prefix of it."""

    out: Tensor        # [B, H, C, Dv] outputs o_t
    state: Tensor      # [B, H, Dk, Dv] state after the whole chunk
    keys: Tensor       # [B, H, C, Dk] the (normalised) keys
    u: Tensor          # [B, H, C, Dv] the delta-rule writes u_t
    cum: Tensor        # [B, H, C] cumulative log decay G_t


def unit_lower_inverse(a: Tensor) -> Tensor:
    """``(I + A)^-1`` for strictly lower-triangular ``A`` ``[..., C, C]`` with ``C <= 16``.

    ``A`` is nilpotent (``A^C = 0``), so ``(I + A)^-1 = (I - A)(I + A^2)(I + A^4)(I + A^8)``:
    seven batched matmuls, no triangular-solve library call (graph-capturable).
    """
    c = a.shape[-1]
    if c > 16:
        raise ValueError("unit_lower_inverse handles chunks of at most 16")
    eye = torch.eye(c, dtype=a.dtype, device=a.device)
    inv = eye - a
    power = a @ a
    span = 2
    while span < c:
        inv = inv @ (eye + power)
        power = power @ power
        span *= 2
    return inv


def delta_rule_chunk(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor, state: Tensor, *,
                     unit_keys: bool) -> DeltaChunk:
    """One chunk of the gated delta rule in closed (WY) form, fp32, batched over ``[B, H]``.

    With ``G_t = sum_{s<=t} g_s`` the recurrence unrolls to the unit lower-triangular system
    ``(I + A) U = diag(beta) (V - diag(e^G) K S_0)``, ``A_ts = beta_t e^{G_t - G_s} k_t.k_s``
    for ``s < t``; then ``o_t = e^{G_t} S_0^T q_t + sum_{s<=t} e^{G_t - G_s} (q_t.k_s) u_s`` and
    the state after token ``j`` is ``e^{G_j} S_0 + sum_{s<=j} e^{G_j - G_s} k_s u_s^T``.
    Every decay factor used is ``e^{G_t - G_s}`` with ``s <= t`` (at most 1).

    ``unit_keys``: the keys are L2-normalised, so ``|A_ts| <= 1`` and the matmul-only inverse
    is exact to fp32 rounding; otherwise a triangular solve is used.
    Shapes: q, k ``[B,H,C,Dk]``, v ``[B,H,C,Dv]``, g, beta ``[B,H,C]``, state ``[B,H,Dk,Dv]``.
    """
    c = q.shape[2]
    cum = torch.cumsum(g, dim=-1)
    diff = cum[..., :, None] - cum[..., None, :]
    causal = torch.ones((c, c), dtype=torch.bool, device=q.device).tril()
    decay = torch.where(causal, diff, torch.full_like(diff, -math.inf)).exp()     # 0 above the diagonal
    a = (decay * (k @ k.transpose(-1, -2)) * beta[..., :, None]).tril(-1)
    head = cum.exp()[..., None]                                                    # e^{G_t}
    rhs = beta[..., None] * (v - head * (k @ state))
    if unit_keys and c <= 16:
        u = unit_lower_inverse(a) @ rhs
    else:
        eye = torch.eye(c, dtype=q.dtype, device=q.device)
        u = torch.linalg.solve_triangular(eye + a, rhs, upper=False, unitriangular=True)
    out = head * (q @ state) + (decay * (q @ k.transpose(-1, -2))) @ u
    new_state = state_after(state, k, u, cum, c)
    return DeltaChunk(out, new_state, k, u, cum)


def state_after(state: Tensor, keys: Tensor, u: Tensor, cum: Tensor, j: int) -> Tensor:
    """State after the first ``j`` tokens of a chunk (``j = 0``: the chunk's initial state)."""
    if j == 0:
        return state
    last = cum[..., j - 1:j]                                                       # G_j
    tail = (last - cum[..., :j]).exp()[..., None]                                  # e^{G_j - G_s}
    return last[..., None].exp() * state + (keys[..., :j, :] * tail).transpose(-1, -2) @ u[..., :j, :]


def l2_normalise(x: Tensor) -> Tensor:
    """``x / sqrt(|x|^2 + 1e-6)`` over the last axis (the kernel-side Q/K normalisation)."""
    return x * (x.square().sum(-1, keepdim=True) + 1e-6).rsqrt()


def delta_rule(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor, state: Tensor, *,
               normalise: bool, valid: Optional[Tensor] = None) -> tuple[Tensor, Tensor, list[DeltaChunk]]:
    """Gated delta rule over head-major fp32 ``[B, H, S, .]`` inputs, in chunks of 16.

    ``q`` is scaled by ``Dk^-1/2`` here (after the optional L2 normalisation).  Tokens where
    ``valid [B, 1, S]`` is false enter with ``g = beta = 0`` (the state passes through) and
    output zeros.  Returns the outputs ``[B, H, S, Dv]``, the final state and the chunks.
    """
    if normalise:
        q, k = l2_normalise(q), l2_normalise(k)
    q = q * q.shape[-1] ** -0.5
    if valid is not None:
        g = torch.where(valid, g, torch.zeros_like(g))
        beta = torch.where(valid, beta, torch.zeros_like(beta))
    s = q.shape[2]
    chunks = []
    for c0 in range(0, s, CHUNK):
        c1 = min(s, c0 + CHUNK)
        ch = delta_rule_chunk(q[:, :, c0:c1], k[:, :, c0:c1], v[:, :, c0:c1], g[:, :, c0:c1], beta[:, :, c0:c1],
                              state, unit_keys=normalise)
        chunks.append(ch)
        state = ch.state
    out = torch.cat([ch.out for ch in chunks], dim=2) if len(chunks) > 1 else chunks[0].out
    if valid is not None:
        out = torch.where(valid[..., None], out, torch.zeros_like(out))
    return out, state, chunks


def rms_normalise(x: Tensor, weight: Tensor, eps: float, addend: float) -> Tensor:
    """fp32 ``x / rms(x) * (weight + addend)`` (the quantized target's norm arithmetic,
    ``fused/model.py:206-215``: reductions and gamma in fp32, one offset)."""
    xf = x.float()
    inv = (xf.square().mean(-1, keepdim=True) + eps).rsqrt()
    return xf * inv * (weight.float() + addend)


def rotary_tables(positions: Tensor, inv_freq: Tensor) -> tuple[Tensor, Tensor]:
    """cos, sin ``[S, rotary_dim]`` for fp32 positions (``fused/model.py:262-269``)."""
    freq = positions.float()[:, None] * inv_freq[None, :]
    angle = torch.cat((freq, freq), dim=-1)
    return angle.cos(), angle.sin()


def apply_rotary(x: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
    """Rotate the first ``rotary_dim`` features of ``x [..., S, D]`` (half-split pairs), keep the rest."""
    width = cos.shape[-1]
    a, tail = x[..., :width], x[..., width:]
    first, second = a.chunk(2, dim=-1)
    rotated = a * cos + torch.cat((-second, first), dim=-1) * sin
    return torch.cat((rotated, tail), dim=-1)


def inverse_frequencies(rotary_dim: int, theta: float, device=None) -> Tensor:
    return 1.0 / (theta ** (torch.arange(0, rotary_dim, 2, dtype=torch.float32, device=device) / rotary_dim))


def grouped_attention(q: Tensor, keys: Tensor, values: Tensor, query_start: int, scale: float) -> Tensor:
    """Causal GQA in fp32: ``q [B,H,S,D]`` over ``keys/values [B,Hkv,T,D]`` (``T = query_start + S``).

    The query heads sharing a KV head are stacked into one block of rows, so each KV head is
    read once and never repeated.
    """
    b, heads, s, d = q.shape
    kv, t = keys.shape[1], keys.shape[2]
    group = heads // kv
    rows = q.float().reshape(b, kv, group * s, d)
    scores = (rows @ keys.float().transpose(2, 3).contiguous()) * scale
    pos = torch.arange(s, device=q.device).repeat(group) + query_start
    hidden = torch.arange(t, device=q.device)[None, :] > pos[:, None]
    probs = torch.softmax(scores.masked_fill(hidden, -math.inf), dim=-1)
    return (probs @ values.float()).reshape(b, heads, s, d)
