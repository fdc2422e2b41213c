"""Oracle: one decoder layer of the Qwen3.5-MoE target (GDN or attention mixer + routed MoE).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Restates ``model/qwen35_moe_dflash/fused/model.py`` on the CPU, on dequantised
weights, the plain way: every projection a float64 product over the dequantised
matrix (``oracle.w4.qlinear``), the gated delta rule token by token and head by
head (``fused/ops.py:54-71`` defines it by that recurrence), attention with an
explicit per-head softmax over the repeated KV heads, the MoE through
``oracle.moe``.  Which function follows which lines:

* ``norm``            -- ``_norm`` quantized branch (``:206-215``): fp32 ``x * rsqrt(mean x^2 + eps) * (w + addend)``;
* ``gdn_layer``       -- ``_gdn`` (``:227-260``) with ``_gated_norm`` (``:217-225``);
* ``attention_layer`` -- ``_attention`` (``:271-288``) and ``_rotary`` (``:262-269``);
* ``moe_layer``       -- ``_moe`` (``:296-307``) via ``oracle.moe.moe`` (shared expert included);
* ``decoder_layer``   -- one iteration of ``_forward_hidden`` (``:397-405``).

The values rounded to bf16 are the ones the MI355X stack hands between its
kernels as bf16 (norm outputs entering a qlinear, qlinear outputs, the conv
history, the gated GDN output, the keys/values written to the cache, the
attention output entering o_proj, the MoE output), so the comparison measures
arithmetic, not a different choice of rounding points.

Pinning: ``tests/test_oracle_stack.py`` checks the delta-rule loop against closed
forms (beta = 0 decays only; orthonormal keys store values exactly), the
attention against uniform-key means, the norm against hand values, and the
whole layer against its own invariants (T = 1 then T - 1 tokens equals T tokens
at once).
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

from . import moe as oracle_moe, w4


def bf16(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16).to(torch.float32)


def norm(x: torch.Tensor, weight: torch.Tensor, eps: float, addend: float) -> torch.Tensor:
    xf = x.to(torch.float32)
    return xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + eps) * (weight.to(torch.float32) + addend)


def linear(x: torch.Tensor, bank) -> torch.Tensor:
    """bf16 activations times a packed bank ``(packed, scales, group)`` -> bf16-rounded fp32."""
    packed, scales, group = bank
    out = w4.qlinear(x.to(torch.bfloat16), packed.numpy(), scales, group)
    return bf16(torch.from_numpy(np.asarray(out, dtype=np.float64)).to(torch.float32))


def delta_rule(q, k, v, g, beta, state):
    """Token-by-token gated delta rule for one sequence, fp64.

    q, k ``[T, H, Dk]`` (already L2-normalised and scaled), v ``[T, H, Dv]``, g, beta ``[T, H]``,
    state ``[H, Dk, Dv]``.  Returns outputs ``[T, H, Dv]`` and the states after every token
    ``[T + 1, H, Dk, Dv]`` (index 0 is the initial state).
    """
    q, k, v, g, beta = (t.to(torch.float64) for t in (q, k, v, g, beta))
    s = state.to(torch.float64).clone()
    outs, states = [], [s.clone()]
    for t in range(q.shape[0]):
        for h in range(q.shape[1]):
            st = s[h] * math.exp(float(g[t, h]))
            u = float(beta[t, h]) * (v[t, h] - st.T @ k[t, h])
            s[h] = st + torch.outer(k[t, h], u)
        outs.append(torch.einsum("hkv,hk->hv", s, q[t]))
        states.append(s.clone())
    return torch.stack(outs), torch.stack(states)


def gdn_layer(x: torch.Tensor, lw: dict, conv_hist: torch.Tensor, state: torch.Tensor, c) -> dict:
    """GDN mixer of bf16-valued ``x [T, H]`` (the normed input); returns its output and states."""
    t = x.shape[0]
    kw, vw = c.linear_key_heads * c.linear_key_dim, c.linear_value_heads * c.linear_value_dim
    hv, hk, dk, dv = c.linear_value_heads, c.linear_key_heads, c.linear_key_dim, c.linear_value_dim
    proj = linear(x, lw["mixer_in"])
    qkv, z, b, a = proj.split((2 * kw + vw, vw, hv, hv), dim=-1)
    window = torch.cat((conv_hist.to(torch.float32), qkv.t()), dim=1)            # [C, K-1+T]
    taps = c.conv_kernel
    conv = torch.stack([(window[:, s:s + taps] * lw["conv"][:, 0, :].float()).sum(-1) for s in range(t)])
    mixed = F.silu(conv)                                                          # [T, C]
    q, k, v = mixed.split((kw, kw, vw), dim=-1)
    rep = hv // hk
    q = q.reshape(t, hk, dk).repeat_interleave(rep, dim=1)
    k = k.reshape(t, hk, dk).repeat_interleave(rep, dim=1)
    v = v.reshape(t, hv, dv)
    q = q / torch.sqrt(q.square().sum(-1, keepdim=True) + 1e-6) * dk ** -0.5
    k = k / torch.sqrt(k.square().sum(-1, keepdim=True) + 1e-6)
    beta = torch.sigmoid(b)
    g = -torch.exp(lw["a_log"].float()) * F.softplus(a + lw["dt_bias"].float())
    core, states = delta_rule(q, k, v, g, beta, state[0])
    gated = norm(core.to(torch.float32), lw["gdn_norm"], c.rms_eps, 0.0) * F.silu(z.reshape(t, hv, dv))
    out = linear(bf16(gated.reshape(t, vw)), lw["mixer_out"])
    return {"out": out, "window": window, "states": states}


def attention_layer(x: torch.Tensor, lw: dict, keys: torch.Tensor, values: torch.Tensor, position: int, c) -> dict:
    """Attention mixer of bf16-valued ``x [T, H]`` over a cache holding ``position`` tokens
    (``keys/values [Hkv, >= position, D]``); returns its output and the new cache rows."""
    t, heads, kv, d = x.shape[0], c.heads, c.kv_heads, c.head_dim
    proj = linear(x, lw["mixer_in"])
    qg, k, v = proj.split((2 * heads * d, kv * d, kv * d), dim=-1)
    qg = qg.reshape(t, heads, 2 * d)
    q, gate = qg[..., :d], qg[..., d:]
    q = norm(q, lw["q_norm"], c.rms_eps, 1.0)
    k = norm(k.reshape(t, kv, d), lw["k_norm"], c.rms_eps, 1.0)
    width = c.rotary_dim
    inv = 1.0 / (c.rope_theta ** (torch.arange(0, width, 2, dtype=torch.float64) / width))
    pos = torch.arange(position, position + t, dtype=torch.float64)
    angle = torch.cat((pos[:, None] * inv[None], pos[:, None] * inv[None]), dim=-1)
    cos, sin = angle.cos().float()[:, None, :], angle.sin().float()[:, None, :]

    def rotate(m):
        a_, tail = m[..., :width], m[..., width:]
        first, second = a_.chunk(2, dim=-1)
        return torch.cat((a_ * cos + torch.cat((-second, first), dim=-1) * sin, tail), dim=-1)
    q, k = rotate(q), bf16(rotate(k))
    v = v.reshape(t, kv, d)
    all_k = torch.cat((keys[:, :position].to(torch.float32), k.transpose(0, 1)), dim=1)      # [Hkv, P+T, D]
    all_v = torch.cat((values[:, :position].to(torch.float32), v.transpose(0, 1)), dim=1)
    group = heads // kv
    out = torch.empty((t, heads, d))
    for h in range(heads):
        kk, vv = all_k[h // group].double(), all_v[h // group].double()
        for i in range(t):
            visible = position + i + 1
            scores = (kk[:visible] @ q[i, h].double()) * d ** -0.5
            p = torch.softmax(scores, dim=0)
            out[i, h] = (p @ vv[:visible]).float()
    mixed = out.reshape(t, heads * d) * torch.sigmoid(gate.reshape(t, heads * d))
    return {"out": linear(bf16(mixed), lw["mixer_out"]), "keys": k.transpose(0, 1), "values": v.transpose(0, 1)}


def moe_layer(x: torch.Tensor, lw: dict, top_k: int, logits=None) -> dict:
    """Routed experts + gated shared expert of bf16-valued ``x [T, H]`` (``oracle.moe``); the
    routing runs on ``logits`` when given (fp32 ``[T, E]``), else on the oracle's own."""
    if logits is None:
        logits = oracle_moe.router_logits(x.to(torch.bfloat16), lw["router"])
    gu, dn = lw["gate_up"], lw["down"]
    sgu, sdn, sgate = lw["shared"]
    golden = oracle_moe.moe(x.to(torch.bfloat16), logits, top_k, (gu[0], gu[1]), (dn[0], dn[1]), gu[2],
                            shared=((sgu[0], sgu[1]), (sdn[0], sdn[1]), sgate))
    return {"out": bf16(golden["out_f32"]), "ids": golden["ids"]}


def decoder_layer(hidden: torch.Tensor, lw: dict, layer_state: dict, position: int, c, *, moe_logits=None) -> dict:
    """One layer on the fp32 residual ``[T, H]``: ``h += mixer(norm(h)); h += moe(norm(h))``."""
    normed = bf16(norm(hidden, lw["input_norm"], c.rms_eps, 1.0))
    if lw["kind"] == "linear_attention":
        mix = gdn_layer(normed, lw, layer_state["conv"], layer_state["recurrent"], c)
    else:
        mix = attention_layer(normed, lw, layer_state["keys"], layer_state["values"], position, c)
    mid = hidden + mix["out"]
    moe_in = bf16(norm(mid, lw["post_norm"], c.rms_eps, 1.0))
    moe = moe_layer(moe_in, lw, c.top_k, moe_logits)
    return {"hidden": mid + moe["out"], "mid": mid, "moe_in": moe_in, "mixer": mix, "ids": moe["ids"]}
