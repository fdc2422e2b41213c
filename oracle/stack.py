"""Oracle: one decoder layer of the Qwen3.5-MoE target (GDN or attention mixer + routed MoE).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Restates ``model/qwen35_moe_dflash/fused/model.py`` on the CPU, on dequantised
weights, the plain way: every projection a float64 product over the dequantised
matrix (``oracle.w4.qlinear``), the gated delta rule token by token and head by
head (``fused/ops.py:54-71`` defines it by that recurrence), attention with an
explicit per-head softmax, the MoE through ``oracle.moe``.  Which function
follows which lines:

* ``norm``             -- ``_norm`` quantized branch (``:206-217``): fp32 ``x * rsqrt(mean x^2 + eps) * (w + addend)``;
* ``split_gdn_projection``, ``key_heads_to_value_heads``, ``gated_norm``, ``gdn_layer``
                       -- ``_gdn`` (``:227-263``) with ``_gated_norm`` (``:219-225``);
* ``split_query_gate`` -- the q_proj split of ``_attention`` (``:281``);
* ``rotary``           -- ``_rotary`` (``:265-276``);
* ``attend``           -- the attention op's contract (``reference/fused_ops.py:127-144``,
                          ``fused/ops.py:92-106``): causal GQA, query i sees keys ``<= start + i``;
* ``attention_layer``  -- ``_attention`` (``:278-294``);
* ``moe_layer``        -- ``_moe`` (``:296-307``) via ``oracle.moe.moe`` (shared expert included);
* ``decoder_layer``    -- one iteration of ``_forward_hidden`` (``:396-405``).

The values rounded to bf16 are the ones the MI355X stack hands between its
kernels as bf16 (norm outputs entering a qlinear, qlinear outputs, the conv
history, the gated GDN output, the keys/values written to the cache, the
attention output entering o_proj, the MoE output), so the comparison measures
arithmetic, not a different choice of rounding points.

Pinning (``tests/test_oracle_stack.py``): the delta-rule loop by closed forms
(beta = 0 decays only; orthonormal keys store values exactly); ``rotary`` by the
complex-number rotation of each (i, i + width/2) pair, identity at position 0
and invariance of q.k under a common shift; ``attend`` by one visible key
returning its value, equal keys giving the mean of exactly the visible values,
the two-key softmax in closed form and the query-head -> KV-head map;
``attention_layer`` by a closed form in which zero query rows make the
attention uniform, so the output is o_proj of (mean of the visible values)
times sigmoid(second half of each head's q_proj rows); ``gdn_layer`` by a
one-token closed form (all-ones input, beta = 0 by construction) that depends
on the projection split order, the key-head map, the conv window and the gated
norm; the norm on hand values; the whole GDN layer by its causal invariant
(T tokens at once equals two blocks with the state carried).  Each closed form
is shown to fail on a planted mistake (gate and query halves swapped, rotary
halves swapped or interleaved, an off-by-one mask, the wrong head map, the
projection split reordered, a zero-centred gated norm, a dropped decay).
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


def split_gdn_projection(proj: torch.Tensor, c):
    """The stacked GDN input projection ``[T, qkv | z | b | a]`` in that order (``:231-245``)."""
    kw, vw = c.linear_key_heads * c.linear_key_dim, c.linear_value_heads * c.linear_value_dim
    hv = c.linear_value_heads
    return proj.split((2 * kw + vw, vw, hv, hv), dim=-1)


def key_heads_to_value_heads(m: torch.Tensor, value_heads: int) -> torch.Tensor:
    """``[T, Hk, D] -> [T, Hv, D]``: value head h reads key head ``h // (Hv / Hk)``
    (``repeat_interleave`` over the head axis, ``:240``)."""
    return m.repeat_interleave(value_heads // m.shape[1], dim=1)


def gated_norm(core: torch.Tensor, z: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """``_gated_norm`` quantized branch (``:219-223``): fp32 RMS norm over each head's features
    with the weight applied as is (not zero-centred), times SiLU(z)."""
    return norm(core.to(torch.float32), weight, eps, 0.0) * F.silu(z.to(torch.float32))


def gdn_layer(x: torch.Tensor, lw: dict, conv_hist: torch.Tensor, state: torch.Tensor, c) -> dict:
    """GDN mixer of bf16-valued ``x [T, H]`` (the normed input); returns its output and states."""
    t = x.shape[0]
    kw, vw = c.linear_key_heads * c.linear_key_dim, c.linear_value_heads * c.linear_value_dim
    hv, hk, dk, dv = c.linear_value_heads, c.linear_key_heads, c.linear_key_dim, c.linear_value_dim
    proj = linear(x, lw["mixer_in"])
    qkv, z, b, a = split_gdn_projection(proj, c)
    window = torch.cat((conv_hist.to(torch.float32), qkv.t()), dim=1)            # [C, K-1+T]
    taps = c.conv_kernel
    conv = torch.stack([(window[:, s:s + taps] * lw["conv"][:, 0, :].float()).sum(-1) for s in range(t)])
    mixed = F.silu(conv)                                                          # [T, C]
    q, k, v = mixed.split((kw, kw, vw), dim=-1)
    q = key_heads_to_value_heads(q.reshape(t, hk, dk), hv)
    k = key_heads_to_value_heads(k.reshape(t, hk, dk), hv)
    v = v.reshape(t, hv, dv)
    q = q / torch.sqrt(q.square().sum(-1, keepdim=True) + 1e-6) * dk ** -0.5
    k = k / torch.sqrt(k.square().sum(-1, keepdim=True) + 1e-6)
    beta = torch.sigmoid(b)
    g = -torch.exp(lw["a_log"].float()) * F.softplus(a + lw["dt_bias"].float())
    core, states = delta_rule(q, k, v, g, beta, state[0])
    gated = gated_norm(core, z.reshape(t, hv, dv), lw["gdn_norm"], c.rms_eps)
    out = linear(bf16(gated.reshape(t, vw)), lw["mixer_out"])
    return {"out": out, "window": window, "states": states}


def split_query_gate(proj: torch.Tensor, heads: int, d: int):
    """q_proj output ``[T, heads * 2d]`` -> query and output gate ``[T, heads, d]`` each: head h
    owns rows ``[2d h, 2d h + 2d)``, its query first and its gate second (``:281``)."""
    qg = proj.reshape(proj.shape[0], heads, 2 * d)
    return qg[..., :d], qg[..., d:]


def rotary(m: torch.Tensor, positions: torch.Tensor, width: int, theta: float) -> torch.Tensor:
    """``_rotary`` (``:265-276``) of ``m [T, heads, D]`` at ``positions [T]``: the first ``width``
    features rotate-half style (feature i < width/2 pairs with i + width/2, angle
    position * theta^(-2i / width)), the rest unchanged; fp32 cos/sin as the quantized path."""
    inv = 1.0 / (theta ** (torch.arange(0, width, 2, dtype=torch.float64) / width))
    angle = positions.to(torch.float64)[:, None] * inv[None]
    angle = torch.cat((angle, angle), dim=-1)
    cos, sin = angle.cos().float()[:, None, :], angle.sin().float()[:, None, :]
    a_, tail = m[..., :width], m[..., width:]
    first, second = a_.chunk(2, dim=-1)
    return torch.cat((a_ * cos + torch.cat((-second, first), dim=-1) * sin, tail), dim=-1)


def visible_keys(position: int, i: int) -> int:
    """Keys query i of a block starting at ``position`` attends to: positions ``<= position + i``."""
    return position + i + 1


def query_kv_head(h: int, group: int) -> int:
    """KV head read by query head h when ``group`` query heads share one (``repeat_interleave``
    of the cache over heads, ``reference/fused_ops.py:137-139``)."""
    return h // group


def attend(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, position: int, scale: float) -> torch.Tensor:
    """Causal GQA in float64: ``q [T, heads, D]`` over ``keys/values [Hkv, >= position + T, D]``;
    query head h reads KV head ``query_kv_head``, query i the first ``visible_keys`` rows."""
    t, heads, d = q.shape
    group = heads // keys.shape[0]
    out = torch.empty((t, heads, d))
    for h in range(heads):
        kv = query_kv_head(h, group)
        kk, vv = keys[kv].double(), values[kv].double()
        for i in range(t):
            n = visible_keys(position, i)
            p = torch.softmax((kk[:n] @ q[i, h].double()) * scale, dim=0)
            out[i, h] = (p @ vv[:n]).float()
    return out


def attention_layer(x: torch.Tensor, lw: dict, keys: torch.Tensor, values: torch.Tensor, position: int, c) -> dict:
    """Attention mixer of bf16-valued ``x [T, H]`` over a cache holding ``position`` tokens
    (``keys/values [Hkv, >= position, D]``); returns its output and the new cache rows."""
    t, heads, kv, d = x.shape[0], c.heads, c.kv_heads, c.head_dim
    proj = linear(x, lw["mixer_in"])
    qg, k, v = proj.split((2 * heads * d, kv * d, kv * d), dim=-1)
    q, gate = split_query_gate(qg, heads, d)
    q = norm(q, lw["q_norm"], c.rms_eps, 1.0)
    k = norm(k.reshape(t, kv, d), lw["k_norm"], c.rms_eps, 1.0)
    pos = torch.arange(position, position + t)
    q = rotary(q, pos, c.rotary_dim, c.rope_theta)
    k = bf16(rotary(k, pos, c.rotary_dim, c.rope_theta))
    v = v.reshape(t, kv, d)
    all_k = torch.cat((keys[:, :position].to(torch.float32), k.transpose(0, 1)), dim=1)      # [Hkv, P+T, D]
    all_v = torch.cat((values[:, :position].to(torch.float32), v.transpose(0, 1)), dim=1)
    out = attend(q, all_k, all_v, position, d ** -0.5)
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
