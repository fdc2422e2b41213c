"""Verify forward of the Qwen3.5-MoE target over a block of tokens, on the HIP kernels.

The decoder follows the reference's stateful target with an original-W4
quantization adapter (``model/qwen35_moe_dflash/fused/model.py``):

* ``_forward_hidden`` (``:386-427``): per layer ``h += mixer(norm(h))`` then
  ``h += moe(norm(h))`` with an fp32 residual stream, feature taps after the
  layers the drafter reads, final norm, LM head;
* ``_gdn`` (``:227-260``): in_proj_qkv -> conv-state update -> depthwise causal
  conv -> SiLU -> q/k/v split, q/k repeated to the value heads; beta =
  sigmoid(in_proj_b); g = -exp(A_log) * softplus(in_proj_a + dt_bias); gated
  delta rule with Q/K L2 normalisation; per-head RMS norm gated by SiLU(z);
  out_proj;
* ``_attention`` (``:271-288``): q_proj gives q and a gate per head; q/k RMS
  norms (weight + 1); partial rotary; cache append; causal GQA; output times
  sigmoid(gate); o_proj;
* ``_moe`` (``:296-307``): routed experts plus the shared expert scaled by
  sigmoid(x . w_gate) -- here one ``dflash_moe_w4a16`` launch sequence with the
  shared expert as one more slot.

What runs where: every int4 projection (``plan.int4_keys``) is a
``dflash_qlinear_w4a16`` launch, the projections that read the same activations
stacked into one matrix (GDN: qkv|z|b|a, attention: q|k|v); the MoE layer is
``dflash_moe_w4a16``; the rest (norms, conv, delta rule, rotary, attention,
residual adds) is batched PyTorch on the same stream (``layers``).

State layout (resident in HBM, sized once): per attention layer a KV cache
``[1, Hkv, capacity, D]`` bf16 written in place at ``[position, position+T)``;
per GDN layer the conv history ``[1, C, K-1]`` bf16 and the recurrent state
``[1, Hv, Dk, Dv]`` fp32.  A forward leaves the committed state untouched
(KV slots past ``position`` are not part of it) and returns a ``Pending``
record; ``commit(state, pending, j)`` then advances the state by the first
``j`` tokens of the block: the KV cache by moving ``position``, the conv
history by slicing the block's conv window, the recurrent state by rebuilding
it from the block's delta-rule writes (``layers.state_after``).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import NamedTuple, Optional

import torch
import torch.nn.functional as F
from torch import Tensor

from . import layers, ops
from .packing import PackedW4, SharedExpert
from .plan import TargetConfig

DRAFT_FEATURE_LAYERS = (1, 6, 11, 16, 22, 27, 32, 37)   # specs/draft-config.json target_layer_ids


def small_config(layers_: tuple = ("linear_attention", "full_attention"), vocab: int = 1024) -> TargetConfig:
    """A reduced-width geometry every kernel accepts (H 512, 16 experts): for tests."""
    return TargetConfig(hidden=512, layer_types=tuple(layers_), vocab=vocab, heads=4, kv_heads=2, head_dim=128,
                        linear_key_heads=4, linear_value_heads=16, linear_key_dim=128, linear_value_dim=128,
                        conv_kernel=4, experts=16, top_k=4, moe_inter=512, shared_inter=512)


# ------------------------------------------------------------------ weights
@dataclass
class LayerWeights:
    kind: str
    input_norm: Tensor                      # fp32 [H] (applied as weight + 1)
    post_norm: Tensor                       # fp32 [H]
    mixer_in: PackedW4                      # GDN: qkv|z|b|a stacked; attention: q|k|v stacked
    mixer_out: PackedW4                     # out_proj / o_proj
    router: Tensor                          # bf16 [E, H]
    gate_up: PackedW4                       # [E, 2I, H]
    down: PackedW4                          # [E, H, I]
    shared: SharedExpert
    conv: Optional[Tensor] = None           # GDN: bf16 [C, 1, K]
    a_log: Optional[Tensor] = None          # GDN: fp32 [Hv]
    dt_bias: Optional[Tensor] = None        # GDN: fp32 [Hv]
    gdn_norm: Optional[Tensor] = None       # GDN: fp32 [Dv] (applied as is)
    q_norm: Optional[Tensor] = None         # attention: fp32 [D] (weight + 1)
    k_norm: Optional[Tensor] = None


@dataclass
class TargetWeights:
    config: TargetConfig
    embedding: Tensor                       # int8 [V, H]
    embedding_scale: Tensor                 # fp32 [V, 1]
    final_norm: Tensor                      # fp32 [H] (weight + 1)
    lm_head: PackedW4                       # [V, H]
    layers: list = field(default_factory=list)


def _bank(gen, shape, device, group=128):
    """Random packed int4 bank on the device: uniform bytes (two uniform nibbles), scales U(0.005, 0.02)."""
    packed = torch.randint(0, 256, (*shape[:-1], shape[-1] // 2), dtype=torch.uint8, device=device, generator=gen)
    scales = torch.rand((*shape[:-1], shape[-1] // group), device=device, generator=gen) * 0.015 + 0.005
    return PackedW4(packed, scales.to(torch.bfloat16).contiguous(), group)


def random_weights(config: TargetConfig, *, seed: int = 0, device="cuda", layout: str = "tiled",
                   generate_on=None) -> TargetWeights:
    """Random-init W4 group-128 weights of the whole target (every projection, expert and the
    LM head packed int4; router and small vectors floating).  ``generate_on`` draws the random
    numbers on another device (e.g. ``"cpu"`` for a reproducible oracle check) and moves them."""
    config.validate()
    src = torch.device(generate_on) if generate_on is not None else torch.device(device)
    gen = torch.Generator(device=src).manual_seed(seed)
    c = config
    h = c.hidden

    def bank(*shape):
        b = _bank(gen, shape, src)
        b = b.to(device)
        return b.tiled() if layout == "tiled" else b

    def vec(n, lo, hi):
        return (torch.rand((n,), device=src, generator=gen) * (hi - lo) + lo).to(device)

    kw, vw = c.linear_key_heads * c.linear_key_dim, c.linear_value_heads * c.linear_value_dim
    hv = c.linear_value_heads
    out = TargetWeights(
        config=c,
        embedding=torch.randint(-127, 128, (c.vocab, h), dtype=torch.int8, device=src, generator=gen).to(device),
        embedding_scale=(torch.rand((c.vocab, 1), device=src, generator=gen) * 0.01 + 0.005).to(device),
        final_norm=vec(h, -0.1, 0.1), lm_head=bank(c.vocab, h))
    for kind in c.layer_types:
        common = dict(input_norm=vec(h, -0.1, 0.1), post_norm=vec(h, -0.1, 0.1))
        if kind == "linear_attention":
            mix = dict(mixer_in=bank(2 * kw + vw + vw + 2 * hv, h), mixer_out=bank(h, vw),
                       conv=(torch.randn((2 * kw + vw, 1, c.conv_kernel), device=src, generator=gen) * 0.3
                             ).to(torch.bfloat16).to(device),
                       a_log=torch.log(vec(hv, 1.0, 16.0)), dt_bias=vec(hv, -0.5, 0.5),
                       gdn_norm=vec(c.linear_value_dim, 0.9, 1.1))
        else:
            d = c.head_dim
            mix = dict(mixer_in=bank(2 * c.heads * d + 2 * c.kv_heads * d, h), mixer_out=bank(h, c.heads * d),
                       q_norm=vec(d, -0.1, 0.1), k_norm=vec(d, -0.1, 0.1))
        router = (torch.randn((c.experts, h), device=src, generator=gen) * 0.02).to(torch.bfloat16).to(device)
        gate_up, down = bank(c.experts, 2 * c.moe_inter, h), bank(c.experts, h, c.moe_inter)
        shared = SharedExpert(bank(2 * c.shared_inter, h), bank(h, c.shared_inter),
                              (torch.randn((h,), device=src, generator=gen) * 0.02).to(torch.bfloat16).to(device))
        out.layers.append(LayerWeights(kind=kind, router=router, gate_up=gate_up, down=down, shared=shared,
                                       **common, **mix))
    return out


def to_device(w: TargetWeights, device, *, layout: str = "tiled") -> TargetWeights:
    """A copy of ``w`` on ``device``, every packed bank in ``layout``."""
    def move(v):
        if isinstance(v, PackedW4):
            b = v.to(device)
            return b.tiled() if layout == "tiled" and b.layout != "tiled" else b
        if isinstance(v, SharedExpert):
            return SharedExpert(move(v.gate_up), move(v.down), v.gate_weight.to(device))
        if isinstance(v, Tensor):
            return v.to(device)
        return v
    out = TargetWeights(w.config, move(w.embedding), move(w.embedding_scale), move(w.final_norm), move(w.lm_head))
    for lw in w.layers:
        out.layers.append(LayerWeights(**{k: move(v) for k, v in vars(lw).items()}))
    return out


# ------------------------------------------------------------------ state
@dataclass
class TargetState:
    """Caches after ``position`` consumed tokens (``fused/session.py:55-76`` keeps the same
    fields per layer; here the KV caches have a fixed capacity and are written in place)."""

    position: int
    conv: list                  # per layer: bf16 [1, C, K-1] (GDN) or None
    recurrent: list             # per layer: fp32 [1, Hv, Dk, Dv] (GDN) or None
    keys: list                  # per layer: bf16 [1, Hkv, capacity, D] (attention) or None
    values: list

    @property
    def capacity(self) -> int:
        return next((k.shape[2] for k in self.keys if k is not None), 1 << 62)

    def clone(self) -> "TargetState":
        c = lambda t: None if t is None else t.clone()  # noqa: E731
        return TargetState(self.position, [c(t) for t in self.conv], [c(t) for t in self.recurrent],
                           [c(t) for t in self.keys], [c(t) for t in self.values])


class GdnPending(NamedTuple):
    window: Tensor              # bf16 [1, C, K-1+T]: conv history followed by the block's columns
    state: Tensor               # fp32 [1, Hv, Dk, Dv]: recurrent state before the block
    chunks: list                # layers.DeltaChunk per 16 tokens


class Pending(NamedTuple):
    """What a forward over a block leaves for ``commit``."""

    position: int
    tokens: int
    gdn: list                   # per layer: GdnPending or None


class Output(NamedTuple):
    hidden: Tensor              # fp32 [T, H] after the final norm
    top1: Optional[Tensor]      # int32 [T] argmax of the LM head (when asked for)
    features: Optional[Tensor]  # bf16 [T, len(feature_layers) * H] (when asked for)
    pending: Pending


# ------------------------------------------------------------------ model
class TargetModel:
    def __init__(self, weights: TargetWeights, *, capacity: int = 4096 + 64,
                 feature_layers: tuple = ()):
        self.w = weights
        self.config = c = weights.config
        self.capacity = capacity
        self.feature_layers = tuple(i for i in feature_layers if i < c.layers)
        self.device = weights.embedding.device
        self.inv_freq = layers.inverse_frequencies(c.rotary_dim, c.rope_theta, self.device)

    # -- state
    def new_state(self) -> TargetState:
        c, dev = self.config, self.device
        conv, rec, keys, vals = [], [], [], []
        for kind in c.layer_types:
            if kind == "linear_attention":
                conv.append(torch.zeros((1, c.conv_channels, c.conv_kernel - 1), dtype=torch.bfloat16, device=dev))
                rec.append(torch.zeros((1, c.linear_value_heads, c.linear_key_dim, c.linear_value_dim),
                                       dtype=torch.float32, device=dev))
                keys.append(None)
                vals.append(None)
            else:
                shape = (1, c.kv_heads, self.capacity, c.head_dim)
                keys.append(torch.zeros(shape, dtype=torch.bfloat16, device=dev))
                vals.append(torch.zeros(shape, dtype=torch.bfloat16, device=dev))
                conv.append(None)
                rec.append(None)
        return TargetState(0, conv, rec, keys, vals)

    def synthetic_context(self, length: int, *, seed: int = 0) -> TargetState:
        """A state as if ``length`` tokens had been consumed: random KV entries and GDN states of
        the magnitudes a forward produces (unit-RMS keys/values, bounded recurrent state)."""
        if length > self.capacity:
            raise ValueError("context longer than the KV capacity")
        st = self.new_state()
        gen = torch.Generator(device=self.device).manual_seed(seed)
        for i in range(self.config.layers):
            if st.keys[i] is not None:
                st.keys[i][:, :, :length] = torch.randn(st.keys[i][:, :, :length].shape, device=self.device,
                                                        generator=gen).to(torch.bfloat16)
                st.values[i][:, :, :length] = torch.randn(st.values[i][:, :, :length].shape, device=self.device,
                                                          generator=gen).to(torch.bfloat16)
            else:
                st.conv[i].copy_(torch.randn(st.conv[i].shape, device=self.device, generator=gen))
                st.recurrent[i].copy_(torch.randn(st.recurrent[i].shape, device=self.device, generator=gen) * 0.1)
        st.position = length
        return st

    # -- pieces
    def embed(self, ids: Tensor) -> Tensor:
        """int8 rows times their fp32 scale: the fp32 residual stream (``fused/quantization.py:138-141``)."""
        idx = ids.reshape(-1).long()
        return self.w.embedding[idx].float() * self.w.embedding_scale[idx]

    def _gdn(self, x: Tensor, lw: LayerWeights, conv_hist: Tensor, state: Tensor):
        c = self.config
        t = x.shape[0]
        kw, vw = c.linear_key_heads * c.linear_key_dim, c.linear_value_heads * c.linear_value_dim
        hv, hk, dk, dv = c.linear_value_heads, c.linear_key_heads, c.linear_key_dim, c.linear_value_dim
        proj = ops.qlinear(x, lw.mixer_in)                                    # bf16 [T, 2kw+vw | vw | Hv | Hv]
        qkv, z, b, a = proj.split((2 * kw + vw, vw, hv, hv), dim=-1)
        window = torch.cat((conv_hist, qkv.t()[None]), dim=2)               # [1, C, K-1+T]
        taps = window.unfold(2, c.conv_kernel, 1)[0].float()                  # [C, T, K]
        mixed = F.silu((taps * lw.conv[:, 0, None, :].float()).sum(-1)).t()   # fp32 [T, C]
        q, k, v = mixed.split((kw, kw, vw), dim=-1)
        rep = hv // hk
        q = q.reshape(t, hk, dk).repeat_interleave(rep, dim=1).transpose(0, 1)[None]   # [1, Hv, T, Dk]
        k = k.reshape(t, hk, dk).repeat_interleave(rep, dim=1).transpose(0, 1)[None]
        v = v.reshape(t, hv, dv).transpose(0, 1)[None]
        beta = torch.sigmoid(b.float()).t()[None]                              # [1, Hv, T]
        g = (-torch.exp(lw.a_log) * F.softplus(a.float() + lw.dt_bias)).t()[None]
        core, _, chunks = layers.delta_rule(q, k, v, g, beta, state, normalise=True)
        core = core[0].transpose(0, 1)                                        # [T, Hv, Dv]
        gated = layers.rms_normalise(core, lw.gdn_norm, c.rms_eps, 0.0) * F.silu(z.float().reshape(t, hv, dv))
        out = ops.qlinear(gated.reshape(t, vw).to(torch.bfloat16), lw.mixer_out)
        return out, GdnPending(window, state, chunks)

    def _attention(self, x: Tensor, lw: LayerWeights, keys: Tensor, values: Tensor, pos: int):
        c = self.config
        t, heads, kv, d = x.shape[0], c.heads, c.kv_heads, c.head_dim
        if pos + t > keys.shape[2]:
            raise ValueError("block would exceed the KV cache capacity")
        proj = ops.qlinear(x, lw.mixer_in)
        qg, k, v = proj.split((2 * heads * d, kv * d, kv * d), dim=-1)
        qg = qg.reshape(t, heads, 2 * d)
        q, gate = qg[..., :d], qg[..., d:]
        q = layers.rms_normalise(q, lw.q_norm, c.rms_eps, 1.0)
        k = layers.rms_normalise(k.reshape(t, kv, d), lw.k_norm, c.rms_eps, 1.0)
        cos, sin = layers.rotary_tables(torch.arange(pos, pos + t, device=x.device), self.inv_freq)
        q = layers.apply_rotary(q.transpose(0, 1), cos, sin)                  # [heads, T, D]
        k = layers.apply_rotary(k.transpose(0, 1), cos, sin)                  # [kv, T, D]
        keys[0, :, pos:pos + t] = k.to(torch.bfloat16)
        values[0, :, pos:pos + t] = v.reshape(t, kv, d).transpose(0, 1)
        att = layers.grouped_attention(q[None], keys[:, :, :pos + t], values[:, :, :pos + t], pos, d ** -0.5)
        mixed = att[0].transpose(0, 1).reshape(t, heads * d) * torch.sigmoid(gate.float().reshape(t, heads * d))
        return ops.qlinear(mixed.to(torch.bfloat16), lw.mixer_out)

    def _moe(self, x: Tensor, lw: LayerWeights, workspace: Optional[Tensor]):
        return ops.moe_w4a16(x, lw.gate_up, lw.down, top_k=self.config.top_k, router_weight=lw.router,
                             shared=lw.shared, workspace=workspace)

    def layer(self, i: int, hidden: Tensor, state: TargetState, workspace: Optional[Tensor] = None,
              trace: Optional[dict] = None):
        """One decoder layer on the fp32 residual ``[T, H]``; returns (hidden, GdnPending or None).
        ``trace`` (a dict) receives the residual after the mixer and the MoE input."""
        c, lw = self.config, self.w.layers[i]
        normed = layers.rms_normalise(hidden, lw.input_norm, c.rms_eps, 1.0).to(torch.bfloat16)
        pending = None
        if lw.kind == "linear_attention":
            mixed, pending = self._gdn(normed, lw, state.conv[i], state.recurrent[i])
        else:
            mixed = self._attention(normed, lw, state.keys[i], state.values[i], state.position)
        hidden = hidden + mixed.float()
        normed = layers.rms_normalise(hidden, lw.post_norm, c.rms_eps, 1.0).to(torch.bfloat16)
        if trace is not None:
            trace.update(mid=hidden, moe_in=normed)
        return hidden + self._moe(normed, lw, workspace).float(), pending

    def forward_hidden(self, hidden: Tensor, state: TargetState, *, top1: bool = True,
                       workspace: Optional[Tensor] = None) -> Output:
        """All layers, final norm and (``top1``) the LM head argmax over fp32 ``hidden [T, H]``."""
        t = hidden.shape[0]
        if state.position + t > self.capacity:
            raise ValueError("input would exceed the target context capacity")
        gdn, feats = [], []
        for i in range(self.config.layers):
            hidden, p = self.layer(i, hidden, state, workspace)
            gdn.append(p)
            if i in self.feature_layers:
                feats.append(hidden)
        final = layers.rms_normalise(hidden, self.w.final_norm, self.config.rms_eps, 1.0)
        best = None
        if top1:
            logits = ops.qlinear(final.to(torch.bfloat16), self.w.lm_head)
            best = logits.argmax(dim=-1).to(torch.int32)
        features = torch.cat(feats, dim=-1).to(torch.bfloat16) if feats else None
        return Output(final, best, features, Pending(state.position, t, gdn))

    def forward(self, ids: Tensor, state: TargetState, **kw) -> Output:
        return self.forward_hidden(self.embed(ids), state, **kw)

    def commit(self, state: TargetState, pending: Pending, accepted: int) -> None:
        """Advance ``state`` (in place) by the first ``accepted`` tokens of the block ``pending``
        describes.  ``accepted = 0`` leaves it as it was."""
        if pending.position != state.position:
            raise RuntimeError("pending block does not start at the state's position")
        if type(accepted) is not int or not 0 <= accepted <= pending.tokens:
            raise ValueError("accepted must be an integer in [0, block tokens]")
        if accepted == 0:
            return
        keep = self.config.conv_kernel - 1
        for i, p in enumerate(pending.gdn):
            if p is None:
                continue
            state.conv[i] = p.window[:, :, accepted:accepted + keep].clone()
            full, rest = divmod(accepted, layers.CHUNK)
            s = p.state
            for ch in p.chunks[:full]:
                s = ch.state
            if rest:
                ch = p.chunks[full]
                s = layers.state_after(s, ch.keys, ch.u, ch.cum, rest)
            state.recurrent[i] = s.clone() if s is p.state else s
        state.position += accepted
