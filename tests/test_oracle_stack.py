"""CPU: pin the decoder-layer oracle (``oracle/stack.py``).

Closed forms for its pieces -- the token-by-token delta rule (beta = 0 only
decays the state; orthonormal keys with beta = 1, g = 0 store the values
exactly), the norm on hand values, the rotary embedding as a complex rotation
of each (i, i + width/2) pair, causal GQA attention (one visible key, equal
keys, two keys, the head map) -- closed forms of both whole mixers (the
attention layer with zero query rows, the GDN layer on one all-ones token with
beta = 0), and an invariant of the whole GDN layer: consuming T tokens at once
equals consuming them in two blocks with the conv window and recurrent state
carried between (the layer is a causal recurrence).  Every closed form is shown
to fail on a planted mistake, planted by replacing the oracle's own helper.
"""
import math

import pytest
import torch

from oracle import stack

from stack_util import oracle_layer_weights


def test_norm_hand_values():
    x = torch.tensor([[3.0, -4.0]])
    out = stack.norm(x, torch.tensor([0.5, -1.0]), 0.0, 1.0)
    rms = math.sqrt((9 + 16) / 2)
    torch.testing.assert_close(out, torch.tensor([[3 / rms * 1.5, -4 / rms * 0.0]]))


def _delta_inputs(seed, t=6, h=2, dk=4, dv=3):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn((t, h, dk), generator=gen)
    k = torch.randn((t, h, dk), generator=gen)
    k = k / k.norm(dim=-1, keepdim=True)
    v = torch.randn((t, h, dv), generator=gen)
    g = -torch.rand((t, h), generator=gen)
    beta = torch.rand((t, h), generator=gen)
    s0 = torch.randn((h, dk, dv), generator=gen)
    return q, k, v, g, beta, s0


def test_delta_rule_without_writes_only_decays():
    q, k, v, g, _, s0 = _delta_inputs(1)
    out, states = stack.delta_rule(q, k, v, g, torch.zeros_like(g), s0)
    cum = torch.cumsum(g.double(), dim=0)
    for t in range(q.shape[0]):
        expect = s0.double() * cum[t].exp()[:, None, None]
        torch.testing.assert_close(states[t + 1], expect)
        torch.testing.assert_close(out[t], torch.einsum("hkv,hk->hv", expect, q[t].double()))


def test_delta_rule_stores_values_at_orthonormal_keys():
    dk, dv, t = 5, 3, 4
    basis, _ = torch.linalg.qr(torch.randn((dk, dk), generator=torch.Generator().manual_seed(2), dtype=torch.float64))
    k = basis[:t, None, :].float()
    v = torch.randn((t, 1, dv), generator=torch.Generator().manual_seed(3))
    s0 = torch.randn((1, dk, dv), generator=torch.Generator().manual_seed(4))
    _, states = stack.delta_rule(k, k, v, torch.zeros((t, 1)), torch.ones((t, 1)), s0)
    # the keys are orthonormal to fp32 rounding (they enter as float32)
    torch.testing.assert_close((k[:, 0].double() @ states[-1][0]), v[:, 0].double(), rtol=1e-6, atol=1e-6)


def test_planted_missing_decay_fails_the_closed_form():
    """The closed form above is sensitive: a recurrence that forgets e^g misses it."""
    q, k, v, g, _, s0 = _delta_inputs(5)
    _, states = stack.delta_rule(q, k, v, torch.zeros_like(g), torch.zeros_like(g), s0)
    expect = s0.double() * torch.cumsum(g.double(), dim=0)[-1].exp()[:, None, None]
    assert (states[-1] - expect).abs().max() > 1e-2


def test_gdn_layer_is_a_causal_recurrence(pkg):
    c = pkg.target.small_config(("linear_attention",))
    w = pkg.target.random_weights(c, seed=7, device="cpu", layout="portable", generate_on="cpu")
    lw = oracle_layer_weights(w.layers[0])
    gen = torch.Generator().manual_seed(8)
    x = torch.randn((6, c.hidden), generator=gen).to(torch.bfloat16).float()
    conv = torch.randn((c.conv_channels, c.conv_kernel - 1), generator=gen).to(torch.bfloat16)
    rec = torch.randn((1, c.linear_value_heads, c.linear_key_dim, c.linear_value_dim), generator=gen) * 0.1
    whole = stack.gdn_layer(x, lw, conv, rec, c)
    first = stack.gdn_layer(x[:4], lw, conv, rec, c)
    carried_conv = first["window"][:, -(c.conv_kernel - 1):].to(torch.bfloat16)
    second = stack.gdn_layer(x[4:], lw, carried_conv, first["states"][-1][None].float(), c)
    torch.testing.assert_close(torch.cat([first["out"], second["out"]]), whole["out"], rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(second["states"][-1], whole["states"][-1], rtol=1e-5, atol=1e-5)


# ------------------------------------------------------------------ rotary (fused/model.py:265-276)
def _complex_rotation(m, positions, width, theta):
    """Independent statement: feature pair (i, i + width/2) is the complex number
    m_i + j m_{i + width/2}, turned by position * theta^(-2i / width)."""
    half = width // 2
    z = m[..., :half].double() + 1j * m[..., half:width].double()
    freq = theta ** (-torch.arange(half, dtype=torch.float64) * 2 / width)
    turn = torch.exp(1j * positions.double()[:, None] * freq[None])[:, None, :]
    r = z * turn
    return torch.cat((r.real, r.imag, m[..., width:].double()), dim=-1)


def _rotary_pinned(fn) -> bool:
    gen = torch.Generator().manual_seed(21)
    m = torch.randn((5, 3, 32), generator=gen)
    pos = torch.tensor([0, 1, 7, 4095, 100000])
    got = fn(m, pos, 16, 10_000_000.0).double()
    return torch.allclose(got, _complex_rotation(m, pos, 16, 10_000_000.0), rtol=1e-5, atol=1e-5)


def _rotary_swapped_halves(m, positions, width, theta):
    a_, tail = m[..., :width], m[..., width:]
    first, second = a_.chunk(2, dim=-1)
    rot = stack.rotary(torch.cat((second, first, tail), dim=-1), positions, width, theta)
    f2, s2 = rot[..., :width].chunk(2, dim=-1)
    return torch.cat((s2, f2, rot[..., width:]), dim=-1)


def _rotary_interleaved(m, positions, width, theta):
    """The other RoPE convention (pairs 2i, 2i + 1): a plausible misreading."""
    idx = torch.cat((torch.arange(0, width, 2), torch.arange(1, width, 2), torch.arange(width, m.shape[-1])))
    back = torch.argsort(idx)
    return stack.rotary(m[..., idx], positions, width, theta)[..., back]


def test_rotary_is_the_complex_rotation_of_half_pairs():
    assert _rotary_pinned(stack.rotary)
    assert not _rotary_pinned(_rotary_swapped_halves)
    assert not _rotary_pinned(_rotary_interleaved)


def test_rotary_identity_at_zero_and_shift_invariant_dot():
    gen = torch.Generator().manual_seed(22)
    q, k = torch.randn((1, 2, 64), generator=gen), torch.randn((1, 2, 64), generator=gen)
    torch.testing.assert_close(stack.rotary(q, torch.tensor([0]), 16, 1e6), q)
    tail = stack.rotary(q, torch.tensor([999]), 16, 1e6)[..., 16:]
    torch.testing.assert_close(tail, q[..., 16:])  # partial rotary: only the first width features turn
    dots = []
    for shift in (0, 17, 3000):
        rq = stack.rotary(q, torch.tensor([40 + shift]), 16, 1e6).double()
        rk = stack.rotary(k, torch.tensor([9 + shift]), 16, 1e6).double()
        dots.append((rq * rk).sum(-1))
    torch.testing.assert_close(dots[1], dots[0], rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(dots[2], dots[0], rtol=1e-5, atol=1e-5)


# ------------------------------------------------------------------ attention (reference/fused_ops.py:127-144)
def test_attend_one_visible_key_returns_its_value():
    gen = torch.Generator().manual_seed(23)
    q = torch.randn((1, 4, 8), generator=gen)
    keys, values = torch.randn((2, 3, 8), generator=gen), torch.randn((2, 3, 8), generator=gen)
    out = stack.attend(q, keys, values, 0, 0.3)
    for h in range(4):
        torch.testing.assert_close(out[0, h], values[h // 2, 0])


def _uniform_attention_pinned() -> bool:
    """Equal keys: query i of a block at position 2 averages exactly the first 3 + i values of
    its KV head (query head h reads KV head h // 2)."""
    gen = torch.Generator().manual_seed(24)
    t, position = 3, 2
    q = torch.randn((t, 4, 8), generator=gen)
    keys = torch.randn((1, 1, 8), generator=gen).expand(2, position + t, 8).clone()
    values = torch.randn((2, position + t, 8), generator=gen)
    out = stack.attend(q, keys, values, position, 0.125)
    for i in range(t):
        for h in range(4):
            expect = values[h // 2, :position + i + 1].double().mean(0).float()
            if not torch.allclose(out[i, h], expect, rtol=1e-6, atol=1e-6):
                return False
    return True


def test_attend_equal_keys_average_exactly_the_visible_values(monkeypatch):
    assert _uniform_attention_pinned()
    with monkeypatch.context() as mp:  # off-by-one mask
        mp.setattr(stack, "visible_keys", lambda position, i: position + i)
        assert not _uniform_attention_pinned()
    with monkeypatch.context() as mp:  # query heads spread round-robin over the KV heads
        mp.setattr(stack, "query_kv_head", lambda h, group: h % 2)
        assert not _uniform_attention_pinned()


def test_attend_two_keys_closed_form():
    q = torch.tensor([[[1.0, 2.0]]])
    keys = torch.tensor([[[0.5, 0.0], [0.0, 1.0]]])
    values = torch.tensor([[[1.0, -1.0], [3.0, 5.0]]])
    out = stack.attend(q, keys, values, 1, 0.7)
    p1 = 1.0 / (1.0 + math.exp(0.7 * (2.0 - 0.5)))  # weight of key 0: sigmoid(s0 - s1)
    expect = torch.tensor([p1 * 1.0 + (1 - p1) * 3.0, p1 * -1.0 + (1 - p1) * 5.0])
    torch.testing.assert_close(out[0, 0], expect)


def _attention_weights(pkg, seed):
    c = pkg.target.small_config(("full_attention",))
    w = pkg.target.random_weights(c, seed=seed, device="cpu", layout="portable", generate_on="cpu")
    return c, oracle_layer_weights(w.layers[0])


def _attention_layer_pinned(c, lw, x, keys, values, position) -> bool:
    """Zero query rows make every score 0 (q_norm of 0 is 0), so query i of head h returns the
    mean of the first position + i + 1 values of KV head h // (heads / kv_heads), times
    sigmoid of its gate: the second d of head h's 2d q_proj rows."""
    t, heads, kv, d = x.shape[0], c.heads, c.kv_heads, c.head_dim
    proj = stack.linear(x, lw["mixer_in"])
    gate_rows = [2 * d * h + d + j for h in range(heads) for j in range(d)]
    gate = proj[:, gate_rows].reshape(t, heads, d)
    v_new = proj[:, 2 * heads * d + kv * d:].reshape(t, kv, d)
    all_v = torch.cat((values[:, :position].float(), v_new.transpose(0, 1)), dim=1).double()
    mixed = torch.empty((t, heads, d), dtype=torch.float64)
    for i in range(t):
        for h in range(heads):
            mixed[i, h] = all_v[h // (heads // kv), :position + i + 1].mean(0)
    mixed = mixed.float() * torch.sigmoid(gate)
    expect = stack.linear(stack.bf16(mixed.reshape(t, heads * d)), lw["mixer_out"])
    got = stack.attention_layer(x, lw, keys, values, position, c)["out"]
    return torch.allclose(got, expect, rtol=2e-2, atol=2e-2 * float(expect.abs().max()))


def test_attention_layer_closed_form(pkg, monkeypatch):
    c, lw = _attention_weights(pkg, 31)
    d = c.head_dim
    packed, scales, group = lw["mixer_in"]
    packed = packed.clone()
    for h in range(c.heads):
        packed[2 * d * h:2 * d * h + d] = 0          # every query row 0, the gate rows untouched
    lw["mixer_in"] = (packed, scales, group)
    gen = torch.Generator().manual_seed(32)
    position, t = 5, 3
    x = stack.bf16(torch.randn((t, c.hidden), generator=gen))
    keys = torch.randn((c.kv_heads, position, d), generator=gen).to(torch.bfloat16)
    values = torch.randn((c.kv_heads, position, d), generator=gen).to(torch.bfloat16)
    assert _attention_layer_pinned(c, lw, x, keys, values, position)
    with monkeypatch.context() as mp:   # query and gate halves swapped
        mp.setattr(stack, "split_query_gate", lambda proj, heads, dd: tuple(
            reversed(proj.reshape(proj.shape[0], heads, 2 * dd).split(dd, dim=-1))))
        assert not _attention_layer_pinned(c, lw, x, keys, values, position)
    with monkeypatch.context() as mp:   # off-by-one causal mask
        mp.setattr(stack, "visible_keys", lambda p, i: p + i)
        assert not _attention_layer_pinned(c, lw, x, keys, values, position)
    with monkeypatch.context() as mp:   # wrong query-head -> KV-head map
        mp.setattr(stack, "query_kv_head", lambda h, group: h % c.kv_heads)
        assert not _attention_layer_pinned(c, lw, x, keys, values, position)


# ------------------------------------------------------------------ GDN (fused/model.py:219-263)
def _gdn_layer_pinned(c, lw, conv, rec) -> bool:
    """One all-ones token with every in_proj_b row at -8 (beta = sigmoid(-8 * sum of scales *
    128) = 0 to fp32) and in_proj_a rows at 0: the block writes nothing, so head h's core is
    e^(g_h) S0_h^T q_h with q_h the L2-normalised, dk^-1/2-scaled query of key head
    h // (Hv / Hk), g_h = -exp(A_log_h) softplus(dt_bias_h); then the per-head RMS norm
    (weight as is) times SiLU(z_h) and out_proj."""
    kw, vw = c.linear_key_heads * c.linear_key_dim, c.linear_value_heads * c.linear_value_dim
    hv, hk, dk, dv = c.linear_value_heads, c.linear_key_heads, c.linear_key_dim, c.linear_value_dim
    x = torch.ones((1, c.hidden))
    proj = stack.linear(x, lw["mixer_in"])[0]
    qkv, z = proj[:2 * kw + vw], proj[2 * kw + vw:2 * kw + 2 * vw]
    w = lw["conv"][:, 0, :].double()
    conv_out = (conv.double() * w[:, :-1]).sum(-1) + qkv.double() * w[:, -1]
    mixed = conv_out * torch.sigmoid(conv_out)
    g = -torch.exp(lw["a_log"].double()) * torch.nn.functional.softplus(lw["dt_bias"].double())
    gated = torch.empty((hv, dv), dtype=torch.float64)
    for h in range(hv):
        q = mixed[(h // (hv // hk)) * dk:(h // (hv // hk) + 1) * dk]
        q = q / torch.sqrt(q.square().sum() + 1e-6) * dk ** -0.5
        core = math.exp(float(g[h])) * (rec[0, h].double().T @ q)
        zz = z[h * dv:(h + 1) * dv].double()
        gated[h] = core / torch.sqrt(core.square().mean() + c.rms_eps) * lw["gdn_norm"].double() * zz * torch.sigmoid(zz)
    expect = stack.linear(stack.bf16(gated.reshape(1, vw).float()), lw["mixer_out"])
    got = stack.gdn_layer(x, lw, conv, rec, c)["out"]
    return torch.allclose(got, expect, rtol=2e-2, atol=2e-2 * float(expect.abs().max()))


def test_gdn_layer_closed_form(pkg, monkeypatch):
    c = pkg.target.small_config(("linear_attention",))
    w = pkg.target.random_weights(c, seed=41, device="cpu", layout="portable", generate_on="cpu")
    lw = oracle_layer_weights(w.layers[0])
    kw, vw = c.linear_key_heads * c.linear_key_dim, c.linear_value_heads * c.linear_value_dim
    hv = c.linear_value_heads
    packed, scales, group = lw["mixer_in"]
    packed = packed.clone()
    b0 = 2 * kw + 2 * vw
    packed[b0:b0 + hv] = 0x88                        # in_proj_b: every weight -8
    packed[b0 + hv:b0 + 2 * hv] = 0                  # in_proj_a: every weight 0
    lw["mixer_in"] = (packed, scales, group)
    gen = torch.Generator().manual_seed(42)
    conv = torch.randn((c.conv_channels, c.conv_kernel - 1), generator=gen).to(torch.bfloat16)
    rec = torch.randn((1, hv, c.linear_key_dim, c.linear_value_dim), generator=gen)
    assert _gdn_layer_pinned(c, lw, conv, rec)
    with monkeypatch.context() as mp:   # projection read as qkv | b | a | z
        def reordered(proj, cc):
            qkv, b, a, z = proj.split((2 * kw + vw, hv, hv, vw), dim=-1)
            return qkv, z, b, a
        mp.setattr(stack, "split_gdn_projection", reordered)
        assert not _gdn_layer_pinned(c, lw, conv, rec)
    with monkeypatch.context() as mp:   # key heads tiled over the value heads (h % Hk)
        mp.setattr(stack, "key_heads_to_value_heads", lambda m, n: m.repeat(1, n // m.shape[1], 1))
        assert not _gdn_layer_pinned(c, lw, conv, rec)
    with monkeypatch.context() as mp:   # zero-centred gated norm (weight + 1)
        mp.setattr(stack, "gated_norm", lambda core, z, wt, eps: stack.norm(core.float(), wt, eps, 1.0)
                   * torch.nn.functional.silu(z.float()))
        assert not _gdn_layer_pinned(c, lw, conv, rec)
