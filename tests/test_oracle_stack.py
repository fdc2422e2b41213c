"""CPU: pin the decoder-layer oracle (``oracle/stack.py``).

Closed forms for its pieces -- the token-by-token delta rule (beta = 0 only
decays the state; orthonormal keys with beta = 1, g = 0 store the values
exactly), the norm on hand values -- and an invariant of the whole GDN layer:
consuming T tokens at once equals consuming them in two blocks with the conv
window and recurrent state carried between (the layer is a causal recurrence).
A planted mistake (a dropped decay factor) fails the closed form.
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
