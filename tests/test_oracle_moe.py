"""CPU: pin the MoE oracle (expert FFN, combine, shared expert).

Checks: the golden MoE vector of the pure-Python brute force (fp64 loops,
bf16 rounding of the SiLU*up intermediate), an independent dense formulation
(every token through every expert, masked by a one-hot routing matrix),
the E=1/k=1 reduction to a dense SwiGLU MLP, a zero-weight expert contributing
nothing, and the bf16 reference-order restatement staying within bf16 noise.
"""
import json
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

from oracle import metrics, moe, routing, w4

GOLDEN = json.loads((Path(__file__).resolve().parent / "golden" / "moe_golden.json").read_text())


def _golden_inputs():
    g = GOLDEN
    t = lambda v, dt=torch.float32: torch.tensor(v, dtype=dt)  # noqa: E731
    x = t(g["x"]).to(torch.bfloat16)
    gu = (t(g["gate_up_packed"], torch.uint8), t(g["gate_up_scales"]))
    dn = (t(g["down_packed"], torch.uint8), t(g["down_scales"]))
    sh = ((t(g["shared_gate_up_packed"], torch.uint8), t(g["shared_gate_up_scales"])),
          (t(g["shared_down_packed"], torch.uint8), t(g["shared_down_scales"])), t(g["shared_gate"]).to(torch.bfloat16))
    return x, np.array(g["logits"], np.float32), gu, dn, sh


def test_golden_vector():
    x, logits, gu, dn, sh = _golden_inputs()
    routed = moe.moe(x, logits, GOLDEN["k"], gu, dn, GOLDEN["group"])
    total = moe.moe(x, logits, GOLDEN["k"], gu, dn, GOLDEN["group"], shared=sh)
    np.testing.assert_array_equal(routed["ids"], np.array(GOLDEN["ids"], np.int32))
    # The golden sums in fp64, the oracle in fp32 over inner dimensions of 16: what separates
    # them is a few fp32 roundings (2^-24 ~ 6e-8 each; 5e-8 and 7e-8 observed).  1e-6 leaves
    # that room and nothing more: a bf16 combine or a bf16 expert output (2^-9 ~ 2e-3) fails it.
    assert metrics.compare(routed["out_f32"], np.array(GOLDEN["out_routed"]))["max_rel"] < 1e-6
    assert metrics.compare(total["out_f32"], np.array(GOLDEN["out_total"]))["max_rel"] < 1e-6


def test_golden_bar_rejects_a_bf16_combine():
    """Plant: the same layer with each expert output rounded to bf16 before the weighted sum
    misses the golden by far more than the bar above allows."""
    x, logits, gu, dn, _ = _golden_inputs()
    k, g = GOLDEN["k"], GOLDEN["group"]
    ids, wts = routing.topk(logits, k)
    xf = x.to(torch.float32)
    out = torch.zeros_like(xf)
    for t in range(xf.shape[0]):
        for slot in range(k):
            e = int(ids[t, slot])
            gate, up = (xf[t] @ _deq((gu[0][e:e + 1], gu[1][e:e + 1]), g)[0].T).chunk(2)
            h = (F.silu(gate) * up).to(torch.bfloat16).to(torch.float32)
            y = (h @ _deq((dn[0][e:e + 1], dn[1][e:e + 1]), g)[0].T).to(torch.bfloat16).to(torch.float32)
            out[t] += float(wts[t, slot]) * y
    assert metrics.compare(out, np.array(GOLDEN["out_routed"]))["max_rel"] > 1e-5


def _random_layer(seed, t=16, h=256, i=128, e=8, k=2, g=128):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn((t, h), generator=gen).to(torch.bfloat16)
    gu = (torch.randint(0, 256, (e, 2 * i, h // 2), dtype=torch.uint8, generator=gen),
          (torch.rand((e, 2 * i, h // g), generator=gen) * 0.015 + 0.005).to(torch.bfloat16))
    dn = (torch.randint(0, 256, (e, h, i // 2), dtype=torch.uint8, generator=gen),
          (torch.rand((e, h, i // g), generator=gen) * 0.015 + 0.005).to(torch.bfloat16))
    logits = torch.randn((t, e), generator=gen).numpy()
    return x, logits, gu, dn


def _deq(bank, g):
    return torch.from_numpy(w4.dequantize(bank[0].numpy(), bank[1], g))


def test_matches_dense_masked_formulation():
    x, logits, gu, dn = _random_layer(3)
    out = moe.moe(x, logits, 2, gu, dn, 128)
    ids, wts = routing.topk(logits, 2)
    gate_up, down = _deq(gu, 128), _deq(dn, 128)
    xf = x.float()
    dense = torch.zeros_like(xf)
    for e in range(gate_up.shape[0]):  # all experts, all tokens, weight 0 when not routed
        g, u = (xf @ gate_up[e].T).chunk(2, dim=-1)
        y = (F.silu(g) * u).to(torch.bfloat16).float() @ down[e].T
        mask = torch.from_numpy(((ids == e) * wts).sum(-1))
        dense += mask[:, None] * y
    assert metrics.compare(out["out_f32"], dense)["max_rel"] < 1e-5


def test_single_expert_reduces_to_dense_swiglu():
    x, _, gu, dn = _random_layer(4, e=1, k=1)
    logits = np.zeros((x.shape[0], 1), np.float32)
    out = moe.moe(x, logits, 1, gu, dn, 128)
    gate_up, down = _deq(gu, 128)[0], _deq(dn, 128)[0]
    g, u = (x.float() @ gate_up.T).chunk(2, dim=-1)
    ref = (F.silu(g) * u).to(torch.bfloat16).float() @ down.T
    assert metrics.compare(out["out_f32"], ref)["max_rel"] < 1e-6
    np.testing.assert_allclose(out["weights"], 1.0)


def test_zero_weight_expert_contributes_nothing():
    x, logits, gu, dn = _random_layer(5, e=4, k=4)
    logits[:, 3] = -np.inf  # selected (k == E) but with weight exp(-inf) = 0
    full = moe.moe(x, logits, 4, gu, dn, 128)
    assert np.all(full["weights"][:, 3] == 0)
    trimmed_logits = logits[:, :3].copy()
    trimmed = moe.moe(x, trimmed_logits, 3, (gu[0][:3], gu[1][:3]), (dn[0][:3], dn[1][:3]), 128)
    assert metrics.compare(full["out_f32"], trimmed["out_f32"])["max_rel"] < 1e-6


def test_reference_bf16_order_is_close():
    x, logits, gu, dn = _random_layer(6, e=8, k=2)
    golden = moe.moe(x, logits, 2, gu, dn, 128)["out_f32"]
    ref = moe.moe_reference_order(x, logits, 2, _deq(gu, 128).to(torch.bfloat16), _deq(dn, 128).to(torch.bfloat16))
    assert metrics.compare(ref, golden)["max_rel"] < 2e-2


def test_dense_baseline_form_matches():
    x, logits, gu, dn = _random_layer(7)
    golden = moe.moe(x, logits, 2, gu, dn, 128, round_hidden=False)["out_f32"]
    dense = moe.moe_dense(x, logits, 2, _deq(gu, 128), _deq(dn, 128))
    assert metrics.compare(dense, golden)["max_rel"] < 1e-2


def test_dense_baseline_with_shared_expert_and_on_the_fly_dequant():
    """The CPU baseline's two timed forms (pre-dequantised bf16 banks; hit experts dequantised
    inside the call) both give the golden layer, shared expert included."""
    x, logits, gu, dn = _random_layer(8)
    gen = torch.Generator().manual_seed(9)
    sgu = (torch.randint(0, 256, (256, 128), dtype=torch.uint8, generator=gen),
           (torch.rand((256, 2), generator=gen) * 0.015 + 0.005).to(torch.bfloat16))
    sdn = (torch.randint(0, 256, (256, 64), dtype=torch.uint8, generator=gen),
           (torch.rand((256, 1), generator=gen) * 0.015 + 0.005).to(torch.bfloat16))
    sgate = (torch.randn(256, generator=gen) * 0.02).to(torch.bfloat16)
    golden = moe.moe(x, logits, 2, gu, dn, 128, shared=(sgu, sdn, sgate))["out_f32"]
    dense_shared = (w4.dequantize_torch(*sgu, 128), w4.dequantize_torch(*sdn, 128), sgate)
    pre = moe.moe_dense(x, logits, 2, _deq(gu, 128).to(torch.bfloat16), _deq(dn, 128).to(torch.bfloat16),
                        shared=dense_shared)
    fly = moe.moe_dense(x, logits, 2, None, None, shared=dense_shared,
                        dequantize=lambda e: (w4.dequantize_torch(gu[0][e], gu[1][e], 128),
                                              w4.dequantize_torch(dn[0][e], dn[1][e], 128)))
    assert torch.equal(pre, fly)
    assert metrics.compare(pre, golden)["max_rel"] < 2e-2


def test_metrics_definitions():
    a = np.array([1.0, -2.0, 3.0])
    r = metrics.compare(a, a)
    assert r["max_rel"] == 0 and r["cosine"] == 1.0 and r["rel_l2"] == 0
    r = metrics.compare(a + np.array([0.0, 0.03, 0.0]), a)
    assert abs(r["max_rel"] - 0.01) < 1e-12
    assert metrics.compare(np.zeros(3), np.zeros(3))["cosine"] == 1.0
