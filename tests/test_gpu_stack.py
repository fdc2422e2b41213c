"""GPU: the verify stack (``target.TargetModel``) -- qlinear and MoE on the HIP kernels, the
rest in PyTorch-ROCm -- against the decoder-layer oracle (``oracle/stack.py``).

Slice check: a reduced-width two-layer target (one GDN layer, one attention layer, H=512,
16 experts top-4 + shared, vocab 1024, all W4 g128 tiled) runs a 16-token block over a
40-token context.  Each layer is checked on the GPU's own input to it (teacher forcing,
so layer 2 is not judged on layer 1's rounding): the residual after the layer within the
bar max|y - r| / max|r| <= 1e-2, the MoE routing bit-exact against the oracle's top-k of
the GPU's router logits, the recurrent state after every accepted prefix (commit) within
1e-2 of the oracle's token-by-token states, the KV rows written in place.
"""
import numpy as np
import pytest
import torch

from oracle import metrics, routing as oracle_routing, stack
from stack_util import oracle_layer_state, oracle_layer_weights

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _slice(pkg, device, seed=3, context=40):
    c = pkg.target.small_config()
    host = pkg.target.random_weights(c, seed=seed, device="cpu", layout="portable", generate_on="cpu")
    w = pkg.target.to_device(host, device, layout="tiled")
    model = pkg.target.TargetModel(w, capacity=96)
    state = model.synthetic_context(context, seed=seed + 1)
    return c, host, model, state


def test_stack_slice_layers_match_oracle(pkg, device):
    print("stack slice: GDN + attention, T=16 over 40 tokens", flush=True)
    c, host, model, state = _slice(pkg, device)
    ids = torch.randint(0, c.vocab, (16,), generator=torch.Generator().manual_seed(5))
    hidden = model.embed(ids.to(device))
    before = [oracle_layer_state(state, i) for i in range(c.layers)]
    position = state.position
    for i in range(c.layers):
        trace = {}
        x_in = hidden
        hidden, pending = model.layer(i, hidden, state, trace=trace)
        lw = oracle_layer_weights(host.layers[i])
        logits = pkg.ops.router_logits(trace["moe_in"], model.w.layers[i].router).cpu().numpy()
        ref = stack.decoder_layer(x_in.cpu(), lw, before[i], position, c, moe_logits=logits)
        rep_mid = metrics.compare(trace["mid"].cpu(), ref["mid"])
        rep = metrics.compare(hidden.cpu(), ref["hidden"])
        print(f"  layer {i} {host.layers[i].kind}: mixer {rep_mid} layer {rep}", flush=True)
        assert rep_mid["max_rel"] <= TOL and rep["max_rel"] <= TOL, (rep_mid, rep)
        lwg = model.w.layers[i]
        _, r, lg = pkg.ops.moe_w4a16(trace["moe_in"], lwg.gate_up, lwg.down, top_k=c.top_k, router_weight=lwg.router,
                                     shared=lwg.shared, return_routing=True)
        ids_ref, _ = oracle_routing.topk(lg.cpu().numpy(), c.top_k)
        np.testing.assert_array_equal(r.ids.cpu().numpy(), ids_ref)
        if host.layers[i].kind == "full_attention":
            got_k = state.keys[i][0, :, position:position + 16].float().cpu()
            assert metrics.compare(got_k, ref["mixer"]["keys"])["max_rel"] <= TOL
            got_v = state.values[i][0, :, position:position + 16].float().cpu()
            assert metrics.compare(got_v, ref["mixer"]["values"])["max_rel"] <= TOL
        else:
            for j in (0, 1, 9, 16):           # the state after every accepted prefix length
                trial = state.clone()
                gdn = [None] * c.layers
                gdn[i] = pending
                model.commit(trial, pkg.target.Pending(position, 16, gdn), j)
                got = trial.recurrent[i][0].cpu()
                r = metrics.compare(got, ref["mixer"]["states"][j].float())
                assert r["max_rel"] <= TOL, (j, r)
                want_conv = ref["mixer"]["window"][:, j:j + c.conv_kernel - 1]
                assert metrics.compare(trial.conv[i][0].float().cpu(), want_conv)["max_rel"] <= TOL, j


def test_stack_commit_equals_the_shorter_block(pkg, device):
    """Committing j tokens of a 16-token block gives the state a j-token block gives, and the
    first j outputs agree (the forward is causal)."""
    c, _, model, state = _slice(pkg, device, seed=11)
    ids = torch.randint(0, c.vocab, (16,), generator=torch.Generator().manual_seed(6)).to(device)
    full = model.forward(ids, state)
    for j in (1, 7, 16):
        print(f"stack commit j={j}", flush=True)
        a, b = state.clone(), state.clone()
        model.commit(a, full.pending, j)
        short = model.forward(ids[:j], b)
        model.commit(b, short.pending, j)
        assert a.position == b.position == state.position + j
        for i in range(c.layers):
            if a.recurrent[i] is not None:
                assert metrics.compare(a.recurrent[i].cpu(), b.recurrent[i].cpu())["max_rel"] <= 1e-3
                assert torch.equal(a.conv[i], b.conv[i])
            else:
                assert torch.equal(a.keys[i][:, :, :a.position], b.keys[i][:, :, :b.position])
        assert metrics.compare(full.hidden[:j].cpu(), short.hidden.cpu())["max_rel"] <= TOL
    nothing = state.clone()
    model.commit(nothing, full.pending, 0)
    assert nothing.position == state.position and torch.equal(nothing.recurrent[0], state.recurrent[0])
    with pytest.raises(ValueError):
        model.commit(state.clone(), full.pending, 17)


@pytest.mark.timeout(300)
def test_full_target_verify_block(pkg, device):
    """The 40-layer target (30 GDN + 10 attention, 256 experts top-8 + shared, vocab 248320) runs
    a 16-token verify block over a 4096-token context: finite outputs, one top-1 per token, and
    the features of the drafter's eight layers."""
    print("stack full: 40 layers, T=16 over 4096", flush=True)
    c = pkg.plan.TargetConfig()
    w = pkg.target.random_weights(c, seed=0, device=device)
    model = pkg.target.TargetModel(w, capacity=4096 + 32, feature_layers=pkg.target.DRAFT_FEATURE_LAYERS)
    state = model.synthetic_context(4096, seed=1)
    ids = torch.randint(0, c.vocab, (16,), device=device)
    out = model.forward(ids, state)
    torch.cuda.synchronize()
    assert tuple(out.hidden.shape) == (16, 2048) and bool(torch.isfinite(out.hidden).all())
    assert tuple(out.top1.shape) == (16,) and out.top1.dtype == torch.int32
    assert int(out.top1.min()) >= 0 and int(out.top1.max()) < c.vocab
    assert tuple(out.features.shape) == (16, 8 * 2048)
    model.commit(state, out.pending, 16)
    assert state.position == 4096 + 16
