"""GPU: the no-allocation MoE entry point (``dflash_moe_w4a16_noalloc``).

Its scratch is a static device array of the library instead of a caller
workspace; everything else is ``dflash_moe_w4a16``, except that the static
array has no room for the opt-in split-K down's partial rows, so it always runs
the down GEMM as a launch of its own.  Two calls in a row -- the second with a
smaller block, so stale scratch from the first is present -- must each give the
same routing and logits as the workspace entry point on the same inputs, the
same output bits as that entry point with the split-K down off (its default),
and an output within the oracle bar of its split-K output; a layer that needs
more scratch than the array holds is refused before anything is launched.
"""
import numpy as np
import pytest
import torch

from oracle import metrics, moe as oracle_moe

pytestmark = pytest.mark.gpu


def _layer(pkg, device, tokens, seed, experts=256, hidden=2048):
    layer = pkg.synthetic.moe_layer(tokens, hidden=hidden, experts=experts, seed=seed)
    s = layer.shared
    sh = pkg.SharedExpert(s.gate_up.to(device), s.down.to(device), s.gate_weight.to(device)).tiled()
    return layer, layer.gate_up.to(device).tiled(), layer.down.to(device).tiled(), sh


@pytest.mark.parametrize("given_logits", [False, True])
def test_noalloc_equals_workspace_entry_on_two_calls(pkg, device, given_logits):
    for tokens, seed in ((16, 0), (5, 3)):
        print(f"noalloc T={tokens} seed={seed} given_logits={given_logits}", flush=True)
        layer, gu, dn, sh = _layer(pkg, device, tokens, seed)
        x, rw = layer.hidden.to(device), layer.router_weight.to(device)
        kw = {"router_logits": pkg.ops.router_logits(x, rw)} if given_logits else {"router_weight": rw}
        with pkg.ops.split_down(False):
            two = pkg.ops.moe_w4a16(x, gu, dn, top_k=8, shared=sh, **kw)
        with pkg.ops.split_down(True):
            ref, r_ref, lg_ref = pkg.ops.moe_w4a16(x, gu, dn, top_k=8, shared=sh, return_routing=True, **kw)
        out, r, lg = pkg.ops.moe_w4a16_noalloc(x, gu, dn, top_k=8, shared=sh, **kw)
        torch.cuda.synchronize()
        assert torch.equal(out, two)
        assert metrics.compare(out.cpu(), ref.float().cpu().numpy())["max_rel"] <= 1e-2
        for a, b in zip(r, r_ref):
            assert torch.equal(a, b)
        assert torch.equal(lg, lg_ref)
        if tokens == 16:   # and the oracle's bar, once
            ogu = (layer.gate_up.packed, layer.gate_up.scales)
            odn = (layer.down.packed, layer.down.scales)
            s = layer.shared
            osh = ((s.gate_up.packed, s.gate_up.scales), (s.down.packed, s.down.scales), s.gate_weight)
            golden = oracle_moe.moe(layer.hidden, lg.cpu().numpy(), 8, ogu, odn, 128, shared=osh)
            np.testing.assert_array_equal(r.ids.cpu().numpy(), golden["ids"])
            assert metrics.compare(out.cpu(), golden["out_f32"])["max_rel"] <= 1e-2


def test_noalloc_refuses_layers_above_its_scratch(pkg, device):
    layer, gu, dn, sh = _layer(pkg, device, 512, 9, experts=64, hidden=512)
    need = pkg.ops.moe_workspace_bytes(512, 512, 512, 64, 8, 128, True)
    assert need > pkg.ops.NOALLOC_SCRATCH_BYTES
    with pytest.raises(pkg._lib.DflashError, match="scratch"):
        pkg.ops.moe_w4a16_noalloc(layer.hidden.to(device), gu, dn, top_k=8, shared=sh,
                                  router_weight=layer.router_weight.to(device))
