"""GPU: the tiled weight layout.

``dflash_w4_to_tiled`` must reproduce the oracle's permutation (``oracle.w4.to_tiled``)
byte for byte, and every expert kernel that reads tiled banks (verify block,
streaming, prefill tile) must give the same bits as on the portable banks it
came from -- the layout changes where bytes live, not what is computed -- and
meet the oracle's bar.  Paths whose kernels read portable rows only refuse
tiled banks before launching anything.
"""
import numpy as np
import pytest
import torch

from oracle import metrics, moe as oracle_moe, w4

pytestmark = pytest.mark.gpu
TOL = 1e-2


@pytest.mark.parametrize("experts,rows,cols,group,scale_dtype", [
    (1, 512, 2048, 128, torch.bfloat16),
    (3, 64, 512, 128, torch.float32),
    (2, 48, 1024, 256, torch.bfloat16),
    (5, 2048, 512, 128, torch.bfloat16),
])
def test_to_tiled_matches_oracle(pkg, device, experts, rows, cols, group, scale_dtype):
    print(f"to_tiled E={experts} N={rows} K={cols} g={group} {scale_dtype}", flush=True)
    gen = torch.Generator().manual_seed(rows + cols)
    shape = (experts, rows, cols) if experts > 1 else (rows, cols)
    w = pkg.synthetic.int4_weight(gen, shape, group, scale_dtype)
    t = w.to(device).tiled()
    assert t.layout == "tiled" and t.packed.shape == w.packed.shape and t.scales.shape == w.scales.shape
    ref_p, ref_s = w4.to_tiled(w.packed.numpy(), w.scales.view(torch.int16 if scale_dtype == torch.bfloat16
                                                                 else torch.int32).numpy())
    np.testing.assert_array_equal(t.packed.cpu().numpy(), ref_p)
    got_s = t.scales.cpu().view(torch.int16 if scale_dtype == torch.bfloat16 else torch.int32).numpy()
    np.testing.assert_array_equal(got_s, ref_s)


@pytest.mark.parametrize("m,n,k,group,scale_dtype", [
    (16, 512, 2048, 128, torch.bfloat16),   # small-block kernel
    (5, 96, 1024, 128, torch.float32),
    (32, 160, 4096, 256, torch.float32),    # small-block kernel: two row tiles, 4 k-blocks a wave, g256
    (16, 12384, 2048, 256, torch.float32),  # its streaming form, g256 fp32 scales
    (7, 40960, 2048, 128, torch.bfloat16),  # staging verify kernel (linear mode)
    (64, 256, 2048, 128, torch.bfloat16),   # streaming kernel
    (48, 64, 512, 128, torch.float32),
])
def test_qlinear_tiled_equals_portable(pkg, device, m, n, k, group, scale_dtype):
    print(f"qlinear tiled m={m} n={n} k={k} g={group} {scale_dtype}", flush=True)
    gen = torch.Generator().manual_seed(m + n + k)
    x = torch.randn((m, k), generator=gen).to(torch.bfloat16)
    w = pkg.synthetic.int4_weight(gen, (n, k), group, scale_dtype)
    wd = w.to(device)
    y_p = pkg.ops.qlinear(x.to(device), wd)
    y_t = pkg.ops.qlinear(x.to(device), wd.tiled())
    assert torch.equal(y_p, y_t)
    report = metrics.compare(y_t.cpu(), w4.qlinear(x, w.packed.numpy(), w.scales, group))
    assert report["max_rel"] <= TOL, report


def _banks(pkg, layer, device, tiled):
    gu, dn = layer.gate_up.to(device), layer.down.to(device)
    sh = None
    if layer.shared is not None:
        s = layer.shared
        sh = pkg.SharedExpert(s.gate_up.to(device), s.down.to(device), s.gate_weight.to(device))
    if tiled:
        gu, dn = gu.tiled(), dn.tiled()
        sh = sh.tiled() if sh is not None else None
    return gu, dn, sh


@pytest.mark.parametrize("tokens,experts,k,hidden,inter,group,scale_dtype,skew", [
    (16, 256, 8, 2048, 512, 128, torch.bfloat16, False),   # the verify block (routing in the gate/up launch)
    (5, 8, 2, 512, 512, 128, torch.bfloat16, False),
    (32, 64, 8, 2048, 512, 128, torch.float32, False),
    (128, 256, 8, 2048, 512, 128, torch.bfloat16, True),   # streaming kernel, skewed routing
    (300, 16, 4, 1024, 512, 128, torch.float32, False),    # prefill tile kernel, fp32 scales
    (256, 8, 2, 2048, 512, 256, torch.bfloat16, False),    # prefill tile kernel, group 256
    (16, 256, 8, 2048, 512, 256, torch.float32, False),   # verify block, group 256 fp32 scales
])
def test_moe_tiled_equals_portable(pkg, device, tokens, experts, k, hidden, inter, group, scale_dtype, skew):
    print(f"moe tiled T={tokens} E={experts} k={k} H={hidden} I={inter} g={group} {scale_dtype} skew={skew}",
          flush=True)
    layer = pkg.synthetic.moe_layer(tokens, hidden=hidden, inter=inter, experts=experts, group_size=group,
                                    seed=tokens + 3, shared=True, scale_dtype=scale_dtype)
    x = layer.hidden.to(device)
    rw = layer.router_weight.to(device)
    logits = pkg.ops.router_logits(x, rw)
    if skew:
        logits = (logits + pkg.synthetic.skewed_bias(layer).to(device)).contiguous()
    outs = []
    for tiled in (False, True):
        gu, dn, sh = _banks(pkg, layer, device, tiled)
        out, r, _ = pkg.ops.moe_w4a16(x, gu, dn, top_k=k, router_logits=logits, shared=sh, return_routing=True)
        outs.append((out, r))
    (out_p, r_p), (out_t, r_t) = outs
    assert torch.equal(out_p, out_t)
    assert torch.equal(r_p.perm, r_t.perm) and torch.equal(r_p.ids, r_t.ids)
    s = layer.shared
    golden = oracle_moe.moe(layer.hidden, logits.cpu().numpy(), k, (layer.gate_up.packed, layer.gate_up.scales),
                            (layer.down.packed, layer.down.scales), group,
                            shared=((s.gate_up.packed, s.gate_up.scales), (s.down.packed, s.down.scales),
                                    s.gate_weight))
    np.testing.assert_array_equal(r_t.ids.cpu().numpy(), golden["ids"])
    report = metrics.compare(out_t.cpu(), golden["out_f32"])
    print(f"  report={report}", flush=True)
    assert report["max_rel"] <= TOL, report


def test_tiled_on_a_portable_only_path_raises(pkg, device):
    """Group 256 with 33 rows has no tiled-reading kernel: refused with a message, nothing launched."""
    gen = torch.Generator().manual_seed(2)
    w = pkg.synthetic.int4_weight(gen, (64, 1024), 256).to(device).tiled()
    x = torch.randn((33, 1024), generator=gen).to(torch.bfloat16).to(device)
    with pytest.raises(pkg._lib.DflashError, match="tiled"):
        pkg.ops.qlinear(x, w)
