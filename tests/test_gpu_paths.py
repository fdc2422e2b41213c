"""GPU parity, one case per kernel path that no workload shape reaches.

The library picks the expert/linear kernel from the shape (``csrc/api.hip``):

* ``w4_verify`` -- T <= 32 tokens (m <= 32 rows for qlinear; 16 per launch at K = 4096)
  whose LDS plan fits (``verify_layout``);
* ``w4_tile``   -- long prefill, T*k >= 16*E;
* ``w4_stream`` -- everything else with K in {512, 1024, 2048} and group 128, including
  blocks of T <= 32 whose verify LDS plan does not fit (large k and E);
* ``w4_gemm``   -- the per-wave fallback for the rest: K outside {512, 1024, 2048}
  (e.g. 4096) or group 256 above 32 rows.  It reads the portable layout only.

Each case below is chosen so its path is the one named, and is checked against the
oracle at the usual bar (max|y - r| / max|r| <= 1e-2, routing bit-exact).
"""
import numpy as np
import pytest
import torch

from oracle import metrics, moe as oracle_moe, w4

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _moe_case(pkg, device, tokens, experts, k, hidden, inter, group, seed):
    layer = pkg.synthetic.moe_layer(tokens, hidden=hidden, inter=inter, experts=experts, group_size=group,
                                    seed=seed, shared=True)
    s = layer.shared
    sh = pkg.SharedExpert(s.gate_up.to(device), s.down.to(device), s.gate_weight.to(device))
    out, r, logits = pkg.ops.moe_w4a16(layer.hidden.to(device), layer.gate_up.to(device), layer.down.to(device),
                                       top_k=k, router_weight=layer.router_weight.to(device), shared=sh,
                                       return_routing=True)
    golden = oracle_moe.moe(layer.hidden, logits.cpu().numpy(), k, (layer.gate_up.packed, layer.gate_up.scales),
                            (layer.down.packed, layer.down.scales), group,
                            shared=((s.gate_up.packed, s.gate_up.scales), (s.down.packed, s.down.scales),
                                    s.gate_weight))
    np.testing.assert_array_equal(r.ids.cpu().numpy(), golden["ids"])
    np.testing.assert_array_equal(r.perm.cpu().numpy(), golden["perm"])
    np.testing.assert_array_equal(r.offsets.cpu().numpy(), golden["offsets"])
    report = metrics.compare(out.cpu(), golden["out_f32"])
    print(f"  report={report}", flush=True)
    assert report["max_rel"] <= TOL and report["cosine"] > 0.9999, report


def test_stream_kernel_takes_small_blocks_the_verify_plan_cannot_hold(pkg, device):
    """T=32, E=128, k=64 at H=2048: the verify gate/up plan (32 x rows of x, 258 pass
    descriptors, 2048 token slots) exceeds the LDS, so both GEMMs run on w4_stream with
    32-row passes and the multi-workgroup routing kernels."""
    print("path w4_stream: moe T=32 E=128 k=64 H=2048", flush=True)
    _moe_case(pkg, device, 32, 128, 64, 2048, 512, 128, seed=71)


def test_per_wave_fallback_group_256_moe(pkg, device):
    """T=64, E=64, k=4 with group 256: neither the verify (T > 32), tile (T*k < 16*E) nor the
    streaming kernel (group 128 only) applies, so both GEMMs run on w4_gemm."""
    print("path w4_gemm: moe T=64 E=64 k=4 g=256", flush=True)
    _moe_case(pkg, device, 64, 64, 4, 1024, 512, 256, seed=72)


@pytest.mark.parametrize("m,n,k,group", [(64, 256, 4096, 128), (40, 128, 2048, 256)])
def test_per_wave_fallback_qlinear(pkg, device, m, n, k, group):
    """qlinear above 32 rows at K = 4096 (the output projections of a prefill) or group 256:
    w4_gemm on portable weights."""
    print(f"path w4_gemm: qlinear m={m} n={n} k={k} g={group}", flush=True)
    gen = torch.Generator().manual_seed(m + n + k)
    x = torch.randn((m, k), generator=gen).to(torch.bfloat16)
    weight = pkg.synthetic.int4_weight(gen, (n, k), group)
    y = pkg.ops.qlinear(x.to(device), weight.to(device)).cpu()
    report = metrics.compare(y, w4.qlinear(x, weight.packed.numpy(), weight.scales, group))
    assert report["max_rel"] <= TOL and report["cosine"] > 0.9999, report
