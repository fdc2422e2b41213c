"""GPU parity: router logits, top-k routing and the stable expert permutation.

Routing ids, the permutation, its inverse and the segment offsets must be
bit-exact against the oracle on the same fp32 logits; the renormalised
weights agree to fp32 rounding (|dw| <= 2e-6).  Router logits (fp32
accumulation in a different order than the fp64 oracle) agree to 1e-5 of
their max magnitude.
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import metrics, moe as oracle_moe, routing

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden" / "routing_golden.json"


def _check(pkg, device, logits: np.ndarray, k: int):
    r = pkg.ops.route(torch.from_numpy(logits).to(device), k)
    ids, wts = routing.topk(logits, k)
    perm, inv, offsets = routing.permutation(ids, logits.shape[1])
    np.testing.assert_array_equal(r.ids.cpu().numpy(), ids)
    np.testing.assert_array_equal(r.perm.cpu().numpy(), perm)
    np.testing.assert_array_equal(r.inv.cpu().numpy(), inv)
    np.testing.assert_array_equal(r.offsets.cpu().numpy(), offsets)
    np.testing.assert_allclose(r.weights.cpu().numpy(), wts, rtol=0, atol=2e-6)


def _decode(v):
    return {"-inf": -np.inf, "-0.0": -0.0}.get(v, v) if isinstance(v, str) else v


def test_route_golden_vectors(pkg, device):
    for case in json.loads(GOLDEN.read_text()):
        k, e = case["k"], case["experts"]
        logits = np.array([[_decode(v) for v in row] for row in case["logits"]], dtype=np.float32).reshape(-1, e)
        print(f"golden route T={logits.shape[0]} E={e} k={k}", flush=True)
        r = pkg.ops.route(torch.from_numpy(logits).to(device), k)
        np.testing.assert_array_equal(r.ids.cpu().numpy().reshape(-1, k), np.array(case["ids"], np.int32).reshape(-1, k))
        np.testing.assert_array_equal(r.perm.cpu().numpy(), np.array(case["perm"], np.int32))
        np.testing.assert_array_equal(r.inv.cpu().numpy(), np.array(case["inv"], np.int32))
        np.testing.assert_array_equal(r.offsets.cpu().numpy(), np.array(case["offsets"], np.int32))
        np.testing.assert_allclose(r.weights.cpu().numpy().reshape(-1, k),
                                   np.array(case["weights"], np.float32).reshape(-1, k), rtol=0, atol=2e-6)


@pytest.mark.parametrize("tokens,experts,k", [
    (1, 256, 8), (16, 256, 8), (32, 256, 8),                      # single-workgroup path (T <= 32)
    (128, 256, 8), (256, 256, 8), (257, 256, 8), (2048, 256, 8),  # multi-workgroup, experts counted in the permutation launch
    (64, 1024, 64), (300, 1000, 3), (40, 7, 7), (33, 64, 1),
    (2100, 256, 8), (4096, 64, 6),                                # T*k > 16384: the separate count launch
])
def test_route_random(pkg, device, tokens, experts, k):
    print(f"route T={tokens} E={experts} k={k}", flush=True)
    rng = np.random.default_rng(tokens * 1000 + experts + k)
    _check(pkg, device, rng.standard_normal((tokens, experts)).astype(np.float32), k)


@pytest.mark.parametrize("tokens", [16, 600])
def test_route_ties(pkg, device, tokens):
    """Coarse-grid logits: many exact ties, including at the k-th position."""
    print(f"route ties T={tokens}", flush=True)
    rng = np.random.default_rng(tokens)
    logits = (rng.integers(-24, 24, (tokens, 256)) / 8.0).astype(np.float32)
    logits[0, :] = 0.0
    logits[1, ::2] = -0.0
    _check(pkg, device, logits, 8)


def test_route_skewed(pkg, device):
    """16 hot experts take ~half of 1024 assignments (the batch-of-8-blocks workload)."""
    layer = pkg.synthetic.moe_layer(128, seed=2, banks=False)
    bias = pkg.synthetic.skewed_bias(layer)
    logits = (layer.hidden.float() @ layer.router_weight.float().T + bias).numpy().astype(np.float32)
    _check(pkg, device, logits, 8)


@pytest.mark.parametrize("tokens", [1, 16, 128, 2048])
def test_router_logits(pkg, device, tokens):
    print(f"router T={tokens}", flush=True)
    layer = pkg.synthetic.moe_layer(tokens, seed=tokens, banks=False)
    got = pkg.ops.router_logits(layer.hidden.to(device), layer.router_weight.to(device)).cpu()
    golden = oracle_moe.router_logits(layer.hidden, layer.router_weight)
    report = metrics.compare(got, golden)
    assert report["max_rel"] <= 1e-5, report


@pytest.mark.parametrize("tokens,experts,hidden", [
    # 16 x 16 tiles (T < 1024, or H outside {512, 1024, 2048})
    (100, 100, 1024), (65, 200, 768), (300, 200, 512), (64, 64, 2048), (1000, 256, 1024),
    (1024, 64, 768),
    # 32 x 64 tiles (T >= 1024, H in {512, 1024, 2048}), taken in groups of 8 token tiles
    (1100, 200, 512),     # 35 token tiles (the last holds 12 rows): 4 whole groups and one of 3; 4 expert tiles (the last 8 experts)
    (1030, 256, 1024),    # 33 token tiles (the last holds 6 rows): 4 whole groups and one of 1
    (2048, 100, 2048),    # 64 token tiles in whole groups; 2 expert tiles (the last 36 experts)
])
def test_router_logits_ragged_tiles(pkg, device, tokens, experts, hidden):
    """Token and expert counts that leave partial router tiles and partial groups of token tiles."""
    print(f"router T={tokens} E={experts} H={hidden}", flush=True)
    gen = torch.Generator().manual_seed(tokens + experts)
    x = torch.randn((tokens, hidden), generator=gen).to(torch.bfloat16)
    w = (0.02 * torch.randn((experts, hidden), generator=gen)).to(torch.bfloat16)
    got = pkg.ops.router_logits(x.to(device), w.to(device)).cpu()
    golden = oracle_moe.router_logits(x, w)
    report = metrics.compare(got, golden)
    assert report["max_rel"] <= 1e-5, report
