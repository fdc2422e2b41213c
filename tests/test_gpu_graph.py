"""GPU: the kernels are HIP-graph capturable (no memset nodes, no allocation, no sync).

Each graph is replayed several times with unrelated eager work and
synchronisations between replays; every replay must equal the eager result
bit for bit (the combine is deterministic).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _replays_match(fn, eager, replays=4):
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        out = fn()
    for i in range(replays):
        out.zero_()
        scratch = torch.randn(1 << 20, device=out.device) * (i + 1)  # unrelated eager work between replays
        scratch.sum().item()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i} differs from the eager result"


def test_moe_layer_graph_replay(pkg, device):
    layer = pkg.synthetic.moe_layer(16, seed=21)
    sh = layer.shared
    shared = pkg.SharedExpert(sh.gate_up.to(device), sh.down.to(device), sh.gate_weight.to(device))
    gu, dn = layer.gate_up.to(device), layer.down.to(device)
    x, rw = layer.hidden.to(device), layer.router_weight.to(device)
    fn = lambda: pkg.ops.moe_w4a16(x, gu, dn, top_k=8, router_weight=rw, shared=shared)  # noqa: E731
    eager = fn()
    torch.cuda.synchronize()
    _replays_match(fn, eager)


def test_moe_prefill_graph_replay(pkg, device):
    """The multi-workgroup routing path (zero kernel + top-k + permute) under a graph."""
    layer = pkg.synthetic.moe_layer(600, hidden=512, inter=512, experts=64, seed=22)
    gu, dn = layer.gate_up.to(device), layer.down.to(device)
    x, rw = layer.hidden.to(device), layer.router_weight.to(device)
    fn = lambda: pkg.ops.moe_w4a16(x, gu, dn, top_k=8, router_weight=rw)  # noqa: E731
    eager = fn()
    torch.cuda.synchronize()
    _replays_match(fn, eager)


def test_qlinear_graph_replay(pkg, device):
    gen = torch.Generator().manual_seed(23)
    x = torch.randn((16, 2048), generator=gen).to(torch.bfloat16).to(device)
    w = pkg.synthetic.int4_weight(gen, (512, 2048)).to(device)
    fn = lambda: pkg.ops.qlinear(x, w)  # noqa: E731
    eager = fn()
    torch.cuda.synchronize()
    _replays_match(fn, eager)
