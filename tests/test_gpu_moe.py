"""GPU parity: the routed-MoE layer (router, routing, gate/up + SiLU*up, down, combine).

Routing is compared bit-exactly: the oracle routes on the very fp32 logits
the GPU produced (fp32 GEMV accumulation order is not part of the contract).
The bf16 output must satisfy max|y - r| / max|r| <= 1e-2 against the
fp32-accumulated golden (``oracle.moe.moe``: fp32 GEMMs on dequantised
weights, bf16 SiLU*up intermediate, fp32 combine, one bf16 rounding).
"""
import contextlib

import numpy as np
import pytest
import torch

from oracle import metrics, moe as oracle_moe, routing as oracle_routing

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _oracle_banks(layer):
    gu = (layer.gate_up.packed, layer.gate_up.scales)
    dn = (layer.down.packed, layer.down.scales)
    sh = None
    if layer.shared is not None:
        s = layer.shared
        sh = ((s.gate_up.packed, s.gate_up.scales), (s.down.packed, s.down.scales), s.gate_weight)
    return gu, dn, sh


def _to(pkg, layer, device):
    sh = None
    if layer.shared is not None:
        s = layer.shared
        sh = pkg.SharedExpert(s.gate_up.to(device), s.down.to(device), s.gate_weight.to(device))
    return layer.gate_up.to(device), layer.down.to(device), sh


def _run_and_check(pkg, device, layer, k, bias=None, expect_hit=None):
    gu, dn, sh = _to(pkg, layer, device)
    x = layer.hidden.to(device)
    if bias is None:
        out, r, logits = pkg.ops.moe_w4a16(x, gu, dn, top_k=k, router_weight=layer.router_weight.to(device),
                                           shared=sh, return_routing=True)
    else:
        lg = (pkg.ops.router_logits(x, layer.router_weight.to(device)) + bias.to(device)).contiguous()
        out, r, logits = pkg.ops.moe_w4a16(x, gu, dn, top_k=k, router_logits=lg, shared=sh, return_routing=True)
    logits = logits.cpu().numpy()
    ogu, odn, osh = _oracle_banks(layer)
    golden = oracle_moe.moe(layer.hidden, logits, k, ogu, odn, layer.gate_up.group_size, shared=osh)
    np.testing.assert_array_equal(r.ids.cpu().numpy(), golden["ids"])
    np.testing.assert_array_equal(r.perm.cpu().numpy(), golden["perm"])
    np.testing.assert_array_equal(r.inv.cpu().numpy(), golden["inv"])
    np.testing.assert_array_equal(r.offsets.cpu().numpy(), golden["offsets"])
    np.testing.assert_allclose(r.weights.cpu().numpy(), golden["weights"], rtol=0, atol=2e-6)
    report = metrics.compare(out.cpu(), golden["out_f32"])
    print(f"  hit experts={len(np.unique(golden['ids']))} report={report}", flush=True)
    assert out.dtype == torch.bfloat16 and tuple(out.shape) == tuple(layer.hidden.shape)
    assert report["max_rel"] <= TOL, report
    assert report["cosine"] > 0.9999, report
    # the reference-order (bf16 everywhere) restatement for information
    return report


def test_moe_verify_block_t16(pkg, device):
    """The verify-block workload: T=16, H=2048, I=512, 256 experts top-8 + shared, g128 bf16 scales."""
    print("moe T=16 E=256 k=8 shared", flush=True)
    layer = pkg.synthetic.moe_layer(16, seed=0)
    _run_and_check(pkg, device, layer, 8)


def test_moe_batch_of_blocks_skewed_t128(pkg, device):
    """T=128 with 16 hot experts biased to take ~50% of assignments."""
    print("moe T=128 skewed", flush=True)
    layer = pkg.synthetic.moe_layer(128, seed=1)
    bias = pkg.synthetic.skewed_bias(layer)
    _run_and_check(pkg, device, layer, 8, bias=bias)


@pytest.mark.timeout(300)
def test_moe_prefill_t2048(pkg, device):
    """T=2048 uniform routing, every expert hit (~64 rows each), on portable banks and on the
    tiled banks the prefill workload runs on: both meet the bar and give identical bits."""
    print("moe T=2048 portable", flush=True)
    layer = pkg.synthetic.moe_layer(2048, seed=4)
    _run_and_check(pkg, device, layer, 8)
    print("moe T=2048 tiled", flush=True)
    gu, dn, sh = _to(pkg, layer, device)
    x, rw = layer.hidden.to(device), layer.router_weight.to(device)
    out_p, r_p, _ = pkg.ops.moe_w4a16(x, gu, dn, top_k=8, router_weight=rw, shared=sh, return_routing=True)
    out_t, r_t, _ = pkg.ops.moe_w4a16(x, gu.tiled(), dn.tiled(), top_k=8, router_weight=rw, shared=sh.tiled(),
                                      return_routing=True)
    assert torch.equal(r_p.perm, r_t.perm) and torch.equal(r_p.offsets, r_t.offsets)
    assert torch.equal(out_p, out_t)


def _tile_pass_subtiles(offsets, tokens, rows=96):
    """16-row subtiles of every pass of the tile kernels, in their queue order: the shared
    expert's passes, then the routed passes by descending subtile count."""
    routed = []
    for c in (offsets[1:] - offsets[:-1]).tolist():
        routed += [min(rows, c - i) // 16 + (min(rows, c - i) % 16 > 0) for i in range(0, c, rows)]
    shared = [min(rows, tokens - i) // 16 + (min(rows, tokens - i) % 16 > 0) for i in range(0, tokens, rows)]
    return shared + sorted(routed, reverse=True)


@pytest.mark.timeout(300)
def test_prefill_tail_pieces(pkg, device):
    """Each tail split of the tile kernels (whole tiles, 2 half-width pieces, 4 pieces with row
    halves -- uneven halves of odd-subtile passes included) against the fp64 golden, and the
    three against each other: routing identical, outputs within the fp32 summation order of h's
    -136*sum partials."""
    layer = pkg.synthetic.moe_layer(2304, seed=21)
    gu, dn, sh = _to(pkg, layer, device)
    gu, dn, sh = gu.tiled(), dn.tiled(), sh.tiled()
    x, rw = layer.hidden.to(device), layer.router_weight.to(device)
    outs = {}
    for pieces in (1, 2, 4):
        print(f"prefill T=2304 tail pieces={pieces}", flush=True)
        with pkg.ops.tile_pieces(pieces):
            out, r, logits = pkg.ops.moe_w4a16(x, gu, dn, top_k=8, router_weight=rw, shared=sh, return_routing=True)
        outs[pieces] = (out.cpu(), r.ids.cpu(), r.offsets.cpu())
    offsets = outs[1][2]
    grid = torch.cuda.get_device_properties(device).multi_processor_count
    subtiles = _tile_pass_subtiles(offsets, 2304)
    for name, ntiles in (("gate/up", 2), ("down", 4)):
        rest = len(subtiles) * ntiles % grid
        tail = subtiles[len(subtiles) - (rest + ntiles - 1) // ntiles:] if rest else []
        print(f"  {name}: {len(subtiles)} passes, {rest} tail tiles of {grid}, their passes' subtiles "
              f"{sorted(set(tail))}", flush=True)
        assert rest, "every tile in full rounds: no tail to split"
        assert any(n % 2 for n in tail), "no odd-subtile pass in the tail: the uneven row halves go untested"
    ogu, odn, osh = _oracle_banks(layer)
    golden = oracle_moe.moe(layer.hidden, logits.cpu().numpy(), 8, ogu, odn, 128, shared=osh)
    for pieces, (out, ids, off) in outs.items():
        assert torch.equal(ids, outs[1][1]) and torch.equal(off, offsets)
        report = metrics.compare(out, golden["out_f32"])
        versus = metrics.compare(out, outs[1][0].float().numpy())
        print(f"  pieces={pieces} {report} vs whole tiles max_rel={versus['max_rel']:.2e}", flush=True)
        assert report["max_rel"] <= TOL and report["cosine"] > 0.9999, report
        assert versus["max_rel"] <= 4e-3, versus


@pytest.mark.timeout(300)
def test_moe_prefill_past_the_prep_block_cap(pkg, device):
    """T=16400 (above the 16384 prep blocks of a route_topk launch, so 16 prep blocks convert a
    second row): every token's routing and output equal those of the same tokens run as two
    halves of 8200 (rows are independent; outputs within the fp32 order of the tail pieces)."""
    print("moe T=16400 E=64 k=4: whole vs halves", flush=True)
    layer = pkg.synthetic.moe_layer(16400, experts=64, seed=12)
    gu, dn, sh = _to(pkg, layer, device)
    gu, dn, sh = gu.tiled(), dn.tiled(), sh.tiled()
    x, rw = layer.hidden.to(device), layer.router_weight.to(device)
    whole, r, _ = pkg.ops.moe_w4a16(x, gu, dn, top_k=4, router_weight=rw, shared=sh, return_routing=True)
    parts = [pkg.ops.moe_w4a16(x[a:a + 8200].contiguous(), gu, dn, top_k=4, router_weight=rw, shared=sh,
                               return_routing=True) for a in (0, 8200)]
    assert torch.equal(r.ids, torch.cat([q[1].ids for q in parts]))
    halves = torch.cat([q[0] for q in parts])
    report = metrics.compare(whole.float().cpu(), halves.float().cpu().numpy())
    print(f"  whole vs halves {report}", flush=True)
    assert report["max_rel"] <= 4e-3 and report["cosine"] > 0.99999, report
    tail = metrics.compare(whole[16384:].float().cpu(), halves[16384:].float().cpu().numpy())
    assert tail["max_rel"] <= 4e-3, tail


def _logit_error_bound(hidden, router_weight):
    """Worst-case error of an fp32 dot product of bf16 vectors (products exact in fp32, n-term
    recursive sum): |err| <= n * 2^-24 / (1 - n * 2^-24) * sum|x_i w_i|, per (token, expert)."""
    x = hidden.reshape(-1, hidden.shape[-1]).to(torch.float64).abs()
    w = router_weight.to(torch.float64).abs()
    n = hidden.shape[-1]
    u = 2.0 ** -24
    return (x @ w.T).numpy() * (n * u / (1 - n * u))


@pytest.mark.parametrize("tokens,seed", [(16, 0), (128, 1), (2048, 4)])
def test_routing_from_hidden_matches_oracle_logits(pkg, device, tokens, seed):
    """End to end from (hidden, router_weight): the GPU's ids equal the oracle's ids computed on
    the oracle's own logits (fp64 dot products rounded to fp32) on every row whose k+1 largest
    logits are separated by more than twice the fp32 dot-product error bound -- there no
    admissible fp32 summation order can change the selection or its order."""
    print(f"routing end to end T={tokens}", flush=True)
    k = 8
    layer = pkg.synthetic.moe_layer(tokens, seed=seed)
    x, rw = layer.hidden.to(device), layer.router_weight.to(device)
    gu, dn, sh = _to(pkg, layer, device)
    _, r, gpu_logits = pkg.ops.moe_w4a16(x, gu.tiled(), dn.tiled(), top_k=k, router_weight=rw, shared=sh.tiled(),
                                         return_routing=True)
    logits = oracle_moe.router_logits(layer.hidden, layer.router_weight)
    bound = _logit_error_bound(layer.hidden, layer.router_weight)
    assert np.all(np.abs(gpu_logits.cpu().numpy() - logits) <= bound + np.abs(logits) * 2.0 ** -23)
    ids, wts = oracle_routing.topk(logits, k)
    top = -np.sort(-logits, axis=1)[:, :k + 1]
    sep = (top[:, :-1] - top[:, 1:]).min(axis=1) > 2 * bound.max(axis=1)
    assert sep.mean() > 0.4, sep.mean()        # the seeds give 53-63% of rows; the check must cover many
    got = r.ids.cpu().numpy()
    np.testing.assert_array_equal(got[sep], ids[sep])
    np.testing.assert_allclose(r.weights.cpu().numpy()[sep], wts[sep], rtol=0, atol=1e-5)
    # every row: what the GPU selects lies within the error band of the oracle's k-th logit, and
    # every expert clearly above the oracle's (k+1)-th logit is selected
    band = 2 * bound.max(axis=1)
    chosen = np.take_along_axis(logits, got.astype(np.int64), axis=1)
    assert np.all(chosen >= (top[:, k - 1] - band)[:, None])
    for t in range(tokens):
        clear = set(np.nonzero(logits[t] > top[t, k] + band[t])[0].tolist())
        assert clear <= set(got[t].tolist()), t
    print(f"  rows checked bit-exactly: {int(sep.sum())} of {tokens}", flush=True)


@pytest.mark.parametrize("tokens,experts,k,hidden,inter,group,scale_dtype,shared", [
    (1, 8, 2, 512, 512, 128, torch.bfloat16, True),
    (5, 8, 2, 512, 512, 128, torch.bfloat16, False),
    (40, 4, 1, 1024, 512, 256, torch.bfloat16, True),
    (37, 16, 4, 512, 1024, 128, torch.float32, True),
    (70, 4, 4, 512, 512, 128, torch.bfloat16, True),          # E == k: every token hits every expert
    (20, 16, 4, 1024, 1024, 128, torch.float32, True),        # small-T kernel: K = 1024 both ways, fp32 scales
    (32, 64, 8, 2048, 512, 128, torch.bfloat16, True),        # small-T kernel at its largest T
    (9, 8, 8, 512, 512, 128, torch.bfloat16, True),           # small-T kernel, E == k
    (300, 16, 4, 1024, 512, 128, torch.float32, True),        # tiled prefill kernel, fp32 scales
    (256, 8, 2, 2048, 512, 256, torch.bfloat16, False),       # tiled prefill kernel, group 256
    (2100, 64, 8, 512, 512, 128, torch.bfloat16, True),       # tiled prefill kernel past 16384 pairs: count launch, sorted passes
    (16, 256, 8, 2048, 512, 256, torch.float32, True),        # verify kernels, the reference quantizer's g256 fp32
    (5, 8, 2, 512, 512, 256, torch.bfloat16, False),          # verify kernels, group 256, K = 512 (one group per 2 k-blocks)
    (32, 64, 8, 2048, 1024, 256, torch.float32, True),        # verify kernels at their largest T, group 256
    (16, 200, 8, 512, 512, 128, torch.bfloat16, True),        # half-wave routing, 8 keys a lane, E not a multiple of 32
    (16, 512, 8, 512, 512, 128, torch.bfloat16, True),        # verify kernels, block routing (E > 256)
    (24, 1024, 4, 512, 512, 128, torch.float32, False),       # block routing at the largest expert count
    (32, 300, 8, 512, 512, 256, torch.bfloat16, True),        # block routing, two token passes, group 256
])
def test_moe_small_shapes(pkg, device, tokens, experts, k, hidden, inter, group, scale_dtype, shared):
    print(f"moe T={tokens} E={experts} k={k} H={hidden} I={inter} g={group} {scale_dtype} shared={shared}",
          flush=True)
    layer = pkg.synthetic.moe_layer(tokens, hidden=hidden, inter=inter, experts=experts, group_size=group,
                                    seed=tokens + experts, shared=shared, scale_dtype=scale_dtype)
    _run_and_check(pkg, device, layer, k)


def test_moe_experts_entry_with_oracle_routing(pkg, device):
    """dflash_moe_experts_w4a16 driven by a routing computed on the CPU."""
    from oracle import routing
    layer = pkg.synthetic.moe_layer(24, hidden=512, inter=512, experts=32, seed=9)
    logits = oracle_moe.router_logits(layer.hidden, layer.router_weight)
    ids, wts = routing.topk(logits, 4)
    perm, inv, offsets = routing.permutation(ids, 32)
    r = pkg.ops.Routing(*(torch.from_numpy(a).to(device) for a in (ids, wts, perm, inv, offsets)))
    gu, dn, sh = _to(pkg, layer, device)
    out = pkg.ops.moe_experts(layer.hidden.to(device), r, gu, dn, shared=sh)
    ogu, odn, osh = _oracle_banks(layer)
    golden = oracle_moe.moe(layer.hidden, logits, 4, ogu, odn, 128, shared=osh)
    assert metrics.compare(out.cpu(), golden["out_f32"])["max_rel"] <= TOL


def test_fused_ops_moe_reference_signature(pkg, device):
    """moe(hidden [1,T,H], router_weight, gate_up, down, top_k=k): routed experts only."""
    layer = pkg.synthetic.moe_layer(16, hidden=512, inter=512, experts=64, seed=12, shared=False)
    gu, dn, _ = _to(pkg, layer, device)
    x = layer.hidden.reshape(1, 16, 512).to(device)
    rw = layer.router_weight.to(device)
    out = pkg.fused_ops.moe(x, rw, gu, dn, top_k=8)
    assert tuple(out.shape) == (1, 16, 512) and out.dtype == torch.bfloat16
    logits = pkg.ops.router_logits(x, rw).cpu().numpy()
    ogu, odn, _ = _oracle_banks(layer)
    golden = oracle_moe.moe(layer.hidden, logits, 8, ogu, odn, 128)
    assert metrics.compare(out.cpu().reshape(16, 512), golden["out_f32"])["max_rel"] <= TOL


def test_moe_repeat_calls_are_identical(pkg, device):
    """Deterministic combine: the same inputs give bit-identical outputs."""
    layer = pkg.synthetic.moe_layer(16, seed=5)
    gu, dn, sh = _to(pkg, layer, device)
    x, rw = layer.hidden.to(device), layer.router_weight.to(device)
    a = pkg.ops.moe_w4a16(x, gu, dn, top_k=8, router_weight=rw, shared=sh)
    b = pkg.ops.moe_w4a16(x, gu, dn, top_k=8, router_weight=rw, shared=sh)
    assert torch.equal(a, b)


@pytest.mark.timeout(300)
@pytest.mark.parametrize("tokens,pieces,layout", [(2048, 4, "portable"), (2048, 4, "tiled"), (2048, None, "tiled"),
                                                  (128, None, "tiled")])
def test_long_block_repeat_calls_are_identical(pkg, device, tokens, pieces, layout):
    """Bit-identical outputs over repeated calls on the prefill tile kernels (every tail tile in
    four pieces, or the grid's own split) and on the gathered-pass verify kernels (T=128): a
    weight stage read before its direct-to-LDS loads have landed shows up as differences from
    call to call, not as a tolerance failure on every run."""
    print(f"moe T={tokens} pieces={pieces} {layout}: 4 calls", flush=True)
    layer = pkg.synthetic.moe_layer(tokens, seed=4)
    gu, dn, sh = _to(pkg, layer, device)
    if layout == "tiled":
        gu, dn, sh = gu.tiled(), dn.tiled(), sh.tiled()
    x, rw = layer.hidden.to(device), layer.router_weight.to(device)
    ctx = pkg.ops.tile_pieces(pieces) if pieces else contextlib.nullcontext()
    with ctx:
        outs = [pkg.ops.moe_w4a16(x, gu, dn, top_k=8, router_weight=rw, shared=sh) for _ in range(4)]
    for i, o in enumerate(outs[1:], 1):
        diff = (o.float() - outs[0].float()).abs()
        assert torch.equal(o, outs[0]), f"call {i}: {int((diff > 0).sum())} elements differ, max {float(diff.max()):.3g}"


@pytest.fixture
def two_launches(pkg):
    """The verify block's down GEMM as a launch of its own for one test (the split-K down off)."""
    with pkg.ops.split_down(False):
        yield


@pytest.fixture
def split_on(pkg):
    """The opt-in split-K down switched on for one test."""
    with pkg.ops.split_down(True):
        yield


@pytest.mark.parametrize("tokens", [16, 40, 128])
def test_measure_stage_relaunches_one_kernel(pkg, device, tokens, two_launches):
    """Measurement mode re-runs one stage on the workspace of a full call and rewrites identical
    bytes (gate/up and down as separate launches: verify block, gathered verify, T=128)."""
    layer = pkg.synthetic.moe_layer(tokens, seed=6)
    gu, dn, sh = _to(pkg, layer, device)
    x, rw = layer.hidden.to(device), layer.router_weight.to(device)
    assert not pkg.ops.moe_split_down(tokens, 2048, 512, 256, 8, 128, True)
    ws = torch.empty(pkg.ops.moe_workspace_bytes(tokens, 2048, 512, 256, 8, 128, True), dtype=torch.uint8,
                     device=device)
    ref = pkg.ops.moe_w4a16(x, gu, dn, top_k=8, router_weight=rw, shared=sh, workspace=ws)
    torch.cuda.synchronize()
    snapshot = ws.clone()
    for stage in (pkg.ops.STAGE_GATE_UP, pkg.ops.STAGE_DOWN, pkg.ops.STAGE_EXPERTS):
        pkg.ops.set_measure_stage(stage)
        try:
            pkg.ops.moe_w4a16(x, gu, dn, top_k=8, router_weight=rw, shared=sh, workspace=ws)
        finally:
            pkg.ops.set_measure_stage(0)
        torch.cuda.synchronize()
        assert torch.equal(ws, snapshot), stage
    again = pkg.ops.moe_w4a16(x, gu, dn, top_k=8, router_weight=rw, shared=sh, workspace=ws)
    assert torch.equal(again, ref)


def test_measure_stage_relaunches_the_split_kernel(pkg, device, split_on):
    """T=16: measurement of EXPERTS with the call's router logits relaunches the gate/up launch
    that also runs the split-K down, which rewrites identical bytes."""
    layer = pkg.synthetic.moe_layer(16, seed=6)
    gu, dn, sh = _to(pkg, layer, device)
    gu, dn, sh = gu.tiled(), dn.tiled(), sh.tiled()
    assert pkg.ops.moe_split_down(16, 2048, 512, 256, 8, 128, True)
    x, rw = layer.hidden.to(device), layer.router_weight.to(device)
    lg = pkg.ops.router_logits(x, rw)
    ws = torch.empty(pkg.ops.moe_workspace_bytes(16, 2048, 512, 256, 8, 128, True), dtype=torch.uint8, device=device)
    ref = pkg.ops.moe_w4a16(x, gu, dn, top_k=8, router_logits=lg, shared=sh, workspace=ws)
    torch.cuda.synchronize()
    snapshot = ws.clone()
    pkg.ops.set_measure_stage(pkg.ops.STAGE_EXPERTS)
    try:
        for _ in range(3):
            pkg.ops.moe_w4a16(x, gu, dn, top_k=8, router_logits=lg, shared=sh, workspace=ws)
    finally:
        pkg.ops.set_measure_stage(0)
    torch.cuda.synchronize()
    assert torch.equal(ws, snapshot)
    again = pkg.ops.moe_w4a16(x, gu, dn, top_k=8, router_logits=lg, shared=sh, workspace=ws)
    assert torch.equal(again, ref)


@pytest.mark.parametrize("tokens,experts,k,hidden,inter,group,scale_dtype,shared,layout", [
    (16, 256, 8, 2048, 512, 128, torch.bfloat16, True, "tiled"),      # the verify block
    (16, 256, 8, 2048, 512, 128, torch.bfloat16, True, "portable"),
    (1, 256, 8, 2048, 512, 128, torch.bfloat16, True, "tiled"),       # one token: a pass spans ~28 workgroups
    (5, 64, 4, 1024, 1024, 256, torch.float32, True, "tiled"),        # down over K = 1024, group 256, fp32 scales
    (24, 16, 4, 1024, 512, 128, torch.bfloat16, True, "tiled"),       # full 16-row passes, two shared passes
    (16, 32, 2, 512, 512, 128, torch.bfloat16, False, "tiled"),       # H = 512, no shared expert
])
def test_split_down_layer(pkg, device, tokens, experts, k, hidden, inter, group, scale_dtype, shared, layout,
                          split_on):
    """The down GEMM inside the gate/up launch (split over K by each workgroup's strips, partial
    rows added by the combine): on one workspace, a call, a repeat and a smaller block after it
    each route bit-exactly, meet the oracle bar, repeat bit-identically, and agree with the two
    launches to within the fp32 summation order."""
    ws = torch.empty(pkg.ops.moe_workspace_bytes(tokens, hidden, inter, experts, k, group, shared),
                     dtype=torch.uint8, device=device)
    prev = None
    for t in (tokens, tokens, max(1, tokens // 3)):
        print(f"split down T={t} E={experts} k={k} H={hidden} I={inter} g={group} {layout}", flush=True)
        assert pkg.ops.moe_split_down(t, hidden, inter, experts, k, group, shared, scale_dtype, layout)
        layer = pkg.synthetic.moe_layer(t, hidden=hidden, inter=inter, experts=experts, group_size=group,
                                        seed=t + 3 * experts, shared=shared, scale_dtype=scale_dtype)
        gu, dn, sh = _to(pkg, layer, device)
        if layout == "tiled":
            gu, dn, sh = gu.tiled(), dn.tiled(), sh.tiled() if sh else None
        x, rw = layer.hidden.to(device), layer.router_weight.to(device)
        out, r, logits = pkg.ops.moe_w4a16(x, gu, dn, top_k=k, router_weight=rw, shared=sh, return_routing=True,
                                           workspace=ws)
        if prev is not None and prev[0] == t:
            assert torch.equal(out, prev[1])
        prev = (t, out.clone())
        with pkg.ops.split_down(False):
            two = pkg.ops.moe_w4a16(x, gu, dn, top_k=k, router_weight=rw, shared=sh)
        ogu, odn, osh = _oracle_banks(layer)
        golden = oracle_moe.moe(layer.hidden, logits.cpu().numpy(), k, ogu, odn, group, shared=osh)
        np.testing.assert_array_equal(r.ids.cpu().numpy(), golden["ids"])
        np.testing.assert_array_equal(r.perm.cpu().numpy(), golden["perm"])
        np.testing.assert_array_equal(r.inv.cpu().numpy(), golden["inv"])
        np.testing.assert_array_equal(r.offsets.cpu().numpy(), golden["offsets"])
        report = metrics.compare(out.cpu(), golden["out_f32"])
        versus = metrics.compare(out.cpu(), two.float().cpu().numpy())
        print(f"  T={t} report={report} vs two launches max_rel={versus['max_rel']:.2e}", flush=True)
        assert report["max_rel"] <= TOL and report["cosine"] > 0.9999, report
        assert versus["max_rel"] <= 4e-3, versus


def test_split_down_refused_shapes_run_two_launches(pkg, device, split_on):
    """Shapes outside the split-K down -- unit ranges of more than two passes (T=32 at E=256,
    top-8), H outside {512, 1024, 2048}, blocks routed outside the gate/up launch -- run the
    separate down launch and still meet the oracle bar."""
    assert not pkg.ops.moe_split_down(32, 2048, 512, 256, 8, 128, True)
    assert not pkg.ops.moe_split_down(16, 1536, 512, 64, 8, 128, True)
    assert not pkg.ops.moe_split_down(40, 2048, 512, 256, 8, 128, True)
    layer = pkg.synthetic.moe_layer(32, seed=77)
    _run_and_check(pkg, device, layer, 8)


def test_empty_batch(pkg, device):
    """Zero tokens: empty outputs and the oracle's all-zero expert offsets from every entry point."""
    from oracle import routing
    layer = pkg.synthetic.moe_layer(4, hidden=512, inter=512, experts=8, seed=2)
    gu, dn, sh = _to(pkg, layer, device)
    _, _, offsets = routing.permutation(np.zeros((0, 2), np.int32), 8)
    x = torch.empty((0, 512), dtype=torch.bfloat16, device=device)
    out, r, logits = pkg.ops.moe_w4a16(x, gu, dn, top_k=2, router_weight=layer.router_weight.to(device), shared=sh,
                                       return_routing=True)
    assert tuple(out.shape) == (0, 512) and tuple(r.ids.shape) == (0, 2) and tuple(logits.shape) == (0, 8)
    np.testing.assert_array_equal(r.offsets.cpu().numpy(), offsets)
    r2 = pkg.ops.route(torch.empty((0, 8), dtype=torch.float32, device=device), 2)
    np.testing.assert_array_equal(r2.offsets.cpu().numpy(), offsets)
    assert tuple(pkg.ops.moe_experts(x, r2, gu, dn, shared=sh).shape) == (0, 512)
    w = pkg.packing.quantize_w4(torch.randn((64, 512)).to(torch.bfloat16), 128).to(device)
    assert tuple(pkg.ops.qlinear(x, w).shape) == (0, 64)


@pytest.mark.parametrize("tokens,experts,k", [(16, 256, 8), (32, 64, 8), (7, 128, 4)])
def test_moe_in_kernel_routing_ties(pkg, device, tokens, experts, k):
    """Logits on a coarse grid (many equal values per token, -0.0 and +0.0 among them): the
    routing inside the gate/up launch must break ties by the lowest expert id, as the oracle does."""
    print(f"moe ties T={tokens} E={experts} k={k}", flush=True)
    layer = pkg.synthetic.moe_layer(tokens, hidden=2048, inter=512, experts=experts, seed=40 + tokens)
    gen = torch.Generator().manual_seed(tokens * 7 + experts)
    lg = torch.round(torch.randn((tokens, experts), generator=gen) * 1.5) / 2
    lg[lg == 0] = torch.where(torch.rand(int((lg == 0).sum()), generator=gen) < 0.5, -0.0, 0.0)
    gu, dn, sh = _to(pkg, layer, device)
    out, r, _ = pkg.ops.moe_w4a16(layer.hidden.to(device), gu, dn, top_k=k, router_logits=lg.to(device), shared=sh,
                                  return_routing=True)
    ogu, odn, osh = _oracle_banks(layer)
    golden = oracle_moe.moe(layer.hidden, lg.numpy(), k, ogu, odn, layer.gate_up.group_size, shared=osh)
    np.testing.assert_array_equal(r.ids.cpu().numpy(), golden["ids"])
    np.testing.assert_array_equal(r.perm.cpu().numpy(), golden["perm"])
    np.testing.assert_array_equal(r.offsets.cpu().numpy(), golden["offsets"])
    np.testing.assert_allclose(r.weights.cpu().numpy(), golden["weights"], rtol=0, atol=2e-6)
    assert metrics.compare(out.cpu(), golden["out_f32"])["max_rel"] <= TOL
