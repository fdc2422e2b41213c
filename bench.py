"""Benchmark: one routed-MoE layer (W4A16, g128) of the verify block on one MI355X.

Step = one whole MoE layer forward at T=16 tokens (router logits, top-8
routing and permutation, grouped gate/up + SiLU*up, down, weighted combine,
gated shared expert) through ``dflash_moe_w4a16``.  Inputs are resident in
HBM before timing.  Three independent weight sets (~1.25 GB) and eight hidden
blocks are rotated so that the 256 MB Infinity Cache cannot serve the
~167 MB per-step working set.

Steps are replayed from HIP graphs (24 layer-steps per graph, the way a
multi-layer verify forward would be issued), so host launch overhead is not
part of the measurement.

Prints ONE JSON line.  ``value`` is microseconds per MoE layer (lower is
better).  ``roofline`` is the dominant kernel, the layer's gate/up launch as it
runs in the layer: it routes the block in its prologue (from the step's router
logits) and streams the hit experts' gate/up rows.  HIP events on its launch
stream bracket graph replays that hold only that kernel's launches
(measurement mode of the library), one per step over the same rotation of
weight sets and hidden blocks; achieved = its algorithmic bytes (int4 gate/up
rows + bf16 scales of the hit experts and the shared expert, x in, h out) /
mean launch duration.  ``traffic`` is the HBM bytes the same kernel moves per
launch, from the rocprofv3 FETCH_SIZE / WRITE_SIZE passes recorded in
``profiles/hbm_traffic_gate_up_t16.json`` (scaled by the counters' reading
of a plain copy of known size), or null when that file is absent.
``stages`` times the layer's other expert launches; ``split_down_opt_in`` the
same layer with the down GEMM inside the gate/up launch (split over K,
partial y rows added by the combine), which is not the default.
``prefill`` reports the T=2048 layer in TFLOP/s against bf16 MFMA peak.
``cpu_baseline`` times the oracle's CPU restatement of the same layer.
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import statistics
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
PKG_DIR = ROOT / "qwen3.5-35b-dflash_amd"
PKG_NAME = "qwen35_dflash_amd"

METRIC = "µs per MoE layer at T=16 verify (HBM GB/s %); TFLOP/s at T=2048 prefill"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2516.6
INT4_BYTES_PER_EXPERT = 2 * 512 * 2048 // 2 + 2048 * 512 // 2        # gate_up + down, packed int4
SCALE_BYTES_PER_EXPERT = (2 * 512 * 2048 // 128 + 2048 * 512 // 128) * 2  # bf16 group-128 scales


def load_package():
    if PKG_NAME in sys.modules:
        return sys.modules[PKG_NAME]
    spec = importlib.util.spec_from_file_location(PKG_NAME, PKG_DIR / "__init__.py",
                                                  submodule_search_locations=[str(PKG_DIR)])
    module = importlib.util.module_from_spec(spec)
    sys.modules[PKG_NAME] = module
    spec.loader.exec_module(module)
    return module


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def device_bank(pkg, gen, shape, device):
    """Random packed int4 bank generated on the device (uniform bytes = two uniform int4)."""
    return pkg.synthetic.device_bank(gen, shape, device)


def weight_sets(pkg, nsets, device, seed=1234, hidden=2048, inter=512, experts=256, tiled=True):
    """Random banks per set; repacked once into the kernels' tiled layout (as a model load would) unless tiled=False."""
    gen = torch.Generator(device=device).manual_seed(seed)
    sets = []
    for _ in range(nsets):
        gu = device_bank(pkg, gen, (experts, 2 * inter, hidden), device)
        dn = device_bank(pkg, gen, (experts, hidden, inter), device)
        sh = pkg.SharedExpert(device_bank(pkg, gen, (2 * inter, hidden), device),
                              device_bank(pkg, gen, (hidden, inter), device),
                              (torch.randn((hidden,), device=device, generator=gen) * 0.02).to(torch.bfloat16))
        router = (torch.randn((experts, hidden), device=device, generator=gen) * 0.02).to(torch.bfloat16)
        if tiled:
            gu, dn, sh = gu.tiled(), dn.tiled(), sh.tiled()
        sets.append((gu, dn, sh, router))
    torch.cuda.synchronize()
    return sets


# The target model's quantized non-expert projections and its LM head (graph/quant_plan.py:25-32,55-56),
# N x K: GDN in_proj_qkv / in_proj_z / in_proj_a|b / out_proj (16 key heads, 32 value heads, head
# dims 128: fused/ops.py:354-360); attention q (gated) / k|v / o (16 heads, 2 KV heads, head_dim 256).
QLINEAR_SHAPES = (
    ("linear_attn.in_proj_qkv", 8192, 2048), ("linear_attn.in_proj_z", 4096, 2048),
    ("linear_attn.in_proj_a", 32, 2048), ("linear_attn.in_proj_b", 32, 2048),
    ("linear_attn.out_proj", 2048, 4096),
    ("self_attn.q_proj", 8192, 2048), ("self_attn.k_proj", 512, 2048), ("self_attn.v_proj", 512, 2048),
    ("self_attn.o_proj", 2048, 4096),
    ("lm_head", 248320, 2048),
)


def time_qlinear(pkg, device, steps, warmup, nsets=3, tokens=16):
    """W4A16 qlinear per projection at a 16-token block: tiled weights, `nsets` rotated copies."""
    gen = torch.Generator(device=device).manual_seed(4321)
    x = torch.randn((tokens, 4096), device=device, generator=gen).to(torch.bfloat16)
    out = {}
    for name, n, k in QLINEAR_SHAPES:
        ws_ = [device_bank(pkg, gen, (n, k), device).tiled() for _ in range(nsets)]
        xk = x[:, :k].contiguous()
        work = torch.empty(pkg.ops.qlinear_workspace_bytes(tokens, k, 128), dtype=torch.uint8, device=device)
        ms = time_steps(lambda j: pkg.ops.qlinear(xk, ws_[j % nsets], workspace=work), steps, warmup)
        nbytes = n * k // 2 + n * (k // 128) * 2
        out[name] = {"n": n, "k": k, "us": round(ms * 1e3, 2), "weight_gbs": round(nbytes / (ms * 1e-3) / 1e9, 1)}
        del ws_
    gdn = sum(out[f"linear_attn.{p}"]["us"] for p in ("in_proj_qkv", "in_proj_z", "in_proj_a", "in_proj_b", "out_proj"))
    attn = sum(out[f"self_attn.{p}"]["us"] for p in ("q_proj", "k_proj", "v_proj", "o_proj"))
    # projections reading the same x stacked into one matrix (pkg.concat_rows): one launch each
    stacked = {}
    for name, n in (("linear_attn.in_proj_qkv+z+a+b", 8192 + 4096 + 32 + 32), ("self_attn.q+k+v_proj", 8192 + 512 + 512)):
        ws_ = [device_bank(pkg, gen, (n, 2048), device).tiled() for _ in range(nsets)]
        xk = x[:, :2048].contiguous()
        work = torch.empty(pkg.ops.qlinear_workspace_bytes(tokens, 2048, 128), dtype=torch.uint8, device=device)
        ms = time_steps(lambda j: pkg.ops.qlinear(xk, ws_[j % nsets], workspace=work), steps, warmup)
        stacked[name] = {"n": n, "k": 2048, "us": round(ms * 1e3, 2)}
        del ws_
    gdn_s = stacked["linear_attn.in_proj_qkv+z+a+b"]["us"] + out["linear_attn.out_proj"]["us"]
    attn_s = stacked["self_attn.q+k+v_proj"]["us"] + out["self_attn.o_proj"]["us"]
    return {"tokens": tokens, "group_size": 128, "projections": out, "stacked": stacked,
            "gdn_layer_projections_us": round(gdn, 2), "attention_layer_projections_us": round(attn, 2),
            "gdn_layer_projections_stacked_us": round(gdn_s, 2),
            "attention_layer_projections_stacked_us": round(attn_s, 2)}


def moe_flops(tokens, k, hidden=2048, inter=512):
    per_row = 2 * (2 * inter * hidden + hidden * inter)
    return per_row * (tokens * k + tokens)


def _graph(fn, length):
    """Capture `length` consecutive steps fn(0..length-1) into one HIP graph."""
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for j in range(length):      # eager pass: warms up and settles the graph's allocations
            fn(j)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for j in range(length):
            fn(j)
    torch.cuda.synchronize()
    return graph


def time_steps(fn, steps, warmup, period=24):
    """Time exactly `steps` steps, replayed from HIP graphs of `period` steps, with HIP events."""
    full, rest = divmod(steps, period)
    main = _graph(fn, period) if full else None
    tail = _graph(fn, rest) if rest else None
    for _ in range(max(1, warmup // period)):
        (main or tail).replay()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(full):
        main.replay()
    if tail is not None:
        tail.replay()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps


def time_layer(pkg, sets, blocks, top_k, steps, warmup, workspace):
    """Whole-layer time per step; step j uses weight set j % sets and hidden block j % blocks."""
    def step(j):
        gu, dn, sh, router = sets[j % len(sets)]
        pkg.ops.moe_w4a16(blocks[j % len(blocks)], gu, dn, top_k=top_k, router_weight=router, shared=sh,
                          workspace=workspace)
    return time_steps(step, steps, warmup)


def time_experts(pkg, sets, blocks, top_k, steps, warmup, workspace):
    """Expert-stage time per step (routing prepared beforehand) and the mean hit-expert count."""
    period = 24
    prepared = []
    for j in range(period):
        gu, dn, sh, router = sets[j % len(sets)]
        x = blocks[j % len(blocks)]
        r = pkg.ops.route(pkg.ops.router_logits(x, router), top_k)
        hit = int((r.offsets[1:] > r.offsets[:-1]).sum().item())
        prepared.append((x, r, gu, dn, sh, hit))
    torch.cuda.synchronize()

    def step(j):
        x, r, gu, dn, sh, _ = prepared[j % period]
        pkg.ops.moe_experts(x, r, gu, dn, shared=sh, workspace=workspace)
    ms = time_steps(step, steps, warmup, period)
    return ms, statistics.mean(p[5] for p in prepared)


GATE_UP_BYTES_PER_EXPERT = 2 * 512 * 2048 // 2 + 2 * 512 * (2048 // 128) * 2   # int4 + bf16 scales
DOWN_BYTES_PER_EXPERT = 2048 * 512 // 2 + 2048 * (512 // 128) * 2


def split_part_rows(offsets, tokens, grid, strips=32, shared=True):
    """Partial y rows the split-K down writes for one routing: pass P (16-row passes of every hit
    expert in id order, then the shared expert's) is spread over workgroups
    floor((G (x + 1) - 1) / U) of its first and last units x, each writing the pass's rows."""
    counts = [int(c) for c in (offsets[1:] - offsets[:-1]).tolist()]
    rows = [min(16, c - 16 * i) for c in counts if c > 0 for i in range((c + 15) // 16)]
    if shared:
        rows += [min(16, tokens - 16 * i) for i in range((tokens + 15) // 16)]
    units = len(rows) * strips
    total = 0
    for p_, r in enumerate(rows):
        b0 = (grid * (p_ * strips + 1) - 1) // units
        b1 = (grid * (p_ + 1) * strips - 1) // units
        total += r * (b1 - b0 + 1)
    return total


def time_stage(pkg, sets, blocks, top_k, steps, warmup, stage=None, given_logits=False):
    """Average launch duration of one expert-stage kernel, timed with HIP events.

    For each of `period` steps (weight set j % sets, hidden block j % blocks)
    a full layer call fills its own workspace; then, in measurement mode,
    layer calls launch only the stage's kernel on that workspace.  A HIP graph
    of those single-kernel steps is replayed between two events on torch's
    current stream (the stream the library launches on), so the timed region
    holds nothing but back-to-back launches of the kernel.  Returns the mean
    duration per launch (ms), the mean number of hit experts and the mean number of
    partial y rows a split-K down launch writes for those routings.
    """
    stage = pkg.ops.STAGE_GATE_UP if stage is None else stage
    period = 24
    device = blocks[0].device
    tokens = blocks[0].shape[0]
    grid = torch.cuda.get_device_properties(device).multi_processor_count
    nbytes = pkg.ops.moe_workspace_bytes(tokens, 2048, 512, 256, top_k, 128, True)
    wss = [torch.empty(nbytes, dtype=torch.uint8, device=device) for _ in range(period)]
    # with given_logits the calls pass each step's router logits, so the verify gate/up kernel
    # routes in its prologue exactly as inside the layer; else it reads the work table
    logits = [pkg.ops.router_logits(blocks[j % len(blocks)], sets[j % len(sets)][3]) for j in range(period)]
    hits, parts = [], []

    def call(j):
        gu, dn, sh, router = sets[j % len(sets)]
        kw = {"router_logits": logits[j % period]} if given_logits else {"router_weight": router}
        return pkg.ops.moe_w4a16(blocks[j % len(blocks)], gu, dn, top_k=top_k, shared=sh, workspace=wss[j % period],
                                 return_routing=True, **kw)
    for j in range(period):
        _, r, _ = call(j)
        hits.append(int((r.offsets[1:] > r.offsets[:-1]).sum().item()))
        parts.append(split_part_rows(r.offsets.cpu(), tokens, grid))
    torch.cuda.synchronize()

    def step(j):
        call(j)
    pkg.ops.set_measure_stage(stage)
    try:
        ms = time_steps(step, steps, warmup, period)
    finally:
        pkg.ops.set_measure_stage(0)
    return ms, statistics.mean(hits), statistics.mean(parts)


def time_stack(pkg, device, steps, warmup, context=4096, tokens=16):
    """The 40-layer target's verify forward over a 16-token block at a 4096-token context.

    Step = embedding, 30 GDN + 10 attention layers (each: norm, mixer, norm, routed MoE with
    the shared expert), final norm, LM head and top-1, replayed from HIP graphs (period 4).
    ``kernel_share`` = time of the same qlinear + MoE launches alone (the same shapes, in a
    graph of their own) / time of the whole forward.
    """
    c = pkg.plan.TargetConfig()
    w = pkg.target.random_weights(c, seed=7, device=device)
    model = pkg.target.TargetModel(w, capacity=context + 64, feature_layers=pkg.target.DRAFT_FEATURE_LAYERS)
    state = model.synthetic_context(context, seed=8)
    gen = torch.Generator(device=device).manual_seed(9)
    ids = torch.randint(0, c.vocab, (tokens,), device=device, generator=gen)
    ws = torch.empty(pkg.ops.moe_workspace_bytes(tokens, c.hidden, c.moe_inter, c.experts, c.top_k, 128, True),
                     dtype=torch.uint8, device=device)
    torch.cuda.synchronize()
    full_ms = time_steps(lambda j: model.forward(ids, state, workspace=ws), steps, warmup, period=4)
    hidden = model.embed(ids)
    gdn_ms = time_steps(lambda j: model.layer(0, hidden, state, ws), steps, warmup, period=8)
    attn_ms = time_steps(lambda j: model.layer(3, hidden, state, ws), steps, warmup, period=8)
    head_ms = time_steps(lambda j: pkg.ops.qlinear(hidden.to(torch.bfloat16), w.lm_head).argmax(-1), steps, warmup,
                         period=8)
    x = torch.randn((tokens, c.hidden), device=device, generator=gen).to(torch.bfloat16)
    x_gdn = torch.randn((tokens, c.linear_value_heads * c.linear_value_dim), device=device,
                        generator=gen).to(torch.bfloat16)
    x_att = torch.randn((tokens, c.heads * c.head_dim), device=device, generator=gen).to(torch.bfloat16)

    def kernels_only(j):
        for lw in w.layers:
            pkg.ops.qlinear(x, lw.mixer_in)
            pkg.ops.qlinear(x_gdn if lw.kind == "linear_attention" else x_att, lw.mixer_out)
            pkg.ops.moe_w4a16(x, lw.gate_up, lw.down, top_k=c.top_k, router_weight=lw.router, shared=lw.shared,
                              workspace=ws)
        pkg.ops.qlinear(x, w.lm_head)
    kern_ms = time_steps(kernels_only, steps, warmup, period=4)
    n_gdn = sum(k == "linear_attention" for k in c.layer_types)
    del model, w, state
    torch.cuda.empty_cache()
    return {"workload": f"40-layer target verify forward: T={tokens} over a {context}-token context, batch 1 "
                        "(30 GDN + 10 attention layers, 256 experts top-8 + shared, all projections, experts and "
                        "the LM head W4A16 g128 tiled; router bf16); embedding through LM head top-1",
            "us_total": round(full_ms * 1e3, 1), "us_per_layer": round((full_ms - head_ms) * 1e3 / c.layers, 1),
            "us_gdn_layer": round(gdn_ms * 1e3, 1), "us_attention_layer": round(attn_ms * 1e3, 1),
            "us_lm_head": round(head_ms * 1e3, 1), "gdn_layers": n_gdn, "attention_layers": c.layers - n_gdn,
            "us_kernels_only": round(kern_ms * 1e3, 1), "kernel_share": round(kern_ms / full_ms, 3),
            "steps": steps, "graph_period": 4}


def time_skewed(pkg, sets, device, top_k, steps, warmup, tokens=128, hot=16):
    """The T=128 layer (8 verify blocks) with 16 hot experts taking ~50% of the assignments.

    The bias b on the hot experts' logits is calibrated once on the first block's logits
    (``synthetic.hot_expert_bias``); each step computes the router logits, adds the bias and
    runs the layer on those logits (router, bias add and layer all timed).
    """
    gen = torch.Generator(device=device).manual_seed(128)
    blocks = [torch.randn((tokens, 2048), device=device, generator=gen).to(torch.bfloat16) for _ in range(4)]
    hot_ids = torch.randperm(256, generator=torch.Generator().manual_seed(7919))[:hot].to(device)
    base = pkg.ops.router_logits(blocks[0], sets[0][3])
    b = pkg.synthetic.hot_expert_bias(base, hot_ids, top_k)
    bias = torch.zeros(256, device=device)
    bias[hot_ids] = b
    ws = torch.empty(pkg.ops.moe_workspace_bytes(tokens, 2048, 512, 256, top_k, 128, True), dtype=torch.uint8,
                     device=device)
    hits, hot_frac = [], []
    for j in range(len(sets) * len(blocks)):
        gu, dn, sh, router = sets[j % len(sets)]
        lg = pkg.ops.router_logits(blocks[j % len(blocks)], router) + bias
        _, r, _ = pkg.ops.moe_w4a16(blocks[j % len(blocks)], gu, dn, top_k=top_k, router_logits=lg, shared=sh,
                                    workspace=ws, return_routing=True)
        hits.append(int((r.offsets[1:] > r.offsets[:-1]).sum().item()))
        hot_frac.append(float(torch.isin(r.ids.long(), hot_ids).float().mean().item()))

    def step(j):
        gu, dn, sh, router = sets[j % len(sets)]
        x = blocks[j % len(blocks)]
        pkg.ops.moe_w4a16(x, gu, dn, top_k=top_k, router_logits=pkg.ops.router_logits(x, router) + bias, shared=sh,
                          workspace=ws)
    ms = time_steps(step, steps, warmup)
    hit = statistics.mean(hits)
    int4 = (hit + 1) * INT4_BYTES_PER_EXPERT
    gbs = int4 / (ms * 1e-3) / 1e9
    return {"tokens": tokens, "hot_experts": hot, "bias": round(b, 4),
            "hot_assignment_frac": round(statistics.mean(hot_frac), 3), "hit_experts_mean": round(hit, 1),
            "us_per_layer": round(ms * 1e3, 2), "int4_bytes": int(int4), "int4_gbs": round(gbs, 1),
            "hbm_frac_int4": round(gbs / HBM_PEAK_GBS, 4), "steps": steps,
            "note": "router logits + bias add + layer per step, 3 rotated weight sets"}


def measured_mfma():
    """MFMA counters of the prefill gate/up tile kernel from the committed rocprofv3 passes, or None."""
    path = ROOT / "profiles" / "mfma_prefill_t2048.json"
    if not path.is_file():
        return None
    return json.loads(path.read_text())


def measured_traffic():
    """HBM bytes per T=16 gate/up launch (routing prologue) from the committed counter passes, or None."""
    path = ROOT / "profiles" / "hbm_traffic_gate_up_t16.json"
    if not path.is_file():
        return None
    rec = json.loads(path.read_text())
    return int(round((rec["fetch_kib"] * rec["fetch_scale"] + rec["write_kib"] * rec["write_scale"]) * 1024))


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_run(run, warmups=3, measured=10, budget_s=12.0):
    """Median wall time of `measured` runs after `warmups` (fewer if the budget runs out, at least 3)."""
    for _ in range(warmups):
        run()
    times, t_start = [], time.perf_counter()
    for _ in range(measured):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s and len(times) >= 3:
            break
    return statistics.median(times), len(times)


def cpu_baseline(pkg, sets, blocks, top_k):
    """The oracle's CPU restatement of the same T=16 layer, shared expert included, on the host,
    on the GPU leg's own tensors: hidden block 0 and weight set 0, the hit experts' banks copied
    to the host and taken back from the tiled to the portable order.

    Protocol: 3 warmups + 10 timed runs, median; torch intra-op threads = every CPU this
    process may run on.  ``value``: dense bf16 banks of the hit experts dequantised before the
    timed region (the reference ``moe`` takes dense logical banks).  Also reported: the same
    with every hit expert dequantised inside the timed call, and the single-qlinear workload
    (``[16,2048] x [512,2048]``, dense and dequant-inclusive).
    """
    import numpy as np
    from oracle import moe as oracle_moe, routing as oracle_routing, w4 as oracle_w4

    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    torch.set_num_threads(threads)
    gu_d, dn_d, sh_d, router = sets[0]
    hidden = blocks[0].cpu()
    tokens = hidden.shape[0]
    logits = oracle_moe.router_logits(hidden, router.cpu())
    ids, _ = oracle_routing.topk(logits, top_k)
    hit = np.unique(ids).tolist()

    def portable(bank, e=None):
        packed = bank.packed if e is None else bank.packed[e]
        scales = bank.scales if e is None else bank.scales[e]
        pk, sc = oracle_w4.from_tiled(packed.cpu().numpy(), scales.float().cpu().numpy())
        return torch.from_numpy(pk), torch.from_numpy(sc)

    host = {e: (portable(gu_d, e), portable(dn_d, e)) for e in hit}
    sh_host = (portable(sh_d.gate_up), portable(sh_d.down), sh_d.gate_weight.cpu())

    def deq(pair):
        return oracle_w4.dequantize_torch(pair[0], pair[1], 128)
    # dense bf16 banks, materialised for the hit experts only (the others are never read)
    gate_up = torch.zeros((gu_d.experts, gu_d.rows, gu_d.cols), dtype=torch.bfloat16)
    down = torch.zeros((dn_d.experts, dn_d.rows, dn_d.cols), dtype=torch.bfloat16)
    for e in hit:
        gate_up[e], down[e] = deq(host[e][0]), deq(host[e][1])
    shared_dense = (deq(sh_host[0]), deq(sh_host[1]), sh_host[2])
    layer_hidden = hidden
    dense_s, n_dense = _median_run(lambda: oracle_moe.moe_dense(layer_hidden, logits, top_k, gate_up, down,
                                                                  shared=shared_dense))
    fly_s, n_fly = _median_run(lambda: oracle_moe.moe_dense(
        layer_hidden, logits, top_k, None, None, dequantize=lambda e: (deq(host[e][0]), deq(host[e][1])),
        shared=(deq(sh_host[0]), deq(sh_host[1]), sh_host[2])))
    # config 1: the single W4A16 qlinear
    gen = torch.Generator().manual_seed(1)
    x1 = torch.randn((16, 2048), generator=gen).to(torch.bfloat16)
    w1 = pkg.synthetic.int4_weight(gen, (512, 2048), 128)
    w1_dense = deq((w1.packed, w1.scales))
    ql_s, _ = _median_run(lambda: torch.nn.functional.linear(x1, w1_dense), warmups=3, measured=10)
    ql_fly_s, _ = _median_run(lambda: torch.nn.functional.linear(x1, deq((w1.packed, w1.scales))), warmups=3,
                              measured=10)
    return {"value": round(dense_s * 1e6, 1), "unit": "us/layer", "cores": threads, "kind": "port",
            "cpu_model": _cpu_model(), "cpu_count": os.cpu_count(),
            "sample": f"oracle.moe.moe_dense: the GPU leg's T={tokens} layer (its hidden block 0 and weight set "
                      f"0, router logits given, top-{top_k} over 256 experts, {len(hit)} hit experts + the gated "
                      f"shared expert, fp32 combine) on dense bf16 banks dequantised before timing; median of "
                      f"{n_dense} runs after 3 warmups, torch threads={threads}",
            "dequant_inclusive_us": round(fly_s * 1e6, 1), "dequant_inclusive_runs": n_fly,
            "qlinear_config1_us": round(ql_s * 1e6, 1), "qlinear_config1_dequant_inclusive_us": round(ql_fly_s * 1e6, 1)}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--sets", type=int, default=3, help="independent weight sets rotated per step")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-qlinear", action="store_true")
    ap.add_argument("--no-stack", action="store_true")
    ap.add_argument("--no-config3", action="store_true")
    ap.add_argument("--only-stack", action="store_true", help="time the 40-layer stack only (no JSON metric line)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a plain 256 MiB device copy (reference dispatch for HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported (the MoE layer would shard by "
              "expert parallelism)", file=sys.stderr)
        return 2
    pkg = load_package()
    assert torch.cuda.is_available(), "bench.py needs a ROCm device"
    device = torch.device("cuda:0")
    pkg._lib.load()
    top_k, tokens = 8, 16
    if args.only_stack:
        print(json.dumps({"stack": time_stack(pkg, device, max(8, args.steps // 10), max(4, args.warmup // 5))}))
        return 0

    log("generating weight sets on the device")
    sets = weight_sets(pkg, args.sets, device)
    gen = torch.Generator(device=device).manual_seed(99)
    blocks = [torch.randn((tokens, 2048), device=device, generator=gen).to(torch.bfloat16) for _ in range(8)]
    ws = torch.empty(pkg.ops.moe_workspace_bytes(2048, 2048, 512, 256, top_k, 128, True), dtype=torch.uint8,
                     device=device)

    if args.calibrate_copy:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=device).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    log("timing the T=16 layer")
    ms = time_layer(pkg, sets, blocks, top_k, args.steps, args.warmup, ws)
    log("timing the expert stage")
    exp_ms, hits = time_experts(pkg, sets, blocks, top_k, args.steps, args.warmup, ws)
    int4_bytes = (hits + 1) * INT4_BYTES_PER_EXPERT
    all_bytes = (hits + 1) * (INT4_BYTES_PER_EXPERT + SCALE_BYTES_PER_EXPERT)
    layer_gbs = int4_bytes / (ms * 1e-3) / 1e9
    log("timing the expert kernels with HIP events")
    # the layer's dominant kernel: the gate/up launch that routes the block in its prologue
    # (measurement of GATE_UP with the step's logits relaunches exactly that kernel), then the
    # down launch, both together, and the gate/up stream alone (routing given as a work table)
    gu_ms, gu_hits, _ = time_stage(pkg, sets, blocks, top_k, args.steps, args.warmup, given_logits=True)
    two_ms, _, _ = time_stage(pkg, sets, blocks, top_k, args.steps, args.warmup, pkg.ops.STAGE_EXPERTS,
                              given_logits=True)
    stream_ms, _, _ = time_stage(pkg, sets, blocks, top_k, args.steps, args.warmup)
    dn_ms, _, _ = time_stage(pkg, sets, blocks, top_k, args.steps, args.warmup, pkg.ops.STAGE_DOWN)
    # the opt-in split-K down (the down GEMM inside the gate/up launch, partial rows added by the
    # combine): its layer and its one expert kernel
    log("timing the split-K down form")
    with pkg.ops.split_down(True):
        split = pkg.ops.moe_split_down(tokens, 2048, 512, 256, top_k, 128, True)
        split_layer_ms = time_layer(pkg, sets, blocks, top_k, args.steps, args.warmup, ws)
        split_ms, split_hits, split_parts = time_stage(pkg, sets, blocks, top_k, args.steps, args.warmup,
                                                       pkg.ops.STAGE_EXPERTS, given_logits=True)
    # algorithmic bytes of the gate/up launch: the hit experts' and the shared expert's int4 gate/up
    # rows + bf16 scales, x (bf16) read, h (bf16) written; of the split launch: gate/up and down
    # rows + scales, x read, the fp32 partial y rows written (h stays in LDS)
    rows = tokens * top_k + tokens
    gu_bytes = (gu_hits + 1) * GATE_UP_BYTES_PER_EXPERT + tokens * 2048 * 2 + rows * 512 * 2
    split_bytes = ((split_hits + 1) * (GATE_UP_BYTES_PER_EXPERT + DOWN_BYTES_PER_EXPERT) + tokens * 2048 * 2
                   + split_parts * 2048 * 4)
    achieved = gu_bytes / (gu_ms * 1e-3) / 1e9

    result = {
        "metric": METRIC, "value": round(ms * 1e3, 2), "unit": "us/layer", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded; int4 weights uniform in [-8,7], bf16 group-128 scales U(0.005,0.02), "
                "activations N(0,1); 3 rotated weight sets)",
        "config": {"workload": "routed MoE layer, DFlash verify block: T=16, H=2048, I=512, 256 experts top-8 "
                               "+ shared expert, W4A16 group 128, router included",
                   "tokens": tokens, "hidden": 2048, "inter": 512, "experts": 256, "top_k": top_k,
                   "group_size": 128, "weight_sets": args.sets},
        "layer_int4_gbs": round(layer_gbs, 1),
        "layer_hbm_frac_int4": round(layer_gbs / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "kernel": "w4_verify_kernel<1, 16, unsigned short> (routing prologue + grouped gate/up "
                               "+ SiLU*up, T=16, tiled banks)",
                     "kernel_us": round(gu_ms * 1e3, 2), "hit_experts_mean": round(gu_hits, 2),
                     "bytes_per_launch": int(gu_bytes)},
        "stages": {"expert_stage_us": round(exp_ms * 1e3, 2),
                   "expert_kernels_us": round(two_ms * 1e3, 2),
                   "gate_up_us": round(gu_ms * 1e3, 2),
                   "down_us": round(dn_ms * 1e3, 2),
                   "gate_up_stream_only_us": round(stream_ms * 1e3, 2),
                   "expert_int4_bytes": int(int4_bytes), "expert_weight_bytes": int(all_bytes),
                   "expert_stage_int4_gbs": round(int4_bytes / (exp_ms * 1e-3) / 1e9, 1)},
        "split_down_opt_in": {"runs": bool(split), "layer_us": round(split_layer_ms * 1e3, 2),
                              "kernel_us": round(split_ms * 1e3, 2),
                              "kernel_gbs": round(split_bytes / (split_ms * 1e-3) / 1e9, 1),
                              "partial_rows_mean": round(split_parts, 1), "bytes_per_launch": int(split_bytes)},
    }
    if not args.no_prefill:
        log("timing the T=2048 prefill layer")
        blocks_p = [torch.randn((2048, 2048), device=device, generator=gen).to(torch.bfloat16) for _ in range(2)]
        steps_p = max(5, args.steps // 10)
        ms_p = time_layer(pkg, sets, blocks_p, top_k, steps_p, max(2, args.warmup // 10), ws)
        tflops = moe_flops(2048, top_k) / (ms_p * 1e-3) / 1e12
        gu_p_ms, _, _ = time_stage(pkg, sets, blocks_p, top_k, steps_p, max(2, args.warmup // 10))
        dn_p_ms, _, _ = time_stage(pkg, sets, blocks_p, top_k, steps_p, max(2, args.warmup // 10),
                                   pkg.ops.STAGE_DOWN)
        gu_flops = 2 * (2048 * top_k + 2048) * 1024 * 2048
        gu_tf = gu_flops / (gu_p_ms * 1e-3) / 1e12
        result["prefill"] = {
            "tokens": 2048, "us_per_layer": round(ms_p * 1e3, 1), "tflops": round(tflops, 2),
            "mfma_frac": round(tflops / BF16_PEAK_TFLOPS, 4), "steps": steps_p,
            "roofline": {"bound": "mfma", "achieved": round(gu_tf, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(gu_tf / BF16_PEAK_TFLOPS, 4), "traffic": None,
                         "kernel": "w4_tile_kernel<1, unsigned short> (grouped gate/up + SiLU*up, T=2048, tiled)",
                         "kernel_us": round(gu_p_ms * 1e3, 2), "flops_per_launch": gu_flops,
                         "counters": measured_mfma()},
            "down_kernel_us": round(dn_p_ms * 1e3, 2),
            "down_kernel_tflops": round(2 * (2048 * top_k + 2048) * 2048 * 512 / (dn_p_ms * 1e-3) / 1e12, 1)}
    if not args.no_config3:
        log("timing the T=128 skewed layer")
        result["skewed_t128"] = time_skewed(pkg, sets, device, top_k, max(24, args.steps // 2), args.warmup)
    if not args.no_stack:
        log("timing the 40-layer verify stack")
        result["stack"] = time_stack(pkg, device, max(8, args.steps // 10), max(4, args.warmup // 5))
    if not args.no_qlinear:
        log("timing the qlinear projections and the LM head")
        result["qlinear"] = time_qlinear(pkg, device, max(24, args.steps // 2), args.warmup)
    if not args.no_cpu_baseline:
        log("timing the CPU baseline")
        result["cpu_baseline"] = cpu_baseline(pkg, sets, blocks, top_k)
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
