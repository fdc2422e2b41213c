"""Per-workgroup phase timeline of the expert kernels (profiling build).

``python timeline.py [--reps N] [--no-prefill]`` loads ``libdflash_hip_timeline.so``
(``python build.py --timeline``: the product kernels compiled with
``-DDFLASH_TIMELINE``, which record s_memrealtime ticks at 100 MHz), runs the
routed-MoE layer on device-generated random banks (H=2048, I=512, 256 experts
top-8 + shared expert, bf16 group-128 scales, tiled layout) and prints, as
markdown:

* T=16 verify block, gate/up and down launches (the layer's default separate
  launches): per phase the spread over workgroups of its time since the
  launch's first workgroup started, and per wave the median time its k-loop
  ended (waves w and w + 4 share a SIMD);
* T=2048 prefill, gate/up and down tile launches: work items per workgroup,
  the spread of workgroup end times, the median whole-tile duration by 16-row
  subtile count, the count and median duration of the pieces the last
  tiles are split into, and where a wave's time goes inside a work item
  (set-up, k-loop, epilogue).

The timestamps come from thread 0 (lane 0 of each wave for the k-loop ends)
after the workgroup's own stores have completed; they include the cost of the
timestamping itself (a few stores per workgroup).
"""
from __future__ import annotations

import argparse
import collections
import ctypes
import importlib.util
import sys
from pathlib import Path

import numpy as np
import torch

PKG_DIR = Path(__file__).resolve().parent
PKG_NAME = "qwen35_dflash_amd"
VERIFY_SLOTS = 16
WORKGROUPS = 1024
TILES = 8


def _package():
    if PKG_NAME in sys.modules:
        return sys.modules[PKG_NAME]
    spec = importlib.util.spec_from_file_location(PKG_NAME, PKG_DIR / "__init__.py",
                                                  submodule_search_locations=[str(PKG_DIR)])
    module = importlib.util.module_from_spec(spec)
    sys.modules[PKG_NAME] = module
    spec.loader.exec_module(module)
    return module


def _weights(pkg, device, seed=1234, hidden=2048, inter=512, experts=256):
    gen = torch.Generator(device=device).manual_seed(seed)
    bank = lambda shape: pkg.synthetic.device_bank(gen, shape, device)
    gu, dn = bank((experts, 2 * inter, hidden)), bank((experts, hidden, inter))
    sh = pkg.SharedExpert(bank((2 * inter, hidden)), bank((hidden, inter)),
                          (torch.randn((hidden,), device=device, generator=gen) * 0.02).to(torch.bfloat16))
    router = (torch.randn((experts, hidden), device=device, generator=gen) * 0.02).to(torch.bfloat16)
    return gu.tiled(), dn.tiled(), sh.tiled(), router


def _spread(ticks) -> str:
    v = np.asarray(ticks, dtype=np.float64) / 100.0
    if v.size == 0:
        return "-"
    p = np.percentile(v, [0, 50, 90, 100])
    return " | ".join(f"{x:.2f}" for x in p)


def verify_report(lib, pkg, device, reps: int) -> list[str]:
    gu, dn, sh, router = _weights(pkg, device)
    gen = torch.Generator(device=device).manual_seed(99)
    blocks = [torch.randn((16, 2048), device=device, generator=gen).to(torch.bfloat16) for _ in range(reps + 4)]
    ws = torch.empty(pkg.ops.moe_workspace_bytes(16, 2048, 512, 256, 8, 128, True), dtype=torch.uint8, device=device)
    buf = np.zeros(2 * WORKGROUPS * VERIFY_SLOTS, dtype=np.uint64)
    for x in blocks[:4]:
        pkg.ops.moe_w4a16(x, gu, dn, top_k=8, router_weight=router, shared=sh, workspace=ws)
    torch.cuda.synchronize()
    phases = {"gate/up": collections.defaultdict(list), "down": collections.defaultdict(list)}
    grid = 0
    for x in blocks[4:]:
        lib.dflash_timeline_clear()
        pkg.ops.moe_w4a16(x, gu, dn, top_k=8, router_weight=router, shared=sh, workspace=ws)
        torch.cuda.synchronize()
        if lib.dflash_timeline_read(0, buf.ctypes.data, buf.nbytes):
            raise RuntimeError("dflash_timeline_read failed")
        t = buf.reshape(2, WORKGROUPS, VERIFY_SLOTS).astype(np.int64)
        for m, name in enumerate(("gate/up", "down")):
            live = t[m, :, 0] > 0
            grid = int(live.sum())
            tm = t[m, live]
            t0 = tm[:, 0].min()
            for slot, label in ((0, "start"), (1, "passes known"), (2, "first chunk staged"),
                                (12, "partials exchanged"), (13, "end")):
                phases[name][label].extend((tm[:, slot] - t0).tolist())
            for w in range(8):
                phases[name][f"wave {w} k-loop done"].extend((tm[:, 4 + w] - t0).tolist())
            for x in range(8):
                phases[name][f"end, XCD {x}"].extend((tm[tm[:, 3] == x, 13] - t0).tolist())
    out = [f"### T=16 verify block ({reps} layer calls, {grid} workgroups per launch)", "",
           "Time since the launch's first workgroup started, over workgroups and calls (us): "
           "min | median | p90 | max.", ""]
    for name, rows in phases.items():
        out += [f"**{name} launch**", "", "| phase | min \\| median \\| p90 \\| max (us) |", "|---|---|"]
        for label in ("start", "passes known", "first chunk staged", *[f"wave {w} k-loop done" for w in range(8)],
                      "partials exchanged", "end", *[f"end, XCD {x}" for x in range(8)]):
            out.append(f"| {label} | {_spread(rows[label])} |")
        out.append("")
    return out


def tile_report(lib, pkg, device, reps: int) -> list[str]:
    gu, dn, sh, router = _weights(pkg, device)
    gen = torch.Generator(device=device).manual_seed(7)
    blocks = [torch.randn((2048, 2048), device=device, generator=gen).to(torch.bfloat16) for _ in range(2)]
    ws = torch.empty(pkg.ops.moe_workspace_bytes(2048, 2048, 512, 256, 8, 128, True), dtype=torch.uint8, device=device)
    buf = np.zeros(2 * WORKGROUPS * TILES * 3, dtype=np.uint64)
    cyc = np.zeros(2 * WORKGROUPS * TILES * 8 * 6, dtype=np.uint64)
    cyc_sum = np.zeros((2, 6), dtype=np.float64)
    for j in range(3):
        pkg.ops.moe_w4a16(blocks[j % 2], gu, dn, top_k=8, router_weight=router, shared=sh, workspace=ws)
    torch.cuda.synchronize()
    out = [f"### T=2048 prefill tile launches ({reps} layer calls)", ""]
    stats = {"gate/up": collections.defaultdict(list), "down": collections.defaultdict(list)}
    for r in range(reps):
        lib.dflash_timeline_clear()
        pkg.ops.moe_w4a16(blocks[r % 2], gu, dn, top_k=8, router_weight=router, shared=sh, workspace=ws)
        torch.cuda.synchronize()
        if lib.dflash_timeline_read(1, buf.ctypes.data, buf.nbytes):
            raise RuntimeError("dflash_timeline_read failed")
        if lib.dflash_timeline_read(2, cyc.ctypes.data, cyc.nbytes):
            raise RuntimeError("dflash_timeline_read failed")
        cyc_sum += cyc.reshape(2, -1, 6).astype(np.float64).sum(axis=1)
        t = buf.reshape(2, WORKGROUPS, TILES, 3).astype(np.int64)
        for m, name in enumerate(("gate/up", "down")):
            used = t[m, :, :, 2] > 0
            wgs = used.any(axis=1)
            st, en = t[m, :, :, 0], t[m, :, :, 1]
            t0 = st[used].min()
            s = stats[name]
            s["tiles"].append(int(used.sum()))
            s["span"].append(int(en[used].max() - t0))
            s["per_wg"].extend(used[wgs].sum(axis=1).tolist())
            s["wg_end"].extend((np.where(used, en, 0).max(axis=1)[wgs] - t0).tolist())
            rows = t[m, :, :, 2] & 0xFFFF
            piece = used & (((t[m, :, :, 2] >> 56) & 1) == 1)
            whole = used & ~piece
            for sub, d in zip(((rows[whole] + 15) // 16).tolist(), (en - st)[whole].tolist()):
                s[f"sub{sub}"].append(d)
            s["pieces"].append(int(piece.sum()))
            s["piece_us"].extend((en - st)[piece].tolist())
            # a workgroup's consecutive items: the queue claim between them
            nxt = used[:, 1:] & used[:, :-1]
            s["gap"].extend((st[:, 1:] - en[:, :-1])[nxt].tolist())
    for m, name in enumerate(stats):
        s = stats[name]
        ids, bar, first, loop, epi, n = cyc_sum[m]
        pro = ids + bar + first
        whole = loop + epi + pro
        hist = np.bincount(s["per_wg"])
        pieces = s["pieces"][0]
        out += [f"**{name} launch**: {s['tiles'][0]} work items ({s['tiles'][0] - pieces} whole tiles, {pieces} "
                f"pieces of split tiles), span {np.median(s['span']) / 100:.1f} us (median of calls)",
                "", f"- work items per workgroup (count of workgroups, over calls): "
                f"{ {i: int(c) for i, c in enumerate(hist) if c} }",
                f"- workgroup end (us): min | median | p90 | max = {_spread(s['wg_end'])}",
                "- median whole-tile duration by 16-row subtiles (us): " +
                ", ".join(f"{k[3:]}: {np.median(v) / 100:.1f} ({len(v) // reps} tiles)"
                          for k, v in sorted(s.items()) if k.startswith("sub")),
                f"- pieces: median {np.median(s['piece_us']) / 100 if s['piece_us'] else 0:.1f} us, "
                f"max {max(s['piece_us'], default=0) / 100:.1f} us",
                f"- a wave's time per work item (s_memtime cycles, summed over waves and items, {int(n)} "
                f"samples): set-up {pro / whole:.1%} (pass entry {ids / whole:.1%}, barrier with the row "
                f"id loads and the previous item's stores {bar / whole:.1%}, first stage loads "
                f"{first / whole:.1%}), "
                f"k-loop {loop / whole:.1%}, "
                f"epilogue {epi / whole:.1%}; mean item {whole / max(n, 1):.0f} cycles",
                f"- between a workgroup's consecutive items (the queue claim): median "
                f"{np.median(s['gap']) / 100 if s['gap'] else 0:.2f} us, p90 "
                f"{np.percentile(s['gap'], 90) / 100 if s['gap'] else 0:.2f} us", ""]
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--reps", type=int, default=6)
    ap.add_argument("--no-prefill", action="store_true")
    args = ap.parse_args(argv)
    pkg = _package()
    lib = pkg._lib.load(PKG_DIR / "libdflash_hip_timeline.so")
    lib.dflash_timeline_read.restype = ctypes.c_int
    lib.dflash_timeline_read.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t]
    lib.dflash_timeline_clear.restype = ctypes.c_int
    lib.dflash_timeline_clear.argtypes = []
    device = torch.device("cuda:0")
    lines = ["## Expert-kernel timeline (profiling build)", "",
             f"Device: {torch.cuda.get_device_name(device)}; `python qwen3.5-35b-dflash_amd/timeline.py"
             f" --reps {args.reps}{' --no-prefill' if args.no_prefill else ''}`.", ""]
    lines += verify_report(lib, pkg, device, args.reps)
    if not args.no_prefill:
        lines += tile_report(lib, pkg, device, max(2, args.reps // 2))
    print("\n".join(lines))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
