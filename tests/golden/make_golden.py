"""Write the golden vectors that pin the oracle (pure Python, no numpy/torch).

Independent restatement: bit-level nibble handling on Python ints, exact
``fractions.Fraction`` arithmetic for the W4A16 dot products, ``sorted`` with
explicit ``(-logit, id)`` keys for routing, explicit bucket loops for the
permutation, and a scalar bf16 rounding helper.  None of it imports the
oracle or the product.  Sources of each rule (reference files):

* nibble order / quantiser: ``model/qwen35_moe_dflash/graph/quant_weights.py:138-148``
* routing: ``reference/fused_ops.py:160-164`` with fp32-logit ranking, lowest id on ties
* permutation: ``docs/reference/qwen35-moe-operators-and-quantization-analysis.md:685-707``
* MoE: ``reference/fused_ops.py:165-173``, ``target/prefill_t64/cpu_reference.py:160-181``,
  ``fused/model.py:305-307``

Run ``python tests/golden/make_golden.py`` to regenerate; outputs are small
JSON files beside this script.
"""
from __future__ import annotations

import json
import math
import random
import struct
from fractions import Fraction
from pathlib import Path

HERE = Path(__file__).resolve().parent


# ---------------------------------------------------------------- scalar helpers
def f32(value: float) -> float:
    return struct.unpack("<f", struct.pack("<f", value))[0]


def bf16(value: float) -> float:
    """Round a Python float to the nearest bf16 (ties to even) through its fp32 bits."""
    bits = struct.unpack("<I", struct.pack("<f", value))[0]
    lsb = (bits >> 16) & 1
    bits = (bits + 0x7FFF + lsb) & 0xFFFF0000
    return struct.unpack("<f", struct.pack("<I", bits))[0]


def rint_even(value: float) -> int:
    floor = math.floor(value)
    frac = value - floor
    if frac > 0.5 or (frac == 0.5 and floor % 2 == 1):
        return floor + 1
    return floor


def nibble(byte: int, high: bool) -> int:
    raw = (byte >> 4) & 15 if high else byte & 15
    return raw - 16 if raw >= 8 else raw


def pack_row(values: list[int]) -> list[int]:
    out = []
    for j in range(0, len(values), 2):
        out.append((values[j] & 15) | ((values[j + 1] & 15) << 4))
    return out


def unpack_row(row: list[int]) -> list[int]:
    out = []
    for byte in row:
        out.append(nibble(byte, False))
        out.append(nibble(byte, True))
    return out


def silu(v: float) -> float:
    return v / (1.0 + math.exp(-v))


# ---------------------------------------------------------------- W4 vectors
def w4_vectors(rng: random.Random) -> dict:
    # Every nibble value in both positions of one byte.
    nibble_table = []
    for low in range(-8, 8):
        for high in range(-8, 8):
            nibble_table.append([low, high, pack_row([low, high])[0]])
    # Quantiser known answers: groups of 4 values with hand-checkable results.
    groups = [
        [0.0, 0.0, 0.0, 0.0],              # zero group -> scale 1, q 0
        [7.0, -7.0, 3.5, -3.5],            # scale 1; 3.5 -> 4 and -3.5 -> -4 (ties to even)
        [1.4, 0.1, -0.3, 0.7],             # scale 0.2
        [-14.0, 2.0, 5.0, 1.0],            # scale 2; -14/2 = -7, 5/2 = 2.5 -> 2 (ties to even)
        [0.25, -0.5, 0.125, 1.75],         # scale 0.25; 0.125/0.25 = 0.5 -> 0
    ]
    quant = []
    for g in groups:
        g32 = [f32(v) for v in g]
        maxima = max(abs(v) for v in g32)
        scale = 1.0 if maxima == 0 else f32(maxima / 7.0)
        q = [max(-8, min(7, rint_even(f32(v / scale)))) for v in g32]
        quant.append(dict(values=g32, scale=scale, q=q))
    # Tiny qlinear cases with bf16-exact inputs, exact expected outputs.
    linear_cases = []
    for (m, n, k, g) in [(1, 1, 8, 8), (2, 3, 16, 8), (3, 4, 32, 16), (4, 2, 24, 8)]:
        q = [[rng.randint(-8, 7) for _ in range(k)] for _ in range(n)]
        scales = [[bf16(rng.choice([0.5, 0.25, 0.0078125, 1.5, 0.01171875, 3.0])) for _ in range(k // g)]
                  for _ in range(n)]
        x = [[bf16(rng.randint(-64, 64) / 16.0) for _ in range(k)] for _ in range(m)]
        packed = [pack_row(row) for row in q]
        assert all(unpack_row(p) == row for p, row in zip(packed, q))
        y = []
        for mi in range(m):
            out_row = []
            for ni in range(n):
                acc = Fraction(0)
                for gi in range(k // g):
                    dot = sum(Fraction(x[mi][kk]) * q[ni][kk] for kk in range(gi * g, (gi + 1) * g))
                    acc += dot * Fraction(scales[ni][gi])
                out_row.append(float(acc))
            y.append(out_row)
        linear_cases.append(dict(m=m, n=n, k=k, group=g, x=x, packed=packed, scales=scales, y=y))
    return dict(nibble_table=nibble_table, quantize=quant, qlinear=linear_cases)


# ---------------------------------------------------------------- routing vectors
def route_row(logits: list[float], k: int) -> tuple[list[int], list[float]]:
    keyed = sorted(range(len(logits)), key=lambda e: (-logits[e], e))[:k]
    top = logits[keyed[0]]
    exps = [math.exp(logits[e] - top) for e in keyed]
    total = sum(exps)
    return keyed, [f32(v / total) for v in exps]


def permutation(ids: list[list[int]], experts: int) -> tuple[list[int], list[int], list[int]]:
    buckets = [[] for _ in range(experts)]
    k = len(ids[0]) if ids else 0
    for t, row in enumerate(ids):
        for s, e in enumerate(row):
            buckets[e].append(t * k + s)
    perm = [flat for bucket in buckets for flat in bucket]
    inv = [0] * len(perm)
    for pos, flat in enumerate(perm):
        inv[flat] = pos
    offsets = [0]
    for bucket in buckets:
        offsets.append(offsets[-1] + len(bucket))
    return perm, inv, offsets


def routing_vectors(rng: random.Random) -> list[dict]:
    cases = []
    # Hand-made rows with exact ties, negative zero and infinities.
    cases.append(dict(experts=6, k=3, logits=[[1.0, 2.0, 2.0, 0.0, 2.0, 2.0],
                                             [0.0, -0.0, 0.0, -0.0, 1.0, -1.0],
                                             [-1.0, -1.0, -1.0, -1.0, -1.0, -1.0],
                                             [5.0, -math.inf, 4.0, 5.0, 3.0, 4.0]]))
    cases.append(dict(experts=8, k=8, logits=[[f32(rng.gauss(0, 1)) for _ in range(8)] for _ in range(3)]))
    # A 256-expert block of 16 tokens with values drawn from a coarse grid so ties occur.
    cases.append(dict(experts=256, k=8,
                      logits=[[rng.randint(-40, 40) / 8.0 for _ in range(256)] for _ in range(16)]))
    # 64 tokens over 32 experts, k=4, continuous values.
    cases.append(dict(experts=32, k=4, logits=[[f32(rng.gauss(0, 2)) for _ in range(32)] for _ in range(64)]))
    # No tokens at all.
    cases.append(dict(experts=16, k=2, logits=[]))
    for case in cases:
        rows = [route_row(row, case["k"]) for row in case["logits"]]
        case["ids"] = [r[0] for r in rows]
        case["weights"] = [r[1] for r in rows]
        perm, inv, offsets = permutation(case["ids"], case["experts"])
        case.update(perm=perm, inv=inv, offsets=offsets)
        case["logits"] = [[("-inf" if v == -math.inf else ("-0.0" if v == 0 and math.copysign(1, v) < 0 else v))
                           for v in row] for row in case["logits"]]
    return cases


# ---------------------------------------------------------------- MoE vectors
def moe_vector(rng: random.Random) -> dict:
    tokens, hidden, inter, experts, k, group = 5, 16, 8, 4, 2, 8

    def bank(rows, cols):
        q = [[[rng.randint(-8, 7) for _ in range(cols)] for _ in range(rows)] for _ in range(experts)]
        s = [[[bf16(rng.choice([0.03125, 0.0625, 0.046875, 0.09375])) for _ in range(cols // group)]
              for _ in range(rows)] for _ in range(experts)]
        return q, s

    gu_q, gu_s = bank(2 * inter, hidden)
    dn_q, dn_s = bank(hidden, inter)
    sh_gu_q = [[rng.randint(-8, 7) for _ in range(hidden)] for _ in range(2 * inter)]
    sh_gu_s = [[0.0625 for _ in range(hidden // group)] for _ in range(2 * inter)]
    sh_dn_q = [[rng.randint(-8, 7) for _ in range(inter)] for _ in range(hidden)]
    sh_dn_s = [[0.03125 for _ in range(inter // group)] for _ in range(hidden)]
    sh_gate = [bf16(rng.randint(-8, 8) / 32.0) for _ in range(hidden)]
    x = [[bf16(rng.randint(-32, 32) / 16.0) for _ in range(hidden)] for _ in range(tokens)]
    logits = [[f32(rng.gauss(0, 1)) for _ in range(experts)] for _ in range(tokens)]
    ids, weights = zip(*[route_row(row, k) for row in logits])

    def matvec(qm, sm, vec):
        out = []
        for row_q, row_s in zip(qm, sm):
            acc = 0.0
            for kk, v in enumerate(vec):
                acc += v * row_q[kk] * row_s[kk // group]
            out.append(acc)
        return out

    def ffn(vec, guq, gus, dnq, dns):
        gu = matvec(guq, gus, vec)
        h = [bf16(silu(gu[i]) * gu[inter + i]) for i in range(inter)]
        return matvec(dnq, dns, h)

    out_routed, out_total = [], []
    for t in range(tokens):
        acc = [0.0] * hidden
        for s in range(k):
            e = ids[t][s]
            y = ffn(x[t], gu_q[e], gu_s[e], dn_q[e], dn_s[e])
            for i in range(hidden):
                acc[i] += weights[t][s] * y[i]
        out_routed.append(list(acc))
        shared = ffn(x[t], sh_gu_q, sh_gu_s, sh_dn_q, sh_dn_s)
        gate = 1.0 / (1.0 + math.exp(-sum(a * b for a, b in zip(x[t], sh_gate))))
        out_total.append([acc[i] + gate * shared[i] for i in range(hidden)])
    return dict(tokens=tokens, hidden=hidden, inter=inter, experts=experts, k=k, group=group,
                x=x, logits=logits,
                gate_up_packed=[[pack_row(r) for r in e] for e in gu_q], gate_up_scales=gu_s,
                down_packed=[[pack_row(r) for r in e] for e in dn_q], down_scales=dn_s,
                shared_gate_up_packed=[pack_row(r) for r in sh_gu_q], shared_gate_up_scales=sh_gu_s,
                shared_down_packed=[pack_row(r) for r in sh_dn_q], shared_down_scales=sh_dn_s,
                shared_gate=sh_gate, ids=[list(r) for r in ids], weights=[list(r) for r in weights],
                out_routed=out_routed, out_total=out_total)


def main() -> None:
    rng = random.Random(20261201)
    (HERE / "w4_golden.json").write_text(json.dumps(w4_vectors(rng)) + "\n")
    (HERE / "routing_golden.json").write_text(json.dumps(routing_vectors(rng)) + "\n")
    (HERE / "moe_golden.json").write_text(json.dumps(moe_vector(rng)) + "\n")


if __name__ == "__main__":
    main()
