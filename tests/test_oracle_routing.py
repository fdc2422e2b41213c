"""CPU: pin the routing oracle (top-k, renormalised weights, stable permutation).

Checks: golden vectors from the pure-Python brute force (including exact ties,
-0.0 vs +0.0, -inf and an empty batch), agreement with torch.topk over
torch.softmax on tie-free rows (the reference's own selection,
reference/fused_ops.py:162-164), and invariants of the permutation.
"""
import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import routing

GOLDEN = json.loads((Path(__file__).resolve().parent / "golden" / "routing_golden.json").read_text())


def _decode(v):
    return {"-inf": -math.inf, "-0.0": -0.0}.get(v, v) if isinstance(v, str) else v


@pytest.mark.parametrize("case", range(len(GOLDEN)))
def test_golden(case):
    c = GOLDEN[case]
    logits = np.array([[_decode(v) for v in row] for row in c["logits"]], np.float32).reshape(-1, c["experts"])
    ids, w = routing.topk(logits, c["k"])
    np.testing.assert_array_equal(ids.reshape(-1), np.array(c["ids"], np.int32).reshape(-1))
    np.testing.assert_allclose(w.reshape(-1), np.array(c["weights"], np.float32).reshape(-1), rtol=0, atol=1e-7)
    perm, inv, offsets = routing.permutation(ids, c["experts"])
    np.testing.assert_array_equal(perm, np.array(c["perm"], np.int32))
    np.testing.assert_array_equal(inv, np.array(c["inv"], np.int32))
    np.testing.assert_array_equal(offsets, np.array(c["offsets"], np.int32))


def test_matches_torch_topk_on_tie_free_rows():
    rng = np.random.default_rng(1)
    logits = rng.standard_normal((512, 256)).astype(np.float32)
    probs = torch.softmax(torch.from_numpy(logits), dim=-1)
    vals, ref_ids = torch.topk(probs, 8, dim=-1)
    ref_w = (vals / vals.sum(-1, keepdim=True)).numpy()
    ids, w = routing.topk(logits, 8)
    checked = 0
    for t in range(logits.shape[0]):
        p = probs[t].numpy()
        kth, nxt = np.sort(p)[::-1][7:9]
        if kth == nxt or len(set(vals[t].tolist())) < 8:
            continue  # probability tie: torch.topk's order is unspecified
        checked += 1
        np.testing.assert_array_equal(ids[t], ref_ids[t].numpy())
        np.testing.assert_allclose(w[t], ref_w[t], rtol=1e-5)
    assert checked > 500


def test_invariants():
    rng = np.random.default_rng(2)
    logits = (rng.integers(-6, 6, (300, 64)) / 2).astype(np.float32)  # many ties
    ids, w = routing.topk(logits, 6)
    assert all(len(set(r)) == 6 for r in ids.tolist())
    np.testing.assert_allclose(w.sum(-1), 1.0, rtol=1e-6)
    for t in range(300):  # selection is the top of a descending order, lowest id first on ties
        sel = logits[t, ids[t]]
        assert np.all(np.diff(sel) <= 0)
        rest = np.setdiff1d(np.arange(64), ids[t])
        assert logits[t, rest].max() <= sel[-1]
        for a, b in zip(ids[t][:-1], ids[t][1:]):
            if logits[t, a] == logits[t, b]:
                assert a < b
    perm, inv, offsets = routing.permutation(ids, 64)
    flat = ids.reshape(-1)
    np.testing.assert_array_equal(np.sort(perm), np.arange(flat.size))
    np.testing.assert_array_equal(perm[inv], np.arange(flat.size))
    assert offsets[-1] == flat.size
    for e in range(64):
        seg = perm[offsets[e]:offsets[e + 1]]
        assert np.all(flat[seg] == e)
        assert np.all(np.diff(seg) > 0)  # stable: tokens ascending


def test_rejects_nan_and_bad_k():
    with pytest.raises(ValueError):
        routing.topk(np.array([[np.nan, 1.0]], np.float32), 1)
    with pytest.raises(ValueError):
        routing.topk(np.zeros((1, 4), np.float32), 5)
    with pytest.raises(ValueError):
        routing.topk(np.zeros((1, 4), np.float64), 1)
