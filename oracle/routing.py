"""Oracle: router top-k with renormalised weights, stable expert permutation.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Selection (``reference/fused_ops.py:161-164``, ``graph/fused/quant_target.py:168-172``,
``fused/quantization.py:184-186``): fp32 softmax over all experts, top-k, selected
probabilities divided by their sum.  Softmax is strictly monotone, so ranking
the fp32 *logits* gives the same order; ties (equal logits) go to the lowest
expert id, which makes the result a function of the logits alone (``torch.topk``
has no documented tie order).  The renormalised weights need only the selected
logits because the full-softmax denominator cancels:
``w_i = exp(l_i - l_max) / sum_sel exp(l_j - l_max)``.

Permutation (``npu_moe_init_routing_v2`` contract, reference
``docs/reference/qwen35-moe-operators-and-quantization-analysis.md:685-707``;
call site ``fused/quantization.py:188-192``): the ``T*k`` (token, slot) pairs,
flattened as ``t*k + slot``, are sorted by expert id, stably, so each expert's
segment lists its tokens in ascending order.  ``perm[j]`` is the flat pair at
sorted position ``j``; ``inv[t*k + slot]`` is its sorted position;
``offsets[e] .. offsets[e+1]`` is expert ``e``'s segment (``tokens_per_expert``
is ``diff(offsets)``).

Pinning: the pure-Python brute force in ``tests/golden/make_golden.py``
(``sorted`` on ``(-logit, id)`` keys and explicit bucket loops) writes the
``routing_golden.json`` vectors, including rows with exact ties; agreement
with ``torch.topk`` over ``torch.softmax`` on tie-free rows; invariants
(distinct ids, weights sum to 1, segments contiguous and ascending).
"""
from __future__ import annotations

import numpy as np


def topk(logits: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray]:
    """fp32 logits ``[T, E]`` -> (ids int32 ``[T, k]`` by descending logit, weights fp32 ``[T, k]``)."""
    logits = np.asarray(logits)
    if logits.dtype != np.float32 or logits.ndim != 2:
        raise ValueError("router logits must be float32 [T, E]")
    t, e = logits.shape
    if not 0 < k <= e:
        raise ValueError("top_k must lie in (0, E]")
    if np.isnan(logits).any():
        raise ValueError("router logits must not contain NaN")
    # Stable ascending sort of the negated logits == descending order with the
    # lowest expert id first among equal logits (-0.0 and +0.0 compare equal).
    order = np.argsort(-logits, axis=-1, kind="stable")[:, :k]
    ids = order.astype(np.int32)
    chosen = np.take_along_axis(logits, order, axis=-1).astype(np.float64)
    if t:
        shifted = np.exp(chosen - chosen[:, :1])
        weights = (shifted / shifted.sum(-1, keepdims=True)).astype(np.float32)
    else:
        weights = np.zeros((0, k), np.float32)
    return ids, weights


def permutation(ids: np.ndarray, num_experts: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """ids ``[T, k]`` -> (perm int32 ``[T*k]``, inv int32 ``[T*k]``, offsets int32 ``[E+1]``)."""
    flat = np.asarray(ids).reshape(-1).astype(np.int64)
    if flat.size and (flat.min() < 0 or flat.max() >= num_experts):
        raise ValueError("expert id out of range")
    perm = np.argsort(flat, kind="stable").astype(np.int32)
    inv = np.empty_like(perm)
    inv[perm] = np.arange(flat.size, dtype=np.int32)
    counts = np.bincount(flat, minlength=num_experts)
    offsets = np.concatenate(([0], np.cumsum(counts))).astype(np.int32)
    return perm, inv, offsets
