"""Oracle: fp64 comparison metrics for float outputs.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Cosine, relative-L2 and max-abs follow ``common/accuracy.py:49-127`` (all sums
in float64; two all-zero tensors give cosine 1 and relative-L2 0).  The parity
bar is the norm-relative maximum error ``max|a - g| / max|g|`` <= 1e-2, since an
elementwise relative error is undefined near zero.
"""
from __future__ import annotations

import math

import numpy as np
import torch

MAX_REL_TOLERANCE = 1e-2


def _f64(value) -> np.ndarray:
    if isinstance(value, torch.Tensor):
        return value.detach().cpu().to(torch.float64).numpy()
    return np.asarray(value, dtype=np.float64)


def compare(actual, golden) -> dict:
    a, g = _f64(actual), _f64(golden)
    if a.shape != g.shape:
        raise ValueError(f"shape mismatch {a.shape} vs {g.shape}")
    if not (np.isfinite(a).all() and np.isfinite(g).all()):
        return dict(finite=False, max_rel=math.inf, max_abs=math.inf, rel_l2=math.inf, cosine=0.0)
    delta = a - g
    gmax = float(np.abs(g).max()) if g.size else 0.0
    max_abs = float(np.abs(delta).max()) if g.size else 0.0
    gnorm, enorm = float(np.linalg.norm(g)), float(np.linalg.norm(delta))
    anorm = float(np.linalg.norm(a))
    if anorm and gnorm:
        cosine = float(np.sum(a * g) / anorm / gnorm)
    else:
        cosine = 1.0 if anorm == gnorm == 0.0 else 0.0
    return dict(finite=True,
                max_rel=(max_abs / gmax) if gmax else (0.0 if max_abs == 0 else math.inf),
                max_abs=max_abs,
                rel_l2=(enorm / gnorm) if gnorm else (0.0 if enorm == 0 else math.inf),
                cosine=cosine)
