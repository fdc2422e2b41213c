"""Oracle: portable K-packed int4 weights, group quantiser, W4A16 linear.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Format (reference ``graph/quant_weights.py:19,147-148``,
``graph/quant_plan.py:76-87,165``): a logical weight ``W[..., N, K]`` is stored
as ``uint8[..., N, K/2]``; byte ``j`` of a row holds signed two's-complement
nibbles ``q[2j]`` in bits 0-3 and ``q[2j+1]`` in bits 4-7.  Scales are
``[..., N, K/G]``, one per group of ``G`` consecutive K values; the dequantised
weight is ``q[n, k] * s[n, k // G]``.

The *tiled* layout (this build's own streaming order, defined in
``include/dflash_hip.h``; no counterpart in the reference) is restated by
``to_tiled``: per ``[..., 16-row tile t, 128-column block b]`` one kilobyte whose
16-byte chunk ``l`` is bytes ``64 b + 16 (l // 16) ..+15`` of row ``16 t + l % 16``;
scales ``[..., N/16, K/G, 16]``.

Pinning: ``to_tiled`` by a per-byte brute force of that definition on small
banks and by ``from_tiled`` (its inverse) round trips; ``pack``/``unpack`` by brute force over all 16 nibble values in both
positions and by the hand-written known-answer bytes in
``tests/golden/w4_golden.json``; ``quantize`` by the known-answer groups in the
same file (written by an independent pure-Python restatement); ``qlinear`` by
an exact ``fractions.Fraction`` brute force on tiny shapes, by closed forms
(one-hot and all-ones activations) and by a float64 matmul at full size.
"""
from __future__ import annotations

import numpy as np
import torch


def quantize(weight: torch.Tensor, group_size: int) -> tuple[np.ndarray, np.ndarray]:
    """Symmetric int4 group quantiser; returns ``(q int8 [...,N,K], scale f32 [...,N,K/G])``.

    Follows ``graph/quant_weights.py:138-145``: statistics in float32,
    ``scale = max|group| / 7`` with an all-zero group given scale 1,
    ``q = clip(rint(w / scale), -8, 7)`` (``rint`` rounds ties to even).
    The reference fixes ``G = 256`` (``quant_weights.py:76-77``); here ``G`` is a
    parameter because the W4A16 plan allows 128 or 256
    (``reference/quantization.py:87-89``).
    """
    values = weight.detach().to(torch.float32).cpu().numpy()
    k = values.shape[-1]
    if group_size <= 0 or k % group_size:
        raise ValueError("K must be a positive multiple of group_size")
    grouped = values.reshape(*values.shape[:-1], k // group_size, group_size)
    maxima = np.max(np.abs(grouped), axis=-1)
    scale = (maxima / np.float32(7)).astype(np.float32)
    scale[maxima == 0] = np.float32(1)
    q = np.clip(np.rint(grouped / scale[..., None]), -8, 7).astype(np.int8)
    return q.reshape(values.shape), scale


def pack(q: np.ndarray) -> np.ndarray:
    """int8 ``[..., K]`` in [-8, 7] -> uint8 ``[..., K/2]``, even k in the low nibble."""
    q = np.asarray(q)
    if q.dtype != np.int8 or q.shape[-1] % 2:
        raise ValueError("pack needs int8 values with an even K")
    if q.size and (q.min() < -8 or q.max() > 7):
        raise ValueError("int4 values must lie in [-8, 7]")
    nibbles = q.astype(np.uint8) & np.uint8(15)
    return (nibbles[..., 0::2] | (nibbles[..., 1::2] << np.uint8(4))).astype(np.uint8)


def unpack(packed: np.ndarray) -> np.ndarray:
    """uint8 ``[..., K/2]`` -> int8 ``[..., K]`` (sign-extended two's-complement nibbles)."""
    packed = np.asarray(packed)
    if packed.dtype != np.uint8:
        raise ValueError("unpack needs uint8 bytes")
    low = (packed & np.uint8(15)).astype(np.int16)
    high = (packed >> np.uint8(4)).astype(np.int16)
    out = np.empty((*packed.shape[:-1], packed.shape[-1] * 2), dtype=np.int16)
    out[..., 0::2] = low
    out[..., 1::2] = high
    out[out >= 8] -= 16
    return out.astype(np.int8)


def _scales_f32(scales) -> np.ndarray:
    if isinstance(scales, torch.Tensor):
        return scales.detach().to(torch.float32).cpu().numpy()
    return np.asarray(scales, dtype=np.float32)


def dequantize(packed, scales, group_size: int) -> np.ndarray:
    """Exact float32 weights ``q * s`` (a 4-bit by 8/24-bit product is exact in float32)."""
    if isinstance(packed, torch.Tensor):
        packed = packed.cpu().numpy()
    q = unpack(packed).astype(np.float32)
    s = _scales_f32(scales)
    k = q.shape[-1]
    if k % group_size or s.shape != (*q.shape[:-1], k // group_size):
        raise ValueError("scales must be [..., N, K/G]")
    return q * np.repeat(s, group_size, axis=-1)


def dequantize_torch(packed: torch.Tensor, scales: torch.Tensor, group_size: int,
                     dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """``dequantize`` with torch CPU ops (multi-threaded), rounded to ``dtype``: the form the CPU
    baseline times when it dequantises experts on the fly.  Equal to ``dequantize`` in float32."""
    low = (packed & 15).to(torch.int8)
    high = (packed >> 4).to(torch.int8)
    q = torch.stack((low, high), dim=-1).reshape(*packed.shape[:-1], packed.shape[-1] * 2)
    q = torch.where(q >= 8, q - 16, q).to(torch.float32)
    s = scales.to(torch.float32).repeat_interleave(group_size, dim=-1)
    return (q * s).to(dtype)


def qlinear(x: torch.Tensor, packed, scales, group_size: int, *, accumulate: str = "fp64") -> np.ndarray:
    """W4A16 linear ``y[m, n] = sum_k x[m, k] * q[n, k] * s[n, k // G]`` as float64/float32.

    The group-scaled dot structure follows ``target/layer_probe/qlinear_math.py:73-118``
    with the activation kept in its bf16 value (A16, no dynamic quant,
    ``specs/dflash-contract.json:104-113``).  ``accumulate="fp64"`` is the golden;
    ``"fp32"`` is the fp32-accumulated variant.
    """
    w = dequantize(packed, scales, group_size)
    xv = x.detach().to(torch.float32).cpu().numpy()
    if accumulate == "fp64":
        return xv.astype(np.float64) @ w.astype(np.float64).T
    if accumulate == "fp32":
        return (torch.from_numpy(xv) @ torch.from_numpy(w).T).numpy()
    raise ValueError("accumulate must be fp64 or fp32")


def to_tiled(packed: np.ndarray, scales: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Portable ``packed [..., N, K/2]``, ``scales [..., N, K/G]`` -> the tiled order, same shapes."""
    packed = np.asarray(packed)
    scales = np.asarray(scales)
    *lead, n, half = packed.shape
    k = half * 2
    if n % 16 or k % 128:
        raise ValueError("the tiled layout needs N % 16 == 0 and K % 128 == 0")
    groups = scales.shape[-1]
    # [..., t, r, b, q, 16 bytes] -> [..., t, b, q, r, 16 bytes]: chunk l = 16 q + r
    chunks = packed.reshape(*lead, n // 16, 16, k // 128, 4, 16)
    tiled = np.moveaxis(chunks, -4, -2).reshape(packed.shape)
    s = scales.reshape(*lead, n // 16, 16, groups)
    tiled_s = np.swapaxes(s, -1, -2).reshape(scales.shape)
    return np.ascontiguousarray(tiled), np.ascontiguousarray(tiled_s)


def from_tiled(packed: np.ndarray, scales: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Inverse of ``to_tiled``."""
    packed = np.asarray(packed)
    scales = np.asarray(scales)
    *lead, n, half = packed.shape
    k = half * 2
    groups = scales.shape[-1]
    chunks = packed.reshape(*lead, n // 16, k // 128, 4, 16, 16)
    portable = np.moveaxis(chunks, -2, -4).reshape(packed.shape)
    s = scales.reshape(*lead, n // 16, groups, 16)
    portable_s = np.swapaxes(s, -1, -2).reshape(scales.shape)
    return np.ascontiguousarray(portable), np.ascontiguousarray(portable_s)


def from_int8(values: np.ndarray, scales: np.ndarray, *, tiled: bool) -> tuple[np.ndarray, np.ndarray]:
    """The original checkpoint's int8-carried int4 ``values [..., N, K]`` and group
    ``scales [..., N, K/G]`` (fp16/fp32; a linear's trailing ``[.., 1]`` axis dropped)
    -> ``(packed uint8 [..., N, K/2], scales float32)``, in the tiled order when asked.

    Follows the checks of ``target/original_quant.py:252-272`` (values in [-8, 7],
    scales finite and nonnegative, same messages); the packing is ``pack`` (the same
    nibble order the reader's I4ZN packer uses inside each byte, ``:107-109``) and the
    scale widening is exact.  Pinned by its parts: ``pack``, ``to_tiled``, and the
    ``unpack`` round trip in the tests.
    """
    values = np.asarray(values)
    scales = np.asarray(scales)
    if values.dtype != np.int8:
        raise ValueError("logical original quantized weights must have dtype int8")
    if np.any(values < -8) or np.any(values > 7):
        raise ValueError("original quantized weight contains values outside signed I4 [-8,7]")
    if scales.ndim == values.ndim + 1 and scales.shape[-1] == 1:
        scales = scales[..., 0]
    wide = scales.astype(np.float32)
    if not np.isfinite(wide).all() or np.any(wide < 0):
        raise ValueError("original quantization scales must be finite and nonnegative")
    packed = pack(values)
    return to_tiled(packed, wide) if tiled else (packed, wide)

