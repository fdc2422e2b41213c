"""Packed int4 weight types and the host-side quantiser/packer.

Format (reference ``model/qwen35_moe_dflash/graph/quant_weights.py:19,138-148``;
``graph/quant_plan.py:76-87,165``): ``W[..., N, K]`` is stored as uint8
``[..., N, K/2]`` with signed two's-complement nibbles, ``k = 2j`` in the low
nibble of byte ``j``; scales are ``[..., N, K/G]`` (bf16 or fp32) and the
dequantised weight is ``q * scale[k // G]``.  The reference fixes ``G = 256``
and fp32 scales; here ``G`` is 128 or 256 and bf16 scales are accepted too
(W4A16 plan, ``reference/quantization.py:87-89``).

A bank may also be held in the *tiled* layout (``layout="tiled"``, made once by
``PackedW4.tiled()`` on the device): the same bytes and scales permuted so that
each 16-row tile and 128-column block is one contiguous kilobyte in the order
the expert kernels' 64 lanes load it, and scales are ``[..., N/16, K/G, 16]``
(byte-exact definition in ``include/dflash_hip.h``).  Tensor shapes are those
of the portable layout; only the order of the bytes differs.
"""
from __future__ import annotations

from typing import NamedTuple

import torch

GROUP_SIZES = (128, 256)
LAYOUTS = ("portable", "tiled")


class PackedW4(NamedTuple):
    """One packed matrix ``[N, K/2]`` or expert bank ``[E, N, K/2]`` with its group scales."""

    packed: torch.Tensor
    scales: torch.Tensor
    group_size: int
    layout: str = "portable"

    @property
    def experts(self) -> int:
        return self.packed.shape[0] if self.packed.ndim == 3 else 1

    @property
    def rows(self) -> int:
        return self.packed.shape[-2]

    @property
    def cols(self) -> int:
        return self.packed.shape[-1] * 2

    def validate(self, name: str = "weight") -> None:
        p, s, g = self.packed, self.scales, self.group_size
        if not isinstance(p, torch.Tensor) or not isinstance(s, torch.Tensor):
            raise ValueError(f"{name}: packed and scales must be tensors")
        if p.dtype != torch.uint8 or p.ndim not in (2, 3):
            raise ValueError(f"{name}: packed int4 must be uint8 [N, K/2] or [E, N, K/2]")
        if type(g) is not int or g not in GROUP_SIZES:
            raise ValueError(f"{name}: group_size must be one of {GROUP_SIZES}")
        if s.dtype not in (torch.bfloat16, torch.float32):
            raise ValueError(f"{name}: scales must be bfloat16 or float32")
        k = p.shape[-1] * 2
        if k % g or tuple(s.shape) != (*p.shape[:-1], k // g):
            raise ValueError(f"{name}: scales must be [..., N, K/{g}] for packed {tuple(p.shape)}")
        if p.device != s.device:
            raise ValueError(f"{name}: packed and scales on different devices")
        if not p.is_contiguous() or not s.is_contiguous():
            raise ValueError(f"{name}: packed and scales must be contiguous")
        if self.layout not in LAYOUTS:
            raise ValueError(f"{name}: layout must be one of {LAYOUTS}")
        if self.layout == "tiled" and (p.shape[-2] % 16 or k % 128):
            raise ValueError(f"{name}: the tiled layout needs N % 16 == 0 and K % 128 == 0")

    def to(self, device) -> "PackedW4":
        return PackedW4(self.packed.to(device), self.scales.to(device), self.group_size, self.layout)

    def tiled(self) -> "PackedW4":
        """This bank in the tiled layout (a one-time repack on its ROCm device)."""
        from .ops import to_tiled
        return to_tiled(self)


def concat_rows(*banks: PackedW4) -> PackedW4:
    """Matrices ``[N_i, K]`` that read the same activations, stacked into one ``[sum N_i, K]``
    so a single qlinear launch computes all of them (split its output at the ``N_i``).

    The tiled layout orders bytes per 16-row tile, so stacking tiled matrices whose row
    counts are multiples of 16 is a plain concatenation of their bytes and scales, like
    the portable one.  Every output column is computed from its own weight row as in a
    separate call; only the order in which a column's k-block partial sums are added can
    differ (the kernels split each workgroup's share of the stacked matrix over its waves),
    so results agree to fp32 rounding before the one bf16 rounding.
    """
    if not banks:
        raise ValueError("concat_rows needs at least one matrix")
    first = banks[0]
    for i, b in enumerate(banks):
        b.validate(f"bank {i}")
        if b.packed.ndim != 2:
            raise ValueError("concat_rows stacks 2-D matrices [N, K/2]")
        if (b.cols, b.group_size, b.layout, b.scales.dtype, b.packed.device) != (
                first.cols, first.group_size, first.layout, first.scales.dtype, first.packed.device):
            raise ValueError("concat_rows needs one K, group size, layout, scale dtype and device")
    return PackedW4(torch.cat([b.packed for b in banks]).contiguous(), torch.cat([b.scales for b in banks]).contiguous(),
                    first.group_size, first.layout)


class SharedExpert(NamedTuple):
    """Always-on shared expert: gate/up rows stacked ``[2I, H]``, down ``[H, I]``, gate vector ``[H]``.

    Output is ``down(silu(gate(x)) * up(x)) * sigmoid(x . gate_weight)``
    (reference ``fused/model.py:305-307``).
    """

    gate_up: PackedW4
    down: PackedW4
    gate_weight: torch.Tensor

    def tiled(self) -> "SharedExpert":
        """Both banks in the tiled layout."""
        return SharedExpert(self.gate_up.tiled(), self.down.tiled(), self.gate_weight)


def pack_int4(q: torch.Tensor) -> torch.Tensor:
    """int8 ``[..., K]`` in [-8, 7] -> uint8 ``[..., K/2]`` (even k in the low nibble)."""
    if q.dtype != torch.int8 or q.shape[-1] % 2:
        raise ValueError("pack_int4 needs int8 values with even K")
    nib = (q.to(torch.int16) & 15).to(torch.uint8)
    return (nib[..., 0::2] | (nib[..., 1::2] << 4)).contiguous()


def quantize_w4(weight: torch.Tensor, group_size: int = 128, scale_dtype: torch.dtype = torch.bfloat16) -> PackedW4:
    """Symmetric group quantisation of ``W[..., N, K]`` to the portable packed format.

    Same rule as ``graph/quant_weights.py:138-145``: fp32 statistics,
    ``scale = max|group| / 7`` (all-zero group -> 1), ``q = clip(rint(w / scale), -8, 7)``
    with ties to even.  With ``scale_dtype=bfloat16`` the scale is rounded to
    bf16 *before* the division, so ``q * scale`` uses exactly the stored scale.
    """
    if group_size not in GROUP_SIZES:
        raise ValueError(f"group_size must be one of {GROUP_SIZES}")
    w = weight.to(torch.float32)
    k = w.shape[-1]
    if k % group_size:
        raise ValueError("K must be a multiple of group_size")
    grouped = w.reshape(*w.shape[:-1], k // group_size, group_size)
    maxima = grouped.abs().amax(dim=-1)
    scale = torch.where(maxima == 0, torch.ones_like(maxima), maxima / 7.0)
    scale = scale.to(scale_dtype)
    q = torch.clamp(torch.round(grouped / scale.to(torch.float32)[..., None]), -8, 7).to(torch.int8)
    return PackedW4(pack_int4(q.reshape(w.shape)), scale.contiguous(), group_size)
