"""PyTorch-ROCm wrappers over the C ABI of ``libdflash_hip.so``.

Tensors must live on a ROCm device; every call is enqueued on the current
torch stream of that device, allocates its outputs and workspace through
torch, and raises :class:`DflashError` with the library's message on any
nonzero status.  There is no CPU or dense fallback (reference policy,
``model/qwen35_moe_dflash/fused/ops.py:133-135``).
"""
from __future__ import annotations

import contextlib
import ctypes
from typing import NamedTuple, Optional

import torch

from . import _lib
from .packing import PackedW4, SharedExpert


class Routing(NamedTuple):
    """Device routing of ``T`` tokens over ``E`` experts (see ``include/dflash_hip.h``)."""

    ids: torch.Tensor        # int32 [T, k]
    weights: torch.Tensor    # fp32 [T, k]
    perm: torch.Tensor       # int32 [T*k]
    inv: torch.Tensor        # int32 [T*k]
    offsets: torch.Tensor    # int32 [E+1]


def _require_device(*tensors) -> torch.device:
    device = None
    for t in tensors:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
            raise ValueError("mi355x-hip operations require tensors on a ROCm device")
        if device is None:
            device = t.device
        elif t.device != device:
            raise ValueError("all tensors must be on the same device")
    if device is None:
        raise ValueError("no tensor given")
    return device


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _desc(w: PackedW4) -> _lib.W4Desc:
    return _lib.W4Desc(
        packed=w.packed.data_ptr(), scales=w.scales.data_ptr(), experts=w.experts, rows=w.rows, cols=w.cols,
        group_size=w.group_size,
        scale_dtype=_lib.DTYPE_F32 if w.scales.dtype == torch.float32 else _lib.DTYPE_BF16,
        layout=_lib.LAYOUT_TILED if w.layout == "tiled" else _lib.LAYOUT_PORTABLE)


def _workspace(nbytes: int, device: torch.device, workspace: Optional[torch.Tensor]) -> torch.Tensor:
    if workspace is not None:
        if workspace.dtype != torch.uint8 or workspace.numel() < nbytes or workspace.device != device:
            raise ValueError(f"workspace must be a uint8 tensor of at least {nbytes} bytes on {device}")
        return workspace
    return torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)


_SOURCE_SCALE_DTYPES = {torch.float32: _lib.DTYPE_F32, torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16}


def from_int8(values: torch.Tensor, scales: torch.Tensor, group_size: int, *, layout: str = "tiled") -> PackedW4:
    """Pack the original checkpoint's int8-carried int4 weights into a bank with fp32 scales.

    ``values`` int8 ``[N, K]`` or ``[E, N, K]`` in [-8, 7]; ``scales`` fp16/fp32/bf16
    ``[..., N, K/G]`` (a linear's ``[N, K/G, 1]`` is accepted, as the reference's
    reader stores it: ``target/original_quant.py:214-240``).  Raises ``ValueError``
    with the reader's messages for values outside [-8, 7] and for negative or
    non-finite scales (``:252-272``); synchronises the stream to check them, as a
    load-time step.
    """
    device = _require_device(values, scales)
    if values.dtype != torch.int8 or values.ndim not in (2, 3):
        raise ValueError("original quantized weights must be int8 [N, K] or [E, N, K]")
    if layout not in ("portable", "tiled"):
        raise ValueError("layout must be 'portable' or 'tiled'")
    *lead, n, k = values.shape
    if k % group_size:
        raise ValueError(f"K={k} is not a multiple of group_size={group_size}")
    sc = scales.reshape(*scales.shape[:-1]) if scales.ndim == values.ndim + 1 and scales.shape[-1] == 1 else scales
    if tuple(sc.shape) != (*lead, n, k // group_size) or sc.dtype not in _SOURCE_SCALE_DTYPES:
        raise ValueError(f"scales must be fp16/fp32/bf16 [{', '.join(map(str, (*lead, n, k // group_size)))}]")
    vals, sc = values.contiguous(), sc.contiguous()
    packed = torch.empty((*lead, n, k // 2), dtype=torch.uint8, device=device)
    out_scales = torch.empty((*lead, n, k // group_size), dtype=torch.float32, device=device)
    invalid = torch.empty(2, dtype=torch.int32, device=device)
    _lib.call("dflash_w4_from_int8", _ptr(vals), _ptr(sc), _SOURCE_SCALE_DTYPES[sc.dtype], lead[0] if lead else 1,
              n, k, group_size, _lib.LAYOUT_TILED if layout == "tiled" else _lib.LAYOUT_PORTABLE, _ptr(packed),
              _ptr(out_scales), _ptr(invalid), _stream(device))
    bad_values, bad_scales = (int(v) for v in invalid.cpu())
    if bad_values:
        raise ValueError("original quantized weight contains values outside signed I4 [-8,7]")
    if bad_scales:
        raise ValueError("original quantization scales must be finite and nonnegative")
    return PackedW4(packed, out_scales, group_size, layout)


def to_tiled(w: PackedW4) -> PackedW4:
    """Repack a portable bank into the tiled layout (new tensors, same shapes, on w's device)."""
    w.validate("weight")
    if w.layout != "portable":
        raise ValueError("to_tiled needs a portable bank")
    device = _require_device(w.packed)
    packed = torch.empty_like(w.packed)
    scales = torch.empty_like(w.scales)
    desc = _desc(w)
    _lib.call("dflash_w4_to_tiled", ctypes.byref(desc), _ptr(packed), _ptr(scales), _stream(device))
    return PackedW4(packed, scales, w.group_size, "tiled")


def qlinear(x: torch.Tensor, weight: PackedW4, *, workspace: Optional[torch.Tensor] = None,
            out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """W4A16 linear ``x[..., K] -> [..., N]`` (bf16 in, fp32 accumulation; bf16 out, or the
    unrounded fp32 sums with ``out_dtype=torch.float32``)."""
    weight.validate("weight")
    if weight.packed.ndim != 2:
        raise ValueError("qlinear takes one packed matrix [N, K/2]")
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("qlinear writes bfloat16 or float32")
    device = _require_device(x, weight.packed)
    if x.dtype != torch.bfloat16 or x.shape[-1] != weight.cols:
        raise ValueError(f"x must be bfloat16 [..., {weight.cols}]")
    flat = x.reshape(-1, weight.cols).contiguous()
    m = flat.shape[0]
    out = torch.empty((m, weight.rows), dtype=out_dtype, device=device)
    lib = _lib.load()
    ws = _workspace(lib.dflash_qlinear_workspace_bytes(m, weight.cols, weight.group_size), device, workspace)
    desc = _desc(weight)
    entry = "dflash_qlinear_w4a16_f32" if out_dtype == torch.float32 else "dflash_qlinear_w4a16"
    _lib.call(entry, _ptr(flat), m, ctypes.byref(desc), _ptr(out), _ptr(ws), ws.numel(), _stream(device))
    return out.reshape(*x.shape[:-1], weight.rows)


def router_logits(hidden: torch.Tensor, router_weight: torch.Tensor) -> torch.Tensor:
    """fp32 ``[T, E]`` logits from bf16 ``hidden [..., H]`` and bf16 ``router_weight [E, H]``."""
    device = _require_device(hidden, router_weight)
    if hidden.dtype != torch.bfloat16 or router_weight.dtype != torch.bfloat16:
        raise ValueError("router needs bfloat16 hidden and router_weight")
    if router_weight.ndim != 2 or router_weight.shape[1] != hidden.shape[-1]:
        raise ValueError("router_weight must be [E, H]")
    flat = hidden.reshape(-1, hidden.shape[-1]).contiguous()
    w = router_weight.contiguous()
    logits = torch.empty((flat.shape[0], w.shape[0]), dtype=torch.float32, device=device)
    _lib.call("dflash_router_logits", _ptr(flat), flat.shape[0], flat.shape[1], _ptr(w), w.shape[0], _ptr(logits),
              _stream(device))
    return logits


def _routing_buffers(t: int, e: int, k: int, device) -> Routing:
    return Routing(
        ids=torch.empty((t, k), dtype=torch.int32, device=device),
        weights=torch.empty((t, k), dtype=torch.float32, device=device),
        perm=torch.empty((t * k,), dtype=torch.int32, device=device),
        inv=torch.empty((t * k,), dtype=torch.int32, device=device),
        offsets=torch.empty((e + 1,), dtype=torch.int32, device=device))


def route(logits: torch.Tensor, top_k: int, *, workspace: Optional[torch.Tensor] = None) -> Routing:
    """Top-k routing and stable expert permutation from fp32 logits ``[T, E]``."""
    device = _require_device(logits)
    if logits.dtype != torch.float32 or logits.ndim != 2:
        raise ValueError("router logits must be float32 [T, E]")
    if type(top_k) is not int:
        raise ValueError("top_k must be an int")
    logits = logits.contiguous()
    t, e = logits.shape
    r = _routing_buffers(t, e, top_k, device)
    lib = _lib.load()
    ws = _workspace(lib.dflash_moe_route_workspace_bytes(t, e, top_k), device, workspace)
    _lib.call("dflash_moe_route", _ptr(logits), t, e, top_k, _ptr(r.ids), _ptr(r.weights), _ptr(r.perm),
              _ptr(r.inv), _ptr(r.offsets), _ptr(ws), ws.numel(), _stream(device))
    return r


def _shared_args(shared: Optional[SharedExpert]):
    if shared is None:
        return None, None, None, None
    if not isinstance(shared, SharedExpert):
        raise ValueError("shared must be a SharedExpert")
    shared.gate_up.validate("shared.gate_up")
    shared.down.validate("shared.down")
    gw = shared.gate_weight
    if gw.dtype != torch.bfloat16:
        raise ValueError("shared.gate_weight must be bfloat16 [H]")
    gw = gw.reshape(-1).contiguous()
    return _desc(shared.gate_up), _desc(shared.down), gw, (shared.gate_up.packed, shared.down.packed)


def _moe_common(hidden, gate_up: PackedW4, down: PackedW4, shared):
    gate_up.validate("gate_up")
    down.validate("down")
    if gate_up.packed.ndim != 3 or down.packed.ndim != 3:
        raise ValueError("expert banks must be [E, N, K/2]")
    device = _require_device(hidden, gate_up.packed, down.packed)
    if hidden.dtype != torch.bfloat16:
        raise ValueError("hidden must be bfloat16")
    h = hidden.shape[-1]
    flat = hidden.reshape(-1, h).contiguous()
    sgu, sdn, sgate, keep = _shared_args(shared)
    if keep is not None:
        _require_device(hidden, *keep, sgate)
    return device, flat, sgu, sdn, sgate


def _check_routing(routing: Routing, t: int, e: int, device: torch.device) -> int:
    """Validate a caller-given routing against the layer (the kernels index with it); returns top_k."""
    if not isinstance(routing, Routing):
        raise ValueError("routing must be a Routing (ids, weights, perm, inv, offsets)")
    ids = routing.ids
    if not isinstance(ids, torch.Tensor) or ids.ndim != 2 or ids.shape[0] != t:
        raise ValueError(f"routing.ids must be int32 [{t}, k]")
    k = ids.shape[1]
    if not 0 < k <= e:
        raise ValueError(f"routing top_k must be in (0, {e}]")
    expected = {"ids": (torch.int32, (t, k)), "weights": (torch.float32, (t, k)), "perm": (torch.int32, (t * k,)),
                "inv": (torch.int32, (t * k,)), "offsets": (torch.int32, (e + 1,))}
    for name, (dtype, shape) in expected.items():
        v = getattr(routing, name)
        if (not isinstance(v, torch.Tensor) or v.dtype != dtype or tuple(v.shape) != shape
                or v.device != device or not v.is_contiguous()):
            raise ValueError(f"routing.{name} must be a contiguous {dtype} {list(shape)} tensor on {device}")
    return k


def moe_experts(hidden: torch.Tensor, routing: Routing, gate_up: PackedW4, down: PackedW4, *,
                shared: Optional[SharedExpert] = None, workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Expert FFN + combine for a given routing (as ``route`` returns it); bf16 ``[T, H]``.

    The routing's arrays are checked for device, dtype, shape and contiguity;
    their values are trusted (a routing not made by ``route`` must satisfy its
    invariants: a permutation, offsets ascending from 0 to T*k).
    """
    device, flat, sgu, sdn, sgate = _moe_common(hidden, gate_up, down, shared)
    t, h = flat.shape
    k = _check_routing(routing, t, gate_up.experts, device)
    out = torch.empty_like(flat)
    lib = _lib.load()
    ws = _workspace(lib.dflash_moe_workspace_bytes(t, h, gate_up.rows // 2, gate_up.experts, k, gate_up.group_size,
                                                   int(shared is not None)), device, workspace)
    gu, dn = _desc(gate_up), _desc(down)
    _lib.call("dflash_moe_experts_w4a16", _ptr(flat), t, h, k, _ptr(routing.weights),
              _ptr(routing.perm), _ptr(routing.inv), _ptr(routing.offsets), ctypes.byref(gu), ctypes.byref(dn),
              None if sgu is None else ctypes.byref(sgu), None if sdn is None else ctypes.byref(sdn), _ptr(sgate),
              _ptr(out), _ptr(ws), ws.numel(), _stream(device))
    return out


def moe_w4a16(hidden: torch.Tensor, gate_up: PackedW4, down: PackedW4, *, top_k: int,
              router_weight: Optional[torch.Tensor] = None, router_logits: Optional[torch.Tensor] = None,
              shared: Optional[SharedExpert] = None, workspace: Optional[torch.Tensor] = None,
              return_routing: bool = False):
    """Whole routed-MoE layer (+ optional shared expert) on packed banks; bf16 ``[T, H]``.

    With ``return_routing=True`` also returns ``(Routing, logits)``; ``logits``
    are the fp32 router logits the routing was computed from.
    """
    device, flat, sgu, sdn, sgate = _moe_common(hidden, gate_up, down, shared)
    if type(top_k) is not int:
        raise ValueError("top_k must be an int")
    t, h = flat.shape
    e = gate_up.experts
    if router_logits is not None:
        _require_device(router_logits)
        if router_logits.dtype != torch.float32 or tuple(router_logits.shape) != (t, e):
            raise ValueError(f"router_logits must be float32 [{t}, {e}]")
        logits_in = router_logits.contiguous()
        logits_out = logits_in
    else:
        if router_weight is None:
            raise ValueError("router_weight or router_logits is required")
        _require_device(router_weight)
        if router_weight.dtype != torch.bfloat16 or tuple(router_weight.shape) != (e, h):
            raise ValueError(f"router_weight must be bfloat16 [{e}, {h}]")
        logits_in = None
        logits_out = torch.empty((t, e), dtype=torch.float32, device=device)
    rw = None if router_weight is None else router_weight.contiguous()
    r = _routing_buffers(t, e, top_k, device)
    out = torch.empty_like(flat)
    lib = _lib.load()
    ws = _workspace(lib.dflash_moe_workspace_bytes(t, h, gate_up.rows // 2, e, top_k, gate_up.group_size,
                                                   int(shared is not None)), device, workspace)
    gu, dn = _desc(gate_up), _desc(down)
    _lib.call("dflash_moe_w4a16", _ptr(flat), t, h, _ptr(logits_in), _ptr(rw), top_k, ctypes.byref(gu),
              ctypes.byref(dn), None if sgu is None else ctypes.byref(sgu), None if sdn is None else ctypes.byref(sdn),
              _ptr(sgate), _ptr(out), _ptr(logits_out if logits_in is None else None), _ptr(r.ids), _ptr(r.weights),
              _ptr(r.perm), _ptr(r.inv), _ptr(r.offsets), _ptr(ws), ws.numel(), _stream(device))
    if return_routing:
        return out, r, logits_out
    return out


NOALLOC_SCRATCH_BYTES = 8 << 20


def moe_w4a16_noalloc(hidden: torch.Tensor, gate_up: PackedW4, down: PackedW4, *, top_k: int,
                      router_weight: Optional[torch.Tensor] = None, router_logits: Optional[torch.Tensor] = None,
                      shared: Optional[SharedExpert] = None, out: Optional[torch.Tensor] = None,
                      routing: Optional[Routing] = None, logits_out: Optional[torch.Tensor] = None):
    """``moe_w4a16`` through ``dflash_moe_w4a16_noalloc``: no workspace, the library's static scratch.

    The library allocates nothing; this wrapper allocates the outputs only when the caller
    does not pass them (``out`` bf16 ``[T, H]``, ``routing`` buffers, ``logits_out`` fp32
    ``[T, E]``).  Returns ``(out, routing, logits)``.  Layers needing more than
    ``NOALLOC_SCRATCH_BYTES`` of scratch raise :class:`DflashError`.
    """
    device, flat, sgu, sdn, sgate = _moe_common(hidden, gate_up, down, shared)
    if type(top_k) is not int:
        raise ValueError("top_k must be an int")
    t, h = flat.shape
    e = gate_up.experts
    if router_logits is not None:
        _require_device(router_logits)
        if router_logits.dtype != torch.float32 or tuple(router_logits.shape) != (t, e):
            raise ValueError(f"router_logits must be float32 [{t}, {e}]")
        router_logits = router_logits.contiguous()
        logits_out = router_logits
    else:
        if router_weight is None:
            raise ValueError("router_weight or router_logits is required")
        _require_device(router_weight)
        if router_weight.dtype != torch.bfloat16 or tuple(router_weight.shape) != (e, h):
            raise ValueError(f"router_weight must be bfloat16 [{e}, {h}]")
        router_weight = router_weight.contiguous()
        if logits_out is None:
            logits_out = torch.empty((t, e), dtype=torch.float32, device=device)
        elif (logits_out.dtype != torch.float32 or tuple(logits_out.shape) != (t, e) or logits_out.device != device
              or not logits_out.is_contiguous()):
            raise ValueError(f"logits_out must be a contiguous float32 [{t}, {e}] tensor on {device}")
    if routing is None:
        routing = _routing_buffers(t, e, top_k, device)
    elif _check_routing(routing, t, e, device) != top_k:
        raise ValueError("routing buffers must hold top_k slots per token")
    if out is None:
        out = torch.empty_like(flat)
    elif out.dtype != torch.bfloat16 or tuple(out.shape) != (t, h) or out.device != device or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous bfloat16 [{t}, {h}] tensor on {device}")
    gu, dn = _desc(gate_up), _desc(down)
    r = routing
    _lib.call("dflash_moe_w4a16_noalloc", _ptr(flat), t, h, _ptr(router_logits), _ptr(router_weight), top_k,
              ctypes.byref(gu), ctypes.byref(dn), None if sgu is None else ctypes.byref(sgu),
              None if sdn is None else ctypes.byref(sdn), _ptr(sgate), _ptr(out),
              None if router_logits is not None else _ptr(logits_out), _ptr(r.ids), _ptr(r.weights), _ptr(r.perm),
              _ptr(r.inv), _ptr(r.offsets), _stream(device))
    return out, routing, logits_out


def qlinear_workspace_bytes(m: int, k: int, group_size: int = 128) -> int:
    return int(_lib.load().dflash_qlinear_workspace_bytes(m, k, group_size))


def moe_workspace_bytes(tokens: int, hidden: int, inter: int, experts: int, top_k: int, group_size: int,
                        has_shared: bool) -> int:
    return int(_lib.load().dflash_moe_workspace_bytes(tokens, hidden, inter, experts, top_k, group_size,
                                                      int(has_shared)))


_split_down = False  # the library's process-wide switch, as last set through set_split_down


def set_split_down(enable: bool) -> None:
    """Process-wide: run a verify block's down GEMM inside its gate/up launch where it fits
    (opt-in; off, the default, runs the separate down launch)."""
    global _split_down
    _lib.call("dflash_set_split_down", int(bool(enable)))
    _split_down = bool(enable)


@contextlib.contextmanager
def split_down(enable: bool):
    """Sets the split-K down switch for a block of calls and restores the previous setting."""
    prev = _split_down
    set_split_down(enable)
    try:
        yield
    finally:
        set_split_down(prev)


@contextlib.contextmanager
def tile_pieces(pieces: int):
    """Forces the prefill tile kernels' tail split (1, 2 or 4 pieces) for a block of calls,
    then restores the grid-chosen default."""
    _lib.call("dflash_set_tile_pieces", int(pieces))
    try:
        yield
    finally:
        _lib.call("dflash_set_tile_pieces", 0)


def moe_split_down(tokens: int, hidden: int, inter: int, experts: int, top_k: int, group_size: int,
                   has_shared: bool, scale_dtype: torch.dtype = torch.bfloat16, layout: str = "tiled") -> bool:
    """Whether a ``moe_w4a16`` call of this shape runs the split-K down on the current device."""
    return bool(_lib.load().dflash_moe_split_down(
        tokens, hidden, inter, experts, top_k, group_size, int(has_shared),
        _lib.DTYPE_F32 if scale_dtype == torch.float32 else _lib.DTYPE_BF16,
        _lib.LAYOUT_TILED if layout == "tiled" else _lib.LAYOUT_PORTABLE))


STAGE_GATE_UP = _lib.STAGE_GATE_UP
STAGE_DOWN = _lib.STAGE_DOWN
STAGE_EXPERTS = _lib.STAGE_EXPERTS


def set_measure_stage(stage: int) -> None:
    """Measurement mode: later MoE calls launch only ``stage``'s kernel (0 restores full calls).

    The kernel reuses what an earlier full call with the same arguments left
    in the same workspace; the layer output is not written.
    """
    _lib.call("dflash_set_measure_stage", int(stage))
