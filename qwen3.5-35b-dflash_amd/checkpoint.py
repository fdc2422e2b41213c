"""Readers of the reference's two on-disk int4 weight formats, onto this library's banks.

* **Original quantized checkpoint** (``target/original_quant.py:18-45,153-276``):
  ``data*.safetensors`` shards that carry, per packed projection or expert bank,
  ``<stem>_quant_weight`` int8 ``[..., N, K]`` (one int4 value in [-8, 7] per
  byte) and ``<stem>_quant_scale`` fp16/fp32 group-256 scales (``[E, N, K/256]``
  for expert banks, ``[N, K/256, 1]`` for linears).  :class:`OriginalShards`
  validates the shard headers the way the reference's reader does (prefix
  length, one JSON object, no duplicate keys within or across shards, known
  dtypes, extents that fit the file and do not overlap), maps the tensors
  read-only, and :meth:`OriginalShards.bank` packs them on the GPU in one pass
  (``dflash_w4_from_int8``: fp32 scales, portable or tiled order, the reader's
  range checks).  The reference packs the same values into its vendor I4ZN
  carrier instead (``pack_i4zn``, ``:80-112``).
* **Portable logical cache** (``graph/quant_prepare.py:103-199``, payloads
  written by ``graph/quant_weights.py:110-178``): ``manifest.json``,
  ``plan.json``, one ``tensors/NNNNN.json`` record per tensor and its
  ``weights/NNNNN.weight.bin`` / ``.scale.bin`` payloads -- int4 already in this
  library's portable byte order (``uint8 [..., K/2]``, even k in the low nibble)
  and fp32 ``[..., K/256]`` scales, row-major little-endian.
  :class:`PortableCache` checks the manifest's record files and each record's
  own hash (``quant_prepare.py:22-24,192-197``), then the payloads' sizes and
  SHA-256 (``common/artifacts.py:59-65``) as a tensor is loaded;
  :meth:`PortableCache.bank` returns the bank as stored or tiled.

Both raise ``ValueError`` with the reference readers' messages where a check
fails.  Host-side parsing needs no GPU; the banks are built on the device of the
caller's choice (packing and tiling are kernels of this library).
"""
from __future__ import annotations

import hashlib
import json
import math
import re
import struct
from pathlib import Path
from typing import Iterable, Mapping, Optional

import numpy as np
import torch

from . import ops, plan
from .packing import PackedW4

ORIGINAL_GROUP_SIZE = 256
# safetensors dtype widths the reader accepts in a header, and the ones it maps
_WIDTHS = {"BOOL": 1, "U8": 1, "I8": 1, "I16": 2, "U16": 2, "I32": 4, "U32": 4, "I64": 8, "U64": 8,
           "F16": 2, "BF16": 2, "F32": 4, "F64": 8}
_NUMPY = {"I8": np.dtype("i1"), "F16": np.dtype("<f2"), "F32": np.dtype("<f4")}
# original checkpoint names: projections lose their ".weight", expert banks keep their name
_ORIGINAL_LINEARS = frozenset(s[:-len(".weight")] for s in plan.LINEAR_SUFFIXES)
_CHECK_CHUNK = 1 << 20


def original_keys(key: str) -> tuple[str, str]:
    """Target tensor name -> (``<stem>_quant_weight``, ``<stem>_quant_scale``) of the original
    checkpoint (``target/original_quant.py:30-45``)."""
    if key == "target.lm_head.weight":
        stem = "lm_head"
    else:
        m = re.fullmatch(r"target\.layers\.([0-9]+)\.(.+)", key)
        if m is None:
            raise ValueError(f"not an original target quantized weight: {key}")
        suffix = m[2]
        if suffix.endswith(".weight") and suffix[:-len(".weight")] in _ORIGINAL_LINEARS:
            suffix = suffix[:-len(".weight")]
        elif suffix not in plan.EXPERT_SUFFIXES:
            raise ValueError(f"not an original target quantized weight: {key}")
        stem = f"model.layers.{m[1]}.{suffix}"
    return stem + "_quant_weight", stem + "_quant_scale"


def _no_duplicates(pairs):
    out = {}
    for k, v in pairs:
        if k in out:
            raise ValueError("duplicate safetensors JSON key: " + k)
        out[k] = v
    return out


def _stamp(path: Path):
    st = path.stat()
    return (st.st_dev, st.st_ino, st.st_size, st.st_mtime_ns)


def _shape(shape) -> tuple:
    shape = tuple(shape)
    if len(shape) not in (2, 3) or any(type(x) is not int or x <= 0 for x in shape):
        raise ValueError("weight shape must have positive integer dimensions and rank two or three")
    return shape


class OriginalShards:
    """Read-only view of an original quantized checkpoint directory (``data*.safetensors``)."""

    def __init__(self, root):
        self.root = Path(root).resolve()
        paths = sorted(self.root.glob("data*.safetensors"))
        if not 0 < len(paths) <= 4096:
            raise ValueError("original quantized directory must contain 1..4096 data*.safetensors shards")
        self.tensors: dict[str, dict] = {}
        self._stamps: dict[str, tuple] = {}
        for named in paths:
            path = named.resolve()
            if named.is_symlink() or self.root not in path.parents or not path.is_file():
                raise ValueError("quantized shard must be a regular file inside the supplied directory")
            stamp = _stamp(path)
            with path.open("rb") as f:
                prefix = f.read(8)
                if len(prefix) != 8:
                    raise ValueError(f"{path.name}: truncated safetensors prefix")
                n = struct.unpack("<Q", prefix)[0]
                if not 2 <= n <= min(32 << 20, stamp[2] - 8):
                    raise ValueError(f"{path.name}: invalid safetensors header length")
                header = json.loads(f.read(n), object_pairs_hook=_no_duplicates)
            if not isinstance(header, dict):
                raise ValueError(f"{path.name}: safetensors header must be an object")
            start, extents = 8 + n, []
            for key, spec in header.items():
                if key == "__metadata__":
                    continue
                if key in self.tensors:
                    raise ValueError(f"duplicate quantized tensor across shards: {key}")
                if not isinstance(spec, dict):
                    raise ValueError(f"{key}: invalid safetensors tensor descriptor")
                dtype, shape, offsets = spec.get("dtype"), spec.get("shape"), spec.get("data_offsets")
                if (not isinstance(dtype, str) or dtype not in _WIDTHS or not isinstance(shape, list)
                        or any(type(x) is not int or x < 0 for x in shape) or not isinstance(offsets, list)
                        or len(offsets) != 2 or any(type(x) is not int for x in offsets)):
                    raise ValueError(f"{key}: invalid dtype, shape or offsets")
                begin, end = offsets
                size = math.prod(shape) * _WIDTHS[dtype]
                if begin < 0 or end < begin or end - begin != size or start + end > stamp[2]:
                    raise ValueError(f"{key}: invalid safetensors data extent")
                if size:
                    extents.append((begin, end, key))
                self.tensors[key] = {"shard": path.name, "dtype": dtype, "shape": list(shape),
                                     "offset": start + begin, "bytes": size}
            last = 0
            for begin, end, key in sorted(extents):
                if begin < last:
                    raise ValueError(f"{key}: overlapping safetensors data extents")
                last = end
            if _stamp(path) != stamp:
                raise ValueError("quantized shard changed while reading its header")
            self._stamps[path.name] = stamp

    def _unchanged(self, names: Iterable[str]) -> None:
        for name in set(names):
            if _stamp(self.root / name) != self._stamps[name]:
                raise ValueError(f"quantized shard changed since header validation: {name}")

    def describe(self, key: str, shape) -> dict:
        """Validate the weight/scale pair of ``key`` (logical ``shape``) from the headers alone
        (``target/original_quant.py:196-227``)."""
        shape = _shape(shape)
        wkey, skey = original_keys(key)
        expert = key.endswith(tuple(plan.EXPERT_SUFFIXES))
        if len(shape) != (3 if expert else 2):
            raise ValueError(f"{key}: rank does not match linear/expert role")
        n, k = shape[-2:]
        if k % ORIGINAL_GROUP_SIZE or n % 16:
            raise ValueError(f"{key}: group-256 I4ZN requires K%256=0 and N%16=0")
        sshape = (*shape[:-1], k // ORIGINAL_GROUP_SIZE) if expert else (n, k // ORIGINAL_GROUP_SIZE, 1)
        for name, expect, types in ((wkey, shape, {"I8"}), (skey, sshape, {"F16", "F32"})):
            rec = self.tensors.get(name)
            if rec is None:
                raise ValueError("original quantized tensor missing: " + name)
            if tuple(rec["shape"]) != expect or rec["dtype"] not in types:
                raise ValueError(f"{name}: expected {list(expect)} with dtype in {sorted(types)}")
        w, s = self.tensors[wkey], self.tensors[skey]
        self._unchanged((w["shard"], s["shard"]))
        return {"key": key, "shape": list(shape), "expert": expert, "weight": dict(w), "scale": dict(s)}

    def _map(self, rec: dict) -> np.ndarray:
        return np.memmap(self.root / rec["shard"], mode="r", dtype=_NUMPY[rec["dtype"]], offset=rec["offset"],
                         shape=tuple(rec["shape"]))

    def logical(self, key: str, shape) -> tuple[np.ndarray, np.ndarray]:
        """Read-only int8 values and float scales of ``key``, range-checked on the host in chunks
        (``target/original_quant.py:243-257``): values in [-8, 7], scales finite and >= 0."""
        meta = self.describe(key, shape)
        weight, scale = self._map(meta["weight"]), self._map(meta["scale"])
        for arr, is_scale in ((weight, False), (scale, True)):
            flat = arr.reshape(-1)
            for i in range(0, flat.size, _CHECK_CHUNK):
                v = flat[i:i + _CHECK_CHUNK]
                if is_scale:
                    if not np.isfinite(v).all() or np.any(v < 0):
                        raise ValueError("original quantization scales must be finite and nonnegative")
                elif np.any(v < -8) or np.any(v > 7):
                    raise ValueError("original quantized weight contains values outside signed I4 [-8,7]")
        self._unchanged((meta["weight"]["shard"], meta["scale"]["shard"]))
        return weight, scale

    def bank(self, key: str, shape, device, *, layout: str = "tiled") -> PackedW4:
        """The packed bank of ``key`` on ``device``: int8 values and scales copied as they are,
        packed by ``dflash_w4_from_int8`` (its range checks raise the reader's ``ValueError``s)."""
        meta = self.describe(key, shape)
        weight, scale = self._map(meta["weight"]), self._map(meta["scale"])
        values = torch.from_numpy(np.array(weight, copy=True)).to(device)   # the maps are read-only
        scales = torch.from_numpy(np.array(scale, copy=True)).to(device)
        self._unchanged((meta["weight"]["shard"], meta["scale"]["shard"]))
        return ops.from_int8(values, scales, ORIGINAL_GROUP_SIZE, layout=layout)


# ------------------------------------------------------------------ portable cache
CACHE_KIND = "qwen35-portable-quant-weights"
CACHE_STATUS = "WEIGHTS_PREPARED_LAYOUT_PENDING"
INT4_FORMAT = "PORTABLE_LOGICAL_INT4_ROW_MAJOR_LOW_NIBBLE_FIRST"
INT8_FORMAT = "PORTABLE_LOGICAL_INT8_ROW_MAJOR"
SCALE_FORMAT = "LOGICAL_SCALES_ROW_MAJOR_FP32_LE"


def record_identity(value) -> str:
    """SHA-256 of the canonical JSON text of ``value`` (``graph/quant_prepare.py:22-24``)."""
    return hashlib.sha256(json.dumps(value, sort_keys=True, separators=(",", ":"),
                                     allow_nan=False).encode()).hexdigest()


def _sha256(path: Path) -> str:
    h = hashlib.sha256()
    with path.open("rb") as f:
        for block in iter(lambda: f.read(8 << 20), b""):
            h.update(block)
    return h.hexdigest()


def _checked_file(root: Path, item: Mapping, *, verify: bool = True) -> Path:
    """A payload or record named by ``item`` ({path, bytes, sha256}) inside ``root``, of that size
    and hash (``common/artifacts.py:59-65``)."""
    path = (root / item["path"]).resolve()
    if root not in path.parents or not path.is_file():
        raise ValueError(f"artifact missing or escapes bundle: {item['path']}")
    if path.stat().st_size != item["bytes"] or (verify and _sha256(path) != item["sha256"]):
        raise ValueError(f"artifact SHA256/size mismatch: {item['path']}")
    return path


class PortableCache:
    """A prepared portable weight directory: its manifest, plan and per-tensor records."""

    def __init__(self, root, *, verify: bool = True):
        self.root = Path(root).resolve()
        self.verify = verify
        manifest = json.loads((self.root / "manifest.json").read_text())
        if (manifest.get("artifact_kind") != CACHE_KIND or manifest.get("schema_version") != 1
                or manifest.get("status") != CACHE_STATUS):
            raise ValueError("not a prepared portable quantized weight cache")
        plan_doc = json.loads((self.root / "plan.json").read_text())
        contract = plan_doc.get("contract")
        if (plan_doc.get("contract_sha256") != record_identity(contract)
                or manifest.get("contract_sha256") != plan_doc.get("contract_sha256")):
            raise ValueError("portable cache plan does not match its manifest")
        self.contract = contract
        self.records: dict[str, dict] = {}
        for entry in manifest.get("tensors", []):
            record = json.loads(_checked_file(self.root, entry, verify=verify).read_text())
            body = {k: v for k, v in record.items() if k != "record_sha256"}
            if (record.get("status") != "TENSOR_PREPARED" or record.get("record_sha256") != record_identity(body)
                    or record.get("spec", {}).get("key") != entry.get("key")):
                raise ValueError(f"tensor record does not match the planned tensor: {entry.get('key')}")
            self.records[entry["key"]] = record

    def keys(self) -> list[str]:
        return list(self.records)

    def _payload(self, key: str, field: str, fmt: str, dtype: np.dtype, count: int) -> np.ndarray:
        item = self.records[key]["converted"].get(field)
        if item is None or item.get("format") != fmt or item.get("bytes") != count * dtype.itemsize:
            raise ValueError(f"{key}: {field} payload is not {fmt} of {count} elements")
        return np.fromfile(_checked_file(self.root, item, verify=self.verify), dtype=dtype)

    def host(self, key: str) -> tuple[np.ndarray, np.ndarray]:
        """Packed bytes ``uint8 [..., N, K/2]`` and fp32 scales ``[..., N, K/G]`` of an int4 tensor."""
        rec = self.records.get(key)
        if rec is None:
            raise ValueError(f"portable cache has no tensor {key}")
        spec = rec["spec"]
        if spec.get("kind") not in ("linear_int4", "expert_int4"):
            raise ValueError(f"{key} is not an int4 tensor")
        shape, g = tuple(spec["shape"]), spec["group_size"]
        if shape[-1] % g or tuple(spec["weight_shape"]) != (*shape[:-1], shape[-1] // 2):
            raise ValueError(f"{key}: inconsistent int4 descriptor")
        packed = self._payload(key, "weights", INT4_FORMAT, np.dtype("u1"), math.prod(shape) // 2)
        scales = self._payload(key, "scales", SCALE_FORMAT, np.dtype("<f4"), math.prod(shape) // g)
        return packed.reshape(*shape[:-1], shape[-1] // 2), scales.reshape(*shape[:-1], shape[-1] // g)

    def bank(self, key: str, device, *, layout: str = "tiled") -> PackedW4:
        packed, scales = self.host(key)
        g = self.records[key]["spec"]["group_size"]
        bank = PackedW4(torch.from_numpy(packed).to(device), torch.from_numpy(scales).to(device), g)
        bank.validate(key)
        return bank.tiled() if layout == "tiled" else bank

    def embedding(self, key: str = "target.embed_tokens.weight", device="cpu") -> tuple[torch.Tensor, torch.Tensor]:
        """int8 ``[V, H]`` rows and their fp32 ``[V, 1]`` scales (``graph/quant_weights.py:181-186``)."""
        rec = self.records.get(key)
        if rec is None or rec["spec"].get("kind") != "embedding_int8":
            raise ValueError(f"portable cache has no int8 embedding {key}")
        v, h = rec["spec"]["shape"]
        rows = self._payload(key, "weights", INT8_FORMAT, np.dtype("i1"), v * h).reshape(v, h)
        scale = self._payload(key, "scales", SCALE_FORMAT, np.dtype("<f4"), v).reshape(v, 1)
        return torch.from_numpy(rows).to(device), torch.from_numpy(scale).to(device)


def quantized_weights(cache: PortableCache, shapes: Mapping[str, tuple], device, *, layout: str = "tiled",
                      keys: Optional[Iterable[str]] = None):
    """A :class:`quantized.QuantizedWeights` over every int4 tensor of ``cache`` (or ``keys``) and its
    embedding, for the reference model's ``quantization`` seam."""
    from .quantized import QuantizedWeights
    wanted = list(keys) if keys is not None else [
        k for k in cache.keys() if cache.records[k]["spec"].get("kind") in ("linear_int4", "expert_int4")]
    banks = {k: cache.bank(k, device, layout=layout) for k in wanted}
    return QuantizedWeights(shapes, banks, cache.embedding(device=device), layout=layout)
