"""The on-disk weight formats the reference reads, loaded onto this library's banks.

CPU: tiny original checkpoints (``data*.safetensors`` shards written by the
``safetensors`` library) and tiny portable caches (``manifest.json``,
``plan.json``, records and payloads, written here by the format of
``graph/quant_prepare.py:103-199`` with the oracle's quantizer) load back to the
exact values written, and every header, record and payload check the reference
readers make raises on a tampered copy.

GPU: a routed-MoE layer and a qlinear on banks loaded from each format agree with
the oracle on the values that were written (routing bit-exact, outputs within
the 1e-2 bar).
"""
import hashlib
import json
import math
import shutil
import struct

import numpy as np
import pytest
import torch
from safetensors.numpy import save_file

from oracle import metrics, moe as oracle_moe, routing as oracle_routing, w4 as oracle_w4

LIN = "target.layers.0.self_attn.k_proj.weight"
GU = "target.layers.0.mlp.experts.gate_up_proj"
DN = "target.layers.0.mlp.experts.down_proj"
E, H, I = 8, 512, 512


def _original_values(seed=0):
    rng = np.random.default_rng(seed)
    vals = {
        LIN: rng.integers(-8, 8, size=(64, H), dtype=np.int8),
        GU: rng.integers(-8, 8, size=(E, 2 * I, H), dtype=np.int8),
        DN: rng.integers(-8, 8, size=(E, H, I), dtype=np.int8),
    }
    scales = {
        LIN: rng.uniform(0.005, 0.02, size=(64, H // 256, 1)).astype(np.float16),
        GU: rng.uniform(0.005, 0.02, size=(E, 2 * I, H // 256)).astype(np.float32),
        DN: rng.uniform(0.005, 0.02, size=(E, H, I // 256)).astype(np.float16),
    }
    return vals, scales


def _write_original(root, vals, scales, pkg):
    root.mkdir(parents=True, exist_ok=True)
    names = {k: pkg.checkpoint.original_keys(k) for k in vals}
    save_file({names[LIN][0]: vals[LIN], names[LIN][1]: scales[LIN], names[GU][1]: scales[GU]},
              str(root / "data-00001.safetensors"))
    save_file({names[GU][0]: vals[GU], names[DN][0]: vals[DN], names[DN][1]: scales[DN]},
              str(root / "data-00002.safetensors"))
    return root


def _shape(key, vals):
    return tuple(int(x) for x in vals[key].shape)


def test_original_shards_read_back(pkg, tmp_path):
    vals, scales = _original_values()
    ck = pkg.checkpoint.OriginalShards(_write_original(tmp_path / "orig", vals, scales, pkg))
    for key in (LIN, GU, DN):
        w, s = ck.logical(key, _shape(key, vals))
        assert np.array_equal(np.asarray(w), vals[key])
        assert np.array_equal(np.asarray(s), scales[key]) and s.dtype == scales[key].dtype
    with pytest.raises(ValueError, match="expected"):
        ck.describe(LIN, (64, 2 * H))
    with pytest.raises(ValueError, match="rank does not match"):
        ck.describe(GU, (2 * I, H))
    with pytest.raises(ValueError, match="missing"):
        ck.describe("target.layers.1.self_attn.k_proj.weight", (64, H))
    with pytest.raises(ValueError, match="not an original target quantized weight"):
        pkg.checkpoint.original_keys("target.layers.0.input_layernorm.weight")


def test_original_value_and_scale_checks(pkg, tmp_path):
    vals, scales = _original_values(1)
    bad = dict(vals)
    bad[GU] = vals[GU].copy()
    bad[GU][3, 7, 11] = 8
    ck = pkg.checkpoint.OriginalShards(_write_original(tmp_path / "v", bad, scales, pkg))
    with pytest.raises(ValueError, match="outside signed I4"):
        ck.logical(GU, _shape(GU, vals))
    neg = dict(scales)
    neg[DN] = scales[DN].copy()
    neg[DN][0, 0, 0] = -1
    ck = pkg.checkpoint.OriginalShards(_write_original(tmp_path / "s", vals, neg, pkg))
    with pytest.raises(ValueError, match="finite and nonnegative"):
        ck.logical(DN, _shape(DN, vals))


def _raw_shard(path, header: dict, payload: bytes):
    text = json.dumps(header).encode()
    path.write_bytes(struct.pack("<Q", len(text)) + text + payload)


def test_original_header_checks(pkg, tmp_path):
    cls = pkg.checkpoint.OriginalShards
    with pytest.raises(ValueError, match="1..4096"):
        cls(tmp_path)
    d = tmp_path / "overlap"
    d.mkdir()
    _raw_shard(d / "data-1.safetensors", {"a": {"dtype": "I8", "shape": [8], "data_offsets": [0, 8]},
                                          "b": {"dtype": "I8", "shape": [8], "data_offsets": [4, 12]}}, bytes(12))
    with pytest.raises(ValueError, match="overlapping"):
        cls(d)
    d = tmp_path / "extent"
    d.mkdir()
    _raw_shard(d / "data-1.safetensors", {"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 8]}}, bytes(16))
    with pytest.raises(ValueError, match="data extent"):
        cls(d)
    d = tmp_path / "dup"
    d.mkdir()
    text = b'{"a": {"dtype": "I8", "shape": [1], "data_offsets": [0, 1]}, "a": {"dtype": "I8", "shape": [1], "data_offsets": [0, 1]}}'
    (d / "data-1.safetensors").write_bytes(struct.pack("<Q", len(text)) + text + bytes(1))
    with pytest.raises(ValueError, match="duplicate safetensors JSON key"):
        cls(d)
    d = tmp_path / "across"
    d.mkdir()
    for n in (1, 2):
        _raw_shard(d / f"data-{n}.safetensors", {"a": {"dtype": "I8", "shape": [1], "data_offsets": [0, 1]}}, bytes(1))
    with pytest.raises(ValueError, match="across shards"):
        cls(d)
    d = tmp_path / "length"
    d.mkdir()
    (d / "data-1.safetensors").write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    with pytest.raises(ValueError, match="header length"):
        cls(d)
    d = tmp_path / "link"
    d.mkdir()
    _raw_shard(tmp_path / "outside.safetensors", {"a": {"dtype": "I8", "shape": [1], "data_offsets": [0, 1]}}, bytes(1))
    (d / "data-1.safetensors").symlink_to(tmp_path / "outside.safetensors")
    with pytest.raises(ValueError, match="regular file inside"):
        cls(d)


# ------------------------------------------------------------------ portable cache
def _identity(value):
    return hashlib.sha256(json.dumps(value, sort_keys=True, separators=(",", ":"), allow_nan=False).encode()).hexdigest()


def _file_item(root, rel, fmt, shape, dtype):
    data = (root / rel).read_bytes()
    return {"path": rel, "shape": list(shape), "dtype": dtype, "format": fmt, "bytes": len(data),
            "sha256": hashlib.sha256(data).hexdigest()}


def _write_cache(root, tensors: dict, embedding=None, group=256):
    """A prepared cache in the reference's layout: logical int4 [..., K/2] and fp32 scales from the
    oracle's quantiser of float weights (``graph/quant_weights.py:110-178``)."""
    (root / "weights").mkdir(parents=True)
    (root / "tensors").mkdir()
    contract = {"artifact_kind": "qwen35-portable-quant-weights", "schema_version": 1, "plan": {"group_size": group}}
    (root / "plan.json").write_text(json.dumps({"contract": contract, "contract_sha256": _identity(contract)}))
    entries, written = [], {}
    items = list(tensors.items()) + ([("target.embed_tokens.weight", embedding)] if embedding is not None else [])
    for index, (key, weight) in enumerate(items):
        shape = tuple(weight.shape)
        wrel, srel = f"weights/{index:05d}.weight.bin", f"weights/{index:05d}.scale.bin"
        if key == "target.embed_tokens.weight":
            scale = np.maximum(np.abs(weight).max(-1), 1e-8).astype(np.float32) / np.float32(127)
            q = np.clip(np.rint(weight / scale[:, None]), -128, 127).astype(np.int8)
            (root / wrel).write_bytes(q.tobytes())
            (root / srel).write_bytes(scale.astype("<f4").tobytes())
            spec = {"key": key, "kind": "embedding_int8", "shape": list(shape)}
            converted = {"weights": _file_item(root, wrel, "PORTABLE_LOGICAL_INT8_ROW_MAJOR", shape, "int8"),
                         "scales": _file_item(root, srel, "LOGICAL_SCALES_ROW_MAJOR_FP32_LE", shape[:1], "float32")}
            written[key] = (q, scale)
        else:
            q, s = oracle_w4.quantize(torch.from_numpy(weight), group)
            packed = oracle_w4.pack(q)
            (root / wrel).write_bytes(packed.tobytes())
            (root / srel).write_bytes(s.astype("<f4").tobytes())
            kind = "expert_int4" if len(shape) == 3 else "linear_int4"
            spec = {"key": key, "kind": kind, "shape": list(shape), "group_size": group,
                    "weight_shape": [*shape[:-1], shape[-1] // 2], "weight_dtype": "uint8"}
            converted = {"weights": _file_item(root, wrel, "PORTABLE_LOGICAL_INT4_ROW_MAJOR_LOW_NIBBLE_FIRST", shape, "int4"),
                         "scales": _file_item(root, srel, "LOGICAL_SCALES_ROW_MAJOR_FP32_LE", s.shape, "float32"),
                         "device_ready": False, "device_pack": "NOT_PERFORMED"}
            written[key] = (packed, s)
        record = {"status": "TENSOR_PREPARED", "spec": spec, "converted": converted, "reused_from": None}
        record["record_sha256"] = _identity(record)
        rpath = root / "tensors" / f"{index:05d}.json"
        rpath.write_text(json.dumps(record))
        data = rpath.read_bytes()
        entries.append({"key": key, "path": f"tensors/{index:05d}.json", "bytes": len(data),
                        "sha256": hashlib.sha256(data).hexdigest()})
    manifest = {"schema_version": 1, "artifact_kind": "qwen35-portable-quant-weights",
                "status": "WEIGHTS_PREPARED_LAYOUT_PENDING", "contract_sha256": _identity(contract),
                "tensors": entries}
    (root / "manifest.json").write_text(json.dumps(manifest))
    return written


def _float_weights(seed):
    gen = torch.Generator().manual_seed(seed)
    return {LIN: (torch.randn((64, H), generator=gen) * 0.02).numpy(),
            GU: (torch.randn((E, 2 * I, H), generator=gen) * 0.02).numpy(),
            DN: (torch.randn((E, H, I), generator=gen) * 0.02).numpy()}


def test_portable_cache_reads_back(pkg, tmp_path):
    written = _write_cache(tmp_path / "c", _float_weights(2),
                           embedding=np.random.default_rng(3).standard_normal((32, H)).astype(np.float32))
    cache = pkg.checkpoint.PortableCache(tmp_path / "c")
    for key in (LIN, GU, DN):
        packed, scales = cache.host(key)
        assert np.array_equal(packed, written[key][0]) and np.array_equal(scales, written[key][1])
    rows, scale = cache.embedding()
    assert rows.dtype == torch.int8 and scale.shape == (32, 1)
    assert np.array_equal(rows.numpy(), written["target.embed_tokens.weight"][0])
    with pytest.raises(ValueError, match="no tensor"):
        cache.host("target.layers.9.self_attn.k_proj.weight")


def test_portable_cache_checks(pkg, tmp_path):
    src = tmp_path / "c"
    _write_cache(src, {LIN: _float_weights(4)[LIN]})
    cls = pkg.checkpoint.PortableCache
    bad = tmp_path / "payload"
    shutil.copytree(src, bad)
    blob = bytearray((bad / "weights/00000.weight.bin").read_bytes())
    blob[5] ^= 0x11
    (bad / "weights/00000.weight.bin").write_bytes(bytes(blob))
    cache = cls(bad)
    with pytest.raises(ValueError, match="SHA256/size mismatch"):
        cache.host(LIN)
    bad = tmp_path / "record"
    shutil.copytree(src, bad)
    rec = json.loads((bad / "tensors/00000.json").read_text())
    rec["spec"]["group_size"] = 128
    (bad / "tensors/00000.json").write_text(json.dumps(rec))
    with pytest.raises(ValueError, match="SHA256/size mismatch"):      # the manifest pins the record file
        cls(bad)
    man = json.loads((bad / "manifest.json").read_text())
    data = (bad / "tensors/00000.json").read_bytes()
    man["tensors"][0].update(bytes=len(data), sha256=hashlib.sha256(data).hexdigest())
    (bad / "manifest.json").write_text(json.dumps(man))
    with pytest.raises(ValueError, match="does not match the planned tensor"):   # its own hash does not
        cls(bad)
    bad = tmp_path / "kind"
    shutil.copytree(src, bad)
    man = json.loads((bad / "manifest.json").read_text())
    man["status"] = "FAILED"
    (bad / "manifest.json").write_text(json.dumps(man))
    with pytest.raises(ValueError, match="not a prepared"):
        cls(bad)
    bad = tmp_path / "escape"
    shutil.copytree(src, bad)
    man = json.loads((bad / "manifest.json").read_text())
    man["tensors"][0]["path"] = "../c/tensors/00000.json"
    (bad / "manifest.json").write_text(json.dumps(man))
    with pytest.raises(ValueError, match="escapes bundle"):
        cls(bad)


# ------------------------------------------------------------------ GPU: layers from loaded banks
def _layer_vs_oracle(pkg, device, gate_up, down, gu_ref, dn_ref, group, seed):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn((16, H), generator=gen).to(torch.bfloat16)
    router = (torch.randn((E, H), generator=gen) * 0.02).to(torch.bfloat16)
    out, r, logits = pkg.ops.moe_w4a16(x.to(device), gate_up, down, top_k=2, router_weight=router.to(device),
                                       return_routing=True)
    golden = oracle_moe.moe(x, logits.cpu().numpy(), 2, gu_ref, dn_ref, group)
    assert torch.equal(r.ids.cpu(), torch.from_numpy(golden["ids"]))
    assert torch.equal(r.perm.cpu(), torch.from_numpy(golden["perm"]))
    rep = metrics.compare(out.cpu(), golden["out_f32"])
    assert rep["max_rel"] <= metrics.MAX_REL_TOLERANCE, rep
    return x


@pytest.mark.gpu
@pytest.mark.parametrize("layout", ["tiled", "portable"])
def test_layer_from_original_shards(pkg, device, tmp_path, layout):
    vals, scales = _original_values(5)
    ck = pkg.checkpoint.OriginalShards(_write_original(tmp_path / "orig", vals, scales, pkg))
    gu = ck.bank(GU, _shape(GU, vals), device, layout=layout)
    dn = ck.bank(DN, _shape(DN, vals), device, layout=layout)
    assert gu.layout == layout and gu.scales.dtype == torch.float32 and gu.group_size == 256
    ref = {k: (torch.from_numpy(oracle_w4.pack(vals[k])), torch.from_numpy(scales[k].astype(np.float32)))
           for k in (GU, DN)}
    _layer_vs_oracle(pkg, device, gu, dn, ref[GU], ref[DN], 256, 6)
    lin = ck.bank(LIN, _shape(LIN, vals), device, layout=layout)
    x = torch.randn((16, H), generator=torch.Generator().manual_seed(7)).to(torch.bfloat16)
    y = pkg.ops.qlinear(x.to(device), lin).cpu()
    want = oracle_w4.qlinear(x, oracle_w4.pack(vals[LIN]), scales[LIN][..., 0].astype(np.float32), 256)
    assert metrics.compare(y, want)["max_rel"] <= metrics.MAX_REL_TOLERANCE
    bad = dict(vals)
    bad[DN] = vals[DN].copy()
    bad[DN][1, 2, 3] = -9
    ck = pkg.checkpoint.OriginalShards(_write_original(tmp_path / "bad", bad, scales, pkg))
    with pytest.raises(ValueError, match="outside signed I4"):
        ck.bank(DN, _shape(DN, vals), device, layout=layout)


@pytest.mark.gpu
def test_layer_from_portable_cache(pkg, device, tmp_path):
    written = _write_cache(tmp_path / "c", _float_weights(8))
    cache = pkg.checkpoint.PortableCache(tmp_path / "c")
    gu, dn = cache.bank(GU, device), cache.bank(DN, device)
    ref = {k: (torch.from_numpy(written[k][0]), torch.from_numpy(written[k][1])) for k in (GU, DN)}
    _layer_vs_oracle(pkg, device, gu, dn, ref[GU], ref[DN], 256, 9)
    lin = cache.bank(LIN, device, layout="portable")
    x = torch.randn((16, H), generator=torch.Generator().manual_seed(10)).to(torch.bfloat16)
    y = pkg.ops.qlinear(x.to(device), lin).cpu()
    want = oracle_w4.qlinear(x, written[LIN][0], written[LIN][1], 256)
    assert metrics.compare(y, want)["max_rel"] <= metrics.MAX_REL_TOLERANCE
