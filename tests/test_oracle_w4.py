"""CPU: pin the W4 oracle (pack/unpack, quantiser, dequant linear).

Checks: golden vectors written by the independent pure-Python brute force in
``tests/golden/make_golden.py`` (exact nibble table, known quantiser groups,
Fraction-exact W4A16 dot products), brute force over all nibble pairs,
closed forms (one-hot and all-ones activations), and agreement of the product's
host packer (``packing.quantize_w4``) with the oracle quantiser.
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import w4

GOLDEN = json.loads((Path(__file__).resolve().parent / "golden" / "w4_golden.json").read_text())


def test_nibble_table():
    for low, high, byte in GOLDEN["nibble_table"]:
        q = np.array([low, high], dtype=np.int8)
        assert int(w4.pack(q)[0]) == byte
        np.testing.assert_array_equal(w4.unpack(np.array([byte], np.uint8)), q)


def test_pack_unpack_round_trip_all_bytes():
    every = np.arange(256, dtype=np.uint8).reshape(2, 128)
    np.testing.assert_array_equal(w4.pack(w4.unpack(every)), every)
    q = w4.unpack(every)
    assert q.min() == -8 and q.max() == 7


def test_pack_rejects_out_of_range():
    with pytest.raises(ValueError):
        w4.pack(np.array([8, 0], np.int8))
    with pytest.raises(ValueError):
        w4.pack(np.array([1, 2, 3], np.int8))


def test_quantize_known_groups():
    for case in GOLDEN["quantize"]:
        q, s = w4.quantize(torch.tensor([case["values"]], dtype=torch.float32), 4)
        assert float(s[0, 0]) == pytest.approx(case["scale"], rel=0, abs=0)
        np.testing.assert_array_equal(q[0], np.array(case["q"], np.int8))


@pytest.mark.parametrize("case", range(len(GOLDEN["qlinear"])))
def test_qlinear_exact_golden(case):
    c = GOLDEN["qlinear"][case]
    x = torch.tensor(c["x"], dtype=torch.float32).to(torch.bfloat16)
    assert torch.equal(x.float(), torch.tensor(c["x"], dtype=torch.float32))  # inputs are bf16-exact
    packed = np.array(c["packed"], np.uint8)
    scales = torch.tensor(c["scales"], dtype=torch.float32)
    y = w4.qlinear(x, packed, scales, c["group"])
    np.testing.assert_array_equal(y, np.array(c["y"], np.float64))  # dyadic values: fp64 is exact here
    y32 = w4.qlinear(x, packed, scales, c["group"], accumulate="fp32")
    np.testing.assert_allclose(y32, np.array(c["y"]), rtol=1e-6, atol=1e-6)


def test_qlinear_closed_forms():
    rng = np.random.default_rng(0)
    packed = rng.integers(0, 256, (32, 256), dtype=np.uint8)
    scales = torch.from_numpy(rng.uniform(0.005, 0.02, (32, 4)).astype(np.float32)).to(torch.bfloat16)
    deq = w4.dequantize(packed, scales, 128)
    x = torch.zeros((2, 512), dtype=torch.bfloat16)
    x[0, 77] = 1.0
    x[1, :] = 1.0
    y = w4.qlinear(x, packed, scales, 128)
    np.testing.assert_array_equal(y[0], deq[:, 77].astype(np.float64))
    np.testing.assert_allclose(y[1], deq.astype(np.float64).sum(axis=1), rtol=1e-12)


def test_dequantize_uses_the_right_group_scale():
    packed = w4.pack(np.full((1, 256), 1, np.int8))
    scales = np.array([[0.5, 2.0]], np.float32)
    deq = w4.dequantize(packed, scales, 128)
    assert np.all(deq[0, :128] == 0.5) and np.all(deq[0, 128:] == 2.0)


@pytest.mark.parametrize("group,scale_dtype", [(128, torch.bfloat16), (256, torch.float32)])
def test_product_packer_matches_oracle(pkg, group, scale_dtype):
    gen = torch.Generator().manual_seed(group)
    w = torch.randn((3, 64, 512), generator=gen)
    w[0, 0, :group] = 0.0  # an all-zero group gets scale 1
    packed = pkg.quantize_w4(w, group, scale_dtype)
    s = packed.scales.float()
    q_oracle, s_oracle = w4.quantize(w / 1.0, group)
    if scale_dtype == torch.float32:
        np.testing.assert_array_equal(s.numpy(), s_oracle)
        np.testing.assert_array_equal(w4.unpack(packed.packed.numpy()), q_oracle)
    # in every case the stored scale reproduces q = clip(rint(w / s), -8, 7) exactly
    q = np.clip(np.rint(w.numpy().reshape(3, 64, -1, group) / s.numpy()[..., None]), -8, 7).reshape(w.shape)
    np.testing.assert_array_equal(w4.unpack(packed.packed.numpy()), q.astype(np.int8))
    assert float(s[0, 0, 0]) == 1.0


@pytest.mark.parametrize("lead,n,k,groups", [((), 16, 256, 2), ((2,), 32, 512, 4), ((3,), 48, 256, 1)])
def test_to_tiled_follows_the_bytewise_definition(lead, n, k, groups):
    """Chunk l of block (t, b) is bytes 64b + 16(l // 16) .. +15 of row 16t + l % 16; scales [t][g][c] = [16t + c][g]."""
    rng = np.random.default_rng(n + k)
    packed = rng.integers(0, 256, (*lead, n, k // 2), dtype=np.uint8)
    scales = rng.random((*lead, n, groups)).astype(np.float32)
    tiled, tiled_s = w4.to_tiled(packed, scales)
    assert tiled.shape == packed.shape and tiled_s.shape == scales.shape
    flat_p = packed.reshape(-1, n, k // 2)
    flat_t = tiled.reshape(flat_p.shape[0], -1)
    flat_s = scales.reshape(-1, n, groups)
    flat_ts = tiled_s.reshape(flat_s.shape[0], -1)
    for e in range(flat_p.shape[0]):
        for t in range(n // 16):
            for b in range(k // 128):
                for lane in range(64):
                    o = (t * (k // 128) + b) * 1024 + lane * 16
                    src = flat_p[e, 16 * t + lane % 16, 64 * b + 16 * (lane // 16): 64 * b + 16 * (lane // 16) + 16]
                    assert (flat_t[e, o:o + 16] == src).all()
            for g in range(groups):
                for c in range(16):
                    assert flat_ts[e, (t * groups + g) * 16 + c] == flat_s[e, 16 * t + c, g]
    back, back_s = w4.from_tiled(tiled, tiled_s)
    assert (back == packed).all() and (back_s == scales).all()


def test_to_tiled_rejects_untileable_shapes():
    with pytest.raises(ValueError):
        w4.to_tiled(np.zeros((24, 64), np.uint8), np.zeros((24, 1), np.float32))


def test_from_int8_round_trips_and_widens_scales_exactly():
    """The int8-carried reader format: packing then unpacking returns the values, the
    tiled order is the bytewise to_tiled, fp16 scales widen exactly, the trailing
    [.., 1] scale axis of a linear is dropped."""
    rng = np.random.default_rng(3)
    values = rng.integers(-8, 8, size=(2, 32, 512), dtype=np.int8)
    scales = (rng.random((2, 32, 2)) * 0.02).astype(np.float16)
    packed, wide = w4.from_int8(values, scales, tiled=False)
    np.testing.assert_array_equal(w4.unpack(packed), values)
    assert wide.dtype == np.float32 and np.array_equal(wide, scales.astype(np.float32))
    tp, ts = w4.from_int8(values, scales, tiled=True)
    ep, es = w4.to_tiled(packed, wide)
    np.testing.assert_array_equal(tp, ep)
    np.testing.assert_array_equal(ts, es)
    lp, ls = w4.from_int8(values[0], scales[0][..., None], tiled=False)
    np.testing.assert_array_equal(lp, packed[0])
    np.testing.assert_array_equal(ls, wide[0])


@pytest.mark.parametrize("case", ["value", "negative", "nan", "inf"])
def test_from_int8_rejects_what_the_reader_rejects(case):
    values = np.zeros((16, 256), dtype=np.int8)
    scales = np.ones((16, 1), dtype=np.float32)
    if case == "value":
        values[3, 7] = 8
        match = "outside signed I4"
    else:
        scales[5, 0] = {"negative": -1.0, "nan": np.nan, "inf": np.inf}[case]
        match = "finite and nonnegative"
    with pytest.raises(ValueError, match=match):
        w4.from_int8(values, scales, tiled=False)



def test_dequantize_torch_equals_dequantize():
    """The CPU baseline's vectorised dequantiser equals the oracle's, every byte value included."""
    gen = torch.Generator().manual_seed(17)
    packed = torch.randint(0, 256, (3, 32, 256), dtype=torch.uint8, generator=gen)
    packed[0, 0, :] = torch.arange(256, dtype=torch.uint8)
    scales = (torch.rand((3, 32, 4), generator=gen) * 0.015 + 0.005).to(torch.bfloat16)
    got = w4.dequantize_torch(packed, scales, 128, torch.float32)
    np.testing.assert_array_equal(got.numpy(), w4.dequantize(packed.numpy(), scales, 128))
