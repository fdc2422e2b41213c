"""GPU parity: load-time repack of the original checkpoint's int8-carried int4
weights (``dflash_w4_from_int8``) against the oracle, byte for byte.

The reader of that format is ``target/original_quant.py:214-272``: int8 values
in [-8, 7] (``[N, K]`` linears, ``[E, N, K]`` expert banks) and fp16/fp32 group-256
scales (``[N, K/256, 1]`` / ``[E, N, K/256]``), rejected with ``ValueError`` when a
value is out of range or a scale negative or not finite.  Bar: bit-exact packed
bytes and fp32 scales in both layouts; a layer built from the repacked banks
equals the one built from the oracle's bytes exactly.
"""
import numpy as np
import pytest
import torch

from oracle import metrics, w4
from oracle import moe as oracle_moe

pytestmark = pytest.mark.gpu


def _source(shape, group, scale_dtype, seed, linear_axis=False):
    gen = torch.Generator().manual_seed(seed)
    values = torch.randint(-8, 8, shape, dtype=torch.int8, generator=gen)
    sshape = (*shape[:-1], shape[-1] // group) + ((1,) if linear_axis else ())
    scales = (torch.rand(sshape, generator=gen) * 0.015 + 0.005).to(scale_dtype)
    return values, scales


@pytest.mark.parametrize("shape,group,scale_dtype,linear_axis", [
    ((512, 2048), 256, torch.float16, True),      # a linear as the reader stores it
    ((4, 1024, 2048), 256, torch.float32, False),  # an expert gate_up bank (E = 4 of 256)
    ((3, 2048, 512), 256, torch.float32, False),   # an expert down bank
    ((64, 1024), 128, torch.bfloat16, False),
])
@pytest.mark.parametrize("layout", ["portable", "tiled"])
def test_from_int8_matches_oracle(pkg, device, shape, group, scale_dtype, linear_axis, layout):
    print(f"from_int8 {shape} g={group} {scale_dtype} {layout}", flush=True)
    values, scales = _source(shape, group, scale_dtype, seed=sum(shape))
    w = pkg.ops.from_int8(values.to(device), scales.to(device), group, layout=layout)
    ep, es = w4.from_int8(values.numpy(), scales.float().numpy() if scale_dtype == torch.bfloat16 else scales.numpy(),
                          tiled=layout == "tiled")
    assert w.layout == layout and w.scales.dtype == torch.float32
    np.testing.assert_array_equal(w.packed.cpu().numpy(), ep)
    np.testing.assert_array_equal(w.scales.cpu().numpy(), es)


@pytest.mark.parametrize("case", ["value", "negative", "nan"])
def test_from_int8_rejects_what_the_reader_rejects(pkg, device, case):
    values, scales = _source((32, 512), 256, torch.float32, seed=1)
    if case == "value":
        values[7, 300] = -9
        match = "outside signed I4"
    else:
        scales[9, 1] = -0.5 if case == "negative" else float("nan")
        match = "finite and nonnegative"
    with pytest.raises(ValueError, match=match):
        pkg.ops.from_int8(values.to(device), scales.to(device), 256)


def test_layer_from_int8_banks(pkg, device):
    """A T=16 layer on banks repacked from the int8-carried format (g256 fp32, the
    verify kernels) equals the same layer on the oracle's bytes exactly, and the
    fp32-accumulated golden within the 1e-2 bar."""
    E, H, I, k, T = 32, 2048, 512, 8, 16
    print(f"layer from int8 banks T={T} E={E} g256 fp32", flush=True)
    vgu, sgu = _source((E, 2 * I, H), 256, torch.float32, seed=11)
    vdn, sdn = _source((E, H, I), 256, torch.float32, seed=12)
    gu = pkg.ops.from_int8(vgu.to(device), sgu.to(device), 256)
    dn = pkg.ops.from_int8(vdn.to(device), sdn.to(device), 256)
    pgu, pdn = torch.from_numpy(w4.pack(vgu.numpy())), torch.from_numpy(w4.pack(vdn.numpy()))
    gu_ref = pkg.PackedW4(pgu, sgu, 256).to(device).tiled()
    dn_ref = pkg.PackedW4(pdn, sdn, 256).to(device).tiled()
    gen = torch.Generator().manual_seed(13)
    x = torch.randn((T, H), generator=gen).to(torch.bfloat16)
    router = (torch.randn((E, H), generator=gen) * 0.02).to(torch.bfloat16)
    y, _, logits = pkg.ops.moe_w4a16(x.to(device), gu, dn, top_k=k, router_weight=router.to(device),
                                     return_routing=True)
    y_ref = pkg.ops.moe_w4a16(x.to(device), gu_ref, dn_ref, top_k=k, router_weight=router.to(device))
    assert torch.equal(y.cpu(), y_ref.cpu())
    golden = oracle_moe.moe(x, logits.cpu().numpy(), k, (pgu, sgu), (pdn, sdn), 256)
    report = metrics.compare(y.cpu(), golden["out_f32"])
    assert report["max_rel"] <= 1e-2 and report["cosine"] > 0.9999, report
