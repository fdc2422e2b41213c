"""GPU parity: W4A16 qlinear (HIP, through the C ABI) against the fp64 oracle.

Bar: norm-relative max error max|y - r| / max|r| <= 1e-2 against the
fp64-accumulated golden (the kernel accumulates in fp32 and rounds to bf16
once; observed errors are ~1e-3, dominated by the bf16 output rounding).
"""
import numpy as np
import pytest
import torch

from oracle import metrics, w4

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _case(pkg, m, n, k, group, scale_dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn((m, k), generator=gen).to(torch.bfloat16)
    weight = pkg.synthetic.int4_weight(gen, (n, k), group, scale_dtype)
    return x, weight


@pytest.mark.parametrize("m,n,k,group,scale_dtype", [
    (16, 512, 2048, 128, torch.bfloat16),   # the single-qlinear workload
    (1, 512, 2048, 128, torch.bfloat16),
    (5, 32, 512, 128, torch.bfloat16),
    (17, 1024, 2048, 128, torch.bfloat16),
    (33, 64, 4096, 256, torch.bfloat16),
    (64, 96, 1024, 128, torch.float32),
    (16, 2048, 512, 128, torch.bfloat16),
    (32, 64, 1024, 128, torch.float32),
    (24, 128, 2048, 128, torch.float32),
    (16, 512, 2048, 256, torch.float32),    # the reference quantizer's g256 fp32 scales, verify kernel
    (16, 256, 4096, 256, torch.bfloat16),   # g256 at K = 4096
    (16, 8192, 2048, 128, torch.bfloat16),  # the widest output of the small-block kernel
    (17, 10272, 2048, 128, torch.bfloat16), # 17 rows: the staging kernel
    (16, 32800, 1024, 128, torch.bfloat16), # past the streaming form: the staging kernel
    (32, 96, 512, 256, torch.float32),      # small-block kernel: two row tiles, waves past K
    (16, 12384, 2048, 128, torch.bfloat16), # its streaming form (x in registers), 4-tile batches, last one half
    (5, 16448, 4096, 256, torch.float32),   # streaming form at K = 4096: 2-tile batches
    (9, 12320, 1024, 128, torch.bfloat16),  # streaming form, 8-tile batches, last one a quarter
])
def test_qlinear_matches_oracle(pkg, device, m, n, k, group, scale_dtype):
    print(f"qlinear m={m} n={n} k={k} g={group} {scale_dtype}", flush=True)
    x, weight = _case(pkg, m, n, k, group, scale_dtype, seed=m * 7 + n)
    y = pkg.ops.qlinear(x.to(device), weight.to(device)).cpu()
    golden = w4.qlinear(x, weight.packed.numpy(), weight.scales, group)
    report = metrics.compare(y, golden)
    assert y.dtype == torch.bfloat16 and tuple(y.shape) == (m, n)
    assert report["max_rel"] <= TOL, report
    assert report["cosine"] > 0.9999, report


@pytest.mark.parametrize("m,n,k,group,scale_dtype", [
    (16, 256, 2048, 128, torch.bfloat16),   # a packed router's logits: small-block kernel
    (3, 12384, 1024, 256, torch.float32),   # streaming form
    (16, 40960, 2048, 128, torch.bfloat16), # staging verify kernel
    (20, 2048, 512, 128, torch.bfloat16),   # small-block kernel, two row tiles
])
def test_qlinear_fp32_output(pkg, device, m, n, k, group, scale_dtype):
    """The unrounded fp32 output (dflash_qlinear_w4a16_f32): within fp32 summation-order error of
    the fp64 golden, and its bf16 rounding equal to the bf16 entry's output."""
    print(f"qlinear fp32 out m={m} n={n} k={k} g={group} {scale_dtype}", flush=True)
    x, weight = _case(pkg, m, n, k, group, scale_dtype, seed=m + n + 1)
    xd, wd = x.to(device), weight.to(device)
    y32 = pkg.ops.qlinear(xd, wd, out_dtype=torch.float32)
    y16 = pkg.ops.qlinear(xd, wd)
    assert y32.dtype == torch.float32 and tuple(y32.shape) == (m, n)
    golden = w4.qlinear(x, weight.packed.numpy(), weight.scales, group)
    report = metrics.compare(y32.cpu(), golden)
    assert report["max_rel"] <= 5e-5, report  # fp32 sums of -136-offset products, no bf16 rounding
    assert torch.equal(y32.to(torch.bfloat16), y16)


# The target model's quantized projections at a 16-token verify block (graph/quant_plan.py:25-32):
# GDN in_proj_qkv / in_proj_z / in_proj_a|b / out_proj (32 value heads x 128, 16 key heads x 128,
# fused/ops.py:354-360), attention q (gated) / k|v / o (head_dim 256), shared expert gate|up / down.
MODEL_PROJECTIONS = [
    ("linear_attn.in_proj_qkv", 8192, 2048), ("linear_attn.in_proj_z", 4096, 2048),
    ("linear_attn.in_proj_a", 32, 2048), ("linear_attn.out_proj", 2048, 4096),
    ("self_attn.q_proj", 8192, 2048), ("self_attn.k_proj", 512, 2048), ("self_attn.o_proj", 2048, 4096),
    ("mlp.shared_expert.down_proj", 2048, 512),
]


@pytest.mark.parametrize("name,n,k", MODEL_PROJECTIONS, ids=[p[0] for p in MODEL_PROJECTIONS])
@pytest.mark.parametrize("layout", ["portable", "tiled"])
def test_qlinear_model_projections(pkg, device, name, n, k, layout):
    print(f"qlinear {name} m=16 n={n} k={k} {layout}", flush=True)
    x, weight = _case(pkg, 16, n, k, 128, torch.bfloat16, seed=n + k)
    w = weight.to(device)
    if layout == "tiled":
        w = w.tiled()
    y = pkg.ops.qlinear(x.to(device), w).cpu()
    golden = w4.qlinear(x, weight.packed.numpy(), weight.scales, 128)
    report = metrics.compare(y, golden)
    assert report["max_rel"] <= TOL and report["cosine"] > 0.9999, report


@pytest.mark.parametrize("layout", ["portable", "tiled"])
def test_qlinear_stacked_projections(pkg, device, layout):
    """The GDN input projections (qkv, z, a, b) stacked into one matrix: one launch; every part
    within the bar of the oracle and of its separate call (the k-block partial sums of a column
    may be added in another order, so bits can differ)."""
    parts = [("qkv", 8192), ("z", 4096), ("a", 32), ("b", 32)]
    gen = torch.Generator().manual_seed(21)
    x = torch.randn((16, 2048), generator=gen).to(torch.bfloat16)
    host = [pkg.synthetic.int4_weight(gen, (n, 2048), 128) for _, n in parts]
    banks = [h.to(device) for h in host]
    if layout == "tiled":
        banks = [b.tiled() for b in banks]
    stacked = pkg.concat_rows(*banks)
    assert stacked.layout == layout and stacked.rows == sum(n for _, n in parts)
    y = pkg.ops.qlinear(x.to(device), stacked).cpu()
    col = 0
    for (name, n), h, b in zip(parts, host, banks):
        part = y[:, col:col + n]
        golden = w4.qlinear(x, h.packed.numpy(), h.scales, 128)
        assert metrics.compare(part, golden)["max_rel"] <= TOL, name
        separate = pkg.ops.qlinear(x.to(device), b).cpu()
        assert metrics.compare(part, separate)["max_rel"] <= TOL, name
        col += n


@pytest.mark.parametrize("m", [5, 16, 17, 24, 32, 33])
@pytest.mark.parametrize("layout", ["portable", "tiled"])
def test_qlinear_k4096_row_counts(pkg, device, m, layout):
    """K = 4096: the verify kernel stages at most 16 rows, so 17..32 rows run as two launches of
    16 (row 16 is the first row of the second launch); above 32 rows the portable layout takes
    the per-wave kernel and the tiled layout is refused (no kernel streams it at that shape)."""
    print(f"qlinear K=4096 m={m} {layout}", flush=True)
    x, weight = _case(pkg, m, 256, 4096, 128, torch.bfloat16, seed=m)
    w = weight.to(device)
    if layout == "tiled":
        w = w.tiled()
        if m > 32:
            with pytest.raises(pkg._lib.DflashError, match="tiled"):
                pkg.ops.qlinear(x.to(device), w)
            return
    y = pkg.ops.qlinear(x.to(device), w).cpu()
    report = metrics.compare(y, w4.qlinear(x, weight.packed.numpy(), weight.scales, 128))
    assert report["max_rel"] <= TOL and report["cosine"] > 0.9999, report
    if m > 16 and m <= 32:   # every row, the first of the second launch included, is right on its own
        rows = metrics.compare(y[16:17], w4.qlinear(x[16:17], weight.packed.numpy(), weight.scales, 128))
        assert rows["max_rel"] <= TOL, rows


def test_qlinear_lm_head(pkg, device):
    """The LM head [248320, 2048] at a 16-token block: every column on the GPU, a seeded
    sample of 4096 columns against the oracle (the full oracle product is 8 GMAC)."""
    n, k, m = 248320, 2048, 16
    print(f"qlinear lm_head m={m} n={n} k={k}", flush=True)
    x, weight = _case(pkg, m, n, k, 128, torch.bfloat16, seed=248)
    y = pkg.ops.qlinear(x.to(device), weight.to(device).tiled()).cpu()
    assert tuple(y.shape) == (m, n) and torch.isfinite(y.float()).all()
    cols = torch.randperm(n, generator=torch.Generator().manual_seed(7))[:4096].sort().values
    golden = w4.qlinear(x, weight.packed[cols].numpy(), weight.scales[cols], 128)
    report = metrics.compare(y[:, cols], golden)
    assert report["max_rel"] <= TOL and report["cosine"] > 0.9999, report


def test_qlinear_known_answers(pkg, device):
    """One-hot rows pick out a dequantised column; all-ones rows give row sums."""
    n, k, group = 64, 512, 128
    gen = torch.Generator().manual_seed(11)
    weight = pkg.synthetic.int4_weight(gen, (n, k), group)
    deq = w4.dequantize(weight.packed.numpy(), weight.scales, group)
    x = torch.zeros((3, k), dtype=torch.bfloat16)
    x[0, 5] = 1.0
    x[1, k - 1] = 1.0
    x[2, :] = 1.0
    y = pkg.ops.qlinear(x.to(device), weight.to(device)).cpu().float().numpy()
    expect = np.stack([deq[:, 5], deq[:, k - 1], deq.sum(axis=1)])
    expect_bf16 = torch.from_numpy(expect).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(y[:2], expect_bf16[:2])
    assert np.abs(y[2] - expect[2]).max() <= 1e-2 * np.abs(expect[2]).max()


def test_qlinear_through_fused_ops(pkg, device):
    x, weight = _case(pkg, 16, 512, 2048, 128, torch.bfloat16, seed=3)
    w = weight.to(device)
    y = pkg.fused_ops.qlinear(x.to(device).reshape(1, 16, 2048), w.packed, w.scales, group_size=128)
    assert tuple(y.shape) == (1, 16, 512)
    golden = w4.qlinear(x, weight.packed.numpy(), weight.scales, 128)
    assert metrics.compare(y.cpu().reshape(16, 512), golden)["max_rel"] <= TOL


def test_qlinear_rejects_bad_shapes(pkg, device):
    x, weight = _case(pkg, 4, 48, 512, 128, torch.bfloat16, seed=5)
    with pytest.raises(pkg._lib.DflashError, match="N % 32"):
        pkg.ops.qlinear(x.to(device), weight.to(device))
    x, weight = _case(pkg, 4, 32, 640, 128, torch.bfloat16, seed=5)
    with pytest.raises(pkg._lib.DflashError, match="K % 512"):
        pkg.ops.qlinear(x.to(device), weight.to(device))
