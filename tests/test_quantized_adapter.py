"""The quantized-weights adapter (seam 2): interface and binding on the CPU, results on the GPU.

CPU: the members ``FusedTargetModel`` calls exist and validate like the reference
adapter (``fused/quantization.py:67-202``); ``bind`` makes an instance pass an
``isinstance`` check against a stand-in for the reference class while every
member resolves to this adapter; the tensor inventory (``plan``) matches the
reference's per-tensor kinds.

GPU: ``linear`` equals ``dflash_qlinear_w4a16`` (fp16 cast of the same bits),
``moe`` equals ``dflash_moe_w4a16`` routed-only, and the reference model's
``_moe`` composition over this adapter (routed experts + shared expert through
three ``linear`` calls and the float gate, ``fused/model.py:296-307``) agrees
with the stack's fused shared expert within the bf16 bar.
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import metrics


def _small(pkg, device="cpu"):
    c = pkg.target.small_config()
    c = type(c)(**{**vars(c), "linear_value_heads": 32})        # a/b projections of 32 rows (qlinear N % 32)
    w = pkg.target.random_weights(c, seed=2, device=device, layout="portable",
                                  generate_on="cpu" if device == "cpu" else None)
    return c, w


def test_inventory_kinds(pkg):
    c = pkg.plan.TargetConfig()
    shapes = pkg.plan.target_shapes(c)
    assert len([k for k in shapes if k.startswith("target.layers.0.")]) == 18     # 11 GDN + 7 MoE tensors
    kinds = {k: pkg.plan.tensor_kind(k, s) for k, s in shapes.items()}
    assert kinds["target.embed_tokens.weight"] == "embedding_int8"
    assert kinds["target.lm_head.weight"] == "linear_int4"
    assert kinds["target.layers.3.self_attn.q_proj.weight"] == "linear_int4"
    assert kinds["target.layers.0.mlp.experts.gate_up_proj"] == "expert_int4"
    assert kinds["target.layers.0.linear_attn.A_log"] == "float"
    with pytest.raises(ValueError, match="unrecognized"):
        pkg.plan.tensor_kind("target.layers.0.mlp.bogus", (4, 4))
    rec = pkg.plan.describe("target.layers.0.mlp.experts.down_proj", shapes["target.layers.0.mlp.experts.down_proj"])
    assert rec["weight_shape"] == [256, 2048, 256] and rec["scale_shape"] == [256, 2048, 4]
    assert rec["weight_bytes"] == 256 * 2048 * 512 // 2
    keys = pkg.plan.int4_keys(shapes)
    assert "target.layers.0.mlp.gate.weight" not in keys and "target.lm_head.weight" in keys
    dopt = pkg.plan.int4_keys(shapes, keep_float=pkg.plan.DOPT_W4A16_FLOAT)
    assert "target.lm_head.weight" not in dopt and "target.layers.0.linear_attn.in_proj_a.weight" not in dopt
    # every projection of a layer is int4 except the router; 40 layers x 13 + the LM head
    assert len(keys) == 30 * (5 + 2 + 3) + 10 * (4 + 2 + 3) + 1


def test_adapter_interface_and_errors(pkg):
    c, w = _small(pkg)
    q = pkg.quantized.from_target_weights(w, layout="portable")
    shapes = pkg.plan.target_shapes(c)
    q.validate_shapes(shapes)
    with pytest.raises(ValueError, match="geometry does not match"):
        q.validate_shapes({**shapes, "target.norm.weight": (7,)})
    assert q.has_weight("target.embed_tokens.weight") and q.has_weight("target.lm_head.weight")
    assert q.has_weight("target.layers.0.linear_attn.in_proj_a.weight")
    assert q.has_weight("target.layers.0.mlp.gate.weight")
    assert not q.has_weight("target.layers.0.input_layernorm.weight")
    ids = torch.tensor([[3, 7, 3]])
    emb = q.embedding(ids)
    assert emb.dtype == torch.float32 and tuple(emb.shape) == (1, 3, c.hidden)
    torch.testing.assert_close(emb[0, 0], w.embedding[3].float() * w.embedding_scale[3])
    with pytest.raises(ValueError, match="invalid original quant linear invocation"):
        q.linear(torch.zeros((1, 2, c.hidden + 1)), "target.lm_head.weight")
    with pytest.raises(ValueError, match="invalid original quant linear invocation"):
        q.linear(torch.zeros((1, 2, c.hidden)), "target.layers.0.input_layernorm.weight")
    with pytest.raises(ValueError, match="INT8"):
        pkg.quantized.QuantizedWeights(shapes, {}, (w.embedding.float(), w.embedding_scale))


def test_bind_passes_the_models_isinstance_check(pkg):
    """A stand-in with the reference class's shape: an nn.Module whose __init__ needs a vendor
    binding.  The bound class is an instance of it, never runs its __init__, and every member
    the model calls is the adapter's."""
    class OriginalQuantizedWeights(torch.nn.Module):
        def __init__(self, shapes, reader, embedding, *, ops, device="cpu"):
            raise AssertionError("the reference constructor must not run")

        def linear(self, x, key):
            raise AssertionError("the reference member must not be called")

        moe = has_weight = validate_shapes = embedding = linear

    _, w = _small(pkg)
    bound = pkg.quantized.bind(OriginalQuantizedWeights)
    q = pkg.quantized.from_target_weights(w, layout="portable")
    adapter = bound(q.shapes, dict(q._banks), (w.embedding, w.embedding_scale), routers=dict(q._routers),
                    layout="portable")
    assert isinstance(adapter, OriginalQuantizedWeights) and isinstance(adapter, pkg.quantized.QuantizedWeights)
    for member in ("linear", "moe", "has_weight", "validate_shapes", "embedding"):
        assert getattr(type(adapter), member) is getattr(pkg.quantized.QuantizedWeights, member)
    assert adapter.has_weight("target.lm_head.weight") and adapter.device == torch.device("cpu")
    with pytest.raises(TypeError):
        pkg.quantized.bind(object)


@pytest.mark.gpu
def test_adapter_linear_and_moe_on_the_kernels(pkg, device):
    c, w = _small(pkg, device)
    wt = pkg.target.to_device(w, device, layout="tiled")
    q = pkg.quantized.from_target_weights(wt)
    gen = torch.Generator().manual_seed(4)
    x = torch.randn((1, 16, c.hidden), generator=gen).to(device)       # fp32, as the model's residual
    xb = x.reshape(16, -1).to(torch.bfloat16)
    lw = wt.layers[0]
    key = "target.layers.0.linear_attn.in_proj_z.weight"
    got = q.linear(x, key)
    assert got.dtype == torch.float16 and tuple(got.shape) == (1, 16, c.linear_value_heads * c.linear_value_dim)
    ref = pkg.ops.qlinear(xb, q._banks[key])
    assert torch.equal(got.reshape(16, -1), ref.to(torch.float16))
    routed = q.moe(x, "target.layers.0.mlp", top_k=c.top_k)
    ref_routed = pkg.ops.moe_w4a16(xb, lw.gate_up, lw.down, top_k=c.top_k, router_weight=lw.router)
    assert routed.dtype == torch.float16 and torch.equal(routed.reshape(16, -1), ref_routed.to(torch.float16))
    # fused/model.py:296-307 over the adapter: routed + shared expert through linear() and the float gate
    p = "target.layers.0.mlp"
    shared = F.silu(q.linear(x, p + ".shared_expert.gate_proj.weight")) * q.linear(x, p + ".shared_expert.up_proj.weight")
    shared = q.linear(shared, p + ".shared_expert.down_proj.weight")
    gate = torch.sigmoid(F.linear(x, lw.shared.gate_weight.reshape(1, -1).to(x.dtype)))
    composed = routed + shared * gate
    fused = pkg.ops.moe_w4a16(xb, lw.gate_up, lw.down, top_k=c.top_k, router_weight=lw.router, shared=lw.shared)
    rep = metrics.compare(composed.reshape(16, -1).float().cpu(), fused.float().cpu())
    print(f"  composed vs fused shared expert: {rep}", flush=True)
    assert rep["max_rel"] <= 2e-2 and rep["cosine"] > 0.999


@pytest.mark.gpu
def test_packed_router_routes_on_unrounded_logits(pkg, device):
    """A packed int4 router (``linear_int4`` in the portable plan): its logits come from the
    fp32-output qlinear, unrounded, and the layer's routing is bit-exact against the oracle's
    top-k and permutation of those very logits (``fused/quantization.py:183-192``)."""
    from oracle import moe as oracle_moe, routing as oracle_routing, w4 as oracle_w4
    c = pkg.target.small_config()
    c = type(c)(**{**vars(c), "linear_value_heads": 32, "experts": 32})   # router rows: qlinear N % 32
    w = pkg.target.random_weights(c, seed=5, device=device, layout="portable")
    q0 = pkg.quantized.from_target_weights(w, layout="portable")
    key = "target.layers.0.mlp.gate.weight"
    gen = torch.Generator().manual_seed(6)
    router = pkg.synthetic.int4_weight(gen, (c.experts, c.hidden))
    banks = dict(q0._banks)
    banks[key] = pkg.PackedW4(router.packed.to(device), router.scales.to(device), router.group_size)
    routers = {k: v for k, v in q0._routers.items() if k != key}
    q = pkg.quantized.QuantizedWeights(q0.shapes, banks, (w.embedding, w.embedding_scale), routers=routers)
    x = torch.randn((1, 16, c.hidden), generator=gen).to(device)
    xb = x.reshape(16, -1).to(torch.bfloat16)
    logits = q.router_logits(xb, key)
    assert logits.dtype == torch.float32
    ref_logits = oracle_w4.qlinear(xb.cpu(), router.packed.numpy(), router.scales, 128)
    ref_logits = torch.as_tensor(ref_logits, dtype=torch.float64)
    err = (logits.double().cpu() - ref_logits).abs().max() / ref_logits.abs().max()
    assert err < 1e-5, err                                             # fp32 sums, not a bf16 rounding
    assert not torch.equal(logits, logits.to(torch.bfloat16).float())
    lw = w.layers[0]
    gu, dn = lw.gate_up.tiled(), lw.down.tiled()
    out, r, used = pkg.ops.moe_w4a16(xb, gu, dn, top_k=c.top_k, router_logits=logits, return_routing=True)
    ids, wts = oracle_routing.topk(used.cpu().numpy(), c.top_k)
    perm, inv, offsets = oracle_routing.permutation(ids, c.experts)
    assert torch.equal(r.ids.cpu(), torch.from_numpy(ids))
    assert torch.equal(r.perm.cpu(), torch.from_numpy(perm)) and torch.equal(r.inv.cpu(), torch.from_numpy(inv))
    assert torch.equal(r.offsets.cpu(), torch.from_numpy(offsets))
    torch.testing.assert_close(r.weights.cpu(), torch.from_numpy(wts), rtol=2e-6, atol=2e-6)
    routed = q.moe(x, "target.layers.0.mlp", top_k=c.top_k)
    assert torch.equal(routed.reshape(16, -1), out.to(torch.float16))
    golden = oracle_moe.moe(xb.cpu(), logits.cpu().numpy(), c.top_k, (lw.gate_up.packed.cpu(), lw.gate_up.scales.cpu()),
                            (lw.down.packed.cpu(), lw.down.scales.cpu()), 128)
    rep = metrics.compare(out.cpu(), golden["out_f32"])
    assert rep["max_rel"] <= metrics.MAX_REL_TOLERANCE, rep
