"""CPU: the FusedOps adapter module (seam 1) and its six non-hot operations.

Admission: the checks ``ModuleFusedOps`` applies before binding a module
(``model/qwen35_moe_dflash/fused/ops.py:148-176``) are restated here as
plain predicates and applied to ``fused_ops``.

The non-hot operations run on whatever device their inputs are on; here they
are pinned on the CPU against closed forms, invariants, library routines that
compute the same textbook operation (``F.conv1d``, ``F.scaled_dot_product_attention``),
and -- for the gated delta rule, whose product code is a chunked closed form --
the token-by-token recurrence it must equal (the FusedOps protocol defines the
operation by that recurrence, ``fused/ops.py:54-71``).
"""
import math
from types import ModuleType

import pytest
import torch
import torch.nn.functional as F

REQUIRED = ("rms_norm", "conv_state_update", "causal_conv1d", "chunk_gated_delta_rule", "cache_update",
            "attention", "moe")


@pytest.fixture(scope="module")
def fo(pkg):
    return pkg.fused_ops


# ------------------------------------------------------------------ admission (seam 1)
def admit(module, *, allow_reference=False):
    """The admission rules of ``ModuleFusedOps.__init__`` (``fused/ops.py:148-176``), as predicates."""
    if not isinstance(module, ModuleType):
        raise TypeError("fused operators require an explicit Python adapter module")
    version = getattr(module, "FUSED_OPS_ABI", None)
    if type(version) is not int or version != 1:
        raise ValueError("fused adapter must declare FUSED_OPS_ABI=1")
    backend = getattr(module, "BACKEND_ID", None)
    if not isinstance(backend, str) or not backend.strip():
        raise ValueError("fused adapter must declare a nonempty BACKEND_ID")
    reference = getattr(module, "IS_REFERENCE_BACKEND", False)
    if type(reference) is not bool:
        raise ValueError("IS_REFERENCE_BACKEND must be a bool when declared")
    if reference and not allow_reference:
        raise ValueError("host reference backend requires explicit allow_reference=True")
    missing = [n for n in REQUIRED if not callable(getattr(module, n, None))]
    if missing:
        raise ValueError("fused adapter is missing callable operations: " + ", ".join(missing))
    return {n: getattr(module, n) for n in REQUIRED}


def test_module_is_admitted_without_allow_reference(fo):
    bound = admit(fo)
    assert set(bound) == set(REQUIRED)
    assert fo.FUSED_OPS_ABI == 1 and type(fo.FUSED_OPS_ABI) is int
    assert fo.BACKEND_ID == "mi355x-hip" and fo.IS_REFERENCE_BACKEND is False
    assert callable(fo.qlinear)


def test_admission_rules_reject_broken_modules(fo):
    """The restated rules are live: each mutation of a copy of the module fails the way
    ``ModuleFusedOps`` would."""
    def clone(**changes):
        m = ModuleType("probe")
        m.__dict__.update({k: getattr(fo, k) for k in ("FUSED_OPS_ABI", "BACKEND_ID", "IS_REFERENCE_BACKEND",
                                                       *REQUIRED)})
        for k, v in changes.items():
            if v is None:
                delattr(m, k)
            else:
                setattr(m, k, v)
        return m
    for change, message in (({"FUSED_OPS_ABI": True}, "FUSED_OPS_ABI"), ({"FUSED_OPS_ABI": 2}, "FUSED_OPS_ABI"),
                            ({"BACKEND_ID": "  "}, "BACKEND_ID"), ({"IS_REFERENCE_BACKEND": 1}, "bool"),
                            ({"IS_REFERENCE_BACKEND": True}, "allow_reference"), ({"moe": None}, "moe"),
                            ({"attention": 3}, "attention")):
        with pytest.raises(ValueError, match=message):
            admit(clone(**change))
    with pytest.raises(TypeError):
        admit(object())


# ------------------------------------------------------------------ rms_norm
def test_rms_norm_closed_forms(fo):
    x = torch.full((3, 8), -2.0)
    gamma = torch.arange(1.0, 9.0)
    out = fo.rms_norm(x, gamma, 1e-6)
    torch.testing.assert_close(out, -gamma.expand(3, 8) * (2.0 / math.sqrt(4.0 + 1e-6)), rtol=1e-6, atol=0)
    y = torch.randn((5, 64), generator=torch.Generator().manual_seed(0))
    unit = fo.rms_norm(y, torch.ones(64), 1e-12)
    torch.testing.assert_close(unit.square().mean(-1), torch.ones(5), rtol=1e-5, atol=0)
    torch.testing.assert_close(fo.rms_norm(7.5 * y, torch.ones(64), 1e-12), unit, rtol=1e-5, atol=1e-6)


def test_rms_norm_rounds_once_then_scales(fo):
    """bf16 input: the normalised value is rounded to bf16 before the gamma product."""
    x = torch.randn((4, 32), generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    gamma = torch.rand(32, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16) + 0.5
    xf = x.float()
    normed = (xf / torch.sqrt(xf.square().mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16)
    assert torch.equal(fo.rms_norm(x, gamma, 1e-6), normed * gamma)


@pytest.mark.parametrize("eps,gamma_len", [(0.0, 8), (float("nan"), 8), (1e-6, 7)])
def test_rms_norm_contract_errors(fo, eps, gamma_len):
    with pytest.raises(ValueError, match="RMSNorm needs positive epsilon and one gamma per feature"):
        fo.rms_norm(torch.ones((2, 8)), torch.ones(gamma_len), eps)


# ------------------------------------------------------------------ conv state + depthwise conv
def test_conv_state_update_window_and_history(fo):
    gen = torch.Generator().manual_seed(3)
    proj = torch.randn((2, 5, 6), generator=gen)
    hist = torch.randn((2, 6, 3), generator=gen)
    new_hist, window = fo.conv_state_update(proj, hist)
    assert torch.equal(window, torch.cat([hist, proj.transpose(1, 2)], dim=2))
    assert torch.equal(new_hist, window[:, :, -3:]) and new_hist.data_ptr() != window.data_ptr()
    # chaining two updates equals one update over the concatenated tokens
    a, b = proj[:, :2], proj[:, 2:]
    h1, _ = fo.conv_state_update(a, hist)
    h2, _ = fo.conv_state_update(b, h1)
    assert torch.equal(h2, new_hist)
    # no history columns (kernel width 1)
    h0, w0 = fo.conv_state_update(proj, torch.zeros((2, 6, 0)))
    assert h0.shape == (2, 6, 0) and torch.equal(w0, proj.transpose(1, 2))


def test_conv_state_update_contract_errors(fo):
    with pytest.raises(ValueError, match="conv state requires projected"):
        fo.conv_state_update(torch.zeros((1, 4, 6)), torch.zeros((1, 5, 3)))
    with pytest.raises(ValueError, match="conv state requires projected"):
        fo.conv_state_update(torch.zeros((1, 4, 6)), torch.zeros((1, 6, 3), dtype=torch.float16))


def test_causal_conv1d_against_conv1d_and_impulses(fo):
    gen = torch.Generator().manual_seed(4)
    padded = torch.randn((2, 8, 3 + 16), generator=gen)
    weight = torch.randn((8, 1, 4), generator=gen)
    out = fo.causal_conv1d(padded, weight)
    assert out.shape == (2, 16, 8)
    torch.testing.assert_close(out, F.conv1d(padded, weight, groups=8).transpose(1, 2), rtol=1e-5, atol=1e-5)
    # an impulse at window position p reaches output s = p - j through tap j
    imp = torch.zeros((1, 8, 3 + 5))
    imp[0, :, 4] = 1.0
    resp = fo.causal_conv1d(imp, weight)[0]          # [S, C]
    for s in range(5):
        j = 4 - s
        expect = weight[:, 0, j] if 0 <= j < 4 else torch.zeros(8)
        torch.testing.assert_close(resp[s], expect)


def test_causal_conv1d_contract_errors(fo):
    with pytest.raises(ValueError, match="depthwise conv requires"):
        fo.causal_conv1d(torch.zeros((1, 8, 2)), torch.zeros((8, 1, 4)))
    with pytest.raises(ValueError, match="depthwise conv requires"):
        fo.causal_conv1d(torch.zeros((1, 8, 6)), torch.zeros((8, 2, 4)))


# ------------------------------------------------------------------ gated delta rule
def recurrence(q, k, v, g, beta, state, length, l2norm):
    """The gated delta rule token by token (``fused/ops.py:54-71``): per head,
    S <- e^g S;  u = beta (v - S^T k);  S <- S + k u^T;  o = S^T q  (q scaled by Dk^-1/2)."""
    q, k, v, g, beta = (t.double() for t in (q, k, v, g, beta))
    if l2norm:
        q = q / torch.sqrt(q.square().sum(-1, keepdim=True) + 1e-6)
        k = k / torch.sqrt(k.square().sum(-1, keepdim=True) + 1e-6)
    q = q * q.shape[-1] ** -0.5
    b, s, h, _ = q.shape
    st = state.double().clone()
    out = torch.zeros((b, s, h, v.shape[-1]), dtype=torch.float64)
    for bi in range(b):
        for t in range(int(length[bi])):
            for hi in range(h):
                S = st[bi, hi] * math.exp(float(g[bi, t, hi]))
                u = float(beta[bi, t, hi]) * (v[bi, t, hi] - S.T @ k[bi, t, hi])
                S = S + torch.outer(k[bi, t, hi], u)
                st[bi, hi] = S
                out[bi, t, hi] = S.T @ q[bi, t, hi]
    return out, st


def _gdn_inputs(seed, b=1, s=16, h=3, dk=8, dv=5):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn((b, s, h, dk), generator=gen)
    k = torch.randn((b, s, h, dk), generator=gen)
    v = torch.randn((b, s, h, dv), generator=gen)
    g = -torch.rand((b, s, h), generator=gen) * 0.5
    beta = torch.rand((b, s, h), generator=gen)
    state = torch.randn((b, h, dk, dv), generator=gen) * 0.3
    return q, k, v, g, beta, state


@pytest.mark.parametrize("s,l2", [(1, True), (16, True), (16, False), (64, True), (65, True), (130, True)])
def test_gdn_chunk_form_equals_the_recurrence(fo, s, l2):
    q, k, v, g, beta, state = _gdn_inputs(10 + s, b=2, s=s)
    length = torch.tensor([s, max(0, s - 3)], dtype=torch.int16)
    core, final = fo.chunk_gated_delta_rule(q, k, v, g, beta, state, length, chunk_size=64 if s > 1 else 1,
                                            use_qk_l2norm_in_kernel=l2)
    ref_core, ref_state = recurrence(q, k, v, g, beta, state, length, l2)
    assert core.dtype == torch.float32 and final.dtype == torch.float32
    torch.testing.assert_close(core.double(), ref_core, rtol=2e-5, atol=2e-5)
    torch.testing.assert_close(final.double(), ref_state, rtol=2e-5, atol=2e-5)


def test_gdn_zero_beta_only_decays(fo):
    """beta = 0: nothing is written; S_t = e^{G_t} S_0 and o_t = S_t^T q_t."""
    q, k, v, g, beta, state = _gdn_inputs(20)
    core, final = fo.chunk_gated_delta_rule(q, k, v, g, torch.zeros_like(beta), state,
                                            torch.tensor([16], dtype=torch.int16), chunk_size=64,
                                            use_qk_l2norm_in_kernel=False)
    cum = torch.cumsum(g[0], dim=0)                                     # [S, H]
    torch.testing.assert_close(final[0], state[0] * cum[-1].exp()[:, None, None], rtol=1e-5, atol=1e-6)
    expect = torch.einsum("sh,hkv,shk->shv", cum.exp(), state[0], q[0] * 8 ** -0.5)
    torch.testing.assert_close(core[0], expect, rtol=1e-5, atol=1e-6)


def test_gdn_stores_values_exactly_at_orthonormal_keys(fo):
    """g = 0, beta = 1, orthonormal keys: the delta rule writes v_i at key k_i exactly, so a
    query equal to k_i reads back v_i (times the Dk^-1/2 query scale)."""
    dk, dv, s = 8, 4, 5
    basis, _ = torch.linalg.qr(torch.randn((dk, dk), generator=torch.Generator().manual_seed(5), dtype=torch.float64))
    keys = basis[:s].float()
    v = torch.randn((1, s, 1, dv), generator=torch.Generator().manual_seed(6))
    k = keys[None, :, None, :]
    state = torch.randn((1, 1, dk, dv), generator=torch.Generator().manual_seed(7))
    _, final = fo.chunk_gated_delta_rule(k.clone(), k, v, torch.zeros((1, s, 1)), torch.ones((1, s, 1)), state,
                                         torch.tensor([s], dtype=torch.int16), chunk_size=64,
                                         use_qk_l2norm_in_kernel=False)
    torch.testing.assert_close(keys @ final[0, 0], v[0, :, 0], rtol=1e-5, atol=1e-5)


def test_gdn_effective_length_and_chaining(fo):
    """Tokens past effective_length change nothing and output zeros; running 10 then 6 tokens
    from the carried state equals running 16 at once."""
    q, k, v, g, beta, state = _gdn_inputs(30)
    full_core, full_state = fo.chunk_gated_delta_rule(q, k, v, g, beta, state, torch.tensor([16], dtype=torch.int16),
                                                      chunk_size=64, use_qk_l2norm_in_kernel=True)
    part_core, part_state = fo.chunk_gated_delta_rule(q, k, v, g, beta, state, torch.tensor([10], dtype=torch.int16),
                                                      chunk_size=64, use_qk_l2norm_in_kernel=True)
    assert torch.count_nonzero(part_core[:, 10:]) == 0
    head_core, head_state = fo.chunk_gated_delta_rule(q[:, :10], k[:, :10], v[:, :10], g[:, :10], beta[:, :10],
                                                      state, torch.tensor([10], dtype=torch.int16), chunk_size=64,
                                                      use_qk_l2norm_in_kernel=True)
    torch.testing.assert_close(part_state, head_state)
    torch.testing.assert_close(part_core[:, :10], head_core)
    tail_core, tail_state = fo.chunk_gated_delta_rule(q[:, 10:], k[:, 10:], v[:, 10:], g[:, 10:], beta[:, 10:],
                                                      head_state, torch.tensor([6], dtype=torch.int16),
                                                      chunk_size=64, use_qk_l2norm_in_kernel=True)
    torch.testing.assert_close(tail_state, full_state, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(torch.cat([head_core, tail_core], 1), full_core, rtol=1e-5, atol=1e-6)


def test_gdn_fp16_state_round_trip(fo):
    q, k, v, g, beta, state = _gdn_inputs(40)
    core, final = fo.chunk_gated_delta_rule(q.half(), k.half(), v.half(), g.half(), beta.half(), state.half(),
                                            torch.tensor([16], dtype=torch.int16), chunk_size=64,
                                            use_qk_l2norm_in_kernel=True)
    assert core.dtype == torch.float16 and final.dtype == torch.float16


@pytest.mark.parametrize("kwargs,message", [
    ({"chunk_size": 32}, "chunk_size must be 1 or 64"),
    ({"chunk_size": True}, "chunk_size must be 1 or 64"),
    ({"use_qk_l2norm_in_kernel": 1}, "must be bool"),
    ({"state_shape": (1, 3, 8, 4)}, "initial_state must be FP16/FP32"),
    ({"length": torch.tensor([17], dtype=torch.int16)}, "effective_length must be INT16"),
    ({"length": torch.tensor([16], dtype=torch.int32)}, "effective_length must be INT16"),
    ({"gate_shape": (1, 16, 2)}, "GDN requires compatible"),
    ({"dtype": torch.bfloat16}, "GDN floating inputs"),
])
def test_gdn_contract_errors(fo, kwargs, message):
    q, k, v, g, beta, state = _gdn_inputs(50)
    if "state_shape" in kwargs:
        state = torch.zeros(kwargs["state_shape"])
    if "gate_shape" in kwargs:
        g = torch.zeros(kwargs["gate_shape"])
    if "dtype" in kwargs:
        q, k, v, g, beta = (t.to(kwargs["dtype"]) for t in (q, k, v, g, beta))
    length = kwargs.get("length", torch.tensor([16], dtype=torch.int16))
    with pytest.raises(ValueError, match=message):
        fo.chunk_gated_delta_rule(q, k, v, g, beta, state, length, chunk_size=kwargs.get("chunk_size", 64),
                                  use_qk_l2norm_in_kernel=kwargs.get("use_qk_l2norm_in_kernel", True))


# ------------------------------------------------------------------ KV cache + attention
def test_cache_update_appends_private_copies(fo):
    gen = torch.Generator().manual_seed(8)
    k0, v0 = torch.randn((1, 2, 5, 4), generator=gen), torch.randn((1, 2, 5, 4), generator=gen)
    k1, v1 = torch.randn((1, 2, 3, 4), generator=gen), torch.randn((1, 2, 3, 4), generator=gen)
    nk, nv = fo.cache_update(k0, v0, k1, v1)
    assert torch.equal(nk[:, :, :5], k0) and torch.equal(nk[:, :, 5:], k1) and torch.equal(nv[:, :, 5:], v1)
    ek, ev = fo.cache_update(None, None, k1, v1)
    assert torch.equal(ek, k1) and ek.data_ptr() != k1.data_ptr() and ev.data_ptr() != v1.data_ptr()
    with pytest.raises(ValueError, match="KV caches must appear together"):
        fo.cache_update(k0, None, k1, v1)
    with pytest.raises(ValueError, match="dimensions/dtypes do not match"):
        fo.cache_update(k0.half(), v0.half(), k1, v1)
    with pytest.raises(ValueError, match="lengths differ"):
        fo.cache_update(k0, v0[:, :, :4], k1, v1)


def _attn_case(seed, b=1, heads=4, kv=2, s=3, start=5, d=8):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn((b, heads, s, d), generator=gen)
    key = torch.randn((b, kv, start + s, d), generator=gen)
    val = torch.randn((b, kv, start + s, d), generator=gen)
    return q, key, val


def test_attention_matches_sdpa_with_repeated_heads(fo):
    q, key, val = _attn_case(9, heads=16, kv=2, s=16, start=40, d=32)
    out = fo.attention(q, key, val, query_start=40, scale=32 ** -0.5)
    rep = 8
    visible = torch.arange(56)[None, :] <= (torch.arange(16) + 40)[:, None]
    ref = F.scaled_dot_product_attention(q, key.repeat_interleave(rep, 1), val.repeat_interleave(rep, 1),
                                         attn_mask=visible, scale=32 ** -0.5)
    torch.testing.assert_close(out, ref, rtol=1e-5, atol=1e-5)


def test_attention_causal_window_closed_form(fo):
    """Equal keys: every visible position gets the same weight, so row i is the mean of the
    first query_start + i + 1 values."""
    q, key, val = _attn_case(10)
    key = torch.ones_like(key)
    out = fo.attention(q, key, val, query_start=5, scale=0.5)
    for h in range(4):
        for i in range(3):
            torch.testing.assert_close(out[0, h, i], val[0, h // 2, :6 + i].mean(0), rtol=1e-5, atol=1e-6)


def test_attention_contract_errors(fo):
    q, key, val = _attn_case(11)
    for kwargs in ({"query_start": 4}, {"query_start": True}, {"query_start": 5, "scale": 0.0}):
        with pytest.raises(ValueError, match="attention requires causal append-only GQA"):
            fo.attention(q, key, val, query_start=kwargs["query_start"], scale=kwargs.get("scale", 1.0))
    with pytest.raises(ValueError, match="attention requires causal append-only GQA"):
        fo.attention(q[:, :3], key, val, query_start=5, scale=1.0)     # 3 heads over 2 KV heads
