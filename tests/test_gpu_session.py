"""GPU: the batched verify session against the serial one it replaces.

The reference verifies a proposal block token by token (one forward and one state
checkpoint per proposal, ``fused/session.py:316-341``).  ``VerifySession.verify`` runs
the block as one forward; its observable results must be those of the serial
procedure: the expected next tokens (the prediction before each proposal, and the
bonus after the block), the accepted prefix, and -- after ``commit(r)`` -- the state,
next token and last feature row that ``r`` serial ``step`` calls leave.  The serial
procedure here is this same session's ``step`` (one-token forwards), so the check is
batched-vs-serial on identical weights.  Data are seeded on the CPU and the kernels are
deterministic; the greedy tokens' top-2 logit margins are asserted to exceed the
batched/serial difference, so the token comparisons cannot flip on a near-tie.
"""
import pytest
import torch

from oracle import metrics

pytestmark = pytest.mark.gpu


def _model(pkg, device, seed=21):
    c = pkg.target.small_config()
    host = pkg.target.random_weights(c, seed=seed, device="cpu", layout="portable", generate_on="cpu")
    w = pkg.target.to_device(host, device, layout="tiled")
    return c, pkg.target.TargetModel(w, capacity=128, feature_layers=(0, 1))


def test_batched_verify_equals_serial_steps(pkg, device):
    c, model = _model(pkg, device)
    prefix = torch.randint(0, c.vocab, (24,), generator=torch.Generator().manual_seed(1)).tolist()
    serial = pkg.session.VerifySession(model)
    serial.prefill(prefix)
    greedy = []
    for _ in range(3):
        t = serial.next_token
        greedy.append(t)
        serial.step(t)
    after3 = serial.next_token
    wrong = (after3 + 1) % c.vocab
    proposals = greedy + [wrong, 5, 9, 11, 13]
    print(f"session: greedy {greedy} then {after3}; proposals {proposals}", flush=True)

    batched = pkg.session.VerifySession(model)
    batched.prefill(prefix)
    assert batched.next_token == greedy[0]
    v = batched.verify(proposals)
    assert v.max_accepted_prefix == 3
    assert v.expected_next_tokens[:4] == (greedy[0], greedy[1], greedy[2], after3)
    assert len(v.expected_next_tokens) == len(proposals) + 1
    # logits of the block rows the serial run also computed: within the bf16 bar, and the
    # greedy choices are separated by far more than that
    final = v.output.hidden[:3].to(torch.bfloat16)
    block_logits = pkg.ops.qlinear(final, model.w.lm_head).float()
    top2 = block_logits.topk(2, dim=-1).values
    assert bool(((top2[:, 0] - top2[:, 1]) > 0.05).all()), top2
    state = v.commit(3)
    assert batched.position == serial.position == 27 and state.position == 27
    assert batched.next_token == after3
    a, b = batched.state, serial.state
    for i in range(c.layers):
        if a.recurrent[i] is not None:
            r = metrics.compare(a.recurrent[i].cpu(), b.recurrent[i].cpu())
            assert r["max_rel"] <= 1e-2, r
            assert metrics.compare(a.conv[i].float().cpu(), b.conv[i].float().cpu())["max_rel"] <= 1e-2
        else:
            r = metrics.compare(a.keys[i][:, :, :27].float().cpu(), b.keys[i][:, :, :27].float().cpu())
            assert r["max_rel"] <= 1e-2, r
    fa, fb = batched.last_features, serial.last_features
    assert tuple(fa.shape) == (1, 1, 2 * c.hidden)
    assert metrics.compare(fa.float().cpu(), fb.float().cpu())["max_rel"] <= 1e-2
    # both sessions continue identically from the committed state
    assert batched.step(after3).top1.tolist() == serial.step(after3).top1.tolist()


def test_verify_transactions(pkg, device):
    c, model = _model(pkg, device, seed=22)
    s = pkg.session.VerifySession(model)
    with pytest.raises(RuntimeError, match="prefill"):
        s.verify([1, 2])
    s.prefill([3, 4, 5, 6])
    with pytest.raises(RuntimeError, match="only once"):
        s.prefill([1])
    with pytest.raises(ValueError):
        s.verify([c.vocab])
    with pytest.raises(ValueError):
        s.verify([])
    v1 = s.verify([7, 8, 9])
    v2 = s.verify([7, 8, 9])
    with pytest.raises(RuntimeError, match="stale"):
        v1.commit(0)
    # a block the context cannot hold is refused before it runs and leaves v2 open
    with pytest.raises(ValueError, match="capacity"):
        s.verify([1] * (model.capacity - s.position + 1))
    with pytest.raises(ValueError, match="exceeds"):
        v2.commit(v2.max_accepted_prefix + 1)
    before = s.state
    v2.commit(0)
    after = s.state
    assert after.position == before.position == 4
    assert torch.equal(after.recurrent[0], before.recurrent[0])
    with pytest.raises(RuntimeError, match="closed"):
        v2.commit(0)
    v3 = s.verify([s.next_token, 1])
    assert v3.max_accepted_prefix >= 1
    v3.abort()
    with pytest.raises(RuntimeError, match="closed"):
        v3.commit(0)
    s.step(2)
    assert s.position == 5
