"""Target session with a batched speculative verify (one forward per proposal block).

The reference session (``model/qwen35_moe_dflash/fused/session.py:243-391``)
verifies a DFlash proposal block token by token: one target forward per
proposal, a cloned state checkpoint after each (``StateTransaction.record``,
``:111-175``), then ``commit(r)`` publishes checkpoint ``r``.  Here the block is
one forward of ``T`` tokens (``target.TargetModel``), and the checkpoints are
implicit: the forward's ``Pending`` record rebuilds the state after any prefix
``r`` of the block (KV rows are already in place, the conv history is a slice
of the block's window, the GDN state comes from the block's delta-rule writes).

Same observable contract as the reference's ``FusedTargetSession``:

* ``prefill(ids)`` once on an empty session; ``step(token)`` consumes one token;
* ``next_token`` is the target's prediction after the committed prefix,
  ``last_features`` the committed last token's feature row ``[1, 1, F]``;
* ``verify(proposals)`` returns a :class:`Verification` whose
  ``expected_next_tokens[i]`` is the prediction *before* consuming proposal
  ``i`` (the last entry is the bonus prediction after the block),
  ``max_accepted_prefix`` the number of leading proposals that match, and
  ``commit(r)`` (``0 <= r <= max_accepted_prefix``) / ``abort()``;
* a verification made stale by a later commit or step raises on commit
  ("stale state transaction").  Because the block's KV rows are written in
  place past the committed position, a newer ``verify`` or ``step`` also makes
  an open verification stale.
"""
from __future__ import annotations

from threading import RLock
from typing import Optional, Sequence

import torch
from torch import Tensor

from .target import Output, TargetModel


def _tokens(values, vocab: int) -> list:
    if isinstance(values, Tensor):
        if values.dtype not in (torch.int32, torch.int64) or values.ndim != 2 or values.shape[0] != 1:
            raise ValueError("token tensor must be an integer [1, sequence] tensor")
        values = values.detach().cpu().tolist()[0]
    elif isinstance(values, (str, bytes)) or not isinstance(values, Sequence):
        raise ValueError("tokens must be a sequence of integers or a [1,S] tensor")
    out = []
    for v in values:
        if type(v) is not int or not 0 <= v < vocab:
            raise ValueError("token IDs must be integers inside the vocabulary, not bool")
        out.append(v)
    if not out:
        raise ValueError("tokens must contain at least one token; padding is not inferred")
    return out


class VerifySession:
    def __init__(self, model: TargetModel, *, block_limit: int = 2048):
        self.model = model
        self._state = model.new_state()
        self._generation = 0
        self._prefilled = False
        self._next_token: Optional[int] = None
        self._last_features: Optional[Tensor] = None
        self._block_limit = block_limit
        self._lock = RLock()

    # -- committed view
    @property
    def position(self) -> int:
        return self._state.position

    @property
    def state(self):
        with self._lock:
            return self._state.clone()

    @property
    def next_token(self) -> int:
        with self._lock:
            self._require_prefill()
            return self._next_token

    @property
    def last_features(self) -> Tensor:
        with self._lock:
            self._require_prefill()
            return self._last_features.clone()

    def _require_prefill(self):
        if not self._prefilled:
            raise RuntimeError("prefill must complete before decoding or verification")

    def _ids(self, values: list) -> Tensor:
        return torch.tensor(values, dtype=torch.int64, device=self.model.device)

    def _run(self, values: list) -> Output:
        if self._state.position + len(values) > self.model.capacity:
            raise ValueError("input would exceed the target context capacity")
        return self.model.forward(self._ids(values), self._state)

    @staticmethod
    def _features_row(out: Output, i: int) -> Optional[Tensor]:
        return None if out.features is None else out.features[i:i + 1][None].clone()

    # -- transitions
    def prefill(self, ids) -> Output:
        values = _tokens(ids, self.model.config.vocab)
        with self._lock:
            if self._prefilled or self._state.position != 0:
                raise RuntimeError("prefill is allowed only once on an empty session")
            out = None
            for start in range(0, len(values), self._block_limit):
                out = self._run(values[start:start + self._block_limit])
                self.model.commit(self._state, out.pending, out.pending.tokens)
            self._generation += 1
            self._next_token = int(out.top1[-1])
            self._last_features = self._features_row(out, out.pending.tokens - 1)
            self._prefilled = True
            return out

    def step(self, token: int) -> Output:
        values = _tokens([token], self.model.config.vocab)
        with self._lock:
            self._require_prefill()
            out = self._run(values)
            self.model.commit(self._state, out.pending, 1)
            self._generation += 1
            self._next_token = int(out.top1[0])
            self._last_features = self._features_row(out, 0)
            return out

    def verify(self, proposals) -> "Verification":
        values = _tokens(proposals, self.model.config.vocab)
        with self._lock:
            self._require_prefill()
            if len(values) > self._block_limit:
                raise ValueError("proposal block longer than the session's block limit")
            if self._state.position + len(values) > self.model.capacity:
                raise ValueError("input would exceed the target context capacity")
            # the forward writes this block's KV rows where an older open verification keeps its
            # own (one pending region per session), so from here that verification is stale;
            # a refused block above leaves it open
            self._generation += 1
            out = self._run(values)
            predicted = out.top1.tolist()
            expected = (self._next_token, *predicted)
            accepted = 0
            while accepted < len(values) and values[accepted] == expected[accepted]:
                accepted += 1
            return Verification(self, self._generation, out, expected, accepted)

    def _commit(self, generation: int, out: Output, accepted: int, expected: tuple) -> None:
        with self._lock:
            if generation != self._generation:
                raise RuntimeError("stale state transaction: another branch has committed")
            self.model.commit(self._state, out.pending, accepted)
            self._generation += 1
            self._next_token = expected[accepted]
            if accepted:
                self._last_features = self._features_row(out, accepted - 1)


class Verification:
    """An uncommitted verification of one proposal block (``fused/session.py:344-391``)."""

    def __init__(self, session: VerifySession, generation: int, out: Output, expected: tuple, accepted: int):
        self._session = session
        self._generation = generation
        self._out = out
        self._expected = tuple(int(v) for v in expected)
        self._accepted = accepted
        self._closed = False

    @property
    def expected_next_tokens(self) -> tuple:
        return self._expected

    @property
    def max_accepted_prefix(self) -> int:
        return self._accepted

    @property
    def closed(self) -> bool:
        return self._closed

    @property
    def output(self) -> Output:
        return self._out

    def commit(self, accepted: int):
        if self._closed:
            raise RuntimeError("state transaction is closed")
        if type(accepted) is not int or not 0 <= accepted <= self._accepted:
            raise ValueError("accepted count exceeds the matching proposal prefix")
        self._session._commit(self._generation, self._out, accepted, self._expected)
        self._closed = True
        self._out = None
        return self._session.state

    def abort(self) -> None:
        if self._closed:
            raise RuntimeError("state transaction is closed")
        self._closed = True
        self._out = None
