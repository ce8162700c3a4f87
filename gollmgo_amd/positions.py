"""The device decision returned as the engine's `StepOutput.LogitsPerPosition`.

The engine (internal/engine/serving.go:496-570) takes the verify result from per-position
logit rows: `Verify(drafts, rows[:K])` (internal/engine/speculative.go:68-84) gives the
accepted count and the corrected token (argmax of the first mismatching row), and on full
acceptance `Sampler.Sample(rows[K])` gives the bonus token. The device already decided
`(accepted, token)` for every sequence, so a runner hands back rows that make the engine's
own code reach that decision, as the reference's mock runner does with ragged one-hot rows
(internal/backend/mock_runner.go:44-61):

  row j < accepted   one-hot at drafts[j]   (Verify: argmax == draft, accepted)
  row accepted       one-hot at token       (Verify: argmax == token != draft -> corrected;
                                             or, after the last draft, Sample -> token)

The row for token t is the shortest legal one: length t + 1, -inf before t and 0 at t.
argmax returns t (the only finite maximum), and every Sampler setting returns t: softmax
maps -inf to 0 (sampling.go:112-136), so t holds probability 1 under any temperature,
top-k or top-p. All rows are views into one constant buffer of V -inf values followed by
a 0 (row t = buffer[V - t:]); building them copies nothing, so the host cost of the return
path is the engine's own scans (argmax reads t + 1 floats per row). Neither Verify nor
Sample writes to its rows, so the views can be shared.

The decision is always representable: a rejected draft is never the returned token (the
greedy correction is an argmax that differs from the draft; the rejection sampler's
residual is 0 at the rejected draft), which `rows_for` checks.
"""
from __future__ import annotations

import numpy as np


class LogitsPerPosition:
    """One-hot row views over a vocabulary of `vocab` tokens (float32, like the engine's rows)."""

    def __init__(self, vocab: int):
        if vocab < 1:
            raise ValueError("vocab must be positive")
        self.vocab = vocab
        self._base = np.full(vocab + 1, -np.inf, dtype=np.float32)
        self._base[vocab] = 0.0
        self._base.setflags(write=False)

    def row(self, token: int) -> np.ndarray:
        """The row whose argmax and every sample is `token`: length token + 1."""
        if not 0 <= token < self.vocab:
            raise ValueError(f"token {token} outside [0, {self.vocab})")
        return self._base[self.vocab - token:]

    def rows_for(self, drafts, n_drafts: int, accepted: int, token: int) -> list[np.ndarray]:
        """The rows of one sequence: accepted + 1 of them (drafts[0..accepted) then token)."""
        if not 0 <= accepted <= n_drafts:
            raise ValueError(f"accepted {accepted} outside [0, {n_drafts}]")
        if accepted < n_drafts and int(drafts[accepted]) == token:
            raise ValueError("the token after a rejected draft equals that draft")
        out = [self.row(int(drafts[j])) for j in range(accepted)]
        out.append(self.row(token))
        return out

    def batch(self, drafts, n_drafts, accepted, tokens) -> list[list[np.ndarray]]:
        """LogitsPerPosition of a step from host copies of the device outputs:
        drafts [B][K], n_drafts [B], accepted [B], tokens [B]."""
        drafts = np.asarray(drafts)
        K = drafts.shape[1] if drafts.ndim == 2 else 0
        out = []
        for b in range(len(accepted)):
            n = min(max(int(n_drafts[b]), 0), K)
            out.append(self.rows_for(drafts[b], n, int(accepted[b]), int(tokens[b])))
        return out
