"""Device drafting for a runner: each sequence's token history kept on the device and the
next step drafted there, right after the acceptance (gg_history_append_draft).

This is the Python twin of the Go runner's drafts.go (internal/backend/rocm/drafts.go),
line for line in its bookkeeping, so the flow is tested here. The engine drafts with
NGramDrafter.Draft over seq.TokenIDs (maybeDraft, internal/engine/serving.go:608-620);
a runner that serves drafts answers `drafts(seq_id, hist_len)` only when its own history
of the sequence has the engine's length, so any divergence falls back to the host drafter.

The host keeps a mirror of every history (the truth). A device row is (re)seeded from it
whenever the row's length does not match: a sequence seen for the first time after its
prefill, a rewritten position, an evicted row. Per step only the B*K next drafts and their
counts come back, with the decision.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import numpy as np
import torch

from . import verify as gv


@dataclass
class _History:
    tokens: list = field(default_factory=list)  # prompt + generated (the engine's seq.TokenIDs)
    row: int = -1          # device row, -1 if none
    dev_len: int = -1      # the device row's length as last set (-1: unusable)
    used: int = 0          # step of last use (eviction)

    def put(self, p: int, t: int) -> None:
        """Token t at position p (a rewrite drops what follows p; a gap forgets the history)."""
        if p == len(self.tokens):
            self.tokens.append(int(t))
        elif p < len(self.tokens):
            del self.tokens[p:]
            self.tokens.append(int(t))
            self.dev_len = -1
        else:
            self.tokens = []
            self.dev_len = -1


class DeviceDrafter:
    def __init__(self, n: int, k: int, stride: int, rows: int, max_batch: int):
        self.n = max(n, 2)
        self.k = k if k >= 1 else 4
        self.stride = stride
        self.scratch_row = rows
        self.hist = torch.zeros(rows + 1, stride, dtype=torch.int32, device="cuda")
        self.hist_len = torch.full((rows + 1,), -1, dtype=torch.int32, device="cuda")
        self.max_batch = max_batch
        self.seqs: dict[int, _History] = {}
        self.free = list(range(rows))
        self.clock = 0
        self.next: dict[int, tuple[int, list]] = {}

    # -- prefill: the prompt tokens at their positions (chunked prefill included)
    def prefill(self, seq_ids, tokens_per_seq, positions_per_seq) -> None:
        for sid, toks, pos in zip(seq_ids, tokens_per_seq, positions_per_seq):
            h = self.seqs.setdefault(sid, _History())
            for t, p in zip(toks, pos):
                h.put(int(p), int(t))

    def _alloc_row(self, h: _History) -> bool:
        if not self.free:
            victims = [o for o in self.seqs.values() if o.row >= 0 and o.used < self.clock]
            if not victims:
                return False
            v = min(victims, key=lambda o: o.used)
            self.free.append(v.row)
            v.row, v.dev_len = -1, -1
        h.row = self.free.pop()
        h.dev_len = -1
        return True

    # -- before a decode step: current tokens into the histories; rows seeded where needed
    def prepare(self, seq_ids, current_tokens, current_positions) -> np.ndarray:
        self.clock += 1
        if self.clock % 256 == 0:
            for sid in [s for s, h in self.seqs.items() if self.clock - h.used > 256]:
                if self.seqs[sid].row >= 0:
                    self.free.append(self.seqs[sid].row)
                del self.seqs[sid]
                self.next.pop(sid, None)
        rows = np.full(len(seq_ids), self.scratch_row, np.int32)
        for b, sid in enumerate(seq_ids):
            h = self.seqs.setdefault(sid, _History())
            h.used = self.clock
            p = int(current_positions[b])
            if len(h.tokens) < p:  # never saw the start of this sequence
                h.tokens = []
            else:
                h.put(p, int(current_tokens[b]))
            if not h.tokens or len(h.tokens) > self.stride:
                continue
            if h.row < 0 and not self._alloc_row(h):
                continue
            rows[b] = h.row
            if h.dev_len != len(h.tokens):
                n = len(h.tokens)
                self.hist[h.row, :n] = torch.tensor(h.tokens, dtype=torch.int32)
                self.hist_len[h.row] = n
                h.dev_len = n
        return rows

    # -- after the acceptance, on the same stream: append + next drafts on the device
    def launch(self, rows: np.ndarray, drafts: torch.Tensor, accepted: torch.Tensor, token: torch.Tensor):
        return gv.history_append_draft(self.hist, self.hist_len, drafts, accepted, token, self.n, self.k,
                                       hist_rows=torch.from_numpy(rows).cuda())

    # -- after the stream synchronised: mirrors get the emitted tokens; drafts kept
    def finish(self, seq_ids, rows, drafts: np.ndarray, n_drafts, accepted, token, next_d, next_n) -> None:
        for b, sid in enumerate(seq_ids):
            h = self.seqs[sid]
            acc = min(max(int(accepted[b]), 0), int(n_drafts[b]))
            emitted = [int(x) for x in drafts[b, :acc]] + ([int(token[b])] if token[b] >= 0 else [])
            self.next.pop(sid, None)
            if not h.tokens:
                continue
            h.tokens.extend(emitted)
            if rows[b] == self.scratch_row:
                continue
            if h.dev_len + len(emitted) > self.stride:
                h.dev_len = -1
                continue
            h.dev_len += len(emitted)
            self.next[sid] = (len(h.tokens), [int(x) for x in next_d[b, :int(next_n[b])]])

    def drafts(self, seq_id: int, hist_len: int) -> Optional[list]:
        """DraftSource.Drafts: the device drafts if the engine's history has this length."""
        nd = self.next.get(seq_id)
        if nd is None or nd[0] != hist_len:
            return None
        return nd[1]
