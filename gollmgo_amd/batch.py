"""The engine's `backend.Batch` packed into the verify ABI's arrays.

`Batch` (internal/backend/runner.go:29-54) is flattened per token: sequence i contributes
SeqTokenCounts[i] consecutive entries of TokenIDs / Positions / SlotMapping (the current
token, then its drafts), and carries its whole slot table and its draft list. The ABI
wants rectangular per-sequence arrays: rows_per_seq R = the batch's largest token count,
ctx_lens, row_counts, block tables of physical block ids, drafts [B][R-1] and n_drafts.
`pack_batch` is that mapping; the Go runner's PackBatch
(internal/backend/rocm/batch.go) is the same function line for line, and
tests/test_runner_batch.py holds the cases both follow.

Block ids come from the slot table: the KV manager hands out whole blocks and fills them
in order (internal/kvcache/block_table.go:24-42), so block b of a sequence is
SeqSlotTables[i][b * bs] / bs, and every slot of that block is block * bs + offset.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import numpy as np


@dataclass
class Batch:
    """backend.Batch (internal/backend/runner.go:29-54)."""
    sequence_ids: list[int]
    token_ids: list[int]
    positions: list[int]
    slot_mapping: list[int]
    is_prefill: list[bool]
    seq_token_counts: list[int]
    seq_context_lens: list[int]
    seq_slot_tables: list[list[int]]
    draft_tokens: Optional[list[list[int]]] = None


@dataclass
class StepInputs:
    """The ABI's view of one verify step (host arrays, int32)."""
    num_seqs: int
    rows_per_seq: int
    max_blocks: int
    tokens: np.ndarray        # [B][R], padding rows 0
    positions: np.ndarray     # [B][R], padding rows repeat the last position
    slots: np.ndarray         # [B * R] for gg_kv_append, padding rows -1 (skipped)
    ctx_lens: np.ndarray      # [B]
    row_counts: np.ndarray    # [B]
    block_tables: np.ndarray  # [B][max_blocks], padding -1
    drafts: np.ndarray        # [B][R - 1], padding 0
    n_drafts: np.ndarray      # [B]


class BatchError(ValueError):
    pass


def pack_batch(batch: Batch, block_size: int, max_blocks: int = 0, rows_per_seq: int = 0) -> StepInputs:
    """Pack a decode batch (no prefill sequences). max_blocks / rows_per_seq: the
    workspace shape fixed at warm-up (0 = the batch's own)."""
    B = len(batch.sequence_ids)
    if B == 0:
        raise BatchError("empty batch")
    if any(batch.is_prefill):
        raise BatchError("prefill sequences go to the model's prefill path")
    counts = [int(c) for c in batch.seq_token_counts]
    if len(counts) != B or len(batch.seq_context_lens) != B or len(batch.seq_slot_tables) != B:
        raise BatchError("per-sequence fields disagree with SequenceIDs")
    n_tok = sum(counts)
    if len(batch.token_ids) != n_tok or len(batch.positions) != n_tok or len(batch.slot_mapping) != n_tok:
        raise BatchError("flattened token fields disagree with SeqTokenCounts")
    if min(counts) < 1:
        raise BatchError("a decode sequence has at least its current token")
    R = max(counts)
    if rows_per_seq:
        if R > rows_per_seq:
            raise BatchError(f"{R} rows exceed the warmed-up {rows_per_seq}")
        R = rows_per_seq
    K = R - 1
    drafts_in = batch.draft_tokens if batch.draft_tokens else [[] for _ in range(B)]
    if len(drafts_in) != B:
        raise BatchError("DraftTokens disagrees with SequenceIDs")
    need_blocks = max((int(c) + block_size - 1) // block_size for c in batch.seq_context_lens)
    MB = max_blocks or max(need_blocks, 1)
    if need_blocks > MB:
        raise BatchError(f"{need_blocks} blocks exceed the warmed-up {MB}")

    tokens = np.zeros((B, R), np.int32)
    positions = np.zeros((B, R), np.int32)
    slots = np.full(B * R, -1, np.int32)
    ctx = np.zeros(B, np.int32)
    rows = np.zeros(B, np.int32)
    tables = np.full((B, MB), -1, np.int32)
    drafts = np.zeros((B, max(K, 0)), np.int32)
    nd = np.zeros(B, np.int32)
    t0 = 0
    for i in range(B):
        c = counts[i]
        d = list(drafts_in[i])
        if len(d) != c - 1:
            raise BatchError(f"sequence {i}: {c} tokens but {len(d)} drafts")
        tok = batch.token_ids[t0:t0 + c]
        if list(tok[1:]) != d:
            raise BatchError(f"sequence {i}: the tokens after the current one are not its drafts")
        tokens[i, :c] = tok
        positions[i, :c] = batch.positions[t0:t0 + c]
        positions[i, c:] = batch.positions[t0 + c - 1]
        slots[i * R:i * R + c] = batch.slot_mapping[t0:t0 + c]
        t0 += c
        L = int(batch.seq_context_lens[i])
        st = batch.seq_slot_tables[i]
        if L < c or len(st) != L:
            raise BatchError(f"sequence {i}: context {L} with a slot table of {len(st)} and {c} rows")
        for b in range((L + block_size - 1) // block_size):
            s0 = int(st[b * block_size])
            if s0 < 0 or s0 % block_size:
                raise BatchError(f"sequence {i}: block {b} starts at slot {s0}, not a block boundary")
            tables[i, b] = s0 // block_size
        for j in range(c):
            if int(st[L - c + j]) != int(slots[i * R + j]):
                raise BatchError(f"sequence {i}: SlotMapping of row {j} is not its slot-table entry")
        ctx[i] = L
        rows[i] = c
        drafts[i, :c - 1] = d
        nd[i] = c - 1
    check_block_runs(slots, block_size)
    return StepInputs(B, R, MB, tokens, positions, slots, ctx, rows, tables, drafts, nd)


def check_block_runs(slots: np.ndarray, block_size: int) -> None:
    """gg_kv_append's rule for PER_BLOCK pools: the rows of one block are adjacent in the
    slot mapping (skipped rows, slot < 0, may sit between them) with increasing offsets. A
    block that reappears after another block's rows would get two leaders on the device."""
    seen: set = set()
    cur, last_off = -1, -1
    for s in np.asarray(slots).tolist():
        if s < 0:
            continue
        blk, off = divmod(int(s), block_size)
        if blk != cur:
            if blk in seen:
                raise BatchError(f"block {blk} appears in two separate runs of the slot mapping")
            seen.add(blk)
            cur, last_off = blk, -1
        if off <= last_off:
            raise BatchError(f"block {blk}: offsets not increasing in the slot mapping")
        last_off = off
