"""Verify-step workloads: the five configurations this path is measured on, and
builders for their synthetic inputs (block tables, slot mappings, histories).

Inputs are synthetic, seeded and shaped like each configuration; nothing is
downloaded. Block layouts come from the host block manager mirror (blocks.py) so
they look like what the engine produces: per-sequence block tables over a
shuffled physical pool, appends landing in fresh or partially filled blocks, and
(config 3) prefix blocks shared by pairs of sequences with refcount 2.
"""
from __future__ import annotations

from dataclasses import dataclass, field, replace

import numpy as np

from .blocks import BlockPool, BlockTable


@dataclass(frozen=True)
class VerifyConfig:
    name: str
    num_seqs: int
    max_drafts: int            # K; query rows per sequence R = K + 1
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    ctx: tuple                 # ("uniform", lo, hi) or ("list", c0, c1, ...): cached tokens before the step
    kv_dtype: str              # f32 | f16 | bf16 | fp8 | int8
    q_dtype: str               # f32 | f16 | bf16
    vocab: int
    logits_dtype: str          # f32 | bf16 | f16
    accept: str                # greedy | rejection
    temperature: float = 0.0
    top_p: float = 1.0
    draft_probs: bool = False
    shared_prefix_frac: float = 0.0
    partition: int = 0         # split-K partition tokens (0 = library default)
    layers: int = 1            # L in verified tokens/s = B*R / (L*(t_append+t_attn) + t_accept)
    pool_blocks: int = 0       # 0 = just enough (+ slack)
    history_len: int = 0       # n-gram history per sequence (config 5)
    ngram_n: int = 3
    repeat_rate: float = 0.0
    seed: int = 0

    @property
    def rows(self) -> int:
        return self.max_drafts + 1


CONFIGS: dict[int, VerifyConfig] = {
    1: VerifyConfig("tiny-fp32", 4, 4, 8, 2, 64, 16, ("list", 64, 128, 192, 256), "f32", "f32", 32000,
                    "f32", "greedy", layers=1, history_len=256, repeat_rate=0.3, seed=20261202),
    2: VerifyConfig("llama3.2-3b-bf16", 32, 4, 24, 8, 128, 16, ("uniform", 512, 4096), "bf16", "bf16",
                    128256, "bf16", "greedy", layers=28, pool_blocks=65536, seed=20261203),
    3: VerifyConfig("llama3.1-8b-fp8", 64, 5, 32, 8, 128, 16, ("uniform", 1024, 8192), "fp8", "bf16",
                    128256, "f32", "rejection", temperature=0.8, draft_probs=True,
                    shared_prefix_frac=0.2, layers=32, seed=20261204),
    4: VerifyConfig("long-int8", 8, 8, 32, 8, 128, 16, ("uniform", 16384, 32768), "int8", "bf16", 128256,
                    "bf16", "greedy", partition=512, layers=32, seed=20261205),
    5: VerifyConfig("mix-bf16", 128, 5, 32, 8, 128, 16, ("uniform", 256, 2048), "bf16", "bf16", 128256,
                    "f32", "rejection", temperature=0.8, top_p=0.95, layers=32, history_len=8192,
                    repeat_rate=0.4, seed=20261206),
}


@dataclass
class Layout:
    """Host-side block layout of one verify step."""
    ctx_before: np.ndarray     # [B] cached tokens before the step
    keys: np.ndarray           # [B] ctx_before + rows (SeqContextLens)
    block_tables: np.ndarray   # [B, max_blocks] int32 (padded with 0)
    append_slots: np.ndarray   # [B*R] slots of the verify rows
    fill_slots: np.ndarray     # [n_fill] slots of context tokens to write at set-up
    fill_rows: np.ndarray      # [n_fill] (seq, position) of each fill slot, for data generation
    num_blocks: int
    refcounts: np.ndarray = field(default=None)


def context_lengths(cfg: VerifyConfig, rng: np.random.Generator) -> np.ndarray:
    kind = cfg.ctx[0]
    if kind == "list":
        vals = np.array(cfg.ctx[1:], dtype=np.int64)
        assert len(vals) == cfg.num_seqs
        return vals
    lo, hi = cfg.ctx[1], cfg.ctx[2]
    return rng.integers(lo, hi + 1, size=cfg.num_seqs).astype(np.int64)


def build_layout(cfg: VerifyConfig, seed: int | None = None) -> Layout:
    rng = np.random.default_rng(cfg.seed if seed is None else seed)
    B, R, bs = cfg.num_seqs, cfg.rows, cfg.block_size
    ctx = context_lengths(cfg, rng)
    keys = ctx + R
    need = int(np.sum((keys + bs - 1) // bs))
    total = max(cfg.pool_blocks, need + B + 16)
    order = rng.permutation(total).tolist()  # physical blocks handed out in random order
    pool = BlockPool(total, bs, order=order)
    tables = [BlockTable(pool) for _ in range(B)]
    fill_slots: list[int] = []
    fill_rows: list[tuple[int, int]] = []
    # Prefix sharing: sequences (2i, 2i+1) share their first floor(frac * blocks) full blocks.
    shared: dict[int, list[int]] = {}
    if cfg.shared_prefix_frac > 0:
        for i in range(0, B - 1, 2):
            nb = int(cfg.shared_prefix_frac * min(ctx[i], ctx[i + 1]) // bs)
            if nb > 0:
                shared[i] = nb
    for b in range(B):
        t = tables[b]
        start = 0
        if b % 2 == 1 and (b - 1) in shared:
            nb = shared[b - 1]
            t.attach_shared(tables[b - 1].blocks[:nb])
            start = nb * bs
        for p in range(start, int(ctx[b])):
            fill_slots.append(t.append())
            fill_rows.append((b, p))
    append_slots = []
    for b in range(B):
        append_slots.extend(tables[b].append_n(R))
    max_blocks = max(len(t.blocks) for t in tables)
    bt = np.zeros((B, max_blocks), dtype=np.int32)
    for b, t in enumerate(tables):
        bt[b, :len(t.blocks)] = t.blocks
    return Layout(ctx_before=ctx.astype(np.int32), keys=keys.astype(np.int32), block_tables=bt,
                  append_slots=np.asarray(append_slots, dtype=np.int32),
                  fill_slots=np.asarray(fill_slots, dtype=np.int32),
                  fill_rows=np.asarray(fill_rows, dtype=np.int32).reshape(-1, 2),
                  num_blocks=total, refcounts=np.asarray(pool.refcounts, dtype=np.int32))


def make_histories(cfg: VerifyConfig, length: int, seed: int | None = None) -> np.ndarray:
    """Token histories with injected repeated 3-grams (rate = cfg.repeat_rate): with that
    probability a position copies a 3-gram seen earlier, so the drafter finds matches."""
    rng = np.random.default_rng((cfg.seed if seed is None else seed) + 7)
    B = cfg.num_seqs
    h = rng.integers(0, cfg.vocab, size=(B, length), dtype=np.int64)
    for b in range(B):
        p = 3
        while p + 3 <= length:
            if rng.random() < cfg.repeat_rate:
                src = int(rng.integers(0, p - 2))
                h[b, p:p + 3] = h[b, src:src + 3]
                p += 3
            else:
                p += 1
    return h.astype(np.int32)


def scaled(cfg: VerifyConfig, **kw) -> VerifyConfig:
    """A copy of cfg with some fields replaced (used for parity tests at oracle-friendly sizes)."""
    return replace(cfg, **kw)
