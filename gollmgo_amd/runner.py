"""The runner's verify step over the device path: the Python twin of the Go runner
(internal/backend/rocm/runner.go, Runner.Step), statement for statement in what it calls and
in which order, so the sequence is executed and tested here.

A decode step (internal/backend/runner.go:84-93, Step):
  pack the engine's Batch (batch.pack_batch) and upload it;
  embed the B x R rows; plan the attention schedule once for the step;
  per layer: the model's QKV, the draft-KV append fused into the verify attention
  (gg_verify_append_attention_planned), the model's output projection / MLP;
  the LM head's logits [B][R][V];
  the acceptance on the device:
    greedy    : gg_accept_greedy_sample with the engine's SamplingParams — greedy Verify and,
                when every draft is accepted, the bonus drawn as Sampler.Sample draws it
                (temperature <= 1e-9: the argmax), with a uniform from the runner's seeded
                stream in place of the engine's rng.Float64();
    bonus_row : greedy Verify on the device; when every draft is accepted the bonus row's
                real logits go back to the engine, whose own Sampler (and random stream)
                draws the bonus, exactly as with the reference's runner;
    rejection : speculative sampling (gg_accept_rejection) at the engine's temperature /
                top-p, one-hot draft distributions (the n-gram drafter);
  optional device drafting (drafting.DeviceDrafter) right after the acceptance;
  copy back the decision and return it as LogitsPerPosition rows (positions.py).
The engine then runs its own emitSpeculative (internal/engine/serving.go:496-593) on those
rows, and truncates the rejected drafts' slots from its block tables.

The model is whatever the caller passes (embed / qkv / post / logits over the runner's
[B][R] row layout): the forward outside the verify path stays the model's.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Optional, Protocol

import numpy as np
import torch

from . import verify as gv
from ._lib import DType
from .batch import Batch, pack_batch
from .positions import LogitsPerPosition

ACCEPT_GREEDY = "greedy"
ACCEPT_BONUS_ROW = "bonus_row"
ACCEPT_REJECTION = "rejection"


@dataclass
class SamplingParams:
    """engine.SamplingParams (internal/engine/sampling.go:10-15): the same values the engine
    was configured with."""
    temperature: float = 0.0
    top_k: int = 0
    top_p: float = 0.0
    seed: Optional[int] = None


@dataclass
class RunnerConfig:
    num_blocks: int
    block_size: int
    kv_dtype: DType
    max_drafts: int
    sampling: SamplingParams = field(default_factory=SamplingParams)
    acceptance: str = ACCEPT_GREEDY


@dataclass
class StepOutput:
    """backend.StepOutput (internal/backend/runner.go:57-68)."""
    logits: list
    logits_per_position: list


class Model(Protocol):
    num_layers: int
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    vocab: int

    def embed(self, tokens: torch.Tensor) -> None: ...              # tokens [B][R] int32
    def qkv(self, layer: int, positions: torch.Tensor): ...         # -> q [B,R,Hq,D], k, v [B*R,Hkv,D]
    def post(self, layer: int, attn_out: torch.Tensor) -> None: ...  # attn_out [B,R,Hq,D]
    def logits(self) -> torch.Tensor: ...                            # [B,R,V] bf16


class VerifyRunner:
    def __init__(self, model: Model, cfg: RunnerConfig):
        if cfg.acceptance not in (ACCEPT_GREEDY, ACCEPT_BONUS_ROW, ACCEPT_REJECTION):
            raise ValueError(f"unknown acceptance {cfg.acceptance!r}")
        self.model, self.cfg = model, cfg
        scale_mode_dtype = DType(cfg.kv_dtype)
        self.kv = gv.KVCache(model.num_layers, cfg.num_blocks, cfg.block_size, model.num_kv_heads, model.head_dim,
                             scale_mode_dtype)
        self.rows = LogitsPerPosition(model.vocab)
        seed = cfg.sampling.seed if cfg.sampling.seed is not None else 0
        self.rng = np.random.default_rng(seed)
        self.max_batch = self.max_blocks = 0
        # kept for tests: the last step's device logits, uniforms and decision
        self.last_logits = self.last_uniforms = self.last_decision = None
        self.last_inputs = None

    def warmup(self, max_batch: int, max_seq_len: int) -> None:
        """Workspaces sized once (Runner.Warmup)."""
        B, R, V = max_batch, self.cfg.max_drafts + 1, self.model.vocab
        self.max_batch = max_batch
        self.max_blocks = (max_seq_len + self.cfg.block_size - 1) // self.cfg.block_size
        self.attn_ws = self.kv.attention_workspace(B, R, self.model.num_q_heads, self.max_blocks)
        if self.cfg.acceptance == ACCEPT_REJECTION:
            self.acc_ws = gv.rejection_workspace(B, R - 1, V)
        else:
            self.acc_ws = gv.sample_workspace(B, R - 1, V)

    def _uniforms(self, B: int, R: int):
        """The runner's stream in place of the engine's rng.Float64() (one value per
        sequence for the bonus draw; one per row for the rejection acceptance)."""
        if self.cfg.acceptance == ACCEPT_REJECTION:
            return torch.from_numpy(self.rng.random((B, R), dtype=np.float32)).cuda()
        return torch.from_numpy(self.rng.random(B)).cuda()

    def step(self, batch: Batch) -> StepOutput:
        if any(batch.is_prefill):
            raise ValueError("prefill batches go to the model's own path")
        if len(batch.sequence_ids) > self.max_batch:
            raise ValueError("batch exceeds the warmed-up size")
        cfg, m = self.cfg, self.model
        inp = pack_batch(batch, cfg.block_size, self.max_blocks, cfg.max_drafts + 1)
        B, R, MB, K = inp.num_seqs, inp.rows_per_seq, inp.max_blocks, inp.rows_per_seq - 1
        dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
        tokens, positions = dev(inp.tokens), dev(inp.positions)
        ctx, rows, tables = dev(inp.ctx_lens), dev(inp.row_counts), dev(inp.block_tables)
        drafts, n_drafts = dev(inp.drafts.reshape(B, K)), dev(inp.n_drafts)
        uniforms = self._uniforms(B, R)
        scale = 1.0 / math.sqrt(m.head_dim)  # as gollmgo_model.cu
        m.embed(tokens)
        self.kv.attention_plan(ctx, R, m.num_q_heads, MB, self.attn_ws, row_counts=rows)
        for layer in range(m.num_layers):
            q, k, v = m.qkv(layer, positions)
            out = torch.empty_like(q)
            self.kv.append_attention(layer, k, v, q, out, ctx, tables, scale, self.attn_ws, row_counts=rows)
            m.post(layer, out)
        logits = m.logits()
        sp = cfg.sampling
        if cfg.acceptance == ACCEPT_REJECTION:
            acc, tok = gv.accept_rejection(logits, drafts, n_drafts, uniforms, sp.temperature, sp.top_p,
                                           workspace=self.acc_ws)
        elif cfg.acceptance == ACCEPT_BONUS_ROW:
            acc, tok = gv.accept_greedy(logits, drafts, n_drafts, workspace=self.acc_ws)
        else:
            acc, tok = gv.accept_greedy_sample(logits, drafts, n_drafts, uniforms, sp.temperature, sp.top_k,
                                               sp.top_p, workspace=self.acc_ws)
        h_acc, h_tok = acc.cpu().numpy(), tok.cpu().numpy()  # the one synchronising copy
        self.last_logits, self.last_uniforms = logits, uniforms.cpu().numpy()
        self.last_decision, self.last_inputs = (h_acc, h_tok), inp
        out = StepOutput([None] * B, [None] * B)
        for i in range(B):
            n = int(inp.n_drafts[i])
            r = self.rows.rows_for(inp.drafts[i], n, int(h_acc[i]), int(h_tok[i]))
            if cfg.acceptance == ACCEPT_BONUS_ROW and h_acc[i] == n:
                r[-1] = logits[i, n].float().cpu().numpy()  # the engine's Sampler draws the bonus
            out.logits[i] = r[0]
            if n > 0:
                out.logits_per_position[i] = r
        return out

    def close(self) -> None:
        self.kv.close()
