"""Host-side mirror of the verify path over torch device tensors.

Thin plumbing around the C ABI (include/gg_verify.h): torch provides device
memory and the current HIP stream; every computation runs in the HIP kernels
of libgg_verify.so. Names follow the reference's domain:

  KVCache            ~ CUDAKVCache (internal/backend/cuda/kvcache_bridge.go:16-91)
  KVCache.append     ~ CUDAKVCache.Write / gollmgo_kvcache_write
  KVCache.attention  ~ gollmgo_kvcache_attention, for k+1 verify rows per sequence
  accept_greedy      ~ Verify + argmax as emitSpeculative drives them
                       (internal/engine/speculative.go:68-84, serving.go:514-566)
  accept_greedy_sample ~ the same with the bonus token drawn by Sampler.Sample
                       (internal/engine/sampling.go:40-72) at the engine's temperature/top-k/top-p
  accept_rejection   ~ speculative sampling with Sampler's temperature/top-p rules
  ngram_draft        ~ NGramDrafter.Draft (internal/engine/speculative.go:24-62)
"""
from __future__ import annotations

import ctypes as C
from typing import Optional

import torch

from ._lib import DType, ScaleMode, check, lib

_TORCH_TO_DT = {torch.float32: DType.F32, torch.float16: DType.F16, torch.bfloat16: DType.BF16}


def dtype_of(t: torch.Tensor) -> DType:
    try:
        return _TORCH_TO_DT[t.dtype]
    except KeyError as e:
        raise TypeError(f"unsupported tensor dtype {t.dtype}") from e


def _stream(stream: Optional[torch.cuda.Stream]) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def _dev(t: torch.Tensor, name: str, dtype=None) -> int:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    return t.data_ptr()


class _DeviceBuffer:
    """Exposes raw device memory to torch through __cuda_array_interface__."""

    def __init__(self, ptr: int, nbytes: int):
        self.__cuda_array_interface__ = {
            "shape": (nbytes,), "typestr": "|u1", "data": (ptr, False), "version": 3, "strides": None,
        }


_ELEM_BYTES = {DType.F32: 4, DType.F16: 2, DType.BF16: 2, DType.FP8_E4M3: 1, DType.INT8: 1}


def device_bytes(ptr: int, nbytes: int) -> torch.Tensor:
    """A uint8 torch view of `nbytes` of device memory at `ptr` (no copy)."""
    return torch.as_tensor(_DeviceBuffer(ptr, nbytes), device="cuda")


class KVCache:
    """Paged K/V pools for all layers (K[blk][Hkv][bs][D], V[blk][Hkv][D][bs]; in device
    memory the K and V tiles of each (block, head) are adjacent)."""

    def __init__(self, num_layers: int, num_blocks: int, block_size: int, num_kv_heads: int,
                 head_dim: int, dtype: DType):
        self.num_layers, self.num_blocks, self.block_size = num_layers, num_blocks, block_size
        self.num_kv_heads, self.head_dim, self.dtype = num_kv_heads, head_dim, DType(dtype)
        self.scale_mode = {DType.FP8_E4M3: ScaleMode.PER_HEAD, DType.INT8: ScaleMode.PER_BLOCK}.get(
            self.dtype, ScaleMode.NONE)
        torch.cuda.init()
        h = C.c_void_p()
        check(lib().gg_kv_create(num_layers, num_blocks, block_size, num_kv_heads, head_dim,
                                 int(self.dtype), int(self.scale_mode), C.byref(h)), "gg_kv_create")
        self.handle = h

    def close(self) -> None:
        if getattr(self, "handle", None):
            torch.cuda.synchronize()
            check(lib().gg_kv_destroy(self.handle), "gg_kv_destroy")
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def layer_bytes(self) -> int:
        return lib().gg_kv_layer_bytes(self.handle)

    def _pool(self, ptr: int) -> torch.Tensor:
        # The K and V tiles of each (block, head) alternate in device memory; gather one
        # pool's tiles into its logical [blocks][heads][tile] bytes (a device copy).
        tile = self.block_size * self.head_dim * _ELEM_BYTES[self.dtype]
        n = self.num_blocks * self.num_kv_heads
        raw = device_bytes(ptr, (2 * n - 1) * tile)
        return torch.as_strided(raw, (n, tile), (2 * tile, 1)).reshape(-1)

    def k_pool(self, layer: int) -> torch.Tensor:
        """Layer's K pool, K[blk][Hkv][bs][D], as uint8 bytes (a copy)."""
        return self._pool(lib().gg_kv_k_layer_ptr(self.handle, layer))

    def v_pool(self, layer: int) -> torch.Tensor:
        """Layer's V pool, V[blk][Hkv][D][bs], as uint8 bytes (a copy)."""
        return self._pool(lib().gg_kv_v_layer_ptr(self.handle, layer))

    def scales(self, layer: int) -> tuple[torch.Tensor, torch.Tensor]:
        """(k, v) scales: PER_HEAD fp32 [Hkv]; PER_BLOCK fp16 [blocks, Hkv]."""
        if self.scale_mode == ScaleMode.PER_HEAD:
            n, dt = self.num_kv_heads * 4, torch.float32
        elif self.scale_mode == ScaleMode.PER_BLOCK:
            n, dt = self.num_blocks * self.num_kv_heads * 2, torch.float16
        else:
            raise ValueError("pool has no scales")
        k = device_bytes(lib().gg_kv_k_scale_ptr(self.handle, layer), n).view(dt)
        v = device_bytes(lib().gg_kv_v_scale_ptr(self.handle, layer), n).view(dt)
        if self.scale_mode == ScaleMode.PER_BLOCK:
            k, v = k.view(self.num_blocks, self.num_kv_heads), v.view(self.num_blocks, self.num_kv_heads)
        return k, v

    def set_head_scales(self, layer: int, k_scales, v_scales) -> None:
        ks = (C.c_float * self.num_kv_heads)(*[float(x) for x in k_scales])
        vs = (C.c_float * self.num_kv_heads)(*[float(x) for x in v_scales])
        check(lib().gg_kv_set_head_scales(self.handle, layer, ks, vs), "gg_kv_set_head_scales")

    def append(self, layer: int, k: torch.Tensor, v: torch.Tensor, slot_mapping: torch.Tensor,
               stream: Optional[torch.cuda.Stream] = None) -> None:
        n = int(slot_mapping.numel())
        if k.shape != v.shape or k.numel() != n * self.num_kv_heads * self.head_dim:
            raise ValueError("k/v must be [n_rows, num_kv_heads, head_dim] matching slot_mapping")
        check(lib().gg_kv_append(self.handle, layer, _dev(k, "k"), _dev(v, "v", k.dtype), int(dtype_of(k)),
                                 _dev(slot_mapping, "slot_mapping", torch.int32), n, _stream(stream)),
              "gg_kv_append")

    def snapshot_bytes(self, num_blocks: int) -> int:
        return lib().gg_kv_snapshot_bytes(self.handle, num_blocks)

    def snapshot(self, block_ids: torch.Tensor, host: Optional[torch.Tensor] = None,
                 staging: Optional[torch.Tensor] = None, stream: Optional[torch.cuda.Stream] = None):
        """Snapshot of the given blocks over every layer (gg_kv_snapshot): returns
        (staging, host); `host` (uint8, ideally pinned) receives a copy when given."""
        n = int(block_ids.numel())
        nbytes = self.snapshot_bytes(n)
        if staging is None:
            staging = torch.empty(max(nbytes, 16), dtype=torch.uint8, device="cuda")
        if host is not None and host.numel() < nbytes:
            raise ValueError("host buffer too small")
        check(lib().gg_kv_snapshot(self.handle, _dev(block_ids, "block_ids", torch.int32), n, staging.data_ptr(),
                                   staging.numel(), host.data_ptr() if host is not None else None,
                                   _stream(stream)), "gg_kv_snapshot")
        return staging, host

    def restore(self, block_ids: torch.Tensor, staging: torch.Tensor, host: Optional[torch.Tensor] = None,
                stream: Optional[torch.cuda.Stream] = None) -> None:
        """Writes a snapshot back into blocks `block_ids` (gg_kv_restore), from `host` when
        given (through `staging`), else from `staging`."""
        n = int(block_ids.numel())
        check(lib().gg_kv_restore(self.handle, _dev(block_ids, "block_ids", torch.int32), n, staging.data_ptr(),
                                  staging.numel(), host.data_ptr() if host is not None else None,
                                  _stream(stream)), "gg_kv_restore")

    def attention_workspace(self, num_seqs: int, rows_per_seq: int, num_q_heads: int,
                            max_blocks_per_seq: int, partition_tokens: int = 0) -> torch.Tensor:
        n = lib().gg_verify_attention_workspace_size(self.handle, num_seqs, rows_per_seq, num_q_heads,
                                                     max_blocks_per_seq, partition_tokens)
        return torch.empty(max(n, 16), dtype=torch.uint8, device="cuda")

    def attention(self, layer: int, q: torch.Tensor, out: torch.Tensor, ctx_lens: torch.Tensor,
                  block_tables: torch.Tensor, scale: float, row_counts: Optional[torch.Tensor] = None,
                  partition_tokens: int = 0, workspace: Optional[torch.Tensor] = None,
                  stream: Optional[torch.cuda.Stream] = None, planned: bool = False) -> torch.Tensor:
        """q, out: [num_seqs, rows_per_seq, num_q_heads, head_dim]. planned=True uses the
        schedule attention_plan put in `workspace` (required then)."""
        if q.dim() != 4 or q.shape[-1] != self.head_dim or out.shape != q.shape:
            raise ValueError("q/out must be [num_seqs, rows_per_seq, num_q_heads, head_dim]")
        B, R, Hq, _ = q.shape
        if block_tables.dim() != 2 or block_tables.shape[0] != B:
            raise ValueError("block_tables must be [num_seqs, max_blocks_per_seq]")
        mb = block_tables.shape[1]
        if workspace is None:
            if planned:
                raise ValueError("a planned call needs the workspace that holds the plan")
            workspace = self.attention_workspace(B, R, Hq, mb, partition_tokens)
        rc = _dev(row_counts, "row_counts", torch.int32) if row_counts is not None else None
        if planned:
            if partition_tokens:
                raise ValueError("a planned call uses the automatic schedule (partition_tokens = 0)")
            check(lib().gg_verify_attention_planned(
                self.handle, layer, _dev(q, "q"), int(dtype_of(q)), _dev(out, "out"), int(dtype_of(out)),
                _dev(ctx_lens, "ctx_lens", torch.int32), rc, _dev(block_tables, "block_tables", torch.int32),
                mb, B, R, Hq, float(scale), workspace.data_ptr(), workspace.numel(), _stream(stream)),
                "gg_verify_attention_planned")
            return out
        check(lib().gg_verify_attention(
            self.handle, layer, _dev(q, "q"), int(dtype_of(q)), _dev(out, "out"), int(dtype_of(out)),
            _dev(ctx_lens, "ctx_lens", torch.int32), rc, _dev(block_tables, "block_tables", torch.int32),
            mb, B, R, Hq, float(scale), partition_tokens, workspace.data_ptr(), workspace.numel(),
            _stream(stream)), "gg_verify_attention")
        return out

    def append_attention(self, layer: int, k_new: torch.Tensor, v_new: torch.Tensor, q: torch.Tensor,
                         out: torch.Tensor, ctx_lens: torch.Tensor, block_tables: torch.Tensor, scale: float,
                         workspace: torch.Tensor, row_counts: Optional[torch.Tensor] = None,
                         stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
        """Draft-KV append of the verify rows and planned attention in one call
        (gg_verify_append_attention_planned). k_new, v_new: [num_seqs * rows_per_seq,
        Hkv, head_dim]; row b*R + j goes to key position ctx_lens[b] - row_count + j.
        `workspace` must hold the step's plan (attention_plan)."""
        if q.dim() != 4 or q.shape[-1] != self.head_dim or out.shape != q.shape:
            raise ValueError("q/out must be [num_seqs, rows_per_seq, num_q_heads, head_dim]")
        B, R, Hq, _ = q.shape
        if k_new.shape != (B * R, self.num_kv_heads, self.head_dim) or v_new.shape != k_new.shape:
            raise ValueError("k_new/v_new must be [num_seqs * rows_per_seq, num_kv_heads, head_dim]")
        if block_tables.dim() != 2 or block_tables.shape[0] != B:
            raise ValueError("block_tables must be [num_seqs, max_blocks_per_seq]")
        if k_new.dtype != v_new.dtype:
            raise ValueError("k_new and v_new must share a dtype")
        rc = _dev(row_counts, "row_counts", torch.int32) if row_counts is not None else None
        check(lib().gg_verify_append_attention_planned(
            self.handle, layer, _dev(k_new, "k_new"), _dev(v_new, "v_new"), int(dtype_of(k_new)),
            _dev(q, "q"), int(dtype_of(q)), _dev(out, "out"), int(dtype_of(out)),
            _dev(ctx_lens, "ctx_lens", torch.int32), rc, _dev(block_tables, "block_tables", torch.int32),
            block_tables.shape[1], B, R, Hq, float(scale), workspace.data_ptr(), workspace.numel(),
            _stream(stream)), "gg_verify_append_attention_planned")
        return out

    def attention_plan(self, ctx_lens: torch.Tensor, rows_per_seq: int, num_q_heads: int,
                       max_blocks_per_seq: int, workspace: torch.Tensor, row_counts: Optional[torch.Tensor] = None,
                       stream: Optional[torch.cuda.Stream] = None) -> None:
        """Schedule of one verify step into `workspace`, for attention(..., planned=True) on
        every layer while ctx_lens / row_counts keep their contents."""
        rc = _dev(row_counts, "row_counts", torch.int32) if row_counts is not None else None
        check(lib().gg_verify_attention_plan(
            self.handle, _dev(ctx_lens, "ctx_lens", torch.int32), rc, max_blocks_per_seq, ctx_lens.numel(),
            rows_per_seq, num_q_heads, workspace.data_ptr(), workspace.numel(), _stream(stream)),
            "gg_verify_attention_plan")


def greedy_workspace(num_seqs: int, max_drafts: int, vocab: int) -> torch.Tensor:
    n = lib().gg_accept_greedy_workspace_size(num_seqs, max_drafts, vocab)
    return torch.empty(max(n, 16), dtype=torch.uint8, device="cuda")


def sample_workspace(num_seqs: int, max_drafts: int, vocab: int) -> torch.Tensor:
    n = lib().gg_accept_greedy_sample_workspace_size(num_seqs, max_drafts, vocab)
    return torch.empty(max(n, 16), dtype=torch.uint8, device="cuda")


def rejection_workspace(num_seqs: int, max_drafts: int, vocab: int) -> torch.Tensor:
    n = lib().gg_accept_rejection_workspace_size(num_seqs, max_drafts, vocab)
    return torch.empty(max(n, 16), dtype=torch.uint8, device="cuda")


def accept_greedy(logits: torch.Tensor, drafts: torch.Tensor, n_drafts: torch.Tensor,
                  workspace: Optional[torch.Tensor] = None, out: Optional[tuple] = None,
                  stream: Optional[torch.cuda.Stream] = None):
    """logits [B, K+1, V]; drafts [B, K] int32; n_drafts [B] int32 -> (accepted [B], token [B])."""
    B, R, V = logits.shape
    K = R - 1
    if drafts.shape != (B, K) and not (K == 0 and drafts.numel() == 0):
        raise ValueError("drafts must be [num_seqs, max_drafts]")
    if workspace is None:
        workspace = greedy_workspace(B, K, V)
    acc, tok = out if out is not None else (torch.empty(B, dtype=torch.int32, device="cuda"),
                                            torch.empty(B, dtype=torch.int32, device="cuda"))
    check(lib().gg_accept_greedy(
        _dev(logits, "logits"), int(dtype_of(logits)), B, K, V,
        drafts.data_ptr() if drafts.numel() else None, _dev(n_drafts, "n_drafts", torch.int32),
        _dev(acc, "accepted", torch.int32), _dev(tok, "token", torch.int32), workspace.data_ptr(),
        workspace.numel(), _stream(stream)), "gg_accept_greedy")
    return acc, tok


SAMPLE_EXACT = 1  # GG_SAMPLE_EXACT: every draw through the sequential path


def accept_greedy_sample(logits: torch.Tensor, drafts: torch.Tensor, n_drafts: torch.Tensor,
                         uniforms: torch.Tensor, temperature: float, top_k: int = 0, top_p: float = 0.0,
                         flags: int = 0, workspace: Optional[torch.Tensor] = None, out: Optional[tuple] = None,
                         stream: Optional[torch.cuda.Stream] = None):
    """Greedy Verify; when every draft is accepted the bonus is Sampler.Sample(row n) with
    (temperature, top_k, top_p) and uniforms[b] (float64) in place of rng.Float64().
    logits [B, K+1, V]; drafts [B, K] int32; n_drafts [B] int32 -> (accepted [B], token [B])."""
    B, R, V = logits.shape
    K = R - 1
    if drafts.shape != (B, K) and not (K == 0 and drafts.numel() == 0):
        raise ValueError("drafts must be [num_seqs, max_drafts]")
    if uniforms.shape != (B,):
        raise ValueError("uniforms must be [num_seqs]")
    if workspace is None:
        workspace = sample_workspace(B, K, V)
    acc, tok = out if out is not None else (torch.empty(B, dtype=torch.int32, device="cuda"),
                                            torch.empty(B, dtype=torch.int32, device="cuda"))
    check(lib().gg_accept_greedy_sample(
        _dev(logits, "logits"), int(dtype_of(logits)), B, K, V,
        drafts.data_ptr() if drafts.numel() else None, _dev(n_drafts, "n_drafts", torch.int32),
        float(temperature), int(top_k), float(top_p), _dev(uniforms, "uniforms", torch.float64), int(flags),
        _dev(acc, "accepted", torch.int32), _dev(tok, "token", torch.int32), workspace.data_ptr(),
        workspace.numel(), _stream(stream)), "gg_accept_greedy_sample")
    return acc, tok


def accept_rejection(target_logits: torch.Tensor, drafts: torch.Tensor, n_drafts: torch.Tensor,
                     uniforms: torch.Tensor, temperature: float, top_p: float = 1.0,
                     draft_probs: Optional[torch.Tensor] = None, workspace: Optional[torch.Tensor] = None,
                     out: Optional[tuple] = None, stream: Optional[torch.cuda.Stream] = None):
    """target_logits [B, K+1, V]; draft_probs [B, K, V] fp32 or None (one-hot drafter);
    uniforms [B, K+1] fp32 -> (accepted [B], token [B])."""
    B, R, V = target_logits.shape
    K = R - 1
    if uniforms.shape != (B, R):
        raise ValueError("uniforms must be [num_seqs, max_drafts + 1]")
    if draft_probs is not None and draft_probs.shape != (B, K, V):
        raise ValueError("draft_probs must be [num_seqs, max_drafts, vocab]")
    if workspace is None:
        workspace = rejection_workspace(B, K, V)
    acc, tok = out if out is not None else (torch.empty(B, dtype=torch.int32, device="cuda"),
                                            torch.empty(B, dtype=torch.int32, device="cuda"))
    dp = _dev(draft_probs, "draft_probs", torch.float32) if draft_probs is not None else None
    check(lib().gg_accept_rejection(
        _dev(target_logits, "target_logits"), int(dtype_of(target_logits)), dp, B, K, V,
        drafts.data_ptr() if drafts.numel() else None, _dev(n_drafts, "n_drafts", torch.int32),
        _dev(uniforms, "uniforms", torch.float32), float(temperature), float(top_p),
        _dev(acc, "accepted", torch.int32), _dev(tok, "token", torch.int32), workspace.data_ptr(),
        workspace.numel(), _stream(stream)), "gg_accept_rejection")
    return acc, tok


def ngram_draft(history: torch.Tensor, hist_len: torch.Tensor, n: int, max_drafts: int,
                out: Optional[tuple] = None, stream: Optional[torch.cuda.Stream] = None):
    """history [B, stride] int32, hist_len [B] int32 -> (drafts [B, K'], n_out [B]),
    K' = max_drafts after NewNGramDrafter's normalisation (< 1 -> 4)."""
    B, stride = history.shape
    K = max_drafts if max_drafts >= 1 else 4
    d, nn = out if out is not None else (torch.zeros(B, K, dtype=torch.int32, device="cuda"),
                                         torch.empty(B, dtype=torch.int32, device="cuda"))
    check(lib().gg_ngram_draft(_dev(history, "history", torch.int32), stride,
                               _dev(hist_len, "hist_len", torch.int32), B, n, max_drafts,
                               _dev(d, "drafts", torch.int32), _dev(nn, "n_out", torch.int32),
                               _stream(stream)), "gg_ngram_draft")
    return d, nn


def history_append_draft(history: torch.Tensor, hist_len: torch.Tensor, drafts: torch.Tensor,
                         accepted: torch.Tensor, token: torch.Tensor, n: int, max_drafts: int,
                         hist_rows: Optional[torch.Tensor] = None, out: Optional[tuple] = None,
                         stream: Optional[torch.cuda.Stream] = None):
    """Append each sequence's emitted tokens (drafts[b][:accepted[b]], then token[b]) to
    its history row (hist_rows[b], or b) and draft the next step from it.
    history [rows, stride] int32 and hist_len [rows] int32 are updated in place;
    drafts [B, K_in] int32; accepted, token [B] int32 -> (next drafts [B, K'], n_out [B])."""
    B = accepted.shape[0]
    stride = history.shape[1]
    if drafts.dim() != 2 or drafts.shape[0] != B or token.shape != (B,):
        raise ValueError("drafts must be [num_seqs, drafts_per_seq], token [num_seqs]")
    if hist_rows is not None and hist_rows.shape != (B,):
        raise ValueError("hist_rows must be [num_seqs]")
    K = max_drafts if max_drafts >= 1 else 4
    d, nn = out if out is not None else (torch.zeros(B, K, dtype=torch.int32, device="cuda"),
                                         torch.empty(B, dtype=torch.int32, device="cuda"))
    check(lib().gg_history_append_draft(
        _dev(history, "history", torch.int32), stride, _dev(hist_len, "hist_len", torch.int32),
        _dev(hist_rows, "hist_rows", torch.int32) if hist_rows is not None else None, B,
        _dev(drafts, "drafts", torch.int32) if drafts.numel() else None, drafts.shape[1],
        _dev(accepted, "accepted", torch.int32),
        _dev(token, "token", torch.int32), n, max_drafts, _dev(d, "drafts", torch.int32),
        _dev(nn, "n_out", torch.int32), _stream(stream)), "gg_history_append_draft")
    return d, nn
