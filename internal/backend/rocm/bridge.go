//go:build rocm

package rocm

/*
#cgo CFLAGS: -I${SRCDIR}/../../../third_party/gg_verify/include -D__HIP_PLATFORM_AMD__ -I/opt/rocm/include
#cgo LDFLAGS: -L${SRCDIR}/../../../third_party/gg_verify/lib -lgg_verify -L/opt/rocm/lib -lamdhip64
#include "gg_verify.h"
#include <hip/hip_runtime_api.h>
#include <stdlib.h>
*/
import "C"

import (
	"fmt"
	"unsafe"
)

// ggErr turns a status into a Go error carrying the library's last-error text, as
// the CUDA bridge does with gollmgo_backend_last_error.
func ggErr(where string, st C.gg_status_t) error {
	if st == C.GG_OK {
		return nil
	}
	return fmt.Errorf("rocm: %s: status %d: %s", where, int(st), C.GoString(C.gg_last_error()))
}

// Device memory and streams (the runtime calls a runner needs around the library).

func hipErr(where string, st C.hipError_t) error {
	if st == C.hipSuccess {
		return nil
	}
	return fmt.Errorf("rocm: %s: %s", where, C.GoString(C.hipGetErrorString(st)))
}

func deviceAlloc(n uintptr) (unsafe.Pointer, error) {
	var p unsafe.Pointer
	if n == 0 {
		n = 16
	}
	return p, hipErr("hipMalloc", C.hipMalloc(&p, C.size_t(n)))
}

// hostAlloc is pinned host memory (hipHostMalloc): asynchronous copies need it.
func hostAlloc(n uintptr) (unsafe.Pointer, error) {
	var p unsafe.Pointer
	if n == 0 {
		n = 16
	}
	return p, hipErr("hipHostMalloc", C.hipHostMalloc(&p, C.size_t(n), 0))
}

func deviceFree(p unsafe.Pointer) {
	if p != nil {
		C.hipFree(p)
	}
}

func hostFree(p unsafe.Pointer) {
	if p != nil {
		C.hipHostFree(p)
	}
}

func copyH2D(dst, src unsafe.Pointer, n uintptr, stream unsafe.Pointer) error {
	return hipErr("hipMemcpyAsync", C.hipMemcpyAsync(dst, src, C.size_t(n), C.hipMemcpyHostToDevice,
		C.hipStream_t(stream)))
}

// copyH2DSync copies from Go memory: synchronous, so C holds the Go pointer only during
// the call, as cgo requires.
func copyH2DSync(dst, src unsafe.Pointer, n uintptr) error {
	return hipErr("hipMemcpy", C.hipMemcpy(dst, src, C.size_t(n), C.hipMemcpyHostToDevice))
}

func copyD2H(dst, src unsafe.Pointer, n uintptr, stream unsafe.Pointer) error {
	return hipErr("hipMemcpyAsync", C.hipMemcpyAsync(dst, src, C.size_t(n), C.hipMemcpyDeviceToHost,
		C.hipStream_t(stream)))
}

func newStream() (unsafe.Pointer, error) {
	var s C.hipStream_t
	if err := hipErr("hipStreamCreate", C.hipStreamCreate(&s)); err != nil {
		return nil, err
	}
	return unsafe.Pointer(s), nil
}

func destroyStream(s unsafe.Pointer) {
	if s != nil {
		C.hipStreamDestroy(C.hipStream_t(s))
	}
}

func syncStream(s unsafe.Pointer) error { return ggErr("gg_sync", C.gg_sync(s)) }

// KVCache owns the paged K/V pools of all layers (device memory).
type KVCache struct {
	h         C.gg_kv_t
	blockSize int
}

func NewKVCache(layers, numBlocks, blockSize, kvHeads, headDim, dtype, scales int) (*KVCache, error) {
	var h C.gg_kv_t
	st := C.gg_kv_create(C.int(layers), C.int(numBlocks), C.int(blockSize), C.int(kvHeads),
		C.int(headDim), C.gg_dtype_t(dtype), C.gg_scale_mode_t(scales), &h)
	if err := ggErr("gg_kv_create", st); err != nil {
		return nil, err
	}
	return &KVCache{h: h, blockSize: blockSize}, nil
}

func (c *KVCache) Close() error { return ggErr("gg_kv_destroy", C.gg_kv_destroy(c.h)) }

// Append writes n new K/V rows (device [n][Hkv][D], bf16) of one layer to their slots
// (device int32[n], the engine's Batch.SlotMapping).
func (c *KVCache) Append(layer int, k, v unsafe.Pointer, slots unsafe.Pointer, n int, stream unsafe.Pointer) error {
	return ggErr("gg_kv_append", C.gg_kv_append(c.h, C.int(layer), k, v, C.GG_DTYPE_BF16,
		(*C.int32_t)(slots), C.int(n), stream))
}

// Attention runs the verify attention of one layer for B sequences with up to R rows.
// q/out: device [B][R][Hq][D] bf16; ctxLens, rowCounts: device int32[B];
// blockTables: device int32[B][maxBlocks]; ws: device workspace of wsBytes.
func (c *KVCache) Attention(layer int, q, out, ctxLens, rowCounts, blockTables unsafe.Pointer,
	maxBlocks, B, R, Hq int, scale float32, ws unsafe.Pointer, wsBytes uintptr, stream unsafe.Pointer) error {
	st := C.gg_verify_attention(c.h, C.int(layer), q, C.GG_DTYPE_BF16, out, C.GG_DTYPE_BF16,
		(*C.int32_t)(ctxLens), (*C.int32_t)(rowCounts), (*C.int32_t)(blockTables), C.int(maxBlocks),
		C.int(B), C.int(R), C.int(Hq), C.float(scale), 0, ws, C.size_t(wsBytes), stream)
	return ggErr("gg_verify_attention", st)
}

// Plan computes the step's attention schedule into ws (once per Step: it depends only on
// ctxLens / rowCounts); AttentionPlanned then runs any layer with it.
func (c *KVCache) Plan(ctxLens, rowCounts unsafe.Pointer, maxBlocks, B, R, Hq int, ws unsafe.Pointer,
	wsBytes uintptr, stream unsafe.Pointer) error {
	return ggErr("gg_verify_attention_plan", C.gg_verify_attention_plan(c.h, (*C.int32_t)(ctxLens),
		(*C.int32_t)(rowCounts), C.int(maxBlocks), C.int(B), C.int(R), C.int(Hq), ws, C.size_t(wsBytes), stream))
}

func (c *KVCache) AttentionPlanned(layer int, q, out, ctxLens, rowCounts, blockTables unsafe.Pointer,
	maxBlocks, B, R, Hq int, scale float32, ws unsafe.Pointer, wsBytes uintptr, stream unsafe.Pointer) error {
	st := C.gg_verify_attention_planned(c.h, C.int(layer), q, C.GG_DTYPE_BF16, out, C.GG_DTYPE_BF16,
		(*C.int32_t)(ctxLens), (*C.int32_t)(rowCounts), (*C.int32_t)(blockTables), C.int(maxBlocks),
		C.int(B), C.int(R), C.int(Hq), C.float(scale), ws, C.size_t(wsBytes), stream)
	return ggErr("gg_verify_attention_planned", st)
}

// AppendAttention appends the step's K/V rows of one layer (device [B*R][Hkv][D] bf16,
// row b*R+j = row j of sequence b) and runs the planned attention in one call: the rows go
// to key positions ctxLens[b]-rowCounts[b]+j through the block table, so no slot mapping
// is needed. PER_BLOCK INT8 pools included.
func (c *KVCache) AppendAttention(layer int, kNew, vNew, q, out, ctxLens, rowCounts, blockTables unsafe.Pointer,
	maxBlocks, B, R, Hq int, scale float32, ws unsafe.Pointer, wsBytes uintptr, stream unsafe.Pointer) error {
	st := C.gg_verify_append_attention_planned(c.h, C.int(layer), kNew, vNew, C.GG_DTYPE_BF16, q,
		C.GG_DTYPE_BF16, out, C.GG_DTYPE_BF16, (*C.int32_t)(ctxLens), (*C.int32_t)(rowCounts),
		(*C.int32_t)(blockTables), C.int(maxBlocks), C.int(B), C.int(R), C.int(Hq), C.float(scale), ws,
		C.size_t(wsBytes), stream)
	return ggErr("gg_verify_append_attention_planned", st)
}

// SnapshotKV / RestoreKV for the engine's KVSwapper (internal/backend/runner.go:94-106):
// blockIDs device int32[n]; staging device bytes >= SnapshotBytes(n); host pinned
// (C.hipHostMalloc) for an asynchronous copy. Restore may target other (fresh) block ids.
func (c *KVCache) SnapshotBytes(n int) uintptr { return uintptr(C.gg_kv_snapshot_bytes(c.h, C.int(n))) }

func (c *KVCache) Snapshot(blockIDs unsafe.Pointer, n int, staging unsafe.Pointer, stagingBytes uintptr,
	host unsafe.Pointer, stream unsafe.Pointer) error {
	return ggErr("gg_kv_snapshot", C.gg_kv_snapshot(c.h, (*C.int32_t)(blockIDs), C.int(n), staging,
		C.size_t(stagingBytes), host, stream))
}

func (c *KVCache) Restore(blockIDs unsafe.Pointer, n int, staging unsafe.Pointer, stagingBytes uintptr,
	host unsafe.Pointer, stream unsafe.Pointer) error {
	return ggErr("gg_kv_restore", C.gg_kv_restore(c.h, (*C.int32_t)(blockIDs), C.int(n), staging,
		C.size_t(stagingBytes), host, stream))
}

// AttentionWorkspace is the workspace size for a (B, R, Hq, maxBlocks) shape; allocate it
// once per warm-up profile (Runner.Warmup), never per step.
func (c *KVCache) AttentionWorkspace(B, R, Hq, maxBlocks int) uintptr {
	return uintptr(C.gg_verify_attention_workspace_size(c.h, C.int(B), C.int(R), C.int(Hq), C.int(maxBlocks), 0))
}

// AcceptGreedy: logits device [B][K+1][V] (f32/bf16), drafts device int32[B][K],
// nDrafts device int32[B] -> accepted, token device int32[B].
func AcceptGreedy(logits unsafe.Pointer, dt int, B, K, V int, drafts, nDrafts,
	accepted, token, ws unsafe.Pointer, wsBytes uintptr, stream unsafe.Pointer) error {
	st := C.gg_accept_greedy(logits, C.gg_dtype_t(dt), C.int(B), C.int(K), C.int(V), (*C.int32_t)(drafts),
		(*C.int32_t)(nDrafts), (*C.int32_t)(accepted), (*C.int32_t)(token), ws, C.size_t(wsBytes), stream)
	return ggErr("gg_accept_greedy", st)
}

// AcceptGreedySample: AcceptGreedy whose bonus token (every draft accepted) is drawn as the
// engine's Sampler.Sample draws it, with temperature, topK and topP of the engine's
// SamplingParams and uniforms (device float64 [B]) in place of rng.Float64().
func AcceptGreedySample(logits unsafe.Pointer, dt int, B, K, V int, drafts, nDrafts unsafe.Pointer,
	temperature float64, topK int, topP float64, uniforms, accepted, token, ws unsafe.Pointer, wsBytes uintptr,
	stream unsafe.Pointer) error {
	st := C.gg_accept_greedy_sample(logits, C.gg_dtype_t(dt), C.int(B), C.int(K), C.int(V), (*C.int32_t)(drafts),
		(*C.int32_t)(nDrafts), C.double(temperature), C.int(topK), C.double(topP), (*C.double)(uniforms), 0,
		(*C.int32_t)(accepted), (*C.int32_t)(token), ws, C.size_t(wsBytes), stream)
	return ggErr("gg_accept_greedy_sample", st)
}

// AcceptRejection: as AcceptGreedy plus draftProbs (device float [B][K][V], or nil for
// the one-hot n-gram drafter), uniforms (device float [B][K+1]), temperature, topP.
func AcceptRejection(logits unsafe.Pointer, dt int, draftProbs unsafe.Pointer, B, K, V int,
	drafts, nDrafts, uniforms unsafe.Pointer, temperature, topP float32,
	accepted, token, ws unsafe.Pointer, wsBytes uintptr, stream unsafe.Pointer) error {
	st := C.gg_accept_rejection(logits, C.gg_dtype_t(dt), (*C.float)(draftProbs), C.int(B), C.int(K), C.int(V),
		(*C.int32_t)(drafts), (*C.int32_t)(nDrafts), (*C.float)(uniforms), C.float(temperature),
		C.float(topP), (*C.int32_t)(accepted), (*C.int32_t)(token), ws, C.size_t(wsBytes), stream)
	return ggErr("gg_accept_rejection", st)
}

// NGramDraft: history device int32[B][stride], histLen device int32[B] ->
// drafts device int32[B][K], nDrafts device int32[B].
func NGramDraft(history unsafe.Pointer, stride int, histLen unsafe.Pointer, B, n, K int,
	drafts, nDrafts unsafe.Pointer, stream unsafe.Pointer) error {
	st := C.gg_ngram_draft((*C.int32_t)(history), C.int(stride), (*C.int32_t)(histLen), C.int(B),
		C.int(n), C.int(K), (*C.int32_t)(drafts), (*C.int32_t)(nDrafts), stream)
	return ggErr("gg_ngram_draft", st)
}

// HistoryAppendDraft appends each sequence's emitted tokens (drafts[b][:accepted[b]],
// then token[b]) to its device history row (rows[b], or b when rows is nil) and drafts
// the next step from it: next device int32[B][K], nNext device int32[B]. A row the
// tokens would overflow gets length -1 and no drafts.
func HistoryAppendDraft(history unsafe.Pointer, stride int, histLen, rows unsafe.Pointer, B int,
	drafts unsafe.Pointer, kIn int, accepted, token unsafe.Pointer, n, K int, next, nNext unsafe.Pointer,
	stream unsafe.Pointer) error {
	st := C.gg_history_append_draft((*C.int32_t)(history), C.int(stride), (*C.int32_t)(histLen),
		(*C.int32_t)(rows), C.int(B), (*C.int32_t)(drafts), C.int(kIn), (*C.int32_t)(accepted),
		(*C.int32_t)(token), C.int(n), C.int(K), (*C.int32_t)(next), (*C.int32_t)(nNext), stream)
	return ggErr("gg_history_append_draft", st)
}

func AcceptGreedyWorkspace(B, K, V int) uintptr {
	return uintptr(C.gg_accept_greedy_workspace_size(C.int(B), C.int(K), C.int(V)))
}

func AcceptGreedySampleWorkspace(B, K, V int) uintptr {
	return uintptr(C.gg_accept_greedy_sample_workspace_size(C.int(B), C.int(K), C.int(V)))
}

func AcceptRejectionWorkspace(B, K, V int) uintptr {
	return uintptr(C.gg_accept_rejection_workspace_size(C.int(B), C.int(K), C.int(V)))
}

// Element types and scale modes of gg_verify.h, for callers outside this file.
const (
	DtypeF32  = int(C.GG_DTYPE_F32)
	DtypeF16  = int(C.GG_DTYPE_F16)
	DtypeBF16 = int(C.GG_DTYPE_BF16)
	DtypeFP8  = int(C.GG_DTYPE_FP8_E4M3)
	DtypeINT8 = int(C.GG_DTYPE_INT8)

	ScaleNone     = int(C.GG_SCALE_NONE)
	ScalePerHead  = int(C.GG_SCALE_PER_HEAD)
	ScalePerBlock = int(C.GG_SCALE_PER_BLOCK)
)
