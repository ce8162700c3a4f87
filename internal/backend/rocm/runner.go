//go:build rocm

package rocm

import (
	"context"
	"fmt"
	"math"
	"math/rand"
	"unsafe"

	"github.com/TensorGreed/gollmgo/internal/backend"
	"github.com/TensorGreed/gollmgo/internal/engine"
)

// Model is the part of a step that lives outside libgg_verify: embeddings, the
// per-layer projections, norms, RoPE and MLP, and the LM head (the reference's
// kernels/gollmgo_model.cu run_layer, minus its KV write and attention). It works on the
// runner's [B][R] row layout: row j of sequence b is device row b*R+j, and padding rows
// (j >= the sequence's token count) are computed and ignored. Every call is asynchronous
// on the given stream.
type Model interface {
	NumLayers() int
	NumQHeads() int
	NumKVHeads() int
	HeadDim() int
	Vocab() int
	// Embed loads the step's tokens (device int32 [B][R]) into the hidden state.
	Embed(tokens unsafe.Pointer, B, R int, stream unsafe.Pointer) error
	// QKV writes layer's q [B][R][Hq][D] and k, v [B][R][Hkv][D] (bf16, RoPE applied at
	// positions, device int32 [B][R]).
	QKV(layer int, positions, q, k, v unsafe.Pointer, stream unsafe.Pointer) error
	// Post takes layer's attention output [B][R][Hq][D] (bf16) through the output
	// projection, residual and MLP.
	Post(layer int, attnOut unsafe.Pointer, stream unsafe.Pointer) error
	// Logits writes every row's logits, device bf16 [B][R][V].
	Logits(logits unsafe.Pointer, stream unsafe.Pointer) error
	// Prefill runs a batch that holds prefill sequences on the model's own path.
	Prefill(ctx context.Context, batch *backend.Batch) (*backend.StepOutput, error)
}

// Acceptance selects how the device decides a step's drafts.
type Acceptance int

const (
	// AcceptGreedy: the reference's Verify on the device; when every draft is accepted the
	// bonus token is drawn on the device as the engine's Sampler.Sample would draw it, with
	// Config.Sampling (the engine's own SamplingParams) and the runner's uniform stream.
	AcceptGreedy Acceptance = iota
	// AcceptBonusRow: Verify on the device; when every draft is accepted the bonus row's real
	// logits are copied back, so the engine's Sampler (and its random stream) draws the
	// bonus exactly as with the reference's runner. One D2H row per such sequence.
	AcceptBonusRow
	// AcceptRejection: speculative sampling at Sampling's temperature and top-p (no
	// counterpart in the reference), one-hot draft distributions.
	AcceptRejection
)

// Config fixes the pools and the acceptance rule.
type Config struct {
	NumBlocks  int
	BlockSize  int
	KVDtype    int // Dtype* of bridge.go
	KVScales   int // Scale*: PerHead for FP8, PerBlock for INT8, None otherwise
	MaxDrafts  int // K: rows per sequence are K+1
	Acceptance Acceptance
	// Sampling must be the SamplingParams the engine was built with
	// (ServingEngineConfig.Sampling): the device draws with them.
	Sampling engine.SamplingParams
	// Device drafting (drafts.go): each sequence's history kept on the device and the
	// next step drafted there after the acceptance, served through Drafts.
	DeviceDrafts  bool
	NGramN        int // the engine's n-gram size (NewNGramDrafter)
	HistoryStride int // longest history kept on the device (0: the warm-up MaxSeqLen)
	HistoryRows   int // sequences with a device history (0: 4 x the warm-up batch)
}

// Runner implements backend.Runner (internal/backend/runner.go:84-93) and
// backend.KVSwapper (runner.go:94-106) for decode steps with drafts. Per step the host
// packs the batch (PackBatch), uploads it in one copy, runs the model with the verify
// attention of every layer, the acceptance, and copies back 2*B int32s: the decision,
// returned to the engine as one-hot LogitsPerPosition rows (OneHotRows).
type Runner struct {
	model  Model
	cfg    Config
	kv     *KVCache
	stream unsafe.Pointer
	rows   *OneHotRows
	rng    *rand.Rand

	maxB, maxR, maxBlocks int
	hq, hkv, d, vocab     int
	drafts                *deviceDrafts // nil without DeviceDrafts

	// Device buffers (allocated once at Warmup).
	dIn                       unsafe.Pointer // the packed int32 inputs + uniforms, one upload
	dQ, dK, dV, dOut, dLogits unsafe.Pointer
	dAttnWS, dAccWS, dDec     unsafe.Pointer
	attnWS, accWS             uintptr
	// Pinned host staging of the same layout, of the decision and (AcceptBonusRow) of the
	// bonus rows.
	hIn, hDec, hBonus unsafe.Pointer
	inBytes           uintptr
}

// New creates the pools; buffers follow at Warmup.
func New(model Model, cfg Config) (*Runner, error) {
	kv, err := NewKVCache(model.NumLayers(), cfg.NumBlocks, cfg.BlockSize, model.NumKVHeads(), model.HeadDim(),
		cfg.KVDtype, cfg.KVScales)
	if err != nil {
		return nil, err
	}
	s, err := newStream()
	if err != nil {
		kv.Close()
		return nil, err
	}
	seed := int64(1)
	if cfg.Sampling.Seed != nil {
		seed = int64(*cfg.Sampling.Seed)
	}
	return &Runner{
		model: model, cfg: cfg, kv: kv, stream: s, rows: NewOneHotRows(model.Vocab()),
		rng: rand.New(rand.NewSource(seed)),
		hq:  model.NumQHeads(), hkv: model.NumKVHeads(), d: model.HeadDim(), vocab: model.Vocab(),
	}, nil
}

// Input layout of one step (int32 words): tokens, positions, slots [B*R]; ctx, rows,
// n_drafts, history rows [B]; tables [B*maxBlocks]; drafts [B*K]; then the uniforms, at an
// even word: float32 [B*R] (rejection) or float64 [B] (the bonus draw).
type inLayout struct {
	tokens, positions, slots, ctx, rows, tables, drafts, nDrafts, histRows, uniforms, words int
}

func layout(B, R, MB int) inLayout {
	var l inLayout
	off := 0
	take := func(n int) int { o := off; off += n; return o }
	l.tokens, l.positions, l.slots = take(B*R), take(B*R), take(B*R)
	l.ctx, l.rows, l.nDrafts, l.histRows = take(B), take(B), take(B), take(B)
	l.tables, l.drafts = take(B*MB), take(B*(R-1))
	off += off & 1
	uw := B * R
	if uw < 2*B {
		uw = 2 * B
	}
	l.uniforms = take(uw)
	l.words = off
	return l
}

func (r *Runner) Warmup(_ context.Context, p backend.WarmupProfile) error {
	if p.BlockSize != 0 && p.BlockSize != r.cfg.BlockSize {
		return fmt.Errorf("rocm: warm-up block size %d, pools use %d", p.BlockSize, r.cfg.BlockSize)
	}
	r.release()
	r.maxB, r.maxR = p.MaxBatchSize, r.cfg.MaxDrafts+1
	r.maxBlocks = (p.MaxSeqLen + r.cfg.BlockSize - 1) / r.cfg.BlockSize
	B, R := r.maxB, r.maxR
	r.inBytes = uintptr(layout(B, R, r.maxBlocks).words) * 4
	r.attnWS = r.kv.AttentionWorkspace(B, R, r.hq, r.maxBlocks)
	if r.cfg.Acceptance == AcceptRejection {
		r.accWS = AcceptRejectionWorkspace(B, R-1, r.vocab)
	} else {
		r.accWS = AcceptGreedySampleWorkspace(B, R-1, r.vocab)
	}
	rowBytes := uintptr(B*R) * 2
	var err error
	for _, a := range []struct {
		p *unsafe.Pointer
		n uintptr
	}{
		{&r.dIn, r.inBytes}, {&r.dQ, rowBytes * uintptr(r.hq*r.d)}, {&r.dOut, rowBytes * uintptr(r.hq*r.d)},
		{&r.dK, rowBytes * uintptr(r.hkv*r.d)}, {&r.dV, rowBytes * uintptr(r.hkv*r.d)},
		{&r.dLogits, rowBytes * uintptr(r.vocab)}, {&r.dAttnWS, r.attnWS}, {&r.dAccWS, r.accWS},
		{&r.dDec, uintptr(2*B) * 4},
	} {
		if *a.p, err = deviceAlloc(a.n); err != nil {
			r.release()
			return err
		}
	}
	if r.hIn, err = hostAlloc(r.inBytes); err == nil {
		r.hDec, err = hostAlloc(uintptr(2*B) * 4)
	}
	if err == nil && r.cfg.Acceptance == AcceptBonusRow {
		r.hBonus, err = hostAlloc(uintptr(B*r.vocab) * 2)
	}
	if err == nil && r.cfg.DeviceDrafts {
		stride, rows := r.cfg.HistoryStride, r.cfg.HistoryRows
		if stride <= 0 {
			stride = p.MaxSeqLen
		}
		if rows <= 0 {
			rows = 4 * B
		}
		r.drafts, err = newDeviceDrafts(r.cfg.NGramN, r.cfg.MaxDrafts, stride, rows, B)
	}
	if err != nil {
		r.release()
	}
	return err
}

func i32(base unsafe.Pointer, word int, n int) []int32 {
	return unsafe.Slice((*int32)(unsafe.Add(base, 4*word)), n)
}

func at(base unsafe.Pointer, word int) unsafe.Pointer { return unsafe.Add(base, 4*word) }

func (r *Runner) Step(ctx context.Context, batch *backend.Batch) (*backend.StepOutput, error) {
	for _, p := range batch.IsPrefill {
		if p {
			if r.drafts != nil {
				r.drafts.prefill(batch)
			}
			return r.model.Prefill(ctx, batch)
		}
	}
	if r.dIn == nil {
		return nil, fmt.Errorf("rocm: Step before Warmup")
	}
	if len(batch.SequenceIDs) > r.maxB {
		return nil, fmt.Errorf("rocm: batch of %d exceeds the warmed-up %d", len(batch.SequenceIDs), r.maxB)
	}
	in, err := PackBatch(batch, r.cfg.BlockSize, r.maxBlocks, r.maxR)
	if err != nil {
		return nil, err
	}
	B, R, MB, K := in.NumSeqs, in.RowsPerSeq, in.MaxBlocks, in.RowsPerSeq-1
	l := layout(B, R, MB)
	copy(i32(r.hIn, l.tokens, B*R), in.Tokens)
	copy(i32(r.hIn, l.positions, B*R), in.Positions)
	copy(i32(r.hIn, l.slots, B*R), in.Slots)
	copy(i32(r.hIn, l.ctx, B), in.CtxLens)
	copy(i32(r.hIn, l.rows, B), in.RowCounts)
	copy(i32(r.hIn, l.nDrafts, B), in.NDrafts)
	copy(i32(r.hIn, l.tables, B*MB), in.BlockTables)
	copy(i32(r.hIn, l.drafts, B*K), in.Drafts)
	if r.cfg.Acceptance == AcceptRejection {
		u := unsafe.Slice((*float32)(at(r.hIn, l.uniforms)), B*R)
		for i := range u {
			u[i] = r.rng.Float32()
		}
	} else {
		u := unsafe.Slice((*float64)(at(r.hIn, l.uniforms)), B)
		for i := range u {
			u[i] = r.rng.Float64()
		}
	}
	s := r.stream
	histRows := i32(r.hIn, l.histRows, B)
	if r.drafts != nil { // the current tokens into the histories; rows seeded where needed
		if err := r.drafts.prepare(in, batch.SequenceIDs, histRows, s); err != nil {
			return nil, err
		}
	}
	if err := copyH2D(r.dIn, r.hIn, uintptr(l.words)*4, s); err != nil {
		return nil, err
	}
	d := func(word int) unsafe.Pointer { return at(r.dIn, word) }
	scale := float32(1.0 / math.Sqrt(float64(r.d))) // as gollmgo_model.cu
	if err := r.model.Embed(d(l.tokens), B, R, s); err != nil {
		return nil, err
	}
	if err := r.kv.Plan(d(l.ctx), d(l.rows), MB, B, R, r.hq, r.dAttnWS, r.attnWS, s); err != nil {
		return nil, err
	}
	for layer := 0; layer < r.model.NumLayers(); layer++ {
		if err := r.model.QKV(layer, d(l.positions), r.dQ, r.dK, r.dV, s); err != nil {
			return nil, err
		}
		// The rows' K/V are appended inside the attention call (PER_BLOCK INT8 pools
		// included: the workgroup that reads a block with new rows re-scales it first).
		if err := r.kv.AppendAttention(layer, r.dK, r.dV, r.dQ, r.dOut, d(l.ctx), d(l.rows), d(l.tables), MB, B,
			R, r.hq, scale, r.dAttnWS, r.attnWS, s); err != nil {
			return nil, err
		}
		if err := r.model.Post(layer, r.dOut, s); err != nil {
			return nil, err
		}
	}
	if err := r.model.Logits(r.dLogits, s); err != nil {
		return nil, err
	}
	acc, tok := r.dDec, unsafe.Add(r.dDec, 4*B)
	sp := r.cfg.Sampling
	switch r.cfg.Acceptance {
	case AcceptRejection:
		err = AcceptRejection(r.dLogits, DtypeBF16, nil, B, K, r.vocab, d(l.drafts), d(l.nDrafts), d(l.uniforms),
			float32(sp.Temperature), float32(sp.TopP), acc, tok, r.dAccWS, r.accWS, s)
	case AcceptBonusRow:
		err = AcceptGreedy(r.dLogits, DtypeBF16, B, K, r.vocab, d(l.drafts), d(l.nDrafts), acc, tok, r.dAccWS,
			r.accWS, s)
	default:
		err = AcceptGreedySample(r.dLogits, DtypeBF16, B, K, r.vocab, d(l.drafts), d(l.nDrafts), sp.Temperature,
			sp.TopK, sp.TopP, d(l.uniforms), acc, tok, r.dAccWS, r.accWS, s)
	}
	if err != nil {
		return nil, err
	}
	if r.drafts != nil { // emitted tokens appended on the device, next drafts computed there
		if err := r.drafts.launch(d(l.histRows), d(l.drafts), B, K, acc, tok, s); err != nil {
			return nil, err
		}
	}
	if err := copyD2H(r.hDec, r.dDec, uintptr(2*B)*4, s); err != nil {
		return nil, err
	}
	if err := syncStream(s); err != nil {
		return nil, err
	}
	hAcc, hTok := i32(r.hDec, 0, B), i32(r.hDec, B, B)
	var bonus [][]float32
	if r.cfg.Acceptance == AcceptBonusRow {
		if bonus, err = r.bonusRows(in, hAcc, B, R); err != nil {
			return nil, err
		}
	}
	if r.drafts != nil {
		r.drafts.finish(in, batch.SequenceIDs, histRows, hAcc, hTok)
	}
	out := &backend.StepOutput{
		Logits:            make([][]float32, B),
		LogitsPerPosition: make([][][]float32, B),
	}
	for i := 0; i < B; i++ {
		n := int(in.NDrafts[i])
		rows, err := r.rows.RowsFor(in.Drafts[i*K:i*K+n], int(hAcc[i]), hTok[i])
		if err != nil {
			return nil, fmt.Errorf("rocm: sequence %d: %w", i, err)
		}
		if bonus != nil && bonus[i] != nil {
			rows[len(rows)-1] = bonus[i] // the engine's Sampler draws the bonus
		}
		out.Logits[i] = rows[0]
		if n > 0 {
			out.LogitsPerPosition[i] = rows
		}
	}
	return out, nil
}

// bonusRows copies back, for every sequence that accepted all its drafts, the logits of its
// bonus row (bf16 on the device) as float32, as the reference's runner returns rows
// (kernels/gollmgo_model.cu:1057-1060). Other sequences get nil.
func (r *Runner) bonusRows(in *StepInputs, hAcc []int32, B, R int) ([][]float32, error) {
	V := r.vocab
	need := false
	for i := 0; i < B; i++ {
		if int(hAcc[i]) == int(in.NDrafts[i]) {
			src := unsafe.Add(r.dLogits, uintptr((i*R+int(in.NDrafts[i]))*V)*2)
			if err := copyD2H(unsafe.Add(r.hBonus, uintptr(i*V)*2), src, uintptr(V)*2, r.stream); err != nil {
				return nil, err
			}
			need = true
		}
	}
	if !need {
		return nil, nil
	}
	if err := syncStream(r.stream); err != nil {
		return nil, err
	}
	out := make([][]float32, B)
	for i := 0; i < B; i++ {
		if int(hAcc[i]) != int(in.NDrafts[i]) {
			continue
		}
		h := unsafe.Slice((*uint16)(unsafe.Add(r.hBonus, uintptr(i*V)*2)), V)
		row := make([]float32, V)
		for j, b := range h {
			row[j] = math.Float32frombits(uint32(b) << 16)
		}
		out[i] = row
	}
	return out, nil
}

func (r *Runner) Capabilities() backend.Capabilities {
	return backend.Capabilities{
		FP16: true, BF16: true, FP8: true, INT8: true,
		PagedAttention:      true,
		CUDAGraphs:          false, // the step is capture-safe; this runner does not capture yet
		SpeculativeDecoding: true,  // K+1 rows per sequence in one Step
		KVSwap:              true,
	}
}

func (r *Runner) release() {
	for _, p := range []*unsafe.Pointer{&r.dIn, &r.dQ, &r.dK, &r.dV, &r.dOut, &r.dLogits, &r.dAttnWS, &r.dAccWS,
		&r.dDec} {
		deviceFree(*p)
		*p = nil
	}
	hostFree(r.hIn)
	hostFree(r.hDec)
	hostFree(r.hBonus)
	r.hIn, r.hDec, r.hBonus = nil, nil, nil
	if r.drafts != nil {
		r.drafts.close()
		r.drafts = nil
	}
}

func (r *Runner) Close() error {
	if r.kv == nil {
		return nil
	}
	syncStream(r.stream)
	r.release()
	destroyStream(r.stream)
	err := r.kv.Close()
	r.kv, r.stream = nil, nil
	return err
}

// Snapshot is a KV swap snapshot held in pinned host memory.
type Snapshot struct {
	host   unsafe.Pointer
	bytes  uintptr
	blocks int
}

func (s *Snapshot) NumBlocks() int     { return s.blocks }
func (s *Snapshot) BytesOnHost() int64 { return int64(s.bytes) }
func (s *Snapshot) Release() error {
	hostFree(s.host)
	s.host = nil
	return nil
}

// swapIO uploads the block ids and allocates the device staging of one swap (a swap is
// a preemption event, not a per-step call, so it may allocate).
func (r *Runner) swapIO(blockIDs []int32) (ids, staging unsafe.Pointer, n uintptr, err error) {
	n = r.kv.SnapshotBytes(len(blockIDs))
	if ids, err = deviceAlloc(uintptr(4 * len(blockIDs))); err != nil {
		return
	}
	if staging, err = deviceAlloc(n); err != nil {
		deviceFree(ids)
		return
	}
	if err = syncStream(r.stream); err == nil { // earlier work on the stream first
		err = copyH2DSync(ids, unsafe.Pointer(&blockIDs[0]), uintptr(4*len(blockIDs)))
	}
	if err != nil {
		deviceFree(ids)
		deviceFree(staging)
	}
	return
}

func (r *Runner) SnapshotKV(_ context.Context, blockIDs []int32) (backend.KVSnapshot, error) {
	if len(blockIDs) == 0 {
		return &Snapshot{}, nil
	}
	ids, staging, n, err := r.swapIO(blockIDs)
	if err != nil {
		return nil, err
	}
	defer deviceFree(ids)
	defer deviceFree(staging)
	host, err := hostAlloc(n)
	if err != nil {
		return nil, err
	}
	if err = r.kv.Snapshot(ids, len(blockIDs), staging, n, host, r.stream); err == nil {
		err = syncStream(r.stream)
	}
	if err != nil {
		hostFree(host)
		return nil, err
	}
	return &Snapshot{host: host, bytes: n, blocks: len(blockIDs)}, nil
}

func (r *Runner) RestoreKV(_ context.Context, snap backend.KVSnapshot, blockIDs []int32) error {
	s, ok := snap.(*Snapshot)
	if !ok {
		return fmt.Errorf("rocm: snapshot of another backend")
	}
	if s.blocks != len(blockIDs) {
		return fmt.Errorf("rocm: snapshot of %d blocks restored into %d", s.blocks, len(blockIDs))
	}
	if len(blockIDs) == 0 {
		return nil
	}
	ids, staging, n, err := r.swapIO(blockIDs)
	if err != nil {
		return err
	}
	defer deviceFree(ids)
	defer deviceFree(staging)
	if err := r.kv.Restore(ids, len(blockIDs), staging, n, s.host, r.stream); err != nil {
		return err
	}
	return syncStream(r.stream)
}

var (
	_ backend.Runner    = (*Runner)(nil)
	_ backend.KVSwapper = (*Runner)(nil)
)
