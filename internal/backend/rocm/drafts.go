//go:build rocm

package rocm

import (
	"unsafe"

	"github.com/TensorGreed/gollmgo/internal/backend"
)

// DraftSource is the engine-side hook this file serves. It is not in the engine yet: the
// interface would sit in internal/backend next to Runner, and maybeDraft
// (internal/engine/serving.go:608-620) would ask the runner first and fall back to its
// host NGramDrafter when the runner has nothing for the sequence:
//
//	if ds, ok := e.runner.(backend.DraftSource); ok {
//		if d, ok := ds.Drafts(seq.ID, len(seq.TokenIDs)); ok {
//			return d
//		}
//	}
//	return e.drafter.Draft(seq.TokenIDs)
//
// histLen is the length of the engine's history (prompt + generated); the runner answers
// only when its own history of the sequence has that length, so any divergence (a stop
// at EOS, a preemption, a sequence it never saw from the start) falls back to the host.
type DraftSource interface {
	Drafts(seqID uint64, histLen int) ([]int32, bool)
}

// deviceDrafts keeps each sequence's token history on the device and drafts the next step
// there, in the launch after the acceptance (gg_history_append_draft), so no history
// crosses PCIe per step: only the B*K next drafts come back with the decision. The host
// keeps a mirror of every history (the truth: it seeds or reseeds a device row whenever
// the row's length does not match), built from the prefill tokens, each step's current
// token and the emitted tokens of the device decision.
type deviceDrafts struct {
	n, k, stride, nRows int
	dHist, dLen        unsafe.Pointer // device int32 [nRows][stride], [nRows]
	hSeed              unsafe.Pointer // pinned int32 [maxB][stride] rows to (re)seed, then [maxB] lengths
	maxB               int
	dNext              unsafe.Pointer // device int32 [maxB][k] drafts, then [maxB] counts
	hNext              unsafe.Pointer // pinned copy of dNext
	scratchRow         int32          // a row whose length is kept at -1 (no drafts)
	seqs               map[uint64]*seqHistory
	free               []int32
	clock              uint64
	next               map[uint64]nextDrafts
}

type seqHistory struct {
	tokens []int32 // prompt + generated, as the engine's seq.TokenIDs
	row    int32   // device row, -1 if none
	devLen int32   // the device row's length as last set (-1: unusable)
	used   uint64  // step of last use (for eviction)
}

type nextDrafts struct {
	histLen int
	drafts  []int32
}

func newDeviceDrafts(n, k, stride, nRows, maxB int) (*deviceDrafts, error) {
	if n < 2 {
		n = 2
	}
	if k < 1 {
		k = 4
	}
	dd := &deviceDrafts{n: n, k: k, stride: stride, nRows: nRows + 1, scratchRow: int32(nRows), maxB: maxB,
		seqs: map[uint64]*seqHistory{}, next: map[uint64]nextDrafts{}}
	var err error
	for _, a := range []struct {
		p *unsafe.Pointer
		n uintptr
	}{
		{&dd.dHist, uintptr(dd.nRows*stride) * 4}, {&dd.dLen, uintptr(dd.nRows) * 4},
		{&dd.dNext, uintptr(maxB*(k+1)) * 4},
	} {
		if *a.p, err = deviceAlloc(a.n); err != nil {
			dd.close()
			return nil, err
		}
	}
	if dd.hSeed, err = hostAlloc(uintptr(maxB*(stride+1)) * 4); err == nil {
		dd.hNext, err = hostAlloc(uintptr(maxB*(k+1)) * 4)
	}
	if err != nil {
		dd.close()
		return nil, err
	}
	// Every row starts unusable (length -1), the scratch row stays so.
	lens := make([]int32, dd.nRows)
	for i := range lens {
		lens[i] = -1
	}
	if err = copyH2DSync(dd.dLen, unsafe.Pointer(&lens[0]), uintptr(4*dd.nRows)); err != nil {
		dd.close()
		return nil, err
	}
	for r := int32(0); r < int32(nRows); r++ {
		dd.free = append(dd.free, r)
	}
	return dd, nil
}

func (dd *deviceDrafts) close() {
	for _, p := range []*unsafe.Pointer{&dd.dHist, &dd.dLen, &dd.dNext} {
		deviceFree(*p)
		*p = nil
	}
	hostFree(dd.hSeed)
	hostFree(dd.hNext)
	dd.hSeed, dd.hNext = nil, nil
}

// prefill records the prompt tokens of the batch's prefill sequences (chunked prefill
// included: each token lands at its position).
func (dd *deviceDrafts) prefill(b *backend.Batch) {
	t0 := 0
	for i, id := range b.SequenceIDs {
		c := int(b.SeqTokenCounts[i])
		if b.IsPrefill[i] {
			h := dd.seqs[id]
			if h == nil {
				h = &seqHistory{row: -1, devLen: -1}
				dd.seqs[id] = h
			}
			for j := 0; j < c; j++ {
				h.put(int(b.Positions[t0+j]), b.TokenIDs[t0+j])
			}
		}
		t0 += c
	}
}

// put writes token t at position p of the history (a rewrite drops what follows p).
func (h *seqHistory) put(p int, t int32) {
	switch {
	case p == len(h.tokens):
		h.tokens = append(h.tokens, t)
	case p < len(h.tokens):
		h.tokens = append(h.tokens[:p], t)
		h.devLen = -1 // the device row no longer matches
	default: // a gap: this history is unknown
		h.tokens = nil
		h.devLen = -1
	}
}

// prepare runs before a decode step: each sequence's history gets its current token
// (position positions[b*R]), and a row whose device length does not match is seeded
// from the mirror. It fills rows[b] (the scratch row for sequences without a usable
// history) and issues the seed copies on the stream.
func (dd *deviceDrafts) prepare(in *StepInputs, ids []uint64, rows []int32, stream unsafe.Pointer) error {
	dd.clock++
	if dd.clock%256 == 0 { // forget sequences unseen for 256 steps (finished or evicted)
		for id, h := range dd.seqs {
			if dd.clock-h.used > 256 {
				if h.row >= 0 {
					dd.free = append(dd.free, h.row)
				}
				delete(dd.seqs, id)
				delete(dd.next, id)
			}
		}
	}
	R := in.RowsPerSeq
	seeded := 0
	for b := 0; b < in.NumSeqs; b++ {
		h := dd.seqs[ids[b]]
		if h == nil {
			h = &seqHistory{row: -1, devLen: -1}
			dd.seqs[ids[b]] = h
		}
		h.used = dd.clock
		p := int(in.Positions[b*R])
		if len(h.tokens) < p { // never saw the start of this sequence
			h.tokens = nil
		} else {
			h.put(p, in.Tokens[b*R])
		}
		if len(h.tokens) == 0 || len(h.tokens) > dd.stride {
			rows[b] = dd.scratchRow
			continue
		}
		if h.row < 0 && !dd.allocRow(h) {
			rows[b] = dd.scratchRow
			continue
		}
		rows[b] = h.row
		if int(h.devLen) != len(h.tokens) {
			// Seed: the history into the pinned staging, then into the row and its length.
			stage := unsafe.Add(dd.hSeed, 4*seeded*dd.stride)
			copy(unsafe.Slice((*int32)(stage), len(h.tokens)), h.tokens)
			n := int32(len(h.tokens))
			if err := copyH2D(unsafe.Add(dd.dHist, 4*int(h.row)*dd.stride), stage, uintptr(4*len(h.tokens)),
				stream); err != nil {
				return err
			}
			lenStage := unsafe.Add(dd.hSeed, 4*(dd.maxB*dd.stride+seeded))
			*(*int32)(lenStage) = n
			if err := copyH2D(unsafe.Add(dd.dLen, 4*int(h.row)), lenStage, 4, stream); err != nil {
				return err
			}
			h.devLen = n
			seeded++
		}
	}
	return nil
}

// allocRow gives h a device row, evicting the least recently used sequence's row when
// none is free.
func (dd *deviceDrafts) allocRow(h *seqHistory) bool {
	if len(dd.free) == 0 {
		var victim *seqHistory
		for _, o := range dd.seqs {
			if o.row >= 0 && o.used < dd.clock && (victim == nil || o.used < victim.used) {
				victim = o
			}
		}
		if victim == nil {
			return false
		}
		dd.free = append(dd.free, victim.row)
		victim.row, victim.devLen = -1, -1
	}
	h.row = dd.free[len(dd.free)-1]
	dd.free = dd.free[:len(dd.free)-1]
	h.devLen = -1
	return true
}

// launch appends the decision's emitted tokens and drafts the next step on the device
// (after the acceptance on the same stream), and queues the drafts' copy back.
func (dd *deviceDrafts) launch(dRows, dDrafts unsafe.Pointer, B, kIn int, acc, tok unsafe.Pointer,
	stream unsafe.Pointer) error {
	next, nNext := dd.dNext, unsafe.Add(dd.dNext, 4*B*dd.k)
	if err := HistoryAppendDraft(dd.dHist, dd.stride, dd.dLen, dRows, B, dDrafts, kIn, acc, tok, dd.n, dd.k,
		next, nNext, stream); err != nil {
		return err
	}
	return copyD2H(dd.hNext, dd.dNext, uintptr(4*B*(dd.k+1)), stream)
}

// finish runs after the stream synchronised: the mirrors get the emitted tokens (the
// device rows did the same, or set their length to -1 on overflow), and the next drafts
// are kept for Drafts.
func (dd *deviceDrafts) finish(in *StepInputs, ids []uint64, rows []int32, hAcc, hTok []int32) {
	B, K := in.NumSeqs, in.RowsPerSeq-1
	next := unsafe.Slice((*int32)(dd.hNext), B*(dd.k+1))
	for b := 0; b < B; b++ {
		h := dd.seqs[ids[b]]
		acc := int(hAcc[b])
		if acc < 0 {
			acc = 0
		}
		if acc > int(in.NDrafts[b]) {
			acc = int(in.NDrafts[b])
		}
		emitted := append([]int32(nil), in.Drafts[b*K:b*K+acc]...)
		if hTok[b] >= 0 {
			emitted = append(emitted, hTok[b])
		}
		delete(dd.next, ids[b])
		if len(h.tokens) == 0 {
			continue
		}
		h.tokens = append(h.tokens, emitted...)
		if rows[b] == dd.scratchRow {
			continue
		}
		if int(h.devLen)+len(emitted) > dd.stride {
			h.devLen = -1
			continue
		}
		h.devLen += int32(len(emitted))
		nb := int(next[B*dd.k+b])
		dd.next[ids[b]] = nextDrafts{histLen: len(h.tokens), drafts: append([]int32(nil), next[b*dd.k:b*dd.k+nb]...)}
	}
}

// Drafts implements DraftSource: the drafts computed on the device at the end of the
// sequence's last step, when the engine's history has the length the runner's has.
func (r *Runner) Drafts(seqID uint64, histLen int) ([]int32, bool) {
	if r.drafts == nil {
		return nil, false
	}
	nd, ok := r.drafts.next[seqID]
	if !ok || nd.histLen != histLen {
		return nil, false
	}
	return nd.drafts, true
}
