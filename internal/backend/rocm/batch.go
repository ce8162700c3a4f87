// Package rocm is gollmgo's MI355X runner for the speculative verify step, over the C ABI
// of libgg_verify (include/gg_verify.h). The files belong at internal/backend/rocm in the
// gollmgo tree. They are not compiled in this repository (its image has no Go
// toolchain); gollmgo_amd/batch.py and gollmgo_amd/positions.py are the same functions in
// Python, and tests/test_runner_batch.py and tests/test_positions.py run them.
// batch_test.go and positions_test.go hold the Go side of those cases (positions_test.go
// reads the rows with the engine's own Verify and Sampler).
//
// batch.go and positions.go are plain Go (no cgo, no build tag); bridge.go and runner.go
// need the "rocm" build tag, cgo and the ROCm runtime.
package rocm

import (
	"fmt"

	"github.com/TensorGreed/gollmgo/internal/backend"
)

// StepInputs is the ABI's view of one verify step: rectangular per-sequence arrays.
type StepInputs struct {
	NumSeqs     int
	RowsPerSeq  int     // R: the largest token count (or the warmed-up maximum)
	MaxBlocks   int     // block-table row length
	Tokens      []int32 // [B][R], padding rows 0
	Positions   []int32 // [B][R], padding rows repeat the last position
	Slots       []int32 // [B*R] for gg_kv_append, padding rows -1 (skipped)
	CtxLens     []int32 // [B]
	RowCounts   []int32 // [B]
	BlockTables []int32 // [B][MaxBlocks], padding -1
	Drafts      []int32 // [B][R-1], padding 0
	NDrafts     []int32 // [B]
}

// PackBatch maps a decode batch (backend.Batch, internal/backend/runner.go:29-54) onto
// the ABI's arrays. Sequence i owns SeqTokenCounts[i] consecutive entries of the
// flattened TokenIDs / Positions / SlotMapping (current token, then its drafts). Block b
// of a sequence is SeqSlotTables[i][b*bs] / bs: the KV manager allocates whole blocks and
// fills them in order (internal/kvcache/block_table.go:24-42). maxBlocks / rowsPerSeq are
// the shapes fixed at warm-up (0 = the batch's own). Prefill sequences are refused.
func PackBatch(batch *backend.Batch, bs, maxBlocks, rowsPerSeq int) (*StepInputs, error) {
	B := len(batch.SequenceIDs)
	if B == 0 {
		return nil, fmt.Errorf("rocm: empty batch")
	}
	for _, p := range batch.IsPrefill {
		if p {
			return nil, fmt.Errorf("rocm: prefill sequences go to the model's prefill path")
		}
	}
	if len(batch.SeqTokenCounts) != B || len(batch.SeqContextLens) != B || len(batch.SeqSlotTables) != B {
		return nil, fmt.Errorf("rocm: per-sequence fields disagree with SequenceIDs")
	}
	nTok, R := 0, 0
	for _, c := range batch.SeqTokenCounts {
		if c < 1 {
			return nil, fmt.Errorf("rocm: a decode sequence has at least its current token")
		}
		nTok += int(c)
		if int(c) > R {
			R = int(c)
		}
	}
	if len(batch.TokenIDs) != nTok || len(batch.Positions) != nTok || len(batch.SlotMapping) != nTok {
		return nil, fmt.Errorf("rocm: flattened token fields disagree with SeqTokenCounts")
	}
	if rowsPerSeq > 0 {
		if R > rowsPerSeq {
			return nil, fmt.Errorf("rocm: %d rows exceed the warmed-up %d", R, rowsPerSeq)
		}
		R = rowsPerSeq
	}
	K := R - 1
	drafts := batch.DraftTokens
	if len(drafts) == 0 {
		drafts = make([][]int32, B)
	}
	if len(drafts) != B {
		return nil, fmt.Errorf("rocm: DraftTokens disagrees with SequenceIDs")
	}
	need := 0
	for _, L := range batch.SeqContextLens {
		if nb := (int(L) + bs - 1) / bs; nb > need {
			need = nb
		}
	}
	MB := maxBlocks
	if MB == 0 {
		MB = need
		if MB < 1 {
			MB = 1
		}
	}
	if need > MB {
		return nil, fmt.Errorf("rocm: %d blocks exceed the warmed-up %d", need, MB)
	}

	in := &StepInputs{
		NumSeqs: B, RowsPerSeq: R, MaxBlocks: MB,
		Tokens: make([]int32, B*R), Positions: make([]int32, B*R), Slots: make([]int32, B*R),
		CtxLens: make([]int32, B), RowCounts: make([]int32, B), BlockTables: make([]int32, B*MB),
		Drafts: make([]int32, B*K), NDrafts: make([]int32, B),
	}
	for i := range in.Slots {
		in.Slots[i] = -1
	}
	for i := range in.BlockTables {
		in.BlockTables[i] = -1
	}
	t0 := 0
	for i := 0; i < B; i++ {
		c := int(batch.SeqTokenCounts[i])
		d := drafts[i]
		if len(d) != c-1 {
			return nil, fmt.Errorf("rocm: sequence %d: %d tokens but %d drafts", i, c, len(d))
		}
		for j := 1; j < c; j++ {
			if batch.TokenIDs[t0+j] != d[j-1] {
				return nil, fmt.Errorf("rocm: sequence %d: the tokens after the current one are not its drafts", i)
			}
		}
		for j := 0; j < R; j++ {
			if j < c {
				in.Tokens[i*R+j] = batch.TokenIDs[t0+j]
				in.Positions[i*R+j] = batch.Positions[t0+j]
				in.Slots[i*R+j] = batch.SlotMapping[t0+j]
			} else {
				in.Positions[i*R+j] = batch.Positions[t0+c-1]
			}
		}
		t0 += c
		L := int(batch.SeqContextLens[i])
		st := batch.SeqSlotTables[i]
		if L < c || len(st) != L {
			return nil, fmt.Errorf("rocm: sequence %d: context %d with a slot table of %d and %d rows", i, L, len(st), c)
		}
		for b := 0; b < (L+bs-1)/bs; b++ {
			s0 := int(st[b*bs])
			if s0 < 0 || s0%bs != 0 {
				return nil, fmt.Errorf("rocm: sequence %d: block %d starts at slot %d, not a block boundary", i, b, s0)
			}
			in.BlockTables[i*MB+b] = int32(s0 / bs)
		}
		for j := 0; j < c; j++ {
			if st[L-c+j] != in.Slots[i*R+j] {
				return nil, fmt.Errorf("rocm: sequence %d: SlotMapping of row %d is not its slot-table entry", i, j)
			}
		}
		in.CtxLens[i] = int32(L)
		in.RowCounts[i] = int32(c)
		copy(in.Drafts[i*K:i*K+c-1], d)
		in.NDrafts[i] = int32(c - 1)
	}
	if err := CheckBlockRuns(in.Slots, bs); err != nil {
		return nil, err
	}
	return in, nil
}

// CheckBlockRuns enforces gg_kv_append's rule for PER_BLOCK pools: the rows of one block
// are adjacent in the slot mapping (skipped rows, slot < 0, may sit between them) with
// increasing offsets. A block that reappears after another block's rows would get two
// leaders on the device.
func CheckBlockRuns(slots []int32, bs int) error {
	seen := map[int]bool{}
	cur, lastOff := -1, -1
	for _, s := range slots {
		if s < 0 {
			continue
		}
		blk, off := int(s)/bs, int(s)%bs
		if blk != cur {
			if seen[blk] {
				return fmt.Errorf("rocm: block %d appears in two separate runs of the slot mapping", blk)
			}
			seen[blk] = true
			cur, lastOff = blk, -1
		}
		if off <= lastOff {
			return fmt.Errorf("rocm: block %d: offsets not increasing in the slot mapping", blk)
		}
		lastOff = off
	}
	return nil
}
