package rocm

import (
	"strings"
	"testing"

	"github.com/TensorGreed/gollmgo/internal/backend"
)

// Two decode sequences with block size 4, built the way the engine builds them:
// sequence 0 has 5 cached tokens in blocks 7 and 3 and verifies its current token and two
// drafts (positions 5..7), sequence 1 has 2 cached tokens in block 5 and no drafts.
// The same case is tests/test_runner_batch.py's engine_step in miniature.
func twoSeqBatch() *backend.Batch {
	return &backend.Batch{
		SequenceIDs:    []uint64{10, 11},
		TokenIDs:       []int32{100, 41, 42, 200},
		Positions:      []int32{5, 6, 7, 2},
		SlotMapping:    []int32{13, 14, 15, 22},
		IsPrefill:      []bool{false, false},
		SeqTokenCounts: []int32{3, 1},
		SeqContextLens: []int32{8, 3},
		SeqSlotTables:  [][]int32{{28, 29, 30, 31, 12, 13, 14, 15}, {20, 21, 22}},
		DraftTokens:    [][]int32{{41, 42}, {}},
	}
}

func eq(t *testing.T, what string, got, want []int32) {
	t.Helper()
	if len(got) != len(want) {
		t.Fatalf("%s: %v, want %v", what, got, want)
	}
	for i := range got {
		if got[i] != want[i] {
			t.Fatalf("%s: %v, want %v", what, got, want)
		}
	}
}

func TestPackBatch(t *testing.T) {
	in, err := PackBatch(twoSeqBatch(), 4, 0, 0)
	if err != nil {
		t.Fatal(err)
	}
	if in.NumSeqs != 2 || in.RowsPerSeq != 3 || in.MaxBlocks != 2 {
		t.Fatalf("shape %d %d %d", in.NumSeqs, in.RowsPerSeq, in.MaxBlocks)
	}
	eq(t, "tokens", in.Tokens, []int32{100, 41, 42, 200, 0, 0})
	eq(t, "positions", in.Positions, []int32{5, 6, 7, 2, 2, 2})
	eq(t, "slots", in.Slots, []int32{13, 14, 15, 22, -1, -1})
	eq(t, "ctx", in.CtxLens, []int32{8, 3})
	eq(t, "rows", in.RowCounts, []int32{3, 1})
	eq(t, "tables", in.BlockTables, []int32{7, 3, 5, -1})
	eq(t, "drafts", in.Drafts, []int32{41, 42, 0, 0})
	eq(t, "n_drafts", in.NDrafts, []int32{2, 0})
}

func TestPackBatchWarmedUpShape(t *testing.T) {
	in, err := PackBatch(twoSeqBatch(), 4, 5, 6)
	if err != nil {
		t.Fatal(err)
	}
	if in.RowsPerSeq != 6 || in.MaxBlocks != 5 || len(in.Drafts) != 2*5 {
		t.Fatalf("shape %d %d %d", in.RowsPerSeq, in.MaxBlocks, len(in.Drafts))
	}
	if _, err := PackBatch(twoSeqBatch(), 4, 1, 0); err == nil {
		t.Fatal("more blocks than warmed up: accepted")
	}
	if _, err := PackBatch(twoSeqBatch(), 4, 0, 2); err == nil {
		t.Fatal("more rows than warmed up: accepted")
	}
}

func TestPackBatchRefusesInconsistentBatches(t *testing.T) {
	cases := map[string]func(b *backend.Batch){
		"prefill":         func(b *backend.Batch) { b.IsPrefill[1] = true },
		"drafts":          func(b *backend.Batch) { b.DraftTokens[0] = []int32{41} },
		"draft tokens":    func(b *backend.Batch) { b.TokenIDs[2] = 7 },
		"slot mapping":    func(b *backend.Batch) { b.SlotMapping[1] = 30 },
		"block boundary":  func(b *backend.Batch) { b.SeqSlotTables[0][4] = 13 },
		"context length":  func(b *backend.Batch) { b.SeqContextLens[1] = 4 },
		"token counts":    func(b *backend.Batch) { b.SeqTokenCounts[1] = 2 },
	}
	for name, mutate := range cases {
		b := twoSeqBatch()
		mutate(b)
		if _, err := PackBatch(b, 4, 0, 0); err == nil {
			t.Errorf("%s: accepted", name)
		} else if !strings.HasPrefix(err.Error(), "rocm: ") {
			t.Errorf("%s: %v", name, err)
		}
	}
}

func TestCheckBlockRuns(t *testing.T) {
	if err := CheckBlockRuns([]int32{32, 33, -1, 34, 16, 17, 48}, 16); err != nil {
		t.Fatal(err)
	}
	if err := CheckBlockRuns([]int32{32, 33, 16, 34}, 16); err == nil {
		t.Fatal("a block in two runs: accepted")
	}
	if err := CheckBlockRuns([]int32{33, 32}, 16); err == nil {
		t.Fatal("decreasing offsets: accepted")
	}
}
