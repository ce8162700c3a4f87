package rocm

import (
	"math"
	"math/rand"
	"testing"

	"github.com/TensorGreed/gollmgo/internal/engine"
)

func TestOneHotRowShape(t *testing.T) {
	o := NewOneHotRows(1000)
	for _, tok := range []int32{0, 1, 999} {
		r, err := o.Row(tok)
		if err != nil {
			t.Fatal(err)
		}
		if len(r) != int(tok)+1 || r[tok] != 0 {
			t.Fatalf("row %d: len %d", tok, len(r))
		}
		for i := 0; i < int(tok); i++ {
			if !math.IsInf(float64(r[i]), -1) {
				t.Fatalf("row %d: element %d is %v", tok, i, r[i])
			}
		}
	}
	if _, err := o.Row(1000); err == nil {
		t.Fatal("token past the vocabulary: accepted")
	}
	if _, err := o.RowsFor([]int32{7, 8}, 1, 8); err == nil {
		t.Fatal("the rejected draft as the token: accepted")
	}
}

// The engine's own reading of the rows (emitSpeculative, internal/engine/serving.go:496-570)
// gives back the decision the rows were built from, for the greedy Verify and for
// samplers with temperature, top-p and top-k on the bonus row. tests/test_positions.py checks the
// same property through the oracle's restatement of Verify and Sample.
func TestOneHotRowsReproduceTheDecision(t *testing.T) {
	const V, K = 5000, 6
	o := NewOneHotRows(V)
	rng := rand.New(rand.NewSource(1))
	seed := uint64(3)
	samplers := []*engine.Sampler{
		engine.NewSampler(engine.SamplingParams{Temperature: 0}),
		engine.NewSampler(engine.SamplingParams{Temperature: 0.8, TopP: 0.95, Seed: &seed}),
		engine.NewSampler(engine.SamplingParams{Temperature: 1.3, TopK: 40, Seed: &seed}),
	}
	for trial := 0; trial < 2000; trial++ {
		n := rng.Intn(K + 1)
		drafts := make([]int32, n)
		for j := range drafts {
			drafts[j] = int32(rng.Intn(V))
		}
		acc := rng.Intn(n + 1)
		tok := int32(rng.Intn(V))
		for acc < n && tok == drafts[acc] {
			tok = int32(rng.Intn(V))
		}
		rows, err := o.RowsFor(drafts, acc, tok)
		if err != nil {
			t.Fatal(err)
		}
		for _, s := range samplers {
			draftRows := rows
			if len(draftRows) > n {
				draftRows = draftRows[:n]
			}
			gotAcc, corrected := engine.Verify(drafts, draftRows)
			var got int32
			switch {
			case n == 0:
				got = s.Sample(rows[0])
			case gotAcc < n:
				got = corrected
			default:
				got = s.Sample(rows[n])
			}
			if gotAcc != acc || got != tok {
				t.Fatalf("trial %d: drafts %v decision (%d, %d), engine read (%d, %d)", trial, drafts, acc, tok,
					gotAcc, got)
			}
		}
	}
}
