package rocm

import (
	"fmt"
	"math"
)

// OneHotRows hands the device's verify decision back to the engine as
// StepOutput.LogitsPerPosition. The engine reads those rows with its own Verify
// (internal/engine/speculative.go:68-84) and, after the last draft, Sampler.Sample
// (internal/engine/serving.go:556-566); the rows make both return the device decision:
//
//	row j < accepted   one-hot at drafts[j]  (argmax == draft: accepted)
//	row accepted       one-hot at token      (argmax == token != draft: corrected;
//	                                          after the last draft, Sample -> token)
//
// The row of token t is the shortest legal one, as the mock runner's ragged rows are
// (internal/backend/mock_runner.go:44-61): length t+1, -Inf before t and 0 at t. argmax
// gives t, and softmax maps -Inf to 0 (internal/engine/sampling.go:112-136), so every
// temperature, top-k or top-p returns t. All rows are subslices of one constant buffer
// (row t = base[V-t:]): nothing is allocated or copied per step, and Verify and Sample
// only read their rows.
type OneHotRows struct {
	base  []float32 // V times -Inf, then 0
	vocab int
}

func NewOneHotRows(vocab int) *OneHotRows {
	base := make([]float32, vocab+1)
	for i := 0; i < vocab; i++ {
		base[i] = float32(math.Inf(-1))
	}
	return &OneHotRows{base: base, vocab: vocab}
}

// Row is the row whose argmax and every sample is tok.
func (o *OneHotRows) Row(tok int32) ([]float32, error) {
	if tok < 0 || int(tok) >= o.vocab {
		return nil, fmt.Errorf("rocm: token %d outside [0, %d)", tok, o.vocab)
	}
	return o.base[o.vocab-int(tok) : o.vocab+1 : o.vocab+1], nil
}

// RowsFor is one sequence's LogitsPerPosition: accepted+1 rows. A token equal to the
// draft it replaces cannot be expressed (Verify would accept it); the device never
// returns one (a greedy correction differs from the draft by definition, and the
// rejection sampler's residual is 0 at the rejected draft), so it is an error here.
func (o *OneHotRows) RowsFor(drafts []int32, accepted int, tok int32) ([][]float32, error) {
	if accepted < 0 || accepted > len(drafts) {
		return nil, fmt.Errorf("rocm: accepted %d outside [0, %d]", accepted, len(drafts))
	}
	if accepted < len(drafts) && drafts[accepted] == tok {
		return nil, fmt.Errorf("rocm: the token after a rejected draft equals that draft")
	}
	rows := make([][]float32, accepted+1)
	for j := 0; j <= accepted; j++ {
		t := tok
		if j < accepted {
			t = drafts[j]
		}
		r, err := o.Row(t)
		if err != nil {
			return nil, err
		}
		rows[j] = r
	}
	return rows, nil
}
