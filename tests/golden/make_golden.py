"""Writes tests/golden/reference_cases.json: the known-answer cases of the
reference's own Go tests for this path, as data (inputs and expected outputs).

Sources (read as text, nothing imported or run):
  internal/engine/speculative_test.go:5-92   NGramDrafter.Draft and Verify cases
  internal/engine/sampling_test.go:8-24       argmax cases
  internal/engine/sampling_test.go:77-97      topPFilter case
  internal/engine/sampling_test.go:99-130     softmax cases
  internal/kvcache/block_table_test.go:5-140  BlockTable append / truncate / free cases
"""
import json
from pathlib import Path


def one_hot_row(n, idx, val=5.0):
    r = [0.0] * n
    r[idx] = val
    return r


cases = {
    "ngram_draft": [
        {"n": 3, "k": 4, "history": [10, 20, 30, 40, 10, 50], "expect": []},
        {"n": 3, "k": 4, "history": [1, 2, 3, 1, 2, 3, 1, 2, 3], "expect": [1, 2, 3, 1]},
        {"n": 3, "k": 4, "history": [1], "expect": []},
    ],
    "verify": [
        # TestVerifyAllAccepted: rows of lengths 11, 21, 31 with the 5 at the draft index.
        {"drafts": [10, 20, 30], "rows": [one_hot_row(11, 10), one_hot_row(21, 20), one_hot_row(31, 30)],
         "expect_accepted": 3, "expect_corrected": None},
        # TestVerifyPartialAccept
        {"drafts": [10, 20, 30], "rows": [one_hot_row(32, 10), one_hot_row(32, 25)],
         "expect_accepted": 1, "expect_corrected": 25},
        # TestVerifyNoDrafts
        {"drafts": [], "rows": [], "expect_accepted": 0, "expect_corrected": None},
    ],
    "argmax": [
        {"logits": [1, 3, 2], "expect": 1},
        {"logits": [5], "expect": 0},
        {"logits": [-1, -2, -0.5], "expect": 2},
        {"logits": [0, 0, 0, 1], "expect": 3},
    ],
    "greedy_sample": [{"logits": [0.1, 0.9, 0.5, 0.3], "expect": 1}],
    "top_p": [{"probs": [0.5, 0.3, 0.1, 0.05, 0.05], "p": 0.8, "kept": [0, 1], "sum": 1.0, "tol": 1e-6}],
    "softmax": [
        {"logits": [1.0, 2.0, 3.0], "sum": 1.0, "tol": 1e-9, "increasing": True},
        {"logits": [1.0, "-inf", 2.0], "sum": 1.0, "tol": 1e-9, "zero_at": 1},
    ],
    "block_table": [
        {"pool": 100, "bs": 4, "append": 6, "num_tokens": 6, "num_blocks": 2},
        {"pool": 100, "bs": 4, "append": 10, "num_blocks": 3},
        {"pool": 10, "bs": 4, "append": 8, "free_after_append": 8, "free_after_free": 10},
        {"pool": 2, "bs": 4, "append": 8, "then_append_fails": True},
        {"pool": 10, "bs": 4, "append": 6, "truncate": 2, "num_tokens": 4, "num_blocks": 1, "free": 9},
        {"pool": 10, "bs": 4, "append": 0, "truncate": 5, "num_tokens": 0},
    ],
}

if __name__ == "__main__":
    out = Path(__file__).with_name("reference_cases.json")
    out.write_text(json.dumps(cases, indent=1))
    print(f"wrote {out}")
