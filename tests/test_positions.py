"""The device decision handed back as the engine's LogitsPerPosition (one-hot rows) and the
oracle's restatement of how emitSpeculative reads them. CPU only."""
import numpy as np
import pytest

from gollmgo_amd.positions import LogitsPerPosition


def test_emit_positions_reference_verify_cases(ora, golden):
    """The reference's Verify known answers over its own ragged rows (no padding)."""
    for c in golden["verify"]:
        d = np.array([c["drafts"]], np.int32).reshape(1, -1)
        acc, tok = ora.emit_positions(d, [len(c["drafts"])], [[np.array(r, np.float32) for r in c["rows"]]])
        assert acc[0] == c["expect_accepted"]
        if c["expect_corrected"] is not None:
            assert tok[0] == c["expect_corrected"]
        elif acc[0] == len(c["drafts"]):
            assert tok[0] == -1  # every draft accepted, no bonus row


def test_emit_positions_matches_dense_verify(ora):
    """Full-width rows, greedy: the same decisions as the dense Verify + argmax bonus."""
    rng = np.random.default_rng(3)
    B, K, V = 60, 4, 300
    lg = rng.normal(0, 2, (B, K + 1, V)).astype(np.float32)
    drafts = rng.integers(0, V, (B, K)).astype(np.int32)
    for b in range(B):
        for j in range(K):
            if rng.random() < 0.7:
                drafts[b, j] = int(np.argmax(lg[b, j]))
    n = rng.integers(0, K + 1, B).astype(np.int32)
    ea, et = ora.accept_greedy(lg, drafts, n)
    acc, tok = ora.emit_positions(drafts, n, [[lg[b, j] for j in range(K + 1)] for b in range(B)])
    assert np.array_equal(acc, ea) and np.array_equal(tok, et)


def random_decisions(rng, B, K, V):
    drafts = rng.integers(0, V, (B, K)).astype(np.int32)
    n = rng.integers(0, K + 1, B).astype(np.int32)
    acc = np.array([rng.integers(0, n[b] + 1) for b in range(B)], np.int32)
    tok = rng.integers(0, V, B).astype(np.int32)
    for b in range(B):
        while acc[b] < n[b] and tok[b] == drafts[b, acc[b]]:
            tok[b] = rng.integers(0, V)
    return drafts, n, acc, tok


@pytest.mark.parametrize("T,top_p", [(0.0, 1.0), (0.8, 1.0), (0.8, 0.95), (1.3, 0.5)])
def test_one_hot_rows_reproduce_the_decision(ora, T, top_p):
    rng = np.random.default_rng(int(T * 10 + top_p * 100))
    B, K, V = 300, 6, 5000
    drafts, n, acc, tok = random_decisions(rng, B, K, V)
    lpp = LogitsPerPosition(V)
    pos = lpp.batch(drafts, n, acc, tok)
    for b in range(B):
        assert len(pos[b]) == acc[b] + 1
        for j, row in enumerate(pos[b]):
            t = drafts[b, j] if j < acc[b] else tok[b]
            assert len(row) == t + 1 and row[t] == 0 and np.all(np.isneginf(row[:t]))
            assert np.shares_memory(row, pos[0][0])  # views of one buffer, nothing copied
    u = rng.random(B)
    ea, et = ora.emit_positions(drafts, n, pos, T, top_p, u)
    assert np.array_equal(ea, acc) and np.array_equal(et, tok)


def test_one_hot_row_extremes(ora):
    V = 128256
    lpp = LogitsPerPosition(V)
    for t in (0, 1, V - 1):
        r = lpp.row(t)
        assert len(r) == t + 1 and ora.argmax(r) == t
        assert ora.sample_f64(r, 0.8, 0.95, 0.999999) == t
        assert ora.sample_f64(r, 0.8, 0.95, 0.0) == t
    with pytest.raises(ValueError):
        lpp.row(V)
    with pytest.raises(ValueError):
        lpp.row(-1)
    assert not lpp.row(5).flags.writeable


def test_unrepresentable_decision_is_refused():
    lpp = LogitsPerPosition(100)
    with pytest.raises(ValueError):
        lpp.rows_for([7, 8], 2, 1, 8)  # rejected draft 8 returned as the token
    with pytest.raises(ValueError):
        lpp.rows_for([7, 8], 2, 3, 1)  # accepted beyond the drafts
    assert len(lpp.rows_for([7, 8], 2, 2, 8)) == 3  # all accepted: the bonus may repeat a draft
