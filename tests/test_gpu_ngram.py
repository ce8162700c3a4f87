"""GPU parity: n-gram draft lookup against the oracle (hash-map restatement of
NGramDrafter.Draft) and the reference's known answers."""
import numpy as np
import pytest
import torch

import gollmgo_amd.verify as gv
from gollmgo_amd.workloads import CONFIGS, make_histories, scaled
from helpers import say
from oracle import oracle as ora

pytestmark = pytest.mark.gpu


def run(hist_list, n, k):
    B = len(hist_list)
    stride = max(1, max(len(h) for h in hist_list))
    h = np.zeros((B, stride), np.int32)
    lens = np.zeros(B, np.int32)
    for b, x in enumerate(hist_list):
        h[b, :len(x)] = x
        lens[b] = len(x)
    d, nn = gv.ngram_draft(torch.from_numpy(h).cuda(), torch.from_numpy(lens).cuda(), n, k)
    torch.cuda.synchronize()
    d, nn = d.cpu().numpy(), nn.cpu().numpy()
    return [d[b, :nn[b]].tolist() for b in range(B)]


def test_ngram_reference_cases(gpu, golden):
    say("ngram reference cases")
    cases = golden["ngram_draft"]
    got = run([c["history"] for c in cases], 3, 4)
    assert got == [c["expect"] for c in cases]


@pytest.mark.parametrize("n", [2, 3, 5, 9])
@pytest.mark.parametrize("k", [0, 1, 5, 8])
def test_ngram_random_small_alphabet(gpu, n, k):
    say(f"ngram random n={n} k={k}")
    rng = np.random.default_rng(n * 10 + k)
    hists = [rng.integers(0, 4, int(rng.integers(0, 200))).tolist() for _ in range(40)]
    got = run(hists, n, k)
    want = [ora.ngram_draft(h, n, k) for h in hists]
    assert got == want


def test_ngram_config5_histories(gpu):
    """Config-5 shape: 8192-token histories with 40% injected repeats (scaled batch)."""
    say("ngram config5 histories")
    cfg = scaled(CONFIGS[5], num_seqs=16)
    h = make_histories(cfg, cfg.history_len)
    got = run([row.tolist() for row in h], cfg.ngram_n, cfg.max_drafts)
    want = [ora.ngram_draft(row, cfg.ngram_n, cfg.max_drafts) for row in h]
    assert got == want


def test_ngram_long_history_crosses_tiles(gpu):
    say("ngram long history")
    rng = np.random.default_rng(77)
    h = rng.integers(0, 50000, 20000).tolist()
    h[100:103] = [1, 2, 3]
    h[-2:] = [1, 2]     # the only match is far from the end (several LDS tiles back)
    assert run([h], 3, 3) == [ora.ngram_draft(h, 3, 3)]


@pytest.mark.parametrize("seed", range(12))
def test_ngram_random_mixed(gpu, seed):
    """Seeded batches mixing history lengths on both sides of the LDS-resident limit
    (12288 tokens) and past the tile width, small alphabets (many matches, so chained
    lookups run long) and large ones, odd row strides (unaligned rows), n = 2..9."""
    r = np.random.default_rng(900 + seed)
    n = int(r.integers(2, 10))
    k = int(r.integers(0, 9))
    B = int(r.integers(1, 12))
    alphabet = int(r.choice([2, 5, 50, 32000]))
    lens = [int(r.choice([0, 1, n - 1, n, int(r.integers(0, 4000)), 12287, 12288, 12289, int(r.integers(12289, 30000))]))
            for _ in range(B)]
    hists = []
    for L in lens:
        h = r.integers(0, alphabet, L)
        if L > 2 * n and r.random() < 0.5:  # plant the final key far back in the history
            pos = int(r.integers(0, L - 2 * n))
            h[pos:pos + n - 1] = h[L - (n - 1):]
        hists.append(h.tolist())
    stride = max(1, max(lens)) + int(r.integers(0, 3))  # 1 or 2 extra: rows not 16-byte aligned
    say(f"ngram random case {seed}: n={n} k={k} lens={lens} alphabet={alphabet} stride={stride}")
    h = np.zeros((B, stride), np.int32)
    ln = np.zeros(B, np.int32)
    for b, x in enumerate(hists):
        h[b, :len(x)] = x
        ln[b] = len(x)
    d, nn = gv.ngram_draft(torch.from_numpy(h).cuda(), torch.from_numpy(ln).cuda(), n, k)
    torch.cuda.synchronize()
    d, nn = d.cpu().numpy(), nn.cpu().numpy()
    got = [d[b, :nn[b]].tolist() for b in range(B)]
    want = [ora.ngram_draft(x, n, k) for x in hists]
    assert got == want


# ------------------------------------------------- history append + next drafts (one launch)

def _emit(drafts_b, acc, tok):
    """emitSpeculative's emitted tokens (internal/engine/serving.go:541-566): the accepted
    drafts, then the corrected or bonus token (none when the device had no mass, tok < 0)."""
    return list(drafts_b[:acc]) + ([int(tok)] if tok >= 0 else [])


@pytest.mark.parametrize("seed", range(6))
def test_history_append_draft_matches_host_drafter(gpu, seed):
    """gg_history_append_draft against the host flow it replaces: the emitted tokens
    appended to each sequence's history, then NGramDrafter.Draft over the whole history.
    Histories live in rows of a larger pool (hist_rows maps sequences to rows, unused rows
    untouched), lengths on both sides of the LDS-resident limit, some rows full enough to
    overflow (left unchanged, length -1, no drafts), a negative length staying -1, and two
    steps in a row, the second drafting from the first one's output."""
    r = np.random.default_rng(1300 + seed)
    n = int(r.integers(2, 6))
    k_in = int(r.integers(0, 7))
    k = int(r.integers(1, 7))
    rows_total, B = 24, int(r.integers(1, 16))
    alphabet = int(r.choice([3, 7, 50]))
    stride = int(r.choice([64, 3000, 13000]))
    pool = np.zeros((rows_total, stride), np.int32)
    lens = np.zeros(rows_total, np.int32)
    for row in range(rows_total):
        L = int(r.integers(0, stride + 1))
        if r.random() < 0.2:
            L = stride - int(r.integers(0, 3))  # about to overflow
        pool[row, :L] = r.integers(0, alphabet, L)
        lens[row] = L
    lens[int(r.integers(0, rows_total))] = -1
    hist_rows = r.permutation(rows_total)[:B].astype(np.int32)
    dev_pool, dev_lens = torch.from_numpy(pool).cuda(), torch.from_numpy(lens).cuda()
    host = [pool[row, :max(lens[row], 0)].tolist() if lens[row] >= 0 else None for row in range(rows_total)]
    drafts = r.integers(0, alphabet, (B, k_in)).astype(np.int32)
    for step in range(2):
        acc = np.array([int(r.integers(0, k_in + 1)) for _ in range(B)], np.int32)
        tok = r.integers(-1, alphabet, B).astype(np.int32)
        say(f"history append+draft seed {seed} step {step}: n={n} k_in={k_in} k={k} B={B} stride={stride}")
        d, nn = gv.history_append_draft(dev_pool, dev_lens, torch.from_numpy(drafts).cuda(),
                                        torch.from_numpy(acc).cuda(), torch.from_numpy(tok).cuda(), n, k,
                                        hist_rows=torch.from_numpy(hist_rows).cuda())
        torch.cuda.synchronize()
        d, nn = d.cpu().numpy(), nn.cpu().numpy()
        for b in range(B):
            row = int(hist_rows[b])
            emitted = _emit(drafts[b], int(acc[b]), int(tok[b]))
            if host[row] is None or len(host[row]) + len(emitted) > stride:
                host[row] = None
                assert nn[b] == 0
                continue
            host[row] = host[row] + emitted
            assert d[b, :nn[b]].tolist() == ora.ngram_draft(host[row], n, k), (b, row)
        got_lens = dev_lens.cpu().numpy()
        got_pool = dev_pool.cpu().numpy()
        for row in range(rows_total):
            if host[row] is None:
                assert got_lens[row] == -1
            else:
                assert got_lens[row] == len(host[row])
                assert got_pool[row, :len(host[row])].tolist() == host[row]
        # The next step verifies this step's drafts (padded to k_in with zeros).
        nd = np.zeros((B, k_in), np.int32)
        for b in range(B):
            m = min(int(nn[b]), k_in)
            nd[b, :m] = d[b, :m]
        drafts = nd


def test_history_append_draft_identity_rows(gpu):
    """hist_rows NULL: sequence b is row b; a sequence with nothing accepted and no token
    appends nothing and drafts from its history as gg_ngram_draft does."""
    say("history append+draft identity rows")
    h = np.array([[1, 2, 3, 1, 2, 0, 0, 0], [5, 5, 5, 5, 0, 0, 0, 0]], np.int32)
    ln = np.array([5, 4], np.int32)
    drafts = np.array([[3, 9], [7, 7]], np.int32)
    acc = np.array([1, 0], np.int32)
    tok = np.array([1, -1], np.int32)
    hp, lp = torch.from_numpy(h).cuda(), torch.from_numpy(ln).cuda()
    d, nn = gv.history_append_draft(hp, lp, torch.from_numpy(drafts).cuda(), torch.from_numpy(acc).cuda(),
                                    torch.from_numpy(tok).cuda(), 3, 4)
    torch.cuda.synchronize()
    assert lp.cpu().tolist() == [7, 4]
    assert hp.cpu().numpy()[0, :7].tolist() == [1, 2, 3, 1, 2, 3, 1]
    d, nn = d.cpu().numpy(), nn.cpu().numpy()
    assert d[0, :nn[0]].tolist() == ora.ngram_draft([1, 2, 3, 1, 2, 3, 1], 3, 4)
    assert d[1, :nn[1]].tolist() == ora.ngram_draft([5, 5, 5, 5], 3, 4)


def test_device_drafter_serves_the_engine_drafts(gpu):
    """The runner-side device drafting flow (gollmgo_amd/drafting.py, the twin of the Go
    runner's drafts.go) driven by a simulated engine over many steps: prompts recorded at
    prefill (one sequence chunked, one never seen), each step's current token, the device
    decision's emitted tokens, fewer device rows than sequences (eviction and reseeding),
    and a sequence rolled back by two tokens. Whenever the runner answers
    Drafts(seq, len(history)), its drafts equal NGramDrafter.Draft over the engine's
    history (the oracle's restatement); otherwise the engine drafts on the host."""
    from gollmgo_amd.drafting import DeviceDrafter
    say("device drafter flow")
    r = np.random.default_rng(77)
    n, K, alphabet = 3, 4, 6
    S = 10
    dd = DeviceDrafter(n, K, stride=600, rows=6, max_batch=S)
    hist = {}
    for sid in range(S):
        prompt = r.integers(0, alphabet, int(r.integers(5, 60))).tolist()
        hist[sid] = prompt
        if sid == 9:
            continue  # the runner never sees this prefill: host drafts only
        if sid == 3:  # chunked prefill
            h = len(prompt) // 2
            dd.prefill([sid], [prompt[:h]], [list(range(h))])
            dd.prefill([sid], [prompt[h:]], [list(range(h, len(prompt)))])
        else:
            dd.prefill([sid], [prompt], [list(range(len(prompt)))])
        hist[sid].append(int(r.integers(0, alphabet)))  # the token sampled from the prefill logits
    hist[9].append(int(r.integers(0, alphabet)))
    device_answers = 0
    for step in range(40):
        active = sorted(r.choice(S, size=int(r.integers(3, 9)), replace=False).tolist())
        if step == 20:
            hist[active[0]] = hist[active[0]][:-2]  # a rollback: the runner's mirror diverges
        drafts = np.zeros((len(active), K), np.int32)
        nd = np.zeros(len(active), np.int32)
        for b, sid in enumerate(active):
            want = ora.ngram_draft(hist[sid], n, K)
            got = dd.drafts(sid, len(hist[sid]))
            if got is not None:
                assert got == want, (step, sid)
                device_answers += 1
            d = got if got is not None else want
            drafts[b, :len(d)] = d
            nd[b] = len(d)
        cur = [hist[sid][-1] for sid in active]
        pos = [len(hist[sid]) - 1 for sid in active]
        rows = dd.prepare(active, cur, pos)
        acc = np.array([int(r.integers(0, nd[b] + 1)) for b in range(len(active))], np.int32)
        tok = r.integers(0, alphabet, len(active)).astype(np.int32)
        next_d, next_n = dd.launch(rows, torch.from_numpy(drafts).cuda(), torch.from_numpy(acc).cuda(),
                                   torch.from_numpy(tok).cuda())
        torch.cuda.synchronize()
        dd.finish(active, rows, drafts, nd, acc, tok, next_d.cpu().numpy(), next_n.cpu().numpy())
        for b, sid in enumerate(active):  # emitSpeculative
            hist[sid] = hist[sid] + drafts[b, :acc[b]].tolist() + [int(tok[b])]
    print(f"  device answers: {device_answers}")
    assert device_answers > 40
    assert dd.drafts(9, len(hist[9])) is None
