"""The drafter / acceptance restatement, pinned by brute force, known
answers and the speculative == plain greedy invariant."""

import random

from oracle.spec_oracle import accept, ngram_draft, plain_greedy, speculative_greedy


def brute_draft(hist, L, n, k):
    """Every start j whose n tokens equal the last n and whose k-token
    continuation ends at or before L; the most recent wins."""
    pat = hist[L - n + 1:L + 1] if L - n + 1 >= 0 else None
    best = -1
    for j in range(len(hist)):
        if pat is None or j + n + k - 1 > L:
            continue
        if hist[j:j + n] == pat:
            best = j
    return best


def test_known_answers():
    #        0  1  2  3  4  5  6  7  8  9 10 11
    hist = [5, 6, 7, 8, 9, 5, 6, 7, 1, 2, 5, 6, 7, 0, 0, 0, 0, 0, 0, 0]
    L = 12  # current token hist[12] = 7, pattern (3-gram) = 5 6 7
    ids, d = ngram_draft(hist, L, 3, 2, 3)
    # matches at 0 and 5; the most recent with a complete continuation is 5
    assert d == [1, 2, 5] and ids == [7, 1, 2, 5]
    # k too long for the start at 5 -> falls back to the start at 0
    ids, d = ngram_draft(hist, L, 3, 2, 5)
    assert d == [1, 2, 5, 6, 7]  # continuation ends exactly at L: still complete
    ids, d = ngram_draft(hist, L, 3, 2, 6)
    assert d == [8, 9, 5, 6, 7, 1]
    # no 3-gram, but a 2-gram: pattern "6 9" absent; "x 9"...
    h2 = [1, 2, 3, 4, 2, 3, 0, 0, 0, 0]
    ids, d = ngram_draft(h2, 5, 3, 2, 1)  # 3-gram 4 2 3 absent; 2-gram 2 3 at 1 -> cont 4
    assert d == [4]
    # nothing matches -> zero draft
    h3 = [1, 2, 3, 4, 5, 6, 0, 0]
    ids, d = ngram_draft(h3, 5, 3, 2, 4)
    assert d == [0, 0, 0, 0] and ids == [6, 0, 0, 0, 0]
    # short history: pattern indices clamp at 0 and never read before the row
    ids, d = ngram_draft([9, 0, 0, 0], 0, 3, 2, 2)
    assert ids[0] == 9 and d == [0, 0]


def test_draft_matches_brute_force():
    rng = random.Random(7)
    for _ in range(300):
        cap = rng.randint(8, 40)
        hist = [rng.randint(0, 3) for _ in range(cap)]
        L = rng.randint(0, cap - 1)
        k = rng.randint(1, 5)
        ids, d = ngram_draft(hist, L, 3, 2, k)
        bp = brute_draft(hist, L, 3, k)
        bb = brute_draft(hist, L, 2, k)
        best, n = (bp, 3) if bp >= 0 else (bb, 2)
        exp = [hist[best + n + t] for t in range(k)] if best >= 0 else [0] * k
        assert d == exp and ids == [hist[L]] + exp


def test_accept_known_answers():
    hist = list(range(10)) + [0] * 10
    a, L = accept([7, 8, 9, 4], [7, 8, 1], hist, 9, 3, stop_len=100)
    assert a == 2 and L == 12 and hist[10:13] == [7, 8, 9] and hist[13] == 0
    hist = [0] * 10
    a, L = accept([3, 4], [5], hist, 4, 1, stop_len=100)
    assert a == 0 and L == 5 and hist[5] == 3 and hist[6] == 0
    # frozen sequence: nothing written, length kept
    hist = [0] * 10
    a, L = accept([3, 4], [3], hist, 6, 1, stop_len=6)
    assert a == 0 and L == 6 and hist == [0] * 10
    # bounded by the history length
    hist = [0] * 6
    a, L = accept([1, 2, 3], [1, 2], hist, 3, 2, stop_len=100)
    assert a == 2 and L == 6 and hist[4:6] == [1, 2]


def test_speculative_equals_plain_greedy():
    rng = random.Random(11)
    table = {}

    def next_token(prefix):
        # deterministic toy model with long-range structure: repeats motifs
        key = tuple(prefix[-3:])
        if key not in table:
            table[key] = rng.randint(0, 6)
        return table[key]

    for trial in range(20):
        prompt = [rng.randint(0, 6) for _ in range(rng.randint(4, 30))]
        n = rng.randint(1, 40)
        want = plain_greedy(next_token, prompt, n)
        got, iters = speculative_greedy(next_token, prompt, n, k=rng.randint(1, 8))
        assert got == want
        assert iters <= max(n - 1, 0)
