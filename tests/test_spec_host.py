"""The host side of speculative decoding, without a GPU: the n-gram index the
acceptance gate uses restates the device drafter exactly, and the predictor
scores every position with the acceptance a verify iteration would have had."""

import random

from oracle.spec_oracle import accept, ngram_draft
from qdec.spec import AcceptancePredictor, NgramIndex


def test_ngram_index_equals_drafter_on_random_histories():
    rng = random.Random(0)
    for _ in range(400):
        n = rng.randint(1, 70)
        hist = [rng.randint(0, 4) for _ in range(n)]
        k = rng.randint(1, 8)
        ix = NgramIndex(3, 2, k)
        for t in hist:
            ix.append(t)
        for L in range(n):
            # the device row is the history followed by unwritten slots
            _, want = ngram_draft(hist + [0] * (k + 2), L, 3, 2, k)
            if L >= 2:  # below that the kernel's clamped patterns repeat hist[0]
                assert ix.draft(L) == want, (hist, L, k)


def test_predictor_scores_what_a_verify_iteration_would_accept():
    """Each scored position's sample equals 1 + the acceptance of the oracle's
    draft at that position against the tokens that followed."""
    rng = random.Random(1)
    for _ in range(100):
        k = rng.randint(1, 6)
        prompt = [rng.randint(0, 3) for _ in range(rng.randint(1, 20))]
        gen = [rng.randint(0, 3) for _ in range(rng.randint(k + 1, 40))]
        p = AcceptancePredictor(1, 3, 2, k)
        p.start(0, prompt, gen[0])
        for i in range(1, len(gen), 3):
            p.extend(0, gen[i:i + 3])
        hist = prompt + gen
        S = len(prompt)
        want = []
        for L in range(S, len(hist) - k):
            _, d = ngram_draft(hist + [0] * (k + 2), L, 3, 2, k)
            out_tok = hist[L + 1:L + 1 + k] + [0]
            a, _ = accept(out_tok, d, list(hist) + [0] * (k + 2), L, k, 10 ** 9)
            want.append(a + 1)
        assert p.positions == len(want)
        assert p.total == sum(want)
        assert p.hits == sum(1 for w in want if w > 1)


def test_predictor_on_a_repeating_stream_opens_and_on_noise_stays_shut():
    k = 4
    p = AcceptancePredictor(1, 3, 2, k)
    motif = [11, 12, 13, 14, 15, 16, 17, 18]
    p.start(0, motif * 4, motif[0])
    for i in range(40):
        p.extend(0, [motif[(i + 1) % len(motif)]])
    assert p.predicted() == k + 1
    q = AcceptancePredictor(1, 3, 2, k)
    rng = random.Random(2)
    q.start(0, [rng.randint(0, 10 ** 6) for _ in range(64)], 5)
    for _ in range(40):
        q.extend(0, [rng.randint(0, 10 ** 6)])
    assert q.predicted() == 1.0
