"""CPU restatement of the n-gram drafter and the acceptance rule --
TEST INFRASTRUCTURE ONLY (imported by tests/ and nothing on the product path).

Follows notes/v10/spec.py of the reference:

* ``ngram_draft``  -- _ngram_draft_kernel, spec.py:36-97;
* ``accept``       -- _accept_kernel, spec.py:185-214;
* ``speculative_greedy`` -- the iteration the reference describes at
  notes/attempts.md:372-404 (draft, verify K+1 rows, accept), driven by any
  ``next_tokens(seq_prefix_rows)`` model function.

Pins (tests/test_spec_oracle.py): brute-force search over every candidate
position on small histories, hand-built known answers (most-recent match,
complete-continuation rule, backoff, zero fill, clamped pattern at short
histories, frozen sequences), and the invariant that speculative output
equals plain greedy output for a deterministic toy model.
"""


def ngram_draft(hist, L, primary, backoff, k):
    """Draft for one sequence.

    ``hist`` is the token history (list), ``L`` the number of tokens already
    in the cache, so ``hist[L]`` is the current (not yet fed) token.
    Returns ``(ids, draft)``: ``ids = [hist[L]] + draft`` (k + 1 verify rows)
    and the k draft tokens (zeros when nothing matches)."""
    cap = len(hist)

    def best_match(n):
        pattern = [hist[max(L - n + 1 + i, 0)] for i in range(n)]
        limit = L - n - k + 2            # continuation hist[j+n .. j+n+k-1] ends at <= L
        best = -1
        for j in range(0, min(limit, cap)):
            if all(hist[j + i] == pattern[i] for i in range(n)):
                best = j                 # keep the most recent (largest) start
        return best

    bp = best_match(primary)
    if bp >= 0:
        best, n = bp, primary
    else:
        best, n = best_match(backoff), backoff
    draft = [hist[best + n + t] if best >= 0 else 0 for t in range(k)]
    return [hist[L]] + draft, draft


def accept(out_tok, draft, hist, L, k, stop_len):
    """Acceptance for one sequence; mutates ``hist`` and returns ``(a, L')``.

    ``out_tok`` holds the k + 1 verify-row picks.  ``a`` is the number of
    leading drafts that equal the pick of their row; rows ``0..a`` are
    written to ``hist[L+1 .. L+1+a]`` (bounded by the history length) and the
    length advances by ``a + 1``.  A sequence with ``L >= stop_len`` is
    frozen: ``a = 0`` and nothing changes."""
    a = 0
    run = 1
    for t in range(k):
        run = run * (1 if out_tok[t] == draft[t] else 0)
        a += run
    live = L < stop_len
    if not live:
        return 0, L
    for t in range(k + 1):
        idx = L + 1 + t
        if t <= a and idx < len(hist):
            hist[idx] = out_tok[t]
    return a, L + a + 1


def plain_greedy(next_token, prompt, n_new):
    """Greedy continuation with a one-token-at-a-time model function
    ``next_token(prefix) -> token``."""
    seq = list(prompt)
    out = []
    for _ in range(n_new):
        t = next_token(seq)
        out.append(t)
        seq.append(t)
    return out


def speculative_greedy(next_token, prompt, n_new, primary=3, backoff=2, k=8):
    """Speculative decoding of one sequence with exact verification.
    Returns ``(tokens, iterations)``."""
    S = len(prompt)
    cap = S + n_new + 2 * (k + 1)
    hist = list(prompt) + [0] * (cap - S)
    hist[S] = next_token(list(prompt))   # prefill's token
    L = S
    stop_len = S + n_new - 1
    iters = 0
    while L < stop_len:
        ids, draft = ngram_draft(hist, L, primary, backoff, k)
        prefix = hist[:L]
        out_tok = []
        for t in range(k + 1):
            out_tok.append(next_token(prefix + ids[:t + 1]))
        a, L = accept(out_tok, draft, hist, L, k, stop_len)
        iters += 1
    return hist[S:S + n_new], iters
