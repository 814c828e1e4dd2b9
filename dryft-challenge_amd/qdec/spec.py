"""Lossless n-gram speculative decoding on top of ``DecodeState``.

One iteration, captured as one hipGraph and replayed (the loop the reference
describes at notes/attempts.md:372-404; its kernels are
notes/v10/spec.py:36-224):

1. ``qdec_ngram_draft``: per sequence, the most recent earlier occurrence of
   the last ``primary`` tokens (else ``backoff`` tokens) whose ``k``-token
   continuation lies inside the history; the continuation is the draft.
   Writes the verify rows ``[current token, draft...]``.
2. one forward over ``k + 1`` rows per sequence at positions
   ``lens[b] .. lens[b] + k``; its K/V land in those cache slots and the
   greedy pick of every row goes to ``out_tok``.
3. ``qdec_spec_accept``: ``a`` = number of leading drafts equal to the pick
   of the row before them; rows ``0..a`` are genuine greedy tokens and are
   appended to the history, ``lens[b] += a + 1``.  Slots past the new length
   hold rejected drafts' K/V; the next iteration overwrites them (rollback by
   length).  Sequences that already have all their tokens are frozen.

Because every kernel computes a row the same way whatever the number of rows
in the call (see qdec.runtime), a verified row reproduces the plain decode
step bit for bit, so the emitted stream is exactly the plain greedy stream.

Acceptance gate (the reference's rule at notes/attempts.md:396-404: keep
speculating only while tokens per iteration beat the cost ratio).  A second
graph runs the same iteration with ``k = 0`` -- a plain step that keeps the
history.  The decoder measures the time ratio of the two graphs once and
predicts, without spending a verify pass, what a verify iteration would
yield: the host keeps an index of every sequence's n-grams (``NgramIndex``,
the drafter's search rule restated over the tokens it has already received)
and, for every position, compares the draft the device would have made there
with the greedy tokens that actually followed.  Greedy decoding is
deterministic and the history is the same in both modes, so that comparison
is exactly the acceptance a verify iteration at that position would have
had.  The decoder verifies while the mean over the recent positions beats
the cost ratio by 5%, and runs ``k = 0`` iterations otherwise; there are no
probe iterations.  Both graphs emit greedy tokens, so the gate changes the
speed, never the tokens.

The host only reads ``naccept`` and ``out_tok`` after each iteration, through
a pinned ring and one event per iteration, with up to LOOKAHEAD iterations in
flight.
"""

import bisect
import collections

import torch

from . import capi

LOOKAHEAD = 3
MARGIN = 1.05       # verify must beat the cost ratio by 5%
WINDOW = 64         # positions (over all sequences) in the predicted acceptance mean
MIN_SAMPLES = 8     # positions needed before the gate may open


class NgramIndex:
    """One sequence's history on the host and, per n-gram length, the start
    positions of every n-gram in it (appended in increasing order).

    ``draft(L)`` returns the k drafts qdec_ngram_draft makes at length L
    (``hist[L]`` = the current token): the most recent earlier occurrence of
    the last ``primary`` tokens whose k-token continuation ends at or before
    L, else the same for ``backoff`` tokens, else zeros (notes/v10/spec.py:
    36-97).  Patterns are clamped at the start of the history as the kernel
    clamps them."""

    def __init__(self, primary, backoff, k):
        self.ns, self.k = (primary, backoff), k
        self.hist = []
        self.starts = {n: {} for n in set(self.ns)}

    def append(self, tok):
        h = self.hist
        h.append(tok)
        i = len(h) - 1
        for n, table in self.starts.items():
            j = i - n + 1
            if j >= 0:
                table.setdefault(tuple(h[j:i + 1]), []).append(j)

    def draft(self, L):
        h = self.hist
        for n in self.ns:
            pattern = tuple(h[max(L - n + 1 + i, 0)] for i in range(n))
            found = self.starts[n].get(pattern)
            if found:
                i = bisect.bisect_left(found, L - n - self.k + 2) - 1
                if i >= 0:
                    j = found[i]
                    return h[j + n:j + n + self.k]
        return [0] * self.k


class AcceptancePredictor:
    """For every position of every sequence, the tokens a verify iteration
    started there would have emitted (1 + the leading drafts equal to the
    greedy tokens that followed), known k tokens later; the mean over the
    last WINDOW positions predicts the next verify iteration."""

    def __init__(self, batch, primary, backoff, k):
        self.k = k
        self.index = [NgramIndex(primary, backoff, k) for _ in range(batch)]
        self.pending = [collections.deque() for _ in range(batch)]
        self.recent = collections.deque(maxlen=WINDOW)
        self.positions = self.hits = 0
        self.total = 0

    def start(self, b, prompt, first):
        """Sequence b's prompt (history only: no verify iteration starts
        inside it) and the first generated token (position S, the first
        place a verify iteration can start)."""
        for t in prompt:
            self.index[b].append(t)
        self.extend(b, [first])

    def extend(self, b, tokens):
        """Append generated tokens of sequence b; every new length is a
        position whose would-be verify iteration is scored k tokens later."""
        ix, pend = self.index[b], self.pending[b]
        for t in tokens:
            ix.append(t)
            L = len(ix.hist) - 1
            while pend and pend[0][0] + self.k <= L:
                L0, d = pend.popleft()
                follow = ix.hist[L0 + 1:L0 + 1 + self.k]
                a = 0
                while a < self.k and d[a] == follow[a]:
                    a += 1
                self.recent.append(a + 1)
                self.positions += 1
                self.hits += a > 0
                self.total += a + 1
            pend.append((L, ix.draft(L)))

    def predicted(self):
        """Tokens per sequence a verify iteration is expected to emit (1.0
        until MIN_SAMPLES positions are known)."""
        if len(self.recent) < MIN_SAMPLES:
            return 1.0
        return sum(self.recent) / len(self.recent)


class SpecDecoder:
    def __init__(self, engine, state, primary, backoff, k):
        self.engine, self.state, self.lib = engine, state, state.lib
        self.primary, self.backoff, self.k = primary, backoff, k
        self.T = k + 1
        B, dev = state.batch, state.model.device
        if k < 1:
            raise ValueError("speculation needs k >= 1 drafts")
        if self.T > state.max_t:
            raise ValueError(f"verify rows {self.T} > state max_t {state.max_t}")
        self.hist = torch.zeros((B, state.cap), dtype=torch.int64, device=dev)
        self.draft = torch.zeros((B * k,), dtype=torch.int64, device=dev)
        self.naccept = torch.zeros((B,), dtype=torch.int32, device=dev)
        self.graphs = {}       # k -> graph, for the current stop length
        self.graph_stop = None
        self.cost_ratio = None  # time of a verify iteration / a k = 0 iteration
        self.last_stats = {}

    def _draft(self, k):
        """Write the verify rows ``ids[b*(k+1) ..]`` = [current token, k
        drafts] and ``draft`` (the n-gram drafter kernel)."""
        st = self.state
        s = torch.cuda.current_stream(st.model.device).cuda_stream
        d = capi.DraftArgs()
        d.hist, d.lens, d.ids, d.draft = (self.hist.data_ptr(), st.lens.data_ptr(), st.ids.data_ptr(),
                                          self.draft.data_ptr())
        d.batch, d.cap, d.primary, d.backoff, d.k = st.batch, st.cap, self.primary, self.backoff, k
        self.lib.ngram_draft(d, s)

    def _iteration(self, k, stop_len):
        st, lib = self.state, self.lib
        s = torch.cuda.current_stream(st.model.device).cuda_stream
        B = st.batch
        self._draft(k)
        st.step(t_rows=k + 1, lm_head=True, ids_out=st.out_tok, advance=False)
        a = capi.AcceptArgs()
        a.out_tok, a.draft, a.hist, a.lens, a.naccept = (st.out_tok.data_ptr(), self.draft.data_ptr(),
                                                         self.hist.data_ptr(), st.lens.data_ptr(),
                                                         self.naccept.data_ptr())
        a.batch, a.cap, a.k, a.stop_len = B, st.cap, k, stop_len
        lib.spec_accept(a, s)

    def _ensure_graphs(self, stop_len):
        if not self.engine.use_graphs:
            return
        if self.graphs and self.graph_stop == stop_len:
            return
        self.graphs = {}
        for k in (self.k, 0):
            self.graphs[k] = self.engine._capture(lambda k=k: self._iteration(k, stop_len))
        self.graph_stop = stop_len
        if self.cost_ratio is None:
            # The replays scribble on cache slots and lengths that generate()
            # resets (prefill, history) before it starts.
            t = {}
            for k, g in self.graphs.items():
                g.replay()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(5):
                    g.replay()
                e1.record()
                torch.cuda.synchronize()
                t[k] = e0.elapsed_time(e1)
            self.cost_ratio = t[self.k] / t[0]

    def _run(self, k, stop_len):
        g = self.graphs.get(k)
        if g is not None:
            g.replay()
        else:
            self._iteration(k, stop_len)

    def generate(self, prompt, steps, gate=True):
        st = self.state
        B, S = prompt.shape
        T, dev = self.T, st.model.device
        stop_len = S + steps - 1
        if stop_len + 2 * T > st.cap:
            raise ValueError(f"capacity {st.cap} too small for {S} + {steps} with k={self.k}")
        self._ensure_graphs(stop_len)
        ratio = (self.cost_ratio or 1.0) if gate else 0.0  # 0: always verify
        prompt_d = prompt.to(dev)
        st.prefill(prompt_d)
        self.hist.zero_()
        self.hist[:, :S].copy_(prompt_d)
        self.hist[:, S].copy_(st.ids[:B])
        first = self.engine._checked(st.ids[:B].to("cpu", non_blocking=False).tolist())
        out = [[t] for t in first]
        counts = [1] * B
        pred = AcceptancePredictor(B, self.primary, self.backoff, self.k)
        for b, row in enumerate(prompt.tolist()):
            pred.start(b, row, first[b])
        yield [out[b][0] for b in range(B)]
        emitted = 1
        ring = 2 * LOOKAHEAD + 2
        h_acc = torch.empty((ring, B), dtype=torch.int32, pin_memory=True)
        h_tok = torch.empty((ring, B * T), dtype=torch.int64, pin_memory=True)
        events = [torch.cuda.Event() for _ in range(ring)]
        kinds = [0] * ring
        launched = done = 0
        n_verify = n_plain = 0
        verify_tokens = 0.0

        def choose():
            return self.k if pred.predicted() >= ratio * MARGIN else 0

        def launch(slot):
            k = choose()
            kinds[slot] = k
            self._run(k, stop_len)
            h_acc[slot].copy_(self.naccept, non_blocking=True)
            h_tok[slot, :B * (k + 1)].copy_(st.out_tok[:B * (k + 1)], non_blocking=True)
            events[slot].record()

        # Every iteration emits >= 1 token per live sequence, so at most
        # steps - 1 iterations are ever needed.
        max_iters = steps - 1
        while emitted < steps:
            while launched < max_iters and launched - done < LOOKAHEAD:
                launch(launched % ring)
                launched += 1
            slot = done % ring
            events[slot].synchronize()
            done += 1
            k = kinds[slot]
            Tk = k + 1
            acc = h_acc[slot].tolist()
            tok = self.engine._checked(h_tok[slot, :B * (k + 1)].tolist())
            gained, live = 0, 0
            for b in range(B):
                if counts[b] >= steps:
                    continue
                a = acc[b]
                new = tok[b * Tk:b * Tk + a + 1]
                out[b].extend(new)
                pred.extend(b, new)
                counts[b] += len(new)
                gained += len(new)
                live += 1
            if k:
                n_verify += 1
                if live:
                    verify_tokens += gained / live
            else:
                n_plain += 1
            ready = min(counts)
            while emitted < min(ready, steps):
                yield [out[b][emitted] for b in range(B)]
                emitted += 1
            if done >= max_iters and emitted < steps:
                raise RuntimeError("speculative decoding made no progress")
        # Drain iterations queued past the end (their results are unused).
        for j in range(done, launched):
            events[j % ring].synchronize()
        self.last_stats = {
            "iterations": done,
            "verify_iterations": n_verify,
            "plain_iterations": n_plain,
            "tokens_per_seq": steps,
            "mean_accept_len": (steps - 1) / max(done, 1),
            "tokens_per_verify": verify_tokens / max(n_verify, 1),
            "cost_ratio": None if self.cost_ratio is None else round(self.cost_ratio, 4),
            # every position's would-be verify iteration (host prediction, exact
            # for greedy decoding): first draft right, and tokens it would emit
            "draft_hit_rate": pred.hits / max(pred.positions, 1),
            "predicted_tokens_per_verify": pred.total / max(pred.positions, 1),
            "positions_scored": pred.positions,
        }
