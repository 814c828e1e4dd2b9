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
history.  The decoder measures the time ratio of the two graphs once, tracks
the mean tokens emitted per sequence by recent verify iterations, and runs
``k = 0`` iterations while that mean is below the ratio (plus a margin),
probing with a few verify iterations after ``PROBE_EVERY`` plain ones (a
gap that doubles while probes keep failing).  Both
graphs emit greedy tokens, so the gate changes the speed, never the tokens.

The host only reads ``naccept`` and ``out_tok`` after each iteration, through
a pinned ring and one event per iteration, with up to LOOKAHEAD iterations in
flight.
"""

import torch

from . import capi

LOOKAHEAD = 3
MARGIN = 1.05       # verify must beat the cost ratio by 5%
EMA = 0.25          # weight of the newest verify iteration in the running mean
PROBE_EVERY = 32    # plain iterations before the first probe while the gate is shut
PROBE_MAX = 512     # the gap doubles after every probe that does not reopen the gate
PROBE_LEN = 3       # verify iterations per probe


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
        first = st.ids[:B].to("cpu", non_blocking=False).tolist()
        out = [[t] for t in first]
        counts = [1] * B
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
        mean_tokens = float(T)  # optimistic start: speculate first
        plain_run = 0
        probe_left = 0
        probe_gap = PROBE_EVERY

        def choose():
            nonlocal plain_run, probe_left, probe_gap
            if probe_left > 0:
                probe_left -= 1
                return self.k
            if mean_tokens >= ratio * MARGIN:
                probe_gap = PROBE_EVERY
                return self.k
            plain_run += 1
            if plain_run >= probe_gap:
                plain_run = 0
                probe_left = PROBE_LEN - 1
                probe_gap = min(2 * probe_gap, PROBE_MAX)
                return self.k
            return 0

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
            tok = h_tok[slot].tolist()
            gained, live = 0, 0
            for b in range(B):
                if counts[b] >= steps:
                    continue
                a = acc[b]
                new = tok[b * Tk:b * Tk + a + 1]
                out[b].extend(new)
                counts[b] += len(new)
                gained += len(new)
                live += 1
            if k:
                n_verify += 1
                if live:
                    mean_tokens = (1 - EMA) * mean_tokens + EMA * (gained / live)
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
        }
