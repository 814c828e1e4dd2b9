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
The host only reads ``naccept`` and ``out_tok`` after each iteration, through
a pinned ring and one event per iteration, with up to LOOKAHEAD iterations in
flight.
"""

import torch

from . import capi

LOOKAHEAD = 2


class SpecDecoder:
    def __init__(self, engine, state, primary, backoff, k):
        self.engine, self.state, self.lib = engine, state, state.lib
        self.primary, self.backoff, self.k = primary, backoff, k
        self.T = k + 1
        B, dev = state.batch, state.model.device
        if self.T > state.max_t:
            raise ValueError(f"verify rows {self.T} > state max_t {state.max_t}")
        self.hist = torch.zeros((B, state.cap), dtype=torch.int64, device=dev)
        self.draft = torch.zeros((B * k,), dtype=torch.int64, device=dev)
        self.naccept = torch.zeros((B,), dtype=torch.int32, device=dev)
        self.stop_len = torch.zeros((), dtype=torch.int32)  # host copy of the last stop length
        self.graph = None
        self.graph_stop = None
        self.last_stats = {}

    def _iteration(self, stop_len):
        st, lib = self.state, self.lib
        s = torch.cuda.current_stream(st.model.device).cuda_stream
        B = st.batch
        d = capi.DraftArgs()
        d.hist, d.lens, d.ids, d.draft = (self.hist.data_ptr(), st.lens.data_ptr(), st.ids.data_ptr(),
                                          self.draft.data_ptr())
        d.batch, d.cap, d.primary, d.backoff, d.k = B, st.cap, self.primary, self.backoff, self.k
        lib.ngram_draft(d, s)
        st.step(t_rows=self.T, lm_head=True, ids_out=st.out_tok, advance=False)
        a = capi.AcceptArgs()
        a.out_tok, a.draft, a.hist, a.lens, a.naccept = (st.out_tok.data_ptr(), self.draft.data_ptr(),
                                                         self.hist.data_ptr(), st.lens.data_ptr(),
                                                         self.naccept.data_ptr())
        a.batch, a.cap, a.k, a.stop_len = B, st.cap, self.k, stop_len
        lib.spec_accept(a, s)

    def _ensure_graph(self, stop_len):
        if not self.engine.use_graphs:
            return
        if self.graph is not None and self.graph_stop == stop_len:
            return
        self.graph = None
        self.graph = self.engine._capture(lambda: self._iteration(stop_len))
        self.graph_stop = stop_len

    def generate(self, prompt, steps):
        st = self.state
        B, S = prompt.shape
        T, dev = self.T, st.model.device
        stop_len = S + steps - 1
        if stop_len + 2 * T > st.cap:
            raise ValueError(f"capacity {st.cap} too small for {S} + {steps} with k={self.k}")
        self._ensure_graph(stop_len)
        prompt_d = prompt.to(dev)
        st.prefill(prompt_d)
        self.hist.zero_()
        self.hist[:, :S].copy_(prompt_d)
        self.hist[:, S].copy_(st.ids[:B])
        first = st.ids[:B].to("cpu", non_blocking=False).tolist()
        out = [[t] for t in first]
        counts = [1] * B
        emitted = 0
        yield [out[b][0] for b in range(B)]
        emitted = 1
        ring = 2 * LOOKAHEAD + 2
        h_acc = torch.empty((ring, B), dtype=torch.int32, pin_memory=True)
        h_tok = torch.empty((ring, B * T), dtype=torch.int64, pin_memory=True)
        events = [torch.cuda.Event() for _ in range(ring)]
        iters = 0
        launched = done = 0

        def launch(slot):
            if self.graph is not None:
                self.graph.replay()
            else:
                self._iteration(stop_len)
            h_acc[slot].copy_(self.naccept, non_blocking=True)
            h_tok[slot].copy_(st.out_tok[:B * T], non_blocking=True)
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
            iters += 1
            acc = h_acc[slot].tolist()
            tok = h_tok[slot].tolist()
            for b in range(B):
                if counts[b] >= steps:
                    continue
                a = acc[b]
                new = tok[b * T:b * T + a + 1]
                out[b].extend(new)
                counts[b] += len(new)
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
            "iterations": iters,
            "tokens_per_seq": steps,
            "mean_accept_len": (steps - 1) / max(iters, 1),
        }
