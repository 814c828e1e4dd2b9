"""Qwen3 greedy decoder for one MI355X: hand-written HIP kernels, hipGraph steps.

Public surface (the reference's engine/engine.py:215-241, 1024-1063):

    engine = Engine(model_path)                 # HF checkpoint directory
    for step in engine.generate(input_ids, n):  # yields [B] token ids, n times
        ...

* Weights are read from the checkpoint's safetensors files and repacked once
  into the MFMA tile layout of include/qdec.h (``qdec.runtime.DeviceModel``).
* Every operation of a decode step is a kernel of libqdec.so, called through
  its C ABI: embedding gather; per layer the QKV projection with the input
  RMSNorm folded in, GQA attention with head norm + RoPE + KV write folded in,
  the O projection with the residual add, gate/up with the post-attention
  norm and SwiGLU, down with the residual add; the tied lm_head with the
  final norm and the greedy argmax.  5 launches per layer, 182 per step.
* A step reads its token ids and cache lengths from device buffers and writes
  the next ids and lengths itself, so it is captured once per shape as a
  hipGraph and replayed; up to LOOKAHEAD replays are queued ahead of the
  consumer, each followed by an async copy of its ids into pinned host memory
  and an event (engine/engine.py:1007-1063).
* Optional n-gram speculative decoding (``speculate=True``): a suffix-match
  drafter over each sequence's own history, one verify forward over K+1 rows
  per sequence, longest-prefix acceptance and rollback by length.  The
  kernels give every row the same arithmetic whatever the row count, so the
  emitted tokens are exactly those of the plain greedy path.
* The engine never falls back to another implementation: a missing or
  failing kernel library raises.
"""

import os
import sys
import time

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
if _HERE not in sys.path:
    sys.path.insert(0, _HERE)

from qdec import capi, selfcheck  # noqa: E402
from qdec.checkpoint import load_config, load_tensors  # noqa: E402
from qdec.runtime import DecodeState, DeviceModel, max_rows_per_seq  # noqa: E402

# Decode steps queued ahead of the one being handed to the caller (as the
# reference, engine/engine.py:66); one before the first token.
LOOKAHEAD = 3
# n-gram drafter settings of speculative decoding (notes/v10/spec.py:13-16).
SPEC_PRIMARY = 3
SPEC_BACKOFF = 2
SPEC_K_MAX = 8


def spec_k(batch):
    """Drafts per sequence per verify iteration: up to SPEC_K_MAX, and few
    enough that the batch's verify rows fit one 16-row MFMA tile (the GEMMs'
    fast path), so a verify iteration costs about a plain step.  0 = no
    speculation at this batch size.  The verify pass's k + 1 rows per
    sequence also stay within what the state's attention takes."""
    return max(0, min(SPEC_K_MAX, 16 // batch - 1, max_rows_per_seq(batch) - 1))


def _log(message):
    print(f"[engine] {message}", file=sys.stderr, flush=True)


class _Shape:
    """Per (batch, prompt, new tokens) state: decode state, graphs, host ring."""

    def __init__(self, engine, batch, prompt_len, new_tokens, speculate):
        self.key = (batch, prompt_len, new_tokens, speculate)
        self.batch = batch
        # The verify slack is reserved in both modes: attention chunking is a
        # function of (batch, capacity), and plain and speculative runs of one
        # shape must chunk alike to produce the same bits.
        self.spec_k = spec_k(batch)
        slack = 2 * (self.spec_k + 1)
        self.capacity = prompt_len + new_tokens + slack
        max_t = (self.spec_k + 1) if (speculate and self.spec_k) else 16
        self.state = DecodeState(engine.model, batch, self.capacity, max_t=max_t)
        self.graph = None
        self.spec_graph = None
        self.host = torch.empty((new_tokens, batch), dtype=torch.int64, pin_memory=True)
        self.events = [torch.cuda.Event() for _ in range(new_tokens)]


class Engine:
    def __init__(self, model_path: str, speculate: bool = False) -> None:
        """Load the checkpoint at ``model_path`` (HF layout, local files only)."""
        start = time.perf_counter()
        if not torch.cuda.is_available():
            raise RuntimeError("Engine needs a HIP device (torch.cuda.is_available() is False)")
        cfg = load_config(model_path)
        tensors = load_tensors(model_path)
        self._setup(cfg, tensors, speculate)
        del tensors
        _log(f"engine ready in {time.perf_counter() - start:.1f}s "
             f"({self.model.weight_bytes() / 1e9:.2f} GB of packed weights)")

    @classmethod
    def from_tensors(cls, cfg, tensors, speculate=False, use_graphs=True):
        """Build around in-memory HF-named tensors (tests)."""
        self = cls.__new__(cls)
        self._setup(cfg, tensors, speculate, use_graphs)
        return self

    def _setup(self, cfg, tensors, speculate, use_graphs=True):
        self.device = torch.device("cuda:0")
        torch.cuda.set_device(self.device)
        self.lib = capi.lib()
        self.model = DeviceModel(cfg, tensors, self.device)
        # Known-answer checks of every kernel family on this device, with the
        # model's own weights and plans; raises on a mismatch (no fallback).
        selfcheck.run(DecodeState(self.model, 1, 64, max_t=1))
        self.speculate = bool(speculate)
        self.spec_gate = True  # speculation falls back to plain steps when drafts do not pay
        self.use_graphs = use_graphs
        self.shape = None
        self.stats = {}

    # ----------------------------------------------------------- per shape
    def _shape_for(self, batch, prompt_len, new_tokens):
        key = (batch, prompt_len, new_tokens, self.speculate)
        if self.shape is not None and self.shape.key == key:
            return self.shape
        self.shape = None
        torch.cuda.empty_cache()
        start = time.perf_counter()
        sh = _Shape(self, batch, prompt_len, new_tokens, self.speculate)
        if self.use_graphs:
            sh.graph = self._capture(lambda: sh.state.step(t_rows=1))
        self.shape = sh
        _log(f"shape B={batch} S={prompt_len} N={new_tokens}: capacity {sh.state.cap}, "
             f"attention chunk {sh.state.chunk}, graph={'yes' if sh.graph else 'no'}, "
             f"setup {time.perf_counter() - start:.2f}s")
        return sh

    def _capture(self, fn):
        """Run ``fn`` once eagerly (it only scribbles on slots the prefill
        rewrites), then record it into a graph."""
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fn()
        torch.cuda.synchronize()
        return graph

    # ---------------------------------------------------------- generation
    def _launch(self, sh, step):
        if sh.graph is not None:
            sh.graph.replay()
        else:
            sh.state.step(t_rows=1)
        self._publish(sh, step)

    def _publish(self, sh, step):
        sh.host[step].copy_(sh.state.ids[:sh.batch], non_blocking=True)
        sh.events[step].record()

    def _fetch(self, sh, step):
        sh.events[step].synchronize()
        return self._checked(sh.host[step].tolist())

    def _checked(self, toks):
        """Tokens as emitted, or an error if the device flagged invalid state
        (capi.NAN_ID: an out-of-range token id or cache length made a row
        NaN; the kernels never substitute a value)."""
        vocab = self.model.cfg.vocab
        for t in toks:
            if not 0 <= t < vocab:
                raise capi.QdecError("generate", -1, f"device emitted token id {t} (vocab {vocab}): an "
                                     "out-of-range token id or cache length reached a kernel")
        return toks

    def generate(self, input_ids: list[list[int]], max_new_tokens: int):
        """Greedy continuation of every sequence, one step at a time.

        Yields a list with one token id per sequence for each output step,
        exactly ``max_new_tokens`` times (nothing for ``max_new_tokens <=
        0``).  Every sequence has the same length; end-of-sequence tokens do
        not stop generation."""
        steps = int(max_new_tokens)
        if steps <= 0:
            return
        ids = torch.tensor(input_ids, dtype=torch.int64)
        if ids.dim() != 2 or ids.shape[1] < 1:
            raise ValueError("input_ids must be a non-empty list of equal-length lists")
        batch, prompt_len = ids.shape
        if int(ids.min()) < 0 or int(ids.max()) >= self.model.cfg.vocab:
            raise ValueError(f"input_ids must lie in [0, {self.model.cfg.vocab})")
        if self.speculate:
            yield from self._generate_spec(ids, steps)
            return
        sh = self._shape_for(batch, prompt_len, steps)
        yield from self._generate_plain(sh, ids, steps)

    def _generate_plain(self, sh, ids, steps):
        sh.state.prefill(ids.to(self.device, non_blocking=True))
        self._publish(sh, 0)
        ahead = LOOKAHEAD if sh.graph is not None else 1
        launched = 1
        for step in range(steps):
            target = min(steps, step + 1 + (1 if step == 0 else ahead))
            while launched < target:
                self._launch(sh, launched)
                launched += 1
            yield self._fetch(sh, step)

    # --------------------------------------------------------- speculation
    def _generate_spec(self, ids, steps):
        from qdec.spec import SpecDecoder

        batch, prompt_len = ids.shape
        sh = self._shape_for(batch, prompt_len, steps)
        if sh.spec_k == 0:  # no room for drafts at this batch size
            yield from self._generate_plain(sh, ids, steps)
            self.stats["spec"] = {"iterations": steps - 1, "verify_iterations": 0, "plain_iterations": steps - 1}
            return
        dec = getattr(sh, "spec", None)
        if dec is None:
            dec = sh.spec = SpecDecoder(self, sh.state, SPEC_PRIMARY, SPEC_BACKOFF, sh.spec_k)
        yield from dec.generate(ids, steps, gate=self.spec_gate)
        self.stats["spec"] = dec.last_stats
