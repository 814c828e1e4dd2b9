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
  norm and SwiGLU, down with the residual add; the lm_head (the embedding
  when tied) with the final norm and the greedy argmax.  5 launches per
  layer, 182 per step for Qwen3-4B.
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
# One launch per layer (qdec_layer) instead of five, as the reference's
# MEGA_ENABLED / MEGA_FORCE / MARGIN (engine/engine.py:81-91, 123): when
# enabled, a shape of plain decode that qdec_layer takes is checked against
# the per-operation step and raced against it, and kept only if it is faster
# by the margin.  Off by default: on MI355X a layer's four grid barriers cost
# more than the four launch boundaries they replace.
MEGA_ENABLED = False
MEGA_FORCE = False
MEGA_MARGIN = 0.97
# n-gram drafter settings of speculative decoding (notes/v10/spec.py:13-16).
SPEC_PRIMARY = 3
SPEC_BACKOFF = 2
SPEC_K_MAX = 8


def spec_k(batch, group=4):
    """Drafts per sequence per verify iteration: up to SPEC_K_MAX, and few
    enough that the batch's verify rows fit one 16-row MFMA tile (the GEMMs'
    fast path), so a verify iteration costs about a plain step.  0 = no
    speculation at this batch size.  The verify pass's k + 1 rows per
    sequence also stay within what the state's attention takes."""
    return max(0, min(SPEC_K_MAX, 16 // batch - 1, max_rows_per_seq(batch, group=group) - 1))


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
        self.spec_k = spec_k(batch, engine.model.cfg.group)
        slack = 2 * (self.spec_k + 1)
        self.capacity = prompt_len + new_tokens + slack
        max_t = (self.spec_k + 1) if (speculate and self.spec_k) else 16
        self.state = DecodeState(engine.model, batch, self.capacity, max_t=max_t)
        self.graph = None
        self.spec_graph = None
        self.host = torch.empty((new_tokens, batch), dtype=torch.int64, pin_memory=True)
        # the layer kernel's error word after each step (one launch per layer only)
        self.host_err = torch.zeros((new_tokens,), dtype=torch.int32, pin_memory=True)
        self.events = [torch.cuda.Event() for _ in range(new_tokens)]


class Engine:
    def __init__(self, model_path: str, speculate: bool = False, mega=None) -> None:
        """Load the checkpoint at ``model_path`` (HF layout, local files only).
        ``mega``: try one launch per layer for plain decode (None: MEGA_ENABLED)."""
        start = time.perf_counter()
        if not torch.cuda.is_available():
            raise RuntimeError("Engine needs a HIP device (torch.cuda.is_available() is False)")
        cfg = load_config(model_path)
        tensors = load_tensors(model_path)
        self._setup(cfg, tensors, speculate, mega=mega)
        del tensors
        _log(f"engine ready in {time.perf_counter() - start:.1f}s "
             f"({self.model.weight_bytes() / 1e9:.2f} GB of packed weights)")

    @classmethod
    def from_tensors(cls, cfg, tensors, speculate=False, use_graphs=True, mega=None):
        """Build around in-memory HF-named tensors (tests)."""
        self = cls.__new__(cls)
        self._setup(cfg, tensors, speculate, use_graphs, mega=mega)
        return self

    @classmethod
    def from_model(cls, model, device="cuda:0", use_triton=True, use_graphs=True):
        """The reference's test hook (engine/engine.py:243-248): build around
        an already-loaded Transformers Qwen3 model (its config and weights).
        The engine runs its HIP kernels on ``device`` (a HIP device) or
        nothing: ``use_triton=False``, which selects the reference's PyTorch
        ops, and a CPU device are refused, since there is no other path."""
        dev = torch.device(device)
        if dev.type != "cuda":
            raise ValueError(f"Engine runs on a HIP device (got {device!r}); it has no CPU path")
        if not use_triton:
            raise ValueError("use_triton=False selects the reference's PyTorch ops; this engine only has its HIP "
                             "kernels (use_triton=True runs them)")
        cfg = model.config.to_dict()
        tensors = {k: v.detach() for k, v in model.state_dict().items()}
        return cls.from_tensors(cfg, tensors, use_graphs=use_graphs)

    def _setup(self, cfg, tensors, speculate, use_graphs=True, mega=None):
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
        self.mega = MEGA_ENABLED if mega is None else bool(mega)
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
        # Known-answer checks of this shape's own plans (every row count it
        # replays) before it serves; raises, and the shape is not kept.
        t_rows = (1, sh.spec_k + 1) if (self.speculate and sh.spec_k) else (1,)
        selfcheck.run_shape(sh.state, t_rows)
        if self.use_graphs:
            sh.graph = self._capture(lambda: sh.state.step(t_rows=1))
            if self.mega and not self.speculate and sh.state.layer_supported():
                self._try_mega(sh, prompt_len, new_tokens)
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

    # ------------------------------------------------ one launch per layer
    def _check_mega(self, st, prompt_len, n_check=3):
        """Logits of the one-launch-per-layer step against the per-operation
        step on the same prompt and the same forced tokens, over a few
        consecutive positions (engine/engine.py:691-734): the layer kernel
        sums O and down over 4 waves, the per-operation plans over 8, so the
        two agree to rounding, not bit for bit."""
        B, dev = st.batch, self.device
        g = torch.Generator().manual_seed(4321)
        prompt = torch.randint(100, self.model.cfg.vocab, (B, prompt_len), generator=g)
        toks = torch.randint(100, self.model.cfg.vocab, (n_check, B), generator=g).to(dev)
        st.logits = torch.empty((st.max_rows, self.model.cfg.vocab), dtype=torch.bfloat16, device=dev)
        try:
            st.prefill(prompt.to(dev))
            out = {}
            for layer_launch in (False, True):
                st.layer_launch = layer_launch
                rows = []
                for t in range(n_check):
                    st.lens.fill_(prompt_len + t)
                    st.ids[:B].copy_(toks[t])
                    st.run_step(t_rows=1, advance=False)
                    rows.append(st.logits[:B].float().clone())
                out[layer_launch] = torch.stack(rows)
            torch.cuda.synchronize(dev)
        finally:
            st.logits = None
        err = st.layer_error()
        ref, got = out[False], out[True]
        if err or not torch.isfinite(got).all():
            return False, f"error word {err}, finite {bool(torch.isfinite(got).all())}"
        diff = (got - ref).abs()
        max_d, mean_d = diff.max().item(), diff.mean().item()
        agree = int((got.argmax(-1) == ref.argmax(-1)).sum())
        # the reference's gate (engine/engine.py:733): max over the vocabulary
        # and the mean over bf16 logits, read as a pair
        ok = max_d <= 1.5 and mean_d <= 0.1
        return ok, f"max|dlogit|={max_d:.3f} mean={mean_d:.4f} argmax {agree}/{n_check * B}"

    def _time_graph(self, st, graph, start_len, reps):
        st.lens.fill_(start_len)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            graph.replay()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / reps

    def _try_mega(self, sh, prompt_len, new_tokens):
        """Opt-in one-launch-per-layer path for this shape: write its layer
        plans, compare its logits with the five-launch step's (_check_mega),
        time both graphs over the same positions, and replay the layer graph
        from now on only when its time is under MEGA_MARGIN of the other's
        (or MEGA_FORCE); the reference's race, engine/engine.py:856-884."""
        start = time.perf_counter()
        st = sh.state
        st.enable_layer_launch()
        ok, detail = self._check_mega(st, prompt_len)
        info = {"check": detail, "ok": ok, "used": False}
        if ok:
            graph = self._capture(lambda: st.step(t_rows=1))
            reps = max(1, min(16, new_tokens))
            t_cur, t_mega = [], []
            for _ in range(2):
                st.disable_layer_launch()
                t_cur.append(self._time_graph(st, sh.graph, prompt_len, reps))
                st.layer_launch = True
                t_mega.append(self._time_graph(st, graph, prompt_len, reps))
            t_cur, t_mega = min(t_cur), min(t_mega)
            err = st.layer_error()
            use = err == 0 and (MEGA_FORCE or t_mega < t_cur * MEGA_MARGIN)
            info.update(per_op_ms=round(t_cur, 4), layer_ms=round(t_mega, 4), error_word=err, used=use)
            if use:
                sh.graph = graph
        st.layer_launch = info["used"]
        info["setup_s"] = round(time.perf_counter() - start, 2)
        self.stats["mega"] = info
        _log(f"layer-launch step: {info}")

    # ---------------------------------------------------------- generation
    def _launch(self, sh, step):
        if sh.graph is not None:
            sh.graph.replay()
        else:
            sh.state.step(t_rows=1)
        self._publish(sh, step)

    def _publish(self, sh, step):
        sh.host[step].copy_(sh.state.ids[:sh.batch], non_blocking=True)
        if sh.state.layer_launch:
            sh.host_err[step:step + 1].copy_(sh.state.layer_ctl[2:3], non_blocking=True)
        sh.events[step].record()

    def _fetch(self, sh, step):
        sh.events[step].synchronize()
        if sh.state.layer_launch and int(sh.host_err[step]):
            # The step's stages ran unsynchronised: refuse its tokens, clear
            # the barrier state and drop the shape (its graph holds layer
            # launches), so the next call builds the per-operation step.
            err = int(sh.host_err[step])
            torch.cuda.synchronize(self.device)
            sh.state.reset_layer_ctl()
            sh.state.disable_layer_launch()
            self.shape = None
            raise capi.QdecError("generate", -1, f"layer kernel error word {err} at step {step} (a grid barrier "
                                 "wait ran out of polls, a stale plan, or another workgroup count)")
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
        """A generator of greedy decode steps over the batch ``input_ids``
        (B prompts of one common length, ids in the vocabulary).

        Each ``next()`` hands back B token ids, the pick of every sequence at
        that position; there are ``max_new_tokens`` of them in all (none when
        it is not positive), whatever the tokens are -- an end-of-sequence id
        is emitted like any other."""
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
