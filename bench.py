"""Decode benchmark: Qwen3-4B bf16 greedy decode on one MI355X.

    python bench.py [--steps K] [--warmup W] [--config c2|c3|c4|c5] [--gpus 1]

Workload (the config the headline metric is quoted
on): Qwen3-4B architecture, bf16, random-init N(0, 0.02) weights from seed 0
written as a Hugging Face checkpoint directory and loaded through
``Engine(model_path)``; batch 1, 512 prompt tokens uniform over the vocab
(seed 1), 256 greedy new tokens.  A step is one decode step of the whole
batch (one hipGraph replay: embed, 36 layers, lm_head + argmax).  The timed
region holds exactly K replays bracketed by device synchronisations; the
prompt is prefilled before it and positions cycle through the workload's
own range [512, 767], so every timed step does the work of a real step of
this workload.

Printed JSON fields beyond the driver contract:
  roofline      gate/up GEMM (the dominant kernel, 44.6% of weight bytes),
                algorithmic bytes per launch / its average duration measured
                with HIP events on the engine's stream;
  cpu_baseline  the Transformers CPU greedy loop on the same checkpoint
                (the reference's own oracle path), on a bounded sample;
  step_hbm      algorithmic bytes per step (weights + KV read/write) / step time;
  generate      the same workload through the public generate() (host loop
                included): time per output token from the first yielded
                token to the last;
  prefill       prompt processing of the headline prompt (time to first
                token: the prompt through the 36 layers on the matrix cores,
                lm_head + argmax of the last position), tok/s and TFLOP/s;
  layer_launch  the same decode step with each layer as one qdec_layer launch
                (38 launches instead of 182): its logit check against the
                per-operation step and both graphs timed over the same
                positions (skip with --no-layer);
  batched       decode tok/s and step_hbm of configs[2] (batch 8, 1024
                prompt tokens) and configs[3] (batch 32, 4096), each after a
                real (timed) prefill of its random prompts (skip with
                --no-batched);
  speculation   BASELINE.json configs[4] through the same engine: batch 4,
                1024-token prompts tiling a seeded 64-token motif with 10%
                random substitutions, 512 new tokens, n-gram drafter (n=3,
                backoff 2, up to 8 drafts); plain and speculative generate()
                timed from the first emitted token to the last, tokens
                compared for identity (skip with --no-spec).  Its "ceiling"
                runs the same verify / accept loop with drafts taken from the
                plain run's own output (every draft right): an upper bound of
                the speculative path, not a drafter result.
"""

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(REPO, "dryft-challenge_amd")
for _p in (PKG, REPO):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
# HBM bytes per gate/up launch at batch 1 measured with rocprofv3 counters
# (bench.py --pmc-role gate_up; FETCH_SIZE x 1.99994 + WRITE_SIZE, the scale
# factors read off a 512 MiB device copy).
GATE_UP_TRAFFIC_BYTES = 99_898_266

CONFIGS = {
    # name: (batch, prompt, new tokens, description)
    "c2": (1, 512, 256, "qwen3-4b bf16 bs1 prompt512 new256"),
    "c3": (8, 1024, 512, "qwen3-4b bf16 bs8 prompt1024 new512"),
    "c4": (32, 4096, 256, "qwen3-4b bf16 bs32 prompt4096 new256"),
    # config 5's batch and prompt length through plain decode (its motif
    # prompts and speculative decoding run in the `speculation` object)
    "c5": (4, 1024, 512, "qwen3-4b bf16 bs4 prompt1024 new512"),
}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def step_bytes(model_cfg, weight_bytes, batch, pos):
    """Algorithmic HBM bytes of one decode step at position ``pos``: all
    weights once, the KV read of slots 0..pos and the KV write of slot pos."""
    per_tok = 2 * model_cfg.n_layers * model_cfg.nkv * model_cfg.head_dim * 2
    return weight_bytes + batch * per_tok * (pos + 1) + batch * per_tok


ROLES = ("qkv", "attn", "o", "gate_up", "down", "lm")


def time_gemm_role(engine, state, role, reps=5, t_rows=1):
    """Average duration (s) of one launch of ``role``'s kernel (a GEMM, or
    ``attn``: the decode attention as the step launches it), over all
    layers' weights / caches (so nothing is served from the 256 MB MALL),
    HIP events on the engine's stream.  ``t_rows`` > 1: the verify pass's
    calls (batch x t_rows rows)."""
    import torch
    lib = engine.lib
    rows = state.batch * t_rows
    n = engine.model.cfg.n_layers if role != "lm" else 1
    if role == "attn":
        pm = state._merge_in_o(t_rows)
        args = [state._attn_args(i, t_rows, partials=pm) for i in range(n)]
        call = lib.attn
    elif role == "o" and state._merge_in_o(t_rows):  # merges the attention's chunk partials, as in the step
        args = [state._gemm_args(role, i, rows, x_attn=state._attn_args(i, 1, partials=True)) for i in range(n)]
        call = lib.gemm
    else:
        args = [state._gemm_args(role, i, rows) for i in range(n)]
        call = lib.gemm
    s = torch.cuda.current_stream()
    for a in args:  # warm
        call(a, s.cuda_stream)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(s)
    for _ in range(reps):
        for a in args:
            call(a, s.cuda_stream)
    e1.record(s)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3 / (reps * len(args))


def read_ceiling(lib, device, gib=2, reps=5):
    """Streaming-read bandwidth of this device (bytes/s): qdec_read_probe over
    a buffer 8x the 256 MB memory-side cache, 16-byte non-temporal loads as
    the decode kernels issue them; mean of ``reps`` launches timed with HIP
    events on the current stream."""
    import torch
    buf = torch.empty(gib << 30, dtype=torch.uint8, device=device)
    blocks = 8192
    sink = torch.zeros(blocks, dtype=torch.int32, device=device)
    s = torch.cuda.current_stream()
    lib.read_probe(buf.data_ptr(), buf.numel(), sink.data_ptr(), blocks, s.cuda_stream)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(reps):
        lib.read_probe(buf.data_ptr(), buf.numel(), sink.data_ptr(), blocks, s.cuda_stream)
    e1.record(s)
    torch.cuda.synchronize()
    sec = e0.elapsed_time(e1) / 1e3 / reps
    del buf
    return (gib << 30) / sec


def prefill_flops(mc, batch, prompt_len):
    """Algorithmic flops of a prefill: every layer matrix once per prompt
    token (2 flops per weight), causal attention (QK and PV over slots
    0..t for position t), the lm_head for the last position of each
    sequence."""
    per_tok = mc.n_layers * (mc.n_qkv * mc.hidden + mc.hidden * mc.nq * mc.head_dim
                             + 2 * mc.inter * mc.hidden + mc.hidden * mc.inter)
    attn = mc.n_layers * mc.nq * 4 * mc.head_dim * prompt_len * (prompt_len + 1) // 2
    return batch * (2 * per_tok * prompt_len + attn + 2 * mc.vocab * mc.hidden)


def time_prefill(state, prompt, reps=2):
    """Prefill of ``prompt`` (device [B, S]) into ``state``: the best of
    ``reps`` runs (the first also allocates the prefill buffers), wall clock
    around device synchronisations."""
    import torch
    best = float("inf")
    for _ in range(reps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        state.prefill(prompt)
        torch.cuda.synchronize()
        best = min(best, time.perf_counter() - t0)
    B, S = prompt.shape
    fl = prefill_flops(state.model.cfg, B, S)
    return {"tokens": B * S, "ms": round(best * 1e3, 3), "tok_s": round(B * S / best, 1),
            "tflops": round(fl / best / 1e12, 1)}


def motif_prompts(batch, length, vocab, seed, motif=64, subst=0.10):
    """Each sequence tiles its own seeded random ``motif``-token pattern to
    ``length`` tokens, then replaces a ``subst`` fraction of positions with
    uniform random tokens."""
    import torch
    g = torch.Generator().manual_seed(seed)
    out = []
    for _ in range(batch):
        pat = torch.randint(0, vocab, (motif,), generator=g)
        seq = pat.repeat((length + motif - 1) // motif)[:length].clone()
        mask = torch.rand(length, generator=g) < subst
        seq[mask] = torch.randint(0, vocab, (int(mask.sum()),), generator=g)
        out.append(seq.tolist())
    return out


def spec_bench(eng, vocab, batch=4, prompt_len=1024, new_tokens=512, seed=5):
    """Plain vs speculative greedy decode of the same prompts (decode phase
    only: first emitted token to last), and whether the tokens agree."""
    import torch
    prompts = motif_prompts(batch, prompt_len, vocab, seed)
    res = {}
    for spec in (False, True):
        eng.speculate = spec
        for _ in range(2):  # the first call captures the graphs
            toks, t_first = [], None
            for i, step in enumerate(eng.generate(prompts, new_tokens)):
                if i == 0:
                    t_first = time.perf_counter()
                toks.append(step)
            dt = time.perf_counter() - t_first
        res[spec] = (toks, dt)
        log(f"{'speculative' if spec else 'plain'} B={batch} S={prompt_len} N={new_tokens}: "
            f"{dt * 1e3:.1f} ms for {new_tokens - 1} decode steps")
    stats = dict(eng.stats.get("spec", {}))
    n_draft = eng.shape.spec_k if eng.shape is not None else None
    n_tok = batch * (new_tokens - 1)
    # How predictable the plain greedy stream is from its own history: the
    # fraction of generated positions whose trailing 3-gram already occurred
    # earlier in the sequence (prompt included).
    plain_rows = list(map(list, zip(*res[False][0])))
    rep = tot = 0
    for b in range(batch):
        seq = prompts[b] + plain_rows[b]
        seen = {tuple(seq[j:j + 3]) for j in range(len(prompts[b]) - 2)}
        for i in range(len(prompts[b]), len(seq)):
            g3 = tuple(seq[i - 2:i + 1])
            rep += g3 in seen
            tot += 1
            seen.add(g3)
    plain_tps, spec_tps = n_tok / res[False][1], n_tok / res[True][1]
    ceiling = spec_ceiling(eng, prompts, res[False][0], new_tokens, plain_tps)
    log(f"speculation ceiling (drafts = the plain run's tokens): {ceiling}")
    eng.speculate = False
    torch.cuda.empty_cache()
    return {"workload": f"qwen3-4b bf16 bs{batch} motif prompt{prompt_len} new{new_tokens}, drafter n=3/2 k<=8",
            "plain_tok_s": round(plain_tps, 2), "spec_tok_s": round(spec_tps, 2),
            "speedup": round(spec_tps / plain_tps, 3),
            "mean_accept_len": round(stats.get("mean_accept_len", float("nan")), 3),
            "tokens_per_verify": round(stats.get("tokens_per_verify", float("nan")), 3),
            "iterations": stats.get("iterations"),
            "verify_iterations": stats.get("verify_iterations"),
            "plain_iterations": stats.get("plain_iterations"),
            "verify_cost_ratio": stats.get("cost_ratio"),
            "drafts_per_verify": n_draft,
            "draft_hit_rate": round(stats.get("draft_hit_rate", float("nan")), 4),
            "predicted_tokens_per_verify": round(stats.get("predicted_tokens_per_verify", float("nan")), 4),
            "positions_scored": stats.get("positions_scored"),
            "repeated_3gram_frac": round(rep / max(tot, 1), 4),
            "token_identical": res[False][0] == res[True][0],
            "ceiling": ceiling}


def spec_ceiling(eng, prompts, plain_steps, new_tokens, plain_tps):
    """The speculative loop with every draft right: the drafts of an
    iteration are the plain run's next tokens after the sequence's current
    length, written on the device (gather by ``lens``) in place of the n-gram
    drafter; verify, accept, rollback and the host loop are unchanged.
    Tokens must still equal the plain run's."""
    import torch
    from engine import SPEC_BACKOFF, SPEC_PRIMARY
    from qdec.spec import SpecDecoder
    eng.speculate = True
    B, S = len(prompts), len(prompts[0])
    sh = eng._shape_for(B, S, new_tokens)
    k = sh.spec_k
    dev = eng.device
    # future[b, i] = plain token i of sequence b, padded so every gather is in range
    plain = torch.tensor(plain_steps, dtype=torch.int64).T.contiguous()  # [B, N]
    future = torch.cat([plain, plain[:, -1:].expand(B, k + 1)], 1).to(dev)
    offs = torch.arange(1, k + 1, device=dev)[None, :]

    class Forced(SpecDecoder):
        def _draft(self, kk):
            st = self.state
            L = st.lens[:B].long()
            cur = self.hist.gather(1, L[:, None])
            if kk == 0:
                st.ids[:B].copy_(cur[:, 0])
                return
            d = future.gather(1, (L - S)[:, None] + offs[:, :kk])
            self.draft[:B * kk].view(B, kk).copy_(d)
            st.ids[:B * (kk + 1)].view(B, kk + 1).copy_(torch.cat([cur, d], 1))

    dec = Forced(eng, sh.state, SPEC_PRIMARY, SPEC_BACKOFF, k)
    prompt_t = torch.tensor(prompts, dtype=torch.int64)
    for _ in range(2):  # the first call captures the graphs
        toks, t_first = [], None
        for i, step in enumerate(dec.generate(prompt_t, new_tokens, gate=False)):
            if i == 0:
                t_first = time.perf_counter()
            toks.append(step)
        dt = time.perf_counter() - t_first
    stats = dec.last_stats
    tps = B * (new_tokens - 1) / dt
    eng.shape = None
    return {"spec_tok_s": round(tps, 2), "speedup": round(tps / plain_tps, 3),
            "tokens_per_verify": round(stats.get("tokens_per_verify", float("nan")), 3),
            "verify_cost_ratio": stats.get("cost_ratio"), "drafts_per_verify": k,
            "token_identical": toks == plain_steps}


def layer_launch_bench(eng, sh, prompt, new_tokens, steps):
    """The one-launch-per-layer step (qdec_layer) on the headline shape: its
    logit check against the per-operation step (the engine's own gate), then
    both graphs replayed over the same positions, best of 3 rounds."""
    st = sh.state
    B, S = prompt.shape
    st.enable_layer_launch()
    ok, detail = eng._check_mega(st, S)
    st.prefill(prompt)
    layer_graph = eng._capture(lambda: st.step(t_rows=1))
    reps = max(1, min(steps, new_tokens - 2))
    per_op, layer = [], []
    for _ in range(3):
        per_op.append(eng._time_graph(st, sh.graph, S, reps))
        layer.append(eng._time_graph(st, layer_graph, S, reps))
    err = st.layer_error()
    st.disable_layer_launch()
    n = eng.model.cfg.n_layers
    return {"check": detail, "ok": ok, "error_word": err, "steps": reps,
            "per_op_ms_per_step": round(min(per_op), 4), "layer_ms_per_step": round(min(layer), 4),
            "launches_per_step": {"per_op": 5 * n + 2, "layer": n + 2}}


def hbm_fraction(total_bytes, elapsed, ceiling):
    """Achieved algorithmic HBM rate of a timed run, against the nominal
    peak and the streaming-read ceiling measured on this device."""
    tbs = total_bytes / elapsed / 1e12
    out = {"achieved_TBs": round(tbs, 4), "peak_TBs": HBM_PEAK_GBS / 1e3, "frac": round(tbs * 1e3 / HBM_PEAK_GBS, 4)}
    if ceiling:
        out["measured_read_ceiling_TBs"] = round(ceiling / 1e12, 4)
        out["frac_of_measured_ceiling"] = round(tbs * 1e12 / ceiling, 4)
    return out


def generate_tpot(eng, prompt, new_tokens):
    """Time per output token through the public ``generate`` (host loop,
    LOOKAHEAD queueing, pinned-ring copies and events included): from the
    first yielded token to the last, second of two calls (the first captures
    nothing new but warms the host path)."""
    ids = prompt.tolist()
    for _ in range(2):
        t_first = None
        n = 0
        for i, _step in enumerate(eng.generate(ids, new_tokens)):
            if i == 0:
                t_first = time.perf_counter()
            n += 1
        dt = time.perf_counter() - t_first
    tpot = dt / (n - 1)
    return {"tpot_ms": round(tpot * 1e3, 4), "tok_s": round(prompt.shape[0] / tpot, 2), "decode_steps": n - 1,
            "timed": "generate(): first yielded token to the last, wall clock"}


def batched_decode(eng, batch, prompt_len, new_tokens, steps, warmup, seed, ceiling=None):
    """Decode throughput of a batched configuration: its prompts (uniform
    random tokens from ``seed``) are prefilled for real (timed), every
    sequence then sits at ``prompt_len`` cached tokens, and the timed replays
    walk the workload's positions like the headline measurement.  Its
    ``step_hbm``: algorithmic bytes of the positions walked (weights + KV
    read and write) over the timed region."""
    import torch
    mc = eng.model.cfg
    sh = eng._shape_for(batch, prompt_len, new_tokens)
    st = sh.state
    g = torch.Generator().manual_seed(seed)
    prompt = torch.randint(0, mc.vocab, (batch, prompt_len), generator=g).to(eng.device)
    pf = time_prefill(st, prompt)
    log(f"prefill {batch}x{prompt_len}: {pf}")
    last_pos = prompt_len + new_tokens - 2
    span = last_pos - prompt_len + 1
    done = [0]

    def run(k):
        for _ in range(k):
            if done[0] % span == 0 and done[0]:
                st.lens.fill_(prompt_len)
            done[0] += 1
            sh.graph.replay()

    run(warmup)
    done[0] = 0
    wbytes = eng.model.weight_bytes()
    total_bytes = sum(step_bytes(mc, wbytes, batch, prompt_len + i % span) for i in range(steps))
    st.lens.fill_(prompt_len)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    run(steps)
    e1.record()
    torch.cuda.synchronize()
    elapsed = max(time.perf_counter() - t0, e0.elapsed_time(e1) / 1e3)
    kv_bytes = 2 * mc.n_layers * batch * mc.nkv * st.cap * mc.head_dim * 2
    res = {"workload": f"qwen3-4b bf16 bs{batch} prompt{prompt_len} new{new_tokens}",
           "tok_s": round(batch * steps / elapsed, 2), "ms_per_step": round(1e3 * elapsed / steps, 4),
           "steps": steps, "cache": f"prefilled from the prompts, {kv_bytes / 1e9:.1f} GB allocated",
           "step_hbm": dict(hbm_fraction(total_bytes, elapsed, ceiling),
                            bytes_per_step_mean=int(total_bytes / steps)),
           "prefill": pf}
    eng.shape = None
    del sh, st
    torch.cuda.empty_cache()
    return res


def cpu_baseline(ckpt, cfg, prompt_len, budget_s=25.0):
    """Transformers' greedy loop on the host CPU over the same checkpoint
    (bf16, sdpa), bounded: a short prefill, then decode steps until the
    budget or 8 steps.  Falls back to the oracle restatement if Transformers
    is unavailable."""
    import torch
    cores = len(os.sched_getaffinity(0))
    threads = min(cores, 16)
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, cfg["vocab_size"], (1, prompt_len), generator=g)
    try:
        from transformers import AutoModelForCausalLM, DynamicCache
        os.environ.setdefault("USE_HUB_KERNELS", "0")
        t0 = time.perf_counter()
        model = AutoModelForCausalLM.from_pretrained(ckpt, dtype=torch.bfloat16, attn_implementation="sdpa",
                                                     local_files_only=True).eval()
        log(f"cpu baseline: transformers loaded in {time.perf_counter() - t0:.1f}s")
        kind = "reference"
        with torch.no_grad():
            cache = DynamicCache(config=model.config)
            out = model(input_ids=ids, past_key_values=cache, use_cache=True, logits_to_keep=1)
            nxt = out.logits[:, -1].argmax(-1, keepdim=True)
            times = []
            start = time.perf_counter()
            while len(times) < 8 and time.perf_counter() - start < budget_s:
                t = time.perf_counter()
                out = model(input_ids=nxt, past_key_values=cache, use_cache=True, logits_to_keep=1)
                nxt = out.logits[:, -1].argmax(-1, keepdim=True)
                times.append(time.perf_counter() - t)
        what = "transformers Qwen3ForCausalLM bf16 sdpa"
    except ImportError:
        from oracle.qwen3_oracle import Qwen3Oracle
        from qdec.checkpoint import load_tensors
        kind = "port"
        o = Qwen3Oracle(cfg, load_tensors(ckpt), mode="bf16")
        kc, vc = o.new_cache(1, prompt_len + 16)
        nxt = o.forward(ids, [0], kc, vc)[:, -1].argmax(-1, keepdim=True)
        times = []
        start = time.perf_counter()
        while len(times) < 8 and time.perf_counter() - start < budget_s:
            t = time.perf_counter()
            nxt = o.forward(nxt, [prompt_len + len(times)], kc, vc)[:, -1].argmax(-1, keepdim=True)
            times.append(time.perf_counter() - t)
        what = "oracle restatement (torch CPU fp32 with bf16 rounding)"
    times.sort()
    med = times[len(times) // 2]
    return {"value": round(1.0 / med, 4), "unit": "tok/s", "cores": threads, "host_cores": cores,
            "torch_threads": torch.get_num_threads(), "kind": kind,
            "sample": f"{what}; batch 1, prefill {prompt_len} tokens (untimed), then {len(times)} greedy "
                      f"decode steps, median {med:.3f} s/step; same seed-0 checkpoint as the GPU run; "
                      f"{threads} threads of {cores} host cores in this process's affinity"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--ckpt", default=os.environ.get("QDEC_BENCH_CKPT", "/tmp/qdec_qwen3_4b_seed0"))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-spec", action="store_true")
    ap.add_argument("--no-batched", action="store_true")
    ap.add_argument("--no-generate", action="store_true",
                    help="skip timing generate() after the replays (so a kernel trace ends with the timed steps)")
    ap.add_argument("--no-layer", action="store_true",
                    help="skip timing the one-launch-per-layer step (qdec_layer) beside the per-op step")
    ap.add_argument("--pmc-role", choices=ROLES + ("all",),
                    help="only launch this role's kernel over every layer (6 rounds, rows = the "
                         "config's batch; 'all' = every role in turn), then a 512 MiB device copy "
                         "as the counter calibration, for rocprofv3 --pmc")
    ap.add_argument("--pmc-t-rows", type=int, default=1,
                    help="with --pmc-role: rows per sequence of every call (a verify pass: drafts + 1)")
    ap.add_argument("--cpu-prompt", type=int, default=512, help="prompt tokens of the CPU baseline's prefill "
                    "(config 2's 512 by default)")
    ap.add_argument("--prefill-only", type=int, default=0, metavar="REPS",
                    help="only prefill the config's prompts REPS times and print their timing (for profiling)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (every box has one MI355X); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    from engine import Engine
    from qdec.checkpoint import ensure_checkpoint, qwen3_config

    B, S, N, desc = CONFIGS[args.config]
    cfg = qwen3_config()
    t0 = time.perf_counter()
    ensure_checkpoint(args.ckpt, cfg, seed=0)
    log(f"checkpoint ready at {args.ckpt} ({time.perf_counter() - t0:.1f}s)")
    t0 = time.perf_counter()
    eng = Engine(args.ckpt)
    log(f"engine loaded ({time.perf_counter() - t0:.1f}s)")
    mc = eng.model.cfg
    wbytes = eng.model.weight_bytes()

    g = torch.Generator().manual_seed(1)
    prompt = torch.randint(0, mc.vocab, (B, S), generator=g)
    sh = eng._shape_for(B, S, N)
    st = sh.state
    if args.prefill_only:
        pf = time_prefill(st, prompt.to(eng.device), reps=args.prefill_only)
        print(json.dumps({"prefill": pf, "config": desc}), flush=True)
        return
    if args.pmc_role:
        # the config's real prompt, so the attention reads a real cache length
        st.prefill(prompt.to(eng.device))
        for role in (ROLES if args.pmc_role == "all" else (args.pmc_role,)):
            time_gemm_role(eng, st, role, reps=5, t_rows=args.pmc_t_rows)
        src = torch.empty(512 << 20, dtype=torch.uint8, device=eng.device)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"pmc: {args.pmc_role} x {mc.n_layers} layers x 6 rounds, then 6 copies of {src.numel()} bytes")
        return
    prefill = time_prefill(st, prompt.to(eng.device), reps=3)
    log(f"prefill {B}x{S}: {prefill}")
    graph = sh.graph
    last_pos = S + N - 2  # the last decode step of the workload feeds position S+N-2
    span = last_pos - S + 1

    positions = []

    def run(k):
        for _ in range(k):
            p = S + (len(positions) % span)
            if p == S and positions:
                st.lens.fill_(S)
            positions.append(p)
            graph.replay()

    run(args.warmup)
    positions.clear()
    st.lens.fill_(S)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    run(args.steps)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_s = e0.elapsed_time(e1) / 1e3
    elapsed = max(wall, gpu_s)
    tok_s = B * args.steps / elapsed
    ms = 1e3 * elapsed / args.steps
    total_bytes = sum(step_bytes(mc, wbytes, B, p) for p in positions)
    step_tbs = total_bytes / elapsed / 1e12
    log(f"{args.steps} steps: {ms:.4f} ms/step (events {1e3 * gpu_s / args.steps:.4f}), "
        f"{tok_s:.1f} tok/s, {step_tbs:.3f} TB/s algorithmic")

    gen = None if args.no_generate else generate_tpot(eng, prompt, N)
    log(f"generate(): {gen}")
    ceiling = read_ceiling(eng.lib, eng.device)
    log(f"streaming-read ceiling (2 GiB, non-temporal 16-byte loads): {ceiling / 1e12:.3f} TB/s")
    # dominant kernel: gate/up (NORM_IN + GLU), bytes = both weight halves +
    # activations in + act out.
    t_gu = time_gemm_role(eng, st, "gate_up")
    gu_bytes = 2 * mc.inter * mc.hidden * 2 + B * mc.hidden * 2 + B * mc.inter * 2 + mc.hidden * 2
    gu_gbs = gu_bytes / t_gu / 1e9
    log(f"gate_up GEMM: {t_gu * 1e6:.2f} us/launch, {gu_gbs:.1f} GB/s")
    roles = {}
    for role in ("qkv", "attn", "o", "down", "lm"):
        roles[role] = round(time_gemm_role(eng, st, role) * 1e6, 2)
    log(f"other roles us/launch: {roles}")

    layer = None
    if not args.no_layer and st.layer_supported():
        layer = layer_launch_bench(eng, sh, prompt.to(eng.device), N, args.steps)
        log(f"one launch per layer: {layer}")

    batched = {}
    if not args.no_batched:
        del sh, st, graph
        eng.shape = None
        torch.cuda.empty_cache()
        for name, seed in (("c3", 2), ("c4", 3)):
            bB, bS, bN, _ = CONFIGS[name]
            batched[f"batch{bB}"] = r = batched_decode(eng, bB, bS, bN, max(10, args.steps // 4), 3, seed, ceiling)
            log(f"{name}: {r}")

    spec = None
    if not args.no_spec:
        sh = st = graph = None
        eng.shape = None
        torch.cuda.empty_cache()
        spec = spec_bench(eng, mc.vocab)
        log(f"speculation: {spec}")

    cpu = None
    if not args.no_cpu_baseline:
        del eng
        torch.cuda.empty_cache()
        try:
            cpu = cpu_baseline(args.ckpt, cfg, args.cpu_prompt)
        except Exception as exc:  # reported, never fatal for the GPU number
            log(f"cpu baseline failed: {type(exc).__name__}: {exc}")

    line = {
        "metric": "Qwen3-4B bf16 decode tok/s (bs1, bs32) + achieved HBM TB/s vs peak",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init N(0,0.02) weights seed 0, uniform random prompt tokens seed 1)",
        "config": {"workload": desc, "batch": B, "prompt_len": S, "new_tokens": N,
                   "decode_positions": [S, last_pos], "graph": "hipGraph per decode step",
                   "parallelism": "single GPU"},
        "step_hbm": dict(hbm_fraction(total_bytes, elapsed, ceiling),
                         bytes_per_step_mean=int(total_bytes / len(positions))),
        "generate": gen,
        "roofline": {"bound": "hbm", "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / HBM_PEAK_GBS, 4), "traffic": GATE_UP_TRAFFIC_BYTES,
                     "traffic_source": "rocprofv3 FETCH_SIZE + WRITE_SIZE per dispatch, calibrated on a "
                                       "512 MiB copy (profiles/gate_up_hbm_traffic_bs1.md; every role: "
                                       "profiles/decode_hbm_traffic_all_roles.md)",
                     "kernel": "gemm_kernel<1, NORM_IN|GLU> (gate/up, 9728x2x2560)",
                     "algorithmic_bytes_per_launch": gu_bytes,
                     "avg_launch_us": round(t_gu * 1e6, 3)},
        "role_us_per_launch": roles,
        "prefill": prefill,
        "batched": batched or None,
        "layer_launch": layer,
        "speculation": spec,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
