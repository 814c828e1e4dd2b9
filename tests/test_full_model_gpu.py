"""The full Qwen3-4B shape (36 layers) on the GPU, scored against fp32 truth.

Three plans, all through the engine's own decode-step code:

* config 2 of BASELINE.json (below);
* config 3's batched plan (batch 8: 8-wave attention over 416-slot chunks,
  row-major activations), with short prompts;
* config 4's batched plan (batch 32, capacity 4384: one whole-cache
  attention chunk per (sequence, kv head) with 8 waves, attention and SwiGLU
  outputs in fragment order, the down projection split four ways and merged
  by the next NORM_IN call into the other residual buffer, two output tiles
  per wave, the 8-tile lm_head), with short prompts so the CPU references
  stay quick.

the seed-0 random-init checkpoint (the one
bench.py measures, written once to /tmp and reused), batch 1, a 512-token
prompt drawn as bench.py draws it, then decode steps through the engine's
own config-2 plan (capacity 512 + 256 + 2 -> 800, 96-slot attention chunks
merged inside the O projection, 4 attention waves).

The reference point is the oracle in fp32 (``mode="fp32"``: no bf16 rounding
anywhere), which tests/test_oracle.py pins to Transformers fp32 within 5e-7.
Two bf16 implementations are scored against it teacher-forced on the
engine's tokens:

* the engine (bf16 weights and activations, its own summation order);
* Transformers in bf16 (sdpa attention, its default), the reference's
  correctness oracle (engine/engine.py:218-236).

The metric is the normalised max logit error (max |a - b| / max |b| per
row).  At this depth bf16 rounding alone moves the logits by a few percent
of their range, whoever computes them, so the north-star bound of 2e-2 is
not met by either implementation; the assertion is that the engine is no
further from fp32 truth than Transformers bf16 is, with a 25% margin.
Every emitted token must also lie within the reference judge's tie margin
(2.0 logits, QWEN_ENGINE_CONTRACT.md:109-118) of the fp32 argmax.
"""

import time

import pytest
import torch

from oracle.qwen3_oracle import Qwen3Oracle, normalized_max_err
from qdec.checkpoint import ensure_checkpoint, load_tensors, qwen3_config

pytestmark = pytest.mark.gpu

MARGIN = 1.25     # engine error may be at most this multiple of Transformers-bf16's
TIE_MARGIN = 2.0  # logits, the reference judge's tieMarginLogits
CKPT = "/tmp/qdec_qwen3_4b_seed0"


def _say(msg):
    print(f"[full-model] {msg}", flush=True)


def _deficit(ref, toks):
    """How far each emitted token's logit sits below the row's best."""
    return ref.amax(-1) - ref.gather(-1, toks[..., None]).squeeze(-1)


def _run_engine(st, prompt, n):
    """Prefill, then n - 1 plain decode steps; tokens and logits per step."""
    B = prompt.shape[0]
    st.prefill(prompt.to(st.ids.device))
    toks, logits = [st.ids[:B].cpu()], [st.logits[:B].float().cpu()]
    for _ in range(n - 1):
        st.run_step(t_rows=1)
        toks.append(st.ids[:B].cpu())
        logits.append(st.logits[:B].float().cpu())
    torch.cuda.synchronize()
    return torch.stack(toks, 1), torch.stack(logits, 1)


def _score(cfg, prompt, toks, logits, label, t0):
    """The engine's logits and Transformers-bf16's against the fp32 oracle,
    teacher-forced on the engine's tokens; asserts both bounds."""
    n = toks.shape[1]
    tensors = load_tensors(CKPT)
    oracle = Qwen3Oracle(cfg, tensors, mode="fp32")
    with torch.no_grad():
        ref = oracle.teacher_forced(prompt, toks)
    del oracle
    _say(f"{label}: fp32 oracle replayed ({time.perf_counter() - t0:.0f}s)")

    from transformers import AutoModelForCausalLM
    hf = AutoModelForCausalLM.from_pretrained(CKPT, dtype=torch.bfloat16, attn_implementation="sdpa",
                                              local_files_only=True).eval()
    with torch.no_grad():
        hf_logits = hf(input_ids=torch.cat([prompt, toks[:, :-1]], 1), logits_to_keep=n).logits.float()
    del hf, tensors
    _say(f"{label}: transformers bf16 replayed ({time.perf_counter() - t0:.0f}s)")

    err = normalized_max_err(logits, ref)
    err_hf = normalized_max_err(hf_logits, ref)
    _say(f"{label} normalised max err vs fp32: engine {err.max().item():.4f} (mean {err.mean().item():.4f}), "
         f"transformers bf16 {err_hf.max().item():.4f} (mean {err_hf.mean().item():.4f})")
    assert err.max().item() <= MARGIN * err_hf.max().item()
    d = _deficit(ref, toks)
    _say(f"{label} emitted tokens vs fp32 argmax: {int((d > 0).sum())} of {toks.numel()} below it, "
         f"by at most {d.max().item():.4f} logits")
    assert d.max().item() <= TIE_MARGIN


def _engine():
    from engine import Engine
    cfg = qwen3_config()
    assert cfg["num_hidden_layers"] == 36
    ensure_checkpoint(CKPT, cfg, seed=0)
    return cfg, Engine(CKPT)


@pytest.mark.timeout(900)
def test_full_depth_config2_vs_fp32():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")
    from engine import spec_k
    from qdec.runtime import DecodeState

    t0 = time.perf_counter()
    cfg, eng = _engine()
    _say(f"checkpoint ready ({time.perf_counter() - t0:.0f}s)")
    B, S, N, n = 1, 512, 256, 9
    g = torch.Generator().manual_seed(1)  # bench.py's config-2 prompt
    prompt = torch.randint(0, cfg["vocab_size"], (B, S), generator=g)
    st = DecodeState(eng.model, B, S + N + 2 * (spec_k(B) + 1), max_t=16, keep_logits=True)
    assert st.cap == 800 and st.chunk == 96 and st.attn_waves == 4 and st._merge_in_o(1)
    toks, logits = _run_engine(st, prompt, n)
    _say(f"engine: prefill + {n - 1} decode steps ({time.perf_counter() - t0:.0f}s)")
    del st, eng
    torch.cuda.empty_cache()
    _score(cfg, prompt, toks, logits, "B=1", t0)


@pytest.mark.timeout(900)
def test_full_depth_config3_plan_vs_fp32():
    """Config 3's plan at full depth: 8 sequences of 24 tokens in a state of
    config 3's capacity (1024 + 512 + the speculation slack -> 1568): 8-wave
    attention over four 416-slot chunks merged by the last chunk to finish (no
    merge in O past 2 sequences), 8 register-staged rows for QKV and
    row-major activations (below the fragment-order threshold), the down
    projection unsplit; 4 decode steps after the first token."""
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")
    from engine import spec_k
    from qdec.runtime import FRAG_ROWS, DecodeState

    t0 = time.perf_counter()
    cfg, eng = _engine()
    B, S, n = 8, 24, 5
    g = torch.Generator().manual_seed(3)
    prompt = torch.randint(0, cfg["vocab_size"], (B, S), generator=g)
    st = DecodeState(eng.model, B, 1024 + 512 + 2 * (spec_k(B) + 1), max_t=1, keep_logits=True)
    assert st.cap == 1568 and st.chunk == 416 and st.attn_waves == 8 and not st._merge_in_o(1)
    assert B < FRAG_ROWS and st.down_parts is None and st.plans["down"][0] == 1
    toks, logits = _run_engine(st, prompt, n)
    _say(f"engine B={B}: prefill + {n - 1} decode steps ({time.perf_counter() - t0:.0f}s)")
    del st, eng
    torch.cuda.empty_cache()
    _score(cfg, prompt, toks, logits, f"B={B}", t0)


@pytest.mark.timeout(900)
def test_full_depth_config4_plan_vs_fp32():
    """Config 4's plan at full depth: 32 sequences of 24 tokens in a state
    of config 4's capacity (4096 + 256 + 2), 4 decode steps after the first
    token, scored like config 2 above."""
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")
    from qdec.runtime import FRAG_ROWS, DecodeState

    t0 = time.perf_counter()
    cfg, eng = _engine()
    B, S, n = 32, 24, 5
    g = torch.Generator().manual_seed(4)
    prompt = torch.randint(0, cfg["vocab_size"], (B, S), generator=g)
    st = DecodeState(eng.model, B, 4096 + 256 + 2, max_t=1, keep_logits=True)
    assert st.cap == 4384 and st.chunk == 4384 and st.attn_waves == 8 and B >= FRAG_ROWS
    assert st.down_parts is not None and st.plans["down"][0] == 4 and st.plans["qkv"][1] == 4
    toks, logits = _run_engine(st, prompt, n)
    _say(f"engine B={B}: prefill + {n - 1} decode steps ({time.perf_counter() - t0:.0f}s)")
    del st, eng
    torch.cuda.empty_cache()
    _score(cfg, prompt, toks, logits, f"B={B}", t0)
