"""The full Qwen3-4B shape (36 layers) on the GPU against the oracle and
against Transformers.

The 2-layer engine tests pin every kernel at full widths within 2e-2 of the
row's max |logit|. Over the real depth, bf16 results computed in different
summation orders drift apart. Measured with this test's prompt, as the
normalised max logit error:

| Depth | engine vs oracle | engine vs Transformers | oracle vs Transformers |
|---|---:|---:|---:|
| 2 layers | 0.009 | 0.015 | 0.015 |
| 8 layers | 0.017 | 0.024 | 0.023 |
| 36 layers | 0.036 | 0.040 | 0.041 |

So no implementation with another summation order meets 2e-2 at 36 layers,
not even the oracle against Transformers. The full-depth checks are:
* the engine's logits are no further from the oracle than Transformers'
  (bf16, eager attention, the same checkpoint) are;
* every emitted token is within the reference contract's tie margin (2.0
  logits) of the argmax of both replays (QWEN_ENGINE_CONTRACT.md:109-118).
  With random-init weights, logits span about +-5, so near ties are common.

The checkpoint is the same seed-0 random-init one as bench.py's, written
once to /tmp and reused when present.
"""

import time

import pytest
import torch

from oracle.qwen3_oracle import Qwen3Oracle, normalized_max_err
from qdec.checkpoint import ensure_checkpoint, load_tensors, qwen3_config

pytestmark = pytest.mark.gpu

TOL = 2e-2
TIE_MARGIN = 2.0  # logits, the reference judge's tieMarginLogits
CKPT = "/tmp/qdec_qwen3_4b_seed0"


def _say(msg):
    print(f"[full-model] {msg}", flush=True)


def _deficit(ref, toks):
    """How far each emitted token's logit sits below the row's best."""
    return ref.amax(-1) - ref.gather(-1, toks[..., None]).squeeze(-1)


def test_full_depth_logits_and_tokens():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")
    from engine import Engine
    from qdec.runtime import DecodeState

    t0 = time.perf_counter()
    cfg = qwen3_config()
    assert cfg["num_hidden_layers"] == 36
    ensure_checkpoint(CKPT, cfg, seed=0)
    _say(f"checkpoint ready ({time.perf_counter() - t0:.0f}s)")
    eng = Engine(CKPT)
    B, S, n = 2, 24, 5
    g = torch.Generator().manual_seed(21)
    prompt = torch.randint(0, cfg["vocab_size"], (B, S), generator=g)
    st = DecodeState(eng.model, B, S + n + 18, max_t=16, keep_logits=True)
    st.prefill(prompt.to(eng.device))
    toks, logits = [st.ids[:B].cpu()], [st.logits[:B].float().cpu()]
    for _ in range(n - 1):
        st.run_step(t_rows=1)
        toks.append(st.ids[:B].cpu())
        logits.append(st.logits[:B].float().cpu())
    torch.cuda.synchronize()
    toks, logits = torch.stack(toks, 1), torch.stack(logits, 1)
    _say(f"engine decoded {n} steps ({time.perf_counter() - t0:.0f}s)")
    del st, eng
    torch.cuda.empty_cache()

    oracle = Qwen3Oracle(cfg, load_tensors(CKPT), mode="bf16", attn="decode")
    ref = oracle.teacher_forced(prompt, toks)
    del oracle
    _say(f"oracle replayed ({time.perf_counter() - t0:.0f}s)")

    from transformers import AutoModelForCausalLM
    hf = AutoModelForCausalLM.from_pretrained(CKPT, dtype=torch.bfloat16, attn_implementation="eager",
                                              local_files_only=True).eval()
    with torch.no_grad():
        hf_logits = hf(input_ids=torch.cat([prompt, toks[:, :-1]], 1)).logits[:, S - 1:].float()
    del hf
    _say(f"transformers replayed ({time.perf_counter() - t0:.0f}s)")

    err = normalized_max_err(logits, ref).max().item()
    spread = normalized_max_err(hf_logits, ref).max().item()
    _say(f"normalised max err: engine vs oracle {err:.4f}, transformers vs oracle {spread:.4f}")
    assert err <= max(TOL, spread)
    for name, r in (("oracle", ref), ("transformers", hf_logits)):
        d = _deficit(r, toks)
        _say(f"emitted tokens vs {name}: {int((d > 0).sum())} of {toks.numel()} below the argmax, "
             f"by at most {d.max().item():.4f} logits")
        assert d.max().item() <= TIE_MARGIN
