"""BASELINE.json configs[0]'s tiny model through the engine on the GPU,
against the Transformers golden fixtures in tests/golden/.

The fixtures were written by tests/golden/make_golden.py with Transformers'
Qwen3ForCausalLM from the seed-0 tiny checkpoint (head_dim 64, 4 query / 2 kv
heads, hidden 256, vocab 1024, 2 layers, tied embeddings): bf16 greedy runs
with eager and sdpa attention (2 prompts of 24 tokens, 8 new) and an fp32 run
(1 prompt of 32 tokens, 16 new).  The engine loads the same fp32 tensors and
casts them to bf16, as the bf16 fixtures did.  The bar is the one the
reference's contract sets for decode: every greedy token equal (the smallest
top-2 gap in these fixtures is 3% of the row's max |logit|, so no near-tie
excuse applies) and per-step logits within 2e-2 of the row's max |logit|
(QWEN_ENGINE_CONTRACT.md:105-123).  Against the fp32 run the engine's bf16
logits carry bf16 rounding; the oracle in bf16 mode sits 0.012 from them at
worst, under the same bound.
"""

import os

import numpy as np
import pytest
import torch

from oracle.qwen3_oracle import normalized_max_err
from qdec.checkpoint import TINY, generate_tensors

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
TOL = 2e-2


@pytest.fixture(scope="module")
def engine():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")
    from engine import Engine
    eng = Engine.from_tensors(TINY, dict(generate_tensors(TINY, 0, torch.float32)))
    c = eng.model.cfg
    assert (c.head_dim, c.nq, c.nkv, c.vocab) == (64, 4, 2, 1024)
    yield eng
    del eng
    torch.cuda.empty_cache()


def step_logits(engine, prompt, n):
    """Greedy tokens [B, n] and per-step logits [B, n, V] from eager decode
    steps of a DecodeState (the kernels the captured step replays)."""
    from qdec.runtime import DecodeState
    B, S = prompt.shape
    st = DecodeState(engine.model, B, S + n + 8, max_t=16, keep_logits=True)
    st.prefill(prompt.to(engine.device))
    toks, logits = [st.ids[:B].cpu()], [st.logits[:B].float().cpu()]
    for _ in range(n - 1):
        st.run_step(t_rows=1)
        toks.append(st.ids[:B].cpu())
        logits.append(st.logits[:B].float().cpu())
    torch.cuda.synchronize()
    return torch.stack(toks, 1), torch.stack(logits, 1)


@pytest.mark.parametrize("hf_attn", ["eager", "sdpa"])
def test_generate_equals_transformers_bf16(engine, hf_attn):
    fx = np.load(os.path.join(GOLDEN, f"tiny_bf16_{hf_attn}.npz"))
    prompt, want = fx["prompt"], fx["tokens"]
    got = np.array(list(engine.generate(prompt.tolist(), want.shape[1]))).T
    assert got.tolist() == want.tolist()


@pytest.mark.parametrize("hf_attn", ["eager", "sdpa"])
def test_step_logits_vs_transformers_bf16(engine, hf_attn):
    fx = np.load(os.path.join(GOLDEN, f"tiny_bf16_{hf_attn}.npz"))
    ref = torch.from_numpy(fx["step_logits_bits"]).view(torch.bfloat16).float()
    toks, logits = step_logits(engine, torch.from_numpy(fx["prompt"]), ref.shape[1])
    assert toks.tolist() == fx["tokens"].tolist()
    err = normalized_max_err(logits, ref)
    print(f"bf16 {hf_attn}: normalised max err {err.max().item():.4g}")
    assert err.max().item() <= TOL


def test_step_logits_vs_transformers_fp32(engine):
    fx = np.load(os.path.join(GOLDEN, "tiny_fp32.npz"))
    ref = torch.from_numpy(fx["step_logits"])
    toks, logits = step_logits(engine, torch.from_numpy(fx["prompt"]), ref.shape[1])
    assert toks.tolist() == fx["tokens"].tolist()
    err = normalized_max_err(logits, ref)
    print(f"fp32: normalised max err {err.max().item():.4g}")
    assert err.max().item() <= TOL
