"""Other Qwen3 head layouts end to end on the GPU against the oracle.

Qwen3-4B has 4 query heads per kv head; the rest of the family has 2
(0.6B, 1.7B), 5 (14B) or 8 (32B), all at head_dim 128
configs[0]'s tiny model has head_dim 64 with 2 per kv head.  Each case is a
2-layer random checkpoint with that layout (norm weights jittered
N(1, 0.05)), prompts through whichever prefill route the shape takes (the
prefill kernels for 2 and 8 query heads per kv head at head_dim 128, the
decode kernels otherwise), then decode steps with logits, judged
teacher-forced as tests/test_engine_gpu.py judges Qwen3-4B: logits within
2e-2 of the row's max |logit|, every token the oracle's argmax or a
documented near-tie.  Batch 8 runs the 8-wave attention.  The 40/8 and 64/8
cases have their own lm_head.weight (untied, as Qwen3-14B and -32B).
"""

import pytest
import torch

from oracle.qwen3_oracle import Qwen3Oracle, normalized_max_err, top2_gap
from qdec.checkpoint import load_tensors, qwen3_config, write_checkpoint

pytestmark = pytest.mark.gpu

TOL = 2e-2

SHAPES = {
    # Qwen3-1.7B widths: 16 query heads / 8 kv heads
    "g2": dict(hidden_size=2048, intermediate_size=6144, num_attention_heads=16, num_key_value_heads=8),
    # Qwen3-14B's head layout (40 / 8) at a smaller width, untied lm_head as 14B
    "g5": dict(hidden_size=1024, intermediate_size=3072, num_attention_heads=40, num_key_value_heads=8,
               tie_word_embeddings=False),
    # Qwen3-32B's head layout (64 / 8) at a smaller width, untied lm_head as 32B
    "g8": dict(hidden_size=1024, intermediate_size=3072, num_attention_heads=64, num_key_value_heads=8,
               tie_word_embeddings=False),
    # BASELINE.json configs[0]'s tiny model: head_dim 64, 4 / 2 heads, vocab 1024
    "tiny": dict(hidden_size=256, intermediate_size=768, num_attention_heads=4, num_key_value_heads=2, head_dim=64,
                 vocab_size=1024, tie_word_embeddings=True),
}


@pytest.fixture(scope="module", params=sorted(SHAPES))
def model(request, tmp_path_factory):
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")
    from engine import Engine
    cfg = qwen3_config(num_hidden_layers=2, **SHAPES[request.param])
    path = str(tmp_path_factory.mktemp(f"qwen3_{request.param}"))
    write_checkpoint(path, cfg, seed=5, norm_jitter=0.05)
    eng = Engine(path)
    ora = Qwen3Oracle(cfg, load_tensors(path), mode="bf16", attn="decode")
    yield request.param, cfg, eng, ora, path
    del eng
    torch.cuda.empty_cache()


def run_state(engine, prompt, n):
    """Eager steps with logits kept: (tokens [B, n], logits [B, n, V])."""
    from qdec.runtime import DecodeState
    B, S = prompt.shape
    st = DecodeState(engine.model, B, S + n + 18, max_t=16, keep_logits=True)
    st.prefill(prompt.to(engine.device))
    toks, logits = [st.ids[:B].cpu()], [st.logits[:B].float().cpu()]
    for _ in range(n - 1):
        st.run_step(t_rows=1)
        toks.append(st.ids[:B].cpu())
        logits.append(st.logits[:B].float().cpu())
    torch.cuda.synchronize()
    assert st.lens.cpu().tolist() == [S + n - 1] * B
    return torch.stack(toks, 1), torch.stack(logits, 1), st


# (1, 300): 96-slot chunks, so the attention's chunks are merged by the last
# arriving workgroup (merging in O takes 4 query heads per kv head only).
@pytest.mark.parametrize("B,S,n,seed", [(1, 40, 6, 71), (3, 21, 5, 72), (8, 17, 4, 73), (1, 300, 4, 74)])
def test_head_layouts_vs_oracle(model, B, S, n, seed):
    name, cfg, eng, ora, _ = model
    c = eng.model.cfg
    assert c.group == cfg["num_attention_heads"] // cfg["num_key_value_heads"]
    assert (eng.model.lm_w is eng.model.emb) == bool(cfg["tie_word_embeddings"])
    g = torch.Generator().manual_seed(seed)
    prompt = torch.randint(0, cfg["vocab_size"], (B, S), generator=g)
    toks, logits, st = run_state(eng, prompt, n)
    assert st.max_t * c.group <= (32 if st.attn_waves == 8 else 64)
    if S == 300:
        assert st.cap // st.chunk >= 3
    assert not st._merge_in_o(1) or c.group == 4
    ref = ora.teacher_forced(prompt, toks)
    err = normalized_max_err(logits, ref)
    print(f"{name} B={B} S={S}: normalised max err {err.max().item():.4g}, prefill kernels {c.prefill_kernels}")
    assert err.max().item() <= TOL
    mism = ref.argmax(-1) != toks
    near = top2_gap(ref) < TOL * ref.abs().amax(-1)
    assert bool((~mism | near).all()), f"non-near-tie divergence: {mism.nonzero().tolist()}"


def test_head_layouts_generate_and_speculate(model):
    """generate through the captured graph, plainly and with every step a
    verify pass (the speculative engine with its gate open): the same tokens,
    with verify rows within the attention's query rows per kv head."""
    name, cfg, eng, _, path = model
    from engine import Engine
    spec = Engine.from_tensors(cfg, load_tensors(path), speculate=True)
    spec.spec_gate = False  # always verify
    g = torch.Generator().manual_seed(81)
    for B, S in ((2, 30), (1, 200)):  # (1, 200): verify rows over several attention chunks
        prompt = torch.randint(0, cfg["vocab_size"], (B, S), generator=g)
        plain = list(eng.generate(prompt.tolist(), 8))
        fast = list(spec.generate(prompt.tolist(), 8))
        assert fast == plain, (name, B, S)
        assert spec.stats["spec"]["plain_iterations"] == 0
