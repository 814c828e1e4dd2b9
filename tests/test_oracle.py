"""The oracle, pinned: Transformers golden fixtures (tiny config, fp32 and
bf16) plus closed forms and invariants chosen so that a dropped term, a wrong
sign or a misplaced cast fails one of them."""

import json
import os

import numpy as np
import pytest
import torch

from oracle.qwen3_oracle import (Qwen3Oracle, apply_rope, argmax_lowest, attention, bf16, head_norm_rope,
                                 linear, normalized_max_err, rms_norm, rope_tables, rotate_half, silu_mul)
from qdec.checkpoint import TINY, generate_tensors

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _meta():
    with open(os.path.join(GOLDEN, "golden_meta.json")) as f:
        return json.load(f)


def _digest(cfg, seed, dtype, jitter):
    import hashlib
    h = hashlib.sha256()
    for name, t in generate_tensors(cfg, seed, dtype, norm_jitter=jitter):
        h.update(name.encode())
        h.update(t.contiguous().view(torch.uint8).numpy().tobytes())
    return h.hexdigest()


@pytest.fixture(scope="module")
def tiny_tensors():
    return {jit: dict(generate_tensors(TINY, 0, torch.float32, norm_jitter=jit)) for jit in (0.0, 0.05)}


# ------------------------------------------------------------ golden vectors

@pytest.mark.parametrize("tag,jit", [("tiny", 0.0), ("tiny_jitter", 0.05)])
def test_checkpoint_matches_fixture_weights(tag, jit):
    assert _digest(TINY, 0, torch.float32, jit) == _meta()[f"{tag}_fp32"]["sha256"]


@pytest.mark.parametrize("tag,jit", [("tiny", 0.0), ("tiny_jitter", 0.05)])
def test_fp32_matches_transformers(tiny_tensors, tag, jit):
    """fp32 mode = Transformers fp32 (eager) to float rounding: tokens exact,
    cached-loop logits and the teacher-forced replay within 1e-5."""
    fx = np.load(os.path.join(GOLDEN, f"{tag}_fp32.npz"))
    o = Qwen3Oracle(TINY, tiny_tensors[jit], mode="fp32")
    prompt = torch.from_numpy(fx["prompt"])
    toks, logits = o.greedy(prompt, 16)
    assert toks.tolist() == fx["tokens"].tolist()
    assert (torch.stack(logits, 1) - torch.from_numpy(fx["step_logits"])).abs().max() < 1e-5
    tf = o.teacher_forced(prompt, torch.from_numpy(fx["tokens"]))
    assert (tf - torch.from_numpy(fx["tf_logits"])).abs().max() < 1e-5


def test_fp32_chunked_prefill_is_same(tiny_tensors):
    fx = np.load(os.path.join(GOLDEN, "tiny_fp32.npz"))
    o = Qwen3Oracle(TINY, tiny_tensors[0.0], mode="fp32")
    toks, _ = o.greedy(torch.from_numpy(fx["prompt"]), 16, chunk=5)
    assert toks.tolist() == fx["tokens"].tolist()


def test_rope_tables_match_transformers():
    fx = np.load(os.path.join(GOLDEN, "tiny_fp32.npz"))
    c, s = rope_tables(48, 64, 5e6, "fp32")
    assert torch.equal(c, torch.from_numpy(fx["cos"])) and torch.equal(s, torch.from_numpy(fx["sin"]))
    fb = np.load(os.path.join(GOLDEN, "tiny_bf16_eager.npz"))
    c, s = rope_tables(48, 64, 5e6, "bf16")
    assert torch.equal(c, torch.from_numpy(fb["cos_bits"]).view(torch.bfloat16).float())
    assert torch.equal(s, torch.from_numpy(fb["sin_bits"]).view(torch.bfloat16).float())


def test_engine_rope_tables_equal_oracle():
    from qdec.runtime import rope_tables as engine_rope
    c, s = engine_rope(300, 128, 5e6)
    oc, os_ = rope_tables(300, 128, 5e6, "bf16")
    assert torch.equal(c.float(), oc) and torch.equal(s.float(), os_)


@pytest.mark.parametrize("hf_attn", ["eager", "sdpa"])
@pytest.mark.parametrize("attn", ["eager", "decode"])
def test_bf16_matches_transformers(tiny_tensors, hf_attn, attn):
    """bf16 mode vs Transformers in bf16: same greedy tokens, per-step
    logits within 2e-2 of the row's max |logit| (only summation order
    differs), and the eager restatement of eager is mostly bit-exact."""
    fx = np.load(os.path.join(GOLDEN, f"tiny_bf16_{hf_attn}.npz"))
    ref = torch.from_numpy(fx["step_logits_bits"]).view(torch.bfloat16).float()
    tb = {k: v.to(torch.bfloat16) for k, v in tiny_tensors[0.0].items()}
    o = Qwen3Oracle(TINY, tb, mode="bf16", attn=attn)
    toks, logits = o.greedy(torch.from_numpy(fx["prompt"]), 8)
    assert toks.tolist() == fx["tokens"].tolist()
    lg = torch.stack(logits, 1)
    assert normalized_max_err(lg, ref).max() < 2e-2
    if attn == hf_attn == "eager":
        assert (lg == ref).float().mean() > 0.6


# ------------------------------------------------------- closed forms / KATs

def test_bf16_rounding_is_rne():
    x = torch.tensor([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -9, -(1.0 + 2 ** -8)])
    assert bf16(x).tolist() == [1.0, 1.0 + 2 ** -6, 1.0, -1.0]


def test_rms_norm_cast_point():
    """w * bf16(h * rstd), not bf16(w * h * rstd): a weight that is not a power
    of two tells the two apart (cf. the reference's cast-boundary test,
    tests/test_kernels_sim.py:234-271)."""
    g = torch.Generator().manual_seed(3)
    h = bf16(torch.randn(4, 256, generator=g) * 3)
    w = bf16(1 + 0.3 * torch.randn(256, generator=g))
    y = rms_norm(h, w, 1e-6)
    hf = h.double()
    n = (hf * torch.rsqrt((hf * hf).mean(-1, keepdim=True) + 1e-6)).float()
    assert torch.equal(y, bf16(w * bf16(n)))
    assert not torch.equal(y, bf16(w * n))
    # unit weights: output rms ~= 1
    y1 = rms_norm(h, torch.ones(256), 1e-6)
    assert torch.allclose((y1 * y1).mean(-1), torch.ones(4), atol=2e-2)


def test_linear_identity_and_one_hot():
    x = bf16(torch.randn(3, 64))
    assert torch.equal(linear(x, torch.eye(64)), x)
    w = torch.zeros(5, 64)
    w[2, 7] = 1.0
    assert torch.equal(linear(x, w)[:, 2], x[:, 7])
    # brute force on tiny k: fp32 sum of products, one rounding
    xs, ws = bf16(torch.randn(2, 8)), bf16(torch.randn(3, 8))
    ref = torch.tensor([[sum(float(xs[i, j]) * float(ws[o, j]) for j in range(8)) for o in range(3)] for i in range(2)])
    assert torch.allclose(linear(xs, ws, "fp32"), ref.float(), atol=1e-5)


def test_rope_position_zero_and_rotation():
    c, s = rope_tables(64, 128, 5e6, "bf16")
    assert torch.all(c[0] == 1) and torch.all(s[0] == 0)
    y = bf16(torch.randn(2, 128))
    assert torch.equal(apply_rope(y, c[0], s[0]), y)  # pos 0 = identity
    # rotate_half sign: first half takes -x2
    x = torch.arange(8.0)
    assert rotate_half(x).tolist() == [-4.0, -5.0, -6.0, -7.0, 0.0, 1.0, 2.0, 3.0]
    # fp32 rotation preserves the norm of every (i, i + d/2) pair
    cf, sf = rope_tables(64, 128, 5e6, "fp32")
    z = torch.randn(128)
    r = apply_rope(z, cf[37], sf[37], "fp32")
    assert torch.allclose(r.norm(), z.norm(), rtol=1e-5)
    assert torch.allclose(r[:64] ** 2 + r[64:] ** 2, z[:64] ** 2 + z[64:] ** 2, rtol=1e-4, atol=1e-6)


def test_head_norm_then_rope_order():
    c, s = rope_tables(16, 128, 5e6, "bf16")
    x = bf16(torch.randn(128) * 5)
    w = bf16(1 + 0.2 * torch.randn(128))
    out = head_norm_rope(x, w, c[9], s[9], 1e-6)
    assert torch.equal(out, apply_rope(rms_norm(x, w, 1e-6), c[9], s[9]))
    assert not torch.equal(out, rms_norm(apply_rope(x, c[9], s[9]), w, 1e-6))


def test_attention_invariants():
    g = torch.Generator().manual_seed(5)
    q = bf16(torch.randn(4, 128, generator=g))
    k = bf16(torch.randn(10, 128, generator=g))
    v = bf16(torch.randn(10, 128, generator=g))
    one = torch.zeros(4, 10, dtype=torch.bool)
    one[:, 0] = True
    assert torch.equal(attention(q, k, v, one, 128 ** -0.5), v[0].expand(4, 128))  # one slot -> V
    kz = torch.zeros_like(k)
    allv = torch.ones(4, 10, dtype=torch.bool)
    mean = bf16(v.sum(0) / 10)
    assert torch.allclose(attention(q, kz, v, allv, 128 ** -0.5), mean.expand(4, 128), atol=1e-2)
    # decode and eager formulations agree to bf16 precision, fp32 to softmax
    ref = torch.softmax((q @ k.T) * 128 ** -0.5, -1) @ v
    for attn in ("decode", "eager"):
        assert (attention(q, k, v, allv, 128 ** -0.5, attn=attn) - ref).abs().max() < 3e-2


def test_silu_mul_closed_form():
    g = bf16(torch.tensor([0.0, 1.0, -2.0, 10.0]))
    u = bf16(torch.tensor([1.0, 2.0, 3.0, 0.5]))
    out = silu_mul(g, u)
    s = [x / (1 + np.exp(-x)) for x in g.tolist()]
    exp = bf16(bf16(torch.tensor(s, dtype=torch.float32)) * u)
    assert torch.equal(out, exp)
    assert out[0] == 0


def test_argmax_lowest_ties():
    x = torch.tensor([[1.0, 3.0, 3.0, 2.0], [5.0, 5.0, 5.0, 5.0], [-1.0, -2.0, -1.0, -3.0]])
    assert argmax_lowest(x).tolist() == [1, 0, 0]
    r = torch.randn(7, 1000)
    assert torch.equal(argmax_lowest(r), r.argmax(-1))
