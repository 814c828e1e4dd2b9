"""Seeded random-init Qwen3 checkpoints in the Hugging Face directory layout.

``write_checkpoint(path, cfg, seed)`` writes ``config.json`` plus
``model.safetensors`` that both this engine (``Engine(path)``) and
Transformers (``from_pretrained(path, local_files_only=True)``) load.  The
init follows Transformers' ``_init_weights`` (modeling_utils.py:2391-2419):
every Linear and Embedding weight ~ N(0, initializer_range = 0.02), RMSNorm
weights = 1.  ``norm_jitter > 0`` instead draws the norm weights from
N(1, norm_jitter), so that a norm gain read from the wrong layer changes the
output (the reference's tiny-model test does the same,
tests/test_engine_cpu.py:43-59).

The draws are counter-based: every tensor, and every 16 Mi-element chunk of
it, has its own PCG64 stream derived from (seed, tensor index, chunk index),
so the bytes do not depend on the thread count and a 4 B-parameter
checkpoint generates in seconds on a multi-core host.
"""

import concurrent.futures as cf
import json
import os

import numpy as np
import torch

QWEN3_4B = {
    "architectures": ["Qwen3ForCausalLM"],
    "model_type": "qwen3",
    "hidden_size": 2560,
    "intermediate_size": 9728,
    "num_hidden_layers": 36,
    "num_attention_heads": 32,
    "num_key_value_heads": 8,
    "head_dim": 128,
    "vocab_size": 151936,
    "max_position_embeddings": 262144,
    "rms_norm_eps": 1e-6,
    "rope_theta": 5000000.0,
    "rope_parameters": {"rope_type": "default", "rope_theta": 5000000.0},
    "tie_word_embeddings": True,
    "hidden_act": "silu",
    "attention_bias": False,
    "attention_dropout": 0.0,
    "initializer_range": 0.02,
    "use_cache": True,
    "torch_dtype": "bfloat16",
    "bos_token_id": 151643,
    "eos_token_id": 151645,
}

# the reference's CPU-runnable plumbing model.
TINY = dict(QWEN3_4B, hidden_size=256, intermediate_size=768, num_hidden_layers=2,
            num_attention_heads=4, num_key_value_heads=2, head_dim=64, vocab_size=1024,
            torch_dtype="float32", bos_token_id=1, eos_token_id=2,
            max_position_embeddings=4096)

CHUNK = 1 << 24


def qwen3_config(**overrides):
    """Qwen3-4B config dict with keyword overrides (e.g. fewer layers)."""
    cfg = dict(QWEN3_4B)
    cfg.update(overrides)
    return cfg


def param_shapes(cfg):
    """(name, shape, kind) of every parameter, in generation order."""
    H, I = cfg["hidden_size"], cfg["intermediate_size"]
    nq, nkv = cfg["num_attention_heads"], cfg["num_key_value_heads"]
    D = cfg.get("head_dim") or H // nq
    out = [("model.embed_tokens.weight", (cfg["vocab_size"], H), "normal")]
    for i in range(cfg["num_hidden_layers"]):
        p = f"model.layers.{i}."
        out += [
            (p + "input_layernorm.weight", (H,), "norm"),
            (p + "self_attn.q_proj.weight", (nq * D, H), "normal"),
            (p + "self_attn.k_proj.weight", (nkv * D, H), "normal"),
            (p + "self_attn.v_proj.weight", (nkv * D, H), "normal"),
            (p + "self_attn.o_proj.weight", (H, nq * D), "normal"),
            (p + "self_attn.q_norm.weight", (D,), "norm"),
            (p + "self_attn.k_norm.weight", (D,), "norm"),
            (p + "post_attention_layernorm.weight", (H,), "norm"),
            (p + "mlp.gate_proj.weight", (I, H), "normal"),
            (p + "mlp.up_proj.weight", (I, H), "normal"),
            (p + "mlp.down_proj.weight", (H, I), "normal"),
        ]
    out.append(("model.norm.weight", (H,), "norm"))
    if not cfg.get("tie_word_embeddings", False):  # untied unless stated, as the runtime reads it
        out.append(("lm_head.weight", (cfg["vocab_size"], H), "normal"))
    return out


def _fill_normal(out, seed, index, pool):
    n = out.size
    nchunks = (n + CHUNK - 1) // CHUNK

    def one(c):
        ss = np.random.SeedSequence([seed, index, c])
        g = np.random.Generator(np.random.PCG64(ss))
        g.standard_normal(out=out[c * CHUNK:min(n, (c + 1) * CHUNK)], dtype=np.float32)

    list(pool.map(one, range(nchunks)))


def generate_tensors(cfg, seed, dtype=torch.bfloat16, std=None, norm_jitter=0.0, threads=None):
    """Yield (name, tensor) of a seeded random init, one tensor at a time."""
    std = cfg.get("initializer_range", 0.02) if std is None else std
    threads = threads or max(1, min(16, len(os.sched_getaffinity(0))))
    with cf.ThreadPoolExecutor(threads) as pool:
        for idx, (name, shape, kind) in enumerate(param_shapes(cfg)):
            n = int(np.prod(shape))
            if kind == "norm" and norm_jitter <= 0:
                t = torch.ones(shape, dtype=torch.float32)
            else:
                buf = np.empty(n, dtype=np.float32)
                _fill_normal(buf, seed, idx, pool)
                t = torch.from_numpy(buf).view(shape)
                if kind == "norm":
                    t = 1.0 + norm_jitter * t
                else:
                    t = t * std
            yield name, t.to(dtype)


def write_checkpoint(path, cfg, seed=0, dtype=torch.bfloat16, norm_jitter=0.0, std=None):
    """Write ``config.json`` and ``model.safetensors`` under ``path``."""
    from safetensors.torch import save_file

    os.makedirs(path, exist_ok=True)
    cfg = dict(cfg)
    cfg["torch_dtype"] = {torch.bfloat16: "bfloat16", torch.float32: "float32",
                          torch.float16: "float16"}[dtype]
    tensors = dict(generate_tensors(cfg, seed, dtype, std=std, norm_jitter=norm_jitter))
    save_file(tensors, os.path.join(path, "model.safetensors"), metadata={"format": "pt"})
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(cfg, f, indent=2, sort_keys=True)
    with open(os.path.join(path, "qdec_seed.json"), "w") as f:
        json.dump({"seed": seed, "norm_jitter": norm_jitter, "std": std}, f)
    return path


def ensure_checkpoint(path, cfg, seed=0, dtype=torch.bfloat16, norm_jitter=0.0):
    """Write the checkpoint unless ``path`` already holds the same one."""
    stamp = os.path.join(path, "qdec_seed.json")
    if os.path.exists(stamp) and os.path.exists(os.path.join(path, "model.safetensors")):
        try:
            with open(stamp) as f:
                meta = json.load(f)
            with open(os.path.join(path, "config.json")) as f:
                old = json.load(f)
            same_cfg = all(old.get(k) == v for k, v in cfg.items() if k != "torch_dtype")
            if meta.get("seed") == seed and meta.get("norm_jitter") == norm_jitter and same_cfg:
                return path
        except (OSError, ValueError):
            pass
    return write_checkpoint(path, cfg, seed, dtype, norm_jitter)


def load_config(path):
    with open(os.path.join(path, "config.json")) as f:
        return json.load(f)


def load_tensors(path, device="cpu"):
    """All tensors of a checkpoint directory (``*.safetensors``)."""
    from safetensors.torch import load_file

    out = {}
    for fn in sorted(os.listdir(path)):
        if fn.endswith(".safetensors"):
            out.update(load_file(os.path.join(path, fn), device=device))
    return out
