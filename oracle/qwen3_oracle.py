"""CPU restatement of Qwen3 greedy decode -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module, and only as the checker.  The
product path (``dryft-challenge_amd/``) never imports it; it fails loudly
when its HIP library is missing instead of falling back to anything here.

What it restates
----------------
The Transformers Qwen3 forward (the reference engine's correctness oracle,
engine/engine.py:218-236 loads it; its maths is in
transformers/models/qwen3/modeling_qwen3.py, pinned at 4.51.3 by
requirements.txt:11, read here from the installed 5.15.0 whose Qwen3 maths is
unchanged), with every bf16 materialisation made explicit:

* RMSNorm            TF :59-64   ``w * bf16(h * rsqrt(mean(h^2) + eps))``, then
                                  bf16 (the product of two bf16 tensors);
* rotary tables      TF :106-137 ``inv_freq = 1/theta^(2i/d)``; ``freqs = pos *
                                  inv_freq`` (fp32); cos/sin fp32 then bf16;
* RoPE               TF :148-170 ``bf16(bf16(y*cos) + bf16(rotate_half(y)*sin))``;
* q/k head norm      TF :246-247 RMSNorm over head_dim before RoPE;
* attention          TF :183-204 (eager) -- see ``attention``;
* MLP                TF :81-83   ``bf16(bf16(silu(g)) * u)``;
* residual adds      TF :310-325 rounded to bf16;
* linear layers      fp32 accumulation of bf16 products, one rounding;
* lm_head            tied to the embedding (engine/engine.py:266-269).

``mode="fp32"`` drops every rounding (an fp32 checkpoint run by Transformers
in fp32), which pins the wiring against Transformers' own outputs.

The decode-attention formulation (``attn="decode"``) is the reference
engine's kernel maths (engine/kernels/ops.py:275-339 with one split): fp32
scores, fp32 max/exp, probabilities rounded to bf16 before the P.V product,
fp32 accumulation, one rounding of the output.  ``attn="eager"`` is
Transformers' eager_attention_forward in bf16 (scores rounded, softmax in
fp32 then bf16, bf16 P.V).

Parity pins (tests/test_oracle.py): Transformers golden fixtures for the tiny
configuration in fp32 and bf16 (tests/golden/), closed forms and invariants
of every function below.  None is "parity unpinned".
"""

import torch

__all__ = [
    "bf16", "rms_norm", "linear", "rope_tables", "rotate_half", "apply_rope",
    "head_norm_rope", "attention", "silu_mul", "argmax_lowest", "Qwen3Oracle",
]


def bf16(x):
    """Round an fp32 tensor to bf16 precision (RNE) and return it as fp32."""
    return x.to(torch.bfloat16).to(torch.float32)


def _r(x, mode):
    return bf16(x) if mode == "bf16" else x


def rms_norm(h, w, eps, mode="bf16"):
    """Qwen3RMSNorm, TF modeling_qwen3.py:59-64 (and ops.py:71-76).

    ``h`` holds the bf16 values of the input in fp32; the variance is the fp32
    mean of squares, the normalised value is rounded to bf16 *before* the
    weight multiply, and the product is rounded again."""
    hf = h.to(torch.float32)
    var = (hf * hf).mean(-1, keepdim=True)
    n = hf * torch.rsqrt(var + eps)
    if mode == "bf16":
        return bf16(w * bf16(n))
    return w * n


def linear(x, w, mode="bf16"):
    """``x @ w.T`` with fp32 accumulation and one rounding (nn.Linear in bf16)."""
    return _r(x.to(torch.float32) @ w.to(torch.float32).T, mode)


def rope_tables(cap, head_dim, theta, mode="bf16"):
    """cos/sin ``[cap, head_dim]``, TF modeling_qwen3.py:106-137.

    ``freqs[p, i] = fl(p * inv_freq[i])`` -- one fp32 product, as the
    ``[d/2, 1] @ [1, cap]`` matmul of the reference computes it."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).to(torch.float32) / head_dim))
    pos = torch.arange(cap, dtype=torch.float32)
    freqs = pos[:, None] * inv_freq[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    cos, sin = emb.cos(), emb.sin()
    return _r(cos, mode), _r(sin, mode)


def rotate_half(x):
    """TF modeling_qwen3.py:140-144: ``cat(-x[..., d/2:], x[..., :d/2])``."""
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_rope(y, cos, sin, mode="bf16"):
    """TF modeling_qwen3.py:148-170, each product and the sum rounded."""
    return _r(_r(y * cos, mode) + _r(rotate_half(y) * sin, mode), mode)


def head_norm_rope(x, w, cos, sin, eps, mode="bf16"):
    """Per-head RMSNorm (q_norm / k_norm, TF :246-247) followed by RoPE.
    ``x`` is ``[..., head_dim]``; ``cos``/``sin`` broadcast against it."""
    return apply_rope(rms_norm(x, w, eps, mode), cos, sin, mode)


def attention(q, k, v, visible, scale, mode="bf16", attn="decode"):
    """Masked attention of query rows over key slots.

    ``q`` ``[..., R, D]``, ``k``/``v`` ``[..., S, D]`` (bf16 values in fp32),
    ``visible`` a bool mask broadcastable to ``[..., R, S]``.

    * ``decode``: fp32 scores, fp32 softmax numerator against the row max,
      numerators rounded to bf16 before P.V, fp32 accumulation, division by
      the fp32 sum, one rounding (ops.py:275-339 single split).
    * ``eager``: TF eager_attention_forward (TF :183-204) in bf16.
    """
    neg = torch.tensor(float("-inf"))
    if mode != "bf16":
        s = (q @ k.transpose(-1, -2)) * scale
        s = torch.where(visible, s, neg)
        return torch.softmax(s, dim=-1) @ v
    if attn == "eager":
        s = bf16(bf16(q @ k.transpose(-1, -2)) * scale)
        s = torch.where(visible, s, neg)
        p = bf16(torch.softmax(s, dim=-1))
        return bf16(p @ v)
    s = (q @ k.transpose(-1, -2)) * scale
    s = torch.where(visible, s, neg)
    m = s.max(dim=-1, keepdim=True).values
    e = torch.exp(s - m)
    return bf16((bf16(e) @ v) / e.sum(dim=-1, keepdim=True))


def silu_mul(g, u, mode="bf16"):
    """Qwen3MLP activation, TF modeling_qwen3.py:81-83 (ops.py:265-267):
    ``bf16(bf16(silu(g)) * u)`` with ``silu(g) = g / (1 + exp(-g))``."""
    return _r(_r(g / (1.0 + torch.exp(-g)), mode) * u, mode)


def argmax_lowest(logits):
    """Greedy pick with ties to the lowest index (torch.argmax semantics,
    engine/engine.py:492-498).  Restated as a scan so it does not depend on
    torch.argmax itself: the first index whose value equals the row max."""
    mx = logits.max(dim=-1, keepdim=True).values
    hit = logits == mx
    idx = torch.arange(logits.shape[-1]).expand_as(logits)
    return torch.where(hit, idx, logits.shape[-1]).min(dim=-1).values


class Qwen3Oracle:
    """Greedy decode over a static KV cache, restated on the CPU.

    ``tensors`` maps Hugging Face parameter names to tensors (any float dtype;
    bf16 checkpoints stay exactly representable in fp32).  ``cfg`` is the HF
    config dict."""

    def __init__(self, cfg, tensors, mode="bf16", attn="decode"):
        self.mode, self.attn = mode, attn
        self.hidden = cfg["hidden_size"]
        self.inter = cfg["intermediate_size"]
        self.n_layers = cfg["num_hidden_layers"]
        self.nq = cfg["num_attention_heads"]
        self.nkv = cfg["num_key_value_heads"]
        self.d = cfg.get("head_dim") or self.hidden // self.nq
        self.vocab = cfg["vocab_size"]
        self.eps = cfg.get("rms_norm_eps", 1e-6)
        rp = cfg.get("rope_parameters") or {}
        self.theta = float(rp.get("rope_theta", cfg.get("rope_theta", 10000.0)))
        self.scale = self.d ** -0.5
        f = lambda name: tensors[name].to(torch.float32)  # noqa: E731
        self.embed = f("model.embed_tokens.weight")
        self.lm = f("lm_head.weight") if "lm_head.weight" in tensors else self.embed
        self.norm = f("model.norm.weight")
        self.layers = []
        for i in range(self.n_layers):
            p = f"model.layers.{i}."
            self.layers.append({
                "in": f(p + "input_layernorm.weight"),
                "post": f(p + "post_attention_layernorm.weight"),
                "q": f(p + "self_attn.q_proj.weight"),
                "k": f(p + "self_attn.k_proj.weight"),
                "v": f(p + "self_attn.v_proj.weight"),
                "o": f(p + "self_attn.o_proj.weight"),
                "qn": f(p + "self_attn.q_norm.weight"),
                "kn": f(p + "self_attn.k_norm.weight"),
                "g": f(p + "mlp.gate_proj.weight"),
                "u": f(p + "mlp.up_proj.weight"),
                "dn": f(p + "mlp.down_proj.weight"),
            })
        self.cos = self.sin = None

    # -------------------------------------------------------------- caches
    def new_cache(self, batch, cap):
        self._ensure_rope(cap)
        shape = (self.n_layers, batch, self.nkv, cap, self.d)
        return torch.zeros(shape), torch.zeros(shape)

    def _ensure_rope(self, cap):
        if self.cos is None or self.cos.shape[0] < cap:
            self.cos, self.sin = rope_tables(cap, self.d, self.theta, self.mode)

    # ------------------------------------------------------------- forward
    def forward(self, ids, lens, kc, vc, last=None):
        """Feed ``ids`` ``[B, T]``; row ``t`` of sequence ``b`` sits at
        position ``lens[b] + t`` and sees cache slots ``0 .. lens[b] + t``.
        Writes K/V of the new slots into ``kc``/``vc`` and returns the
        logits ``[B, T, V]`` (bf16 values in fp32 in bf16 mode), or only
        those of the last ``last`` rows ``[B, last, V]``."""
        mode = self.mode
        B, T = ids.shape
        lens = torch.as_tensor(lens, dtype=torch.int64).reshape(B)
        pos = lens[:, None] + torch.arange(T)[None, :]              # [B, T]
        cap = kc.shape[3]
        self._ensure_rope(cap)
        cos, sin = self.cos[pos][:, :, None, :], self.sin[pos][:, :, None, :]  # [B,T,1,D]
        slots = torch.arange(cap)
        visible = slots[None, None, :] <= pos[:, :, None]            # [B, T, cap]
        h = self.embed[ids]                                          # [B, T, H]
        G = self.nq // self.nkv
        for i, ly in enumerate(self.layers):
            x = rms_norm(h, ly["in"], self.eps, mode)
            q = linear(x, ly["q"], mode).view(B, T, self.nq, self.d)
            k = linear(x, ly["k"], mode).view(B, T, self.nkv, self.d)
            v = linear(x, ly["v"], mode).view(B, T, self.nkv, self.d)
            q = head_norm_rope(q, ly["qn"], cos, sin, self.eps, mode)
            k = head_norm_rope(k, ly["kn"], cos, sin, self.eps, mode)
            for b in range(B):
                kc[i, b, :, pos[b]] = k[b].transpose(0, 1)
                vc[i, b, :, pos[b]] = v[b].transpose(0, 1)
            # [B, nkv, G*T, D] query rows grouped by kv head
            qg = q.permute(0, 2, 1, 3).reshape(B, self.nkv, G, T, self.d).reshape(B, self.nkv, G * T, self.d)
            vis = visible[:, None, None, :, :].expand(B, 1, G, T, cap).reshape(B, 1, G * T, cap)
            o = attention(qg, kc[i], vc[i], vis, self.scale, mode, self.attn)
            o = o.reshape(B, self.nkv, G, T, self.d).permute(0, 3, 1, 2, 4).reshape(B, T, self.nq * self.d)
            h = _r(h + linear(o, ly["o"], mode), mode)
            x = rms_norm(h, ly["post"], self.eps, mode)
            a = silu_mul(linear(x, ly["g"], mode), linear(x, ly["u"], mode), mode)
            h = _r(h + linear(a, ly["dn"], mode), mode)
        if last is not None:
            h = h[:, T - last:]
        return linear(rms_norm(h, self.norm, self.eps, mode), self.lm, mode)

    # ------------------------------------------------------------- drivers
    def greedy(self, prompt, n_new, chunk=None):
        """Plain greedy decode: prefill, then one token per step.

        Returns ``(tokens [B, n_new], step_logits list of [B, V])`` where
        step ``i`` holds the logits that produced token ``i``."""
        prompt = torch.as_tensor(prompt, dtype=torch.int64)
        B, S = prompt.shape
        kc, vc = self.new_cache(B, S + n_new)
        chunk = chunk or S
        logits = None
        for c0 in range(0, S, chunk):
            ids = prompt[:, c0:c0 + chunk]
            logits = self.forward(ids, [c0] * B, kc, vc)[:, -1]
        toks, step_logits = [], []
        cur = argmax_lowest(logits)
        for i in range(n_new):
            toks.append(cur)
            step_logits.append(logits)
            if i == n_new - 1:
                break
            logits = self.forward(cur[:, None], [S + i] * B, kc, vc)[:, 0]
            cur = argmax_lowest(logits)
        return torch.stack(toks, 1), step_logits

    def teacher_forced(self, prompt, generated):
        """Logits at every generated position, feeding ``prompt`` then
        ``generated[:, :-1]`` in one pass (the judge's replay,
        tests/test_engine_cpu.py:118-140 of the reference).  Returns
        ``[B, N, V]`` where row ``i`` predicts ``generated[:, i]``."""
        prompt = torch.as_tensor(prompt, dtype=torch.int64)
        generated = torch.as_tensor(generated, dtype=torch.int64)
        B, S = prompt.shape
        N = generated.shape[1]
        seq = torch.cat([prompt, generated[:, :-1]], dim=1)
        kc, vc = self.new_cache(B, S + N)
        return self.forward(seq, [0] * B, kc, vc, last=N)


def normalized_max_err(a, b):
    """The logit agreement metric of the parity tests: ``max|a - b| /
    max|b|`` per row (the scale of engine/engine.py:349-358 ``_agree``)."""
    a, b = a.to(torch.float32), b.to(torch.float32)
    return ((a - b).abs().max(dim=-1).values / b.abs().max(dim=-1).values.clamp_min(1e-30))


def top2_gap(logits):
    """Gap between the two largest logits of each row."""
    top = logits.to(torch.float32).topk(2, dim=-1).values
    return top[..., 0] - top[..., 1]
