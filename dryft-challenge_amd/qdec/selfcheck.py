"""Known-answer checks of the kernel library, run once per engine on its device.

The reference checks its kernels when it loads: each Triton path must agree
with the PyTorch path on the real shapes before it is used
(engine/engine.py:296-358 ``_select_kernels`` / ``_agree``, and the fused-step
logit gate at :691-734).  Here every kernel family of a decode step runs once
on inputs whose exact answer is known without a second implementation, with
the model's own packed weights and launch plans, so the same code paths the
step replays are exercised:

* each projection role at one row with a one-hot activation: the output
  column is the weight column, times the normalised one-hot value under
  NORM_IN (one bf16 product, exact in fp32), plus the residual under RES_OUT;
  SwiGLU within one bf16 rounding step; the lm_head's argmax is the lowest
  index of the (often repeated) largest weight of that column;
* the attention at cache length 0: every head's output is the new value row,
  and the value row lands in cache slot 0;
* the n-gram drafter and the acceptance rule on a short history with a
  known match.

A mismatch raises ``QdecError``: the engine never falls back to another
implementation.
"""

import torch

from . import capi


class SelfCheckError(capi.QdecError):
    pass


def _fail(what, detail):
    raise SelfCheckError("self-check", -1, f"{what}: {detail}")


def _tiled_column(w_tiled, n, k, c, device):
    """Column c of the [n, k] matrix stored in the tiled layout of
    include/qdec.h (qdec_tiled_offset), as fp32 [n]."""
    rows = torch.arange(n, device=device)
    lane = rows % 16 + 16 * ((c % 32) // 8)
    off = (((rows // 16) * (k // 32) + c // 32) * 64 + lane) * 8 + c % 8
    return w_tiled.reshape(-1)[off].float()


def _bf16(x):
    return x.to(torch.bfloat16).float()


def run(state):
    """Check every kernel family through ``state`` (a DecodeState): its model,
    launch plans and scratch buffers.  Leaves the state's buffers in an
    arbitrary state (callers prefill before decoding)."""
    m, lib, c = state.model, state.lib, state.model.cfg
    dev = m.device
    s = torch.cuda.current_stream(dev).cuda_stream
    H = c.hidden
    col = 7  # one-hot position (any index below every k)

    def one_hot(k, scale):
        x = torch.zeros((1, k), dtype=torch.bfloat16, device=dev)
        x[0, col] = scale
        return x

    def normalised(k, norm_w):
        # x = e_col: mean of squares 1/k; the normalised value is
        # bf16(w[col] * bf16(rstd)), one product away from every output.
        t = torch.tensor(1.0 / k, dtype=torch.float32)
        rstd = 1.0 / torch.sqrt(t + torch.tensor(c.eps, dtype=torch.float32))
        return float(_bf16(norm_w[col].float().cpu() * _bf16(rstd)))

    # ---- projections, one row, the state's own plans
    for role in ("qkv", "o", "gate_up", "down", "lm"):
        a = state._gemm_args(role, 0, 1, pending=False)
        n, k = a.n, a.k
        x = one_hot(k, 1.0)
        src = {"qkv": state.h, "o": state.attn_out, "gate_up": state.h, "down": state.act, "lm": state.h}[role]
        src[:1, :k].copy_(x)
        w = {"qkv": m.w_qkv[0], "o": m.w_o[0], "gate_up": m.w_gu[0], "down": m.w_down[0], "lm": m.lm_w}[role]
        if role == "down" and a.parts_out:
            # split k, partials left for the next NORM_IN call: the split
            # holding the one-hot column gives the weight column, the others 0
            parts = state.down_parts
            parts.fill_(float("nan"))
            lib.gemm(a, s)
            ks = parts.shape[0]
            want = torch.zeros((ks, n), device=dev)
            want[col // (k // ks)] = _tiled_column(w, n, k, col, dev)
            if not torch.equal(parts[:, 0], want):
                _fail(role, "split partials differ from the weight column")
            continue
        if role in ("o", "down"):
            res0 = torch.linspace(-3, 3, n, device=dev).to(torch.bfloat16)[None]
            state._hb(0)[:1].copy_(res0)
            lib.gemm(a, s)
            got = state._hb(0)[0].float()
            want = _bf16(res0[0].float() + _tiled_column(w, n, k, col, dev))
            if not torch.equal(got, want):
                _fail(role, f"{int((got != want).sum())} of {n} outputs differ from weight column + residual")
            continue
        v = normalised(k, {"qkv": m.in_w[0], "gate_up": m.post_w[0], "lm": m.norm_w}[role])
        if role == "qkv":
            lib.gemm(a, s)
            got = state.qkv[0].float()
            want = _bf16(v * _tiled_column(w, n, k, col, dev))
            if not torch.equal(got, want):
                _fail(role, f"{int((got != want).sum())} of {n} outputs differ from the scaled weight column")
        elif role == "gate_up":
            lib.gemm(a, s)
            got = state.act[0, :n].float()
            wc = _tiled_column(w, 2 * n, k, col, dev)
            g, u = _bf16(v * wc[:n]), _bf16(v * wc[n:])
            want = _bf16(_bf16(g / (1.0 + torch.exp(-g))) * u)
            # expf on the device and exp here may differ by an ulp before
            # the rounding: allow one bf16 step of the larger magnitude.
            step = torch.maximum(got.abs(), want.abs()) * 2.0 ** -7 + 1e-30
            if bool(((got - want).abs() > step).any()):
                _fail(role, "SwiGLU outputs beyond one bf16 rounding step of the one-hot answer")
        else:
            ids = torch.full((1,), -1, dtype=torch.int64, device=dev)
            a = state._gemm_args("lm", 0, 1, ids_out=ids, pending=False)
            lib.gemm(a, s)
            logits = _bf16(v * _tiled_column(w, n, k, col, dev))
            best = logits.max()
            want = int(torch.nonzero(logits == best)[0, 0])
            if int(ids[0]) != want:
                _fail("lm_head", f"argmax {int(ids[0])}, lowest index of the maximum is {want} "
                                 f"({int((logits == best).sum())} tied)")

    # ---- attention at cache length 0: the output is the new value row
    D, G = c.head_dim, c.nq // c.nkv
    g = torch.Generator(device="cpu").manual_seed(1234)
    row = (torch.randn(c.n_qkv, generator=g) * 2).to(torch.bfloat16).to(dev)
    state.qkv[:1].copy_(row[None])
    lens_saved = state.lens.clone()
    state.lens.zero_()
    a = state._attn_args(0, 1)
    lib.attn(a, s)
    v_raw = row[(c.nq + c.nkv) * D:].view(c.nkv, D)
    want = v_raw.repeat_interleave(G, 0).reshape(-1)
    got = state.attn_out[0]
    if not torch.equal(got.view(torch.int16), want.view(torch.int16)):
        _fail("attention", "output at cache length 0 differs from the value row")
    # V cache slot 0 of sequence 0: channel-major [cap/8][D][8], element 0 of each 8
    vs = state.v_cache[0, 0].reshape(c.nkv, state.cap // 8, D, 8)[:, 0, :, 0]
    if not torch.equal(vs.view(torch.int16), v_raw.view(torch.int16)):
        _fail("attention", "value row not written to cache slot 0")
    state.lens.copy_(lens_saved)

    # ---- drafter and acceptance on a history with a known match
    hist = torch.tensor([[5, 6, 7, 8, 9, 5, 6, 7, 0, 0, 0, 0]], dtype=torch.int64, device=dev)
    lens = torch.tensor([7], dtype=torch.int32, device=dev)  # last fed token at index 7
    K = 2
    ids = torch.zeros(K + 1, dtype=torch.int64, device=dev)
    draft = torch.zeros(K, dtype=torch.int64, device=dev)
    d = capi.DraftArgs(hist=hist.data_ptr(), lens=lens.data_ptr(), ids=ids.data_ptr(), draft=draft.data_ptr(),
                       batch=1, cap=hist.shape[1], primary=3, backoff=2, k=K)
    lib.ngram_draft(d, s)
    if ids.tolist() != [7, 8, 9] or draft.tolist() != [8, 9]:
        _fail("ngram_draft", f"ids {ids.tolist()} draft {draft.tolist()}, expected [7, 8, 9] / [8, 9]")
    out_tok = torch.tensor([8, 4, 3], dtype=torch.int64, device=dev)  # first draft right, second wrong
    nacc = torch.zeros(1, dtype=torch.int32, device=dev)
    acc = capi.AcceptArgs(out_tok=out_tok.data_ptr(), draft=draft.data_ptr(), hist=hist.data_ptr(),
                          lens=lens.data_ptr(), naccept=nacc.data_ptr(), batch=1, cap=hist.shape[1], k=K,
                          stop_len=100)
    lib.spec_accept(acc, s)
    if int(nacc[0]) != 1 or int(lens[0]) != 9 or hist[0, 8:10].tolist() != [8, 4]:
        _fail("spec_accept", f"accepted {int(nacc[0])}, length {int(lens[0])}, history {hist[0].tolist()}")
    torch.cuda.synchronize(dev)
