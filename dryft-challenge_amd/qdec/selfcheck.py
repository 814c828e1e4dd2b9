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


# --------------------------------------------------------------- per shape
def _tiled_rows(w_tiled, n, k, rows):
    """Rows ``rows`` (int64 tensor) of the [n, k] matrix stored in the tiled
    layout of include/qdec.h, as fp32 [len(rows), k]."""
    r = rows[:, None]
    c = torch.arange(k, device=rows.device)[None, :]
    lane = r % 16 + 16 * ((c % 32) // 8)
    off = (((r // 16) * (k // 32) + c // 32) * 64 + lane) * 8 + c % 8
    return w_tiled.reshape(-1)[off].float()


def _frag_index(rows, cols, device):
    """Flat offsets of elements (m, c) of a [rows, cols] matrix written in
    the fragment order of include/qdec.h (x_frag / out_frag)."""
    nmt = (rows + 15) // 16
    m = torch.arange(rows, device=device)[:, None]
    c = torch.arange(cols, device=device)[None, :]
    return (((c // 32) * nmt + m // 16) * 64 + m % 16 + 16 * ((c % 32) // 8)) * 8 + c % 8


def _put_rows(buf, rows, frag):
    """Write ``rows`` [R, k] into activation buffer ``buf`` (row-major, or in
    fragment order); the rest of the buffer is zeroed."""
    R, k = rows.shape
    flat = buf.view(-1)
    flat.zero_()
    if frag:
        flat[_frag_index(R, k, buf.device).reshape(-1)] = rows.reshape(-1).to(buf.dtype)
    else:
        flat[:R * k] = rows.reshape(-1).to(buf.dtype)


def _get_rows(buf, R, k, frag):
    flat = buf.view(-1)
    if frag:
        return flat[_frag_index(R, k, buf.device).reshape(-1)].view(R, k)
    return flat[:R * k].view(R, k)


def _shape_gemms(state, t):
    """Every projection role of a step over B*t rows, one-hot rows at
    distinct columns, through the state's own launch plans and buffers
    (fragment-order hand-overs, the down projection's k split and the merge
    of its partials in the next NORM_IN call, two tiles per wave, the
    lm_head's tile grouping and argmax keys)."""
    m, lib, c = state.model, state.lib, state.model.cfg
    dev = m.device
    s = torch.cuda.current_stream(dev).cuda_stream
    R = state.batch * t
    rows_i = torch.arange(R, device=dev)
    L = c.n_layers
    split = state.down_parts is not None

    def cols(k):
        return (7 + 37 * rows_i) % k  # distinct for every k here (k >= 64, gcd(37, k) = 1 or k > 37 * 63)

    def one_hot(k):
        x = torch.zeros((R, k), dtype=torch.bfloat16, device=dev)
        x[rows_i, cols(k)] = 1.0
        return x

    def wcols(w, n, k):
        """[R, n]: row m holds column cols(k)[m] of the tiled [n, k] matrix."""
        cc = cols(k)
        nn = torch.arange(n, device=dev)[None, :]
        ci = cc[:, None]
        lane = nn % 16 + 16 * ((ci % 32) // 8)
        off = (((nn // 16) * (k // 32) + ci // 32) * 64 + lane) * 8 + ci % 8
        return w.reshape(-1)[off].float()

    def scale(k, norm_w):
        """bf16(norm_w[c] * bf16(rstd)) of a one-hot row at column c, per row."""
        tk = torch.tensor(1.0 / k, dtype=torch.float32)
        rstd = _bf16(1.0 / torch.sqrt(tk + torch.tensor(c.eps, dtype=torch.float32)))
        return _bf16(norm_w.float()[cols(k)].cpu() * rstd).to(dev)[:, None]

    def set_residual(a, layer, k):
        """x of a NORM_IN call at the start of ``layer``: the one-hot rows,
        or (down split) zero rows plus one-hot split partials, which the call
        merges into x_merged first."""
        if a.x_parts:
            # (with a split O the down projection's update belongs to hpost)
            (state._hb(layer - 1) if state.o_parts is None else state.hpost)[:R].zero_()
            parts = split_parts()
            state.down_parts.zero_()
            parts[rows_i % parts.shape[0], rows_i, cols(k)] = 1.0
            state._hb(layer)[:R].fill_(float("nan"))
        else:
            state._hb(layer)[:R].copy_(one_hot(k))

    def split_parts(buf=None):
        # a split projection's partials of an R-row call: [ks][R][hidden]
        buf = state.down_parts if buf is None else buf
        ks = buf.shape[0]
        return buf.view(-1)[:ks * R * c.hidden].view(ks, R, c.hidden)

    def check_merged(a, layer, k, role):
        if a.x_parts and not torch.equal(state._hb(layer)[:R].float(), one_hot(k).float()):
            _fail(role, f"{R} rows: the merged residual differs from the split partials' sum")

    # QKV (layer 1 when the down projection splits: the merge of its partials)
    lq = 1 if (split and L > 1) else 0
    a = state._gemm_args("qkv", lq, R)
    set_residual(a, lq, c.hidden)
    lib.gemm(a, s)
    check_merged(a, lq, c.hidden, "qkv")
    want = _bf16(scale(c.hidden, m.in_w[lq]) * wcols(m.w_qkv[lq], c.n_qkv, c.hidden))
    if not torch.equal(state.qkv[:R].float(), want):
        _fail("qkv", f"{R} rows: {int((state.qkv[:R].float() != want).sum())} outputs differ")

    # O: residual + weight column, or the k split's partials
    a = state._gemm_args("o", 0, R)
    kq = c.nq * c.head_dim
    _put_rows(state.attn_out, one_hot(kq), a.x_frag)
    res0 = (torch.linspace(-3, 3, c.hidden, device=dev)[None] + 0.25 * rows_i[:, None]).to(torch.bfloat16)
    wo = wcols(m.w_o[0], c.hidden, kq)
    if a.parts_out:
        state.o_parts.fill_(float("nan"))
        lib.gemm(a, s)
        parts = split_parts(state.o_parts)
        ko = parts.shape[0]
        want = torch.zeros((ko, R, c.hidden), device=dev)
        want[cols(kq) // (kq // ko), rows_i] = wo
        if not torch.equal(parts, want):
            _fail("o", f"{R} rows: split partials differ from the weight column")
    else:
        state._hb(0)[:R].copy_(res0)
        lib.gemm(a, s)
        want = _bf16(res0.float() + wo)
        if not torch.equal(state._hb(0)[:R].float(), want):
            _fail("o", f"{R} rows: {int((state._hb(0)[:R].float() != want).sum())} outputs differ "
                       "from weight column + residual")

    # gate/up + SwiGLU (output in fragment order from FRAG_ROWS rows); with a
    # split O it first merges one-hot split partials into hpost
    a = state._gemm_args("gate_up", 0, R)
    if a.x_parts:
        state._hb(0)[:R].zero_()
        parts = split_parts(state.o_parts)
        state.o_parts.zero_()
        parts[rows_i % parts.shape[0], rows_i, cols(c.hidden)] = 1.0
        state.hpost[:R].fill_(float("nan"))
    else:
        state._hb(0)[:R].copy_(one_hot(c.hidden))
    lib.gemm(a, s)
    if a.x_parts and not torch.equal(state.hpost[:R].float(), one_hot(c.hidden).float()):
        _fail("gate_up", f"{R} rows: the merged residual differs from the split partials' sum")
    got = _get_rows(state.act, R, c.inter, a.out_frag).float()
    wc = wcols(m.w_gu[0], 2 * c.inter, c.hidden)
    v = scale(c.hidden, m.post_w[0])
    g, u = _bf16(v * wc[:, :c.inter]), _bf16(v * wc[:, c.inter:])
    want = _bf16(_bf16(g / (1.0 + torch.exp(-g))) * u)
    step = torch.maximum(got.abs(), want.abs()) * 2.0 ** -7 + 1e-30
    if bool(((got - want).abs() > step).any()):
        _fail("gate_up", f"{R} rows: SwiGLU outputs beyond one bf16 rounding step of the one-hot answer")

    # down: residual + weight column, or the k split's partials
    a = state._gemm_args("down", 0, R)
    _put_rows(state.act, one_hot(c.inter), a.x_frag)
    wdn = wcols(m.w_down[0], c.hidden, c.inter)
    if a.parts_out:
        state.down_parts.fill_(float("nan"))
        lib.gemm(a, s)
        parts = split_parts()
        ks = parts.shape[0]
        want = torch.zeros((ks, R, c.hidden), device=dev)
        want[cols(c.inter) // (c.inter // ks), rows_i] = wdn
        if not torch.equal(parts, want):
            _fail("down", f"{R} rows: split partials differ from the weight column")
    else:
        state._hb(0)[:R].copy_(res0)
        lib.gemm(a, s)
        want = _bf16(res0.float() + wdn)
        if not torch.equal(state._hb(0)[:R].float(), want):
            _fail("down", f"{R} rows: outputs differ from weight column + residual")

    # final norm + lm_head + argmax (merging the last down projection's split)
    ids = torch.full((R,), -1, dtype=torch.int64, device=dev)
    inc = torch.zeros((R,), dtype=torch.int32, device=dev)
    a = state._gemm_args("lm", 0, R, ids_out=ids, lens_inc=inc if t == 1 else None)
    set_residual(a, L, c.hidden)
    lib.gemm(a, s)
    check_merged(a, L, c.hidden, "lm_head")
    logits = _bf16(scale(c.hidden, m.norm_w) * wcols(m.lm_w, c.vocab, c.hidden))
    best = logits.max(-1, keepdim=True).values
    idx = torch.arange(c.vocab, device=dev)[None].expand(R, -1)
    want = torch.where(logits == best, idx, c.vocab).min(-1).values
    if not torch.equal(ids, want):
        bad = int((ids != want).sum())
        _fail("lm_head", f"{R} rows: {bad} argmax ids differ from the lowest index of each row's maximum")
    if t == 1 and not bool((inc == 1).all()):
        _fail("lm_head", f"{R} rows: cache lengths not advanced by one")


def _shape_attention(state, t):
    """The attention of a step over t rows per sequence, through the state's
    chunking, wave count, output order (or the O projection's merge of its
    partials): every query row is (1, 1) on the lowest-frequency RoPE pair,
    the new keys are zero and one cached key per (sequence, kv head) -- at a
    slot spread over the chunks -- points along the rotated query, so that
    slot's softmax weight is 1 and every other weight underflows to exactly
    0.  The output is then that slot's value row, bit for bit, whatever the
    chunk or wave that holds it; the new rows' values land in the cache."""
    m, lib, c = state.model, state.lib, state.model.cfg
    dev = m.device
    s = torch.cuda.current_stream(dev).cuda_stream
    B, D, nkv, nq, cap = state.batch, c.head_dim, c.nkv, c.nq, state.cap
    G = nq // nkv
    R = B * t
    g = torch.Generator(device="cpu").manual_seed(4242 + R)
    gd = torch.Generator(device=dev).manual_seed(4243 + R)
    # the lowest-frequency pairs (rotation angle ~1e-6 per position); the
    # one whose q-norm weights are largest carries the query
    qw = m.q_norm[0].float().cpu()
    half = D // 2
    j = max(range(8), key=lambda i: float(qw[half - 1 - i].abs() + qw[D - 1 - i].abs()))
    i1, i2 = half - 1 - j, D - 1 - j
    rstd = 1.0 / (2.0 / D + c.eps) ** 0.5
    q1, q2 = float(qw[i1]) * rstd, float(qw[i2]) * rstd
    if abs(q1) + abs(q2) < 1e-3:
        _fail("attention", "q-norm weights of the lowest-frequency RoPE pairs are all ~0; no known-answer query")
    # scores of the hot slot ~ 400 in log2 units: every other weight is exp2(<= -400) = 0
    alpha = 400.0 / ((D ** -0.5) * 1.4426950408889634 * (abs(q1) + abs(q2)))
    lens = [max(1, cap - t - 1 - (37 * b) % max(1, cap // 4)) for b in range(B)]
    hot = torch.tensor([[((b * 131 + h * 71 + 11) * 977) % lens[b] for h in range(nkv)] for b in range(B)])
    kc, vc = state.k_cache[0], state.v_cache[0]
    kc.zero_()
    hot_key = torch.zeros(D, dtype=torch.float32)
    hot_key[i1] = alpha * (1.0 if q1 >= 0 else -1.0)
    hot_key[i2] = alpha * (1.0 if q2 >= 0 else -1.0)
    bi = torch.arange(B)[:, None].expand(B, nkv).reshape(-1).to(dev)
    hi = torch.arange(nkv)[None, :].expand(B, nkv).reshape(-1).to(dev)
    hs = hot.reshape(-1).to(dev)
    kc[bi, hi, hs] = hot_key.to(torch.bfloat16).to(dev)
    vc.copy_(torch.randn(vc.shape, generator=gd, device=dev).to(torch.bfloat16))
    v8 = vc.view(B, nkv, cap // 8, D, 8)  # channel-major: slot s, channel d at [s // 8, d, s % 8]
    qkv = torch.zeros((R, c.n_qkv), dtype=torch.bfloat16)
    qkv[:, [h * D + i1 for h in range(nq)]] = 1.0
    qkv[:, [h * D + i2 for h in range(nq)]] = 1.0
    vnew = torch.randn(R, nkv * D, generator=g).to(torch.bfloat16)
    qkv[:, (nq + nkv) * D:] = vnew
    state.qkv[:R].copy_(qkv.to(dev))
    state.lens.copy_(torch.tensor(lens, dtype=torch.int32, device=dev))
    # the expected rows: [R, nq * D]
    hv = v8[bi, hi, hs // 8, :, hs % 8].view(B, nkv, D)
    want = hv.repeat_interleave(G, 1).reshape(B, 1, nq * D).expand(B, t, nq * D).reshape(R, nq * D)
    pm = state._merge_in_o(t)
    a = state._attn_args(0, t, partials=pm)
    if pm:
        # partials merged by the O projection: its output must equal O over
        # the known rows fed the ordinary way
        state.attn_out.fill_(7.0)
        lib.attn(a, s)
        res0 = torch.linspace(-2, 2, c.hidden, device=dev).to(torch.bfloat16)[None].expand(R, -1)
        state._hb(0)[:R].copy_(res0)
        lib.gemm(state._gemm_args("o", 0, R, x_attn=a), s)
        got = state._hb(0)[:R].clone()
        o = state._gemm_args("o", 0, R)
        _put_rows(state.attn_out, want, o.x_frag)
        state._hb(0)[:R].copy_(res0)
        lib.gemm(o, s)
        if not torch.equal(got.view(torch.int16), state._hb(0)[:R].view(torch.int16)):
            _fail("attention", f"{R} rows: the O projection's merge of the chunk partials differs from the "
                               "known attention output")
    else:
        lib.attn(a, s)
        got = _get_rows(state.attn_out, R, nq * D, a.out_frag)
        if not torch.equal(got.view(torch.int16), want.view(torch.int16)):
            bad = int((got.view(torch.int16) != want.view(torch.int16)).any(-1).sum())
            _fail("attention", f"{R} rows (chunk {state.chunk}, {state.attn_waves} waves): {bad} rows differ "
                               "from the hot slot's value row")
    # the new rows' values and (zero) keys in the cache
    pos = torch.tensor(lens)[:, None] + torch.arange(t)[None, :]  # [B, t]
    b3 = torch.arange(B)[:, None, None].expand(B, t, nkv).reshape(-1).to(dev)
    h3 = torch.arange(nkv)[None, None, :].expand(B, t, nkv).reshape(-1).to(dev)
    p3 = pos[:, :, None].expand(B, t, nkv).reshape(-1).to(dev)
    vs = v8[b3, h3, p3 // 8, :, p3 % 8].view(B, t, nkv, D)
    if not torch.equal(vs.reshape(R, nkv * D).view(torch.int16).cpu(), vnew.view(torch.int16)):
        _fail("attention", f"{R} rows: new value rows not written to their cache slots")
    if bool((kc[b3, h3, p3] != 0).any()):
        _fail("attention", f"{R} rows: new (zero) key rows not written to their cache slots")
    kc.zero_()
    vc.zero_()
    state.lens.zero_()


def run_shape(state, t_rows=(1,)):
    """Known-answer checks of one decode shape's own launch plans, on its own
    buffers, before it serves (the reference checks each new shape's fused
    step against its plain step before using it, engine/engine.py:691-734,
    778, 891-925): for every row count the shape replays (``t_rows`` rows per
    sequence: 1 for plain decode, k + 1 for a verify pass) the embedding
    gather, all five projection roles and the attention run through
    ``state``'s plans -- attention waves and chunking, fragment-order
    hand-overs, the down projection's k split and its merge, several tiles
    per wave, the lm_head's grouping and argmax.  Raises SelfCheckError on a
    mismatch; leaves the cache zeroed and the other buffers arbitrary
    (callers prefill before decoding)."""
    m, lib, c = state.model, state.lib, state.model.cfg
    dev = m.device
    s = torch.cuda.current_stream(dev).cuda_stream
    for t in t_rows:
        R = state.batch * t
        # embedding gather
        ids = (torch.arange(R, device=dev, dtype=torch.int64) * 7919 + 13) % c.vocab
        state.ids[:R].copy_(ids)
        e = capi.EmbedArgs(ids=state.ids.data_ptr(), emb=m.emb.data_ptr(), h=state.h.data_ptr(), rows=R,
                           hidden=c.hidden, vocab=c.vocab)
        lib.embed(e, s)
        if not torch.equal(state.h[:R].float(), _tiled_rows(m.emb, c.vocab, c.hidden, ids)):
            _fail("embed", f"{R} rows: gathered rows differ from the embedding")
        _shape_gemms(state, t)
        _shape_attention(state, t)
    torch.cuda.synchronize(dev)
