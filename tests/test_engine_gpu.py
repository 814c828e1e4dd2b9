"""The engine end to end on the GPU against the oracle.

Model: Qwen3-4B widths (hidden 2560, intermediate 9728, 32 q / 8 kv heads,
head_dim 128, vocab 151936, tied, theta 5e6) with 2 layers, seeded random
init, norm weights jittered N(1, 0.05) so a norm applied at the wrong place
shows.  Parity is judged teacher-forced on the engine's own tokens, as the
reference's judge replays a submission (QWEN_ENGINE_CONTRACT.md:105-123):

* per-step logits within 2e-2 of the row's max |logit| (normalised max err);
* every emitted token is the oracle's argmax, or the oracle's top-2 gap at
  that step is below the tolerance (a documented near-tie);
* the graph-replayed generate, the eager step and the speculative path emit
  identical tokens.
"""

import os

import pytest
import torch

from oracle.qwen3_oracle import Qwen3Oracle, normalized_max_err, top2_gap
from qdec.checkpoint import load_tensors, qwen3_config, write_checkpoint

pytestmark = pytest.mark.gpu

TOL = 2e-2


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")
    cfg = qwen3_config(num_hidden_layers=2)
    path = str(tmp_path_factory.mktemp("qwen3_l2"))
    write_checkpoint(path, cfg, seed=0, norm_jitter=0.05)
    return path, cfg


@pytest.fixture(scope="module")
def engine(ckpt):
    from engine import Engine
    return Engine(ckpt[0])


@pytest.fixture(scope="module")
def oracle(ckpt):
    path, cfg = ckpt
    return Qwen3Oracle(cfg, load_tensors(path), mode="bf16", attn="decode")


def prompts(B, S, seed, vocab=151936):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, vocab, (B, S), generator=g)


def run_state(engine, prompt, n):
    """Eager runtime steps with logits kept: (tokens [B, n], logits [B, n, V])."""
    from qdec.runtime import DecodeState
    B, S = prompt.shape
    st = DecodeState(engine.model, B, S + n + 18, max_t=16, keep_logits=True)
    st.prefill(prompt.to(engine.device))
    first_logits = st.logits[:B].float().cpu()
    toks = [st.ids[:B].cpu()]
    logits = [first_logits]
    for _ in range(n - 1):
        st.run_step(t_rows=1)
        toks.append(st.ids[:B].cpu())
        logits.append(st.logits[:B].float().cpu())
    torch.cuda.synchronize()
    assert st.lens.cpu().tolist() == [S + n - 1] * B
    return torch.stack(toks, 1), torch.stack(logits, 1)


# B = 48 and 64 run three and four M tiles per GEMM (the lm_head one tile
# per workgroup); 64 rows is the most a step takes.
# B = 32 and 20 run the batched step of config 4 (>= 17 rows): attention
# over one whole-cache chunk per (sequence, kv head) with 8 waves and its
# output in fragment order, the O / down projections reading fragment order,
# the normalisation pre-passes of QKV / gate/up / lm_head, SwiGLU written in
# fragment order, and the 8-tile lm_head + argmax.  B = 12 runs the 8-wave
# attention over two 512-slot chunks merged by the last arriver.
@pytest.mark.parametrize("B,S,n,seed", [(1, 40, 10, 1), (3, 21, 8, 2), (8, 17, 5, 4), (32, 300, 4, 31),
                                        (20, 150, 4, 32), (12, 700, 3, 33), (48, 60, 3, 34), (64, 40, 3, 35)])
def test_logits_and_tokens_vs_oracle(engine, oracle, B, S, n, seed):
    if B >= 17:
        from qdec.runtime import FRAG_ROWS, DecodeState
        st = DecodeState(engine.model, B, S + n + 18, max_t=16)
        assert st.chunk == st.cap and st.attn_waves == 8 and B >= FRAG_ROWS
        del st
    prompt = prompts(B, S, seed)
    toks, logits = run_state(engine, prompt, n)
    ref = oracle.teacher_forced(prompt, toks)  # [B, n, V]
    err = normalized_max_err(logits, ref)
    print(f"B={B} S={S}: normalised max err {err.max().item():.4g}, mean {err.mean().item():.4g}")
    assert err.max().item() <= TOL
    ref_pick = ref.argmax(-1)
    gap = top2_gap(ref)
    mism = (ref_pick != toks)
    near = gap < TOL * ref.abs().amax(-1)
    assert bool((~mism | near).all()), f"non-near-tie divergence: {mism.nonzero().tolist()}"


def v_rows(v):
    """Rows [..., cap, D] of a V cache stored channel-major ([..., cap/8, D, 8]
    in the same memory)."""
    *lead, cap, d = v.shape
    return v.reshape(*lead, cap // 8, d, 8).transpose(-1, -2).reshape(*lead, cap, d)


@pytest.mark.parametrize("B,S,seed", [(1, 100, 11), (3, 70, 12), (2, 12, 13), (1, 16, 14), (1, 40, 15), (3, 21, 16)])
def test_prefill_vs_oracle_and_chunking(engine, oracle, B, S, seed):
    """The prefill against the oracle's forward over the whole prompt
    (first-token logits and the filled K/V slots), against the decode-kernel
    route, and bit for bit against itself in 16-position chunks.  Prompts
    one decode step holds (12 and 16 tokens here) take the decode-kernel
    route themselves; prompts of at most PREFILL_SKINNY_ROWS rows (40 and
    3 x 21 here) run their products as the decode GEMMs."""
    from qdec.runtime import DecodeState, Prefill
    prompt = prompts(B, S, seed)
    dprompt = prompt.to(engine.device)
    st = DecodeState(engine.model, B, S + 18, max_t=16, keep_logits=True)
    st.prefill(dprompt)
    logits, ids = st.logits[:B].float().cpu(), st.ids[:B].cpu()
    kc, vc = st.k_cache.clone(), st.v_cache.clone()
    assert st.lens.cpu().tolist() == [S] * B
    okc, ovc = oracle.new_cache(B, st.cap)
    ref = oracle.forward(prompt, [0] * B, okc, ovc)[:, -1]
    err = normalized_max_err(logits, ref)
    print(f"B={B} S={S}: prefill logits normalised max err {err.max().item():.4g}")
    assert err.max().item() <= TOL
    near = top2_gap(ref) < TOL * ref.abs().amax(-1)
    assert bool(((ref.argmax(-1) == ids) | near).all())
    for got, want in ((kc[:, :, :, :S].float().cpu(), okc[:, :, :, :S]),
                      (v_rows(vc.float().cpu())[:, :, :, :S], ovc[:, :, :, :S])):
        assert (got - want).abs().max().item() <= TOL * want.abs().max().item()
    # the decode kernels, 16 positions per step, land on the same cache
    st2 = DecodeState(engine.model, B, S + 18, max_t=16, keep_logits=True)
    st2.prefill_steps(dprompt)
    t_last = (S - 1) % st2.max_t + 1
    steps_logits = st2.logits[:B * t_last].view(B, t_last, -1)[:, t_last - 1].float().cpu()
    assert normalized_max_err(steps_logits, ref).max().item() <= TOL
    from qdec.runtime import max_rows_per_seq
    if S <= max_rows_per_seq(B):  # prefill took this very route
        assert torch.equal(st2.k_cache, kc) and torch.equal(st2.v_cache, vc)
        assert torch.equal(steps_logits, logits) and torch.equal(st2.ids[:B].cpu(), ids)
    # chunking does not change a bit of the matrix-core route (the other
    # routes are checked against the oracle instead)
    from qdec.runtime import PREFILL_SKINNY_ROWS
    st3 = DecodeState(engine.model, B, S + 18, max_t=16, keep_logits=True)
    st3._prefill = Prefill(st3, S, rows=16 * B)
    st3.prefill(dprompt)
    assert st3._prefill.chunk == min(16, S)
    if S > max_rows_per_seq(B) and B * S > PREFILL_SKINNY_ROWS:
        assert torch.equal(st3.k_cache, kc) and torch.equal(st3.v_cache, vc)
        assert torch.equal(st3.ids[:B].cpu(), ids)
    elif S > max_rows_per_seq(B):
        assert not st3._prefill.skinny  # 16-position chunks: the products
        for got, want in ((st3.k_cache[:, :, :, :S].float().cpu(), okc[:, :, :, :S]),
                          (v_rows(st3.v_cache.float().cpu())[:, :, :, :S], ovc[:, :, :, :S])):
            assert (got - want).abs().max().item() <= TOL * want.abs().max().item()


def test_generate_matches_eager_steps(engine):
    prompt = prompts(2, 33, 5)
    toks, _ = run_state(engine, prompt, 12)
    out = list(engine.generate(prompt.tolist(), 12))
    assert len(out) == 12 and all(len(s) == 2 for s in out)
    assert torch.tensor(out).T.tolist() == toks.tolist()
    # a second call of the same shape reuses the graph and resets all state
    out2 = list(engine.generate(prompt.tolist(), 12))
    assert out2 == out


def test_generate_contract(engine):
    assert list(engine.generate([[1, 2, 3]], 0)) == []
    assert list(engine.generate([[1, 2, 3]], -4)) == []
    steps = list(engine.generate([[5, 6, 7, 8]], 3))
    assert len(steps) == 3 and all(isinstance(t, int) for s in steps for t in s)
    one = list(engine.generate([[9] * 70], 1))
    assert len(one) == 1 and len(one[0]) == 1


def motif_prompts(B, S, seed, vocab=151936, motif=64, noise=0.1):
    """a seeded 64-token motif tiled to S, with a
    fraction of positions replaced by uniform random tokens."""
    g = torch.Generator().manual_seed(seed)
    base = torch.randint(0, vocab, (motif,), generator=g)
    rows = []
    for b in range(B):
        r = base.repeat((S + motif - 1) // motif)[:S].clone()
        m = torch.rand(S, generator=g) < noise
        r[m] = torch.randint(0, vocab, (int(m.sum()),), generator=g)
        rows.append(r)
    return torch.stack(rows)


def test_speculative_equals_plain_greedy(ckpt, engine):
    from engine import Engine
    spec = Engine.from_tensors(engine.model.cfg.raw, load_tensors(ckpt[0]), speculate=True)
    for B, S, n, seed in ((4, 200, 40, 7), (2, 64, 25, 8), (1, 30, 17, 9), (3, 100, 12, 13), (5, 90, 12, 14), (6, 90, 12, 12),
                          (8, 40, 12, 11), (16, 40, 9, 10)):
        prompt = motif_prompts(B, S, seed)
        plain = list(engine.generate(prompt.tolist(), n))
        for gate in (False, True):  # always verify / acceptance gate
            spec.spec_gate = gate
            fast = list(spec.generate(prompt.tolist(), n))
            assert fast == plain, (B, S, n, gate)
            stats = spec.stats["spec"]
            print(f"spec B={B} S={S} n={n} gate={gate}: {stats}")
            assert stats["iterations"] <= n - 1
            if not gate and B < 16:
                assert stats["plain_iterations"] == 0



# ------------------------------------------------- one layer per launch
def _layer_state(engine, B, S, seed, **kw):
    from qdec.runtime import DecodeState
    st = DecodeState(engine.model, B, S + 30, max_t=1, keep_logits=True)
    st.prefill(prompts(B, S, seed).to(engine.device))
    st.enable_layer_launch(**kw)
    torch.cuda.synchronize()
    return st


def _snapshot(st):
    return [t.clone() for t in (st.hbuf, st.k_cache, st.v_cache, st.qkv, st.act, st.attn_partial, st.ids, st.lens)]


def _restore(st, snap):
    for t, v in zip((st.hbuf, st.k_cache, st.v_cache, st.qkv, st.act, st.attn_partial, st.ids, st.lens), snap):
        t.copy_(v)


def _stage_launches(st):
    """The layers of a plain step as the five per-operation calls under the
    layer kernel's plans (what each qdec_layer launch runs as its stages)."""
    from qdec import capi
    lib, c = st.lib, st.model.cfg
    s = torch.cuda.current_stream().cuda_stream
    e = capi.EmbedArgs()
    e.ids, e.emb, e.h = st.ids.data_ptr(), st.model.emb.data_ptr(), st.h.data_ptr()
    e.rows, e.hidden, e.vocab = st.batch, c.hidden, c.vocab
    lib.embed(e, s)
    for i in range(c.n_layers):
        at = st.layer_attn_args(i)
        lib.gemm(st.layer_gemm_args("qkv", i), s)
        lib.attn(at, s)
        lib.gemm(st.layer_gemm_args("o", i, x_attn=at), s)
        lib.gemm(st.layer_gemm_args("gate_up", i), s)
        lib.gemm(st.layer_gemm_args("down", i), s)


def _same(a, b):
    """Bit-identical (NaN payloads included)."""
    return torch.equal(a.contiguous().view(torch.uint8), b.contiguous().view(torch.uint8))


# The norm hand-over (O / down writing the next NORM_IN call's normalised
# rows as their last workgroups finish) against the pre-pass launches it
# replaces: plain steps at 8 rows (gate/up only), 12 (down without a k split
# hands to 4-wave QKV and lm_head), 20 and 32 (down's four split partials
# merged and handed to 8-wave QKV: a 4-wave producer emulating an 8-wave
# statistic), and verify steps of 16 and 18 rows.  Logits, tokens and both
# residual buffers bit for bit.
@pytest.mark.parametrize("B,S,t_rows,seed", [(8, 40, 1, 61), (12, 33, 1, 62), (20, 50, 1, 63), (32, 70, 1, 64),
                                             (4, 30, 4, 65), (2, 25, 9, 66)])
def test_norm_hand_over_equals_the_pre_pass(engine, B, S, t_rows, seed):
    from qdec.runtime import DecodeState
    rows = B * t_rows
    outs = []
    for hand in (True, False):
        st = DecodeState(engine.model, B, S + 40, max_t=16, keep_logits=True)
        st.hand_over = hand
        # With the hand-over, gate/up keeps its pre-pass plan at 6..8 rows (O
        # hands it the rows); without, it runs resident: the same bits.
        st.resident = not hand
        if hand:
            assert st._hand_threads("o", rows) == 256
            assert st._hand_threads("down", rows) == (None if rows < 9 else 64 * st.plans["qkv"][1])
        st.prefill(prompts(B, S, seed).to(engine.device))
        for _ in range(3):
            st.run_step(t_rows=1)
        if t_rows > 1:
            st.run_step(t_rows=t_rows, advance=False)
        torch.cuda.synchronize()
        outs.append((st.logits[:rows].clone(), st.ids[:rows].clone(), st.hbuf[:, :rows].clone(), st.lens.clone()))
        assert not torch.isnan(st.logits[:rows].float()).any()
        del st
    for a, b in zip(*outs):
        assert _same(a, b)


def _tickets(st):
    """(top ticket, arrivals summed over the 8 groups) of the layer kernel's
    barrier state: the top at byte 0, group g's arrivals at 128 + 128 g."""
    w = st.layer_ctl.cpu().view(torch.int64).tolist()
    return w[0], sum(w[16 + 16 * g] for g in range(8))


@pytest.mark.parametrize("B,S,seed", [(1, 150, 41), (3, 333, 42), (4, 90, 43)])
def test_layer_launch_equals_its_stage_launches(engine, B, S, seed):
    """qdec_layer runs the per-block code of each stage's own launch: the
    residual, the new cache slots, the SwiGLU activations and the attention
    partials come out bit for bit as from the five calls with the same
    plans."""
    st = _layer_state(engine, B, S, seed)
    snap = _snapshot(st)
    _stage_launches(st)
    torch.cuda.synchronize()
    want = _snapshot(st)
    _restore(st, snap)
    top0, arr0 = _tickets(st)
    st.run_step(t_rows=1, lm_head=False, advance=False)
    torch.cuda.synchronize()
    got = _snapshot(st)
    names = ("hbuf", "k_cache", "v_cache", "qkv", "act", "attn_partial", "ids", "lens")
    for name, g, w in zip(names, got, want):
        assert _same(g, w), name
    assert st.layer_error() == 0
    # every workgroup passed 4 barriers per layer; a group's last arrival
    # went on to the top
    top, arr = _tickets(st)
    barriers = 4 * engine.model.cfg.n_layers
    assert top - top0 == 8 * barriers
    assert (arr - arr0) % barriers == 0 and (arr - arr0) // barriers >= 304  # gate/up has 304 blocks
    assert not torch.equal(snap[0], got[0])  # the step did something


@pytest.mark.parametrize("B,S,n,seed", [(1, 60, 8, 51), (4, 45, 6, 52)])
def test_layer_launch_vs_oracle(engine, oracle, B, S, n, seed):
    """Plain decode with one launch per layer, teacher-forced against the
    oracle: the same logit tolerance and near-tie rule as the per-operation
    step."""
    from qdec.runtime import DecodeState
    prompt = prompts(B, S, seed)
    st = DecodeState(engine.model, B, S + n + 30, max_t=1, keep_logits=True)
    st.prefill(prompt.to(engine.device))
    st.enable_layer_launch()
    toks, logits = [st.ids[:B].cpu()], [st.logits[:B].float().cpu()]
    for _ in range(n - 1):
        st.run_step(t_rows=1)
        toks.append(st.ids[:B].cpu())
        logits.append(st.logits[:B].float().cpu())
    torch.cuda.synchronize()
    assert st.layer_error() == 0
    toks, logits = torch.stack(toks, 1), torch.stack(logits, 1)
    ref = oracle.teacher_forced(prompt, toks)
    err = normalized_max_err(logits, ref)
    print(f"layer launch B={B}: normalised max err {err.max().item():.4g}")
    assert err.max().item() <= TOL
    mism = ref.argmax(-1) != toks
    near = top2_gap(ref) < TOL * ref.abs().amax(-1)
    assert bool((~mism | near).all()), mism.nonzero().tolist()


def test_layer_wait_limit_and_stale_plan(engine):
    """The bounded barrier wait, forced from the host: with a limit of one
    poll a wait runs out, the error word says 1 and every workgroup still
    finishes.  A call whose arguments differ from the prepared plan runs
    nothing and says 2.  After a reset the same state steps correctly; then
    a launch of another workgroup count on the same ctl runs nothing and
    says 3."""
    st = _layer_state(engine, 1, 64, 61, spin_limit=1)
    snap = _snapshot(st)
    st.run_step(t_rows=1, lm_head=False, advance=False)
    torch.cuda.synchronize()
    assert st.layer_error() == 1
    _restore(st, snap)  # the stages ran unsynchronised: whatever they left
    st.reset_layer_ctl()
    st.enable_layer_launch()
    la = st._layer_args[0]
    la.qkv.contents.eps = 1e-3  # no longer the prepared plan
    st.lib.layer(la, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert st.layer_error() == 2
    assert all(_same(g, w) for g, w in zip(_snapshot(st), snap))
    la.qkv.contents.eps = engine.model.cfg.eps
    st.reset_layer_ctl()
    _stage_launches(st)
    want = _snapshot(st)
    _restore(st, snap)
    st.run_step(t_rows=1, lm_head=False, advance=False)
    torch.cuda.synchronize()
    assert st.layer_error() == 0
    assert all(_same(g, w) for g, w in zip(_snapshot(st), want))
    # A launch with another workgroup count on a ctl whose tickets were
    # counted with the first launch's: nothing runs and the word says 3.
    n_first = int(st.layer_ctl[3].item())  # uint32 at ctl + 12
    assert n_first >= 8
    st.enable_layer_launch(workgroups=n_first - 8)
    before = _snapshot(st)
    st.lib.layer(st._layer_args[0], torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert st.layer_error() == 3
    assert all(_same(g, w) for g, w in zip(_snapshot(st), before))
    st.reset_layer_ctl()


def test_engine_mega_check_race_and_force(ckpt, engine, oracle):
    """Engine(mega=True): the layer step is checked against the
    per-operation step and raced; with MEGA_FORCE it is used, and its
    tokens are the oracle's greedy picks up to near-ties."""
    import engine as engine_mod
    from engine import Engine
    mega = Engine.from_tensors(engine.model.cfg.raw, load_tensors(ckpt[0]), mega=True)
    prompt = prompts(1, 48, 71)
    out = list(mega.generate(prompt.tolist(), 6))
    info = mega.stats["mega"]
    print(f"mega race: {info}")
    assert info["ok"] and info["error_word"] == 0 and info["layer_ms"] > 0 and info["per_op_ms"] > 0
    assert len(out) == 6
    engine_mod.MEGA_FORCE = True
    try:
        mega.shape = None
        out = list(mega.generate(prompt.tolist(), 6))
    finally:
        engine_mod.MEGA_FORCE = False
    assert mega.stats["mega"]["used"] and mega.shape.state.layer_launch
    toks = torch.tensor(out).T  # [B, n]
    ref = oracle.teacher_forced(prompt, toks)
    mism = ref.argmax(-1) != toks
    near = top2_gap(ref) < TOL * ref.abs().amax(-1)
    assert bool((~mism | near).all()), mism.nonzero().tolist()


def test_invalid_inputs_raise(engine):
    """Out-of-range prompt ids are refused on the host; an out-of-range id
    that reaches the device makes the step emit capi.NAN_ID, which the engine
    refuses instead of yielding."""
    from qdec import capi
    from qdec.runtime import DecodeState
    with pytest.raises(ValueError):
        list(engine.generate([[1, 151936]], 2))
    with pytest.raises(ValueError):
        list(engine.generate([[-1, 5]], 2))
    st = DecodeState(engine.model, 1, 64, max_t=1)
    st.ids.fill_(10 ** 6)
    st.lens.fill_(5)
    st.run_step(t_rows=1)
    torch.cuda.synchronize()
    assert st.ids[0].item() == capi.NAN_ID
    with pytest.raises(capi.QdecError):
        engine._checked(st.ids[:1].tolist())


def test_selfcheck_detects_a_wrong_answer(engine, monkeypatch):
    """The load-time self-check passes on this device and fails loudly when a
    kernel's answer is wrong (simulated on the host: the O projection's
    launch is dropped, so the residual comes back unchanged)."""
    from qdec import capi, selfcheck
    from qdec.runtime import DecodeState
    st = DecodeState(engine.model, 1, 64, max_t=1)
    selfcheck.run(st)
    real = st.lib.gemm

    def drop_o(args, stream):
        if not (args.flags == capi.RES_OUT and args.k == engine.model.cfg.nq * engine.model.cfg.head_dim):
            real(args, stream)

    monkeypatch.setattr(st.lib, "gemm", drop_o)
    with pytest.raises(selfcheck.SelfCheckError, match="^self-check failed .*o:"):
        selfcheck.run(st)


@pytest.mark.parametrize("what", ["qkv", "attn", "o", "gate_up", "down", "lm"])
def test_shape_selfcheck_detects_a_dropped_launch(engine, monkeypatch, what):
    """Every new shape runs the known-answer checks through its own plans
    before its first token (here batch 32: the 8-wave attention over one
    whole-cache chunk, fragment-order hand-overs, the down projection's k
    split merged by the next NORM_IN call, two tiles per wave, the 8-tile
    lm_head).  Dropping one of its 32-row launches (simulated on the host)
    makes generate raise before it yields anything, and the shape is not
    kept; with the launch back the same shape serves."""
    from qdec import capi, selfcheck
    c = engine.model.cfg
    B, S = 32, 24
    lib = engine.model.lib
    real_gemm, real_attn = lib.gemm, lib.attn

    def role(a):
        if a.flags & capi.ARGMAX:
            return "lm"
        if a.flags & capi.GLU:
            return "gate_up"
        if a.flags & capi.RES_OUT:
            return "o" if a.k == c.nq * c.head_dim else "down"
        return "qkv"

    def gemm(a, s):
        if not (role(a) == what and a.rows == B):
            real_gemm(a, s)

    def attn(a, s):
        if not (what == "attn" and a.batch * a.t_rows == B):
            real_attn(a, s)

    prompt = prompts(B, S, 41).tolist()
    engine.shape = None  # a new shape, checked before it serves
    monkeypatch.setattr(lib, "gemm", gemm)
    monkeypatch.setattr(lib, "attn", attn)
    gen = engine.generate(prompt, 3)
    with pytest.raises(selfcheck.SelfCheckError, match="^self-check failed"):
        next(gen)
    assert engine.shape is None
    monkeypatch.undo()
    toks = list(engine.generate(prompt, 3))
    assert len(toks) == 3 and all(len(t) == B for t in toks)


@pytest.mark.parametrize("B,spec", [(1, False), (3, True), (8, False), (12, False), (20, False), (64, False)])
def test_shape_selfcheck_passes(ckpt, engine, B, spec):
    """The per-shape checks pass on every plan family: merge in O (1),
    verify rows of a speculative state (3: t = 1 and k + 1), register-staged
    rows and 8-wave 512-slot chunks (8, 12), two tiles per wave and the down
    split (20), four M tiles (64)."""
    from engine import spec_k
    from qdec import selfcheck
    from qdec.runtime import DecodeState
    k = spec_k(B) if spec else 0
    st = DecodeState(engine.model, B, 1500, max_t=k + 1 if k else 1)
    selfcheck.run_shape(st, (1, k + 1) if k else (1,))
    assert int(st.k_cache.abs().sum()) == 0 and int(st.v_cache.abs().sum()) == 0


def test_from_model_hook(ckpt, engine):
    """Engine.from_model (the reference's test hook, engine/engine.py:243-248)
    on a Transformers Qwen3 model loaded from the test checkpoint emits the
    same tokens as the engine built from the checkpoint directory; a CPU
    device or use_triton=False is refused (no other path)."""
    from transformers import AutoModelForCausalLM
    from engine import Engine
    hf = AutoModelForCausalLM.from_pretrained(ckpt[0], dtype=torch.bfloat16, local_files_only=True).eval()
    eng2 = Engine.from_model(hf, "cuda:0")
    prompt = prompts(2, 19, 81).tolist()
    assert list(eng2.generate(prompt, 5)) == list(engine.generate(prompt, 5))
    with pytest.raises(ValueError):
        Engine.from_model(hf, "cpu", use_triton=False)
    with pytest.raises(ValueError):
        Engine.from_model(hf, "cuda:0", use_triton=False)
