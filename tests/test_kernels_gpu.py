"""Every kernel of libqdec.so against the oracle, on the GPU, through the C ABI.

Tolerances: bit-exact for layout, gather, cache writes, argmax and the
drafter / acceptance; for the floating-point products the reference's own
agreement rule (engine/engine.py:349-358 ``_agree``): max |err| <= 2% of the
reference's max |value| and, where only the fp32 summation order differs, at
least 98% of the bf16 outputs bit-identical.  Row- and t_rows-invariance is
checked bit for bit: it is what makes speculative decoding lossless.
"""

import ctypes
import math
import zlib

import pytest
import torch

from helpers import near_exact

from oracle.qwen3_oracle import (argmax_lowest, attention, bf16, head_norm_rope, linear, rms_norm,
                                 rope_tables, silu_mul)
from oracle.spec_oracle import accept as accept_ref
from oracle.spec_oracle import ngram_draft as draft_ref

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
H, I, V, NQ, NKV, D = 2560, 9728, 151936, 32, 8, 128
HEADS_4B = (NQ, NKV, D)


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")
    from qdec import capi
    return capi.lib()


def stream():
    return torch.cuda.current_stream().cuda_stream


def rnd(*shape, scale=1.0, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def agree(fast, ref, min_exact=0.98, tol=0.02):
    fast, ref = fast.float().cpu(), ref.float().cpu()
    assert torch.isfinite(fast).all()
    exact = (fast == ref).float().mean().item()
    err = (fast - ref).abs().max().item()
    scale = ref.abs().max().item()
    assert err <= tol * scale + 1e-3, f"max err {err} vs scale {scale}"
    assert exact >= min_exact, f"exact fraction {exact}"
    return exact, err


def pack(lib, w):
    n, k = w.shape
    dst = torch.empty(n * k, dtype=torch.bfloat16, device=DEV)
    lib.pack_tiles(w.data_ptr(), dst.data_ptr(), n, k, stream())
    return dst


class Gemm:
    """Call qdec_gemm for one role with device tensors."""

    def __init__(self, lib, flags, n, k, ksplit=1, waves=4, tiles=1):
        from qdec import capi
        self.lib, self.capi = lib, capi
        self.flags, self.n, self.k = flags, n, k
        self.ksplit, self.waves, self.tiles = ksplit, waves, tiles
        self.partial = torch.zeros(8 << 20, dtype=torch.float32, device=DEV)
        self.counters = torch.zeros(16384, dtype=torch.int32, device=DEV)

    def __call__(self, x, w_tiled, out=None, res=None, norm_w=None, ids=None, lens=None):
        a = self.capi.GemmArgs()
        a.x, a.w = x.data_ptr(), w_tiled.data_ptr()
        a.out = out.data_ptr() if out is not None else None
        a.res = res.data_ptr() if res is not None else None
        a.norm_w = norm_w.data_ptr() if norm_w is not None else None
        a.partial, a.counters = self.partial.data_ptr(), self.counters.data_ptr()
        a.ids_out = ids.data_ptr() if ids is not None else None
        a.lens_inc = lens.data_ptr() if lens is not None else None
        a.eps, a.rows, a.n, a.k = 1e-6, x.shape[0], self.n, self.k
        a.flags, a.ksplit, a.waves, a.tiles_per_wg = self.flags, self.ksplit, self.waves, self.tiles
        pb, _ = self.lib.gemm_workspace(a)
        assert pb <= self.partial.numel() * 4
        assert x.shape[1] == self.k and x.is_contiguous() and w_tiled.numel() == self.k * self.n * (
            2 if self.flags & self.capi.GLU else 1)
        self.lib.gemm(a, stream())
        torch.cuda.synchronize()
        assert int(self.counters.abs().sum()) == 0, "arrival counters not reset"


# ----------------------------------------------------------------- layout

def test_pack_tiles_layout(lib):
    n, k = 48, 96
    w = torch.arange(n * k, dtype=torch.int32).view(n, k)
    src = w.to(torch.float32).to(torch.bfloat16)  # exact for < 256? use bits instead
    src = w.to(torch.int16).view(torch.bfloat16).contiguous().to(DEV)
    out = pack(lib, src).view(torch.int16).cpu().to(torch.int32)
    idx = torch.tensor([lib.tiled_offset(r, c, k) for r in range(n) for c in range(k)])
    assert torch.equal(out[idx], w.flatten().to(torch.int16).to(torch.int32))


def test_embed_gather_exact(lib):
    from qdec import capi
    vocab, hid = 512, 256
    E = rnd(vocab, hid, seed=1)
    Et = pack(lib, E.to(DEV))
    ids = torch.tensor([0, 511, 7, 7, 300], dtype=torch.int64, device=DEV)
    h = torch.zeros(5, hid, dtype=torch.bfloat16, device=DEV)
    e = capi.EmbedArgs(ids=ids.data_ptr(), emb=Et.data_ptr(), h=h.data_ptr(), rows=5, hidden=hid, vocab=vocab)
    lib.embed(e, stream())
    torch.cuda.synchronize()
    assert torch.equal(h.cpu(), E[ids.cpu()])


# ------------------------------------------------------------------- GEMM

@pytest.mark.parametrize("rows", [1, 4, 7, 9, 16, 17, 36, 64])
@pytest.mark.parametrize("role", ["qkv", "o", "gate_up", "down"])
def test_gemm_roles_vs_oracle(lib, role, rows):
    from qdec import capi
    from qdec.runtime import role_plan
    n, k, flags = {"qkv": (6144, H, capi.NORM_IN), "o": (H, 4096, capi.RES_OUT),
                   "gate_up": (I, H, capi.NORM_IN | capi.GLU), "down": (H, I, capi.RES_OUT)}[role]
    ks, waves, _ = role_plan(n, k, role)
    seed = (zlib.crc32(role.encode()) + 7 * rows) % 1000  # stable across processes
    x = rnd(rows, k, scale=3.0, seed=seed)
    wn = 2 * n if flags & capi.GLU else n
    W = rnd(wn, k, scale=0.02, seed=seed + 1)
    nw = bf16(1 + 0.2 * torch.randn(k, generator=torch.Generator().manual_seed(seed + 2))).to(torch.bfloat16)
    g = Gemm(lib, flags, n, k, ksplit=ks, waves=waves)
    xd, Wt = x.to(DEV), pack(lib, W.to(DEV))
    if flags & capi.NORM_IN:
        xin = rms_norm(x.float(), nw.float(), 1e-6)
    else:
        xin = x.float()
    if flags & capi.GLU:
        out = torch.zeros(rows, n, dtype=torch.bfloat16, device=DEV)
        g(xd, Wt, out=out, norm_w=nw.to(DEV))
        ref = silu_mul(linear(xin, W[:n].float()), linear(xin, W[n:].float()))
    elif flags & capi.RES_OUT:
        res0 = rnd(rows, n, scale=2.0, seed=seed + 3)
        res = res0.to(DEV).clone()
        g(xd, Wt, res=res)
        out = res
        ref = bf16(res0.float() + linear(xin, W.float()))
    else:
        out = torch.zeros(rows, n, dtype=torch.bfloat16, device=DEV)
        g(xd, Wt, out=out, norm_w=nw.to(DEV))
        ref = linear(xin, W.float())
    # bf16 outputs agree bit for bit except where the fp32 sums straddle a
    # rounding boundary (summation order differs from torch's); SwiGLU
    # rounds three times, so more of its outputs straddle one.
    agree(out, ref, min_exact=0.97 if flags & capi.GLU else 0.98)


@pytest.mark.parametrize("role", ["qkv", "o", "gate_up", "down"])
def test_gemm_row_invariance_bitexact(lib, role):
    """A row's output bits do not depend on how many rows share the call or
    where the row sits (MFMA column, M tile, LDS pass, activations staged in
    LDS or read directly after the normalisation pre-pass)."""
    from qdec import capi
    from qdec.runtime import role_plan
    n, k, flags = {"qkv": (6144, H, capi.NORM_IN), "o": (H, 4096, capi.RES_OUT),
                   "gate_up": (I, H, capi.NORM_IN | capi.GLU), "down": (H, I, capi.RES_OUT)}[role]
    ks, waves, _ = role_plan(n, k, role)
    big = 64
    x = rnd(big, k, scale=3.0, seed=11).to(DEV)
    W = pack(lib, rnd(2 * n if flags & capi.GLU else n, k, scale=0.02, seed=12).to(DEV))
    nw = rnd(k, scale=0.2, seed=13).to(DEV)
    res0 = rnd(big, n, scale=2.0, seed=14).to(DEV)
    g = Gemm(lib, flags, n, k, ksplit=ks, waves=waves)

    def run(rows_idx):
        xs = x[rows_idx].contiguous()
        if flags & capi.RES_OUT:
            r = res0[rows_idx].contiguous().clone()
            g(xs, W, res=r)
            return r
        o = torch.zeros(len(rows_idx), n, dtype=torch.bfloat16, device=DEV)
        g(xs, W, out=o, norm_w=nw)
        return o

    full = run(list(range(big)))
    for rows_idx in ([5], [0, 1, 2, 3], list(range(36)), [63, 9, 40], list(range(17, 34)), list(range(16)),
                     list(range(40, 49)), [7] * 12, list(range(40, 48)), [5, 6, 7, 8, 9, 10]):
        part = run(rows_idx)
        assert torch.equal(part.view(torch.int16), full[rows_idx].view(torch.int16)), rows_idx


@pytest.mark.parametrize("rows", [3, 32])
@pytest.mark.parametrize("role", ["gate_up", "down"])
def test_gemm_split_multi_tile_vs_oracle(lib, role, rows):
    """k split across workgroups that own several output tiles each: a
    workgroup that is not the last split of one tile goes on to the next."""
    from qdec import capi
    n, k, flags = {"gate_up": (I, H, capi.NORM_IN | capi.GLU), "down": (H, I, capi.RES_OUT)}[role]
    ks, waves, tiles = (4, 4, 8) if role == "gate_up" else (8, 2, 4)
    seed = (zlib.crc32(role.encode()) + 13 * rows) % 1000
    x = rnd(rows, k, scale=3.0, seed=seed)
    W = rnd(2 * n if flags & capi.GLU else n, k, scale=0.02, seed=seed + 1)
    nw = bf16(1 + 0.2 * torch.randn(k, generator=torch.Generator().manual_seed(seed + 2))).to(torch.bfloat16)
    g = Gemm(lib, flags, n, k, ksplit=ks, waves=waves, tiles=tiles)
    xd, Wt = x.to(DEV), pack(lib, W.to(DEV))
    if flags & capi.GLU:
        xin = rms_norm(x.float(), nw.float(), 1e-6)
        out = torch.zeros(rows, n, dtype=torch.bfloat16, device=DEV)
        g(xd, Wt, out=out, norm_w=nw.to(DEV))
        ref = silu_mul(linear(xin, W[:n].float()), linear(xin, W[n:].float()))
    else:
        res0 = rnd(rows, n, scale=2.0, seed=seed + 3)
        out = res0.to(DEV).clone()
        g(xd, Wt, res=out)
        ref = bf16(res0.float() + linear(x.float(), W.float()))
    agree(out, ref, min_exact=0.97 if flags & capi.GLU else 0.98)


@pytest.mark.parametrize("rows", [1, 5, 17, 32])
def test_lmhead_argmax_and_ties(lib, rows):
    """Greedy pick over 151936 columns: the lowest index of the max bf16
    logit, bit-exact; logits within tolerance of the oracle; lens advance.
    Tiles per workgroup as the engine plans them (qdec.runtime: the role plan
    at one row, LM_TILES_BATCHED from two), so rows 17 and 32 run config 4's
    two-M-tile NORM_IN|ARGMAX path with the normalisation pre-pass."""
    from qdec import capi
    from qdec.runtime import LM_TILES_BATCHED, role_plan
    _, waves, tiles = role_plan(V, H, "lm")
    if rows > 1:
        tiles = LM_TILES_BATCHED
    x = rnd(rows, H, scale=2.0, seed=21 + rows)
    E = rnd(V, H, scale=0.02, seed=22)
    # plant exact ties: duplicate rows -> identical logits at two indices.
    E[100000] = E[77]
    E[150000] = E[3]
    nw = bf16(1 + 0.1 * torch.randn(H, generator=torch.Generator().manual_seed(23))).to(torch.bfloat16)
    # make rows 0/1 (and the last row) pick the planted duplicates: x aligned
    # with E[77] / E[3]
    x[0] = (E[77].float() * 200).to(torch.bfloat16)
    x[rows - 1] = (E[3].float() * 200).to(torch.bfloat16)
    if rows > 2:
        x[1] = x[rows - 1]
    Et = pack(lib, E.to(DEV))
    g = Gemm(lib, capi.NORM_IN | capi.ARGMAX, V, H, waves=waves, tiles=tiles)
    logits = torch.zeros(rows, V, dtype=torch.bfloat16, device=DEV)
    ids = torch.full((rows,), -1, dtype=torch.int64, device=DEV)
    lens = torch.arange(rows, dtype=torch.int32, device=DEV)
    g(x.to(DEV), Et, out=logits, norm_w=nw.to(DEV), ids=ids, lens=lens)
    lg = logits.float().cpu()
    got = ids.cpu().tolist()
    assert got == argmax_lowest(lg).tolist()
    assert got[0] == 77 or rows == 1
    assert got[rows - 1] == 3 and (rows < 3 or got[1] == 3)
    assert lens.cpu().tolist() == list(range(1, rows + 1))
    ref = linear(rms_norm(x.float(), nw.float(), 1e-6), E.float())
    agree(lg, ref)


# -------------------------------------------------------------- attention

def v_layout(v):
    """[..., cap, D] -> the channel-major V cache layout [..., cap/8, D, 8]."""
    *lead, cap, d = v.shape
    return v.reshape(*lead, cap // 8, 8, d).transpose(-1, -2).contiguous()


def attn_case(lib, B, T, lens, cap, chunk, seed, waves=4, out_frag=0, valid=True, strided=0):
    from qdec import capi
    g = torch.Generator().manual_seed(seed)
    W = (NQ + 2 * NKV) * D
    qkv = (torch.randn(B * T, W, generator=g) * 2).to(torch.bfloat16)
    qn = bf16(1 + 0.2 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kn = bf16(1 + 0.2 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kc = (torch.randn(B, NKV, cap, D, generator=g)).to(torch.bfloat16)
    vc = (torch.randn(B, NKV, cap, D, generator=g)).to(torch.bfloat16)
    cos, sin = rope_tables(cap, D, 5e6, "bf16")
    lens_t = torch.tensor(lens, dtype=torch.int32)
    a = capi.AttnArgs()
    dq = qkv.to(DEV)
    dqn, dkn = qn.to(DEV), kn.to(DEV)
    dcos, dsin = cos.to(torch.bfloat16).to(DEV), sin.to(torch.bfloat16).to(DEV)
    dl = lens_t.to(DEV)
    dk, dv = kc.to(DEV).contiguous(), v_layout(vc).to(DEV)
    out = torch.zeros((B * T + 15) // 16 * 16, NQ * D, dtype=torch.bfloat16, device=DEV)
    a.qkv, a.q_norm_w, a.k_norm_w, a.cos_tab, a.sin_tab, a.lens = (dq.data_ptr(), dqn.data_ptr(), dkn.data_ptr(),
                                                                 dcos.data_ptr(), dsin.data_ptr(), dl.data_ptr())
    a.k_cache, a.v_cache, a.out = dk.data_ptr(), dv.data_ptr(), out.data_ptr()
    a.eps, a.sm_scale = 1e-6, D ** -0.5
    a.batch, a.t_rows, a.nq, a.nkv, a.head_dim, a.cap, a.chunk = B, T, NQ, NKV, D, cap, chunk
    a.waves, a.out_frag, a.strided = waves, out_frag, strided
    pb, cb = lib.attn_workspace(a)
    part = torch.zeros(max(pb, 16) // 4, dtype=torch.float32, device=DEV)
    cnt = torch.zeros(max(cb, 4) // 4, dtype=torch.int32, device=DEV)
    a.partial, a.counters = part.data_ptr(), cnt.data_ptr()
    assert not valid or max(lens) + T <= cap
    lib.attn(a, stream())
    torch.cuda.synchronize()
    assert int(cnt.abs().sum()) == 0
    rows = frag_to_rows(out, B * T, NQ * D) if out_frag else out[:B * T]
    return dict(qkv=qkv, qn=qn, kn=kn, kc=kc, vc=vc, cos=cos, sin=sin, lens=lens, out=rows.cpu(),
                k_after=dk.cpu(), v_after=dv.cpu())


@pytest.mark.parametrize("waves", [4, 8])
@pytest.mark.parametrize("B,lens,cap,chunk,strided", [
    (1, [640], 800, 96, 0), (1, [767], 800, 96, 0), (1, [640], 800, 128, 0), (1, [100], 800, 128, 0),
    (3, [700, 31, 257], 800, 128, 0), (2, [200, 90], 256, 256, 0), (1, [4000], 4384, 256, 0),
    (1, [640], 800, 96, 1), (3, [700, 31, 257], 800, 224, 1), (2, [4000, 33], 4384, 1120, 1)])
def test_o_projection_merges_attention_partials_bitexact(lib, B, lens, cap, chunk, strided, waves):
    if strided and waves != 8:
        pytest.skip("strided chunks run 8 waves")
    """Attention with out_partials + an O projection reading x_attn gives the
    same bits as the attention's own merged output fed to the O projection
    (one chunk and several; the attention's out buffer is left untouched).
    The first cases are config 2's plan: 4 waves, 96-slot chunks of an
    800-slot cache, 512..767 cached slots."""
    from qdec import capi
    from qdec.runtime import role_plan
    g = torch.Generator().manual_seed(sum(lens) + B)
    W = (NQ + 2 * NKV) * D
    qkv = (torch.randn(B, W, generator=g) * 2).to(torch.bfloat16).to(DEV)
    qn = bf16(1 + 0.2 * torch.randn(D, generator=g)).to(torch.bfloat16).to(DEV)
    kn = bf16(1 + 0.2 * torch.randn(D, generator=g)).to(torch.bfloat16).to(DEV)
    kc0 = torch.randn(B, NKV, cap, D, generator=g).to(torch.bfloat16)
    vc0 = v_layout(torch.randn(B, NKV, cap, D, generator=g).to(torch.bfloat16))
    cos, sin = rope_tables(cap, D, 5e6, "bf16")
    dcos, dsin = cos.to(torch.bfloat16).to(DEV), sin.to(torch.bfloat16).to(DEV)
    dl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    Wo = pack(lib, rnd(H, NQ * D, scale=0.02, seed=5).to(DEV))
    res0 = rnd(B, H, scale=2.0, seed=6).to(DEV)
    ks, o_waves, _ = role_plan(H, NQ * D, "o")
    results = []
    for partials in (0, 1):
        kc, vc = kc0.to(DEV), vc0.to(DEV)
        out = torch.full((B, NQ * D), 7.0, dtype=torch.bfloat16, device=DEV)
        a = capi.AttnArgs(qkv=qkv.data_ptr(), q_norm_w=qn.data_ptr(), k_norm_w=kn.data_ptr(), cos_tab=dcos.data_ptr(),
                          sin_tab=dsin.data_ptr(), lens=dl.data_ptr(), k_cache=kc.data_ptr(), v_cache=vc.data_ptr(),
                          out=out.data_ptr(), eps=1e-6, sm_scale=D ** -0.5, batch=B, t_rows=1, nq=NQ, nkv=NKV,
                          head_dim=D, cap=cap, chunk=chunk, waves=waves, out_partials=partials, strided=strided)
        pb, cb = lib.attn_workspace(a)
        part = torch.zeros(max(pb, 16) // 4, dtype=torch.float32, device=DEV)
        cnt = torch.zeros(max(cb, 4) // 4, dtype=torch.int32, device=DEV)
        a.partial, a.counters = part.data_ptr(), cnt.data_ptr()
        lib.attn(a, stream())
        res = res0.clone()
        o = capi.GemmArgs(x=out.data_ptr(), w=Wo.data_ptr(), res=res.data_ptr(), eps=1e-6, rows=B, n=H, k=NQ * D,
                          flags=capi.RES_OUT, ksplit=ks, waves=o_waves, tiles_per_wg=1)
        if partials:
            o.x_attn = ctypes.addressof(a)
        lib.gemm(o, stream())
        torch.cuda.synchronize()
        if partials:
            assert bool((out == 7.0).all()), "out_partials must leave out untouched"
        results.append(res.cpu())
    assert torch.equal(results[0].view(torch.int16), results[1].view(torch.int16))


def frag_to_rows(buf, rows, cols):
    """Row-major [rows, cols] view of a buffer written in fragment order
    (include/qdec.h): element (m, c) at ((c/32*nmt + m/16)*64 + m%16 +
    16*(c%32/8))*8 + c%8."""
    nmt = (rows + 15) // 16
    m = torch.arange(rows)[:, None]
    c = torch.arange(cols)[None, :]
    idx = (((c // 32) * nmt + m // 16) * 64 + m % 16 + 16 * ((c % 32) // 8)) * 8 + c % 8
    return buf.flatten()[idx.flatten().to(buf.device)].view(rows, cols)


@pytest.mark.parametrize("B,lens,cap,chunk", [(8, [700, 31, 257, 5, 1000, 640, 64, 300], 1056, 512),
                                               (20, [100 + 37 * i for i in range(20)], 896, 896)])
def test_attention_to_o_in_fragment_order_bitexact(lib, B, lens, cap, chunk):
    """Attention writing its output in fragment order and the O projection
    reading it that way give the same bits as the row-major handover."""
    from qdec import capi
    from qdec.runtime import role_plan
    g = torch.Generator().manual_seed(sum(lens))
    W = (NQ + 2 * NKV) * D
    qkv = (torch.randn(B, W, generator=g) * 2).to(torch.bfloat16).to(DEV)
    qn = bf16(1 + 0.2 * torch.randn(D, generator=g)).to(torch.bfloat16).to(DEV)
    kn = bf16(1 + 0.2 * torch.randn(D, generator=g)).to(torch.bfloat16).to(DEV)
    kc0 = torch.randn(B, NKV, cap, D, generator=g).to(torch.bfloat16)
    vc0 = v_layout(torch.randn(B, NKV, cap, D, generator=g).to(torch.bfloat16))
    cos, sin = rope_tables(cap, D, 5e6, "bf16")
    dcos, dsin = cos.to(torch.bfloat16).to(DEV), sin.to(torch.bfloat16).to(DEV)
    dl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    Wo = pack(lib, rnd(H, NQ * D, scale=0.02, seed=15).to(DEV))
    res0 = rnd(B, H, scale=2.0, seed=16).to(DEV)
    ks, waves, _ = role_plan(H, NQ * D, "o")
    outs, results = [], []
    for frag in (0, 1):
        kc, vc = kc0.to(DEV), vc0.to(DEV)
        out = torch.zeros((B + 15) // 16 * 16, NQ * D, dtype=torch.bfloat16, device=DEV)
        a = capi.AttnArgs(qkv=qkv.data_ptr(), q_norm_w=qn.data_ptr(), k_norm_w=kn.data_ptr(), cos_tab=dcos.data_ptr(),
                          sin_tab=dsin.data_ptr(), lens=dl.data_ptr(), k_cache=kc.data_ptr(), v_cache=vc.data_ptr(),
                          out=out.data_ptr(), eps=1e-6, sm_scale=D ** -0.5, batch=B, t_rows=1, nq=NQ, nkv=NKV,
                          head_dim=D, cap=cap, chunk=chunk, waves=4, out_frag=frag)
        pb, cb = lib.attn_workspace(a)
        part = torch.zeros(max(pb, 16) // 4, dtype=torch.float32, device=DEV)
        cnt = torch.zeros(max(cb, 4) // 4, dtype=torch.int32, device=DEV)
        a.partial, a.counters = part.data_ptr(), cnt.data_ptr()
        lib.attn(a, stream())
        res = res0.clone()
        gw = Gemm(lib, capi.RES_OUT, H, NQ * D, ksplit=ks, waves=waves)
        o = capi.GemmArgs(x=out.data_ptr(), w=Wo.data_ptr(), res=res.data_ptr(), eps=1e-6, rows=B, n=H, k=NQ * D,
                          flags=capi.RES_OUT, ksplit=ks, waves=waves, tiles_per_wg=1, x_frag=frag,
                          partial=gw.partial.data_ptr(), counters=gw.counters.data_ptr())
        lib.gemm(o, stream())
        torch.cuda.synchronize()
        outs.append(frag_to_rows(out, B, NQ * D).cpu() if frag else out[:B].cpu())
        results.append(res.cpu())
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    assert torch.equal(results[0].view(torch.int16), results[1].view(torch.int16))


@pytest.mark.parametrize("rows", [5, 8, 17, 40])
def test_glu_to_down_in_fragment_order_bitexact(lib, rows):
    """gate/up writing SwiGLU in fragment order and down reading it that way
    give the same bits as the row-major handover."""
    from qdec import capi
    from qdec.runtime import role_plan
    x = rnd(rows, H, scale=3.0, seed=41).to(DEV)
    Wgu = pack(lib, rnd(2 * I, H, scale=0.02, seed=42).to(DEV))
    Wd = pack(lib, rnd(H, I, scale=0.02, seed=43).to(DEV))
    nw = rnd(H, scale=0.2, seed=44).to(DEV)
    res0 = rnd(rows, H, scale=2.0, seed=45).to(DEV)
    pg, pd = role_plan(I, H, "gate_up"), role_plan(H, I, "down")
    acts, results = [], []
    for frag in (0, 1):
        act = torch.zeros((rows + 15) // 16 * 16, I, dtype=torch.bfloat16, device=DEV)
        g1 = Gemm(lib, capi.NORM_IN | capi.GLU, I, H, ksplit=pg[0], waves=pg[1])
        a = capi.GemmArgs(x=x.data_ptr(), w=Wgu.data_ptr(), out=act.data_ptr(), norm_w=nw.data_ptr(), eps=1e-6,
                          rows=rows, n=I, k=H, flags=capi.NORM_IN | capi.GLU, ksplit=pg[0], waves=pg[1],
                          tiles_per_wg=1, out_frag=frag, partial=g1.partial.data_ptr(), counters=g1.counters.data_ptr())
        lib.gemm(a, stream())
        res = res0.clone()
        d = capi.GemmArgs(x=act.data_ptr(), w=Wd.data_ptr(), res=res.data_ptr(), eps=1e-6, rows=rows, n=H, k=I,
                          flags=capi.RES_OUT, ksplit=pd[0], waves=pd[1], tiles_per_wg=1, x_frag=frag,
                          partial=g1.partial.data_ptr(), counters=g1.counters.data_ptr())
        lib.gemm(d, stream())
        torch.cuda.synchronize()
        acts.append(frag_to_rows(act, rows, I).cpu() if frag else act[:rows].cpu())
        results.append(res.cpu())
    assert torch.equal(acts[0].view(torch.int16), acts[1].view(torch.int16))
    assert torch.equal(results[0].view(torch.int16), results[1].view(torch.int16))


@pytest.mark.parametrize("frag", [0, 1])
@pytest.mark.parametrize("rows", [1, 2, 3, 5, 6, 7, 8, 17, 24, 32])
def test_glu_resident_bitexact(lib, rows, frag):
    """gate/up with its rows resident in LDS (one workgroup per CU; at 6..8
    rows normalising the rows itself, no pre-pass; at 17..32 copying the
    pre-pass's rows in) gives the bits of the pre-pass + direct path, in
    row-major and fragment-order output, and agrees with the oracle.  Rows
    of very different magnitude check that each row keeps its own
    statistic."""
    from qdec import capi
    from qdec.runtime import role_plan
    ks, waves, _ = role_plan(I, H, "gate_up")
    x = rnd(rows, H, scale=3.0, seed=90 + rows)
    x[min(1, rows - 1)] = (x[min(1, rows - 1)].float() * 40.0).to(torch.bfloat16)
    x[rows - 1] = (x[rows - 1].float() * 0.01).to(torch.bfloat16)
    W = rnd(2 * I, H, scale=0.02, seed=91)
    nw = bf16(1 + 0.2 * torch.randn(H, generator=torch.Generator().manual_seed(92))).to(torch.bfloat16)
    xd, Wt, nwd = x.to(DEV), pack(lib, W.to(DEV)), nw.to(DEV)
    g = Gemm(lib, capi.NORM_IN | capi.GLU, I, H, ksplit=ks, waves=waves)
    outs = []
    for resident in (0, 1):
        out = torch.full(((rows + 15) // 16 * 16, I), float("nan"), dtype=torch.bfloat16, device=DEV)
        a = capi.GemmArgs(x=xd.data_ptr(), w=Wt.data_ptr(), out=out.data_ptr(), norm_w=nwd.data_ptr(), eps=1e-6,
                          rows=rows, n=I, k=H, flags=capi.NORM_IN | capi.GLU, ksplit=ks, waves=waves,
                          tiles_per_wg=1, out_frag=frag, resident=resident, partial=g.partial.data_ptr(),
                          counters=g.counters.data_ptr())
        pb, _ = lib.gemm_workspace(a)
        assert pb <= g.partial.numel() * 4
        assert (pb == 0) == bool(resident and rows <= 8 or rows < 6)
        assert lib.gemm_prepass(a)[0] == (not (resident and rows <= 8) and rows >= 6)
        lib.gemm(a, stream())
        torch.cuda.synchronize()
        outs.append(frag_to_rows(out, rows, I).cpu() if frag else out[:rows].cpu())
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    xin = rms_norm(x.float(), nw.float(), 1e-6)
    agree(outs[1], silu_mul(linear(xin, W[:I].float()), linear(xin, W[I:].float())), min_exact=0.97)


@pytest.mark.parametrize("frag", [0, 1])
@pytest.mark.parametrize("rows", [1, 3, 5, 6, 7, 8, 17, 24, 32])
def test_qkv_resident_bitexact(lib, rows, frag):
    """QKV (NORM_IN alone) on the resident plan with single tiles -- 1 or 2
    tiles per workgroup; up to 8 rows the workgroup normalises its rows into
    LDS itself, at 17..32 it copies the pre-pass's rows in -- gives the bits
    of the plain call, in row-major and fragment-order output, and agrees
    with the oracle."""
    from qdec import capi
    from qdec.runtime import role_plan
    n = 6144
    ks, waves, _ = role_plan(n, H, "qkv", batch=rows)
    x = rnd(rows, H, scale=3.0, seed=80 + rows)
    x[0] = (x[0].float() * 40.0).to(torch.bfloat16)
    x[rows - 1] = (x[rows - 1].float() * 0.01).to(torch.bfloat16)
    W = rnd(n, H, scale=0.02, seed=81)
    nw = bf16(1 + 0.2 * torch.randn(H, generator=torch.Generator().manual_seed(82))).to(torch.bfloat16)
    xd, Wt, nwd = x.to(DEV), pack(lib, W.to(DEV)), nw.to(DEV)
    g = Gemm(lib, capi.NORM_IN, n, H, ksplit=ks, waves=waves)
    outs = []
    for resident in (0, 1):
        out = torch.full(((rows + 15) // 16 * 16, n), float("nan"), dtype=torch.bfloat16, device=DEV)
        a = capi.GemmArgs(x=xd.data_ptr(), w=Wt.data_ptr(), out=out.data_ptr(), norm_w=nwd.data_ptr(), eps=1e-6,
                          rows=rows, n=n, k=H, flags=capi.NORM_IN, ksplit=ks, waves=waves, tiles_per_wg=1,
                          out_frag=frag, resident=resident, partial=g.partial.data_ptr(),
                          counters=g.counters.data_ptr())
        pb, _ = lib.gemm_workspace(a)
        assert pb <= g.partial.numel() * 4
        if resident and rows <= 8:
            assert pb == 0 and not lib.gemm_prepass(a)[0]
        lib.gemm(a, stream())
        torch.cuda.synchronize()
        outs.append(frag_to_rows(out, rows, n).cpu() if frag else out[:rows].cpu())
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    agree(outs[1], linear(rms_norm(x.float(), nw.float(), 1e-6), W.float()), min_exact=0.97)


@pytest.mark.parametrize("n", [32, 48, 64, 4096])
def test_norm_in_resident_small_grids_bitexact(lib, n):
    """NORM_IN alone on the resident plan for matrices of 2, 3, 4 and 256
    tiles: every workgroup gets two tiles or one beside the normalising
    waves, and the output equals the plain call's bits."""
    from qdec import capi
    rows = 8
    x = rnd(rows, H, scale=2.0, seed=70 + n)
    W = rnd(n, H, scale=0.02, seed=71)
    nw = bf16(1 + 0.2 * torch.randn(H, generator=torch.Generator().manual_seed(72))).to(torch.bfloat16)
    xd, Wt, nwd = x.to(DEV), pack(lib, W.to(DEV)), nw.to(DEV)
    g = Gemm(lib, capi.NORM_IN, n, H)
    outs = []
    for resident in (0, 1):
        out = torch.full((rows, n), float("nan"), dtype=torch.bfloat16, device=DEV)
        a = capi.GemmArgs(x=xd.data_ptr(), w=Wt.data_ptr(), out=out.data_ptr(), norm_w=nwd.data_ptr(), eps=1e-6,
                          rows=rows, n=n, k=H, flags=capi.NORM_IN, ksplit=1, waves=4, tiles_per_wg=1,
                          resident=resident, partial=g.partial.data_ptr(), counters=g.counters.data_ptr())
        lib.gemm(a, stream())
        torch.cuda.synchronize()
        outs.append(out.cpu())
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    agree(outs[1], linear(rms_norm(x.float(), nw.float(), 1e-6), W.float()), min_exact=0.97)


@pytest.mark.parametrize("rows", [8, 24])
@pytest.mark.parametrize("n", [32, 48, 80, 1040])
def test_glu_resident_half_pairs_bitexact(lib, n, rows):
    """gate/up on the resident plan with workgroups owning runs of half
    pairs: 2, 3, 5 and 65 tile pairs give workgroups of two whole pairs, a
    whole pair beside a half pair (either side), two whole pairs beside a
    half pair, and mixes of four and five half pairs.  The output equals the
    plain call's bits."""
    from qdec import capi
    x = rnd(rows, H, scale=2.0, seed=60 + n + rows)
    x[rows - 1] = (x[rows - 1].float() * 0.05).to(torch.bfloat16)
    W = rnd(2 * n, H, scale=0.02, seed=61)
    nw = bf16(1 + 0.2 * torch.randn(H, generator=torch.Generator().manual_seed(62))).to(torch.bfloat16)
    xd, Wt, nwd = x.to(DEV), pack(lib, W.to(DEV)), nw.to(DEV)
    g = Gemm(lib, capi.NORM_IN | capi.GLU, n, H)
    outs = []
    for resident in (0, 1):
        out = torch.full(((rows + 15) // 16 * 16, n), float("nan"), dtype=torch.bfloat16, device=DEV)
        a = capi.GemmArgs(x=xd.data_ptr(), w=Wt.data_ptr(), out=out.data_ptr(), norm_w=nwd.data_ptr(), eps=1e-6,
                          rows=rows, n=n, k=H, flags=capi.NORM_IN | capi.GLU, ksplit=1, waves=4, tiles_per_wg=1,
                          resident=resident, partial=g.partial.data_ptr(), counters=g.counters.data_ptr())
        lib.gemm(a, stream())
        torch.cuda.synchronize()
        outs.append(out[:rows].cpu())
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    xin = rms_norm(x.float(), nw.float(), 1e-6)
    agree(outs[1], silu_mul(linear(xin, W[:n].float()), linear(xin, W[n:].float())), min_exact=0.97)


@pytest.mark.parametrize("role,rows", [("down", 1), ("down", 2), ("down", 3), ("down", 5), ("down", 8), ("o", 1),
                                      ("o", 3), ("o", 4), ("o", 8)])
def test_res_out_rows_in_lds_bitexact(lib, role, rows):
    """A RES_OUT call with its rows copied into LDS first (resident: a
    weights-only ring) gives the bits of the same call without, and agrees
    with the oracle."""
    from qdec import capi
    from qdec.runtime import role_plan
    n, k = {"down": (H, I), "o": (H, 4096)}[role]
    ks, waves, _ = role_plan(n, k, role, batch=rows)
    x = rnd(rows, k, scale=1.0, seed=95 + rows)
    W = rnd(n, k, scale=0.02, seed=96)
    res0 = rnd(rows, n, scale=2.0, seed=97)
    xd, Wt = x.to(DEV), pack(lib, W.to(DEV))
    g = Gemm(lib, capi.RES_OUT, n, k, ksplit=ks, waves=waves)
    outs = []
    for resident in (0, 1):
        res = res0.to(DEV).clone()
        a = capi.GemmArgs(x=xd.data_ptr(), w=Wt.data_ptr(), res=res.data_ptr(), eps=1e-6, rows=rows, n=n, k=k,
                          flags=capi.RES_OUT, ksplit=ks, waves=waves, tiles_per_wg=1, resident=resident,
                          partial=g.partial.data_ptr(), counters=g.counters.data_ptr())
        lib.gemm(a, stream())
        torch.cuda.synchronize()
        outs.append(res.cpu())
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    agree(outs[1], bf16(res0.float() + linear(x.float(), W.float())))


@pytest.mark.parametrize("rows", [17, 24, 32])
def test_down_split_parts_in_lds_bitexact(lib, rows):
    """The split down projection with each k part's rows copied into LDS once
    per workgroup (resident) leaves the same fp32 partials as without, and
    their sum agrees with the oracle."""
    from qdec import capi
    from qdec.runtime import DOWN_SPLIT, role_plan
    ks, waves, _ = role_plan(H, I, "down", batch=32)
    assert ks == DOWN_SPLIT and waves == 4
    mt = (rows + 15) // 16
    x = rnd(rows, I, scale=1.0, seed=101 + rows)
    W = rnd(H, I, scale=0.02, seed=102)
    xf = torch.zeros(mt * 16 * I, dtype=torch.bfloat16)
    for m in range(rows):  # fragment order (include/qdec.h)
        for c0 in range(0, I, 8):
            off = ((c0 // 32 * mt + m // 16) * 64 + m % 16 + 16 * (c0 % 32 // 8)) * 8
            xf[off:off + 8] = x[m, c0:c0 + 8]
    xd, Wt = xf.to(DEV), pack(lib, W.to(DEV))
    outs = []
    for resident in (0, 1):
        parts = torch.full((ks, rows, H), float("nan"), dtype=torch.float32, device=DEV)
        res = torch.zeros(rows, H, dtype=torch.bfloat16, device=DEV)
        a = capi.GemmArgs(x=xd.data_ptr(), w=Wt.data_ptr(), res=res.data_ptr(), eps=1e-6, rows=rows, n=H, k=I,
                          flags=capi.RES_OUT, ksplit=ks, waves=waves, tiles_per_wg=2, x_frag=1,
                          parts_out=parts.data_ptr(), resident=resident)
        lib.gemm(a, stream())
        torch.cuda.synchronize()
        outs.append(parts.cpu())
    assert torch.equal(outs[0].view(torch.int32), outs[1].view(torch.int32))
    ref = linear(x.float(), W.float())
    got = outs[1].sum(0)
    assert (got - ref).abs().max().item() <= 0.02 * ref.abs().max().item()


@pytest.mark.parametrize("rows,resident", [(5, 0), (24, 0), (24, 1), (32, 1)])
def test_glu_merges_split_update_bitexact(lib, rows, resident):
    """gate/up with a pending split residual update (x_parts: a split O
    projection's partials) merges it in its pre-pass: x_merged holds
    bf16(x + bf16(p0 + p1)) and the output has the bits of the same call on
    the merged rows."""
    from qdec import capi
    from qdec.runtime import role_plan
    ks, waves, _ = role_plan(I, H, "gate_up")
    x = rnd(rows, H, scale=2.0, seed=111 + rows)
    parts = (torch.randn(2, rows, H, generator=torch.Generator().manual_seed(112)) * 0.5).float()
    W = rnd(2 * I, H, scale=0.02, seed=113)
    nw = bf16(1 + 0.2 * torch.randn(H, generator=torch.Generator().manual_seed(114))).to(torch.bfloat16)
    merged_ref = bf16(x.float() + bf16(parts[0] + parts[1])).to(torch.bfloat16)
    xd, pd, Wt, nwd = x.to(DEV), parts.to(DEV), pack(lib, W.to(DEV)), nw.to(DEV)
    g = Gemm(lib, capi.NORM_IN | capi.GLU, I, H, ksplit=ks, waves=waves)
    outs = []
    for with_parts in (True, False):
        out = torch.zeros(((rows + 15) // 16 * 16, I), dtype=torch.bfloat16, device=DEV)
        merged = torch.full((rows, H), float("nan"), dtype=torch.bfloat16, device=DEV)
        src = xd if with_parts else merged_ref.to(DEV)
        a = capi.GemmArgs(x=src.data_ptr(), w=Wt.data_ptr(), out=out.data_ptr(), norm_w=nwd.data_ptr(), eps=1e-6,
                          rows=rows, n=I, k=H, flags=capi.NORM_IN | capi.GLU, ksplit=ks, waves=waves,
                          tiles_per_wg=1, resident=resident, partial=g.partial.data_ptr(),
                          counters=g.counters.data_ptr())
        if with_parts:
            a.x_parts, a.x_nparts, a.x_merged = pd.data_ptr(), 2, merged.data_ptr()
        lib.gemm(a, stream())
        torch.cuda.synchronize()
        if with_parts:
            assert torch.equal(merged.cpu().view(torch.int16), merged_ref.view(torch.int16))
        outs.append(out[:rows].cpu())
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))


def attn_oracle(c, B, T):
    qkv = c["qkv"].float().view(B, T, NQ + 2 * NKV, D)
    kc, vc = c["kc"].float().clone(), c["vc"].float().clone()
    outs = torch.zeros(B, T, NQ, D)
    for b in range(B):
        L = c["lens"][b]
        pos = torch.arange(L, L + T)
        cs, sn = c["cos"][pos][:, None, :], c["sin"][pos][:, None, :]
        q = head_norm_rope(qkv[b, :, :NQ], c["qn"].float(), cs, sn, 1e-6)
        k = head_norm_rope(qkv[b, :, NQ:NQ + NKV], c["kn"].float(), cs, sn, 1e-6)
        v = qkv[b, :, NQ + NKV:]
        kc[b, :, pos] = k.transpose(0, 1)
        vc[b, :, pos] = v.transpose(0, 1)
        cap = kc.shape[2]
        for h in range(NQ):
            kvh = h // (NQ // NKV)
            vis = torch.arange(cap)[None, :] <= pos[:, None]
            outs[b, :, h] = attention(q[:, h], kc[b, kvh], vc[b, kvh], vis, D ** -0.5)
    return outs.view(B * T, NQ * D), kc, vc


@pytest.mark.parametrize("B,T,lens,cap,chunk,waves", [
    (1, 1, [0], 64, 64, 4),
    (1, 1, [31], 64, 64, 4),
    (1, 1, [100], 256, 64, 4),
    (2, 1, [63, 200], 256, 64, 4),
    (3, 1, [5, 64, 129], 192, 128, 4),
    (1, 4, [60], 128, 64, 4),
    (2, 9, [0, 170], 256, 64, 4),
    (4, 9, [1000, 1017, 31, 64], 1056, 96, 4),
    (1, 1, [100], 256, 64, 8),
    (3, 1, [5, 64, 129], 192, 128, 8),
    (2, 8, [0, 170], 256, 64, 8),
    (8, 2, [1000, 1017, 31, 64, 0, 511, 512, 700], 1056, 512, 8),
    (2, 1, [4000, 3100], 4384, 576, 4),
    (1, 3, [2200], 2336, 320, 4),
])
def test_attention_vs_oracle(lib, B, T, lens, cap, chunk, waves):
    c = attn_case(lib, B, T, lens, cap, chunk, seed=B * 100 + T * 10 + lens[0], waves=waves)
    check_attention(c, B, T, lens)


# Strided chunks (chunk c takes blocks c, c + C, ...): config 3's plan (batch
# 8, 1568-slot cache, 4 chunks of 416, 8 waves) at lengths around its decode,
# lengths that leave chunks empty, and verify-shaped rows over block bounds.
@pytest.mark.parametrize("B,T,lens,cap,chunk,waves", [
    (8, 1, [1024, 1023, 1055, 1300, 0, 31, 96, 1535], 1568, 416, 8),
    (8, 2, [1000, 1017, 31, 64, 0, 511, 512, 700], 1056, 288, 8),
    (2, 8, [0, 170], 256, 64, 8),
    (3, 1, [5, 64, 129], 192, 64, 8),
    (2, 4, [3, 170], 256, 64, 8),
    (1, 1, [4000], 4384, 576, 8),
])
def test_attention_strided_vs_oracle(lib, B, T, lens, cap, chunk, waves):
    c = attn_case(lib, B, T, lens, cap, chunk, seed=B * 100 + T * 10 + lens[0] + 1, waves=waves, strided=1)
    check_attention(c, B, T, lens)


# Config 4's decode attention as the engine plans it (qdec.runtime attn_chunk /
# attn_waves / FRAG_ROWS for batch 32, capacity 4096 + 256 + 2 -> 4384): one
# whole-cache chunk per (sequence, kv head), 8 waves, output in fragment order
# for the O projection.  Lengths 4090..4100 as at the start of config 4's
# decode (4096 cached), plus short and boundary ones; the verify-shaped
# T = 2 case is batch 20's plan.
C4_LENS = [4090 + i % 11 for i in range(27)] + [0, 31, 32, 1000, 4351]


@pytest.mark.parametrize("B,T,lens,cap", [(32, 1, C4_LENS, 4384), (20, 2, C4_LENS[:17] + [5, 64, 4382], 4384)])
def test_attention_config4_vs_oracle(lib, B, T, lens, cap):
    from qdec.runtime import FRAG_ROWS, attn_chunk, attn_waves
    chunk, waves = attn_chunk(B, NKV, cap), attn_waves(B)
    assert chunk == cap and waves == 8 and B * T >= FRAG_ROWS
    c = attn_case(lib, B, T, lens, cap, chunk, seed=4096 + B, waves=waves, out_frag=1)
    check_attention(c, B, T, lens)


def check_attention(c, B, T, lens):
    ref, kc, vc = attn_oracle(c, B, T)
    agree(c["out"], ref, min_exact=0.0, tol=0.02)
    # raw V bit-exact in the cache; new K (normed, rotated) equal but for rare
    # one-ulp flips of a rounding boundary (1/sqrtf and the wave sum order
    # against torch.rsqrt); every other slot untouched
    assert torch.equal(c["v_after"].float(), v_layout(vc.to(torch.bfloat16)).float())
    k_after, k_before = c["k_after"].float(), c["kc"].float()
    new = torch.zeros(k_after.shape[:3], dtype=torch.bool)
    for b, L in enumerate(lens):
        new[b, :, L:L + T] = True
    assert torch.equal(k_after[~new], k_before[~new])
    near_exact(k_after[new], kc[new])


@pytest.mark.parametrize("cap,chunk,L,T,waves,strided", [
    (256, 64, 100, 9, 4, 0), (256, 64, 63, 9, 4, 0), (1056, 96, 1000, 9, 4, 0), (512, 128, 0, 9, 4, 0),
    (256, 64, 100, 8, 8, 0), (1056, 512, 1000, 8, 8, 0),
    (1056, 96, 1000, 8, 8, 1), (256, 64, 100, 8, 8, 1), (1568, 416, 1020, 8, 8, 1),
    (1056, 288, 90, 8, 8, 1)])
def test_attention_t_invariance_bitexact(lib, cap, chunk, L, T, waves, strided):
    """Verify row t (t_rows = T) at position L + t equals the plain T = 1 step
    at that position, bit for bit, given the same cache contents (4 waves up
    to 16 rows per sequence, 8 waves up to 8)."""
    B = 2
    c9 = attn_case(lib, B, T, [L, L + 3], cap, chunk, seed=77, waves=waves, strided=strided)
    for t in range(T):
        # plain step at position L + t: cache holds the verify pass's K/V for
        # slots < L + t (the first pass already wrote them) and the same qkv row.
        pos_lens = [L + t, L + 3 + t]
        one = attn_case_from(lib, c9, B, T, t, pos_lens, cap, chunk, waves=waves, strided=strided)
        for b in range(B):
            assert torch.equal(one[b].view(torch.int16), c9["out"][b * T + t].view(torch.int16)), (t, b)


def attn_case_from(lib, c9, B, T, t, lens, cap, chunk, waves=4, strided=0):
    """Run T = 1 on row t of every sequence of case c9, with the cache as the
    T = 9 call left it."""
    from qdec import capi
    W = (NQ + 2 * NKV) * D
    qkv = c9["qkv"].view(B, T, W)[:, t].contiguous()
    dq, dqn, dkn = qkv.to(DEV), c9["qn"].to(DEV), c9["kn"].to(DEV)
    dcos, dsin = c9["cos"].to(torch.bfloat16).to(DEV), c9["sin"].to(torch.bfloat16).to(DEV)
    dl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    dk, dv = c9["k_after"].to(DEV).clone(), c9["v_after"].to(DEV).clone()
    out = torch.zeros(B, NQ * D, dtype=torch.bfloat16, device=DEV)
    a = capi.AttnArgs()
    a.qkv, a.q_norm_w, a.k_norm_w, a.cos_tab, a.sin_tab, a.lens = (dq.data_ptr(), dqn.data_ptr(), dkn.data_ptr(),
                                                                 dcos.data_ptr(), dsin.data_ptr(), dl.data_ptr())
    a.k_cache, a.v_cache, a.out = dk.data_ptr(), dv.data_ptr(), out.data_ptr()
    a.eps, a.sm_scale = 1e-6, D ** -0.5
    a.batch, a.t_rows, a.nq, a.nkv, a.head_dim, a.cap, a.chunk = B, 1, NQ, NKV, D, cap, chunk
    a.waves, a.strided = waves, strided
    pb, cb = lib.attn_workspace(a)
    part = torch.zeros(max(pb, 16) // 4, dtype=torch.float32, device=DEV)
    cnt = torch.zeros(max(cb, 4) // 4, dtype=torch.int32, device=DEV)
    a.partial, a.counters = part.data_ptr(), cnt.data_ptr()
    lib.attn(a, stream())
    torch.cuda.synchronize()
    return out.cpu()


# ---------------------------------------------------------- speculation

@pytest.mark.parametrize("K", [6, 0])
def test_draft_and_accept_vs_oracle(lib, K):
    """k = 0 is the plain step of the acceptance gate: only the current
    token is fed and one pick is appended."""
    from qdec import capi
    import random
    rng = random.Random(3 + K)
    B, cap = 5, 96
    T = K + 1
    for trial in range(20):
        hist = [[rng.randint(0, 4) for _ in range(cap)] for _ in range(B)]
        lens = [rng.randint(0, cap - 2 * T - 1) for _ in range(B)]
        dh = torch.tensor(hist, dtype=torch.int64, device=DEV)
        dl = torch.tensor(lens, dtype=torch.int32, device=DEV)
        ids = torch.zeros(B * T, dtype=torch.int64, device=DEV)
        dr = torch.zeros(max(B * K, 1), dtype=torch.int64, device=DEV)
        d = capi.DraftArgs(hist=dh.data_ptr(), lens=dl.data_ptr(), ids=ids.data_ptr(), draft=dr.data_ptr(),
                           batch=B, cap=cap, primary=3, backoff=2, k=K)
        lib.ngram_draft(d, stream())
        torch.cuda.synchronize()
        exp_ids, exp_dr = [], []
        for b in range(B):
            i, dd = draft_ref(hist[b], lens[b], 3, 2, K)
            exp_ids += i
            exp_dr += dd
        assert ids.cpu().tolist() == exp_ids and dr.cpu().tolist()[:B * K] == exp_dr
        # accept with model outputs that agree with the draft for a random prefix
        out_tok = []
        for b in range(B):
            agree_n = rng.randint(0, K)
            row = [exp_ids[b * T + 1 + t] if t < agree_n else rng.randint(5, 9) for t in range(K)]
            out_tok += row + [rng.randint(0, 9)]
        stop = rng.randint(0, cap)
        dot = torch.tensor(out_tok, dtype=torch.int64, device=DEV)
        nacc = torch.zeros(B, dtype=torch.int32, device=DEV)
        a = capi.AcceptArgs(out_tok=dot.data_ptr(), draft=dr.data_ptr(), hist=dh.data_ptr(), lens=dl.data_ptr(),
                            naccept=nacc.data_ptr(), batch=B, cap=cap, k=K, stop_len=stop)
        lib.spec_accept(a, stream())
        torch.cuda.synchronize()
        for b in range(B):
            h = list(hist[b])
            na, nl = accept_ref(out_tok[b * T:(b + 1) * T], exp_dr[b * K:(b + 1) * K], h, lens[b], K, stop)
            assert nacc[b].item() == na and dl[b].item() == nl and dh[b].cpu().tolist() == h


# --------------------------------------------- split residual update pipeline

@pytest.mark.parametrize("rows", [1, 3, 9, 17, 32])
def test_down_split_merged_by_next_norm_in_call(lib, rows):
    """The engine's down projection (k split 4 ways, partials left in
    parts_out) followed by the next layer's QKV and the lm_head merging them
    (x_parts): the merged residual equals bf16(res + bf16(act . Wd^T)) within
    one rounding, the QKV output matches the oracle on it, and every merged
    row and output is bit-identical to the one-row call's (a verify pass
    reproduces plain decode)."""
    from qdec import capi
    from qdec.runtime import LM_TILES_BATCHED, role_plan
    pd, pq = role_plan(H, I, "down", batch=32), role_plan(6144, H, "qkv")
    assert pd[0] > 1
    big = 32
    act_all = rnd(big, I, scale=1.0, seed=81)
    res_all = rnd(big, H, scale=2.0, seed=82)
    Wd = rnd(H, I, scale=0.02, seed=83)
    Wq = rnd(6144, H, scale=0.02, seed=84)
    E = rnd(2048, H, scale=0.02, seed=85)
    nw = bf16(1 + 0.2 * torch.randn(H, generator=torch.Generator().manual_seed(86))).to(torch.bfloat16)
    Wdt, Wqt, Et = pack(lib, Wd.to(DEV)), pack(lib, Wq.to(DEV)), pack(lib, E.to(DEV))

    def run(idx):
        R = len(idx)
        act, res = act_all[idx].contiguous().to(DEV), res_all[idx].contiguous().to(DEV)
        parts = torch.full((pd[0], R, H), float("nan"), dtype=torch.float32, device=DEV)
        d = capi.GemmArgs(x=act.data_ptr(), w=Wdt.data_ptr(), res=res.data_ptr(), eps=1e-6, rows=R, n=H, k=I,
                          flags=capi.RES_OUT, ksplit=pd[0], waves=pd[1], tiles_per_wg=1,
                          parts_out=parts.data_ptr())
        lib.gemm(d, stream())
        merged = torch.zeros(R, H, dtype=torch.bfloat16, device=DEV)
        out = torch.zeros(R, 6144, dtype=torch.bfloat16, device=DEV)
        g = Gemm(lib, capi.NORM_IN, 6144, H, ksplit=pq[0], waves=pq[1])
        q = capi.GemmArgs(x=res.data_ptr(), w=Wqt.data_ptr(), out=out.data_ptr(), norm_w=nw.to(DEV).data_ptr(),
                          eps=1e-6, rows=R, n=6144, k=H, flags=capi.NORM_IN, ksplit=pq[0], waves=pq[1],
                          tiles_per_wg=1, x_parts=parts.data_ptr(), x_nparts=pd[0], x_merged=merged.data_ptr(),
                          partial=g.partial.data_ptr(), counters=g.counters.data_ptr())
        nwd = nw.to(DEV)
        q.norm_w = nwd.data_ptr()
        lib.gemm(q, stream())
        merged2 = torch.zeros(R, H, dtype=torch.bfloat16, device=DEV)
        ids = torch.full((R,), -1, dtype=torch.int64, device=DEV)
        lm = capi.GemmArgs(x=res.data_ptr(), w=Et.data_ptr(), norm_w=nwd.data_ptr(), ids_out=ids.data_ptr(), eps=1e-6,
                           rows=R, n=2048, k=H, flags=capi.NORM_IN | capi.ARGMAX, ksplit=1, waves=4,
                           tiles_per_wg=LM_TILES_BATCHED if R > 1 else 4, x_parts=parts.data_ptr(),
                           x_nparts=pd[0], x_merged=merged2.data_ptr(),
                           partial=g.partial.data_ptr(), counters=g.counters.data_ptr())
        lib.gemm(lm, stream())
        torch.cuda.synchronize()
        assert torch.equal(merged, merged2)
        return merged.cpu(), out.cpu(), ids.cpu()

    idx = list(range(rows)) if rows < big else list(range(big))
    merged, out, ids = run(idx)
    want_h = bf16(res_all[idx].float() + linear(act_all[idx].float(), Wd.float()))
    agree(merged, want_h, min_exact=0.98)
    agree(out, linear(rms_norm(merged.float(), nw.float(), 1e-6), Wq.float()), min_exact=0.98)
    one_m, one_o, one_i = run([idx[-1]])
    assert torch.equal(one_m[0].view(torch.int16), merged[-1].view(torch.int16))
    assert torch.equal(one_o[0].view(torch.int16), out[-1].view(torch.int16))
    assert one_i[0] == ids[-1]


@pytest.mark.parametrize("rows", [17, 24, 32])
@pytest.mark.parametrize("role", ["qkv", "o", "gate_up", "down", "down_split", "lm"])
def test_two_tiles_per_wave_bitexact(lib, role, rows):
    """At two M tiles a workgroup with an even number of output tiles runs two
    per wave (each activation fragment feeds both; gate/up keeps one per wave
    and runs its two in turn): every output bit, the split partials and the
    argmax equal the one-tile-per-workgroup call's, for each role in the
    engine's layouts and batch-32 plans (fragment-order activations into O
    and down, SwiGLU written in fragment order, the normalisation pre-pass of
    QKV, the 8-tile lm_head)."""
    from qdec import capi
    from qdec.runtime import LM_TILES_BATCHED, WIDE_TILES, role_plan
    assert WIDE_TILES == 2
    n, k, flags, r = {"qkv": (6144, H, capi.NORM_IN, "qkv"), "o": (H, 4096, capi.RES_OUT, "o"),
                      "gate_up": (I, H, capi.NORM_IN | capi.GLU, "gate_up"), "down": (H, I, capi.RES_OUT, "down"),
                      "down_split": (H, I, capi.RES_OUT, "down"), "lm": (V, H, capi.NORM_IN | capi.ARGMAX, "lm")}[role]
    ks, waves, _ = role_plan(n, k, r, batch=1 if role == "down" else 32)
    # at batch 32 the down and O projections split k (partials to parts_out)
    assert (ks > 1) == (role in ("down_split", "o"))
    seed = (zlib.crc32(role.encode()) + 5 * rows) % 1000
    mt_rows = (rows + 15) // 16 * 16
    frag = role in ("o", "down", "down_split")
    # fragment order covers whole M tiles (lanes past the last row use zeros)
    x = rnd(mt_rows if frag else rows, k, scale=1.0 if frag else 3.0, seed=seed).to(DEV)
    W = pack(lib, rnd(2 * n if flags & capi.GLU else n, k, scale=0.02, seed=seed + 1).to(DEV))
    nw = (1 + 0.2 * rnd(k, seed=seed + 2).float()).to(torch.bfloat16).to(DEV)
    res0 = rnd(rows, n, scale=2.0, seed=seed + 3).to(DEV)
    ws = Gemm(lib, flags, n, k)

    def run(tiles):
        a = capi.GemmArgs(x=x.data_ptr(), w=W.data_ptr(), eps=1e-6, rows=rows, n=n, k=k, flags=flags, ksplit=ks,
                          waves=waves, tiles_per_wg=tiles, partial=ws.partial.data_ptr(),
                          counters=ws.counters.data_ptr())
        outs = []
        if frag:
            a.x_frag = 1
            res = res0.clone()
            a.res = res.data_ptr()
            outs.append(res)
            if ks > 1:
                parts = torch.full((ks, rows, n), float("nan"), dtype=torch.float32, device=DEV)
                a.parts_out = parts.data_ptr()
                outs.append(parts)
        else:
            a.norm_w = nw.data_ptr()
            out = torch.zeros(mt_rows if flags & capi.GLU else rows, n, dtype=torch.bfloat16, device=DEV)
            a.out = out.data_ptr()
            outs.append(out)
            if flags & capi.GLU:
                a.out_frag = 1
            if flags & capi.ARGMAX:
                ids = torch.full((rows,), -1, dtype=torch.int64, device=DEV)
                a.ids_out = ids.data_ptr()
                outs.append(ids)
        pb, _ = lib.gemm_workspace(a)
        assert pb <= ws.partial.numel() * 4
        lib.gemm(a, stream())
        torch.cuda.synchronize()
        assert int(ws.counters.abs().sum()) == 0
        return [t.cpu() for t in outs]

    wide = LM_TILES_BATCHED if role == "lm" else WIDE_TILES
    one, two = run(1), run(wide)
    for t1, t2 in zip(one, two):
        if t1.dtype == torch.bfloat16:
            t1, t2 = t1.view(torch.int16), t2.view(torch.int16)
        elif t1.dtype == torch.float32:
            t1, t2 = t1.view(torch.int32), t2.view(torch.int32)
        assert torch.equal(t1, t2)
    if role in ("down_split", "o"):
        assert not torch.isnan(two[1]).any()  # every partial written


# ------------------------------------------------------ invalid inputs, bands

def test_invalid_length_and_id_give_nan_not_stale_output(lib):
    """A cache length outside [0, cap - t_rows] touches no cache memory and
    makes that sequence's rows NaN (the other sequences are unaffected); an
    out-of-range token id makes its embedding row NaN.  Both reach the
    argmax as capi.NAN_ID."""
    from qdec import capi
    B, T, cap, chunk = 3, 1, 256, 64
    good = attn_case(lib, B, T, [100, 7, 50], cap, chunk, seed=91)
    for bad_len in (cap, -1):
        c = attn_case(lib, B, T, [100, bad_len, 50], cap, chunk, seed=91, valid=False)
        out = c["out"].float()
        assert bool(torch.isnan(out[1]).all())
        assert torch.equal(out[[0, 2]], good["out"].float()[[0, 2]])
        assert torch.equal(c["k_after"][1], c["kc"][1]) and torch.equal(c["v_after"][1], v_layout(c["vc"])[1])
    vocab, hid = 512, 256
    Et = pack(lib, rnd(vocab, hid, seed=92).to(DEV))
    ids = torch.tensor([3, vocab, -5, 0], dtype=torch.int64, device=DEV)
    h = torch.zeros(4, hid, dtype=torch.bfloat16, device=DEV)
    lib.embed(capi.EmbedArgs(ids=ids.data_ptr(), emb=Et.data_ptr(), h=h.data_ptr(), rows=4, hidden=hid,
                             vocab=vocab), stream())
    torch.cuda.synchronize()
    hn = torch.isnan(h.float()).all(1).cpu().tolist()
    assert hn == [False, True, True, False]
    # an all-NaN row picks NAN_ID
    x = torch.full((2, H), float("nan"), dtype=torch.bfloat16)
    x[1] = rnd(H, seed=93)
    E = pack(lib, rnd(1024, H, scale=0.02, seed=94).to(DEV))
    g = Gemm(lib, capi.NORM_IN | capi.ARGMAX, 1024, H, waves=4, tiles=4)
    out_ids = torch.full((2,), -1, dtype=torch.int64, device=DEV)
    g(x.to(DEV), E, norm_w=torch.ones(H, dtype=torch.bfloat16, device=DEV), ids=out_ids)
    assert out_ids[0].item() == capi.NAN_ID and 0 <= out_ids[1].item() < 1024


CANARY = -12345.0  # bf16-exact


def banded(n_elems, dtype=torch.bfloat16, pad=4096, fill=CANARY):
    """A buffer with canary bands of `pad` elements on both sides of an
    n_elems-element window; returns (whole, window)."""
    whole = torch.full((pad + n_elems + pad,), fill, dtype=dtype, device=DEV)
    return whole, whole[pad:pad + n_elems]


def bands_intact(whole, n_elems, pad=4096, fill=CANARY):
    w = whole.cpu()
    return bool((w[:pad] == fill).all()) and bool((w[pad + n_elems:] == fill).all())


@pytest.mark.parametrize("rows", [1, 5, 17, 40])
def test_gemm_epilogues_stay_in_bounds(lib, rows):
    """GEMM outputs (row-major and fragment order with its padding rows),
    residuals, argmax ids and the argmax / pre-pass workspace written into
    the middle of larger buffers: nothing outside the window changes."""
    from qdec import capi
    from qdec.runtime import LM_TILES_BATCHED, role_plan
    pg, pd = role_plan(I, H, "gate_up"), role_plan(H, I, "down")
    x = rnd(rows, H, scale=3.0, seed=61).to(DEV)
    Wgu = pack(lib, rnd(2 * I, H, scale=0.02, seed=62).to(DEV))
    Wd = pack(lib, rnd(H, I, scale=0.02, seed=63).to(DEV))
    nw = rnd(H, scale=0.2, seed=64).to(DEV)
    frag = 1 if rows >= 17 else 0
    act_elems = ((rows + 15) // 16 * 16 if frag else rows) * I
    act_whole, act = banded(act_elems)
    a = capi.GemmArgs(x=x.data_ptr(), w=Wgu.data_ptr(), out=act.data_ptr(), norm_w=nw.data_ptr(), eps=1e-6,
                      rows=rows, n=I, k=H, flags=capi.NORM_IN | capi.GLU, ksplit=pg[0], waves=pg[1],
                      tiles_per_wg=1, out_frag=frag)
    pb, cb = lib.gemm_workspace(a)
    ws_whole, ws = banded(max(pb, 4) // 4, dtype=torch.float32)
    cnt_whole, cnt = banded(max(cb, 4) // 4, dtype=torch.int32, fill=0)
    a.partial, a.counters = ws.data_ptr(), cnt.data_ptr()
    lib.gemm(a, stream())
    res_whole, res = banded(rows * H)
    res.copy_(rnd(rows * H, scale=2.0, seed=65).to(DEV))
    d = capi.GemmArgs(x=act.data_ptr(), w=Wd.data_ptr(), res=res.data_ptr(), eps=1e-6, rows=rows, n=H, k=I,
                      flags=capi.RES_OUT, ksplit=pd[0], waves=pd[1], tiles_per_wg=1, x_frag=frag)
    dpb, dcb = lib.gemm_workspace(d)
    dws_whole, dws = banded(max(dpb, 4) // 4, dtype=torch.float32)
    dcnt_whole, dcnt = banded(max(dcb, 4) // 4, dtype=torch.int32, fill=0)
    d.partial, d.counters = dws.data_ptr(), dcnt.data_ptr()
    lib.gemm(d, stream())
    # the down call leaving its k-split partials (as the engine runs it from batch 16)
    ps = role_plan(H, I, "down", batch=32)
    parts_elems = ps[0] * rows * H
    parts_whole, parts = banded(parts_elems, dtype=torch.float32)
    d2 = capi.GemmArgs(x=act.data_ptr(), w=Wd.data_ptr(), res=res.data_ptr(), eps=1e-6, rows=rows, n=H, k=I,
                       flags=capi.RES_OUT, ksplit=ps[0], waves=ps[1], tiles_per_wg=1, x_frag=frag,
                       parts_out=parts.data_ptr())
    assert lib.gemm_workspace(d2) == (0, 0)
    lib.gemm(d2, stream())
    # lm_head + argmax (argmax keys in the counters and, from 9 rows, the normalised rows in the workspace)
    Vs = 4096
    E = pack(lib, rnd(Vs, H, scale=0.02, seed=66).to(DEV))
    ids_whole, ids = banded(rows, dtype=torch.int64, fill=-7)
    lm = capi.GemmArgs(x=x.data_ptr(), w=E.data_ptr(), norm_w=nw.data_ptr(), ids_out=ids.data_ptr(), eps=1e-6,
                       rows=rows, n=Vs, k=H, flags=capi.NORM_IN | capi.ARGMAX, ksplit=1, waves=4,
                       tiles_per_wg=LM_TILES_BATCHED if rows > 1 else 4)
    lpb, lcb = lib.gemm_workspace(lm)
    lws_whole, lws = banded(max(lpb, 4) // 4, dtype=torch.float32)
    lcnt_whole, lcnt = banded(max(lcb, 4) // 4, dtype=torch.int32, fill=0)
    lm.partial, lm.counters = lws.data_ptr(), lcnt.data_ptr()
    lib.gemm(lm, stream())
    torch.cuda.synchronize()
    assert bands_intact(act_whole, act_elems), "SwiGLU output"
    assert bands_intact(res_whole, rows * H), "down residual"
    assert bands_intact(dws_whole, max(dpb, 4) // 4) and bands_intact(dcnt_whole, max(dcb, 4) // 4, fill=0)
    assert bands_intact(parts_whole, parts_elems), "down split partials"
    assert bands_intact(ws_whole, max(pb, 4) // 4), "GEMM workspace"
    assert bands_intact(cnt_whole, max(cb, 4) // 4, fill=0) and int(cnt.abs().sum()) == 0, "counters"
    assert bands_intact(ids_whole, rows, fill=-7) and bool((ids >= 0).all()), "argmax ids"
    assert bands_intact(lws_whole, max(lpb, 4) // 4), "argmax workspace"
    assert bands_intact(lcnt_whole, max(lcb, 4) // 4, fill=0) and int(lcnt.abs().sum()) == 0, "argmax counters"


@pytest.mark.parametrize("B,T,lens,cap,chunk,waves,frag,partials,layout", [
    (1, 1, [640], 800, 96, 4, 0, 1, None), (3, 1, [700, 31, 257], 800, 128, 4, 0, 0, None),
    (8, 1, [1024, 1023, 0, 1535, 5, 416, 832, 1300], 1568, 416, 8, 1, 0, "strided"),
    (8, 2, [1024, 1023, 0, 1534, 5, 416, 832, 1300], 1568, 416, 8, 0, 1, "strided"),
    (20, 1, [100 + 37 * i for i in range(20)], 896, 896, 8, 1, 0, None), (4, 4, [60, 0, 7, 100], 128, 64, 4, 0, 0, None),
    # the tiny model's 4 / 2 heads at head_dim 64, and Qwen3-14B's 40 / 8
    (1, 1, [300], 416, 96, 4, 0, 1, (4, 2, 64)), (5, 4, [60, 0, 7, 100, 33], 128, 64, 4, 1, 0, (4, 2, 64)),
    (3, 1, [700, 31, 257], 800, 128, 8, 0, 0, (40, 8, 128))])
def test_attention_stays_in_bounds(lib, B, T, lens, cap, chunk, waves, frag, partials, layout):
    """Attention output (row-major or fragment order), chunk partials and
    counters written into the middle of larger buffers: the bands and every
    cache slot outside the new ones stay untouched."""
    from qdec import capi
    strided = int(layout == "strided")
    NQ, NKV, D = HEADS_4B if layout in (None, "strided") else layout
    g = torch.Generator().manual_seed(cap + B)
    W = (NQ + 2 * NKV) * D
    qkv = (torch.randn(B * T, W, generator=g) * 2).to(torch.bfloat16).to(DEV)
    qn = rnd(D, scale=0.2, seed=71).to(DEV)
    kn = rnd(D, scale=0.2, seed=72).to(DEV)
    kc_whole, kc = banded(B * NKV * cap * D)
    vc_whole, vc = banded(B * NKV * cap * D)
    kc.copy_(torch.randn(kc.numel(), generator=g).to(torch.bfloat16).to(DEV))
    vc.copy_(torch.randn(vc.numel(), generator=g).to(torch.bfloat16).to(DEV))
    kc0, vc0 = kc.clone(), vc.clone()
    cos, sin = rope_tables(cap, D, 5e6, "bf16")
    dcos, dsin = cos.to(torch.bfloat16).to(DEV), sin.to(torch.bfloat16).to(DEV)
    dl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    rows = B * T
    out_elems = ((rows + 15) // 16 * 16 if frag else rows) * NQ * D
    out_whole, out = banded(out_elems)
    a = capi.AttnArgs(qkv=qkv.data_ptr(), q_norm_w=qn.data_ptr(), k_norm_w=kn.data_ptr(), cos_tab=dcos.data_ptr(),
                      sin_tab=dsin.data_ptr(), lens=dl.data_ptr(), k_cache=kc.data_ptr(), v_cache=vc.data_ptr(),
                      out=out.data_ptr(), eps=1e-6, sm_scale=D ** -0.5, batch=B, t_rows=T, nq=NQ, nkv=NKV,
                      head_dim=D, cap=cap, chunk=chunk, waves=waves, out_partials=partials, out_frag=frag,
                      strided=strided)
    pb, cb = lib.attn_workspace(a)
    pw_whole, pw = banded(max(pb, 4) // 4, dtype=torch.float32)
    cw_whole, cw = banded(max(cb, 4) // 4, dtype=torch.int32, fill=0)
    a.partial, a.counters = pw.data_ptr(), cw.data_ptr()
    lib.attn(a, stream())
    torch.cuda.synchronize()
    assert bands_intact(out_whole, out_elems), "attention output"
    assert bands_intact(pw_whole, max(pb, 4) // 4), "chunk partials"
    assert bands_intact(cw_whole, max(cb, 4) // 4, fill=0) and int(cw.abs().sum()) == 0, "counters"
    assert bands_intact(kc_whole, kc.numel()) and bands_intact(vc_whole, vc.numel()), "cache slabs"
    new = torch.zeros(B, NKV, cap, dtype=torch.bool)
    for b, L in enumerate(lens):
        new[b, :, L:L + T] = True
    k_after = kc.view(B, NKV, cap, D).cpu()
    assert torch.equal(k_after[~new], kc0.view(B, NKV, cap, D).cpu()[~new])
    v_rows_after = vc.view(B, NKV, cap // 8, D, 8).transpose(-1, -2).reshape(B, NKV, cap, D).cpu()
    v_rows_before = vc0.view(B, NKV, cap // 8, D, 8).transpose(-1, -2).reshape(B, NKV, cap, D).cpu()
    assert torch.equal(v_rows_after[~new], v_rows_before[~new])
