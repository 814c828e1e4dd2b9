"""Prefill kernels (qdec_rownorm, qdec_prefill_gemm, qdec_prefill_qk,
qdec_prefill_attn) on the GPU.

* The product is pinned bit for bit on small-integer operands (every product
  and partial sum exact in fp32, every result exact in bf16), so a wrong
  tile, fragment or row index cannot hide; on random operands it is compared
  with the fp32 product of the same bf16 values, rounded once.
* Head norm / RoPE / cache fill: the values are the oracle's except for
  rare one-ulp flips (the fp32 sum of squares is reduced in another order,
  and 1/sqrtf is not torch.rsqrt, so a rounding boundary can fall either
  way); values are copied exactly.
* Causal attention is compared with the oracle's decode-formulation
  attention (fp32 scores, bf16 probabilities, fp32 accumulation) within the
  logit tolerance, for prompts starting at slot 0 and chunks continuing a
  cached prefix.
"""

import pytest
import torch

from helpers import near_exact

from oracle.qwen3_oracle import attention, bf16, head_norm_rope, rms_norm, rope_tables, silu_mul

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
NQ, NKV, D = 32, 8, 128
ROW_TILE = 256


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")
    from qdec import capi
    return capi.lib()


def stream():
    return torch.cuda.current_stream().cuda_stream


def round_up(x, m):
    return (x + m - 1) // m * m


def rnd(*shape, scale=1.0, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def small_ints(*shape, lo=-1, hi=1, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(lo, hi + 1, shape, generator=g).to(torch.bfloat16)


def pack(lib, w):
    n, k = w.shape
    src = w.to(DEV).contiguous()
    dst = torch.empty(n * k, dtype=torch.bfloat16, device=DEV)
    lib.pack_tiles(src.data_ptr(), dst.data_ptr(), n, k, stream())
    return dst


def frag_to_rows(buf, rows, cols, nmt):
    """Row-major [rows, cols] view of a buffer in fragment order with nmt M
    tiles: element (m, c) at ((c/32*nmt + m/16)*64 + m%16 + 16*(c%32/8))*8 + c%8."""
    m = torch.arange(rows)[:, None]
    c = torch.arange(cols)[None, :]
    idx = (((c // 32) * nmt + m // 16) * 64 + m % 16 + 16 * ((c % 32) // 8)) * 8 + c % 8
    return buf.flatten()[idx.flatten().to(buf.device)].view(rows, cols)


def to_frag(lib, x, tiles, norm_w=None, eps=1e-6):
    from qdec import capi
    rows, k = x.shape
    src = x.to(DEV).contiguous()
    out = torch.full((tiles * 16 * k,), float("nan"), dtype=torch.bfloat16, device=DEV)
    a = capi.RownormArgs()
    a.x, a.out, a.eps, a.rows, a.k, a.tiles = src.data_ptr(), out.data_ptr(), eps, rows, k, tiles
    nw = norm_w.to(DEV) if norm_w is not None else None
    a.norm_w = nw.data_ptr() if nw is not None else None
    lib.rownorm(a, stream())
    torch.cuda.synchronize()
    return out


def pgemm(lib, xf, wp, rows, n, k, tiles, flags=0, res=None, out_frag=0, tile=(0, 0)):
    from qdec import capi
    n_out = n // 2 if flags == capi.GLU else n
    out = torch.full((tiles * 16 if out_frag else rows, n_out), float("nan"), dtype=torch.bfloat16, device=DEV)
    if flags == capi.RES_OUT:
        out = res.to(DEV).contiguous().clone()
    a = capi.PgemmArgs()
    a.x, a.w, a.out = xf.data_ptr(), wp.data_ptr(), out.data_ptr()
    a.res = out.data_ptr() if flags == capi.RES_OUT else None
    a.flags, a.rows, a.n, a.k, a.tiles, a.out_frag = flags, rows, n, k, tiles, out_frag
    a.tile_rows, a.tile_cols = tile
    lib.prefill_gemm(a, stream())
    torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.parametrize("rows", [37, 5000])  # per-row kernel / 16-row tile kernel
def test_rownorm_layout_and_norm(lib, rows):
    k = 2560
    x = rnd(rows, k, scale=3, seed=1)
    w = bf16(1 + 0.1 * torch.randn(k, generator=torch.Generator().manual_seed(2))).to(torch.bfloat16)
    tiles = round_up(rows, ROW_TILE) // 16
    plain = to_frag(lib, x, tiles)
    full = frag_to_rows(plain, tiles * 16, k, tiles).cpu()
    assert torch.equal(full[:rows], x)
    assert (full[rows:] == 0).all()
    normed = frag_to_rows(to_frag(lib, x, tiles, norm_w=w), rows, k, tiles).cpu().float()
    ref = rms_norm(x.float(), w.float(), 1e-6)
    exact = (normed == ref).float().mean().item()
    assert (normed - ref).abs().max().item() <= 0.01 * ref.abs().max().item()
    assert exact >= 0.99


TILES = [(256, 128), (256, 256), (64, 64)]


@pytest.mark.parametrize("tile", TILES)
@pytest.mark.parametrize("rows,n,k", [(1, 256, 64), (37, 256, 128), (256, 384, 192), (300, 512, 512),
                                      (700, 128, 256), (90, 192, 320)])
def test_prefill_gemm_exact_small_ints(lib, rows, n, k, tile):
    from qdec import capi
    if n % tile[1]:
        pytest.skip("n is not a multiple of the tile")
    x, w = small_ints(rows, k, seed=rows), small_ints(n, k, seed=n + k)
    tiles = round_up(rows, ROW_TILE) // 16
    xf, wp = to_frag(lib, x, tiles), pack(lib, w)
    ref = x.float() @ w.float().T  # exact integers
    kw = dict(tile=tile)
    assert torch.equal(pgemm(lib, xf, wp, rows, n, k, tiles, **kw).float(), ref)
    res = small_ints(rows, n, lo=-8, hi=8, seed=3)
    assert torch.equal(pgemm(lib, xf, wp, rows, n, k, tiles, capi.RES_OUT, res=res, **kw).float(), res.float() + ref)
    fr = pgemm(lib, xf, wp, rows, n, k, tiles, out_frag=1, **kw)
    assert torch.equal(frag_to_rows(fr, rows, n, tiles).float(), ref)


@pytest.mark.parametrize("tile", [(64, 64), (0, 0)])
@pytest.mark.parametrize("rows,n,k", [(1, 256, 64), (37, 384, 192), (64, 128, 256), (130, 512, 512)])
def test_prefill_gemm_64_row_padding(lib, rows, n, k, tile):
    """Buffers padded to 64 rows (a short prompt): the 64 x 64 tile, picked
    automatically, gives the exact products; 256-row tiles are refused."""
    from qdec import capi
    x, w = small_ints(rows, k, seed=rows + 7), small_ints(n, k, seed=n + k + 7)
    tiles = round_up(rows, 64) // 16
    xf, wp = to_frag(lib, x, tiles), pack(lib, w)
    ref = x.float() @ w.float().T
    assert torch.equal(pgemm(lib, xf, wp, rows, n, k, tiles, tile=tile).float(), ref)
    fr = pgemm(lib, xf, wp, rows, n, k, tiles, out_frag=1, tile=tile)
    assert torch.equal(frag_to_rows(fr, rows, n, tiles).float(), ref)
    if tiles % 16:
        with pytest.raises(capi.QdecError):
            pgemm(lib, xf, wp, rows, n, k, tiles, tile=(256, 128))


@pytest.mark.parametrize("tile", TILES)
@pytest.mark.parametrize("rows,n,k", [(5, 256, 128), (300, 512, 2560), (512, 1024, 640)])
def test_prefill_gemm_glu(lib, rows, n, k, tile):
    from qdec import capi
    x, w = rnd(rows, k, seed=4), rnd(n, k, scale=0.05, seed=5)
    tiles = round_up(rows, ROW_TILE) // 16
    xf, wp = to_frag(lib, x, tiles), pack(lib, w)
    acc = x.float() @ w.float().T
    g, u = bf16(acc[:, : n // 2]), bf16(acc[:, n // 2:])
    ref = silu_mul(g, u)
    for out_frag in (0, 1):
        out = pgemm(lib, xf, wp, rows, n, k, tiles, capi.GLU, out_frag=out_frag, tile=tile)
        got = frag_to_rows(out, rows, n // 2, tiles) if out_frag else out
        got = got.float()
        assert torch.isfinite(got).all()
        assert (got - ref).abs().max().item() <= 0.02 * ref.abs().max().item()
        assert (got == ref).float().mean().item() >= 0.97


@pytest.mark.parametrize("rows,n,k", [(64, 6144, 2560), (300, 2560, 4096), (1000, 256, 9728)])
def test_prefill_gemm_random_vs_fp32(lib, rows, n, k):
    x, w = rnd(rows, k, seed=6), rnd(n, k, scale=0.02, seed=7)
    tiles = round_up(rows, ROW_TILE) // 16
    out = pgemm(lib, to_frag(lib, x, tiles), pack(lib, w), rows, n, k, tiles).float()
    ref = bf16(x.float() @ w.float().T)
    assert (out - ref).abs().max().item() <= 0.01 * ref.abs().max().item()
    assert (out == ref).float().mean().item() >= 0.95


def v_layout(v):
    """[..., cap, D] -> the channel-major V cache layout [..., cap/8, D, 8]."""
    *lead, cap, d = v.shape
    return v.reshape(*lead, cap // 8, 8, d).transpose(-1, -2).contiguous()


def prefill_case(lib, B, T, pos0, cap, seed):
    """Random qkv rows for positions pos0 .. pos0+T-1 over a cache whose
    slots hold random values (the prefix below pos0 stays visible)."""
    from qdec import capi
    g = torch.Generator().manual_seed(seed)
    W = (NQ + 2 * NKV) * D
    qkv = (torch.randn(B * T, W, generator=g) * 2).to(torch.bfloat16)
    qn = bf16(1 + 0.2 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kn = bf16(1 + 0.2 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kc = torch.randn(B, NKV, cap, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(B, NKV, cap, D, generator=g).to(torch.bfloat16)
    cos, sin = rope_tables(cap, D, 5e6, "bf16")
    dq = qkv.to(DEV)
    dqn, dkn = qn.to(DEV), kn.to(DEV)
    dcos, dsin = cos.to(torch.bfloat16).to(DEV), sin.to(torch.bfloat16).to(DEV)
    dk, dv = kc.to(DEV).contiguous(), v_layout(vc).to(DEV)
    tiles = round_up(B * T, 16) // 16
    out = torch.full((tiles * 16 * NQ * D,), float("nan"), dtype=torch.bfloat16, device=DEV)
    q = capi.PrefillQkArgs()
    q.qkv, q.q_norm_w, q.k_norm_w, q.cos_tab, q.sin_tab = (dq.data_ptr(), dqn.data_ptr(), dkn.data_ptr(),
                                                          dcos.data_ptr(), dsin.data_ptr())
    q.k_cache, q.v_cache, q.eps = dk.data_ptr(), dv.data_ptr(), 1e-6
    q.batch, q.t_rows, q.pos0, q.nq, q.nkv, q.head_dim, q.cap = B, T, pos0, NQ, NKV, D, cap
    lib.prefill_qk(q, stream())
    a = capi.PrefillAttnArgs()
    a.qkv, a.k_cache, a.v_cache, a.out, a.sm_scale = dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), out.data_ptr(), D ** -0.5
    a.batch, a.t_rows, a.pos0, a.nq, a.nkv, a.head_dim, a.cap, a.tiles = B, T, pos0, NQ, NKV, D, cap, tiles
    lib.prefill_attn(a, stream())
    torch.cuda.synchronize()
    return dict(qkv=qkv, qn=qn, kn=kn, kc=kc, vc=vc, cos=cos, sin=sin, q_after=dq.cpu(),
                out=frag_to_rows(out, B * T, NQ * D, tiles).cpu(), k_after=dk.cpu(), v_after=dv.cpu())


def prefill_oracle(c, B, T, pos0):
    qkv = c["qkv"].float().view(B, T, NQ + 2 * NKV, D)
    kc, vc = c["kc"].float().clone(), c["vc"].float().clone()
    cap = kc.shape[2]
    pos = torch.arange(pos0, pos0 + T)
    cs, sn = c["cos"][pos][:, None, :], c["sin"][pos][:, None, :]
    outs = torch.zeros(B, T, NQ, D)
    qs = torch.zeros(B, T, NQ, D)
    vis = torch.arange(cap)[None, :] <= pos[:, None]
    for b in range(B):
        q = head_norm_rope(qkv[b, :, :NQ], c["qn"].float(), cs, sn, 1e-6)
        k = head_norm_rope(qkv[b, :, NQ:NQ + NKV], c["kn"].float(), cs, sn, 1e-6)
        kc[b, :, pos] = k.transpose(0, 1)
        vc[b, :, pos] = qkv[b, :, NQ + NKV:].transpose(0, 1)
        qs[b] = q
        for h in range(NQ):
            outs[b, :, h] = attention(q[:, h], kc[b, h // (NQ // NKV)], vc[b, h // (NQ // NKV)], vis, D ** -0.5)
    return outs.view(B * T, NQ * D), qs.view(B * T, NQ * D), kc, vc


@pytest.mark.parametrize("B,T,pos0,cap", [(1, 1, 0, 64), (1, 64, 0, 64), (2, 100, 0, 128), (2, 77, 37, 128),
                                          (1, 300, 200, 512), (3, 129, 64, 224), (1, 33, 991, 1024),
                                          (33, 131, 21, 160), (32, 130, 0, 160)])
# the last two take the grouped QK kernel (>= 4096 rows): unaligned groups, then
# aligned ones with a ragged last group
def test_prefill_qk_and_attention_vs_oracle(lib, B, T, pos0, cap):
    c = prefill_case(lib, B, T, pos0, cap, seed=B * 1000 + T + pos0)
    ref, q_ref, kc, vc = prefill_oracle(c, B, T, pos0)
    # head norm / RoPE / cache fill; the key / value columns of qkv untouched
    q_got = c["q_after"].float().view(B * T, NQ + 2 * NKV, D)[:, :NQ].reshape(B * T, NQ * D)
    near_exact(q_got, q_ref)
    assert torch.equal(c["q_after"][:, NQ * D:], c["qkv"][:, NQ * D:])
    near_exact(c["k_after"], kc)
    assert torch.equal(c["v_after"].float(), v_layout(vc.to(torch.bfloat16)).float())
    out = c["out"].float()
    assert torch.isfinite(out).all()
    err = (out - ref).abs().max().item()
    assert err <= 0.02 * ref.abs().max().item(), err
