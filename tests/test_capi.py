"""The C ABI without a GPU: the library loads, exports every symbol that
include/qdec.h declares, validates arguments before touching HIP, and its
layout helper agrees with the tiled layout the kernels assume."""

import ctypes

import pytest

from qdec import capi


def test_exports_every_declared_symbol(qlib):
    names = capi.declared_functions()
    assert len(names) >= 12
    missing = [n for n in names if not hasattr(qlib.so, n)]
    assert not missing, missing
    assert qlib.version() == 1


def test_structs_match_header_fields():
    """Every field of every args struct in the header exists in the ctypes
    mirror, in the same order."""
    import re
    text = open(capi.HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    for cname, st in (("qdec_embed_args", capi.EmbedArgs), ("qdec_gemm_args", capi.GemmArgs),
                      ("qdec_attn_args", capi.AttnArgs), ("qdec_draft_args", capi.DraftArgs),
                      ("qdec_accept_args", capi.AcceptArgs), ("qdec_rownorm_args", capi.RownormArgs),
                      ("qdec_pgemm_args", capi.PgemmArgs), ("qdec_prefill_qk_args", capi.PrefillQkArgs),
                      ("qdec_prefill_attn_args", capi.PrefillAttnArgs), ("qdec_layer_args", capi.LayerArgs)):
        body = re.search(r"typedef struct (?:\w+ )?\{([^{}]*)\}\s*" + cname + ";", text).group(1)
        fields = re.findall(r"\*?\s*(\w+)\s*;", body)
        assert fields == [f[0] for f in st._fields_], cname


def test_device_count_without_gpu_is_safe(qlib):
    assert qlib.device_count() >= 0


def test_tiled_offset_layout(qlib):
    K = 96
    seen = set()
    for n in range(32):
        for k in range(K):
            off = qlib.tiled_offset(n, k, K)
            nt, ks = n // 16, k // 32
            lane = (n % 16) + 16 * ((k % 32) // 8)
            assert off == ((nt * (K // 32) + ks) * 64 + lane) * 8 + k % 8
            seen.add(off)
    assert seen == set(range(32 * K))  # a permutation of the matrix
    assert qlib.tiled_offset(0, 0, 100) == -1
    assert qlib.tiled_offset(0, 96, 96) == -1


def _gemm(**kw):
    a = capi.GemmArgs()
    a.x = a.w = a.out = a.res = a.norm_w = a.partial = a.counters = a.ids_out = 16
    a.eps, a.rows, a.n, a.k, a.flags, a.ksplit, a.waves, a.tiles_per_wg = 1e-6, 1, 256, 256, 0, 1, 4, 1
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,code,needle", [
    (dict(rows=0), -1, "rows"),
    (dict(rows=65), -1, "rows"),
    (dict(n=250), -1, "multiple of 16"),
    (dict(k=100), -1, "multiple of 32"),
    (dict(waves=9), -1, "waves"),
    (dict(ksplit=3), -1, "ksplit"),
    (dict(flags=capi.GLU | capi.RES_OUT), -3, "not supported"),
    (dict(flags=capi.GLU), -3, "x_frag = 1"),
    (dict(flags=capi.ARGMAX | capi.NORM_IN, ksplit=2), -3, "ksplit 1"),
    (dict(tiles_per_wg=3), -1, "tiles_per_wg"),
    (dict(x_frag=2), -1, "x_frag"),
    (dict(flags=capi.RES_OUT, res=16, out_frag=1), -3, "out_frag"),
    (dict(flags=capi.NORM_IN, norm_w=16, x_frag=1), -3, "x_frag"),
    (dict(x=8), -2, "aligned"),
    (dict(out=None), -1, "null out"),
])
def test_gemm_validation(qlib, kw, code, needle):
    rc = qlib.so.qdec_gemm(ctypes.byref(_gemm(**kw)), None)
    assert rc == code
    assert needle in qlib.last_error()
    with pytest.raises(capi.QdecError):
        qlib.gemm(_gemm(**kw), None)


def test_gemm_workspace_sizes(qlib):
    pb, cb = qlib.gemm_workspace(_gemm(flags=capi.RES_OUT, ksplit=2, n=2560, k=4096, rows=3))
    assert pb == 2 * 3 * 2560 * 4 and cb == 160 * 4
    pb, cb = qlib.gemm_workspace(_gemm(flags=capi.NORM_IN | capi.ARGMAX, n=151936, k=2560, rows=2,
                                       tiles_per_wg=4))
    assert pb == 0 and cb == 8 + 8 * 16 * 2  # arrival counter, 16 64-bit argmax keys per row
    pb, cb = qlib.gemm_workspace(_gemm(flags=capi.NORM_IN | capi.ARGMAX, n=151936, k=2560, rows=1,
                                       tiles_per_wg=4))
    assert pb == 8 * (9496 // 4) and cb == 8 + 8 * 16  # one row: a 64-bit key per workgroup
    pb, cb = qlib.gemm_workspace(_gemm(flags=capi.NORM_IN, n=6144, k=2560))
    assert pb == 0 and cb == 0


def test_gemm_prepass_query(qlib):
    """Which NORM_IN calls normalise in a pre-pass launch of their own (the
    consumers a norm hand-over serves), and with how many threads."""
    gu = dict(flags=capi.NORM_IN | capi.GLU, n=9728, k=2560, waves=4)
    assert qlib.gemm_prepass(_gemm(rows=4, **gu)) == (False, 256)  # rows staged from registers
    assert qlib.gemm_prepass(_gemm(rows=5, **gu)) == (False, 256)  # staged through LDS
    assert qlib.gemm_prepass(_gemm(rows=6, **gu)) == (True, 256)  # GLU: direct path from 6 rows
    assert qlib.gemm_prepass(_gemm(rows=8, **gu)) == (True, 256)
    assert qlib.gemm_prepass(_gemm(rows=8, flags=capi.NORM_IN, n=6144, k=2560)) == (False, 256)
    assert qlib.gemm_prepass(_gemm(rows=20, flags=capi.NORM_IN, n=6144, k=2560, waves=8, tiles_per_wg=2)) == (True, 512)
    assert qlib.gemm_prepass(_gemm(rows=20, flags=capi.RES_OUT, n=2560, k=4096, x_frag=1)) == (False, 256)
    assert qlib.so.qdec_gemm_prepass(ctypes.byref(_gemm(rows=0)), None) == -1


GU_RES = dict(flags=capi.NORM_IN | capi.GLU, n=9728, k=2560, waves=4, rows=8, resident=1)


@pytest.mark.parametrize("kw,code,needle", [
    (dict(resident=2), -1, "resident 2"),
    (dict(flags=capi.GLU, x_frag=1, out_frag=1), -3, "NORM_IN (with or without GLU)"),
    (dict(ksplit=2), -3, "ksplit 1"),
    (dict(waves=8), -3, "4 waves"),
    (dict(tiles_per_wg=2), -3, "one tile"),
    (dict(x_frag=1, flags=capi.GLU), -3, "row-major x"),
    (dict(rows=9), -3, "1..8 or 17..32 rows"),
    (dict(rows=16), -3, "1..8 or 17..32 rows"),
    (dict(rows=33), -3, "1..8 or 17..32 rows"),
    (dict(n=16), -3, "two output tiles"),
    (dict(k=4096), -3, "k <= 2560"),
    (dict(k=1024), -3, "multiple of 10"),
    (dict(flags=capi.NORM_IN, n=6144, rows=9), -3, "1..8 or 17..32 rows"),
    (dict(flags=capi.NORM_IN, n=6144, rows=33), -3, "1..8 or 17..32 rows"),
    (dict(flags=capi.NORM_IN, n=6144, k=1280), -3, "multiple of 20"),
    (dict(flags=capi.NORM_IN, n=16), -3, "two output tiles"),
])
def test_gemm_resident_validation(qlib, kw, code, needle):
    """The resident gate/up plan takes exactly the shapes its kernel was
    built for and refuses the rest before any launch."""
    args = dict(GU_RES, **kw)
    rc = qlib.so.qdec_gemm(ctypes.byref(_gemm(**args)), None)
    assert rc == code
    assert needle in qlib.last_error()


DN_RES = dict(flags=capi.RES_OUT, res=16, n=2560, k=9728, waves=8, rows=8, resident=1)


@pytest.mark.parametrize("kw,code,needle", [
    (dict(ksplit=2), -3, "ksplit 1"),
    (dict(tiles_per_wg=2), -3, "one tile"),
    (dict(x_frag=1), -3, "row-major x"),
    (dict(rows=9), -3, "1..8 rows"),
    (dict(k=9696, waves=1), -3, "a multiple of 16"),
    (dict(k=10240), -3, "at most 304"),
    (dict(resident=3), -1, "resident 3"),
])
def test_gemm_resident_res_out_validation(qlib, kw, code, needle):
    rc = qlib.so.qdec_gemm(ctypes.byref(_gemm(**dict(DN_RES, **kw))), None)
    assert rc == code
    assert needle in qlib.last_error()


DS_RES = dict(DN_RES, rows=32, waves=4, ksplit=4, tiles_per_wg=2, x_frag=1, parts_out=16)


@pytest.mark.parametrize("kw,needle", [
    (dict(rows=16), "17..32 rows"),
    (dict(rows=33), "rows"),
    (dict(waves=2), "4 waves"),
    (dict(x_frag=0), "x_frag = 1"),
    (dict(ksplit=2), "76 k steps per split"),
])
def test_gemm_resident_split_validation(qlib, kw, needle):
    """The split RES_OUT resident plan (k parts left in parts_out) takes
    only the shapes its kernel was built for."""
    rc = qlib.so.qdec_gemm(ctypes.byref(_gemm(**dict(DS_RES, **kw))), None)
    assert rc < 0
    assert needle in qlib.last_error()
    assert qlib.gemm_workspace(_gemm(**DS_RES)) == (0, 0)


def test_gemm_glu_takes_pending_split_update():
    """gate/up merges a split O projection's partials (x_parts) in its
    normalisation pre-pass: accepted wherever its plan has one, resident or
    not; the resident 6..8-row plan (no pre-pass) refuses them."""
    from qdec import capi as c
    lib = c.lib()
    gu = dict(flags=capi.NORM_IN | capi.GLU, n=9728, k=2560, waves=4, x_parts=16, x_nparts=2, x_merged=32)
    for rows in (1, 4, 8, 17, 32):
        lib.gemm_workspace(_gemm(rows=rows, **gu))
    for rows in (17, 24, 32):
        lib.gemm_workspace(_gemm(rows=rows, resident=1, **gu))
        assert lib.gemm_prepass(_gemm(rows=rows, resident=1, **gu))[0]
    with pytest.raises(capi.QdecError, match="resident with x_parts"):
        lib.gemm_workspace(_gemm(rows=8, resident=1, **gu))


def test_gemm_resident_res_out_needs_no_workspace(qlib):
    for rows in (1, 2, 5, 8):
        assert qlib.gemm_workspace(_gemm(**dict(DN_RES, rows=rows))) == (0, 0)


def test_gemm_resident_workspace_and_prepass(qlib):
    """At 6..8 rows the resident call normalises its rows itself (no
    workspace, no pre-pass); at 17..32 the pre-pass still writes the two M
    tiles of normalised rows into the workspace, as without resident."""
    for rows in (1, 3, 6, 7, 8):
        assert qlib.gemm_workspace(_gemm(**dict(GU_RES, rows=rows))) == (0, 0)
        assert qlib.gemm_prepass(_gemm(**dict(GU_RES, rows=rows))) == (False, 256)
        assert qlib.gemm_prepass(_gemm(**dict(GU_RES, rows=rows, resident=0))) == (rows >= 6, 256)
        # QKV (NORM_IN alone) likewise
        qkv = dict(GU_RES, flags=capi.NORM_IN, n=6144, rows=rows)
        assert qlib.gemm_workspace(_gemm(**qkv)) == (0, 0)
        assert qlib.gemm_prepass(_gemm(**qkv)) == (False, 256)
    for rows in (17, 32):
        ws = qlib.gemm_workspace(_gemm(**dict(GU_RES, rows=rows)))
        assert ws == qlib.gemm_workspace(_gemm(**dict(GU_RES, rows=rows, resident=0)))
        assert ws[0] >= 32 * 2560 * 2
        assert qlib.gemm_prepass(_gemm(**dict(GU_RES, rows=rows))) == (True, 256)


def test_gemm_glu_argmax_alone_need_fragment_order(qlib):
    for f in (capi.GLU, capi.ARGMAX):
        assert qlib.so.qdec_gemm(ctypes.byref(_gemm(flags=f, rows=20, n=9728 if f == capi.GLU else 151936,
                                                    k=2560)), None) == -3
        assert "x_frag" in qlib.last_error()
    qlib.gemm_workspace(_gemm(flags=capi.GLU, rows=20, n=9728, k=2560, x_frag=1, out_frag=1))
    qlib.gemm_workspace(_gemm(flags=capi.ARGMAX, rows=20, n=151936, k=2560, x_frag=1, tiles_per_wg=8))


def _hand(**kw):
    """An O-shaped RES_OUT call on the direct path handing over to gate/up."""
    base = dict(flags=capi.RES_OUT, n=2560, k=4096, rows=20, waves=8, x_frag=1, next_norm_w=16, next_xn=16,
                next_threads=256)
    return _gemm(**{**base, **kw})


@pytest.mark.parametrize("kw,code,needle", [
    (dict(flags=0), -3, "RES_OUT alone"),
    (dict(rows=4, x_frag=0, waves=8), -3, "direct path"),
    (dict(ksplit=2), -3, "parts_out"),
    (dict(ksplit=8, waves=4, parts_out=16), -3, "at most 4 splits"),
    (dict(next_threads=96), -3, "next_threads"),
    (dict(next_threads=1536), -3, "next_threads"),
    (dict(next_threads=128), -3, "next_threads"),       # a 2560-wide row is 320 vectors: 2 per thread at most
    (dict(waves=1, next_threads=128, k=256), -3, "next_threads"),  # 128 threads from 64: one vector each
    (dict(n=256, k=4096, next_threads=64), -3, "workgroups"),  # 16 workgroups for 32 hand-over rows
    (dict(next_xn=None), -1, "next_xn"),
    (dict(counters=None), -1, "counters"),
    (dict(ksplit=4, waves=4, parts_out=16, next_merged=None), -1, "next_merged"),
    (dict(next_xn=24), -2, "16-byte"),
])
def test_gemm_hand_over_validation(qlib, kw, code, needle):
    rc = qlib.so.qdec_gemm(ctypes.byref(_hand(**kw)), None)
    assert rc == code, qlib.last_error()
    assert needle in qlib.last_error()


def test_gemm_hand_over_workspace(qlib):
    # three counter words (arrival, departure, give-up) beyond what the call needs otherwise
    assert qlib.gemm_workspace(_hand()) == (0, 12)
    assert qlib.gemm_workspace(_hand(ksplit=4, waves=4, parts_out=16, next_merged=16, next_threads=512)) == (0, 12)


def _attn(**kw):
    a = capi.AttnArgs()
    for f in ("qkv", "q_norm_w", "k_norm_w", "cos_tab", "sin_tab", "lens", "k_cache", "v_cache", "out",
              "partial", "counters"):
        setattr(a, f, 16)
    a.eps, a.sm_scale = 1e-6, 128 ** -0.5
    a.batch, a.t_rows, a.nq, a.nkv, a.head_dim, a.cap, a.chunk, a.waves = 2, 1, 32, 8, 128, 256, 64, 4
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,code", [
    (dict(head_dim=96), -3), (dict(head_dim=64, waves=8), -3), (dict(nq=20), -3), (dict(nq=4), -3), (dict(t_rows=17), -1), (dict(cap=100), -1),
    (dict(nq=64, t_rows=9), -3),  # 8 query heads per kv head: 72 query rows > 64
    (dict(nq=64, t_rows=5, waves=8), -3),  # 40 > 32 with 8 waves
    (dict(nq=40, t_rows=13), -3),  # 5 per kv head: 65 > 64
    (dict(chunk=48), -1), (dict(waves=5), -1), (dict(waves=2), -1), (dict(out=None), -1), (dict(partial=None), -1), (dict(qkv=8), -2),
    (dict(waves=8, t_rows=9), -3),
    (dict(strided=1), -3), (dict(strided=2, waves=8), -1),  # strided chunks run 8 waves; the flag is 0 or 1
])
def test_attn_validation(qlib, kw, code):
    assert qlib.so.qdec_attn(ctypes.byref(_attn(**kw)), None) == code


def test_attn_workspace(qlib):
    pb, cb = qlib.attn_workspace(_attn(t_rows=3, batch=2, cap=256, chunk=64))
    assert pb == 4 * 2 * 8 * 4 * 12 * 130 and cb == 2 * 8 * 4
    pb, cb = qlib.attn_workspace(_attn(cap=64, chunk=64))
    assert pb == 0 and cb == 0


def _layer(**kw):
    """qdec_layer arguments of a batch-1 Qwen3-4B layer under the layer
    kernel's plans (pointer values are placeholders: these calls are
    refused before anything touches a GPU)."""
    at = _attn(batch=1, out_partials=1, cap=800, chunk=96)
    g = dict(qkv=_gemm(flags=capi.NORM_IN, n=6144, k=2560),
             o=_gemm(flags=capi.RES_OUT, n=2560, k=4096),
             gate_up=_gemm(flags=capi.NORM_IN | capi.GLU, n=19456, k=2560, tiles_per_wg=2),
             down=_gemm(flags=capi.RES_OUT, n=2560, k=9728))
    g["o"].x_attn = ctypes.addressof(at)
    la = capi.LayerArgs(plan=4096, ctl=64)
    la.attn = ctypes.pointer(at)
    for name, a in g.items():
        setattr(la, name, ctypes.pointer(a))
    la._keep = (at, g)
    for k, v in kw.items():
        if callable(v):
            v(la, at, g)
        else:
            setattr(la, k, v)
    return la


def _set(obj, **kw):
    def f(la, at, g):
        target = at if obj == "attn" else g[obj]
        for k, v in kw.items():
            setattr(target, k, v)
    return f


@pytest.mark.parametrize("kw,code,needle", [
    (dict(plan=8), -2, "plan"),
    (dict(ctl=12), -2, "ctl"),
    (dict(fix=_set("attn", t_rows=2)), -3, "t_rows"),
    (dict(fix=_set("attn", batch=5)), -3, "batch"),
    (dict(fix=_set("attn", out_partials=0)), -3, "out_partials"),
    (dict(fix=_set("o", x_attn=None)), -3, "x_attn"),
    (dict(fix=_set("qkv", waves=8)), -3, "qkv plan"),
    (dict(fix=_set("down", ksplit=4)), -3, "down plan"),
    (dict(fix=_set("gate_up", flags=capi.NORM_IN)), -3, "gate_up plan"),
    (dict(fix=_set("qkv", rows=2)), -3, "qkv plan"),
])
def test_layer_validation(qlib, kw, code, needle):
    fix = kw.pop("fix", None)
    la = _layer(**kw) if fix is None else _layer(fix=fix)
    assert qlib.so.qdec_layer(ctypes.byref(la), None) == code
    assert needle in qlib.last_error()
    assert qlib.so.qdec_layer_prepare(ctypes.byref(la)) == code
    assert qlib.so.qdec_layer(None, None) == -1


def test_other_validation(qlib):
    assert qlib.so.qdec_pack_tiles(None, None, 16, 32, None) == -1
    assert qlib.so.qdec_pack_tiles(16, 16, 17, 32, None) == -1
    e = capi.EmbedArgs(ids=16, emb=16, h=16, rows=1, hidden=100, vocab=16)
    assert qlib.so.qdec_embed(ctypes.byref(e), None) == -1
    d = capi.DraftArgs(hist=16, lens=16, ids=16, draft=16, batch=1, cap=8, primary=3, backoff=2, k=-1)
    assert qlib.so.qdec_ngram_draft(ctypes.byref(d), None) == -1
    a = capi.AcceptArgs(out_tok=16, draft=16, hist=16, lens=16, naccept=None, batch=1, cap=8, k=1, stop_len=1)
    assert qlib.so.qdec_spec_accept(ctypes.byref(a), None) == -1


def test_role_plans_do_not_depend_on_rows():
    from qdec.runtime import attn_chunk, role_plan, round_up
    for role, n, k in (("qkv", 6144, 2560), ("o", 2560, 4096), ("gate_up", 9728, 2560),
                       ("down", 2560, 9728), ("lm", 151936, 2560)):
        ks, w, t = role_plan(n, k, role)
        assert (k // 32) % (ks * w) == 0
        assert (n // 16) % t == 0
    # from batch 16 down splits k four ways (partials merged by the next
    # NORM_IN call's pre-pass); O always runs whole tiles
    assert role_plan(2560, 9728, "down") == (1, 8, 1) and role_plan(2560, 4096, "o")[0] == 1
    assert role_plan(2560, 9728, "down", batch=16)[:2] == (4, 4)
    assert role_plan(2560, 9728, "down", batch=8) == (1, 8, 1)
    assert role_plan(2560, 4096, "o", batch=8) == (1, 8, 1) and role_plan(2560, 4096, "o", batch=9) == (1, 4, 1)
    # QKV from 17 rows: k over 4 waves on the resident plan, else 8 waves of two tiles
    assert role_plan(6144, 2560, "qkv", batch=17)[:2] == (1, 4) and role_plan(6144, 2560, "qkv", batch=16)[:2] == (1, 4)
    assert role_plan(6144, 2560, "qkv", batch=33)[:2] == (1, 8)
    # the 160-tile roles run 8 waves, the others 4; the lm_head 4 tiles per workgroup
    assert [role_plan(n, k, r)[1] for r, n, k in (("qkv", 6144, 2560), ("o", 2560, 4096),
                                                  ("gate_up", 9728, 2560), ("down", 2560, 9728),
                                                  ("lm", 151936, 2560))] == [4, 8, 4, 8, 4]
    assert role_plan(151936, 2560, "lm")[2] == 4
    for b, cap in ((1, 800), (4, 1568), (32, 4384)):
        c = attn_chunk(b, 8, cap)
        assert c % 32 == 0 and 64 <= c <= cap
    # from batch 6 every workgroup resident at once (8 kv heads, 256 CUs), in
    # equal chunks, at most one per 256 slots of the cache
    assert attn_chunk(8, 8, 1568) == 416 and attn_chunk(32, 8, 4384) == 4384
    assert attn_chunk(6, 8, 1568) == 320 and attn_chunk(8, 8, 800) == 224 and attn_chunk(8, 8, 256) == 256
    assert attn_chunk(16, 8, 4384) == 2208 and attn_chunk(16, 8, 1568) == 800
    assert attn_chunk(12, 8, 1568) == 800 and attn_chunk(20, 8, 4384) == 4384
    for b in range(6, 65):
        for cap in (64, 544, 1568, 4384, 8192):
            c = attn_chunk(b, 8, cap)
            assert c % 32 == 0 and c <= round_up(cap, 32)
            assert b * 8 * -(-round_up(cap, 32) // c) <= max(256, b * 8)
            assert -(-round_up(cap, 32) // c) <= -(-round_up(cap, 32) // 256)  # chunks: at most one per 256 slots


def _pgemm(**kw):
    a = capi.PgemmArgs(x=16, w=16, out=16, res=None, flags=0, rows=300, n=256, k=128, tiles=32, out_frag=0)
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,code,needle", [
    (dict(flags=capi.NORM_IN), -3, "flags"),
    (dict(n=200), -1, "multiple of 64"),
    (dict(n=384, tile_rows=256, tile_cols=256), -1, "multiple of 256"),
    (dict(n=320, tile_rows=256, tile_cols=128), -1, "multiple of 128"),
    (dict(tile_rows=256, tile_cols=64), -1, "tile 256 x 64"),
    (dict(tile_cols=128), -1, "tile 0 x 128"),
    (dict(k=96), -1, "k of 64"),
    (dict(tiles=24, tile_rows=256, tile_cols=128), -1, "multiple of 16"),  # 256-row tiles: whole ones
    (dict(tiles=22), -1, "multiple of 4"),  # 64-row granularity otherwise
    (dict(rows=513), -1, "tiles"),
    (dict(flags=capi.RES_OUT), -3, "RES_OUT"),
    (dict(flags=capi.RES_OUT, res=16, out_frag=1), -3, "RES_OUT"),
    (dict(out_frag=2), -1, "out_frag"),
    (dict(x=8), -2, "aligned"),
    (dict(w=None), -1, "null"),
])
def test_prefill_gemm_validation(qlib, kw, code, needle):
    rc = qlib.so.qdec_prefill_gemm(ctypes.byref(_pgemm(**kw)), None)
    assert rc == code
    assert needle in qlib.last_error()


def test_prefill_validation(qlib):
    r = capi.RownormArgs(x=16, norm_w=None, out=16, eps=1e-6, rows=20, k=2560, tiles=1)
    assert qlib.so.qdec_rownorm(ctypes.byref(r), None) == -1  # 20 rows need 2 tiles
    r.tiles, r.k = 2, 100
    assert qlib.so.qdec_rownorm(ctypes.byref(r), None) == -1
    q = dict(qkv=16, q_norm_w=16, k_norm_w=16, cos_tab=16, sin_tab=16, k_cache=16, v_cache=16, eps=1e-6,
             batch=2, t_rows=100, pos0=0, nq=32, nkv=8, head_dim=128, cap=128)
    assert qlib.so.qdec_prefill_qk(ctypes.byref(capi.PrefillQkArgs(**{**q, "head_dim": 64})), None) == -3
    assert qlib.so.qdec_prefill_qk(ctypes.byref(capi.PrefillQkArgs(**{**q, "pos0": 40})), None) == -1
    assert qlib.so.qdec_prefill_qk(ctypes.byref(capi.PrefillQkArgs(**{**q, "cap": 120})), None) == -1
    at = dict(qkv=16, k_cache=16, v_cache=16, out=16, sm_scale=0.088, batch=2, t_rows=100, pos0=0, nq=32,
              nkv=8, head_dim=128, cap=128, tiles=13)
    assert qlib.so.qdec_prefill_attn(ctypes.byref(capi.PrefillAttnArgs(**{**at, "nq": 40})), None) == -3  # 5 per kv head
    assert qlib.so.qdec_prefill_attn(ctypes.byref(capi.PrefillAttnArgs(**{**at, "nq": 20})), None) == -3
    assert qlib.so.qdec_prefill_attn(ctypes.byref(capi.PrefillAttnArgs(**{**at, "tiles": 12})), None) == -1
    assert qlib.so.qdec_prefill_attn(ctypes.byref(capi.PrefillAttnArgs(**{**at, "t_rows": 129})), None) == -1
    assert qlib.so.qdec_prefill_attn(ctypes.byref(capi.PrefillAttnArgs(**{**at, "out": 8})), None) == -2

