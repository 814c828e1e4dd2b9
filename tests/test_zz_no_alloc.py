"""qdec_attn_noalloc (library-owned scratch) against qdec_attn (caller
workspace), through the C ABI: the same output and cache bits on two calls
in a row, the second smaller; a first call made under hipGraph capture (in a
fresh process, so the library sets its scratch up inside the capture),
replayed; and a clear error for calls the scratch cannot hold."""

import os
import subprocess
import sys

import pytest
import torch

from qdec import capi

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
NQ, NKV, D = 32, 8, 128


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _case(B, T, lens, cap, chunk, waves, seed):
    """Inputs of one attention call (device tensors) and its argument block."""
    g = torch.Generator().manual_seed(seed)
    W = (NQ + 2 * NKV) * D
    t = dict(
        qkv=(torch.randn(B * T, W, generator=g) * 2).to(torch.bfloat16),
        qn=(1 + 0.2 * torch.randn(D, generator=g)).to(torch.bfloat16),
        kn=(1 + 0.2 * torch.randn(D, generator=g)).to(torch.bfloat16),
        kc=torch.randn(B, NKV, cap, D, generator=g).to(torch.bfloat16),
        vc=torch.randn(B, NKV, cap, D, generator=g).to(torch.bfloat16),
    )
    pos = torch.arange(cap, dtype=torch.float32)[:, None]
    inv = 1.0 / (5e6 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    emb = torch.cat([pos * inv, pos * inv], 1)
    t["cos"], t["sin"] = emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)
    t["lens"] = torch.tensor(lens, dtype=torch.int32)
    t = {k: v.to(DEV) for k, v in t.items()}
    a = capi.AttnArgs(eps=1e-6, sm_scale=D ** -0.5, batch=B, t_rows=T, nq=NQ, nkv=NKV, head_dim=D, cap=cap,
                      chunk=chunk, waves=waves, out_partials=0, out_frag=0)
    return t, a


def _run(lib, t, a, noalloc):
    """One call on fresh copies of the caches; returns (out, k cache, v cache)."""
    kc, vc = t["kc"].clone(), t["vc"].clone()
    out = torch.full((a.batch * a.t_rows, NQ * D), 3.0, dtype=torch.bfloat16, device=DEV)
    a.qkv, a.q_norm_w, a.k_norm_w = t["qkv"].data_ptr(), t["qn"].data_ptr(), t["kn"].data_ptr()
    a.cos_tab, a.sin_tab, a.lens = t["cos"].data_ptr(), t["sin"].data_ptr(), t["lens"].data_ptr()
    a.k_cache, a.v_cache, a.out = kc.data_ptr(), vc.data_ptr(), out.data_ptr()
    if noalloc:
        a.partial, a.counters = None, None
        lib.attn_noalloc(a, _stream())
        torch.cuda.synchronize()
        return out.cpu(), kc.cpu(), vc.cpu(), None
    pb, cb = lib.attn_workspace(a)
    part = torch.zeros(max(pb, 16) // 4, dtype=torch.float32, device=DEV)
    cnt = torch.zeros(max(cb, 4) // 4, dtype=torch.int32, device=DEV)
    a.partial, a.counters = part.data_ptr(), cnt.data_ptr()
    lib.attn(a, _stream())
    torch.cuda.synchronize()
    return out.cpu(), kc.cpu(), vc.cpu(), cnt.cpu()


def test_noalloc_attention_matches_workspace_attention():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")
    lib = capi.lib()
    # first call: batch 4 at config 5's scale, 11 chunks, merged across
    # workgroups through the arrival counters; second call smaller (fewer
    # sequences, shorter cache, 2 rows per sequence, 8 waves).
    for B, T, lens, cap, chunk, waves in ((4, 1, [1000, 1017, 31, 64], 1056, 96, 4),
                                          (2, 2, [100, 7], 256, 64, 8)):
        t, a = _case(B, T, lens, cap, chunk, waves, seed=B * 10 + T)
        pb, cb = lib.attn_workspace(a)
        assert 0 < pb <= capi.NOALLOC_PARTIAL_BYTES and 0 < cb <= capi.NOALLOC_COUNTER_BYTES
        ref_out, ref_k, ref_v, cnt = _run(lib, t, a, noalloc=False)
        assert int(cnt.abs().sum()) == 0
        out, k, v, _ = _run(lib, t, a, noalloc=True)
        print(f"B={B} T={T} cap={cap} chunk={chunk}: partials {pb} B, counters {cb} B", flush=True)
        assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16))
        assert torch.equal(k.view(torch.int16), ref_k.view(torch.int16))
        assert torch.equal(v.view(torch.int16), ref_v.view(torch.int16))
        assert not bool((out == 3.0).all(dim=1).any()), "a row was left unwritten"


def test_noalloc_attention_rejects_what_it_cannot_hold():
    lib = capi.lib()
    # 64 sequences x 4096 chunks of 32 slots: far more partials than the scratch
    a = capi.AttnArgs(eps=1e-6, sm_scale=D ** -0.5, batch=64, t_rows=1, nq=NQ, nkv=NKV, head_dim=D, cap=131072,
                      chunk=32, waves=4)
    with pytest.raises(capi.QdecError, match="library scratch"):
        lib.attn_noalloc(a, None)
    a = capi.AttnArgs(eps=1e-6, sm_scale=D ** -0.5, batch=1, t_rows=1, nq=NQ, nkv=NKV, head_dim=D, cap=256,
                      chunk=64, waves=4, out_partials=1)
    with pytest.raises(capi.QdecError, match="out_partials"):
        lib.attn_noalloc(a, None)


_CAPTURE_SCRIPT = r"""
import sys
import torch
sys.path[:0] = [{pkg!r}, {repo!r}, {tests!r}]
from qdec import capi
import test_zz_no_alloc as T

lib = capi.lib()
s = torch.cuda.current_stream()
# 11 chunks merged across workgroups through the scratch's arrival counters
t, a = T._case(4, 1, [1000, 1017, 31, 64], 1056, 96, 4, seed=77)
ref_out, ref_k, ref_v, cnt = T._run(lib, t, a, noalloc=False)
assert int(cnt.abs().sum()) == 0
kc, vc = t["kc"].clone(), t["vc"].clone()
out = torch.full((4, T.NQ * T.D), 3.0, dtype=torch.bfloat16, device=T.DEV)
a.qkv, a.q_norm_w, a.k_norm_w = t["qkv"].data_ptr(), t["qn"].data_ptr(), t["kn"].data_ptr()
a.cos_tab, a.sin_tab, a.lens = t["cos"].data_ptr(), t["sin"].data_ptr(), t["lens"].data_ptr()
a.k_cache, a.v_cache, a.out = kc.data_ptr(), vc.data_ptr(), out.data_ptr()
a.partial, a.counters = None, None
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):
    # the process's first noalloc call: the scratch address is taken and the
    # counter-clearing kernel recorded into the graph
    lib.attn_noalloc(a, torch.cuda.current_stream().cuda_stream)
torch.cuda.synchronize()
for rep in range(3):
    out.fill_(3.0)
    kc.copy_(t["kc"])
    vc.copy_(t["vc"])
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    for name, got, want in (("out", out, ref_out), ("k", kc, ref_k), ("v", vc, ref_v)):
        assert torch.equal(got.cpu().view(torch.int16), want.view(torch.int16)), (rep, name)
    print(f"replay {{rep}}: bits equal to qdec_attn", flush=True)
# eager calls after the replays, several chunks: the counters were left at zero
for B, T_, lens, cap, chunk, waves in ((3, 1, [700, 31, 257], 800, 128, 4), (2, 2, [300, 77], 512, 64, 8)):
    t2, a2 = T._case(B, T_, lens, cap, chunk, waves, seed=B + 5)
    r_out, r_k, r_v, _ = T._run(lib, t2, a2, noalloc=False)
    o2, k2, v2, _ = T._run(lib, t2, a2, noalloc=True)
    assert torch.equal(o2.view(torch.int16), r_out.view(torch.int16)) and torch.equal(k2.view(torch.int16), r_k.view(torch.int16))
    assert torch.equal(v2.view(torch.int16), r_v.view(torch.int16))
    print(f"eager B={{B}} T={{T_}} after the replays: bits equal", flush=True)
print("CAPTURE_OK", flush=True)
"""


def test_noalloc_first_call_under_graph_capture():
    """The header's use case: a caller under hipGraph capture.  In a fresh
    process the first qdec_attn_noalloc call is made inside a
    torch.cuda.graph capture (the library takes the scratch address and
    records its counter-clearing kernel there); the graph is replayed three
    times with eager work between the replays, each replay bit-equal to
    qdec_attn with a caller workspace; eager noalloc calls with several
    chunks afterwards still match, so the counters were left at zero."""
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")
    here = os.path.dirname(os.path.abspath(__file__))
    repo = os.path.dirname(here)
    script = _CAPTURE_SCRIPT.format(pkg=os.path.join(repo, "dryft-challenge_amd"), repo=repo, tests=here)
    print("[no-alloc] capture case in a fresh process", flush=True)
    res = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True, timeout=240)
    print(res.stdout[-2000:], res.stderr[-2000:], flush=True)
    assert res.returncode == 0 and "CAPTURE_OK" in res.stdout
