"""ctypes binding of libqdec.so (the C ABI declared in include/qdec.h).

Argument blocks mirror the C structs field for field.  Every call raises
``QdecError`` with ``qdec_last_error()`` when the library returns an error.
There is no fallback: if the library is missing the import of the engine
fails loudly.
"""

import ctypes
import os
import re

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libqdec.so")
HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))),
                      "include", "qdec.h")

NORM_IN, GLU, RES_OUT, ARGMAX = 1, 2, 4, 8
# Greedy pick of a row whose logits are all NaN (QDEC_NAN_ID): the kernels turn
# an out-of-range token id or cache length into NaN rows instead of guessing.
NAN_ID = 2147483647
# Library-owned scratch of qdec_attn_noalloc (QDEC_NOALLOC_*_BYTES).
NOALLOC_PARTIAL_BYTES = 8 << 20
NOALLOC_COUNTER_BYTES = 64 << 10
# Device memory of a qdec_layer call (QDEC_LAYER_PLAN_BYTES, QDEC_LAYER_CTL_BYTES).
LAYER_PLAN_BYTES = 4096
LAYER_CTL_BYTES = 1152

P = ctypes.c_void_p
I32 = ctypes.c_int32
F32 = ctypes.c_float


class QdecError(RuntimeError):
    """A libqdec entry point returned a negative status."""

    def __init__(self, fn, code, msg):
        super().__init__(f"{fn} failed ({code}): {msg}")
        self.code = code


class EmbedArgs(ctypes.Structure):
    _fields_ = [("ids", P), ("emb", P), ("h", P), ("rows", I32), ("hidden", I32), ("vocab", I32)]


class GemmArgs(ctypes.Structure):
    _fields_ = [("x", P), ("w", P), ("out", P), ("res", P), ("norm_w", P), ("partial", P),
                ("counters", P), ("ids_out", P), ("lens_inc", P), ("eps", F32), ("rows", I32),
                ("n", I32), ("k", I32), ("flags", ctypes.c_uint32), ("ksplit", I32), ("waves", I32),
                ("tiles_per_wg", I32), ("x_attn", P), ("x_frag", I32), ("out_frag", I32),
                ("parts_out", P), ("x_parts", P), ("x_nparts", I32), ("x_merged", P),
                ("next_norm_w", P), ("next_xn", P), ("next_merged", P), ("next_threads", I32),
                ("resident", I32)]


class AttnArgs(ctypes.Structure):
    _fields_ = [("qkv", P), ("q_norm_w", P), ("k_norm_w", P), ("cos_tab", P), ("sin_tab", P),
                ("lens", P), ("k_cache", P), ("v_cache", P), ("out", P), ("partial", P),
                ("counters", P), ("eps", F32), ("sm_scale", F32), ("batch", I32), ("t_rows", I32),
                ("nq", I32), ("nkv", I32), ("head_dim", I32), ("cap", I32), ("chunk", I32),
                ("waves", I32), ("out_partials", I32), ("out_frag", I32), ("strided", I32)]


class LayerArgs(ctypes.Structure):
    _fields_ = [("qkv", ctypes.POINTER(GemmArgs)), ("attn", ctypes.POINTER(AttnArgs)),
                ("o", ctypes.POINTER(GemmArgs)), ("gate_up", ctypes.POINTER(GemmArgs)),
                ("down", ctypes.POINTER(GemmArgs)), ("plan", P), ("ctl", P),
                ("spin_limit", ctypes.c_uint32), ("workgroups", I32)]


class DraftArgs(ctypes.Structure):
    _fields_ = [("hist", P), ("lens", P), ("ids", P), ("draft", P), ("batch", I32), ("cap", I32),
                ("primary", I32), ("backoff", I32), ("k", I32)]


class AcceptArgs(ctypes.Structure):
    _fields_ = [("out_tok", P), ("draft", P), ("hist", P), ("lens", P), ("naccept", P),
                ("batch", I32), ("cap", I32), ("k", I32), ("stop_len", I32)]


class RownormArgs(ctypes.Structure):
    _fields_ = [("x", P), ("norm_w", P), ("out", P), ("eps", F32), ("rows", I32), ("k", I32), ("tiles", I32)]


class PgemmArgs(ctypes.Structure):
    _fields_ = [("x", P), ("w", P), ("out", P), ("res", P), ("flags", ctypes.c_uint32), ("rows", I32),
                ("n", I32), ("k", I32), ("tiles", I32), ("out_frag", I32), ("tile_rows", I32),
                ("tile_cols", I32)]


class PrefillQkArgs(ctypes.Structure):
    _fields_ = [("qkv", P), ("q_norm_w", P), ("k_norm_w", P), ("cos_tab", P), ("sin_tab", P),
                ("k_cache", P), ("v_cache", P), ("eps", F32), ("batch", I32), ("t_rows", I32),
                ("pos0", I32), ("nq", I32), ("nkv", I32), ("head_dim", I32), ("cap", I32)]


class PrefillAttnArgs(ctypes.Structure):
    _fields_ = [("qkv", P), ("k_cache", P), ("v_cache", P), ("out", P), ("sm_scale", F32),
                ("batch", I32), ("t_rows", I32), ("pos0", I32), ("nq", I32), ("nkv", I32),
                ("head_dim", I32), ("cap", I32), ("tiles", I32)]


def declared_functions(header=HEADER):
    """Names of every function declared in include/qdec.h."""
    with open(header) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qdec_[a-z_0-9]+)\s*\(", text)))


class Lib:
    """Thin wrapper: one method per entry point, raising on error."""

    def __init__(self, path=LIB_PATH):
        if not os.path.exists(path):
            raise RuntimeError(
                f"libqdec.so not found at {path}; build it with "
                "`python -m qdec.build` (or __graft_entry__.build())")
        self.path = path
        self.so = ctypes.CDLL(path)
        so = self.so
        so.qdec_version.restype = ctypes.c_int
        so.qdec_last_error.restype = ctypes.c_char_p
        so.qdec_device_count.restype = ctypes.c_int
        so.qdec_tiled_offset.restype = ctypes.c_int64
        so.qdec_tiled_offset.argtypes = [ctypes.c_int64] * 3
        so.qdec_pack_tiles.argtypes = [P, P, ctypes.c_int64, ctypes.c_int64, P]
        so.qdec_read_probe.argtypes = [P, ctypes.c_int64, P, I32, P]
        so.qdec_read_probe.restype = ctypes.c_int
        for name, st in (("qdec_embed", EmbedArgs), ("qdec_gemm", GemmArgs), ("qdec_attn", AttnArgs),
                         ("qdec_attn_noalloc", AttnArgs),
                         ("qdec_ngram_draft", DraftArgs), ("qdec_spec_accept", AcceptArgs),
                         ("qdec_rownorm", RownormArgs), ("qdec_prefill_gemm", PgemmArgs),
                         ("qdec_prefill_qk", PrefillQkArgs), ("qdec_prefill_attn", PrefillAttnArgs)):
            fn = getattr(so, name)
            fn.argtypes = [ctypes.POINTER(st), P]
            fn.restype = ctypes.c_int
        so.qdec_layer_prepare.argtypes = [ctypes.POINTER(LayerArgs)]
        so.qdec_layer_prepare.restype = ctypes.c_int
        so.qdec_layer.argtypes = [ctypes.POINTER(LayerArgs), P]
        so.qdec_layer.restype = ctypes.c_int
        for name, st in (("qdec_gemm_workspace", GemmArgs), ("qdec_attn_workspace", AttnArgs)):
            fn = getattr(so, name)
            fn.argtypes = [ctypes.POINTER(st), ctypes.POINTER(ctypes.c_size_t),
                           ctypes.POINTER(ctypes.c_size_t)]
            fn.restype = ctypes.c_int
        so.qdec_gemm_prepass.argtypes = [ctypes.POINTER(GemmArgs), ctypes.POINTER(I32)]
        so.qdec_gemm_prepass.restype = ctypes.c_int

    def _check(self, fn, rc):
        if rc != 0:
            raise QdecError(fn, rc, self.so.qdec_last_error().decode(errors="replace"))

    def version(self):
        return self.so.qdec_version()

    def device_count(self):
        return self.so.qdec_device_count()

    def last_error(self):
        return self.so.qdec_last_error().decode(errors="replace")

    def tiled_offset(self, n, k, K):
        return self.so.qdec_tiled_offset(n, k, K)

    def pack_tiles(self, src, dst, n, k, stream):
        self._check("qdec_pack_tiles", self.so.qdec_pack_tiles(src, dst, n, k, stream))

    def read_probe(self, buf, nbytes, sink, blocks, stream):
        self._check("qdec_read_probe", self.so.qdec_read_probe(buf, nbytes, sink, blocks, stream))

    def embed(self, args, stream):
        self._check("qdec_embed", self.so.qdec_embed(ctypes.byref(args), stream))

    def gemm(self, args, stream):
        self._check("qdec_gemm", self.so.qdec_gemm(ctypes.byref(args), stream))

    def attn(self, args, stream):
        self._check("qdec_attn", self.so.qdec_attn(ctypes.byref(args), stream))

    def attn_noalloc(self, args, stream):
        self._check("qdec_attn_noalloc", self.so.qdec_attn_noalloc(ctypes.byref(args), stream))

    def layer_prepare(self, args):
        self._check("qdec_layer_prepare", self.so.qdec_layer_prepare(ctypes.byref(args)))

    def layer(self, args, stream):
        self._check("qdec_layer", self.so.qdec_layer(ctypes.byref(args), stream))

    def ngram_draft(self, args, stream):
        self._check("qdec_ngram_draft", self.so.qdec_ngram_draft(ctypes.byref(args), stream))

    def spec_accept(self, args, stream):
        self._check("qdec_spec_accept", self.so.qdec_spec_accept(ctypes.byref(args), stream))

    def rownorm(self, args, stream):
        self._check("qdec_rownorm", self.so.qdec_rownorm(ctypes.byref(args), stream))

    def prefill_gemm(self, args, stream):
        self._check("qdec_prefill_gemm", self.so.qdec_prefill_gemm(ctypes.byref(args), stream))

    def prefill_qk(self, args, stream):
        self._check("qdec_prefill_qk", self.so.qdec_prefill_qk(ctypes.byref(args), stream))

    def prefill_attn(self, args, stream):
        self._check("qdec_prefill_attn", self.so.qdec_prefill_attn(ctypes.byref(args), stream))

    def gemm_workspace(self, args):
        pb, cb = ctypes.c_size_t(), ctypes.c_size_t()
        self._check("qdec_gemm_workspace",
                    self.so.qdec_gemm_workspace(ctypes.byref(args), ctypes.byref(pb), ctypes.byref(cb)))
        return pb.value, cb.value

    def gemm_prepass(self, args):
        """(runs a normalisation pre-pass of its own, its workgroup size) of a
        qdec_gemm call with these arguments."""
        t = I32()
        rc = self.so.qdec_gemm_prepass(ctypes.byref(args), ctypes.byref(t))
        if rc < 0:
            self._check("qdec_gemm_prepass", rc)
        return rc == 1, t.value

    def attn_workspace(self, args):
        pb, cb = ctypes.c_size_t(), ctypes.c_size_t()
        self._check("qdec_attn_workspace",
                    self.so.qdec_attn_workspace(ctypes.byref(args), ctypes.byref(pb), ctypes.byref(cb)))
        return pb.value, cb.value


_LIB = None


def lib():
    """The process-wide library handle (loaded on first use)."""
    global _LIB
    if _LIB is None:
        _LIB = Lib()
    return _LIB
