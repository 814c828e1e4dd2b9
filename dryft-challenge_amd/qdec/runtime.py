"""Device-side state of the decode engine and the step that drives the kernels.

``DeviceModel`` holds the packed weights of one Qwen3 checkpoint in HBM:

* per role one contiguous buffer over all layers, each layer's matrix in the
  tiled MFMA layout of include/qdec.h -- ``qkv`` ([q; k; v] rows, 6144 x 2560
  for Qwen3-4B, as engine/engine.py:273-275 concatenates them), ``o``,
  ``gate_up`` ([gate; up] rows, engine/engine.py:277), ``down``;
* the embedding once, tiled; a tied lm_head streams the same buffer
  (engine/engine.py:266-269), an untied one (Qwen3-8B and up) its own;
* norm weights row-major.

``DecodeState`` holds everything one (batch, capacity) shape needs: the static
KV cache, the activation buffers, the per-step device scalars (``ids``,
``lens``) and the scratch of the split reductions.  ``run_step`` issues one
forward over ``t_rows`` rows per sequence -- plain decode (1), speculative
verify (k + 1) or a prefill chunk -- as ~5 kernel launches per layer on one
stream, so it can be captured into a hipGraph as is.

Per-role launch plans are functions of the matrix shape only, never of the
row count: that keeps every output element's summation order the same for a
1-row and a 36-row call (the basis of lossless speculation).

``Prefill`` fills the cache from a prompt with the prefill kernels: every
prompt position of every sequence goes through a layer at once (in position
chunks of about ``PREFILL_ROWS`` rows), so each weight matrix is read once
per chunk and the products run on the matrix cores.
"""

import ctypes
import math

import torch

from . import capi

GEMM_MAX_ROWS = 64
ATTN_MAX_T = 16
# Rows (sequences x positions) of one prefill chunk: activations of 32K rows
# take about 2.2 GB; at that size O and down still make 1280 workgroups of
# the 256 x 256 product tile (32 x 4096 prompts: 1.33 s at 16K rows, 1.27 s
# at 32K, 1.29 s at 64K; the tokens are the same for any chunking).
PREFILL_ROWS = 32768
# Row tile of the prefill product (kPgRows of qdec_kernels.h); a chunk of
# fewer rows is padded to PREFILL_ROW_TILE_SMALL instead (kPgRowsSmall, the
# 64 x 64 tile), see prefill_tiles.
PREFILL_ROW_TILE = 256
PREFILL_ROW_TILE_SMALL = 64
# A prompt of at most this many rows in all (batch x length) runs its layer
# products through the decode GEMMs (qdec_gemm) instead of the matrix-core
# prefill products, which make too few workgroups at so few rows.
PREFILL_SKINNY_ROWS = GEMM_MAX_ROWS
# lm_head output tiles per workgroup from 2 rows (the role plan's 4 stays at
# 1 row).  Grouping changes no sum and the argmax partials are scanned
# lowest index first, so tokens and logits do not depend on it (MI355X,
# ms/step at 4 vs 8 tiles: batch 8 3.055 -> 3.031, batch 32 3.78 -> 3.72;
# batch 1 2.160 vs 2.170; again with the resident plans, 4 / 8 tiles: batch 8
# 2.443 / 2.442, batch 32 5.407 / 5.404).
LM_TILES_BATCHED = 8
# Plain decode up to this batch merges attention chunks in the O projection;
# above it the attention's last-arriving chunk merges them.  Same-box A/B,
# ms per step (merge in O / in the attention): batch 1 2.129 / 2.203 (512
# prompt), 2.228 / 2.320 (2048); batch 2 2.282 / 2.347 (512), 2.294 / 2.353
# (1024), 2.507 / 2.551 (4096); batch 3 2.427 / 2.413 (1024), 2.403 / 2.385
# (256); batch 4 2.538 / 2.474 (512), 2.569 / 2.483 (1024), 2.866 / 2.767
# (4096).  Both give the same bits.  Measured again once O could copy its
# rows into LDS when it merges nothing (O / attention us per launch, ms per
# step, merge in O / in the attention): batch 1 8.27 / 6.95 and 6.82 / 10.86,
# 2.070 / 2.143 ms; batch 2 (1024) 9.5 / 8.85 and 6.9 / 12.9, 2.228 / 2.256.
MERGE_IN_O_MAX_BATCH = 2
# qdec_layer (one launch per layer) takes plain decode up to this batch: its
# GEMM stages stage their rows from registers (kLayerMaxRows).
LAYER_MAX_BATCH = 4
# From this many rows per call the attention output and the SwiGLU output
# are written in MFMA fragment order and read that way by the O and down
# projections: one contiguous KiB per fragment load and no re-layout
# pre-pass.  Same-box A/B, ms per step (1024-token prompts): batch 16 3.61
# with fragment order from 17 rows, 3.11 from 9; batch 12 3.18 / 3.15;
# batch 8 (8-row plain steps) 2.96 / 2.95; batch 32 3.86 vs 4.09 row-major.
FRAG_ROWS = 9
# Norm hand-over: a RES_OUT call (O, or down) that feeds a NORM_IN call which
# would normalise its rows in a pre-pass launch of its own (gate/up from 6
# rows; the next QKV or the lm_head from 9) writes those rows itself, as its
# last workgroups finish (qdec_gemm's next_norm_w), and the consumer runs as
# a plain fragment-order call: one launch fewer, the same bits.  Off: on
# MI355X the in-launch hand-off (device-scope output stores, the arrival
# ticket, the wait, device-scope row loads) costs more than the launch it
# saves.  Same-box A/B, ms per step with / without: batch 8 3.002 / 2.966,
# batch 12 3.202 / 3.157, batch 20 4.138 / 4.011, batch 32 5.839 / 5.687
# (tokens identical).
HAND_OVER = False
# Loss-free speculation needs identical arithmetic in the plain and verify
# steps, so attention chunking depends on (batch, capacity) only.
# k splits of the down projection from this batch size (see role_plan).
DOWN_SPLIT = 4
DOWN_SPLIT_MIN_BATCH = 16
# From this batch the O projection runs 4 waves per workgroup instead of 8
# (see role_plan).
O_FOUR_WAVES_MIN_BATCH = 9
# k splits of the O projection at O_SPLIT_MIN_BATCH..O_SPLIT_MAX_BATCH (see
# role_plan): the partials go to the gate/up call's normalisation pre-pass.
O_SPLIT = 2
O_SPLIT_MIN_BATCH = 17
O_SPLIT_MAX_BATCH = 32
# Output tiles per workgroup of QKV and down at two M tiles (WIDE_MIN_ROWS..32
# rows).  Paired tiles run two per wave, so each activation fragment a wave
# loads feeds both (the sums do not change).  MI355X, 32 rows, us per launch
# (one tile / two): QKV 18.6 / 15.3 with 8 waves (pre-pass included), down
# 16.1 / 15.0; gate/up (28.4 / 30.4) and O (10.5 / 13.5) keep one.
WIDE_TILES = 2
WIDE_MIN_ROWS = 17
# gate/up at RESIDENT_ROWS rows runs with its rows resident in LDS
# (qdec_gemm's resident: one workgroup per CU reads its operands from one
# LDS copy of the normalised rows; up to 8 rows it normalises them itself,
# no pre-pass launch; the same bits as the plain path) wherever the
# library's plan takes the shape.  With runs of half pairs, same-box A/B at
# 1024-token prompts, gate/up us per launch and ms per step (plain /
# resident): batch 5 23.3 / 20.1 and 2.489 / 2.342, batch 4 20.05 / 20.2
# and 2.308 / 2.302; batch 3 19.4 / 20.2 and 2.262 / 2.278, batch 2 19.0 /
# 20.2, batch 1 (512 tokens) 19.06 / 20.2 and 2.074 / 2.121.
RESIDENT_GLU = True
RESIDENT_ROWS = ((4, 8), (17, 32))
# The RES_OUT roles that copy their 1..8 rows into LDS first (qdec_gemm's
# resident for RES_OUT: a weights-only ring; the same bits).  Same-box A/B,
# ms per step at 1024-token prompts (neither / down / down and O): batch 8
# 2.794 / 2.696 / 2.661, batch 4 2.469 / 2.420 / 2.398; down at one row (O
# takes the attention partials there): batch 1 2.138 -> 2.113.
RESIDENT_RES_ROLES = ("down", "o")
RESIDENT_RES_ROWS = (1, 8)
# ... and the split down projection (DOWN_SPLIT parts) at these rows, each
# part's rows copied into LDS once per workgroup (same-box A/B, ms per step:
# batch 32 at 4096-token prompts 5.635 -> 5.551, batch 20 at 1024 3.393 ->
# 3.311; down 15.1 -> 12.7 us per launch).
RESIDENT_SPLIT_ROWS = (17, 32)
# QKV (NORM_IN alone) at these rows takes gate/up's resident plan with single
# tiles: the workgroup normalises its rows into LDS itself.  Same-box A/B,
# QKV us per launch and ms per step, the same tokens: batch 8 (1024-token
# prompts) 11.5 -> 8.7, 2.651 -> 2.549; batch 4 9.65 -> 7.81, 2.364 ->
# 2.320; batch 1 (512) 8.82 -> 7.80.  gate/up stays off the resident plan
# below 6 rows: 19.0 -> 21.0 us at batch 1, 20.1 -> 21.1 at batch 4.  At
# 17..32 rows the pre-pass's rows are copied in and k splits over 4 waves
# (role_plan): batch 32 at 4096-token prompts 5.481 -> 5.449 ms per step.
RESIDENT_QKV_ROWS = ((1, 8), (17, 32))


def round_up(x, m):
    return (x + m - 1) // m * m


def prefill_tiles(rows):
    """16-row tiles of a prefill chunk of ``rows`` rows: rows rounded up to
    PREFILL_ROW_TILE_SMALL below PREFILL_ROW_TILE, else to PREFILL_ROW_TILE.
    So a short prompt's products run over its rows rounded up to 64, not to
    a whole 256-row tile."""
    g = PREFILL_ROW_TILE_SMALL if rows < PREFILL_ROW_TILE else PREFILL_ROW_TILE
    return round_up(rows, g) // 16


class ModelConfig:
    """The shape fields of a Hugging Face Qwen3 config dict."""

    def __init__(self, cfg):
        self.raw = dict(cfg)
        self.hidden = cfg["hidden_size"]
        self.inter = cfg["intermediate_size"]
        self.n_layers = cfg["num_hidden_layers"]
        self.nq = cfg["num_attention_heads"]
        self.nkv = cfg["num_key_value_heads"]
        self.head_dim = cfg.get("head_dim") or self.hidden // self.nq
        self.vocab = cfg["vocab_size"]
        self.eps = float(cfg.get("rms_norm_eps", 1e-6))
        rp = cfg.get("rope_parameters") or {}
        self.theta = float(rp.get("rope_theta", cfg.get("rope_theta", 10000.0)))
        # Transformers Qwen3Config default (configuration_qwen3.py:74): untied
        # unless the config says otherwise.
        self.tied = bool(cfg.get("tie_word_embeddings", False))
        self.n_qkv = (self.nq + 2 * self.nkv) * self.head_dim
        # query heads per kv head (2 for Qwen3-0.6B / 1.7B, 4 for 4B / 8B, 5
        # for 14B, 8 for 32B)
        self.group = self.nq // self.nkv if self.nkv and self.nq % self.nkv == 0 else 0

    @property
    def prefill_kernels(self):
        """Whether the prefill attention and head-norm kernels take this
        shape (head_dim 128, 2, 4 or 8 query heads per kv head, at most 80 heads of q and
        k); otherwise prompts go through the decode kernels
        (DecodeState.prefill_steps)."""
        return self.head_dim == 128 and self.group in (2, 4, 8) and self.nq + self.nkv <= 80

    def check_supported(self):
        problems = []
        if self.head_dim not in (128, 64):
            problems.append(f"head_dim {self.head_dim} (kernels implement 128 and 64)")
        if not 1 <= self.group <= 16:
            problems.append(f"{self.nq} q heads / {self.nkv} kv heads (kernels take 1..16 query heads per kv head)")
        for name, v, m in (("hidden", self.hidden, 32), ("intermediate", self.inter, 32),
                           ("vocab", self.vocab, 16)):
            if v % m:
                problems.append(f"{name} {v} not a multiple of {m}")
        if problems:
            raise ValueError("unsupported Qwen3 shape: " + "; ".join(problems))


def rope_tables(cap, head_dim, theta):
    """bf16 cos/sin ``[cap, head_dim]`` exactly as Transformers' rotary module
    builds them (transformers/models/qwen3/modeling_qwen3.py:106-137): fp32
    ``inv_freq``, one fp32 product per (position, frequency), fp32 cos/sin,
    then one rounding to bf16.  Computed on the host so the values do not
    depend on a device libm."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).to(torch.float32) / head_dim))
    pos = torch.arange(cap, dtype=torch.float32)
    freqs = pos[:, None] * inv_freq[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)


def role_plan(n, k, role, batch=1):
    """(ksplit, waves, tiles_per_wg) of one projection role at a batch size.

    Output tiles are 16 columns, one workgroup per tile (4 per workgroup for
    the lm_head), no k split across workgroups: a split's cross-workgroup
    reduction cost more than it won back on MI355X.  The roles with few
    tiles (N = hidden: O and down, 160 tiles for 256 CUs) run 8 waves per
    workgroup, which doubles the weight blocks each busy CU keeps in flight
    (O 7.6 -> 7.0 us, down 14.2 -> 13.5 us at batch 1); O goes back to 4
    from O_FOUR_WAVES_MIN_BATCH.  The lm_head runs 4
    tiles per workgroup (137 us against 144 us with 8 and 146 us with 2,
    non-temporal weight loads).  Only (n, k, role) and the batch decide it,
    never the row count, so a verify pass over batch x (k + 1) rows sums
    every element as the plain step of the same batch does."""
    ks = k // 32
    ntiles = n // 16
    ksplit = 1
    waves = 8 if ntiles <= 256 else 4
    if (role == "down" and batch >= DOWN_SPLIT_MIN_BATCH and DOWN_SPLIT > 1 and ntiles <= 256
            and ks % (DOWN_SPLIT * 4) == 0):
        # Few tiles and a long k: split k in DOWN_SPLIT, four waves each, and
        # leave the partials to the next NORM_IN call (x_parts), whose
        # normalisation pre-pass merges them (Qwen3-4B: 640 workgroups instead
        # of 160).  Measured on MI355X, ms per step: batch 32 3.69 -> 3.62;
        # batch 8 3.01 -> 3.09 and batch 1 2.145 -> 2.155 (QKV then needs the
        # pre-pass, or merges four partials per workgroup), so only from
        # DOWN_SPLIT_MIN_BATCH.
        return DOWN_SPLIT, 4, 1
    if (role == "o" and O_SPLIT_MIN_BATCH <= batch <= O_SPLIT_MAX_BATCH and O_SPLIT > 1 and ntiles <= 256
            and ks % (O_SPLIT * 4) == 0):
        # Split k in O_SPLIT, four waves each, and leave the partials to the
        # gate/up call's normalisation pre-pass, like the down projection's
        # to the next QKV's: each part's rows then fit the LDS of the resident
        # split plan (qdec_gemm resident; 128 KiB per part at 32 rows).
        # Same-box A/B at batch 32 and 4096-token prompts: O 10.5 -> 7.6 us
        # per launch.
        return O_SPLIT, 4, 1
    if role == "qkv" and batch >= WIDE_MIN_ROWS and not any(lo <= batch <= hi for lo, hi in RESIDENT_QKV_ROWS[1:]):
        # two tiles per wave (WIDE_TILES): 192 workgroups, 8 waves each; the
        # resident plan (RESIDENT_QKV_ROWS) splits k over 4 waves
        waves = 8
    if role == "o" and batch >= O_FOUR_WAVES_MIN_BATCH:
        # From 9 rows O takes the direct path (fragments loaded beside each
        # weight block), where 4 waves of 32 k steps beat 8 of 16.  Same-box
        # A/B, ms per step at 1024-token prompts (8 waves / 4), measured on
        # the direct path: batch 8 2.969 / 2.943, 10 3.091 / 3.073, 12 3.143 /
        # 3.123, 16 3.126 / 3.096, 32 3.609 / 3.610; with the rows staged in
        # LDS 4 waves lose: batch 7 2.993 / 3.073, 5 2.710 / 2.802, 3 2.404 /
        # 2.449, and, since 8 rows copy their rows into LDS too (the resident
        # plan), batch 8: O 7.21 / 7.78 us per launch, 2.448 / 2.467 ms.
        waves = 4
    while ks % waves:
        waves //= 2
    tiles = 1
    if role == "lm":
        for cand in (4, 2, 1):
            if ntiles % cand == 0:
                tiles = cand
                break
    return ksplit, waves, tiles


# From this batch the attention runs 8 waves per workgroup with the
# residency chunking of attn_chunk.  Same-box A/B, ms per step at 1024-token
# prompts, 8 waves / 4 waves: batch 8 2.964 / 3.017, batch 6 2.891 / 2.953;
# once the 8-wave chunks were equal over all CUs also batch 5 2.685 /
# 2.718 (2048 tokens 2.833 / 2.962), batch 4 2.460 / 2.482 (2048 tokens
# 2.545 / 2.554, 4096 tokens 2.728 / 2.774).  With strided chunks batch
# 3 gains too (512 tokens 2.234 / 2.281, 1024 2.263 / 2.307, 2048 2.372 /
# 2.359, 4096 2.542 / 2.554).  Batch 2, whose attention partials O merges,
# is mixed (1024 tokens 2.195 / 2.228, 2048 2.404 / 2.283: ten chunks to
# merge), and batch 1 (2.089 / 2.077) stays on 4.
ATTN8_MIN_BATCH = 3
# Rows per sequence an 8-wave attention workgroup takes (two M tiles of
# query rows per kv head).
ATTN8_MAX_T = 8
# From ATTN8_MIN_BATCH the chunks of a sequence take interleaved 32-slot
# blocks (qdec_attn strided): chunk c holds blocks c, c + C, ...  A partly
# filled cache then gives every chunk's workgroup the same work, where
# contiguous chunks sized for the capacity leave the last ones short or
# empty (and still loading their first blocks).  Same-box A/B at 1024-token
# prompts and 512 new tokens, attention us per launch / ms per step
# (contiguous / strided): batch 8 15.91 / 14.59, 2.560 / 2.521; batch 4
# 12.3 / 12.3, 2.379 / 2.370.
ATTN_STRIDED = True


def attn_waves(batch):
    """Wavefronts per attention workgroup: 8 from ATTN8_MIN_BATCH, so all
    blocks of a 512-slot chunk (or two per wave of a whole-cache one) are in
    flight at once (MI355X, ms/step: batch 8 3.100 -> 3.076, batch 32 6.129
    -> 6.098; with 1024-token prompts batch 6 2.970 -> 2.893 and batch 7
    3.070 -> 2.978; batch 4 and 5 once its chunks were spread over every
    CU, see ATTN8_MIN_BATCH), else 4.  A row's arithmetic depends on the count, so it is a function of the
    batch alone: plain and speculative states of one batch agree.  8 waves
    take at most ATTN8_MAX_T rows per sequence (max_rows_per_seq)."""
    return 8 if batch >= ATTN8_MIN_BATCH else 4


def max_rows_per_seq(batch, requested=ATTN_MAX_T, group=4):
    """Rows per sequence a state of ``batch`` runs per call (verify passes,
    prefill through the decode kernels): at most ``requested``, ATTN_MAX_T,
    GEMM_MAX_ROWS in all, and ATTN8_MAX_T when the attention runs 8 waves;
    with ``group`` query heads per kv head, at most 64 query rows per kv
    head (32 with 8 waves) -- the same bound at Qwen3-4B's 4."""
    eight = attn_waves(batch) == 8
    cap = min(ATTN8_MAX_T if eight else ATTN_MAX_T, (32 if eight else 64) // group)
    return max(1, min(requested, cap, GEMM_MAX_ROWS // batch))


def attn_chunk(batch, nkv, cap):
    """Slots per attention workgroup (a multiple of 32; absolute-slot
    chunking).  Measured on MI355X with 4-wave workgroups (graph-replayed,
    36 layers; below ATTN8_MIN_BATCH now): once batch x kv heads fills half
    the CUs one chunk per sequence is fastest (no merge); below that,
    smaller chunks trade the cross-workgroup merge against parallelism --
    256 at batch 2..5 and at batch 1 with long caches, 96 at batch 1 up to 1024
    slots (10.4 us at 128 vs 12.0 us at 256 for 640 cached slots; 21.5 vs
    17.1 us at 4000; with two attention workgroups per CU a batch-1 step at
    512..766 cached slots takes 2.187 ms at 96, 2.203 at 128, 2.250 at 64,
    2.241 at 192; at batch 8, 512 stays ahead of 256, 384 and 768).

    From ATTN8_MIN_BATCH (8-wave workgroups, one per CU) every workgroup of the
    launch should be resident at once: the cache in as many equal chunks as
    the 256 CUs hold (batch x kv heads x chunks), down to one, and at most
    one per 256 slots (rounded up).  A workgroup's K/V streams through
    one CU, so equal chunks over every CU beat 512-slot chunks that leave
    CUs idle or end in a short one: ms per step (512-slot chunks while they
    fit one round / equal chunks), 1024-token prompts batch 6 2.862 / 2.771
    (320 slots), 7 2.905 / 2.833 (416), 8 2.928 / 2.860 (416); batch 8 at
    512 tokens 2.894 / 2.773 (224), at 128 tokens 2.705 / 2.607.  Attention
    alone, 8 kv heads, us per launch: batch 16 at 4200 cached slots 69.0 in
    one chunk, 50.5 in two (57.4 in four, 64.8 in three); batch 16 at 1300
    slots 25.4 / 23.5; batch 12 at 1300 slots 24.4 in one, 33.0 in 512-slot
    chunks (288 workgroups: two rounds) and 21.8 in two; batch 10 at 1300
    slots 32.4 in 512-slot chunks, 19.1 in 544; batch 8 at 4200 slots 46.2
    in 512-slot chunks, 30.3 in 1120; batch 20, 24 and 32 stay faster in one
    chunk (71.6, 74.9, 86.7 against 86.8, 89.2, 97.5 in two)."""
    cap = round_up(cap, 32)
    if batch >= ATTN8_MIN_BATCH:
        pairs = batch * nkv
        n_chunks = max(1, min(256 // pairs, -(-cap // 256)))
        return round_up(-(-cap // n_chunks), 32)
    if batch * nkv >= 128:
        return cap
    # Below ATTN8_MIN_BATCH (4 waves, two workgroups per CU): 96 slots at
    # batch 1 up to 1024 slots, else about an eighth of the cache -- at batch
    # 1 at least 160 slots and at most the larger of 320 and a sixteenth,
    # from batch 2 at least 256.  Whole step, ms (batch 1): 1024-token
    # prompts 2.212 at 256, 2.157 at 192; 2048 tokens 2.279 at 256, 2.222 at
    # 288, 2.234 at 320; 4096 tokens 2.397 at 256, 2.310 at 320 (2.330 at
    # 384, 2.375 at 448); 8192 tokens 2.553 at 320, 2.513 at 512, 2.562 at
    # 768; 512 tokens 2.125 at 96, 2.136 at 128, 2.158 at 192.  Batch 2 at
    # 4096 tokens 2.823 at 256, 2.499 at 576; batch 3 at 2048 tokens 2.768
    # at 256, 2.517 at 320; batch 4 at 4096 tokens 3.602 at 256, 2.859 at
    # 576, at 1024 tokens 2.59 at 256 against 2.60-2.97 at 128-512.
    if batch == 1 and cap <= 1024:
        return min(cap, 96)
    eighth = round_up(-(-cap // 8), 32)
    if batch == 1:
        return min(cap, max(160, min(eighth, max(320, round_up(-(-cap // 16), 32)))))
    return min(cap, max(256, eighth))


class DeviceModel:
    """Packed Qwen3 weights in device memory."""

    def __init__(self, cfg, tensors, device="cuda:0", stream=None):
        self.cfg = ModelConfig(cfg)
        self.cfg.check_supported()
        self.device = torch.device(device)
        self.lib = capi.lib()
        c = self.cfg
        L, H, I, V = c.n_layers, c.hidden, c.inter, c.vocab
        dev = self.device
        bf = torch.bfloat16
        stream = stream or torch.cuda.current_stream(dev)
        s = stream.cuda_stream

        def get(name):
            t = tensors[name]
            return t.to(device=dev, dtype=bf).contiguous()

        # A tied checkpoint may still carry lm_head.weight; the engine then
        # streams the embedding for the lm_head, so the two must be the same
        # matrix.  An untied one (Qwen3-8B, -14B, -32B) must carry its own.
        if c.tied and "lm_head.weight" in tensors and not torch.equal(tensors["lm_head.weight"],
                                                                      tensors["model.embed_tokens.weight"]):
            raise ValueError("config ties the embeddings but lm_head.weight differs from "
                             "model.embed_tokens.weight")
        if not c.tied and "lm_head.weight" not in tensors:
            raise ValueError("config unties the embeddings (tie_word_embeddings false) but the checkpoint "
                             "has no lm_head.weight")

        def pack(dst, src):
            n, k = src.shape
            self.lib.pack_tiles(src.data_ptr(), dst.data_ptr(), n, k, s)

        self.w_qkv = torch.empty((L, c.n_qkv * H), dtype=bf, device=dev)
        self.w_o = torch.empty((L, H * c.nq * c.head_dim), dtype=bf, device=dev)
        self.w_gu = torch.empty((L, 2 * I * H), dtype=bf, device=dev)
        self.w_down = torch.empty((L, H * I), dtype=bf, device=dev)
        self.in_w = torch.empty((L, H), dtype=bf, device=dev)
        self.post_w = torch.empty((L, H), dtype=bf, device=dev)
        self.q_norm = torch.empty((L, c.head_dim), dtype=bf, device=dev)
        self.k_norm = torch.empty((L, c.head_dim), dtype=bf, device=dev)
        with torch.cuda.stream(stream):
            for i in range(L):
                p = f"model.layers.{i}."
                qkv = torch.cat([get(p + "self_attn.q_proj.weight"), get(p + "self_attn.k_proj.weight"),
                                 get(p + "self_attn.v_proj.weight")], dim=0)
                pack(self.w_qkv[i], qkv)
                pack(self.w_o[i], get(p + "self_attn.o_proj.weight"))
                gu = torch.cat([get(p + "mlp.gate_proj.weight"), get(p + "mlp.up_proj.weight")], dim=0)
                pack(self.w_gu[i], gu)
                pack(self.w_down[i], get(p + "mlp.down_proj.weight"))
                self.in_w[i].copy_(get(p + "input_layernorm.weight"))
                self.post_w[i].copy_(get(p + "post_attention_layernorm.weight"))
                self.q_norm[i].copy_(get(p + "self_attn.q_norm.weight"))
                self.k_norm[i].copy_(get(p + "self_attn.k_norm.weight"))
                del qkv, gu
            self.norm_w = get("model.norm.weight")
            self.emb = torch.empty((V * H,), dtype=bf, device=dev)
            pack(self.emb, get("model.embed_tokens.weight"))
            # the lm_head's weights: the embedding itself when tied
            self.lm_w = self.emb
            if not c.tied:
                self.lm_w = torch.empty((V * H,), dtype=bf, device=dev)
                pack(self.lm_w, get("lm_head.weight"))
        stream.synchronize()
        self.plans = {
            "qkv": role_plan(c.n_qkv, H, "qkv"),
            "o": role_plan(H, c.nq * c.head_dim, "o"),
            "gate_up": role_plan(I, H, "gate_up"),
            "down": role_plan(H, I, "down"),
            "lm": role_plan(V, H, "lm"),
        }

    def weight_bytes(self):
        """Bytes of weights one decode step streams (norm vectors included)."""
        ts = (self.w_qkv, self.w_o, self.w_gu, self.w_down, self.lm_w, self.in_w, self.post_w,
              self.q_norm, self.k_norm, self.norm_w)
        return sum(t.numel() * t.element_size() for t in ts)


class DecodeState:
    """Buffers for one (batch, capacity) shape and the step over them."""

    def __init__(self, model, batch, capacity, max_t=1, keep_logits=False):
        c = model.cfg
        self.model, self.lib = model, model.lib
        self.batch = batch
        self.cap = round_up(capacity, 32)
        self.max_t = max_rows_per_seq(batch, max_t, c.group)
        if batch > GEMM_MAX_ROWS:
            raise ValueError(f"batch {batch} > {GEMM_MAX_ROWS} rows per step")
        self.max_rows = batch * self.max_t
        dev, bf = model.device, torch.bfloat16
        L, H, D = c.n_layers, c.hidden, c.head_dim
        self.chunk = attn_chunk(batch, c.nkv, self.cap)
        # head_dim 64 (the tiny test configurations): four 16-channel output
        # tiles, one per wave of a 4-wave workgroup
        self.attn_waves = attn_waves(batch) if c.head_dim == 128 else 4
        assert self.attn_waves == 4 or self.max_t <= 8
        cache_shape = (L, batch, c.nkv, self.cap, D)
        self.k_cache = torch.zeros(cache_shape, dtype=bf, device=dev)
        self.v_cache = torch.zeros(cache_shape, dtype=bf, device=dev)
        self.layer_elems = batch * c.nkv * self.cap * D
        R = self.max_rows
        # The residual stream alternates between two buffers: the down
        # projection leaves its update as k-split partials (down_parts) and
        # the next layer's QKV (or the lm_head) merges them into the other
        # buffer while it reads the first.  Layer l's residual is
        # hbuf[l % 2]; the embedding and the prefill hand-off write hbuf[0].
        self.hbuf = torch.zeros((2, R, H), dtype=bf, device=dev)
        self.h = self.hbuf[0]
        self.plans = dict(model.plans)
        self.plans["down"] = role_plan(H, c.inter, "down", batch)
        self.plans["qkv"] = role_plan(c.n_qkv, H, "qkv", batch)
        self.plans["o"] = role_plan(H, c.nq * c.head_dim, "o", batch)
        ks, _, _ = self.plans["down"]
        self.down_parts = torch.zeros((ks, R, H), dtype=torch.float32, device=dev) if ks > 1 else None
        # A split O projection leaves its update as partials too (o_parts);
        # the gate/up call's pre-pass merges them into hpost, the residual
        # after the attention, to which the down projection's partials then
        # belong.
        ko, _, _ = self.plans["o"]
        assert ko == 1 or ks > 1, "a split O needs a split down (the residual then always moves by merges)"
        self.o_parts = torch.zeros((ko, R, H), dtype=torch.float32, device=dev) if ko > 1 else None
        self.hpost = torch.zeros((R, H), dtype=bf, device=dev) if ko > 1 else None
        self.qkv = torch.zeros((R, c.n_qkv), dtype=bf, device=dev)
        # attention -> O and gate/up -> down hand over in fragment order from
        # FRAG_ROWS rows: whole M tiles.
        self.attn_out = torch.zeros((round_up(R, 16), c.nq * D), dtype=bf, device=dev)
        self.act = torch.zeros((round_up(R, 16), c.inter), dtype=bf, device=dev)
        self.logits = torch.zeros((R, c.vocab), dtype=bf, device=dev) if keep_logits else None
        self.ids = torch.zeros((R,), dtype=torch.int64, device=dev)
        self.out_tok = torch.zeros((R,), dtype=torch.int64, device=dev)
        self.lens = torch.zeros((batch,), dtype=torch.int32, device=dev)
        cos, sin = rope_tables(self.cap, D, c.theta)
        self.cos, self.sin = cos.to(dev), sin.to(dev)
        # Norm hand-over target: the consumer's rows in fragment order.
        self.hand_over = HAND_OVER
        self._hand_cache = {}
        # the resident plans of qdec_gemm (RESIDENT_GLU: gate/up at
        # RESIDENT_ROWS, the RESIDENT_RES_ROLES at RESIDENT_RES_ROWS); a state
        # may turn them off before its first step
        self.resident = RESIDENT_GLU
        self.xn_hand = torch.zeros((round_up(R, 16) * H,), dtype=bf, device=dev)
        # scratch: sized for the largest call of every kernel.
        gw = 0
        gc = 1
        for role in ("qkv", "o", "gate_up", "down", "lm"):
            for t in range(1, self.max_t + 1):  # the plan (and its workspace) depends on the row count
                a = self._gemm_args(role, 0, batch * t, hand=self.hand_over)
                pb, cb = self.lib.gemm_workspace(a)
                gw, gc = max(gw, pb), max(gc, cb)
        self.gemm_partial = torch.zeros((max(gw, 16) // 4 + 4,), dtype=torch.float32, device=dev)
        self.gemm_counters = torch.zeros((max(gc, 4) // 4 + 4,), dtype=torch.int32, device=dev)
        aw, ac = self.lib.attn_workspace(self._attn_args(0, self.max_t))
        aw = max(aw, self.lib.attn_workspace(self._attn_args(0, 1, partials=True))[0])
        self.attn_partial = torch.zeros((max(aw, 16) // 4 + 4,), dtype=torch.float32, device=dev)
        self.attn_counters = torch.zeros((max(ac, 4) // 4 + 4,), dtype=torch.int32, device=dev)
        self._gemm_cache = {}
        self._attn_cache = {}
        self.layer_launch = False  # plain steps as one qdec_layer launch per layer

    # ----------------------------------------------------------- arguments
    def _merge_in_o(self, t_rows):
        """Plain decode of up to MERGE_IN_O_MAX_BATCH sequences: the
        attention leaves its chunk partials and the O projection merges them
        while staging its activations (no arrival pass); bit-identical to
        the merged output.  The O-side merge takes 4 query heads per kv
        head; other shapes merge in the attention."""
        c = self.model.cfg
        return t_rows == 1 and self.batch <= MERGE_IN_O_MAX_BATCH and c.group == 4 and c.head_dim == 128

    def _resident(self, a, role):
        """Whether the call ``a`` of ``role`` (resident still 0) runs
        resident: self.resident, the role and its row count in the resident
        plans (gate/up at RESIDENT_ROWS, RESIDENT_RES_ROLES at
        RESIDENT_RES_ROWS), and a plan the library accepts for this shape
        (asked once per role and row count)."""
        if not self.resident or a.x_attn or a.next_norm_w:
            return False
        if role == "gate_up":
            ok = not a.x_frag and any(lo <= a.rows <= hi for lo, hi in RESIDENT_ROWS)
        elif role == "qkv":
            ok = (not a.x_frag and any(lo <= a.rows <= hi for lo, hi in RESIDENT_QKV_ROWS)
                  and (not a.x_parts or a.rows >= WIDE_MIN_ROWS))
        elif role not in RESIDENT_RES_ROLES:
            ok = False
        elif a.parts_out:
            ok = RESIDENT_SPLIT_ROWS[0] <= a.rows <= RESIDENT_SPLIT_ROWS[1]
        else:
            ok = not a.x_frag and RESIDENT_RES_ROWS[0] <= a.rows <= RESIDENT_RES_ROWS[1]
        if not ok:
            return False
        cache = self.__dict__.setdefault("_resident_cache", {})
        key = (role, a.rows, bool(a.parts_out), bool(a.x_frag))
        if key not in cache:
            a.resident = 1
            try:
                self.lib.gemm_workspace(a)
                cache[key] = True
            except capi.QdecError:
                cache[key] = False
            a.resident = 0
        return cache[key]

    def _hb(self, layer):
        """Residual buffer of ``layer`` (hbuf[0] throughout when down does not
        split: its RES_OUT epilogue then updates the residual in place)."""
        return self.hbuf[layer % 2] if self.down_parts is not None else self.hbuf[0]

    def _residual_in(self, a, layer, pending):
        """x of a NORM_IN call at the start of ``layer`` (``layer`` =
        n_layers: the lm_head): the previous layer's residual, with the down
        projection's split update still to merge -- unless ``pending`` is
        False: rows written directly into hbuf[0], as the prefill hand-off
        does."""
        if not pending:
            a.x = self.hbuf[0].data_ptr()
        elif layer > 0 and self.down_parts is not None:
            a.x = (self._hb(layer - 1) if self.o_parts is None else self.hpost).data_ptr()
            a.x_parts, a.x_nparts = self.down_parts.data_ptr(), self.down_parts.shape[0]
            a.x_merged = self._hb(layer).data_ptr()
        else:
            a.x = self._hb(layer).data_ptr()

    def _hand_threads(self, prod_role, rows, last=False):
        """Workgroup size of the NORM_IN call that reads what ``prod_role``
        writes (O: gate/up; down: the next QKV, or the lm_head after the last
        layer) when that call would run a normalisation pre-pass of its own
        and ``prod_role`` can hand it its rows instead (qdec_gemm_prepass,
        and the producer's plan accepting next_norm_w); else None.  Both
        calls have ``rows`` rows, and the answer depends on nothing else."""
        key = (prod_role, rows, last)
        if key not in self._hand_cache:
            c = self.model.cfg
            cons = "gate_up" if prod_role == "o" else ("lm" if last else "qkv")
            pre, threads = self.lib.gemm_prepass(self._gemm_args(cons, c.n_layers if last else 1, rows))
            t = None
            if pre:
                pa = self._gemm_args(prod_role, 0, rows)
                pa.next_norm_w, pa.next_threads = self.model.norm_w.data_ptr(), threads
                try:
                    self.lib.gemm_workspace(pa)
                    t = threads
                except capi.QdecError:
                    t = None
            self._hand_cache[key] = t
        return self._hand_cache[key]

    def _take_hand(self, a):
        """A NORM_IN call whose producer handed it its normalised rows: a
        plain fragment-order call on them."""
        a.flags &= ~capi.NORM_IN
        a.x, a.x_frag, a.norm_w = self.xn_hand.data_ptr(), 1, None
        a.x_parts, a.x_nparts, a.x_merged = None, 0, None
        a.resident = 0

    def _gemm_args(self, role, layer, rows, ids_out=None, lens_inc=None, x_attn=None, pending=True, hand=False):
        """qdec_gemm arguments of ``role`` in ``layer`` over ``rows`` rows.
        ``hand``: the arguments of the step's own sequence of calls, where O
        and down hand the next NORM_IN call its rows when that pays
        (_hand_threads) and that call takes them."""
        m, c = self.model, self.model.cfg
        ksplit, waves, tiles = self.plans[role]
        a = capi.GemmArgs()
        a.eps, a.rows, a.ksplit, a.waves, a.tiles_per_wg = c.eps, rows, ksplit, waves, 1
        h = self._hb(layer)
        if role == "qkv":
            self._residual_in(a, layer, pending)
            a.w, a.out = m.w_qkv[layer].data_ptr(), self.qkv.data_ptr()
            a.norm_w = m.in_w[layer].data_ptr()
            a.n, a.k, a.flags = c.n_qkv, c.hidden, capi.NORM_IN
        elif role == "o":
            a.x, a.w, a.res = self.attn_out.data_ptr(), m.w_o[layer].data_ptr(), h.data_ptr()
            a.n, a.k, a.flags = c.hidden, c.nq * c.head_dim, capi.RES_OUT
            if x_attn is not None:
                a.x_attn = ctypes.addressof(x_attn)
                a._x_attn = x_attn  # keeps the referenced struct alive
            else:
                a.x_frag = 1 if rows >= FRAG_ROWS else 0
            if self.o_parts is not None:
                a.parts_out = self.o_parts.data_ptr()
        elif role == "gate_up":
            a.x, a.w, a.out = h.data_ptr(), m.w_gu[layer].data_ptr(), self.act.data_ptr()
            a.norm_w = m.post_w[layer].data_ptr()
            a.n, a.k, a.flags = c.inter, c.hidden, capi.NORM_IN | capi.GLU
            a.out_frag = 1 if rows >= FRAG_ROWS else 0
            if self.o_parts is not None:
                a.x_parts, a.x_nparts = self.o_parts.data_ptr(), self.o_parts.shape[0]
                a.x_merged = self.hpost.data_ptr()
        elif role == "down":
            hd = h if self.o_parts is None else self.hpost  # the residual down's update belongs to
            a.x, a.w, a.res = self.act.data_ptr(), m.w_down[layer].data_ptr(), hd.data_ptr()
            a.n, a.k, a.flags = c.hidden, c.inter, capi.RES_OUT
            a.x_frag = 1 if rows >= FRAG_ROWS else 0
            if self.down_parts is not None:
                a.parts_out = self.down_parts.data_ptr()
        elif role == "lm":
            self._residual_in(a, c.n_layers, pending)
            a.w = m.lm_w.data_ptr()
            a.norm_w = m.norm_w.data_ptr()
            a.n, a.k, a.flags = c.vocab, c.hidden, capi.NORM_IN | capi.ARGMAX
            # 8 tiles per workgroup from 2 rows; past two M tiles (33+ rows,
            # verify passes only) one, so the direct path's ring fits the
            # workgroup's k range (the grouping changes no sum).
            if rows == 1:
                a.tiles_per_wg = tiles
            elif rows <= 32 and (c.vocab // 16) % LM_TILES_BATCHED == 0:
                a.tiles_per_wg = LM_TILES_BATCHED
            else:
                a.tiles_per_wg = 1
            a.out = self.logits.data_ptr() if self.logits is not None else None
            a.ids_out = (ids_out if ids_out is not None else self.ids).data_ptr()
            a.lens_inc = lens_inc.data_ptr() if lens_inc is not None else None
        # two output tiles per workgroup for QKV and down at two M tiles
        if role in ("qkv", "down") and WIDE_MIN_ROWS <= rows <= 32 and (a.n // 16) % WIDE_TILES == 0:
            a.tiles_per_wg = WIDE_TILES
        if hasattr(self, "gemm_partial"):
            a.partial = self.gemm_partial.data_ptr()
            a.counters = self.gemm_counters.data_ptr()
        if role in ("gate_up", "qkv") + RESIDENT_RES_ROLES:
            wide = a.tiles_per_wg
            if role == "qkv":
                a.tiles_per_wg = 1  # the resident plan takes one tile per workgroup
            a.resident = 1 if self._resident(a, role) else 0
            if not a.resident:
                a.tiles_per_wg = wide
        if hand:
            L = c.n_layers
            if role in ("o", "down"):
                last = role == "down" and layer == L - 1
                t = self._hand_threads(role, rows, last)
                if t:
                    nw = m.post_w[layer] if role == "o" else (m.norm_w if last else m.in_w[layer + 1])
                    a.next_norm_w, a.next_xn, a.next_threads = nw.data_ptr(), self.xn_hand.data_ptr(), t
                    if role == "down" and self.down_parts is not None:
                        a.next_merged = self._hb(layer + 1).data_ptr()  # the consumer's x_merged
                    if role == "o" and self.o_parts is not None:
                        a.next_merged = self.hpost.data_ptr()
            elif role == "gate_up" and self._hand_threads("o", rows):
                self._take_hand(a)
            elif role == "qkv" and layer > 0 and pending and self._hand_threads("down", rows):
                self._take_hand(a)
            elif role == "lm" and pending and self._hand_threads("down", rows, last=True):
                self._take_hand(a)
        return a

    def _attn_args(self, layer, t_rows, partials=False):
        m, c = self.model, self.model.cfg
        a = capi.AttnArgs()
        a.out_partials = 1 if partials else 0
        a.out_frag = 1 if (not partials and self.batch * t_rows >= FRAG_ROWS) else 0
        a.qkv, a.q_norm_w, a.k_norm_w = self.qkv.data_ptr(), m.q_norm[layer].data_ptr(), m.k_norm[layer].data_ptr()
        a.cos_tab, a.sin_tab, a.lens = self.cos.data_ptr(), self.sin.data_ptr(), self.lens.data_ptr()
        a.k_cache = self.k_cache[layer].data_ptr()
        a.v_cache = self.v_cache[layer].data_ptr()
        a.out = self.attn_out.data_ptr()
        if hasattr(self, "attn_partial"):
            a.partial, a.counters = self.attn_partial.data_ptr(), self.attn_counters.data_ptr()
        a.eps, a.sm_scale = c.eps, c.head_dim ** -0.5
        a.batch, a.t_rows, a.nq, a.nkv, a.head_dim = self.batch, t_rows, c.nq, c.nkv, c.head_dim
        a.cap, a.chunk, a.waves = self.cap, self.chunk, self.attn_waves
        a.strided = 1 if (ATTN_STRIDED and self.attn_waves == 8 and self.chunk < self.cap) else 0
        return a

    # ---------------------------------------------------------------- step
    def run_step(self, t_rows=1, lm_head=True, ids_out=None, advance=True, stream=None):
        """One forward of ``t_rows`` rows per sequence at positions
        ``lens[b] .. lens[b] + t_rows - 1`` (device ``lens``), fed from
        ``ids[b * t_rows + t]``.

        With ``lm_head`` the greedy pick of every row goes to ``ids_out``
        (default ``ids``: the next step's input) and, with ``advance``,
        ``lens[b] += 1`` (plain decode; requires ``t_rows == 1``)."""
        if t_rows < 1 or t_rows > self.max_t:
            raise ValueError(f"t_rows {t_rows} not in [1, {self.max_t}]")
        if advance and lm_head and t_rows != 1:
            raise ValueError("advance needs t_rows == 1")
        lib, m, c = self.lib, self.model, self.model.cfg
        s = (stream or torch.cuda.current_stream(m.device)).cuda_stream
        rows = self.batch * t_rows
        e = capi.EmbedArgs()
        e.ids, e.emb, e.h = self.ids.data_ptr(), m.emb.data_ptr(), self.h.data_ptr()
        e.rows, e.hidden, e.vocab = rows, c.hidden, c.vocab
        lib.embed(e, s)
        pm = self._merge_in_o(t_rows)
        by_layer = self.layer_launch and t_rows == 1
        for i in range(c.n_layers):
            if by_layer:
                lib.layer(self._layer_args[i], s)
                continue
            lib.gemm(self._cached_gemm("qkv", i, rows), s)
            lib.attn(self._cached_attn(i, t_rows, pm), s)
            lib.gemm(self._cached_gemm("o", i, rows, self._cached_attn(i, t_rows, pm) if pm else None), s)
            lib.gemm(self._cached_gemm("gate_up", i, rows), s)
            lib.gemm(self._cached_gemm("down", i, rows), s)
        if lm_head:
            a = self._gemm_args("lm", 0, rows, ids_out=ids_out,
                                lens_inc=self.lens if (advance and t_rows == 1) else None, hand=self.hand_over)
            lib.gemm(a, s)

    def _cached_gemm(self, role, layer, rows, x_attn=None):
        key = (role, layer, rows, x_attn is not None, self.hand_over)
        a = self._gemm_cache.get(key)
        if a is None:
            a = self._gemm_args(role, layer, rows, x_attn=x_attn, hand=self.hand_over)
            self._gemm_cache[key] = a
        return a

    def _cached_attn(self, layer, t_rows, partials=False):
        key = (layer, t_rows, partials)
        a = self._attn_cache.get(key)
        if a is None:
            a = self._attn_args(layer, t_rows, partials)
            self._attn_cache[key] = a
        return a

    def step(self, t_rows=1, lm_head=True, ids_out=None, advance=True, stream=None):
        """One forward (``run_step``); the name every caller captures."""
        self.run_step(t_rows=t_rows, lm_head=lm_head, ids_out=ids_out, advance=advance, stream=stream)

    # ------------------------------------------------ one layer per launch
    def layer_supported(self):
        """Whether qdec_layer takes this state's plain decode steps: up to
        LAYER_MAX_BATCH sequences (its O stage always merges the attention
        partials, whatever MERGE_IN_O_MAX_BATCH says for five launches)."""
        return self.batch <= LAYER_MAX_BATCH and self.model.cfg.group == 4 and self.model.cfg.head_dim == 128

    def layer_attn_args(self, layer):
        """The attention stage of qdec_layer: this state's arguments with
        the layer kernel's 4 waves (its one block size) and contiguous
        chunks (strided ones run 8 waves), partials left for the O stage."""
        at = self._attn_args(layer, 1, partials=True)
        at.waves, at.strided = 4, 0
        return at

    def layer_gemm_args(self, role, layer, x_attn=None):
        """A GEMM stage of qdec_layer: the role's arguments under the layer
        kernel's plan (4 waves, no k split; gate/up two tiles per workgroup
        so every stage has at most one block per workgroup)."""
        a = self._gemm_args(role, layer, self.batch, x_attn=x_attn)
        a.ksplit, a.waves = 1, 4
        a.tiles_per_wg = 2 if role == "gate_up" else 1
        a.resident = 0  # the layer kernel's stages run the per-block code of the plain plans
        return a

    def enable_layer_launch(self, spin_limit=0, workgroups=0):
        """Run plain decode steps (t_rows 1) as one qdec_layer launch per
        layer: writes every layer's plan to device memory now (synchronous,
        so not under graph capture).  Verify passes (t_rows > 1) keep the
        per-operation launches; the layer kernel's 4-wave O and down sum in
        another order than this state's plans, so its rows are not
        bit-identical to theirs (within the logit tolerance instead)."""
        if not self.layer_supported():
            raise ValueError(f"qdec_layer takes at most {LAYER_MAX_BATCH} sequences (batch {self.batch})")
        c, dev = self.model.cfg, self.model.device
        if getattr(self, "layer_plan", None) is None:
            self.layer_plan = torch.zeros((c.n_layers, capi.LAYER_PLAN_BYTES), dtype=torch.uint8, device=dev)
            self.layer_ctl = torch.zeros((capi.LAYER_CTL_BYTES // 4,), dtype=torch.int32, device=dev)
        self._layer_args = []
        for i in range(c.n_layers):
            at = self.layer_attn_args(i)
            g = [self.layer_gemm_args("qkv", i), self.layer_gemm_args("o", i, x_attn=at),
                 self.layer_gemm_args("gate_up", i), self.layer_gemm_args("down", i)]
            la = capi.LayerArgs()
            la.qkv, la.o, la.gate_up, la.down = (ctypes.pointer(x) for x in g)
            la.attn = ctypes.pointer(at)
            la._keep = (at, g)  # the structs the pointers refer to
            la.plan, la.ctl = self.layer_plan[i].data_ptr(), self.layer_ctl.data_ptr()
            la.spin_limit, la.workgroups = spin_limit, workgroups
            self.lib.layer_prepare(la)
            self._layer_args.append(la)
        torch.cuda.synchronize(dev)
        self.layer_launch = True

    def disable_layer_launch(self):
        self.layer_launch = False

    def layer_error(self):
        """The layer kernel's error word: 0, 1 (a barrier wait ran out of
        polls), 2 (a launch whose plan was written for other arguments) or 3
        (a launch whose workgroup count differs from the one this ctl's
        tickets were counted with)."""
        return int(self.layer_ctl[2].item()) if getattr(self, "layer_ctl", None) is not None else 0

    def reset_layer_ctl(self):
        """Zero the barrier state (after an error, before the next launch)."""
        self.layer_ctl.zero_()

    # ------------------------------------------------------------- prefill
    def prefill(self, prompt, stream=None):
        """Fill cache slots ``0 .. S-1`` from ``prompt`` ``[B, S]`` (device
        int64) with the prefill kernels (``Prefill``), or with one decode
        step when the prompt fits one (``prefill_steps``); returns with
        ``ids[:B]`` = the first generated token, ``logits[:B]`` (if kept) its
        logits and ``lens[:] = S``."""
        B, S = prompt.shape
        if B != self.batch:
            raise ValueError(f"prompt batch {B} != state batch {self.batch}")
        if S < 1 or S >= self.cap:
            raise ValueError(f"prompt length {S} must be in [1, {self.cap})")
        if S <= max_rows_per_seq(B, group=self.model.cfg.group) or not self.model.cfg.prefill_kernels:
            # A prompt one decode step holds goes through the decode kernels:
            # with few rows the prefill products have too few workgroups
            # (MI355X, time to the first token, 16 tokens: 3.08 ms against
            # 5.35 at batch 1, 4.51 against 5.50 at batch 4; 8 tokens at
            # batch 8: 4.30 against 5.50).  The rule depends on (batch,
            # length) only, and the decode kernels give the same bits in any
            # number of steps, so plain and speculative states agree.
            self.prefill_steps(prompt, stream=stream)
            t = (S - 1) % self.max_t + 1
            if self.logits is not None and t > 1:  # logits[:B]: each sequence's last position
                self.logits[:B].copy_(self.logits[:B * t].view(B, t, -1)[:, t - 1].clone())
            return
        pf = getattr(self, "_prefill", None)
        if pf is None or pf.chunk < min(S, pf.max_chunk):
            pf = self._prefill = Prefill(self, S)
        pf.run(prompt, stream=stream)

    def prefill_steps(self, prompt, stream=None):
        """Fill cache slots ``0 .. S-1`` from ``prompt`` ``[B, S]`` (device
        int64) in chunks of ``max_t`` rows per sequence through the same
        kernels as decode; returns with ``ids[:B]`` = the first generated
        token and ``lens[:] = S``."""
        B, S = prompt.shape
        if B != self.batch:
            raise ValueError(f"prompt batch {B} != state batch {self.batch}")
        if S < 1 or S >= self.cap:
            raise ValueError(f"prompt length {S} must be in [1, {self.cap})")
        T = self.max_t
        for c0 in range(0, S, T):
            t = min(T, S - c0)
            self.ids[:B * t].view(B, t).copy_(prompt[:, c0:c0 + t])
            self.lens.fill_(c0)
            last = c0 + t >= S
            self.run_step(t_rows=t, lm_head=last, ids_out=self.out_tok, advance=False, stream=stream)
        t = (S - 1) % T + 1
        self.ids[:B].copy_(self.out_tok[:B * t].view(B, t)[:, t - 1])
        self.lens.fill_(S)


class Prefill:
    """Prompt processing for one ``DecodeState``.

    A chunk of ``chunk`` positions of every sequence (row ``b * T + t`` =
    sequence ``b`` at position ``c0 + t``) goes through each layer as
    rownorm -> QKV product -> head norm / RoPE / cache fill -> causal
    attention over the cache -> O product + residual -> rownorm -> gate/up
    product with SwiGLU -> down product + residual, the products on the
    matrix cores (qdec_prefill_gemm).  A prompt of at most
    PREFILL_SKINNY_ROWS rows runs its products as the decode GEMMs instead
    (qdec_gemm over all its rows, each weight read once; MI355X, one
    sequence: see DecodeState.prefill).  After the last chunk the final row
    of each sequence goes through the decode lm_head + argmax.

    Replaces engine/engine.py:448-490 (``_layers_forward`` over the whole
    prompt, ``_attend_prefill``, ``_prefill``)."""

    def __init__(self, state, prompt_len, rows=PREFILL_ROWS):
        c = state.model.cfg
        B = state.batch
        self.state = state
        self.max_chunk = max(1, rows // B)
        self.chunk = min(prompt_len, self.max_chunk)
        # The whole prompt in one chunk of at most PREFILL_SKINNY_ROWS rows:
        # the decode GEMMs (see _skinny_args).
        self.skinny = B * prompt_len <= min(PREFILL_SKINNY_ROWS, B * self.max_chunk)
        rows = prefill_tiles(B * self.chunk) * 16
        dev, bf = state.model.device, torch.bfloat16
        self.h = torch.zeros((rows, c.hidden), dtype=bf, device=dev)
        self.xn = torch.zeros((rows * c.hidden,), dtype=bf, device=dev)
        self.qkv = torch.zeros((rows, c.n_qkv), dtype=bf, device=dev)
        self.att = torch.zeros((rows * c.nq * c.head_dim,), dtype=bf, device=dev)
        self.act = torch.zeros((rows * c.inter,), dtype=bf, device=dev)
        self.ids = torch.zeros((rows,), dtype=torch.int64, device=dev)
        self.partial = self.counters = None

    def _skinny_args(self, role, layer, R):
        """qdec_gemm arguments of one layer product over all R prompt rows
        (row b*S + t): x of QKV and gate/up is the residual h (row-major,
        NORM_IN), the attention output comes in fragment order, and gate/up
        hands its SwiGLU rows to down in fragment order from FRAG_ROWS rows,
        as the decode step does.  Plans as the decode step's for R rows
        (two tiles per wave at 17-32 rows), without a k split."""
        st, m, c = self.state, self.state.model, self.state.model.cfg
        ksplit, waves, _ = m.plans[role]
        if role == "qkv" and R >= WIDE_MIN_ROWS:
            waves = 8
        a = capi.GemmArgs()
        a.eps, a.rows, a.ksplit, a.waves, a.tiles_per_wg = c.eps, R, 1, waves, 1
        frag = 1 if R >= FRAG_ROWS else 0
        if role == "qkv":
            a.x, a.w, a.out, a.norm_w = self.h.data_ptr(), m.w_qkv[layer].data_ptr(), self.qkv.data_ptr(), \
                m.in_w[layer].data_ptr()
            a.n, a.k, a.flags = c.n_qkv, c.hidden, capi.NORM_IN
        elif role == "o":
            a.x, a.w, a.res = self.att.data_ptr(), m.w_o[layer].data_ptr(), self.h.data_ptr()
            a.n, a.k, a.flags, a.x_frag = c.hidden, c.nq * c.head_dim, capi.RES_OUT, 1
        elif role == "gate_up":
            a.x, a.w, a.out, a.norm_w = self.h.data_ptr(), m.w_gu[layer].data_ptr(), self.act.data_ptr(), \
                m.post_w[layer].data_ptr()
            a.n, a.k, a.flags, a.out_frag = c.inter, c.hidden, capi.NORM_IN | capi.GLU, frag
        else:
            a.x, a.w, a.res = self.act.data_ptr(), m.w_down[layer].data_ptr(), self.h.data_ptr()
            a.n, a.k, a.flags, a.x_frag = c.hidden, c.inter, capi.RES_OUT, frag
        if role in ("qkv", "down") and WIDE_MIN_ROWS <= R <= 32 and (a.n // 16) % WIDE_TILES == 0:
            a.tiles_per_wg = WIDE_TILES
        if self.partial is not None:
            a.partial, a.counters = self.partial.data_ptr(), self.counters.data_ptr()
        return a

    def _skinny_workspace(self, R):
        """Scratch of the decode GEMMs over R rows (the plan, and so its
        scratch, depends on the row count); grown, never shrunk."""
        pb = cb = 16
        for role in ("qkv", "o", "gate_up", "down"):
            p_, c_ = self.state.lib.gemm_workspace(self._skinny_args(role, 0, R))
            pb, cb = max(pb, p_), max(cb, c_)
        if self.partial is None or self.partial.numel() * 4 < pb or self.counters.numel() * 4 < cb:
            dev = self.state.model.device
            self.partial = torch.zeros((pb // 4 + 4,), dtype=torch.float32, device=dev)
            self.counters = torch.zeros((cb // 4 + 4,), dtype=torch.int32, device=dev)

    def _gemm(self, x, w, out, n, k, rows, tiles, flags=0, res=None, out_frag=0):
        a = capi.PgemmArgs()
        a.x, a.w, a.out = x.data_ptr(), w.data_ptr(), out.data_ptr()
        a.res = res.data_ptr() if res is not None else None
        a.flags, a.rows, a.n, a.k, a.tiles, a.out_frag = flags, rows, n, k, tiles, out_frag
        return a

    def run(self, prompt, stream=None):
        st = self.state
        m, c, lib = st.model, st.model.cfg, st.lib
        B, S = prompt.shape
        s = (stream or torch.cuda.current_stream(m.device)).cuda_stream
        H, D = c.hidden, c.head_dim
        T = self.chunk
        for c0 in range(0, S, self.chunk):
            T = min(self.chunk, S - c0)
            R = B * T
            tiles = prefill_tiles(R)
            self.ids[:R].view(B, T).copy_(prompt[:, c0:c0 + T])
            e = capi.EmbedArgs()
            e.ids, e.emb, e.h = self.ids.data_ptr(), m.emb.data_ptr(), self.h.data_ptr()
            e.rows, e.hidden, e.vocab = R, H, c.vocab
            lib.embed(e, s)
            norm = capi.RownormArgs()
            norm.x, norm.out, norm.eps, norm.rows, norm.k, norm.tiles = (
                self.h.data_ptr(), self.xn.data_ptr(), c.eps, R, H, tiles)
            qk = capi.PrefillQkArgs()
            qk.qkv, qk.cos_tab, qk.sin_tab = self.qkv.data_ptr(), st.cos.data_ptr(), st.sin.data_ptr()
            qk.eps, qk.batch, qk.t_rows, qk.pos0 = c.eps, B, T, c0
            qk.nq, qk.nkv, qk.head_dim, qk.cap = c.nq, c.nkv, D, st.cap
            at = capi.PrefillAttnArgs()
            at.qkv, at.out, at.sm_scale = self.qkv.data_ptr(), self.att.data_ptr(), D ** -0.5
            at.batch, at.t_rows, at.pos0, at.nq, at.nkv = B, T, c0, c.nq, c.nkv
            at.head_dim, at.cap, at.tiles = D, st.cap, tiles
            if self.skinny:
                self._skinny_workspace(R)
                at.tiles = -(-R // 16)  # the fragment order of the decode GEMMs
                for i in range(c.n_layers):
                    lib.gemm(self._skinny_args("qkv", i, R), s)
                    qk.q_norm_w, qk.k_norm_w = m.q_norm[i].data_ptr(), m.k_norm[i].data_ptr()
                    qk.k_cache, qk.v_cache = st.k_cache[i].data_ptr(), st.v_cache[i].data_ptr()
                    lib.prefill_qk(qk, s)
                    at.k_cache, at.v_cache = qk.k_cache, qk.v_cache
                    lib.prefill_attn(at, s)
                    for role in ("o", "gate_up", "down"):
                        lib.gemm(self._skinny_args(role, i, R), s)
                continue
            g_qkv = self._gemm(self.xn, m.w_qkv[0], self.qkv, c.n_qkv, H, R, tiles)
            g_o = self._gemm(self.att, m.w_o[0], self.h, H, c.nq * D, R, tiles, capi.RES_OUT, res=self.h)
            g_gu = self._gemm(self.xn, m.w_gu[0], self.act, 2 * c.inter, H, R, tiles, capi.GLU, out_frag=1)
            g_dn = self._gemm(self.act, m.w_down[0], self.h, H, c.inter, R, tiles, capi.RES_OUT, res=self.h)
            for i in range(c.n_layers):
                norm.norm_w = m.in_w[i].data_ptr()
                lib.rownorm(norm, s)
                g_qkv.w = m.w_qkv[i].data_ptr()
                lib.prefill_gemm(g_qkv, s)
                qk.q_norm_w, qk.k_norm_w = m.q_norm[i].data_ptr(), m.k_norm[i].data_ptr()
                qk.k_cache, qk.v_cache = st.k_cache[i].data_ptr(), st.v_cache[i].data_ptr()
                lib.prefill_qk(qk, s)
                at.k_cache, at.v_cache = qk.k_cache, qk.v_cache
                lib.prefill_attn(at, s)
                g_o.w = m.w_o[i].data_ptr()
                lib.prefill_gemm(g_o, s)
                norm.norm_w = m.post_w[i].data_ptr()
                lib.rownorm(norm, s)
                g_gu.w = m.w_gu[i].data_ptr()
                lib.prefill_gemm(g_gu, s)
                g_dn.w = m.w_down[i].data_ptr()
                lib.prefill_gemm(g_dn, s)
        # The last position of every sequence: final norm, lm_head, argmax.
        st.h[:B].copy_(self.h[:B * T].view(B, T, H)[:, T - 1])
        lib.gemm(st._gemm_args("lm", 0, B, ids_out=st.ids, pending=False), s)
        st.lens.fill_(S)
