// Launch parameter blocks and launchers of the qdec kernels (internal).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qdec {

// Register budget of the GEMM: weight blocks a wave holds in flight per pass.
constexpr int kGemmKpMax = 20;
constexpr int kGemmKpMaxGlu = 10;
// LDS the GEMM may use for staged activations.
constexpr int kGemmLdsX = 64 * 1024;
// Direct path without NORM_IN: from this many rows (two M tiles) the
// activations are first copied into fragment order; below it the extra
// launch costs more than the uncoalesced fragment loads.
constexpr int kGemmRetileRows = 17;
// NORM_IN calls of at least this many rows take the direct path (with GLU,
// whose staged path stops at 4 register rows, from 6).
constexpr int kGemmDirectNormRows = 9;
constexpr int kGemmDirectGluRows = 6;
// Rows the pass path stages from registers (kFastRows of gemm_dev.h).
constexpr int kFastRowsMax = 4;
// 64-bit argmax keys per row (ARGMAX), each workgroup folding into one.
constexpr int kArgSlots = 16;
// Resident gate/up (gemm_resident.hip): NORM_IN | GLU calls with one
// workgroup per CU holding the normalised rows in LDS -- kResMinRows..
// kResMaxRows rows normalised by the workgroup itself, kResMinRows2..
// kResMaxRows2 rows (two M tiles) normalised by the pre-pass and copied in;
// at most kResMaxPairs units (tile pairs or half pairs, 4 waves each) per
// workgroup and
// kResMaxKSteps k steps (k <= 2560).  NORM_IN alone (QKV) takes the first
// kind with single tiles in place of the pairs.
constexpr int kResMinRows = 1;
constexpr int kResMaxRows = 8;
constexpr int kResMinRows2 = 17;
constexpr int kResMaxRows2 = 32;
constexpr int kResMaxPairs = 3;
constexpr int kResMaxKSteps = 80;
constexpr int kResRing = 10;  // weight ring slots (gate|up block pairs) per wave
constexpr int kResRing1 = 20;  // weight ring slots per wave without GLU (NORM_IN alone)
constexpr int kResMaxTiles1 = 2;  // tiles per workgroup without GLU
// RES_OUT with its rows staged in LDS by DMA (gemm_resident.hip): 2..
// kResLdsRows rows, at most kResLdsKSteps k steps (8 rows x 64 bytes each),
// kResLdsRing weight blocks in flight per wave.
constexpr int kResLdsRows = 8;
constexpr int kResLdsKSteps = 304;
constexpr int kResLdsRing = 20;
// RES_OUT split into k parts at two M tiles with each part's rows in LDS
// (gemm_resident.hip): at most kResSplitKSteps k steps per part (2 KiB each),
// kResSplitRing weight blocks in flight per wave.
constexpr int kResSplitKSteps = 76;
constexpr int kResSplitRing = 10;

struct GemmParams {
  const void *x;
  const void *w;
  void *out;
  void *res;
  const void *norm_w;
  float *partial;
  uint32_t *counters;
  int64_t *ids_out;
  int32_t *lens_inc;
  float eps;
  int rows, n, k;
  int ksplit, waves, tiles_per_wg;
  int KS;        // k / 32
  int ksw;       // k steps per wave
  int kp;        // k steps per wave per LDS pass
  int npass;
  int up_tiles;  // GLU: tile offset of the up half
  int xstride;   // LDS row stride of staged activations (elements)
  int lds_red_off, lds_x_off;
  int xfast;     // activations staged from registers (see gemm.hip)
  int lds_all;   // the workgroup's whole k range of x is staged in LDS once
  int rw;        // weight ring registers per wave (window path), 0 = passes
  int xd;        // window path with B fragments loaded straight from x (no LDS staging)
  uint16_t *xn;  // xd: pre-pass copy of x (normalised under NORM_IN) in the workspace
  int xt;        // > 0: xd reads x (or xn) in fragment order with this many M tiles
  int xpre;      // xd: run the pre-pass into xn first
  int tw;        // xd: output tiles per wave (1, or 2 at two M tiles)
  int ofrag;     // > 0: out is written in fragment order with this many M tiles
  // Activations merged from attention chunk partials (x_attn): layout of
  // attn_dev.h, head_dim 128, 4 query heads per kv head.
  int amerge;
  const float *apart;
  const int32_t *alens;
  int a_t_rows, a_nkv, a_chunk, a_nchunks, a_cap, a_strided;
  // Split residual updates: a RES_OUT producer writes its k-split partials
  // (parts_out); a NORM_IN consumer merges xnparts of them into x first
  // (xparts) and writes the merged residual rows to xmerged.
  float *parts_out;
  const float *xparts;
  int xnparts;
  uint16_t *xmerged;
  // Norm hand-over (RES_OUT, direct path; gemm_dev.h hand_over_row): the
  // next NORM_IN call's rows, normalised in fragment order with hxt M tiles
  // (hxn), the merged residual with parts_out (hmerged), the consumer's
  // workgroup size (hthreads), and the arrival / departure words (hsync).
  const uint16_t *hnorm_w;
  uint16_t *hxn;
  uint16_t *hmerged;
  int hthreads, hxt;
  uint32_t *hsync;
  int resident;  // gemm_resident.hip: 1 NORM_IN | GLU with the normalised rows in LDS, 2 RES_OUT with the rows in LDS,
                 // 3 RES_OUT split into k parts, each part's rows in LDS, 4 NORM_IN alone as 1
  int res_waves;  // resident: waves per workgroup (set by the launcher)
  int res_half;   // resident GLU: the units are runs of half pairs (set by the launcher)
  size_t lds_bytes;
};
// Template flag of the hand-over instantiations (beside the QDEC_* flags).
constexpr uint32_t kGemmHandOver = 1u << 8;
// Polls a hand-over row waits for the last arrival before it writes NaN.
constexpr uint32_t kHandSpin = 1u << 22;
// Split partials a hand-over merges (the pre-pass it replaces keeps them in
// registers up to this many).
constexpr int kHandMaxParts = 4;
bool gemm_flags_supported(uint32_t flags);
bool gemm_fast_path(const GemmParams &p, uint32_t flags);
int gemm_ring(int ksw, uint32_t flags);
int gemm_ring_direct(int mt, uint32_t flags, int tw, int ksw, int groups);
hipError_t launch_rownorm(const GemmParams &p, dim3 block, bool do_norm, hipStream_t s);
hipError_t launch_gemm(const GemmParams &p, uint32_t flags, hipStream_t s);
hipError_t launch_glu_resident(const GemmParams &p, hipStream_t s);
hipError_t launch_res_rows(const GemmParams &p, hipStream_t s);
hipError_t launch_res_split(const GemmParams &p, hipStream_t s);

struct AttnParams {
  const void *qkv;
  const void *q_norm_w;
  const void *k_norm_w;
  const void *cos_tab;
  const void *sin_tab;
  const int32_t *lens;
  void *k_cache;
  void *v_cache;
  void *out;
  float *partial;
  uint32_t *counters;
  float eps;
  float scale_log2;  // log2(e) / sqrt(head_dim)
  int batch, t_rows, nq, nkv, cap, chunk, nchunks, waves;
  int out_partials;
  int ofrag;  // > 0: out is written in fragment order with this many M tiles
  int head_dim;  // 128, or 64 (four waves)
  int strided;   // chunk c takes blocks c, c + nchunks, ... (else contiguous slots)
};
hipError_t launch_attn(const AttnParams &p, hipStream_t s);

// ---- one decode layer per launch (layer.hip)
// Barrier state of the layer kernel: tickets that only grow, in two levels
// (workgroup w arrives at group w % kLayerGroups, the last of a group at the
// top), each counter on its own 128-byte line; an error word (1: a
// barrier wait ran out of polls, 2: a stale plan, 3: a launch whose
// workgroup count differs from the one the tickets were counted with); and
// that workgroup count, recorded by the first launch on a zeroed ctl.
constexpr int kLayerGroups = 8;
struct LayerCtl {
  uint64_t ticket;  // top level: one arrival per group and barrier
  uint32_t err;
  uint32_t nwg;     // workgroups per launch (0 until the first launch)
  uint32_t pad0[28];
  struct Group {
    uint64_t arrive;   // one per workgroup and barrier
    uint64_t release;  // barriers this group has been released from
    uint64_t pad[14];
  } group[kLayerGroups];
};
// Stages in order: g[0] QKV, a attention, g[1] O, g[2] gate/up, g[3] down;
// nblk[i] = workgroups of g[i]'s own launch.  A launch reads it from device
// memory (a plan qdec_layer_prepare wrote), each stage when it starts: as
// kernel arguments all of it would be loaded at entry and held across the
// layer.  key: a hash of the rest, which the launch passes too.
struct LayerParams {
  uint64_t key;
  GemmParams g[4];
  AttnParams a;
  int nblk[4];
  int nwg;  // workgroups of the launch (in the key: a plan is for one count)
};
constexpr int kLayerThreads = 256;  // 4 waves: the plans of every stage
constexpr int kLayerMaxRows = 4;    // the GEMM stages stage their rows from registers
// Workgroups of one launch on the current device (all resident at once).
hipError_t layer_workgroups(size_t lds_bytes, int *out);
hipError_t launch_layer(const LayerParams *plan, uint64_t key, LayerCtl *ctl, uint32_t spin_limit, int workgroups,
                        size_t lds_bytes, hipStream_t s);
size_t layer_attn_lds_bytes();


// ---- prefill (prefill.hip)
// Product tiles of a workgroup (activation rows x weight rows): 256 x 128,
// 256 x 256 or 64 x 64; k a multiple of kPgStageK; the activation buffers
// hold whole row tiles of the tile used: kPgRows rows, or kPgRowsSmall with
// the 64 x 64 tile (the only one a call of fewer whole kPgRows tiles takes).
constexpr int kPqMaxHeads = 80;  // query + key heads per row of qdec_prefill_qk (Qwen3-32B: 72)
constexpr int kPgRows = 256;
constexpr int kPgRowsSmall = 64;
constexpr int kPgStageK = 64;
struct PgemmParams {
  const uint16_t *x;
  const uint16_t *w;
  uint16_t *out;
  const uint16_t *res;
  int rows, n, k;
  int tiles;     // M tiles of x (and of out in fragment order)
  int ofrag;     // out in fragment order
  int n_out;     // columns of out (n, or n/2 with GLU)
  int up_tiles;  // GLU: tile offset of the up half (n/32)
  int tile_rows; // activation rows per workgroup tile: 256 or 64
  int tile_cols; // weight rows per workgroup tile: 128 or 256 (64 with 64 rows)
  int wg_n;      // workgroup tiles along n
};
hipError_t launch_pgemm(const PgemmParams &p, uint32_t flags, hipStream_t s);

struct PqkParams {
  uint16_t *qkv;
  const uint16_t *q_norm_w, *k_norm_w, *cos_tab, *sin_tab;
  uint16_t *k_cache, *v_cache;
  float eps;
  int batch, t_rows, pos0, nq, nkv, cap;
};
hipError_t launch_prefill_qk(const PqkParams &p, hipStream_t s);

// Positions of one prefill attention workgroup.
constexpr int kPaRows = 64;
struct PattnParams {
  const uint16_t *qkv;
  const uint16_t *k_cache, *v_cache;
  uint16_t *out;
  float scale_log2;
  int batch, t_rows, pos0, nq, nkv, cap, tiles;
};
hipError_t launch_prefill_attn(const PattnParams &p, hipStream_t s);

hipError_t launch_rownorm_rows(const void *x, const void *norm_w, void *out, float eps, int rows, int k,
                               int tiles, hipStream_t s);
// One workgroup per 16-row tile (prefill.hip): for k up to 4096 and enough
// rows to fill the GPU.
bool pnorm_fits(int k, int rows);
hipError_t launch_pnorm(const void *x, const void *norm_w, void *out, float eps, int rows, int k, int tiles,
                        hipStream_t s);

hipError_t launch_embed(const int64_t *ids, const void *emb, void *h, int rows, int hidden,
                        int vocab, hipStream_t s);
hipError_t launch_pack(const void *src, void *dst, int64_t n, int64_t k, hipStream_t s);
hipError_t launch_read(const void *buf, int64_t bytes, uint32_t *sink, int blocks, hipStream_t s);
hipError_t launch_draft(const int64_t *hist, const int32_t *lens, int64_t *ids, int64_t *draft,
                        int batch, int cap, int primary, int backoff, int k, hipStream_t s);
hipError_t launch_accept(const int64_t *out_tok, const int64_t *draft, int64_t *hist,
                         int32_t *lens, int32_t *naccept, int batch, int cap, int k,
                         int stop_len, hipStream_t s);

}  // namespace qdec
