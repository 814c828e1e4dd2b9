// extern "C" entry points of libqdec.so: argument validation, workspace
// sizing and launch-plan derivation around the kernels.  Validation runs
// before any HIP call, so a bad call fails cleanly even without a GPU.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>

#include "qdec_common.h"
#include "qdec_kernels.h"

namespace qdec {

static thread_local char g_err[512] = "";

int set_error(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char *what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(QDEC_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  g_err[0] = '\0';
  return QDEC_OK;
}

static bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

static int launch_status(hipError_t e, const char *what) {
  if (e != hipSuccess) return set_error(QDEC_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
  return check_launch(what);
}

// Workspace of a planned GEMM call: fp32 k-split partials or the argmax
// partials, then (direct activations with NORM_IN) the normalised rows.
static void gemm_scratch(const qdec_gemm_args *a, const GemmParams &p, size_t *partial_bytes,
                         size_t *counter_bytes, size_t *xn_off) {
  const int ntiles = a->n / 16;
  size_t pb = 0, cb = 0;
  if (a->flags & QDEC_ARGMAX) {
    // one row: a key per workgroup; more: the arrival counter, then the keys
    if (a->rows == 1) pb = sizeof(uint64_t) * (size_t)(ntiles / a->tiles_per_wg);
    cb = 8 + sizeof(uint64_t) * kArgSlots * (size_t)a->rows;
  } else if (a->ksplit > 1 && !a->parts_out) {
    pb = sizeof(float) * (size_t)a->ksplit * a->rows * a->n * ((a->flags & QDEC_GLU) ? 2 : 1);
    cb = sizeof(uint32_t) * (size_t)ntiles;
  }
  if (a->next_norm_w) cb = std::max(cb, (size_t)12);  // hand-over arrival, departure and give-up words
  size_t off = 0;
  if ((p.xd || p.resident) && p.xpre) {
    off = (pb + 255) & ~(size_t)255;
    pb = off + sizeof(uint16_t) * (size_t)(p.xt ? p.xt * 16 : a->rows) * a->k;
  }
  *partial_bytes = pb;
  *counter_bytes = cb;
  *xn_off = off;
}

// Derive the launch plan of a GEMM call; returns QDEC_OK or an error code.
static int plan_gemm(const qdec_gemm_args *a, GemmParams *p, bool need_scratch) {
  if (!a) return set_error(QDEC_EINVAL, "qdec_gemm: null args");
  *p = GemmParams{};
  const uint32_t f = a->flags;
  if (!gemm_flags_supported(f)) return set_error(QDEC_EUNSUPPORTED, "qdec_gemm: flags 0x%x not supported", f);
  if (a->rows < 1 || a->rows > 64) return set_error(QDEC_EINVAL, "qdec_gemm: rows %d not in [1, 64]", a->rows);
  if (a->n <= 0 || a->n % 16) return set_error(QDEC_EINVAL, "qdec_gemm: n %d not a positive multiple of 16", a->n);
  if (a->k <= 0 || a->k % 32) return set_error(QDEC_EINVAL, "qdec_gemm: k %d not a positive multiple of 32", a->k);
  if (a->waves < 1 || a->waves > 8) return set_error(QDEC_EINVAL, "qdec_gemm: waves %d not in [1, 8]", a->waves);
  if (a->ksplit < 1) return set_error(QDEC_EINVAL, "qdec_gemm: ksplit %d < 1", a->ksplit);
  const int KS = a->k / 32;
  if (KS % a->ksplit) return set_error(QDEC_EINVAL, "qdec_gemm: k/32=%d not divisible by ksplit %d", KS, a->ksplit);
  if ((KS / a->ksplit) % a->waves)
    return set_error(QDEC_EINVAL, "qdec_gemm: k steps per split %d not divisible by waves %d", KS / a->ksplit, a->waves);
  const bool arg = (f & QDEC_ARGMAX) != 0;
  const bool glu = (f & QDEC_GLU) != 0;
  const int ntiles = a->n / 16;
  if (a->tiles_per_wg < 1) return set_error(QDEC_EINVAL, "qdec_gemm: tiles_per_wg %d < 1", a->tiles_per_wg);
  if (ntiles % a->tiles_per_wg) return set_error(QDEC_EINVAL, "qdec_gemm: n/16=%d not divisible by tiles_per_wg %d", ntiles, a->tiles_per_wg);
  if (arg && a->ksplit != 1) return set_error(QDEC_EUNSUPPORTED, "qdec_gemm: QDEC_ARGMAX needs ksplit 1");
  if ((a->x_frag != 0 && a->x_frag != 1) || (a->out_frag != 0 && a->out_frag != 1))
    return set_error(QDEC_EINVAL, "qdec_gemm: x_frag %d / out_frag %d not 0 or 1", a->x_frag, a->out_frag);
  if (a->out_frag && (f & (QDEC_RES_OUT | QDEC_ARGMAX)))
    return set_error(QDEC_EUNSUPPORTED, "qdec_gemm: out_frag with RES_OUT or ARGMAX");
  if (a->x_frag && ((f & QDEC_NORM_IN) || a->x_attn))
    return set_error(QDEC_EUNSUPPORTED, "qdec_gemm: x_frag needs no NORM_IN and no x_attn");
  if ((f == QDEC_GLU || f == QDEC_ARGMAX) && !a->x_frag)
    return set_error(QDEC_EUNSUPPORTED, "qdec_gemm: GLU or ARGMAX without NORM_IN needs x_frag = 1");
  if (a->parts_out && (f != QDEC_RES_OUT || a->ksplit < 2))
    return set_error(QDEC_EUNSUPPORTED, "qdec_gemm: parts_out needs RES_OUT alone and ksplit > 1");
  if (a->x_parts) {
    if (!(f & QDEC_NORM_IN) || a->ksplit != 1 || a->x_attn)
      return set_error(QDEC_EUNSUPPORTED, "qdec_gemm: x_parts needs NORM_IN, ksplit 1 and no x_attn");
    if (a->x_nparts < 1 || a->x_nparts > 8) return set_error(QDEC_EINVAL, "qdec_gemm: x_nparts %d not in [1, 8]", a->x_nparts);
    if (need_scratch && (!a->x_merged || a->x_merged == a->x))
      return set_error(QDEC_EINVAL, "qdec_gemm: x_parts needs x_merged, a buffer other than x");
    if ((reinterpret_cast<uintptr_t>(a->x_parts) & 15u) || (a->x_merged && !aligned16(a->x_merged)))
      return set_error(QDEC_EALIGN, "qdec_gemm: x_parts and x_merged must be 16-byte aligned");
  }
  const qdec_attn_args *xa = a->x_attn;
  if (xa) {
    if (f & QDEC_NORM_IN) return set_error(QDEC_EUNSUPPORTED, "qdec_gemm: x_attn with NORM_IN");
    if (!xa->out_partials) return set_error(QDEC_EINVAL, "qdec_gemm: x_attn call was not made with out_partials");
    if (xa->head_dim != 128 || xa->nkv < 1 || xa->nq != 4 * xa->nkv || xa->chunk < 32 || xa->cap < 32 ||
        xa->t_rows < 1 || xa->batch < 1)
      return set_error(QDEC_EINVAL, "qdec_gemm: x_attn shape");
    if (a->rows != xa->batch * xa->t_rows || a->k != xa->nq * xa->head_dim)
      return set_error(QDEC_EINVAL, "qdec_gemm: x_attn rows %d / k %d do not match the attention call", a->rows, a->k);
    if (need_scratch && (!xa->partial || !xa->lens)) return set_error(QDEC_EINVAL, "qdec_gemm: x_attn needs partial and lens");
  }
  if (need_scratch && ((!a->x && !xa) || !a->w)) return set_error(QDEC_EINVAL, "qdec_gemm: null x or w");
  if (need_scratch && (f & QDEC_NORM_IN) && !a->norm_w) return set_error(QDEC_EINVAL, "qdec_gemm: NORM_IN needs norm_w");
  if (need_scratch && (f & QDEC_RES_OUT) && !a->res) return set_error(QDEC_EINVAL, "qdec_gemm: RES_OUT needs res");
  if (need_scratch && !(f & (QDEC_RES_OUT | QDEC_ARGMAX)) && !a->out) return set_error(QDEC_EINVAL, "qdec_gemm: null out");
  if (need_scratch && arg && (!a->ids_out || !a->counters || (a->rows == 1 && !a->partial)))
    return set_error(QDEC_EINVAL, "qdec_gemm: ARGMAX needs ids_out, counters and (one row) partial");
  if (arg && ((reinterpret_cast<uintptr_t>(a->counters) & 7u) || (reinterpret_cast<uintptr_t>(a->partial) & 7u)))
    return set_error(QDEC_EALIGN, "qdec_gemm: ARGMAX needs 8-byte aligned counters and partial");
  if (need_scratch && a->ksplit > 1 && !a->parts_out && (!a->partial || !a->counters))
    return set_error(QDEC_EINVAL, "qdec_gemm: ksplit > 1 needs partial and counters (or parts_out)");
  if (!aligned16(a->x) || !aligned16(a->w) || (a->out && !aligned16(a->out)) || (a->res && !aligned16(a->res)) ||
      (a->norm_w && !aligned16(a->norm_w)))
    return set_error(QDEC_EALIGN, "qdec_gemm: x, w, out, res and norm_w must be 16-byte aligned");

  const int nacc = glu ? 2 : 1;
  const int mt = (a->rows + 15) / 16;
  p->x = a->x; p->w = a->w; p->out = a->out; p->res = a->res; p->norm_w = a->norm_w;
  p->partial = a->partial; p->counters = a->counters; p->ids_out = a->ids_out; p->lens_inc = a->lens_inc;
  p->eps = a->eps; p->rows = a->rows; p->n = a->n; p->k = a->k;
  p->ksplit = a->ksplit; p->waves = a->waves; p->tiles_per_wg = a->tiles_per_wg;
  p->KS = KS;
  p->xt = 0;
  p->xpre = 0;
  p->ofrag = a->out_frag ? (a->rows + 15) / 16 : 0;
  p->ksw = KS / a->ksplit / a->waves;
  p->up_tiles = ntiles;
  p->resident = 0;
  if (a->resident && f == QDEC_RES_OUT && a->parts_out) {
    // k parts left to the next NORM_IN call, each part's rows copied into
    // LDS once per workgroup (gemm_resident.hip); the direct path's
    // arithmetic.
    if (a->resident != 1) return set_error(QDEC_EINVAL, "qdec_gemm: resident %d not 0 or 1", a->resident);
    const int kp = a->ksplit > 0 ? KS / a->ksplit : 0;
    if (a->ksplit < 2 || a->waves != 4 || !a->x_frag || xa || a->next_norm_w || a->rows < 17 || a->rows > 32 ||
        kp > kResSplitKSteps)
      return set_error(QDEC_EUNSUPPORTED, "qdec_gemm: resident RES_OUT with parts_out needs ksplit > 1, 4 waves, "
                       "x_frag = 1, 17..32 rows and at most %d k steps per split (no x_attn or next_norm_w)",
                       kResSplitKSteps);
    p->resident = 3;
    p->rw = kResSplitRing;
    p->xt = 2;
    p->parts_out = a->parts_out;
    p->lds_bytes = 0;  // static LDS
    return QDEC_OK;
  }
  if (a->resident && f == QDEC_RES_OUT) {
    // The rows copied into LDS by each workgroup, weights-only ring
    // (gemm_resident.hip); the direct path's arithmetic.
    if (a->resident != 1) return set_error(QDEC_EINVAL, "qdec_gemm: resident %d not 0 or 1", a->resident);
    if (a->ksplit != 1 || a->tiles_per_wg != 1 || a->x_frag || xa || a->parts_out || a->next_norm_w)
      return set_error(QDEC_EUNSUPPORTED, "qdec_gemm: resident RES_OUT needs ksplit 1, one tile per workgroup and "
                       "row-major x (no x_frag, x_attn, parts_out or next_norm_w)");
    if (a->rows > kResLdsRows)
      return set_error(QDEC_EUNSUPPORTED, "qdec_gemm: resident RES_OUT takes 1..%d rows, not %d", kResLdsRows, a->rows);
    if (KS > kResLdsKSteps || (KS & 15))
      return set_error(QDEC_EUNSUPPORTED, "qdec_gemm: resident RES_OUT needs k/32 a multiple of 16 and at most %d (k %d)",
                       kResLdsKSteps, a->k);
    p->resident = 2;
    p->rw = kResLdsRing;
    p->lds_bytes = 0;  // static LDS
    return QDEC_OK;
  }
  if (a->resident) {
    // One workgroup per CU normalising the rows into LDS (gemm_resident.hip);
    // its arithmetic is that of the plan below (pre-pass + direct path).
    if (a->resident != 1) return set_error(QDEC_EINVAL, "qdec_gemm: resident %d not 0 or 1", a->resident);
    if ((f != (QDEC_NORM_IN | QDEC_GLU) && f != QDEC_NORM_IN) || a->ksplit != 1 || a->waves != 4 ||
        a->tiles_per_wg != 1 || a->x_frag || xa || a->next_norm_w)
      return set_error(QDEC_EUNSUPPORTED, "qdec_gemm: resident needs NORM_IN (with or without GLU), ksplit 1, 4 waves, "
                       "one tile per workgroup and row-major x (no x_frag, x_attn or next_norm_w)");
    const bool two = a->rows >= kResMinRows2 && a->rows <= kResMaxRows2;
    if (!two && (a->rows < kResMinRows || a->rows > kResMaxRows))
      return set_error(QDEC_EUNSUPPORTED, "qdec_gemm: resident takes %d..%d or %d..%d rows, not %d", kResMinRows,
                       kResMaxRows, kResMinRows2, kResMaxRows2, a->rows);
    const int ring = glu ? kResRing : kResRing1;
    if (KS > kResMaxKSteps || p->ksw % ring)
      return set_error(QDEC_EUNSUPPORTED, "qdec_gemm: resident needs k <= %d with k/128 a multiple of %d (k %d)",
                       kResMaxKSteps * 32, ring, a->k);
    if (ntiles < 2) return set_error(QDEC_EUNSUPPORTED, "qdec_gemm: resident needs at least two output tiles");
    p->resident = glu ? 1 : 4;
    p->rw = ring;
    p->kp = 0;
    p->npass = 0;
    p->lds_bytes = 0;  // static LDS
    if (a->x_parts && !two)
      return set_error(QDEC_EUNSUPPORTED, "qdec_gemm: resident with x_parts takes %d..%d rows (the pre-pass merges "
                       "them), not %d", kResMinRows2, kResMaxRows2, a->rows);
    if (two) {
      // the normalisation pre-pass writes the rows in fragment order first
      // (merging a pending split residual update into x_merged on the way)
      p->xpre = 1;
      p->xt = 2;
      p->xparts = a->x_parts;
      p->xnparts = a->x_parts ? a->x_nparts : 0;
      p->xmerged = reinterpret_cast<uint16_t *>(a->x_merged);
    }
    size_t pb = 0, cb = 0, xn_off = 0;
    gemm_scratch(a, *p, &pb, &cb, &xn_off);
    if (need_scratch && pb && !a->partial) return set_error(QDEC_EINVAL, "qdec_gemm: this call needs a partial workspace");
    if (p->xpre && a->partial) p->xn = reinterpret_cast<uint16_t *>(reinterpret_cast<char *>(a->partial) + xn_off);
    return QDEC_OK;
  }
  const int kpmax = glu ? kGemmKpMaxGlu : kGemmKpMax;
  // k steps per pass: register budget, then LDS budget for rows x waves x kp x 32.
  const size_t red_bytes = (size_t)(a->waves - 1) * nacc * mt * 64 * 16;
  const size_t head = 784;
  const size_t budget = kGemmLdsX - red_bytes - head;
  // Register passes of up to kpmax k steps; x staged for the whole range at
  // once when it fits the LDS budget, else per pass (fewer steps per pass).
  int kp = std::min(p->ksw, kpmax);
  const bool lds_all = (size_t)a->rows * (a->waves * p->ksw * 32 + 8) * 2 <= budget;
  if (!lds_all)
    while (kp > 1 && (size_t)a->rows * (a->waves * kp * 32 + 8) * 2 > budget) --kp;
  p->kp = kp;
  p->npass = (p->ksw + kp - 1) / kp;
  p->lds_all = lds_all ? 1 : 0;
  p->xstride = a->waves * (lds_all ? p->ksw : kp) * 32 + 8;
  p->lds_red_off = (int)head;
  p->lds_x_off = (int)(head + red_bytes);
  p->lds_bytes = head + red_bytes + (size_t)a->rows * p->xstride * 2;
  p->xfast = gemm_fast_path(*p, f) ? 1 : 0;
  // Weight ring: x staged in LDS when it fits (one M tile); otherwise (no k
  // split) B fragments straight from x, with NORM_IN's normalised rows
  // written to the workspace by a pre-pass; passes only when neither fits.
  p->rw = 0;
  p->xd = 0;
  p->tw = 1;
  p->xn = nullptr;
  const int ring = gemm_ring(p->ksw, f);
  // Direct path: two tiles per wave at two M tiles when the workgroup's
  // tiles pair up, without GLU (sums unchanged: every tile keeps its own
  // MFMA chain).  gate/up stays at one: at 32 rows its four weight streams
  // per wave cost a third wave per SIMD (30.4 against 28.4 us).
  int tw = (mt == 2 && !glu && a->tiles_per_wg % 2 == 0 && (a->ksplit == 1 || a->parts_out)) ? 2 : 1;
  int ring_d = gemm_ring_direct(mt, f, tw, p->ksw, a->tiles_per_wg / tw);
  if (!ring_d && tw == 2) {
    tw = 1;
    ring_d = gemm_ring_direct(mt, f, 1, p->ksw, a->tiles_per_wg);
  }
  const size_t lds_direct = head + red_bytes * tw;
  // Past its register-staged rows a NORM_IN call does better on the direct
  // path: one normalisation pre-pass instead of every workgroup reading
  // whole rows for the statistics and then again for staging (gate/up at 8
  // rows 25.2 us vs 27.6 on MI355X; ms per step staged / direct, two
  // same-box A/Bs in either order: batch 6 2.914 / 2.880 and 2.917 / 2.868,
  // batch 7 2.986 / 2.917 and 2.983 / 2.907, batch 5 even (+-0.3%), and at
  // 4 rows, still from registers, 2.476 / 2.617).
  const bool stage_norm = !(f & QDEC_NORM_IN) || a->rows < (glu ? kGemmDirectGluRows : kGemmDirectNormRows);
  if (a->x_frag) {
    // x already in fragment order: the direct path reads it as it is.
    if (!ring_d) return set_error(QDEC_EUNSUPPORTED, "qdec_gemm: x_frag: no direct ring for rows %d", a->rows);
    p->rw = ring_d;
    p->xd = 1;
    p->tw = tw;
    p->xt = mt;
    p->xfast = 0;
    p->lds_all = 0;
    p->lds_bytes = lds_direct;
  } else if (mt == 1 && lds_all && ring && stage_norm) {
    p->rw = ring;
  } else if (a->ksplit == 1 && ring_d) {
    p->rw = ring_d;
    p->xd = 1;
    p->tw = tw;
    p->xfast = 0;
    p->lds_all = 0;
    p->lds_bytes = lds_direct;
    // The pre-pass writes x in fragment order (normalised under NORM_IN):
    // row-major fragments would cost a cache access per lane.
    if ((f & QDEC_NORM_IN) || a->rows >= kGemmRetileRows) {
      p->xt = mt;
      p->xpre = 1;
    }
  }
  // Register staging of 5..8 rows has a window-path instantiation only; on
  // the pass path (a wave's k range that no ring divides, e.g. the lm_head's
  // 8 k steps at hidden 1024) the rows are staged through LDS instead.
  if (p->xfast && a->rows > kFastRowsMax && p->rw == 0) p->xfast = 0;
  // A pending split residual update is merged by the register-staged
  // prologue at one row, else by the normalisation pre-pass (once per row;
  // per workgroup it would re-read every partial for every row).
  p->parts_out = a->parts_out;
  p->xparts = a->x_parts;
  p->xnparts = a->x_parts ? a->x_nparts : 0;
  p->xmerged = reinterpret_cast<uint16_t *>(a->x_merged);
  if (a->x_parts && !(a->rows == 1 && !glu && p->xfast && p->rw > 0 && a->x_nparts <= 4)) {
    if (!ring_d)
      return set_error(QDEC_EUNSUPPORTED, "qdec_gemm: x_parts at %d rows needs the direct path, which this tile "
                       "grouping does not allow", a->rows);
    p->rw = ring_d;
    p->xd = 1;
    p->tw = tw;
    p->xfast = 0;
    p->lds_all = 0;
    p->lds_bytes = lds_direct;
    p->xt = mt;
    p->xpre = 1;
  }
  p->amerge = 0;
  p->apart = nullptr;
  p->alens = nullptr;
  if (xa) {
    if (!p->xfast || p->xd || a->ksplit != 1)
      return set_error(QDEC_EUNSUPPORTED, "qdec_gemm: x_attn needs activations staged from registers (rows %d)", a->rows);
    p->amerge = 1;
    p->apart = xa->partial;
    p->alens = xa->lens;
    p->a_t_rows = xa->t_rows;
    p->a_nkv = xa->nkv;
    p->a_chunk = xa->chunk;
    p->a_nchunks = (xa->cap + xa->chunk - 1) / xa->chunk;
    p->a_cap = xa->cap;
    p->a_strided = xa->strided;
  }
  size_t pb = 0, cb = 0, xn_off = 0;
  gemm_scratch(a, *p, &pb, &cb, &xn_off);
  if (need_scratch && pb && !a->partial) return set_error(QDEC_EINVAL, "qdec_gemm: this call needs a partial workspace");
  if (p->xd && p->xpre && a->partial)
    p->xn = reinterpret_cast<uint16_t *>(reinterpret_cast<char *>(a->partial) + xn_off);
  if (p->lds_bytes > (size_t)kGemmLdsX)
    return set_error(QDEC_EUNSUPPORTED, "qdec_gemm: rows %d x waves %d needs %zu B of LDS", a->rows, a->waves,
                     p->lds_bytes);
  // Norm hand-over to the next NORM_IN call (gemm_dev.h hand_over_row).
  p->hnorm_w = nullptr;
  p->hxn = nullptr;
  p->hmerged = nullptr;
  p->hthreads = 0;
  p->hxt = 0;
  p->hsync = nullptr;
  if (a->next_norm_w) {
    const int nblk = (ntiles / a->tiles_per_wg) * a->ksplit;
    const int nr = mt * 16;
    if (f != QDEC_RES_OUT || !p->xd || (a->ksplit > 1 && !a->parts_out))
      return set_error(QDEC_EUNSUPPORTED, "qdec_gemm: next_norm_w needs RES_OUT alone on the direct path "
                       "(x_frag = 1 or 17+ rows), ksplit 1 or parts_out");
    if (a->parts_out && a->ksplit > kHandMaxParts)
      return set_error(QDEC_EUNSUPPORTED, "qdec_gemm: next_norm_w with parts_out merges at most %d splits", kHandMaxParts);
    // Two 16-byte vectors of the row per thread of this call (hand_over_row).
    const int vec_cap = a->next_threads > 64 * a->waves ? a->next_threads : 2 * a->next_threads;
    if (a->next_threads < 64 || a->next_threads % 64 || a->next_threads > 2 * 64 * a->waves || a->n / 8 > vec_cap)
      return set_error(QDEC_EUNSUPPORTED,
                       "qdec_gemm: next_threads %d (a multiple of 64, at most twice this call's %d threads; n / 8 = %d "
                       "vectors at most twice it, or at most it when it exceeds %d)",
                       a->next_threads, 64 * a->waves, a->n / 8, 64 * a->waves);
    if (nblk < nr)
      return set_error(QDEC_EUNSUPPORTED, "qdec_gemm: next_norm_w needs %d workgroups, the plan has %d", nr, nblk);
    if (need_scratch && (!a->next_xn || !a->counters || (a->parts_out && !a->next_merged)))
      return set_error(QDEC_EINVAL, "qdec_gemm: next_norm_w needs next_xn, counters and (with parts_out) next_merged");
    if (!aligned16(a->next_norm_w) || (a->next_xn && !aligned16(a->next_xn)) ||
        (a->next_merged && !aligned16(a->next_merged)))
      return set_error(QDEC_EALIGN, "qdec_gemm: next_norm_w, next_xn and next_merged must be 16-byte aligned");
    p->hnorm_w = reinterpret_cast<const uint16_t *>(a->next_norm_w);
    p->hxn = reinterpret_cast<uint16_t *>(a->next_xn);
    p->hmerged = reinterpret_cast<uint16_t *>(a->next_merged);
    p->hthreads = a->next_threads;
    p->hxt = mt;
    p->hsync = a->counters;
  }
  return QDEC_OK;
}

static int plan_attn(const qdec_attn_args *a, AttnParams *p, bool need_scratch) {
  if (!a) return set_error(QDEC_EINVAL, "qdec_attn: null args");
  if (a->head_dim != 128 && a->head_dim != 64)
    return set_error(QDEC_EUNSUPPORTED, "qdec_attn: head_dim %d (128, or 64 with 4 waves)", a->head_dim);
  if (a->head_dim == 64 && a->waves != 4)
    return set_error(QDEC_EUNSUPPORTED, "qdec_attn: head_dim 64 runs 4 waves (waves %d)", a->waves);
  if (a->nkv < 1 || a->nq < a->nkv || a->nq % a->nkv)
    return set_error(QDEC_EUNSUPPORTED, "qdec_attn: nq %d / nkv %d (a whole number of query heads per kv head)", a->nq,
                     a->nkv);
  if (a->batch < 1 || a->batch > 65535) return set_error(QDEC_EINVAL, "qdec_attn: batch %d", a->batch);
  if (a->t_rows < 1 || a->t_rows > 16) return set_error(QDEC_EINVAL, "qdec_attn: t_rows %d not in [1, 16]", a->t_rows);
  if (a->t_rows * (a->nq / a->nkv) > (a->waves == 8 ? 32 : 64))
    return set_error(QDEC_EUNSUPPORTED, "qdec_attn: %d query rows per kv head (t_rows x nq / nkv; at most 64, 32 with 8 waves)",
                     a->t_rows * (a->nq / a->nkv));
  if (a->cap < 32 || a->cap % 32) return set_error(QDEC_EINVAL, "qdec_attn: cap %d not a positive multiple of 32", a->cap);
  if (a->chunk < 32 || a->chunk % 32) return set_error(QDEC_EINVAL, "qdec_attn: chunk %d not a positive multiple of 32", a->chunk);
  if (a->waves != 4 && a->waves != 8)
    return set_error(QDEC_EINVAL, "qdec_attn: waves %d (the kernel runs 4 or 8 wavefronts)", a->waves);
  if (a->waves == 8 && a->t_rows > 8)
    return set_error(QDEC_EUNSUPPORTED, "qdec_attn: 8 waves take at most 8 rows per sequence (t_rows %d)", a->t_rows);
  if (a->out_partials != 0 && a->out_partials != 1)
    return set_error(QDEC_EINVAL, "qdec_attn: out_partials %d not 0 or 1", a->out_partials);
  if (a->out_frag != 0 && a->out_frag != 1) return set_error(QDEC_EINVAL, "qdec_attn: out_frag %d not 0 or 1", a->out_frag);
  if (a->strided != 0 && a->strided != 1) return set_error(QDEC_EINVAL, "qdec_attn: strided %d not 0 or 1", a->strided);
  if (a->strided && a->waves != 8)
    return set_error(QDEC_EUNSUPPORTED, "qdec_attn: strided chunks run 8 waves (waves %d)", a->waves);
  const int nchunks = (a->cap + a->chunk - 1) / a->chunk;
  if (!need_scratch) goto fill;
  if (!a->qkv || !a->q_norm_w || !a->k_norm_w || !a->cos_tab || !a->sin_tab || !a->lens || !a->k_cache ||
      !a->v_cache || !a->out)
    return set_error(QDEC_EINVAL, "qdec_attn: null pointer argument");
  if (nchunks > 1 && !a->out_partials && (!a->partial || !a->counters))
    return set_error(QDEC_EINVAL, "qdec_attn: more than one chunk needs partial and counters");
  if (a->out_partials && !a->partial) return set_error(QDEC_EINVAL, "qdec_attn: out_partials needs partial");
  if (!aligned16(a->qkv) || !aligned16(a->q_norm_w) || !aligned16(a->k_norm_w) || !aligned16(a->cos_tab) ||
      !aligned16(a->sin_tab) || !aligned16(a->k_cache) || !aligned16(a->v_cache) || !aligned16(a->out))
    return set_error(QDEC_EALIGN, "qdec_attn: tensor pointers must be 16-byte aligned");
fill:
  p->qkv = a->qkv; p->q_norm_w = a->q_norm_w; p->k_norm_w = a->k_norm_w;
  p->cos_tab = a->cos_tab; p->sin_tab = a->sin_tab; p->lens = a->lens;
  p->k_cache = a->k_cache; p->v_cache = a->v_cache; p->out = a->out;
  p->partial = a->partial; p->counters = a->counters;
  p->eps = a->eps;
  p->scale_log2 = a->sm_scale * 1.4426950408889634f;
  p->batch = a->batch; p->t_rows = a->t_rows; p->nq = a->nq; p->nkv = a->nkv;
  p->cap = a->cap; p->chunk = a->chunk; p->nchunks = nchunks; p->waves = a->waves;
  p->out_partials = a->out_partials;
  p->ofrag = (a->out_frag && !a->out_partials) ? (a->batch * a->t_rows + 15) / 16 : 0;
  p->head_dim = a->head_dim;
  p->strided = a->strided;
  return QDEC_OK;
}

// ------------------------------------------- attention without a workspace
// qdec_attn_noalloc runs qdec_attn with its arrival counters and chunk
// partials in this library-owned device array instead of caller buffers.
// Every GPU holds its own copy until the process ends; its device address is
// taken once per device with hipGetSymbolAddress and only that address is
// used from the host (the array's name is a host-side stand-in).  Calls on
// one GPU share it, so two such calls must not overlap (same stream, or
// ordered streams); every kernel leaves the counters at zero again.
static __device__ __align__(256) unsigned char scratch[QDEC_NOALLOC_COUNTER_BYTES + QDEC_NOALLOC_PARTIAL_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
unsigned char *g_scratch_ptr[kMaxDevices];

__global__ void clear_kernel(uint4 *p, int n16) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += gridDim.x * blockDim.x) p[i] = zero4();
}

// Device address of `scratch` on the current device; the first call on a
// device takes it and clears the counter region with a kernel on `s` (a
// kernel, not a memset, so a first call under hipGraph capture records a
// node that is safe to replay).
int scratch_on_current_device(hipStream_t s, unsigned char **out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    return set_error(QDEC_ENODEV, "qdec_attn_noalloc: no current HIP device (or id >= %d)", kMaxDevices);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return set_error(QDEC_ELAUNCH, "qdec_attn_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                       hipGetErrorString(e));
    hipLaunchKernelGGL(clear_kernel, dim3(16), dim3(256), 0, s, reinterpret_cast<uint4 *>(ptr),
                       (int)(QDEC_NOALLOC_COUNTER_BYTES / 16));
    const int rc = check_launch("qdec_attn_noalloc: clearing the scratch counters");
    if (rc != QDEC_OK) return rc;
    g_scratch_ptr[dev] = reinterpret_cast<unsigned char *>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return QDEC_OK;
}

}  // namespace

// ------------------------------------------------- one layer per launch
// Everything a qdec_layer call launches, from its arguments: each stage's
// plan (the same validation as its own call), checked against the stage
// plans layer_kernel is compiled for; the launch's workgroups and LDS.
namespace {

constexpr size_t kLayerLdsMax = 80u << 10;  // two workgroups per CU
static_assert(sizeof(LayerParams) <= QDEC_LAYER_PLAN_BYTES, "plan fits its buffer");
static_assert(sizeof(LayerCtl) == QDEC_LAYER_CTL_BYTES, "ctl layout");

uint64_t fnv1a(const void *p, size_t n) {
  const unsigned char *b = static_cast<const unsigned char *>(p);
  uint64_t h = 1469598103934665603ull;
  for (size_t i = 0; i < n; ++i) h = (h ^ b[i]) * 1099511628211ull;
  return h;
}

int plan_layer(const qdec_layer_args *a, LayerParams *L, int *workgroups, size_t *lds) {
  if (!a || !a->qkv || !a->attn || !a->o || !a->gate_up || !a->down)
    return set_error(QDEC_EINVAL, "qdec_layer: null argument");
  if (!a->plan || !aligned16(a->plan)) return set_error(QDEC_EALIGN, "qdec_layer: plan must be 16-byte aligned");
  if (!a->ctl || (reinterpret_cast<uintptr_t>(a->ctl) & 7u)) return set_error(QDEC_EALIGN, "qdec_layer: ctl must be 8-byte aligned");
  const qdec_attn_args &at = *a->attn;
  if (at.t_rows != 1 || at.waves != 4 || at.out_partials != 1 || at.batch < 1 || at.batch > kLayerMaxRows)
    return set_error(QDEC_EUNSUPPORTED,
                     "qdec_layer: attention t_rows %d waves %d out_partials %d batch %d (1, 4, 1, at most %d)",
                     at.t_rows, at.waves, at.out_partials, at.batch, kLayerMaxRows);
  if (a->o->x_attn != a->attn) return set_error(QDEC_EUNSUPPORTED, "qdec_layer: o must merge the attention (x_attn == attn)");
  memset(L, 0, sizeof *L);  // the key hashes the bytes, padding included
  const qdec_gemm_args *ga[4] = {a->qkv, a->o, a->gate_up, a->down};
  static const char *const names[4] = {"qkv", "o", "gate_up", "down"};
  static const uint32_t flags[4] = {QDEC_NORM_IN, QDEC_RES_OUT, QDEC_NORM_IN | QDEC_GLU, QDEC_RES_OUT};
  static const int rings[4] = {20, 16, 10, 20};
  for (int i = 0; i < 4; ++i) {
    const int rc = plan_gemm(ga[i], &L->g[i], true);
    if (rc != QDEC_OK) return rc;
    const GemmParams &p = L->g[i];
    const bool direct = i == 3;
    if (ga[i]->flags != flags[i] || p.rows != at.batch || p.waves != 4 || p.ksplit != 1 || p.rw != rings[i] ||
        (p.xd != 0) != direct || (!direct && !p.xfast) || p.xt || p.xpre || p.tw != 1 || p.ofrag || p.xparts ||
        p.parts_out || p.hxn || (p.amerge != 0) != (i == 1))
      return set_error(QDEC_EUNSUPPORTED,
                       "qdec_layer: %s plan (flags 0x%x rows %d waves %d ksplit %d ring %d direct %d) is not the "
                       "layer kernel's",
                       names[i], ga[i]->flags, p.rows, p.waves, p.ksplit, p.rw, p.xd);
    L->nblk[i] = (p.n / 16 / p.tiles_per_wg) * p.ksplit;
  }
  const int rc = plan_attn(a->attn, &L->a, true);
  if (rc != QDEC_OK) return rc;
  size_t need = layer_attn_lds_bytes();
  for (int i = 0; i < 4; ++i) need = std::max(need, L->g[i].lds_bytes);
  if (need > kLayerLdsMax) return set_error(QDEC_EUNSUPPORTED, "qdec_layer: %zu B of LDS per workgroup", need);
  // Workgroups that fit at once, queried once per device (the first call,
  // qdec_layer_prepare, runs outside stream capture).
  static std::mutex mu;
  static int wgs[kMaxDevices];
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    return set_error(QDEC_ENODEV, "qdec_layer: no current HIP device (or id >= %d)", kMaxDevices);
  }
  int maxw = 0;
  {
    std::lock_guard<std::mutex> lock(mu);
    if (!wgs[dev]) {
      const hipError_t e = layer_workgroups(kLayerLdsMax, &wgs[dev]);
      if (e != hipSuccess) {
        wgs[dev] = 0;
        return set_error(QDEC_ELAUNCH, "qdec_layer: occupancy query: %s", hipGetErrorString(e));
      }
    }
    maxw = wgs[dev];
  }
  const int w = a->workgroups ? a->workgroups : maxw - maxw % kLayerGroups;
  if (w < kLayerGroups || w > maxw || w % kLayerGroups)
    return set_error(QDEC_EINVAL, "qdec_layer: workgroups %d not a multiple of %d in [%d, %d] (all resident at once)",
                     a->workgroups, kLayerGroups, kLayerGroups, maxw);
  int blocks = L->a.nchunks * L->a.nkv * L->a.batch;
  for (int i = 0; i < 4; ++i) blocks = std::max(blocks, L->nblk[i]);
  if (blocks > w)
    return set_error(QDEC_EUNSUPPORTED, "qdec_layer: a stage has %d blocks for %d workgroups", blocks, w);
  L->nwg = w;
  L->key = fnv1a(L, sizeof *L) | 1ull;  // never 0, the value of zeroed memory
  *workgroups = w;
  *lds = need;
  return QDEC_OK;
}

}  // namespace

}  // namespace qdec

using namespace qdec;

extern "C" {

int qdec_version(void) { return QDEC_ABI_VERSION; }

const char *qdec_last_error(void) { return g_err; }

int qdec_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n;
}

int64_t qdec_tiled_offset(int64_t n, int64_t k, int64_t K) {
  if (K <= 0 || K % 32 || n < 0 || k < 0 || k >= K) return -1;
  const int64_t nt = n / 16, ks = k / 32;
  const int64_t lane = (n % 16) + 16 * ((k % 32) / 8);
  return ((nt * (K / 32) + ks) * 64 + lane) * 8 + (k % 8);
}

int qdec_pack_tiles(const void *src, void *dst, int64_t n, int64_t k, qdec_stream_t stream) {
  if (!src || !dst) return set_error(QDEC_EINVAL, "qdec_pack_tiles: null pointer");
  if (n <= 0 || n % 16 || k <= 0 || k % 32)
    return set_error(QDEC_EINVAL, "qdec_pack_tiles: shape [%lld, %lld] needs n %% 16 == 0 and k %% 32 == 0",
                     (long long)n, (long long)k);
  if (!aligned16(src) || !aligned16(dst)) return set_error(QDEC_EALIGN, "qdec_pack_tiles: pointers must be 16-byte aligned");
  return launch_status(launch_pack(src, dst, n, k, (hipStream_t)stream), "qdec_pack_tiles");
}

int qdec_read_probe(const void *buf, int64_t bytes, uint32_t *sink, int32_t blocks, qdec_stream_t stream) {
  if (!buf || !sink) return set_error(QDEC_EINVAL, "qdec_read_probe: null pointer");
  if (bytes <= 0 || bytes % 16 || blocks < 1)
    return set_error(QDEC_EINVAL, "qdec_read_probe: bytes %lld (a positive multiple of 16), blocks %d",
                     (long long)bytes, blocks);
  if (!aligned16(buf)) return set_error(QDEC_EALIGN, "qdec_read_probe: buf must be 16-byte aligned");
  return launch_status(launch_read(buf, bytes, sink, blocks, (hipStream_t)stream), "qdec_read_probe");
}

int qdec_embed(const qdec_embed_args *a, qdec_stream_t stream) {
  if (!a || !a->ids || !a->emb || !a->h) return set_error(QDEC_EINVAL, "qdec_embed: null pointer");
  if (a->rows < 1 || a->hidden <= 0 || a->hidden % 32 || a->vocab <= 0 || a->vocab % 16)
    return set_error(QDEC_EINVAL, "qdec_embed: rows %d hidden %d vocab %d", a->rows, a->hidden, a->vocab);
  if (!aligned16(a->emb) || !aligned16(a->h)) return set_error(QDEC_EALIGN, "qdec_embed: emb and h must be 16-byte aligned");
  return launch_status(launch_embed(a->ids, a->emb, a->h, a->rows, a->hidden, a->vocab, (hipStream_t)stream),
                       "qdec_embed");
}

int qdec_gemm_workspace(const qdec_gemm_args *a, size_t *partial_bytes, size_t *counter_bytes) {
  GemmParams p;
  const int rc = plan_gemm(a, &p, false);
  if (rc != QDEC_OK) return rc;
  size_t pb = 0, cb = 0, xn_off = 0;
  gemm_scratch(a, p, &pb, &cb, &xn_off);
  if (partial_bytes) *partial_bytes = pb;
  if (counter_bytes) *counter_bytes = cb;
  return QDEC_OK;
}

int qdec_gemm_prepass(const qdec_gemm_args *a, int32_t *threads) {
  GemmParams p;
  const int rc = plan_gemm(a, &p, false);
  if (rc != QDEC_OK) return rc;
  if (threads) *threads = 64 * a->waves;
  return ((p.xd || p.resident) && p.xpre) ? 1 : 0;
}

int qdec_gemm(const qdec_gemm_args *a, qdec_stream_t stream) {
  GemmParams p;
  const int rc = plan_gemm(a, &p, true);
  if (rc != QDEC_OK) return rc;
  return launch_status(launch_gemm(p, a->flags, (hipStream_t)stream), "qdec_gemm");
}

int qdec_attn_workspace(const qdec_attn_args *a, size_t *partial_bytes, size_t *counter_bytes) {
  AttnParams p;
  const int rc = plan_attn(a, &p, false);
  if (rc != QDEC_OK) return rc;
  const size_t R = (size_t)a->t_rows * (a->nq / a->nkv);
  const bool parts = p.nchunks > 1 || a->out_partials;
  if (partial_bytes)
    *partial_bytes = parts ? sizeof(float) * (size_t)a->batch * a->nkv * p.nchunks * R * (a->head_dim + 2) : 0;
  if (counter_bytes) *counter_bytes = (p.nchunks > 1 && !a->out_partials) ? sizeof(uint32_t) * (size_t)a->batch * a->nkv : 0;
  return QDEC_OK;
}

int qdec_attn(const qdec_attn_args *a, qdec_stream_t stream) {
  AttnParams p;
  const int rc = plan_attn(a, &p, true);
  if (rc != QDEC_OK) return rc;
  return launch_status(launch_attn(p, (hipStream_t)stream), "qdec_attn");
}

int qdec_attn_noalloc(const qdec_attn_args *a, qdec_stream_t stream) {
  if (!a) return set_error(QDEC_EINVAL, "qdec_attn_noalloc: null args");
  if (a->out_partials)
    return set_error(QDEC_EUNSUPPORTED,
                     "qdec_attn_noalloc: out_partials leaves the partials for a later qdec_gemm; "
                     "use qdec_attn with a caller workspace");
  size_t pb = 0, cb = 0;
  const int rc = qdec_attn_workspace(a, &pb, &cb);
  if (rc != QDEC_OK) return rc;
  if (pb > QDEC_NOALLOC_PARTIAL_BYTES || cb > QDEC_NOALLOC_COUNTER_BYTES)
    return set_error(QDEC_EINVAL,
                     "qdec_attn_noalloc: this call needs %zu B of chunk partials and %zu B of counters; the "
                     "library scratch holds %u and %u (use qdec_attn with a caller workspace)",
                     pb, cb, (unsigned)QDEC_NOALLOC_PARTIAL_BYTES, (unsigned)QDEC_NOALLOC_COUNTER_BYTES);
  unsigned char *base = nullptr;
  const int rs = scratch_on_current_device((hipStream_t)stream, &base);
  if (rs != QDEC_OK) return rs;
  qdec_attn_args b = *a;
  b.counters = reinterpret_cast<uint32_t *>(base);
  b.partial = reinterpret_cast<float *>(base + QDEC_NOALLOC_COUNTER_BYTES);
  return qdec_attn(&b, stream);
}

int qdec_layer_prepare(const qdec_layer_args *a) {
  LayerParams L;
  int w = 0;
  size_t lds = 0;
  const int rc = plan_layer(a, &L, &w, &lds);
  if (rc != QDEC_OK) return rc;
  const hipError_t e = hipMemcpy(a->plan, &L, sizeof L, hipMemcpyHostToDevice);
  if (e != hipSuccess) return set_error(QDEC_ELAUNCH, "qdec_layer_prepare: copy of the plan: %s", hipGetErrorString(e));
  return QDEC_OK;
}

int qdec_layer(const qdec_layer_args *a, qdec_stream_t stream) {
  LayerParams L;
  int w = 0;
  size_t lds = 0;
  const int rc = plan_layer(a, &L, &w, &lds);
  if (rc != QDEC_OK) return rc;
  return launch_status(launch_layer(static_cast<const LayerParams *>(a->plan), L.key, static_cast<LayerCtl *>(a->ctl),
                                    a->spin_limit ? a->spin_limit : (1u << 22), w, lds, (hipStream_t)stream),
                       "qdec_layer");
}

int qdec_ngram_draft(const qdec_draft_args *a, qdec_stream_t stream) {
  if (!a || !a->hist || !a->lens || !a->ids || !a->draft) return set_error(QDEC_EINVAL, "qdec_ngram_draft: null pointer");
  if (a->batch < 1 || a->cap < 1 || a->k < 0 || a->primary < 1 || a->backoff < 1)
    return set_error(QDEC_EINVAL, "qdec_ngram_draft: batch %d cap %d k %d primary %d backoff %d", a->batch, a->cap,
                     a->k, a->primary, a->backoff);
  return launch_status(
      launch_draft(a->hist, a->lens, a->ids, a->draft, a->batch, a->cap, a->primary, a->backoff, a->k,
                   (hipStream_t)stream),
      "qdec_ngram_draft");
}

int qdec_spec_accept(const qdec_accept_args *a, qdec_stream_t stream) {
  if (!a || !a->out_tok || !a->draft || !a->hist || !a->lens || !a->naccept)
    return set_error(QDEC_EINVAL, "qdec_spec_accept: null pointer");
  if (a->batch < 1 || a->cap < 1 || a->k < 0)
    return set_error(QDEC_EINVAL, "qdec_spec_accept: batch %d cap %d k %d", a->batch, a->cap, a->k);
  return launch_status(launch_accept(a->out_tok, a->draft, a->hist, a->lens, a->naccept, a->batch, a->cap, a->k,
                                     a->stop_len, (hipStream_t)stream),
                       "qdec_spec_accept");
}

// ------------------------------------------------------------- prefill
int qdec_rownorm(const qdec_rownorm_args *a, qdec_stream_t stream) {
  if (!a || !a->x || !a->out) return set_error(QDEC_EINVAL, "qdec_rownorm: null pointer");
  if (a->rows < 1 || a->k < 32 || a->k % 32 || a->tiles < (a->rows + 15) / 16)
    return set_error(QDEC_EINVAL, "qdec_rownorm: rows %d k %d tiles %d", a->rows, a->k, a->tiles);
  if (!aligned16(a->x) || !aligned16(a->out) || (a->norm_w && !aligned16(a->norm_w)))
    return set_error(QDEC_EALIGN, "qdec_rownorm: pointers must be 16-byte aligned");
  const hipError_t e = pnorm_fits(a->k, a->rows)
                          ? launch_pnorm(a->x, a->norm_w, a->out, a->eps, a->rows, a->k, a->tiles, (hipStream_t)stream)
                          : launch_rownorm_rows(a->x, a->norm_w, a->out, a->eps, a->rows, a->k, a->tiles,
                                                (hipStream_t)stream);
  return launch_status(e, "qdec_rownorm");
}

int qdec_prefill_gemm(const qdec_pgemm_args *a, qdec_stream_t stream) {
  if (!a || !a->x || !a->w || !a->out) return set_error(QDEC_EINVAL, "qdec_prefill_gemm: null pointer");
  const uint32_t f = a->flags;
  if (f != 0u && f != QDEC_RES_OUT && f != QDEC_GLU)
    return set_error(QDEC_EUNSUPPORTED, "qdec_prefill_gemm: flags 0x%x not supported (0, RES_OUT or GLU)", f);
  // Workgroup tile (activation rows x weight rows): 256 x 256 reads a third
  // fewer LDS bytes per MFMA than 256 x 128 but makes half the workgroups;
  // 64 x 64 makes 8x the workgroups of 256 x 128 for few rows.  Picked by
  // the launch size: 256 x 256 from 600 workgroups (at 16K rows QKV and
  // gate/up ~+10%, down +6%, O even with 640 workgroups; at 8K rows O and
  // down, 320 workgroups, are 10% faster on 256 x 128), 256 x 128 from 512,
  // else 64 x 64 (a 512-token prompt: O and down would have 40 workgroups
  // of 256 x 128) -- unless one round of large tiles fills 128-256 CUs.
  int trows = a->tile_rows, tcols = a->tile_cols;
  const bool pair_ok = (trows == 0 && tcols == 0) || (trows == 256 && (tcols == 128 || tcols == 256)) ||
                       (trows == 64 && tcols == 64);
  if (!pair_ok)
    return set_error(QDEC_EINVAL, "qdec_prefill_gemm: tile %d x %d (0 x 0, 256 x 128, 256 x 256 or 64 x 64)",
                     trows, tcols);
  // Buffers of fewer whole 256-row tiles than the call covers (a short
  // prompt padded to 64 rows) take the 64 x 64 tile only.
  const bool whole256 = a->tiles % (kPgRows / 16) == 0;
  if (trows == 0 && !whole256) trows = 64, tcols = 64;
  if (trows == 0) {
    // Workgroups of each large tile; from 600 (256 x 256) or 512 (256 x 128)
    // they run in several rounds.  Below that a large tile still pays when
    // one round of them covers half to all of the 256 CUs: the prefill of
    // one sequence on MI355X, ms (64 x 64 / chosen), gate/up 256 x 256 at
    // 512 rows 9.46 / 8.67 and at 768 rows 12.41 / 10.49, gate/up 256 x 128
    // at 256 rows 7.11 / 6.85, QKV 256 x 128 at 1024 rows 14.62 / 14.11.
    const int64_t row_tiles = a->tiles / 16;
    const int64_t w256 = a->n % 256 == 0 ? (a->n / 256) * row_tiles : 0;
    const int64_t w128 = a->n % 128 == 0 ? (a->n / 128) * row_tiles : 0;
    if (w256 >= 600 || (w256 >= 128 && w256 <= 256)) {
      trows = 256, tcols = 256;
    } else if (w128 >= 512 || (w128 >= 128 && w128 <= 256)) {
      trows = 256, tcols = 128;
    } else {
      trows = 64, tcols = 64;
    }
  }
  if (a->rows < 1 || a->k < kPgStageK || a->k % kPgStageK || a->n < tcols || a->n % tcols)
    return set_error(QDEC_EINVAL, "qdec_prefill_gemm: rows %d n %d k %d (n a multiple of %d, k of %d)", a->rows,
                     a->n, a->k, tcols, kPgStageK);
  const int gran = (trows == 64 ? kPgRowsSmall : kPgRows) / 16;
  if (a->tiles < 1 || a->tiles % gran || a->rows > a->tiles * 16)
    return set_error(QDEC_EINVAL, "qdec_prefill_gemm: tiles %d must be a multiple of %d (tile %d x %d) covering %d rows",
                     a->tiles, gran, trows, tcols, a->rows);
  if ((f & QDEC_RES_OUT) && (!a->res || a->out_frag))
    return set_error(QDEC_EUNSUPPORTED, "qdec_prefill_gemm: RES_OUT needs res and a row-major out");
  if (a->out_frag != 0 && a->out_frag != 1) return set_error(QDEC_EINVAL, "qdec_prefill_gemm: out_frag must be 0 or 1");
  if (!aligned16(a->x) || !aligned16(a->w) || !aligned16(a->out) || (a->res && !aligned16(a->res)))
    return set_error(QDEC_EALIGN, "qdec_prefill_gemm: pointers must be 16-byte aligned");
  PgemmParams p;
  p.x = reinterpret_cast<const uint16_t *>(a->x);
  p.w = reinterpret_cast<const uint16_t *>(a->w);
  p.out = reinterpret_cast<uint16_t *>(a->out);
  p.res = reinterpret_cast<const uint16_t *>(a->res);
  p.rows = a->rows;
  p.n = a->n;
  p.k = a->k;
  p.tiles = a->tiles;
  p.ofrag = a->out_frag;
  const bool glu = (f & QDEC_GLU) != 0;
  p.n_out = glu ? a->n / 2 : a->n;
  p.up_tiles = a->n / 32;
  p.tile_rows = trows;
  p.tile_cols = tcols;
  p.wg_n = glu ? (a->n / 2) / (tcols / 2) : a->n / tcols;
  return launch_status(launch_pgemm(p, f, (hipStream_t)stream), "qdec_prefill_gemm");
}

int qdec_prefill_qk(const qdec_prefill_qk_args *a, qdec_stream_t stream) {
  if (!a || !a->qkv || !a->q_norm_w || !a->k_norm_w || !a->cos_tab || !a->sin_tab || !a->k_cache || !a->v_cache)
    return set_error(QDEC_EINVAL, "qdec_prefill_qk: null pointer");
  if (a->head_dim != 128 || a->nq < 1 || a->nkv < 1 || a->nq + a->nkv > kPqMaxHeads)
    return set_error(QDEC_EUNSUPPORTED, "qdec_prefill_qk: head_dim %d nq %d nkv %d (head_dim 128, nq + nkv <= %d)",
                     a->head_dim, a->nq, a->nkv, kPqMaxHeads);
  if (a->batch < 1 || a->t_rows < 1 || a->pos0 < 0 || a->cap < 32 || a->cap % 32 || a->pos0 + a->t_rows > a->cap)
    return set_error(QDEC_EINVAL, "qdec_prefill_qk: batch %d t_rows %d pos0 %d cap %d", a->batch, a->t_rows, a->pos0,
                     a->cap);
  if (!aligned16(a->qkv) || !aligned16(a->k_cache) || !aligned16(a->v_cache))
    return set_error(QDEC_EALIGN, "qdec_prefill_qk: qkv and caches must be 16-byte aligned");
  PqkParams p;
  p.qkv = reinterpret_cast<uint16_t *>(a->qkv);
  p.q_norm_w = reinterpret_cast<const uint16_t *>(a->q_norm_w);
  p.k_norm_w = reinterpret_cast<const uint16_t *>(a->k_norm_w);
  p.cos_tab = reinterpret_cast<const uint16_t *>(a->cos_tab);
  p.sin_tab = reinterpret_cast<const uint16_t *>(a->sin_tab);
  p.k_cache = reinterpret_cast<uint16_t *>(a->k_cache);
  p.v_cache = reinterpret_cast<uint16_t *>(a->v_cache);
  p.eps = a->eps;
  p.batch = a->batch;
  p.t_rows = a->t_rows;
  p.pos0 = a->pos0;
  p.nq = a->nq;
  p.nkv = a->nkv;
  p.cap = a->cap;
  return launch_status(launch_prefill_qk(p, (hipStream_t)stream), "qdec_prefill_qk");
}

int qdec_prefill_attn(const qdec_prefill_attn_args *a, qdec_stream_t stream) {
  if (!a || !a->qkv || !a->k_cache || !a->v_cache || !a->out) return set_error(QDEC_EINVAL, "qdec_prefill_attn: null pointer");
  if (a->head_dim != 128 || a->nkv < 1 || a->nq % a->nkv ||
      (a->nq / a->nkv != 2 && a->nq / a->nkv != 4 && a->nq / a->nkv != 8))
    return set_error(QDEC_EUNSUPPORTED, "qdec_prefill_attn: head_dim %d nq %d nkv %d (head_dim 128; 2, 4 or 8 query heads per kv head)",
                     a->head_dim, a->nq, a->nkv);
  if (a->batch < 1 || a->t_rows < 1 || a->pos0 < 0 || a->cap < 32 || a->cap % 32 || a->pos0 + a->t_rows > a->cap)
    return set_error(QDEC_EINVAL, "qdec_prefill_attn: batch %d t_rows %d pos0 %d cap %d", a->batch, a->t_rows,
                     a->pos0, a->cap);
  const int64_t rows = (int64_t)a->batch * a->t_rows;
  if (a->tiles < (rows + 15) / 16) return set_error(QDEC_EINVAL, "qdec_prefill_attn: tiles %d < rows %lld / 16", a->tiles, (long long)rows);
  if (!aligned16(a->qkv) || !aligned16(a->k_cache) || !aligned16(a->v_cache) || !aligned16(a->out))
    return set_error(QDEC_EALIGN, "qdec_prefill_attn: pointers must be 16-byte aligned");
  PattnParams p;
  p.qkv = reinterpret_cast<const uint16_t *>(a->qkv);
  p.k_cache = reinterpret_cast<const uint16_t *>(a->k_cache);
  p.v_cache = reinterpret_cast<const uint16_t *>(a->v_cache);
  p.out = reinterpret_cast<uint16_t *>(a->out);
  p.scale_log2 = a->sm_scale * 1.4426950408889634f;
  p.batch = a->batch;
  p.t_rows = a->t_rows;
  p.pos0 = a->pos0;
  p.nq = a->nq;
  p.nkv = a->nkv;
  p.cap = a->cap;
  p.tiles = a->tiles;
  return launch_status(launch_prefill_attn(p, (hipStream_t)stream), "qdec_prefill_attn");
}

}  // extern "C"
