// Weight-streaming skinny GEMM for the decode step: y = x' . W^T, 1..64 rows.
//
// One workgroup owns one 16-column output tile (or several, for the lm_head)
// and a contiguous k range; its waves split that range into equal contiguous
// pieces.  Each wave streams its part of the tiled weight -- one 1 KiB block
// per k step, one 16-byte load per lane -- straight into the A operand of
// v_mfma_f32_16x16x32_bf16, while the activations (normalised on the way in
// when NORM_IN) are staged in LDS and read as the B operand.  The product is
// computed transposed (y^T = W . x'^T), so a lane ends up holding 4
// consecutive output columns of one row.
//
// Two ways of streaming the weights:
//  * window (up to 16 rows, the workgroup's whole k range of x in LDS): a
//    ring of RW weight registers per wave.  The block consumed at ring slot r
//    is immediately replaced by the block RW steps further along the wave's
//    sequence (k steps of its tile, then of its next tile), so RW loads stay
//    in flight from the first MFMA to the last and the stream never drains
//    between passes or tiles.  RW divides the wave's k steps per tile, which
//    keeps slot r on k step r (mod RW) in every tile.
//  * passes (everything else): up to 20 blocks per wave per pass, activations
//    staged per pass when the whole range does not fit LDS.
// In both, the activations are loaded before the first weights: they are
// cache hits, and the statistics and LDS staging computed from them overlap
// the weight stream (loads complete in issue order).
//
// Summation order of an output element: MFMA chain over the wave's k steps in
// increasing order, then waves 0..W-1 added in order, then k splits 0..S-1
// added in order by the workgroup that arrives last.  The RMSNorm statistic
// of a row is summed by thread t over the row's 16-byte vectors t, t+T, ...
// and then across lanes and waves in a fixed tree, whatever the path.  None
// of it depends on the number of rows, which is what lets a verify pass over
// B*T rows reproduce the plain B-row step bit for bit.  (The path is chosen
// per role from (n, k) and the row count's M tiles; rows 1..16 share one.)
//
// Reference behaviour replaced: engine/kernels/fused.py:33-235 (_gemv_kernel,
// _gemv_vec_kernel, _gemv_splitk_kernel + reduce) and the lm_head + argmax of
// engine/engine.py:492-498, 542-545.
//
// The body takes its workgroup index and count as arguments, so that the
// per-operation launches (gemm.hip) and the one-layer-per-launch kernel
// (layer.hip) run the same code.
#pragma once
#include "qdec_common.h"
#include "qdec_kernels.h"

namespace qdec {

// Weight blocks are read once per step and never reused within it: load them
// with the non-temporal hint so they stream past the caches that hold the
// activations (measured: 6% off a batch-1 decode step on MI355X).
__device__ __forceinline__ uint4 ldw(const uint4 *p) { return ld_nt(p); }

namespace {

// Weight registers a wave holds per pass: 20 blocks, or 2 x 10 with GLU.
constexpr int kWbuf = 20;
static_assert(kGemmKpMax == kWbuf && 2 * kGemmKpMaxGlu == kWbuf, "pass register budget");

// Activations from registers: up to kFastRows rows (kFastRowsNorm under
// NORM_IN, in a separate instantiation), 2 vectors per thread per row.
constexpr int kFastRows = 4;
constexpr int kFastRowsNorm = 8;
constexpr int kFastVec = 2;

// Sum one fp32 value per thread of the workgroup for up to 8 rows in a fixed
// order (lane tree, then waves in order); thread m < nrows gets row m's total.
__device__ __forceinline__ void block_row_sums(float (&ss)[8], float *s_red, int nrows, float *dst_rstd, int m0,
                                               int k, float eps) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, tid = threadIdx.x;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float v = wave_sum(ss[j]);
    if (lane == 0) s_red[wave * 8 + j] = v;
  }
  __syncthreads();
  if (tid < 8 && tid < nrows) {
    float t = 0.f;
    for (int w2 = 0; w2 < (int)(blockDim.x >> 6); ++w2) t += s_red[w2 * 8 + tid];
    dst_rstd[m0 + tid] = 1.0f / sqrtf(t / (float)k + eps);
  }
  __syncthreads();
}

// Activation vector (8 consecutive elements from k index kk) of row m,
// merged from the attention chunk partials the previous launch left with
// out_partials (attn_dev.h: per (sequence, kv head, chunk) acc [R][128],
// max [R], sum [R], R = t_rows * 4).  The same operations in the same order
// as the attention's own chunk merge, so the bf16 result is bit-identical
// to the output that call would have written.
template <bool COH>
__device__ __forceinline__ uint4 attn_merge8(const GemmParams &p, int m, int kk) {
  constexpr int D = 128, G = 4, CB = 8;
  const int T = p.a_t_rows, R = T * G;
  const int b = m / T, t = m - b * T;
  const int h = kk / D, d0 = kk - h * D;
  const int kvh = h / G;
  const int r = t * G + (h - kvh * G);
  const size_t cstride = (size_t)R * (D + 2);
  const float *part_b = p.apart + ((size_t)b * p.a_nkv + kvh) * p.a_nchunks * cstride;
  const int L = p.alens[b];
  // A length the attention rejected (it wrote no partials) gives NaN, never
  // a merge of stale partials; the NaN reaches the argmax, whose pick is
  // then an out-of-vocabulary id the host refuses.
  if (L < 0 || L + T - 1 >= p.a_cap) return make_uint4(0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u);
  const int n_active = min((L + T - 1) / p.a_chunk + 1, p.a_nchunks);
  const float NEG_INF = -__builtin_huge_valf();
  float mc[CB], lc[CB];
  f32x4_t a0[CB], a1[CB];
  auto load_group = [&](int cc) {
#pragma unroll
    for (int j = 0; j < CB; ++j) {
      const float *pr = part_b + (size_t)min(cc + j, n_active - 1) * cstride;
      mc[j] = ldf<COH>(pr + (size_t)R * D + r);
      lc[j] = ldf<COH>(pr + (size_t)R * D + R + r);
      a0[j] = ldf4<COH>(pr + (size_t)r * D + d0);
      a1[j] = ldf4<COH>(pr + (size_t)r * D + d0 + 4);
    }
  };
  load_group(0);
  float mmax = NEG_INF;
#pragma unroll
  for (int j = 0; j < CB; ++j)
    if (j < n_active) mmax = fmaxf(mmax, mc[j]);
  for (int cc = CB; cc < n_active; cc += CB) {
    float mg[CB];
#pragma unroll
    for (int j = 0; j < CB; ++j) mg[j] = ldf<COH>(part_b + (size_t)min(cc + j, n_active - 1) * cstride + (size_t)R * D + r);
#pragma unroll
    for (int j = 0; j < CB; ++j)
      if (cc + j < n_active) mmax = fmaxf(mmax, mg[j]);
  }
  float lsum = 0.f;
  f32x4_t o0 = f32x4_t{0.f, 0.f, 0.f, 0.f}, o1 = f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (int cc = 0; cc < n_active; cc += CB) {
    if (cc > 0) load_group(cc);
#pragma unroll
    for (int j = 0; j < CB; ++j) {
      if (cc + j >= n_active || mc[j] == NEG_INF) continue;
      const float w = exp2f(mc[j] - mmax);
      lsum += lc[j] * w;
      o0 += a0[j] * w;
      o1 += a1[j] * w;
    }
  }
  uint4 v;
  v.x = pack2(o0[0] / lsum, o0[1] / lsum);
  v.y = pack2(o0[2] / lsum, o0[3] / lsum);
  v.z = pack2(o1[0] / lsum, o1[1] / lsum);
  v.w = pack2(o1[2] / lsum, o1[3] / lsum);
  return v;
}

// Residual vector (8 consecutive elements from k index kk) of row m with a
// pending split update applied: bf16(x + bf16(((p0 + p1) + p2) + ...)), the
// rounding of the RES_OUT epilogue, over the partials a split producer left
// in p.xparts ([j][rows][k] fp32).
__device__ __forceinline__ uint4 merge_res8(const float *__restrict__ parts, int nparts, int rows, int k, uint4 xv,
                                            int m, int kk) {
  const float *q = parts + (size_t)m * k + kk;
  const size_t stride = (size_t)rows * k;
  f32x4_t s0 = *reinterpret_cast<const f32x4_t *>(q), s1 = *reinterpret_cast<const f32x4_t *>(q + 4);
  for (int j = 1; j < nparts; ++j) {
    s0 += *reinterpret_cast<const f32x4_t *>(q + j * stride);
    s1 += *reinterpret_cast<const f32x4_t *>(q + j * stride + 4);
  }
  uint4 o;
  o.x = pack2(lo16(xv.x) + rbf(s0[0]), hi16(xv.x) + rbf(s0[1]));
  o.y = pack2(lo16(xv.y) + rbf(s0[2]), hi16(xv.y) + rbf(s0[3]));
  o.z = pack2(lo16(xv.z) + rbf(s1[0]), hi16(xv.z) + rbf(s1[1]));
  o.w = pack2(lo16(xv.w) + rbf(s1[2]), hi16(xv.w) + rbf(s1[3]));
  return o;
}

// Pending split residual updates merged from registers (one row): at most
// this many partials (the down projection leaves four).
constexpr int kMergeParts = 4;

// XP: the instantiation that merges a pending split residual update into its
// one register-staged row (FR = 1); 0 elsewhere.
// TW: output tiles per wave on the direct path.  Each activation fragment a
// wave loads then feeds TW tiles' MFMAs, so from two M tiles the activation
// reads per weight byte halve at TW = 2 and the ring's registers go to
// weights instead (a tile's sums are the same whatever TW is).
// COH: activations and outputs at device scope (ldv16 and friends), for a
// body that shares its launch with the workgroups that produce or consume them.
template <int MT, uint32_t FLAGS, int RW, bool XD, int FR = kFastRows, bool XP = false, int TW = 1, bool COH = false>
__device__ __forceinline__ void gemm_body(const GemmParams p, const int blk, const int nblk,
                                          unsigned char *__restrict__ smem) {
  constexpr bool NORM = (FLAGS & QDEC_NORM_IN) != 0;
  constexpr bool GLU = (FLAGS & QDEC_GLU) != 0;
  constexpr bool RES = (FLAGS & QDEC_RES_OUT) != 0;
  constexpr bool ARG = (FLAGS & QDEC_ARGMAX) != 0;
  constexpr int NACC = GLU ? 2 : 1;
  static_assert(TW == 1 || XD, "several tiles per wave: direct path only");
  // Weight streams and accumulators per wave: tile tw's gate (or only)
  // stream at tw * NACC, its up stream at tw * NACC + 1.
  constexpr int NA = NACC * TW;
  constexpr bool WIN = RW > 0;
  static_assert(!WIN || MT == 1 || XD, "LDS-staged windows serve one M tile");
  static_assert(!XD || (WIN && !NORM), "direct activations: window path, x already normalised");
  constexpr int NB = WIN ? RW : (GLU ? kGemmKpMaxGlu : kGemmKpMax);  // weight registers per accumulator

  float *s_rstd = reinterpret_cast<float *>(smem);              // [64]
  uint32_t *s_flag = reinterpret_cast<uint32_t *>(smem + 256);  // [4]
  float *s_red = reinterpret_cast<float *>(smem + 272);         // [64 floats]
  uint16_t *s_x = reinterpret_cast<uint16_t *>(smem + p.lds_x_off);  // [rows][xstride]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nthr = blockDim.x;
  const int nw = nthr >> 6;
  const int rows = p.rows;
  const int col = lane & 15;  // row of x inside an M tile
  const int grp = lane >> 4;  // k group / output column group

  const int tg = blk / p.ksplit;                // tile group
  const int split = blk - tg * p.ksplit;
  const int ks_wg = split * (p.KS / p.ksplit);  // first k step of this workgroup
  const int ks_wave = ks_wg + wave * p.ksw;     // first k step of this wave
  const int xstride = p.xstride;
  const uint4 *__restrict__ W = reinterpret_cast<const uint4 *>(p.w);
  const uint16_t *__restrict__ X = reinterpret_cast<const uint16_t *>(p.x);
  const size_t up_off = (size_t)p.up_tiles * p.KS * 64;
  const int tile0 = tg * p.tiles_per_wg;

  // RES_OUT with one tile and no k split: wave 0 loads its residual values
  // first, so the epilogue does not wait on a dependent load after the last
  // MFMA (the residual was written by an earlier launch).
  const bool res_early = RES && p.tiles_per_wg == 1 && p.ksplit == 1;
  uint2 res_v[MT];
  if constexpr (RES) {
    if (res_early && wave == 0) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = mt * 16 + col;
        res_v[mt] = ldv8<COH>(reinterpret_cast<const uint16_t *>(p.res) +
                                                     (size_t)(m < rows ? m : 0) * p.n + tile0 * 16 + grp * 4);
      }
    }
  }

  uint4 wb[NA][NB];
  // Direct activations: the B fragment of ring slot r, loaded from global
  // (cache-resident x) right behind the slot's weight block.
  uint4 xb[XD ? MT : 1][XD ? NB : 1];
  const bool xrow_ok = col < rows;  // lanes past the last row read row 0 and use zeros
  // Row mt*16 + col of x at the wave's first k step; with p.xt the
  // normalisation pre-pass wrote x in fragment order (k step, M tile, lane),
  // so a fragment load is one contiguous KiB instead of 16 row pieces.
  const uint16_t *xg[MT];
  const int xkstep = p.xt ? p.xt * 512 : 32;  // elements between k steps
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + col;
    xg[mt] = p.xt ? X + ((size_t)ks_wave * p.xt + mt) * 512 + lane * 8
                  : X + (size_t)(m < rows ? m : 0) * p.k + (size_t)ks_wave * 32 + grp * 8;
  }
  // Weight block of k step i (relative to the wave's range) of `tile`.
  auto wptr = [&](int tile, int i) { return W + ((size_t)tile * p.KS + ks_wave + i) * 64 + lane; };
  const size_t tstride = (size_t)p.KS * 64;  // between consecutive tiles' blocks
  // Passes: straight-line loads of one pass; indices past the pass are clamped
  // to its last block (a redundant, cache-served load) instead of branched
  // around, so all of them stay in flight together.
  auto issue_pass = [&](int tile, int kbeg, int kcnt) {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const uint4 *q = wptr(tile, kbeg + min(i, kcnt - 1));
      wb[0][i] = ldw(q);
      if constexpr (GLU) wb[1][i] = ldw(q + up_off);
    }
  };
  // Window: the first RW k steps of the first tile (RW divides ksw).
  auto issue_first = [&]() {
    if constexpr (WIN) {
      const uint4 *q = wptr(tile0, 0);
#pragma unroll
      for (int r = 0; r < NB; ++r) {
        const int rr = min(r, p.ksw - 1);  // a range shorter than the ring repeats its last block
#pragma unroll
        for (int tw = 0; tw < TW; ++tw) {
          wb[tw * NACC][r] = ldw(q + tw * tstride + rr * 64);
          if constexpr (GLU) wb[tw * NACC + 1][r] = ldw(q + tw * tstride + rr * 64 + up_off);
        }
        if constexpr (XD) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            xb[mt][r] = ldv16<COH>(xg[mt] + (size_t)min(r, p.ksw - 1) * xkstep);
        }
      }
    } else {
      issue_pass(tile0, 0, min(p.kp, p.ksw));
    }
  };

  // ---- activations.
  const int lds_steps = p.lds_all ? p.ksw : p.kp;  // LDS columns per wave
  bool staged = false;
  if constexpr (XD) {
    issue_first();
  } else if (p.xfast) {
    // Row m, vectors vr = tid + j*nthr of the workgroup's k range (per_row
    // of them), loaded into registers before the first weights.  (Attention
    // partials are merged before the weights go out too: loads complete in
    // issue order, so weights issued first would hold the merge back until
    // they had all arrived -- O at batch 1 measured 9.3 against 8.3 us.)
    const int per_row = p.ksw * nw * 4;
    const bool merge = !XD && !NORM && p.amerge;
    uint4 xr[FR][kFastVec];
    // NORM_IN without GLU: this thread's norm-weight vectors, loaded with x
    // (gate/up reads them after the weights instead: 8 more registers would
    // cost it its third wave per SIMD).
    constexpr bool NPRE = NORM && !GLU;
    uint4 nr[NPRE ? kFastVec : 1];
#pragma unroll
    for (int j = 0; j < (NPRE ? kFastVec : 1); ++j) {
      const int vr = tid + j * nthr;
      nr[j] = (NPRE && vr < per_row)
                  ? *reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(p.norm_w) + ks_wg * 32 + 8 * vr)
                  : zero4();
    }
#pragma unroll
    for (int m = 0; m < FR; ++m)
#pragma unroll
      for (int j = 0; j < kFastVec; ++j) {
        const int vr = tid + j * nthr;
        const bool ok = m < rows && vr < per_row;
        const int mm = ok ? m : 0, vv = ok ? vr : 0;
        if (merge) {
          xr[m][j] = ok ? attn_merge8<COH>(p, mm, ks_wg * 32 + 8 * vv) : zero4();
        } else {
          const uint4 v = ldv16<COH>(X + (size_t)mm * p.k + ks_wg * 32 + 8 * vv);
          xr[m][j] = ok ? v : zero4();
        }
      }
    // XP: the raw partials of the pending residual update are loaded with x,
    // before the weights, and merged after the weights went out (loads
    // complete in issue order: merging first would hold the weights back).
    f32x4_t xp[XP ? kFastVec : 1][XP ? kMergeParts : 1][2];
    if constexpr (XP) {
      static_assert(FR == 1 && NORM && !GLU, "one row, NORM_IN without GLU");
#pragma unroll
      for (int j = 0; j < kFastVec; ++j) {
        const int vr = tid + j * nthr;
        const float *q = p.xparts + ks_wg * 32 + 8 * (vr < per_row ? vr : 0);
#pragma unroll
        for (int part = 0; part < kMergeParts; ++part) {
          const bool live = vr < per_row && part < p.xnparts;
          const float *qp = q + (size_t)(live ? part : 0) * p.k;  // rows == 1: part stride is k
          xp[j][part][0] = *reinterpret_cast<const f32x4_t *>(qp);
          xp[j][part][1] = *reinterpret_cast<const f32x4_t *>(qp + 4);
        }
      }
    }
    issue_first();
    if constexpr (XP) {
      // bf16(x + bf16(((p0 + p1) + p2) + p3)): merge_res8's order and rounding.
#pragma unroll
      for (int j = 0; j < kFastVec; ++j) {
        const int vr = tid + j * nthr;
        if (vr < per_row) {
          f32x4_t s0 = xp[j][0][0], s1 = xp[j][0][1];
#pragma unroll
          for (int part = 1; part < kMergeParts; ++part)
            if (part < p.xnparts) {
              s0 += xp[j][part][0];
              s1 += xp[j][part][1];
            }
          const uint4 xv = xr[0][j];
          uint4 o;
          o.x = pack2(lo16(xv.x) + rbf(s0[0]), hi16(xv.x) + rbf(s0[1]));
          o.y = pack2(lo16(xv.y) + rbf(s0[2]), hi16(xv.y) + rbf(s0[3]));
          o.z = pack2(lo16(xv.z) + rbf(s1[0]), hi16(xv.z) + rbf(s1[1]));
          o.w = pack2(lo16(xv.w) + rbf(s1[2]), hi16(xv.w) + rbf(s1[3]));
          xr[0][j] = o;
          // the first workgroup (its range is the whole row: ksplit 1) keeps it
          if (blk == 0) *reinterpret_cast<uint4 *>(p.xmerged + ks_wg * 32 + 8 * vr) = o;
        }
      }
    }
    if constexpr (NORM) {
      float ss[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) ss[j] = 0.f;
#pragma unroll
      for (int m = 0; m < FR; ++m)
#pragma unroll
        for (int j = 0; j < kFastVec; ++j) {
          float f[8];
          unpack8(xr[m][j], f);
#pragma unroll
          for (int e = 0; e < 8; ++e) ss[m] += f[e] * f[e];
        }
      block_row_sums(ss, s_red, rows, s_rstd, 0, p.k, p.eps);
    }
#pragma unroll
    for (int m = 0; m < FR; ++m)
#pragma unroll
      for (int j = 0; j < kFastVec; ++j) {
        const int vr = tid + j * nthr;
        if (m < rows && vr < per_row) {
          uint4 xv = xr[m][j];
          if constexpr (NPRE)
            xv = norm8(xv, nr[j], s_rstd[m]);
          else if constexpr (NORM)
            xv = norm8(xv, *reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(p.norm_w) + ks_wg * 32 + 8 * vr),
                       s_rstd[m]);
          *reinterpret_cast<uint4 *>(s_x + (size_t)m * xstride + 8 * vr) = xv;
        }
      }
    __syncthreads();
    staged = true;
  } else {
    issue_first();
    if constexpr (NORM) {
      // Whole-row statistics, same per-thread vector assignment and order.
      const int nvec = p.k >> 3;
      for (int m0 = 0; m0 < rows; m0 += 8) {
        float ss[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) ss[j] = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int m = m0 + j;
          if (m < rows) {
            const uint16_t *xrow = X + (size_t)m * p.k;
            for (int v = tid; v < nvec; v += nthr) {
              float f[8];
              unpack8(ldv16<COH>(xrow + 8 * v), f);
#pragma unroll
              for (int e = 0; e < 8; ++e) ss[j] += f[e] * f[e];
            }
          }
        }
        block_row_sums(ss, s_red, rows - m0, s_rstd, m0, p.k, p.eps);
      }
    }
    if (p.lds_all) {
      // The whole k range of the workgroup fits in LDS: stage it once.
      const int per_row = nw * p.ksw * 4;  // 16-byte vectors per row
      const int tot = rows * per_row;
      for (int v = tid; v < tot; v += nthr) {
        const int m = v / per_row;
        const int vr = v - m * per_row;
        const int kg = ks_wg * 32 + 8 * vr;
        uint4 xv = ldv16<COH>(X + (size_t)m * p.k + kg);
        if constexpr (NORM)
          xv = norm8(xv, *reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(p.norm_w) + kg), s_rstd[m]);
        *reinterpret_cast<uint4 *>(s_x + (size_t)m * xstride + 8 * vr) = xv;
      }
      __syncthreads();
      staged = true;
    }
  }

  // ARGMAX running best per M tile (lane-local, rows = mt*16 + col).
  float best_v[MT];
  int best_i[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    best_v[mt] = -__builtin_huge_valf();
    best_i[mt] = 0x7fffffff;
  }

  bool have_w = true;  // wb holds the next pass's weights already (pass path)
  for (int tt = 0; tt < p.tiles_per_wg; tt += TW) {
    const int tile = tile0 + tt;  // this wave's tiles: tile .. tile + TW - 1
    f32x4_t acc[NA][MT];
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[a][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    if constexpr (WIN) {
      // B operand rows: lane col < rows reads its row, the others read row 0
      // and use zeros.
      const uint16_t *xs = s_x + (size_t)(xrow_ok ? col : 0) * xstride + wave * p.ksw * 32 + grp * 8;
      const bool more_tiles = tt + TW < p.tiles_per_wg;
      if constexpr (!XD) {
        // Slot r always holds k step r (mod RW): refill with k step i + RW of
        // this tile while it exists, else the same offset into the next tile;
        // none past the last tile.  The chunk's LDS reads are all issued
        // before its first MFMA, so their latency is paid once per chunk.
        for (int i0 = 0; i0 < p.ksw; i0 += RW) {
          const bool same_tile = i0 + RW < p.ksw;
          const bool refill = same_tile || more_tiles;
          const uint4 *qn = same_tile ? wptr(tile, i0 + RW) : wptr(tile + 1, i0 + RW - p.ksw);
          uint4 bq[RW];
#pragma unroll
          for (int r = 0; r < RW; ++r) {
            const uint4 bx = *reinterpret_cast<const uint4 *>(xs + (i0 + r) * 32);
            bq[r] = xrow_ok ? bx : zero4();
          }
#pragma unroll
          for (int r = 0; r < RW; ++r) {
#pragma unroll
            for (int a = 0; a < NACC; ++a) acc[a][0] = mfma16x16x32(wb[a][r], bq[r], acc[a][0]);
            if (refill) {
              wb[0][r] = ldw(qn + r * 64);
              if constexpr (GLU) wb[1][r] = ldw(qn + r * 64 + up_off);
            }
          }
        }
      } else {
        // Direct activations: the same ring, and a ragged last chunk when RW
        // does not divide the range (one group of TW tiles per workgroup
        // then).  Every tile spans the same k range of x.
        for (int i0 = 0; i0 < p.ksw; i0 += RW) {
          const bool same_tile = i0 + RW < p.ksw;
          const uint4 *qn = same_tile ? wptr(tile, i0 + RW) : wptr(tile + TW, i0 + RW - p.ksw);
#pragma unroll
          for (int r = 0; r < RW; ++r) {
            const int i = i0 + r;
            if (i < p.ksw) {
#pragma unroll
              for (int mt = 0; mt < MT; ++mt) {
                const uint4 b = (mt * 16 + col < rows) ? xb[mt][r] : zero4();
#pragma unroll
                for (int a = 0; a < NA; ++a) acc[a][mt] = mfma16x16x32(wb[a][r], b, acc[a][mt]);
              }
              if (i + RW < p.ksw || (!same_tile && more_tiles)) {
#pragma unroll
                for (int tw = 0; tw < TW; ++tw) {
                  wb[tw * NACC][r] = ldw(qn + tw * tstride + r * 64);
                  if constexpr (GLU) wb[tw * NACC + 1][r] = ldw(qn + tw * tstride + r * 64 + up_off);
                }
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                  xb[mt][r] = ldv16<COH>(xg[mt] + (size_t)((i + RW) % p.ksw) * xkstep);
              }
            }
          }
        }
      }
    } else {
      for (int pass = 0; pass < p.npass; ++pass) {
        const int kbeg = pass * p.kp;
        const int kcnt = min(p.kp, p.ksw - kbeg);
        if (!have_w) issue_pass(tile, kbeg, kcnt);
        have_w = false;
        if (!staged) {
          if (pass > 0 || tt > 0) __syncthreads();  // previous readers are done
          const int per_row = nw * kcnt * 4;        // 16-byte vectors per row in this pass
          const int tot = rows * per_row;
          for (int v = tid; v < tot; v += nthr) {
            const int m = v / per_row;
            int r = v - m * per_row;
            const int w2 = r / (kcnt * 4);
            r -= w2 * (kcnt * 4);
            const int i = r >> 2;
            const int q = r & 3;
            const int kg = (ks_wg + w2 * p.ksw + kbeg + i) * 32 + q * 8;
            uint4 xv = ldv16<COH>(X + (size_t)m * p.k + kg);
            if constexpr (NORM)
              xv = norm8(xv, *reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(p.norm_w) + kg),
                         s_rstd[m]);
            *reinterpret_cast<uint4 *>(s_x + (size_t)m * xstride + (w2 * p.kp + i) * 32 + q * 8) = xv;
          }
          __syncthreads();
          staged = p.npass == 1;  // several passes restage per pass
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) {
          if (i < kcnt) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
              const int m = mt * 16 + col;
              uint4 b = zero4();
              if (m < rows)
                b = *reinterpret_cast<const uint4 *>(s_x + (size_t)m * xstride +
                                                     (wave * lds_steps + (p.lds_all ? kbeg : 0) + i) * 32 + grp * 8);
#pragma unroll
              for (int a = 0; a < NACC; ++a) acc[a][mt] = mfma16x16x32(wb[a][i], b, acc[a][mt]);
            }
          }
        }
      }
      // Request the next tile's weights before this tile's epilogue.
      if (p.npass == 1 && tt + 1 < p.tiles_per_wg) {
        issue_pass(tile + 1, 0, min(p.kp, p.ksw));
        have_w = true;
      }
    }

    // ---- merge the waves of the workgroup in wave order.
    if (nw > 1) {
      __syncthreads();
      float4 *red = reinterpret_cast<float4 *>(smem + p.lds_red_off);
      if (wave > 0) {
#pragma unroll
        for (int a = 0; a < NA; ++a)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            red[(((wave - 1) * NA + a) * MT + mt) * 64 + lane] =
                make_float4(acc[a][mt][0], acc[a][mt][1], acc[a][mt][2], acc[a][mt][3]);
      }
      __syncthreads();
      if (wave == 0) {
        for (int w2 = 1; w2 < nw; ++w2) {
#pragma unroll
          for (int a = 0; a < NA; ++a)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
              const float4 r = red[(((w2 - 1) * NA + a) * MT + mt) * 64 + lane];
              acc[a][mt][0] += r.x;
              acc[a][mt][1] += r.y;
              acc[a][mt][2] += r.z;
              acc[a][mt][3] += r.w;
            }
        }
      }
    }

    auto out_at = [&](int m, int n) {
      uint16_t *o = reinterpret_cast<uint16_t *>(p.out);
      return p.ofrag ? o + frag_off(m, n, p.ofrag) : o + (size_t)m * p.n + n;
    };
#pragma unroll
    for (int tw = 0; tw < TW; ++tw) {
      const int ct = tile + tw;           // output tile
      const int n0 = ct * 16 + grp * 4;   // first of this lane's 4 output columns

      // ---- k split left to the next NORM_IN call: raw partials, no epilogue.
      if (RES && p.parts_out) {
        if (wave == 0) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const int m = mt * 16 + col;
            if (m < rows)
              *reinterpret_cast<f32x4_t *>(p.parts_out + ((size_t)split * rows + m) * p.n + n0) = acc[tw * NACC][mt];
          }
        }
        continue;
      }
      // ---- k split across workgroups: partials, last arrival sums them.
      if (p.ksplit > 1) {
        if (wave == 0) {
#pragma unroll
          for (int a = 0; a < NACC; ++a)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
              const int m = mt * 16 + col;
              if (m < rows)
                store_coherent4(p.partial + ((size_t)(a * p.ksplit + split) * rows + m) * p.n + n0, acc[tw * NACC + a][mt]);
            }
        }
        // Not the last split of this tile: go on with the next tile.
        if (!arrive_last(p.counters + ct, (uint32_t)p.ksplit, s_flag)) continue;
        if (wave == 0) {
#pragma unroll
          for (int a = 0; a < NACC; ++a)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
              const int m = mt * 16 + col;
              if (m < rows) {
                f32x4_t t = load_coherent4(p.partial + ((size_t)(a * p.ksplit) * rows + m) * p.n + n0);
                for (int s = 1; s < p.ksplit; ++s)
                  t += load_coherent4(p.partial + ((size_t)(a * p.ksplit + s) * rows + m) * p.n + n0);
                acc[tw * NACC + a][mt] = t;
              }
            }
        }
      }

      // ---- epilogues (wave 0 holds the finished tile).
      if (wave == 0) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int m = mt * 16 + col;
          if (m >= rows) continue;
          const f32x4_t g4 = acc[tw * NACC][mt];
          if constexpr (ARG) {
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = rbf(g4[i]);
            if (p.out) {
              uint2 o;
              o.x = pack2(v[0], v[1]);
              o.y = pack2(v[2], v[3]);
              *reinterpret_cast<uint2 *>(reinterpret_cast<uint16_t *>(p.out) + (size_t)m * p.n + n0) = o;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (v[i] > best_v[mt]) {
                best_v[mt] = v[i];
                best_i[mt] = n0 + i;
              }
          } else if constexpr (RES) {
            uint16_t *rp = reinterpret_cast<uint16_t *>(p.res) + (size_t)m * p.n + n0;
            const uint2 r = res_early ? res_v[mt] : ldv8<COH>(rp);
            uint2 o;
            o.x = pack2(lo16(r.x) + rbf(g4[0]), hi16(r.x) + rbf(g4[1]));
            o.y = pack2(lo16(r.y) + rbf(g4[2]), hi16(r.y) + rbf(g4[3]));
            stv8<COH>(rp, o);
          } else if constexpr (GLU) {
            const f32x4_t u4 = acc[tw * NACC + 1][mt];
            float o4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float g = rbf(g4[i]);
              const float u = rbf(u4[i]);
              const float sg = rbf(g / (1.0f + expf(-g)));
              o4[i] = sg * u;
            }
            uint2 o;
            o.x = pack2(o4[0], o4[1]);
            o.y = pack2(o4[2], o4[3]);
            stv8<COH>(out_at(m, n0), o);
          } else {
            uint2 o;
            o.x = pack2(g4[0], g4[1]);
            o.y = pack2(g4[2], g4[3]);
            stv8<COH>(out_at(m, n0), o);
          }
        }
      }
    }
  }

  if constexpr (ARG) {
    // Each row's best over the workgroup's 4 column groups (lowest index on
    // equal values) as a 64-bit key (argmax_key: the maximum key is the
    // argmax), then the row maxima over all workgroups:
    //  * one row: every workgroup stores its key in the partial workspace
    //    and the workgroup that arrives last scans them;
    //  * more rows: every workgroup folds its keys into kArgSlots keys per
    //    row (slot = workgroup mod kArgSlots, so concurrent workgroups do not
    //    queue on one address) with device-scope atomic max, kept in the
    //    counters workspace after the arrival counter and zero between
    //    calls; the last arriver takes the maximum of each row's slots (a
    //    scan of rows x workgroups partials would be one serial pass per
    //    row: 72 us of the lm_head's 213 at 32 rows on MI355X; the atomics
    //    cost 9 us at one row against the scan's 1).
    static_assert(kArgSlots == 16, "one 16-lane row of slots per row");
    uint64_t *keys = reinterpret_cast<uint64_t *>(p.counters + 2);  // [rows][kArgSlots]
    uint64_t *pk = reinterpret_cast<uint64_t *>(p.partial);         // [nblk], one row
    if (wave == 0) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int off = 16; off <= 32; off <<= 1) {
          const float ov = shfl_xor(best_v[mt], off);
          const int oi = __shfl_xor(best_i[mt], off, kWave);
          if (ov > best_v[mt] || (ov == best_v[mt] && oi < best_i[mt])) {
            best_v[mt] = ov;
            best_i[mt] = oi;
          }
        }
        const int m = mt * 16 + col;
        if (grp == 0 && m < rows) {
          const uint64_t key = argmax_key(best_v[mt], best_i[mt]);
          if (rows == 1)
            st64_dev(pk + blk, key);
          else
            __hip_atomic_fetch_max(keys + (size_t)m * kArgSlots + (blk & (kArgSlots - 1)), key, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
    if (!arrive_last(p.counters, (uint32_t)nblk, s_flag)) return;
    if (rows == 1) {
      uint64_t b4[4] = {0ull, 0ull, 0ull, 0ull};
      for (int g = tid; g < nblk; g += 4 * nthr) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int gu = g + u * nthr;
          const uint64_t kk = gu < nblk ? ld64_dev(pk + gu) : 0ull;
          b4[u] = kk > b4[u] ? kk : b4[u];
        }
      }
      uint64_t best = b4[0] > b4[1] ? b4[0] : b4[1];
      const uint64_t b23 = b4[2] > b4[3] ? b4[2] : b4[3];
      best = row16_max(b23 > best ? b23 : best);
      uint64_t *s_key = reinterpret_cast<uint64_t *>(s_red);  // [waves][4]
      if ((lane & 15) == 0) s_key[wave * 4 + (lane >> 4)] = best;
      __syncthreads();
      if (tid == 0) {
        for (int i = 1; i < 4 * nw; ++i) best = s_key[i] > best ? s_key[i] : best;
        p.ids_out[0] = (int64_t)argmax_index(best);
        if (p.lens_inc) p.lens_inc[0] += 1;
      }
      return;
    }
    // A wave takes 4 rows per pass (16 lanes, one slot each), four passes'
    // loads in flight at once.
    for (int j0 = 0; j0 * nw * 4 < rows; j0 += 4) {
      uint64_t kv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int m = ((j0 + j) * nw + wave) * 4 + (lane >> 4);
        kv[j] = m < rows ? ld64_dev(keys + (size_t)m * kArgSlots + (lane & 15)) : 0ull;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int m = ((j0 + j) * nw + wave) * 4 + (lane >> 4);
        if (m < rows) st64_dev(keys + (size_t)m * kArgSlots + (lane & 15), 0ull);
        const uint64_t best = row16_max(kv[j]);
        if ((lane & 15) == 0 && m < rows) {
          p.ids_out[m] = (int64_t)argmax_index(best);
          if (p.lens_inc) p.lens_inc[m] += 1;
        }
      }
    }
  }
}

}  // namespace
}  // namespace qdec
