// Device body of the skinny GEMM, shared by the standalone kernel (gemm.hip)
// and the persistent step kernel (step.hip).  See gemm.hip for the design.
#pragma once

#include "qdec_common.h"
#include "qdec_kernels.h"

namespace qdec {

// Weight registers a wave holds per pass: 20 blocks, or 2 x 10 with GLU.
constexpr int kWbuf = 20;

// Fast activation path: up to kFastRows rows, 2 vectors per thread per row.
constexpr int kFastRows = 4;
constexpr int kFastVec = 2;

// Sum one fp32 value per thread of the workgroup for up to 8 rows in a fixed
// order (lane tree, then waves in order); thread m < nrows gets row m's total.
__device__ __forceinline__ void block_row_sums(float (&ss)[8], float *s_red, int nrows,
                                               float *dst_rstd, int m0, int k, float eps) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, tid = threadIdx.x;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    float v = ss[j];
    v += shfl_xor(v, 32);
    v += shfl_xor(v, 16);
    v += shfl_xor(v, 8);
    v += shfl_xor(v, 4);
    v += shfl_xor(v, 2);
    v += shfl_xor(v, 1);
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

// Issue the first pass's weight loads of block `blk` into `wbuf` (the
// persistent kernel calls this before it waits for the previous phase).
template <uint32_t FLAGS>
__device__ __forceinline__ void gemm_prefetch(const GemmParams &p, const int blk, uint4 (&wbuf)[kWbuf]) {
  constexpr bool GLU = (FLAGS & QDEC_GLU) != 0;
  constexpr int KPMAX = GLU ? kGemmKpMaxGlu : kGemmKpMax;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tg = blk / p.ksplit;
  const int split = blk - tg * p.ksplit;
  const int ks_wave = split * (p.KS / p.ksplit) + wave * p.ksw;
  const int kcnt = min(p.kp, p.ksw);
  const uint4 *__restrict__ W = reinterpret_cast<const uint4 *>(p.w);
  const size_t up_off = (size_t)p.up_tiles * p.KS * 64;
  const size_t blk0 = ((size_t)(tg * p.tiles_per_wg) * p.KS + ks_wave) * 64 + lane;
#pragma unroll
  for (int i = 0; i < KPMAX; ++i) {
    const size_t off = blk0 + (size_t)min(i, kcnt - 1) * 64;
    wbuf[i] = W[off];
    if constexpr (GLU) wbuf[KPMAX + i] = W[off + up_off];
  }
}


template <int MT, uint32_t FLAGS, bool COH>
__device__ __forceinline__ bool gemm_block(const GemmParams &p, const int blk, const int nblk,
                                           unsigned char *smem, uint4 (&wbuf)[kWbuf], bool have_first,
                                           const int next_blk = -1) {
  constexpr bool NORM = (FLAGS & QDEC_NORM_IN) != 0;
  constexpr bool GLU = (FLAGS & QDEC_GLU) != 0;
  constexpr bool RES = (FLAGS & QDEC_RES_OUT) != 0;
  constexpr bool ARG = (FLAGS & QDEC_ARGMAX) != 0;
  constexpr int NACC = GLU ? 2 : 1;
  constexpr int KPMAX = GLU ? kGemmKpMaxGlu : kGemmKpMax;

  float *s_rstd = reinterpret_cast<float *>(smem);                     // [64]
  uint32_t *s_flag = reinterpret_cast<uint32_t *>(smem + 256);         // [4]
  float *s_red = reinterpret_cast<float *>(smem + 272);                // [64 floats]
  uint16_t *s_x = reinterpret_cast<uint16_t *>(smem + p.lds_x_off);    // [rows][xstride]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nthr = blockDim.x;
  const int nw = nthr >> 6;
  const int rows = p.rows;
  const int col = lane & 15;   // row of x inside an M tile
  const int grp = lane >> 4;   // k group / output column group

  const int tg = blk / p.ksplit;               // tile group
  const int split = blk - tg * p.ksplit;
  const int ks_wg = split * (p.KS / p.ksplit); // first k step of this workgroup
  const int ks_wave = ks_wg + wave * p.ksw;    // first k step of this wave
  const int xstride = p.xstride;
  const uint4 *__restrict__ W = reinterpret_cast<const uint4 *>(p.w);
  const uint16_t *__restrict__ X = reinterpret_cast<const uint16_t *>(p.x);
  const size_t up_off = (size_t)p.up_tiles * p.KS * 64;

  // Straight-line weight loads of one pass; indices past the pass are clamped
  // to its last block (a redundant, cache-served load) instead of branched
  // around, so all of them stay in flight together.
  static_assert(NACC * KPMAX == kWbuf, "weight buffer size");
  auto issue_w = [&](int tile, int kbeg, int kcnt) {
    const size_t blk0 = ((size_t)tile * p.KS + ks_wave + kbeg) * 64 + lane;
#pragma unroll
    for (int i = 0; i < KPMAX; ++i) {
      const size_t off = blk0 + (size_t)min(i, kcnt - 1) * 64;
      wbuf[i] = W[off];
      if constexpr (GLU) wbuf[KPMAX + i] = W[off + up_off];
    }
  };

  const int tile0 = tg * p.tiles_per_wg;
  // LDS column of the wave's k step i (absolute within the wave's range when
  // the whole range is staged, pass-relative otherwise).
  const int lds_steps = p.lds_all ? p.ksw : p.kp;

  bool staged = false;
  if (p.xfast) {
    // Activations into registers -- issued before the weights: they are
    // cache hits, and the statistics and LDS staging computed from them then
    // overlap the weight stream (loads complete in issue order).  Row m,
    // vectors vr = tid + j*nthr of the workgroup's k range (per_row of them).
    const int per_row = p.ksw * nw * 4;
    uint4 xr[kFastRows][kFastVec];
#pragma unroll
    for (int m = 0; m < kFastRows; ++m)
#pragma unroll
      for (int j = 0; j < kFastVec; ++j) {
        const int vr = tid + j * nthr;
        const bool ok = m < rows && vr < per_row;
        const int mm = ok ? m : 0, vv = ok ? vr : 0;
        const uint4 v = ld16<COH>(X + (size_t)mm * p.k + ks_wg * 32 + 8 * vv);
        xr[m][j] = ok ? v : zero4();
      }
    if (!have_first) issue_w(tile0, 0, min(p.kp, p.ksw));
    if constexpr (NORM) {
      float ss[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) ss[j] = 0.f;
#pragma unroll
      for (int m = 0; m < kFastRows; ++m)
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
    for (int m = 0; m < kFastRows; ++m)
#pragma unroll
      for (int j = 0; j < kFastVec; ++j) {
        const int vr = tid + j * nthr;
        if (m < rows && vr < per_row) {
          uint4 xv = xr[m][j];
          if constexpr (NORM) {
            const uint4 nv = *reinterpret_cast<const uint4 *>(
                reinterpret_cast<const uint16_t *>(p.norm_w) + ks_wg * 32 + 8 * vr);
            float f[8], g[8];
            unpack8(xv, f);
            unpack8(nv, g);
            const float rs = s_rstd[m];
#pragma unroll
            for (int e = 0; e < 8; ++e) f[e] = g[e] * rbf(f[e] * rs);
            xv = pack8(f);
          }
          *reinterpret_cast<uint4 *>(s_x + (size_t)m * xstride + 8 * vr) = xv;
        }
      }
    __syncthreads();
    staged = true;
  } else {
    if (!have_first) issue_w(tile0, 0, min(p.kp, p.ksw));
  }
  if (!p.xfast) {
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
            unpack8(ld16<COH>(xrow + 8 * v), f);
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
      const int total = rows * per_row;
      for (int v = tid; v < total; v += nthr) {
        const int m = v / per_row;
        const int vr = v - m * per_row;
        const int kg = ks_wg * 32 + 8 * vr;
        uint4 xv = ld16<COH>(X + (size_t)m * p.k + kg);
        if constexpr (NORM) {
          const uint4 nv = *reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(p.norm_w) + kg);
          float f[8], g[8];
          unpack8(xv, f);
          unpack8(nv, g);
          const float rs = s_rstd[m];
#pragma unroll
          for (int e = 0; e < 8; ++e) f[e] = g[e] * rbf(f[e] * rs);
          xv = pack8(f);
        }
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

  bool have_w = true;  // wb holds the next pass's weights already
  bool next_ready = false;  // wbuf holds next_blk's first pass on return
  for (int tt = 0; tt < p.tiles_per_wg; ++tt) {
    const int tile = tile0 + tt;
    f32x4_t acc[NACC][MT];
#pragma unroll
    for (int a = 0; a < NACC; ++a)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[a][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    for (int pass = 0; pass < p.npass; ++pass) {
      const int kbeg = pass * p.kp;
      const int kcnt = min(p.kp, p.ksw - kbeg);
      if (!have_w) issue_w(tile, kbeg, kcnt);
      have_w = false;
      if (!staged) {
        if (pass > 0 || tt > 0) __syncthreads();  // previous readers are done
        const int per_row = nw * kcnt * 4;  // 16-byte vectors per row in this pass
        const int total = rows * per_row;
        for (int v = tid; v < total; v += nthr) {
          const int m = v / per_row;
          int r = v - m * per_row;
          const int w2 = r / (kcnt * 4);
          r -= w2 * (kcnt * 4);
          const int i = r >> 2;
          const int q = r & 3;
          const int kg = (ks_wg + w2 * p.ksw + kbeg + i) * 32 + q * 8;
          uint4 xv = ld16<COH>(X + (size_t)m * p.k + kg);
          if constexpr (NORM) {
            const uint4 nv = *reinterpret_cast<const uint4 *>(
                reinterpret_cast<const uint16_t *>(p.norm_w) + kg);
            float f[8], g[8];
            unpack8(xv, f);
            unpack8(nv, g);
            const float rs = s_rstd[m];
#pragma unroll
            for (int e = 0; e < 8; ++e) f[e] = g[e] * rbf(f[e] * rs);
            xv = pack8(f);
          }
          *reinterpret_cast<uint4 *>(s_x + (size_t)m * xstride + (w2 * p.kp + i) * 32 + q * 8) = xv;
        }
        __syncthreads();
        staged = p.npass == 1;  // several passes restage per pass
      }
      // MFMA over this pass.
#pragma unroll
      for (int i = 0; i < KPMAX; ++i) {
        if (i < kcnt) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const int m = mt * 16 + col;
            uint4 b = zero4();
            if (m < rows)
              b = *reinterpret_cast<const uint4 *>(
                  s_x + (size_t)m * xstride +
                  (wave * lds_steps + (p.lds_all ? kbeg : 0) + i) * 32 + grp * 8);
#pragma unroll
            for (int a = 0; a < NACC; ++a) acc[a][mt] = mfma16x16x32(wbuf[a * KPMAX + i], b, acc[a][mt]);
          }
        }
      }
    }
    // Request the next tile's (or the next block's) weights before this
    // tile's epilogue.
    if (p.npass == 1 && tt + 1 < p.tiles_per_wg) {
      issue_w(tile + 1, 0, min(p.kp, p.ksw));
      have_w = true;
    } else if (tt + 1 == p.tiles_per_wg && next_blk >= 0) {
      gemm_prefetch<FLAGS>(p, next_blk, wbuf);
      next_ready = true;
    }

    // ---- merge the waves of the workgroup in wave order.
    if (nw > 1) {
      __syncthreads();
      float4 *red = reinterpret_cast<float4 *>(smem + p.lds_red_off);
      if (wave > 0) {
#pragma unroll
        for (int a = 0; a < NACC; ++a)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            red[(((wave - 1) * NACC + a) * MT + mt) * 64 + lane] =
                make_float4(acc[a][mt][0], acc[a][mt][1], acc[a][mt][2], acc[a][mt][3]);
      }
      __syncthreads();
      if (wave == 0) {
        for (int w2 = 1; w2 < nw; ++w2) {
#pragma unroll
          for (int a = 0; a < NACC; ++a)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
              const float4 r = red[(((w2 - 1) * NACC + a) * MT + mt) * 64 + lane];
              acc[a][mt][0] += r.x;
              acc[a][mt][1] += r.y;
              acc[a][mt][2] += r.z;
              acc[a][mt][3] += r.w;
            }
        }
      }
    }

    const int n0 = tile * 16 + grp * 4;  // first of this lane's 4 output columns

    // ---- k split across workgroups: partials, last arrival sums them.
    if (p.ksplit > 1) {
      if (wave == 0) {
#pragma unroll
        for (int a = 0; a < NACC; ++a)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const int m = mt * 16 + col;
            if (m < rows) {
              float *dst = p.partial + ((size_t)(a * p.ksplit + split) * rows + m) * p.n + n0;
              store_coherent4(dst, acc[a][mt]);
            }
          }
      }
      if (!arrive_last(p.counters + tile, (uint32_t)p.ksplit, s_flag)) return next_ready;
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
              acc[a][mt] = t;
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
        if constexpr (ARG) {
          float v[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] = rbf(acc[0][mt][i]);
          if (p.out) {
            uint2 o;
            o.x = pack2(v[0], v[1]);
            o.y = pack2(v[2], v[3]);
            st8<COH>(reinterpret_cast<uint16_t *>(p.out) + (size_t)m * p.n + n0, o);
          }
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (v[i] > best_v[mt]) {
              best_v[mt] = v[i];
              best_i[mt] = n0 + i;
            }
        } else if constexpr (RES) {
          uint16_t *rp = reinterpret_cast<uint16_t *>(p.res) + (size_t)m * p.n + n0;
          const uint2 r = ld8<COH>(rp);
          uint2 o;
          o.x = pack2(lo16(r.x) + rbf(acc[0][mt][0]), hi16(r.x) + rbf(acc[0][mt][1]));
          o.y = pack2(lo16(r.y) + rbf(acc[0][mt][2]), hi16(r.y) + rbf(acc[0][mt][3]));
          st8<COH>(rp, o);
        } else if constexpr (GLU) {
          float o4[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float g = rbf(acc[0][mt][i]);
            const float u = rbf(acc[1][mt][i]);
            const float s = rbf(g / (1.0f + expf(-g)));
            o4[i] = s * u;
          }
          uint2 o;
          o.x = pack2(o4[0], o4[1]);
          o.y = pack2(o4[2], o4[3]);
          st8<COH>(reinterpret_cast<uint16_t *>(p.out) + (size_t)m * p.n + n0, o);
        } else {
          uint2 o;
          o.x = pack2(acc[0][mt][0], acc[0][mt][1]);
          o.y = pack2(acc[0][mt][2], acc[0][mt][3]);
          st8<COH>(reinterpret_cast<uint16_t *>(p.out) + (size_t)m * p.n + n0, o);
        }
      }
    }
  }

  if constexpr (ARG) {
    // Reduce the 4 column groups of each row, lowest index on equal values.
    float *pv = p.partial;                                                    // [G][rows]
    int *pi = reinterpret_cast<int *>(p.partial + (size_t)nblk * rows);  // [G][rows]
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
          store_coherent(pv + (size_t)blk * rows + m, best_v[mt]);
          store_coherent_i(pi + (size_t)blk * rows + m, best_i[mt]);
        }
      }
    }
    if (!arrive_last(p.counters, (uint32_t)nblk, s_flag)) return next_ready;
    float *sv = s_red;                                      // [waves]
    int *si = reinterpret_cast<int *>(s_red + 8);           // [waves]
    for (int m = 0; m < rows; ++m) {
      float bv = -__builtin_huge_valf();
      int bi = 0x7fffffff;
      for (int g = tid; g < nblk; g += nthr) {
        const float v = load_coherent(pv + (size_t)g * rows + m);
        const int i = load_coherent_i(pi + (size_t)g * rows + m);
        if (v > bv || (v == bv && i < bi)) {
          bv = v;
          bi = i;
        }
      }
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) {
        const float ov = shfl_xor(bv, off);
        const int oi = __shfl_xor(bi, off, kWave);
        if (ov > bv || (ov == bv && oi < bi)) {
          bv = ov;
          bi = oi;
        }
      }
      if (lane == 0) {
        sv[wave] = bv;
        si[wave] = bi;
      }
      __syncthreads();
      if (tid == 0) {
        for (int w2 = 1; w2 < nw; ++w2)
          if (sv[w2] > bv || (sv[w2] == bv && si[w2] < bi)) {
            bv = sv[w2];
            bi = si[w2];
          }
        p.ids_out[m] = (int64_t)bi;
        if (p.lens_inc) p.lens_inc[m] += 1;
      }
      __syncthreads();
    }
  }
  return next_ready;
}


}  // namespace qdec
