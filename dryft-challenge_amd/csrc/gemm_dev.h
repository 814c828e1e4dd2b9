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
// The body itself is gemm_body.inc, included by the per-operation kernel
// (gemm_kernel, gemm.hip) and by gemm_body below, which takes its workgroup
// index and count as arguments for the one-layer-per-launch kernel
// (layer.hip): both run the same code.
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
static_assert(kFastRows == kFastRowsMax, "the planner's bound on register-staged rows of the pass path");

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
  const int n_active = min((p.a_strided ? (L + T - 1) >> 5 : (L + T - 1) / p.a_chunk) + 1, p.a_nchunks);
  const float NEG_INF = -__builtin_huge_valf();
  float mc[CB], lc[CB];
  f32x4_t a0[CB], a1[CB];
  auto load_group = [&](int cc) {
#pragma unroll
    for (int j = 0; j < CB; ++j) {
      const float *pr = part_b + (size_t)min(cc + j, n_active - 1) * cstride;
      if constexpr (COH) {
        mc[j] = load_coherent(pr + (size_t)R * D + r);
        lc[j] = load_coherent(pr + (size_t)R * D + R + r);
        a0[j] = load_coherent4(pr + (size_t)r * D + d0);
        a1[j] = load_coherent4(pr + (size_t)r * D + d0 + 4);
      } else {
        mc[j] = pr[(size_t)R * D + r];
        lc[j] = pr[(size_t)R * D + R + r];
        a0[j] = *reinterpret_cast<const f32x4_t *>(pr + (size_t)r * D + d0);
        a1[j] = *reinterpret_cast<const f32x4_t *>(pr + (size_t)r * D + d0 + 4);
      }
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
    for (int j = 0; j < CB; ++j) {
      const float *q = part_b + (size_t)min(cc + j, n_active - 1) * cstride + (size_t)R * D + r;
      if constexpr (COH)
        mg[j] = load_coherent(q);
      else
        mg[j] = *q;
    }
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
static_assert(kHandMaxParts == kMergeParts, "a hand-over merges what the pre-pass keeps in registers");

// Norm hand-over, the last step of a RES_OUT call that feeds a NORM_IN call
// (template flag kGemmHandOver): that call's normalisation needs every output
// tile of this one, so it is done here, after the last tile, instead of by a
// pre-pass launch of the consumer.  Every workgroup, once its outputs are
// stored (at device scope: a row is read back by a workgroup on another
// XCD), takes an arrival ticket (hsync[0]); the last NR = hxt*16 to arrive
// each take one row, wait until all nblk have arrived, and write that row
// as the consumer's pre-pass (rownorm_kernel) would: the merged residual
// with split partials, then bf16(norm_w * bf16(r * rstd)) in fragment
// order.  The statistic follows a workgroup of hthreads threads -- virtual
// thread t sums vectors t and t + hthreads, lanes in wave_sum's tree, then
// virtual waves in order -- which this workgroup emulates when it is half
// or twice that size (a zero contribution leaves an fp32 sum unchanged), so
// the row is bit-identical to the pre-pass's.  Rows past `rows` are zeros.
// The row that leaves last (hsync[1]) resets both words.  A wait past
// kHandSpin polls (a workgroup that never arrives) writes a NaN row instead
// of hanging, and sets hsync[2], after which every hand-over row writes NaN
// until the caller zeroes the counters.
//
// Its parameters are read from the kernel's argument segment (GemmParams is
// gemm_kernel's only argument, at offset 0) through a pointer the compiler
// cannot see through, so none of those loads is hoisted into the GEMM's loop,
// where the scalar registers holding them would cost the loop a wave per
// SIMD.  (Through the address of the parameter the whole block would be
// copied to scratch.)
typedef const __attribute__((address_space(4))) GemmParams *KernargParams;
__device__ __forceinline__ uint4 nan8() { return make_uint4(0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u); }
// The thread index comes from the lane count (mbcnt) and the wave index in
// a scalar register (wave_s), so no vector register has to keep threadIdx
// across the loop for it.
__device__ __forceinline__ void hand_over_row(const int nblk, const int wave_s, float *s_red, uint32_t *s_flag) {
  KernargParams pp = (KernargParams)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(pp));
  const auto &p = *pp;
  const int lane = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  const int wave = wave_s, tid = wave * 64 + lane;
  const int R = blockDim.x, V = p.hthreads, NR = p.hxt * 16;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  if (tid == 0) {
    const uint32_t old = __hip_atomic_fetch_add(p.hsync, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    int row = (int)old - (nblk - NR);
    uint32_t ok = 1u;
    if (row >= NR) row = -1;
    if (row >= 0) {
      uint32_t polls = 0;
      while (__hip_atomic_load(p.hsync, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < (uint32_t)nblk) {
        if (++polls >= kHandSpin) {
          ok = 0u;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      // A give-up is sticky (hsync[2]): late arrivals of that call leave
      // hsync[0] off for every later call, so those write NaN rows too until
      // the caller zeroes the counters.
      if (!ok)
        __hip_atomic_store(p.hsync + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      else if (__hip_atomic_load(p.hsync + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u)
        ok = 0u;
      const uint32_t d = __hip_atomic_fetch_add(p.hsync + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (d == (uint32_t)NR - 1u) {
        __hip_atomic_store(p.hsync, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(p.hsync + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    s_flag[0] = (uint32_t)row;
    s_flag[1] = ok;
  }
  __syncthreads();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  const int m = (int)s_flag[0];
  if (m < 0) return;
  const bool ok = s_flag[1] != 0u;
  const int k = p.n, nvec = k >> 3;
  auto dst = [&](int v) {
    return p.hxn + (((size_t)(v >> 2) * p.hxt + (m >> 4)) * 64 + (m & 15) + 16 * (v & 3)) * 8;
  };
  if (m >= p.rows) {
    for (int v = tid; v < nvec; v += R) *reinterpret_cast<uint4 *>(dst(v)) = zero4();
    return;
  }
  const uint16_t *xrow = reinterpret_cast<const uint16_t *>(p.res) + (size_t)m * k;
  const bool parts = p.parts_out != nullptr;
  // Two vector slots per thread.  Same size (nsl = 1): virtual thread tid,
  // its vectors tid and tid + V.  Half the consumer's size (nsl = 2, where
  // the plan ensures a row of at most V vectors): virtual threads tid and
  // tid + R, one vector each.
  const int nsl = V > R ? 2 : 1;
  uint4 xv[2];
  float ss[2] = {0.f, 0.f};
  int vs[2];
#pragma unroll
  for (int sl = 0; sl < 2; ++sl) {
    const int t = nsl == 2 ? tid + sl * R : tid;
    const int v = nsl == 2 ? t : t + sl * V;
    vs[sl] = (t < V && v < nvec) ? v : -1;
  }
#pragma unroll
  for (int sl = 0; sl < 2; ++sl) {
    const int v = vs[sl];
    const int vv = v >= 0 ? v : 0;
    if (parts) {
      // bf16(x + bf16(((p0 + p1) + p2) + p3)): merge_res8's order and rounding
      const uint4 x = *reinterpret_cast<const uint4 *>(xrow + 8 * vv);
      const float *q = p.parts_out + (size_t)m * k + 8 * vv;
      const size_t stride = (size_t)p.rows * k;
      f32x4_t pa[kMergeParts][2];
#pragma unroll
      for (int part = 0; part < kMergeParts; ++part) {
        const float *qp = q + (part < p.ksplit ? part : 0) * stride;
        pa[part][0] = load_coherent4(qp);
        pa[part][1] = load_coherent4(qp + 4);
      }
      f32x4_t s0 = pa[0][0], s1 = pa[0][1];
#pragma unroll
      for (int part = 1; part < kMergeParts; ++part)
        if (part < p.ksplit) {
          s0 += pa[part][0];
          s1 += pa[part][1];
        }
      uint4 o;
      o.x = pack2(lo16(x.x) + rbf(s0[0]), hi16(x.x) + rbf(s0[1]));
      o.y = pack2(lo16(x.y) + rbf(s0[2]), hi16(x.y) + rbf(s0[3]));
      o.z = pack2(lo16(x.z) + rbf(s1[0]), hi16(x.z) + rbf(s1[1]));
      o.w = pack2(lo16(x.w) + rbf(s1[2]), hi16(x.w) + rbf(s1[3]));
      xv[sl] = o;
      if (v >= 0) *reinterpret_cast<uint4 *>(p.hmerged + (size_t)m * k + 8 * v) = ok ? o : nan8();
    } else {
      xv[sl] = ldv16<true>(xrow + 8 * vv);
    }
    if (v >= 0) {
      float f[8];
      unpack8(xv[sl], f);
      float &acc = ss[nsl == 2 ? sl : 0];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc += f[e] * f[e];
    }
  }
  // The norm weights only now: their latency overlaps the reduction.
  uint4 wv[2];
#pragma unroll
  for (int sl = 0; sl < 2; ++sl) wv[sl] = *reinterpret_cast<const uint4 *>(p.hnorm_w + 8 * (vs[sl] >= 0 ? vs[sl] : 0));
  // s_red[w'] = sum of virtual wave w' (real wave w' mod R/64, slice w' / (R/64))
#pragma unroll
  for (int sl = 0; sl < 2; ++sl) {
    if (sl >= nsl) break;
    const float s = wave_sum(ss[sl]);
    if (lane == 0) s_red[wave + sl * (R >> 6)] = s;
  }
  __syncthreads();
  if (tid == 0) {
    float t = 0.f;
    for (int w2 = 0; w2 < (V >> 6); ++w2) t += s_red[w2];
    s_red[16] = 1.0f / sqrtf(t / (float)k + p.eps);
  }
  __syncthreads();
  const float rs = s_red[16];
#pragma unroll
  for (int sl = 0; sl < 2; ++sl)
    if (vs[sl] >= 0) *reinterpret_cast<uint4 *>(dst(vs[sl])) = ok ? norm8(xv[sl], wv[sl], rs) : nan8();
}

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
#define QDEC_LDX16(q) ldv16<COH>(q)
#define QDEC_LDX8(q) ldv8<COH>(q)
#define QDEC_STX8(q, v) stv8<COH>((q), (v))
#define QDEC_MERGE8(pp, m, kk) attn_merge8<COH>((pp), (m), (kk))
#include "gemm_body.inc"
#undef QDEC_LDX16
#undef QDEC_LDX8
#undef QDEC_STX8
#undef QDEC_MERGE8
}

}  // namespace
}  // namespace qdec
