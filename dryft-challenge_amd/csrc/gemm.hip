// Launchers of the weight-streaming skinny GEMM (its design: gemm_dev.h; its
// body: gemm_body.inc) and the row-normalisation pre-pass.
#include "gemm_dev.h"

namespace qdec {
namespace {

// One workgroup per block of the plan (the body and its design: gemm_body.inc,
// gemm_dev.h).
template <int MT, uint32_t FLAGS, int RW, bool XD, int FR = kFastRows, bool XP = false, int TW = 1>
__global__ void __launch_bounds__(512) gemm_kernel(const GemmParams p) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int blk = blockIdx.x, nblk = gridDim.x;
#define QDEC_LDX16(q) (*reinterpret_cast<const uint4 *>(q))
#define QDEC_LDX8(q) (*reinterpret_cast<const uint2 *>(q))
#define QDEC_STX8(q, v) (*reinterpret_cast<uint2 *>(q) = (v))
#define QDEC_MERGE8(pp, m, kk) attn_merge8<false>((pp), (m), (kk))
#include "gemm_body.inc"
#undef QDEC_LDX16
#undef QDEC_LDX8
#undef QDEC_STX8
#undef QDEC_MERGE8
}

// x' = norm_w * bf16(x * rstd) of one row per workgroup, written to xn: the
// same statistic (thread t sums vectors t, t+T, ..., then block_row_sums)
// and the same rounding as the GEMM's own staging, so a row comes out
// bit-identical whichever path stages it.
__global__ void __launch_bounds__(512) rownorm_kernel(const uint16_t *__restrict__ X, const uint16_t *__restrict__ norm_w,
                                                       uint16_t *__restrict__ xn, int k, float eps, int rows, int nmt,
                                                       int do_norm, const float *__restrict__ parts, int nparts,
                                                       uint16_t *__restrict__ xmerged) {
  __shared__ float s_red[8 * 8];
  __shared__ float s_rstd[8];
  const int m = blockIdx.x, tid = threadIdx.x, nthr = blockDim.x;
  const int nvec = k >> 3;
  // Fragment order (nmt > 0): vector v of row m goes to k step v/4, M tile
  // m/16, lane (m%16) + 16*(v%4); rows past the last real one are zeros.
  auto dst = [&](int v) -> uint16_t * {
    if (nmt == 0) return xn + (size_t)m * k + 8 * v;
    return xn + (((size_t)(v >> 2) * nmt + (m >> 4)) * 64 + (m & 15) + 16 * (v & 3)) * 8;
  };
  if (m >= rows) {
    for (int v = tid; v < nvec; v += nthr) *reinterpret_cast<uint4 *>(dst(v)) = zero4();
    return;
  }
  const uint16_t *xrow = X + (size_t)m * k;
  if (nvec <= 2 * nthr && nparts <= kMergeParts) {
    // The whole row in registers, two vectors per thread: every load (x,
    // the pending partials, the norm weights) is issued before the first is
    // used, and the row is read once.  Same statistic order and roundings
    // as the loop below.
    uint4 xv[2], wv[2];
    f32x4_t pv[2][kMergeParts][2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int v = tid + j * nthr;
      const int vv = v < nvec ? v : 0;
      xv[j] = *reinterpret_cast<const uint4 *>(xrow + 8 * vv);
      if (parts) {
        const float *q = parts + (size_t)m * k + 8 * vv;
#pragma unroll
        for (int part = 0; part < kMergeParts; ++part) {
          const float *qp = q + (size_t)(part < nparts ? part : 0) * rows * k;
          pv[j][part][0] = *reinterpret_cast<const f32x4_t *>(qp);
          pv[j][part][1] = *reinterpret_cast<const f32x4_t *>(qp + 4);
        }
      }
      wv[j] = do_norm ? *reinterpret_cast<const uint4 *>(norm_w + 8 * vv) : zero4();
    }
    float ss[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) ss[j] = 0.f;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int v = tid + j * nthr;
      if (v >= nvec) continue;
      if (parts) {
        // bf16(x + bf16(((p0 + p1) + p2) + p3)): merge_res8's order and rounding
        f32x4_t s0 = pv[j][0][0], s1 = pv[j][0][1];
#pragma unroll
        for (int part = 1; part < kMergeParts; ++part)
          if (part < nparts) {
            s0 += pv[j][part][0];
            s1 += pv[j][part][1];
          }
        const uint4 x = xv[j];
        uint4 o;
        o.x = pack2(lo16(x.x) + rbf(s0[0]), hi16(x.x) + rbf(s0[1]));
        o.y = pack2(lo16(x.y) + rbf(s0[2]), hi16(x.y) + rbf(s0[3]));
        o.z = pack2(lo16(x.z) + rbf(s1[0]), hi16(x.z) + rbf(s1[1]));
        o.w = pack2(lo16(x.w) + rbf(s1[2]), hi16(x.w) + rbf(s1[3]));
        xv[j] = o;
        *reinterpret_cast<uint4 *>(xmerged + (size_t)m * k + 8 * v) = o;
      }
      float f[8];
      unpack8(xv[j], f);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss[0] += f[e] * f[e];
    }
    if (!do_norm) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int v = tid + j * nthr;
        if (v < nvec) *reinterpret_cast<uint4 *>(dst(v)) = xv[j];
      }
      return;
    }
    block_row_sums(ss, s_red, 1, s_rstd, 0, k, eps);
    const float rs = s_rstd[0];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int v = tid + j * nthr;
      if (v < nvec) *reinterpret_cast<uint4 *>(dst(v)) = norm8(xv[j], wv[j], rs);
    }
    return;
  }
  if (parts) {
    // Apply the pending split residual update once, into xmerged; both
    // loops below then read the merged row (each thread its own vectors).
    uint16_t *mrow = xmerged + (size_t)m * k;
    for (int v = tid; v < nvec; v += nthr)
      *reinterpret_cast<uint4 *>(mrow + 8 * v) =
          merge_res8(parts, nparts, rows, k, *reinterpret_cast<const uint4 *>(xrow + 8 * v), m, 8 * v);
    xrow = mrow;
  }
  if (!do_norm) {  // re-layout only
    for (int v = tid; v < nvec; v += nthr) *reinterpret_cast<uint4 *>(dst(v)) = *reinterpret_cast<const uint4 *>(xrow + 8 * v);
    return;
  }
  float ss[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) ss[j] = 0.f;
  for (int v = tid; v < nvec; v += nthr) {
    float f[8];
    unpack8(*reinterpret_cast<const uint4 *>(xrow + 8 * v), f);
#pragma unroll
    for (int e = 0; e < 8; ++e) ss[0] += f[e] * f[e];
  }
  block_row_sums(ss, s_red, 1, s_rstd, 0, k, eps);
  const float rs = s_rstd[0];
  for (int v = tid; v < nvec; v += nthr)
    *reinterpret_cast<uint4 *>(dst(v)) =
        norm8(*reinterpret_cast<const uint4 *>(xrow + 8 * v), *reinterpret_cast<const uint4 *>(norm_w + 8 * v), rs);
}

template <int MT, int RW>
hipError_t launch_flags(const GemmParams &p, uint32_t flags, dim3 grid, dim3 block, size_t lds, hipStream_t s) {
  switch (flags) {
    case 0u: hipLaunchKernelGGL((gemm_kernel<MT, 0u, RW, false>), grid, block, lds, s, p); break;
    case QDEC_NORM_IN: hipLaunchKernelGGL((gemm_kernel<MT, QDEC_NORM_IN, RW, false>), grid, block, lds, s, p); break;
    case QDEC_RES_OUT: hipLaunchKernelGGL((gemm_kernel<MT, QDEC_RES_OUT, RW, false>), grid, block, lds, s, p); break;
    case QDEC_NORM_IN | QDEC_ARGMAX:
      hipLaunchKernelGGL((gemm_kernel<MT, QDEC_NORM_IN | QDEC_ARGMAX, RW, false>), grid, block, lds, s, p);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipSuccess;
}

template <int MT>
hipError_t launch_pass(const GemmParams &p, uint32_t flags, dim3 grid, dim3 block, size_t lds, hipStream_t s) {
  if (flags == (QDEC_NORM_IN | QDEC_GLU)) {
    hipLaunchKernelGGL((gemm_kernel<MT, QDEC_NORM_IN | QDEC_GLU, 0, false>), grid, block, lds, s, p);
    return hipSuccess;
  }
  return launch_flags<MT, 0>(p, flags, grid, block, lds, s);
}

}  // namespace

bool gemm_flags_supported(uint32_t flags) {
  // GLU and ARGMAX alone: the direct path only (x_frag, the input a norm
  // hand-over leaves), checked by the planner.
  return flags == 0u || flags == QDEC_NORM_IN || flags == (QDEC_NORM_IN | QDEC_GLU) || flags == QDEC_RES_OUT ||
         flags == (QDEC_NORM_IN | QDEC_ARGMAX) || flags == QDEC_GLU || flags == QDEC_ARGMAX;
}

bool gemm_fast_path(const GemmParams &p, uint32_t flags) {
  const int per_row = p.ksw * p.waves * 4;
  // 8 register rows pay for NORM_IN without GLU (qkv 12.7 us at 8 rows vs
  // 14.6 through the pre-pass); gate/up keeps its 3 waves per SIMD instead.
  const bool norm8 = (flags & QDEC_NORM_IN) && !(flags & QDEC_GLU);
  return p.lds_all && p.rows <= (norm8 ? kFastRowsNorm : kFastRows) &&
         per_row <= kFastVec * 64 * p.waves &&
         (!(flags & QDEC_NORM_IN) || p.ksplit == 1);
}

int gemm_ring(int ksw, uint32_t flags) {
  if (flags & QDEC_GLU) return ksw % 10 == 0 ? 10 : 0;
  // 20 and 16 measured faster than passes on MI355X; a 19-register ring
  // (k = 9728 with 4 waves) was slower than 20-block passes.
  for (const int rw : {20, 16})
    if (ksw % rw == 0) return rw;
  return 0;
}

namespace {

template <int MT, int RW, int TW = 1>
hipError_t launch_direct(const GemmParams &p, uint32_t flags, dim3 grid, dim3 block, size_t lds, hipStream_t s) {
  switch (flags & ~QDEC_NORM_IN) {
    case 0u: hipLaunchKernelGGL((gemm_kernel<MT, 0u, RW, true, kFastRows, false, TW>), grid, block, lds, s, p); break;
    case QDEC_RES_OUT:
      hipLaunchKernelGGL((gemm_kernel<MT, QDEC_RES_OUT, RW, true, kFastRows, false, TW>), grid, block, lds, s, p);
      break;
    case QDEC_RES_OUT | kGemmHandOver:
      hipLaunchKernelGGL((gemm_kernel<MT, QDEC_RES_OUT | kGemmHandOver, RW, true, kFastRows, false, TW>), grid, block,
                         lds, s, p);
      break;
    case QDEC_ARGMAX:
      hipLaunchKernelGGL((gemm_kernel<MT, QDEC_ARGMAX, RW, true, kFastRows, false, TW>), grid, block, lds, s, p);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipSuccess;
}

template <int MT, int RWG, int TW = 1>
hipError_t launch_direct_glu(const GemmParams &p, dim3 grid, dim3 block, size_t lds, hipStream_t s) {
  hipLaunchKernelGGL((gemm_kernel<MT, QDEC_GLU, RWG, true, kFastRows, false, TW>), grid, block, lds, s, p);
  return hipSuccess;
}

template <int MT, int RW, int RWG>
hipError_t launch_direct_mt(const GemmParams &p, uint32_t flags, dim3 grid, dim3 block, size_t lds, hipStream_t s) {
  if (flags & QDEC_GLU) {
    if (p.rw != RWG) return hipErrorInvalidValue;
    return launch_direct_glu<MT, RWG>(p, grid, block, lds, s);
  }
  if (p.rw != RW) return hipErrorInvalidValue;
  return launch_direct<MT, RW>(p, flags, grid, block, lds, s);
}

// Two tiles per wave, two M tiles, no GLU: the rings gemm_ring_direct offers.
hipError_t launch_direct_tw2(const GemmParams &p, uint32_t flags, dim3 grid, dim3 block, size_t lds, hipStream_t s) {
  if (flags & QDEC_GLU) return hipErrorInvalidValue;
  switch (p.rw) {
    case 5: return launch_direct<2, 5, 2>(p, flags, grid, block, lds, s);
    case 8: return launch_direct<2, 8, 2>(p, flags, grid, block, lds, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

int gemm_ring_direct(int mt, uint32_t flags, int tw, int ksw, int groups) {
  // (tw weight streams + mt activation fragments) x 4 registers per ring
  // slot stays near 128 registers.  GLU at two M tiles and one tile per
  // wave: 5 slots keep the kernel at three waves per SIMD, so all 608
  // gate/up workgroups of Qwen3-4B are resident at once (8 slots: two per
  // SIMD, a second round of 96; batch 32 on MI355X 3.788 -> 3.770 ms per
  // step).  Two tiles per wave (no GLU): 5 slots, three waves per SIMD (8
  // slots take two; QKV at 32 rows 15.3 vs 15.6 us, down 15.0 vs 15.3).  A
  // wave with several groups of tiles keeps slot r on k step r (mod RW) in
  // every group, so RW must then divide its k steps; with one group the last
  // chunk may be ragged.
  const bool glu = (flags & QDEC_GLU) != 0;
  auto fits = [&](int rw) { return (groups == 1 || ksw % rw == 0) ? rw : 0; };
  if (tw == 2) {
    if (mt != 2 || glu) return 0;
    return fits(5) ? 5 : fits(8);
  }
  if (tw != 1) return 0;
  switch (mt) {
    case 1: return fits(glu ? 10 : 20);
    case 2: return fits(glu ? 5 : 10);
    case 3: return fits(glu ? 6 : 8);
    case 4: return fits(glu ? 4 : 8);
    default: return 0;
  }
}

hipError_t launch_rownorm(const GemmParams &p, dim3 block, bool do_norm, hipStream_t s) {
  const int nrow = p.xt ? p.xt * 16 : p.rows;
  hipLaunchKernelGGL(rownorm_kernel, dim3(nrow), block, 0, s, reinterpret_cast<const uint16_t *>(p.x),
                     reinterpret_cast<const uint16_t *>(p.norm_w), p.xn, p.k, p.eps, p.rows, p.xt, do_norm ? 1 : 0,
                     p.xparts, p.xnparts, p.xmerged);
  return hipSuccess;
}

hipError_t launch_rownorm_rows(const void *x, const void *norm_w, void *out, float eps, int rows, int k,
                               int tiles, hipStream_t s) {
  hipLaunchKernelGGL(rownorm_kernel, dim3(tiles * 16), dim3(256), 0, s, reinterpret_cast<const uint16_t *>(x),
                     reinterpret_cast<const uint16_t *>(norm_w), reinterpret_cast<uint16_t *>(out), k, eps, rows,
                     tiles, norm_w ? 1 : 0, nullptr, 0, nullptr);
  return hipSuccess;
}

hipError_t launch_gemm(const GemmParams &p, uint32_t flags, hipStream_t s) {
  if (p.resident == 2) return launch_res_rows(p, s);
  if (p.resident == 3) return launch_res_split(p, s);
  if (p.resident) {
    if (p.xpre) {
      const hipError_t e = launch_rownorm(p, dim3(64 * p.waves), true, s);
      if (e != hipSuccess) return e;
    }
    return launch_glu_resident(p, s);
  }
  const int mt = (p.rows + 15) / 16;
  const int ntiles = p.n / 16;
  dim3 grid((ntiles / p.tiles_per_wg) * p.ksplit);
  dim3 block(64 * p.waves);
  const size_t lds = p.lds_bytes;
  if (p.xd) {
    GemmParams q = p;
    if (p.hxn) flags |= kGemmHandOver;
    if (p.xpre) {
      const hipError_t e = launch_rownorm(p, block, (flags & QDEC_NORM_IN) != 0, s);
      if (e != hipSuccess) return e;
      q.x = p.xn;
    }
    if (p.tw == 2) return mt == 2 ? launch_direct_tw2(q, flags, grid, block, lds, s) : hipErrorInvalidValue;
    if (p.tw != 1) return hipErrorInvalidValue;
    switch (mt) {
      case 1: return launch_direct_mt<1, 20, 10>(q, flags, grid, block, lds, s);
      case 2: return launch_direct_mt<2, 10, 5>(q, flags, grid, block, lds, s);
      case 3: return launch_direct_mt<3, 8, 6>(q, flags, grid, block, lds, s);
      case 4: return launch_direct_mt<4, 8, 4>(q, flags, grid, block, lds, s);
      default: return hipErrorInvalidValue;
    }
  }
  if (p.rw > 0) {
    if (mt != 1) return hipErrorInvalidValue;
    if (p.xfast && p.xparts) {  // one row merging a pending split residual update
      if (p.rows != 1 || p.xnparts > kMergeParts) return hipErrorInvalidValue;
      if (flags == QDEC_NORM_IN && p.rw == 20)
        hipLaunchKernelGGL((gemm_kernel<1, QDEC_NORM_IN, 20, false, 1, true>), grid, block, lds, s, p);
      else if (flags == QDEC_NORM_IN && p.rw == 16)
        hipLaunchKernelGGL((gemm_kernel<1, QDEC_NORM_IN, 16, false, 1, true>), grid, block, lds, s, p);
      else if (flags == (QDEC_NORM_IN | QDEC_ARGMAX) && p.rw == 20)
        hipLaunchKernelGGL((gemm_kernel<1, QDEC_NORM_IN | QDEC_ARGMAX, 20, false, 1, true>), grid, block, lds, s, p);
      else if (flags == (QDEC_NORM_IN | QDEC_ARGMAX) && p.rw == 16)
        hipLaunchKernelGGL((gemm_kernel<1, QDEC_NORM_IN | QDEC_ARGMAX, 16, false, 1, true>), grid, block, lds, s, p);
      else
        return hipErrorInvalidValue;
      return hipSuccess;
    }
    if (p.xfast && p.rows > kFastRows) {  // 5..8 rows under NORM_IN (no GLU) from registers
      constexpr int R8 = kFastRowsNorm;
      if (flags == QDEC_NORM_IN && p.rw == 20)
        hipLaunchKernelGGL((gemm_kernel<1, QDEC_NORM_IN, 20, false, R8>), grid, block, lds, s, p);
      else if (flags == QDEC_NORM_IN && p.rw == 16)
        hipLaunchKernelGGL((gemm_kernel<1, QDEC_NORM_IN, 16, false, R8>), grid, block, lds, s, p);
      else if (flags == (QDEC_NORM_IN | QDEC_ARGMAX) && p.rw == 20)
        hipLaunchKernelGGL((gemm_kernel<1, QDEC_NORM_IN | QDEC_ARGMAX, 20, false, R8>), grid, block, lds, s, p);
      else if (flags == (QDEC_NORM_IN | QDEC_ARGMAX) && p.rw == 16)
        hipLaunchKernelGGL((gemm_kernel<1, QDEC_NORM_IN | QDEC_ARGMAX, 16, false, R8>), grid, block, lds, s, p);
      else
        return hipErrorInvalidValue;
      return hipSuccess;
    }
    if (flags == (QDEC_NORM_IN | QDEC_GLU)) {
      if (p.rw != 10) return hipErrorInvalidValue;
      hipLaunchKernelGGL((gemm_kernel<1, QDEC_NORM_IN | QDEC_GLU, 10, false>), grid, block, lds, s, p);
      return hipSuccess;
    }
    switch (p.rw) {
      case 16: return launch_flags<1, 16>(p, flags, grid, block, lds, s);
      case 20: return launch_flags<1, 20>(p, flags, grid, block, lds, s);
      default: return hipErrorInvalidValue;
    }
  }
  if (p.xfast && p.rows > kFastRows) return hipErrorInvalidValue;  // the pass kernels stage kFastRows from registers
  switch (mt) {
    case 1: return launch_pass<1>(p, flags, grid, block, lds, s);
    case 2: return launch_pass<2>(p, flags, grid, block, lds, s);
    case 3: return launch_pass<3>(p, flags, grid, block, lds, s);
    case 4: return launch_pass<4>(p, flags, grid, block, lds, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qdec
