// Weight-streaming skinny GEMM for the decode step: y = x' . W^T, 1..64 rows.
//
// One workgroup owns one 16-column output tile (or several, for the lm_head)
// and a contiguous k range; its waves split that range into equal contiguous
// pieces.  Each wave streams its part of the tiled weight -- one 1 KiB block
// per k step, one 16-byte load per lane -- straight into the A operand of
// v_mfma_f32_16x16x32_bf16, while the activations (normalised on the way in
// when NORM_IN) are staged once per workgroup in LDS and read as the B
// operand.  The product is computed transposed (y^T = W . x'^T), so a lane
// ends up holding 4 consecutive output columns of one row.
//
// Latency: the first pass's weight loads are issued before anything else;
// for small row counts the activations are then loaded once into registers
// (statistics and LDS staging come from those registers), so the norm
// prologue overlaps the weight stream instead of preceding it.  With several
// tiles per workgroup the next tile's weights are requested before the
// current tile's epilogue.
//
// Summation order of an output element: MFMA chain over the wave's k steps in
// increasing order, then waves 0..W-1 added in order, then k splits 0..S-1
// added in order by the workgroup that arrives last.  The RMSNorm statistic
// of a row is summed by thread t over the row's 16-byte vectors t, t+T, ...
// and then across lanes and waves in a fixed tree, whatever the path.  None
// of it depends on the number of rows, which is what lets a verify pass over
// B*T rows reproduce the plain B-row step bit for bit.
//
// Reference behaviour replaced: engine/kernels/fused.py:33-235 (_gemv_kernel,
// _gemv_vec_kernel, _gemv_splitk_kernel + reduce) and the lm_head + argmax of
// engine/engine.py:492-498, 542-545.
#include "gemm_dev.h"

namespace qdec {

namespace {

template <int MT, uint32_t FLAGS>
__global__ void __launch_bounds__(512) gemm_kernel(const GemmParams p) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint4 wbuf[kWbuf];
  gemm_block<MT, FLAGS, false>(p, blockIdx.x, gridDim.x, smem, wbuf, false);
}

template <int MT>
hipError_t launch_mt(const GemmParams &p, uint32_t flags, dim3 grid, dim3 block, size_t lds,
                     hipStream_t s) {
  switch (flags) {
    case 0:
      hipLaunchKernelGGL((gemm_kernel<MT, 0u>), grid, block, lds, s, p);
      break;
    case QDEC_NORM_IN:
      hipLaunchKernelGGL((gemm_kernel<MT, QDEC_NORM_IN>), grid, block, lds, s, p);
      break;
    case QDEC_NORM_IN | QDEC_GLU:
      hipLaunchKernelGGL((gemm_kernel<MT, QDEC_NORM_IN | QDEC_GLU>), grid, block, lds, s, p);
      break;
    case QDEC_RES_OUT:
      hipLaunchKernelGGL((gemm_kernel<MT, QDEC_RES_OUT>), grid, block, lds, s, p);
      break;
    case QDEC_NORM_IN | QDEC_ARGMAX:
      hipLaunchKernelGGL((gemm_kernel<MT, QDEC_NORM_IN | QDEC_ARGMAX>), grid, block, lds, s, p);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipSuccess;
}

}  // namespace

bool gemm_flags_supported(uint32_t flags) {
  return flags == 0u || flags == QDEC_NORM_IN || flags == (QDEC_NORM_IN | QDEC_GLU) ||
         flags == QDEC_RES_OUT || flags == (QDEC_NORM_IN | QDEC_ARGMAX);
}

bool gemm_fast_path(const GemmParams &p, uint32_t flags) {
  const int per_row = p.ksw * p.waves * 4;
  return p.lds_all && p.rows <= kFastRows && per_row <= kFastVec * 64 * p.waves &&
         (!(flags & QDEC_NORM_IN) || p.ksplit == 1);
}

hipError_t launch_gemm(const GemmParams &p, uint32_t flags, hipStream_t s) {
  const int mt = (p.rows + 15) / 16;
  const int ntiles = p.n / 16;
  dim3 grid((ntiles / p.tiles_per_wg) * p.ksplit);
  dim3 block(64 * p.waves);
  const size_t lds = p.lds_bytes;
  switch (mt) {
    case 1: return launch_mt<1>(p, flags, grid, block, lds, s);
    case 2: return launch_mt<2>(p, flags, grid, block, lds, s);
    case 3: return launch_mt<3>(p, flags, grid, block, lds, s);
    case 4: return launch_mt<4>(p, flags, grid, block, lds, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qdec
