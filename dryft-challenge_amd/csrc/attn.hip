// Launcher of the GQA decode attention (head RMSNorm, RoPE and KV-cache
// write fused in; t_rows query rows per sequence: 1 = plain decode, K+1 =
// verify).  The kernel body and its dataflow are attn_block in attn_dev.h;
// this file instantiates it per (head_dim, query heads per kv head, query
// M tiles, waves) and picks the instantiation from the call.
//
// Reference behaviour replaced: engine/kernels/fused.py:360-479
// (_attn_fused_split_kernel), engine/kernels/ops.py:84-431 (_qkv_post_kernel,
// _decode_attn_split_kernel, _decode_attn_reduce_kernel) and
// notes/v10/spec.py:111-182 (_spec_attn_kernel).
#include "attn_dev.h"

namespace qdec {

namespace {

// Up to 32 query rows per kv head the body fits 256 registers without
// spills: two 4-wave workgroups per CU, or one of 8 waves.
template <int D, int GQ, int MTQ, int NW, bool STR = false>
__global__ void __launch_bounds__(64 * NW, NW == 4 && MTQ <= 2 ? 2 : 1) attn_kernel(const AttnParams p) {
  __shared__ __align__(16) unsigned char smem[AttnLds<NW>::bytes];
  attn_block<D, GQ, MTQ, NW, false, STR>(p, blockIdx.x, blockIdx.y, blockIdx.z, smem);
}

}  // namespace

template <int GQ>
hipError_t launch_attn_g(const AttnParams &p, int mtq, dim3 grid, dim3 block, hipStream_t s) {
  if (p.waves == 8) {
    switch (mtq * 2 + (p.strided ? 1 : 0)) {
      case 2: hipLaunchKernelGGL((attn_kernel<128, GQ, 1, 8>), grid, block, 0, s, p); break;
      case 3: hipLaunchKernelGGL((attn_kernel<128, GQ, 1, 8, true>), grid, block, 0, s, p); break;
      case 4: hipLaunchKernelGGL((attn_kernel<128, GQ, 2, 8>), grid, block, 0, s, p); break;
      case 5: hipLaunchKernelGGL((attn_kernel<128, GQ, 2, 8, true>), grid, block, 0, s, p); break;
      default: return hipErrorInvalidValue;
    }
    return hipSuccess;
  }
  if (p.strided) return hipErrorInvalidValue;  // strided chunks run 8 waves
  switch (mtq) {
    case 1: hipLaunchKernelGGL((attn_kernel<128, GQ, 1, 4>), grid, block, 0, s, p); break;
    case 2: hipLaunchKernelGGL((attn_kernel<128, GQ, 2, 4>), grid, block, 0, s, p); break;
    case 3: hipLaunchKernelGGL((attn_kernel<128, GQ, 3, 4>), grid, block, 0, s, p); break;
    case 4: hipLaunchKernelGGL((attn_kernel<128, GQ, 4, 4>), grid, block, 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipSuccess;
}

hipError_t launch_attn(const AttnParams &p, hipStream_t s) {
  const int R = p.t_rows * (p.nq / p.nkv);
  const int mtq = (R + 15) / 16;
  dim3 grid(p.nchunks, p.nkv, p.batch);
  dim3 block(64 * p.waves);
  if (p.head_dim == 64) {  // four waves, group size from p
    if (p.waves != 4) return hipErrorInvalidValue;
    switch (mtq) {
      case 1: hipLaunchKernelGGL((attn_kernel<64, 0, 1, 4>), grid, block, 0, s, p); break;
      case 2: hipLaunchKernelGGL((attn_kernel<64, 0, 2, 4>), grid, block, 0, s, p); break;
      case 3: hipLaunchKernelGGL((attn_kernel<64, 0, 3, 4>), grid, block, 0, s, p); break;
      case 4: hipLaunchKernelGGL((attn_kernel<64, 0, 4, 4>), grid, block, 0, s, p); break;
      default: return hipErrorInvalidValue;
    }
    return hipSuccess;
  }
  // 4 query heads per kv head as a constant; other group sizes read it from p
  return p.nq == 4 * p.nkv ? launch_attn_g<4>(p, mtq, grid, block, s) : launch_attn_g<0>(p, mtq, grid, block, s);
}

}  // namespace qdec
