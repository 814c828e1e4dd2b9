// One decode layer in one launch: QKV (input RMSNorm folded in), attention
// (head norm, RoPE and the cache write folded in, chunk partials left for O),
// O (merging the partials, residual add), gate/up (post-attention RMSNorm,
// SwiGLU) and down (residual add) as the stages of a single kernel.
//
// The launch has at most as many workgroups as fit the GPU at once (all
// resident); in each stage workgroup i runs block i of that stage, exactly
// the per-block code of the stage's own launch (gemm_dev.h, attn_dev.h)
// under its 4-wave plan, so a layer computes what the five launches of those
// plans compute.  What one stage hands to the next (the projection rows, the
// attention partials, the residual O updates, the SwiGLU activations) is
// written and read at device scope (the bodies' COH accesses): another XCD's
// L2 never serves a stale copy, and no cache-wide fence is needed, which on
// MI355X costs 8-16 us per barrier against 3.3 for the barrier itself.
// Between stages a grid barrier:
//  * every thread waits for its own stores to complete, the workgroup meets,
//    and one thread arrives at its group's ticket (workgroup w at group
//    w % 8); the last of a group arrives at the top ticket, waits for all
//    groups, then releases its group; the others wait for that release.
//    Every workgroup passes every barrier, whether or not it had a block in
//    the stage before;
//  * the tickets only grow: a group's n-th arrival belongs to its barrier
//    n / (group size), so nothing is ever reset;
//  * the waits are bounded: after spin_limit polls a workgroup sets the
//    error word and goes on, and every later wait gives up as soon as it sees
//    the word, so a launch that cannot have all its workgroups resident ends
//    with wrong numbers and a flag the host reads, never with a hang.
//
// Reference behaviour replaced: engine/kernels/layer.py:46-66
// (_arrive_and_wait: flag barriers with a SPIN_LIMIT) and :69-285
// (_layer_kernel, the five stages of a layer in one launch).
#include "attn_dev.h"
#include "gemm_dev.h"

namespace qdec {
namespace {

static_assert(kLayerMaxRows == kFastRows, "GEMM stages stage their rows from registers");

// Polls *p until it reaches target; false (and the error word set) when the
// wait gives up.
__device__ __forceinline__ bool wait_at_least(uint64_t *p, uint64_t target, LayerCtl *ctl, uint32_t spin_limit) {
  uint32_t polls = 0;
  while (__hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
    if (++polls > spin_limit) {
      __hip_atomic_store(&ctl->err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
    if ((polls & 255u) == 1u && __hip_atomic_load(&ctl->err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u)
      return false;
    __builtin_amdgcn_s_sleep(1);
  }
  return true;
}

__device__ __forceinline__ void layer_barrier(LayerCtl *ctl, uint32_t nwg, uint32_t spin_limit) {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);  // this thread's device-scope stores have completed
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  if (threadIdx.x == 0) {
    LayerCtl::Group &g = ctl->group[blockIdx.x % kLayerGroups];
    const uint64_t per_group = nwg / kLayerGroups;
    const uint64_t t = __hip_atomic_fetch_add(&g.arrive, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t round = t / per_group;
    if (t % per_group == per_group - 1) {
      const uint64_t u = __hip_atomic_fetch_add(&ctl->ticket, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      wait_at_least(&ctl->ticket, (u / kLayerGroups + 1) * kLayerGroups, ctl, spin_limit);
      __hip_atomic_fetch_add(&g.release, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    wait_at_least(&g.release, round + 1, ctl, spin_limit);
  }
  __syncthreads();
}

// Stage plans (api.hip checks every call against them): QKV NORM_IN from
// registers with a 20-block ring; O merging the attention partials, 16-block
// ring; gate/up NORM_IN + GLU, 10 block pairs; down with its activations read
// straight from x, 20-block ring; attention 4 waves, one M tile of queries.
__global__ void __launch_bounds__(kLayerThreads, 2)
    layer_kernel(const LayerParams *__restrict__ P, const uint64_t key, LayerCtl *ctl, const uint32_t spin_limit) {
  extern __shared__ __align__(16) unsigned char smem[];
  // A plan written for other arguments: nothing runs, the error word says 2.
  if (P->key != key) {
    if (blockIdx.x == 0 && threadIdx.x == 0)
      __hip_atomic_store(&ctl->err, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  // The tickets count arrivals per group of gridDim.x / 8 workgroups: a ctl
  // keeps the count of its first launch, and a launch of another size runs
  // nothing (every workgroup sees the same recorded count) and says 3.
  // (The word goes through the dynamic LDS, which no stage has touched yet:
  // a static array would add to every workgroup's LDS and halve residency.)
  uint32_t *s_nwg = reinterpret_cast<uint32_t *>(smem);
  if (threadIdx.x == 0) {
    uint32_t want = 0u;
    __hip_atomic_compare_exchange_strong(&ctl->nwg, &want, gridDim.x, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    *s_nwg = want == 0u ? gridDim.x : want;  // on failure `want` holds the recorded count
    if (*s_nwg != gridDim.x) __hip_atomic_store(&ctl->err, 3u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  const bool same_count = *s_nwg == gridDim.x;
  __syncthreads();  // every wave has read the word before the first stage writes LDS
  if (!same_count) return;
  // Every stage has at most one block per workgroup (the host admits no
  // more blocks than workgroups): a loop over blocks would keep its state
  // live across the body, and the attention body would spill.
  const int G = gridDim.x;
  if ((int)blockIdx.x < P->nblk[0]) gemm_body<1, QDEC_NORM_IN, 20, false, kFastRows, false, 1, true>(P->g[0], blockIdx.x, P->nblk[0], smem);
  layer_barrier(ctl, G, spin_limit);
  {
    const AttnParams &a = P->a;
    const int nc = a.nchunks, u = blockIdx.x;
    if (u < nc * a.nkv * a.batch) {
      const int r = u / nc;
      attn_block<128, 4, 1, 4, true>(a, u - r * nc, r % a.nkv, r / a.nkv, smem);
    }
  }
  layer_barrier(ctl, G, spin_limit);
  if ((int)blockIdx.x < P->nblk[1]) gemm_body<1, QDEC_RES_OUT, 16, false, kFastRows, false, 1, true>(P->g[1], blockIdx.x, P->nblk[1], smem);
  layer_barrier(ctl, G, spin_limit);
  if ((int)blockIdx.x < P->nblk[2]) gemm_body<1, QDEC_NORM_IN | QDEC_GLU, 10, false, kFastRows, false, 1, true>(P->g[2], blockIdx.x, P->nblk[2], smem);
  layer_barrier(ctl, G, spin_limit);
  if ((int)blockIdx.x < P->nblk[3]) gemm_body<1, QDEC_RES_OUT, 20, true, kFastRows, false, 1, true>(P->g[3], blockIdx.x, P->nblk[3], smem);
}

}  // namespace

size_t layer_attn_lds_bytes() { return AttnLds<4>::bytes; }

hipError_t layer_workgroups(size_t lds_bytes, int *out) {
  int dev = 0, cus = 0, per_cu = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e == hipSuccess)
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, layer_kernel, kLayerThreads, lds_bytes);
  if (e != hipSuccess) return e;
  *out = cus * per_cu;
  return hipSuccess;
}

hipError_t launch_layer(const LayerParams *plan, uint64_t key, LayerCtl *ctl, uint32_t spin_limit, int workgroups,
                        size_t lds_bytes, hipStream_t s) {
  hipLaunchKernelGGL(layer_kernel, dim3(workgroups), dim3(kLayerThreads), lds_bytes, s, plan, key, ctl, spin_limit);
  return hipSuccess;
}

}  // namespace qdec
