// Persistent decode-step kernel: a whole forward (embed, 36 x [QKV, attention,
// O, gate/up, down], lm_head + argmax) in one launch.
//
// One workgroup per CU walks a table of phases prepared on the host
// (qdec_step_encode_*).  Inside a phase the workgroups take the phase's blocks
// round robin and run exactly the per-block code of the standalone kernels
// (gemm_block / attn_block), so the results are bit-identical to the
// multi-kernel path.  Between phases a grid barrier; before waiting on it,
// every workgroup issues the weight loads of its first block of the next
// phase, so the weight stream does not drain while the activations of the
// previous phase settle.
//
// Coherence inside the launch: activations are written and read with
// cache-bypassing accesses (COH = true in the block code); weights, norm
// vectors, rotary tables and KV-cache slots written by earlier launches are
// read normally.  The barrier is a 64-bit arrival ticket in device memory,
// touched only with device-scope atomics, with a bounded spin: a
// workgroup that waits longer than `spin_limit` polls sets the error word,
// after which every workgroup runs to the end without waiting (the host
// checks the word and raises), so a scheduling failure can never hang the
// device.
//
// Reference behaviour replaced: the per-step graph of launches of
// engine/engine.py:517-546 (_decode_step_fused) and the one-launch layer
// of engine/kernels/layer.py:46-285 (flag barriers with SPIN_LIMIT).
#include "attn_dev.h"
#include "gemm_dev.h"

namespace qdec {

namespace {

__device__ __forceinline__ void embed_block(const StepEmbed &e, int m) {
  int64_t id = e.ids[m];
  if (id < 0 || id >= e.vocab) id = 0;
  const int KS = e.hidden / 32;
  const int nvec = e.hidden / 8;
  const int64_t nt = id >> 4;
  const int r = (int)(id & 15);
  const uint4 *emb = reinterpret_cast<const uint4 *>(e.emb);
  uint16_t *h = reinterpret_cast<uint16_t *>(e.h);
  for (int j = threadIdx.x; j < nvec; j += blockDim.x) {
    const int ks = j >> 2;
    const int lane = r + 16 * (j & 3);
    st16<true>(h + ((size_t)m * nvec + j) * 8, emb[((size_t)nt * KS + ks) * 64 + lane]);
  }
}

// Ticket grid barrier (see the file comment): one device-scope atomic per
// workgroup, then polls until every workgroup of this barrier has arrived.
// The 64-bit ticket only grows, so nothing is ever reset.
__device__ __forceinline__ void grid_barrier(StepCtl *ctl, uint32_t nwg, uint32_t spin_limit) {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);  // this thread's stores have completed
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint64_t t = __hip_atomic_fetch_add(&ctl->ticket, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t target = (t / nwg + 1) * nwg;
    uint32_t it = 0;
    while (__hip_atomic_load(&ctl->ticket, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
      if (++it > spin_limit) {
        __hip_atomic_store(&ctl->err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      if ((it & 1023u) == 0u &&
          __hip_atomic_load(&ctl->err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u)
        break;
      __builtin_amdgcn_s_sleep(1);
    }
  }
  __syncthreads();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

template <int MT>
__device__ __forceinline__ bool run_gemm(const GemmParams &g, uint32_t flags, int blk, int nblk,
                                         unsigned char *smem, uint4 (&wbuf)[kWbuf], bool have, int next) {
  switch (flags) {
    case 0u: return gemm_block<MT, 0u, true>(g, blk, nblk, smem, wbuf, have, next);
    case QDEC_NORM_IN: return gemm_block<MT, QDEC_NORM_IN, true>(g, blk, nblk, smem, wbuf, have, next);
    case QDEC_NORM_IN | QDEC_GLU:
      return gemm_block<MT, QDEC_NORM_IN | QDEC_GLU, true>(g, blk, nblk, smem, wbuf, have, next);
    case QDEC_RES_OUT: return gemm_block<MT, QDEC_RES_OUT, true>(g, blk, nblk, smem, wbuf, have, next);
    case QDEC_NORM_IN | QDEC_ARGMAX:
      return gemm_block<MT, QDEC_NORM_IN | QDEC_ARGMAX, true>(g, blk, nblk, smem, wbuf, have, next);
    default: return false;
  }
}

__device__ __forceinline__ void prefetch_gemm(const GemmParams &g, uint32_t flags, int blk,
                                              uint4 (&wbuf)[kWbuf]) {
  if (flags & QDEC_GLU) gemm_prefetch<QDEC_NORM_IN | QDEC_GLU>(g, blk, wbuf);
  else gemm_prefetch<0u>(g, blk, wbuf);
}

template <int MT, int MTQ>
__global__ void __launch_bounds__(256) step_kernel(const StepPhase *__restrict__ phases, int nphases,
                                                    StepCtl *ctl, uint32_t spin_limit, uint64_t *trace) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint4 wbuf[kWbuf];
  bool have = false;
  const int nwg = gridDim.x;
  for (int i = 0; i < nphases; ++i) {
    const StepPhase &P = phases[i];
    const int kind = P.kind;
    const int nblk = P.nblk;
    if (trace && threadIdx.x == 0) trace[((size_t)blockIdx.x * nphases + i) * 2] = __builtin_amdgcn_s_memrealtime();
    for (int blk = blockIdx.x; blk < nblk; blk += nwg) {
      if (kind == kPhaseGemm) {
        if (P.g.rows > 16 * MT) {  // table built for more rows than this launch holds
          if (threadIdx.x == 0) __hip_atomic_store(&ctl->err, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        const int next = blk + nwg < nblk ? blk + nwg : -1;
        have = run_gemm<MT>(P.g, P.flags, blk, nblk, smem, wbuf, have, next);
      } else if (kind == kPhaseAttn) {
        if (P.a.t_rows * 4 > 16 * MTQ) {
          if (threadIdx.x == 0) __hip_atomic_store(&ctl->err, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        const int nc = P.a.nchunks;
        const int c = blk % nc;
        const int bk = blk / nc;
        attn_block<128, 4, MTQ, true>(P.a, c, bk % P.a.nkv, bk / P.a.nkv, smem);
        have = false;
      } else {
        embed_block(P.e, blk);
        have = false;
      }
    }
    if (i + 1 < nphases) {
      const StepPhase &Q = phases[i + 1];
      if (Q.kind == kPhaseGemm && (int)blockIdx.x < Q.nblk) {
        prefetch_gemm(Q.g, Q.flags, blockIdx.x, wbuf);
        have = true;
      } else {
        have = false;
      }
      if (trace && threadIdx.x == 0) trace[((size_t)blockIdx.x * nphases + i) * 2 + 1] = __builtin_amdgcn_s_memrealtime();
      grid_barrier(ctl, (uint32_t)nwg, spin_limit);
    } else if (trace && threadIdx.x == 0) {
      trace[((size_t)blockIdx.x * nphases + i) * 2 + 1] = __builtin_amdgcn_s_memrealtime();
    }
  }
}

template <int MT>
hipError_t launch_mtq(int mtq, const StepPhase *phases, int nphases, StepCtl *ctl, uint32_t spin_limit,
                      int nwg, size_t lds, uint64_t *trace, hipStream_t s) {
  switch (mtq) {
    case 1: hipLaunchKernelGGL((step_kernel<MT, 1>), dim3(nwg), dim3(256), lds, s, phases, nphases, ctl, spin_limit, trace); break;
    case 2: hipLaunchKernelGGL((step_kernel<MT, 2>), dim3(nwg), dim3(256), lds, s, phases, nphases, ctl, spin_limit, trace); break;
    case 3: hipLaunchKernelGGL((step_kernel<MT, 3>), dim3(nwg), dim3(256), lds, s, phases, nphases, ctl, spin_limit, trace); break;
    case 4: hipLaunchKernelGGL((step_kernel<MT, 4>), dim3(nwg), dim3(256), lds, s, phases, nphases, ctl, spin_limit, trace); break;
    default: return hipErrorInvalidValue;
  }
  return hipSuccess;
}

}  // namespace

hipError_t launch_step(const StepPhase *phases, int nphases, StepCtl *ctl, uint32_t spin_limit, int mt,
                       int mtq, int nwg, size_t lds, uint64_t *trace, hipStream_t s) {
  switch (mt) {
    case 1: return launch_mtq<1>(mtq, phases, nphases, ctl, spin_limit, nwg, lds, trace, s);
    case 2: return launch_mtq<2>(mtq, phases, nphases, ctl, spin_limit, nwg, lds, trace, s);
    case 3: return launch_mtq<3>(mtq, phases, nphases, ctl, spin_limit, nwg, lds, trace, s);
    case 4: return launch_mtq<4>(mtq, phases, nphases, ctl, spin_limit, nwg, lds, trace, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qdec
