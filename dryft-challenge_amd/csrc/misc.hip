// Small kernels of the decode step: weight tiling, embedding gather, and the
// n-gram drafter / acceptance of speculative decoding.
#include "qdec_common.h"
#include "qdec_kernels.h"

namespace qdec {

namespace {

// dst vector v (16 bytes) = lane (v % 64) of block (v / 64).
__global__ void pack_kernel(const uint4 *__restrict__ src, uint4 *__restrict__ dst, int64_t n,
                            int64_t k) {
  const int64_t KS = k / 32;
  const int64_t total = (n / 16) * KS * 64;
  for (int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; v < total;
       v += (int64_t)gridDim.x * blockDim.x) {
    const int lane = (int)(v & 63);
    const int64_t blk = v >> 6;
    const int64_t nt = blk / KS;
    const int64_t ks = blk - nt * KS;
    const int64_t row = nt * 16 + (lane & 15);
    const int64_t kk = ks * 32 + (lane >> 4) * 8;
    dst[v] = src[(row * k + kk) >> 3];
  }
}

// h[m] = E[ids[m]] from the tiled embedding (the tied lm_head weight).
// Reference: engine/kernels/fused.py:341-350 (_embed_kernel).
__global__ void embed_kernel(const int64_t *__restrict__ ids, const uint4 *__restrict__ emb,
                             uint4 *__restrict__ h, int hidden, int vocab) {
  const int m = blockIdx.x;
  const int64_t id = ids[m];
  const int KS = hidden / 32;
  const int nvec = hidden / 8;
  if (id < 0 || id >= vocab) {
    // Never read outside the table; the row becomes NaN, so the step's
    // argmax yields an out-of-vocabulary id that the host refuses.
    for (int j = threadIdx.x; j < nvec; j += blockDim.x)
      h[(size_t)m * nvec + j] = make_uint4(0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u);
    return;
  }
  const int64_t nt = id >> 4;
  const int r = (int)(id & 15);
  for (int j = threadIdx.x; j < nvec; j += blockDim.x) {
    const int ks = j >> 2;
    const int lane = r + 16 * (j & 3);
    h[(size_t)m * nvec + j] = emb[((size_t)nt * KS + ks) * 64 + lane];
  }
}

// One workgroup per sequence.  Reference: notes/v10/spec.py:36-97.
__global__ void draft_kernel(const int64_t *__restrict__ hist, const int32_t *__restrict__ lens,
                             int64_t *__restrict__ ids, int64_t *__restrict__ draft, int cap,
                             int primary, int backoff, int K) {
  __shared__ int s_best[2][4];
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int T = K + 1;
  const int64_t *h = hist + (size_t)b * cap;
  int L = lens[b];
  if (L < 0) L = 0;
  if (L >= cap) L = cap - 1;  // a frozen or corrupt length never reads out of the row
  const int ngram[2] = {primary, backoff};
  int best[2] = {-1, -1};
  for (int which = 0; which < 2 && K > 0; ++which) {  // k = 0: feed the current token only
    const int n = ngram[which];
    const int limit = min(L - n - K + 2, cap);
    int mine = -1;
    for (int j = tid; j < limit; j += blockDim.x) {
      bool ok = true;
      for (int i = 0; i < n && ok; ++i) {
        const int pat_at = max(L - n + 1 + i, 0);
        ok = (h[j + i] == h[pat_at]);
      }
      if (ok) mine = j;  // j increases per thread, so this is the thread's latest
    }
    for (int off = 32; off >= 1; off >>= 1) mine = max(mine, __shfl_xor(mine, off, 64));
    if (lane == 0) s_best[which][wave] = mine;
    __syncthreads();
    int v = -1;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) v = max(v, s_best[which][w]);
    best[which] = v;
    __syncthreads();
  }
  const bool has_primary = best[0] >= 0;
  const int pick = has_primary ? best[0] : best[1];
  const int n = has_primary ? primary : backoff;
  if (tid == 0) ids[(size_t)b * T] = h[L];
  for (int t = tid; t < K; t += blockDim.x) {
    const int64_t tok = (pick >= 0) ? h[pick + n + t] : 0;
    draft[(size_t)b * K + t] = tok;
    ids[(size_t)b * T + 1 + t] = tok;
  }
}

// One thread per sequence.  Reference: notes/v10/spec.py:185-214.
__global__ void accept_kernel(const int64_t *__restrict__ out_tok, const int64_t *__restrict__ draft,
                              int64_t *__restrict__ hist, int32_t *__restrict__ lens,
                              int32_t *__restrict__ naccept, int batch, int cap, int K,
                              int stop_len) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= batch) return;
  const int T = K + 1;
  const int L = lens[b];
  int a = 0, run = 1;
  for (int t = 0; t < K; ++t) {
    run = run * ((out_tok[(size_t)b * T + t] == draft[(size_t)b * K + t]) ? 1 : 0);
    a += run;
  }
  const bool live = L < stop_len;
  if (!live) a = 0;
  if (live) {
    for (int t = 0; t <= a; ++t) {
      const int idx = L + 1 + t;
      if (idx >= 0 && idx < cap) hist[(size_t)b * cap + idx] = out_tok[(size_t)b * T + t];
    }
  }
  naccept[b] = a;
  lens[b] = L + (live ? a + 1 : 0);
}

// Streaming-read ceiling of the device: every 16-byte vector of `buf` is read
// once with the non-temporal hint (like the weight loads of the step), eight
// loads in flight per thread; the XOR of everything is stored only if it
// equals a value it never takes here, so no load can be optimised away.
__global__ void __launch_bounds__(256) read_kernel(const uint4 *__restrict__ buf, int64_t nvec,
                                                   uint32_t *__restrict__ sink) {
  const int64_t per_block = (nvec + gridDim.x - 1) / gridDim.x;
  const int64_t v0 = (int64_t)blockIdx.x * per_block;
  const int64_t v1 = min(v0 + per_block, nvec);
  uint32_t acc = 0u;
  for (int64_t v = v0 + threadIdx.x; v < v1; v += 8 * 256) {
    uint4 r[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t i = v + (int64_t)j * 256;
      r[j] = i < v1 ? ld_nt(buf + i) : zero4();
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) acc ^= r[j].x ^ r[j].y ^ r[j].z ^ r[j].w;
  }
  if (acc == 0x9e3779b9u && threadIdx.x == 0) sink[blockIdx.x] = acc;
}

}  // namespace

hipError_t launch_read(const void *buf, int64_t bytes, uint32_t *sink, int blocks, hipStream_t s) {
  hipLaunchKernelGGL(read_kernel, dim3(blocks), dim3(256), 0, s, reinterpret_cast<const uint4 *>(buf), bytes / 16,
                     sink);
  return hipSuccess;
}

hipError_t launch_pack(const void *src, void *dst, int64_t n, int64_t k, hipStream_t s) {
  const int64_t total = (n / 16) * (k / 32) * 64;
  const int64_t blocks = std::min<int64_t>((total + 255) / 256, 65536);
  hipLaunchKernelGGL(pack_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                     reinterpret_cast<const uint4 *>(src), reinterpret_cast<uint4 *>(dst), n, k);
  return hipSuccess;
}

hipError_t launch_embed(const int64_t *ids, const void *emb, void *h, int rows, int hidden,
                        int vocab, hipStream_t s) {
  hipLaunchKernelGGL(embed_kernel, dim3(rows), dim3(256), 0, s, ids,
                     reinterpret_cast<const uint4 *>(emb), reinterpret_cast<uint4 *>(h), hidden,
                     vocab);
  return hipSuccess;
}

hipError_t launch_draft(const int64_t *hist, const int32_t *lens, int64_t *ids, int64_t *draft,
                        int batch, int cap, int primary, int backoff, int k, hipStream_t s) {
  hipLaunchKernelGGL(draft_kernel, dim3(batch), dim3(256), 0, s, hist, lens, ids, draft, cap,
                     primary, backoff, k);
  return hipSuccess;
}

hipError_t launch_accept(const int64_t *out_tok, const int64_t *draft, int64_t *hist,
                         int32_t *lens, int32_t *naccept, int batch, int cap, int k, int stop_len,
                         hipStream_t s) {
  hipLaunchKernelGGL(accept_kernel, dim3((batch + 63) / 64), dim3(64), 0, s, out_tok, draft, hist,
                     lens, naccept, batch, cap, k, stop_len);
  return hipSuccess;
}

}  // namespace qdec
