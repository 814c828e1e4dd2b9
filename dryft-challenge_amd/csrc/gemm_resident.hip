// Gate/up projection (NORM_IN | GLU) of a few rows with the normalised rows
// resident in LDS: one workgroup per compute unit.
//
// The per-operation call above its register-staged rows normalises the rows
// in a pre-pass launch, and each of its workgroups (one tile pair, 608 for
// Qwen3-4B, two or three per CU) then reads the whole normalised matrix from
// L2 as its MFMA B operands.  Here the grid is one workgroup per CU, each
// owning a contiguous run of tile pairs (two or three), and the workgroup
// normalises the raw rows itself, once, into LDS in fragment order; every
// wave then reads its B operands from LDS.  The pre-pass launch and the
// per-tile activation reads from L2 are gone.
//
// The arithmetic is the pre-pass + direct path's, step for step, so the
// output is bit-identical to it (and therefore row-invariant like it):
//  * the row statistic is the pre-pass's (rownorm_kernel at 256 threads):
//    virtual thread t sums the squares of vectors t and t + 256 of the row,
//    the 64 lanes of each virtual wave are added by wave_sum, and the four
//    virtual waves in order; here the workgroup's last four waves compute
//    virtual wave w % 4 of every row;
//  * x' = bf16(norm_w * bf16(x * rstd)) per element (norm8);
//  * wave q of a pair streams k steps [q ksw, (q + 1) ksw) of the pair's gate
//    and up tiles through an RW-slot register ring, the MFMA chain in k
//    order; the pair's four waves are added in wave order; then the SwiGLU
//    epilogue of the direct path.
// A pair's sums do not depend on which workgroup computes it, so the grid
// (the device's CU count) does not change a bit.
//
// Measured on MI355X (Qwen3-4B gate/up, 8 rows): 21.0 us per launch against
// 24.0 for the pre-pass and the direct call, and batch-8 decode 2.912 ->
// 2.797 ms per step (config 3, same box).
//
// NORM_IN alone (the QKV projection) runs the same kernel with GLU = false:
// single output tiles in place of the pairs, one or two per workgroup, and
// the plain bf16 epilogue (QKV at 8 rows: 11.5 -> 8.7 us per launch).
//
// Reference behaviour replaced: the NORM_IN + GLU path of
// engine/kernels/fused.py:33-172 (_gemv_kernel with the RMSNorm prologue and
// the SiLU-gated epilogue).
#include <algorithm>

#include "gemm_dev.h"

namespace qdec {
namespace {

constexpr int kResVThreads = 256;  // the pre-pass workgroup whose statistic order is followed

// Position of fragment slot `slot` (B operand lane: row slot % 16, k group
// slot / 16) within the LDS KiB of k step s.  A bijection of the 64 slots
// that XORs the row bits with the k group and s % 4: the 16 lanes of every
// group the LDS serves together then touch 16 different 16-byte bank groups,
// both when a lane of the MFMA reads its slot and when the normalisation
// writes a row's 16 consecutive vectors (in plain fragment order those all
// sit in one bank group: measured on MI355X, the writes took about 8 us per
// launch).
__device__ __forceinline__ int res_pos(int slot, int s) { return slot ^ (((slot >> 4) & 3) | ((s & 3) << 2)); }

// Polls of an LDS flag before a wave gives up waiting (a bound that a
// correct launch never reaches: the flags are set by waves of the same
// workgroup that wait on nothing but their own loads).
constexpr uint32_t kResSpin = 1u << 22;

__device__ __forceinline__ void res_wait(const uint32_t *flag, uint32_t target) {
  for (uint32_t i = 0; i < kResSpin; ++i) {
    if (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= target) break;
    __builtin_amdgcn_s_sleep(1);
  }
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// One arrival of this wave at an LDS flag, after its own LDS writes are done
// (s_waitcnt lgkmcnt(0)).
__device__ __forceinline__ void res_signal(uint32_t *flag) {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);
  if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Units of a gate/up workgroup owning the half pairs [h0, h1): half pair
// 2t + h is columns 8h .. 8h + 7 of gate tile t with the same columns of up
// tile t, and a half pair whose partner lies in the same range joins it as
// one whole pair.  Unit u of the walk: its pair and kind (0 whole pair,
// 1 + h half pair h), or false past the last unit.  With at most five half
// pairs per range a workgroup has at most three units.
__host__ __device__ inline bool res_unit(unsigned h0, unsigned h1, int u, unsigned &pair, int &kind) {
  unsigned h = h0;
  for (int i = 0; i < kResMaxPairs; ++i) {
    if (h >= h1) return false;
    const int kd = (h & 1u) ? 2 : (h + 2 <= h1 ? 0 : 1);
    if (i == u) {
      pair = h >> 1;
      kind = kd;
      return true;
    }
    h += kd == 0 ? 2u : 1u;
  }
  return false;
}

// Unit j of this workgroup: runs of half pairs (GLU with p.res_half), else
// a contiguous run of whole pairs (GLU) or tiles.  False when the workgroup
// has fewer units.
template <bool GLU>
__device__ __forceinline__ bool res_unit_of(const GemmParams &p, int j, unsigned &tile, int &kind) {
  const unsigned P = (unsigned)p.n >> 4;  // tile pairs (GLU) or tiles
  if (GLU && p.res_half) {
    const unsigned H = 2 * P;
    return res_unit(blockIdx.x * H / gridDim.x, (blockIdx.x + 1) * H / gridDim.x, j, tile, kind);
  }
  const unsigned u0 = blockIdx.x * P / gridDim.x;
  tile = u0 + j;
  kind = 0;
  return j < (int)((blockIdx.x + 1) * P / gridDim.x - u0);
}

// This lane's offset (16-byte units) within a k step's weight block: its
// own slot, or for half pair h the slot of row 8h + (row % 8) and the same
// k group in the gate block (rows below 8) or the up block (rows 8..15).
__device__ __forceinline__ size_t res_lane_off(bool half, int kind, int lane, size_t up_off) {
  if (!half) return (size_t)lane;
  const int col = lane & 15, grp = lane >> 4;
  return (col < 8 ? (size_t)0 : up_off) + (size_t)((col & 7) + 8 * (kind - 1) + 16 * grp);
}

// GLU: (gate, up) tile pairs and the SwiGLU epilogue; otherwise single
// tiles (NORM_IN alone: QKV) and a bf16 store.
//
// With p.res_half (GLU) a workgroup owns a run of half pairs instead of
// whole pairs (res_unit): 608 pairs over 256 CUs then put at most 2.5 pairs
// of weights on a CU instead of 3 (a read-only probe of the two launch
// shapes on MI355X: 16.5 against 18.3 us for gate/up's 99.6 MB).  A half
// pair's wave takes the MFMA A operand from two blocks -- rows 8h .. 8h+7
// of the gate block in lanes whose row is below 8, the same rows of the up
// block in the others, 128-byte runs of each -- so one MFMA chain gives the
// gate columns in lanes 0..31 and the up columns in lanes 32..63, and each
// output element's sum is the whole pair's, bit for bit (the MFMA's sum of
// one output does not depend on the row it sits in).  The unit's ring puts
// k steps i .. i+RW-1 in wg and i+RW .. i+2RW-1 in wu, issued in the same
// register order as a whole pair's, so the compiler's wait counts agree on
// both paths.
template <int RW, bool GLU>
__global__ void __launch_bounds__(64 * 4 * (GLU ? kResMaxPairs : kResMaxTiles1)) glu_resident_kernel(const GemmParams p) {
  constexpr int NA = GLU ? 2 : 1;
  __shared__ __align__(16) uint4 s_x[kResMaxKSteps * 64];                  // [k step][slot]
  __shared__ __align__(16) float4 s_red[kResMaxPairs * 3 * NA * 64];      // [unit][wave 1..3][gate, up][lane]
  __shared__ float s_part[kResMaxRows * 4];                               // [row][virtual wave]
  // Arrivals of the four normalising waves: [0] row loads issued, [1]
  // statistic partials written, [2] rows normalised into s_x.
  __shared__ uint32_t s_sync[3];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nw = p.res_waves;  // blockDim.x / 64, from the kernel arguments (a scalar load)
  const int rows = p.rows, k = p.k, KS = p.KS, ksw = p.ksw;
  const int col = lane & 15, grp = lane >> 4;
  const int j = wave >> 2, q = wave & 3;  // unit within the workgroup, k quarter
  unsigned tile = 0;
  int kind = 0;  // 0 a whole pair (or tile), 1 + h half pair h
  const bool active = res_unit_of<GLU>(p, j, tile, kind);
  const bool half = GLU && kind != 0;
  if (tid == 0) s_sync[0] = s_sync[1] = s_sync[2] = 0u;
  __syncthreads();

  const uint4 *W = reinterpret_cast<const uint4 *>(p.w);
  const size_t up_off = (size_t)p.up_tiles * KS * 64;
  const int ksw_w = active ? ksw : 0;
  const uint4 *wq = W + ((size_t)(active ? tile : 0) * KS + (size_t)q * ksw) * 64 + res_lane_off(half, kind, lane, up_off);
  // wu[r]'s block: the up tile's, or (half pair) RW k steps on
  const size_t second = half ? (size_t)RW * 64 : up_off;
  uint4 wg[RW], wu[GLU ? RW : 1];
  // The first RW k steps of this wave's range (2 RW for a half pair).
  auto issue_ring = [&]() {
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      wg[r] = ldw(wq + r * 64);
      if constexpr (GLU) wu[r] = ldw(wq + r * 64 + second);
    }
  };

  // Two roles, so that the weight stream starts at once and the
  // normalisation still runs at full speed (measured on MI355X: a wave that
  // has issued its ring stalls in the issue of those loads for several us,
  // and every instruction behind them waits with it).
  //  * the last four waves (pair nw/4 - 1, or no pair at all in a workgroup
  //    with fewer pairs) load the rows, compute the statistic and write the
  //    normalised rows to LDS, and only then issue their own ring;
  //  * every other wave issues its ring as soon as the row loads have gone
  //    out ahead of it, and waits for the rows.
  if (wave >= nw - 4) {
    // Virtual wave vw = wave % 4 of every row: lane l holds vectors
    // vw * 64 + l and vw * 64 + l + 256 of the row.  Loads are unconditional
    // (clamped to a valid address, the value discarded).
    const int vw = wave & 3;
    const int v0 = vw * 64 + lane, v1 = v0 + kResVThreads;
    const bool ok0 = v0 < (k >> 3), ok1 = v1 < (k >> 3);
    const int c0 = ok0 ? v0 : 0, c1 = ok1 ? v1 : 0;
    const uint16_t *X = reinterpret_cast<const uint16_t *>(p.x);
    const uint16_t *NW = reinterpret_cast<const uint16_t *>(p.norm_w);
    uint4 xa[kResMaxRows], xb[kResMaxRows];
#pragma unroll
    for (int m = 0; m < kResMaxRows; ++m) {
      const uint16_t *xr = X + (size_t)(m < rows ? m : 0) * k;
      xa[m] = *reinterpret_cast<const uint4 *>(xr + 8 * c0);
      xb[m] = *reinterpret_cast<const uint4 *>(xr + 8 * c1);
    }
    const uint4 nw0 = *reinterpret_cast<const uint4 *>(NW + 8 * c0);
    const uint4 nw1 = *reinterpret_cast<const uint4 *>(NW + 8 * c1);
    res_signal(&s_sync[0]);

    // Statistic partial of every row for this virtual wave.
#pragma unroll
    for (int m = 0; m < kResMaxRows; ++m) {
      float ss = 0.f;
      if (ok0) {
        float f[8];
        unpack8(xa[m], f);
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += f[e] * f[e];
      }
      if (ok1) {  // uniform per wave: only virtual wave 0 has a second vector
        float f[8];
        unpack8(xb[m], f);
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += f[e] * f[e];
      }
      const float s = wave_sum(ss);
      if (lane == 0 && m < rows) s_part[m * 4 + vw] = s;
    }
    res_signal(&s_sync[1]);
    res_wait(&s_sync[1], 4u);

    // Normalise this virtual wave's vectors of every row into LDS, fragment
    // order with the slots of each k step's KiB permuted: vector v of row m
    // is k step s = v / 4, slot m + 16 (v % 4), at position res_pos(slot, s).
#pragma unroll
    for (int m = 0; m < kResMaxRows; ++m) {
      if (m >= rows) continue;
      float t = 0.f;
#pragma unroll
      for (int w2 = 0; w2 < 4; ++w2) t += s_part[m * 4 + w2];
      const float rs = 1.0f / sqrtf(t / (float)k + p.eps);
      if (ok0) s_x[(v0 >> 2) * 64 + res_pos(m + 16 * (v0 & 3), v0 >> 2)] = norm8(xa[m], nw0, rs);
      if (ok1) s_x[(v1 >> 2) * 64 + res_pos(m + 16 * (v1 & 3), v1 >> 2)] = norm8(xb[m], nw1, rs);
    }
    res_signal(&s_sync[2]);
    if (active) issue_ring();
  } else {
    res_wait(&s_sync[0], 4u);
    if (active) issue_ring();
  }
  res_wait(&s_sync[2], 4u);

  // ---- the ring: slot r holds k step r (mod RW) of the wave's range.
  f32x4_t ag = f32x4_t{0.f, 0.f, 0.f, 0.f}, au = ag;
  const bool xrow_ok = col < rows;  // lanes past the last row multiply zeros
  if (!half) {
    for (int i0 = 0; i0 < ksw_w; i0 += RW) {
      const bool refill = i0 + RW < ksw_w;
      const uint4 *qn = wq + (size_t)(i0 + RW) * 64;
      uint4 bq[RW];
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        const int s = q * ksw + i0 + r;  // k step
        bq[r] = xrow_ok ? s_x[s * 64 + res_pos(lane, s)] : zero4();
      }
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        ag = mfma16x16x32(wg[r], bq[r], ag);
        if constexpr (GLU) au = mfma16x16x32(wu[r], bq[r], au);
        if (refill) {
          wg[r] = ldw(qn + r * 64);
          if constexpr (GLU) wu[r] = ldw(qn + r * 64 + up_off);
        }
      }
    }
  } else if constexpr (GLU) {
    // A half pair: k steps i0 .. i0+RW-1 from wg, then the next RW from wu,
    // one MFMA chain in k order.
    for (int i0 = 0; i0 < ksw_w; i0 += 2 * RW) {
      const bool refill = i0 + 2 * RW < ksw_w;
      const uint4 *qn = wq + (size_t)(i0 + 2 * RW) * 64;
      auto pass = [&](uint4(&a)[RW], const int hh) {
        uint4 bq[RW];
#pragma unroll
        for (int r = 0; r < RW; ++r) {
          const int s = q * ksw + i0 + hh * RW + r;  // k step
          bq[r] = xrow_ok ? s_x[s * 64 + res_pos(lane, s)] : zero4();
        }
#pragma unroll
        for (int r = 0; r < RW; ++r) {
          ag = mfma16x16x32(a[r], bq[r], ag);
          if (refill) a[r] = ldw(qn + (size_t)(hh * RW + r) * 64);
        }
      };
      pass(wg, 0);
      pass(wu, 1);
    }
  }
  if (active && q > 0) {
    s_red[((j * 3 + q - 1) * NA + 0) * 64 + lane] = make_float4(ag[0], ag[1], ag[2], ag[3]);
    if constexpr (GLU) s_red[((j * 3 + q - 1) * NA + 1) * 64 + lane] = make_float4(au[0], au[1], au[2], au[3]);
  }
  __syncthreads();
  if (!active || q != 0) return;

  // ---- the pair's four waves in wave order, then SwiGLU (the direct path's
  // epilogue).
#pragma unroll
  for (int w2 = 1; w2 < 4; ++w2) {
    const float4 rg = s_red[((j * 3 + w2 - 1) * NA + 0) * 64 + lane];
    ag[0] += rg.x; ag[1] += rg.y; ag[2] += rg.z; ag[3] += rg.w;
    if constexpr (GLU) {
      const float4 ru = s_red[((j * 3 + w2 - 1) * NA + 1) * 64 + lane];
      au[0] += ru.x; au[1] += ru.y; au[2] += ru.z; au[3] += ru.w;
    }
  }
  if constexpr (GLU) {
    if (half) {  // lanes 32..63 hold the up columns of lanes 0..31's gate columns
#pragma unroll
      for (int i = 0; i < 4; ++i) au[i] = shfl_xor(ag[i], 32);
    }
  }
  const int m = col;
  if (m >= rows || (half && grp >= 2)) return;
  const int n0 = tile * 16 + (half ? 8 * (kind - 1) : 0) + grp * 4;
  uint2 o;
  if constexpr (GLU) {
    float o4[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float g = rbf(ag[i]);
      const float u = rbf(au[i]);
      const float sg = rbf(g / (1.0f + expf(-g)));
      o4[i] = sg * u;
    }
    o.x = pack2(o4[0], o4[1]);
    o.y = pack2(o4[2], o4[3]);
  } else {
    o.x = pack2(ag[0], ag[1]);
    o.y = pack2(ag[2], ag[3]);
  }
  uint16_t *out = reinterpret_cast<uint16_t *>(p.out);
  *reinterpret_cast<uint2 *>(p.ofrag ? out + frag_off(m, n0, p.ofrag) : out + (size_t)m * p.n + n0) = o;
}

// 16 bytes per lane from global memory into LDS at byte address lds_addr +
// 16 * lane (global_load_lds_dwordx4; M0 holds the wave's LDS address),
// from inline assembly: the compiler does not count these loads, so the
// caller waits for them (vmcnt) itself.  They are issued before any load the
// compiler counts, so its own waits stay correct (loads complete in order).
__device__ __forceinline__ void res_dma16(const void *g, uint32_t lds_addr) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds_addr))
      : "memory");
}
// s_waitcnt vmcnt(n) alone (gfx9 encoding: vmcnt in bits 3:0 and 15:14).
constexpr int res_vmcnt(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// Two M tiles (17..32 rows): the rows, normalised in fragment order by the
// pre-pass (p.xn), are copied once per workgroup into LDS -- the whole
// 160 KiB of LDS for k = 2560, so nothing else lives there until the k loop
// is done -- instead of every tile pair's workgroup reading them from L2 as
// ring operands (608 x 164 KB per launch for Qwen3-4B at 32 rows).  The
// ring then holds weights only (RW slots of gate and up blocks).  Sums,
// order and epilogue are the direct path's at two M tiles.
template <int RW, bool GLU>
__global__ void __launch_bounds__(64 * 4 * kResMaxPairs) glu_resident2_kernel(const GemmParams p) {
  constexpr int MT = 2;
  constexpr int NA = GLU ? 2 : 1;
  __shared__ __align__(16) uint4 s_x[kResMaxKSteps * MT * 64];  // [k step][M tile][lane]; then the wave merge

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nw = p.res_waves;
  const int rows = p.rows, KS = p.KS, ksw = p.ksw;
  const int col = lane & 15, grp = lane >> 4;
  const int j = wave >> 2, q = wave & 3;  // unit within the workgroup, k quarter
  unsigned tile = 0;
  int kind = 0;  // 0 a whole pair (or tile), 1 + h half pair h
  const bool active = res_unit_of<GLU>(p, j, tile, kind);
  const bool half = GLU && kind != 0;

  // ---- the rows into LDS: fragment f = (k step, M tile) is one KiB, wave w
  // copies fragments w, w + nw, ...  (LDS DMA, no registers).
  const uint4 *xn = reinterpret_cast<const uint4 *>(p.xn);
  const int nfrag = KS * MT;
  const uint32_t xbase = (uint32_t)reinterpret_cast<uintptr_t>(s_x);
  int ndma = 0;
  for (int f = wave; f < nfrag; f += nw, ++ndma) res_dma16(xn + (size_t)f * 64 + lane, xbase + (uint32_t)f * 1024u);

  // ---- the ring: the first RW k steps of this wave's range.
  const uint4 *W = reinterpret_cast<const uint4 *>(p.w);
  const size_t up_off = (size_t)p.up_tiles * KS * 64;
  const int ksw_w = active ? ksw : 0;
  const uint4 *wq = W + ((size_t)(active ? tile : 0) * KS + (size_t)q * ksw) * 64 + res_lane_off(half, kind, lane, up_off);
  // wu[r]'s block: the up tile's, or (half pair) RW k steps on
  const size_t second = half ? (size_t)RW * 64 : up_off;
  uint4 wg[RW], wu[GLU ? RW : 1];
  if (active) {
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      wg[r] = ldw(wq + r * 64);
      if constexpr (GLU) wu[r] = ldw(wq + r * 64 + second);
    }
  }
  // The copies are older than every ring load: once at most NA RW loads are
  // outstanding (none when the wave has no unit), they have landed.
  if (active)
    __builtin_amdgcn_s_waitcnt(res_vmcnt(NA * RW));
  else
    __builtin_amdgcn_s_waitcnt(res_vmcnt(0));
  (void)ndma;
  __syncthreads();

  f32x4_t ag[MT], au[GLU ? MT : 1];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    ag[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    if constexpr (GLU) au[mt] = ag[mt];
  }
  const bool xrow0 = col < rows, xrow1 = 16 + col < rows;
  constexpr int CH = 5;  // k steps whose B operands are read from LDS ahead
  static_assert(RW % CH == 0, "chunks within a ring pass");
  if (!half) {
    for (int i0 = 0; i0 < ksw_w; i0 += RW) {
      const bool refill = i0 + RW < ksw_w;
      const uint4 *qn = wq + (size_t)(i0 + RW) * 64;
#pragma unroll
      for (int c0 = 0; c0 < RW; c0 += CH) {
        uint4 b0[CH], b1[CH];
#pragma unroll
        for (int c = 0; c < CH; ++c) {
          const int s = q * ksw + i0 + c0 + c;
          b0[c] = xrow0 ? s_x[(s * MT + 0) * 64 + lane] : zero4();
          b1[c] = xrow1 ? s_x[(s * MT + 1) * 64 + lane] : zero4();
        }
#pragma unroll
        for (int c = 0; c < CH; ++c) {
          const int r = c0 + c;
          ag[0] = mfma16x16x32(wg[r], b0[c], ag[0]);
          ag[1] = mfma16x16x32(wg[r], b1[c], ag[1]);
          if constexpr (GLU) {
            au[0] = mfma16x16x32(wu[r], b0[c], au[0]);
            au[1] = mfma16x16x32(wu[r], b1[c], au[1]);
          }
          if (refill) {
            wg[r] = ldw(qn + r * 64);
            if constexpr (GLU) wu[r] = ldw(qn + r * 64 + up_off);
          }
        }
      }
    }
  } else if constexpr (GLU) {
    // A half pair: k steps i0 .. i0+RW-1 from wg, then the next RW from wu,
    // one MFMA chain per M tile in k order.
    for (int i0 = 0; i0 < ksw_w; i0 += 2 * RW) {
      const bool refill = i0 + 2 * RW < ksw_w;
      const uint4 *qn = wq + (size_t)(i0 + 2 * RW) * 64;
      auto pass = [&](uint4(&a)[RW], const int hh) {
#pragma unroll
        for (int c0 = 0; c0 < RW; c0 += CH) {
          uint4 b0[CH], b1[CH];
#pragma unroll
          for (int c = 0; c < CH; ++c) {
            const int s = q * ksw + i0 + hh * RW + c0 + c;
            b0[c] = xrow0 ? s_x[(s * MT + 0) * 64 + lane] : zero4();
            b1[c] = xrow1 ? s_x[(s * MT + 1) * 64 + lane] : zero4();
          }
#pragma unroll
          for (int c = 0; c < CH; ++c) {
            const int r = c0 + c;
            ag[0] = mfma16x16x32(a[r], b0[c], ag[0]);
            ag[1] = mfma16x16x32(a[r], b1[c], ag[1]);
            if (refill) a[r] = ldw(qn + (size_t)(hh * RW + r) * 64);
          }
        }
      };
      pass(wg, 0);
      pass(wu, 1);
    }
  }

  // ---- the unit's four waves in wave order (the merge reuses the rows'
  // LDS), then SwiGLU or the plain store.
  __syncthreads();
  float4 *red = reinterpret_cast<float4 *>(s_x);  // [unit][wave 1..3][gate, up][M tile][lane]
  if (active && q > 0) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      red[((((j * 3 + q - 1) * NA + 0) * MT + mt) * 64) + lane] = make_float4(ag[mt][0], ag[mt][1], ag[mt][2], ag[mt][3]);
      if constexpr (GLU)
        red[((((j * 3 + q - 1) * NA + 1) * MT + mt) * 64) + lane] = make_float4(au[mt][0], au[mt][1], au[mt][2], au[mt][3]);
    }
  }
  __syncthreads();
  if (!active || q != 0) return;
#pragma unroll
  for (int w2 = 1; w2 < 4; ++w2) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const float4 rg = red[((((j * 3 + w2 - 1) * NA + 0) * MT + mt) * 64) + lane];
      ag[mt][0] += rg.x; ag[mt][1] += rg.y; ag[mt][2] += rg.z; ag[mt][3] += rg.w;
      if constexpr (GLU) {
        const float4 ru = red[((((j * 3 + w2 - 1) * NA + 1) * MT + mt) * 64) + lane];
        au[mt][0] += ru.x; au[mt][1] += ru.y; au[mt][2] += ru.z; au[mt][3] += ru.w;
      }
    }
  }
  if constexpr (GLU) {
    if (half) {  // lanes 32..63 hold the up columns of lanes 0..31's gate columns
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) au[mt][i] = shfl_xor(ag[mt][i], 32);
    }
  }
  if (half && grp >= 2) return;
  const int n0 = tile * 16 + (half ? 8 * (kind - 1) : 0) + grp * 4;
  uint16_t *out = reinterpret_cast<uint16_t *>(p.out);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + col;
    if (m >= rows) continue;
    uint2 o;
    if constexpr (GLU) {
      float o4[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float g = rbf(ag[mt][i]);
        const float u = rbf(au[mt][i]);
        const float sg = rbf(g / (1.0f + expf(-g)));
        o4[i] = sg * u;
      }
      o.x = pack2(o4[0], o4[1]);
      o.y = pack2(o4[2], o4[3]);
    } else {
      o.x = pack2(ag[mt][0], ag[mt][1]);
      o.y = pack2(ag[mt][2], ag[mt][3]);
    }
    *reinterpret_cast<uint2 *>(p.ofrag ? out + frag_off(m, n0, p.ofrag) : out + (size_t)m * p.n + n0) = o;
  }
}

// RES_OUT without a k split at 1..kResLdsRows rows, x row-major: each
// workgroup (one output tile, its waves splitting k as in the direct path)
// first copies the rows into LDS with LDS DMA -- up to 8 rows x 64 bytes per
// k step, 152 KiB for the down projection's k = 9728 -- and its weight ring
// then holds weights only.  In the direct path every ring slot also loads
// the k step's B fragment from x, 16 row pieces of 64 bytes per load (a
// cache access per lane); here one DMA instruction gathers 2 to 16 k steps.
// The MFMA chain, the wave merge and the RES_OUT epilogue are the direct
// path's, so the result is bit-identical to it.
template <int RW>
__global__ void __launch_bounds__(512) res_rows_kernel(const GemmParams p) {
  __shared__ __align__(16) uint4 s_x[kResLdsKSteps * 32];  // [k step][row 0..7][k group]; then the wave merge
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nw = p.waves;
  const int rows = p.rows, k = p.k, KS = p.KS, ksw = p.ksw;
  const int col = lane & 15, grp = lane >> 4;
  const int tile = blockIdx.x;
  const uint16_t *X = reinterpret_cast<const uint16_t *>(p.x);

  // Residual values of this lane's outputs, loaded first (the direct path's
  // res_early): the epilogue then waits on no dependent load.
  uint2 res_v = make_uint2(0u, 0u);
  if (wave == 0) res_v = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint16_t *>(p.res) +
                                                         (size_t)(col < rows ? col : 0) * p.n + tile * 16 + grp * 4);

  // ---- the rows into LDS, R = rows rounded up to 1, 2, 4 or 8 of them per
  // k step (R x 64 bytes): DMA instruction i covers the 16 / R k steps from
  // i * 16 / R; lane L takes k step L / (4 R) of them, row (L / 4) % R, k
  // group L % 4 (rows past the last read row 0; their B lanes use zeros).
  const int R = rows <= 1 ? 1 : rows <= 2 ? 2 : rows <= 4 ? 4 : 8;
  const int lr = R == 1 ? 0 : R == 2 ? 1 : R == 4 ? 2 : 3;  // log2 R
  const uint32_t xbase = (uint32_t)reinterpret_cast<uintptr_t>(s_x);
  {
    const int r = (lane >> 2) & (R - 1), g = lane & 3;
    const int sl = lane >> (2 + lr);  // k step within the instruction
    const uint16_t *src = X + (size_t)(r < rows ? r : 0) * k + sl * 32 + g * 8;
    const int per = 16 >> lr;  // k steps per instruction
    for (int i = wave; i < KS / per; i += nw) res_dma16(src + (size_t)i * per * 32, xbase + (uint32_t)i * 1024u);
  }

  // ---- the ring: the first RW k steps of this wave's range.
  const uint4 *W = reinterpret_cast<const uint4 *>(p.w);
  const uint4 *wq = W + ((size_t)tile * KS + (size_t)wave * ksw) * 64 + lane;
  uint4 wb[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) wb[r] = ldw(wq + min(r, ksw - 1) * 64);
  // The copies are older than every ring load (and the residual load):
  // once at most RW loads are outstanding they have landed.
  __builtin_amdgcn_s_waitcnt(res_vmcnt(RW));
  __syncthreads();

  f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const bool xrow_ok = col < rows;
  const int kb = wave * ksw;  // first k step of this wave
  for (int i0 = 0; i0 < ksw; i0 += RW) {
    uint4 bq[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int s = kb + min(i0 + r, ksw - 1);
      bq[r] = xrow_ok ? s_x[((s << lr) + col) * 4 + grp] : zero4();
    }
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int i = i0 + r;
      if (i < ksw) {
        acc = mfma16x16x32(wb[r], bq[r], acc);
        if (i + RW < ksw) wb[r] = ldw(wq + (size_t)(i + RW) * 64);
      }
    }
  }

  // ---- waves in order (the merge reuses the rows' LDS), then RES_OUT.
  __syncthreads();
  float4 *red = reinterpret_cast<float4 *>(s_x);
  if (wave > 0) red[(wave - 1) * 64 + lane] = make_float4(acc[0], acc[1], acc[2], acc[3]);
  __syncthreads();
  if (wave != 0) return;
  for (int w2 = 1; w2 < nw; ++w2) {
    const float4 r = red[(w2 - 1) * 64 + lane];
    acc[0] += r.x;
    acc[1] += r.y;
    acc[2] += r.z;
    acc[3] += r.w;
  }
  const int m = col;
  if (m >= rows) return;
  uint16_t *rp = reinterpret_cast<uint16_t *>(p.res) + (size_t)m * p.n + tile * 16 + grp * 4;
  uint2 o;
  o.x = pack2(lo16(res_v.x) + rbf(acc[0]), hi16(res_v.x) + rbf(acc[1]));
  o.y = pack2(lo16(res_v.y) + rbf(acc[2]), hi16(res_v.y) + rbf(acc[3]));
  *reinterpret_cast<uint2 *>(rp) = o;
}

// RES_OUT with its k split S ways into partials (parts_out) at two M tiles
// (17..32 rows), x in fragment order: the workgroups of one k part share its
// slice of the rows.  Workgroup w takes k part w % S and a contiguous run of
// 2 or 3 output tiles (the S parts of the grid interleave over the XCDs);
// its waves are four per tile, wave (j, q) streaming k steps [q kw, (q + 1)
// kw) of its part of tile j, where the direct path gives the same k steps
// to wave q of the tile's (or tile pair's) workgroup.  The part's rows are
// copied into LDS once per workgroup by DMA (152 KiB for the down
// projection's quarter of k = 9728), and the ring holds weights only.  A
// tile's partial is each wave's MFMA chain in k order, the four waves added
// in order, stored to parts_out[part] -- the direct path's arithmetic, the
// same bits.
template <int RW>
__global__ void __launch_bounds__(64 * 4 * kResMaxPairs) res_split_kernel(const GemmParams p) {
  constexpr int MT = 2;
  __shared__ __align__(16) uint4 s_x[kResSplitKSteps * MT * 64];  // [k step of the part][M tile][lane]; then the merge
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nw = p.res_waves;
  const int rows = p.rows, KS = p.KS, S = p.ksplit;
  const int kp = KS / S;       // k steps of a part
  const int kw = p.ksw;        // k steps of a wave (kp / 4)
  const int col = lane & 15, grp = lane >> 4;
  const int part = blockIdx.x % S;
  const unsigned G = gridDim.x / S, g = blockIdx.x / S;
  const unsigned T = (unsigned)p.n >> 4;
  const unsigned t0 = g * T / G;
  const int ntile = (int)((g + 1) * T / G - t0);
  const int j = wave >> 2, q = wave & 3;
  const bool active = j < ntile;
  const int tile = (int)t0 + j;

  // ---- the part's rows into LDS: fragment f = (k step of the part, M tile).
  const uint4 *xf = reinterpret_cast<const uint4 *>(p.x) + (size_t)part * kp * MT * 64;
  const uint32_t xbase = (uint32_t)reinterpret_cast<uintptr_t>(s_x);
  for (int f = wave; f < kp * MT; f += nw) res_dma16(xf + (size_t)f * 64 + lane, xbase + (uint32_t)f * 1024u);

  // ---- the ring: the first RW k steps of this wave's range (a range
  // shorter than the ring repeats its last block).
  const uint4 *W = reinterpret_cast<const uint4 *>(p.w);
  const int kb = q * kw;  // first k step of this wave within the part
  const uint4 *wq = W + ((size_t)(active ? tile : 0) * KS + (size_t)part * kp + kb) * 64 + lane;
  const int kw_w = active ? kw : 0;
  uint4 wb[RW];
  if (active) {
#pragma unroll
    for (int r = 0; r < RW; ++r) wb[r] = ldw(wq + min(r, kw - 1) * 64);
  }
  if (active)
    __builtin_amdgcn_s_waitcnt(res_vmcnt(RW));
  else
    __builtin_amdgcn_s_waitcnt(res_vmcnt(0));
  __syncthreads();

  f32x4_t acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const bool xrow0 = col < rows, xrow1 = 16 + col < rows;
  for (int i0 = 0; i0 < kw_w; i0 += RW) {
    uint4 b0[RW], b1[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int s2 = kb + min(i0 + r, kw - 1);
      b0[r] = xrow0 ? s_x[(s2 * MT + 0) * 64 + lane] : zero4();
      b1[r] = xrow1 ? s_x[(s2 * MT + 1) * 64 + lane] : zero4();
    }
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int i = i0 + r;
      if (i < kw_w) {
        acc[0] = mfma16x16x32(wb[r], b0[r], acc[0]);
        acc[1] = mfma16x16x32(wb[r], b1[r], acc[1]);
        if (i + RW < kw_w) wb[r] = ldw(wq + (size_t)(i + RW) * 64);
      }
    }
  }

  // ---- the tile's four waves in order (the merge reuses the rows' LDS),
  // then the partial to parts_out[part].
  __syncthreads();
  float4 *red = reinterpret_cast<float4 *>(s_x);  // [tile][wave 1..3][M tile][lane]
  if (active && q > 0) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      red[((j * 3 + q - 1) * MT + mt) * 64 + lane] = make_float4(acc[mt][0], acc[mt][1], acc[mt][2], acc[mt][3]);
  }
  __syncthreads();
  if (!active || q != 0) return;
#pragma unroll
  for (int w2 = 1; w2 < 4; ++w2)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const float4 r = red[((j * 3 + w2 - 1) * MT + mt) * 64 + lane];
      acc[mt][0] += r.x;
      acc[mt][1] += r.y;
      acc[mt][2] += r.z;
      acc[mt][3] += r.w;
    }
  const int n0 = tile * 16 + grp * 4;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + col;
    if (m < rows) *reinterpret_cast<f32x4_t *>(p.parts_out + ((size_t)part * rows + m) * p.n + n0) = acc[mt];
  }
}

}  // namespace

hipError_t launch_res_split(const GemmParams &p, hipStream_t s) {
  int dev = 0, ncu = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  e = hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  const int S = p.ksplit, T = p.n / 16;
  if (S < 1 || p.KS % S || (p.KS / S) % 4 || p.KS / S > kResSplitKSteps || p.ksw * 4 != p.KS / S || p.rows < 17 ||
      p.rows > 32 || !p.parts_out || !p.xt || p.rw != kResSplitRing)
    return hipErrorInvalidValue;
  // Workgroups per part: one per CU in all, 2 or 3 tiles each.
  const int G = std::max((T + kResMaxPairs - 1) / kResMaxPairs, std::min(ncu / S, T / 2));
  if (G < 1) return hipErrorInvalidValue;
  const int tiles = (T + G - 1) / G;
  if (tiles > kResMaxPairs) return hipErrorInvalidValue;
  GemmParams q = p;
  q.res_waves = 4 * tiles;
  hipLaunchKernelGGL((res_split_kernel<kResSplitRing>), dim3(G * S), dim3(64 * q.res_waves), 0, s, q);
  return hipSuccess;
}

hipError_t launch_res_rows(const GemmParams &p, hipStream_t s) {
  if (p.rw != kResLdsRing || p.rows < 1 || p.rows > kResLdsRows || p.KS > kResLdsKSteps || (p.KS & 15) ||
      p.tiles_per_wg != 1 || p.ksplit != 1)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL((res_rows_kernel<kResLdsRing>), dim3(p.n / 16), dim3(64 * p.waves), 0, s, p);
  return hipSuccess;
}

hipError_t launch_glu_resident(const GemmParams &p, hipStream_t s) {
  int dev = 0, ncu = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  e = hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  const bool glu = p.resident == 1;  // otherwise NORM_IN alone (4)
  const int P = p.n / 16;
  // One workgroup per CU with two or three tile pairs each (GLU) or up to
  // two single tiles: more workgroups than CUs for a matrix past that many
  // units per CU, fewer for a small one -- but always a workgroup with two
  // units, whose last four waves normalise the rows (at most 8 rows).
  const int umax = glu ? kResMaxPairs : kResMaxTiles1;
  if ((p.rw != kResRing && p.rw != kResRing1) || p.ksw % p.rw || P < 1) return hipErrorInvalidValue;
  // gate/up takes runs of half pairs (res_unit) when a wave's k range is
  // whole ring passes of 2 RW k steps: at most five half pairs per
  // workgroup, so at most three units.
  const bool half = glu && p.ksw % (2 * p.rw) == 0;
  int grid, units = 0;
  if (half) {
    grid = std::max((2 * P + 4) / 5, std::min(ncu, P / 2));
    for (int b = 0; b < grid; ++b) {
      const unsigned h0 = (unsigned)b * 2u * P / grid, h1 = (unsigned)(b + 1) * 2u * P / grid;
      unsigned t = 0;
      int kd = 0, u = 0;
      while (u < kResMaxPairs && res_unit(h0, h1, u, t, kd)) ++u;
      if (h1 - h0 > 5) return hipErrorInvalidValue;
      units = std::max(units, u);
    }
  } else {
    grid = std::max((P + umax - 1) / umax, std::min(ncu, glu ? P / 2 : P - 1));
    if (grid < 1) return hipErrorInvalidValue;
    units = (P + grid - 1) / grid;
  }
  if (units > umax) return hipErrorInvalidValue;
  GemmParams q = p;
  q.res_waves = 4 * units;
  q.res_half = half ? 1 : 0;
  if (p.rows <= kResMaxRows) {
    // The last four waves normalise the rows, so the others are at least one
    // unit's.
    if (units < 2) return hipErrorInvalidValue;
    if (glu && p.rw == kResRing)
      hipLaunchKernelGGL((glu_resident_kernel<kResRing, true>), dim3(grid), dim3(64 * q.res_waves), 0, s, q);
    else if (!glu && p.rw == kResRing1)
      hipLaunchKernelGGL((glu_resident_kernel<kResRing1, false>), dim3(grid), dim3(64 * q.res_waves), 0, s, q);
    else
      return hipErrorInvalidValue;
  } else {
    if (p.rows > 32 || !p.xn || p.KS > kResMaxKSteps) return hipErrorInvalidValue;
    if (glu && p.rw == kResRing)
      hipLaunchKernelGGL((glu_resident2_kernel<kResRing, true>), dim3(grid), dim3(64 * q.res_waves), 0, s, q);
    else if (!glu && p.rw == kResRing1)
      hipLaunchKernelGGL((glu_resident2_kernel<kResRing1, false>), dim3(grid), dim3(64 * q.res_waves), 0, s, q);
    else
      return hipErrorInvalidValue;
  }
  return hipSuccess;
}

}  // namespace qdec
