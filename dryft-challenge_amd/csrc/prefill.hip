// Prompt-processing (prefill) kernels for gfx950: the large-M product on the
// matrix cores, the batched head norm / RoPE / cache fill, and causal GQA
// flash attention over the cache.
//
// Reference behaviour replaced: engine/engine.py:448-490 (_layers_forward,
// _attend_prefill, _prefill: F.linear, ops.qkv_post_rows, SDPA flash
// attention), engine/kernels/ops.py:149-205 (_qkv_post_rows_kernel) and
// :242-267 (_silu_mul_kernel).
#include "qdec_common.h"
#include "qdec_kernels.h"

namespace qdec {
namespace {

// ------------------------------------------------------------------ product
// A workgroup of 2 x NWM wavefronts computes a (16 NWM XW) x (32 WN) tile of
// the transposed product D = W . x^T: a weight fragment (16 weight rows x 32
// k) is the A operand and an activation fragment (32 k x 16 rows) the B
// operand of v_mfma_f32_16x16x32_bf16, and both are one contiguous KiB in
// their layouts.  Wave (wn, wm) owns WN weight x XW activation fragments.
// Every fragment moves from global memory straight into LDS
// (global_load_lds_dwordx4: one instruction per 1 KiB fragment, no
// registers) through a ring of stage buffers, RING - 1 stages in flight
// while one computes:
//   256 x 256 (8 waves of WN 8 x XW 4): stages of one k step (32 KiB),
//     RING 4 -- a third fewer LDS bytes per MFMA than 256 x 128;
//   256 x 128 (8 waves of WN 4 x XW 4): stages of two k steps (48 KiB),
//     RING 3 -- twice the workgroups;
//   64 x 64 (4 waves of WN 2 x XW 2): stages of two k steps (16 KiB),
//     RING 3 -- for few rows: 8x the workgroups of 256 x 128, several per
//     CU.
// Eight waves of half the accumulators (~240 and ~100 registers) run two
// per SIMD, so one wave's LDS reads overlap another's MFMAs: 5-15% over four
// waves of twice the tile per wave.
template <int WN, int XW, int NWM = 2>
struct PgShape {
  static constexpr int NW = 2 * NWM;                // waves: 2 along n x NWM along rows
  static constexpr int Wf = 2 * WN;                 // weight fragments per k step
  static constexpr int Xf = NWM * XW;               // activation fragments per k step
  static constexpr int KS = WN == 8 ? 1 : 2;        // k steps per stage
  static constexpr int RING = WN == 8 ? 4 : 3;      // stage buffers
  static constexpr int Frags = Wf + Xf;             // fragments per k step
  static constexpr int Stage = KS * Frags;          // fragments per stage
  static constexpr int Loads = Stage / NW;          // loads per wave per stage
  static constexpr int WQ = Wf / NW;                // weight loads per wave per k step
  static_assert(Wf % NW == 0 && Xf % NW == 0, "each wave loads whole fragments");
};
constexpr int kPgGroupN = 4;  // column tiles walked together (x reuse in L2)
constexpr int kPg256Xw = 4;   // 256 x 256 and 256 x 128 tiles: activation fragments per wave
constexpr int kPg128Xw = 4;   //   (4: 8 waves; 8 would be 4 waves of twice the accumulators)

__device__ __forceinline__ uint4 ld16(const uint16_t *p) { return *reinterpret_cast<const uint4 *>(p); }

// 16 bytes per lane from global memory into LDS at byte address lds_addr +
// 16 * lane (global_load_lds_dwordx4; M0 holds the wave's LDS address).
// Issued from inline assembly so the compiler does not make every later LDS
// read wait for all of these loads; the caller waits (vmcnt) and
// synchronises the workgroup itself.
// M0 is saved and restored around the load.
__device__ __forceinline__ void dma16(const void *g, uint32_t lds_addr) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds_addr))
      : "memory");
}
__device__ __forceinline__ uint32_t lds_addr(const void *p) { return (uint32_t)reinterpret_cast<uintptr_t>(p); }

// Maximum of v over the lane pairs (l, l ^ 16) and then (l, l ^ 32), with
// gfx950's row swaps instead of LDS permutes: after v_permlane16_swap the two
// outputs hold the odd / even 16-lane rows exchanged, after
// v_permlane32_swap the two halves, so the maximum of both outputs is the
// pairwise maximum in every lane.
__device__ __forceinline__ float max_xor16_32(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// s_waitcnt encodings (gfx9 family): vmcnt in bits 3:0 and 15:14, expcnt
// 6:4, lgkmcnt 11:8; the other counters at their maximum (no wait).
constexpr int vmcnt_enc(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
constexpr int kVmcnt0 = vmcnt_enc(0);

template <uint32_t FLAGS, int WN, int XW, int NWM>
__global__ void __launch_bounds__(128 * NWM, 1) pgemm_kernel(const PgemmParams p) {
  using S = PgShape<WN, XW, NWM>;
  constexpr bool GLU = (FLAGS & QDEC_GLU) != 0;
  constexpr bool RES = (FLAGS & QDEC_RES_OUT) != 0;
  __shared__ uint4 lds[S::RING * S::Stage * 64];  // [ring slot][k step][fragment][lane]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int wn = wave & 1, wm = wave >> 1;

  // Tile order: workgroup i runs on XCD i % 8, so each XCD gets a contiguous
  // range of the sequence; the sequence walks groups of kPgGroupN column
  // tiles across all row tiles (the group's weights stay in L2, each row
  // tile of x is read by the group's workgroups together).
  int id = blockIdx.x;
  const int G = gridDim.x;
  if ((G & 7) == 0) id = (id & 7) * (G >> 3) + (id >> 3);
  const int ntm = p.tiles / S::Xf;
  const int gsz = kPgGroupN * ntm;
  const int g = id / gsz, r = id - g * gsz;
  const int gn = min(kPgGroupN, p.wg_n - g * kPgGroupN);
  const int tm = r / gn, tn = g * kPgGroupN + (r - (r / gn) * gn);

  const int KS = p.k >> 5;
  // Weight tile of workgroup fragment f (GLU: WN gate tiles, then the WN
  // matching up tiles).
  auto wtile = [&](int f) -> int {
    if constexpr (GLU)
      return f < WN ? tn * WN + f : p.up_tiles + tn * WN + f - WN;
    else
      return tn * S::Wf + f;
  };
  // Loads of one k step: this wave moves fragments wave + NW q (q < WQ:
  // weights, then activations).
  const uint16_t *wb[S::WQ];
#pragma unroll
  for (int q = 0; q < S::WQ; ++q) wb[q] = p.w + (size_t)wtile(wave + S::NW * q) * KS * 512 + lane * 8;
  const uint16_t *xb = p.x + (size_t)(tm * S::Xf + wave) * 512 + lane * 8;
  const size_t xks = (size_t)p.tiles * 512;  // elements per k step of x
  const uint32_t lds0 = lds_addr(lds);
  auto dma = [&](int s, int slot) {
#pragma unroll
    for (int j = 0; j < S::KS; ++j) {
      const int ks = s * S::KS + j;
      const uint32_t dst = lds0 + (uint32_t)(((slot * S::KS + j) * S::Frags + wave) * 1024);
#pragma unroll
      for (int q = 0; q < S::WQ; ++q) dma16(wb[q] + (size_t)ks * 512, dst + q * S::NW * 1024);
#pragma unroll
      for (int q = 0; q < S::Xf / S::NW; ++q)
        dma16(xb + ks * xks + q * S::NW * 512, dst + (S::WQ + q) * S::NW * 1024);
    }
  };
  // This wave's weight fragments (GLU: gate i pairs with up i + WN/2).
  auto wf = [&](int i) -> int {
    if constexpr (GLU)
      return i < WN / 2 ? wn * (WN / 2) + i : WN + wn * (WN / 2) + i - WN / 2;
    else
      return wn * WN + i;
  };

  f32x4_t acc[WN][XW];
#pragma unroll
  for (int i = 0; i < WN; ++i)
#pragma unroll
    for (int q = 0; q < XW; ++q) acc[i][q] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  if constexpr (WN == 8) {
    // 256 x 256 tiles (one k step per stage): the next step's fragments are
    // read while this step multiplies (+5-10% there; the other tiles, two
    // steps per stage, measured slower with it and read each step's
    // fragments right before its MFMAs).
    // k steps run through two register sets of fragments: the fragments of
    // step t+1 are read from LDS while step t's MFMAs run.  Entering a new
    // stage (before reading its first step) waits for this wave's loads of
    // it, then a barrier makes every wave's visible and frees the slot of the
    // stage before it -- all of whose steps are already in registers -- for
    // the stage RING - 1 ahead.
    const int nst = p.k / (32 * S::KS);
    const int nsteps = nst * S::KS;
    auto slot_of = [&](int st) { return st % S::RING; };
    auto enter_stage = [&](int st) {
      const int younger = min(S::RING - 2, nst - 1 - st);
      if (younger >= 2)
        __builtin_amdgcn_s_waitcnt(vmcnt_enc(2 * S::Loads));
      else if (younger == 1)
        __builtin_amdgcn_s_waitcnt(vmcnt_enc(S::Loads));
      else
        __builtin_amdgcn_s_waitcnt(kVmcnt0);
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      if (st + S::RING - 1 < nst) dma(st + S::RING - 1, slot_of(st + S::RING - 1));
    };
    auto read_frags = [&](int t, uint4 (&a)[WN], uint4 (&bx)[XW]) {
      const uint4 *L = lds + (size_t)(slot_of(t / S::KS) * S::KS + t % S::KS) * S::Frags * 64 + lane;
  #pragma unroll
      for (int i = 0; i < WN; ++i) a[i] = L[wf(i) * 64];
  #pragma unroll
      for (int q = 0; q < XW; ++q) bx[q] = L[(S::Wf + wm * XW + q) * 64];
    };
    auto mma = [&](const uint4 (&a)[WN], const uint4 (&bx)[XW]) {
  #pragma unroll
      for (int i = 0; i < WN; ++i)
  #pragma unroll
        for (int q = 0; q < XW; ++q) acc[i][q] = mfma16x16x32(a[i], bx[q], acc[i][q]);
    };
    // One step: prepare step t+1 into (na, nb), multiply step t from (ca, cb).
    auto step = [&](int t, const uint4 (&ca)[WN], const uint4 (&cb)[XW], uint4 (&na)[WN], uint4 (&nb)[XW]) {
      const int tn = t + 1;
      if (tn < nsteps) {
        if (tn % S::KS == 0) enter_stage(tn / S::KS);
        read_frags(tn, na, nb);
      }
      mma(ca, cb);
    };

  #pragma unroll
    for (int st = 0; st < S::RING - 1; ++st)
      if (st < nst) dma(st, st);
    uint4 a0[WN], b0[XW], a1[WN], b1[XW];
    // stage 0 (younger stages in flight as inside the loop)
    {
      const int younger = min(S::RING - 2, nst - 1);
      if (younger >= 2)
        __builtin_amdgcn_s_waitcnt(vmcnt_enc(2 * S::Loads));
      else if (younger == 1)
        __builtin_amdgcn_s_waitcnt(vmcnt_enc(S::Loads));
      else
        __builtin_amdgcn_s_waitcnt(kVmcnt0);
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      if (S::RING - 1 < nst) dma(S::RING - 1, S::RING - 1);
    }
    read_frags(0, a0, b0);
    int t = 0;
    for (; t + 1 < nsteps; t += 2) {
      step(t, a0, b0, a1, b1);
      step(t + 1, a1, b1, a0, b0);
    }
    if (t < nsteps) mma(a0, b0);
  } else {
    const int nst = p.k / (32 * S::KS);
  #pragma unroll
    for (int s = 0; s < S::RING - 1; ++s)
      if (s < nst) dma(s, s);
    int slot = 0;
    for (int s = 0; s < nst; ++s) {
      // this wave's loads of stage s are done once at most the younger
      // stages' are outstanding; the barrier makes every wave's visible and
      // frees the slot of stage s-1 for stage s + RING - 1
      const int younger = min(S::RING - 2, nst - 1 - s);
      if (younger >= 2)
        __builtin_amdgcn_s_waitcnt(vmcnt_enc(2 * S::Loads));
      else if (younger == 1)
        __builtin_amdgcn_s_waitcnt(vmcnt_enc(S::Loads));
      else
        __builtin_amdgcn_s_waitcnt(kVmcnt0);
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      if (s + S::RING - 1 < nst) dma(s + S::RING - 1, slot == 0 ? S::RING - 1 : slot - 1);
  #pragma unroll
      for (int j = 0; j < S::KS; ++j) {
        const uint4 *L = lds + (size_t)(slot * S::KS + j) * S::Frags * 64 + lane;
        uint4 a[WN], bx[XW];
  #pragma unroll
        for (int i = 0; i < WN; ++i) a[i] = L[wf(i) * 64];
  #pragma unroll
        for (int q = 0; q < XW; ++q) bx[q] = L[(S::Wf + wm * XW + q) * 64];
  #pragma unroll
        for (int i = 0; i < WN; ++i)
  #pragma unroll
          for (int q = 0; q < XW; ++q) acc[i][q] = mfma16x16x32(a[i], bx[q], acc[i][q]);
      }
      slot = slot == S::RING - 1 ? 0 : slot + 1;
    }
  }

  // Epilogue: lane holds columns n0 .. n0+3 of row m for every fragment pair.
  auto store = [&](int m, int n0, uint2 o) {
    uint16_t *dst = p.ofrag ? p.out + frag_off(m, n0, p.tiles) : p.out + (size_t)m * p.n_out + n0;
    *reinterpret_cast<uint2 *>(dst) = o;
  };
  const int m_base = (tm * S::Xf + wm * XW) * 16 + col;
#pragma unroll
  for (int q = 0; q < XW; ++q) {
    const int m = m_base + q * 16;
    if (m >= p.rows) continue;
    if constexpr (GLU) {
#pragma unroll
      for (int i = 0; i < WN / 2; ++i) {
        float o4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float gv = rbf(acc[i][q][e]);
          const float uv = rbf(acc[i + WN / 2][q][e]);
          o4[e] = rbf(gv / (1.0f + expf(-gv))) * uv;
        }
        store(m, wtile(wf(i)) * 16 + 4 * grp, make_uint2(pack2(o4[0], o4[1]), pack2(o4[2], o4[3])));
      }
    } else {
#pragma unroll
      for (int i = 0; i < WN; ++i) {
        const int n0 = wtile(wf(i)) * 16 + 4 * grp;
        uint2 o;
        if constexpr (RES) {
          const uint2 rv = *reinterpret_cast<const uint2 *>(p.res + (size_t)m * p.n_out + n0);
          o.x = pack2(lo16(rv.x) + rbf(acc[i][q][0]), hi16(rv.x) + rbf(acc[i][q][1]));
          o.y = pack2(lo16(rv.y) + rbf(acc[i][q][2]), hi16(rv.y) + rbf(acc[i][q][3]));
        } else {
          o.x = pack2(acc[i][q][0], acc[i][q][1]);
          o.y = pack2(acc[i][q][2], acc[i][q][3]);
        }
        store(m, n0, o);
      }
    }
  }
}

// ------------------------------------------------------- head norm + RoPE
constexpr int kPqHeadsPerWave = kPqMaxHeads / 4;  // per wave of the per-row kernel

// Few rows: one workgroup per row, wave w normalising and rotating heads w,
// w+4, ...  The values move in groups of 8 slots, the channel-major V
// cache's 16-byte cells: the row that starts a group (its slot a multiple of
// 8, or the call's first row) writes every row of the group that the call
// holds, one vector per (kv head, channel) when all 8 are there, element by
// element at the call's ragged ends.
__global__ void __launch_bounds__(256) pqk_row_kernel(const PqkParams p) {
  constexpr int D = 128;
  const int m = blockIdx.x;
  const int b = m / p.t_rows, t = m - b * p.t_rows;
  const int pos = p.pos0 + t;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int width = (p.nq + 2 * p.nkv) * D;
  uint16_t *row = p.qkv + (size_t)m * width;
  const uint32_t cw = *reinterpret_cast<const uint32_t *>(p.cos_tab + (size_t)pos * D + 2 * lane);
  const uint32_t sw = *reinterpret_cast<const uint32_t *>(p.sin_tab + (size_t)pos * D + 2 * lane);
  const uint32_t qw = *reinterpret_cast<const uint32_t *>(p.q_norm_w + 2 * lane);
  const uint32_t kw = *reinterpret_cast<const uint32_t *>(p.k_norm_w + 2 * lane);
  // Every head of this wave loaded before the first is reduced, so their
  // latencies overlap (the host admits at most 4 * kPqHeadsPerWave heads).
  const int nh = p.nq + p.nkv;
  uint32_t raw[kPqHeadsPerWave];
#pragma unroll
  for (int j = 0; j < kPqHeadsPerWave; ++j) {
    const int h = wave + 4 * j;
    raw[j] = h < nh ? *reinterpret_cast<const uint32_t *>(row + (size_t)h * D + 2 * lane) : 0u;
  }
#pragma unroll
  for (int j = 0; j < kPqHeadsPerWave; ++j) {
    const int h = wave + 4 * j;
    if (h >= nh) break;
    const uint32_t o = head_norm_rope2(raw[j], h < p.nq ? qw : kw, cw, sw, p.eps);
    if (h < p.nq)
      *reinterpret_cast<uint32_t *>(row + (size_t)h * D + 2 * lane) = o;
    else
      *reinterpret_cast<uint32_t *>(p.k_cache + (((size_t)b * p.nkv + (h - p.nq)) * p.cap + pos) * D + 2 * lane) = o;
  }
  if ((pos & 7) != 0 && t != 0) return;  // another row writes this group
  const int n = min(8 - (pos & 7), p.t_rows - t);  // rows of the group in this call
  for (int i = threadIdx.x; i < p.nkv * D; i += blockDim.x) {
    const int kvh = i >> 7, ch = i & 127;
    const uint16_t *src = row + (size_t)(p.nq + p.nkv + kvh) * D + ch;
    uint16_t *vb = p.v_cache + ((size_t)b * p.nkv + kvh) * p.cap * D + ((size_t)(pos >> 3) * D + ch) * 8;
    if (n == 8) {
      uint16_t v[8];
#pragma unroll
      for (int r = 0; r < 8; ++r) v[r] = src[(size_t)r * width];
      *reinterpret_cast<uint4 *>(vb) = make_uint4(v[0] | ((uint32_t)v[1] << 16), v[2] | ((uint32_t)v[3] << 16),
                                                  v[4] | ((uint32_t)v[5] << 16), v[6] | ((uint32_t)v[7] << 16));
    } else {
      for (int r = 0; r < n; ++r) vb[(pos & 7) + r] = src[(size_t)r * width];
    }
  }
}

// Many rows: a workgroup takes 8 consecutive positions of one sequence.  Wave w
// normalises and rotates the 40 heads of rows 2w and 2w+1 (queries back into
// qkv, keys into the K cache); then each thread moves the raw values of 4
// (kv head, channel) pairs: 8 positions of one channel are one 16-byte
// vector of the channel-major V cache when the group starts on a multiple of
// 8 slots and is complete (element stores otherwise).
constexpr int kPqRows = 8;

__global__ void __launch_bounds__(256) pqk_kernel(const PqkParams p) {
  constexpr int D = 128;
  const int T = p.t_rows;
  const int ngrp = (T + kPqRows - 1) / kPqRows;
  const int b = blockIdx.x / ngrp, t0 = (blockIdx.x - b * ngrp) * kPqRows;
  const int nrow = min(kPqRows, T - t0);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int width = (p.nq + 2 * p.nkv) * D;
  uint16_t *rows = p.qkv + (size_t)(b * T + t0) * width;
  const uint32_t qw = *reinterpret_cast<const uint32_t *>(p.q_norm_w + 2 * lane);
  const uint32_t kw = *reinterpret_cast<const uint32_t *>(p.k_norm_w + 2 * lane);
#pragma unroll
  for (int i = 0; i < kPqRows / 4; ++i) {
    const int r = wave * (kPqRows / 4) + i;
    if (r >= nrow) break;
    const int pos = p.pos0 + t0 + r;
    uint16_t *row = rows + (size_t)r * width;
    const uint32_t cw = *reinterpret_cast<const uint32_t *>(p.cos_tab + (size_t)pos * D + 2 * lane);
    const uint32_t sw = *reinterpret_cast<const uint32_t *>(p.sin_tab + (size_t)pos * D + 2 * lane);
    for (int h = 0; h < p.nq + p.nkv; ++h) {
      uint32_t *cell = reinterpret_cast<uint32_t *>(row + (size_t)h * D + 2 * lane);
      const uint32_t o = head_norm_rope2(*cell, h < p.nq ? qw : kw, cw, sw, p.eps);
      if (h < p.nq)
        *cell = o;
      else
        *reinterpret_cast<uint32_t *>(p.k_cache + (((size_t)b * p.nkv + (h - p.nq)) * p.cap + pos) * D + 2 * lane) = o;
    }
  }
  const int slot0 = p.pos0 + t0;
  const bool whole = nrow == kPqRows && (slot0 & 7) == 0;
  for (int i = threadIdx.x; i < p.nkv * D; i += blockDim.x) {
    const int kvh = i >> 7, ch = i & 127;
    const uint16_t *src = rows + (size_t)(p.nq + p.nkv + kvh) * D + ch;
    uint16_t *vb = p.v_cache + ((size_t)b * p.nkv + kvh) * p.cap * D;
    if (whole) {
      uint16_t v[kPqRows];
#pragma unroll
      for (int r = 0; r < kPqRows; ++r) v[r] = src[(size_t)r * width];
      uint4 o;
      o.x = v[0] | ((uint32_t)v[1] << 16);
      o.y = v[2] | ((uint32_t)v[3] << 16);
      o.z = v[4] | ((uint32_t)v[5] << 16);
      o.w = v[6] | ((uint32_t)v[7] << 16);
      *reinterpret_cast<uint4 *>(vb + ((size_t)(slot0 >> 3) * D + ch) * 8) = o;
    } else {
      for (int r = 0; r < nrow; ++r) {
        const int slot = slot0 + r;
        vb[((size_t)(slot >> 3) * D + ch) * 8 + (slot & 7)] = src[(size_t)r * width];
      }
    }
  }
}

// ------------------------------------------------------------ row norm
// RMSNorm of 16 rows (one M tile) per workgroup into fragment order: thread
// (row r, group g) holds k steps g, g+16, ... of row r in registers (read
// once), the row's sum of squares is reduced over its 16 threads, and every
// store is one lane's 16 bytes of a fragment -- the 16 threads of a group
// write 256 contiguous bytes per vector.  Rows past `rows` are zeros.
constexpr int kPnSteps = 8;  // k steps per thread: k up to 16 * 8 * 32 = 4096

__global__ void __launch_bounds__(256) pnorm_kernel(const uint16_t *__restrict__ X, const uint16_t *__restrict__ norm_w,
                                                    uint16_t *__restrict__ out, int k, float eps, int rows, int tiles) {
  __shared__ float s_red[4][16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = tid & 15, g = tid >> 4;
  const int mt = blockIdx.x;
  const int m = mt * 16 + r;
  const int KS = k >> 5;
  const bool real = m < rows;
  const uint16_t *xrow = X + (size_t)(real ? m : 0) * k;
  uint4 v[kPnSteps][4];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kPnSteps; ++i) {
    const int ks = g + 16 * i;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[i][j] = (real && ks < KS) ? *reinterpret_cast<const uint4 *>(xrow + ks * 32 + j * 8) : zero4();
      float f[8];
      unpack8(v[i][j], f);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += f[e] * f[e];
    }
  }
  // the 16 threads of row r: lanes r + 16 * (g % 4) of wave g / 4
  ss += shfl_xor(ss, 16);
  ss += shfl_xor(ss, 32);
  if (lane < 16) s_red[wave][lane] = ss;
  __syncthreads();
  const float tot = s_red[0][r] + s_red[1][r] + s_red[2][r] + s_red[3][r];
  const float rs = 1.0f / sqrtf(tot / (float)k + eps);
#pragma unroll
  for (int i = 0; i < kPnSteps; ++i) {
    const int ks = g + 16 * i;
    if (ks >= KS) break;
    uint16_t *blk = out + ((size_t)ks * tiles + mt) * 512;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint4 o = zero4();
      if (real)
        o = norm_w ? norm8(v[i][j], *reinterpret_cast<const uint4 *>(norm_w + ks * 32 + j * 8), rs) : v[i][j];
      *reinterpret_cast<uint4 *>(blk + (r + 16 * j) * 8) = o;
    }
  }
}

// ---------------------------------------------------------------- attention
// A workgroup takes kPaRows positions of G = 2 or 4 query heads of one kv
// head of one sequence; wave w takes head w % G of them and its share of
// the positions, 2 M tiles of 16 rows (two waves per head: 4 or 8 waves).
// Eight query heads per kv head run as two such workgroups.  Blocks of 32 cache slots
// go from global memory straight into LDS (global_load_lds_dwordx4 with
// per-lane gather addresses, so every fragment lands in MFMA operand
// order), three blocks in a ring, two ahead of the compute, shared by the
// waves:
//   K fragment (s, h): lane (c, g) holds slot 8*(c >> 2) + (c & 3) + 4h,
//     channels 32s + 8g .. +8: the slot order that makes the score registers
//     of S^T = K . Q^T exactly the B operand of O^T += V^T . P^T (each lane
//     ends up with 8 consecutive slots of one query row);
//   V fragment dt: lane (c, g) holds channel 16dt + c, slots 8g .. 8g+7 --
//     16 contiguous bytes of the channel-major cache.
// Online softmax in base 2 with fp32 state per row (running max kept in
// score units, exp2(s * scale - m * scale) as one FMA), probabilities rounded
// to bf16 for the P.V product, two tiles at a time in straight-line code
// (independent MFMA chains and softmaxes interleave).  Only blocks that
// cross some row's position are masked; the accumulators are rescaled only
// when some row's max moved.
// Slots past the block's last row are zeroed in V after the LDS read (the
// cache may hold anything there, and 0 * NaN would poison the product).
constexpr int kPaKFrags = 8, kPaVFrags = 8;
constexpr int kPaBlockVec = (kPaKFrags + kPaVFrags) * 64;  // uint4 per staged block
constexpr int kPaRing = 3;
// Waves per query head: two, each taking 2 M tiles (a workgroup of G = 2
// or 4 query heads has 4 or 8 waves).
constexpr int pa_wph(int G) { return 2; }

// G query heads per workgroup out of GS per kv head: GS = 8 (Qwen3-32B's
// layout) runs as two workgroups of 4 heads per (kv head, row block), each
// reading the kv head's K/V (8 heads in one workgroup would need 64
// accumulator rows per wave and spill).
template <int G, int GS = G>
__global__ void __launch_bounds__(64 * G * pa_wph(G), 1) pattn_kernel(const PattnParams p) {
  constexpr int D = 128;
  constexpr int WPH = pa_wph(G);
  constexpr int MT = 4 / WPH;                  // M tiles of 16 positions per wave
  constexpr int NWV = G * WPH;                 // waves
  constexpr int NSUB = GS / G;                 // workgroups per (kv head, row block)
  static_assert(MT % 2 == 0 && (G == 2 || G == 4) && GS % G == 0, "tiles taken in pairs; 2 or 4 heads");
  constexpr int FPW = (kPaKFrags + kPaVFrags) / NWV;  // fragments each wave loads per block
  __shared__ uint4 lds[kPaRing * kPaBlockVec];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int head = wave % G, half = wave / G;  // query head of the group, which 16*MT positions
  const int T = p.t_rows;
  const int nqb = (T + kPaRows - 1) / kPaRows;
  const int cells = p.batch * p.nkv * NSUB;
  const int qb = nqb - 1 - (int)(blockIdx.x / cells);  // longest rows first
  const int cell = (int)(blockIdx.x % cells);
  const int bk = cell / NSUB, sub = cell - bk * NSUB;
  const int b = bk / p.nkv, kvh = bk - b * p.nkv;
  const int hq = kvh * GS + sub * G + head;
  const int width = (p.nq + 2 * p.nkv) * D;
  const int t0 = qb * kPaRows;
  const int tw = t0 + half * 16 * MT;  // this wave's first position
  const int tlast = min(T, t0 + kPaRows) - 1;
  const int last = p.pos0 + tlast;  // highest slot any row of the block sees
  const int nb = last / 32 + 1;
  const size_t slab = ((size_t)b * p.nkv + kvh) * (size_t)p.cap * D;
  const uint16_t *kc = p.k_cache + slab;
  const uint16_t *vc = p.v_cache + slab;
  const float NEG_INF = -__builtin_huge_valf();
  const float scale = p.scale_log2;
  const bool rows_full = t0 + kPaRows - 1 <= tlast;  // all 64 rows are real

  // Queries as B operands: row col of M tile mt, channels 32s + 8*grp.
  uint4 qf[MT][4];
  int qpos[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int t = tw + mt * 16 + col;
    const bool valid = t <= tlast;
    qpos[mt] = valid ? p.pos0 + t : -1;
    const uint16_t *qrow = p.qkv + (size_t)(b * T + min(t, tlast)) * width + (size_t)hq * D + grp * 8;
#pragma unroll
    for (int s = 0; s < 4; ++s) qf[mt][s] = valid ? ld16(qrow + s * 32) : zero4();
  }

  // Block j into ring slot `slot`: this wave gathers K fragments wave + NWV*i
  // (index 2s + h) and V fragments wave + NWV*i.
  const uint32_t lds0 = lds_addr(lds);
  const uint16_t *kg = kc + (size_t)(8 * (col >> 2) + (col & 3)) * D + 8 * grp;
  const uint16_t *vg = vc + (size_t)grp * D * 8 + col * 8;
  auto dma_block = [&](int j, int slot) {
    const int s0 = j * 32;
    const uint32_t base = lds0 + (uint32_t)(slot * kPaBlockVec * 16);
#pragma unroll
    for (int i = 0; i < FPW / 2; ++i) {
      const int f = wave + NWV * i;
      dma16(kg + (size_t)(s0 + 4 * (f & 1)) * D + 32 * (f >> 1), base + f * 1024);
    }
#pragma unroll
    for (int i = 0; i < FPW / 2; ++i) {
      const int dt = wave + NWV * i;
      dma16(vg + (size_t)(s0 >> 3) * D * 8 + dt * 128, base + (kPaKFrags + dt) * 1024);
    }
  };

  f32x4_t acc[MT][8];
  float m_run[MT], l_run[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    m_run[mt] = NEG_INF;
    l_run[mt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[mt][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  // The query loads complete here, so no wait inside the loop (where it
  // would also wait for the blocks in flight) is needed for them.
  __builtin_amdgcn_s_waitcnt(kVmcnt0);
  dma_block(0, 0);
  if (nb > 1) dma_block(1, 1);
  int slot = 0;
  for (int j = 0; j < nb; ++j) {
    // this wave's loads of block j are done once at most the next block's
    // are outstanding; the barrier makes every wave's visible and frees the
    // slot of block j-1 for block j+2
    if (j + 1 < nb)
      __builtin_amdgcn_s_waitcnt(vmcnt_enc(FPW));
    else
      __builtin_amdgcn_s_waitcnt(kVmcnt0);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (j + 2 < nb) dma_block(j + 2, slot == 0 ? kPaRing - 1 : slot - 1);
    const uint4 *B = lds + slot * kPaBlockVec + lane;
    uint4 ka[4], kb[4], vf[8];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      ka[s] = B[(s * 2) * 64];
      kb[s] = B[(s * 2 + 1) * 64];
    }
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) vf[dt] = B[(kPaKFrags + dt) * 64];
    const int s0 = j * 32;
    const int sb = s0 + 8 * grp;  // first of this lane's 8 slots
    if (sb + 7 > last) {          // slots past the last row: zero V
      uint32_t keep[4];
#pragma unroll
      for (int d = 0; d < 4; ++d)
        keep[d] = (sb + 2 * d <= last ? 0x0000ffffu : 0u) | (sb + 2 * d + 1 <= last ? 0xffff0000u : 0u);
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        vf[dt].x &= keep[0];
        vf[dt].y &= keep[1];
        vf[dt].z &= keep[2];
        vf[dt].w &= keep[3];
      }
    }
    // Online softmax of one tile's 8 scores per lane (masked ones -inf):
    // updates the row state, returns the rescale factor and the bf16
    // probabilities as the B operand of the P.V product.
    auto softmax = [&](int mt, const float (&sc)[8], float &alpha, uint4 &pf) {
      float bmax = sc[0];
#pragma unroll
      for (int e = 1; e < 8; ++e) bmax = fmaxf(bmax, sc[e]);
      bmax = max_xor16_32(bmax);
      const float m_new = fmaxf(m_run[mt], bmax);
      alpha = (m_new == NEG_INF) ? 1.0f : __builtin_amdgcn_exp2f((m_run[mt] - m_new) * scale);
      const float mc = m_new * scale;
      float pj[8];
      float psum = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pj[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[e], scale, -mc));
        psum += pj[e];
      }
      l_run[mt] = l_run[mt] * alpha + psum;
      m_run[mt] = m_new;
      pf = pack8(pj);
    };
    // Masks only where the block crosses some row's position (the diagonal,
    // rows past the end); a tile that sees none of the block gets all -inf
    // and leaves its rows unchanged (alpha 1, p 0).
    const bool masked = !(rows_full && s0 + 31 <= p.pos0 + t0);
#pragma unroll
    for (int m2 = 0; m2 < MT; m2 += 2) {
      f32x4_t sa[2], sbv[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) sa[u] = sbv[u] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          sa[u] = mfma16x16x32(ka[s], qf[m2 + u][s], sa[u]);
          sbv[u] = mfma16x16x32(kb[s], qf[m2 + u][s], sbv[u]);
        }
      float alpha[2];
      uint4 pf[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        float sc[8] = {sa[u][0], sa[u][1], sa[u][2], sa[u][3], sbv[u][0], sbv[u][1], sbv[u][2], sbv[u][3]};
        if (masked) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (sb + i > qpos[m2 + u]) sc[i] = NEG_INF;
            if (sb + 4 + i > qpos[m2 + u]) sc[4 + i] = NEG_INF;
          }
        }
        softmax(m2 + u, sc, alpha[u], pf[u]);
      }
#pragma unroll
      for (int u = 0; u < 2; ++u)
        if (__any(alpha[u] != 1.0f)) {
#pragma unroll
          for (int dt = 0; dt < 8; ++dt) acc[m2 + u][dt] *= alpha[u];
        }
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int u = 0; u < 2; ++u) acc[m2 + u][dt] = mfma16x16x32(vf[dt], pf[u], acc[m2 + u][dt]);
    }
    slot = slot == kPaRing - 1 ? 0 : slot + 1;
  }

  // Rows in fragment order for the O projection: lane holds channels
  // 16dt + 4*grp .. +3 of its row.
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    if (tw + mt * 16 > tlast) continue;
    float l = l_run[mt] + shfl_xor(l_run[mt], 16);
    l += shfl_xor(l, 32);
    const int t = tw + mt * 16 + col;
    if (t > tlast) continue;
    const int m = b * T + t;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      uint2 o;
      o.x = pack2(acc[mt][dt][0] / l, acc[mt][dt][1] / l);
      o.y = pack2(acc[mt][dt][2] / l, acc[mt][dt][3] / l);
      *reinterpret_cast<uint2 *>(p.out + frag_off(m, hq * D + dt * 16 + 4 * grp, p.tiles)) = o;
    }
  }
}

}  // namespace

template <int WN, int XW, int NWM>
hipError_t launch_pgemm_tile(const PgemmParams &p, uint32_t flags, hipStream_t s) {
  const dim3 grid(p.wg_n * (p.tiles / PgShape<WN, XW, NWM>::Xf)), block(128 * NWM);
  switch (flags) {
    case 0u: hipLaunchKernelGGL((pgemm_kernel<0u, WN, XW, NWM>), grid, block, 0, s, p); break;
    case QDEC_RES_OUT: hipLaunchKernelGGL((pgemm_kernel<QDEC_RES_OUT, WN, XW, NWM>), grid, block, 0, s, p); break;
    case QDEC_GLU: hipLaunchKernelGGL((pgemm_kernel<QDEC_GLU, WN, XW, NWM>), grid, block, 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipSuccess;
}

hipError_t launch_pgemm(const PgemmParams &p, uint32_t flags, hipStream_t s) {
  if (p.tile_rows == 64) return launch_pgemm_tile<2, 2, 2>(p, flags, s);
  return p.tile_cols == 256 ? launch_pgemm_tile<8, kPg256Xw, 256 / (16 * kPg256Xw)>(p, flags, s)
                            : launch_pgemm_tile<4, kPg128Xw, 256 / (16 * kPg128Xw)>(p, flags, s);
}

// Grouped row kernels from this many rows (below it one workgroup per row
// or per 16-row tile leaves the GPU short of workgroups: a 512-token prompt
// measured 10.0 ms with the per-row kernels and 11.8 with the grouped ones;
// 32 x 1024-row chunks 5% faster with the grouped ones).
constexpr int kGroupedRows = 4096;

hipError_t launch_prefill_qk(const PqkParams &p, hipStream_t s) {
  if (p.batch * p.t_rows < kGroupedRows) {
    hipLaunchKernelGGL(pqk_row_kernel, dim3(p.batch * p.t_rows), dim3(256), 0, s, p);
    return hipSuccess;
  }
  const int ngrp = (p.t_rows + kPqRows - 1) / kPqRows;
  hipLaunchKernelGGL(pqk_kernel, dim3(p.batch * ngrp), dim3(256), 0, s, p);
  return hipSuccess;
}

bool pnorm_fits(int k, int rows) { return k <= 16 * kPnSteps * 32 && rows >= kGroupedRows; }

hipError_t launch_pnorm(const void *x, const void *norm_w, void *out, float eps, int rows, int k, int tiles,
                        hipStream_t s) {
  hipLaunchKernelGGL(pnorm_kernel, dim3(tiles), dim3(256), 0, s, reinterpret_cast<const uint16_t *>(x),
                     reinterpret_cast<const uint16_t *>(norm_w), reinterpret_cast<uint16_t *>(out), k, eps, rows,
                     tiles);
  return hipSuccess;
}

hipError_t launch_prefill_attn(const PattnParams &p, hipStream_t s) {
  const int nqb = (p.t_rows + kPaRows - 1) / kPaRows;
  const dim3 grid(nqb * p.batch * p.nkv);
  switch (p.nq / p.nkv) {
    case 2: hipLaunchKernelGGL(pattn_kernel<2>, grid, dim3(64 * 2 * pa_wph(2)), 0, s, p); break;
    case 4: hipLaunchKernelGGL(pattn_kernel<4>, grid, dim3(64 * 4 * pa_wph(4)), 0, s, p); break;
    case 8: hipLaunchKernelGGL((pattn_kernel<4, 8>), dim3(2 * grid.x), dim3(64 * 4 * pa_wph(4)), 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipSuccess;
}

}  // namespace qdec
