// Device body of the GQA decode attention with the head RMSNorm, RoPE and KV-cache write fused
// in, for t_rows query rows per sequence (1 = plain decode, K+1 = verify).
//
// Grid (chunk, kv head, sequence); a workgroup of NW = 4 or 8 wavefronts per
// cell (the wave count, like the chunk, is part of the call: a row's
// arithmetic depends on both, never on t_rows).  A chunk is a contiguous
// slot range, or (strided, 8 waves) every C-th 32-slot block of the cache.
//   1. Query row r = G*t + g and new key/value row t go to the wave whose
//      row index rw (wave + 4 mod 8 with 8 waves, else the wave) is r or t
//      mod NW.  A wave holding rows loads them, and a lane holds two
//      channels of a row, so the head RMSNorm is one wave reduction and the
//      rotate_half partner sits in lane ^ 32.  Normalised, rotated queries
//      go to LDS; new keys go to LDS in row layout, new values in the
//      channel-major cache layout, and the chunk owning a new slot writes it
//      to the cache (nobody reads those cache slots in this launch).
//      K/V blocks: a wave issues its first 32-slot block before the sequence
//      length arrives (its first two in contiguous chunk 0) and a second one
//      once the length says the chunk needs it -- except, with fewer query
//      rows than waves (plain decode at 8 waves), the waves holding rows,
//      which prepare them first and then issue their blocks.
//   2. Each wave reads the queries back in the B-operand layout of
//      v_mfma_f32_16x16x32_bf16 (query row r sits in MFMA column r % 16 of M
//      tile r / 16) and walks its blocks (block j to wave j % NW, two blocks in
//      flight): S^T = K . Q^T (two 16-slot MFMA tiles whose slot order makes
//      the score registers exactly the B operand of the next product), online
//      softmax in base 2, then O^T += V^T . P^T with V read from the
//      channel-major V cache.  The block holding the new slots takes them
//      from LDS with masks; slots past the last new one are zero.
//   3. The waves merge in LDS in wave order; a sequence that needs one chunk
//      is written out directly, otherwise the workgroup stores (acc, m, l) and
//      the last chunk to arrive merges all chunks in chunk order -- or, with
//      out_partials, every chunk stores its partials and the consuming GEMM
//      merges them (gemm.hip, attn_merge8) with the same arithmetic.
// Block-to-wave dealing and chunk boundaries are keyed to absolute slot
// numbers, and every row's arithmetic is the same whatever t_rows is, so
// verify rows reproduce plain decode bit for bit.
//
// Reference behaviour replaced: engine/kernels/fused.py:360-479
// (_attn_fused_split_kernel), engine/kernels/ops.py:84-431 (_qkv_post_kernel,
// _decode_attn_split_kernel, _decode_attn_reduce_kernel) and
// notes/v10/spec.py:111-182 (_spec_attn_kernel).
#pragma once

#include "qdec_common.h"
#include "qdec_kernels.h"

namespace qdec {

constexpr int kMaxT = 16;
constexpr int kAttnRowStride = 128 + 8;  // bf16 per LDS row of queries / new keys (bank spread)
// LDS layout of a workgroup of NW waves (bytes).
template <int NW>
struct AttnLds {
  static constexpr int kn = 0;                             // new keys [kMaxT][row stride]
  static constexpr int vp = kn + kMaxT * kAttnRowStride * 2;  // new values [3][128][8]
  static constexpr int q = vp + 3 * 128 * 8 * 2;           // queries [64][row stride] or
                                                           // wave partials [NW][8][64] f32x4
  static constexpr int m = q + NW * 8 * 64 * 16;           // wave row maxima [NW][16]
  static constexpr int l = m + NW * 16 * 4;                // wave row sums [NW][16]
  static constexpr int flag = l + NW * 16 * 4;
  static constexpr int bytes = flag + 16;
  static_assert(64 * kAttnRowStride * 2 <= NW * 8 * 64 * 16, "query rows fit the partials area");
};

// COH: the projection rows are read and the chunk partials written at device
// scope, for a body that shares its launch with their producer and consumer.
// GQ: query heads per kv head, 4 (Qwen3-4B and -8B) or 0 for the group
// size of the call (nq / nkv: 2 for Qwen3-0.6B and -1.7B, 5 for -14B, 8 for
// -32B), with at most 16 * MTQ query rows per kv head.
// STR: strided chunks (the call's strided flag, as a constant).
template <int D, int GQ, int MTQ, int NW, bool COH = false, bool STR = false>
__device__ __forceinline__ void attn_block(const AttnParams &p, const int c, const int kvh, const int b,
                                           unsigned char *smem) {
  static_assert((D == 128 && (GQ == 4 || GQ == 0)) || (D == 64 && GQ == 0),
                "head_dim 128 (4 query heads per kv head, or the call's count) or 64");
  static_assert((D / 16) % NW == 0, "every wave finishes whole 16-channel tiles");
  const int G = GQ > 0 ? GQ : p.nq / p.nkv;
  static_assert(NW == 4 || NW == 8, "4 or 8 waves");
  using LY = AttnLds<NW>;
  constexpr int DS = D / 32;              // MFMA k steps over the head dimension
  constexpr int DT = D / 16;              // 16-channel output tiles
  constexpr int DTW = DT / NW;            // output tiles each wave finishes
  constexpr bool DB = MTQ == 1;           // two blocks in flight (register budget)
  constexpr int QPW = MTQ * 16 / NW;      // query rows per wave, at most
  constexpr int KPW = kMaxT / NW;         // new rows per wave, at most
  constexpr int RS = kAttnRowStride;
  // A head row is 2 channels per lane on lanes 0 .. D/2 - 1; with D = 64 the
  // other lanes load lane D/2 - 1's channels, use zeros and store nothing.
  constexpr int LH = D / 2;

  uint16_t *s_kn = reinterpret_cast<uint16_t *>(smem + LY::kn);
  uint16_t *s_vp = reinterpret_cast<uint16_t *>(smem + LY::vp);
  uint16_t *s_q = reinterpret_cast<uint16_t *>(smem + LY::q);
  f32x4_t *s_acc = reinterpret_cast<f32x4_t *>(smem + LY::q);
  float *s_m = reinterpret_cast<float *>(smem + LY::m);
  float *s_l = reinterpret_cast<float *>(smem + LY::l);
  uint32_t *s_flag = reinterpret_cast<uint32_t *>(smem + LY::flag);

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int cl = 2 * min(lane, LH - 1);  // this lane's first channel of a head row
  const bool lv = lane < LH;
  const int T = p.t_rows;
  const int R = T * G;
  // Chunk c takes the contiguous slots [c0, c1), or with strided chunks the
  // 32-slot blocks c, c + C, c + 2C, ... of the cache (C = p.nchunks): then
  // every chunk of a partly filled cache has the same number of blocks, give
  // or take one.  Local block j of the chunk starts at slot bs0(j).
  const int C = p.nchunks;
  constexpr bool strided = STR;
  const int c0 = strided ? 32 * c : c * p.chunk;
  const int c1 = c0 + p.chunk;  // exclusive end of a contiguous chunk
  auto bs0 = [&](int j) { return strided ? 32 * (c + C * j) : c0 + 32 * j; };
  const int nq = p.nq, nkv = p.nkv;
  const int width = (nq + 2 * nkv) * D;
  const uint16_t *qkv = reinterpret_cast<const uint16_t *>(p.qkv);
  const uint16_t *cos_t = reinterpret_cast<const uint16_t *>(p.cos_tab);
  const uint16_t *sin_t = reinterpret_cast<const uint16_t *>(p.sin_tab);
  const size_t slab = ((size_t)b * nkv + kvh) * (size_t)p.cap * D;
  uint16_t *kc = reinterpret_cast<uint16_t *>(p.k_cache) + slab;
  uint16_t *vc = reinterpret_cast<uint16_t *>(p.v_cache) + slab;
  const float NEG_INF = -__builtin_huge_valf();

  // K / V fragments of one 32-slot block.  K tile a row m -> slot
  // s0 + 8*(m>>2) + (m&3), tile b -> +4; V from the channel-major cache.
  struct Frag {
    uint4 ka[DS], kb[DS], vf[DT];
  };
  auto load_block = [&](int s0, Frag &f) {
    const int slot_a = s0 + 8 * (col >> 2) + (col & 3);
    const int slot_b = slot_a + 4;
#pragma unroll
    for (int s = 0; s < DS; ++s) {
      f.ka[s] = ld_nt(kc + (size_t)slot_a * D + s * 32 + grp * 8);
      f.kb[s] = ld_nt(kc + (size_t)slot_b * D + s * 32 + grp * 8);
    }
    const uint16_t *vblk = vc + ((size_t)((s0 >> 3) + grp) * D) * 8;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      f.vf[dt] = ld_nt(vblk + (size_t)(dt * 16 + col) * 8);
  };
  // The first block of this wave (both, in chunk 0) and the raw query / new
  // key / new value rows go out before the sequence length is known: none
  // of their addresses depends on it (blocks are issued when they lie inside
  // the chunk and the cache; the ones past the length are never used).  A
  // later chunk's second block waits for the length: the chunk holding the
  // newest slots is usually part-filled, and the one after it empty
  // (MI355X, ms per step: batch 8 at 1300 tokens 2.987 -> 2.963, batch 4 at
  // 1024 2.486 -> 2.464).
  //
  // Rows go to waves by rw: with 8 waves the query rows and new key rows
  // start at wave 4, whose blocks (4..7 mod 8) are a chunk's last to get a
  // second one.  With fewer query rows than waves (a plain step at 8 waves)
  // the waves holding rows load and prepare them first and only then issue
  // their blocks: a wave that has issued its block loads stalls in that
  // issue until the memory pipeline drains (measured on MI355X), and the
  // rows would wait with it.  The other waves issue their blocks first.
  const int rw = NW == 8 ? (wave + 4) & 7 : wave;
  const bool late = R < NW && rw < R;
  auto block_in = [&](int j) { return (strided || 32 * j < p.chunk) && bs0(j) + 32 <= p.cap; };
  Frag f0, f1;
  if (!late) {
    if (block_in(wave)) load_block(bs0(wave), f0);
    if constexpr (DB) {
      if constexpr (!STR) {
        if (c == 0 && block_in(wave + NW)) load_block(bs0(wave + NW), f1);
      }
    }
  }
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  // Only the waves holding rows load them (and their norm weights and
  // rotation tables): an unused load still pending where its register is
  // reused would make the wave wait for every load issued after it.
  uint32_t qraw[QPW], kraw[KPW], vraw[KPW];
#pragma unroll
  for (int i = 0; i < QPW; ++i) {
    const int r = rw + NW * i;
    qraw[i] = 0u;
    if (r < R) {  // uniform per wave
      const int t = r / G, hq = r % G;
      qraw[i] = ldv4<COH>(qkv + (size_t)(b * T + t) * width + (size_t)(kvh * G + hq) * D + cl);
      if (!lv) qraw[i] = 0u;
    }
  }
#pragma unroll
  for (int i = 0; i < KPW; ++i) {
    const int t = rw + NW * i;
    kraw[i] = vraw[i] = 0u;
    if (t < T) {
      const uint16_t *row = qkv + (size_t)(b * T + t) * width;
      kraw[i] = ldv4<COH>(row + (size_t)(nq + kvh) * D + cl);
      vraw[i] = ldv4<COH>(row + (size_t)(nq + nkv + kvh) * D + cl);
      if (!lv) kraw[i] = 0u;
    }
  }
  const bool has_q = rw < R, has_k = rw < T;
  const uint32_t qw =
      has_q ? *reinterpret_cast<const uint32_t *>(reinterpret_cast<const uint16_t *>(p.q_norm_w) + cl) : 0u;
  const uint32_t kw =
      has_k ? *reinterpret_cast<const uint32_t *>(reinterpret_cast<const uint16_t *>(p.k_norm_w) + cl) : 0u;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);

  const int L = p.lens[b];
  const int last = L + T - 1;
  uint16_t *out = reinterpret_cast<uint16_t *>(p.out);
  // Output row m, column k (row-major, or fragment order for a direct GEMM).
  auto out_at = [&](int m, int k) { return p.ofrag ? out + frag_off(m, k, p.ofrag) : out + (size_t)m * nq * D + k; };
  if (L < 0 || last >= p.cap) {
    // Never index outside the cache slab.  The rows of this (sequence, kv
    // head) become NaN (written by chunk 0; with out_partials the consuming
    // GEMM's merge makes the same check), so the step's argmax yields an
    // out-of-vocabulary id instead of a token computed from stale data.
    if (c == 0 && !p.out_partials) {
      for (int i = threadIdx.x; i < R * (D / 4); i += blockDim.x) {
        const int r = i / (D / 4), k4 = (i - r * (D / 4)) * 4;
        *reinterpret_cast<uint2 *>(out_at(b * T + r / G, (kvh * G + r % G) * D + k4)) = make_uint2(0x7fc07fc0u, 0x7fc07fc0u);
      }
    }
    return;
  }
  if (c0 > last) return;  // (strided: the chunk's first block lies past the last slot)
  const int n_active = strided ? min(C, (last >> 5) + 1) : last / p.chunk + 1;
  const int nb = strided ? ((last >> 5) - c) / C + 1 : (min(c1, last + 1) - c0 + 31) / 32;  // blocks in this chunk
  if constexpr (DB) {
    if (!late && (c > 0 || strided) && wave + NW < nb) load_block(bs0(wave + NW), f1);
  }
  __atomic_signal_fence(__ATOMIC_SEQ_CST);

  // ---- 1. rotation tables of the rows' positions.
  // this chunk holds some of the new slots L..last (blocks L/32 .. last/32)
  const bool overlap = strided ? ((last >> 5) - (L >> 5) + 1 >= C || (c - (L >> 5) % C + C) % C <= (last >> 5) - (L >> 5))
                               : c1 > L;
  uint32_t qcos[QPW], qsin[QPW], kcos[KPW], ksin[KPW];
#pragma unroll
  for (int i = 0; i < QPW; ++i) {
    const int r = rw + NW * i;
    qcos[i] = qsin[i] = 0u;
    if (r < R) {
      const int t = r / G;
      qcos[i] = *reinterpret_cast<const uint32_t *>(cos_t + (size_t)(L + t) * D + cl);
      qsin[i] = *reinterpret_cast<const uint32_t *>(sin_t + (size_t)(L + t) * D + cl);
    }
  }
#pragma unroll
  for (int i = 0; i < KPW; ++i) {
    const int t = rw + NW * i;
    kcos[i] = ksin[i] = 0u;
    if (overlap && t < T) {
      kcos[i] = *reinterpret_cast<const uint32_t *>(cos_t + (size_t)(L + t) * D + cl);
      ksin[i] = *reinterpret_cast<const uint32_t *>(sin_t + (size_t)(L + t) * D + cl);
    }
  }

  // Head RMSNorm and RoPE of the two channels 2*lane, 2*lane+1 of one head row.
  auto norm_rope = [&](uint32_t raw, uint32_t w, uint32_t cw, uint32_t sw) -> uint32_t {
    return head_norm_rope<D>(raw, w, cw, sw, p.eps);
  };
#pragma unroll
  for (int i = 0; i < QPW; ++i) {
    const int r = rw + NW * i;
    if (r < R) {  // uniform per wave: the norm's wave sum runs on every lane
      const uint32_t qo = norm_rope(qraw[i], qw, qcos[i], qsin[i]);
      if (lv) *reinterpret_cast<uint32_t *>(s_q + r * RS + cl) = qo;
    }
  }
  uint32_t kout[KPW];
  if (overlap) {
    const int g0 = L >> 3;
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
      const int t = rw + NW * i;
      if (t < T) {
        kout[i] = norm_rope(kraw[i], kw, kcos[i], ksin[i]);
        const uint32_t vr = vraw[i];
        const int slot = L + t;
        const int gi = (slot >> 3) - g0, e = slot & 7;
        if (lv) {
          *reinterpret_cast<uint32_t *>(s_kn + t * RS + cl) = kout[i];
          s_vp[(gi * D + cl) * 8 + e] = (uint16_t)(vr & 0xffffu);
          s_vp[(gi * D + cl + 1) * 8 + e] = (uint16_t)(vr >> 16);
        }
      }
    }
  }
  // With contiguous chunks the late waves' blocks go out here, before the
  // cache write below (a pending store would hold them back); with strided
  // chunks after the barrier (below).
  if (late && !STR) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (wave < nb) load_block(bs0(wave), f0);
    if constexpr (DB) {
      if (wave + NW < nb) load_block(bs0(wave + NW), f1);
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
  }
  // The chunk owning a new slot writes it to the cache (nobody reads those
  // cache slots in this launch).
  if (overlap) {
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
      const int t = rw + NW * i;
      const int slot = L + t;
      if (t < T && lv && (strided ? (slot >> 5) % C == c : (slot >= c0 && slot < c1))) {
        const uint32_t vr = vraw[i];
        const int e = slot & 7;
        *reinterpret_cast<uint32_t *>(kc + (size_t)slot * D + cl) = kout[i];
        uint16_t *vb = vc + ((size_t)(slot >> 3) * D) * 8 + e;
        vb[(size_t)cl * 8] = (uint16_t)(vr & 0xffffu);
        vb[(size_t)(cl + 1) * 8] = (uint16_t)(vr >> 16);
      }
    }
  }
  lds_barrier();  // the rows are in LDS; the blocks may still be in flight
  // Strided chunks: the late waves issue their blocks only now (a wave
  // stalls in the issue of its block loads, and the other waves would wait
  // for it at the barrier).  Measured on MI355X, attention us per launch
  // (before / after the barrier): batch 8 14.58 / 13.89; but batch 32's
  // whole-cache chunks 84.1 / 84.6, so contiguous chunks issue them before.
  if (late && STR) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (wave < nb) load_block(bs0(wave), f0);
    if constexpr (DB) {
      if (wave + NW < nb) load_block(bs0(wave + NW), f1);
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
  }

  // ---- 2. flash-decode over this wave's blocks.
  uint4 qf[MTQ][DS];
  f32x4_t acc[MTQ][DT];
  float m_run[MTQ], l_run[MTQ];
  int lim[MTQ];  // highest slot each row may see
#pragma unroll
  for (int mt = 0; mt < MTQ; ++mt) {
    const int r = mt * 16 + col;
#pragma unroll
    for (int s = 0; s < DS; ++s)
      qf[mt][s] = (r < R) ? *reinterpret_cast<const uint4 *>(s_q + r * RS + s * 32 + grp * 8) : zero4();
    m_run[mt] = NEG_INF;
    l_run[mt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[mt][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    lim[mt] = (r < R) ? L + r / G : -1;
  }

  // New slots L..last come from LDS; slots past `last` are zero (the cache
  // may hold anything there, and 0 * NaN would poison the product).
  auto patch = [&](Frag &f, int s0) {
    const int slot_a = s0 + 8 * (col >> 2) + (col & 3);
    const int slot_b = slot_a + 4;
    const int ia = slot_a - L, ib = slot_b - L;
    const bool new_a = (unsigned)ia < (unsigned)T, new_b = (unsigned)ib < (unsigned)T;
    const bool zero_a = slot_a > last, zero_b = slot_b > last;
    const uint16_t *kna = s_kn + min(max(ia, 0), kMaxT - 1) * RS + grp * 8;
    const uint16_t *knb = s_kn + min(max(ib, 0), kMaxT - 1) * RS + grp * 8;
#pragma unroll
    for (int s = 0; s < DS; ++s) {
      const uint4 va = *reinterpret_cast<const uint4 *>(kna + s * 32);
      const uint4 vb = *reinterpret_cast<const uint4 *>(knb + s * 32);
      f.ka[s] = new_a ? va : (zero_a ? zero4() : f.ka[s]);
      f.kb[s] = new_b ? vb : (zero_b ? zero4() : f.kb[s]);
    }
    // V: this lane's 8 slots vs0..vs0+7 of one channel per tile; keep the
    // cache below L, take LDS for L..last, zero above.
    const int vs0 = s0 + 8 * grp;
    const int gi = min(max((vs0 >> 3) - (L >> 3), 0), 2);
    uint32_t keep[4], take[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const int e0 = vs0 + 2 * d, e1 = e0 + 1;
      keep[d] = (e0 < L ? 0x0000ffffu : 0u) | (e1 < L ? 0xffff0000u : 0u);
      take[d] = ((e0 >= L && e0 <= last) ? 0x0000ffffu : 0u) | ((e1 >= L && e1 <= last) ? 0xffff0000u : 0u);
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const uint4 vn = *reinterpret_cast<const uint4 *>(s_vp + (size_t)(gi * D + dt * 16 + col) * 8);
      uint4 &v = f.vf[dt];
      v.x = (v.x & keep[0]) | (vn.x & take[0]);
      v.y = (v.y & keep[1]) | (vn.y & take[1]);
      v.z = (v.z & keep[2]) | (vn.z & take[2]);
      v.w = (v.w & keep[3]) | (vn.w & take[3]);
    }
  };

  auto process = [&](Frag &f, int j) {
    const int s0 = bs0(j);
    if (s0 + 32 > L) patch(f, s0);  // block touches new or unwritten slots
#pragma unroll
    for (int mt = 0; mt < MTQ; ++mt) {
      f32x4_t sa = f32x4_t{0.f, 0.f, 0.f, 0.f}, sb = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < DS; ++s) {
        sa = mfma16x16x32(f.ka[s], qf[mt][s], sa);
        sb = mfma16x16x32(f.kb[s], qf[mt][s], sb);
      }
      // lane holds slots s0 + 8*grp + j, j = 0..7, of query row mt*16 + col.
      float sc[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int sl_a = s0 + 8 * grp + i;
        sc[i] = (sl_a <= lim[mt]) ? sa[i] * p.scale_log2 : NEG_INF;
        sc[4 + i] = (sl_a + 4 <= lim[mt]) ? sb[i] * p.scale_log2 : NEG_INF;
      }
      float bmax = sc[0];
#pragma unroll
      for (int e = 1; e < 8; ++e) bmax = fmaxf(bmax, sc[e]);
      bmax = fmaxf(bmax, shfl_xor(bmax, 16));
      bmax = fmaxf(bmax, shfl_xor(bmax, 32));
      const float m_new = fmaxf(m_run[mt], bmax);
      const float alpha = (m_new == NEG_INF) ? 1.0f : exp2f(m_run[mt] - m_new);
      float pj[8];
      float psum = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pj[e] = (sc[e] == NEG_INF) ? 0.f : exp2f(sc[e] - m_new);
        psum += pj[e];
      }
      l_run[mt] = l_run[mt] * alpha + psum;
      m_run[mt] = m_new;
      const uint4 pf = pack8(pj);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        acc[mt][dt] *= alpha;
        acc[mt][dt] = mfma16x16x32(f.vf[dt], pf, acc[mt][dt]);
      }
    }
  };

  if constexpr (DB) {
    for (int j = wave; j < nb; j += 2 * NW) {
      process(f0, j);
      if (j + 2 * NW < nb) load_block(bs0(j + 2 * NW), f0);
      if (j + NW < nb) {
        process(f1, j + NW);
        if (j + 3 * NW < nb) load_block(bs0(j + 3 * NW), f1);
      }
    }
  } else {
    for (int j = wave; j < nb; j += NW) {
      if (j != wave) load_block(bs0(j), f0);
      process(f0, j);
    }
  }

  // ---- 3. merge the waves (wave order), then output or chunk partials.
  // A sequence that needs one chunk is written out directly, unless the
  // caller asked for partials (a GEMM merging them in its prologue, with the
  // arithmetic of the merge below: one chunk gives tot * 1 / (Lrow * 1)).
  const bool direct = n_active == 1 && !p.out_partials;
  const size_t cstride = (size_t)R * (D + 2);  // floats per chunk partial: acc [R][D], m [R], l [R]
  float *part_b = p.partial + ((size_t)b * nkv + kvh) * p.nchunks * cstride;
  float *part = part_b + (size_t)c * cstride;
#pragma unroll
  for (int mt = 0; mt < MTQ; ++mt) {
    const int r = mt * 16 + col;
    float lw = l_run[mt] + shfl_xor(l_run[mt], 16);
    lw += shfl_xor(lw, 32);  // this wave's row sum
    __syncthreads();         // queries / the previous tile's partials are consumed
    if (grp == 0) {
      s_m[wave * 16 + col] = m_run[mt];
      s_l[wave * 16 + col] = lw;
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) s_acc[(wave * DT + dt) * 64 + lane] = acc[mt][dt];
    __syncthreads();
    float mw[NW];
    float M = NEG_INF;
#pragma unroll
    for (int w2 = 0; w2 < NW; ++w2) {
      mw[w2] = s_m[w2 * 16 + col];
      M = fmaxf(M, mw[w2]);
    }
    float scw[NW];
    float Lrow = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < NW; ++w2) {
      scw[w2] = (mw[w2] == NEG_INF) ? 0.f : exp2f(mw[w2] - M);
      Lrow += s_l[w2 * 16 + col] * scw[w2];
    }
#pragma unroll
    for (int i = 0; i < DTW; ++i) {
      const int dt = wave + NW * i;
      f32x4_t tot = s_acc[dt * 64 + lane] * scw[0];
#pragma unroll
      for (int w2 = 1; w2 < NW; ++w2) tot += s_acc[(w2 * DT + dt) * 64 + lane] * scw[w2];
      if (r < R) {
        if (direct) {
          const int t = r / G, hq = r % G;
          uint2 o;
          o.x = pack2(tot[0] / Lrow, tot[1] / Lrow);
          o.y = pack2(tot[2] / Lrow, tot[3] / Lrow);
          *reinterpret_cast<uint2 *>(out_at(b * T + t, (kvh * G + hq) * D + dt * 16 + grp * 4)) = o;
        } else {
          float *dst = part + (size_t)r * D + dt * 16 + grp * 4;
          if (p.out_partials && !COH)  // read by the next launch only
            *reinterpret_cast<f32x4_t *>(dst) = tot;
          else
            store_coherent4(dst, tot);
        }
      }
    }
    if (!direct && wave == 0 && grp == 0 && r < R) {
      if (p.out_partials && !COH) {
        part[(size_t)R * D + r] = M;
        part[(size_t)R * D + R + r] = Lrow;
      } else {
        store_coherent(part + (size_t)R * D + r, M);
        store_coherent(part + (size_t)R * D + R + r, Lrow);
      }
    }
  }
  if (direct || p.out_partials) return;  // done, or the consuming GEMM merges
  if (!arrive_last(p.counters + (size_t)b * nkv + kvh, (uint32_t)n_active, s_flag)) return;

  // Merge chunks 0..n_active-1 in order (chunks a row cannot see have
  // m = -inf and are skipped).  Up to CB chunks are loaded in one batch; more
  // take one batch of maxima and one of partials per CB chunks.
  constexpr int CB = 8;
#pragma unroll
  for (int mt = 0; mt < MTQ; ++mt) {
    const int r = mt * 16 + col;
    if (r >= R) continue;
    float mc[CB], lc[CB];
    f32x4_t av[DTW][CB];
    auto load_group = [&](int cc) {
#pragma unroll
      for (int j = 0; j < CB; ++j) {
        const float *pr = part_b + (size_t)min(cc + j, n_active - 1) * cstride;
        mc[j] = load_coherent(pr + (size_t)R * D + r);
        lc[j] = load_coherent(pr + (size_t)R * D + R + r);
#pragma unroll
        for (int i = 0; i < DTW; ++i) av[i][j] = load_coherent4(pr + (size_t)r * D + (wave + NW * i) * 16 + grp * 4);
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
      for (int j = 0; j < CB; ++j)
        mg[j] = load_coherent(part_b + (size_t)min(cc + j, n_active - 1) * cstride + (size_t)R * D + r);
#pragma unroll
      for (int j = 0; j < CB; ++j)
        if (cc + j < n_active) mmax = fmaxf(mmax, mg[j]);
    }
    float lsum = 0.f;
    f32x4_t o[DTW];
#pragma unroll
    for (int i = 0; i < DTW; ++i) o[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int cc = 0; cc < n_active; cc += CB) {
      if (cc > 0) load_group(cc);
#pragma unroll
      for (int j = 0; j < CB; ++j) {
        if (cc + j >= n_active || mc[j] == NEG_INF) continue;
        const float w = exp2f(mc[j] - mmax);
        lsum += lc[j] * w;
#pragma unroll
        for (int i = 0; i < DTW; ++i) o[i] += av[i][j] * w;
      }
    }
    const int t = r / G, hq = r % G;
#pragma unroll
    for (int i = 0; i < DTW; ++i) {
      uint2 ov;
      ov.x = pack2(o[i][0] / lsum, o[i][1] / lsum);
      ov.y = pack2(o[i][2] / lsum, o[i][3] / lsum);
      *reinterpret_cast<uint2 *>(out_at(b * T + t, (kvh * G + hq) * D + (wave + NW * i) * 16 + grp * 4)) = ov;
    }
  }
}

}  // namespace qdec
