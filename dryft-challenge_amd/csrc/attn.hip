// GQA decode attention with the head RMSNorm, RoPE and KV-cache write fused
// in, for t_rows query rows per sequence (1 = plain decode, K+1 = verify).
//
// Grid (chunk, kv head, sequence), one wavefront each.  The wave:
//   1. builds the normalised, rotated queries of its G heads x t_rows rows in
//      registers, already in the B-operand layout of v_mfma_f32_16x16x32_bf16
//      (query row r = G*t + g sits in MFMA column r % 16 of M tile r / 16);
//   2. if its chunk overlaps the new slots lens[b] .. lens[b]+t_rows-1, builds
//      the new keys/values in LDS, and the chunk owning each new slot writes
//      it to the cache (nobody reads those cache slots in this launch);
//   3. walks its slots 32 at a time: S^T = K . Q^T (two 16-slot MFMA tiles
//      whose slot order is chosen so that the score registers are exactly the
//      B operand of the next product), online softmax in base 2, then
//      O^T += V^T . P^T with V read from the channel-major V cache;
//   4. writes o / l directly when the sequence needs one chunk, else stores
//      (acc, m, l) and the last chunk to arrive merges all chunks in order.
// Chunks are keyed to absolute slot numbers and every row's arithmetic is the
// same whatever t_rows is, so verify rows reproduce plain decode bit for bit.
//
// Reference behaviour replaced: engine/kernels/fused.py:360-479
// (_attn_fused_split_kernel), engine/kernels/ops.py:84-431 (_qkv_post_kernel,
// _decode_attn_split_kernel, _decode_attn_reduce_kernel) and
// notes/v10/spec.py:111-182 (_spec_attn_kernel).
#include "qdec_common.h"
#include "qdec_kernels.h"

namespace qdec {

namespace {

constexpr int kMaxT = 16;

template <int D, int G, int MTQ>
__global__ void __launch_bounds__(64) attn_kernel(const AttnParams p) {
  static_assert(D == 128, "head_dim 128 only");
  constexpr int DS = D / 32;   // MFMA k steps over the head dimension
  constexpr int DT = D / 16;   // 16-channel output tiles
  constexpr int HALF = DS / 2; // k-step distance of the rotate_half partner

  __shared__ __align__(16) uint16_t s_kn[kMaxT * D];
  __shared__ __align__(16) uint16_t s_vn[kMaxT * D];
  __shared__ uint32_t s_flag;

  const int c = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  const int lane = threadIdx.x;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int T = p.t_rows;
  const int R = T * G;
  const int L = p.lens[b];
  const int last = L + T - 1;
  const int c0 = c * p.chunk;
  if (L < 0 || last >= p.cap) return;  // never index outside the cache slab
  if (c0 > last) return;
  const int n_active = last / p.chunk + 1;
  const int nq = p.nq, nkv = p.nkv;
  const int width = (nq + 2 * nkv) * D;
  const uint16_t *qkv = reinterpret_cast<const uint16_t *>(p.qkv);
  const uint16_t *cos_t = reinterpret_cast<const uint16_t *>(p.cos_tab);
  const uint16_t *sin_t = reinterpret_cast<const uint16_t *>(p.sin_tab);
  const size_t slab = ((size_t)b * nkv + kvh) * (size_t)p.cap * D;
  uint16_t *kc = reinterpret_cast<uint16_t *>(p.k_cache) + slab;
  uint16_t *vc = reinterpret_cast<uint16_t *>(p.v_cache) + slab;

  // ---- 1. queries: RMSNorm over the head, RoPE, bf16, B-operand layout.
  uint4 qf[MTQ][DS];
  {
    uint4 wq[DS];
#pragma unroll
    for (int s = 0; s < DS; ++s)
      wq[s] = *reinterpret_cast<const uint4 *>(
          reinterpret_cast<const uint16_t *>(p.q_norm_w) + s * 32 + grp * 8);
#pragma unroll
    for (int mt = 0; mt < MTQ; ++mt) {
      const int r = mt * 16 + col;
      const bool valid = r < R;
      const int t = valid ? r / G : 0;
      const int hq = valid ? r % G : 0;
      float x[DS][8];
      float ss = 0.f;
      if (valid) {
        const uint16_t *src = qkv + (size_t)(b * T + t) * width + (size_t)(kvh * G + hq) * D;
#pragma unroll
        for (int s = 0; s < DS; ++s) {
          unpack8(*reinterpret_cast<const uint4 *>(src + s * 32 + grp * 8), x[s]);
#pragma unroll
          for (int e = 0; e < 8; ++e) ss += x[s][e] * x[s][e];
        }
      } else {
#pragma unroll
        for (int s = 0; s < DS; ++s)
#pragma unroll
          for (int e = 0; e < 8; ++e) x[s][e] = 0.f;
      }
      ss += shfl_xor(ss, 16);
      ss += shfl_xor(ss, 32);
      if (valid) {
        const float rstd = 1.0f / sqrtf(ss / (float)D + p.eps);
        float y[DS][8];
#pragma unroll
        for (int s = 0; s < DS; ++s) {
          float w[8];
          unpack8(wq[s], w);
#pragma unroll
          for (int e = 0; e < 8; ++e) y[s][e] = rbf(w[e] * rbf(x[s][e] * rstd));
        }
        const int pos = L + t;
#pragma unroll
        for (int s = 0; s < DS; ++s) {
          float cs[8], sn[8], o[8];
          unpack8(*reinterpret_cast<const uint4 *>(cos_t + (size_t)pos * D + s * 32 + grp * 8), cs);
          unpack8(*reinterpret_cast<const uint4 *>(sin_t + (size_t)pos * D + s * 32 + grp * 8), sn);
          const int ps = s ^ HALF;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float rot = (s < HALF) ? -y[ps][e] : y[ps][e];
            o[e] = rbf(y[s][e] * cs[e]) + rbf(rot * sn[e]);
          }
          qf[mt][s] = pack8(o);
        }
      } else {
#pragma unroll
        for (int s = 0; s < DS; ++s) qf[mt][s] = zero4();
      }
    }
  }

  // ---- 2. new keys / values of slots L .. last.
  const int c1 = c0 + p.chunk;  // exclusive end of this chunk
  const bool overlap = c1 > L;
  if (overlap) {
    const uint16_t *kw = reinterpret_cast<const uint16_t *>(p.k_norm_w);
    const float w0 = bf2f(kw[2 * lane]), w1 = bf2f(kw[2 * lane + 1]);
    for (int t = 0; t < T; ++t) {
      const uint16_t *row = qkv + (size_t)(b * T + t) * width;
      const uint32_t kr = *reinterpret_cast<const uint32_t *>(row + (size_t)(nq + kvh) * D + 2 * lane);
      const uint32_t vr =
          *reinterpret_cast<const uint32_t *>(row + (size_t)(nq + nkv + kvh) * D + 2 * lane);
      const float k0 = lo16(kr), k1 = hi16(kr);
      float ss = k0 * k0 + k1 * k1;
      ss += shfl_xor(ss, 32);
      ss += shfl_xor(ss, 16);
      ss += shfl_xor(ss, 8);
      ss += shfl_xor(ss, 4);
      ss += shfl_xor(ss, 2);
      ss += shfl_xor(ss, 1);
      const float rstd = 1.0f / sqrtf(ss / (float)D + p.eps);
      const float y0 = rbf(w0 * rbf(k0 * rstd));
      const float y1 = rbf(w1 * rbf(k1 * rstd));
      // channel 2*lane pairs with 2*lane +- D/2, held by lane ^ 32.
      const float p0 = shfl_xor(y0, 32), p1 = shfl_xor(y1, 32);
      const bool first_half = lane < 32;
      const float r0 = first_half ? -p0 : p0;
      const float r1 = first_half ? -p1 : p1;
      const int pos = L + t;
      const uint32_t cw = *reinterpret_cast<const uint32_t *>(cos_t + (size_t)pos * D + 2 * lane);
      const uint32_t sw = *reinterpret_cast<const uint32_t *>(sin_t + (size_t)pos * D + 2 * lane);
      const float o0 = rbf(y0 * lo16(cw)) + rbf(r0 * lo16(sw));
      const float o1 = rbf(y1 * hi16(cw)) + rbf(r1 * hi16(sw));
      const uint32_t kout = pack2(o0, o1);
      *reinterpret_cast<uint32_t *>(s_kn + t * D + 2 * lane) = kout;
      *reinterpret_cast<uint32_t *>(s_vn + t * D + 2 * lane) = vr;
      if (pos >= c0 && pos < c1) {  // this chunk owns the slot
        *reinterpret_cast<uint32_t *>(kc + (size_t)pos * D + 2 * lane) = kout;
        uint16_t *vb = vc + ((size_t)(pos >> 3) * D) * 8 + (pos & 7);
        vb[(size_t)(2 * lane) * 8] = (uint16_t)(vr & 0xffffu);
        vb[(size_t)(2 * lane + 1) * 8] = (uint16_t)(vr >> 16);
      }
    }
    __syncthreads();
  }

  // ---- 3. flash-decode over the chunk.
  const float NEG_INF = -__builtin_huge_valf();
  f32x4_t acc[MTQ][DT];
  float m_run[MTQ], l_run[MTQ];
#pragma unroll
  for (int mt = 0; mt < MTQ; ++mt) {
    m_run[mt] = NEG_INF;
    l_run[mt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[mt][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  // Per-row visibility limit (highest slot the row may see).
  int lim[MTQ];
#pragma unroll
  for (int mt = 0; mt < MTQ; ++mt) {
    const int r = mt * 16 + col;
    lim[mt] = (r < R) ? L + r / G : -1;
  }

  const int end = min(c1, last + 1);
  for (int s0 = c0; s0 < end; s0 += 32) {
    // K operand: tile a rows m -> slot s0 + 8*(m>>2) + (m&3), tile b -> +4.
    const int slot_a = s0 + 8 * (col >> 2) + (col & 3);
    const int slot_b = slot_a + 4;
    uint4 ka[DS], kb[DS], vf[DT];
    const bool fresh = s0 + 32 > L;  // block touches new or unwritten slots
#pragma unroll
    for (int s = 0; s < DS; ++s) {
      ka[s] = *reinterpret_cast<const uint4 *>(kc + (size_t)slot_a * D + s * 32 + grp * 8);
      kb[s] = *reinterpret_cast<const uint4 *>(kc + (size_t)slot_b * D + s * 32 + grp * 8);
    }
    const uint16_t *vblk = vc + ((size_t)((s0 >> 3) + grp) * D) * 8;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      vf[dt] = *reinterpret_cast<const uint4 *>(vblk + (size_t)(dt * 16 + col) * 8);
    if (fresh) {
#pragma unroll
      for (int s = 0; s < DS; ++s) {
        if (slot_a >= L)
          ka[s] = (slot_a <= last) ? *reinterpret_cast<const uint4 *>(s_kn + (slot_a - L) * D + s * 32 + grp * 8)
                                   : zero4();
        if (slot_b >= L)
          kb[s] = (slot_b <= last) ? *reinterpret_cast<const uint4 *>(s_kn + (slot_b - L) * D + s * 32 + grp * 8)
                                   : zero4();
      }
      const int vs0 = s0 + 8 * grp;  // first slot of this lane's V group
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        uint16_t e16[8];
        *reinterpret_cast<uint4 *>(e16) = vf[dt];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int slot = vs0 + e;
          if (slot > last)
            e16[e] = 0;
          else if (slot >= L)
            e16[e] = s_vn[(slot - L) * D + dt * 16 + col];
        }
        vf[dt] = *reinterpret_cast<const uint4 *>(e16);
      }
    }
#pragma unroll
    for (int mt = 0; mt < MTQ; ++mt) {
      f32x4_t sa = f32x4_t{0.f, 0.f, 0.f, 0.f}, sb = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < DS; ++s) {
        sa = mfma16x16x32(ka[s], qf[mt][s], sa);
        sb = mfma16x16x32(kb[s], qf[mt][s], sb);
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
      for (int j = 1; j < 8; ++j) bmax = fmaxf(bmax, sc[j]);
      bmax = fmaxf(bmax, shfl_xor(bmax, 16));
      bmax = fmaxf(bmax, shfl_xor(bmax, 32));
      const float m_new = fmaxf(m_run[mt], bmax);
      const float alpha = (m_new == NEG_INF) ? 1.0f : exp2f(m_run[mt] - m_new);
      float pj[8];
      float psum = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        pj[j] = (sc[j] == NEG_INF) ? 0.f : exp2f(sc[j] - m_new);
        psum += pj[j];
      }
      l_run[mt] = l_run[mt] * alpha + psum;
      m_run[mt] = m_new;
      const uint4 pf = pack8(pj);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        acc[mt][dt] *= alpha;
        acc[mt][dt] = mfma16x16x32(vf[dt], pf, acc[mt][dt]);
      }
    }
  }

  // ---- 4. output or chunk partials + merge.
  float l_tot[MTQ];
#pragma unroll
  for (int mt = 0; mt < MTQ; ++mt) {
    float v = l_run[mt] + shfl_xor(l_run[mt], 16);
    v += shfl_xor(v, 32);
    l_tot[mt] = v;
  }
  uint16_t *out = reinterpret_cast<uint16_t *>(p.out);
  if (n_active == 1) {
#pragma unroll
    for (int mt = 0; mt < MTQ; ++mt) {
      const int r = mt * 16 + col;
      if (r >= R) continue;
      const int t = r / G, hq = r % G;
      uint16_t *dst = out + (size_t)(b * T + t) * nq * D + (size_t)(kvh * G + hq) * D;
      const float inv_l = l_tot[mt];
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        uint2 o;
        o.x = pack2(acc[mt][dt][0] / inv_l, acc[mt][dt][1] / inv_l);
        o.y = pack2(acc[mt][dt][2] / inv_l, acc[mt][dt][3] / inv_l);
        *reinterpret_cast<uint2 *>(dst + dt * 16 + grp * 4) = o;
      }
    }
    return;
  }

  // partial layout per (b, kvh, chunk): R rows x (D acc + m + l) floats.
  const size_t rstride = D + 2;
  const size_t seq_base = ((size_t)b * nkv + kvh) * p.nchunks;
  float *part = p.partial + (seq_base + c) * (size_t)R * rstride;
#pragma unroll
  for (int mt = 0; mt < MTQ; ++mt) {
    const int r = mt * 16 + col;
    if (r >= R) continue;
    float *pr = part + (size_t)r * rstride;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) store_coherent(pr + dt * 16 + grp * 4 + i, acc[mt][dt][i]);
    if (grp == 0) {
      store_coherent(pr + D, m_run[mt]);
      store_coherent(pr + D + 1, l_tot[mt]);
    }
  }
  if (!arrive_last(p.counters + (size_t)b * nkv + kvh, (uint32_t)n_active, &s_flag)) return;

#pragma unroll
  for (int mt = 0; mt < MTQ; ++mt) {
    const int r = mt * 16 + col;
    if (r >= R) continue;
    float mmax = NEG_INF;
    for (int cc = 0; cc < n_active; ++cc) {
      const float *pr = p.partial + (seq_base + cc) * (size_t)R * rstride + (size_t)r * rstride;
      mmax = fmaxf(mmax, load_coherent(pr + D));
    }
    float lsum = 0.f;
    f32x4_t o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int cc = 0; cc < n_active; ++cc) {
      const float *pr = p.partial + (seq_base + cc) * (size_t)R * rstride + (size_t)r * rstride;
      const float mc = load_coherent(pr + D);
      if (mc == NEG_INF) continue;
      const float w = exp2f(mc - mmax);
      lsum += load_coherent(pr + D + 1) * w;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) o[dt][i] += load_coherent(pr + dt * 16 + grp * 4 + i) * w;
    }
    const int t = r / G, hq = r % G;
    uint16_t *dst = out + (size_t)(b * T + t) * nq * D + (size_t)(kvh * G + hq) * D;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      uint2 ov;
      ov.x = pack2(o[dt][0] / lsum, o[dt][1] / lsum);
      ov.y = pack2(o[dt][2] / lsum, o[dt][3] / lsum);
      *reinterpret_cast<uint2 *>(dst + dt * 16 + grp * 4) = ov;
    }
  }
}

}  // namespace

hipError_t launch_attn(const AttnParams &p, hipStream_t s) {
  const int R = p.t_rows * (p.nq / p.nkv);
  const int mtq = (R + 15) / 16;
  dim3 grid(p.nchunks, p.nkv, p.batch);
  dim3 block(64);
  switch (mtq) {
    case 1: hipLaunchKernelGGL((attn_kernel<128, 4, 1>), grid, block, 0, s, p); break;
    case 2: hipLaunchKernelGGL((attn_kernel<128, 4, 2>), grid, block, 0, s, p); break;
    case 3: hipLaunchKernelGGL((attn_kernel<128, 4, 3>), grid, block, 0, s, p); break;
    case 4: hipLaunchKernelGGL((attn_kernel<128, 4, 4>), grid, block, 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipSuccess;
}

}  // namespace qdec
