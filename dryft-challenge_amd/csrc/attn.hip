// GQA decode attention with the head RMSNorm, RoPE and KV-cache write fused
// in, for t_rows query rows per sequence (1 = plain decode, K+1 = verify).
//
// Grid (chunk, kv head, sequence); a workgroup of NW wavefronts per cell.
//   1. Every wave builds the normalised, rotated queries of the G heads x
//      t_rows rows in registers, already in the B-operand layout of
//      v_mfma_f32_16x16x32_bf16 (query row r = G*t + g sits in MFMA column
//      r % 16 of M tile r / 16).
//   2. If the chunk overlaps the new slots lens[b] .. lens[b]+t_rows-1, wave 0
//      builds the new keys/values in LDS, and the chunk owning each new slot
//      writes it to the cache (nobody reads those cache slots in this launch).
//   3. The chunk's 32-slot blocks are dealt to the waves round robin (block j
//      to wave j % NW); each wave walks its blocks with the next one already
//      in flight: S^T = K . Q^T (two 16-slot MFMA tiles whose slot order makes
//      the score registers exactly the B operand of the next product), online
//      softmax in base 2, then O^T += V^T . P^T with V read from the
//      channel-major V cache.
//   4. The waves merge in LDS in wave order; a sequence that needs one chunk
//      is written out directly, otherwise the workgroup stores (acc, m, l) and
//      the last chunk to arrive merges all chunks in chunk order.
// Block-to-wave dealing and chunk boundaries are keyed to absolute slot
// numbers, and every row's arithmetic is the same whatever t_rows is, so
// verify rows reproduce plain decode bit for bit.
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
constexpr int kMaxWaves = 4;

template <int D, int G, int MTQ>
__global__ void __launch_bounds__(256) attn_kernel(const AttnParams p) {
  static_assert(D == 128, "head_dim 128 only");
  constexpr int DS = D / 32;   // MFMA k steps over the head dimension
  constexpr int DT = D / 16;   // 16-channel output tiles
  constexpr int HALF = DS / 2; // k-step distance of the rotate_half partner
  constexpr int DTH = DT / 2;  // output tiles merged per LDS round
  constexpr bool DB = MTQ == 1; // double-buffered block loads (register budget)

  __shared__ __align__(16) uint16_t s_kn[kMaxT * D];
  __shared__ __align__(16) uint16_t s_vn[kMaxT * D];
  __shared__ __align__(16) f32x4_t s_acc[kMaxWaves][DTH][64];
  __shared__ float s_m[kMaxWaves][16];
  __shared__ float s_l[kMaxWaves][16];
  __shared__ uint32_t s_flag;

  const int c = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int NW = blockDim.x >> 6;
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
  const int c1 = c0 + p.chunk;                    // exclusive end of this chunk
  const int nb = (min(c1, last + 1) - c0 + 31) / 32;  // blocks in this chunk
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
      f.ka[s] = *reinterpret_cast<const uint4 *>(kc + (size_t)slot_a * D + s * 32 + grp * 8);
      f.kb[s] = *reinterpret_cast<const uint4 *>(kc + (size_t)slot_b * D + s * 32 + grp * 8);
    }
    const uint16_t *vblk = vc + ((size_t)((s0 >> 3) + grp) * D) * 8;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      f.vf[dt] = *reinterpret_cast<const uint4 *>(vblk + (size_t)(dt * 16 + col) * 8);
  };
  // This wave's first block goes out before the query prologue.
  Frag cur, nxt;
  if (wave < nb) load_block(c0 + 32 * wave, nxt);

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
      {
        const uint16_t *src = qkv + (size_t)(b * T + t) * width + (size_t)(kvh * G + hq) * D;
#pragma unroll
        for (int s = 0; s < DS; ++s) {
          unpack8(*reinterpret_cast<const uint4 *>(src + s * 32 + grp * 8), x[s]);
#pragma unroll
          for (int e = 0; e < 8; ++e) ss += x[s][e] * x[s][e];
        }
      }
      ss += shfl_xor(ss, 16);
      ss += shfl_xor(ss, 32);
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
        qf[mt][s] = valid ? pack8(o) : zero4();
      }
    }
  }

  // ---- 2. new keys / values of slots L .. last (wave 0), shared via LDS.
  const bool overlap = c1 > L;
  if (overlap) {
    if (wave == 0) {
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
    }
    __syncthreads();
  }

  // ---- 3. flash-decode over this wave's blocks.
  f32x4_t acc[MTQ][DT];
  float m_run[MTQ], l_run[MTQ];
  int lim[MTQ];  // highest slot each row may see
#pragma unroll
  for (int mt = 0; mt < MTQ; ++mt) {
    m_run[mt] = NEG_INF;
    l_run[mt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[mt][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const int r = mt * 16 + col;
    lim[mt] = (r < R) ? L + r / G : -1;
  }

  for (int j = wave; j < nb; j += NW) {
    const int s0 = c0 + 32 * j;
    if constexpr (DB) {
      cur = nxt;
      if (j + NW < nb) load_block(s0 + 32 * NW, nxt);  // keep the next block in flight
    } else {
      if (j == wave) cur = nxt;
      else load_block(s0, cur);
    }
    if (s0 + 32 > L) {  // block touches new or unwritten slots
      const int slot_a = s0 + 8 * (col >> 2) + (col & 3);
      const int slot_b = slot_a + 4;
#pragma unroll
      for (int s = 0; s < DS; ++s) {
        if (slot_a >= L)
          cur.ka[s] = (slot_a <= last)
                          ? *reinterpret_cast<const uint4 *>(s_kn + (slot_a - L) * D + s * 32 + grp * 8)
                          : zero4();
        if (slot_b >= L)
          cur.kb[s] = (slot_b <= last)
                          ? *reinterpret_cast<const uint4 *>(s_kn + (slot_b - L) * D + s * 32 + grp * 8)
                          : zero4();
      }
      const int vs0 = s0 + 8 * grp;  // first slot of this lane's V group
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        uint16_t e16[8];
        *reinterpret_cast<uint4 *>(e16) = cur.vf[dt];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int slot = vs0 + e;
          if (slot > last)
            e16[e] = 0;
          else if (slot >= L)
            e16[e] = s_vn[(slot - L) * D + dt * 16 + col];
        }
        cur.vf[dt] = *reinterpret_cast<const uint4 *>(e16);
      }
    }
#pragma unroll
    for (int mt = 0; mt < MTQ; ++mt) {
      f32x4_t sa = f32x4_t{0.f, 0.f, 0.f, 0.f}, sb = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < DS; ++s) {
        sa = mfma16x16x32(cur.ka[s], qf[mt][s], sa);
        sb = mfma16x16x32(cur.kb[s], qf[mt][s], sb);
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
        acc[mt][dt] = mfma16x16x32(cur.vf[dt], pf, acc[mt][dt]);
      }
    }
  }

  // ---- 4. merge the waves (wave order), then output or chunk partials.
  uint16_t *out = reinterpret_cast<uint16_t *>(p.out);
  const size_t cstride = (size_t)R * (D + 2);  // floats per chunk partial: acc [R][D], m [R], l [R]
  float *part_b = p.partial + ((size_t)b * nkv + kvh) * p.nchunks * cstride;
  float *part = part_b + (size_t)c * cstride;
#pragma unroll
  for (int mt = 0; mt < MTQ; ++mt) {
    const int r = mt * 16 + col;
    float lw = l_run[mt] + shfl_xor(l_run[mt], 16);
    lw += shfl_xor(lw, 32);  // this wave's row sum
    __syncthreads();
    if (grp == 0) s_m[wave][col] = m_run[mt];
    __syncthreads();
    float M = NEG_INF;
    for (int w2 = 0; w2 < NW; ++w2) M = fmaxf(M, s_m[w2][col]);
    const float scale = (m_run[mt] == NEG_INF) ? 0.f : exp2f(m_run[mt] - M);
    if (grp == 0) s_l[wave][col] = lw * scale;
    float Lrow = 0.f;
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int dd = 0; dd < DTH; ++dd) s_acc[wave][dd][lane] = acc[mt][h * DTH + dd] * scale;
      __syncthreads();
      if (h == 0) {
        for (int w2 = 0; w2 < NW; ++w2) Lrow += s_l[w2][col];
      }
      // wave w reduces output tiles dd = w, w + NW, ... of this half
      for (int dd = wave; dd < DTH; dd += NW) {
        f32x4_t tot = s_acc[0][dd][lane];
        for (int w2 = 1; w2 < NW; ++w2) tot += s_acc[w2][dd][lane];
        const int dt = h * DTH + dd;
        if (r < R) {
          if (n_active == 1) {
            const int t = r / G, hq = r % G;
            uint16_t *dst = out + (size_t)(b * T + t) * nq * D + (size_t)(kvh * G + hq) * D;
            uint2 o;
            o.x = pack2(tot[0] / Lrow, tot[1] / Lrow);
            o.y = pack2(tot[2] / Lrow, tot[3] / Lrow);
            *reinterpret_cast<uint2 *>(dst + dt * 16 + grp * 4) = o;
          } else {
            store_coherent4(part + (size_t)r * D + dt * 16 + grp * 4, tot);
          }
        }
      }
      __syncthreads();
    }
    if (n_active > 1 && wave == 0 && grp == 0 && r < R) {
      store_coherent(part + (size_t)R * D + r, M);
      store_coherent(part + (size_t)R * D + R + r, Lrow);
    }
  }
  if (n_active == 1) return;
  if (!arrive_last(p.counters + (size_t)b * nkv + kvh, (uint32_t)n_active, &s_flag)) return;

  // Merge chunks 0..n_active-1 in order (chunks a row cannot see have
  // m = -inf and are skipped).  Wave w merges output tiles w, w+NW, ...
  constexpr int MB = 4;
#pragma unroll
  for (int mt = 0; mt < MTQ; ++mt) {
    const int r = mt * 16 + col;
    if (r >= R) continue;
    float mmax = NEG_INF;
    for (int cc = 0; cc < n_active; cc += 8) {
      float mv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int ch = min(cc + j, n_active - 1);
        mv[j] = load_coherent(part_b + (size_t)ch * cstride + (size_t)R * D + r);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (cc + j < n_active) mmax = fmaxf(mmax, mv[j]);
    }
    for (int dt = wave; dt < DT; dt += NW) {
      float lsum = 0.f;
      f32x4_t o = f32x4_t{0.f, 0.f, 0.f, 0.f};
      for (int cc = 0; cc < n_active; cc += MB) {
        float mc[MB], lc[MB];
        f32x4_t av[MB];
#pragma unroll
        for (int j = 0; j < MB; ++j) {
          const int ch = min(cc + j, n_active - 1);
          const float *pr = part_b + (size_t)ch * cstride;
          mc[j] = load_coherent(pr + (size_t)R * D + r);
          lc[j] = load_coherent(pr + (size_t)R * D + R + r);
          av[j] = load_coherent4(pr + (size_t)r * D + dt * 16 + grp * 4);
        }
#pragma unroll
        for (int j = 0; j < MB; ++j) {
          if (cc + j >= n_active || mc[j] == NEG_INF) continue;
          const float w = exp2f(mc[j] - mmax);
          lsum += lc[j] * w;
#pragma unroll
          for (int i = 0; i < 4; ++i) o[i] += av[j][i] * w;
        }
      }
      const int t = r / G, hq = r % G;
      uint16_t *dst = out + (size_t)(b * T + t) * nq * D + (size_t)(kvh * G + hq) * D;
      uint2 ov;
      ov.x = pack2(o[0] / lsum, o[1] / lsum);
      ov.y = pack2(o[2] / lsum, o[3] / lsum);
      *reinterpret_cast<uint2 *>(dst + dt * 16 + grp * 4) = ov;
    }
  }
}

}  // namespace

hipError_t launch_attn(const AttnParams &p, hipStream_t s) {
  const int R = p.t_rows * (p.nq / p.nkv);
  const int mtq = (R + 15) / 16;
  dim3 grid(p.nchunks, p.nkv, p.batch);
  dim3 block(64 * p.waves);
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
