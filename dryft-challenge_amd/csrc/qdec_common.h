// Shared device helpers of the qdec kernels (gfx950 / CDNA4 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qdec.h"

namespace qdec {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kTileN = 16;   // tile rows of a weight block (output columns)
constexpr int kTileK = 32;   // k per MFMA step
constexpr int kBlockElems = kTileN * kTileK;  // 512 bf16 = 1 KiB

// ---------------------------------------------------------------- bf16 math
// float -> bf16 with round-to-nearest-even, the rounding torch's
// .to(bfloat16) performs, in one gfx950 instruction (v_cvt_pk_bf16_f32, two
// values at a time).  NaN stays NaN (torch writes the canonical 0x7fc0; no
// NaN reaches a comparison in this library).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}
__device__ __forceinline__ uint32_t f2bf(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __forceinline__ float bf2f(uint32_t b) { return __uint_as_float(b << 16); }
// Value of f after a round trip through bf16.
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

// The 8 bf16 of a 16-byte vector.
__device__ __forceinline__ float lo16(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi16(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ void unpack8(const uint4 &v, float f[8]) {
  f[0] = lo16(v.x); f[1] = hi16(v.x);
  f[2] = lo16(v.y); f[3] = hi16(v.y);
  f[4] = lo16(v.z); f[5] = hi16(v.z);
  f[6] = lo16(v.w); f[7] = hi16(v.w);
}
__device__ __forceinline__ uint4 pack8(const float f[8]) {
  uint4 v;
  v.x = pack2(f[0], f[1]);
  v.y = pack2(f[2], f[3]);
  v.z = pack2(f[4], f[5]);
  v.w = pack2(f[6], f[7]);
  return v;
}

// D = A(16x32) * B(32x16) + C; lane l supplies A row / B column (l & 15),
// k = 8*(l >> 4) .. +8; the result lane l holds rows 4*(l >> 4) + i, column
// (l & 15), i = 0..3.
__device__ __forceinline__ f32x4_t mfma16x16x32(const uint4 &a, const uint4 &b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ uint4 zero4() { return make_uint4(0u, 0u, 0u, 0u); }

// x' = norm_w * bf16(x * rstd) of 8 consecutive elements (one 16-byte
// vector), rounded to bf16 on packing.
__device__ __forceinline__ uint4 norm8(const uint4 &xv, const uint4 &nv, float rs) {
  float f[8], g[8];
  unpack8(xv, f);
  unpack8(nv, g);
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = g[e] * rbf(f[e] * rs);
  return pack8(f);
}

// Activations in MFMA fragment order: element (m, k) of a [rows, K] matrix
// with nmt = ceil(rows / 16) M tiles lives in the 1 KiB block of (k step
// k/32, M tile m/16), lane (m % 16) + 16 * ((k % 32) / 8), element k % 8 --
// exactly the B fragment a lane of a 16x16x32 MFMA loads, so one fragment
// load is one contiguous KiB.  4 consecutive k from a multiple of 4 stay
// contiguous.
__device__ __forceinline__ size_t frag_off(int m, int k, int nmt) {
  return (((size_t)(k >> 5) * nmt + (m >> 4)) * 64 + (m & 15) + 16 * ((k >> 3) & 3)) * 8 + (k & 7);
}

// 16-byte load with the non-temporal hint, for data read once per step
// (weights, cached keys and values).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_nt(const void *p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Workgroup barrier for an LDS hand-over: waits for this wave's LDS
// operations only (lgkmcnt 0), not for its outstanding global loads, which
// the workgroup-scope release fence of __syncthreads() also drains.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Global loads that bypass caches which another XCD may hold stale, for data
// written by other workgroups of the same grid (split partials).
__device__ __forceinline__ float load_coherent(const float *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_coherent(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Device-scope 64-bit relaxed atomics compile to plain global_load/store_dwordx2
// with the device-scope cache policy, so they pipeline like ordinary loads.
__device__ __forceinline__ uint64_t ld64_dev(const void *p) {
  return __hip_atomic_load(reinterpret_cast<const uint64_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st64_dev(void *p, uint64_t v) {
  __hip_atomic_store(reinterpret_cast<uint64_t *>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 16-byte fp32 partials handed between workgroups (device scope).
__device__ __forceinline__ f32x4_t load_coherent4(const float *p) {
  const uint64_t a = ld64_dev(p), b = ld64_dev(p + 2);
  return f32x4_t{__uint_as_float((uint32_t)a), __uint_as_float((uint32_t)(a >> 32)), __uint_as_float((uint32_t)b),
                 __uint_as_float((uint32_t)(b >> 32))};
}
__device__ __forceinline__ void store_coherent4(float *p, f32x4_t v) {
  st64_dev(p, (uint64_t)__float_as_uint(v[0]) | ((uint64_t)__float_as_uint(v[1]) << 32));
  st64_dev(p + 2, (uint64_t)__float_as_uint(v[2]) | ((uint64_t)__float_as_uint(v[3]) << 32));
}
// Activation accesses of a kernel body, plain or (COH) at device scope: COH
// is for a body that runs inside a launch whose other workgroups wrote the
// data or will read it (the one-launch-per-layer kernel); per-operation
// launches hand their data over at the launch boundary and use plain ones.
template <bool COH>
__device__ __forceinline__ uint4 ldv16(const void *p) {
  if constexpr (COH) {
    const uint64_t a = ld64_dev(p), b = ld64_dev(static_cast<const char *>(p) + 8);
    return make_uint4((uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32));
  } else {
    return *reinterpret_cast<const uint4 *>(p);
  }
}
template <bool COH>
__device__ __forceinline__ uint2 ldv8(const void *p) {
  if constexpr (COH) {
    const uint64_t a = ld64_dev(p);
    return make_uint2((uint32_t)a, (uint32_t)(a >> 32));
  } else {
    return *reinterpret_cast<const uint2 *>(p);
  }
}
template <bool COH>
__device__ __forceinline__ void stv8(void *p, uint2 v) {
  if constexpr (COH)
    st64_dev(p, (uint64_t)v.x | ((uint64_t)v.y << 32));
  else
    *reinterpret_cast<uint2 *>(p) = v;
}
template <bool COH>
__device__ __forceinline__ uint32_t ldv4(const void *p) {
  if constexpr (COH)
    return __hip_atomic_load(reinterpret_cast<const uint32_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else
    return *reinterpret_cast<const uint32_t *>(p);
}

__device__ __forceinline__ int load_coherent_i(const int *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_coherent_i(int *p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Arrival at a per-tile counter after this workgroup's partial results were
// stored (all threads must call it).  Returns true in every thread of the
// workgroup that arrived last; that workgroup resets the counter to zero.
//
// Protocol (no cache-wide fences): every value handed between workgroups is
// written with store_coherent and read with load_coherent, i.e. device-scope
// accesses that are performed at the device's point of coherence and never
// served from a stale cache line of another XCD.  Ordering is then only a
// matter of completion: each thread waits for its own stores to complete
// (s_waitcnt 0) before the workgroup barrier, and thread 0 bumps the counter
// after the barrier, so the counter can only reach `expected` once every
// partial of every arriving workgroup is visible; the last arriver reads the
// partials after it has seen that value.  A full __threadfence() here would
// write back and invalidate the whole L2 of the XCD for every workgroup.
__device__ __forceinline__ bool arrive_last(uint32_t *counter, uint32_t expected,
                                            uint32_t *lds_flag) {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t old = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t last = (old == expected - 1u) ? 1u : 0u;
    if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *lds_flag = last;
  }
  __syncthreads();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  return *lds_flag != 0u;
}

// Argmax as an unsigned maximum: the high word orders fp32 values (non-NaN;
// -0 counts as +0), the low word is the complement of the index, so equal
// values keep the lowest index.  A row whose every value is -inf or NaN
// keeps its initial (-inf, 0x7fffffff) and decodes to that index.
__device__ __forceinline__ uint64_t argmax_key(float v, int idx) {
  uint32_t b = __float_as_uint(v == 0.f ? 0.f : v);
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((uint64_t)b << 32) | (uint64_t)(0xffffffffu - (uint32_t)idx);
}
__device__ __forceinline__ int argmax_index(uint64_t key) { return (int)(0xffffffffu - (uint32_t)key); }

// Cross-lane helpers (wave64).
__device__ __forceinline__ float shfl_xor(float v, int m) { return __shfl_xor(v, m, kWave); }

template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, 0xf, 0xf, true);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, 0xf, 0xf, true);
  return ((uint64_t)hi << 32) | lo;
}
// Maximum over each 16-lane row of the wave (all lanes active), in every
// lane of the row.
__device__ __forceinline__ uint64_t row16_max(uint64_t v) {
  uint64_t o = dpp_u64<0xB1>(v);   // quad_perm [1,0,3,2]
  v = o > v ? o : v;
  o = dpp_u64<0x4E>(v);            // quad_perm [2,3,0,1]
  v = o > v ? o : v;
  o = dpp_u64<0x141>(v);           // row_half_mirror
  v = o > v ? o : v;
  o = dpp_u64<0x140>(v);           // row_mirror
  return o > v ? o : v;
}

// v of the lane chosen by DPP control CTRL (every lane active).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
}
__device__ __forceinline__ float lane_f(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// Sum over the 64 lanes of a wave (all active), the same bits in every lane,
// without a round trip through the LDS crossbar: partners lane^1 and lane^2
// (quad permutations), then the lane mirrored within 8 and within 16 --
// after the quad steps every quad holds its quad sum, so the mirrored lane
// holds the lane^4 (then lane^8) partner's value -- then the four 16-lane row
// sums as (r0 + r1) + (r2 + r3).  The pairing of a full xor butterfly.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);  // row_half_mirror
  v += dpp_f<0x140>(v);  // row_mirror
  return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}

// Per-head RMSNorm (weight w) and RoPE of one D-channel head row spread
// over a wavefront: lane l < D/2 holds channels 2l and 2l+1 (raw, w, cos cw
// and sin sw as packed bf16 pairs; the lanes past D/2 pass raw = 0 and their
// result is not used); channel i pairs with i +- D/2, held by lane ^ D/4.
// rotate_half(y) = [-y[D/2:], y[:D/2]].  Returns the two rotated channels as
// packed bf16:
//   y = bf16(w * bf16(x * rstd)),  out = bf16(bf16(y * cos) + bf16(rot * sin)).
template <int D>
__device__ __forceinline__ uint32_t head_norm_rope(uint32_t raw, uint32_t w, uint32_t cw, uint32_t sw, float eps) {
  static_assert(D == 128 || D == 64, "head_dim 128 or 64");
  const int lane = threadIdx.x & 63;
  const float x0 = lo16(raw), x1 = hi16(raw);
  const float ss = wave_sum(x0 * x0 + x1 * x1);
  const float rstd = 1.0f / sqrtf(ss / (float)D + eps);
  const float y0 = rbf(lo16(w) * rbf(x0 * rstd));
  const float y1 = rbf(hi16(w) * rbf(x1 * rstd));
  const float p0 = shfl_xor(y0, D / 4), p1 = shfl_xor(y1, D / 4);
  const bool first_half = (lane & (D / 2 - 1)) < D / 4;
  const float r0 = first_half ? -p0 : p0;
  const float r1 = first_half ? -p1 : p1;
  const float o0 = rbf(y0 * lo16(cw)) + rbf(r0 * lo16(sw));
  const float o1 = rbf(y1 * hi16(cw)) + rbf(r1 * hi16(sw));
  return pack2(o0, o1);
}
__device__ __forceinline__ uint32_t head_norm_rope2(uint32_t raw, uint32_t w, uint32_t cw, uint32_t sw, float eps) {
  return head_norm_rope<128>(raw, w, cw, sw, eps);
}

}  // namespace qdec

// Error plumbing shared by the entry points (api.hip).
namespace qdec {
int set_error(int code, const char *fmt, ...);
int check_launch(const char *what);
}  // namespace qdec
