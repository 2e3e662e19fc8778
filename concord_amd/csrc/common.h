// common.h -- device helpers shared by the gfx950 kernels of the packed path.
//
// Numerical conventions (identical on every kernel):
//  * binary32 +,-,*,/ and sqrt correctly rounded, no FMA contraction (the
//    library is built with -ffp-contract=off; the __f*_rn intrinsics below
//    make the intent explicit);
//  * float -> int32 by v_cvt_i32_f32: truncate, saturate, NaN -> 0;
//  * int32 arithmetic on the packed fields wraps modulo 2^32;
//  * fp32 -> bf16 rounds to nearest even (v_cvt_pk_bf16_f32).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "concord_amd.h"

#define CONCORD_DEV __device__ __forceinline__

namespace concord {

// ---- error reporting ----------------------------------------------------
void set_error(const char* fmt, ...);
int launch_status(const char* what);

#define CONCORD_CHECK(cond, ...)      \
  do {                                \
    if (!(cond)) {                    \
      ::concord::set_error(__VA_ARGS__); \
      return CONCORD_EINVAL;          \
    }                                 \
  } while (0)

// ---- integer helpers (wrap-around) -----------------------------------------
CONCORD_DEV int32_t wadd(int32_t a, int32_t b) { return (int32_t)((uint32_t)a + (uint32_t)b); }
CONCORD_DEV int32_t wsub(int32_t a, int32_t b) { return (int32_t)((uint32_t)a - (uint32_t)b); }
CONCORD_DEV int32_t wshl(int32_t a, int s) { return (int32_t)((uint32_t)a << s); }
CONCORD_DEV int32_t clampi(int32_t v, int32_t lo, int32_t hi) { return min(max(v, lo), hi); }

// float -> int32 with the hardware's saturating semantics.
CONCORD_DEV int32_t f2i(float f) {
  int32_t r;
  asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(f));
  return r;
}

CONCORD_DEV float bf16_to_f32(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

// two floats -> packed bf16x2 (lo = a), round to nearest even.
CONCORD_DEV uint32_t pack_bf16x2(float a, float b) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  bf2 v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}

// ---- packed word --------------------------------------------------------------
// concord/packed_b.py:143-147 (unpack) and 674-678 (pack)
struct Fields {
  int32_t sf, ss, vs;
};
CONCORD_DEV Fields unpack(int32_t w) {
  Fields f;
  f.sf = w >> 16;
  f.ss = __builtin_amdgcn_sbfe(w, 8, 8);
  f.vs = __builtin_amdgcn_sbfe(w, 0, 8);
  return f;
}
CONCORD_DEV int32_t pack(int32_t sf, int32_t ss, int32_t vs) {
  return (int32_t)(((uint32_t)sf << 16) | (((uint32_t)ss & 0xFFu) << 8) | ((uint32_t)vs & 0xFFu));
}

// ---- the SR hash: concord/packed_b.py:109-117 ------------------------------------
// u = hash(x ^ pos_salt) in [0, 1), 24 bits
CONCORD_DEV float hash_mix(int32_t h) {
  h = h ^ wshl(h, 13);
  h = h ^ (h >> 17);
  h = h ^ wshl(h, 5);
  h = h ^ (h >> 7);
  return __fmul_rn((float)(h & 0xFFFFFF), 5.9604644775390625e-08f);
}
CONCORD_DEV float hash_uniform(int32_t x, int32_t pos_salt) { return hash_mix(x ^ pos_salt); }
// hash_uniform(x, pos ^ c): the three-way xor is one v_bitop3_b32
CONCORD_DEV float hash_uniform3(int32_t x, int32_t pos, int32_t c) {
  return hash_mix((int32_t)__builtin_amdgcn_bitop3_b32((uint32_t)x, (uint32_t)pos, (uint32_t)c, 0x96));
}

// int(floor(d) + (u < d - floor(d))), concord/packed_b.py:596-598.
// Formed as int(floor(d)) + (u < fr): equal, because u < fr needs fr > 0,
// so d is not an integer, |d| < 2^23 and floor(d) + 1 is exact; otherwise
// both forms convert floor(d) alone (NaN -> 0, +-inf saturate alike).
CONCORD_DEV int32_t sr_tick(float d, float u) {
  const float fl = floorf(d);
  const float fr = __fsub_rn(d, fl);
  return f2i(fl) + (int32_t)(u < fr);
}

// ---- Philox4x32-10 (triton/language/random.py:13-44) ------------------------
CONCORD_DEV void philox4x32_10(uint32_t& c0, uint32_t& c1, uint32_t& c2, uint32_t& c3, uint32_t k0,
                               uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    // one 32 x 32 -> 64-bit multiply gives both halves (v_mad_u64_u32)
    const uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
    const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    const uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    c0 = hi1 ^ c1 ^ k0;
    c1 = lo1;
    c2 = hi0 ^ c3 ^ k1;
    c3 = lo0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
}

// tl.rand (triton/language/random.py:127-157): counter (offset, 0, 0, 0),
// key = the sign-extended seed, word 0 mapped to [0, 1)
CONCORD_DEV float tl_rand(int32_t seed, int32_t offset) {
  uint32_t c0 = (uint32_t)offset, c1 = 0, c2 = 0, c3 = 0;
  philox4x32_10(c0, c1, c2, c3, (uint32_t)seed, (uint32_t)(seed >> 31));
  int32_t x = (int32_t)c0;
  if (x < 0) x = wsub(-1, x);
  return __fmul_rn((float)x, 4.6566127342e-10f);
}

// ---- deterministic (x)^p for p outside {0, 0.5}; same op sequence as
// oracle_pow_p (atanh-series log2, Taylor exp2) --------------------------------
CONCORD_DEV float det_log2(float x) {
  uint32_t u = __float_as_uint(x);
  int32_t e = 0;
  if ((u & 0x7F800000u) == 0) {
    x = __fmul_rn(x, 8388608.0f);
    u = __float_as_uint(x);
    e = -23;
  }
  e += (int32_t)((u >> 23) & 0xFF) - 127;
  float m = __uint_as_float((u & 0x007FFFFFu) | 0x3F800000u);
  if (m > 1.41421356f) {
    m = __fmul_rn(m, 0.5f);
    e += 1;
  }
  const float t = __fdiv_rn(__fsub_rn(m, 1.0f), __fadd_rn(m, 1.0f));
  const float t2 = __fmul_rn(t, t);
  float s = 1.0f / 11.0f;
  s = __fadd_rn(__fmul_rn(s, t2), 1.0f / 9.0f);
  s = __fadd_rn(__fmul_rn(s, t2), 1.0f / 7.0f);
  s = __fadd_rn(__fmul_rn(s, t2), 1.0f / 5.0f);
  s = __fadd_rn(__fmul_rn(s, t2), 1.0f / 3.0f);
  s = __fadd_rn(__fmul_rn(s, t2), 1.0f);
  const float ln_m = __fmul_rn(__fmul_rn(2.0f, t), s);
  return __fadd_rn((float)e, __fmul_rn(ln_m, 1.44269504f));
}

CONCORD_DEV float exp2i(int32_t e) {
  e = min(max(e, -300), 300);
  return ldexpf(1.0f, e);
}
// exp2i for |e| <= 300, where its clamp does not bind
CONCORD_DEV float exp2i_nc(int32_t e) { return ldexpf(1.0f, e); }

CONCORD_DEV float det_exp2(float y) {
  if (y != y) return y;
  if (y >= 128.0f) return __builtin_inff();
  if (y < -150.0f) return 0.0f;
  const float n = floorf(__fadd_rn(y, 0.5f));
  const float f = __fsub_rn(y, n);
  const float z = __fmul_rn(f, 0.693147181f);
  float p = 1.0f / 40320.0f;
  p = __fadd_rn(__fmul_rn(p, z), 1.0f / 5040.0f);
  p = __fadd_rn(__fmul_rn(p, z), 1.0f / 720.0f);
  p = __fadd_rn(__fmul_rn(p, z), 1.0f / 120.0f);
  p = __fadd_rn(__fmul_rn(p, z), 1.0f / 24.0f);
  p = __fadd_rn(__fmul_rn(p, z), 1.0f / 6.0f);
  p = __fadd_rn(__fmul_rn(p, z), 0.5f);
  p = __fadd_rn(__fmul_rn(p, z), 1.0f);
  p = __fadd_rn(__fmul_rn(p, z), 1.0f);
  const int32_t ni = (int32_t)n;
  const int32_t a = ni / 2, b = ni - a;
  return __fmul_rn(__fmul_rn(p, exp2i(a)), exp2i(b));
}

// correctly rounded sqrt.  __builtin_sqrtf expands to v_sqrt_f32 plus the
// +-1 ulp fma correction, wrapped in a 2^32 pre-scale for x < 2^-96 and a
// class test that returns x itself for +-0 and +inf.  For x >= 2^-96
// (and +inf, where the corrections leave v_sqrt's inf) the scale and the
// class test change nothing, so only the correction runs; a wave with any
// lane below 2^-96, zero, negative or NaN takes the full expansion.
CONCORD_DEV float sqrt_rn(float x) {
  float s = __builtin_amdgcn_sqrtf(x);
  const float sdn = __int_as_float(__float_as_int(s) - 1);
  const float sup = __int_as_float(__float_as_int(s) + 1);
  const float rdn = __builtin_fmaf(-sdn, s, x);
  const float rup = __builtin_fmaf(-sup, s, x);
  s = rdn <= 0.0f ? sdn : s;
  s = rup > 0.0f ? sup : s;
  if (__builtin_amdgcn_ballot_w64(!(x >= 0x1p-96f))) {
    float y = x;
    asm volatile("" : "+v"(y));   // keep the full expansion behind the branch
    const float full = __builtin_sqrtf(y);
    s = x >= 0x1p-96f ? s : full;
  }
  return s;
}

// cos(2 pi u) and sin(2 pi u) for u in [0, 1) on a 2^-24 grid: quadrant
// q = floor(4u) and theta = (4u - q) pi/2 are exact up to the one product;
// cos and sin of theta by Taylor polynomials in theta^2 (degree 10 and 11;
// |error| below 1e-6 on [0, pi/2]), evaluated in a fixed order, then rotated
// by q quarter turns
CONCORD_DEV void det_sincos2pi(float u, float& cs, float& sn2) {
  const float t = __fmul_rn(u, 4.0f);
  const float qf = floorf(t);
  const int q = (int)qf;
  const float th = __fmul_rn(__fsub_rn(t, qf), 1.57079632679489662f);
  const float s = __fmul_rn(th, th);
  float c = -1.0f / 3628800.0f;
  c = __fadd_rn(__fmul_rn(c, s), 1.0f / 40320.0f);
  c = __fadd_rn(__fmul_rn(c, s), -1.0f / 720.0f);
  c = __fadd_rn(__fmul_rn(c, s), 1.0f / 24.0f);
  c = __fadd_rn(__fmul_rn(c, s), -0.5f);
  c = __fadd_rn(__fmul_rn(c, s), 1.0f);
  float sn = -1.0f / 39916800.0f;
  sn = __fadd_rn(__fmul_rn(sn, s), 1.0f / 362880.0f);
  sn = __fadd_rn(__fmul_rn(sn, s), -1.0f / 5040.0f);
  sn = __fadd_rn(__fmul_rn(sn, s), 1.0f / 120.0f);
  sn = __fadd_rn(__fmul_rn(sn, s), -1.0f / 6.0f);
  sn = __fadd_rn(__fmul_rn(sn, s), 1.0f);
  sn = __fmul_rn(sn, th);
  cs = q == 0 ? c : q == 1 ? -sn : q == 2 ? -c : sn;
  sn2 = q == 0 ? sn : q == 1 ? c : q == 2 ? -sn : -c;
}

CONCORD_DEV float det_cos2pi(float u) {
  float c, s;
  det_sincos2pi(u, c, s);
  return c;
}

// Box-Muller radius sqrt(-2 ln u1) of a Philox word w, u1 = ((w >> 8) + 1)
// 2^-24 in (0, 1], ln u1 = log2(u1) ln 2; and the angle's u2 = (w >> 8) 2^-24
CONCORD_DEV float bm_radius(uint32_t w) {
  const float u1 = __fmul_rn((float)((w >> 8) + 1u), 5.9604644775390625e-08f);
  return sqrt_rn(__fmul_rn(-2.0f, __fmul_rn(det_log2(u1), 0.693147180559945309f)));
}
CONCORD_DEV float bm_angle(uint32_t w) { return __fmul_rn((float)(w >> 8), 5.9604644775390625e-08f); }

// Standard normal draw `idx` of stream (seed, tag): Box-Muller on one
// Philox4x32-10 block, counter (idx, 0, 0, 0), key (seed, tag); the per-token
// draw of the Sigma_g noise uses tag 0x5369676D:
//   z = sqrt(-2 ln u1) cos(2 pi u2), u1 from word 0, u2 from word 1.
// A fixed sequence of IEEE ops (det_log2, sqrt_rn, det_cos2pi), so the CPU
// restatement draws the same bits.
constexpr uint32_t kNoiseTagIso = 0x6E6F6973u, kNoiseTagToken = 0x5369676Du;
CONCORD_DEV float normal_draw(int32_t seed, uint32_t idx, uint32_t tag) {
  uint32_t c0 = idx, c1 = 0, c2 = 0, c3 = 0;
  philox4x32_10(c0, c1, c2, c3, (uint32_t)seed, tag);
  return __fmul_rn(bm_radius(c0), det_cos2pi(bm_angle(c1)));
}

// The isotropic stream (tag 0x6E6F6973): four draws per Philox block, counter
// (blk, 0, 0, 0).  Words 0, 1 and words 2, 3 are two Box-Muller pairs, and
// each pair gives both its cos and its sin draw:
//   z[0] = r0 cos(2 pi a1), z[1] = r0 sin(2 pi a1),
//   z[2] = r2 cos(2 pi a3), z[3] = r2 sin(2 pi a3)
// (r_i = bm_radius(word i), a_i = bm_angle(word i)).  Element e of a gradient
// takes z[e & 3] of block e >> 2; z[0] equals normal_draw(seed, blk, tag).
CONCORD_DEV void normal_draw4(int32_t seed, uint32_t blk, float z[4]) {
  uint32_t c0 = blk, c1 = 0, c2 = 0, c3 = 0;
  philox4x32_10(c0, c1, c2, c3, (uint32_t)seed, kNoiseTagIso);
  const float r0 = bm_radius(c0), r2 = bm_radius(c2);
  float ca, sa, cb, sb;
  det_sincos2pi(bm_angle(c1), ca, sa);
  det_sincos2pi(bm_angle(c3), cb, sb);
  z[0] = __fmul_rn(r0, ca);
  z[1] = __fmul_rn(r0, sa);
  z[2] = __fmul_rn(r2, cb);
  z[3] = __fmul_rn(r2, sb);
}

CONCORD_DEV float pow_p(float x, float p) {
  if (p == 0.5f) return sqrt_rn(x);
  if (p == 0.0f) return 1.0f;
  return det_exp2(__fmul_rn(p, det_log2(x)));
}

// ---- reductions ------------------------------------------------------------------
// lane j's value, j wave-uniform (a scalar read; a shuffle would take an LDS
// round trip)
CONCORD_DEV float lane_value(float v, int j) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), j));
}

// Sum of the `count` terms v[i * stride] as 64 lane sums and a tree: lane l
// adds v[l], v[l + 64], ... in index order from 0.0f (a round of 16 terms
// per lane in flight at once), then the halving tree over the 64 lane sums
// (for h = 32 .. 1, lane l < h adds lane l + h's sum).  The result goes to
// every lane; called by all 64 lanes of a wave.
CONCORD_DEV float wave_tree_sum(const float* __restrict__ v, int64_t count, int64_t stride) {
  constexpr int B = 16;
  const int lane = threadIdx.x & 63;
  float s = 0.0f;
  for (int64_t c0 = 0; c0 < count; c0 += 64 * B) {
    float a[B];
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const int64_t i = c0 + 64 * b + lane;
      a[b] = i < count ? v[i * stride] : 0.0f;
    }
#pragma unroll
    for (int b = 0; b < B; ++b)
      if (c0 + 64 * b + lane < count) s = __fadd_rn(s, a[b]);
  }
#pragma unroll
  for (int h = 32; h >= 1; h >>= 1) s = __fadd_rn(s, __shfl_down(s, h, 64));
  return lane_value(s, 0);
}

// wave_tree_sum of the interleaved pairs: *s0 over v[0], v[2], ...; *s1 over
// v[1], v[3], ... (`count` pairs), each in the same order.
CONCORD_DEV void wave_tree_sum2(const float* __restrict__ v, int64_t count, float* s0, float* s1) {
  constexpr int B = 8;
  const int lane = threadIdx.x & 63;
  float x0 = 0.0f, x1 = 0.0f;
  for (int64_t c0 = 0; c0 < count; c0 += 64 * B) {
    float a[B], b[B];
#pragma unroll
    for (int q = 0; q < B; ++q) {
      const int64_t i = c0 + 64 * q + lane;
      a[q] = i < count ? v[2 * i] : 0.0f;
      b[q] = i < count ? v[2 * i + 1] : 0.0f;
    }
#pragma unroll
    for (int q = 0; q < B; ++q)
      if (c0 + 64 * q + lane < count) {
        x0 = __fadd_rn(x0, a[q]);
        x1 = __fadd_rn(x1, b[q]);
      }
  }
#pragma unroll
  for (int h = 32; h >= 1; h >>= 1) {
    x0 = __fadd_rn(x0, __shfl_down(x0, h, 64));
    x1 = __fadd_rn(x1, __shfl_down(x1, h, 64));
  }
  *s0 = lane_value(x0, 0);
  *s1 = lane_value(x1, 0);
}

// max over the wave's 64 lanes of NON-NEGATIVE values, as a wave-uniform
// value.  DPP steps: prefix maxima within each 16-lane row (row_shr 1, 2, 4,
// 8), so lane 15 of row r holds the row's maximum M_r; then row_bcast:15
// (lane 15 of each row into the next row: lane 63 = max(M_3, M_2), lane 31 =
// max(M_1, M_0)) and row_bcast:31 (lane 31 into rows 2 and 3): lane 63 then
// holds max(M_0 .. M_3).  A lane with no source reads 0 (bound_ctrl, old =
// 0), which leaves a non-negative maximum unchanged, and every step writes
// all rows (the other lanes' results are not used), so each step is one
// v_max_i32 with a DPP operand; an old value of v, or partial row masks, would
// need a copy and a separate DPP move per step.  A shuffle butterfly would
// cost an LDS round trip per step.
CONCORD_DEV int32_t wave_max(int32_t v) {
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true));
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true));
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true));
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, true));
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x142, 0xF, 0xF, true));
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x143, 0xF, 0xF, true));
  return __builtin_amdgcn_readlane(v, 63);
}

__host__ __device__ inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Every launch of this library keeps grid.y and grid.z at or below
// kMaxGridY.  A kernel whose row-block count can exceed it is launched with
// grid.y = grid_y(count) and strides over the row blocks by gridDim.y; the
// entry points of the others reject sizes whose grid would exceed it.
constexpr int64_t kMaxGridY = 65535;
inline unsigned grid_y(int64_t blocks) { return (unsigned)(blocks < kMaxGridY ? blocks : kMaxGridY); }

}  // namespace concord
