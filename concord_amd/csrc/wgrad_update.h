// wgrad_update.h -- the packed update carried by the WGRAD launch of the
// backward entry (concord_dgrad_wgrad_update): the finalize of
// vhat_finalize_kernel and the element of apply_adamw_fast_kernel, run by the
// workgroups of that launch after their tiles instead of by two more launches.
//
//   phase 1  WGRAD workgroups: the tile product, its v-hat partials and bias
//            partials (stored coherently: agent-scope atomic stores); the
//            other workgroups: the dgrad's split-K reduction.
//   barrier 1
//   phase 2  the finalize, spread over the grid (upd_finalize).
//   barrier 2
//   phase 3  each WGRAD workgroup updates the packed words of its tile from the
//            accumulators it still holds (upd_apply); no bf16 weight gradient
//            is written unless the caller asks for a copy.
//   exit     the last workgroup out advances the salt and re-arms the counters.
//
// Reference: the v-hat EMA and update of FusedConcordLinearPackedB.backward,
// concord/packed_b.py:1281-1327 (update op order 494-689).
//
// Cross-workgroup data.  Every value one workgroup writes and another reads
// within the launch (v-hat and bias partials, v_row, v_col, the 256-row
// totals, the zeroed watermarks) is stored with a relaxed agent-scope atomic
// store and read with a relaxed agent-scope atomic load, which on gfx950 write
// through and read past the per-XCD L2; each wave waits for its own memory
// operations (s_waitcnt 0) before its workgroup arrives at a barrier, and the
// reads are issued after the barrier's wait returned.  This is the ordering the
// finalize's ticket relies on (vhat.hip), not acquire/release: an agent-scope
// release would write back a whole XCD's L2.
//
// The grid barrier needs every workgroup of the launch resident at once (one
// per CU here; the host checks the occupancy before choosing this launch).
// Its wait is bounded: a workgroup that waits longer than timeout_ticks of the
// constant clock marks the barrier poisoned; every workgroup that then sees
// the mark skips its remaining writes, and the last one out sets *fault for
// the host (concord_wgrad_update_fault).
#pragma once
#include "common.h"
#include "gemm.h"
#include "update_fast.h"

namespace concord {

struct WgradUpd {
  // finalize (vhat_finalize_kernel's sums, in its orders)
  float* v_row;
  float* v_col;
  float* bsum;        // one total per 256-row block
  float* sum_v_inv;
  int32_t* row_max;   // NULL: no watermarks
  int32_t* col_max;
  int32_t* salt;
  uint16_t* grad_bias;   // NULL: no bias
  int64_t nbp;           // bias partial rows (tiles_j)
  float b2, omb2;
  // grid barrier: arrivals, exits (both zero between calls) and the fault flag
  uint32_t* bar;
  uint32_t* exitc;
  uint32_t* fault;
  int64_t timeout_ticks;
  // update (apply_adamw_fast_kernel's arguments)
  int32_t* packed;
  int64_t ld_p;
  const int8_t* row_exp;
  const int8_t* col_exp;
  float* coh_pre;
  int64_t ld_c;
  concord_update_params p;
  concord_device_scalars s;
  uint32_t flags;
};

constexpr uint32_t kGridPoison = 1u << 24;

CONCORD_DEV float coh_load(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
CONCORD_DEV void coh_store(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Grid barrier: thread 0 of every workgroup adds one to *bar and waits until it
// reads at least `target` (the arrivals at this and the earlier barriers).
// Returns true (for the whole workgroup) when the barrier is poisoned.
CONCORD_DEV bool grid_sync(const WgradUpd& u, uint32_t target, int* s_flag) {
  __builtin_amdgcn_s_waitcnt(0);   // this wave's stores are complete
  __syncthreads();
  if (threadIdx.x == 0) {
    __hip_atomic_fetch_add(u.bar, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const long long t0 = wall_clock64();
    int poisoned = 0;
    for (;;) {
      const uint32_t v = __hip_atomic_load(u.bar, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (v >= kGridPoison) {
        poisoned = 1;
        break;
      }
      if (v >= target) break;
      if (wall_clock64() - t0 > u.timeout_ticks) {
        __hip_atomic_fetch_add(u.bar, kGridPoison, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        poisoned = 1;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    *s_flag = poisoned;
  }
  __syncthreads();
  return *s_flag != 0;
}

// The last workgroup out (every workgroup passes here once, after its last
// write) advances the salt for the next step (the finalize's salt + 1,
// concord/packed_b.py:910-911; every update element of this launch used the
// advanced value) and re-arms the counters.  The salt is left alone when the
// barrier was poisoned.
CONCORD_DEV void grid_exit(const WgradUpd& u) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t e = __hip_atomic_fetch_add(u.exitc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (e == gridDim.x - 1) {
      const uint32_t v = __hip_atomic_load(u.bar, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (v >= kGridPoison) coh_store(u.fault, 1u);
      else if (u.salt) u.salt[0] = wadd(u.salt[0], 1);
      coh_store(u.bar, 0u);
      coh_store(u.exitc, 0u);
    }
  }
}

// sum of src[j * stride] for j < count, ascending from 0.0f, coherent loads,
// 32 in flight
CONCORD_DEV float coh_ordered_sum(const float* src, int64_t stride, int64_t count) {
  float s = 0.0f;
  for (int64_t b = 0; b < count; b += 32) {
    const int n = (int)min((int64_t)32, count - b);
    float a[32];
#pragma unroll
    for (int e = 0; e < 32; ++e) a[e] = e < n ? coh_load(src + (b + e) * stride) : 0.0f;
#pragma unroll
    for (int e = 0; e < 32; ++e)
      if (e < n) s = __fadd_rn(s, a[e]);
  }
  return s;
}

// Phase 2, vhat_finalize_kernel spread over the grid (512 threads per
// workgroup): workgroup b < rb = cdiv(N, 256) takes row block b (threads
// 0..255: g^2 row sums over the column-tile partials, the v_row EMA, the
// watermark zeroing and the block's halving-tree total) and the block's bias
// rows (threads 256..511); workgroups rb .. take 512 columns each.  The host
// launches at least rb + cdiv(K, 512) workgroups.
CONCORD_DEV void upd_finalize(const GemmArgs& g, const WgradUpd& u, float* s_part) {
  const int64_t N = g.I, K = g.J;
  const int64_t rb = cdiv(N, 256), nc = cdiv(K, 64), nr = cdiv(N, 64);
  const int t = threadIdx.x;
  const int64_t wg = blockIdx.x;
  if (wg < rb) {
    const int64_t i = wg * 256 + (t & 255);
    if (t < 256) {
      float vn = 0.0f;
      if (i < N) {
        const float s = coh_ordered_sum(g.vh_pr + i, N, nc);
        vn = __fadd_rn(__fmul_rn(coh_load(u.v_row + i), u.b2), __fmul_rn(u.omb2, s));
        coh_store(u.v_row + i, vn);
        if (u.row_max) coh_store(u.row_max + i, 0);
      }
      s_part[t] = vn;
    } else if (u.grad_bias && i < N) {
      const float sb = coh_ordered_sum(g.bpart + i, N, u.nbp);
      u.grad_bias[i] = (uint16_t)(pack_bf16x2(sb, 0.0f) & 0xFFFFu);
    }
    __syncthreads();
    for (int h = 128; h >= 1; h >>= 1) {
      if (t < h) s_part[t] = __fadd_rn(s_part[t], s_part[t + h]);
      __syncthreads();
    }
    if (t == 0) coh_store(u.bsum + wg, s_part[0]);
  } else {
    const int64_t k = (wg - rb) * 512 + t;
    if (k < K) {
      const float s = coh_ordered_sum(g.vh_pc + k, K, nr);
      coh_store(u.v_col + k, __fadd_rn(__fmul_rn(coh_load(u.v_col + k), u.b2), __fmul_rn(u.omb2, s)));
      if (u.col_max) coh_store(u.col_max + k, 0);
    }
  }
}

// value of lane (l - n) mod 16 within each 16-lane row, as an int
template <int n>
CONCORD_DEV int32_t row_ror_i(int32_t v) {
  return __builtin_amdgcn_update_dpp(0, v, 0x120 + n, 0xF, 0xF, false);
}

// Phase 3: the update of one wave's 64 x 64 accumulator tile (rows row0 +
// [0, 64), columns col0 + [0, 64); lane 16 q + p holds rows 16 x + p, columns
// 16 y + 4 q .. + 3) with apply_adamw_fast_kernel's element, uniforms and
// hash positions.  g = the bf16 value the WGRAD epilogue would store.  The
// watermarks: per row over the wave's 4 q lanes, per column over its 16 p
// lanes, then over the workgroup's waves in LDS (s_rmax: 2 x 256 rows,
// s_cmax: 4 x 128 columns) and one atomic max per row and column of the tile.
template <bool RATIO>
CONCORD_DEV void upd_apply(const GemmArgs& g, const WgradUpd& u, f32x4 (&acc)[4][4], int64_t i0, int64_t j0,
                           int wi, int wj, int32_t* s_rmax, int32_t* s_cmax) {
  const int64_t N = g.I, K = g.J;
  const int t = threadIdx.x, lane = t & 63;
  const int p = lane & 15, q = lane >> 4;
  const int64_t row0 = i0 + wi * 64, col0 = j0 + wj * 64;
  // 1 / max(sum v_row, 1e-30): the 256-row totals chained in order
  const int64_t rb = cdiv(N, 256);
  float tot = 0.0f;
  for (int64_t c0 = 0; c0 < rb; c0 += 64) {
    const float v = c0 + lane < rb ? coh_load(u.bsum + c0 + lane) : 0.0f;
    const int cnt = (int)min((int64_t)64, rb - c0);
    for (int j = 0; j < cnt; ++j) tot = __fadd_rn(tot, lane_value(v, j));
  }
  Uniform U;
  U.lr = *u.s.lr;
  U.eps = *u.s.eps;
  U.chase_floor = RATIO ? *u.s.chase_floor : 0.0f;
  U.leak_floor = RATIO ? *u.s.leak_floor : 0.0f;
  U.v_bc = 1.0f;
  U.cons = 1;
  U.consf = 1.0f;
  U.salt = wadd(*u.salt, 1);   // the finalize's advanced salt
  U.svi = __fdiv_rn(1.0f, fmaxf(tot, 1e-30f));
  if (blockIdx.x == 0 && t == 0) *u.sum_v_inv = U.svi;
  const bool track = u.flags & CONCORD_TRACK_REBALANCE;
  const float C = u.p.drift_cancel_C, alpha = u.p.alpha, avf = u.p.alpha_v_fast;
  const float lr_kappa = __fmul_rn(U.lr, u.p.gf_consol);

  float vc[4][4];
  int32_t ce[4][4], cmax[4][4];
#pragma unroll
  for (int y = 0; y < 4; ++y) {
    const int64_t j = col0 + 16 * y + 4 * q;
    const bool ok = j < K;
    const int32_t e4 = ok ? *reinterpret_cast<const int32_t*>(u.col_exp + j) : 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      ce[y][e] = __builtin_amdgcn_sbfe(e4, 8 * e, 8);
      vc[y][e] = ok ? coh_load(u.v_col + j + e) : 0.0f;
      cmax[y][e] = 0;
    }
  }
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    const int64_t i = row0 + 16 * x + p;
    const bool rok = i < N;
    const int32_t te_row = rok ? (int32_t)u.row_exp[i] - u.p.mantissa_bias : 0;
    const float vr = rok ? coh_load(u.v_row + i) : 0.0f;
    const int32_t psr = wshl((int32_t)i, 16) ^ U.salt;
    int32_t rmax = 0;
#pragma unroll
    for (int y = 0; y < 4; ++y) {
      const int64_t j = col0 + 16 * y + 4 * q;
      if (!rok || j >= K) continue;   // K % 8 == 0: j < K covers all four columns
      int32_t* pp = u.packed + i * u.ld_p + j;
      const int4 wv = *reinterpret_cast<const int4*>(pp);
      const int32_t w[4] = {wv.x, wv.y, wv.z, wv.w};
      float cp[4] = {1.0f, 1.0f, 1.0f, 1.0f};
      float* cpp = RATIO ? nullptr : u.coh_pre + i * u.ld_c + j;
      if (!RATIO) {
        const float4 cv = *reinterpret_cast<const float4*>(cpp);
        cp[0] = cv.x; cp[1] = cv.y; cp[2] = cv.z; cp[3] = cv.w;
      }
      // the epilogue's stored value: bf16(acc * 1 + 0)
      const uint32_t lo = pack_bf16x2(__fadd_rn(acc[x][y][0], 0.0f), __fadd_rn(acc[x][y][1], 0.0f));
      const uint32_t hi = pack_bf16x2(__fadd_rn(acc[x][y][2], 0.0f), __fadd_rn(acc[x][y][3], 0.0f));
      const float gv[4] = {__uint_as_float(lo << 16), __uint_as_float(lo & 0xFFFF0000u),
                           __uint_as_float(hi << 16), __uint_as_float(hi & 0xFFFF0000u)};
      int32_t out[4], m[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int32_t te = te_row + ce[y][e];
        out[e] = adamw_element_fast<RATIO>(w[e], gv[e], exp2i_nc(te), exp2i_nc(-te), vr, vc[y][e], &cp[e],
                                           psr ^ (int32_t)(j + e), C, alpha, avf, lr_kappa, U, &m[e]);
        const int32_t am = abs(m[e]);
        rmax = max(rmax, am);
        cmax[y][e] = max(cmax[y][e], am);
      }
      *reinterpret_cast<int4*>(pp) = make_int4(out[0], out[1], out[2], out[3]);
      if (!RATIO) *reinterpret_cast<float4*>(cpp) = make_float4(cp[0], cp[1], cp[2], cp[3]);
    }
    if (track) {
      rmax = max(rmax, __shfl_xor(rmax, 16, 64));
      rmax = max(rmax, __shfl_xor(rmax, 32, 64));
      if (q == 0) s_rmax[wj * 256 + wi * 64 + 16 * x + p] = rmax;
    }
  }
  if (!track) return;
#pragma unroll
  for (int y = 0; y < 4; ++y)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      int32_t c = cmax[y][e];
      c = max(c, row_ror_i<8>(c));
      c = max(c, row_ror_i<4>(c));
      c = max(c, row_ror_i<2>(c));
      c = max(c, row_ror_i<1>(c));
      if (p == 0) s_cmax[wi * 128 + wj * 64 + 16 * y + 4 * q + e] = c;
    }
  __syncthreads();
  if (t < 256) {
    const int64_t i = i0 + t;
    if (i < N) atomicMax(u.row_max + i, max(s_rmax[t], s_rmax[256 + t]));
  } else if (t < 384) {
    const int c = t - 256;
    const int64_t k = j0 + c;
    if (k < K)
      atomicMax(u.col_max + k, max(max(s_cmax[c], s_cmax[128 + c]), max(s_cmax[256 + c], s_cmax[384 + c])));
  }
}

}  // namespace concord
