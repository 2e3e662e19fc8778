// update.hip -- the packed optimizer update on gfx950.
//
// concord_apply_adamw: _apply_packed_adamw_kernel, concord/packed_b.py:422-703
//   (+ prototype extension notebook/src/prototype_packed_b.py:454-778 and the
//   Muon drive of docs/MUON_IMPLEMENTATION.md:87-119).
// concord_apply_sgd:   _apply_packed_sgd_kernel, concord/packed_b.py:173-312.
//
// Layout: a block of 256 threads (4 waves) owns a tile of TN rows x 256
// columns; a lane owns 4 consecutive columns and walks the tile's rows with
// its wave, so every row access of a wave is one contiguous 1 KB (packed) +
// 512 B (bf16 grad) segment.  Row watermarks are reduced across the wave and
// written with one atomic max per row; column watermarks are reduced across
// the 4 waves in LDS and written with one atomic max per column.
#include <cstdint>
#include <type_traits>
#include "common.h"
#include "update_fast.h"

namespace concord {

// v-hat enters the update through the trust-region denominator (not under
// the Muon drive, whose step is the supplied drive) and through the
// non-fixed coherence gate; otherwise v_row / v_col / sum_v_inv are not read
// (docs/MUON_IMPLEMENTATION.md:75-80: the Muon path needs no v-hat).
__host__ __device__ inline bool update_needs_vhat(uint32_t flags) {
  const bool denom = (flags & CONCORD_GF_TRUST_REGION) && !(flags & CONCORD_MUON);
  const bool gate = !(flags & CONCORD_FIXED_COH) &&
                    (flags & (CONCORD_GF_CONSOLIDATION | CONCORD_COHPRE | CONCORD_RATIO_COH));
  return denom || gate;
}

struct AdamwArgs {
  int32_t* packed;
  const uint16_t* grad;
  uint16_t* wbuf;
  const int8_t* row_exp;
  const int8_t* col_exp;
  int32_t* row_max;
  int32_t* col_max;
  const float* v_row;
  const float* v_col;
  const float* sum_v_inv;
  float* coh_pre;
  // fast kernel only: when bsum is set, 1 / sum v_row is formed here from the
  // finalize's 256-row totals (bsum[nbsum], chained in order as the finalize
  // would) instead of read from sum_v_inv, and stored to svi_out
  const float* bsum;
  int64_t nbsum;
  float* svi_out;
  int64_t ld_p, ld_g, ld_w, ld_c;
  int64_t N, K;
  concord_update_params p;
  concord_device_scalars s;
  uint32_t flags;
  int tn;
};


// One element of the update.  Op order = concord/packed_b.py:494-689 (the
// prototype's consf / v_bc / beta1 form when PROTO_CONSF is set).
CONCORD_DEV int32_t adamw_element(int32_t word, float g, int32_t te, float vr, float vc,
                                  float* coh_pre, int n, int k, const concord_update_params& P,
                                  const Uniform& U, uint32_t flags, int32_t* m_out) {
  const bool proto = flags & CONCORD_PROTO_CONSF;
  Fields f = unpack(word);
  int32_t sf = f.sf, ss = f.ss, vs = f.vs;
  const int32_t vsf = vs * 128;
  const float scale_fwd = exp2i(te);
  const float scale_inv = exp2i(-te);
  const float d_fs = (float)sf;
  const float d_sv = (float)wsub(ss * 128, vsf);
  const float noise = __fsub_rn(d_fs, __fmul_rn(P.drift_cancel_C, d_sv));
  const float nw = __fmul_rn(noise, scale_fwd);
  float v_proxy = __fmul_rn(__fmul_rn(nw, nw), P.v_scale);
  float v_hat = 0.0f, coh = 0.0f;
  if (flags & (CONCORD_GF_TRUST_REGION | CONCORD_GF_CONSOLIDATION | CONCORD_COHPRE |
               CONCORD_RATIO_COH)) {
    v_hat = __fmul_rn(__fmul_rn(vr, vc), U.svi);
    if (proto) v_hat = __fmul_rn(v_hat, U.v_bc);
  }
  if (flags & CONCORD_GF_TRUST_REGION)
    v_proxy = __fadd_rn(v_proxy, __fmul_rn(P.gf_trust_delta_sq, v_hat));
  if (flags & (CONCORD_GF_CONSOLIDATION | CONCORD_COHPRE | CONCORD_RATIO_COH)) {
    if (flags & CONCORD_FIXED_COH) {
      const float sig_w = __fmul_rn(__fmul_rn(P.drift_cancel_C, d_sv), scale_fwd);
      const float sig2 = __fmul_rn(sig_w, sig_w);
      coh = __fdiv_rn(sig2, __fadd_rn(__fadd_rn(sig2, __fmul_rn(nw, nw)), 1e-30f));
    } else {
      const float mg = __fmul_rn(__fmul_rn(P.alpha_v_fast, d_sv), scale_fwd);
      coh = __fdiv_rn(__fmul_rn(mg, mg), __fadd_rn(v_hat, 1e-12f));
    }
    coh = fminf(fmaxf(coh, 0.0f), 1.0f);
  }
  float step;
  if (flags & CONCORD_MUON) {
    step = g;
  } else {
    step = __fdiv_rn(g, pow_p(__fadd_rn(v_proxy, U.eps), P.precond_p));
    step = fminf(fmaxf(step, -P.step_cap), P.step_cap);
  }
  float evap;
  if (flags & CONCORD_GF_CONSOLIDATION) {
    evap = __fmul_rn(__fmul_rn(__fmul_rn(U.lr, P.gf_consol), __fsub_rn(1.0f, coh)), d_fs);
  } else {
    step = __fadd_rn(step, __fmul_rn(P.weight_decay, __fmul_rn(d_fs, scale_fwd)));
    evap = 0.0f;
  }
  const float delta_grad = __fmul_rn(__fmul_rn(-U.lr, step), scale_inv);
  float delta_t;
  if (proto)
    delta_t = __fadd_rn(delta_grad,
                        __fmul_rn(U.consf, __fsub_rn(__fmul_rn(__fmul_rn(P.beta1, coh), d_fs), evap)));
  else
    delta_t = __fsub_rn(__fsub_rn(delta_grad, __fmul_rn(P.beta1, d_fs)), evap);

  const int32_t ps = wshl(n, 16) ^ k ^ U.salt;
  sf = wadd(sf, sr_tick(delta_t, hash_uniform(sf, ps)));

  int32_t new_v = vs;
  if (flags & CONCORD_APPLY_CHASE) {
    float gate = 1.0f;
    if (flags & CONCORD_RATIO_COH) {
      gate = __fadd_rn(U.chase_floor, __fmul_rn(__fsub_rn(1.0f, U.chase_floor), coh));
    } else if (flags & CONCORD_COHPRE) {
      const float cp = *coh_pre;
      gate = __fadd_rn(coh, __fmul_rn(cp, __fsub_rn(1.0f, coh)));
      *coh_pre = __fadd_rn(__fmul_rn(__fsub_rn(1.0f, P.alpha_v_fast), cp),
                           __fmul_rn(P.alpha_v_fast, coh));
    }
    float chase = __fmul_rn(__fmul_rn(__fmul_rn(P.alpha, gate), P.gate_gain), (float)sf);
    if (proto) chase = __fmul_rn(chase, U.consf);
    const int32_t t2 = sr_tick(__fmul_rn(chase, 0.0078125f), hash_uniform3(sf, ps, 0x5A5A5A5A));
    ss = wadd(ss, t2);
    sf = wsub(sf, wshl(t2, 7));

    float dv8 = __fmul_rn(__fmul_rn(P.alpha_v_fast, (float)wsub(wshl(ss, 7), vsf)), 0.0078125f);
    if (proto) dv8 = __fmul_rn(dv8, U.consf);
    if (flags & CONCORD_RATIO_COH)
      dv8 = __fmul_rn(dv8, __fadd_rn(U.leak_floor, __fmul_rn(__fsub_rn(1.0f, U.leak_floor), coh)));
    const int32_t t3 = sr_tick(dv8, hash_uniform3(sf, ps, 0x33335555));
    new_v = clampi(wadd(vs, t3), -128, 127);
    if (flags & CONCORD_MASS_PRESERVE) ss = wsub(ss, wsub(new_v, vs));

    if (P.wd_sv != 0.0f || P.wd_sf != 0.0f) {
      const int32_t vpost = new_v * 128;
      float wdsv = __fmul_rn(__fmul_rn(__fmul_rn(U.lr, P.wd_sv), (float)wsub(wshl(ss, 7), vpost)),
                             0.0078125f);
      if (proto) wdsv = __fmul_rn(wdsv, U.consf);
      ss = wsub(ss, sr_tick(wdsv, hash_uniform3(sf, ps, 0x66665555)));
      float wdsf = __fmul_rn(__fmul_rn(U.lr, P.wd_sf), (float)wsub(wadd(wshl(ss, 7), sf), vpost));
      if (proto) wdsf = __fmul_rn(wdsf, U.consf);
      sf = wsub(sf, sr_tick(wdsf, hash_uniform3(sf, ps, 0x77770000)));
    }
  }
  const int32_t sfc = clampi(sf, -32768, 32767);
  const int32_t ssc = clampi(ss, -128, 127);
  *m_out = ssc * 128 + sfc + new_v * 128;
  return pack(sfc, ssc, new_v);
}

// The wd_sv/wd_sf terms are skipped only when both rates are zero: then both
// SR deltas are +-0 and their ticks are exactly 0 (floor(+-0) + (u < 0) = 0).

template <bool RATIO>
__global__ __launch_bounds__(256) void apply_adamw_fast_kernel(AdamwArgs a) {
  __shared__ int32_t s_cmax[4][256];
  // wave in a scalar register: the row walk below is scalar control flow
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t kb = (int64_t)blockIdx.x * 256;
  const int64_t k0 = kb + lane * 4;
  const bool track = a.flags & CONCORD_TRACK_REBALANCE;
  const bool emit = a.flags & CONCORD_EMIT_WEIGHT;
  const float C = a.p.drift_cancel_C, alpha = a.p.alpha, avf = a.p.alpha_v_fast;
  Uniform U;
  float lr_kappa = 0.0f;
  int32_t ce[4], cmax[4];
  float vc[4];
  // the per-block set-up: the scalars, 1 / sum v_row, the lane's column
  // exponents and v_col (issued after the wave's first row loads, so that
  // both round trips overlap)
  auto setup = [&]() {
    U.lr = *a.s.lr;
    U.eps = *a.s.eps;
    U.chase_floor = RATIO ? *a.s.chase_floor : 0.0f;
    U.leak_floor = RATIO ? *a.s.leak_floor : 0.0f;
    U.v_bc = 1.0f;
    U.cons = 1;
    U.consf = 1.0f;
    U.salt = *a.s.salt_counter;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool ok = k0 + j < a.K;
      ce[j] = ok ? (int32_t)a.col_exp[k0 + j] : 0;
      vc[j] = ok ? a.v_col[k0 + j] : 0.0f;
      cmax[j] = 0;
    }
    if (a.bsum) {
      float tot = 0.0f;
      for (int64_t c0 = 0; c0 < a.nbsum; c0 += 64) {
        const float v = c0 + lane < a.nbsum ? a.bsum[c0 + lane] : 0.0f;
        const int cnt = (int)min((int64_t)64, a.nbsum - c0);
        for (int j = 0; j < cnt; ++j) tot = __fadd_rn(tot, lane_value(v, j));
      }
      U.svi = __fdiv_rn(1.0f, fmaxf(tot, 1e-30f));
      if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) *a.svi_out = U.svi;
    } else {
      U.svi = *a.sum_v_inv;
    }
    lr_kappa = __fmul_rn(U.lr, a.p.gf_consol);
  };

  // one row's inputs for the lane's 4 columns, as loaded
  struct RowIn {
    int4 w;
    uint2 g;      // 4 bf16
    float4 c;     // coh_pre (1.0 when unused)
    int32_t re;   // row exponent
    float vr;
  };
  // FULL: all 256 columns of the block lie inside the matrix (uniform over
  // the block), so no lane masks its loads, stores or watermark terms.
  // No branch around any load: a lane past column K - 1 reads column K - 1
  // and drops the value, so the count of loads in flight is the same on
  // every path and the wait for a row never drains the next row's loads
  auto load_row = [&](int64_t n, RowIn& in, auto full_c) {
    constexpr bool FULL = decltype(full_c)::value;
    in.re = a.row_exp[n];
    in.vr = a.v_row[n];
    const int32_t* pp = a.packed + n * a.ld_p;
    const uint16_t* gp = a.grad + n * a.ld_g;
    const float* cpp = RATIO ? nullptr : a.coh_pre + n * a.ld_c;
    if (FULL) {
      in.w = *reinterpret_cast<const int4*>(pp + k0);
      in.g = *reinterpret_cast<const uint2*>(gp + k0);
      in.c = RATIO ? make_float4(1.0f, 1.0f, 1.0f, 1.0f) : *reinterpret_cast<const float4*>(cpp + k0);
    } else {
      int32_t w[4];
      uint32_t h[4];
      float c[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool ok = k0 + j < a.K;
        const int64_t kj = ok ? k0 + j : a.K - 1;
        const int32_t wl = pp[kj];
        const uint32_t hl = gp[kj];
        w[j] = ok ? wl : 0;
        h[j] = ok ? hl : 0u;
        if (RATIO) {
          c[j] = 1.0f;
        } else {
          const float cl = cpp[kj];
          c[j] = ok ? cl : 1.0f;
        }
      }
      in.w = make_int4(w[0], w[1], w[2], w[3]);
      in.g = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
      in.c = make_float4(c[0], c[1], c[2], c[3]);
    }
  };
  auto compute_row = [&](int64_t n, const RowIn& in, auto full_c) {
    constexpr bool FULL = decltype(full_c)::value;
    const bool full = FULL || k0 + 4 <= a.K;
    const int32_t te_row = in.re - a.p.mantissa_bias;
    const int32_t psr = wshl((int32_t)n, 16) ^ U.salt;
    const int32_t w[4] = {in.w.x, in.w.y, in.w.z, in.w.w};
    const float g[4] = {__uint_as_float(in.g.x << 16), __uint_as_float(in.g.x & 0xFFFF0000u),
                        __uint_as_float(in.g.y << 16), __uint_as_float(in.g.y & 0xFFFF0000u)};
    float cp[4] = {in.c.x, in.c.y, in.c.z, in.c.w};
    int32_t* pp = a.packed + n * a.ld_p + k0;
    float* cpp = RATIO ? nullptr : a.coh_pre + n * a.ld_c + k0;
    int32_t out[4], m[4];
    int32_t rmax = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int32_t te = te_row + ce[j];
      out[j] = adamw_element_fast<RATIO>(w[j], g[j], exp2i_nc(te), exp2i_nc(-te), in.vr, vc[j], &cp[j],
                                         psr ^ (int32_t)(k0 + j), C, alpha, avf, lr_kappa, U, &m[j]);
      const int32_t am = (full || k0 + j < a.K) ? abs(m[j]) : 0;
      rmax = max(rmax, am);
      cmax[j] = max(cmax[j], am);
    }
    if (full) {
      *reinterpret_cast<int4*>(pp) = make_int4(out[0], out[1], out[2], out[3]);
      if (!RATIO) *reinterpret_cast<float4*>(cpp) = make_float4(cp[0], cp[1], cp[2], cp[3]);
      if (emit) {
        uint2 wv;
        wv.x = pack_bf16x2(__fmul_rn((float)m[0], exp2i(te_row + ce[0])),
                           __fmul_rn((float)m[1], exp2i(te_row + ce[1])));
        wv.y = pack_bf16x2(__fmul_rn((float)m[2], exp2i(te_row + ce[2])),
                           __fmul_rn((float)m[3], exp2i(te_row + ce[3])));
        *reinterpret_cast<uint2*>(a.wbuf + n * a.ld_w + k0) = wv;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (k0 + j < a.K) {
          pp[j] = out[j];
          if (!RATIO) cpp[j] = cp[j];
          if (emit)
            a.wbuf[n * a.ld_w + k0 + j] =
                (uint16_t)(pack_bf16x2(__fmul_rn((float)m[j], exp2i(te_row + ce[j])), 0.0f) & 0xFFFFu);
        }
      }
    }
    if (track) {
      rmax = wave_max(rmax);
      if (lane == 0) atomicMax(a.row_max + n, rmax);
    }
  };
  // the wave's rows: row blocks blockIdx.y, blockIdx.y + gridDim.y, ...
  // (grid.y <= kMaxGridY) of tn rows each, rows wave, wave + 4, ... of each;
  // the next row's loads go out before the current row's arithmetic
  // the loads of a row past the last (the walk's end) read row N - 1
  auto run = [&](auto full_c) {
    const int64_t step = (int64_t)gridDim.y * a.tn;
    int64_t nb = (int64_t)blockIdx.y * a.tn;
    int r = wave;
    RowIn cur, nxt;
    load_row(min(nb + r, a.N - 1), cur, full_c);
    setup();
    while (nb + r < a.N) {
      const int64_t n = nb + r;
      r += 4;
      if (r >= a.tn || nb + r >= a.N) {
        nb += step;
        r = wave;
      }
      load_row(min(nb + r, a.N - 1), nxt, full_c);
      compute_row(n, cur, full_c);
      cur = nxt;
    }
  };
  if (kb + 256 <= a.K) run(std::true_type());
  else run(std::false_type());
  if (track) {
#pragma unroll
    for (int j = 0; j < 4; ++j) s_cmax[wave][lane * 4 + j] = cmax[j];
    __syncthreads();
    const int64_t k = kb + threadIdx.x;
    if (k < a.K) {
      const int32_t v = max(max(s_cmax[0][threadIdx.x], s_cmax[1][threadIdx.x]),
                            max(s_cmax[2][threadIdx.x], s_cmax[3][threadIdx.x]));
      atomicMax(a.col_max + k, v);
    }
  }
}


template <int VEC>
__global__ __launch_bounds__(256) void apply_adamw_kernel(AdamwArgs a) {
  __shared__ int32_t s_cmax[4][256];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t kb = (int64_t)blockIdx.x * (64 * VEC);
  const int64_t k0 = kb + lane * VEC;
  const uint32_t flags = a.flags;

  Uniform U;
  U.lr = *a.s.lr;
  U.eps = *a.s.eps;
  U.chase_floor = (flags & CONCORD_RATIO_COH) ? *a.s.chase_floor : 0.0f;
  U.leak_floor = (flags & CONCORD_RATIO_COH) ? *a.s.leak_floor : 0.0f;
  const bool proto = flags & CONCORD_PROTO_CONSF;
  U.v_bc = (proto && a.s.v_bc) ? *a.s.v_bc : 1.0f;
  U.cons = (proto && a.s.consolidate) ? *a.s.consolidate : 1;
  U.consf = (float)U.cons;
  U.salt = *a.s.salt_counter;
  const bool need_vhat = update_needs_vhat(flags);
  U.svi = need_vhat ? *a.sum_v_inv : 0.0f;
  const bool track = (flags & CONCORD_TRACK_REBALANCE) && U.cons == 1;
  const bool emit = (flags & CONCORD_EMIT_WEIGHT) && U.cons == 1;
  const bool cohpre = (flags & CONCORD_COHPRE) && (flags & CONCORD_APPLY_CHASE) &&
                      !(flags & CONCORD_RATIO_COH);

  int32_t ce[VEC];
  float vc[VEC];
  int32_t cmax[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) {
    const int64_t k = k0 + j;
    const bool ok = k < a.K;
    ce[j] = ok ? (int32_t)a.col_exp[k] : 0;
    vc[j] = (ok && need_vhat) ? a.v_col[k] : 0.0f;
    cmax[j] = 0;
  }
  const bool full = k0 + VEC <= a.K;

  // row blocks blockIdx.y, blockIdx.y + gridDim.y, ... (grid.y <= kMaxGridY)
  for (int64_t nb = (int64_t)blockIdx.y * a.tn; nb < a.N; nb += (int64_t)gridDim.y * a.tn)
  for (int r = wave; r < a.tn; r += 4) {
    const int64_t n = nb + r;
    if (n >= a.N) break;
    const int32_t te_row = (int32_t)a.row_exp[n] - a.p.mantissa_bias;
    const float vr = need_vhat ? a.v_row[n] : 0.0f;
    int32_t w[VEC];
    float g[VEC];
    float cp[VEC];
    int32_t* pp = a.packed + n * a.ld_p + k0;
    const uint16_t* gp = a.grad + n * a.ld_g + k0;
    float* cpp = cohpre ? a.coh_pre + n * a.ld_c + k0 : nullptr;
    if (VEC == 4 && full) {
      const int4 wv = *reinterpret_cast<const int4*>(pp);
      const uint2 gv = *reinterpret_cast<const uint2*>(gp);
      w[0] = wv.x; w[1] = wv.y; w[2] = wv.z; w[3] = wv.w;
      g[0] = __uint_as_float(gv.x << 16);
      g[1] = __uint_as_float(gv.x & 0xFFFF0000u);
      g[2] = __uint_as_float(gv.y << 16);
      g[3] = __uint_as_float(gv.y & 0xFFFF0000u);
      if (cohpre) {
        const float4 cv = *reinterpret_cast<const float4*>(cpp);
        cp[0] = cv.x; cp[1] = cv.y; cp[2] = cv.z; cp[3] = cv.w;
      }
    } else {
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const bool ok = k0 + j < a.K;
        w[j] = ok ? pp[j] : 0;
        g[j] = ok ? bf16_to_f32(gp[j]) : 0.0f;
        cp[j] = (ok && cohpre) ? cpp[j] : 1.0f;
      }
    }
    int32_t out[VEC], m[VEC];
    int32_t rmax = 0;
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      out[j] = adamw_element(w[j], g[j], te_row + ce[j], vr, vc[j], &cp[j], (int)n, (int)(k0 + j),
                             a.p, U, flags, &m[j]);
      const int32_t am = (full || k0 + j < a.K) ? abs(m[j]) : 0;
      rmax = max(rmax, am);
      cmax[j] = max(cmax[j], am);
    }
    if (VEC == 4 && full) {
      *reinterpret_cast<int4*>(pp) = make_int4(out[0], out[1], out[2], out[3]);
      if (cohpre) *reinterpret_cast<float4*>(cpp) = make_float4(cp[0], cp[1], cp[2], cp[3]);
      if (emit) {
        uint2 wv;
        wv.x = pack_bf16x2(__fmul_rn((float)m[0], exp2i(te_row + ce[0])),
                           __fmul_rn((float)m[1], exp2i(te_row + ce[1])));
        wv.y = pack_bf16x2(__fmul_rn((float)m[2], exp2i(te_row + ce[2])),
                           __fmul_rn((float)m[3], exp2i(te_row + ce[3])));
        *reinterpret_cast<uint2*>(a.wbuf + n * a.ld_w + k0) = wv;
      }
    } else {
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        if (k0 + j < a.K) {
          pp[j] = out[j];
          if (cohpre) cpp[j] = cp[j];
          if (emit) {
            const float v = __fmul_rn((float)m[j], exp2i(te_row + ce[j]));
            a.wbuf[n * a.ld_w + k0 + j] = (uint16_t)(pack_bf16x2(v, 0.0f) & 0xFFFFu);
          }
        }
      }
    }
    if (track) {
      rmax = wave_max(rmax);
      if (lane == 0) atomicMax(a.row_max + n, rmax);
    }
  }
  if (track) {
#pragma unroll
    for (int j = 0; j < VEC; ++j) s_cmax[wave][lane * VEC + j] = cmax[j];
    __syncthreads();
    for (int c = threadIdx.x; c < 64 * VEC; c += 256) {
      const int64_t k = kb + c;
      if (k < a.K) {
        const int32_t v = max(max(s_cmax[0][c], s_cmax[1][c]), max(s_cmax[2][c], s_cmax[3][c]));
        atomicMax(a.col_max + k, v);
      }
    }
  }
}

// ---- SGD -----------------------------------------------------------------------
struct SgdArgs {
  int32_t* packed;
  const uint16_t* grad;
  uint16_t* wbuf;
  const int8_t* row_exp;
  const int8_t* col_exp;
  int32_t* row_max;
  int32_t* col_max;
  int64_t ld_p, ld_g, ld_w, N, K;
  const float* lr;
  const int32_t* salt;
  int32_t mantissa_bias;
  float alpha, beta1, alpha_v_fast;
  uint32_t flags;
  int tn;
};

__global__ __launch_bounds__(256) void apply_sgd_kernel(SgdArgs a) {
  __shared__ int32_t s_cmax[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t k = (int64_t)blockIdx.x * 64 + lane;
  const float lr = *a.lr;
  const int32_t salt = *a.salt;
  const bool track = a.flags & CONCORD_TRACK_REBALANCE;
  const bool emit = a.flags & CONCORD_EMIT_WEIGHT;
  const bool kok = k < a.K;
  const int32_t ce = kok ? (int32_t)a.col_exp[k] : 0;
  int32_t cmax = 0;
  // row blocks blockIdx.y, blockIdx.y + gridDim.y, ... (grid.y <= kMaxGridY)
  for (int64_t nb = (int64_t)blockIdx.y * a.tn; nb < a.N; nb += (int64_t)gridDim.y * a.tn)
  for (int r = wave; r < a.tn; r += 4) {
    const int64_t n = nb + r;
    if (n >= a.N) break;
    int32_t am = 0;
    if (kok) {
      Fields f = unpack(a.packed[n * a.ld_p + k]);
      int32_t sf = f.sf, ss = f.ss;
      const float g = bf16_to_f32(a.grad[n * a.ld_g + k]);
      const int32_t te = (int32_t)a.row_exp[n] + ce - a.mantissa_bias;
      const float delta_grad = __fmul_rn(__fmul_rn(-lr, g), exp2i(-te));
      const float delta_t = __fsub_rn(delta_grad, __fmul_rn(a.beta1, (float)sf));
      const int32_t ps = wshl((int32_t)n, 16) ^ (int32_t)k ^ salt;
      sf = wadd(sf, sr_tick(delta_t, hash_uniform(sf, ps)));
      const float c8 = __fmul_rn(__fmul_rn(a.alpha, (float)sf), 0.0078125f);
      const int32_t t2 = sr_tick(c8, hash_uniform3(sf, ps, 0x5A5A5A5A));
      ss = wadd(ss, t2);
      sf = wsub(sf, wshl(t2, 7));
      const float dv8 =
          __fmul_rn(__fmul_rn(a.alpha_v_fast, (float)wsub(wshl(ss, 7), f.vs * 128)), 0.0078125f);
      const int32_t t3 = sr_tick(dv8, hash_uniform3(sf, ps, 0x33335555));
      const int32_t new_v = clampi(wadd(f.vs, t3), -128, 127);
      if (a.flags & CONCORD_MASS_PRESERVE) ss = wsub(ss, wsub(new_v, f.vs));
      const int32_t sfc = clampi(sf, -32768, 32767), ssc = clampi(ss, -128, 127);
      a.packed[n * a.ld_p + k] = pack(sfc, ssc, new_v);
      const int32_t m = ssc * 128 + sfc + new_v * 128;
      if (emit)
        a.wbuf[n * a.ld_w + k] = (uint16_t)(pack_bf16x2(__fmul_rn((float)m, exp2i(te)), 0.0f) & 0xFFFFu);
      am = abs(m);
    }
    cmax = max(cmax, am);
    if (track) {
      const int32_t rm = wave_max(am);
      if (lane == 0) atomicMax(a.row_max + n, rm);
    }
  }
  if (track) {
    s_cmax[wave][lane] = cmax;
    __syncthreads();
    if (threadIdx.x < 64) {
      const int64_t kk = (int64_t)blockIdx.x * 64 + threadIdx.x;
      if (kk < a.K)
        atomicMax(a.col_max + kk, max(max(s_cmax[0][threadIdx.x], s_cmax[1][threadIdx.x]),
                                      max(s_cmax[2][threadIdx.x], s_cmax[3][threadIdx.x])));
    }
  }
}

__global__ void salt_bump_kernel(int32_t* c) {
  if (threadIdx.x == 0 && blockIdx.x == 0) c[0] = wadd(c[0], 1);
}

// rows per block: the smallest count of block rounds times (rows per block
// + 2), a round being the blocks resident at once (5 blocks of 4 waves per
// CU at this kernel's register count, 256 CUs); the +2 prices the per-block
// set-up (the scalar loads, the column exponents and v_col), which dominated
// at one row per wave (the 640 x 5760 conv weight: 35 us at 4 rows per
// block, 29 us at 8); ties go to more rows per block
static int choose_tn(int64_t N, int64_t col_blocks) {
  const int64_t slots = 256 * 5;
  int best = 8;
  int64_t best_cost = INT64_MAX;
  for (int tn = 8; tn <= 64; tn += 4) {
    const int64_t blocks = col_blocks * cdiv(N, tn);
    const int64_t cost = cdiv(blocks, slots) * (tn + 2);
    if (cost <= best_cost) {
      best_cost = cost;
      best = tn;
    }
  }
  return best;
}

static bool aligned(const void* p, int a) { return ((uintptr_t)p % a) == 0; }

}  // namespace concord

using namespace concord;

extern "C" int concord_salt_bump(int32_t* salt_counter, void* stream) {
  CONCORD_CHECK(salt_counter, "concord_salt_bump: salt_counter is NULL");
  hipLaunchKernelGGL(salt_bump_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, salt_counter);
  return launch_status("salt_bump");
}

namespace concord {

// concord_apply_adamw; with bsum set, the fast kernel (which the caller has
// checked applies: adamw_fast_eligible) forms 1 / sum v_row from the 256-row
// totals and stores it to svi_out
static int apply_adamw_impl(int32_t* packed, int64_t ld_p, const uint16_t* grad, int64_t ld_g,
                            uint16_t* weight_buf, int64_t ld_w, const int8_t* row_exp, const int8_t* col_exp,
                            int32_t* row_max, int32_t* col_max, const float* v_row, const float* v_col,
                            const float* sum_v_inv, float* coh_pre, int64_t ld_c, int64_t N, int64_t K,
                            const concord_update_params* params, const concord_device_scalars* scalars,
                            uint32_t flags, void* stream, const float* bsum, int64_t nbsum, float* svi_out) {
  CONCORD_CHECK(N >= 0 && K >= 0, "concord_apply_adamw: negative size");
  CONCORD_CHECK(N < ((int64_t)1 << 31) && K < ((int64_t)1 << 31),
                "concord_apply_adamw: N=%lld K=%lld outside the int32 index range",
                (long long)N, (long long)K);
  CONCORD_CHECK(params && scalars, "concord_apply_adamw: params/scalars NULL");
  if (N == 0 || K == 0) return CONCORD_OK;
  CONCORD_CHECK(packed && grad && row_exp && col_exp, "concord_apply_adamw: NULL tensor");
  CONCORD_CHECK(ld_p >= K && ld_g >= K, "concord_apply_adamw: leading dimension < K");
  CONCORD_CHECK(scalars->lr && scalars->eps && scalars->salt_counter,
                "concord_apply_adamw: lr/eps/salt_counter NULL");
  const bool need_vhat = update_needs_vhat(flags);
  CONCORD_CHECK(!need_vhat || (v_row && v_col && (sum_v_inv || bsum)),
                "concord_apply_adamw: gf_trust/gf_consol/coh_pre/ratio_coh need v_row, v_col, sum_v_inv");
  CONCORD_CHECK(!(flags & CONCORD_RATIO_COH) || (scalars->chase_floor && scalars->leak_floor),
                "concord_apply_adamw: RATIO_COH needs chase_floor/leak_floor");
  const bool cohpre = (flags & CONCORD_COHPRE) && (flags & CONCORD_APPLY_CHASE) &&
                      !(flags & CONCORD_RATIO_COH);
  CONCORD_CHECK(!cohpre || (coh_pre && ld_c >= K), "concord_apply_adamw: COHPRE needs coh_pre");
  CONCORD_CHECK(!(flags & CONCORD_EMIT_WEIGHT) || (weight_buf && ld_w >= K),
                "concord_apply_adamw: EMIT_WEIGHT needs weight_buf");
  CONCORD_CHECK(!(flags & CONCORD_TRACK_REBALANCE) || (row_max && col_max),
                "concord_apply_adamw: TRACK_REBALANCE needs row_max/col_max");
  hipStream_t st = (hipStream_t)stream;
  if (!(flags & CONCORD_SALT_PREBUMPED)) {
    hipLaunchKernelGGL(salt_bump_kernel, dim3(1), dim3(64), 0, st, scalars->salt_counter);
  }
  AdamwArgs a;
  a.packed = packed; a.grad = grad; a.wbuf = weight_buf; a.row_exp = row_exp;
  a.col_exp = col_exp; a.row_max = row_max; a.col_max = col_max; a.v_row = v_row;
  a.v_col = v_col; a.sum_v_inv = sum_v_inv; a.coh_pre = coh_pre;
  a.bsum = bsum; a.nbsum = nbsum; a.svi_out = svi_out;
  a.ld_p = ld_p; a.ld_g = ld_g; a.ld_w = ld_w; a.ld_c = ld_c; a.N = N; a.K = K;
  a.p = *params; a.s = *scalars; a.flags = flags;
  const bool vec4 = (ld_p % 4 == 0) && (ld_g % 4 == 0) && aligned(packed, 16) &&
                    aligned(grad, 8) && (!cohpre || (ld_c % 4 == 0 && aligned(coh_pre, 16))) &&
                    (!(flags & CONCORD_EMIT_WEIGHT) || (ld_w % 4 == 0 && aligned(weight_buf, 8)));
  const int fast = vec4 ? update_fast_path(*params, flags) : 0;
  CONCORD_CHECK(!bsum || (fast != 0 && svi_out), "apply_adamw: the totals form needs the fast kernel");
  if (vec4) {
    const int64_t cb = cdiv(K, 256);
    a.tn = choose_tn(N, cb);
    const dim3 grid((unsigned)cb, grid_y(cdiv(N, a.tn)));
    switch (fast) {
      case 2: hipLaunchKernelGGL(apply_adamw_fast_kernel<true>, grid, dim3(256), 0, st, a); break;
      case 1: hipLaunchKernelGGL(apply_adamw_fast_kernel<false>, grid, dim3(256), 0, st, a); break;
      default: hipLaunchKernelGGL(apply_adamw_kernel<4>, grid, dim3(256), 0, st, a); break;
    }
  } else {
    const int64_t cb = cdiv(K, 64);
    a.tn = choose_tn(N, cb);
    hipLaunchKernelGGL(apply_adamw_kernel<1>, dim3((unsigned)cb, grid_y(cdiv(N, a.tn))), dim3(256), 0, st, a);
  }
  return launch_status("apply_adamw");
}

bool adamw_fast_eligible(const concord_update_params& p, uint32_t flags, const int32_t* packed, int64_t ld_p,
                         const uint16_t* grad, int64_t ld_g, const float* coh_pre, int64_t ld_c) {
  const bool cohpre = (flags & CONCORD_COHPRE) && (flags & CONCORD_APPLY_CHASE) && !(flags & CONCORD_RATIO_COH);
  const bool vec4 = (ld_p % 4 == 0) && (ld_g % 4 == 0) && aligned(packed, 16) && aligned(grad, 8) &&
                    (!cohpre || (coh_pre && ld_c % 4 == 0 && aligned(coh_pre, 16))) &&
                    !(flags & CONCORD_EMIT_WEIGHT);
  return vec4 && update_fast_path(p, flags) != 0;
}

int apply_adamw_fast_bsum(int32_t* packed, int64_t ld_p, const uint16_t* grad, int64_t ld_g, const int8_t* row_exp,
                          const int8_t* col_exp, int32_t* row_max, int32_t* col_max, const float* v_row,
                          const float* v_col, const float* bsum, int64_t nbsum, float* sum_v_inv, float* coh_pre,
                          int64_t ld_c, int64_t N, int64_t K, const concord_update_params* params,
                          const concord_device_scalars* scalars, uint32_t flags, hipStream_t stream) {
  return apply_adamw_impl(packed, ld_p, grad, ld_g, nullptr, K, row_exp, col_exp, row_max, col_max, v_row, v_col,
                          nullptr, coh_pre, ld_c, N, K, params, scalars, flags, stream, bsum, nbsum, sum_v_inv);
}

}  // namespace concord

using namespace concord;

extern "C" int concord_apply_adamw(int32_t* packed, int64_t ld_p, const uint16_t* grad,
                                   int64_t ld_g, uint16_t* weight_buf, int64_t ld_w,
                                   const int8_t* row_exp, const int8_t* col_exp, int32_t* row_max,
                                   int32_t* col_max, const float* v_row, const float* v_col,
                                   const float* sum_v_inv, float* coh_pre, int64_t ld_c, int64_t N,
                                   int64_t K, const concord_update_params* params,
                                   const concord_device_scalars* scalars, uint32_t flags,
                                   void* stream) {
  return apply_adamw_impl(packed, ld_p, grad, ld_g, weight_buf, ld_w, row_exp, col_exp, row_max, col_max, v_row,
                          v_col, sum_v_inv, coh_pre, ld_c, N, K, params, scalars, flags, stream, nullptr, 0,
                          nullptr);
}

extern "C" int concord_apply_sgd(int32_t* packed, int64_t ld_p, const uint16_t* grad, int64_t ld_g,
                                 uint16_t* weight_buf, int64_t ld_w, const int8_t* row_exp,
                                 const int8_t* col_exp, int32_t* row_max, int32_t* col_max,
                                 int64_t N, int64_t K, const float* lr, int32_t mantissa_bias,
                                 float alpha, float beta1, float alpha_v_fast,
                                 int32_t* salt_counter, uint32_t flags, void* stream) {
  CONCORD_CHECK(N >= 0 && K >= 0, "concord_apply_sgd: negative size");
  CONCORD_CHECK(N < ((int64_t)1 << 31) && K < ((int64_t)1 << 31), "concord_apply_sgd: size too large");
  if (N == 0 || K == 0) return CONCORD_OK;
  CONCORD_CHECK(packed && grad && row_exp && col_exp && lr && salt_counter,
                "concord_apply_sgd: NULL argument");
  CONCORD_CHECK(ld_p >= K && ld_g >= K, "concord_apply_sgd: leading dimension < K");
  CONCORD_CHECK(!(flags & CONCORD_EMIT_WEIGHT) || (weight_buf && ld_w >= K),
                "concord_apply_sgd: EMIT_WEIGHT needs weight_buf");
  CONCORD_CHECK(!(flags & CONCORD_TRACK_REBALANCE) || (row_max && col_max),
                "concord_apply_sgd: TRACK_REBALANCE needs row_max/col_max");
  hipStream_t st = (hipStream_t)stream;
  if (!(flags & CONCORD_SALT_PREBUMPED))
    hipLaunchKernelGGL(salt_bump_kernel, dim3(1), dim3(64), 0, st, salt_counter);
  SgdArgs a;
  a.packed = packed; a.grad = grad; a.wbuf = weight_buf; a.row_exp = row_exp;
  a.col_exp = col_exp; a.row_max = row_max; a.col_max = col_max;
  a.ld_p = ld_p; a.ld_g = ld_g; a.ld_w = ld_w; a.N = N; a.K = K; a.lr = lr; a.salt = salt_counter;
  a.mantissa_bias = mantissa_bias; a.alpha = alpha; a.beta1 = beta1; a.alpha_v_fast = alpha_v_fast;
  a.flags = flags;
  const int64_t cb = cdiv(K, 64);
  a.tn = choose_tn(N, cb);
  hipLaunchKernelGGL(apply_sgd_kernel, dim3((unsigned)cb, grid_y(cdiv(N, a.tn))), dim3(256), 0, st, a);
  return launch_status("apply_sgd");
}
