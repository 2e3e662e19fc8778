// update_fast.h -- the packed update's element for the two production flag
// sets (the fast path of apply_adamw_fast_kernel), shared by the update
// kernel and the WGRAD kernel that carries the update (gemm_fast.hip).
// Op order = concord/packed_b.py:494-689.
#pragma once
#include "common.h"

namespace concord {

struct Uniform {
  float lr, eps, chase_floor, leak_floor, v_bc, svi;
  int32_t salt, cons;
  float consf;
};

// Field operands taken straight from the packed word by SDWA operand
// selects (sign-extended byte 0 = vs, byte 1 = ss, high half-word = sf), so
// the fields need no extract instructions of their own.
CONCORD_DEV int32_t w_ss_minus_vs(int32_t w) {
  int32_t r;
  asm("v_sub_u32_sdwa %0, sext(%1), sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1 src1_sel:BYTE_0"
      : "=v"(r) : "v"(w));
  return r;
}
CONCORD_DEV float w_sf_float(int32_t w) {
  float r;
  asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:WORD_1" : "=v"(r) : "v"(w));
  return r;
}
CONCORD_DEV int32_t w_plus_sf(int32_t x, int32_t w) {
  int32_t r;
  asm("v_add_u32_sdwa %0, %1, sext(%2) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:WORD_1"
      : "=v"(r) : "v"(x), "v"(w));
  return r;
}
CONCORD_DEV int32_t w_xor_sf(int32_t x, int32_t w) {
  int32_t r;
  asm("v_xor_b32_sdwa %0, %1, sext(%2) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:WORD_1"
      : "=v"(r) : "v"(x), "v"(w));
  return r;
}
CONCORD_DEV int32_t w_plus_ss(int32_t x, int32_t w) {
  int32_t r;
  asm("v_add_u32_sdwa %0, %1, sext(%2) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1"
      : "=v"(r) : "v"(x), "v"(w));
  return r;
}
CONCORD_DEV int32_t w_plus_vs(int32_t x, int32_t w) {
  int32_t r;
  asm("v_add_u32_sdwa %0, %1, sext(%2) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0"
      : "=v"(r) : "v"(x), "v"(w));
  return r;
}
CONCORD_DEV int32_t w_minus_vs(int32_t x, int32_t w) {
  int32_t r;
  asm("v_sub_u32_sdwa %0, %1, sext(%2) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0"
      : "=v"(r) : "v"(x), "v"(w));
  return r;
}

// Specialised element for the two production configurations, chosen by the
// host only when every dropped term is an exact no-op:
//   RATIO (winner): ratio-coherence gates + gf evaporation, no coh_pre;
//   !RATIO (bare default): coh_pre-gated chase, no evaporation.
// Preconditions: FIXED_COH, TRUST with delta^2 = 1, v_scale = 0, p = 0.5,
// beta1 = 0, weight_decay = wd_sv = wd_sf = 0, gate_gain = 1, APPLY_CHASE,
// MASS_PRESERVE, no PROTO/MUON.  Then v_proxy = nw^2 * 0 + 1 * v_hat = v_hat
// exactly; the beta1 and weight-decay terms add +-0 (the SR tick of a +-0
// delta is 0 whatever the zero's sign); the Wiener gain sig2/(sig2+nw2+1e-30)
// already lies in [0, 1], so its clamp is the identity.
template <bool RATIO>
CONCORD_DEV int32_t adamw_element_fast(int32_t word, float g, float scale_fwd, float scale_inv,
                                       float vr, float vc, float* coh_pre, int32_t ps,
                                       float C, float alpha, float avf, float lr_kappa,
                                       const Uniform& U, int32_t* m_out) {
  const int32_t w = word;
  const float d_fs = w_sf_float(w);                      // (float) sf
  const float d_sv = (float)wshl(w_ss_minus_vs(w), 7);   // (float) (ss * 128 - vs * 128)
  const float cd = __fmul_rn(C, d_sv);
  const float nw = __fmul_rn(__fsub_rn(d_fs, cd), scale_fwd);
  const float v_hat = __fmul_rn(__fmul_rn(vr, vc), U.svi);
  const float sig_w = __fmul_rn(cd, scale_fwd);
  const float sig2 = __fmul_rn(sig_w, sig_w);
  const float coh = __fdiv_rn(sig2, __fadd_rn(__fadd_rn(sig2, __fmul_rn(nw, nw)), 1e-30f));
  float step = __fdiv_rn(g, sqrt_rn(__fadd_rn(v_hat, U.eps)));
  step = fminf(fmaxf(step, -10.0f), 10.0f);
  float delta_t = __fmul_rn(__fmul_rn(-U.lr, step), scale_inv);
  if (RATIO) delta_t = __fsub_rn(delta_t, __fmul_rn(__fmul_rn(lr_kappa, __fsub_rn(1.0f, coh)), d_fs));
  int32_t sf = w_plus_sf(sr_tick(delta_t, hash_mix(w_xor_sf(ps, w))), w);   // sf + tick, hash of the old sf

  float gate;
  if (RATIO) {
    gate = __fadd_rn(U.chase_floor, __fmul_rn(__fsub_rn(1.0f, U.chase_floor), coh));
  } else {
    const float cp = *coh_pre;
    gate = __fadd_rn(coh, __fmul_rn(cp, __fsub_rn(1.0f, coh)));
    *coh_pre = __fadd_rn(__fmul_rn(__fsub_rn(1.0f, avf), cp), __fmul_rn(avf, coh));
  }
  const float chase = __fmul_rn(__fmul_rn(alpha, gate), (float)sf);
  const int32_t t2 = sr_tick(__fmul_rn(chase, 0.0078125f), hash_uniform3(sf, ps, 0x5A5A5A5A));
  int32_t ss = w_plus_ss(t2, w);                         // ss + t2
  sf = wsub(sf, wshl(t2, 7));
  float dv8 = __fmul_rn(__fmul_rn(avf, (float)wshl(w_minus_vs(ss, w), 7)), 0.0078125f);
  if (RATIO) dv8 = __fmul_rn(dv8, __fadd_rn(U.leak_floor, __fmul_rn(__fsub_rn(1.0f, U.leak_floor), coh)));
  const int32_t t3 = sr_tick(dv8, hash_uniform3(sf, ps, 0x33335555));
  const int32_t new_v = clampi(w_plus_vs(t3, w), -128, 127);   // vs + t3, clamped
  ss = wsub(ss, w_minus_vs(new_v, w));                  // ss - (new_v - vs)
  const int32_t sfc = clampi(sf, -32768, 32767);
  const int32_t ssc = clampi(ss, -128, 127);
  *m_out = ssc * 128 + sfc + new_v * 128;
  return pack(sfc, ssc, new_v);
}

// whether concord_apply_adamw with these arguments runs the fast kernel
// (update.hip)
bool adamw_fast_eligible(const concord_update_params& p, uint32_t flags, const int32_t* packed, int64_t ld_p,
                         const uint16_t* grad, int64_t ld_g, const float* coh_pre, int64_t ld_c);
// concord_apply_adamw without weight_buf through the fast kernel, 1 / sum v_row
// formed from the finalize's 256-row totals bsum[nbsum] (the finalize's
// chain) and stored to sum_v_inv (update.hip); adamw_fast_eligible must hold
int apply_adamw_fast_bsum(int32_t* packed, int64_t ld_p, const uint16_t* grad, int64_t ld_g, const int8_t* row_exp,
                          const int8_t* col_exp, int32_t* row_max, int32_t* col_max, const float* v_row,
                          const float* v_col, const float* bsum, int64_t nbsum, float* sum_v_inv, float* coh_pre,
                          int64_t ld_c, int64_t N, int64_t K, const concord_update_params* params,
                          const concord_device_scalars* scalars, uint32_t flags, hipStream_t stream);

// 0 = generic kernel, 1 = bare fast path, 2 = winner fast path
inline int update_fast_path(const concord_update_params& p, uint32_t flags) {
  const uint32_t need = CONCORD_FIXED_COH | CONCORD_GF_TRUST_REGION | CONCORD_APPLY_CHASE |
                        CONCORD_MASS_PRESERVE;
  if ((flags & need) != need) return 0;
  if (flags & (CONCORD_PROTO_CONSF | CONCORD_MUON)) return 0;
  if (!(p.v_scale == 0.0f && p.gf_trust_delta_sq == 1.0f && p.precond_p == 0.5f &&
        p.beta1 == 0.0f && p.weight_decay == 0.0f && p.wd_sv == 0.0f && p.wd_sf == 0.0f &&
        p.gate_gain == 1.0f && p.step_cap == 10.0f))
    return 0;
  // the scale exponents +-(row_exp + col_exp - mantissa_bias) of int8
  // exponents stay inside exp2i's clamp of +-300, so the fast kernels form
  // the scales with exp2i_nc
  if (p.mantissa_bias < -40 || p.mantissa_bias > 40) return 0;
  const bool ratio = flags & CONCORD_RATIO_COH, consol = flags & CONCORD_GF_CONSOLIDATION,
             cohpre = flags & CONCORD_COHPRE;
  if (ratio && consol) return 2;
  if (!ratio && !consol && cohpre) return 1;
  return 0;
}

}  // namespace concord
