/*
 * concord_oracle.h -- CPU restatement of Concord's packed-weight linear path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the concord_amd package,
 * its HIP kernels or its C-ABI) includes, links or calls this code.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and
 * only as the checker (or as the timed CPU baseline), never as the thing
 * measured or shipped.
 *
 * Every function follows one reference function op for op (citations are
 * relative to the reference repository root).  The semantics that the
 * reference leaves to its compiler are fixed here, and the HIP kernels follow
 * the same fixed semantics:
 *   - IEEE binary32 +,-,*,/ with round-to-nearest-even, no FMA contraction
 *     (build with -ffp-contract=off), denormals kept;
 *   - float -> int32 conversion truncates toward zero, saturates out-of-range
 *     values to INT32_MIN/INT32_MAX and maps NaN to 0 (gfx950 v_cvt_i32_f32);
 *   - int32 additions/shifts wrap modulo 2^32 (Triton's i32 semantics);
 *   - fminf/fmaxf (IEEE maxNum: a NaN operand yields the other operand);
 *   - the Padam power (v+eps)^p is sqrtf() for p == 0.5, 1 for p == 0 and
 *     concord_pow_p() (defined below, deterministic) otherwise;
 *   - fp32 -> bf16 is round-to-nearest-even (NaN -> 0x7FC0);
 *   - the v-hat row/column reductions use the fixed order documented at
 *     oracle_vhat_ema().
 */
#ifndef CONCORD_ORACLE_H
#define CONCORD_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Update-flag bits (shared numbering with the product's C-ABI header). */
#define OR_MASS_PRESERVE      (1u << 0)
#define OR_APPLY_CHASE        (1u << 1)
#define OR_TRACK_REBALANCE    (1u << 2)
#define OR_GF_TRUST_REGION    (1u << 3)
#define OR_GF_CONSOLIDATION   (1u << 4)
#define OR_COHPRE             (1u << 5)
#define OR_FIXED_COH          (1u << 6)
#define OR_RATIO_COH          (1u << 7)
#define OR_EMIT_WEIGHT        (1u << 8)
#define OR_PROTO_CONSF        (1u << 9)
#define OR_MUON               (1u << 10)

typedef struct {
    float alpha, beta1, weight_decay, step_cap, v_scale, precond_p;
    float gf_consol, drift_cancel_C, alpha_v_fast, wd_sv, wd_sf;
    float gf_trust_delta_sq, gate_gain;
    int32_t mantissa_bias;
} oracle_update_params;

/* Device-scalar values (read from device memory by the kernels). */
typedef struct {
    float lr, eps, chase_floor, leak_floor, v_bc;
    int32_t salt, consolidate;
} oracle_update_scalars;

float    oracle_hash_uniform(int32_t x, int32_t pos, int32_t salt);
void     oracle_philox4x32_10(uint32_t ctr[4], uint32_t key[2]);
float    oracle_tl_rand(int32_t seed, int32_t offset);
int32_t  oracle_f2i(float f);
uint16_t oracle_f32_to_bf16(float f);
float    oracle_pow_p(float x, float p);
double   oracle_drift_cancel_C(double alpha, double alpha_v_fast,
                               double alpha_v_slow, int refit_period,
                               int mass_preserve);

void oracle_materialize(const int32_t* packed, const int8_t* row_exp,
                        const int8_t* col_exp, int64_t N, int64_t K,
                        int32_t mantissa_bias, int consolidated,
                        uint16_t* out_bf16);
/* concord/packed_b.py:1763-1772: bf16(((ss*128 + g*sf) + vs*128) * 2^exp) */
void oracle_materialize_gated(const int32_t* packed, const int8_t* row_exp,
                              const int8_t* col_exp, int64_t N, int64_t K,
                              int32_t mantissa_bias, float fast_gain,
                              uint16_t* out_bf16);

void oracle_apply_adamw(int32_t* packed, const uint16_t* grad_bf16,
                        uint16_t* weight_bf16, const int8_t* row_exp,
                        const int8_t* col_exp, int32_t* row_max,
                        int32_t* col_max, const float* v_row,
                        const float* v_col, float sum_v_inv, float* coh_pre,
                        int64_t N, int64_t K, const oracle_update_params* p,
                        const oracle_update_scalars* s, uint32_t flags);

void oracle_apply_sgd(int32_t* packed, const uint16_t* grad_bf16,
                      uint16_t* weight_bf16, const int8_t* row_exp,
                      const int8_t* col_exp, int32_t* row_max,
                      int32_t* col_max, int64_t N, int64_t K, float lr,
                      int32_t mantissa_bias, float alpha, float beta1,
                      float alpha_v_fast, int32_t salt, uint32_t flags);

void oracle_i8_medians(const int32_t* packed, int64_t N, int64_t K,
                       int32_t* row_med, int32_t* col_med);

void oracle_rebalance(int32_t* packed, int8_t* row_exp, int8_t* col_exp,
                      const int32_t* row_max, const int32_t* col_max,
                      const int32_t* row_med, const int32_t* col_med,
                      int64_t N, int64_t K, int32_t max_m, int32_t exp_max,
                      int32_t exp_min, int32_t seed, int allow_tickdown);

void oracle_vhat_ema(const uint16_t* grad_bf16, int64_t N, int64_t K,
                     float* v_row, float* v_col, float* sum_v_inv,
                     double beta2);

void oracle_load_weights(const float* W, int64_t N, int64_t K,
                         int32_t exp_min, int32_t exp_max,
                         int32_t mantissa_bias, int finetune,
                         int32_t* packed, int8_t* row_exp, int8_t* col_exp);

float oracle_frob_sumsq(const uint16_t* g, int64_t N, int64_t K);
/* sum of gate_coherence_from_fields (concord/packed_b.py:2081-2091) over the
 * N x K words, in the library's block / lane / tree order */
float oracle_coherence_sum(const int32_t* packed, int64_t N, int64_t K, float C);
/* standard normal draw idx of stream (seed, tag): Box-Muller on one
 * Philox4x32-10 block (counter (idx, 0, 0, 0), key (seed, tag)), words 0 and
 * 1, cos output, with this build's fixed-order log2 / sqrt / cos(2 pi u); the
 * per-token draws of the Sigma_g noise use tag 0x5369676D */
float oracle_normal_draw_tag(int32_t seed, uint32_t idx, uint32_t tag);
/* the isotropic stream: the four draws of Philox block blk under key (seed,
 * 0x6E6F6973), words (0, 1) and (2, 3) as two Box-Muller pairs, cos then sin
 * of each; element e of a gradient takes draw e & 3 of block e >> 2 */
void oracle_iso_draw4(int32_t seed, uint32_t blk, float z[4]);
float oracle_iso_draw(int32_t seed, int64_t e);
/* sum of the per-token draws 0 .. M-1 in the library's block / lane / tree order */
float oracle_token_sum(int32_t seed, int64_t M);
/* Sigma_g combine in place (prototype_packed_b.py:1489-1500), P the product
 * (eps * dy)^T x as bf16: noise = P - S * (g / M), then
 * g <- bf16(g + noise * (sigma * ||g|| / max(||noise||, 1e-12))) */
void oracle_sigmag_combine(uint16_t* g, const uint16_t* P, int64_t N, int64_t K, float S, float Mf,
                           float sigma);
/* isotropic gradient noise in place: g <- bf16(g + xi * (sigma * ||g|| /
 * max(||xi||, 1e-12))), xi_e = oracle_iso_draw(salt, e)
 * (notebook/src/prototype_packed_b.py:1484-1501, isotropic branch) */
void oracle_iso_noise(uint16_t* g, int64_t N, int64_t K, float sigma, int32_t salt);
void oracle_muon_ns5(const uint16_t* g, int64_t N, int64_t K, float gamma, uint16_t* out);

void oracle_set_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
