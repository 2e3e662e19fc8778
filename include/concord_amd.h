/*
 * concord_amd.h -- C ABI of the MI355X (gfx950) packed-weight linear path.
 *
 * Every entry point takes raw device pointers, sizes and leading dimensions,
 * plus the hipStream_t (passed as void*) to enqueue on.  No entry point
 * allocates device memory, synchronises the host or reads device values back
 * to the host, so every call is asynchronous and can be captured into a HIP
 * graph.  Scratch space is a caller-owned workspace (concord_workspace_bytes).
 *
 * Tensors are row-major with an explicit leading dimension (elements):
 *   packed  int32 [N, ld_p]   one word per weight: s_fast int16 in bits 31..16,
 *                             s_slow int8 in 15..8, v_slow int8 in 7..0
 *   row_exp int8  [N], col_exp int8 [K]
 *   live weight  W[n,k] = (s_fast + 128 s_slow + 128 v_slow) * 2^(row_exp[n] + col_exp[k] - mantissa_bias)
 *   bf16 tensors are passed as uint16_t bit patterns.
 *
 * Return value: CONCORD_OK (0) or a negative CONCORD_E* code; the message of
 * the last failure on the calling thread is returned by concord_last_error().
 *
 * Reference citations are relative to the reference repository root.
 */
#ifndef CONCORD_AMD_H
#define CONCORD_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CONCORD_OK 0
#define CONCORD_EINVAL (-1)     /* bad argument (null pointer, size, stride, flag) */
#define CONCORD_ELAUNCH (-2)    /* a kernel launch failed */
#define CONCORD_EWORKSPACE (-3) /* workspace missing or too small */

/* Update flags (concord/packed_b.py:451-458 constexprs, plus this build's). */
#define CONCORD_MASS_PRESERVE (1u << 0)
#define CONCORD_APPLY_CHASE (1u << 1)
#define CONCORD_TRACK_REBALANCE (1u << 2)
#define CONCORD_GF_TRUST_REGION (1u << 3)
#define CONCORD_GF_CONSOLIDATION (1u << 4)
#define CONCORD_COHPRE (1u << 5)
#define CONCORD_FIXED_COH (1u << 6)
#define CONCORD_RATIO_COH (1u << 7)
#define CONCORD_EMIT_WEIGHT (1u << 8)   /* write the bf16 live weight (materialize-merge) */
#define CONCORD_PROTO_CONSF (1u << 9)   /* notebook/src/prototype_packed_b.py:454-778 semantics */
#define CONCORD_MUON (1u << 10)         /* step = supplied drive (docs/MUON_IMPLEMENTATION.md:87-119) */
#define CONCORD_SALT_PREBUMPED (1u << 16) /* the caller already advanced the salt counter */

/* Launch-time scalars of the update (concord/packed_b.py:436-445). */
typedef struct concord_update_params {
  float alpha, beta1, weight_decay, step_cap, v_scale, precond_p;
  float gf_consol, drift_cancel_C, alpha_v_fast, wd_sv, wd_sf;
  float gf_trust_delta_sq, gate_gain;
  int32_t mantissa_bias;
} concord_update_params;

/* Per-step scalars read from device memory so that a captured graph sees
 * their current values (concord/packed_b.py:462-468; prototype 474-485).
 * lr, eps: fp32[1]; chase_floor, leak_floor, v_bc: fp32[1] (may be NULL when
 * RATIO_COH / PROTO_CONSF are off); salt_counter: int32[1], advanced by one on
 * device before each update unless CONCORD_SALT_PREBUMPED; consolidate:
 * int32[1] (NULL = 1). */
typedef struct concord_device_scalars {
  const float* lr;
  const float* eps;
  const float* chase_floor;
  const float* leak_floor;
  const float* v_bc;
  int32_t* salt_counter;
  const int32_t* consolidate;
} concord_device_scalars;

const char* concord_last_error(void);
int concord_version(void);

/* Bytes of caller-owned workspace the entry points below need for a layer of
 * N x K weights and M activation rows.  The workspace must be zero-filled
 * once when allocated; every call leaves its counters at zero again. */
size_t concord_workspace_bytes(int64_t N, int64_t K, int64_t M);

/* salt_counter[0] += 1 on device.  Replaces step_counter.add_(1),
 * concord/packed_b.py:910-911. */
int concord_salt_bump(int32_t* salt_counter, void* stream);

/* bf16 decode of the packed state.  consolidated = 0: live weight
 * (_materialize_packed_bf16_kernel, concord/packed_b.py:120-170; get_weight
 * 1617-1630).  consolidated = 1: deploy weight without s_fast
 * (consolidated_weight, concord/packed_b.py:1632-1649). */
int concord_materialize(const int32_t* packed, int64_t ld_p, const int8_t* row_exp,
                        const int8_t* col_exp, int64_t N, int64_t K, int32_t mantissa_bias,
                        int consolidated, uint16_t* out, int64_t ld_out, void* stream);

/* The forward weight with s_fast gated by fast_gain in [0, 1):
 * bf16(((128 s_slow + fast_gain s_fast) + 128 v_slow) * 2^(row_exp + col_exp -
 * mantissa_bias)), fp32 ops in that order.  Replaces the torch re-materialise
 * branch of ConcordLinearPackedB.forward, concord/packed_b.py:1763-1772. */
int concord_materialize_gated(const int32_t* packed, int64_t ld_p, const int8_t* row_exp,
                              const int8_t* col_exp, int64_t N, int64_t K, int32_t mantissa_bias,
                              float fast_gain, uint16_t* out, int64_t ld_out, void* stream);

/* The packed optimizer update with a supplied bf16 gradient: apply_packed_adamw
 * + _apply_packed_adamw_kernel, concord/packed_b.py:863-951 and 422-703
 * (prototype extension notebook/src/prototype_packed_b.py:454-778 under
 * CONCORD_PROTO_CONSF).  Mutates packed (and coh_pre, weight_buf, row_max,
 * col_max) in place; row_max/col_max receive atomic maxima and must be
 * zeroed by the caller (or by concord_vhat_ema). */
int concord_apply_adamw(int32_t* packed, int64_t ld_p, const uint16_t* grad, int64_t ld_g,
                        uint16_t* weight_buf, int64_t ld_w, const int8_t* row_exp,
                        const int8_t* col_exp, int32_t* row_max, int32_t* col_max,
                        const float* v_row, const float* v_col, const float* sum_v_inv,
                        float* coh_pre, int64_t ld_c, int64_t N, int64_t K,
                        const concord_update_params* params,
                        const concord_device_scalars* scalars, uint32_t flags, void* stream);

/* SGD path: apply_packed_sgd + _apply_packed_sgd_kernel,
 * concord/packed_b.py:362-394 and 173-312.  flags: MASS_PRESERVE,
 * TRACK_REBALANCE, EMIT_WEIGHT, SALT_PREBUMPED. */
int concord_apply_sgd(int32_t* packed, int64_t ld_p, const uint16_t* grad, int64_t ld_g,
                      uint16_t* weight_buf, int64_t ld_w, const int8_t* row_exp,
                      const int8_t* col_exp, int32_t* row_max, int32_t* col_max, int64_t N,
                      int64_t K, const float* lr, int32_t mantissa_bias, float alpha,
                      float beta1, float alpha_v_fast, int32_t* salt_counter, uint32_t flags,
                      void* stream);

/* AdaFactor rank-1 second moment of a bf16 gradient, in place:
 * v_row = b2 v_row + (1-b2) sum_k g^2, v_col likewise, sum_v_inv =
 * 1/max(sum v_row, 1e-30) (FusedConcordLinearPackedB.backward,
 * concord/packed_b.py:1288-1303), in the fixed reduction order of
 * oracle_vhat_ema; b2 = (float)beta2 and 1-b2 = (float)(1 - beta2) as torch
 * forms them from a Python float.  When row_max/col_max are non-NULL they are zeroed
 * (1281-1283); when salt_counter is non-NULL it is advanced by one, so the
 * following concord_apply_adamw takes CONCORD_SALT_PREBUMPED. */
int concord_vhat_ema(const uint16_t* grad, int64_t ld_g, int64_t N, int64_t K, double beta2,
                     float* v_row, float* v_col, float* sum_v_inv, int32_t* row_max,
                     int32_t* col_max, int32_t* salt_counter, void* workspace,
                     size_t workspace_bytes, void* stream);

/* rebalance(): ConcordLinearPackedB.rebalance + rebalance_packed +
 * _rebalance_packed_decide_kernel, concord/packed_b.py:1792-1814, 1129-1190,
 * 959-1095.  Folds row_max/col_max into the high-watermarks (when non-NULL),
 * advances seed[0] when advance_seed != 0 (rebalance() does, rebalance_packed
 * does not: concord/packed_b.py:1808), decides per-row/column exponent ticks from the
 * pre-call exponents, SR-shifts the fired words and updates the exponents.
 * A call where nothing fires touches O(N + K) memory. */
int concord_rebalance(int32_t* packed, int64_t ld_p, int8_t* row_exp, int8_t* col_exp,
                      const int32_t* row_max, const int32_t* col_max, int32_t* row_hwm,
                      int32_t* col_hwm, int32_t* seed, int64_t N, int64_t K, int32_t max_m,
                      int32_t exp_max, int32_t exp_min, int allow_tickdown, int advance_seed,
                      void* workspace, size_t workspace_bytes, void* stream);

/* concord_rebalance without a workspace argument.  It has no counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, kernels and results as concord_rebalance;
 * its scratch is a static device array of 2.1 MB per device (held until the
 * process ends), so N and K are each at most 131072 (larger layers get
 * CONCORD_EINVAL; use concord_rebalance).  The stream must belong to the
 * current device.  It calls no allocator.  Every call on one device shares
 * that scratch: calls that overlap on one GPU (concurrent streams or host
 * threads) race; calls in stream order do not. */
int concord_rebalance_noalloc(int32_t* packed, int64_t ld_p, int8_t* row_exp, int8_t* col_exp,
                              const int32_t* row_max, const int32_t* col_max, int32_t* row_hwm,
                              int32_t* col_hwm, int32_t* seed, int64_t N, int64_t K, int32_t max_m,
                              int32_t exp_max, int32_t exp_min, int allow_tickdown, int advance_seed,
                              void* stream);

/* Gated rebalance of a group of layers: GatedRebalance.__call__
 * (notebook/src/concord_winner.py:206-262), `if peak > MAX_M: for m in
 * layers: m.rebalance()`, with the comparison made on the device.
 *
 * concord_rebalance_group_plan (host only, no GPU call): `layers` holds
 * n_layers records of CONCORD_RG_FIELDS int64, indexed by CONCORD_RG_*:
 * the device pointers and sizes of one layer's concord_rebalance call
 * (packed, ld_p, row_exp, col_exp, row_max, col_max, row_hwm, col_hwm
 * (either may be 0), seed, N, K, max_m, exp_max, exp_min; the last two
 * fields are ignored).  Writes the plan (n_layers * CONCORD_RG_FIELDS +
 * 2 (n_layers + 1) int64) and the int32 scratch words a call needs.  The
 * plan is copied to device memory by the caller, once.
 *
 * concord_rebalance_group (two launches, no host read): when *peak >
 * gate_max, every layer of the plan is rebalanced exactly as
 * concord_rebalance(..., allow_tickdown = 0, advance_seed = 1) would do it,
 * and fires[0] (when non-NULL) is advanced by one; otherwise nothing is
 * written.  `plan` is the device copy of the plan; the workspace holds
 * scratch_words int32.  The layers must not share packed words, exponents,
 * watermark high-water marks or seeds.  Graph-capturable. */
#define CONCORD_RG_FIELDS 16
enum {
  CONCORD_RG_PACKED = 0, CONCORD_RG_LD, CONCORD_RG_ROW_EXP, CONCORD_RG_COL_EXP, CONCORD_RG_ROW_MAX,
  CONCORD_RG_COL_MAX, CONCORD_RG_ROW_HWM, CONCORD_RG_COL_HWM, CONCORD_RG_SEED, CONCORD_RG_N, CONCORD_RG_K,
  CONCORD_RG_MAX_M, CONCORD_RG_EXP_MAX, CONCORD_RG_EXP_MIN
};
int concord_rebalance_group_plan(const int64_t* layers, int32_t n_layers, int64_t* plan, int64_t plan_len,
                                 int64_t* scratch_words);
int concord_rebalance_group(const int64_t* plan, int32_t n_layers, const int32_t* peak, int32_t gate_max,
                            int32_t* fires, void* workspace, size_t workspace_bytes, int64_t scratch_words,
                            void* stream);

/* load_weights / load_weights_finetune (concord/packed_b.py:1570-1603,
 * 1816-1856): fp32 W[N, ld_w] -> packed state, row_exp, col_exp = 0. */
int concord_load_weights(const float* W, int64_t ld_w, int64_t N, int64_t K, int32_t exp_min,
                         int32_t exp_max, int32_t mantissa_bias, int finetune, int32_t* packed,
                         int64_t ld_p, int8_t* row_exp, int8_t* col_exp, void* stream);

/* The GEMM entry points below take an optional split-K workspace (NULL /
 * 0 = never split): concord_gemm_workspace_bytes(M, N, K) bytes, zero-filled
 * once when allocated; each call leaves its tile counters at zero again.
 * With a workspace, a GEMM whose tile grid is too small for the chip is split
 * 2-way along the reduction and the halves are added in a fixed way
 * (bit-identical whichever half finishes first). */
size_t concord_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K);

/* Dequant-GEMM forward: y[M,N] = x[M,K] . decode(packed)[N,K]^T (+ bias[N]),
 * bf16 in/out, fp32 accumulation on bf16 MFMA.  Replaces
 * F.linear(x, weight_buf, bias), concord/packed_b.py:1216-1219.  bias may be
 * NULL. */
int concord_dqgemm_fwd(const uint16_t* x, int64_t ld_x, const int32_t* packed, int64_t ld_p,
                       const int8_t* row_exp, const int8_t* col_exp, int32_t mantissa_bias,
                       const uint16_t* bias, uint16_t* y, int64_t ld_y, int64_t M, int64_t N,
                       int64_t K, void* workspace, size_t workspace_bytes, void* stream);

/* Dequant-GEMM dgrad: dx[M,K] = dy[M,N] . decode(packed)[N,K], on the
 * pre-update weight.  Replaces grad_y @ weight, concord/packed_b.py:1263. */
int concord_dqgemm_dgrad(const uint16_t* dy, int64_t ld_dy, const int32_t* packed, int64_t ld_p,
                         const int8_t* row_exp, const int8_t* col_exp, int32_t mantissa_bias,
                         uint16_t* dx, int64_t ld_dx, int64_t M, int64_t N, int64_t K,
                         void* workspace, size_t workspace_bytes,
                         void* stream);

/* wgrad: grad_w[N,K] = bf16(dy[M,N]^T . x[M,K]) with fp32 accumulation.
 * Replaces grad_y_flat.T @ x_flat, concord/packed_b.py:1269-1277. */
int concord_wgrad(const uint16_t* dy, int64_t ld_dy, const uint16_t* x, int64_t ld_x,
                  uint16_t* grad_w, int64_t ld_gw, int64_t M, int64_t N, int64_t K,
                  void* workspace, size_t workspace_bytes, void* stream);

/* wgrad followed by the v-hat EMA, with the v-hat partial sums formed in the
 * wgrad epilogue from the bf16 values it stores (no re-read of grad_w):
 * grad_y_flat.T @ x_flat, the watermark zeroing and the v_row/v_col EMA of
 * FusedConcordLinearPackedB.backward, concord/packed_b.py:1269-1303.  The
 * grad_w / v_row / v_col / sum_v_inv results are bit-identical to
 * concord_wgrad followed by concord_vhat_ema with the same arguments.  When
 * grad_bias is non-NULL it receives bf16(sum_m dy[m, n]) (grad_y_flat.sum(0),
 * 1338-1340), formed from the dy fragments the product already reads.
 * workspace: concord_workspace_bytes(N, K, M) bytes; gemm_workspace
 * (optional): concord_gemm_workspace_bytes(M, N, K) bytes. */
int concord_wgrad_vhat(const uint16_t* dy, int64_t ld_dy, const uint16_t* x, int64_t ld_x,
                       uint16_t* grad_w, int64_t ld_gw, int64_t M, int64_t N, int64_t K,
                       double beta2, float* v_row, float* v_col, float* sum_v_inv,
                       int32_t* row_max, int32_t* col_max, int32_t* salt_counter,
                       uint16_t* grad_bias, void* workspace, size_t workspace_bytes,
                       void* gemm_workspace, size_t gemm_workspace_bytes, void* stream);

/* concord_dqgemm_dgrad followed by concord_wgrad_vhat in one call, with the
 * same results: the backward's two products of the fused-forward layer
 * (concord/packed_b.py:1263, 1269-1303, 1338-1340).  When the dgrad splits
 * its reduction and the WGRAD grid leaves CUs idle, the dgrad's split-K
 * reduction runs in extra workgroups of the WGRAD launch instead of a launch
 * of its own.  Workspaces as for the two calls (gemm_workspace holds the
 * dgrad's partials). */
int concord_dgrad_wgrad_vhat(const uint16_t* dy, int64_t ld_dy, const int32_t* packed, int64_t ld_p,
                             const int8_t* row_exp, const int8_t* col_exp, int32_t mantissa_bias,
                             uint16_t* dx, int64_t ld_dx, const uint16_t* x, int64_t ld_x,
                             uint16_t* grad_w, int64_t ld_gw, int64_t M, int64_t N, int64_t K,
                             double beta2, float* v_row, float* v_col, float* sum_v_inv,
                             int32_t* row_max, int32_t* col_max, int32_t* salt_counter,
                             uint16_t* grad_bias, void* workspace, size_t workspace_bytes,
                             void* gemm_workspace, size_t gemm_workspace_bytes, void* stream);

/* The whole backward of the fused-forward layer with the v-hat drive:
 * concord_dgrad_wgrad_vhat (salt_counter = scalars->salt_counter) followed by
 * concord_apply_adamw(packed, ..., grad_w, ..., flags | CONCORD_SALT_PREBUMPED)
 * (FusedConcordLinearPackedB.backward, concord/packed_b.py:1263-1327,
 * 1338-1340), with the same results.  With fuse non-zero, when the flags and
 * parameters are one of the update's two fast sets (winner or bare) and the
 * shapes take the combined launch, the v-hat finalize and the update run in
 * the workgroups of the WGRAD launch, from the accumulators of its tiles
 * (*fused = 1): the bf16 weight gradient is then written to grad_w only when
 * copy_grad is non-zero.  Otherwise the separate launches run and grad_w
 * holds the gradient; when the update runs its fast kernel, 1 / sum v_row is
 * then formed in the update from the finalize's 256-row totals.  That launch's grid barriers are bounded; should a wait exceed
 * its bound (its workgroups not all resident), the launch skips its writes
 * and concord_wgrad_update_fault reports it.  CONCORD_EMIT_WEIGHT is not
 * taken.  Workspaces as for concord_dgrad_wgrad_vhat; fused may be NULL. */
int concord_dgrad_wgrad_update(const uint16_t* dy, int64_t ld_dy, int32_t* packed, int64_t ld_p,
                               const int8_t* row_exp, const int8_t* col_exp, uint16_t* dx, int64_t ld_dx,
                               const uint16_t* x, int64_t ld_x, uint16_t* grad_w, int64_t ld_gw, int copy_grad,
                               int fuse, int64_t M, int64_t N, int64_t K, double beta2, float* v_row, float* v_col,
                               float* sum_v_inv, int32_t* row_max, int32_t* col_max, float* coh_pre,
                               int64_t ld_c, uint16_t* grad_bias, const concord_update_params* params,
                               const concord_device_scalars* scalars, uint32_t flags, void* workspace,
                               size_t workspace_bytes, void* gemm_workspace, size_t gemm_workspace_bytes,
                               int* fused, void* stream);

/* Reads (and clears) the fault flag of concord_dgrad_wgrad_update's combined
 * launch in this workspace: *fault = 1 when a launch since the last read gave
 * up a grid-barrier wait.  Synchronises the stream. */
int concord_wgrad_update_fault(void* workspace, size_t workspace_bytes, int* fault, void* stream);

/* Muon drive (A13): out[N,K] = bf16(gamma * NS5(g / ||g||_F)), the quintic
 * Newton-Schulz orthogonalisation of experiments/cpu_dynamics/exp9_muon.py:44-55
 * used as the drive of MuonConcord.step (58-100; gamma = sqrt(max(N, K))) and
 * specified for the packed layer in docs/MUON_IMPLEMENTATION.md:27-40, 87-119.
 * bf16 iterates and products with fp32 accumulation; the result is the step
 * the update takes under CONCORD_MUON.  workspace:
 * concord_muon_workspace_bytes(N, K) bytes, zero-filled once when allocated. */
size_t concord_muon_workspace_bytes(int64_t N, int64_t K);
int concord_muon_ns5(const uint16_t* g, int64_t ld_g, int64_t N, int64_t K, float gamma,
                     uint16_t* out, int64_t ld_out, void* workspace, size_t workspace_bytes,
                     void* stream);

/* The forward and dgrad products over a materialised bf16 weight w[N,K]: the
 * reference's cached weight_buf path, F.linear(x, weight_buf, bias) and
 * grad_y @ weight_buf (concord/packed_b.py:1219, 1263). */
int concord_gemm_bf16_fwd(const uint16_t* x, int64_t ld_x, const uint16_t* w, int64_t ld_w,
                          const uint16_t* bias, uint16_t* y, int64_t ld_y, int64_t M, int64_t N,
                          int64_t K, void* workspace, size_t workspace_bytes, void* stream);
int concord_gemm_bf16_dgrad(const uint16_t* dy, int64_t ld_dy, const uint16_t* w, int64_t ld_w,
                            uint16_t* dx, int64_t ld_dx, int64_t M, int64_t N, int64_t K,
                            void* workspace, size_t workspace_bytes, void* stream);

/* A symmetric bf16 product c[M,M] with fp32 accumulation, as the Muon
 * drive's NS5 iteration forms it (experiments/cpu_dynamics/exp9_muon.py:52-53,
 * A = X X^T and A A): b_rows = 1: c = a b^T with b [M,R] row-major (b = a
 * gives X X^T); b_rows = 0: c = a b with b [R,M] (R = M; a and b symmetric
 * and commuting, e.g. b = a).  Only the tiles meeting the upper triangle are
 * computed; each element (i, j) with i <= j is stored at (i, j) and (j, i),
 * so c is exactly symmetric.  The same tile and split plans as concord_muon_ns5's.
 * workspace: concord_muon_workspace_bytes of the NS5 shape, or any split-K
 * workspace of at least concord_gemm_sym_workspace_bytes(M, R, b_rows). */
size_t concord_gemm_sym_workspace_bytes(int64_t M, int64_t R, int b_rows);
int concord_gemm_bf16_sym(const uint16_t* a, int64_t ld_a, const uint16_t* b, int64_t ld_b, int b_rows,
                          uint16_t* c, int64_t ld_c, int64_t M, int64_t R, void* workspace,
                          size_t workspace_bytes, void* stream);

/* grad_bias[N] = bf16(sum_m dy[m, n]) with fp32 accumulation.  Replaces
 * grad_y_flat.sum(0), concord/packed_b.py:1338-1340. */
int concord_bias_grad(const uint16_t* dy, int64_t ld_dy, int64_t M, int64_t N,
                      uint16_t* grad_bias, void* workspace, size_t workspace_bytes,
                      void* stream);

/* Multi-layer statistics over the packed state.  workspace:
 * concord_stats_workspace_bytes(n_watermarks, n_words) bytes (no zeroing
 * needed); each call is two launches and writes one scalar.
 *
 * concord_watermark_peak: *out = max of rows[0, n_rows) and cols[0, n_cols)
 * (the update's |m_eff| watermarks, all >= 0).  This is the one reduction of
 * GatedRebalance.__call__ over the shared row / column watermark slabs of every
 * layer (notebook/src/concord_winner.py:206-262: torch.maximum(row_all.max(),
 * col_all.max())); rebalance runs only when it exceeds MAX_M.
 *
 * concord_coherence_sum: *out_sum = sum over the N x K words of the gate's
 * Wiener gain sig^2 / (sig^2 + noise^2 + 1e-30), sig = C * 128 (s_slow -
 * v_slow), noise = s_fast - sig (gate_coherence_from_fields,
 * concord/packed_b.py:2081-2091); the layer mean of measure_coherence
 * (2094-2106) is out_sum / (N K).  Fixed order: 8192-word blocks, lanes
 * chaining a stride-256 set each, a halving tree; the block totals as 64
 * lane sums (totals l, l + 64, ... ascending) and a halving tree. */
size_t concord_stats_workspace_bytes(int64_t n_watermarks, int64_t n_words);
int concord_watermark_peak(const int32_t* rows, int64_t n_rows, const int32_t* cols, int64_t n_cols,
                           int32_t* out, void* workspace, size_t workspace_bytes, void* stream);
int concord_coherence_sum(const int32_t* packed, int64_t ld_p, int64_t N, int64_t K,
                          float drift_cancel_C, float* out_sum, void* workspace,
                          size_t workspace_bytes, void* stream);

/* Isotropic gradient-noise injection in place on the bf16 weight gradient
 * (notebook/src/prototype_packed_b.py:876-916 and the isotropic branch of
 * 1484-1501): g <- bf16(g + xi * (sigma * ||g|| / max(||xi||, 1e-12))), sigma
 * read from device memory.  xi_e is a standard normal from a counter-based
 * stream keyed by the salt counter's current value: draw e & 3 of
 * Philox4x32-10 block e >> 2, whose words (0, 1) and (2, 3) are two
 * Box-Muller pairs giving cos then sin, with fixed-order log2 / sqrt /
 * sincos.  So the result is reproducible.  The salt counter is read, not advanced.
 * workspace: concord_noise_workspace_bytes(N, K) bytes (block partials, and
 * the draws, 4 B per element, kept between the norm and apply passes); no
 * zeroing needed. */
size_t concord_noise_workspace_bytes(int64_t N, int64_t K);
int concord_iso_noise(uint16_t* grad_w, int64_t ld_g, int64_t N, int64_t K, const float* sigma,
                      const int32_t* salt_counter, void* workspace, size_t workspace_bytes, void* stream);

/* Patch matrix of the packed Conv2d (ConcordConv2dPackedB; reference class
 * concord/packed_b.py:2028-2065, which runs the conv on its cached bf16
 * weight): x is (B, C, H, W) bf16, contiguous; cols is
 * (B * Ho * Wo, C * kh * kw) bf16 with
 *   cols[(b * Ho + ho) * Wo + wo][(c * kh + i) * kw + j]
 *     = x[b][c][ho * sh - ph + i][wo * sw - pw + j]   (0 outside the image),
 * Ho = (H + 2 ph - kh) / sh + 1, Wo likewise: nn.Conv2d's (c, i, j) weight
 * flattening, so the conv's products are the packed linear entries on cols. */
int concord_conv_im2col(const uint16_t* x, int64_t B, int64_t C, int64_t H, int64_t W, int64_t kh, int64_t kw,
                        int64_t sh, int64_t sw, int64_t ph, int64_t pw, uint16_t* cols, void* stream);
/* Its adjoint, the input gradient of the conv from the patch gradient dcols
 * (same layout as cols): dx[b][c][h][w] = bf16(sum over i ascending, then j
 * ascending, of dcols[(b * Ho + ho) * Wo + wo][(c * kh + i) * kw + j]) over
 * the (i, j) with ho * sh = h + ph - i, wo * sw = w + pw - j, 0 <= ho < Ho,
 * 0 <= wo < Wo; fp32 accumulation.  Replaces the conv's input-gradient path
 * of the reference's conv class (cuDNN there).  concord_conv_col2im_fits
 * says whether the window fits the kernel's staged LDS tile (non-zero) for
 * the given kernel size and stride; a window that does not is gathered by
 * an unstaged kernel with the same summation order. */
int concord_conv_col2im(const uint16_t* dcols, int64_t B, int64_t C, int64_t H, int64_t W, int64_t kh, int64_t kw,
                        int64_t sh, int64_t sw, int64_t ph, int64_t pw, uint16_t* dx, void* stream);
int concord_conv_col2im_fits(int64_t kh, int64_t kw, int64_t sh, int64_t sw);

/* Implicit-GEMM convolution: FusedConcordConv2dPackedB's three products
 * (concord/packed_b.py:1889-1941: F.conv2d, conv2d_input and conv2d_weight
 * on the cached bf16 weight, cuDNN there) with the patches gathered inside
 * the GEMM kernels, never written.  Geometry (B, Cin, H, W, Cout, kh, kw,
 * sh, sw, ph, pw) as nn.Conv2d's: Ho = (H + 2 ph - kh) / sh + 1, Wo
 * likewise.  Activations are channels-last (NHWC) bf16: x[B][H][W][Cin],
 * y and dy [B][Ho][Wo][Cout], dx [B][H][W][Cin].  The weight is tap-major,
 * wt[Cout][kh * kw][Cin] (concord_conv_weight_taps); the WGRAD writes its
 * gradient gt in that order and concord_conv_grad_from_taps puts it back in
 * the packed words' (Cin, kh, kw) order.  The products accumulate in fp32
 * and round once to bf16 (split-K partials summed in a fixed order).
 * concord_conv_implicit_ok: non-zero when the kernels take the geometry
 * (Cin and Cout multiples of 64, strides 1 or 2, fewer than 2^24 positions
 * and operands below 2^30 bytes); the three products return CONCORD_EINVAL
 * otherwise.  The workspace (concord_conv_workspace_bytes, zero-initialised
 * once, kept between calls) holds split-K counters and partials. */
int concord_conv_implicit_ok(int64_t B, int64_t Cin, int64_t H, int64_t W, int64_t Cout, int64_t kh, int64_t kw,
                             int64_t sh, int64_t sw, int64_t ph, int64_t pw);
size_t concord_conv_workspace_bytes(int64_t B, int64_t Cin, int64_t H, int64_t W, int64_t Cout, int64_t kh,
                                    int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw);
/* wt[n][t][c] = the forward weight of packed word (n, c * taps + t):
 * bf16(((128 ss + g sf) + 128 vs) 2^(row_exp + col_exp - bias)) in fp32
 * (concord/packed_b.py:1763-1772; g = fast_gain, 1 for the plain decode of
 * 120-170).  taps <= 64. */
int concord_conv_weight_taps(const int32_t* packed, int64_t ld_p, const int8_t* row_exp, const int8_t* col_exp,
                             int64_t Cout, int64_t Cin, int64_t taps, int32_t mantissa_bias, float fast_gain,
                             uint16_t* wt, void* stream);
/* g[n][c * taps + t] = gt[n][t][c] (ld_g >= Cin * taps); taps <= 64. */
int concord_conv_grad_from_taps(const uint16_t* gt, int64_t Cout, int64_t Cin, int64_t taps, uint16_t* g,
                                int64_t ld_g, void* stream);
/* y = conv(x, wt) + bias (bias may be NULL), y[b][ho][wo][n]. */
int concord_conv_fwd(const uint16_t* x, const uint16_t* wt, const uint16_t* bias, uint16_t* y, int64_t B,
                     int64_t Cin, int64_t H, int64_t W, int64_t Cout, int64_t kh, int64_t kw, int64_t sh,
                     int64_t sw, int64_t ph, int64_t pw, void* workspace, size_t workspace_bytes, void* stream);
/* dx = conv2d_input(dy, wt): dx[b][h][w][c] = sum over (ky, kx, n) with
 * ho sh = h + ph - ky, wo sw = w + pw - kx inside the output grid of
 * dy[b][ho][wo][n] wt[n][ky kw + kx][c]. */
int concord_conv_dgrad(const uint16_t* dy, const uint16_t* wt, uint16_t* dx, int64_t B, int64_t Cin, int64_t H,
                       int64_t W, int64_t Cout, int64_t kh, int64_t kw, int64_t sh, int64_t sw, int64_t ph,
                       int64_t pw, void* workspace, size_t workspace_bytes, void* stream);
/* gt = conv2d_weight(x, dy) in tap-major order: gt[n][ky kw + kx][c] =
 * sum over positions (b, ho, wo) of dy[b][ho][wo][n] x[b][ho sh - ph + ky]
 * [wo sw - pw + kx][c] (0 outside the image). */
int concord_conv_wgrad(const uint16_t* dy, const uint16_t* x, uint16_t* gt, int64_t B, int64_t Cin, int64_t H,
                       int64_t W, int64_t Cout, int64_t kh, int64_t kw, int64_t sh, int64_t sw, int64_t ph,
                       int64_t pw, void* workspace, size_t workspace_bytes, void* stream);
/* The conv layer's weight-gradient step of the backward
 * (FusedConcordConv2dPackedB.backward, concord/packed_b.py:1863-2021, with
 * the v-hat EMA of 1281-1303): concord_conv_wgrad into gt, then
 * concord_conv_grad_from_taps into grad_w[Cout][Cin * taps] (ld_gw >=
 * Cin * taps), then concord_vhat_ema on grad_w, with bit-identical results;
 * for 3 x 3 kernels the reorder and the v-hat partials are one pass.  With
 * grad_bias, also the bias gradient sum over positions of dy (concord/
 * packed_b.py:2003-2005), from the dy fragments the product already reads,
 * summed over its partial rows in a fixed order.  workspace:
 * concord_workspace_bytes(Cout, Cin * taps, B * Ho * Wo) bytes (as for
 * concord_wgrad_vhat); gemm_workspace: concord_conv_workspace_bytes. */
int concord_conv_wgrad_vhat(const uint16_t* dy, const uint16_t* x, uint16_t* gt, uint16_t* grad_w, int64_t ld_gw,
                            int64_t B, int64_t Cin, int64_t H, int64_t W, int64_t Cout, int64_t kh, int64_t kw,
                            int64_t sh, int64_t sw, int64_t ph, int64_t pw, double beta2, float* v_row,
                            float* v_col, float* sum_v_inv, int32_t* row_max, int32_t* col_max,
                            int32_t* salt_counter, uint16_t* grad_bias, void* workspace, size_t workspace_bytes,
                            void* gemm_workspace, size_t gemm_workspace_bytes, void* stream);

/* The Sigma_g-shaped draw, the reference's default when its noise is on
 * (notebook/src/prototype_packed_b.py:1489-1500): in place on the bf16
 * gradient g of dy[M,N]^T x[M,K],
 *   n = (eps * dy)^T x - (sum_m eps_m) * (g / M),   eps_m ~ N(0, 1) per token,
 *   g <- bf16(g + n * (sigma * ||g|| / max(||n||, 1e-12))).
 * eps_m is the counter-based normal stream of concord_iso_noise with its own
 * key (second word 0x5369676D) at the salt counter's current value (read,
 * not advanced); the product is this library's WGRAD on bf16(eps_m dy[m,:])
 * with fp32 accumulation.  workspace: concord_sigmag_noise_workspace_bytes(M,
 * N, K) bytes (the scaled dy, the product, reductions, a split-K region),
 * zero-filled once when allocated. */
size_t concord_sigmag_noise_workspace_bytes(int64_t M, int64_t N, int64_t K);
int concord_sigmag_noise(uint16_t* grad_w, int64_t ld_g, const uint16_t* dy, int64_t ld_dy, const uint16_t* x,
                         int64_t ld_x, int64_t M, int64_t N, int64_t K, const float* sigma,
                         const int32_t* salt_counter, void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif
