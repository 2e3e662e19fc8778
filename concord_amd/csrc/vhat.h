// vhat.h -- launchers of the v-hat kernels shared by concord_vhat_ema and the
// wgrad entry that forms the partials in its epilogue.
#pragma once
#include "common.h"

namespace concord {

// row / column partial sums of g^2 (vhat_tile.h order) of a bf16 gradient
void vhat_partials_launch(const uint16_t* grad, int64_t ld, int64_t N, int64_t K, float* pr, float* pc,
                          hipStream_t st);
// EMA of v_row / v_col from the partials, watermark zeroing, 1 / sum v_row,
// salt advance (row_max, col_max, salt may be NULL).  sum_v_inv == NULL:
// bsum[cdiv(N, 256)] is left holding the 256-row totals of v_row, and the
// update that follows forms 1 / sum v_row from them (apply_adamw_fast_bsum)
// bpart / nbp / grad_bias (optional): grad_bias[n] = bf16(sum over b < nbp
// ascending of bpart[b][n])
// ticket: a zero-initialised counter the call leaves at zero again
void vhat_finish_launch(const float* pr, const float* pc, float* bsum, uint32_t* ticket, int64_t N, int64_t K,
                        double beta2, float* v_row, float* v_col, float* sum_v_inv, int32_t* row_max,
                        int32_t* col_max, int32_t* salt, hipStream_t st, const float* bpart = nullptr,
                        int64_t nbp = 0, uint16_t* grad_bias = nullptr);

// grad_bias[N] = bf16(sum_m dy[m][n]) (fp32, 64-row slabs, slabs ascending);
// part: cdiv(M, 64) * N floats of scratch
void bias_grad_launch(const uint16_t* dy, int64_t ld, int64_t M, int64_t N, uint16_t* grad_bias, float* part,
                      hipStream_t st);

// p[r][c] = 0 for r < rows, c < cols (row stride ld elements); a kernel, not
// hipMemsetAsync, so that a captured graph replays it correctly
void fill_zero_bf16_launch(uint16_t* p, int64_t ld, int64_t rows, int64_t cols, hipStream_t st);

// the weight gradient of an empty batch (M = 0): grad_w = 0, then the v-hat
// EMA of that zero gradient (the v_row / v_col decay, watermark zeroing, salt
// advance) and a zero bias gradient, as the product path would give them
void wgrad_vhat_empty_batch(uint16_t* grad_w, int64_t ld_gw, int64_t N, int64_t K, double beta2, float* v_row,
                            float* v_col, float* sum_v_inv, int32_t* row_max, int32_t* col_max,
                            int32_t* salt_counter, uint16_t* grad_bias, void* workspace, hipStream_t st);

}  // namespace concord
