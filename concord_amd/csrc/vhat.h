// vhat.h -- launchers of the v-hat kernels shared by concord_vhat_ema and the
// wgrad entry that forms the partials in its epilogue.
#pragma once
#include "common.h"

namespace concord {

// row / column partial sums of g^2 (vhat_tile.h order) of a bf16 gradient
void vhat_partials_launch(const uint16_t* grad, int64_t ld, int64_t N, int64_t K, float* pr, float* pc,
                          hipStream_t st);
// EMA of v_row / v_col from the partials, watermark zeroing, 1 / sum v_row,
// salt advance (row_max, col_max, salt may be NULL)
void vhat_finish_launch(const float* pr, const float* pc, float* bsum, int64_t N, int64_t K, double beta2,
                        float* v_row, float* v_col, float* sum_v_inv, int32_t* row_max, int32_t* col_max,
                        int32_t* salt, hipStream_t st);

}  // namespace concord
