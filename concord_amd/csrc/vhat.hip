// vhat.hip -- AdaFactor rank-1 second moment and bias gradient.
//
// concord_vhat_ema:  FusedConcordLinearPackedB.backward, concord/packed_b.py:1281-1303
//                    (zero row/col watermarks, v_row/v_col EMA of grad^2, 1/sum v_row).
// concord_bias_grad: grad_y_flat.sum(0), concord/packed_b.py:1338-1340.
//
// Reduction order: the tile order of vhat_tile.h (also restated by
// oracle_vhat_ema); g2_row[n] = sum of the row partials over column tiles
// ascending, g2_col[k] likewise over row tiles; sum v_row: halving tree per
// block of 256 rows, then the block totals ascending.
#include "common.h"
#include "vhat.h"
#include "vhat_tile.h"
#include "vhat_finalize.h"
#include "workspace.h"

namespace concord {

// One wave per 64 x 64 tile of g, loaded in the MFMA accumulator layout of
// vhat_tile.h (lane 16 q + p: rows 16 x + p, columns 16 y + 4 q .. + 3).
__global__ __launch_bounds__(256) void vhat_partials_kernel(const uint16_t* __restrict__ g,
                                                            int64_t ld, int64_t N, int64_t K,
                                                            float* __restrict__ pr,
                                                            float* __restrict__ pc) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t ntc = cdiv(K, 64), nt = cdiv(N, 64) * ntc;
  const int64_t tile = (int64_t)blockIdx.x * 4 + wave;
  if (tile >= nt) return;
  const int64_t row0 = (tile / ntc) * 64, col0 = (tile % ntc) * 64;
  const int p = lane & 15, q = lane >> 4;
  const bool vec = (ld % 4) == 0 && ((uintptr_t)g % 8) == 0;
  float g2[4][4][4];
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    const int64_t n = row0 + 16 * x + p;
#pragma unroll
    for (int y = 0; y < 4; ++y) {
      const int64_t k = col0 + 16 * y + 4 * q;
      float v[4];
      if (n < N && k + 4 <= K && vec) {
        const uint2 w = *reinterpret_cast<const uint2*>(g + n * ld + k);
        v[0] = __uint_as_float(w.x << 16);
        v[1] = __uint_as_float(w.x & 0xFFFF0000u);
        v[2] = __uint_as_float(w.y << 16);
        v[3] = __uint_as_float(w.y & 0xFFFF0000u);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (n < N && k + e < K) ? bf16_to_f32(g[n * ld + k + e]) : 0.0f;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) g2[x][y][e] = __fmul_rn(v[e], v[e]);
    }
  }
  vhat_tile_partials(g2, lane, row0, col0, N, K, pr, pc);
}

// sum of v[0], v[stride], ..., v[(count - 1) stride] ascending from 0.0f,
// with the loads of 32 terms in flight at a time
CONCORD_DEV float ordered_sum(const float* __restrict__ v, int64_t stride, int64_t count) {
  float s = 0.0f;
  int64_t b = 0;
  for (; b + 32 <= count; b += 32) {
    float a[32];
#pragma unroll
    for (int e = 0; e < 32; ++e) a[e] = v[(b + e) * stride];
#pragma unroll
    for (int e = 0; e < 32; ++e) s = __fadd_rn(s, a[e]);
  }
  if (b < count) {
    float a[32];
#pragma unroll
    for (int e = 0; e < 32; ++e) a[e] = b + e < count ? v[(b + e) * stride] : 0.0f;
#pragma unroll
    for (int e = 0; e < 32; ++e)
      if (b + e < count) s = __fadd_rn(s, a[e]);
  }
  return s;
}

__global__ __launch_bounds__(256) void vhat_finalize_kernel(
    const float* __restrict__ pr, const float* __restrict__ pc, int64_t N, int64_t K, float b2,
    float omb2, float* v_row, float* v_col, int32_t* row_max, int32_t* col_max, float* bsum,
    const float* __restrict__ bpart, int64_t nbp, uint16_t* grad_bias, uint32_t* ticket,
    float* sum_v_inv, int32_t* salt) {
  vhat_finalize_block(blockIdx.x, pr, pc, N, K, b2, omb2, v_row, v_col, row_max, col_max, bsum, bpart, nbp,
                      grad_bias, ticket, sum_v_inv, salt);
}

void vhat_partials_launch(const uint16_t* grad, int64_t ld, int64_t N, int64_t K, float* pr, float* pc,
                          hipStream_t st) {
  const int64_t nt = cdiv(N, 64) * cdiv(K, 64);
  hipLaunchKernelGGL(vhat_partials_kernel, dim3((unsigned)cdiv(nt, 4)), dim3(256), 0, st, grad, ld, N, K,
                     pr, pc);
}

void vhat_finish_launch(const float* pr, const float* pc, float* bsum, uint32_t* ticket, int64_t N, int64_t K,
                        double beta2, float* v_row, float* v_col, float* sum_v_inv, int32_t* row_max,
                        int32_t* col_max, int32_t* salt, hipStream_t st, const float* bpart, int64_t nbp,
                        uint16_t* grad_bias) {
  const float b2 = (float)beta2;
  const float omb2 = (float)(1.0 - beta2);
  hipLaunchKernelGGL(vhat_finalize_kernel, dim3((unsigned)vhat_finalize_blocks(N, K, grad_bias != nullptr)),
                     dim3(256), 0, st, pr, pc,
                     N, K, b2, omb2, v_row, v_col, row_max, col_max, bsum, bpart, nbp, grad_bias, ticket,
                     sum_v_inv, salt);
}

// bias gradient: a thread sums 4 adjacent columns over a slab of 64 rows
// (rows ascending; 8-byte loads, a wave reads 512 contiguous bytes per row),
// then the slabs are combined in order.
constexpr int BG_ROWS = 64;

__global__ __launch_bounds__(256) void colsum_partials_kernel(const uint16_t* __restrict__ dy,
                                                              int64_t ld, int64_t M, int64_t N,
                                                              float* __restrict__ part) {
  const int64_t n = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (n >= N) return;
  const bool vec = (n + 4 <= N) && (ld % 4 == 0) && (((uintptr_t)dy % 8) == 0);
  // slabs blockIdx.y, blockIdx.y + gridDim.y, ... (grid.y <= kMaxGridY)
  for (int64_t slab = blockIdx.y; slab * BG_ROWS < M; slab += gridDim.y) {
  const int64_t m0 = slab * BG_ROWS;
  const int64_t m1 = min(M, m0 + BG_ROWS);
  float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (vec) {
    int64_t m = m0;
    for (; m + 8 <= m1; m += 8) {
      uint2 w[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) w[e] = *reinterpret_cast<const uint2*>(dy + (m + e) * ld + n);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        s[0] = __fadd_rn(s[0], __uint_as_float(w[e].x << 16));
        s[1] = __fadd_rn(s[1], __uint_as_float(w[e].x & 0xFFFF0000u));
        s[2] = __fadd_rn(s[2], __uint_as_float(w[e].y << 16));
        s[3] = __fadd_rn(s[3], __uint_as_float(w[e].y & 0xFFFF0000u));
      }
    }
    for (; m < m1; ++m) {
      const uint2 w = *reinterpret_cast<const uint2*>(dy + m * ld + n);
      s[0] = __fadd_rn(s[0], __uint_as_float(w.x << 16));
      s[1] = __fadd_rn(s[1], __uint_as_float(w.x & 0xFFFF0000u));
      s[2] = __fadd_rn(s[2], __uint_as_float(w.y << 16));
      s[3] = __fadd_rn(s[3], __uint_as_float(w.y & 0xFFFF0000u));
    }
  } else {
    for (int64_t m = m0; m < m1; ++m)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (n + c < N) s[c] = __fadd_rn(s[c], bf16_to_f32(dy[m * ld + n + c]));
  }
#pragma unroll
  for (int c = 0; c < 4; ++c)
    if (n + c < N) part[slab * N + n + c] = s[c];
  }
}

__global__ __launch_bounds__(256) void colsum_finalize_kernel(const float* __restrict__ part,
                                                              int64_t slabs, int64_t N,
                                                              uint16_t* out) {
  const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (n >= N) return;
  const float s = ordered_sum(part + n, N, slabs);
  out[n] = (uint16_t)(pack_bf16x2(s, 0.0f) & 0xFFFFu);
}

void bias_grad_launch(const uint16_t* dy, int64_t ld, int64_t M, int64_t N, uint16_t* grad_bias, float* part,
                      hipStream_t st) {
  const int64_t slabs = cdiv(M, BG_ROWS);  // 0 when M == 0: the combine writes zeros
  if (slabs > 0)
    hipLaunchKernelGGL(colsum_partials_kernel, dim3((unsigned)cdiv(N, 1024), grid_y(slabs)), dim3(256), 0,
                       st, dy, ld, M, N, part);
  hipLaunchKernelGGL(colsum_finalize_kernel, dim3((unsigned)cdiv(N, 256)), dim3(256), 0, st, part, slabs, N,
                     grad_bias);
}

__global__ __launch_bounds__(256) void fill_zero_bf16_kernel(uint16_t* p, int64_t ld, int64_t rows, int64_t cols) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= cols) return;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) p[r * ld + c] = 0;
}

void fill_zero_bf16_launch(uint16_t* p, int64_t ld, int64_t rows, int64_t cols, hipStream_t st) {
  if (rows <= 0 || cols <= 0) return;
  hipLaunchKernelGGL(fill_zero_bf16_kernel, dim3((unsigned)cdiv(cols, 256), grid_y(rows)), dim3(256), 0, st, p,
                     ld, rows, cols);
}

void wgrad_vhat_empty_batch(uint16_t* grad_w, int64_t ld_gw, int64_t N, int64_t K, double beta2, float* v_row,
                            float* v_col, float* sum_v_inv, int32_t* row_max, int32_t* col_max,
                            int32_t* salt_counter, uint16_t* grad_bias, void* workspace, hipStream_t st) {
  const Workspace ws = workspace_layout(N, K, 0);
  const VhatScratch v = vhat_scratch(N, K);
  float* pr = (float*)((char*)workspace + ws.scratch);
  float* pc = pr + v.pr;
  float* bsum = pc + v.pc;
  fill_zero_bf16_launch(grad_w, ld_gw, N, K, st);
  vhat_partials_launch(grad_w, ld_gw, N, K, pr, pc, st);
  // no bias partial rows: the finalize writes grad_bias = bf16(0)
  vhat_finish_launch(pr, pc, bsum, (uint32_t*)((char*)workspace + ws.vhat_ticket), N, K, beta2, v_row, v_col,
                     sum_v_inv, row_max, col_max, salt_counter, st, nullptr, 0, grad_bias);
}

}  // namespace concord

using namespace concord;

extern "C" int concord_vhat_ema(const uint16_t* grad, int64_t ld_g, int64_t N, int64_t K,
                                double beta2, float* v_row, float* v_col, float* sum_v_inv,
                                int32_t* row_max, int32_t* col_max, int32_t* salt_counter,
                                void* workspace, size_t workspace_bytes, void* stream) {
  CONCORD_CHECK(N > 0 && K > 0 && N < (1LL << 31) && K < (1LL << 31),
                "concord_vhat_ema: bad size N=%lld K=%lld", (long long)N, (long long)K);
  CONCORD_CHECK(grad && v_row && v_col && sum_v_inv, "concord_vhat_ema: NULL argument");
  CONCORD_CHECK(ld_g >= K, "concord_vhat_ema: leading dimension < K");
  const Workspace ws = workspace_layout(N, K, 0);
  if (!workspace || workspace_bytes < ws.total) {
    set_error("concord_vhat_ema: workspace of %zu bytes needed", ws.total);
    return CONCORD_EWORKSPACE;
  }
  const VhatScratch v = vhat_scratch(N, K);
  float* pr = (float*)((char*)workspace + ws.scratch);
  float* pc = pr + v.pr;
  float* bsum = pc + v.pc;
  hipStream_t st = (hipStream_t)stream;
  vhat_partials_launch(grad, ld_g, N, K, pr, pc, st);
  vhat_finish_launch(pr, pc, bsum, (uint32_t*)((char*)workspace + ws.vhat_ticket), N, K, beta2, v_row, v_col,
                     sum_v_inv, row_max, col_max, salt_counter, st);
  return launch_status("vhat_ema");
}

extern "C" int concord_bias_grad(const uint16_t* dy, int64_t ld_dy, int64_t M, int64_t N,
                                 uint16_t* grad_bias, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  CONCORD_CHECK(M >= 0 && N > 0, "concord_bias_grad: bad size");
  CONCORD_CHECK(dy && grad_bias, "concord_bias_grad: NULL argument");
  CONCORD_CHECK(ld_dy >= N, "concord_bias_grad: leading dimension < N");
  const Workspace ws = workspace_layout(N, 1, M);
  if (!workspace || workspace_bytes < ws.total) {
    set_error("concord_bias_grad: workspace of %zu bytes needed", ws.total);
    return CONCORD_EWORKSPACE;
  }
  bias_grad_launch(dy, ld_dy, M, N, grad_bias, (float*)((char*)workspace + ws.scratch), (hipStream_t)stream);
  return launch_status("bias_grad");
}
