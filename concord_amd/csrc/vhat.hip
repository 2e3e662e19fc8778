// vhat.hip -- AdaFactor rank-1 second moment and bias gradient.
//
// concord_vhat_ema:  FusedConcordLinearPackedB.backward, concord/packed_b.py:1281-1303
//                    (zero row/col watermarks, v_row/v_col EMA of grad^2, 1/sum v_row).
// concord_bias_grad: grad_y_flat.sum(0), concord/packed_b.py:1338-1340.
//
// Reduction order (fixed, also restated by oracle_vhat_ema):
//   P_r[c][n] = sum_{k in [64c, 64c+64)} g^2 ascending; P_c[r][k] = sum_{n in
//   [128r, 128r+128)} g^2 ascending; g2_row[n] = sum_c P_r[c][n] ascending c;
//   g2_col[k] = sum_r P_c[r][k] ascending r; sum v_row by 256 strided lanes
//   followed by the halving tree.
#include "common.h"
#include "workspace.h"

namespace concord {

constexpr int VH_ROWS = 128;   // rows per column partial
constexpr int VH_SUB = 32;     // rows staged in LDS at a time

// One block: a slab of 128 rows x 256 columns, staged 32 rows at a time as
// g^2 in LDS (257-float row stride: both walks are bank-conflict free).
__global__ __launch_bounds__(256) void vhat_partials_kernel(const uint16_t* __restrict__ g,
                                                            int64_t ld, int64_t N, int64_t K,
                                                            float* __restrict__ pr,
                                                            float* __restrict__ pc) {
  __shared__ float t[VH_SUB * 257];
  const int64_t kb = (int64_t)blockIdx.x * 256, nb0 = (int64_t)blockIdx.y * VH_ROWS;
  const int tid = threadIdx.x;
  const int64_t nc = cdiv(K, 64);
  const bool vec = (ld % 8) == 0;
  float colsum = 0.0f;
  for (int sub = 0; sub < VH_ROWS / VH_SUB; ++sub) {
    const int64_t nb = nb0 + sub * VH_SUB;
    if (nb >= N) break;
    // load: thread -> (row = tid / 32 + 8 i, 8 columns at (tid % 32) * 8)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = tid / 32 + 8 * i, c = (tid % 32) * 8;
      const int64_t n = nb + r, k = kb + c;
      float v[8];
      if (n < N && k + 8 <= K && vec) {
        const uint4 q = *reinterpret_cast<const uint4*>(g + n * ld + k);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[2 * j] = __uint_as_float(w[j] << 16);
          v[2 * j + 1] = __uint_as_float(w[j] & 0xFFFF0000u);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          v[j] = (n < N && k + j < K) ? bf16_to_f32(g[n * ld + k + j]) : 0.0f;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) t[r * 257 + c + j] = __fmul_rn(v[j], v[j]);
    }
    __syncthreads();
    if (tid < 128) {
      const int r = tid % 32, ch = tid / 32;
      const int64_t n = nb + r, cg = (int64_t)blockIdx.x * 4 + ch;
      if (n < N && cg < nc) {
        float s = 0.0f;
        const float* row = t + r * 257 + ch * 64;
#pragma unroll 16
        for (int j = 0; j < 64; ++j) s = __fadd_rn(s, row[j]);
        pr[cg * N + n] = s;
      }
    }
#pragma unroll 8
    for (int r = 0; r < VH_SUB; ++r) colsum = __fadd_rn(colsum, t[r * 257 + tid]);
    __syncthreads();
  }
  const int64_t k = kb + tid;
  if (k < K) pc[(int64_t)blockIdx.y * K + k] = colsum;
}

// Row/column EMA and watermark zeroing; the last block to finish computes
// 1/sum(v_row), advances the salt and re-arms the counter.
__global__ __launch_bounds__(256) void vhat_finalize_kernel(
    const float* __restrict__ pr, const float* __restrict__ pc, int64_t N, int64_t K, float b2,
    float omb2, float* v_row, float* v_col, float* sum_v_inv, int32_t* row_max, int32_t* col_max,
    int32_t* salt, uint32_t* counter) {
  __shared__ float s_part[256];
  __shared__ bool s_last;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t nc = cdiv(K, 64), nr = cdiv(N, VH_ROWS);
  if (i < N) {
    float s = 0.0f;
    int64_t c = 0;
    for (; c + 4 <= nc; c += 4) {   // loads issued ahead, adds in ascending c
      const float a0 = pr[c * N + i], a1 = pr[(c + 1) * N + i];
      const float a2 = pr[(c + 2) * N + i], a3 = pr[(c + 3) * N + i];
      s = __fadd_rn(__fadd_rn(__fadd_rn(__fadd_rn(s, a0), a1), a2), a3);
    }
    for (; c < nc; ++c) s = __fadd_rn(s, pr[c * N + i]);
    v_row[i] = __fadd_rn(__fmul_rn(v_row[i], b2), __fmul_rn(omb2, s));
    if (row_max) row_max[i] = 0;
  } else if (i < N + K) {
    const int64_t k = i - N;
    float s = 0.0f;
    int64_t r = 0;
    for (; r + 4 <= nr; r += 4) {
      const float a0 = pc[r * K + k], a1 = pc[(r + 1) * K + k];
      const float a2 = pc[(r + 2) * K + k], a3 = pc[(r + 3) * K + k];
      s = __fadd_rn(__fadd_rn(__fadd_rn(__fadd_rn(s, a0), a1), a2), a3);
    }
    for (; r < nr; ++r) s = __fadd_rn(s, pc[r * K + k]);
    v_col[k] = __fadd_rn(__fmul_rn(v_col[k], b2), __fmul_rn(omb2, s));
    if (col_max) col_max[k] = 0;
  }
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) s_last = atomicAdd(counter, 1u) == gridDim.x - 1;
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  float s = 0.0f;
  for (int64_t n = threadIdx.x; n < N; n += 256) s = __fadd_rn(s, v_row[n]);
  s_part[threadIdx.x] = s;
  __syncthreads();
  for (int h = 128; h >= 1; h >>= 1) {
    if (threadIdx.x < h) s_part[threadIdx.x] = __fadd_rn(s_part[threadIdx.x], s_part[threadIdx.x + h]);
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    *sum_v_inv = __fdiv_rn(1.0f, fmaxf(s_part[0], 1e-30f));
    if (salt) salt[0] = wadd(salt[0], 1);
    *counter = 0u;
  }
}

// bias gradient: a thread sums two adjacent columns over a 256-row slab
// (rows ascending, 8 loads in flight), then the slabs are combined in order.
__global__ __launch_bounds__(256) void colsum_partials_kernel(const uint16_t* __restrict__ dy,
                                                              int64_t ld, int64_t M, int64_t N,
                                                              float* __restrict__ part) {
  const int64_t n = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 2;
  if (n >= N) return;
  const int64_t m0 = (int64_t)blockIdx.y * 256;
  const int64_t m1 = min(M, m0 + 256);
  const bool pair = (n + 1 < N) && (ld % 2 == 0);
  float s0 = 0.0f, s1 = 0.0f;
  int64_t m = m0;
  if (pair) {
    for (; m + 8 <= m1; m += 8) {
      uint32_t w[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) w[e] = *reinterpret_cast<const uint32_t*>(dy + (m + e) * ld + n);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        s0 = __fadd_rn(s0, __uint_as_float(w[e] << 16));
        s1 = __fadd_rn(s1, __uint_as_float(w[e] & 0xFFFF0000u));
      }
    }
  }
  for (; m < m1; ++m) {
    s0 = __fadd_rn(s0, bf16_to_f32(dy[m * ld + n]));
    if (n + 1 < N) s1 = __fadd_rn(s1, bf16_to_f32(dy[m * ld + n + 1]));
  }
  part[(int64_t)blockIdx.y * N + n] = s0;
  if (n + 1 < N) part[(int64_t)blockIdx.y * N + n + 1] = s1;
}

__global__ __launch_bounds__(256) void colsum_finalize_kernel(const float* __restrict__ part,
                                                              int64_t slabs, int64_t N,
                                                              uint16_t* out) {
  const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (n >= N) return;
  float s = 0.0f;
  for (int64_t b = 0; b < slabs; ++b) s = __fadd_rn(s, part[b * N + n]);
  out[n] = (uint16_t)(pack_bf16x2(s, 0.0f) & 0xFFFFu);
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
  char* base = (char*)workspace;
  float* pr = (float*)(base + ws.scratch);
  float* pc = pr + cdiv(K, 64) * N;
  uint32_t* counter = (uint32_t*)(base + ws.vhat_counter);
  hipStream_t st = (hipStream_t)stream;
  const float b2 = (float)beta2;
  const float omb2 = (float)(1.0 - beta2);
  hipLaunchKernelGGL(vhat_partials_kernel,
                     dim3((unsigned)cdiv(K, 256), (unsigned)cdiv(N, VH_ROWS)), dim3(256), 0, st,
                     grad, ld_g, N, K, pr, pc);
  hipLaunchKernelGGL(vhat_finalize_kernel, dim3((unsigned)cdiv(N + K, 256)), dim3(256), 0, st, pr,
                     pc, N, K, b2, omb2, v_row, v_col, sum_v_inv, row_max, col_max, salt_counter,
                     counter);
  return launch_status("vhat_ema");
}

extern "C" int concord_bias_grad(const uint16_t* dy, int64_t ld_dy, int64_t M, int64_t N,
                                 uint16_t* grad_bias, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  CONCORD_CHECK(M >= 0 && N > 0, "concord_bias_grad: bad size");
  CONCORD_CHECK(dy && grad_bias, "concord_bias_grad: NULL argument");
  CONCORD_CHECK(ld_dy >= N, "concord_bias_grad: leading dimension < N");
  const int64_t slabs = cdiv(M, 256);  // 0 when M == 0: the combine writes zeros
  const Workspace ws = workspace_layout(N, 1, M);
  if (!workspace || workspace_bytes < ws.total) {
    set_error("concord_bias_grad: workspace of %zu bytes needed", ws.total);
    return CONCORD_EWORKSPACE;
  }
  float* part = (float*)((char*)workspace + ws.scratch);
  hipStream_t st = (hipStream_t)stream;
  if (slabs > 0)
    hipLaunchKernelGGL(colsum_partials_kernel, dim3((unsigned)cdiv(N, 512), (unsigned)slabs),
                       dim3(256), 0, st, dy, ld_dy, M, N, part);
  hipLaunchKernelGGL(colsum_finalize_kernel, dim3((unsigned)cdiv(N, 256)), dim3(256), 0, st, part,
                     slabs, N, grad_bias);
  return launch_status("bias_grad");
}
