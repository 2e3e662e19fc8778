// stats.hip -- multi-layer reductions over the packed state: the watermark
// peak that gates rebalance (notebook/src/concord_winner.py:206-262,
// GatedRebalance) and the layer-mean coherence meter
// (concord/packed_b.py:2081-2106, gate_coherence_from_fields /
// measure_coherence).
#include "common.h"

namespace concord {

constexpr int kPeakPerBlock = 256 * 16;   // watermarks per block
constexpr int kCohBlock = 8192;           // words per coherence partial

// per-block max of rows[0, nr) followed by cols[0, nc) (all values >= 0)
__global__ __launch_bounds__(256) void peak_partials_kernel(const int32_t* __restrict__ rows, int64_t nr,
                                                            const int32_t* __restrict__ cols, int64_t nc,
                                                            int32_t* __restrict__ part) {
  __shared__ int32_t s[4];
  const int64_t b0 = (int64_t)blockIdx.x * kPeakPerBlock;
  int32_t m = 0;
#pragma unroll 4
  for (int i = 0; i < kPeakPerBlock / 256; ++i) {
    const int64_t e = b0 + threadIdx.x + 256 * i;
    if (e < nr) m = max(m, rows[e]);
    else if (e - nr < nc) m = max(m, cols[e - nr]);
  }
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) part[blockIdx.x] = max(max(s[0], s[1]), max(s[2], s[3]));
}

__global__ __launch_bounds__(256) void peak_final_kernel(const int32_t* __restrict__ part, int64_t nb,
                                                         int32_t* out) {
  __shared__ int32_t s[4];
  int32_t m = 0;
  for (int64_t b = threadIdx.x; b < nb; b += 256) m = max(m, part[b]);
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) *out = max(max(s[0], s[1]), max(s[2], s[3]));
}

// The gate's Wiener gain of one word, from its integer fields (the
// exponents cancel): sig = C (128 (ss - vs)), noise = sf - sig,
// coh = sig^2 / ((sig^2 + noise^2) + 1e-30)   (concord/packed_b.py:2081-2091)
CONCORD_DEV float word_coherence(int32_t w, float C) {
  const Fields f = unpack(w);
  const float sig = __fmul_rn(C, (float)((f.ss - f.vs) * 128));
  const float noise = __fsub_rn((float)f.sf, sig);
  const float sig2 = __fmul_rn(sig, sig);
  return __fdiv_rn(sig2, __fadd_rn(__fadd_rn(sig2, __fmul_rn(noise, noise)), 1e-30f));
}

// Sum of the coherence over kCohBlock words per block, in a fixed order:
// lane t chains words b0 + t + 256 i (i ascending), then a halving tree over
// the 256 lanes (oracle_coherence_sum restates it).
__global__ __launch_bounds__(256) void coherence_partials_kernel(const int32_t* __restrict__ p, int64_t ld,
                                                                 int64_t N, int64_t K, float C,
                                                                 float* __restrict__ part) {
  __shared__ float s[256];
  const int64_t total = N * K;
  const int64_t b0 = (int64_t)blockIdx.x * kCohBlock;
  // the block's 32 words per lane loaded first, then chained in order
  int32_t w[kCohBlock / 256];
#pragma unroll
  for (int i = 0; i < kCohBlock / 256; ++i) {
    const int64_t e = b0 + threadIdx.x + 256 * i;
    w[i] = e < total ? (ld == K ? p[e] : p[(e / K) * ld + e % K]) : 0;
  }
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < kCohBlock / 256; ++i)
    if (b0 + threadIdx.x + 256 * i < total) acc = __fadd_rn(acc, word_coherence(w[i], C));
  s[threadIdx.x] = acc;
  __syncthreads();
  for (int h = 128; h >= 1; h >>= 1) {
    if (threadIdx.x < h) s[threadIdx.x] = __fadd_rn(s[threadIdx.x], s[threadIdx.x + h]);
    __syncthreads();
  }
  if (threadIdx.x == 0) part[blockIdx.x] = s[0];
}

// the block partials added as 64 lane sums and a tree (one wave, wave_tree_sum)
__global__ __launch_bounds__(64) void coherence_final_kernel(const float* __restrict__ part, int64_t nb,
                                                             float* out) {
  const float s = wave_tree_sum(part, nb, 1);
  if (threadIdx.x == 0) *out = s;
}

}  // namespace concord

using namespace concord;

extern "C" size_t concord_stats_workspace_bytes(int64_t n_watermarks, int64_t n_words) {
  const int64_t a = n_watermarks > 0 ? cdiv(n_watermarks, kPeakPerBlock) * 4 : 0;
  const int64_t b = n_words > 0 ? cdiv(n_words, kCohBlock) * 4 : 0;
  return (size_t)((std::max(a, b) + 255) / 256 * 256 + 256);
}

extern "C" int concord_watermark_peak(const int32_t* rows, int64_t n_rows, const int32_t* cols, int64_t n_cols,
                                      int32_t* out, void* workspace, size_t workspace_bytes, void* stream) {
  CONCORD_CHECK(n_rows >= 0 && n_cols >= 0 && n_rows + n_cols < (1LL << 40), "concord_watermark_peak: bad size");
  CONCORD_CHECK(out && (rows || n_rows == 0) && (cols || n_cols == 0), "concord_watermark_peak: NULL argument");
  const int64_t n = n_rows + n_cols;
  const int64_t nb = n > 0 ? cdiv(n, kPeakPerBlock) : 0;
  if (!workspace || workspace_bytes < concord_stats_workspace_bytes(n, 0)) {
    set_error("concord_watermark_peak: workspace of %zu bytes needed", concord_stats_workspace_bytes(n, 0));
    return CONCORD_EWORKSPACE;
  }
  hipStream_t st = (hipStream_t)stream;
  int32_t* part = (int32_t*)workspace;
  if (nb > 0)
    hipLaunchKernelGGL(peak_partials_kernel, dim3((unsigned)nb), dim3(256), 0, st, rows, n_rows, cols, n_cols,
                       part);
  hipLaunchKernelGGL(peak_final_kernel, dim3(1), dim3(256), 0, st, part, nb, out);
  return launch_status("watermark_peak");
}

extern "C" int concord_coherence_sum(const int32_t* packed, int64_t ld_p, int64_t N, int64_t K,
                                     float drift_cancel_C, float* out_sum, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  CONCORD_CHECK(N >= 0 && K >= 0 && N * K < (1LL << 40), "concord_coherence_sum: bad size");
  CONCORD_CHECK(out_sum && (packed || N * K == 0), "concord_coherence_sum: NULL argument");
  CONCORD_CHECK(ld_p >= K, "concord_coherence_sum: leading dimension < K");
  const int64_t nb = N * K > 0 ? cdiv(N * K, kCohBlock) : 0;
  if (!workspace || workspace_bytes < concord_stats_workspace_bytes(0, N * K)) {
    set_error("concord_coherence_sum: workspace of %zu bytes needed", concord_stats_workspace_bytes(0, N * K));
    return CONCORD_EWORKSPACE;
  }
  hipStream_t st = (hipStream_t)stream;
  float* part = (float*)workspace;
  if (nb > 0)
    hipLaunchKernelGGL(coherence_partials_kernel, dim3((unsigned)nb), dim3(256), 0, st, packed, ld_p, N, K,
                       drift_cancel_C, part);
  hipLaunchKernelGGL(coherence_final_kernel, dim3(1), dim3(64), 0, st, part, nb, out_sum);
  return launch_status("coherence_sum");
}
