// noise.hip -- isotropic gradient-noise injection into the bf16 weight
// gradient, in the units of its own norm:
//   grad_W <- bf16(g + xi * (sigma * ||g|| / max(||xi||, 1e-12))),  xi ~ N(0, 1)
// (notebook/src/prototype_packed_b.py:876-916 and the isotropic branch of
// 1484-1501; sigma is a device scalar so a captured graph sees schedule
// changes).  xi is normal_draw(salt, element index): counter-based, so the
// three passes regenerate the same draws instead of storing them.
#include "common.h"

namespace concord {

constexpr int kNoiseBlock = 8192;   // elements per partial

// sums of g^2 and xi^2 over kNoiseBlock elements: lane t chains elements
// b0 + t + 256 i (i ascending), then a halving tree over the 256 lanes
__global__ __launch_bounds__(256) void noise_partials_kernel(const uint16_t* __restrict__ g, int64_t ld,
                                                             int64_t N, int64_t K, const int32_t* salt,
                                                             float* __restrict__ part) {
  __shared__ float sg[256], sx[256];
  const int64_t total = N * K;
  const int64_t b0 = (int64_t)blockIdx.x * kNoiseBlock;
  const int32_t seed = *salt;
  float ag = 0.0f, ax = 0.0f;
  for (int i = 0; i < kNoiseBlock / 256; ++i) {
    const int64_t e = b0 + threadIdx.x + 256 * i;
    if (e < total) {
      const float v = bf16_to_f32(g[(e / K) * ld + e % K]);
      const float z = normal_draw(seed, (uint32_t)e);
      ag = __fadd_rn(ag, __fmul_rn(v, v));
      ax = __fadd_rn(ax, __fmul_rn(z, z));
    }
  }
  sg[threadIdx.x] = ag;
  sx[threadIdx.x] = ax;
  __syncthreads();
  for (int h = 128; h >= 1; h >>= 1) {
    if (threadIdx.x < h) {
      sg[threadIdx.x] = __fadd_rn(sg[threadIdx.x], sg[threadIdx.x + h]);
      sx[threadIdx.x] = __fadd_rn(sx[threadIdx.x], sx[threadIdx.x + h]);
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    part[2 * blockIdx.x] = sg[0];
    part[2 * blockIdx.x + 1] = sx[0];
  }
}

// scale = (sigma * sqrt(sum g^2)) / max(sqrt(sum xi^2), 1e-12), partials
// chained in ascending order
__global__ __launch_bounds__(64) void noise_scale_kernel(const float* __restrict__ part, int64_t nb,
                                                         const float* sigma, float* scale) {
  const int lane = threadIdx.x;
  float sg = 0.0f, sx = 0.0f;
  for (int64_t c0 = 0; c0 < nb; c0 += 32) {
    const float v = c0 + (lane >> 1) < nb ? part[2 * c0 + lane] : 0.0f;
    const int cnt = (int)min((int64_t)32, nb - c0);
    for (int j = 0; j < cnt; ++j) {
      sg = __fadd_rn(sg, lane_value(v, 2 * j));
      sx = __fadd_rn(sx, lane_value(v, 2 * j + 1));
    }
  }
  if (lane == 0) {
    const float ng = sqrt_rn(sg);
    const float nx = fmaxf(sqrt_rn(sx), 1e-12f);
    *scale = __fdiv_rn(__fmul_rn(*sigma, ng), nx);
  }
}

__global__ __launch_bounds__(256) void noise_apply_kernel(uint16_t* __restrict__ g, int64_t ld, int64_t N,
                                                          int64_t K, const int32_t* salt, const float* scale) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= N * K) return;
  const int32_t seed = *salt;
  const float s = *scale;
  uint16_t* p = g + (e / K) * ld + e % K;
  const float v = __fadd_rn(bf16_to_f32(*p), __fmul_rn(normal_draw(seed, (uint32_t)e), s));
  *p = (uint16_t)(pack_bf16x2(v, 0.0f) & 0xFFFFu);
}

}  // namespace concord

using namespace concord;

extern "C" size_t concord_noise_workspace_bytes(int64_t N, int64_t K) {
  const int64_t nb = N * K > 0 ? cdiv(N * K, kNoiseBlock) : 0;
  return (size_t)((2 * nb * 4 + 255) / 256 * 256 + 256);
}

extern "C" int concord_iso_noise(uint16_t* grad_w, int64_t ld_g, int64_t N, int64_t K, const float* sigma,
                                 const int32_t* salt_counter, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  CONCORD_CHECK(N >= 0 && K >= 0 && N * K < (1LL << 32), "concord_iso_noise: bad size");
  if (N == 0 || K == 0) return CONCORD_OK;
  CONCORD_CHECK(grad_w && sigma && salt_counter, "concord_iso_noise: NULL argument");
  CONCORD_CHECK(ld_g >= K, "concord_iso_noise: leading dimension < K");
  if (!workspace || workspace_bytes < concord_noise_workspace_bytes(N, K)) {
    set_error("concord_iso_noise: workspace of %zu bytes needed", concord_noise_workspace_bytes(N, K));
    return CONCORD_EWORKSPACE;
  }
  const int64_t nb = cdiv(N * K, kNoiseBlock);
  float* part = (float*)workspace;
  float* scale = (float*)((char*)workspace + concord_noise_workspace_bytes(N, K) - 256);
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(noise_partials_kernel, dim3((unsigned)nb), dim3(256), 0, st, grad_w, ld_g, N, K,
                     salt_counter, part);
  hipLaunchKernelGGL(noise_scale_kernel, dim3(1), dim3(64), 0, st, part, nb, sigma, scale);
  hipLaunchKernelGGL(noise_apply_kernel, dim3((unsigned)cdiv(N * K, 256)), dim3(256), 0, st, grad_w, ld_g, N,
                     K, salt_counter, scale);
  return launch_status("iso_noise");
}
