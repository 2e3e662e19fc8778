// noise.hip -- isotropic gradient-noise injection into the bf16 weight
// gradient, in the units of its own norm:
//   grad_W <- bf16(g + xi * (sigma * ||g|| / max(||xi||, 1e-12))),  xi ~ N(0, 1)
// (notebook/src/prototype_packed_b.py:876-916 and the isotropic branch of
// 1484-1501; sigma is a device scalar so a captured graph sees schedule
// changes).  xi is counter-based: element e takes draw e & 3 of the Philox
// block e >> 2 of normal_draw4(salt, .).  The first pass draws it and keeps
// it (fp32, in the workspace) for the apply pass.
//
// Element e of an N x K gradient with row stride ld sits at (e / K) * ld + e % K;
// with ld == K that is e itself (no division).  A thread takes the four
// elements of one Philox block; when K and ld are multiples of 4 they share a
// row and move as one 8-byte access.
#include "common.h"
#include "gemm.h"

namespace concord {

CONCORD_DEV int64_t elem_off(int64_t e, int64_t K, int64_t ld) { return ld == K ? e : (e / K) * ld + e % K; }

constexpr int kNoiseBlock = 8192;   // elements per partial

// sums of g^2 and xi^2 over kNoiseBlock elements: lane t chains the quads
// q = b0 / 4 + t + 256 i (i ascending), elements 4q .. 4q + 3 in turn, then a
// halving tree over the 256 lanes
__global__ __launch_bounds__(256) void noise_partials_kernel(const uint16_t* __restrict__ g, int64_t ld,
                                                             int64_t N, int64_t K, const int32_t* salt,
                                                             float* __restrict__ part, float* __restrict__ xi) {
  __shared__ float sg[256], sx[256];
  const int64_t total = N * K;
  const int64_t b0 = (int64_t)blockIdx.x * kNoiseBlock;
  const int32_t seed = *salt;
  const bool vg = (K % 4) == 0 && (ld % 4) == 0 && ((uintptr_t)g % 8) == 0;
  const bool vx = ((uintptr_t)xi % 16) == 0;
  float ag = 0.0f, ax = 0.0f;
  for (int i = 0; i < kNoiseBlock / 1024; ++i) {
    const int64_t e0 = b0 + 4 * (threadIdx.x + 256 * i);
    if (e0 < total) {
      float z[4], v[4];
      normal_draw4(seed, (uint32_t)(e0 >> 2), z);
      const bool full = e0 + 4 <= total;
      if (full && vg) {
        const uint2 w = *reinterpret_cast<const uint2*>(g + elem_off(e0, K, ld));
        v[0] = __uint_as_float(w.x << 16);
        v[1] = __uint_as_float(w.x & 0xFFFF0000u);
        v[2] = __uint_as_float(w.y << 16);
        v[3] = __uint_as_float(w.y & 0xFFFF0000u);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = e0 + r < total ? bf16_to_f32(g[elem_off(e0 + r, K, ld)]) : 0.0f;
      }
      if (full && vx) {
        *reinterpret_cast<float4*>(xi + e0) = make_float4(z[0], z[1], z[2], z[3]);
      } else {
        for (int r = 0; r < 4 && e0 + r < total; ++r) xi[e0 + r] = z[r];
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (e0 + r < total) {
          ag = __fadd_rn(ag, __fmul_rn(v[r], v[r]));
          ax = __fadd_rn(ax, __fmul_rn(z[r], z[r]));
        }
      }
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

// scale = (sigma * sqrt(sum g^2)) / max(sqrt(sum xi^2), 1e-12), the block
// partials of each sum added as 64 lane sums and a tree (wave_tree_sum2)
__global__ __launch_bounds__(64) void noise_scale_kernel(const float* __restrict__ part, int64_t nb,
                                                         const float* sigma, float* scale) {
  const int lane = threadIdx.x;
  float sg, sx;
  wave_tree_sum2(part, nb, &sg, &sx);
  if (lane == 0) {
    const float ng = sqrt_rn(sg);
    const float nx = fmaxf(sqrt_rn(sx), 1e-12f);
    *scale = __fdiv_rn(__fmul_rn(*sigma, ng), nx);
  }
}

__global__ __launch_bounds__(256) void noise_apply_kernel(uint16_t* __restrict__ g, int64_t ld, int64_t N,
                                                          int64_t K, const float* __restrict__ xi,
                                                          const float* scale) {
  const int64_t total = N * K;
  const int64_t e0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (e0 >= total) return;
  const float s = *scale;
  if (e0 + 4 <= total && (K % 4) == 0 && (ld % 4) == 0 && ((uintptr_t)g % 8) == 0 && ((uintptr_t)xi % 16) == 0) {
    uint2* p = reinterpret_cast<uint2*>(g + elem_off(e0, K, ld));
    const uint2 w = *p;
    const float4 z = *reinterpret_cast<const float4*>(xi + e0);
    const float v0 = __fadd_rn(__uint_as_float(w.x << 16), __fmul_rn(z.x, s));
    const float v1 = __fadd_rn(__uint_as_float(w.x & 0xFFFF0000u), __fmul_rn(z.y, s));
    const float v2 = __fadd_rn(__uint_as_float(w.y << 16), __fmul_rn(z.z, s));
    const float v3 = __fadd_rn(__uint_as_float(w.y & 0xFFFF0000u), __fmul_rn(z.w, s));
    *p = make_uint2(pack_bf16x2(v0, v1), pack_bf16x2(v2, v3));
  } else {
    for (int64_t e = e0; e < e0 + 4 && e < total; ++e) {
      uint16_t* p = g + elem_off(e, K, ld);
      const float v = __fadd_rn(bf16_to_f32(*p), __fmul_rn(xi[e], s));
      *p = (uint16_t)(pack_bf16x2(v, 0.0f) & 0xFFFFu);
    }
  }
}

// ---- the Sigma_g-shaped draw (prototype_packed_b.py:1489-1496) ---------------
// noise = (eps * dy)^T x - (sum eps) * (g / M), eps_m = normal_draw(salt, m,
// kNoiseTagToken): a draw whose covariance is the empirical per-token
// gradient covariance, centred.  The product runs on the WGRAD kernels (bf16
// operands, fp32 accumulation); everything around it is elementwise or a
// fixed-order reduction.

// dyt[m][n] = bf16(eps_m * dy[m][n]), eps as drawn by token_sum_partials_kernel.
// A thread takes 8 consecutive columns (16-byte accesses when the rows allow).
__global__ __launch_bounds__(256) void token_scale_kernel(const uint16_t* __restrict__ dy, int64_t ld, int64_t M,
                                                          int64_t N, const float* __restrict__ eps,
                                                          uint16_t* __restrict__ out) {
  const int64_t n = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (n >= N) return;
  const bool vec = n + 8 <= N && (ld % 8) == 0 && (N % 8) == 0 && ((uintptr_t)dy % 16) == 0 &&
                   ((uintptr_t)out % 16) == 0;
  // rows strided by the grid's y extent (capped at the y-dimension limit)
  for (int64_t m = blockIdx.y; m < M; m += gridDim.y) {
    const float e = eps[m];
    if (vec) {
      const uint4 d = *reinterpret_cast<const uint4*>(dy + m * ld + n);
      const uint32_t dw[4] = {d.x, d.y, d.z, d.w};
      uint32_t o[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        o[q] = pack_bf16x2(__fmul_rn(e, __uint_as_float(dw[q] << 16)),
                           __fmul_rn(e, __uint_as_float(dw[q] & 0xFFFF0000u)));
      *reinterpret_cast<uint4*>(out + m * N + n) = make_uint4(o[0], o[1], o[2], o[3]);
    } else {
      for (int64_t c = n; c < n + 8 && c < N; ++c)
        out[m * N + c] = (uint16_t)(pack_bf16x2(__fmul_rn(e, bf16_to_f32(dy[m * ld + c])), 0.0f) & 0xFFFFu);
    }
  }
}

// sum of eps_0 .. eps_{M-1} in kNoiseBlock blocks (lane chains, halving tree);
// token_sum_final_kernel adds the block partials (64 lane sums and a tree)
__global__ __launch_bounds__(256) void token_sum_partials_kernel(int64_t M, const int32_t* salt,
                                                                 float* __restrict__ part,
                                                                 float* __restrict__ eps) {
  __shared__ float s[256];
  const int64_t b0 = (int64_t)blockIdx.x * kNoiseBlock;
  const int32_t seed = *salt;
  float a = 0.0f;
  for (int i = 0; i < kNoiseBlock / 256; ++i) {
    const int64_t m = b0 + threadIdx.x + 256 * i;
    if (m < M) {
      const float z = normal_draw(seed, (uint32_t)m, kNoiseTagToken);
      eps[m] = z;   // each token's draw, once, for the scaling of dy
      a = __fadd_rn(a, z);
    }
  }
  s[threadIdx.x] = a;
  __syncthreads();
  for (int h = 128; h >= 1; h >>= 1) {
    if (threadIdx.x < h) s[threadIdx.x] = __fadd_rn(s[threadIdx.x], s[threadIdx.x + h]);
    __syncthreads();
  }
  if (threadIdx.x == 0) part[blockIdx.x] = s[0];
}

__global__ __launch_bounds__(64) void token_sum_final_kernel(const float* __restrict__ part, int64_t nb,
                                                             float* out) {
  const float s = wave_tree_sum(part, nb, 1);
  if (threadIdx.x == 0) *out = s;
}

// noise_e = f32(P_e) - S * (g_e / M)
CONCORD_DEV float sigmag_noise(float p, float g, float S, float Mf) {
  return __fsub_rn(p, __fmul_rn(S, __fdiv_rn(g, Mf)));
}

__global__ __launch_bounds__(256) void sigmag_partials_kernel(const uint16_t* __restrict__ g, int64_t ld,
                                                              const uint16_t* __restrict__ P, int64_t N,
                                                              int64_t K, const float* Ssum, float Mf,
                                                              float* __restrict__ part) {
  __shared__ float sg[256], sx[256];
  const int64_t total = N * K;
  const int64_t b0 = (int64_t)blockIdx.x * kNoiseBlock;
  const float S = *Ssum;
  float ag = 0.0f, ax = 0.0f;
  for (int i = 0; i < kNoiseBlock / 256; ++i) {
    const int64_t e = b0 + threadIdx.x + 256 * i;
    if (e < total) {
      const float v = bf16_to_f32(g[elem_off(e, K, ld)]);
      const float z = sigmag_noise(bf16_to_f32(P[e]), v, S, Mf);
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

__global__ __launch_bounds__(256) void sigmag_apply_kernel(uint16_t* __restrict__ g, int64_t ld,
                                                           const uint16_t* __restrict__ P, int64_t N, int64_t K,
                                                           const float* Ssum, float Mf, const float* scale) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= N * K) return;
  const float S = *Ssum, sc = *scale;
  uint16_t* p = g + elem_off(e, K, ld);
  const float v = bf16_to_f32(*p);
  const float r = __fadd_rn(v, __fmul_rn(sigmag_noise(bf16_to_f32(P[e]), v, S, Mf), sc));
  *p = (uint16_t)(pack_bf16x2(r, 0.0f) & 0xFFFFu);
}

struct SigmagLayout {
  size_t dyt, prod, part, tpart, ssum, scale, eps, gemm, total;
};
static SigmagLayout sigmag_layout(int64_t M, int64_t N, int64_t K) {
  auto r256 = [](size_t b) { return (b + 255) / 256 * 256; };
  SigmagLayout L;
  size_t o = 0;
  // the product's split-K region first: its tile counters sit at the
  // workspace's start for every shape (see muon_layout)
  L.gemm = o; o += r256(gemm_splitk_need(MODE_WGRAD, N, K, M));
  L.dyt = o; o += r256((size_t)M * N * 2);
  L.prod = o; o += r256((size_t)N * K * 2);
  L.part = o; o += r256((size_t)2 * cdiv(N * K, kNoiseBlock) * 4);
  L.tpart = o; o += r256((size_t)cdiv(M, kNoiseBlock) * 4);
  L.ssum = o; o += 256;
  L.scale = o; o += 256;
  L.eps = o; o += r256((size_t)M * 4);
  L.total = o;
  return L;
}

}  // namespace concord

using namespace concord;

extern "C" size_t concord_sigmag_noise_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  return sigmag_layout(M > 0 ? M : 1, N > 0 ? N : 1, K > 0 ? K : 1).total;
}

extern "C" int concord_sigmag_noise(uint16_t* grad_w, int64_t ld_g, const uint16_t* dy, int64_t ld_dy,
                                    const uint16_t* x, int64_t ld_x, int64_t M, int64_t N, int64_t K,
                                    const float* sigma, const int32_t* salt_counter, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  CONCORD_CHECK(M >= 0 && N >= 0 && K >= 0 && N * K < (1LL << 32) && M * N < (1LL << 40) && M < (1LL << 31),
                "concord_sigmag_noise: bad size");
  if (N == 0 || K == 0) return CONCORD_OK;
  CONCORD_CHECK(grad_w && dy && x && sigma && salt_counter, "concord_sigmag_noise: NULL argument");
  CONCORD_CHECK(ld_g >= K && ld_dy >= N && ld_x >= K, "concord_sigmag_noise: bad leading dimension");
  const SigmagLayout L = sigmag_layout(M > 0 ? M : 1, N, K);
  if (!workspace || workspace_bytes < L.total) {
    set_error("concord_sigmag_noise: workspace of %zu bytes needed", L.total);
    return CONCORD_EWORKSPACE;
  }
  char* w = (char*)workspace;
  uint16_t* dyt = (uint16_t*)(w + L.dyt);
  uint16_t* prod = (uint16_t*)(w + L.prod);
  float* part = (float*)(w + L.part);
  float* tpart = (float*)(w + L.tpart);
  float* ssum = (float*)(w + L.ssum);
  float* scale = (float*)(w + L.scale);
  float* eps = (float*)(w + L.eps);
  hipStream_t st = (hipStream_t)stream;
  const int64_t tb = M > 0 ? cdiv(M, kNoiseBlock) : 0;
  if (M > 0) {
    hipLaunchKernelGGL(token_sum_partials_kernel, dim3((unsigned)tb), dim3(256), 0, st, M, salt_counter, tpart,
                       eps);
    hipLaunchKernelGGL(token_scale_kernel, dim3((unsigned)cdiv(N, 2048), grid_y(M)),
                       dim3(256), 0, st, dy, ld_dy, M, N, eps, dyt);
  }
  hipLaunchKernelGGL(token_sum_final_kernel, dim3(1), dim3(64), 0, st, tpart, tb, ssum);
  // P = dyt^T x (the WGRAD product of the scaled dy), bf16
  const int rc = gemm_bf16_run(MODE_WGRAD, dyt, N, x, ld_x, prod, K, N, K, M, w + L.gemm,
                               L.dyt - L.gemm, st, "sigmag_noise");
  if (rc != CONCORD_OK) return rc;
  const float Mf = (float)(M > 1 ? M : 1);
  const int64_t nb = cdiv(N * K, kNoiseBlock);
  hipLaunchKernelGGL(sigmag_partials_kernel, dim3((unsigned)nb), dim3(256), 0, st, grad_w, ld_g, prod, N, K, ssum,
                     Mf, part);
  hipLaunchKernelGGL(noise_scale_kernel, dim3(1), dim3(64), 0, st, part, nb, sigma, scale);
  hipLaunchKernelGGL(sigmag_apply_kernel, dim3((unsigned)cdiv(N * K, 256)), dim3(256), 0, st, grad_w, ld_g, prod,
                     N, K, ssum, Mf, scale);
  return launch_status("sigmag_noise");
}

namespace concord {

// isotropic workspace: the block partials, the scale (256 bytes), then the
// draws xi (fp32, one per element)
struct IsoLayout {
  size_t part, scale, xi, total;
};
static IsoLayout iso_layout(int64_t N, int64_t K) {
  auto r256 = [](size_t b) { return (b + 255) / 256 * 256; };
  const int64_t nk = N * K > 0 ? N * K : 0;
  IsoLayout L;
  L.part = 0;
  L.scale = r256((size_t)2 * cdiv(nk, kNoiseBlock) * 4);
  L.xi = L.scale + 256;
  L.total = L.xi + r256((size_t)nk * 4);
  return L;
}

}  // namespace concord

extern "C" size_t concord_noise_workspace_bytes(int64_t N, int64_t K) { return iso_layout(N, K).total; }

namespace concord {
namespace {
int iso_noise_launch(uint16_t* grad_w, int64_t ld_g, int64_t N, int64_t K, const float* sigma,
                     const int32_t* salt_counter, void* workspace, hipStream_t st) {
  const IsoLayout L = iso_layout(N, K);
  const int64_t nb = cdiv(N * K, kNoiseBlock);
  char* w = (char*)workspace;
  float* part = (float*)(w + L.part);
  float* scale = (float*)(w + L.scale);
  float* xi = (float*)(w + L.xi);
  hipLaunchKernelGGL(noise_partials_kernel, dim3((unsigned)nb), dim3(256), 0, st, grad_w, ld_g, N, K,
                     salt_counter, part, xi);
  hipLaunchKernelGGL(noise_scale_kernel, dim3(1), dim3(64), 0, st, part, nb, sigma, scale);
  hipLaunchKernelGGL(noise_apply_kernel, dim3((unsigned)cdiv(N * K, 1024)), dim3(256), 0, st, grad_w, ld_g, N,
                     K, xi, scale);
  return launch_status("iso_noise");
}
}  // namespace
}  // namespace concord

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
  return iso_noise_launch(grad_w, ld_g, N, K, sigma, salt_counter, workspace, (hipStream_t)stream);
}
