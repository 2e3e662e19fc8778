// muon.hip -- the Muon drive: O = gamma * NS5(g / ||g||_F) in bf16.
//
// experiments/cpu_dynamics/exp9_muon.py:44-55 (ns5) and 58-100 (the drive
// sqrt(max(N, K)) * ns5(g / ||g||)); docs/MUON_IMPLEMENTATION.md:27-40 (bf16
// NS on the backward's grad_W) and 87-119 (O is the apply kernel's step).
//
// Numerics (oracle_muon_ns5 restates them):
//   ||g||^2  blocks of 8192 elements of the row-major flattening; lane t of a
//            block sums elements t, t + 256, ... ascending, then the halving
//            tree over 256 lanes; block totals: lane l of 64 sums totals l,
//            l + 64, ... ascending, then the halving tree over the 64 lanes.
//            norm = sqrt (RN).
//   X0 = bf16(g / (n (norm / n + 1e-7))), n = max(norm, 1e-12), transposed
//   when N > K (X is m x n, m <= n)
//   5 x:  A = bf16(X X^T); AA = bf16(A A); B = bf16(b A + c AA);
//         BX = bf16(B X); X = bf16(a X + BX)      (products: bf16 MFMA, fp32 acc)
//   out = bf16(gamma X), transposed back.
// The three products run on the library's bf16 GEMM kernels; the symmetric
// two (X X^T, and A A with B's combination) compute only the tiles that meet
// the upper triangle and store each upper element at its mirror position too
// (gemm_bf16_sym).  The two
// combinations ride in the epilogue of the product they follow (A A -> B,
// B X -> the new X; gemm_bf16_combine), which writes into a second buffer:
// B goes to the AA buffer and X ping-pongs between two buffers.  Operands the
// fast kernels do not take fall back to an elementwise combination kernel;
// both routes round identically (combine_bf16x2).
#include <utility>

#include "common.h"
#include "gemm.h"
#include "workspace.h"

namespace concord {

constexpr int kFrobBlock = 8192;   // elements per block of the ||g||^2 partials

// per-block partial of sum g^2 in the order above
__global__ __launch_bounds__(256) void frob_partials_kernel(const uint16_t* __restrict__ g, int64_t ld,
                                                            int64_t N, int64_t K, float* __restrict__ part) {
  __shared__ float s[256];
  __shared__ __align__(16) uint16_t tile[kFrobBlock];
  const int t = threadIdx.x;
  const int64_t total = N * K;
  const int64_t b0 = (int64_t)blockIdx.x * kFrobBlock;
  float acc = 0.0f;
  if (ld == K && b0 + kFrobBlock <= total && ((uintptr_t)g % 16) == 0) {
    // a whole contiguous block: 16-byte loads into LDS, then each lane chains
    // its elements t, t + 256, ... from there in the same order
#pragma unroll
    for (int q = 0; q < kFrobBlock / 2048; ++q) {
      const int o = 2048 * q + 8 * t;
      *reinterpret_cast<uint4*>(tile + o) = *reinterpret_cast<const uint4*>(g + b0 + o);
    }
    __syncthreads();
#pragma unroll 8
    for (int i = 0; i < kFrobBlock / 256; ++i) {
      const float v = bf16_to_f32(tile[t + 256 * i]);
      acc = __fadd_rn(acc, __fmul_rn(v, v));
    }
  } else {
#pragma unroll 8
    for (int i = 0; i < kFrobBlock / 256; ++i) {
      const int64_t e = b0 + t + 256 * i;
      float v = 0.0f;
      if (e < total) v = bf16_to_f32(ld == K ? g[e] : g[(e / K) * ld + e % K]);
      acc = __fadd_rn(acc, __fmul_rn(v, v));
    }
  }
  s[t] = acc;
  __syncthreads();
  for (int h = 128; h >= 1; h >>= 1) {
    if (t < h) s[t] = __fadd_rn(s[t], s[t + h]);
    __syncthreads();
  }
  if (t == 0) part[blockIdx.x] = s[0];
}

// den = n (||g|| / n + 1e-7), n = max(||g||, 1e-12), ||g|| = sqrt of the
// block partials summed as above (lane l of one wave: partials l, l + 64,
// ... ascending, every lane's partials in flight at once; then the halving
// tree over the 64 lanes): the drive normalises g by max(||g||, 1e-12) and
// ns5 then divides by (the result's norm + 1e-7) (exp9_muon.py:75, 82, 47).
// For ||g|| >= 1e-12 the quotient is exactly 1 and the sum fl(1 + 1e-7);
// below, ||g|| / n < 1 and the input is brought back to unit norm as the
// reference's second division does.
__global__ __launch_bounds__(64) void frob_den_kernel(const float* __restrict__ part, int64_t nb, float* den) {
  constexpr int kPer = 16;
  const int t = threadIdx.x;
  float tot = 0.0f;
  for (int64_t c0 = 0; c0 < nb; c0 += 64 * kPer) {
    float v[kPer];
#pragma unroll
    for (int e = 0; e < kPer; ++e) {
      const int64_t i = c0 + 64 * e + t;
      v[e] = i < nb ? part[i] : 0.0f;
    }
#pragma unroll
    for (int e = 0; e < kPer; ++e)
      if (c0 + 64 * e + t < nb) tot = __fadd_rn(tot, v[e]);
  }
#pragma unroll
  for (int h = 32; h >= 1; h >>= 1) tot = __fadd_rn(tot, __shfl_down(tot, h, 64));
  if (t == 0) {
    const float norm = sqrt_rn(tot);
    const float n = fmaxf(norm, 1e-12f);
    *den = __fmul_rn(n, __fadd_rn(__fdiv_rn(norm, n), 1e-7f));
  }
}

// dst[r][c] = bf16(op(src)) over a 64 x 64 tile, where the destination is
// R x C; with TRANS the source element of dst[r][c] is src[c][r].
// DIV: src / *den (the first NS input); else gamma * src (the output).
template <bool TRANS, bool DIV>
__global__ __launch_bounds__(256) void ns5_copy_kernel(const uint16_t* __restrict__ src, int64_t lds,
                                                       uint16_t* __restrict__ dst, int64_t ldd, int64_t R,
                                                       int64_t C, const float* den, float gamma) {
  __shared__ float t[64][65];
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  const float d = DIV ? *den : gamma;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int i = ty; i < 64; i += 4) {
    // read coalesced along the source's rows
    if (TRANS) {
      const int64_t sr = c0 + i, sc = r0 + tx;   // src[sr][sc] -> dst[sc][sr]
      float v = 0.0f;
      if (sr < C && sc < R) v = bf16_to_f32(src[sr * lds + sc]);
      t[tx][i] = v;
    } else {
      const int64_t sr = r0 + i, sc = c0 + tx;
      float v = 0.0f;
      if (sr < R && sc < C) v = bf16_to_f32(src[sr * lds + sc]);
      t[i][tx] = v;
    }
  }
  __syncthreads();
  for (int i = ty; i < 64; i += 4) {
    const int64_t r = r0 + i, c = c0 + tx;
    if (r < R && c < C) {
      const float v = t[i][tx];
      const float o = DIV ? __fdiv_rn(v, d) : __fmul_rn(d, v);
      dst[r * ldd + c] = (uint16_t)(pack_bf16x2(o, 0.0f) & 0xFFFFu);
    }
  }
}

// ns5_copy_kernel with 16-byte accesses (bases 16-byte aligned, leading
// dimensions multiples of 8): a thread moves 8 consecutive elements; chunks
// crossing the matrix edge take 2-byte accesses.  The transpose goes through
// a bf16 LDS tile whose 16-byte chunk q of row r sits at chunk q ^ swz(r),
// so that both the chunk writes and the column reads spread over the banks.
CONCORD_DEV int ns5_swz(int r) { return (r & 7) ^ ((r >> 3) & 7); }
template <bool TRANS, bool DIV>
__global__ __launch_bounds__(256) void ns5_copy_vec_kernel(const uint16_t* __restrict__ src, int64_t lds,
                                                           uint16_t* __restrict__ dst, int64_t ldd, int64_t R,
                                                           int64_t C, const float* den, float gamma) {
  __shared__ __align__(16) uint16_t t[64 * 64];
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;   // destination tile
  const float d = DIV ? *den : gamma;
  const int cq = threadIdx.x & 7, rr = threadIdx.x >> 3;
  auto op = [&](float v) { return DIV ? __fdiv_rn(v, d) : __fmul_rn(d, v); };
  auto store8 = [&](int64_t r, int64_t c, const float (&v)[8]) {
    if (c + 8 <= C) {
      *reinterpret_cast<uint4*>(dst + r * ldd + c) =
          make_uint4(pack_bf16x2(op(v[0]), op(v[1])), pack_bf16x2(op(v[2]), op(v[3])),
                     pack_bf16x2(op(v[4]), op(v[5])), pack_bf16x2(op(v[6]), op(v[7])));
    } else {
      for (int e = 0; e < 8 && c + e < C; ++e) dst[r * ldd + c + e] = (uint16_t)(pack_bf16x2(op(v[e]), 0.0f) & 0xFFFFu);
    }
  };
  if (!TRANS) {
    for (int h = 0; h < 2; ++h) {
      const int64_t r = r0 + rr + 32 * h, c = c0 + 8 * cq;
      if (r >= R || c >= C) continue;
      float v[8];
      if (c + 8 <= C) {
        const uint4 w = *reinterpret_cast<const uint4*>(src + r * lds + c);
        const uint32_t q[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[2 * e] = __uint_as_float(q[e] << 16);
          v[2 * e + 1] = __uint_as_float(q[e] & 0xFFFF0000u);
        }
      } else {
        for (int e = 0; e < 8; ++e) v[e] = c + e < C ? bf16_to_f32(src[r * lds + c + e]) : 0.0f;
      }
      store8(r, c, v);
    }
    return;
  }
  // dst[r][c] = op(src[c][r]): the source tile is rows c0 .. c0 + 63 (< C)
  // and columns r0 .. r0 + 63 (< R) of the C x R source
  for (int h = 0; h < 2; ++h) {
    const int sr = rr + 32 * h;
    const int64_t gr = c0 + sr, gc = r0 + 8 * cq;
    uint4 w = make_uint4(0u, 0u, 0u, 0u);
    if (gr < C) {
      if (gc + 8 <= R) {
        w = *reinterpret_cast<const uint4*>(src + gr * lds + gc);
      } else {
        uint32_t q[4] = {0u, 0u, 0u, 0u};
        for (int e = 0; e < 8 && gc + e < R; ++e) q[e >> 1] |= (uint32_t)src[gr * lds + gc + e] << (16 * (e & 1));
        w = make_uint4(q[0], q[1], q[2], q[3]);
      }
    }
    *reinterpret_cast<uint4*>(t + sr * 64 + 8 * (cq ^ ns5_swz(sr))) = w;
  }
  __syncthreads();
  for (int h = 0; h < 2; ++h) {
    const int dr = rr + 32 * h;   // destination row in the tile = source column
    const int64_t r = r0 + dr, c = c0 + 8 * cq;
    if (r >= R || c >= C) continue;
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int sr = 8 * cq + e;
      v[e] = bf16_to_f32(t[sr * 64 + 8 * ((dr >> 3) ^ ns5_swz(sr)) + (dr & 7)]);
    }
    store8(r, c, v);
  }
}

// y = bf16(s * y + t * x), elementwise over n values (B from A and AA with
// s = b, t = c; the new X from X and BX with s = a, t = 1)
__global__ __launch_bounds__(256) void ns5_axpby_kernel(uint16_t* __restrict__ y, const uint16_t* __restrict__ x,
                                                        int64_t n, float s, float t) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= n) return;
  if (i + 4 <= n) {
    const uint2 yv = *reinterpret_cast<const uint2*>(y + i);
    const uint2 xv = *reinterpret_cast<const uint2*>(x + i);
    const uint32_t yw[2] = {yv.x, yv.y}, xw[2] = {xv.x, xv.y};
    uint32_t o[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      o[h] = combine_bf16x2(yw[h], xw[h], s, t);
    }
    *reinterpret_cast<uint2*>(y + i) = make_uint2(o[0], o[1]);
  } else {
    for (int64_t j = i; j < n; ++j) {
      y[j] = (uint16_t)(combine_bf16x2(y[j], x[j], s, t) & 0xFFFFu);
    }
  }
}

struct MuonLayout {
  size_t x, bx, a, aa, part, den, gemm, total;
};

static MuonLayout muon_layout(int64_t N, int64_t K) {
  const int64_t m = N < K ? N : K, n = N < K ? K : N;
  auto r256 = [](size_t b) { return (b + 255) / 256 * 256; };
  MuonLayout L;
  size_t o = 0;
  // split-K region of the three products first: its tile counters sit at
  // the workspace's start for every shape, so the zero state each product
  // leaves them in holds across calls of different shapes
  size_t g = gemm_splitk_need(MODE_FWD_BF16, m, m, n);
  const size_t g2 = gemm_splitk_need(MODE_DGRAD_BF16, m, m, m), g3 = gemm_splitk_need(MODE_DGRAD_BF16, m, n, m);
  const size_t g4 = gemm_sym_splitk_need(MODE_FWD_BF16, m, n), g5 = gemm_sym_splitk_need(MODE_DGRAD_BF16, m, m);
  for (size_t v : {g2, g3, g4, g5})
    if (v > g) g = v;
  L.gemm = o; o += r256(g);
  L.x = o; o += r256((size_t)m * n * 2);
  L.bx = o; o += r256((size_t)m * n * 2);
  L.a = o; o += r256((size_t)m * m * 2);
  L.aa = o; o += r256((size_t)m * m * 2);
  L.part = o; o += r256((size_t)cdiv(N * K, kFrobBlock) * 4);
  L.den = o; o += 256;
  L.total = o;
  return L;
}

}  // namespace concord

using namespace concord;

extern "C" size_t concord_muon_workspace_bytes(int64_t N, int64_t K) {
  if (N <= 0 || K <= 0) return 256;
  return muon_layout(N, K).total;
}

extern "C" int concord_muon_ns5(const uint16_t* g, int64_t ld_g, int64_t N, int64_t K, float gamma,
                                uint16_t* out, int64_t ld_out, void* workspace, size_t workspace_bytes,
                                void* stream) {
  CONCORD_CHECK(N > 0 && K > 0 && N < (1LL << 30) && K < (1LL << 30) && N * K < (1LL << 40),
                "concord_muon_ns5: bad size N=%lld K=%lld", (long long)N, (long long)K);
  CONCORD_CHECK(g && out, "concord_muon_ns5: NULL argument");
  CONCORD_CHECK(ld_g >= K && ld_out >= K, "concord_muon_ns5: leading dimension < K");
  CONCORD_CHECK(cdiv(N, 64) <= kMaxGridY && cdiv(K, 64) <= kMaxGridY,
                "concord_muon_ns5: N=%lld K=%lld exceed the transpose kernel's grid (at most %lld per side)",
                (long long)N, (long long)K, (long long)(kMaxGridY * 64));
  const MuonLayout L = muon_layout(N, K);
  if (!workspace || workspace_bytes < L.total) {
    set_error("concord_muon_ns5: workspace of %zu bytes needed", L.total);
    return CONCORD_EWORKSPACE;
  }
  char* base = (char*)workspace;
  uint16_t* X = (uint16_t*)(base + L.x);
  uint16_t* BX = (uint16_t*)(base + L.bx);
  uint16_t* A = (uint16_t*)(base + L.a);
  uint16_t* AA = (uint16_t*)(base + L.aa);
  float* part = (float*)(base + L.part);
  float* den = (float*)(base + L.den);
  void* gws = base + L.gemm;
  const size_t gws_bytes = L.x - L.gemm;
  hipStream_t st = (hipStream_t)stream;
  const bool tr = N > K;
  const int64_t m = tr ? K : N, n = tr ? N : K;
  const int64_t nb = cdiv(N * K, kFrobBlock);

  hipLaunchKernelGGL(frob_partials_kernel, dim3((unsigned)nb), dim3(256), 0, st, g, ld_g, N, K, part);
  hipLaunchKernelGGL(frob_den_kernel, dim3(1), dim3(64), 0, st, part, nb, den);
  const dim3 gx((unsigned)cdiv(n, 64), (unsigned)cdiv(m, 64));
  // 16-byte accesses where the gradient and X allow them (X's rows are n
  // elements from a 256-byte aligned base)
  const bool vin = ((uintptr_t)g % 16) == 0 && ld_g % 8 == 0 && n % 8 == 0;
  if (tr && vin)
    hipLaunchKernelGGL((ns5_copy_vec_kernel<true, true>), gx, dim3(256), 0, st, g, ld_g, X, n, m, n, den, 0.0f);
  else if (vin)
    hipLaunchKernelGGL((ns5_copy_vec_kernel<false, true>), gx, dim3(256), 0, st, g, ld_g, X, n, m, n, den, 0.0f);
  else if (tr)
    hipLaunchKernelGGL((ns5_copy_kernel<true, true>), gx, dim3(256), 0, st, g, ld_g, X, n, m, n, den, 0.0f);
  else
    hipLaunchKernelGGL((ns5_copy_kernel<false, true>), gx, dim3(256), 0, st, g, ld_g, X, n, m, n, den, 0.0f);
  int rc = launch_status("muon_ns5");
  if (rc != CONCORD_OK) return rc;
  const float a = 3.4445f, b = -4.7750f, c = 2.0315f;
  for (int it = 0; it < 5; ++it) {
    // A = X X^T and A A are symmetric: only the tiles meeting the upper
    // triangle are computed, each upper element also stored at its mirror
    rc = gemm_bf16_sym(MODE_FWD_BF16, X, n, X, n, A, m, m, n, nullptr, 0, 0.0f, 0.0f, gws, gws_bytes, st,
                       "muon_ns5 X X^T");
    if (rc == -1) rc = gemm_bf16_run(MODE_FWD_BF16, X, n, X, n, A, m, m, m, n, gws, gws_bytes, st, "muon_ns5 X X^T");
    if (rc != CONCORD_OK) return rc;
    // AA buffer <- B = bf16(b A + c bf16(A A)), symmetric as A is
    rc = gemm_bf16_sym(MODE_DGRAD_BF16, A, m, A, m, AA, m, m, m, A, m, b, c, gws, gws_bytes, st, "muon_ns5 A A");
    if (rc == -1)
      rc = gemm_bf16_combine(MODE_DGRAD_BF16, A, m, A, m, AA, m, m, m, m, A, m, b, c, gws, gws_bytes, st,
                             "muon_ns5 A A");
    if (rc == -1) {
      rc = gemm_bf16_run(MODE_DGRAD_BF16, A, m, A, m, AA, m, m, m, m, gws, gws_bytes, st, "muon_ns5 A A");
      if (rc != CONCORD_OK) return rc;
      hipLaunchKernelGGL(ns5_axpby_kernel, dim3((unsigned)cdiv(cdiv(m * m, 4), 256)), dim3(256), 0, st, A, AA,
                         m * m, b, c);
      std::swap(A, AA);   // B now in the AA slot, as on the fused route
    }
    if (rc != CONCORD_OK) return rc;
    // BX buffer <- the new X = bf16(a X + bf16(B X)); then X and BX trade places
    rc = gemm_bf16_combine(MODE_DGRAD_BF16, AA, m, X, n, BX, n, m, n, m, X, n, a, 1.0f, gws, gws_bytes, st,
                           "muon_ns5 B X");
    if (rc == -1) {
      rc = gemm_bf16_run(MODE_DGRAD_BF16, AA, m, X, n, BX, n, m, n, m, gws, gws_bytes, st, "muon_ns5 B X");
      if (rc != CONCORD_OK) return rc;
      hipLaunchKernelGGL(ns5_axpby_kernel, dim3((unsigned)cdiv(cdiv(m * n, 4), 256)), dim3(256), 0, st, X, BX,
                         m * n, a, 1.0f);
      std::swap(X, BX);   // the new X now in the BX slot, as on the fused route
    }
    if (rc != CONCORD_OK) return rc;
    std::swap(X, BX);
  }
  // out[N][K] = bf16(gamma X) (X^T when transposed)
  const dim3 go((unsigned)cdiv(K, 64), (unsigned)cdiv(N, 64));
  const bool vout = ((uintptr_t)out % 16) == 0 && ld_out % 8 == 0 && n % 8 == 0;
  if (tr && vout)
    hipLaunchKernelGGL((ns5_copy_vec_kernel<true, false>), go, dim3(256), 0, st, X, n, out, ld_out, N, K, den,
                       gamma);
  else if (vout)
    hipLaunchKernelGGL((ns5_copy_vec_kernel<false, false>), go, dim3(256), 0, st, X, n, out, ld_out, N, K, den,
                       gamma);
  else if (tr)
    hipLaunchKernelGGL((ns5_copy_kernel<true, false>), go, dim3(256), 0, st, X, n, out, ld_out, N, K, den, gamma);
  else
    hipLaunchKernelGGL((ns5_copy_kernel<false, false>), go, dim3(256), 0, st, X, n, out, ld_out, N, K, den, gamma);
  return launch_status("muon_ns5");
}
