// conv.hip -- the patch matrix of ConcordConv2dPackedB (concord/packed_b.py:
// 2028-2065, a Conv2d over the packed (out, in * kh * kw) state).
//
// cols[m][k] = x[b][c][ho * sh - ph + i][wo * sw - pw + j] (0 outside the
// image), m = (b * Ho + ho) * Wo + wo, k = (c * kh + i) * kw + j: the rows are
// the output positions and the columns nn.Conv2d's (c, i, j) weight
// flattening, so the layer's forward, dgrad and wgrad are the packed linear
// products on cols.  im2col builds cols in one pass; col2im, its adjoint,
// gathers dx from the patch gradient (see below).
#include <algorithm>

#include "common.h"
#include "gemm.h"
#include "vhat.h"
#include "vhat_tile.h"
#include "workspace.h"

namespace concord {

struct ConvGeom {
  int64_t B, C, H, W, kh, kw, sh, sw, ph, pw, Ho, Wo, K;
};

// A block fills a 64-row x 64-column tile of cols.  Loads: wave w takes
// columns w, w + 4, ..., each lane one row (output position), so a wave reads
// 64 consecutive positions of one input row -- contiguous along w for stride
// 1 -- into LDS.  Stores: a thread writes 8 consecutive columns of one row
// (16 bytes when K % 8 == 0).
constexpr int kTileM = 64, kTileK = 64, kTileLd = kTileK + 2;

__global__ __launch_bounds__(256) void im2col_kernel(const uint16_t* __restrict__ x, ConvGeom g,
                                                     uint16_t* __restrict__ cols) {
  __shared__ uint16_t tile[kTileM * kTileLd];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t M = g.B * g.Ho * g.Wo;
  const int64_t m0 = (int64_t)blockIdx.x * kTileM, k0 = (int64_t)blockIdx.y * kTileK;
  const int64_t m = m0 + lane;
  const int64_t wo = m % g.Wo, r = m / g.Wo;
  const int64_t ho = r % g.Ho, b = r / g.Ho;
  const bool mok = m < M;
  const uint16_t* xb = x + (mok ? b : 0) * g.C * g.H * g.W;
  // this lane's window origin; (c, i, j) of the wave's first column, then
  // stepped by 4 columns per iteration (wave-uniform, 32-bit)
  const int hb = (int)(ho * g.sh - g.ph), wb = (int)(wo * g.sw - g.pw);
  const int H = (int)g.H, W = (int)g.W, kh = (int)g.kh, kw = (int)g.kw;
  const int64_t kfirst = k0 + wave;
  int c = (int)(kfirst / (g.kh * g.kw));
  int ij = (int)(kfirst % (g.kh * g.kw));
  int i = ij / kw, j = ij - i * kw;
  // the wave's 16 columns are loaded before any is stored
  uint16_t v[kTileK / 4];
#pragma unroll
  for (int n = 0; n < kTileK / 4; ++n) {
    const int q = wave + 4 * n;
    v[n] = 0;
    if (k0 + q < g.K && mok) {
      const int h = hb + i, w = wb + j;
      if (h >= 0 && h < H && w >= 0 && w < W) v[n] = xb[((int64_t)c * H + h) * W + w];
    }
    j += 4;
    while (j >= kw) {
      j -= kw;
      if (++i == kh) {
        i = 0;
        ++c;
      }
    }
  }
#pragma unroll
  for (int n = 0; n < kTileK / 4; ++n) tile[lane * kTileLd + wave + 4 * n] = v[n];
  __syncthreads();
  const bool vec = (g.K % 8) == 0 && ((uintptr_t)cols % 16) == 0;
  for (int q = threadIdx.x; q < kTileM * (kTileK / 8); q += 256) {
    const int ml = q / (kTileK / 8), kg = (q % (kTileK / 8)) * 8;
    const int64_t mm = m0 + ml, kc = k0 + kg;
    if (mm >= M || kc >= g.K) continue;
    const uint16_t* src = tile + ml * kTileLd + kg;
    uint16_t* dst = cols + mm * g.K + kc;
    if (vec) {
      *reinterpret_cast<uint4*>(dst) =
          make_uint4(src[0] | ((uint32_t)src[1] << 16), src[2] | ((uint32_t)src[3] << 16),
                     src[4] | ((uint32_t)src[5] << 16), src[6] | ((uint32_t)src[7] << 16));
    } else {
      for (int e = 0; e < 8 && kc + e < g.K; ++e) dst[e] = src[e];
    }
  }
}

// ---- col2im: the adjoint of im2col, a fixed-order gather -------------------
// dx[b][c][h][w] = bf16(sum over i ascending, then j ascending, of
// dcols[(b * Ho + ho) * Wo + wo][(c * kh + i) * kw + j]) over the (i, j) with
// ho * sh = h + ph - i and wo * sw = w + pw - j exactly, 0 <= ho < Ho,
// 0 <= wo < Wo; fp32 accumulation.
// A block owns 4 rows x 64 columns of the image for `cc` channels.  It stages
// the dcols segments those outputs read -- rows (ho, wo) of its window, the
// cc * kh * kw contiguous columns of its channels -- in LDS (each (ho, wo)
// segment padded to an odd number of dwords), then a lane per column w sums
// and writes rows of dx along w.
constexpr int kC2iH = 4, kC2iW = 64;

struct Col2imTile {
  int nho, nwo, cc, seg, ld;   // staged rows / columns, channels per block, segment, padded segment
};

__device__ __forceinline__ int64_t ceil_div_nn(int64_t a, int64_t b) { return (a + b - 1) / b; }

__global__ __launch_bounds__(256) void col2im_kernel(const uint16_t* __restrict__ dcols, ConvGeom g, Col2imTile T,
                                                     uint16_t* __restrict__ dx) {
  extern __shared__ uint16_t stage[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t hblocks = (g.H + kC2iH - 1) / kC2iH;
  const int64_t w0 = (int64_t)blockIdx.x * kC2iW;
  const int64_t b = blockIdx.y / hblocks, h0 = (blockIdx.y % hblocks) * kC2iH;
  const int64_t c0 = (int64_t)blockIdx.z * T.cc;
  const int ncl = (int)min((int64_t)T.cc, g.C - c0);
  const int kk = (int)(g.kh * g.kw);
  const int64_t ho_lo = ceil_div_nn(max(h0 + g.ph - (g.kh - 1), (int64_t)0), g.sh);
  const int64_t wo_lo = ceil_div_nn(max(w0 + g.pw - (g.kw - 1), (int64_t)0), g.sw);
  const int seg = ncl * kk;
  const int npairs = T.nho * T.nwo;
  // 8-byte staging when every segment starts 8-byte aligned in dcols and in
  // LDS: lane l of a wave moves chunk l % cpp of row p0 + l / cpp
  const int cpp = seg / 4;
  const bool vec8 = (seg % 4) == 0 && (g.K % 4) == 0 && ((c0 * kk) % 4) == 0 && (T.ld % 4) == 0 &&
                    ((uintptr_t)dcols % 8) == 0 && cpp > 0 && cpp <= 64;
  if (vec8) {
    const int per = 64 / cpp;            // rows per wave instruction
    const int pl = lane / cpp, ch = lane - pl * cpp;
    constexpr int U8 = 4;
    for (int p0 = wave * per; p0 < npairs; p0 += 4 * per * U8) {
      uint2 v[U8];
#pragma unroll
      for (int u = 0; u < U8; ++u) {
        const int p = p0 + 4 * per * u + pl;
        const int rl = p / T.nwo, cl = p - rl * T.nwo;
        const int64_t ho = ho_lo + rl, wo = wo_lo + cl;
        const bool ok = pl < per && p < npairs && ho < g.Ho && wo < g.Wo;
        v[u] = ok ? *reinterpret_cast<const uint2*>(dcols + ((b * g.Ho + ho) * g.Wo + wo) * g.K + c0 * kk + 4 * ch)
                  : make_uint2(0, 0);
      }
#pragma unroll
      for (int u = 0; u < U8; ++u) {
        const int p = p0 + 4 * per * u + pl;
        if (pl < per && p < npairs) *reinterpret_cast<uint2*>(stage + p * T.ld + 4 * ch) = v[u];
      }
    }
  }
  // otherwise a wave per (ho, wo) row, the lanes along its segment (at most 3
  // elements per lane); 8 rows' loads are issued before any is written
  constexpr int U = 8;
  for (int p0 = wave; !vec8 && p0 < npairs; p0 += 4 * U) {
    uint16_t v[U][3];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int p = p0 + 4 * u;
      const int rl = p / T.nwo, cl = p - rl * T.nwo;
      const int64_t ho = ho_lo + rl, wo = wo_lo + cl;
      const bool ok = p < npairs && ho < g.Ho && wo < g.Wo;
      const uint16_t* src = dcols + (ok ? ((b * g.Ho + ho) * g.Wo + wo) * g.K + c0 * kk : 0);
#pragma unroll
      for (int r = 0; r < 3; ++r) {
        const int e = lane + 64 * r;
        v[u][r] = ok && e < seg ? src[e] : (uint16_t)0;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int p = p0 + 4 * u;
      if (p >= npairs) break;
#pragma unroll
      for (int r = 0; r < 3; ++r) {
        const int e = lane + 64 * r;
        if (e < seg) stage[p * T.ld + e] = v[u][r];
      }
    }
  }
  __syncthreads();
  // gather: 32-bit offsets relative to the staged window
  const int w = (int)(w0 + lane);
  const bool unit = g.sh == 1 && g.sw == 1;
  const int kh = (int)g.kh, kw = (int)g.kw, sh = (int)g.sh, sw = (int)g.sw;
  const int Ho = (int)g.Ho, Wo = (int)g.Wo, hol = (int)ho_lo, wol = (int)wo_lo;
  const int ph = (int)g.ph, pw = (int)g.pw;
  for (int q = wave; q < ncl * kC2iH; q += 4) {
    const int cl = q / kC2iH;
    const int h = (int)h0 + (q - cl * kC2iH);
    if (h >= g.H || w >= g.W) continue;
    const uint16_t* base = stage + cl * kk;
    float acc = 0.0f;
    if (unit) {
      // the (i, j) with 0 <= h + ph - i < Ho and 0 <= w + pw - j < Wo, ascending
      const int i1 = min(kh - 1, h + ph), i0 = max(0, h + ph - (Ho - 1));
      const int j1 = min(kw - 1, w + pw), j0 = max(0, w + pw - (Wo - 1));
      for (int i = i0; i <= i1; ++i) {
        const uint16_t* row = base + (h + ph - i - hol) * T.nwo * T.ld + i * kw + (w + pw - wol) * T.ld;
        for (int j = j0; j <= j1; ++j) acc = __fadd_rn(acc, bf16_to_f32(row[j - j * T.ld]));
      }
      dx[((b * g.C + c0 + cl) * g.H + h) * g.W + w] = (uint16_t)(pack_bf16x2(acc, 0.0f) & 0xFFFFu);
      continue;
    }
    for (int i = 0; i < kh; ++i) {
      const int hh = h + ph - i;
      if (hh < 0) break;
      if (!unit && hh % sh) continue;
      const int ho = unit ? hh : hh / sh;
      if (ho >= Ho) continue;
      const uint16_t* row = base + (ho - hol) * T.nwo * T.ld + i * kw;
      for (int j = 0; j < kw; ++j) {
        const int ww = w + pw - j;
        if (ww < 0) break;
        if (!unit && ww % sw) continue;
        const int wo = unit ? ww : ww / sw;
        if (wo >= Wo) continue;
        acc = __fadd_rn(acc, bf16_to_f32(row[(wo - wol) * T.ld + j]));
      }
    }
    dx[((b * g.C + c0 + cl) * g.H + h) * g.W + w] = (uint16_t)(pack_bf16x2(acc, 0.0f) & 0xFFFFu);
  }
}

// col2im for windows too large for the staged tile: one lane per dx
// element, the same fixed (i ascending, j ascending) fp32 sum, reading dcols
// from global memory
__global__ __launch_bounds__(256) void col2im_direct_kernel(const uint16_t* __restrict__ dcols, ConvGeom g,
                                                            uint16_t* __restrict__ dx) {
  const int64_t total = g.B * g.C * g.H * g.W;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int64_t w = e % g.W, t1 = e / g.W;
    const int64_t h = t1 % g.H, t2 = t1 / g.H;
    const int64_t c = t2 % g.C, b = t2 / g.C;
    float acc = 0.0f;
    for (int64_t i = 0; i < g.kh; ++i) {
      const int64_t hh = h + g.ph - i;
      if (hh < 0 || hh % g.sh) continue;
      const int64_t ho = hh / g.sh;
      if (ho >= g.Ho) continue;
      for (int64_t j = 0; j < g.kw; ++j) {
        const int64_t ww = w + g.pw - j;
        if (ww < 0 || ww % g.sw) continue;
        const int64_t wo = ww / g.sw;
        if (wo >= g.Wo) continue;
        acc = __fadd_rn(acc, bf16_to_f32(dcols[((b * g.Ho + ho) * g.Wo + wo) * g.K + (c * g.kh + i) * g.kw + j]));
      }
    }
    dx[e] = (uint16_t)(pack_bf16x2(acc, 0.0f) & 0xFFFFu);
  }
}

// ---- implicit-GEMM convolution: weight and gradient in tap-major order -----
// W'[n][t][c] = the forward weight of packed word (n, c * taps + t): the
// GEMMs of the implicit convolution reduce over (tap, channel) with channels
// contiguous.  A block takes one row n and kTapC channels: it reads their
// kTapC * taps contiguous words (16 bytes per lane), decodes them
// (materialize_gated's fp32 order: (128 ss + g sf) + 128 vs; with g = 1 this
// equals the ungated decode, every term being an integer below 2^24) into an
// LDS tile [taps][kTapC], then writes taps rows of kTapC channels (8 bytes
// per lane).
// TAPS: the tap count when known at compile time (9 for 3 x 3), so that the
// index splits are multiplies; 0 = the runtime `taps_rt`.
constexpr int kTapC = 256;
constexpr int kTapLd = kTapC + 4;   // LDS row of weight_taps_kernel: tap rows 2 banks apart, 8-byte aligned

template <int TAPS>
__global__ __launch_bounds__(256) void weight_taps_kernel(const int32_t* __restrict__ packed, int64_t ld_p,
                                                          const int8_t* row_exp, const int8_t* col_exp,
                                                          int64_t Cin, int taps_rt, int32_t bias, float gain,
                                                          uint16_t* __restrict__ wt) {
  extern __shared__ uint16_t tl[];   // [taps][kTapLd]
  const int taps = TAPS ? TAPS : taps_rt;
  const int64_t n = blockIdx.y;
  const int64_t c0 = (int64_t)blockIdx.x * kTapC;
  const int nc = (int)min((int64_t)kTapC, Cin - c0);
  const int ne = nc * taps;
  const int32_t te_row = (int32_t)row_exp[n] - bias;
  const int32_t* src = packed + n * ld_p + c0 * taps;
  const int8_t* ce = col_exp + c0 * taps;
  auto dec = [&](int32_t w, int e) -> uint16_t {
    const Fields f = unpack(w);
    const float m = __fadd_rn(__fadd_rn((float)(f.ss * 128), __fmul_rn(gain, (float)f.sf)), (float)(f.vs * 128));
    const float v = __fmul_rn(m, exp2i(te_row + (int32_t)ce[e]));
    return (uint16_t)(pack_bf16x2(v, 0.0f) & 0xFFFFu);
  };
  auto put = [&](int e, uint16_t v) {
    const int cl = e / taps, t = e - cl * taps;
    tl[t * kTapLd + cl] = v;
  };
  const bool vec = ((uintptr_t)src % 16) == 0;
  if (vec) {
    for (int e = threadIdx.x * 4; e < ne; e += 256 * 4) {
      if (e + 4 <= ne) {
        const int4 w4 = *reinterpret_cast<const int4*>(src + e);
        put(e, dec(w4.x, e));
        put(e + 1, dec(w4.y, e + 1));
        put(e + 2, dec(w4.z, e + 2));
        put(e + 3, dec(w4.w, e + 3));
      } else {
        for (int q = e; q < ne; ++q) put(q, dec(src[q], q));
      }
    }
  } else {
    for (int e = threadIdx.x; e < ne; e += 256) put(e, dec(src[e], e));
  }
  __syncthreads();
  uint16_t* dst = wt + n * taps * Cin + c0;
  const bool v8 = (nc % 4) == 0 && (Cin % 4) == 0 && ((uintptr_t)wt % 8) == 0 && (c0 % 4) == 0;
  if (v8) {
    const int q4 = nc / 4;
    const bool full = nc == kTapC;   // q4 = 64: the split is a shift
    for (int e = threadIdx.x; e < q4 * taps; e += 256) {
      const int t = full ? e >> 6 : e / q4, cl = (e - t * q4) * 4;
      *reinterpret_cast<uint2*>(dst + (int64_t)t * Cin + cl) = *reinterpret_cast<const uint2*>(tl + t * kTapLd + cl);
    }
  } else {
    for (int e = threadIdx.x; e < ne; e += 256) {
      const int t = e / nc, cl = e - t * nc;
      dst[(int64_t)t * Cin + cl] = tl[t * kTapLd + cl];
    }
  }
}

// g[n][c * taps + t] = gt[n][t][c]: a conv gradient from the tap-major order
// of the implicit WGRAD back to the packed words' (c, tap) order.  Same
// blocking as weight_taps_kernel, with the LDS tile [kTapC][taps].
template <int TAPS>
__global__ __launch_bounds__(256) void grad_from_taps_kernel(const uint16_t* __restrict__ gt, int64_t Cin,
                                                             int taps_rt, uint16_t* __restrict__ g, int64_t ld_g) {
  extern __shared__ uint16_t tl[];   // [kTapC][taps]
  const int taps = TAPS ? TAPS : taps_rt;
  const int64_t n = blockIdx.y;
  const int64_t c0 = (int64_t)blockIdx.x * kTapC;
  const int nc = (int)min((int64_t)kTapC, Cin - c0);
  const int ne = nc * taps;
  const uint16_t* src = gt + n * taps * Cin + c0;
  const bool v8 = (nc % 4) == 0 && (Cin % 4) == 0 && ((uintptr_t)gt % 8) == 0 && (c0 % 4) == 0;
  if (v8) {
    const int q4 = nc / 4;
    const bool full = nc == kTapC;
    for (int e = threadIdx.x; e < q4 * taps; e += 256) {
      const int t = full ? e >> 6 : e / q4, cl = (e - t * q4) * 4;
      const uint2 v = *reinterpret_cast<const uint2*>(src + (int64_t)t * Cin + cl);
      tl[cl * taps + t] = (uint16_t)(v.x & 0xFFFFu);
      tl[(cl + 1) * taps + t] = (uint16_t)(v.x >> 16);
      tl[(cl + 2) * taps + t] = (uint16_t)(v.y & 0xFFFFu);
      tl[(cl + 3) * taps + t] = (uint16_t)(v.y >> 16);
    }
  } else {
    for (int e = threadIdx.x; e < ne; e += 256) {
      const int t = e / nc, cl = e - t * nc;
      tl[cl * taps + t] = src[(int64_t)t * Cin + cl];
    }
  }
  __syncthreads();
  uint16_t* dst = g + n * ld_g + c0 * taps;
  const bool w8 = (ne % 4) == 0 && ((uintptr_t)dst % 8) == 0;
  if (w8) {
    for (int e = threadIdx.x * 4; e < ne; e += 256 * 4)
      *reinterpret_cast<uint2*>(dst + e) = *reinterpret_cast<const uint2*>(tl + e);
  } else {
    for (int e = threadIdx.x; e < ne; e += 256) dst[e] = tl[e];
  }
}

// grad_from_taps_kernel and vhat_partials_kernel in one pass, for 3 x 3
// kernels (9 taps): a block takes 64 output channels n0 .. n0 + 63 and 64
// input channels c0 .. c0 + 63, i.e. the 64 x 576 block of the packed
// gradient g[n][c * 9 + t] whose columns start at 9 c0 (c0 and the channel
// counts are multiples of 64, so there are no edges).  It reads gt[n][t][c0 ..]
// (128-byte runs, 16 bytes per lane) and writes the values into LDS in the
// packed order, rows kTvLd apart; then it writes the packed rows with 16-byte
// stores and forms the v-hat partials of its nine 64 x 64 tiles of g exactly
// as vhat_partials_kernel does (vhat_tile.h order, the same bf16 values).
constexpr int kTvTaps = 9;
constexpr int kTvCols = 64 * kTvTaps;   // packed columns of a block
constexpr int kTvLd = kTvCols + 8;      // LDS row (halves): 16-byte rows, v-hat reads spread over the banks

__global__ __launch_bounds__(256) void taps_vhat_kernel(const uint16_t* __restrict__ gt, int64_t Cin,
                                                        uint16_t* __restrict__ g, int64_t ld_g, int64_t N,
                                                        float* __restrict__ pr, float* __restrict__ pc) {
  __shared__ __attribute__((aligned(16))) uint16_t tl[64 * kTvLd];   // [row][c * 9 + t]
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int64_t c0 = (int64_t)blockIdx.x * 64, n0 = (int64_t)blockIdx.y * 64;
  const int64_t K = Cin * kTvTaps;
  constexpr int RUNS = 8 * kTvTaps;     // 16-byte chunks per row: (t, 8-channel group)
  constexpr int PER = 64 * RUNS / 256;  // chunks per thread
  {
    uint4 v[PER];
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const int u = t + 256 * e;
      const int row = u / RUNS, rem = u - row * RUNS, tp = rem >> 3, ch = rem & 7;
      v[e] = *reinterpret_cast<const uint4*>(gt + (n0 + row) * K + tp * Cin + c0 + ch * 8);
    }
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const int u = t + 256 * e;
      const int row = u / RUNS, rem = u - row * RUNS, tp = rem >> 3, ch = rem & 7;
      uint16_t* d = tl + row * kTvLd + (ch * 8) * kTvTaps + tp;
      const uint32_t w[4] = {v[e].x, v[e].y, v[e].z, v[e].w};
#pragma unroll
      for (int k = 0; k < 8; ++k) d[k * kTvTaps] = (uint16_t)(w[k >> 1] >> (16 * (k & 1)));
    }
  }
  __syncthreads();
  // packed rows, 8 columns (16 bytes) per item
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    const int u = t + 256 * e;
    const int row = u / RUNS, kc = (u - row * RUNS) * 8;
    *reinterpret_cast<uint4*>(g + (n0 + row) * ld_g + c0 * kTvTaps + kc) =
        *reinterpret_cast<const uint4*>(tl + row * kTvLd + kc);
  }
  // v-hat partials: one wave per 64 x 64 tile (columns 64 jt .. of the block)
  const int p = lane & 15, q = lane >> 4;
  for (int jt = wave; jt < kTvTaps; jt += 4) {
    float g2[4][4][4];
#pragma unroll
    for (int x = 0; x < 4; ++x)
#pragma unroll
      for (int y = 0; y < 4; ++y) {
        const uint2 w = *reinterpret_cast<const uint2*>(tl + (16 * x + p) * kTvLd + 64 * jt + 16 * y + 4 * q);
        const float f[4] = {__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xFFFF0000u),
                            __uint_as_float(w.y << 16), __uint_as_float(w.y & 0xFFFF0000u)};
#pragma unroll
        for (int e = 0; e < 4; ++e) g2[x][y][e] = __fmul_rn(f[e], f[e]);
      }
    vhat_tile_partials(g2, lane, n0, c0 * kTvTaps + 64 * jt, N, K, pr, pc);
  }
}

constexpr size_t kCol2imLdsBudget = 64 * 1024;   // two blocks per CU

// staged rows and columns a block needs at most, and the channels per block
// that fit the LDS budget (cc = 0: the geometry does not fit)
static Col2imTile col2im_tile(const ConvGeom& g) {
  Col2imTile T;
  T.nho = (int)((kC2iH - 1 + g.kh - 1) / g.sh + 1);
  T.nwo = (int)((kC2iW - 1 + g.kw - 1) / g.sw + 1);
  const int kk = (int)(g.kh * g.kw);
  T.cc = 0;
  for (int cc = 16; cc >= 1; cc /= 2) {
    if (cc * kk > 3 * 64) continue;   // the staging moves at most 3 elements per lane per row
    int ld = cc * kk;
    // rows 8-byte aligned when the segment allows 8-byte staging, with a dword
    // stride of 2 mod 4 (2-way LDS bank conflicts in the gather at most);
    // otherwise an odd number of dwords per row
    if (ld % 4 == 0) {
      if ((ld / 2) % 4 != 2) ld += 4;
    } else if ((ld & 1) == 0 && ((ld / 2) & 1) == 0) {
      ld += 2;
    }
    if ((size_t)T.nho * T.nwo * ld * 2 <= kCol2imLdsBudget) {
      T.cc = cc;
      T.ld = ld;
      break;
    }
  }
  T.seg = T.cc * kk;
  return T;
}

}  // namespace concord

using namespace concord;

extern "C" int concord_conv_im2col(const uint16_t* x, int64_t B, int64_t C, int64_t H, int64_t W, int64_t kh,
                                   int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw, uint16_t* cols,
                                   void* stream) {
  CONCORD_CHECK(B >= 0 && C > 0 && H > 0 && W > 0 && kh > 0 && kw > 0 && sh > 0 && sw > 0 && ph >= 0 &&
                    pw >= 0,
                "concord_conv_im2col: bad geometry");
  CONCORD_CHECK(x && cols, "concord_conv_im2col: NULL argument");
  ConvGeom g{B, C, H, W, kh, kw, sh, sw, ph, pw, (H + 2 * ph - kh) / sh + 1, (W + 2 * pw - kw) / sw + 1,
             C * kh * kw};
  CONCORD_CHECK(H + 2 * ph >= kh && W + 2 * pw >= kw, "concord_conv_im2col: kernel larger than the image");
  CONCORD_CHECK(H + 2 * ph < ((int64_t)1 << 30) && W + 2 * pw < ((int64_t)1 << 30) && C * H * W < ((int64_t)1 << 40),
                "concord_conv_im2col: image too large");
  const int64_t M = B * g.Ho * g.Wo;
  CONCORD_CHECK(cdiv(M, kTileM) < ((int64_t)1 << 31) && cdiv(g.K, kTileK) <= kMaxGridY && B * C * H * W < ((int64_t)1 << 40),
                "concord_conv_im2col: size too large");
  if (M == 0) return CONCORD_OK;
  hipLaunchKernelGGL(im2col_kernel, dim3((unsigned)cdiv(M, kTileM), (unsigned)cdiv(g.K, kTileK)), dim3(256), 0,
                     (hipStream_t)stream, x, g, cols);
  return launch_status("conv_im2col");
}

extern "C" int concord_conv_col2im(const uint16_t* dcols, int64_t B, int64_t C, int64_t H, int64_t W, int64_t kh,
                                   int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw, uint16_t* dx,
                                   void* stream) {
  CONCORD_CHECK(B >= 0 && C > 0 && H > 0 && W > 0 && kh > 0 && kw > 0 && sh > 0 && sw > 0 && ph >= 0 &&
                    pw >= 0 && H + 2 * ph >= kh && W + 2 * pw >= kw,
                "concord_conv_col2im: bad geometry");
  CONCORD_CHECK(dcols && dx, "concord_conv_col2im: NULL argument");
  CONCORD_CHECK(H + 2 * ph < ((int64_t)1 << 30) && W + 2 * pw < ((int64_t)1 << 30) && B * C * H * W < ((int64_t)1 << 40),
                "concord_conv_col2im: image too large");
  ConvGeom g{B, C, H, W, kh, kw, sh, sw, ph, pw, (H + 2 * ph - kh) / sh + 1, (W + 2 * pw - kw) / sw + 1,
             C * kh * kw};
  const Col2imTile T = col2im_tile(g);
  if (B == 0) return CONCORD_OK;
  if (T.cc == 0) {
    // a window too large for the staged tile: the unstaged gather
    const int64_t total = B * C * H * W;
    hipLaunchKernelGGL(col2im_direct_kernel, dim3((unsigned)std::min<int64_t>(cdiv(total, 256), 65536)), dim3(256),
                       0, (hipStream_t)stream, dcols, g, dx);
    return launch_status("conv_col2im");
  }
  const int64_t gy = B * ((H + kC2iH - 1) / kC2iH);
  CONCORD_CHECK(gy <= kMaxGridY && cdiv(C, T.cc) <= kMaxGridY && cdiv(W, kC2iW) < ((int64_t)1 << 31),
                "concord_conv_col2im: grid too large (batch x rows / 4 must stay below 65536)");
  const size_t lds = (size_t)T.nho * T.nwo * T.ld * 2;
  hipLaunchKernelGGL(col2im_kernel, dim3((unsigned)cdiv(W, kC2iW), (unsigned)gy, (unsigned)cdiv(C, T.cc)),
                     dim3(256), lds, (hipStream_t)stream, dcols, g, T, dx);
  return launch_status("conv_col2im");
}

extern "C" int concord_conv_col2im_fits(int64_t kh, int64_t kw, int64_t sh, int64_t sw) {
  ConvGeom g{};
  g.kh = kh; g.kw = kw; g.sh = sh; g.sw = sw;
  return kh > 0 && kw > 0 && sh > 0 && sw > 0 && col2im_tile(g).cc > 0;
}

// ---- implicit-GEMM convolution entry points -----------------------------------
namespace concord {

struct ConvShape {
  int64_t B, Cin, H, W, Cout, kh, kw, sh, sw, ph, pw, Ho, Wo;
};

static bool conv_shape(int64_t B, int64_t Cin, int64_t H, int64_t W, int64_t Cout, int64_t kh, int64_t kw,
                       int64_t sh, int64_t sw, int64_t ph, int64_t pw, ConvShape& s) {
  if (!(B >= 0 && Cin > 0 && H > 0 && W > 0 && Cout > 0 && kh > 0 && kw > 0 && sh > 0 && sw > 0 && ph >= 0 &&
        pw >= 0 && H + 2 * ph >= kh && W + 2 * pw >= kw && H < (1 << 20) && W < (1 << 20) && kh < 64 && kw < 64))
    return false;
  s = ConvShape{B, Cin, H, W, Cout, kh, kw, sh, sw, ph, pw, (H + 2 * ph - kh) / sh + 1, (W + 2 * pw - kw) / sw + 1};
  return true;
}

// the implicit kernels take the shape: channels in 64-element stages, strides
// 1 or 2, positions below 2^24 (exact magic division), operands below 2^30
// bytes (32-bit buffer offsets)
static bool conv_implicit_shape(const ConvShape& s) {
  const int64_t lim = ((int64_t)1 << 24) - 64;
  return s.Cin % 64 == 0 && s.Cout % 64 == 0 && (s.sh == 1 || s.sh == 2) && (s.sw == 1 || s.sw == 2) &&
         s.kh * s.kw <= 64 &&
         s.B * s.H * s.W < lim && s.B * s.Ho * s.Wo < lim && s.B * s.H * s.W * s.Cin * 2 < ((int64_t)1 << 30) &&
         s.B * s.Ho * s.Wo * s.Cout * 2 < ((int64_t)1 << 30) &&
         s.Cout * s.kh * s.kw * s.Cin * 2 < ((int64_t)1 << 30);
}

// ConvIdx of one product: gathered activation (C channels on Hg x Wg), GEMM
// positions on Hr x Wr
static ConvIdx conv_idx(const ConvShape& s, int64_t C, int64_t Hg, int64_t Wg, int64_t Hr, int64_t Wr,
                        int64_t cb, int64_t act_bytes, int64_t w_bytes) {
  ConvIdx c{};
  c.C = (int32_t)C;
  c.Hg = (int32_t)Hg;
  c.Wg = (int32_t)Wg;
  c.Hr = (int32_t)Hr;
  c.Wr = (int32_t)Wr;
  c.kw = (int32_t)s.kw;
  c.ph = (int32_t)s.ph;
  c.pw = (int32_t)s.pw;
  c.slh = s.sh == 2 ? 1 : 0;
  c.slw = s.sw == 2 ? 1 : 0;
  c.cb = (int32_t)cb;
  conv_magic((uint32_t)Wr, c.mw, c.shw);
  conv_magic((uint32_t)Hr, c.mh, c.shh);
  c.act_bytes = (uint32_t)act_bytes;
  c.w_bytes = (uint32_t)w_bytes;
  return c;
}

static GemmArgs conv_args(const uint16_t* a, int64_t lda, const void* b, int64_t ldb, uint16_t* c, int64_t ldc,
                          int64_t I, int64_t J, int64_t R, const uint16_t* bias) {
  GemmArgs g{};
  g.a = a;
  g.b = b;
  g.lda = lda;
  g.ldb = ldb;
  g.c = c;
  g.ldc = ldc;
  g.I = I;
  g.J = J;
  g.R = R;
  g.vbias = bias;
  g.splits = 1;
  return g;
}

}  // namespace concord

#define CONV_GEOM_ARGS                                                                                      \
  int64_t B, int64_t Cin, int64_t H, int64_t W, int64_t Cout, int64_t kh, int64_t kw, int64_t sh, int64_t sw, \
      int64_t ph, int64_t pw

extern "C" int concord_conv_implicit_ok(CONV_GEOM_ARGS) {
  ConvShape s;
  return conv_shape(B, Cin, H, W, Cout, kh, kw, sh, sw, ph, pw, s) && conv_implicit_shape(s);
}

extern "C" size_t concord_conv_workspace_bytes(CONV_GEOM_ARGS) {
  ConvShape s;
  if (!conv_shape(B, Cin, H, W, Cout, kh, kw, sh, sw, ph, pw, s)) return kSplitkCounterBytes;
  const int64_t T = kh * kw, Mo = std::max<int64_t>(1, B * s.Ho * s.Wo), Mi = std::max<int64_t>(1, B * H * W);
  const size_t a = gemm_conv_partial_bytes(MODE_FWD_BF16, Mo, Cout, T * Cin);
  const size_t b = gemm_conv_partial_bytes(MODE_DGRAD_BF16, Mi, Cin, T * Cout);
  const size_t c = gemm_conv_partial_bytes(MODE_WGRAD, Cout, T * Cin, Mo);
  const size_t m = std::max(a, std::max(b, c));
  return kSplitkCounterBytes + ((m + 255) / 256) * 256;
}

extern "C" int concord_conv_weight_taps(const int32_t* packed, int64_t ld_p, const int8_t* row_exp,
                                        const int8_t* col_exp, int64_t Cout, int64_t Cin, int64_t taps,
                                        int32_t mantissa_bias, float fast_gain, uint16_t* wt, void* stream) {
  CONCORD_CHECK(Cout >= 0 && Cin > 0 && taps > 0 && taps <= 64 && Cout < (1LL << 31) && Cin * taps < (1LL << 31),
                "concord_conv_weight_taps: bad size (at most 64 taps)");
  if (Cout == 0) return CONCORD_OK;
  CONCORD_CHECK(packed && row_exp && col_exp && wt, "concord_conv_weight_taps: NULL argument");
  CONCORD_CHECK(ld_p >= Cin * taps, "concord_conv_weight_taps: leading dimension < in_channels * taps");
  CONCORD_CHECK(Cout <= kMaxGridY, "concord_conv_weight_taps: more than %lld output channels",
                (long long)kMaxGridY);
  const dim3 grid((unsigned)cdiv(Cin, kTapC), (unsigned)Cout);
  const size_t lds = (size_t)taps * kTapLd * 2;
  if (taps == 9)
    hipLaunchKernelGGL(weight_taps_kernel<9>, grid, dim3(256), lds, (hipStream_t)stream, packed, ld_p, row_exp,
                       col_exp, Cin, (int)taps, mantissa_bias, fast_gain, wt);
  else
    hipLaunchKernelGGL(weight_taps_kernel<0>, grid, dim3(256), lds, (hipStream_t)stream, packed, ld_p, row_exp,
                       col_exp, Cin, (int)taps, mantissa_bias, fast_gain, wt);
  return launch_status("conv_weight_taps");
}

extern "C" int concord_conv_grad_from_taps(const uint16_t* gt, int64_t Cout, int64_t Cin, int64_t taps, uint16_t* g,
                                           int64_t ld_g, void* stream) {
  CONCORD_CHECK(Cout >= 0 && Cin > 0 && taps > 0 && taps <= 64 && Cout < (1LL << 31) && Cin * taps < (1LL << 31),
                "concord_conv_grad_from_taps: bad size (at most 64 taps)");
  if (Cout == 0) return CONCORD_OK;
  CONCORD_CHECK(gt && g, "concord_conv_grad_from_taps: NULL argument");
  CONCORD_CHECK(ld_g >= Cin * taps, "concord_conv_grad_from_taps: leading dimension < in_channels * taps");
  CONCORD_CHECK(Cout <= kMaxGridY, "concord_conv_grad_from_taps: more than %lld output channels",
                (long long)kMaxGridY);
  const dim3 grid((unsigned)cdiv(Cin, kTapC), (unsigned)Cout);
  const size_t lds = (size_t)taps * kTapC * 2;
  if (taps == 9)
    hipLaunchKernelGGL(grad_from_taps_kernel<9>, grid, dim3(256), lds, (hipStream_t)stream, gt, Cin, (int)taps, g,
                       ld_g);
  else
    hipLaunchKernelGGL(grad_from_taps_kernel<0>, grid, dim3(256), lds, (hipStream_t)stream, gt, Cin, (int)taps, g,
                       ld_g);
  return launch_status("conv_grad_from_taps");
}

extern "C" int concord_conv_fwd(const uint16_t* x, const uint16_t* wt, const uint16_t* bias, uint16_t* y,
                                CONV_GEOM_ARGS, void* workspace, size_t workspace_bytes, void* stream) {
  ConvShape s;
  CONCORD_CHECK(conv_shape(B, Cin, H, W, Cout, kh, kw, sh, sw, ph, pw, s), "concord_conv_fwd: bad geometry");
  CONCORD_CHECK(conv_implicit_shape(s), "concord_conv_fwd: shape not taken by the implicit kernels "
                                        "(concord_conv_implicit_ok)");
  if (B == 0) return CONCORD_OK;
  CONCORD_CHECK(x && wt && y, "concord_conv_fwd: NULL argument");
  const int64_t T = kh * kw;
  GemmArgs g = conv_args(x, Cin, wt, T * Cin, y, Cout, B * s.Ho * s.Wo, Cout, T * Cin, bias);
  g.cv = conv_idx(s, Cin, H, W, s.Ho, s.Wo, Cin, B * H * W * Cin * 2, Cout * T * Cin * 2);
  const int rc = gemm_conv_launch(MODE_FWD_BF16, g, workspace, workspace_bytes, (hipStream_t)stream, "conv_fwd");
  CONCORD_CHECK(rc != -1, "concord_conv_fwd: operands not aligned for the implicit kernels (16-byte x and "
                          "weight, 8-byte y and bias)");
  return rc;
}

extern "C" int concord_conv_dgrad(const uint16_t* dy, const uint16_t* wt, uint16_t* dx, CONV_GEOM_ARGS,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  ConvShape s;
  CONCORD_CHECK(conv_shape(B, Cin, H, W, Cout, kh, kw, sh, sw, ph, pw, s), "concord_conv_dgrad: bad geometry");
  CONCORD_CHECK(conv_implicit_shape(s), "concord_conv_dgrad: shape not taken by the implicit kernels "
                                        "(concord_conv_implicit_ok)");
  if (B == 0) return CONCORD_OK;
  CONCORD_CHECK(dy && wt && dx, "concord_conv_dgrad: NULL argument");
  const int64_t T = kh * kw;
  GemmArgs g = conv_args(dy, Cout, wt, T * Cin, dx, Cin, B * H * W, Cin, T * Cout, nullptr);
  g.cv = conv_idx(s, Cout, s.Ho, s.Wo, H, W, Cin, B * s.Ho * s.Wo * Cout * 2, Cout * T * Cin * 2);
  const int rc = gemm_conv_launch(MODE_DGRAD_BF16, g, workspace, workspace_bytes, (hipStream_t)stream,
                                  "conv_dgrad");
  CONCORD_CHECK(rc != -1, "concord_conv_dgrad: operands not aligned for the implicit kernels");
  return rc;
}

extern "C" int concord_conv_wgrad(const uint16_t* dy, const uint16_t* x, uint16_t* gt, CONV_GEOM_ARGS,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  ConvShape s;
  CONCORD_CHECK(conv_shape(B, Cin, H, W, Cout, kh, kw, sh, sw, ph, pw, s), "concord_conv_wgrad: bad geometry");
  CONCORD_CHECK(conv_implicit_shape(s), "concord_conv_wgrad: shape not taken by the implicit kernels "
                                        "(concord_conv_implicit_ok)");
  CONCORD_CHECK(gt && (B == 0 || (dy && x)), "concord_conv_wgrad: NULL argument");
  const int64_t T = kh * kw;
  if (B == 0) {   // an empty batch: the sum over no positions
    fill_zero_bf16_launch(gt, T * Cin, Cout, T * Cin, (hipStream_t)stream);
    return launch_status("conv_wgrad");
  }
  GemmArgs g = conv_args(dy, Cout, x, T * Cin, gt, T * Cin, Cout, T * Cin, B * s.Ho * s.Wo, nullptr);
  g.cv = conv_idx(s, Cin, H, W, s.Ho, s.Wo, Cin, B * H * W * Cin * 2, 0);
  const int rc = gemm_conv_launch(MODE_WGRAD, g, workspace, workspace_bytes, (hipStream_t)stream, "conv_wgrad");
  CONCORD_CHECK(rc != -1, "concord_conv_wgrad: operands not aligned for the implicit kernels");
  return rc;
}

extern "C" int concord_conv_wgrad_vhat(const uint16_t* dy, const uint16_t* x, uint16_t* gt, uint16_t* grad_w,
                                       int64_t ld_gw, CONV_GEOM_ARGS, double beta2, float* v_row, float* v_col,
                                       float* sum_v_inv, int32_t* row_max, int32_t* col_max,
                                       int32_t* salt_counter, uint16_t* grad_bias, void* workspace,
                                       size_t workspace_bytes, void* gemm_workspace, size_t gemm_workspace_bytes,
                                       void* stream) {
  ConvShape s;
  CONCORD_CHECK(conv_shape(B, Cin, H, W, Cout, kh, kw, sh, sw, ph, pw, s),
                "concord_conv_wgrad_vhat: bad geometry");
  CONCORD_CHECK(conv_implicit_shape(s), "concord_conv_wgrad_vhat: shape not taken by the implicit kernels "
                                        "(concord_conv_implicit_ok)");
  CONCORD_CHECK(gt && grad_w && v_row && v_col && sum_v_inv && (B == 0 || (dy && x)),
                "concord_conv_wgrad_vhat: NULL argument");
  const int64_t T = kh * kw, N = Cout, K = T * Cin, M = B * s.Ho * s.Wo;
  CONCORD_CHECK(ld_gw >= K, "concord_conv_wgrad_vhat: leading dimension < in_channels * taps");
  CONCORD_CHECK(Cout <= kMaxGridY, "concord_conv_wgrad_vhat: more than %lld output channels", (long long)kMaxGridY);
  const hipStream_t st = (hipStream_t)stream;
  const Workspace ws = workspace_layout(N, K, grad_bias ? M : 0);
  CONCORD_CHECK(workspace && workspace_bytes >= ws.total, "concord_conv_wgrad_vhat: workspace of %zu bytes needed",
                ws.total);
  if (B == 0) {   // an empty batch: zero tap-major and packed-order gradients, then their v-hat EMA
    fill_zero_bf16_launch(gt, K, Cout, K, st);
    wgrad_vhat_empty_batch(grad_w, ld_gw, N, K, beta2, v_row, v_col, sum_v_inv, row_max, col_max, salt_counter,
                           grad_bias, workspace, st);
    return launch_status("conv_wgrad_vhat");
  }
  const VhatScratch v = vhat_scratch(N, K);
  float* pr = (float*)((char*)workspace + ws.scratch);
  float* pc = pr + v.pr;
  float* bsum = pc + v.pc;
  float* bpart = bsum + v.bsum;
  uint32_t* ticket = (uint32_t*)((char*)workspace + ws.vhat_ticket);
  // the product (tap-major gt), with the bias partials of dy when asked for
  GemmArgs g = conv_args(dy, Cout, x, K, gt, K, Cout, K, M, nullptr);
  g.cv = conv_idx(s, Cin, H, W, s.Ho, s.Wo, Cin, B * H * W * Cin * 2, 0);
  g.bpart = grad_bias ? bpart : nullptr;
  int bias_rows = 0;
  const int rc = gemm_conv_launch(MODE_WGRAD, g, gemm_workspace, gemm_workspace ? gemm_workspace_bytes : 0, st,
                                  "conv_wgrad_vhat", &bias_rows);
  CONCORD_CHECK(rc != -1, "concord_conv_wgrad_vhat: operands not aligned for the implicit kernels");
  if (rc != CONCORD_OK) return rc;
  // the packed-order gradient and its v-hat partials
  const bool fused = T == kTvTaps && ld_gw % 8 == 0 && ((uintptr_t)grad_w % 16) == 0 && ((uintptr_t)gt % 16) == 0;
  if (fused) {
    hipLaunchKernelGGL(taps_vhat_kernel, dim3((unsigned)(Cin / 64), (unsigned)(Cout / 64)), dim3(256), 0, st, gt,
                       Cin, grad_w, ld_gw, N, pr, pc);
  } else {
    const int rc2 = concord_conv_grad_from_taps(gt, Cout, Cin, T, grad_w, ld_gw, stream);
    if (rc2 != CONCORD_OK) return rc2;
    vhat_partials_launch(grad_w, ld_gw, N, K, pr, pc, st);
  }
  vhat_finish_launch(pr, pc, bsum, ticket, N, K, beta2, v_row, v_col, sum_v_inv, row_max, col_max, salt_counter,
                     st, bpart, bias_rows, grad_bias);
  return launch_status("conv_wgrad_vhat");
}
