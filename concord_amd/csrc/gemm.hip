// gemm.hip -- bf16 MFMA GEMMs of the packed linear layer on gfx950.
//
//   FWD        y [M,N] = x[M,K]  . W[N,K]^T   W = decode(packed)  (A6; concord/packed_b.py:1219)
//   DGRAD      dx[M,K] = dy[M,N] . W[N,K]                         (A7; concord/packed_b.py:1263)
//   WGRAD      gw[N,K] = dy[M,N]^T . x[M,K]                       (A5; concord/packed_b.py:1273)
//   FWD_BF16 / DGRAD_BF16: the same products over a materialised bf16 W
//   (the reference's cached weight_buf path).
//
// All are C[i][j] = sum_r A(i,r) B(r,j) with fp32 accumulation on
// v_mfma_f32_32x32x16_bf16.  Packed words are decoded to bf16 on the way into
// LDS: bf16(m_eff * 2^(row_exp + col_exp - bias)), bit-identical to the
// materialised weight.
//
// Block: 256 threads (4 waves as 2 x 2), tile 128 (i) x 128 (j) x 64 (r), LDS
// double-buffered, next tile's global loads in flight during the MFMAs.  Both
// LDS operands are stored r-contiguous ([i][r] and [j][r], 144 B row stride),
// so each lane's MFMA operand is one ds_read_b128.  Operands whose global
// layout is r-strided are transposed in registers in 8 (r) x 4 blocks.
#include "common.h"

namespace concord {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

enum { MODE_FWD = 0, MODE_DGRAD = 1, MODE_WGRAD = 2, MODE_FWD_BF16 = 3, MODE_DGRAD_BF16 = 4 };

constexpr int TI = 128, TJ = 128, TR = 64;
constexpr int LDS_STRIDE = 72;  // bf16 elements per LDS row (64 + 8 pad)
constexpr int LDS_TILE = 128 * LDS_STRIDE;

struct GemmArgs {
  const uint16_t* a;      // FWD: x[M,K]; DGRAD, WGRAD, *_BF16 dgrad: dy[M,N]
  const void* b;          // packed[N,K] int32 | x[M,K] bf16 (WGRAD) | W[N,K] bf16 (*_BF16)
  int64_t lda, ldb;
  const int8_t* row_exp;  // packed rows (n)
  const int8_t* col_exp;  // packed cols (k)
  int32_t bias;           // mantissa bias
  const uint16_t* vbias;  // bias[J] added in the epilogue, or NULL
  uint16_t* c;
  int64_t ldc;
  int64_t I, J, R;        // C is I x J, reduction R
};

CONCORD_DEV float decode_word(int32_t w, int32_t e) {
  const Fields f = unpack(w);
  return __fmul_rn((float)(f.ss * 128 + f.sf + f.vs * 128), exp2i(e));
}

// 8 rows (r) x 4 columns (2 dwords = 4 bf16 per row) -> 4 vectors of 8 consecutive r
CONCORD_DEV void transpose_8x4(const uint32_t (&in)[8][2], uint4 (&out)[4]) {
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int dw = c >> 1;
    const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
    uint32_t o[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) o[p] = __builtin_amdgcn_perm(in[2 * p + 1][dw], in[2 * p][dw], sel);
    out[c] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// ---- tile loaders -------------------------------------------------------------
// rows-copy: bf16 [rows][R] r-contiguous -> 4 x 16 B per thread
// (rows t/8 + 32q, r chunk (t%8)*8), stored to LDS [row][r].
struct RowsCopy {
  uint4 v[4];
  CONCORD_DEV void load(const uint16_t* base, int64_t ld, int64_t rows, int64_t R, int64_t i0,
                        int64_t r0, int t) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t i = i0 + t / 8 + 32 * q, r = r0 + (t % 8) * 8;
      const uint16_t* p = base + i * ld + r;
      if (i < rows && r + 8 <= R && (ld % 8) == 0) {
        v[q] = *reinterpret_cast<const uint4*>(p);
      } else {
        uint32_t w[4] = {0, 0, 0, 0};
        if (i < rows) {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (r + e < R) w[e / 2] |= (uint32_t)p[e] << (16 * (e & 1));
        }
        v[q] = make_uint4(w[0], w[1], w[2], w[3]);
      }
    }
  }
  CONCORD_DEV void store(uint16_t* lds, int t) const {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *reinterpret_cast<uint4*>(lds + (t / 8 + 32 * q) * LDS_STRIDE + (t % 8) * 8) = v[q];
  }
};

// transposed: bf16 [R][cols] col-contiguous -> thread owns 4 columns (4*(t%32))
// x 8 r (8*(t/32)), stored to LDS [col][r] as 4 x 16 B.
struct ColsTranspose {
  uint4 v[4];
  CONCORD_DEV void load(const uint16_t* base, int64_t ld, int64_t cols, int64_t R, int64_t c0,
                        int64_t r0, int t) {
    const int64_t c = c0 + 4 * (t % 32), rb = r0 + 8 * (t / 32);
    uint32_t blk[8][2];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int64_t r = rb + e;
      const uint16_t* p = base + r * ld + c;
      if (r < R && c + 4 <= cols && (ld % 4) == 0) {
        const uint2 w = *reinterpret_cast<const uint2*>(p);
        blk[e][0] = w.x;
        blk[e][1] = w.y;
      } else {
        uint32_t w[2] = {0, 0};
        if (r < R) {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (c + q < cols) w[q / 2] |= (uint32_t)p[q] << (16 * (q & 1));
        }
        blk[e][0] = w[0];
        blk[e][1] = w[1];
      }
    }
    transpose_8x4(blk, v);
  }
  CONCORD_DEV void store(uint16_t* lds, int t) const {
#pragma unroll
    for (int c = 0; c < 4; ++c)
      *reinterpret_cast<uint4*>(lds + (4 * (t % 32) + c) * LDS_STRIDE + 8 * (t / 32)) = v[c];
  }
};

// packed W as B(r=k, j=n) = W[n][k]: [J][R] r-contiguous.  thread -> rows
// t/16 + 16q (8 rows), r chunk (t%16)*4; decode with row_exp[n] + col_exp[k].
struct PackedRows {
  uint4 v[8];
  int32_t ce[4];
  int32_t re[8];  // row_exp - bias of the thread's 8 rows (fixed per block)
  CONCORD_DEV void init(const GemmArgs& g, int64_t j0, int t) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int64_t j = j0 + t / 16 + 16 * q;
      re[q] = ((j < g.J) ? (int32_t)g.row_exp[j] : 0) - g.bias;
    }
  }
  CONCORD_DEV void load(const GemmArgs& g, int64_t j0, int64_t r0, int t) {
    const int32_t* pk = reinterpret_cast<const int32_t*>(g.b);
    const int64_t r = r0 + (t % 16) * 4;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int64_t j = j0 + t / 16 + 16 * q;
      const int32_t* p = pk + j * g.ldb + r;
      if (j < g.J && r + 4 <= g.R && (g.ldb % 4) == 0) {
        v[q] = *reinterpret_cast<const uint4*>(p);
      } else {
        uint32_t w[4] = {0, 0, 0, 0};
        if (j < g.J) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (r + e < g.R) w[e] = (uint32_t)p[e];
        }
        v[q] = make_uint4(w[0], w[1], w[2], w[3]);
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) ce[e] = (r + e < g.R) ? (int32_t)g.col_exp[r + e] : 0;
  }
  CONCORD_DEV void store(uint16_t* lds, int t) const {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const uint4 w = v[q];
      uint2 o;
      o.x = pack_bf16x2(decode_word((int32_t)w.x, re[q] + ce[0]), decode_word((int32_t)w.y, re[q] + ce[1]));
      o.y = pack_bf16x2(decode_word((int32_t)w.z, re[q] + ce[2]), decode_word((int32_t)w.w, re[q] + ce[3]));
      *reinterpret_cast<uint2*>(lds + (t / 16 + 16 * q) * LDS_STRIDE + (t % 16) * 4) = o;
    }
  }
};

// packed W as B(r=n, j=k) = W[n][k]: [R][J] j-contiguous.  thread -> 4 columns
// 4*(t%32) x 8 rows 8*(t/32); decode, transpose, store [j][r].
struct PackedCols {
  uint4 v[8];
  int32_t re[8];
  int32_t ce[4];  // col_exp - bias of the thread's 4 columns (fixed per block)
  CONCORD_DEV void init(const GemmArgs& g, int64_t j0, int t) {
    const int64_t j = j0 + 4 * (t % 32);
#pragma unroll
    for (int c = 0; c < 4; ++c) ce[c] = ((j + c < g.J) ? (int32_t)g.col_exp[j + c] : 0) - g.bias;
  }
  CONCORD_DEV void load(const GemmArgs& g, int64_t j0, int64_t r0, int t) {
    const int32_t* pk = reinterpret_cast<const int32_t*>(g.b);
    const int64_t j = j0 + 4 * (t % 32), rb = r0 + 8 * (t / 32);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int64_t r = rb + e;
      const int32_t* p = pk + r * g.ldb + j;
      if (r < g.R && j + 4 <= g.J && (g.ldb % 4) == 0) {
        v[e] = *reinterpret_cast<const uint4*>(p);
      } else {
        uint32_t w[4] = {0, 0, 0, 0};
        if (r < g.R) {
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (j + c < g.J) w[c] = (uint32_t)p[c];
        }
        v[e] = make_uint4(w[0], w[1], w[2], w[3]);
      }
      re[e] = (r < g.R) ? (int32_t)g.row_exp[r] : 0;
    }
  }
  CONCORD_DEV void store(uint16_t* lds, int t) const {
    uint32_t blk[8][2];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint4 w = v[e];
      blk[e][0] = pack_bf16x2(decode_word((int32_t)w.x, re[e] + ce[0]), decode_word((int32_t)w.y, re[e] + ce[1]));
      blk[e][1] = pack_bf16x2(decode_word((int32_t)w.z, re[e] + ce[2]), decode_word((int32_t)w.w, re[e] + ce[3]));
    }
    uint4 o[4];
    transpose_8x4(blk, o);
#pragma unroll
    for (int c = 0; c < 4; ++c)
      *reinterpret_cast<uint4*>(lds + (4 * (t % 32) + c) * LDS_STRIDE + 8 * (t / 32)) = o[c];
  }
};

template <int MODE>
struct Tiles {
  RowsCopy ar;        // A for all but WGRAD
  ColsTranspose at;   // A for WGRAD
  PackedRows bpr;     // B for FWD
  PackedCols bpc;     // B for DGRAD
  ColsTranspose bt;   // B for WGRAD, DGRAD_BF16
  RowsCopy br;        // B for FWD_BF16

  CONCORD_DEV void init(const GemmArgs& g, int64_t j0, int t) {
    if (MODE == MODE_FWD) bpr.init(g, j0, t);
    if (MODE == MODE_DGRAD) bpc.init(g, j0, t);
  }
  CONCORD_DEV void load(const GemmArgs& g, int64_t i0, int64_t j0, int64_t r0, int t) {
    if (MODE == MODE_WGRAD) at.load(g.a, g.lda, g.I, g.R, i0, r0, t);
    else ar.load(g.a, g.lda, g.I, g.R, i0, r0, t);
    const uint16_t* bb = reinterpret_cast<const uint16_t*>(g.b);
    if (MODE == MODE_FWD) bpr.load(g, j0, r0, t);
    if (MODE == MODE_DGRAD) bpc.load(g, j0, r0, t);
    if (MODE == MODE_WGRAD || MODE == MODE_DGRAD_BF16) bt.load(bb, g.ldb, g.J, g.R, j0, r0, t);
    if (MODE == MODE_FWD_BF16) br.load(bb, g.ldb, g.J, g.R, j0, r0, t);
  }
  CONCORD_DEV void store(uint16_t* la, uint16_t* lb, int t) const {
    if (MODE == MODE_WGRAD) at.store(la, t);
    else ar.store(la, t);
    if (MODE == MODE_FWD) bpr.store(lb, t);
    if (MODE == MODE_DGRAD) bpc.store(lb, t);
    if (MODE == MODE_WGRAD || MODE == MODE_DGRAD_BF16) bt.store(lb, t);
    if (MODE == MODE_FWD_BF16) br.store(lb, t);
  }
};

template <int MODE>
__global__ __launch_bounds__(256, 2) void gemm_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[2][2][LDS_TILE];
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wi = wave >> 1, wj = wave & 1;
  const int64_t i0 = (int64_t)blockIdx.x * TI;
  const int64_t j0 = (int64_t)blockIdx.y * TJ;

  Tiles<MODE> T;
  T.init(g, j0, t);

  f32x16 acc[2][2];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[x][y][e] = 0.0f;

  const int64_t nr = (g.R + TR - 1) / TR;
  if (nr > 0) {
    T.load(g, i0, j0, 0, t);
    T.store(lds[0][0], lds[0][1], t);
  }
  __syncthreads();

  const int lrow = lane & 31, lk = (lane >> 5) * 8;
  for (int64_t rt = 0; rt < nr; ++rt) {
    const int cur = (int)(rt & 1);
    if (rt + 1 < nr) T.load(g, i0, j0, (rt + 1) * TR, t);
    const uint16_t* la = lds[cur][0];
    const uint16_t* lb = lds[cur][1];
#pragma unroll
    for (int kk = 0; kk < TR / 16; ++kk) {
      bf16x8 af[2], bfr[2];
#pragma unroll
      for (int x = 0; x < 2; ++x)
        af[x] = __builtin_bit_cast(
            bf16x8, *reinterpret_cast<const uint4*>(la + (wi * 64 + x * 32 + lrow) * LDS_STRIDE + kk * 16 + lk));
#pragma unroll
      for (int y = 0; y < 2; ++y)
        bfr[y] = __builtin_bit_cast(
            bf16x8, *reinterpret_cast<const uint4*>(lb + (wj * 64 + y * 32 + lrow) * LDS_STRIDE + kk * 16 + lk));
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int y = 0; y < 2; ++y)
          acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[x], bfr[y], acc[x][y], 0, 0, 0);
    }
    if (rt + 1 < nr) T.store(lds[cur ^ 1][0], lds[cur ^ 1][1], t);
    __syncthreads();
  }

  // epilogue: lane holds column j = lane % 32 and rows 8*(e/4) + 4*(lane/32) + e%4
#pragma unroll
  for (int y = 0; y < 2; ++y) {
    const int64_t j = j0 + wj * 64 + y * 32 + (lane & 31);
    if (j >= g.J) continue;
    const float bj = g.vbias ? bf16_to_f32(g.vbias[j]) : 0.0f;
#pragma unroll
    for (int x = 0; x < 2; ++x) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t i = i0 + wi * 64 + x * 32 + 8 * (e / 4) + 4 * (lane >> 5) + (e & 3);
        if (i < g.I) {
          const float v = __fadd_rn(acc[x][y][e], bj);
          g.c[i * g.ldc + j] = (uint16_t)(pack_bf16x2(v, 0.0f) & 0xFFFFu);
        }
      }
    }
  }
}

template <int MODE>
static int launch_gemm(const GemmArgs& g, hipStream_t st, const char* what) {
  if (g.I == 0 || g.J == 0) return CONCORD_OK;
  dim3 grid((unsigned)cdiv(g.I, TI), (unsigned)cdiv(g.J, TJ));
  hipLaunchKernelGGL(gemm_kernel<MODE>, grid, dim3(256), 0, st, g);
  return launch_status(what);
}

static bool sizes_ok(int64_t M, int64_t N, int64_t K) {
  return M >= 0 && N >= 0 && K >= 0 && M < (1LL << 31) && N < (1LL << 31) && K < (1LL << 31);
}

}  // namespace concord

using namespace concord;

extern "C" int concord_dqgemm_fwd(const uint16_t* x, int64_t ld_x, const int32_t* packed,
                                  int64_t ld_p, const int8_t* row_exp, const int8_t* col_exp,
                                  int32_t mantissa_bias, const uint16_t* bias, uint16_t* y,
                                  int64_t ld_y, int64_t M, int64_t N, int64_t K, void* stream) {
  CONCORD_CHECK(sizes_ok(M, N, K), "concord_dqgemm_fwd: bad size");
  if (M == 0 || N == 0) return CONCORD_OK;
  CONCORD_CHECK(x && packed && row_exp && col_exp && y, "concord_dqgemm_fwd: NULL argument");
  CONCORD_CHECK(ld_x >= K && ld_p >= K && ld_y >= N, "concord_dqgemm_fwd: bad leading dimension");
  GemmArgs g{x, packed, ld_x, ld_p, row_exp, col_exp, mantissa_bias, bias, y, ld_y, M, N, K};
  return launch_gemm<MODE_FWD>(g, (hipStream_t)stream, "dqgemm_fwd");
}

extern "C" int concord_dqgemm_dgrad(const uint16_t* dy, int64_t ld_dy, const int32_t* packed,
                                    int64_t ld_p, const int8_t* row_exp, const int8_t* col_exp,
                                    int32_t mantissa_bias, uint16_t* dx, int64_t ld_dx, int64_t M,
                                    int64_t N, int64_t K, void* stream) {
  CONCORD_CHECK(sizes_ok(M, N, K), "concord_dqgemm_dgrad: bad size");
  if (M == 0 || K == 0) return CONCORD_OK;
  CONCORD_CHECK(dy && packed && row_exp && col_exp && dx, "concord_dqgemm_dgrad: NULL argument");
  CONCORD_CHECK(ld_dy >= N && ld_p >= K && ld_dx >= K, "concord_dqgemm_dgrad: bad leading dimension");
  GemmArgs g{dy, packed, ld_dy, ld_p, row_exp, col_exp, mantissa_bias, nullptr, dx, ld_dx, M, K, N};
  return launch_gemm<MODE_DGRAD>(g, (hipStream_t)stream, "dqgemm_dgrad");
}

extern "C" int concord_wgrad(const uint16_t* dy, int64_t ld_dy, const uint16_t* x, int64_t ld_x,
                             uint16_t* grad_w, int64_t ld_gw, int64_t M, int64_t N, int64_t K,
                             void* stream) {
  CONCORD_CHECK(sizes_ok(M, N, K), "concord_wgrad: bad size");
  if (N == 0 || K == 0) return CONCORD_OK;
  CONCORD_CHECK(dy && x && grad_w, "concord_wgrad: NULL argument");
  CONCORD_CHECK(ld_dy >= N && ld_x >= K && ld_gw >= K, "concord_wgrad: bad leading dimension");
  GemmArgs g{dy, x, ld_dy, ld_x, nullptr, nullptr, 0, nullptr, grad_w, ld_gw, N, K, M};
  return launch_gemm<MODE_WGRAD>(g, (hipStream_t)stream, "wgrad");
}

extern "C" int concord_gemm_bf16_fwd(const uint16_t* x, int64_t ld_x, const uint16_t* w,
                                     int64_t ld_w, const uint16_t* bias, uint16_t* y, int64_t ld_y,
                                     int64_t M, int64_t N, int64_t K, void* stream) {
  CONCORD_CHECK(sizes_ok(M, N, K), "concord_gemm_bf16_fwd: bad size");
  if (M == 0 || N == 0) return CONCORD_OK;
  CONCORD_CHECK(x && w && y, "concord_gemm_bf16_fwd: NULL argument");
  CONCORD_CHECK(ld_x >= K && ld_w >= K && ld_y >= N, "concord_gemm_bf16_fwd: bad leading dimension");
  GemmArgs g{x, w, ld_x, ld_w, nullptr, nullptr, 0, bias, y, ld_y, M, N, K};
  return launch_gemm<MODE_FWD_BF16>(g, (hipStream_t)stream, "gemm_bf16_fwd");
}

extern "C" int concord_gemm_bf16_dgrad(const uint16_t* dy, int64_t ld_dy, const uint16_t* w,
                                       int64_t ld_w, uint16_t* dx, int64_t ld_dx, int64_t M,
                                       int64_t N, int64_t K, void* stream) {
  CONCORD_CHECK(sizes_ok(M, N, K), "concord_gemm_bf16_dgrad: bad size");
  if (M == 0 || K == 0) return CONCORD_OK;
  CONCORD_CHECK(dy && w && dx, "concord_gemm_bf16_dgrad: NULL argument");
  CONCORD_CHECK(ld_dy >= N && ld_w >= K && ld_dx >= K, "concord_gemm_bf16_dgrad: bad leading dimension");
  GemmArgs g{dy, w, ld_dy, ld_w, nullptr, nullptr, 0, nullptr, dx, ld_dx, M, K, N};
  return launch_gemm<MODE_DGRAD_BF16>(g, (hipStream_t)stream, "gemm_bf16_dgrad");
}
