// gemm.hip -- bf16 MFMA GEMMs of the packed linear layer on gfx950.
//
//   FWD        y [M,N] = x[M,K]  . W[N,K]^T   W = decode(packed)  (A6; concord/packed_b.py:1219)
//   DGRAD      dx[M,K] = dy[M,N] . W[N,K]                         (A7; concord/packed_b.py:1263)
//   WGRAD      gw[N,K] = dy[M,N]^T . x[M,K]                       (A5; concord/packed_b.py:1273)
//   FWD_BF16 / DGRAD_BF16: the same products over a materialised bf16 W
//   (the reference's cached weight_buf path).
//
// All are C[i][j] = sum_r A(i,r) B(r,j), fp32 accumulation on
// v_mfma_f32_16x16x32_bf16.  Packed words are decoded to bf16 on the way into
// LDS, bf16(m_eff * 2^(row_exp + col_exp - bias)): bit-identical to the
// materialised weight.
//
// Block = 256 threads (4 waves).  Tile BI x BJ x 64, LDS double-buffered
// ([i][r] and [j][r], r-contiguous, 144 B row stride: each MFMA operand is one
// conflict-free ds_read_b128), next tile's global loads in flight during the
// MFMAs.  The MFMA computes C^T blocks (its A operand is the j-tile), so each
// lane holds 4 consecutive j of one i: one 8-byte store per block.
// Tile shapes are picked per problem so that about one tile lands on each of
// the 256 CUs; a too-small grid is split 2-way along r with a deterministic
// fixup (the second finisher adds the first's fp32 partial: a + b = b + a).
// Tiles are mapped XCD-aware: workgroup w runs on XCD w % 8, and each XCD
// gets a compact block of the tile grid so its L2 serves shared operands.
#include "gemm.h"
#include "update_fast.h"
#include "vhat.h"
#include "wgrad_update.h"
#include "workspace.h"

namespace concord {

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

// ---- tile loaders (256 threads; work split in chunks, ceil(chunks / 256) each) ----

// bf16 [rows][R] r-contiguous -> LDS [row][r]; chunk = 8 bf16 (16 B)
template <int ROWS>
struct RowsCopy {
  static constexpr int NCH = ROWS * (TR / 8);
  static constexpr int PER = (NCH + 255) / 256;
  uint4 v[PER];
  CONCORD_DEV void load(const uint16_t* base, int64_t ld, int64_t nrows, int64_t i0, int64_t r0,
                        int64_t r_end, int t, int vec) {
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int ch = t + 256 * q;
      const int64_t i = i0 + ch / 8, r = r0 + (ch % 8) * 8;
      const uint16_t* p = base + i * ld + r;
      uint32_t w[4] = {0, 0, 0, 0};
      if (ch < NCH && i < nrows) {
        if (r + 8 <= r_end && vec) {
          const uint4 x = *reinterpret_cast<const uint4*>(p);
          w[0] = x.x; w[1] = x.y; w[2] = x.z; w[3] = x.w;
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (r + e < r_end) w[e / 2] |= (uint32_t)p[e] << (16 * (e & 1));
        }
      }
      v[q] = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
  CONCORD_DEV void store(uint16_t* lds, int t) const {
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int ch = t + 256 * q;
      if (ch < NCH) *reinterpret_cast<uint4*>(lds + (ch / 8) * LDS_STRIDE + (ch % 8) * 8) = v[q];
    }
  }
};

// bf16 [R][cols] col-contiguous -> LDS [col][r]; block = 8 r x 4 cols
template <int COLS>
struct ColsTranspose {
  static constexpr int NB = (TR / 8) * (COLS / 4);
  static constexpr int PER = (NB + 255) / 256;
  uint4 v[PER][4];
  CONCORD_DEV void load(const uint16_t* base, int64_t ld, int64_t ncols, int64_t c0, int64_t r0,
                        int64_t r_end, int t, int vec) {
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int b = t + 256 * q;
      const int64_t c = c0 + 4 * (b % (COLS / 4)), rb = r0 + 8 * (b / (COLS / 4));
      uint32_t blk[8][2];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int64_t r = rb + e;
        const uint16_t* p = base + r * ld + c;
        uint32_t w[2] = {0, 0};
        if (b < NB && r < r_end) {
          if (c + 4 <= ncols && vec) {
            const uint2 x = *reinterpret_cast<const uint2*>(p);
            w[0] = x.x; w[1] = x.y;
          } else {
#pragma unroll
            for (int q2 = 0; q2 < 4; ++q2)
              if (c + q2 < ncols) w[q2 / 2] |= (uint32_t)p[q2] << (16 * (q2 & 1));
          }
        }
        blk[e][0] = w[0];
        blk[e][1] = w[1];
      }
      transpose_8x4(blk, v[q]);
    }
  }
  CONCORD_DEV void store(uint16_t* lds, int t) const {
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int b = t + 256 * q;
      if (b < NB) {
        const int c = 4 * (b % (COLS / 4)), r = 8 * (b / (COLS / 4));
#pragma unroll
        for (int k = 0; k < 4; ++k) *reinterpret_cast<uint4*>(lds + (c + k) * LDS_STRIDE + r) = v[q][k];
      }
    }
  }
};

// packed W as B(r=k, j=n): [J][R] r-contiguous; chunk = 4 words
template <int ROWS>
struct PackedRows {
  static constexpr int NCH = ROWS * (TR / 4);
  static constexpr int PER = (NCH + 255) / 256;
  uint4 v[PER];
  int32_t re[PER];  // row exponent - bias per chunk
  int32_t ce[4];    // column exponents: ch % 16 == t % 16 for every chunk of a thread
  CONCORD_DEV void load(const GemmArgs& g, int64_t j0, int64_t r0, int64_t r_end, int t) {
    const int32_t* pk = reinterpret_cast<const int32_t*>(g.b);
    const int64_t r = r0 + (t % 16) * 4;
#pragma unroll
    for (int k = 0; k < 4; ++k) ce[k] = (r + k < r_end) ? (int32_t)g.col_exp[r + k] : 0;
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int ch = t + 256 * q;
      const int64_t j = j0 + ch / 16;
      const int32_t* p = pk + j * g.ldb + r;
      uint32_t w[4] = {0, 0, 0, 0};
      int32_t e = 0;
      if (ch < NCH && j < g.J) {
        e = (int32_t)g.row_exp[j];
        if (r + 4 <= r_end && g.vec_b) {
          const uint4 x = *reinterpret_cast<const uint4*>(p);
          w[0] = x.x; w[1] = x.y; w[2] = x.z; w[3] = x.w;
        } else {
#pragma unroll
          for (int k = 0; k < 4; ++k)
            if (r + k < r_end) w[k] = (uint32_t)p[k];
        }
      }
      v[q] = make_uint4(w[0], w[1], w[2], w[3]);
      re[q] = e - g.bias;
    }
  }
  CONCORD_DEV void store(uint16_t* lds, int t) const {
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int ch = t + 256 * q;
      if (ch < NCH) {
        uint2 o;
        o.x = pack_bf16x2(decode_word((int32_t)v[q].x, re[q] + ce[0]), decode_word((int32_t)v[q].y, re[q] + ce[1]));
        o.y = pack_bf16x2(decode_word((int32_t)v[q].z, re[q] + ce[2]), decode_word((int32_t)v[q].w, re[q] + ce[3]));
        *reinterpret_cast<uint2*>(lds + (ch / 16) * LDS_STRIDE + (ch % 16) * 4) = o;
      }
    }
  }
};

// packed W as B(r=n, j=k): [R][J] j-contiguous; block = 8 r x 4 cols
template <int COLS>
struct PackedCols {
  static constexpr int NB = (TR / 8) * (COLS / 4);
  static constexpr int PER = (NB + 255) / 256;
  uint4 v[PER][8];
  int32_t re[PER][8];
  int32_t ce[PER][4];
  CONCORD_DEV void load(const GemmArgs& g, int64_t j0, int64_t r0, int64_t r_end, int t) {
    const int32_t* pk = reinterpret_cast<const int32_t*>(g.b);
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int b = t + 256 * q;
      const int64_t j = j0 + 4 * (b % (COLS / 4)), rb = r0 + 8 * (b / (COLS / 4));
#pragma unroll
      for (int c = 0; c < 4; ++c)
        ce[q][c] = ((b < NB && j + c < g.J) ? (int32_t)g.col_exp[j + c] : 0) - g.bias;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int64_t r = rb + e;
        const int32_t* p = pk + r * g.ldb + j;
        uint32_t w[4] = {0, 0, 0, 0};
        int32_t rexp = 0;
        if (b < NB && r < r_end) {
          rexp = (int32_t)g.row_exp[r];
          if (j + 4 <= g.J && g.vec_b) {
            const uint4 x = *reinterpret_cast<const uint4*>(p);
            w[0] = x.x; w[1] = x.y; w[2] = x.z; w[3] = x.w;
          } else {
#pragma unroll
            for (int c = 0; c < 4; ++c)
              if (j + c < g.J) w[c] = (uint32_t)p[c];
          }
        }
        v[q][e] = make_uint4(w[0], w[1], w[2], w[3]);
        re[q][e] = rexp;
      }
    }
  }
  CONCORD_DEV void store(uint16_t* lds, int t) const {
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int b = t + 256 * q;
      if (b < NB) {
        uint32_t blk[8][2];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          blk[e][0] = pack_bf16x2(decode_word((int32_t)v[q][e].x, re[q][e] + ce[q][0]),
                                  decode_word((int32_t)v[q][e].y, re[q][e] + ce[q][1]));
          blk[e][1] = pack_bf16x2(decode_word((int32_t)v[q][e].z, re[q][e] + ce[q][2]),
                                  decode_word((int32_t)v[q][e].w, re[q][e] + ce[q][3]));
        }
        uint4 o[4];
        transpose_8x4(blk, o);
        const int c = 4 * (b % (COLS / 4)), r = 8 * (b / (COLS / 4));
#pragma unroll
        for (int k = 0; k < 4; ++k) *reinterpret_cast<uint4*>(lds + (c + k) * LDS_STRIDE + r) = o[k];
      }
    }
  }
};

// A operand loader (i side) and B operand loader (j side) per mode
template <int MODE, int BI> struct ALoad;
template <int BI> struct ALoad<MODE_FWD, BI> : RowsCopy<BI> {};
template <int BI> struct ALoad<MODE_DGRAD, BI> : RowsCopy<BI> {};
template <int BI> struct ALoad<MODE_FWD_BF16, BI> : RowsCopy<BI> {};
template <int BI> struct ALoad<MODE_DGRAD_BF16, BI> : RowsCopy<BI> {};
template <int BI> struct ALoad<MODE_WGRAD, BI> : ColsTranspose<BI> {};

template <int MODE, int BI, int BJ>
struct Tiles {
  ALoad<MODE, BI> a;
  PackedRows<BJ> bpr;       // FWD
  PackedCols<BJ> bpc;       // DGRAD
  ColsTranspose<BJ> bt;     // WGRAD, DGRAD_BF16
  RowsCopy<BJ> br;          // FWD_BF16

  CONCORD_DEV void load(const GemmArgs& g, int64_t i0, int64_t j0, int64_t r0, int64_t r_end, int t) {
    a.load(g.a, g.lda, g.I, i0, r0, r_end, t, g.vec_a);
    const uint16_t* bb = reinterpret_cast<const uint16_t*>(g.b);
    if (MODE == MODE_FWD) bpr.load(g, j0, r0, r_end, t);
    if (MODE == MODE_DGRAD) bpc.load(g, j0, r0, r_end, t);
    if (MODE == MODE_WGRAD || MODE == MODE_DGRAD_BF16) bt.load(bb, g.ldb, g.J, j0, r0, r_end, t, g.vec_b);
    if (MODE == MODE_FWD_BF16) br.load(bb, g.ldb, g.J, j0, r0, r_end, t, g.vec_b);
  }
  CONCORD_DEV void store(uint16_t* la, uint16_t* lb, int t) const {
    a.store(la, t);
    if (MODE == MODE_FWD) bpr.store(lb, t);
    if (MODE == MODE_DGRAD) bpc.store(lb, t);
    if (MODE == MODE_WGRAD || MODE == MODE_DGRAD_BF16) bt.store(lb, t);
    if (MODE == MODE_FWD_BF16) br.store(lb, t);
  }
};

template <int MODE, int BI, int BJ, int WI, int WJ>
__global__ __launch_bounds__(256, 1) void gemm_kernel(GemmArgs g) {
  constexpr int WTI = BI / WI, WTJ = BJ / WJ;   // wave tile
  constexpr int NI = WTI / 16, NJ = WTJ / 16;   // 16x16 blocks per wave
  static_assert(WI * WJ == 4, "4 waves");
  static_assert(WTI % 16 == 0 && WTJ % 16 == 0, "wave tile must be a multiple of 16");
  __shared__ __attribute__((aligned(16))) uint16_t lds_a[2][BI * LDS_STRIDE];
  __shared__ __attribute__((aligned(16))) uint16_t lds_b[2][BJ * LDS_STRIDE];
  __shared__ uint32_t s_old;

  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wi = wave / WJ, wj = wave % WJ;
  const int tiles = g.tiles_i * g.tiles_j;
  const int wg = blockIdx.x;
  const int split = wg / tiles;
  int bi, bj;
  tile_of(wg % tiles, g.tiles_i, g.tiles_j, tiles, bi, bj);
  const int64_t i0 = (int64_t)bi * BI, j0 = (int64_t)bj * BJ;
  const int64_t r_begin = (int64_t)split * g.r_split;
  const int64_t r_end = min(g.R, r_begin + g.r_split);

  Tiles<MODE, BI, BJ> T;
  f32x4 acc[NI][NJ];
#pragma unroll
  for (int x = 0; x < NI; ++x)
#pragma unroll
    for (int y = 0; y < NJ; ++y) acc[x][y] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int64_t nr = (r_end > r_begin) ? (r_end - r_begin + TR - 1) / TR : 0;
  if (nr > 0) {
    T.load(g, i0, j0, r_begin, r_end, t);
    T.store(lds_a[0], lds_b[0], t);
  }
  __syncthreads();

  const int lrow = lane & 15, lk = (lane >> 4) * 8;
  for (int64_t rt = 0; rt < nr; ++rt) {
    const int cur = (int)(rt & 1);
    if (rt + 1 < nr) T.load(g, i0, j0, r_begin + (rt + 1) * TR, r_end, t);
    const uint16_t* la = lds_a[cur];
    const uint16_t* lb = lds_b[cur];
#pragma unroll
    for (int kk = 0; kk < TR / 32; ++kk) {
      bf16x8 fa[NI], fb[NJ];
#pragma unroll
      for (int x = 0; x < NI; ++x)
        fa[x] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(
                                               la + (wi * WTI + x * 16 + lrow) * LDS_STRIDE + kk * 32 + lk));
#pragma unroll
      for (int y = 0; y < NJ; ++y)
        fb[y] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(
                                               lb + (wj * WTJ + y * 16 + lrow) * LDS_STRIDE + kk * 32 + lk));
      // D^T: MFMA rows = j (from the B tile), columns = i (from the A tile)
#pragma unroll
      for (int x = 0; x < NI; ++x)
#pragma unroll
        for (int y = 0; y < NJ; ++y)
          acc[x][y] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[y], fa[x], acc[x][y], 0, 0, 0);
    }
    if (rt + 1 < nr) T.store(lds_a[cur ^ 1], lds_b[cur ^ 1], t);
    __syncthreads();
  }

  // lane holds C[i0 + wi*WTI + x*16 + lane%16][j0 + wj*WTJ + y*16 + 4*(lane/16) + e], e = 0..3
  const int64_t ib = i0 + wi * WTI + (lane & 15);
  const int64_t jb = j0 + wj * WTJ + 4 * (lane >> 4);
  if (g.splits == 2) {
    // deterministic 2-way fixup: both halves publish, the second finisher sums
    float* mine = g.part + (int64_t)split * g.I * g.J;
    const float* other = g.part + (int64_t)(split ^ 1) * g.I * g.J;
#pragma unroll
    for (int x = 0; x < NI; ++x)
#pragma unroll
      for (int y = 0; y < NJ; ++y) {
        const int64_t i = ib + x * 16, j = jb + y * 16;
        if (i < g.I)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (j + e < g.J) mine[i * g.J + j + e] = acc[x][y][e];
      }
    __threadfence();
    __syncthreads();
    if (t == 0) s_old = atomicAdd(g.tile_cnt + (wg % tiles), 1u);
    __syncthreads();
    if (s_old == 0) return;
    __threadfence();
#pragma unroll
    for (int x = 0; x < NI; ++x)
#pragma unroll
      for (int y = 0; y < NJ; ++y) {
        const int64_t i = ib + x * 16, j = jb + y * 16;
        if (i < g.I)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (j + e < g.J) acc[x][y][e] = __fadd_rn(acc[x][y][e], other[i * g.J + j + e]);
      }
    if (t == 0) g.tile_cnt[wg % tiles] = 0u;
  }
#pragma unroll
  for (int x = 0; x < NI; ++x) {
    const int64_t i = ib + x * 16;
    if (i >= g.I) continue;
#pragma unroll
    for (int y = 0; y < NJ; ++y) {
      const int64_t j = jb + y * 16;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float bj = (g.vbias && j + e < g.J) ? bf16_to_f32(g.vbias[j + e]) : 0.0f;
        v[e] = __fadd_rn(acc[x][y][e], bj);
      }
      uint16_t* out = g.c + i * g.ldc + j;
      if (j + 4 <= g.J && g.vec_c) {
        *reinterpret_cast<uint2*>(out) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (j + e < g.J) out[e] = (uint16_t)(pack_bf16x2(v[e], 0.0f) & 0xFFFFu);
      }
    }
  }
}

// ---- tile shape selection -------------------------------------------------------
enum Shape { SH_256x160 = 0, SH_128x160 = 1, SH_160x160 = 2, SH_128x128 = 3 };
struct ShapeDims { int bi, bj; };
static const ShapeDims kShapes[4] = {{256, 160}, {128, 160}, {160, 160}, {128, 128}};
constexpr int kCUs = 256;

struct Plan {
  int shape, splits, ti, tj;
  int64_t r_split;
};

// Estimated time ~ waves of tiles x work per tile (plus a fixup charge for a
// split), over the four shapes and splits {1, 2}.
static Plan plan_gemm(int64_t I, int64_t J, int64_t R, bool allow_split) {
  Plan best{SH_128x128, 1, 0, 0, R};
  double best_cost = 1e300;
  for (int s = 0; s < 4; ++s) {
    for (int sp = 1; sp <= (allow_split ? 2 : 1); ++sp) {
      const int64_t ti = cdiv(I, kShapes[s].bi), tj = cdiv(J, kShapes[s].bj);
      const int64_t blocks = ti * tj * sp;
      const int64_t rs = cdiv(cdiv(R, sp), TR) * TR;
      const double waves = (double)cdiv(blocks, kCUs);
      const double eff = (kShapes[s].bi * kShapes[s].bj >= 256 * 160) ? 1.0
                         : (kShapes[s].bi * kShapes[s].bj >= 160 * 160) ? 0.93 : 0.85;
      double cost = waves * (double)kShapes[s].bi * kShapes[s].bj * (double)rs / eff;
      if (sp == 2) cost += 2.0 * (double)I * J * 4.0 / 64.0;   // fixup traffic
      if (cost < best_cost) {
        best_cost = cost;
        best = Plan{s, sp, (int)ti, (int)tj, rs};
      }
    }
  }
  return best;
}

template <int MODE>
static int launch_gemm(GemmArgs g, void* workspace, size_t ws_bytes, hipStream_t st,
                       const char* what) {
  if (g.I == 0 || g.J == 0) return CONCORD_OK;
  const int fast = gemm_fast_launch(MODE, g, workspace, ws_bytes, st, what);
  if (fast != -1) return fast;
  const bool can_split = workspace != nullptr;
  Plan p = plan_gemm(g.I, g.J, g.R, can_split);
  if (p.splits == 2 &&
      (ws_bytes < gemm_splitk_bytes(g.I, g.J) || !gemm_splitk_fits((int64_t)p.ti * p.tj)))
    p = plan_gemm(g.I, g.J, g.R, false);
  g.splits = p.splits;
  g.r_split = p.r_split;
  g.tiles_i = p.ti;
  g.tiles_j = p.tj;
  if (p.splits == 2) {
    char* base = (char*)workspace;
    g.tile_cnt = (uint32_t*)base;
    g.part = (float*)(base + kSplitkCounterBytes);
  }
  const dim3 grid((unsigned)((int64_t)p.ti * p.tj * p.splits)), block(256);
  switch (p.shape) {
    case SH_256x160: hipLaunchKernelGGL((gemm_kernel<MODE, 256, 160, 4, 1>), grid, block, 0, st, g); break;
    case SH_128x160: hipLaunchKernelGGL((gemm_kernel<MODE, 128, 160, 2, 2>), grid, block, 0, st, g); break;
    case SH_160x160: hipLaunchKernelGGL((gemm_kernel<MODE, 160, 160, 2, 2>), grid, block, 0, st, g); break;
    default: hipLaunchKernelGGL((gemm_kernel<MODE, 128, 128, 2, 2>), grid, block, 0, st, g); break;
  }
  return launch_status(what);
}

static bool sizes_ok(int64_t M, int64_t N, int64_t K) {
  return M >= 0 && N >= 0 && K >= 0 && M < (1LL << 31) && N < (1LL << 31) && K < (1LL << 31);
}

static GemmArgs make_args(const uint16_t* a, const void* b, int64_t lda, int64_t ldb,
                          const int8_t* re, const int8_t* ce, int32_t bias, const uint16_t* vb,
                          uint16_t* c, int64_t ldc, int64_t I, int64_t J, int64_t R, bool b_packed) {
  GemmArgs g{};
  g.a = a; g.b = b; g.lda = lda; g.ldb = ldb; g.row_exp = re; g.col_exp = ce; g.bias = bias;
  g.vbias = vb; g.c = c; g.ldc = ldc; g.I = I; g.J = J; g.R = R;
  auto al = [](const void* p, int n) { return ((uintptr_t)p % n) == 0; };
  g.vec_a = al(a, 16) && (lda % 8) == 0;
  g.vec_b = al(b, 16) && (ldb % (b_packed ? 4 : 8)) == 0;
  g.vec_c = al(c, 8) && (ldc % 4) == 0;
  return g;
}

}  // namespace concord

using namespace concord;

// split-K partial bytes one GEMM may use (fast or generic kernel), 0 if unsplit
static size_t splitk_partials(int mode, int64_t I, int64_t J, int64_t R) {
  const size_t fast = gemm_fast_partial_bytes(mode, I, J, R);
  const size_t generic = plan_gemm(I, J, R, true).splits > 1 ? (size_t)2 * I * J * sizeof(float) : 0;
  return fast > generic ? fast : generic;
}

namespace concord {

int gemm_bf16_run(int mode, const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb, uint16_t* c,
                  int64_t ldc, int64_t I, int64_t J, int64_t R, void* ws, size_t ws_bytes, hipStream_t st,
                  const char* what) {
  GemmArgs g = make_args(a, b, lda, ldb, nullptr, nullptr, 0, nullptr, c, ldc, I, J, R, false);
  if (mode == MODE_FWD_BF16) return launch_gemm<MODE_FWD_BF16>(g, ws, ws_bytes, st, what);
  if (mode == MODE_DGRAD_BF16) return launch_gemm<MODE_DGRAD_BF16>(g, ws, ws_bytes, st, what);
  if (mode == MODE_WGRAD) return launch_gemm<MODE_WGRAD>(g, ws, ws_bytes, st, what);
  set_error("%s: unsupported product", what);
  return CONCORD_EINVAL;
}

int gemm_bf16_combine(int mode, const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb, uint16_t* c,
                      int64_t ldc, int64_t I, int64_t J, int64_t R, const uint16_t* y, int64_t ldy, float s,
                      float t, void* ws, size_t ws_bytes, hipStream_t st, const char* what) {
  if (mode != MODE_FWD_BF16 && mode != MODE_DGRAD_BF16) return -1;
  if (I == 0 || J == 0) return CONCORD_OK;
  GemmArgs g = make_args(a, b, lda, ldb, nullptr, nullptr, 0, nullptr, c, ldc, I, J, R, false);
  g.ay = y;
  g.ldy = ldy;
  g.as = s;
  g.at = t;
  return gemm_fast_launch(mode, g, ws, ws_bytes, st, what);
}

size_t gemm_splitk_need(int mode, int64_t I, int64_t J, int64_t R) {
  return kSplitkCounterBytes + ((splitk_partials(mode, I, J, R) + 255) / 256) * 256;
}

}  // namespace concord

extern "C" size_t concord_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  // tile counters + the split-K partials of the largest need among the layer's
  // three products: y [M,N] (reduce K), dx [M,K] (reduce N), gw [N,K] (reduce M)
  if (M < 1) M = 1;
  if (N < 1) N = 1;
  if (K < 1) K = 1;
  const size_t a = splitk_partials(MODE_FWD, M, N, K), b = splitk_partials(MODE_DGRAD, M, K, N),
               c = splitk_partials(MODE_WGRAD, N, K, M);
  const size_t m = a > b ? (a > c ? a : c) : (b > c ? b : c);
  return kSplitkCounterBytes + ((m + 255) / 256) * 256;
}

extern "C" int concord_dqgemm_fwd(const uint16_t* x, int64_t ld_x, const int32_t* packed,
                                  int64_t ld_p, const int8_t* row_exp, const int8_t* col_exp,
                                  int32_t mantissa_bias, const uint16_t* bias, uint16_t* y,
                                  int64_t ld_y, int64_t M, int64_t N, int64_t K, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  CONCORD_CHECK(sizes_ok(M, N, K), "concord_dqgemm_fwd: bad size");
  if (M == 0 || N == 0) return CONCORD_OK;
  CONCORD_CHECK(x && packed && row_exp && col_exp && y, "concord_dqgemm_fwd: NULL argument");
  CONCORD_CHECK(ld_x >= K && ld_p >= K && ld_y >= N, "concord_dqgemm_fwd: bad leading dimension");
  GemmArgs g = make_args(x, packed, ld_x, ld_p, row_exp, col_exp, mantissa_bias, bias, y, ld_y, M, N, K, true);
  return launch_gemm<MODE_FWD>(g, workspace, workspace_bytes, (hipStream_t)stream, "dqgemm_fwd");
}

extern "C" int concord_dqgemm_dgrad(const uint16_t* dy, int64_t ld_dy, const int32_t* packed,
                                    int64_t ld_p, const int8_t* row_exp, const int8_t* col_exp,
                                    int32_t mantissa_bias, uint16_t* dx, int64_t ld_dx, int64_t M,
                                    int64_t N, int64_t K, void* workspace, size_t workspace_bytes,
                                    void* stream) {
  CONCORD_CHECK(sizes_ok(M, N, K), "concord_dqgemm_dgrad: bad size");
  if (M == 0 || K == 0) return CONCORD_OK;
  CONCORD_CHECK(dy && packed && row_exp && col_exp && dx, "concord_dqgemm_dgrad: NULL argument");
  CONCORD_CHECK(ld_dy >= N && ld_p >= K && ld_dx >= K, "concord_dqgemm_dgrad: bad leading dimension");
  GemmArgs g = make_args(dy, packed, ld_dy, ld_p, row_exp, col_exp, mantissa_bias, nullptr, dx, ld_dx, M, K, N, true);
  return launch_gemm<MODE_DGRAD>(g, workspace, workspace_bytes, (hipStream_t)stream, "dqgemm_dgrad");
}

extern "C" int concord_wgrad(const uint16_t* dy, int64_t ld_dy, const uint16_t* x, int64_t ld_x,
                             uint16_t* grad_w, int64_t ld_gw, int64_t M, int64_t N, int64_t K,
                             void* workspace, size_t workspace_bytes, void* stream) {
  CONCORD_CHECK(sizes_ok(M, N, K), "concord_wgrad: bad size");
  if (N == 0 || K == 0) return CONCORD_OK;
  CONCORD_CHECK(grad_w && (M == 0 || (dy && x)), "concord_wgrad: NULL argument");
  CONCORD_CHECK(ld_dy >= N && ld_x >= K && ld_gw >= K, "concord_wgrad: bad leading dimension");
  if (M == 0) {   // an empty batch: the sum over no tokens
    fill_zero_bf16_launch(grad_w, ld_gw, N, K, (hipStream_t)stream);
    return launch_status("wgrad");
  }
  GemmArgs g = make_args(dy, x, ld_dy, ld_x, nullptr, nullptr, 0, nullptr, grad_w, ld_gw, N, K, M, false);
  return launch_gemm<MODE_WGRAD>(g, workspace, workspace_bytes, (hipStream_t)stream, "wgrad");
}

// wgrad with the v-hat EMA (and bias gradient); with gd, the dgrad product
// `gd` first, its split-K reduction carried by the WGRAD launch when the
// shapes allow (gemm_dgrad_wgrad_vhat_launch), else the two products in turn
static int wgrad_vhat_impl(const GemmArgs* gd, const uint16_t* dy, int64_t ld_dy, const uint16_t* x,
                           int64_t ld_x, uint16_t* grad_w, int64_t ld_gw, int64_t M, int64_t N, int64_t K,
                           double beta2, float* v_row, float* v_col, float* sum_v_inv, int32_t* row_max,
                           int32_t* col_max, int32_t* salt_counter, uint16_t* grad_bias, void* workspace,
                           size_t workspace_bytes, void* gemm_workspace, size_t gemm_workspace_bytes,
                           hipStream_t st, const char* what) {
  const Workspace ws = workspace_layout(N, K, grad_bias ? M : 0);
  if (!workspace || workspace_bytes < ws.total) {
    set_error("%s: workspace of %zu bytes needed", what, ws.total);
    return CONCORD_EWORKSPACE;
  }
  if (M == 0) {   // an empty batch: no dgrad rows, a zero weight gradient
    wgrad_vhat_empty_batch(grad_w, ld_gw, N, K, beta2, v_row, v_col, sum_v_inv, row_max, col_max, salt_counter,
                           grad_bias, workspace, st);
    return launch_status(what);
  }
  const VhatScratch v = vhat_scratch(N, K);
  float* pr = (float*)((char*)workspace + ws.scratch);
  float* pc = pr + v.pr;
  float* bsum = pc + v.pc;
  float* bpart = bsum + v.bsum;
  uint32_t* ticket = (uint32_t*)((char*)workspace + ws.vhat_ticket);
  GemmArgs g = make_args(dy, x, ld_dy, ld_x, nullptr, nullptr, 0, nullptr, grad_w, ld_gw, N, K, M, false);
  g.vh_pr = pr;
  g.vh_pc = pc;
  g.bpart = grad_bias ? bpart : nullptr;
  int tiles_j = 0;
  int rc = -1;
  GemmArgs pend;        // a dgrad split-K reduction the finalize launch carries
  int pend_rbi = 0;
  if (gd && gd->I > 0 && gd->J > 0) {
    rc = gemm_dgrad_wgrad_vhat_launch(*gd, gemm_workspace, gemm_workspace ? gemm_workspace_bytes : 0, g, st,
                                      what, &tiles_j, &pend, &pend_rbi);
    if (rc == -1)
      rc = gemm_wgrad_split_dgrad_launch(*gd, g, gemm_workspace, gemm_workspace ? gemm_workspace_bytes : 0, st,
                                         what, &tiles_j);
    if (rc == -1) {   // the products in turn
      rc = launch_gemm<MODE_DGRAD>(*gd, gemm_workspace, gemm_workspace_bytes, st, what);
      if (rc != CONCORD_OK) return rc;
      rc = -1;
    }
  }
  if (rc == -1) rc = gemm_wgrad_vhat_launch(g, gemm_workspace ? gemm_workspace_bytes : 0, st, what, &tiles_j);
  if (rc == -1) rc = gemm_wgrad_vhat_split_launch(g, gemm_workspace, gemm_workspace_bytes, st, what, &tiles_j);
  if (rc == -1) {   // unaligned WGRAD: the plain product, then the partials kernels
    g.bpart = nullptr;
    rc = launch_gemm<MODE_WGRAD>(g, gemm_workspace, gemm_workspace_bytes, st, what);
    if (rc != CONCORD_OK) return rc;
    vhat_partials_launch(grad_w, ld_gw, N, K, pr, pc, st);
    if (grad_bias) bias_grad_launch(dy, ld_dy, M, N, grad_bias, bpart, st);
    vhat_finish_launch(pr, pc, bsum, ticket, N, K, beta2, v_row, v_col, sum_v_inv, row_max, col_max,
                       salt_counter, st);
  } else if (rc != CONCORD_OK) {
    return rc;
  } else if (pend_rbi) {
    vhat_finish_carry_launch(pr, pc, bsum, ticket, N, K, beta2, v_row, v_col, sum_v_inv, row_max, col_max,
                             salt_counter, st, bpart, tiles_j, grad_bias, pend, pend_rbi);
  } else {
    vhat_finish_launch(pr, pc, bsum, ticket, N, K, beta2, v_row, v_col, sum_v_inv, row_max, col_max,
                       salt_counter, st, bpart, tiles_j, grad_bias);
  }
  return launch_status(what);
}

extern "C" int concord_wgrad_vhat(const uint16_t* dy, int64_t ld_dy, const uint16_t* x, int64_t ld_x,
                                  uint16_t* grad_w, int64_t ld_gw, int64_t M, int64_t N, int64_t K,
                                  double beta2, float* v_row, float* v_col, float* sum_v_inv,
                                  int32_t* row_max, int32_t* col_max, int32_t* salt_counter,
                                  uint16_t* grad_bias, void* workspace, size_t workspace_bytes,
                                  void* gemm_workspace, size_t gemm_workspace_bytes, void* stream) {
  CONCORD_CHECK(sizes_ok(M, N, K) && N > 0 && K > 0, "concord_wgrad_vhat: bad size");
  CONCORD_CHECK(grad_w && v_row && v_col && sum_v_inv && (M == 0 || (dy && x)), "concord_wgrad_vhat: NULL argument");
  CONCORD_CHECK(ld_dy >= N && ld_x >= K && ld_gw >= K, "concord_wgrad_vhat: bad leading dimension");
  return wgrad_vhat_impl(nullptr, dy, ld_dy, x, ld_x, grad_w, ld_gw, M, N, K, beta2, v_row, v_col, sum_v_inv,
                         row_max, col_max, salt_counter, grad_bias, workspace, workspace_bytes, gemm_workspace,
                         gemm_workspace_bytes, (hipStream_t)stream, "wgrad_vhat");
}

extern "C" int concord_dgrad_wgrad_vhat(const uint16_t* dy, int64_t ld_dy, const int32_t* packed, int64_t ld_p,
                                        const int8_t* row_exp, const int8_t* col_exp, int32_t mantissa_bias,
                                        uint16_t* dx, int64_t ld_dx, const uint16_t* x, int64_t ld_x,
                                        uint16_t* grad_w, int64_t ld_gw, int64_t M, int64_t N, int64_t K,
                                        double beta2, float* v_row, float* v_col, float* sum_v_inv,
                                        int32_t* row_max, int32_t* col_max, int32_t* salt_counter,
                                        uint16_t* grad_bias, void* workspace, size_t workspace_bytes,
                                        void* gemm_workspace, size_t gemm_workspace_bytes, void* stream) {
  CONCORD_CHECK(sizes_ok(M, N, K) && N > 0 && K > 0, "concord_dgrad_wgrad_vhat: bad size");
  CONCORD_CHECK(packed && row_exp && col_exp && grad_w && v_row && v_col && sum_v_inv && (M == 0 || (dy && dx && x)),
                "concord_dgrad_wgrad_vhat: NULL argument");
  CONCORD_CHECK(ld_dy >= N && ld_p >= K && ld_dx >= K && ld_x >= K && ld_gw >= K,
                "concord_dgrad_wgrad_vhat: bad leading dimension");
  const GemmArgs gd =
      make_args(dy, packed, ld_dy, ld_p, row_exp, col_exp, mantissa_bias, nullptr, dx, ld_dx, M, K, N, true);
  return wgrad_vhat_impl(&gd, dy, ld_dy, x, ld_x, grad_w, ld_gw, M, N, K, beta2, v_row, v_col, sum_v_inv,
                         row_max, col_max, salt_counter, grad_bias, workspace, workspace_bytes, gemm_workspace,
                         gemm_workspace_bytes, (hipStream_t)stream, "dgrad_wgrad_vhat");
}

// constant-clock ticks of the grid barrier's bound (100 ms), per device
static int64_t grid_timeout_ticks() {
  constexpr int kMaxDev = 64;
  static int64_t ticks[kMaxDev];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return 0;
  if (ticks[dev] == 0) {
    int khz = 0;
    if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess || khz <= 0) return 0;
    ticks[dev] = (int64_t)khz * 100;
  }
  return ticks[dev];
}

extern "C" int concord_dgrad_wgrad_update(
    const uint16_t* dy, int64_t ld_dy, int32_t* packed, int64_t ld_p, const int8_t* row_exp, const int8_t* col_exp,
    uint16_t* dx, int64_t ld_dx, const uint16_t* x, int64_t ld_x, uint16_t* grad_w, int64_t ld_gw, int copy_grad,
    int fuse, int64_t M, int64_t N, int64_t K, double beta2, float* v_row, float* v_col, float* sum_v_inv, int32_t* row_max,
    int32_t* col_max, float* coh_pre, int64_t ld_c, uint16_t* grad_bias, const concord_update_params* params,
    const concord_device_scalars* scalars, uint32_t flags, void* workspace, size_t workspace_bytes,
    void* gemm_workspace, size_t gemm_workspace_bytes, int* fused, void* stream) {
  const char* what = "dgrad_wgrad_update";
  if (fused) *fused = 0;
  CONCORD_CHECK(sizes_ok(M, N, K) && N > 0 && K > 0, "concord_dgrad_wgrad_update: bad size");
  CONCORD_CHECK(params && scalars && scalars->lr && scalars->eps && scalars->salt_counter,
                "concord_dgrad_wgrad_update: params/scalars NULL");
  CONCORD_CHECK(packed && row_exp && col_exp && grad_w && v_row && v_col && sum_v_inv && (M == 0 || (dy && dx && x)),
                "concord_dgrad_wgrad_update: NULL argument");
  CONCORD_CHECK(ld_dy >= N && ld_p >= K && ld_dx >= K && ld_x >= K && ld_gw >= K,
                "concord_dgrad_wgrad_update: bad leading dimension");
  CONCORD_CHECK(!(flags & CONCORD_EMIT_WEIGHT), "concord_dgrad_wgrad_update: EMIT_WEIGHT needs the separate update");
  CONCORD_CHECK(!(flags & CONCORD_TRACK_REBALANCE) || (row_max && col_max),
                "concord_dgrad_wgrad_update: TRACK_REBALANCE needs row_max/col_max");
  CONCORD_CHECK(!(flags & CONCORD_RATIO_COH) || (scalars->chase_floor && scalars->leak_floor),
                "concord_dgrad_wgrad_update: RATIO_COH needs chase_floor/leak_floor");
  const int upd = update_fast_path(*params, flags);
  const Workspace ws = workspace_layout(N, K, grad_bias ? M : 0);
  if (!workspace || workspace_bytes < ws.total) {
    set_error("%s: workspace of %zu bytes needed", what, ws.total);
    return CONCORD_EWORKSPACE;
  }
  hipStream_t st = (hipStream_t)stream;
  const GemmArgs gd =
      make_args(dy, packed, ld_dy, ld_p, row_exp, col_exp, params->mantissa_bias, nullptr, dx, ld_dx, M, K, N, true);
  const int64_t ticks = grid_timeout_ticks();
  const bool layout_ok = ld_p % 4 == 0 && ((uintptr_t)packed % 16) == 0 && ((uintptr_t)col_exp % 4) == 0 &&
                         (upd != 1 || (coh_pre && ld_c >= K && ld_c % 4 == 0 && ((uintptr_t)coh_pre % 16) == 0));
  if (fuse && M > 0 && upd != 0 && layout_ok && ticks > 0) {
    const VhatScratch v = vhat_scratch(N, K);
    float* pr = (float*)((char*)workspace + ws.scratch);
    float* pc = pr + v.pr;
    float* bsum = pc + v.pc;
    float* bpart = bsum + v.bsum;
    GemmArgs gw = make_args(dy, x, ld_dy, ld_x, nullptr, nullptr, 0, nullptr, grad_w, ld_gw, N, K, M, false);
    gw.vh_pr = pr;
    gw.vh_pc = pc;
    gw.bpart = grad_bias ? bpart : nullptr;
    if (!copy_grad) gw.c = nullptr;
    WgradUpd u{};
    u.v_row = v_row;
    u.v_col = v_col;
    u.bsum = bsum;
    u.sum_v_inv = sum_v_inv;
    u.row_max = row_max;
    u.col_max = col_max;
    u.salt = scalars->salt_counter;
    u.grad_bias = grad_bias;
    u.b2 = (float)beta2;
    u.omb2 = (float)(1.0 - beta2);
    u.bar = (uint32_t*)((char*)workspace + kGridBarrierOffset);
    u.exitc = (uint32_t*)((char*)workspace + kGridExitOffset);
    u.fault = (uint32_t*)((char*)workspace + kGridFaultOffset);
    u.timeout_ticks = ticks;
    u.packed = packed;
    u.ld_p = ld_p;
    u.row_exp = row_exp;
    u.col_exp = col_exp;
    u.coh_pre = coh_pre;
    u.ld_c = ld_c;
    u.p = *params;
    u.s = *scalars;
    u.flags = flags | CONCORD_SALT_PREBUMPED;
    const int rc = gemm_dgrad_wgrad_update_launch(gd, gemm_workspace, gemm_workspace ? gemm_workspace_bytes : 0, gw,
                                                  u, upd, st, what);
    if (rc != -1) {
      if (rc == CONCORD_OK && fused) *fused = 1;
      return rc;
    }
  }
  // the separate launches: products + v-hat EMA, then the update.  When the
  // update runs the fast kernel, the finalize leaves its 256-row totals and
  // the update chains them into 1 / sum v_row (the finalize's own chain, so
  // the same bits), which saves the finalize's ticket round trips
  const bool defer = adamw_fast_eligible(*params, flags, packed, ld_p, grad_w, ld_gw, coh_pre, ld_c);
  const int rc = wgrad_vhat_impl(&gd, dy, ld_dy, x, ld_x, grad_w, ld_gw, M, N, K, beta2, v_row, v_col,
                                 defer ? nullptr : sum_v_inv, row_max, col_max, scalars->salt_counter, grad_bias,
                                 workspace, workspace_bytes, gemm_workspace, gemm_workspace_bytes, st, what);
  if (rc != CONCORD_OK) return rc;
  if (defer) {
    const VhatScratch v = vhat_scratch(N, K);
    const float* bsum = (const float*)((char*)workspace + ws.scratch) + v.pr + v.pc;
    return apply_adamw_fast_bsum(packed, ld_p, grad_w, ld_gw, row_exp, col_exp, row_max, col_max, v_row, v_col,
                                 bsum, cdiv(N, 256), sum_v_inv, coh_pre, ld_c, N, K, params, scalars,
                                 flags | CONCORD_SALT_PREBUMPED, st);
  }
  return concord_apply_adamw(packed, ld_p, grad_w, ld_gw, nullptr, K, row_exp, col_exp, row_max, col_max, v_row,
                             v_col, sum_v_inv, coh_pre, ld_c, N, K, params, scalars, flags | CONCORD_SALT_PREBUMPED,
                             stream);
}

extern "C" int concord_wgrad_update_fault(void* workspace, size_t workspace_bytes, int* fault, void* stream) {
  CONCORD_CHECK(workspace && fault && workspace_bytes >= kGridFaultOffset + sizeof(uint32_t),
                "concord_wgrad_update_fault: bad argument");
  hipStream_t st = (hipStream_t)stream;
  uint32_t v = 0;
  uint32_t* flag = (uint32_t*)((char*)workspace + kGridFaultOffset);
  if (hipMemcpyAsync(&v, flag, sizeof(v), hipMemcpyDeviceToHost, st) != hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess) {
    set_error("concord_wgrad_update_fault: reading the flag failed");
    return CONCORD_ELAUNCH;
  }
  *fault = (int)v;
  if (v != 0 && (hipMemsetAsync(flag, 0, sizeof(v), st) != hipSuccess || hipStreamSynchronize(st) != hipSuccess)) {
    set_error("concord_wgrad_update_fault: clearing the flag failed");
    return CONCORD_ELAUNCH;
  }
  return CONCORD_OK;
}

extern "C" int concord_gemm_bf16_fwd(const uint16_t* x, int64_t ld_x, const uint16_t* w,
                                     int64_t ld_w, const uint16_t* bias, uint16_t* y, int64_t ld_y,
                                     int64_t M, int64_t N, int64_t K, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  CONCORD_CHECK(sizes_ok(M, N, K), "concord_gemm_bf16_fwd: bad size");
  if (M == 0 || N == 0) return CONCORD_OK;
  CONCORD_CHECK(x && w && y, "concord_gemm_bf16_fwd: NULL argument");
  CONCORD_CHECK(ld_x >= K && ld_w >= K && ld_y >= N, "concord_gemm_bf16_fwd: bad leading dimension");
  GemmArgs g = make_args(x, w, ld_x, ld_w, nullptr, nullptr, 0, bias, y, ld_y, M, N, K, false);
  return launch_gemm<MODE_FWD_BF16>(g, workspace, workspace_bytes, (hipStream_t)stream, "gemm_bf16_fwd");
}

extern "C" int concord_gemm_bf16_dgrad(const uint16_t* dy, int64_t ld_dy, const uint16_t* w,
                                       int64_t ld_w, uint16_t* dx, int64_t ld_dx, int64_t M,
                                       int64_t N, int64_t K, void* workspace,
                                       size_t workspace_bytes, void* stream) {
  CONCORD_CHECK(sizes_ok(M, N, K), "concord_gemm_bf16_dgrad: bad size");
  if (M == 0 || K == 0) return CONCORD_OK;
  CONCORD_CHECK(dy && w && dx, "concord_gemm_bf16_dgrad: NULL argument");
  CONCORD_CHECK(ld_dy >= N && ld_w >= K && ld_dx >= K, "concord_gemm_bf16_dgrad: bad leading dimension");
  GemmArgs g = make_args(dy, w, ld_dy, ld_w, nullptr, nullptr, 0, nullptr, dx, ld_dx, M, K, N, false);
  return launch_gemm<MODE_DGRAD_BF16>(g, workspace, workspace_bytes, (hipStream_t)stream, "gemm_bf16_dgrad");
}

extern "C" size_t concord_gemm_sym_workspace_bytes(int64_t M, int64_t R, int b_rows) {
  if (M < 1) M = 1;
  if (R < 1) R = 1;
  return gemm_sym_splitk_need(b_rows ? MODE_FWD_BF16 : MODE_DGRAD_BF16, M, R);
}

extern "C" int concord_gemm_bf16_sym(const uint16_t* a, int64_t ld_a, const uint16_t* b, int64_t ld_b, int b_rows,
                                     uint16_t* c, int64_t ld_c, int64_t M, int64_t R, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  CONCORD_CHECK(sizes_ok(M, M, R), "concord_gemm_bf16_sym: bad size");
  CONCORD_CHECK(b_rows || R == M, "concord_gemm_bf16_sym: a b of symmetric matrices needs R == M");
  if (M == 0) return CONCORD_OK;
  CONCORD_CHECK(a && b && c, "concord_gemm_bf16_sym: NULL argument");
  CONCORD_CHECK(ld_a >= R && ld_b >= (b_rows ? R : M) && ld_c >= M, "concord_gemm_bf16_sym: bad leading dimension");
  const int mode = b_rows ? MODE_FWD_BF16 : MODE_DGRAD_BF16;
  CONCORD_CHECK(workspace_bytes >= gemm_sym_splitk_need(mode, M, R) || !workspace,
                "concord_gemm_bf16_sym: workspace of %zu bytes needed", gemm_sym_splitk_need(mode, M, R));
  const int rc = gemm_bf16_sym(mode, a, ld_a, b, ld_b, c, ld_c, M, R, nullptr, 0, 0.0f, 0.0f, workspace,
                               workspace_bytes, (hipStream_t)stream, "gemm_bf16_sym");
  CONCORD_CHECK(rc != -1, "concord_gemm_bf16_sym: operands not aligned for the fast kernels (16-byte bases, "
                          "leading dimensions and M multiples of 8)");
  return rc;
}
