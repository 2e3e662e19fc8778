// gemm.h -- shared definitions of the GEMM kernels (gemm.hip: generic
// kernel for any strides; gemm_fast.hip: branch-free kernels for aligned
// operands).
#pragma once
#include "common.h"

namespace concord {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

enum { MODE_FWD = 0, MODE_DGRAD = 1, MODE_WGRAD = 2, MODE_FWD_BF16 = 3, MODE_DGRAD_BF16 = 4 };

constexpr int TR = 64;          // reduction depth per LDS stage
constexpr int LDS_STRIDE = 72;  // bf16 per LDS row (64 + 8 pad)

// Implicit-GEMM convolution (stride 1 or 2 per axis, zero padding): one
// operand is an NHWC activation read as the patch matrix without forming it.
// Patch index r = tap * C + c, tap = ky * kw + kx (C % 64 == 0, so a 64-deep
// stage stays inside one tap).  A GEMM row (FWD, DGRAD) or reduction index
// (WGRAD) is a position (b, y, x) of an Hr x Wr grid, split by exact
// magic-number division (conv_magic).
struct ConvIdx {
  int32_t C;              // channels of the gathered activation
  int32_t Hg, Wg;         // its spatial size
  int32_t Hr, Wr;         // the grid of the GEMM's positions
  int32_t kw;             // kernel width (taps per kernel row)
  int32_t ph, pw;         // padding
  int32_t slh, slw;       // log2 of the strides
  int32_t cb;             // DGRAD: channels of a tap block of the weight operand (its in-channels)
  uint32_t mw, mh;        // magic multipliers for / Wr and / Hr
  int32_t shw, shh;       // and their shifts
  uint32_t act_bytes;     // bytes of the gathered activation
  uint32_t w_bytes;       // DGRAD: bytes of the weight operand
};

// (mg, sh) with floor(m mg / 2^sh) = floor(m / d) for every 0 <= m < 2^24:
// sh = 24 + ceil(log2 d), mg = ceil(2^sh / d) < 2^25.  With e = mg d - 2^sh
// in [0, d): m mg / 2^sh = m / d + m e / (d 2^sh), and m e < 2^24 d <= 2^sh,
// so the excess stays below 1 / d.
inline void conv_magic(uint32_t d, uint32_t& mg, int32_t& sh) {
  int l = 0;
  while ((1u << l) < d) ++l;
  sh = 24 + l;
  mg = (uint32_t)((((uint64_t)1 << sh) + d - 1) / d);
}

struct GemmArgs {
  const uint16_t* a;      // FWD: x[M,K]; DGRAD*, WGRAD: dy[M,N]
  const void* b;          // packed[N,K] int32 | x[M,K] bf16 (WGRAD) | W[N,K] bf16 (*_BF16)
  int64_t lda, ldb;
  const int8_t* row_exp;  // packed rows (n)
  const int8_t* col_exp;  // packed cols (k)
  int32_t bias;           // mantissa bias
  const uint16_t* vbias;  // bias[J] added in the epilogue, or NULL
  uint16_t* c;
  int64_t ldc;
  int64_t I, J, R;        // C is I x J, reduction R
  int64_t r_split;        // reduction length per split (multiple of TR)
  float* part;            // split-K: 2 x I x J fp32 partials
  uint32_t* tile_cnt;     // split-K: one counter per (i, j) tile, zero between calls
  int tiles_i, tiles_j, splits;
  int vec_a, vec_b, vec_c;  // base pointers and leading dimensions allow 16 B / 8 B accesses
  float* vh_pr;           // WGRAD with v-hat partials: row / column partial sums of g^2
  float* vh_pc;
  float* bpart;           // WGRAD with v-hat partials: bias-gradient partials [tiles_j][I], or NULL
  // optional combine (fast kernels only): C = bf16(as * ay + at * bf16(product)),
  // ay[I][J] with leading dimension ldy, in combine_bf16x2's float order
  const uint16_t* ay;
  int64_t ldy;
  float as, at;
  ConvIdx cv;             // implicit-GEMM convolution kernels only
  // symmetric product (FWD / DGRAD kernels, I == J): the count of tiles that
  // meet the upper triangle j >= i, which alone are computed (sym_tile); the
  // split-K slots are indexed in that order.  0: the full tile grid.
  int sym;
  // i-tiles per group of the grouped tile order (grouped_tile); 0: 8.  The
  // order only decides which workgroup computes which tile, never a result.
  int gi;
};

// s * y + t * x as the Newton-Schulz combination steps take it (x is the
// bf16-rounded product; the t = 1 case skips the multiply by t)
CONCORD_DEV float combine1(float s, float y, float t, float x) {
  return t == 1.0f ? __fadd_rn(__fmul_rn(s, y), x) : __fadd_rn(__fmul_rn(s, y), __fmul_rn(t, x));
}
// two bf16 lanes of y and x -> two bf16 lanes of bf16(s y + t x)
CONCORD_DEV uint32_t combine_bf16x2(uint32_t yw, uint32_t xw, float s, float t) {
  return pack_bf16x2(combine1(s, __uint_as_float(yw << 16), t, __uint_as_float(xw << 16)),
                     combine1(s, __uint_as_float(yw & 0xFFFF0000u), t, __uint_as_float(xw & 0xFFFF0000u)));
}

// grouped row-major tile order: groups of GI i-tiles, j-tiles ascending
// within a group, i-tiles fastest (a bijection of [0, ti tj) for any GI >= 1)
__host__ __device__ inline void grouped_tile(int lin, int ti, int tj, int& bi, int& bj, int GI = 8) {
  const int group = lin / (GI * tj);
  const int first_i = group * GI;
  const int gsize = ti - first_i < GI ? ti - first_i : GI;
  const int in = lin % (GI * tj);
  bi = first_i + in % gsize;
  bj = in / gsize;
}

// XCD x (workgroups w = x mod 8) owns q + (x < rem) consecutive indices
// starting at x*q + min(x, rem), q = total / 8, rem = total % 8: a bijection
// of [0, total) for any total
__host__ __device__ inline int xcd_linear(int w, int total) {
  const int xcd = w % 8, slot = w / 8;
  const int q = total / 8, rem = total % 8;
  return xcd * q + (xcd < rem ? xcd : rem) + slot;
}

// XCD-aware tile order: workgroup w runs on XCD w % 8.  XCD x owns tile
// indices [x*T/8, (x+1)*T/8) of the grouped order, so the CUs of one XCD
// share i- and j-tiles in their L2.
CONCORD_DEV void tile_of(int w, int ti, int tj, int total, int& bi, int& bj, int GI = 8) {
  grouped_tile(xcd_linear(w, total), ti, tj, bi, bj, GI);
}

// Split-K launches (splits x tiles workgroups): XCD x owns a contiguous range
// of the split-major order (split, then the grouped tiles), so its CUs share
// one split's slices of both operands in L2, rather than every XCD reading
// the whole reduction range of its tiles.  The split-K partial slots are
// keyed by the row-major tile index bi * tiles_j + bj.
__host__ __device__ inline void split_tile_of(int w, int ti, int tj, int splits, int& split, int& bi, int& bj,
                                              int GI = 8) {
  const int tiles = ti * tj;
  const int lin = xcd_linear(w, tiles * splits);
  split = lin / tiles;
  grouped_tile(lin % tiles, ti, tj, bi, bj, GI);
}

// Symmetric products: tile row bi (rows [bi BI, bi BI + BI)) meets the upper
// triangle j >= i in the tile columns bj >= sym_lo(bi) = floor(bi BI / BJ),
// the first whose columns reach past the row block's first row.  Every
// element (i, j) with j >= i lies in such a tile.
__host__ __device__ inline int sym_lo(int bi, int BI, int BJ) { return (int)(((int64_t)bi * BI) / BJ); }
__host__ __device__ inline int sym_tile_count(int ti, int tj, int BI, int BJ) {
  int n = 0;
  for (int bi = 0; bi < ti; ++bi) {
    const int lo = sym_lo(bi, BI, BJ);
    n += lo < tj ? tj - lo : 0;
  }
  return n;
}
// the t-th tile of that set, rows ascending and columns ascending in a row
CONCORD_DEV void sym_tile(int t, int ti, int tj, int BI, int BJ, int& bi, int& bj) {
  bi = 0;
  bj = 0;
  for (int r = 0; r < ti; ++r) {
    const int lo = min(tj, sym_lo(r, BI, BJ));
    if (t < tj - lo) {
      bi = r;
      bj = lo + t;
      return;
    }
    t -= tj - lo;
  }
}
// tile (bi, bj), split and split-K slot of workgroup w of a FWD / DGRAD
// launch: split_tile_of over the full grid (slot bi * tiles_j + bj), or for
// a symmetric product the same XCD-contiguous split-major order over the
// g.sym tiles of the upper triangle (slot = the tile's index among them)
template <int BI, int BJ>
CONCORD_DEV void gemm_tile_of(const GemmArgs& g, int w, int& split, int& bi, int& bj, int& slot) {
  if (g.sym) {
    const int lin = xcd_linear(w, g.sym * g.splits);
    split = lin / g.sym;
    slot = lin % g.sym;
    sym_tile(slot, g.tiles_i, g.tiles_j, BI, BJ, bi, bj);
  } else {
    split_tile_of(w, g.tiles_i, g.tiles_j, g.splits, split, bi, bj, g.gi > 0 ? g.gi : 8);
    slot = bi * g.tiles_j + bj;
  }
}

// launch a fast-path kernel when the operands satisfy its alignment rules;
// returns CONCORD_OK, an error code, or -1 when the generic kernel must run
int gemm_fast_launch(int mode, const GemmArgs& g, void* workspace, size_t ws_bytes,
                     hipStream_t st, const char* what);
// WGRAD whose epilogue also writes the v-hat partial sums of the bf16 output
// (vhat_tile.h order) into vh_pr / vh_pc; -1 when the shape or its alignment
// does not run the transpose-read kernel, or when the plan given split_room
// bytes of split-K workspace would split it (the caller then runs the plain
// WGRAD and the separate partials kernel)
int gemm_wgrad_vhat_launch(const GemmArgs& g, size_t split_room, hipStream_t st, const char* what,
                           int* tiles_j);
// a split WGRAD with the same results as gemm_wgrad_vhat_launch: the split
// product (bias partials per split and j-tile when g.bpart is set), then one
// reduction that also writes the v-hat partials and folds the bias rows over
// the splits; *bias_rows = the bias partial rows left (tiles_j).  -1 when the
// plan does not split or the operands do not take the transpose-read kernel.
int gemm_wgrad_vhat_split_launch(const GemmArgs& g, void* workspace, size_t ws_bytes, hipStream_t st,
                                 const char* what, int* bias_rows);
// dgrad (split, its reduction deferred) then the VH WGRAD whose spare
// workgroups run that reduction on the CUs the WGRAD tiles leave idle; or,
// when both grids fit the chip at once, both products in one launch
// (gemm_dgt_tr_kernel) and the dgrad's reduction after it: left to the
// caller when `pending` is given (*pending_rbi = its tile rows, 0 = none; the
// caller passes them to vhat_finish_carry_launch), else launched here.  -1
// when the shapes do not take these paths (the caller then issues the two
// products separately).  The dgrad's split-K partials use `workspace`.
int gemm_dgrad_wgrad_vhat_launch(const GemmArgs& gd, void* workspace, size_t ws_bytes, const GemmArgs& gw,
                                 hipStream_t st, const char* what, int* tiles_j, GemmArgs* pending = nullptr,
                                 int* pending_rbi = nullptr);
// vhat_finish_launch's finalize with a dgrad's split-K reduction (rd, tile rows
// rbi, from gemm_dgrad_wgrad_vhat_launch) carried by extra blocks of the launch
void vhat_finish_carry_launch(const float* pr, const float* pc, float* bsum, uint32_t* ticket, int64_t N, int64_t K,
                              double beta2, float* v_row, float* v_col, float* sum_v_inv, int32_t* row_max,
                              int32_t* col_max, int32_t* salt, hipStream_t st, const float* bpart, int64_t nbp,
                              uint16_t* grad_bias, const GemmArgs& rd, int rbi);
// tiles along J of the WGRAD launch above (the bias partials' row count)
int64_t gemm_wgrad_vhat_tiles_j(int64_t J);
// the other pairing: a split WGRAD with v-hat partials first, then the unsplit
// dgrad carrying its split-K reduction; -1 when the plans are not of that form
int gemm_wgrad_split_dgrad_launch(const GemmArgs& gd, const GemmArgs& gw, void* workspace, size_t ws_bytes,
                                  hipStream_t st, const char* what, int* bias_rows);
// the products of gemm_dgrad_wgrad_vhat_launch with the v-hat finalize and the
// packed update carried by the WGRAD launch (wgrad_update.h); upd = 1 bare,
// 2 winner (update_fast_path).  -1 when that launch does not apply.
struct WgradUpd;
int gemm_dgrad_wgrad_update_launch(const GemmArgs& gd, void* workspace, size_t ws_bytes, const GemmArgs& gw,
                                   const WgradUpd& u, int upd, hipStream_t st, const char* what);
// c = bf16(s * y + t * bf16(product)) for MODE_FWD_BF16 / MODE_DGRAD_BF16 on
// the fast kernels (the combine applied in their epilogue or split-K
// reduction); -1 when the operands do not take the fast kernels (the caller
// then runs the product and the combination separately)
int gemm_bf16_combine(int mode, const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb, uint16_t* c,
                      int64_t ldc, int64_t I, int64_t J, int64_t R, const uint16_t* y, int64_t ldy, float s,
                      float t, void* ws, size_t ws_bytes, hipStream_t st, const char* what);
// a symmetric bf16 product C[I][I] (MODE_FWD_BF16: a b^T with b = a; or
// MODE_DGRAD_BF16: a b of two commuting symmetric matrices, e.g. b = a),
// optionally combined as gemm_bf16_combine does (y symmetric too, or NULL):
// only the tiles meeting the upper triangle are computed, and each of their
// elements (i, j) with i <= j is stored at (i, j) and (j, i) by the epilogue
// or the split-K reduction.  -1 when the operands do not take the fast
// kernels.
int gemm_bf16_sym(int mode, const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb, uint16_t* c,
                  int64_t ldc, int64_t I, int64_t R, const uint16_t* y, int64_t ldy, float s, float t, void* ws,
                  size_t ws_bytes, hipStream_t st, const char* what);
// split-K workspace bytes (counters + partials) gemm_bf16_sym may use
size_t gemm_sym_splitk_need(int mode, int64_t I, int64_t R);
// a plain bf16 product through the fast or generic kernels: MODE_FWD_BF16
// (C[I][J] = sum_r a[i][r] b[j][r]) or MODE_DGRAD_BF16 (sum_r a[i][r] b[r][j])
int gemm_bf16_run(int mode, const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb, uint16_t* c,
                  int64_t ldc, int64_t I, int64_t J, int64_t R, void* ws, size_t ws_bytes, hipStream_t st,
                  const char* what);
// implicit-GEMM convolution products (g.cv set): MODE_FWD_BF16 (x gathered,
// W' [N][taps * C] rows), MODE_DGRAD_BF16 (dy gathered, W' rows (n, tap) by
// the tap's column block) or MODE_WGRAD (x gathered as the column operand);
// -1 when the operands do not take the kernels.  A MODE_WGRAD launch with
// g.bpart set also leaves the bias partials of dy in its first *bias_rows
// rows of I values (one per j-tile; a split launch sums its splits' rows
// into them, in split order).
int gemm_conv_launch(int mode, const GemmArgs& g, void* workspace, size_t ws_bytes, hipStream_t st,
                     const char* what, int* bias_rows = nullptr);
// split-K partial bytes gemm_conv_launch plans for an I x J x R product
size_t gemm_conv_partial_bytes(int mode, int64_t I, int64_t J, int64_t R);
// split-K workspace bytes (counters + partials) one such product may use
size_t gemm_splitk_need(int mode, int64_t I, int64_t J, int64_t R);
// split-K partial bytes the fast kernels plan for an I x J x R problem
// given unlimited workspace (0 when they do not split it)
size_t gemm_fast_partial_bytes(int mode, int64_t I, int64_t J, int64_t R);

}  // namespace concord
