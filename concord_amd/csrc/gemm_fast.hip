// gemm_fast.hip -- branch-free bf16 MFMA GEMM kernels for aligned operands
// (the problem statement and modes are in gemm.h; gemm.hip holds the generic
// kernel that serves every other stride and alignment).
//
// What makes these kernels fast on gfx950:
//  * every global read is a buffer load; a lane whose element lies outside the
//    operand gets an offset past the buffer end and the hardware returns zero.
//    Edge tiles and the reduction tail need no branches, so one pipeline stage
//    is one basic block the scheduler can interleave freely.
//  * a packed word decodes with plain integer/float VALU ops only (the matrix
//    core runs them alongside the MFMAs; v_dot4 and v_cvt_f32_i32 would
//    stall it): m_eff = sf + 128 (ss + vs) is added to the bit pattern M of
//    1.5 * 2^(23+e), and subtracting that float leaves m_eff * 2^e exactly,
//    e being the exponent that varies along the reduction.  The exponent of
//    the other side is constant along each output column and is applied in
//    the epilogue: scaling by a power of two commutes with fp32 rounding, so
//    the result equals the product with the fully decoded weight
//    bf16(m_eff * 2^(row_exp + col_exp - bias)).
//  * the large tiles split each block into compute waves (LDS fragments ->
//    MFMA, and the activation operand moved straight from global memory into
//    LDS by buffer-load DMA) and producer waves (weight loads two stages
//    ahead, decode, LDS writes).
//  * split-K over S ways is deterministic: the last block of a tile to finish
//    sums the S fp32 partials in split order.
#include <algorithm>
#include <type_traits>
#include <cmath>

#include "gemm.h"
#include "vhat_finalize.h"
#include "vhat_tile.h"
#include "wgrad_update.h"
#include "workspace.h"

namespace concord {
namespace {

typedef __amdgpu_buffer_rsrc_t Rsrc;
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x2 __attribute__((ext_vector_type(2)));

// a voffset at or past every buffer's num_records (which stay below 2^31)
constexpr uint32_t kOOB = 0x80000000u;
constexpr int kMaxSplits = kGemmMaxSplits;

// num_records of an operand band: (last row's offset + its length) in bytes,
// 0 when the band is empty (R = 0 or no rows left makes the formula negative,
// and a wrapped 32-bit count would put kOOB inside the buffer)
CONCORD_DEV uint32_t nrec(int64_t bytes) { return bytes > 0 ? (uint32_t)bytes : 0u; }
CONCORD_DEV Rsrc make_rsrc(const void* p, uint32_t bytes) {
  // dword 3 = 0x00020000: 32-bit data format, raw (stride 0) addressing
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
// soffset is the stage offset, the same for the whole wave; readfirstlane
// states that to the compiler, which otherwise may wrap each load in a
// per-lane loop when it cannot prove the value uniform
CONCORD_DEV uint32_t uni(uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)v); }
CONCORD_DEV i32x4 ld128(Rsrc r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, uni(soff), 0);
}
CONCORD_DEV i32x2 ld64(Rsrc r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, voff, uni(soff), 0);
}
CONCORD_DEV int32_t ld32(Rsrc r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voff, uni(soff), 0);
}

// m_eff * 2^e of one packed word, exactly, with plain integer/float VALU ops
// only (they co-execute with MFMAs; v_dot4 and v_cvt_f32_i32 do not):
// with M = bits of 1.5 * 2^(23+e), the float whose bits are M + m is
// 1.5 * 2^(23+e) + m * 2^e for |m| < 2^22, so subtracting 1.5 * 2^(23+e)
// leaves m * 2^e.  m_eff = sf + 128 (ss + vs) lies in [-65536, 65279].
// Four VALU ops per word: the two integer adds take their sign-extended
// byte and half-word operands straight from the word through SDWA operand
// selects (the producer waves' decode shares the SIMDs with the MFMA waves,
// and separate v_bfe / v_ashr extracts made it 6.5 ops per word).
CONCORD_DEV uint32_t magic(int32_t e) { return ((uint32_t)(150 + e) << 23) | 0x400000u; }
// magic() of the sign-extended byte I of a packed word of four exponents:
// (sext(byte) << 23) by one SDWA shift, then one add, since
// (150 + e) << 23 | 2^22 = (e << 23) + 0x4B400000 (two ops where the byte
// extract, shift and add took three)
template <int I> CONCORD_DEV uint32_t magic_byte(int32_t ex) {
  static_assert(I >= 0 && I < 4, "byte of the exponent word");
  uint32_t r;
  if constexpr (I == 0)
    asm("v_lshlrev_b32_sdwa %0, 23, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0"
        : "=v"(r) : "v"(ex));
  else if constexpr (I == 1)
    asm("v_lshlrev_b32_sdwa %0, 23, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1"
        : "=v"(r) : "v"(ex));
  else if constexpr (I == 2)
    asm("v_lshlrev_b32_sdwa %0, 23, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2"
        : "=v"(r) : "v"(ex));
  else
    asm("v_lshlrev_b32_sdwa %0, 23, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3"
        : "=v"(r) : "v"(ex));
  return r + 0x4B400000u;
}
CONCORD_DEV float dec(int32_t w, uint32_t M) {
  int32_t t;   // ss + vs
  asm("v_add_u32_sdwa %0, sext(%1), sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1 src1_sel:BYTE_0"
      : "=v"(t)
      : "v"(w));
  const uint32_t u = ((uint32_t)t << 7) + M;   // + 128 (ss + vs)
  uint32_t b;  // + sf
  asm("v_add_u32_sdwa %0, %1, sext(%2) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:WORD_1"
      : "=v"(b)
      : "v"(u), "v"(w));
  return __fsub_rn(__uint_as_float(b), __uint_as_float(M));
}

CONCORD_DEV int32_t sbyte(int32_t v, int i) { return __builtin_amdgcn_sbfe(v, 8 * i, 8); }

// Redefine raw load registers at the point of their decode.  The decode is
// pure arithmetic, which the compiler would otherwise hoist across the LDS
// barrier into the previous pipeline stage, forcing that stage to wait for
// loads issued only just before it.
template <typename T> CONCORD_DEV void pin(T& v) { asm volatile("" : "+v"(v)); }

// ---- operand loaders --------------------------------------------------------
// Each loader owns per-thread byte offsets (fixed for the whole reduction; a
// lane outside the operand holds kOOB) and moves one TR-deep stage of its tile
// from global memory into a Raw register set (load) and from there into LDS as
// bf16 [row][r] with r contiguous (store).  `rem` = reduction elements left
// from the stage start; r >= rem reads zero.  NT = threads per block.

// bf16 [rows][R], r contiguous; chunk = 8 bf16.  Thread t: r = 8 (t % 8),
// rows t/8 + (NT/8) q.  When the rows do not split evenly, the surplus rows
// read zeros into LDS padding rows (LROWS >= ROWS).
template <int ROWS, int NT>
struct RowsBf16 {
  static constexpr int PER = (ROWS * 8 + NT - 1) / NT;
  static constexpr int LROWS = PER * NT / 8;
  static constexpr int NLOADS = PER, NWRITES = PER, NVALU = PER;
  struct Raw { i32x4 v[PER]; };
  uint32_t voff[PER];
  int32_t kc;
  Rsrc rs;
  CONCORD_DEV void init(const uint16_t* band, int64_t ld, int64_t rows_left, int64_t R, int t) {
    kc = (t % 8) * 8;
    rs = make_rsrc(band, nrec(((rows_left - 1) * ld + R) * 2));
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int64_t row = t / 8 + (NT / 8) * q;
      voff[q] = (row < rows_left && row < ROWS) ? (uint32_t)((row * ld + kc) * 2) : kOOB;
    }
  }
  CONCORD_DEV void load(Raw& r, int64_t r0, int64_t rem) const {
    const bool ok = kc < rem;
    const uint32_t so = (uint32_t)(r0 * 2);
#pragma unroll
    for (int q = 0; q < PER; ++q) r.v[q] = ld128(rs, ok ? voff[q] : kOOB, so);
  }
  CONCORD_DEV void store(Raw& r, uint16_t* lds, int t) const {
#pragma unroll
    for (int q = 0; q < PER; ++q)
      *reinterpret_cast<i32x4*>(lds + (t / 8 + (NT / 8) * q) * LDS_STRIDE + kc) = r.v[q];
  }
  // into the swizzled [row][64] tile that stage_mfma_swz reads: the thread's
  // 16-byte chunk kc / 8 of rows t / 8 + (NT / 8) q, whose (row >> 1) & 7 is
  // the same for every q
  CONCORD_DEV void store_swz(Raw& r, uint16_t* lds, int t) const {
    const int c = (((t % 8) ^ ((t / 8) >> 1)) & 7) * 8;
#pragma unroll
    for (int q = 0; q < PER; ++q)
      *reinterpret_cast<i32x4*>(lds + (t / 8 + (NT / 8) * q) * 64 + c) = r.v[q];
  }
};

// packed [rows][R] int32, r contiguous (the forward's W[n][k]); chunk = 4
// words.  Thread t: r = 4 (t % 16), rows t/16 + (NT/16) q.  The per-r
// column exponents are applied while decoding.
template <int ROWS, int NT>
struct RowsPacked {
  static constexpr int PER = ROWS * 16 / NT;
  static constexpr int LROWS = ROWS;
  static constexpr int NLOADS = PER + 1, NWRITES = PER, NVALU = 19 * PER + 4;
  static_assert(PER * NT == ROWS * 16, "tile rows must split evenly over the threads");
  struct Raw { i32x4 v[PER]; int32_t ex; };
  uint32_t voff[PER];
  int32_t kc;
  Rsrc rs, es;
  CONCORD_DEV void init(const int32_t* band, int64_t ld, int64_t rows_left, int64_t R,
                        const int8_t* exps, int t) {
    kc = (t % 16) * 4;
    rs = make_rsrc(band, nrec(((rows_left - 1) * ld + R) * 4));
    es = make_rsrc(exps, (uint32_t)R);
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int64_t row = t / 16 + (NT / 16) * q;
      voff[q] = row < rows_left ? (uint32_t)((row * ld + kc) * 4) : kOOB;
    }
  }
  CONCORD_DEV void load(Raw& r, int64_t r0, int64_t rem) const {
    const bool ok = kc < rem;
    const uint32_t so = (uint32_t)(r0 * 4);
#pragma unroll
    for (int q = 0; q < PER; ++q) r.v[q] = ld128(rs, ok ? voff[q] : kOOB, so);
    r.ex = ld32(es, ok ? (uint32_t)kc : kOOB, (uint32_t)r0);
  }
  template <bool SWZ = false>
  CONCORD_DEV void store(Raw& r, uint16_t* lds, int t, int swz_col = 0) const {
    pin(r.ex);
#pragma unroll
    for (int q = 0; q < PER; ++q) pin(r.v[q]);
    const uint32_t e0 = magic_byte<0>(r.ex), e1 = magic_byte<1>(r.ex), e2 = magic_byte<2>(r.ex),
                   e3 = magic_byte<3>(r.ex);
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      uint2 o;
      o.x = pack_bf16x2(dec(r.v[q].x, e0), dec(r.v[q].y, e1));
      o.y = pack_bf16x2(dec(r.v[q].z, e2), dec(r.v[q].w, e3));
      if (SWZ)
        *reinterpret_cast<uint2*>(lds + (t / 16 + (NT / 16) * q) * 64 + swz_col) = o;
      else
        *reinterpret_cast<uint2*>(lds + (t / 16 + (NT / 16) * q) * LDS_STRIDE + kc) = o;
    }
  }
  // the thread's 4 columns kc .. kc + 3 (half of 16-byte chunk kc / 8) in the
  // swizzled [row][64] tile; (row >> 1) & 7 is the same for all its rows
  CONCORD_DEV int swz_cols(int t) const {
    return ((((t % 16) >> 1) ^ ((t / 16) >> 1)) & 7) * 8 + (t & 1) * 4;
  }
  CONCORD_DEV void store_swz(Raw& r, uint16_t* lds, int t) const { store<true>(r, lds, t, swz_cols(t)); }
};

// Column loaders: [R][cols] with cols contiguous, moved in blocks of RB r x 4
// cols.  Thread t: r = RB (t % (TR/RB)) .. +RB-1, cols 4 (t / (TR/RB) +
// (NT / (TR/RB)) q).  RB = 8 when the tile has enough blocks for every
// thread, else 4.
template <int COLS, int NT>
struct ColGeom {
  static constexpr int RB = (TR / 8) * (COLS / 4) >= NT ? 8 : 4;
  static constexpr int NRB = TR / RB;   // row blocks per stage
  static constexpr int PER = NRB * (COLS / 4) / NT;
  static_assert(PER >= 1 && PER * NT == NRB * (COLS / 4), "column tile must split evenly over the threads");
  static CONCORD_DEV int rb(int t) { return (t % NRB) * RB; }
  static CONCORD_DEV int col(int t, int q) { return 4 * (t / NRB + (NT / NRB) * q); }
};

// packed int32 (the dgrad's W[n][k] with r = n).  Per-r row exponents are
// applied while decoding, and the bf16 pairs are formed along r, so the
// transpose costs nothing.
template <int COLS, int NT>
struct ColsPacked {
  typedef ColGeom<COLS, NT> G;
  static constexpr int PER = G::PER, RB = G::RB, LROWS = COLS;
  static constexpr int NLOADS = PER * RB + RB / 4, NWRITES = 4 * PER, NVALU = PER * (RB * 18 + RB) + RB;
  struct Raw { i32x4 v[PER][RB]; int32_t ex[RB / 4]; };
  uint32_t voff[PER];
  uint32_t ld4;
  int32_t rb;
  Rsrc rs, es;
  CONCORD_DEV void init(const int32_t* band, int64_t ld, int64_t cols_left, int64_t R,
                        const int8_t* exps, int t) {
    rb = G::rb(t);
    ld4 = (uint32_t)(ld * 4);
    rs = make_rsrc(band, nrec(((R - 1) * ld + cols_left) * 4));
    es = make_rsrc(exps, (uint32_t)R);
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int64_t col = G::col(t, q);
      voff[q] = col < cols_left ? (uint32_t)((rb * ld + col) * 4) : kOOB;
    }
  }
  CONCORD_DEV void load(Raw& r, int64_t r0, int64_t rem) const {
    const uint32_t so = (uint32_t)(r0 * (int64_t)ld4);
#pragma unroll
    for (int e = 0; e < RB; ++e) {
      const bool ok = rb + e < rem;
#pragma unroll
      for (int q = 0; q < PER; ++q) r.v[q][e] = ld128(rs, ok ? voff[q] + e * ld4 : kOOB, so);
    }
#pragma unroll
    for (int h = 0; h < RB / 4; ++h)
      r.ex[h] = ld32(es, rb + 4 * h < rem ? (uint32_t)(rb + 4 * h) : kOOB, (uint32_t)r0);
  }
  CONCORD_DEV void store(Raw& r, uint16_t* lds, int t) const {
#pragma unroll
    for (int h = 0; h < RB / 4; ++h) pin(r.ex[h]);
#pragma unroll
    for (int q = 0; q < PER; ++q)
#pragma unroll
      for (int e = 0; e < RB; ++e) pin(r.v[q][e]);
    uint32_t ex[RB];
#pragma unroll
    for (int e = 0; e < RB; ++e) ex[e] = magic(sbyte(r.ex[e / 4], e % 4));
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int col = G::col(t, q);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        int32_t o[RB / 2];
#pragma unroll
        for (int p = 0; p < RB / 2; ++p)
          o[p] = (int32_t)pack_bf16x2(dec(r.v[q][2 * p][c], ex[2 * p]), dec(r.v[q][2 * p + 1][c], ex[2 * p + 1]));
        uint16_t* dst = lds + (col + c) * LDS_STRIDE + rb;
        if (RB == 8) *reinterpret_cast<i32x4*>(dst) = i32x4{o[0], o[1], o[2 % (RB / 2)], o[3 % (RB / 2)]};
        else *reinterpret_cast<i32x2*>(dst) = i32x2{o[0], o[1]};
      }
    }
  }
};

// bf16 (wgrad's dy and x, dgrad's bf16 W): 8-byte loads, transposed with
// byte permutes.
template <int COLS, int NT>
struct ColsBf16 {
  typedef ColGeom<COLS, NT> G;
  static constexpr int PER = G::PER, RB = G::RB, LROWS = COLS;
  static constexpr int NLOADS = PER * RB, NWRITES = 4 * PER, NVALU = PER * (2 * RB + RB);
  struct Raw { i32x2 v[PER][RB]; };
  uint32_t voff[PER];
  uint32_t ld2;
  int32_t rb;
  Rsrc rs;
  CONCORD_DEV void init(const uint16_t* band, int64_t ld, int64_t cols_left, int64_t R, int t) {
    rb = G::rb(t);
    ld2 = (uint32_t)(ld * 2);
    rs = make_rsrc(band, nrec(((R - 1) * ld + cols_left) * 2));
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int64_t col = G::col(t, q);
      voff[q] = col < cols_left ? (uint32_t)((rb * ld + col) * 2) : kOOB;
    }
  }
  CONCORD_DEV void load(Raw& r, int64_t r0, int64_t rem) const {
    const uint32_t so = (uint32_t)(r0 * (int64_t)ld2);
#pragma unroll
    for (int e = 0; e < RB; ++e) {
      const bool ok = rb + e < rem;
#pragma unroll
      for (int q = 0; q < PER; ++q) r.v[q][e] = ld64(rs, ok ? voff[q] + e * ld2 : kOOB, so);
    }
  }
  CONCORD_DEV void store(Raw& r, uint16_t* lds, int t) const {
#pragma unroll
    for (int q = 0; q < PER; ++q)
#pragma unroll
      for (int e = 0; e < RB; ++e) pin(r.v[q][e]);
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int col = G::col(t, q);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        // column c of the RB x 4 block: rows (2p, 2p+1) -> dword p
        const int dw = c >> 1;
        const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
        int32_t o[RB / 2];
#pragma unroll
        for (int p = 0; p < RB / 2; ++p)
          o[p] = (int32_t)__builtin_amdgcn_perm((uint32_t)r.v[q][2 * p + 1][dw],
                                                (uint32_t)r.v[q][2 * p][dw], sel);
        uint16_t* dst = lds + (col + c) * LDS_STRIDE + rb;
        if (RB == 8) *reinterpret_cast<i32x4*>(dst) = i32x4{o[0], o[1], o[2 % (RB / 2)], o[3 % (RB / 2)]};
        else *reinterpret_cast<i32x2*>(dst) = i32x2{o[0], o[1]};
      }
    }
  }
};

// ---- per-mode operand pairs -------------------------------------------------
template <int MODE, int BI, int BJ, int NT> struct Ops;

template <int BI, int BJ, int NT> struct Ops<MODE_FWD, BI, BJ, NT> {
  RowsBf16<BI, NT> a;
  RowsPacked<BJ, NT> b;
  CONCORD_DEV void init(const GemmArgs& g, int64_t i0, int64_t j0, int t) {
    a.init(g.a + i0 * g.lda, g.lda, g.I - i0, g.R, t);
    b.init(reinterpret_cast<const int32_t*>(g.b) + j0 * g.ldb, g.ldb, g.J - j0, g.R, g.col_exp, t);
  }
};
template <int BI, int BJ, int NT> struct Ops<MODE_FWD_BF16, BI, BJ, NT> {
  RowsBf16<BI, NT> a;
  RowsBf16<BJ, NT> b;
  CONCORD_DEV void init(const GemmArgs& g, int64_t i0, int64_t j0, int t) {
    a.init(g.a + i0 * g.lda, g.lda, g.I - i0, g.R, t);
    b.init(reinterpret_cast<const uint16_t*>(g.b) + j0 * g.ldb, g.ldb, g.J - j0, g.R, t);
  }
};
template <int BI, int BJ, int NT> struct Ops<MODE_DGRAD, BI, BJ, NT> {
  RowsBf16<BI, NT> a;
  ColsPacked<BJ, NT> b;
  CONCORD_DEV void init(const GemmArgs& g, int64_t i0, int64_t j0, int t) {
    a.init(g.a + i0 * g.lda, g.lda, g.I - i0, g.R, t);
    b.init(reinterpret_cast<const int32_t*>(g.b) + j0, g.ldb, g.J - j0, g.R, g.row_exp, t);
  }
};
template <int BI, int BJ, int NT> struct Ops<MODE_DGRAD_BF16, BI, BJ, NT> {
  RowsBf16<BI, NT> a;
  ColsBf16<BJ, NT> b;
  CONCORD_DEV void init(const GemmArgs& g, int64_t i0, int64_t j0, int t) {
    a.init(g.a + i0 * g.lda, g.lda, g.I - i0, g.R, t);
    b.init(reinterpret_cast<const uint16_t*>(g.b) + j0, g.ldb, g.J - j0, g.R, t);
  }
};
template <int BI, int BJ, int NT> struct Ops<MODE_WGRAD, BI, BJ, NT> {
  ColsBf16<BI, NT> a;
  ColsBf16<BJ, NT> b;
  CONCORD_DEV void init(const GemmArgs& g, int64_t i0, int64_t j0, int t) {
    a.init(g.a + i0, g.lda, g.I - i0, g.R, t);
    b.init(reinterpret_cast<const uint16_t*>(g.b) + j0, g.ldb, g.J - j0, g.R, t);
  }
};

// Workgroup barrier that orders LDS only.  __syncthreads() also acquires
// global memory, which waits for every outstanding buffer load (vmcnt(0)) and
// so would cap the prefetch distance at one stage.
// s_waitcnt immediate (gfx9 encoding) that waits until at most n vector
// memory operations are outstanding and leaves the other counters alone
constexpr int vmcnt_imm(int n) { return (n & 0xF) | (0x7 << 4) | (0xF << 8) | (((n >> 4) & 3) << 14); }

CONCORD_DEV void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ---- instruction schedule of one pipeline stage -------------------------------
// Per wave and stage: NRD fragment reads per 32-deep sub-step, NM MFMAs, NLD
// buffer loads of stage s+2, NWR LDS writes of stage s+1 and NV decode VALU
// ops.  The order handed to the scheduler: the first sub-step's fragment
// reads; then the first half of the MFMAs, each followed by one buffer load
// (with the VALU op that picks its offset) and one fragment read of the
// second sub-step; then the second half of the MFMAs, each followed by its
// share of the decode and the LDS writes.  The decode of stage s+1 thereby
// starts half a stage after the loads of stage s+2 are on their way, and the
// matrix core, the VALU, the LDS and the memory pipeline overlap.
template <int NM, int NRD, int NLD, int NWR, int NV>
CONCORD_DEV void sched_stage() {
  constexpr int H = NM / 2;
  constexpr int VPM = (NV + (NM - H) - 1) / (NM - H);
  __builtin_amdgcn_sched_group_barrier(0x100, NRD, 0);   // DS read: sub-step 0 fragments
#pragma unroll
  for (int i = 0; i < H; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
    if (i < NLD) {
      __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);   // VALU: the load's offset
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // VMEM read
    }
    if (i >= 1 && i < 1 + NRD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read: sub-step 1
  }
#pragma unroll
  for (int i = H; i < NM; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
    __builtin_amdgcn_sched_group_barrier(0x002, VPM, 0);  // VALU: decode
    if (((i - H) % 2) == 1 && (i - H) / 2 < NWR) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);   // DS write
  }
}

// ---- epilogue shared by the kernels ------------------------------------------
// NAW waves hold accumulators (aw = this wave's index among them, -1 for a
// wave without); lane holds C[i0 + ra + 16x + lane%16][j0 + rb + 16y + 4(lane/16) + e].
// Split-K: each split stores its accumulators in register order (one
// contiguous 1 KB per wave instruction) into its slot of the partial buffer
// and is done; splitk_reduce_kernel sums the slots in split order afterwards
// (a device-scope fence here would write back a whole XCD's L2).
// Otherwise the column scale 2^(exp - bias) of the side not decoded in the
// loop and the bias are applied, the tile is rounded to bf16 into LDS
// (`stage`, at least BI x (BJ + 8) bf16, free once the main loop is done)
// and written out row-contiguous.
template <int NAW, int NI, int NJ>
CONCORD_DEV float* partial_slot(const GemmArgs& g, int tile, int split, int aw) {
  return g.part + ((int64_t)tile * g.splits + split) * ((int64_t)NAW * NI * NJ * 256) + (int64_t)aw * NI * NJ * 256;
}

template <int MODE, int NI, int NJ, int BI, int BJ, int NAW>
CONCORD_DEV void epilogue(const GemmArgs& g, f32x4 (&acc)[NI][NJ], int64_t i0, int64_t j0, int ra, int rb,
                          int split, int tile, int aw, int t, int nthreads, uint16_t* stage) {
  constexpr int LDO = BJ + 8;   // bf16 per staged row (16-byte multiple, shifts banks by 4)
  static_assert((int64_t)NAW * NI * NJ * 256 == (int64_t)BI * BJ, "accumulator waves must cover the tile");
  const int lane = t & 63;
  if (g.splits > 1) {
    if (aw >= 0) {
      float* mine = partial_slot<NAW, NI, NJ>(g, tile, split, aw) + lane * 4;
#pragma unroll
      for (int x = 0; x < NI; ++x)
#pragma unroll
        for (int y = 0; y < NJ; ++y) *reinterpret_cast<f32x4*>(mine + (x * NJ + y) * 256) = acc[x][y];
    }
    return;
  }
  // column scale and bias in registers, bf16 tile into LDS
  __syncthreads();
  if (aw >= 0) {
    const int8_t* cexp = MODE == MODE_FWD ? g.row_exp : MODE == MODE_DGRAD ? g.col_exp : nullptr;
#pragma unroll
    for (int y = 0; y < NJ; ++y) {
      const int cl = rb + y * 16 + 4 * (lane >> 4);   // tile-local column
      const int64_t j = j0 + cl;
      float sc[4] = {1.f, 1.f, 1.f, 1.f}, bs[4] = {0.f, 0.f, 0.f, 0.f};
      if (j < g.J) {
        if (cexp) {
          const int32_t e4 = *reinterpret_cast<const int32_t*>(cexp + j);
#pragma unroll
          for (int e = 0; e < 4; ++e) sc[e] = exp2i(sbyte(e4, e) - g.bias);
        }
        if (g.vbias) {
          const uint2 b4 = *reinterpret_cast<const uint2*>(g.vbias + j);
          bs[0] = __uint_as_float(b4.x << 16);
          bs[1] = __uint_as_float(b4.x & 0xFFFF0000u);
          bs[2] = __uint_as_float(b4.y << 16);
          bs[3] = __uint_as_float(b4.y & 0xFFFF0000u);
        }
      }
#pragma unroll
      for (int x = 0; x < NI; ++x) {
        const int rl = ra + x * 16 + (lane & 15);
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = __fadd_rn(__fmul_rn(acc[x][y][e], sc[e]), bs[e]);
        *reinterpret_cast<uint2*>(stage + rl * LDO + cl) =
            make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
      }
    }
  }
  __syncthreads();
  // row-contiguous stores: 8 bf16 (16 bytes) per thread when the output
  // allows, else 4 (J % 4 == 0, ldc % 4 == 0, 8-byte aligned base)
  const bool v16 = (g.ldc % 8 == 0) && (g.J % 8 == 0) && (((uintptr_t)g.c % 16) == 0);
  if (g.sym) {
    // symmetric product: each element (i, j) with i <= j goes to (i, j) and
    // (j, i); the tile's elements below the diagonal are left to the tile
    // holding their mirror image (every element is written once)
    for (int c = t; c < BI * BJ; c += nthreads) {
      const int rl = c % BI, cl = c / BI;   // consecutive threads: consecutive i, so (j, i) stores coalesce
      const int64_t i = i0 + rl, j = j0 + cl;
      if (i <= j && j < g.J) {
        uint32_t o = stage[rl * LDO + cl];
        if (g.ay) o = combine_bf16x2(g.ay[i * g.ldy + j], o, g.as, g.at) & 0xFFFFu;
        g.c[i * g.ldc + j] = (uint16_t)o;
        g.c[j * g.ldc + i] = (uint16_t)o;
      }
    }
  } else if (v16) {
    constexpr int CPR = BJ / 8;
    for (int c = t; c < BI * CPR; c += nthreads) {
      const int rl = c / CPR, cl = (c % CPR) * 8;
      const int64_t i = i0 + rl, j = j0 + cl;
      if (i < g.I && j < g.J) {
        uint4 o = *reinterpret_cast<const uint4*>(stage + rl * LDO + cl);
        if (g.ay) {
          const uint4 yv = *reinterpret_cast<const uint4*>(g.ay + i * g.ldy + j);
          o = make_uint4(combine_bf16x2(yv.x, o.x, g.as, g.at), combine_bf16x2(yv.y, o.y, g.as, g.at),
                         combine_bf16x2(yv.z, o.z, g.as, g.at), combine_bf16x2(yv.w, o.w, g.as, g.at));
        }
        *reinterpret_cast<uint4*>(g.c + i * g.ldc + j) = o;
      }
    }
  } else {
    constexpr int CPR = BJ / 4;
    for (int c = t; c < BI * CPR; c += nthreads) {
      const int rl = c / CPR, cl = (c % CPR) * 4;
      const int64_t i = i0 + rl, j = j0 + cl;
      if (i < g.I && j < g.J) {
        uint2 o = *reinterpret_cast<const uint2*>(stage + rl * LDO + cl);
        if (g.ay) {
          const uint2 yv = *reinterpret_cast<const uint2*>(g.ay + i * g.ldy + j);
          o = make_uint2(combine_bf16x2(yv.x, o.x, g.as, g.at), combine_bf16x2(yv.y, o.y, g.as, g.at));
        }
        *reinterpret_cast<uint2*>(g.c + i * g.ldc + j) = o;
      }
    }
  }
}

// Split-K reduction: one thread per (tile, accumulator wave, 16x16 block,
// lane) sums the splits' partials in split order, applies the column scale
// and bias, and stores 4 bf16.
template <int MODE, int NI, int NJ, int BI, int BJ, int WI, int WJ>
CONCORD_DEV int64_t splitk_reduce_items(const GemmArgs& g) {
  const int64_t tiles = g.sym ? g.sym : (int64_t)g.tiles_i * g.tiles_j;
  return tiles * WI * WJ * NI * NJ * 64;
}

template <int MODE, int NI, int NJ, int BI, int BJ, int WI, int WJ, int SP>
CONCORD_DEV void splitk_reduce_item_sp(const GemmArgs& g, int64_t idx) {
  constexpr int NAW = WI * WJ, WTI = BI / WI, WTJ = BJ / WJ;
  const int lane = (int)(idx % 64);
  int64_t r = idx / 64;
  const int y = (int)(r % NJ); r /= NJ;
  const int x = (int)(r % NI); r /= NI;
  const int aw = (int)(r % NAW);
  const int tile = (int)(r / NAW);   // the split-K slot: row-major tile index, or the symmetric set's index
  int bi = tile / g.tiles_j, bj = tile % g.tiles_j;
  if (g.sym) sym_tile(tile, g.tiles_i, g.tiles_j, BI, BJ, bi, bj);
  const int64_t i = (int64_t)bi * BI + (aw / WJ) * WTI + x * 16 + (lane & 15);
  const int64_t j = (int64_t)bj * BJ + (aw % WJ) * WTJ + y * 16 + 4 * (lane >> 4);
  if (i >= g.I || j >= g.J) return;
  const int64_t PT = (int64_t)NAW * NI * NJ * 256;
  const float* p = g.part + (int64_t)tile * g.splits * PT + (int64_t)aw * NI * NJ * 256 + (x * NJ + y) * 256 + lane * 4;
  // every split's partial loaded before any is summed (one memory round trip)
  f32x4 part[SP];
#pragma unroll
  for (int s2 = 0; s2 < SP; ++s2) part[s2] = *reinterpret_cast<const f32x4*>(p + s2 * PT);
  f32x4 sum = part[0];
#pragma unroll
  for (int s2 = 1; s2 < SP; ++s2)
#pragma unroll
    for (int e = 0; e < 4; ++e) sum[e] = __fadd_rn(sum[e], part[s2][e]);
  const int8_t* cexp = MODE == MODE_FWD ? g.row_exp : MODE == MODE_DGRAD ? g.col_exp : nullptr;
  float sc[4] = {1.f, 1.f, 1.f, 1.f}, bs[4] = {0.f, 0.f, 0.f, 0.f};
  if (cexp) {
    const int32_t e4 = *reinterpret_cast<const int32_t*>(cexp + j);
#pragma unroll
    for (int e = 0; e < 4; ++e) sc[e] = exp2i(sbyte(e4, e) - g.bias);
  }
  if (g.vbias) {
    const uint2 b4 = *reinterpret_cast<const uint2*>(g.vbias + j);
    bs[0] = __uint_as_float(b4.x << 16);
    bs[1] = __uint_as_float(b4.x & 0xFFFF0000u);
    bs[2] = __uint_as_float(b4.y << 16);
    bs[3] = __uint_as_float(b4.y & 0xFFFF0000u);
  }
  float v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = __fadd_rn(__fmul_rn(sum[e], sc[e]), bs[e]);
  uint2 o = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
  if (g.ay) {
    const uint2 yv = *reinterpret_cast<const uint2*>(g.ay + i * g.ldy + j);
    o = make_uint2(combine_bf16x2(yv.x, o.x, g.as, g.at), combine_bf16x2(yv.y, o.y, g.as, g.at));
  }
  if (g.sym) {
    // symmetric product: (i, j + e) with i <= j + e goes to both positions
    // (as the epilogue's sym branch); elements below the diagonal are skipped
    if (i > j + 3) return;
    if (i <= j) *reinterpret_cast<uint2*>(g.c + i * g.ldc + j) = o;
    const uint16_t h[4] = {(uint16_t)(o.x & 0xFFFFu), (uint16_t)(o.x >> 16), (uint16_t)(o.y & 0xFFFFu),
                           (uint16_t)(o.y >> 16)};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (i <= j + e) {
        if (i > j) g.c[i * g.ldc + j + e] = h[e];
        g.c[(j + e) * g.ldc + i] = h[e];
      }
    }
    return;
  }
  *reinterpret_cast<uint2*>(g.c + i * g.ldc + j) = o;
}

// splitk_reduce_item_sp for the launch's split count (uniform), 2 .. kGemmMaxSplits
template <int MODE, int NI, int NJ, int BI, int BJ, int WI, int WJ>
CONCORD_DEV void splitk_reduce_item(const GemmArgs& g, int64_t idx) {
  static_assert(kGemmMaxSplits == 16, "one case per split count");
  switch (g.splits) {
    case 2: splitk_reduce_item_sp<MODE, NI, NJ, BI, BJ, WI, WJ, 2>(g, idx); break;
    case 3: splitk_reduce_item_sp<MODE, NI, NJ, BI, BJ, WI, WJ, 3>(g, idx); break;
    case 4: splitk_reduce_item_sp<MODE, NI, NJ, BI, BJ, WI, WJ, 4>(g, idx); break;
    case 5: splitk_reduce_item_sp<MODE, NI, NJ, BI, BJ, WI, WJ, 5>(g, idx); break;
    case 6: splitk_reduce_item_sp<MODE, NI, NJ, BI, BJ, WI, WJ, 6>(g, idx); break;
    case 7: splitk_reduce_item_sp<MODE, NI, NJ, BI, BJ, WI, WJ, 7>(g, idx); break;
    case 8: splitk_reduce_item_sp<MODE, NI, NJ, BI, BJ, WI, WJ, 8>(g, idx); break;
    case 9: splitk_reduce_item_sp<MODE, NI, NJ, BI, BJ, WI, WJ, 9>(g, idx); break;
    case 10: splitk_reduce_item_sp<MODE, NI, NJ, BI, BJ, WI, WJ, 10>(g, idx); break;
    case 11: splitk_reduce_item_sp<MODE, NI, NJ, BI, BJ, WI, WJ, 11>(g, idx); break;
    case 12: splitk_reduce_item_sp<MODE, NI, NJ, BI, BJ, WI, WJ, 12>(g, idx); break;
    case 13: splitk_reduce_item_sp<MODE, NI, NJ, BI, BJ, WI, WJ, 13>(g, idx); break;
    case 14: splitk_reduce_item_sp<MODE, NI, NJ, BI, BJ, WI, WJ, 14>(g, idx); break;
    case 15: splitk_reduce_item_sp<MODE, NI, NJ, BI, BJ, WI, WJ, 15>(g, idx); break;
    default: splitk_reduce_item_sp<MODE, NI, NJ, BI, BJ, WI, WJ, 16>(g, idx); break;
  }
}

// bias rows of a split WGRAD (g.bpart): value f = (bj, i) of the split-0 row
// becomes the sum over the splits' rows, in split order (as
// splitk_reduce_vh_kernel folds them)
CONCORD_DEV void bias_fold_item(const GemmArgs& g, int64_t f) {
  const int64_t bj = f / g.I, i = f % g.I;
  float* b = g.bpart + bj * g.I + i;
  float s = *b;
  for (int sp = 1; sp < g.splits; ++sp) s = __fadd_rn(s, b[(int64_t)sp * g.tiles_j * g.I]);
  *b = s;
}

// threads [0, items) reduce the product; for a WGRAD with bias partials the
// next tiles_j * I fold them
template <int MODE, int NI, int NJ, int BI, int BJ, int WI, int WJ>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(GemmArgs g) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t items = splitk_reduce_items<MODE, NI, NJ, BI, BJ, WI, WJ>(g);
  if (idx < items) {
    splitk_reduce_item<MODE, NI, NJ, BI, BJ, WI, WJ>(g, idx);
  } else if (MODE == MODE_WGRAD && g.bpart && idx - items < (int64_t)g.tiles_j * g.I) {
    bias_fold_item(g, idx - items);
  }
}

// Split-K reduction of a WGRAD launch, with the v-hat partials: one block per
// 64 x 64 accumulator wave tile, its four waves one 16-row block each, sums
// the splits' partials in split order (the additions of splitk_reduce_item),
// stores the bf16 tile and leaves the squares of the stored values in LDS;
// wave 0 then forms the tile's v-hat partials in vhat_tile_partials' order,
// as the VH epilogue does for an unsplit launch.  With bias partials
// (g.bpart), blocks of column 0 of each tile also sum its j-tile's bias
// partial rows over the splits, in split order, into the split-0 row, so the
// finalize reads tiles_j rows as for an unsplit launch.
template <int BI, int BJ, int WI, int WJ>
struct ReduceVh {
  static constexpr int NAW = WI * WJ, WTI = BI / WI, WTJ = BJ / WJ, NI = WTI / 16, NJ = WTJ / 16;
  static_assert(NI == 4 && NJ == 4, "v-hat partials take 64 x 64 wave tiles");
  static constexpr int LDS_FLOATS = NI * NJ * 4 * 64;   // [x][y][e][lane]: the squares, for wave 0
  // blocks of one launch: one per accumulator wave tile
  static int blocks(const GemmArgs& g) { return g.tiles_i * g.tiles_j * NAW; }
  // part 1 of block `blk` on threads tid in [0, 256): the split sums, the bf16
  // tile, the squares into s_g2, the bias fold
  static CONCORD_DEV void part1(const GemmArgs& g, int blk, int tid, float* s_g2) {
    const int lane = tid & 63, x = tid >> 6;   // wave x takes row block x of the tile
    // row-major tile index
    const int tile = blk / NAW, aw = blk % NAW;
    const int bi = tile / g.tiles_j, bj = tile % g.tiles_j;
    const int64_t row0 = (int64_t)bi * BI + (aw / WJ) * WTI, col0 = (int64_t)bj * BJ + (aw % WJ) * WTJ;
    const int64_t PT = (int64_t)NAW * NI * NJ * 256;
    const float* base = g.part + (int64_t)tile * g.splits * PT + (int64_t)aw * NI * NJ * 256 + lane * 4;
    {
      // the row of 4 blocks, eight splits' partials loaded before any of them
      // is summed (one memory round trip per eight splits), summed in order.
      // The loads have no branch around them (a split past the last reads the
      // last again, unused): a load under a branch let the compiler copy its
      // result at the join, which waited for it before the rest were issued
      constexpr int CH = 8;
      static_assert(kGemmMaxSplits <= 2 * CH, "two chunks of splits");
      f32x4 sums[NJ];
#pragma unroll
      for (int c0 = 0; c0 < 2 * CH; c0 += CH) {
        if (c0 >= g.splits) break;
        f32x4 part[NJ][CH];
#pragma unroll
        for (int y = 0; y < NJ; ++y)
#pragma unroll
          for (int s2 = 0; s2 < CH; ++s2)
            part[y][s2] = *reinterpret_cast<const f32x4*>(base + (x * NJ + y) * 256 +
                                                          (int64_t)min(c0 + s2, g.splits - 1) * PT);
#pragma unroll
        for (int y = 0; y < NJ; ++y) {
          if (c0 == 0) sums[y] = part[y][0];
#pragma unroll
          for (int s2 = (c0 == 0 ? 1 : 0); s2 < CH; ++s2)
            if (c0 + s2 < g.splits)
#pragma unroll
              for (int e = 0; e < 4; ++e) sums[y][e] = __fadd_rn(sums[y][e], part[y][s2][e]);
        }
      }
#pragma unroll
      for (int y = 0; y < NJ; ++y) {
        const f32x4 sum = sums[y];
        const uint32_t lo = pack_bf16x2(sum[0], sum[1]), hi = pack_bf16x2(sum[2], sum[3]);
        const float v[4] = {__uint_as_float(lo << 16), __uint_as_float(lo & 0xFFFF0000u),
                            __uint_as_float(hi << 16), __uint_as_float(hi & 0xFFFF0000u)};
#pragma unroll
        for (int e = 0; e < 4; ++e) s_g2[((x * NJ + y) * 4 + e) * 64 + lane] = __fmul_rn(v[e], v[e]);
        const int64_t i = row0 + x * 16 + (lane & 15), j = col0 + y * 16 + 4 * (lane >> 4);
        if (i < g.I && j < g.J) *reinterpret_cast<uint2*>(g.c + i * g.ldc + j) = make_uint2(lo, hi);
      }
    }
    if (x == 1 && g.bpart && aw % WJ == 0) {
      const int64_t i = row0 + lane;
      if (i < g.I) {
        float* b = g.bpart + (int64_t)bj * g.I + i;
        const int64_t rs = (int64_t)g.tiles_j * g.I;   // one split's rows
        // every split's value in flight at once (unconditional loads, as
        // above), then summed in split order
        float v[kGemmMaxSplits];
#pragma unroll
        for (int s2 = 0; s2 < kGemmMaxSplits; ++s2) v[s2] = b[(int64_t)min(s2, g.splits - 1) * rs];
        float sb = v[0];
#pragma unroll
        for (int s2 = 1; s2 < kGemmMaxSplits; ++s2)
          if (s2 < g.splits) sb = __fadd_rn(sb, v[s2]);
        b[0] = sb;
      }
    }
  }
  // part 2 (after a barrier over part 1's threads): wave 0 forms the tile's
  // v-hat partials from s_g2
  static CONCORD_DEV void part2(const GemmArgs& g, int blk, int tid, const float* s_g2) {
    if (tid >= 64) return;
    const int lane = tid;
    const int tile = blk / NAW, aw = blk % NAW;
    const int bi = tile / g.tiles_j, bj = tile % g.tiles_j;
    const int64_t row0 = (int64_t)bi * BI + (aw / WJ) * WTI, col0 = (int64_t)bj * BJ + (aw % WJ) * WTJ;
    float g2[4][4][4];
#pragma unroll
    for (int xx = 0; xx < NI; ++xx)
#pragma unroll
      for (int y = 0; y < NJ; ++y)
#pragma unroll
        for (int e = 0; e < 4; ++e) g2[xx][y][e] = s_g2[((xx * NJ + y) * 4 + e) * 64 + lane];
    vhat_tile_partials(g2, lane, row0, col0, g.I, g.J, g.vh_pr, g.vh_pc);
  }
};

template <int BI, int BJ, int WI, int WJ>
__global__ __launch_bounds__(256) void splitk_reduce_vh_kernel(GemmArgs g) {
  typedef ReduceVh<BI, BJ, WI, WJ> RV;
  __shared__ float s_g2[RV::LDS_FLOATS];
  RV::part1(g, (int)blockIdx.x, (int)threadIdx.x, s_g2);
  __syncthreads();
  RV::part2(g, (int)blockIdx.x, (int)threadIdx.x, s_g2);
}

// MFMAs of one TR-deep stage for a wave tile of NI x NJ 16x16 blocks whose
// rows start at LDS rows ra (A) and rb (B).
template <int NI, int NJ>
CONCORD_DEV void stage_mfma(f32x4 (&acc)[NI][NJ], const uint16_t* la, const uint16_t* lb, int ra, int rb,
                            int lane) {
  const int lrow = lane & 15, lk = (lane >> 4) * 8;
#pragma unroll
  for (int kk = 0; kk < TR / 32; ++kk) {
    bf16x8 fa[NI], fb[NJ];
#pragma unroll
    for (int x = 0; x < NI; ++x)
      fa[x] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const i32x4*>(
                                             la + (ra + x * 16 + lrow) * LDS_STRIDE + kk * 32 + lk));
#pragma unroll
    for (int y = 0; y < NJ; ++y)
      fb[y] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const i32x4*>(
                                             lb + (rb + y * 16 + lrow) * LDS_STRIDE + kk * 32 + lk));
    // D^T: MFMA rows = j (B tile), columns = i (A tile)
#pragma unroll
    for (int x = 0; x < NI; ++x)
#pragma unroll
      for (int y = 0; y < NJ; ++y)
        acc[x][y] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[y], fa[x], acc[x][y], 0, 0, 0);
  }
}

// ---- the kernel -------------------------------------------------------------
// DB: two raw register sets (loads two stages ahead) or one (one stage ahead,
// for tiles whose raw footprint would not fit twice)
template <int MODE, int BI, int BJ, int WI, int WJ, int MINB, bool DB, bool SCHED>
__global__ __launch_bounds__(64 * WI * WJ, MINB) void gemm_fast_kernel(GemmArgs g) {
  constexpr int NT = 64 * WI * WJ;
  constexpr int WTI = BI / WI, WTJ = BJ / WJ;   // wave tile
  constexpr int NI = WTI / 16, NJ = WTJ / 16;
  static_assert(WTI % 16 == 0 && WTJ % 16 == 0, "wave tile must be a multiple of 16");
  typedef Ops<MODE, BI, BJ, NT> OpsT;
  constexpr int LA = decltype(OpsT::a)::LROWS, LB = decltype(OpsT::b)::LROWS;
  static_assert(LA >= BI && LB >= BJ, "LDS tile rows");
  __shared__ __attribute__((aligned(16))) uint16_t lds_a[2][LA * LDS_STRIDE];
  __shared__ __attribute__((aligned(16))) uint16_t lds_b[2][LB * LDS_STRIDE];

  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wi = wave / WJ, wj = wave % WJ;
  const int wg = blockIdx.x;
  int split, bi, bj, slot;
  gemm_tile_of<BI, BJ>(g, wg, split, bi, bj, slot);
  const int64_t i0 = (int64_t)bi * BI, j0 = (int64_t)bj * BJ;
  const int64_t r_begin = (int64_t)split * g.r_split;
  const int64_t r_end = min(g.R, r_begin + g.r_split);
  const int nst = r_end > r_begin ? (int)((r_end - r_begin + TR - 1) / TR) : 0;

  OpsT op;
  op.init(g, i0, j0, t);
  // per-stage instruction counts for the schedule hint
  constexpr int NLD = decltype(OpsT::a)::NLOADS + decltype(OpsT::b)::NLOADS;
  constexpr int NWR = decltype(OpsT::a)::NWRITES + decltype(OpsT::b)::NWRITES;
  constexpr int NV = decltype(OpsT::a)::NVALU + decltype(OpsT::b)::NVALU;
  typename decltype(op.a)::Raw ra0, ra1;
  typename decltype(op.b)::Raw rb0, rb1;

  f32x4 acc[NI][NJ];
#pragma unroll
  for (int x = 0; x < NI; ++x)
#pragma unroll
    for (int y = 0; y < NJ; ++y) acc[x][y] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int lrow = lane & 15, lk = (lane >> 4) * 8;
  auto compute = [&](const uint16_t* la, const uint16_t* lb) {
#pragma unroll
    for (int kk = 0; kk < TR / 32; ++kk) {
      bf16x8 fa[NI], fb[NJ];
#pragma unroll
      for (int x = 0; x < NI; ++x)
        fa[x] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const i32x4*>(
                                               la + (wi * WTI + x * 16 + lrow) * LDS_STRIDE + kk * 32 + lk));
#pragma unroll
      for (int y = 0; y < NJ; ++y)
        fb[y] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const i32x4*>(
                                               lb + (wj * WTJ + y * 16 + lrow) * LDS_STRIDE + kk * 32 + lk));
      // D^T: MFMA rows = j (B tile), columns = i (A tile)
#pragma unroll
      for (int x = 0; x < NI; ++x)
#pragma unroll
        for (int y = 0; y < NJ; ++y)
          acc[x][y] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[y], fa[x], acc[x][y], 0, 0, 0);
    }
  };

  if (!DB) {
    if (nst > 0) {
      op.a.load(ra0, r_begin, r_end - r_begin);
      op.b.load(rb0, r_begin, r_end - r_begin);
      op.a.store(ra0, lds_a[0], t);
      op.b.store(rb0, lds_b[0], t);
      op.a.load(ra0, r_begin + TR, r_end - r_begin - TR);
      op.b.load(rb0, r_begin + TR, r_end - r_begin - TR);
    }
    lds_barrier();
    for (int s = 0; s < nst; ++s) {
      // stage s from LDS buffer s&1; stage s+1 (registers) -> the other
      // buffer; then stage s+2 -> registers
      const int cur = s & 1;
      compute(lds_a[cur], lds_b[cur]);
      op.a.store(ra0, lds_a[cur ^ 1], t);
      op.b.store(rb0, lds_b[cur ^ 1], t);
      const int64_t r2 = r_begin + (int64_t)(s + 2) * TR;
      op.a.load(ra0, r2, r_end - r2);
      op.b.load(rb0, r2, r_end - r2);
      lds_barrier();
    }
  } else {
  if (nst > 0) {
    op.a.load(ra0, r_begin, r_end - r_begin);
    op.b.load(rb0, r_begin, r_end - r_begin);
    op.a.load(ra1, r_begin + TR, r_end - r_begin - TR);
    op.b.load(rb1, r_begin + TR, r_end - r_begin - TR);
    op.a.store(ra0, lds_a[0], t);
    op.b.store(rb0, lds_b[0], t);
  }
  lds_barrier();
  for (int s = 0; s < nst; s += 2) {
    // stage s from LDS buffer 0; stage s+1 (register set 1) -> LDS buffer 1;
    // stage s+2 -> register set 0
    int64_t r2 = r_begin + (int64_t)(s + 2) * TR;
    op.a.load(ra0, r2, r_end - r2);
    op.b.load(rb0, r2, r_end - r2);
    compute(lds_a[0], lds_b[0]);
    op.a.store(ra1, lds_a[1], t);
    op.b.store(rb1, lds_b[1], t);
    if (SCHED) sched_stage<2 * NI * NJ, NI + NJ, NLD, NWR, NV>();
    lds_barrier();
    if (s + 1 >= nst) break;
    r2 += TR;
    op.a.load(ra1, r2, r_end - r2);
    op.b.load(rb1, r2, r_end - r2);
    compute(lds_a[1], lds_b[1]);
    op.a.store(ra0, lds_a[0], t);
    op.b.store(rb0, lds_b[0], t);
    if (SCHED) sched_stage<2 * NI * NJ, NI + NJ, NLD, NWR, NV>();
    lds_barrier();
  }
  }

  static_assert(sizeof(lds_a) >= (size_t)BI * (BJ + 8) * 2, "output staging fits in the A tiles");
  epilogue<MODE, NI, NJ, BI, BJ, WI * WJ>(g, acc, i0, j0, wi * WTI, wj * WTJ, split, slot, wave, t, NT,
                                           &lds_a[0][0]);
}

// ---- the role-split kernel ----------------------------------------------------
// 8 waves: waves 0-3 compute (LDS fragments -> MFMA, a 2 x 2 grid of
// BI/2 x BJ/2 wave tiles), waves 4-7 produce (global loads two stages ahead,
// decode, LDS writes).  A compute wave and a producer wave share each SIMD,
// so the producer's VALU work runs while the compute wave's MFMAs execute.
// One LDS-only barrier per stage; both roles pass the same number of them.
template <int MODE, int BI, int BJ>
__global__ __launch_bounds__(512, 1) void gemm_ws_kernel(GemmArgs g) {
  constexpr int NP = 256;   // producer threads
  constexpr int WTI = BI / 2, WTJ = BJ / 2;
  constexpr int NI = WTI / 16, NJ = WTJ / 16;
  static_assert(WTI % 16 == 0 && WTJ % 16 == 0, "wave tile must be a multiple of 16");
  typedef Ops<MODE, BI, BJ, NP> OpsT;
  constexpr int LA = decltype(OpsT::a)::LROWS, LB = decltype(OpsT::b)::LROWS;
  static_assert(LA >= BI && LB >= BJ, "LDS tile rows");
  __shared__ __attribute__((aligned(16))) uint16_t lds_a[2][LA * LDS_STRIDE];
  __shared__ __attribute__((aligned(16))) uint16_t lds_b[2][LB * LDS_STRIDE];

  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const bool producer = wave >= 4;
  const int wg = blockIdx.x;
  int split, bi, bj;
  split_tile_of(wg, g.tiles_i, g.tiles_j, g.splits, split, bi, bj, g.gi > 0 ? g.gi : 8);
  const int64_t i0 = (int64_t)bi * BI, j0 = (int64_t)bj * BJ;
  const int64_t r_begin = (int64_t)split * g.r_split;
  const int64_t r_end = min(g.R, r_begin + g.r_split);
  const int nst = r_end > r_begin ? (int)((r_end - r_begin + TR - 1) / TR) : 0;

  f32x4 acc[NI][NJ];
#pragma unroll
  for (int x = 0; x < NI; ++x)
#pragma unroll
    for (int y = 0; y < NJ; ++y) acc[x][y] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int wi = (wave & 3) >> 1, wj = wave & 1;

  if (producer) {
    const int tp = t - NP;
    OpsT op;
    op.init(g, i0, j0, tp);
    typename decltype(op.a)::Raw ra0, ra1;
    typename decltype(op.b)::Raw rb0, rb1;
    // stage 0 -> set 0 -> LDS 0; stage 1 -> set 1; stage 2 -> set 0
    op.a.load(ra0, r_begin, r_end - r_begin);
    op.b.load(rb0, r_begin, r_end - r_begin);
    op.a.load(ra1, r_begin + TR, r_end - r_begin - TR);
    op.b.load(rb1, r_begin + TR, r_end - r_begin - TR);
    op.a.store(ra0, lds_a[0], tp);
    op.b.store(rb0, lds_b[0], tp);
    op.a.load(ra0, r_begin + 2 * TR, r_end - r_begin - 2 * TR);
    op.b.load(rb0, r_begin + 2 * TR, r_end - r_begin - 2 * TR);
    lds_barrier();
    for (int s = 0; s < nst; s += 2) {
      // while stage s is computed: stage s+1 (set 1) -> LDS 1, stage s+3 -> set 1
      int64_t r3 = r_begin + (int64_t)(s + 3) * TR;
      op.a.store(ra1, lds_a[1], tp);
      op.b.store(rb1, lds_b[1], tp);
      op.a.load(ra1, r3, r_end - r3);
      op.b.load(rb1, r3, r_end - r3);
      lds_barrier();
      if (s + 1 >= nst) break;
      // while stage s+1 is computed: stage s+2 (set 0) -> LDS 0, stage s+4 -> set 0
      r3 += TR;
      op.a.store(ra0, lds_a[0], tp);
      op.b.store(rb0, lds_b[0], tp);
      op.a.load(ra0, r3, r_end - r3);
      op.b.load(rb0, r3, r_end - r3);
      lds_barrier();
    }
  } else {
    lds_barrier();
    for (int s = 0; s < nst; ++s) {
      stage_mfma<NI, NJ>(acc, lds_a[s & 1], lds_b[s & 1], wi * WTI, wj * WTJ, lane);
      lds_barrier();
    }
  }

  static_assert(sizeof(lds_a) >= (size_t)BI * (BJ + 8) * 2, "output staging fits in the A tiles");
  epilogue<MODE, NI, NJ, BI, BJ, 4>(g, acc, i0, j0, wi * WTI, wj * WTJ, split, bi * g.tiles_j + bj, producer ? -1 : wave,
                                     t, 512, &lds_a[0][0]);
}

// ---- LDS-DMA kernel ------------------------------------------------------------
// The A operand (bf16 rows, r contiguous) goes from global memory straight
// into LDS (buffer_load ... lds, 16 bytes per lane: lane l of a wave
// instruction writes LDS bytes [16 l, 16 l + 16) above the instruction's base;
// an out-of-range lane writes zeros).  A stage of A is an unpadded LDS tile of
// 128-byte rows; chunk c (8 bf16) of row r sits in slot c ^ ((r >> 1) & 7), so
// the 16 rows of one MFMA fragment read fall in 16 distinct bank groups.  The
// loads need no VGPRs, so the compute waves issue them themselves, three
// stages ahead in a ring of three LDS tiles.
typedef __attribute__((address_space(3))) void* lds_ptr_t;

// One LDS-DMA buffer load, issued as inline assembly so the compiler does not
// track it: it cannot tell which ring slot a DMA writes and would otherwise
// wait for every outstanding DMA before any LDS read.  The kernel waits for
// its DMAs itself (vmcnt) before each barrier and before it ends.
CONCORD_DEV void dma16(i32x4 rsrc, uint32_t voff, uint32_t soff, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %3\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
               :
               : "v"(voff), "s"(rsrc), "s"(soff), "s"(lds_base)
               : "memory", "m0");
}
CONCORD_DEV uint32_t lds_addr(const void* p) {
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(uintptr_t)(lds_ptr_t)p);
}

template <int ROWS, int NW>
struct RowsDma {
  static constexpr int INSTR = ROWS / 8;   // wave instructions per stage (8 rows each)
  static constexpr int PER = INSTR / NW;   // per issuing wave
  static_assert(PER * NW == INSTR, "rows must split evenly over the issuing waves");
  uint32_t voff[PER];
  int32_t kcq[PER];   // r offset of this lane's chunk, for the reduction tail
  i32x4 rs;
  int w;
  CONCORD_DEV void init(const uint16_t* band, int64_t ld, int64_t rows_left, int64_t R, int wave, int lane) {
    w = wave;
    // raw buffer descriptor: base address, stride 0, num_records, dword 3
    const uint64_t base = (uint64_t)(uintptr_t)band;
    rs = i32x4{(int32_t)(uint32_t)base, (int32_t)(uint32_t)((base >> 32) & 0xFFFF),
               (int32_t)nrec(((rows_left - 1) * ld + R) * 2), 0x00020000};
    for (int e = 0; e < 4; ++e) rs[e] = __builtin_amdgcn_readfirstlane(rs[e]);
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int r = (w * PER + q) * 8 + lane / 8;
      const int c = (lane % 8) ^ ((r >> 1) & 7);
      kcq[q] = c * 8;
      voff[q] = r < rows_left ? (uint32_t)((r * ld + c * 8) * 2) : kOOB;
    }
  }
  // tile = LDS tile of this stage (ROWS x 64 bf16)
  CONCORD_DEV void load(uint16_t* tile, int64_t r0, int64_t rem) const {
    const uint32_t so = uni((uint32_t)(r0 * 2));
    const uint32_t base = lds_addr(tile);
#pragma unroll
    for (int q = 0; q < PER; ++q)
      dma16(rs, kcq[q] < rem ? voff[q] : kOOB, so, uni(base + (uint32_t)((w * PER + q) * 1024)));
  }
};

// ---- implicit-GEMM convolution: gathered row operands ----------------------
// exact m / d for 0 <= m < 2^24, (mg, sh) from conv_magic(d)
CONCORD_DEV int32_t cdivm(int32_t m, uint32_t mg, int32_t sh) {
  return (int32_t)(((uint64_t)(uint32_t)m * mg) >> sh);
}

// RowsDma's tile (ROWS rows x 64 columns per stage, same LDS layout and
// swizzle) for a conv GEMM whose rows are positions and whose 64 stage
// columns are channels c0 .. c0 + 63 of one tap.
//   !DG (forward): row = output position (b, ho, wo); the row of the stage
//       reads x[b][ho sh - ph + ky][wo sw - pw + kx][c0 ..], 0 outside.
//   DG (dgrad): row = input position (b, h, w); it reads
//       dy[b][(h + ph - ky) / sh][(w + pw - kx) / sw][c0 ..] where the
//       division is exact and lands inside the output grid, 0 otherwise.
// MASK (kernels with at most kMaskTaps taps): init resolves each row's taps
// once into a bit mask of the taps that fall outside (or, DG, between) the
// grid's positions and the byte offset of its tap-(0, 0) position; a stage
// then adds the tap's offset, the same for every row (for DG as well: for
// the taps whose division is exact, (h + ph - ky) >> s = ((h + ph) >> s) -
// (ky >> s)), and sets bit 31 for a masked tap, which puts the load past
// the buffer (num_records < 2^30).  Four VALU ops per row and stage instead
// of the bounds arithmetic.  The stages a block loads past its reduction
// range (at most two, tap index below taps + 2 <= 31) read masked or
// ignored data.
constexpr int kMaskTaps = 29;
template <int ROWS, int NW, bool DG, bool MASK = false>
struct RowsDmaConv {
  static constexpr int INSTR = ROWS / 8;
  static constexpr int PER = INSTR / NW;
  static_assert(PER * NW == INSTR, "rows must split evenly over the issuing waves");
  uint32_t kc2[PER];          // byte offset of this lane's 8-channel chunk in the stage
  int32_t yy[PER], xx[PER];   // !DG: y, x of tap (0, 0); DG: h + ph, w + pw
  int32_t bb[PER];            // b * Hg; -1 for rows past the GEMM's last row
  uint32_t moff[PER], inv[PER];   // MASK: tap-(0, 0) byte offset, masked taps
  i32x4 rs;
  int w;
  int32_t C, Hg, Wg, kw, slh, slw;
  CONCORD_DEV void init(const GemmArgs& g, int64_t i0, int wave, int lane) {
    const ConvIdx& c = g.cv;
    w = wave;
    C = c.C;
    Hg = c.Hg;
    Wg = c.Wg;
    kw = c.kw;
    slh = c.slh;
    slw = c.slw;
    const uint64_t base = (uint64_t)(uintptr_t)g.a;
    rs = i32x4{(int32_t)(uint32_t)base, (int32_t)(uint32_t)((base >> 32) & 0xFFFF), (int32_t)c.act_bytes,
               0x00020000};
    for (int e = 0; e < 4; ++e) rs[e] = __builtin_amdgcn_readfirstlane(rs[e]);
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int r = (w * PER + q) * 8 + lane / 8;
      const int cc = (lane % 8) ^ ((r >> 1) & 7);
      kc2[q] = (uint32_t)(cc * 16);
      yy[q] = xx[q] = 0;
      bb[q] = -1;
      if (i0 + r < g.I) {
        const int32_t m = (int32_t)(i0 + r);
        const int32_t t = cdivm(m, c.mw, c.shw);
        const int32_t xr = m - t * c.Wr;
        const int32_t b = cdivm(t, c.mh, c.shh);
        const int32_t yr = t - b * c.Hr;
        yy[q] = DG ? yr + c.ph : (yr << c.slh) - c.ph;
        xx[q] = DG ? xr + c.pw : (xr << c.slw) - c.pw;
        bb[q] = b * c.Hg;
      }
      if constexpr (MASK) {
        // taps = kh * kw <= kMaskTaps; row ky and column kx of the kernel
        const int32_t kh = (int32_t)(g.R / C) / kw;
        uint32_t colv = 0;   // kernel columns kx that land on a position
        for (int32_t kx = 0; kx < kw; ++kx) {
          const int32_t xn = DG ? xx[q] - kx : xx[q] + kx;
          const bool ok = DG ? (xn >= 0 && (xn & ((1 << slw) - 1)) == 0 && (xn >> slw) < Wg)
                             : (xn >= 0 && xn < Wg);
          colv |= ok ? 1u << kx : 0u;
        }
        uint32_t valid = 0;
        for (int32_t ky = 0; ky < kh; ++ky) {
          const int32_t yn = DG ? yy[q] - ky : yy[q] + ky;
          const bool ok = DG ? (yn >= 0 && (yn & ((1 << slh) - 1)) == 0 && (yn >> slh) < Hg)
                             : (yn >= 0 && yn < Hg);
          valid |= ok ? colv << (ky * kw) : 0u;
        }
        inv[q] = bb[q] >= 0 ? ~valid : ~0u;
        const int32_t y0 = DG ? yy[q] >> slh : yy[q], x0 = DG ? xx[q] >> slw : xx[q];
        moff[q] = (uint32_t)(((bb[q] + y0) * Wg + x0) * (C * 2)) + kc2[q];
      }
    }
  }
  CONCORD_DEV void load(uint16_t* tile, int64_t r0, int64_t rem) const {
    if constexpr (MASK) {
      const int32_t tap = (int32_t)r0 / C;
      const int32_t c0 = (int32_t)r0 - tap * C;
      const int32_t ky = tap / kw, kx = tap - ky * kw;
      const int32_t toff = DG ? -(((ky >> slh) * Wg + (kx >> slw)) * (C * 2)) : (ky * Wg + kx) * (C * 2);
      const uint32_t so = uni((uint32_t)c0 * 2u);
      const uint32_t base = lds_addr(tile);
#pragma unroll
      for (int q = 0; q < PER; ++q) {
        const uint32_t vo = (moff[q] + (uint32_t)toff) | (__builtin_amdgcn_ubfe(inv[q], (uint32_t)tap, 1u) << 31);
        dma16(rs, vo, so, uni(base + (uint32_t)((w * PER + q) * 1024)));
      }
      return;
    }
    const int32_t tap = (int32_t)r0 / C;
    const int32_t c0 = (int32_t)r0 - tap * C;
    const int32_t ky = tap / kw, kx = tap - ky * kw;
    const uint32_t so = uni((uint32_t)c0 * 2u);
    const uint32_t base = lds_addr(tile);
    const int32_t mh = (1 << slh) - 1, mw = (1 << slw) - 1;
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      int32_t y, x;
      bool ok;
      if (!DG) {
        y = yy[q] + ky;
        x = xx[q] + kx;
        ok = (uint32_t)y < (uint32_t)Hg && (uint32_t)x < (uint32_t)Wg;
      } else {
        const int32_t yn = yy[q] - ky, xn = xx[q] - kx;
        y = yn >> slh;
        x = xn >> slw;
        ok = yn >= 0 && xn >= 0 && (yn & mh) == 0 && (xn & mw) == 0 && y < Hg && x < Wg;
      }
      ok = ok && bb[q] >= 0 && (int64_t)(kc2[q] >> 1) < rem;
      const uint32_t vo = ok ? ((uint32_t)(bb[q] + y) * (uint32_t)Wg + (uint32_t)x) * (uint32_t)(C * 2) + kc2[q]
                            : kOOB;
      dma16(rs, vo, so, uni(base + (uint32_t)((w * PER + q) * 1024)));
    }
  }
};

// MFMAs of one stage: A and B from [row][64] tiles whose 16-byte chunk c of
// row r sits at chunk c ^ ((r >> 1) & 7) (the A tile written by DMA, the B
// tile by the producer waves' store_swz); ra and rb are multiples of 16
template <int NI, int NJ>
CONCORD_DEV void stage_mfma_swz(f32x4 (&acc)[NI][NJ], const uint16_t* la, const uint16_t* lb, int ra, int rb,
                                int lane) {
  const int lrow = lane & 15;
  const int sw = (lane & 14) >> 1;   // (row >> 1) & 7 for row = ra + 16x + lrow (or rb + 16y + lrow)
#pragma unroll
  for (int kk = 0; kk < TR / 32; ++kk) {
    const int aoff = lrow * 64 + (((kk * 4 + (lane >> 4)) ^ sw) * 8);
    bf16x8 fa[NI], fb[NJ];
#pragma unroll
    for (int x = 0; x < NI; ++x)
      fa[x] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const i32x4*>(la + (ra + x * 16) * 64 + aoff));
#pragma unroll
    for (int y = 0; y < NJ; ++y)
      fb[y] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const i32x4*>(lb + (rb + y * 16) * 64 + aoff));
#pragma unroll
    for (int x = 0; x < NI; ++x)
#pragma unroll
      for (int y = 0; y < NJ; ++y)
        acc[x][y] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[y], fa[x], acc[x][y], 0, 0, 0);
  }
}

// B-side loader per mode (the A side is RowsDma for every mode here)
template <int MODE, int BJ, int NT> struct BSide;
template <int BJ, int NT> struct BSide<MODE_FWD, BJ, NT> {
  RowsPacked<BJ, NT> b;
  CONCORD_DEV void init(const GemmArgs& g, int64_t j0, int t) {
    b.init(reinterpret_cast<const int32_t*>(g.b) + j0 * g.ldb, g.ldb, g.J - j0, g.R, g.col_exp, t);
  }
};
template <int BJ, int NT> struct BSide<MODE_FWD_BF16, BJ, NT> {
  RowsBf16<BJ, NT> b;
  CONCORD_DEV void init(const GemmArgs& g, int64_t j0, int t) {
    b.init(reinterpret_cast<const uint16_t*>(g.b) + j0 * g.ldb, g.ldb, g.J - j0, g.R, t);
  }
};
template <int BJ, int NT> struct BSide<MODE_DGRAD, BJ, NT> {
  ColsPacked<BJ, NT> b;
  CONCORD_DEV void init(const GemmArgs& g, int64_t j0, int t) {
    b.init(reinterpret_cast<const int32_t*>(g.b) + j0, g.ldb, g.J - j0, g.R, g.row_exp, t);
  }
};
template <int BJ, int NT> struct BSide<MODE_DGRAD_BF16, BJ, NT> {
  ColsBf16<BJ, NT> b;
  CONCORD_DEV void init(const GemmArgs& g, int64_t j0, int t) {
    b.init(reinterpret_cast<const uint16_t*>(g.b) + j0, g.ldb, g.J - j0, g.R, t);
  }
};

// 8 waves: waves 0-3 compute and move A by DMA (stage s+2 while computing s),
// waves 4-7 load B three stages ahead in registers, decode it and write it
// into a double-buffered swizzled LDS tile (the A tile's layout).  One LDS
// barrier per stage; before it every compute wave waits until its own DMA of
// the next stage has landed.
// CONV: the A operand is the conv forward's gathered x (RowsDmaConv).
template <int MODE, int BI, int BJ, int CONV = 0>
__global__ __launch_bounds__(512, 1) void gemm_dma_kernel(GemmArgs g) {
  constexpr int NP = 256;
  constexpr int WTI = BI / 2, WTJ = BJ / 2;
  constexpr int NI = WTI / 16, NJ = WTJ / 16;
  typedef BSide<MODE, BJ, NP> BS;
  typedef typename std::conditional<CONV != 0, RowsDmaConv<BI, 4, false, CONV == 1>, RowsDma<BI, 4>>::type AD;
  constexpr int LB = decltype(BS::b)::LROWS;
  static_assert(LB >= BJ, "LDS tile rows");
  __shared__ __attribute__((aligned(1024))) uint16_t lds_a[3][BI * 64];
  __shared__ __attribute__((aligned(1024))) uint16_t lds_b[2][LB * 64];

  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const bool producer = wave >= 4;
  const int wg = blockIdx.x;
  int split, bi, bj, slot;
  gemm_tile_of<BI, BJ>(g, wg, split, bi, bj, slot);
  const int64_t i0 = (int64_t)bi * BI, j0 = (int64_t)bj * BJ;
  const int64_t r_begin = (int64_t)split * g.r_split;
  const int64_t r_end = min(g.R, r_begin + g.r_split);
  const int nst = r_end > r_begin ? (int)((r_end - r_begin + TR - 1) / TR) : 0;
  // both roles pass an even number of stage barriers; the producers' extra
  // stage reads zeros (out-of-range loads) and the compute waves skip it
  const int nst2 = (nst + 1) & ~1;

  f32x4 acc[NI][NJ];
#pragma unroll
  for (int x = 0; x < NI; ++x)
#pragma unroll
    for (int y = 0; y < NJ; ++y) acc[x][y] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int wi = (wave & 3) >> 1, wj = wave & 1;

  if (producer) {
    const int tp = t - NP;
    BS bs;
    bs.init(g, j0, tp);
    typename decltype(bs.b)::Raw r0, r1;
    auto stage_r = [&](int st) { return r_begin + (int64_t)st * TR; };
    bs.b.load(r0, stage_r(0), r_end - stage_r(0));
    bs.b.load(r1, stage_r(1), r_end - stage_r(1));
    bs.b.store_swz(r0, lds_b[0], tp);
    bs.b.load(r0, stage_r(2), r_end - stage_r(2));
    lds_barrier();
    // iteration s: stage s+1 -> LDS buffer (s+1)&1, then stage s+3 into its
    // registers.  Two sets in flight measured faster than three (deeper
    // prefetch only adds L2 pressure).  One back-edge and no early exit, so
    // the compiler sees the same order of outstanding loads from the prologue
    // and from the loop.
    for (int s = 0; s < nst2; s += 2) {
      bs.b.store_swz(r1, lds_b[1], tp);
      bs.b.load(r1, stage_r(s + 3), r_end - stage_r(s + 3));
      lds_barrier();
      bs.b.store_swz(r0, lds_b[0], tp);
      bs.b.load(r0, stage_r(s + 4), r_end - stage_r(s + 4));
      lds_barrier();
    }
  } else {
    AD ad;
    if constexpr (CONV) ad.init(g, i0, wave, lane);
    else ad.init(g.a + i0 * g.lda, g.lda, g.I - i0, g.R, wave, lane);
    ad.load(lds_a[0], r_begin, r_end - r_begin);
    ad.load(lds_a[1], r_begin + TR, r_end - r_begin - TR);
    // own DMA of stage 0 landed (stage 1's PER loads may still fly)
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(AD::PER));
    lds_barrier();
    // stage s reads A slot s % 3 and B slot s % 2; unrolled by their period
    // of six (constant slot addresses; the gathered conv operand's DMA then
    // needs no per-stage LDS base arithmetic); nst2 is even, so two or four
    // stages remain after the unrolled loop
    auto cstage = [&](int s, auto ph) {
      constexpr int P = decltype(ph)::value;
      const int64_t r2 = r_begin + (int64_t)(s + 2) * TR;
      ad.load(lds_a[(P + 2) % 3], r2, r_end - r2);
      if (s < nst) stage_mfma_swz<NI, NJ>(acc, lds_a[P % 3], lds_b[P & 1], wi * WTI, wj * WTJ, lane);
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(AD::PER));
      lds_barrier();
    };
    int s = 0;
    for (; s + 6 <= nst2; s += 6) {
      cstage(s, std::integral_constant<int, 0>());
      cstage(s + 1, std::integral_constant<int, 1>());
      cstage(s + 2, std::integral_constant<int, 2>());
      cstage(s + 3, std::integral_constant<int, 3>());
      cstage(s + 4, std::integral_constant<int, 4>());
      cstage(s + 5, std::integral_constant<int, 5>());
    }
    if (s < nst2) {
      cstage(s, std::integral_constant<int, 0>());
      cstage(s + 1, std::integral_constant<int, 1>());
    }
    if (s + 2 < nst2) {
      cstage(s + 2, std::integral_constant<int, 2>());
      cstage(s + 3, std::integral_constant<int, 3>());
    }
    // no DMA may still be writing LDS when the block ends
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  }

  static_assert(sizeof(lds_a) >= (size_t)BI * (BJ + 8) * 2, "output staging fits in the A tiles");
  epilogue<MODE, NI, NJ, BI, BJ, 4>(g, acc, i0, j0, wi * WTI, wj * WTJ, split, slot, producer ? -1 : wave,
                                     t, 512, &lds_a[0][0]);
}

// ---- WGRAD: both operands by DMA, fragments by transpose reads -------------
// Both WGRAD operands are r-major (dy[m][n], x[m][k]), and an MFMA fragment
// needs 8 consecutive r of one column per lane.  A stage of each operand goes
// from global memory straight into LDS by DMA as a row-major [r][col] tile,
// and ds_read_b64_tr_b16 turns it around: in each 16-lane group, lane p
// addresses row r0 + (p >> 2), columns c0 + 4 (p & 3) .. +3, and receives
// column c0 + p of rows r0 .. r0 + 3.  Two such reads make one fragment.
// LDS layout of a stage tile (ROWB bytes per row): the 32-byte window w of
// row r is stored at window w ^ trf(r), trf(r) = (r & 3) | ((r >> 1) & 4), so
// the 8 rows one half-wave touches (r0 .. r0+3 and r0+8 .. r0+11, r0 a
// multiple of 4) fall in 8 distinct 32-byte bank groups.
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

CONCORD_DEV int trf(int r) { return (r & 3) | ((r >> 1) & 4); }

// DMA of one operand's stage: TR rows x COLS bf16 (COLS >= 128 so that the
// window swizzle stays inside a row)
template <int COLS, int NW>
struct TrDma {
  static constexpr int ROWB = COLS * 2;        // bytes per LDS row
  static constexpr int RPI = 1024 / ROWB;      // rows per wave instruction (1 KB)
  static constexpr int INSTR = TR / RPI;
  static constexpr int PER = INSTR / NW;       // per wave
  static_assert(COLS >= 128 && COLS <= 512 && PER * NW == INSTR, "TrDma tile");
  uint32_t voff[PER];   // kOOB for chunks past the operand's last column
  int32_t lrow;         // this lane's row within an instruction
  i32x4 rs;
  int64_t ld2;
  int w;
  // band = operand + first column of the tile; cols_left = columns from there
  CONCORD_DEV void init(const uint16_t* band, int64_t ld, int64_t cols_left, int64_t R, int wave, int lane) {
    w = wave;
    ld2 = ld * 2;
    lrow = lane / (ROWB / 16);
    const uint64_t base = (uint64_t)(uintptr_t)band;
    const int64_t bytes = ((R - 1) * ld + (cols_left < COLS ? cols_left : COLS)) * 2;
    rs = i32x4{(int32_t)(uint32_t)base, (int32_t)(uint32_t)((base >> 32) & 0xFFFF), (int32_t)nrec(bytes),
               0x00020000};
    for (int e = 0; e < 4; ++e) rs[e] = __builtin_amdgcn_readfirstlane(rs[e]);
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int r = (w * PER + q) * RPI + lrow;
      const int c = (lane % (ROWB / 16)) ^ (trf(r) << 1);   // 16-byte chunk this lane's slot holds
      voff[q] = c * 8 < cols_left ? (uint32_t)((r * ld + c * 8) * 2) : kOOB;
    }
  }
  // tile = LDS byte address of this operand's stage tile; rows r0 + [0, TR)
  CONCORD_DEV void load(uint32_t tile, int64_t r0, int64_t rem) const {
    const uint32_t so = uni(rem > 0 ? (uint32_t)(r0 * ld2) : 0u);
    const int rem32 = (int)(rem < TR ? rem : TR);
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int row0 = (w * PER + q) * RPI;
      dma16(rs, lrow < rem32 - row0 ? voff[q] : kOOB, so, uni(tile + (uint32_t)((w * PER + q) * 1024)));
    }
  }
};

// TrDma's tile (TR rows x COLS columns, same layout and swizzle) for the
// WGRAD of a conv: rows are output positions m = (b, ho, wo) (the
// reduction), columns r = tap * C + c of the patch matrix; the lane's 8
// columns read x[b][ho sh - ph + ky][wo sw - pw + kx][c ..], 0 outside.
template <int COLS, int NW>
struct TrDmaConv {
  static constexpr int ROWB = COLS * 2;
  static constexpr int RPI = 1024 / ROWB;
  static constexpr int INSTR = TR / RPI;
  static constexpr int PER = INSTR / NW;
  static_assert(COLS >= 128 && COLS <= 512 && PER * NW == INSTR, "TrDma tile");
  uint32_t cin2[PER];          // byte offset of this lane's 8 channels within a position
  int32_t oy[PER], ox[PER];    // ky - ph, kx - pw of their tap; oy huge negative past the tile's columns
  int32_t lrow;
  i32x4 rs;
  int w;
  int32_t Cb2, Hg, Wg, Hr, Wr, slh, slw, shw, shh;
  uint32_t mw, mh;
  CONCORD_DEV void init(const GemmArgs& g, int64_t j0, int wave, int lane) {
    const ConvIdx& c = g.cv;
    w = wave;
    Cb2 = c.C * 2;
    Hg = c.Hg;
    Wg = c.Wg;
    Hr = c.Hr;
    Wr = c.Wr;
    slh = c.slh;
    slw = c.slw;
    mw = c.mw;
    mh = c.mh;
    shw = c.shw;
    shh = c.shh;
    lrow = lane / (ROWB / 16);
    const uint64_t base = (uint64_t)(uintptr_t)g.b;
    rs = i32x4{(int32_t)(uint32_t)base, (int32_t)(uint32_t)((base >> 32) & 0xFFFF), (int32_t)c.act_bytes,
               0x00020000};
    for (int e = 0; e < 4; ++e) rs[e] = __builtin_amdgcn_readfirstlane(rs[e]);
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int r = (w * PER + q) * RPI + lrow;
      const int cc = (lane % (ROWB / 16)) ^ (trf(r) << 1);
      cin2[q] = 0;
      oy[q] = -(1 << 28);
      ox[q] = 0;
      if (cc * 8 < g.J - j0) {
        const int32_t col = (int32_t)(j0 + cc * 8);
        const int32_t tap = col / c.C;
        const int32_t ky = tap / c.kw;
        cin2[q] = (uint32_t)((col - tap * c.C) * 2);
        oy[q] = ky - c.ph;
        ox[q] = tap - ky * c.kw - c.pw;
      }
    }
  }
  CONCORD_DEV void load(uint32_t tile, int64_t r0, int64_t rem) const {
    const int rem32 = (int)(rem < TR ? rem : TR);
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int rl = (w * PER + q) * RPI + lrow;
      const int32_t m = (int32_t)r0 + rl;
      const int32_t t = cdivm(m, mw, shw);
      const int32_t xo = m - t * Wr;
      const int32_t b = cdivm(t, mh, shh);
      const int32_t yo = t - b * Hr;
      const int32_t y = (yo << slh) + oy[q], x = (xo << slw) + ox[q];
      const bool ok = rl < rem32 && (uint32_t)y < (uint32_t)Hg && (uint32_t)x < (uint32_t)Wg;
      const uint32_t vo =
          ok ? ((uint32_t)(b * Hg + y) * (uint32_t)Wg + (uint32_t)x) * (uint32_t)Cb2 + cin2[q] : kOOB;
      dma16(rs, vo, 0u, uni(tile + (uint32_t)((w * PER + q) * 1024)));
    }
  }
};

typedef __attribute__((address_space(3))) char lds_char;

// fragments of reduction step kk (32 r) of a stage tile for the 16-column
// groups cw0 .. cw0 + NF - 1.  lbase = (8 (lane >> 4) + (lane & 15) / 4) ROWB
// + 8 (lane & 3); fsw = trf of every row this lane reads, times 32.
template <int NF, int ROWB>
CONCORD_DEV void tr_frags(bf16x8 (&fr)[NF], const lds_char* tile, uint32_t lbase, uint32_t fsw, int cw0, int kk) {
#pragma unroll
  for (int x = 0; x < NF; ++x) {
    const lds_char* q = tile + (lbase + ((uint32_t)((cw0 + x) * 32) ^ fsw)) + kk * 32 * ROWB;
    const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)q);
    const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(q + 4 * ROWB));
    fr[x] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  }
}

template <int NI, int NJ>
CONCORD_DEV void mfma_block(f32x4 (&acc)[NI][NJ], const bf16x8 (&fa)[NI], const bf16x8 (&fb)[NJ]) {
#pragma unroll
  for (int x = 0; x < NI; ++x)
#pragma unroll
    for (int y = 0; y < NJ; ++y)
      acc[x][y] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[y], fa[x], acc[x][y], 0, 0, 0);
}

// WI x WJ waves, each BI/WI x BJ/WJ; every wave computes and issues its share
// of both operands' DMA.  Ring of three stages: stage s + 3 is loaded into
// the slot of stage s as soon as every wave has finished reading stage s.
// Per stage: fragments of the second half-stage are read while the first
// half-stage's MFMAs issue, then (after the barrier) the next stage's first
// half is read while the second half's MFMAs issue.
// bias-gradient partial of one wave: sum_r a(i, r) for each of its
// i-fragments, as an MFMA against an all-ones operand (every output column
// j of the 16 x 16 block then holds the same column sum)
template <int NI>
CONCORD_DEV void bias_acc(f32x4 (&b)[NI], const bf16x8 (&fa)[NI]) {
  const bf16x8 ones = {(__bf16)1.0f, (__bf16)1.0f, (__bf16)1.0f, (__bf16)1.0f,
                       (__bf16)1.0f, (__bf16)1.0f, (__bf16)1.0f, (__bf16)1.0f};
#pragma unroll
  for (int x = 0; x < NI; ++x) b[x] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, fa[x], b[x], 0, 0, 0);
}

// VH: also write the v-hat partials of the bf16-rounded output (64 x 64 wave
// tiles, vhat_tile.h order); only without split-K (a split launch forms them
// in splitk_reduce_vh_kernel).  With g.bpart set, the waves wj = 0 of block
// (bi, bj) of split sp also sum the A operand over the split's stages
// s = bj, bj + tiles_j, ... (an MFMA against ones per fragment, fp32
// accumulation), giving bpart[sp * tiles_j + bj][i]; the bias gradient is the
// sum of the partials over that row index ascending (vhat_finalize).
// The split-K reduction shape of the dgrad kernel (gemm_dgt_kernel<DGRAD, 256,
// 128>, 2 x 2 accumulator waves of 128 x 64), which a VH launch can carry.
#define CONCORD_DGRAD_REDUCE MODE_DGRAD, RBI / 32, 4, RBI, 128, 2, 2

// Workgroups [0, tr_blocks) compute WGRAD tiles.  A VH launch may carry more:
// workgroups from tr_blocks on run the split-K reduction `rd` of the dgrad
// kernel issued just before on the stream, on the CUs the WGRAD grid leaves
// idle (200 tiles on 256 CUs at 1280 -> 5120).
// CONV: the B operand (x) is the conv wgrad's gathered patch matrix (TrDmaConv).
// UPD (1 bare, 2 winner; VH launches with the dgrad reduction only): the
// launch also carries the v-hat finalize and the packed update
// (wgrad_update.h); every workgroup meets the grid barriers, the WGRAD
// workgroups update their tiles from the accumulators, and the bf16 weight
// gradient is stored only when g.c is set.
template <int BI, int BJ, int WI, int WJ, bool VH, bool CONV, int RBI, int UPD>
CONCORD_DEV void gemm_tr_body(const GemmArgs& g, const GemmArgs& rd, int tr_blocks, const WgradUpd& u, uint32_t wg,
                              uint32_t ngrid, uint16_t* ring_mem, int* s_flag_mem) {
  constexpr int NW = WI * WJ, NT = 64 * NW, WTI = BI / WI, WTJ = BJ / WJ;
  constexpr int NI = WTI / 16, NJ = WTJ / 16;
  typedef TrDma<BI, NW> DA;
  typedef typename std::conditional<CONV, TrDmaConv<BJ, NW>, TrDma<BJ, NW>>::type DB;
  constexpr int ABYTES = TR * BI * 2, STAGE = ABYTES + TR * BJ * 2;
  constexpr int PERT = DA::PER + DB::PER;
  static_assert(TR == 64, "two 32-deep MFMA steps per stage");
  static_assert(UPD == 0 || (VH && !CONV && NW == 8), "the update rides on the VH launch of 8 waves");
  // the LDS ring (tr_ring_bytes, 1024-aligned) and the barrier flag
  typedef uint16_t Ring[3 * STAGE / 2];
  Ring& ring = *reinterpret_cast<Ring*>(ring_mem);
  int& s_flag = *s_flag_mem;
  static_assert(sizeof(ring) >= (size_t)BI * (BJ + 8) * 2, "output staging fits in the ring");
  if (VH && (int)wg >= tr_blocks) {
    const int64_t items = splitk_reduce_items<CONCORD_DGRAD_REDUCE>(rd);
    const int64_t stride = (int64_t)(ngrid - tr_blocks) * NT;
    for (int64_t idx = (int64_t)(wg - tr_blocks) * NT + threadIdx.x; idx < items; idx += stride)
      splitk_reduce_item<CONCORD_DGRAD_REDUCE>(rd, idx);
    if constexpr (UPD != 0) {
      if (!grid_sync(u, ngrid, &s_flag)) upd_finalize(g, u, reinterpret_cast<float*>(ring));
      grid_sync(u, 2 * ngrid, &s_flag);
      grid_exit(u);
    }
    return;
  }

  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  int split, bi, bj;
  split_tile_of(wg, g.tiles_i, g.tiles_j, g.splits, split, bi, bj, g.gi > 0 ? g.gi : 8);
  const int64_t i0 = (int64_t)bi * BI, j0 = (int64_t)bj * BJ;
  const int64_t r_begin = (int64_t)split * g.r_split;
  const int64_t r_end = min(g.R, r_begin + g.r_split);
  const int nst = r_end > r_begin ? (int)((r_end - r_begin + TR - 1) / TR) : 0;
  const int wi = wave / WJ, wj = wave % WJ;

  f32x4 acc[NI][NJ];
#pragma unroll
  for (int x = 0; x < NI; ++x)
#pragma unroll
    for (int y = 0; y < NJ; ++y) acc[x][y] = f32x4{0.f, 0.f, 0.f, 0.f};

  DA da;
  DB db;
  da.init(g.a + i0, g.lda, g.I - i0, g.R, wave, lane);
  if constexpr (CONV) db.init(g, j0, wave, lane);
  else db.init(reinterpret_cast<const uint16_t*>(g.b) + j0, g.ldb, g.J - j0, g.R, wave, lane);
  const uint32_t ring_lds = lds_addr(ring);
  const lds_char* ring_p = (const lds_char*)ring;
  auto dma_stage = [&](int s) {
    const int64_t r0 = r_begin + (int64_t)s * TR;
    const uint32_t slot = ring_lds + (uint32_t)((s % 3) * STAGE);
    da.load(slot, r0, r_end - r0);
    db.load(slot + ABYTES, r0, r_end - r0);
  };
  const int p = lane & 15, gq = lane >> 4;
  const uint32_t fsw = (uint32_t)(((p >> 2) | ((gq & 1) << 2)) * 32);
  const uint32_t la = (uint32_t)((8 * gq + (p >> 2)) * DA::ROWB + 8 * (p & 3));
  const uint32_t lb = (uint32_t)(ABYTES + (8 * gq + (p >> 2)) * DB::ROWB + 8 * (p & 3));
  const int cwa = wi * WTI / 16, cwb = wj * WTJ / 16;

  dma_stage(0);
  dma_stage(1);
  dma_stage(2);
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * PERT));   // own stage-0 DMA landed
  lds_barrier();
  bf16x8 fa0[NI], fb0[NJ], fa1[NI], fb1[NJ];
  const bool bg = g.bpart != nullptr && wj == 0;   // uniform per wave
  f32x4 bsum[NI];
#pragma unroll
  for (int x = 0; x < NI; ++x) bsum[x] = f32x4{0.f, 0.f, 0.f, 0.f};
  tr_frags<NI, DA::ROWB>(fa0, ring_p, la, fsw, cwa, 0);
  tr_frags<NJ, DB::ROWB>(fb0, ring_p, lb, fsw, cwb, 0);
  // stage s reads ring slot SL = s % 3.  The loop is unrolled by the three
  // slots so that every slot address is the ring's base plus a constant: the
  // transpose reads then take their row and sub-step offsets in the
  // instruction's offset field (one address per fragment), where a run-time
  // slot cost two VALU ops per read (76 per stage and wave, against 32 MFMAs).
  auto stage = [&](int s, auto slot) {
    constexpr int SL = decltype(slot)::value;
    const lds_char* cur = ring_p + SL * STAGE;
    tr_frags<NI, DA::ROWB>(fa1, cur, la, fsw, cwa, 1);
    tr_frags<NJ, DB::ROWB>(fb1, cur, lb, fsw, cwb, 1);
    mfma_block<NI, NJ>(acc, fa0, fb0);
    const bool bgs = bg && (s % g.tiles_j) == bj;
    if (bgs) bias_acc<NI>(bsum, fa0);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(PERT));     // own stage s+1 DMA landed
    lds_barrier();                                    // stage s fully read by every wave
    {
      // stage s + 3 into the slot stage s just left
      const int64_t r0 = r_begin + (int64_t)(s + 3) * TR;
      const uint32_t sl = ring_lds + (uint32_t)(SL * STAGE);
      da.load(sl, r0, r_end - r0);
      db.load(sl + ABYTES, r0, r_end - r0);
    }
    // after the last stage this reads a ring slot no MFMA uses (in bounds)
    const lds_char* nxt = ring_p + ((SL + 1) % 3) * STAGE;
    tr_frags<NI, DA::ROWB>(fa0, nxt, la, fsw, cwa, 0);
    tr_frags<NJ, DB::ROWB>(fb0, nxt, lb, fsw, cwb, 0);
    mfma_block<NI, NJ>(acc, fa1, fb1);
    if (bgs) bias_acc<NI>(bsum, fa1);
  };
  int s = 0;
  for (; s + 3 <= nst; s += 3) {
    stage(s, std::integral_constant<int, 0>());
    stage(s + 1, std::integral_constant<int, 1>());
    stage(s + 2, std::integral_constant<int, 2>());
  }
  if (s < nst) stage(s, std::integral_constant<int, 0>());
  if (s + 1 < nst) stage(s + 1, std::integral_constant<int, 1>());
  if (bg) {
#pragma unroll
    for (int x = 0; x < NI; ++x) {
      const int64_t i = i0 + wi * WTI + 16 * x + (lane & 15);
      if (lane < 16 && i < g.I) {
        float* dst = g.bpart + ((int64_t)split * g.tiles_j + bj) * g.I + i;
        if (UPD != 0) coh_store(dst, bsum[x][0]);
        else *dst = bsum[x][0];
      }
    }
  }
  // no DMA may still be writing LDS when the ring is reused for the output
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  if constexpr (VH) {
    static_assert(NI == 4 && NJ == 4, "v-hat partials take 64 x 64 wave tiles");
    float g2[4][4][4];
#pragma unroll
    for (int x = 0; x < 4; ++x)
#pragma unroll
      for (int y = 0; y < 4; ++y) {
        // the values the epilogue stores: acc rounded to bf16
        const uint32_t lo = pack_bf16x2(acc[x][y][0], acc[x][y][1]);
        const uint32_t hi = pack_bf16x2(acc[x][y][2], acc[x][y][3]);
        const float v[4] = {__uint_as_float(lo << 16), __uint_as_float(lo & 0xFFFF0000u),
                            __uint_as_float(hi << 16), __uint_as_float(hi & 0xFFFF0000u)};
#pragma unroll
        for (int e = 0; e < 4; ++e) g2[x][y][e] = __fmul_rn(v[e], v[e]);
      }
    vhat_tile_partials<UPD != 0>(g2, lane, i0 + wi * WTI, j0 + wj * WTJ, g.I, g.J, g.vh_pr, g.vh_pc);
  }
  if (UPD == 0 || g.c)
    epilogue<MODE_WGRAD, NI, NJ, BI, BJ, NW>(g, acc, i0, j0, wi * WTI, wj * WTJ, split, bi * g.tiles_j + bj, wave, t,
                                             NT, ring);
  if constexpr (UPD != 0) {
    const bool bad = grid_sync(u, ngrid, &s_flag);
    if (!bad) upd_finalize(g, u, reinterpret_cast<float*>(ring));
    if (!grid_sync(u, 2 * ngrid, &s_flag) && !bad) {
      int32_t* lds = reinterpret_cast<int32_t*>(ring);
      upd_apply<UPD == 2>(g, u, acc, i0, j0, wi, wj, lds, lds + 512);
    }
    grid_exit(u);
  }
}

// LDS bytes of gemm_tr_body's ring
template <int BI, int BJ>
constexpr int tr_ring_bytes() { return 3 * (TR * BI * 2 + TR * BJ * 2); }

// one LDS array per kernel: the ring at offset 0 (its swizzled addresses fold
// into instruction offsets), the barrier flag after it
template <int BI, int BJ, int WI, int WJ, bool VH, bool CONV = false, int RBI = 256>
__global__ __launch_bounds__(64 * WI * WJ, 1) void gemm_tr_kernel(GemmArgs g, GemmArgs rd, int tr_blocks) {
  __shared__ __attribute__((aligned(1024))) char lds[tr_ring_bytes<BI, BJ>() + 16];
  gemm_tr_body<BI, BJ, WI, WJ, VH, CONV, RBI, 0>(g, rd, tr_blocks, WgradUpd{}, blockIdx.x, gridDim.x,
                                                 reinterpret_cast<uint16_t*>(lds),
                                                 reinterpret_cast<int*>(lds + tr_ring_bytes<BI, BJ>()));
}

// the WGRAD launch of the backward entry carrying the finalize and the update
// (wgrad_update.h); RBI = the dgrad reduction's tile rows, UPD = 1 bare, 2 winner
template <int RBI, int UPD>
__global__ __launch_bounds__(512, 1) void wgrad_update_kernel(GemmArgs g, GemmArgs rd, int tr_blocks, WgradUpd u) {
  __shared__ __attribute__((aligned(1024))) char lds[tr_ring_bytes<256, 128>() + 16];
  gemm_tr_body<256, 128, 4, 2, true, false, RBI, UPD>(g, rd, tr_blocks, u, blockIdx.x, gridDim.x,
                                                      reinterpret_cast<uint16_t*>(lds),
                                                      reinterpret_cast<int*>(lds + tr_ring_bytes<256, 128>()));
}

// ---- DGRAD with a row-major weight tile and transpose reads -------------------
// DGRAD's weight operand W[n][k] is r-major (r = n).  The producer waves load
// two full rows of the tile per wave instruction (lane: 4 consecutive columns
// of one row), decode them with their row's exponent and write bf16 rows into
// a row-major [r][col] tile (ds_write_b64, the 32-byte windows swizzled as in
// TrDma); the compute waves read the MFMA fragments with ds_read_b64_tr_b16.
// Thread t: columns 4 (t % (COLS / 4)), rows 8 (t / (COLS / 4)) .. + 7.
// CONV (bf16 only): the weight operand of a conv dgrad, W'[n][tap][c] with
// rows r = tap * N + n of the reduction: a stage (64 rows of one tap) starts
// at n0 = r0 % N, tap = r0 / N, i.e. at W' + n0 * ld + tap * cb.
template <int COLS, int NT, bool PACKED, bool CONV = false>
struct TrRowsB {
  static_assert(!(CONV && PACKED), "the conv dgrad reads a bf16 weight");
  static constexpr int CG = COLS / 4, RG = NT / CG;
  static_assert(CG * RG == NT && 8 * RG == TR, "one 8-row group per thread covers the stage");
  static constexpr int ROWB = COLS * 2;
  static constexpr int LBYTES = TR * ROWB;   // bytes of one LDS stage tile
  typedef typename std::conditional<PACKED, i32x4, i32x2>::type Chunk;
  struct Raw { Chunk v[8]; i32x2 ex; };
  uint32_t voff;   // row 8 rg, this thread's 4 columns (kOOB past the last column)
  uint32_t ldb;    // row stride in bytes
  int32_t rg, col;
  int32_t nrows, cb2;   // CONV: rows per tap (N), bytes of a tap block (cb * 2)
  Rsrc rs, es;
  CONCORD_DEV void init(const void* band, int64_t ld, int64_t cols_left, int64_t R, const int8_t* exps, int t) {
    constexpr int ES = PACKED ? 4 : 2;
    col = 4 * (t % CG);
    rg = t / CG;
    ldb = (uint32_t)(ld * ES);
    rs = make_rsrc(band, nrec(((R - 1) * ld + cols_left) * ES));
    if (PACKED) es = make_rsrc(exps, (uint32_t)R);
    voff = col < cols_left ? (uint32_t)((8 * rg * ld + col) * ES) : kOOB;
  }
  // CONV: band = W' + first column of the tile (bf16), ld = taps * cb
  CONCORD_DEV void init_conv(const GemmArgs& g, const uint16_t* band, int64_t j0, int t) {
    col = 4 * (t % CG);
    rg = t / CG;
    ldb = (uint32_t)(g.ldb * 2);
    nrows = g.cv.C;
    cb2 = g.cv.cb * 2;
    rs = make_rsrc(band, g.cv.w_bytes - (uint32_t)(j0 * 2));
    voff = col < g.J - j0 ? (uint32_t)(8 * rg) * ldb + (uint32_t)(col * 2) : kOOB;
  }
  CONCORD_DEV void load(Raw& r, int64_t r0, int64_t rem) const {
    uint32_t so;
    if constexpr (CONV) {
      const int32_t tap = (int32_t)r0 / nrows;
      so = (uint32_t)((int32_t)r0 - tap * nrows) * ldb + (uint32_t)(tap * cb2);
    } else {
      so = (uint32_t)(r0 * (int64_t)ldb);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t o = 8 * rg + e < rem ? voff + e * ldb : kOOB;
      if constexpr (PACKED) r.v[e] = ld128(rs, o, so);
      else r.v[e] = ld64(rs, o, so);
    }
    // the 8 rows' exponents (R % 8 == 0: the 8 bytes are all in range or all out)
    if constexpr (PACKED) r.ex = ld64(es, 8 * rg < rem ? (uint32_t)(8 * rg) : kOOB, (uint32_t)r0);
  }
  // tile = LDS byte address of the stage tile
  CONCORD_DEV void store(Raw& r, char* tile) const {
    if constexpr (PACKED) pin(r.ex);
#pragma unroll
    for (int e = 0; e < 8; ++e) pin(r.v[e]);
    const int cw = col / 16, cb = 2 * (col % 16);   // 32-byte window, byte in window
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int row = 8 * rg + e;
      i32x2 o;
      if constexpr (PACKED) {
        const int32_t exw = r.ex[e / 4];
        const uint32_t M = (e % 4) == 0 ? magic_byte<0>(exw) : (e % 4) == 1 ? magic_byte<1>(exw)
                         : (e % 4) == 2 ? magic_byte<2>(exw) : magic_byte<3>(exw);
        o[0] = (int32_t)pack_bf16x2(dec(r.v[e][0], M), dec(r.v[e][1], M));
        o[1] = (int32_t)pack_bf16x2(dec(r.v[e][2], M), dec(r.v[e][3], M));
      } else {
        o = r.v[e];
      }
      *reinterpret_cast<i32x2*>(tile + row * ROWB + ((cw ^ trf(row)) * 32) + cb) = o;
    }
  }
};

// MFMAs of one stage: A from a swizzled DMA tile (ds_read_b128), B from a
// row-major tile by transpose reads.
template <int NI, int NJ, int ROWB>
CONCORD_DEV void stage_mfma_swz_tr(f32x4 (&acc)[NI][NJ], const uint16_t* la, const lds_char* lb, int ra,
                                   int rb, int lane) {
  const int lrow = lane & 15;
  const int sw = (lane & 14) >> 1;
  const int p = lane & 15, gq = lane >> 4;
  const uint32_t fsw = (uint32_t)(((p >> 2) | ((gq & 1) << 2)) * 32);
  const uint32_t lbase = (uint32_t)((8 * gq + (p >> 2)) * ROWB + 8 * (p & 3));
#pragma unroll
  for (int kk = 0; kk < TR / 32; ++kk) {
    const int aoff = lrow * 64 + (((kk * 4 + (lane >> 4)) ^ sw) * 8);
    bf16x8 fa[NI], fb[NJ];
#pragma unroll
    for (int x = 0; x < NI; ++x)
      fa[x] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const i32x4*>(la + (ra + x * 16) * 64 + aoff));
    tr_frags<NJ, ROWB>(fb, lb, lbase, fsw, rb / 16, kk);
    mfma_block<NI, NJ>(acc, fa, fb);
  }
}

// 8 waves: waves 0-3 compute and move A (dy) by DMA, waves 4-7 load W rows
// two stages ahead, decode them and write the row-major B tile.
// CONV (MODE_DGRAD_BF16): the conv dgrad, dy gathered by RowsDmaConv and the
// weight rows (n, tap) by TrRowsB's conv stage offsets.
// CARRY (MODE_DGRAD only): workgroups from dg_blocks on run the split-K
// reduction with v-hat partials (splitk_reduce_vh_kernel's blocks, two per
// workgroup) of the WGRAD launch `rw` issued just before on the stream, on
// the CUs the dgrad grid leaves idle.
// LDS of gemm_dgt_body: three A stage tiles of BI x 64 bf16 (dgt_a_bytes)
// and two B stage tiles of the weight loader (dgt_b_bytes each), each set
// 1024-aligned
template <int BI>
constexpr int dgt_a_bytes() { return 3 * BI * 64 * 2; }
template <int MODE, int BJ, int CONV>
constexpr int dgt_b_bytes() { return TrRowsB<BJ, 256, MODE == MODE_DGRAD, (CONV != 0)>::LBYTES; }

template <int MODE, int BI, int BJ, int CONV, bool CARRY>
CONCORD_DEV void gemm_dgt_body(const GemmArgs& g, const GemmArgs& rw, int dg_blocks, int wg, int ngrid,
                               uint16_t* lds_a_mem, char* lds_b_mem) {
  constexpr int NP = 256;
  constexpr int WTI = BI / 2, WTJ = BJ / 2;
  constexpr int NI = WTI / 16, NJ = WTJ / 16;
  typedef TrRowsB<BJ, NP, MODE == MODE_DGRAD, (CONV != 0)> BL;
  typedef typename std::conditional<CONV != 0, RowsDmaConv<BI, 4, true, CONV == 1>, RowsDma<BI, 4>>::type AD;
  typedef uint16_t LdsA[3][BI * 64];
  typedef char LdsB[2][BL::LBYTES];
  LdsA& lds_a = *reinterpret_cast<LdsA*>(lds_a_mem);
  LdsB& lds_b = *reinterpret_cast<LdsB*>(lds_b_mem);
  if constexpr (CARRY) {
    typedef ReduceVh<256, 128, 4, 2> RV;
    static_assert(sizeof(lds_a) >= 2 * RV::LDS_FLOATS * sizeof(float), "two reduction blocks fit");
    if (wg >= dg_blocks) {
      const int nblk = rw.tiles_i * rw.tiles_j * RV::NAW;
      const int half = threadIdx.x >> 8, tid = threadIdx.x & 255;
      float* s_g2 = reinterpret_cast<float*>(&lds_a[0][0]) + half * RV::LDS_FLOATS;
      const int stride = 2 * (ngrid - dg_blocks);
      for (int b0 = 2 * (wg - dg_blocks); b0 < nblk; b0 += stride) {
        const int blk = b0 + half;
        if (blk < nblk) RV::part1(rw, blk, tid, s_g2);
        __syncthreads();
        if (blk < nblk) RV::part2(rw, blk, tid, s_g2);
        __syncthreads();   // s_g2 is reused by the next pair
      }
      return;
    }
  }

  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const bool producer = wave >= 4;
  int split, bi, bj, slot;
  gemm_tile_of<BI, BJ>(g, wg, split, bi, bj, slot);
  const int64_t i0 = (int64_t)bi * BI, j0 = (int64_t)bj * BJ;
  const int64_t r_begin = (int64_t)split * g.r_split;
  const int64_t r_end = min(g.R, r_begin + g.r_split);
  const int nst = r_end > r_begin ? (int)((r_end - r_begin + TR - 1) / TR) : 0;
  const int nst2 = (nst + 1) & ~1;

  f32x4 acc[NI][NJ];
#pragma unroll
  for (int x = 0; x < NI; ++x)
#pragma unroll
    for (int y = 0; y < NJ; ++y) acc[x][y] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int wi = (wave & 3) >> 1, wj = wave & 1;

  if (producer) {
    const int tp = t - NP;
    BL bl;
    const int esz = MODE == MODE_DGRAD ? 4 : 2;
    if constexpr (CONV) bl.init_conv(g, reinterpret_cast<const uint16_t*>(g.b) + j0, j0, tp);
    else bl.init(reinterpret_cast<const char*>(g.b) + j0 * esz, g.ldb, g.J - j0, g.R, g.row_exp, tp);
    typename BL::Raw r0, r1;
    auto stage_r = [&](int st) { return r_begin + (int64_t)st * TR; };
    bl.load(r0, stage_r(0), r_end - stage_r(0));
    bl.load(r1, stage_r(1), r_end - stage_r(1));
    bl.store(r0, lds_b[0]);
    bl.load(r0, stage_r(2), r_end - stage_r(2));
    lds_barrier();
    for (int s = 0; s < nst2; s += 2) {
      bl.store(r1, lds_b[1]);
      bl.load(r1, stage_r(s + 3), r_end - stage_r(s + 3));
      lds_barrier();
      bl.store(r0, lds_b[0]);
      bl.load(r0, stage_r(s + 4), r_end - stage_r(s + 4));
      lds_barrier();
    }
  } else {
    AD ad;
    if constexpr (CONV) ad.init(g, i0, wave, lane);
    else ad.init(g.a + i0 * g.lda, g.lda, g.I - i0, g.R, wave, lane);
    ad.load(lds_a[0], r_begin, r_end - r_begin);
    ad.load(lds_a[1], r_begin + TR, r_end - r_begin - TR);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(AD::PER));
    lds_barrier();
    // stage s reads A slot s % 3 and B slot s % 2; unrolled by their period
    // of six, so that every slot address is a constant (the transpose reads
    // and the DMA's LDS base then need no per-stage address arithmetic);
    // nst2 is even, so two or four stages remain after the unrolled loop
    auto cstage = [&](int s, auto ph) {
      constexpr int P = decltype(ph)::value;
      const int64_t r2 = r_begin + (int64_t)(s + 2) * TR;
      ad.load(lds_a[(P + 2) % 3], r2, r_end - r2);
      if (s < nst)
        stage_mfma_swz_tr<NI, NJ, BL::ROWB>(acc, lds_a[P % 3], (const lds_char*)lds_b[P & 1], wi * WTI,
                                             wj * WTJ, lane);
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(AD::PER));
      lds_barrier();
    };
    int s = 0;
    for (; s + 6 <= nst2; s += 6) {
      cstage(s, std::integral_constant<int, 0>());
      cstage(s + 1, std::integral_constant<int, 1>());
      cstage(s + 2, std::integral_constant<int, 2>());
      cstage(s + 3, std::integral_constant<int, 3>());
      cstage(s + 4, std::integral_constant<int, 4>());
      cstage(s + 5, std::integral_constant<int, 5>());
    }
    if (s < nst2) {
      cstage(s, std::integral_constant<int, 0>());
      cstage(s + 1, std::integral_constant<int, 1>());
    }
    if (s + 2 < nst2) {
      cstage(s + 2, std::integral_constant<int, 2>());
      cstage(s + 3, std::integral_constant<int, 3>());
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  }

  static_assert(sizeof(lds_a) >= (size_t)BI * (BJ + 8) * 2, "output staging fits in the A tiles");
  epilogue<MODE, NI, NJ, BI, BJ, 4>(g, acc, i0, j0, wi * WTI, wj * WTJ, split, slot, producer ? -1 : wave,
                                     t, 512, &lds_a[0][0]);
}

template <int MODE, int BI, int BJ, int CONV = 0>
__global__ __launch_bounds__(512, 1) void gemm_dgt_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(1024))) uint16_t lds_a[dgt_a_bytes<BI>() / 2];
  __shared__ __attribute__((aligned(1024))) char lds_b[2 * dgt_b_bytes<MODE, BJ, CONV>()];
  gemm_dgt_body<MODE, BI, BJ, CONV, false>(g, g, 0, blockIdx.x, gridDim.x, lds_a, lds_b);
}

// the dgrad launch carrying the split WGRAD's v-hat reduction (rw): workgroups
// [0, dg_blocks) compute dgrad tiles, the rest run reduction blocks
template <int BI, int BJ>
__global__ __launch_bounds__(512, 1) void gemm_dgt_carry_kernel(GemmArgs g, GemmArgs rw, int dg_blocks) {
  __shared__ __attribute__((aligned(1024))) uint16_t lds_a[dgt_a_bytes<BI>() / 2];
  __shared__ __attribute__((aligned(1024))) char lds_b[2 * dgt_b_bytes<MODE_DGRAD, BJ, 0>()];
  gemm_dgt_body<MODE_DGRAD, BI, BJ, 0, true>(g, rw, dg_blocks, blockIdx.x, gridDim.x, lds_a, lds_b);
}

// The dgrad and the WGRAD with its v-hat partials in one launch, for batches
// whose two grids together fit the chip at once (a few hundred tokens: each
// product alone leaves most CUs idle, and each takes about the same fixed
// latency of prologue, a few stages and epilogue, so in one launch they
// overlap).  Workgroups [0, dg_blocks) run dgrad tiles (split-K partials when
// the plan splits), the rest WGRAD tiles; both bodies compute what their own
// launches would.  One LDS array holds either body's tiles.
template <int DBI>
__global__ __launch_bounds__(512, 1) void gemm_dgt_tr_kernel(GemmArgs gd, GemmArgs gw, int dg_blocks) {
  constexpr int A = dgt_a_bytes<DBI>(), B = 2 * dgt_b_bytes<MODE_DGRAD, 128, 0>();
  constexpr int T = tr_ring_bytes<256, 128>();
  static_assert(A % 1024 == 0, "the dgrad's B tiles stay 1024-aligned");
  constexpr int BYTES = A + B > T + 16 ? A + B : T + 16;
  __shared__ __attribute__((aligned(1024))) char lds[BYTES];
  const int wg = blockIdx.x;
  if (wg < dg_blocks) {
    gemm_dgt_body<MODE_DGRAD, DBI, 128, 0, false>(gd, gd, 0, wg, dg_blocks, reinterpret_cast<uint16_t*>(lds),
                                                  lds + A);
  } else {
    const int tw = (int)gridDim.x - dg_blocks;   // every remaining workgroup has a tile: no carried blocks
    gemm_tr_body<256, 128, 4, 2, true, false, 256, 0>(gw, gw, tw, WgradUpd{}, (uint32_t)(wg - dg_blocks),
                                                      (uint32_t)tw, reinterpret_cast<uint16_t*>(lds),
                                                      reinterpret_cast<int*>(lds + T));
  }
}

// vhat_finalize_kernel's blocks [0, fin_blocks) and, on the rest, the split-K
// reduction of the dgrad (rd, RBI x 128 tiles) that gemm_dgt_tr_kernel left
// (one item per thread, as splitk_reduce_kernel)
template <int RBI>
__global__ __launch_bounds__(256) void vhat_finalize_carry_kernel(
    const float* __restrict__ pr, const float* __restrict__ pc, int64_t N, int64_t K, float b2, float omb2,
    float* v_row, float* v_col, int32_t* row_max, int32_t* col_max, float* bsum, const float* __restrict__ bpart,
    int64_t nbp, uint16_t* grad_bias, uint32_t* ticket, float* sum_v_inv, int32_t* salt, GemmArgs rd,
    int fin_blocks) {
  if ((int)blockIdx.x < fin_blocks) {
    vhat_finalize_block(blockIdx.x, pr, pc, N, K, b2, omb2, v_row, v_col, row_max, col_max, bsum, bpart, nbp,
                        grad_bias, ticket, sum_v_inv, salt);
    return;
  }
  const int64_t idx = (int64_t)(blockIdx.x - fin_blocks) * 256 + threadIdx.x;
  if (idx < splitk_reduce_items<CONCORD_DGRAD_REDUCE>(rd)) splitk_reduce_item<CONCORD_DGRAD_REDUCE>(rd, idx);
}

// ---- planning -----------------------------------------------------------------
// weight: measured time per FLOP relative to the 8-wave kernels; the 4-wave
// 128 x 128 kernel ran at ~255 TFLOP/s against ~650 for the transpose-read
// WGRAD on the same conv-shaped product (640 x 5760, reduction 8192); the
// 192-row tiles (more of them where 256-row tiles leave CUs idle) cost ~5%
// more per FLOP than 256 rows (the 2048 x 1280 dgrad, reduction 5120: 220
// tiles of 192 x 128 at 0.76 ps per unit against 240 of 256 x 128 at 0.72)
struct FastShape { int bi, bj, waves, minb; double weight; };

// tile shapes per mode (index into the launch switch below); 8-wave tiles run
// two waves per SIMD, 4-wave 128 x 128 tiles two blocks per CU
constexpr FastShape kFwdShapes[] = {{256, 160, 8, 1, 1.0}, {256, 128, 8, 1, 1.0}, {128, 128, 4, 2, 2.0},
                                    {192, 160, 8, 1, 1.05}, {192, 128, 8, 1, 1.05}};
constexpr FastShape kColShapes[] = {{256, 128, 8, 1, 1.0}, {128, 128, 4, 2, 2.0}, {192, 128, 8, 1, 1.05}};
constexpr FastShape kWgrShapes[] = {{256, 128, 8, 1, 1.0}, {128, 128, 4, 2, 2.0}};
// the conv WGRAD (I = out channels, J = taps x in channels): 128-row tiles
// leave no empty rows for 320 and 640 channels where 256-row tiles pad I by
// 20-60% and run a second round of blocks
constexpr FastShape kConvWgrShapes[] = {{256, 128, 8, 1, 1.0}, {128, 256, 8, 1, 1.0}};
constexpr int kCUs = 256;

struct FastPlan { int shape, splits, ti, tj; int64_t r_split; };

// room = bytes available for split-K partials (each split of each tile
// takes a full BI x BJ fp32 slot)
// sym: a symmetric product (I == J) computing only the tiles that meet the
// upper triangle (sym_tile_count of them; gemm_tile_of)
template <int NS>
static FastPlan plan(const FastShape (&shapes)[NS], int64_t I, int64_t J, int64_t R, size_t room,
                     bool sym = false, double sym_part_cost = 2.2) {
  FastPlan best{0, 1, 0, 0, R};
  double best_cost = 1e300;
  for (int s = 0; s < NS; ++s) {
    const int64_t ti = cdiv(I, shapes[s].bi), tj = cdiv(J, shapes[s].bj);
    const int64_t tiles = sym ? sym_tile_count((int)ti, (int)tj, shapes[s].bi, shapes[s].bj) : ti * tj;
    const size_t slot = (size_t)tiles * shapes[s].bi * shapes[s].bj * sizeof(float);
    const int max_splits = (int)std::min<size_t>(kMaxSplits, std::max<size_t>(1, room / slot));
    for (int sp = 1; sp <= max_splits; ++sp) {
      // split only a grid that leaves CUs idle (then up to kMaxSplits, the
      // cost below deciding); a grid that fills the chip stays unsplit
      if (sp > 1 && (!gemm_splitk_fits(tiles) || tiles >= kCUs * shapes[s].minb)) break;
      const int64_t rs = cdiv(cdiv(R, sp), TR) * TR;
      if (sp > 1 && (sp - 1) * rs >= R) break;
      const double slots = (double)kCUs * shapes[s].minb;
      const double waves = std::ceil((double)(tiles * sp) / slots);
      // a resident block's MFMA rate falls when two share a CU
      const double per_block = (double)shapes[s].bi * shapes[s].bj * (double)(rs + 2 * TR) * shapes[s].minb;
      double cost = waves * per_block * shapes[s].weight;
      // split-K partials: each split writes I x J fp32 (the computed tiles'
      // share of it when symmetric) and the reduction reads them back, 8 B
      // per element and split at ~5 TB/s, in the units of per_block (~0.73 ps
      // per unit for an 8-wave tile at full occupancy)
      if (sp > 1)
        cost += sym ? (double)sp * tiles * shapes[s].bi * shapes[s].bj * sym_part_cost : (double)sp * I * J * 2.2;
      if (cost < best_cost * 0.999) {
        best_cost = cost;
        best = FastPlan{s, sp, (int)ti, (int)tj, rs};
      }
    }
  }
  return best;
}

static bool al(const void* p, int n) { return ((uintptr_t)p % n) == 0; }
// operand extents stay below 2^30 bytes, so kOOB plus any in-tile offset plus
// the stage's soffset never wraps 32 bits
static bool fits31(int64_t bytes) { return bytes < ((int64_t)1 << 30); }

// alignment and extent rules of the fast kernels, per mode
static bool eligible(int mode, const GemmArgs& g) {
  if (!(g.ldc % 4 == 0 && g.J % 4 == 0 && al(g.c, 8))) return false;
  // the combine operand is read at the output's positions, 16 bytes at a time
  if (g.ay && !(g.ldy % 8 == 0 && g.ldc % 8 == 0 && g.J % 8 == 0 && al(g.ay, 16) && al(g.c, 16))) return false;
  if (g.vbias && !al(g.vbias, 8)) return false;
  switch (mode) {
    case MODE_FWD:
      return g.lda % 8 == 0 && g.R % 8 == 0 && al(g.a, 16) && g.ldb % 4 == 0 && al(g.b, 16) &&
             al(g.col_exp, 4) && al(g.row_exp, 4) && fits31(((g.I - 1) * g.lda + g.R) * 2) &&
             fits31(((g.J - 1) * g.ldb + g.R) * 4);
    case MODE_FWD_BF16:
      return g.lda % 8 == 0 && g.R % 8 == 0 && al(g.a, 16) && g.ldb % 8 == 0 && al(g.b, 16) &&
             fits31(((g.I - 1) * g.lda + g.R) * 2) && fits31(((g.J - 1) * g.ldb + g.R) * 2);
    case MODE_DGRAD:
      return g.lda % 8 == 0 && g.R % 8 == 0 && al(g.a, 16) && g.ldb % 4 == 0 && al(g.b, 16) &&
             al(g.row_exp, 4) && al(g.col_exp, 4) && fits31(((g.I - 1) * g.lda + g.R) * 2) &&
             fits31(((g.R - 1) * g.ldb + g.J) * 4);
    case MODE_DGRAD_BF16:
      return g.lda % 8 == 0 && g.R % 8 == 0 && al(g.a, 16) && g.ldb % 4 == 0 && al(g.b, 8) &&
             fits31(((g.I - 1) * g.lda + g.R) * 2) && fits31(((g.R - 1) * g.ldb + g.J) * 2);
    case MODE_WGRAD:
      return g.lda % 4 == 0 && g.I % 4 == 0 && al(g.a, 8) && g.ldb % 4 == 0 && al(g.b, 8) &&
             fits31(((g.R - 1) * g.lda + g.I) * 2) && fits31(((g.R - 1) * g.ldb + g.J) * 2);
  }
  return false;
}

// the transpose-read WGRAD kernel moves 16-byte chunks of both operands
static bool tr_eligible(const GemmArgs& g) {
  return g.lda % 8 == 0 && g.I % 8 == 0 && al(g.a, 16) && g.ldb % 8 == 0 && g.J % 8 == 0 && al(g.b, 16);
}

// split-K: sum the partials once every split has stored them
template <int MODE, int BI, int BJ, int WI, int WJ>
static void launch_reduce(const GemmArgs& g, hipStream_t st) {
  if (g.splits <= 1) return;
  constexpr int NI = BI / WI / 16, NJ = BJ / WJ / 16;
  int64_t threads = (g.sym ? (int64_t)g.sym : (int64_t)g.tiles_i * g.tiles_j) * WI * WJ * NI * NJ * 64;
  if (MODE == MODE_WGRAD && g.bpart) threads += (int64_t)g.tiles_j * g.I;   // the bias fold
  hipLaunchKernelGGL((splitk_reduce_kernel<MODE, NI, NJ, BI, BJ, WI, WJ>), dim3((unsigned)cdiv(threads, 256)),
                     dim3(256), 0, st, g);
}

template <int MODE, int BI, int BJ>
static void launch_dgt(const GemmArgs& g, int blocks, hipStream_t st) {
  hipLaunchKernelGGL((gemm_dgt_kernel<MODE, BI, BJ>), dim3(blocks), dim3(512), 0, st, g);
  launch_reduce<MODE, BI, BJ, 2, 2>(g, st);
}

template <int MODE, int BI, int BJ>
static void launch_dma(const GemmArgs& g, int blocks, hipStream_t st) {
  hipLaunchKernelGGL((gemm_dma_kernel<MODE, BI, BJ>), dim3(blocks), dim3(512), 0, st, g);
  launch_reduce<MODE, BI, BJ, 2, 2>(g, st);
}

template <int BI, int BJ, int WI, int WJ>
static void launch_tr(const GemmArgs& g, int blocks, hipStream_t st) {
  hipLaunchKernelGGL((gemm_tr_kernel<BI, BJ, WI, WJ, false>), dim3(blocks), dim3(64 * WI * WJ), 0, st, g,
                     GemmArgs{}, blocks);
  launch_reduce<MODE_WGRAD, BI, BJ, WI, WJ>(g, st);
}

template <int MODE, int BI, int BJ>
static void launch_ws(const GemmArgs& g, int blocks, hipStream_t st) {
  hipLaunchKernelGGL((gemm_ws_kernel<MODE, BI, BJ>), dim3(blocks), dim3(512), 0, st, g);
  launch_reduce<MODE, BI, BJ, 2, 2>(g, st);
}

template <int MODE, int BI, int BJ, int WI, int WJ, int MINB, bool DB = true, bool SCHED = true>
static void launch(const GemmArgs& g, int blocks, hipStream_t st) {
  hipLaunchKernelGGL((gemm_fast_kernel<MODE, BI, BJ, WI, WJ, MINB, DB, SCHED>), dim3(blocks),
                     dim3(64 * WI * WJ), 0, st, g);
  launch_reduce<MODE, BI, BJ, WI, WJ>(g, st);
}

// The grouped tile order's group size for a launch whose workgroups are all
// resident at once (at most one per CU): XCD x runs the workgroups w = x mod 8,
// and its L2 holds the operand bands those tiles read.  For each candidate
// group size, count per XCD the distinct (split, i-tile) and (split, j-tile)
// bands its share of split_tile_of's order touches, weighted by one band's
// bytes per reduction step (wa = BI x A's element size, wb = BJ x B's), and
// keep the least; ties keep 8.  One evaluation costs ~15 us of host time, so
// results are cached per grid (512 entries per thread: a network's distinct
// launch grids, config 4's ~60 among them, stay resident in eager loops).
static int choose_gi(int ti, int tj, int splits, int wa, int wb) {
  const int tiles = ti * tj, total = tiles * splits;
  if (total > kCUs || total < 16 || ti < 2) return 8;
  struct Entry { uint64_t key; int gi; };
  constexpr int kSlots = 512;
  thread_local Entry cache[kSlots] = {};
  const uint64_t key = ((uint64_t)ti << 48) ^ ((uint64_t)tj << 36) ^ ((uint64_t)splits << 28) ^
                       ((uint64_t)(uint32_t)wa << 14) ^ (uint64_t)(uint32_t)wb ^ 1ull;
  Entry& e = cache[(key ^ (key >> 17) ^ (key >> 33) ^ (key >> 47)) & (kSlots - 1)];
  if (e.key == key) return e.gi;
  auto cost = [&](int gi) {
    int64_t c = 0;
    for (int x = 0; x < 8; ++x) {
      unsigned char seen_a[kCUs] = {}, seen_b[kCUs] = {};
      int na = 0, nb = 0;
      for (int w = x; w < total; w += 8) {
        int split, bi, bj;
        split_tile_of(w, ti, tj, splits, split, bi, bj, gi);
        const int ia = split * ti + bi, ib = split * tj + bj;   // < total <= kCUs
        if (!seen_a[ia]) { seen_a[ia] = 1; ++na; }
        if (!seen_b[ib]) { seen_b[ib] = 1; ++nb; }
      }
      c += (int64_t)na * wa + (int64_t)nb * wb;
    }
    return c;
  };
  int best = 8;
  int64_t best_cost = cost(8);
  for (int gi = 1; gi <= (ti < 16 ? ti : 16); ++gi) {
    const int64_t c = cost(gi);
    if (c < best_cost) {
      best_cost = c;
      best = gi;
    }
  }
  e.key = key;
  e.gi = best;
  return best;
}

// element bytes of the A and B operands' bands per mode (the packed weight
// moves 4-byte words)
static int band_bytes_a(int) { return 2; }
static int band_bytes_b(int mode) { return (mode == MODE_FWD || mode == MODE_DGRAD) ? 4 : 2; }
static int plan_gi(int mode, const FastPlan& p, int BI, int BJ) {
  return choose_gi(p.ti, p.tj, p.splits, BI * band_bytes_a(mode), BJ * band_bytes_b(mode));
}

// sym_part_cost: the split-K partial cost of a symmetric product run by the
// dgrad kernel, measured rather than modelled: NS5's A A (1280 x 1280 x 1280,
// 40 upper-triangle tiles of 192 x 128) ran 382.5 us per drive with 3 splits
// against 389.8 us with the 4 the plain coefficient picks (and 384.4 with 2);
// the forward kernel's X X^T keeps the plain coefficient (6 splits, best of
// 4, 5, 6 and 8 in the same sweep)
static FastPlan plan_mode(int mode, int64_t I, int64_t J, int64_t R, size_t room, bool sym = false) {
  if (mode == MODE_FWD || mode == MODE_FWD_BF16) return plan(kFwdShapes, I, J, R, room, sym);
  if (mode == MODE_WGRAD) return plan(kWgrShapes, I, J, R, room);
  return plan(kColShapes, I, J, R, room, sym, 4.0);
}

static const FastShape& shape_of(int mode, int idx) {
  if (mode == MODE_FWD || mode == MODE_FWD_BF16) return kFwdShapes[idx];
  if (mode == MODE_WGRAD) return kWgrShapes[idx];
  return kColShapes[idx];
}

}  // namespace

size_t gemm_fast_partial_bytes(int mode, int64_t I, int64_t J, int64_t R) {
  if (I <= 0 || J <= 0) return 0;
  const FastPlan p = plan_mode(mode, I, J, R, (size_t)-1 / 2);
  if (p.splits <= 1) return 0;
  const FastShape& sh = shape_of(mode, p.shape);
  return (size_t)p.ti * p.tj * sh.bi * sh.bj * sizeof(float) * p.splits;
}

int64_t gemm_wgrad_vhat_tiles_j(int64_t J) { return cdiv(J, 128); }

int gemm_wgrad_vhat_launch(const GemmArgs& g0, size_t split_room, hipStream_t st, const char* what,
                           int* tiles_j) {
  if (!eligible(MODE_WGRAD, g0) || !tr_eligible(g0)) return -1;
  const size_t room = split_room > kSplitkCounterBytes ? split_room - kSplitkCounterBytes : 0;
  const FastPlan p = plan_mode(MODE_WGRAD, g0.I, g0.J, g0.R, room);
  if (p.shape != 0 || p.splits != 1) return -1;
  *tiles_j = p.tj;
  GemmArgs g = g0;
  g.splits = 1;
  g.r_split = p.r_split;
  g.tiles_i = p.ti;
  g.tiles_j = p.tj;
  g.gi = plan_gi(MODE_WGRAD, p, 256, 128);
  hipLaunchKernelGGL((gemm_tr_kernel<256, 128, 4, 2, true>), dim3(p.ti * p.tj), dim3(512), 0, st, g,
                     GemmArgs{}, p.ti * p.tj);
  return launch_status(what);
}

int gemm_wgrad_vhat_split_launch(const GemmArgs& g0, void* workspace, size_t ws_bytes, hipStream_t st,
                                 const char* what, int* bias_rows) {
  if (!eligible(MODE_WGRAD, g0) || !tr_eligible(g0) || !workspace) return -1;
  const size_t room = ws_bytes > kSplitkCounterBytes ? ws_bytes - kSplitkCounterBytes : 0;
  const FastPlan p = plan_mode(MODE_WGRAD, g0.I, g0.J, g0.R, room);
  if (p.shape != 0 || p.splits < 2) return -1;
  GemmArgs g = g0;
  g.splits = p.splits;
  g.r_split = p.r_split;
  g.tiles_i = p.ti;
  g.tiles_j = p.tj;
  g.gi = plan_gi(MODE_WGRAD, p, 256, 128);
  g.part = (float*)((char*)workspace + kSplitkCounterBytes);
  const int tiles = p.ti * p.tj;
  *bias_rows = p.tj;   // the reduction folds the splits' bias rows
  hipLaunchKernelGGL((gemm_tr_kernel<256, 128, 4, 2, false>), dim3(tiles * p.splits), dim3(512), 0, st, g,
                     GemmArgs{}, tiles * p.splits);
  hipLaunchKernelGGL((splitk_reduce_vh_kernel<256, 128, 4, 2>), dim3((unsigned)(tiles * 8)), dim3(256), 0, st, g);
  return launch_status(what);
}

// A split WGRAD with v-hat partials and an unsplit dgrad: the WGRAD product
// first, then the dgrad launch with extra workgroups that run the WGRAD's
// split-K v-hat reduction (gemm_dgt_carry_kernel) on the CUs its tiles leave
// idle, in place of splitk_reduce_vh_kernel after it.  Same products, plans
// and bits as gemm_wgrad_vhat_split_launch and the dgrad launched alone.
// The unsplit dgrad tile rows (192 or 256, both x 128) for the launch that
// carries the split WGRAD's v-hat reduction (nblk blocks of 256 threads, two
// per spare workgroup at a time).  The launch lasts as long as the longer of
// the dgrad tiles and the carried rounds, so fewer, larger dgrad tiles can
// win where they leave more CUs to the reduction: config 4's 1280 x 1280
// layers at 4096 tokens take 160 tiles of 256 x 128 (96 spare CUs, 3 rounds)
// instead of 220 of 192 x 128 (36 spare CUs, 6 rounds): 115.3 -> 110.0 us
// per layer step.  A round is priced at kCarryRoundUnits in the planner's
// units (~0.69 ps each): the 36-CU carry ran 6 rounds in ~34 us.
constexpr double kCarryRoundUnits = 8.0e6;
static FastPlan carry_dgrad_shape(const FastPlan& pd, int64_t I, int64_t R, int nblk) {
  FastPlan best = pd;
  double best_cost = 1e300;
  for (int s : {0, 2}) {   // kColShapes: 256 x 128, 192 x 128 (8 waves, one block per CU)
    const FastShape& sh = kColShapes[s];
    const int ti = (int)cdiv(I, sh.bi), td = ti * pd.tj;
    const int extra = kCUs - td;
    if (extra < 16) continue;
    const double dgrad = (double)sh.bi * sh.bj * (double)(R + 2 * TR) * sh.weight;
    const double carry = std::ceil((double)nblk / (2.0 * extra)) * kCarryRoundUnits;
    const double cost = std::max(dgrad, carry);
    if (cost < best_cost * 0.999) {
      best_cost = cost;
      best = FastPlan{s, 1, ti, pd.tj, pd.r_split};
    }
  }
  return best;
}

int gemm_wgrad_split_dgrad_launch(const GemmArgs& gd0, const GemmArgs& gw0, void* workspace, size_t ws_bytes,
                                  hipStream_t st, const char* what, int* bias_rows) {
  if (!eligible(MODE_DGRAD, gd0) || !eligible(MODE_WGRAD, gw0) || !tr_eligible(gw0) || !workspace) return -1;
  const size_t room = ws_bytes > kSplitkCounterBytes ? ws_bytes - kSplitkCounterBytes : 0;
  FastPlan pd = plan_mode(MODE_DGRAD, gd0.I, gd0.J, gd0.R, room);
  const FastPlan pw = plan_mode(MODE_WGRAD, gw0.I, gw0.J, gw0.R, room);
  if ((pd.shape != 0 && pd.shape != 2) || pd.splits != 1 || pw.shape != 0 || pw.splits < 2) return -1;
  pd = carry_dgrad_shape(pd, gd0.I, gd0.R, pw.ti * pw.tj * 8);
  const int td = pd.ti * pd.tj;
  const int extra = kCUs - td;
  if (extra < 16) return -1;   // the dgrad grid leaves too few CUs to carry the reduction
  GemmArgs gw = gw0;
  gw.splits = pw.splits;
  gw.r_split = pw.r_split;
  gw.tiles_i = pw.ti;
  gw.tiles_j = pw.tj;
  gw.gi = plan_gi(MODE_WGRAD, pw, 256, 128);
  gw.part = (float*)((char*)workspace + kSplitkCounterBytes);
  GemmArgs gd = gd0;
  gd.splits = 1;
  gd.r_split = pd.r_split;
  gd.tiles_i = pd.ti;
  gd.tiles_j = pd.tj;
  gd.gi = plan_gi(MODE_DGRAD, pd, pd.shape == 0 ? 256 : 192, 128);
  *bias_rows = pw.tj;
  const int tiles = pw.ti * pw.tj;
  hipLaunchKernelGGL((gemm_tr_kernel<256, 128, 4, 2, false>), dim3(tiles * pw.splits), dim3(512), 0, st, gw,
                     GemmArgs{}, tiles * pw.splits);
  if (pd.shape == 0)
    hipLaunchKernelGGL((gemm_dgt_carry_kernel<256, 128>), dim3(td + extra), dim3(512), 0, st, gd, gw, td);
  else
    hipLaunchKernelGGL((gemm_dgt_carry_kernel<192, 128>), dim3(td + extra), dim3(512), 0, st, gd, gw, td);
  return launch_status(what);
}

int gemm_dgrad_wgrad_vhat_launch(const GemmArgs& gd0, void* workspace, size_t ws_bytes, const GemmArgs& gw0,
                                 hipStream_t st, const char* what, int* tiles_j, GemmArgs* pending,
                                 int* pending_rbi) {
  if (pending_rbi) *pending_rbi = 0;
  if (!eligible(MODE_DGRAD, gd0) || !eligible(MODE_WGRAD, gw0) || !tr_eligible(gw0)) return -1;
  const size_t room = (workspace && ws_bytes > kSplitkCounterBytes) ? ws_bytes - kSplitkCounterBytes : 0;
  const FastPlan pd = plan_mode(MODE_DGRAD, gd0.I, gd0.J, gd0.R, room);
  // the WGRAD plan of gemm_wgrad_vhat_launch with the same room, so that both
  // routes take the same product (and so the same bits)
  const FastPlan pw = plan_mode(MODE_WGRAD, gw0.I, gw0.J, gw0.R, room);
  if ((pd.shape != 0 && pd.shape != 2) || pw.shape != 0 || pw.splits != 1) return -1;
  const int tw = pw.ti * pw.tj;
  const int nd = pd.ti * pd.tj * pd.splits;
  // both grids resident at once: one launch of both products, then the
  // dgrad's split-K reduction (gemm_dgt_tr_kernel)
  const bool together = nd + tw <= kCUs;
  if (!together && pd.splits < 2) return -1;
  const int extra = kCUs - tw;
  if (!together && extra < 16) return -1;   // the WGRAD grid leaves too few CUs to carry the reduction
  GemmArgs gd = gd0;
  gd.splits = pd.splits;
  gd.r_split = pd.r_split;
  gd.tiles_i = pd.ti;
  gd.tiles_j = pd.tj;
  gd.gi = plan_gi(MODE_DGRAD, pd, pd.shape == 0 ? 256 : 192, 128);
  gd.part = (float*)((char*)workspace + kSplitkCounterBytes);
  GemmArgs gw = gw0;
  gw.splits = 1;
  gw.r_split = pw.r_split;
  gw.tiles_i = pw.ti;
  gw.tiles_j = pw.tj;
  gw.gi = plan_gi(MODE_WGRAD, pw, 256, 128);
  *tiles_j = pw.tj;
  if (together) {
    if (pd.splits < 2) gd.part = nullptr;
    const bool defer = pending && pending_rbi && pd.splits > 1;
    if (pd.shape == 0) {
      hipLaunchKernelGGL((gemm_dgt_tr_kernel<256>), dim3(nd + tw), dim3(512), 0, st, gd, gw, nd);
      if (!defer) launch_reduce<MODE_DGRAD, 256, 128, 2, 2>(gd, st);
    } else {
      hipLaunchKernelGGL((gemm_dgt_tr_kernel<192>), dim3(nd + tw), dim3(512), 0, st, gd, gw, nd);
      if (!defer) launch_reduce<MODE_DGRAD, 192, 128, 2, 2>(gd, st);
    }
    if (defer) {
      *pending = gd;
      *pending_rbi = pd.shape == 0 ? 256 : 192;
    }
    return launch_status(what);
  }
  if (pd.shape == 0) {
    hipLaunchKernelGGL((gemm_dgt_kernel<MODE_DGRAD, 256, 128>), dim3(pd.ti * pd.tj * pd.splits), dim3(512), 0, st,
                       gd);
    hipLaunchKernelGGL((gemm_tr_kernel<256, 128, 4, 2, true>), dim3(tw + extra), dim3(512), 0, st, gw, gd, tw);
  } else {
    hipLaunchKernelGGL((gemm_dgt_kernel<MODE_DGRAD, 192, 128>), dim3(pd.ti * pd.tj * pd.splits), dim3(512), 0, st,
                       gd);
    hipLaunchKernelGGL((gemm_tr_kernel<256, 128, 4, 2, true, false, 192>), dim3(tw + extra), dim3(512), 0, st, gw,
                       gd, tw);
  }
  return launch_status(what);
}

// gemm_dgrad_wgrad_vhat_launch's products with the finalize and the update
// carried by the WGRAD launch (wgrad_update_kernel).  -1 when the shapes do not
// take that launch, when the grid (one workgroup per CU) would not be resident
// at once, or when it has too few workgroups for the finalize's rows and columns.
template <int RBI, int UPD>
static bool wgrad_update_resident(int grid) {
  constexpr int kMaxDev = 64;
  static int cap[kMaxDev];   // resident workgroups per device, 0 = not yet known
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return false;
  if (cap[dev] == 0) {
    int cus = 0, per = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, (const void*)wgrad_update_kernel<RBI, UPD>, 512, 0) !=
            hipSuccess)
      return false;
    cap[dev] = cus * per > 0 ? cus * per : -1;
  }
  return grid <= cap[dev];
}

int gemm_dgrad_wgrad_update_launch(const GemmArgs& gd0, void* workspace, size_t ws_bytes, const GemmArgs& gw0,
                                   const WgradUpd& u0, int upd, hipStream_t st, const char* what) {
  if (upd != 1 && upd != 2) return -1;
  if (!eligible(MODE_DGRAD, gd0) || !eligible(MODE_WGRAD, gw0) || !tr_eligible(gw0)) return -1;
  const size_t room = (workspace && ws_bytes > kSplitkCounterBytes) ? ws_bytes - kSplitkCounterBytes : 0;
  const FastPlan pd = plan_mode(MODE_DGRAD, gd0.I, gd0.J, gd0.R, room);
  const FastPlan pw = plan_mode(MODE_WGRAD, gw0.I, gw0.J, gw0.R, room);
  if ((pd.shape != 0 && pd.shape != 2) || pd.splits < 2 || pw.shape != 0 || pw.splits != 1) return -1;
  const int tw = pw.ti * pw.tj;
  const int extra = kCUs - tw;
  if (extra < 16) return -1;
  if (cdiv(gw0.I, 256) + cdiv(gw0.J, 512) > tw + extra) return -1;
  const bool r192 = pd.shape == 2;
  const bool resident = r192 ? (upd == 2 ? wgrad_update_resident<192, 2>(tw + extra)
                                         : wgrad_update_resident<192, 1>(tw + extra))
                             : (upd == 2 ? wgrad_update_resident<256, 2>(tw + extra)
                                         : wgrad_update_resident<256, 1>(tw + extra));
  if (!resident) return -1;
  GemmArgs gd = gd0;
  gd.splits = pd.splits;
  gd.r_split = pd.r_split;
  gd.tiles_i = pd.ti;
  gd.tiles_j = pd.tj;
  gd.gi = plan_gi(MODE_DGRAD, pd, pd.shape == 0 ? 256 : 192, 128);
  gd.part = (float*)((char*)workspace + kSplitkCounterBytes);
  GemmArgs gw = gw0;
  gw.splits = 1;
  gw.r_split = pw.r_split;
  gw.tiles_i = pw.ti;
  gw.tiles_j = pw.tj;
  gw.gi = plan_gi(MODE_WGRAD, pw, 256, 128);
  WgradUpd u = u0;
  u.nbp = pw.tj;
  const dim3 grid(tw + extra), block(512);
  if (!r192) {
    hipLaunchKernelGGL((gemm_dgt_kernel<MODE_DGRAD, 256, 128>), dim3(pd.ti * pd.tj * pd.splits), block, 0, st, gd);
    if (upd == 2) hipLaunchKernelGGL((wgrad_update_kernel<256, 2>), grid, block, 0, st, gw, gd, tw, u);
    else hipLaunchKernelGGL((wgrad_update_kernel<256, 1>), grid, block, 0, st, gw, gd, tw, u);
  } else {
    hipLaunchKernelGGL((gemm_dgt_kernel<MODE_DGRAD, 192, 128>), dim3(pd.ti * pd.tj * pd.splits), block, 0, st, gd);
    if (upd == 2) hipLaunchKernelGGL((wgrad_update_kernel<192, 2>), grid, block, 0, st, gw, gd, tw, u);
    else hipLaunchKernelGGL((wgrad_update_kernel<192, 1>), grid, block, 0, st, gw, gd, tw, u);
  }
  return launch_status(what);
}

// the conv products take the 8-wave DMA kernels only (shape 0 of each mode)
static FastPlan plan_conv(int mode, int64_t I, int64_t J, int64_t R, size_t room) {
  if (mode == MODE_WGRAD) return plan(kConvWgrShapes, I, J, R, room);
  const FastShape one[1] = {mode == MODE_FWD_BF16 ? kFwdShapes[0] : kColShapes[0]};
  return plan(one, I, J, R, room);
}
static FastShape conv_shape(int mode, int idx) {
  return mode == MODE_WGRAD ? kConvWgrShapes[idx] : mode == MODE_FWD_BF16 ? kFwdShapes[0] : kColShapes[0];
}

size_t gemm_conv_partial_bytes(int mode, int64_t I, int64_t J, int64_t R) {
  if (I <= 0 || J <= 0) return 0;
  const FastPlan p = plan_conv(mode, I, J, R, (size_t)-1 / 2);
  if (p.splits <= 1) return 0;
  const FastShape sh = conv_shape(mode, p.shape);
  return (size_t)p.ti * p.tj * sh.bi * sh.bj * sizeof(float) * p.splits;
}

int gemm_conv_launch(int mode, const GemmArgs& g0, void* workspace, size_t ws_bytes, hipStream_t st,
                     const char* what, int* bias_rows) {
  // the output is written 8 bytes at a time; the non-gathered operand moves
  // 16-byte chunks
  if (!(g0.ldc % 4 == 0 && g0.J % 4 == 0 && al(g0.c, 8)) || (g0.vbias && !al(g0.vbias, 8))) return -1;
  if (g0.cv.C % 64 != 0 || !al(mode == MODE_WGRAD ? g0.b : g0.a, 16)) return -1;
  if (mode == MODE_FWD_BF16 && !(g0.ldb % 8 == 0 && al(g0.b, 16) && fits31(((g0.J - 1) * g0.ldb + g0.R) * 2)))
    return -1;
  if (mode == MODE_DGRAD_BF16 && !(g0.ldb % 4 == 0 && al(g0.b, 8) && g0.cv.cb % 4 == 0)) return -1;
  if (mode == MODE_WGRAD && !(g0.lda % 8 == 0 && g0.I % 8 == 0 && al(g0.a, 16) && g0.J % 8 == 0 &&
                              fits31(((g0.R - 1) * g0.lda + g0.I) * 2)))
    return -1;
  GemmArgs g = g0;
  const size_t room = (workspace && ws_bytes > kSplitkCounterBytes) ? ws_bytes - kSplitkCounterBytes : 0;
  const FastPlan p = plan_conv(mode, g.I, g.J, g.R, room);
  g.splits = p.splits;
  g.r_split = p.r_split;
  g.tiles_i = p.ti;
  g.tiles_j = p.tj;
  {
    const FastShape sh = conv_shape(mode, p.shape);
    g.gi = plan_gi(mode, p, sh.bi, sh.bj);
  }
  if (p.splits > 1) g.part = (float*)((char*)workspace + kSplitkCounterBytes);
  if (mode != MODE_WGRAD) g.bpart = nullptr;
  if (bias_rows) *bias_rows = g.bpart ? p.tj : 0;   // split launches fold their rows in the reduction
  const int blocks = p.ti * p.tj * p.splits;
  // the gathered operand's taps resolved once per row (FWD, DGRAD: R = taps * C)
  const bool masked = g.R / g.cv.C <= kMaskTaps;
  switch (mode) {
    case MODE_FWD_BF16:
      if (masked)
        hipLaunchKernelGGL((gemm_dma_kernel<MODE_FWD_BF16, 256, 160, 1>), dim3(blocks), dim3(512), 0, st, g);
      else
        hipLaunchKernelGGL((gemm_dma_kernel<MODE_FWD_BF16, 256, 160, 2>), dim3(blocks), dim3(512), 0, st, g);
      launch_reduce<MODE_FWD_BF16, 256, 160, 2, 2>(g, st);
      break;
    case MODE_DGRAD_BF16:
      if (masked)
        hipLaunchKernelGGL((gemm_dgt_kernel<MODE_DGRAD_BF16, 256, 128, 1>), dim3(blocks), dim3(512), 0, st, g);
      else
        hipLaunchKernelGGL((gemm_dgt_kernel<MODE_DGRAD_BF16, 256, 128, 2>), dim3(blocks), dim3(512), 0, st, g);
      launch_reduce<MODE_DGRAD_BF16, 256, 128, 2, 2>(g, st);
      break;
    case MODE_WGRAD:
      if (p.shape == 1) {
        hipLaunchKernelGGL((gemm_tr_kernel<128, 256, 2, 4, false, true>), dim3(blocks), dim3(512), 0, st, g,
                           GemmArgs{}, blocks);
        launch_reduce<MODE_WGRAD, 128, 256, 2, 4>(g, st);
      } else {
        hipLaunchKernelGGL((gemm_tr_kernel<256, 128, 4, 2, false, true>), dim3(blocks), dim3(512), 0, st, g,
                           GemmArgs{}, blocks);
        launch_reduce<MODE_WGRAD, 256, 128, 4, 2>(g, st);
      }
      break;
    default:
      return -1;
  }
  return launch_status(what);
}

// sym: the symmetric tile set (FWD / DGRAD modes; the epilogue or the
// split-K reduction also stores each upper element's mirror image)
static int fast_launch(int mode, const GemmArgs& g0, void* workspace, size_t ws_bytes, hipStream_t st,
                       const char* what, bool sym) {
  if (!eligible(mode, g0)) return -1;
  GemmArgs g = g0;
  // split-K needs room for its partials behind the counters
  const size_t room = (workspace && ws_bytes > kSplitkCounterBytes) ? ws_bytes - kSplitkCounterBytes : 0;
  const FastPlan p = plan_mode(mode, g.I, g.J, g.R, room, sym);
  g.splits = p.splits;
  g.r_split = p.r_split;
  g.tiles_i = p.ti;
  g.tiles_j = p.tj;
  const FastShape& sh = shape_of(mode, p.shape);
  g.sym = sym ? sym_tile_count(p.ti, p.tj, sh.bi, sh.bj) : 0;
  if (!sym) g.gi = plan_gi(mode, p, sh.bi, sh.bj);
  if (p.splits > 1) g.part = (float*)((char*)workspace + kSplitkCounterBytes);
  const int blocks = (sym ? g.sym : p.ti * p.tj) * p.splits;
  switch (mode) {
    case MODE_FWD:
      if (p.shape == 0) launch_dma<MODE_FWD, 256, 160>(g, blocks, st);
      else if (p.shape == 1) launch_dma<MODE_FWD, 256, 128>(g, blocks, st);
      else if (p.shape == 3) launch_dma<MODE_FWD, 192, 160>(g, blocks, st);
      else if (p.shape == 4) launch_dma<MODE_FWD, 192, 128>(g, blocks, st);
      else launch<MODE_FWD, 128, 128, 2, 2, 2>(g, blocks, st);
      break;
    case MODE_FWD_BF16:
      if (p.shape == 0) launch_dma<MODE_FWD_BF16, 256, 160>(g, blocks, st);
      else if (p.shape == 1) launch_dma<MODE_FWD_BF16, 256, 128>(g, blocks, st);
      else if (p.shape == 3) launch_dma<MODE_FWD_BF16, 192, 160>(g, blocks, st);
      else if (p.shape == 4) launch_dma<MODE_FWD_BF16, 192, 128>(g, blocks, st);
      else launch<MODE_FWD_BF16, 128, 128, 2, 2, 2>(g, blocks, st);
      break;
    case MODE_DGRAD:
      if (p.shape == 0) launch_dgt<MODE_DGRAD, 256, 128>(g, blocks, st);
      else if (p.shape == 2) launch_dgt<MODE_DGRAD, 192, 128>(g, blocks, st);
      else launch<MODE_DGRAD, 128, 128, 2, 2, 2>(g, blocks, st);
      break;
    case MODE_DGRAD_BF16:
      if (p.shape == 0) launch_dgt<MODE_DGRAD_BF16, 256, 128>(g, blocks, st);
      else if (p.shape == 2) launch_dgt<MODE_DGRAD_BF16, 192, 128>(g, blocks, st);
      else launch<MODE_DGRAD_BF16, 128, 128, 2, 2, 2>(g, blocks, st);
      break;
    case MODE_WGRAD:
      // 8 waves of 64 x 64 (measured faster than 4 waves of 128 x 64)
      if (p.shape == 0 && tr_eligible(g)) launch_tr<256, 128, 4, 2>(g, blocks, st);
      else if (p.shape == 0) launch_ws<MODE_WGRAD, 256, 128>(g, blocks, st);
      else launch<MODE_WGRAD, 128, 128, 2, 2, 2>(g, blocks, st);
      break;
    default:
      return -1;
  }
  return launch_status(what);
}

int gemm_fast_launch(int mode, const GemmArgs& g0, void* workspace, size_t ws_bytes,
                     hipStream_t st, const char* what) {
  return fast_launch(mode, g0, workspace, ws_bytes, st, what, false);
}


int gemm_bf16_sym(int mode, const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb, uint16_t* c,
                  int64_t ldc, int64_t I, int64_t R, const uint16_t* y, int64_t ldy, float s, float t, void* ws,
                  size_t ws_bytes, hipStream_t st, const char* what) {
  if (mode != MODE_FWD_BF16 && mode != MODE_DGRAD_BF16) return -1;
  if (I == 0) return CONCORD_OK;
  GemmArgs g{};
  g.a = a;
  g.b = b;
  g.lda = lda;
  g.ldb = ldb;
  g.c = c;
  g.ldc = ldc;
  g.I = I;
  g.J = I;
  g.R = R;
  g.ay = y;
  g.ldy = ldy;
  g.as = s;
  g.at = t;
  return fast_launch(mode, g, ws, ws_bytes, st, what, true);
}

size_t gemm_sym_splitk_need(int mode, int64_t I, int64_t R) {
  if (I <= 0) return kSplitkCounterBytes;
  const FastPlan p = plan_mode(mode, I, I, R, (size_t)-1 / 2, true);
  size_t part = 0;
  if (p.splits > 1) {
    const FastShape& sh = shape_of(mode, p.shape);
    part = (size_t)sym_tile_count(p.ti, p.tj, sh.bi, sh.bj) * sh.bi * sh.bj * sizeof(float) * p.splits;
  }
  return kSplitkCounterBytes + ((part + 255) / 256) * 256;
}

void vhat_finish_carry_launch(const float* pr, const float* pc, float* bsum, uint32_t* ticket, int64_t N, int64_t K,
                              double beta2, float* v_row, float* v_col, float* sum_v_inv, int32_t* row_max,
                              int32_t* col_max, int32_t* salt, hipStream_t st, const float* bpart, int64_t nbp,
                              uint16_t* grad_bias, const GemmArgs& rd, int rbi) {
  const float b2 = (float)beta2;
  const float omb2 = (float)(1.0 - beta2);
  const int fin = (int)vhat_finalize_blocks(N, K, grad_bias != nullptr);
  // splitk_reduce_items: tiles x 4 accumulator waves x (RBI / 32) x 4 blocks x 64 lanes
  const int64_t items = (int64_t)rd.tiles_i * rd.tiles_j * 4 * (rbi / 32) * 4 * 64;
  const dim3 grid((unsigned)(fin + cdiv(items, 256)));
  if (rbi == 256)
    hipLaunchKernelGGL(vhat_finalize_carry_kernel<256>, grid, dim3(256), 0, st, pr, pc, N, K, b2, omb2, v_row, v_col,
                       row_max, col_max, bsum, bpart, nbp, grad_bias, ticket, sum_v_inv, salt, rd, fin);
  else
    hipLaunchKernelGGL(vhat_finalize_carry_kernel<192>, grid, dim3(256), 0, st, pr, pc, N, K, b2, omb2, v_row, v_col,
                       row_max, col_max, bsum, bpart, nbp, grad_bias, ticket, sum_v_inv, salt, rd, fin);
}

}  // namespace concord
