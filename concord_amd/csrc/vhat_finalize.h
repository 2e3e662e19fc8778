// vhat_finalize.h -- the v-hat finalize (the row / column EMA of the g^2
// partials, the watermark zeroing, the 256-row totals of v_row, the bias
// gradient) as a block function, run by vhat_finalize_kernel (vhat.hip) and
// by the launch that also carries a dgrad's split-K reduction (gemm_fast.hip).
#pragma once
#include "common.h"

namespace concord {

constexpr int VH_COLS = 64;        // columns per column block of the finalize
constexpr int VH_CHUNK = 128;      // row tiles of column partials staged at a time
constexpr int VH_RSTAGE = 64;      // partial rows staged at a time by a row block

// Sum over j < terms, ascending, of src[j * N + i] for this thread's row
// i = i0 + threadIdx.x of a 256-row block (called by the whole block).  The
// block stages VH_RSTAGE partial rows at a time in LDS, each wave moving
// whole partial rows with 16-byte loads, and every thread then chains its own
// row's values.  Stage loads are unconditional (the partial row and the row
// within the block clamped to the last valid ones; such copies land where no
// chain reads them, or are not stored), so no wait separates them; the next
// stage's loads are in flight while the current stage is summed.
CONCORD_DEV float staged_row_sum(const float* __restrict__ src, int64_t terms, int64_t N, int64_t i0, float* stage) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int nrow = (int)min((int64_t)256, N - i0);
  // 16-byte loads of whole 256-row blocks (uniform over the block)
  const bool full = nrow == 256 && (N % 4) == 0 && ((uintptr_t)src % 16) == 0;
  typedef float f32x4v __attribute__((ext_vector_type(4)));
  f32x4v v[VH_RSTAGE / 4];
  const int r = 4 * lane;   // lane: rows 4 lane .. + 3 of staged partial row q
  auto load_stage = [&](int64_t j0) {
    const int cnt = (int)min((int64_t)VH_RSTAGE, terms - j0);
    auto row_src = [&](int e) { return src + (j0 + min(wave + 4 * e, cnt - 1)) * N + i0; };
    if (full) {
      // 16-byte streaming loads: each partial is read once (a plain load
      // here is folded into the scalar path below by the compiler)
#pragma unroll
      for (int e = 0; e < VH_RSTAGE / 4; ++e)
        v[e] = __builtin_nontemporal_load(reinterpret_cast<const f32x4v*>(row_src(e) + r));
    } else {
      const int last = nrow - 1;
#pragma unroll
      for (int e = 0; e < VH_RSTAGE / 4; ++e) {
        const float* q = row_src(e);
        v[e] = f32x4v{q[min(r, last)], q[min(r + 1, last)], q[min(r + 2, last)], q[min(r + 3, last)]};
      }
    }
  };
  float s = 0.0f;
  if (terms > 0) load_stage(0);
  for (int64_t j0 = 0; j0 < terms; j0 += VH_RSTAGE) {
    const int cnt = (int)min((int64_t)VH_RSTAGE, terms - j0);
    __syncthreads();   // the previous stage is consumed
#pragma unroll
    for (int e = 0; e < VH_RSTAGE / 4; ++e)
      if (wave + 4 * e < cnt) *reinterpret_cast<f32x4v*>(stage + (wave + 4 * e) * 256 + r) = v[e];
    __syncthreads();
    if (j0 + VH_RSTAGE < terms) load_stage(j0 + VH_RSTAGE);
    if (t < nrow) {
#pragma unroll 16
      for (int q = 0; q < cnt; ++q) s = __fadd_rn(s, stage[q * 256 + t]);
    }
  }
  return s;
}

// Row/column EMA and watermark zeroing.  Blocks [0, rb = cdiv(N, 256)) take
// rows: a row's g^2 sum adds its column-tile partials in tile order
// (staged_row_sum), and the block leaves the halving-tree total of its 256
// new v_row values in bsum.  With a bias gradient, blocks [rb, 2 rb) sum the
// bias partial rows likewise, alongside.  The remaining blocks take VH_COLS
// columns each: the four waves load the column partials of interleaved row
// tiles into LDS, one thread per column then sums them in row-tile order.
// The last row block to finish (a device-scope ticket) chains the totals in
// ascending order into 1 / max(sum v_row, 1e-30) and advances the salt.
// sum_v_inv == NULL: the chain is left to the update that follows (it reads
// the totals in bsum); the row blocks only store their totals, and block 0
// advances the salt (no block of this kernel reads it).  The
// totals and the ticket are device-scope atomics (cache-coherent across the
// XCDs), each total stored and complete before its block takes a ticket, so
// the last block reads every total without a device-wide cache write-back.
// One block of the finalize (blk: its index in [0, vhat_finalize_blocks)),
// called by all 256 threads of a block.
CONCORD_DEV void vhat_finalize_block(int64_t blk, const float* __restrict__ pr, const float* __restrict__ pc,
                                     int64_t N, int64_t K, float b2, float omb2, float* v_row, float* v_col,
                                     int32_t* row_max, int32_t* col_max, float* bsum,
                                     const float* __restrict__ bpart, int64_t nbp, uint16_t* grad_bias,
                                     uint32_t* ticket, float* sum_v_inv, int32_t* salt) {
  __shared__ float s_part[256];
  __shared__ union {
    float rows[VH_RSTAGE * 256];      // row and bias blocks: staged partial rows
    float cols[VH_CHUNK * VH_COLS];   // column blocks
  } S;
  float* const s_cols = S.cols;
  __shared__ uint32_t s_ticket;
  const int64_t rb = cdiv(N, 256);
  const int64_t rbb = grad_bias ? rb : 0;   // bias blocks
  const int64_t nc = cdiv(K, 64), nr = cdiv(N, 64);
  if (!sum_v_inv && salt && blk == 0 && threadIdx.x == 0) salt[0] = wadd(salt[0], 1);
  if (blk >= rb && blk < rb + rbb) {
    const int64_t i0 = (blk - rb) * 256, i = i0 + threadIdx.x;
    const float sb = staged_row_sum(bpart, nbp, N, i0, S.rows);
    if (i < N) grad_bias[i] = (uint16_t)(pack_bf16x2(sb, 0.0f) & 0xFFFFu);
    return;
  }
  if (blk < rb) {
    const int lane = threadIdx.x & 63;
    const int64_t i0 = blk * 256, i = i0 + threadIdx.x;
    const float s = staged_row_sum(pr, nc, N, i0, S.rows);
    float vn = 0.0f;
    if (i < N) {
      vn = __fadd_rn(__fmul_rn(v_row[i], b2), __fmul_rn(omb2, s));
      v_row[i] = vn;
      if (row_max) row_max[i] = 0;
    }
    s_part[threadIdx.x] = vn;
    __syncthreads();
    for (int h = 128; h >= 1; h >>= 1) {
      if (threadIdx.x < h) s_part[threadIdx.x] = __fadd_rn(s_part[threadIdx.x], s_part[threadIdx.x + h]);
      __syncthreads();
    }
    if (!sum_v_inv) {   // the update chains the totals
      if (threadIdx.x == 0) bsum[blk] = s_part[0];
      return;
    }
    if (threadIdx.x == 0) {
      __hip_atomic_store(bsum + blk, s_part[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __builtin_amdgcn_s_waitcnt(0);   // the total is stored before the ticket is taken
      s_ticket = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (s_ticket != (uint32_t)(rb - 1) || threadIdx.x >= 64) return;
    // last row block, one wave: totals 64 at a time, chained in order
    float tot = 0.0f;
    for (int64_t c0 = 0; c0 < rb; c0 += 64) {
      const float v = c0 + lane < rb ? __hip_atomic_load(bsum + c0 + lane, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT) : 0.0f;
      const int cnt = (int)min((int64_t)64, rb - c0);
      for (int j = 0; j < cnt; ++j) tot = __fadd_rn(tot, lane_value(v, j));
    }
    if (lane == 0) {
      *sum_v_inv = __fdiv_rn(1.0f, fmaxf(tot, 1e-30f));
      if (salt) salt[0] = wadd(salt[0], 1);
      __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);   // re-armed
    }
  } else {
    const int c = threadIdx.x % VH_COLS, grp = threadIdx.x / VH_COLS;
    const int64_t k = (blk - rb - rbb) * VH_COLS + c;
    float s = 0.0f;
    for (int64_t r0 = 0; r0 < nr; r0 += VH_CHUNK) {
      const int rows = (int)min((int64_t)VH_CHUNK, nr - r0);
      __syncthreads();   // the previous chunk is consumed
      float a[VH_CHUNK / 4];
#pragma unroll
      for (int e = 0; e < VH_CHUNK / 4; ++e) {
        const int r = grp + 4 * e;
        a[e] = r < rows && k < K ? pc[(r0 + r) * K + k] : 0.0f;
      }
#pragma unroll
      for (int e = 0; e < VH_CHUNK / 4; ++e) s_cols[(grp + 4 * e) * VH_COLS + c] = a[e];
      __syncthreads();
      if (grp == 0 && k < K)
        for (int r = 0; r < rows; ++r) s = __fadd_rn(s, s_cols[r * VH_COLS + c]);
    }
    if (grp == 0 && k < K) {
      v_col[k] = __fadd_rn(__fmul_rn(v_col[k], b2), __fmul_rn(omb2, s));
      if (col_max) col_max[k] = 0;
    }
  }
}

// blocks of one finalize: rows, bias rows (with a bias gradient), columns
inline int64_t vhat_finalize_blocks(int64_t N, int64_t K, bool bias) {
  return cdiv(N, 256) * (bias ? 2 : 1) + cdiv(K, VH_COLS);
}

}  // namespace concord
