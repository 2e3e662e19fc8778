// vhat.hip -- AdaFactor rank-1 second moment and bias gradient.
//
// concord_vhat_ema:  FusedConcordLinearPackedB.backward, concord/packed_b.py:1281-1303
//                    (zero row/col watermarks, v_row/v_col EMA of grad^2, 1/sum v_row).
// concord_bias_grad: grad_y_flat.sum(0), concord/packed_b.py:1338-1340.
//
// Reduction order: the tile order of vhat_tile.h (also restated by
// oracle_vhat_ema); g2_row[n] = sum of the row partials over column tiles
// ascending, g2_col[k] likewise over row tiles; sum v_row: halving tree per
// block of 256 rows, then the block totals ascending.
#include "common.h"
#include "vhat.h"
#include "vhat_tile.h"
#include "workspace.h"

namespace concord {

// One wave per 64 x 64 tile of g, loaded in the MFMA accumulator layout of
// vhat_tile.h (lane 16 q + p: rows 16 x + p, columns 16 y + 4 q .. + 3).
__global__ __launch_bounds__(256) void vhat_partials_kernel(const uint16_t* __restrict__ g,
                                                            int64_t ld, int64_t N, int64_t K,
                                                            float* __restrict__ pr,
                                                            float* __restrict__ pc) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t ntc = cdiv(K, 64), nt = cdiv(N, 64) * ntc;
  const int64_t tile = (int64_t)blockIdx.x * 4 + wave;
  if (tile >= nt) return;
  const int64_t row0 = (tile / ntc) * 64, col0 = (tile % ntc) * 64;
  const int p = lane & 15, q = lane >> 4;
  const bool vec = (ld % 4) == 0 && ((uintptr_t)g % 8) == 0;
  float g2[4][4][4];
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    const int64_t n = row0 + 16 * x + p;
#pragma unroll
    for (int y = 0; y < 4; ++y) {
      const int64_t k = col0 + 16 * y + 4 * q;
      float v[4];
      if (n < N && k + 4 <= K && vec) {
        const uint2 w = *reinterpret_cast<const uint2*>(g + n * ld + k);
        v[0] = __uint_as_float(w.x << 16);
        v[1] = __uint_as_float(w.x & 0xFFFF0000u);
        v[2] = __uint_as_float(w.y << 16);
        v[3] = __uint_as_float(w.y & 0xFFFF0000u);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (n < N && k + e < K) ? bf16_to_f32(g[n * ld + k + e]) : 0.0f;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) g2[x][y][e] = __fmul_rn(v[e], v[e]);
    }
  }
  vhat_tile_partials(g2, lane, row0, col0, N, K, pr, pc);
}

// sum of v[0], v[stride], ..., v[(count - 1) stride] ascending from 0.0f,
// with the loads of 32 terms in flight at a time
CONCORD_DEV float ordered_sum(const float* __restrict__ v, int64_t stride, int64_t count) {
  float s = 0.0f;
  int64_t b = 0;
  for (; b + 32 <= count; b += 32) {
    float a[32];
#pragma unroll
    for (int e = 0; e < 32; ++e) a[e] = v[(b + e) * stride];
#pragma unroll
    for (int e = 0; e < 32; ++e) s = __fadd_rn(s, a[e]);
  }
  if (b < count) {
    float a[32];
#pragma unroll
    for (int e = 0; e < 32; ++e) a[e] = b + e < count ? v[(b + e) * stride] : 0.0f;
#pragma unroll
    for (int e = 0; e < 32; ++e)
      if (b + e < count) s = __fadd_rn(s, a[e]);
  }
  return s;
}

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
__global__ __launch_bounds__(256) void vhat_finalize_kernel(
    const float* __restrict__ pr, const float* __restrict__ pc, int64_t N, int64_t K, float b2,
    float omb2, float* v_row, float* v_col, int32_t* row_max, int32_t* col_max, float* bsum,
    const float* __restrict__ bpart, int64_t nbp, uint16_t* grad_bias, uint32_t* ticket,
    float* sum_v_inv, int32_t* salt) {
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
  if (!sum_v_inv && salt && blockIdx.x == 0 && threadIdx.x == 0) salt[0] = wadd(salt[0], 1);
  if ((int64_t)blockIdx.x >= rb && (int64_t)blockIdx.x < rb + rbb) {
    const int64_t i0 = ((int64_t)blockIdx.x - rb) * 256, i = i0 + threadIdx.x;
    const float sb = staged_row_sum(bpart, nbp, N, i0, S.rows);
    if (i < N) grad_bias[i] = (uint16_t)(pack_bf16x2(sb, 0.0f) & 0xFFFFu);
    return;
  }
  if ((int64_t)blockIdx.x < rb) {
    const int lane = threadIdx.x & 63;
    const int64_t i0 = (int64_t)blockIdx.x * 256, i = i0 + threadIdx.x;
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
      if (threadIdx.x == 0) bsum[blockIdx.x] = s_part[0];
      return;
    }
    if (threadIdx.x == 0) {
      __hip_atomic_store(bsum + blockIdx.x, s_part[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
    const int64_t k = ((int64_t)blockIdx.x - rb - rbb) * VH_COLS + c;
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

void vhat_partials_launch(const uint16_t* grad, int64_t ld, int64_t N, int64_t K, float* pr, float* pc,
                          hipStream_t st) {
  const int64_t nt = cdiv(N, 64) * cdiv(K, 64);
  hipLaunchKernelGGL(vhat_partials_kernel, dim3((unsigned)cdiv(nt, 4)), dim3(256), 0, st, grad, ld, N, K,
                     pr, pc);
}

void vhat_finish_launch(const float* pr, const float* pc, float* bsum, uint32_t* ticket, int64_t N, int64_t K,
                        double beta2, float* v_row, float* v_col, float* sum_v_inv, int32_t* row_max,
                        int32_t* col_max, int32_t* salt, hipStream_t st, const float* bpart, int64_t nbp,
                        uint16_t* grad_bias) {
  const float b2 = (float)beta2;
  const float omb2 = (float)(1.0 - beta2);
  const int64_t rb = cdiv(N, 256), rbb = grad_bias ? rb : 0;
  hipLaunchKernelGGL(vhat_finalize_kernel, dim3((unsigned)(rb + rbb + cdiv(K, VH_COLS))), dim3(256), 0, st, pr, pc,
                     N, K, b2, omb2, v_row, v_col, row_max, col_max, bsum, bpart, nbp, grad_bias, ticket,
                     sum_v_inv, salt);
}

// bias gradient: a thread sums 4 adjacent columns over a slab of 64 rows
// (rows ascending; 8-byte loads, a wave reads 512 contiguous bytes per row),
// then the slabs are combined in order.
constexpr int BG_ROWS = 64;

__global__ __launch_bounds__(256) void colsum_partials_kernel(const uint16_t* __restrict__ dy,
                                                              int64_t ld, int64_t M, int64_t N,
                                                              float* __restrict__ part) {
  const int64_t n = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (n >= N) return;
  const bool vec = (n + 4 <= N) && (ld % 4 == 0) && (((uintptr_t)dy % 8) == 0);
  // slabs blockIdx.y, blockIdx.y + gridDim.y, ... (grid.y <= kMaxGridY)
  for (int64_t slab = blockIdx.y; slab * BG_ROWS < M; slab += gridDim.y) {
  const int64_t m0 = slab * BG_ROWS;
  const int64_t m1 = min(M, m0 + BG_ROWS);
  float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (vec) {
    int64_t m = m0;
    for (; m + 8 <= m1; m += 8) {
      uint2 w[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) w[e] = *reinterpret_cast<const uint2*>(dy + (m + e) * ld + n);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        s[0] = __fadd_rn(s[0], __uint_as_float(w[e].x << 16));
        s[1] = __fadd_rn(s[1], __uint_as_float(w[e].x & 0xFFFF0000u));
        s[2] = __fadd_rn(s[2], __uint_as_float(w[e].y << 16));
        s[3] = __fadd_rn(s[3], __uint_as_float(w[e].y & 0xFFFF0000u));
      }
    }
    for (; m < m1; ++m) {
      const uint2 w = *reinterpret_cast<const uint2*>(dy + m * ld + n);
      s[0] = __fadd_rn(s[0], __uint_as_float(w.x << 16));
      s[1] = __fadd_rn(s[1], __uint_as_float(w.x & 0xFFFF0000u));
      s[2] = __fadd_rn(s[2], __uint_as_float(w.y << 16));
      s[3] = __fadd_rn(s[3], __uint_as_float(w.y & 0xFFFF0000u));
    }
  } else {
    for (int64_t m = m0; m < m1; ++m)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (n + c < N) s[c] = __fadd_rn(s[c], bf16_to_f32(dy[m * ld + n + c]));
  }
#pragma unroll
  for (int c = 0; c < 4; ++c)
    if (n + c < N) part[slab * N + n + c] = s[c];
  }
}

__global__ __launch_bounds__(256) void colsum_finalize_kernel(const float* __restrict__ part,
                                                              int64_t slabs, int64_t N,
                                                              uint16_t* out) {
  const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (n >= N) return;
  const float s = ordered_sum(part + n, N, slabs);
  out[n] = (uint16_t)(pack_bf16x2(s, 0.0f) & 0xFFFFu);
}

void bias_grad_launch(const uint16_t* dy, int64_t ld, int64_t M, int64_t N, uint16_t* grad_bias, float* part,
                      hipStream_t st) {
  const int64_t slabs = cdiv(M, BG_ROWS);  // 0 when M == 0: the combine writes zeros
  if (slabs > 0)
    hipLaunchKernelGGL(colsum_partials_kernel, dim3((unsigned)cdiv(N, 1024), grid_y(slabs)), dim3(256), 0,
                       st, dy, ld, M, N, part);
  hipLaunchKernelGGL(colsum_finalize_kernel, dim3((unsigned)cdiv(N, 256)), dim3(256), 0, st, part, slabs, N,
                     grad_bias);
}

__global__ __launch_bounds__(256) void fill_zero_bf16_kernel(uint16_t* p, int64_t ld, int64_t rows, int64_t cols) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= cols) return;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) p[r * ld + c] = 0;
}

void fill_zero_bf16_launch(uint16_t* p, int64_t ld, int64_t rows, int64_t cols, hipStream_t st) {
  if (rows <= 0 || cols <= 0) return;
  hipLaunchKernelGGL(fill_zero_bf16_kernel, dim3((unsigned)cdiv(cols, 256), grid_y(rows)), dim3(256), 0, st, p,
                     ld, rows, cols);
}

void wgrad_vhat_empty_batch(uint16_t* grad_w, int64_t ld_gw, int64_t N, int64_t K, double beta2, float* v_row,
                            float* v_col, float* sum_v_inv, int32_t* row_max, int32_t* col_max,
                            int32_t* salt_counter, uint16_t* grad_bias, void* workspace, hipStream_t st) {
  const Workspace ws = workspace_layout(N, K, 0);
  const VhatScratch v = vhat_scratch(N, K);
  float* pr = (float*)((char*)workspace + ws.scratch);
  float* pc = pr + v.pr;
  float* bsum = pc + v.pc;
  fill_zero_bf16_launch(grad_w, ld_gw, N, K, st);
  vhat_partials_launch(grad_w, ld_gw, N, K, pr, pc, st);
  // no bias partial rows: the finalize writes grad_bias = bf16(0)
  vhat_finish_launch(pr, pc, bsum, (uint32_t*)((char*)workspace + ws.vhat_ticket), N, K, beta2, v_row, v_col,
                     sum_v_inv, row_max, col_max, salt_counter, st, nullptr, 0, grad_bias);
}

}  // namespace concord

using namespace concord;

extern "C" int concord_vhat_ema(const uint16_t* grad, int64_t ld_g, int64_t N, int64_t K,
                                double beta2, float* v_row, float* v_col, float* sum_v_inv,
                                int32_t* row_max, int32_t* col_max, int32_t* salt_counter,
                                void* workspace, size_t workspace_bytes, void* stream) {
  CONCORD_CHECK(N > 0 && K > 0 && N < (1LL << 31) && K < (1LL << 31),
                "concord_vhat_ema: bad size N=%lld K=%lld", (long long)N, (long long)K);
  CONCORD_CHECK(grad && v_row && v_col && sum_v_inv, "concord_vhat_ema: NULL argument");
  CONCORD_CHECK(ld_g >= K, "concord_vhat_ema: leading dimension < K");
  const Workspace ws = workspace_layout(N, K, 0);
  if (!workspace || workspace_bytes < ws.total) {
    set_error("concord_vhat_ema: workspace of %zu bytes needed", ws.total);
    return CONCORD_EWORKSPACE;
  }
  const VhatScratch v = vhat_scratch(N, K);
  float* pr = (float*)((char*)workspace + ws.scratch);
  float* pc = pr + v.pr;
  float* bsum = pc + v.pc;
  hipStream_t st = (hipStream_t)stream;
  vhat_partials_launch(grad, ld_g, N, K, pr, pc, st);
  vhat_finish_launch(pr, pc, bsum, (uint32_t*)((char*)workspace + ws.vhat_ticket), N, K, beta2, v_row, v_col,
                     sum_v_inv, row_max, col_max, salt_counter, st);
  return launch_status("vhat_ema");
}

extern "C" int concord_bias_grad(const uint16_t* dy, int64_t ld_dy, int64_t M, int64_t N,
                                 uint16_t* grad_bias, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  CONCORD_CHECK(M >= 0 && N > 0, "concord_bias_grad: bad size");
  CONCORD_CHECK(dy && grad_bias, "concord_bias_grad: NULL argument");
  CONCORD_CHECK(ld_dy >= N, "concord_bias_grad: leading dimension < N");
  const Workspace ws = workspace_layout(N, 1, M);
  if (!workspace || workspace_bytes < ws.total) {
    set_error("concord_bias_grad: workspace of %zu bytes needed", ws.total);
    return CONCORD_EWORKSPACE;
  }
  bias_grad_launch(dy, ld_dy, M, N, grad_bias, (float*)((char*)workspace + ws.scratch), (hipStream_t)stream);
  return launch_status("bias_grad");
}
