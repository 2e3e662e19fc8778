// rebalance.hip -- exponent ratchet of the packed state.
//
// ConcordLinearPackedB.rebalance (concord/packed_b.py:1792-1814), rebalance_packed
// (1129-1190) and _rebalance_packed_decide_kernel (959-1095), as three kernels:
//   1. (tick-down only) count, per row and column, the words whose
//      max(|s_slow|, |v_slow|) <= 31: the lower median of that magnitude is
//      <= 31 exactly when more than (count - 1) / 2 of them are;
//   2. decide (one block): high-watermarks, seed + 1, per-row/column tick
//      t in {-1, 0, +1} from the PRE-call exponents, new exponents, "fired" flag;
//   3. shift: each tile whose rows and columns all have t = 0 exits without
//      touching the packed words, so a call where nothing fires costs O(N + K).
// The decisions of every tile come from the same pre-call exponents.  (In the
// reference the tiles with pid_k == 0 store the new row exponents while other
// tiles of the same launch may still be loading them.)
#include "common.h"
#include "workspace.h"

namespace concord {

__global__ void fill_i32_kernel(int32_t* p, int64_t n, int32_t v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// counts of words with max(|ss|,|vs|) <= 31; tile 32 rows x 256 columns
__global__ __launch_bounds__(256) void i8_small_count_kernel(const int32_t* __restrict__ packed,
                                                             int64_t ld, int64_t N, int64_t K,
                                                             int32_t* cnt_row, int32_t* cnt_col) {
  __shared__ int32_t s_col[4][256];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t k0 = (int64_t)blockIdx.x * 256 + lane * 4;
  const int64_t nb = (int64_t)blockIdx.y * 32;
  int32_t cc[4] = {0, 0, 0, 0};
  for (int r = wave; r < 32; r += 4) {
    const int64_t n = nb + r;
    if (n >= N) break;
    int32_t rc = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (k0 + j < K) {
        const Fields f = unpack(packed[n * ld + k0 + j]);
        const int32_t small = max(abs(f.ss), abs(f.vs)) <= 31 ? 1 : 0;
        rc += small;
        cc[j] += small;
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) rc += __shfl_xor(rc, o, 64);
    if (lane == 0 && rc) atomicAdd(cnt_row + n, rc);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) s_col[wave][lane * 4 + j] = cc[j];
  __syncthreads();
  const int64_t k = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (k < K) {
    const int32_t v = s_col[0][threadIdx.x] + s_col[1][threadIdx.x] + s_col[2][threadIdx.x] +
                      s_col[3][threadIdx.x];
    if (v) atomicAdd(cnt_col + k, v);
  }
}

__global__ __launch_bounds__(1024) void rebalance_decide_kernel(
    int8_t* row_exp, int8_t* col_exp, const int32_t* row_max, const int32_t* col_max,
    int32_t* row_hwm, int32_t* col_hwm, const int32_t* cnt_row, const int32_t* cnt_col,
    int32_t* seed, int64_t N, int64_t K, int32_t max_m, int32_t exp_max, int32_t exp_min,
    int allow_tickdown, int advance_seed, int32_t* row_t, int32_t* col_t, int32_t* fired) {
  __shared__ int s_any;
  if (threadIdx.x == 0) s_any = 0;
  __syncthreads();
  int any = 0;
  for (int64_t n = threadIdx.x; n < N; n += blockDim.x) {
    const int32_t mx = row_max[n];
    if (row_hwm) row_hwm[n] = max(row_hwm[n], mx);
    const int32_t e = row_exp[n];
    const int up = (mx > max_m) && (e < exp_max);
    // lower median <= 31  <=>  count(<= 31) > (K - 1) / 2
    const int dn = allow_tickdown && (mx <= max_m) && (cnt_row[n] > (K - 1) / 2) && (e > exp_min);
    const int32_t t = up - dn;
    row_t[n] = t;
    row_exp[n] = (int8_t)(e + t);
    any |= t;
  }
  for (int64_t k = threadIdx.x; k < K; k += blockDim.x) {
    const int32_t mx = col_max[k];
    if (col_hwm) col_hwm[k] = max(col_hwm[k], mx);
    const int32_t e = col_exp[k];
    const int up = (mx > max_m) && (e < exp_max);
    const int dn = allow_tickdown && (mx <= max_m) && (cnt_col[k] > (N - 1) / 2) && (e > exp_min);
    const int32_t t = up - dn;
    col_t[k] = t;
    col_exp[k] = (int8_t)(e + t);
    any |= t;
  }
  if (any) s_any = 1;
  __syncthreads();
  if (threadIdx.x == 0) {
    *fired = s_any;
    if (advance_seed) seed[0] = wadd(seed[0], 1);
  }
}

// tile 32 rows x 256 columns; lane owns one column, waves walk rows
__global__ __launch_bounds__(256) void rebalance_shift_kernel(int32_t* __restrict__ packed,
                                                              int64_t ld, int64_t N, int64_t K,
                                                              const int32_t* row_t,
                                                              const int32_t* col_t,
                                                              const int32_t* fired,
                                                              const int32_t* seed_p) {
  if (*fired == 0) return;
  const int64_t kb = (int64_t)blockIdx.x * 256, nb = (int64_t)blockIdx.y * 32;
  const int64_t k = kb + threadIdx.x;
  const int32_t ct = k < K ? col_t[k] : 0;
  const int32_t rt_probe = (threadIdx.x < 32 && nb + threadIdx.x < N) ? row_t[nb + threadIdx.x] : 0;
  if (!__syncthreads_or(ct != 0 || rt_probe != 0)) return;
  if (k >= K) return;
  const int32_t seed = *seed_p;
  const int32_t nk = (int32_t)((uint32_t)N * (uint32_t)K);
  for (int r = 0; r < 32; ++r) {
    const int64_t n = nb + r;
    if (n >= N) break;
    const int32_t net = row_t[n] + ct;
    if (net == 0) continue;
    int32_t* p = packed + n * ld + k;
    const Fields f = unpack(*p);
    int32_t sfn, ssn, vn;
    if (net < 0) {
      const int lsh = -net;
      sfn = wshl(f.sf, lsh);
      ssn = wshl(f.ss, lsh);
      vn = wshl(f.vs, lsh);
    } else {
      const int rsh = net;
      const float two_pos = (float)(1 << rsh);
      const int32_t off = wadd((int32_t)((uint32_t)n * (uint32_t)K), (int32_t)k);
      int32_t q = f.sf >> rsh;
      const int32_t sfs =
          q + ((__fmul_rn(tl_rand(seed, off), two_pos) < (float)wsub(f.sf, wshl(q, rsh))) ? 1 : 0);
      q = f.ss >> rsh;
      const int32_t ssu =
          q + ((__fmul_rn(tl_rand(seed, wadd(off, nk)), two_pos) < (float)wsub(f.ss, wshl(q, rsh))) ? 1 : 0);
      const int32_t ssr = wsub(wshl(f.ss, 7 - rsh), wshl(ssu, 7));
      q = f.vs >> rsh;
      const int32_t vu =
          q + ((__fmul_rn(tl_rand(seed, wadd(off, wshl(nk, 1))), two_pos) < (float)wsub(f.vs, wshl(q, rsh))) ? 1 : 0);
      const int32_t vr = wsub(wshl(f.vs, 7 - rsh), wshl(vu, 7));
      sfn = wadd(wadd(sfs, ssr), vr);
      ssn = ssu;
      vn = vu;
    }
    *p = pack(clampi(sfn, -32768, 32767), clampi(ssn, -128, 127), clampi(vn, -128, 127));
  }
}

}  // namespace concord

using namespace concord;

extern "C" int concord_rebalance(int32_t* packed, int64_t ld_p, int8_t* row_exp, int8_t* col_exp,
                                 const int32_t* row_max, const int32_t* col_max,
                                 int32_t* row_hwm, int32_t* col_hwm, int32_t* seed, int64_t N,
                                 int64_t K, int32_t max_m, int32_t exp_max, int32_t exp_min,
                                 int allow_tickdown, int advance_seed, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  CONCORD_CHECK(N > 0 && K > 0 && N < (1LL << 31) && K < (1LL << 31),
                "concord_rebalance: bad size");
  CONCORD_CHECK(packed && row_exp && col_exp && row_max && col_max && seed,
                "concord_rebalance: NULL argument");
  CONCORD_CHECK(ld_p >= K, "concord_rebalance: leading dimension < K");
  const Workspace ws = workspace_layout(N, K, 0);
  if (!workspace || workspace_bytes < ws.total) {
    set_error("concord_rebalance: workspace of %zu bytes needed", ws.total);
    return CONCORD_EWORKSPACE;
  }
  char* base = (char*)workspace;
  int32_t* row_t = (int32_t*)(base + ws.scratch);
  int32_t* col_t = row_t + N;
  int32_t* cnt_row = col_t + K;
  int32_t* cnt_col = cnt_row + N;
  int32_t* fired = (int32_t*)(base + ws.reb_fired);
  hipStream_t st = (hipStream_t)stream;
  if (allow_tickdown) {
    hipLaunchKernelGGL(fill_i32_kernel, dim3((unsigned)cdiv(N + K, 256)), dim3(256), 0, st, cnt_row,
                       N + K, 0);
    hipLaunchKernelGGL(i8_small_count_kernel, dim3((unsigned)cdiv(K, 256), (unsigned)cdiv(N, 32)),
                       dim3(256), 0, st, packed, ld_p, N, K, cnt_row, cnt_col);
  }
  hipLaunchKernelGGL(rebalance_decide_kernel, dim3(1), dim3(1024), 0, st, row_exp, col_exp, row_max,
                     col_max, row_hwm, col_hwm, cnt_row, cnt_col, seed, N, K, max_m, exp_max,
                     exp_min, allow_tickdown, advance_seed, row_t, col_t, fired);
  hipLaunchKernelGGL(rebalance_shift_kernel, dim3((unsigned)cdiv(K, 256), (unsigned)cdiv(N, 32)),
                     dim3(256), 0, st, packed, ld_p, N, K, row_t, col_t, fired, seed);
  return launch_status("rebalance");
}
