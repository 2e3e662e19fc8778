// rebalance.hip -- exponent ratchet of the packed state.
//
// ConcordLinearPackedB.rebalance (concord/packed_b.py:1792-1814), rebalance_packed
// (1129-1190) and _rebalance_packed_decide_kernel (959-1095), as three kernels:
//   1. (tick-down only) count, per row and column, the words whose
//      max(|s_slow|, |v_slow|) <= 31: the lower median of that magnitude is
//      <= 31 exactly when more than (count - 1) / 2 of them are;
//   2. decide (a thread per row or column): high-watermarks, seed + 1,
//      per-row/column tick t in {-1, 0, +1} from the PRE-call exponents,
//      new exponents;
//   3. shift: each tile whose rows and columns all have t = 0 exits without
//      touching the packed words, so a call where nothing fires costs O(N + K);
//      a tile that fires deals its words to full waves (see below).
// The decisions of every tile come from the same pre-call exponents.  (In the
// reference the tiles with pid_k == 0 store the new row exponents while other
// tiles of the same launch may still be loading them.)
#include <mutex>

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

// One thread per row (blocks [0, cdiv(N, 256))) or column (the rest):
// high-watermark, tick decision from the pre-call exponent, new exponent.
// Thread 0 of block 0 advances the seed.
__global__ __launch_bounds__(256) void rebalance_decide_kernel(
    int8_t* row_exp, int8_t* col_exp, const int32_t* row_max, const int32_t* col_max,
    int32_t* row_hwm, int32_t* col_hwm, const int32_t* cnt_row, const int32_t* cnt_col,
    int32_t* seed, int64_t N, int64_t K, int32_t max_m, int32_t exp_max, int32_t exp_min,
    int allow_tickdown, int advance_seed, int32_t* row_t, int32_t* col_t, int32_t* bfired) {
  const int64_t rb = cdiv(N, 256);
  if (blockIdx.x == 0 && threadIdx.x == 0 && advance_seed) seed[0] = wadd(seed[0], 1);
  int32_t t = 0;
  if ((int64_t)blockIdx.x < rb) {
    const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (n < N) {
      const int32_t mx = row_max[n];
      if (row_hwm) row_hwm[n] = max(row_hwm[n], mx);
      const int32_t e = row_exp[n];
      const int up = (mx > max_m) && (e < exp_max);
      // lower median <= 31  <=>  count(<= 31) > (K - 1) / 2
      const int dn = allow_tickdown && (mx <= max_m) && (cnt_row[n] > (K - 1) / 2) && (e > exp_min);
      t = up - dn;
      row_t[n] = t;
      if (t) row_exp[n] = (int8_t)(e + t);
    }
  } else {
    const int64_t k = ((int64_t)blockIdx.x - rb) * 256 + threadIdx.x;
    if (k < K) {
      const int32_t mx = col_max[k];
      if (col_hwm) col_hwm[k] = max(col_hwm[k], mx);
      const int32_t e = col_exp[k];
      const int up = (mx > max_m) && (e < exp_max);
      const int dn = allow_tickdown && (mx <= max_m) && (cnt_col[k] > (N - 1) / 2) && (e > exp_min);
      t = up - dn;
      col_t[k] = t;
      if (t) col_exp[k] = (int8_t)(e + t);
    }
  }
  // per-block "something ticks" flag for the shift kernel's early exit
  const int any = __syncthreads_or(t != 0);
  if (threadIdx.x == 0) bfired[blockIdx.x] = any;
}

// SR shift of one word by net = row_t + col_t (concord/packed_b.py:1048-1090)
CONCORD_DEV void shift_word(int32_t* p, int32_t net, int64_t n, int64_t k, int64_t K, int32_t seed, int32_t nk) {
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

// tile 32 rows x 256 columns.  The words to shift are those in a fired
// column (every row) or a fired row (the other columns).  The tile lists its
// fired columns, unfired columns and fired rows in LDS and deals the words
// out to all 256 threads, so waves stay full however sparse the firing.
// Each word's result depends only on its own (n, k) and the seed, so the
// order of the lists is immaterial.
__global__ __launch_bounds__(256) void rebalance_shift_kernel(int32_t* __restrict__ packed,
                                                              int64_t ld, int64_t N, int64_t K,
                                                              const int32_t* row_t,
                                                              const int32_t* col_t,
                                                              const int32_t* bfired,
                                                              const int32_t* seed_p) {
  __shared__ int32_t s_fc[256], s_uc[256], s_fr[32];
  __shared__ int32_t s_nfc, s_nuc, s_nfr;
  const int64_t kb = (int64_t)blockIdx.x * 256, nb = (int64_t)blockIdx.y * 32;
  // the decide blocks covering this tile's 32 rows and 256 columns
  if (bfired[nb / 256] == 0 && bfired[cdiv(N, 256) + kb / 256] == 0) return;
  const int t = threadIdx.x;
  const int64_t k = kb + t;
  const int32_t ct = k < K ? col_t[k] : 0;
  const int32_t rt_probe = (t < 32 && nb + t < N) ? row_t[nb + t] : 0;
  if (!__syncthreads_or(ct != 0 || rt_probe != 0)) return;
  if (t == 0) {
    s_nfc = 0;
    s_nuc = 0;
    s_nfr = 0;
  }
  __syncthreads();
  if (k < K) {
    if (ct != 0) s_fc[atomicAdd(&s_nfc, 1)] = t;
    else s_uc[atomicAdd(&s_nuc, 1)] = t;
  }
  if (rt_probe != 0) s_fr[atomicAdd(&s_nfr, 1)] = t;
  __syncthreads();
  const int nfc = s_nfc, nuc = s_nuc, nfr = s_nfr;
  const int rows = (int)min((int64_t)32, N - nb);
  const int32_t seed = *seed_p;
  const int32_t nk = (int32_t)((uint32_t)N * (uint32_t)K);
  // fired columns, all rows of the tile
  for (int it = t; it < nfc * rows; it += 256) {
    const int c = s_fc[it / rows], r = it % rows;
    const int64_t n = nb + r, kk = kb + c;
    const int32_t net = row_t[n] + col_t[kk];
    if (net != 0) shift_word(packed + n * ld + kk, net, n, kk, K, seed, nk);
  }
  // fired rows, the columns that did not fire
  for (int it = t; it < nfr * nuc; it += 256) {
    const int r = s_fr[it / nuc], c = s_uc[it % nuc];
    const int64_t n = nb + r, kk = kb + c;
    shift_word(packed + n * ld + kk, row_t[n], n, kk, K, seed, nk);
  }
}

}  // namespace concord

namespace concord {

// The launches of one rebalance call; `scr` holds 2 (N + K) + cdiv(N, 256) +
// cdiv(K, 256) int32 of scratch (ticks, tick-down counts, decide-block flags).
// Every word of it that a kernel reads is written earlier in the same call.
static int rebalance_launch(int32_t* packed, int64_t ld_p, int8_t* row_exp, int8_t* col_exp,
                            const int32_t* row_max, const int32_t* col_max, int32_t* row_hwm,
                            int32_t* col_hwm, int32_t* seed, int64_t N, int64_t K, int32_t max_m,
                            int32_t exp_max, int32_t exp_min, int allow_tickdown, int advance_seed,
                            int32_t* scr, hipStream_t st) {
  int32_t* row_t = scr;
  int32_t* col_t = row_t + N;
  int32_t* cnt_row = col_t + K;
  int32_t* cnt_col = cnt_row + N;
  int32_t* bfired = cnt_col + K;   // one flag per decide block
  if (allow_tickdown) {
    hipLaunchKernelGGL(fill_i32_kernel, dim3((unsigned)cdiv(N + K, 256)), dim3(256), 0, st, cnt_row,
                       N + K, 0);
    hipLaunchKernelGGL(i8_small_count_kernel, dim3((unsigned)cdiv(K, 256), (unsigned)cdiv(N, 32)),
                       dim3(256), 0, st, packed, ld_p, N, K, cnt_row, cnt_col);
  }
  hipLaunchKernelGGL(rebalance_decide_kernel, dim3((unsigned)(cdiv(N, 256) + cdiv(K, 256))), dim3(256), 0, st,
                     row_exp, col_exp, row_max, col_max, row_hwm, col_hwm, cnt_row, cnt_col, seed, N, K,
                     max_m, exp_max, exp_min, allow_tickdown, advance_seed, row_t, col_t, bfired);
  hipLaunchKernelGGL(rebalance_shift_kernel, dim3((unsigned)cdiv(K, 256), (unsigned)cdiv(N, 32)),
                     dim3(256), 0, st, packed, ld_p, N, K, row_t, col_t, bfired, seed);
  return launch_status("rebalance");
}

// Scratch of concord_rebalance_noalloc: a file-scope device array, one copy
// per device, held until the process ends.  Host code uses the device
// address hipGetSymbolAddress returns for it (per device), never the array's
// name, which on the host is only a stand-in.
constexpr int64_t kNoAllocMaxDim = 131072;   // rows and columns, each
constexpr int64_t kNoAllocScratchWords = 4 * kNoAllocMaxDim + 2 * (kNoAllocMaxDim / 256);
static __device__ __align__(256) int32_t scratch[kNoAllocScratchWords];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static int32_t* g_scratch_ptr[kMaxDevices];

// the device address of `scratch` on device `dev`, looked up once per device
// with that device current
static int32_t* scratch_on(int dev) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error("concord_rebalance_noalloc: hipGetSymbolAddress of the scratch array failed on device %d: %s",
                dev, hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = (int32_t*)p;
  }
  return g_scratch_ptr[dev];
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
  CONCORD_CHECK(cdiv(N, 32) <= kMaxGridY,
                "concord_rebalance: N=%lld rows exceed the shift kernel's grid (at most %lld rows)",
                (long long)N, (long long)(kMaxGridY * 32));
  const Workspace ws = workspace_layout(N, K, 0);
  if (!workspace || workspace_bytes < ws.total) {
    set_error("concord_rebalance: workspace of %zu bytes needed", ws.total);
    return CONCORD_EWORKSPACE;
  }
  return rebalance_launch(packed, ld_p, row_exp, col_exp, row_max, col_max, row_hwm, col_hwm, seed, N, K, max_m,
                          exp_max, exp_min, allow_tickdown, advance_seed,
                          (int32_t*)((char*)workspace + ws.scratch), (hipStream_t)stream);
}

extern "C" int concord_rebalance_noalloc(int32_t* packed, int64_t ld_p, int8_t* row_exp, int8_t* col_exp,
                                         const int32_t* row_max, const int32_t* col_max, int32_t* row_hwm,
                                         int32_t* col_hwm, int32_t* seed, int64_t N, int64_t K, int32_t max_m,
                                         int32_t exp_max, int32_t exp_min, int allow_tickdown, int advance_seed,
                                         void* stream) {
  CONCORD_CHECK(N > 0 && K > 0, "concord_rebalance_noalloc: bad size");
  CONCORD_CHECK(N <= kNoAllocMaxDim && K <= kNoAllocMaxDim,
                "concord_rebalance_noalloc: N=%lld K=%lld exceed the static scratch (at most %lld rows and %lld "
                "columns); use concord_rebalance with a workspace",
                (long long)N, (long long)K, (long long)kNoAllocMaxDim, (long long)kNoAllocMaxDim);
  CONCORD_CHECK(packed && row_exp && col_exp && row_max && col_max && seed,
                "concord_rebalance_noalloc: NULL argument");
  CONCORD_CHECK(ld_p >= K, "concord_rebalance_noalloc: leading dimension < K");
  hipStream_t st = (hipStream_t)stream;
  int cur = -1, sdev = -1;
  CONCORD_CHECK(hipGetDevice(&cur) == hipSuccess && hipStreamGetDevice(st, &sdev) == hipSuccess,
                "concord_rebalance_noalloc: cannot query the current device or the stream's device");
  CONCORD_CHECK(cur == sdev && cur >= 0 && cur < kMaxDevices,
                "concord_rebalance_noalloc: the stream belongs to device %d, the current device is %d", sdev, cur);
  int32_t* scr = scratch_on(cur);
  if (scr == nullptr) return CONCORD_ELAUNCH;
  return rebalance_launch(packed, ld_p, row_exp, col_exp, row_max, col_max, row_hwm, col_hwm, seed, N, K, max_m,
                          exp_max, exp_min, allow_tickdown, advance_seed, scr, st);
}
