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

// Decision for one row (item < N) or column (item - N < K): high-watermark,
// tick t in {-1, 0, +1} from the pre-call exponent, new exponent.  Returns t.
CONCORD_DEV int32_t decide_item(int64_t item, int8_t* row_exp, int8_t* col_exp, const int32_t* row_max,
                                const int32_t* col_max, int32_t* row_hwm, int32_t* col_hwm,
                                const int32_t* cnt_row, const int32_t* cnt_col, int64_t N, int64_t K,
                                int32_t max_m, int32_t exp_max, int32_t exp_min, int allow_tickdown,
                                int32_t* row_t, int32_t* col_t) {
  const bool is_row = item < N;
  const int64_t i = is_row ? item : item - N;
  const int32_t mx = is_row ? row_max[i] : col_max[i];
  int32_t* hwm = is_row ? row_hwm : col_hwm;
  if (hwm) hwm[i] = max(hwm[i], mx);
  int8_t* ex = is_row ? row_exp : col_exp;
  const int32_t e = ex[i];
  const int up = (mx > max_m) && (e < exp_max);
  // lower median <= 31  <=>  count(<= 31) > (count - 1) / 2
  const int dn = allow_tickdown && (mx <= max_m) &&
                 ((is_row ? cnt_row[i] : cnt_col[i]) > ((is_row ? K : N) - 1) / 2) && (e > exp_min);
  const int32_t t = up - dn;
  (is_row ? row_t : col_t)[i] = t;
  if (t) ex[i] = (int8_t)(e + t);
  return t;
}

// One thread per row (blocks [0, cdiv(N, 256))) or column (the rest).
// Thread 0 of block 0 advances the seed.
__global__ __launch_bounds__(256) void rebalance_decide_kernel(
    int8_t* row_exp, int8_t* col_exp, const int32_t* row_max, const int32_t* col_max,
    int32_t* row_hwm, int32_t* col_hwm, const int32_t* cnt_row, const int32_t* cnt_col,
    int32_t* seed, int64_t N, int64_t K, int32_t max_m, int32_t exp_max, int32_t exp_min,
    int allow_tickdown, int advance_seed, int32_t* row_t, int32_t* col_t, int32_t* bfired) {
  const int64_t rb = cdiv(N, 256);
  if (blockIdx.x == 0 && threadIdx.x == 0 && advance_seed) seed[0] = wadd(seed[0], 1);
  // rows fill whole blocks: the columns start at block rb
  const int64_t b = blockIdx.x;
  const int64_t item = b < rb ? b * 256 + threadIdx.x : N + (b - rb) * 256 + threadIdx.x;
  int32_t t = 0;
  if (b < rb ? item < N : item - N < K)
    t = decide_item(item, row_exp, col_exp, row_max, col_max, row_hwm, col_hwm, cnt_row, cnt_col, N, K, max_m,
                    exp_max, exp_min, allow_tickdown, row_t, col_t);
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

// rows of a shift tile
constexpr int kShiftRows = 16;

// One tile of kShiftRows rows x 256 columns (rows from nb, columns from kb).  The
// words to shift are those in a fired column (every row) or a fired row (the
// other columns).  The tile lists its fired columns, unfired columns and
// fired rows in LDS and deals the words out to all 256 threads, so waves stay
// full however sparse the firing.  Each word's result depends only on its own
// (n, k) and the seed, so the order of the lists is immaterial.  Called by
// every thread of the block with the same arguments; it begins with a
// barrier, so consecutive calls may reuse the lists.
struct ShiftLists {
  int32_t fc[256], uc[256], fr[kShiftRows];
  int32_t nfc, nuc, nfr;
};

CONCORD_DEV void shift_tile(int32_t* __restrict__ packed, int64_t ld, int64_t N, int64_t K,
                            const int32_t* row_t, const int32_t* col_t, int32_t seed, int64_t kb, int64_t nb,
                            ShiftLists& L) {
  const int t = threadIdx.x;
  const int64_t k = kb + t;
  const int32_t ct = k < K ? col_t[k] : 0;
  const int32_t rt_probe = (t < kShiftRows && nb + t < N) ? row_t[nb + t] : 0;
  if (!__syncthreads_or(ct != 0 || rt_probe != 0)) return;
  if (t == 0) {
    L.nfc = 0;
    L.nuc = 0;
    L.nfr = 0;
  }
  __syncthreads();
  if (k < K) {
    if (ct != 0) L.fc[atomicAdd(&L.nfc, 1)] = t;
    else L.uc[atomicAdd(&L.nuc, 1)] = t;
  }
  if (rt_probe != 0) L.fr[atomicAdd(&L.nfr, 1)] = t;
  __syncthreads();
  const int nfc = L.nfc, nuc = L.nuc, nfr = L.nfr;
  const int rows = (int)min((int64_t)kShiftRows, N - nb);
  const int32_t nk = (int32_t)((uint32_t)N * (uint32_t)K);
  // fired columns, all rows of the tile
  for (int it = t; it < nfc * rows; it += 256) {
    const int c = L.fc[it / rows], r = it % rows;
    const int64_t n = nb + r, kk = kb + c;
    const int32_t net = row_t[n] + col_t[kk];
    if (net != 0) shift_word(packed + n * ld + kk, net, n, kk, K, seed, nk);
  }
  // fired rows, the columns that did not fire
  for (int it = t; it < nfr * nuc; it += 256) {
    const int r = L.fr[it / nuc], c = L.uc[it % nuc];
    const int64_t n = nb + r, kk = kb + c;
    shift_word(packed + n * ld + kk, row_t[n], n, kk, K, seed, nk);
  }
}

__global__ __launch_bounds__(256) void rebalance_shift_kernel(int32_t* __restrict__ packed,
                                                              int64_t ld, int64_t N, int64_t K,
                                                              const int32_t* row_t,
                                                              const int32_t* col_t,
                                                              const int32_t* bfired,
                                                              const int32_t* seed_p) {
  __shared__ ShiftLists L;
  const int64_t kb = (int64_t)blockIdx.x * 256, nb = (int64_t)blockIdx.y * kShiftRows;
  // the decide blocks covering this tile's rows and 256 columns
  if (bfired[nb / 256] == 0 && bfired[cdiv(N, 256) + kb / 256] == 0) return;
  shift_tile(packed, ld, N, K, row_t, col_t, *seed_p, kb, nb, L);
}

// ---------------------------------------------------------------------------
// Gated rebalance of a group of layers (GatedRebalance,
// notebook/src/concord_winner.py:206-262): the gate (the largest watermark of
// every layer > gate_max) is read on the device, so a step that does not fire
// costs two launches whose blocks exit at once, with no host read.  When it
// fires, every layer is rebalanced as concord_rebalance(..., allow_tickdown 0,
// advance_seed 1) would.  The plan (built on the host by
// concord_rebalance_group_plan) holds one record of kRgFields int64 per layer,
// then the prefix sums of decide blocks and of shift tiles over the layers.
// ---------------------------------------------------------------------------
enum {
  RG_PACKED, RG_LD, RG_ROW_EXP, RG_COL_EXP, RG_ROW_MAX, RG_COL_MAX, RG_ROW_HWM, RG_COL_HWM, RG_SEED,
  RG_N, RG_K, RG_MAX_M, RG_EXP_MAX, RG_EXP_MIN, RG_SCR, RG_RESERVED, kRgFields
};

struct RgLayer {
  int32_t* packed;
  int64_t ld;
  int8_t *row_exp, *col_exp;
  const int32_t *row_max, *col_max;
  int32_t *row_hwm, *col_hwm, *seed;
  int64_t N, K;
  int32_t max_m, exp_max, exp_min;
  int32_t *row_t, *col_t, *bfired;
};

CONCORD_DEV RgLayer rg_layer(const int64_t* plan, int l, int32_t* scratch) {
  const int64_t* r = plan + (int64_t)l * kRgFields;
  RgLayer L;
  L.packed = (int32_t*)r[RG_PACKED];
  L.ld = r[RG_LD];
  L.row_exp = (int8_t*)r[RG_ROW_EXP];
  L.col_exp = (int8_t*)r[RG_COL_EXP];
  L.row_max = (const int32_t*)r[RG_ROW_MAX];
  L.col_max = (const int32_t*)r[RG_COL_MAX];
  L.row_hwm = (int32_t*)r[RG_ROW_HWM];
  L.col_hwm = (int32_t*)r[RG_COL_HWM];
  L.seed = (int32_t*)r[RG_SEED];
  L.N = r[RG_N];
  L.K = r[RG_K];
  L.max_m = (int32_t)r[RG_MAX_M];
  L.exp_max = (int32_t)r[RG_EXP_MAX];
  L.exp_min = (int32_t)r[RG_EXP_MIN];
  L.row_t = scratch + r[RG_SCR];
  L.col_t = L.row_t + L.N;
  L.bfired = L.col_t + L.K;
  return L;
}

// the layer l with pref[l] <= x < pref[l + 1] (pref non-decreasing, pref[0] = 0, x < pref[n])
CONCORD_DEV int rg_find(const int64_t* pref, int n, int64_t x) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (pref[mid] <= x) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// grid-stride over the decide blocks of every layer
__global__ __launch_bounds__(256) void rebalance_group_decide_kernel(const int64_t* __restrict__ plan, int n,
                                                                     const int32_t* peak, int32_t gate_max,
                                                                     int32_t* fires, int32_t* scratch) {
  if (peak[0] <= gate_max) return;
  if (blockIdx.x == 0 && threadIdx.x == 0 && fires) fires[0] = wadd(fires[0], 1);
  const int64_t* dpref = plan + (int64_t)n * kRgFields;
  const int64_t total = dpref[n];
  for (int64_t g = blockIdx.x; g < total; g += gridDim.x) {
    const int l = rg_find(dpref, n, g);
    const RgLayer L = rg_layer(plan, l, scratch);
    const int64_t b = g - dpref[l], rb = cdiv(L.N, 256);
    if (b == 0 && threadIdx.x == 0) L.seed[0] = wadd(L.seed[0], 1);
    const int64_t item = b < rb ? b * 256 + threadIdx.x : L.N + (b - rb) * 256 + threadIdx.x;
    int32_t t = 0;
    if (b < rb ? item < L.N : item - L.N < L.K)
      t = decide_item(item, L.row_exp, L.col_exp, L.row_max, L.col_max, L.row_hwm, L.col_hwm, nullptr, nullptr,
                      L.N, L.K, L.max_m, L.exp_max, L.exp_min, 0, L.row_t, L.col_t);
    const int any = __syncthreads_or(t != 0);
    if (threadIdx.x == 0) L.bfired[b] = any;
  }
}

// Each block walks a contiguous range of the shift tiles of every layer.  A
// layer none of whose decide blocks fired is skipped whole; inside a layer
// that fired, each wave tests 64 tiles' decide flags at once and jumps to the
// next flagged tile.  Every wave makes the same loads of data this kernel does
// not write, so the control flow is uniform across the block.
__global__ __launch_bounds__(256) void rebalance_group_shift_kernel(const int64_t* __restrict__ plan, int n,
                                                                    const int32_t* peak, int32_t gate_max,
                                                                    int32_t* scratch) {
  __shared__ ShiftLists LS;
  if (peak[0] <= gate_max) return;
  const int lane = threadIdx.x & 63;
  const int64_t* tpref = plan + (int64_t)n * kRgFields + (n + 1);
  const int64_t total = tpref[n];
  const int64_t per = cdiv(total, (int64_t)gridDim.x);
  int64_t x = (int64_t)blockIdx.x * per;
  const int64_t x_end = min(total, x + per);
  if (x >= x_end) return;
  int l = rg_find(tpref, n, x);
  while (x < x_end) {
    while (tpref[l + 1] <= x) ++l;
    const RgLayer L = rg_layer(plan, l, scratch);
    const int64_t l_end = min(x_end, tpref[l + 1]);
    const int64_t rb = cdiv(L.N, 256), nd = rb + cdiv(L.K, 256);
    int any = 0;
    for (int64_t i = lane; i < nd; i += 64) any |= L.bfired[i];
    if (__ballot(any != 0) == 0) {
      x = l_end;
      continue;
    }
    const int64_t ct = cdiv(L.K, 256);
    const int32_t seed = L.seed[0];
    while (x < l_end) {
      const int64_t y = x - tpref[l] + lane;   // this lane's tile in the layer
      const int64_t yb = y / ct;
      const bool flagged =
          x + lane < l_end && (L.bfired[(yb * kShiftRows) / 256] != 0 || L.bfired[rb + (y - yb * ct)] != 0);
      const uint64_t m = __ballot(flagged);
      if (m == 0) {
        x = min(x + 64, l_end);   // the range may go on into the next layer
        continue;
      }
      x += __builtin_ctzll(m);
      const int64_t yt = x - tpref[l];
      shift_tile(L.packed, L.ld, L.N, L.K, L.row_t, L.col_t, seed, (yt % ct) * 256, (yt / ct) * kShiftRows, LS);
      ++x;
    }
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
  hipLaunchKernelGGL(rebalance_shift_kernel, dim3((unsigned)cdiv(K, 256), (unsigned)cdiv(N, kShiftRows)),
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
  CONCORD_CHECK(cdiv(N, kShiftRows) <= kMaxGridY,
                "concord_rebalance: N=%lld rows exceed the shift kernel's grid (at most %lld rows)",
                (long long)N, (long long)(kMaxGridY * kShiftRows));
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

extern "C" int concord_rebalance_group_plan(const int64_t* layers, int32_t n_layers, int64_t* plan,
                                            int64_t plan_len, int64_t* scratch_words) {
  CONCORD_CHECK(n_layers > 0 && n_layers < (1 << 24), "concord_rebalance_group_plan: bad layer count %d",
                (int)n_layers);
  CONCORD_CHECK(layers && plan && scratch_words, "concord_rebalance_group_plan: NULL argument");
  const int64_t n = n_layers;
  CONCORD_CHECK(plan_len >= n * kRgFields + 2 * (n + 1),
                "concord_rebalance_group_plan: plan needs %lld int64, got %lld",
                (long long)(n * kRgFields + 2 * (n + 1)), (long long)plan_len);
  int64_t* dpref = plan + n * kRgFields;
  int64_t* tpref = dpref + (n + 1);
  int64_t scr = 0;
  dpref[0] = tpref[0] = 0;
  for (int64_t l = 0; l < n; ++l) {
    const int64_t* r = layers + l * kRgFields;
    const int64_t N = r[RG_N], K = r[RG_K];
    CONCORD_CHECK(N > 0 && K > 0 && N < (1LL << 31) && K < (1LL << 31),
                  "concord_rebalance_group_plan: layer %lld: bad size %lld x %lld", (long long)l, (long long)N,
                  (long long)K);
    CONCORD_CHECK(r[RG_LD] >= K, "concord_rebalance_group_plan: layer %lld: leading dimension < K",
                  (long long)l);
    CONCORD_CHECK(r[RG_PACKED] && r[RG_ROW_EXP] && r[RG_COL_EXP] && r[RG_ROW_MAX] && r[RG_COL_MAX] && r[RG_SEED],
                  "concord_rebalance_group_plan: layer %lld: NULL pointer", (long long)l);
    CONCORD_CHECK(r[RG_MAX_M] >= INT32_MIN && r[RG_MAX_M] <= INT32_MAX && r[RG_EXP_MAX] >= -128 &&
                      r[RG_EXP_MAX] <= 127 && r[RG_EXP_MIN] >= -128 && r[RG_EXP_MIN] <= 127,
                  "concord_rebalance_group_plan: layer %lld: MAX_M or exponent range out of range", (long long)l);
    int64_t* o = plan + l * kRgFields;
    for (int f = 0; f < kRgFields; ++f) o[f] = r[f];
    o[RG_SCR] = scr;
    o[RG_RESERVED] = 0;
    const int64_t nd = cdiv(N, 256) + cdiv(K, 256);
    scr += N + K + nd;
    dpref[l + 1] = dpref[l] + nd;
    tpref[l + 1] = tpref[l] + cdiv(N, kShiftRows) * cdiv(K, 256);
  }
  *scratch_words = scr;
  return CONCORD_OK;
}

extern "C" int concord_rebalance_group(const int64_t* plan, int32_t n_layers, const int32_t* peak,
                                       int32_t gate_max, int32_t* fires, void* workspace,
                                       size_t workspace_bytes, int64_t scratch_words, void* stream) {
  CONCORD_CHECK(n_layers > 0 && n_layers < (1 << 24), "concord_rebalance_group: bad layer count %d",
                (int)n_layers);
  CONCORD_CHECK(plan && peak, "concord_rebalance_group: NULL argument");
  CONCORD_CHECK(scratch_words > 0, "concord_rebalance_group: bad scratch size");
  if (!workspace || workspace_bytes < (size_t)scratch_words * 4) {
    set_error("concord_rebalance_group: workspace of %zu bytes needed", (size_t)scratch_words * 4);
    return CONCORD_EWORKSPACE;
  }
  hipStream_t st = (hipStream_t)stream;
  int32_t* scr = (int32_t*)workspace;
  hipLaunchKernelGGL(rebalance_group_decide_kernel, dim3(1024), dim3(256), 0, st, plan, (int)n_layers, peak,
                     gate_max, fires, scr);
  hipLaunchKernelGGL(rebalance_group_shift_kernel, dim3(2048), dim3(256), 0, st, plan, (int)n_layers, peak,
                     gate_max, scr);
  return launch_status("rebalance_group");
}
