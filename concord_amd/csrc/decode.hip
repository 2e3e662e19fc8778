// decode.hip -- packed state <-> dense weights.
//
// concord_materialize:  _materialize_packed_bf16_kernel (concord/packed_b.py:120-170),
//                       get_weight (1617-1630), consolidated_weight (1632-1649).
// concord_load_weights: load_weights (1570-1603), load_weights_finetune (1816-1856).
//
// Both are HBM-bound streams: materialize reads 4 B and writes 2 B per weight.
#include "common.h"

namespace concord {

// A lane decodes 8 consecutive words (two 16 B loads, one 16 B store); a
// block of 256 lanes covers 2048 columns of rows blockIdx.y, blockIdx.y +
// gridDim.y, ...
template <bool CONSOLIDATED, bool VEC>
__global__ __launch_bounds__(256) void materialize_kernel(const int32_t* __restrict__ packed,
                                                          int64_t ld_p, const int8_t* row_exp,
                                                          const int8_t* col_exp, int64_t N,
                                                          int64_t K, int32_t bias,
                                                          uint16_t* __restrict__ out,
                                                          int64_t ld_o) {
  const int64_t k0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (k0 >= K) return;
  for (int64_t n = blockIdx.y; n < N; n += gridDim.y) {
    const int32_t te_row = (int32_t)row_exp[n] - bias;
    const int32_t* src = packed + n * ld_p + k0;
    uint16_t* dst = out + n * ld_o + k0;
    auto decode = [&](int32_t w, int64_t k) -> float {
      const Fields f = unpack(w);
      const int32_t m = CONSOLIDATED ? (f.ss + f.vs) * 128 : f.ss * 128 + f.sf + f.vs * 128;
      return __fmul_rn((float)m, exp2i(te_row + (int32_t)col_exp[k]));
    };
    if (VEC && k0 + 8 <= K) {
      const int4 a = *reinterpret_cast<const int4*>(src);
      const int4 b = *reinterpret_cast<const int4*>(src + 4);
      uint4 o;
      o.x = pack_bf16x2(decode(a.x, k0 + 0), decode(a.y, k0 + 1));
      o.y = pack_bf16x2(decode(a.z, k0 + 2), decode(a.w, k0 + 3));
      o.z = pack_bf16x2(decode(b.x, k0 + 4), decode(b.y, k0 + 5));
      o.w = pack_bf16x2(decode(b.z, k0 + 6), decode(b.w, k0 + 7));
      *reinterpret_cast<uint4*>(dst) = o;
    } else {
      for (int j = 0; j < 8 && k0 + j < K; ++j)
        dst[j] = (uint16_t)(pack_bf16x2(decode(src[j], k0 + j), 0.0f) & 0xFFFFu);
    }
  }
}

// The forward weight with s_fast smoothly gated out (concord/packed_b.py:1763-1772):
// bf16(((128 ss + g sf) + 128 vs) * 2^(row_exp + col_exp - bias)), fp32 ops in
// that order.  One lane per word; rows strided by gridDim.y.
__global__ __launch_bounds__(256) void materialize_gated_kernel(const int32_t* __restrict__ packed,
                                                                int64_t ld_p, const int8_t* row_exp,
                                                                const int8_t* col_exp, int64_t N,
                                                                int64_t K, int32_t bias, float g,
                                                                uint16_t* __restrict__ out,
                                                                int64_t ld_o) {
  const int64_t k = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (k >= K) return;
  for (int64_t n = blockIdx.y; n < N; n += gridDim.y) {
    const Fields f = unpack(packed[n * ld_p + k]);
    const float m = __fadd_rn(__fadd_rn((float)(f.ss * 128), __fmul_rn(g, (float)f.sf)), (float)(f.vs * 128));
    const float v = __fmul_rn(m, exp2i((int32_t)row_exp[n] - bias + (int32_t)col_exp[k]));
    out[n * ld_o + k] = (uint16_t)(pack_bf16x2(v, 0.0f) & 0xFFFFu);
  }
}

// One block per row: row max |W| (exact), exponent, then quantise the row.
// row_exp = clamp(ceil(log2(max) + 1)) evaluated exactly from the exponent
// field: a power of two 2^q gives q + 1, anything in (2^q, 2^(q+1)) gives q + 2.
__global__ __launch_bounds__(256) void load_weights_kernel(const float* __restrict__ W,
                                                           int64_t ld_w, int64_t K,
                                                           int32_t exp_min, int32_t exp_max,
                                                           int32_t bias, int finetune,
                                                           int32_t* __restrict__ packed,
                                                           int64_t ld_p, int8_t* row_exp) {
  __shared__ float s_max[4];
  const int64_t n = blockIdx.x;
  const float* w = W + n * ld_w;
  float mx = 0.0f;
  for (int64_t k = threadIdx.x; k < K; k += 256) mx = fmaxf(mx, fabsf(w[k]));
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  if ((threadIdx.x & 63) == 0) s_max[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));
  mx = fmaxf(mx, 1e-30f);
  // mx is a normal float >= 1e-30: mx = 1.f * 2^q with q = biased exponent - 127
  const uint32_t u = __float_as_uint(mx);
  const int32_t q = (int32_t)((u >> 23) & 0xFF) - 127;
  int32_t e = ((u & 0x7FFFFFu) == 0) ? q + 1 : q + 2;
  e = clampi(e, exp_min, exp_max);
  if (threadIdx.x == 0) row_exp[n] = (int8_t)e;
  const float inv_scale = exp2i(bias - e);  // W / 2^(e - bias), exact
  for (int64_t k = threadIdx.x; k < K; k += 256) {
    const int32_t m = f2i(rintf(__fmul_rn(w[k], inv_scale)));
    int32_t sf, ss = 0, vs = 0;
    if (!finetune) {
      sf = clampi(m, -32768, 32767);
    } else {
      const int32_t tv = f2i(rintf(__fmul_rn((float)m, 0.5f)));
      vs = clampi(f2i(rintf(__fmul_rn((float)tv, 0.0078125f))), -128, 127);
      const int32_t rem = wsub(m, vs * 128);
      ss = clampi(f2i(rintf(__fmul_rn((float)rem, 0.0078125f))), -128, 127);
      sf = clampi(wsub(rem, ss * 128), -32768, 32767);
    }
    packed[n * ld_p + k] = pack(sf, ss, vs);
  }
}

__global__ void zero_i8_kernel(int8_t* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

}  // namespace concord

using namespace concord;

extern "C" int concord_materialize(const int32_t* packed, int64_t ld_p, const int8_t* row_exp,
                                   const int8_t* col_exp, int64_t N, int64_t K,
                                   int32_t mantissa_bias, int consolidated, uint16_t* out,
                                   int64_t ld_out, void* stream) {
  CONCORD_CHECK(N >= 0 && K >= 0 && N < (1LL << 31), "concord_materialize: bad size");
  if (N == 0 || K == 0) return CONCORD_OK;
  CONCORD_CHECK(packed && row_exp && col_exp && out, "concord_materialize: NULL argument");
  CONCORD_CHECK(ld_p >= K && ld_out >= K, "concord_materialize: leading dimension < K");
  const bool vec = (ld_p % 4 == 0) && (ld_out % 8 == 0) && ((uintptr_t)packed % 16 == 0) &&
                   ((uintptr_t)out % 16 == 0);
  dim3 grid((unsigned)cdiv(K, 2048), grid_y(N));
  hipStream_t st = (hipStream_t)stream;
#define LAUNCH(C, V)                                                                       \
  hipLaunchKernelGGL((materialize_kernel<C, V>), grid, dim3(256), 0, st, packed, ld_p, row_exp, \
                     col_exp, N, K, mantissa_bias, out, ld_out)
  if (consolidated) {
    if (vec) LAUNCH(true, true); else LAUNCH(true, false);
  } else {
    if (vec) LAUNCH(false, true); else LAUNCH(false, false);
  }
#undef LAUNCH
  return launch_status("materialize");
}

extern "C" int concord_materialize_gated(const int32_t* packed, int64_t ld_p, const int8_t* row_exp,
                                         const int8_t* col_exp, int64_t N, int64_t K,
                                         int32_t mantissa_bias, float fast_gain, uint16_t* out,
                                         int64_t ld_out, void* stream) {
  CONCORD_CHECK(N >= 0 && K >= 0 && N < (1LL << 31), "concord_materialize_gated: bad size");
  if (N == 0 || K == 0) return CONCORD_OK;
  CONCORD_CHECK(packed && row_exp && col_exp && out, "concord_materialize_gated: NULL argument");
  CONCORD_CHECK(ld_p >= K && ld_out >= K, "concord_materialize_gated: leading dimension < K");
  hipLaunchKernelGGL(materialize_gated_kernel, dim3((unsigned)cdiv(K, 256), grid_y(N)), dim3(256), 0,
                     (hipStream_t)stream, packed, ld_p, row_exp, col_exp, N, K, mantissa_bias, fast_gain, out,
                     ld_out);
  return launch_status("materialize_gated");
}

extern "C" int concord_load_weights(const float* W, int64_t ld_w, int64_t N, int64_t K,
                                    int32_t exp_min, int32_t exp_max, int32_t mantissa_bias,
                                    int finetune, int32_t* packed, int64_t ld_p, int8_t* row_exp,
                                    int8_t* col_exp, void* stream) {
  CONCORD_CHECK(N >= 0 && K >= 0 && N < (1LL << 31), "concord_load_weights: bad size");
  if (N == 0 || K == 0) return CONCORD_OK;
  CONCORD_CHECK(W && packed && row_exp && col_exp, "concord_load_weights: NULL argument");
  CONCORD_CHECK(ld_w >= K && ld_p >= K, "concord_load_weights: leading dimension < K");
  CONCORD_CHECK(exp_min <= exp_max, "concord_load_weights: exp_min > exp_max");
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(zero_i8_kernel, dim3((unsigned)cdiv(K, 256)), dim3(256), 0, st, col_exp, K);
  hipLaunchKernelGGL(load_weights_kernel, dim3((unsigned)N), dim3(256), 0, st, W, ld_w, K, exp_min,
                     exp_max, mantissa_bias, finetune, packed, ld_p, row_exp);
  return launch_status("load_weights");
}
