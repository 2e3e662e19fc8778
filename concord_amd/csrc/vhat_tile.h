// vhat_tile.h -- row and column partial sums of g^2 over one 64 x 64 tile,
// formed by one wave from values held in the MFMA accumulator layout.
//
// Lane l = 16 q + p holds, for x, y in [0, 4) and v in [0, 4), the value of
// tile row 16 x + p, column 16 y + 4 q + v.  The sums are taken in one fixed
// order (oracle_vhat_ema restates it); each lane first chains what it holds,
// then one cross-lane tree per row or column:
//   row partial    s(y, q) = ((g2_0 + g2_1) + g2_2) + g2_3 over the lane's 4 columns,
//                  u(q) = ((s(0,q) + s(1,q)) + s(2,q)) + s(3,q),
//                  P_r = (u(0) + u(1)) + (u(2) + u(3))     [lanes p, p+16, p+32, p+48]
//   column partial w(p) = ((a(p) + a(16+p)) + a(32+p)) + a(48+p) over the lane's 4 rows,
//                  P_c = pairwise tree over p, pairs (p, p+8), (p, p+4), (p, p+2), (p, p+1)
// Every cross-lane step adds the same two values on both lanes of a pair
// (a + b == b + a exactly), so all lanes of a group end with one value.
#pragma once
#include "common.h"

namespace concord {

// value of lane (l - n) mod 16 within each 16-lane row
template <int n>
CONCORD_DEV float row_ror(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + n, 0xF, 0xF, false));
}

// g2[x][y][v] = g^2 of this lane's values; row0 / col0 = first row / column of
// the tile (multiples of 64).  Writes P_r[col0 / 64][row] (rows < N) and
// P_c[row0 / 64][col] (columns < K); a tile that starts past N or K writes nothing.
// COH: every partial is stored with a relaxed agent-scope atomic store, for a
// reader in the same launch on another XCD.
template <bool COH = false>
CONCORD_DEV void vhat_tile_partials(const float (&g2)[4][4][4], int lane, int64_t row0, int64_t col0,
                                    int64_t N, int64_t K, float* __restrict__ pr,
                                    float* __restrict__ pc) {
  if (row0 >= N || col0 >= K) return;   // a wave past the matrix edge (uniform)
  const int p = lane & 15, q = lane >> 4;
  // rows
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    float u = 0.0f;
#pragma unroll
    for (int y = 0; y < 4; ++y) {
      const float s = __fadd_rn(__fadd_rn(__fadd_rn(g2[x][y][0], g2[x][y][1]), g2[x][y][2]), g2[x][y][3]);
      u = y == 0 ? s : __fadd_rn(u, s);
    }
    const float h = __fadd_rn(u, __shfl_xor(u, 16, 64));
    const float t = __fadd_rn(h, __shfl_xor(h, 32, 64));
    const int64_t n = row0 + 16 * x + p;
    if (q == 0 && n < N) {
      if (COH) __hip_atomic_store(pr + (col0 / 64) * N + n, t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      else pr[(col0 / 64) * N + n] = t;
    }
  }
  // columns
  float cs[4][4];
#pragma unroll
  for (int y = 0; y < 4; ++y)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float w = __fadd_rn(__fadd_rn(__fadd_rn(g2[0][y][v], g2[1][y][v]), g2[2][y][v]), g2[3][y][v]);
      w = __fadd_rn(w, row_ror<8>(w));
      w = __fadd_rn(w, row_ror<4>(w));
      w = __fadd_rn(w, row_ror<2>(w));
      w = __fadd_rn(w, row_ror<1>(w));
      cs[y][v] = w;
    }
  if (p == 0) {
    float* dst = pc + (row0 / 64) * K;
#pragma unroll
    for (int y = 0; y < 4; ++y) {
      const int64_t k = col0 + 16 * y + 4 * q;
      if (COH) {
#pragma unroll
        for (int v = 0; v < 4; ++v)
          if (k + v < K) __hip_atomic_store(dst + k + v, cs[y][v], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else if (k + 4 <= K && (K % 4) == 0) {
        *reinterpret_cast<float4*>(dst + k) = make_float4(cs[y][0], cs[y][1], cs[y][2], cs[y][3]);
      } else {
#pragma unroll
        for (int v = 0; v < 4; ++v)
          if (k + v < K) dst[k + v] = cs[y][v];
      }
    }
  }
}

}  // namespace concord
