// workspace.h -- layout of the caller-owned workspaces.
//
// Update-side workspace:
// [0, 256)       counters: the v-hat "row blocks done" ticket (byte 0), the
//                grid barrier's arrivals (byte 64) and exits (byte 128) of
//                the WGRAD launch that carries the update; zero when the
//                workspace is created and zero again after every call.  Its
//                fault flag (byte 192) stays set until the host reads it
//                (concord_wgrad_update_fault).
// [256, total)   scratch shared by the entry points (they run in stream order):
//                v-hat partials, rebalance decisions, bias-gradient partials.
//                No entry point needs its contents to survive between calls.
#pragma once
#include <stddef.h>
#include <stdint.h>

namespace concord {

// the most ways a GEMM splits its reduction
constexpr int kGemmMaxSplits = 16;

struct Workspace {
  size_t vhat_ticket, scratch, total;
};
constexpr size_t kGridBarrierOffset = 64, kGridExitOffset = 128, kGridFaultOffset = 192;

// v-hat scratch (floats, each region a multiple of 64 so the next stays
// 256-byte aligned): row partials per 64-column tile, column partials per
// 64-row tile, one total per 256-row block of v_row
struct VhatScratch {
  int64_t pr, pc, bsum;
};
inline VhatScratch vhat_scratch(int64_t N, int64_t K) {
  auto cd = [](int64_t a, int64_t b) { return (a + b - 1) / b; };
  return VhatScratch{cd(cd(K, 64) * N, 64) * 64, cd(cd(N, 64) * K, 64) * 64, cd(cd(N, 256), 64) * 64};
}

inline Workspace workspace_layout(int64_t N, int64_t K, int64_t M) {
  auto cd = [](int64_t a, int64_t b) { return (a + b - 1) / b; };
  Workspace w;
  w.vhat_ticket = 0;
  w.scratch = 256;
  const VhatScratch v = vhat_scratch(N, K);
  const size_t vhat = (size_t)(v.pr + v.pc + v.bsum) * sizeof(float);
  // rebalance: ticks and tick-down counts per row and column, decide-block flags
  const size_t reb = (size_t)(2 * (N + K) + cd(N, 256) + cd(K, 256)) * sizeof(int32_t);
  // bias gradient partials (concord_wgrad_vhat places them after the v-hat
  // partials, which are still live when they are written)
  // (slab partials of the bias-gradient kernels, or [splits * cdiv(K, 128)][N]
  // partials of the wgrad kernel)
  size_t bias = (size_t)(cd(M, 64) * (N > K ? N : K)) * sizeof(float);
  const size_t bias_w = M > 0 ? (size_t)(kGemmMaxSplits * cd(K, 128) * N) * sizeof(float) : 0;
  if (bias_w > bias) bias = bias_w;
  size_t s = vhat + bias;
  if (reb > s) s = reb;
  w.total = w.scratch + ((s + 255) / 256) * 256;
  return w;
}

// GEMM split-K workspace (its own buffer): a fixed region of tile counters
// (the same offsets for every problem, so one call's fp32 partials can never
// sit where a later call expects zeroed counters), then two fp32 partial
// outputs [I][J].  Split-K is only used when the tile grid fits the counters.
constexpr int64_t kSplitkMaxTiles = 4096;
constexpr size_t kSplitkCounterBytes = (size_t)kSplitkMaxTiles * sizeof(uint32_t);
inline bool gemm_splitk_fits(int64_t tiles) { return tiles <= kSplitkMaxTiles; }
inline size_t gemm_splitk_bytes(int64_t I, int64_t J) {
  return kSplitkCounterBytes + (size_t)2 * (size_t)I * (size_t)J * sizeof(float);
}

}  // namespace concord
