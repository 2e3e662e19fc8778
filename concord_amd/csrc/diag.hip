// diag.hip -- measurement kernels for the data path the GEMM kernels use
// (no counterpart in the reference; declared in concord_amd_diag.h).
//
// concord_diag_dma_copy: a device copy whose reads are the LDS-DMA loads the
//   GEMM kernels issue (buffer_load_dwordx4 ... lds, 1 KB per wave
//   instruction), each source byte read once and written once from LDS with
//   16-byte stores.  Its FETCH_SIZE / WRITE_SIZE counters against the bytes
//   moved calibrate the traffic figures of kernels that load through LDS-DMA.
// concord_diag_l2_stream: every workgroup streams the region of its XCD
//   (workgroup w runs on XCD w mod 8; region x = bytes [x R, (x + 1) R)),
//   `reps` times, with `depth` 16 KB chunks in flight per workgroup, either
//   by LDS-DMA into a ring of LDS slots or by 16-byte loads into registers.
//   With R well below the 4 MB L2 of an XCD every pass after the first hits
//   in L2, so bytes / time / CU is the L2-to-CU rate of that load path.
#include "common.h"

namespace concord {
namespace {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr int kChunk = 16384;   // bytes per chunk: 4 waves x 4 instructions x 1 KB

// s_waitcnt immediate (gfx9 encoding): at most n vector memory operations
// outstanding, the other counters untouched
constexpr int vmcnt_imm(int n) { return (n & 0xF) | (0x7 << 4) | (0xF << 8) | (((n >> 4) & 3) << 14); }

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(uintptr_t)(lds_ptr_t)p);
}
__device__ __forceinline__ i32x4 rsrc(const void* p, uint32_t bytes) {
  const uint64_t base = (uint64_t)(uintptr_t)p;
  i32x4 r = i32x4{(int32_t)(uint32_t)base, (int32_t)(uint32_t)((base >> 32) & 0xFFFF), (int32_t)bytes, 0x00020000};
  for (int e = 0; e < 4; ++e) r[e] = __builtin_amdgcn_readfirstlane(r[e]);
  return r;
}
// lane l's 16 bytes at voff land at LDS lds_base + 16 l
__device__ __forceinline__ void dma16(i32x4 rs, uint32_t voff, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(voff), "s"(rs), "s"(lds_base)
               : "memory", "m0");
}

__global__ __launch_bounds__(256) void dma_copy_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                       uint32_t bytes) {
  __shared__ __attribute__((aligned(1024))) uint8_t slot[kChunk];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const i32x4 rs = rsrc(src, bytes);
  const uint32_t chunks = bytes / kChunk;
  for (uint32_t c = blockIdx.x; c < chunks; c += gridDim.x) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t off = (uint32_t)(wave * 4 + q) * 1024;
      dma16(rs, c * kChunk + off + lane * 16, lds_addr(slot + off));
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    // each lane reads back only the bytes its own loads wrote
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t off = (uint32_t)(wave * 4 + q) * 1024 + lane * 16;
      *reinterpret_cast<uint4*>(dst + (size_t)c * kChunk + off) = *reinterpret_cast<const uint4*>(slot + off);
    }
  }
}

// DEPTH chunks in flight; LDS: DEPTH slots (the DMA form)
template <int DEPTH, bool DMA>
__global__ __launch_bounds__(256) void l2_stream_kernel(const uint8_t* __restrict__ src, uint32_t region, int reps,
                                                        uint32_t* sink) {
  __shared__ __attribute__((aligned(1024))) uint8_t slot[DMA ? DEPTH * kChunk : 16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint8_t* base = src + (size_t)(blockIdx.x % 8) * region;
  const i32x4 rs = rsrc(base, region);
  const uint32_t chunks = region / kChunk;
  const uint32_t total = chunks * (uint32_t)reps;
  uint32_t acc = 0;
  if (DMA) {
    for (uint32_t i = 0; i < total; ++i) {
      const uint32_t c = i % chunks;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t off = (uint32_t)(wave * 4 + q) * 1024;
        dma16(rs, c * kChunk + off + lane * 16, lds_addr(slot + (i % DEPTH) * kChunk + off));
      }
      // the chunk issued DEPTH - 1 chunks ago has landed
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(4 * (DEPTH - 1)));
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  } else {
    // batches of DEPTH chunks: all their loads issued, then consumed
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), (short)0, (int)region, 0x00020000);
    for (uint32_t i = 0; i + DEPTH <= total; i += DEPTH) {
      i32x4 v[DEPTH][4];
#pragma unroll
      for (int d = 0; d < DEPTH; ++d)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          v[d][q] = __builtin_amdgcn_raw_buffer_load_b128(
              rb, ((i + d) % chunks) * kChunk + (uint32_t)(wave * 4 + q) * 1024 + lane * 16, 0, 0);
#pragma unroll
      for (int d = 0; d < DEPTH; ++d)
#pragma unroll
        for (int q = 0; q < 4; ++q) acc ^= (uint32_t)(v[d][q][0] ^ v[d][q][1] ^ v[d][q][2] ^ v[d][q][3]);
    }
    if (acc == 0x9E3779B9u) sink[0] = acc;   // keeps the register loads
  }
}

}  // namespace
}  // namespace concord

using namespace concord;

extern "C" int concord_diag_dma_copy(const void* src, void* dst, size_t bytes, void* stream) {
  CONCORD_CHECK(src && dst, "concord_diag_dma_copy: NULL argument");
  CONCORD_CHECK(bytes % kChunk == 0 && bytes < ((size_t)1 << 31),
                "concord_diag_dma_copy: bytes must be a multiple of %d below 2^31", kChunk);
  CONCORD_CHECK(((uintptr_t)src % 16) == 0 && ((uintptr_t)dst % 16) == 0, "concord_diag_dma_copy: 16-byte alignment");
  if (bytes == 0) return CONCORD_OK;
  const uint32_t chunks = (uint32_t)(bytes / kChunk);
  hipLaunchKernelGGL(dma_copy_kernel, dim3(chunks < 4096 ? chunks : 4096), dim3(256), 0, (hipStream_t)stream,
                     (const uint8_t*)src, (uint8_t*)dst, (uint32_t)bytes);
  return launch_status("diag_dma_copy");
}

extern "C" int concord_diag_l2_stream(const void* src, size_t region_bytes, int reps, int blocks, int depth,
                                      int lds_dma, uint32_t* sink, void* stream) {
  CONCORD_CHECK(src && sink, "concord_diag_l2_stream: NULL argument");
  CONCORD_CHECK(region_bytes % kChunk == 0 && region_bytes > 0 && region_bytes < ((size_t)1 << 28),
                "concord_diag_l2_stream: region must be a positive multiple of %d below 2^28", kChunk);
  CONCORD_CHECK(reps > 0 && blocks > 0 && blocks <= 65535, "concord_diag_l2_stream: bad reps or blocks");
  CONCORD_CHECK(((uintptr_t)src % 16) == 0, "concord_diag_l2_stream: 16-byte alignment");
  const hipStream_t st = (hipStream_t)stream;
  const uint8_t* s = (const uint8_t*)src;
  const uint32_t r = (uint32_t)region_bytes;
#define CONCORD_L2S(D, M) \
  hipLaunchKernelGGL((l2_stream_kernel<D, M>), dim3(blocks), dim3(256), 0, st, s, r, reps, sink)
  if (lds_dma) {
    switch (depth) {
      case 2: CONCORD_L2S(2, true); break;
      case 4: CONCORD_L2S(4, true); break;
      case 8: CONCORD_L2S(8, true); break;
      default: set_error("concord_diag_l2_stream: depth must be 2, 4 or 8"); return CONCORD_EINVAL;
    }
  } else {
    switch (depth) {
      case 2: CONCORD_L2S(2, false); break;
      case 4: CONCORD_L2S(4, false); break;
      case 8: CONCORD_L2S(8, false); break;
      default: set_error("concord_diag_l2_stream: depth must be 2, 4 or 8"); return CONCORD_EINVAL;
    }
  }
#undef CONCORD_L2S
  return launch_status("diag_l2_stream");
}
