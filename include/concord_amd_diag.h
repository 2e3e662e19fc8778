/* concord_amd_diag.h -- measurement entry points of libconcord_amd.so.
 *
 * They have no counterpart in the reference: they exercise the data path the
 * GEMM kernels use, for the roofline and counter figures of this build.
 * Same conventions as concord_amd.h (device pointers, the caller's stream,
 * 0 on success, concord_last_error()). */
#ifndef CONCORD_AMD_DIAG_H
#define CONCORD_AMD_DIAG_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dst = src, `bytes` (a multiple of 16384, below 2^31; 16-byte aligned
 * pointers) read by LDS-DMA loads (buffer_load_dwordx4 ... lds) and written
 * from LDS: the counter calibration of the LDS-DMA load path. */
int concord_diag_dma_copy(const void* src, void* dst, size_t bytes, void* stream);

/* `blocks` workgroups each read the region of their XCD (workgroup w runs on
 * XCD w mod 8; region x = src bytes [x region_bytes, (x + 1) region_bytes),
 * so src holds 8 regions) `reps` times in 16 KB chunks with `depth` (2, 4
 * or 8) chunks in flight, by LDS-DMA (lds_dma != 0) or by 16-byte loads into
 * registers; sink: one word, written only to keep the register loads. */
int concord_diag_l2_stream(const void* src, size_t region_bytes, int reps, int blocks, int depth, int lds_dma,
                           uint32_t* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif
