/*
 * mi_peaks.h -- measurement entry points of libmiqmm.so: the device's own
 * peaks, microbenchmarked on the box rather than read off a spec sheet.
 *
 * The reference measures its chip the same way before it prices any kernel
 * (autotuner/measure/peaks.py:1-7: bandwidth from a read of 1 GB, matrix
 * flops from a large matmul, launch cost from a chain of launches; the best
 * reading is kept, :34-42). These entries are the gfx950 kernels behind that
 * measurement; metal-autotune_amd/measure.py times them with HIP events and
 * bench.py reports the result beside the spec-sheet fractions. They compute
 * nothing a region uses.
 *
 * Conventions as in mi_qmm.h: device pointers, hipStream_t as void*, status
 * codes with mi_last_error().
 */
#ifndef MI_PEAKS_H
#define MI_PEAKS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Dense bf16 MFMA issue rate: `blocks` workgroups of 256 threads, each wave
 * running iters x 16 v_mfma_f32_32x32x16_bf16 (32,768 flops each) over four
 * independent accumulators, so the matrix pipe, not a dependency chain, is
 * the limit. sink: float [blocks * 4] (a checksum per wave, so nothing is
 * optimized away). clk: int64 [blocks * 4 * 2] or NULL; per wave the
 * s_memtime and s_memrealtime (100 MHz) deltas of its loop, whose ratio is
 * the shader clock the MFMAs ran at. */
int mi_peak_mfma_bf16(int blocks, int iters, float *sink, int64_t *clk, void *stream);

/* HBM read rate: every 16-byte word of src[0, bytes) read once by a grid of
 * `blocks` workgroups (each streams one contiguous chunk with non-temporal
 * loads, eight in flight per lane), folded into sink (uint32 [blocks], the
 * xor of the chunk's words). bytes a multiple of 64, src 16-byte aligned. */
int mi_peak_read(const void *src, int64_t bytes, int blocks, uint32_t *sink, void *stream);

/* An empty kernel (one workgroup of 64 threads): the fixed cost of a launch,
 * timed as a chain of launches inside a HIP graph. */
int mi_peak_empty(void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MI_PEAKS_H */
