/*
 * hcg_probe.h -- hardware ceiling probes for MI355X (gfx950), the
 * measurement side of the GEMM library (libhcg_probe.so, built beside
 * libhcg_gfx950.so).  Not part of the GEMM ABI: the reference has no
 * counterpart.  bench.py runs them on the box it measures, so that each
 * roofline fraction can be read against what the same board sustains:
 *
 *   hcg_probe_mfma   -- pure MFMA issue (v_mfma_f32_32x32x16_{f16,bf16})
 *                       on every CU, with the shader clock it ran at;
 *   hcg_probe_mfma16 -- the same flops as v_mfma_f32_16x16x32_{f16,bf16};
 *   hcg_probe_read   -- streaming HBM read of a 2-D region in strips
 *                       (the access pattern of the streaming GEMM kernels)
 *                       or contiguously;
 *   hcg_probe_write  -- streaming HBM write (the GEMM epilogue's pattern).
 *
 * All launches are asynchronous on `stream`; time them with events.
 * Status codes as in hcg_gemm.h (0 ok, 1 invalid argument, 2 HIP error);
 * hcg_probe_last_error() holds the text.
 */
#ifndef HCG_PROBE_H
#define HCG_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* `blocks` workgroups of 256 threads (4 waves); each wave issues `iters`
 * (a multiple of 4) rounds of 8 independent 32x32x16 MFMAs (dtype 0 fp16, 1 bf16) on
 * pseudo-random operands in [-1, 1) -- 2 * 32 * 32 * 16 * 8 * iters flops
 * per wave.  `sink` (blocks * 256 floats) receives the accumulators' sums;
 * `clocks` (2 * blocks uint64) receives, per workgroup, the shader-clock
 * cycles (s_memtime) and the 100 MHz real-time ticks (s_memrealtime) its
 * first wave spent in the loop. */
int hcg_probe_mfma(int dtype, int iters, int blocks, float* sink, uint64_t* clocks, void* stream);

/* As hcg_probe_mfma with 16 independent 16x16x32 MFMAs per round (the same
 * 2 * 16 * 16 * 32 * 16 * iters flops per wave as 8 of 32x32x16). */
int hcg_probe_mfma16(int dtype, int iters, int blocks, float* sink, uint64_t* clocks, void* stream);

/* Reads `rows` rows of `pitch` bytes from `src`: the row is cut into
 * strips of `width` bytes (16 <= width <= 4096, a power of two dividing
 * `pitch`), and each strip's rows into `row_splits` runs; one 256-thread
 * workgroup per (strip, run), each thread with `unroll` (1, 2, 4, 8 or 16)
 * 16-byte loads in flight.  width == pitch reads contiguous runs of rows.
 * `sink` (one uint32 per thread) receives an XOR of what was read. */
int hcg_probe_read(const void* src, int64_t pitch, int width, int64_t rows, int row_splits, int unroll,
                   uint32_t* sink, void* stream);

/* Writes `bytes` (a multiple of 16) to `dst` with 16-byte stores from
 * `blocks` workgroups of 256 threads in a grid-stride loop; `nontemporal`
 * selects non-temporal stores. */
int hcg_probe_write(void* dst, int64_t bytes, int blocks, int nontemporal, void* stream);

/* Text of the calling thread's last probe error ("" if none). */
const char* hcg_probe_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* HCG_PROBE_H */
