/*
 * hcg_mfma.h -- C ABI of one gfx950 matrix-core step executed for a single
 * 64-lane wavefront: the device side of the `mfma_gfx950` / `mfma16_gfx950`
 * intrinsics' `amdgpu-gfx950` lowering.
 *
 * In the reference an intrinsic's `.lower(target=...)` callback replaces
 * the intrinsic's fallback body for that target and must keep its
 * observable semantics -- result type, logical shape, masking and layout
 * (hc/core.py:282-307, doc/langref.md:838-899; the gfx11 example lowering
 * examples/amdgpu_gfx11_wmma_matmul.py:200-228 emits one `amdgpu.wmma` op per
 * lane).  The reference emits MLIR and never executes the op; this entry
 * point executes the instruction that op names, so the lane contract the
 * fallback body states can be checked against the hardware.
 *
 * One call runs one wave (64 lanes) of
 *   m x n x k = 32 x 32 x 16: v_mfma_f32_32x32x16_{f16,bf16}, 16 floats per lane
 *   m x n x k = 16 x 16 x 32: v_mfma_f32_16x16x32_{f16,bf16},  4 floats per lane
 * on an m x k A tile and a k x n B tile (16-bit elements, row-major, dense:
 * element (i, kk) of A at A[i*k + kk], (kk, j) of B at B[kk*n + j]).  Masks
 * are bytes in the same layout, nonzero = active; an inactive element counts
 * as +0 (the fallback's with_inactive(value=0)); NULL = all active.
 * acc_in and acc_out hold the accumulators lane-major: lane l's register r
 * at [l*R + r], R = m*n/64.  Register r of lane l is output element
 *   32x32x16: row 8*(r/4) + 4*(l/32) + r%4, column l%32
 *   16x16x32: row 4*(l/16) + r,             column l%16
 * and after the call holds acc_in's value plus the sum over kk of
 * A[row][kk] * B[kk][column], products exact and accumulated in float32.
 *
 * All pointers are device pointers; the call is asynchronous on `stream`.
 * Status codes as in hcg_gemm.h.
 */
#ifndef HCG_MFMA_H
#define HCG_MFMA_H

#include <stdint.h>

#include "hcg_gemm.h"

#ifdef __cplusplus
extern "C" {
#endif

/* One matrix-core step of one wave: the op recorded from the intrinsic's
 * `amdgpu-gfx950` lowering callback (`rocdl.mfma.f32.32x32x16` or
 * `rocdl.mfma.f32.16x16x32`, examples/amdgpu_gfx11_wmma_matmul.py:200-228 is
 * the reference's gfx11 counterpart), executed.  (m, n, k) must be
 * (32, 32, 16) or (16, 16, 32); dtype HCG_F16 or HCG_BF16. */
int hcg_mfma_step(int dtype, int m, int n, int k, const void* A, const void* B, const uint8_t* a_mask,
                  const uint8_t* b_mask, const float* acc_in, float* acc_out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HCG_MFMA_H */
