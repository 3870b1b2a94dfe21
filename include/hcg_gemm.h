/*
 * hcg_gemm.h -- C ABI of the gfx950 (MI355X) backend for the hc tiled
 * matrix-core GEMM.
 *
 * The reference (Hardcode84/5, the `hc` DSL) has no launch ABI: its only
 * executable form of this kernel is the NumPy simulator, reached through
 * `hc.simulator.launch(fn, *args, target=None)` (hc/simulator.py:165-186),
 * and the future compiled entry `CompiledKernel.__call__`
 * (hc/_compile.py:57-62) raises NotImplementedError.  These entry points are
 * what that launch surface binds to on gfx950: plain pointers, sizes and a
 * HIP stream; no framework types.
 *
 * Layouts (all row-major, as bound by the kernel's Buffer annotations
 * `a: Buffer[M, K, f16]`, `b: Buffer[K, N, f16]`, `c: Buffer[M, N, f32]`,
 * examples/amdgpu_gfx11_wmma_matmul.py:306-311):
 *   A: M x K, element (i,k) at A[i*lda + k]
 *   B: K x N, element (k,j) at B[k*ldb + j]
 *   C: M x N float32, element (i,j) at C[i*ldc + j]
 * A and B are 16-bit (fp16 or bf16, selected by `dtype`); accumulation is
 * float32; C is written, never read, and only its M x N elements are
 * touched (hc/simulator.py:1441-1458).
 *
 * Status codes: HCG_OK, HCG_EINVAL (argument rejected before any launch; the
 * Python layer raises LaunchError), HCG_EHIP (a HIP runtime call failed; the
 * text is in hcg_last_error()).  M == 0 or N == 0 is a no-op that launches
 * nothing (hc/simulator.py:175-176); K == 0 writes zeros into C.
 *
 * All launches are asynchronous on `stream` (a hipStream_t; NULL = the
 * null stream).  The entry points are re-entrant; error text is per thread.
 */
#ifndef HCG_GEMM_H
#define HCG_GEMM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HCG_OK 0
#define HCG_EINVAL 1
#define HCG_EHIP 2

/* Operand element types. */
#define HCG_F16 0
#define HCG_BF16 1

/* Kernel selection for hcg_gemm_algo. */
#define HCG_ALGO_AUTO 0
#define HCG_ALGO_TILED 1  /* LDS-tiled MFMA kernel, tile shape and K split picked by shape (compute-bound) */
#define HCG_ALGO_SKINNY 2 /* split-K streaming kernel for M <= 128 (HBM-bound shapes; any layout) */
#define HCG_ALGO_GENERIC 3 /* pointer-based tiled kernel: any alignment and size (fallback) */
/* The LDS-tiled kernel with a fixed output tile shape (rows x columns), never split along K. */
#define HCG_ALGO_TILED_256x256 4
#define HCG_ALGO_TILED_256x192 5
#define HCG_ALGO_TILED_128x256 6
#define HCG_ALGO_TILED_128x128 7
#define HCG_ALGO_TILED_256x64 8
/* Streaming kernel for N <= 64 (A streamed once in 256-byte row pieces, K split to fill the
 * chip; HBM-bound shapes).  Any layout: A and B read in place by DMA at any row alignment; an
 * operand whose last 16-byte piece cannot be read safely goes through registers (A) or is
 * repacked (B). */
#define HCG_ALGO_NARROW 9

/* Idempotent one-time set-up (device properties).  Replaces the reference's
 * once-per-process registration, lib/CAPI/HC.cpp:22-29.  Optional: every
 * other entry point calls it. */
int hcg_init(void);

/* C = A @ B, the launch of `tiled_gfx11_wmma_matmul`
 * (examples/amdgpu_gfx11_wmma_matmul.py:301-326) through
 * hc.simulator.launch (hc/simulator.py:165-186).  Picks the kernel by shape;
 * a few rows or columns past a multiple of 256 may run on a streaming
 * kernel beside the tiled one (two launches on the stream). */
int hcg_gemm(int dtype, const void* A, int64_t lda, const void* B, int64_t ldb, float* C,
             int64_t ldc, int64_t M, int64_t N, int64_t K, void* stream);

/* Same as hcg_gemm with an explicit kernel choice (HCG_ALGO_*).  Used by
 * tests and the benchmark to exercise each kernel; HCG_ALGO_SKINNY rejects
 * M > 128, and M > 16 with a B of fewer than 8 elements (or K past 2^23),
 * and HCG_ALGO_NARROW rejects N > 64, with HCG_EINVAL. */
int hcg_gemm_algo(int algo, int dtype, const void* A, int64_t lda, const void* B, int64_t ldb,
                  float* C, int64_t ldc, int64_t M, int64_t N, int64_t K, void* stream);

/* Bytes of the per-GPU scratch array behind hcg_gemm_noalloc. */
#define HCG_NOALLOC_SCRATCH_BYTES (32u << 20)

/* Same as hcg_gemm, allocating nothing: no hipMalloc, hipFree or allocating
 * library call on any path, for callers that cannot allocate (code under
 * HIP graph capture, tight serving loops, harnesses that forbid it).  No
 * counterpart in the reference, which has no launch ABI.  Scratch
 * (split-K partials, and operands repacked when they cannot be read in
 * place) comes from one static device array of HCG_NOALLOC_SCRATCH_BYTES
 * per GPU, held from the library's first use on that GPU until the process
 * ends; K splits are limited to what fits, and a call that still needs more
 * (a large operand that must be repacked) fails with HCG_EINVAL before any
 * launch.  Every
 * call on one GPU shares that array: calls that overlap in time on one GPU
 * (other streams, other host threads, concurrent graph replays) race, so
 * the caller must order them.  Nothing in the array needs to start at zero:
 * every byte a call reads was written earlier in the same call. */
int hcg_gemm_noalloc(int dtype, const void* A, int64_t lda, const void* B, int64_t ldb, float* C,
                     int64_t ldc, int64_t M, int64_t N, int64_t K, void* stream);

/* Text of the calling thread's last error ("" if none). */
const char* hcg_last_error(void);

/* ABI version of this library (major * 100 + minor). */
int hcg_version(void);

/* Whether the DMA kernels read a 16-bit rows x cols operand at `base` (row
 * stride ld elements) in place: 1 in place, 0 copied first into zero-padded
 * rows, -1 for bad arguments (text in hcg_last_error()).  Rows that are 16-byte
 * aligned are read in place; other rows are read in 16-byte pieces, which
 * reach up to 30 bytes past the last element, so they are read in place only
 * when those bytes lie in the last element's 4 KB page, or inside the
 * operand's device allocation and mapped.  Queries the HIP runtime about the
 * pointer and launches nothing.  No counterpart in the reference (which has
 * no device memory); for tests and diagnostics. */
int hcg_operand_in_place(const void* base, int64_t rows, int64_t cols, int64_t ld);

#ifdef __cplusplus
}
#endif

#endif /* HCG_GEMM_H */
