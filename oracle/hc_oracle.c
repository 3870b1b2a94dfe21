/*
 * CPU oracle for the hc tiled matrix-core GEMM -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker or the timed CPU baseline. The
 * product path (5_amd/) never links, loads or calls it.
 *
 * What it restates.  The reference executes the GEMM only in its NumPy
 * simulator.  Per workgroup and K-step, the intrinsic fallback body of
 * `wmma_gfx11` (examples/amdgpu_gfx11_wmma_matmul.py:177-190) does
 *
 *     accum = np.float32(acc_frag[index])
 *     for k_idx in range(16):
 *         accum += np.float32(a_tile[row, k_idx]) * np.float32(b_tile[k_idx, col])
 *
 * on tiles whose out-of-bounds lanes were replaced by +0
 * (`with_inactive(value=0)`, :178-179; the masked tile load is
 * hc/simulator.py:1338-1357).  The accumulator starts from `vzeros`
 * (:249-256) and is threaded through the K loop (:315-324) in ascending k0,
 * so every output element is one strictly sequential float32 fold
 *
 *     C[i][j] = fold_{k=0..K-1}  s <- RN32(s + RN32(a_ik * b_kj)),  s0 = +0
 *
 * An fp16 or bf16 product is exact in float32 (11x11 resp. 8x8 significand
 * bits <= 24; the smallest fp16 subnormal product 2^-48 is a normal float),
 * so RN32(a*b) == a*b, and a fused multiply-add would give the same bits.
 * Masked K-tail terms add +0 * x = +-0, which leaves s unchanged except for a
 * -0 + +0 edge that cannot arise because s0 = +0.  Only in-bounds C is
 * written (hc/simulator.py:1441-1458).
 *
 * Loop order: the k loop is outermost per (row block, column chunk) and the
 * column loop innermost, so each C[i][j] still sees its terms in ascending k;
 * vectorising over j changes nothing per element.
 *
 * Conversions are this file's own: fp16 -> float through a 65536-entry table
 * built from the IEEE-754 binary16 definition, bf16 -> float by a 16-bit
 * shift.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

enum { HCO_F16 = 0, HCO_BF16 = 1 };

static float g_f16_table[65536];
static int g_f16_ready = 0;

/* binary16: 1 sign, 5 exponent (bias 15), 10 fraction bits. */
static float f16_bits_to_float(uint16_t h) {
  const int sign = (h >> 15) & 1;
  const int exp = (h >> 10) & 0x1f;
  const int frac = h & 0x3ff;
  float v;
  if (exp == 0) {
    v = ldexpf((float)frac, -24); /* subnormal: frac * 2^-24 */
  } else if (exp == 31) {
    v = frac ? NAN : INFINITY;
  } else {
    v = ldexpf((float)(frac | 0x400), exp - 25); /* (1.f) * 2^(exp-15) */
  }
  return sign ? -v : v;
}

static void ensure_f16_table(void) {
  if (g_f16_ready) return;
  for (uint32_t h = 0; h < 65536u; ++h) g_f16_table[h] = f16_bits_to_float((uint16_t)h);
  g_f16_ready = 1;
}

static inline float bf16_bits_to_float(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, sizeof f);
  return f;
}

static inline float to_f32(int dtype, uint16_t h) {
  return dtype == HCO_BF16 ? bf16_bits_to_float(h) : g_f16_table[h];
}

/* Exposed for the oracle's own tests: converts n 16-bit patterns. */
void hco_to_float(int dtype, const uint16_t* src, float* dst, int64_t n) {
  ensure_f16_table();
  for (int64_t i = 0; i < n; ++i) dst[i] = to_f32(dtype, src[i]);
}

#define HCO_ROWS 4
#define HCO_COLS 256

/*
 * C[r][j] for the rows listed in `rows` (nrows entries, or rows 0..nrows-1
 * when rows == NULL) and all columns j < N.  A is M x K (row stride lda), B is
 * K x N (row stride ldb), C rows are written at C + r_out * ldc where r_out is
 * the position in `rows` when compact != 0, else the row index itself.
 */
static void gemm_rows(int dtype, const uint16_t* A, int64_t lda, const float* Bf,
                      int64_t N, int64_t K, const int64_t* rows, int64_t nrows,
                      float* C, int64_t ldc, int compact, int nthreads) {
  const int64_t nblk = (nrows + HCO_ROWS - 1) / HCO_ROWS;
  const int64_t ncc = (N + HCO_COLS - 1) / HCO_COLS;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) collapse(2) num_threads(nthreads)
#endif
  for (int64_t rb = 0; rb < nblk; ++rb) {
    for (int64_t cc = 0; cc < ncc; ++cc) {
      float acc[HCO_ROWS][HCO_COLS];
      int64_t ridx[HCO_ROWS];
      const int64_t r0 = rb * HCO_ROWS;
      const int nr = (int)((nrows - r0) < HCO_ROWS ? (nrows - r0) : HCO_ROWS);
      const int64_t j0 = cc * HCO_COLS;
      const int nc = (int)((N - j0) < HCO_COLS ? (N - j0) : HCO_COLS);
      for (int r = 0; r < nr; ++r) {
        ridx[r] = rows ? rows[r0 + r] : (r0 + r);
        for (int j = 0; j < nc; ++j) acc[r][j] = 0.0f;
      }
      for (int64_t k = 0; k < K; ++k) {
        const float* brow = Bf + k * N + j0;
        for (int r = 0; r < nr; ++r) {
          const float a = to_f32(dtype, A[ridx[r] * lda + k]);
          float* s = acc[r];
          for (int j = 0; j < nc; ++j) s[j] = s[j] + a * brow[j];
        }
      }
      for (int r = 0; r < nr; ++r) {
        float* crow = C + (compact ? (r0 + r) : ridx[r]) * ldc + j0;
        memcpy(crow, acc[r], (size_t)nc * sizeof(float));
      }
    }
  }
  (void)nthreads;
}

static float* widen_b(int dtype, const uint16_t* B, int64_t ldb, int64_t K, int64_t N) {
  float* Bf = (float*)malloc((size_t)(K > 0 ? K : 1) * (size_t)(N > 0 ? N : 1) * sizeof(float));
  if (!Bf) return NULL;
  for (int64_t k = 0; k < K; ++k)
    for (int64_t j = 0; j < N; ++j) Bf[k * N + j] = to_f32(dtype, B[k * ldb + j]);
  return Bf;
}

/* Full GEMM: C (M x N, row stride ldc) = sequential-fold(A @ B).  Returns 0 on
 * success, -1 on bad arguments, -2 when the float copy of B cannot be made. */
int hco_gemm(int dtype, const uint16_t* A, int64_t lda, const uint16_t* B, int64_t ldb,
             float* C, int64_t ldc, int64_t M, int64_t N, int64_t K, int nthreads) {
  if (M < 0 || N < 0 || K < 0 || (dtype != HCO_F16 && dtype != HCO_BF16)) return -1;
  if (M == 0 || N == 0) return 0;
  if (lda < K || ldb < N || ldc < N) return -1;
  ensure_f16_table();
  float* Bf = widen_b(dtype, B, ldb, K, N);
  if (!Bf) return -2;
  gemm_rows(dtype, A, lda, Bf, N, K, NULL, M, C, ldc, 0, nthreads < 1 ? 1 : nthreads);
  free(Bf);
  return 0;
}

/* Selected rows only: out (nrows x N, row stride N) gets C[rows[i]][:].  Used
 * to check full-size shapes on a sample of rows and as the bounded CPU
 * baseline. */
int hco_gemm_rows(int dtype, const uint16_t* A, int64_t lda, const uint16_t* B, int64_t ldb,
                  int64_t M, int64_t N, int64_t K, const int64_t* rows, int64_t nrows,
                  float* out, int nthreads) {
  if (M < 0 || N < 0 || K < 0 || nrows < 0 || (dtype != HCO_F16 && dtype != HCO_BF16)) return -1;
  for (int64_t i = 0; i < nrows; ++i)
    if (rows[i] < 0 || rows[i] >= M) return -1;
  if (nrows == 0 || N == 0) return 0;
  if (lda < K || ldb < N) return -1;
  ensure_f16_table();
  float* Bf = widen_b(dtype, B, ldb, K, N);
  if (!Bf) return -2;
  gemm_rows(dtype, A, lda, Bf, N, K, rows, nrows, out, N, 1, nthreads < 1 ? 1 : nthreads);
  free(Bf);
  return 0;
}

int hco_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
