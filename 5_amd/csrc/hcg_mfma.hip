// hcg_mfma.hip -- one wave of one gfx950 matrix-core instruction, executed
// on a masked A tile, a masked B tile and per-lane accumulators (the C ABI of
// include/hcg_mfma.h).
//
// This is what the `amdgpu-gfx950` lowering of the DSL's mfma intrinsics
// names (hc/core.py:282-307: a lowering replaces the fallback body on its
// target): the Python side records the op the lowering callback creates and
// runs it here, so each lane's result can be compared with the fallback
// body's statement of that lane (5_amd/hc/gfx950/kernels.py).
//
// Operand fragments: lane l holds 8 K-contiguous elements of A row l % m and
// of B column l % n, starting at k = 8 * (l / m); both operands use the same
// lane -> k assignment, so each output element gets every product once
// whatever order the hardware sums them in.  Output registers follow the
// CDNA accumulator layout stated in include/hcg_mfma.h.

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "hcg_mfma.h"
#include "hcg_runtime.h"

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

struct StepArgs {
  const uint16_t* A;
  const uint16_t* B;
  const uint8_t* am;
  const uint8_t* bm;
  const float* acc_in;
  float* acc_out;
};

// M x N x K with 8 K values per lane: K / 8 lane groups of M lanes.
template <int DT, int M, int N, int K>
__global__ __launch_bounds__(64) void mfma_step_kernel(StepArgs g) {
  static_assert(M * (K / 8) == 64 && M == N, "one fragment of 8 k per lane");
  constexpr int R = M * N / 64;
  const int lane = threadIdx.x;
  const int row = lane % M, col = lane % N, k0 = 8 * (lane / M);
  u16x8 a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int ia = row * K + k0 + i, ib = (k0 + i) * N + col;
    a[i] = (g.am == nullptr || g.am[ia]) ? g.A[ia] : uint16_t(0);
    b[i] = (g.bm == nullptr || g.bm[ib]) ? g.B[ib] : uint16_t(0);
  }
  if constexpr (R == 16) {
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = g.acc_in[lane * R + r];
    if constexpr (DT == HCG_F16)
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), acc,
                                                   0, 0, 0);
    else
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                    acc, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < R; ++r) g.acc_out[lane * R + r] = acc[r];
  } else {
    f32x4 acc;
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = g.acc_in[lane * R + r];
    if constexpr (DT == HCG_F16)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), acc,
                                                   0, 0, 0);
    else
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                    acc, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < R; ++r) g.acc_out[lane * R + r] = acc[r];
  }
}

}  // namespace

extern "C" {

int hcg_mfma_step(int dtype, int m, int n, int k, const void* A, const void* B, const uint8_t* a_mask,
                  const uint8_t* b_mask, const float* acc_in, float* acc_out, void* stream) {
  if (dtype != HCG_F16 && dtype != HCG_BF16)
    return hcg::set_error(HCG_EINVAL, "hcg_mfma_step: dtype must be HCG_F16 (0) or HCG_BF16 (1), got %d", dtype);
  const bool big = m == 32 && n == 32 && k == 16;
  const bool small = m == 16 && n == 16 && k == 32;
  if (!big && !small)
    return hcg::set_error(HCG_EINVAL,
                          "hcg_mfma_step: no gfx950 matrix-core instruction for m x n x k = %d x %d x %d "
                          "(32 x 32 x 16 and 16 x 16 x 32 are implemented)",
                          m, n, k);
  if (A == nullptr || B == nullptr || acc_in == nullptr || acc_out == nullptr)
    return hcg::set_error(HCG_EINVAL, "hcg_mfma_step: A, B, acc_in and acc_out must not be NULL");
  StepArgs g{static_cast<const uint16_t*>(A), static_cast<const uint16_t*>(B), a_mask, b_mask, acc_in, acc_out};
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (big) {
    if (dtype == HCG_F16)
      mfma_step_kernel<HCG_F16, 32, 32, 16><<<1, 64, 0, s>>>(g);
    else
      mfma_step_kernel<HCG_BF16, 32, 32, 16><<<1, 64, 0, s>>>(g);
  } else {
    if (dtype == HCG_F16)
      mfma_step_kernel<HCG_F16, 16, 16, 32><<<1, 64, 0, s>>>(g);
    else
      mfma_step_kernel<HCG_BF16, 16, 16, 32><<<1, 64, 0, s>>>(g);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return hcg::set_error(HCG_EHIP, "mfma_step_kernel launch failed: %s", hipGetErrorString(e));
  hcg::t_last_error.clear();
  return HCG_OK;
}

}  // extern "C"
