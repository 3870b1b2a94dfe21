// hcg_torch.cpp -- the device-tensor binding of hcg_gemm_algo as a Python
// extension (host code only): the checks and stride rules of the Python
// wrapper hc.gfx950.gemm, made on the tensors' C++ attributes, and the
// current HIP stream of the device, so that a small GEMM costs about the
// host time of the launch itself.  It handles the common case only (three
// device tensors on the current device, fp16 or bf16 operands, a float32
// C that can be written in place) and returns -1 for anything else, which
// the Python wrapper then takes through its general path; otherwise it
// returns hcg_gemm_algo's status (the message is hcg_last_error's).

#include <torch/extension.h>
#include <c10/hip/HIPFunctions.h>
#include <c10/hip/HIPStream.h>

#include <algorithm>

#include "hcg_gemm.h"

namespace {

int64_t gemm(const at::Tensor& a, const at::Tensor& b, const at::Tensor& c, int64_t algo) {
  if (a.dim() != 2 || b.dim() != 2 || c.dim() != 2) return -1;
  if (!a.is_cuda() || !b.is_cuda() || !c.is_cuda()) return -1;
  const c10::DeviceIndex dev = a.get_device();
  if (b.get_device() != dev || c.get_device() != dev || c10::hip::current_device() != dev) return -1;
  const at::ScalarType st = a.scalar_type();
  int dtype;
  if (st == at::kHalf)
    dtype = HCG_F16;
  else if (st == at::kBFloat16)
    dtype = HCG_BF16;
  else
    return -1;
  if (b.scalar_type() != st || c.scalar_type() != at::kFloat) return -1;
  const int64_t m = a.size(0), k = a.size(1), n = b.size(1);
  if (b.size(0) != k || c.size(0) != m || c.size(1) != n || m == 0 || n == 0) return -1;
  // Row-major views only (the Python wrapper copies other layouts first); a
  // one-row matrix's row stride is unused, so the smallest legal one is passed.
  if (k > 0 && (a.stride(1) != 1 || (m > 1 && a.stride(0) < k))) return -1;
  if (k > 0 && (b.stride(1) != 1 || (k > 1 && b.stride(0) < n))) return -1;
  if (!(c.stride(1) == 1 || n == 1) || !(m == 1 || c.stride(0) >= n)) return -1;
  const int64_t lda = m > 1 ? std::max<int64_t>(a.stride(0), k) : std::max<int64_t>(k, 1);
  const int64_t ldb = k > 1 ? std::max<int64_t>(b.stride(0), n) : std::max<int64_t>(n, 1);
  const int64_t ldc = m > 1 ? std::max<int64_t>(c.stride(0), n) : std::max<int64_t>(n, 1);
  hipStream_t stream = c10::hip::getCurrentHIPStream(dev).stream();
  return hcg_gemm_algo((int)algo, dtype, a.data_ptr(), lda, b.data_ptr(), ldb, static_cast<float*>(c.data_ptr()),
                       ldc, m, n, k, stream);
}

}  // namespace

PYBIND11_MODULE(_hcg_torch, mod) {
  mod.def("gemm", &gemm, "C = A @ B on the current HIP stream; -1 when the case is not handled here");
}
