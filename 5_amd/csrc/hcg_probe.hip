// hcg_probe.hip -- hardware ceiling probes for MI355X (gfx950): pure MFMA
// issue with the shader clock it runs at, and streaming HBM reads and
// writes in the access patterns the GEMM kernels use.  The C ABI is in
// include/hcg_probe.h; bench.py runs these on the box it measures.

#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include <string>

#include "hcg_probe.h"

namespace {

thread_local std::string t_probe_error;

int probe_error(int code, const char* fmt, ...) {
  char buf[256];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  t_probe_error = buf;
  return code;
}

#define PROBE_HIP_CHECK(expr)                                                             \
  do {                                                                                    \
    hipError_t _e = (expr);                                                               \
    if (_e != hipSuccess) return probe_error(2, "%s failed: %s", #expr, hipGetErrorString(_e)); \
  } while (0)

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// A 32-bit mix (splitmix-style) for reproducible operand bits.
__device__ __forceinline__ uint32_t mix(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

// Two 16-bit values in [-1, 1) packed in a word: fp16 or bf16 bit patterns
// of a sign, an exponent in [-8, -1] and random mantissa bits.
template <int DT>
__device__ __forceinline__ uint32_t random_pair(uint32_t h) {
  uint32_t out = 0;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const uint32_t r = (h >> (16 * half)) & 0xffffu;
    const uint32_t sign = (r >> 15) & 1u;
    const uint32_t e = 7u + ((r >> 12) & 7u);  // unbiased -8 .. -1
    uint32_t bits;
    if constexpr (DT == 0) {
      bits = (sign << 15) | (e << 10) | (mix(r) & 0x3ffu);                  // fp16 bias 15
    } else {
      bits = (sign << 15) | ((e + 112u) << 7) | (mix(r) & 0x7fu);            // bf16 bias 127
    }
    out |= bits << (16 * half);
  }
  return out;
}

template <int DT>
__device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (DT == 0) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                  c, 0, 0, 0);
  }
}

// Each wave: 8 independent accumulator chains over 4 A and 4 B operand
// fragments, so every MFMA issues without waiting on its predecessor.
template <int DT>
__global__ __launch_bounds__(256) void probe_mfma_kernel(int iters, float* sink, uint64_t* clocks) {
  const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
  u32x4 fa[4], fb[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      fa[j][w] = random_pair<DT>(mix(gid * 32u + j * 4u + w));
      fb[j][w] = random_pair<DT>(mix(gid * 32u + 16u + j * 4u + w + 0x9e3779b9u));
    }
  }
  f32x16 acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = f32x16{};
  const uint64_t t0 = __builtin_amdgcn_s_memtime();
  const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
  // Four rounds (32 MFMAs) per trip, so the loop's branch (several cycles
  // per taken branch) costs little; iters is a multiple of 4.
  for (int i = 0; i < iters; i += 4) {
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = mfma<DT>(fa[j & 3], fb[(j + (j >> 2)) & 3], acc[j]);
  }
  const uint64_t t1 = __builtin_amdgcn_s_memtime();
  const uint64_t r1 = __builtin_amdgcn_s_memrealtime();
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) s += acc[j][r];
  sink[gid] = s;
  if (threadIdx.x == 0) {
    clocks[2 * blockIdx.x] = t1 - t0;
    clocks[2 * blockIdx.x + 1] = r1 - r0;
  }
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int DT>
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (DT == 0) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                  c, 0, 0, 0);
  }
}

// The same flops as probe_mfma_kernel per round, as 16 independent chains
// of the 16x16x32 instruction (the streaming kernels' MFMA shape).
template <int DT>
__global__ __launch_bounds__(256) void probe_mfma16_kernel(int iters, float* sink, uint64_t* clocks) {
  const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
  u32x4 fa[4], fb[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      fa[j][w] = random_pair<DT>(mix(gid * 32u + j * 4u + w));
      fb[j][w] = random_pair<DT>(mix(gid * 32u + 16u + j * 4u + w + 0x9e3779b9u));
    }
  }
  f32x4 acc[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = f32x4{};
  const uint64_t t0 = __builtin_amdgcn_s_memtime();
  const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
  for (int i = 0; i < iters; i += 4) {
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[j] = mfma16<DT>(fa[j & 3], fb[(j + (j >> 2)) & 3], acc[j]);
  }
  const uint64_t t1 = __builtin_amdgcn_s_memtime();
  const uint64_t r1 = __builtin_amdgcn_s_memrealtime();
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 16; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) s += acc[j][r];
  sink[gid] = s;
  if (threadIdx.x == 0) {
    clocks[2 * blockIdx.x] = t1 - t0;
    clocks[2 * blockIdx.x + 1] = r1 - r0;
  }
}

// Strip read: workgroup w reads strip w % nstrips over run w / nstrips of
// the rows; thread t covers 16-byte column t % width16 of rows t / width16
// + k * (256 / width16) of each group of U row steps.
template <int U>
__global__ __launch_bounds__(256) void probe_read_kernel(const u32x4* __restrict__ src, int64_t pitch16,
                                                         int width16, int64_t rows, int64_t run_rows,
                                                         int nstrips, uint32_t* sink) {
  const int strip = blockIdx.x % nstrips;
  const int64_t run = blockIdx.x / nstrips;
  const int tid = threadIdx.x;
  const int col = tid % width16;
  const int rows_per_step = 256 / width16;
  const int64_t r_begin = run * run_rows;
  const int64_t r_end = r_begin + run_rows < rows ? r_begin + run_rows : rows;
  const u32x4* base = src + (int64_t)strip * width16 + col;
  uint32_t x = 0;
  int64_t r = r_begin + tid / width16;
  for (; r + (int64_t)(U - 1) * rows_per_step < r_end; r += (int64_t)U * rows_per_step) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = base[(r + (int64_t)u * rows_per_step) * pitch16];
#pragma unroll
    for (int u = 0; u < U; ++u) x ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  for (; r < r_end; r += rows_per_step) {
    const u32x4 v = base[r * pitch16];
    x ^= v[0] ^ v[1] ^ v[2] ^ v[3];
  }
  sink[blockIdx.x * 256 + tid] = x;
}

template <bool NT>
__global__ __launch_bounds__(256) void probe_write_kernel(u32x4* dst, int64_t n16) {
  const u32x4 v = {blockIdx.x, threadIdx.x, 0x5a5a5a5au, 1u};
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (int64_t)gridDim.x * 256) {
    if constexpr (NT)
      __builtin_nontemporal_store(v, dst + i);
    else
      dst[i] = v;
  }
}

}  // namespace

extern "C" {

int hcg_probe_mfma(int dtype, int iters, int blocks, float* sink, uint64_t* clocks, void* stream) {
  if (dtype != 0 && dtype != 1) return probe_error(1, "dtype must be 0 (fp16) or 1 (bf16), got %d", dtype);
  if (iters <= 0 || blocks <= 0 || iters % 4 != 0)
    return probe_error(1, "iters must be a positive multiple of 4 and blocks positive");
  if (!sink || !clocks) return probe_error(1, "sink or clocks is NULL");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == 0)
    probe_mfma_kernel<0><<<blocks, 256, 0, s>>>(iters, sink, clocks);
  else
    probe_mfma_kernel<1><<<blocks, 256, 0, s>>>(iters, sink, clocks);
  PROBE_HIP_CHECK(hipGetLastError());
  t_probe_error.clear();
  return 0;
}

int hcg_probe_mfma16(int dtype, int iters, int blocks, float* sink, uint64_t* clocks, void* stream) {
  if (dtype != 0 && dtype != 1) return probe_error(1, "dtype must be 0 (fp16) or 1 (bf16), got %d", dtype);
  if (iters <= 0 || blocks <= 0 || iters % 4 != 0)
    return probe_error(1, "iters must be a positive multiple of 4 and blocks positive");
  if (!sink || !clocks) return probe_error(1, "sink or clocks is NULL");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == 0)
    probe_mfma16_kernel<0><<<blocks, 256, 0, s>>>(iters, sink, clocks);
  else
    probe_mfma16_kernel<1><<<blocks, 256, 0, s>>>(iters, sink, clocks);
  PROBE_HIP_CHECK(hipGetLastError());
  t_probe_error.clear();
  return 0;
}

int hcg_probe_read(const void* src, int64_t pitch, int width, int64_t rows, int row_splits, int unroll,
                   uint32_t* sink, void* stream) {
  if (!src || !sink) return probe_error(1, "src or sink is NULL");
  if (width < 16 || width > 4096 || (width & (width - 1)) != 0 || pitch % width != 0 || pitch <= 0)
    return probe_error(1, "width must be a power of two in [16, 4096] dividing pitch");
  if (reinterpret_cast<uintptr_t>(src) % 16 != 0) return probe_error(1, "src must be 16-byte aligned");
  if (rows <= 0 || row_splits <= 0 || row_splits > rows) return probe_error(1, "need 0 < row_splits <= rows");
  const int width16 = width / 16;
  const int64_t nstrips = pitch / width;
  if (width16 > 256) return probe_error(1, "width above 4096 bytes");
  const int64_t grid = nstrips * row_splits;
  if (grid > 0x7fffffff) return probe_error(1, "too many workgroups");
  const int64_t run_rows = (rows + row_splits - 1) / row_splits;
  const u32x4* p = static_cast<const u32x4*>(src);
  const int64_t pitch16 = pitch / 16;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // A width of 4096 bytes: one row per 256 threads, so "rows per step" is 1.
  switch (unroll) {
    case 1: probe_read_kernel<1><<<(unsigned)grid, 256, 0, s>>>(p, pitch16, width16, rows, run_rows, (int)nstrips, sink); break;
    case 2: probe_read_kernel<2><<<(unsigned)grid, 256, 0, s>>>(p, pitch16, width16, rows, run_rows, (int)nstrips, sink); break;
    case 4: probe_read_kernel<4><<<(unsigned)grid, 256, 0, s>>>(p, pitch16, width16, rows, run_rows, (int)nstrips, sink); break;
    case 8: probe_read_kernel<8><<<(unsigned)grid, 256, 0, s>>>(p, pitch16, width16, rows, run_rows, (int)nstrips, sink); break;
    case 16: probe_read_kernel<16><<<(unsigned)grid, 256, 0, s>>>(p, pitch16, width16, rows, run_rows, (int)nstrips, sink); break;
    default: return probe_error(1, "unroll must be 1, 2, 4, 8 or 16");
  }
  PROBE_HIP_CHECK(hipGetLastError());
  t_probe_error.clear();
  return 0;
}

int hcg_probe_write(void* dst, int64_t bytes, int blocks, int nontemporal, void* stream) {
  if (!dst) return probe_error(1, "dst is NULL");
  if (bytes <= 0 || bytes % 16 != 0 || reinterpret_cast<uintptr_t>(dst) % 16 != 0)
    return probe_error(1, "bytes must be a positive multiple of 16 and dst 16-byte aligned");
  if (blocks <= 0) return probe_error(1, "blocks must be positive");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (nontemporal)
    probe_write_kernel<true><<<blocks, 256, 0, s>>>(static_cast<u32x4*>(dst), bytes / 16);
  else
    probe_write_kernel<false><<<blocks, 256, 0, s>>>(static_cast<u32x4*>(dst), bytes / 16);
  PROBE_HIP_CHECK(hipGetLastError());
  t_probe_error.clear();
  return 0;
}

const char* hcg_probe_last_error(void) { return t_probe_error.c_str(); }

}  // extern "C"
