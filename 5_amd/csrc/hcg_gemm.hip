// hcg_gemm.hip -- gfx950 (MI355X, CDNA4) kernels and C ABI for the hc tiled
// matrix-core GEMM: C[M,N] (f32) = A[M,K] @ B[K,N], A/B fp16 or bf16, all
// row-major, float32 accumulation.
//
// This is the device implementation behind the hc launch surface
// (hc/simulator.py:165-186 binding the kernel of
// examples/amdgpu_gfx11_wmma_matmul.py:301-326).  The reference describes a
// wave32 16x16x16 WMMA tile per workgroup; on CDNA4 the work is re-tiled for
// 64-wide wavefronts and the v_mfma_f32_{32x32x16,16x16x32}_{f16,bf16}
// matrix cores:
//
//   * gemm_tiled_kernel -- compute-bound shapes.  256x256 output tile per
//     256-thread workgroup (4 waves in 2x2, each 128x128 = 4x4 MFMA 32x32x16
//     tiles), K step 64, double-buffered LDS, 128-bit global loads, B
//     transposed in registers on its way to LDS so both MFMA operands read
//     K-contiguous 128-bit fragments, XOR-swizzled LDS rows, XCD-aware tile
//     order, masked M/N/K tails.
//   * gemm_skinny_kernel -- M <= 16 (HBM-bound).  One 16-row MFMA 16x16x32
//     block covers all of A; B is streamed exactly once with 128-bit loads,
//     transposed 8x8 in registers, split over K across waves and workgroups;
//     partial sums are reduced in a fixed order (deterministic).
//
// Numerics: products of fp16/bf16 values are exact in float32 and the MFMA
// accumulates in float32; only the order of the float32 additions differs
// from the reference's strictly sequential fold.

#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <string>

#include "hcg_gemm.h"

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// Matrix-core wrappers.  Operand layout (both 32x32x16 and 16x16x32): a lane
// holds 8 K-contiguous 16-bit values of one A row / one B column; both
// operands use the same lane -> k assignment, so the contraction is exact
// regardless of how the hardware orders k inside one instruction.
// ---------------------------------------------------------------------------

template <int DT>
__device__ __forceinline__ f32x16 mfma32x32x16(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (DT == HCG_F16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                 __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
}

template <int DT>
__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (DT == HCG_F16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                 __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
}

// 8 consecutive 16-bit elements of one row, starting at column col0; columns
// at or beyond ncols read as +0 (the masked tile load of
// hc/simulator.py:1338-1357 followed by with_inactive(0)).  kVec: the row is
// 16-byte aligned at every multiple of 8 columns, so a whole in-bounds chunk
// is one 128-bit load.
template <bool kVec>
__device__ __forceinline__ u32x4 load8(const uint16_t* rowp, int col0, int ncols) {
  if (kVec && col0 + 8 <= ncols) return *reinterpret_cast<const u32x4*>(rowp + col0);
  uint32_t w[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int c = col0 + 2 * p;
    const uint32_t lo = (c < ncols) ? rowp[c] : 0u;
    const uint32_t hi = (c + 1 < ncols) ? rowp[c + 1] : 0u;
    w[p] = lo | (hi << 16);
  }
  return u32x4{w[0], w[1], w[2], w[3]};
}

// 8x8 transpose of 16-bit elements held as 8 rows of 128 bits: on return
// out[n] holds column n, i.e. (in[0][n], in[1][n], ..., in[7][n]).
__device__ __forceinline__ void transpose8x8(const u32x4 (&in)[8], u32x4 (&out)[8]) {
#pragma unroll
  for (int n = 0; n < 8; ++n) {
    const int w = n >> 1;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t lo = in[2 * q][w];
      const uint32_t hi = in[2 * q + 1][w];
      out[n][q] = (n & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
    }
  }
}

// ---------------------------------------------------------------------------
// Tiled kernel
// ---------------------------------------------------------------------------

constexpr int kTileM = 256;
constexpr int kTileN = 256;
constexpr int kTileK = 64;
constexpr int kTiledThreads = 256;
constexpr int kGroupM = 4;  // tile rows per group in the tile order (L2 reuse of B)

struct TiledArgs {
  const uint16_t* A;
  const uint16_t* B;
  float* C;
  int64_t lda, ldb, ldc;
  int M, N, K;
  int tiles_m, tiles_n;
};

// LDS row of kTileK 16-bit values = 8 chunks of 16 bytes.  The chunk index is
// XORed with bits of the row so that 8 consecutive lanes of every access
// pattern used below (row-chunk A stores, transposed B stores, fragment
// reads) hit 8 distinct 16-byte bank groups.
__device__ __forceinline__ int swz(int row, int chunk) {
  return row * 8 + (chunk ^ (row & 7) ^ ((row >> 3) & 7));
}

// blockIdx -> output tile.  Workgroups are dispatched round-robin over the 8
// XCDs (id % 8); the first remap gives each XCD a contiguous run of logical
// tiles, the second orders logical tiles in groups of kGroupM tile rows so
// that tiles sharing an XCD's L2 also share A rows and B columns.
__device__ __forceinline__ void tile_coords(int tiles_m, int tiles_n, int& tm, int& tn) {
  const int nt = tiles_m * tiles_n;
  const int wg = blockIdx.x;
  const int per = nt >> 3, rem = nt & 7, xcd = wg & 7, idx = wg >> 3;
  const int logical =
      (xcd < rem) ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
  const int span = kGroupM * tiles_n;
  const int group = logical / span;
  const int first_m = group * kGroupM;
  const int gsize = min(tiles_m - first_m, kGroupM);
  const int in_group = logical - group * span;
  tm = first_m + in_group % gsize;
  tn = in_group / gsize;
}

template <int DT, bool kVecA, bool kVecB>
__global__ __launch_bounds__(kTiledThreads) void gemm_tiled_kernel(TiledArgs g) {
  __shared__ u32x4 lds_a[2][kTileM * 8];
  __shared__ u32x4 lds_b[2][kTileN * 8];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  int tm, tn;
  tile_coords(g.tiles_m, g.tiles_n, tm, tn);
  const int m0 = tm * kTileM, n0 = tn * kTileN;
  const int nk = (g.K + kTileK - 1) / kTileK;

  // Staging roles.  A: thread owns chunk a_c of rows a_r + 32 i (8 lanes read
  // one contiguous 128-byte row segment).  B: thread owns an 8(k) x 8(n)
  // block, rows b_kb*8 + i, columns b_n*8 .. +7 (32 lanes read 512 contiguous
  // bytes of one row).
  const int a_c = tid & 7, a_r = tid >> 3;
  const int b_n = tid & 31, b_kb = tid >> 5;

  u32x4 ra[8], rb[8];
  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

  auto load_regs = [&](int kt) {
    const int k0 = kt * kTileK;
    const bool a_full = kVecA && (m0 + kTileM <= g.M) && (k0 + kTileK <= g.K);
    const bool b_full = kVecB && (n0 + kTileN <= g.N) && (k0 + kTileK <= g.K);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = m0 + a_r + 32 * i;
      const uint16_t* p = g.A + (int64_t)row * g.lda;
      if (a_full) {
        ra[i] = *reinterpret_cast<const u32x4*>(p + k0 + a_c * 8);
      } else {
        ra[i] = (row < g.M) ? load8<kVecA>(p, k0 + a_c * 8, g.K) : u32x4{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int k = k0 + b_kb * 8 + i;
      const uint16_t* p = g.B + (int64_t)k * g.ldb;
      if (b_full) {
        rb[i] = *reinterpret_cast<const u32x4*>(p + n0 + b_n * 8);
      } else {
        rb[i] = (k < g.K) ? load8<kVecB>(p, n0 + b_n * 8, g.N) : u32x4{0, 0, 0, 0};
      }
    }
  };

  auto store_lds = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 8; ++i) lds_a[buf][swz(a_r + 32 * i, a_c)] = ra[i];
    u32x4 bt[8];
    transpose8x8(rb, bt);
#pragma unroll
    for (int n = 0; n < 8; ++n) lds_b[buf][swz(b_n * 8 + n, b_kb)] = bt[n];
  };

  auto compute = [&](int buf) {
#pragma unroll
    for (int kk = 0; kk < kTileK / 16; ++kk) {
      const int c = kk * 2 + (lane >> 5);
      u32x4 af[4], bf[4];
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) af[mi] = lds_a[buf][swz(wm * 128 + mi * 32 + (lane & 31), c)];
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) bf[ni] = lds_b[buf][swz(wn * 128 + ni * 32 + (lane & 31), c)];
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = mfma32x32x16<DT>(af[mi], bf[ni], acc[mi][ni]);
    }
  };

  load_regs(0);
  store_lds(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load_regs(kt + 1);
    compute(buf);
    if (kt + 1 < nk) store_lds(buf ^ 1);
    __syncthreads();
  }

  // Epilogue.  32x32 accumulator layout: register r of lane l holds
  // row 8*(r/4) + 4*(l/32) + r%4, column l%32.  Only in-bounds C is written.
  const int col_l = lane & 31;
  const int row_l = (lane >> 5) * 4;
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) {
      const int col = n0 + wn * 128 + ni * 32 + col_l;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * 128 + mi * 32 + (r >> 2) * 8 + row_l + (r & 3);
        if (row < g.M && col < g.N) g.C[(int64_t)row * g.ldc + col] = acc[mi][ni][r];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Skinny (M <= 16) kernel
// ---------------------------------------------------------------------------

constexpr int kSkinnyN = 128;       // output columns per workgroup
constexpr int kSkinnyStep = 32;     // k rows per wave step (one MFMA 16x16x32)
constexpr int kSkinnyWaves = 4;
constexpr int kSkinnyThreads = 64 * kSkinnyWaves;

struct SkinnyArgs {
  const uint16_t* A;
  const uint16_t* B;
  float* C;    // used when splits == 1
  float* ws;   // [splits][16][N] partial sums when splits > 1
  int64_t lda, ldb, ldc;
  int M, N, K;
  int kchunk;  // k rows per split (multiple of kSkinnyStep * kSkinnyWaves)
  int splits;
};

template <int DT, bool kVecA, bool kVecB>
__device__ __forceinline__ void skinny_load(const SkinnyArgs& g, int k0, int lane, int ncol0,
                                            u32x4& af, u32x4 (&rb)[8]) {
  const int grp = lane >> 4;
  const int kr = k0 + grp * 8;
  const int arow = lane & 15;
  af = (arow < g.M) ? load8<kVecA>(g.A + (int64_t)arow * g.lda, kr, g.K) : u32x4{0, 0, 0, 0};
  const bool full = kVecB && (k0 + kSkinnyStep <= g.K) && (ncol0 + 8 <= g.N);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int k = kr + i;
    const uint16_t* p = g.B + (int64_t)k * g.ldb;
    if (full) {
      rb[i] = *reinterpret_cast<const u32x4*>(p + ncol0);
    } else {
      rb[i] = (k < g.K) ? load8<kVecB>(p, ncol0, g.N) : u32x4{0, 0, 0, 0};
    }
  }
}

template <int DT, bool kVecA, bool kVecB>
__global__ __launch_bounds__(kSkinnyThreads) void gemm_skinny_kernel(SkinnyArgs g) {
  __shared__ float red[kSkinnyWaves][16][kSkinnyN];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n0 = blockIdx.x * kSkinnyN;
  const int split = blockIdx.y;
  const int kbeg = split * g.kchunk;
  const int kend = min(g.K, kbeg + g.kchunk);
  const int ncol0 = n0 + (lane & 15) * 8;

  // Lane l, step at k0: A operand = A[l%16][k0 + 8*(l/16) .. +7]; B operand
  // for instruction t = B[k0 + 8*(l/16) .. +7][n0 + 8*(l%16) + t].  Output
  // column j = l%16 of instruction t is C column n0 + 8*j + t.
  f32x4 acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = f32x4{};

  int k0 = kbeg + wave * kSkinnyStep;
  u32x4 af, rb[8];
  if (k0 < kend) skinny_load<DT, kVecA, kVecB>(g, k0, lane, ncol0, af, rb);
  for (; k0 < kend; k0 += kSkinnyWaves * kSkinnyStep) {
    const int kn = k0 + kSkinnyWaves * kSkinnyStep;
    u32x4 naf, nrb[8];
    if (kn < kend) skinny_load<DT, kVecA, kVecB>(g, kn, lane, ncol0, naf, nrb);
    u32x4 bt[8];
    transpose8x8(rb, bt);
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = mfma16x16x32<DT>(af, bt[t], acc[t]);
    if (kn < kend) {
      af = naf;
#pragma unroll
      for (int i = 0; i < 8; ++i) rb[i] = nrb[i];
    }
  }

  // 16x16 accumulator layout: register r of lane l holds row 4*(l/16) + r,
  // column l%16.
#pragma unroll
  for (int t = 0; t < 8; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][(lane >> 4) * 4 + r][(lane & 15) * 8 + t] = acc[t][r];
  __syncthreads();

  // Sum the waves in a fixed order.
#pragma unroll
  for (int e = 0; e < (16 * kSkinnyN) / kSkinnyThreads; ++e) {
    const int idx = e * kSkinnyThreads + tid;
    const int row = idx / kSkinnyN, col = idx % kSkinnyN;
    float v = red[0][row][col];
#pragma unroll
    for (int w = 1; w < kSkinnyWaves; ++w) v += red[w][row][col];
    const int gc = n0 + col;
    if (gc < g.N) {
      if (g.splits == 1) {
        if (row < g.M) g.C[(int64_t)row * g.ldc + gc] = v;
      } else {
        g.ws[((int64_t)split * 16 + row) * g.N + gc] = v;
      }
    }
  }
}

// C[i][j] = sum over splits s = 0..S-1 (in order) of ws[s][i][j].
__global__ __launch_bounds__(256) void skinny_reduce_kernel(const float* ws, float* C, int64_t ldc,
                                                            int M, int N, int splits) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)M * N) return;
  const int row = (int)(idx / N), col = (int)(idx % N);
  float v = ws[(int64_t)row * N + col];
  for (int s = 1; s < splits; ++s) v += ws[((int64_t)s * 16 + row) * N + col];
  C[(int64_t)row * ldc + col] = v;
}

__global__ __launch_bounds__(256) void fill_zero_kernel(float* C, int64_t ldc, int M, int N) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)M * N) return;
  C[(idx / N) * ldc + (idx % N)] = 0.0f;
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

thread_local std::string t_last_error;

int set_error(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  t_last_error = buf;
  return code;
}

#define HCG_HIP_CHECK(expr)                                                               \
  do {                                                                                    \
    hipError_t _e = (expr);                                                               \
    if (_e != hipSuccess)                                                                 \
      return set_error(HCG_EHIP, "%s failed: %s", #expr, hipGetErrorString(_e));          \
  } while (0)

constexpr int kMaxDevices = 64;

struct DeviceState {
  std::once_flag once;
  int init_status = HCG_OK;
  std::string init_error;
  int num_cus = 256;
  std::mutex ws_mutex;
  float* ws = nullptr;
  size_t ws_bytes = 0;
};

DeviceState g_devices[kMaxDevices];
int g_skinny_splits_override = 0;
std::once_flag g_global_once;

void global_init() {
  const char* s = getenv("HCG_SKINNY_SPLITS");
  if (s) g_skinny_splits_override = atoi(s);
}

int current_device_state(DeviceState** out) {
  std::call_once(g_global_once, global_init);
  int dev = 0;
  HCG_HIP_CHECK(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return set_error(HCG_EINVAL, "device %d out of range", dev);
  DeviceState& st = g_devices[dev];
  std::call_once(st.once, [&] {
    int cus = 0;
    hipError_t e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) {
      st.init_status = HCG_EHIP;
      st.init_error = std::string("hipDeviceGetAttribute failed: ") + hipGetErrorString(e);
      return;
    }
    st.num_cus = cus > 0 ? cus : 256;
  });
  if (st.init_status != HCG_OK) return set_error(st.init_status, "%s", st.init_error.c_str());
  *out = &st;
  return HCG_OK;
}

// Library-owned split-K workspace, grown on demand and kept per device.
int device_workspace(DeviceState* st, size_t bytes, float** out) {
  std::lock_guard<std::mutex> lock(st->ws_mutex);
  if (st->ws_bytes < bytes) {
    if (st->ws) {
      HCG_HIP_CHECK(hipDeviceSynchronize());
      HCG_HIP_CHECK(hipFree(st->ws));
      st->ws = nullptr;
      st->ws_bytes = 0;
    }
    void* p = nullptr;
    HCG_HIP_CHECK(hipMalloc(&p, bytes));
    st->ws = static_cast<float*>(p);
    st->ws_bytes = bytes;
  }
  *out = st->ws;
  return HCG_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <int DT>
int launch_tiled(const TiledArgs& a, bool vec_a, bool vec_b, hipStream_t stream) {
  const dim3 grid((unsigned)(a.tiles_m * a.tiles_n));
  const dim3 block(kTiledThreads);
  if (vec_a && vec_b) {
    gemm_tiled_kernel<DT, true, true><<<grid, block, 0, stream>>>(a);
  } else if (vec_a) {
    gemm_tiled_kernel<DT, true, false><<<grid, block, 0, stream>>>(a);
  } else if (vec_b) {
    gemm_tiled_kernel<DT, false, true><<<grid, block, 0, stream>>>(a);
  } else {
    gemm_tiled_kernel<DT, false, false><<<grid, block, 0, stream>>>(a);
  }
  HCG_HIP_CHECK(hipGetLastError());
  return HCG_OK;
}

template <int DT>
int launch_skinny(const SkinnyArgs& a, bool vec_a, bool vec_b, hipStream_t stream) {
  const dim3 grid((unsigned)((a.N + kSkinnyN - 1) / kSkinnyN), (unsigned)a.splits);
  const dim3 block(kSkinnyThreads);
  if (vec_a && vec_b) {
    gemm_skinny_kernel<DT, true, true><<<grid, block, 0, stream>>>(a);
  } else if (vec_a) {
    gemm_skinny_kernel<DT, true, false><<<grid, block, 0, stream>>>(a);
  } else if (vec_b) {
    gemm_skinny_kernel<DT, false, true><<<grid, block, 0, stream>>>(a);
  } else {
    gemm_skinny_kernel<DT, false, false><<<grid, block, 0, stream>>>(a);
  }
  HCG_HIP_CHECK(hipGetLastError());
  if (a.splits > 1) {
    const int64_t total = (int64_t)a.M * a.N;
    skinny_reduce_kernel<<<(unsigned)((total + 255) / 256), 256, 0, stream>>>(a.ws, a.C, a.ldc, a.M,
                                                                             a.N, a.splits);
    HCG_HIP_CHECK(hipGetLastError());
  }
  return HCG_OK;
}

int skinny_splits(const DeviceState* st, int N, int K) {
  const int nblocks = (N + kSkinnyN - 1) / kSkinnyN;
  const int kunit = kSkinnyStep * kSkinnyWaves;
  const int kunits = (K + kunit - 1) / kunit;
  int splits = g_skinny_splits_override;
  if (splits <= 0) {
    // Aim for two workgroups per CU; each split keeps at least 2 steps/wave.
    const int want = 2 * st->num_cus;
    splits = (want + nblocks - 1) / nblocks;
    const int max_by_k = kunits / 2 > 0 ? kunits / 2 : 1;
    if (splits > max_by_k) splits = max_by_k;
  }
  if (splits > kunits) splits = kunits;
  if (splits < 1) splits = 1;
  return splits;
}

int gemm_impl(int algo, int dtype, const void* A, int64_t lda, const void* B, int64_t ldb,
              float* C, int64_t ldc, int64_t M, int64_t N, int64_t K, void* stream_ptr) {
  if (dtype != HCG_F16 && dtype != HCG_BF16)
    return set_error(HCG_EINVAL, "dtype must be HCG_F16 (0) or HCG_BF16 (1), got %d", dtype);
  if (algo != HCG_ALGO_AUTO && algo != HCG_ALGO_TILED && algo != HCG_ALGO_SKINNY)
    return set_error(HCG_EINVAL, "unknown algo %d", algo);
  if (M < 0 || N < 0 || K < 0)
    return set_error(HCG_EINVAL, "negative extent: M=%lld N=%lld K=%lld", (long long)M,
                     (long long)N, (long long)K);
  const int64_t kMaxExtent = (int64_t)1 << 30;
  if (M > kMaxExtent || N > kMaxExtent || K > kMaxExtent)
    return set_error(HCG_EINVAL, "extent above 2^30: M=%lld N=%lld K=%lld", (long long)M,
                     (long long)N, (long long)K);
  if (algo == HCG_ALGO_SKINNY && M > 16)
    return set_error(HCG_EINVAL, "the skinny kernel needs M <= 16, got M=%lld", (long long)M);
  if (M == 0 || N == 0) {
    t_last_error.clear();
    return HCG_OK;
  }
  if (C == nullptr) return set_error(HCG_EINVAL, "C is NULL");
  if (ldc < N) return set_error(HCG_EINVAL, "ldc (%lld) < N (%lld)", (long long)ldc, (long long)N);
  if (K > 0) {
    if (A == nullptr || B == nullptr) return set_error(HCG_EINVAL, "A or B is NULL");
    if (lda < K) return set_error(HCG_EINVAL, "lda (%lld) < K (%lld)", (long long)lda, (long long)K);
    if (ldb < N) return set_error(HCG_EINVAL, "ldb (%lld) < N (%lld)", (long long)ldb, (long long)N);
  }
  DeviceState* st = nullptr;
  int rc = current_device_state(&st);
  if (rc != HCG_OK) return rc;
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);

  if (K == 0) {
    const int64_t total = M * N;
    fill_zero_kernel<<<(unsigned)((total + 255) / 256), 256, 0, stream>>>(C, ldc, (int)M, (int)N);
    HCG_HIP_CHECK(hipGetLastError());
    t_last_error.clear();
    return HCG_OK;
  }

  const bool vec_a = aligned16(A) && (lda % 8 == 0);
  const bool vec_b = aligned16(B) && (ldb % 8 == 0);
  const bool use_skinny = algo == HCG_ALGO_SKINNY || (algo == HCG_ALGO_AUTO && M <= 16);

  if (use_skinny) {
    SkinnyArgs a{};
    a.A = static_cast<const uint16_t*>(A);
    a.B = static_cast<const uint16_t*>(B);
    a.C = C;
    a.lda = lda;
    a.ldb = ldb;
    a.ldc = ldc;
    a.M = (int)M;
    a.N = (int)N;
    a.K = (int)K;
    a.splits = skinny_splits(st, (int)N, (int)K);
    const int kunit = kSkinnyStep * kSkinnyWaves;
    const int kunits = ((int)K + kunit - 1) / kunit;
    a.kchunk = ((kunits + a.splits - 1) / a.splits) * kunit;
    a.splits = ((int)K + a.kchunk - 1) / a.kchunk;  // drop empty trailing splits
    a.ws = nullptr;
    if (a.splits > 1) {
      rc = device_workspace(st, (size_t)a.splits * 16 * (size_t)N * sizeof(float), &a.ws);
      if (rc != HCG_OK) return rc;
    }
    rc = dtype == HCG_F16 ? launch_skinny<HCG_F16>(a, vec_a, vec_b, stream)
                          : launch_skinny<HCG_BF16>(a, vec_a, vec_b, stream);
  } else {
    TiledArgs a{};
    a.A = static_cast<const uint16_t*>(A);
    a.B = static_cast<const uint16_t*>(B);
    a.C = C;
    a.lda = lda;
    a.ldb = ldb;
    a.ldc = ldc;
    a.M = (int)M;
    a.N = (int)N;
    a.K = (int)K;
    a.tiles_m = (int)((M + kTileM - 1) / kTileM);
    a.tiles_n = (int)((N + kTileN - 1) / kTileN);
    if ((int64_t)a.tiles_m * a.tiles_n > 0x7fffffff)
      return set_error(HCG_EINVAL, "too many output tiles");
    rc = dtype == HCG_F16 ? launch_tiled<HCG_F16>(a, vec_a, vec_b, stream)
                          : launch_tiled<HCG_BF16>(a, vec_a, vec_b, stream);
  }
  if (rc == HCG_OK) t_last_error.clear();
  return rc;
}

}  // namespace

extern "C" {

int hcg_init(void) {
  DeviceState* st = nullptr;
  const int rc = current_device_state(&st);
  if (rc == HCG_OK) t_last_error.clear();
  return rc;
}

int hcg_gemm(int dtype, const void* A, int64_t lda, const void* B, int64_t ldb, float* C,
             int64_t ldc, int64_t M, int64_t N, int64_t K, void* stream) {
  return gemm_impl(HCG_ALGO_AUTO, dtype, A, lda, B, ldb, C, ldc, M, N, K, stream);
}

int hcg_gemm_algo(int algo, int dtype, const void* A, int64_t lda, const void* B, int64_t ldb,
                  float* C, int64_t ldc, int64_t M, int64_t N, int64_t K, void* stream) {
  return gemm_impl(algo, dtype, A, lda, B, ldb, C, ldc, M, N, K, stream);
}

const char* hcg_last_error(void) { return t_last_error.c_str(); }

int hcg_version(void) { return 100; }

}  // extern "C"
