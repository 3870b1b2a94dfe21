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
//   * gemm_dma_kernel -- compute-bound shapes.  TM x TN output tile per
//     256-thread workgroup (256x256, 256x192, 128x256, 128x128 or 256x64, picked by
//     size; 4 waves in 2x2, each (TM/2) x (TN/2) of MFMA 32x32x16 tiles),
//     K step 32 through an LDS ring filled by direct global->LDS DMA loads
//     (buffer_load ... lds; 256-row tiles move A two K steps at a time),
//     operand rows read in place at any 2-byte alignment, B kept row-major
//     in LDS and read with transposing LDS loads (ds_read_b64_tr_b16),
//     XOR-swizzled bank-conflict-free layouts, XCD-aware tile order, masked
//     M/N/K tails by the buffer range check (and the A elements past K
//     cleared in the last K tile), and an LDS-staged 16-byte epilogue;
//     shapes with few tiles and a long K split K over workgroups (partials
//     summed in a fixed order by stream_reduce_kernel).
//   * gemm_stream_kernel -- M <= 128, N > 64 (HBM-bound).  B streams HBM ->
//     LDS once by DMA, split over K across workgroups mapped so every XCD
//     covers all column residues, against 1, 2, 4 or 8 16-row blocks of A;
//     the split partials are summed in a fixed order (deterministic) by
//     the last workgroup of each column block to arrive (R <= 2) or by
//     stream_reduce_kernel, skinny_reduce_kernel or, past 16 splits,
//     split_reduce_kernel.  Its UB form stages B through registers when
//     B's last row piece cannot be read safely in place.
//   * gemm_generic_kernel -- fallback (plain pointers, register staging, any
//     alignment) for unaligned operands whose byte offsets do not fit 31
//     bits; aligned ones that large run the DMA kernel's WIDE form.
//   * gemm_rowstream_kernel -- N <= 64, any layout (HBM-bound): A streams
//     HBM -> LDS once in 256-byte row pieces, by DMA in place (through
//     registers when its last row piece cannot be read safely), split over
//     K; partials reduced as for gemm_stream_kernel.
//   * gemm_skinny_kernel -- M <= 16 when the streaming kernels cannot take
//     the operands: B streamed with 128-bit loads, transposed 8x8 in
//     registers, split over K; partial sums reduced in a fixed order.
//   * repack_kernel -- copies an operand that cannot be read in place (its
//     last row piece not safely readable, or its offsets past 2^31) into
//     zero-padded 16-byte aligned rows for the DMA kernels.
//
// Numerics: products of fp16/bf16 values are exact in float32 and the MFMA
// accumulates in float32; only the order of the float32 additions differs
// from the reference's strictly sequential fold.

#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <mutex>
#include <vector>
#include <type_traits>
#include <string>

#include "hcg_gemm.h"
#include "hcg_runtime.h"
#include "hcg_tile.h"

namespace hcg {

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

}  // namespace hcg

namespace {

using hcg::dma16;
using hcg::dma_offset;
using hcg::kOobOffset;
using hcg::lds_void;
using hcg::load_row8_u16;
using hcg::make_rsrc;

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
// Four floats at a 4-byte aligned address (one 16-byte vector access).
typedef float f32x4u __attribute__((ext_vector_type(4), aligned(4)));
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
// Generic tiled kernel (global pointers; any alignment and size)
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
__device__ __forceinline__ void tile_coords(int tiles_m, int tiles_n, int& tm, int& tn, int wg) {
  const int nt = tiles_m * tiles_n;
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
__global__ __launch_bounds__(kTiledThreads) void gemm_generic_kernel(TiledArgs g) {
  __shared__ u32x4 lds_a[2][kTileM * 8];
  __shared__ u32x4 lds_b[2][kTileN * 8];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  int tm, tn;
  tile_coords(g.tiles_m, g.tiles_n, tm, tn, blockIdx.x);
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
        ra[i] = (row < g.M) ? load_row8_u16<kVecA>(p, k0 + a_c * 8, g.K) : u32x4{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int k = k0 + b_kb * 8 + i;
      const uint16_t* p = g.B + (int64_t)k * g.ldb;
      if (b_full) {
        rb[i] = *reinterpret_cast<const u32x4*>(p + n0 + b_n * 8);
      } else {
        rb[i] = (k < g.K) ? load_row8_u16<kVecB>(p, n0 + b_n * 8, g.N) : u32x4{0, 0, 0, 0};
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
// Fast tiled kernel (LDS DMA; rows at any 2-byte alignment; offsets < 2^31)
// ---------------------------------------------------------------------------

struct FastArgs {
  const uint16_t* A;
  const uint16_t* B;
  float* C;
  int lda, ldb;  // elements; multiples of 8
  int64_t ldc;
  int M, N, K;
  int tiles_m, tiles_n;
  int a_bytes, b_bytes;  // buffer extents for the hardware range check
  bool c_vec;            // C rows are 16-byte aligned at every 4th column
  // Split-K (splits > 1): workgroup s * tiles + t computes tile t over K
  // rows [s * kchunk, (s + 1) * kchunk) into ws + s * M * N (row stride N).
  int splits, kchunk;
  float* ws;
  bool ws_vec;           // N is a multiple of 4 (16-byte partial rows)
#ifdef HCG_STAMPS
  int stamp_slot;
#endif
};

// Scheduling-group masks for __builtin_amdgcn_sched_group_barrier.
constexpr int kSgMfma = 0x008;
constexpr int kSgVmemRead = 0x020;
constexpr int kSgDsRead = 0x100;

// ---------------------------------------------------------------------------
// DMA tiled kernel: global -> LDS with buffer_load ... lds (no VGPR staging)
// ---------------------------------------------------------------------------
//
// TM x TN output tile, 4 waves (2x2, each TM/2 x TN/2 = TM/64 x TN/64 MFMA
// 32x32x16 tiles), K step 32, and a STAGES-deep LDS ring:
// a stage is refilled (tile kt + STAGES) as soon as the barrier after its
// last fragment reads has passed.  TM = 256 uses 4 stages (128 KB, one
// workgroup per CU); TM = 128 uses 3 stages (72 KB) so two workgroups share
// a CU -- for shapes with too few large tiles to fill the chip.
//
// Stage layout: A as [TM rows][32 k] (64-byte rows of 4 chunks of 16 bytes),
// B as [32 k][256 n] (512-byte rows of 32 chunks, whatever TN; chunks past
// TN are zero-filled and never read); chunks are XOR-swizzled
// per row (a_chunk_swz, b_chunk_swz).  A fragments are one ds_read_b128; B
// fragments are two ds_read_b64_tr_b16, which within each 16-lane group
// hand lane i element i%4 of source lane 4j + i/4 (j = 0..3): source lanes
// point at 4 consecutive k rows x 16 columns, so lane i receives 4
// consecutive k of column i, the MFMA B operand.
//
// Requirements (checked on the host): A and B readable in place (rows at
// any 2-byte alignment, the bytes the last chunk reads past an operand
// safely mapped; otherwise repacked into zero-padded aligned rows).  K and N
// need not be multiples of 8: the chunk holding column N - 1 also loads up
// to 7 padding columns of B, which reach only C columns >= N (never
// stored), and the KT form clears A's elements past K.  Chunks past
// K or N are redirected past the buffer extent, so the hardware range check
// returns zeros; rows past M (A) or K (B) are past it already.

constexpr int kDmaK = 32;

typedef short s16x4 __attribute__((ext_vector_type(4)));

// s_waitcnt with only vmcnt (lgkmcnt / expcnt left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0f70 | (N & 15) | ((N >> 4) << 14));
}
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xc07f); }

// Per-workgroup timing records, in the HCG_STAMPS build of this file only
// (libhcg_gfx950_stamps.so; in the product build every member is empty).
// mark(i) reads the 100 MHz constant clock (s_memrealtime) and the shader
// clock (s_memtime) at the workgroup's start (0), the end of its prologue
// (1), the end of its K loop (2); write() waits for the workgroup's stores
// to be acknowledged, marks its end (3) and has lane 0 store, with vector
// stores, one record of 8 words at g_stamp_buf + 8 * (slot * gridDim.x +
// blockIdx.x):
//   [0..3] clock at marks 0..3, [4] shader cycles of the K loop (2 - 1),
//   [5] shader cycles start to end (3 - 0), [6] XCC id (bits 3:0), grid size
//   (bits 47:8) and record slot (bit 48), [7] HW_ID.
// hcg_stamps_set() names the buffer; bench.py --stamps reads it.  Launches
// alternate between the two slots (record areas), so two consecutive
// launches can be compared.
#ifdef HCG_STAMPS
__device__ uint64_t* g_stamp_buf = nullptr;
__device__ int64_t g_stamp_cap = 0;
std::atomic<int> g_stamp_launches{0};  // host: launches so far (their parity is the slot)
#define HCG_STAMP_SLOT(g) (g).stamp_slot
#define HCG_STAMP_ARGS(Args, a) \
  Args a##_s = a;               \
  a##_s.stamp_slot = g_stamp_launches.fetch_add(1, std::memory_order_relaxed) & 1;
#define HCG_STAMPED(a) a##_s
#else
#define HCG_STAMP_SLOT(g) 0
#define HCG_STAMP_ARGS(Args, a)
#define HCG_STAMPED(a) a
#endif
struct WgStamps {
#ifdef HCG_STAMPS
  int slot;
  uint64_t t[4] = {}, c[4] = {};
  __device__ explicit WgStamps(int s) : slot(s) {}
  __device__ __forceinline__ void mark(int i) {
    t[i] = __builtin_amdgcn_s_memrealtime();
    c[i] = __builtin_amdgcn_s_memtime();
  }
  __device__ __forceinline__ void write() {
    wait_vmcnt<0>();
    mark(3);
    uint64_t* buf = g_stamp_buf;
    const int64_t index = (int64_t)blockIdx.x + (int64_t)gridDim.x * slot;
    if (threadIdx.x == 0 && buf != nullptr && index < g_stamp_cap) {
      const uint64_t xcc = __builtin_amdgcn_s_getreg((3 << 11) | 20);  // HW_REG_XCC_ID[3:0]
      const uint64_t hw = __builtin_amdgcn_s_getreg((31 << 11) | 4);   // HW_REG_HW_ID
      uint64_t* r = buf + 8 * index;
      r[0] = t[0];
      r[1] = t[1];
      r[2] = t[2];
      r[3] = t[3];
      r[4] = c[2] - c[1];
      r[5] = c[3] - c[0];
      r[6] = xcc | ((uint64_t)gridDim.x << 8) | ((uint64_t)slot << 48);
      r[7] = hw;
    }
  }
#else
  __device__ explicit WgStamps(int) {}
  __device__ __forceinline__ void mark(int) {}
  __device__ __forceinline__ void write() {}
#endif
};

template <int TM>
constexpr int dma_stage_bytes() {
  return (TM + kTileN) * kDmaK * 2;
}

// Each stage is a separate LDS object and every access names its stage at
// compile time, so the compiler can tell a DMA into one stage from reads of
// another and does not serialize them with a full vmcnt wait.
__shared__ __attribute__((aligned(1024))) unsigned char g_t256_s0[dma_stage_bytes<256>()];
__shared__ __attribute__((aligned(1024))) unsigned char g_t256_s1[dma_stage_bytes<256>()];
__shared__ __attribute__((aligned(1024))) unsigned char g_t256_s2[dma_stage_bytes<256>()];
__shared__ __attribute__((aligned(1024))) unsigned char g_t256_s3[dma_stage_bytes<256>()];
__shared__ __attribute__((aligned(1024))) unsigned char g_t128_s0[dma_stage_bytes<128>()];
__shared__ __attribute__((aligned(1024))) unsigned char g_t128_s1[dma_stage_bytes<128>()];
__shared__ __attribute__((aligned(1024))) unsigned char g_t128_s2[dma_stage_bytes<128>()];

// A2 layout (TM = 256, 4 stages): A moves in 64-wide K pairs of tiles, one
// 128-byte piece per row, into two 32 KB double stages; B keeps four 16 KB
// stages.  Separate objects, so that no DMA shares an object with reads in
// flight.
__shared__ __attribute__((aligned(1024))) unsigned char g_a2_d0[256 * 64 * 2];
__shared__ __attribute__((aligned(1024))) unsigned char g_a2_d1[256 * 64 * 2];
__shared__ __attribute__((aligned(1024))) unsigned char g_b2_s0[kDmaK * kTileN * 2];
__shared__ __attribute__((aligned(1024))) unsigned char g_b2_s1[kDmaK * kTileN * 2];
__shared__ __attribute__((aligned(1024))) unsigned char g_b2_s2[kDmaK * kTileN * 2];
__shared__ __attribute__((aligned(1024))) unsigned char g_b2_s3[kDmaK * kTileN * 2];
template <int D>
__device__ __forceinline__ unsigned char* a2_dstage() {
  if constexpr (D == 0) return g_a2_d0;
  else return g_a2_d1;
}
template <int S>
__device__ __forceinline__ unsigned char* b2_stage() {
  if constexpr (S == 0) return g_b2_s0;
  else if constexpr (S == 1) return g_b2_s1;
  else if constexpr (S == 2) return g_b2_s2;
  else return g_b2_s3;
}
// Physical 16-byte chunk of logical chunk c (of 8) in an A2 row: rows two
// apart take different chunks, so a 16-lane group of ds_read_b128 (16
// consecutive rows of 128 bytes) covers all 64 banks once.
__device__ __forceinline__ int a2_chunk_swz(int row, int c) { return c ^ ((row >> 1) & 7); }

template <int TM, int S>
__device__ __forceinline__ unsigned char* dma_stage() {
  if constexpr (TM == 256) {
    if constexpr (S == 0) return g_t256_s0;
    else if constexpr (S == 1) return g_t256_s1;
    else if constexpr (S == 2) return g_t256_s2;
    else return g_t256_s3;
  } else {
    if constexpr (S == 0) return g_t128_s0;
    else if constexpr (S == 1) return g_t128_s1;
    else return g_t128_s2;
  }
}

template <int S>
using StageC = std::integral_constant<int, S>;

// Physical 16-byte chunk of logical chunk c in A row `row` (4 chunks/row).
// 16 consecutive rows read at one chunk land on 16 distinct 16-byte bank
// groups (64 banks), and any 8 consecutive rows on 8 (32 banks).
__device__ __forceinline__ int a_chunk_swz(int row, int c) {
  return c ^ ((row >> 1) & 3) ^ ((row >> 3) & 1);
}

// Physical chunk of logical chunk c in B row k (16 or 32 chunks/row).  A
// 32-lane transposed read touches 4 consecutive k rows x 4 consecutive
// chunks; the XOR pattern {0, 4, 10, 14} makes those 16 accesses distinct
// modulo 16 (64 banks) and each 16-lane half distinct modulo 8 (32 banks).
__device__ __forceinline__ int b_chunk_swz(int k, int c) {
  const int m = k & 3;
  return c ^ ((m >> 1) * 10 + (m & 1) * 4);
}

// WIDE: operands whose byte offsets reach 2^31.  The A resource then starts
// at the tile's first row and the B resource at (k0, n0), rebuilt for every
// B issue, with extents that end at the last valid element of that range
// (B: at the end of the chunk holding it), so every offset stays small; the
// range check still zero-fills rows past M and K, and chunks past N are
// redirected past the extent.
//
// KT: A is read in place with K not a multiple of 8, so the chunk holding
// column K - 1 also brings up to 7 elements past K (the next row or row
// padding, possibly Inf or NaN), which would meet B's zero-filled rows past
// K.  The fragments of the tile holding K - 1 are masked: those elements
// become +0.  (The DMA reads 16-byte chunks at any 2-byte alignment, so
// operands with unaligned rows are read in place; the host checks that the
// bytes a last chunk reads past an operand's end stay in the page of its
// last element.)
//
// A2 (TM = 256, 4 stages, not WIDE): A moves HBM -> LDS for two K tiles at
// a time, one 128-byte piece of each row per DMA lane group, instead of a
// 64-byte piece per tile: half the L2 requests for A, and never two lines
// for one tile's piece when rows are not 128-byte aligned.  Per-workgroup
// timestamps showed those requests, not MFMA issue, setting the K loop's
// pace at K ~ 1K (4096 x 3008 x 1024: 28.7k shader cycles at lda = 1024
// against 38.2k at lda = 1032; with A's requests collapsed, 27.5k for both).
template <int DT, int TM, int TN, int STAGES, bool WIDE = false, bool KT = false, bool A2 = false>
__global__ __launch_bounds__(kTiledThreads, TM == 256 ? 1 : 2) void gemm_dma_kernel(FastArgs g) {
  static_assert((TM == 256 && STAGES == 4) || (TM == 128 && STAGES == 3), "tile variant");
  static_assert(!A2 || (TM == 256 && STAGES == 4 && !WIDE), "A2 form");
  constexpr int kADma2 = TM / 32;  // A2: A DMA instructions per wave per pair of K tiles
  static_assert(TN == 256 || TN == 192 || TN == 128 || TN == 64, "tile width");
  constexpr int kMi = TM / 64;            // 32-row MFMA tiles per wave
  constexpr int kNi = TN / 64;            // 32-column MFMA tiles per wave
  constexpr int kADma = TM / 64;          // A DMA instructions per wave per stage
  constexpr int kDmaPerWave = kADma + 4;  // + 4 for B
  constexpr int kABytes = TM * kDmaK * 2;

  WgStamps stamps(HCG_STAMP_SLOT(g));
  stamps.mark(0);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // Wave index as a provably uniform value: it feeds the LDS base (M0) of
  // the DMA loads.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  int wg = blockIdx.x;
  if (g.splits > 1) {
    // This split's K range becomes the whole problem: shifted operand bases
    // and range-check extents (rows past M and columns past N stay past
    // them), K cut to the range, and C redirected to the split's partial.
    const int ntiles = g.tiles_m * g.tiles_n;
    const int split = wg / ntiles;
    wg -= split * ntiles;
    const int kbeg = split * g.kchunk;
    g.A += kbeg;
    g.B += (int64_t)kbeg * g.ldb;
    g.a_bytes -= kbeg * 2;
    g.b_bytes -= kbeg * g.ldb * 2;
    g.K = min(g.K - kbeg, g.kchunk);
    g.C = g.ws + (int64_t)split * g.M * g.N;
    g.ldc = g.N;
    g.c_vec = g.ws_vec;
  }
  int tm, tn;
  tile_coords(g.tiles_m, g.tiles_n, tm, tn, wg);
  const int m0 = tm * TM, n0 = tn * TN;
  const int nk = (g.K + kDmaK - 1) / kDmaK;

  const __amdgpu_buffer_rsrc_t rsrc_a =
      WIDE ? make_rsrc(g.A + (int64_t)m0 * g.lda, ((min(g.M - m0, TM) - 1) * g.lda + g.K) * 2)
           : make_rsrc(g.A, g.a_bytes);
  const __amdgpu_buffer_rsrc_t rsrc_b = make_rsrc(g.B, g.b_bytes);
  const int a_row0 = WIDE ? 0 : m0;  // A rows are counted from the resource base

  // DMA roles.  Each wave instruction fills 1 KB of LDS, lane l at byte
  // 16*l.  A: wave w owns 16-row blocks kADma*w .. +kADma-1; lane l covers
  // row blk*16 + l/4 at physical chunk l%4, so it loads the logical chunk
  // that the swizzle puts there (the swizzles are XOR involutions).  B: wave
  // w owns 2-row blocks 4w..4w+3; lane l covers k row blk*2 + l/32 at
  // physical chunk l%32.  B rows in LDS are always 32 chunks (512 bytes);
  // for TN < 256 the chunks past TN are dead and load zeros.
  int a_off[kADma], a_col[kADma], b_off[4], b_row[4];
#pragma unroll
  for (int i = 0; i < kADma; ++i) {
    const int blk = wave * kADma + i;
    const int row = blk * 16 + (lane >> 2);
    const int c = a_chunk_swz(row, lane & 3);
    a_col[i] = c * 8;
    a_off[i] = ((a_row0 + row) * g.lda + c * 8) * 2;
    // KT: rows past M start at the extent, so that they read zeros whatever
    // the K advance (with rows of fewer than round_up(K, 8) elements, which
    // only K % 8 != 0 allows, row M's first chunk would otherwise lie partly
    // inside it).
    if constexpr (KT && !WIDE)
      if (m0 + row >= g.M) a_off[i] = g.a_bytes;
  }
  // A2 roles: wave w fills rows 64w .. 64w + 63 of a double stage, 8 rows
  // (1 KB) per instruction; lane l covers row 64w + 8i + l/8 at physical
  // chunk l%8 (logical chunk a2_chunk_swz of it) of the 64-wide K pair.
  int a2_off[A2 ? kADma2 : 1], a2_col[A2 ? kADma2 : 1];
  if constexpr (A2) {
#pragma unroll
    for (int i = 0; i < kADma2; ++i) {
      const int row = 64 * wave + 8 * i + (lane >> 3);
      const int c = a2_chunk_swz(row, lane & 7);
      a2_col[i] = c * 8;
      a2_off[i] = ((m0 + row) * g.lda + c * 8) * 2;
      if constexpr (KT)
        if (m0 + row >= g.M) a2_off[i] = g.a_bytes;
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int blk = wave * 4 + i;
    const int kr = blk * 2 + (lane >> 5);
    const int cb = b_chunk_swz(kr, lane & 31);
    // Columns past N never change with k: push such a chunk's row out of
    // range once so the per-tile row test also covers them, and point its
    // offset at the end of B so the unchecked issue below reads zeros too.
    const bool live = cb < TN / 8 && n0 + cb * 8 < g.N;
    b_row[i] = live ? kr : 0x3fffffff;
    if constexpr (WIDE)
      b_off[i] = live ? (kr * g.ldb + cb * 8) * 2 : kOobOffset;
    else
      b_off[i] = live ? (kr * g.ldb + n0 + cb * 8) * 2 : g.b_bytes;
  }

  // The A part (kADma loads) or B part (4 loads) of tile kt into stage sc.
  // Checked form (full = false): every chunk past K (A columns, B rows) or
  // N is redirected past the buffer extent.  Unchecked form for tiles
  // wholly inside K (k0 + 32 <= K): the per-lane offsets stay fixed and the
  // K advance travels in the scalar offset, so the issue costs no vector
  // instructions.  Rows past M (A) and columns past N (B) have lane offsets
  // at or beyond the buffer extent on their own, so they read zeros whether
  // or not the hardware range check counts the scalar offset; all sums stay
  // below 2^32 (extents and K advances are below 2^31 each).
  auto issue_a = [&](auto sc, auto full, int kt) {
    unsigned char* st = dma_stage<TM, decltype(sc)::value>();
    const int k0 = kt * kDmaK;
#pragma unroll
    for (int i = 0; i < kADma; ++i) {
      lds_void* dst = (lds_void*)(st + (wave * kADma + i) * 1024);
      if constexpr (decltype(full)::value)
        dma16(rsrc_a, dst, a_off[i], k0 * 2);
      else
        dma16(rsrc_a, dst, dma_offset(k0 + a_col[i] < g.K, a_off[i] + k0 * 2));
    }
  };
  // A2: the A parts of K tiles kt and kt + 1 (kt even) into double stage D.
  auto issue_a2 = [&](auto dc, auto full, int kt) {
    unsigned char* st = a2_dstage<decltype(dc)::value>();
    const int k0 = kt * kDmaK;
#pragma unroll
    for (int i = 0; i < kADma2; ++i) {
      lds_void* dst = (lds_void*)(st + (wave * kADma2 + i) * 1024);
      if constexpr (decltype(full)::value)
        dma16(rsrc_a, dst, a2_off[i], k0 * 2);
      else
        dma16(rsrc_a, dst, dma_offset(k0 + a2_col[i] < g.K, a2_off[i] + k0 * 2));
    }
  };
  auto issue_b = [&](auto sc, auto full, int kt) {
    unsigned char* bst;  // the stage's B part
    if constexpr (A2)
      bst = b2_stage<decltype(sc)::value>();
    else
      bst = dma_stage<TM, decltype(sc)::value>() + kABytes;
    const int k0 = kt * kDmaK;
    if constexpr (WIDE) {
      // Resource for rows k0 .. k0 + 31 from column n0; rows past K are past
      // its extent (empty once k0 >= K).  The last row's extent is rounded
      // up to the 8-column chunk that holds column N - 1.
      const int rows = min(kDmaK, g.K - k0);
      const __amdgpu_buffer_rsrc_t rk = make_rsrc(
          g.B + (int64_t)k0 * g.ldb + n0, rows > 0 ? ((rows - 1) * g.ldb + ((g.N - n0 + 7) & ~7)) * 2 : 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) dma16(rk, (lds_void*)(bst + (wave * 4 + i) * 1024), b_off[i]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        lds_void* dst = (lds_void*)(bst + (wave * 4 + i) * 1024);
        if constexpr (decltype(full)::value)
          dma16(rsrc_b, dst, b_off[i], k0 * g.ldb * 2);
        else
          dma16(rsrc_b, dst, dma_offset(k0 + b_row[i] < g.K, b_off[i] + k0 * g.ldb * 2));
      }
    }
  };

  // Fragment addresses (bytes within a stage).
  int fa_addr[2][kMi], fb_addr[2][kNi][2];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
    for (int mi = 0; mi < kMi; ++mi) {
      const int row = wm * (TM / 2) + mi * 32 + (lane & 31);
      const int c = kk * 2 + (lane >> 5);
      // A2: the first tile of the pair; the second's chunk is c + 4, which
      // flips bit 2 of the physical chunk (address bit 6).
      fa_addr[kk][mi] = A2 ? row * 128 + a2_chunk_swz(row, c) * 16 : row * 64 + a_chunk_swz(row, c) * 16;
    }
#pragma unroll
    for (int ni = 0; ni < kNi; ++ni) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int sl = lane & 15, grp = lane >> 4;
        const int krow = kk * 16 + 8 * (grp >> 1) + 4 * h + (sl >> 2);
        const int ncol = wn * (TN / 2) + ni * 32 + 16 * (grp & 1) + 4 * (sl & 3);
        fb_addr[kk][ni][h] = (A2 ? 0 : kABytes) + krow * 512 + b_chunk_swz(krow, ncol >> 3) * 16 + (ncol & 7) * 2;
      }
    }
  }

  auto read_frags = [&](auto sc, int kk, u32x4 (&fa)[kMi], u32x4 (&fb)[kNi]) {
    constexpr int S = decltype(sc)::value;
    const unsigned char* ast;
    const unsigned char* bst;
    if constexpr (A2) {
      ast = a2_dstage<(S >> 1) & 1>();
      bst = b2_stage<S>();
    } else {
      ast = bst = dma_stage<TM, S>();
    }
    constexpr int kHalf = (A2 && (S & 1)) ? 64 : 0;  // A2: second tile of the pair
#pragma unroll
    for (int mi = 0; mi < kMi; ++mi) fa[mi] = *reinterpret_cast<const u32x4*>(ast + (fa_addr[kk][mi] ^ kHalf));
#pragma unroll
    for (int ni = 0; ni < kNi; ++ni) {
      const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4*)(bst + fb_addr[kk][ni][0]));
      const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4*)(bst + fb_addr[kk][ni][1]));
      const uint64_t l64 = __builtin_bit_cast(uint64_t, lo), h64 = __builtin_bit_cast(uint64_t, hi);
      fb[ni] = u32x4{(uint32_t)l64, (uint32_t)(l64 >> 32), (uint32_t)h64, (uint32_t)(h64 >> 32)};
    }
  };

  // KT: clear the A fragment elements at k >= K of 16-wide K step kk of
  // tile kt (a lane's fragment holds 8 consecutive k of one row; word w
  // holds elements 2w and 2w + 1).
  auto mask_tail = [&](u32x4 (&fa)[kMi], int kt, int kk) {
    const int v = min(max(g.K - (kt * kDmaK + kk * 16 + (lane >> 5) * 8), 0), 8);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t m = (2 * w < v ? 0x0000ffffu : 0u) | (2 * w + 1 < v ? 0xffff0000u : 0u);
#pragma unroll
      for (int mi = 0; mi < kMi; ++mi) fa[mi][w] &= m;
    }
  };

  f32x16 acc[kMi][kNi];
#pragma unroll
  for (int i = 0; i < kMi; ++i)
#pragma unroll
    for (int j = 0; j < kNi; ++j) acc[i][j] = f32x16{};

  auto mfma_block = [&](const u32x4 (&fa)[kMi], const u32x4 (&fb)[kNi]) {
#pragma unroll
    for (int mi = 0; mi < kMi; ++mi)
#pragma unroll
      for (int ni = 0; ni < kNi; ++ni) acc[mi][ni] = mfma32x32x16<DT>(fa[mi], fb[ni], acc[mi][ni]);
  };

  constexpr int kReads = kMi + 2 * kNi;  // LDS reads per 16-wide K step
  constexpr int kMfmas = kMi * kNi;      // MFMAs per 16-wide K step
  u32x4 fa0[kMi], fb0[kNi], fa1[kMi], fb1[kNi];

  // Instruction order of one 16-wide K step: fragment reads two at a time
  // behind the first MFMAs, and nv DMA loads spread evenly over the step
  // (bunched DMA issue stalls the wave on the address path).
  // DMA load v of nv goes behind MFMA slot v*kMfmas/nv (+1 when the slots
  // are at least two apart, so the first load does not share the first
  // slot with two fragment reads).
  auto schedule = [&](auto nv_c) {
    constexpr int nv = decltype(nv_c)::value;
    constexpr int shift = kMfmas >= 2 * nv ? 1 : 0;
#pragma unroll
    for (int m = 0; m < kMfmas; ++m) {
      __builtin_amdgcn_sched_group_barrier(kSgMfma, 1, 0);
      if (2 * m < kReads) __builtin_amdgcn_sched_group_barrier(kSgDsRead, 2, 0);
      int loads = 0;
      if constexpr (nv > 0) {
#pragma unroll
        for (int v = 0; v < nv; ++v) loads += (v * kMfmas / nv + shift == m) ? 1 : 0;
      }
      if (loads == 1) __builtin_amdgcn_sched_group_barrier(kSgVmemRead, 1, 0);
      if (loads == 2) __builtin_amdgcn_sched_group_barrier(kSgVmemRead, 2, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  // One K tile from stage S.  On entry fa0/fb0 hold its first 16-wide K
  // step; on exit they hold the next tile's.  A stage is refilled as soon
  // as the barrier after its last fragment reads has passed: tile
  // kt + STAGES goes into stage S, its A part after this tile's barrier
  // and its B part before the next one.  kFull: both tiles requested here
  // (B of kt + STAGES - 1, A of kt + STAGES) lie wholly inside K; tiles
  // past K load zeros and are never multiplied.
  auto iteration = [&](auto sc, auto full, int kt) {
    constexpr int S = decltype(sc)::value;
    // (Tiles read by full iterations lie wholly inside K: no tail mask.)
    constexpr bool kMask = KT && !decltype(full)::value;
    read_frags(sc, 1, fa1, fb1);
    if constexpr (kMask) mask_tail(fa1, kt, 1);
    issue_b(StageC<(S + STAGES - 1) % STAGES>{}, full, kt + STAGES - 1);
    mfma_block(fa0, fb0);
    schedule(std::integral_constant<int, 4>{});
    // Tile kt+1 has landed for this wave (the two tiles requested after it
    // may still be in flight); this wave's fragment reads of tile kt are
    // complete.  A2: after tile kt+1's last load this wave issued the B
    // parts of kt+2 and kt+3, and for even kt also the A pair (kt+2, kt+3).
    if constexpr (A2)
      wait_vmcnt<(S & 1) ? 8 : 8 + kADma2>();
    else
      wait_vmcnt<(STAGES - 2) * kDmaPerWave>();
    wait_lgkm0();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    // Every wave is past its reads of tile kt: stage S takes tile kt+STAGES
    // (A2: after odd kt, the A double stage of kt-1 and kt takes the pair
    // kt+3, kt+4).
    read_frags(StageC<(S + 1) % STAGES>{}, 0, fa0, fb0);
    if constexpr (kMask) mask_tail(fa0, kt + 1, 0);
    if constexpr (!A2) {
      issue_a(sc, full, kt + STAGES);
      mfma_block(fa1, fb1);
      schedule(std::integral_constant<int, kADma>{});
    } else if constexpr (S & 1) {
      issue_a2(std::integral_constant<int, (S >> 1) & 1>{}, full, kt + 3);
      mfma_block(fa1, fb1);
      schedule(std::integral_constant<int, kADma2>{});
    } else {
      mfma_block(fa1, fb1);
      schedule(std::integral_constant<int, 0>{});
    }
  };

  // Prologue: tiles 0..STAGES-2 and the A part of tile STAGES-1 in flight
  // (A2: A pairs (0, 1) and (2, 3), B of tiles 0..2); wait for tile 0.
  if constexpr (A2) {
    issue_a2(std::integral_constant<int, 0>{}, std::false_type{}, 0);
    issue_b(StageC<0>{}, std::false_type{}, 0);
    issue_b(StageC<1>{}, std::false_type{}, 1);
    issue_b(StageC<2>{}, std::false_type{}, 2);
    issue_a2(std::integral_constant<int, 1>{}, std::false_type{}, 2);
    wait_vmcnt<8 + kADma2>();
  } else {
    issue_a(StageC<0>{}, std::false_type{}, 0);
    issue_b(StageC<0>{}, std::false_type{}, 0);
    issue_a(StageC<1>{}, std::false_type{}, 1);
    issue_b(StageC<1>{}, std::false_type{}, 1);
    if constexpr (STAGES == 4) {
      issue_a(StageC<2>{}, std::false_type{}, 2);
      issue_b(StageC<2>{}, std::false_type{}, 2);
    }
    issue_a(StageC<STAGES - 1>{}, std::false_type{}, STAGES - 1);
    wait_vmcnt<(STAGES - 2) * kDmaPerWave + kADma>();
  }
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  stamps.mark(1);
  read_frags(StageC<0>{}, 0, fa0, fb0);
  if constexpr (KT) mask_tail(fa0, 0, 0);

  using Full = std::true_type;
  using Checked = std::false_type;
  int kt = 0;
  // Trips whose requested tiles (kt + STAGES - 1 .. kt + 2 * STAGES - 1)
  // all lie inside K, then the checked remainder.
  const int nfull = g.K / kDmaK;
  for (; kt + 2 * STAGES <= nfull; kt += STAGES) {
    iteration(StageC<0>{}, Full{}, kt);
    iteration(StageC<1>{}, Full{}, kt + 1);
    iteration(StageC<2>{}, Full{}, kt + 2);
    if constexpr (STAGES == 4) iteration(StageC<3 % STAGES>{}, Full{}, kt + 3);
  }
  for (; kt + STAGES <= nk; kt += STAGES) {
    iteration(StageC<0>{}, Checked{}, kt);
    iteration(StageC<1>{}, Checked{}, kt + 1);
    iteration(StageC<2>{}, Checked{}, kt + 2);
    if constexpr (STAGES == 4) iteration(StageC<3 % STAGES>{}, Checked{}, kt + 3);
  }
  if (kt < nk) iteration(StageC<0>{}, Checked{}, kt++);
  if (kt < nk) iteration(StageC<1>{}, Checked{}, kt++);
  if constexpr (STAGES == 4)
    if (kt < nk) iteration(StageC<2>{}, Checked{}, kt++);
  // No DMA may still be writing LDS when the workgroup retires.
  wait_vmcnt<0>();
  stamps.mark(2);

  // Epilogue.  The accumulators go through LDS so that C leaves in full
  // 512-byte row segments (32 lanes x 16 bytes) instead of 4-byte scatters.
  // 32x32 accumulator layout: register r of lane l holds row
  // 8*(r/4) + 4*(l/32) + r%4, column l%32, so registers 0-7 cover rows 0-15
  // and 8-15 rows 16-31.  Each wave stages 16 rows x 128 columns at a time in
  // its own 8.5 KB slice of the (now idle) stage memory; rows are padded to
  // 136 floats so the two 32-lane halves of each 4-byte write land on
  // disjoint banks.
  __builtin_amdgcn_s_barrier();  // every wave is done reading the stages
  constexpr int kEpRow = 136;     // floats per staged row
  unsigned char* ep_base;
  if constexpr (A2)
    ep_base = wave < 2 ? a2_dstage<0>() : a2_dstage<1>();
  else
    ep_base = wave < 2 ? dma_stage<TM, 0>() : dma_stage<TM, 1>();
  float* ep = reinterpret_cast<float*>(ep_base + (wave & 1) * (16 * kEpRow * 4));
  const bool full = g.c_vec && (m0 + TM <= g.M) && (n0 + TN <= g.N);
  const int col_l = lane & 31;
  const int row_l = (lane >> 5) * 4;
  const int c4 = (lane & 31) * 4;
  const int gcol = n0 + wn * (TN / 2) + c4;
  const bool col_live = c4 < TN / 2;  // lanes past the wave's TN/2 columns store nothing
#pragma unroll
  for (int mi = 0; mi < kMi; ++mi) {
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
      for (int ni = 0; ni < kNi; ++ni)
#pragma unroll
        for (int r = 8 * hh; r < 8 * hh + 8; ++r)
          ep[(((r >> 2) & 1) * 8 + row_l + (r & 3)) * kEpRow + ni * 32 + col_l] = acc[mi][ni][r];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      if (full) {
        // Lane l stores columns 4*(l%32) .. +3 of staged rows 2*i + l/32.
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int lr = 2 * i + (lane >> 5);
          const f32x4 v = *reinterpret_cast<const f32x4*>(ep + lr * kEpRow + c4);
          const int grow = m0 + wm * (TM / 2) + mi * 32 + hh * 16 + lr;
          float* dst = g.C + (int64_t)grow * g.ldc + gcol;
          if (col_live) __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(dst));
        }
      } else if (g.c_vec && (g.N & 3) == 0) {
        // Edge tiles of 16-byte aligned C rows with N a multiple of 4 (every
        // chunk whole): non-temporal as in full tiles, rows past M and chunks
        // past N skipped.  Plain stores leave dirty L2 lines that the end of
        // the launch must write back: 4096 x 3008 x 1024 took 34.1-34.4 us per
        // launch with its last tile column stored plainly, 31.7 us this way
        // (per-workgroup stamps: 7.6 -> 4.1 us from the last workgroup's end
        // to the next launch's start).  A chunk straddling N would mix plain
        // element stores into a line written non-temporally, which cost more
        // (2000 x 3003 x 1000, ldc 3004: 24.1 -> 25.5 us), so those tiles
        // keep the path below.
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int lr = 2 * i + (lane >> 5);
          const f32x4 v = *reinterpret_cast<const f32x4*>(ep + lr * kEpRow + c4);
          const int grow = m0 + wm * (TM / 2) + mi * 32 + hh * 16 + lr;
          float* dst = g.C + (int64_t)grow * g.ldc + gcol;
          if (col_live && grow < g.M && gcol < g.N) __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(dst));
        }
      } else {
        // C rows without 16-byte alignment: the same lane layout, 16-byte
        // stores at 4-byte aligned addresses (C is float, so every address
        // is; gfx950 takes unaligned vector stores), rows past M skipped and
        // a chunk reaching past N stored element by element.  (4-byte stores
        // of one column per lane ran 1.4 us slower on 4095 x 3001 x 1027,
        // whose C rows are 12004 bytes apart; non-temporal stores at these
        // addresses, or write-through ones, made its epilogue 5-13 us longer.)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int lr = 2 * i + (lane >> 5);
          const int grow = m0 + wm * (TM / 2) + mi * 32 + hh * 16 + lr;
          const f32x4 v = *reinterpret_cast<const f32x4*>(ep + lr * kEpRow + c4);
          float* dst = g.C + (int64_t)grow * g.ldc + gcol;
          if (col_live && grow < g.M) {
            if (gcol + 3 < g.N) {
              *reinterpret_cast<f32x4u*>(dst) = v;
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (gcol + e < g.N) dst[e] = v[e];
            }
          }
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }
  stamps.write();
}

// Copies of up to two rows x cols 16-bit matrices (row stride ld) into
// zero-padded copies with row stride ld_out (a multiple of 8), so the DMA
// kernels can use aligned 128-bit loads.  Columns [cols, ld_out) become 0.
struct RepackJob {
  const uint16_t* src;
  int64_t ld;
  int rows, cols;
  uint16_t* dst;
  int ld_out;
  int64_t chunks;  // rows * ld_out / 8
};

// Bytes [o, o + 16) of the 32 bytes w0:w1 (o even, 0 .. 14): a word rotate
// by o / 4 (two selects, on named registers so that no register array is
// indexed dynamically) and a byte funnel shift by o % 4.
__device__ __forceinline__ u32x4 shift_join(u32x4 w0, u32x4 w1, int o) {
  const uint32_t a0 = w0[0], a1 = w0[1], a2 = w0[2], a3 = w0[3], a4 = w1[0], a5 = w1[1], a6 = w1[2], a7 = w1[3];
  const bool s1 = (o >> 2) & 1, s2 = (o >> 3) & 1;
  const uint32_t b0 = s2 ? a2 : a0, b1 = s2 ? a3 : a1, b2 = s2 ? a4 : a2, b3 = s2 ? a5 : a3, b4 = s2 ? a6 : a4,
                 b5 = s2 ? a7 : a5;
  const uint32_t c0 = s1 ? b1 : b0, c1 = s1 ? b2 : b1, c2 = s1 ? b3 : b2, c3 = s1 ? b4 : b3, c4 = s1 ? b5 : b4;
  const int bs = o & 3;
  return u32x4{__builtin_amdgcn_alignbyte(c1, c0, bs), __builtin_amdgcn_alignbyte(c2, c1, bs),
               __builtin_amdgcn_alignbyte(c3, c2, bs), __builtin_amdgcn_alignbyte(c4, c3, bs)};
}

// Output chunks (8 elements, 16 bytes) per thread, gridDim.x * 256 apart;
// all their loads are issued before any is shifted and stored.
constexpr int kRepackPer = 2;

// Each output chunk's source bytes are addressed from the 16-byte boundary
// at or below src ("aligned bytes"): the chunk starts at aligned byte
// 2f + pre (f = flat element index, pre = src's offset in its 16-byte
// block) and lies in aligned chunks q and q + 1, both read with aligned
// 16-byte loads and joined by shift_join.  Chunk q + 1 is read only when it
// holds a byte of the operand (a 16-byte chunk never crosses a page, so one
// holding any valid byte can be read whole); elements past the row's
// `cols` are cleared after the join.
__global__ __launch_bounds__(256) void repack_kernel(RepackJob a, RepackJob b) {
  const int64_t n = a.chunks + b.chunks;
  const int64_t stride = (int64_t)gridDim.x * 256;
  const int64_t first = (int64_t)blockIdx.x * 256 + threadIdx.x;
  u32x4 w0[kRepackPer], w1[kRepackPer];
  int o[kRepackPer], valid[kRepackPer];
  uint16_t* dst[kRepackPer];
#pragma unroll
  for (int i = 0; i < kRepackPer; ++i) {
    int64_t idx = first + i * stride;
    dst[i] = nullptr;
    valid[i] = 0;
    o[i] = 0;
    w0[i] = u32x4{0, 0, 0, 0};
    w1[i] = u32x4{0, 0, 0, 0};
    if (idx >= n) continue;
    const bool in_a = idx < a.chunks;
    if (!in_a) idx -= a.chunks;
    const uint16_t* src = in_a ? a.src : b.src;
    const int64_t ld = in_a ? a.ld : b.ld;
    const int rows = in_a ? a.rows : b.rows;
    const int cols = in_a ? a.cols : b.cols;
    const int ld_out = in_a ? a.ld_out : b.ld_out;
    // chunks < 2^27 (a repacked operand stays below 2^31 bytes), so 32-bit
    // division suffices.
    const uint32_t per_row = (uint32_t)ld_out / 8;
    const int row = (int)((uint32_t)idx / per_row);
    const int c0 = (int)((uint32_t)idx - (uint32_t)row * per_row) * 8;
    dst[i] = (in_a ? a.dst : b.dst) + (int64_t)row * ld_out + c0;
    valid[i] = cols - c0;
    if (c0 >= cols) continue;
    const uintptr_t base = reinterpret_cast<uintptr_t>(src) & ~(uintptr_t)15;
    const int pre = (int)(reinterpret_cast<uintptr_t>(src) & 15);
    const int64_t start = ((int64_t)row * ld + c0) * 2 + pre;
    const int64_t last = (((int64_t)rows - 1) * ld + cols) * 2 - 1 + pre;
    const int64_t q = start >> 4;
    o[i] = (int)(start & 15);
    const u32x4* p = reinterpret_cast<const u32x4*>(base) + q;
    w0[i] = p[0];
    if (o[i] != 0 && (q + 1) * 16 <= last) w1[i] = p[1];
  }
#pragma unroll
  for (int i = 0; i < kRepackPer; ++i) {
    if (dst[i] == nullptr) continue;
    u32x4 out = u32x4{0, 0, 0, 0};
    if (valid[i] > 0) {
      out = shift_join(w0[i], w1[i], o[i]);
      if (valid[i] < 8) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          if (2 * k >= valid[i]) out[k] = 0;
          else if (2 * k + 1 >= valid[i]) out[k] &= 0xffffu;
        }
      }
    }
    *reinterpret_cast<u32x4*>(dst[i]) = out;
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
  af = (arow < g.M) ? load_row8_u16<kVecA>(g.A + (int64_t)arow * g.lda, kr, g.K) : u32x4{0, 0, 0, 0};
  const bool full = kVecB && (k0 + kSkinnyStep <= g.K) && (ncol0 + 8 <= g.N);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int k = kr + i;
    const uint16_t* p = g.B + (int64_t)k * g.ldb;
    if (full) {
      rb[i] = *reinterpret_cast<const u32x4*>(p + ncol0);
    } else {
      rb[i] = (k < g.K) ? load_row8_u16<kVecB>(p, ncol0, g.N) : u32x4{0, 0, 0, 0};
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

// ---------------------------------------------------------------------------
// Streaming skinny kernel: B through LDS by DMA, split-K with an in-order
// reduction
// ---------------------------------------------------------------------------
//
// Workgroup (256 threads) = NB = 128 columns x kchunk rows of B.  B moves
// HBM -> LDS with buffer_load ... lds in 32-row stages (8 KB, 256-byte row
// segments, the strip width that streams best on this part), kStStages deep.
// Wave w owns columns 32w .. 32w+31: per stage it reads its B operands with
// transposing LDS loads (ds_read_b64_tr_b16) and issues 2 MFMA 16x16x32
// against each of the R 16-row blocks of A (R = 1, 2, 4, 8 for M up to 16,
// 32, 64, 128; rows >= M read as zero), so every B fragment read from LDS
// feeds R MFMAs.  Each block's 16x32 slice of a stage arrives by one more
// DMA instruction (block rb from wave rb % 4).
//
// Split-K partials go to a workspace [splits][16 R][N].  With at most
// kStFuseMaxSplits(R) splits, R <= 2 and N a multiple of 4 the workgroups of a
// column block reduce them themselves: each publishes its partial with
// agent-scope (L2-coherent across XCDs) stores and counts its arrival on the
// column block's counter; the last to arrive sums the partials in order
// s = 0..S-1, writes C and resets the counter.  Otherwise (and for the
// allocation-free entry point, which has no counters) stream_reduce_kernel
// sums them in a second launch, in the same order: results are bit-identical
// either way.

constexpr int kStN = 128;
constexpr int kStStep = 32;
constexpr int kStStages = 8;
constexpr int kStBBytes = kStStep * kStN * 2;  // 8 KB
constexpr int kStABytes = 16 * kStStep * 2;    // 1 KB per 16-row block of A
constexpr int kStMaxRowBlocks = 8;              // M <= 128
constexpr int kStMaxSplits = 16;      // partials stream_reduce_kernel holds in registers
// Splits the in-kernel reduction takes with R row blocks (its registers
// hold every other split's partial; more would cost the kernel occupancy).
constexpr int kStFuseMaxSplits(int R) { return R == 1 ? 8 : 4; }
constexpr int kStCounterBytes = 16384;  // arrival counters ahead of each workspace: 4096 column blocks
// Cache policy of a buffer access coherent at agent scope on gfx950 (SC1):
// the bits the compiler gives a relaxed agent-scope atomic load or store.
constexpr int kCpolAgent = 16;
constexpr int kStMaxSplitsLoop = 256;  // K splits at all (more than 16: split_reduce_kernel)

struct StreamArgs {
  const uint16_t* A;
  const uint16_t* B;
  float* C;
  float* ws;      // [splits][16 * row blocks][N] partial sums (splits > 1)
  int lda, ldb;   // elements (any pitch: rows are read at any 2-byte alignment)
  int64_t ldc;
  int M, N, K;
  int kchunk;     // rows per split, multiple of kStStep
  int splits;     // 1 .. kStMaxSplitsLoop
  int rblocks;    // 16-row blocks of A: 1, 2, 4 or 8 (M <= 16 * rblocks)
  int a_bytes, b_bytes;
  bool c_vec;     // C rows 16-byte aligned at every 4th column
  unsigned* counters;  // per column block arrival counters (all zero between launches), or null
  int ws_bytes;        // bytes of the partials (with counters: below 2^31)
#ifdef HCG_STAMPS
  int stamp_slot;
#endif
};

#define HCG_ST_STAGE(i) \
  __shared__ __attribute__((aligned(1024))) unsigned char g_stb##i[kStBBytes];
HCG_ST_STAGE(0)
HCG_ST_STAGE(1)
HCG_ST_STAGE(2)
HCG_ST_STAGE(3)
HCG_ST_STAGE(4)
HCG_ST_STAGE(5)
HCG_ST_STAGE(6)
HCG_ST_STAGE(7)
#undef HCG_ST_STAGE
// A stages, one set per row-block count R (a kernel allocates only its own).
#define HCG_ST_ASTAGES(r)                                                                  \
  __shared__ __attribute__((aligned(1024))) unsigned char g_sta##r##_0[kStABytes * r];   \
  __shared__ __attribute__((aligned(1024))) unsigned char g_sta##r##_1[kStABytes * r];   \
  __shared__ __attribute__((aligned(1024))) unsigned char g_sta##r##_2[kStABytes * r];   \
  __shared__ __attribute__((aligned(1024))) unsigned char g_sta##r##_3[kStABytes * r];   \
  __shared__ __attribute__((aligned(1024))) unsigned char g_sta##r##_4[kStABytes * r];   \
  __shared__ __attribute__((aligned(1024))) unsigned char g_sta##r##_5[kStABytes * r];   \
  __shared__ __attribute__((aligned(1024))) unsigned char g_sta##r##_6[kStABytes * r];   \
  __shared__ __attribute__((aligned(1024))) unsigned char g_sta##r##_7[kStABytes * r];
HCG_ST_ASTAGES(1)
HCG_ST_ASTAGES(2)
HCG_ST_ASTAGES(4)
HCG_ST_ASTAGES(8)
#undef HCG_ST_ASTAGES

template <int S>
__device__ __forceinline__ unsigned char* st_b() {
  if constexpr (S == 0) return g_stb0;
  else if constexpr (S == 1) return g_stb1;
  else if constexpr (S == 2) return g_stb2;
  else if constexpr (S == 3) return g_stb3;
  else if constexpr (S == 4) return g_stb4;
  else if constexpr (S == 5) return g_stb5;
  else if constexpr (S == 6) return g_stb6;
  else return g_stb7;
}
#define HCG_ST_ASEL(r)                          \
  if constexpr (S == 0) return g_sta##r##_0;     \
  else if constexpr (S == 1) return g_sta##r##_1; \
  else if constexpr (S == 2) return g_sta##r##_2; \
  else if constexpr (S == 3) return g_sta##r##_3; \
  else if constexpr (S == 4) return g_sta##r##_4; \
  else if constexpr (S == 5) return g_sta##r##_5; \
  else if constexpr (S == 6) return g_sta##r##_6; \
  else return g_sta##r##_7;
template <int R, int S>
__device__ __forceinline__ unsigned char* st_a() {
  static_assert(R == 1 || R == 2 || R == 4 || R == 8, "row blocks");
  if constexpr (R == 1) {
    HCG_ST_ASEL(1)
  } else if constexpr (R == 2) {
    HCG_ST_ASEL(2)
  } else if constexpr (R == 4) {
    HCG_ST_ASEL(4)
  } else {
    HCG_ST_ASEL(8)
  }
}
#undef HCG_ST_ASEL

// A stage: 16 rows x 32 k (64-byte rows of 4 chunks); chunk c of row r is
// stored at c ^ ((r >> 2) & 3), so the 16 rows read at one chunk hit 16
// distinct 16-byte bank groups.
__device__ __forceinline__ int sta_swz(int row, int c) { return c ^ ((row >> 2) & 3); }

// The split-K reduction inside the streaming kernel (R <= 2 row blocks,
// N % 4 == 0, splits <= kStFuseMaxSplits(R); the host checks).  Called by every
// thread of the workgroup of (column block nb, split) after its K loop,
// with the wave's 16x16 accumulators (register r of lane l: row 4 (l/16) + r,
// column l%16 of the wave's column block j).
template <int R>
__device__ __forceinline__ void stream_fused_reduce(const StreamArgs& g, const f32x4 (&acc)[R][kStN / 64],
                                                    int nb, int split) {
  constexpr int NB = kStN;
  constexpr int kColsPerWave = NB / 4;
  constexpr int kBlocks = kColsPerWave / 16;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n0 = nb * NB;
  // The arrival count is broadcast through B stage 7 (free after the K loop;
  // a separate LDS variable would push two R = 2 workgroups past the CU's
  // 160 KB).
  unsigned* s_arrived = reinterpret_cast<unsigned*>(st_b<kStStages - 1>());
  // Stage the 16R x 128 partial through LDS (row block rb in B stage rb:
  // 16 x 128 floats = 8 KB), so that each thread then holds two whole
  // 16-byte row pieces.  Every wave has finished reading the stages.
  __syncthreads();
#pragma unroll
  for (int rb = 0; rb < R; ++rb) {
    float* ep = reinterpret_cast<float*>(rb == 0 ? st_b<0>() : st_b<1>());
#pragma unroll
    for (int j = 0; j < kBlocks; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        ep[((lane >> 4) * 4 + r) * NB + wave * kColsPerWave + 16 * j + (lane & 15)] = acc[rb][j][r];
  }
  __syncthreads();
  // Piece c (of 512 per row block): row c / 32, columns 4 (c % 32) .. +3.
  // N % 4 == 0, so a piece is either wholly inside N or wholly past it.
  const __amdgpu_buffer_rsrc_t rws = make_rsrc(g.ws, g.ws_bytes);
  u32x4 mine[R][2];
#pragma unroll
  for (int rb = 0; rb < R; ++rb)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = tid + 256 * h, row = c >> 5, col = n0 + (c & 31) * 4;
      const float* ep = reinterpret_cast<const float*>(rb == 0 ? st_b<0>() : st_b<1>());
      mine[rb][h] = *reinterpret_cast<const u32x4*>(ep + row * NB + (c & 31) * 4);
      if (col < g.N)
        __builtin_amdgcn_raw_buffer_store_b128(mine[rb][h], rws,
                                               (int)((((int64_t)split * 16 * R + 16 * rb + row) * g.N + col) * 4), 0,
                                               kCpolAgent);
    }
  // The partial is visible at agent scope once its stores have completed;
  // only then is the arrival counted.
  wait_vmcnt<0>();
  __syncthreads();
  if (tid == 0) *s_arrived = __hip_atomic_fetch_add(g.counters + nb, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (*s_arrived != (unsigned)(g.splits - 1)) return;
  // Last arrival: every other split's partial is complete.  The counter is
  // reset for the next launch (which follows this one in stream order).
  if (tid == 0) __hip_atomic_store(g.counters + nb, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  constexpr int kMaxSplits = kStFuseMaxSplits(R);
  u32x4 part[kMaxSplits][R][2];
#pragma unroll
  for (int sp = 0; sp < kMaxSplits; ++sp)
#pragma unroll
    for (int rb = 0; rb < R; ++rb)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int c = tid + 256 * h, row = c >> 5, col = n0 + (c & 31) * 4;
        part[sp][rb][h] = u32x4{0, 0, 0, 0};
        if (sp < g.splits && sp != split && col < g.N)
          part[sp][rb][h] = __builtin_amdgcn_raw_buffer_load_b128(
              rws, (int)((((int64_t)sp * 16 * R + 16 * rb + row) * g.N + col) * 4), 0, kCpolAgent);
      }
  // Sum in split order, as stream_reduce_kernel does.
#pragma unroll
  for (int rb = 0; rb < R; ++rb)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = tid + 256 * h, row = 16 * rb + (c >> 5), col = n0 + (c & 31) * 4;
      if (row >= g.M || col >= g.N) continue;
      f32x4 v = __builtin_bit_cast(f32x4, split == 0 ? mine[rb][h] : part[0][rb][h]);
#pragma unroll
      for (int sp = 1; sp < kMaxSplits; ++sp)
        if (sp < g.splits) v += __builtin_bit_cast(f32x4, sp == split ? mine[rb][h] : part[sp][rb][h]);
      float* dst = g.C + (int64_t)row * g.ldc + col;
      if (g.c_vec) {
        *reinterpret_cast<f32x4*>(dst) = v;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[e] = v[e];
      }
    }
}

// UB (B's last row piece not safely readable in place, so no DMA for B):
// each lane fetches the two aligned 16-byte blocks around its B chunk PF
// stages ahead into a register set of its own, and writes the chunk (shift_join of the
// two) just before that stage's barrier to the LDS bytes the DMA would have
// filled.  Every lane issues two loads per chunk (the wait counts double the
// B part): chunks past N or rows past the split's K range read B's first
// block and are cleared, and a second block past B's last byte is replaced
// by the first (its bytes reach only columns >= N).  Needs B 2-byte aligned
// and (K - 1) * ldb + N >= 8.
// PF: stages requested ahead of the one being multiplied (at most
// kStStages - 1).  Fewer bytes in flight stream faster here: C4 (16 x 8192 x
// 8192 fp16, B from HBM) takes 28.2 us with 7 stages ahead and 25.9 us with
// 3; see launch_stream().
template <int DT, int R, bool UB = false, int PF = kStStages - 1>
__global__ __launch_bounds__(256) void gemm_stream_kernel(StreamArgs g) {
  static_assert(PF >= 2 && PF < kStStages, "prefetch distance");
  static_assert(R >= 1 && R <= kStMaxRowBlocks, "row blocks");
  constexpr int NB = kStN;
  constexpr int kRowBytes = NB * 2;           // bytes per staged B row
  constexpr int kRowsPerDma = 1024 / kRowBytes;
  constexpr int kDmaPerWave = NB / 64;        // B DMA instructions per wave per stage
  constexpr int kColsPerWave = NB / 4;
  constexpr int kBlocks = kColsPerWave / 16;  // MFMA column blocks per wave

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Workgroup -> (column block, split).  Workgroups are dispatched
  // round-robin over the 8 XCDs (id % 8); the mapping gives every XCD, in
  // every split, column blocks of all 8 residues mod 8, so that no XCD
  // streams a fixed subset of B's 256-byte column positions.
  int nb, split;
  {
    const int id = blockIdx.x;
    const int per_split = gridDim.x / g.splits;  // column blocks (padded to a multiple of 8)
    split = id / per_split;
    const int r = id - split * per_split;
    const int x = r & 7, q = r >> 3;
    nb = 8 * q + ((x + q + split) & 7);
  }
  if (nb * NB >= g.N) return;
  WgStamps stamps(HCG_STAMP_SLOT(g));
  stamps.mark(0);
  const int n0 = nb * NB;
  const int kbeg = split * g.kchunk;
  const int kend = min(g.K, kbeg + g.kchunk);
  const int nsteps = (kend - kbeg + kStStep - 1) / kStStep;

  const __amdgpu_buffer_rsrc_t rsrc_a = make_rsrc(g.A, g.a_bytes);
  const __amdgpu_buffer_rsrc_t rsrc_b = make_rsrc(g.B, g.b_bytes);

  // DMA roles.  B: wave w fills row blocks w*kDmaPerWave + i of the stage;
  // lane l covers row kRowsPerDma*blk + l/(NB/8), physical chunk l%(NB/8).
  // A (wave 0): lane l covers row l/4, physical chunk l%4.  Rows past this
  // split's K range, rows past M and chunks past N go past the range check
  // and load zeros.
  int b_off[kDmaPerWave], b_row[kDmaPerWave];
#pragma unroll
  for (int i = 0; i < kDmaPerWave; ++i) {
    const int blk = wave * kDmaPerWave + i;
    const int kr = blk * kRowsPerDma + lane / (NB / 8);
    const int cb = b_chunk_swz(kr, lane % (NB / 8));
    b_row[i] = (n0 + cb * 8 < g.N) ? kr : 0x3fffffff;
    b_off[i] = (kr * g.ldb + n0 + cb * 8) * 2;
  }
  // A: 16-row block rb (of R) is loaded by wave rb % 4, lane l covering row
  // 16 rb + l/4 at physical chunk l%4; a wave loads kAPer or kAPer - 1 blocks.
  constexpr int kAPer = (R + 3) / 4;
  const int a_r = lane >> 2;
  const int a_c = sta_swz(a_r, lane & 3);
  bool a_ok[kAPer];
  int a_off[kAPer];
#pragma unroll
  for (int i = 0; i < kAPer; ++i) {
    const int row = 16 * (wave + 4 * i) + a_r;
    a_ok[i] = wave + 4 * i < R && row < g.M;
    a_off[i] = (row * g.lda + a_c * 8) * 2;
  }

  // UB: register sets of the stages in flight (the two aligned 16-byte
  // blocks around each chunk), and per chunk its byte offset in the first
  // block, or -1 for a cleared chunk.
  u32x4 breg[UB ? kStStages : 1][kDmaPerWave][2];
  int bsh[UB ? kStStages : 1][kDmaPerWave];
  u32x4 areg[UB ? kStStages : 1][kAPer];
  bool alive[UB ? kStStages : 1][kAPer];
  const uintptr_t b_base = reinterpret_cast<uintptr_t>(g.B);
  const uintptr_t b_end = b_base + ((uintptr_t)(g.K - 1) * g.ldb + g.N) * 2;  // one past B's last byte

  auto issue = [&](auto sc, int step) {
    constexpr int S = decltype(sc)::value;
    const int k0 = kbeg + step * kStStep;
    if constexpr (UB) {
#pragma unroll
      for (int i = 0; i < kDmaPerWave; ++i) {
        const int row = k0 + (wave * kDmaPerWave + i) * kRowsPerDma + lane / (NB / 8);
        const int col = n0 + b_chunk_swz(row - k0, lane % (NB / 8)) * 8;
        const bool live = row < kend && col < g.N;
        // Selects, not branches: a branch around the address math lets the
        // compiler's wait insertion fall back to waiting for every load.
        const int row_c = live ? row : 0, col_c = live ? col : 0;
        const uintptr_t p = b_base + ((uintptr_t)((uint64_t)(uint32_t)row_c * (uint32_t)g.ldb) + (uint32_t)col_c) * 2;
        const uintptr_t q = p & ~(uintptr_t)15;
        // The second block is read only when it holds a byte of B (a 16-byte
        // block never crosses a page); otherwise the first is read again.
        const uintptr_t q1 = q + 16 < b_end ? q + 16 : q;
        bsh[S][i] = live ? (int)(p - q) : -1;
        // Global (not generic) pointers: a flat load also counts on lgkmcnt,
        // so the wait for LDS writes before each barrier would drain it.
        using gvec = const __attribute__((address_space(1))) u32x4;
        breg[S][i][0] = *reinterpret_cast<gvec*>(q);
        breg[S][i][1] = *reinterpret_cast<gvec*>(q1);
      }
    } else {
#pragma unroll
      for (int i = 0; i < kDmaPerWave; ++i) {
        const int off = dma_offset(k0 + b_row[i] < kend, b_off[i] + k0 * g.ldb * 2);
        dma16(rsrc_b, (lds_void*)(st_b<S>() + (wave * kDmaPerWave + i) * 1024), off);
      }
    }
#pragma unroll
    for (int i = 0; i < kAPer; ++i) {
      if (wave + 4 * i < R) {
        const bool live = a_ok[i] && k0 + a_c * 8 < kend;
        if constexpr (UB) {
          // A through registers too: with an LDS DMA in flight the compiler
          // waits for it (and so for every older load) before LDS reads.
          using gvec = const __attribute__((address_space(1))) u32x4;
          const int off = live ? (a_off[i] + k0 * 2) / 2 : 0;
          areg[S][i] = *reinterpret_cast<gvec*>(reinterpret_cast<uintptr_t>(g.A + off));
          alive[S][i] = live;
        } else {
          dma16(rsrc_a, (lds_void*)(st_a<R, S>() + (wave + 4 * i) * kStABytes), dma_offset(live, a_off[i] + k0 * 2));
        }
      }
    }
  };

  // Fragment addresses.  A operand: row l%16, k chunk l/16.  B operand for
  // column block j of this wave, half h: source lane s = l%16 of group
  // q = l/16 points at k row 8q + 4h + s/4, column w*NB/4 + 16j + 4(s%4).
  const int fa = (lane & 15) * 64 + sta_swz(lane & 15, lane >> 4) * 16;
  int fb[kBlocks][2];
#pragma unroll
  for (int j = 0; j < kBlocks; ++j)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int sl = lane & 15, q = lane >> 4;
      const int krow = 8 * q + 4 * h + (sl >> 2);
      const int ncol = wave * kColsPerWave + 16 * j + 4 * (sl & 3);
      fb[j][h] = krow * kRowBytes + b_chunk_swz(krow, ncol >> 3) * 16 + (ncol & 7) * 2;
    }

  f32x4 acc[R][kBlocks];
#pragma unroll
  for (int rb = 0; rb < R; ++rb)
#pragma unroll
    for (int j = 0; j < kBlocks; ++j) acc[rb][j] = f32x4{};

  // kv: elements of the stage below K, counted from its first k.  Under K
  // (kv < kStStep: the last stage, when K is not a multiple of 8) the chunk
  // of A straddling K arrived whole; its elements past K (the next row, or
  // row padding that may hold NaN) are cleared.  Lane l's fragment holds
  // k = 8(l/16) .. +7 of the stage.
  auto compute = [&](auto sc, int kv) {
    constexpr int S = decltype(sc)::value;
    u32x4 af[R];
#pragma unroll
    for (int rb = 0; rb < R; ++rb) af[rb] = *reinterpret_cast<const u32x4*>(st_a<R, S>() + rb * kStABytes + fa);
    if (kv < kStStep) {
      const int v = min(max(kv - 8 * (lane >> 4), 0), 8);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t m = (2 * w < v ? 0x0000ffffu : 0u) | (2 * w + 1 < v ? 0xffff0000u : 0u);
#pragma unroll
        for (int rb = 0; rb < R; ++rb) af[rb][w] &= m;
      }
    }
#pragma unroll
    for (int j = 0; j < kBlocks; ++j) {
      const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4*)(st_b<S>() + fb[j][0]));
      const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4*)(st_b<S>() + fb[j][1]));
      const uint64_t l64 = __builtin_bit_cast(uint64_t, lo), h64 = __builtin_bit_cast(uint64_t, hi);
      const u32x4 bf = u32x4{(uint32_t)l64, (uint32_t)(l64 >> 32), (uint32_t)h64, (uint32_t)(h64 >> 32)};
#pragma unroll
      for (int rb = 0; rb < R; ++rb) acc[rb][j] = mfma16x16x32<DT>(af[rb], bf, acc[rb][j]);
    }
  };

  // One step from stage S: wait for it (this wave's DMAs; PF - 1 newer
  // stages may still be in flight), barrier (everyone's DMAs landed and
  // everyone finished with stage S + PF, last read PF - kStStages steps ago),
  // refill stage S + PF with step + PF, multiply.  Waves below R % 4 load
  // one more A block per stage than the others.
  constexpr int kLater = PF - 1;
  auto step_fn = [&](auto sc, int step) {
    constexpr int S = decltype(sc)::value;
    constexpr int kBLoads = UB ? 2 * kDmaPerWave : kDmaPerWave;  // B memory instructions per stage
    if constexpr (R % 4 == 0) {
      wait_vmcnt<(kBLoads + R / 4) * kLater>();
    } else if (wave < R % 4) {
      wait_vmcnt<(kBLoads + R / 4 + 1) * kLater>();
    } else {
      wait_vmcnt<(kBLoads + R / 4) * kLater>();
    }
    if constexpr (UB) {
      // This wave's B chunks of the stage have landed in registers.
#pragma unroll
      for (int i = 0; i < kDmaPerWave; ++i) {
        const int sh = bsh[S][i];
        const u32x4 v = sh < 0 ? u32x4{0, 0, 0, 0} : shift_join(breg[S][i][0], breg[S][i][1], sh);
        *reinterpret_cast<u32x4*>(st_b<S>() + (wave * kDmaPerWave + i) * 1024 + lane * 16) = v;
      }
#pragma unroll
      for (int i = 0; i < kAPer; ++i)
        if (wave + 4 * i < R)
          *reinterpret_cast<u32x4*>(st_a<R, S>() + (wave + 4 * i) * kStABytes + lane * 16) =
              alive[S][i] ? areg[S][i] : u32x4{0, 0, 0, 0};
    }
    wait_lgkm0();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    issue(StageC<(S + PF) % kStStages>{}, step + PF);
    compute(sc, g.K - (kbeg + step * kStStep));
    __builtin_amdgcn_sched_barrier(0);
  };

  issue(StageC<0>{}, 0);
  issue(StageC<1>{}, 1);
  if constexpr (PF > 2) issue(StageC<2>{}, 2);
  if constexpr (PF > 3) issue(StageC<3>{}, 3);
  if constexpr (PF > 4) issue(StageC<4>{}, 4);
  if constexpr (PF > 5) issue(StageC<5>{}, 5);
  if constexpr (PF > 6) issue(StageC<6>{}, 6);

  stamps.mark(1);
  int step = 0;
  for (; step + kStStages <= nsteps; step += kStStages) {
    step_fn(StageC<0>{}, step);
    step_fn(StageC<1>{}, step + 1);
    step_fn(StageC<2>{}, step + 2);
    step_fn(StageC<3>{}, step + 3);
    step_fn(StageC<4>{}, step + 4);
    step_fn(StageC<5>{}, step + 5);
    step_fn(StageC<6>{}, step + 6);
    step_fn(StageC<7>{}, step + 7);
  }
  if (step < nsteps) step_fn(StageC<0>{}, step++);
  if (step < nsteps) step_fn(StageC<1>{}, step++);
  if (step < nsteps) step_fn(StageC<2>{}, step++);
  if (step < nsteps) step_fn(StageC<3>{}, step++);
  if (step < nsteps) step_fn(StageC<4>{}, step++);
  if (step < nsteps) step_fn(StageC<5>{}, step++);
  if (step < nsteps) step_fn(StageC<6>{}, step++);
  wait_vmcnt<0>();  // no DMA may still be writing LDS at exit
  stamps.mark(2);

  // 16x16 accumulator layout: register r of lane l holds row 4*(l/16) + r,
  // column l%16 of the block.
  const int ocol = n0 + wave * kColsPerWave + (lane & 15);
  if (g.splits == 1) {
#pragma unroll
    for (int rb = 0; rb < R; ++rb)
#pragma unroll
      for (int j = 0; j < kBlocks; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 16 * rb + (lane >> 4) * 4 + r, col = ocol + 16 * j;
          if (row < g.M && col < g.N) g.C[(int64_t)row * g.ldc + col] = acc[rb][j][r];
        }
    stamps.write();
    return;
  }
  if constexpr (R <= 2) {
    if (g.counters != nullptr) {
      stream_fused_reduce<R>(g, acc, nb, split);
      stamps.write();
      return;
    }
  }
#pragma unroll
  for (int rb = 0; rb < R; ++rb)
#pragma unroll
    for (int j = 0; j < kBlocks; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * rb + (lane >> 4) * 4 + r, col = ocol + 16 * j;
        if (col < g.N) g.ws[((int64_t)split * 16 * R + row) * g.N + col] = acc[rb][j][r];
      }
  stamps.write();
}

// ---------------------------------------------------------------------------
// Narrow-N streaming kernel: A through LDS by DMA in 256-byte row pieces
// ---------------------------------------------------------------------------
//
// For N <= 64 the product is bound by reading A (M x K) once, and the
// tiled kernel's 64-byte row pieces per 32-wide K step stream poorly.  Here
// a workgroup (256 threads) takes 64 rows of A over a run of K (split-K
// when the row blocks alone do not fill the chip); wave w owns rows
// 16w .. 16w+15 and all NB (16 or 32, >= N) columns.  A moves HBM -> LDS in
// stages of 128 k -- 256 bytes of each of the 64 rows, 16 KB -- kRsStages
// deep, and B's 128 x NB slice of each stage comes along (every workgroup
// reads all of B, which stays in L2).  Per stage a wave issues 4 x NB/16
// MFMA 16x16x32: A fragments by ds_read_b128 (row l%16, 8 k at chunk l/16,
// chunks XOR-swizzled by row), B fragments by two transposing reads as in
// the skinny streaming kernel.  Rows past M, k past the run and columns
// past N load as zero (range check or redirect); K need not be a multiple
// of 8 (the chunk straddling K is cleared past K in the last stage's
// fragments), nor N (the straddling chunk's extra columns only reach C
// columns >= N).

constexpr int kRsRows = 64;
constexpr int kRsStep = 128;
constexpr int kRsStages = 6;            // NB <= 32 (24 KB per stage)
constexpr int kRs64Stages = 5;          // NB = 64 (32 KB per stage: 160 KB, all of a CU's LDS)
constexpr int kRsABytes = kRsRows * kRsStep * 2;  // 16 KB
constexpr int kRsBBytes = kRsStep * 32 * 2;       // 8 KB (NB <= 32)
constexpr int kRsB64Bytes = kRsStep * 64 * 2;     // 16 KB (NB = 64)

struct RowStreamArgs {
  const uint16_t* A;
  const uint16_t* B;
  float* C;
  float* ws;      // [splits][M][N] partial sums (splits > 1)
  int lda, ldb;   // elements; multiples of 8 (lda not when A is register-staged)
  int64_t ldc;
  int M, N, K;
  int kchunk;     // K per split, multiple of kRsStep
  int splits;
  int a_bytes, b_bytes;
  int rot_groups;  // distinct start steps over the row blocks (>= the run's steps: every step)
};

#define HCG_RS_STAGE(i)                                                         \
  __shared__ __attribute__((aligned(1024))) unsigned char g_rsa##i[kRsABytes]; \
  __shared__ __attribute__((aligned(1024))) unsigned char g_rsb##i[kRsBBytes];
HCG_RS_STAGE(0)
HCG_RS_STAGE(1)
HCG_RS_STAGE(2)
HCG_RS_STAGE(3)
HCG_RS_STAGE(4)
HCG_RS_STAGE(5)
#undef HCG_RS_STAGE

// NB = 64: A and B of a stage in one object (a kernel allocates only the
// objects it names).
#define HCG_RS64_STAGE(i) \
  __shared__ __attribute__((aligned(1024))) unsigned char g_rsc##i[kRsABytes + kRsB64Bytes];
HCG_RS64_STAGE(0)
HCG_RS64_STAGE(1)
HCG_RS64_STAGE(2)
HCG_RS64_STAGE(3)
HCG_RS64_STAGE(4)
#undef HCG_RS64_STAGE

template <int NB, int S>
__device__ __forceinline__ unsigned char* rs_a() {
  if constexpr (NB == 64) {
    if constexpr (S == 0) return g_rsc0;
    else if constexpr (S == 1) return g_rsc1;
    else if constexpr (S == 2) return g_rsc2;
    else if constexpr (S == 3) return g_rsc3;
    else return g_rsc4;
  } else {
    if constexpr (S == 0) return g_rsa0;
    else if constexpr (S == 1) return g_rsa1;
    else if constexpr (S == 2) return g_rsa2;
    else if constexpr (S == 3) return g_rsa3;
    else if constexpr (S == 4) return g_rsa4;
    else return g_rsa5;
  }
}
template <int NB, int S>
__device__ __forceinline__ unsigned char* rs_b() {
  if constexpr (NB == 64) {
    return rs_a<NB, S>() + kRsABytes;
  } else {
    if constexpr (S == 0) return g_rsb0;
    else if constexpr (S == 1) return g_rsb1;
    else if constexpr (S == 2) return g_rsb2;
    else if constexpr (S == 3) return g_rsb3;
    else if constexpr (S == 4) return g_rsb4;
    else return g_rsb5;
  }
}

// UA (A's last row piece not safely readable in place, so no DMA for A):
// each lane loads the two aligned 16-byte blocks around its A chunk
// kRsStages - 1 stages ahead into registers, and just before the stage's
// barrier writes the funnel-shifted chunk, elements at k >= K cleared (the
// row padding may hold Inf or NaN), to the LDS bytes the DMA would fill.  B
// (in place, or repacked when its last piece is not readable) comes through
// registers too:
// with an LDS DMA in flight the compiler waits for it, and so for every
// older load, before LDS reads.  A second block past A's last byte is
// replaced by the first (its bytes are k >= K, cleared).
template <int DT, int NB, bool UA = false, int ST = 0>
__global__ __launch_bounds__(NB == 64 ? 512 : 256) void gemm_rowstream_kernel(RowStreamArgs g) {
  static_assert(NB == 16 || NB == 32 || NB == 64, "column block");
  // ST = 3 (NB <= 32, register-staged A): a 72 KB ring, so two workgroups
  // share a CU -- twice the waves to cover the register path's latency
  // (65536 x 13 x 4095 fp16: 155 -> 110 us; by DMA the 6-stage ring stays
  // ahead, 125 against 135 us at 65536 x 8 x 4096).
  constexpr int STAGES = ST ? ST : (NB == 64 ? kRs64Stages : kRsStages);
  static_assert(STAGES >= 3 && STAGES <= 6 && (NB < 64 || STAGES <= kRs64Stages), "stages");
  // NB = 64 runs 8 waves (512 threads): the waves of a pair share a 16-row
  // block and take 32 columns each, so a CU holds twice the waves at the
  // same LDS (the register-staged form needs them to cover its latency).
  constexpr int kWaves = NB == 64 ? 8 : 4;
  constexpr int kColSplit = kWaves / 4;            // waves per 16-row block
  constexpr int kRowsPerWave = kRsRows / kWaves;   // A rows each wave loads: 16 or 8
  constexpr int kAInst = kRowsPerWave / 4;         // A DMA instructions per wave per stage
  constexpr int kChunksB = NB / 8;                 // 16-byte chunks per staged B row
  constexpr int kRowsPerBDma = 64 / kChunksB;      // B rows per DMA instruction
  constexpr int kBDmaPerWave = kRsStep / kRowsPerBDma / kWaves;
  constexpr int kDmaPerWave = kAInst + kBDmaPerWave;
  constexpr int kLoadsPerWave = UA ? 2 * kAInst + kBDmaPerWave : kDmaPerWave;  // memory instructions per stage
  constexpr int kBlocks = NB / 16 / kColSplit;     // MFMA column blocks per wave
  static_assert(kBDmaPerWave >= 1 && kAInst >= 1, "work split");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nrb = (g.M + kRsRows - 1) / kRsRows;
  const int split = blockIdx.x / nrb;
  const int m0 = (blockIdx.x - split * nrb) * kRsRows;
  const int kbeg = split * g.kchunk;
  const int kend = min(g.K, kbeg + g.kchunk);
  const int nsteps = (kend - kbeg + kRsStep - 1) / kRsStep;

  const __amdgpu_buffer_rsrc_t rsrc_a = make_rsrc(g.A, g.a_bytes);
  const __amdgpu_buffer_rsrc_t rsrc_b = make_rsrc(g.B, g.b_bytes);

  // DMA roles.  A: wave w loads its kRowsPerWave rows from row
  // kRowsPerWave * w in kAInst instructions of 4 rows; lane l covers row
  // 4i + l/16 of them at physical chunk l%16, i.e. logical chunk
  // (l%16) ^ (row%16).  B: wave w loads kBDmaPerWave blocks of kRowsPerBDma
  // k rows; lane l covers row l / kChunksB, chunk l % kChunksB.
  int a_off[kAInst], a_col[kAInst];
#pragma unroll
  for (int i = 0; i < kAInst; ++i) {
    const int row = kRowsPerWave * wave + 4 * i + (lane >> 4);
    const int c = (lane & 15) ^ (row & 15);
    a_col[i] = c * 8;
    a_off[i] = UA ? 0 : ((m0 + row) * g.lda + c * 8) * 2;  // (UA reads through 64-bit pointers)
  }
  int b_off[kBDmaPerWave], b_row[kBDmaPerWave];
#pragma unroll
  for (int i = 0; i < kBDmaPerWave; ++i) {
    const int kr = (wave * kBDmaPerWave + i) * kRowsPerBDma + lane / kChunksB;
    const int cb = lane % kChunksB;
    b_row[i] = cb * 8 < g.N ? kr : 0x3fffffff;
    b_off[i] = (kr * g.ldb + cb * 8) * 2;
  }
  // UA: register sets of the stages in flight; per A chunk its byte offset
  // in the first block (-1: cleared) and its elements below K.
  using gvec = const __attribute__((address_space(1))) u32x4;
  u32x4 areg[UA ? STAGES : 1][kAInst][2];
  int ash[UA ? STAGES : 1][kAInst], avld[UA ? STAGES : 1][kAInst];
  u32x4 breg[UA ? STAGES : 1][kBDmaPerWave];
  bool bok[UA ? STAGES : 1][kBDmaPerWave];
  const uintptr_t a_base = reinterpret_cast<uintptr_t>(g.A), b_base = reinterpret_cast<uintptr_t>(g.B);
  const uintptr_t a_end = a_base + ((uintptr_t)(g.M - 1) * g.lda + g.K) * 2;  // one past A's last byte
  uintptr_t a_rowp[kAInst];
  bool a_rowok[kAInst];
#pragma unroll
  for (int i = 0; i < kAInst; ++i) {
    const int row = m0 + kRowsPerWave * wave + 4 * i + (lane >> 4);
    a_rowok[i] = row < g.M;
    a_rowp[i] = a_base + (uintptr_t)(a_rowok[i] ? row : 0) * (uintptr_t)g.lda * 2;
  }

  // Row block rb walks its run of K starting at step rb % nsteps (wrapping):
  // with all blocks starting at the same k, a power-of-two row stride puts
  // every concurrent 256-byte piece at the same address offset modulo the
  // stride, and the reads pile onto a few HBM channels (16384 x 8 x 16384
  // fp16: 146 us unrotated vs 103 us at K = 16392).  With 8 KB rows the
  // blocks start at 16 evenly spaced steps instead (rot_groups; 65536 x 8 x
  // 4096: 102 us, against 125 us at every step and 106 us unrotated).  Steps
  // past the run load zeros.
  const int rg = min(g.rot_groups, nsteps);
  const int rot = ((blockIdx.x - split * nrb) % rg) * (nsteps / rg);
  auto issue = [&](auto sc, int step) {
    constexpr int S = decltype(sc)::value;
    int s = step + rot;
    if (s >= nsteps) s -= nsteps;
    const int k0 = step < nsteps ? kbeg + s * kRsStep : kend;
    if constexpr (UA) {
#pragma unroll
      for (int i = 0; i < kAInst; ++i) {
        const int kc = k0 + a_col[i];  // the chunk's first k
        const bool live = a_rowok[i] && kc < kend;
        const uintptr_t p = live ? a_rowp[i] + (uintptr_t)kc * 2 : a_base;
        const uintptr_t q = p & ~(uintptr_t)15;
        const uintptr_t q1 = q + 16 < a_end ? q + 16 : q;
        ash[S][i] = live ? (int)(p - q) : -1;
        avld[S][i] = min(8, g.K - kc);
        areg[S][i][0] = *reinterpret_cast<gvec*>(q);
        areg[S][i][1] = *reinterpret_cast<gvec*>(q1);
      }
#pragma unroll
      for (int i = 0; i < kBDmaPerWave; ++i) {
        const bool live = k0 + b_row[i] < kend;
        bok[S][i] = live;
        breg[S][i] = *reinterpret_cast<gvec*>(live ? b_base + (uintptr_t)(b_off[i] + k0 * g.ldb * 2) : b_base);
      }
    } else {
#pragma unroll
      for (int i = 0; i < kAInst; ++i)
        dma16(rsrc_a, (lds_void*)(rs_a<NB, S>() + (kRowsPerWave * wave + 4 * i) * 256),
              dma_offset(k0 + a_col[i] < kend, a_off[i] + k0 * 2));
#pragma unroll
      for (int i = 0; i < kBDmaPerWave; ++i)
        dma16(rsrc_b, (lds_void*)(rs_b<NB, S>() + (wave * kBDmaPerWave + i) * 1024),
              dma_offset(k0 + b_row[i] < kend, b_off[i] + k0 * g.ldb * 2));
    }
  };

  // Fragment addresses.  A, k step j: row 16w + l%16, chunk 4j + l/16.  B,
  // k step j, column block cb, half h: source lane s = l%16 of group
  // q = l/16 points at k row 32j + 8q + 4h + s/4, column 16cb + 4(s%4).
  const int a_r = 16 * (wave / kColSplit) + (lane & 15);
  const int col0 = (wave % kColSplit) * (NB / kColSplit);  // this wave's first column
  int fa[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) fa[j] = a_r * 256 + ((4 * j + (lane >> 4)) ^ (a_r & 15)) * 16;
  int fb[4][kBlocks][2];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int cb = 0; cb < kBlocks; ++cb)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int sl = lane & 15, q = lane >> 4;
        fb[j][cb][h] = (32 * j + 8 * q + 4 * h + (sl >> 2)) * (NB * 2) + (col0 + 16 * cb + 4 * (sl & 3)) * 2;
      }

  f32x4 acc[kBlocks];
#pragma unroll
  for (int cb = 0; cb < kBlocks; ++cb) acc[cb] = f32x4{};

  // kv: elements of the stage below K, counted from its first k.  Under K
  // (kv < kRsStep, only the last stage when K is not a multiple of 8) the
  // DMA brought the whole chunk that straddles K: its elements past K (the
  // next row, or row padding that may hold NaN) are cleared.  Lane l's
  // fragment j holds k = 32j + 8(l/16) .. +7 of the stage.
  auto compute = [&](auto sc, int kv) {
    constexpr int S = decltype(sc)::value;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      u32x4 af = *reinterpret_cast<const u32x4*>(rs_a<NB, S>() + fa[j]);
      if constexpr (!UA) {
        if (kv < kRsStep) {
          const int v = min(max(kv - (32 * j + 8 * (lane >> 4)), 0), 8);
#pragma unroll
          for (int w = 0; w < 4; ++w)
            af[w] &= (2 * w < v ? 0x0000ffffu : 0u) | (2 * w + 1 < v ? 0xffff0000u : 0u);
        }
      }
#pragma unroll
      for (int cb = 0; cb < kBlocks; ++cb) {
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s16x4*)(rs_b<NB, S>() + fb[j][cb][0]));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s16x4*)(rs_b<NB, S>() + fb[j][cb][1]));
        const uint64_t l64 = __builtin_bit_cast(uint64_t, lo), h64 = __builtin_bit_cast(uint64_t, hi);
        const u32x4 bf = u32x4{(uint32_t)l64, (uint32_t)(l64 >> 32), (uint32_t)h64, (uint32_t)(h64 >> 32)};
        acc[cb] = mfma16x16x32<DT>(af, bf, acc[cb]);
      }
    }
  };

  // Same step structure as the skinny streaming kernel: wait for stage S
  // (STAGES - 2 newer stages may be in flight), barrier, refill the
  // stage freed one step earlier, multiply.
  constexpr int kLater = STAGES - 2;
  auto step_fn = [&](auto sc, int step) {
    constexpr int S = decltype(sc)::value;
    wait_vmcnt<kLoadsPerWave * kLater>();
    if constexpr (UA) {
      // This wave's chunks of the stage have landed in registers.
#pragma unroll
      for (int i = 0; i < kAInst; ++i) {
        const int sh = ash[S][i], nv = avld[S][i];
        u32x4 v = sh < 0 ? u32x4{0, 0, 0, 0} : shift_join(areg[S][i][0], areg[S][i][1], sh);
#pragma unroll
        for (int w = 0; w < 4; ++w)  // elements 2w, 2w + 1 (k >= K cleared)
          v[w] = 2 * w + 1 < nv ? v[w] : (2 * w < nv ? v[w] & 0xffffu : 0u);
        *reinterpret_cast<u32x4*>(rs_a<NB, S>() + (kRowsPerWave * wave + 4 * i) * 256 + lane * 16) = v;
      }
#pragma unroll
      for (int i = 0; i < kBDmaPerWave; ++i)
        *reinterpret_cast<u32x4*>(rs_b<NB, S>() + (wave * kBDmaPerWave + i) * 1024 + lane * 16) =
            bok[S][i] ? breg[S][i] : u32x4{0, 0, 0, 0};
    }
    wait_lgkm0();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    issue(StageC<(S + STAGES - 1) % STAGES>{}, step + STAGES - 1);
    int s_k = step + rot;
    if (s_k >= nsteps) s_k -= nsteps;
    compute(sc, g.K - (kbeg + s_k * kRsStep));
    __builtin_amdgcn_sched_barrier(0);
  };

  issue(StageC<0>{}, 0);
  issue(StageC<1>{}, 1);
  if constexpr (STAGES > 3) issue(StageC<2 % STAGES>{}, 2);
  if constexpr (STAGES > 4) issue(StageC<3 % STAGES>{}, 3);
  if constexpr (STAGES > 5) issue(StageC<4 % STAGES>{}, 4);

  int step = 0;
  for (; step + STAGES <= nsteps; step += STAGES) {
    step_fn(StageC<0>{}, step);
    step_fn(StageC<1>{}, step + 1);
    step_fn(StageC<2>{}, step + 2);
    if constexpr (STAGES > 3) step_fn(StageC<3 % STAGES>{}, step + 3);
    if constexpr (STAGES > 4) step_fn(StageC<4 % STAGES>{}, step + 4);
    if constexpr (STAGES > 5) step_fn(StageC<5 % STAGES>{}, step + 5);
  }
  if (step < nsteps) step_fn(StageC<0>{}, step++);
  if (step < nsteps) step_fn(StageC<1>{}, step++);
  if constexpr (STAGES > 3)
    if (step < nsteps) step_fn(StageC<2 % STAGES>{}, step++);
  if constexpr (STAGES > 4)
    if (step < nsteps) step_fn(StageC<3 % STAGES>{}, step++);
  if constexpr (STAGES > 5)
    if (step < nsteps) step_fn(StageC<4 % STAGES>{}, step++);
  wait_vmcnt<0>();  // no DMA may still be writing LDS at exit

  // 16x16 accumulator layout: register r of lane l holds row 4*(l/16) + r,
  // column l%16 of the block.
  float* dst = g.splits > 1 ? g.ws + (int64_t)split * g.M * g.N : g.C;
  const int64_t ld = g.splits > 1 ? (int64_t)g.N : g.ldc;
#pragma unroll
  for (int cb = 0; cb < kBlocks; ++cb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = m0 + 16 * (wave / kColSplit) + (lane >> 4) * 4 + r, col = col0 + 16 * cb + (lane & 15);
      if (row < g.M && col < g.N) dst[(int64_t)row * ld + col] = acc[cb][r];
    }
}

// C[i][j] = sum over splits s = 0..S-1 (in order) of ws[s][i][j] (ws rows:
// `mrows` per split), four columns per thread (N is a multiple of 4 on this
// path).
__global__ __launch_bounds__(256) void stream_reduce_kernel(const float* ws, float* C, int64_t ldc, int M,
                                                            int N, int mrows, int splits, bool c_vec) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t per_row = N / 4;
  if (idx >= (int64_t)M * per_row) return;
  const int row = (int)(idx / per_row), col = (int)(idx % per_row) * 4;
  f32x4 part[kStMaxSplits];
#pragma unroll
  for (int sp = 0; sp < kStMaxSplits; ++sp)
    if (sp < splits) part[sp] = *reinterpret_cast<const f32x4*>(ws + ((int64_t)sp * mrows + row) * N + col);
  f32x4 v = part[0];
#pragma unroll
  for (int sp = 1; sp < kStMaxSplits; ++sp)
    if (sp < splits) v += part[sp];
  float* dst = C + (int64_t)row * ldc + col;
  if (c_vec) {
    *reinterpret_cast<f32x4*>(dst) = v;
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) dst[e] = v[e];
  }
}

// C[i][j] = sum over splits s = 0..S-1 (in order) of ws[s][i][j] (ws rows:
// `mrows` per split), one element per thread: any N.
__global__ __launch_bounds__(256) void skinny_reduce_kernel(const float* ws, float* C, int64_t ldc,
                                                            int M, int N, int mrows, int splits) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)M * N) return;
  const int row = (int)(idx / N), col = (int)(idx % N);
  float v = ws[(int64_t)row * N + col];
  for (int s = 1; s < splits; ++s) v += ws[((int64_t)s * mrows + row) * N + col];
  C[(int64_t)row * ldc + col] = v;
}

// C[i][j] = sum over many splits (more than kStMaxSplits) of ws[s][i][j]
// (ws rows: `mrows` per split).  A workgroup of kSrWaves waves takes 64
// consecutive outputs, one per lane (coalesced reads of each split); wave w
// sums splits w, w + kSrWaves, ... in increasing order and the waves' sums
// are added in order w = 0 .. kSrWaves - 1: a fixed order, so results repeat
// bit for bit.  (One element per thread over 256 partials ran at 8x the
// time: each thread's loads wait on the next.)
constexpr int kSrWaves = 16;
__global__ __launch_bounds__(64 * kSrWaves) void split_reduce_kernel(const float* ws, float* C, int64_t ldc,
                                                                     int M, int N, int mrows, int splits) {
  __shared__ float sums[kSrWaves][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t idx = (int64_t)blockIdx.x * 64 + lane;
  const bool live = idx < (int64_t)M * N;
  const int row = live ? (int)(idx / N) : 0, col = live ? (int)(idx % N) : 0;
  float v = 0.0f;
  if (live)
    for (int sp = wave; sp < splits; sp += kSrWaves) v += ws[((int64_t)sp * mrows + row) * N + col];
  sums[wave][lane] = v;
  __syncthreads();
  if (wave == 0 && live) {
    float t = sums[0][lane];
#pragma unroll
    for (int w = 1; w < kSrWaves; ++w) t += sums[w][lane];
    C[(int64_t)row * ldc + col] = t;
  }
}

// Grid-stride: a launch holds at most 2^32 - 1 work-items, and C may hold
// more elements than that.
__global__ __launch_bounds__(256) void fill_zero_kernel(float* C, int64_t ldc, int M, int N) {
  const int64_t total = (int64_t)M * N, stride = (int64_t)gridDim.x * 256;
  for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += stride)
    C[(idx / N) * ldc + (idx % N)] = 0.0f;
}

constexpr int64_t kFillMaxBlocks = (int64_t)1 << 20;
unsigned fill_blocks(int64_t total) {
  const int64_t blocks = (total + 255) / 256;
  return (unsigned)(blocks < kFillMaxBlocks ? blocks : kFillMaxBlocks);
}


}  // namespace

// Scratch of hcg_gemm_noalloc (repacked operands and split-K partials): one
// array per GPU, resident from the library's first use on that GPU until
// the process ends.  In host code the name is a stand-in, not a device
// address: the address comes from hipGetSymbolAddress, per device, at
// set-up (DeviceState::scratch), and only that pointer is passed on.
static __device__ __align__(256) unsigned char scratch[HCG_NOALLOC_SCRATCH_BYTES];

namespace {

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

using hcg::set_error;
using hcg::t_last_error;

#define HCG_HIP_CHECK(expr)                                                               \
  do {                                                                                    \
    hipError_t _e = (expr);                                                               \
    if (_e != hipSuccess)                                                                 \
      return set_error(HCG_EHIP, "%s failed: %s", #expr, hipGetErrorString(_e));          \
  } while (0)

constexpr int kMaxDevices = 64;
constexpr int kMaxStreamWorkspaces = 16;

// Library-owned scratch (split-K partials, repacked operands), one grow-only
// buffer per (device, stream) so that concurrent streams never share it.  A
// buffer handed out while its stream is being captured into a HIP graph is
// pinned: the graph keeps its address, so it is never freed, and no eager
// call uses it again -- the first call on its stream that is not being
// captured retires it (kept allocated until the process ends) and takes a
// fresh buffer, so a replay never races with eager work.  Graphs captured
// on one stream with no eager call on that stream between the captures
// share one pinned buffer.  With more than kMaxStreamWorkspaces streams in
// use, slots are evicted round-robin; an evicted buffer is freed with
// hipFree, which synchronises the device.
struct Workspace {
  void* stream = nullptr;
  void* ptr = nullptr;  // kStCounterBytes of arrival counters, then `bytes` of scratch
  size_t bytes = 0;
  bool pinned = false;
  bool counters_zeroed = false;  // the counters were cleared on this buffer's stream
};

struct DeviceState {
  std::once_flag once;
  int init_status = HCG_OK;
  std::string init_error;
  int num_cus = 256;
  // Device address of this GPU's `scratch` array (hcg_gemm_noalloc), or
  // null with scratch_error set if the lookup failed.
  void* scratch = nullptr;
  std::string scratch_error;
  std::mutex ws_mutex;
  Workspace ws[kMaxStreamWorkspaces];
  int ws_next = 0;
  std::vector<void*> retired;  // pinned buffers replaced in their slot
};

DeviceState g_devices[kMaxDevices];
std::once_flag g_global_once;
int g_skinny_splits_override = 0;
int g_tiled_splits_override = 0;  // HCG_TILED_SPLITS: split count for the tiled kernel, if valid
// HCG_UNALIGNED_DMA=0: never read rows that are not 16-byte aligned in place
// (repack or register-stage them, the paths for operands the DMA cannot
// read); for tests of those paths.
bool g_unaligned_dma = true;

void global_init() {
  if (const char* s = getenv("HCG_SKINNY_SPLITS")) g_skinny_splits_override = atoi(s);
  if (const char* s = getenv("HCG_TILED_SPLITS")) g_tiled_splits_override = atoi(s);
  if (const char* s = getenv("HCG_UNALIGNED_DMA")) g_unaligned_dma = atoi(s) != 0;
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
    // With this device current: its copy of the scratch array.
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      st.scratch_error = std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e);
      (void)hipGetLastError();  // the other entry points do not depend on it
    } else {
      st.scratch = ptr;
    }
  });
  if (st.init_status != HCG_OK) return set_error(st.init_status, "%s", st.init_error.c_str());
  *out = &st;
  return HCG_OK;
}

// The caller holds st->ws_mutex from this call until every kernel that uses
// *out is enqueued: another thread's call (on the same stream, needing more
// bytes, or evicting the slot) frees the buffer, and hipFree waits only for
// work already enqueued.  With `counters`, also returns the buffer's arrival
// counters, first clearing them (a fill kernel on `stream`, never a memset,
// so a capture records a kernel node) when the buffer is new or the stream
// is being captured (a graph must not depend on what ran before a replay).
int stream_workspace(DeviceState* st, hipStream_t stream, size_t bytes, void** out,
                     unsigned** counters = nullptr) {
  // The null stream is never captured (and querying it during another
  // stream's capture is itself an error), so only real streams are asked.
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  if (stream != nullptr) HCG_HIP_CHECK(hipStreamIsCapturing(stream, &capture));
  const bool capturing = capture == hipStreamCaptureStatusActive;
  Workspace* w = nullptr;
  for (auto& cand : st->ws)
    if (cand.ptr && cand.stream == (void*)stream) w = &cand;
  if (!w) {
    for (auto& cand : st->ws)
      if (!cand.ptr) {
        w = &cand;
        break;
      }
  }
  if (!w) {  // evict round-robin; hipFree waits for work that uses it
    w = &st->ws[st->ws_next];
    st->ws_next = (st->ws_next + 1) % kMaxStreamWorkspaces;
  }
  if (w->ptr && (w->stream != (void*)stream || w->bytes < bytes || (w->pinned && !capturing))) {
    if (w->pinned) {
      st->retired.push_back(w->ptr);
    } else {
      HCG_HIP_CHECK(hipFree(w->ptr));
    }
    w->ptr = nullptr;
    w->bytes = 0;
    w->pinned = false;
  }
  if (!w->ptr) {
    void* p = nullptr;
    const size_t want = bytes < ((size_t)2 << 20) ? ((size_t)2 << 20) : bytes;
    HCG_HIP_CHECK(hipMalloc(&p, want + kStCounterBytes));
    w->ptr = p;
    w->bytes = want;
    w->counters_zeroed = false;
  }
  w->stream = (void*)stream;
  if (capturing) w->pinned = true;
  *out = static_cast<char*>(w->ptr) + kStCounterBytes;
  if (counters) {
    *counters = static_cast<unsigned*>(w->ptr);
    if (!w->counters_zeroed || capturing) {
      constexpr int n = kStCounterBytes / 4;
      fill_zero_kernel<<<(n + 255) / 256, 256, 0, stream>>>(static_cast<float*>(w->ptr), n, 1, n);
      HCG_HIP_CHECK(hipGetLastError());
      w->counters_zeroed = true;
    }
  }
  return HCG_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// True when the DMA may read the whole 8-element chunk that holds an
// operand's last element (row rows - 1, column cols - 1, row stride ld,
// 16-bit elements) and 16 bytes more: with rows that are not 16-byte
// aligned the DMA kernels read up to 14 bytes past an operand's last
// element.  Those bytes are safe when they lie in the last element's 4 KB
// page, or inside the device allocation that holds the operand (a tight
// operand of a whole number of pages ends exactly at a page boundary).
bool chunk_tail_readable(const void* base, int64_t rows, int64_t cols, int64_t ld) {
  if (!g_unaligned_dma) return false;
  const uintptr_t p = reinterpret_cast<uintptr_t>(base);
  const uintptr_t last = p + (uintptr_t)(((rows - 1) * ld + cols) * 2) - 1;
  const uintptr_t end = p + (uintptr_t)(((rows - 1) * ld + (int64_t)round_up(cols, 8)) * 2) + 16;
  if ((last >> 12) == ((end - 1) >> 12)) return true;
  // The bytes past the last element reach one more page (at most 30 bytes
  // are read past it).  It is readable when it lies inside the operand's
  // allocation and is mapped: an address range reserved for virtual memory
  // management can extend past what is mapped, so the page of the last byte
  // read is also asked whether it is mapped (where the runtime cannot say,
  // the allocation range decides).
  hipDeviceptr_t alloc = nullptr;
  size_t alloc_bytes = 0;
  if (hipMemGetAddressRange(&alloc, &alloc_bytes, const_cast<void*>(base)) != hipSuccess) {
    (void)hipGetLastError();  // not device memory of this process: stay on the safe side
    return false;
  }
  if (end > reinterpret_cast<uintptr_t>(alloc) + alloc_bytes) return false;
  int mapped = 1;
  if (hipPointerGetAttribute(&mapped, HIP_POINTER_ATTRIBUTE_MAPPED, static_cast<hipDeviceptr_t>(
                                 reinterpret_cast<void*>(end - 1))) != hipSuccess) {
    (void)hipGetLastError();
    mapped = 1;
  }
  return mapped != 0;
}

// 16-bit operands: any element address is 2-byte aligned.
bool aligned2(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 1u) == 0; }

// Where a call's scratch comes from: its stream's library workspace
// (allocated on demand, see stream_workspace), or a fixed device buffer of
// `cap` bytes that is never grown (hcg_gemm_noalloc).  Planners that size
// split-K partials keep them within room(); repacked operands must fit.
struct Scratch {
  DeviceState* st = nullptr;
  hipStream_t stream = nullptr;
  void* fixed = nullptr;
  size_t cap = 0;

  // Bytes available for split partials once `used` bytes are taken.
  size_t room(size_t used) const {
    if (!fixed) return SIZE_MAX;
    return used < cap ? cap - used : 0;
  }
};

// `counters` (optional) receives the workspace's arrival counters, or null
// for the fixed buffer, which has none.
int get_scratch(const Scratch& sc, size_t bytes, void** out, unsigned** counters = nullptr) {
  if (counters) *counters = nullptr;
  if (sc.fixed) {
    if (bytes > sc.cap)
      return set_error(HCG_EINVAL,
                       "this call needs %zu bytes of scratch (repacked operands and split partials); the "
                       "allocation-free entry point has %zu",
                       bytes, sc.cap);
    *out = sc.fixed;
    return HCG_OK;
  }
  return stream_workspace(sc.st, sc.stream, bytes, out, counters);
}

// Largest split count (at most `splits`, at least 1) whose partials of
// `per_split` bytes each fit in `room` bytes.
int fit_splits(int splits, size_t per_split, size_t room) {
  if (per_split == 0 || room == SIZE_MAX) return splits;
  const size_t most = room / per_split;
  if ((size_t)splits > most) splits = most >= 2 ? (int)most : 1;
  return splits;
}

// Sums `splits` partial slices ws[s][0 .. mrows)[0 .. N) into the M x N
// output C in the fixed order s = 0 .. splits - 1 (bit-reproducible): past
// kStMaxSplits with a wave per residue class of splits, else four columns
// per thread when N is a multiple of 4 (16-byte partial rows: the
// workspace base is 256-byte aligned), else one element per thread.
int launch_reduce(const float* ws, float* C, int64_t ldc, int M, int N, int mrows, int splits, bool c_vec,
                  hipStream_t stream) {
  if (splits > kStMaxSplits) {
    const int64_t total = (int64_t)M * N;
    split_reduce_kernel<<<(unsigned)((total + 63) / 64), 64 * kSrWaves, 0, stream>>>(ws, C, ldc, M, N, mrows,
                                                                                   splits);
  } else if (N % 4 == 0) {
    const int64_t total = (int64_t)M * (N / 4);
    stream_reduce_kernel<<<(unsigned)((total + 255) / 256), 256, 0, stream>>>(ws, C, ldc, M, N, mrows, splits,
                                                                             c_vec);
  } else {
    const int64_t total = (int64_t)M * N;
    skinny_reduce_kernel<<<(unsigned)((total + 255) / 256), 256, 0, stream>>>(ws, C, ldc, M, N, mrows, splits);
  }
  HCG_HIP_CHECK(hipGetLastError());
  return HCG_OK;
}

template <int DT>
int launch_generic(const TiledArgs& a, bool vec_a, bool vec_b, hipStream_t stream) {
  const dim3 grid((unsigned)(a.tiles_m * a.tiles_n));
  const dim3 block(kTiledThreads);
  if (vec_a && vec_b) {
    gemm_generic_kernel<DT, true, true><<<grid, block, 0, stream>>>(a);
  } else if (vec_a) {
    gemm_generic_kernel<DT, true, false><<<grid, block, 0, stream>>>(a);
  } else if (vec_b) {
    gemm_generic_kernel<DT, false, true><<<grid, block, 0, stream>>>(a);
  } else {
    gemm_generic_kernel<DT, false, false><<<grid, block, 0, stream>>>(a);
  }
  HCG_HIP_CHECK(hipGetLastError());
  return HCG_OK;
}

// Output tile shapes of the DMA kernel.  TM = 256: 4-stage ring, one
// workgroup per CU; TM = 128: 3-stage ring, two workgroups per CU.
struct TileShape {
  int tm, tn;
  int per_cu;   // workgroups resident per CU
  float eff;    // relative MFMA issue efficiency of the K loop (measured)
};
constexpr TileShape kTileShapes[] = {
    {256, 256, 1, 1.00f},
    {256, 192, 1, 0.97f},
    {128, 256, 2, 0.93f},
    {128, 128, 2, 0.75f},
    {256, 64, 1, 0.75f},  // narrow N (<= 64): the A stream dominates
};
constexpr int kNumTileShapes = sizeof(kTileShapes) / sizeof(kTileShapes[0]);

// Picks the tile shape with the least modelled time: the busiest CU's
// share of tiles times tile area times K steps (scaled by the shape's K-loop
// efficiency), plus a fixed cost per round of resident workgroups
// (prologue, epilogue, launch) worth about eight 256x256 K tiles, or four
// where two workgroups share a CU and each hides part of the other's.  The
// constants were fitted to 24 shapes timed with every tile shape forced;
// the pick was within 6% of the fastest on all of them.
//
// With splits > 1 (split-K), each tile's K range is cut into `splits`
// parts run by separate workgroups whose partial products a second kernel
// sums in a fixed order; that reduction is charged as its launch plus the
// partials' HBM traffic ((splits + 1) x M x N floats), converted to K tiles
// at 0.73 us per 256x256 K tile.
struct TilePlan {
  int shape;
  int splits;
};

constexpr int kSplitCandidates[] = {1, 2, 3, 4, 6, 8};
constexpr int kMinKTilesPerSplit = 8;
constexpr size_t kMaxSplitWorkspace = (size_t)512 << 20;

// `room`: scratch bytes available for the partials (kMaxSplitWorkspace at
// most).
bool split_ok(int splits, int M, int N, int K, size_t room) {
  const int nk = (K + kDmaK - 1) / kDmaK;
  const size_t limit = room < kMaxSplitWorkspace ? room : kMaxSplitWorkspace;
  return splits == 1 || (splits <= 64 && (nk + splits - 1) / splits >= kMinKTilesPerSplit &&
                         (size_t)splits * M * N * sizeof(float) <= limit);
}

double plan_cost(const TileShape& t, int splits, int num_cus, int M, int N, int K) {
  const int64_t nk = (K + kDmaK - 1) / kDmaK;
  const int64_t tiles = (int64_t)((M + t.tm - 1) / t.tm) * ((N + t.tn - 1) / t.tn) * splits;
  const int64_t per_cu = (tiles + num_cus - 1) / num_cus;
  const int64_t rounds = (per_cu + t.per_cu - 1) / t.per_cu;
  const double fixed = t.per_cu == 1 ? 8.0 : 4.0;
  const double unit = 256.0 * 256.0;
  double cost = (double)per_cu * t.tm * t.tn * (double)((nk + splits - 1) / splits) / t.eff + (double)rounds * fixed * unit;
  if (splits > 1) {
    const double reduce_us = 2.0 + (double)(splits + 1) * M * N * sizeof(float) / 4.5e6;
    cost += reduce_us / 0.73 * unit;
  }
  return cost;
}

TilePlan plan_tiles(int num_cus, int M, int N, int K, int force_shape, bool allow_split,
                    double* cost_out = nullptr, size_t room = kMaxSplitWorkspace) {
  TilePlan best{force_shape >= 0 ? force_shape : 0, 1};
  double best_cost = -1;
  const int forced_splits =
      allow_split && g_tiled_splits_override > 0 && split_ok(g_tiled_splits_override, M, N, K, room)
          ? g_tiled_splits_override
          : 0;
  for (int i = 0; i < kNumTileShapes; ++i) {
    if (force_shape >= 0 && i != force_shape) continue;
    const TileShape& t = kTileShapes[i];
    if ((int64_t)((M + t.tm - 1) / t.tm) * ((N + t.tn - 1) / t.tn) * 64 > 0x7fffffff) continue;
    for (int c = 0; c < (forced_splits > 0 ? 1 : (int)(sizeof(kSplitCandidates) / sizeof(int))); ++c) {
      const int splits = forced_splits > 0 ? forced_splits : kSplitCandidates[c];
      if (splits > 1 && !allow_split) break;
      if (!split_ok(splits, M, N, K, room)) continue;
      const double cost = plan_cost(t, splits, num_cus, M, N, K);
      if (best_cost < 0 || cost < best_cost) {
        best = TilePlan{i, splits};
        best_cost = cost;
      }
    }
  }
  if (cost_out) *cost_out = best_cost;
  return best;
}


template <int DT, bool WIDE, bool KT = false>
int launch_dma(const FastArgs& a, int shape, hipStream_t stream) {
  const dim3 grid((unsigned)(a.tiles_m * a.tiles_n * (a.splits > 1 ? a.splits : 1)));
  const dim3 block(kTiledThreads);
  HCG_STAMP_ARGS(FastArgs, a)
  // 256-row tiles move A as 64-wide K pairs (A2) unless the operands need
  // the WIDE form.
  constexpr bool kA2 = !WIDE;
  switch (shape) {
    case 0: gemm_dma_kernel<DT, 256, 256, 4, WIDE, KT, kA2><<<grid, block, 0, stream>>>(HCG_STAMPED(a)); break;
    case 1: gemm_dma_kernel<DT, 256, 192, 4, WIDE, KT, kA2><<<grid, block, 0, stream>>>(HCG_STAMPED(a)); break;
    case 2: gemm_dma_kernel<DT, 128, 256, 3, WIDE, KT><<<grid, block, 0, stream>>>(HCG_STAMPED(a)); break;
    case 3: gemm_dma_kernel<DT, 128, 128, 3, WIDE, KT><<<grid, block, 0, stream>>>(HCG_STAMPED(a)); break;
    default: gemm_dma_kernel<DT, 256, 64, 4, WIDE, KT, kA2><<<grid, block, 0, stream>>>(HCG_STAMPED(a)); break;
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
                                                                             a.N, 16, a.splits);
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

// Split count for the streaming kernel: about one workgroup per CU, each
// split at least 8 stages (256 rows) long.
// The K split: the most working workgroups (column blocks times splits; the
// grid's padding workgroups exit at once) that do not exceed `per_cu` per
// CU, each split at least 8 steps, at most kStMaxSplitsLoop (tiny outputs
// with a long K: 64 x 32 x 2^20 runs 256 workgroups instead of 16).
// Overshooting by a few workgroups leaves a short second round:
// 16 x 12288 x 4096 fp16 28.4 us at 3 splits (288 workgroups) against 22.4
// us at 2, 16 x 5120 x 13824 40.2 us at 7 against 29.7 at 6.
int stream_splits(const DeviceState* st, int nblocks, int K, int per_cu) {
  const int ksteps = (K + kStStep - 1) / kStStep;
  int splits = g_skinny_splits_override;
  if (splits <= 0) {
    splits = per_cu * st->num_cus / nblocks;
    const int max_by_k = ksteps / 8 > 0 ? ksteps / 8 : 1;
    if (splits > max_by_k) splits = max_by_k;
  }
  if (splits > ksteps) splits = ksteps;
  if (splits > kStMaxSplitsLoop) splits = kStMaxSplitsLoop;
  if (splits < 1) splits = 1;
  return splits;
}

template <int DT, bool UB>
int launch_stream(const StreamArgs& a, hipStream_t stream) {
  // Column blocks padded to a multiple of 8 per split (see the workgroup
  // mapping in gemm_stream_kernel); padding workgroups exit at once.
  const int nblocks = (a.N + kStN - 1) / kStN;
  const dim3 grid((unsigned)(round_up(nblocks, 8) * a.splits));
  HCG_STAMP_ARGS(StreamArgs, a)
  // Prefetch distance by row blocks (measured, fp16, B from HBM, us, 7 / 5 /
  // 4 / 3 stages ahead): 16 x 8192 x 8192 28.2 / 27.6 / 26.7 / 25.9,
  // 32 x 8192 x 8192 29.8 / 29.2 / 28.1 / 26.8, 64 x 8192 x 8192
  // 30.1 / 29.7 / 29.5 / 29.7, 128 x 8192 x 8192 39.6 / 39.1 / 39.5 / 40.4;
  // register-staged B (16 x 8191 x 8192) 37.5 / 36.6 / 36.0 / 35.9.
  switch (a.rblocks) {
    case 1: gemm_stream_kernel<DT, 1, UB, 3><<<grid, dim3(256), 0, stream>>>(HCG_STAMPED(a)); break;
    case 2: gemm_stream_kernel<DT, 2, UB, 3><<<grid, dim3(256), 0, stream>>>(HCG_STAMPED(a)); break;
    case 4: gemm_stream_kernel<DT, 4, UB, 4><<<grid, dim3(256), 0, stream>>>(HCG_STAMPED(a)); break;
    case 8: gemm_stream_kernel<DT, 8, UB, 5><<<grid, dim3(256), 0, stream>>>(HCG_STAMPED(a)); break;
    default: return set_error(HCG_EINVAL, "internal: %d row blocks", a.rblocks);
  }
  HCG_HIP_CHECK(hipGetLastError());
  if (a.splits > 1 && a.counters == nullptr)
    return launch_reduce(a.ws, a.C, a.ldc, a.M, a.N, 16 * a.rblocks, a.splits, a.c_vec, stream);
  return HCG_OK;
}

// 16-row blocks of A the streaming kernel runs with for M rows (M <= 128).
int stream_rblocks(int64_t M) { return M <= 16 ? 1 : M <= 32 ? 2 : M <= 64 ? 4 : 8; }

// The streaming kernel masks at 8-element granularity through the buffer
// range check (chunks past the split's K range or past N, and rows past M,
// load zeros).  N need not be a multiple of 8 (the chunk holding column
// N - 1 also loads up to 7 padding columns, which reach only output columns
// >= N, never stored).  A (at most 128 rows) and B are read in place where
// that is safe (below); otherwise A is repacked into zero-padded rows of
// round_up(K, 8) and B is register-staged (UB).  A's byte offsets stay
// below 2^31.
bool stream_extent_a(int64_t lda, int64_t M, int64_t K) {
  return ((int64_t)16 * stream_rblocks(M) * lda + K) * 2 < ((int64_t)1 << 31);
}
// The DMA reads 16-byte chunks at any 2-byte alignment: rows that are not
// 16-byte aligned are read in place when the last chunk's bytes past the
// operand stay in its last page (chunk_tail_readable).  A chunk of A that
// straddles K is cleared past K in the kernel's fragments.
bool stream_a_in_place(const void* A, int64_t lda, int64_t M, int64_t K) {
  return stream_extent_a(lda, M, (int64_t)round_up(K, 8)) &&
         ((aligned16(A) && lda % 8 == 0) || (K > 0 && aligned2(A) && chunk_tail_readable(A, M, K, lda)));
}
bool stream_b_dma(const void* B, int64_t ldb, int64_t N, int64_t K) {
  return ((int64_t)round_up(K, kStStep) * ldb + round_up(N, kStN)) * 2 < ((int64_t)1 << 31) &&
         ((aligned16(B) && ldb % 8 == 0) || (aligned2(B) && chunk_tail_readable(B, K, N, ldb)));
}
// B that the DMA cannot take (last chunk not safely readable, or offsets
// past 2^31) is register-staged: 16-byte loads at any 2-byte alignment, all
// inside B's extent, which must then hold at least 8 elements.
bool stream_fits(const void* A, int64_t lda, const void* B, int64_t ldb, int64_t M, int64_t N, int64_t K) {
  return M <= 16 * kStMaxRowBlocks && ldb < ((int64_t)1 << 31) &&
         (stream_b_dma(B, ldb, N, K) || (K - 1) * ldb + N >= 8) &&
         (stream_a_in_place(A, lda, M, K) || stream_extent_a(round_up(K, 8), M, K));
}

int run_skinny(const Scratch& sc, int dtype, const void* A, int64_t lda, const void* B, int64_t ldb,
               float* C, int64_t ldc, int M, int N, int K) {
  DeviceState* st = sc.st;
  hipStream_t stream = sc.stream;
  if (stream_fits(A, lda, B, ldb, M, N, K)) {
    const bool a_in_place = stream_a_in_place(A, lda, M, K);
    const int64_t lda_use = a_in_place ? lda : (int64_t)round_up(K, 8);
    StreamArgs a{};
    a.A = static_cast<const uint16_t*>(A);
    a.B = static_cast<const uint16_t*>(B);
    a.C = C;
    a.lda = (int)lda_use;
    a.ldb = (int)ldb;
    a.ldc = ldc;
    a.M = M;
    a.N = N;
    a.K = K;
    // Register-staged B needs more waves in flight: two workgroups per CU
    // for one or two row blocks (16 x 8191 x 8192 fp16: 39.9 -> 37.3 us; at
    // four row blocks the larger partials cost more than that gains).
    const bool b_dma = stream_b_dma(B, ldb, N, K);
    const size_t a_sz = a_in_place ? 0 : round_up((size_t)M * lda_use * 2, 256);
    a.splits = stream_splits(st, (N + kStN - 1) / kStN, K, !b_dma && stream_rblocks(M) <= 2 ? 2 : 1);
    a.splits = fit_splits(a.splits, (size_t)16 * stream_rblocks(M) * N * sizeof(float), sc.room(a_sz));
    const int ksteps = (K + kStStep - 1) / kStStep;
    a.kchunk = ((ksteps + a.splits - 1) / a.splits) * kStStep;
    a.splits = (K + a.kchunk - 1) / a.kchunk;  // drop empty trailing splits
    a.rblocks = stream_rblocks(M);
    // Extents end with the chunk that holds the last element.
    a.a_bytes = (int)((((int64_t)M - 1) * lda_use + (int64_t)round_up(K, 8)) * 2);
    // (register-staged B reads through plain pointers: no extent)
    a.b_bytes = b_dma ? (int)((((int64_t)K - 1) * ldb + (int64_t)round_up(N, 8)) * 2) : 0;
    a.c_vec = aligned16(C) && ldc % 4 == 0;
    a.ws = nullptr;
    a.counters = nullptr;
    // Workspace: A repacked (when it cannot be used in place), then the
    // split partials.
    const size_t p_sz = a.splits > 1 ? (size_t)a.splits * 16 * a.rblocks * (size_t)N * sizeof(float) : 0;
    // The in-kernel reduction (see stream_fused_reduce) replaces the reduce
    // launch: 16 x 8192 x 8192 fp16 25.9-26.0 -> 25.6-25.7 us.
    const bool fuse = a.splits > 1 && a.rblocks <= 2 && a.splits <= kStFuseMaxSplits(a.rblocks) && N % 4 == 0 &&
                      (N + kStN - 1) / kStN <= kStCounterBytes / 4 && p_sz < ((size_t)1 << 31);
    if (a_sz + p_sz > 0) {
      void* ws = nullptr;
      unsigned* counters = nullptr;
      const int rc = get_scratch(sc, a_sz + p_sz, &ws, fuse ? &counters : nullptr);
      if (rc != HCG_OK) return rc;
      if (fuse && counters) {
        a.counters = counters;
        a.ws_bytes = (int)p_sz;
      }
      if (!a_in_place) {
        uint16_t* a_p = static_cast<uint16_t*>(ws);
        const RepackJob ja{a.A, lda, M, K, a_p, (int)lda_use, (int64_t)M * (lda_use / 8)};
        const RepackJob jb{};
        const int64_t per_block = (int64_t)256 * kRepackPer;
        repack_kernel<<<(unsigned)((ja.chunks + per_block - 1) / per_block), 256, 0, stream>>>(ja, jb);
        HCG_HIP_CHECK(hipGetLastError());
        a.A = a_p;
      }
      if (a.splits > 1) a.ws = reinterpret_cast<float*>(static_cast<char*>(ws) + a_sz);
    }
    if (b_dma)
      return dtype == HCG_F16 ? launch_stream<HCG_F16, false>(a, stream) : launch_stream<HCG_BF16, false>(a, stream);
    return dtype == HCG_F16 ? launch_stream<HCG_F16, true>(a, stream) : launch_stream<HCG_BF16, true>(a, stream);
  }
  // Fallback for unaligned operands (M <= 16): register-staged kernel +
  // reduce kernel.
  if (M > 16)
    return set_error(HCG_EINVAL,
                     "the skinny kernel cannot take this layout for M > 16 (B under 8 elements, or offsets "
                     "of A past 2^31) "
                     "(M=%d)", M);
  SkinnyArgs a{};
  a.A = static_cast<const uint16_t*>(A);
  a.B = static_cast<const uint16_t*>(B);
  a.C = C;
  a.lda = lda;
  a.ldb = ldb;
  a.ldc = ldc;
  a.M = M;
  a.N = N;
  a.K = K;
  a.splits = fit_splits(skinny_splits(st, N, K), (size_t)16 * N * sizeof(float), sc.room(0));
  const int kunit = kSkinnyStep * kSkinnyWaves;
  const int kunits = (K + kunit - 1) / kunit;
  a.kchunk = ((kunits + a.splits - 1) / a.splits) * kunit;
  a.splits = (K + a.kchunk - 1) / a.kchunk;  // drop empty trailing splits
  a.ws = nullptr;
  if (a.splits > 1) {
    void* ws = nullptr;
    const int rc = get_scratch(sc, (size_t)a.splits * 16 * (size_t)N * sizeof(float), &ws);
    if (rc != HCG_OK) return rc;
    a.ws = static_cast<float*>(ws);
  }
  const bool vec_a = aligned16(A) && (lda % 8 == 0);
  const bool vec_b = aligned16(B) && (ldb % 8 == 0);
  return dtype == HCG_F16 ? launch_skinny<HCG_F16>(a, vec_a, vec_b, stream)
                          : launch_skinny<HCG_BF16>(a, vec_a, vec_b, stream);
}

// The narrow-N streaming kernel: N <= 64, A by DMA or through registers,
// byte offsets below 2^31.
// B's rows need not be aligned: B (at most 64 columns) is read in place by
// the DMA when its last chunk is safely readable (chunk_tail_readable; the
// chunk holding column N - 1 brings columns that reach only C columns >= N)
// and repacked otherwise.  A goes by DMA when its rows are 16-byte aligned
// or its last chunk is safely readable, and its offsets stay below 2^31
// (the chunk straddling K is cleared past K in the fragments); through
// registers otherwise.
bool rowstream_a_dma(const void* A, int64_t lda, int64_t M, int64_t K) {
  return ((int64_t)round_up(M, kRsRows) * lda + round_up(K, kRsStep)) * 2 < ((int64_t)1 << 31) &&
         ((aligned16(A) && lda % 8 == 0) || (K > 0 && aligned2(A) && chunk_tail_readable(A, M, K, lda)));
}
bool rowstream_b_in_place(const void* B, int64_t ldb, int64_t N, int64_t K) {
  return (aligned16(B) && ldb % 8 == 0) || (aligned2(B) && chunk_tail_readable(B, K, N, ldb));
}
bool rowstream_fits(const void* A, int64_t lda, const void* B, int64_t ldb, int64_t M, int64_t N, int64_t K) {
  const int64_t ldb_use = rowstream_b_in_place(B, ldb, N, K) ? ldb : round_up(N, 8);
  return N <= 64 && lda < ((int64_t)1 << 31) &&
         ((int64_t)round_up(K, kRsStep) * ldb_use + 64) * 2 < ((int64_t)1 << 31);
}

template <int DT, int NB>
void launch_rowstream(const RowStreamArgs& a, bool ua, bool short_ring, dim3 grid, hipStream_t stream) {
  if constexpr (NB <= 32) {
    if (short_ring) {
      if (ua)
        gemm_rowstream_kernel<DT, NB, true, 3><<<grid, dim3(256), 0, stream>>>(a);
      else
        gemm_rowstream_kernel<DT, NB, false, 3><<<grid, dim3(256), 0, stream>>>(a);
      return;
    }
  }
  const dim3 block(NB == 64 ? 512 : 256);
  if (ua)
    gemm_rowstream_kernel<DT, NB, true><<<grid, block, 0, stream>>>(a);
  else
    gemm_rowstream_kernel<DT, NB, false><<<grid, block, 0, stream>>>(a);
}

int run_rowstream(const Scratch& sc, int dtype, const void* A, int64_t lda, const void* B, int64_t ldb,
                  float* C, int64_t ldc, int M, int N, int K) {
  DeviceState* st = sc.st;
  hipStream_t stream = sc.stream;
  RowStreamArgs a{};
  a.A = static_cast<const uint16_t*>(A);
  a.B = static_cast<const uint16_t*>(B);
  a.C = C;
  a.lda = (int)lda;
  a.ldb = (int)ldb;
  a.ldc = ldc;
  a.M = M;
  a.N = N;
  a.K = K;
  // Row blocks, then the most K splits whose workgroups do not exceed the
  // CUs -- twice over for register-staged A, whose 3-stage ring fits two
  // workgroups per CU when N <= 32 (each split at least 4 stages of 128 k).
  // Rounding up left a short second round: 5000 x 8 x 16384 fp16 39.1 us
  // at 4 splits (316 workgroups) against 30.3 us at 3.
  const bool a_dma = rowstream_a_dma(A, lda, M, K);
  const bool short_ring = !a_dma && N <= 32;
  const int nrb = (M + kRsRows - 1) / kRsRows;
  const int ksteps = (K + kRsStep - 1) / kRsStep;
  const int target = short_ring ? 2 * st->num_cus : st->num_cus;
  int splits = target / nrb;
  const int max_by_k = ksteps / 4 > 0 ? ksteps / 4 : 1;
  if (splits > max_by_k) splits = max_by_k;
  if (splits > kStMaxSplitsLoop) splits = kStMaxSplitsLoop;
  if (splits < 1) splits = 1;
  // Workspace: B repacked to zero-padded 16-byte aligned rows (when the DMA
  // cannot read it in place), then the split partials [splits][M][N].
  const bool b_ok = rowstream_b_in_place(B, ldb, N, K);
  const int64_t ldb_use = b_ok ? ldb : round_up(N, 8);
  const size_t b_sz = b_ok ? 0 : round_up((size_t)K * ldb_use * 2, 256);
  splits = fit_splits(splits, (size_t)M * N * sizeof(float), sc.room(b_sz));
  a.kchunk = (ksteps + splits - 1) / splits * kRsStep;
  a.rot_groups = lda == 4096 ? 16 : 0x7fffffff;  // measured: 8 KB rows prefer 16 start steps
  a.splits = (K + a.kchunk - 1) / a.kchunk;
  const size_t p_sz = a.splits > 1 ? (size_t)a.splits * M * N * sizeof(float) : 0;
  if (b_sz + p_sz > 0) {
    void* ws = nullptr;
    const int rc = get_scratch(sc, b_sz + p_sz, &ws);
    if (rc != HCG_OK) return rc;
    if (!b_ok) {
      uint16_t* b_p = static_cast<uint16_t*>(ws);
      const RepackJob ja{};
      const RepackJob jb{a.B, ldb, K, N, b_p, (int)ldb_use, (int64_t)K * (ldb_use / 8)};
      const int64_t per_block = (int64_t)256 * kRepackPer;
      repack_kernel<<<(unsigned)((jb.chunks + per_block - 1) / per_block), 256, 0, stream>>>(ja, jb);
      HCG_HIP_CHECK(hipGetLastError());
      a.B = b_p;
      a.ldb = (int)ldb_use;
    }
    if (a.splits > 1) a.ws = reinterpret_cast<float*>(static_cast<char*>(ws) + b_sz);
  }
  // Extents end with the chunk that holds the last element.
  a.a_bytes = a_dma ? (int)((((int64_t)M - 1) * lda + (int64_t)round_up(K, 8)) * 2) : 0;
  a.b_bytes = (int)((((int64_t)K - 1) * a.ldb + (int64_t)round_up(N, 8)) * 2);
  const dim3 grid((unsigned)(nrb * a.splits));
  const int nb = N <= 16 ? 16 : N <= 32 ? 32 : 64;
  if (dtype == HCG_F16) {
    if (nb == 16) launch_rowstream<HCG_F16, 16>(a, !a_dma, short_ring, grid, stream);
    else if (nb == 32) launch_rowstream<HCG_F16, 32>(a, !a_dma, short_ring, grid, stream);
    else launch_rowstream<HCG_F16, 64>(a, !a_dma, short_ring, grid, stream);
  } else {
    if (nb == 16) launch_rowstream<HCG_BF16, 16>(a, !a_dma, short_ring, grid, stream);
    else if (nb == 32) launch_rowstream<HCG_BF16, 32>(a, !a_dma, short_ring, grid, stream);
    else launch_rowstream<HCG_BF16, 64>(a, !a_dma, short_ring, grid, stream);
  }
  HCG_HIP_CHECK(hipGetLastError());
  if (a.splits > 1) return launch_reduce(a.ws, C, ldc, M, N, M, a.splits, aligned16(C) && ldc % 4 == 0, stream);
  return HCG_OK;
}

int run_generic(int dtype, const void* A, int64_t lda, const void* B, int64_t ldb, float* C,
                int64_t ldc, int M, int N, int K, hipStream_t stream) {
  TiledArgs a{};
  a.A = static_cast<const uint16_t*>(A);
  a.B = static_cast<const uint16_t*>(B);
  a.C = C;
  a.lda = lda;
  a.ldb = ldb;
  a.ldc = ldc;
  a.M = M;
  a.N = N;
  a.K = K;
  a.tiles_m = (M + kTileM - 1) / kTileM;
  a.tiles_n = (N + kTileN - 1) / kTileN;
  if ((int64_t)a.tiles_m * a.tiles_n > 0x7fffffff) return set_error(HCG_EINVAL, "too many output tiles");
  const bool vec_a = aligned16(A) && (lda % 8 == 0);
  const bool vec_b = aligned16(B) && (ldb % 8 == 0);
  return dtype == HCG_F16 ? launch_generic<HCG_F16>(a, vec_a, vec_b, stream)
                          : launch_generic<HCG_BF16>(a, vec_a, vec_b, stream);
}

// Largest byte offset the fast kernel forms for A (rows up to the padded tile
// extent) or B (rows up to the padded K extent); must stay below 2^31.
int64_t fast_extent_a(int M, int K, int64_t lda) {
  return ((int64_t)round_up(M, kTileM) * lda + round_up(K, kTileK) + 8) * 2;
}
int64_t fast_extent_b(int N, int K, int64_t ldb) {
  return ((int64_t)round_up(K, kTileK) * ldb + round_up(N, kTileN) + 8) * 2;
}

int run_tiled(const Scratch& sc, int dtype, const void* A, int64_t lda, const void* B, int64_t ldb,
              float* C, int64_t ldc, int M, int N, int K, bool force_generic, int force_shape) {
  DeviceState* st = sc.st;
  hipStream_t stream = sc.stream;
  const int64_t kLimit = (int64_t)1 << 31;
  // The DMA kernel moves 16-byte chunks (8 elements) at any 2-byte
  // alignment, so operands are read in place whenever the last chunk's
  // bytes past the operand stay in its last page (chunk_tail_readable);
  // otherwise they are repacked into zero-padded aligned rows.  A chunk of A
  // straddling K brings elements past K (the next row or row padding), which
  // the kernel clears (KT); B's chunk straddling N brings columns past N,
  // which reach only C columns >= N, never stored.
  const bool a_aligned = aligned16(A) && lda % 8 == 0 && K % 8 == 0;
  const bool b_aligned = aligned16(B) && ldb % 8 == 0;
  const bool a_ok = a_aligned || (K > 0 && aligned2(A) && chunk_tail_readable(A, M, K, lda));
  const bool b_ok = b_aligned || (N > 0 && aligned2(B) && chunk_tail_readable(B, K, N, ldb));
  const bool k_tail = a_ok && K % 8 != 0;
  const int64_t lda_p = a_ok ? lda : (int64_t)round_up(K, 8);
  const int64_t ldb_p = b_ok ? ldb : (int64_t)round_up(N, 8);
  const int64_t tiles = (int64_t)((M + kTileM - 1) / kTileM) * ((N + kTileN - 1) / kTileN);
  const bool fits = fast_extent_a(M, K, lda_p) < kLimit && fast_extent_b(N, K, ldb_p) < kLimit &&
                    tiles <= 0x7fffffff;
  // Aligned operands too large for 32-bit offsets from their base run the
  // WIDE form (per-tile / per-K-tile resources) when one 256-row panel of A
  // and one 32-row panel of B stay below 2^31 bytes.
  const bool wide = !fits && a_aligned && b_aligned && (int64_t)kTileM * lda * 2 < kLimit &&
                    (int64_t)kDmaK * ldb * 2 < kLimit && tiles <= 0x7fffffff;
  if (force_generic || (!fits && !wide)) return run_generic(dtype, A, lda, B, ldb, C, ldc, M, N, K, stream);
  if (wide) {
    const TilePlan plan = plan_tiles(st->num_cus, M, N, K, force_shape, false);
    const TileShape& ts = kTileShapes[plan.shape];
    FastArgs f{};
    f.A = static_cast<const uint16_t*>(A);
    f.B = static_cast<const uint16_t*>(B);
    f.C = C;
    f.lda = (int)lda;
    f.ldb = (int)ldb;
    f.ldc = ldc;
    f.M = M;
    f.N = N;
    f.K = K;
    f.tiles_m = (M + ts.tm - 1) / ts.tm;
    f.tiles_n = (N + ts.tn - 1) / ts.tn;
    f.c_vec = aligned16(C) && ldc % 4 == 0;
    f.splits = 1;
    return dtype == HCG_F16 ? launch_dma<HCG_F16, true>(f, plan.shape, stream)
                            : launch_dma<HCG_BF16, true>(f, plan.shape, stream);
  }
  // Workspace: repacked operands (those that cannot be read in place), then
  // the split partials [splits][M][N].
  const size_t a_sz = a_ok ? 0 : round_up((size_t)M * lda_p * 2, 256);
  const size_t b_sz = b_ok ? 0 : round_up((size_t)K * ldb_p * 2, 256);
  // Explicit tile shapes run without a K split; "auto" and "tiled" may split.
  const TilePlan plan = plan_tiles(st->num_cus, M, N, K, force_shape, force_shape < 0, nullptr,
                                   sc.room(a_sz + b_sz));
  const TileShape& ts = kTileShapes[plan.shape];
  if ((int64_t)((M + ts.tm - 1) / ts.tm) * ((N + ts.tn - 1) / ts.tn) * plan.splits > 0x7fffffff)
    return run_generic(dtype, A, lda, B, ldb, C, ldc, M, N, K, stream);
  const size_t p_sz = plan.splits > 1 ? (size_t)plan.splits * M * N * sizeof(float) : 0;
  void* ws = nullptr;
  if (a_sz + b_sz + p_sz > 0) {
    const int rc = get_scratch(sc, a_sz + b_sz + p_sz, &ws);
    if (rc != HCG_OK) return rc;
  }
  const uint16_t* a_use = static_cast<const uint16_t*>(A);
  const uint16_t* b_use = static_cast<const uint16_t*>(B);
  if (!a_ok || !b_ok) {
    // Operands that cannot be read in place: zero-padded, 16-byte aligned copies.
    uint16_t* a_p = static_cast<uint16_t*>(ws);
    uint16_t* b_p = reinterpret_cast<uint16_t*>(static_cast<char*>(ws) + a_sz);
    RepackJob ja{}, jb{};
    if (!a_ok) {
      ja = RepackJob{a_use, lda, M, K, a_p, (int)lda_p, (int64_t)M * (lda_p / 8)};
      a_use = a_p;
    }
    if (!b_ok) {
      jb = RepackJob{b_use, ldb, K, N, b_p, (int)ldb_p, (int64_t)K * (ldb_p / 8)};
      b_use = b_p;
    }
    const int64_t n = ja.chunks + jb.chunks;
    const int64_t per_block = (int64_t)256 * kRepackPer;
    repack_kernel<<<(unsigned)((n + per_block - 1) / per_block), 256, 0, stream>>>(ja, jb);
    HCG_HIP_CHECK(hipGetLastError());
  }
  FastArgs f{};
  f.A = a_use;
  f.B = b_use;
  f.C = C;
  f.lda = (int)lda_p;
  f.ldb = (int)ldb_p;
  f.ldc = ldc;
  f.M = M;
  f.N = N;
  f.K = K;
  f.tiles_m = (M + ts.tm - 1) / ts.tm;
  f.tiles_n = (N + ts.tn - 1) / ts.tn;
  // Range-check extents cover the chunk that holds the last valid element
  // (never past that chunk).
  f.a_bytes = (int)((((int64_t)M - 1) * lda_p + (int64_t)round_up(K, 8)) * 2);
  f.b_bytes = (int)((((int64_t)K - 1) * ldb_p + (int64_t)round_up(N, 8)) * 2);
  f.c_vec = aligned16(C) && ldc % 4 == 0;
  f.splits = 1;
  if (plan.splits > 1) {
    // K cut into equal runs of whole 32-row K tiles; no split is empty.
    const int nk = (K + kDmaK - 1) / kDmaK;
    f.kchunk = (nk + plan.splits - 1) / plan.splits * kDmaK;
    f.splits = (K + f.kchunk - 1) / f.kchunk;
    f.ws = reinterpret_cast<float*>(static_cast<char*>(ws) + a_sz + b_sz);
    f.ws_vec = N % 4 == 0;  // 16-byte partial rows (the workspace base is 256-byte aligned)
  }
  const int rc = k_tail ? (dtype == HCG_F16 ? launch_dma<HCG_F16, false, true>(f, plan.shape, stream)
                                          : launch_dma<HCG_BF16, false, true>(f, plan.shape, stream))
                        : (dtype == HCG_F16 ? launch_dma<HCG_F16, false>(f, plan.shape, stream)
                                            : launch_dma<HCG_BF16, false>(f, plan.shape, stream));
  if (rc != HCG_OK || f.splits == 1) return rc;
  return launch_reduce(f.ws, C, ldc, M, N, M, f.splits, aligned16(C) && ldc % 4 == 0, stream);
}

// Remainder peeling (HCG_ALGO_AUTO only).  A few rows or columns past a
// multiple of 256 can cost the tiled kernel a whole extra round of tiles
// (4100 x 4096 x 4096: 272 tiles of 256 x 256 for 256 CUs).  When the model
// prefers it, the tile-aligned bulk runs on the tiled kernel and the
// remainder -- up to 128 rows, or up to 64 columns -- on the matching
// streaming kernel, each writing its own rows or columns of C.
struct Peel {
  int rows = 0, cols = 0;
};

double tiled_cost(int num_cus, int M, int N, int K) {
  double cost = 0;
  plan_tiles(num_cus, M, N, K, -1, true, &cost);
  return cost;
}

// A streaming launch in the tile model's units (0.73 us per 256 x 256 x 1):
// a fixed 8 us (launch behind the tiled kernel, ramp-up, the K split's
// reduce) plus its bytes at 5 TB/s.  Fitted so that short-K shapes
// (4100 x 4096 x 256: 20.4 us unpeeled, 23.1 us peeled) stay unpeeled.
double stream_units(double bytes) { return (8.0 + bytes / 5.0e6) / 0.73 * 65536.0; }

Peel plan_peel(const DeviceState* st, const void* A, int64_t lda, const void* B, int64_t ldb, int M, int N,
               int K) {
  Peel p;
  double best = 0.95 * tiled_cost(st->num_cus, M, N, K);  // a clear gain pays for the second launch
  const int rm = M % 256;
  if (M > 256 && rm > 0 && rm <= 128 &&
      (rm <= 16 || stream_fits(static_cast<const uint16_t*>(A) + (int64_t)(M - rm) * lda, lda, B, ldb, rm, N, K))) {
    const double c = tiled_cost(st->num_cus, M - rm, N, K) +
                     stream_units(2.0 * K * N + 2.0 * rm * K + 4.0 * rm * N);
    if (c < best) {
      best = c;
      p.rows = rm;
    }
  }
  const int rn = N % 256;
  if (N > 256 && rn > 0 && rn <= 64 &&
      rowstream_fits(A, lda, static_cast<const uint16_t*>(B) + (N - rn), ldb, M, rn, K)) {
    const double c = tiled_cost(st->num_cus, M, N - rn, K) +
                     stream_units(2.0 * M * K + 2.0 * K * rn + 4.0 * M * rn);
    if (c < best) {
      best = c;
      p.rows = 0;
      p.cols = rn;
    }
  }
  return p;
}

// `fixed` / `fixed_bytes`: a caller-owned scratch buffer that replaces the
// stream's library workspace (nothing is allocated); null for the default.
int gemm_impl(int algo, int dtype, const void* A, int64_t lda, const void* B, int64_t ldb,
              float* C, int64_t ldc, int64_t M, int64_t N, int64_t K, void* stream_ptr,
              bool no_alloc = false) {
  if (dtype != HCG_F16 && dtype != HCG_BF16)
    return set_error(HCG_EINVAL, "dtype must be HCG_F16 (0) or HCG_BF16 (1), got %d", dtype);
  if (algo < HCG_ALGO_AUTO || algo > HCG_ALGO_NARROW)
    return set_error(HCG_EINVAL, "unknown algo %d", algo);
  if (M < 0 || N < 0 || K < 0)
    return set_error(HCG_EINVAL, "negative extent: M=%lld N=%lld K=%lld", (long long)M,
                     (long long)N, (long long)K);
  const int64_t kMaxExtent = (int64_t)1 << 30;
  if (M > kMaxExtent || N > kMaxExtent || K > kMaxExtent)
    return set_error(HCG_EINVAL, "extent above 2^30: M=%lld N=%lld K=%lld", (long long)M,
                     (long long)N, (long long)K);
  if (algo == HCG_ALGO_SKINNY && M > 16 * kStMaxRowBlocks)
    return set_error(HCG_EINVAL, "the skinny kernel needs M <= 128, got M=%lld", (long long)M);
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
    fill_zero_kernel<<<fill_blocks(total), 256, 0, stream>>>(C, ldc, (int)M, (int)N);
    HCG_HIP_CHECK(hipGetLastError());
    t_last_error.clear();
    return HCG_OK;
  }

  // N <= 64 is HBM-bound on A: stream A in 256-byte row pieces (for M <=
  // 128 too -- 64 x 32 x 2^20 fp16: 36 us against 154 us on the skinny
  // kernel, which streams B in 128-column blocks mostly past N).
  const bool use_narrow = algo == HCG_ALGO_NARROW ||
                          (algo == HCG_ALGO_AUTO && rowstream_fits(A, lda, B, ldb, M, N, K));
  // Otherwise M <= 16, and M <= 64 where the streaming kernel applies, is
  // HBM-bound: B is streamed once through a skinny kernel instead of
  // occupying only N/128 workgroups of the tiled kernel.  Rows 65..128 (the
  // streaming kernel's eight row blocks) go to the tiled kernel, which splits
  // K to fill the chip, when it reads B in place: fp16 us, streaming ->
  // tiled: 128^3 5.9 -> 4.4, 128 x 512 x 512 9.2 -> 6.4, 128 x 2048 x 2048
  // 14.1 -> 11.1, 128 x 8192 x 1024 16.2 -> 9.8, 128 x 16384 x 512 17.2 ->
  // 7.3, 128 x 8192 x 8192 38.3 -> 35.7; with B's rows unaligned 128 x 3001
  // x 1027 16.4 -> 14.0, 100 x 50257 x 1024 35.4 -> 23.6, 72 x 12289 x 4096
  // 34.1 -> 27.8.  The streaming kernel led by at most 9% (80 x 4096 x 4096
  // 16.6 against 18.0, 128 x 1001 x 2048 12.1 / 13.2).
  const bool tiled_rows = M > 64 && ((aligned16(B) && ldb % 8 == 0) ||
                                     (K > 0 && N > 0 && aligned2(B) && chunk_tail_readable(B, K, N, ldb)));
  const bool use_skinny =
      !use_narrow && (algo == HCG_ALGO_SKINNY ||
                      (algo == HCG_ALGO_AUTO && (M <= 16 || (!tiled_rows && stream_fits(A, lda, B, ldb, M, N, K)))));
  if (algo == HCG_ALGO_NARROW && !rowstream_fits(A, lda, B, ldb, M, N, K))
    return set_error(HCG_EINVAL,
                     "the narrow kernel needs N <= 64 (and offsets of B below 2^31) "
                     "(M=%lld N=%lld K=%lld)", (long long)M, (long long)N, (long long)K);
  Scratch sc;
  sc.st = st;
  sc.stream = stream;
  if (no_alloc) {
    if (st->scratch == nullptr) return set_error(HCG_EHIP, "%s", st->scratch_error.c_str());
    sc.fixed = st->scratch;
    sc.cap = HCG_NOALLOC_SCRATCH_BYTES;
  }
  // Workspaces stay valid while ws_mutex is held (see stream_workspace), so
  // the lock covers the launches too; a launch only enqueues work.  The two
  // launches of a peeled shape share the scratch in stream order.
  std::lock_guard<std::mutex> lock(st->ws_mutex);
  if (use_narrow) {
    rc = run_rowstream(sc, dtype, A, lda, B, ldb, C, ldc, (int)M, (int)N, (int)K);
  } else if (use_skinny) {
    rc = run_skinny(sc, dtype, A, lda, B, ldb, C, ldc, (int)M, (int)N, (int)K);
  } else {
    const int force_shape = algo >= HCG_ALGO_TILED_256x256 ? algo - HCG_ALGO_TILED_256x256 : -1;
    Peel peel = algo == HCG_ALGO_AUTO ? plan_peel(st, A, lda, B, ldb, (int)M, (int)N, (int)K) : Peel{};
    // With fixed scratch, peel only when the remainder's repacked operand
    // fits too, so that a call that cannot run fails before any launch.
    if (sc.fixed && peel.rows > 0 &&
        !stream_a_in_place(static_cast<const uint16_t*>(A) + (M - peel.rows) * lda, lda, peel.rows, K) &&
        round_up((size_t)peel.rows * round_up(K, 8) * 2, 256) > sc.cap)
      peel = Peel{};
    if (sc.fixed && peel.cols > 0 && !(aligned16(static_cast<const uint16_t*>(B) + (N - peel.cols)) && ldb % 8 == 0) &&
        round_up((size_t)K * round_up(peel.cols, 8) * 2, 256) > sc.cap)
      peel = Peel{};
    if (peel.rows > 0) {
      const int mm = (int)M - peel.rows;
      rc = run_tiled(sc, dtype, A, lda, B, ldb, C, ldc, mm, (int)N, (int)K, false, -1);
      if (rc == HCG_OK)
        rc = run_skinny(sc, dtype, static_cast<const uint16_t*>(A) + (int64_t)mm * lda, lda, B, ldb,
                        C + (int64_t)mm * ldc, ldc, peel.rows, (int)N, (int)K);
    } else if (peel.cols > 0) {
      const int nn = (int)N - peel.cols;
      rc = run_tiled(sc, dtype, A, lda, B, ldb, C, ldc, (int)M, nn, (int)K, false, -1);
      if (rc == HCG_OK)
        rc = run_rowstream(sc, dtype, A, lda, static_cast<const uint16_t*>(B) + nn, ldb, C + nn, ldc, (int)M,
                           peel.cols, (int)K);
    } else {
      rc = run_tiled(sc, dtype, A, lda, B, ldb, C, ldc, (int)M, (int)N, (int)K, algo == HCG_ALGO_GENERIC,
                     force_shape);
    }
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

int hcg_gemm_noalloc(int dtype, const void* A, int64_t lda, const void* B, int64_t ldb, float* C,
                     int64_t ldc, int64_t M, int64_t N, int64_t K, void* stream) {
  return gemm_impl(HCG_ALGO_AUTO, dtype, A, lda, B, ldb, C, ldc, M, N, K, stream, true);
}

const char* hcg_last_error(void) { return t_last_error.c_str(); }

int hcg_version(void) { return 100; }

#ifdef HCG_STAMPS
// The HCG_STAMPS build only (no counterpart in the reference; for bench.py
// --stamps): the device buffer of `records` 8-word records that the tiled and
// streaming GEMM kernels fill, record b for workgroup b (NULL: none).
int hcg_stamps_set(void* buf, int64_t records) {
  t_last_error.clear();
  uint64_t* p = static_cast<uint64_t*>(buf);
  const int64_t cap = buf ? records : 0;
  HCG_HIP_CHECK(hipMemcpyToSymbol(HIP_SYMBOL(g_stamp_buf), &p, sizeof p));
  HCG_HIP_CHECK(hipMemcpyToSymbol(HIP_SYMBOL(g_stamp_cap), &cap, sizeof cap));
  return HCG_OK;
}
#endif

int hcg_operand_in_place(const void* base, int64_t rows, int64_t cols, int64_t ld) {
  t_last_error.clear();
  std::call_once(g_global_once, global_init);
  if (base == nullptr || rows <= 0 || cols <= 0 || ld < cols) {
    set_error(HCG_EINVAL, "operand: base %s, rows %lld, cols %lld, ld %lld", base ? "set" : "NULL",
              (long long)rows, (long long)cols, (long long)ld);
    return -1;
  }
  if (aligned16(base) && ld % 8 == 0) return 1;
  return aligned2(base) && chunk_tail_readable(base, rows, cols, ld) ? 1 : 0;
}

}  // extern "C"
