// hcg_tile.hip -- masked tile gather / scatter on gfx950: the hc DSL's
// group.load(view, shape=) / group.load(view, mask=), with_inactive(fill),
// .mask and group.store(view, tile) over batches of tiles, built on the
// primitives of hcg_tile.h (the tail machinery of the GEMM kernels).
//
// Reference semantics: hc/simulator.py:1304-1357 (_load_value,
// _load_masked, _copy_loaded_value: the in-bounds overlap is copied, the
// rest of the tile is inactive), hc/simulator.py:1416-1458 (_store_value,
// _store_from_value: only active elements inside the target view are
// written), doc/langref.md:530-596 (masking, with_inactive, .mask).
//
// One thread handles one chunk of 16 bytes of one tile row (8, 4 or 2
// elements); chunks wholly inside the source row and 16-byte aligned move
// as one vector access, edge chunks element by element, and elements
// outside the view are never read or written.

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "hcg_runtime.h"
#include "hcg_tile.h"
#include "hcg_tile_ops.h"

namespace {

struct TileJob {
  const void* src;  // load: source view; store: unused
  void* dst;        // store: target view; load: unused
  int64_t ld;       // view row stride, elements
  int64_t rows, cols;
  const int64_t* origins;  // [ntiles][2] = (row0, col0)
  int64_t ntiles, th, tw;
  int64_t chunks_per_row;  // ceil(tw / elements per chunk)
  int64_t total_chunks;    // ntiles * th * chunks_per_row
  const uint8_t* mask_in;  // load: mask= operand; store: the tile's activity (NULL: all active)
  const void* tiles_in;    // store: the tiles
  void* tiles_out;         // load: the tiles
  uint8_t* mask_out;       // load: the tiles' activity (may be NULL)
  uint64_t fill_bits;      // load: with_inactive value, low sizeof(T) bytes
};

template <typename T>
__device__ __forceinline__ void decompose(const TileJob& j, int64_t idx, int64_t& t, int64_t& r, int64_t& c0) {
  const int64_t row_id = idx / j.chunks_per_row;  // t * th + r
  c0 = (idx - row_id * j.chunks_per_row) * (16 / (int64_t)sizeof(T));
  t = row_id / j.th;
  r = row_id - t * j.th;
}

template <typename T>
__global__ __launch_bounds__(256) void tile_load_kernel(TileJob j) {
  constexpr int kN = 16 / sizeof(T);
  T fill;
  __builtin_memcpy(&fill, &j.fill_bits, sizeof(T));
  for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < j.total_chunks;
       idx += (int64_t)gridDim.x * 256) {
    int64_t t, r, c0;
    decompose<T>(j, idx, t, r, c0);
    const int n = (int)min((int64_t)kN, j.tw - c0);
    const int64_t row = j.origins[2 * t] + r;
    const int64_t col = j.origins[2 * t + 1] + c0;
    const int64_t out_off = (t * j.th + r) * j.tw + c0;
    uint32_t active = hcg::chunk_active_bits(row, j.rows, col, j.cols, n);
    if (j.mask_in) {
#pragma unroll
      for (int e = 0; e < kN; ++e)
        if (e < n && j.mask_in[out_off + e] == 0) active &= ~(1u << e);
    }
    // Rows outside the view are never addressed (active is 0 for them).
    const T* rowp = static_cast<const T*>(j.src) + (active ? row * j.ld : 0);
    T v[8];
    hcg::load_chunk<T>(rowp, col, n, active, fill, v);
    hcg::store_chunk<T>(static_cast<T*>(j.tiles_out) + (t * j.th + r) * j.tw, c0, n, (1u << n) - 1u, v);
    if (j.mask_out) {
#pragma unroll
      for (int e = 0; e < kN; ++e)
        if (e < n) j.mask_out[out_off + e] = (active >> e) & 1u;
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void tile_store_kernel(TileJob j) {
  constexpr int kN = 16 / sizeof(T);
  for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < j.total_chunks;
       idx += (int64_t)gridDim.x * 256) {
    int64_t t, r, c0;
    decompose<T>(j, idx, t, r, c0);
    const int n = (int)min((int64_t)kN, j.tw - c0);
    const int64_t row = j.origins[2 * t] + r;
    const int64_t col = j.origins[2 * t + 1] + c0;
    const int64_t in_off = (t * j.th + r) * j.tw + c0;
    uint32_t write = hcg::chunk_active_bits(row, j.rows, col, j.cols, n);
    if (j.mask_in) {
#pragma unroll
      for (int e = 0; e < kN; ++e)
        if (e < n && j.mask_in[in_off + e] == 0) write &= ~(1u << e);
    }
    if (write == 0) continue;
    T v[8];
    hcg::load_chunk<T>(static_cast<const T*>(j.tiles_in) + (t * j.th + r) * j.tw, c0, n, (1u << n) - 1u, T{},
                       v);
    hcg::store_chunk<T>(static_cast<T*>(j.dst) + row * j.ld, col, n, write, v);
  }
}

// Argument checks shared by both entry points; fills the geometry of j.
int prepare(int elem_bytes, int64_t ld, int64_t rows, int64_t cols, const void* view, const int64_t* origins,
            int64_t ntiles, int64_t th, int64_t tw, const char* what, TileJob& j) {
  if (elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8)
    return hcg::set_error(HCG_EINVAL, "%s: elem_bytes must be 2, 4 or 8, got %d", what, elem_bytes);
  if (rows < 0 || cols < 0 || ntiles < 0 || th < 0 || tw < 0)
    return hcg::set_error(HCG_EINVAL, "%s: negative extent (rows=%lld cols=%lld ntiles=%lld th=%lld tw=%lld)",
                          what, (long long)rows, (long long)cols, (long long)ntiles, (long long)th,
                          (long long)tw);
  if (rows > 0 && cols > 0) {
    if (view == nullptr) return hcg::set_error(HCG_EINVAL, "%s: view pointer is NULL", what);
    if (ld < cols) return hcg::set_error(HCG_EINVAL, "%s: ld (%lld) < cols (%lld)", what, (long long)ld,
                                         (long long)cols);
  }
  if (ntiles > 0 && origins == nullptr) return hcg::set_error(HCG_EINVAL, "%s: origins is NULL", what);
  const int64_t n = 16 / elem_bytes;
  j.ld = ld;
  j.rows = rows;
  j.cols = cols;
  j.origins = origins;
  j.ntiles = ntiles;
  j.th = th;
  j.tw = tw;
  j.chunks_per_row = (tw + n - 1) / n;
  j.total_chunks = ntiles * th * j.chunks_per_row;
  return HCG_OK;
}

unsigned grid_for(int64_t chunks) {
  const int64_t blocks = (chunks + 255) / 256;
  return (unsigned)(blocks < 65536 ? blocks : 65536);
}

}  // namespace

extern "C" {

int hcg_tile_load(int elem_bytes, const void* src, int64_t ld, int64_t rows, int64_t cols, const int64_t* origins,
                  int64_t ntiles, int64_t th, int64_t tw, const uint8_t* in_mask, uint64_t fill_bits, void* out,
                  uint8_t* out_mask, void* stream) {
  TileJob j{};
  int rc = prepare(elem_bytes, ld, rows, cols, src, origins, ntiles, th, tw, "hcg_tile_load", j);
  if (rc != HCG_OK) return rc;
  if (j.total_chunks == 0) {
    hcg::t_last_error.clear();
    return HCG_OK;
  }
  if (out == nullptr) return hcg::set_error(HCG_EINVAL, "hcg_tile_load: out is NULL");
  j.src = src;
  j.mask_in = in_mask;
  j.tiles_out = out;
  j.mask_out = out_mask;
  j.fill_bits = fill_bits;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned grid = grid_for(j.total_chunks);
  if (elem_bytes == 2)
    tile_load_kernel<uint16_t><<<grid, 256, 0, s>>>(j);
  else if (elem_bytes == 4)
    tile_load_kernel<uint32_t><<<grid, 256, 0, s>>>(j);
  else
    tile_load_kernel<uint64_t><<<grid, 256, 0, s>>>(j);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hcg::set_error(HCG_EHIP, "tile_load_kernel launch failed: %s", hipGetErrorString(e));
  hcg::t_last_error.clear();
  return HCG_OK;
}

int hcg_tile_store(int elem_bytes, void* dst, int64_t ld, int64_t rows, int64_t cols, const int64_t* origins,
                   int64_t ntiles, int64_t th, int64_t tw, const void* tiles, const uint8_t* tile_mask,
                   void* stream) {
  TileJob j{};
  int rc = prepare(elem_bytes, ld, rows, cols, dst, origins, ntiles, th, tw, "hcg_tile_store", j);
  if (rc != HCG_OK) return rc;
  if (j.total_chunks == 0 || rows == 0 || cols == 0) {
    hcg::t_last_error.clear();
    return HCG_OK;
  }
  if (tiles == nullptr) return hcg::set_error(HCG_EINVAL, "hcg_tile_store: tiles is NULL");
  j.dst = dst;
  j.tiles_in = tiles;
  j.mask_in = tile_mask;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned grid = grid_for(j.total_chunks);
  if (elem_bytes == 2)
    tile_store_kernel<uint16_t><<<grid, 256, 0, s>>>(j);
  else if (elem_bytes == 4)
    tile_store_kernel<uint32_t><<<grid, 256, 0, s>>>(j);
  else
    tile_store_kernel<uint64_t><<<grid, 256, 0, s>>>(j);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hcg::set_error(HCG_EHIP, "tile_store_kernel launch failed: %s", hipGetErrorString(e));
  hcg::t_last_error.clear();
  return HCG_OK;
}

}  // extern "C"
