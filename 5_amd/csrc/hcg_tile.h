// hcg_tile.h -- masked tile access primitives for gfx950 device code.
//
// The hc DSL's tile semantics (hc/simulator.py:1304-1357, 1416-1458;
// doc/langref.md:530-596):
//   * group.load(view, shape=(h, w)) returns an h x w tile whose element
//     (r, c) is active iff it lies inside the view's extent; the payload of
//     inactive elements is poison, and with_inactive(v) replaces it with v;
//   * group.load(view, mask=m) additionally requires m[r][c] to be active
//     and true;
//   * group.store(view, tile) writes only the active elements that lie
//     inside the view's extent; nothing else in memory changes.
// On gfx950 these become bounds-predicated vector accesses: an element
// outside the extent is never read (its payload is the fill value) and
// never written.  Two forms are provided:
//   * row-chunk loads/stores through plain pointers (up to 8 consecutive
//     elements of one row, one 16-byte access when the chunk is whole and
//     aligned, element accesses at the edges), used by register-staged
//     kernels and the tile gather/scatter entry points;
//   * buffer-resource DMA into LDS (buffer_load ... lds), where the
//     hardware range check returns zeros for offsets at or beyond the
//     extent and a per-lane redirect (dma_offset) sends chunks that are out
//     of range in 2-D (past the row's columns or the matrix's rows) beyond
//     it, used by the DMA-fed GEMM kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hcg {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

// ---------------------------------------------------------------------------
// Row chunks through plain pointers
// ---------------------------------------------------------------------------

// 8 consecutive 16-bit elements of one row starting at column col0, packed
// two per 32-bit word; columns at or beyond ncols read as `fill` (the
// masked load followed by with_inactive(fill)).  kVec: the row is 16-byte
// aligned at every multiple of 8 columns, so a whole in-range chunk is one
// 128-bit load.
template <bool kVec>
__device__ __forceinline__ u32x4 load_row8_u16(const uint16_t* rowp, int64_t col0, int64_t ncols,
                                               uint16_t fill = 0) {
  if (kVec && col0 + 8 <= ncols) return *reinterpret_cast<const u32x4*>(rowp + col0);
  uint32_t w[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int64_t c = col0 + 2 * p;
    const uint32_t lo = (c < ncols) ? rowp[c] : fill;
    const uint32_t hi = (c + 1 < ncols) ? rowp[c + 1] : fill;
    w[p] = lo | (hi << 16);
  }
  return u32x4{w[0], w[1], w[2], w[3]};
}

// Bit e of the result is set iff column col0 + e (e < n) is inside
// [0, ncols) and row is inside [0, nrows): the activity of a chunk of a
// shape= load.
__device__ __forceinline__ uint32_t chunk_active_bits(int64_t row, int64_t nrows, int64_t col0, int64_t ncols,
                                                      int n) {
  if (row < 0 || row >= nrows) return 0u;
  uint32_t bits = 0;
  for (int e = 0; e < n; ++e) {
    const int64_t c = col0 + e;
    if (c >= 0 && c < ncols) bits |= 1u << e;
  }
  return bits;
}

// Loads the n (<= 8) elements of T at rowp[col0 + e] whose bit is set in
// `active` (one vector access when all n are active and the chunk is
// 16-byte aligned); others get `fill`.
template <typename T>
__device__ __forceinline__ void load_chunk(const T* rowp, int64_t col0, int n, uint32_t active, T fill,
                                           T (&out)[8]) {
  const T* p = rowp + col0;
  const bool whole = n * sizeof(T) == 16 && active == (1u << n) - 1u &&
                     (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
  if (whole) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(p);
    __builtin_memcpy(out, &v, 16);
    return;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) out[e] = (e < n && ((active >> e) & 1u)) ? p[e] : fill;
}

// Stores the elements of `v` whose bit is set in `write` to rowp[col0 + e]
// (one vector access when all n are written and the chunk is 16-byte
// aligned); nothing else is touched.
template <typename T>
__device__ __forceinline__ void store_chunk(T* rowp, int64_t col0, int n, uint32_t write, const T (&v)[8]) {
  T* p = rowp + col0;
  const bool whole = n * sizeof(T) == 16 && write == (1u << n) - 1u &&
                     (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
  if (whole) {
    u32x4 w;
    __builtin_memcpy(&w, v, 16);
    *reinterpret_cast<u32x4*>(p) = w;
    return;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (e < n && ((write >> e) & 1u)) p[e] = v[e];
}

// ---------------------------------------------------------------------------
// Buffer-resource DMA into LDS
// ---------------------------------------------------------------------------

// Raw buffer resource: base, no swizzle/stride, `bytes` records.  Loads at
// or beyond `bytes` return 0 (the hardware range check).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}

// A byte offset past every extent used here (extents stay below 2^31 - 16).
constexpr int kOobOffset = 0x7ffffff0;

// 16 bytes per lane from the buffer at voff + soff into LDS at dst + 16*lane.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, lds_void* dst, int voff, int soff = 0) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, voff, soff, 0, 0);
}

// The offset a lane's DMA uses for a chunk: its byte offset when the chunk
// is inside the 2-D extent, else kOobOffset so the range check zero-fills
// it.
__device__ __forceinline__ int dma_offset(bool inside, int offset) { return inside ? offset : kOobOffset; }

}  // namespace hcg
