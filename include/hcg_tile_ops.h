/*
 * hcg_tile_ops.h -- C ABI of the gfx950 masked tile gather / scatter: the hc
 * DSL's tile loads and stores with their masking rules, over batches of
 * tiles of a 2-D row-major view.
 *
 * A view is `rows` x `cols` elements of `elem_bytes` bytes (2, 4 or 8) with
 * row stride `ld` elements (ld >= cols).  Tile t (0 <= t < ntiles) is
 * th x tw with its origin at view element (origins[2t], origins[2t+1]);
 * tiles are stored densely, tile-major then row-major: element (t, r, c) at
 * index (t*th + r)*tw + c.  Element (t, r, c) lies inside the view iff
 * 0 <= origin_row + r < rows and 0 <= origin_col + c < cols.  Masks are
 * bytes, nonzero = active.  All pointers are device pointers; calls are
 * asynchronous on `stream`.  Status codes as in hcg_gemm.h.
 */
#ifndef HCG_TILE_OPS_H
#define HCG_TILE_OPS_H

#include <stdint.h>

#include "hcg_gemm.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Tile gather: group.load(view[row0:, col0:], shape=(th, tw)) -- or with
 * in_mask, group.load(..., mask=m) -- then with_inactive(fill) and .mask
 * (hc/simulator.py:1304-1357, doc/langref.md:530-596).  Element (t, r, c)
 * is active iff it lies inside the view and, when in_mask is not NULL,
 * in_mask[(t*th + r)*tw + c] != 0.  out gets the view's element where
 * active and the low elem_bytes bytes of fill_bits elsewhere; out_mask (if
 * not NULL) gets 1 / 0.  Elements outside the view are never read.
 * Replaces the simulator's per-workgroup masked tile load
 * (SimCurrentGroup.load, hc/simulator.py:302-330). */
int hcg_tile_load(int elem_bytes, const void* src, int64_t ld, int64_t rows, int64_t cols, const int64_t* origins,
                  int64_t ntiles, int64_t th, int64_t tw, const uint8_t* in_mask, uint64_t fill_bits, void* out,
                  uint8_t* out_mask, void* stream);

/* Tile scatter: group.store(view[row0:, col0:], tile) (hc/simulator.py:355-358,
 * 1416-1458).  Writes tiles[(t*th + r)*tw + c] to the view for every
 * element that lies inside the view and is active (tile_mask NULL: all
 * active); no other memory is written.  Where two tiles write the same
 * view element, which one lands is unspecified. */
int hcg_tile_store(int elem_bytes, void* dst, int64_t ld, int64_t rows, int64_t cols, const int64_t* origins,
                   int64_t ntiles, int64_t th, int64_t tw, const void* tiles, const uint8_t* tile_mask,
                   void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HCG_TILE_OPS_H */
