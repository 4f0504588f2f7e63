// Ordered per-row stream compaction (compact.hip).
#pragma once
#include "glif_internal.h"

namespace glif {

// Scratch bytes for compacting a [rows][cols] predicate.
size_t compact_scratch_bytes(int64_t rows, int64_t cols);

// For inputs x [T][B][C] uint8: per step t, the ascending list of columns c with any
// x[t][b][c] > 0 (pre[]) and their batch masks (mask[]); row_off [T+1] int64 holds
// each step's start.  pre/mask need room for T*C entries.
int build_batch_mask_lists(const uint8_t *x, int32_t T, int32_t B, int64_t C, int64_t *row_off,
                           int32_t *pre, uint32_t *mask, void *scratch, hipStream_t s);

// Backward windows (see compact.hip SrcWindowMask): per window j the ascending
// columns with any input in the window's W reverse steps, masks over w*B + b.
int build_window_mask_lists(const uint8_t *x, int32_t T, int32_t B, int64_t C, int32_t W,
                            int32_t n_windows, int64_t *row_off, int32_t *pre, uint32_t *mask,
                            void *scratch, hipStream_t s);

}  // namespace glif
