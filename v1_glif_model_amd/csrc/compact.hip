// Ordered stream compaction (tf.where(z > 0), models.py:128).
//
// A [rows][cols] predicate is cut into tiles of kTile consecutive elements that
// never cross a row.  Pass 1 counts the active elements of every tile, pass 2
// scans the tile counts (one block), pass 3 re-evaluates the predicate and writes
// each active element at its row-major rank: within a tile, 256-element rounds are
// ranked with wave ballots plus a per-wave prefix in LDS.  The output order is the
// row-major order tf.where produces, bit for bit.
#include "glif_internal.h"
#include "compact.h"

namespace glif {

constexpr int kTile = 1024;

__device__ inline int wave_inclusive_scan(int x) {
    const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        int y = __shfl_up(x, o, kWave);
        if (lane >= o) x += y;
    }
    return x;
}

template <class Src>
__global__ void __launch_bounds__(kBlock) k_compact_count(Src src, int64_t cols, int tiles_per_row,
                                                          int32_t *__restrict__ tile_count) {
    __shared__ int wsum[kBlock / kWave];
    const int64_t tile = blockIdx.x;
    const int64_t row = tile / tiles_per_row;
    const int64_t c0 = (tile % tiles_per_row) * kTile;
    int cnt = 0;
    for (int i = threadIdx.x; i < kTile; i += kBlock) {
        int64_t c = c0 + i;
        if (c < cols && src.eval(row, c) != 0u) ++cnt;
    }
    // block reduction
    for (int o = kWave / 2; o > 0; o >>= 1) cnt += __shfl_down(cnt, o, kWave);
    if ((threadIdx.x & (kWave - 1)) == 0) wsum[threadIdx.x / kWave] = cnt;
    __syncthreads();
    if (threadIdx.x == 0) {
        int t = 0;
        for (int w = 0; w < kBlock / kWave; ++w) t += wsum[w];
        tile_count[tile] = t;
    }
}

// Exclusive scan of n counts into off[0..n] (off[n] = total), one block.
__global__ void __launch_bounds__(1024) k_scan_counts(const int32_t *__restrict__ cnt, int64_t n,
                                                      int64_t *__restrict__ off) {
    __shared__ int64_t wsum[1024 / kWave];
    __shared__ int64_t carry;
    if (threadIdx.x == 0) carry = 0;
    __syncthreads();
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    for (int64_t base = 0; base < n; base += 1024) {
        int64_t i = base + threadIdx.x;
        int v = i < n ? cnt[i] : 0;
        int inc = wave_inclusive_scan(v);
        if (lane == kWave - 1) wsum[wid] = inc;
        __syncthreads();
        int64_t before = carry;
        for (int w = 0; w < wid; ++w) before += wsum[w];
        if (i < n) off[i] = before + inc - v;
        __syncthreads();
        if (threadIdx.x == 0) {
            int64_t t = 0;
            for (int w = 0; w < 1024 / kWave; ++w) t += wsum[w];
            carry += t;
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) off[n] = carry;
}

template <class Src, class Sink>
__global__ void __launch_bounds__(kBlock) k_compact_write(Src src, Sink sink, int64_t rows, int64_t cols,
                                                          int tiles_per_row,
                                                          const int64_t *__restrict__ tile_off,
                                                          int64_t *__restrict__ row_off,
                                                          int64_t *__restrict__ total_out) {
    __shared__ int wcnt[kBlock / kWave];
    const int64_t tile = blockIdx.x;
    const int64_t row = tile / tiles_per_row;
    const int64_t c0 = (tile % tiles_per_row) * kTile;
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    if (threadIdx.x == 0) {
        if (row_off && tile % tiles_per_row == 0) row_off[row] = tile_off[tile];
        if (tile == rows * tiles_per_row - 1) {
            if (row_off) row_off[rows] = tile_off[tile + 1];
            if (total_out) *total_out = tile_off[tile + 1];
        }
    }
    int64_t running = tile_off[tile];
    for (int r0 = 0; r0 < kTile; r0 += kBlock) {
        int64_t c = c0 + r0 + threadIdx.x;
        uint32_t val = (c < cols) ? src.eval(row, c) : 0u;
        uint64_t bits = __ballot(val != 0u);
        int rank = __popcll(bits & ((1ull << lane) - 1ull));
        if (lane == 0) wcnt[wid] = __popcll(bits);
        __syncthreads();
        int64_t before = running;
        int total = 0;
        for (int w = 0; w < kBlock / kWave; ++w) {
            if (w < wid) before += wcnt[w];
            total += wcnt[w];
        }
        if (val != 0u) sink.emit(before + rank, row, c, val);
        running += total;
        __syncthreads();
    }
}

size_t compact_scratch_bytes(int64_t rows, int64_t cols) {
    int64_t tpr = (cols + kTile - 1) / kTile;
    int64_t tiles = rows * tpr;
    return static_cast<size_t>(tiles) * sizeof(int32_t) + 256 +
           static_cast<size_t>(tiles + 1) * sizeof(int64_t) + 256;
}

template <class Src, class Sink>
static int run_compact(Src src, Sink sink, int64_t rows, int64_t cols, int64_t *row_off,
                       int64_t *total_out, void *scratch, hipStream_t s) {
    if (rows <= 0 || cols <= 0) return GLIF_OK;
    int64_t tpr = (cols + kTile - 1) / kTile;
    int64_t tiles = rows * tpr;
    if (tiles > INT32_MAX) return fail(GLIF_EINVAL, "compaction too large");
    Carver cv(scratch, SIZE_MAX);
    int32_t *cnt = cv.take<int32_t>(tiles);
    int64_t *off = cv.take<int64_t>(tiles + 1);
    hipLaunchKernelGGL((k_compact_count<Src>), dim3(tiles), dim3(kBlock), 0, s, src, cols,
                       static_cast<int>(tpr), cnt);
    GLIF_HIP(hipGetLastError());
    hipLaunchKernelGGL(k_scan_counts, dim3(1), dim3(1024), 0, s, cnt, tiles, off);
    GLIF_HIP(hipGetLastError());
    hipLaunchKernelGGL((k_compact_write<Src, Sink>), dim3(tiles), dim3(kBlock), 0, s, src, sink,
                       rows, cols, static_cast<int>(tpr), off, row_off, total_out);
    GLIF_HIP(hipGetLastError());
    return GLIF_OK;
}

// ---- predicates and sinks ----------------------------------------------------
struct SrcF32Gt0 {
    const float *z;
    int64_t cols;
    __device__ uint32_t eval(int64_t r, int64_t c) const { return z[r * cols + c] > 0.0f ? 1u : 0u; }
};

struct SinkPairs {
    int64_t *pairs;
    __device__ void emit(int64_t pos, int64_t r, int64_t c, uint32_t) const {
        pairs[2 * pos] = r;
        pairs[2 * pos + 1] = c;
    }
};

// Inputs [T][B][C] uint8: row t, column c is active when any batch entry is > 0;
// the value is the batch mask (bit b set when x[t][b][c] > 0).
struct SrcBatchMask {
    const uint8_t *x;
    int32_t B;
    int64_t C;
    __device__ uint32_t eval(int64_t t, int64_t c) const {
        uint32_t m = 0;
        const uint8_t *p = x + t * B * C + c;
        for (int b = 0; b < B; ++b) m |= (p[b * C] != 0 ? 1u : 0u) << b;
        return m;
    }
};

struct SinkPreMask {
    int32_t *pre;
    uint32_t *mask;
    __device__ void emit(int64_t pos, int64_t, int64_t c, uint32_t v) const {
        pre[pos] = static_cast<int32_t>(c);
        mask[pos] = v;
    }
};

// Dense [B][C] float input, one row: column c is active when any z[b][c] > 0.
// Backward windows over inputs [T][B][C]: window j covers the reverse steps
// s0 - w (w < nw) with t0 = T-1-j*W, s0 = t0-2, nw = min(W, t0-1); column c is
// active when any x[s0-w][b][c] > 0 and its mask has bit w*B + b set for those.
struct SrcWindowMask {
    const uint8_t *x;
    int32_t B, T, W;
    int64_t C;
    __device__ uint32_t eval(int64_t j, int64_t c) const {
        const int t0 = T - 1 - static_cast<int>(j) * W;
        const int s0 = t0 - 2;
        const int nw = min(W, t0 - 1);
        uint32_t m = 0;
        for (int w = 0; w < nw; ++w) {
            const uint8_t *p = x + static_cast<int64_t>(s0 - w) * B * C + c;
            for (int b = 0; b < B; ++b) m |= (p[b * C] != 0 ? 1u : 0u) << (w * B + b);
        }
        return m;
    }
};

int build_window_mask_lists(const uint8_t *x, int32_t T, int32_t B, int64_t C, int32_t W,
                            int32_t n_windows, int64_t *row_off, int32_t *pre, uint32_t *mask,
                            void *scratch, hipStream_t s) {
    return run_compact(SrcWindowMask{x, B, T, W, C}, SinkPreMask{pre, mask}, n_windows, C, row_off,
                       nullptr, scratch, s);
}

int build_batch_mask_lists(const uint8_t *x, int32_t T, int32_t B, int64_t C, int64_t *row_off,
                           int32_t *pre, uint32_t *mask, void *scratch, hipStream_t s) {
    return run_compact(SrcBatchMask{x, B, C}, SinkPreMask{pre, mask}, T, C, row_off, nullptr,
                       scratch, s);
}

}  // namespace glif

using namespace glif;

extern "C" {

size_t glif_where_workspace(int64_t rows, int64_t cols) { return compact_scratch_bytes(rows, cols); }

int glif_where_gt0(const float *z, int64_t rows, int64_t cols, int64_t *pairs, int64_t *count,
                   void *ws, size_t ws_bytes, void *stream) {
    if (rows < 0 || cols < 0) return fail(GLIF_EINVAL, "negative shape");
    if (!count) return fail(GLIF_EINVAL, "count is NULL");
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (rows == 0 || cols == 0) return launch_fill_u32(count, 0u, 2, s);
    if (!z || !pairs) return fail(GLIF_EINVAL, "NULL argument");
    if (ws_bytes < compact_scratch_bytes(rows, cols)) return fail(GLIF_ENOMEM, "workspace too small");
    return run_compact(SrcF32Gt0{z, cols}, SinkPairs{pairs}, rows, cols, nullptr, count, ws, s);
}

}  // extern "C"
