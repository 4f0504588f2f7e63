// Internal declarations of libglif (not part of the C ABI).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <mutex>
#include <string>

#include "../../include/glif.h"

namespace glif {

constexpr int kWave = 64;
constexpr int kBlock = 256;
constexpr int kMaxBasis = 8;
constexpr int kMaxBatch = 32;
constexpr uint32_t kLow24 = 0x00FFFFFFu;
constexpr int kChunkEntries = 512;
// work units of the op-level weight-gradient pass: at most 64 consecutive columns and this many
// synapses, or one chunk of this many synapses of a longer column
constexpr int kDwUnitEntries = 1024;
constexpr int kChunkRows = 63;
// grouped row-sliced backward order: kGsCols columns per lane group,
// kGsSlices equal ranges of G rows, segments padded to kGsPad entries
constexpr int kGsCols = 4;
constexpr int kGsSlices = 4;
constexpr int kGsPad = 8;
constexpr int kGsRowBits = 29;
constexpr uint32_t kGsRowMask = (1u << kGsRowBits) - 1u;
static_assert(kGsCols < 7, "column-in-group 7 marks padding (3 bits above the row)");

// ---- error plumbing -------------------------------------------------------
void set_error(const std::string &msg);
int fail(int code, const std::string &msg);
int hip_fail(hipError_t e, const char *what);

#define GLIF_HIP(call)                                   \
    do {                                                 \
        hipError_t e_ = (call);                          \
        if (e_ != hipSuccess) return hip_fail(e_, #call); \
    } while (0)

// ---- compact G rows of a table ----------------------------------------------
// The G row of a synapse is post * rows + rank, rank = the position of its syn_id among a
// per-post set of types (ascending).
struct CompactRows {
    int32_t rows = 0;              // rows per post, 0: not built
    uint8_t *rank_host = nullptr;  // [n_syn] host copy of the ranks, column-grouped order
    uint32_t *ps = nullptr;        // [n_syn] column-grouped: post | rank << 24
    uint2 *ph_pw = nullptr;        // [n_syn] type-phased order: {compact row, weight bits}
    int64_t n_gs = 0;              // grouped row-sliced order over the compact rows (the table's
    int32_t *gs_seg = nullptr;     // groups of kGsCols columns); 0: not built
    uint2 *gs_pw = nullptr;
    int32_t *gs_src = nullptr;
    uint8_t *gtype = nullptr;      // device [n_post][rows]: syn_id of each rank, 0xFF past the
                                   // post's types (own rows only; a cell keeps its own)
};

// ---- device-resident synapse table (one population) -----------------------
// Column-grouped ("CSC", the reference's pre_ind_table) and post-grouped ("CSR")
// copies of the same synapses.  Index k runs over the column-grouped order,
// j over the post-grouped order.
// Two-pass plan of a large permutation gather dst[k] = src[P[k]] whose indices are far
// apart (a CSR <-> CSC reordering).  Destinations form superblocks of 64K, sources chunks of
// 64K.  Pass 1 (k_perm_runs) copies each chunk's sources into the superblocks they go to: one
// workgroup per (chunk, superblock) run, the run written contiguously, the chunk's 256 KB read
// from cache.  Pass 2 (k_perm_local) places every destination from its superblock's 256 KB of
// staging.  Both passes stream their offsets and stay inside 256 KB windows, where one gather
// over the whole array misses the cache on nearly every element.
constexpr int kPermShift = 16;  // superblock / chunk size 1 << 16
constexpr int64_t kPermMinSyn = int64_t(1) << 20;  // tables from this size get the plans
struct PermPlan {
    int32_t n_runs = 0;        // workgroups of pass 1 (XCD-aware order, padded with empty runs)
    int4 *runs = nullptr;      // {first staging position, length, first source of the chunk, 0}
    uint16_t *off1 = nullptr;  // [n] per staging position: source - first source of its chunk
    uint16_t *off2 = nullptr;  // [n] per destination: staging position - superblock start
    float *mid = nullptr;      // [n] staging of the plan's own, or nullptr (callers pass one)
};

struct Table {
    int64_t n_syn = 0;
    int32_t n_post = 0;
    int64_t n_cols = 0;
    int32_t n_slots = 1;   // delay slots D (cols = pre + n_post * (d - 1))
    int32_t n_pre = 0;     // n_cols / n_slots
    int32_t n_types = 0;
    int32_t n_basis = 0;
    int32_t max_col_len = 0;
    float *basis = nullptr;       // [n_types][n_basis]
    // column-grouped
    int32_t *col_ptr = nullptr;   // [n_cols + 1]  == row_splits
    int32_t *order = nullptr;     // [n_syn]       synapse id at position k
    uint32_t *ps = nullptr;       // [n_syn]       post | syn_id << 24
    float *w_col = nullptr;       // [n_syn]       weight at position k
    // post-grouped, each row in ascending (col, synapse id)
    int32_t *row_ptr = nullptr;   // [n_post + 1]
    int32_t *perm = nullptr;      // [n_syn]       synapse id at position j
    uint32_t *pd = nullptr;       // [n_syn]       pre | (delay - 1) << 24
    uint32_t *pidx = nullptr;     // [n_syn]       (n_slots - delay) * round64(n_pre) + pre, or null
    uint8_t *sid_row = nullptr;   // [n_syn]
    float *w_row = nullptr;       // [n_syn]
    // type-phased (backward): ordered by (syn_id, column, synapse id); the type-s
    // synapses of column c are k in [ph_ptr[s * n_cols + c], ph_ptr[s * n_cols + c + 1])
    // ELL copy of the post-grouped table for single-delay (input) tables whose rows
    // pad to at most twice the synapse count: entry j of post n at j * n_post + n,
    // {pre | syn_id << 24, weight bits}, padding {0, +0.0f}; rows keep the
    // post-grouped (column, synapse id) order.  ell_len = 0: not built.
    int32_t ell_len = 0;
    uint2 *ell_pw = nullptr;      // [ell_len * n_post]
    int32_t *ell_src = nullptr;   // [ell_len * n_post] synapse id, -1 for padding
    // row-aligned chunks of the post-grouped table for the deterministic pull: chunk k
    // is {first row, rows, first entry, end entry}, at most kChunkRows rows and at most
    // kChunkEntries entries unless it is a single longer row
    int32_t n_chunks = 0;
    int4 *chunk_desc = nullptr;   // [n_chunks]
    // work units of the op-level weight-gradient pass over the column-grouped table: unit u is
    // {first column, columns, first position, end position} (kDwUnitEntries)
    int32_t n_dwu = 0;
    int4 *dwu = nullptr;          // [n_dwu]
    // columns whose units hold one column each (a column of more than kDwUnitEntries synapses
    // spreads over several): {column, first unit, units, 0}, for the chunked dz pass
    int32_t n_dzc = 0;
    int4 *dzc = nullptr;          // [n_dzc]
    int32_t *ph_ptr = nullptr;    // [n_types * n_cols + 1]
    int32_t *ph_order = nullptr;  // [n_syn]       synapse id at position k
    uint2 *ph_pw = nullptr;       // [n_syn]       {post, weight bits}
    int32_t *order_inv = nullptr; // [n_syn]       position of synapse s in the column-grouped order
    int32_t *ph_inv = nullptr;    // [n_syn]       position of synapse s in the type-phased order
    int32_t *ph_src = nullptr;    // [n_syn]       column-grouped position of type-phased position k
    // grouped row-sliced order (backward dz walks over 8- and 16-float G rows): lane group g owns
    // columns kGsCols*g ..; its entries in G-row slice p (rows syn_id * n_post + post, slice p
    // = rows [n_rows * p / kGsSlices, n_rows * (p + 1) / kGsSlices)) are positions
    // [gs_seg[g * (kGsSlices + 1) + p], gs_seg[g * (kGsSlices + 1) + p + 1]), ordered by
    // (row, column, synapse id) and padded to a multiple of kGsPad with entries
    // {the segment's last row | 7 << kGsRowBits, +0.0f}.  n_gs = 0: not built.
    int64_t n_gs = 0;             // positions, padding included
    int64_t n_groups = 0;
    int32_t *gs_seg = nullptr;    // [n_groups * (kGsSlices + 1)]
    uint2 *gs_pw = nullptr;       // [n_gs]        {row | column-in-group << kGsRowBits, weight bits}
    int32_t *gs_src = nullptr;    // [n_gs]        column-grouped position of the synapse, -1 for padding
    float *basis_host = nullptr;  // host copy [n_types][n_basis]
    // Compact G rows: a G row per (post, type reaching the post) instead of per (type, post).
    // cg: set by a cell, over the types reaching each post from any of its three populations;
    // og: the table's own types per post, built at creation (the op-level backward uses it).
    // Each is built only when no post receives more than three quarters of the types.  The
    // type-major copies above stay as they are.
    CompactRows cg, og;
    // two-pass plans (tables of at least kPermMinSyn synapses): the column-grouped weight copy
    // (P = order) and weight gradients from the column-grouped order back to the reference
    // order (P = order_inv)
    PermPlan pcol, pinv;
};

// Give a table a cell's compact G rows (Table::cg; rank: [n_syn] in column-grouped order, each
// < g_rows).  A table that already has them keeps them if they are the same, else GLIF_EINVAL.
// Synchronous.
int table_set_g_rows(Table *t, const uint8_t *rank, int32_t g_rows);

// ---- cell ------------------------------------------------------------------
struct Cell {
    glif_cell_config cfg{};
    int32_t N = 0, Np = 0, W = 0;   // neurons, padded to 64, 64-bit words per row
    int32_t D = 0, nb = 0, n_types = 0;
    float *decay = nullptr, *cf = nullptr;   // [N]
    float *asc_decay = nullptr, *asc_amps = nullptr;  // [N*2]
    int32_t *tref = nullptr;                 // [N]
    float syn_decay[kMaxBasis]{}, psc_initial[kMaxBasis]{}, dtsd[kMaxBasis]{};
    Table *rec = nullptr, *lgn = nullptr, *bkg = nullptr;
    int32_t vloss_mode = 0;    // fused voltage regularization: 0 off, 1 range, 2 threshold
    float vloss_cost = 0.0f;
    const uint8_t *vloss_mask = nullptr;  // device [N] core mask of the voltage loss (caller-owned), or null
    int32_t vloss_n = 0;                  // neurons it selects
    // spike-trimming window of the rate losses (loss_functions.py:604-611): the forward
    // counts spikes of ticks [trim_pre, T - trim_post) and the backward broadcasts
    // gz_neuron over the same ticks
    int32_t trim_pre = 0, trim_post = 0;
    // G rows per post: n_types (rows syn_id * N + post), or fewer when the tables carry
    // compact rows (rows post * g_rows + rank, g_type[post * g_rows + rank] = syn_id, 0xFF
    // past the post's types)
    int32_t g_rows = 0;
    bool g_compact = false;
    int32_t g_compact_rows = 0;  // compact rows per post the tables carry, 0: none
    uint8_t *g_type = nullptr;  // device [N * g_compact_rows]
    // event push into per-type slots (with compact rows and a basis with more than one
    // nonzero receptor in some row): one atomic per synapse event into slot [rank][b][post],
    // the step folding the slots through the basis, instead of one atomic per receptor
    bool basis_dense = false;
    bool push_typed = false;
    // The LGN pass of segment s + 1 runs on a stream of the cell's own while the caller's
    // stream runs segment s's ticks (created on first use, on that call's device; events
    // order the two).  The mutex keeps concurrent forwards on one cell from interleaving their
    // event records and waits.
    int side_dev = -1;
    hipStream_t side = nullptr;
    hipEvent_t ev_main = nullptr, ev_seg[2] = {nullptr, nullptr};
    std::mutex side_mu;
};

// Small per-cell constants passed by value to kernels.
struct CellConst {
    int32_t N, Np, W, D, nb, n_types, B, Bp;
    float lr, vgd, om, rd_scale, gauss_std, damp, dt;
    int32_t pseudo_gauss, hard_reset;
    float sd[kMaxBasis], p0[kMaxBasis], dtsd[kMaxBasis];
};

// ---- workspace carving ------------------------------------------------------
struct Carver {
    char *base;
    size_t off = 0;
    size_t cap;
    Carver(void *b, size_t c) : base(static_cast<char *>(b)), cap(c) {}
    template <typename T>
    T *take(size_t n) {
        off = (off + 255) & ~size_t(255);
        T *p = reinterpret_cast<T *>(base ? base + off : nullptr);
        off += n * sizeof(T);
        return p;
    }
    bool ok() const { return off <= cap; }
    // the next region's offset (aligned as take() aligns it)
    size_t mark() {
        off = (off + 255) & ~size_t(255);
        return off;
    }
};

// ---- launch helpers (defined in the .hip files) ----------------------------
int launch_fill_u32(void *p, uint32_t value, size_t n, hipStream_t s);
int launch_gather_f32(float *dst, const float *src, const int32_t *idx, int64_t n, hipStream_t s);
// dst[k] = src[idx[k]] through the plan when it is built (staging through mid, n floats),
// else one gather
int launch_perm_gather(float *dst, const float *src, const int32_t *idx, const PermPlan &plan, int64_t n,
                       float *mid, hipStream_t s);

inline int ceil_div(int64_t a, int64_t b) { return static_cast<int>((a + b - 1) / b); }

// Batch padded to the float4 groups of G (4, 8, 16 or 32).
int batch_pad(int B);
// The op's custom gradient (glif_syn_bwd) on a given G buffer of syn_g_floats(t, B) floats;
// g_ready: G already holds this dy's rows in t's layout (built for a table with
// same_g_layout), so only dz / dW are computed.  partial: n_dwu * batch_pad(B) floats for the
// unit dz pass of tables with few or long columns (nullptr: the walks only).
size_t syn_g_floats(const Table *t, int32_t B);
bool same_g_layout(const Table *a, const Table *b);
int syn_bwd_run(const Table *t, const float *z, const float *dy, int32_t B, int32_t counts, float *dz, float *dw,
                float *G, bool g_ready, float *partial, hipStream_t s);
// Lanes per column for the column-grouped kernels (16, 32 or 64).
int sub_wave_for(const Table *t);
// Blocks for `items` sub-waves of L lanes (capped; kernels grid-stride).
int grid_subwaves(int64_t items, int L);

}  // namespace glif
