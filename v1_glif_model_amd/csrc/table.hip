// Synapse tables: the one-time host build of the column- and post-grouped
// orders (pre_ind_table and the preprocessed copies), their upload, the weight-shadow refresh, and shared helpers.
#include <algorithm>
#include <cstring>
#include <mutex>
#include <vector>

#include "glif_internal.h"

namespace glif {

// ---------------------------------------------------------------- errors ----
static thread_local std::string g_last_error;

void set_error(const std::string &msg) { g_last_error = msg; }

int fail(int code, const std::string &msg) {
    g_last_error = msg;
    return code;
}

int hip_fail(hipError_t e, const char *what) {
    g_last_error = std::string(what) + ": " + hipGetErrorString(e);
    return GLIF_EHIP;
}

// --------------------------------------------------------------- kernels ----
__global__ void k_fill_u32(uint32_t *__restrict__ p, uint32_t v, size_t n) {
    size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (; i < n; i += stride) p[i] = v;
}

__global__ void k_gather_f32(float *__restrict__ dst, const float *__restrict__ src,
                             const int32_t *__restrict__ idx, int64_t n) {
    int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (; i < n; i += stride) dst[i] = src[idx[i]];
}

// Pass 1 of a permutation plan: workgroup = one (chunk, superblock) run, staged contiguously.
__global__ void __launch_bounds__(kBlock)
    k_perm_runs(const float *__restrict__ src, float *__restrict__ mid, const int4 *__restrict__ runs,
                const uint16_t *__restrict__ off1) {
    const int4 r = runs[blockIdx.x];
    for (int i = threadIdx.x; i < r.y; i += blockDim.x) {
        const int32_t m = r.x + i;
        mid[m] = src[static_cast<int64_t>(r.z) + off1[m]];
    }
}

// Pass 2: dst[k] from the staging of k's superblock.  Workgroups go to the 8 XCDs round robin
// (blockIdx % 8); XCD x takes the x-th eighth of the destinations, so each superblock's
// staging is read through one L2.
__global__ void __launch_bounds__(kBlock)
    k_perm_local(const float *__restrict__ mid, float *__restrict__ dst, const uint16_t *__restrict__ off2,
                 int64_t n) {
    const int64_t per = gridDim.x / 8;
    const int64_t lb = static_cast<int64_t>(blockIdx.x % 8) * per + blockIdx.x / 8;
    const int64_t k = lb * blockDim.x + threadIdx.x;
    if (k < n) dst[k] = mid[((k >> kPermShift) << kPermShift) + off2[k]];
}

__global__ void k_gather_pair_w(uint2 *__restrict__ dst, const float *__restrict__ src,
                                const int32_t *__restrict__ idx, int64_t n) {
    int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (; i < n; i += stride) dst[i].y = __float_as_uint(src[idx[i]]);
}

// dst[i].y = weight of synapse idx[i], +0.0f where idx[i] < 0 (padding)
__global__ void k_gather_ell_w(uint2 *__restrict__ dst, const float *__restrict__ src,
                               const int32_t *__restrict__ idx, int64_t n) {
    int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (; i < n; i += stride) dst[i].y = idx[i] >= 0 ? __float_as_uint(src[idx[i]]) : 0u;
}

static int grid_for(int64_t n) {
    int64_t g = (n + kBlock - 1) / kBlock;
    return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(g, 8192)));
}

int launch_fill_u32(void *p, uint32_t value, size_t n, hipStream_t s) {
    if (n == 0) return GLIF_OK;
    hipLaunchKernelGGL(k_fill_u32, dim3(grid_for(static_cast<int64_t>(n))), dim3(kBlock), 0, s,
                       static_cast<uint32_t *>(p), value, n);
    GLIF_HIP(hipGetLastError());
    return GLIF_OK;
}

int launch_gather_f32(float *dst, const float *src, const int32_t *idx, int64_t n, hipStream_t s) {
    if (n == 0) return GLIF_OK;
    hipLaunchKernelGGL(k_gather_f32, dim3(grid_for(n)), dim3(kBlock), 0, s, dst, src, idx, n);
    GLIF_HIP(hipGetLastError());
    return GLIF_OK;
}

int launch_perm_gather(float *dst, const float *src, const int32_t *idx, const PermPlan &plan, int64_t n,
                       float *mid, hipStream_t s) {
    if (!plan.runs) return launch_gather_f32(dst, src, idx, n, s);
    if (!mid) return fail(GLIF_EINVAL, "permutation plan without a staging buffer");
    hipLaunchKernelGGL(k_perm_runs, dim3(plan.n_runs), dim3(kBlock), 0, s, src, mid, plan.runs, plan.off1);
    GLIF_HIP(hipGetLastError());
    const int64_t blocks = 8 * ((n + 8 * kBlock - 1) / (8 * kBlock));
    hipLaunchKernelGGL(k_perm_local, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, s, mid, dst, plan.off2,
                       n);
    GLIF_HIP(hipGetLastError());
    return GLIF_OK;
}

// ------------------------------------------------------------ host builds ----
// Stable counting sort of synapse ids by key (models.py:317-341): order holds, for
// each key in ascending order, the ids with that key in ascending id order.
static void counting_sort(const int64_t *key, const int32_t *ids, int64_t n, int64_t n_keys,
                          int32_t *splits, int32_t *order) {
    std::fill(splits, splits + n_keys + 1, 0);
    for (int64_t i = 0; i < n; ++i) splits[key[ids ? ids[i] : i] + 1] += 1;
    for (int64_t c = 0; c < n_keys; ++c) splits[c + 1] += splits[c];
    std::vector<int32_t> wp(splits, splits + n_keys);
    for (int64_t i = 0; i < n; ++i) {
        int32_t id = ids ? ids[i] : static_cast<int32_t>(i);
        order[wp[key[id]]++] = id;
    }
}

template <typename T>
static int upload(T **dst, const T *src, size_t n) {
    GLIF_HIP(hipMalloc(reinterpret_cast<void **>(dst), std::max<size_t>(n, 1) * sizeof(T)));
    if (n) GLIF_HIP(hipMemcpy(*dst, src, n * sizeof(T), hipMemcpyHostToDevice));
    return GLIF_OK;
}

// Grouped row-sliced order (backward dz walks) over items 0..n-1 (synapses, or positions of
// the column-grouped order) with G row row[i] < n_rows and column col[i]: a stable counting
// sort by (G row, column in group), then by (group, row slice); each (group, slice) segment is
// padded to a multiple of kGsPad with copies of its last row marked as column 7 (weight
// +0.0f).  src[i] goes to gs_src.  False (nothing built) when the rows or positions do not fit.
static bool build_gs(int64_t n, int64_t n_cols, int64_t n_rows, const int64_t *row, const int64_t *col,
                     const int32_t *src, int64_t &n_groups, int64_t &n_gs, std::vector<int32_t> &gs_seg,
                     std::vector<uint2> &gs_pw, std::vector<int32_t> &gs_src) {
    n_groups = n_gs = 0;
    if (n <= 0 || n_rows > static_cast<int64_t>(kGsRowMask) + 1) return false;
    const int64_t groups = (n_cols + kGsCols - 1) / kGsCols;
    std::vector<int64_t> key(n);
    for (int64_t i = 0; i < n; ++i) key[i] = row[i] * kGsCols + col[i] % kGsCols;
    std::vector<int32_t> ptr1(n_rows * kGsCols + 1), ord1(n);
    counting_sort(key.data(), nullptr, n, n_rows * kGsCols, ptr1.data(), ord1.data());
    for (int64_t i = 0; i < n; ++i) key[i] = (col[i] / kGsCols) * kGsSlices + row[i] * kGsSlices / n_rows;
    const int64_t n_seg = groups * kGsSlices;
    std::vector<int32_t> ptr2(n_seg + 1), ord2(n);
    counting_sort(key.data(), ord1.data(), n, n_seg, ptr2.data(), ord2.data());
    int64_t total = 0;
    for (int64_t b = 0; b < n_seg; ++b) total += (ptr2[b + 1] - ptr2[b] + kGsPad - 1) / kGsPad * kGsPad;
    if (total >= INT32_MAX) return false;
    gs_seg.resize(groups * (kGsSlices + 1));
    gs_pw.resize(total);
    gs_src.resize(total);
    int64_t pos = 0;
    for (int64_t g = 0; g < groups; ++g) {
        for (int p = 0; p < kGsSlices; ++p) {
            const int64_t b = g * kGsSlices + p;
            gs_seg[g * (kGsSlices + 1) + p] = static_cast<int32_t>(pos);
            uint32_t last = 0;
            for (int32_t r = ptr2[b]; r < ptr2[b + 1]; ++r, ++pos) {
                const int32_t i = ord2[r];
                last = static_cast<uint32_t>(row[i]);
                gs_pw[pos] = make_uint2(last | static_cast<uint32_t>(col[i] % kGsCols) << kGsRowBits, 0u);
                gs_src[pos] = src[i];
            }
            for (; pos % kGsPad; ++pos) {
                gs_pw[pos] = make_uint2(last | 7u << kGsRowBits, 0u);
                gs_src[pos] = -1;
            }
        }
        gs_seg[g * (kGsSlices + 1) + kGsSlices] = static_cast<int32_t>(pos);
    }
    n_groups = groups;
    n_gs = total;
    return true;
}

static void free_plan(PermPlan &pp) {
    void *ptrs[] = {pp.runs, pp.off1, pp.off2, pp.mid};
    for (void *p : ptrs)
        if (p) (void)hipFree(p);
    pp = PermPlan{};
}

// The two-pass plan of dst[k] = src[P[k]], k < n (P a permutation of 0..n-1).  Staging
// position of source j: in the superblock of its destination, after the sources j' < j that go
// there, so each (chunk, superblock) pair's sources are one contiguous run.  With own_mid the
// plan allocates its staging (n floats); otherwise each caller passes one.
static int build_perm_plan(PermPlan *pp, const int32_t *P, int64_t n, bool own_mid) {
    constexpr int64_t kSB = int64_t(1) << kPermShift;
    const int64_t nsb = (n + kSB - 1) / kSB;
    std::vector<int32_t> Pinv(n), mpos(n), fill(nsb, 0), snap(nsb);
    for (int64_t k = 0; k < n; ++k) Pinv[P[k]] = static_cast<int32_t>(k);
    std::vector<uint16_t> off1(n), off2(n);
    std::vector<int4> by_xcd[8];
    for (int64_t c = 0; c * kSB < n; ++c) {
        std::copy(fill.begin(), fill.end(), snap.begin());
        const int64_t j1 = std::min(n, (c + 1) * kSB);
        for (int64_t j = c * kSB; j < j1; ++j) {
            const int64_t sb = Pinv[j] >> kPermShift;
            const int64_t m = sb * kSB + fill[sb]++;
            mpos[j] = static_cast<int32_t>(m);
            off1[m] = static_cast<uint16_t>(j - c * kSB);
        }
        for (int64_t sb = 0; sb < nsb; ++sb)
            if (fill[sb] > snap[sb])
                by_xcd[c % 8].push_back(make_int4(static_cast<int32_t>(sb * kSB + snap[sb]), fill[sb] - snap[sb],
                                                  static_cast<int32_t>(c * kSB), 0));
    }
    for (int64_t k = 0; k < n; ++k) off2[k] = static_cast<uint16_t>(mpos[P[k]] - ((k >> kPermShift) << kPermShift));
    // block b runs on XCD b % 8: XCD x takes the runs of chunks x, x + 8, .., so a chunk's 256 KB
    // of sources is read through one L2
    size_t slots = 0;
    for (auto &v : by_xcd) slots = std::max(slots, v.size());
    std::vector<int4> runs(8 * slots, make_int4(0, 0, 0, 0));
    for (int x = 0; x < 8; ++x)
        for (size_t i = 0; i < by_xcd[x].size(); ++i) runs[i * 8 + x] = by_xcd[x][i];
    int rc;
    if ((rc = upload(&pp->runs, runs.data(), runs.size())) || (rc = upload(&pp->off1, off1.data(), off1.size())) ||
        (rc = upload(&pp->off2, off2.data(), off2.size()))) {
        free_plan(*pp);
        return rc;
    }
    if (own_mid) {
        hipError_t e = hipMalloc(reinterpret_cast<void **>(&pp->mid), n * sizeof(float));
        if (e != hipSuccess) {
            free_plan(*pp);
            return hip_fail(e, "hipMalloc(permutation staging)");
        }
    }
    pp->n_runs = static_cast<int32_t>(runs.size());
    return GLIF_OK;
}

static void free_table(Table *t) {
    if (!t) return;
    free_plan(t->pcol);
    free_plan(t->pinv);
    void *ptrs[] = {t->basis, t->col_ptr, t->order, t->ps, t->w_col, t->row_ptr, t->perm,
                    t->pd, t->sid_row, t->w_row, t->ph_ptr, t->ph_order, t->ph_pw, t->ell_pw, t->ell_src,
                    t->chunk_desc, t->dwu, t->dzc, t->pidx, t->order_inv, t->ph_inv, t->ph_src, t->gs_seg, t->gs_pw, t->gs_src,
                    t->cg.ps, t->cg.ph_pw, t->cg.gs_seg, t->cg.gs_pw, t->cg.gs_src, t->cg.gtype,
                    t->og.ps, t->og.ph_pw, t->og.gs_seg, t->og.gs_pw, t->og.gs_src, t->og.gtype};
    for (void *p : ptrs)
        if (p) (void)hipFree(p);
    delete[] t->basis_host;
    delete[] t->cg.rank_host;
    delete[] t->og.rank_host;
    delete t;
}

template <typename T>
static int download(std::vector<T> &dst, const T *src, size_t n) {
    dst.resize(n);
    if (n) GLIF_HIP(hipMemcpy(dst.data(), src, n * sizeof(T), hipMemcpyDeviceToHost));
    return GLIF_OK;
}

// Compact rows from host arrays over the column-grouped positions k: col_ptr [n_cols + 1],
// ps[k] = post | syn_id << 24, ph_src [n_syn] (column-grouped position of each type-phased
// position) and rank[k] < rows.  Uploads ps / ph_pw / the grouped order into out (weights
// +0: the caller gathers them from w_col) and keeps a host copy of the ranks.
static int build_compact(const Table *t, const int32_t *col_ptr, const uint32_t *ps, const int32_t *ph_src,
                         const uint8_t *rank, int32_t rows, CompactRows &out) {
    const int64_t n = t->n_syn;
    std::vector<int64_t> row(n), col(n);
    std::vector<int32_t> src(n);
    std::vector<uint32_t> cps(n);
    for (int64_t c = 0; c < t->n_cols; ++c)
        for (int32_t k = col_ptr[c]; k < col_ptr[c + 1]; ++k) col[k] = c;
    for (int64_t k = 0; k < n; ++k) {
        const uint32_t post = ps[k] & kLow24;
        row[k] = static_cast<int64_t>(post) * rows + rank[k];
        cps[k] = post | static_cast<uint32_t>(rank[k]) << 24;
        src[k] = static_cast<int32_t>(k);
    }
    std::vector<uint2> cph_pw(n);
    for (int64_t k = 0; k < n; ++k) cph_pw[k] = make_uint2(static_cast<uint32_t>(row[ph_src[k]]), 0u);
    std::vector<int32_t> gs_seg, gs_src;
    std::vector<uint2> gs_pw;
    int64_t n_groups = 0, n_gs = 0;
    build_gs(n, t->n_cols, static_cast<int64_t>(t->n_post) * rows, row.data(), col.data(), src.data(), n_groups,
             n_gs, gs_seg, gs_pw, gs_src);
    int rc;
    if ((rc = upload(&out.ps, cps.data(), cps.size())) || (rc = upload(&out.ph_pw, cph_pw.data(), cph_pw.size())) ||
        (n_gs && (rc = upload(&out.gs_seg, gs_seg.data(), gs_seg.size()))) ||
        (n_gs && (rc = upload(&out.gs_pw, gs_pw.data(), gs_pw.size()))) ||
        (n_gs && (rc = upload(&out.gs_src, gs_src.data(), gs_src.size()))))
        return rc;
    out.n_gs = n_gs;
    out.rank_host = new uint8_t[std::max<int64_t>(n, 1)];
    if (n) std::memcpy(out.rank_host, rank, n);
    out.rows = rows;
    return GLIF_OK;
}

// the weights of a table's compact copies, gathered from w_col
static int gather_compact_weights(const Table *t, const CompactRows &c, hipStream_t s) {
    if (c.rows && t->n_syn) {
        hipLaunchKernelGGL(k_gather_pair_w, dim3(grid_for(t->n_syn)), dim3(kBlock), 0, s, c.ph_pw, t->w_col,
                           t->ph_src, t->n_syn);
        GLIF_HIP(hipGetLastError());
    }
    if (c.n_gs) {
        hipLaunchKernelGGL(k_gather_ell_w, dim3(grid_for(c.n_gs)), dim3(kBlock), 0, s, c.gs_pw, t->w_col, c.gs_src,
                           c.n_gs);
        GLIF_HIP(hipGetLastError());
    }
    return GLIF_OK;
}

int table_set_g_rows(Table *t, const uint8_t *rank, int32_t g_rows) {
    if (g_rows <= 0 || g_rows > 255) return fail(GLIF_EINVAL, "compact G rows per post must be in [1, 255]");
    // cells created from several threads may share a table
    static std::mutex mu;
    std::lock_guard<std::mutex> lock(mu);
    const int64_t n = t->n_syn;
    if (t->cg.rows) {
        if (t->cg.rows == g_rows && (n == 0 || std::memcmp(t->cg.rank_host, rank, n) == 0)) return GLIF_OK;
        return fail(GLIF_EINVAL, "table already carries a different compact G row map (one per table)");
    }
    for (int64_t k = 0; k < n; ++k)
        if (rank[k] >= g_rows) return fail(GLIF_ERANGE, "G row rank >= rows per post");
    std::vector<int32_t> col_ptr, ph_src;
    std::vector<uint32_t> ps;
    int rc;
    GLIF_HIP(hipDeviceSynchronize());  // weights set on any stream have landed in w_col
    if ((rc = download(col_ptr, t->col_ptr, static_cast<size_t>(t->n_cols) + 1)) ||
        (rc = download(ps, t->ps, n)) || (rc = download(ph_src, t->ph_src, n)))
        return rc;
    if ((rc = build_compact(t, col_ptr.data(), ps.data(), ph_src.data(), rank, g_rows, t->cg))) return rc;
    // the weights the table already holds (later ones arrive through glif_table_set_weights)
    if ((rc = gather_compact_weights(t, t->cg, nullptr))) return rc;
    GLIF_HIP(hipDeviceSynchronize());
    return GLIF_OK;
}

// The table's own compact rows (Table::og) when no post receives more than three quarters of
// the types: ranks over each post's own types.
static int build_own_rows(Table *t, const int32_t *col_ptr, const uint32_t *ps, const int32_t *ph_src) {
    const int nt = t->n_types, words = (nt + 63) / 64;
    if (nt > 255 || t->n_syn == 0) return GLIF_OK;  // 0xFF marks an unused rank
    std::vector<uint64_t> seen(static_cast<size_t>(t->n_post) * words, 0ull);
    for (int64_t k = 0; k < t->n_syn; ++k) {
        const uint32_t sid = ps[k] >> 24;
        seen[static_cast<size_t>(ps[k] & kLow24) * words + sid / 64] |= 1ull << (sid % 64);
    }
    int gk = 1;
    for (int32_t n = 0; n < t->n_post; ++n) {
        int cnt = 0;
        for (int q = 0; q < words; ++q) cnt += __builtin_popcountll(seen[static_cast<size_t>(n) * words + q]);
        gk = std::max(gk, cnt);
    }
    if (gk * 4 > nt * 3) return GLIF_OK;
    std::vector<uint8_t> rank(t->n_syn), gtype(static_cast<size_t>(t->n_post) * gk, 0xFF);
    for (int64_t k = 0; k < t->n_syn; ++k) {
        const uint32_t sid = ps[k] >> 24;
        const uint64_t *sn = &seen[static_cast<size_t>(ps[k] & kLow24) * words];
        int r = 0;
        for (uint32_t q = 0; q < sid / 64; ++q) r += __builtin_popcountll(sn[q]);
        r += __builtin_popcountll(sid % 64 ? sn[sid / 64] & ((1ull << (sid % 64)) - 1ull) : 0ull);
        rank[k] = static_cast<uint8_t>(r);
    }
    for (int32_t n = 0; n < t->n_post; ++n) {
        int q = 0;
        for (int sid = 0; sid < nt; ++sid)
            if ((seen[static_cast<size_t>(n) * words + sid / 64] >> (sid % 64)) & 1ull)
                gtype[static_cast<size_t>(n) * gk + q++] = static_cast<uint8_t>(sid);
    }
    int rc;
    if ((rc = build_compact(t, col_ptr, ps, ph_src, rank.data(), gk, t->og))) return rc;
    return upload(&t->og.gtype, gtype.data(), gtype.size());
}

}  // namespace glif

using namespace glif;

extern "C" {

const char *glif_last_error(void) { return g_last_error.c_str(); }

int glif_version(void) { return 1; }

int glif_make_pre_ind_table(const int64_t *cols, int64_t n_syn, int64_t n_source, int32_t *order,
                            int32_t *row_splits, int64_t *bad_index) {
    if (n_source <= 0)
        return fail(GLIF_EINVAL, "`n_source_neurons` must be > 0, got " + std::to_string(n_source) + ".");
    if (n_syn < 0 || n_syn > INT32_MAX || n_source > INT32_MAX)
        return fail(GLIF_EINVAL, "table too large for int32 order/row_splits");
    for (int64_t i = 0; i < n_syn; ++i) {
        if (cols[i] < 0 || cols[i] >= n_source) {
            if (bad_index) *bad_index = i;
            return fail(GLIF_ERANGE, "Presynaptic index " + std::to_string(cols[i]) +
                                         " is out of bounds for `n_source_neurons=" +
                                         std::to_string(n_source) + "`.");
        }
    }
    counting_sort(cols, nullptr, n_syn, n_source, row_splits, order);
    return GLIF_OK;
}

int glif_table_create(const int64_t *post, const int64_t *col, const uint8_t *syn_id, int64_t n_syn,
                      int32_t n_post, int64_t n_cols, int32_t n_delay_slots, const float *basis,
                      int32_t n_types, int32_t n_basis, glif_table **out) {
    if (!out) return fail(GLIF_EINVAL, "out is NULL");
    *out = nullptr;
    if (n_syn < 0 || n_syn >= INT32_MAX) return fail(GLIF_EINVAL, "n_syn must be in [0, 2^31-1)");
    if (n_post <= 0 || n_post >= (1 << 24)) return fail(GLIF_EINVAL, "n_post must be in [1, 2^24)");
    if (n_delay_slots <= 0 || n_delay_slots > 256) return fail(GLIF_EINVAL, "n_delay_slots must be in [1, 256]");
    if (n_cols <= 0 || n_cols % n_delay_slots != 0 || n_cols / n_delay_slots >= (1 << 24) ||
        n_cols >= INT32_MAX)
        return fail(GLIF_EINVAL, "n_cols must be a positive multiple of n_delay_slots with n_cols/D < 2^24");
    if (n_delay_slots > 1 && n_cols != static_cast<int64_t>(n_delay_slots) * n_post)
        return fail(GLIF_EINVAL, "recurrent table needs n_cols == n_delay_slots * n_post");
    if (n_types <= 0 || n_types > 256) return fail(GLIF_EINVAL, "n_types must be in [1, 256]");
    if (n_basis <= 0 || n_basis > kMaxBasis) return fail(GLIF_EINVAL, "n_basis must be in [1, 8]");
    const int32_t n_pre = static_cast<int32_t>(n_cols / n_delay_slots);
    for (int64_t i = 0; i < n_syn; ++i) {
        if (post[i] < 0 || post[i] >= n_post)
            return fail(GLIF_ERANGE, "postsynaptic index " + std::to_string(post[i]) + " out of range");
        if (col[i] < 0 || col[i] >= n_cols)
            return fail(GLIF_ERANGE, "Presynaptic index " + std::to_string(col[i]) +
                                         " is out of bounds for `n_source_neurons=" +
                                         std::to_string(n_cols) + "`.");
        if (syn_id[i] >= n_types)
            return fail(GLIF_ERANGE, "syn_id " + std::to_string(syn_id[i]) + " >= n_types");
    }

    // column-grouped order (bit-exact with models.py:317-341)
    std::vector<int32_t> col_ptr(n_cols + 1), order(n_syn);
    counting_sort(col, nullptr, n_syn, n_cols, col_ptr.data(), order.data());
    // post-grouped order with each row in ascending (col, id): a stable sort of the
    // column-grouped order by post
    std::vector<int32_t> row_ptr(static_cast<size_t>(n_post) + 1), perm(n_syn);
    counting_sort(post, order.data(), n_syn, n_post, row_ptr.data(), perm.data());

    // type-phased order for the backward: (syn_id, column, synapse id), by a stable
    // counting sort of the column-grouped order by syn_id * n_cols + column
    const int64_t n_ph = static_cast<int64_t>(n_types) * n_cols;
    if (n_ph >= INT32_MAX) return fail(GLIF_EINVAL, "n_types * n_cols must be < 2^31");
    std::vector<int64_t> ph_key(n_syn);
    for (int64_t i = 0; i < n_syn; ++i) ph_key[i] = static_cast<int64_t>(syn_id[i]) * n_cols + col[i];
    std::vector<int32_t> ph_ptr(n_ph + 1), ph_order(n_syn);
    counting_sort(ph_key.data(), order.data(), n_syn, n_ph, ph_ptr.data(), ph_order.data());
    std::vector<uint2> ph_pw(n_syn);
    for (int64_t k = 0; k < n_syn; ++k) {
        ph_pw[k].x = static_cast<uint32_t>(post[ph_order[k]]);
        ph_pw[k].y = 0u;  // the weight, written by glif_table_set_weights
    }

    // inverse permutations: position of synapse s in the column-grouped and type-phased
    // orders (gradients go back to reference order with coalesced writes)
    std::vector<int32_t> order_inv(n_syn), ph_inv(n_syn), ph_src(n_syn);
    for (int64_t k = 0; k < n_syn; ++k) {
        order_inv[order[k]] = static_cast<int32_t>(k);
        ph_inv[ph_order[k]] = static_cast<int32_t>(k);
    }
    // the weight copies other than w_col are gathered from w_col, whose order is close to
    // theirs (the type-phased order sweeps it once per type; a group's grouped entries come
    // from its own columns), rather than from the reference order
    for (int64_t k = 0; k < n_syn; ++k) ph_src[k] = order_inv[ph_order[k]];
    // grouped row-sliced order (backward dz walks) over the type-major rows
    std::vector<int32_t> gs_seg, gs_src;
    std::vector<uint2> gs_pw;
    int64_t n_groups = 0, n_gs = 0;
    {
        std::vector<int64_t> row(n_syn);
        for (int64_t i = 0; i < n_syn; ++i) row[i] = static_cast<int64_t>(syn_id[i]) * n_post + post[i];
        build_gs(n_syn, n_cols, static_cast<int64_t>(n_types) * n_post, row.data(), col, order_inv.data(), n_groups,
                 n_gs, gs_seg, gs_pw, gs_src);
    }

    std::vector<uint32_t> ps(n_syn), pd(n_syn);
    // bit index of the entry's presynaptic spike in a stack of per-slot activity planes
    // of round64(n_pre) bits, slot d at plane n_slots - d (the newest step last)
    const int64_t pre_pad = (static_cast<int64_t>(n_pre) + 63) / 64 * 64;
    const bool with_pidx = static_cast<int64_t>(n_delay_slots) * pre_pad < (int64_t(1) << 31);
    std::vector<uint32_t> pidx(with_pidx ? n_syn : 0);
    std::vector<uint8_t> sid_row(n_syn);
    int32_t max_len = 0;
    for (int64_t c = 0; c < n_cols; ++c) max_len = std::max(max_len, col_ptr[c + 1] - col_ptr[c]);
    for (int64_t k = 0; k < n_syn; ++k) {
        int32_t s = order[k];
        ps[k] = static_cast<uint32_t>(post[s]) | (static_cast<uint32_t>(syn_id[s]) << 24);
    }
    for (int64_t j = 0; j < n_syn; ++j) {
        int32_t s = perm[j];
        int64_t c = col[s];
        uint32_t d1 = static_cast<uint32_t>(c / n_pre), pre = static_cast<uint32_t>(c % n_pre);
        pd[j] = pre | (d1 << 24);
        if (with_pidx) pidx[j] = static_cast<uint32_t>((n_delay_slots - 1 - d1) * pre_pad + pre);
        sid_row[j] = syn_id[s];
    }

    // ELL copy (input tables: one delay slot, little padding)
    int32_t ell_len = 0;
    for (int32_t n = 0; n < n_post; ++n) ell_len = std::max(ell_len, row_ptr[n + 1] - row_ptr[n]);
    if (n_delay_slots != 1 || ell_len == 0 || static_cast<int64_t>(ell_len) * n_post > 2 * n_syn) ell_len = 0;
    std::vector<uint2> ell_pw(static_cast<size_t>(ell_len) * n_post);
    std::vector<int32_t> ell_src(static_cast<size_t>(ell_len) * n_post);
    for (int32_t j = 0; j < ell_len; ++j)
        for (int32_t n = 0; n < n_post; ++n) {
            const size_t i = static_cast<size_t>(j) * n_post + n;
            const int32_t r = row_ptr[n] + j;
            if (r < row_ptr[n + 1]) {
                const int32_t sidx = perm[r];
                ell_pw[i].x = static_cast<uint32_t>(col[sidx]) | (static_cast<uint32_t>(syn_id[sidx]) << 24);
                ell_src[i] = sidx;
            } else {
                ell_pw[i].x = 0u;
                ell_src[i] = -1;
            }
            ell_pw[i].y = 0u;
        }

    Table *t = new Table();
    t->n_syn = n_syn;
    t->n_post = n_post;
    t->n_cols = n_cols;
    t->n_slots = n_delay_slots;
    t->n_pre = n_pre;
    t->n_types = n_types;
    t->n_basis = n_basis;
    t->max_col_len = max_len;
    t->ell_len = ell_len;
    t->n_gs = n_gs;
    t->n_groups = n_groups;
    // row-aligned chunks, greedy in row order
    std::vector<int4> chunk_desc;
    for (int32_t n = 0; n < n_post;) {
        int32_t m = n + 1;
        while (m < n_post && m - n < kChunkRows && row_ptr[m + 1] - row_ptr[n] <= kChunkEntries) ++m;
        chunk_desc.push_back(make_int4(n, m - n, row_ptr[n], row_ptr[m]));
        n = m;
    }
    t->n_chunks = static_cast<int32_t>(chunk_desc.size());
    // weight-gradient work units: runs of short columns, chunks of long ones
    std::vector<int4> dwu;
    for (int64_t c = 0; c < n_cols;) {
        const int32_t k0 = col_ptr[c], k1 = col_ptr[c + 1];
        if (k1 - k0 > kDwUnitEntries) {
            for (int32_t k = k0; k < k1; k += kDwUnitEntries)
                dwu.push_back(make_int4(static_cast<int>(c), 1, k, std::min(k + kDwUnitEntries, k1)));
            ++c;
            continue;
        }
        int64_t m = c + 1;
        while (m < n_cols && m - c < kWave && col_ptr[m + 1] - k0 <= kDwUnitEntries) ++m;
        dwu.push_back(make_int4(static_cast<int>(c), static_cast<int>(m - c), k0, col_ptr[m]));
        c = m;
    }
    t->n_dwu = static_cast<int32_t>(dwu.size());
    std::vector<int4> dzc;
    for (int32_t u = 0; u < t->n_dwu;) {
        if (dwu[u].y != 1) { ++u; continue; }
        int32_t v = u + 1;
        while (v < t->n_dwu && dwu[v].y == 1 && dwu[v].x == dwu[u].x) ++v;
        dzc.push_back(make_int4(dwu[u].x, u, v - u, 0));
        u = v;
    }
    t->n_dzc = static_cast<int32_t>(dzc.size());
    t->basis_host = new float[static_cast<size_t>(n_types) * n_basis];
    std::memcpy(t->basis_host, basis, sizeof(float) * n_types * n_basis);
    int rc = GLIF_OK;
    if ((rc = upload(&t->basis, basis, static_cast<size_t>(n_types) * n_basis)) ||
        (rc = upload(&t->col_ptr, col_ptr.data(), col_ptr.size())) ||
        (rc = upload(&t->order, order.data(), order.size())) ||
        (rc = upload(&t->ps, ps.data(), ps.size())) ||
        (rc = upload(&t->row_ptr, row_ptr.data(), row_ptr.size())) ||
        (rc = upload(&t->chunk_desc, chunk_desc.data(), chunk_desc.size())) ||
        (rc = upload(&t->dwu, dwu.data(), dwu.size())) ||
        (rc = upload(&t->dzc, dzc.data(), dzc.size())) ||
        (rc = upload(&t->perm, perm.data(), perm.size())) ||
        (rc = upload(&t->pd, pd.data(), pd.size())) ||
        (with_pidx && (rc = upload(&t->pidx, pidx.data(), pidx.size()))) ||
        (rc = upload(&t->sid_row, sid_row.data(), sid_row.size())) ||
        (rc = upload(&t->ph_ptr, ph_ptr.data(), ph_ptr.size())) ||
        (rc = upload(&t->ph_order, ph_order.data(), ph_order.size())) ||
        (rc = upload(&t->order_inv, order_inv.data(), order_inv.size())) ||
        (rc = upload(&t->ph_inv, ph_inv.data(), ph_inv.size())) ||
        (rc = upload(&t->ph_src, ph_src.data(), ph_src.size())) ||
        (rc = upload(&t->ph_pw, ph_pw.data(), ph_pw.size())) ||
        (ell_len && (rc = upload(&t->ell_pw, ell_pw.data(), ell_pw.size()))) ||
        (ell_len && (rc = upload(&t->ell_src, ell_src.data(), ell_src.size()))) ||
        (n_gs && (rc = upload(&t->gs_seg, gs_seg.data(), gs_seg.size()))) ||
        (n_gs && (rc = upload(&t->gs_pw, gs_pw.data(), gs_pw.size()))) ||
        (n_gs && (rc = upload(&t->gs_src, gs_src.data(), gs_src.size())))) {
        free_table(t);
        return rc;
    }
    for (float **wp : {&t->w_col, &t->w_row}) {
        hipError_t e = hipMalloc(reinterpret_cast<void **>(wp), std::max<int64_t>(n_syn, 1) * sizeof(float));
        if (e != hipSuccess) {
            free_table(t);
            return hip_fail(e, "hipMalloc(weights)");
        }
        if (n_syn) (void)hipMemset(*wp, 0, n_syn * sizeof(float));
    }
    if ((rc = build_own_rows(t, col_ptr.data(), ps.data(), ph_src.data()))) {
        free_table(t);
        return rc;
    }
    // two-pass plans of the two reorderings done every training step (config 2's recurrent
    // table: 305 us each as one gather).  The weight refresh stages through the table's own
    // buffer (refreshes of one table write its weight copies, so they never overlap); the
    // gradient reorder of a cell's backward stages through that backward's workspace, so
    // backwards on other streams stay independent.
    if (n_syn >= kPermMinSyn && ((rc = build_perm_plan(&t->pcol, order.data(), n_syn, true)) ||
                                 (rc = build_perm_plan(&t->pinv, order_inv.data(), n_syn, false)))) {
        free_table(t);
        return rc;
    }
    *out = reinterpret_cast<glif_table *>(t);
    return GLIF_OK;
}

void glif_table_destroy(glif_table *t) { free_table(reinterpret_cast<Table *>(t)); }

int64_t glif_table_n_syn(const glif_table *t) {
    return t ? reinterpret_cast<const Table *>(t)->n_syn : -1;
}

int glif_table_pre_ind(const glif_table *tt, const int32_t **order, const int32_t **row_splits) {
    if (!tt || !order || !row_splits) return fail(GLIF_EINVAL, "NULL argument");
    const Table *t = reinterpret_cast<const Table *>(tt);
    *order = t->order;
    *row_splits = t->col_ptr;
    return GLIF_OK;
}

int glif_table_set_weights(glif_table *tt, const float *w, void *stream) {
    if (!tt) return fail(GLIF_EINVAL, "NULL argument");
    Table *t = reinterpret_cast<Table *>(tt);
    if (t->n_syn == 0) return GLIF_OK;   // no synapses, no weights (w may be NULL)
    if (!w) return fail(GLIF_EINVAL, "NULL argument");
    hipStream_t s = static_cast<hipStream_t>(stream);
    int rc = launch_perm_gather(t->w_col, w, t->order, t->pcol, t->n_syn, t->pcol.mid, s);
    if (rc) return rc;
    // the type-phased and grouped copies from w_col (near-sequential reads)
    if (t->n_syn) {
        hipLaunchKernelGGL(k_gather_pair_w, dim3(grid_for(t->n_syn)), dim3(kBlock), 0, s, t->ph_pw, t->w_col,
                           t->ph_src, t->n_syn);
        GLIF_HIP(hipGetLastError());
    }
    if (t->n_gs) {
        hipLaunchKernelGGL(k_gather_ell_w, dim3(grid_for(t->n_gs)), dim3(kBlock), 0, s, t->gs_pw, t->w_col,
                           t->gs_src, t->n_gs);
        GLIF_HIP(hipGetLastError());
    }
    // the compact-row copies (a cell's, the table's own)
    int rcc = gather_compact_weights(t, t->cg, s);
    if (!rcc) rcc = gather_compact_weights(t, t->og, s);
    if (rcc) return rcc;
    if (t->ell_len) {
        const int64_t n_ell = static_cast<int64_t>(t->ell_len) * t->n_post;
        hipLaunchKernelGGL(k_gather_ell_w, dim3(grid_for(n_ell)), dim3(kBlock), 0, s, t->ell_pw, w, t->ell_src,
                           n_ell);
        GLIF_HIP(hipGetLastError());
    }
    return launch_gather_f32(t->w_row, w, t->perm, t->n_syn, s);
}

}  // extern "C"
