// Device code of the synaptic-current operator (calculate_synaptic_currents,
// models.py:103-263), shared by the op-level entry points (syn.hip) and the
// T-step cell (cell.hip).
//
// Layouts
//   column-grouped table (Table::col_ptr/ps/w_col): the synapses of presynaptic
//     column c are k in [col_ptr[c], col_ptr[c+1]); ps[k] = post | syn_id << 24.
//   post-grouped table (Table::row_ptr/pd/sid_row/w_row): the synapses of post n
//     are j in [row_ptr[n], row_ptr[n+1]) in ascending (column, synapse id);
//     pd[j] = pre | (delay - 1) << 24.
//   type-phased table (Table::ph_ptr/ph_pw): synapses ordered by (syn_id, column,
//     synapse id); the type-s synapses of column c are
//     k in [ph_ptr[s * n_cols + c], ph_ptr[s * n_cols + c + 1]);
//     ph_pw[k] = {post, weight bits}.
//   grouped row-sliced table (Table::gs_seg/gs_pw, recurrent tables): lane group g's
//     columns 4g..4g+3, by G-row slice, then G row (syn_id * n_post + post); entries
//     {row | column-in-group << 29, weight bits}, each segment padded to 8 entries.
//   I  [B][n_post][nb]  (the reference's i_rec_flat [B*N, nb]).
//   G  [n_types][n_post][R]: G[s][post][e] = sum_r dy[b][post][r] * basis[s][r] for
//     element e (batch b, possibly of several timesteps), the per-synapse-type
//     projection of dy that both dz and dW need.
#pragma once

#include "glif_internal.h"

namespace glif {

// Products and sums are kept as separate roundings (the library is built with
// -ffp-contract=off) so the deterministic path matches the reference's
// Mul-then-UnsortedSegmentSum arithmetic bit for bit.

__device__ inline void load_basis_lds(float *lds, const float *basis, int n) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) lds[i] = basis[i];
    __syncthreads();
}

// Per-batch weight multipliers of an event: 1 for spikes, the Poisson count for
// the background source (models.py:917-931), the dense input value for the
// op-level entry points called with counts.
struct MultOne {
    static constexpr bool kOne = true;
    __device__ float operator()(int) const { return 1.0f; }
};
struct MultU8 {
    static constexpr bool kOne = false;
    const uint8_t *p;
    int64_t stride;
    __device__ float operator()(int b) const { return static_cast<float>(p[b * stride]); }
};
struct MultF32 {
    static constexpr bool kOne = false;
    const float *p;
    int64_t stride;
    __device__ float operator()(int b) const { return p[b * stride]; }
};

// ---- event-driven push of one column ------------------------------------------
// The L lanes of a sub-wave stream column c's synapses and add
// (w * mult_b) * basis[syn_id][r] into I[b][post][r] with fp32 atomics for every
// batch entry b in `bmask`.  mult_b = 1 for spikes, the Poisson count for the
// background source.  Zero products are skipped: adding +/-0 never changes a sum
// that starts at +0.
// I is addressed as I[b * bstride + post * pstride + r * rstride] (the op's
// [B*N][nb] output, or the cell's receptor-major [nb][B][N] accumulator).
template <int L, class Mult>
__device__ inline void push_column(int lane_s, int32_t lo, int32_t hi, uint32_t bmask,
                                   Mult mult, const uint32_t *__restrict__ ps,
                                   const float *__restrict__ w, const float *basis_lds, int nb,
                                   int64_t bstride, int64_t pstride, int64_t rstride,
                                   float *__restrict__ I) {
    for (int32_t k = lo + lane_s; k < hi; k += L) {
        const uint32_t p = ps[k];
        const float wk = w[k];
        const int32_t post = static_cast<int32_t>(p & kLow24);
        const float *bs = basis_lds + (p >> 24) * nb;
        uint32_t m = bmask;
        while (m) {
            const int b = __ffs(m) - 1;
            m &= m - 1;
            const float wv = Mult::kOne ? wk : wk * mult(b);
            float *dst = I + static_cast<int64_t>(b) * bstride + static_cast<int64_t>(post) * pstride;
            for (int r = 0; r < nb; ++r) {
                const float v = wv * bs[r];
                if (v != 0.0f) unsafeAtomicAdd(dst + r * rstride, v);
            }
        }
    }
}

// ---- event-driven push of one column into per-type slots ---------------------------
// As push_column, with one atomic per (synapse, batch entry): (w * mult_b) goes to the
// synapse's type slot of its post, I[rank * rstride + b * bstride + post] (cps[k] = post |
// rank << 24, rank = the position of the synapse's type among the types reaching the post);
// the step then forms each receptor's current as sum over the slots of slot * basis[type][r].
template <int L, class Mult>
__device__ inline void push_column_typed(int lane_s, int32_t lo, int32_t hi, uint32_t bmask, Mult mult,
                                         const uint32_t *__restrict__ cps, const float *__restrict__ w,
                                         int64_t bstride, int64_t rstride, float *__restrict__ I) {
    for (int32_t k = lo + lane_s; k < hi; k += L) {
        const uint32_t p = cps[k];
        const float wk = w[k];
        float *base = I + static_cast<int64_t>(p >> 24) * rstride + static_cast<int64_t>(p & kLow24);
        uint32_t m = bmask;
        while (m) {
            const int b = __ffs(m) - 1;
            m &= m - 1;
            const float wv = Mult::kOne ? wk : wk * mult(b);
            if (wv != 0.0f) unsafeAtomicAdd(base + static_cast<int64_t>(b) * bstride, wv);
        }
    }
}

// ---- fused backward of one column (dz and dW) -------------------------------------
// dz[b] = sum_k w[k] * G[post_k][sid_k][b]   (returned reduced over the sub-wave)
// dw_col[k] += sum_{b in bmask, ascending} G[post_k][sid_k][b] * mult_b
template <int L, int BQ, bool WANT_DZ, class Mult>
__device__ inline void bwd_column(int lane_s, int32_t lo, int32_t hi, uint32_t bmask,
                                  Mult mult, const uint32_t *__restrict__ ps,
                                  const float *__restrict__ w, const float *__restrict__ G,
                                  int32_t n_post, float *__restrict__ dw_col, float (&acc)[4 * BQ]) {
#pragma unroll
    for (int i = 0; i < 4 * BQ; ++i) acc[i] = 0.0f;
    for (int32_t k = lo + lane_s; k < hi; k += L) {
        const uint32_t p = ps[k];
        const float4 *g4 = reinterpret_cast<const float4 *>(
            G + (static_cast<int64_t>(p >> 24) * n_post + (p & kLow24)) * (4 * BQ));
        float g[4 * BQ];
#pragma unroll
        for (int q = 0; q < BQ; ++q) {
            const float4 v = g4[q];
            g[4 * q + 0] = v.x;
            g[4 * q + 1] = v.y;
            g[4 * q + 2] = v.z;
            g[4 * q + 3] = v.w;
        }
        if (WANT_DZ) {
            const float wk = w[k];
#pragma unroll
            for (int i = 0; i < 4 * BQ; ++i) acc[i] += wk * g[i];
        }
        if (bmask) {
            float a = dw_col[k];
#pragma unroll
            for (int b = 0; b < 4 * BQ; ++b)
                if (bmask & (1u << b)) a += Mult::kOne ? g[b] : g[b] * mult(b);
            dw_col[k] = a;
        }
    }
    if (WANT_DZ) {
#pragma unroll
        for (int i = 0; i < 4 * BQ; ++i) {
            float v = acc[i];
#pragma unroll
            for (int o = L / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
            acc[i] = v;
        }
    }
}

// G[s][post][b] = sum_r dy[b][post][r] * basis[s][r]  (sequential r, the order of
// einsum('cr,cr->c') in models.py:232).
__device__ inline void write_G(float *__restrict__ G, int64_t post, int b, int Bp, const float *dy,
                               const float *basis_lds, int n_types, int nb, int32_t n_post) {
    for (int s = 0; s < n_types; ++s) {
        const float *bs = basis_lds + s * nb;
        float e = dy[0] * bs[0];
        for (int r = 1; r < nb; ++r) e = e + dy[r] * bs[r];
        G[(static_cast<int64_t>(s) * n_post + post) * Bp + b] = e;
    }
}

// ---- column backward: dz of every column, dW of its active events ---------------
// G rows hold R floats: n_elem used elements (for the cell, W consecutive reverse
// timesteps x B batch entries, e = w*B + b), zero padding after.  A group of
// LG = R/4 lanes owns one column and walks its synapses type by type in the
// type-phased table, U at a time (U independent entry loads, then U independent
// row gathers); lane q accumulates elements 4q..4q+3 of w * G[s][post].  One G row
// is one 64-byte request per synapse per window, and waves that start together
// work on the same type.  Each synapse is touched by one lane group: dz and dW
// accumulate in a fixed order (deterministic) without atomics.
//
// Measured on MI355X (16.5M synapses, G of 5 types x 66k posts x 64 B = 21 MB):
// random row gathers run at ~230 G rows/s from an L2-resident slice (<= ~4 MB) and
// at ~74 G rows/s from the whole 21 MB (Infinity Cache), and this walk lands near
// the latter.  Tiling the table so one slice of G stays in L2 needs the waves in
// strict lockstep; without a grid barrier the tried forms (64-column blocks by
// phase of type x post chunk with an LDS reduction, resident grids with several
// columns per group) were slower: their L2 hit rate stayed at 40-60% and the
// reduction cost more than it saved.  LDS float atomics (ds_add_f32) ran at ~0.3
// lane-ops per clock per CU, unusable for the dz sums.
struct ColArgs {
    int64_t n_cols;
    int32_t n_post, n_types, n_elem;
    const int32_t *ph_ptr;   // [n_types * n_cols + 1]
    const uint2 *ph_pw;      // {post, weight bits}
    const float *G;          // [n_types][n_post][R], < 4 GiB
    int32_t want_dz;
    float *dw;               // [n_syn] type-phased order, accumulated; or nullptr
    // when set, each synapse's dW is written once, straight to dw[dw_ref[k]] (reference
    // order, the caller zero-fills dw) instead of accumulated at position k
    const int32_t *dw_ref;
    // 1: ph_pw[k].x is the synapse's G row itself (compact rows, post * rows per post +
    // rank), not the post of a type-major row syn_id * n_post + post
    int32_t compact;
};

// Op-level activity: z [B][n_cols] dense, element e = b.
struct ActDense {
    static constexpr bool kUnitMult = false;
    const float *z;
    float *dz;        // [B][n_cols]
    int64_t n_cols;
    int32_t counts;
    using Col = int64_t;
    __device__ Col col(int64_t c) const { return c; }
    __device__ bool on(Col c, int e) const { return z[e * n_cols + c] > 0.0f; }
    __device__ float mult(int64_t c, int e) const { return counts ? z[e * n_cols + c] : 1.0f; }
    __device__ float *out(Col c, int e) const { return dz + e * n_cols + c; }
};

template <int LG, int U, class Act>
__device__ inline void bwd_cols(const ColArgs &a, const Act &act) {
    constexpr int R = 4 * LG;
    const int q = threadIdx.x % LG;
    const int64_t c = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) / LG;
    if (c >= a.n_cols) return;  // the whole lane group leaves together
    const typename Act::Col ci = act.col(c);
    uint32_t bits = 0;
    float mult[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    if (a.dw) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = 4 * q + i;
            if (e < a.n_elem && act.on(ci, e)) {
                bits |= 1u << i;
                if (!Act::kUnitMult) mult[i] = act.mult(c, e);
            }
        }
    }
    uint32_t any = bits;
#pragma unroll
    for (int o = 1; o < LG; o <<= 1) any |= __shfl_xor(any, o, kWave);
    const char *Gb = reinterpret_cast<const char *>(a.G) + static_cast<uint32_t>(q) * 16u;
    const uint32_t type_bytes = a.compact ? 0u : static_cast<uint32_t>(a.n_post) * (R * 4u);
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    // the next type's segment bounds are loaded while the current type is walked
    int32_t nlo = a.ph_ptr[c], nhi = a.ph_ptr[c + 1];
    for (int s = 0; s < a.n_types; ++s) {
        const int32_t lo = nlo, hi = nhi;
        if (s + 1 < a.n_types) {
            const int64_t pi = static_cast<int64_t>(s + 1) * a.n_cols + c;
            nlo = a.ph_ptr[pi];
            nhi = a.ph_ptr[pi + 1];
        }
        const char *Gs = Gb + static_cast<uint32_t>(s) * type_bytes;
        for (int32_t k0 = lo; k0 < hi; k0 += U) {
            uint2 e[U];
#pragma unroll
            for (int u = 0; u < U; ++u) e[u] = a.ph_pw[min(k0 + u, hi - 1)];
            // an active column's dW values travel with the entries (no extra round trip)
            float old[U];
#pragma unroll
            for (int u = 0; u < U; ++u)
                old[u] = (any && q == 0 && k0 + u < hi) ? (a.dw_ref ? 0.0f : a.dw[k0 + u]) : 0.0f;
            int32_t dst[U];
#pragma unroll
            for (int u = 0; u < U; ++u)
                dst[u] = (any && q == 0 && k0 + u < hi) ? (a.dw_ref ? a.dw_ref[k0 + u] : k0 + u) : 0;
            float4 g[U];
#pragma unroll
            for (int u = 0; u < U; ++u) g[u] = *reinterpret_cast<const float4 *>(Gs + e[u].x * (R * 4u));
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (k0 + u >= hi) break;  // uniform within the lane group
                const float w = a.want_dz ? __uint_as_float(e[u].y) : 0.0f;
                acc[0] += w * g[u].x;
                acc[1] += w * g[u].y;
                acc[2] += w * g[u].z;
                acc[3] += w * g[u].w;
            }
            if (any) {  // uniform within the lane group
                // all U partials, then their group reductions, then the stores of the
                // U (distinct, group-owned) dW entries
                float pp[U];
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    pp[u] = 0.0f;
                    if (bits & 1u) pp[u] += g[u].x * mult[0];
                    if (bits & 2u) pp[u] += g[u].y * mult[1];
                    if (bits & 4u) pp[u] += g[u].z * mult[2];
                    if (bits & 8u) pp[u] += g[u].w * mult[3];
                }
#pragma unroll
                for (int o = 1; o < LG; o <<= 1) {
#pragma unroll
                    for (int u = 0; u < U; ++u) pp[u] += __shfl_xor(pp[u], o, kWave);
                }
                if (q == 0) {
#pragma unroll
                    for (int u = 0; u < U; ++u)
                        if (k0 + u < hi) a.dw[dst[u]] = old[u] + pp[u];
                }
            }
        }
    }
    if (a.want_dz) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = 4 * q + i;
            if (e < a.n_elem) *act.out(ci, e) = acc[i];
        }
    }
}

// ---- grouped row-sliced backward (16-float G rows) ------------------------------
// dz of every column over the grouped row-sliced order: lane group g (4 lanes, lane q
// holding floats 4q..4q+3 of a row) owns columns kGsCols*g .. (4 of them); it walks its entries of
// one G-row slice at a time, 8 per step (one 64-byte load, lane q holding entries 2q and
// 2q+1, shared in the group by DPP), and adds w * G[row] into the column's accumulator.
// Every wave finishes a slice before starting the next, so the waves in flight gather
// from one quarter of G at a time, and a group owns its columns, so dz needs no atomics.
// Each column sums its entries in G-row order (syn_id, then post), the order of
// bwd_cols.  The dW of active columns is a separate pass (k_bwd_rec_dw in cell.hip):
// holding it here costs a third more registers and a second walk per group.
//
// Measured on MI355X with a config-2-sized table (16.5M synapses, 330k columns, G 21 MB):
// 146 us per pass against 195 us for the type-phased walk.  The type-phased walk makes
// 27.7M L2 requests (its 8-byte entry loads are re-requested), a row-sorted walk without
// slices 18.5M but misses L2 on 42% of them; the slices bring the misses down while the
// 8-entry loads keep the requests near one per synapse.
struct GsArgs {
    int64_t n_cols, n_groups;
    int32_t n_elem;
    const int32_t *seg;   // [n_groups * (kGsSlices + 1)]
    const uint2 *pw;      // {row | column-in-group << kGsRowBits, weight bits}
    const float *G;       // [rows][4 LG], < 4 GiB
    // the groups walked: [g_lo, g_hi), g_hi = 0 for every group from g_lo; g_lo a multiple of
    // the groups of a wave (kWave / LG)
    int64_t g_lo = 0, g_hi = 0;
};

// value of lane `src` of this lane's quad (DPP quad_perm broadcast)
__device__ inline uint32_t quad_bcast(uint32_t v, int src) {
    switch (src) {
        case 0: return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0x00, 0xF, 0xF, false));
        case 1: return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0x55, 0xF, 0xF, false));
        case 2: return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0xAA, 0xF, 0xF, false));
        default: return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0xFF, 0xF, 0xF, false));
    }
}

// value of lane `src` of this lane's group of LG lanes (LG = 2: the lane pairs of a quad,
// quad_perm [src, src, 2 + src, 2 + src]; LG = 4: the quad)
template <int LG>
__device__ inline uint32_t group_bcast(uint32_t v, int src) {
    static_assert(LG == 2 || LG == 4, "lane groups of 2 or 4");
    if (LG == 4) return quad_bcast(v, src);
    return src == 0 ? static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0xA0, 0xF, 0xF, false))
                    : static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0xF5, 0xF, 0xF, false));
}

// LDS floats per wave for the dz staging of bwd_groups: [R][columns per wave + 1] for
// LG = 4 (16 floats x 16 kGsCols columns) or LG = 2 (8 x 32 kGsCols), whichever is larger
constexpr int kGsStage = 16 * (16 * kGsCols + 1) > 8 * (32 * kGsCols + 1) ? 16 * (16 * kGsCols + 1)
                                                                           : 8 * (32 * kGsCols + 1);

// LG lanes per G row (R = 4 LG floats, LG = 2 or 4), lane q holding floats 4q..4q+3; a chunk
// of 8 entries is 8 / LG entries per lane (one or two 16-byte loads).  stage: kGsStage floats
// of LDS per wave of the block.
template <int LG, class Act>
__device__ inline void bwd_groups(const GsArgs &a, const Act &act, float *stage, int64_t bid) {
    constexpr int R = 4 * LG, EPL = 8 / LG, CW = (kWave / LG) * kGsCols;
    const int q = threadIdx.x % LG;
    const int64_t g = a.g_lo + (bid * blockDim.x + threadIdx.x) / LG;
    // a group past the end walks nothing but still takes part in the staging below
    const bool own = g < (a.g_hi ? a.g_hi : a.n_groups);
    const char *Gb = reinterpret_cast<const char *>(a.G) + static_cast<uint32_t>(q) * 16u;
    float acc[kGsCols][4];
#pragma unroll
    for (int j = 0; j < kGsCols; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[j][i] = 0.0f;
    const int32_t *sg = a.seg + (own ? g : 0) * (kGsSlices + 1);
    int32_t lo = own ? sg[0] : 0;
    for (int p = 0; p < kGsSlices; ++p) {
        const int32_t hi = own ? sg[p + 1] : 0;
        for (int32_t k0 = lo; k0 < hi; k0 += 8) {
            uint2 my[EPL];
#pragma unroll
            for (int h = 0; h < EPL; h += 2) {
                const uint4 v = *reinterpret_cast<const uint4 *>(a.pw + k0 + EPL * q + h);
                my[h] = make_uint2(v.x, v.y);
                my[h + 1] = make_uint2(v.z, v.w);
            }
            float4 gv[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const uint32_t r = group_bcast<LG>(my[u % EPL].x, u / EPL);
                gv[u] = *reinterpret_cast<const float4 *>(Gb + (r & kGsRowMask) * (R * 4u));
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const uint32_t col = group_bcast<LG>(my[u % EPL].x, u / EPL) >> kGsRowBits;
                const float wu = __uint_as_float(group_bcast<LG>(my[u % EPL].y, u / EPL));
                const float t0 = wu * gv[u].x, t1 = wu * gv[u].y, t2 = wu * gv[u].z, t3 = wu * gv[u].w;
                // acc[col] += t with one fma per element: m * t is exactly t or 0, so fma(m, t, acc)
                // rounds acc + t once, as the add does, and leaves acc alone otherwise (acc starts
                // at +0 and never becomes -0, so adding a signed zero changes nothing)
#pragma unroll
                for (int j = 0; j < kGsCols; ++j) {
                    const float m = col == static_cast<uint32_t>(j) ? 1.0f : 0.0f;
                    acc[j][0] = __builtin_fmaf(m, t0, acc[j][0]);
                    acc[j][1] = __builtin_fmaf(m, t1, acc[j][1]);
                    acc[j][2] = __builtin_fmaf(m, t2, acc[j][2]);
                    acc[j][3] = __builtin_fmaf(m, t3, acc[j][3]);
                }
            }
        }
        lo = hi;
    }
    // dz through LDS: the wave's groups own CW consecutive columns, so each element's
    // values leave as coalesced stores
    const int lane = threadIdx.x % kWave;
    float *st = stage + (threadIdx.x / kWave) * kGsStage;
    const int gl = lane / LG;
#pragma unroll
    for (int j = 0; j < kGsCols; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) st[(4 * q + i) * (CW + 1) + kGsCols * gl + j] = acc[j][i];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int64_t cw0 = (g - gl) * kGsCols;
    const int64_t c_end = a.g_hi ? min(a.n_cols, a.g_hi * kGsCols) : a.n_cols;
#pragma unroll
    for (int cc = lane; cc < CW; cc += kWave) {
        const int64_t c = cw0 + cc;
        if (c < c_end) {
            const typename Act::Col ci = act.col(c);
            for (int e = 0; e < a.n_elem; ++e) *act.out(ci, e) = st[e * (CW + 1) + cc];
        }
    }
}

// Row length (floats) of G for B batch entries over W timesteps: a power of two >= 4.
__host__ __device__ inline int g_row(int W, int B) {
    int r = 4;
    while (r < W * B) r <<= 1;
    return r;
}

}  // namespace glif
