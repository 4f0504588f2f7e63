// Op-level entry points of calculate_synaptic_currents (models.py:103-263):
// forward (event push or deterministic pull) and the custom gradient.
#include <algorithm>
#include <cstring>
#include <mutex>

#include "compact.h"
#include "glif_internal.h"
#include "prof.h"
#include "pull_kernels.h"
#include "syn_kernels.h"

namespace glif {

// Tables with a column longer than this take dz over work units and pull in event mode too (the
// background table's shape).  The dz walk sums a column on one lane per 4 batch entries and the
// column scan pushes it on one wave, so their time is the longest column's serial chain (a
// 6600-synapse column: ~4 ms for dz, ~5 ms for the push); the units split long columns over many
// waves and cost at most ~1.5x the walk on short ones (runs of short columns use few lanes).
constexpr int32_t kUnitDzMinColLen = 2 * kDwUnitEntries;
// The event push takes the units when the column scan (a wave per 64 columns) would run on fewer
// waves than this (the LGN table's 17,400 columns: 272 waves) or a column has more synapses than
// one unit (its chunks then go to waves of their own).
constexpr int64_t kPushUnitsMaxScanWaves = 2048;
// dz takes the units too when the walk would run on fewer lanes than this.
constexpr int64_t kUnitDzMaxWalkLanes = 1024 * kWave;

// ---------------------------------------------------------------- forward ----
// Deterministic pull of Poisson-count inputs (the background form, models.py:917-931): thread
// per (b, post) walks the post's row in ascending (column, synapse id) -- the order in which
// TF's CPU UnsortedSegmentSum meets the events of this (b, post) -- scaling each weight by its
// input's count, and writes I[b][post][:] (models.py:141-169).  Spike inputs take the row
// pulls over batch masks (pull_kernels.h), which read each entry once for all batch entries.
__global__ void __launch_bounds__(kBlock)
    k_syn_pull_dense(const float *__restrict__ z, int32_t B, int64_t n_cols, int32_t n_post,
                     int32_t n_pre, const int32_t *__restrict__ row_ptr,
                     const uint32_t *__restrict__ pd, const uint8_t *__restrict__ sid,
                     const float *__restrict__ w, const float *__restrict__ basis, int n_types,
                     int nb, float *__restrict__ I) {
    extern __shared__ float basis_lds[];
    load_basis_lds(basis_lds, basis, n_types * nb);
    const int64_t gt = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (gt >= static_cast<int64_t>(B) * n_post) return;
    const int b = static_cast<int>(gt / n_post);
    const int32_t n = static_cast<int32_t>(gt % n_post);
    float acc[kMaxBasis];
    for (int r = 0; r < nb; ++r) acc[r] = 0.0f;
    const float *zb = z + static_cast<int64_t>(b) * n_cols;
    for (int32_t j = row_ptr[n]; j < row_ptr[n + 1]; ++j) {
        const uint32_t q = pd[j];
        const int64_t c = static_cast<int64_t>(q & kLow24) + static_cast<int64_t>(q >> 24) * n_pre;
        const float a = zb[c];
        if (!(a > 0.0f)) continue;
        const float wv = w[j] * a;
        const float *bs = basis_lds + sid[j] * nb;
        for (int r = 0; r < nb; ++r) acc[r] = acc[r] + wv * bs[r];
    }
    float *dst = I + gt * nb;
    for (int r = 0; r < nb; ++r) dst[r] = acc[r];
}

// Event push straight from z [B][n_cols]: a wave per 64 consecutive columns builds each
// column's batch mask (z > 0, the test of tf.where at models.py:128-130), and all 64 lanes
// push the wave's active columns one after another.  No column list, no count pass.
// The event push over the table's work units (a run of up to 64 short columns, or a chunk of
// at most kDwUnitEntries synapses of a long column), a wave per unit: the lanes hold the
// run's columns' batch masks, and all 64 lanes push each active column's share of the unit.
// For tables whose column scan would run on few waves (few columns, or long ones).
template <bool COUNTS>
__global__ void __launch_bounds__(kBlock)
    k_syn_push_units(const float *__restrict__ z, int32_t B, int64_t n_cols, const int4 *__restrict__ units,
                     int32_t n_units, const int32_t *__restrict__ col_ptr, const uint32_t *__restrict__ ps,
                     const float *__restrict__ w, const float *__restrict__ basis, int n_types, int nb,
                     int32_t n_post, float *__restrict__ I) {
    extern __shared__ float basis_lds[];
    load_basis_lds(basis_lds, basis, n_types * nb);
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t ui = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) +
                       __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
    if (ui >= n_units) return;  // the whole wave leaves together
    const int4 un = units[ui];
    uint32_t m = 0u;
    if (lane < un.y)
        for (int b = 0; b < B; ++b) m |= (z[b * n_cols + un.x + lane] > 0.0f ? 1u : 0u) << b;
    uint64_t act = __ballot(m != 0u);
    while (act) {
        const int l = __builtin_ctzll(act);
        act &= act - 1ull;
        const uint32_t ml = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(m), l));
        const int64_t cl = un.x + l;
        const int32_t lo = un.y == 1 ? un.z : col_ptr[cl];
        const int32_t hi = un.y == 1 ? un.w : col_ptr[cl + 1];
        if (COUNTS)
            push_column<kWave>(lane, lo, hi, ml, MultF32{z + cl, n_cols}, ps, w, basis_lds, nb,
                               static_cast<int64_t>(n_post) * nb, nb, 1, I);
        else
            push_column<kWave>(lane, lo, hi, ml, MultOne{}, ps, w, basis_lds, nb, static_cast<int64_t>(n_post) * nb,
                               nb, 1, I);
    }
}

template <bool COUNTS>
__global__ void __launch_bounds__(kBlock)
    k_syn_push_scan(const float *__restrict__ z, int32_t B, int64_t n_cols, const int32_t *__restrict__ col_ptr,
                    const uint32_t *__restrict__ ps, const float *__restrict__ w, const float *__restrict__ basis,
                    int n_types, int nb, int32_t n_post, float *__restrict__ I) {
    extern __shared__ float basis_lds[];
    load_basis_lds(basis_lds, basis, n_types * nb);
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t n_words = (n_cols + kWave - 1) / kWave;
    const int64_t waves = static_cast<int64_t>(gridDim.x) * (blockDim.x / kWave);
    const int64_t u0 = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) +
                       __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
    for (int64_t u = u0; u < n_words; u += waves) {
        const int64_t c = u * kWave + lane;
        uint32_t m = 0u;
        if (c < n_cols)
            for (int b = 0; b < B; ++b) m |= (z[b * n_cols + c] > 0.0f ? 1u : 0u) << b;
        uint64_t act = __ballot(m != 0u);
        while (act) {
            const int l = __builtin_ctzll(act);
            act &= act - 1ull;
            const uint32_t ml = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(m), l));
            const int64_t cl = u * kWave + l;
            if (COUNTS)
                push_column<kWave>(lane, col_ptr[cl], col_ptr[cl + 1], ml, MultF32{z + cl, n_cols}, ps, w,
                                   basis_lds, nb, static_cast<int64_t>(n_post) * nb, nb, 1, I);
            else
                push_column<kWave>(lane, col_ptr[cl], col_ptr[cl + 1], ml, MultOne{}, ps, w, basis_lds, nb,
                                   static_cast<int64_t>(n_post) * nb, nb, 1, I);
        }
    }
}

// ---------------------------------------------------------------- backward ----
// G rows from dy [B][n_post][nb].  A workgroup takes P consecutive posts: it copies their dy
// into LDS (coalesced), then each thread writes row quarters (four batch entries of one G row,
// one 16-byte store; consecutive threads write consecutive quarters), padding entries b >= B
// written +0 (no separate fill).  Type-major rows: G[s * n_post + post][b] =
// sum_r dy[b][post][r] * basis[s][r]; a table's own compact rows (COMPACT): G[post * rows + q][b]
// with s = gtype[post][q], +0 past the post's types.  Each element sums r ascending from
// dy[0] * bs[0], one rounding per product and per add.
// The workgroups from g_blocks on zero the dense dW instead (grid-stride), which the
// weight-gradient pass after this launch writes for the active synapses.
template <bool COMPACT>
__global__ void __launch_bounds__(kBlock)
    k_make_G(const float *__restrict__ dy, int32_t B, int32_t n_post, int Bp, const float *__restrict__ basis,
             int n_types, int nb, const uint8_t *__restrict__ gtype, int rows, int P, float *__restrict__ G,
             int g_blocks, float *__restrict__ fill, int64_t n_fill) {
    if (static_cast<int>(blockIdx.x) >= g_blocks) {
        const int64_t stride = static_cast<int64_t>(gridDim.x - g_blocks) * blockDim.x;
        for (int64_t i = static_cast<int64_t>(blockIdx.x - g_blocks) * blockDim.x + threadIdx.x; i < n_fill;
             i += stride)
            fill[i] = 0.0f;
        return;
    }
    extern __shared__ float lds_f[];
    float *basis_lds = lds_f;
    float *tile = lds_f + ((n_types * nb + 3) & ~3);   // [B][P][nb]
    for (int i = threadIdx.x; i < n_types * nb; i += blockDim.x) basis_lds[i] = basis[i];
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * P;
    const int np = static_cast<int>(min(static_cast<int64_t>(P), n_post - n0));
    const int span = np * nb, total = B * span;
    for (int base = 0; base < total; base += 8 * static_cast<int>(blockDim.x)) {
        float v[8];   // the loads of a round go out together
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int i = base + k * static_cast<int>(blockDim.x) + static_cast<int>(threadIdx.x);
            const int b = i / span;
            v[k] = i < total ? dy[(static_cast<int64_t>(b) * n_post + n0) * nb + (i - b * span)] : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int i = base + k * static_cast<int>(blockDim.x) + static_cast<int>(threadIdx.x);
            const int b = i / span;
            if (i < total) tile[b * P * nb + (i - b * span)] = v[k];
        }
    }
    __syncthreads();
    const int nrow = COMPACT ? rows : n_types;
    const int nq = Bp / 4;
    const int items = nrow * np * nq;
    for (int it = threadIdx.x; it < items; it += blockDim.x) {
        const int b0 = (it % nq) * 4;
        int p, s;
        int64_t row;
        if (COMPACT) {   // memory order: post, then rank, then quarter
            const int pq = it / nq;
            p = pq / rows;
            row = (n0 + p) * rows + (pq - p * rows);
            s = gtype[row];
        } else {         // type, then post, then quarter
            const int sp = it / nq;
            s = sp / np;
            p = sp - s * np;
            row = static_cast<int64_t>(s) * n_post + n0 + p;
        }
        float e[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (!COMPACT || s != 0xFF) {
            const float *bs = basis_lds + s * nb;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (b0 + j >= B) break;
                const float *d = tile + ((b0 + j) * P + p) * nb;
                float x = d[0] * bs[0];
#pragma unroll
                for (int r = 1; r < kMaxBasis; ++r)
                    if (r < nb) x = x + d[r] * bs[r];
                e[j] = x;
            }
        }
        *reinterpret_cast<float4 *>(G + row * Bp + b0) = make_float4(e[0], e[1], e[2], e[3]);
    }
}

// Posts per workgroup of k_make_G: the dy tile holds at most 2048 floats.
static int make_G_posts(int B, int nb) {
    int P = 64;
    while (P > 1 && B * P * nb > 2048) P >>= 1;
    return P;
}

// Batch masks and "active in some batch entry" bitmaps of a dense z [B][n_cols] in the
// row pull's layout: slot plane n_slots - d holds column pre + n_pre * (d - 1) at bit
// pre (planes of pre_pad = round64(n_pre) bits); one thread per (plane, pre), one wave per
// 64-bit word.
__global__ void __launch_bounds__(kBlock)
    k_op_colmask(const float *__restrict__ z, int32_t B, int64_t n_cols, int32_t n_pre, int32_t n_slots,
                 int32_t pre_pad, uint32_t *__restrict__ cm, uint64_t *__restrict__ bits) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<int64_t>(n_slots) * pre_pad) return;  // whole waves (pre_pad % 64 == 0)
    const int32_t plane = static_cast<int32_t>(i / pre_pad);
    const int32_t pre = static_cast<int32_t>(i - static_cast<int64_t>(plane) * pre_pad);
    uint32_t m = 0u;
    if (pre < n_pre) {
        const int64_t c = pre + static_cast<int64_t>(n_pre) * (n_slots - 1 - plane);
        for (int b = 0; b < B; ++b)
            if (z[static_cast<int64_t>(b) * n_cols + c] > 0.0f) m |= 1u << b;
    }
    cm[i] = m;
    const uint64_t bal = __ballot(m != 0u);
    if ((threadIdx.x & (kWave - 1)) == 0) bits[i >> 6] = bal;
}

template <int LG>
__global__ void __launch_bounds__(kBlock) k_syn_bwd_cols(ColArgs a, ActDense act) {
    bwd_cols<LG, 2>(a, act);
}

// dW of the active columns (z[b][c] > 0) next to the grouped dz walk: a wave per 64
// consecutive columns finds each column's batch mask, then 16-lane sub-groups walk the
// column-grouped synapses of four active columns at a time and write each synapse's dW
// once, straight to reference order: the sum over the set batch entries b, ascending, of
// G[sid][post][b] times the input value (counts) or 1 (spikes).
struct SynDwArgs {
    int64_t n_cols;
    int32_t B, hm, lm, R, counts;  // G row of entry p: (p >> 24) * hm + (p & kLow24) * lm
    const float *z;  // [B][n_cols]
    const int4 *units;  // the table's work units (Table::dwu), one wave each
    int32_t n_units;
    const int32_t *col_ptr;
    const uint32_t *ps;
    const int32_t *order;
    const float *G;
    float *dw;  // reference order, zero-filled by the caller
};

// Workgroup bid of the pass: a wave per work unit -- up to 64 consecutive short columns (lane l
// tests column first + l), or one chunk of a long column, which the wave's four 16-lane
// sub-groups split in quarters, so a table of few long columns (the background's) still spreads
// over many waves.
__device__ inline void syn_dw_body(const SynDwArgs &a, int64_t bid) {
    const int lane = threadIdx.x % kWave;
    const int64_t ui = bid * (blockDim.x / kWave) + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    if (ui >= a.n_units) return;  // the whole wave leaves together
    const int4 un = a.units[ui];
    const int64_t c0 = un.x;
    const bool chunk = un.y == 1;  // one column: its [un.z, un.w) in four quarters
    const int64_t c = c0 + (chunk ? 0 : lane);
    // a chunk's quarters are held by lanes 0, 16, 32, 48, so the loop below gives one to
    // each sub-group; otherwise lane l holds column c0 + l
    const bool mine = chunk ? (lane % 16) == 0 : lane < un.y;
    uint32_t m = 0;
    if (mine)
        for (int b = 0; b < a.B; ++b) m |= (a.z[b * a.n_cols + c] > 0.0f ? 1u : 0u) << b;
    int32_t lo = 0, hi = 0;
    if (m) {
        lo = chunk ? un.z : a.col_ptr[c];
        hi = chunk ? un.w : a.col_ptr[c + 1];
        if (chunk) {   // quarter lane / 16 of the chunk
            const int32_t q = (hi - lo + 3) / 4, s4 = lane / 16;
            lo = min(hi, lo + s4 * q);
            hi = min(hi, lo + q);
        }
    }
    const int sub = lane / 16, sl = lane % 16;
    uint64_t live = __ballot(m != 0u);
    while (live) {
        uint64_t lv = live;
        int src = -1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int f = lv ? __ffsll(static_cast<unsigned long long>(lv)) - 1 : -1;
            if (i == sub) src = f;
            lv &= lv - 1;
        }
        live = lv;
        // every lane takes part in the shuffles; idle sub-groups are masked afterwards
        const int sl_src = src >= 0 ? src : 0;
        const uint32_t msrc = static_cast<uint32_t>(__shfl(static_cast<int>(m), sl_src, kWave));
        const int32_t clo = __shfl(lo, sl_src, kWave);
        const int32_t hsrc = __shfl(hi, sl_src, kWave);
        const uint32_t mm = src >= 0 ? msrc : 0u;
        const int32_t chi = src >= 0 ? hsrc : clo;
        const int64_t cc = chunk ? c0 : c0 + sl_src;
        for (int32_t k0 = clo; k0 < chi; k0 += 64) {
            float d[4];
            const float *gp[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int32_t k = min(k0 + 16 * u + sl, chi - 1);
                const uint32_t p = a.ps[k];
                gp[u] = a.G + (static_cast<int64_t>(p >> 24) * a.hm + static_cast<int64_t>(p & kLow24) * a.lm) * a.R;
                d[u] = 0.0f;
            }
            uint32_t mb = mm;
            while (mb) {
                const int b = __ffs(mb) - 1;
                mb &= mb - 1;
                const float mult = a.counts ? a.z[b * a.n_cols + cc] : 1.0f;
#pragma unroll
                for (int u = 0; u < 4; ++u) d[u] += a.counts ? gp[u][b] * mult : gp[u][b];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (k0 + 16 * u + sl < chi) a.dw[a.order[k0 + 16 * u + sl]] = d[u];
        }
    }
}


// dz over the same work units, for tables whose walk runs on few lanes or whose time a long
// column sets (the input tables).  A wave per unit.  A run of y columns gives each column
// L = 64 / (y rounded up to a power of 2) lanes, which sum every L-th synapse of the column and
// add their sums in a fixed butterfly order; lane 0 of the column's lanes writes dz.  A
// one-column unit (a whole column or one chunk of a long one) uses all 64 lanes the same way
// into partial[unit], and k_dz_chunks adds a column's units in order.  Each term is
// w * G[row][b], as the walks form it.
struct DzUnitArgs {
    int64_t n_cols;
    int32_t B, hm, lm, R;  // G row of entry p: (p >> 24) * hm + (p & kLow24) * lm, R floats
    const int4 *units;
    int32_t n_units;
    const int32_t *col_ptr;
    const uint32_t *ps;
    const float *w;       // column-grouped weights
    const float *G;
    float *dz;            // [B][n_cols]
    float *partial;       // [n_units][R]
};

template <int BP>
__device__ inline void dz_unit_body(const DzUnitArgs &a, int64_t bid) {
    const int lane = threadIdx.x % kWave;
    const int64_t ui = bid * (blockDim.x / kWave) + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    if (ui >= a.n_units) return;  // the whole wave leaves together
    const int4 un = a.units[ui];
    int sh = 0;
    while ((1 << sh) < un.y) ++sh;  // un.y <= 64: sh <= 6, the same in every lane
    const int L = kWave >> sh;
    const int j = lane / L, sl = lane % L;
    float acc[BP];
#pragma unroll
    for (int b = 0; b < BP; ++b) acc[b] = 0.0f;
    int32_t k = 0, k_end = 0;
    if (un.y == 1) {
        k = un.z + lane;
        k_end = un.w;
    } else if (j < un.y) {
        k = a.col_ptr[un.x + j] + sl;
        k_end = a.col_ptr[un.x + j + 1];
    }
    for (; k < k_end; k += L) {
        const uint32_t p = a.ps[k];
        const float wk = a.w[k];
        const float *g = a.G + (static_cast<int64_t>(p >> 24) * a.hm + static_cast<int64_t>(p & kLow24) * a.lm) * a.R;
#pragma unroll
        for (int b = 0; b < BP; ++b)
            if (b < a.B) acc[b] = acc[b] + wk * g[b];
    }
    for (int o = L / 2; o >= 1; o >>= 1)
#pragma unroll
        for (int b = 0; b < BP; ++b) acc[b] = acc[b] + __shfl_xor(acc[b], o, kWave);
    if (un.y == 1) {
        if (lane == 0)
#pragma unroll
            for (int b = 0; b < BP; ++b)
                if (b < a.B) a.partial[ui * a.R + b] = acc[b];
    } else if (sl == 0 && j < un.y) {
#pragma unroll
        for (int b = 0; b < BP; ++b)
            if (b < a.B) a.dz[static_cast<int64_t>(b) * a.n_cols + un.x + j] = acc[b];
    }
}

template <int BP>
__global__ void __launch_bounds__(kBlock) k_dz_units(DzUnitArgs a) { dz_unit_body<BP>(a, blockIdx.x); }

// dz of the one-column units' columns: thread per (column, b), the column's units in order.
__global__ void __launch_bounds__(kBlock)
    k_dz_chunks(const int4 *__restrict__ dzc, int32_t n_dzc, const float *__restrict__ partial, int32_t B, int32_t R,
                int64_t n_cols, float *__restrict__ dz) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<int64_t>(n_dzc) * B) return;
    const int4 d = dzc[i / B];
    const int b = static_cast<int>(i % B);
    float s = partial[static_cast<int64_t>(d.y) * R + b];
    for (int u = 1; u < d.z; ++u) s = s + partial[static_cast<int64_t>(d.y + u) * R + b];
    dz[static_cast<int64_t>(b) * n_cols + d.x] = s;
}

__global__ void __launch_bounds__(kBlock) k_syn_dw_units(SynDwArgs da) { syn_dw_body(da, blockIdx.x); }

// The grouped dz walk (the first walk_blocks workgroups) beside the weight-gradient pass of
// the active columns (the rest): both read G only, the walk is bound by its gathers' latency,
// and one launch overlaps them.
template <int LG>
__global__ void __launch_bounds__(kBlock) k_syn_bwd_gs(GsArgs a, ActDense act, int walk_blocks, SynDwArgs da) {
    __shared__ float stage[kBlock / kWave * kGsStage];
    if (static_cast<int>(blockIdx.x) < walk_blocks) bwd_groups<LG>(a, act, stage, blockIdx.x);
    else syn_dw_body(da, blockIdx.x - walk_blocks);
}

int sub_wave_for(const Table *t) {  // lanes per column: ~ the mean column length
    double avg = t->n_cols ? static_cast<double>(t->n_syn) / t->n_cols : 0.0;
    return avg <= 24.0 ? 16 : (avg <= 48.0 ? 32 : 64);
}

int grid_subwaves(int64_t items, int L) {
    int64_t per_block = kBlock / L;
    int64_t g = (items + per_block - 1) / per_block;
    return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(g, 32768)));
}

int batch_pad(int B) { return B <= 4 ? 4 : (B <= 8 ? 8 : (B <= 16 ? 16 : 32)); }

struct SynWs {
    uint32_t *cm;      // [n_slots * pre_pad] batch masks (deterministic forward)
    uint64_t *cbits;   // [n_slots * pre_pad / 64] activity bitmaps
    float *G;          // the custom gradient's projection
    float *partial;    // [n_dwu][padded B] the unit dz pass's one-column sums
};

// with_G: the backward's projection G too (the forward does not use it)
static SynWs carve_syn(void *ws, const Table *t, int32_t B, size_t *bytes, bool with_G = true) {
    Carver cv(ws, SIZE_MAX);
    SynWs w{};
    const int64_t pre_pad = (static_cast<int64_t>(t->n_pre) + 63) / 64 * 64;
    w.cm = cv.take<uint32_t>(static_cast<size_t>(t->n_slots) * pre_pad);
    w.cbits = cv.take<uint64_t>(static_cast<size_t>(t->n_slots) * pre_pad / 64);
    // G: a row per (type, post), or per (post, own type) with the table's compact rows
    const int rows = t->og.rows ? t->og.rows : t->n_types;
    if (with_G) {
        w.G = cv.take<float>(static_cast<size_t>(t->n_post) * rows * batch_pad(B));
        w.partial = cv.take<float>(std::max<size_t>(static_cast<size_t>(t->n_dwu) * batch_pad(B), 1));
    }
    if (bytes) *bytes = cv.off;
    return w;
}

// Whether the op forward pulls (deterministic mode, or event mode on a table with long
// columns: each active input would cost an atomic per synapse of its column and batch entry,
// and with the background's Poisson counts ~2.4 of them land on each (b, post, receptor) per
// call, 67 against 24 us pulled at B = 5), and whether that pull uses the workspace (batch
// masks and activity bits built from z; Poisson counts take the dense-row pull, which needs
// none).  glif_syn_fwd validates the workspace with the same predicate syn_fwd dispatches on.
static bool fwd_pulls(const Table *t, int32_t mode) {
    return mode == GLIF_MODE_DETERMINISTIC || t->max_col_len > kUnitDzMinColLen;
}
static bool fwd_uses_ws(const Table *t, int32_t counts, int32_t mode) { return fwd_pulls(t, mode) && !counts; }

// The op forward on a carved workspace (every buffer it reads is written first by this call,
// so nothing in it has to start at zero).  Launches only; no allocation, no synchronisation.
static int syn_fwd(const Table *t, const float *z, int32_t B, int32_t counts, int32_t mode, float *I,
                   const SynWs &w, hipStream_t s) {
    const size_t lds = sizeof(float) * t->n_types * t->n_basis;
    const int64_t nI = static_cast<int64_t>(B) * t->n_post;
    // the pull's sums are the reference's, well within the event mode's bar
    if (fwd_pulls(t, mode)) {
        if (fwd_uses_ws(t, counts, mode)) {
            // the row pulls over batch masks and activity bitmaps built from z (one step, t = 0):
            // the resident chunk form where it fits, else the half-wave row pull (B * nb > 64,
            // or bitmaps beyond LDS), which reads each entry once for all batch entries
            const int32_t pre_pad = static_cast<int32_t>((static_cast<int64_t>(t->n_pre) + 63) / 64 * 64);
            PullArgs pa{};
            pa.t = 0;
            pa.T = 1;
            pa.N = t->n_post;
            pa.Np = pre_pad;
            pa.B = B;
            pa.D = t->n_slots;
            pa.nb = t->n_basis;
            pa.n_types = t->n_types;
            pa.os_r = 1;
            pa.os_b = static_cast<int64_t>(t->n_post) * t->n_basis;
            pa.os_n = t->n_basis;
            pa.W = pre_pad / 64;
            pa.Wl = 0;
            pa.rec_chunks = t->chunk_desc ? t->n_chunks : 0;
            pa.rec_cdesc = t->chunk_desc;
            pa.rec_row = t->row_ptr;
            pa.rec_pd = t->pd;
            pa.rec_pidx = t->chunk_desc ? t->pidx : nullptr;   // no chunk form without both
            pa.rec_sid = t->sid_row;
            pa.rec_w = t->w_row;
            pa.zmask = w.cm;
            pa.abits = w.cbits;
            pa.lbits = w.cbits;
            pa.basis = t->basis;
            pa.I = I;
            const int64_t n_mask = static_cast<int64_t>(t->n_slots) * pre_pad;
            hipLaunchKernelGGL(k_op_colmask, dim3(ceil_div(n_mask, kBlock)), dim3(kBlock), 0, s, z, B, t->n_cols,
                               t->n_pre, t->n_slots, pre_pad, w.cm, w.cbits);
            GLIF_HIP(hipGetLastError());
            // a wave per row on tables whose rows average 64 entries or more (the op's output is
            // post-major)
            launch_pull(pa, lds, s, t->n_syn >= static_cast<int64_t>(kWave) * t->n_post);
            GLIF_HIP(hipGetLastError());
            return GLIF_OK;
        }
        // Poisson counts scale the weights: a thread per (b, post) over the post's row
        dim3 grid(ceil_div(nI, kBlock));
        hipLaunchKernelGGL(k_syn_pull_dense, grid, dim3(kBlock), lds, s, z, B, t->n_cols, t->n_post,
                           t->n_pre, t->row_ptr, t->pd, t->sid_row, t->w_row, t->basis, t->n_types, t->n_basis, I);
        GLIF_HIP(hipGetLastError());
        return GLIF_OK;
    }
    int rc = launch_fill_u32(I, 0u, static_cast<size_t>(nI) * t->n_basis, s);
    if (rc) return rc;
    if (t->n_dwu > 0 && (ceil_div(t->n_cols, kWave) < kPushUnitsMaxScanWaves || t->max_col_len > kDwUnitEntries)) {
        const dim3 grid(static_cast<unsigned>(ceil_div(t->n_dwu, kBlock / kWave)));
        if (counts)
            hipLaunchKernelGGL(k_syn_push_units<true>, grid, dim3(kBlock), lds, s, z, B, t->n_cols, t->dwu, t->n_dwu,
                               t->col_ptr, t->ps, t->w_col, t->basis, t->n_types, t->n_basis, t->n_post, I);
        else
            hipLaunchKernelGGL(k_syn_push_units<false>, grid, dim3(kBlock), lds, s, z, B, t->n_cols, t->dwu, t->n_dwu,
                               t->col_ptr, t->ps, t->w_col, t->basis, t->n_types, t->n_basis, t->n_post, I);
        GLIF_HIP(hipGetLastError());
        return GLIF_OK;
    }
    const dim3 grid(static_cast<unsigned>(std::max<int64_t>(
        1, std::min<int64_t>(ceil_div(ceil_div(t->n_cols, kWave), kBlock / kWave), 32768))));
    if (counts)
        hipLaunchKernelGGL(k_syn_push_scan<true>, grid, dim3(kBlock), lds, s, z, B, t->n_cols, t->col_ptr, t->ps,
                           t->w_col, t->basis, t->n_types, t->n_basis, t->n_post, I);
    else
        hipLaunchKernelGGL(k_syn_push_scan<false>, grid, dim3(kBlock), lds, s, z, B, t->n_cols, t->col_ptr, t->ps,
                           t->w_col, t->basis, t->n_types, t->n_basis, t->n_post, I);
    GLIF_HIP(hipGetLastError());
    return GLIF_OK;
}

constexpr int kMaxDevices = 64;

}  // namespace glif

// Scratch of glif_syn_fwd_noalloc: a file-scope device array, so the entry point needs no
// allocation.  Every GPU the library runs on holds its own copy until the process ends.  In host
// code this name is only a handle for hipGetSymbolAddress, never a device address.
static __device__ __align__(256) char scratch[GLIF_NOALLOC_SCRATCH_BYTES];

namespace glif {

static std::mutex g_scratch_mu;
static void *g_scratch_dev[kMaxDevices];

// The device address of `scratch` on the current device, looked up once per device.
static int scratch_on_current_device(void **out) {
    int dev = -1;
    GLIF_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return fail(GLIF_EINVAL, "device index beyond the library's table");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        if (!p) return fail(GLIF_EHIP, "hipGetSymbolAddress(scratch) returned NULL");
        g_scratch_dev[dev] = p;
    }
    *out = g_scratch_dev[dev];
    return GLIF_OK;
}

}  // namespace glif

using namespace glif;

extern "C" {

size_t glif_syn_workspace(const glif_table *tt, int32_t B) {
    if (!tt || B <= 0) return 0;
    size_t bytes = 0;
    carve_syn(nullptr, reinterpret_cast<const Table *>(tt), B, &bytes);
    return bytes;
}

int glif_syn_fwd(const glif_table *tt, const float *z, int32_t B, int32_t counts, int32_t mode,
                 float *I, void *ws, size_t ws_bytes, void *stream) {
    if (!tt || !z || !I) return fail(GLIF_EINVAL, "NULL argument");
    if (B <= 0 || B > kMaxBatch) return fail(GLIF_EINVAL, "B must be in [1, 32]");
    if (mode != GLIF_MODE_EVENT && mode != GLIF_MODE_DETERMINISTIC) return fail(GLIF_EINVAL, "unknown mode");
    const Table *t = reinterpret_cast<const Table *>(tt);
    hipStream_t s = static_cast<hipStream_t>(stream);
    // the row pulls of spikes use the workspace (batch masks and activity bits); the event
    // push and the dense-row pull of counts need none
    if (fwd_uses_ws(t, counts, mode) && (!ws || ws_bytes < glif_syn_workspace(tt, B)))
        return fail(GLIF_ENOMEM, "workspace too small");
    ProfScope prof(kProfSynFwd, s);
    return syn_fwd(t, z, B, counts, mode, I, carve_syn(ws, t, B, nullptr), s);
}

int glif_syn_fwd_noalloc(const glif_table *tt, const float *z, int32_t B, int32_t counts, int32_t mode, float *I,
                         void *stream) {
    if (!tt || !z || !I) return fail(GLIF_EINVAL, "NULL argument");
    if (B <= 0 || B > kMaxBatch) return fail(GLIF_EINVAL, "B must be in [1, 32]");
    if (mode != GLIF_MODE_EVENT && mode != GLIF_MODE_DETERMINISTIC) return fail(GLIF_EINVAL, "unknown mode");
    const Table *t = reinterpret_cast<const Table *>(tt);
    size_t need = 0;
    carve_syn(nullptr, t, B, &need, false);
    if (need > GLIF_NOALLOC_SCRATCH_BYTES)
        return fail(GLIF_ENOMEM, "glif_syn_fwd_noalloc: this table's forward at batch " + std::to_string(B) +
                                     " needs " + std::to_string(need) + " bytes of scratch, above the " +
                                     std::to_string(GLIF_NOALLOC_SCRATCH_BYTES) +
                                     "-byte static array; call glif_syn_fwd with a workspace instead");
    void *p = nullptr;
    const int rc = scratch_on_current_device(&p);
    if (rc) return rc;
    return syn_fwd(t, z, B, counts, mode, I, carve_syn(p, t, B, nullptr, false), static_cast<hipStream_t>(stream));
}

int glif_syn_bwd(const glif_table *tt, const float *z, const float *dy, int32_t B, int32_t counts,
                 float *dz, float *dw, void *ws, size_t ws_bytes, void *stream) {
    if (!tt || !z || !dy) return fail(GLIF_EINVAL, "NULL argument");
    if (B <= 0 || B > kMaxBatch) return fail(GLIF_EINVAL, "B must be in [1, 32]");
    if (!dz && !dw) return GLIF_OK;
    const Table *t = reinterpret_cast<const Table *>(tt);
    size_t need = glif_syn_workspace(tt, B);
    if (!ws || ws_bytes < need) return fail(GLIF_ENOMEM, "workspace too small");
    const SynWs w = carve_syn(ws, t, B, nullptr);
    return syn_bwd_run(t, z, dy, B, counts, dz, dw, w.G, false, w.partial, static_cast<hipStream_t>(stream));
}

}  // extern "C"

namespace glif {

size_t syn_g_floats(const Table *t, int32_t B) {
    const int rows = t->og.rows ? t->og.rows : t->n_types;
    return static_cast<size_t>(t->n_post) * rows * batch_pad(B);
}

bool same_g_layout(const Table *a, const Table *b) {
    return a->og.rows == 0 && b->og.rows == 0 && a->n_post == b->n_post && a->n_types == b->n_types &&
           a->n_basis == b->n_basis &&
           std::memcmp(a->basis_host, b->basis_host, sizeof(float) * a->n_types * a->n_basis) == 0;
}

template <int BP>
static void launch_dz_units(const DzUnitArgs &da, hipStream_t s) {
    hipLaunchKernelGGL(k_dz_units<BP>, dim3(static_cast<unsigned>(ceil_div(da.n_units, kBlock / kWave))),
                       dim3(kBlock), 0, s, da);
}

int syn_bwd_run(const Table *t, const float *z, const float *dy, int32_t B, int32_t counts, float *dz, float *dw,
                float *G, bool g_ready, float *partial, hipStream_t s) {
    if (!dz && !dw) return GLIF_OK;
    const int Bp = batch_pad(B);
    // the table's own compact rows (post * rows + rank) when it has them, else type-major rows
    const CompactRows &oc = t->og;
    const bool cmp = oc.rows > 0;
    const int rows = cmp ? oc.rows : t->n_types;
    if (static_cast<int64_t>(rows) * t->n_post * Bp * 4 >= (int64_t(1) << 32))
        return fail(GLIF_ERANGE, "G rows per post * n_post * padded batch * 4 bytes must be < 4 GiB");
    ProfScope prof(kProfSynBwd, s);
    int rc;
    const bool grouped = (cmp ? oc.n_gs : t->n_gs) && (Bp == 8 || Bp == 16);
    // the work units instead of a walk whose time the longest column sets (the background
    // table's few, long columns) or that runs on few lanes (the LGN table's 17,400 columns):
    // for dz when the caller gives their partial sums room, and for dW, whose grouped-path
    // pass always runs over them
    const int64_t walk_lanes = (grouped ? t->n_groups : t->n_cols) * (Bp / 4);
    const bool prefer_units =
        t->n_dwu > 0 && (t->max_col_len > kUnitDzMinColLen || walk_lanes < kUnitDzMaxWalkLanes);
    const bool dz_units = dz && partial && prefer_units;
    const bool dw_units = dw && (grouped || prefer_units);
    // G, with the zero fill of dW beside it when the units' weight-gradient pass writes only
    // the active synapses
    const int gP = make_G_posts(B, t->n_basis);
    const int g_blocks = g_ready ? 0 : static_cast<int>(ceil_div(static_cast<int64_t>(t->n_post), gP));
    const int fill_blocks = dw_units && t->n_syn ? 256 : 0;
    const int64_t n_fill = fill_blocks ? t->n_syn : 0;
    const dim3 g_grid(g_blocks + fill_blocks);
    const size_t g_lds = sizeof(float) * (((t->n_types * t->n_basis + 3) & ~3) + static_cast<size_t>(B) * gP * t->n_basis);
    if (g_grid.x == 0) {
        // no posts and nothing to fill
    } else if (cmp) {
        hipLaunchKernelGGL(k_make_G<true>, g_grid, dim3(kBlock), g_lds, s, dy, B, t->n_post, Bp, t->basis,
                           t->n_types, t->n_basis, oc.gtype, rows, gP, G, g_blocks, dw, n_fill);
    } else {
        hipLaunchKernelGGL(k_make_G<false>, g_grid, dim3(kBlock), g_lds, s, dy, B, t->n_post, Bp, t->basis,
                           t->n_types, t->n_basis, nullptr, rows, gP, G, g_blocks, dw, n_fill);
    }
    GLIF_HIP(hipGetLastError());
    if (dz_units) {
        DzUnitArgs ua{t->n_cols, B, cmp ? 1 : t->n_post, cmp ? rows : 1, Bp, t->dwu, t->n_dwu, t->col_ptr,
                      cmp ? oc.ps : t->ps, t->w_col, G, dz, partial};
        switch (Bp) {
            case 4: launch_dz_units<4>(ua, s); break;
            case 8: launch_dz_units<8>(ua, s); break;
            case 16: launch_dz_units<16>(ua, s); break;
            default: launch_dz_units<32>(ua, s); break;
        }
        GLIF_HIP(hipGetLastError());
        if (t->n_dzc > 0) {
            hipLaunchKernelGGL(k_dz_chunks, dim3(static_cast<unsigned>(ceil_div(static_cast<int64_t>(t->n_dzc) * B, kBlock))),
                               dim3(kBlock), 0, s, t->dzc, t->n_dzc, partial, B, Bp, t->n_cols, dz);
            GLIF_HIP(hipGetLastError());
        }
        dz = nullptr;   // done; the passes below compute dW only
        if (!dw) return GLIF_OK;
    }
    if (grouped || (dw_units && !dz)) {
        // the grouped row-sliced walk for dz (when grouped and dz is still wanted) beside the
        // active columns' dW over the units (every active synapse's written once, in reference
        // order)
        ActDense act{z, dz, t->n_cols, counts};
        GsArgs ga{t->n_cols, (t->n_cols + kGsCols - 1) / kGsCols, B, cmp ? oc.gs_seg : t->gs_seg,
                  cmp ? oc.gs_pw : t->gs_pw, G};
        SynDwArgs da{t->n_cols, B, cmp ? 1 : t->n_post, cmp ? rows : 1, Bp, counts, z, t->dwu, t->n_dwu,
                     t->col_ptr, cmp ? oc.ps : t->ps, t->order, G, dw};
        const int LG = grouped ? Bp / 4 : 2;   // no walk blocks when not grouped
        const int walk_blocks = dz ? static_cast<int>(ceil_div(t->n_groups * LG, kBlock)) : 0;
        const int dw_blocks = dw ? static_cast<int>(ceil_div(t->n_dwu, kBlock / kWave)) : 0;
        const dim3 grid(walk_blocks + dw_blocks);
        if (grid.x == 0) return GLIF_OK;   // no columns
        if (LG == 2) hipLaunchKernelGGL(k_syn_bwd_gs<2>, grid, dim3(kBlock), 0, s, ga, act, walk_blocks, da);
        else hipLaunchKernelGGL(k_syn_bwd_gs<4>, grid, dim3(kBlock), 0, s, ga, act, walk_blocks, da);
        GLIF_HIP(hipGetLastError());
        return GLIF_OK;
    }
    if (dw_units) {
        // dW over the units (filled beside G), dz by the column walk below (the cell's
        // per-step backward gives no room for partial sums)
        SynDwArgs da{t->n_cols, B, cmp ? 1 : t->n_post, cmp ? rows : 1, Bp, counts, z, t->dwu, t->n_dwu,
                     t->col_ptr, cmp ? oc.ps : t->ps, t->order, G, dw};
        hipLaunchKernelGGL(k_syn_dw_units, dim3(static_cast<unsigned>(ceil_div(t->n_dwu, kBlock / kWave))),
                           dim3(kBlock), 0, s, da);
        GLIF_HIP(hipGetLastError());
        dw = nullptr;
    }
    // the type-phased column walk writes the active columns' synapses; the rest stay 0
    if (dw && (rc = launch_fill_u32(dw, 0u, static_cast<size_t>(t->n_syn), s))) return rc;
    ColArgs ca{t->n_cols, t->n_post, t->n_types, B, t->ph_ptr, cmp ? oc.ph_pw : t->ph_pw, G, dz ? 1 : 0, dw,
               t->ph_order, cmp ? 1 : 0};
    ActDense act{z, dz, t->n_cols, counts};
    const dim3 grid(ceil_div(t->n_cols * (Bp / 4), kBlock));
    switch (Bp / 4) {
        case 1: hipLaunchKernelGGL(k_syn_bwd_cols<1>, grid, dim3(kBlock), 0, s, ca, act); break;
        case 2: hipLaunchKernelGGL(k_syn_bwd_cols<2>, grid, dim3(kBlock), 0, s, ca, act); break;
        case 4: hipLaunchKernelGGL(k_syn_bwd_cols<4>, grid, dim3(kBlock), 0, s, ca, act); break;
        default: hipLaunchKernelGGL(k_syn_bwd_cols<8>, grid, dim3(kBlock), 0, s, ca, act); break;
    }
    GLIF_HIP(hipGetLastError());
    return GLIF_OK;
}

}  // namespace glif
