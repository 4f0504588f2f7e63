// Deterministic row pull of the synaptic currents (shared by the cell's T-step loop and
// the op-level forward): per post row, the active entries in ascending (column, synapse
// id) order from +0 -- the order TF's CPU UnsortedSegmentSum meets the events
// (models.py:141-169, 841-857).
#pragma once

#include <algorithm>
#include <mutex>
#include <vector>

#include "glif_internal.h"
#include "prof.h"
#include "syn_kernels.h"

namespace glif {

// ------------------------------------------------------ deterministic pull ----
// The currents of step t in the reference's order (models.py:141-169 and
// 841-857 summed as TF's CPU UnsortedSegmentSum meets the events): per (b, post, r)
// from +0, the recurrent events in ascending (column, synapse id) of the post row,
// the LGN events likewise, then I = rec + lgn (the background is added by the step
// kernel).  One half-wave (32 lanes) per post row: the lanes test 32 consecutive
// row entries at once (coalesced; one 4-byte batch mask per entry gives every
// batch's spike bit), a ballot finds the active ones, and the active entries are
// added one by one in row order into accumulator lanes, lane a = b * nb + r (+32g).
// Only the adds are sequential; at a few Hz ~2.5% of the entries are active.
struct PullArgs {
    int32_t t, T, N, Np, B, D, nb, n_types, n_lgn;
    int64_t os_r, os_b, os_n;  // output strides of receptor, batch entry, post
    int32_t W, Wl;             // 64-bit words of an abits / lbits row
    int32_t rec_chunks, lgn_chunks;  // row-aligned chunks of the two post-grouped tables
    const int4 *rec_cdesc, *lgn_cdesc;
    float *I2;  // [nb][B][N] LGN currents of the chunk form
    const uint32_t *zmask, *lmask;
    const uint64_t *abits, *lbits;
    const int32_t *rec_row;
    const uint32_t *rec_pd;  // pre | (delay - 1) << 24
    const uint32_t *rec_pidx, *lgn_pidx;  // activity-bitmap bit index of each entry
    const uint8_t *rec_sid;
    const float *rec_w;
    const int32_t *lgn_row;
    const uint32_t *lgn_pd;
    const uint8_t *lgn_sid;
    const float *lgn_w;
    const float *basis;
    float *I;  // [nb][B][N]
};

template <int G, bool REC>
__device__ inline void pull_row(const PullArgs &a, const float *basis_lds, int lane32, int half, int32_t j0,
                                int32_t j1, float (&acc)[G]) {
    constexpr int UC = 4;  // chunks of 32 entries whose loads are issued together
    const uint32_t *pd = REC ? a.rec_pd : a.lgn_pd;
    const uint8_t *sid = REC ? a.rec_sid : a.lgn_sid;
    const float *w = REC ? a.rec_w : a.lgn_w;
    const int BNB = a.B * a.nb;
    for (int32_t base = j0; base < j1; base += 32 * UC) {
        uint32_t e[UC], m[UC];
#pragma unroll
        for (int u = 0; u < UC; ++u) {
            const int32_t j = base + 32 * u + lane32;
            e[u] = j < j1 ? pd[j] : 0u;
        }
        // recurrent entries test their slot's activity bit first (64 columns per word, so the
        // words stay in the L1 / L2) and gather the 4-byte batch mask only where it is set
        uint64_t bw[UC];
#pragma unroll
        for (int u = 0; u < UC; ++u) {
            const int32_t j = base + 32 * u + lane32;
            bw[u] = 0u;
            if (REC && j < j1) {
                const int d = static_cast<int>(e[u] >> 24) + 1;
                bw[u] = a.abits[static_cast<int64_t>(a.t - d + a.D) * a.W + ((e[u] & kLow24) >> 6)];
            }
        }
#pragma unroll
        for (int u = 0; u < UC; ++u) {
            const int32_t j = base + 32 * u + lane32;
            m[u] = 0u;
            if (j < j1) {
                if (REC) {
                    const int d = static_cast<int>(e[u] >> 24) + 1;
                    if ((bw[u] >> (e[u] & 63u)) & 1u)
                        m[u] = a.zmask[static_cast<int64_t>(a.t - d + a.D) * a.Np + (e[u] & kLow24)];
                } else {
                    m[u] = a.lmask[static_cast<int64_t>(a.t) * a.n_lgn + (e[u] & kLow24)];
                }
            }
        }
        // the active lanes fetch their weight and type before the ordered adds
        float wj[UC];
        int sj[UC];
#pragma unroll
        for (int u = 0; u < UC; ++u) {
            const int32_t j = base + 32 * u + lane32;
            wj[u] = m[u] ? w[j] : 0.0f;
            sj[u] = m[u] ? sid[j] : 0;
        }
#pragma unroll
        for (int u = 0; u < UC; ++u) {
            uint32_t act = static_cast<uint32_t>(__ballot(m[u] != 0u) >> (32 * half));
            while (act) {
                const int src = __ffs(act) - 1 + 32 * half;
                act &= act - 1u;
                const uint32_t mm = static_cast<uint32_t>(__shfl(static_cast<int>(m[u]), src, kWave));
                const float wv = __shfl(wj[u], src, kWave);
                const int sv = __shfl(sj[u], src, kWave);
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const int ai = lane32 + 32 * g;
                    if (ai < BNB) {
                        const int b = ai / a.nb, r = ai - b * a.nb;
                        if ((mm >> b) & 1u) acc[g] = acc[g] + wv * basis_lds[sv * a.nb + r];
                    }
                }
            }
        }
    }
}

template <int G>
__global__ void __launch_bounds__(kBlock) k_pull(PullArgs a) {
    extern __shared__ float basis_lds[];
    load_basis_lds(basis_lds, a.basis, a.n_types * a.nb);
    const int64_t row = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) / 32;
    const int lane32 = threadIdx.x & 31, half = (threadIdx.x >> 5) & 1;
    // a half-wave past the last row runs the (empty) loops beside its partner half
    const bool live = row < a.N;
    const int32_t n = live ? static_cast<int32_t>(row) : 0;
    float ar[G], al[G];
#pragma unroll
    for (int g = 0; g < G; ++g) ar[g] = al[g] = 0.0f;
    pull_row<G, true>(a, basis_lds, lane32, half, live ? a.rec_row[n] : 0, live ? a.rec_row[n + 1] : 0, ar);
    // lgn_row null: the LGN currents come from elsewhere (the cell's LGN ring) and I
    // holds the recurrent sum alone
    const bool lgn = a.lgn_row != nullptr;
    if (lgn) pull_row<G, false>(a, basis_lds, lane32, half, live ? a.lgn_row[n] : 0, live ? a.lgn_row[n + 1] : 0, al);
    if (!live) return;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int ai = lane32 + 32 * g;
        if (ai < a.B * a.nb) {
            const int b = ai / a.nb, r = ai - b * a.nb;
            a.I[r * a.os_r + b * a.os_b + n * a.os_n] = lgn ? ar[g] + al[g] : ar[g];
        }
    }
}

// The row pull with a whole wave per post row, for B * nb > 32 accumulator slots: lane a (+64 g)
// holds the pair a = b * nb + r.  A hit's batch mask is then the same in every lane, read with
// readlane, so a slot holding none of its batch entries is skipped by a scalar branch and the
// slots that are visited add by a select on the lane's batch bit -- where the half-wave form's
// two rows per wave make every slot test divergent, and its exec-mask handling bounds it on the
// CU's scalar unit.  Each (b, r) sums its hits in entry order from +0, as the half-wave form.
template <int G, bool REC>
__device__ inline void pull_row_w(const PullArgs &a, const float *basis_lds, int lane, int32_t j0, int32_t j1,
                                  const uint32_t (&gmask)[G], const uint32_t (&bm)[G], const int (&rq)[G],
                                  float (&acc)[G]) {
    constexpr int UC = 4;  // chunks of 64 entries whose loads are issued together
    const uint32_t *pd = REC ? a.rec_pd : a.lgn_pd;
    const uint8_t *sid = REC ? a.rec_sid : a.lgn_sid;
    const float *w = REC ? a.rec_w : a.lgn_w;
    for (int32_t base = j0; base < j1; base += kWave * UC) {
        uint32_t e[UC], m[UC];
#pragma unroll
        for (int u = 0; u < UC; ++u) {
            const int32_t j = base + kWave * u + lane;
            e[u] = j < j1 ? pd[j] : 0u;
        }
        uint64_t bw[UC];
#pragma unroll
        for (int u = 0; u < UC; ++u) {
            const int32_t j = base + kWave * u + lane;
            bw[u] = 0u;
            if (REC && j < j1) {
                const int d = static_cast<int>(e[u] >> 24) + 1;
                bw[u] = a.abits[static_cast<int64_t>(a.t - d + a.D) * a.W + ((e[u] & kLow24) >> 6)];
            }
        }
#pragma unroll
        for (int u = 0; u < UC; ++u) {
            const int32_t j = base + kWave * u + lane;
            m[u] = 0u;
            if (j < j1) {
                if (REC) {
                    const int d = static_cast<int>(e[u] >> 24) + 1;
                    if ((bw[u] >> (e[u] & 63u)) & 1u)
                        m[u] = a.zmask[static_cast<int64_t>(a.t - d + a.D) * a.Np + (e[u] & kLow24)];
                } else {
                    m[u] = a.lmask[static_cast<int64_t>(a.t) * a.n_lgn + (e[u] & kLow24)];
                }
            }
        }
        float wj[UC];
        int sj[UC];
#pragma unroll
        for (int u = 0; u < UC; ++u) {
            const int32_t j = base + kWave * u + lane;
            wj[u] = m[u] ? w[j] : 0.0f;
            sj[u] = m[u] ? sid[j] : 0;
        }
#pragma unroll
        for (int u = 0; u < UC; ++u) {
            uint64_t act = __ballot(m[u] != 0u);
            while (act) {
                const int src = __builtin_ctzll(act);
                act &= act - 1ull;
                const uint32_t mm = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(m[u]), src));
                const float wv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wj[u]), src));
                const int sv = __builtin_amdgcn_readlane(sj[u], src);
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    if (mm & gmask[g]) {
                        const float nv = acc[g] + wv * basis_lds[sv * a.nb + rq[g]];
                        acc[g] = (mm & bm[g]) ? nv : acc[g];
                    }
                }
            }
        }
    }
}

// Rows per k_pull_w workgroup (a wave each); with a receptor-major output their sums leave
// through LDS together, the neighbouring posts of one (b, r) in one store run.
constexpr int kPullWaveRows = kBlock / kWave;

// Floats of k_pull_w's dynamic LDS: the basis, then the staged sums of the workgroup's rows.
static size_t pull_w_lds_floats(int n_types, int nb, int G) {
    return ((static_cast<size_t>(n_types) * nb + 3) & ~size_t(3)) + static_cast<size_t>(kPullWaveRows) * G * kWave;
}

template <int G>
__global__ void __launch_bounds__(kBlock) k_pull_w(PullArgs a) {
    extern __shared__ float smem[];
    float *basis_lds = smem;
    float *stage = smem + ((a.n_types * a.nb + 3) & ~3);   // [kPullWaveRows][G * 64]
    load_basis_lds(basis_lds, a.basis, a.n_types * a.nb);
    const int wv_i = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kPullWaveRows;
    const int64_t row = n0 + wv_i;
    // a wave past the last row runs no entries and still reaches the workgroup barrier below
    const bool live = row < a.N;
    const int32_t n = live ? static_cast<int32_t>(row) : 0;
    const int BNB = a.B * a.nb;
    // slot g: the batch entries its lanes hold (the same in every lane), this lane's batch bit
    // (none past B * nb, so the select never takes it) and basis column
    uint32_t gmask[G], bm[G];
    int rq[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int lo = kWave * g, hi = min(BNB, kWave * (g + 1)) - 1;
        gmask[g] = lo < BNB ? static_cast<uint32_t>(((uint64_t(2) << (hi / a.nb)) - 1u) & ~((uint64_t(1) << (lo / a.nb)) - 1u))
                            : 0u;
        const int ai = lane + kWave * g;
        bm[g] = ai < BNB ? 1u << (ai / a.nb) : 0u;
        rq[g] = ai < BNB ? ai - (ai / a.nb) * a.nb : 0;
    }
    float ar[G], al[G];
#pragma unroll
    for (int g = 0; g < G; ++g) ar[g] = al[g] = 0.0f;
    pull_row_w<G, true>(a, basis_lds, lane, live ? a.rec_row[n] : 0, live ? a.rec_row[n + 1] : 0, gmask, bm, rq,
                        ar);
    const bool lgn = a.lgn_row != nullptr;
    if (lgn)
        pull_row_w<G, false>(a, basis_lds, lane, live ? a.lgn_row[n] : 0, live ? a.lgn_row[n + 1] : 0, gmask, bm,
                             rq, al);
    if (a.os_n != 1) {
        // post-major output (the op's [B*N][nb]): each wave stores its row, a run of nb floats
        // per batch entry (staging it with the workgroup's other rows measured slower: the
        // waves then wait for the slowest row, 129 against 144 us at B = 20)
        if (!live) return;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int ai = lane + kWave * g;
            if (ai < BNB) {
                const int b = ai / a.nb, r = ai - b * a.nb;
                a.I[r * a.os_r + b * a.os_b + n * a.os_n] = lgn ? ar[g] + al[g] : ar[g];
            }
        }
        return;
    }
    // receptor-major output (the cell's [nb][B][N]): the workgroup's rows leave together, the
    // neighbouring posts of one (b, r) in one store run (os_n is the same for the whole grid,
    // so every wave reaches the barrier)
#pragma unroll
    for (int g = 0; g < G; ++g) stage[wv_i * (G * kWave) + lane + kWave * g] = lgn ? ar[g] + al[g] : ar[g];
    __syncthreads();
    const int rows = static_cast<int>(min<int64_t>(kPullWaveRows, a.N - n0));
    for (int v = threadIdx.x; v < BNB * kPullWaveRows; v += blockDim.x) {
        const int pair = v / kPullWaveRows, q = v - pair * kPullWaveRows;
        if (q >= rows) continue;
        const int b = pair / a.nb, r = pair - b * a.nb;
        a.I[r * a.os_r + b * a.os_b + (n0 + q) * a.os_n] = stage[q * (G * kWave) + pair];
    }
}

// Resident chunk form, used when the step's activity bitmaps fit in LDS: bits_lds holds
// the "active in some batch entry" bits of steps t-D..t-1 (D planes of W 64-bit words,
// slot t-d at plane D-d) and of the LGN inputs of step t.  A wave takes row-aligned
// chunks of a table (at most kChunkEntries entries over at most kChunkRows rows, or one
// longer row): it loads the chunk's entries flat (8 coalesced loads per lane), tests
// them against the bitmaps, fetches batch mask, weight and type of the active ones in
// one round, then walks the chunk's rows in order, adding each row's active entries in
// ascending entry order into accumulator lanes a = b * nb + r (+64 g) with wave-uniform
// lane reads.  Recurrent rows write I, LGN rows write I2 (the step adds I + I2): the
// sums and their order are those of k_pull.
constexpr int kPullBlock = 512;

__device__ inline int rdlane(int v, int l) { return __builtin_amdgcn_readlane(v, l); }

// 4-byte load at a 32-bit byte offset (lets the compiler use the scalar-base form)
__device__ inline uint32_t ld_off(const uint32_t *p, uint32_t byte_off) {
    return *reinterpret_cast<const uint32_t *>(reinterpret_cast<const char *>(p) + byte_off);
}

// The loads of one chunk given its descriptor d = {first row, rows, first entry, end
// entry}: the row pointers of its rows (lane l: row l, l <= rows) and its first
// kChunkEntries entries.
template <int U>
__device__ inline void chunk_fetch(const int4 d, const int32_t *row_ptr, const uint32_t *pd, int lane, int32_t &rp,
                                   uint32_t (&e)[U]) {
    rp = lane <= d.y ? row_ptr[static_cast<uint32_t>(d.x + lane)] : 0;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int32_t j = d.z + u * kWave + lane;
        e[u] = j < d.w ? pd[static_cast<uint32_t>(j)] : 0u;
    }
}

// Descriptors of a wave's chunks wave0 + (k0 + l) * waves, one per lane l (zero past the
// end), so that the walk reads them with lane reads instead of waiting on memory.
__device__ inline int4 chunk_descs(const PullArgs &a, int32_t wave0, int32_t waves, int32_t k0, int lane) {
    const int64_t cx = wave0 + static_cast<int64_t>(k0 + lane) * waves;
    if (cx >= static_cast<int64_t>(a.rec_chunks) + a.lgn_chunks) return make_int4(0, 0, 0, 0);
    return cx < a.rec_chunks ? a.rec_cdesc[cx] : a.lgn_cdesc[cx - a.rec_chunks];
}

__device__ inline int4 desc_at(const int4 dl, int l) {
    return make_int4(rdlane(dl.x, l), rdlane(dl.y, l), rdlane(dl.z, l), rdlane(dl.w, l));
}

template <int G>
struct PullLanes {   // this lane's accumulator slots: (b, r) of a = lane + 64 g
    int bq[G], rq[G];
    bool ok[G];
};

template <int G>
__device__ inline void flush_row(const PullLanes<G> &pl, const PullArgs &a, float *out, int64_t n,
                                 float (&acc)[G]) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
        if (pl.ok[g]) out[pl.rq[g] * a.os_r + pl.bq[g] * a.os_b + n * a.os_n] = acc[g];
        acc[g] = 0.0f;
    }
}

// One chunk of the recurrent (REC) or LGN table: rounds of up to kChunkEntries entries
// (one round unless the chunk is a single longer row).  Per round: the activity test
// of every entry against the LDS bitmaps (branch-free, the reads issued together), batch
// mask / weight / type of the active entries, then the hits in entry order, each added
// to the row it falls in; rows are written as the positions pass their ends.
template <int G, bool REC, int U>
__device__ inline void pull_chunk(const PullArgs &a, const float *basis_lds, const uint32_t *bits_lds,
                                  const PullLanes<G> &pl, int lane, int4 dsc, int32_t rp, uint32_t (&e)[U]) {
    const uint32_t *pidx = REC ? a.rec_pidx : a.lgn_pidx;
    const float *w = REC ? a.rec_w : a.lgn_w;
    const uint8_t *sid = REC ? a.rec_sid : a.lgn_sid;
    float *out = REC ? a.I : a.I2;
    // bit offset of the table's planes in LDS: the recurrent planes first, then the LGN one
    const uint32_t base = REC ? 0u : static_cast<uint32_t>(a.D) * static_cast<uint32_t>(a.Np);
    const int32_t r_beg = dsc.x, nr = dsc.y, j_end = dsc.w;
    int row = 0;
    float acc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g] = 0.0f;
    for (int32_t jb = dsc.z; jb < j_end; jb += kChunkEntries) {
        if (jb != dsc.z) {  // later rounds of a single long row
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int32_t j = jb + u * kWave + lane;
                e[u] = j < j_end ? pidx[static_cast<uint32_t>(j)] : 0u;
            }
        }
        // entries past the end are 0: their word is in range
        uint32_t bw[U];
#pragma unroll
        for (int u = 0; u < U; ++u) bw[u] = bits_lds[(base + e[u]) >> 5];
        uint32_t m[U];
        float wj[U];
        int sj[U];
        uint64_t hm[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int32_t j = jb + u * kWave + lane;
            const bool h = j < j_end && ((bw[u] >> ((base + e[u]) & 31u)) & 1u);
            m[u] = 0u;
            wj[u] = 0.0f;
            sj[u] = 0;
            if (h) {
                // zmask rows are Np wide, so slot t - d of pre is at t * Np + pidx
                m[u] = REC ? ld_off(a.zmask, (static_cast<uint32_t>(a.t) * static_cast<uint32_t>(a.Np) + e[u]) * 4u)
                           : ld_off(a.lmask, (static_cast<uint32_t>(a.t) * static_cast<uint32_t>(a.n_lgn) + e[u]) * 4u);
                wj[u] = __uint_as_float(ld_off(reinterpret_cast<const uint32_t *>(w), static_cast<uint32_t>(j) * 4u));
                sj[u] = sid[static_cast<uint32_t>(j)];
            }
            hm[u] = __ballot(h);
        }
        const int32_t je = jb + kChunkEntries < j_end ? jb + kChunkEntries : j_end;
        int32_t rend = rdlane(rp, row + 1) - jb;  // row < nr: this round has entries
#pragma unroll
        for (int u = 0; u < U; ++u) {
            uint64_t mu = hm[u];
            while (mu) {
                const int src = __builtin_ctzll(mu);
                mu &= mu - 1ull;
                const int32_t pos = u * kWave + src;
                while (pos >= rend) {
                    flush_row(pl, a, out, r_beg + row, acc);
                    ++row;
                    rend = rdlane(rp, row + 1) - jb;
                }
                const uint32_t mm = static_cast<uint32_t>(rdlane(static_cast<int>(m[u]), src));
                const float wv = __int_as_float(rdlane(__float_as_int(wj[u]), src));
                const int sv = rdlane(sj[u], src);
#pragma unroll
                for (int g = 0; g < G; ++g)
                    if (pl.ok[g] && ((mm >> pl.bq[g]) & 1u)) acc[g] = acc[g] + wv * basis_lds[sv * a.nb + pl.rq[g]];
            }
        }
        // rows that end within this round
        while (row < nr) {
            if (rdlane(rp, row + 1) > je) break;  // the row goes on in the next round
            flush_row(pl, a, out, r_beg + row, acc);
            ++row;
        }
    }
    // rows without entries at the chunk's end (or a chunk of empty rows)
    for (; row < nr; ++row) flush_row(pl, a, out, r_beg + row, acc);
}

// Copy n 64-bit words global -> LDS with 8 loads in flight per thread.
__device__ inline void copy_to_lds(uint64_t *dst, const uint64_t *src, int n) {
    for (int base = 0; base < n; base += 8 * static_cast<int>(blockDim.x)) {
        uint64_t v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int i = base + k * static_cast<int>(blockDim.x) + static_cast<int>(threadIdx.x);
            v[k] = i < n ? src[i] : 0ull;
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int i = base + k * static_cast<int>(blockDim.x) + static_cast<int>(threadIdx.x);
            if (i < n) dst[i] = v[k];
        }
    }
}

// The chunk walk of workgroup bid of nblocks (the whole grid of k_pull_chunks, or the
// first block range of a launch that runs other work beside it).
template <int G>
__device__ inline void pull_chunks_body(const PullArgs &a, int32_t bid, int32_t nblocks) {
    extern __shared__ float lds_f[];
    float *basis_lds = lds_f;
    const int nbasis = a.n_types * a.nb;
    uint32_t *bits_lds = reinterpret_cast<uint32_t *>(lds_f + ((nbasis + 1) & ~1));
    for (int i = threadIdx.x; i < nbasis; i += blockDim.x) basis_lds[i] = a.basis[i];
    // planes of steps t-D .. t-1 are slots t .. t+D-1 of abits, contiguous; then the
    // LGN plane of step t
    uint64_t *bits64 = reinterpret_cast<uint64_t *>(bits_lds);
    copy_to_lds(bits64, a.abits + static_cast<int64_t>(a.t) * a.W, a.D * a.W);
    copy_to_lds(bits64 + a.D * a.W, a.lbits + static_cast<int64_t>(a.t) * a.Wl, a.Wl);
    __syncthreads();
    constexpr int U = kChunkEntries / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    PullLanes<G> pl;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int ai = lane + kWave * g;
        pl.ok[g] = ai < a.B * a.nb;
        pl.bq[g] = pl.ok[g] ? ai / a.nb : 0;
        pl.rq[g] = pl.ok[g] ? ai - pl.bq[g] * a.nb : 0;
    }
    // wave index made explicitly uniform: chunk indices, descriptors and loop bounds live
    // in scalar registers
    const int32_t waves = static_cast<int32_t>(nblocks * (blockDim.x / kWave));
    const int32_t wave0 = static_cast<int32_t>(bid * (blockDim.x / kWave)) +
                          __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
    const int32_t n_all = a.rec_chunks + a.lgn_chunks;

    int32_t c = wave0;
    int32_t k0 = 0;  // iteration of lane 0's descriptor
    int4 dl = chunk_descs(a, wave0, waves, 0, lane);
    int4 dsc = desc_at(dl, 0);
    int32_t rp = 0;
    uint32_t e[U];
#pragma unroll
    for (int u = 0; u < U; ++u) e[u] = 0u;
    if (c < n_all) {
        if (c < a.rec_chunks) chunk_fetch<U>(dsc, a.rec_row, a.rec_pidx, lane, rp, e);
        else chunk_fetch<U>(dsc, a.lgn_row, a.lgn_pidx, lane, rp, e);
    }
    for (int32_t k = 0; c < n_all; c += waves, ++k) {
        // the next chunk's loads go out before this chunk is processed
        const int32_t cn = c + waves;
        if (k + 1 - k0 == kWave) {
            k0 += kWave;
            dl = chunk_descs(a, wave0, waves, k0, lane);
        }
        const int4 dn = desc_at(dl, k + 1 - k0);
        int32_t rpn = 0;
        uint32_t en[U];
#pragma unroll
        for (int u = 0; u < U; ++u) en[u] = 0u;
        if (cn < n_all) {
            if (cn < a.rec_chunks) chunk_fetch<U>(dn, a.rec_row, a.rec_pidx, lane, rpn, en);
            else chunk_fetch<U>(dn, a.lgn_row, a.lgn_pidx, lane, rpn, en);
        }
        if (c < a.rec_chunks) pull_chunk<G, true, U>(a, basis_lds, bits_lds, pl, lane, dsc, rp, e);
        else pull_chunk<G, false, U>(a, basis_lds, bits_lds, pl, lane, dsc, rp, e);
        dsc = dn;
        rp = rpn;
#pragma unroll
        for (int u = 0; u < U; ++u) e[u] = en[u];
    }
}

template <int G, int BLOCK>
__global__ void __launch_bounds__(BLOCK) k_pull_chunks(PullArgs a) {
    pull_chunks_body<G>(a, blockIdx.x, gridDim.x);
}

static size_t chunk_lds_bytes(const PullArgs &pa) {
    return sizeof(float) * ((pa.n_types * pa.nb + 1) & ~1) + 8 * (static_cast<size_t>(pa.D) * pa.W + pa.Wl);
}

struct DevShape {
    int n_cu = 0;
    size_t lds_per_block = 0, lds_per_cu = 0;
};

// Launch-shape caches below are shared by every host thread: their lookups and fills hold
// this lock (a fill queries the runtime once per device and key).
static std::mutex &shape_mutex() {
    static std::mutex mu;
    return mu;
}

static const DevShape &dev_shape() {
    static DevShape d[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    std::lock_guard<std::mutex> lock(shape_mutex());
    if (d[dev].n_cu == 0) {
        int v = 0;
        DevShape x;
        x.n_cu = hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess ? v : 1;
        x.lds_per_block = hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess
                              ? static_cast<size_t>(v) : 65536;
        x.lds_per_cu = hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) ==
                               hipSuccess ? static_cast<size_t>(v) : x.lds_per_block;
        d[dev] = x;
    }
    return d[dev];
}

// whether the resident chunk form runs (bitmaps fit in LDS, accumulators in 4 lane slots)
static bool pull_chunked(const PullArgs &pa) {
    const DevShape &ds = dev_shape();
    const size_t lb = chunk_lds_bytes(pa);
    // 32-bit offsets of the batch-mask gathers
    const bool fits = static_cast<int64_t>(pa.T + pa.D) * pa.Np < (int64_t(1) << 32) &&
                      static_cast<int64_t>(pa.T) * pa.n_lgn < (int64_t(1) << 32);
    // one accumulator slot per lane (B * nb <= 64): with more, every hit costs several slot
    // passes and the half-wave row pull (two rows per wave) was measured faster
    return fits && pa.rec_pidx && (pa.lgn_chunks == 0 || pa.lgn_pidx) && lb <= ds.lds_per_block &&
           pa.B * pa.nb <= kWave;
}

// Resident workgroups per CU of kernel fn with workgroups of `block` lanes and lb bytes of
// dynamic LDS on the current device (at least 1).
static int resident_per_cu(const void *fn, int block, size_t lb) {
    struct Entry {
        int dev;
        const void *fn;
        int block;
        size_t lb;
        int per_cu;
    };
    static std::vector<Entry> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    std::lock_guard<std::mutex> lock(shape_mutex());
    for (const Entry &e : cache)
        if (e.dev == dev && e.fn == fn && e.block == block && e.lb == lb) return e.per_cu;
    if (lb > 65536) (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lb));
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, block, lb) != hipSuccess || per_cu < 1) per_cu = 1;
    cache.push_back(Entry{dev, fn, block, lb, per_cu});
    return per_cu;
}

// The resident chunk kernel, when pull_chunked(pa); false (nothing launched) otherwise.
// Workgroups of kPullBlock lanes, as many as stay resident; when the bitmaps leave room
// for only one workgroup per CU, workgroups of 2 * kPullBlock lanes instead.
static bool launch_pull_chunks(const PullArgs &pa, hipStream_t s) {
    if (!pull_chunked(pa)) return false;
    const DevShape &ds = dev_shape();
    const size_t lb = chunk_lds_bytes(pa);
    // pull_chunked: B * nb <= 64, one accumulator slot per lane (G = 1)
    const bool wide = ds.lds_per_cu / lb < 2;
    const void *fn = wide ? reinterpret_cast<const void *>(&k_pull_chunks<1, 2 * kPullBlock>)
                          : reinterpret_cast<const void *>(&k_pull_chunks<1, kPullBlock>);
    const int per_cu = resident_per_cu(fn, wide ? 2 * kPullBlock : kPullBlock, lb);
    const dim3 grid(ds.n_cu * per_cu);
    if (wide) GLIF_PROF_LAUNCH((k_pull_chunks<1, 2 * kPullBlock>), grid, dim3(2 * kPullBlock), lb, s, pa);
    else GLIF_PROF_LAUNCH((k_pull_chunks<1, kPullBlock>), grid, dim3(kPullBlock), lb, s, pa);
    return true;
}

// wave_rows: a whole wave per post row when B * nb > 32 (k_pull_w), measured faster for the
// cell (config 4's pull at B = 32: 270 -> 216 us per tick at 5 Hz) and for the op on tables whose
// rows average at least 64 entries (the recurrent table at B = 20 and 32: 175 -> 128 and
// 269 -> 189 us); otherwise two rows per wave, so that short rows (the LGN table's 40 entries)
// do not leave most of a 64-lane chunk idle.
static void launch_pull(const PullArgs &pa, size_t lds, hipStream_t s, bool wave_rows = false) {
    if (launch_pull_chunks(pa, s)) return;
    const int BNB = pa.B * pa.nb;   // <= 32 * kMaxBasis = 256 (checked at the entry points)
    if (BNB <= 32 || !wave_rows) {
        const int G = (BNB + 31) / 32;
        const dim3 grid(ceil_div(static_cast<int64_t>(pa.N) * 32, kBlock));
        switch (G <= 1 ? 1 : G <= 2 ? 2 : G <= 4 ? 4 : 8) {
            case 1: GLIF_PROF_LAUNCH(k_pull<1>, grid, dim3(kBlock), lds, s, pa); break;
            case 2: GLIF_PROF_LAUNCH(k_pull<2>, grid, dim3(kBlock), lds, s, pa); break;
            case 4: GLIF_PROF_LAUNCH(k_pull<4>, grid, dim3(kBlock), lds, s, pa); break;
            default: GLIF_PROF_LAUNCH(k_pull<8>, grid, dim3(kBlock), lds, s, pa); break;
        }
        return;
    }
    const dim3 grid(ceil_div(static_cast<int64_t>(pa.N), kPullWaveRows));
    const int G = BNB <= 64 ? 1 : BNB <= 128 ? 2 : 4;
    const size_t lw = sizeof(float) * pull_w_lds_floats(pa.n_types, pa.nb, G);
    switch (G) {
        case 1: GLIF_PROF_LAUNCH(k_pull_w<1>, grid, dim3(kBlock), lw, s, pa); break;
        case 2: GLIF_PROF_LAUNCH(k_pull_w<2>, grid, dim3(kBlock), lw, s, pa); break;
        default: GLIF_PROF_LAUNCH(k_pull_w<4>, grid, dim3(kBlock), lw, s, pa); break;
    }
}

}  // namespace glif
