// The GLIF_3 cell over T steps (V1Column.call, models.py:1059-1135) and its BPTT.
//
// Forward, per step t (one stream, no host round trip):
//   LGN (B <= 8; event mode from B = 3 and without per-type slots): k_lgn_rows computes
//                 the LGN currents of 64 ticks at a time, per post row in the reference's
//                 order, into a ring of current slots ahead of the ticks that read them
//                 (otherwise the LGN events are pushed or pulled per tick as below);
//   event mode:   k_push(t)   the spike words of steps t-1..t-D (set bits = columns of
//                             the recurrent table), and without the LGN ring the step's
//                             LGN (column, batch-mask) list, are streamed through the
//                             column-grouped tables and added into I with fp32 atomics;
//                 k_step(t)   background pull, GLIF_3 update, spike bits (wave
//                             ballots); I is re-zeroed after reading (not with the
//                             LGN ring, which the next LGN segment rewrites).
//   deterministic: the row pull (pull_kernels.h) sums rec (and without the LGN ring,
//                 LGN) per post row in the reference's accumulation order and k_step
//                 adds the LGN and background currents and does the same update; with
//                 the resident chunk pull both run in one launch per tick (k_pull_step:
//                 the pull of t beside the step of t, whose R takes the currents of t - 1).
// Backward, in windows of Wwin reverse ticks t0, t0-1, .. (lagged adjoint, k_adj):
//   k_adj         per tick t: gz_t -> gV_t -> gP_{t-1} -> gR_{t-2} -> G_{t-2}
//   k_bwd_rec_gs_dw  dz of the window's steps t0-2, t0-3, .. over the recurrent columns
//                 of delays <= 2 Wwin - 3, one pass over the grouped row-sliced table
//                 (16-float G rows), with the dW of the window's active columns behind
//                 it; the other columns' dz run in the next window's adjoint launch
//                 (k_adj_dw); other row lengths: k_bwd_rec, dz and dW in one type-phased pass
//   k_bwd_in      dW of the LGN / background events of the window's steps
// A window is legal because dz_s depends only on dz_{>= s+3}: a spike reaches the
// rise current one step later, the PSC the next, the voltage the one after.
#include <algorithm>
#include <cstring>
#include <vector>

#include "compact.h"
#include "glif_internal.h"
#include "prof.h"
#include "pull_kernels.h"
#include "syn_kernels.h"

namespace glif {

// ------------------------------------------------------------------ state ----
constexpr int kVlossBlocks = 1024;  // blocks of the voltage-penalty reduction
struct CellWs {
    float *I;           // [2][nb][B][N]   pushed rec + LGN currents (event mode), or
                        // [2][g_rows][B][N] type sums with per-type slots
    float *R, *P;       // [nb][B][N]   psc_rise, psc (receptor-major copies of the state)
    float *A;           // [2][B][N]    asc
    uint64_t *zbits;    // [(T + D)][B][W]   slot t + D holds z_t
    uint64_t *refbits;  // [T][B][W]         r_t > 0
    uint32_t *zmask;    // [(T + D)][Np]     bit b: z_t[b][n] (slot t + D), deterministic pull
    uint32_t *lmask;    // [T][n_lgn]        bit b: LGN input x_t[b][pre] > 0
    uint64_t *abits;    // [(T + D)][W]      bit n: z_t[b][n] for some b (slot t + D)
    uint64_t *lbits;    // [T][Wl]           bit pre: x_t[b][pre] > 0 for some b
    float *I2;          // [2][nb][B][N]   LGN currents (deterministic chunk pull)
    float *IL;          // [kLgnRing][nb][B][N]  LGN currents computed ahead of the loop (B <= 8):
                        // the event push adds onto them, the deterministic step adds them
    uint64_t *lgnT;     // [ceil(T / 64)][n_lgn][B]  LGN tick masks (bit k: tick 64 seg + k)
    float *vsave;       // [T][B][N]
    int64_t *lgn_off;   // [T + 1]           per-step LGN (column, batch-mask) lists
    int32_t *lgn_pre;   // [T * n_lgn]
    uint32_t *lgn_mask;
    int64_t *lw_off;    // [n_win + 1]       per-backward-window LGN lists
    int32_t *lw_pre;
    uint32_t *lw_mask;
    int64_t *kw_off;    // [n_win + 1]       per-backward-window background lists
    int32_t *kw_pre;
    uint32_t *kw_mask;
    uint8_t *bkg_cnt;   // [T][B][n_bkg]
    void *scratch;
    float *dZ;          // [ring][B][D * N]
    float *stage;       // from dZ on: staging of the gradient reorderings (after the walks)
    float *G;           // [2][n_types][N][R], or [2][N][g_rows][R] with compact rows
                        // (windows alternate between the two)
    float *gV;          // [B][N]
    float *gP, *gR;     // [nb][B][N]
    float *vloss_part;  // [kVlossBlocks] partial sums of the voltage penalty
    float *dw_rec;      // column-grouped order with the grouped walk, else type-phased
    float *dw_lgn, *dw_bkg;  // column-grouped order
};

// ------------------------------------------------- LGN currents ahead of the loop ----
// The LGN inputs of a rollout are known before its first tick, so their currents are
// computed in segments of kLgnSeg ticks ahead of the T loop instead of being pushed with
// atomics (event mode) or pulled row by row inside it (deterministic mode).  Each
// segment's currents land in a ring of kLgnRing current slots [nb][B][N], which the
// event push then adds the recurrent events to, or which the deterministic step adds to
// the pulled recurrent currents.  The pass of segment s + 1 runs on the cell's side stream
// beside segment s's ticks: it is enqueued at tick 64 s after an event on the caller's
// stream (all launches before tick 64 s), and tick 64 (s + 1)'s launch waits for it.  Ring
// safety: it overwrites the slots of ticks 64 (s + 1) - 130 .. 64 s - 3, whose last reader
// (the step of that tick) ran in launch 64 s - 2 at the latest.
constexpr int kLgnSeg = 64;
constexpr int kLgnRing = 2 * kLgnSeg + 2;
constexpr int kLgnPosts = 8;     // posts (waves) per k_lgn_rows workgroup
constexpr int kLgnMaxBatch = 8;      // batch accumulators per lane of k_lgn_rows
constexpr int kLgnEventMinBatch = 3; // event mode computes LGN ahead from this batch size up

constexpr int kLgnAheadMinTicks = 16;   // shorter rollouts (a per-step call: T = 1) push or pull
                                        // the LGN events per tick: a segment pass costs as much
                                        // for one tick as for 64
// Whether this cell computes its LGN currents ahead of the loop at batch size B over T ticks.
static bool lgn_ahead(const Cell *c, int B, int T) {
    return B <= kLgnMaxBatch && T >= kLgnAheadMinTicks && c->lgn->n_cols > 0;
}

static void release_side(Cell *c) {
    if (!c->side) return;
    int cur = 0;
    const bool restore = hipGetDevice(&cur) == hipSuccess && cur != c->side_dev;
    if (restore) (void)hipSetDevice(c->side_dev);
    (void)hipStreamDestroy(c->side);
    for (hipEvent_t e : {c->ev_main, c->ev_seg[0], c->ev_seg[1]})
        if (e) (void)hipEventDestroy(e);
    if (restore) (void)hipSetDevice(cur);
    c->side = nullptr;
    c->ev_main = c->ev_seg[0] = c->ev_seg[1] = nullptr;
    c->side_dev = -1;
}

// The cell's side stream on the current device (default priority) and its events; false
// when they cannot be made (the LGN passes then run on the caller's stream).
static bool ensure_side(Cell *c) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return false;
    if (c->side && c->side_dev == dev) return true;
    release_side(c);
    if (hipStreamCreateWithFlags(&c->side, hipStreamNonBlocking) != hipSuccess) {
        c->side = nullptr;
        return false;
    }
    c->side_dev = dev;
    for (hipEvent_t *e : {&c->ev_main, &c->ev_seg[0], &c->ev_seg[1]})
        if (hipEventCreateWithFlags(e, hipEventDisableTiming) != hipSuccess) {
            *e = nullptr;
            release_side(c);
            return false;
        }
    return true;
}

// Backward window width (reverse ticks per table pass) and G row length.
static int win_width(int B) { return 3 * B <= 16 ? 3 : 1; }
static int n_windows(int T, int Wwin) { return T >= 3 ? (T - 2 + Wwin - 1) / Wwin : 0; }
static int ring_size(const Cell *c) { return c->D + 6; }

// Current slots per (b, n) of I: the receptors, or in event mode with per-type slots the
// compact rows when there are more of them.
static int i_slots(const Cell *c) { return std::max(c->nb, c->push_typed ? c->g_rows : 0); }

// The regions a backward reads of its forward (spike bits, saved voltages, input lists) come
// first, at offsets that depend on B, T and the network only; the two whose size depends on the
// G layout (glif_cell_set_g_layout) -- G and the pushed currents I -- come after them, so a
// backward run after a layout switch still finds its forward's data.
static CellWs carve_cell(void *ws, const Cell *c, int32_t B, int32_t T, size_t *bytes) {
    Carver cv(ws, SIZE_MAX);
    CellWs w{};
    const int64_t BN = static_cast<int64_t>(B) * c->N;
    const int64_t nl = c->lgn->n_cols, nk = c->bkg->n_cols;
    w.R = cv.take<float>(BN * c->nb);
    w.P = cv.take<float>(BN * c->nb);
    w.A = cv.take<float>(BN * 2);
    w.zbits = cv.take<uint64_t>(static_cast<size_t>(T + c->D) * B * c->W);
    w.refbits = cv.take<uint64_t>(static_cast<size_t>(T) * B * c->W);
    w.zmask = cv.take<uint32_t>(static_cast<size_t>(T + c->D) * c->Np);
    w.lmask = cv.take<uint32_t>(static_cast<size_t>(T) * nl);
    w.abits = cv.take<uint64_t>(static_cast<size_t>(T + c->D) * c->W);
    w.lbits = cv.take<uint64_t>(static_cast<size_t>(T) * ((nl + 63) / 64));
    w.I2 = cv.take<float>(2 * BN * c->nb);  // deterministic pull beside the step: two halves
    if (lgn_ahead(c, B, T)) {
        w.IL = cv.take<float>(static_cast<size_t>(kLgnRing) * BN * c->nb);
        w.lgnT = cv.take<uint64_t>(static_cast<size_t>((T + kLgnSeg - 1) / kLgnSeg) * nl * B);
    }
    w.vsave = cv.take<float>(static_cast<size_t>(T) * BN);
    w.lgn_off = cv.take<int64_t>(T + 1);
    w.lgn_pre = cv.take<int32_t>(static_cast<size_t>(T) * nl);
    w.lgn_mask = cv.take<uint32_t>(static_cast<size_t>(T) * nl);
    const int Wwin = win_width(B), nwin = std::max(n_windows(T, Wwin), 1);
    w.lw_off = cv.take<int64_t>(nwin + 1);
    w.lw_pre = cv.take<int32_t>(static_cast<size_t>(nwin) * nl);
    w.lw_mask = cv.take<uint32_t>(static_cast<size_t>(nwin) * nl);
    w.kw_off = cv.take<int64_t>(nwin + 1);
    w.kw_pre = cv.take<int32_t>(static_cast<size_t>(nwin) * nk);
    w.kw_mask = cv.take<uint32_t>(static_cast<size_t>(nwin) * nk);
    w.bkg_cnt = cv.take<uint8_t>(static_cast<size_t>(T) * B * nk);
    w.scratch = cv.take<char>(std::max(compact_scratch_bytes(T, nl), compact_scratch_bytes(T, nk)));
    // the dz ring and G, then (when they are shorter) enough bytes that the span from the ring's
    // start holds the staging of the gradient reorderings, which run after the last reader of both
    const size_t z0 = cv.mark();
    w.dZ = cv.take<float>(static_cast<size_t>(ring_size(c)) * B * c->D * c->N);
    w.G = cv.take<float>(2 * static_cast<size_t>(c->N) * c->g_rows * g_row(Wwin, B));
    const size_t stage_bytes = sizeof(float) * static_cast<size_t>(std::max(
        c->rec->pinv.runs ? c->rec->n_syn : 0, c->lgn->pinv.runs ? c->lgn->n_syn : 0));
    if (cv.off - z0 < stage_bytes) cv.take<char>(stage_bytes - (cv.off - z0));
    w.stage = w.dZ;
    w.gV = cv.take<float>(BN);
    w.gP = cv.take<float>(BN * c->nb);
    w.gR = cv.take<float>(BN * c->nb);
    w.vloss_part = cv.take<float>(kVlossBlocks);
    w.dw_rec = cv.take<float>(std::max<int64_t>(c->rec->n_syn, 1));
    w.dw_lgn = cv.take<float>(std::max<int64_t>(c->lgn->n_syn, 1));
    w.dw_bkg = cv.take<float>(std::max<int64_t>(c->bkg->n_syn, 1));
    w.I = cv.take<float>(2 * BN * i_slots(c));   // event mode alternates between the two halves by tick
    if (bytes) *bytes = cv.off;
    return w;
}

static CellConst make_const(const Cell *c, int B) {
    CellConst k{};
    k.N = c->N;
    k.Np = c->Np;
    k.W = c->W;
    k.D = c->D;
    k.nb = c->nb;
    k.n_types = c->n_types;
    k.B = B;
    k.Bp = batch_pad(B);
    k.lr = c->cfg.lr_scale;
    float vgd = std::min(1.0f, std::max(0.0f, c->cfg.voltage_gradient_dampening));
    k.vgd = vgd;
    k.om = 1.0f - vgd;
    float rd = std::min(1.0f, std::max(0.0f, c->cfg.recurrent_dampening));
    // straight_through_dampen(z_buf, 1 - rd) scales the spike-buffer gradient by 1 - (1 - rd)
    k.rd_scale = 1.0f - (1.0f - rd);
    k.gauss_std = c->cfg.gauss_std;
    k.damp = c->cfg.dampening_factor;
    k.dt = c->cfg.dt;
    k.pseudo_gauss = c->cfg.pseudo_gauss;
    k.hard_reset = c->cfg.hard_reset;
    for (int q = 0; q < c->nb; ++q) {
        k.sd[q] = c->syn_decay[q];
        k.p0[q] = c->psc_initial[q];
        k.dtsd[q] = c->dtsd[q];
    }
    return k;
}

__device__ inline bool zbit(const uint64_t *zbits, int slot, int b, int B, int W, int n) {
    return (zbits[(static_cast<int64_t>(slot) * B + b) * W + (n >> 6)] >> (n & 63)) & 1ull;
}

// ---------------------------------------------------------- history init ----
// z_buf [B][D*N] (slot d-1 = z_{-d}) -> spike bits (slot D-d) and, for the
// deterministic pull, the batch masks and activity bitmaps of steps -1..-D.
__global__ void __launch_bounds__(kBlock)
    k_init_history(const float *__restrict__ z_buf, CellConst k, uint64_t *__restrict__ zbits,
                   uint32_t *__restrict__ zmask, uint64_t *__restrict__ abits) {
    const int64_t gt = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t per_slot = static_cast<int64_t>(k.B) * k.Np;
    if (gt >= per_slot * k.D) return;
    const int d = static_cast<int>(gt / per_slot) + 1;
    const int b = static_cast<int>((gt % per_slot) / k.Np);
    const int n = static_cast<int>(gt % k.Np);
    const int lane = threadIdx.x & (kWave - 1);
    bool z = n < k.N && z_buf[static_cast<int64_t>(b) * k.D * k.N + static_cast<int64_t>(d - 1) * k.N + n] > 0.0f;
    const uint64_t bits = __ballot(z);
    const int slot = k.D - d;
    if (lane == 0) zbits[(static_cast<int64_t>(slot) * k.B + b) * k.W + (n >> 6)] = bits;
    if (zmask && z) atomicOr(zmask + static_cast<int64_t>(slot) * k.Np + n, 1u << b);
    if (abits && lane == 0 && bits) atomicOr(abits + static_cast<int64_t>(slot) * k.W + (n >> 6), bits);
}

// lmask[t][pre] = batch mask of the LGN inputs x_t[b][pre] > 0, and lbits[t] the
// bitmap of the inputs active in some batch entry (rows padded to Wl 64-bit words;
// one wave per word).
__global__ void __launch_bounds__(kBlock)
    k_lgn_mask(const uint8_t *__restrict__ x, int T, int B, int32_t n_in, int32_t Wl,
               uint32_t *__restrict__ lmask, uint64_t *__restrict__ lbits) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t row = static_cast<int64_t>(Wl) * 64;
    if (i >= static_cast<int64_t>(T) * row) return;  // whole waves only
    const int64_t t = i / row;
    const int32_t pre = static_cast<int32_t>(i - t * row);
    uint32_t m = 0;
    if (pre < n_in) {
        for (int b = 0; b < B; ++b)
            if (x[(t * B + b) * n_in + pre] > 0) m |= 1u << b;
        lmask[t * n_in + pre] = m;
    }
    const uint64_t bits = __ballot(m != 0u);
    if ((threadIdx.x & (kWave - 1)) == 0) lbits[t * Wl + (pre >> 6)] = bits;
}

// lgnT[(seg * n_in + pre) * B + b] = tick mask of input pre in batch entry b over segment seg:
// bit k = x[64 seg + k][b][pre] > 0 (0 past T).  Thread per (b, pre), reads coalesced over
// the inputs.
__global__ void __launch_bounds__(kBlock)
    k_lgn_tmask(const uint8_t *__restrict__ x, int T, int B, int32_t n_in, uint64_t *__restrict__ lgnT) {
    const int seg = blockIdx.y;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<int64_t>(B) * n_in) return;
    const int b = static_cast<int>(i / n_in);
    const int32_t pre = static_cast<int32_t>(i - static_cast<int64_t>(b) * n_in);
    const int k_end = min(kLgnSeg, T - seg * kLgnSeg);
    uint64_t m = 0;
    for (int k = 0; k < k_end; ++k) {
        const int64_t t = static_cast<int64_t>(seg) * kLgnSeg + k;
        if (x[(t * B + b) * n_in + pre] > 0) m |= 1ull << k;
    }
    lgnT[(static_cast<int64_t>(seg) * n_in + pre) * B + b] = m;
}

struct LgnRowArgs {
    int32_t seg, T, N, B, nb, n_types, n_in;
    const int32_t *row;   // post-grouped LGN table: row pointers,
    const uint32_t *pd;   // pre | (delay - 1) << 24,
    const uint8_t *sid;   // synapse type,
    const float *w;       // weight, in ascending (column, synapse id) order per row
    const uint64_t *lgnT; // tick masks per (input, batch entry) (k_lgn_tmask)
    const float *basis;   // [n_types][nb]
    float *ring;          // kLgnRing slots of [nb][B][N]
};

// One wave per post, lane k = tick 64 seg + k: the row's entries are wave-uniform, and the
// 64-tick mask of the entry's input in batch entry b selects the lanes that add
// w * basis[type][r] into their (b, r) accumulators, in entry order from +0
// -- per (tick, b, post, r) the reference's order over the LGN events, the same sum the
// deterministic row pull forms.  Zero products are skipped (adding +/-0 to a sum started
// at +0 never changes it), so only the receptors the type's basis feeds are visited.  The
// workgroup's 8 posts then write each (b, r) plane through LDS as 32-byte runs.
template <int NB, int BB>
__global__ void __launch_bounds__(kLgnPosts * kWave) k_lgn_rows(LgnRowArgs a) {
    __shared__ float tile[2][kLgnSeg][kLgnPosts + 1];
    extern __shared__ float basis_lds[];  // [n_types][nb], then the per-type receptor masks
    uint32_t *nz_lds = reinterpret_cast<uint32_t *>(basis_lds + a.n_types * NB);
    load_basis_lds(basis_lds, a.basis, a.n_types * NB);
    for (int s = threadIdx.x; s < a.n_types; s += blockDim.x) {
        uint32_t m = 0;
        for (int q = 0; q < NB; ++q)
            if (a.basis[s * NB + q] != 0.0f) m |= 1u << q;
        nz_lds[s] = m;
    }
    __syncthreads();
    const int lane = threadIdx.x & (kWave - 1);
    const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
    // XCD-aware order: workgroups go to the 8 XCDs round robin (blockIdx % 8), so group g of
    // consecutive posts is given to workgroup (g % per) * 8 + g / per: neighbouring groups,
    // whose 32-byte output runs share 128-byte lines, are written through the same L2
    const int32_t per = static_cast<int32_t>(gridDim.x) / 8;
    const int32_t grp = static_cast<int32_t>(blockIdx.x % 8) * per + static_cast<int32_t>(blockIdx.x / 8);
    const int32_t n = grp * kLgnPosts + wv;
    float acc[BB][NB];
#pragma unroll
    for (int b = 0; b < BB; ++b)
#pragma unroll
        for (int q = 0; q < NB; ++q) acc[b][q] = 0.0f;
    if (n < a.N) {
        const uint64_t *tm = a.lgnT + static_cast<int64_t>(a.seg) * a.n_in * BB;
        const int32_t j0 = a.row[n], j1 = a.row[n + 1];
        // Up to 64 entries at a time: lane l loads entry jb + l (input, type, weight; three
        // coalesced loads, indices clamped to the row's last entry), forms its products
        // w * basis[type][r] and the receptors its type feeds; the walk reads them back with
        // lane reads.  Per entry the BB tick masks of its input are scalar loads (4 entries'
        // at a time), and each mask is the lane mask of that batch entry's adds.
        for (int32_t jb = j0; jb < j1; jb += kWave) {
            const int cnt = min(j1 - jb, kWave);
            const int32_t jl = min(jb + lane, j1 - 1);
            const int pre_l = static_cast<int>(a.pd[jl] & kLow24);
            const int sid_l = a.sid[jl];
            const float w_l = a.w[jl];
            const int nz_l = static_cast<int>(nz_lds[sid_l]);
            int v_l[NB];
#pragma unroll
            for (int q = 0; q < NB; ++q) v_l[q] = __float_as_int(w_l * basis_lds[sid_l * NB + q]);
            for (int ub = 0; ub < cnt; ub += 4) {
                uint64_t M[4][BB];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int pre = __builtin_amdgcn_readlane(pre_l, min(ub + u, kWave - 1));
#pragma unroll
                    for (int b = 0; b < BB; ++b) M[u][b] = tm[static_cast<int64_t>(pre) * BB + b];
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    if (ub + u >= cnt) break;
                    uint64_t any = 0;
#pragma unroll
                    for (int b = 0; b < BB; ++b) any |= M[u][b];
                    if (any == 0ull) continue;
                    const uint32_t nz = static_cast<uint32_t>(__builtin_amdgcn_readlane(nz_l, ub + u));
#pragma unroll
                    for (int q = 0; q < NB; ++q) {
                        if (!((nz >> q) & 1u)) continue;
                        const float v = __int_as_float(__builtin_amdgcn_readlane(v_l[q], ub + u));
#pragma unroll
                        for (int b = 0; b < BB; ++b)
                            if (M[u][b] != 0ull && __builtin_amdgcn_inverse_ballot_w64(M[u][b]))
                                acc[b][q] = acc[b][q] + v;
                    }
                }
            }
        }
    }
    // every wave takes part in the write-out (barriers), live or not
    const int64_t BN = static_cast<int64_t>(a.B) * a.N;
    const int kt = threadIdx.x / kLgnPosts, p = threadIdx.x % kLgnPosts;
    const int t = a.seg * kLgnSeg + kt;
    const int32_t np = grp * kLgnPosts + p;
    float *slot = a.ring + static_cast<int64_t>(t % kLgnRing) * NB * BN;
    int buf = 0;
#pragma unroll
    for (int b = 0; b < BB; ++b) {
#pragma unroll
        for (int q = 0; q < NB; ++q) {
            tile[buf][lane][wv] = acc[b][q];
            __syncthreads();
            if (t < a.T && np < a.N) slot[q * BN + static_cast<int64_t>(b) * a.N + np] = tile[buf][kt][p];
            buf ^= 1;
        }
    }
}

template <int NB>
static void launch_lgn_rows_nb(const LgnRowArgs &la, dim3 grid, size_t lds, hipStream_t s) {
    switch (la.B) {
#define GLIF_LGN_ROWS(BB) \
    case BB: GLIF_PROF_LAUNCH((k_lgn_rows<NB, BB>), grid, dim3(kLgnPosts * kWave), lds, s, la); break;
        GLIF_LGN_ROWS(1) GLIF_LGN_ROWS(2) GLIF_LGN_ROWS(3) GLIF_LGN_ROWS(4) GLIF_LGN_ROWS(5)
        GLIF_LGN_ROWS(6) GLIF_LGN_ROWS(7) GLIF_LGN_ROWS(8)
#undef GLIF_LGN_ROWS
        default: break;
    }
}

static void launch_lgn_rows(const LgnRowArgs &la, hipStream_t s) {
    // a multiple of 8 workgroups (the XCD-aware order); groups past the last post idle
    const dim3 grid(static_cast<unsigned>(8 * ceil_div(static_cast<int64_t>(la.N), 8 * kLgnPosts)));
    const size_t lds = sizeof(float) * la.n_types * (la.nb + 1);
    switch (la.nb) {
        case 1: launch_lgn_rows_nb<1>(la, grid, lds, s); break;
        case 2: launch_lgn_rows_nb<2>(la, grid, lds, s); break;
        case 3: launch_lgn_rows_nb<3>(la, grid, lds, s); break;
        case 4: launch_lgn_rows_nb<4>(la, grid, lds, s); break;
        case 5: launch_lgn_rows_nb<5>(la, grid, lds, s); break;
        case 6: launch_lgn_rows_nb<6>(la, grid, lds, s); break;
        case 7: launch_lgn_rows_nb<7>(la, grid, lds, s); break;
        case 8: launch_lgn_rows_nb<8>(la, grid, lds, s); break;
        default: break;
    }
}

// z_buf out = [z_{T-1}, ..., z_{T-D}].
__global__ void __launch_bounds__(kBlock)
    k_write_zbuf(float *__restrict__ z_buf, CellConst k, int T, const uint64_t *__restrict__ zbits) {
    const int64_t gt = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t per_slot = static_cast<int64_t>(k.B) * k.N;
    if (gt >= per_slot * k.D) return;
    const int d = static_cast<int>(gt / per_slot) + 1;
    const int b = static_cast<int>((gt % per_slot) / k.N);
    const int n = static_cast<int>(gt % k.N);
    const bool z = zbit(zbits, T - d + k.D, b, k.B, k.W, n);
    z_buf[static_cast<int64_t>(b) * k.D * k.N + static_cast<int64_t>(d - 1) * k.N + n] = z ? 1.0f : 0.0f;
}

// Reference-layout state (psc_rise/psc [B][N*nb], asc [B][N*2]) <-> the rollout's
// receptor-major copies ([nb][B][N], [2][B][N]) so every state access of the step
// kernel is one coalesced row.
__global__ void __launch_bounds__(kBlock)
    k_state_layout(float *__restrict__ R_ref, float *__restrict__ P_ref, float *__restrict__ A_ref,
                   float *__restrict__ R, float *__restrict__ P, float *__restrict__ A, int64_t BN,
                   int nb, int to_soa) {
    const int64_t bn = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (bn >= BN) return;
    for (int q = 0; q < nb; ++q) {
        if (to_soa) {
            R[q * BN + bn] = R_ref[bn * nb + q];
            P[q * BN + bn] = P_ref[bn * nb + q];
        } else {
            R_ref[bn * nb + q] = R[q * BN + bn];
            P_ref[bn * nb + q] = P[q * BN + bn];
        }
    }
    for (int j = 0; j < 2; ++j) {
        if (to_soa)
            A[j * BN + bn] = A_ref[bn * 2 + j];
        else
            A_ref[bn * 2 + j] = A[j * BN + bn];
    }
}

// ------------------------------------------------------------ event push ----
struct PushArgs {
    int32_t t, D, N, B, W, nb, n_types, chunks_lgn;
    int32_t d_lo, d_hi;   // delay slots pushed (1-based, inclusive)
    int32_t lgn;          // push the step's LGN events too
    int32_t typed;        // per-type slots (rec_ps / lgn_ps are then {post | rank} entries)
    const uint64_t *zbits;  // [(T + D)][B][W] spike bits, slot s + D holds z_s
    const int32_t *rec_colptr;
    const uint32_t *rec_ps;
    const float *rec_w;
    const int64_t *lgn_off;
    const int32_t *lgn_pre;
    const uint32_t *lgn_mask;
    const int32_t *lgn_colptr;
    const uint32_t *lgn_ps;
    const float *lgn_w;
    const float *basis;
    float *I;
};

// Work units, one wave each: the 64-bit spike words of steps t-1..t-D (D * B * W
// words; each set bit is one spike, i.e. one column of the recurrent table, pushed
// whole), then (column, chunk) units of the step's LGN columns (a chunk is
// kWave * kChunkIters synapses, so long columns spread over several waves).  The
// spike words come straight from the step kernel's ballots: no spike list, no
// counter that every spiking wave would have to increment.
constexpr int kChunkIters = 4;

__device__ inline void push_body(const PushArgs &a, int64_t bid, int64_t nblk) {
    constexpr int L = kWave;
    extern __shared__ float basis_lds[];
    load_basis_lds(basis_lds, a.basis, a.n_types * a.nb);
    const int64_t BW = static_cast<int64_t>(a.B) * a.W;
    const int64_t n_words = a.d_hi >= a.d_lo ? static_cast<int64_t>(a.d_hi - a.d_lo + 1) * BW : 0;
    const int64_t l0 = a.lgn ? a.lgn_off[a.t] : 0, n_lgn = a.lgn ? a.lgn_off[a.t + 1] - l0 : 0;
    const int64_t units = n_words + n_lgn * a.chunks_lgn;
    const int lane_s = threadIdx.x % L;
    const int64_t n_subs = nblk * blockDim.x / L;
    const int64_t BN = static_cast<int64_t>(a.B) * a.N;
    // the unit index is uniform across the wave: keep it (and the spike word) scalar
    const int64_t u0 = bid * (blockDim.x / L) + __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / L));
    for (int64_t u = u0; u < units; u += n_subs) {
        if (u < n_words) {
            const int d = static_cast<int>(u / BW) + a.d_lo;
            const int64_t rem = u - static_cast<int64_t>(d - a.d_lo) * BW;
            const int b = static_cast<int>(rem / a.W);
            const int wi = static_cast<int>(rem - static_cast<int64_t>(b) * a.W);
            uint64_t word = a.zbits[(static_cast<int64_t>(a.t - d + a.D) * a.B + b) * a.W + wi];
            while (word) {
                const int bit = __builtin_ctzll(word);
                word &= word - 1ull;
                const int32_t col = wi * 64 + bit + (d - 1) * a.N;
                if (a.typed)
                    push_column_typed<L>(lane_s, a.rec_colptr[col], a.rec_colptr[col + 1], 1u << b, MultOne{},
                                         a.rec_ps, a.rec_w, a.N, BN, a.I);
                else
                    push_column<L>(lane_s, a.rec_colptr[col], a.rec_colptr[col + 1], 1u << b, MultOne{}, a.rec_ps,
                                   a.rec_w, basis_lds, a.nb, a.N, 1, BN, a.I);
            }
        } else {
            const int64_t v = u - n_words;
            const int64_t it = l0 + v / a.chunks_lgn;
            const int ch = static_cast<int>(v % a.chunks_lgn);
            const int32_t c = a.lgn_pre[it];
            const int32_t lo = a.lgn_colptr[c] + ch * L * kChunkIters;
            const int32_t hi = min(a.lgn_colptr[c + 1], lo + L * kChunkIters);
            if (a.typed)
                push_column_typed<L>(lane_s, lo, hi, a.lgn_mask[it], MultOne{}, a.lgn_ps, a.lgn_w, a.N, BN, a.I);
            else
                push_column<L>(lane_s, lo, hi, a.lgn_mask[it], MultOne{}, a.lgn_ps, a.lgn_w, basis_lds,
                               a.nb, a.N, 1, BN, a.I);
        }
    }
}

__global__ void __launch_bounds__(kBlock) k_push(PushArgs a) { push_body(a, blockIdx.x, gridDim.x); }

// ------------------------------------------------------------- GLIF step ----
struct StepArgs {
    CellConst k;
    int32_t t;
    int32_t count_t0, count_t1;  // spike_count takes ticks [count_t0, count_t1)
    float *v;
    int16_t *r;
    float *A;   // [2][B][N]
    float *R;   // [nb][B][N]
    float *P;   // [nb][B][N]
    const float *decay, *cf, *ad, *amp;
    const int32_t *tref;
    float *I;
    const float *I2;  // deterministic chunk pull: LGN currents, I holds the recurrent ones
    uint64_t *zbits;
    uint64_t *refbits;
    uint32_t *zmask;
    uint64_t *abits;
    float *vsave;
    float *z_out, *v_out;
    int32_t *spike_count;
    const int32_t *rec_row;
    const uint32_t *rec_pd;
    const uint8_t *rec_sid;
    const float *rec_w;
    const int32_t *lgn_row;
    const uint32_t *lgn_pd;
    const uint8_t *lgn_sid;
    const float *lgn_w;
    const uint8_t *lgn_x;  // [B][n_lgn] of step t
    int32_t n_lgn;
    const int32_t *bkg_row;
    const uint32_t *bkg_pd;
    const uint8_t *bkg_sid;
    const float *bkg_w;
    const uint2 *bkg_ell;  // ELL copy of the background table, or nullptr
    int32_t bkg_ell_len;
    const uint8_t *bkg_x;  // [B][n_bkg] of step t
    int32_t n_bkg;
    const float *basis;
    // event mode: each wave pushes the delay-1 columns of its spikes into the next tick's
    // currents (nullptr: no push)
    float *I_next;
    const int32_t *p1_colptr;
    const uint32_t *p1_ps;
    const float *p1_w;
    // event mode with per-type slots: I holds [gk][B][N] type sums (p1_ps {post | rank});
    // receptor r's current is sum_q I[q] * basis[gtype[n][q]][r], ascending q.  0: [nb][B][N]
    int32_t gk;
    const uint8_t *gtype;
    // deterministic pull beside the step (lag = 1): R takes tick t - 1's currents (I, I2
    // and bkg_x point at that tick; none at t = 0), P the R of tick t - 1 so updated
    int32_t lag;
    // event mode: I is a slot of the LGN ring, which the LGN pass rewrites before its next
    // use, so the step leaves it as it is (0: the step clears I after reading it)
    int32_t keep_I;
};

// The input of R for (b, n) at one tick, (I_rec + I_lgn) + I_bkg, times lr_scale
// (models.py:896-931, 979-990): the pushed (event, [nb][B][N] or per-type slots, cleared
// after reading) or pulled (deterministic) rec + LGN currents, plus the background, every
// synapse of the row times its Poisson count.
template <bool DET, int NB>
__device__ inline void step_inputs(const StepArgs &a, const float *basis_lds, int n, int b, int64_t bn,
                                   float (&in)[kMaxBasis]) {
    const CellConst &k = a.k;
    constexpr int nb = NB;
    const int64_t BN = static_cast<int64_t>(k.B) * k.N;
    float Irl[kMaxBasis], Ib[kMaxBasis];
    for (int q = 0; q < nb; ++q) Ib[q] = 0.0f;
    if (!DET && a.gk) {
        // the pushed rec + LGN type sums, folded through the basis (a slot past the
        // post's types holds +0 and is skipped)
        for (int q = 0; q < nb; ++q) Irl[q] = 0.0f;
        const uint8_t *gt = a.gtype + static_cast<int64_t>(n) * a.gk;
        for (int j = 0; j < a.gk; ++j) {
            float *Ip = a.I + j * BN + bn;
            const float x = *Ip;
            *Ip = 0.0f;
            const int sj = gt[j];
            if (sj == 0xFF) continue;
            const float *bs = basis_lds + sj * nb;
#pragma unroll
            for (int q = 0; q < nb; ++q) Irl[q] = Irl[q] + x * bs[q];
        }

    } else {
        // the pushed (event) or pulled (deterministic) rec + LGN currents
        for (int q = 0; q < nb; ++q) {
            float *Ip = a.I + q * BN + bn;
            Irl[q] = *Ip;
            if (DET && a.I2) Irl[q] = Irl[q] + a.I2[q * BN + bn];
            if (!DET && !a.keep_I) *Ip = 0.0f;
        }
    }
    // background: every synapse of the row, weight times the Poisson count.  A zero
    // count adds +/-0, which leaves a sum started at +0 unchanged, so the
    // branch-free loop equals the reference's event-only sum bit for bit.
    const uint8_t *xb = a.bkg_x + static_cast<int64_t>(b) * a.n_bkg;
    if (a.bkg_ell) {
        // ELL rows: entry j of every post in one coalesced 8-byte load; the padding
        // ({pre 0, w +0}) adds +0, which leaves the sum unchanged
        for (int32_t jb = 0; jb < a.bkg_ell_len; jb += 8) {
            uint2 e[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                e[u] = jb + u < a.bkg_ell_len ? a.bkg_ell[static_cast<int64_t>(jb + u) * k.N + n] : make_uint2(0u, 0u);
            float cnt[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) cnt[u] = static_cast<float>(xb[e[u].x & kLow24]);
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                if (jb + u >= a.bkg_ell_len) break;
                const float wv = __uint_as_float(e[u].y) * cnt[u];
                const float *bs = basis_lds + (e[u].x >> 24) * nb;
#pragma unroll
                for (int r = 0; r < nb; ++r) Ib[r] = Ib[r] + wv * bs[r];
            }
        }
    } else {
        // 8 synapses at a time: their table entries, then their counts, are loaded
        // together before the (in-order) accumulation
        const int32_t j0 = a.bkg_row[n], j1 = a.bkg_row[n + 1];
        for (int32_t jb = j0; jb < j1; jb += 8) {
            uint32_t pd[8];
            float wj[8];
            int sj[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const bool ok = jb + u < j1;
                pd[u] = ok ? a.bkg_pd[jb + u] : 0u;
                wj[u] = ok ? a.bkg_w[jb + u] : 0.0f;
                sj[u] = ok ? a.bkg_sid[jb + u] : 0;
            }
            float cnt[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) cnt[u] = (jb + u < j1) ? static_cast<float>(xb[pd[u] & kLow24]) : 0.0f;
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                if (jb + u >= j1) break;
                const float wv = wj[u] * cnt[u];
                const float *bs = basis_lds + sj[u] * nb;
#pragma unroll
                for (int r = 0; r < nb; ++r) Ib[r] = Ib[r] + wv * bs[r];
            }
        }
    }
    for (int q = 0; q < nb; ++q) in[q] = (Irl[q] + Ib[q]) * k.lr;
}

// One GLIF_3 update per thread (b, n), models.py:979-1028 and 1059-1135:
//   I      = ((I_rec + I_lgn) + I_bkg) * lr_scale
//   R'     = R * sd + I * p0                P' = P * sd + (dt * sd) * R
//   A'     = ad * A + z_prev * amp          c  = sum_r P + (A_0 + A_1)   (old P, A)
//   V'     = (decay * (V * (1 - vgd) + V * vgd) + cf * c) - z_prev
//   r'     = max(r + z_prev * tref - 1, 0); hard reset: V' = 0 while r' > 0
//   z      = r' > 0 ? 0 : (V' - 1 > 0)
// V', r' and z take the old P and A only, so tick t's currents can arrive one launch late
// (a.lag): R is then brought to tick t - 1 here and P' takes that R.
template <bool DET, int NB>
__device__ inline void step_body(const StepArgs &a, int64_t bid) {
    extern __shared__ float basis_lds[];
    const CellConst &k = a.k;
    load_basis_lds(basis_lds, a.basis, k.n_types * k.nb);
    const int64_t gt = bid * blockDim.x + threadIdx.x;
    if (gt >= static_cast<int64_t>(k.B) * k.Np) return;  // whole waves only (Np % 64 == 0)
    // wave w: batch entry w % B of neurons 64 (w / B) ..: the B waves of a neuron block run
    // back to back and share its background table entries in cache
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t wv = bid * (blockDim.x / kWave) + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int b = static_cast<int>(wv % k.B);
    const int n = static_cast<int>(wv / k.B) * kWave + lane;
    constexpr int nb = NB;
    const int t = a.t;
    bool spike = false, refr = false;
    if (n < k.N) {
        const int64_t BN = static_cast<int64_t>(k.B) * k.N;
        const int64_t bn = static_cast<int64_t>(b) * k.N + n;
        const bool upd = !a.lag || t > 0;  // with the lag, R of tick -1 is the state
        float in[kMaxBasis];
        if (upd) step_inputs<DET, NB>(a, basis_lds, n, b, bn, in);
        const float zp = zbit(a.zbits, t - 1 + k.D, b, k.B, k.W, n) ? 1.0f : 0.0f;
        float Pold[kMaxBasis];
        for (int q = 0; q < nb; ++q) Pold[q] = a.P[q * BN + bn];
        float sumP = Pold[0];
        for (int q = 1; q < nb; ++q) sumP = sumP + Pold[q];
        const float A0 = a.A[bn], A1 = a.A[BN + bn];
        const float c1 = sumP + (A0 + A1);
        for (int q = 0; q < nb; ++q) {
            float *Rq = a.R + q * BN + bn;
            const float Rold = *Rq;
            const float Rnew = upd ? Rold * k.sd[q] + in[q] * k.p0[q] : Rold;
            if (upd) *Rq = Rnew;
            a.P[q * BN + bn] = Pold[q] * k.sd[q] + k.dtsd[q] * (a.lag ? Rnew : Rold);
        }
        a.A[bn] = a.ad[2 * n] * A0 + zp * a.amp[2 * n];
        a.A[BN + bn] = a.ad[2 * n + 1] * A1 + zp * a.amp[2 * n + 1];
        const float vv = a.v[bn];
        const float dv = vv * k.om + vv * k.vgd;
        float vn = (a.decay[n] * dv + a.cf[n] * c1) - zp;
        int rn = static_cast<int>(a.r[bn]) + static_cast<int>(zp) * a.tref[n] - 1;
        rn = rn < 0 ? 0 : rn;
        refr = rn > 0;
        if (k.hard_reset && refr) vn = 0.0f;
        spike = !refr && (vn - 1.0f) > 0.0f;
        a.v[bn] = vn;
        a.r[bn] = static_cast<int16_t>(rn);
        const int64_t tbn = static_cast<int64_t>(t) * BN + bn;
        a.vsave[tbn] = vn;
        if (a.z_out) a.z_out[tbn] = spike ? 1.0f : 0.0f;
        if (a.v_out) a.v_out[tbn] = vn;
        if (a.spike_count && spike && t >= a.count_t0 && t < a.count_t1) a.spike_count[bn] += 1;
        if (DET && spike) atomicOr(a.zmask + static_cast<int64_t>(t + k.D) * k.Np + n, 1u << b);
    }
    const uint64_t zb = __ballot(spike), rb = __ballot(refr);
    const int64_t word = static_cast<int64_t>(b) * k.W + (n >> 6);
    if (lane == 0) {
        a.zbits[static_cast<int64_t>(t + k.D) * k.B * k.W + word] = zb;
        a.refbits[static_cast<int64_t>(t) * k.B * k.W + word] = rb;
        if (DET && zb) atomicOr(a.abits + static_cast<int64_t>(t + k.D) * k.W + (n >> 6), zb);
    }
    if (!DET && a.I_next) {
        // the wave's spikes (a wave-uniform word) reach their delay-1 posts at tick t + 1:
        // column pre + 0 * N of the recurrent table, all 64 lanes over its synapses
        const int64_t BN = static_cast<int64_t>(k.B) * k.N;
        const int32_t n0 = n & ~(kWave - 1);
        uint64_t zw = zb;
        while (zw) {
            const int bit = __builtin_ctzll(zw);
            zw &= zw - 1ull;
            const int32_t col = n0 + bit;
            if (a.gk)
                push_column_typed<kWave>(lane, a.p1_colptr[col], a.p1_colptr[col + 1], 1u << b, MultOne{}, a.p1_ps,
                                         a.p1_w, k.N, BN, a.I_next);
            else
                push_column<kWave>(lane, a.p1_colptr[col], a.p1_colptr[col + 1], 1u << b, MultOne{}, a.p1_ps,
                                   a.p1_w, basis_lds, nb, k.N, 1, BN, a.I_next);
        }
    }
}

template <bool DET, int NB>
__global__ void __launch_bounds__(kBlock) k_step(StepArgs a) {
    step_body<DET, NB>(a, blockIdx.x);
}

// Deterministic mode: the row pull of tick t (the first pull_blocks workgroups, resident,
// into one half of the double-buffered currents) beside the step of tick t with R one tick
// late (the other workgroups, reading the other half).  The pull streams the tables and is
// bound by its chains of dependent loads and ordered adds, the step streams the state, and
// one launch overlaps them.
template <int NB>
__global__ void __launch_bounds__(kPullBlock) k_pull_step(PullArgs pa, int pull_blocks, StepArgs sa) {
    if (static_cast<int>(blockIdx.x) < pull_blocks) pull_chunks_body<1>(pa, blockIdx.x, pull_blocks);
    else step_body<true, NB>(sa, blockIdx.x - pull_blocks);
}

// After the lagged loop: R of the last tick from its currents and background.
template <int NB>
__global__ void __launch_bounds__(kBlock) k_r_last(StepArgs a) {
    extern __shared__ float basis_lds[];
    const CellConst &k = a.k;
    load_basis_lds(basis_lds, a.basis, k.n_types * k.nb);
    const int64_t gt = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (gt >= static_cast<int64_t>(k.B) * k.Np) return;
    const int b = static_cast<int>(gt / k.Np), n = static_cast<int>(gt % k.Np);
    if (n >= k.N) return;
    const int64_t BN = static_cast<int64_t>(k.B) * k.N, bn = static_cast<int64_t>(b) * k.N + n;
    float in[kMaxBasis];
    step_inputs<true, NB>(a, basis_lds, n, b, bn, in);
    for (int q = 0; q < NB; ++q) {
        float *Rq = a.R + q * BN + bn;
        *Rq = *Rq * k.sd[q] + in[q] * k.p0[q];
    }
}

// Event mode: the push of tick t's events that do not depend on the step of tick t - 1
// (delay slots >= 2 and the LGN inputs; the first gridDim.x - step_blocks blocks) with that
// step (the last step_blocks blocks; each wave also pushes its spikes' delay-1 events), all
// into tick t's current buffer:
// the step streams state through HBM while the push is bound by atomics, and one launch
// overlaps them.
// 8 waves per SIMD (its SGPRs otherwise allow 7; a few scalar values then live in vector lanes):
// 39.4 against 39.8 us per tick.
template <int NB>
__global__ void __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(8, 8)))
k_step_push(StepArgs sa, int step_blocks, PushArgs pa) {
    // the push blocks come first, so the atomic-bound push (the longer part) starts at once
    // and the step blocks fill the machine behind it
    const int64_t bid = blockIdx.x;
    const int64_t push_blocks = gridDim.x - step_blocks;
    if (bid < push_blocks)
        push_body(pa, bid, push_blocks);
    else
        step_body<false, NB>(sa, bid - push_blocks);
}

// ------------------------------------------------- voltage regularization ----
// VoltageRegularization (loss_functions.py:1047-1119): penalty of the cell's output
// voltage, range mode relu(|v - 0.5| - 0.5)^2 (zero inside [0, 1]), threshold mode
// (v - 1)^2; the loss is cost * mean over (T, B, N).  Its gradient enters the adjoint
// like dL/dv (relu' = 0 at the kink, as TF's).
__device__ inline float vpenalty(int mode, float v) {
    if (mode == 1) {
        const float m = fabsf(v - 0.5f) - 0.5f;
        return m > 0.0f ? m * m : 0.0f;
    }
    const float d = v - 1.0f;
    return d * d;
}

__device__ inline float vpenalty_grad(int mode, float v) {
    if (mode == 1) {
        const float x = v - 0.5f;
        const float m = fabsf(x) - 0.5f;
        return m > 0.0f ? (2.0f * m) * (x > 0.0f ? 1.0f : -1.0f) : 0.0f;
    }
    return 2.0f * (v - 1.0f);
}

// Fixed-order reduction (run to run identical): block partials, then one block.
__global__ void __launch_bounds__(kBlock)
    k_vloss_partial(const float *__restrict__ v, int64_t n, int mode, const uint8_t *__restrict__ mask, int32_t N,
                    float *__restrict__ part) {
    __shared__ float red[kBlock];
    float acc = 0.0f;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        if (!mask || mask[i % N]) acc += vpenalty(mode, v[i]);
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int o = kBlock / 2; o > 0; o >>= 1) {
        if (static_cast<int>(threadIdx.x) < o) red[threadIdx.x] += red[threadIdx.x + o];
        __syncthreads();
    }
    if (threadIdx.x == 0) part[blockIdx.x] = red[0];
}

__global__ void __launch_bounds__(kBlock)
    k_vloss_final(const float *__restrict__ part, int n_part, float scale, float *__restrict__ out) {
    __shared__ float red[kBlock];
    float acc = 0.0f;
    for (int i = threadIdx.x; i < n_part; i += kBlock) acc += part[i];
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int o = kBlock / 2; o > 0; o >>= 1) {
        if (static_cast<int>(threadIdx.x) < o) red[threadIdx.x] += red[threadIdx.x + o];
        __syncthreads();
    }
    if (threadIdx.x == 0) *out = red[0] * scale;
}

// --------------------------------------------------------------- adjoint ----
constexpr int kDelayUnroll = 8;
constexpr int kAdjMaxWin = 3;  // reverse ticks per window (3 when 3 * B <= 16, else 1)

struct AdjArgs {
    CellConst k;
    int32_t t0, nw, T, ring, R;
    int32_t tc;      // types per staged chunk of G rows
    int32_t vmode;   // fused voltage regularization (0 off, 1 range, 2 threshold)
    float vscale;    // its cost / (T * B * selected neurons)
    const uint8_t *vmask;  // [N] the selected neurons (core mask), or nullptr: all
    const float *vsave;
    const uint64_t *refbits;
    const float *gz, *gz_neuron, *gv;
    int32_t gzn_t0, gzn_t1;  // gz_neuron applies to ticks [gzn_t0, gzn_t1)
    const float *dZ;
    float *gV, *gP, *gR;
    const float *decay, *cf;
    float *G;
    const float *basis;
    int32_t gk;             // compact G rows per post, 0: type-major rows
    const uint8_t *gtype;   // [N][gk] syn_id of each compact row, 0xFF: none
};

// Lagged reverse ticks t = t0, t0-1, .., t0-nw+1 (nw <= window width; every t >= 2).
// Carried per (b, n): gV'_{t+1}, gP_t, gR_{t-1}.
//   gz_t   = sum_{d=D..1, t+d <= T-3} rd * dZ_{t+d}[b][(d-1)N + n]  + dL/dz_t
//   gV_t   = gz_t * psi(V_t - 1) [r_t == 0] + dL/dV_t + (gV'_{t+1} * decay) * (1 - vgd)
//   gV'_t  = hard_reset && r_t > 0 ? 0 : gV_t
//   gP_{t-1} = gP_t * sd + gV'_t * cf              (P_{t-1} feeds P_t and V_t)
//   gR_{t-2} = gR_{t-1} * sd + gP_{t-1} * (dt*sd)  (R_{t-2} feeds R_{t-1} and P_{t-1})
//   dy_{t-2} = (gR_{t-2} * p0) * lr_scale;  G[s][n][w*B + b] = sum_r dy_r basis[s][r]
// dZ_s for s >= T-2 is zero (nothing downstream of I_{T-2}, I_{T-1} is observed).
// The ticks of one window only read dZ of earlier (later-in-time) windows.
// A workgroup takes nr = kBlock / B neurons x all B batch entries (thread b * nr + i ->
// (b, n0 + i): every [B][N] access is a few contiguous runs).  The window's dy stay in
// registers until its ticks are done; then the G rows of the workgroup's neurons go out a
// chunk of a.tc types at a time through LDS, each type's rows as one contiguous run (with 121
// types x 4 receptors G is ~0.5 GB per window: written row by row, not element by element).
template <int NB>
__device__ inline void adj_body(const AdjArgs &a, int64_t bid) {
    extern __shared__ float lds_f[];
    float *basis_lds = lds_f;
    const CellConst &k = a.k;
    load_basis_lds(basis_lds, a.basis, k.n_types * k.nb);
    const int64_t BN = static_cast<int64_t>(k.B) * k.N;
    float *Gl = lds_f + k.n_types * k.nb;   // [tc][nr][R]
    const int nr = kBlock / k.B;
    const int32_t n0 = static_cast<int32_t>(bid) * nr;
    const int b = static_cast<int>(threadIdx.x) / nr;
    const int n = n0 + static_cast<int>(threadIdx.x) - b * nr;
    const bool live = b < k.B && n < k.N;
    constexpr int nb = NB;
    float dyw[kAdjMaxWin][kMaxBasis];
#pragma unroll
    for (int w = 0; w < kAdjMaxWin; ++w)
#pragma unroll
        for (int q = 0; q < kMaxBasis; ++q) dyw[w][q] = 0.0f;
    if (live) {
    const int64_t bn = static_cast<int64_t>(b) * k.N + n;
    const int64_t DN = static_cast<int64_t>(k.D) * k.N;
    float gVc = a.gV[bn];
    float gP[kMaxBasis], gR[kMaxBasis];
    for (int q = 0; q < nb; ++q) {
        gP[q] = a.gP[static_cast<int64_t>(q) * BN + bn];
        gR[q] = a.gR[static_cast<int64_t>(q) * BN + bn];
    }
    const float decay = a.decay[n], cfn = a.cf[n];
    // one reverse tick given its loaded inputs: dL/dz (ring sum + loss terms), refractory
    // bit, saved voltage, dL/dv
    auto tick = [&](int w, float gz, bool refr, float vsv, float gvx) {
        float psi = 0.0f;
        if (!refr) {
            const float vsc = vsv - 1.0f;
            if (k.pseudo_gauss) {
                const float q = -(vsc * vsc) / (k.gauss_std * k.gauss_std);
                psi = expf(q) * k.damp;
            } else {
                const float m = 1.0f - fabsf(vsc);
                psi = k.damp * (m > 0.0f ? m : 0.0f);
            }
        }
        float gV = gz * psi;
        if (a.gv) gV = gV + gvx;
        if (a.vmode && (!a.vmask || a.vmask[n])) gV = gV + vpenalty_grad(a.vmode, vsv) * a.vscale;
        gV = gV + (gVc * decay) * k.om;
        gVc = (k.hard_reset && refr) ? 0.0f : gV;
        for (int q = 0; q < nb; ++q) {
            gP[q] = gP[q] * k.sd[q] + gVc * cfn;
            gR[q] = gR[q] * k.sd[q] + gP[q] * k.dtsd[q];
            dyw[w][q] = (gR[q] * k.p0[q]) * k.lr;
        }
    };
    auto refbit = [&](int t) {
        return ((a.refbits[(static_cast<int64_t>(t) * k.B + b) * k.W + (n >> 6)] >> (n & 63)) & 1ull) != 0ull;
    };
    const float gzn = a.gz_neuron ? a.gz_neuron[n] : 0.0f;
    if (k.D <= kDelayUnroll && a.nw <= kAdjMaxWin) {
        // every input of the window's ticks is loaded up front (none of them is written
        // by this window), then the ticks run in order
        float zv[kAdjMaxWin][kDelayUnroll];
        float lz[kAdjMaxWin], vs[kAdjMaxWin], gvw[kAdjMaxWin];
        bool rf[kAdjMaxWin];
#pragma unroll
        for (int w = 0; w < kAdjMaxWin; ++w) {
            const int t = a.t0 - w;
            const bool on = w < a.nw;
#pragma unroll
            for (int d = 1; d <= kDelayUnroll; ++d) {
                const int s = t + d;
                zv[w][d - 1] = (on && d <= k.D && s <= a.T - 3)
                                   ? a.dZ[(static_cast<int64_t>(s % a.ring) * k.B + b) * DN +
                                          static_cast<int64_t>(d - 1) * k.N + n]
                                   : 0.0f;
            }
            const int64_t tbn = static_cast<int64_t>(on ? t : a.t0) * BN + bn;
            lz[w] = (on && a.gz) ? a.gz[tbn] : 0.0f;
            rf[w] = on ? refbit(t) : false;
            vs[w] = on ? a.vsave[tbn] : 0.0f;
            gvw[w] = (on && a.gv) ? a.gv[tbn] : 0.0f;
        }
#pragma unroll
        for (int w = 0; w < kAdjMaxWin; ++w) {
            if (w >= a.nw) break;
            const int t = a.t0 - w;
            // the D ring values summed from d = D down to 1, then the loss terms
            float gz = 0.0f;
#pragma unroll
            for (int d = kDelayUnroll; d >= 1; --d)
                if (d <= k.D && t + d <= a.T - 3) gz = gz + zv[w][d - 1] * k.rd_scale;
            if (a.gz) gz = gz + lz[w];
            if (a.gz_neuron && t >= a.gzn_t0 && t < a.gzn_t1) gz = gz + gzn;
            tick(w, gz, rf[w], vs[w], gvw[w]);
        }
    } else {
#pragma unroll
        for (int w = 0; w < kAdjMaxWin; ++w) {
            if (w >= a.nw) break;
            const int t = a.t0 - w;
            float gz = 0.0f;
            for (int d = k.D; d >= 1; --d) {
                const int s = t + d;
                if (s > a.T - 3) continue;
                gz = gz + a.dZ[(static_cast<int64_t>(s % a.ring) * k.B + b) * DN +
                               static_cast<int64_t>(d - 1) * k.N + n] *
                              k.rd_scale;
            }
            const int64_t tbn = static_cast<int64_t>(t) * BN + bn;
            if (a.gz) gz = gz + a.gz[tbn];
            if (a.gz_neuron && t >= a.gzn_t0 && t < a.gzn_t1) gz = gz + gzn;
            tick(w, gz, refbit(t), a.vsave[tbn], a.gv ? a.gv[tbn] : 0.0f);
        }
    }
    a.gV[bn] = gVc;
    for (int q = 0; q < nb; ++q) {
        a.gP[static_cast<int64_t>(q) * BN + bn] = gP[q];
        a.gR[static_cast<int64_t>(q) * BN + bn] = gR[q];
    }
    }  // live
    const int nn = min(nr, k.N - n0);
    if (a.gk) {
        // compact rows: G[n * gk + q][w*B + b] = sum_r dy_r basis[gtype[n][q]][r], a.tc ranks at
        // a time; a neuron's rows of one chunk are one contiguous run (the whole block's rows
        // are one run when the chunk holds every rank)
        for (int q0 = 0; q0 < a.gk; q0 += a.tc) {
            const int nq = min(a.tc, a.gk - q0);
            const int per_n = nq * a.R;
            for (int i = threadIdx.x; i < nr * per_n; i += blockDim.x) Gl[i] = 0.0f;
            __syncthreads();
            if (live) {
                for (int qi = 0; qi < nq; ++qi) {
                    const int s = a.gtype[static_cast<int64_t>(n) * a.gk + q0 + qi];
                    if (s == 0xFF) continue;
                    const float *bs = basis_lds + s * nb;
#pragma unroll
                    for (int w = 0; w < kAdjMaxWin; ++w) {
                        if (w >= a.nw) break;
                        float g = dyw[w][0] * bs[0];
#pragma unroll
                        for (int r = 1; r < nb; ++r) g = g + dyw[w][r] * bs[r];
                        Gl[(n - n0) * per_n + qi * a.R + w * k.B + b] = g;
                    }
                }
            }
            __syncthreads();
            for (int i = threadIdx.x; i < nn * per_n; i += blockDim.x) {
                const int ni = i / per_n, rem = i - ni * per_n;
                a.G[(static_cast<int64_t>(n0 + ni) * a.gk + q0) * a.R + rem] = Gl[i];
            }
            __syncthreads();
        }
        return;
    }
    // G[s][n][w*B + b] = sum_r dy_r basis[s][r], a.tc types at a time (elements of ticks past
    // nw and the row padding are zero)
    const int per_type = nn * a.R;
    for (int s0 = 0; s0 < k.n_types; s0 += a.tc) {
        const int ns = min(a.tc, k.n_types - s0);
        for (int i = threadIdx.x; i < ns * nr * a.R; i += blockDim.x) Gl[i] = 0.0f;
        __syncthreads();
        if (live) {
            for (int si = 0; si < ns; ++si) {
                const float *bs = basis_lds + (s0 + si) * nb;
#pragma unroll
                for (int w = 0; w < kAdjMaxWin; ++w) {
                    if (w >= a.nw) break;
                    float g = dyw[w][0] * bs[0];
#pragma unroll
                    for (int r = 1; r < nb; ++r) g = g + dyw[w][r] * bs[r];
                    Gl[(si * nr + (n - n0)) * a.R + w * k.B + b] = g;
                }
            }
        }
        __syncthreads();
        for (int i = threadIdx.x; i < ns * per_type; i += blockDim.x) {
            const int si = i / per_type, rem = i - si * per_type;
            a.G[(static_cast<int64_t>(s0 + si) * k.N + n0) * a.R + rem] = Gl[si * nr * a.R + rem];
        }
        __syncthreads();
    }
}

template <int NB>
__global__ void __launch_bounds__(kBlock) k_adj(AdjArgs a) {
    adj_body<NB>(a, blockIdx.x);
}

// ------------------------------------------------------ backward synapses ----
// Recurrent activity of element e = w*B + b of column c = pre + N*(d-1) in the
// window of steps s0, s0-1, ..: the spike z_{s0-w-d}[b][pre] (models.py:128 on the
// spike buffer of step s0-w); dz of that element goes to the ring slot of step s0-w.
struct ActWin {
    static constexpr bool kUnitMult = true;
    const uint64_t *zbits;
    float *dZ;
    int64_t n_cols;
    int32_t s0, B, D, W, n_pre, ring;
    struct Col {
        int32_t c, pre, slot0;  // slot0: spike-history slot of z_{s0-d}
    };
    __device__ Col col(int64_t c64) const {
        const int32_t c = static_cast<int32_t>(c64);
        const int32_t d1 = c / n_pre;
        return Col{c, c - d1 * n_pre, s0 - (d1 + 1) + D};
    }
    __device__ bool on(const Col &ci, int e) const {
        const int w = e / B, b = e - w * B;
        return zbit(zbits, ci.slot0 - w, b, B, W, ci.pre);
    }
    // the spike word of element e and its bit (on() in two steps, so that a group of
    // lookups can be issued before any of them is tested)
    __device__ uint64_t word(const Col &ci, int e) const {
        const int w = e / B, b = e - w * B;
        return zbits[(static_cast<int64_t>(ci.slot0 - w) * B + b) * W + (ci.pre >> 6)];
    }
    __device__ bool bit(const Col &ci, uint64_t wd) const { return ((wd >> (ci.pre & 63)) & 1ull) != 0ull; }
    __device__ float mult(int64_t, int) const { return 1.0f; }
    __device__ float *out(const Col &ci, int e) const {
        const int w = e / B, b = e - w * B;
        return dZ + (static_cast<int64_t>((s0 - w) % ring) * B + b) * n_cols + ci.c;
    }
};

template <int LG>
__global__ void __launch_bounds__(kBlock) k_bwd_rec(ColArgs a, ActWin act) {
    bwd_cols<LG, 2>(a, act);
}

__global__ void __launch_bounds__(kBlock) k_bwd_rec_gs(GsArgs a, ActWin act) {
    __shared__ float stage[kBlock / kWave * kGsStage];
    bwd_groups<4>(a, act, stage, blockIdx.x);
}

// dW of one window's active recurrent columns next to the grouped walk (which computes
// dz only): a wave per 64 consecutive columns; lane l finds the activity of column c0 + l
// over the window's elements (the spikes z_{s0-w-d}[b][pre] of ActWin), then 16-lane
// sub-groups walk the column-grouped synapses of the active columns, a lane per synapse,
// adding G[sid][post][e] for the set elements e in ascending order (reverse time, then
// batch).
// G row of entry p = (p >> 24) * hm + (p & kLow24) * lm: {syn_id | post} entries with
// type-major rows (hm = n_post, lm = 1), {rank | post} entries with compact rows (hm = 1,
// lm = rows per post).
struct RecDwArgs {
    int64_t n_cols;
    int32_t n_elem, hm, lm, R;
    const int32_t *col_ptr;
    const uint32_t *ps;
    const float *G;
    float *dw;  // column-grouped order, accumulated
};

__device__ inline void rec_dw_body(const RecDwArgs &a, const ActWin &act, int64_t bid) {
    const int lane = threadIdx.x % kWave;
    const int64_t c0 = bid * blockDim.x + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave) * kWave;
    if (c0 >= a.n_cols) return;  // the whole wave leaves together
    const int64_t c = c0 + lane;
    uint32_t m = 0;
    int32_t lo = 0, hi = 0;
    {
        // the element lookups are issued at clamped, in-range positions before any is tested
        const ActWin::Col ci = act.col(min(c, a.n_cols - 1));
        uint64_t wd[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) wd[e] = act.word(ci, min(e, a.n_elem - 1));
#pragma unroll
        for (int e = 0; e < 16; ++e)
            if (e < a.n_elem && act.bit(ci, wd[e])) m |= 1u << e;
        if (c >= a.n_cols) m = 0;
        if (m) {
            lo = a.col_ptr[c];
            hi = a.col_ptr[c + 1];
        }
    }
    // four 16-lane sub-groups take the next four active columns, four synapses per lane
    // in flight
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
        // every lane takes part in the shuffles (a lane left out would read back wrong to
        // the lanes that use it as their source); idle sub-groups are masked afterwards
        const int sl_src = src >= 0 ? src : 0;
        const uint32_t msrc = static_cast<uint32_t>(__shfl(static_cast<int>(m), sl_src, kWave));
        const int32_t clo = __shfl(lo, sl_src, kWave);
        const int32_t hsrc = __shfl(hi, sl_src, kWave);
        const uint32_t mm = src >= 0 ? msrc : 0u;
        const int32_t chi = src >= 0 ? hsrc : clo;
        for (int32_t k0 = clo; k0 < chi; k0 += 64) {
            float d[4];
            const float *gp[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int32_t k = min(k0 + 16 * u + sl, chi - 1);
                const uint32_t p = a.ps[k];
                gp[u] = a.G + (static_cast<int64_t>(p >> 24) * a.hm + static_cast<int64_t>(p & kLow24) * a.lm) * a.R;
                d[u] = a.dw[k];
            }
            uint32_t mb = mm;
            while (mb) {
                const int e = __ffs(mb) - 1;
                mb &= mb - 1;
#pragma unroll
                for (int u = 0; u < 4; ++u) d[u] += gp[u][e];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (k0 + 16 * u + sl < chi) a.dw[k0 + 16 * u + sl] = d[u];
        }
    }
}

struct BwdInArgs {
    int32_t j, s0, B, R, hm, lm, chunks;  // G rows as in RecDwArgs
    int64_t n_in;
    const int64_t *off;
    const int32_t *pre;
    const uint32_t *mask;
    const uint8_t *cnt;  // [T][B][n_in] (background counts) or nullptr (spikes)
    const int32_t *col_ptr;
    const uint32_t *ps;
    const float *G;
    float *dw;           // column-grouped order, accumulated
};

// dW of one window's input events (the LGN weight gradient, models.py:814-863 autodiff, and the
// background source): item (column, mask over w*B + b) -> every synapse k of the
// column adds G[sid][post][e] * mult for the set elements e in ascending order
// (reverse time, then batch), the order in which the reference's per-step
// gradients accumulate.
template <bool COUNTS>
__device__ inline void bwd_in_body(const BwdInArgs &a, int64_t bid, int64_t nblk) {
    constexpr int L = kWave;
    const int64_t gt = bid * blockDim.x + threadIdx.x;
    const int lane_s = threadIdx.x % L;
    const int64_t n_subs = nblk * blockDim.x / L;
    const int64_t i0 = a.off[a.j], units = (a.off[a.j + 1] - i0) * a.chunks;
    for (int64_t u = gt / L; u < units; u += n_subs) {
        const int64_t it = i0 + u / a.chunks;
        const int ch = static_cast<int>(u % a.chunks);
        const int32_t c = a.pre[it];
        const uint32_t m = a.mask[it];
        const int32_t lo = a.col_ptr[c] + ch * L * kChunkIters;
        const int32_t hi = min(a.col_ptr[c + 1], lo + L * kChunkIters);
        for (int32_t k = lo + lane_s; k < hi; k += L) {
            const uint32_t p = a.ps[k];
            const float *g = a.G + (static_cast<int64_t>(p >> 24) * a.hm + static_cast<int64_t>(p & kLow24) * a.lm) * a.R;
            float d = a.dw[k];
            uint32_t mm = m;
            while (mm) {
                const int e = __ffs(mm) - 1;
                mm &= mm - 1;
                if (COUNTS) {
                    const int w = e / a.B, b = e - w * a.B;
                    d += g[e] * static_cast<float>(a.cnt[(static_cast<int64_t>(a.s0 - w) * a.B + b) * a.n_in + c]);
                } else {
                    d += g[e];
                }
            }
            a.dw[k] = d;
        }
    }
}

// ------------------------------------------------------------ launchers ----
static void launch_bwd_rec(const ColArgs &ca, int R, const ActWin &act, hipStream_t s) {
    const int LG = R / 4;
    const dim3 grid(ceil_div(ca.n_cols * LG, kBlock));
    if (LG == 1) GLIF_PROF_LAUNCH(k_bwd_rec<1>, grid, dim3(kBlock), 0, s, ca, act);
    else if (LG == 2) GLIF_PROF_LAUNCH(k_bwd_rec<2>, grid, dim3(kBlock), 0, s, ca, act);
    else if (LG == 4) GLIF_PROF_LAUNCH(k_bwd_rec<4>, grid, dim3(kBlock), 0, s, ca, act);
    else GLIF_PROF_LAUNCH(k_bwd_rec<8>, grid, dim3(kBlock), 0, s, ca, act);
}


template <bool COUNTS>
__global__ void __launch_bounds__(kBlock) k_bwd_in(BwdInArgs a) {
    bwd_in_body<COUNTS>(a, blockIdx.x, gridDim.x);
}

// The adjoint of window j (blocks [0, adj_blocks) after the walk's, writing G buffer j % 2)
// with the weight gradients of window j - 1 (the rest: the recurrent dW pass, then the LGN
// dW, reading G buffer (j - 1) % 2): the adjoint streams state through HBM while the dW passes are chains
// of dependent loads, and one launch keeps the dW work out of window j's dz walk.
// With a split dz walk, also the second part of window j - 1's walk (the columns of delays
// above what window j's adjoint reads, blocks [0, walk_blocks), first since they run longest):
// the adjoint of tick t reads dz of tick t + d at delay d only, so window j's adjoint needs
// window j - 1's dz of delays <= 2 W - 3, and the rest of that walk can share its launch.
// Window j's weight-gradient passes (recurrent, LGN), run behind the first part of its dz
// walk in one launch (they read G(j) and the window's spikes only, not dz).
struct WinDw {
    RecDwArgs da;
    ActWin act;
    BwdInArgs la;
    int32_t rec_blocks, lgn_blocks;
};

__global__ void __launch_bounds__(kBlock) k_bwd_rec_gs_dw(GsArgs a, ActWin act, int walk_blocks, WinDw p) {
    __shared__ float stage[kBlock / kWave * kGsStage];
    int64_t bid = blockIdx.x;
    if (bid < walk_blocks) {
        bwd_groups<4>(a, act, stage, bid);
        return;
    }
    bid -= walk_blocks;
    if (bid < p.rec_blocks) rec_dw_body(p.da, p.act, bid);
    else bwd_in_body<false>(p.la, bid - p.rec_blocks, p.lgn_blocks);
}

// The rest of window j - 1's dz walk (the columns of delays > 2 W - 3, which the next
// window's adjoint does not read), run beside window j's adjoint, and with a large G window
// j - 1's weight-gradient passes too (dw.rec_blocks / lgn_blocks 0: they ran beside the walk).
struct WalkRest {
    GsArgs gb;
    ActWin act;
    int32_t walk_blocks;
    WinDw dw;
};

template <int NB>
__global__ void __launch_bounds__(kBlock) k_adj_dw(AdjArgs a, int adj_blocks, WalkRest p) {
    int64_t bid = blockIdx.x;
    if (bid < p.walk_blocks) {
        extern __shared__ float lds_f[];  // kBlock / kWave * kGsStage floats of the launch's LDS
        bwd_groups<4>(p.gb, p.act, lds_f, bid);
        return;
    }
    bid -= p.walk_blocks;
    if (bid < adj_blocks) adj_body<NB>(a, bid);
    else if (bid < adj_blocks + p.dw.rec_blocks) rec_dw_body(p.dw.da, p.dw.act, bid - adj_blocks);
    else bwd_in_body<false>(p.dw.la, bid - adj_blocks - p.dw.rec_blocks, p.dw.lgn_blocks);
}

static void launch_bwd_in(const BwdInArgs &ia, int64_t max_units, hipStream_t s) {
    const dim3 grid(grid_subwaves(max_units, kWave));
    if (ia.cnt)
        GLIF_PROF_LAUNCH(k_bwd_in<true>, grid, dim3(kBlock), 0, s, ia);
    else
        GLIF_PROF_LAUNCH(k_bwd_in<false>, grid, dim3(kBlock), 0, s, ia);
}

static void launch_step_push(const StepArgs &sa, int step_blocks, const PushArgs &pa, int push_blocks, int nb,
                             size_t lds, hipStream_t s) {
    const dim3 grid(step_blocks + push_blocks);
    switch (nb) {
#define GLIF_STEP_PUSH(NB) \
    case NB: GLIF_PROF_LAUNCH((k_step_push<NB>), grid, dim3(kBlock), lds, s, sa, step_blocks, pa); break;
        GLIF_STEP_PUSH(1) GLIF_STEP_PUSH(2) GLIF_STEP_PUSH(3) GLIF_STEP_PUSH(4) GLIF_STEP_PUSH(5)
        GLIF_STEP_PUSH(6) GLIF_STEP_PUSH(7) GLIF_STEP_PUSH(8)
#undef GLIF_STEP_PUSH
        default: break;
    }
}

// Pull workgroups of the fused deterministic launch: all the workgroups that stay resident
// but a quarter of one per CU, so that the step's workgroups start beside the pull's (the
// pull walks a fixed share of the chunks per workgroup and its workgroups come first);
// config 2, 3 resident per CU: 2.75 per CU gave 56.3 us per tick, 2: 58.7, 2.5: 57.4, 3
// (the step behind the pull): 57.4, 1.5: 72.3, the step's workgroups first: 64.4.  0 when
// the pull is not the resident chunk form or only one workgroup fits a CU (then pull and
// step run as two launches).
static const void *pull_step_kernel(int nb) {
    switch (nb) {
        case 1: return reinterpret_cast<const void *>(&k_pull_step<1>);
        case 2: return reinterpret_cast<const void *>(&k_pull_step<2>);
        case 3: return reinterpret_cast<const void *>(&k_pull_step<3>);
        case 4: return reinterpret_cast<const void *>(&k_pull_step<4>);
        case 5: return reinterpret_cast<const void *>(&k_pull_step<5>);
        case 6: return reinterpret_cast<const void *>(&k_pull_step<6>);
        case 7: return reinterpret_cast<const void *>(&k_pull_step<7>);
        default: return reinterpret_cast<const void *>(&k_pull_step<8>);
    }
}

static int fused_pull_blocks(const PullArgs &pl, int nb) {
    if (!pull_chunked(pl) || nb < 1 || nb > kMaxBasis) return 0;
    const DevShape &ds = dev_shape();
    const size_t lb = chunk_lds_bytes(pl);
    if (ds.lds_per_cu / lb < 2) return 0;
    const int per_cu = resident_per_cu(pull_step_kernel(nb), kPullBlock, lb);
    return per_cu < 2 ? 0 : ds.n_cu * per_cu - ds.n_cu / 4;
}

static void launch_pull_step(const PullArgs &pa, int pull_blocks, const StepArgs &sa, int step_blocks, int nb,
                             size_t lds, hipStream_t s) {
    const dim3 grid(pull_blocks + step_blocks);
    switch (nb) {
#define GLIF_PULL_STEP(NB) \
    case NB: GLIF_PROF_LAUNCH((k_pull_step<NB>), grid, dim3(kPullBlock), lds, s, pa, pull_blocks, sa); break;
        GLIF_PULL_STEP(1) GLIF_PULL_STEP(2) GLIF_PULL_STEP(3) GLIF_PULL_STEP(4) GLIF_PULL_STEP(5)
        GLIF_PULL_STEP(6) GLIF_PULL_STEP(7) GLIF_PULL_STEP(8)
#undef GLIF_PULL_STEP
        default: break;
    }
}

static void launch_r_last(const StepArgs &sa, int nb, dim3 grid, size_t lds, hipStream_t s) {
    switch (nb) {
#define GLIF_R_LAST(NB) \
    case NB: hipLaunchKernelGGL((k_r_last<NB>), grid, dim3(kBlock), lds, s, sa); break;
        GLIF_R_LAST(1) GLIF_R_LAST(2) GLIF_R_LAST(3) GLIF_R_LAST(4) GLIF_R_LAST(5) GLIF_R_LAST(6) GLIF_R_LAST(7)
        GLIF_R_LAST(8)
#undef GLIF_R_LAST
        default: break;
    }
}

template <bool DET>
static void launch_step(const StepArgs &sa, int nb, dim3 grid, size_t lds, hipStream_t s) {
    switch (nb) {
#define GLIF_STEP(NB) \
    case NB: GLIF_PROF_LAUNCH((k_step<DET, NB>), grid, dim3(kBlock), lds, s, sa); break;
        GLIF_STEP(1) GLIF_STEP(2) GLIF_STEP(3) GLIF_STEP(4) GLIF_STEP(5) GLIF_STEP(6) GLIF_STEP(7) GLIF_STEP(8)
#undef GLIF_STEP
        default: break;
    }
}

constexpr size_t kAdjStageLds = 64 * 1024;  // LDS budget of the adjoint's G staging

// Types (type-major rows) or ranks (compact rows, rows = rows per post) per staged chunk of
// the adjoint: as many as fit the budget beside the basis table.
static int adj_type_chunk(const CellConst &k, int R, int rows) {
    const size_t nr = kBlock / k.B;
    const size_t basis = sizeof(float) * static_cast<size_t>(k.n_types) * k.nb;
    const size_t per_type = sizeof(float) * nr * R;
    const size_t fit = kAdjStageLds > basis ? (kAdjStageLds - basis) / per_type : 0;
    return static_cast<int>(std::max<size_t>(1, std::min<size_t>(fit, static_cast<size_t>(rows))));
}

static size_t adj_stage_lds(const CellConst &k, int R, int tc) {
    const int nr = kBlock / k.B;
    return sizeof(float) * (static_cast<size_t>(k.n_types) * k.nb + static_cast<size_t>(tc) * nr * R);
}

// prev: the weight-gradient passes (and the rest of the dz walk) of the previous window to run
// in the same launch, or null; with_adj false: those alone (after the last window)
static void launch_adj(const AdjArgs &aa, int nb, hipStream_t s, const WalkRest *prev = nullptr,
                       bool with_adj = true) {
    const CellConst &k = aa.k;
    size_t use = with_adj ? adj_stage_lds(k, aa.R, aa.tc) : 0;
    if (prev && prev->walk_blocks) use = std::max(use, sizeof(float) * (kBlock / kWave) * kGsStage);
    const int adj_blocks = with_adj ? ceil_div(k.N, kBlock / k.B) : 0;
    const dim3 grid(adj_blocks + (prev ? prev->walk_blocks + prev->dw.rec_blocks + prev->dw.lgn_blocks : 0));
    if (grid.x == 0) return;
    switch (nb) {
#define GLIF_ADJ(NB)                                                                                   \
    case NB:                                                                                           \
        if (prev) GLIF_PROF_LAUNCH((k_adj_dw<NB>), grid, dim3(kBlock), use, s, aa, adj_blocks, *prev); \
        else GLIF_PROF_LAUNCH((k_adj<NB>), grid, dim3(kBlock), use, s, aa);                           \
        break;
        GLIF_ADJ(1) GLIF_ADJ(2) GLIF_ADJ(3) GLIF_ADJ(4) GLIF_ADJ(5) GLIF_ADJ(6) GLIF_ADJ(7) GLIF_ADJ(8)
#undef GLIF_ADJ
        default: break;
    }
}

// G rows per post.  Each post's G rows serve only the synapse types that reach it; with the
// reference's basis table (a type per (presynaptic class, postsynaptic class) pair) a post
// receives about one type in eleven, so when the most types any post receives (over the
// three populations) is at most three quarters of n_types, the tables get compact rows
// (post * rows + rank) and G shrinks by that factor.  Otherwise the rows stay type-major.
static int plan_g_rows(Cell *c) {
    const int N = c->N, nt = c->n_types, words = (nt + 63) / 64;
    Table *ts[3] = {c->rec, c->lgn, c->bkg};
    c->g_rows = nt;
    c->g_compact = false;
    c->push_typed = false;
    for (int s = 0; s < nt && !c->basis_dense; ++s) {
        int nz = 0;
        for (int r = 0; r < c->nb; ++r) nz += c->rec->basis_host[static_cast<size_t>(s) * c->nb + r] != 0.0f;
        c->basis_dense = nz > 1;
    }
    if (nt > 255) return GLIF_OK;  // 0xFF marks an unused compact row
    GLIF_HIP(hipDeviceSynchronize());
    std::vector<uint32_t> ps[3];
    std::vector<uint64_t> seen(static_cast<size_t>(N) * words, 0ull);
    for (int i = 0; i < 3; ++i) {
        ps[i].resize(ts[i]->n_syn);
        if (ts[i]->n_syn)
            GLIF_HIP(hipMemcpy(ps[i].data(), ts[i]->ps, ps[i].size() * sizeof(uint32_t), hipMemcpyDeviceToHost));
        for (const uint32_t p : ps[i]) {
            const uint32_t sid = p >> 24;
            seen[static_cast<size_t>(p & kLow24) * words + sid / 64] |= 1ull << (sid % 64);
        }
    }
    int gk = 1;
    for (int n = 0; n < N; ++n) {
        int cnt = 0;
        for (int q = 0; q < words; ++q) cnt += __builtin_popcountll(seen[static_cast<size_t>(n) * words + q]);
        gk = std::max(gk, cnt);
    }
    if (gk * 4 > nt * 3) return GLIF_OK;
    auto rank_of = [&](uint32_t p) {
        const uint32_t sid = p >> 24;
        const uint64_t *sn = &seen[static_cast<size_t>(p & kLow24) * words];
        int r = 0;
        for (uint32_t q = 0; q < sid / 64; ++q) r += __builtin_popcountll(sn[q]);
        const uint64_t below = sid % 64 ? sn[sid / 64] & ((1ull << (sid % 64)) - 1ull) : 0ull;
        return static_cast<uint8_t>(r + __builtin_popcountll(below));
    };
    std::vector<uint8_t> gtype(static_cast<size_t>(N) * gk, 0xFF);
    for (int n = 0; n < N; ++n) {
        int q = 0;
        for (int sid = 0; sid < nt; ++sid)
            if ((seen[static_cast<size_t>(n) * words + sid / 64] >> (sid % 64)) & 1ull)
                gtype[static_cast<size_t>(n) * gk + q++] = static_cast<uint8_t>(sid);
    }
    for (int i = 0; i < 3; ++i) {
        std::vector<uint8_t> rank(ps[i].size());
        for (size_t k = 0; k < rank.size(); ++k) rank[k] = rank_of(ps[i][k]);
        int rc = table_set_g_rows(ts[i], rank.data(), gk);
        if (rc) return rc;
    }
    GLIF_HIP(hipMalloc(reinterpret_cast<void **>(&c->g_type), gtype.size()));
    GLIF_HIP(hipMemcpy(c->g_type, gtype.data(), gtype.size(), hipMemcpyHostToDevice));
    c->g_rows = c->g_compact_rows = gk;
    c->g_compact = true;
    c->push_typed = c->basis_dense;
    return GLIF_OK;
}

static int chunks_for(const Table *t, int L) {
    return std::max(1, ceil_div(std::max(t->max_col_len, 1), static_cast<int64_t>(L) * kChunkIters));
}

}  // namespace glif

using namespace glif;

// ------------------------------------------------------- one step's backward ----
// The gradient of one V1Column.call (models.py:1059-1135) as the reference's tape takes it
// when the Keras RNN runs the cell step by step: from the gradients of the step's outputs
// (z, v) and of its new state to those of its old state and of the three weight vectors.
// Per (b, n), with V' the step's voltage and r' its refractory counter:
//   gV'   = [r' == 0] gz psi(V' - 1) + dL/dv + dL/dv_state,  gz = dL/dz + dL/dz_buf'[slot 0]
//           (zero where r' > 0 under hard reset, whose where() cuts the path)
//   gv    = (gV' decay)(1 - vgd)                       (straight_through_dampen(v, vgd))
//   gasc_j = gasc'_j asc_decay_j + gV' cf              (c1 = sum P + sum asc, old P and asc)
//   gP_r  = gP'_r sd_r + gV' cf
//   gR_r  = gR'_r sd_r + gP'_r (dt sd_r)               (P' = P sd + (dt sd) R)
//   dy_r  = (gR'_r p0_r) lr                            (R' = R sd + (I lr) p0)
// dy then goes through the synaptic op's gradient (glif_syn_bwd): dz over all recurrent
// synapses, scaled by rd (straight_through_dampen(z_buf, 1 - rd)) and added to the shifted
// dL/dz_buf' (z_buf' = [z, z_buf[:, :-N]]), and the weight gradients of the step's events.
struct StepAdjArgs {
    CellConst k;
    const float *decay, *cf, *asc_decay;
    const float *v_new;
    const int16_t *r_new;
    const float *gz, *gv;                                   // [B][N] (nullable)
    const float *gzb_new, *gv_new, *gasc_new, *gR_new, *gP_new;  // the new state's (nullable)
    float *gv_old, *gasc_old, *gR_old, *gP_old;             // the old state's (nullable)
    float *dy;                                              // [B * N][nb]
};

__global__ void __launch_bounds__(kBlock) k_step_adj(StepAdjArgs a) {
    const CellConst &k = a.k;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<int64_t>(k.B) * k.N) return;
    const int n = static_cast<int>(i % k.N);
    const int64_t b = i / k.N;
    const bool refr = a.r_new[i] > 0;
    float gzz = a.gz ? a.gz[i] : 0.0f;
    if (a.gzb_new) gzz = gzz + a.gzb_new[b * k.D * k.N + n];
    float gV = 0.0f;
    if (!refr) {
        const float vsc = a.v_new[i] - 1.0f;
        float psi;
        if (k.pseudo_gauss) {
            const float q = -(vsc * vsc) / (k.gauss_std * k.gauss_std);
            psi = expf(q) * k.damp;
        } else {
            const float m = 1.0f - fabsf(vsc);
            psi = k.damp * (m > 0.0f ? m : 0.0f);
        }
        gV = gzz * psi;
    }
    if (a.gv) gV = gV + a.gv[i];
    if (a.gv_new) gV = gV + a.gv_new[i];
    if (k.hard_reset && refr) gV = 0.0f;
    if (a.gv_old) a.gv_old[i] = (gV * a.decay[n]) * k.om;
    const float gc = gV * a.cf[n];
    if (a.gasc_old)
        for (int j = 0; j < 2; ++j)
            a.gasc_old[i * 2 + j] = (a.gasc_new ? a.gasc_new[i * 2 + j] * a.asc_decay[n * 2 + j] : 0.0f) + gc;
    for (int q = 0; q < k.nb; ++q) {
        const int64_t e = i * k.nb + q;
        const float gRn = a.gR_new ? a.gR_new[e] : 0.0f;
        const float gPn = a.gP_new ? a.gP_new[e] : 0.0f;
        if (a.gP_old) a.gP_old[e] = gPn * k.sd[q] + gc;
        if (a.gR_old) a.gR_old[e] = gRn * k.sd[q] + gPn * k.dtsd[q];
        a.dy[e] = (gRn * k.p0[q]) * k.lr;
    }
}

// gzb[b][c] = rd * dz[b][c] + dL/dz_buf'[b][c + N] (the shifted slots; the last slot has none)
__global__ void __launch_bounds__(kBlock)
    k_step_zbuf_grad(float *__restrict__ gzb, const float *__restrict__ gzb_new, int64_t n, int64_t DN, int32_t N,
                     float rd) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float g = gzb[i] * rd;
    if (gzb_new && i % DN < DN - N) g = g + gzb_new[i + N];
    gzb[i] = g;
}

__global__ void __launch_bounds__(kBlock) k_u8_to_f32(float *__restrict__ dst, const uint8_t *__restrict__ src,
                                                        int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = static_cast<float>(src[i]);
}

struct StepWs {
    float *dy;      // [B * N][nb]
    float *xl, *xk; // the step's LGN spikes and background counts as floats
    float *G;       // the op gradients' projection, shared by the tables whose G layouts agree
};

static StepWs carve_step(void *ws, const Cell *c, int32_t B, size_t *bytes) {
    Carver cv(ws, SIZE_MAX);
    StepWs w{};
    const int64_t BN = static_cast<int64_t>(B) * c->N;
    w.dy = cv.take<float>(BN * c->nb);
    w.xl = cv.take<float>(std::max<int64_t>(static_cast<int64_t>(B) * c->lgn->n_cols, 1));
    w.xk = cv.take<float>(std::max<int64_t>(static_cast<int64_t>(B) * c->bkg->n_cols, 1));
    size_t g = 1;
    for (const Table *t : {c->rec, c->lgn, c->bkg}) g = std::max(g, syn_g_floats(t, B));
    w.G = cv.take<float>(g);
    if (bytes) *bytes = cv.off;
    return w;
}

extern "C" {

int glif_cell_create(const glif_cell_config *cfg, const float *decay, const float *current_factor,
                     const float *asc_decay, const float *asc_amps, const int32_t *t_ref_steps,
                     const float *syn_decay, const float *psc_initial, glif_table *rec, glif_table *lgn,
                     glif_table *bkg, glif_cell **out) {
    if (!cfg || !out || !rec || !lgn || !bkg || !decay || !current_factor || !asc_decay || !asc_amps ||
        !t_ref_steps || !syn_decay || !psc_initial)
        return fail(GLIF_EINVAL, "NULL argument");
    *out = nullptr;
    Table *tr = reinterpret_cast<Table *>(rec), *tl = reinterpret_cast<Table *>(lgn),
          *tb = reinterpret_cast<Table *>(bkg);
    const int N = cfg->n_neurons, D = cfg->n_delay, nb = cfg->n_basis;
    if (N <= 0 || N >= (1 << 24)) return fail(GLIF_EINVAL, "n_neurons must be in [1, 2^24)");
    if (D <= 0 || D > 256) return fail(GLIF_EINVAL, "n_delay must be in [1, 256]");
    if (nb <= 0 || nb > kMaxBasis) return fail(GLIF_EINVAL, "n_basis must be in [1, 8]");
    if (tr->n_post != N || tl->n_post != N || tb->n_post != N)
        return fail(GLIF_EINVAL, "table n_post differs from n_neurons");
    if (tr->n_slots != D || tr->n_cols != static_cast<int64_t>(D) * N)
        return fail(GLIF_EINVAL, "recurrent table must have n_delay slots of n_neurons columns");
    if (tl->n_slots != 1 || tb->n_slots != 1) return fail(GLIF_EINVAL, "input tables take no delays");
    for (Table *t : {tr, tl, tb}) {
        if (t->n_basis != nb || t->n_types != tr->n_types ||
            std::memcmp(t->basis_host, tr->basis_host, sizeof(float) * tr->n_types * nb) != 0)
            return fail(GLIF_EINVAL, "all tables must share one basis table");
    }
    for (int i = 0; i < N; ++i)
        if (t_ref_steps[i] < 1 || t_ref_steps[i] > 32767)
            return fail(GLIF_EINVAL, "t_ref_steps must be in [1, 32767]");
    Cell *c = new Cell();
    c->cfg = *cfg;
    c->N = N;
    c->Np = (N + kWave - 1) / kWave * kWave;
    c->W = c->Np / kWave;
    c->D = D;
    c->nb = nb;
    c->n_types = tr->n_types;
    for (int q = 0; q < nb; ++q) {
        c->syn_decay[q] = syn_decay[q];
        c->psc_initial[q] = psc_initial[q];
        c->dtsd[q] = cfg->dt * syn_decay[q];
    }
    c->rec = tr;
    c->lgn = tl;
    c->bkg = tb;
    auto up = [](auto **dst, const auto *src, size_t n) -> hipError_t {
        hipError_t e = hipMalloc(reinterpret_cast<void **>(dst), n * sizeof(**dst));
        if (e != hipSuccess) return e;
        return hipMemcpy(*dst, src, n * sizeof(**dst), hipMemcpyHostToDevice);
    };
    hipError_t e;
    if ((e = up(&c->decay, decay, N)) != hipSuccess || (e = up(&c->cf, current_factor, N)) != hipSuccess ||
        (e = up(&c->asc_decay, asc_decay, 2 * static_cast<size_t>(N))) != hipSuccess ||
        (e = up(&c->asc_amps, asc_amps, 2 * static_cast<size_t>(N))) != hipSuccess ||
        (e = up(&c->tref, t_ref_steps, N)) != hipSuccess) {
        glif_cell_destroy(reinterpret_cast<glif_cell *>(c));
        return hip_fail(e, "cell upload");
    }
    if (int rc = plan_g_rows(c)) {
        glif_cell_destroy(reinterpret_cast<glif_cell *>(c));
        return rc;
    }
    *out = reinterpret_cast<glif_cell *>(c);
    return GLIF_OK;
}

void glif_cell_destroy(glif_cell *cc) {
    Cell *c = reinterpret_cast<Cell *>(cc);
    if (!c) return;
    release_side(c);
    for (void *p : {static_cast<void *>(c->decay), static_cast<void *>(c->cf),
                    static_cast<void *>(c->asc_decay), static_cast<void *>(c->asc_amps),
                    static_cast<void *>(c->tref), static_cast<void *>(c->g_type)})
        if (p) (void)hipFree(p);
    delete c;
}

size_t glif_cell_workspace(const glif_cell *cc, int32_t B, int32_t T) {
    if (!cc || B <= 0 || T <= 0) return 0;
    size_t bytes = 0;
    carve_cell(nullptr, reinterpret_cast<const Cell *>(cc), B, T, &bytes);
    return bytes;
}

int glif_cell_forward(glif_cell *cc, int32_t B, int32_t T, int32_t mode, const uint8_t *lgn,
                      const uint8_t *bkg, glif_state *st, float *z_out, float *v_out,
                      int32_t *spike_count, void *ws, size_t ws_bytes, void *stream) {
    Cell *c = reinterpret_cast<Cell *>(cc);
    if (!c || !lgn || !bkg || !st || !st->z_buf || !st->v || !st->r || !st->asc || !st->psc_rise || !st->psc)
        return fail(GLIF_EINVAL, "NULL argument");
    if (B <= 0 || B > kMaxBatch) return fail(GLIF_EINVAL, "B must be in [1, 32]");
    if (T <= 0) return fail(GLIF_EINVAL, "T must be > 0");
    if (mode != GLIF_MODE_EVENT && mode != GLIF_MODE_DETERMINISTIC) return fail(GLIF_EINVAL, "unknown mode");
    if (!ws || ws_bytes < glif_cell_workspace(cc, B, T)) return fail(GLIF_ENOMEM, "workspace too small");
    hipStream_t s = static_cast<hipStream_t>(stream);
    CellWs w = carve_cell(ws, c, B, T, nullptr);
    const CellConst k = make_const(c, B);
    const bool event = mode == GLIF_MODE_EVENT;
    const Table *tr = c->rec, *tl = c->lgn, *tb = c->bkg;
    int rc;
    // event push into per-type slots ([gk][B][N] per tick) or receptor currents ([nb][B][N])
    const bool typed = event && c->push_typed;
    // LGN currents computed ahead of the loop, segment by segment, into the LGN ring: in event
    // mode the ring's slots are the current buffer the push adds to, in deterministic mode the
    // step adds them to the pulled recurrent currents.  Event mode keeps pushing the LGN
    // events where that was measured cheaper: below kLgnEventMinBatch batch entries (config 3
    // at B = 1: 16.96 against 15.88 ms per rollout) and with per-type slots, whose single LGN
    // atomic per event the launch hides (class-pair types: 61.2 against 59.8 ms per step)
    const bool ahead = lgn_ahead(c, B, T) && (!event || (!typed && B >= kLgnEventMinBatch));
    const bool ring_is_I = event && ahead;

    // input lists (LGN push in the forward, LGN / background dW in the backward)
    if (event && !ahead &&
        (rc = build_batch_mask_lists(lgn, T, B, tl->n_cols, w.lgn_off, w.lgn_pre, w.lgn_mask, w.scratch, s)))
        return rc;
    const int nseg = (T + kLgnSeg - 1) / kLgnSeg;
    // with more than one segment, each segment's LGN pass after the first runs on the cell's
    // side stream beside the previous segment's ticks (held for the rest of this call)
    std::unique_lock<std::mutex> side_lock(c->side_mu, std::defer_lock);
    bool side = false;
    if (ahead && nseg > 1) {
        side_lock.lock();
        side = ensure_side(c);
        if (!side) side_lock.unlock();
    }
    if (ahead) {
        hipLaunchKernelGGL(k_lgn_tmask, dim3(ceil_div(static_cast<int64_t>(B) * tl->n_cols, kBlock), nseg),
                           dim3(kBlock), 0, s, lgn, T, B, static_cast<int32_t>(tl->n_cols), w.lgnT);
        GLIF_HIP(hipGetLastError());
    }
    LgnRowArgs la{};
    la.T = T;
    la.N = c->N;
    la.B = B;
    la.nb = c->nb;
    la.n_types = c->n_types;
    la.n_in = static_cast<int32_t>(tl->n_cols);
    la.row = tl->row_ptr;
    la.pd = tl->pd;
    la.sid = tl->sid_row;
    la.w = tl->w_row;
    la.lgnT = w.lgnT;
    la.basis = tr->basis;
    la.ring = w.IL;
    const int Wwin = win_width(B), nwin = n_windows(T, Wwin);
    if (nwin > 0) {
        if ((rc = build_window_mask_lists(lgn, T, B, tl->n_cols, Wwin, nwin, w.lw_off, w.lw_pre, w.lw_mask,
                                          w.scratch, s)))
            return rc;
        if ((rc = build_window_mask_lists(bkg, T, B, tb->n_cols, Wwin, nwin, w.kw_off, w.kw_pre, w.kw_mask,
                                          w.scratch, s)))
            return rc;
    }
    GLIF_HIP(hipMemcpyAsync(w.bkg_cnt, bkg, static_cast<size_t>(T) * B * tb->n_cols, hipMemcpyDeviceToDevice, s));
    // spike history of the initial state
    const int64_t n_init = static_cast<int64_t>(c->D) * B * c->Np;
    if (!event && ((rc = launch_fill_u32(w.zmask, 0u, static_cast<size_t>(T + c->D) * c->Np, s)) ||
                   (rc = launch_fill_u32(w.abits, 0u, static_cast<size_t>(T + c->D) * c->W * 2, s))))
        return rc;
    hipLaunchKernelGGL(k_init_history, dim3(ceil_div(n_init, kBlock)), dim3(kBlock), 0, s, st->z_buf, k,
                       w.zbits, event ? nullptr : w.zmask,
                       event ? nullptr : w.abits);
    GLIF_HIP(hipGetLastError());
    const int slots = typed ? c->g_rows : c->nb;
    if (event && !ring_is_I && (rc = launch_fill_u32(w.I, 0u, 2 * static_cast<size_t>(B) * c->N * slots, s)))
        return rc;
    const int64_t BNs = static_cast<int64_t>(B) * c->N;
    hipLaunchKernelGGL(k_state_layout, dim3(ceil_div(BNs, kBlock)), dim3(kBlock), 0, s, st->psc_rise, st->psc,
                       st->asc, w.R, w.P, w.A, BNs, c->nb, 1);
    GLIF_HIP(hipGetLastError());

    const size_t lds = sizeof(float) * c->n_types * c->nb;
    StepArgs sa{};
    sa.k = k;
    sa.v = st->v;
    sa.r = st->r;
    sa.A = w.A;
    sa.R = w.R;
    sa.P = w.P;
    sa.decay = c->decay;
    sa.cf = c->cf;
    sa.ad = c->asc_decay;
    sa.amp = c->asc_amps;
    sa.tref = c->tref;
    sa.I = w.I;
    sa.zbits = w.zbits;
    sa.refbits = w.refbits;
    sa.zmask = w.zmask;
    sa.abits = w.abits;
    sa.vsave = w.vsave;
    sa.z_out = z_out;
    sa.v_out = v_out;
    sa.spike_count = spike_count;
    sa.count_t0 = c->trim_pre;
    sa.count_t1 = T - c->trim_post;
    sa.rec_row = tr->row_ptr;
    sa.rec_pd = tr->pd;
    sa.rec_sid = tr->sid_row;
    sa.rec_w = tr->w_row;
    sa.lgn_row = tl->row_ptr;
    sa.lgn_pd = tl->pd;
    sa.lgn_sid = tl->sid_row;
    sa.lgn_w = tl->w_row;
    sa.n_lgn = static_cast<int32_t>(tl->n_cols);
    sa.bkg_row = tb->row_ptr;
    sa.bkg_pd = tb->pd;
    sa.bkg_sid = tb->sid_row;
    sa.bkg_w = tb->w_row;
    sa.bkg_ell = tb->ell_len ? tb->ell_pw : nullptr;
    sa.bkg_ell_len = tb->ell_len;
    sa.n_bkg = static_cast<int32_t>(tb->n_cols);
    sa.basis = tr->basis;
    sa.gk = typed ? c->g_rows : 0;
    sa.gtype = c->g_type;
    sa.keep_I = ring_is_I;

    PushArgs pa{};
    pa.D = c->D;
    pa.N = c->N;
    pa.B = B;
    pa.nb = c->nb;
    pa.n_types = c->n_types;
    pa.chunks_lgn = chunks_for(tl, kWave);
    pa.d_lo = 1;
    pa.d_hi = c->D;
    pa.lgn = ahead ? 0 : 1;
    pa.zbits = w.zbits;
    pa.W = c->W;
    pa.typed = typed ? 1 : 0;
    pa.rec_colptr = tr->col_ptr;
    pa.rec_ps = typed ? tr->cg.ps : tr->ps;
    pa.rec_w = tr->w_col;
    pa.lgn_off = w.lgn_off;
    pa.lgn_pre = w.lgn_pre;
    pa.lgn_mask = w.lgn_mask;
    pa.lgn_colptr = tl->col_ptr;
    pa.lgn_ps = typed ? tl->cg.ps : tl->ps;
    pa.lgn_w = tl->w_col;
    pa.basis = tr->basis;
    pa.I = w.I;
    // Push grids (blocks of 256 that stride over the events): 2048 where a push runs alone,
    // 768 beside the step in the fused launch, which fills the rest of the chip (config 2:
    // 38.4 us per tick; 384: 40.8, 512: 39.3, 640: 38.5, 1024: 39.4, 1280: 39.5).
    const int push_grid = 2048, fused_push_grid = 768;
    const dim3 step_grid(ceil_div(static_cast<int64_t>(B) * c->Np, kBlock));

    PullArgs pl{};
    if (!event) {
        pl.N = c->N;
        pl.Np = c->Np;
        pl.os_r = BNs;
        pl.os_b = c->N;
        pl.os_n = 1;
        pl.T = T;
        pl.B = B;
        pl.D = c->D;
        pl.nb = c->nb;
        pl.n_types = c->n_types;
        pl.n_lgn = static_cast<int32_t>(tl->n_cols);
        pl.zmask = w.zmask;
        pl.lmask = w.lmask;
        pl.abits = w.abits;
        pl.lbits = w.lbits;
        pl.W = c->W;
        pl.Wl = static_cast<int32_t>((tl->n_cols + 63) / 64);
        pl.rec_row = tr->row_ptr;
        pl.rec_pd = tr->pd;
        pl.rec_sid = tr->sid_row;
        pl.rec_w = tr->w_row;
        pl.lgn_row = tl->row_ptr;
        pl.lgn_pd = tl->pd;
        pl.lgn_sid = tl->sid_row;
        pl.lgn_w = tl->w_row;
        pl.basis = tr->basis;
        pl.I = w.I;
        pl.rec_chunks = tr->n_chunks;
        pl.lgn_chunks = tl->n_chunks;
        pl.rec_pidx = tr->pidx;
        pl.lgn_pidx = tl->pidx;
        pl.rec_cdesc = tr->chunk_desc;
        pl.lgn_cdesc = tl->chunk_desc;
        pl.I2 = w.I2;
        if (ahead) {
            // the pull sums the recurrent rows only; the step adds the LGN ring's currents
            pl.lgn_chunks = 0;
            pl.lgn_row = nullptr;
            pl.Wl = 0;
        }
        // the step adds the chunk form's LGN currents (I2); k_pull writes rec + lgn to I
        sa.I2 = ahead ? w.IL : pull_chunked(pl) ? w.I2 : nullptr;
        const int64_t n_lm = static_cast<int64_t>(T) * pl.Wl * 64;
        if (n_lm > 0) {
            hipLaunchKernelGGL(k_lgn_mask, dim3(ceil_div(n_lm, kBlock)), dim3(kBlock), 0, s, lgn, T, B,
                               static_cast<int32_t>(tl->n_cols), pl.Wl, w.lmask, w.lbits);
            GLIF_HIP(hipGetLastError());
        }
    }

    // Event mode: tick t's currents accumulate in half t % 2 of I.  One launch per tick runs
    // the step of tick t - 1, whose waves push their spikes' delay-1 events, with the push of
    // tick t's delay-2..D and LGN events (which do not depend on it).
    float *Ih[2] = {w.I, w.I + static_cast<size_t>(B) * c->N * slots};
    // Deterministic mode: one launch per tick runs the row pull of tick t (into half t % 2 of
    // I and I2) beside the step of tick t, whose R takes the currents of tick t - 1.
    float *I2h[2] = {w.I2, w.I2 + BNs * c->nb};
    // With the LGN ring, tick t's currents start in ring slot t % kLgnRing (event mode: the
    // push adds onto them; deterministic mode: the step adds them to the pulled ones).
    auto ring_slot = [&](int t) { return w.IL + static_cast<size_t>(t % kLgnRing) * BNs * c->nb; };
    auto cur = [&](int t) { return ring_is_I ? ring_slot(t) : Ih[t & 1]; };
    auto lgn_cur = [&](int t) { return ahead ? ring_slot(t) : I2h[t & 1]; };
    const int pull_fused = event ? 0 : fused_pull_blocks(pl, c->nb);
    const int fused_step_blocks = static_cast<int>(ceil_div(static_cast<int64_t>(B) * c->Np, kPullBlock));
    auto step_args = [&](int t) {
        StepArgs x = sa;
        x.t = t;
        x.I = cur(t);
        x.lgn_x = lgn + static_cast<int64_t>(t) * B * tl->n_cols;
        x.bkg_x = bkg + static_cast<int64_t>(t) * B * tb->n_cols;
        return x;
    };
    for (int t = 0; t < T; ++t) {
        sa.t = t;
        sa.lgn_x = lgn + static_cast<int64_t>(t) * B * tl->n_cols;
        sa.bkg_x = bkg + static_cast<int64_t>(t) * B * tb->n_cols;
        if (ahead && t % kLgnSeg == 0) {
            const int sg = t / kLgnSeg;
            if (!side) {
                la.seg = sg;
                ProfScope p(kProfLgn, s, true);
                launch_lgn_rows(la, s);
            } else {
                if (sg == 0) {
                    la.seg = 0;
                    ProfScope p(kProfLgn, s, true);
                    launch_lgn_rows(la, s);
                } else {
                    GLIF_HIP(hipStreamWaitEvent(s, c->ev_seg[sg & 1], 0));
                }
                if (sg + 1 < nseg) {
                    // segment sg + 1 on the side stream, after every launch enqueued so far
                    GLIF_HIP(hipEventRecord(c->ev_main, s));
                    GLIF_HIP(hipStreamWaitEvent(c->side, c->ev_main, 0));
                    la.seg = sg + 1;
                    {
                        ProfScope p(kProfLgn, c->side, true);
                        launch_lgn_rows(la, c->side);
                    }
                    GLIF_HIP(hipEventRecord(c->ev_seg[(sg + 1) & 1], c->side));
                }
            }
        }
        if (event) {
            PushArgs early = pa;
            early.t = t;
            early.I = cur(t);
            if (t == 0) {
                // tick 0: every delay slot (the initial history) and the LGN inputs
                ProfScope p(kProfPush, s, true);
                GLIF_PROF_LAUNCH(k_push, dim3(push_grid), dim3(kBlock), lds, s, early);
            } else {
                early.d_lo = 2;   // d_hi = D; nothing recurrent when D = 1
                StepArgs x = step_args(t - 1);
                x.I_next = cur(t);
                x.p1_colptr = tr->col_ptr;
                x.p1_ps = typed ? tr->cg.ps : tr->ps;
                x.p1_w = tr->w_col;
                ProfScope p(kProfStep, s, true);
                launch_step_push(x, static_cast<int>(step_grid.x), early, fused_push_grid, c->nb, lds, s);
            }
            if (t == T - 1) {
                ProfScope p(kProfStep, s, true);
                launch_step<false>(step_args(t), c->nb, step_grid, lds, s);
            }
        } else if (pull_fused) {
            pl.t = t;
            pl.I = Ih[t & 1];
            pl.I2 = I2h[t & 1];
            StepArgs x = sa;
            x.lag = 1;
            x.I = Ih[(t + 1) & 1];
            x.I2 = ahead || sa.I2 ? lgn_cur(t > 0 ? t - 1 : 0) : nullptr;  // not read at t = 0
            x.bkg_x = bkg + static_cast<int64_t>(t > 0 ? t - 1 : 0) * B * tb->n_cols;
            ProfScope p(kProfStep, s, true);
            launch_pull_step(pl, pull_fused, x, fused_step_blocks, c->nb, chunk_lds_bytes(pl), s);
        } else {
            pl.t = t;
            {
                ProfScope p(kProfPush, s, true);
                launch_pull(pl, lds, s, true);   // a wave per post row above 32 (b, r) slots
            }
            StepArgs x = sa;
            if (ahead) x.I2 = ring_slot(t);
            ProfScope p(kProfStep, s, true);
            launch_step<true>(x, c->nb, step_grid, lds, s);
        }
    }
    if (pull_fused) {
        // R of the last tick
        StepArgs x = sa;
        x.t = T;
        x.lag = 1;
        x.I = Ih[(T - 1) & 1];
        x.I2 = ahead || sa.I2 ? lgn_cur(T - 1) : nullptr;
        x.bkg_x = bkg + static_cast<int64_t>(T - 1) * B * tb->n_cols;
        launch_r_last(x, c->nb, step_grid, lds, s);
    }
    GLIF_HIP(hipGetLastError());
    hipLaunchKernelGGL(k_state_layout, dim3(ceil_div(BNs, kBlock)), dim3(kBlock), 0, s, st->psc_rise, st->psc,
                       st->asc, w.R, w.P, w.A, BNs, c->nb, 0);
    GLIF_HIP(hipGetLastError());
    const int64_t n_out = static_cast<int64_t>(c->D) * B * c->N;
    hipLaunchKernelGGL(k_write_zbuf, dim3(ceil_div(n_out, kBlock)), dim3(kBlock), 0, s, st->z_buf, k, T,
                       w.zbits);
    GLIF_HIP(hipGetLastError());
    return GLIF_OK;
}

int glif_cell_backward(glif_cell *cc, int32_t B, int32_t T, const float *gz, const float *gz_neuron,
                       const float *gv, float *dw_rec, float *dw_lgn, float *dw_bkg, void *ws,
                       size_t ws_bytes, void *stream) {
    Cell *c = reinterpret_cast<Cell *>(cc);
    if (!c) return fail(GLIF_EINVAL, "NULL cell");
    if (B <= 0 || B > kMaxBatch) return fail(GLIF_EINVAL, "B must be in [1, 32]");
    if (T <= 0) return fail(GLIF_EINVAL, "T must be > 0");
    if (!ws || ws_bytes < glif_cell_workspace(cc, B, T)) return fail(GLIF_ENOMEM, "workspace too small");
    hipStream_t s = static_cast<hipStream_t>(stream);
    CellWs w = carve_cell(ws, c, B, T, nullptr);
    const CellConst k = make_const(c, B);
    const Table *tr = c->rec, *tl = c->lgn, *tb = c->bkg;
    const int64_t BN = static_cast<int64_t>(B) * c->N;
    int rc;
    if ((rc = launch_fill_u32(w.gV, 0u, BN, s)) || (rc = launch_fill_u32(w.gP, 0u, BN * c->nb, s)) ||
        (rc = launch_fill_u32(w.gR, 0u, BN * c->nb, s)))
        return rc;
    // padding elements of each G row stay zero
    const size_t g_elems = static_cast<size_t>(c->N) * c->g_rows * g_row(win_width(B), B);
    if ((rc = launch_fill_u32(w.G, 0u, 2 * g_elems, s))) return rc;
    // the grouped row-sliced walk serves 16-float G rows
    const bool cg = c->g_compact;
    const bool gs = (cg ? tr->cg.n_gs : tr->n_gs) > 0 && g_row(win_width(B), B) == 16;
    if (dw_rec && (rc = launch_fill_u32(w.dw_rec, 0u, tr->n_syn, s))) return rc;
    if (dw_lgn && (rc = launch_fill_u32(w.dw_lgn, 0u, tl->n_syn, s))) return rc;
    if (dw_bkg && (rc = launch_fill_u32(w.dw_bkg, 0u, tb->n_syn, s))) return rc;

    const int Wwin = win_width(B), ring = ring_size(c), Rg = g_row(Wwin, B);
    if (static_cast<int64_t>(c->g_rows) * c->N * Rg * 4 >= (int64_t(1) << 32))
        return fail(GLIF_ERANGE, "G rows per neuron * n_neurons * G row * 4 bytes must be < 4 GiB");
    AdjArgs aa{};
    aa.k = k;
    aa.T = T;
    aa.ring = ring;
    aa.R = Rg;
    aa.tc = adj_type_chunk(k, Rg, c->g_rows);
    aa.gk = cg ? c->g_rows : 0;
    aa.gtype = c->g_type;
    aa.vmode = c->vloss_mode;
    aa.vmask = c->vloss_mask;
    aa.vscale = c->vloss_mode ? c->vloss_cost / (static_cast<float>(T) * static_cast<float>(B) *
                                                 static_cast<float>(c->vloss_mask ? c->vloss_n : c->N))
                              : 0.0f;
    aa.vsave = w.vsave;
    aa.refbits = w.refbits;
    aa.gz = gz;
    aa.gz_neuron = gz_neuron;
    aa.gzn_t0 = c->trim_pre;
    aa.gzn_t1 = T - c->trim_post;
    aa.gv = gv;
    aa.dZ = w.dZ;
    aa.gV = w.gV;
    aa.gP = w.gP;
    aa.gR = w.gR;
    aa.decay = c->decay;
    aa.cf = c->cf;
    aa.G = w.G;
    aa.basis = tr->basis;

    // G rows of the {hi | post} entries: syn_id * N + post, or post * g_rows + rank
    const int32_t hm = cg ? 1 : c->N, lm = cg ? c->g_rows : 1;
    ColArgs ca{tr->n_cols, c->N, c->n_types, 0, tr->ph_ptr, cg ? tr->cg.ph_pw : tr->ph_pw, w.G, 1,
               dw_rec ? w.dw_rec : nullptr, nullptr, cg ? 1 : 0};
    GsArgs ga{tr->n_cols, (tr->n_cols + kGsCols - 1) / kGsCols, 0, cg ? tr->cg.gs_seg : tr->gs_seg,
              cg ? tr->cg.gs_pw : tr->gs_pw, w.G};
    RecDwArgs da{tr->n_cols, 0, hm, lm, Rg, tr->col_ptr, cg ? tr->cg.ps : tr->ps, w.G, w.dw_rec};
    ActWin act{w.zbits, w.dZ, tr->n_cols, 0, B, c->D, c->W, c->N, ring};

    BwdInArgs la{}, ka{};
    la.B = ka.B = B;
    la.R = ka.R = Rg;
    la.hm = ka.hm = hm;
    la.lm = ka.lm = lm;
    la.G = ka.G = w.G;
    la.chunks = chunks_for(tl, kWave);
    la.n_in = tl->n_cols;
    la.off = w.lw_off;
    la.pre = w.lw_pre;
    la.mask = w.lw_mask;
    la.cnt = nullptr;
    la.col_ptr = tl->col_ptr;
    la.ps = cg ? tl->cg.ps : tl->ps;
    la.dw = w.dw_lgn;
    ka.chunks = chunks_for(tb, kWave);
    ka.n_in = tb->n_cols;
    ka.off = w.kw_off;
    ka.pre = w.kw_pre;
    ka.mask = w.kw_mask;
    ka.cnt = w.bkg_cnt;
    ka.col_ptr = tb->col_ptr;
    ka.ps = cg ? tb->cg.ps : tb->ps;
    ka.dw = w.dw_bkg;
    const int64_t lgn_units = tl->n_cols * static_cast<int64_t>(la.chunks);
    const int64_t bkg_units = tb->n_cols * static_cast<int64_t>(ka.chunks);

    // With the grouped walk, the dz walk of window j covers the columns of delays <= 2 W - 3
    // (the ones window j + 1's adjoint reads, groups [0, g_split)) in its own launch, with
    // window j's weight-gradient passes (recurrent, then LGN) behind it (k_bwd_rec_gs_dw), and
    // the rest of the walk in window j + 1's adjoint launch (k_adj_dw); windows alternate
    // between two G buffers so that launch reads one while the adjoint writes the other.
    // dW in the walk's launch instead of the adjoint's: 53.4 against 53.7 ms per training step
    // at config 2 (one G buffer 21 MB).  With a larger G the dW passes' gathers over it evict the
    // slices the walk reads from the L2, and they run in window j + 1's adjoint launch instead
    // (class-pair types, 46 MB: 39.4 against 37.7 ms of backward per step beside the walk; 121
    // type-major rows, 511 MB: 108.4 against 103.3).
    const bool defer = gs && dw_rec;
    const bool dw_with_walk = defer && g_elems * sizeof(float) <= (size_t(32) << 20);
    WalkRest prev{};
    bool have_prev = false;
    const int64_t n_groups = (tr->n_cols + kGsCols - 1) / kGsCols;
    int64_t g_split = n_groups;
    if (defer) {
        const int64_t d_need = std::max(0, 2 * Wwin - 3);
        constexpr int64_t wave_groups = kWave / 4;  // g_lo of a range: whole waves of groups
        const int64_t g = (d_need * c->N + kGsCols - 1) / kGsCols;
        g_split = std::min(n_groups, (g + wave_groups - 1) / wave_groups * wave_groups);
    }
    int j = 0;
    for (int t0 = T - 1; t0 >= 2; t0 -= Wwin, ++j) {
        const int nw = std::min(Wwin, t0 - 1);
        const int s0 = t0 - 2;
        float *Gj = w.G + static_cast<size_t>(j & 1) * g_elems;
        aa.G = Gj;
        ca.G = ga.G = da.G = la.G = ka.G = Gj;
        aa.t0 = t0;
        aa.nw = nw;
        {
            ProfScope p(kProfAdj, s, true);
            launch_adj(aa, c->nb, s, have_prev ? &prev : nullptr);
        }
        ca.n_elem = ga.n_elem = da.n_elem = nw * B;
        act.s0 = s0;
        la.j = j;
        la.s0 = s0;
        {
            ProfScope p(kProfBwdRec, s, true);
            if (dw_with_walk) {
                GsArgs g1 = ga;
                g1.g_hi = g_split;
                WinDw dw{};
                dw.da = da;
                dw.act = act;
                dw.la = la;
                dw.rec_blocks = ceil_div(tr->n_cols, kBlock);
                dw.lgn_blocks = dw_lgn ? grid_subwaves(lgn_units, kWave) : 0;
                const int wb = g_split > 0 ? ceil_div(g_split * 4, kBlock) : 0;
                GLIF_PROF_LAUNCH(k_bwd_rec_gs_dw, dim3(wb + dw.rec_blocks + dw.lgn_blocks), dim3(kBlock), 0, s, g1,
                                 act, wb, dw);
            } else if (gs) {
                GsArgs g1 = ga;
                g1.g_hi = g_split;
                if (g_split > 0)
                    GLIF_PROF_LAUNCH(k_bwd_rec_gs, dim3(ceil_div(g_split * 4, kBlock)), dim3(kBlock), 0, s, g1, act);
            } else {
                launch_bwd_rec(ca, Rg, act, s);
            }
        }
        if (defer) {
            prev.act = act;
            prev.dw = WinDw{};
            if (!dw_with_walk) {
                prev.dw.da = da;
                prev.dw.act = act;
                prev.dw.la = la;
                prev.dw.rec_blocks = ceil_div(tr->n_cols, kBlock);
                prev.dw.lgn_blocks = dw_lgn ? grid_subwaves(lgn_units, kWave) : 0;
            }
            prev.gb = ga;
            prev.gb.g_lo = g_split;
            prev.walk_blocks = g_split < n_groups ? ceil_div((n_groups - g_split) * 4, kBlock) : 0;
            have_prev = true;
        } else if (dw_lgn) {
            ProfScope p(kProfBwdLgn, s, true);
            launch_bwd_in(la, lgn_units, s);
        }
        if (dw_bkg) {
            ka.j = j;
            ka.s0 = s0;
            ProfScope p(kProfBwdBkg, s, true);
            launch_bwd_in(ka, bkg_units, s);
        }
    }
    if (have_prev && prev.walk_blocks + prev.dw.rec_blocks + prev.dw.lgn_blocks > 0) {
        // the rest of the last window's dz walk (and its dW passes where they follow the adjoint)
        ProfScope p(kProfAdj, s, true);
        launch_adj(aa, c->nb, s, &prev, false);
    }
    GLIF_HIP(hipGetLastError());
    if (dw_rec && (rc = gs ? launch_perm_gather(dw_rec, w.dw_rec, tr->order_inv, tr->pinv, tr->n_syn, w.stage, s)
                           : launch_gather_f32(dw_rec, w.dw_rec, tr->ph_inv, tr->n_syn, s)))
        return rc;
    if (dw_lgn &&
        (rc = launch_perm_gather(dw_lgn, w.dw_lgn, tl->order_inv, tl->pinv, tl->n_syn, w.stage, s)))
        return rc;
    if (dw_bkg && (rc = launch_gather_f32(dw_bkg, w.dw_bkg, tb->order_inv, tb->n_syn, s))) return rc;
    return GLIF_OK;
}

int glif_cell_set_voltage_loss(glif_cell *cc, int32_t mode, float cost) {
    Cell *c = reinterpret_cast<Cell *>(cc);
    if (!c) return fail(GLIF_EINVAL, "NULL cell");
    if (mode < 0 || mode > 2) return fail(GLIF_EINVAL, "mode must be 0 (off), 1 (range) or 2 (threshold)");
    c->vloss_mode = mode;
    c->vloss_cost = cost;
    return GLIF_OK;
}

int glif_cell_set_voltage_mask(glif_cell *cc, const uint8_t *mask, int32_t n_selected) {
    Cell *c = reinterpret_cast<Cell *>(cc);
    if (!c) return fail(GLIF_EINVAL, "NULL cell");
    if (mask && (n_selected <= 0 || n_selected > c->N))
        return fail(GLIF_EINVAL, "n_selected must be in [1, n_neurons] with a mask");
    c->vloss_mask = mask;
    c->vloss_n = mask ? n_selected : c->N;
    return GLIF_OK;
}

int glif_cell_set_trim(glif_cell *cc, int32_t pre_delay, int32_t post_delay) {
    Cell *c = reinterpret_cast<Cell *>(cc);
    if (!c) return fail(GLIF_EINVAL, "NULL cell");
    if (pre_delay < 0 || post_delay < 0) return fail(GLIF_EINVAL, "pre_delay and post_delay must be >= 0");
    c->trim_pre = pre_delay;
    c->trim_post = post_delay;
    return GLIF_OK;
}

int glif_cell_set_g_layout(glif_cell *cc, int32_t compact) {
    Cell *c = reinterpret_cast<Cell *>(cc);
    if (!c) return fail(GLIF_EINVAL, "NULL cell");
    if (compact && !c->g_compact_rows)
        return fail(GLIF_EINVAL, "no compact G rows for this cell (some neuron receives > 3/4 of the types)");
    c->g_compact = compact != 0;
    c->g_rows = c->g_compact ? c->g_compact_rows : c->n_types;
    c->push_typed = c->g_compact && c->basis_dense;
    return GLIF_OK;
}

int glif_cell_g_layout(const glif_cell *cc, int32_t *rows_per_post, int32_t *compact) {
    const Cell *c = reinterpret_cast<const Cell *>(cc);
    if (!c || !rows_per_post || !compact) return fail(GLIF_EINVAL, "NULL argument");
    *rows_per_post = c->g_rows;
    *compact = c->g_compact ? 1 : 0;
    return GLIF_OK;
}

int glif_cell_voltage_loss(glif_cell *cc, int32_t B, int32_t T, float *loss_out, void *ws, size_t ws_bytes,
                           void *stream) {
    Cell *c = reinterpret_cast<Cell *>(cc);
    if (!c || !loss_out) return fail(GLIF_EINVAL, "NULL argument");
    if (c->vloss_mode == 0) return fail(GLIF_EINVAL, "voltage loss not enabled (glif_cell_set_voltage_loss)");
    if (B <= 0 || B > kMaxBatch || T <= 0) return fail(GLIF_EINVAL, "bad B or T");
    if (!ws || ws_bytes < glif_cell_workspace(cc, B, T)) return fail(GLIF_ENOMEM, "workspace too small");
    hipStream_t s = static_cast<hipStream_t>(stream);
    CellWs w = carve_cell(ws, c, B, T, nullptr);
    const int64_t n = static_cast<int64_t>(T) * B * c->N;
    hipLaunchKernelGGL(k_vloss_partial, dim3(kVlossBlocks), dim3(kBlock), 0, s, w.vsave, n, c->vloss_mode,
                       c->vloss_mask, c->N, w.vloss_part);
    const float scale =
        c->vloss_cost / static_cast<float>(c->vloss_mask ? static_cast<int64_t>(T) * B * c->vloss_n : n);
    hipLaunchKernelGGL(k_vloss_final, dim3(1), dim3(kBlock), 0, s, w.vloss_part, kVlossBlocks, scale, loss_out);
    GLIF_HIP(hipGetLastError());
    return GLIF_OK;
}

size_t glif_step_workspace(const glif_cell *cc, int32_t B) {
    const Cell *c = reinterpret_cast<const Cell *>(cc);
    if (!c || B <= 0 || B > kMaxBatch) return 0;
    size_t bytes = 0;
    carve_step(nullptr, c, B, &bytes);
    return bytes;
}

int glif_step_backward(glif_cell *cc, int32_t B, const uint8_t *lgn, const uint8_t *bkg, const float *z_buf,
                       const float *v_new, const int16_t *r_new, const float *gz, const float *gv,
                       const glif_state_grad *g_new, glif_state_grad *g_old, float *dw_rec, float *dw_lgn,
                       float *dw_bkg, void *ws, size_t ws_bytes, void *stream) {
    Cell *c = reinterpret_cast<Cell *>(cc);
    if (!c || !v_new || !r_new) return fail(GLIF_EINVAL, "NULL argument");
    if (B <= 0 || B > kMaxBatch) return fail(GLIF_EINVAL, "B must be in [1, 32]");
    const bool want_dz = g_old && g_old->z_buf;
    if ((want_dz || dw_rec) && !z_buf) return fail(GLIF_EINVAL, "z_buf is needed for dL/dz_buf and dw_rec");
    if (dw_lgn && !lgn) return fail(GLIF_EINVAL, "lgn is needed for dw_lgn");
    if (dw_bkg && !bkg) return fail(GLIF_EINVAL, "bkg is needed for dw_bkg");
    if (!ws || ws_bytes < glif_step_workspace(cc, B)) return fail(GLIF_ENOMEM, "workspace too small");
    hipStream_t s = static_cast<hipStream_t>(stream);
    StepWs w = carve_step(ws, c, B, nullptr);
    const int64_t BN = static_cast<int64_t>(B) * c->N;
    StepAdjArgs a{};
    a.k = make_const(c, B);
    a.decay = c->decay;
    a.cf = c->cf;
    a.asc_decay = c->asc_decay;
    a.v_new = v_new;
    a.r_new = r_new;
    a.gz = gz;
    a.gv = gv;
    if (g_new) {
        a.gzb_new = g_new->z_buf;
        a.gv_new = g_new->v;
        a.gasc_new = g_new->asc;
        a.gR_new = g_new->psc_rise;
        a.gP_new = g_new->psc;
    }
    if (g_old) {
        a.gv_old = g_old->v;
        a.gasc_old = g_old->asc;
        a.gR_old = g_old->psc_rise;
        a.gP_old = g_old->psc;
    }
    a.dy = w.dy;
    hipLaunchKernelGGL(k_step_adj, dim3(ceil_div(BN, kBlock)), dim3(kBlock), 0, s, a);
    GLIF_HIP(hipGetLastError());
    int rc;
    // G is built once for the step's dy and reused by every table with the same layout
    const Table *g_of = nullptr;
    auto run = [&](const Table *t, const float *x, int32_t counts, float *dz, float *dw) {
        const bool ready = g_of && same_g_layout(g_of, t);
        const int r = syn_bwd_run(t, x, w.dy, B, counts, dz, dw, w.G, ready, nullptr, s);
        if (!r && (dz || dw)) g_of = t;
        return r;
    };
    if ((want_dz || dw_rec) && (rc = run(c->rec, z_buf, 0, want_dz ? g_old->z_buf : nullptr, dw_rec))) return rc;
    if (want_dz) {
        const int64_t DN = static_cast<int64_t>(c->D) * c->N, n = static_cast<int64_t>(B) * DN;
        hipLaunchKernelGGL(k_step_zbuf_grad, dim3(ceil_div(n, kBlock)), dim3(kBlock), 0, s, g_old->z_buf,
                           g_new ? g_new->z_buf : nullptr, n, DN, c->N, a.k.rd_scale);
        GLIF_HIP(hipGetLastError());
    }
    if (dw_lgn) {
        const int64_t n = static_cast<int64_t>(B) * c->lgn->n_cols;
        if (n) hipLaunchKernelGGL(k_u8_to_f32, dim3(ceil_div(n, kBlock)), dim3(kBlock), 0, s, w.xl, lgn, n);
        if ((rc = run(c->lgn, w.xl, 0, nullptr, dw_lgn))) return rc;
    }
    if (dw_bkg) {
        const int64_t n = static_cast<int64_t>(B) * c->bkg->n_cols;
        if (n) hipLaunchKernelGGL(k_u8_to_f32, dim3(ceil_div(n, kBlock)), dim3(kBlock), 0, s, w.xk, bkg, n);
        if ((rc = run(c->bkg, w.xk, 1, nullptr, dw_bkg))) return rc;
    }
    GLIF_HIP(hipGetLastError());
    return GLIF_OK;
}

}  // extern "C"
