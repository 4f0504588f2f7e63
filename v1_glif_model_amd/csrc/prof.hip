// Optional per-kernel timing with HIP events recorded on the launch stream.
// Off by default; when a kernel class is enabled every launch of it (or every n-th,
// glif_prof_stride, so that classes launched once per timestep are sampled without the
// host cost of two event records per launch) is bracketed by two events and
// glif_prof_collect() sums the elapsed times.
#include <mutex>
#include <vector>

#include "glif_internal.h"
#include "prof.h"

namespace glif {

namespace {
struct Rec {
    int kind;
    hipEvent_t a, b;
};
std::mutex g_mu;
uint32_t g_mask = 0;
int32_t g_every = 1;                // bracket every g_every-th launch of an enabled class
int64_t g_seq[kProfKinds] = {};     // launches of each class seen while enabled
std::vector<Rec> g_recs;
std::vector<hipEvent_t> g_pool;
double g_total[kProfKinds] = {};
int64_t g_count[kProfKinds] = {};

hipEvent_t get_event() {
    if (!g_pool.empty()) {
        hipEvent_t e = g_pool.back();
        g_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}
}  // namespace

const char *const kProfNames[kProfKinds] = {"push", "step", "adj", "bwd_rec", "bwd_lgn", "bwd_bkg",
                                            "syn_fwd", "syn_bwd", "lgn"};

namespace {
thread_local hipEvent_t t_pend_a = nullptr, t_pend_b = nullptr;  // a one-launch scope's pair
thread_local bool t_taken = false;
}  // namespace

void prof_take(hipEvent_t *a, hipEvent_t *b) {
    *a = t_pend_a;
    *b = t_pend_b;
    if (t_pend_a) t_taken = true;
    t_pend_a = t_pend_b = nullptr;
}

ProfScope::ProfScope(int kind, hipStream_t s, bool one_launch) : kind_(kind), s_(s), one_(one_launch) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!(g_mask & (1u << kind))) return;
    if (g_seq[kind]++ % g_every != 0) return;
    a_ = get_event();
    b_ = get_event();
    if (!a_ || !b_) {
        a_ = b_ = nullptr;
        return;
    }
    if (one_) {
        t_pend_a = a_;
        t_pend_b = b_;
        t_taken = false;
    } else if (hipEventRecord(a_, s_) != hipSuccess) {
        a_ = nullptr;
    }
}

ProfScope::~ProfScope() {
    if (!a_ || !b_) return;
    std::lock_guard<std::mutex> lk(g_mu);
    if (one_) {
        const bool taken = t_taken;
        t_pend_a = t_pend_b = nullptr;
        t_taken = false;
        if (taken) g_recs.push_back({kind_, a_, b_});
        else {  // nothing was launched: the pair goes back unused
            g_pool.push_back(a_);
            g_pool.push_back(b_);
        }
        return;
    }
    if (hipEventRecord(b_, s_) == hipSuccess) g_recs.push_back({kind_, a_, b_});
}

}  // namespace glif

using namespace glif;

extern "C" {

int glif_prof_enable(uint32_t mask) {
    std::lock_guard<std::mutex> lk(g_mu);
    g_mask = mask;
    for (int64_t &q : g_seq) q = 0;
    return GLIF_OK;
}

int glif_prof_stride(int32_t every) {
    if (every < 1) return fail(GLIF_EINVAL, "every must be >= 1");
    std::lock_guard<std::mutex> lk(g_mu);
    g_every = every;
    return GLIF_OK;
}

int glif_prof_collect(double *total_ms, int64_t *count, int32_t n) {
    std::lock_guard<std::mutex> lk(g_mu);
    for (Rec &r : g_recs) {
        if (hipEventSynchronize(r.b) != hipSuccess) continue;
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, r.a, r.b) == hipSuccess) {
            g_total[r.kind] += ms;
            g_count[r.kind] += 1;
        }
        g_pool.push_back(r.a);
        g_pool.push_back(r.b);
    }
    g_recs.clear();
    for (int i = 0; i < n && i < kProfKinds; ++i) {
        if (total_ms) total_ms[i] = g_total[i];
        if (count) count[i] = g_count[i];
        g_total[i] = 0.0;
        g_count[i] = 0;
    }
    return GLIF_OK;
}

const char *glif_prof_name(int32_t kind) {
    return (kind >= 0 && kind < kProfKinds) ? kProfNames[kind] : "";
}

}  // extern "C"
