// Per-kernel event timing (prof.hip).
#pragma once
#include <hip/hip_ext.h>

#include "glif_internal.h"

namespace glif {

enum ProfKind {
    kProfPush = 0,
    kProfStep,
    kProfAdj,
    kProfBwdRec,
    kProfBwdLgn,
    kProfBwdBkg,
    kProfSynFwd,
    kProfSynBwd,
    kProfLgn,
    kProfKinds
};

// Times the launches issued during its lifetime when the kind is enabled (glif_prof_enable)
// and this launch is sampled (glif_prof_stride): with two events recorded on `s` around
// them, or, for a scope made with one_launch = true around a single GLIF_PROF_LAUNCH, with
// the events passed into that launch's dispatch (hipExtLaunchKernel), which time the kernel
// alone, without the dispatch gap an event record before the launch would include.
class ProfScope {
  public:
    ProfScope(int kind, hipStream_t s, bool one_launch = false);
    ~ProfScope();
    ProfScope(const ProfScope &) = delete;
    ProfScope &operator=(const ProfScope &) = delete;

  private:
    int kind_;
    hipStream_t s_;
    bool one_ = false;
    hipEvent_t a_ = nullptr, b_ = nullptr;
};

// The event pair a one-launch ProfScope of this thread hands to its launch (nullptrs when
// there is none or it was taken).
void prof_take(hipEvent_t *a, hipEvent_t *b);

}  // namespace glif

// A launch that carries the pending one-launch ProfScope's events, if any.
#define GLIF_PROF_LAUNCH(kernel, grid, block, lds, stream, ...)                                      \
    do {                                                                                          \
        hipEvent_t glif_pa_ = nullptr, glif_pb_ = nullptr;                                        \
        ::glif::prof_take(&glif_pa_, &glif_pb_);                                                  \
        if (glif_pa_)                                                                             \
            hipExtLaunchKernelGGL(kernel, grid, block, lds, stream, glif_pa_, glif_pb_, 0, __VA_ARGS__); \
        else                                                                                      \
            hipLaunchKernelGGL(kernel, grid, block, lds, stream, __VA_ARGS__);                    \
    } while (0)
