// Per-kernel event timing (prof.hip).
#pragma once
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
    kProfKinds
};

// Brackets the launches issued during its lifetime with two events on `s` when
// the kind is enabled (glif_prof_enable).
class ProfScope {
  public:
    ProfScope(int kind, hipStream_t s);
    ~ProfScope();
    ProfScope(const ProfScope &) = delete;
    ProfScope &operator=(const ProfScope &) = delete;

  private:
    int kind_;
    hipStream_t s_;
    hipEvent_t a_ = nullptr, b_ = nullptr;
};

}  // namespace glif
