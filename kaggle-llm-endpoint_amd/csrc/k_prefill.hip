// One (mode, form) instantiation set of the prefill GEMMs, compiled once per combination by build.py with
// -DMI_PF_MODE=<0 gate/up, 1 down> -DMI_PF_FORM=<kPf* rounding-form bits>; exports launch_prefill_<mode>_<form>.
#include "prefill_gemm.h"

#ifndef MI_PF_MODE
#error "MI_PF_MODE must be defined"
#endif
#ifndef MI_PF_FORM
#error "MI_PF_FORM must be defined"
#endif

namespace mi {

#define MI_PF_NAME2(M, F) launch_prefill_##M##_##F
#define MI_PF_NAME(M, F) MI_PF_NAME2(M, F)

int MI_PF_NAME(MI_PF_MODE, MI_PF_FORM)(int qtype, dim3 grid, hipStream_t s, const PfArgs &a) {
    return launch_prefill<MI_PF_MODE, MI_PF_FORM>(qtype, grid, s, a);
}

}  // namespace mi
