// One mode of the CU-balanced multi-token CB3 kernels, compiled once per mode by build.py with
// -DMI_UMODE=<0 gate/up | 1 down>; exports launch_cumulti_<mode>, dispatching over the rows per wavefront (16 RTW)
// and, for down, the one- or two-instruction form of h.
#include "cumulti.h"

#ifndef MI_UMODE
#error "MI_UMODE must be defined"
#endif

namespace mi {

#define MI_UNAME2(P, M) P##_##M
#define MI_UNAME(P, M) MI_UNAME2(P, M)

template <bool TWO>
static void launch(int rtw, dim3 grid, size_t lds, hipStream_t s, const MArgs &a) {
    const dim3 block(64 * kCuWaves);
    if (rtw == 1) hipLaunchKernelGGL((cumulti_kernel<MI_UMODE, 1, TWO>), grid, block, lds, s, a);
    else if (rtw == 2) hipLaunchKernelGGL((cumulti_kernel<MI_UMODE, 2, TWO>), grid, block, lds, s, a);
    else hipLaunchKernelGGL((cumulti_kernel<MI_UMODE, 4, TWO>), grid, block, lds, s, a);
}

void MI_UNAME(launch_cumulti, MI_UMODE)(int rtw, dim3 grid, size_t lds, hipStream_t s, const MArgs &a) {
#if MI_UMODE == 1
    if (a.N > 8) {
        launch<true>(rtw, grid, lds, s, a);
        return;
    }
#endif
    launch<false>(rtw, grid, lds, s, a);
}

}  // namespace mi
