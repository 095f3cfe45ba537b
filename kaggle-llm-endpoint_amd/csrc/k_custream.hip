// One mode of the CU-balanced single-token CB3 kernels, compiled once per mode by build.py with
// -DMI_CMODE=<0 gate/up | 1 down>; exports launch_custream_<mode>, dispatching over the rows per wavefront (16 RTW).
#include "custream.h"

#ifndef MI_CMODE
#error "MI_CMODE must be defined"
#endif

namespace mi {

#define MI_CNAME2(P, M) P##_##M
#define MI_CNAME(P, M) MI_CNAME2(P, M)

void MI_CNAME(launch_custream, MI_CMODE)(int rtw, dim3 grid, size_t lds, hipStream_t s, const CArgs &a) {
    const dim3 block(64 * cu_waves<MI_CMODE>());
    if (rtw == 1) hipLaunchKernelGGL((custream_kernel<MI_CMODE, 1>), grid, block, lds, s, a);
    else if (rtw == 2) hipLaunchKernelGGL((custream_kernel<MI_CMODE, 2>), grid, block, lds, s, a);
    else hipLaunchKernelGGL((custream_kernel<MI_CMODE, 4>), grid, block, lds, s, a);
}

}  // namespace mi
