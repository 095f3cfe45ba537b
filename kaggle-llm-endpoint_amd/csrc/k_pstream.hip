// One (mode, token class) instantiation set of the persistent grouped CB3 kernels, compiled once per combination by
// build.py with -DMI_PMODE=<0 gate/up | 1 down> -DMI_PTC=<8|16>; exports launch_pstream_<mode>_<tc> and
// occupancy_pstream_<mode>_<tc>, each dispatching over the rows per wavefront (1, 2 or 4 row tiles).
#include "pstream.h"

#ifndef MI_PMODE
#error "MI_PMODE must be defined"
#endif
#ifndef MI_PTC
#error "MI_PTC must be defined"
#endif

namespace mi {

#define MI_PNAME2(P, M, T) P##_##M##_##T
#define MI_PNAME(P, M, T) MI_PNAME2(P, M, T)

template <int RTW>
static int occ_of(size_t lds) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, (const void *)pstream_kernel<MI_PMODE, MI_PTC, RTW>,
                                                     64 * kWgWaves, lds) != hipSuccess)
        return 0;
    return n;
}

int MI_PNAME(occupancy_pstream, MI_PMODE, MI_PTC)(int rtw, size_t lds) {
    return rtw == 1 ? occ_of<1>(lds) : rtw == 2 ? occ_of<2>(lds) : occ_of<4>(lds);
}

void MI_PNAME(launch_pstream, MI_PMODE, MI_PTC)(int rtw, dim3 grid, size_t lds, hipStream_t s, const PArgs &a) {
    const dim3 block(64 * kWgWaves);
    if (rtw == 1) hipLaunchKernelGGL((pstream_kernel<MI_PMODE, MI_PTC, 1>), grid, block, lds, s, a);
    else if (rtw == 2) hipLaunchKernelGGL((pstream_kernel<MI_PMODE, MI_PTC, 2>), grid, block, lds, s, a);
    else hipLaunchKernelGGL((pstream_kernel<MI_PMODE, MI_PTC, 4>), grid, block, lds, s, a);
}

}  // namespace mi
