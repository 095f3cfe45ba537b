// One (mode, format) instantiation set of the grouped kernels, compiled once per combination by build.py with
// -DMI_KMODE=<0 gate/up, 1 down, 2 matvec> -DMI_KQT=<1 CB3, 2 IQ3_S>; exports launch_grouped_<mode>_<qt>.
#include "grouped.h"

#ifndef MI_KMODE
#error "MI_KMODE must be defined"
#endif
#ifndef MI_KQT
#error "MI_KQT must be defined"
#endif

namespace mi {

#define MI_LAUNCH_NAME2(M, Q) launch_grouped_##M##_##Q
#define MI_LAUNCH_NAME(M, Q) MI_LAUNCH_NAME2(M, Q)
#define MI_OCC_NAME2(M, Q) occupancy_grouped_##M##_##Q
#define MI_OCC_NAME(M, Q) MI_OCC_NAME2(M, Q)

template <int TC>
static int occ_of(size_t lds) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, (const void *)grouped_kernel<MI_KMODE, MI_KQT, TC>,
                                                     64 * kWgWaves, lds) != hipSuccess)
        return 0;
    return n;
}

// Resident workgroups per CU of the instance a launch with this token class and dynamic LDS would use (0: unknown).
int MI_OCC_NAME(MI_KMODE, MI_KQT)(int tcmax, size_t lds) {
#if MI_KQT == MI_QT_CB3
    return tcmax <= 8 ? occ_of<8>(lds) : occ_of<16>(lds);
#else
    switch (tcmax) {
        case 1: return occ_of<1>(lds);
        case 2: return occ_of<2>(lds);
        case 4: return occ_of<4>(lds);
        case 8: return occ_of<8>(lds);
        default: return occ_of<16>(lds);
    }
#endif
}

void MI_LAUNCH_NAME(MI_KMODE, MI_KQT)(int tcmax, dim3 grid, dim3 block, size_t lds, hipStream_t s, const KArgs &a) {
#if MI_KQT == MI_QT_CB3
    // matrix-core path: every token class shares one 16-column tile; only groups of more than 8 tokens with f32
    // activations need the two-instruction variant
    if (tcmax <= 8) hipLaunchKernelGGL((grouped_kernel<MI_KMODE, MI_KQT, 8>), grid, block, lds, s, a);
    else hipLaunchKernelGGL((grouped_kernel<MI_KMODE, MI_KQT, 16>), grid, block, lds, s, a);
#else
    switch (tcmax) {
        case 1: hipLaunchKernelGGL((grouped_kernel<MI_KMODE, MI_KQT, 1>), grid, block, lds, s, a); break;
        case 2: hipLaunchKernelGGL((grouped_kernel<MI_KMODE, MI_KQT, 2>), grid, block, lds, s, a); break;
        case 4: hipLaunchKernelGGL((grouped_kernel<MI_KMODE, MI_KQT, 4>), grid, block, lds, s, a); break;
        case 8: hipLaunchKernelGGL((grouped_kernel<MI_KMODE, MI_KQT, 8>), grid, block, lds, s, a); break;
        default: hipLaunchKernelGGL((grouped_kernel<MI_KMODE, MI_KQT, 16>), grid, block, lds, s, a); break;
    }
#endif
}

}  // namespace mi
