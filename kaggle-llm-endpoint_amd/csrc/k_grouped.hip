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

void MI_LAUNCH_NAME(MI_KMODE, MI_KQT)(int tcmax, dim3 grid, dim3 block, size_t lds, hipStream_t s, const KArgs &a) {
    switch (tcmax) {
        case 1: hipLaunchKernelGGL((grouped_kernel<MI_KMODE, MI_KQT, 1>), grid, block, lds, s, a); break;
        case 2: hipLaunchKernelGGL((grouped_kernel<MI_KMODE, MI_KQT, 2>), grid, block, lds, s, a); break;
        case 4: hipLaunchKernelGGL((grouped_kernel<MI_KMODE, MI_KQT, 4>), grid, block, lds, s, a); break;
        case 8: hipLaunchKernelGGL((grouped_kernel<MI_KMODE, MI_KQT, 8>), grid, block, lds, s, a); break;
        default: hipLaunchKernelGGL((grouped_kernel<MI_KMODE, MI_KQT, 16>), grid, block, lds, s, a); break;
    }
}

}  // namespace mi
