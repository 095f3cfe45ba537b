// One (mode, format) instantiation set of the grouped kernels, compiled once per combination by build.py with
// -DMI_KMODE=<0 gate/up, 1 down, 2 matvec> -DMI_KQT=<1 CB3, 2 IQ3_S, 3 IQ4_XS, 4 IQ2_S, 5 Q2_K, 6 Q3_K>;
// exports launch_grouped_<mode>_<qt>.
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

template <int TC, int RTW>
static int occ_of(size_t lds) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, (const void *)grouped_kernel<MI_KMODE, MI_KQT, TC, RTW>,
                                                     64 * kWgWaves, lds) != hipSuccess)
        return 0;
    return n;
}

template <int TC, int RTW>
static void launch(dim3 grid, dim3 block, size_t lds, hipStream_t s, const KArgs &a) {
    hipLaunchKernelGGL((grouped_kernel<MI_KMODE, MI_KQT, TC, RTW>), grid, block, lds, s, a);
}

#if MI_KQT == MI_QT_CB3
// matrix-core path: every token class shares one 16-column tile; only groups of more than 8 tokens with f32
// activations need the two-instruction variant.  RTW: row tiles per wavefront (1, 2 or 4).
#define MI_CB3_DISPATCH(F, ...)                                                                       \
    if (tcmax <= 8) {                                                                               \
        if (rtw == 1) return F<8, 1>(__VA_ARGS__);                                                   \
        if (rtw == 2) return F<8, 2>(__VA_ARGS__);                                                   \
        return F<8, 4>(__VA_ARGS__);                                                                 \
    }                                                                                               \
    if (rtw == 1) return F<16, 1>(__VA_ARGS__);                                                      \
    if (rtw == 2) return F<16, 2>(__VA_ARGS__);                                                      \
    return F<16, 4>(__VA_ARGS__);
#endif

// Resident workgroups per CU of the instance a launch would use (0: unknown).
int MI_OCC_NAME(MI_KMODE, MI_KQT)(int tcmax, int rtw, size_t lds) {
#if MI_KQT == MI_QT_CB3
    MI_CB3_DISPATCH(occ_of, lds)
#else
    (void)rtw;
    switch (tcmax) {
        case 1: return occ_of<1, 1>(lds);
        case 2: return occ_of<2, 1>(lds);
        case 4: return occ_of<4, 1>(lds);
        case 8: return occ_of<8, 1>(lds);
        default: return occ_of<16, 1>(lds);
    }
#endif
}

void MI_LAUNCH_NAME(MI_KMODE, MI_KQT)(int tcmax, int rtw, dim3 grid, dim3 block, size_t lds, hipStream_t s,
                                     const KArgs &a) {
#if MI_KQT == MI_QT_CB3
    MI_CB3_DISPATCH(launch, grid, block, lds, s, a)
#else
    (void)rtw;
    switch (tcmax) {
        case 1: return launch<1, 1>(grid, block, lds, s, a);
        case 2: return launch<2, 1>(grid, block, lds, s, a);
        case 4: return launch<4, 1>(grid, block, lds, s, a);
        case 8: return launch<8, 1>(grid, block, lds, s, a);
        default: return launch<16, 1>(grid, block, lds, s, a);
    }
#endif
}

}  // namespace mi
