// Instantiations of the one-launch CB3 decode layer (fused_decode.h): 32 or 64 rows per wavefront in both phases;
// exports launch_fused and occupancy_fused.
#include "fused_decode.h"

namespace mi {

template <int RTW>
static int occ_of(size_t lds) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, (const void *)fused_decode_kernel<RTW>, 64 * kWgWaves, lds) !=
        hipSuccess)
        return 0;
    return n;
}

int occupancy_fused(int rtw, size_t lds) { return rtw == 2 ? occ_of<2>(lds) : occ_of<4>(lds); }

void launch_fused(int rtw, dim3 grid, size_t lds, hipStream_t s, const FArgs &a) {
    const dim3 block(64 * kWgWaves);
    if (rtw == 2) hipLaunchKernelGGL((fused_decode_kernel<2>), grid, block, lds, s, a);
    else hipLaunchKernelGGL((fused_decode_kernel<4>), grid, block, lds, s, a);
}

}  // namespace mi
