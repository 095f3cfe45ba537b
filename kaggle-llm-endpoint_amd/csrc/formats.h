// The reference's planar IQ3_S tables as the gfx950 kernels address them (the decoders: iq3_mfma.h for decode and
// matvec, prefill.hip for the prefill GEMMs).
#pragma once
#include "common.h"

namespace mi {

__device__ __forceinline__ uint4 ldl(const uint32_t *__restrict__ base, uint32_t lane_off) {
    // wave-uniform base (SGPRs) + the lane's row offset in 32 bits (rows < 2^30): the scalar-base addressing form
    return *(const uint4 *)((const char *)base + (lane_off << 2));
}

// ------------------------------------------------------------------------------------------------ IQ3_S
// The reference's planar IQ3_S tables (planes.py:22-25): word w of a row covers inputs 16w .. 16w+15, group
// j = 0..3 of the word covers 4 inputs 16w+4j .. 16w+4j+3.
struct Iq3Table {
    const uint32_t *qs, *sg, *qh, *sc, *d;
    int R, K, nblk, W;
    static constexpr int kUnitCols = 256;   // one 256-weight block
};

}  // namespace mi
