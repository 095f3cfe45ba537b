// The reference's planar IQ2_S, IQ3_S and IQ4_XS tables as the gfx950 kernels address them (the decoders:
// iq2_mfma.h, iq3_mfma.h and iq4_mfma.h for decode and matvec, prefill.hip for the prefill GEMMs).
#pragma once
#include "common.h"

namespace mi {

#ifndef MI_IQ_NT
#define MI_IQ_NT 1
#endif
__device__ __forceinline__ uint4 ldl(const uint32_t *__restrict__ base, uint32_t lane_off) {
    // wave-uniform base (SGPRs) + the lane's row offset in 32 bits (rows < 2^30): the scalar-base addressing form;
    // the decoders read every plane word once: non-temporal loads
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 *p = (const u32x4 *)((const char *)base + (lane_off << 2));
    if constexpr (MI_IQ_NT) return __builtin_bit_cast(uint4, __builtin_nontemporal_load(p));
    else return __builtin_bit_cast(uint4, *p);
}

// ldl's 16 bytes when `use` (wave-uniform), else zeros: a buffer load through a descriptor whose range is empty
// when unused returns zeros without touching memory, so no branch surrounds the load.  (A load under a branch
// makes the compiler wait for every load in flight where the branch rejoins: in the decoders' loops that drained
// the next half-block's prefetched words at every half-block.)  NT: non-temporal (words read once); the scale and
// d words, read again by the next half-block, keep the default policy.
template <bool NT = MI_IQ_NT>
__device__ __forceinline__ uint4 ldl_if(const uint32_t *base, uint32_t lane_off, bool use) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, use ? 0x7fffffff : 0, 0x00020000);
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)(lane_off << 2), 0, NT ? 2 : 0));
}

// ------------------------------------------------------------------------------------------------ IQ3_S
// The reference's planar IQ3_S tables (planes.py:22-25): word w of a row covers inputs 16w .. 16w+15, group
// j = 0..3 of the word covers 4 inputs 16w+4j .. 16w+4j+3.
struct Iq3Table {
    const uint32_t *qs, *sg, *qh, *sc, *d;
    int R, K, nblk, W;
    static constexpr int kUnitCols = 256;   // one 256-weight block
};

// The reference's planar IQ4_XS tables (planes.py:26-28): word w = qs bytes 4w .. 4w+3 of a row; byte j holds input
// 32 (w/4) + 4 (w%4) + j in its low nibble and that + 16 in its high nibble; per block one u32 of low scale nibbles
// (sl), one of high scale bit pairs (sh) and, per two blocks, one u32 of f16 d.
struct Iq4Table {
    const uint32_t *qs, *sl, *sh, *d;
    int R, K, nblk, W;                      // W = 32 nblk words per row
    static constexpr int kUnitCols = 256;
};

// The reference's planar IQ2_S tables (planes.py:17-21): word w of a row covers inputs 32w .. 32w+31, byte j of the
// qs and sg words is group j = inputs 32w+8j .. 32w+8j+7 (low index bits, signs); byte w%4 of qh / sc u32 w/4 holds
// the word's high index bits (2 per group) and its two 4-bit scales (one per 16 inputs).
struct Iq2Table {
    const uint32_t *qs, *sg, *qh, *sc, *d;
    int R, K, nblk, W;                      // W = 8 nblk words per row
    static constexpr int kUnitCols = 256;
};

// The reference's planar K-quant tables (planes.py:34-41): qs u32 [16 nblk, R] (word w: byte j holds the 2-bit values
// of inputs 256 b + 128 n + 32 s + 4 (w % 8) + j at shift 2s, b = w / 16, n = (w % 16) / 8); sc u32 [4 nblk, R]
// (the block's 16 scale bytes); d u32 [nblk, R] (f16 d | f16 dmin << 16 for Q2_K); Q3_K also hm u32 [8 nblk, R]
// (the hmask bytes: bit 4n + s of byte l).
struct KqTable {
    const uint32_t *qs, *sc, *d, *hm;       // hm: Q3_K only
    int R, K, nblk;
    static constexpr int kUnitCols = 256;
};

}  // namespace mi
