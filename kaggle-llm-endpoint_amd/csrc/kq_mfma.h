// Q2_K and Q3_K rows (the MTP layer's experts) of the grouped decode / matvec launches on the gfx950 matrix cores.
//
// The reference's planar K-quant tables (planes.py:34-41,136-170) are read as stored: word w of a row = 4 qs bytes;
// block b = w / 16, half n = (w % 16) / 8, q' = w % 8; byte j of the word holds the 2-bit values of inputs
// 256 b + 128 n + 32 s + 4 q' + j at shift 2s.  A k-step is one 32-column stripe (b, n, s): lane group q holds words
// q' = 2q and 2q + 1 of the half at shift s, i.e. columns 32 s + 8 q .. 32 s + 8 q + 7 of the half in natural order.
// The 2-bit values (Q3_K: with the hmask bit as bit 2) become bf16 levels through byte-table v_perm lookups, exact
// (Q2_K: v in 0..3; Q3_K: v - 4 + 4 hbit in -4..3).  A stripe spans two 16-weight scale groups (lane groups 0, 1 and
// 2, 3): as for IQ2_S every k-step runs twice with the other group's activations read as zeros, and each partial takes
// its rows' f32 scale (Q2_K d * sc, Q3_K d * (sc - 32), exact).  Q2_K's min term, -dmin * m * sum(x over the group),
// takes the group sums from one more pair of matrix-core steps against a ones operand, shared by the 4 row tiles.
// Q3_K weights are exact in f32; a Q2_K weight d*sc*v - dmin*m is rounded once by the reference (iqquant.py:213):
// here its two exact terms enter separately (a difference of ~1 ulp of the weight).
#pragma once
#include "iq3_mfma.h"

namespace mi {

struct KqLds {
    uint4 zero[16];        // the zeroed activations of the lane groups outside a k-step's scale group
};

__device__ __forceinline__ void kq_fill_lds(KqLds &t) {
    if (threadIdx.x < 16) t.zero[threadIdx.x] = make_uint4(0, 0, 0, 0);
}

// Level byte tables for v_perm: entry x (0..7) -> the low / high byte of bf16(level(x)).
//   Q2_K: level(x) = x (x = 0..3);  Q3_K: level(x) = x - 4 (x = v + 4 hbit = 0..7)
template <bool Q3>
struct KqLevels {
    static constexpr uint32_t lo0 = Q3 ? 0x80004080u : 0x40008000u, lo1 = Q3 ? 0x40008000u : 0u;
    static constexpr uint32_t hi0 = Q3 ? 0xBFC0C0C0u : 0x40403F00u, hi1 = Q3 ? 0x40403F00u : 0u;
};

// the 4 byte-sized indices of t -> their 4 bf16 levels (two dwords, index 0 in the low half of the first)
template <bool Q3>
__device__ __forceinline__ uint2 kq_levels(uint32_t t) {
    using T = KqLevels<Q3>;
    const uint32_t L = perm(T::lo1, T::lo0, t), H = perm(T::hi1, T::hi0, t);
    return make_uint2(perm(H, L, 0x05010400u), perm(H, L, 0x07030602u));
}

template <bool TWO, bool Q3, class Stage>
__device__ __forceinline__ void kqm_accum(const KqTable &tb, int e, int row0, int u0, int u1, int c0, const KqLds &L,
                                          const uint32_t *xa, const uint32_t *xb, f32x4 (&acc)[4], Stage &&stage) {
    const int lane = threadIdx.x & 63, q = lane >> 4;
    const size_t R = (size_t)tb.R;
    const int nblk = tb.nblk;
    const uint32_t lo = (uint32_t)(row0 + 4 * (lane & 15));
    const uint32_t *qs = tb.qs + (size_t)e * (16 * nblk) * R;
    const uint32_t *sc = tb.sc + (size_t)e * (4 * nblk) * R;
    const uint32_t *dd = tb.d + (size_t)e * nblk * R;
    const uint32_t *hm = Q3 ? tb.hm + (size_t)e * (8 * nblk) * R : nullptr;   // Q3_K only
    const bool first = q < 2;
    const uint4 z4 = make_uint4(0, 0, 0, 0);
    // half-blocks h = 2 b + n: qs words 8h + 2q, 8h + 2q + 1; sc rows 2h, 2h + 1 (scale bytes 8n .. 8n + 7 of block
    // b); d row b; hm rows 8b + 2q, 8b + 2q + 1 (the hmask bytes of columns 4 q' + j, both halves)
    const int h0 = 2 * u0, h1 = 2 * u1;
    // the lane's words (2 q, 2 q + 1) go into its offsets: a buffer load's descriptor must be wave-uniform
    const uint32_t lo_a = lo + (uint32_t)(2 * q * R), lo_b = lo_a + (uint32_t)R;
    uint4 qa = ldl(qs + (size_t)(8 * h0 + 2 * q) * R, lo), qb = ldl(qs + (size_t)(8 * h0 + 2 * q + 1) * R, lo);
    uint4 sa = ldl(sc + (size_t)(2 * h0) * R, lo), sb = ldl(sc + (size_t)(2 * h0 + 1) * R, lo);
    uint4 d_c = ldl(dd + (size_t)(h0 >> 1) * R, lo);
    uint4 ha = z4, hb = z4;
    if (Q3) {
        ha = ldl(hm + (size_t)(8 * (h0 >> 1) + 2 * q) * R, lo);
        hb = ldl(hm + (size_t)(8 * (h0 >> 1) + 2 * q + 1) * R, lo);
    }
    stage();
    const uint32_t *xa0 = xa - (c0 >> 1), *xb0 = xb - (c0 >> 1);
    const uint32_t *zero = (const uint32_t *)L.zero;
    const uint4 ones4 = make_uint4(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);
    for (int h = h0; h < h1; ++h) {
        const int n = h & 1;
        // next half-block's words and its block's d (and hmask), one half-block ahead: zeros past the split, and a
        // block's d and hmask read again for its second half-block, so no load sits under a branch
        const bool more = h + 1 < h1;
        const uint4 qa_n = ldl_if(qs + (size_t)(8 * (h + 1)) * R, lo_a, more);
        const uint4 qb_n = ldl_if(qs + (size_t)(8 * (h + 1)) * R, lo_b, more);
        const uint4 sa_n = ldl_if(sc + (size_t)(2 * (h + 1)) * R, lo, more);
        const uint4 sb_n = ldl_if(sc + (size_t)(2 * (h + 1) + 1) * R, lo, more);
        const uint4 d_n = ldl_if<false>(dd + (size_t)((h + 1) >> 1) * R, lo, more);
        uint4 ha_n = ha, hb_n = hb;
        if constexpr (Q3) {
            ha_n = ldl_if<false>(hm + (size_t)(8 * ((h + 1) >> 1)) * R, lo_a, more);
            hb_n = ldl_if<false>(hm + (size_t)(8 * ((h + 1) >> 1)) * R, lo_b, more);
        }
        float dv[4], mv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            dv[r] = f16_bits_to_f32(u4c(d_c, r) & 0xffffu);
            mv[r] = Q3 ? 0.0f : f16_bits_to_f32(u4c(d_c, r) >> 16);
        }
        const uint32_t *xr = xa0 + 64 * h, *xr2 = xb0 + 64 * h;     // 64 dwords: the half-block's 128 columns
        const uint32_t *pa0 = first ? xr : zero, *pa1 = first ? zero : xr;
        const uint32_t *pb0 = first ? xr2 : zero, *pb1 = first ? zero : xr2;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            __builtin_amdgcn_sched_barrier(0);
            const uint4 a0 = *(const uint4 *)(pa0 + 16 * s), a1 = *(const uint4 *)(pa1 + 16 * s);
            uint4 b0 = a0, b1 = a1;
            if (TWO) {
                b0 = *(const uint4 *)(pb0 + 16 * s);
                b1 = *(const uint4 *)(pb1 + 16 * s);
            }
            const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
            f32x4 g0 = zero4, g1 = zero4;                           // Q2_K: the two groups' activation sums
            if (!Q3) {
                const bf16x8 ob = __builtin_bit_cast(bf16x8, ones4);
                g0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a0), ob, zero4, 0, 0, 0);
                g1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a1), ob, zero4, 0, 0, 0);
                if (TWO) {
                    g0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, b0), ob, g0, 0, 0, 0);
                    g1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, b1), ob, g1, 0, 0, 0);
                }
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                uint32_t t0 = (u4c(qa, r) >> (2 * s)) & 0x03030303u, t1 = (u4c(qb, r) >> (2 * s)) & 0x03030303u;
                if (Q3) {                                           // hmask bit 4n + s of each byte -> index bit 2
                    t0 |= ((u4c(ha, r) >> (4 * n + s)) & 0x01010101u) << 2;
                    t1 |= ((u4c(hb, r) >> (4 * n + s)) & 0x01010101u) << 2;
                }
                const uint2 l0 = kq_levels<Q3>(t0), l1 = kq_levels<Q3>(t1);
                const bf16x8 wb = __builtin_bit_cast(bf16x8, make_uint4(l0.x, l0.y, l1.x, l1.y));
                f32x4 p0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a0), wb, zero4, 0, 0, 0);
                f32x4 p1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a1), wb, zero4, 0, 0, 0);
                if (TWO) {
                    p0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, b0), wb, p0, 0, 0, 0);
                    p1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, b1), wb, p1, 0, 0, 0);
                }
                // scale bytes 8n + 2s (first group) and 8n + 2s + 1: bytes 2 (s % 2), 2 (s % 2) + 1 of sc row 2h + s/2
                const uint32_t sw = u4c(s >> 1 ? sb : sa, r) >> (16 * (s & 1));
                if (Q3) {
                    const float s0 = fmaf((float)(sw & 255u), dv[r], -32.0f * dv[r]);
                    const float s1 = fmaf((float)((sw >> 8) & 255u), dv[r], -32.0f * dv[r]);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[r][i] = fmaf(s1, p1[i], fmaf(s0, p0[i], acc[r][i]));
                } else {
                    const float s0 = dv[r] * (float)(sw & 15u), m0 = mv[r] * (float)((sw >> 4) & 15u);
                    const float s1 = dv[r] * (float)((sw >> 8) & 15u), m1 = mv[r] * (float)((sw >> 12) & 15u);
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        acc[r][i] = fmaf(-m1, g1[i], fmaf(-m0, g0[i], fmaf(s1, p1[i], fmaf(s0, p0[i], acc[r][i]))));
                }
            }
        }
        qa = qa_n;
        qb = qb_n;
        sa = sa_n;
        sb = sb_n;
        d_c = d_n;
        ha = ha_n;
        hb = hb_n;
    }
}

template <bool HILO, int TCMAX, bool Q3, class Stage>
__device__ __forceinline__ void kqm_run_and_store(const KqTable &tb, int e, int row0, int u0, int u1, int c0,
                                                  const KqLds &L, const uint32_t *xh, const uint32_t *xl, int xsp,
                                                  int t_rows, int n, const int *slots, float *part_base, int R,
                                                  Stage &&stage) {
    iqm_run_and_store<HILO, TCMAX>(row0, xh, xl, xsp, t_rows, n, slots, part_base, R,
                                   [&](auto two, const uint32_t *xa, const uint32_t *xb, f32x4(&acc)[4]) {
                                       kqm_accum<decltype(two)::value, Q3>(tb, e, row0, u0, u1, c0, L, xa, xb, acc,
                                                                           stage);
                                   });
}

}  // namespace mi
