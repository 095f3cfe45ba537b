// IQ2_S rows of the grouped decode / matvec launches on the gfx950 matrix cores.
//
// The reference's planar IQ2_S tables (planes.py:17-21,136-170: word w of a row covers inputs 32w .. 32w+31, four
// groups of 8 weights, one grid index and one sign byte per group; per word one qh byte and one sc byte (two 4-bit
// scales, one per 16 weights); per 8 words one f16 d) are read as stored.  As for IQ3_S (iq3_mfma.h) the weights are
// the B operand of the matrix-core instruction and the activations the A operand, so a lane's output column is the
// weight row it decoded.  One k-step of 32 columns is one word: lane group q holds group q of the word, i.e. the 8
// weights 32w + 8q .. 32w + 8q + 7, in natural column order.
//
// A weight is d * (0.5 + sc) * 0.25 * (+-level) = (d / 8) * ((2 sc + 1) * (+-level)) with level in {8, 25, 43} and
// 2 sc + 1 <= 31: the integer (2 sc + 1) * level <= 1333 is exact in f16 (11 significant bits), so the B operand is
// f16 (the lane's scale group's odd factor times its signed levels, one packed f16 multiply per pair) and the
// matrix cores run v_mfma_f32_16x16x32_f16 with the activations staged as f16.  Each staged activation row is first
// scaled by a power of two that puts its largest magnitude in [2^14, 2^15) (up for small rows, down for large ones),
// so f16 holds the row's values exactly (bf16 values; f32 values as an f16 high part + remainder) whatever their
// scale; each token's sums are multiplied back by the same power of two, which is exact.  A whole word (both scale
// groups) is then one instruction, and the f32 factor d / 8 of the
// 256-weight block is applied once per half-block (4 k-steps) instead of per k-step and scale group.  Products are
// exact and accumulate in f32: every weight enters exactly as the reference's f32 dequantization defines it
// (planes.py:246-259, pallas_moe.py:105-124, iqquant.py:110-120).
//
// A wavefront owns 64 rows, loaded 4 rows per uint4 as four interleaved 16-row tiles (tile r = rows 4i + r of lane
// (i, q)); the four lane groups load the same word and each decodes its own byte of it.
#pragma once
#include "iq3_mfma.h"

namespace mi {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// LDS tables of the decoder, and the staging's activation row scales.
struct Iq2Lds {
    uint4 level[1024];     // grid entry -> its 8 levels as f16 (four pairs)
    uint2 smask[16];       // 4 sign bits -> the sign bits (15, 31) of 2 f16 pairs (32 banks: reads never conflict)
    uint32_t cf2[16];      // 4-bit scale sc -> the odd factor 2 sc + 1 as an f16 pair
    uint32_t amax[kMaxT];  // per staged activation row: bits of its largest |value| over the staged columns
};

// grid: 2 words per entry, byte k of the 8 = level of position k.  Every thread of the workgroup takes part; a
// barrier must follow before the tables are read.
__device__ __forceinline__ void iq2_fill_lds(Iq2Lds &t, const uint32_t *grid) {
    for (int i = threadIdx.x; i < 1024; i += blockDim.x) {
        const uint32_t a = grid[2 * i], b = grid[2 * i + 1];
        uint32_t v[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const uint32_t w = p < 2 ? a : b, s = 16 * (p & 1);
            const f16x2 h = {(_Float16)(float)((w >> s) & 255u), (_Float16)(float)((w >> (s + 8)) & 255u)};
            v[p] = __builtin_bit_cast(uint32_t, h);
        }
        t.level[i] = make_uint4(v[0], v[1], v[2], v[3]);
    }
    if (threadIdx.x < 16) {
        const uint32_t s = threadIdx.x;
        t.smask[s] = make_uint2((s & 1u) << 15 | ((s >> 1) & 1u) << 31, ((s >> 2) & 1u) << 15 | ((s >> 3) & 1u) << 31);
        const _Float16 c = (_Float16)(float)(2u * s + 1u);
        t.cf2[s] = __builtin_bit_cast(uint32_t, (f16x2){c, c});
    }
    if (threadIdx.x < kMaxT) t.amax[threadIdx.x] = 0u;
}

// The power of two p a row is staged at (values times 2^-p): the row's largest magnitude (as f32 bits, exponent e)
// lands in [2^14, 2^15).  0 for an all-zero row.  A subnormal maximum (biased exponent 0) takes p = -141, which
// still leaves every value below 2^15.
__device__ __forceinline__ int iq2_xshift(uint32_t amax) {
    return amax ? (int)((amax >> 23) & 255u) - 127 - 14 : 0;
}

// One activation value (the f32 value of the staged bf16 element, or of the bf16 high part + remainder) -> f16 high
// part and remainder at scale 2^-shift.
__device__ __forceinline__ void iq2_x16(float f, int shift, uint32_t &hi, uint32_t &lo) {
    f = ldexpf(f, -shift);
    const _Float16 h = (_Float16)f;
    const _Float16 l = (_Float16)(f - (float)h);
    hi = __builtin_bit_cast(uint16_t, h);
    lo = __builtin_bit_cast(uint16_t, l);
}

// Rows row0 .. row0 + 63 of expert e over blocks [u0, u1) (256 columns each), activations staged (f16, each row at
// its own power of two) from column c0: acc[r][i] += sum_k W[row0 + 4 (lane % 16) + r][k] * x[token 4 (lane / 16) +
// i][k].  xa / xb as for iq3m_accum.  PAIR: A rows m >= 8 are the remainders of row m - 8 (iqm_run_and_store).
template <bool TWO, bool PAIR, class Stage>
__device__ __forceinline__ void iq2m_accum(const Iq2Table &tb, int e, int row0, int u0, int u1, int c0,
                                           const Iq2Lds &L, const uint32_t *xa, const uint32_t *xb, int t_rows,
                                           f32x4 (&acc)[4], Stage &&stage) {
    const int lane = threadIdx.x & 63, q = lane >> 4;
    const size_t R = (size_t)tb.R;
    const int W = tb.W;
    const uint32_t lo = (uint32_t)(row0 + 4 * (lane & 15));
    const uint32_t *qs = tb.qs + (size_t)e * W * R;
    const uint32_t *sg = tb.sg + (size_t)e * W * R;
    const uint32_t *qh = tb.qh + (size_t)e * (W / 4) * R;
    const uint32_t *sc = tb.sc + (size_t)e * (W / 4) * R;
    const uint32_t *dd = tb.d + (size_t)e * ((tb.nblk + 1) / 2) * R;
    const uint32_t qsh = 8 * q;                                     // the lane group's byte of a qs / sg word
    const uint32_t scsh = q < 2 ? 0u : 4u;                          // its scale group's nibble of a sc byte
    // half-blocks h (4 words, 4 k-steps): word 4h + j in step j; its qh and sc bytes are byte j of row h of those
    // planes; d in row h / 4 (half (h / 2) % 2)
    const int h0 = 2 * u0, h1 = 2 * u1;
    uint4 rq[4], rs[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        rq[j] = ldl(qs + (size_t)(4 * h0 + j) * R, lo);
        rs[j] = ldl(sg + (size_t)(4 * h0 + j) * R, lo);
    }
    // half-block h's qh, sc and d words, each loaded one half-block ahead (d again for every half-block: the loads
    // never sit under a branch)
    uint4 qh_n = ldl(qh + (size_t)h0 * R, lo), sc_n = ldl(sc + (size_t)h0 * R, lo);
    uint4 d_n = ldl_if<false>(dd + (size_t)(h0 >> 2) * R, lo, true);
    stage();
    const float dmul = 0.125f;                                      // d / 8
    const uint32_t *xa0 = xa - (c0 >> 1), *xb0 = xb - (c0 >> 1);
    for (int h = h0; h < h1; ++h) {
        const uint4 qh_c = qh_n, sc_c = sc_n, d_c = d_n;
        const bool more = h + 1 < h1;
        qh_n = ldl_if(qh + (size_t)(h + 1) * R, lo, more);
        sc_n = ldl_if(sc + (size_t)(h + 1) * R, lo, more);
        d_n = ldl_if<false>(dd + (size_t)((h + 1) >> 2) * R, lo, more);
        const uint32_t *xr = xa0 + 64 * h, *xr2 = xb0 + 64 * h;    // 64 dwords: the half-block's 128 columns
        f32x4 ph[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) ph[r] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            __builtin_amdgcn_sched_barrier(0);
            const uint4 a0 = *(const uint4 *)(xr + 16 * j);
            uint4 b0 = a0;
            if (TWO) b0 = *(const uint4 *)(xr2 + 16 * j);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                // step j's qh and sc bytes are byte j of the lane's qh / sc words
                const uint32_t idx = ((u4c(rq[j], r) >> qsh) & 255u) | (((u4c(qh_c, r) >> (8 * j + 2 * q)) & 3u) << 8);
                const uint32_t sb = (u4c(rs[j], r) >> qsh) & 255u;
                const uint4 g = L.level[idx];
                const uint2 m0 = L.smask[sb & 15u], m1 = L.smask[sb >> 4];
                // the lane's scale group's odd factor 2 sc + 1 as an f16 pair (a table: no conversions)
                const f16x2 c2 = __builtin_bit_cast(f16x2, L.cf2[(u4c(sc_c, r) >> (8 * j + scsh)) & 15u]);
                const uint4 wu = make_uint4(__builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, g.x | m0.x) * c2),
                                            __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, g.y | m0.y) * c2),
                                            __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, g.z | m1.x) * c2),
                                            __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, g.w | m1.y) * c2));
                const f16x8 wb = __builtin_bit_cast(f16x8, wu);
                ph[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a0), wb, ph[r], 0, 0, 0);
                if (TWO) ph[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, b0), wb, ph[r], 0, 0, 0);
            }
            // the ring slot takes step j of the next half-block (zeros past the split)
            rq[j] = ldl_if(qs + (size_t)(4 * (h + 1) + j) * R, lo, more);
            rs[j] = ldl_if(sg + (size_t)(4 * (h + 1) + j) * R, lo, more);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float dv = dmul * f16_bits_to_f32(u4c(d_c, r) >> (16 * ((h >> 1) & 1)));
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[r][i] = fmaf(dv, ph[r][i], acc[r][i]);
        }
    }
    // undo each row's staging scale: output row 4 q + i of the tile is activation row (PAIR ? m & 7 : m), clamped as
    // the A operand's rows are
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = 4 * q + i;
        const int shift = iq2_xshift(L.amax[min(PAIR ? (m & 7) : m, t_rows - 1)]);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r][i] = ldexpf(acc[r][i], shift);
    }
}

template <bool HILO, int TCMAX, class Stage>
__device__ __forceinline__ void iq2m_run_and_store(const Iq2Table &tb, int e, int row0, int u0, int u1, int c0,
                                                   const Iq2Lds &L, const uint32_t *xh, const uint32_t *xl, int xsp,
                                                   int t_rows, int n, const int *slots, float *part_base, int R,
                                                   Stage &&stage) {
    iqm_run_and_store<HILO, TCMAX>(row0, xh, xl, xsp, t_rows, n, slots, part_base, R,
                                   [&](auto two, const uint32_t *xa, const uint32_t *xb, f32x4(&acc)[4]) {
                                       constexpr bool kTwo = decltype(two)::value;
                                       iq2m_accum<kTwo, HILO && !kTwo>(tb, e, row0, u0, u1, c0, L, xa, xb, t_rows,
                                                                       acc, stage);
                                   });
}

}  // namespace mi
