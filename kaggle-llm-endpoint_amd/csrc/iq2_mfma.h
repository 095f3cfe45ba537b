// IQ2_S rows of the grouped decode / matvec launches on the gfx950 matrix cores.
//
// The reference's planar IQ2_S tables (planes.py:17-21,136-170: word w of a row covers inputs 32w .. 32w+31, four
// groups of 8 weights, one grid index and one sign byte per group; per word one qh byte and one sc byte (two 4-bit
// scales, one per 16 weights); per 8 words one f16 d) are read as stored.  As for IQ3_S (iq3_mfma.h) the weights are
// the B operand of v_mfma_f32_16x16x32_bf16 and the activations the A operand, so a lane's output column is the
// weight row it decoded.  One k-step of 32 columns is one word: lane group q holds group q of the word, i.e. the 8
// weights 32w + 8q .. 32w + 8q + 7, in natural column order.  A word spans two scale groups (lane groups 0, 1 and
// 2, 3), so every k-step runs twice, once with the activations of lane groups 2, 3 zeroed and once with those of
// lane groups 0, 1 zeroed, and each partial is scaled by its rows' f32 scale f16(d) * (0.5 + sc) * 0.25.  The B
// operand holds the signed grid levels 8, 25, 43 (exact in bf16): every weight enters exactly as the reference's f32
// dequantization defines it (planes.py:246-259, pallas_moe.py:105-124, iqquant.py:110-120).
//
// A wavefront owns 64 rows, loaded 4 rows per uint4 as four interleaved 16-row tiles (tile r = rows 4i + r of lane
// (i, q)); the four lane groups load the same word and each decodes its own byte of it.
#pragma once
#include "iq3_mfma.h"

namespace mi {

// LDS tables of the decoder.
struct Iq2Lds {
    uint4 level[1024];     // grid entry -> its 8 levels as bf16 (four pairs)
    uint2 smask[16];       // 4 sign bits -> the sign bits (15, 31) of 2 bf16 pairs (32 banks: reads never conflict)
    uint4 zero[16];        // the zeroed activations of the lane groups outside a k-step's scale group
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
            v[p] = (__float_as_uint((float)((w >> s) & 255u)) >> 16) |
                   (__float_as_uint((float)((w >> (s + 8)) & 255u)) & 0xffff0000u);
        }
        t.level[i] = make_uint4(v[0], v[1], v[2], v[3]);
    }
    if (threadIdx.x < 16) {
        const uint32_t s = threadIdx.x;
        t.smask[s] = make_uint2((s & 1u) << 15 | ((s >> 1) & 1u) << 31, ((s >> 2) & 1u) << 15 | ((s >> 3) & 1u) << 31);
        t.zero[s] = make_uint4(0, 0, 0, 0);
    }
}

// Rows row0 .. row0 + 63 of expert e over blocks [u0, u1) (256 columns each), activations staged from column c0:
// acc[r][i] += sum_k W[row0 + 4 (lane % 16) + r][k] * x[token 4 (lane / 16) + i][k].  xa / xb as for iq3m_accum.
template <bool TWO, class Stage>
__device__ __forceinline__ void iq2m_accum(const Iq2Table &tb, int e, int row0, int u0, int u1, int c0,
                                           const Iq2Lds &L, const uint32_t *xa, const uint32_t *xb, f32x4 (&acc)[4],
                                           Stage &&stage) {
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
    const bool first = q < 2;                                       // its group lies in the word's first scale group
    // half-blocks h (4 words, 4 k-steps): word 4h + j in step j; its qh and sc bytes are byte j of row h of those
    // planes; d in row h / 4 (half (h / 2) % 2)
    const int h0 = 2 * u0, h1 = 2 * u1;
    const uint4 z4 = make_uint4(0, 0, 0, 0);
    uint4 rq[4], rs[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        rq[j] = ldl(qs + (size_t)(4 * h0 + j) * R, lo);
        rs[j] = ldl(sg + (size_t)(4 * h0 + j) * R, lo);
    }
    uint4 qh_c = ldl(qh + (size_t)h0 * R, lo), sc_c = ldl(sc + (size_t)h0 * R, lo);
    uint4 qh_n = h0 + 1 < h1 ? ldl(qh + (size_t)(h0 + 1) * R, lo) : z4;
    uint4 sc_n = h0 + 1 < h1 ? ldl(sc + (size_t)(h0 + 1) * R, lo) : z4;
    uint4 d_c = ldl(dd + (size_t)(h0 >> 2) * R, lo);
    uint4 d_n = (h0 & ~3) + 4 < h1 ? ldl(dd + (size_t)((h0 >> 2) + 1) * R, lo) : z4;
    stage();
    const uint32_t *xa0 = xa - (c0 >> 1), *xb0 = xb - (c0 >> 1);
    const uint32_t *zero = (const uint32_t *)L.zero;
    for (int h = h0; h < h1; ++h) {
        if (h > h0) {
            qh_c = qh_n;
            sc_c = sc_n;
            qh_n = h + 1 < h1 ? ldl(qh + (size_t)(h + 1) * R, lo) : z4;
            sc_n = h + 1 < h1 ? ldl(sc + (size_t)(h + 1) * R, lo) : z4;
            if ((h & 3) == 0) {
                d_c = d_n;
                d_n = h + 4 < h1 ? ldl(dd + (size_t)((h >> 2) + 1) * R, lo) : z4;
            }
        }
        float d4[4], d8[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float dv = f16_bits_to_f32(u4c(d_c, r) >> (16 * ((h >> 1) & 1)));
            d4[r] = 0.25f * dv;
            d8[r] = 0.125f * dv;
        }
        // the two scale groups' A operands: the lane's activations, or zeros (read from LDS, not selected in registers)
        const uint32_t *xr = xa0 + 64 * h, *xr2 = xb0 + 64 * h;    // 64 dwords: the half-block's 128 columns
        const uint32_t *pa0 = first ? xr : zero, *pa1 = first ? zero : xr;
        const uint32_t *pb0 = first ? xr2 : zero, *pb1 = first ? zero : xr2;
        const bool more = h + 1 < h1;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            __builtin_amdgcn_sched_barrier(0);
            const uint4 a0 = *(const uint4 *)(pa0 + 16 * j), a1 = *(const uint4 *)(pa1 + 16 * j);
            uint4 b0 = a0, b1 = a1;
            if (TWO) {
                b0 = *(const uint4 *)(pb0 + 16 * j);
                b1 = *(const uint4 *)(pb1 + 16 * j);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                // step j's qh and sc bytes are byte j of the lane's qh / sc words
                const uint32_t idx = ((u4c(rq[j], r) >> qsh) & 255u) | (((u4c(qh_c, r) >> (8 * j + 2 * q)) & 3u) << 8);
                const uint32_t sb = (u4c(rs[j], r) >> qsh) & 255u;
                const uint4 g = L.level[idx];
                const uint2 m0 = L.smask[sb & 15u], m1 = L.smask[sb >> 4];
                const uint4 w = make_uint4(g.x | m0.x, g.y | m0.y, g.z | m1.x, g.w | m1.y);
                const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
                const bf16x8 wb = __builtin_bit_cast(bf16x8, w);
                f32x4 p0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a0), wb, zero, 0, 0, 0);
                f32x4 p1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a1), wb, zero, 0, 0, 0);
                if (TWO) {
                    p0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, b0), wb, p0, 0, 0, 0);
                    p1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, b1), wb, p1, 0, 0, 0);
                }
                // f16(d) * (0.5 + sc) * 0.25 = sc * d/4 + d/8, exact
                const uint32_t scb = u4c(sc_c, r) >> (8 * j);
                const float s0 = fmaf((float)(scb & 15u), d4[r], d8[r]);
                const float s1 = fmaf((float)((scb >> 4) & 15u), d4[r], d8[r]);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[r][i] = fmaf(s1, p1[i], fmaf(s0, p0[i], acc[r][i]));
            }
            // the ring slot takes step j of the next half-block
            if (more) {
                rq[j] = ldl(qs + (size_t)(4 * (h + 1) + j) * R, lo);
                rs[j] = ldl(sg + (size_t)(4 * (h + 1) + j) * R, lo);
            }
        }
    }
}

template <bool HILO, int TCMAX, class Stage>
__device__ __forceinline__ void iq2m_run_and_store(const Iq2Table &tb, int e, int row0, int u0, int u1, int c0,
                                                   const Iq2Lds &L, const uint32_t *xh, const uint32_t *xl, int xsp,
                                                   int t_rows, int n, const int *slots, float *part_base, int R,
                                                   Stage &&stage) {
    iqm_run_and_store<HILO, TCMAX>(row0, xh, xl, xsp, t_rows, n, slots, part_base, R,
                                   [&](auto two, const uint32_t *xa, const uint32_t *xb, f32x4(&acc)[4]) {
                                       iq2m_accum<decltype(two)::value>(tb, e, row0, u0, u1, c0, L, xa, xb, acc,
                                                                        stage);
                                   });
}

}  // namespace mi
