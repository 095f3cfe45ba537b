// IQ3_S row decoder of the gfx950 MoE kernels (vector ALU path).  Each lane owns 4 consecutive matrix rows r0..r0+3
// of one expert and accumulates, for TC activation rows, acc[i][t] += sum_n W[r0+i][n] * x_t[n] over a column range.
// Activations are staged in LDS as bf16 pairs (dword d of row t = columns c0+2d, c0+2d+1); with HILO the f32
// activations are staged twice, as their bf16 high part and the bf16 remainder, and both are dotted.
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

// bf16 pair of two signed odd grid levels (exact): level bytes l0, l1 in 1..15, sign bits s0, s1.
__device__ __forceinline__ uint32_t iq3_pair(uint32_t l0, uint32_t l1, uint32_t s0, uint32_t s1) {
    const uint32_t a = __float_as_uint((float)l0) >> 16;
    const uint32_t b = __float_as_uint((float)l1) & 0xffff0000u;
    return a | b | (s0 << 15) | (s1 << 31);
}

template <int TC, bool HILO, class Stage>
__device__ __forceinline__ void iq3_accum(const Iq3Table &tb, int e, int r0, int u0, int u1, int c0, const uint32_t *__restrict__ grid,
                          const uint32_t *__restrict__ xh, const uint32_t *__restrict__ xl, int xs,
                          float (&acc)[4][TC], Stage &&stage) {
    const size_t R = (size_t)tb.R;
    const int W = tb.W;
    const uint32_t lo = (uint32_t)r0;
    const uint32_t *qs = tb.qs + (size_t)e * W * R;
    const uint32_t *sg = tb.sg + (size_t)e * (W / 2) * R;
    const uint32_t *qh = tb.qh + (size_t)e * (W / 8) * R;
    const uint32_t *sc = tb.sc + (size_t)e * (W / 16) * R;
    const uint32_t *dd = tb.d + (size_t)e * ((tb.nblk + 1) / 2) * R;
    const int w_begin = 16 * u0, w_end = 16 * u1;
    const uint4 z4 = make_uint4(0, 0, 0, 0);
    // pipelines: q two words ahead; sg / qh / sc / d one period ahead (current + next value)
    uint4 q0 = ldl(qs + (size_t)w_begin * R, lo), q1 = ldl(qs + (size_t)(w_begin + 1) * R, lo);
    uint4 sg_c = ldl(sg + (size_t)(w_begin >> 1) * R, lo);
    uint4 sg_n = (w_begin + 2 < w_end) ? ldl(sg + (size_t)((w_begin >> 1) + 1) * R, lo) : z4;
    uint4 qh_c = ldl(qh + (size_t)(w_begin >> 3) * R, lo);
    uint4 qh_n = (w_begin + 8 < w_end) ? ldl(qh + (size_t)((w_begin >> 3) + 1) * R, lo) : z4;
    uint4 sc_c = ldl(sc + (size_t)(w_begin >> 4) * R, lo);
    uint4 sc_n = (w_begin + 16 < w_end) ? ldl(sc + (size_t)((w_begin >> 4) + 1) * R, lo) : z4;
    uint4 d_c = ldl(dd + (size_t)(w_begin >> 5) * R, lo);
    uint4 d_n = ((w_begin & ~31) + 32 < w_end) ? ldl(dd + (size_t)((w_begin >> 5) + 1) * R, lo) : z4;
    stage();
#pragma unroll 2
    for (int w = w_begin; w < w_end; ++w) {
        if (w > w_begin) {
            if ((w & 1) == 0) {
                sg_c = sg_n;
                if (w + 2 < w_end) sg_n = ldl(sg + (size_t)((w >> 1) + 1) * R, lo);
            }
            if ((w & 7) == 0) {
                qh_c = qh_n;
                if (w + 8 < w_end) qh_n = ldl(qh + (size_t)((w >> 3) + 1) * R, lo);
            }
            if ((w & 15) == 0) {
                sc_c = sc_n;
                if (w + 16 < w_end) sc_n = ldl(sc + (size_t)((w >> 4) + 1) * R, lo);
            }
            if ((w & 31) == 0) {
                d_c = d_n;
                if (w + 32 < w_end) d_n = ldl(dd + (size_t)((w >> 5) + 1) * R, lo);
            }
        }
        const uint4 q = q0;
        q0 = q1;
        if (w + 2 < w_end) q1 = ldl(qs + (size_t)(w + 2) * R, lo);
        const uint4 sgw = sg_c, qhw = qh_c, scw = sc_c, dw = d_c;
        const uint32_t Q[4] = {q.x, q.y, q.z, q.w}, SG[4] = {sgw.x, sgw.y, sgw.z, sgw.w};
        const uint32_t QH[4] = {qhw.x, qhw.y, qhw.z, qhw.w}, SC[4] = {scw.x, scw.y, scw.z, scw.w};
        const uint32_t DW[4] = {dw.x, dw.y, dw.z, dw.w};
        const int xi = (16 * w - c0) >> 1;
        // decode the word for the 4 rows: 8 signed bf16 pairs per row + the row's scale
        uint32_t pr[4][8];
        float scale[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t sgh = (SG[i] >> ((w & 1) * 16)) & 0xffffu;
            const uint32_t qhn = (QH[i] >> ((w & 7) * 4)) & 15u;
            const uint32_t scn = (SC[i] >> (((w >> 1) & 7) * 4)) & 15u;
            const uint32_t dbits = DW[i] >> (((w >> 4) & 1) * 16);
            scale[i] = f16_bits_to_f32(dbits) * (1.0f + 2.0f * (float)scn);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t idx = ((Q[i] >> (8 * j)) & 255u) | (((qhn >> j) & 1u) << 8);
                const uint32_t ent = grid[idx];
                const uint32_t sn = (sgh >> (4 * j)) & 15u;
                pr[i][2 * j] = iq3_pair(ent & 255u, (ent >> 8) & 255u, sn & 1u, (sn >> 1) & 1u);
                pr[i][2 * j + 1] = iq3_pair((ent >> 16) & 255u, ent >> 24, (sn >> 2) & 1u, (sn >> 3) & 1u);
            }
        }
#pragma unroll
        for (int t = 0; t < TC; ++t) {
            float sub[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int m = 0; m < 8; ++m) {
                const uint32_t xv = xh[t * xs + xi + m];
                const uint32_t lv = HILO ? xl[t * xs + xi + m] : 0u;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    sub[i] = dot2(pr[i][m], xv, sub[i]);
                    if (HILO) sub[i] = dot2(pr[i][m], lv, sub[i]);
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i][t] = fmaf(scale[i], sub[i], acc[i][t]);
        }
    }
}

}  // namespace mi
