// Per-format row decoders of the gfx950 MoE kernels.  Each lane owns 4 consecutive matrix rows r0..r0+3 of one
// expert and accumulates, for TC activation rows, acc[i][t] += sum_n W[r0+i][n] * x_t[n] over a column range.
// Activations are staged in LDS as bf16 pairs (dword d of row t = columns c0+2d, c0+2d+1); with HILO the f32
// activations are staged twice, as their bf16 high part and the bf16 remainder, and both are dotted.
#pragma once
#include "common.h"

namespace mi {

// ------------------------------------------------------------------------------------------------ CB3
// Kernel bit layout of the code plane (written by formats.py, same byte count as the canonical 10-codes-per-u32
// packing).  Codes are handled in pairs of words covering 20 columns c = 20P .. 20P+19:
//   word 2P   byte j = code[c+j] | code[c+4+j] << 3 | (code[c+16+j] & 3) << 6                  (j = 0..3)
//   word 2P+1 byte j = code[c+8+j] | code[c+12+j] << 3 | (code[c+16+j] >> 2) << 6
// so one AND (and a shift) yields 4 byte-sized selectors.  A trailing single word (odd word count) holds
// code[c+j] | code[c+4+j] << 3 in byte j and code[c+8], code[c+9] split over bits 6-7 of bytes 0,1 (low 2 bits)
// and bit 6 of bytes 2,3 (high bit).
// Codebook plane: per (row, group g of 128 columns) 4 dwords: lo-bytes of centroids 0-3, 4-7, hi-bytes 0-3, 4-7.
struct Cb3Table {
    const uint32_t *qs;
    const uint32_t *cb;
    int R, K, Wd, G;
    static constexpr int kUnitCols = 20;   // one word pair
};

// 4 bf16 weights (codes in the 4 selector bytes of s) -> two bf16 pairs (w0,w1), (w2,w3)
__device__ __forceinline__ void cb3_lookup(uint32_t s, uint32_t lo03, uint32_t lo47, uint32_t hi03, uint32_t hi47,
                                           uint32_t &p01, uint32_t &p23) {
    const uint32_t lo = perm(lo47, lo03, s);
    const uint32_t hi = perm(hi47, hi03, s);
    p01 = perm(hi, lo, 0x05010400u);
    p23 = perm(hi, lo, 0x07030602u);
}

template <int TC, bool HILO>
__device__ void cb3_accum(const Cb3Table &tb, int e, int r0, int u0, int u1, int c0,
                          const uint32_t *__restrict__ xh, const uint32_t *__restrict__ xl, int xs,
                          float (&acc)[4][TC]) {
    const size_t R = (size_t)tb.R;
    const uint32_t *qs = tb.qs + (size_t)e * tb.Wd * R + r0;
    const uint32_t *cb = tb.cb + (size_t)e * tb.G * 4 * R + r0;
    int cur_g = -1;
    uint4 lo03 = {}, lo47 = {}, hi03 = {}, hi47 = {};
#pragma unroll 1
    for (int P = u0; P < u1; ++P) {
        const int w0 = 2 * P;
        const bool has_u1 = (w0 + 1) < tb.Wd;
        const uint4 a = *(const uint4 *)(qs + (size_t)w0 * R);
        const uint4 b = has_u1 ? *(const uint4 *)(qs + (size_t)(w0 + 1) * R) : make_uint4(0, 0, 0, 0);
        const int base = 20 * P;
        const int nf = has_u1 ? 5 : 3;
        for (int f = 0; f < nf; ++f) {
            const int col = base + 4 * f;
            if (col >= tb.K) break;
            const int g = col >> 7;
            if (g != cur_g) {
                const uint32_t *cg = cb + (size_t)g * 4 * R;
                lo03 = *(const uint4 *)(cg);
                lo47 = *(const uint4 *)(cg + R);
                hi03 = *(const uint4 *)(cg + 2 * R);
                hi47 = *(const uint4 *)(cg + 3 * R);
                cur_g = g;
            }
            const bool two = has_u1 || f < 2;        // a tail-word C field covers one column pair only
            const int xi = (col - c0) >> 1;
            const uint32_t ua[4] = {a.x, a.y, a.z, a.w};
            const uint32_t ub[4] = {b.x, b.y, b.z, b.w};
            const uint32_t L03[4] = {lo03.x, lo03.y, lo03.z, lo03.w}, L47[4] = {lo47.x, lo47.y, lo47.z, lo47.w};
            const uint32_t H03[4] = {hi03.x, hi03.y, hi03.z, hi03.w}, H47[4] = {hi47.x, hi47.y, hi47.z, hi47.w};
            uint32_t p01[4], p23[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint32_t s;
                if (f == 0) s = ua[i] & 0x07070707u;
                else if (f == 1) s = (ua[i] >> 3) & 0x07070707u;
                else if (f == 2) {
                    if (has_u1) s = ub[i] & 0x07070707u;
                    else {
                        const uint32_t t2 = (ua[i] >> 6) & 0x03030303u;
                        s = t2 | (t2 >> 14);
                    }
                } else if (f == 3) s = (ub[i] >> 3) & 0x07070707u;
                else s = ((ua[i] >> 6) & 0x03030303u) | ((ub[i] >> 4) & 0x04040404u);
                cb3_lookup(s, L03[i], L47[i], H03[i], H47[i], p01[i], p23[i]);
            }
#pragma unroll
            for (int t = 0; t < TC; ++t) {
                const uint32_t xa = xh[t * xs + xi];
                const uint32_t xb = two ? xh[t * xs + xi + 1] : 0u;
                uint32_t la = 0, lb = 0;
                if (HILO) {
                    la = xl[t * xs + xi];
                    lb = two ? xl[t * xs + xi + 1] : 0u;
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float v = dot2(p01[i], xa, acc[i][t]);
                    v = dot2(p23[i], xb, v);
                    if (HILO) {
                        v = dot2(p01[i], la, v);
                        v = dot2(p23[i], lb, v);
                    }
                    acc[i][t] = v;
                }
            }
        }
    }
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

template <int TC, bool HILO>
__device__ void iq3_accum(const Iq3Table &tb, int e, int r0, int u0, int u1, int c0, const uint32_t *__restrict__ grid,
                          const uint32_t *__restrict__ xh, const uint32_t *__restrict__ xl, int xs,
                          float (&acc)[4][TC]) {
    const size_t R = (size_t)tb.R;
    const int W = tb.W;
    const uint32_t *qs = tb.qs + (size_t)e * W * R + r0;
    const uint32_t *sg = tb.sg + (size_t)e * (W / 2) * R + r0;
    const uint32_t *qh = tb.qh + (size_t)e * (W / 8) * R + r0;
    const uint32_t *sc = tb.sc + (size_t)e * (W / 16) * R + r0;
    const uint32_t *dd = tb.d + (size_t)e * ((tb.nblk + 1) / 2) * R + r0;
#pragma unroll 1
    for (int w = 16 * u0; w < 16 * u1; ++w) {
        const uint4 q = *(const uint4 *)(qs + (size_t)w * R);
        const uint4 sgw = *(const uint4 *)(sg + (size_t)(w >> 1) * R);
        const uint4 qhw = *(const uint4 *)(qh + (size_t)(w >> 3) * R);
        const uint4 scw = *(const uint4 *)(sc + (size_t)(w >> 4) * R);
        const uint4 dw = *(const uint4 *)(dd + (size_t)(w >> 5) * R);
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
