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
    static constexpr int kUnitCols = 640;  // one super-tile: 32 word pairs = 5 codebook groups
};

// 4 bf16 weights (codes in the 4 selector bytes of s) -> two bf16 pairs (w0,w1), (w2,w3)
__device__ __forceinline__ void cb3_lookup(uint32_t s, uint32_t lo03, uint32_t lo47, uint32_t hi03, uint32_t hi47,
                                           uint32_t &p01, uint32_t &p23) {
    const uint32_t lo = perm(lo47, lo03, s);
    const uint32_t hi = perm(hi47, hi03, s);
    p01 = perm(hi, lo, 0x05010400u);
    p23 = perm(hi, lo, 0x07030602u);
}

__device__ __forceinline__ uint4 ld16(const uint32_t *p) { return *(const uint4 *)p; }
// wave-uniform base (SGPRs) + the lane's 32-bit row offset: lets every load use the scalar-base addressing form
// instead of a 64-bit vector address per load
__device__ __forceinline__ uint4 ldl(const uint32_t *__restrict__ base, uint32_t lane_off) {
    // byte offset computed in 32 bits (rows < 2^30), so the address is "SGPR base + 32-bit VGPR offset"
    return *(const uint4 *)((const char *)base + (lane_off << 2));
}

#ifndef MI_CB3_PF
#define MI_CB3_PF 8          // word pairs kept in flight per lane (8 pairs = 16 KB per wavefront)
#endif

// Codebook state of the 4 rows: the current group (lo03, lo47, hi03, hi47) and the prefetched next group.
struct Cb3Book {
    uint4 lo03, lo47, hi03, hi47, n03, n47, m03, m47;
    int cur_g, g_last;
};

__device__ __forceinline__ void cb3_load_group(const uint32_t *cb, size_t R, int g, uint32_t lo, uint4 &a, uint4 &b,
                                               uint4 &c, uint4 &d) {
    const uint32_t *cg = cb + (size_t)g * 4 * R;
    a = ldl(cg, lo);
    b = ldl(cg + R, lo);
    c = ldl(cg + 2 * R, lo);
    d = ldl(cg + 3 * R, lo);
}

// One word pair P (columns 20P .. 20P+19, fields of 4 columns; a single trailing word has 10 columns).
template <int TC, bool HILO>
__device__ __forceinline__ void cb3_pair(const uint4 a, const uint4 b, const int P, const bool has_u1, const int K,
                                         const int c0, const uint32_t *cb, const size_t R, const uint32_t lo,
                                         Cb3Book &bk,
                                         const uint32_t *__restrict__ xh, const uint32_t *__restrict__ xl,
                                         const int xs, float (&acc)[4][TC]) {
    const int base = 20 * P;
    const int nf = has_u1 ? 5 : 3;
#pragma unroll
    for (int f = 0; f < 5; ++f) {
        const int col = base + 4 * f;
        if (f >= nf || col >= K) break;
        const int g = col >> 7;
        if (g != bk.cur_g) {                 // wave-uniform: rotate in the prefetched group, prefetch the next
            bk.lo03 = bk.n03;
            bk.lo47 = bk.n47;
            bk.hi03 = bk.m03;
            bk.hi47 = bk.m47;
            bk.cur_g = g;
            if (g + 1 <= bk.g_last) cb3_load_group(cb, R, g + 1, lo, bk.n03, bk.n47, bk.m03, bk.m47);
        }
        const bool two = has_u1 || f < 2;    // a trailing single word's C field covers one column pair only
        const int xi = (col - c0) >> 1;
        const uint32_t ua[4] = {a.x, a.y, a.z, a.w};
        const uint32_t ub[4] = {b.x, b.y, b.z, b.w};
        const uint32_t L03[4] = {bk.lo03.x, bk.lo03.y, bk.lo03.z, bk.lo03.w};
        const uint32_t L47[4] = {bk.lo47.x, bk.lo47.y, bk.lo47.z, bk.lo47.w};
        const uint32_t H03[4] = {bk.hi03.x, bk.hi03.y, bk.hi03.z, bk.hi03.w};
        const uint32_t H47[4] = {bk.hi47.x, bk.hi47.y, bk.hi47.z, bk.hi47.w};
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
            uint32_t xa, xb = 0u, la = 0u, lb = 0u;
            if (two) {
                const uint2 v = *(const uint2 *)(xh + t * xs + xi);
                xa = v.x;
                xb = v.y;
                if (HILO) {
                    const uint2 l = *(const uint2 *)(xl + t * xs + xi);
                    la = l.x;
                    lb = l.y;
                }
            } else {
                xa = xh[t * xs + xi];
                if (HILO) la = xl[t * xs + xi];
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

// ---- static super-tile path -------------------------------------------------------------------------------------
// 128-column codebook groups and 20-column word pairs realign every 640 columns (32 pairs = 5 groups): within such
// a super-tile every group boundary falls on a 4-column field boundary at a compile-time position, so the whole tile
// is straight-line code -- ring slots, codebook registers and LDS offsets are all static and the compiler keeps the
// loads in flight.  Codebook buffers: group 0 of a tile lives in cN (prefetched by the previous tile), odd groups
// in cA, even groups > 0 in cB; each group's successor is requested at the group's first field.
struct Cb3Ring {
    uint4 a[MI_CB3_PF], b[MI_CB3_PF];
};
struct Cb3Bufs {
    uint4 N[4], A[4], B[4];
};

template <int G>
__device__ __forceinline__ uint4 (&cb3_buf(Cb3Bufs &c))[4] {
    if constexpr (G == 0) return c.N;
    else if constexpr (G & 1) return c.A;
    else return c.B;
}

template <int TC, bool HILO, int F, bool SINGLE>
__device__ __forceinline__ void cb3_field(const uint4 a, const uint4 b, const uint4 (&cbk)[4],
                                          const uint32_t *__restrict__ xh, const uint32_t *__restrict__ xl,
                                          const int xs, const int xi, float (&acc)[4][TC]) {
    const uint32_t ua[4] = {a.x, a.y, a.z, a.w};
    const uint32_t ub[4] = {b.x, b.y, b.z, b.w};
    const uint32_t L03[4] = {cbk[0].x, cbk[0].y, cbk[0].z, cbk[0].w};
    const uint32_t L47[4] = {cbk[1].x, cbk[1].y, cbk[1].z, cbk[1].w};
    const uint32_t H03[4] = {cbk[2].x, cbk[2].y, cbk[2].z, cbk[2].w};
    const uint32_t H47[4] = {cbk[3].x, cbk[3].y, cbk[3].z, cbk[3].w};
    uint32_t p01[4], p23[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t s;
        if constexpr (F == 0) s = ua[i] & 0x07070707u;
        else if constexpr (F == 1) s = (ua[i] >> 3) & 0x07070707u;
        else if constexpr (F == 2 && SINGLE) {
            const uint32_t t2 = (ua[i] >> 6) & 0x03030303u;
            s = t2 | (t2 >> 14);
        } else if constexpr (F == 2) s = ub[i] & 0x07070707u;
        else if constexpr (F == 3) s = (ub[i] >> 3) & 0x07070707u;
        else s = ((ua[i] >> 6) & 0x03030303u) | ((ub[i] >> 4) & 0x04040404u);
        cb3_lookup(s, L03[i], L47[i], H03[i], H47[i], p01[i], p23[i]);
    }
    constexpr bool ONE = SINGLE && F == 2;       // a trailing single word's C field covers one column pair
#pragma unroll
    for (int t = 0; t < TC; ++t) {
        uint32_t xa, xb = 0u, la = 0u, lb = 0u;
        if constexpr (!ONE) {
            const uint2 v = *(const uint2 *)(xh + t * xs + xi);
            xa = v.x;
            xb = v.y;
            if constexpr (HILO) {
                const uint2 l = *(const uint2 *)(xl + t * xs + xi);
                la = l.x;
                lb = l.y;
            }
        } else {
            xa = xh[t * xs + xi];
            if constexpr (HILO) la = xl[t * xs + xi];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float v = dot2(p01[i], xa, acc[i][t]);
            if constexpr (!ONE) v = dot2(p23[i], xb, v);
            if constexpr (HILO) {
                v = dot2(p01[i], la, v);
                if constexpr (!ONE) v = dot2(p23[i], lb, v);
            }
            acc[i][t] = v;
        }
    }
}

// Everything a tile needs besides the per-slot constants.
struct Cb3TileCtx {
    const uint32_t *qt;     // this tile's first code word (lane rows)
    const uint32_t *qn;     // next tile's first code word, or qt when there is no next tile (harmless reload)
    const uint32_t *cbt;    // this tile's first codebook group
    const uint32_t *cbn;    // next tile's first group, or cbt
    const uint32_t *xh, *xl;
    size_t R;
    int nwn;                // code words of the next tile (0 = no next tile); ring refills of words beyond it
                            // re-read the current tile's first word instead (valid memory, value never used)
    uint32_t lo;            // the lane's first row (32-bit offset added to every uniform base)
    int xs, xb;             // LDS row stride and this tile's dword offset in the staged rows
};

template <int TC, bool HILO, int GT, int P, int F>
__device__ __forceinline__ void cb3_slot_field(const uint4 a, const uint4 b, const Cb3TileCtx &c, Cb3Bufs &cbs,
                                               float (&acc)[4][TC]) {
    constexpr int NCOL = 128 * GT;
    constexpr int NWORD = (NCOL + 9) / 10;
    constexpr bool SINGLE = 2 * P + 1 >= NWORD;
    constexpr int col = 20 * P + 4 * F;
    if constexpr (col < NCOL && !(SINGLE && F >= 3)) {
        constexpr int g = col >> 7;
        if constexpr ((col & 127) == 0) {             // first field of group g: request its successor
            if constexpr (g + 1 < GT) cb3_load_group(c.cbt, c.R, g + 1, c.lo, cb3_buf<g + 1>(cbs)[0],
                                                      cb3_buf<g + 1>(cbs)[1], cb3_buf<g + 1>(cbs)[2],
                                                      cb3_buf<g + 1>(cbs)[3]);
            else if constexpr (GT == 5) cb3_load_group(c.cbn, c.R, 0, c.lo, cbs.N[0], cbs.N[1], cbs.N[2], cbs.N[3]);
        }
        cb3_field<TC, HILO, F, SINGLE>(a, b, cb3_buf<g>(cbs), c.xh, c.xl, c.xs, c.xb + 10 * P + 2 * F, acc);
    }
}

template <int TC, bool HILO, int GT, int P>
__device__ __forceinline__ void cb3_slot(const Cb3TileCtx &c, Cb3Ring &ring, Cb3Bufs &cbs, float (&acc)[4][TC]) {
    constexpr int PF = MI_CB3_PF;
    constexpr int NCOL = 128 * GT;
    constexpr int NWORD = (NCOL + 9) / 10;
    constexpr int NSLOT = (NWORD + 1) / 2;
    if constexpr (P < NSLOT) {
        // keep each slot's instructions in place: the ring alone sets how far loads run ahead
        __builtin_amdgcn_sched_barrier(0);
        const uint4 a = ring.a[P % PF], b = ring.b[P % PF];
        constexpr int pn = P + PF;                    // refill the slot: this tile's slot pn or the next tile's
        if constexpr (pn < NSLOT) {
            ring.a[P % PF] = ldl(c.qt + (size_t)(2 * pn) * c.R, c.lo);
            if constexpr (2 * pn + 1 < NWORD) ring.b[P % PF] = ldl(c.qt + (size_t)(2 * pn + 1) * c.R, c.lo);
        } else if constexpr (GT == 5) {
            constexpr int wa = 2 * (pn - NSLOT), wb = wa + 1;   // next tile's words (it may be a short last tile)
            ring.a[P % PF] = ldl(wa < c.nwn ? c.qn + (size_t)wa * c.R : c.qt, c.lo);
            ring.b[P % PF] = ldl(wb < c.nwn ? c.qn + (size_t)wb * c.R : c.qt, c.lo);
        }
        cb3_slot_field<TC, HILO, GT, P, 0>(a, b, c, cbs, acc);
        cb3_slot_field<TC, HILO, GT, P, 1>(a, b, c, cbs, acc);
        cb3_slot_field<TC, HILO, GT, P, 2>(a, b, c, cbs, acc);
        cb3_slot_field<TC, HILO, GT, P, 3>(a, b, c, cbs, acc);
        cb3_slot_field<TC, HILO, GT, P, 4>(a, b, c, cbs, acc);
        cb3_slot<TC, HILO, GT, P + 1>(c, ring, cbs, acc);
    }
}

// Super-tiles st0 .. st1-1 of one expert's rows (tile st covers columns 640*st .. min(K, 640*st+640)).
template <int TC, bool HILO, class Stage>
__device__ __forceinline__ void cb3_accum_tiles(const Cb3Table &tb, int e, int r0, int st0, int st1, int c0,
                                const uint32_t *__restrict__ xh, const uint32_t *__restrict__ xl, int xs,
                                float (&acc)[4][TC], Stage &&stage) {
    static_assert(32 % MI_CB3_PF == 0, "ring must divide a tile");
    constexpr int PF = MI_CB3_PF;
    const size_t R = (size_t)tb.R;
    const uint32_t lo = (uint32_t)r0;
    const uint32_t *qs = tb.qs + (size_t)e * tb.Wd * R;
    const uint32_t *cb = tb.cb + (size_t)e * tb.G * 4 * R;
    const int n_full = tb.K / 640;
    Cb3Ring ring;
    Cb3Bufs cbs;
    // code words in tile st (a full tile has 64; the row's last tile may be short)
    auto tile_words = [&](int st) { return min(64, tb.Wd - 64 * st); };
    {   // prologue: ring slots 0..PF-1 and group 0 of tile st0; words beyond the tile re-read its first word
        const uint32_t *qt = qs + (size_t)(64 * st0) * R;
        const int nw = tile_words(st0);
#pragma unroll
        for (int j = 0; j < PF; ++j) {
            ring.a[j] = ldl(2 * j < nw ? qt + (size_t)(2 * j) * R : qt, lo);
            ring.b[j] = ldl(2 * j + 1 < nw ? qt + (size_t)(2 * j + 1) * R : qt, lo);
        }
        cb3_load_group(cb, R, 5 * st0, lo, cbs.N[0], cbs.N[1], cbs.N[2], cbs.N[3]);
        cbs.A[0] = cbs.A[1] = cbs.A[2] = cbs.A[3] = make_uint4(0, 0, 0, 0);
        cbs.B[0] = cbs.B[1] = cbs.B[2] = cbs.B[3] = make_uint4(0, 0, 0, 0);
    }
    stage();
    Cb3TileCtx c;
    c.xh = xh;
    c.xl = xl;
    c.R = R;
    c.lo = lo;
    c.xs = xs;
    int st = st0;
    const int full_end = min(st1, n_full);
    for (; st < full_end; ++st) {
        const bool has_next = st + 1 < st1;
        c.qt = qs + (size_t)(64 * st) * R;
        c.qn = has_next ? c.qt + (size_t)64 * R : c.qt;
        c.nwn = has_next ? tile_words(st + 1) : 0;
        c.cbt = cb + (size_t)(5 * st) * 4 * R;
        c.cbn = has_next ? c.cbt + (size_t)20 * R : c.cbt;
        c.xb = (640 * st - c0) >> 1;
        cb3_slot<TC, HILO, 5, 0>(c, ring, cbs, acc);
    }
    if (st < st1) {                                  // the row's last, partial tile
        c.qt = c.qn = qs + (size_t)(64 * st) * R;
        c.nwn = 0;
        c.cbt = c.cbn = cb + (size_t)(5 * st) * 4 * R;
        c.xb = (640 * st - c0) >> 1;
        switch ((tb.K - 640 * st) >> 7) {
            case 1: cb3_slot<TC, HILO, 1, 0>(c, ring, cbs, acc); break;
            case 2: cb3_slot<TC, HILO, 2, 0>(c, ring, cbs, acc); break;
            case 3: cb3_slot<TC, HILO, 3, 0>(c, ring, cbs, acc); break;
            default: cb3_slot<TC, HILO, 4, 0>(c, ring, cbs, acc); break;
        }
    }
}

// Streams word pairs u0 .. u1-1 (columns 20*u0 .. min(K, 20*u1)).  Code words are prefetched MI_CB3_PF pairs
// ahead through a static register ring (slot j of the ring is refilled right after it is consumed), the codebook
// one group ahead, so every wavefront keeps several 1 KB loads in flight while it decodes.
template <int TC, bool HILO, class Stage>
__device__ __forceinline__ void cb3_accum(const Cb3Table &tb, int e, int r0, int u0, int u1, int c0,
                          const uint32_t *__restrict__ xh, const uint32_t *__restrict__ xl, int xs,
                          float (&acc)[4][TC], Stage &&stage) {
    // more activation rows = more ALU work per byte to hide latency behind, and more accumulators: shallower ring
    constexpr int PF = TC <= 2 ? MI_CB3_PF : (TC <= 8 ? 2 : 1);
    const size_t R = (size_t)tb.R;
    const int Wd = tb.Wd, K = tb.K;
    const uint32_t lo = (uint32_t)r0;
    const uint32_t *qs = tb.qs + (size_t)e * Wd * R;
    const uint32_t *cb = tb.cb + (size_t)e * tb.G * 4 * R;
    const uint4 z4 = make_uint4(0, 0, 0, 0);
    uint4 ra[PF], rb[PF];
#pragma unroll
    for (int j = 0; j < PF; ++j) {
        ra[j] = rb[j] = z4;
        const int P = u0 + j;
        if (P < u1) {
            ra[j] = ldl(qs + (size_t)(2 * P) * R, lo);
            if (2 * P + 1 < Wd) rb[j] = ldl(qs + (size_t)(2 * P + 1) * R, lo);
        }
    }
    Cb3Book bk;
    bk.g_last = (min(K, 20 * u1) - 1) >> 7;
    bk.cur_g = (20 * u0) >> 7;
    cb3_load_group(cb, R, bk.cur_g, lo, bk.lo03, bk.lo47, bk.hi03, bk.hi47);
    bk.n03 = bk.n47 = bk.m03 = bk.m47 = z4;
    if (bk.cur_g + 1 <= bk.g_last) cb3_load_group(cb, R, bk.cur_g + 1, lo, bk.n03, bk.n47, bk.m03, bk.m47);
    stage();

    int P = u0;
    for (; P + PF <= u1; P += PF) {
#pragma unroll
        for (int j = 0; j < PF; ++j) {
            const int Pj = P + j;
            const uint4 a = ra[j], b = rb[j];
            const int Pn = Pj + PF;
            if (Pn < u1) {
                ra[j] = ldl(qs + (size_t)(2 * Pn) * R, lo);
                rb[j] = (2 * Pn + 1 < Wd) ? ldl(qs + (size_t)(2 * Pn + 1) * R, lo) : z4;
            }
            cb3_pair<TC, HILO>(a, b, Pj, 2 * Pj + 1 < Wd, K, c0, cb, R, lo, bk, xh, xl, xs, acc);
        }
    }
#pragma unroll
    for (int j = 0; j < PF; ++j) {           // remainder (< PF pairs, already in the ring)
        const int Pj = P + j;
        if (Pj < u1) cb3_pair<TC, HILO>(ra[j], rb[j], Pj, 2 * Pj + 1 < Wd, K, c0, cb, R, lo, bk, xh, xl, xs, acc);
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
