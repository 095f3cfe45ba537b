// Grouped codebook-dequant expert matvec: host side of the C ABI (argument validation, split planning, workspace
// layout, launches) and the exact dequant kernel.  The grouped kernels themselves live in grouped.h.
#include "cumulti.h"
#include "pstream.h"
#include "tuning.h"

#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <mutex>

namespace mi {

// ------------------------------------------------------------------------------------------------ dequant (debug)
__global__ void dequant_kernel(Table tb, int e, float *out) {
    // one thread per (row, 16 columns); writes the exact f32 weights in natural order
    const int R = tb.qtype == MI_QT_CB3    ? tb.cb3.R
                  : tb.qtype == MI_QT_IQ3_S  ? tb.iq3.R
                  : tb.qtype == MI_QT_IQ4_XS ? tb.iq4.R
                  : tb.qtype == MI_QT_IQ2_S  ? tb.iq2.R
                                             : tb.kq.R;
    const int K = tb.qtype == MI_QT_CB3    ? tb.cb3.K
                  : tb.qtype == MI_QT_IQ3_S  ? tb.iq3.K
                  : tb.qtype == MI_QT_IQ4_XS ? tb.iq4.K
                  : tb.qtype == MI_QT_IQ2_S  ? tb.iq2.K
                                             : tb.kq.K;
    const int per_row = K / 16;
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)R * per_row) return;
    const int r = (int)(i / per_row);
    const int c0 = (int)(i - (long long)r * per_row) * 16;
    const size_t Rz = (size_t)R;
    for (int c = c0; c < c0 + 16; ++c) {
        float v;
        if (tb.qtype == MI_QT_CB3) {
            // tile layout of cb3_tiles.h: column c -> tile ct, k-step m, k-chunk q, position j; code n = 8m + j
            const Cb3Table &t = tb.cb3;
            const int ct = c / kCb3TileCols, o = c % kCb3TileCols;
            const int m = o >> 5, q = (o >> 3) & 3, j = o & 7;
            const int nn = 8 * m + j, p = nn / 20, cc = nn % 20;
            const int lane = 16 * q + (r & 15);
            const uint32_t *wp = t.qs + (((size_t)e * t.CT + ct) * t.RT + (r >> 4)) * 256 + 4 * lane;
            const uint32_t a = wp[2 * p], b = wp[2 * p + 1];
            uint32_t code;
            if (cc < 4) code = (a >> (8 * cc)) & 7u;
            else if (cc < 8) code = (a >> (8 * (cc - 4) + 3)) & 7u;
            else if (cc < 12) code = (b >> (8 * (cc - 8))) & 7u;
            else if (cc < 16) code = (b >> (8 * (cc - 12) + 3)) & 7u;
            else code = ((a >> (8 * (cc - 16) + 6)) & 3u) | (((b >> (8 * (cc - 16) + 6)) & 1u) << 2);
            const uint32_t *cw = t.cb + (((size_t)e * t.G + (c >> 7)) * t.R + r) * 4;
            const uint32_t lo = cw[code >> 2], hi = cw[2 + (code >> 2)];
            const uint32_t sh = 8 * (code & 3u);
            v = bf16_to_f32(((lo >> sh) & 255u) | (((hi >> sh) & 255u) << 8));
        } else if (tb.qtype == MI_QT_Q2_K || tb.qtype == MI_QT_Q3_K) {
            // column c = 256 b + 128 n + 32 s + l (l = 4 q' + j): qs word 16 b + 8 n + q', byte j, shift 2s;
            // scale byte 8 n + 2 s + (l >= 16); Q3_K hmask byte l, bit 4 n + s
            const KqTable &t = tb.kq;
            const int b = c >> 8, n = (c >> 7) & 1, s = (c >> 5) & 3, l = c & 31, j = l & 3;
            const uint32_t q = t.qs[((size_t)e * 16 * t.nblk + 16 * b + 8 * n + (l >> 2)) * Rz + r];
            const float vq = (float)((q >> (8 * j + 2 * s)) & 3u);
            const int is = 8 * n + 2 * s + (l >= 16 ? 1 : 0);
            const uint32_t scb = (t.sc[((size_t)e * 4 * t.nblk + 4 * b + (is >> 2)) * Rz + r] >> (8 * (is & 3))) & 255u;
            const uint32_t dw = t.d[((size_t)e * t.nblk + b) * Rz + r];
            if (tb.qtype == MI_QT_Q2_K) {
                const float dl = f16_bits_to_f32(dw & 0xffffu) * (float)(scb & 15u);
                const float ml = f16_bits_to_f32(dw >> 16) * (float)(scb >> 4);
                v = dl * vq - ml;                                   // dl * vq is exact: one rounding
            } else {
                const uint32_t hmb = (t.hm[((size_t)e * 8 * t.nblk + 8 * b + (l >> 2)) * Rz + r] >> (8 * j)) & 255u;
                const float hb = (float)((hmb >> (4 * n + s)) & 1u);
                v = f16_bits_to_f32(dw & 0xffffu) * ((float)scb - 32.0f) * (vq - 4.0f * (1.0f - hb));
            }
        } else if (tb.qtype == MI_QT_IQ2_S) {
            // column c: word w, group j, position k (c = 32 w + 8 j + k); block w / 8
            const Iq2Table &t = tb.iq2;
            const int w = c >> 5, j = (c >> 3) & 3, k = c & 7;
            const uint32_t q = t.qs[((size_t)e * t.W + w) * Rz + r];
            const uint32_t sgw = t.sg[((size_t)e * t.W + w) * Rz + r];
            const uint32_t qhb = (t.qh[((size_t)e * (t.W / 4) + (w >> 2)) * Rz + r] >> (8 * (w & 3))) & 255u;
            const uint32_t scb = (t.sc[((size_t)e * (t.W / 4) + (w >> 2)) * Rz + r] >> (8 * (w & 3))) & 255u;
            const uint32_t dw = t.d[((size_t)e * ((t.nblk + 1) / 2) + (w >> 4)) * Rz + r];
            const float scale = f16_bits_to_f32(dw >> (((w >> 3) & 1) * 16)) *
                                (0.5f + (float)((scb >> (4 * (j >> 1))) & 15u)) * 0.25f;
            const uint32_t idx = ((q >> (8 * j)) & 255u) | (((qhb >> (2 * j)) & 3u) << 8);
            const uint32_t lv = (kGrid2Const[2 * idx + (k >> 2)] >> (8 * (k & 3))) & 255u;
            const uint32_t sb = (sgw >> (8 * j + k)) & 1u;
            v = scale * (float)lv * (sb ? -1.0f : 1.0f);
        } else if (tb.qtype == MI_QT_IQ4_XS) {
            // column c: block b, sub-block i, word 4i + wq, byte j, nibble pos (c = 256 b + 32 i + 16 pos + 4 wq + j)
            const Iq4Table &t = tb.iq4;
            const int b = c >> 8, i = (c >> 5) & 7, pos = (c >> 4) & 1, wq = (c >> 2) & 3, j = c & 3;
            const uint32_t q = t.qs[((size_t)e * t.W + 32 * b + 4 * i + wq) * Rz + r];
            const uint32_t slw = t.sl[((size_t)e * t.nblk + b) * Rz + r];
            const uint32_t shw = t.sh[((size_t)e * t.nblk + b) * Rz + r];
            const uint32_t dw = t.d[((size_t)e * ((t.nblk + 1) / 2) + (b >> 1)) * Rz + r];
            const int sv = (int)(((slw >> (4 * i)) & 15u) | (((shw >> (2 * i)) & 3u) << 4)) - 32;
            const uint32_t nib = (q >> (8 * j + 4 * pos)) & 15u;
            v = f16_bits_to_f32(dw >> (16 * (b & 1))) * (float)sv * (float)kKvConst[nib];
        } else {
            const Iq3Table &t = tb.iq3;
            const int w = c >> 4, jj = (c >> 2) & 3, kk = c & 3;
            const uint32_t q = t.qs[((size_t)e * t.W + w) * Rz + r];
            const uint32_t sgw = t.sg[((size_t)e * (t.W / 2) + (w >> 1)) * Rz + r];
            const uint32_t qhw = t.qh[((size_t)e * (t.W / 8) + (w >> 3)) * Rz + r];
            const uint32_t scw = t.sc[((size_t)e * (t.W / 16) + (w >> 4)) * Rz + r];
            const uint32_t dw = t.d[((size_t)e * ((t.nblk + 1) / 2) + (w >> 5)) * Rz + r];
            const uint32_t sgh = (sgw >> ((w & 1) * 16)) & 0xffffu;
            const uint32_t qhn = (qhw >> ((w & 7) * 4)) & 15u;
            const uint32_t scn = (scw >> (((w >> 1) & 7) * 4)) & 15u;
            const float scale = f16_bits_to_f32(dw >> (((w >> 4) & 1) * 16)) * (1.0f + 2.0f * (float)scn);
            const uint32_t idx = ((q >> (8 * jj)) & 255u) | (((qhn >> jj) & 1u) << 8);
            const uint32_t lv = (kGridConst[idx] >> (8 * kk)) & 255u;
            const uint32_t sb = (sgh >> (4 * jj + kk)) & 1u;
            v = scale * (float)lv * (sb ? -1.0f : 1.0f);
        }
        out[(size_t)r * K + c] = v;
    }
}

// ------------------------------------------------------------------------------------------------ finishing kernels
// Routing-weighted combine of the down partials: out[n] = sum_j w[n, j] * sum_s part[s][n*k + j]  (+ the shared
// expert's sum_s part[s][n_route + n]), experts in routing order, splits in order.  Invalid ids (outside [0, E))
// contribute nothing.  One thread per output row of one token, so a wave reads 256 contiguous bytes per partial and
// even one token spreads over D/64 waves.  The work is a few MB at most, so the launch is bound by round trips:
// every load of a chunk of experts -- up to kCombineSplits splits of each, the routing ids and the weights -- is issued
// in bounds and without a branch before the first add (a missing split or slot reads split s0 / slot 0, whose value
// is then left out), one round trip per chunk instead of one per split plus two for the ids and weights.
constexpr int kCombineChunk = 9;
constexpr int kCombineSplits = 8;
__global__ void __launch_bounds__(64) combine_kernel(const float *__restrict__ part, int S, int NS, int D, int N,
                                                     int k, const int32_t *__restrict__ idx,
                                                     const float *__restrict__ w, int E, int shared, int n_route,
                                                     float *out_f32, uint16_t *out_bf16) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N * D) return;
    const int tok = i / D, r = i - tok * D;
    const int nj = k + (shared >= 0 ? 1 : 0);
    float acc = 0.f;
    for (int j0 = 0; j0 < nj; j0 += kCombineChunk) {
        int slot[kCombineChunk], e[kCombineChunk];
        float wt[kCombineChunk], ys[kCombineChunk];
#pragma unroll
        for (int jj = 0; jj < kCombineChunk; ++jj) {
            const int j = j0 + jj;
            slot[jj] = j < k ? tok * k + j : j < nj ? n_route + tok : 0;
            const int rj = tok * k + (j < k ? j : 0);          // in bounds: k >= 1
            e[jj] = idx[rj];
            wt[jj] = w[rj];
            ys[jj] = 0.f;
        }
        for (int s0 = 0; s0 < S; s0 += kCombineSplits) {
            float p[kCombineSplits][kCombineChunk];
#pragma unroll
            for (int ss = 0; ss < kCombineSplits; ++ss) {
                const int s = s0 + ss < S ? s0 + ss : s0;
#pragma unroll
                for (int jj = 0; jj < kCombineChunk; ++jj) p[ss][jj] = part[((size_t)s * NS + slot[jj]) * D + r];
            }
#pragma unroll
            for (int ss = 0; ss < kCombineSplits; ++ss)
                if (s0 + ss < S) {
#pragma unroll
                    for (int jj = 0; jj < kCombineChunk; ++jj) ys[jj] += p[ss][jj];
                }
        }
#pragma unroll
        for (int jj = 0; jj < kCombineChunk; ++jj) {
            const int j = j0 + jj;
            if (j < k) {
                if (e[jj] >= 0 && e[jj] < E) acc = fmaf(wt[jj], ys[jj], acc);
            } else if (j < nj) {
                acc += ys[jj];
            }
        }
    }
    if (out_f32) out_f32[(size_t)tok * D + r] = acc;
    if (out_bf16) out_bf16[(size_t)tok * D + r] = (uint16_t)f32_to_bf16_rne(acc);
}

// h = silu(min(g, L)) * clip(u, -L, L) (model.py:119-122) of the gate/up split partials, splits summed in order:
// h[slot][c] from p1[s][0 = gate | 1 = up][slot][c].  h is stored as its bf16 high part (truncated) and the bf16
// remainder (hi + lo keeps 16 mantissa bits of the f32 h), the two bf16 operands the down projection multiplies.
// One thread per 4 columns of one slot.
__global__ void __launch_bounds__(64) swiglu_kernel(const float *__restrict__ p1, int S1, int NS, int I, float limit,
                                                    uint16_t *__restrict__ h_hi, uint16_t *__restrict__ h_lo) {
    const size_t n4 = (size_t)NS * I / 4;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n4) return;
    float4 g = make_float4(0.f, 0.f, 0.f, 0.f), u = g;
#pragma unroll 4
    for (int s = 0; s < S1; ++s) {
        const float4 pg = ((const float4 *)(p1 + (size_t)(2 * s) * NS * I))[i];
        const float4 pu = ((const float4 *)(p1 + (size_t)(2 * s + 1) * NS * I))[i];
        g.x += pg.x; g.y += pg.y; g.z += pg.z; g.w += pg.w;
        u.x += pu.x; u.y += pu.y; u.z += pu.z; u.w += pu.w;
    }
    const float hv[4] = {swiglu_clamped(g.x, u.x, limit), swiglu_clamped(g.y, u.y, limit),
                         swiglu_clamped(g.z, u.z, limit), swiglu_clamped(g.w, u.w, limit)};
    uint32_t hi[4], lo[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) split_bf16(hv[j], hi[j], lo[j]);
    ((uint2 *)h_hi)[i] = make_uint2(hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16));
    ((uint2 *)h_lo)[i] = make_uint2(lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16));
}

// Zero n words (the one-launch decode's counter block, before every launch of it).
__global__ void zero_words_kernel(uint32_t *__restrict__ p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

// Split reduction of a matvec: out[slot] = sum_s part[s][slot], splits in order.
__global__ void split_reduce_kernel(const float *__restrict__ part, int S, int NS, int R, float *__restrict__ out) {
    const size_t n4 = (size_t)NS * R / 4;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n4) return;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s = 0; s < S; ++s) {
        const float4 p = ((const float4 *)(part + (size_t)s * NS * R))[i];
        v.x += p.x; v.y += p.y; v.z += p.z; v.w += p.w;
    }
    ((float4 *)out)[i] = v;
}

// ------------------------------------------------------------------------------------------------ host side
static int validate_table(const mi_table *t) {
    if (!t) return MI_ERR_NULL;
    if (t->qtype < MI_QT_CB3 || t->qtype > MI_QT_Q3_K) return MI_ERR_QTYPE;
    if (t->rows <= 0 || t->rows % (t->qtype == MI_QT_CB3 ? kCb3RowAlign : kIq3WaveRows)) return MI_ERR_SHAPE;
    if (t->n_experts <= 0 || t->n_experts > kMaxExperts) return MI_ERR_SHAPE;
    if (t->qtype == MI_QT_CB3) {
        if (t->cols <= 0 || t->cols % 128) return MI_ERR_SHAPE;
        if (!t->plane[0] || !t->plane[1]) return MI_ERR_NULL;
    } else {
        if (t->cols <= 0 || t->cols % 256) return MI_ERR_SHAPE;
        const int np = t->qtype == MI_QT_Q2_K ? 3 : (t->qtype == MI_QT_IQ4_XS || t->qtype == MI_QT_Q3_K) ? 4 : 5;
        for (int i = 0; i < np; ++i)
            if (!t->plane[i]) return MI_ERR_NULL;
    }
    return MI_OK;
}

static Table make_table(const mi_table *t) {
    Table tb{};
    tb.qtype = t->qtype;
    if (t->qtype == MI_QT_CB3) {
        tb.cb3.qs = t->plane[0];
        tb.cb3.cb = t->plane[1];
        tb.cb3.R = t->rows;
        tb.cb3.K = t->cols;
        tb.cb3.CT = (t->cols + kCb3TileCols - 1) / kCb3TileCols;
        tb.cb3.RT = t->rows / 16;
        tb.cb3.G = t->cols / 128;
    } else if (t->qtype == MI_QT_Q2_K || t->qtype == MI_QT_Q3_K) {
        const bool q3 = t->qtype == MI_QT_Q3_K;
        tb.kq.qs = t->plane[0];
        tb.kq.hm = q3 ? t->plane[1] : nullptr;
        tb.kq.sc = t->plane[q3 ? 2 : 1];
        tb.kq.d = t->plane[q3 ? 3 : 2];
        tb.kq.R = t->rows;
        tb.kq.K = t->cols;
        tb.kq.nblk = t->cols / 256;
    } else if (t->qtype == MI_QT_IQ2_S) {
        tb.iq2.qs = t->plane[0];
        tb.iq2.sg = t->plane[1];
        tb.iq2.qh = t->plane[2];
        tb.iq2.sc = t->plane[3];
        tb.iq2.d = t->plane[4];
        tb.iq2.R = t->rows;
        tb.iq2.K = t->cols;
        tb.iq2.nblk = t->cols / 256;
        tb.iq2.W = 8 * (t->cols / 256);
    } else if (t->qtype == MI_QT_IQ4_XS) {
        tb.iq4.qs = t->plane[0];
        tb.iq4.sl = t->plane[1];
        tb.iq4.sh = t->plane[2];
        tb.iq4.d = t->plane[3];
        tb.iq4.R = t->rows;
        tb.iq4.K = t->cols;
        tb.iq4.nblk = t->cols / 256;
        tb.iq4.W = 32 * (t->cols / 256);
    } else {
        tb.iq3.qs = t->plane[0];
        tb.iq3.sg = t->plane[1];
        tb.iq3.qh = t->plane[2];
        tb.iq3.sc = t->plane[3];
        tb.iq3.d = t->plane[4];
        tb.iq3.R = t->rows;
        tb.iq3.K = t->cols;
        tb.iq3.nblk = t->cols / 256;
        tb.iq3.W = 16 * (t->cols / 256);
    }
    return tb;
}

static int cb3_ct(const mi_table *t) { return (t->cols + kCb3TileCols - 1) / kCb3TileCols; }
static int n_units_of(const mi_table *t) {
    if (t->qtype == MI_QT_CB3) return cb3_ct(t);                 // 160-column tiles
    return t->cols / 256;                                        // IQ2_S / IQ3_S / IQ4_XS blocks
}
// Rows per wavefront: CB3 16 rtw (rtw row tiles), IQ2_S / IQ3_S / IQ4_XS 64 (four interleaved row tiles).
static int wave_rows_of(const mi_table *t, int rtw) { return t->qtype == MI_QT_CB3 ? 16 * rtw : kIq3WaveRows; }
static int unit_cols(const mi_table *t) { return t->qtype == MI_QT_CB3 ? kCb3TileCols : 256; }


static int class_rows(int max_slots_per_group) {
    int c = 1;
    while (c < max_slots_per_group && c < kMaxT) c <<= 1;
    return c;
}

// Split s of S over nu units: [u0, u1), boundaries at multiples of `align` units (CB3: align 4 = whole super tiles,
// so no split streams lead-in column tiles).  The grouped kernel computes the same bounds.
static void split_bounds(int nu, int S, int align, int s, int *u0, int *u1) {
    const int nb = (nu + align - 1) / align;
    const int a = align * (int)((long long)s * nb / S), b = align * (int)((long long)(s + 1) * nb / S);
    *u0 = a < nu ? a : nu;
    *u1 = b < nu ? b : nu;
}

// Staging of S splits over the table's units: the largest LDS row pitch (dwords) and the largest number of units a
// wavefront streams (CB3 streams from the start of the super tile holding its first column tile, with a 4-dword skew
// on the LDS rows).
static void split_extent(const mi_table *t, int S, int align, int *xs_max, int *units_max) {
    const int nu = n_units_of(t), uc = unit_cols(t);
    const bool cb3 = t->qtype == MI_QT_CB3;
    const int cend = cb3 ? kCb3TileCols * cb3_ct(t) : t->cols;
    int bx = 0, bu = 0;
    for (int s = 0; s < S; ++s) {
        int u0, u1;
        split_bounds(nu, S, align, s, &u0, &u1);
        const int ua = cb3 ? 4 * (u0 / 4) : u0;
        const int c1 = u1 * uc < cend ? u1 * uc : cend;
        const int xs = cb3_row_pitch((c1 - ua * uc) / 2);
        if (xs > bx) bx = xs;
        if (u1 - ua > bu) bu = u1 - ua;
    }
    if (xs_max) *xs_max = bx;
    if (units_max) *units_max = bu;
}
struct Split {
    int S, align;
};
static int max_xs(const mi_table *t, Split sp) {
    int xs = 0;
    split_extent(t, sp.S, sp.align, &xs, nullptr);
    return xs;
}

static int cu_count() {
    static int n = 0;
    if (n <= 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
    }
    return n;
}

#define MI_DECL_OCC(M, Q) int occupancy_grouped_##M##_##Q(int tcmax, int rtw, size_t lds);
MI_DECL_OCC(0, 1)
MI_DECL_OCC(0, 2)
MI_DECL_OCC(0, 3)
MI_DECL_OCC(0, 4)
MI_DECL_OCC(0, 5)
MI_DECL_OCC(0, 6)
MI_DECL_OCC(1, 1)
MI_DECL_OCC(1, 2)
MI_DECL_OCC(1, 3)
MI_DECL_OCC(1, 4)
MI_DECL_OCC(1, 5)
MI_DECL_OCC(1, 6)
MI_DECL_OCC(2, 1)
MI_DECL_OCC(2, 2)
MI_DECL_OCC(2, 3)
MI_DECL_OCC(2, 4)
MI_DECL_OCC(2, 5)
MI_DECL_OCC(2, 6)
#undef MI_DECL_OCC

// Resident workgroups per CU of a grouped-kernel launch (the runtime's occupancy for that instance and LDS size;
// 2 when it cannot be queried), cached per (mode, format, token class, rows per wavefront, 512-byte LDS bucket).
static int wgs_per_cu(int mode, int qtype, int tcmax, int rtw, size_t lds) {
    static int cache[3][6][5][3][161];
    const int qi = qtype - 1;                                   // MI_QT_CB3 .. MI_QT_Q3_K
    int ti = 0, ri = rtw == 4 ? 2 : rtw - 1;
    while ((1 << ti) < tcmax && ti < 4) ++ti;
    const size_t bucket = (lds + 511) / 512;
    int *slot = bucket <= 160 ? &cache[mode][qi][ti][ri][bucket] : nullptr;
    if (slot && *slot > 0) return *slot;
    const size_t l = bucket * 512;
    int n;
    typedef int (*Occ)(int, int, size_t);
    static const Occ occ[3][6] = {{occupancy_grouped_0_1, occupancy_grouped_0_2, occupancy_grouped_0_3,
                                   occupancy_grouped_0_4, occupancy_grouped_0_5, occupancy_grouped_0_6},
                                  {occupancy_grouped_1_1, occupancy_grouped_1_2, occupancy_grouped_1_3,
                                   occupancy_grouped_1_4, occupancy_grouped_1_5, occupancy_grouped_1_6},
                                  {occupancy_grouped_2_1, occupancy_grouped_2_2, occupancy_grouped_2_3,
                                   occupancy_grouped_2_4, occupancy_grouped_2_5, occupancy_grouped_2_6}};
    n = occ[mode][qi](tcmax, rtw, l);
    if (n <= 0) n = 2;
    if (slot) *slot = n;
    return n;
}

// Launch shape of one grouped launch: column splits (S, boundary alignment in units), rows per wavefront (rtw row
// tiles for CB3) and the resulting row groups (RB per matrix, RBG workgroup row ranges).
struct Shape {
    Split sp;
    int rtw, RB, RBG;
};

// Pick the launch shape.  A launch has groups * RBG * S workgroups of 4 wavefronts; the runtime's occupancy gives
// the slots (resident workgroups over the chip), so the workgroups run in ceil(total / slots) rounds, each as long
// as a wavefront's stream: the column units it streams (CB3: from the start of its first super tile) times the
// kilobytes per unit (rtw for CB3), plus a fixed cost (first loads, staging, partial stores).  Minimise that over
// S, the boundary alignment (CB3: column tiles or whole super tiles) and rtw, with a split's LDS staging within
// 48 KB.  Overrides (mi_tuning_set, tests and measurements): knob = S, knob + 1 = rtw, knob + 2 = alignment.
static Shape choose_shape(const mi_table *t, int mode, int tcmax, int groups, int rows_lds, int bytes_per_col,
                          Knob knob, size_t lds_cap = 48 * 1024, long long fixed_slots = 0, int max_rtw = 4,
                          double fixed = 8.0, int min_rtw = 1) {
    const int nu = n_units_of(t);
    const bool cb3 = t->qtype == MI_QT_CB3;
    const int rg_per_wg = mode == kGateUp ? 2 : kWgWaves;
    // fixed: per-task cost in kilobyte-units (start, routing, staging, stores; small when tasks are pipelined)
    const int forced_rtw = tuning((Knob)(knob + 1), 0), forced_s = tuning(knob, 0),
              forced_al = tuning((Knob)(knob + 2), 1);
    Shape best{{1, 1}, cb3 ? max_rtw : 1, 0, 0};
    double best_cost = 1e30;
    long long best_tot = 0;
    for (int rtw = cb3 ? max_rtw : 1; rtw >= (cb3 ? min_rtw : 1); rtw /= 2) {
        if (forced_rtw > 0 && cb3 && rtw != forced_rtw) continue;
        const int RB = t->rows / wave_rows_of(t, rtw);
        const int RBG = (RB + rg_per_wg - 1) / rg_per_wg;
        // kilobytes a wavefront streams per unit: CB3 one 1 KB code tile per row tile + codebook; IQ2_S / IQ3_S /
        // IQ4_XS 64 rows of an 82 / 110 / 136-byte block
        const int block_bytes = t->qtype == MI_QT_IQ2_S ? 82 : t->qtype == MI_QT_IQ4_XS ? 136
                              : t->qtype == MI_QT_Q2_K ? 84 : t->qtype == MI_QT_Q3_K ? 116 : 110;
        const double kb_per_unit = cb3 ? rtw * 1.25 : 64 * block_bytes / 1024.0;
        const int aligns[2] = {cb3 ? 4 : 1, 1};
        for (int ai = 0; ai < 2; ++ai) {
            const int align = aligns[ai];
            const int nb = (nu + align - 1) / align;
            for (int s = 1; s <= nb; ++s) {
                if (forced_s > 0 && (s != (forced_s < nb ? forced_s : nb) || align != forced_al)) continue;
                int xs, units;
                split_extent(t, s, align, &xs, &units);
                const size_t lds = (size_t)xs * bytes_per_col * rows_lds;
                if (lds > lds_cap) continue;
                const long long slots =
                    fixed_slots > 0 ? fixed_slots : (long long)wgs_per_cu(mode, t->qtype, tcmax, rtw, lds) * cu_count();
                const long long tot = (long long)groups * RBG * s;
                const long long rounds = (tot + slots - 1) / slots;
                const double cost = (double)rounds * (units * kb_per_unit + fixed);
                // equal cost: more workgroups fill more of the round's slots, so every CU gets a more equal share
                // (IQ2_S gate/up at one token: 7 splits, 1008 of 1024 slots, 35.3 us against 36.7 us at 6)
                const bool tie_more = !cb3 && cost < best_cost + 1e-9 && tot > best_tot;
                if (cost < best_cost - 1e-9 || tie_more) {
                    best_cost = cost;
                    best_tot = tot;
                    best = Shape{Split{s, align}, rtw, RB, RBG};
                }
            }
        }
        if (!cb3) break;
    }
    if (best.RB == 0) {            // nothing fits the LDS budget with the overrides: one split per unit
        best.sp = Split{nu, 1};
        best.RB = t->rows / wave_rows_of(t, best.rtw);
        best.RBG = (best.RB + rg_per_wg - 1) / rg_per_wg;
    }
    return best;
}

#define MI_DECL_PSTREAM(M, T)                                                                    \
    int occupancy_pstream_##M##_##T(int rtw, size_t lds);                                        \
    void launch_pstream_##M##_##T(int rtw, dim3 grid, size_t lds, hipStream_t s, const PArgs &a);
MI_DECL_PSTREAM(0, 8)
MI_DECL_PSTREAM(0, 16)
MI_DECL_PSTREAM(1, 8)
MI_DECL_PSTREAM(1, 16)
#undef MI_DECL_PSTREAM

void launch_custream_0(int rtw, dim3 grid, size_t lds, hipStream_t s, const CArgs &a);
void launch_custream_1(int rtw, dim3 grid, size_t lds, hipStream_t s, const CArgs &a);
static void custream_launch(int mode, int rtw, dim3 grid, size_t lds, hipStream_t s, const CArgs &a) {
    (mode == kGateUp ? launch_custream_0 : launch_custream_1)(rtw, grid, lds, s, a);
}
void launch_cumulti_0(int rtw, dim3 grid, size_t lds, hipStream_t s, const MArgs &a);
void launch_cumulti_1(int rtw, dim3 grid, size_t lds, hipStream_t s, const MArgs &a);
static void cumulti_launch(int mode, int rtw, dim3 grid, size_t lds, hipStream_t s, const MArgs &a) {
    (mode == kGateUp ? launch_cumulti_0 : launch_cumulti_1)(rtw, grid, lds, s, a);
}

static int pstream_occupancy(int mode, int tc, int rtw, size_t lds) {
    if (mode == kGateUp) return (tc <= 8 ? occupancy_pstream_0_8 : occupancy_pstream_0_16)(rtw, lds);
    return (tc <= 8 ? occupancy_pstream_1_8 : occupancy_pstream_1_16)(rtw, lds);
}
static void pstream_launch(int mode, int tc, int rtw, dim3 grid, size_t lds, hipStream_t s, const PArgs &a) {
    if (mode == kGateUp) (tc <= 8 ? launch_pstream_0_8 : launch_pstream_0_16)(rtw, grid, lds, s, a);
    else (tc <= 8 ? launch_pstream_1_8 : launch_pstream_1_16)(rtw, grid, lds, s, a);
}

// Token counts above which the CB3 gate/up and down launches are persistent (below, a workgroup would get about one
// task: the one-workgroup-per-task launches start their first tiles sooner).  Measured on MI355X at the benchmark
// layer: batch 1 and 8 run faster as one workgroup per task, batch 16 as persistent ranges.
constexpr int kPersistentMinTokens = 8;

struct DecodePlan {
    int G, rows1, rows2, NS;
    int cu;                     // CB3, one token: the CU-balanced launches (custream.h), one workgroup per CU
    int cgmax;                  // their down launch: most groups one workgroup's share touches
    int cu_combine;             // their down launch does the routing-weighted combine (no combine launch)
    int cum;                    // CB3, 2..16 tokens: the CU-balanced multi-token launches (cumulti.h)
    int mgmax;                  // their down launch: groups staged at a time
    int xsp1, xsp2;             // their staged row pitches (dwords)
    int persistent;             // CB3 gate/up and down as persistent launches
    Shape s1, s2;
    int P1, P2;                 // persistent: workgroups of the two launches
    size_t lds1, lds2;          // CB3: their dynamic LDS
    size_t off_part1, off_h, off_part2, total;
};

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }
constexpr size_t kLdsPerCu = 160 * 1024;

// A persistent CB3 launch: the grid is what stays resident (the runtime's occupancy for the instance and its LDS),
// never more workgroups than the largest possible task count.
static void plan_pstream(int mode, int tc, const Shape &sh, int G, size_t staging, size_t scratch, int *P,
                         size_t *lds) {
    *lds = staging > scratch ? staging : scratch;
    int occ = pstream_occupancy(mode, tc, sh.rtw, *lds);
    if (occ <= 0) occ = 1;
    long long p = (long long)occ * cu_count();
    const long long tasks = (long long)G * sh.RBG * sh.sp.S;
    if (p > tasks) p = tasks;
    *P = (int)(p < 1 ? 1 : p);
}

// Static LDS of cumulti_kernel besides its dynamic staging and codebook slots (group table, counters).
constexpr size_t kCumultiStaticLds = 8 * 1024;

// The CU-balanced multi-token launches (cumulti.h): one workgroup per CU, the workgroups dealt to the column splits
// in proportion to their columns.  gate/up stages every token's x row of its split; down the h rows (high part and
// remainder) of up to mgmax groups at a time.  False when a split would get no workgroup or the staging cannot fit.
static bool plan_cumulti(const mi_table *gate, const mi_table *down, int N, DecodePlan &p) {
    const int P = cu_count();
    const int nu1 = n_units_of(gate), nu2 = n_units_of(down);
    const int nb1 = (nu1 + 3) / 4, nb2 = (nu2 + 3) / 4;
    // measured best at D 6144, I 2048 (8 and 16 tokens; with the rows staged by 16-byte loads, 3 gate/up splits at
    // 16 tokens: 199.3-199.6 against 202.0-202.4 us with 4, and 2 at 8: 140.3-141.2 against 142.0-142.5 with 3)
    int S1 = tuning(kTuneMS1, N <= 8 ? 2 : 3), S2 = tuning(kTuneMS2, 2);
    int r1 = tuning(kTuneMS1Rtw, 1), r2 = tuning(kTuneMS2Rtw, 2);
    S1 = S1 < 1 ? 1 : S1 > nb1 ? nb1 : S1;
    S2 = S2 < 1 ? 1 : S2 > nb2 ? nb2 : S2;
    r1 = (r1 == 2 || r1 == 4) ? r1 : 1;
    r2 = (r2 == 2 || r2 == 4) ? r2 : 1;
    // the widest split (whole super tiles) and every split's workgroup count
    auto widest = [&](int nu, int nb, int S, bool *ok) {
        int w = 0;
        *ok = true;
        for (int s = 0; s < S; ++s) {
            const int a0 = std::min(nu, 4 * (int)((long long)s * nb / S));
            const int a1 = std::min(nu, 4 * (int)((long long)(s + 1) * nb / S));
            w = std::max(w, a1 - a0);
            const long long w0 = (long long)P * a0 / nu, w1 = s + 1 < S ? (long long)P * a1 / nu : P;
            if (w1 <= w0 || a1 <= a0) *ok = false;
        }
        return w;
    };
    bool ok1, ok2;
    const int t1 = widest(nu1, nb1, S1, &ok1), t2 = widest(nu2, nb2, S2, &ok2);
    if (!ok1 || !ok2) return false;
    p.s1 = Shape{Split{S1, 4}, r1, gate->rows / (16 * r1), 0};
    p.s2 = Shape{Split{S2, 4}, r2, down->rows / (16 * r2), 0};
    p.P1 = p.P2 = P;
    p.xsp1 = cb3_row_pitch(80 * t1);
    p.xsp2 = cb3_row_pitch(80 * t2);
    const size_t cbl = sizeof(uint4) * kCuWaves * 5 * 64;
    const size_t budget = kLdsPerCu - kCumultiStaticLds;
    p.lds1 = sizeof(uint32_t) * (size_t)N * p.xsp1 + cbl;
    // groups a down share touches: at most NS groups (every slot its own), shared by the split's workgroups
    int ps_min = P;
    for (int s = 0; s < S2; ++s) {
        const int a0 = std::min(nu2, 4 * (int)((long long)s * nb2 / S2));
        const int a1 = std::min(nu2, 4 * (int)((long long)(s + 1) * nb2 / S2));
        const int w0 = (int)((long long)P * a0 / nu2), w1 = s + 1 < S2 ? (int)((long long)P * a1 / nu2) : P;
        ps_min = std::min(ps_min, w1 - w0);
    }
    const long long units = ((long long)p.NS * p.s2.RB + ps_min - 1) / ps_min;
    int gmax = (int)((units + p.s2.RB - 1) / p.s2.RB) + 1;
    const size_t per_g = sizeof(uint32_t) * 2 * (size_t)N * p.xsp2;
    const int fit = (int)((budget - cbl) / per_g);
    if (p.lds1 > budget || fit < 1) return false;
    p.mgmax = gmax < fit ? gmax : fit;
    const int forced = tuning(kTuneMGMax, 0);          // tests: fewer groups per epoch (more epochs)
    if (forced > 0 && forced < p.mgmax) p.mgmax = forced;
    p.lds2 = per_g * p.mgmax + cbl;
    // more than half of a CU's LDS: one workgroup per CU
    const size_t half = kLdsPerCu / 2 + 1024;
    if (p.lds1 < half) p.lds1 = half;
    if (p.lds2 < half) p.lds2 = half;
    return true;
}

// Plan of the single-token CU-balanced launches (custream.h); false when a launch's LDS would not fit a CU.
static bool plan_custream(const mi_table *gate, const mi_table *down, int n_route, DecodePlan &p) {
    // equal shares of (group, matrix, split, row tile) units over one workgroup per CU; splits are whole super
    // tiles (the staged rows are the full activation, so a split never starts inside a super tile)
    const int P = cu_count();
    const int nb1 = (n_units_of(gate) + 3) / 4, nb2 = (n_units_of(down) + 3) / 4;
    int S1 = tuning(kTuneCS1, 2), S2 = tuning(kTuneCS2, 1);      // measured best at D 6144, I 2048
    int r1 = tuning(kTuneCS1Rtw, 1), r2 = tuning(kTuneCS2Rtw, 1);
    S1 = S1 < 1 ? 1 : S1 > nb1 ? nb1 : S1;
    S2 = S2 < 1 ? 1 : S2 > nb2 ? nb2 : S2;
    r1 = (r1 == 2 || r1 == 4) ? r1 : 1;
    r2 = (r2 == 2 || r2 == 4) ? r2 : 1;
    p.s1 = Shape{Split{S1, 4}, r1, gate->rows / (16 * r1), 0};
    p.s2 = Shape{Split{S2, 4}, r2, down->rows / (16 * r2), 0};
    p.P1 = p.P2 = P;
    const long long per_g2 = (long long)S2 * p.s2.RB;
    const long long share = ((long long)p.NS * per_g2 + P - 1) / P;     // one group per slot
    p.cgmax = (int)((share + per_g2 - 1) / per_g2) + 1;
    if (p.cgmax > p.NS) p.cgmax = p.NS;
    // codebook slots: 5 groups x 64 lanes per wavefront (the down launch has more wavefronts)
    const size_t cbl1 = sizeof(uint4) * cu_waves<kGateUp>() * 5 * 64;
    const size_t cbl2 = sizeof(uint4) * cu_waves<kDown>() * 5 * 64;
    const size_t xsp1 = cb3_row_pitch(n_units_of(gate) * kCb3TileCols / 2);
    const size_t xsp2 = cb3_row_pitch(n_units_of(down) * kCb3TileCols / 2);
    const size_t scratch = 4 * (2 * (size_t)gate->n_experts + (size_t)n_route);
    p.lds1 = sizeof(uint32_t) * xsp1 + cbl1;
    p.lds2 = sizeof(uint32_t) * 2 * (size_t)p.cgmax * xsp2 + cbl2;
    if (p.lds1 < scratch) p.lds1 = scratch;
    if (p.lds2 < scratch) p.lds2 = scratch;
    // more than half of a CU's LDS: a second workgroup never fits beside the first, whatever the register count
    const size_t half = kLdsPerCu / 2 + 1024;
    if (p.lds1 < half) p.lds1 = half;
    if (p.lds2 < half) p.lds2 = half;
    // the down launch combines its row tiles itself when no share completes more than kCuMaxLast of them
    const long long share2 = ((long long)p.NS * S2 * p.s2.RB + P - 1) / P;
    p.cu_combine = tuning(kTuneCuCombine, 1) != 0 && share2 <= kCuMaxLast;
    // the launches' static LDS (routing copy, counters, row-tile list) is < 2 KB
    const size_t cap = kLdsPerCu - 2048;
    return p.lds1 <= cap && p.lds2 <= cap;
}

// xf32: f32 activations (staged as bf16 high part + remainder, one workgroup per task).
static DecodePlan plan_decode(const mi_table *gate, const mi_table *down, int N, int k, int shared,
                              bool xf32 = false) {
    DecodePlan p{};
    const int n_route = N * k;
    // token class of the launch: an expert sees at most one slot per token under top-k routing, so groups are
    // capped at N slots (any duplicate routing just forms additional groups)
    p.rows1 = class_rows(N < kMaxT ? N : kMaxT);
    p.rows2 = p.rows1;
    p.G = max_groups(n_route, gate->n_experts, N, shared, p.rows1);
    p.NS = n_route + (shared >= 0 ? N : 0);
    int est = N == 1 ? p.G : (p.G * 6 + 5) / 10;
    if (est < 1) est = 1;
    p.cu = gate->qtype == MI_QT_CB3 && down->qtype == MI_QT_CB3 && !xf32 && N == 1 &&
           tuning(kTuneCustream, 1) != 0;
    if (p.cu && !plan_custream(gate, down, n_route, p)) {
        p.cu = p.cu_combine = p.cgmax = 0;
        p.lds1 = p.lds2 = 0;
    }
    p.cum = !p.cu && gate->qtype == MI_QT_CB3 && down->qtype == MI_QT_CB3 && !xf32 && N >= 2 &&
            tuning(kTuneCumulti, 1) != 0;
    if (p.cum && !plan_cumulti(gate, down, N, p)) p.cum = 0;
    p.persistent = !p.cu && !p.cum && gate->qtype == MI_QT_CB3 && down->qtype == MI_QT_CB3 && !xf32 &&
                   N > tuning(kTunePersistAbove, kPersistentMinTokens);
    if (p.cum || p.cu) {
        // planned above
    } else if (p.persistent) {
        // persistent launches: tasks are pipelined, so the per-task fixed cost is small
        const long long slots = 3LL * cu_count();
        p.s1 = choose_shape(gate, kGateUp, p.rows1, est, p.rows1, 4, kTuneS1, 48 * 1024, slots, 4, 2.0);
        p.s2 = choose_shape(down, kDown, p.rows2, est, p.rows2, 8, kTuneS2, 48 * 1024, slots, 4, 2.0);
        const int tc = p.rows1 <= 8 ? 8 : 16;
        const size_t scratch = 4 * (2 * (size_t)gate->n_experts + (size_t)n_route);
        plan_pstream(kGateUp, tc, p.s1, p.G, sizeof(uint32_t) * (size_t)p.rows1 * max_xs(gate, p.s1.sp), scratch,
                     &p.P1, &p.lds1);
        plan_pstream(kDown, tc, p.s2, p.G, sizeof(uint32_t) * 2 * (size_t)p.rows2 * max_xs(down, p.s2.sp), scratch,
                     &p.P2, &p.lds2);
    } else {
        p.s1 = choose_shape(gate, kGateUp, p.rows1, est, p.rows1, xf32 ? 8 : 4, kTuneS1);
        p.s2 = choose_shape(down, kDown, p.rows2, est, p.rows2, 8, kTuneS2);
    }
    size_t off = 0;
    p.off_part1 = off;
    off = align256(off + sizeof(float) * (size_t)p.s1.sp.S * 2 * p.NS * gate->rows);
    p.off_h = off;
    off = align256(off + sizeof(float) * (size_t)p.NS * gate->rows);
    p.off_part2 = off;
    off = align256(off + sizeof(float) * (size_t)p.s2.sp.S * p.NS * down->rows);
    p.total = off;
    return p;
}

// ------------------------------------------------------------------------------------------------ fused decode
// Counter block of the fused decode kernel at the start of the decode workspace (its size depends on the table shapes
// only, so a workspace sized for any N keeps it in place): per-group h counters, per-row-range down counters, the
// error word (each on its own 128-byte line), then the dense per-(group, row range) split counters.
// After them, the row-tile counters of the single-token down launch's combine (custream.h: one per 16 rows of down,
// each on its own 128-byte line).
struct CtrLayout {
    size_t hcnt, cnt2, err, cnt1, rt, bytes;     // word offsets, total bytes
};
static CtrLayout ctr_layout(const mi_table *gate, const mi_table *down) {
    CtrLayout c{};
    const size_t rbg2_max = (size_t)(down->rows + 63) / 64, rbg1_max = (size_t)(gate->rows + 31) / 32;
    c.hcnt = 0;
    c.cnt2 = c.hcnt + (size_t)kMaxGroups * kCtrStride;
    c.err = c.cnt2 + rbg2_max * kCtrStride;
    c.cnt1 = c.err + kCtrStride;
    c.rt = (c.cnt1 + (size_t)kMaxGroups * rbg1_max + 63) & ~(size_t)63;
    c.bytes = align256(4 * (c.rt + (size_t)kRtCtrStride * (down->rows / 16)));
    return c;
}

// The counter region at the start of a decode workspace: at least kDecodeCtrRegion bytes, so the partials and h start
// at one offset for every layer shape whose counters fit.  A workspace shared by layers of different shapes then
// never holds one shape's data where another keeps counters, which must be zero when its call starts (the counter
// positions depend on the shape; every call leaves its own zero).
constexpr size_t kDecodeCtrRegion = (size_t)1 << 20;
static size_t ctr_region(const mi_table *gate, const mi_table *down) {
    const size_t b = ctr_layout(gate, down).bytes;
    return b > kDecodeCtrRegion ? b : kDecodeCtrRegion;
}

int occupancy_fused(int rtw, size_t lds);
void launch_fused(int rtw, dim3 grid, size_t lds, hipStream_t s, const FArgs &a);

// Static LDS of the fused kernel besides the dynamic staging area (group table, codebook slots, slot list, flag).
constexpr size_t kFusedStaticLds = sizeof(GroupTable) + sizeof(uint4) * kWgWaves * 5 * 64 + sizeof(int) * (kMaxT + 1);

struct FusedPlan {
    int ok;                     // the one launch applies (CB3, at most 8 tokens per group)
    int rows, G, NS, P;
    Shape s1, s2;
    size_t lds;
    int xs_max;
    size_t off_part1, off_h, off_part2, total;   // data offsets after the counter block; total incl. the block
};

// Plan of the fused launch: both phases stream with the same rows per wavefront (32 or 64: the SwiGLU of a row
// range then fills whole 128-byte lines of h's bf16 planes); the column splits come from the separate launches' cost
// model with the slots of the persistent grid (3 workgroups per CU) and a small per-task cost (tasks are pipelined).
// Overrides (mi_tuning_set): FS1[_AL|_RTW], FS2[_AL] as for choose_shape.
static FusedPlan plan_fused(const mi_table *gate, const mi_table *down, int N, int k, int shared) {
    FusedPlan p{};
    if (gate->qtype != MI_QT_CB3 || down->qtype != MI_QT_CB3 || N > kFusedMaxTokens) return p;
    const int n_route = N * k;
    p.rows = class_rows(N);
    p.G = max_groups(n_route, gate->n_experts, N, shared, p.rows);
    p.NS = n_route + (shared >= 0 ? N : 0);
    int est = N == 1 ? p.G : (p.G * 6 + 5) / 10;
    if (est < 1) est = 1;
    const long long slots = 3LL * cu_count();
    const size_t cap = kLdsPerCu / 3 - kFusedStaticLds - 256;
    p.s1 = choose_shape(gate, kGateUp, p.rows, est, p.rows, 8, kTuneFS1, cap, slots, 4, 2.0, 2);
    const int rtw = p.s1.rtw;
    p.s2 = choose_shape(down, kDown, p.rows, est, p.rows, 8, kTuneFS2, cap, slots, rtw, 2.0, rtw);
    if (p.s1.RB == 0 || p.s2.RB == 0 || p.s2.rtw != rtw || rtw < 2) return p;
    const int xs1 = max_xs(gate, p.s1.sp), xs2 = max_xs(down, p.s2.sp);
    p.xs_max = xs1 > xs2 ? xs1 : xs2;
    size_t lds = sizeof(uint32_t) * 2 * (size_t)p.rows * p.xs_max;
    const size_t scratch = 4 * (2 * (size_t)gate->n_experts + (size_t)n_route);
    if (scratch > lds) lds = scratch;
    p.lds = lds;
    int occ = occupancy_fused(rtw, lds);
    if (occ <= 0) return p;
    long long P = (long long)occ * cu_count();
    const long long tasks = (long long)p.G * (p.s1.RBG * p.s1.sp.S + p.s2.RBG * p.s2.sp.S);
    if (P > tasks) P = tasks;
    p.P = (int)(P < 1 ? 1 : P);
    size_t off = ctr_region(gate, down);
    p.off_part1 = off;
    off = align256(off + sizeof(float) * (size_t)p.s1.sp.S * 2 * p.NS * gate->rows);
    p.off_h = off;
    off = align256(off + sizeof(uint16_t) * 2 * (size_t)p.NS * gate->rows);
    p.off_part2 = off;
    off = align256(off + sizeof(float) * (size_t)p.s2.sp.S * p.NS * down->rows);
    p.total = off;
    p.ok = 1;
    return p;
}

static int launch_status() {
    hipError_t err = hipGetLastError();
    return err == hipSuccess ? MI_OK : MI_ERR_LAUNCH;
}

// The grouped kernels are instantiated in separate translation units (k_grouped.hip, built once per (mode, format))
// so the build compiles them in parallel; each unit exports one launcher.
#define MI_DECL_LAUNCH(M, Q) \
    void launch_grouped_##M##_##Q(int tcmax, int rtw, dim3 grid, dim3 block, size_t lds, hipStream_t s, const KArgs &a);
MI_DECL_LAUNCH(0, 1)
MI_DECL_LAUNCH(0, 2)
MI_DECL_LAUNCH(0, 3)
MI_DECL_LAUNCH(0, 4)
MI_DECL_LAUNCH(0, 5)
MI_DECL_LAUNCH(0, 6)
MI_DECL_LAUNCH(1, 1)
MI_DECL_LAUNCH(1, 2)
MI_DECL_LAUNCH(1, 3)
MI_DECL_LAUNCH(1, 4)
MI_DECL_LAUNCH(1, 5)
MI_DECL_LAUNCH(1, 6)
MI_DECL_LAUNCH(2, 1)
MI_DECL_LAUNCH(2, 2)
MI_DECL_LAUNCH(2, 3)
MI_DECL_LAUNCH(2, 4)
MI_DECL_LAUNCH(2, 5)
MI_DECL_LAUNCH(2, 6)
#undef MI_DECL_LAUNCH

template <int MODE>
static void launch_grouped(int qtype, int tcmax, int rtw, dim3 grid, size_t lds, hipStream_t s, const KArgs &a) {
    typedef void (*Launch)(int, int, dim3, dim3, size_t, hipStream_t, const KArgs &);
    static const Launch fn[3][6] = {{launch_grouped_0_1, launch_grouped_0_2, launch_grouped_0_3, launch_grouped_0_4,
                                     launch_grouped_0_5, launch_grouped_0_6},
                                    {launch_grouped_1_1, launch_grouped_1_2, launch_grouped_1_3, launch_grouped_1_4,
                                     launch_grouped_1_5, launch_grouped_1_6},
                                    {launch_grouped_2_1, launch_grouped_2_2, launch_grouped_2_3, launch_grouped_2_4,
                                     launch_grouped_2_5, launch_grouped_2_6}};
    fn[MODE][qtype - 1](tcmax, rtw, grid, dim3(64 * kWgWaves), lds, s, a);
}

}  // namespace mi

using namespace mi;

extern "C" {

size_t mi_moe_decode_workspace(const mi_table *gate, const mi_table *down, int32_t N, int32_t k,
                               int32_t shared_expert) {
    if (validate_table(gate) || validate_table(down) || N <= 0 || k <= 0) return 0;
    if (N > kMaxT || N * k > MI_MAX_SLOTS) return 0;
    // counter block, then the largest of the layouts (the fused launch's and the separate launches' for bf16 and
    // f32 activations)
    const size_t sep_b = plan_decode(gate, down, N, k, shared_expert).total;
    const size_t sep_f = plan_decode(gate, down, N, k, shared_expert, true).total;
    const size_t sep = ctr_region(gate, down) + (sep_b > sep_f ? sep_b : sep_f);
    const size_t fused = plan_fused(gate, down, N, k, shared_expert).total;
    return sep > fused ? sep : fused;
}

}  // extern "C"

namespace mi {

// Host-side argument checks of the separate-launch decode (every status before any launch).
static int decode_validate(const mi_table *gate, const mi_table *up, const mi_table *down, const void *x,
                           int N, int k, const int32_t *idx, const float *w, int shared_expert, float limit,
                           const float *out_f32, const uint16_t *out_bf16, int phases) {
    int st;
    if (phases < 1 || phases > 3) return MI_ERR_ARG;
    if ((st = validate_table(gate)) || (st = validate_table(up)) || (st = validate_table(down))) return st;
    if (!x || !idx || !w || ((phases & 2) && !out_f32 && !out_bf16)) return MI_ERR_NULL;
    if (up->qtype != gate->qtype || up->rows != gate->rows || up->cols != gate->cols ||
        up->n_experts != gate->n_experts)
        return MI_ERR_MISMATCH;
    if (down->cols != gate->rows || down->n_experts != gate->n_experts) return MI_ERR_MISMATCH;
    if (N <= 0 || N > kMaxT || k <= 0 || N * k > MI_MAX_SLOTS) return MI_ERR_TOKENS;
    if (shared_expert >= gate->n_experts || shared_expert < -1) return MI_ERR_ARG;
    if (!(limit > 0.0f)) return MI_ERR_ARG;
    return MI_OK;
}

// The separate launches of one decode layer (arguments already validated): ws is the data region (partials, h) of
// p.total bytes -- past the counter block of a caller's workspace, or the library's static scratch.
// x: bf16 [N, D], or f32 [N, D] when xf32 (the plan must have been made for it).
// ws: the data region (partials, h); rt_ctr: the row-tile counters of the single-token down launch's combine (zero
// between launches), or null where that launch is to leave the combine to the combine launch.
static int decode_launch(const DecodePlan &p, const mi_table *gate, const mi_table *up, const mi_table *down,
                         const void *x, bool xf32, int N, int k, const int32_t *idx, const float *w,
                         int shared_expert, float limit, float *out_f32, uint16_t *out_bf16, char *ws, int phases,
                         hipStream_t s, uint32_t *rt_ctr = nullptr) {
    const uint16_t *x_bf16 = xf32 ? nullptr : (const uint16_t *)x;
    int st;
    KArgs a{};
    a.E = gate->n_experts;
    a.n_route = N * k;
    a.N = N;
    a.k = k;
    a.shared_expert = shared_expert;
    a.idx = idx;
    a.NS = p.NS;

    // phase 1: gate + up -> split-K partials [S1, 2, NS, I]
    a.t0 = make_table(gate);
    a.t1 = make_table(up);
    a.R = gate->rows;
    a.K = gate->cols;
    a.S = p.s1.sp.S;
    a.ualign = p.s1.sp.align;
    a.n_units = n_units_of(gate);
    a.RB = p.s1.RB;
    a.RBW = 2;
    a.RBG = p.s1.RBG;
    a.xs_max = max_xs(gate, p.s1.sp);
    a.t_rows = p.rows1;
    a.x_bf16 = x_bf16;
    a.x_f32 = xf32 ? (const float *)x : nullptr;
    a.x_stride = gate->cols;
    a.part = (float *)(ws + p.off_part1);
    size_t lds1 = sizeof(uint32_t) * (xf32 ? 2 : 1) * (size_t)a.t_rows * a.xs_max;
    const bool cb3 = p.persistent;
    const int tc = a.t_rows <= 8 ? 8 : 16;
    PArgs pa{};
    if (cb3) {
        pa.t0 = a.t0.cb3;
        pa.t1 = a.t1.cb3;
        pa.R = a.R;
        pa.K = a.K;
        pa.E = a.E;
        pa.n_route = a.n_route;
        pa.N = N;
        pa.k = k;
        pa.shared_expert = shared_expert;
        pa.NS = p.NS;
        pa.t_rows = a.t_rows;
        pa.S = a.S;
        pa.al = a.ualign;
        pa.nu = a.n_units;
        pa.RB = a.RB;
        pa.RBG = a.RBG;
        pa.xs_max = a.xs_max;
        pa.P = p.P1;
        pa.x = x_bf16;
        pa.x_lo = nullptr;
        pa.idx = idx;
        pa.part = a.part;
    }
    // the CU-balanced single-token launches: one workgroup per CU, equal unit shares
    CArgs ca{};
    if (p.cu) {
        ca.t0 = a.t0.cb3;
        ca.t1 = a.t1.cb3;
        ca.R = gate->rows;
        ca.K = gate->cols;
        ca.E = a.E;
        ca.n_route = a.n_route;
        ca.N = N;
        ca.k = k;
        ca.shared_expert = shared_expert;
        ca.NS = p.NS;
        ca.S = p.s1.sp.S;
        ca.al = 4;
        ca.nu = n_units_of(gate);
        ca.RT = p.s1.RB;
        ca.P = p.P1;
        ca.gmax = 1;
        ca.xsp = cb3_row_pitch(ca.nu * kCb3TileCols / 2);
        ca.x = x_bf16;
        ca.x_lo = nullptr;
        ca.idx = idx;
        ca.part = a.part;
    }
    // the CU-balanced multi-token launches
    MArgs ma{};
    if (p.cum) {
        ma.t0 = a.t0.cb3;
        ma.t1 = a.t1.cb3;
        ma.R = gate->rows;
        ma.K = gate->cols;
        ma.E = a.E;
        ma.n_route = a.n_route;
        ma.N = N;
        ma.k = k;
        ma.shared_expert = shared_expert;
        ma.NS = p.NS;
        ma.S = p.s1.sp.S;
        ma.al = 4;
        ma.nu = n_units_of(gate);
        ma.RT = p.s1.RB;
        ma.P = p.P1;
        ma.gmax = 0;
        ma.xsp = p.xsp1;
        ma.x = x_bf16;
        ma.x_lo = nullptr;
        ma.idx = idx;
        ma.part = a.part;
    }
    if (phases & 1) {
        if (p.cum) cumulti_launch(kGateUp, p.s1.rtw, dim3(p.P1), p.lds1, s, ma);
        else if (p.cu) custream_launch(kGateUp, p.s1.rtw, dim3(p.P1), p.lds1, s, ca);
        else if (cb3) pstream_launch(kGateUp, tc, p.s1.rtw, dim3(p.P1), p.lds1, s, pa);
        else launch_grouped<kGateUp>(gate->qtype, a.t_rows, p.s1.rtw, dim3(p.G * p.s1.RBG * p.s1.sp.S), lds1, s, a);
        if ((st = launch_status())) return st;
    }
    if (!(phases & 2)) return MI_OK;

    // phase 2: h = SwiGLU(sum of the phase-1 partials) [NS, I]; down -> split partials [S2, NS, D]; the
    // routing-weighted combine (+ shared expert) -> out [N, D].  Stream order publishes each launch's results.
    uint16_t *h_hi = (uint16_t *)(ws + p.off_h), *h_lo = h_hi + (size_t)p.NS * gate->rows;
    // One workgroup per task (the grouped launches): at one token the down launch forms h itself while staging its
    // rows (the SwiGLU launch's arithmetic, from the gate/up partials) instead of a SwiGLU launch: the down launch
    // waits ~2.5 us longer for the split partials, the layer is 0.4-1.0 us faster (IQ2_S + IQ4_XS, IQ3_S, IQ4_XS).
    // At 8 tokens that wait costs 8-18 us per layer, so the SwiGLU launch stays.  The FUSE_SWIGLU override (0 / 1)
    // forces either (measurement).
    const bool fuse_h = !cb3 && !p.cu && !p.cum && tuning(kTuneFuseSwiglu, N == 1 ? 1 : 0) == 1;
    // the CU-balanced down launch forms h itself while staging (bit-identical h, one launch fewer: ~2 us at one token;
    // the CU_FORM_H override 0 keeps the SwiGLU launch, for measurement)
    const bool cu_form = p.cu && tuning(kTuneCuFormH, 1) != 0 &&
                         (long long)p.cgmax * (n_units_of(down) * kCb3TileCols / 4) <=
                             (long long)kCuFormIt * 64 * cu_waves<kDown>();
    if (!fuse_h && !cu_form) {
        const size_t n4 = (size_t)p.NS * gate->rows / 4;
        hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((n4 + 63) / 64)), dim3(64), 0, s,
                           (const float *)(ws + p.off_part1), p.s1.sp.S, p.NS, gate->rows, limit, h_hi, h_lo);
        if ((st = launch_status())) return st;
    }
    KArgs b = a;
    b.t0 = make_table(down);
    b.t1 = b.t0;
    b.R = down->rows;
    b.K = down->cols;
    b.S = p.s2.sp.S;
    b.ualign = p.s2.sp.align;
    b.n_units = n_units_of(down);
    b.RB = p.s2.RB;
    b.RBW = kWgWaves;
    b.RBG = p.s2.RBG;
    b.xs_max = max_xs(down, p.s2.sp);
    b.t_rows = p.rows2;
    b.x_bf16 = h_hi;
    b.x_lo = h_lo;
    b.x_f32 = nullptr;
    b.x_stride = gate->rows;
    b.gu_part = fuse_h ? (const float *)(ws + p.off_part1) : nullptr;
    b.gu_S = p.s1.sp.S;
    b.limit = limit;
    b.part = (float *)(ws + p.off_part2);
    size_t lds2 = sizeof(uint32_t) * 2 * (size_t)b.t_rows * b.xs_max;
    if (p.cum) {
        MArgs mb = ma;
        mb.t0 = mb.t1 = b.t0.cb3;
        mb.R = down->rows;
        mb.K = down->cols;
        mb.S = p.s2.sp.S;
        mb.nu = n_units_of(down);
        mb.RT = p.s2.RB;
        mb.P = p.P2;
        mb.gmax = p.mgmax;
        mb.xsp = p.xsp2;
        mb.x = h_hi;
        mb.x_lo = h_lo;
        mb.part = b.part;
        cumulti_launch(kDown, p.s2.rtw, dim3(p.P2), p.lds2, s, mb);
    } else if (p.cu) {
        CArgs cb = ca;
        cb.t0 = cb.t1 = b.t0.cb3;
        cb.R = down->rows;
        cb.K = down->cols;
        cb.S = p.s2.sp.S;
        cb.nu = n_units_of(down);
        cb.RT = p.s2.RB;
        cb.P = p.P2;
        cb.gmax = p.cgmax;
        cb.xsp = cb3_row_pitch(cb.nu * kCb3TileCols / 2);
        cb.x = h_hi;
        cb.x_lo = h_lo;
        cb.gu_part = cu_form ? (const float *)(ws + p.off_part1) : nullptr;
        cb.gu_S = p.s1.sp.S;
        cb.limit = limit;
        cb.part = b.part;
        if (p.cu_combine && rt_ctr) {
            cb.w = w;
            cb.rt_ctr = rt_ctr;
            cb.out_f32 = out_f32;
            cb.out_bf16 = out_bf16;
        }
        custream_launch(kDown, p.s2.rtw, dim3(p.P2), p.lds2, s, cb);
        if (cb.rt_ctr) return launch_status();      // the launch combined its row tiles
    } else if (cb3) {
        PArgs pb = pa;
        pb.t0 = b.t0.cb3;
        pb.t1 = b.t0.cb3;
        pb.R = b.R;
        pb.K = b.K;
        pb.S = b.S;
        pb.al = b.ualign;
        pb.nu = b.n_units;
        pb.RB = b.RB;
        pb.RBG = b.RBG;
        pb.xs_max = b.xs_max;
        pb.P = p.P2;
        pb.x = h_hi;
        pb.x_lo = h_lo;
        pb.part = b.part;
        pstream_launch(kDown, tc, p.s2.rtw, dim3(p.P2), p.lds2, s, pb);
    } else {
        launch_grouped<kDown>(down->qtype, b.t_rows, p.s2.rtw, dim3(p.G * p.s2.RBG * p.s2.sp.S), lds2, s, b);
    }
    if ((st = launch_status())) return st;
    const int D = down->rows, nthr = N * D;
    hipLaunchKernelGGL(combine_kernel, dim3((nthr + 63) / 64), dim3(64), 0, s, b.part, p.s2.sp.S, p.NS, D, N, k, idx, w,
                       gate->n_experts, shared_expert, N * k, out_f32, out_bf16);
    return launch_status();
}

// ------------------------------------------------------------------------------------------------ static scratch
// The working memory of mi_moe_decode_noalloc: one array per GPU, alive until the process ends.  Its first
// kNoallocCtrBytes hold the single-token down launch's row-tile counters (zeroed once per device, and left zero by
// every launch), the rest is the data region (partials, h).  In host code the array's name only stands in for it; its device address
// comes from hipGetSymbolAddress, taken once per device with that device current, and only that address is ever
// handed to a kernel.
static __device__ __align__(256) uint8_t scratch[MI_NOALLOC_SCRATCH_BYTES];
constexpr size_t kNoallocCtrBytes = 256 * 1024;

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void *g_scratch_ptr[kMaxDevices];

// Device address of the current device's scratch array (nullptr when it cannot be resolved).  The first call on a
// device also clears the counter region with a fill kernel on `s` (no memset node if the call is captured).
static void *scratch_ptr(hipStream_t s) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
        const int nw = (int)(kNoallocCtrBytes / 4);
        hipLaunchKernelGGL(zero_words_kernel, dim3((nw + 255) / 256), dim3(256), 0, s, (uint32_t *)ptr, nw);
        if (hipGetLastError() != hipSuccess) return nullptr;
        g_scratch_ptr[dev] = ptr;
    }
    return g_scratch_ptr[dev];
}

}  // namespace mi

extern "C" {

int mi_moe_decode_phases(const mi_table *gate, const mi_table *up, const mi_table *down, const uint16_t *x_bf16,
                         int32_t N, int32_t k, const int32_t *idx, const float *w, int32_t shared_expert,
                         float limit, float *out_f32, uint16_t *out_bf16, void *workspace, size_t workspace_bytes,
                         int32_t phases, void *stream) {
    const int st = decode_validate(gate, up, down, x_bf16, N, k, idx, w, shared_expert, limit, out_f32, out_bf16,
                                   phases);
    if (st) return st;
    const DecodePlan p = plan_decode(gate, down, N, k, shared_expert);
    const CtrLayout cl = ctr_layout(gate, down);
    const size_t region = ctr_region(gate, down);
    if (!workspace || workspace_bytes < region + p.total) return MI_ERR_WORKSPACE;
    // the single-token down launch's combine uses its row-tile counters of the block at the start of the workspace; the
    // fused launch's counters stay untouched
    return decode_launch(p, gate, up, down, x_bf16, false, N, k, idx, w, shared_expert, limit, out_f32, out_bf16,
                         (char *)workspace + region, phases, (hipStream_t)stream, (uint32_t *)workspace + cl.rt);
}

int mi_moe_decode_x(const mi_table *gate, const mi_table *up, const mi_table *down, const void *x, int32_t x_dtype,
                    int32_t N, int32_t k, const int32_t *idx, const float *w, int32_t shared_expert, float limit,
                    float *out_f32, uint16_t *out_bf16, void *workspace, size_t workspace_bytes, void *stream) {
    if (x_dtype != MI_X_BF16 && x_dtype != MI_X_F32) return MI_ERR_ARG;
    const int st = decode_validate(gate, up, down, x, N, k, idx, w, shared_expert, limit, out_f32, out_bf16, 3);
    if (st) return st;
    const bool xf32 = x_dtype == MI_X_F32;
    const DecodePlan p = plan_decode(gate, down, N, k, shared_expert, xf32);
    const size_t ctr_bytes = ctr_region(gate, down);
    if (!workspace || workspace_bytes < ctr_bytes + p.total) return MI_ERR_WORKSPACE;
    return decode_launch(p, gate, up, down, x, xf32, N, k, idx, w, shared_expert, limit, out_f32, out_bf16,
                         (char *)workspace + ctr_bytes, 3, (hipStream_t)stream);
}

int mi_moe_decode_noalloc(const mi_table *gate, const mi_table *up, const mi_table *down, const uint16_t *x_bf16,
                          int32_t N, int32_t k, const int32_t *idx, const float *w, int32_t shared_expert,
                          float limit, float *out_f32, uint16_t *out_bf16, void *stream) {
    const int st = decode_validate(gate, up, down, x_bf16, N, k, idx, w, shared_expert, limit, out_f32, out_bf16, 3);
    if (st) return st;
    const DecodePlan p = plan_decode(gate, down, N, k, shared_expert);
    if (p.total > (size_t)MI_NOALLOC_SCRATCH_BYTES - kNoallocCtrBytes) return MI_ERR_WORKSPACE;
    char *base = (char *)scratch_ptr((hipStream_t)stream);
    if (!base) return MI_ERR_LAUNCH;
    // the down launch's row-tile counters in the array's first kNoallocCtrBytes (when the table's row tiles fit there)
    const bool ctr_fits = 4 * (size_t)kRtCtrStride * (down->rows / 16) <= kNoallocCtrBytes;
    return decode_launch(p, gate, up, down, x_bf16, false, N, k, idx, w, shared_expert, limit, out_f32, out_bf16,
                         base + kNoallocCtrBytes, 3, (hipStream_t)stream, ctr_fits ? (uint32_t *)base : nullptr);
}

int mi_moe_decode(const mi_table *gate, const mi_table *up, const mi_table *down, const uint16_t *x_bf16,
                  int32_t N, int32_t k, const int32_t *idx, const float *w, int32_t shared_expert, float limit,
                  float *out_f32, uint16_t *out_bf16, void *workspace, size_t workspace_bytes, void *stream) {
    return mi_moe_decode_phases(gate, up, down, x_bf16, N, k, idx, w, shared_expert, limit, out_f32, out_bf16,
                                workspace, workspace_bytes, 3, stream);
}

int mi_moe_decode_fused(const mi_table *gate, const mi_table *up, const mi_table *down, const uint16_t *x_bf16,
                        int32_t N, int32_t k, const int32_t *idx, const float *w, int32_t shared_expert, float limit,
                        float *out_f32, uint16_t *out_bf16, void *workspace, size_t workspace_bytes, void *stream) {
    int st;
    if ((st = validate_table(gate)) || (st = validate_table(up)) || (st = validate_table(down))) return st;
    if (gate->qtype != MI_QT_CB3) return MI_ERR_QTYPE;
    if (N <= 0 || N > kFusedMaxTokens || k <= 0 || N * k > MI_MAX_SLOTS) return MI_ERR_TOKENS;
    if (shared_expert >= gate->n_experts || shared_expert < -1) return MI_ERR_ARG;
    const FusedPlan p = plan_fused(gate, down, N, k, shared_expert);
    if (!p.ok) return MI_ERR_SHAPE;
    if (!x_bf16 || !idx || !w || (!out_f32 && !out_bf16)) return MI_ERR_NULL;
    if (up->qtype != gate->qtype || up->rows != gate->rows || up->cols != gate->cols ||
        up->n_experts != gate->n_experts)
        return MI_ERR_MISMATCH;
    if (down->qtype != gate->qtype || down->cols != gate->rows || down->n_experts != gate->n_experts)
        return MI_ERR_MISMATCH;
    if (shared_expert < -1) return MI_ERR_ARG;
    if (!(limit > 0.0f)) return MI_ERR_ARG;
    if (!workspace || workspace_bytes < p.total) return MI_ERR_WORKSPACE;
    char *ws = (char *)workspace;
    uint32_t *ctr = (uint32_t *)workspace;
    const CtrLayout cl = ctr_layout(gate, down);
    FArgs a{};
    a.gate = make_table(gate).cb3;
    a.up = make_table(up).cb3;
    a.down = make_table(down).cb3;
    a.D = gate->cols;
    a.I = gate->rows;
    a.E = gate->n_experts;
    a.N = N;
    a.k = k;
    a.n_route = N * k;
    a.shared_expert = shared_expert;
    a.NS = p.NS;
    a.t_rows = p.rows;
    a.limit = limit;
    a.x = x_bf16;
    a.idx = idx;
    a.w = w;
    a.part1 = (float *)(ws + p.off_part1);
    a.h_hi = (uint16_t *)(ws + p.off_h);
    a.h_lo = a.h_hi + (size_t)p.NS * gate->rows;
    a.part2 = (float *)(ws + p.off_part2);
    a.out_f32 = out_f32;
    a.out_bf16 = out_bf16;
    a.hcnt = ctr + cl.hcnt;
    a.cnt2 = ctr + cl.cnt2;
    a.err = ctr + cl.err;
    a.cnt1 = ctr + cl.cnt1;
    a.S1 = p.s1.sp.S;
    a.al1 = p.s1.sp.align;
    a.nu1 = n_units_of(gate);
    a.RB1 = p.s1.RB;
    a.RBG1 = p.s1.RBG;
    a.S2 = p.s2.sp.S;
    a.al2 = p.s2.sp.align;
    a.nu2 = n_units_of(down);
    a.RB2 = p.s2.RB;
    a.RBG2 = p.s2.RBG;
    a.xs_max = p.xs_max;
    a.P = p.P;
    // polls before a wait gives up: the SPIN_LIMIT override replaces the default (tests force a give-up with it)
    const int spin = tuning(kTuneSpinLimit, -1);
    a.spin_limit = spin >= 0 ? (uint32_t)spin : kSpinLimit;
    // a fresh counter block and error word for this launch (a fill kernel: no memset node if the call is captured)
    const int nw = (int)(cl.bytes / 4);
    hipLaunchKernelGGL(zero_words_kernel, dim3((nw + 255) / 256), dim3(256), 0, (hipStream_t)stream, ctr, nw);
    if ((st = launch_status())) return st;
    launch_fused(p.s1.rtw, dim3(p.P), p.lds, (hipStream_t)stream, a);
    return launch_status();
}

int mi_moe_decode_plan(const mi_table *gate, const mi_table *down, int32_t N, int32_t k, int32_t shared_expert,
                       int32_t *info, int32_t n_info) {
    if (validate_table(gate) || validate_table(down) || !info || N <= 0 || N > kMaxT || k <= 0 ||
        N * k > MI_MAX_SLOTS)
        return MI_ERR_ARG;
    int32_t v[27] = {0};
    {
        const DecodePlan d = plan_decode(gate, down, N, k, shared_expert);
        const bool pers = d.persistent || d.cu || d.cum;
        const int32_t f[8] = {d.s1.sp.S, d.s1.rtw, pers ? d.P1 : 0, d.s2.sp.S, d.s2.rtw, pers ? d.P2 : 0,
                              (int32_t)d.lds1, (int32_t)d.lds2};
        for (int i = 0; i < 8; ++i) v[16 + i] = f[i];
        v[24] = d.cum ? 3 : d.cu ? 2 : d.persistent ? 1 : 0;
        v[25] = d.cu && d.cu_combine ? 1 : 0;
    }
    const FusedPlan p = plan_fused(gate, down, N, k, shared_expert);
    if (p.ok) {
        const int32_t f[14] = {1, p.P, 0, p.s1.sp.S, p.s1.sp.align, p.s1.rtw, p.s1.RBG, p.s2.sp.S, p.s2.sp.align,
                               p.s2.rtw, p.s2.RBG, (int32_t)p.lds, p.G, p.rows};
        for (int i = 0; i < 14; ++i) v[i] = f[i];
    }
    v[14] = (int32_t)ctr_layout(gate, down).err;
    v[15] = (int32_t)ctr_layout(gate, down).bytes;
    for (int i = 0; i < n_info && i < 27; ++i) info[i] = v[i];
    return MI_OK;
}

// Split count of mi_matvec: a function of (table, n_slots) only, so the workspace size is known beforehand.  The LDS
// budget is checked for f32 activations (the larger staging), which also covers bf16.
static Shape matvec_shape(const mi_table *t, int n_slots) {
    const int rows = class_rows(n_slots < kMaxT ? n_slots : kMaxT);
    const int G = max_groups(n_slots, t->n_experts, 0, -1, rows);
    return choose_shape(t, kMatvec, rows, G, rows, 8, kTuneSMV);
}

size_t mi_matvec_workspace(const mi_table *t, int32_t n_slots) {
    if (validate_table(t) || n_slots <= 0 || n_slots > MI_MAX_SLOTS) return 0;
    const int S = matvec_shape(t, n_slots).sp.S;
    // one split writes the output directly; more keep their partials here for the split reduction
    return S == 1 ? 256 : align256(sizeof(float) * (size_t)S * n_slots * t->rows);
}

int mi_matvec(const mi_table *t, const int32_t *idx, int32_t n_slots, const void *x, int32_t x_dtype,
              int32_t x_stride, float *out, void *workspace, size_t workspace_bytes, void *stream) {
    int st;
    if ((st = validate_table(t))) return st;
    if (!idx || !x || !out) return MI_ERR_NULL;
    if (n_slots <= 0 || n_slots > MI_MAX_SLOTS) return MI_ERR_TOKENS;
    if (x_dtype != MI_X_BF16 && x_dtype != MI_X_F32) return MI_ERR_ARG;
    if (x_stride < t->cols || x_stride % 4) return MI_ERR_ARG;
    const size_t need = mi_matvec_workspace(t, n_slots);
    if (!workspace || workspace_bytes < need) return MI_ERR_WORKSPACE;
    const int rows = class_rows(n_slots < kMaxT ? n_slots : kMaxT);
    const int G = max_groups(n_slots, t->n_experts, 0, -1, rows);
    const Shape sh = matvec_shape(t, n_slots);
    const Split sp = sh.sp;
    const int S = sp.S;
    const int nu = n_units_of(t);
    KArgs a{};
    a.t0 = make_table(t);
    a.t1 = a.t0;
    a.R = t->rows;
    a.K = t->cols;
    a.E = t->n_experts;
    a.n_route = n_slots;
    a.N = 0;
    a.k = 1;
    a.shared_expert = -1;
    a.S = S;
    a.ualign = sp.align;
    a.n_units = nu;
    a.RB = sh.RB;
    a.RBW = kWgWaves;
    a.RBG = sh.RBG;
    a.xs_max = max_xs(t, sp);
    a.t_rows = rows;
    a.x_bf16 = x_dtype == MI_X_BF16 ? (const uint16_t *)x : nullptr;
    a.x_f32 = x_dtype == MI_X_F32 ? (const float *)x : nullptr;
    a.x_stride = x_stride;
    a.idx = idx;
    a.NS = n_slots;
    a.part = S == 1 ? out : (float *)workspace;
    size_t lds = sizeof(uint32_t) * (x_dtype == MI_X_F32 ? 2 : 1) * (size_t)a.t_rows * a.xs_max;
    launch_grouped<kMatvec>(t->qtype, a.t_rows, sh.rtw, dim3(G * a.RBG * S), lds, (hipStream_t)stream, a);
    if ((st = launch_status()) || S == 1) return st;
    const size_t n4 = (size_t)n_slots * t->rows / 4;
    hipLaunchKernelGGL(split_reduce_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       a.part, S, n_slots, t->rows, out);
    return launch_status();
}

int mi_dequant(const mi_table *t, int32_t expert, float *out, void *stream) {
    int st;
    if ((st = validate_table(t))) return st;
    if (!out) return MI_ERR_NULL;
    if (expert < 0 || expert >= t->n_experts) return MI_ERR_ARG;
    const long long n = (long long)t->rows * (t->cols / 16);
    const int bs = 256;
    hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)((n + bs - 1) / bs)), dim3(bs), 0, (hipStream_t)stream,
                       make_table(t), expert, out);
    return launch_status();
}

const char *mi_strerror(int status) {
    switch (status) {
        case MI_OK: return "ok";
        case MI_ERR_NULL: return "a required pointer is NULL";
        case MI_ERR_QTYPE: return "unsupported qtype";
        case MI_ERR_SHAPE: return "unsupported table shape";
        case MI_ERR_TOKENS: return "token / slot count outside the entry point's limits";
        case MI_ERR_WORKSPACE: return "workspace missing or too small";
        case MI_ERR_MISMATCH: return "gate/up/down tables do not chain";
        case MI_ERR_LAUNCH: return "HIP launch error";
        case MI_ERR_ARG: return "invalid argument";
        default: return "unknown status";
    }
}

int mi_version(void) { return 1; }

}  // extern "C"
