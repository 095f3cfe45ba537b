// IQ3_S rows of the grouped decode / matvec launches on the gfx950 matrix cores.
//
// The reference's planar IQ3_S tables (planes.py:22-25,136-170: word w of a row covers inputs 16w .. 16w+15; per
// 2 words one 4-bit scale, per 16 words one f16 d) are read as stored.  The weights are the B operand of
// v_mfma_f32_16x16x32_bf16 and the activations the A operand, so a lane's output column is the weight row it
// decoded.  One k-step of 32 columns is exactly one scale group (2 words, one scale), so each k-step's 16 x 16
// partial is scaled by its rows' f32 group scale f16(d) * (1 + 2 sc) in the lanes that decoded those rows.  The B
// operand holds the signed odd grid levels, which are exact in bf16: every weight enters exactly as the reference's
// f32 dequantization defines it (planes.py:262-276, pallas_moe.py:127-144, iqquant.py:123-132).
//
// A wavefront owns 64 rows.  Lane (i, q) (i = lane % 16, q = lane / 16) loads rows 4i .. 4i+3 of a plane word with
// one uint4: row i of the four interleaved 16-row tiles r = 0..3 (tile r = rows 4i + r).  In k-step s of a block,
// lane group q holds 8 weights: word 2s + q / 2, weights 8 (q % 2) .. 8 (q % 2) + 7 (two grid indices); the
// activations are read in the same column order (natural order: column 32 s + 8 q + e).
#pragma once
#include <type_traits>

#include "cb3_tiles.h"
#include "formats.h"

namespace mi {

constexpr int kIq3WaveRows = 64;

// LDS tables of the decoder.
struct Iq3Lds {
    uint2 level[512];      // grid entry -> its 4 odd levels as bf16 (two pairs)
    uint2 smask[16];       // 4 sign bits -> the sign bits (15, 31) of 2 bf16 pairs (32 banks: reads never conflict)
};

// Every thread of the workgroup takes part; a barrier must follow before the tables are read.
__device__ __forceinline__ void iq3_fill_lds(Iq3Lds &t, const uint32_t *grid) {
    for (int i = threadIdx.x; i < 512; i += blockDim.x) {
        const uint32_t v = grid[i];
        const uint32_t b0 = __float_as_uint((float)(v & 255u)) >> 16, b1 = __float_as_uint((float)((v >> 8) & 255u)) >> 16;
        const uint32_t b2 = __float_as_uint((float)((v >> 16) & 255u)) >> 16, b3 = __float_as_uint((float)(v >> 24)) >> 16;
        t.level[i] = make_uint2(b0 | (b1 << 16), b2 | (b3 << 16));
    }
    if (threadIdx.x < 16) {
        const uint32_t s = threadIdx.x;
        t.smask[s] = make_uint2((s & 1u) << 15 | ((s >> 1) & 1u) << 31, ((s >> 2) & 1u) << 15 | ((s >> 3) & 1u) << 31);
    }
}

__device__ __forceinline__ uint32_t u4c(const uint4 &v, int r) { return r == 0 ? v.x : r == 1 ? v.y : r == 2 ? v.z : v.w; }

// Rows row0 .. row0 + 63 of expert e over blocks [u0, u1) (256 columns each), activations staged from column c0:
// acc[r][i] += sum_k W[row0 + 4 (lane % 16) + r][k] * x[token 4 (lane / 16) + i][k] (the caller maps the A rows to
// tokens).  xa / xb: the lane's A-operand row in the staged activations (+ 4 q dwords), xb the bf16 remainder rows
// for TWO (hi and lo in two instructions).  stage() runs once, after the first loads are issued.
template <bool TWO, class Stage>
__device__ __forceinline__ void iq3m_accum(const Iq3Table &tb, int e, int row0, int u0, int u1, int c0,
                                           const Iq3Lds &L, const uint32_t *xa, const uint32_t *xb, f32x4 (&acc)[4],
                                           Stage &&stage) {
    const int lane = threadIdx.x & 63, q = lane >> 4;
    const size_t R = (size_t)tb.R;
    const int W = tb.W;
    const uint32_t lo = (uint32_t)(row0 + 4 * (lane & 15));
    const uint32_t *qs = tb.qs + (size_t)e * W * R;
    const uint32_t *sg = tb.sg + (size_t)e * (W / 2) * R;
    const uint32_t *qh = tb.qh + (size_t)e * (W / 8) * R;
    const uint32_t *sc = tb.sc + (size_t)e * (W / 16) * R;
    const uint32_t *dd = tb.d + (size_t)e * ((tb.nblk + 1) / 2) * R;
    const int wsel = q >> 1, half = q & 1;
    // lane shifts: the two grid indices in the qs word, the 8 signs in the sg word, the 2 high index bits in qh
    const uint32_t qs_sh = 16 * half, sg_sh = 16 * wsel + 8 * half, qh_sh = 4 * wsel + 2 * half;
    // half-blocks h (8 words, 4 k-steps): word 8h + 2j + wsel in step j, its signs in sg row 4h + j, its high index
    // bits in qh row h (nibble 2j + wsel), its scale in sc row h / 2 (nibble 4 (h % 2) + j), d in row h / 4
    // (half h / 2 % 2)
    const int h0 = 2 * u0, h1 = 2 * u1;
    uint4 rq[4], rs[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        rq[j] = ldl(qs + (size_t)(8 * h0 + 2 * j + wsel) * R, lo);
        rs[j] = ldl(sg + (size_t)(4 * h0 + j) * R, lo);
    }
    // half-block h's qh, sc and d words, each loaded one half-block ahead (sc and d again for every half-block: the
    // loads never sit under a branch)
    // the lane's word (wsel) goes into its offset: a buffer load's descriptor must be wave-uniform
    const uint32_t lo_w = lo + (uint32_t)(wsel * R);
    uint4 qh_n = ldl(qh + (size_t)h0 * R, lo);
    uint4 sc_n = ldl_if<false>(sc + (size_t)(h0 >> 1) * R, lo, true);
    uint4 d_n = ldl_if<false>(dd + (size_t)(h0 >> 2) * R, lo, true);
    stage();
    const uint32_t *xa0 = xa - (c0 >> 1), *xb0 = xb - (c0 >> 1);
    for (int h = h0; h < h1; ++h) {
        const uint4 qh_c = qh_n, sc_c = sc_n, d_c = d_n;
        const bool more = h + 1 < h1;
        qh_n = ldl_if(qh + (size_t)(h + 1) * R, lo, more);
        sc_n = ldl_if<false>(sc + (size_t)((h + 1) >> 1) * R, lo, more);
        d_n = ldl_if<false>(dd + (size_t)((h + 1) >> 2) * R, lo, more);
        float dv[4];
        uint32_t qhl[4];                                            // the lane's high index bits, step j at bit 8j
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            dv[r] = f16_bits_to_f32(u4c(d_c, r) >> (16 * ((h >> 1) & 1)));
            qhl[r] = u4c(qh_c, r) >> qh_sh;
        }
        const int xo = 64 * h;                                      // dwords of the half-block's first column
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            __builtin_amdgcn_sched_barrier(0);
            const uint4 ah = *(const uint4 *)(xa0 + xo + 16 * j);
            uint4 al = ah;
            if (TWO) al = *(const uint4 *)(xb0 + xo + 16 * j);
            const int sn = 4 * (4 * (h & 1) + j);                      // the scale nibble's bit offset
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t t = u4c(rq[j], r) >> qs_sh;              // bytes 0, 1: the two grid indices
                const uint32_t sb = u4c(rs[j], r) >> sg_sh;             // bits 0..7: the 8 weights' signs
                const uint32_t hb = qhl[r] >> (8 * j);                   // bits 0, 1: the indices' high bits
                const uint32_t i0 = (t & 255u) | ((hb << 8) & 256u);
                const uint32_t i1 = ((t >> 8) & 255u) | ((hb << 7) & 256u);
                const uint2 g0 = L.level[i0], g1 = L.level[i1];
                const uint2 m0 = L.smask[sb & 15u], m1 = L.smask[(sb >> 4) & 15u];
                const uint4 b = make_uint4(g0.x | m0.x, g0.y | m0.y, g1.x | m1.x, g1.y | m1.y);
                const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
                f32x4 p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ah),
                                                                  __builtin_bit_cast(bf16x8, b), zero, 0, 0, 0);
                if (TWO)
                    p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, al),
                                                                __builtin_bit_cast(bf16x8, b), p, 0, 0, 0);
                const float nib = (float)((u4c(sc_c, r) >> sn) & 15u);
                const float scale = fmaf(nib, 2.0f * dv[r], dv[r]);   // d (1 + 2 sc), exact
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[r][i] = fmaf(scale, p[i], acc[r][i]);
            }
            // the ring slot takes step j of the next half-block (zeros past the split)
            rq[j] = ldl_if(qs + (size_t)(8 * (h + 1) + 2 * j) * R, lo_w, more);
            rs[j] = ldl_if(sg + (size_t)(4 * (h + 1) + j) * R, lo, more);
        }
    }
}

// 64 rows from row0 (4 interleaved tiles, lane (i, q) holding rows 4i + r), store the partials of the n real rows.
// A-operand rows (tokens of the 16-row tile):
//   bf16 activations: token m;
//   f32 activations (HILO), groups of at most 8 tokens (TCMAX <= 8): hi part of token m (m < 8) or lo part of token
//     m - 8 (m >= 8): one instruction; the two halves of the output are added at the end;
//   f32 activations, up to 16 tokens: hi and lo of token m, two instructions per k-step.
// A rows at or past the staged rows read a clamped row; their outputs are never stored.
// accum<TWO>(xa, xb, acc) runs the rows' k-steps (xa / xb: the lane's A row in the staged activations + 4 q dwords).
template <bool HILO, int TCMAX, class Accum>
__device__ __forceinline__ void iqm_run_and_store(int row0, const uint32_t *xh, const uint32_t *xl, int xsp,
                                                  int t_rows, int n, const int *slots, float *part_base, int R,
                                                  Accum &&accum) {
    const int lane = threadIdx.x & 63, m = lane & 15, q = lane >> 4;
    constexpr bool two = HILO && TCMAX > 8;
    constexpr bool pair = HILO && !two;
    int row = pair ? (m & 7) : m;
    row = min(row, t_rows - 1);
    const uint32_t *xa = ((pair && m >= 8) ? xl : xh) + row * xsp + 4 * q;
    const uint32_t *xb = xl + row * xsp + 4 * q;
    f32x4 acc[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = (f32x4){0.f, 0.f, 0.f, 0.f};
    accum(std::integral_constant<bool, two>{}, xa, xb, acc);
    if (pair) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[r][i] += __shfl_down(acc[r][i], 32);
    }
    // lane (i, q) holds tokens 4 q .. 4 q + 3 of rows row0 + 4 i + r (r = 0..3: one float4 per token)
    if (pair && q >= 2) return;
    float *dst = part_base + row0 + 4 * (lane & 15);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int t = 4 * q + i;
        if (t < n) *(float4 *)(dst + (size_t)slots[t] * R) = make_float4(acc[0][i], acc[1][i], acc[2][i], acc[3][i]);
    }
}

template <bool HILO, int TCMAX, class Stage>
__device__ __forceinline__ void iq3m_run_and_store(const Iq3Table &tb, int e, int row0, int u0, int u1, int c0,
                                                   const Iq3Lds &L, const uint32_t *xh, const uint32_t *xl, int xsp,
                                                   int t_rows, int n, const int *slots, float *part_base, int R,
                                                   Stage &&stage) {
    iqm_run_and_store<HILO, TCMAX>(row0, xh, xl, xsp, t_rows, n, slots, part_base, R,
                                   [&](auto two, const uint32_t *xa, const uint32_t *xb, f32x4(&acc)[4]) {
                                       iq3m_accum<decltype(two)::value>(tb, e, row0, u0, u1, c0, L, xa, xb, acc,
                                                                        stage);
                                   });
}

}  // namespace mi
