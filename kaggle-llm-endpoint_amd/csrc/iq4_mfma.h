// IQ4_XS rows of the grouped decode / matvec launches on the gfx950 matrix cores.
//
// The reference's planar IQ4_XS tables (planes.py:26-28) are read as stored.  As for IQ3_S (iq3_mfma.h) the weights
// are the B operand of v_mfma_f32_16x16x32_bf16 and one k-step of 32 columns is one scale group (a 32-weight
// sub-block, scale f16(d) * (6-bit s - 32)), applied in f32 to the k-step's partial.  The B operand holds the
// non-linear levels kvalues_iq4nl (integers |v| <= 127, exact in bf16), so every weight enters exactly as the
// reference's f32 dequantization defines it (iqquant.py:137-148, planes.py:230-243).
//
// A wavefront owns 64 rows, loaded 4 rows per uint4 as four interleaved 16-row tiles (tile r = rows 4i + r of lane
// (i, q)).  In the k-step of sub-block s, lane group q takes plane word 4s + q: byte j of it holds the weights
// 4q + j (low nibble) and 16 + 4q + j (high nibble) of the sub-block, and one LDS table lookup per byte turns it into
// the bf16 pair of their levels.  The lane's 8 k-values are therefore sub-block columns {4q + j, 16 + 4q + j}
// interleaved, and the activations are staged in that order: staged position 8q + 2j + h of each 32-column group
// holds column 16h + 4q + j (iq4_stage_pos).
#pragma once
#include "iq3_mfma.h"

namespace mi {

// LDS table: byte (two 4-bit indices) -> bf16 pair (level of the low nibble, level of the high nibble).
struct Iq4Lds {
    uint32_t pair[256];
};

// Every thread of the workgroup takes part; a barrier must follow before the table is read.
__device__ __forceinline__ void iq4_fill_lds(Iq4Lds &t, const int8_t *kv) {
    for (int i = threadIdx.x; i < 256; i += blockDim.x) {
        const uint32_t lo = __float_as_uint((float)kv[i & 15]) >> 16, hi = __float_as_uint((float)kv[i >> 4]) >> 16;
        t.pair[i] = lo | (hi << 16);
    }
}

// Staged position (bf16 units, within a 32-column group) of column o (0..31) of the group.
__host__ __device__ __forceinline__ int iq4_stage_pos(int o) { return 8 * ((o >> 2) & 3) + 2 * (o & 3) + (o >> 4); }

// Half-block h (4 k-steps) of a row group: block h / 2's scales (d_c holds the d of blocks 2 (h / 4) and
// 2 (h / 4) + 1), the plane word of k-step j from word(j); done(j) runs after k-step j's matrix-core work.
template <bool TWO, class Word, class Done>
__device__ __forceinline__ void iq4m_half(const Iq4Lds &L, int h, const uint4 &d_c, const uint4 &sl_c,
                                          const uint4 &sh_c, const uint32_t *xa0, const uint32_t *xb0,
                                          f32x4 (&acc)[4], Word &&word, Done &&done) {
    const int b = h >> 1;
    float dv[4], m32[4];
    uint32_t scw[4];                                                // sub-block i's 6-bit scale at bits 8i
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        dv[r] = f16_bits_to_f32(u4c(d_c, r) >> (16 * (b & 1)));
        m32[r] = -32.0f * dv[r];
        const uint32_t l = u4c(sl_c, r) >> (16 * (h & 1)), hb = u4c(sh_c, r) >> (8 * (h & 1));
        scw[r] = (l & 15u) | ((l & 0xf0u) << 4) | ((l & 0xf00u) << 8) | ((l & 0xf000u) << 12) |
                 ((hb & 3u) << 4) | ((hb & 0xcu) << 10) | ((hb & 0x30u) << 16) | ((hb & 0xc0u) << 22);
    }
    const int xo = 64 * h;                                          // dwords of the half-block's first column
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        __builtin_amdgcn_sched_barrier(0);
        const uint4 ah = *(const uint4 *)(xa0 + xo + 16 * j);
        uint4 al = ah;
        if (TWO) al = *(const uint4 *)(xb0 + xo + 16 * j);
        const uint4 wj = word(j);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t u = u4c(wj, r);
            const uint4 bw = make_uint4(L.pair[u & 255u], L.pair[(u >> 8) & 255u], L.pair[(u >> 16) & 255u],
                                        L.pair[u >> 24]);
            const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
            f32x4 p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ah),
                                                              __builtin_bit_cast(bf16x8, bw), zero, 0, 0, 0);
            if (TWO)
                p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, al),
                                                            __builtin_bit_cast(bf16x8, bw), p, 0, 0, 0);
            const float scale = fmaf((float)((scw[r] >> (8 * j)) & 63u), dv[r], m32[r]);   // d (s - 32), exact
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[r][i] = fmaf(scale, p[i], acc[r][i]);
        }
        done(j);
    }
}

// Rows row0 .. row0 + 63 of expert e over blocks [u0, u1), activations staged (permuted) from column c0:
// acc[r][i] += sum_k W[row0 + 4 (lane % 16) + r][k] * x[token 4 (lane / 16) + i][k].
template <bool TWO, class Stage>
__device__ __forceinline__ void iq4m_accum(const Iq4Table &tb, int e, int row0, int u0, int u1, int c0,
                                           const Iq4Lds &L, const uint32_t *xa, const uint32_t *xb, f32x4 (&acc)[4],
                                           Stage &&stage) {
    const int lane = threadIdx.x & 63, q = lane >> 4;
    const size_t R = (size_t)tb.R;
    const uint32_t lo = (uint32_t)(row0 + 4 * (lane & 15));
    const uint32_t *qs = tb.qs + (size_t)e * tb.W * R;
    const uint32_t *sl = tb.sl + (size_t)e * tb.nblk * R;
    const uint32_t *sh = tb.sh + (size_t)e * tb.nblk * R;
    const uint32_t *dd = tb.d + (size_t)e * ((tb.nblk + 1) / 2) * R;
    // half-blocks h (4 sub-blocks): the lane's word in sub-block 4 (h % 2) + j of block h / 2 is 16 h + 4 j + q
    const int h0 = 2 * u0, h1 = 2 * u1;
    uint4 ring[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) ring[j] = ldl(qs + (size_t)(16 * h0 + 4 * j + q) * R, lo);
    // half-block h's block scales and d, each loaded one half-block ahead (again for a block's second half-block:
    // the loads never sit under a branch)
    // the lane's word (q) goes into its offset: a buffer load's descriptor must be wave-uniform
    const uint32_t lo_q = lo + (uint32_t)(q * R);
    uint4 sl_n = ldl_if<false>(sl + (size_t)u0 * R, lo, true), sh_n = ldl_if<false>(sh + (size_t)u0 * R, lo, true);
    uint4 d_n = ldl_if<false>(dd + (size_t)(u0 >> 1) * R, lo, true);
    stage();
    const uint32_t *xa0 = xa - (c0 >> 1), *xb0 = xb - (c0 >> 1);
    for (int h = h0; h < h1; ++h) {
        const uint4 sl_c = sl_n, sh_c = sh_n, d_c = d_n;
        const bool more = h + 1 < h1;
        sl_n = ldl_if<false>(sl + (size_t)((h + 1) >> 1) * R, lo, more);
        sh_n = ldl_if<false>(sh + (size_t)((h + 1) >> 1) * R, lo, more);
        d_n = ldl_if<false>(dd + (size_t)((h + 1) >> 2) * R, lo, more);
        iq4m_half<TWO>(L, h, d_c, sl_c, sh_c, xa0, xb0, acc, [&](int j) { return ring[j]; }, [&](int j) {
            // the ring slot takes step j of the next half-block (zeros past the split)
            ring[j] = ldl_if(qs + (size_t)(16 * (h + 1) + 4 * j) * R, lo_q, more);
        });
    }
}

// The same rows with the plane words and the block scales streamed through an LDS ring instead of registers:
// buffer_load_dwordx4 ... lds (lane l's 16 bytes land at slot + 16 l, where the lane reads them back), issued from
// inline assembly so that the compiler neither counts them nor makes the activation and table reads wait for them
// (it cannot tell that they write other LDS); every wait on them is explicit.  Two half-blocks (8 KB per
// wavefront) are in flight beside the one being decoded, at no register cost.  Loads complete in issue order per
// wavefront; per block b the loads are, in order: (even half) the scales of block b + 1 (sl, sh, d: 3), the plane
// words of half-block 2 b + 2 (4); (odd half) those of 2 b + 3 (4).  So half-block 2 b (and block b's scales,
// issued before it) has landed when at most 4 loads are outstanding, and 2 b + 1 when at most 7 are.  Loads past
// the split's end use an empty buffer range: they return zeros without touching memory, so every block issues the
// same loads.
// ring: this wavefront's kIq4RingUint4 uint4 of LDS: plane-word slots 0 and 1 (4 k-steps x 64 lanes each), then the
// scale slot (sl, sh, d x 64 lanes).
constexpr int kIq4RingUint4 = 2 * 4 * 64 + 3 * 64;
typedef int i32x4 __attribute__((ext_vector_type(4)));

// One direct-to-LDS load of 16 bytes per lane: buffer (SGPR descriptor) at voff + soff -> LDS lds + 16 * lane.
__device__ __forceinline__ void dma16(i32x4 rsrc, uint32_t lds, uint32_t voff, uint32_t soff) {
    uint32_t m0_saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
#if MI_IQ_NT
        "buffer_load_dwordx4 %2, %3, %4 offen nt lds\n\t"
#else
        "buffer_load_dwordx4 %2, %3, %4 offen lds\n\t"
#endif
        "s_mov_b32 m0, %0\n\t"
        "s_nop 0"
        : "=&s"(m0_saved)
        : "s"(lds), "v"(voff), "s"(rsrc), "s"(soff)
        : "memory");
}
template <int N>
__device__ __forceinline__ void vm_wait_asm() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void lgkm_wait_asm() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// A buffer descriptor in SGPRs over bytes [p, p + bytes) (bytes 0: an empty range).
__device__ __forceinline__ i32x4 sgpr_rsrc(const void *p, uint32_t bytes) {
    const uint64_t a = (uint64_t)p;
    return (i32x4){(int)__builtin_amdgcn_readfirstlane((uint32_t)a),
                   (int)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32) & 0xffffu),
                   (int)__builtin_amdgcn_readfirstlane(bytes), kBufferWord3};
}

template <bool TWO, class Stage>
__device__ __forceinline__ void iq4m_accum_lds(const Iq4Table &tb, int e, int row0, int u0, int u1, int c0,
                                               const Iq4Lds &L, uint4 *ring, const uint32_t *xa, const uint32_t *xb,
                                               f32x4 (&acc)[4], Stage &&stage) {
    const int lane = threadIdx.x & 63, q = lane >> 4;
    const uint32_t R = (uint32_t)tb.R, R4 = 4u * R;
    const uint32_t lo = (uint32_t)(row0 + 4 * (lane & 15));
    const int nd = (tb.nblk + 1) / 2;
    const i32x4 rq = sgpr_rsrc(tb.qs + (size_t)e * tb.W * R, (uint32_t)tb.W * R4);
    const i32x4 rsl = sgpr_rsrc(tb.sl + (size_t)e * tb.nblk * R, (uint32_t)tb.nblk * R4);
    const i32x4 rsh = sgpr_rsrc(tb.sh + (size_t)e * tb.nblk * R, (uint32_t)tb.nblk * R4);
    const i32x4 rd = sgpr_rsrc(tb.d + (size_t)e * nd * R, (uint32_t)nd * R4);
    const i32x4 rnull = sgpr_rsrc(tb.qs, 0u);
    const uint32_t vq = (uint32_t)q * R4 + 4u * lo, vs = 4u * lo;   // the lane's bytes: plane word q / 0, rows lo..
    const uint32_t lring = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)ring;
    const int h0 = 2 * u0, h1 = 2 * u1;
    // the 4 plane words of half-block hh (words 16 hh + 4 j + q) into slot hh % 2
    auto issue_words = [&](int hh) {
        const i32x4 r = hh < h1 ? rq : rnull;
        const uint32_t slot = lring + (uint32_t)(hh & 1) * 4096u;
#pragma unroll
        for (int j = 0; j < 4; ++j) dma16(r, slot + 1024u * j, vq, (uint32_t)(16 * hh + 4 * j) * R4);
    };
    // block bb's sl and sh words and its d word (the d of blocks 2 (bb / 2), +1) into the scale slot
    auto issue_scales = [&](int bb) {
        const bool in = bb < u1;
        const uint32_t slot = lring + 8192u;
        dma16(in ? rsl : rnull, slot, vs, (uint32_t)bb * R4);
        dma16(in ? rsh : rnull, slot + 1024u, vs, (uint32_t)bb * R4);
        dma16(in ? rd : rnull, slot + 2048u, vs, (uint32_t)(bb >> 1) * R4);
    };
    issue_scales(u0);
    issue_words(h0);
    issue_words(h0 + 1);
    stage();
    const uint32_t *xa0 = xa - (c0 >> 1), *xb0 = xb - (c0 >> 1);
    const uint4 *mine = ring + lane;
    for (int b = u0; b < u1; ++b) {
        uint4 sl_c, sh_c, d_c;
        // even half-block 2 b
        {
            __builtin_amdgcn_sched_barrier(0);
            vm_wait_asm<4>();
            uint4 w[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) w[j] = mine[64 * j];
            sl_c = mine[512];
            sh_c = mine[576];
            d_c = mine[640];
            // the slots are read before they are refilled
            lgkm_wait_asm();
            __builtin_amdgcn_sched_barrier(0);
            issue_scales(b + 1);
            issue_words(2 * b + 2);
            __builtin_amdgcn_sched_barrier(0);
            iq4m_half<TWO>(L, 2 * b, d_c, sl_c, sh_c, xa0, xb0, acc, [&](int j) { return w[j]; }, [](int) {});
        }
        // odd half-block 2 b + 1
        {
            __builtin_amdgcn_sched_barrier(0);
            vm_wait_asm<7>();
            uint4 w[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) w[j] = mine[256 + 64 * j];
            lgkm_wait_asm();
            __builtin_amdgcn_sched_barrier(0);
            issue_words(2 * b + 3);
            __builtin_amdgcn_sched_barrier(0);
            iq4m_half<TWO>(L, 2 * b + 1, d_c, sl_c, sh_c, xa0, xb0, acc, [&](int j) { return w[j]; }, [](int) {});
        }
    }
    // the loads past the end (empty range) still write their slots: done before the LDS is reused
    vm_wait_asm<0>();
}

// LDSR: stream the plane words through ring, this wavefront's LDS ring (iq4m_accum_lds); else the register ring.
template <bool HILO, int TCMAX, bool LDSR, class Stage>
__device__ __forceinline__ void iq4m_run_and_store(const Iq4Table &tb, int e, int row0, int u0, int u1, int c0,
                                                   const Iq4Lds &L, const uint32_t *xh, const uint32_t *xl, int xsp,
                                                   int t_rows, int n, const int *slots, float *part_base, int R,
                                                   Stage &&stage, uint4 *ring) {
    iqm_run_and_store<HILO, TCMAX>(row0, xh, xl, xsp, t_rows, n, slots, part_base, R,
                                   [&](auto two, const uint32_t *xa, const uint32_t *xb, f32x4(&acc)[4]) {
                                       if constexpr (LDSR)
                                           iq4m_accum_lds<decltype(two)::value>(tb, e, row0, u0, u1, c0, L, ring, xa,
                                                                                xb, acc, stage);
                                       else
                                           iq4m_accum<decltype(two)::value>(tb, e, row0, u0, u1, c0, L, xa, xb, acc,
                                                                            stage);
                                   });
}

}  // namespace mi
