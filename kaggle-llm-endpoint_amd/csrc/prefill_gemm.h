// Grouped GEMMs of the prefill for CB3, IQ2_S, IQ3_S, IQ4_XS, Q2_K and Q3_K experts on the gfx950 matrix cores (the
// reference's moe_ragged_gateup / moe_ragged_down, pallas_moe.py:622-755, and the rounding forms of its other bf16
// prefill branches, resident.py:122-135,169-210):
//   prefill_kernel<MODE, WP, FORM>  one workgroup per (block, row range) streams the block's expert once for all
//                       its rows: each wavefront owns 64 weight rows x up to 80 rows of activations (5 MFMA token
//                       tiles), decodes every weight once (CB3: the decoder of cb3_tiles.h; IQ3_S: the planes straight
//                       into the A operand) and reuses it across the token tiles; the block's activation rows are
//                       staged one column tile (160 / 128 columns) at a time in LDS;
//                         gate/up: h = bf16(silu(min(g, L)) * clip(u, -L, L)), g and u f32    (pallas_moe.py:682)
//                         down:    y = bf16(h Wd^T), f32 accumulation                        (pallas_moe.py:747)
//                       FORM adds the other branches' rounding points at compile time (kPfRoundGU, kPfScaleH, kPfY32).
// Each (MODE, FORM) is instantiated for every format in a translation unit of its own (k_prefill.hip), which
// exports launch_prefill_<MODE>_<FORM>.
#pragma once
#include <type_traits>

#include "cb3_tiles.h"
#include "formats.h"

namespace mi {

// IQ3_S grid levels (internal linkage: every translation unit that launches a kernel carries its own copy)
static __constant__ uint32_t kPfGrid[512] = {
#include "iq3s_grid.inc"
};
static __constant__ uint32_t kPfGrid2[2048] = {
#include "iq2s_grid.inc"
};
static __constant__ int8_t kPfKv[16] = {
#include "iq4nl_kvalues.inc"
};

constexpr int kPfTT = 5;                   // token tiles of 16 rows per block
constexpr int kPfTm = 16 * kPfTT;          // rows per block of the prefill's own plan
constexpr int kPfWaves = 4;
constexpr int kPfRtw = 4;                  // row tiles per wavefront (64 weight rows)
constexpr int kPfXPitch = 88;              // dwords per staged activation row of one column tile (80 + 8: the
                                           // fastest pitch for this read pattern on gfx950, measured)
constexpr int kPfGPitch = kPfTm + 4;       // floats per row of the gate/up epilogue's exchange (skewed banks)
constexpr int kXcds = 8;                   // accelerator complex dies of MI355X (one L2 each)
constexpr uint32_t kXOut = 0x80000000u;    // activation offset past every buffer's byte range (reads zero)

// ------------------------------------------------------------------------------------------------ grouped GEMM
struct PfArgs {
    Cb3Table t0, t1;                       // CB3 tables -- gate/up: gate, up; down: down (twice)
    Iq3Table i0, i1;                       // IQ3_S tables, the same roles
    Iq4Table k0, k1;                       // IQ4_XS tables, the same roles
    Iq2Table j0, j1;                       // IQ2_S tables, the same roles
    KqTable q0, q1;                        // Q2_K / Q3_K tables, the same roles
    int R, K;                              // output columns (rows of the table), input columns
    const int32_t *blk_expert, *blk_n, *n_blocks, *tok_row;
    const uint16_t *x;                     // gate/up: x [T, K] gathered through tok_row; down: h [Rp, K]
    uint32_t x_bytes;                      // bytes of x (< 2^31)
    int gather;
    uint16_t *out;                         // gate/up: h [Rp, R]; down: y [Rp, R]
    float limit;
    int wg_rows;                           // 64-row groups per workgroup: gate/up 2 (x gate, up), down 4
    int RBG;                               // workgroups per block
    const float *w_row;                    // gate/up with kPfScaleH: the plan's routing weight of every row
    float *out32;                          // down with kPfY32: y [Rp, R] in f32
    int P;                                 // workgroups resident at once over the chip
    float *part;                           // split tasks' piece sums: P x kPfPartBytes
    uint32_t *cnt;                         // split tasks' piece counters: P, zero between launches
};

// A task of the launch's last, partial round is split along K into pieces (at most kPfMaxPieces, whole super tiles
// each); a piece stores its accumulators here (kPfPartBytes per workgroup).
constexpr int kPfMaxPieces = 4;
constexpr int kPfPartBytes = kPfWaves * kPfRtw * kPfTT * 64 * 16;

// Rounding forms of the epilogues (FORM, a compile-time set; the ragged kernels use none):
constexpr int kPfRoundGU = 1;   // gate/up: g and u rounded to bf16 before the SwiGLU (the XLA einsums' bf16 outputs)
constexpr int kPfScaleH = 2;    // gate/up: h = bf16(f32(bf16(swiglu)) * w_row[row]) (the sweeps' weighted activations)
constexpr int kPfY32 = 4;       // down: y stored in f32 into out32, not rounded (the sweeps)

// k-steps M..4 of column tile C.  cbr[r] holds the codebook of row tile r's current group: it switches to LDS slot
// C + 1 at step 4 - C and is carried into the next column tile, which starts in that group, so a super tile reads
// each of its five groups from LDS once.  NTT (the block's token tiles) is a compile-time count, so a step's B
// reads and matrix-core instructions form one straight-line block.
template <int NTT, int C, int M>
__device__ __forceinline__ void pf_steps(const uint4 (&wv)[kPfRtw], const uint4 *cbrow, uint4 (&cbr)[kPfRtw],
                                         const uint32_t *xrow, f32x4 (&acc)[kPfRtw][NTT]) {
    if constexpr (M < 5) {
        // one k-step at a time: left free, the scheduler hoists every step's LDS reads and decodes and spills
        if constexpr (M > 0) __builtin_amdgcn_sched_barrier(0);
        if constexpr (M == 4 - C) {
#pragma unroll
            for (int r = 0; r < kPfRtw; ++r) cbr[r] = cbrow[(C + 1) * 64 + 16 * r];
        }
        // the step's B operands first; then row tile by row tile, so the decode of row tile r + 1 (vector ALU)
        // issues while the matrix-core instructions of row tile r run
        uint4 b[NTT];
#pragma unroll
        for (int tt = 0; tt < NTT; ++tt) b[tt] = *(const uint4 *)(xrow + tt * 16 * kPfXPitch + 16 * M);
        uint32_t s0, s1;
        cb3_sel<M>(wv[0], s0, s1);
        bf16x8 A = cb3_weights8(s0, s1, cbr[0]);
#pragma unroll
        for (int r = 0; r < kPfRtw; ++r) {
            bf16x8 An = A;
            if (r + 1 < kPfRtw) {
                cb3_sel<M>(wv[r + 1], s0, s1);
                An = cb3_weights8(s0, s1, cbr[r + 1]);
            }
#pragma unroll
            for (int tt = 0; tt < NTT; ++tt) acc[r][tt] = mfma16(A, b[tt], acc[r][tt]);
            A = An;
        }
        pf_steps<NTT, C, M + 1>(wv, cbrow, cbr, xrow, acc);
    }
}

// Code words of the wavefront's row tiles, two column tiles ahead (the matrix-core work per column tile is long
// enough that a deeper ring only costs registers).
struct PfRegs {
    uint4 ring[2][kPfRtw];    // slot c & 1 = column tile c
    uint4 cbv[5];             // codebook groups of the next super tile, as in Cb3Regs
    uint4 cbr[kPfRtw];        // codebook of the current group, per row tile (lane (q, i): row 16 r + i)
};

// Column tile C of super tile st (codebook slots as in cb3_ctile), B operands from the staged tile.
template <int NTT, int C>
__device__ __forceinline__ void pf_ctile(const Cb3Wave &w, PfRegs &s, int st, const uint32_t *xrow,
                                         f32x4 (&acc)[kPfRtw][NTT]) {
    const int lane = threadIdx.x & 63;
    const int gn = 5 * (st + 1);
    const uint4 *cbrow = w.cbl + (lane & 15);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (C == 0) {
        w.cbl[0 * 64 + lane] = s.cbv[0];
        w.cbl[1 * 64 + lane] = s.cbv[1];
        s.cbv[0] = cb3_group(w, gn);
        s.cbv[1] = cb3_group(w, gn + 1);
#pragma unroll
        for (int r = 0; r < kPfRtw; ++r) s.cbr[r] = cbrow[16 * r];
    } else {
        w.cbl[(C + 1) * 64 + lane] = s.cbv[C + 1];
        s.cbv[C + 1] = cb3_group(w, gn + C + 1);
    }
    const int ct = 4 * st + C;
    uint4 wv[kPfRtw];
#pragma unroll
    for (int r = 0; r < kPfRtw; ++r) {
        wv[r] = s.ring[C & 1][r];
        s.ring[C & 1][r] = cb3_tile(w, ct + 2, r);
    }
    pf_steps<NTT, C, 0>(wv, cbrow, s.cbr, xrow, acc);
}

struct PfShared {
    union {
        uint4 cbl[kPfWaves * 5 * 64];            // CB3: per-wavefront codebook slots (20 KB)
        struct {
            float4 grid[512];                    // IQ3_S: the grid's levels as f32 (8 KB)
            uint4 smask[256];                    // IQ3_S: 8 sign bits -> sign bits of 4 bf16 pairs (4 KB)
        } iq;
        float2 iq4pair[256];                     // IQ4_XS: byte -> (level of its low nibble, of its high nibble)
        struct {
            uint4 level[1024];                   // IQ2_S: grid entry -> its 8 levels as bf16 (16 KB)
            uint4 smask[256];                    // IQ2_S: 8 sign bits -> sign bits of 4 bf16 pairs (4 KB)
        } iq2;
    };
    uint32_t xs[2][kPfTm * kPfXPitch];           // column tiles ct (even/odd) of the block's rows, double-buffered;
                                                 // gate/up epilogue: the gate accumulators of one (gate, up) pair
    uint32_t xrowoff[kPfTm];                     // byte offset of every row's activations, or kXOut
    int last;                                    // split task: this workgroup's piece arrived last
};

// ------------------------------------------------------------------------------------------------ weight providers
// A provider streams the weights of one wavefront's 64 rows (4 row tiles) of expert e, one column tile at a time, and
// runs the tile's k-steps on the matrix cores against the staged activations.  Its state is two values the workgroup
// body keeps as locals: Wave (addressing, fixed per wavefront) and Regs (the loads in flight).
//   init(w, s, a, sh, mat, e, rg, wave, lane, st0, st1)   set up w for super tiles [st0, st1) (column tiles
//                                               [4 st0, 4 st1)), issue the first column tiles' loads into s
//   n_tiles(a, mat)                             column tiles of a row
//   tile<NTT, C>(w, s, st, xt, acc)             column tile 4 st + C; xt = the staged tile at row jt, lane group q
//   kCols, kQOff                                columns per tile; dwords between lane groups' activations in a step
//   kSplit                                      whether the launch's last round of tasks is split into K pieces

// CB3: 160-column tiles of the code-tile layout; codebook slots per 640-column super tile (cb3_tiles.h).
struct PfCb3 {
    static constexpr bool kLdsOnlyBarrier = false;
    static constexpr int kCols = kCb3TileCols;
    static constexpr bool kSplit = false;   // whole tasks only: K pieces measured slower (561 against 536 us)
    static constexpr int kQOff = 4;
    using Wave = Cb3Wave;
    using Regs = PfRegs;
    static __device__ __forceinline__ int n_tiles(const PfArgs &a, int mat) { return (mat ? a.t1 : a.t0).CT; }
    static __device__ __forceinline__ void init(Wave &w, Regs &s, const PfArgs &a, PfShared &sh, int mat, int e,
                                                int rg, int wave, int lane, int st0, int st1) {
        const Cb3Table &tb = mat ? a.t1 : a.t0;
        const uint32_t *qt = tb.qs + (size_t)e * tb.CT * tb.RT * 256;
        const uint32_t *cbe = tb.cb + (size_t)e * tb.G * tb.R * 4;
        w.qb = __builtin_amdgcn_make_buffer_rsrc((void *)qt, (short)0, 0x7fffffff, kBufferWord3);
        w.qnull = __builtin_amdgcn_make_buffer_rsrc((void *)qt, (short)0, 0, kBufferWord3);
        w.cbb = __builtin_amdgcn_make_buffer_rsrc((void *)cbe, (short)0, 0x7fffffff, kBufferWord3);
        w.cbnull = __builtin_amdgcn_make_buffer_rsrc((void *)cbe, (short)0, 0, kBufferWord3);
        w.ct_bytes = (uint32_t)tb.RT * 1024u;
        w.rt_bytes = (uint32_t)(rg * kPfRtw) * 1024u;
        w.g_bytes = (uint32_t)tb.R * 16u;
        w.row_bytes = (uint32_t)(rg * 64) * 16u;
        w.cta = 4 * st0;
        w.ctb = min(tb.CT, 4 * st1);
        w.g_first = 5 * st0;
        w.g_last = min(tb.G, 5 * st1) - 1;
        w.lane16 = (uint32_t)lane * 16u;
        w.cblane16 = (uint32_t)lane * 16u;
        w.xh = w.xl = nullptr;
        w.cbl = sh.cbl + wave * 5 * 64;
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int r = 0; r < kPfRtw; ++r) s.ring[c][r] = cb3_tile(w, 4 * st0 + c, r);
#pragma unroll
        for (int c = 0; c < 5; ++c) s.cbv[c] = cb3_group(w, 5 * st0 + c);
    }
    template <int NTT, int C>
    static __device__ __forceinline__ void tile(const Wave &w, Regs &s, int st, const uint32_t *xt,
                                                f32x4 (&acc)[kPfRtw][NTT]) {
        pf_ctile<NTT, C>(w, s, st, xt, acc);
    }
};

// IQ3_S: the reference's planes (planes.py:136-170, row on the minor axis) decoded straight into the matrix cores'
// A operand.  A column tile is 128 columns = 8 words = half a 256-weight block.  In k-steps 2m and 2m + 1 (m = 0, 1)
// lane (row i, group q) holds weights 0..7 and 8..15 of word 4m + q of the tile: the k order inside a step is free
// as long as the activations are read in the same order.  A weight is bf16(level * scale), scale = f16(d) * (1 + 2 sc)
// in f32 (the product is exact), rounded once to nearest even as the reference's tiles are (pallas_moe.py:341-350,
// with _decode_iq3_s :127-144); the sign is set on the rounded value (the rounding is symmetric).
constexpr int kIq3TileCols = 128;

__device__ __forceinline__ uint32_t pf_bf16_pair(float a, float b) {   // round to nearest even
    const __bf16 v[2] = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
}

// One plane word (4 bytes) per lane at base + off if `use`, else zero: a buffer load through a descriptor whose
// range is empty when unused (no memory touched), so no branch surrounds the load and the compiler's wait counts
// stay exact (a load under a branch made it wait for every load in flight where the branch rejoins).  base must be
// wave-uniform: the lane's word and row go into off.
__device__ __forceinline__ uint32_t pf_word(const char *base, uint32_t off, bool use) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, use ? 0x7fffffff : 0, kBufferWord3);
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}

struct PfIq3Wave {
    const char *qs, *sg, *qh, *sc, *dd;     // expert e's planes
    uint32_t rpitch;                        // bytes per plane row (4 R)
    uint32_t lrow;                          // the lane's byte offset in a plane row (row jt of the wavefront)
    int q;                                  // the lane's group
    int CT;                                 // column tiles of a row
    const float4 *grid;                     // LDS: the grid's levels as f32
    const uint4 *smask;                     // LDS: sign masks
};
struct PfIq3Regs {
    // plane words of column tile ct in slot ct & 1, per row tile: qs of words q and 4 + q, their sg words, qh, sc, d
    uint32_t v[2][kPfRtw][7];
};

struct PfIq3 {
    static constexpr bool kLdsOnlyBarrier = true;
    static constexpr bool kSplit = true;    // the last round's tasks split into K pieces
    static constexpr int kCols = kIq3TileCols;
    static constexpr int kQOff = 8;
    using Wave = PfIq3Wave;
    using Regs = PfIq3Regs;
    static __device__ __forceinline__ int n_tiles(const PfArgs &a, int mat) {
        return (mat ? a.i1 : a.i0).K / kIq3TileCols;
    }
    static __device__ __forceinline__ void load(const Wave &w, int ct, uint32_t (&u)[7], int r, bool use) {
        const uint32_t o = w.lrow + 64u * (uint32_t)r, P = w.rpitch;
        const uint32_t oq = (uint32_t)w.q * P + o, oq2 = (uint32_t)(w.q >> 1) * P + o;
        u[0] = pf_word(w.qs + (size_t)(8 * ct) * P, oq, use);
        u[1] = pf_word(w.qs + (size_t)(8 * ct + 4) * P, oq, use);
        u[2] = pf_word(w.sg + (size_t)(4 * ct) * P, oq2, use);
        u[3] = pf_word(w.sg + (size_t)(4 * ct + 2) * P, oq2, use);
        u[4] = pf_word(w.qh + (size_t)ct * P, o, use);
        u[5] = pf_word(w.sc + (size_t)(ct >> 1) * P, o, use);
        u[6] = pf_word(w.dd + (size_t)(ct >> 2) * P, o, use);
    }
    static __device__ __forceinline__ void init(Wave &w, Regs &s, const PfArgs &a, PfShared &sh, int mat, int e,
                                                int rg, int wave, int lane, int st0, int st1) {
        const Iq3Table &tb = mat ? a.i1 : a.i0;
        const size_t R = (size_t)tb.R;
        w.qs = (const char *)(tb.qs + (size_t)e * tb.W * R);
        w.sg = (const char *)(tb.sg + (size_t)e * (tb.W / 2) * R);
        w.qh = (const char *)(tb.qh + (size_t)e * (tb.W / 8) * R);
        w.sc = (const char *)(tb.sc + (size_t)e * (tb.W / 16) * R);
        w.dd = (const char *)(tb.d + (size_t)e * ((tb.nblk + 1) / 2) * R);
        w.rpitch = 4u * (uint32_t)tb.R;
        w.q = lane >> 4;
        w.lrow = 4u * (uint32_t)(rg * 64 + (lane & 15));
        w.CT = min(tb.K / kIq3TileCols, 4 * st1);          // prefetch no column tile past the range
        w.grid = sh.iq.grid;
        w.smask = sh.iq.smask;
        (void)wave;
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int r = 0; r < kPfRtw; ++r) load(w, 4 * st0 + c, s.v[c][r], r, true);
    }
    // the 8 weights of step j of column tile ct for the row tile whose plane words are u
    static __device__ __forceinline__ bf16x8 weights8(const Wave &w, const uint32_t (&u)[7], int ct, int j) {
        const int m = j >> 1, half = j & 1, q = w.q;
        const uint32_t word = m ? u[1] : u[0];
        const uint32_t s8 = ((m ? u[3] : u[2]) >> (16 * (q & 1) + 8 * half)) & 255u;
        const uint32_t qh4 = (u[4] >> (4 * (4 * m + q))) & 15u;
        const uint32_t nib = (u[5] >> (4 * (4 * (ct & 1) + 2 * m + (q >> 1)))) & 15u;
        const float scale = f16_bits_to_f32(u[6] >> (16 * ((ct >> 1) & 1))) * (float)(1u + 2u * nib);
        const uint32_t i0 = ((word >> (16 * half)) & 255u) | (((qh4 >> (2 * half)) & 1u) << 8);
        const uint32_t i1 = ((word >> (16 * half + 8)) & 255u) | (((qh4 >> (2 * half + 1)) & 1u) << 8);
        const float4 g0 = w.grid[i0], g1 = w.grid[i1];
        const uint4 sm = w.smask[s8];
        uint4 A;
        A.x = pf_bf16_pair(g0.x * scale, g0.y * scale) | sm.x;
        A.y = pf_bf16_pair(g0.z * scale, g0.w * scale) | sm.y;
        A.z = pf_bf16_pair(g1.x * scale, g1.y * scale) | sm.z;
        A.w = pf_bf16_pair(g1.z * scale, g1.w * scale) | sm.w;
        return __builtin_bit_cast(bf16x8, A);
    }
    template <int NTT, int C>
    static __device__ __forceinline__ void tile(const Wave &w, Regs &s, int st, const uint32_t *xt,
                                                f32x4 (&acc)[kPfRtw][NTT]) {
        const int ct = 4 * st + C;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (j > 0) __builtin_amdgcn_sched_barrier(0);
            uint4 b[NTT];
#pragma unroll
            for (int tt = 0; tt < NTT; ++tt)
                b[tt] = *(const uint4 *)(xt + tt * 16 * kPfXPitch + 32 * (j >> 1) + 4 * (j & 1));
            bf16x8 A = weights8(w, s.v[C & 1][0], ct, j);
#pragma unroll
            for (int r = 0; r < kPfRtw; ++r) {
                bf16x8 An = A;
                if (r + 1 < kPfRtw) An = weights8(w, s.v[C & 1][r + 1], ct, j);
#pragma unroll
                for (int tt = 0; tt < NTT; ++tt) acc[r][tt] = mfma16(A, b[tt], acc[r][tt]);
                A = An;
            }
        }
        // the slot's next column tile (ct + 2); past the row's end the loads read zeros (the slot is not read again)
#pragma unroll
        for (int r = 0; r < kPfRtw; ++r) load(w, ct + 2, s.v[C & 1][r], r, ct + 2 < w.CT);
    }
};

// IQ2_S: the reference's planes (planes.py:17-21, 136-170) decoded straight into the A operand.  A column tile is
// 128 columns = 4 words (half a 256-weight block).  In k-step j lane (row i, group q) holds group j of word q of the
// tile, i.e. columns 32q + 8j .. 32q + 8j + 7: the k order inside a step is free as long as the activations are read
// in the same order, and this one lets a lane read only its own word of each plane.  A weight is bf16(level * scale),
// scale = f16(d) * (0.5 + sc) * 0.25 in f32 (the product is exact), rounded once to nearest even as the reference's
// tiles are (pallas_moe.py:105-124, 341-350); the sign is set on the rounded value (the rounding is symmetric).
struct PfIq2Wave {
    const char *qs, *sg, *qh, *sc, *dd;     // expert e's planes
    uint32_t rpitch;                        // bytes per plane row (4 R)
    uint32_t lrow;                          // the lane's byte offset in a plane row (row jt of the wavefront)
    int q, CT;
    const uint4 *level;                     // LDS: grid entry -> 8 bf16 levels
    const uint4 *smask;                     // LDS: sign masks
};
struct PfIq2Regs {
    uint32_t v[2][kPfRtw][5];   // column tile ct in slot ct & 1, per row tile: the lane's qs and sg words, qh, sc, d
};

struct PfIq2 {
    static constexpr bool kLdsOnlyBarrier = true;
    static constexpr bool kSplit = true;    // the last round's tasks split into K pieces
    static constexpr int kCols = 128;
    static constexpr int kQOff = 16;       // dwords: word q of the tile
    using Wave = PfIq2Wave;
    using Regs = PfIq2Regs;
    static __device__ __forceinline__ int n_tiles(const PfArgs &a, int mat) { return (mat ? a.j1 : a.j0).K / 128; }
    static __device__ __forceinline__ void load(const Wave &w, int ct, uint32_t (&u)[5], int r, bool use) {
        const uint32_t o = w.lrow + 64u * (uint32_t)r, P = w.rpitch, oq = (uint32_t)w.q * P + o;
        u[0] = pf_word(w.qs + (size_t)(4 * ct) * P, oq, use);
        u[1] = pf_word(w.sg + (size_t)(4 * ct) * P, oq, use);
        u[2] = pf_word(w.qh + (size_t)ct * P, o, use);                  // byte q: word 4 ct + q
        u[3] = pf_word(w.sc + (size_t)ct * P, o, use);
        u[4] = pf_word(w.dd + (size_t)(ct >> 2) * P, o, use);
    }
    static __device__ __forceinline__ void init(Wave &w, Regs &s, const PfArgs &a, PfShared &sh, int mat, int e,
                                                int rg, int wave, int lane, int st0, int st1) {
        const Iq2Table &tb = mat ? a.j1 : a.j0;
        const size_t R = (size_t)tb.R;
        w.qs = (const char *)(tb.qs + (size_t)e * tb.W * R);
        w.sg = (const char *)(tb.sg + (size_t)e * tb.W * R);
        w.qh = (const char *)(tb.qh + (size_t)e * (tb.W / 4) * R);
        w.sc = (const char *)(tb.sc + (size_t)e * (tb.W / 4) * R);
        w.dd = (const char *)(tb.d + (size_t)e * ((tb.nblk + 1) / 2) * R);
        w.rpitch = 4u * (uint32_t)tb.R;
        w.q = lane >> 4;
        w.lrow = 4u * (uint32_t)(rg * 64 + (lane & 15));
        w.CT = min(tb.K / 128, 4 * st1);                   // prefetch no column tile past the range
        w.level = sh.iq2.level;
        w.smask = sh.iq2.smask;
        (void)wave;
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int r = 0; r < kPfRtw; ++r) load(w, 4 * st0 + c, s.v[c][r], r, true);
    }
    // the 8 weights of step j (group j of the lane's word) for the row tile whose plane words are u
    static __device__ __forceinline__ bf16x8 weights8(const Wave &w, const uint32_t (&u)[5], int ct, int j) {
        const int q = w.q;
        const uint32_t idx = ((u[0] >> (8 * j)) & 255u) | (((u[2] >> (8 * q + 2 * j)) & 3u) << 8);
        const uint32_t s8 = (u[1] >> (8 * j)) & 255u;
        const uint32_t nib = (u[3] >> (8 * q + 4 * (j >> 1))) & 15u;
        const float scale = f16_bits_to_f32(u[4] >> (16 * ((ct >> 1) & 1))) * (0.5f + (float)nib) * 0.25f;
        const uint4 g = w.level[idx];
        const uint4 sm = w.smask[s8];
        uint4 A;
        A.x = pf_bf16_pair(__uint_as_float(g.x << 16) * scale, __uint_as_float(g.x & 0xffff0000u) * scale) | sm.x;
        A.y = pf_bf16_pair(__uint_as_float(g.y << 16) * scale, __uint_as_float(g.y & 0xffff0000u) * scale) | sm.y;
        A.z = pf_bf16_pair(__uint_as_float(g.z << 16) * scale, __uint_as_float(g.z & 0xffff0000u) * scale) | sm.z;
        A.w = pf_bf16_pair(__uint_as_float(g.w << 16) * scale, __uint_as_float(g.w & 0xffff0000u) * scale) | sm.w;
        return __builtin_bit_cast(bf16x8, A);
    }
    template <int NTT, int C>
    static __device__ __forceinline__ void tile(const Wave &w, Regs &s, int st, const uint32_t *xt,
                                                f32x4 (&acc)[kPfRtw][NTT]) {
        const int ct = 4 * st + C;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (j > 0) __builtin_amdgcn_sched_barrier(0);
            uint4 b[NTT];
#pragma unroll
            for (int tt = 0; tt < NTT; ++tt) b[tt] = *(const uint4 *)(xt + tt * 16 * kPfXPitch + 4 * j);
            bf16x8 A = weights8(w, s.v[C & 1][0], ct, j);
#pragma unroll
            for (int r = 0; r < kPfRtw; ++r) {
                bf16x8 An = A;
                if (r + 1 < kPfRtw) An = weights8(w, s.v[C & 1][r + 1], ct, j);
#pragma unroll
                for (int tt = 0; tt < NTT; ++tt) acc[r][tt] = mfma16(A, b[tt], acc[r][tt]);
                A = An;
            }
        }
        // the slot's next column tile (ct + 2); past the row's end the loads read zeros (the slot is not read again)
#pragma unroll
        for (int r = 0; r < kPfRtw; ++r) load(w, ct + 2, s.v[C & 1][r], r, ct + 2 < w.CT);
    }
};

// Q2_K / Q3_K: the reference's planes (planes.py:34-41, 136-170) decoded straight into the A operand.  A column tile
// is 128 columns = half a block (half n = ct % 2); k-step j is the shift-j stripe of the half: lane (row i, group q)
// holds columns 32 j + 8 q .. 32 j + 8 q + 7 = bytes 0..3 of plane words q' = 2q, 2q + 1 at shift 2j (natural
// order), scale byte 8 n + 2 j + (q >= 2).  A weight is the reference's f32 value rounded once to bf16: Q2_K
// fma(v, d * sc, -dmin * m) (d * sc * v is exact: one rounding, as iqquant.py:213), Q3_K (v + 4 hbit - 4) * d * (sc - 32)
// (exact) (pallas_moe.py:165-209, 341-350).
struct PfKqWave {
    const char *qs, *sc, *dd, *hm;          // expert e's planes (hm: Q3_K)
    uint32_t rpitch;                        // bytes per plane row (4 R)
    uint32_t lrow;                          // the lane's byte offset in a plane row (row jt of the wavefront)
    int q, CT;
};
struct PfKqRegs {
    uint32_t v[2][kPfRtw][7];   // column tile ct in slot ct & 1, per row tile: qs words 2q, 2q + 1, sc x 2, d, hm x 2
};

template <bool Q3>
struct PfKq {
    static constexpr bool kLdsOnlyBarrier = true;
    static constexpr bool kSplit = true;    // the last round's tasks split into K pieces
    static constexpr int kCols = 128;
    static constexpr int kQOff = 4;        // dwords: columns 8q .. 8q+7 of a 32-column stripe
    using Wave = PfKqWave;
    using Regs = PfKqRegs;
    static __device__ __forceinline__ int n_tiles(const PfArgs &a, int mat) { return (mat ? a.q1 : a.q0).K / 128; }
    static __device__ __forceinline__ void load(const Wave &w, int ct, uint32_t (&u)[7], int r, bool use) {
        const uint32_t o = w.lrow + 64u * (uint32_t)r, P = w.rpitch;
        const uint32_t oa = (uint32_t)(2 * w.q) * P + o, ob = oa + P;
        const int b = ct >> 1;
        u[0] = pf_word(w.qs + (size_t)(8 * ct) * P, oa, use);
        u[1] = pf_word(w.qs + (size_t)(8 * ct) * P, ob, use);
        u[2] = pf_word(w.sc + (size_t)(2 * ct) * P, o, use);
        u[3] = pf_word(w.sc + (size_t)(2 * ct + 1) * P, o, use);
        u[4] = pf_word(w.dd + (size_t)b * P, o, use);
        if constexpr (Q3) {
            u[5] = pf_word(w.hm + (size_t)(8 * b) * P, oa, use);
            u[6] = pf_word(w.hm + (size_t)(8 * b) * P, ob, use);
        }
    }
    static __device__ __forceinline__ void init(Wave &w, Regs &s, const PfArgs &a, PfShared &sh, int mat, int e,
                                                int rg, int wave, int lane, int st0, int st1) {
        const KqTable &tb = mat ? a.q1 : a.q0;
        const size_t R = (size_t)tb.R;
        w.qs = (const char *)(tb.qs + (size_t)e * 16 * tb.nblk * R);
        w.sc = (const char *)(tb.sc + (size_t)e * 4 * tb.nblk * R);
        w.dd = (const char *)(tb.d + (size_t)e * tb.nblk * R);
        w.hm = Q3 ? (const char *)(tb.hm + (size_t)e * 8 * tb.nblk * R) : nullptr;
        w.rpitch = 4u * (uint32_t)tb.R;
        w.q = lane >> 4;
        w.lrow = 4u * (uint32_t)(rg * 64 + (lane & 15));
        w.CT = min(tb.K / 128, 4 * st1);                   // prefetch no column tile past the range
        (void)sh;
        (void)wave;
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int r = 0; r < kPfRtw; ++r) load(w, 4 * st0 + c, s.v[c][r], r, true);
    }
    // 4 weights from the 4 byte-sized values of t (each 0..3, Q3_K 0..7): f32 -> bf16 pairs
    static __device__ __forceinline__ uint2 four(uint32_t t, float m, float a) {
        const float v0 = (float)(t & 255u), v1 = (float)((t >> 8) & 255u);       // v_cvt_f32_ubyte0..3
        const float v2 = (float)((t >> 16) & 255u), v3 = (float)(t >> 24);
        return make_uint2(pf_bf16_pair(fmaf(v0, m, a), fmaf(v1, m, a)), pf_bf16_pair(fmaf(v2, m, a), fmaf(v3, m, a)));
    }
    // the 8 weights of step j (shift stripe j) for the row tile whose plane words are u
    static __device__ __forceinline__ bf16x8 weights8(const Wave &w, const uint32_t (&u)[7], int ct, int j) {
        const int n = ct & 1;
        const uint32_t sb = ((j >> 1 ? u[3] : u[2]) >> (16 * (j & 1) + 8 * (w.q >> 1))) & 255u;
        const float d = f16_bits_to_f32(u[4] & 0xffffu);
        uint32_t t0 = (u[0] >> (2 * j)) & 0x03030303u, t1 = (u[1] >> (2 * j)) & 0x03030303u;
        float m, a;
        if (Q3) {
            t0 |= ((u[5] >> (4 * n + j)) & 0x01010101u) << 2;
            t1 |= ((u[6] >> (4 * n + j)) & 0x01010101u) << 2;
            m = d * ((float)sb - 32.0f);                              // exact
            a = -4.0f * m;
        } else {
            m = d * (float)(sb & 15u);
            a = -(f16_bits_to_f32(u[4] >> 16) * (float)(sb >> 4));
        }
        const uint2 l0 = four(t0, m, a), l1 = four(t1, m, a);
        return __builtin_bit_cast(bf16x8, make_uint4(l0.x, l0.y, l1.x, l1.y));
    }
    template <int NTT, int C>
    static __device__ __forceinline__ void tile(const Wave &w, Regs &s, int st, const uint32_t *xt,
                                                f32x4 (&acc)[kPfRtw][NTT]) {
        const int ct = 4 * st + C;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (j > 0) __builtin_amdgcn_sched_barrier(0);
            uint4 b[NTT];
#pragma unroll
            for (int tt = 0; tt < NTT; ++tt) b[tt] = *(const uint4 *)(xt + tt * 16 * kPfXPitch + 16 * j);
            bf16x8 A = weights8(w, s.v[C & 1][0], ct, j);
#pragma unroll
            for (int r = 0; r < kPfRtw; ++r) {
                bf16x8 An = A;
                if (r + 1 < kPfRtw) An = weights8(w, s.v[C & 1][r + 1], ct, j);
#pragma unroll
                for (int tt = 0; tt < NTT; ++tt) acc[r][tt] = mfma16(A, b[tt], acc[r][tt]);
                A = An;
            }
        }
        // the slot's next column tile (ct + 2); past the row's end the loads read zeros (the slot is not read again)
#pragma unroll
        for (int r = 0; r < kPfRtw; ++r) load(w, ct + 2, s.v[C & 1][r], r, ct + 2 < w.CT);
    }
};

// IQ4_XS: the reference's planes (planes.py:26-28, 136-170) decoded straight into the A operand.  A column tile is
// 128 columns (4 sub-blocks of 32, half a block); the k-step of sub-block i takes, for lane group q, plane word 4i + q:
// byte j of it holds sub-block columns 4q + j (low nibble) and 16 + 4q + j (high nibble).  The lane's A elements are
// columns 4q .. 4q+3 then 16 + 4q .. 16 + 4q + 3, so the activations are read as two 8-byte pieces of the staged
// tile.  A weight is bf16(level * f16(d) * (s - 32)): the f32 product is exact and rounded once to nearest even, as
// the reference's tiles are (pallas_moe.py:147-162, 341-350).
struct PfIq4Wave {
    const char *qs, *sl, *sh, *dd;          // expert e's planes
    uint32_t rpitch;                        // bytes per plane row (4 R)
    uint32_t lrow;                          // the lane's byte offset in a plane row (row jt of the wavefront)
    int q, CT;
    const float2 *pair;                     // LDS: byte -> its two levels as f32
};
struct PfIq4Regs {
    uint32_t v[2][kPfRtw][7];   // column tile ct in slot ct & 1, per row tile: the 4 words, sl, sh, d
};

struct PfIq4 {
    static constexpr bool kLdsOnlyBarrier = true;
    static constexpr bool kSplit = true;    // the last round's tasks split into K pieces
    static constexpr int kCols = 128;
    static constexpr int kQOff = 2;        // dwords: columns 4q .. 4q+3 of a 32-column group
    using Wave = PfIq4Wave;
    using Regs = PfIq4Regs;
    static __device__ __forceinline__ int n_tiles(const PfArgs &a, int mat) { return (mat ? a.k1 : a.k0).K / 128; }
    static __device__ __forceinline__ void load(const Wave &w, int ct, uint32_t (&u)[7], int r, bool use) {
        const uint32_t o = w.lrow + 64u * (uint32_t)r, P = w.rpitch, oq = (uint32_t)w.q * P + o;
#pragma unroll
        for (int j = 0; j < 4; ++j) u[j] = pf_word(w.qs + (size_t)(16 * ct + 4 * j) * P, oq, use);
        u[4] = pf_word(w.sl + (size_t)(ct >> 1) * P, o, use);
        u[5] = pf_word(w.sh + (size_t)(ct >> 1) * P, o, use);
        u[6] = pf_word(w.dd + (size_t)(ct >> 2) * P, o, use);
    }
    static __device__ __forceinline__ void init(Wave &w, Regs &s, const PfArgs &a, PfShared &sh, int mat, int e,
                                                int rg, int wave, int lane, int st0, int st1) {
        const Iq4Table &tb = mat ? a.k1 : a.k0;
        const size_t R = (size_t)tb.R;
        w.qs = (const char *)(tb.qs + (size_t)e * tb.W * R);
        w.sl = (const char *)(tb.sl + (size_t)e * tb.nblk * R);
        w.sh = (const char *)(tb.sh + (size_t)e * tb.nblk * R);
        w.dd = (const char *)(tb.d + (size_t)e * ((tb.nblk + 1) / 2) * R);
        w.rpitch = 4u * (uint32_t)tb.R;
        w.q = lane >> 4;
        w.lrow = 4u * (uint32_t)(rg * 64 + (lane & 15));
        w.CT = min(tb.K / 128, 4 * st1);                   // prefetch no column tile past the range
        w.pair = sh.iq4pair;
        (void)wave;
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int r = 0; r < kPfRtw; ++r) load(w, 4 * st0 + c, s.v[c][r], r, true);
    }
    // the 8 weights of step j (sub-block 4 (ct % 2) + j) for the row tile whose plane words are u
    static __device__ __forceinline__ bf16x8 weights8(const Wave &w, const uint32_t (&u)[7], int ct, int j) {
        const int i = 4 * (ct & 1) + j;
        const int sv = (int)(((u[4] >> (4 * i)) & 15u) | (((u[5] >> (2 * i)) & 3u) << 4)) - 32;
        const float scale = f16_bits_to_f32(u[6] >> (16 * ((ct >> 1) & 1))) * (float)sv;
        const uint32_t x = u[j];
        const float2 p0 = w.pair[x & 255u], p1 = w.pair[(x >> 8) & 255u], p2 = w.pair[(x >> 16) & 255u],
                     p3 = w.pair[x >> 24];
        uint4 A;
        A.x = pf_bf16_pair(p0.x * scale, p1.x * scale);
        A.y = pf_bf16_pair(p2.x * scale, p3.x * scale);
        A.z = pf_bf16_pair(p0.y * scale, p1.y * scale);
        A.w = pf_bf16_pair(p2.y * scale, p3.y * scale);
        return __builtin_bit_cast(bf16x8, A);
    }
    template <int NTT, int C>
    static __device__ __forceinline__ void tile(const Wave &w, Regs &s, int st, const uint32_t *xt,
                                                f32x4 (&acc)[kPfRtw][NTT]) {
        const int ct = 4 * st + C;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (j > 0) __builtin_amdgcn_sched_barrier(0);
            uint4 b[NTT];
#pragma unroll
            for (int tt = 0; tt < NTT; ++tt) {
                const uint2 lo = *(const uint2 *)(xt + tt * 16 * kPfXPitch + 16 * j);
                const uint2 hi = *(const uint2 *)(xt + tt * 16 * kPfXPitch + 16 * j + 8);
                b[tt] = make_uint4(lo.x, lo.y, hi.x, hi.y);
            }
            bf16x8 A = weights8(w, s.v[C & 1][0], ct, j);
#pragma unroll
            for (int r = 0; r < kPfRtw; ++r) {
                bf16x8 An = A;
                if (r + 1 < kPfRtw) An = weights8(w, s.v[C & 1][r + 1], ct, j);
#pragma unroll
                for (int tt = 0; tt < NTT; ++tt) acc[r][tt] = mfma16(A, b[tt], acc[r][tt]);
                A = An;
            }
        }
        // the slot's next column tile (ct + 2); past the row's end the loads read zeros (the slot is not read again)
#pragma unroll
        for (int r = 0; r < kPfRtw; ++r) load(w, ct + 2, s.v[C & 1][r], r, ct + 2 < w.CT);
    }
};

// One workgroup: block g (expert e, rows row0 .. row0 + n - 1, NTT = ceil(n / 16) token tiles), row range rbg.
// piece / np: the workgroup runs super tiles [piece n_st / np, (piece + 1) n_st / np) of the task (np == 1: all of
// them); sti: the split task's index among the launch's split tasks (counter and piece sums).
template <int MODE, int NTT, class WP, int FORM>
__device__ __forceinline__ void prefill_body(const PfArgs &a, PfShared &sh, int g, int rbg, int e, int n, int piece,
                                             int np, int sti) {
    uint32_t *xs = &sh.xs[0][0], *xrowoff = sh.xrowoff;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int row0 = g * kPfTm;
    const int mat = MODE == 0 ? (wave & 1) : 0;
    const int rg = rbg * a.wg_rows + (MODE == 0 ? (wave >> 1) : wave);   // 64-row group of this wavefront

    const int CT = WP::n_tiles(a, mat);
    const int n_st = (CT + 3) >> 2;                     // super tiles of a row (the last one maybe partial)
    const int s0 = WP::kSplit ? piece * n_st / np : 0, s1 = WP::kSplit ? (piece + 1) * n_st / np : n_st;
    const int ct_end = min(CT, 4 * s1);
    typename WP::Wave w;
    typename WP::Regs s;
    WP::init(w, s, a, sh, mat, e, rg, wave, lane, s0, s1);

    // activation tile: the block's 16 NTT rows x kXU uint4 (WP::kCols columns), staged as buffer loads by
    // kXRows x kXU threads, kXRows rows per pass (thread t: row t / kXU + kXRows j, uint4 column t % kXU), so every
    // pass is a constant offset from the first; rows >= n and columns >= K take an offset past the buffer's range,
    // which reads zero
    constexpr int kXU = WP::kCols / 8;                        // 20 (CB3) or 16 (IQ3_S)
    constexpr int kXRows = (64 * kPfWaves) / kXU;             // 12 or 16
    constexpr int kXBuf = kPfTm * kPfXPitch;                  // dwords per tile buffer
    constexpr int kXJ = (16 * NTT + kXRows - 1) / kXRows;
    const __amdgpu_buffer_rsrc_t xbuf =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.x, (short)0, (int)a.x_bytes, kBufferWord3);
    if (tid < kPfTm) {
        uint32_t o = kXOut;
        if (tid < n) o = (uint32_t)(a.gather ? a.tok_row[row0 + tid] : row0 + tid) * (uint32_t)a.K * 2u;
        xrowoff[tid] = o;
    }
    __syncthreads();
    const int xr0 = tid / kXU, xc8 = tid - xr0 * kXU;
    const bool stager = tid < kXRows * kXU;
    uint4 xr[kXJ];
    // use: whether the tile is staged at all (no branch around the loads: past the range they read zeros)
    auto load_x = [&](int ct, bool use) {
        const int lim = (a.K - WP::kCols * ct) >> 3;          // uint4 columns of this tile inside the row
#pragma unroll
        for (int j = 0; j < kXJ; ++j) {
            const int row = xr0 + kXRows * j;
            uint32_t o = kXOut;
            if (use && stager && row < 16 * NTT && xc8 < lim)
                o = xrowoff[row] + 16u * (uint32_t)xc8 + (uint32_t)(2 * WP::kCols * ct);
            xr[j] = bload(xbuf, o, 0);
        }
    };
    auto store_x = [&](int buf) {
#pragma unroll
        for (int j = 0; j < kXJ; ++j) {
            const int row = xr0 + kXRows * j;
            if (stager && row < 16 * NTT) *(uint4 *)(xs + buf * kXBuf + row * kPfXPitch + 4 * xc8) = xr[j];
        }
    };
    load_x(4 * s0, true);
    store_x(0);

    f32x4 acc[kPfRtw][NTT];
#pragma unroll
    for (int r = 0; r < kPfRtw; ++r)
#pragma unroll
        for (int t = 0; t < NTT; ++t) acc[r][t] = (f32x4){0.f, 0.f, 0.f, 0.f};
    const int jt = lane & 15, q = lane >> 4;
    const uint32_t *xrow = xs + jt * kPfXPitch + WP::kQOff * q;

    // one barrier per column tile: tile ct sits in buffer ct & 1 (= C & 1); the next tile's loads are issued first
    // (ahead of this tile's code and codebook loads, so waiting for them never waits for those) and stored into the
    // other buffer after this tile's matrix-core work, which every wavefront finished reading one barrier earlier.
    // The block formats' barrier orders LDS only (lds_barrier): a full __syncthreads also waits for every weight
    // load in flight, the prefetched next tiles included (IQ3_S 831 -> 761 us at 512 tokens with it).  CB3 keeps the
    // full barrier and the branch around its staging loads: without them its GEMMs measured slower.
    auto step = [&](auto Cc, int st) {
        constexpr int C = decltype(Cc)::value;
        const int ct = 4 * st + C;
        if constexpr (WP::kLdsOnlyBarrier) {
            lds_barrier();
            load_x(ct + 1, ct + 1 < ct_end);                // no branch around the loads
        } else {
            __syncthreads();
            if (ct + 1 < ct_end) load_x(ct + 1, true);
        }
        WP::template tile<NTT, C>(w, s, st, xrow + (C & 1) * kXBuf, acc);
        if (ct + 1 < ct_end) store_x((C + 1) & 1);
    };
    const int st_full = min(CT >> 2, s1);
    int st = s0;
    for (; st < st_full; ++st) {
        step(std::integral_constant<int, 0>{}, st);
        step(std::integral_constant<int, 1>{}, st);
        step(std::integral_constant<int, 2>{}, st);
        step(std::integral_constant<int, 3>{}, st);
    }
    const int nct = ct_end - 4 * st;                    // 0..3 column tiles of a last, partial super tile
    if (nct > 0) step(std::integral_constant<int, 0>{}, st);
    if (nct > 1) step(std::integral_constant<int, 1>{}, st);
    if (nct > 2) step(std::integral_constant<int, 2>{}, st);

    if (WP::kSplit && np > 1) {
        // a piece of a split task: its sums go to memory (stored through this XCD's L2), then the piece is counted;
        // the piece that arrives last adds all of them in piece order (the same order whichever arrives last) and
        // runs the epilogue.  Nothing waits for another workgroup.  The other pieces' sums are read with device-coherent
        // (sc1) loads after the count, so no older copy of a line in this XCD's L2 can be returned.
        const __amdgpu_buffer_rsrc_t pr =
            __builtin_amdgcn_make_buffer_rsrc((void *)a.part, (short)0, 0x7fffffff, kBufferWord3);
        const uint32_t lane_off = 16u * (uint32_t)lane;
        auto piece_off = [&](int pc, int r, int t) {
            return (uint32_t)(sti * np + pc) * (uint32_t)kPfPartBytes +
                   (uint32_t)((wave * kPfRtw + r) * kPfTT + t) * 1024u + lane_off;
        };
#pragma unroll
        for (int r = 0; r < kPfRtw; ++r)
#pragma unroll
            for (int t = 0; t < NTT; ++t) wt_store4(pr, piece_off(piece, r, t), acc[r][t]);
        __builtin_amdgcn_s_waitcnt(0);                  // this wavefront's stores have completed
        __syncthreads();                                // ... and every wavefront's
        if (tid == 0) sh.last = counter_add(a.cnt + sti, 1u) == (uint32_t)(np - 1);
        __syncthreads();
        if (!sh.last) return;
        if (tid == 0) counter_reset(a.cnt + sti);       // zero again for the next launch
        // every piece's sums from memory, this one's too (its stores have completed), added in piece order
#pragma unroll
        for (int r = 0; r < kPfRtw; ++r)
#pragma unroll
            for (int t = 0; t < NTT; ++t) acc[r][t] = (f32x4){0.f, 0.f, 0.f, 0.f};
        for (int pc = 0; pc < np; ++pc) {
#pragma unroll
            for (int r = 0; r < kPfRtw; ++r)
#pragma unroll
                for (int t = 0; t < NTT; ++t)
                    acc[r][t] += coherent_load4(pr, piece_off(pc, r, t));
        }
    }

    // epilogue: lane (jt, q) holds rows 16 r + 4 q + i (i = 0..3) of the wavefront's 64 rows for tokens 16 t + jt
    const int rbase = rg * 64;
    if constexpr (MODE == 0) {
        float *gbuf = (float *)xs;                           // [64 rows][kPfGPitch] gate accumulators of one pair
        for (int pair = 0; pair < 2; ++pair) {
            __syncthreads();
            if (wave == 2 * pair) {
#pragma unroll
                for (int r = 0; r < kPfRtw; ++r)
#pragma unroll
                    for (int t = 0; t < NTT; ++t)
#pragma unroll
                        for (int i = 0; i < 4; ++i) gbuf[(16 * r + 4 * q + i) * kPfGPitch + 16 * t + jt] = acc[r][t][i];
            }
            __syncthreads();
            if (wave == 2 * pair + 1) {
                constexpr bool round_gu = FORM & kPfRoundGU, scale_h = FORM & kPfScaleH;
#pragma unroll
                for (int t = 0; t < NTT; ++t) {
                    const int tok = 16 * t + jt;
                    if (tok < n) {
                        float wr = 1.0f;
                        if constexpr (scale_h) wr = a.w_row[row0 + tok];
#pragma unroll
                        for (int r = 0; r < kPfRtw; ++r) {
                            float hv[4];
#pragma unroll
                            for (int i = 0; i < 4; ++i) {
                                float gv = gbuf[(16 * r + 4 * q + i) * kPfGPitch + tok], uv = acc[r][t][i];
                                if constexpr (round_gu) {
                                    gv = round_bf16(gv);
                                    uv = round_bf16(uv);
                                }
                                hv[i] = swiglu_clamped(gv, uv, a.limit);
                                if constexpr (scale_h) hv[i] = round_bf16(hv[i]) * wr;
                            }
                            uint2 v;
                            v.x = f32_to_bf16_rne(hv[0]) | (f32_to_bf16_rne(hv[1]) << 16);
                            v.y = f32_to_bf16_rne(hv[2]) | (f32_to_bf16_rne(hv[3]) << 16);
                            *(uint2 *)(a.out + (size_t)(row0 + tok) * a.R + rbase + 16 * r + 4 * q) = v;
                        }
                    }
                }
            }
        }
    } else if constexpr ((FORM & kPfY32) != 0) {
#pragma unroll
        for (int t = 0; t < NTT; ++t) {
            const int tok = 16 * t + jt;
            if (tok < n) {
#pragma unroll
                for (int r = 0; r < kPfRtw; ++r)
                    *(float4 *)(a.out32 + (size_t)(row0 + tok) * a.R + rbase + 16 * r + 4 * q) =
                        make_float4(acc[r][t][0], acc[r][t][1], acc[r][t][2], acc[r][t][3]);
            }
        }
    } else {
#pragma unroll
        for (int t = 0; t < NTT; ++t) {
            const int tok = 16 * t + jt;
            if (tok < n) {
#pragma unroll
                for (int r = 0; r < kPfRtw; ++r) {
                    uint2 v;
                    v.x = f32_to_bf16_rne(acc[r][t][0]) | (f32_to_bf16_rne(acc[r][t][1]) << 16);
                    v.y = f32_to_bf16_rne(acc[r][t][2]) | (f32_to_bf16_rne(acc[r][t][3]) << 16);
                    *(uint2 *)(a.out + (size_t)(row0 + tok) * a.R + rbase + 16 * r + 4 * q) = v;
                }
            }
        }
    }
}

template <int MODE, class WP, int FORM>   // MODE 0: gate/up -> h, 1: down -> y; FORM: kPf* rounding forms
__global__ void __launch_bounds__(64 * kPfWaves, 2) prefill_kernel(PfArgs a) {
    __shared__ PfShared sh;
    // workgroups are dispatched to the XCDs round-robin: all workgroups of one block go to the same XCD (block
    // g on XCD g % 8), so the block's activation rows are fetched into one L2 and read there by every workgroup
    // A launch runs n_blocks x RBG tasks on P resident workgroups.  The tasks of the last, partial round (its
    // blocks' tasks: the last sb blocks) are split along K into np pieces each, so that they spread over the slots
    // that free up: np = P / (their tasks), at most kPfMaxPieces and at most the row's super tiles.  Their
    // workgroups follow the unsplit tasks' (which keep the XCD mapping above and skip the split blocks).
    const int nb = *a.n_blocks;
    const int wpad = (nb + kXcds - 1) / kXcds * kXcds * a.RBG;
    int sb = 0, np = 1;
    if constexpr (WP::kSplit) {
        const int r = (nb * a.RBG) % a.P;
        if (r > 0) {
            sb = (r + a.RBG - 1) / a.RBG;
            const int n_st = (WP::n_tiles(a, 0) + 3) >> 2;
            np = min(min(a.P / (sb * a.RBG), kPfMaxPieces), n_st);
            if (np < 2) np = 1, sb = 0;
        }
    }
    int g, rbg, piece = 0, sti = 0, pieces = 1;
    if ((int)blockIdx.x < wpad) {
        const int xcd = blockIdx.x % kXcds, li = blockIdx.x / kXcds;
        g = (li / a.RBG) * kXcds + xcd;
        rbg = li % a.RBG;
        if (g >= nb - sb) return;                       // past the last block, or a split block
    } else {
        const int i = blockIdx.x - wpad;
        if (i >= np * sb * a.RBG) return;
        sti = i / np;
        piece = i - sti * np;
        pieces = np;
        g = nb - sb + sti / a.RBG;
        rbg = sti % a.RBG;
    }
    const int e = __builtin_amdgcn_readfirstlane(a.blk_expert[g]);
    const int n = __builtin_amdgcn_readfirstlane(a.blk_n[g]);
    if constexpr (std::is_same<WP, PfIq3>::value) {
        // the grid's levels as f32 and the sign masks (published by the barrier after the row offsets)
        const int tid = threadIdx.x;
        for (int i = tid; i < 512; i += 64 * kPfWaves) {
            const uint32_t v = kPfGrid[i];
            sh.iq.grid[i] = make_float4((float)(v & 255u), (float)((v >> 8) & 255u), (float)((v >> 16) & 255u),
                                        (float)(v >> 24));
        }
        if (tid < 256) {
            uint32_t m[4];
#pragma unroll
            for (int p = 0; p < 4; ++p) m[p] = (((uint32_t)tid >> (2 * p)) & 1u) << 15 | (((uint32_t)tid >> (2 * p + 1)) & 1u) << 31;
            sh.iq.smask[tid] = make_uint4(m[0], m[1], m[2], m[3]);
        }
    }
    if constexpr (std::is_same<WP, PfIq2>::value) {
        // the grid's levels as bf16 and the sign masks (published by the barrier after the row offsets)
        const int tid = threadIdx.x;
        for (int i = tid; i < 1024; i += 64 * kPfWaves) {
            const uint32_t lo = kPfGrid2[2 * i], hi = kPfGrid2[2 * i + 1];
            uint32_t v[4];
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const uint32_t wd = p < 2 ? lo : hi, sft = 16 * (p & 1);
                v[p] = (__float_as_uint((float)((wd >> sft) & 255u)) >> 16) |
                       (__float_as_uint((float)((wd >> (sft + 8)) & 255u)) & 0xffff0000u);
            }
            sh.iq2.level[i] = make_uint4(v[0], v[1], v[2], v[3]);
        }
        if (tid < 256) {
            uint32_t m[4];
#pragma unroll
            for (int p = 0; p < 4; ++p) m[p] = (((uint32_t)tid >> (2 * p)) & 1u) << 15 | (((uint32_t)tid >> (2 * p + 1)) & 1u) << 31;
            sh.iq2.smask[tid] = make_uint4(m[0], m[1], m[2], m[3]);
        }
    }
    if constexpr (std::is_same<WP, PfIq4>::value) {
        // the level pairs (published by the barrier after the row offsets)
        for (int i = threadIdx.x; i < 256; i += 64 * kPfWaves)
            sh.iq4pair[i] = make_float2((float)kPfKv[i & 15], (float)kPfKv[i >> 4]);
    }
    switch ((n + 15) >> 4) {
        case 1: prefill_body<MODE, 1, WP, FORM>(a, sh, g, rbg, e, n, piece, pieces, sti); break;
        case 2: prefill_body<MODE, 2, WP, FORM>(a, sh, g, rbg, e, n, piece, pieces, sti); break;
        case 3: prefill_body<MODE, 3, WP, FORM>(a, sh, g, rbg, e, n, piece, pieces, sti); break;
        case 4: prefill_body<MODE, 4, WP, FORM>(a, sh, g, rbg, e, n, piece, pieces, sti); break;
        default: prefill_body<MODE, kPfTT, WP, FORM>(a, sh, g, rbg, e, n, piece, pieces, sti); break;
    }
}

// Launches prefill_kernel<MODE, *, FORM> for the table format qtype (MI_QT_*) on grid workgroups.
template <int MODE, int FORM>
int launch_prefill(int qtype, dim3 grid, hipStream_t s, const PfArgs &a) {
    const dim3 block(64 * kPfWaves);
    switch (qtype) {
        case MI_QT_IQ3_S: hipLaunchKernelGGL((prefill_kernel<MODE, PfIq3, FORM>), grid, block, 0, s, a); break;
        case MI_QT_IQ4_XS: hipLaunchKernelGGL((prefill_kernel<MODE, PfIq4, FORM>), grid, block, 0, s, a); break;
        case MI_QT_IQ2_S: hipLaunchKernelGGL((prefill_kernel<MODE, PfIq2, FORM>), grid, block, 0, s, a); break;
        case MI_QT_Q2_K: hipLaunchKernelGGL((prefill_kernel<MODE, PfKq<false>, FORM>), grid, block, 0, s, a); break;
        case MI_QT_Q3_K: hipLaunchKernelGGL((prefill_kernel<MODE, PfKq<true>, FORM>), grid, block, 0, s, a); break;
        case MI_QT_CB3: hipLaunchKernelGGL((prefill_kernel<MODE, PfCb3, FORM>), grid, block, 0, s, a); break;
        default: return MI_ERR_QTYPE;
    }
    return hipGetLastError() == hipSuccess ? MI_OK : MI_ERR_LAUNCH;
}

// the instantiations, one translation unit each (k_prefill.hip)
int launch_prefill_0_0(int qtype, dim3 grid, hipStream_t s, const PfArgs &a);   // ragged gate/up
int launch_prefill_0_1(int qtype, dim3 grid, hipStream_t s, const PfArgs &a);   // kPfRoundGU
int launch_prefill_0_2(int qtype, dim3 grid, hipStream_t s, const PfArgs &a);   // kPfScaleH
int launch_prefill_0_3(int qtype, dim3 grid, hipStream_t s, const PfArgs &a);   // kPfRoundGU | kPfScaleH
int launch_prefill_1_0(int qtype, dim3 grid, hipStream_t s, const PfArgs &a);   // down, bf16 y
int launch_prefill_1_4(int qtype, dim3 grid, hipStream_t s, const PfArgs &a);   // down, f32 y

}  // namespace mi
