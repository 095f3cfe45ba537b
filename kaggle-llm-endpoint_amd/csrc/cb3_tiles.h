// CB3 (3-bit codebook) experts on the gfx950 matrix cores.
//
// Device layout (written by formats.py; the same bytes per row as the canonical 10-codes-per-u32 packing, plus the
// zero padding of the last column tile):
//   code tile (ct, rt): rows 16 rt .. 16 rt + 15 x columns 160 ct .. 160 ct + 159, 1 KB = 64 lanes x 4 words, tiles
//   ordered [expert][ct][rt].  Lane l = 16 q + i holds row 16 rt + i at the columns 160 ct + 32 m + 8 q + j
//   (m = 0..4, j = 0..7), code n = 8 m + j -- exactly the A-operand slice lane l feeds to v_mfma_f32_16x16x32_bf16
//   at k-step m.  Word pair p = 0, 1 (words 2p, 2p+1) holds the codes n = 20 p + c, c = 0..19:
//       word 2p   byte b = code[c=b] | code[c=4+b] << 3 | (code[c=16+b] & 3) << 6
//       word 2p+1 byte b = code[c=8+b] | code[c=12+b] << 3 | (code[c=16+b] >> 2) << 6      (b = 0..3)
//   so one AND (and a shift) yields four byte-sized codebook selectors.  Columns past K hold code 0.
//   codebook: [expert][group g of 128 columns][row] x 4 dwords: lo bytes of centroids 0-3, 4-7, hi bytes 0-3, 4-7.
//
// Decode: v_perm_b32 looks 4 codes up at once in the 8-byte {lo47:lo03} and {hi47:hi03} tables and two more perms
// interleave the bytes into bf16 pairs, so 8 weights (one k-step of one lane) cost 8 perms and ~3 ALU ops; the
// contraction with the activations runs on the matrix cores (16 tokens per instruction), which keeps the vector ALU
// budget per HBM byte independent of the number of tokens sharing the expert.
//
// Column tiles (160) and codebook groups (128) realign every 640 columns (4 tiles = 5 groups): inside such a super
// tile, column tile c uses group c for k-steps m < 4 - c and group c + 1 after, all at compile-time positions, so the
// code ring (one super tile of code words), the five codebook slots and every LDS offset are static.
#pragma once
#include "common.h"

namespace mi {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct Cb3Table {
    const uint32_t *qs;
    const uint32_t *cb;
    int R, K, CT, G, RT;
    static constexpr int kUnitCols = 160;   // column splits are whole column tiles
};

constexpr int kCb3TileCols = 160;
constexpr int kCb3MaxRtw = 4;                 // row tiles per wavefront: RTW = 1, 2 or 4 (16, 32 or 64 rows)
constexpr int kCb3RowAlign = 16 * kCb3MaxRtw; // CB3 tables have R % 64 == 0

// Selectors (4 codes each) of k-step M from the lane's 4 code words.
template <int M>
__device__ __forceinline__ void cb3_sel(const uint4 w, uint32_t &s0, uint32_t &s1) {
    constexpr uint32_t k7 = 0x07070707u;
    if constexpr (M == 0) {
        s0 = w.x & k7;
        s1 = (w.x >> 3) & k7;
    } else if constexpr (M == 1) {
        s0 = w.y & k7;
        s1 = (w.y >> 3) & k7;
    } else if constexpr (M == 2) {
        s0 = ((w.x >> 6) & 0x03030303u) | ((w.y >> 4) & 0x04040404u);
        s1 = w.z & k7;
    } else if constexpr (M == 3) {
        s0 = (w.z >> 3) & k7;
        s1 = w.w & k7;
    } else {
        s0 = (w.w >> 3) & k7;
        s1 = ((w.z >> 6) & 0x03030303u) | ((w.w >> 4) & 0x04040404u);
    }
}

// 8 bf16 weights (k = 0..7 of the step) from two selectors and the row's codebook group.
__device__ __forceinline__ bf16x8 cb3_weights8(uint32_t s0, uint32_t s1, const uint4 cb) {
    const uint32_t lo0 = perm(cb.y, cb.x, s0), hi0 = perm(cb.w, cb.z, s0);
    const uint32_t lo1 = perm(cb.y, cb.x, s1), hi1 = perm(cb.w, cb.z, s1);
    uint4 v;
    v.x = perm(hi0, lo0, 0x05010400u);
    v.y = perm(hi0, lo0, 0x07030602u);
    v.z = perm(hi1, lo1, 0x05010400u);
    v.w = perm(hi1, lo1, 0x07030602u);
    return __builtin_bit_cast(bf16x8, v);
}

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Stream loads are buffer loads: a wave-uniform descriptor (SGPRs) + the lane's byte offset + a scalar tile offset.
// A load the split does not need uses a descriptor with an empty range instead: it returns zeros without touching
// memory, so the instruction stream -- and the compiler's wait counts -- never depend on the split's bounds.
// POL: the load's cache policy bits (kLoadNonTemporal: nt, the line is not kept for reuse).
constexpr int kLoadNonTemporal = 2;
template <int POL = 0>
__device__ __forceinline__ uint4 bload(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, POL));
}
// The code tiles and codebooks are streamed (a decode launch reads each once, a prefill block's workgroups each read
// their own rows): non-temporal loads, so the weight stream does not push out of the caches what is read again
// (staged activations, partials, the routing).  Measured on MI355X (A/B, one box): batch 8 162 -> 146 us, batch 16
// 233 -> 214 us, the batch-1 gate/up launch 32.1 -> 29.1 us, the CB3 prefill 525 -> 515 us.  The prefill's
// activation tiles, read by every workgroup of a block, keep cached loads.
#ifndef MI_CB3_STREAM_POLICY
#define MI_CB3_STREAM_POLICY kLoadNonTemporal
#endif
constexpr int kBufferWord3 = 0x00020000;   // gfx9 buffer descriptor word 3 (32-bit data format)

// Staged activation rows: whole 64-dword chunks (the direct-to-LDS staging loads write 64 lanes x 4 bytes), plus a
// 4-dword skew so the 16 rows of a B-operand read spread over the LDS banks.
__host__ __device__ constexpr int cb3_row_pitch(int xs) { return ((xs + 63) & ~63) + 4; }
// Byte offset past every staged source's range: a buffer load there returns zeros (columns outside the split).
constexpr uint32_t kStageOut = 0x80000000u;

// 16-byte store with the sc1 cache policy: written through this XCD's L2 to memory, so once the store has completed
// (s_waitcnt vmcnt(0)) a coherent load (coherent_load4) on any XCD reads the new value.
__device__ __forceinline__ void wt_store4(__amdgpu_buffer_rsrc_t r, uint32_t voff, f32x4 v) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, (int)voff, 0, kCachePolicySc1);
}

// Per-wavefront stream state.
struct Cb3Wave {
    __amdgpu_buffer_rsrc_t qb, qnull;      // expert's code tiles (full range / empty range)
    __amdgpu_buffer_rsrc_t cbb, cbnull;    // expert's codebook
    uint32_t ct_bytes;     // bytes per column tile row of tiles: RT * 1024
    uint32_t rt_bytes;     // byte offset of the wavefront's first row tile inside a column tile: rt0 * 1024
    uint32_t g_bytes;      // bytes per codebook group: R * 16
    uint32_t row_bytes;    // byte offset of the wavefront's first row inside a group: 16 * rt0 * 16
    int cta, ctb;          // column tiles [cta, ctb) of the wavefront's split
    int g_first, g_last;   // codebook groups the split uses
    uint32_t lane16;       // lane * 16 bytes
    uint32_t cblane16;     // (lane % (16 RTW)) * 16 bytes: the lane's row of a codebook group load
    const uint32_t *xh;    // LDS: B-operand row of this lane (hi / bf16 part) at column 640 * (cta / 4)
    const uint32_t *xl;    // LDS: lo part (two-instruction mode)
    uint4 *cbl;            // LDS: this wavefront's codebook slots, 5 groups x 64 lanes (rows 0 .. 16 RTW - 1)
};

// Codebook path: one 1 KB load brings a group's 16-byte codebooks of the wavefront's 16 RTW rows (lane = row; with
// fewer than 64 rows the remaining lanes repeat them, same addresses, no extra traffic) into the
// register slot of its super-tile position; right before the group is first needed it is written to the
// wavefront's own LDS slot (same-wavefront LDS accesses stay in order, so no barrier) and the register slot is
// reloaded with the next super tile's group.  The decoders read a row's 16 bytes from LDS per k-step, so a lane
// never holds the 4 row tiles' codebooks in registers.
template <int RTW>
struct Cb3Regs {
    uint4 ring[4][RTW];       // code words: slot c = column tile c of a super tile
    uint4 cbv[5];             // codebook groups in flight: slot c = group c of the next super tile
    f32x4 acc[RTW];
};

// Code tile (ct, row tile r of the wavefront) if the split streams it, else zeros.
__device__ __forceinline__ uint4 cb3_tile(const Cb3Wave &w, int ct, int r) {
    const bool need = ct >= w.cta && ct < w.ctb;
    return bload<MI_CB3_STREAM_POLICY>(need ? w.qb : w.qnull, w.lane16, (uint32_t)ct * w.ct_bytes + w.rt_bytes + 1024u * r);
}
// Codebook group g of the wavefront's rows if the split uses it, else zeros.
__device__ __forceinline__ uint4 cb3_group(const Cb3Wave &w, int g) {
    const bool need = g >= w.g_first && g <= w.g_last;
    return bload<MI_CB3_STREAM_POLICY>(need ? w.cbb : w.cbnull, w.cblane16, (uint32_t)g * w.g_bytes + w.row_bytes);
}

// k-steps M..4 of one row tile's column tile (recursion keeps every index static).
template <bool TWO, int C, int M>
__device__ __forceinline__ void cb3_steps(const uint4 wv, const uint4 *cbrow, const int r, const uint4 (&xb)[5],
                                          const uint4 (&xl)[5], f32x4 &acc) {
    if constexpr (M < 5) {
        constexpr int slot = (M < 4 - C) ? C : C + 1;
        uint32_t s0, s1;
        cb3_sel<M>(wv, s0, s1);
        const bf16x8 a = cb3_weights8(s0, s1, cbrow[slot * 64 + 16 * r]);
        acc = mfma16(a, xb[M], acc);
        if constexpr (TWO) acc = mfma16(a, xl[M], acc);
        cb3_steps<TWO, C, M + 1>(wv, cbrow, r, xb, xl, acc);
    }
}

// Column tile C of super tile st: publish the codebook groups first needed here (C = 0: groups 0, 1; else group
// C + 1) and reload their register slots with the next super tile's groups; read the B operands; then per row
// tile decode + MFMA the ring slot's 5 k-steps and refill the slot with column tile C of the next super tile.
template <bool TWO, int RTW, int C>
__device__ __forceinline__ void cb3_ctile(const Cb3Wave &w, Cb3Regs<RTW> &s, int st) {
    const int lane = threadIdx.x & 63;
    const int gn = 5 * (st + 1);
    // keep this tile's LDS publishes and loads here: hoisting a publish would wait for a load issued a super tile
    // later than the one it needs
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (C == 0) {
        w.cbl[0 * 64 + lane] = s.cbv[0];
        w.cbl[1 * 64 + lane] = s.cbv[1];
        s.cbv[0] = cb3_group(w, gn);
        s.cbv[1] = cb3_group(w, gn + 1);
    } else {
        w.cbl[(C + 1) * 64 + lane] = s.cbv[C + 1];
        s.cbv[C + 1] = cb3_group(w, gn + C + 1);
    }
    const int ct = 4 * st + C;
    const int xo = 80 * (ct - (w.cta & ~3));                // dwords
    uint4 xb[5], xl[5];
#pragma unroll
    for (int m = 0; m < 5; ++m) {
        xb[m] = *(const uint4 *)(w.xh + xo + 16 * m);
        if (TWO) xl[m] = *(const uint4 *)(w.xl + xo + 16 * m);
        else xl[m] = xb[m];
    }
    const uint4 *cbrow = w.cbl + (lane & 15);
#pragma unroll
    for (int r = 0; r < RTW; ++r) {
        // decode the slot, then refill it: the load can reuse the slot's registers (refilling first would keep two
        // copies of the ring live and cost a register copy per word every super tile)
        cb3_steps<TWO, C, 0>(s.ring[C][r], cbrow, r, xb, xl, s.acc[r]);
        s.ring[C][r] = cb3_tile(w, ct + 4, r);
    }
}

// Streams column tiles [cta, ctb) of the wavefront's 16 RTW rows, as whole super tiles from the one holding cta: the
// column tiles before cta decode zeros against zero activations (their loads touch no memory; they cost vector ALU
// work only), which keeps the code ring and codebook slots at static positions.  The split's last super tile may end
// early.  `stage` (ending in a workgroup barrier) runs after the first 4 RTW + 5 loads are issued.
template <bool TWO, int RTW, class Stage>
__device__ __forceinline__ void cb3_accum_mfma(const Cb3Wave &w, f32x4 (&acc)[RTW], Stage &&stage) {
    Cb3Regs<RTW> s;
    const int sta = w.cta >> 2;
    // codebook groups first, then the code tiles in the order they are decoded: loads complete in issue order, so
    // the first tile's decode waits for groups 0-1 and that tile only, not for the whole ring
#pragma unroll
    for (int c = 0; c < 5; ++c) s.cbv[c] = cb3_group(w, 5 * sta + c);
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int r = 0; r < RTW; ++r) s.ring[c][r] = cb3_tile(w, 4 * sta + c, r);
#pragma unroll
    for (int r = 0; r < RTW; ++r) s.acc[r] = (f32x4){0.f, 0.f, 0.f, 0.f};
    stage();

    const int st_full = w.ctb >> 2;      // super tiles that end inside the split
    int st = sta;
    for (; st < st_full; ++st) {
        cb3_ctile<TWO, RTW, 0>(w, s, st);
        cb3_ctile<TWO, RTW, 1>(w, s, st);
        cb3_ctile<TWO, RTW, 2>(w, s, st);
        cb3_ctile<TWO, RTW, 3>(w, s, st);
    }
    const int nct = w.ctb - 4 * st;      // 0..3 column tiles of a last, partial super tile
    if (nct > 0) {
        cb3_ctile<TWO, RTW, 0>(w, s, st);
        if (nct > 1) cb3_ctile<TWO, RTW, 1>(w, s, st);
        if (nct > 2) cb3_ctile<TWO, RTW, 2>(w, s, st);
    }
#pragma unroll
    for (int r = 0; r < RTW; ++r) acc[r] = s.acc[r];
}

// ------------------------------------------------------------------------------------------------ staging
// Stages activation rows r < t_rows of columns [c0, c1) (dword d of a row = columns c0 + 2d, c0 + 2d + 1) of one or
// two bf16 planes into LDS (row pitch xsp dwords) with direct-to-LDS loads -- 64 lanes x 16 or 4 bytes per
// instruction, no registers -- spread over the workgroup's wavefronts.  Row r reads plane row row_of(r) (negative: zeros); columns
// outside [cv, cend) read zeros.  The loads complete in issue order with the wavefront's other loads, so a wait for
// "all but the N loads issued since" (vm_wait<N>) followed by a workgroup barrier publishes the rows.
template <bool HILO, class RowOf>
__device__ __forceinline__ void dma_stage(uint32_t *xh, uint32_t *xl, int xsp, int t_rows, int c0, int cv, int c1,
                                          int cend, const uint16_t *ph, const uint16_t *pl, int stride,
                                          RowOf &&row_of, int wave, int lane) {
    const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc((void *)ph, (short)0, 0x7fffffff, kBufferWord3);
    const __amdgpu_buffer_rsrc_t rl =
        __builtin_amdgcn_make_buffer_rsrc((void *)(HILO ? pl : ph), (short)0, 0x7fffffff, kBufferWord3);
    // whole 256-dword chunks of a row with 16 bytes per lane when every bound is a multiple of 8 columns (a lane is
    // then wholly inside or wholly outside [cv, cend)), the rest with 4: an LDS-bound load costs about as much per
    // instruction whatever its width
    const int xs = (c1 - c0) >> 1;
    const int n16 = ((c0 | cv | cend | stride) & 7) == 0 ? xs >> 8 : 0, nt = (xs - 256 * n16 + 63) >> 6;
    const int per16 = (HILO ? 2 : 1) * n16, pert = (HILO ? 2 : 1) * nt;
    for (int i = wave; i < t_rows * per16; i += 4) {
        const int t = i / per16, r = i - t * per16, plane = r / n16, ch = r - plane * n16;
        const int row = row_of(t);
        const int c = c0 + 512 * ch + 8 * lane;
        const uint32_t voff =
            (row >= 0 && c >= cv && c < cend) ? (uint32_t)((size_t)row * stride + c) * 2u : kStageOut;
        uint32_t *dst = (plane ? xl : xh) + t * xsp + 256 * ch;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(plane ? rl : rh, (__attribute__((address_space(3))) void *)dst, 16,
                                                 voff, 0, 0, 0);
    }
    for (int i = wave; i < t_rows * pert; i += 4) {
        const int t = i / pert, r = i - t * pert, plane = r / nt, d0 = 256 * n16 + 64 * (r - plane * nt);
        const int row = row_of(t);
        const int c = c0 + 2 * (d0 + lane);
        const uint32_t voff =
            (row >= 0 && c >= cv && c < cend) ? (uint32_t)((size_t)row * stride + c) * 2u : kStageOut;
        uint32_t *dst = (plane ? xl : xh) + t * xsp + d0;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(plane ? rl : rh, (__attribute__((address_space(3))) void *)dst, 4,
                                                 voff, 0, 0, 0);
    }
}

// ------------------------------------------------------------------------------------------------ continuous stream
// A wavefront that works through a sequence of segments (each one (expert, row group, column split) of its own, as
// cb3_accum_mfma handles one) keeps its code ring and codebook slots full across segment boundaries: during a
// segment's last super tile the refills already fetch the first super tile of the next segment, so the next
// segment's data is in flight while this one finishes and no wavefront waits for a fresh ring at a boundary.

// Column tile C of super tile st of segment w: publish / reload the codebook slots and refill the ring from segment
// `src` at its super tile src_st (w's next super tile, or the next segment's first); decode only if `dec` (the
// column tiles of a last, partial super tile that lie past the segment are not decoded).  INNER: src_st is a super
// tile of src that ends inside its split and is not its first (every refill load is in range: no per-load range
// test, whose scalar selects otherwise cost about a quarter of the instructions of a super tile).
template <bool TWO, int RTW, int C, bool INNER = false>
__device__ __forceinline__ void cb3_ctile_src(const Cb3Wave &w, const Cb3Wave &src, int src_st, Cb3Regs<RTW> &s,
                                              int st, bool dec) {
    const int lane = threadIdx.x & 63;
    const int gn = 5 * src_st;
    auto group = [&](int g) {
        return INNER ? bload<MI_CB3_STREAM_POLICY>(src.cbb, src.cblane16, (uint32_t)g * src.g_bytes + src.row_bytes)
                     : cb3_group(src, g);
    };
    auto tile = [&](int ct, int r) {
        return INNER ? bload<MI_CB3_STREAM_POLICY>(src.qb, src.lane16,
                                                    (uint32_t)ct * src.ct_bytes + src.rt_bytes + 1024u * r)
                     : cb3_tile(src, ct, r);
    };
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (C == 0) {
        w.cbl[0 * 64 + lane] = s.cbv[0];
        w.cbl[1 * 64 + lane] = s.cbv[1];
        s.cbv[0] = group(gn);
        s.cbv[1] = group(gn + 1);
    } else {
        w.cbl[(C + 1) * 64 + lane] = s.cbv[C + 1];
        s.cbv[C + 1] = group(gn + C + 1);
    }
    const int ct = 4 * st + C, nct = 4 * src_st + C;
    if (dec) {
        const int xo = 80 * (ct - (w.cta & ~3));                // dwords
        uint4 xb[5], xl[5];
#pragma unroll
        for (int m = 0; m < 5; ++m) {
            xb[m] = *(const uint4 *)(w.xh + xo + 16 * m);
            if (TWO) xl[m] = *(const uint4 *)(w.xl + xo + 16 * m);
            else xl[m] = xb[m];
        }
        const uint4 *cbrow = w.cbl + (lane & 15);
#pragma unroll
        for (int r = 0; r < RTW; ++r) cb3_steps<TWO, C, 0>(s.ring[C][r], cbrow, r, xb, xl, s.acc[r]);
    }
    // the refills outside the branch: a load under a branch makes the compiler wait for every load in flight where
    // the branch rejoins, which drained the ring at every segment's last super tile (its dec is a run-time value)
#pragma unroll
    for (int r = 0; r < RTW; ++r) s.ring[C][r] = tile(nct, r);
}

// Streams segment w and the ones `next` hands out.
//   next(Cb3Wave &nw) -> bool   the wavefront's next segment (false: none); called at the start of a segment's last
//                               super tile, so that segment's loads are issued while the current one finishes
//   store(f32x4 (&acc)[RTW])    end of a segment: its accumulators (reset to zero afterwards)
//   boundary(const Cb3Wave &nw) between two segments, after store (e.g. restaging activations: all wavefronts of the
//                               workgroup reach it together if they handle one segment per task each)
//   issue()                     once, before the first loads (e.g. direct-to-LDS staging loads, which then complete
//                               ahead of the ring)
//   stage()                     once, after the first 4 RTW + 5 loads are issued (ends in a workgroup barrier)
template <bool TWO, int RTW, class Next, class Store, class Boundary, class Issue, class Stage>
__device__ __forceinline__ void cb3_stream(Cb3Wave w, Next &&next, Store &&store, Boundary &&boundary, Issue &&issue,
                                           Stage &&stage) {
    Cb3Regs<RTW> s;
    issue();
    __builtin_amdgcn_sched_barrier(0);
    {
        const int sta = w.cta >> 2;
#pragma unroll
        for (int c = 0; c < 5; ++c) s.cbv[c] = cb3_group(w, 5 * sta + c);
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int r = 0; r < RTW; ++r) s.ring[c][r] = cb3_tile(w, 4 * sta + c, r);
#pragma unroll
        for (int r = 0; r < RTW; ++r) s.acc[r] = (f32x4){0.f, 0.f, 0.f, 0.f};
    }
    __builtin_amdgcn_sched_barrier(0);
    stage();
    for (;;) {
        const int st_last = (w.ctb - 1) >> 2;       // the segment's last super tile (maybe partial)
        int st = w.cta >> 2;
        // refills of super tiles st + 1 < st_last: whole super tiles inside the split (ct < 4 st_last <= ctb - 1, and
        // their codebook groups <= 5 st_last - 1 <= g_last), none the split's first (ct > cta, groups > g_first)
        for (; st + 1 < st_last; ++st) {
            cb3_ctile_src<TWO, RTW, 0, true>(w, w, st + 1, s, st, true);
            cb3_ctile_src<TWO, RTW, 1, true>(w, w, st + 1, s, st, true);
            cb3_ctile_src<TWO, RTW, 2, true>(w, w, st + 1, s, st, true);
            cb3_ctile_src<TWO, RTW, 3, true>(w, w, st + 1, s, st, true);
        }
        if (st < st_last) {                         // the refills of the last super tile, which may end early
            cb3_ctile_src<TWO, RTW, 0>(w, w, st + 1, s, st, true);
            cb3_ctile_src<TWO, RTW, 1>(w, w, st + 1, s, st, true);
            cb3_ctile_src<TWO, RTW, 2>(w, w, st + 1, s, st, true);
            cb3_ctile_src<TWO, RTW, 3>(w, w, st + 1, s, st, true);
            ++st;
        }
        Cb3Wave nw = w;
        const bool more = next(nw);
        if (!more) {                                // nothing follows: the refills touch no memory
            nw.cta = nw.ctb = 0;
            nw.g_first = 1;
            nw.g_last = 0;
        }
        const int nst = nw.cta >> 2;
        const int nct = w.ctb - 4 * st;             // 1..4 column tiles of the last super tile
        cb3_ctile_src<TWO, RTW, 0>(w, nw, nst, s, st, true);
        cb3_ctile_src<TWO, RTW, 1>(w, nw, nst, s, st, nct > 1);
        cb3_ctile_src<TWO, RTW, 2>(w, nw, nst, s, st, nct > 2);
        cb3_ctile_src<TWO, RTW, 3>(w, nw, nst, s, st, nct > 3);
        store(s.acc);
#pragma unroll
        for (int r = 0; r < RTW; ++r) s.acc[r] = (f32x4){0.f, 0.f, 0.f, 0.f};
        if (!more) break;
        boundary(nw);
        w = nw;
    }
}

}  // namespace mi
