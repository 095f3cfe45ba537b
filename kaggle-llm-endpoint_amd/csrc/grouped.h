// Grouped codebook-dequant expert matvec kernels for gfx950 (MI355X).
//
// One launch covers every (expert group, row range, column split) task of a call.  A workgroup of 4 wavefronts
//   1. regroups the call's routing on the device (find_group: slots sorted by expert, <= 16 slots per group),
//   2. issues its first weight loads, then stages the group's activation rows for its column split in LDS while
//      they are in flight (f32 activations -- h for the down projection -- as bf16 hi + lo parts),
//   3. streams the expert's planes once with 128-bit loads (every wavefront load is 1 KB contiguous) and decodes
//      the codes to bf16 in registers for the matrix cores, all of the group's tokens in one 16-column tile: CB3
//      tiles (16-64 rows per wavefront), IQ2_S, IQ3_S and IQ4_XS planes (64 rows per wavefront, iq2_mfma.h,
//      iq3_mfma.h, iq4_mfma.h),
//   4. writes its f32 partial sums; the next launch reduces them in a fixed order (the SwiGLU kernel forms h from
//      the gate/up partials, the combine kernel sums the down partials with the routing weights, the split
//      reduction finishes a matvec).
// Results are therefore deterministic: no float atomics, every sum in a fixed order.
#pragma once
#include <type_traits>

#include "cb3_tiles.h"
#include "formats.h"
#include "iq2_mfma.h"
#include "iq4_mfma.h"
#include "kq_mfma.h"

namespace mi {

// internal linkage: every translation unit that launches a kernel carries its own copy
static __constant__ uint32_t kGridConst[512] = {
#include "iq3s_grid.inc"
};
static __constant__ uint32_t kGrid2Const[2048] = {
#include "iq2s_grid.inc"
};
static __constant__ int8_t kKvConst[16] = {
#include "iq4nl_kvalues.inc"
};

enum Mode { kGateUp = 0, kDown = 1, kMatvec = 2 };

struct Table {
    int qtype;
    Cb3Table cb3;
    Iq3Table iq3;
    Iq4Table iq4;
    Iq2Table iq2;
    KqTable kq;
};

struct KArgs {
    Table t0, t1;              // gate/up (kGateUp) or the single table
    int R, K;                  // rows, cols of the table(s)
    int E;
    int n_route;               // routed slots (N*k, or n_slots for kMatvec)
    int N, k;
    int shared_expert;
    int S;                     // column splits
    int ualign;                // split boundaries at multiples of this many units
    int n_units;               // column units (CB3: 160-column tiles, IQ3_S: 256-column blocks)
    int RB;                    // row groups of a matrix (R / rows per wavefront)
    int RBW;                   // row groups per workgroup (kDown / kMatvec: 4, kGateUp: 2)
    int RBG;                   // workgroup row ranges: ceil(RB / RBW)
    int xs_max;                // LDS row pitch in dwords (largest over the splits)
    int t_rows;                // LDS rows staged (class of the largest group)
    // activations
    const uint16_t *x_bf16;    // kGateUp bf16: [N, K] tokens; kDown: bf16 high part of h [NS, stride] by slot;
                               // kMatvec bf16: [n_slots, stride]
    const uint16_t *x_lo;      // kDown: bf16 remainder of h [NS, stride] (h = x_bf16 + x_lo to 16 mantissa bits)
    const float *x_f32;        // kGateUp f32: [N, stride] tokens; kMatvec f32: [n_slots, stride] (split into bf16
                               // high + remainder while staging)
    int x_stride;
    // kDown without a SwiGLU launch: h formed while staging from the gate/up split partials [gu_S][2][NS][stride]
    // (sum of the splits in order, clamped SwiGLU, bf16 high + remainder: the SwiGLU kernel's arithmetic)
    const float *gu_part;
    int gu_S;
    float limit;
    const int32_t *idx;
    // partial sums
    float *part;               // [S * nmat * NS * R] written by this launch
    int NS;                    // slots incl. shared
};

__host__ __device__ inline int slot_token(int slot, int n_route, int k) {
    return slot < n_route ? slot / k : slot - n_route;
}

// `stage` stages the activation rows into LDS (ending in a workgroup barrier); the decoders call it right after
// issuing their first weight loads, so the staging latency overlaps the first HBM round trip.

// CB3 rows (16 RTW per wavefront, matrix cores).  B-operand lane (column jt = lane % 16 of the 16x16 tile, k-chunk q):
//   bf16 activations: token jt;
//   f32 activations, launches of at most 8 tokens per group: hi part of token jt (jt < 8) or lo part of token jt - 8
//     (jt >= 8), and the two accumulator columns are added at the end -- one instruction covers hi and lo;
//   f32 activations, launches of up to 16 tokens per group: hi and lo of token jt, two instructions per k-step.
// Columns jt >= the staged rows read a clamped row; their accumulator columns are never stored.
// WT: the partials are stored write-through (sc1), so a workgroup on another XCD can read them inside the same launch
// once the storing workgroup has published a completion count.
template <bool HILO, int TCMAX, int RTW, bool WT = false, class Stage>
__device__ __forceinline__ void cb3_run_and_store(const Cb3Table &tb, int e, int rg, int u0, int u1, int c0,
                                                  const uint32_t *xh, const uint32_t *xl, int xsp, int t_rows, int n,
                                                  const int *slots, float *part_base, int R, uint4 *cbl,
                                                  Stage &&stage) {
    const int lane = threadIdx.x & 63, jt = lane & 15, q = lane >> 4;
    Cb3Wave w;
    const uint32_t *qt = tb.qs + (size_t)e * tb.CT * tb.RT * 256;
    const uint32_t *cbe = tb.cb + (size_t)e * tb.G * tb.R * 4;
    w.qb = __builtin_amdgcn_make_buffer_rsrc((void *)qt, (short)0, 0x7fffffff, kBufferWord3);
    w.qnull = __builtin_amdgcn_make_buffer_rsrc((void *)qt, (short)0, 0, kBufferWord3);
    w.cbb = __builtin_amdgcn_make_buffer_rsrc((void *)cbe, (short)0, 0x7fffffff, kBufferWord3);
    w.cbnull = __builtin_amdgcn_make_buffer_rsrc((void *)cbe, (short)0, 0, kBufferWord3);
    w.ct_bytes = (uint32_t)tb.RT * 1024u;
    w.rt_bytes = (uint32_t)(rg * RTW) * 1024u;
    w.g_bytes = (uint32_t)tb.R * 16u;
    w.row_bytes = (uint32_t)(rg * 16 * RTW) * 16u;
    w.cta = u0;
    w.ctb = u1;
    w.g_first = (kCb3TileCols * u0) >> 7;
    w.g_last = min((kCb3TileCols * u1 - 1) >> 7, tb.G - 1);
    w.lane16 = (uint32_t)lane * 16u;
    w.cblane16 = (uint32_t)(lane & (16 * RTW - 1)) * 16u;
    w.cbl = cbl;
    constexpr bool two = HILO && TCMAX > 8;
    constexpr bool pair = HILO && !two;          // hi / lo in the two halves of the tile's columns
    int row = pair ? (jt & 7) : jt;
    row = min(row, t_rows - 1);
    w.xh = ((pair && jt >= 8) ? xl : xh) + row * xsp + 4 * q;
    w.xl = xl + row * xsp + 4 * q;
    f32x4 acc[RTW];
    cb3_accum_mfma<two, RTW>(w, acc, stage);
    if (pair) {
#pragma unroll
        for (int r = 0; r < RTW; ++r)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[r][i] += __shfl_down(acc[r][i], 8, 16);
    }
    if (jt < n) {
        const size_t off = (size_t)slots[jt] * R + rg * 16 * RTW + 4 * q;
        if constexpr (WT) {
            const __amdgpu_buffer_rsrc_t pr =
                __builtin_amdgcn_make_buffer_rsrc((void *)part_base, (short)0, 0x7fffffff, kBufferWord3);
#pragma unroll
            for (int r = 0; r < RTW; ++r) wt_store4(pr, (uint32_t)(off + 16 * r) * 4u, acc[r]);
        } else {
            float *dst = part_base + off;
#pragma unroll
            for (int r = 0; r < RTW; ++r)
                *(float4 *)(dst + 16 * r) = make_float4(acc[r][0], acc[r][1], acc[r][2], acc[r][3]);
        }
    }
}

// Activation rows staged with direct-to-LDS loads by the grouped kernel: up to this many (token classes 1-4).
constexpr int kDmaStageRows = 4;

// Workgroups are 4 wavefronts sharing one staged activation slice: gate/up = (gate, up) x 2 row groups, down /
// matvec = 4 row groups.  A row group is the rows of one wavefront: 64 (CB3) or 256 (IQ3_S).
constexpr int kWgWaves = 4;

// Rows per wavefront: CB3 16 RTW (RTW row tiles), IQ3_S 64 (four interleaved row tiles).
template <int QT, int RTW>
__host__ __device__ constexpr int wave_rows() { return QT == MI_QT_CB3 ? 16 * RTW : kIq3WaveRows; }

// The kernels are held to MI_CB3_WAVES wavefronts per SIMD (3: <= 168 VGPRs): more HBM requests in flight per CU.
#ifndef MI_CB3_WAVES
#define MI_CB3_WAVES 3
#endif
// Every decoder fits the common bound.
template <int QT>
__host__ __device__ constexpr int min_waves_per_simd() { return MI_CB3_WAVES; }

template <int MODE, int QT, int TCMAX, int RTW>
__global__ void __launch_bounds__(64 * kWgWaves, min_waves_per_simd<QT>()) grouped_kernel(KArgs a) {
    extern __shared__ uint32_t xlds[];
    __shared__ GroupScratch sc;
    // IQ3_S, IQ2_S: grid and sign tables; IQ4_XS: the level-pair table
    __shared__ typename std::conditional<
        QT == MI_QT_IQ3_S, Iq3Lds,
        typename std::conditional<
            QT == MI_QT_IQ4_XS, Iq4Lds,
            typename std::conditional<QT == MI_QT_IQ2_S, Iq2Lds,
                                      typename std::conditional<(QT == MI_QT_Q2_K || QT == MI_QT_Q3_K), KqLds,
                                                                char>::type>::type>::type>::type iq;
    __shared__ uint4 cbl[QT == MI_QT_CB3 ? kWgWaves * 5 * 64 : 1];   // CB3: per-wavefront codebook slots
    // IQ4_XS at one token: the plane words stream through per-wavefront LDS rings (iq4m_accum_lds)
    constexpr bool kIq4Lds = QT == MI_QT_IQ4_XS && TCMAX == 1;
    __shared__ uint4 iq4ring[kIq4Lds ? kWgWaves * kIq4RingUint4 : 1];
    __shared__ int s_tok[kMaxT];

    constexpr bool cb3 = QT == MI_QT_CB3;
    constexpr int WR = wave_rows<QT, RTW>();
    const int tid = threadIdx.x;
    const int task = blockIdx.x;
    const int split = task % a.S;
    const int rbg = (task / a.S) % a.RBG;
    const int gi = task / (a.S * a.RBG);

    find_group(sc, a.idx, a.n_route, a.E, a.shared_expert, a.N, gi, a.t_rows);
    // LDS values and the wavefront index are wave-uniform: keep them (and every address built from them) scalar
    const int e = __builtin_amdgcn_readfirstlane(sc.g.expert);
    if (e < 0) return;
    const int n = __builtin_amdgcn_readfirstlane(sc.g.n);

    // published by the barrier after the slot list
    if constexpr (QT == MI_QT_IQ3_S) iq3_fill_lds(iq, kGridConst);
    if constexpr (QT == MI_QT_IQ4_XS) iq4_fill_lds(iq, kKvConst);
    if constexpr (QT == MI_QT_IQ2_S) iq2_fill_lds(iq, kGrid2Const);
    if constexpr (QT == MI_QT_Q2_K || QT == MI_QT_Q3_K) kq_fill_lds(iq);

    // column range of the split; CB3 stages its padded column tiles (columns >= K are zero)
    const int ucols = cb3 ? Cb3Table::kUnitCols : 256;      // IQ formats: 256-weight blocks
    const int nb = (a.n_units + a.ualign - 1) / a.ualign;
    const int u0 = min(a.n_units, a.ualign * (int)((long long)split * nb / a.S));
    const int u1 = min(a.n_units, a.ualign * (int)((long long)(split + 1) * nb / a.S));
    // CB3 stages from the start of the super tile holding the split's first column tile (zeros before it)
    const int c0 = cb3 ? 4 * kCb3TileCols * (u0 >> 2) : u0 * ucols;
    const int cv = u0 * ucols;                // first column of the split
    const int c1 = cb3 ? u1 * ucols : min(a.K, u1 * ucols);
    const int xs = (c1 - c0) >> 1;            // dwords per staged row
    const int xsp = cb3_row_pitch(xs);        // row pitch: whole 64-dword chunks, skewed by 4 banks per row
    const bool hilo = (MODE == kDown) || a.x_f32 != nullptr;
    uint32_t *xh = xlds;
    uint32_t *xl = xlds + (size_t)a.t_rows * a.xs_max;

    // activation rows t < t_rows (rows >= n are zero) of the split's columns, as bf16 pairs (hi/lo for f32)
    if (tid < kMaxT) s_tok[tid] = tid < n ? sc.g.slot[tid] : -1;
    __syncthreads();
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    // CB3 with bf16 sources (x, or h as its bf16 high part and remainder): the rows go straight from memory to LDS
    // (buffer_load ... lds), issued BEFORE the first weight loads.  A wavefront's loads complete in issue order, so
    // the staging then waits only for these loads, not for the weight ring behind them, and each tile's matrix-core
    // work starts as soon as that tile arrives.
    // (with many staged rows the direct loads outnumber the register path's 8-byte ones: register staging there)
    const bool dma = cb3 && a.x_f32 == nullptr && a.gu_part == nullptr && a.t_rows <= kDmaStageRows;
    bool stage_ring = true;     // the wavefront issues its weight ring before staging (false: it only stages)
    if (dma) {
        const __amdgpu_buffer_rsrc_t rh =
            __builtin_amdgcn_make_buffer_rsrc((void *)a.x_bf16, (short)0, 0x7fffffff, kBufferWord3);
        const __amdgpu_buffer_rsrc_t rl =
            __builtin_amdgcn_make_buffer_rsrc((void *)(hilo ? a.x_lo : a.x_bf16), (short)0, 0x7fffffff, kBufferWord3);
        const int cend = min(c1, a.K);
        // whole 256-dword chunks with 16 bytes per lane when every bound is a multiple of 8 columns, the rest with 4
        const int n16 = ((c0 | cv | cend | a.x_stride) & 7) == 0 ? xs >> 8 : 0, nt = (xs - 256 * n16 + 63) >> 6;
        const int per16 = (hilo ? 2 : 1) * n16, pert = (hilo ? 2 : 1) * nt;
        for (int i = wave; i < a.t_rows * per16; i += kWgWaves) {
            const int t = i / per16, r = i - t * per16, plane = r / n16, ch = r - plane * n16;
            const int slot = s_tok[t];
            const int c = c0 + 512 * ch + 8 * lane;
            const int row = (MODE == kGateUp) ? slot_token(slot, a.n_route, a.k) : slot;
            const uint32_t voff = (slot >= 0 && c >= cv && c < cend) ? (uint32_t)((size_t)row * a.x_stride + c) * 2u
                                                                     : kStageOut;
            uint32_t *dst = (plane ? xl : xh) + t * xsp + 256 * ch;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(plane ? rl : rh, (__attribute__((address_space(3))) void *)dst,
                                                     16, voff, 0, 0, 0);
        }
        for (int i = wave; i < a.t_rows * pert; i += kWgWaves) {
            const int t = i / pert, r = i - t * pert, plane = r / nt, d0 = 256 * n16 + 64 * (r - plane * nt);
            const int slot = s_tok[t];
            const int c = c0 + 2 * (d0 + lane);
            const int row = (MODE == kGateUp) ? slot_token(slot, a.n_route, a.k) : slot;
            const uint32_t voff = (slot >= 0 && c >= cv && c < cend) ? (uint32_t)((size_t)row * a.x_stride + c) * 2u
                                                                     : kStageOut;
            uint32_t *dst = (plane ? xl : xh) + t * xsp + d0;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(plane ? rl : rh, (__attribute__((address_space(3))) void *)dst,
                                                     4, voff, 0, 0, 0);
        }
        // the weight loads must not be scheduled ahead of the staging loads (the staging wait counts them)
        __builtin_amdgcn_sched_barrier(0);
    }
    auto stage = [&]() {
        if (dma) {
            // every load this wavefront issued before the weight ring has completed; then all wavefronts' rows
            __builtin_amdgcn_sched_barrier(0);
            if (stage_ring) vm_wait<4 * RTW + 5>();
            else vm_wait<0>();
            lds_barrier();                          // the weight ring stays in flight
            return;
        }
        const int q4 = xs >> 1;           // 4-column quads per row
        const int nq = a.t_rows * q4;
        // every lane of a wavefront runs the same trips (IQ2_S reduces each row's maximum across the wavefront)
        for (int i0 = 0; i0 < nq; i0 += blockDim.x) {
            const int i = i0 + tid;
            const int t = min(i, nq - 1) / q4, q = i - t * q4;
            const int slot = i < nq ? s_tok[t] : -1;
            const int c = c0 + 4 * q;
            uint2 hv = make_uint2(0, 0), lv = make_uint2(0, 0);
            if (slot >= 0 && c >= cv && c < a.K) {
                if (!hilo) {
                    const int row = (MODE == kGateUp) ? slot_token(slot, a.n_route, a.k) : slot;
                    hv = *(const uint2 *)(a.x_bf16 + (size_t)row * a.x_stride + c);
                } else if (MODE == kDown && a.gu_part != nullptr) {
                    const size_t plane = (size_t)a.NS * a.x_stride, o = (size_t)slot * a.x_stride + c;
                    float4 g = make_float4(0.f, 0.f, 0.f, 0.f), u = g;
                    for (int sp = 0; sp < a.gu_S; ++sp) {
                        const float4 pg = *(const float4 *)(a.gu_part + (size_t)(2 * sp) * plane + o);
                        const float4 pu = *(const float4 *)(a.gu_part + (size_t)(2 * sp + 1) * plane + o);
                        g.x += pg.x; g.y += pg.y; g.z += pg.z; g.w += pg.w;
                        u.x += pu.x; u.y += pu.y; u.z += pu.z; u.w += pu.w;
                    }
                    uint32_t h0, l0, h1, l1, h2, l2, h3, l3;
                    split_bf16(swiglu_clamped(g.x, u.x, a.limit), h0, l0);
                    split_bf16(swiglu_clamped(g.y, u.y, a.limit), h1, l1);
                    split_bf16(swiglu_clamped(g.z, u.z, a.limit), h2, l2);
                    split_bf16(swiglu_clamped(g.w, u.w, a.limit), h3, l3);
                    hv = make_uint2(h0 | (h1 << 16), h2 | (h3 << 16));
                    lv = make_uint2(l0 | (l1 << 16), l2 | (l3 << 16));
                } else if (a.x_f32 == nullptr) {
                    hv = *(const uint2 *)(a.x_bf16 + (size_t)slot * a.x_stride + c);
                    lv = *(const uint2 *)(a.x_lo + (size_t)slot * a.x_stride + c);
                } else {
                    const int row = (MODE == kGateUp) ? slot_token(slot, a.n_route, a.k) : slot;
                    const float4 f = *(const float4 *)(a.x_f32 + (size_t)row * a.x_stride + c);
                    uint32_t h0, l0, h1, l1, h2, l2, h3, l3;
                    split_bf16(f.x, h0, l0);
                    split_bf16(f.y, h1, l1);
                    split_bf16(f.z, h2, l2);
                    split_bf16(f.w, h3, l3);
                    hv = make_uint2(h0 | (h1 << 16), h2 | (h3 << 16));
                    lv = make_uint2(l0 | (l1 << 16), l2 | (l3 << 16));
                }
            }
            if constexpr (QT == MI_QT_IQ2_S) {
                // the row's largest |value| (bf16 element, or high part + remainder): one LDS atomic per wavefront
                // when its quads lie in one row, per lane otherwise
                uint32_t m = 0u;
                if (i < nq) {
                    const uint32_t hw[4] = {hv.x & 0xffffu, hv.x >> 16, hv.y & 0xffffu, hv.y >> 16};
                    const uint32_t lw[4] = {lv.x & 0xffffu, lv.x >> 16, lv.y & 0xffffu, lv.y >> 16};
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        m = max(m, __float_as_uint(fabsf(bf16_to_f32(hw[j]) + (hilo ? bf16_to_f32(lw[j]) : 0.0f))));
                }
                const int t0 = __builtin_amdgcn_readfirstlane(t);
                if (__all(i >= nq || t == t0)) {
#pragma unroll
                    for (int o = 32; o > 0; o >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, o));
                    if (lane == 0 && m != 0u) atomicMax(&iq.amax[t0], m);
                } else if (m != 0u) {
                    atomicMax(&iq.amax[t], m);
                }
            }
            if (i >= nq) continue;
            if constexpr (QT == MI_QT_IQ4_XS) {
                // the decoder's column order inside each 32-column group (iq4_stage_pos)
                uint16_t *dh = (uint16_t *)(xh + t * xsp), *dl = (uint16_t *)(xl + t * xsp);
                const int o = 4 * q, g = o & ~31, p0 = g + iq4_stage_pos(o & 31);
                const uint32_t hw[4] = {hv.x & 0xffffu, hv.x >> 16, hv.y & 0xffffu, hv.y >> 16};
                const uint32_t lw[4] = {lv.x & 0xffffu, lv.x >> 16, lv.y & 0xffffu, lv.y >> 16};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    dh[p0 + 2 * j] = (uint16_t)hw[j];
                    if (hilo) dl[p0 + 2 * j] = (uint16_t)lw[j];
                }
            } else {
                *(uint2 *)(xh + t * xsp + 2 * q) = hv;
                if (hilo) *(uint2 *)(xl + t * xsp + 2 * q) = lv;
            }
        }
        if constexpr (QT == MI_QT_IQ2_S) {
            // in place: f16 high part and remainder of each value at its row's power of two (iq2_mfma.h)
            __syncthreads();
            for (int i = tid; i < nq; i += blockDim.x) {
                const int t = i / q4, q = i - t * q4;
                const int shift = iq2_xshift(iq.amax[t]);
                uint2 hv = *(const uint2 *)(xh + t * xsp + 2 * q), lv = make_uint2(0, 0);
                if (hilo) lv = *(const uint2 *)(xl + t * xsp + 2 * q);
                const uint32_t hw[4] = {hv.x & 0xffffu, hv.x >> 16, hv.y & 0xffffu, hv.y >> 16};
                const uint32_t lw[4] = {lv.x & 0xffffu, lv.x >> 16, lv.y & 0xffffu, lv.y >> 16};
                uint32_t fh[4], fl[4];
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    iq2_x16(bf16_to_f32(hw[j]) + (hilo ? bf16_to_f32(lw[j]) : 0.0f), shift, fh[j], fl[j]);
                *(uint2 *)(xh + t * xsp + 2 * q) = make_uint2(fh[0] | (fh[1] << 16), fh[2] | (fh[3] << 16));
                if (hilo) *(uint2 *)(xl + t * xsp + 2 * q) = make_uint2(fl[0] | (fl[1] << 16), fl[2] | (fl[3] << 16));
            }
        }
        __syncthreads();
    };

    const int mat = MODE == kGateUp ? (wave & 1) : 0;          // gate/up: odd wavefronts run the up matrix
    const Table &tb = mat ? a.t1 : a.t0;
    const int rg = rbg * a.RBW + (MODE == kGateUp ? (wave >> 1) : wave);
    if (rg >= a.RB) {           // wavefront past the last row group: it only helps stage
        stage_ring = false;
        stage();
        return;
    }
    const int nmat = MODE == kGateUp ? 2 : 1;
    float *part_base = a.part + (size_t)(split * nmat + mat) * a.NS * a.R;
    if constexpr (cb3) {
        if (hilo)
            cb3_run_and_store<true, TCMAX, RTW>(tb.cb3, e, rg, u0, u1, c0, xh, xl, xsp, a.t_rows, n, s_tok, part_base, a.R,
                                           cbl + wave * 5 * 64, stage);
        else
            cb3_run_and_store<false, TCMAX, RTW>(tb.cb3, e, rg, u0, u1, c0, xh, xl, xsp, a.t_rows, n, s_tok, part_base,
                                            a.R, cbl + wave * 5 * 64, stage);
    } else if constexpr (QT == MI_QT_IQ3_S) {
        if (hilo)
            iq3m_run_and_store<true, TCMAX>(tb.iq3, e, rg * WR, u0, u1, c0, iq, xh, xl, xsp, a.t_rows, n, s_tok,
                                            part_base, a.R, stage);
        else
            iq3m_run_and_store<false, TCMAX>(tb.iq3, e, rg * WR, u0, u1, c0, iq, xh, xl, xsp, a.t_rows, n, s_tok,
                                             part_base, a.R, stage);
    } else if constexpr (QT == MI_QT_Q2_K || QT == MI_QT_Q3_K) {
        constexpr bool q3 = QT == MI_QT_Q3_K;
        if (hilo)
            kqm_run_and_store<true, TCMAX, q3>(tb.kq, e, rg * WR, u0, u1, c0, iq, xh, xl, xsp, a.t_rows, n, s_tok,
                                               part_base, a.R, stage);
        else
            kqm_run_and_store<false, TCMAX, q3>(tb.kq, e, rg * WR, u0, u1, c0, iq, xh, xl, xsp, a.t_rows, n, s_tok,
                                                part_base, a.R, stage);
    } else if constexpr (QT == MI_QT_IQ2_S) {
        if (hilo)
            iq2m_run_and_store<true, TCMAX>(tb.iq2, e, rg * WR, u0, u1, c0, iq, xh, xl, xsp, a.t_rows, n, s_tok,
                                            part_base, a.R, stage);
        else
            iq2m_run_and_store<false, TCMAX>(tb.iq2, e, rg * WR, u0, u1, c0, iq, xh, xl, xsp, a.t_rows, n, s_tok,
                                             part_base, a.R, stage);
    } else {
        uint4 *ring = iq4ring + wave * kIq4RingUint4;
        if (hilo)
            iq4m_run_and_store<true, TCMAX, kIq4Lds>(tb.iq4, e, rg * WR, u0, u1, c0, iq, xh, xl, xsp, a.t_rows, n,
                                                     s_tok, part_base, a.R, stage, ring);
        else
            iq4m_run_and_store<false, TCMAX, kIq4Lds>(tb.iq4, e, rg * WR, u0, u1, c0, iq, xh, xl, xsp, a.t_rows, n,
                                                      s_tok, part_base, a.R, stage, ring);
    }
    // The partials are reduced by the next launch (gate/up: the SwiGLU kernel; down: the combine; matvec: the split
    // reduction): kernel order publishes them, so no completion counters or fences are needed.
}

}  // namespace mi
