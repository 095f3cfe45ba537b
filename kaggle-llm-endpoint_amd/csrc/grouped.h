// Grouped codebook-dequant expert matvec kernels for gfx950 (MI355X) and their C ABI.
//
// One launch covers every (expert group, 256-row block, column split) task of a call.  A workgroup
//   1. regroups the call's routing on the device (find_group: slots sorted by expert, <= 16 slots per group),
//   2. issues its first weight loads, then stages the group's activation rows for its column split in LDS while
//      they are in flight (the down projection rebuilds h = SwiGLU(gate, up) here from the gate/up partials),
//   3. streams the expert's planes once -- each lane owns 4 consecutive rows, so every plane access is one
//      128-bit load and the wavefront reads 1 KB contiguous -- decoding codes to bf16 in registers and
//      accumulating bf16-pair dot products in f32 for all the group's rows at once,
//   4. writes its f32 partial sums.  Gate/up stops there: the next launch reduces them.  Matvec and down bump an
//      agent-scope completion counter; the workgroup that completes a (group, row block) -- or, for the down
//      projection, a (row block, token) -- reduces the partials in a fixed order and stores the rows or runs the
//      routing-weighted combine.
// Results are therefore deterministic: no float atomics, every sum in a fixed order.
#pragma once
#include "formats.h"

namespace mi {

// internal linkage: every translation unit that launches a kernel carries its own copy
static __constant__ uint32_t kGridConst[512] = {
#include "iq3s_grid.inc"
};

enum Mode { kGateUp = 0, kDown = 1, kMatvec = 2 };

struct Table {
    int qtype;
    Cb3Table cb3;
    Iq3Table iq3;
};

struct KArgs {
    Table t0, t1;              // gate/up (kGateUp) or the single table
    int R, K;                  // rows, cols of the table(s)
    int E;
    int n_route;               // routed slots (N*k, or n_slots for kMatvec)
    int N, k;
    int shared_expert;
    int S;                     // column splits
    int n_units;               // column units (CB3: word pairs, IQ3_S: blocks)
    int RB;                    // row blocks (R / 256)
    int RBW;                   // row blocks per workgroup (kDown / kMatvec: one per wavefront; kGateUp: 1)
    int RBG;                   // row-block groups: ceil(RB / RBW)
    int xs_max;                // LDS dwords per staged row
    int t_rows;                // LDS rows staged (class of the largest group)
    // activations
    const uint16_t *x_bf16;    // kGateUp: [N, K] tokens; kMatvec bf16: [n_slots, stride]
    const float *x_f32;        // kMatvec f32 activations [n_slots, stride]
    int x_stride;
    const int32_t *idx;
    const float *w;
    float limit;
    // outputs / workspace
    float *part;               // [S * nmat * NS * R] partial sums written by this launch
    const float *p1;           // kDown: the gate/up launch's partials [S1 * 2 * NS * K] (h is rebuilt from them)
    int S1;                    // kDown: column splits of the gate/up launch
    uint32_t *cnt;             // completion counters
    float *out_f32;            // kDown: [N, R]; kMatvec: [n_slots, R]
    uint16_t *out_bf16;        // kDown: [N, R] (optional)
    int NS;                    // slots incl. shared
};

__host__ __device__ inline int slot_token(int slot, int n_route, int k) {
    return slot < n_route ? slot / k : slot - n_route;
}

// `stage` stages the activation rows into LDS (ending in a workgroup barrier); the decoders call it right after
// issuing their first weight loads, so the staging latency overlaps the first HBM round trip.
template <int QT, int TC, bool HILO, class Stage>
__device__ __forceinline__ void accum_rows(const Table &tb, int e, int r0, int u0, int u1, int c0,
                                           const uint32_t *grid, const uint32_t *xh, const uint32_t *xl, int xs,
                                           float (&acc)[4][TC], Stage &&stage) {
    if constexpr (QT == MI_QT_CB3) {
        // units are 640-column super-tiles; 1-2 activation rows take the static straight-line tile path
        if constexpr (TC <= 2) cb3_accum_tiles<TC, HILO>(tb.cb3, e, r0, u0, u1, c0, xh, xl, xs, acc, stage);
        else {
            const int npairs = (tb.cb3.Wd + 1) / 2;
            cb3_accum<TC, HILO>(tb.cb3, e, r0, 32 * u0, min(32 * u1, npairs), c0, xh, xl, xs, acc, stage);
        }
    } else {
        iq3_accum<TC, HILO>(tb.iq3, e, r0, u0, u1, c0, grid, xh, xl, xs, acc, stage);
    }
}

// Accumulate with the smallest token class >= n (classes above TCMAX are not compiled into the launch) and store the
// partials of the n real rows.
template <int QT, bool HILO, int TCMAX, class Stage>
__device__ __forceinline__ void run_and_store(const Table &tb, int e, int r0, int u0, int u1, int c0, const uint32_t *grid,
                              const uint32_t *xh, const uint32_t *xl, int xs, int n, const int *slots,
                              float *part_base, int R, Stage &&stage) {
#define MI_RUN_CLASS(TCV)                                                                          \
    {                                                                                              \
        float acc[4][TCV];                                                                         \
        _Pragma("unroll") for (int i = 0; i < 4; ++i) _Pragma("unroll") for (int t = 0; t < TCV; ++t) acc[i][t] = 0.f; \
        accum_rows<QT, TCV, HILO>(tb, e, r0, u0, u1, c0, grid, xh, xl, xs, acc, stage);            \
        _Pragma("unroll") for (int t = 0; t < TCV; ++t) {                                          \
            if (t < n) {                                                                           \
                float4 v = make_float4(acc[0][t], acc[1][t], acc[2][t], acc[3][t]);                \
                *(float4 *)(part_base + (size_t)slots[t] * R + r0) = v;                            \
            }                                                                                      \
        }                                                                                          \
    }
    if (TCMAX == 1 || n <= 1) MI_RUN_CLASS(1)
    else if (TCMAX == 2 || n <= 2) MI_RUN_CLASS((TCMAX >= 2 ? 2 : 1))
    else if (TCMAX == 4 || n <= 4) MI_RUN_CLASS((TCMAX >= 4 ? 4 : 1))
    else if (TCMAX == 8 || n <= 8) MI_RUN_CLASS((TCMAX >= 8 ? 8 : 1))
    else MI_RUN_CLASS((TCMAX >= 16 ? 16 : 1))
#undef MI_RUN_CLASS
}

// Workgroup shape: gate/up = 2 wavefronts (gate, up) over one row block; down / matvec = kRbWaves wavefronts over
// kRbWaves consecutive row blocks, which share the staged activation slice.
constexpr int kRbWaves = 4;

template <int MODE, int QT, int TCMAX>
__global__ void __launch_bounds__(MODE == kGateUp ? 128 : 64 * kRbWaves) grouped_kernel(KArgs a) {
    extern __shared__ uint32_t xlds[];
    __shared__ GroupScratch sc;
    __shared__ uint32_t grid[512];
    __shared__ int s_tok[kMaxT];

    const int tid = threadIdx.x;
    const int task = blockIdx.x;
    const int split = task % a.S;
    const int rbg = (task / a.S) % a.RBG;
    const int gi = task / (a.S * a.RBG);

    find_group(sc, a.idx, a.n_route, a.E, a.shared_expert, a.N, gi, a.t_rows);
    const int e = sc.g.expert;
    if (e < 0) return;
    const int n = sc.g.n;

    constexpr bool iq3 = QT == MI_QT_IQ3_S;
    if (iq3)
        for (int i = tid; i < 512; i += blockDim.x) grid[i] = kGridConst[i];

    // column range of the split
    const int ucols = iq3 ? Iq3Table::kUnitCols : Cb3Table::kUnitCols;
    const int u0 = (int)((long long)split * a.n_units / a.S);
    const int u1 = (int)((long long)(split + 1) * a.n_units / a.S);
    const int c0 = u0 * ucols;
    const int c1 = min(a.K, u1 * ucols);
    const int xs = (c1 - c0) >> 1;   // dwords per staged row
    const bool hilo = (MODE == kDown) || (MODE == kMatvec && a.x_f32 != nullptr);
    uint32_t *xh = xlds;
    uint32_t *xl = xlds + (size_t)a.t_rows * a.xs_max;

    // activation rows t < t_rows (rows >= n are zero) of the split's columns, as bf16 pairs (hi/lo for f32)
    if (tid < kMaxT) s_tok[tid] = tid < n ? sc.g.slot[tid] : -1;
    __syncthreads();
    auto stage = [&]() {
        const int q4 = xs >> 1;           // 4-column quads per row
        for (int i = tid; i < a.t_rows * q4; i += blockDim.x) {
            const int t = i / q4, q = i - t * q4;
            const int slot = s_tok[t];
            const int c = c0 + 4 * q;
            uint2 hv = make_uint2(0, 0), lv = make_uint2(0, 0);
            if (slot >= 0) {
                if (!hilo) {
                    const int row = (MODE == kGateUp) ? slot_token(slot, a.n_route, a.k) : slot;
                    hv = *(const uint2 *)(a.x_bf16 + (size_t)row * a.x_stride + c);
                } else {
                    float4 f;
                    if (MODE == kDown) {
                        // h = silu(min(g, L)) * clip(u, -L, L) of the gate/up partials, splits summed in order
                        float4 g = make_float4(0.f, 0.f, 0.f, 0.f), u = g;
                        for (int s1 = 0; s1 < a.S1; ++s1) {
                            const float4 pg = *(const float4 *)(a.p1 + ((size_t)(s1 * 2 + 0) * a.NS + slot) * a.K + c);
                            const float4 pu = *(const float4 *)(a.p1 + ((size_t)(s1 * 2 + 1) * a.NS + slot) * a.K + c);
                            g.x += pg.x; g.y += pg.y; g.z += pg.z; g.w += pg.w;
                            u.x += pu.x; u.y += pu.y; u.z += pu.z; u.w += pu.w;
                        }
                        f = make_float4(swiglu_clamped(g.x, u.x, a.limit), swiglu_clamped(g.y, u.y, a.limit),
                                        swiglu_clamped(g.z, u.z, a.limit), swiglu_clamped(g.w, u.w, a.limit));
                    } else {
                        f = *(const float4 *)(a.x_f32 + (size_t)slot * a.x_stride + c);
                    }
                    uint32_t h0, l0, h1, l1, h2, l2, h3, l3;
                    split_bf16(f.x, h0, l0);
                    split_bf16(f.y, h1, l1);
                    split_bf16(f.z, h2, l2);
                    split_bf16(f.w, h3, l3);
                    hv = make_uint2(h0 | (h1 << 16), h2 | (h3 << 16));
                    lv = make_uint2(l0 | (l1 << 16), l2 | (l3 << 16));
                }
            }
            *(uint2 *)(xh + t * xs + 2 * q) = hv;
            if (hilo) *(uint2 *)(xl + t * xs + 2 * q) = lv;
        }
        __syncthreads();
    };

    const int wave = tid >> 6, lane = tid & 63;
    const Table &tb = (MODE == kGateUp && wave == 1) ? a.t1 : a.t0;
    const int rb = rbg * a.RBW + (MODE == kGateUp ? 0 : wave);
    if (rb >= a.RB) {           // wavefront past the last row block: it only helps stage
        stage();
        return;
    }
    const int r0 = rb * kRowBlock + lane * kRowsPerLane;
    const int nmat = MODE == kGateUp ? 2 : 1;
    const int mat = MODE == kGateUp ? wave : 0;   // gate/up: wave 0 = gate, wave 1 = up
    float *part_base = a.part + (size_t)(split * nmat + mat) * a.NS * a.R;
    if (MODE == kDown)
        run_and_store<QT, true, TCMAX>(tb, e, r0, u0, u1, c0, grid, xh, xl, xs, n, s_tok, part_base, a.R, stage);
    else if (MODE == kGateUp)
        run_and_store<QT, false, TCMAX>(tb, e, r0, u0, u1, c0, grid, xh, xl, xs, n, s_tok, part_base, a.R, stage);
    else if (hilo)
        run_and_store<QT, true, TCMAX>(tb, e, r0, u0, u1, c0, grid, xh, xl, xs, n, s_tok, part_base, a.R, stage);
    else
        run_and_store<QT, false, TCMAX>(tb, e, r0, u0, u1, c0, grid, xh, xl, xs, n, s_tok, part_base, a.R, stage);
    // gate/up: the partials are reduced by the down launch while it stages h (kernel order publishes them)
    if (MODE == kGateUp) return;
    // From here on every wavefront works alone on its own row block (no workgroup barriers).
    fence_release_agent();   // this wavefront's partial stores, before its completion count

    if (MODE == kMatvec) {
        // the wavefront completing (group, row block) reduces the splits in order and stores the rows
        uint32_t *c = a.cnt + gi * a.RB + rb;
        uint32_t prev = 0;
        if (lane == 0) prev = counter_add(c, 1u);
        if (__shfl(prev, 0, kWave) != (uint32_t)(a.S - 1)) return;
        fence_acquire_agent();
        for (int t = 0; t < n; ++t) {
            const int slot = s_tok[t];
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            for (int s = 0; s < a.S; ++s) {
                const float4 p = *(const float4 *)(a.part + ((size_t)s * a.NS + slot) * a.R + r0);
                v.x += p.x; v.y += p.y; v.z += p.z; v.w += p.w;
            }
            *(float4 *)(a.out_f32 + (size_t)slot * a.R + r0) = v;
        }
        if (lane == 0) counter_reset(c);
        return;
    }

    // kDown: one completion counter per (row block, token); the last contributor combines that token's rows.
    // lane t < n handles slot t of the group.
    int mylast = 0, mytok = -1;
    if (lane < n) {
        const int slot = s_tok[lane];
        mytok = slot_token(slot, a.n_route, a.k);
        int nvalid = 0;
        for (int j = 0; j < a.k; ++j) {
            const int ej = a.idx[mytok * a.k + j];
            nvalid += (ej >= 0 && ej < a.E) ? 1 : 0;
        }
        nvalid += a.shared_expert >= 0 ? 1 : 0;
        const uint32_t target = (uint32_t)(nvalid * a.S);
        mylast = counter_add(a.cnt + (size_t)rb * a.N + mytok, 1u) == target - 1u;
    }
    uint64_t lastmask = __ballot(mylast);
    if (lastmask) fence_acquire_agent();
    while (lastmask) {
        const int t = __builtin_ctzll(lastmask);
        lastmask &= lastmask - 1;
        const int tok = __shfl(mytok, t, kWave);
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int j = 0; j < a.k; ++j) {
            const int ej = a.idx[tok * a.k + j];
            if (ej < 0 || ej >= a.E) continue;
            const int slot = tok * a.k + j;
            float4 ys = make_float4(0.f, 0.f, 0.f, 0.f);
            for (int s = 0; s < a.S; ++s) {
                const float4 p = *(const float4 *)(a.part + ((size_t)s * a.NS + slot) * a.R + r0);
                ys.x += p.x; ys.y += p.y; ys.z += p.z; ys.w += p.w;
            }
            const float wj = a.w[tok * a.k + j];
            acc.x += wj * ys.x; acc.y += wj * ys.y; acc.z += wj * ys.z; acc.w += wj * ys.w;
        }
        if (a.shared_expert >= 0) {
            const int slot = a.n_route + tok;
            float4 ys = make_float4(0.f, 0.f, 0.f, 0.f);
            for (int s = 0; s < a.S; ++s) {
                const float4 p = *(const float4 *)(a.part + ((size_t)s * a.NS + slot) * a.R + r0);
                ys.x += p.x; ys.y += p.y; ys.z += p.z; ys.w += p.w;
            }
            acc.x += ys.x; acc.y += ys.y; acc.z += ys.z; acc.w += ys.w;
        }
        if (a.out_f32) *(float4 *)(a.out_f32 + (size_t)tok * a.R + r0) = acc;
        if (a.out_bf16) {
            uint2 b;
            b.x = f32_to_bf16_rne(acc.x) | (f32_to_bf16_rne(acc.y) << 16);
            b.y = f32_to_bf16_rne(acc.z) | (f32_to_bf16_rne(acc.w) << 16);
            *(uint2 *)(a.out_bf16 + (size_t)tok * a.R + r0) = b;
        }
        if (lane == 0) counter_reset(a.cnt + (size_t)rb * a.N + tok);
    }
}

}  // namespace mi
