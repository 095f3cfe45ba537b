// Persistent grouped CB3 kernels (gate/up partials, down partials) for gfx950.
//
// The separate grouped kernel gives every (expert group, row range, column split) task a workgroup of its own, so
// every task pays the workgroup start, the routing lookup and a full HBM round trip before its first tile can be
// decoded, and a one-task workgroup leaves HBM idle while it decodes its last super tile.  Here a grid of P resident
// workgroups splits the ordered task list into P contiguous ranges:
//   - the routing is grouped once per workgroup (build_group_table);
//   - every wavefront streams its tasks' segments back to back (cb3_stream): the code ring and the codebook slots
//     are refilled from the next task's first super tile while the current task finishes;
//   - tasks are ordered (group, split, row range), so consecutive tasks of a range mostly share their staged
//     activations; they are restaged (between two workgroup barriers) only when the group or the split changes;
//   - activations are staged with direct-to-LDS loads issued ahead of the weight ring, so a wavefront starts
//     decoding when its first tile lands, not when its whole ring has.
// The tasks are independent (each writes its own partial rows, reduced by the next launch), so nothing waits on
// another workgroup.
#pragma once
#include "fused_decode.h"

namespace mi {

struct PArgs {
    Cb3Table t0, t1;           // gate/up (kGateUp) or down (t0 only)
    int R, K;                  // rows, cols of the table(s)
    int E, n_route, N, k, shared_expert, NS, t_rows;
    int S, al, nu, RB, RBG, xs_max;
    int P;                     // workgroups of the launch
    const uint16_t *x;         // kGateUp: x bf16 [N, K]; kDown: bf16 high part of h [NS, K]
    const uint16_t *x_lo;      // kDown: bf16 remainder of h [NS, K]
    const int32_t *idx;
    float *part;               // [S][nmat][NS][R]
};

template <int MODE, int TC, int RTW>
__global__ void __launch_bounds__(64 * kWgWaves, MI_CB3_WAVES) pstream_kernel(PArgs a) {
    extern __shared__ uint32_t xlds[];
    __shared__ GroupTable gt;
    __shared__ uint4 cbl[kWgWaves * 5 * 64];
    __shared__ int s_tok[kMaxT];
    constexpr bool hilo = MODE == kDown;
    constexpr bool two = hilo && TC > 8;           // hi and lo in two instructions
    constexpr bool pair = hilo && !two;            // hi / lo in the two halves of the tile's columns
    constexpr int nmat = MODE == kGateUp ? 2 : 1;
    constexpr int RBW = MODE == kGateUp ? 2 : kWgWaves;   // row groups per task
    const int tid = threadIdx.x, lane = tid & 63, jt = lane & 15, q = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    build_group_table(gt, xlds, a.idx, a.n_route, a.E, a.shared_expert, a.N, a.t_rows);
    const int n_groups = __builtin_amdgcn_readfirstlane(gt.n_groups);
    const int per_g = a.S * a.RBG;
    const int T = n_groups * per_g;
    int t = (int)((long long)blockIdx.x * T / a.P);
    const int t_end = (int)((long long)(blockIdx.x + 1) * T / a.P);
    if (t >= t_end) return;

    const int mat = MODE == kGateUp ? (wave & 1) : 0;
    const Cb3Table &tb = mat ? a.t1 : a.t0;
    uint32_t *xh = xlds;
    uint32_t *xl = xlds + (size_t)a.t_rows * a.xs_max;

    // task t = (group gi, split, row range rbg), row range fastest
    struct Task {
        int gi, split, rbg, e, n, u0, u1, c0, cv, c1, xsp;
    };
    auto task_of = [&](int tt) {
        Task k;
        k.rbg = tt % a.RBG;
        const int gs = tt / a.RBG;
        k.split = gs % a.S;
        k.gi = gs / a.S;
        k.e = __builtin_amdgcn_readfirstlane(gt.expert[k.gi]);
        k.n = __builtin_amdgcn_readfirstlane(gt.n[k.gi]);
        const int nb = (a.nu + a.al - 1) / a.al;
        k.u0 = min(a.nu, a.al * (int)((long long)k.split * nb / a.S));
        k.u1 = min(a.nu, a.al * (int)((long long)(k.split + 1) * nb / a.S));
        k.c0 = 4 * kCb3TileCols * (k.u0 >> 2);
        k.cv = k.u0 * kCb3TileCols;
        k.c1 = k.u1 * kCb3TileCols;
        k.xsp = cb3_row_pitch((k.c1 - k.c0) >> 1);
        return k;
    };
    // the wavefront's segment of task k; rows past the matrix (a last, partial row range) stream nothing
    auto segment = [&](const Task &k, Cb3Wave &w) {
        const int rg = k.rbg * RBW + (MODE == kGateUp ? (wave >> 1) : wave);
        const bool rows = rg < a.RB;
        const uint32_t *qt = tb.qs + (size_t)k.e * tb.CT * tb.RT * 256;
        const uint32_t *cbe = tb.cb + (size_t)k.e * tb.G * tb.R * 4;
        w.qb = __builtin_amdgcn_make_buffer_rsrc((void *)qt, (short)0, rows ? 0x7fffffff : 0, kBufferWord3);
        w.qnull = __builtin_amdgcn_make_buffer_rsrc((void *)qt, (short)0, 0, kBufferWord3);
        w.cbb = __builtin_amdgcn_make_buffer_rsrc((void *)cbe, (short)0, rows ? 0x7fffffff : 0, kBufferWord3);
        w.cbnull = __builtin_amdgcn_make_buffer_rsrc((void *)cbe, (short)0, 0, kBufferWord3);
        w.ct_bytes = (uint32_t)tb.RT * 1024u;
        w.rt_bytes = (uint32_t)(rg * RTW) * 1024u;
        w.g_bytes = (uint32_t)tb.R * 16u;
        w.row_bytes = (uint32_t)(rg * 16 * RTW) * 16u;
        w.cta = k.u0;
        w.ctb = k.u1;
        w.g_first = (kCb3TileCols * k.u0) >> 7;
        w.g_last = min((kCb3TileCols * k.u1 - 1) >> 7, tb.G - 1);
        w.lane16 = (uint32_t)lane * 16u;
        w.cblane16 = (uint32_t)(lane & (16 * RTW - 1)) * 16u;
        w.cbl = cbl + wave * 5 * 64;
        int row = pair ? (jt & 7) : jt;
        row = min(row, a.t_rows - 1);
        w.xh = ((pair && jt >= 8) ? xl : xh) + row * k.xsp + 4 * q;
        w.xl = xl + row * k.xsp + 4 * q;
    };
    // the task's slot list, then its activation rows (t < t_rows; rows >= n are zero) straight into LDS
    auto slots_of = [&](const Task &k) {
        if (tid < kMaxT) s_tok[tid] = tid < k.n ? (int)gt.slot[k.gi][tid] : -1;
        __syncthreads();
    };
    auto stage_issue = [&](const Task &k) {
        const int cend = min(k.c1, a.K);
        dma_stage<hilo>(xh, xl, k.xsp, a.t_rows, k.c0, k.cv, k.c1, cend, a.x, a.x_lo, a.K,
                        [&](int r) {
                            const int slot = s_tok[r];
                            return slot < 0 ? -1 : (MODE == kGateUp ? slot_token(slot, a.n_route, a.k) : slot);
                        },
                        wave, lane);
    };
    Task cur = task_of(t);
    Cb3Wave w;
    segment(cur, w);
    cb3_stream<two, RTW>(
        w,
        [&](Cb3Wave &nw) {
            if (t + 1 >= t_end) return false;
            segment(task_of(t + 1), nw);
            return true;
        },
        [&](f32x4 (&acc)[RTW]) {
            const int rg = cur.rbg * RBW + (MODE == kGateUp ? (wave >> 1) : wave);
            if (pair) {
#pragma unroll
                for (int r = 0; r < RTW; ++r)
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[r][i] += __shfl_down(acc[r][i], 8, 16);
            }
            if (rg < a.RB && jt < cur.n) {
                float *dst = a.part + ((size_t)(cur.split * nmat + mat) * a.NS + s_tok[jt]) * a.R + rg * 16 * RTW +
                             4 * q;
#pragma unroll
                for (int r = 0; r < RTW; ++r)
                    *(float4 *)(dst + 16 * r) = make_float4(acc[r][0], acc[r][1], acc[r][2], acc[r][3]);
            }
        },
        [&](const Cb3Wave &) {
            const Task nk = task_of(++t);
            const bool restage = nk.gi != cur.gi || nk.split != cur.split;
            cur = nk;
            if (restage) {
                __syncthreads();          // every wavefront has decoded the previous task's activations
                slots_of(cur);
                stage_issue(cur);
                vm_wait<0>();
                __syncthreads();
            }
        },
        [&]() {
            slots_of(cur);
            stage_issue(cur);
        },
        [&]() {
            vm_wait<4 * RTW + 5>();       // the staging loads, issued ahead of the ring
            lds_barrier();                // ... which stays in flight
        });
}

}  // namespace mi
