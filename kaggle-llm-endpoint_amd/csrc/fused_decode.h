// Fused CB3 MoE decode layer in ONE persistent launch (gfx950), for groups of up to 8 tokens.
//
// The layer (resident.py:110-120) is gate/up -> SwiGLU -> down -> routing-weighted combine.  As separate launches,
// each phase pays its own launch ramp and tail, and the SwiGLU and the combine are latency-bound kernels of their own.
// Here a grid of P resident workgroups works through two ordered task lists:
//
//   phase-1 tasks (group, split, row range): gate and up partials of the group's slots.  The LAST split of a (group,
//     row range) to finish sums the splits in order, applies the clamped SwiGLU (model.py:119-122) and publishes h for
//     those rows as its bf16 high part and bf16 remainder; a per-group counter counts the published row ranges.
//   phase-2 tasks (group, split, row range): the down projection of h (hi and lo in the two halves of the matrix-core
//     tile's columns).  The LAST task to finish a down row range (all groups, all splits) combines it:
//     out[n] = sum_j w[n, j] y_{n,j} (+ the shared expert), splits and experts in a fixed order.
//
// Every wavefront streams its range's segments back to back (cb3_stream): the code ring is refilled from the next
// task's first super tile while the current one finishes, so a workgroup whose range runs from phase 1 into phase 2
// has its down weights in flight before it waits for h (it waits only when it stages a phase-2 task's activations).
//
// Cross-XCD hand-off without fences.  Each XCD has its own L2; agent-scope acquire/release fences write back or
// invalidate a whole L2 and serialise across workgroups (measured ~25 ns each on this part).  Instead:
//   - every value another workgroup reads (partials, h) is stored with the sc1 cache policy (written through to
//     memory) and the storing waves wait for their stores to complete (s_waitcnt vmcnt(0)) before a workgroup
//     barrier, after which one thread bumps a counter with a relaxed agent-scope atomic;
//   - readers spin on the counter (relaxed agent-scope loads, which read memory), then read the data with
//     device-coherent (sc1) loads, which return the stored value even if this XCD's L2 held an older copy of the
//     line; the L2s hold nothing from earlier launches (kernel boundaries write back and invalidate them).
//
// Progress.  Each workgroup takes a contiguous slice of the phase-1 tasks, then a contiguous slice of the phase-2
// tasks.  Phase-2 tasks wait only for phase-1 tasks, which never wait, and every workgroup finishes its phase-1 slice
// before its first wait; the grid is sized to what is resident at once (the runtime's occupancy), so every phase-1
// task is held by a running workgroup that reaches it.
//
// The host zero-fills the counter block (counters and the error word) with a small kernel right before every launch,
// so the workspace needs no initialisation and a launch whose wait gave up leaves no stale count behind; within a
// launch every counter also returns to zero (the last split of a row range, the last consumer of a group's h and the
// combining workgroup reset what they counted).  A wait that exceeds its poll limit (2^20 by default; the host may
// set a smaller one) sets the error word and gives up: the launch then ends with wrong results instead of hanging,
// and the error word stays set until the next call on that workspace.
#pragma once
#include "grouped.h"

namespace mi {

constexpr int kMaxGroups = MI_MAX_SLOTS + kMaxT;   // routed groups (<= routed slots) + shared groups (<= 16)
constexpr int kCtrStride = 32;                     // u32 words between separately contended counters (128 B)
constexpr uint32_t kSpinLimit = 1u << 20;          // polls (~1 s) before a wait gives up (the default)

// All groups of one call, built once per workgroup (same content as find_group's single group).
struct GroupTable {
    int n_groups;
    int n_routed;                       // routed groups; shared groups follow
    int16_t expert[kMaxGroups];
    uint8_t n[kMaxGroups];
    uint8_t slot[kMaxGroups][kMaxT];
};

// Build the table: every distinct valid expert (ascending id) gets ceil(count / cap) groups of its slots in ascending
// slot order; the shared expert gets ceil(N / cap) groups of the slots n_route + n.  `scratch` holds 2 E + n_route
// words.  Called by all threads of the workgroup; ends with a barrier.
__device__ inline void build_group_table(GroupTable &gt, uint32_t *scratch, const int32_t *__restrict__ idx,
                                         int n_route, int E, int shared_expert, int N, int cap) {
    uint32_t *count = scratch, *gbase = scratch + E;
    int *sidx = (int *)(scratch + 2 * E);
    const int tid = threadIdx.x;
    for (int e = tid; e < E; e += blockDim.x) count[e] = 0;
    __syncthreads();
    for (int i = tid; i < n_route; i += blockDim.x) {
        const int e = idx[i];
        sidx[i] = e;
        if (e >= 0 && e < E) atomicAdd(&count[e], 1u);
    }
    __syncthreads();
    if (tid < kWave) {
        const int per = (E + kWave - 1) / kWave;
        const int e0 = tid * per, e1 = min(E, e0 + per);
        int ng = 0;
        for (int e = e0; e < e1; ++e) ng += (int)(count[e] + cap - 1) / cap;
        int incl = ng;
        for (int off = 1; off < kWave; off <<= 1) {
            const int v = __shfl_up(incl, off, kWave);
            if (tid >= off) incl += v;
        }
        int base = incl - ng;
        for (int e = e0; e < e1; ++e) {
            gbase[e] = base;
            base += (int)(count[e] + cap - 1) / cap;
        }
        if (tid == kWave - 1) {
            const int ns = shared_expert >= 0 ? (N + cap - 1) / cap : 0;
            gt.n_routed = incl;
            gt.n_groups = incl + ns;
        }
    }
    __syncthreads();
    for (int i = tid; i < n_route; i += blockDim.x) {
        const int e = sidx[i];
        if (e < 0 || e >= E) continue;
        int rank = 0;
        for (int j = 0; j < i; ++j) rank += sidx[j] == e;
        const int gi = (int)gbase[e] + rank / cap, pos = rank % cap;
        gt.slot[gi][pos] = (uint8_t)i;
        if (pos == 0) {
            gt.expert[gi] = (int16_t)e;
            gt.n[gi] = (uint8_t)min(cap, (int)count[e] - rank);
        }
    }
    if (shared_expert >= 0) {
        const int ns = (N + cap - 1) / cap, base = gt.n_routed;
        for (int q = tid; q < ns * cap; q += blockDim.x) {
            const int r = q / cap, t = q - r * cap;
            if (t == 0) {
                gt.expert[base + r] = (int16_t)shared_expert;
                gt.n[base + r] = (uint8_t)min(cap, N - r * cap);
            }
            if (r * cap + t < N) gt.slot[base + r][t] = (uint8_t)(n_route + r * cap + t);
        }
    }
    __syncthreads();
}

struct FArgs {
    Cb3Table gate, up, down;
    int D, I, E, N, k, n_route, shared_expert, NS, t_rows;
    float limit;
    const uint16_t *x;
    const int32_t *idx;
    const float *w;
    float *part1;                  // [S1][2][NS][I]
    uint16_t *h_hi, *h_lo;         // [NS][I]: h = hi + lo (bf16 high part and remainder)
    float *part2;                  // [S2][NS][D]
    float *out_f32;
    uint16_t *out_bf16;
    uint32_t *hcnt;                // [kMaxGroups] x kCtrStride: published h row ranges (+ consumers, for the reset)
    uint32_t *cnt2;                // [RBG2] x kCtrStride: finished down tasks per row range
    uint32_t *cnt1;                // [kMaxGroups * RBG1]: finished gate/up splits per (group, row range)
    uint32_t *err;                 // nonzero: a wait gave up
    uint32_t spin_limit;           // polls before a wait gives up
    int S1, al1, nu1, RB1, RBG1;
    int S2, al2, nu2, RB2, RBG2;
    int xs_max;                    // LDS row pitch (dwords) of the larger staging
    int P;                         // workgroups of the launch
};

__device__ __forceinline__ uint32_t ld_agent(const uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint32_t *p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t add_agent(uint32_t *p, uint32_t v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Every wave: wait until its own stores (and everything else) have completed; then the workgroup barrier.
__device__ __forceinline__ void stores_done_barrier() {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
}

// 8-byte store with the sc1 cache policy (see wt_store4).
__device__ __forceinline__ void wt_store2(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint2 v) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), r, (int)voff, 0, kCachePolicySc1);
}

// Routing-weighted combine of down rows [r0, r0 + nr) for every token (the combine kernel's order: experts in routing
// order, splits in order, the shared expert last).  Per split, every contributing slot's partial is loaded before the
// first add (the loads are independent), so the combine costs one round trip per split, not per expert.
constexpr int kCombineSlots = 3;     // slots per token handled per pass (few registers: the next task's ring is live)
__device__ __forceinline__ void combine_rows(const FArgs &a, int r0, int nr) {
    const int nr4 = nr >> 2;
    const __amdgpu_buffer_rsrc_t rp =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.part2, (short)0, 0x7fffffff, kBufferWord3);
    for (int i = threadIdx.x; i < a.N * nr4; i += blockDim.x) {
        const int tok = i / nr4, r = r0 + 4 * (i - tok * nr4);
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        const int nj = a.k + (a.shared_expert >= 0 ? 1 : 0);
        for (int j0 = 0; j0 < nj; j0 += kCombineSlots) {
            int slot[kCombineSlots];
            float wt[kCombineSlots];
#pragma unroll
            for (int jj = 0; jj < kCombineSlots; ++jj) {
                const int j = j0 + jj;
                slot[jj] = -1;
                wt[jj] = 0.f;
                if (j < a.k) {
                    const int e = a.idx[tok * a.k + j];
                    if (e >= 0 && e < a.E) {
                        slot[jj] = tok * a.k + j;
                        wt[jj] = a.w[tok * a.k + j];
                    }
                } else if (j < nj) {
                    slot[jj] = a.n_route + tok;
                    wt[jj] = 1.0f;
                }
            }
            float4 ys[kCombineSlots];
#pragma unroll
            for (int jj = 0; jj < kCombineSlots; ++jj) ys[jj] = make_float4(0.f, 0.f, 0.f, 0.f);
            for (int s = 0; s < a.S2; ++s) {
                float4 p[kCombineSlots];
#pragma unroll
                for (int jj = 0; jj < kCombineSlots; ++jj)
                    if (slot[jj] >= 0) {
                        const f32x4 v = coherent_load4(rp, (uint32_t)((((size_t)s * a.NS + slot[jj]) * a.D + r) * 4));
                        p[jj] = make_float4(v[0], v[1], v[2], v[3]);
                    } else {
                        p[jj] = make_float4(0.f, 0.f, 0.f, 0.f);
                    }
#pragma unroll
                for (int jj = 0; jj < kCombineSlots; ++jj) {
                    ys[jj].x += p[jj].x; ys[jj].y += p[jj].y; ys[jj].z += p[jj].z; ys[jj].w += p[jj].w;
                }
            }
#pragma unroll
            for (int jj = 0; jj < kCombineSlots; ++jj) {
                if (slot[jj] < 0) continue;
                if (j0 + jj < a.k) {
                    acc.x += wt[jj] * ys[jj].x; acc.y += wt[jj] * ys[jj].y;
                    acc.z += wt[jj] * ys[jj].z; acc.w += wt[jj] * ys[jj].w;
                } else {
                    acc.x += ys[jj].x; acc.y += ys[jj].y; acc.z += ys[jj].z; acc.w += ys[jj].w;
                }
            }
        }
        if (a.out_f32) *(float4 *)(a.out_f32 + (size_t)tok * a.D + r) = acc;
        if (a.out_bf16) {
            uint2 b;
            b.x = f32_to_bf16_rne(acc.x) | (f32_to_bf16_rne(acc.y) << 16);
            b.y = f32_to_bf16_rne(acc.z) | (f32_to_bf16_rne(acc.w) << 16);
            *(uint2 *)(a.out_bf16 + (size_t)tok * a.D + r) = b;
        }
    }
}

// Tokens of a group's matrix-core tile: at most 8 (phase 2 puts h's remainder in the tile's other 8 columns).
constexpr int kFusedMaxTokens = 8;

template <int RTW>
__global__ void __launch_bounds__(64 * kWgWaves, MI_CB3_WAVES) fused_decode_kernel(FArgs a) {
    static_assert(RTW >= 2, "h row ranges must cover whole 128-byte lines of the bf16 planes");
    extern __shared__ uint32_t xlds[];
    __shared__ GroupTable gt;
    __shared__ uint4 cbl[kWgWaves * 5 * 64];
    __shared__ int s_tok[kMaxT];
    __shared__ int s_flag;
    constexpr int WR = 16 * RTW;                   // rows per wavefront
    const int tid = threadIdx.x, lane = tid & 63, jt = lane & 15, q = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    build_group_table(gt, xlds, a.idx, a.n_route, a.E, a.shared_expert, a.N, a.t_rows);
    const int n_groups = __builtin_amdgcn_readfirstlane(gt.n_groups);
    if (n_groups == 0) {               // nothing routed and no shared expert: the layer's output is zero
        if (blockIdx.x == 0)
            for (int i = tid; i < a.N * a.D; i += blockDim.x) {
                if (a.out_f32) a.out_f32[i] = 0.f;
                if (a.out_bf16) a.out_bf16[i] = 0;
            }
        return;
    }
    const int per1 = a.S1 * a.RBG1, per2 = a.S2 * a.RBG2;
    const int T1 = n_groups * per1, T2 = n_groups * per2;
    // this workgroup's tasks: a contiguous slice of the phase-1 list, then a contiguous slice of the phase-2 list
    // (every workgroup streams gate/up first, then has its down weights in flight while the last h rows form)
    const long long b = blockIdx.x;
    const int t1a = (int)(b * T1 / a.P), t1b = (int)((b + 1) * T1 / a.P);
    const int t2a = T1 + (int)(b * T2 / a.P), t2b = T1 + (int)((b + 1) * T2 / a.P);
    int t = 0, t_end = 0;
    uint32_t *xh = xlds;
    uint32_t *xl = xlds + (size_t)a.t_rows * a.xs_max;

    // task t: phase 1 (t < T1) or 2; (group gi, split, row range rbg), row range fastest
    struct Task {
        int ph2, gi, split, rbg, e, n, u0, u1, c0, cv, c1, xsp;
    };
    auto task_of = [&](int tt) {
        Task k;
        k.ph2 = tt >= T1;
        const int u = k.ph2 ? tt - T1 : tt;
        const int RBG = k.ph2 ? a.RBG2 : a.RBG1, S = k.ph2 ? a.S2 : a.S1;
        const int nu = k.ph2 ? a.nu2 : a.nu1, al = k.ph2 ? a.al2 : a.al1;
        k.rbg = u % RBG;
        const int gs = u / RBG;
        k.split = gs % S;
        k.gi = gs / S;
        k.e = __builtin_amdgcn_readfirstlane(gt.expert[k.gi]);
        k.n = __builtin_amdgcn_readfirstlane(gt.n[k.gi]);
        const int nb = (nu + al - 1) / al;
        k.u0 = min(nu, al * (int)((long long)k.split * nb / S));
        k.u1 = min(nu, al * (int)((long long)(k.split + 1) * nb / S));
        k.c0 = 4 * kCb3TileCols * (k.u0 >> 2);
        k.cv = k.u0 * kCb3TileCols;
        k.c1 = k.u1 * kCb3TileCols;
        k.xsp = cb3_row_pitch((k.c1 - k.c0) >> 1);
        return k;
    };
    // the wavefront's row group and matrix in task k
    auto wave_rows = [&](const Task &k, int &rg, int &mat) {
        mat = k.ph2 ? 0 : (wave & 1);
        rg = k.ph2 ? k.rbg * kWgWaves + wave : k.rbg * 2 + (wave >> 1);
    };
    auto segment = [&](const Task &k, Cb3Wave &w) {
        int rg, mat;
        wave_rows(k, rg, mat);
        const Cb3Table &tb = k.ph2 ? a.down : (mat ? a.up : a.gate);
        const bool rows = rg < (k.ph2 ? a.RB2 : a.RB1);
        const uint32_t *qt = tb.qs + (size_t)k.e * tb.CT * tb.RT * 256;
        const uint32_t *cbe = tb.cb + (size_t)k.e * tb.G * tb.R * 4;
        w.qb = __builtin_amdgcn_make_buffer_rsrc((void *)qt, (short)0, rows ? 0x7fffffff : 0, kBufferWord3);
        w.qnull = __builtin_amdgcn_make_buffer_rsrc((void *)qt, (short)0, 0, kBufferWord3);
        w.cbb = __builtin_amdgcn_make_buffer_rsrc((void *)cbe, (short)0, rows ? 0x7fffffff : 0, kBufferWord3);
        w.cbnull = __builtin_amdgcn_make_buffer_rsrc((void *)cbe, (short)0, 0, kBufferWord3);
        w.ct_bytes = (uint32_t)tb.RT * 1024u;
        w.rt_bytes = (uint32_t)(rg * RTW) * 1024u;
        w.g_bytes = (uint32_t)tb.R * 16u;
        w.row_bytes = (uint32_t)(rg * WR) * 16u;
        w.cta = k.u0;
        w.ctb = k.u1;
        w.g_first = (kCb3TileCols * k.u0) >> 7;
        w.g_last = min((kCb3TileCols * k.u1 - 1) >> 7, tb.G - 1);
        w.lane16 = (uint32_t)lane * 16u;
        w.cblane16 = (uint32_t)(lane & (WR - 1)) * 16u;
        w.cbl = cbl + wave * 5 * 64;
        // phase 2: columns 0-7 of the tile carry h's high part, 8-15 its remainder (one instruction covers both)
        const int row = min(k.ph2 ? (jt & 7) : jt, a.t_rows - 1);
        w.xh = ((k.ph2 && jt >= 8) ? xl : xh) + row * k.xsp + 4 * q;
        w.xl = w.xh;
    };
    // a phase-2 task may start once its group's h is published: count it as a consumer (the last consumer resets
    // the counter); `wait` when this workgroup has not yet seen the group's h published
    auto consume_h = [&](const Task &k, bool wait) {
        if (tid == 0) {
            uint32_t *c = a.hcnt + k.gi * kCtrStride;
            if (wait) {
                uint32_t spins = 0;
                while (ld_agent(c) < (uint32_t)a.RBG1) {
                    __builtin_amdgcn_s_sleep(2);
                    if (++spins > a.spin_limit) {
                        st_agent(a.err, 1u);
                        break;
                    }
                }
            }
            if (add_agent(c, 1u) == (uint32_t)(a.RBG1 + per2 - 1)) st_agent(c, 0u);
        }
    };
    // activation rows r < t_rows (rows >= n are zero) of the task's staged columns: x (phase 1) or h's two parts
    auto stage_rows = [&](const Task &k) {
        if (tid < kMaxT) s_tok[tid] = tid < k.n ? (int)gt.slot[k.gi][tid] : -1;
        __syncthreads();
        const int xs = (k.c1 - k.c0) >> 1, q4 = xs >> 1;
        const int K = k.ph2 ? a.I : a.D;
        const int cend = min(k.c1, K);
        const __amdgpu_buffer_rsrc_t rh =
            __builtin_amdgcn_make_buffer_rsrc((void *)a.h_hi, (short)0, 0x7fffffff, kBufferWord3);
        const __amdgpu_buffer_rsrc_t rl =
            __builtin_amdgcn_make_buffer_rsrc((void *)a.h_lo, (short)0, 0x7fffffff, kBufferWord3);
        for (int i = tid; i < a.t_rows * q4; i += blockDim.x) {
            const int r = i / q4, qq = i - r * q4;
            const int slot = s_tok[r];
            const int c = k.c0 + 4 * qq;
            uint2 hv = make_uint2(0, 0), lv = make_uint2(0, 0);
            if (slot >= 0 && c >= k.cv && c < cend) {
                if (k.ph2) {           // h of other workgroups, published by the group's counter
                    const uint32_t off = (uint32_t)((size_t)slot * a.I + c) * 2u;
                    hv = coherent_load2(rh, off);
                    lv = coherent_load2(rl, off);
                } else {
                    hv = *(const uint2 *)(a.x + (size_t)slot_token(slot, a.n_route, a.k) * a.D + c);
                }
            }
            *(uint2 *)(xh + r * k.xsp + 2 * qq) = hv;
            if (k.ph2) *(uint2 *)(xl + r * k.xsp + 2 * qq) = lv;
        }
        __syncthreads();
    };
    // end of a phase-1 task's row range: the last of its S1 splits forms h for those rows
    auto finish_h = [&](const Task &k) {
        const int r0 = k.rbg * 2 * WR;
        const int nr4 = min(2 * WR, a.I - r0) >> 2;
        const __amdgpu_buffer_rsrc_t hh =
            __builtin_amdgcn_make_buffer_rsrc((void *)a.h_hi, (short)0, 0x7fffffff, kBufferWord3);
        const __amdgpu_buffer_rsrc_t hl =
            __builtin_amdgcn_make_buffer_rsrc((void *)a.h_lo, (short)0, 0x7fffffff, kBufferWord3);
        const __amdgpu_buffer_rsrc_t rp =
            __builtin_amdgcn_make_buffer_rsrc((void *)a.part1, (short)0, 0x7fffffff, kBufferWord3);
        for (int i = tid; i < k.n * nr4; i += blockDim.x) {
            const int r_ = i / nr4, r = r0 + 4 * (i - r_ * nr4);
            const int slot = s_tok[r_];
            f32x4 g = (f32x4){0.f, 0.f, 0.f, 0.f}, u = g;
            for (int s = 0; s < a.S1; ++s) {
                g += coherent_load4(rp, (uint32_t)((((size_t)(2 * s) * a.NS + slot) * a.I + r) * 4));
                u += coherent_load4(rp, (uint32_t)((((size_t)(2 * s + 1) * a.NS + slot) * a.I + r) * 4));
            }
            const float hv[4] = {swiglu_clamped(g[0], u[0], a.limit), swiglu_clamped(g[1], u[1], a.limit),
                                 swiglu_clamped(g[2], u[2], a.limit), swiglu_clamped(g[3], u[3], a.limit)};
            uint32_t hi[4], lo[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) split_bf16(hv[j], hi[j], lo[j]);
            const uint32_t off = (uint32_t)((size_t)slot * a.I + r) * 2u;
            wt_store2(hh, off, make_uint2(hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16)));
            wt_store2(hl, off, make_uint2(lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16)));
        }
        stores_done_barrier();
        if (tid == 0) add_agent(a.hcnt + k.gi * kCtrStride, 1u);
    };

    // the two slices are two streams: a workgroup's down weights are requested only after its last gate/up task has
    // finished (a last split's h rows are formed from loads that would otherwise queue behind them)
    for (int ph = 0; ph < 2; ++ph) {
    t = ph ? t2a : t1a;
    t_end = ph ? t2b : t1b;
    if (t >= t_end) continue;
    Task cur = task_of(t);
    Cb3Wave w;
    segment(cur, w);
    cb3_stream<false, RTW>(
        w,
        [&](Cb3Wave &nw) {
            if (t + 1 >= t_end) return false;
            segment(task_of(t + 1), nw);
            return true;
        },
        [&](f32x4 (&acc)[RTW]) {
            int rg, mat;
            wave_rows(cur, rg, mat);
            if (cur.ph2) {
#pragma unroll
                for (int r = 0; r < RTW; ++r)
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[r][i] += __shfl_down(acc[r][i], 8, 16);
            }
            if (rg < (cur.ph2 ? a.RB2 : a.RB1) && jt < cur.n) {
                const int R = cur.ph2 ? a.D : a.I;
                float *base = cur.ph2 ? a.part2 + (size_t)cur.split * a.NS * a.D
                                      : a.part1 + (size_t)(cur.split * 2 + mat) * a.NS * a.I;
                const __amdgpu_buffer_rsrc_t pr =
                    __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, 0x7fffffff, kBufferWord3);
                const size_t off = (size_t)s_tok[jt] * R + rg * WR + 4 * q;
#pragma unroll
                for (int r = 0; r < RTW; ++r) wt_store4(pr, (uint32_t)(off + 16 * r) * 4u, acc[r]);
            }
            stores_done_barrier();
            if (tid == 0) {
                int last;
                if (!cur.ph2) {
                    last = 1;
                    if (a.S1 > 1) {
                        uint32_t *c = a.cnt1 + cur.gi * a.RBG1 + cur.rbg;
                        last = add_agent(c, 1u) == (uint32_t)a.S1 - 1;
                        if (last) st_agent(c, 0u);
                    }
                } else {
                    uint32_t *c = a.cnt2 + cur.rbg * kCtrStride;
                    last = add_agent(c, 1u) == (uint32_t)(n_groups * a.S2 - 1);
                    if (last) st_agent(c, 0u);
                }
                s_flag = last;
            }
            __syncthreads();
            if (s_flag) {
                if (!cur.ph2) {
                    finish_h(cur);
                } else {
                    const int r0 = cur.rbg * kWgWaves * WR;
                    combine_rows(a, r0, min(kWgWaves * WR, a.D - r0));
                }
            }
        },
        [&](const Cb3Wave &) {
            const Task nk = task_of(++t);
            const bool restage = nk.ph2 != cur.ph2 || nk.gi != cur.gi || nk.split != cur.split;
            const bool new_group = nk.ph2 && (!cur.ph2 || nk.gi != cur.gi);
            cur = nk;
            if (cur.ph2) consume_h(cur, new_group);
            if (restage) {
                __syncthreads();          // every wavefront has decoded the previous task's activations
                stage_rows(cur);
            }
        },
        [&]() {
            // phase 1: x rows straight into LDS ahead of the ring; phase 2 stages h once it is published
            if (!cur.ph2) {
                if (tid < kMaxT) s_tok[tid] = tid < cur.n ? (int)gt.slot[cur.gi][tid] : -1;
                __syncthreads();
                dma_stage<false>(xh, xl, cur.xsp, a.t_rows, cur.c0, cur.cv, cur.c1, min(cur.c1, a.D), a.x, a.x, a.D,
                                 [&](int r) {
                                     const int slot = s_tok[r];
                                     return slot < 0 ? -1 : slot_token(slot, a.n_route, a.k);
                                 },
                                 wave, lane);
            }
        },
        [&]() {
            if (cur.ph2) {
                consume_h(cur, true);
                stage_rows(cur);
            } else {
                vm_wait<4 * RTW + 5>();   // the staging loads, issued ahead of the ring
                lds_barrier();            // ... which stays in flight
            }
        });
    __syncthreads();              // the next stream restages the activation rows
    }
}

}  // namespace mi
