// CU-balanced CB3 streams for single-token decode (gate/up partials, down partials) on gfx950.
//
// Measured on MI355X: a CU serves the vector memory requests of its resident workgroups roughly oldest first, so
// when a launch puts 4 or 5 one-task workgroups on a CU the youngest gets its first tile 15-20 us after the oldest,
// and CUs holding one workgroup more than others finish last.  At one token the layer's weight stream is short
// (~20 us at the HBM ceiling), so that imbalance, not the stream itself, set the launch time.
//
// Here the grid is one workgroup per CU (the launch holds exactly as many workgroups as the device has CUs, and the
// workgroup's LDS keeps a second one off the CU), and the ordered list of work units -- (group, matrix, column split,
// 16 RTW-row tile) -- is cut into equal contiguous shares, one per workgroup: every CU streams the same bytes.  Inside
// the workgroup, every wavefront claims its next unit from an LDS counter when it starts its current unit's last
// super tile (cb3_stream refills the ring from the claimed unit while the current one finishes), so a wavefront that
// the CU serves later simply takes fewer units and the workgroup ends within about one unit of its share.
//
// With one token a group is one slot (its expert read straight from the routing ids: no grouping pass before the
// first weight request), every group of the gate/up launch multiplies the same activation row, and the down launch
// stages the h rows (bf16 high part and remainder) of the groups its share touches; the rows go to LDS with
// direct-to-LDS loads issued ahead of the weight ring.  Each unit writes its own f32 partial rows (the next launch
// reduces them in a fixed order), so no workgroup waits on another.
//
// The down launch can also do the routing-weighted combine itself (no combine launch): when a workgroup has streamed
// its share, its partials stored through to memory, it counts each of its units on the unit's 16 RTW-row tile (one
// agent-scope counter per tile, each on its own 128-byte line); the workgroup whose count completes a tile (slots x
// splits units) sums that tile's partials with device-coherent loads in the combine launch's order (combine4) and
// writes the output rows, then resets the counter.  Nothing waits for another workgroup, and the result is
// bit-identical to the combine launch's.
#pragma once
#include <type_traits>

#include "fused_decode.h"

namespace mi {

struct CArgs {
    Cb3Table t0, t1;           // gate, up (kGateUp) or down (t0 only)
    int R, K;                  // rows, cols of the table(s)
    int E, n_route, N, k, shared_expert, NS;
    int S, al, nu;             // column splits: boundaries at multiples of `al` column tiles over nu tiles
    int RT;                    // 16 RTW-row tiles per matrix
    int U;                     // units: groups * nmat * S * RT (upper bound; units past the call's groups are empty)
    int P;                     // workgroups (= CUs)
    int gmax;                  // kDown: most groups any workgroup's share touches (staged rows)
    int xsp;                   // LDS row pitch (dwords) of a staged row
    const uint16_t *x;         // kGateUp: x bf16 [1, K]; kDown: bf16 high part of h [NS, K]
    const uint16_t *x_lo;      // kDown: bf16 remainder of h [NS, K]
    // kDown: h formed while staging from the gate/up split partials [gu_S][2][NS][K] instead of read from x / x_lo
    // (the splits summed in order, the clamped SwiGLU, bf16 high part + remainder: the SwiGLU launch's arithmetic);
    // gmax * (columns / 4) <= 4 * 768 (the host checks it)
    const float *gu_part;
    int gu_S;
    float limit;
    const int32_t *idx;
    float *part;               // [S][nmat][NS][R]
    // kDown with the combine in the launch (rt_ctr not null): routing weights [k], one counter per 16 RTW-row tile
    // (zero between launches; words 32 rt), the outputs [R] (either may be null)
    const float *w;
    uint32_t *rt_ctr;
    float *out_f32;
    uint16_t *out_bf16;
};

// Row tiles one workgroup's down share can complete (the host keeps the share within this many units).
constexpr int kCuMaxLast = 64;
constexpr int kRtCtrStride = 32;         // words between row-tile counters (one 128-byte line each)

// out = routing-weighted sum of a row quad's down partials: slots in routing order (an id outside [0, E) adds
// nothing), splits in order, the shared expert last -- the combine launch's arithmetic (combine_kernel).  Per chunk
// of 9 slots and split, every partial is loaded before the first add: one round trip per (chunk, split).
constexpr int kCuCombineChunk = 9;
__device__ __forceinline__ float4 cu_combine4(const CArgs &a, const int *s_exp, __amdgpu_buffer_rsrc_t rp, int r) {
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    const int nj = a.k + (a.shared_expert >= 0 ? 1 : 0);
    for (int j0 = 0; j0 < nj; j0 += kCuCombineChunk) {
        bool on[kCuCombineChunk];
        float wt[kCuCombineChunk];
        float4 ys[kCuCombineChunk];
#pragma unroll
        for (int jj = 0; jj < kCuCombineChunk; ++jj) {
            const int j = j0 + jj;
            on[jj] = j < nj && (j >= a.k || (s_exp[j] >= 0 && s_exp[j] < a.E));
            wt[jj] = on[jj] && j < a.k ? a.w[j] : 1.0f;
            ys[jj] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        for (int s = 0; s < a.S; ++s) {
            f32x4 p[kCuCombineChunk];
#pragma unroll
            for (int jj = 0; jj < kCuCombineChunk; ++jj)
                p[jj] = on[jj] ? coherent_load4(rp, (uint32_t)((((size_t)s * a.NS + j0 + jj) * a.R + r) * 4))
                               : (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int jj = 0; jj < kCuCombineChunk; ++jj) {
                ys[jj].x += p[jj][0]; ys[jj].y += p[jj][1]; ys[jj].z += p[jj][2]; ys[jj].w += p[jj][3];
            }
        }
#pragma unroll
        for (int jj = 0; jj < kCuCombineChunk; ++jj) {
            if (!on[jj]) continue;
            if (j0 + jj < a.k) {
                acc.x = fmaf(wt[jj], ys[jj].x, acc.x); acc.y = fmaf(wt[jj], ys[jj].y, acc.y);
                acc.z = fmaf(wt[jj], ys[jj].z, acc.z); acc.w = fmaf(wt[jj], ys[jj].w, acc.w);
            } else {
                acc.x += ys[jj].x; acc.y += ys[jj].y; acc.z += ys[jj].z; acc.w += ys[jj].w;
            }
        }
    }
    return acc;
}

#ifndef MI_CU_WAVES
#define MI_CU_WAVES 12
#endif
constexpr int kCuWaves = MI_CU_WAVES;   // wavefronts per workgroup (3 per SIMD): gate/up, and the multi-token launches
// The single-token down launch: 16 wavefronts (4 per SIMD, within 128 registers).  Its share is ~13.5 units of 16
// rows, so with 12 wavefronts some stream two units back to back and set the workgroup's end; with 16 each streams
// at most one.  Measured: layer 47.8-47.9 against 48.2-48.5 µs (seven alternations on two boxes).
constexpr int kCuDownWaves = 16;
template <int MODE>
__host__ __device__ constexpr int cu_waves() { return MODE == kDown ? kCuDownWaves : kCuWaves; }
// h formation in the down launch: each thread forms at most kCuFormIt quads of 4 columns (two keep the launch within
// 128 registers), so a workgroup forms up to kCuFormIt * 64 * kCuDownWaves quads (the host checks it)
constexpr int kCuFormIt = 2;

template <int MODE, int RTW>
__global__ void __launch_bounds__(64 * cu_waves<MODE>(), 1) custream_kernel(CArgs a) {
    // staged rows, then the wavefronts' codebook slots, all read with 16-byte LDS loads: the dynamic segment must
    // start 16-byte aligned (at an 8-byte-aligned start this launch measured 2.8x slower)
    extern __shared__ __attribute__((aligned(16))) uint32_t xlds[];
    __shared__ uint32_t s_next, s_nlast;
    __shared__ int s_exp[MI_MAX_SLOTS + 1];         // expert of every slot (group)
    __shared__ int s_last[MODE == kDown ? kCuMaxLast : 1];     // row tiles this workgroup combines
    constexpr bool hilo = MODE == kDown;            // h: hi in columns 0-7 of the tile, lo in 8-15
    constexpr int nmat = MODE == kGateUp ? 2 : 1;
    constexpr int kWaves = cu_waves<MODE>();
    const int tid = threadIdx.x, lane = tid & 63, jt = lane & 15, q = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    // one token: group gi is slot gi (the k routed slots, then the shared expert's, whose slot is k); a slot with an
    // expert id outside [0, E) has empty units (the combine leaves it out)
    const int n_groups = a.NS;
    const int per_g = nmat * a.S * a.RT;
    const int U = n_groups * per_g;
    const int u_begin = (int)((long long)blockIdx.x * U / a.P);
    const int u_end = (int)((long long)(blockIdx.x + 1) * U / a.P);
    if (u_begin >= u_end) return;
    const bool combine = hilo && a.rt_ctr != nullptr;      // uniform over the launch
    const int g0 = u_begin / per_g;
    const int ng = hilo ? min(a.gmax, n_groups - g0) : 1;
    const int rows = hilo ? 2 * ng : 1;             // gate/up: the token's x row; down: hi and lo of each group's h
    uint4 *cbl = (uint4 *)(xlds + (size_t)rows * a.xsp);    // 16-byte aligned: the pitch is a multiple of 4 dwords
    if (tid == 0) {
        s_next = (uint32_t)u_begin + kWaves;      // the first kWaves units are taken without a claim
        s_nlast = 0;
    }

    // unit u = (group gi, matrix, split, row tile), row tile fastest
    struct Unit {
        int gi, mat, split, rt, e;
    };
    // from_lds: the expert from s_exp (after the staging barrier), else from the routing ids (the first unit only)
    auto unit_of = [&](int u, auto from_lds) {
        Unit k;
        k.rt = u % a.RT;
        int r = u / a.RT;
        k.split = r % a.S;
        r /= a.S;
        k.mat = r % nmat;
        k.gi = r / nmat;
        int e;
        if constexpr (decltype(from_lds)::value) e = s_exp[k.gi];
        else e = k.gi < a.n_route ? a.idx[k.gi] : a.shared_expert;
        k.e = __builtin_amdgcn_readfirstlane(e);
        return k;
    };
    using Lds = std::true_type;
    using Glb = std::false_type;
    auto segment = [&](const Unit &k, Cb3Wave &w) {
        const Cb3Table &tb = k.mat ? a.t1 : a.t0;
        const bool ok = k.e >= 0 && k.e < a.E;
        const uint32_t *qt = tb.qs + (size_t)(ok ? k.e : 0) * tb.CT * tb.RT * 256;
        const uint32_t *cbe = tb.cb + (size_t)(ok ? k.e : 0) * tb.G * tb.R * 4;
        w.qb = __builtin_amdgcn_make_buffer_rsrc((void *)qt, (short)0, ok ? 0x7fffffff : 0, kBufferWord3);
        w.qnull = __builtin_amdgcn_make_buffer_rsrc((void *)qt, (short)0, 0, kBufferWord3);
        w.cbb = __builtin_amdgcn_make_buffer_rsrc((void *)cbe, (short)0, ok ? 0x7fffffff : 0, kBufferWord3);
        w.cbnull = __builtin_amdgcn_make_buffer_rsrc((void *)cbe, (short)0, 0, kBufferWord3);
        const int nb = (a.nu + a.al - 1) / a.al;
        w.cta = min(a.nu, a.al * (int)((long long)k.split * nb / a.S));
        w.ctb = min(a.nu, a.al * (int)((long long)(k.split + 1) * nb / a.S));
        w.ct_bytes = (uint32_t)tb.RT * 1024u;
        w.rt_bytes = (uint32_t)(k.rt * RTW) * 1024u;
        w.g_bytes = (uint32_t)tb.R * 16u;
        w.row_bytes = (uint32_t)(k.rt * 16 * RTW) * 16u;
        w.g_first = (kCb3TileCols * w.cta) >> 7;
        w.g_last = min((kCb3TileCols * w.ctb - 1) >> 7, tb.G - 1);
        w.lane16 = (uint32_t)lane * 16u;
        w.cblane16 = (uint32_t)(lane & (16 * RTW - 1)) * 16u;
        w.cbl = cbl + wave * 5 * 64;
        // B operand: the staged row (down: hi in columns 0-7, lo in 8-15 of the group's two rows), from the column
        // of the super tile holding cta
        const int row = hilo ? 2 * (k.gi - g0) + (jt >= 8 ? 1 : 0) : 0;
        w.xh = xlds + row * a.xsp + 320 * (w.cta >> 2) + 4 * q;
        w.xl = w.xh;
    };
    // h rows of the share's groups from the gate/up partials.  The first pair of splits' partial loads are issued
    // ahead of the wavefront's weight ring (issue): they come from the last-level cache while the ring's first tiles
    // come from HBM, so h is formed before those land (issued behind the ring, the formation waited for them: the
    // staging barrier came ~7 us into the launch)
    constexpr int kFormIt = kCuFormIt;
    float4 fg[kFormIt][2], fu[kFormIt][2];          // a pair of splits' gate / up partials, at most kFormIt quads
    const int fq4 = (a.nu * kCb3TileCols) >> 2;     // quads of 4 columns per staged row
    // buffer loads whose offset leaves the range where no partial is needed (they return zeros): no branch around
    // a load, so the compiler never drains the loads in flight at a join (the partials are < 2 GB)
    auto form_load = [&](int sp0) {
        const __amdgpu_buffer_rsrc_t rgu =
            __builtin_amdgcn_make_buffer_rsrc((void *)a.gu_part, (short)0, 0x7fffffff, kBufferWord3);
        const uint32_t plane = (uint32_t)(a.NS * a.K);
#pragma unroll
        for (int it = 0; it < kFormIt; ++it) {
            const int i = tid + it * (int)blockDim.x, j = i / fq4, c = 4 * (i - j * fq4);
            const bool in = i < ng * fq4 && c < a.K;
            const uint32_t o = (uint32_t)((g0 + j) * a.K + c);          // slot g0 + j (one token)
#pragma unroll
            for (int d = 0; d < 2; ++d) {
                const int sp = sp0 + d;
                const bool ld = in && sp < a.gu_S;
                const uint32_t og = ld ? 4u * ((uint32_t)(2 * sp) * plane + o) : kStageOut;
                const uint32_t ou = ld ? 4u * ((uint32_t)(2 * sp + 1) * plane + o) : kStageOut;
                fg[it][d] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rgu, (int)og, 0, 0));
                fu[it][d] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rgu, (int)ou, 0, 0));
            }
        }
    };
    // h = SwiGLU of the summed partials, as bf16 high part + remainder, into the staged rows
    auto form_write = [&](const float4 (&g)[kFormIt], const float4 (&uu)[kFormIt]) {
#pragma unroll
        for (int it = 0; it < kFormIt; ++it) {
            const int i = tid + it * (int)blockDim.x, j = i / fq4, c = 4 * (i - j * fq4);
            if (i >= ng * fq4) break;
            uint2 hv = make_uint2(0, 0), lv = make_uint2(0, 0);
            if (c < a.K) {
                uint32_t h0, l0, h1, l1, h2, l2, h3, l3;
                split_bf16(swiglu_clamped(g[it].x, uu[it].x, a.limit), h0, l0);
                split_bf16(swiglu_clamped(g[it].y, uu[it].y, a.limit), h1, l1);
                split_bf16(swiglu_clamped(g[it].z, uu[it].z, a.limit), h2, l2);
                split_bf16(swiglu_clamped(g[it].w, uu[it].w, a.limit), h3, l3);
                hv = make_uint2(h0 | (h1 << 16), h2 | (h3 << 16));
                lv = make_uint2(l0 | (l1 << 16), l2 | (l3 << 16));
            }
            *(uint2 *)(xlds + (2 * j) * a.xsp + (c >> 1)) = hv;
            *(uint2 *)(xlds + (2 * j + 1) * a.xsp + (c >> 1)) = lv;
        }
    };
    // the adds of a loaded pair of splits, in split order (sp0 + d < gu_S)
    auto form_add = [&](int sp0, float4 (&g)[kFormIt], float4 (&uu)[kFormIt]) {
#pragma unroll
        for (int it = 0; it < kFormIt; ++it)
#pragma unroll
            for (int d = 0; d < 2; ++d) {
                if (sp0 + d >= a.gu_S) break;
                g[it].x += fg[it][d].x; g[it].y += fg[it][d].y; g[it].z += fg[it][d].z; g[it].w += fg[it][d].w;
                uu[it].x += fu[it][d].x; uu[it].y += fu[it][d].y; uu[it].z += fu[it][d].z; uu[it].w += fu[it][d].w;
            }
    };
    // the splits summed in order from zero, as the SwiGLU launch sums them.  Up to 2 splits (the default) the pair
    // loaded by issue is all there is: straight-line code, so the only loads it waits for are those partials, not
    // the weight ring behind them.  More splits load each later pair here (a round trip each, behind the ring).
    auto form_finish = [&]() {
        float4 g[kFormIt], uu[kFormIt];
#pragma unroll
        for (int it = 0; it < kFormIt; ++it) g[it] = uu[it] = make_float4(0.f, 0.f, 0.f, 0.f);
        form_add(0, g, uu);
        if (a.gu_S > 2) {
            for (int sp0 = 2; sp0 < a.gu_S; sp0 += 2) {
                form_load(sp0);
                form_add(sp0, g, uu);
            }
            form_write(g, uu);
            vm_wait<0>();
        } else {
            form_write(g, uu);
        }
    };
    // staged rows straight into LDS, spread over the wavefronts, issued ahead of every wavefront's weight ring:
    // columns past K read zeros.  Whole 256-dword chunks of a row load 16 bytes per lane, the rest 4: an LDS-bound
    // load costs about as much per instruction whatever its width (a one-token down launch that loaded 64 KB of
    // partials this way per workgroup took 7.4 us longer with 4-byte lanes, 1.7 with 16-byte lanes).
    const bool form_h = hilo && a.gu_part != nullptr;
    auto issue = [&]() {
        const int xs = (a.nu * kCb3TileCols) >> 1;
        const int n16 = (a.K & 7) == 0 ? xs >> 8 : 0, nt = (xs - 256 * n16 + 63) >> 6;
        const __amdgpu_buffer_rsrc_t rh =
            __builtin_amdgcn_make_buffer_rsrc((void *)a.x, (short)0, 0x7fffffff, kBufferWord3);
        const __amdgpu_buffer_rsrc_t rl =
            __builtin_amdgcn_make_buffer_rsrc((void *)(hilo ? a.x_lo : a.x), (short)0, 0x7fffffff, kBufferWord3);
        // columns c .. c + 7 (c and K multiples of 8: a lane is wholly inside K or wholly past it)
        for (int i = wave; i < rows * n16; i += kWaves) {
            const int r = i / n16, ch = i - r * n16;
            const int c = 512 * ch + 8 * lane;
            const int src_row = hilo ? g0 + (r >> 1) : 0;          // slot of group g0 + r / 2 (one token)
            const uint32_t voff = c < a.K ? (uint32_t)((size_t)src_row * a.K + c) * 2u : kStageOut;
            __builtin_amdgcn_raw_ptr_buffer_load_lds((hilo && (r & 1)) ? rl : rh,
                                                     (__attribute__((address_space(3))) void *)(xlds + r * a.xsp +
                                                                                                 256 * ch),
                                                     16, voff, 0, 0, 0);
        }
        for (int i = wave; i < rows * nt; i += kWaves) {
            const int r = i / nt, d0 = 256 * n16 + 64 * (i - r * nt);
            const int c = 2 * (d0 + lane);
            const int src_row = hilo ? g0 + (r >> 1) : 0;
            const uint32_t voff = c < a.K ? (uint32_t)((size_t)src_row * a.K + c) * 2u : kStageOut;
            __builtin_amdgcn_raw_ptr_buffer_load_lds((hilo && (r & 1)) ? rl : rh,
                                                     (__attribute__((address_space(3))) void *)(xlds + r * a.xsp + d0),
                                                     4, voff, 0, 0, 0);
        }
    };
    // Gate/up: the x staging loads go first, before the routing is read (x does not depend on it), so they are in
    // flight during the routing round trip and ahead of every weight load.  The down launch issues its partial
    // loads after the routing, just ahead of the ring: issued here, their registers stayed live across the set-up
    // and the launch spilled at its 128-register bound.
    if (!form_h) issue();
    // every slot's expert into LDS (read there after the staging barrier: a claim then touches LDS only -- a global
    // load inside the stream would make the wavefront wait for every weight load issued before it)
    if (tid < n_groups) s_exp[tid] = tid < a.n_route ? a.idx[tid] : a.shared_expert;
    // the wavefront's first unit, then claims (an empty unit range ends the wavefront after the staging barrier)
    int u = u_begin + wave;
    const bool active = u < u_end;
    Unit cur = unit_of(active ? u : u_begin, Glb{});
    Cb3Wave w;
    segment(cur, w);
    // the combine in the launch: count the share's units on their row tiles once every partial is stored; the
    // arrival that completes a tile sums it (all wavefronts reach the barriers)
    auto combine_share = [&]() __attribute__((always_inline)) {
        vm_wait<0>();
        __syncthreads();
        const uint32_t total = (uint32_t)(a.NS * a.S);
        for (int u0 = u_begin + tid; u0 < u_end; u0 += blockDim.x) {
            const int rt = u0 % a.RT;
            uint32_t *c = a.rt_ctr + kRtCtrStride * rt;
            if (__hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == total - 1u) {
                __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const uint32_t n = atomicAdd(&s_nlast, 1u);
                if (n < (uint32_t)kCuMaxLast) s_last[n] = rt;
            }
        }
        __syncthreads();
        const int nlast = min((int)s_nlast, kCuMaxLast);
        const __amdgpu_buffer_rsrc_t rp =
            __builtin_amdgcn_make_buffer_rsrc((void *)a.part, (short)0, 0x7fffffff, kBufferWord3);
        constexpr int q4 = 4 * RTW;                 // row quads per row tile
        for (int i = tid; i < nlast * q4; i += blockDim.x) {
            const int r = s_last[i / q4] * 16 * RTW + 4 * (i % q4);
            const float4 o = cu_combine4(a, s_exp, rp, r);
            if (a.out_f32) *(float4 *)(a.out_f32 + r) = o;
            if (a.out_bf16) {
                uint2 bv;
                bv.x = f32_to_bf16_rne(o.x) | (f32_to_bf16_rne(o.y) << 16);
                bv.y = f32_to_bf16_rne(o.z) | (f32_to_bf16_rne(o.w) << 16);
                *(uint2 *)(a.out_bf16 + r) = bv;
            }
        }
    };
    if (!active) {
        if (form_h) {
            form_load(0);
            form_finish();
        }
        vm_wait<0>();
        __syncthreads();
        if (combine) combine_share();
        return;
    }
    cb3_stream<false, RTW>(
        w,
        [&](Cb3Wave &nw) {
            const int nu_ = (int)__builtin_amdgcn_readfirstlane(lane == 0 ? atomicAdd(&s_next, 1u) : 0u);
            if (nu_ >= u_end) return false;
            u = nu_;
            segment(unit_of(u, Lds{}), nw);
            return true;
        },
        [&](f32x4 (&acc)[RTW]) {
            if (hilo) {
#pragma unroll
                for (int r = 0; r < RTW; ++r)
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[r][i] += __shfl_down(acc[r][i], 8, 16);
            }
            if (jt == 0 && cur.e >= 0 && cur.e < a.E) {
                const size_t off = ((size_t)(cur.split * nmat + cur.mat) * a.NS + cur.gi) * a.R +
                                   cur.rt * 16 * RTW + 4 * q;
                float *dst = a.part + off;
                if (combine) {                      // read by other workgroups of this launch
                    // the descriptor from the wave-uniform base, the lane's position as its offset: a descriptor
                    // built per lane would need a loop over the lanes' distinct values
                    const __amdgpu_buffer_rsrc_t pr =
                        __builtin_amdgcn_make_buffer_rsrc((void *)a.part, (short)0, 0x7fffffff, kBufferWord3);
#pragma unroll
                    for (int r = 0; r < RTW; ++r) wt_store4(pr, (uint32_t)(4 * off) + 64u * r, acc[r]);
                } else {
#pragma unroll
                    for (int r = 0; r < RTW; ++r)
                        *(float4 *)(dst + 16 * r) = make_float4(acc[r][0], acc[r][1], acc[r][2], acc[r][3]);
                }
            }
        },
        [&](const Cb3Wave &) { cur = unit_of(u, Lds{}); },
        [&]() {                                     // gate/up: the staging loads were issued above
            if (form_h) form_load(0);
        },
        [&]() {
            if (form_h) form_finish();
            else vm_wait<4 * RTW + 5>();            // the staging loads, issued ahead of the ring
            lds_barrier();                          // ... which stays in flight
        });
    if (combine) combine_share();
}

}  // namespace mi
