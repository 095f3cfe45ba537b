// CU-balanced CB3 streams for decode at 2..16 tokens (gate/up partials, down partials) on gfx950.
//
// The single-token launches (custream.h) give every CU an equal contiguous share of the layer's work units and keep
// one workgroup per CU.  With several tokens a unit's activations are no longer one row, so this variant adds:
//   - groups keyed by (expert, occurrence): the o-th slot of a token that names expert e joins group (e, o), so a
//     token appears at most once in a group and column t of the matrix-core tile is token t, for gate/up and down
//     alike.  Every workgroup builds the same group table from the routing ids in LDS (groups in ascending key
//     order, so both occurrences of a repeated expert stream back to back);
//   - split-major shares: the workgroups are dealt to the column splits (workgroups [s P / S, (s + 1) P / S) take
//     split s) and share the split's (group, matrix, row tile) units equally, so a workgroup stages only its split's
//     columns;
//   - gate/up stages x of every token once (N rows of the split's columns); down stages h (bf16 high part and
//     remainder, one row per token, zeros for tokens outside the group) of the groups its share touches, at most
//     `gmax` groups at a time: a share that touches more runs as several epochs, each a stream of its own after a
//     workgroup barrier (the host sizes gmax so that one epoch is the common case).
// Each unit writes its own f32 partial rows (the slots of its group's tokens); the next launch reduces them in a
// fixed order.
#pragma once
#include <climits>

#include "custream.h"

namespace mi {

constexpr int kMuMaxSlots = MI_MAX_SLOTS + kMaxT;    // routed slots + one shared slot per token

struct MArgs {
    Cb3Table t0, t1;           // gate, up (kGateUp) or down (t0 only)
    int R, K;                  // rows, cols of the table(s)
    int E, n_route, N, k, shared_expert, NS;
    int S, al, nu;             // column splits: boundaries at multiples of `al` column tiles over nu tiles
    int RT;                    // 16 RTW-row tiles per matrix
    int P;                     // workgroups (= CUs)
    int gmax;                  // kDown: groups staged at a time
    int xsp;                   // LDS row pitch (dwords) of a staged row (the widest split's columns)
    const uint16_t *x;         // kGateUp: x bf16 [N, K]; kDown: bf16 high part of h [NS, K]
    const uint16_t *x_lo;      // kDown: bf16 remainder of h [NS, K]
    const int32_t *idx;
    float *part;               // [S][nmat][NS][R]
};

// TWO (kDown, more than 8 tokens): h's high part and remainder in two matrix-core instructions; otherwise one, with
// the high part in columns 0-7 and the remainder in 8-15 (added by a lane shuffle at the end).
template <int MODE, int RTW, bool TWO>
__global__ void __launch_bounds__(64 * kCuWaves, 1) cumulti_kernel(MArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint32_t xlds[];
    __shared__ uint32_t s_next;
    __shared__ int s_e[kMuMaxSlots];                // expert of every slot
    __shared__ int s_key[kMuMaxSlots];              // group key of every slot (INT_MAX: invalid expert)
    __shared__ int s_first[kMuMaxSlots];            // 1: the first slot of its key
    __shared__ int s_gexp[kMuMaxSlots];             // expert of every group
    __shared__ int16_t s_gslot[kMuMaxSlots][kMaxT]; // group x token -> slot (-1: the token is not in the group)
    __shared__ int s_ng;
    constexpr bool hilo = MODE == kDown;
    constexpr int nmat = MODE == kGateUp ? 2 : 1;
    const int tid = threadIdx.x, lane = tid & 63, jt = lane & 15, q = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int N = a.N, NS = a.NS, nr = a.n_route;

    // ---- group table (identical in every workgroup)
    for (int i = tid; i < kMuMaxSlots * kMaxT; i += blockDim.x) (&s_gslot[0][0])[i] = -1;
    if (tid == 0) s_ng = 0;
    if (tid < NS) s_e[tid] = tid < nr ? a.idx[tid] : a.shared_expert;
    __syncthreads();
    if (tid < NS) {
        const int e = s_e[tid], t = tid < nr ? tid / a.k : tid - nr;
        // occurrence: the token's earlier slots naming e (its routed slots in column order, then its shared slot)
        const int jend = tid < nr ? tid - t * a.k : a.k;
        int o = 0;
        for (int j = 0; j < jend; ++j) o += s_e[t * a.k + j] == e;
        s_key[tid] = (e >= 0 && e < a.E) ? e * (a.k + 1) + o : INT_MAX;
    }
    __syncthreads();
    if (tid < NS) {
        const int key = s_key[tid];
        int first = key != INT_MAX;
        for (int s2 = 0; s2 < tid; ++s2) first &= s_key[s2] != key;
        s_first[tid] = first;
        if (first) atomicAdd(&s_ng, 1);
    }
    __syncthreads();
    if (tid < NS && s_key[tid] != INT_MAX) {
        const int key = s_key[tid], t = tid < nr ? tid / a.k : tid - nr;
        int g = 0;
        for (int s2 = 0; s2 < NS; ++s2) g += s_first[s2] && s_key[s2] < key;
        s_gslot[g][t] = (int16_t)tid;
        if (s_first[tid]) s_gexp[g] = s_e[tid];
    }
    __syncthreads();
    const int ng = s_ng;

    // ---- this workgroup's split and unit range: unit u = (group, matrix, row tile), row tile fastest.  Split s holds
    // column tiles [ct(s), ct(s + 1)) and workgroups [P ct(s) / nu, P ct(s + 1) / nu), in proportion to its columns
    const int nb = (a.nu + a.al - 1) / a.al;
    auto ct_of = [&](int s) { return min(a.nu, a.al * (int)((long long)s * nb / a.S)); };
    auto wg_of = [&](int s) { return (int)((long long)a.P * ct_of(s) / a.nu); };
    int split = 0;
    while (split + 1 < a.S && (int)blockIdx.x >= wg_of(split + 1)) ++split;
    const int wg0 = wg_of(split), wg1 = split + 1 < a.S ? wg_of(split + 1) : a.P;
    const int per_g = nmat * a.RT;
    const int U = ng * per_g;
    const int lb = blockIdx.x - wg0, Ps = wg1 - wg0;
    const int u_begin = (int)((long long)lb * U / Ps);
    const int u_end = (int)((long long)(lb + 1) * U / Ps);
    if (u_begin >= u_end) return;

    const int cta = ct_of(split), ctb = ct_of(split + 1);
    const int c0 = kCb3TileCols * cta, c1 = min(a.K, kCb3TileCols * ctb);    // the split's columns
    const int rows_per_g = hilo ? 2 * N : 0;
    const int stage_rows = hilo ? rows_per_g * a.gmax : N;
    uint4 *cbl = (uint4 *)(xlds + (size_t)stage_rows * a.xsp);

    struct Unit {
        int g, mat, rt, e;
    };
    auto unit_of = [&](int u) {
        Unit k;
        k.rt = u % a.RT;
        const int r = u / a.RT;
        k.mat = r % nmat;
        k.g = r / nmat;
        k.e = __builtin_amdgcn_readfirstlane(s_gexp[k.g]);
        return k;
    };
    int g_lo = 0;                                   // kDown: first group of the epoch's staging
    auto segment = [&](const Unit &k, Cb3Wave &w) {
        const Cb3Table &tb = k.mat ? a.t1 : a.t0;
        const uint32_t *qt = tb.qs + (size_t)k.e * tb.CT * tb.RT * 256;
        const uint32_t *cbe = tb.cb + (size_t)k.e * tb.G * tb.R * 4;
        w.qb = __builtin_amdgcn_make_buffer_rsrc((void *)qt, (short)0, 0x7fffffff, kBufferWord3);
        w.qnull = __builtin_amdgcn_make_buffer_rsrc((void *)qt, (short)0, 0, kBufferWord3);
        w.cbb = __builtin_amdgcn_make_buffer_rsrc((void *)cbe, (short)0, 0x7fffffff, kBufferWord3);
        w.cbnull = __builtin_amdgcn_make_buffer_rsrc((void *)cbe, (short)0, 0, kBufferWord3);
        w.cta = cta;
        w.ctb = ctb;
        w.ct_bytes = (uint32_t)tb.RT * 1024u;
        w.rt_bytes = (uint32_t)(k.rt * RTW) * 1024u;
        w.g_bytes = (uint32_t)tb.R * 16u;
        w.row_bytes = (uint32_t)(k.rt * 16 * RTW) * 16u;
        w.g_first = (kCb3TileCols * w.cta) >> 7;
        w.g_last = min((kCb3TileCols * w.ctb - 1) >> 7, tb.G - 1);
        w.lane16 = (uint32_t)lane * 16u;
        w.cblane16 = (uint32_t)(lane & (16 * RTW - 1)) * 16u;
        w.cbl = cbl + wave * 5 * 64;
        // B operand: column jt = token jt (columns past N read the last token's row; they are never stored); down
        // with one instruction: the high part in columns 0-7, the remainder in 8-15
        int row;
        if constexpr (!hilo) {
            row = min(jt, N - 1);
        } else if constexpr (TWO) {
            row = (k.g - g_lo) * rows_per_g + min(jt, N - 1);
        } else {
            row = (k.g - g_lo) * rows_per_g + (jt >= 8 ? N : 0) + min(jt & 7, N - 1);
        }
        w.xh = xlds + row * a.xsp + 4 * q;
        w.xl = hilo && TWO ? w.xh + N * a.xsp : w.xh;
    };
    // staged rows straight into LDS, spread over the wavefronts, issued ahead of every wavefront's weight ring:
    // columns past the split read zeros.  Whole 256-dword chunks of a row load 16 bytes per lane, the rest 4 (an
    // LDS-bound load costs about as much per instruction whatever its width)
    auto issue_rows = [&](int g_first_st, int n_st) {
        const int xs = 80 * (ctb - cta);                            // whole column tiles (past K: zeros)
        const int n16 = (a.K & 7) == 0 ? xs >> 8 : 0, nt = (xs - 256 * n16 + 63) >> 6;
        const __amdgpu_buffer_rsrc_t rh =
            __builtin_amdgcn_make_buffer_rsrc((void *)a.x, (short)0, 0x7fffffff, kBufferWord3);
        const __amdgpu_buffer_rsrc_t rl =
            __builtin_amdgcn_make_buffer_rsrc((void *)(hilo ? a.x_lo : a.x), (short)0, 0x7fffffff, kBufferWord3);
        const int rows = hilo ? n_st * rows_per_g : N;
        auto src_of = [&](int r, bool &lo) {
            int src = r;                            // gate/up: token r
            lo = false;
            if constexpr (hilo) {                   // down: group g_first_st + r / 2N, token (r % 2N) % N
                const int lg = r / rows_per_g, rr = r - lg * rows_per_g;
                lo = rr >= N;
                src = s_gslot[g_first_st + lg][rr - (lo ? N : 0)];
            }
            return src;
        };
        // columns c .. c + 7 (c0, c1 and K multiples of 8: a lane is wholly inside the split or wholly past it)
        for (int i = wave; i < rows * n16; i += kCuWaves) {
            const int r = i / n16, ch = i - r * n16;
            const int c = c0 + 512 * ch + 8 * lane;
            bool lo;
            const int src = src_of(r, lo);
            const uint32_t voff = (src >= 0 && c < c1) ? (uint32_t)((size_t)src * a.K + c) * 2u : kStageOut;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(lo ? rl : rh,
                                                     (__attribute__((address_space(3))) void *)(xlds + r * a.xsp +
                                                                                                 256 * ch),
                                                     16, voff, 0, 0, 0);
        }
        for (int i = wave; i < rows * nt; i += kCuWaves) {
            const int r = i / nt, d0 = 256 * n16 + 64 * (i - r * nt);
            const int c = c0 + 2 * (d0 + lane);
            bool lo;
            const int src = src_of(r, lo);
            const uint32_t voff = (src >= 0 && c < c1) ? (uint32_t)((size_t)src * a.K + c) * 2u : kStageOut;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(lo ? rl : rh,
                                                     (__attribute__((address_space(3))) void *)(xlds + r * a.xsp + d0),
                                                     4, voff, 0, 0, 0);
        }
    };

    // ---- epochs: gate/up one; down: the share's groups gmax at a time
    const int g_first_all = u_begin / per_g, g_last_all = (u_end - 1) / per_g;
    for (int ge = g_first_all; ge <= g_last_all; ge += hilo ? a.gmax : INT_MAX / 2) {
        const int ge_end = hilo ? min(g_last_all + 1, ge + a.gmax) : g_last_all + 1;
        const int ub = max(u_begin, ge * per_g), ue = min(u_end, ge_end * per_g);
        g_lo = ge;
        if (ge > g_first_all) __syncthreads();      // every wavefront is done with the previous epoch's rows
        if (tid == 0) s_next = (uint32_t)ub + kCuWaves;
        int u = ub + wave;
        const bool active = u < ue;
        Unit cur = unit_of(active ? u : ub);
        Cb3Wave w;
        segment(cur, w);
        if (!active) {
            issue_rows(ge, ge_end - ge);
            vm_wait<0>();
            __syncthreads();
            continue;
        }
        cb3_stream<TWO, RTW>(
            w,
            [&](Cb3Wave &nw) {
                const int nu_ = (int)__builtin_amdgcn_readfirstlane(lane == 0 ? atomicAdd(&s_next, 1u) : 0u);
                if (nu_ >= ue) return false;
                u = nu_;
                segment(unit_of(u), nw);
                return true;
            },
            [&](f32x4 (&acc)[RTW]) {
                if constexpr (hilo && !TWO) {
#pragma unroll
                    for (int r = 0; r < RTW; ++r)
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[r][i] += __shfl_down(acc[r][i], 8, 16);
                }
                const int slot = jt < N && (!hilo || TWO || jt < 8) ? s_gslot[cur.g][jt] : -1;
                if (slot >= 0) {
                    float *dst = a.part + ((size_t)(split * nmat + cur.mat) * a.NS + slot) * a.R +
                                 cur.rt * 16 * RTW + 4 * q;
#pragma unroll
                    for (int r = 0; r < RTW; ++r)
                        *(float4 *)(dst + 16 * r) = make_float4(acc[r][0], acc[r][1], acc[r][2], acc[r][3]);
                }
            },
            [&](const Cb3Wave &) { cur = unit_of(u); },
            [&]() { issue_rows(ge, ge_end - ge); },
            [&]() {
                vm_wait<4 * RTW + 5>();             // the staging loads, issued ahead of the ring
                lds_barrier();                      // ... which stays in flight
            });
    }
}

}  // namespace mi
