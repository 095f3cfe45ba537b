// Shared device helpers of the gfx950 MoE kernels: bf16 packing, byte-permute lookups, bf16 dot products, the
// agent-scope completion counters and the on-device expert grouping.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mi355moe.h"

namespace mi {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
constexpr int kMaxT = 16;                            // slots per expert group (one wavefront pass)
constexpr int kMaxExperts = 1024;

// v_perm_b32: byte i of the result = byte sel.byte[i] of the 8-byte value {hi:lo} (selector values 0..7).
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// acc + a.bf16[0] * b.bf16[0] + a.bf16[1] * b.bf16[1]  (v_dot2c_f32_bf16; products of bf16 values are exact in f32)
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), acc,
                                           false);
}

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// f32 -> bf16 bits, round to nearest even (the rounding of XLA's astype(bfloat16)).
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;   // quiet NaN
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// f rounded to bf16 (nearest even) and widened back to f32.
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16_rne(f)); }

// f32 = hi + lo with hi = bf16(f) (truncated) and lo = bf16(f - hi): hi + lo carries 16 mantissa bits of f.
__device__ __forceinline__ void split_bf16(float f, uint32_t &hi, uint32_t &lo) {
    uint32_t u = __float_as_uint(f) & 0xffff0000u;
    hi = u >> 16;
    lo = f32_to_bf16_rne(f - __uint_as_float(u));
}

__device__ __forceinline__ float silu_f32(float z) { return z / (1.0f + expf(-z)); }

// silu(min(g, L)) * clip(u, -L, L)  (model.py:119-122)
__device__ __forceinline__ float swiglu_clamped(float g, float u, float limit) {
    g = fminf(g, limit);
    u = fminf(fmaxf(u, -limit), limit);
    return silu_f32(g) * u;
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xffffu));
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// s_waitcnt vmcnt(N) (expcnt and lgkmcnt left alone): N vector memory operations may still be outstanding.
template <int N>
__device__ __forceinline__ void vm_wait() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier for LDS data only, leaving global loads in flight: __syncthreads() waits for every outstanding
// vector memory operation first (its fence covers global memory and direct-to-LDS loads, all counted by vmcnt),
// which drains a weight ring issued ahead of it.  Here the wave's LDS stores complete (lgkmcnt 0), compiler-only
// fences keep every memory access on its side, and the barrier joins the waves.  Data that direct-to-LDS loads
// wrote must be waited for (vm_wait) before it; global memory is not published by it.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xC07F);                   // lgkmcnt(0); vmcnt and expcnt not waited for
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// The sc1 cache policy (buffer instructions' aux bits): stores are written through this XCD's L2 to memory, loads are
// coherent at device scope (the cache bits of a relaxed agent-scope atomic load).
constexpr int kCachePolicySc1 = 16;

// Coherent loads: they return what another workgroup stored through to memory (sc1 stores) earlier in the same launch
// even when this XCD's L2 holds an older copy of the line (a neighbouring value of the same 128-byte line may have
// pulled it in).  Every value one workgroup hands another inside a launch is read this way, after the count that
// publishes it.
__device__ __forceinline__ f32x4 coherent_load4(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, 0, kCachePolicySc1));
}
__device__ __forceinline__ uint2 coherent_load2(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
    return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, 0, kCachePolicySc1));
}

// Completion counters.  On this multi-XCD part an agent-scope release writes back the XCD's L2 and an acquire
// invalidates it, so they are issued as rarely as possible: after a workgroup barrier (which completes every wave's
// stores to L2) ONE thread issues the release fence and the relaxed increment; only the workgroup that observes the
// final count issues the acquire before reading the other workgroups' partials.
__device__ __forceinline__ uint32_t counter_add(uint32_t *c, uint32_t v) {
    return __hip_atomic_fetch_add(c, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void fence_release_agent() { __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent"); }
__device__ __forceinline__ void fence_acquire_agent() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent"); }
__device__ __forceinline__ void counter_reset(uint32_t *c) {
    __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------------------------------------------ expert grouping
// The (slot -> expert) routing of one call, grouped on the device: every distinct expert (ascending id) gets
// ceil(count / cap) groups of at most cap slots (ascending slot order; cap <= kMaxT is the launch's token class);
// the shared expert, if any, gets ceil(N / cap) more groups whose slots are n_route + n.  Every workgroup recomputes it from idx (n_route <= 128
// entries), so no host sync and no extra launch is needed.
struct Group {
    int expert;   // -1: this workgroup has no group (grid padding)
    int n;        // slots in the group (1..kMaxT)
    int slot[kMaxT];
};

struct GroupScratch {
    uint32_t count[kMaxExperts];
    int idx[MI_MAX_SLOTS];
    int lane_base[kWave + 1];
    Group g;
};

// Must be called by all threads of the block (blockDim.x >= 64).  Result in sc.g (after the final barrier).
__device__ inline void find_group(GroupScratch &sc, const int32_t *__restrict__ idx, int n_route, int E,
                                  int shared_expert, int N, int gi, int cap) {
    const int tid = threadIdx.x;
    for (int e = tid; e < E; e += blockDim.x) sc.count[e] = 0;
    __syncthreads();
    for (int i = tid; i < n_route; i += blockDim.x) {
        int e = idx[i];
        sc.idx[i] = e;
        if (e >= 0 && e < E) atomicAdd(&sc.count[e], 1u);
    }
    __syncthreads();
    if (tid < kWave) {
        // lane owns experts [lane*per, (lane+1)*per)
        const int per = (E + kWave - 1) / kWave;
        int e0 = tid * per, e1 = min(E, e0 + per);
        int ng = 0;
        for (int e = e0; e < e1; ++e) ng += (sc.count[e] + cap - 1) / cap;
        // inclusive scan over the wavefront
        int incl = ng;
        for (int off = 1; off < kWave; off <<= 1) {
            int v = __shfl_up(incl, off, kWave);
            if (tid >= off) incl += v;
        }
        int excl = incl - ng;
        int total = __shfl(incl, kWave - 1, kWave);
        if (tid == 0) {
            sc.g.expert = -1;
            sc.g.n = 0;
        }
        __builtin_amdgcn_wave_barrier();
        if (gi >= excl && gi < incl) {
            int r = gi - excl;
            for (int e = e0; e < e1; ++e) {
                int c = (int)sc.count[e];
                int ge = (c + cap - 1) / cap;
                if (r < ge) {
                    sc.g.expert = e;
                    sc.g.n = min(cap, c - r * cap);
                    sc.lane_base[kWave] = r;      // chunk index within the expert
                    break;
                }
                r -= ge;
            }
        }
        if (tid == 0 && gi >= total && shared_expert >= 0) {
            int r = gi - total;
            int ns = (N + cap - 1) / cap;
            if (r < ns) {
                sc.g.expert = shared_expert;
                sc.g.n = min(cap, N - r * cap);
                sc.lane_base[kWave] = -1 - r;     // marks a shared group
            }
        }
    }
    __syncthreads();
    if (tid < kWave && sc.g.expert >= 0) {
        const int e = sc.g.expert;
        const int chunk = sc.lane_base[kWave];
        if (chunk < 0) {
            int r = -1 - chunk;
            if (tid < sc.g.n) sc.g.slot[tid] = n_route + r * cap + tid;
        } else {
            // compact the slots routed to e (ascending), keep positions [chunk*cap, chunk*cap + n)
            int base = 0;
            for (int i0 = 0; i0 < n_route; i0 += kWave) {
                int i = i0 + tid;
                bool hit = (i < n_route) && (sc.idx[i] == e);
                uint64_t m = __ballot(hit);
                int pos = base + __popcll(m & ((1ull << tid) - 1ull));
                int p = pos - chunk * cap;
                if (hit && p >= 0 && p < cap) sc.g.slot[p] = i;
                base += __popcll(m);
            }
        }
    }
    __syncthreads();
}

// Number of groups of one call is at most this (grid size of the grouped kernels).
__host__ __device__ inline int max_groups(int n_route, int E, int N, int shared_expert, int cap) {
    int routed = n_route < E ? n_route : E;
    routed += n_route / cap;                         // extra chunks of experts with more than cap slots
    if (routed > n_route) routed = n_route;
    int shared = shared_expert >= 0 ? (N + cap - 1) / cap : 0;
    return routed + shared;
}

}  // namespace mi
