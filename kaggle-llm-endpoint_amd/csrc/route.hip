// Router of the GLM MoE block on gfx950: the reference's moe_route (model.py:798-808), the step that produces the
// routing the expert kernels consume.
//   logits = f32(x) @ f32(router_w)      x bf16 [N, D], router_w f32 [D, E] (the reference's layout, model.py:17)
//   scores = sigmoid(logits)
//   idx    = top_k(scores + bias, k)     largest first; equal values: the lower expert id first (lax.top_k)
//   w      = scores[idx]; with norm_topk w / (sum_j w + 1e-20); times scaling
// Two launches on the caller's stream:
//   route_logits_kernel  partial logits per 256-column chunk of D and token block (1, 4, 8 or 16 tokens, the smallest
//                        class holding N): the block's activation tile
//                        is staged in LDS (coalesced), a lane owns one expert and reads its router column coalesced
//                        across the wavefront (E consecutive floats per row of router_w), 8 column pairs of loads in
//                        flight at a time (all 32 at once measured slower at 512 tokens: fewer resident wavefronts);
//                        the 4 wavefronts' column quarters are summed in LDS in a fixed order;
//   route_rank_kernel    (E <= 256) one wavefront per token: the chunk partials (loaded 8 at a time) summed in chunk
//                        order, sigmoid, bias; each candidate's rank in top_k order (larger value, then lower id) is
//                        counted against every choice in LDS, the k lowest ranks are the selection in order, and the
//                        weights are summed in that order, normalised and scaled;
//   route_select_kernel  (E > 256) the same with k rounds of a wavefront argmax instead of ranks.
// Deterministic: every sum in a fixed order, no atomics.
#include <math.h>

#include "common.h"

namespace mi {

constexpr int kRouteDc = 256;                 // columns of D per logits workgroup (64 per wavefront)
constexpr int kRouteTb = 16;                  // tokens per logits workgroup (largest class)
constexpr int kRouteMaxE = 1024;
constexpr int kRouteMaxK = 32;

__device__ __forceinline__ float bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }

// part[c][t][e] = sum over the columns d of chunk c of f32(x[t][d]) * w[d][e]; TB tokens per workgroup (1, 4, 8 or 16:
// the smallest class holding N, so a single token does not pay for 16 rows of multiply-adds)
template <int TB>
__global__ void __launch_bounds__(256) route_logits_kernel(const uint16_t *__restrict__ x,
                                                           const float *__restrict__ w, int N, int D, int E,
                                                           float *__restrict__ part) {
    __shared__ float red[4][TB][65];
    __shared__ uint32_t xs[TB][kRouteDc / 2];                    // the tile's activations as bf16 pairs (zero-padded)
    const int c = blockIdx.x, t0 = blockIdx.y * TB;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nt = min(TB, N - t0);
    const int cb = c * kRouteDc;
    for (int i = threadIdx.x; i < TB * kRouteDc / 2; i += 256) {
        const int t = i / (kRouteDc / 2), p = i - t * (kRouteDc / 2), d = cb + 2 * p;
        xs[t][p] = (t < nt && d < D) ? *(const uint32_t *)(x + (size_t)(t0 + t) * D + d) : 0u;
    }
    __syncthreads();
    constexpr int kPairs = kRouteDc / 8;                        // column pairs per wavefront
    const int p0 = wave * kPairs;
    for (int e0 = 0; e0 < E; e0 += 64) {
        const int e = e0 + lane;
        const bool live = e < E;
        float acc[TB];
#pragma unroll
        for (int t = 0; t < TB; ++t) acc[t] = 0.0f;
        for (int pb = 0; pb < kPairs; pb += 8) {
            float w0[8], w1[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {                       // 16 loads in flight; columns past D read as zero
                const int d = cb + 2 * (p0 + pb + u);
                const bool in = live && d < D;
                w0[u] = in ? w[(size_t)d * E + e] : 0.0f;
                w1[u] = in ? w[(size_t)(d + 1) * E + e] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
#pragma unroll
                for (int t = 0; t < TB; ++t) {
                    const uint32_t xx = xs[t][p0 + pb + u];
                    acc[t] = fmaf(bf16_hi(xx), w1[u], fmaf(bf16_lo(xx), w0[u], acc[t]));
                }
            }
        }
#pragma unroll
        for (int t = 0; t < TB; ++t) red[wave][t][lane] = acc[t];
        __syncthreads();
        for (int i = threadIdx.x; i < nt * 64; i += 256) {
            const int t = i >> 6, l = i & 63;
            if (e0 + l < E) {
                const float s = ((red[0][t][l] + red[1][t][l]) + red[2][t][l]) + red[3][t][l];
                part[((size_t)c * N + t0 + t) * E + e0 + l] = s;
            }
        }
        __syncthreads();
    }
}

// (value, id) ordering of top_k: larger value first, equal values: lower id first
__device__ __forceinline__ bool route_better(float v, int i, float v2, int i2) { return v > v2 || (v == v2 && i < i2); }

// the token's scores and choices (score + bias) of experts 64 j + lane, from the chunk partials summed in order
template <int PER>
__device__ __forceinline__ void route_scores(const float *__restrict__ part, int nc, const float *__restrict__ bias,
                                             int N, int E, int t, int lane, float (&sc)[PER], float (&ch)[PER]) {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int e = 64 * j + lane;
        sc[j] = 0.0f;
        ch[j] = -INFINITY;
        if (e < E) {
            float l = 0.0f;
            for (int c0 = 0; c0 < nc; c0 += 8) {                   // 8 loads in flight, added in chunk order
                float v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) v[u] = c0 + u < nc ? part[((size_t)(c0 + u) * N + t) * E + e] : 0.0f;
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (c0 + u < nc) l += v[u];
            }
            const float s = 1.0f / (1.0f + expf(-l));
            sc[j] = s;
            ch[j] = s + (bias ? bias[e] : 0.0f);
        }
    }
}

template <int PER>   // experts per lane: ceil(E / 64) <= 4
__global__ void __launch_bounds__(256) route_rank_kernel(const float *__restrict__ part, int nc,
                                                         const float *__restrict__ bias, int N, int E, int k, int norm,
                                                         float scaling, int32_t *__restrict__ idx,
                                                         float *__restrict__ wout) {
    __shared__ float4 chs[4][16 * PER];                          // each wavefront's E choices (-inf past E)
    __shared__ float wsel[4][kRouteMaxK];
    __shared__ int isel[4][kRouteMaxK];
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + wv;
    const bool live = t < N;                                     // every wavefront reaches the barriers
    float sc[PER], ch[PER];
    route_scores<PER>(part, nc, bias, N, E, live ? t : 0, lane, sc, ch);
    float *cf = (float *)chs[wv];
#pragma unroll
    for (int j = 0; j < PER; ++j) cf[64 * j + lane] = ch[j];
    __syncthreads();
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int e = 64 * j + lane;
        int rank = 0;
        for (int m4 = 0; m4 < 16 * PER; ++m4) {
            const float4 v = chs[wv][m4];
            const int m = 4 * m4;
            rank += (v.x > ch[j] || (v.x == ch[j] && m < e)) + (v.y > ch[j] || (v.y == ch[j] && m + 1 < e)) +
                    (v.z > ch[j] || (v.z == ch[j] && m + 2 < e)) + (v.w > ch[j] || (v.w == ch[j] && m + 3 < e));
        }
        if (e < E && rank < k) {
            isel[wv][rank] = e;
            wsel[wv][rank] = sc[j];
        }
    }
    __syncthreads();
    if (!live) return;
    float sum = 0.0f;
    for (int r = 0; r < k; ++r) sum += wsel[wv][r];             // in top_k order
    const float inv = norm ? 1.0f / (sum + 1e-20f) : 1.0f;
    if (lane < k) {
        idx[(size_t)t * k + lane] = isel[wv][lane];
        const float v = norm ? wsel[wv][lane] * inv : wsel[wv][lane];
        wout[(size_t)t * k + lane] = v * scaling;
    }
}

template <int PER>   // experts per lane: ceil(E / 64)
__global__ void __launch_bounds__(256) route_select_kernel(const float *__restrict__ part, int nc,
                                                           const float *__restrict__ bias, int N, int E, int k,
                                                           int norm, float scaling, int32_t *__restrict__ idx,
                                                           float *__restrict__ wout) {
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (t >= N) return;                                          // the whole wavefront
    float sc[PER], ch[PER];
    route_scores<PER>(part, nc, bias, N, E, t, lane, sc, ch);
    int sel_i[kRouteMaxK];
    float sel_w[kRouteMaxK];
    float sum = 0.0f;
#pragma unroll
    for (int r = 0; r < kRouteMaxK; ++r) {
        if (r >= k) break;
        // the lane's best (its ids rise with j, so the first maximum is the lowest id)
        float bv = -INFINITY, bs = 0.0f;
        int bi = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int e = 64 * j + lane;
            if (e < E && route_better(ch[j], e, bv, bi)) {
                bv = ch[j];
                bi = e;
                bs = sc[j];
            }
        }
        // wavefront argmax; every lane ends with the winner
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            const float ov = __shfl_xor(bv, m), os = __shfl_xor(bs, m);
            const int oi = __shfl_xor(bi, m);
            if (route_better(ov, oi, bv, bi)) {
                bv = ov;
                bi = oi;
                bs = os;
            }
        }
        sel_i[r] = bi;
        sel_w[r] = bs;
        sum += bs;
        // the owner drops the winner from later rounds
#pragma unroll
        for (int j = 0; j < PER; ++j)
            if (64 * j + lane == bi) ch[j] = -INFINITY;
    }
    const float inv = norm ? 1.0f / (sum + 1e-20f) : 1.0f;
#pragma unroll
    for (int r = 0; r < kRouteMaxK; ++r) {
        if (r >= k) break;
        if (lane == r) {
            idx[(size_t)t * k + r] = sel_i[r];
            const float v = norm ? sel_w[r] * inv : sel_w[r];
            wout[(size_t)t * k + r] = v * scaling;
        }
    }
}

static int route_chunks(int D) { return (D + kRouteDc - 1) / kRouteDc; }

}  // namespace mi

using namespace mi;

extern "C" size_t mi_moe_route_workspace(int32_t N, int32_t D, int32_t E) {
    if (N <= 0 || D <= 0 || E <= 0) return 0;
    return (size_t)route_chunks(D) * (size_t)N * (size_t)E * sizeof(float);
}

extern "C" int mi_moe_route(const uint16_t *x_bf16, const float *router_w, const float *bias, int32_t N, int32_t D,
                            int32_t E, int32_t k, int32_t norm_topk, float scaling, int32_t *idx_out, float *w_out,
                            void *workspace, size_t workspace_bytes, void *stream) {
    if (!x_bf16 || !router_w || !idx_out || !w_out) return MI_ERR_NULL;
    if (N <= 0 || N > (1 << 19)) return MI_ERR_TOKENS;
    if (D <= 0 || D % 2 || E <= 0 || E > kRouteMaxE || (long long)D * E >= (1ll << 31)) return MI_ERR_SHAPE;
    if ((uintptr_t)x_bf16 % 4) return MI_ERR_ARG;             // the rows are read as bf16 pairs
    if (k <= 0 || k > E || k > kRouteMaxK || (norm_topk != 0 && norm_topk != 1)) return MI_ERR_ARG;
    const size_t need = mi_moe_route_workspace(N, D, E);
    if (!workspace || workspace_bytes < need) return MI_ERR_WORKSPACE;
    hipStream_t s = (hipStream_t)stream;
    float *part = (float *)workspace;
    const int nc = route_chunks(D);
    const int tb = N == 1 ? 1 : N <= 4 ? 4 : N <= 8 ? 8 : kRouteTb;
    auto lk = tb == 1 ? route_logits_kernel<1> : tb == 4 ? route_logits_kernel<4>
            : tb == 8 ? route_logits_kernel<8> : route_logits_kernel<kRouteTb>;
    hipLaunchKernelGGL(lk, dim3(nc, (N + tb - 1) / tb), dim3(256), 0, s, x_bf16, router_w, N, D, E, part);
    if (hipGetLastError() != hipSuccess) return MI_ERR_LAUNCH;
    const int per = (E + 63) / 64;
    auto sel = per <= 1 ? route_rank_kernel<1> : per <= 2 ? route_rank_kernel<2> : per <= 4 ? route_rank_kernel<4>
             : per <= 8 ? route_select_kernel<8> : route_select_kernel<16>;
    hipLaunchKernelGGL(sel, dim3((N + 3) / 4), dim3(256), 0, s, (const float *)part, nc, bias, N, E, k, norm_topk,
                       scaling, idx_out, w_out);
    return hipGetLastError() == hipSuccess ? MI_OK : MI_ERR_LAUNCH;
}
