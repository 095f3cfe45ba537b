// Prefill MoE for CB3, IQ2_S, IQ3_S, IQ4_XS, Q2_K and Q3_K experts (the reference's ragged prefill,
// resident.py:144-165 with pallas_moe.py:564-592,622-755, and its other bf16 prefill branches, resident.py:122-135,
// 169-210), host side and the small kernels around the grouped GEMMs of prefill_gemm.h:
//   ragged_plan_kernel  the reference's slot layout (pallas_moe.py:564-592) built on the device by one workgroup:
//                       slots stably sorted by expert, every expert padded to whole blocks of tm rows;
//   prefill_combine     out[t] = sum_j wt(t, j) * y[row_slot(t, j)] in f32 with wt = bf16(w) ("matmul" combine,
//                       resident.py:161-163) or wt = w ("gather", resident.py:164-165);
//   prefill_combine_f32 the sweeps' sum of f32 rows (resident.py:169-187) or of bf16-rounded expert groups
//                       (resident.py:189-210).
// The rounding points are the reference's: bf16 activations, bf16 weights (CB3 centroids are bf16 already; IQ2_S /
// IQ3_S / IQ4_XS level * scale rounded once), f32 accumulation, h and y rounded to bf16, routing weights rounded to
// bf16 by the matmul combine; the other branches' forms as mi_moe_prefill_form states them.
#include <climits>

#include "prefill_gemm.h"

namespace mi {
constexpr int kPlanThreads = 1024;
constexpr int kPlanWaves = kPlanThreads / 64;
constexpr int kPlanMaxE = 1024;
constexpr long long kPlanMaxSlots = 1 << 22;
constexpr int kPlanReg = 8;                 // slots per thread held in registers (S <= kPlanReg * kPlanThreads)
constexpr int kPlanMaskE = 512;             // up to this many experts, pass 2 matches ids through LDS words

struct PlanOut {
    int32_t *blk_expert;   // [G]   expert of every block (blocks >= n_blocks repeat the last expert)
    int32_t *n_blocks;     // [1]
    int32_t *tok_row;      // [Rp]  token of every sorted row, -1 = padding
    float *w_row;          // [Rp]  routing weight of every sorted row, 0 = padding
    int32_t *row_slot;     // [T * kk] sorted row of every (token, slot); -1 for an expert id outside [0, E)
    int32_t *blk_n;        // [G]   rows of every block that are not padding (NULL: not written)
    int merge_dups;        // w_row of the first slot of a token's expert = the sum of that token's weights of the
                           // expert in column order, 0 for its later slots (the sweeps' summed routing weight)
    uint32_t *cnt;         // [n_cnt] the grouped GEMMs' split-task counters, zeroed here (NULL: none)
    int n_cnt;
};

// Slot s of the plan: token s / kk, column j = s % kk; columns j < k are the routed slots, column k (kk = k + 1) is
// the shared expert (weight 1) when one is given.  A slot whose expert id is outside [0, E) takes no row.

// Routed weight of column j of token t, expert e, for a plan that merges duplicates: w[t, jj] summed over the token's
// columns jj naming e, in column order, when j is the first of them; 0 for a later one.  Every load of a group of
// columns is issued before the group's compares.
__device__ __forceinline__ float plan_weight_merged(const int32_t *idx, const float *w, int t, int j, int k, int e) {
    float sum = 0.0f;
    bool first = true;
#pragma unroll 4
    for (int jj = 0; jj < k; ++jj) {
        const int ej = idx[t * k + jj];
        const float wj = w[t * k + jj];
        if (ej == e) {
            sum += wj;
            first = first && jj >= j;
        }
    }
    return first ? sum : 0.0f;
}

// Inclusive prefix sum over the kPlanThreads threads of the workgroup (every thread calls it).
__device__ int block_inclusive_scan(int v, int *wsum) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int o = __shfl_up(v, d, 64);
        if (lane >= d) v += o;
    }
    if (lane == 63) wsum[wave] = v;
    __syncthreads();
    for (int i = 0; i < wave; ++i) v += wsum[i];
    __syncthreads();
    return v;
}

// Lanes of this wavefront holding a valid expert id equal to this lane's: the AND, over the id's nbits (<= 10) bits,
// of the ballot of the lanes that agree with this lane on the bit (nbits + 1 ballots, whatever the number of
// distinct ids).
__device__ __forceinline__ uint64_t match_expert(int e, bool valid, int nbits) {
    static_assert(kPlanMaxE <= 1024, "expert ids have at most 10 bits");
    uint64_t m = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 10; ++b) {
        if (b >= nbits) break;
        const uint64_t on = __ballot(valid && ((e >> b) & 1));
        const uint64_t d = (uint64_t)(int64_t)((e << (31 - b)) >> 31);   // all ones when bit b of e is set
        m &= ~(on ^ d);
    }
    return m;
}

// The reference's ragged_plan (pallas_moe.py:564-592), stable: the rows of one expert follow slot order.  Wavefront
// v owns the contiguous slots [v * C, (v + 1) * C), C = 64 * ceil(S / kPlanThreads), walked 64 at a time in slot
// order.  Pass 1 counts every expert's slots per wavefront (LDS atomics); an exclusive prefix over the wavefronts
// gives each wavefront its first row within the expert and the expert's total; pass 2 walks the slots again and
// places slot s at the expert's first padded row + the wavefront's running row + the number of lower lanes of the
// same id (an LDS word per wavefront and id that the lanes OR their bits into, or ballots of the id's bits past
// kPlanMaskE experts).  Expert ids and weights of up to kPlanReg * kPlanThreads slots stay in registers between the passes.
__global__ void __launch_bounds__(kPlanThreads) ragged_plan_kernel(const int32_t *__restrict__ idx,
                                                                   const float *__restrict__ w, int T, int k,
                                                                   int shared, int E, int tm, PlanOut p) {
    static_assert(kPlanWaves == 16, "the prefix over wavefronts scans 16 lanes per expert");
    __shared__ int cntw[kPlanMaxE][kPlanWaves];   // per-wavefront count of every expert, then its running row
    __shared__ int cnt[kPlanMaxE], bend[kPlanMaxE], rbase[kPlanMaxE];
    __shared__ unsigned long long lanes[kPlanWaves][kPlanMaskE];   // pass 2: lanes of every id in this step
    __shared__ int wsum[kPlanWaves];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kk = k + (shared >= 0 ? 1 : 0);
    const int S = T * kk;
    const int G = (S + tm - 1) / tm + E;
    const long long Rp = (long long)G * tm;
    const int nsub = (S + kPlanThreads - 1) / kPlanThreads;   // 64-slot steps per wavefront
    const int s0 = wave * nsub * 64 + lane;                  // this lane's slot in step 0
    int nbits = 0;
    while ((1 << nbits) < E) ++nbits;

    for (int i = tid; i < E * kPlanWaves; i += kPlanThreads) (&cntw[0][0])[i] = 0;
    if (E <= kPlanMaskE)
        for (int i = tid; i < kPlanWaves * kPlanMaskE; i += kPlanThreads) (&lanes[0][0])[i] = 0ull;
    // expert ids, weights and tokens of kPlanReg steps at a time, every load issued before any is used
    int ereg[kPlanReg], treg[kPlanReg];
    float wreg[kPlanReg];
    const int q64 = 64 / kk, r64 = 64 - q64 * kk;   // a step of 64 slots advances q64 tokens and r64 columns
    auto load_steps = [&](int rb) {
        int col[kPlanReg], raw[kPlanReg];
        float wraw[kPlanReg];
        const int sb = s0 + rb * 64;
        int t = sb / kk, j = sb - t * kk;          // token and column of this lane's slot, step by step
#pragma unroll
        for (int r = 0; r < kPlanReg; ++r) {
            const bool in = rb + r < nsub && sb + r * 64 < S;
            col[r] = in ? j : k;                   // column k: the shared expert's (or no slot)
            treg[r] = in ? t : -1;
            const int q = in && j < k ? t * k + j : 0;
            raw[r] = idx[q];
            wraw[r] = w[q];
            t += q64;
            j += r64;
            if (j >= kk) {
                j -= kk;
                ++t;
            }
        }
#pragma unroll
        for (int r = 0; r < kPlanReg; ++r) {
            int e = col[r] < k ? raw[r] : shared;
            if (treg[r] < 0 || e < 0 || e >= E) e = -1;
            ereg[r] = e;
            wreg[r] = col[r] < k ? wraw[r] : 1.0f;
            if (p.merge_dups && e >= 0 && col[r] < k) wreg[r] = plan_weight_merged(idx, w, treg[r], col[r], k, e);
        }
    };
    __syncthreads();

    // pass 1: count (order-free)
    for (int rb = 0; rb < nsub; rb += kPlanReg) {
        load_steps(rb);
#pragma unroll
        for (int r = 0; r < kPlanReg; ++r)
            if (rb + r < nsub && ereg[r] >= 0) atomicAdd(&cntw[ereg[r]][wave], 1);
    }
    // every row starts as padding; the rows of pass 2 overwrite theirs after the wait below
    for (int r = tid; r < (int)Rp; r += kPlanThreads) {   // Rp < 2^31 (checked on the host)
        p.tok_row[r] = -1;
        p.w_row[r] = 0.0f;
    }
    __syncthreads();
    // exclusive prefix over the wavefronts, 16 lanes per expert, and every expert's total
    for (int eb = 0; eb < E; eb += kPlanThreads / kPlanWaves) {
        const int e = eb + (tid >> 4), v = tid & 15;
        const int c = e < E ? cntw[e][v] : 0;
        int incl = c;
#pragma unroll
        for (int d = 1; d < 16; d <<= 1) {
            const int o = __shfl_up(incl, d, 16);
            if (v >= d) incl += o;
        }
        if (e < E) {
            cntw[e][v] = incl - c;
            if (v == 15) cnt[e] = incl;
        }
    }
    __syncthreads();
    // blocks per expert and their inclusive prefix (block end); padded rows start at (bend - nb) * tm
    const int nb_own = tid < E ? (cnt[tid] + tm - 1) / tm : 0;
    const int incl = block_inclusive_scan(nb_own, wsum);
    if (tid < kPlanMaxE) {
        bend[tid] = incl;
        rbase[tid] = (incl - nb_own) * tm;
    }
    __syncthreads();
    const int n_blocks = bend[kPlanMaxE - 1];
    if (tid == 0) *p.n_blocks = n_blocks;
    for (int i = tid; i < p.n_cnt; i += kPlanThreads) p.cnt[i] = 0u;
    vm_wait<0>();                              // this wavefront's padding stores are done ...
    __syncthreads();                            // ... and every other wavefront's

    // pass 2: rows (the loads of pass 1 are still in registers when one batch held every step)
    for (int rb = 0; rb < nsub; rb += kPlanReg) {
        if (nsub > kPlanReg) load_steps(rb);
#pragma unroll
        for (int r = 0; r < kPlanReg; ++r) {
            if (rb + r >= nsub) break;
            const int s = s0 + (rb + r) * 64;
            const int e = ereg[r];
            const bool valid = e >= 0;
            uint64_t m;
            if (E <= kPlanMaskE) {
                // the lanes of each id gather in an LDS word: OR in, read back (LDS operations of one wavefront
                // complete in order, so the read sees every lane's bit); the lowest lane clears it below
                if (valid) atomicOr(&lanes[wave][e], 1ull << lane);
                m = valid ? lanes[wave][e] : 0ull;
            } else {
                m = match_expert(e, valid, nbits);
            }
            const int below = __popcll(m & ((1ull << lane) - 1ull));
            int row = -1;
            if (valid) {
                row = rbase[e] + cntw[e][wave] + below;
                p.tok_row[row] = treg[r];
                p.w_row[row] = wreg[r];
            }
            if (s < S) p.row_slot[s] = row;
            // every lane of the wavefront has read the running row above (LDS operations of one wavefront complete
            // in order) before the lowest lane of each id advances it
            if (valid && below == 0) {
                cntw[e][wave] += __popcll(m);
                if (E <= kPlanMaskE) lanes[wave][e] = 0ull;
            }
        }
    }

    // block -> expert: the first expert whose block end exceeds g; blocks past n_blocks repeat the last one (the
    // expert of block n_blocks - 1, or E - 1 when there is none, as the reference's clamp gives)
    int last = E - 1;
    if (n_blocks > 0) {
        int lo = 0, hi = E - 1;
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (bend[mid] > n_blocks - 1) hi = mid;
            else lo = mid + 1;
        }
        last = lo;
    }
    for (int g = tid; g < G; g += kPlanThreads) {
        int e = last, n = 0;
        if (g < n_blocks) {
            int lo = 0, hi = E - 1;
            while (lo < hi) {
                const int mid = (lo + hi) >> 1;
                if (bend[mid] > g) hi = mid;
                else lo = mid + 1;
            }
            e = lo;
            const int nb = (cnt[e] + tm - 1) / tm;
            n = min(tm, cnt[e] - (g - (bend[e] - nb)) * tm);
        }
        p.blk_expert[g] = e;
        if (p.blk_n) p.blk_n[g] = n;
    }
}

// out[t] = sum_j wt(t, j) * y[row_slot(t, j)] over the plan's kk columns in order, f32; wt = bf16(w) for the matmul
// combine, w for the gather combine (the shared column has weight 1 either way).  One thread per 4 output columns.
__global__ void __launch_bounds__(256) prefill_combine(const uint16_t *__restrict__ y, const int32_t *__restrict__ row_slot,
                                                       const float *__restrict__ w, int T, int k, int kk, int D,
                                                       int bf16_weights, float *out_f32, uint16_t *out_bf16) {
    // one thread per 8 output columns of one token; the rows of up to 8 columns j are loaded before any is added,
    // and added in column order
    const int q8 = D >> 3;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= T * q8) return;
    const int t = i / q8, c = 8 * (i - t * q8);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int j0 = 0; j0 < kk; j0 += 8) {
        int r[8];
        float wt[8];
        uint4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int j = j0 + u;
            r[u] = j < kk ? row_slot[t * kk + j] : -1;
            wt[u] = 1.0f;
            if (j < k) {
                wt[u] = w[t * k + j];
                if (bf16_weights) wt[u] = bf16_to_f32(f32_to_bf16_rne(wt[u]));
            }
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = r[u] >= 0 ? *(const uint4 *)(y + (size_t)r[u] * D + c) : make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if (r[u] < 0) continue;
            const uint32_t vv[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                acc[2 * h] += wt[u] * bf16_to_f32(vv[h] & 0xffffu);
                acc[2 * h + 1] += wt[u] * bf16_to_f32(vv[h] >> 16);
            }
        }
    }
    if (out_f32) {
        *(float4 *)(out_f32 + (size_t)t * D + c) = make_float4(acc[0], acc[1], acc[2], acc[3]);
        *(float4 *)(out_f32 + (size_t)t * D + c + 4) = make_float4(acc[4], acc[5], acc[6], acc[7]);
    }
    if (out_bf16) {
        uint4 b;
        b.x = f32_to_bf16_rne(acc[0]) | (f32_to_bf16_rne(acc[1]) << 16);
        b.y = f32_to_bf16_rne(acc[2]) | (f32_to_bf16_rne(acc[3]) << 16);
        b.z = f32_to_bf16_rne(acc[4]) | (f32_to_bf16_rne(acc[5]) << 16);
        b.w = f32_to_bf16_rne(acc[6]) | (f32_to_bf16_rne(acc[7]) << 16);
        *(uint4 *)(out_bf16 + (size_t)t * D + c) = b;
    }
}

// ------------------------------------------------------------------------------------------------ host side
// out[t] = the sum of the f32 rows y[row_slot(t, j)] over the plan's kk columns (the routing weights are already in
// h).  chunk == 0, the dense sweep (resident.py:169-187): one f32 sum in column order.  chunk > 0, the XLA sweep
// (resident.py:189-210): the columns are grouped by expert / chunk, each group summed in f32 in column order,
// rounded to bf16 once and added to the f32 total in ascending group order.  One thread per 4 output columns.
__global__ void __launch_bounds__(256) prefill_combine_f32(const float *__restrict__ y,
                                                           const int32_t *__restrict__ row_slot,
                                                           const int32_t *__restrict__ idx, int T, int k, int kk,
                                                           int shared, int D, int chunk, float *out_f32,
                                                           uint16_t *out_bf16) {
    const int q4 = D >> 2;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= T * q4) return;
    const int t = i / q4, c = 4 * (i - t * q4);
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    if (chunk <= 0) {
        for (int j0 = 0; j0 < kk; j0 += 8) {
            int r[8];
            float4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) r[u] = j0 + u < kk ? row_slot[t * kk + j0 + u] : -1;
#pragma unroll
            for (int u = 0; u < 8; ++u)
                v[u] = r[u] >= 0 ? *(const float4 *)(y + (size_t)r[u] * D + c) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                if (r[u] < 0) continue;
                acc[0] += v[u].x;
                acc[1] += v[u].y;
                acc[2] += v[u].z;
                acc[3] += v[u].w;
            }
        }
    } else {
        const auto group = [&](int j) { return (j < k ? idx[t * k + j] : shared) / chunk; };
        for (int prev = -1;;) {
            int gmin = INT_MAX;
            for (int j = 0; j < kk; ++j)
                if (row_slot[t * kk + j] >= 0) {
                    const int g = group(j);
                    if (g > prev && g < gmin) gmin = g;
                }
            if (gmin == INT_MAX) break;
            float part[4] = {0.f, 0.f, 0.f, 0.f};
            for (int j = 0; j < kk; ++j) {
                const int r = row_slot[t * kk + j];
                if (r < 0 || group(j) != gmin) continue;
                const float4 v = *(const float4 *)(y + (size_t)r * D + c);
                part[0] += v.x;
                part[1] += v.y;
                part[2] += v.z;
                part[3] += v.w;
            }
#pragma unroll
            for (int h = 0; h < 4; ++h) acc[h] += round_bf16(part[h]);
            prev = gmin;
        }
    }
    if (out_f32) *(float4 *)(out_f32 + (size_t)t * D + c) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    if (out_bf16) {
        uint2 b;
        b.x = f32_to_bf16_rne(acc[0]) | (f32_to_bf16_rne(acc[1]) << 16);
        b.y = f32_to_bf16_rne(acc[2]) | (f32_to_bf16_rne(acc[3]) << 16);
        *(uint2 *)(out_bf16 + (size_t)t * D + c) = b;
    }
}

struct PfLayout {
    int S, G, P;
    long long Rp;
    size_t off_be, off_nb, off_bn, off_tr, off_wr, off_rs, off_h, off_y, off_part, off_cnt, total;
};

// Workgroups of a grouped GEMM launch resident at once: 2 per CU (the 77 KB of LDS and <= 256 VGPRs per wavefront
// of prefill_kernel).  The launches split their last round's tasks by it (prefill_gemm.h).
static int pf_slots() {
    static int slots = 0;
    if (!slots) {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        slots = 2 * cus;
    }
    return slots;
}

static size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

// y holds bf16 rows for the ragged and XLA-gather forms, f32 rows for the sweeps
static bool pf_y32(int combine) { return combine == MI_COMBINE_SWEEP || combine == MI_COMBINE_XLA_SWEEP; }

static PfLayout pf_layout(int T, int kk, int E, int I, int D, bool y32) {
    PfLayout L{};
    L.S = T * kk;
    L.G = (L.S + kPfTm - 1) / kPfTm + E;
    L.Rp = (long long)L.G * kPfTm;
    size_t o = 0;
    L.off_be = o; o = al256(o + 4 * (size_t)L.G);
    L.off_nb = o; o = al256(o + 4);
    L.off_bn = o; o = al256(o + 4 * (size_t)L.G);
    L.off_tr = o; o = al256(o + 4 * (size_t)L.Rp);
    L.off_wr = o; o = al256(o + 4 * (size_t)L.Rp);
    L.off_rs = o; o = al256(o + 4 * (size_t)L.S);
    L.off_h = o; o = al256(o + 2 * (size_t)L.Rp * I);
    L.off_y = o; o = al256(o + (y32 ? 4 : 2) * (size_t)L.Rp * D);
    L.P = pf_slots();
    L.off_part = o; o = al256(o + (size_t)L.P * kPfPartBytes);
    L.off_cnt = o; o = al256(o + 4 * (size_t)L.P);
    L.total = o;
    return L;
}

static Cb3Table pf_table(const mi_table *t) {
    Cb3Table c{};
    c.qs = t->plane[0];
    c.cb = t->plane[1];
    c.R = t->rows;
    c.K = t->cols;
    c.CT = (t->cols + kCb3TileCols - 1) / kCb3TileCols;
    c.RT = t->rows / 16;
    c.G = t->cols / 128;
    return c;
}

static Iq3Table pf_iq3_table(const mi_table *t) {
    Iq3Table c{};
    c.qs = t->plane[0];
    c.sg = t->plane[1];
    c.qh = t->plane[2];
    c.sc = t->plane[3];
    c.d = t->plane[4];
    c.R = t->rows;
    c.K = t->cols;
    c.nblk = t->cols / 256;
    c.W = 16 * c.nblk;
    return c;
}

static KqTable pf_kq_table(const mi_table *t) {
    const bool q3 = t->qtype == MI_QT_Q3_K;
    KqTable c{};
    c.qs = t->plane[0];
    c.hm = q3 ? t->plane[1] : nullptr;
    c.sc = t->plane[q3 ? 2 : 1];
    c.d = t->plane[q3 ? 3 : 2];
    c.R = t->rows;
    c.K = t->cols;
    c.nblk = t->cols / 256;
    return c;
}

static Iq2Table pf_iq2_table(const mi_table *t) {
    Iq2Table c{};
    c.qs = t->plane[0];
    c.sg = t->plane[1];
    c.qh = t->plane[2];
    c.sc = t->plane[3];
    c.d = t->plane[4];
    c.R = t->rows;
    c.K = t->cols;
    c.nblk = t->cols / 256;
    c.W = 8 * c.nblk;
    return c;
}

static Iq4Table pf_iq4_table(const mi_table *t) {
    Iq4Table c{};
    c.qs = t->plane[0];
    c.sl = t->plane[1];
    c.sh = t->plane[2];
    c.d = t->plane[3];
    c.R = t->rows;
    c.K = t->cols;
    c.nblk = t->cols / 256;
    c.W = 32 * c.nblk;
    return c;
}

// Gate and up share one format, down may use another: CB3 (code tiles), IQ2_S, IQ3_S, IQ4_XS, Q2_K or Q3_K (the
// reference's planes, whole 256-weight blocks).
static int pf_validate(const mi_table *g, const mi_table *u, const mi_table *d) {
    if (!g || !u || !d) return MI_ERR_NULL;
    for (const mi_table *t : {g, u, d}) {
        if (t->qtype < MI_QT_CB3 || t->qtype > MI_QT_Q3_K) return MI_ERR_QTYPE;
        const int np = t->qtype == MI_QT_CB3 ? 2 : t->qtype == MI_QT_Q2_K ? 3
                     : (t->qtype == MI_QT_IQ4_XS || t->qtype == MI_QT_Q3_K) ? 4 : 5;
        for (int i = 0; i < np; ++i)
            if (!t->plane[i]) return MI_ERR_NULL;
        if (t->n_experts <= 0 || t->n_experts > kPlanMaxE || t->cols <= 0 || t->cols % 128 || t->rows <= 0)
            return MI_ERR_SHAPE;
        if (t->qtype != MI_QT_CB3 && t->cols % 256) return MI_ERR_SHAPE;
        // an expert's qs plane stays below 4 GiB (32-bit byte offsets)
        if (t->qtype != MI_QT_CB3 && (long long)(t->cols / 8) * t->rows * 4 >= (1ll << 32)) return MI_ERR_SHAPE;
    }
    if (u->qtype != g->qtype) return MI_ERR_MISMATCH;
    if (g->rows % 128 || d->rows % 256) return MI_ERR_SHAPE;   // whole workgroup row ranges
    if (u->rows != g->rows || u->cols != g->cols || u->n_experts != g->n_experts) return MI_ERR_MISMATCH;
    if (d->cols != g->rows || d->n_experts != g->n_experts) return MI_ERR_MISMATCH;
    return MI_OK;
}

static bool plan_sizes_ok(long long T, long long kk, long long E, long long tm) {
    if (T <= 0 || kk <= 0 || E <= 0 || E > kPlanMaxE || tm <= 0 || tm > 65536) return false;
    const long long S = T * kk;
    if (S > kPlanMaxSlots) return false;
    const long long G = (S + tm - 1) / tm + E;
    return G * tm < (1ll << 31);
}

// The activation buffers are addressed with 32-bit byte offsets: x [T, D], h [Rp, I] and y [Rp, D] stay below 2 GiB.
static bool pf_bytes_ok(long long T, long long kk, long long E, long long I, long long D) {
    const long long Rp = ((T * kk + kPfTm - 1) / kPfTm + E) * kPfTm;
    const long long lim = 1ll << 31;
    return T * D * 2 < lim && Rp * I * 2 < lim && Rp * D * 2 < lim;
}

static int launch_plan(const int32_t *idx, const float *w, int T, int k, int shared, int E, int tm, PlanOut p,
                       hipStream_t s) {
    hipLaunchKernelGGL(ragged_plan_kernel, dim3(1), dim3(kPlanThreads), 0, s, idx, w, T, k, shared, E, tm, p);
    return hipGetLastError() == hipSuccess ? MI_OK : MI_ERR_LAUNCH;
}

}  // namespace mi

using namespace mi;

extern "C" {

int mi_ragged_plan(const int32_t *idx, const float *w, int32_t T, int32_t k, int32_t E, int32_t tm,
                   int32_t *blk_expert, int32_t *n_blocks, int32_t *tok_row, float *w_row, int32_t *row_slot,
                   void *stream) {
    if (!idx || !w || !blk_expert || !n_blocks || !tok_row || !w_row || !row_slot) return MI_ERR_NULL;
    if (T <= 0 || k <= 0) return MI_ERR_TOKENS;
    if (E <= 0 || E > kPlanMaxE || tm <= 0 || tm > 65536) return MI_ERR_ARG;
    if (!plan_sizes_ok(T, k, E, tm)) return MI_ERR_TOKENS;
    PlanOut p{blk_expert, n_blocks, tok_row, w_row, row_slot, nullptr, 0, nullptr, 0};
    return launch_plan(idx, w, T, k, -1, E, tm, p, (hipStream_t)stream);
}

size_t mi_moe_prefill_form_workspace(const mi_table *gate, const mi_table *down, int32_t T, int32_t k,
                                     int32_t shared_expert, int32_t combine) {
    if (!gate || !down || k <= 0 || combine < MI_COMBINE_MATMUL || combine > MI_COMBINE_XLA_SWEEP) return 0;
    const int kk = k + (shared_expert >= 0 ? 1 : 0);
    if (!plan_sizes_ok(T, kk, gate->n_experts, kPfTm) || !pf_bytes_ok(T, kk, gate->n_experts, gate->rows, down->rows))
        return 0;
    return pf_layout(T, kk, gate->n_experts, gate->rows, down->rows, pf_y32(combine)).total;
}

size_t mi_moe_prefill_workspace(const mi_table *gate, const mi_table *down, int32_t T, int32_t k,
                                int32_t shared_expert) {
    return mi_moe_prefill_form_workspace(gate, down, T, k, shared_expert, MI_COMBINE_MATMUL);
}

int mi_moe_prefill(const mi_table *gate, const mi_table *up, const mi_table *down, const uint16_t *x_bf16, int32_t T,
                   int32_t k, const int32_t *idx, const float *w, int32_t shared_expert, float limit, int32_t combine,
                   float *out_f32, uint16_t *out_bf16, void *workspace, size_t workspace_bytes, void *stream) {
    if (combine != MI_COMBINE_MATMUL && combine != MI_COMBINE_GATHER) return MI_ERR_ARG;
    return mi_moe_prefill_form(gate, up, down, x_bf16, T, k, idx, w, shared_expert, limit, combine, 0, out_f32,
                               out_bf16, workspace, workspace_bytes, stream);
}

int mi_moe_prefill_form(const mi_table *gate, const mi_table *up, const mi_table *down, const uint16_t *x_bf16,
                        int32_t T, int32_t k, const int32_t *idx, const float *w, int32_t shared_expert, float limit,
                        int32_t combine, int32_t chunk, float *out_f32, uint16_t *out_bf16, void *workspace,
                        size_t workspace_bytes, void *stream) {
    int st;
    if ((st = pf_validate(gate, up, down))) return st;
    if (!x_bf16 || !idx || !w || (!out_f32 && !out_bf16)) return MI_ERR_NULL;
    // the combine writes 8 columns per thread as 16-byte pieces
    if ((uintptr_t)out_f32 % 16 || (uintptr_t)out_bf16 % 16 || (uintptr_t)workspace % 16) return MI_ERR_ARG;
    const int E = gate->n_experts, I = gate->rows, D = down->rows;
    if (T <= 0 || k <= 0) return MI_ERR_TOKENS;
    if (shared_expert >= E || shared_expert < -1) return MI_ERR_ARG;
    const int kk = k + (shared_expert >= 0 ? 1 : 0);
    if (!plan_sizes_ok(T, kk, E, kPfTm) || !pf_bytes_ok(T, kk, E, I, D)) return MI_ERR_TOKENS;
    if (!(limit > 0.0f) || combine < MI_COMBINE_MATMUL || combine > MI_COMBINE_XLA_SWEEP) return MI_ERR_ARG;
    if (combine == MI_COMBINE_XLA_SWEEP && chunk <= 0) return MI_ERR_ARG;
    const bool y32 = pf_y32(combine);
    const PfLayout L = pf_layout(T, kk, E, I, D, y32);
    if (!workspace || workspace_bytes < L.total) return MI_ERR_WORKSPACE;
    char *ws = (char *)workspace;
    hipStream_t s = (hipStream_t)stream;
    PlanOut p;
    p.blk_expert = (int32_t *)(ws + L.off_be);
    p.n_blocks = (int32_t *)(ws + L.off_nb);
    p.blk_n = (int32_t *)(ws + L.off_bn);
    p.tok_row = (int32_t *)(ws + L.off_tr);
    p.w_row = (float *)(ws + L.off_wr);
    p.row_slot = (int32_t *)(ws + L.off_rs);
    p.merge_dups = y32;
    p.cnt = (uint32_t *)(ws + L.off_cnt);
    p.n_cnt = L.P;
    uint16_t *h = (uint16_t *)(ws + L.off_h), *y = (uint16_t *)(ws + L.off_y);
    if ((st = launch_plan(idx, w, T, k, shared_expert, E, kPfTm, p, s))) return st;

    PfArgs a{};
    if (gate->qtype == MI_QT_IQ3_S) {
        a.i0 = pf_iq3_table(gate);
        a.i1 = pf_iq3_table(up);
    } else if (gate->qtype == MI_QT_IQ4_XS) {
        a.k0 = pf_iq4_table(gate);
        a.k1 = pf_iq4_table(up);
    } else if (gate->qtype == MI_QT_IQ2_S) {
        a.j0 = pf_iq2_table(gate);
        a.j1 = pf_iq2_table(up);
    } else if (gate->qtype == MI_QT_Q2_K || gate->qtype == MI_QT_Q3_K) {
        a.q0 = pf_kq_table(gate);
        a.q1 = pf_kq_table(up);
    } else {
        a.t0 = pf_table(gate);
        a.t1 = pf_table(up);
    }
    a.R = I;
    a.K = gate->cols;
    a.blk_expert = p.blk_expert;
    a.blk_n = p.blk_n;
    a.n_blocks = p.n_blocks;
    a.tok_row = p.tok_row;
    a.x = x_bf16;
    a.x_bytes = (uint32_t)((size_t)T * a.K * 2);
    a.gather = 1;
    a.out = h;
    a.limit = limit;
    a.wg_rows = 2;
    a.RBG = I / 128;
    a.w_row = p.w_row;
    a.P = L.P;
    a.part = (float *)(ws + L.off_part);
    a.cnt = p.cnt;
    // blocks rounded up to whole XCD rounds, then the split tasks' pieces (at most P)
    const int g8 = (L.G + kXcds - 1) / kXcds * kXcds;
    const bool round_gu = combine == MI_COMBINE_XLA_GATHER || combine == MI_COMBINE_XLA_SWEEP;
    const dim3 ggu(g8 * a.RBG + L.P);
    if ((st = y32 ? (round_gu ? launch_prefill_0_3(gate->qtype, ggu, s, a) : launch_prefill_0_2(gate->qtype, ggu, s, a))
                  : (round_gu ? launch_prefill_0_1(gate->qtype, ggu, s, a) : launch_prefill_0_0(gate->qtype, ggu, s, a))))
        return st;

    PfArgs b = a;
    if (down->qtype == MI_QT_IQ3_S) b.i0 = b.i1 = pf_iq3_table(down);
    else if (down->qtype == MI_QT_IQ4_XS) b.k0 = b.k1 = pf_iq4_table(down);
    else if (down->qtype == MI_QT_IQ2_S) b.j0 = b.j1 = pf_iq2_table(down);
    else if (down->qtype == MI_QT_Q2_K || down->qtype == MI_QT_Q3_K) b.q0 = b.q1 = pf_kq_table(down);
    else b.t0 = b.t1 = pf_table(down);
    b.R = D;
    b.K = I;
    b.x = h;
    b.x_bytes = (uint32_t)(L.Rp * I * 2);
    b.gather = 0;
    b.out = y;
    b.wg_rows = 4;
    b.RBG = D / 256;
    b.out32 = (float *)y;
    const dim3 gdn(g8 * b.RBG + L.P);
    if ((st = y32 ? launch_prefill_1_4(down->qtype, gdn, s, b) : launch_prefill_1_0(down->qtype, gdn, s, b))) return st;

    if (y32) {
        const long long nthr = (long long)T * (D / 4);
        hipLaunchKernelGGL(prefill_combine_f32, dim3((unsigned)((nthr + 255) / 256)), dim3(256), 0, s,
                           (const float *)y, (const int32_t *)p.row_slot, idx, T, k, kk, shared_expert, D,
                           combine == MI_COMBINE_XLA_SWEEP ? chunk : 0, out_f32, out_bf16);
    } else {
        const long long nthr = (long long)T * (D / 8);
        hipLaunchKernelGGL(prefill_combine, dim3((unsigned)((nthr + 255) / 256)), dim3(256), 0, s,
                           (const uint16_t *)y, (const int32_t *)p.row_slot, w, T, k, kk, D,
                           combine == MI_COMBINE_MATMUL ? 1 : 0, out_f32, out_bf16);
    }
    return hipGetLastError() == hipSuccess ? MI_OK : MI_ERR_LAUNCH;
}

}  // extern "C"
