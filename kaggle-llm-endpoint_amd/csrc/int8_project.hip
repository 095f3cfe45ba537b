// int8 projections for gfx950: y = x @ bf16(f32(q) * s)   (quant8.py:91-99 + the x @ W uses), with the reference's
// per-output-column scales s [1, out] or per-input-row scales s [in, 1] (quant8.py:26-32,59-60), and the lm_head
// form y = (x @ f32(q)) * s[o], the scale applied after the dot (engine.py:345-351).
//
// Weights qT [n_out, n_in] int8 (input-contiguous) stream once from HBM; every wavefront owns a 16-row tile of
// outputs and one column split.  A lane loads 32 consecutive int8 of its row per 128-column block (4 lanes = one
// 128-byte line per row), dequantizes them in registers to exactly the reference's bf16(f32(q) * s):
//   f32: fma(q + 128, s, -128 s) rounds q * s once (q + 128 is an unsigned byte, so one v_cvt_f32_ubyte each);
//   bf16: round to nearest even (v_cvt_pk_bf16_f32)
// (per-row scales: the element's own s[i], staged in LDS beside the activations; the lm_head form: q itself, exact
// in bf16) and feeds v_mfma_f32_16x16x32_bf16 (bf16 x bf16 products are exact, f32 accumulation) with the staged
// activations as the B operand (up to 16 tokens per tile).  Inside a block the lane's 32 bytes are 4 k-steps of 8 columns:
// step c of block p uses columns 128p + 32q + 8c .. +7 (q = lane / 16) for both operands.  Splits write f32
// partials; the workgroup of a row group that completes last adds every split's partial in split order (the same
// order whichever completes last) and writes y -- or, for an MLP's gate/up pair, h -- so the sums need no launch of
// their own (completion counters in the workspace; split_reduce_i8 / swiglu_pair_i8 when there are too many row
// groups for them).  One split writes y directly.
//
// The same kernels take bf16 weights wT [n_out, n_in] (the reference's non-int8 leaves, x @ W with W bf16 [in, out]
// transposed once at load): blocks of 64 columns (the same 128 bytes per row), a lane's two 16-byte loads are its two
// k-steps directly -- step c of block p uses columns 64p + 32c + 8q .. +7 -- with no scale and no conversion.
#include "common.h"
#include "tuning.h"

#include <stdlib.h>

#include <algorithm>

namespace mi {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kI8MaxProj = 8;      // projections sharing one activation matrix per launch
constexpr int kW16 = 3;            // weight form beside the MI_I8_* scale forms: bf16 weights, no scales

struct I8Proj {
    const int8_t *q;       // [n_out, n_in] (int8; bf16 with the kW16 form: 2 n_in bytes per row)
    const float *s;        // [n_out] (MI_I8_COL_SCALES, MI_I8_COL_AFTER) or [n_in] (MI_I8_ROW_SCALES); kW16: unused
    int n_out;
    uint16_t *y_bf16;      // [B, n_out] (S == 1)
    float *y_f32;          // [B, n_out] (S == 1)
    float *part;           // [S, B, n_out] (S > 1)
};

struct I8Args {
    const uint16_t *x;     // bf16 [B, n_in], shared by every projection
    int B, n_in, S;
    int scale_axis;        // MI_I8_* or kW16: one per launch
    int tiled;             // qT in the tiled layout (mi_int8_tile): 2 KB per (128-column block, 16-row tile)
    int blocks;            // blocks per split: 128 columns (int8) or 64 (kW16), 2 KB per 16-row tile either way
    int n_proj;
    int wg_start[kI8MaxProj + 1];   // first workgroup of each projection
    I8Proj p[kI8MaxProj];
    int pair;              // 1: projections 0 and 1 are gate and up of an MLP: partials always (swiglu_pair_i8)
    float limit;           // pair: the SwiGLU clamp
    uint16_t *h;           // pair: h [B, n_out of projection 0] bf16
    uint32_t *cnt;         // completion counters, one per row group (zero between launches); null: separate sums
    int ctr_start[kI8MaxProj];      // first counter of each projection (a pair's gate and up share theirs)
};

// Counters per launch, each on its own 128-byte line (a line's atomics are serialised); an int8 workspace starts
// with two such blocks (the MLP's gate/up and down launches).
constexpr int kI8Ctrs = 1024;
constexpr int kI8CtrStride = 32;        // words
constexpr size_t kI8CtrBytes = 2 * 4 * (size_t)kI8Ctrs * kI8CtrStride;
constexpr int kI8StoreThrough = 16;     // sc1 store: through this XCD's L2 to memory

constexpr int kI8Waves = 4;
constexpr int kI8Ring = 4;          // 128-column blocks in flight per wavefront (2 KB each)
#ifndef MI_I8_NT
#define MI_I8_NT 1
#endif
constexpr int kI8LoadPolicy = MI_I8_NT ? 2 : 0;   // the weights are read once per launch: non-temporal (nt) loads
constexpr int kBufWord3 = 0x00020000;   // gfx9 buffer descriptor word 3 (32-bit data format)
constexpr uint32_t kI8Out = 0x80000000u; // buffer offset past every source's range: the load returns zeros

// LDS pitch (dwords) of a staged activation row of cw dwords: whole 64-dword chunks (a direct-to-LDS load writes 64
// lanes x 4 bytes) plus a 4-dword skew, so the 16 rows of a B-operand read spread over the LDS banks.
__host__ __device__ constexpr int i8_pitch(int cw) { return ((cw + 63) & ~63) + 4; }

__device__ __forceinline__ uint32_t bf16_pair(float a, float b) {
    const bf16x2 v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
}

// 8 int8 weights (two dwords) of one row -> 8 bf16 = bf16(f32(q) * s), round to nearest even.
__device__ __forceinline__ bf16x8 i8_weights8(uint32_t w0, uint32_t w1, float s, float ns128) {
    const uint32_t u0 = w0 ^ 0x80808080u, u1 = w1 ^ 0x80808080u;       // q + 128, unsigned bytes
    uint4 v;
    v.x = bf16_pair(fmaf((float)(u0 & 255u), s, ns128), fmaf((float)((u0 >> 8) & 255u), s, ns128));
    v.y = bf16_pair(fmaf((float)((u0 >> 16) & 255u), s, ns128), fmaf((float)(u0 >> 24), s, ns128));
    v.z = bf16_pair(fmaf((float)(u1 & 255u), s, ns128), fmaf((float)((u1 >> 8) & 255u), s, ns128));
    v.w = bf16_pair(fmaf((float)((u1 >> 16) & 255u), s, ns128), fmaf((float)(u1 >> 24), s, ns128));
    return __builtin_bit_cast(bf16x8, v);
}

// 8 int8 weights of one row with their own scales s[0..7] (per-input-row scales) -> bf16(f32(q) * s), as above.
__device__ __forceinline__ bf16x8 i8_weights8_rs(uint32_t w0, uint32_t w1, float4 sa, float4 sb) {
    const uint32_t u0 = w0 ^ 0x80808080u, u1 = w1 ^ 0x80808080u;
    uint4 v;
    v.x = bf16_pair(fmaf((float)(u0 & 255u), sa.x, -128.0f * sa.x), fmaf((float)((u0 >> 8) & 255u), sa.y, -128.0f * sa.y));
    v.y = bf16_pair(fmaf((float)((u0 >> 16) & 255u), sa.z, -128.0f * sa.z), fmaf((float)(u0 >> 24), sa.w, -128.0f * sa.w));
    v.z = bf16_pair(fmaf((float)(u1 & 255u), sb.x, -128.0f * sb.x), fmaf((float)((u1 >> 8) & 255u), sb.y, -128.0f * sb.y));
    v.w = bf16_pair(fmaf((float)((u1 >> 16) & 255u), sb.z, -128.0f * sb.z), fmaf((float)(u1 >> 24), sb.w, -128.0f * sb.w));
    return __builtin_bit_cast(bf16x8, v);
}

// token tiles of 16 (B <= 16 * TT); SA: MI_I8_* scale form or kW16 (bf16 weights); SUMS: the split sums in the
// launch (a.cnt set)
template <int TT, int SA, bool SUMS>
__global__ void __launch_bounds__(64 * kI8Waves) int8_project_kernel(I8Args a) {
    constexpr bool W16 = SA == kW16;
    constexpr int kCols = W16 ? 64 : 128;            // columns per block
    extern __shared__ uint32_t xs[];                 // [B][cols / 2] bf16 pairs of the split's columns (+ row scales)
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int pj = 0;
    while (pj + 1 < a.n_proj && (int)blockIdx.x >= a.wg_start[pj + 1]) ++pj;
    const I8Proj &P = a.p[pj];
    const int local = blockIdx.x - a.wg_start[pj];
    const int row_groups = (P.n_out + 16 * kI8Waves - 1) / (16 * kI8Waves);
    const int rg = local % row_groups, split = local / row_groups;
    const int o0 = (rg * kI8Waves + wave) * 16;
    const bool active = o0 < P.n_out;                // wavefronts past the last 16-row tile only stage (and count)
    const int i = lane & 15, q = lane >> 4;
    const int cols = kCols * a.blocks, k0 = split * cols;

    // weights: lane's 32 bytes of block p at row o0 + i, columns k0 + 128 p + 32 q, as buffer loads from the
    // wavefront's tile (blocks past the split, and every block of a wavefront past the last row tile, use an
    // empty-range descriptor: zeros, no memory traffic)
    // row layout: row o0 + i at n_in bytes per row, block p at +128 p, the lane's two 16-byte halves 16 apart;
    // tiled layout: 2 KB per (128-column block, 16-row tile), blocks outermost, the lane's halves at lane * 16 and
    // 1024 + lane * 16: every load instruction reads 1 KB of contiguous memory, and the wavefronts working on one
    // block read neighbouring kilobytes;
    // bf16 rows: row o0 + i at 2 n_in bytes per row, block p at +128 p, the lane's k-steps at +16 q and +64 + 16 q
    const int8_t *tile = W16 ? P.q + 2 * ((size_t)(active ? o0 : 0) * a.n_in + k0)
                         : a.tiled ? P.q + ((size_t)(k0 / 128) * (P.n_out / 16) + (active ? o0 / 16 : 0)) * 2048
                                   : P.q + (size_t)(active ? o0 : 0) * a.n_in + k0;
    const int bstride = a.tiled ? (P.n_out / 16) * 2048 : 128, hoff = a.tiled ? 1024 : W16 ? 64 : 16;
    const __amdgpu_buffer_rsrc_t qb =
        __builtin_amdgcn_make_buffer_rsrc((void *)tile, (short)0, active ? 0x7fffffff : 0, kBufWord3);
    const __amdgpu_buffer_rsrc_t qnull = __builtin_amdgcn_make_buffer_rsrc((void *)tile, (short)0, 0, kBufWord3);
    const int voff = W16 ? 2 * i * a.n_in + 16 * q : a.tiled ? 16 * lane : i * a.n_in + 32 * q;
    auto load_block = [&](int p, uint4 &lo, uint4 &hi) {
        const __amdgpu_buffer_rsrc_t r = p < a.blocks ? qb : qnull;
        lo = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, bstride * p, kI8LoadPolicy));
        hi = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff + hoff, bstride * p, kI8LoadPolicy));
    };
    // per-column scales: the row's s; the lm_head form: q itself (scale 1 here, s[o] after the sum).  Loaded first:
    // a load issued after the ring could only be waited for together with it.
    const float sc = SA == MI_I8_COL_SCALES && active ? P.s[o0 + i] : 1.0f;
    // stage the split's activations (bf16 pairs, rows < B, row pitch xsp dwords) and, with per-row scales, its
    // s[k0 .. k0 + cols) straight into LDS -- direct-to-LDS loads, 64 lanes x 16 or 4 bytes each, no registers -- issued
    // ahead of the weight ring: loads complete in issue order, so waiting for all but the ring's loads waits for the
    // activations only, and the ring keeps streaming while the workgroup meets at the barrier
    const int cw = cols / 2, xsp = i8_pitch(cw);
    float *srow = (float *)(xs + a.B * xsp);
    {
        const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void *)a.x, (short)0, 0x7fffffff, kBufWord3);
        const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc((void *)P.s, (short)0, 0x7fffffff, kBufWord3);
        // whole 256-dword chunks of a row with 16 bytes per lane when the row start and the columns are multiples of 8
        // (a lane then wholly inside or past the columns), the rest with 4: an LDS-bound load costs about as much
        // per instruction whatever its width
        const int n16 = ((a.n_in | k0 | cols) & 7) == 0 ? cw >> 8 : 0, nt = (cw - 256 * n16 + 63) >> 6;
        for (int e = wave; e < a.B * n16; e += kI8Waves) {
            const int b = e / n16, ch = e - b * n16, d = 256 * ch + 4 * lane;
            const uint32_t voff = d < cw ? (uint32_t)(((size_t)b * a.n_in + k0) * 2 + 4 * d) : kI8Out;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (__attribute__((address_space(3))) void *)(xs + b * xsp + 256 * ch),
                                                     16, voff, 0, 0, 0);
        }
        const int nrow = a.B * nt, n = nrow + (SA == MI_I8_ROW_SCALES ? cols / 64 : 0);
        for (int e = wave; e < n; e += kI8Waves) {
            if (e < nrow) {
                const int b = e / nt, d0 = 256 * n16 + 64 * (e - b * nt), d = d0 + lane;
                const uint32_t voff = d < cw ? (uint32_t)(((size_t)b * a.n_in + k0) * 2 + 4 * d) : kI8Out;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (__attribute__((address_space(3))) void *)(xs + b * xsp + d0),
                                                         4, voff, 0, 0, 0);
            } else {
                const int ch = e - nrow;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (__attribute__((address_space(3))) void *)(srow + 64 * ch), 4,
                                                         (k0 + 64 * ch + lane) * 4, 0, 0, 0);
            }
        }
    }
    uint4 ring[kI8Ring][2];
#pragma unroll
    for (int d = 0; d < kI8Ring; ++d) load_block(d, ring[d][0], ring[d][1]);
    vm_wait<2 * kI8Ring>();                          // every load but the ring's
    lds_barrier();                                   // the ring stays in flight
    if (!active && !SUMS) return;
    const float ns128 = -128.0f * sc;

    f32x4 acc[TT];
#pragma unroll
    for (int t = 0; t < TT; ++t) acc[t] = (f32x4){0.f, 0.f, 0.f, 0.f};
    // B-operand rows: token jt of tile t (rows >= B read row B-1; those accumulator columns are not stored)
    const uint32_t *xrow[TT];
#pragma unroll
    for (int t = 0; t < TT; ++t) xrow[t] = xs + min(16 * t + i, a.B - 1) * xsp + (W16 ? 4 : 16) * q;

    // block p of the split against the staged activations
    auto consume = [&](int p, uint4 w0, uint4 w1) {
        if constexpr (W16) {                          // the loads are the A operands (columns 64p + 32c + 8q ..)
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const bf16x8 A = __builtin_bit_cast(bf16x8, c ? w1 : w0);
#pragma unroll
                for (int t = 0; t < TT; ++t) {
                    const uint4 xv = *(const uint4 *)(xrow[t] + 32 * p + 16 * c);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, __builtin_bit_cast(bf16x8, xv), acc[t], 0, 0,
                                                                     0);
                }
            }
        } else {
            const uint32_t W[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                bf16x8 A;
                if constexpr (SA == MI_I8_ROW_SCALES) {
                    const float *sp = srow + 128 * p + 32 * q + 8 * c;
                    A = i8_weights8_rs(W[2 * c], W[2 * c + 1], *(const float4 *)sp, *(const float4 *)(sp + 4));
                } else {
                    A = i8_weights8(W[2 * c], W[2 * c + 1], sc, ns128);
                }
#pragma unroll
                for (int t = 0; t < TT; ++t) {
                    const uint4 xv = *(const uint4 *)(xrow[t] + 64 * p + 4 * c);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, __builtin_bit_cast(bf16x8, xv), acc[t], 0, 0,
                                                                     0);
                }
            }
        }
    };
    // whole groups of kI8Ring blocks: each slot refilled right after it is consumed (blocks past the split load zeros
    // from the empty-range descriptor), no branch inside a group and the order pinned, so every slot keeps its
    // registers and a block waits only for its own loads; then the 0 .. kI8Ring - 1 blocks left, already in the ring
    const int groups = active ? a.blocks / kI8Ring : 0;
    for (int g = 0; g < groups; ++g) {
#pragma unroll
        for (int d = 0; d < kI8Ring; ++d) {
            const int p = g * kI8Ring + d;
            __builtin_amdgcn_sched_barrier(0);
            consume(p, ring[d][0], ring[d][1]);
            __builtin_amdgcn_sched_barrier(0);
            load_block(p + kI8Ring, ring[d][0], ring[d][1]);
        }
    }
    const int rest = active ? a.blocks - groups * kI8Ring : 0;
#pragma unroll
    for (int d = 0; d < kI8Ring - 1; ++d)
        if (d < rest) consume(groups * kI8Ring + d, ring[d][0], ring[d][1]);
    // C layout: lane (jt = lane % 16, q) holds output rows o0 + 4q + r for token 16 t + jt
    const int o = o0 + 4 * q;
    if constexpr (SUMS) {
        // the split's partial goes to memory (stored through this XCD's L2), then the row group is counted; the
        // workgroup that counts last adds all of them in split order.  Nothing waits for another workgroup.  The
        // partials are read with device-coherent (sc1) loads after the count: a 128-byte line may hold partials of
        // two row groups (n_out % 32 == 16, or a workspace aligned to 16 bytes only), and the other row group's last
        // workgroup may have pulled it into this XCD's L2 before every split had stored its part.  The flag lives in
        // xs[0]: past the first barrier no wavefront reads the activations (a static __shared__ word would move xs
        // off its 16-byte alignment).
        if (active) {
            const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
                (void *)(P.part + (size_t)split * a.B * P.n_out), (short)0, 0x7fffffff, kBufWord3);
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                const int b = 16 * t + i;
                if (b < a.B)
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[t]), pr,
                                                           (b * P.n_out + o) * 4, 0, kI8StoreThrough);
            }
        }
        __builtin_amdgcn_s_waitcnt(0);              // this wavefront's stores have completed
        __syncthreads();                            // ... and every wavefront's
        uint32_t *ctr = a.cnt + (a.ctr_start[pj] + rg) * kI8CtrStride;
        if (tid == 0) xs[0] = counter_add(ctr, 1u) == (uint32_t)((a.pair ? 2 : 1) * a.S - 1);
        __syncthreads();
        if (!xs[0]) return;
        if (tid == 0) counter_reset(ctr);           // zero again for the next launch
        if (!active) return;
        if (a.pair) {
            // h = bf16(swiglu_clamped(bf16(g), bf16(u))), g and u the split sums of projections 0 and 1
            // (mlp_partial, model.py:119-127), as swiglu_pair_i8
            const __amdgpu_buffer_rsrc_t rg0 =
                __builtin_amdgcn_make_buffer_rsrc((void *)a.p[0].part, (short)0, 0x7fffffff, kBufWord3);
            const __amdgpu_buffer_rsrc_t ru0 =
                __builtin_amdgcn_make_buffer_rsrc((void *)a.p[1].part, (short)0, 0x7fffffff, kBufWord3);
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                const int b = 16 * t + i;
                if (b >= a.B) continue;
                f32x4 g = (f32x4){0.f, 0.f, 0.f, 0.f}, u = g;
                for (int s0 = 0; s0 < a.S; s0 += 4) {      // 8 loads in flight, added in split order
                    f32x4 pg[4], pu[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint32_t e = (uint32_t)((((size_t)(s0 + j) * a.B + b) * P.n_out + o) * 4);
                        const bool in = s0 + j < a.S;
                        pg[j] = in ? coherent_load4(rg0, e) : (f32x4){0.f, 0.f, 0.f, 0.f};
                        pu[j] = in ? coherent_load4(ru0, e) : (f32x4){0.f, 0.f, 0.f, 0.f};
                    }
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        g += pg[j];
                        u += pu[j];
                    }
                }
                uint2 v;
                v.x = f32_to_bf16_rne(swiglu_clamped(round_bf16(g.x), round_bf16(u.x), a.limit)) |
                      (f32_to_bf16_rne(swiglu_clamped(round_bf16(g.y), round_bf16(u.y), a.limit)) << 16);
                v.y = f32_to_bf16_rne(swiglu_clamped(round_bf16(g.z), round_bf16(u.z), a.limit)) |
                      (f32_to_bf16_rne(swiglu_clamped(round_bf16(g.w), round_bf16(u.w), a.limit)) << 16);
                *(uint2 *)(a.h + (size_t)b * P.n_out + o) = v;
            }
            return;
        }
        // y = the split sums in split order, as split_reduce_i8
        const __amdgpu_buffer_rsrc_t rp =
            __builtin_amdgcn_make_buffer_rsrc((void *)P.part, (short)0, 0x7fffffff, kBufWord3);
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            const int b = 16 * t + i;
            f32x4 v = (f32x4){0.f, 0.f, 0.f, 0.f};
            if (b < a.B)
                for (int s0 = 0; s0 < a.S; s0 += 8) {       // 8 loads in flight, added in split order
                    f32x4 pv[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        pv[j] = s0 + j < a.S
                                    ? coherent_load4(rp, (uint32_t)((((size_t)(s0 + j) * a.B + b) * P.n_out + o) * 4))
                                    : (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int j = 0; j < 8; ++j) v += pv[j];
                }
            acc[t] = v;
        }
    } else if (!active) {
        return;
    }
    if constexpr (SA == MI_I8_COL_AFTER) {          // the lm_head form: scale after the whole sum
        if (a.S == 1 || SUMS) {
            const float4 so = *(const float4 *)(P.s + o);
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                acc[t][0] *= so.x; acc[t][1] *= so.y; acc[t][2] *= so.z; acc[t][3] *= so.w;
            }
        }
    }
#pragma unroll
    for (int t = 0; t < TT; ++t) {
        const int b = 16 * t + i;
        if (b >= a.B) continue;
        if ((a.S == 1 && !a.pair) || SUMS) {
            if (P.y_f32) *(float4 *)(P.y_f32 + (size_t)b * P.n_out + o) = make_float4(acc[t][0], acc[t][1], acc[t][2], acc[t][3]);
            if (P.y_bf16) {
                uint2 v;
                v.x = f32_to_bf16_rne(acc[t][0]) | (f32_to_bf16_rne(acc[t][1]) << 16);
                v.y = f32_to_bf16_rne(acc[t][2]) | (f32_to_bf16_rne(acc[t][3]) << 16);
                *(uint2 *)(P.y_bf16 + (size_t)b * P.n_out + o) = v;
            }
        } else {
            *(float4 *)(P.part + ((size_t)split * a.B + b) * P.n_out + o) = make_float4(acc[t][0], acc[t][1], acc[t][2],
                                                                                     acc[t][3]);
        }
    }
}

// y[b, o] = sum_s part[s, b, o] of every projection, splits in order; f32 and/or bf16 out.  One thread per 4 outputs;
// projection j owns threads [q4_start[j], q4_start[j + 1]).
__global__ void __launch_bounds__(256) split_reduce_i8(I8Args a) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    int pj = 0, base = 0;
    while (pj < a.n_proj && i >= base + a.B * a.p[pj].n_out / 4) base += a.B * a.p[pj++].n_out / 4;
    if (pj >= a.n_proj) return;
    const I8Proj &P = a.p[pj];
    const int n = a.B * P.n_out, li = i - base;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s0 = 0; s0 < a.S; s0 += 8) {             // 8 independent loads in flight, summed in split order
        float4 p[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            p[j] = s0 + j < a.S ? ((const float4 *)(P.part + (size_t)(s0 + j) * n))[li] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            v.x += p[j].x; v.y += p[j].y; v.z += p[j].z; v.w += p[j].w;
        }
    }
    if (a.scale_axis == MI_I8_COL_AFTER) {           // the lm_head form: s[o] after the whole sum
        const float4 so = *(const float4 *)(P.s + 4 * li % P.n_out);
        v.x *= so.x; v.y *= so.y; v.z *= so.z; v.w *= so.w;
    }
    if (P.y_f32) ((float4 *)P.y_f32)[li] = v;
    if (P.y_bf16) {
        uint2 b;
        b.x = f32_to_bf16_rne(v.x) | (f32_to_bf16_rne(v.y) << 16);
        b.y = f32_to_bf16_rne(v.z) | (f32_to_bf16_rne(v.w) << 16);
        ((uint2 *)P.y_bf16)[li] = b;
    }
}

// h[b, o] = bf16(swiglu_clamped(bf16(g), bf16(u))) with g, u the split sums (in split order) of projections 0 and 1:
// mlp_partial's x @ gate and x @ up in bf16, then the clamped SwiGLU in bf16 (model.py:119-127).  One thread per 4
// outputs.
__global__ void __launch_bounds__(256) swiglu_pair_i8(I8Args a) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int no = a.p[0].n_out, n = a.B * no;
    if (i >= n / 4) return;
    float4 g = make_float4(0.f, 0.f, 0.f, 0.f), u = g;
    for (int s0 = 0; s0 < a.S; s0 += 4) {            // 8 independent loads in flight, summed in split order
        float4 pg[4], pu[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const bool in = s0 + j < a.S;
            pg[j] = in ? ((const float4 *)(a.p[0].part + (size_t)(s0 + j) * n))[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            pu[j] = in ? ((const float4 *)(a.p[1].part + (size_t)(s0 + j) * n))[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            g.x += pg[j].x; g.y += pg[j].y; g.z += pg[j].z; g.w += pg[j].w;
            u.x += pu[j].x; u.y += pu[j].y; u.z += pu[j].z; u.w += pu[j].w;
        }
    }
    const float h0 = swiglu_clamped(round_bf16(g.x), round_bf16(u.x), a.limit);
    const float h1 = swiglu_clamped(round_bf16(g.y), round_bf16(u.y), a.limit);
    const float h2 = swiglu_clamped(round_bf16(g.z), round_bf16(u.z), a.limit);
    const float h3 = swiglu_clamped(round_bf16(g.w), round_bf16(u.w), a.limit);
    uint2 b;
    b.x = f32_to_bf16_rne(h0) | (f32_to_bf16_rne(h1) << 16);
    b.y = f32_to_bf16_rne(h2) | (f32_to_bf16_rne(h3) << 16);
    ((uint2 *)a.h)[i] = b;
}

// The tiled layout of qT [n_out, n_in]: per 128-column block b (outermost) and 16-row tile t, 2 KB at
// (b * n_out / 16 + t) * 2048 = two halves of 64 lanes x 16 bytes, lane l = i + 16 q of half h holding row 16 t + i,
// columns 128 b + 32 q + 16 h .. + 15 -- what lane l of the projection kernel loads for block b, so each load
// instruction reads 1 KB of contiguous memory and the wavefronts on one block read neighbouring kilobytes (measured
// 59.3-59.7 against 59.9-60.2 us for the int8 layer with the tiles of one row tile adjacent).  One thread per 16
// bytes.
__global__ void __launch_bounds__(256) int8_tile_kernel(const int8_t *__restrict__ qT, int n_out, int n_in,
                                                        int8_t *__restrict__ out) {
    const int nblk = n_in / 128;
    const size_t n16 = (size_t)n_out * n_in / 16;
    for (size_t d = (size_t)blockIdx.x * blockDim.x + threadIdx.x; d < n16; d += (size_t)gridDim.x * blockDim.x) {
        const int l = (int)(d & 63), h = (int)((d >> 6) & 1);
        const size_t tb = d >> 7, t = tb / nblk;
        const int b = (int)(tb - t * nblk);
        const size_t row = 16 * t + (l & 15), col = 128 * (size_t)b + 32 * (l >> 4) + 16 * h;
        const size_t dst = (((size_t)b * (n_out / 16) + t) * 2 + h) * 64 + l;
        *(uint4 *)(out + 16 * dst) = *(const uint4 *)(qT + row * n_in + col);
    }
}

// LDS bytes of a split of `cols` columns: B staged activation rows at the padded pitch (+ one f32 scale per column
// with per-input-row scales).
static size_t i8_lds_bytes(int B, int cols, int scale_axis) {
    return 4 * ((size_t)B * i8_pitch(cols / 2) + (scale_axis == MI_I8_ROW_SCALES ? (size_t)cols : 0));
}

// Columns per 2 KB block of a 16-row tile: 128 int8 or 64 bf16 weights.
static int i8_block_cols(int form) { return form == kW16 ? 64 : 128; }

// Column splits: enough wavefronts to cover the chip (about 3 per SIMD, 3072 over 256 CUs), every wavefront
// streaming at least 4 blocks (8 KB), the split's staged columns within 48 KB of LDS.  `tiles` counts the 16-row
// tiles of every projection of the launch.
static int i8_splits(int B, int n_in, int tiles, int scale_axis) {
    const int nblk = n_in / i8_block_cols(scale_axis);
    const int forced = tuning(kTuneI8S, 0);       // measurements: a forced split count (must divide the blocks)
    if (forced > 0 && nblk % forced == 0 && i8_lds_bytes(B, n_in / forced, scale_axis) <= 48 * 1024) return forced;
    int target = tuning(kTuneI8Waves, 3072);       // wavefronts to aim for
    if (target <= 0) target = 3072;
    int best = 1;
    for (int S = 1; S <= nblk; ++S) {
        if (nblk % S) continue;
        if (i8_lds_bytes(B, n_in / S, scale_axis) > 48 * 1024) continue;
        if (nblk / S < 4 && S > 1) break;
        best = S;
        if ((long long)tiles * S >= target) break;
    }
    return best;
}

static int i8_tiles(const int32_t *n_out, int n_proj) {
    int t = 0;
    for (int j = 0; j < n_proj; ++j) t += n_out[j] / 16;
    return t;
}

// Partial bytes of one launch: the f32 split partials (none with one split, except for an MLP's gate/up pair,
// whose SwiGLU reads them).
static size_t i8_part_bytes(int B, int n_in, const int32_t *n_out, int n_proj, int scale_axis, int pair) {
    scale_axis &= ~MI_I8_TILED;
    size_t total = 0;
    for (int j = 0; j < n_proj; ++j) total += (size_t)n_out[j];
    const int S = i8_splits(B, n_in, i8_tiles(n_out, n_proj), scale_axis);
    return S == 1 && !pair ? 256 : sizeof(float) * (size_t)S * B * total;
}

static size_t al256_i8(size_t v) { return (v + 255) & ~(size_t)255; }

}  // namespace mi

using namespace mi;

// In-launch split sums (completion counters), a bit mask: 1 for projections, 2 for an MLP's gate/up pair (h formed
// in the launch).  The I8_FUSE override replaces it (measurements and tests of the separate sum kernels).
static int i8_fuse() { return tuning(kTuneI8Fuse, 3); }

// One launch of the projections of `projs` over x (+ the split sums, or with `pair` the SwiGLU of gate and up into
// h): partials at `part` (part_bytes), the launch's counter block at `cnt` (kI8Ctrs counters, zero).  scale_axis:
// MI_I8_* (| MI_I8_TILED) for int8 weights, kW16 for bf16 ones (row layout, no scales).
static int i8_launch(const uint16_t *x_bf16, int32_t B, int32_t n_in, const mi_i8_proj *projs, int32_t n_proj,
                     int32_t scale_axis, float *part, size_t part_bytes, uint32_t *cnt, void *stream, int pair,
                     float limit, uint16_t *h) {
    if (!x_bf16 || !projs) return MI_ERR_NULL;
    if (B <= 0 || B > 32) return MI_ERR_TOKENS;
    if (n_proj <= 0 || n_proj > kI8MaxProj || (pair && n_proj != 2)) return MI_ERR_ARG;
    const int tiled = (scale_axis & MI_I8_TILED) != 0;
    scale_axis &= ~MI_I8_TILED;
    if (scale_axis < MI_I8_ROW_SCALES || scale_axis > kW16 || (tiled && scale_axis == kW16)) return MI_ERR_ARG;
    if (n_in <= 0 || n_in % 256) return MI_ERR_SHAPE;
    int32_t n_out[kI8MaxProj];
    for (int j = 0; j < n_proj; ++j) {
        const mi_i8_proj &p = projs[j];
        if (!p.qT || (!p.s && scale_axis != kW16) || (!pair && !p.y_bf16 && !p.y_f32)) return MI_ERR_NULL;
        if (p.n_out <= 0 || p.n_out % 16) return MI_ERR_SHAPE;
        n_out[j] = p.n_out;
    }
    const size_t need = i8_part_bytes(B, n_in, n_out, n_proj, scale_axis, pair);
    if (!part || part_bytes < need || (uintptr_t)part % 16) return MI_ERR_WORKSPACE;
    I8Args a{};
    a.pair = pair;
    a.limit = limit;
    a.h = h;
    a.x = x_bf16;
    a.B = B;
    a.n_in = n_in;
    a.S = i8_splits(B, n_in, i8_tiles(n_out, n_proj), scale_axis);
    a.scale_axis = scale_axis;
    a.tiled = tiled;
    a.blocks = n_in / i8_block_cols(scale_axis) / a.S;
    a.n_proj = n_proj;
    size_t off = 0;
    int wg = 0, ctrs = 0;
    for (int j = 0; j < n_proj; ++j) {
        I8Proj &p = a.p[j];
        p.q = projs[j].qT;
        p.s = projs[j].s;
        p.n_out = projs[j].n_out;
        p.y_bf16 = projs[j].y_bf16;
        p.y_f32 = projs[j].y_f32;
        p.part = part + off;
        off += (size_t)a.S * B * p.n_out;
        a.wg_start[j] = wg;
        const int row_groups = (p.n_out + 16 * kI8Waves - 1) / (16 * kI8Waves);
        wg += row_groups * a.S;
        a.ctr_start[j] = pair ? 0 : ctrs;
        ctrs = a.ctr_start[j] + row_groups;
    }
    a.wg_start[n_proj] = wg;
    // the split sums in this launch when its row groups have counters (and there is more than one split or a pair)
    a.cnt = (a.S > 1 || pair) && ctrs <= kI8Ctrs && (i8_fuse() & (pair ? 2 : 1)) ? cnt : nullptr;
    const size_t lds = i8_lds_bytes(B, i8_block_cols(scale_axis) * a.blocks, scale_axis);
    hipStream_t st = (hipStream_t)stream;
    typedef void (*Kern)(I8Args);
    static const Kern kern[2][2][4] = {
        {{int8_project_kernel<1, 0, false>, int8_project_kernel<1, 1, false>, int8_project_kernel<1, 2, false>,
          int8_project_kernel<1, kW16, false>},
         {int8_project_kernel<2, 0, false>, int8_project_kernel<2, 1, false>, int8_project_kernel<2, 2, false>,
          int8_project_kernel<2, kW16, false>}},
        {{int8_project_kernel<1, 0, true>, int8_project_kernel<1, 1, true>, int8_project_kernel<1, 2, true>,
          int8_project_kernel<1, kW16, true>},
         {int8_project_kernel<2, 0, true>, int8_project_kernel<2, 1, true>, int8_project_kernel<2, 2, true>,
          int8_project_kernel<2, kW16, true>}}};
    hipLaunchKernelGGL(kern[a.cnt ? 1 : 0][B <= 16 ? 0 : 1][scale_axis], dim3(wg), dim3(64 * kI8Waves), lds, st, a);
    if (hipGetLastError() != hipSuccess) return MI_ERR_LAUNCH;
    if (a.cnt) return MI_OK;
    if (pair) {
        const int n4 = B * a.p[0].n_out / 4;
        hipLaunchKernelGGL(swiglu_pair_i8, dim3((n4 + 255) / 256), dim3(256), 0, st, a);
        return hipGetLastError() == hipSuccess ? MI_OK : MI_ERR_LAUNCH;
    }
    if (a.S == 1) return MI_OK;
    int n4 = 0;
    for (int j = 0; j < n_proj; ++j) n4 += B * a.p[j].n_out / 4;
    hipLaunchKernelGGL(split_reduce_i8, dim3((n4 + 255) / 256), dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess ? MI_OK : MI_ERR_LAUNCH;
}



// mlp_partial's two launches over weights of one form per launch (int8 with scales, or kW16): gate and up together
// (their last workgroups form h), then down with its split sums.  Workspace: [counter blocks: gate/up's, down's]
// [gate/up partials][h][down partials].
static size_t mlp_workspace(int32_t B, int32_t D, int32_t I, int32_t gu_form, int32_t dn_form) {
    if (B <= 0 || B > 32 || D <= 0 || I <= 0 || D % 256 || I % 256) return 0;
    const int32_t gu[2] = {I, I}, dn = D;
    return kI8CtrBytes + al256_i8(i8_part_bytes(B, D, gu, 2, gu_form, 1)) + al256_i8(2 * (size_t)B * I) +
           i8_part_bytes(B, I, &dn, 1, dn_form, 0);
}

static int mlp_launches(const uint16_t *x_bf16, int32_t B, int32_t D, int32_t I, const int8_t *gate_w,
                        const float *gate_s, const int8_t *up_w, const float *up_s, int32_t gu_form,
                        const int8_t *down_w, const float *down_s, int32_t dn_form, float limit, uint16_t *y_bf16,
                        float *y_f32, void *workspace, size_t workspace_bytes, void *stream) {
    if (!(limit > 0.0f)) return MI_ERR_ARG;
    const size_t need = mlp_workspace(B, D, I, gu_form & ~MI_I8_TILED, dn_form & ~MI_I8_TILED);
    if (need == 0) return MI_ERR_ARG;
    if (!workspace || workspace_bytes < need || (uintptr_t)workspace % 256) return MI_ERR_WORKSPACE;
    const int32_t gu[2] = {I, I};
    uint32_t *cnt = (uint32_t *)workspace;
    char *gu_part = (char *)workspace + kI8CtrBytes;
    const size_t part = al256_i8(i8_part_bytes(B, D, gu, 2, gu_form, 1));
    uint16_t *h = (uint16_t *)(gu_part + part);
    char *dn_part = gu_part + part + al256_i8(2 * (size_t)B * I);
    const mi_i8_proj p[2] = {{gate_w, gate_s, I, nullptr, nullptr}, {up_w, up_s, I, nullptr, nullptr}};
    int st = i8_launch(x_bf16, B, D, p, 2, gu_form, (float *)gu_part, part, cnt, stream, 1, limit, h);
    if (st) return st;
    const mi_i8_proj pd{down_w, down_s, D, y_bf16, y_f32};
    return i8_launch(h, B, I, &pd, 1, dn_form, (float *)dn_part,
                     workspace_bytes - (size_t)(dn_part - (char *)workspace), cnt + kI8Ctrs * kI8CtrStride, stream, 0,
                     0.0f, nullptr);
}

extern "C" {

size_t mi_int8_project_many_workspace(int32_t B, int32_t n_in, const int32_t *n_out, int32_t n_proj,
                                      int32_t scale_axis) {
    if (B <= 0 || B > 32 || n_in <= 0 || n_in % 256 || !n_out || n_proj <= 0 || n_proj > kI8MaxProj) return 0;
    scale_axis &= ~MI_I8_TILED;
    if (scale_axis < MI_I8_ROW_SCALES || scale_axis > MI_I8_COL_AFTER) return 0;
    for (int j = 0; j < n_proj; ++j)
        if (n_out[j] <= 0 || n_out[j] % 16) return 0;
    return kI8CtrBytes + i8_part_bytes(B, n_in, n_out, n_proj, scale_axis, 0);
}

// Every int8 workspace starts with the counter blocks (kI8CtrBytes), then the launch's data.
int mi_int8_project_many(const uint16_t *x_bf16, int32_t B, int32_t n_in, const mi_i8_proj *projs, int32_t n_proj,
                         int32_t scale_axis, void *workspace, size_t workspace_bytes, void *stream) {
    if ((scale_axis & ~MI_I8_TILED) > MI_I8_COL_AFTER) return MI_ERR_ARG;      // int8 scale forms only
    const bool ok = workspace && workspace_bytes >= kI8CtrBytes;
    return i8_launch(x_bf16, B, n_in, projs, n_proj, scale_axis,
                     ok ? (float *)((char *)workspace + kI8CtrBytes) : nullptr, ok ? workspace_bytes - kI8CtrBytes : 0,
                     (uint32_t *)workspace, stream, 0, 0.0f, nullptr);
}

int mi_int8_tile(const int8_t *qT, int32_t n_out, int32_t n_in, int8_t *tiled, void *stream) {
    if (!qT || !tiled) return MI_ERR_NULL;
    if (n_out <= 0 || n_in <= 0 || n_out % 16 || n_in % 256) return MI_ERR_SHAPE;
    if ((uintptr_t)qT % 16 || (uintptr_t)tiled % 16) return MI_ERR_ARG;
    const size_t n16 = (size_t)n_out * n_in / 16;
    const unsigned grid = (unsigned)std::min<size_t>((n16 + 255) / 256, 8192);
    hipLaunchKernelGGL(int8_tile_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, qT, n_out, n_in, tiled);
    return hipGetLastError() == hipSuccess ? MI_OK : MI_ERR_LAUNCH;
}

size_t mi_int8_project_workspace(int32_t B, int32_t n_in, int32_t n_out, int32_t scale_axis) {
    return mi_int8_project_many_workspace(B, n_in, &n_out, 1, scale_axis);
}

int mi_int8_project(const uint16_t *x_bf16, int32_t B, const int8_t *qT, const float *s, int32_t scale_axis,
                    int32_t n_in, int32_t n_out, uint16_t *y_bf16, float *y_f32, void *workspace,
                    size_t workspace_bytes, void *stream) {
    if (!x_bf16 || !qT || !s || (!y_bf16 && !y_f32)) return MI_ERR_NULL;
    if (B <= 0 || B > 32) return MI_ERR_TOKENS;
    if (n_in <= 0 || n_out <= 0 || n_in % 256 || n_out % 16) return MI_ERR_SHAPE;
    const mi_i8_proj p{qT, s, n_out, y_bf16, y_f32};
    return mi_int8_project_many(x_bf16, B, n_in, &p, 1, scale_axis, workspace, workspace_bytes, stream);
}

size_t mi_int8_mlp_workspace(int32_t B, int32_t D, int32_t I, int32_t gu_scale_axis, int32_t down_scale_axis) {
    gu_scale_axis &= ~MI_I8_TILED;
    down_scale_axis &= ~MI_I8_TILED;
    if (gu_scale_axis != MI_I8_ROW_SCALES && gu_scale_axis != MI_I8_COL_SCALES) return 0;
    if (down_scale_axis != MI_I8_ROW_SCALES && down_scale_axis != MI_I8_COL_SCALES) return 0;
    return mlp_workspace(B, D, I, gu_scale_axis, down_scale_axis);
}

int mi_int8_mlp(const uint16_t *x_bf16, int32_t B, int32_t D, int32_t I, const int8_t *gate_qT, const float *gate_s,
                const int8_t *up_qT, const float *up_s, int32_t gu_scale_axis, const int8_t *down_qT,
                const float *down_s, int32_t down_scale_axis, float limit, uint16_t *y_bf16, float *y_f32,
                void *workspace, size_t workspace_bytes, void *stream) {
    if (!x_bf16 || !gate_qT || !gate_s || !up_qT || !up_s || !down_qT || !down_s || (!y_bf16 && !y_f32))
        return MI_ERR_NULL;
    if (B <= 0 || B > 32) return MI_ERR_TOKENS;
    if (D <= 0 || I <= 0 || D % 256 || I % 256) return MI_ERR_SHAPE;
    if (mi_int8_mlp_workspace(B, D, I, gu_scale_axis, down_scale_axis) == 0) return MI_ERR_ARG;
    return mlp_launches(x_bf16, B, D, I, gate_qT, gate_s, up_qT, up_s, gu_scale_axis, down_qT, down_s,
                        down_scale_axis, limit, y_bf16, y_f32, workspace, workspace_bytes, stream);
}

size_t mi_bf16_project_workspace(int32_t B, int32_t n_in, int32_t n_out) {
    if (B <= 0 || B > 32 || n_in <= 0 || n_in % 256 || n_out <= 0 || n_out % 16) return 0;
    return kI8CtrBytes + i8_part_bytes(B, n_in, &n_out, 1, kW16, 0);
}

int mi_bf16_project(const uint16_t *x_bf16, int32_t B, const uint16_t *wT, int32_t n_in, int32_t n_out,
                    uint16_t *y_bf16, float *y_f32, void *workspace, size_t workspace_bytes, void *stream) {
    if (!x_bf16 || !wT || (!y_bf16 && !y_f32)) return MI_ERR_NULL;
    if (B <= 0 || B > 32) return MI_ERR_TOKENS;
    if (n_in <= 0 || n_out <= 0 || n_in % 256 || n_out % 16) return MI_ERR_SHAPE;
    if ((uintptr_t)wT % 16) return MI_ERR_ARG;
    const bool ok = workspace && workspace_bytes >= kI8CtrBytes;
    const mi_i8_proj p{(const int8_t *)wT, nullptr, n_out, y_bf16, y_f32};
    return i8_launch(x_bf16, B, n_in, &p, 1, kW16, ok ? (float *)((char *)workspace + kI8CtrBytes) : nullptr,
                     ok ? workspace_bytes - kI8CtrBytes : 0, (uint32_t *)workspace, stream, 0, 0.0f, nullptr);
}

size_t mi_bf16_mlp_workspace(int32_t B, int32_t D, int32_t I) { return mlp_workspace(B, D, I, kW16, kW16); }

int mi_bf16_mlp(const uint16_t *x_bf16, int32_t B, int32_t D, int32_t I, const uint16_t *gate_wT,
                const uint16_t *up_wT, const uint16_t *down_wT, float limit, uint16_t *y_bf16, float *y_f32,
                void *workspace, size_t workspace_bytes, void *stream) {
    if (!x_bf16 || !gate_wT || !up_wT || !down_wT || (!y_bf16 && !y_f32)) return MI_ERR_NULL;
    if (B <= 0 || B > 32) return MI_ERR_TOKENS;
    if (D <= 0 || I <= 0 || D % 256 || I % 256) return MI_ERR_SHAPE;
    if ((uintptr_t)gate_wT % 16 || (uintptr_t)up_wT % 16 || (uintptr_t)down_wT % 16) return MI_ERR_ARG;
    return mlp_launches(x_bf16, B, D, I, (const int8_t *)gate_wT, nullptr, (const int8_t *)up_wT, nullptr, kW16,
                        (const int8_t *)down_wT, nullptr, kW16, limit, y_bf16, y_f32, workspace, workspace_bytes,
                        stream);
}

}  // extern "C"
