// int8 per-output-channel projections for gfx950: y = x @ bf16(f32(q) * s)   (quant8.py:91-99 + the x @ W uses).
//
// The weights stream once from HBM as int8 (qT: [n_out, n_in], input-contiguous), are dequantized in registers to
// exactly the reference's bf16(f32(q) * s) (round to nearest even), and feed v_mfma_f32_16x16x32_bf16 with the
// activations as the other operand (bf16 x bf16 products are exact; f32 accumulation).  A wavefront owns 16 output
// channels x one column range; the 4 wavefronts of a workgroup split the range and reduce in LDS; KS workgroups
// split the remaining columns and the one that completes a 16-channel tile sums the KS partials in order.
#include "common.h"

namespace mi {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct I8Args {
    const uint16_t *x;
    const int8_t *q;
    const float *s;
    int B, n_in, n_out, KS;
    uint16_t *y_bf16;
    float *y_f32;
    float *part;       // [KS, n_out, 32]
    uint32_t *cnt;     // [n_out / 16]
};

constexpr int kI8Waves = 4;

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    return f32_to_bf16_rne(a) | (f32_to_bf16_rne(b) << 16);
}

template <int NT>   // token tiles of 16 (B <= 16 * NT)
__global__ void __launch_bounds__(64 * kI8Waves) int8_project_kernel(I8Args a) {
    __shared__ float red[kI8Waves][16][16 * NT];
    __shared__ int s_last;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int tile = blockIdx.x;               // 16 output channels
    const int ks = blockIdx.y;
    const int o0 = tile * 16;
    const int i_row = lane & 15, kq = lane >> 4;
    const int chunk = a.n_in / (a.KS * kI8Waves);      // columns per wavefront (multiple of 32)
    const int k_begin = (ks * kI8Waves + wave) * chunk;
    const float sc = a.s[o0 + i_row];
    const int8_t *qrow = a.q + (size_t)(o0 + i_row) * a.n_in + k_begin + 8 * kq;

    f32x4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = (f32x4){0.f, 0.f, 0.f, 0.f};

    for (int k = 0; k < chunk; k += 32) {
        const uint2 qv = *(const uint2 *)(qrow + k);
        uint32_t wv[4];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t u = h ? qv.y : qv.x;
            const float f0 = (float)(int8_t)(u & 255u) * sc;
            const float f1 = (float)(int8_t)((u >> 8) & 255u) * sc;
            const float f2 = (float)(int8_t)((u >> 16) & 255u) * sc;
            const float f3 = (float)(int8_t)(u >> 24) * sc;
            wv[2 * h] = pack_bf16x2(f0, f1);
            wv[2 * h + 1] = pack_bf16x2(f2, f3);
        }
        const bf16x8 A = __builtin_bit_cast(bf16x8, make_uint4(wv[0], wv[1], wv[2], wv[3]));
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int tok = 16 * t + i_row;
            uint4 xv = make_uint4(0, 0, 0, 0);
            if (tok < a.B) xv = *(const uint4 *)(a.x + (size_t)tok * a.n_in + k_begin + k + 8 * kq);
            const bf16x8 Bv = __builtin_bit_cast(bf16x8, xv);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, Bv, acc[t], 0, 0, 0);
        }
    }
    // C layout: lane holds rows (channels) 4*kq + r, column (token) i_row
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave][4 * kq + r][16 * t + i_row] = acc[t][r];
    __syncthreads();

    const int ntok = 16 * NT;
    if (a.KS == 1) {
        for (int i = tid; i < 16 * ntok; i += blockDim.x) {
            const int c = i / ntok, b = i - c * ntok;
            if (b >= a.B) continue;
            float v = 0.f;
#pragma unroll
            for (int wv = 0; wv < kI8Waves; ++wv) v += red[wv][c][b];
            if (a.y_f32) a.y_f32[(size_t)b * a.n_out + o0 + c] = v;
            if (a.y_bf16) a.y_bf16[(size_t)b * a.n_out + o0 + c] = (uint16_t)f32_to_bf16_rne(v);
        }
        return;
    }
    for (int i = tid; i < 16 * ntok; i += blockDim.x) {
        const int c = i / ntok, b = i - c * ntok;
        float v = 0.f;
#pragma unroll
        for (int wv = 0; wv < kI8Waves; ++wv) v += red[wv][c][b];
        a.part[((size_t)ks * a.n_out + o0 + c) * 32 + b] = v;
    }
    __syncthreads();
    if (tid == 0) {
        fence_release_agent();
        s_last = counter_add(a.cnt + tile, 1u) == (uint32_t)(a.KS - 1);
    }
    __syncthreads();
    if (!s_last) return;
    fence_acquire_agent();
    for (int i = tid; i < 16 * ntok; i += blockDim.x) {
        const int c = i / ntok, b = i - c * ntok;
        if (b >= a.B) continue;
        float v = 0.f;
        for (int s = 0; s < a.KS; ++s) v += a.part[((size_t)s * a.n_out + o0 + c) * 32 + b];
        if (a.y_f32) a.y_f32[(size_t)b * a.n_out + o0 + c] = v;
        if (a.y_bf16) a.y_bf16[(size_t)b * a.n_out + o0 + c] = (uint16_t)f32_to_bf16_rne(v);
    }
    if (tid == 0) counter_reset(a.cnt + tile);
}

static int i8_splits(int n_in, int n_out) {
    const int tiles = n_out / 16;
    int KS = 1;
    // enough workgroups to cover the chip; every wavefront keeps >= 256 columns (8 MFMA steps)
    while (tiles * KS < 512 && n_in % (2 * KS * kI8Waves * 32) == 0 && n_in / (2 * KS * kI8Waves) >= 256) KS *= 2;
    return KS;
}

}  // namespace mi

using namespace mi;

extern "C" {

size_t mi_int8_project_workspace(int32_t B, int32_t n_in, int32_t n_out) {
    if (B <= 0 || B > 32 || n_in <= 0 || n_out <= 0 || n_in % 256 || n_out % 16) return 0;
    const int KS = i8_splits(n_in, n_out);
    const size_t cnt = ((sizeof(uint32_t) * (size_t)(n_out / 16)) + 255) & ~(size_t)255;
    return cnt + sizeof(float) * (size_t)KS * n_out * 32;
}

int mi_int8_project(const uint16_t *x_bf16, int32_t B, const int8_t *qT, const float *s, int32_t n_in,
                    int32_t n_out, uint16_t *y_bf16, float *y_f32, void *workspace, size_t workspace_bytes,
                    void *stream) {
    if (!x_bf16 || !qT || !s || (!y_bf16 && !y_f32)) return MI_ERR_NULL;
    if (B <= 0 || B > 32) return MI_ERR_TOKENS;
    if (n_in <= 0 || n_out <= 0 || n_in % 256 || n_out % 16) return MI_ERR_SHAPE;
    const size_t need = mi_int8_project_workspace(B, n_in, n_out);
    if (!workspace || workspace_bytes < need) return MI_ERR_WORKSPACE;
    I8Args a{};
    a.x = x_bf16;
    a.q = qT;
    a.s = s;
    a.B = B;
    a.n_in = n_in;
    a.n_out = n_out;
    a.KS = i8_splits(n_in, n_out);
    a.y_bf16 = y_bf16;
    a.y_f32 = y_f32;
    const size_t cnt = ((sizeof(uint32_t) * (size_t)(n_out / 16)) + 255) & ~(size_t)255;
    a.cnt = (uint32_t *)workspace;
    a.part = (float *)((char *)workspace + cnt);
    dim3 grid(n_out / 16, a.KS);
    if (B <= 16) hipLaunchKernelGGL(int8_project_kernel<1>, grid, dim3(64 * kI8Waves), 0, (hipStream_t)stream, a);
    else hipLaunchKernelGGL(int8_project_kernel<2>, grid, dim3(64 * kI8Waves), 0, (hipStream_t)stream, a);
    return hipGetLastError() == hipSuccess ? MI_OK : MI_ERR_LAUNCH;
}

}  // extern "C"
