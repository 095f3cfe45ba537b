// GGUF blocks -> the reference's planar tables on the device (the field split of planes.py:136-170, done by
// resident.py:29-60 on the host there).  The raw expert tensor [E][R][nblk][block bytes] is copied to HBM as read
// from the file; one workgroup per (64 rows, pair of blocks, expert) stages its rows' two blocks in LDS (contiguous
// 2-byte reads per row) and writes every plane word of them as 64 consecutive u32 (the row is the minor axis of a
// plane).  Pure byte movement: HBM-bound, bit-exact by construction.
//   IQ2_S  (82 B):  d [0:2] | qs [2:34] | sg [34:66] | qh [66:74] | sc [74:82]      planes {qs, sg, qh, sc, d}
//   IQ3_S  (110 B): d [0:2] | qs [2:66] | qh [66:74] | sg [74:106] | sc [106:110]   planes {qs, sg, qh, sc, d}
//   IQ4_XS (136 B): d [0:2] | sh [2:4] | sl [4:8] | qs [8:136]                     planes {qs, sl, sh, d}
// Every field but sh is whole words; sh is zero-extended to one word per block; d packs the f16 of blocks 2p and
// 2p + 1 into word p (zero for a missing odd block).
#include "common.h"

namespace mi {

constexpr int kPackRows = 64;
constexpr int kPackMaxBB = 136;

struct PackSpec {
    int bb;                      // bytes per block
    int nf;                      // word fields (every plane but d)
    int off[4], len[4];          // byte offset and length of each field in the block (sh: length 2, one word)
    int dplane;                  // plane index of d
};

static PackSpec pack_spec(int qtype) {
    PackSpec s{};
    if (qtype == MI_QT_IQ2_S) s = PackSpec{82, 4, {2, 34, 66, 74}, {32, 32, 8, 8}, 4};
    else if (qtype == MI_QT_IQ3_S) s = PackSpec{110, 4, {2, 74, 66, 106}, {64, 32, 8, 4}, 4};
    else s = PackSpec{136, 3, {8, 4, 2, 0}, {128, 4, 2, 0}, 3};
    return s;
}

struct PackArgs {
    PackSpec sp;
    const uint8_t *blocks;
    uint32_t *plane[5];
    int E, R, nblk;
};

__global__ void __launch_bounds__(256) pack_planes_kernel(PackArgs a) {
    __shared__ uint16_t st[kPackRows][kPackMaxBB];              // 64 rows x two blocks (2 x 136 bytes at most)
    const PackSpec &sp = a.sp;
    const int r0 = blockIdx.x * kPackRows, p = blockIdx.y, e = blockIdx.z;
    const int b0 = 2 * p, nb = min(2, a.nblk - b0);
    const int nr = min(kPackRows, a.R - r0);
    const int hw = nb * sp.bb / 2;                              // halfwords per row
    for (int i = threadIdx.x; i < nr * hw; i += 256) {
        const int r = i / hw, h = i - r * hw;
        const size_t src = (((size_t)e * a.R + r0 + r) * a.nblk + b0) * sp.bb;
        st[r][h] = *(const uint16_t *)(a.blocks + src + 2 * h);
    }
    __syncthreads();
    const uint8_t *sb = (const uint8_t *)st;
    auto byte_at = [&](int r, int o) -> uint32_t { return sb[r * 2 * kPackMaxBB + o]; };
    // word fields: plane f, words per block wpb = ceil(len / 4), row b * wpb + w of expert e
    for (int f = 0; f < sp.nf; ++f) {
        const int wpb = (sp.len[f] + 3) / 4;
        const size_t rows_p = (size_t)a.nblk * wpb;
        const int items = nb * wpb * kPackRows;
        for (int i = threadIdx.x; i < items; i += 256) {
            const int r = i % kPackRows, bw = i / kPackRows, bi = bw / wpb, w = bw - bi * wpb;
            if (r >= nr) continue;
            const int o = bi * sp.bb + sp.off[f] + 4 * w;
            uint32_t v = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (4 * w + k < sp.len[f]) v |= byte_at(r, o + k) << (8 * k);
            a.plane[f][((size_t)e * rows_p + (size_t)(b0 + bi) * wpb + w) * a.R + r0 + r] = v;
        }
    }
    // d: word p = f16 of block 2p | f16 of block 2p + 1 << 16
    if (threadIdx.x < nr) {
        const int r = threadIdx.x;
        uint32_t v = byte_at(r, 0) | byte_at(r, 1) << 8;
        if (nb == 2) v |= (byte_at(r, sp.bb) | byte_at(r, sp.bb + 1) << 8) << 16;
        const size_t rows_p = (size_t)(a.nblk + 1) / 2;
        a.plane[sp.dplane][((size_t)e * rows_p + p) * a.R + r0 + r] = v;
    }
}

}  // namespace mi

using namespace mi;

extern "C" int mi_pack_planes(int32_t qtype, const uint8_t *blocks, int32_t E, int32_t R, int32_t K,
                              void *const *planes, void *stream) {
    if (qtype != MI_QT_IQ2_S && qtype != MI_QT_IQ3_S && qtype != MI_QT_IQ4_XS) return MI_ERR_QTYPE;
    if (!blocks || !planes) return MI_ERR_NULL;
    if (E <= 0 || E > 65535 || R <= 0 || K <= 0 || K % 256) return MI_ERR_SHAPE;
    const int nblk = K / 256;
    if ((nblk + 1) / 2 > 65535) return MI_ERR_SHAPE;
    const PackSpec sp = pack_spec(qtype);
    PackArgs a{};
    a.sp = sp;
    a.blocks = blocks;
    const int np = sp.nf + 1;
    for (int i = 0; i < np; ++i) {
        if (!planes[i]) return MI_ERR_NULL;
        a.plane[i] = (uint32_t *)planes[i];
    }
    if ((uintptr_t)blocks % 2) return MI_ERR_ARG;               // read as 2-byte halves
    a.E = E;
    a.R = R;
    a.nblk = nblk;
    hipLaunchKernelGGL(pack_planes_kernel, dim3((R + kPackRows - 1) / kPackRows, (nblk + 1) / 2, E), dim3(256), 0,
                       (hipStream_t)stream, a);
    return hipGetLastError() == hipSuccess ? MI_OK : MI_ERR_LAUNCH;
}
