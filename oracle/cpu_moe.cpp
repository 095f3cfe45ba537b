// CPU restatement of the batch decode composition in C++ with OpenMP -- test infrastructure only (the CPU baseline
// leg of the benchmark and a cross-check of the NumPy oracle; the product never links it).
//
// The composition is the reference's fused decode, ResidentFetch._apply_kernel (resident.py:110-120): for every
// slot (n, j) with expert e = idx[n, j],
//   g = Wgate_e x_n, u = Wup_e x_n                       (moe_matvec, pallas_moe.py:238-307 == moe_matvec_ref :310-323)
//   h = silu(min(g, L)) * clip(u, -L, L)                  (model.py:119-122, resident.py:118)
//   y = Wdown_e h                                         (resident.py:119)
//   out[n] = sum_j w[n, j] y  (+ the shared expert's y with weight 1 when shared >= 0)   (resident.py:120)
// x is taken as f32 (resident.py:114); every sum is f64 here, as in oracle.moe.decode_apply, so the two agree to
// rounding of f64.  Experts are visited once each, over the slots routed to them.
//
// Weights: the CB3 codebook format in its canonical packing -- words u32 [E][R][ceil(K/10)] with
// code(r, k) = (word[r][k / 10] >> 3 (k % 10)) & 7, codebook u16 [E][R][K/128][8] of bf16 bits, and
// W[r, k] = bf16(cb[r][k / 128][code(r, k)]).
#include <omp.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

namespace {

inline double bf16_value(uint16_t bits) {
    const uint32_t u = (uint32_t)bits << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return (double)f;
}

struct Matrix {          // one expert's matrix, R rows x K inputs
    const uint32_t *words;
    const uint16_t *cb;
    int R, K;
};

Matrix expert(const uint32_t *words, const uint16_t *cb, int e, int R, int K) {
    const size_t wd = (size_t)(K + 9) / 10, groups = (size_t)K / 128;
    return {words + (size_t)e * R * wd, cb + (size_t)e * R * groups * 8, R, K};
}

// y[t][r] = sum_k W[r, k] x[t][k] for t < nt, in f64; rows split over the OpenMP threads.
void matvec(const Matrix &m, const double *x, int nt, double *y) {
    const int wd = (m.K + 9) / 10, groups = m.K / 128;
#pragma omp parallel
    {
        std::vector<double> acc(nt), wrow(m.K);
#pragma omp for schedule(static)
        for (int r = 0; r < m.R; ++r) {
            const uint32_t *wr = m.words + (size_t)r * wd;
            const uint16_t *cr = m.cb + (size_t)r * groups * 8;
            for (int k = 0; k < m.K; ++k) wrow[k] = bf16_value(cr[(k / 128) * 8 + ((wr[k / 10] >> (3 * (k % 10))) & 7u)]);
            for (int t = 0; t < nt; ++t) {
                const double *xt = x + (size_t)t * m.K;
                double s = 0.0;
                for (int k = 0; k < m.K; ++k) s += wrow[k] * xt[k];
                acc[t] = s;
            }
            for (int t = 0; t < nt; ++t) y[(size_t)t * m.R + r] = acc[t];
        }
    }
}

double swiglu_clamped(double g, double u, double limit) {
    g = std::fmin(g, limit);
    u = std::fmin(std::fmax(u, -limit), limit);
    return g / (1.0 + std::exp(-g)) * u;
}

}  // namespace

extern "C" {

// out f64 [N, D] (D = gate cols = down rows, I = gate rows); returns 0, or -1 for invalid arguments.  threads <= 0:
// OpenMP's default.
int cpu_moe_decode_cb3(int32_t E, int32_t D, int32_t I, const uint32_t *gate_words, const uint16_t *gate_cb,
                       const uint32_t *up_words, const uint16_t *up_cb, const uint32_t *down_words,
                       const uint16_t *down_cb, const float *x, int32_t N, int32_t k, const int32_t *idx,
                       const float *w, int32_t shared, float limit, double *out, int32_t threads) {
    if (E <= 0 || D <= 0 || I <= 0 || D % 128 || I % 128 || N <= 0 || k <= 0 || shared >= E || !x || !idx || !w ||
        !out || !gate_words || !gate_cb || !up_words || !up_cb || !down_words || !down_cb)
        return -1;
    for (int i = 0; i < N * k; ++i)
        if (idx[i] < 0 || idx[i] >= E) return -1;
    if (threads > 0) omp_set_num_threads(threads);
    std::memset(out, 0, sizeof(double) * (size_t)N * D);
    std::vector<double> xd((size_t)N * D);
    for (size_t i = 0; i < xd.size(); ++i) xd[i] = (double)x[i];
    std::vector<double> xs, g, u, h, y;
    for (int e = 0; e < E; ++e) {
        // the slots routed to e, in (token, column) order; the shared expert takes every token with weight 1
        std::vector<int> tok;
        std::vector<double> wt;
        for (int n = 0; n < N; ++n)
            for (int j = 0; j < k; ++j)
                if (idx[n * k + j] == e) {
                    tok.push_back(n);
                    wt.push_back((double)w[n * k + j]);
                }
        if (e == shared)
            for (int n = 0; n < N; ++n) {
                tok.push_back(n);
                wt.push_back(1.0);
            }
        const int nt = (int)tok.size();
        if (nt == 0) continue;
        xs.assign((size_t)nt * D, 0.0);
        for (int t = 0; t < nt; ++t) std::memcpy(&xs[(size_t)t * D], &xd[(size_t)tok[t] * D], sizeof(double) * D);
        g.resize((size_t)nt * I);
        u.resize((size_t)nt * I);
        h.resize((size_t)nt * I);
        y.resize((size_t)nt * D);
        matvec(expert(gate_words, gate_cb, e, I, D), xs.data(), nt, g.data());
        matvec(expert(up_words, up_cb, e, I, D), xs.data(), nt, u.data());
        for (size_t i = 0; i < h.size(); ++i) h[i] = swiglu_clamped(g[i], u[i], (double)limit);
        matvec(expert(down_words, down_cb, e, D, I), h.data(), nt, y.data());
        for (int t = 0; t < nt; ++t)
            for (int d = 0; d < D; ++d) out[(size_t)tok[t] * D + d] += wt[t] * y[(size_t)t * D + d];
    }
    return 0;
}

int cpu_moe_threads(void) { return omp_get_max_threads(); }

}  // extern "C"
