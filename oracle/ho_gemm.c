/*
 * ho_gemm.c - dense projection for the CPU oracle (TEST INFRASTRUCTURE ONLY).
 *
 * y[n][o] = sum_i x[n][i] * W[o][i] (+ b[o]): the candle/PyTorch Linear convention used
 * by every projection in crates/huncho-backend/src/qwen3_5.rs (BackboneLinear, 306-515).
 * The reference's CPU GEMM (the gemm crate) blocks its reduction and uses FMA, so no
 * scalar order is reproducible; this file is compiled with FMA contraction allowed and
 * reduces each dot product in 8 interleaved fp32 partial sums.
 */
#include "huncho_oracle.h"

#include <string.h>

typedef float v8f __attribute__((vector_size(32)));

static inline v8f ld8(const float* p) {
    v8f r;
    memcpy(&r, p, sizeof(r));
    return r;
}
static inline float hsum8(v8f v) {
    return ((v[0] + v[4]) + (v[1] + v[5])) + ((v[2] + v[6]) + (v[3] + v[7]));
}

void ho_linear(const float* x, const float* w, const float* b, int n, int in, int out, float* y) {
    const int in8 = in & ~7;
#pragma omp parallel for collapse(2) schedule(static)
    for (int ob = 0; ob < (out + 3) / 4; ++ob)
        for (int nb = 0; nb < (n + 3) / 4; ++nb) {
            for (int oo = ob * 4; oo < ob * 4 + 4 && oo < out; ++oo) {
                const float* wr = w + (size_t)oo * in;
                int nn0 = nb * 4;
                int cnt = n - nn0 < 4 ? n - nn0 : 4;
                v8f acc[4] = {{0}, {0}, {0}, {0}};
                for (int i = 0; i < in8; i += 8) {
                    v8f wv = ld8(wr + i);
                    for (int r = 0; r < cnt; ++r) acc[r] += ld8(x + (size_t)(nn0 + r) * in + i) * wv;
                }
                for (int r = 0; r < cnt; ++r) {
                    const float* xr = x + (size_t)(nn0 + r) * in;
                    float s = hsum8(acc[r]);
                    for (int i = in8; i < in; ++i) s += xr[i] * wr[i];
                    y[(size_t)(nn0 + r) * out + oo] = b ? s + b[oo] : s;
                }
            }
        }
}
