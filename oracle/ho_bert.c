/*
 * ho_bert.c - CPU restatement of the ModernBERT encoder behind Huncho's Laya backend.
 *
 * TEST INFRASTRUCTURE ONLY (see huncho_oracle.h): the parity oracle and CPU baseline for
 * the ModernBERT path; the product never links it.
 *
 * The reference executes ModernBERT through candle-transformers 0.11.0
 * (crates/huncho-backend/src/candle.rs:65-117, 319-416; Cargo.lock:448-451), which is not
 * vendored in the reference tree. This file follows the published ModernBERT definition
 * that library implements, with the reference's own configuration handling:
 *   - config: global_rope_theta / local_rope_theta (or rope_parameters.*), local_attention
 *     (default 128), global_attn_every_n_layers (default 3), layer_norm_eps (default 1e-5)
 *     (candle.rs:157-203);
 *   - embeddings: token embedding -> LayerNorm (weight only, no bias);
 *   - layer i: global attention iff i % global_attn_every_n_layers == 0, otherwise local
 *     attention over keys with |i - j| <= local_attention / 2;
 *     h += Wo(attn(rope(Wqkv(attn_norm(h))))), the attn_norm applied when the checkpoint
 *     carries one (the tiny_modernbert fixture does for layer 0);
 *     h += Wo2(gelu(x1) * x2) with [x1 | x2] = Wi(mlp_norm(h)), gelu the exact erf form;
 *   - final LayerNorm.
 * RoPE is the NeoX rotate-half form on the full head dim with the layer's theta,
 * positions 0..L-1 of each sequence; attention is bidirectional softmax(q.k / sqrt(d)) v
 * inside each sequence of the unpadded varlen batch.
 * With bf16_mode != 0 every stored intermediate (norm outputs, projections, RoPE outputs,
 * attention output, GeGLU output, residual stream) is rounded to bfloat16.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "huncho_oracle.h"

static inline float rb(float x) { return ho_bf16_to_f32(ho_f32_to_bf16(x)); }
static void round_if(float* x, size_t n, int on) {
    if (!on) return;
    for (size_t i = 0; i < n; ++i) x[i] = rb(x[i]);
}

/* LayerNorm without bias: (x - mean) / sqrt(var + eps) * w, var the biased variance,
 * statistics in double then applied in fp32. */
void ho_layer_norm(const float* x, const float* w, int rows, int width, float eps, float* y) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const float* xr = x + (size_t)r * width;
        double s = 0.0;
        for (int i = 0; i < width; ++i) s += xr[i];
        const double mean = s / width;
        double v = 0.0;
        for (int i = 0; i < width; ++i) v += (xr[i] - mean) * (xr[i] - mean);
        const float inv = (float)(1.0 / sqrt(v / width + (double)eps));
        const float m = (float)mean;
        for (int i = 0; i < width; ++i) y[(size_t)r * width + i] = ((xr[i] - m) * inv) * w[i];
    }
}

float ho_gelu_erf(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f)); }

/* Bidirectional attention inside each sequence; q, k, v, out [tokens][heads][d]. Key j is
 * visible to query i iff half_window < 0 or |i - j| <= half_window. */
int ho_bidir_attention(const float* q, const float* k, const float* v, const int32_t* cu_seqlens, int n_seqs,
                       int heads, int d, int half_window, float scale, float* out) {
    for (int s = 0; s < n_seqs; ++s)
        if (cu_seqlens[s + 1] < cu_seqlens[s]) return -1;
#pragma omp parallel
    {
        double* p = NULL;
        int cap = 0;
#pragma omp for collapse(2) schedule(dynamic, 1)
        for (int s = 0; s < n_seqs; ++s)
            for (int h = 0; h < heads; ++h) {
                const int t0 = cu_seqlens[s], L = cu_seqlens[s + 1] - t0;
                if (L > cap) {
                    free(p);
                    cap = L;
                    p = (double*)malloc(sizeof(double) * (size_t)cap);
                }
                for (int i = 0; i < L; ++i) {
                    const float* qi = q + ((size_t)(t0 + i) * heads + h) * d;
                    const int lo = half_window < 0 ? 0 : (i - half_window < 0 ? 0 : i - half_window);
                    const int hi = half_window < 0 ? L - 1 : (i + half_window > L - 1 ? L - 1 : i + half_window);
                    double mx = -INFINITY;
                    for (int j = lo; j <= hi; ++j) {
                        const float* kj = k + ((size_t)(t0 + j) * heads + h) * d;
                        float dot = 0.0f;
                        for (int e = 0; e < d; ++e) dot += qi[e] * kj[e];
                        p[j] = (double)(dot * scale);
                        if (p[j] > mx) mx = p[j];
                    }
                    double sum = 0.0;
                    for (int j = lo; j <= hi; ++j) {
                        p[j] = exp(p[j] - mx);
                        sum += p[j];
                    }
                    float* oi = out + ((size_t)(t0 + i) * heads + h) * d;
                    for (int e = 0; e < d; ++e) {
                        double acc = 0.0;
                        for (int j = lo; j <= hi; ++j) acc += p[j] * v[((size_t)(t0 + j) * heads + h) * d + e];
                        oi[e] = (float)(acc / sum);
                    }
                }
            }
        free(p);
    }
    return 0;
}

int ho_bert_forward(const ho_bert_cfg* c, const ho_bert_layer* layers, const float* embed, const float* emb_norm,
                    const float* final_norm, const int32_t* ids, const int32_t* cu_seqlens, int n_seqs, int bf16_mode,
                    float* out) {
    const int H = c->hidden, nh = c->n_heads, d = c->head_dim, I = c->intermediate;
    const int T = cu_seqlens[n_seqs];
    const int bf = bf16_mode;
    for (int t = 0; t < T; ++t)
        if (ids[t] < 0 || ids[t] >= c->vocab) return -1;
    float* h = (float*)malloc(sizeof(float) * (size_t)T * H);
    float* x = (float*)malloc(sizeof(float) * (size_t)T * H);
    float* qkv = (float*)malloc(sizeof(float) * (size_t)T * 3 * H);
    float* q = (float*)malloc(sizeof(float) * (size_t)T * H);
    float* k = (float*)malloc(sizeof(float) * (size_t)T * H);
    float* v = (float*)malloc(sizeof(float) * (size_t)T * H);
    float* att = (float*)malloc(sizeof(float) * (size_t)T * H);
    float* y = (float*)malloc(sizeof(float) * (size_t)T * H);
    float* gi = (float*)malloc(sizeof(float) * (size_t)T * 2 * I);
    float* act = (float*)malloc(sizeof(float) * (size_t)T * I);
    int32_t* pos = (int32_t*)malloc(sizeof(int32_t) * (size_t)(T > 0 ? T : 1));
    float* cs = (float*)malloc(sizeof(float) * (size_t)(T > 0 ? T : 1) * d);
    float* sn = (float*)malloc(sizeof(float) * (size_t)(T > 0 ? T : 1) * d);
    for (int s = 0; s < n_seqs; ++s)
        for (int t = cu_seqlens[s]; t < cu_seqlens[s + 1]; ++t) pos[t] = t - cu_seqlens[s];

    for (int t = 0; t < T; ++t) memcpy(x + (size_t)t * H, embed + (size_t)ids[t] * H, sizeof(float) * H);
    ho_layer_norm(x, emb_norm, T, H, c->eps, h);
    round_if(h, (size_t)T * H, bf);
    for (int l = 0; l < c->n_layers; ++l) {
        const ho_bert_layer* L = &layers[l];
        const int global = l % c->global_every == 0;
        if (L->attn_norm) {
            ho_layer_norm(h, L->attn_norm, T, H, c->eps, x);
            round_if(x, (size_t)T * H, bf);
        } else {
            memcpy(x, h, sizeof(float) * (size_t)T * H);
        }
        ho_linear(x, L->wqkv, NULL, T, H, 3 * H, qkv);
        round_if(qkv, (size_t)T * 3 * H, bf);
        for (int t = 0; t < T; ++t) {  /* [T][3][heads][d] -> q, k, v */
            memcpy(q + (size_t)t * H, qkv + (size_t)t * 3 * H, sizeof(float) * H);
            memcpy(k + (size_t)t * H, qkv + (size_t)t * 3 * H + H, sizeof(float) * H);
            memcpy(v + (size_t)t * H, qkv + (size_t)t * 3 * H + 2 * H, sizeof(float) * H);
        }
        ho_rope_cos_sin(d, global ? c->global_theta : c->local_theta, pos, T, bf, cs, sn);
        ho_apply_rope(q, T, nh, d, d, cs, sn, bf);
        ho_apply_rope(k, T, nh, d, d, cs, sn, bf);
        ho_bidir_attention(q, k, v, cu_seqlens, n_seqs, nh, d, global ? -1 : c->local_window / 2,
                           (float)(1.0 / sqrt((double)d)), att);
        round_if(att, (size_t)T * H, bf);
        ho_linear(att, L->wo, NULL, T, H, H, y);
        round_if(y, (size_t)T * H, bf);
        for (size_t i = 0; i < (size_t)T * H; ++i) h[i] += y[i];
        round_if(h, (size_t)T * H, bf);
        ho_layer_norm(h, L->mlp_norm, T, H, c->eps, x);
        round_if(x, (size_t)T * H, bf);
        ho_linear(x, L->wi, NULL, T, H, 2 * I, gi);
        round_if(gi, (size_t)T * 2 * I, bf);
        for (int t = 0; t < T; ++t)
            for (int i = 0; i < I; ++i)
                act[(size_t)t * I + i] = ho_gelu_erf(gi[(size_t)t * 2 * I + i]) * gi[(size_t)t * 2 * I + I + i];
        round_if(act, (size_t)T * I, bf);
        ho_linear(act, L->wo2, NULL, T, I, H, y);
        round_if(y, (size_t)T * H, bf);
        for (size_t i = 0; i < (size_t)T * H; ++i) h[i] += y[i];
        round_if(h, (size_t)T * H, bf);
    }
    ho_layer_norm(h, final_norm, T, H, c->eps, out);
    round_if(out, (size_t)T * H, bf);
    free(h); free(x); free(qkv); free(q); free(k); free(v); free(att); free(y); free(gi); free(act);
    free(pos); free(cs); free(sn);
    return 0;
}
