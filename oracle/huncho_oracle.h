/*
 * huncho_oracle.h - CPU restatement of Huncho's Qwen3.5 (Kev) scoring-forward path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity oracle and the timed CPU
 * baseline. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it, and only as the checker. The product path (libhuncho_rocm) never
 * links or calls it.
 *
 * Every function follows a reference file of grafuls/huncho (paths relative to the
 * reference repository root) op for op, in fp32, in the reference's reduction order
 * where the reference fixes one. Functions that take `bf16_mode` round to bfloat16
 * (round-to-nearest-even) at the points where the reference's bf16 execution stores
 * a bf16 tensor between operations.
 *
 * Layouts are token-major: activations [tokens][heads][dim], row-major weights
 * [out][in] (the candle/PyTorch Linear convention).
 */
#ifndef HUNCHO_ORACLE_H
#define HUNCHO_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- numeric helpers ---------------------------------------------------- */
uint16_t ho_f32_to_bf16(float x);           /* round-to-nearest-even, NaN kept quiet */
float ho_bf16_to_f32(uint16_t x);
void ho_round_bf16(float* x, size_t n);     /* in place: x = bf16(x) */
void ho_to_bf16(const float* x, uint16_t* out, size_t n);
void ho_from_bf16(const uint16_t* x, float* out, size_t n);

/* Seeded N(0,1) fp32 stream: splitmix64 -> two 24-bit uniforms -> Box-Muller. */
void ho_normal_fill(uint64_t seed, uint64_t stream, float* out, size_t n, float mean, float std);
/* Seeded integers uniform in [lo, hi] (inclusive), splitmix64 modulo-free rejection. */
void ho_uniform_int_fill(uint64_t seed, uint64_t stream, int32_t* out, size_t n, int32_t lo, int32_t hi);
/* Seeded Fisher-Yates permutation of 0..n-1. */
void ho_permutation(uint64_t seed, uint64_t stream, int32_t* out, int32_t n);

void ho_set_threads(int n);                 /* OpenMP thread count for the parallel loops */
int ho_get_threads(void);

/* ---- norms, qwen3_5.rs:178-214 ------------------------------------------ */
void ho_rms_norm_effective(const float* x, const float* w_eff, int rows, int width, float eps,
                           float* y);
void ho_rms_norm_gated(const float* x, const float* z, const float* w, int rows, int width,
                       float eps, float* y);
void ho_l2norm(const float* x, int rows, int width, float eps, float* y);

/* ---- rotary, qwen3_5.rs:220-283 ----------------------------------------- */
int ho_rotary_dim(int head_dim, double partial_rotary_factor);
/* cos/sin tables [n][rd] for absolute positions; bf16_mode rounds them (qwen3_5.rs:243-244) */
void ho_rope_cos_sin(int rd, double theta, const int32_t* positions, int n, int bf16_mode,
                     float* cos_out, float* sin_out);
/* x [n][heads][head_dim] in place; rotates the first rd dims of every head (NeoX halves);
 * bf16_mode rounds each product and the sum. */
void ho_apply_rope(float* x, int n, int heads, int head_dim, int rd, const float* cos_t,
                   const float* sin_t, int bf16_mode);

/* ---- paged KV, kv_pages.rs:63-98 and :307-341 ----------------------------
 * Pool layout [num_pages][kv_heads][page_size][head_dim] (one reference Page per
 * pool page). Token j of sequence s lives in page block_tables[s*bt_stride + j/P],
 * slot j%P. Element type is 16- or 32-bit (elem_bytes 2 or 4): payloads are copied
 * verbatim. k,v are [tokens][kv_heads][head_dim]; positions give each new token's
 * absolute index inside its sequence (prefix tokens + t). */
int ho_paged_kv_write(const void* k, const void* v, int elem_bytes, const int32_t* cu_seqlens,
                      const int32_t* positions, int n_seqs, int kv_heads, int head_dim,
                      int page_size, const int32_t* block_tables, int bt_stride, int num_pages,
                      void* k_pool, void* v_pool);

/* ---- attention, qwen3_5.rs:669-703 / attention.rs:6-111 / kv_pages.rs:104-174 ----
 * GQA causal softmax attention over paged K/V (fp32 math). q [q_tokens][Hq][d]; sequence
 * s has q_lens = cu_seqlens_q[s+1]-cu_seqlens_q[s] new queries at absolute positions
 * context_lens[s]-q_len .. context_lens[s]-1 and attends to keys 0..pos. K/V are read
 * from the pools (float) through the block table. Query head h reads KV head
 * h / (Hq/Hkv). Output o [q_tokens][Hq][d]. */
int ho_paged_attention_f32(const float* q, const float* k_pool, const float* v_pool,
                           const int32_t* block_tables, int bt_stride, const int32_t* cu_seqlens_q,
                           const int32_t* context_lens, int n_seqs, int q_heads, int kv_heads,
                           int head_dim, int page_size, float scale, float* o);
/* The same with bf16 (uint16) q/pools; math in fp32, output fp32. */
int ho_paged_attention_bf16(const uint16_t* q, const uint16_t* k_pool, const uint16_t* v_pool,
                            const int32_t* block_tables, int bt_stride,
                            const int32_t* cu_seqlens_q, const int32_t* context_lens, int n_seqs,
                            int q_heads, int kv_heads, int head_dim, int page_size, float scale,
                            float* o);

/* ---- gated delta rule, delta_cpu.rs:29-138 (== qwen3_5.rs:950-987) ------
 * Token-major inputs of one sequence batch: q,k [tokens][H][dk], v [tokens][H][dv],
 * g,beta [tokens][H]; sequences delimited by cu_seqlens. state [n_seqs][H][dk][dv]
 * fp32 is read as the initial state (NULL = zero) and overwritten with the final state
 * when final_state != NULL. o [tokens][H][dv]. Reduction order and no-FMA semantics
 * follow delta_cpu.rs (the file is compiled with -ffp-contract=off). */
int ho_gated_delta_rule(const float* q, const float* k, const float* v, const float* g,
                        const float* beta, const int32_t* cu_seqlens, int n_seqs, int heads,
                        int dk, int dv, const float* initial_state, float* o, float* final_state);

/* ---- causal depthwise conv + SiLU, conv_cpu.rs:5-51, qwen3_5.rs:817-870 ----
 * x [T][C] (one sequence, token-major), w [C][K], history [C][K-1] or NULL (the
 * cached tail: the reference prepends it). out [T][C] = silu(conv) in fp32. If
 * tail_out != NULL it receives the new tail [C][K-1] (raw inputs). */
void ho_causal_conv1d_silu(const float* x, int T, int C, const float* w, int K,
                           const float* history, float* out, float* tail_out);

/* ---- Qwen3.5 hybrid model, qwen3_5.rs:1020-1104, 1533-1553 ---------------- */
typedef struct {
    int hidden, n_layers, n_heads, n_kv_heads, head_dim, intermediate, vocab;
    float eps;
    double rope_theta;
    int rotary_dim;
    int conv_k, lin_key_dim, lin_n_k_heads, lin_n_v_heads, lin_v_dim;
    const int32_t* layer_types; /* per layer: 0 = linear attention (GDN), 1 = full attention */
} ho_qwen_cfg;

typedef struct {
    const float* input_norm_eff;   /* [hidden], 1 + w */
    const float* post_norm_eff;    /* [hidden], 1 + w */
    const float *gate_proj, *up_proj, *down_proj; /* [I][H], [I][H], [H][I] */
    /* linear attention (GDN) */
    const float *in_qkv, *in_z, *in_b, *in_a, *out_proj; /* [conv_dim][H], [Vd][H], [Hv][H], [Hv][H], [H][Vd] */
    const float *conv_w;           /* [conv_dim][K] */
    const float *norm_w;           /* [dv] (plain weight) */
    const float *a_log, *dt_bias;  /* [Hv] */
    /* full attention */
    const float *q_proj, *k_proj, *v_proj, *o_proj; /* [2*Hq*d][H], [Hkv*d][H], [Hkv*d][H], [H][Hq*d] */
    const float *q_norm_eff, *k_norm_eff;           /* [d], 1 + w */
} ho_qwen_layer;

/* Full forward of one sequence of T tokens (fresh cache, positions 0..T-1). Returns the
 * final-normed hidden states [T][hidden] (bf16-rounded values in bf16_mode). */
int ho_qwen_forward(const ho_qwen_cfg* cfg, const ho_qwen_layer* layers, const float* embed,
                    const float* final_norm_eff, const int32_t* ids, int T, int bf16_mode,
                    float* hidden_out);

/* y[n][out] = x[n][in] . W[out][in]^T (+ b), fp32 accumulation. */
/* ---- ModernBERT encoder (ho_bert.c; the Laya backend's candle ModernBERT) ---- */
void ho_layer_norm(const float* x, const float* w, int rows, int width, float eps, float* y);
float ho_gelu_erf(float x);
int ho_bidir_attention(const float* q, const float* k, const float* v, const int32_t* cu_seqlens, int n_seqs,
                       int heads, int d, int half_window, float scale, float* out);
typedef struct {
    int hidden, n_layers, n_heads, head_dim, intermediate, vocab;
    float eps;
    int global_every;    /* layer i is global iff i % global_every == 0 */
    int local_window;    /* local layers see keys with |i - j| <= local_window / 2 */
    double global_theta, local_theta;
} ho_bert_cfg;
typedef struct {
    const float* attn_norm;       /* [H] or NULL (identity) */
    const float *wqkv, *wo;       /* [3H][H], [H][H] */
    const float* mlp_norm;        /* [H] */
    const float *wi, *wo2;        /* [2I][H], [H][I] */
} ho_bert_layer;
/* Final-normed hidden states [T][H] of an unpadded varlen batch (cu_seqlens [n_seqs + 1]). */
int ho_bert_forward(const ho_bert_cfg* cfg, const ho_bert_layer* layers, const float* embed, const float* emb_norm,
                    const float* final_norm, const int32_t* ids, const int32_t* cu_seqlens, int n_seqs, int bf16_mode,
                    float* out);

void ho_linear(const float* x, const float* w, const float* b, int n, int in, int out, float* y);

/* ---- readout and calibration -------------------------------------------
 * kev.rs:161-165: q = Wq.h_last + bq; k_i = Wk.h_pos_i + bk; score_i = k_i.q * scale. */
void ho_pointer_head(const float* hidden, int hidden_size, int T, const int32_t* positions,
                     int n_pos, const float* wq, const float* bq, const float* wk,
                     const float* bk, int head_dim, float* scores);
/* calibration.rs:42-60 + 170-173: fp32 exp, fp64 ordered sum/divide. Returns 0, or -1
 * on a non-finite logit / bad temperature / non-finite probability. */
int ho_calibrate(const float* logits, int n, float temperature, float* probs);

#ifdef __cplusplus
}
#endif
#endif
