// attention.hip - paged GQA causal prefill attention for gfx950.
//
// Semantics follow the reference's dense path (crates/huncho-backend/src/qwen3_5.rs:669-703),
// its grouped/query-blocked variants (qwen3_5/attention.rs:6-111) and direct page attention
// (qwen3_5/kv_pages.rs:104-174): O = softmax(Q K^T * scale + causal mask) V, query head h
// reading KV head h / (Hq / Hkv), keys gathered through a block table (token j of a
// sequence lives in page block_tables[s][j / P], slot j % P; pool layout
// [page][kv_head][P][head_dim], the reference's Page tensor [1, Hkv, rows, d]).
//
// Design (one workgroup = one sequence x one KV head x 128 query rows):
//   * the 128 rows are the GQA group's query heads x (128 / group) positions, so every K/V
//     tile that is gathered into LDS serves all query heads of its KV head;
//   * 4 waves x 32 query rows; S^T = K Q^T on MFMA so that each lane owns one query
//     column and the softmax row statistics stay in-lane (one lane-swap per tile);
//   * K rows are loaded into the MFMA A operand in a permuted order so that each lane's
//     accumulator holds 16 consecutive keys; P then feeds P.V directly as the B operand,
//     and V is stored transposed in LDS so the A operand of O^T = V^T P^T is one 16-byte
//     read per MFMA;
//   * online softmax in base 2 with fp32 statistics; O^T accumulates in fp32 registers;
//   * the optional output gate o *= sigmoid(gate) (qwen3_5.rs:706-714) is fused into the
//     epilogue.
// Grid = (kv_heads, n_seqs, q_blocks) with the q-block index reversed, so the longest
// (latest) blocks of every sequence dispatch first; blocks past a sequence's end exit.
// With 8 KV heads the round-robin XCD dispatch keeps each KV head on one XCD, so the
// q-blocks that re-read a sequence's K/V share that XCD's L2.
#include "common.hpp"
#include "kernel_args.hpp"

namespace hk {

constexpr int D = 128;
constexpr int BN = 64;
constexpr int KS_STRIDE_BF16 = D + 8;   // padded LDS row (elements)
constexpr int VT_STRIDE_BF16 = BN + 8;
constexpr int KS_STRIDE_F32 = D + 4;
constexpr int V_STRIDE_F32 = D + 4;

// Key row loaded by accumulator row m so that lane group g, element j sees key g*16 + j.
__device__ __forceinline__ int perm_key(int m) { return ((m >> 2) & 1) * 16 + (m >> 3) * 4 + (m & 3); }

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + __expf(-x)); }

// Pool page of key `key` through the block table; -1 (and the fault flag) when the table
// entry lies past bt_stride or outside [0, num_pages).
__device__ __forceinline__ int page_of(const AttnArgs& a, const int* table, int key) {
    const int idx = key >> a.page_shift;
    const int page = idx < a.bt_stride ? table[idx] : -1;
    if ((unsigned)page >= (unsigned)a.num_pages) {
        atomicOr(a.fault, 2);
        return -1;
    }
    return page;
}

// ---------------------------------------------------------------------------
// 16-bit inputs (bf16 or fp16), fp32 accumulation
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256, 2) void paged_prefill_attn_16(AttnArgs a) {
    typedef typename Mma16<T>::v8 v8;
    typedef typename Mma16<T>::v4 v4;
    __shared__ __attribute__((aligned(16))) T Ks[BN * KS_STRIDE_BF16];
    __shared__ __attribute__((aligned(16))) T Vt[D * VT_STRIDE_BF16];

    const int kvh = blockIdx.x;
    const int seq = blockIdx.y;
    const int qb = gridDim.z - 1 - blockIdx.z;
    const int q0 = a.cu_seqlens_q[seq];
    const int q_len = a.cu_seqlens_q[seq + 1] - q0;
    const int ctx = a.context_lens[seq];
    const int P = a.pos_per_block;
    if (q0 < 0 || q_len < 0 || q0 + q_len > a.n_tokens || q_len > ctx) {
        if (threadIdx.x == 0) atomicOr(a.fault, 1);
        return;
    }
    if (qb * P >= q_len) return;
    const int off = ctx - q_len;  // absolute position of the first new query

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63, g = lane >> 5, col = lane & 31;

    // this lane's query row: (head in group, position)
    const int row = wave * 32 + col;
    const int hg = row / P, p = row % P;
    const int qi = qb * P + p;  // index among the sequence's new queries
    const bool q_valid = qi < q_len;
    const int head = kvh * a.group + hg;
    int qpos = off + (q_valid ? qi : q_len - 1);

    // Q fragment: Q[q][ks*16 + g*8 .. +8] for ks = 0..7
    v8 qf[8];
    {
        const T* qp = (const T*)a.q + (long)(q0 + (q_valid ? qi : 0)) * a.q_tok + (long)head * a.q_head;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            if (q_valid)
                qf[ks] = *(const v8*)(qp + ks * 16 + g * 8);
            else
                qf[ks] = v8{};
        }
    }

    const int last_pos = off + min(q_len, (qb + 1) * P) - 1;  // largest query position in the block
    const int first_pos = off + qb * P;
    const int n_tiles = last_pos / BN + 1;
    const int* table = a.block_tables + (long)seq * a.bt_stride;
    const int pmask = (1 << a.page_shift) - 1;

    // global -> register prefetch of one K/V tile
    // K: thread t loads rows t/16 + 16i (i = 0..3), 16-byte column chunk t % 16
    // V: thread t loads keys 4*(t/16) + i (i = 0..3), 8 dims (t % 16) * 8
    uint4 kr[4], vr[4];
    auto load_tile = [&](int tile) {
        const int n0 = tile * BN;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            int key = n0 + (tid >> 4) + 16 * i;
            int page = key < ctx ? page_of(a, table, key) : -1;
            if (page >= 0) {
                long base = (((long)page * a.kv_heads + kvh) << a.page_shift) + (key & pmask);
                kr[i] = *(const uint4*)((const T*)a.k_pool + base * D + (tid & 15) * 8);
            } else {
                kr[i] = uint4{0, 0, 0, 0};
            }
            int vkey = n0 + 4 * (tid >> 4) + i;
            int vpage = vkey < ctx ? page_of(a, table, vkey) : -1;
            if (vpage >= 0) {
                long base = (((long)vpage * a.kv_heads + kvh) << a.page_shift) + (vkey & pmask);
                vr[i] = *(const uint4*)((const T*)a.v_pool + base * D + (tid & 15) * 8);
            } else {
                vr[i] = uint4{0, 0, 0, 0};
            }
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            *(uint4*)(Ks + ((tid >> 4) + 16 * i) * KS_STRIDE_BF16 + (tid & 15) * 8) = kr[i];
        // transpose V: Vt[d][key]; each thread writes 4 consecutive keys for each of its 8 dims
        const T* v0 = (const T*)&vr[0];
        const T* v1 = (const T*)&vr[1];
        const T* v2 = (const T*)&vr[2];
        const T* v3 = (const T*)&vr[3];
        const int kbase = 4 * (tid >> 4), d0 = (tid & 15) * 8;
#pragma unroll
        for (int dd = 0; dd < 8; ++dd) {
            v4 w = {v0[dd], v1[dd], v2[dd], v3[dd]};
            *(v4*)(Vt + (d0 + dd) * VT_STRIDE_BF16 + kbase) = w;
        }
    };

    f32x16 acc_o[4];
#pragma unroll
    for (int db = 0; db < 4; ++db) acc_o[db] = f32x16{};
    float m_run = -INFINITY, l_run = 0.0f;

    load_tile(0);
    for (int tile = 0; tile < n_tiles; ++tile) {
        __syncthreads();
        store_tile();
        __syncthreads();
        if (tile + 1 < n_tiles) load_tile(tile + 1);

        // S^T = K Q^T for this wave's 32 queries: two 32-key blocks
        f32x16 s[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            s[kb] = f32x16{};
            const T* krow = Ks + (kb * 32 + perm_key(col)) * KS_STRIDE_BF16 + g * 8;
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) {
                v8 af = *(const v8*)(krow + ks * 16);
                s[kb] = Mma16<T>::mma(af, qf[ks], s[kb]);
            }
        }
        // scale to base 2, causal mask (only tiles that reach past the block's first query)
        const int n0 = tile * BN;
        const bool need_mask = n0 + BN - 1 > first_pos;
        float mloc = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                float v = s[kb][j] * a.scale_log2;
                if (need_mask && n0 + kb * 32 + g * 16 + j > qpos) v = -INFINITY;
                s[kb][j] = v;
                mloc = fmaxf(mloc, v);
            }
        const float m_new = fmaxf(m_run, wave_max32(mloc));
        const float alpha = fast_exp2(m_run - m_new);
        m_run = m_new;
        float lsum = 0.0f;
        v8 pf[4];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                v8 t;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    float e = fast_exp2(s[kb][h * 8 + i] - m_new);
                    lsum += e;
                    t[i] = (T)e;
                }
                pf[kb * 2 + h] = t;
            }
        l_run = l_run * alpha + lsum;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int j = 0; j < 16; ++j) acc_o[db][j] *= alpha;
        // O^T += V^T P^T
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            const T* vrow = Vt + (db * 32 + col) * VT_STRIDE_BF16 + g * 16;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int kb = c >> 1, h = c & 1;
                v8 af = *(const v8*)(vrow + kb * 32 + h * 8);
                acc_o[db] = Mma16<T>::mma(af, pf[c], acc_o[db]);
            }
        }
    }

    // epilogue: o = O / l (both lane halves hold partial row sums), optional sigmoid gate
    const float l_tot = l_run + __shfl_xor(l_run, 32);
    const float inv_l = 1.0f / l_tot;
    if (!q_valid) return;
    T* op = (T*)a.o + (long)(q0 + qi) * a.o_tok + (long)head * a.o_head;
    const T* gp = a.gate ? (const T*)a.gate + (long)(q0 + qi) * a.g_tok + (long)head * a.g_head : nullptr;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const int d = db * 32 + jj * 8 + g * 4;
            float r0 = acc_o[db][jj * 4 + 0] * inv_l, r1 = acc_o[db][jj * 4 + 1] * inv_l;
            float r2 = acc_o[db][jj * 4 + 2] * inv_l, r3 = acc_o[db][jj * 4 + 3] * inv_l;
            if (gp) {
                v4 gv = *(const v4*)(gp + d);
                // the reference rounds attn and sigmoid(gate) to the activation dtype, then multiplies
                r0 = (float)(T)r0 * (float)(T)sigmoidf_((float)gv[0]);
                r1 = (float)(T)r1 * (float)(T)sigmoidf_((float)gv[1]);
                r2 = (float)(T)r2 * (float)(T)sigmoidf_((float)gv[2]);
                r3 = (float)(T)r3 * (float)(T)sigmoidf_((float)gv[3]);
            }
            v4 w = {(T)r0, (T)r1, (T)r2, (T)r3};
            *(v4*)(op + d) = w;
        }
}

// ---------------------------------------------------------------------------
// fp32 inputs and accumulation (v_mfma_f32_32x32x2_f32)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256, 1) void paged_prefill_attn_f32(AttnArgs a) {
    __shared__ __attribute__((aligned(16))) float Ks[BN * KS_STRIDE_F32];
    __shared__ __attribute__((aligned(16))) float Vs[BN * V_STRIDE_F32];

    const int kvh = blockIdx.x;
    const int seq = blockIdx.y;
    const int qb = gridDim.z - 1 - blockIdx.z;
    const int q0 = a.cu_seqlens_q[seq];
    const int q_len = a.cu_seqlens_q[seq + 1] - q0;
    const int ctx = a.context_lens[seq];
    const int P = a.pos_per_block;
    if (q0 < 0 || q_len < 0 || q0 + q_len > a.n_tokens || q_len > ctx) {
        if (threadIdx.x == 0) atomicOr(a.fault, 1);
        return;
    }
    if (qb * P >= q_len) return;
    const int off = ctx - q_len;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63, g = lane >> 5, col = lane & 31;
    const int row = wave * 32 + col;
    const int hg = row / P, p = row % P;
    const int qi = qb * P + p;
    const bool q_valid = qi < q_len;
    const int head = kvh * a.group + hg;
    const int qpos = off + (q_valid ? qi : q_len - 1);

    // Q fragment: Q[q][4u + 2g + e], u = 0..31, e = 0..1
    f32x2 qf[32];
    {
        const float* qp = (const float*)a.q + (long)(q0 + (q_valid ? qi : 0)) * a.q_tok + (long)head * a.q_head;
#pragma unroll
        for (int u = 0; u < 32; ++u) qf[u] = q_valid ? *(const f32x2*)(qp + 4 * u + 2 * g) : f32x2{0.f, 0.f};
    }

    const int last_pos = off + min(q_len, (qb + 1) * P) - 1;
    const int first_pos = off + qb * P;
    const int n_tiles = last_pos / BN + 1;
    const int* table = a.block_tables + (long)seq * a.bt_stride;
    const int pmask = (1 << a.page_shift) - 1;

    // tile = 64 rows x 128 floats = 2048 float4; thread t loads float4 chunk t + 256 i, i = 0..7
    float4 kr[8], vr[8];
    auto load_tile = [&](int tile) {
        const int n0 = tile * BN;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            int c = tid + 256 * i;
            int key = n0 + (c >> 5);
            int page = key < ctx ? page_of(a, table, key) : -1;
            if (page >= 0) {
                long base = ((((long)page * a.kv_heads + kvh) << a.page_shift) + (key & pmask)) * D + (c & 31) * 4;
                kr[i] = *(const float4*)((const float*)a.k_pool + base);
                vr[i] = *(const float4*)((const float*)a.v_pool + base);
            } else {
                kr[i] = float4{0.f, 0.f, 0.f, 0.f};
                vr[i] = float4{0.f, 0.f, 0.f, 0.f};
            }
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            int c = tid + 256 * i;
            *(float4*)(Ks + (c >> 5) * KS_STRIDE_F32 + (c & 31) * 4) = kr[i];
            *(float4*)(Vs + (c >> 5) * V_STRIDE_F32 + (c & 31) * 4) = vr[i];
        }
    };

    f32x16 acc_o[4];
#pragma unroll
    for (int db = 0; db < 4; ++db) acc_o[db] = f32x16{};
    float m_run = -INFINITY, l_run = 0.0f;

    load_tile(0);
    for (int tile = 0; tile < n_tiles; ++tile) {
        __syncthreads();
        store_tile();
        __syncthreads();
        if (tile + 1 < n_tiles) load_tile(tile + 1);

        f32x16 s[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            s[kb] = f32x16{};
            const float* krow = Ks + (kb * 32 + perm_key(col)) * KS_STRIDE_F32 + 2 * g;
#pragma unroll
            for (int u = 0; u < 32; ++u) {
                f32x2 kv = *(const f32x2*)(krow + 4 * u);
                s[kb] = mfma_f32(kv[0], qf[u][0], s[kb]);
                s[kb] = mfma_f32(kv[1], qf[u][1], s[kb]);
            }
        }
        const int n0 = tile * BN;
        const bool need_mask = n0 + BN - 1 > first_pos;
        float mloc = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                float v = s[kb][j] * a.scale_log2;
                if (need_mask && n0 + kb * 32 + g * 16 + j > qpos) v = -INFINITY;
                s[kb][j] = v;
                mloc = fmaxf(mloc, v);
            }
        const float m_new = fmaxf(m_run, wave_max32(mloc));
        const float alpha = exp2f(m_run - m_new);
        m_run = m_new;
        float lsum = 0.0f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                float e = exp2f(s[kb][j] - m_new);
                s[kb][j] = e;
                lsum += e;
            }
        l_run = l_run * alpha + lsum;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int j = 0; j < 16; ++j) acc_o[db][j] *= alpha;
        // O^T[d][q] += V[key][d] P[q][key]; MFMA (kb, j) pairs k = g with key kb*32 + g*16 + j
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            const float* vcol = Vs + g * 16 * V_STRIDE_F32 + db * 32 + col;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    acc_o[db] = mfma_f32(vcol[(kb * 32 + j) * V_STRIDE_F32], s[kb][j], acc_o[db]);
        }
    }

    const float l_tot = l_run + __shfl_xor(l_run, 32);
    const float inv_l = 1.0f / l_tot;
    if (!q_valid) return;
    float* op = (float*)a.o + (long)(q0 + qi) * a.o_tok + (long)head * a.o_head;
    const float* gp = a.gate ? (const float*)a.gate + (long)(q0 + qi) * a.g_tok + (long)head * a.g_head : nullptr;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const int d = db * 32 + jj * 8 + g * 4;
            f32x4 r;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float v = acc_o[db][jj * 4 + e] * inv_l;
                if (gp) v = v * sigmoidf_(gp[d + e]);
                r[e] = v;
            }
            *(f32x4*)(op + d) = r;
        }
}

}  // namespace hk

// ---------------------------------------------------------------------------
// launcher (called by the C ABI after validation)
// ---------------------------------------------------------------------------
extern "C" int hk_launch_paged_prefill_attention(int dtype, const hk::AttnArgs* args, int n_seqs,
                                                 int n_qblocks, hipStream_t stream) {
    dim3 grid(args->kv_heads, n_seqs, n_qblocks);
    if (dtype == hk::DT_BF16)
        hipLaunchKernelGGL(hk::paged_prefill_attn_16<hk::bf16>, grid, dim3(256), 0, stream, *args);
    else if (dtype == hk::DT_F16)
        hipLaunchKernelGGL(hk::paged_prefill_attn_16<hk::f16>, grid, dim3(256), 0, stream, *args);
    else
        hipLaunchKernelGGL(hk::paged_prefill_attn_f32, grid, dim3(256), 0, stream, *args);
    return hipGetLastError() == hipSuccess ? HK_OK : HK_ERR_DEVICE;
}
