// bert.hip - the ModernBERT encoder behind Huncho's Laya backend (candle ModernBERT,
// crates/huncho-backend/src/candle.rs:65-117, 319-416) on gfx950.
//
//   bidir_attn_16<T>   bidirectional softmax attention over an unpadded varlen batch, head dim
//                      64, optional window |i - j| <= w (local layers), q/k/v read straight
//                      from the fused Wqkv rows [tokens][3][heads][64]
//   bidir_attn_f32     the same in fp32 (the reference's execution precision)
//   layer_norm<T>      LayerNorm without bias, fp32 statistics
//   geglu<T>           gelu(x1) * x2 with the exact erf GELU
//   rope_qk<T>         NeoX rotate-half RoPE on the q and k parts of the Wqkv rows, in place
//   mean_pool_head<T>  per-sequence mean of the final hidden rows, then a linear head (fp32)
//
// bidir_attn_16 design: one workgroup = one (sequence, head, 128 query positions); 4 waves x
// 32 queries; S^T = K Q^T on v_mfma_f32_32x32x16 (each lane owns a query column, K rows
// permuted so a lane's accumulator holds 16 consecutive keys that feed P.V directly); K and
// V tiles of 64 keys in double-buffered LDS with XOR chunk swizzles (K: row & 7; V:
// (row & 3) << 1 | (row >> 4) & 1, chosen so the permuted K reads, the transposing V reads
// (ds_read_b64_tr_b16) and the row writes all reach the LDS banks evenly); online softmax
// in base 2 with lazy rescaling; only tiles that intersect the block's key range are read.
#include "common.hpp"
#include "kernel_args.hpp"

namespace hk {
namespace bert {

constexpr int D = 64;                       // head dim
constexpr int BN = 64;                      // keys per tile
constexpr int TILE = BN * D;                // elements per K or V tile (8 KB in 16 bits)
constexpr size_t LDS16 = 4 * TILE * 2;      // K and V, double-buffered: 32 KB
constexpr float RESCALE_LOG2 = 8.0f;

__device__ __forceinline__ int perm_key(int m) { return ((m >> 2) & 1) * 16 + (m >> 3) * 4 + (m & 3); }
__device__ __forceinline__ int kswz(int r) { return r & 7; }
__device__ __forceinline__ int vswz(int r) { return ((r & 3) << 1) | ((r >> 4) & 1); }
__device__ __forceinline__ int k_off(int r, int c) { return r * D + 8 * (c ^ kswz(r)); }
__device__ __forceinline__ int v_off(int r, int c) { return r * D + 8 * (c ^ vswz(r)); }

template <typename T>
__global__ __launch_bounds__(256, 2) void bidir_attn_16(BertAttnArgs a) {
    typedef typename Mma16<T>::v8 v8;
    typedef typename Mma16<T>::v4 v4;
    extern __shared__ __attribute__((aligned(16))) char bert_smem[];
    T* const lds = (T*)bert_smem;  // [buf][K | V][64][64]

    const int qb = blockIdx.x, h = blockIdx.y, seq = blockIdx.z;
    const int t0 = a.cu[seq];
    const int L = a.cu[seq + 1] - t0;
    if (t0 < 0 || L < 0 || t0 + L > a.n_tokens) {
        if (threadIdx.x == 0) atomicOr(a.fault, 1);
        return;
    }
    if (qb * 128 >= L) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 5, col = lane & 31;
    const int p = qb * 128 + wave * 32 + col;  // this lane's query position
    const bool q_valid = p < L;
    const int w = a.half_window;

    v8 qf[4];  // Q[p][16 ks + 8 g .. + 8]
    {
        const T* qp = (const T*)a.q + (long)(t0 + (q_valid ? p : 0)) * a.q_tok + (long)h * D;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) qf[ks] = q_valid ? *(const v8*)(qp + ks * 16 + g * 8) : v8{};
    }
    // keys any query of the block may see
    const int blk_lo = qb * 128, blk_hi = min(L, qb * 128 + 128) - 1;
    const int k_lo = w < 0 ? 0 : max(0, blk_lo - w);
    const int k_hi = w < 0 ? L - 1 : min(L - 1, blk_hi + w);
    const int tile_lo = k_lo / BN, n_tiles = k_hi / BN - tile_lo + 1;

    int kro[4], vro[2];
    {
        const int r = perm_key(col);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) kro[ks] = k_off(r, 2 * ks + g);
        const int G = lane >> 4, j = lane & 15;
        const int vrow = (G >> 1) * 16 + (j >> 2);  // + 32 kb + 8 hh + 4 x, which leave vswz unchanged
        const int cl = 2 * (G & 1) + ((j & 3) >> 1);
#pragma unroll
        for (int db = 0; db < 2; ++db) vro[db] = vrow * D + 8 * ((4 * db + cl) ^ vswz(vrow)) + 4 * (j & 1);
    }

    // thread t moves key rows t / 8 and t / 8 + 32 of a tile, 16-byte chunk t % 8, of K and V;
    // keys past the sequence end read its last row (finite; their scores are masked)
    const int lr = tid >> 3, lc = tid & 7;
    uint4 kr[2], vr[2];
    auto load_tile = [&](int tile) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int key = min(tile * BN + lr + 32 * i, L - 1);
            kr[i] = *(const uint4*)((const T*)a.k + (long)(t0 + key) * a.k_tok + (long)h * D + lc * 8);
            vr[i] = *(const uint4*)((const T*)a.v + (long)(t0 + key) * a.v_tok + (long)h * D + lc * 8);
        }
    };
    auto store_tile = [&](int buf) {
        T* Kb = lds + buf * 2 * TILE;
        T* Vb = Kb + TILE;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            *(uint4*)(Kb + k_off(lr + 32 * i, lc)) = kr[i];
            *(uint4*)(Vb + v_off(lr + 32 * i, lc)) = vr[i];
        }
    };

    f32x16 acc_o[2];
    acc_o[0] = f32x16{};
    acc_o[1] = f32x16{};
    float m_use = -INFINITY, l_run = 0.0f;
    const float c = a.scale_log2;

    load_tile(tile_lo);
    store_tile(0);
    __syncthreads();
    for (int it = 0; it < n_tiles; ++it) {
        const int buf = it & 1, tile = tile_lo + it;
        if (it + 1 < n_tiles) load_tile(tile + 1);
        const T* Kb = lds + buf * 2 * TILE;
        const T* Vb = Kb + TILE;
        f32x16 s[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            s[kb] = f32x16{};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
                s[kb] = Mma16<T>::mma(*(const v8*)(Kb + kb * 32 * D + kro[ks]), qf[ks], s[kb]);
        }
        // mask keys past the sequence end or outside this query's window; tiles that lie
        // inside every query's window skip the compare
        const int n0 = tile * BN;
        const bool inside = n0 + BN - 1 < L && (w < 0 || (n0 >= blk_hi - w && n0 + BN - 1 <= blk_lo + w));
        float mloc = -INFINITY;
        if (!inside) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int jj = 0; jj < 16; ++jj) {
                    const int key = n0 + kb * 32 + g * 16 + jj;
                    const int dist = key > p ? key - p : p - key;
                    if (key >= L || (w >= 0 && dist > w)) s[kb][jj] = -INFINITY;
                    mloc = fmaxf(mloc, s[kb][jj]);
                }
        } else {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int jj = 0; jj < 16; ++jj) mloc = fmaxf(mloc, s[kb][jj]);
        }
        const float m_tile = wave_max32(mloc);
        const bool grow = (m_tile - m_use) * c > RESCALE_LOG2;
        if (__any(grow)) {
            const float m_new = grow ? m_tile : m_use;
            // lanes that keep their max keep their sums (alpha 1; also avoids -inf - -inf)
            const float alpha = grow ? fast_exp2((m_use - m_new) * c) : 1.0f;
            m_use = m_new;
            l_run *= alpha;
#pragma unroll
            for (int db = 0; db < 2; ++db)
#pragma unroll
                for (int jj = 0; jj < 16; ++jj) acc_o[db][jj] *= alpha;
        }
        // a query whose keys so far were all masked still has m_use = -inf: its scores are
        // all -inf and exp2 gives 0 with any finite offset
        const float mc = m_use == -INFINITY ? 0.0f : m_use * c;
        float lsum = 0.0f;
        v8 pf[4];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                v8 t;
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const float e = fast_exp2(fmaf(s[kb][hh * 8 + k], c, -mc));
                    lsum += e;
                    t[k] = (T)e;
                }
                pf[kb * 2 + hh] = t;
            }
        l_run += lsum;
#pragma unroll
        for (int db = 0; db < 2; ++db) {
            const T* vb = Vb + vro[db];
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
                const int kb = cc >> 1, hh = cc & 1;
                const i16x4 lo = lds_read_tr16(vb + (kb * 32 + hh * 8) * D);
                const i16x4 hi = lds_read_tr16(vb + (kb * 32 + hh * 8 + 4) * D);
                const v8 af = __builtin_bit_cast(v8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
                acc_o[db] = Mma16<T>::mma(af, pf[cc], acc_o[db]);
            }
        }
        if (it + 1 < n_tiles) store_tile(buf ^ 1);
        __syncthreads();
    }
    const float l_tot = l_run + __shfl_xor(l_run, 32);
    if (!q_valid) return;
    const float inv_l = 1.0f / l_tot;
    T* op = (T*)a.o + (long)(t0 + p) * a.o_tok + (long)h * D;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            v4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = (T)(acc_o[db][jj * 4 + e] * inv_l);
            *(v4*)(op + db * 32 + jj * 8 + g * 4) = o;
        }
}

// fp32: one thread per query (q and the O accumulator in registers); 64 queries of one head
// share 32-key K and V tiles in LDS.
__global__ __launch_bounds__(64) void bidir_attn_f32(BertAttnArgs a) {
    __shared__ float Ks[32][D + 1];
    __shared__ float Vs[32][D + 1];
    const int qb = blockIdx.x, h = blockIdx.y, seq = blockIdx.z;
    const int t0 = a.cu[seq];
    const int L = a.cu[seq + 1] - t0;
    if (t0 < 0 || L < 0 || t0 + L > a.n_tokens) {
        if (threadIdx.x == 0) atomicOr(a.fault, 1);
        return;
    }
    if (qb * 64 >= L) return;
    const int tid = threadIdx.x;
    const int p = qb * 64 + tid;
    const bool q_valid = p < L;
    const int w = a.half_window;
    const float scale = a.scale_log2 * 0.69314718055994531f;  // natural-log scale
    float q[D], o[D];
    {
        const float* qp = (const float*)a.q + (long)(t0 + (q_valid ? p : 0)) * a.q_tok + (long)h * D;
#pragma unroll
        for (int e = 0; e < D; ++e) {
            q[e] = qp[e];
            o[e] = 0.0f;
        }
    }
    const int blk_lo = qb * 64, blk_hi = min(L, qb * 64 + 64) - 1;
    const int k_lo = w < 0 ? 0 : max(0, blk_lo - w);
    const int k_hi = w < 0 ? L - 1 : min(L - 1, blk_hi + w);
    float m = -INFINITY, l = 0.0f;
    for (int base = k_lo; base <= k_hi; base += 32) {
        __syncthreads();
        for (int idx = tid; idx < 32 * D; idx += 64) {
            const int r = idx / D, e = idx % D;
            const int key = min(base + r, L - 1);
            Ks[r][e] = ((const float*)a.k)[(long)(t0 + key) * a.k_tok + (long)h * D + e];
            Vs[r][e] = ((const float*)a.v)[(long)(t0 + key) * a.v_tok + (long)h * D + e];
        }
        __syncthreads();
        const int n = min(32, k_hi - base + 1);
        for (int r = 0; r < n; ++r) {
            const int key = base + r;
            const int dist = key > p ? key - p : p - key;
            if (w >= 0 && dist > w) continue;
            float sdot = 0.0f;
#pragma unroll
            for (int e = 0; e < D; ++e) sdot = fmaf(q[e], Ks[r][e], sdot);
            const float sv = sdot * scale;
            const float m_new = fmaxf(m, sv);
            const float alpha = __expf(m - m_new);
            const float pe = __expf(sv - m_new);
            l = l * alpha + pe;
#pragma unroll
            for (int e = 0; e < D; ++e) o[e] = fmaf(pe, Vs[r][e], o[e] * alpha);
            m = m_new;
        }
    }
    if (!q_valid) return;
    float* op = (float*)a.o + (long)(t0 + p) * a.o_tok + (long)h * D;
    const float inv = 1.0f / l;
#pragma unroll
    for (int e = 0; e < D; ++e) op[e] = o[e] * inv;
}

// LayerNorm without bias over rows of `width` (<= 2048): one wave per row, two passes over
// registers (mean, then the centred sum of squares), statistics in fp32.
template <typename T>
__global__ __launch_bounds__(256) void layer_norm(LayerNormArgs a) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= a.rows) return;
    const T* x = (const T*)a.x + (long)row * a.x_tok;
    T* y = (T*)a.y + (long)row * a.y_tok;
    float v[32];
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < 32; ++k) {
        const int i = lane + 64 * k;
        v[k] = i < a.width ? to_f(x[i]) : 0.0f;
        s += v[k];
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o);
    const float mean = s / (float)a.width;
    float q = 0.0f;
#pragma unroll
    for (int k = 0; k < 32; ++k) {
        const int i = lane + 64 * k;
        const float d = i < a.width ? v[k] - mean : 0.0f;
        q += d * d;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) q += __shfl_xor(q, o);
    const float inv = fast_rsqrt(q / (float)a.width + a.eps);
#pragma unroll
    for (int k = 0; k < 32; ++k) {
        const int i = lane + 64 * k;
        if (i < a.width) y[i] = from_f<T>(((v[k] - mean) * inv) * a.w[i]);
    }
}

__device__ __forceinline__ float gelu_erf(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f)); }

// y[t][i] = gelu(x[t][i]) * x[t][I + i], fp32 arithmetic
template <typename T>
__global__ __launch_bounds__(256) void geglu(GegluArgs a) {
    const long n = (long)a.rows * a.width;
    for (long idx = (long)blockIdx.x * blockDim.x + threadIdx.x; idx < n; idx += (long)gridDim.x * blockDim.x) {
        const long t = idx / a.width;
        const int i = (int)(idx % a.width);
        const T* row = (const T*)a.x + t * a.x_tok;
        ((T*)a.y)[t * a.y_tok + i] = from_f<T>(gelu_erf(to_f(row[i])) * to_f(row[a.width + i]));
    }
}

// RoPE on q (columns 0 .. heads*64) and k (heads*64 .. 2*heads*64) of each row, in place:
// x[i] = x[i] cos - x[i + 32] sin, x[i + 32] = x[i + 32] cos + x[i] sin (i < 32), at the
// token's position within its sequence. Grid (position blocks of 8, sequences).
template <typename T>
__global__ __launch_bounds__(256) void rope_qk(RopeQkArgs a) {
    const int seq = blockIdx.y;
    const int t0 = a.cu[seq], L = a.cu[seq + 1] - t0;
    if (t0 < 0 || L < 0 || t0 + L > a.n_tokens) {
        if (threadIdx.x == 0) atomicOr(a.fault, 1);
        return;
    }
    const int pairs = 2 * a.heads * 32;  // (q | k) x heads x 32 rotation pairs per token
    for (int pp = blockIdx.x * 8; pp < min(L, blockIdx.x * 8 + 8); ++pp) {
        if (pp >= a.max_pos) {
            if (threadIdx.x == 0) atomicOr(a.fault, 4);
            return;
        }
        T* row = (T*)a.x + (long)(t0 + pp) * a.x_tok;
        for (int k = threadIdx.x; k < pairs; k += blockDim.x) {
            const int hh = k / 32, i = k % 32;  // hh < heads: q heads; >= heads: k heads
            T* xh = row + hh * 64;
            const float c = a.cos[(long)pp * 32 + i], s = a.sin[(long)pp * 32 + i];
            const float x1 = to_f(xh[i]), x2 = to_f(xh[i + 32]);
            xh[i] = from_f<T>(x1 * c - x2 * s);
            xh[i + 32] = from_f<T>(x2 * c + x1 * s);
        }
    }
}

// logits[s][o] = head_b[o] + sum_i head_w[o][i] * mean_t x[t][i] over the sequence's rows
template <typename T>
__global__ __launch_bounds__(256) void mean_pool_head(MeanPoolArgs a) {
    extern __shared__ float pooled[];  // [width]
    const int seq = blockIdx.x;
    const int t0 = a.cu[seq], L = a.cu[seq + 1] - t0;
    if (t0 < 0 || L <= 0 || t0 + L > a.n_tokens) {
        if (threadIdx.x == 0) atomicOr(a.fault, 1);
        return;
    }
    for (int i = threadIdx.x; i < a.width; i += blockDim.x) {
        float s = 0.0f;
        for (int t = 0; t < L; ++t) s += to_f(((const T*)a.x)[(long)(t0 + t) * a.x_tok + i]);
        pooled[i] = s / (float)L;
    }
    __syncthreads();
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int o = wave; o < a.n_out; o += blockDim.x / 64) {
        float s = 0.0f;
        for (int i = lane; i < a.width; i += 64) s += to_f(((const T*)a.head_w)[(long)o * a.width + i]) * pooled[i];
#pragma unroll
        for (int k = 32; k >= 1; k >>= 1) s += __shfl_xor(s, k);
        if (lane == 0) a.logits[(long)seq * a.n_out + o] = s + (a.head_b ? a.head_b[o] : 0.0f);
    }
}

}  // namespace bert
}  // namespace hk

#define HK_BERT_DISPATCH(dtype, KERNEL, grid, block, lds, stream, args)                                    \
    do {                                                                                                   \
        if ((dtype) == hk::DT_BF16)                                                                        \
            hipLaunchKernelGGL(hk::bert::KERNEL<hk::bf16>, grid, block, lds, stream, args);                \
        else if ((dtype) == hk::DT_F16)                                                                    \
            hipLaunchKernelGGL(hk::bert::KERNEL<hk::f16>, grid, block, lds, stream, args);                 \
        else                                                                                               \
            hipLaunchKernelGGL(hk::bert::KERNEL<float>, grid, block, lds, stream, args);                   \
    } while (0)

extern "C" int hk_launch_bidir_attention(int dtype, const hk::BertAttnArgs* a, int n_seqs, int max_len,
                                         hipStream_t stream) {
    if (dtype == hk::DT_F32) {
        hipLaunchKernelGGL(hk::bert::bidir_attn_f32, dim3((max_len + 63) / 64, a->heads, n_seqs), dim3(64), 0, stream,
                           *a);
        return hipGetLastError() == hipSuccess ? HK_OK : HK_ERR_DEVICE;
    }
    static bool configured = false;
    if (!configured) {
        if (hipFuncSetAttribute((const void*)hk::bert::bidir_attn_16<hk::bf16>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)hk::bert::LDS16) != hipSuccess ||
            hipFuncSetAttribute((const void*)hk::bert::bidir_attn_16<hk::f16>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)hk::bert::LDS16) != hipSuccess)
            return HK_ERR_DEVICE;
        configured = true;
    }
    const dim3 grid((max_len + 127) / 128, a->heads, n_seqs);
    if (dtype == hk::DT_BF16)
        hipLaunchKernelGGL(hk::bert::bidir_attn_16<hk::bf16>, grid, dim3(256), hk::bert::LDS16, stream, *a);
    else
        hipLaunchKernelGGL(hk::bert::bidir_attn_16<hk::f16>, grid, dim3(256), hk::bert::LDS16, stream, *a);
    return hipGetLastError() == hipSuccess ? HK_OK : HK_ERR_DEVICE;
}

extern "C" int hk_launch_layer_norm(int dtype, const hk::LayerNormArgs* a, hipStream_t stream) {
    HK_BERT_DISPATCH(dtype, layer_norm, dim3((a->rows + 3) / 4), dim3(256), 0, stream, *a);
    return hipGetLastError() == hipSuccess ? HK_OK : HK_ERR_DEVICE;
}

extern "C" int hk_launch_geglu(int dtype, const hk::GegluArgs* a, hipStream_t stream) {
    const long n = (long)a->rows * a->width;
    const int blocks = (int)((n + 255) / 256 < 65536 ? (n + 255) / 256 : 65536);
    HK_BERT_DISPATCH(dtype, geglu, dim3(blocks > 0 ? blocks : 1), dim3(256), 0, stream, *a);
    return hipGetLastError() == hipSuccess ? HK_OK : HK_ERR_DEVICE;
}

extern "C" int hk_launch_rope_qk(int dtype, const hk::RopeQkArgs* a, int n_seqs, int max_len, hipStream_t stream) {
    HK_BERT_DISPATCH(dtype, rope_qk, dim3((max_len + 7) / 8, n_seqs), dim3(256), 0, stream, *a);
    return hipGetLastError() == hipSuccess ? HK_OK : HK_ERR_DEVICE;
}

extern "C" int hk_launch_mean_pool_head(int dtype, const hk::MeanPoolArgs* a, int n_seqs, hipStream_t stream) {
    HK_BERT_DISPATCH(dtype, mean_pool_head, dim3(n_seqs), dim3(256), a->width * sizeof(float), stream, *a);
    return hipGetLastError() == hipSuccess ? HK_OK : HK_ERR_DEVICE;
}
